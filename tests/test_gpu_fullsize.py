"""Size-independent properties at BASELINE full sizes, through the C ABI.

At S = 31,104 (config 2) and S = 129,024 (config 3) with 32 heads the oracle is too slow for a
full comparison, so these tests check what the arithmetic fixes at any size:
  - the fused RoPE quantizer equals the separate route (rope_qknorm_f16, then prepare_qk_i8hm with
    zero mean) bit for bit (tests/kernels.rs:3153-3276 at full size);
  - every quantized row reaches the code +-127 (its absmax element), all codes lie in [-127, 127]
    and scales are positive and finite; capacity rows past the sequence stay untouched;
  - the V transpose is an exact bit permutation with a zero tail.
"""
import math

import numpy as np
import pytest

import h3attn as H
from helpers import filled

pytestmark = pytest.mark.gpu

EXTRA = H.EXTRA_Q


@pytest.mark.parametrize("tokens", [31104, 129024])
def test_fused_operands_at_full_size(dev, tokens):
    import torch

    heads = 32
    width = heads * 128
    cap = H.capacity(tokens)
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    fused = (torch.randn((tokens, 3 * width), generator=g, device=dev)).to(torch.bfloat16)
    w = torch.ones(128, device=dev)
    pos = torch.arange(tokens, device=dev, dtype=torch.float32)[:, None]
    ang = pos * torch.pow(torch.tensor(10000.0, device=dev), -torch.arange(48, device=dev) / 48.0)
    cos_t, sin_t = torch.cos(ang).contiguous(), torch.sin(ang).contiguous()
    print(f"full-size operands tokens={tokens}", flush=True)

    pk = H.PrepareCfg(3 * width, width, heads, 1.0, cap, 1e-5, H.H3_ELEM_BF16)
    codes = filled((heads * cap * 128,), 0x55, np.uint8, dev)
    scales = torch.zeros(heads * cap, dtype=torch.float32, device=dev)
    H.prepare_qk_rope_i8hm(pk, tokens, fused, w, cos_t, sin_t, codes, scales)

    rc = H.RopeCfg(3 * width, heads, heads, width, 1e-5, 0, H.H3_ELEM_BF16)
    q16 = torch.empty((tokens, width), dtype=torch.float16, device=dev)
    k16 = torch.empty((tokens, width), dtype=torch.float16, device=dev)
    H.rope_qknorm_f16(rc, tokens, fused, w, w, cos_t, sin_t, q16, k16)
    sep = filled((heads * cap * 128,), 0x55, np.uint8, dev)
    sep_s = torch.zeros(heads * cap, dtype=torch.float32, device=dev)
    zero_mean = torch.zeros(width, dtype=torch.float32, device=dev)
    H.prepare_qk_i8hm(H.PrepareCfg(width, 0, heads, 1.0, cap, 1e-5, H.H3_ELEM_F16), tokens, k16,
                      zero_mean, sep, sep_s)
    torch.cuda.synchronize()

    assert torch.equal(codes, sep), "fused and separate K operands differ"
    assert torch.equal(scales.view(torch.int32), sep_s.view(torch.int32))
    c = codes.view(torch.int8).view(heads, cap, 128)
    live = c[:, :tokens].to(torch.int16)
    assert int(live.abs().amax(dim=2).min()) == 127, "a row never reaches its absmax code"
    assert int(live.min()) >= -127 and int(live.max()) <= 127
    assert bool((c[:, tokens:].view(torch.uint8) == 0x55).all()), "capacity rows were written"
    s = scales.view(heads, cap)[:, :tokens]
    assert bool(torch.isfinite(s).all()) and float(s.min()) > 0.0


def test_v_transpose_at_full_size(dev):
    import torch

    tokens, heads = 129024, 32
    width = heads * 128
    cap = H.capacity(tokens)
    g = torch.Generator(device=dev)
    g.manual_seed(8)
    fused = torch.randn((tokens, 3 * width), generator=g, device=dev).to(torch.float16)
    vt = filled((width * cap * 2,), 0x77, np.uint8, dev)
    H.transpose_qkv_v_f16(H.TransposeCfg(width, cap, H.H3_ELEM_F16), cap, tokens, fused, vt)
    torch.cuda.synchronize()
    v = vt.view(torch.float16).view(width, cap)
    assert torch.equal(v[:, :tokens], fused[:, 2 * width:].t())
    assert bool((v[:, tokens:].view(torch.int16) == 0).all()), "capacity tail not cleared"
