"""The operand quantizer at the capacity the reference qualifies.

head_major_operand_preparation_proves_scale_rows (tests/compiler.rs:105-140) compiles
prepare_qk_i8hm and prepare_qk_rope_i8hm (Q at head offset 0, K at one projection width) for 56
heads at capacities 89,088 and 1,048,544, so a token's code and scale rows h*capacity + t stay in
bounds for the last head. Here the fused RoPE quantizer runs at capacity 1,048,544:
  - 56 heads over a few tokens: every head's rows < tokens bit-exact against the oracle, the
    rows after them and each head's last capacity row untouched (poisoned), for Q and K offsets;
  - one head over 1,048,528 tokens (the capacity less the 16 rows the reference keeps spare):
    every code and scale bit-exact.
"""
import math

import numpy as np
import pytest

import h3attn as H
import oracle as O
from helpers import filled, to_dev

pytestmark = pytest.mark.gpu

CAP = 1048544
EXTRA = O.config_f32(O.EXTRA_Q_F64)


def fused_rope_inputs(rng, tokens, width):
    f = rng.standard_normal((tokens, 3 * width), np.float32)
    ang = rng.uniform(-math.pi, math.pi, (tokens, 48)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    return O.f16_bits(f), w, np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


@pytest.mark.parametrize("head_offset", [0, 1])
def test_fused_quantizer_at_capacity_1048544_with_56_heads(dev, head_offset):
    import torch

    heads, tokens = 56, 2049
    width = heads * 128
    rng = np.random.default_rng(105 + head_offset)
    fused, w, cos_t, sin_t = fused_rope_inputs(rng, tokens, width)
    extra = EXTRA if head_offset == 0 else 1.0
    cfg = H.PrepareCfg(3 * width, head_offset * width, heads, extra, CAP, 1e-5, H.H3_ELEM_F16)
    codes = filled((heads * CAP * 128,), 0x55, np.uint8, dev)
    scales = filled((heads * CAP * 4,), 0x55, np.uint8, dev)
    print(f"prepare_qk_rope_i8hm capacity={CAP} heads={heads} offset={head_offset}", flush=True)
    H.prepare_qk_rope_i8hm(cfg, tokens, to_dev(fused, dev), to_dev(w, dev), to_dev(cos_t, dev),
                           to_dev(sin_t, dev), codes, scales)
    torch.cuda.synchronize()
    c = codes.view(heads, CAP, 128)
    s = scales.view(heads, CAP, 4)
    roped = O.rope_qknorm_f16(fused, O.F16, tokens, 3 * width, head_offset * width, heads, w,
                              cos_t, sin_t, 1e-5)
    want_w, want_s = O.prepare_qk(roped, O.F16, None, tokens, width, 0, heads, extra, True, tokens)
    got_w = c[:, :tokens].contiguous().cpu().numpy().view(np.int32).reshape(heads, tokens, 32)
    assert np.array_equal(got_w, want_w.reshape(heads, tokens, 32))
    got_s = s[:, :tokens].contiguous().cpu().numpy().view(np.uint32).reshape(heads, tokens)
    assert np.array_equal(got_s, want_s.view(np.uint32).reshape(heads, tokens))
    for part in (c[:, tokens:tokens + 64], c[:, CAP - 1], s[:, tokens:tokens + 64], s[:, CAP - 1]):
        assert bool((part == 0x55).all()), "rows past the tokens were written"


def test_fused_quantizer_over_the_qualified_capacity_with_one_head(dev):
    import torch

    heads, tokens = 1, CAP - 16
    width = 128
    rng = np.random.default_rng(1048)
    fused, w, cos_t, sin_t = fused_rope_inputs(rng, tokens, width)
    cfg = H.PrepareCfg(3 * width, width, heads, 1.0, CAP, 1e-5, H.H3_ELEM_F16)
    codes = filled((CAP * 128,), 0x55, np.uint8, dev)
    scales = filled((CAP * 4,), 0x55, np.uint8, dev)
    print(f"prepare_qk_rope_i8hm tokens={tokens} capacity={CAP}", flush=True)
    H.prepare_qk_rope_i8hm(cfg, tokens, to_dev(fused, dev), to_dev(w, dev), to_dev(cos_t, dev),
                           to_dev(sin_t, dev), codes, scales)
    torch.cuda.synchronize()
    roped = O.rope_qknorm_f16(fused, O.F16, tokens, 3 * width, width, heads, w, cos_t, sin_t,
                              1e-5)
    want_w, want_s = O.prepare_qk(roped, O.F16, None, tokens, width, 0, heads, 1.0, True, CAP)
    got = codes.cpu().numpy()
    assert np.array_equal(got[:tokens * 128].view(np.int32), want_w[:tokens].reshape(-1))
    assert (got[tokens * 128:] == 0x55).all()
    got_s = scales.cpu().numpy()
    assert np.array_equal(got_s[:tokens * 4].view(np.uint32),
                          want_s.reshape(-1)[:tokens].view(np.uint32))
    assert (got_s[tokens * 4:] == 0x55).all()
