"""Kernels against the committed golden vectors (tests/golden/*.npz), through the C ABI.

Quantizer and RoPE outputs must be bit-identical to the vectors; attention outputs must be within
the north-star tolerance (max-abs 2e-2, mean-abs 2e-3) and the reference's short-sequence bound
(1e-3 + 2e-3 relative, tests/kernels.rs:2004-2011).
"""
import pathlib
import sys

import numpy as np
import pytest

import h3attn as H
from helpers import north_star_ok, pack_codes, to_dev

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))
import make_golden as G  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("tokens,heads", [(37, 4), (3, 9), (3, 56)])
def test_quantizer_matches_vectors(dev, tokens, heads):
    import torch

    g = np.load(GOLDEN / f"prepare_qk_i8_t{tokens}_h{heads}.npz")
    x, mean = G.quantizer_case(tokens, heads)
    cfg = H.PrepareCfg(heads * 128, 0, heads, G.EXTRA, 0, 1e-5, H.H3_ELEM_F16)
    codes = torch.zeros(tokens * heads * 32, dtype=torch.int32, device=dev)
    scales = torch.zeros(tokens * heads, dtype=torch.float32, device=dev)
    H.prepare_qk_i8(cfg, tokens, to_dev(x, dev), to_dev(mean, dev), codes, scales)
    torch.cuda.synchronize()
    assert np.array_equal(codes.cpu().numpy(), g["codes"].reshape(-1))
    assert np.array_equal(scales.cpu().numpy().view(np.uint32), g["scales"].reshape(-1).view(np.uint32))


@pytest.mark.parametrize("tokens,heads", [(3, 2), (129, 4)])
def test_rope_routes_match_vectors(dev, tokens, heads):
    import torch

    g = np.load(GOLDEN / f"rope_t{tokens}_h{heads}.npz")
    fused, w, cos_t, sin_t = G.rope_case(tokens, heads)
    width = heads * 128
    cap = int(g["capacity"])
    f_d, w_d = to_dev(fused, dev), to_dev(w, dev)
    c_d, s_d = to_dev(cos_t, dev), to_dev(sin_t, dev)
    # separate route: f16 rotated Q and K
    rc = H.RopeCfg(3 * width, heads, heads, width, 1e-5, 0, H.H3_ELEM_F16)
    q16 = torch.zeros(tokens * width, dtype=torch.int16, device=dev)
    k16 = torch.zeros(tokens * width, dtype=torch.int16, device=dev)
    H.rope_qknorm_f16(rc, tokens, f_d, w_d, w_d, c_d, s_d, q16, k16)
    # fused route: RoPE + quantizer straight to head-major operands
    pq = H.PrepareCfg(3 * width, 0, heads, G.EXTRA, cap, 1e-5, H.H3_ELEM_F16)
    pk = H.PrepareCfg(3 * width, width, heads, 1.0, cap, 1e-5, H.H3_ELEM_F16)
    qw = torch.zeros(heads * cap * 32, dtype=torch.int32, device=dev)
    kw = torch.zeros_like(qw)
    qs = torch.zeros(heads * cap, dtype=torch.float32, device=dev)
    ks = torch.zeros_like(qs)
    H.prepare_qk_rope_i8hm(pq, tokens, f_d, w_d, c_d, s_d, qw, qs)
    H.prepare_qk_rope_i8hm(pk, tokens, f_d, w_d, c_d, s_d, kw, ks)
    torch.cuda.synchronize()
    assert np.array_equal(q16.cpu().numpy().view(np.uint16), g["q"].reshape(-1))
    assert np.array_equal(k16.cpu().numpy().view(np.uint16), g["k"].reshape(-1))
    assert np.array_equal(qw.cpu().numpy(), g["qcodes"].reshape(-1))
    assert np.array_equal(qs.cpu().numpy().view(np.uint32), g["qscales"].reshape(-1).view(np.uint32))
    assert np.array_equal(kw.cpu().numpy(), g["kcodes"].reshape(-1))
    assert np.array_equal(ks.cpu().numpy().view(np.uint32), g["kscales"].reshape(-1).view(np.uint32))


@pytest.mark.parametrize("tokens,heads,seed", [(23, 2, 3), (97, 2, 4)])
def test_attention_matches_vectors(dev, tokens, heads, seed):
    import torch

    g = np.load(GOLDEN / f"attention_i8qkhm_t{tokens}_h{heads}.npz")
    qc, qs, kc, ks, vt, cap = G.attention_case(tokens, heads, seed)
    cfg = H.AttentionCfg(heads * 128, heads * 128, heads * 128, tokens, cap, 1.0)
    out = torch.zeros(tokens * heads * 128, dtype=torch.float16, device=dev)
    H.attention_i8qkhm(cfg, tokens, heads, to_dev(pack_codes(qc).reshape(-1), dev), to_dev(qs, dev),
                       to_dev(pack_codes(kc).reshape(-1), dev), to_dev(ks, dev), to_dev(vt, dev), out)
    torch.cuda.synchronize()
    got = out.cpu().numpy().astype(np.float64).reshape(tokens, heads, 128)
    want = g["out"].astype(np.float64)
    assert np.all(np.abs(got - want) <= 1e-3 + 2e-3 * np.abs(want))
    mx, mean = north_star_ok(got, want)
    assert mx <= 2e-2 and mean <= 2e-3
