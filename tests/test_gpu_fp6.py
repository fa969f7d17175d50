"""The FP6 form of the int4 attention (h3_attention_i4qk_fp6) on the GPU through the C ABI.

  - the workspace it converts into holds, bit for bit, the FP6 rows restated in tests/helpers.py
    (each nibble c as the E2M3 code of c/2, -8 included) and the head-major scales (key scales
    times 4), and rows past `tokens` are left alone;
  - its output matches the f64 attention of the int4 codes (h3o_attention_f64) at the north-star
    tolerance, with codes over the whole signed-nibble range -8..7, across 64-key tile edges and
    past the 64-stage limit of the chained mode, and agrees with h3_attention_i4qk (the int8-MFMA
    int4 kernel) to a few f16 ulps;
  - the reference's packed int4 test inputs (tests/kernels.rs:2335-2392) meet its bound;
  - rows at or past token_count are not written.
"""
import numpy as np
import pytest

import h3attn as H
import oracle as O
from helpers import from_dev, fp6_rows, north_star_ok, read_device, to_dev
from test_gpu_i4 import pack_i4, reference_i4_inputs

pytestmark = pytest.mark.gpu


def operands(rng, tokens, heads, cap, lo=-8):
    stride = heads * 128
    q = rng.integers(lo, 8, (cap, stride)).astype(np.int8)
    k = rng.integers(lo, 8, (cap, stride)).astype(np.int8)
    q[tokens:] = 0
    k[tokens:] = 0
    qs = rng.uniform(0.01, 0.05, (cap, heads)).astype(np.float32)
    ks = rng.uniform(0.01, 0.05, (cap, heads)).astype(np.float32)
    v = O.f16_bits(rng.standard_normal((tokens, stride)).astype(np.float32)).reshape(tokens, stride)
    vt = O.transpose(v, O.F16, tokens, stride, 0, stride, cap, cap)
    return q, k, qs, ks, vt


def run_fp6(dev, q, qs, k, ks, vt, tokens, cap, heads, token_count=None, ws=None):
    import torch

    stride = heads * 128
    token_count = tokens if token_count is None else token_count
    cfg = H.AttentionCfg(stride, stride, stride, tokens, cap, 1.0)
    if ws is None:
        ws = torch.full((H.fp6_workspace_bytes(cfg) // 2,), 0x7E00, dtype=torch.int16, device=dev)
    out = torch.full((token_count, stride), float("nan"), dtype=torch.float16, device=dev)
    H.attention_i4qk_fp6(cfg, token_count, heads, to_dev(pack_i4(q), dev), to_dev(qs, dev),
                         to_dev(pack_i4(k), dev), to_dev(ks, dev), to_dev(vt, dev), out, ws)
    torch.cuda.synchronize()
    return from_dev(out), ws, cfg


def oracle_rows(q, qs, k, ks, vt, tokens, cap, heads, rows):
    qc = q.reshape(cap, heads, 128).transpose(1, 0, 2).copy()
    kc = k.reshape(cap, heads, 128).transpose(1, 0, 2).copy()
    return O.attention_f64(qc, qs.T.copy(), kc, ks.T.copy(), vt, tokens, cap, heads,
                           np.asarray(rows, np.int32))


def test_workspace_holds_the_converted_operands(dev):
    tokens, heads = 97, 3
    cap = H.capacity(tokens)
    rng = np.random.default_rng(1)
    q, k, qs, ks, vt = operands(rng, tokens, heads, cap)
    q[5, :128] = -8
    print("fp6 workspace", flush=True)
    _, ws, cfg = run_fp6(dev, q, qs, k, ks, vt, tokens, cap, heads)
    raw = from_dev(ws).view(np.uint8)
    r = lambda x: (x + 255) // 256 * 256
    off_k = r(heads * cap * 128)
    off_qs = off_k + r(heads * cap * 128)
    off_ks = off_qs + r(heads * cap * 4)
    for off, codes in ((0, q), (off_k, k)):
        got = raw[off:off + heads * cap * 128].reshape(heads, cap, 128)
        want = fp6_rows(pack_i4(codes), heads, tokens, cap).reshape(heads, cap, 128)
        assert np.array_equal(got[:, :tokens], want[:, :tokens])
        assert np.all(got[:, tokens:].view(np.uint16) == 0x7E00)  # rows past tokens untouched
    for off, s, mult in ((off_qs, qs, 1.0), (off_ks, ks, 4.0)):
        got = raw[off:off + heads * cap * 4].view(np.float32).reshape(heads, cap)
        assert np.array_equal(got[:, :tokens], (s[:tokens] * np.float32(mult)).T)


@pytest.mark.parametrize("tokens", [23, 97, 1000, 4097, 8193])
def test_fp6_attention_matches_the_oracle(dev, tokens):
    heads = 3
    cap = H.capacity(tokens)
    rng = np.random.default_rng(tokens + 7)
    q, k, qs, ks, vt = operands(rng, tokens, heads, cap)
    print(f"fp6 attention tokens={tokens}", flush=True)
    got, _, cfg = run_fp6(dev, q, qs, k, ks, vt, tokens, cap, heads)
    a6 = got.view(np.float16).astype(np.float64)
    assert np.isfinite(a6).all()
    rows = np.unique(np.linspace(0, tokens - 1, 9).astype(np.int32))
    want = oracle_rows(q, qs, k, ks, vt, tokens, cap, heads, rows)
    mx, mean = north_star_ok(a6.reshape(tokens, heads, 128)[rows], want)
    print(f"  max {mx:.3e} mean {mean:.3e}", flush=True)
    assert mx <= 2e-2 and mean <= 2e-3, (mx, mean)
    # against the int8-MFMA int4 kernel on the same operands
    import torch

    out4 = torch.zeros((tokens, heads * 128), dtype=torch.float16, device=dev)
    H.attention_i4qk(cfg, tokens, heads, to_dev(pack_i4(q), dev), to_dev(qs, dev),
                     to_dev(pack_i4(k), dev), to_dev(ks, dev), to_dev(vt, dev), out4)
    a4 = from_dev(out4).view(np.float16).astype(np.float64)
    assert np.all(np.abs(a6 - a4) <= 2e-3 + 4e-3 * np.abs(a4))


@pytest.mark.parametrize("waves", [4, 8])
def test_fp6_reference_packed_i4_inputs(dev, waves):
    tokens, heads = 97, 2
    q, k, scales, vt, cap, stride = reference_i4_inputs(tokens, heads, waves)
    got, _, _ = run_fp6(dev, q, scales, k, scales, vt, tokens, cap, heads)
    got = got.view(np.float16).astype(np.float64).reshape(tokens, heads, 128)
    want = oracle_rows(q, scales, k, scales, vt, tokens, cap, heads, np.arange(tokens))
    assert np.all(np.abs(got - want) <= 3e-4 + 0.03 * np.abs(want))
    mx, mean = north_star_ok(got, want)
    assert mx <= 2e-2 and mean <= 2e-3


def test_fp6_token_count_limits_the_rows_written(dev):
    tokens, heads = 700, 2
    cap = H.capacity(tokens)
    rng = np.random.default_rng(9)
    q, k, qs, ks, vt = operands(rng, tokens, heads, cap)
    full, _, _ = run_fp6(dev, q, qs, k, ks, vt, tokens, cap, heads)
    part, _, _ = run_fp6(dev, q, qs, k, ks, vt, tokens, cap, heads, token_count=300)
    assert np.array_equal(part, full[:300])
