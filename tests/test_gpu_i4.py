"""The INT4 QK family on the GPU through the C ABI (h3_prepare_qk_i4, h3_attention_i4qk).

  - the quantizer is bit-exact against the oracle (kernels/prepare_qk_i4.loom) at the shapes the
    int8 quantizer is tested at, with and without a mean, f16 and bf16;
  - the attention reproduces the reference's packed_attention_families test inputs
    (tests/kernels.rs:2335-2460: 97 tokens, 2 heads, codes ((i*37 + seed) % 7) - 3, scales 0.02,
    V = values(0.3)) against the f64 attention of the operands, at the reference's bound and the
    north-star tolerance;
  - int4 attention agrees with the int8 token-major attention run on the same codes widened to
    int8 to a few f16 ulps, and both match the f64 attention of the codes (the int4 kernel
    computes 256x the dot product and folds 1/256 into the query scale; the dequantisation's
    -1.5*2^23*ks term carries the same rounding error in both, relatively 256x smaller in int4,
    so the two are not bit-identical);
  - quantizer + attention at BASELINE config 2's token count on sampled rows;
  - the skip twin (h3_attention_i4qks): with the reference test's tau = 1000 it equals the
    unskipped kernel bit for bit, with tau = 0 its output is finite (tests/kernels.rs:2420-2455),
    and on inputs whose 64-key tiles have clearly separated scores it drops exactly the tiles
    the rule gap < -tau names (the output equals the attention over the kept tiles and differs
    from the full attention).
"""
import numpy as np
import pytest

import h3attn as H
import oracle as O
from helpers import from_dev, north_star_ok, to_dev

pytestmark = pytest.mark.gpu


def pack_i4(codes: np.ndarray) -> np.ndarray:
    """int8 codes in [-8, 7], last axis a multiple of 8 -> i32 words, low nibble first."""
    c = (np.ascontiguousarray(codes, np.int8).astype(np.int64) & 15).astype(np.uint32)
    c = c.reshape(*c.shape[:-1], -1, 8)
    w = np.zeros(c.shape[:-1], np.uint32)
    for j in range(8):
        w |= c[..., j] << np.uint32(4 * j)
    return w.view(np.int32)


@pytest.mark.parametrize("tokens,heads,offset,extra,mean", [
    (1, 1, 0, 1.0, False), (37, 4, 0, 0.25, True), (257, 17, 128, 1.0, True),
    (2049, 56, 128, 0.5, False), (3, 256, 0, 1.0, True)])
@pytest.mark.parametrize("elem", [H.H3_ELEM_F16, H.H3_ELEM_BF16])
def test_prepare_qk_i4_is_bit_exact(dev, tokens, heads, offset, extra, mean, elem):
    import torch

    rng = np.random.default_rng(tokens * 7 + heads)
    stride = offset + heads * 128 + 128
    v = (rng.standard_normal((tokens, stride)) * 1.5).astype(np.float32)
    fmt = O.F16 if elem == H.H3_ELEM_F16 else O.BF16
    x = (O.f16_bits(v) if fmt == O.F16 else O.bf16_bits(v)).reshape(tokens, stride)
    m = rng.standard_normal(stride).astype(np.float32) if mean else None
    wc, ws = O.prepare_qk_i4(x, fmt, m, tokens, stride, offset, heads, extra)
    codes = torch.full((tokens * heads * 16,), -1, dtype=torch.int32, device=dev)
    scales = torch.full((tokens * heads,), -1.0, dtype=torch.float32, device=dev)
    cfg = H.PrepareCfg(stride, offset, heads, extra, 32, 1e-5, elem)
    print(f"prepare_qk_i4 tokens={tokens} heads={heads}", flush=True)
    H.prepare_qk_i4(cfg, tokens, to_dev(x, dev), None if m is None else to_dev(m, dev), codes,
                    scales)
    assert np.array_equal(from_dev(codes).reshape(tokens, heads * 16), wc)
    assert np.array_equal(from_dev(scales).view(np.uint32).reshape(tokens, heads),
                          ws.view(np.uint32))


def reference_i4_inputs(tokens=97, heads=2, waves=8):
    """tests/kernels.rs:2346-2392."""
    d = 128
    block = 16 * waves
    cap = -(-(tokens + 16) // block) * block
    stride = heads * d
    i = np.arange(cap * stride)

    def codes(seed):
        c = (((i * 37 + seed) % 7) - 3).astype(np.int8)
        c[i // stride >= tokens] = 0
        return c.reshape(cap, stride)

    q, k = codes(1), codes(3)
    scales = np.where(np.arange(cap * heads) // heads < tokens, 0.02, 0.0).astype(np.float32)
    scales = scales.reshape(cap, heads)
    v = O.f16_bits(O.values(tokens * stride, 0.3)).reshape(tokens, stride)
    vt = O.transpose(v, O.F16, tokens, stride, 0, stride, cap, cap)
    return q, k, scales, vt, cap, stride


def run_i4(dev, q, qs, k, ks, vt, tokens, cap, heads, kernel):
    import torch

    stride = heads * 128
    cfg = H.AttentionCfg(stride, stride, stride, tokens, cap, 1.0)
    out = torch.zeros((tokens, stride), dtype=torch.float16, device=dev)
    kernel(cfg, tokens, heads, to_dev(q, dev), to_dev(qs, dev), to_dev(k, dev), to_dev(ks, dev),
           to_dev(vt, dev), out)
    torch.cuda.synchronize()
    return from_dev(out)


@pytest.mark.parametrize("waves", [4, 8])
def test_reference_packed_i4_inputs(dev, waves):
    tokens, heads = 97, 2
    q, k, scales, vt, cap, stride = reference_i4_inputs(tokens, heads, waves)
    got = run_i4(dev, pack_i4(q), scales, pack_i4(k), scales, vt, tokens, cap, heads,
                 H.attention_i4qk)
    got = got.view(np.float16).astype(np.float64).reshape(tokens, heads, 128)
    qc = q.reshape(cap, heads, 128).transpose(1, 0, 2).copy()
    kc = k.reshape(cap, heads, 128).transpose(1, 0, 2).copy()
    want = O.attention_f64(qc, scales.T.copy(), kc, scales.T.copy(), vt, tokens, cap, heads,
                           np.arange(tokens))
    # the reference's bound (close(got, want, 3e-4, 0.03)) and the north-star tolerance
    assert np.all(np.abs(got - want) <= 3e-4 + 0.03 * np.abs(want))
    mx, mean = north_star_ok(got, want)
    assert mx <= 2e-2 and mean <= 2e-3


@pytest.mark.parametrize("tokens", [23, 97, 1000, 4097])
def test_i4_attention_agrees_with_int8_attention_on_widened_codes(dev, tokens):
    heads = 3
    rng = np.random.default_rng(tokens)
    stride = heads * 128
    cap = H.capacity(tokens)
    q = rng.integers(-7, 8, (cap, stride)).astype(np.int8)
    k = rng.integers(-7, 8, (cap, stride)).astype(np.int8)
    q[tokens:] = 0
    k[tokens:] = 0
    qs = rng.uniform(0.01, 0.05, (cap, heads)).astype(np.float32)
    ks = rng.uniform(0.01, 0.05, (cap, heads)).astype(np.float32)
    v = O.f16_bits(rng.standard_normal((tokens, stride)).astype(np.float32)).reshape(tokens, stride)
    vt = O.transpose(v, O.F16, tokens, stride, 0, stride, cap, cap)
    print(f"i4 vs i8 tokens={tokens}", flush=True)
    got4 = run_i4(dev, pack_i4(q), qs, pack_i4(k), ks, vt, tokens, cap, heads, H.attention_i4qk)
    got8 = run_i4(dev, q.view(np.int32), qs, k.view(np.int32), ks, vt, tokens, cap, heads,
                  H.attention_i8qk)
    a4 = got4.view(np.float16).astype(np.float64)
    a8 = got8.view(np.float16).astype(np.float64)
    assert np.all(np.abs(a4 - a8) <= 2e-3 + 4e-3 * np.abs(a8))
    rows = np.unique(np.linspace(0, tokens - 1, 9).astype(np.int32))
    qc = q.reshape(cap, heads, 128).transpose(1, 0, 2).copy()
    kc = k.reshape(cap, heads, 128).transpose(1, 0, 2).copy()
    want = O.attention_f64(qc, qs.T.copy(), kc, ks.T.copy(), vt, tokens, cap, heads, rows)
    for got in (a4, a8):
        mx, mean = north_star_ok(got.reshape(tokens, heads, 128)[rows], want)
        assert mx <= 2e-2 and mean <= 2e-3, (mx, mean)


def test_i4_path_at_config2_tokens_on_sampled_rows(dev):
    """Quantize N(0,1) Q and K (K with a per-channel offset, smoothed by its column mean) to int4
    on the GPU, attend, and compare sampled rows with the f64 attention of those operands."""
    import torch

    tokens, heads = 31104, 4
    stride = heads * 128
    cap = H.capacity(tokens)
    g = torch.Generator(device=dev).manual_seed(5)
    q = torch.randn((tokens, stride), generator=g, device=dev).half()
    k = (torch.randn((tokens, stride), generator=g, device=dev)
         + torch.randn((stride,), generator=g, device=dev) * 1.4).half()
    v = torch.randn((tokens, stride), generator=g, device=dev).half()
    mean = torch.empty(stride, dtype=torch.float32, device=dev)
    H.colmean_f32(stride, tokens, k, mean)
    qi = torch.zeros((cap, stride // 8), dtype=torch.int32, device=dev)
    ki = torch.zeros_like(qi)
    qs = torch.zeros((cap, heads), dtype=torch.float32, device=dev)
    ks = torch.zeros_like(qs)
    extra = O.config_f32(O.EXTRA_Q_F64)
    H.prepare_qk_i4(H.PrepareCfg(stride, 0, heads, extra, 32, 1e-5, H.H3_ELEM_F16), tokens, q,
                    None, qi, qs)
    H.prepare_qk_i4(H.PrepareCfg(stride, 0, heads, 1.0, 32, 1e-5, H.H3_ELEM_F16), tokens, k,
                    mean, ki, ks)
    vt = torch.zeros((stride, cap), dtype=torch.float16, device=dev)
    H.transpose_f16(H.TransposeCfg(stride, cap, H.H3_ELEM_F16), cap, tokens, v, vt)
    out = torch.zeros((tokens, stride), dtype=torch.float16, device=dev)
    cfg = H.AttentionCfg(stride, stride, stride, tokens, cap, 1.0)
    print("i4 config-2 tokens", flush=True)
    H.attention_i4qk(cfg, tokens, heads, qi, qs, ki, ks, vt, out)
    torch.cuda.synchronize()
    # the GPU operands equal the oracle quantizer's on sampled rows
    rows = np.array([0, 1, 4096, tokens // 2, tokens - 1])
    xq = from_dev(q)[rows]
    wq, sq = O.prepare_qk_i4(xq, O.F16, None, len(rows), stride, 0, heads, extra)
    assert np.array_equal(from_dev(qi)[rows], wq) and np.array_equal(qs.cpu().numpy()[rows], sq)
    qc = O.unpack_i4(from_dev(qi)).reshape(cap, heads, 128).transpose(1, 0, 2).copy()
    kc = O.unpack_i4(from_dev(ki)).reshape(cap, heads, 128).transpose(1, 0, 2).copy()
    want = O.attention_f64(qc, qs.cpu().numpy().T.copy(), kc, ks.cpu().numpy().T.copy(),
                           from_dev(vt), tokens, cap, heads, rows.astype(np.int32))
    got = from_dev(out).view(np.float16).astype(np.float64).reshape(tokens, heads, 128)[rows]
    mx, mean_err = north_star_ok(got, want)
    assert mx <= 2e-2 and mean_err <= 2e-3, (mx, mean_err)


def skip_run(dev, q, qs, k, ks, vt, tokens, cap, heads, tau):
    import torch

    stride = heads * 128
    cfg = H.AttentionSkipCfg(stride, stride, stride, tokens, cap, 1.0, tau)
    out = torch.zeros((tokens, stride), dtype=torch.float16, device=dev)
    H.attention_i4qks(cfg, tokens, heads, to_dev(q, dev), to_dev(qs, dev), to_dev(k, dev),
                      to_dev(ks, dev), to_dev(vt, dev), out)
    torch.cuda.synchronize()
    return from_dev(out)


@pytest.mark.parametrize("tokens", [97, 4097])
def test_skip_twin_with_large_tau_equals_the_unskipped_kernel(dev, tokens):
    heads = 2
    rng = np.random.default_rng(tokens + 11)
    stride = heads * 128
    cap = H.capacity(tokens)
    q = rng.integers(-7, 8, (cap, stride)).astype(np.int8)
    k = rng.integers(-7, 8, (cap, stride)).astype(np.int8)
    q[tokens:] = 0
    k[tokens:] = 0
    qs = rng.uniform(0.005, 0.03, (cap, heads)).astype(np.float32)
    ks = rng.uniform(0.005, 0.03, (cap, heads)).astype(np.float32)
    v = O.f16_bits(rng.standard_normal((tokens, stride)).astype(np.float32)).reshape(tokens, stride)
    vt = O.transpose(v, O.F16, tokens, stride, 0, stride, cap, cap)
    print(f"skip twin tau=1000 tokens={tokens}", flush=True)
    got = skip_run(dev, pack_i4(q), qs, pack_i4(k), ks, vt, tokens, cap, heads, 1000.0)
    base = run_i4(dev, pack_i4(q), qs, pack_i4(k), ks, vt, tokens, cap, heads, H.attention_i4qk)
    assert np.array_equal(got, base)
    zero = skip_run(dev, pack_i4(q), qs, pack_i4(k), ks, vt, tokens, cap, heads, 0.0)
    assert np.all(np.isfinite(zero.view(np.float16)))


def test_skip_twin_drops_exactly_the_far_tiles(dev):
    """Six 64-key tiles with uniform scores 10, 8.5, 9.8, 5, 10.2, 9 (natural units) for every
    query; tau = 0.5 drops tiles 1, 3 and 5 (gaps -1.5, -5 and -1.2) and keeps 0, 2 and 4."""
    heads, tokens = 1, 384
    stride = 128
    cap = H.capacity(tokens)
    rng = np.random.default_rng(2)
    c = (rng.integers(0, 2, 128) * 14 - 7).astype(np.int8)  # +-7
    dot = float(np.dot(c.astype(np.int64), c.astype(np.int64)))  # 6272
    q = np.zeros((cap, stride), np.int8)
    k = np.zeros((cap, stride), np.int8)
    q[:tokens] = c
    k[:tokens] = c
    scores = [10.0, 8.5, 9.8, 5.0, 10.2, 9.0]
    qs = np.zeros((cap, 1), np.float32)
    ks = np.zeros((cap, 1), np.float32)
    qs[:tokens] = 1.0
    for t, sc in enumerate(scores):
        ks[64 * t:64 * t + 64] = np.float32(sc / dot)
    v = O.f16_bits(rng.standard_normal((tokens, stride)).astype(np.float32)).reshape(tokens, stride)
    vt = O.transpose(v, O.F16, tokens, stride, 0, stride, cap, cap)
    got = skip_run(dev, pack_i4(q), qs, pack_i4(k), ks, vt, tokens, cap, heads, 0.5)
    got = got.view(np.float16).astype(np.float64).reshape(tokens, 1, 128)
    kept = ks.copy()
    for t in (1, 3, 5):
        kept[64 * t:64 * t + 64] = -np.inf
    rows = np.array([0, 31, 32, 200, 383], np.int32)
    qc = q.reshape(cap, 1, 128).transpose(1, 0, 2).copy()
    kc = k.reshape(cap, 1, 128).transpose(1, 0, 2).copy()
    want = O.attention_f64(qc, qs.T.copy(), kc, kept.T.copy(), vt, tokens, cap, 1, rows)
    full = O.attention_f64(qc, qs.T.copy(), kc, ks.T.copy(), vt, tokens, cap, 1, rows)
    mx, mean = north_star_ok(got[rows], want)
    assert mx <= 2e-2 and mean <= 2e-3, (mx, mean)
    assert np.abs(full - want).max() > 0.05  # the dropped tiles carry real weight


@pytest.mark.parametrize("tokens,heads", [(97, 2), (1000, 3), (4097, 2)])
def test_workspace_forms_are_bit_identical(dev, tokens, heads):
    """h3_attention_i4qk_ws, h3_attention_i4qks_ws and h3_attention_i8qk_ws read the key scales
    from a head-major copy in a lent (NaN-filled) workspace: the outputs equal those of the forms
    without _ws bit for bit."""
    import torch

    rng = np.random.default_rng(tokens * 7 + heads)
    stride = heads * 128
    cap = H.capacity(tokens)
    q = rng.integers(-7, 8, (cap, stride)).astype(np.int8)
    k = rng.integers(-7, 8, (cap, stride)).astype(np.int8)
    q[tokens:] = 0
    k[tokens:] = 0
    qs = rng.uniform(0.005, 0.05, (cap, heads)).astype(np.float32)
    ks = rng.uniform(0.005, 0.05, (cap, heads)).astype(np.float32)
    v = O.f16_bits(rng.standard_normal((tokens, stride)).astype(np.float32)).reshape(tokens, stride)
    vt = O.transpose(v, O.F16, tokens, stride, 0, stride, cap, cap)
    cfg = H.AttentionCfg(stride, stride, stride, tokens, cap, 1.0)
    scfg = H.AttentionSkipCfg(stride, stride, stride, tokens, cap, 1.0, 1.5)
    nbytes = H.scales_workspace_bytes(cfg)
    assert nbytes == heads * tokens * 4 and H.scales_workspace_bytes(scfg) == nbytes
    ops = [(pack_i4(q), pack_i4(k), H.attention_i4qk, H.attention_i4qk_ws, cfg),
           (pack_i4(q), pack_i4(k), H.attention_i4qks, H.attention_i4qks_ws, scfg),
           (q.view(np.int32), k.view(np.int32), H.attention_i8qk, H.attention_i8qk_ws, cfg)]
    for qq, kk, plain, lent, c in ops:
        print(f"ws form {plain.__name__} tokens={tokens} heads={heads}", flush=True)
        args = (c, tokens, heads, to_dev(qq, dev), to_dev(qs, dev), to_dev(kk, dev),
                to_dev(ks, dev), to_dev(vt, dev))
        a = torch.zeros((tokens, stride), dtype=torch.float16, device=dev)
        b = torch.zeros_like(a)
        plain(*args, a)
        ws = torch.full((nbytes // 2,), 0x7E00, dtype=torch.int16, device=dev)
        lent(*args, b, ws)
        torch.cuda.synchronize()
        assert np.isfinite(from_dev(b).view(np.float16)).all()
        assert np.array_equal(from_dev(a), from_dev(b)), plain.__name__
