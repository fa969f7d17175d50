"""The CPU oracle of the compact INT8 QKV projection, pinned on the CPU.

h3o_gemm_i8_qkv restates kernels/gemm_packed_256.loom (h3_gemm_i8_qkv_256) in the scalar form
of the reference's own test, compact_qkv_matches_scalar_projection_and_zeroes_v_padding
(tests/kernels.rs:4392-4460). It is checked here against
  - an independent numpy restatement (int64 dot products, float32 array arithmetic,
    astype(float16) rounding) on that test's closed-form inputs, for all of its row counts;
  - the facts that test asserts: the V^T padding columns are zero, NaN scales give NaN, an
    infinite scale gives +-inf (or NaN for a zero dot), and large finite values saturate at
    +-65472 instead of rounding to +-inf;
  - planted mistakes (a dropped clamp, a neighbouring token's scale, V left untransposed) that
    the numpy check must catch.
"""
import numpy as np
import pytest

import oracle as O


def reference_inputs(rows, k=64, n=384):
    """tests/kernels.rs:4396-4408 and 4410-4414."""
    i = np.arange(n * k)
    w = (((i * 17) % 255) - 127).astype(np.int8).reshape(n, k)
    ws = np.array([(c % 13 + 1) * 0.01 for c in range(n)], np.float32)
    ws[0] = 100.0
    ws[2 * n // 3] = 100.0
    ws[2 * n // 3 + 1] = np.inf
    ws[2 * n // 3 + 2] = np.nan
    j = np.arange(rows * k)
    a = (((j * 31) % 255) - 127).astype(np.int8).reshape(rows, k)
    scales = np.array([(r % 7 + 1) * 0.02 for r in range(rows)], np.float32)
    scales[0] = 50.0
    return a, w, ws, scales


def numpy_compact(a, w, ws, as_, k):
    """Independent restatement: exact int64 dots, then (dot*ws)*as + 0 in float32, clamp when
    finite, float16 rounding; laid out as Q/K rows then V^T with zero padding."""
    m, n = a.shape[0], w.shape[0]
    dot = a[:, :k].astype(np.int64) @ w[:, :k].astype(np.int64).T
    with np.errstate(invalid="ignore", over="ignore"):
        raw = (dot.astype(np.float32) * ws[None, :].astype(np.float32)) * as_[:, None].astype(np.float32)
        raw = raw + np.float32(0.0)
        fin = np.isfinite(raw)
        raw = np.where(fin, np.clip(raw, np.float32(-65472.0), np.float32(65472.0)), raw)
    h = raw.astype(np.float16).view(np.uint16)
    qk = 2 * (n // 3)
    cap = -(-m // 256) * 256
    vt = np.zeros((n // 3, cap), np.uint16)
    vt[:, :m] = h[:, qk:].T
    return np.concatenate([np.ascontiguousarray(h[:, :qk]).reshape(-1), vt.reshape(-1)])


def same_bits(got, want):
    """Bit equality, with any NaN matching any NaN (the reference asserts is_nan only)."""
    gf = got.view(np.float16)
    wf = want.view(np.float16)
    nan = np.isnan(wf)
    assert np.array_equal(np.isnan(gf), nan)
    bad = np.flatnonzero((got != want) & ~nan)
    assert bad.size == 0, f"{bad.size} mismatches, first at {bad[:5]}"


@pytest.mark.parametrize("rows", [1, 17, 255, 256, 257, 513])
def test_oracle_matches_numpy_on_the_reference_inputs(rows):
    a, w, ws, scales = reference_inputs(rows)
    got = O.gemm_i8_qkv(a, w, ws, scales, 64)
    same_bits(got, numpy_compact(a, w, ws, scales, 64))


def test_reference_assertions_hold():
    rows, n, k = 257, 384, 64
    a, w, ws, scales = reference_inputs(rows)
    out = O.gemm_i8_qkv(a, w, ws, scales, k)
    qk = 2 * n // 3
    cap = 512
    h = out[:rows * qk].reshape(rows, qk).view(np.float16)
    vt = out[rows * qk:].reshape(n // 3, cap)
    assert np.all(vt[:, rows:] == 0), "V^T padding must be zero"
    dot = a.astype(np.int64) @ w.astype(np.int64).T
    # column 2n/3 + 2 has a NaN scale: NaN everywhere
    assert np.all(np.isnan(vt[2].view(np.float16)[:rows]))
    # column 2n/3 + 1 has an infinite scale: +-inf, NaN where the dot is zero
    col = vt[1].view(np.float16)[:rows].astype(np.float32)
    d = dot[:, qk + 1]
    assert np.all(np.isinf(col[d != 0])) and np.all(np.sign(col[d != 0]) == np.sign(d[d != 0]))
    assert np.all(np.isnan(col[d == 0]))
    # row 0 (scale 50) x column 0 (scale 100): |dot| * 5000 > 65504 saturates at 65472
    assert abs(int(dot[0, 0])) * 5000 > 65520
    assert abs(float(h[0, 0])) == 65472.0


def test_padding_bytes_of_the_rows_are_ignored():
    rng = np.random.default_rng(7)
    m, n, k, stride = 300, 768, 192, 256
    a = rng.integers(-128, 128, (m, stride), dtype=np.int8)
    w = rng.integers(-128, 128, (n, stride), dtype=np.int8)
    ws = rng.uniform(1e-3, 2e-2, n).astype(np.float32)
    as_ = rng.uniform(1e-3, 5e-2, m).astype(np.float32)
    got = O.gemm_i8_qkv(a, w, ws, as_, k)
    same_bits(got, numpy_compact(a, w, ws, as_, k))
    a2 = a.copy()
    a2[:, k:] = 0x55
    w2 = w.copy()
    w2[:, k:] = -0x33
    assert np.array_equal(O.gemm_i8_qkv(a2, w2, ws, as_, k), got)


def test_planted_mistakes_are_caught():
    """The numpy check must fail on plausible slips: a dropped clamp, a row scale taken from
    the neighbouring token, and V stored untransposed."""
    rows, n, k = 257, 384, 64
    a, w, ws, scales = reference_inputs(rows)
    good = numpy_compact(a, w, ws, scales, k)
    same_bits(O.gemm_i8_qkv(a, w, ws, scales, k), good)
    qk = 2 * n // 3
    dot = a.astype(np.int64) @ w.astype(np.int64).T
    with np.errstate(invalid="ignore", over="ignore"):
        raw = (dot.astype(np.float32) * ws[None, :]) * scales[:, None] + np.float32(0)
        no_clamp = raw.astype(np.float16).view(np.uint16)
        shifted = ((dot.astype(np.float32) * ws[None, :]) * np.roll(scales, 1)[:, None]
                   ).astype(np.float16).view(np.uint16)
    for bad in (no_clamp, shifted):
        planted = good.copy()
        planted[:rows * qk] = bad[:, :qk].reshape(-1)
        with pytest.raises(AssertionError):
            same_bits(planted, good)
    untransposed = good.copy()
    vt = good[rows * qk:].reshape(n // 3, 512)
    untransposed[rows * qk:rows * qk + rows * (n // 3)] = vt[:, :rows].T.reshape(-1)
    with pytest.raises(AssertionError):
        same_bits(untransposed, good)
