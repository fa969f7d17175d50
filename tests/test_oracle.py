"""Pins of the CPU oracle (oracle/h3oracle.c) — CPU only.

The oracle is the checker of every HIP kernel, so it is itself checked here against what the
reference fixes: its own f64 test oracle on its closed-form inputs (tests/kernels.rs:1704-1849),
exact special cases (zero head, f16::MAX head), exactness of the fp32 Hadamard butterfly against
the dense Sylvester product, closed forms of attention, and independent numpy restatements.
Each plausible mistake in the quantizer (a sign, an order, a rounding mode, a scale) is planted
in a numpy copy to show that one of these pins fails on it.
"""
import math

import numpy as np
import pytest

import oracle as O

EXTRA = O.config_f32(O.EXTRA_Q_F64)


# --------------------------------------------------------------------- 16-bit formats

def test_half_to_float_matches_numpy_for_every_pattern():
    L = O.lib()
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([L.h3o_half_to_float(int(b)) for b in bits], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_float_to_half_rounds_to_nearest_even_like_numpy():
    L = O.lib()
    rng = np.random.default_rng(1)
    f = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(3.0),
        (rng.standard_normal(5000) * 1e-5).astype(np.float32),      # subnormal halves
        (rng.standard_normal(5000) * 6e4).astype(np.float32),       # near overflow
        # exact ties between adjacent halves
        ((np.arange(2000, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -10)),
        np.array([65504.0, 65519.99, 65520.0, -65520.0, 0.0, -0.0, np.inf, -np.inf], np.float32),
    ])
    want = f.astype(np.float16).view(np.uint16)
    got = np.array([L.h3o_float_to_half(float(x)) for x in f], np.uint16)
    assert np.array_equal(got, want)


# --------------------------------------------------------------------- quantizer

def np_hadamard_butterfly(y):
    """Independent numpy restatement of kernels/prepare_qk_i8.loom:84-156, rows of 128 f32."""
    y = y.astype(np.float32).reshape(-1, 32, 4)
    a, b, c, d = y[..., 0], y[..., 1], y[..., 2], y[..., 3]
    abp, abm, cdp, cdm = a + b, a - b, c + d, c - d
    s = np.stack([abp + cdp, abm + cdm, abp - cdp, abm - cdm], axis=-1)
    lanes = np.arange(32)
    for k in (1, 2, 4, 8, 16):
        p = s[:, lanes ^ k, :]
        hi = ((lanes & k) != 0)[None, :, None]
        s = np.where(hi, p - s, s + p)
    return s.reshape(-1, 128)


def np_quantize(r, extra, rounding=np.rint, scale_div=np.float32(127.0)):
    r = r.astype(np.float32)
    amax = np.maximum(np.abs(r).max(axis=1), np.float32(1e-30)).astype(np.float32)
    sc = (amax / scale_div).astype(np.float32)
    inv = (np.float32(127.0) / amax).astype(np.float32)
    q = np.clip(rounding((r * inv[:, None]).astype(np.float32)), -127, 127).astype(np.int8)
    words = q.view(np.uint8).reshape(-1, 32, 4).astype(np.uint32)
    words = words[..., 0] | (words[..., 1] << 8) | (words[..., 2] << 16) | (words[..., 3] << 24)
    return words.view(np.int32), (sc * np.float32(extra)).astype(np.float32)


def reference_case(tokens, heads):
    """tests/kernels.rs:1758-1769: values() inputs, mean with head 0 zeroed, head 0 all zeros,
    head 1 all f16::MAX when heads == 56."""
    d = 128
    stride = heads * d
    x = O.values(tokens * stride, 0.7).astype(np.float16).reshape(tokens, stride)
    mean = O.values(stride, 0.1)
    mean[:d] = 0.0
    x[:, :d] = 0
    if heads == 56:
        x[:, d:2 * d] = np.float16(65504.0)
    return np.ascontiguousarray(x).view(np.uint16), mean


@pytest.mark.parametrize("tokens,heads", [(37, 4), (3, 9), (3, 56)])
def test_quantizer_matches_reference_f64_oracle(tokens, heads):
    """tests/kernels.rs:1752-1810: fewer than 1/500 words differ (ties), scales 1e-7 + 1e-4 rel."""
    x, mean = reference_case(tokens, heads)
    codes, scales = O.prepare_qk(x, O.F16, mean, tokens, heads * 128, 0, heads, EXTRA)
    want_w, want_s, _ = O.prepared_qk_f64(x, mean, tokens, heads, O.EXTRA_Q_F64)
    differing = int((codes != want_w).sum())
    assert differing * 500 < codes.size, f"{differing} of {codes.size} words differ"
    np.testing.assert_allclose(scales.astype(np.float64), want_s.astype(np.float64),
                               rtol=1e-4, atol=1e-7)


@pytest.mark.parametrize("tokens,heads", [(37, 4), (3, 9), (3, 56)])
def test_quantizer_matches_independent_numpy_restatement_bit_exactly(tokens, heads):
    x, mean = reference_case(tokens, heads)
    codes, scales = O.prepare_qk(x, O.F16, mean, tokens, heads * 128, 0, heads, EXTRA)
    y = (O.widen(x, O.F16).reshape(tokens, heads * 128) - mean[None, :]).astype(np.float32)
    w, s = np_quantize(np_hadamard_butterfly(y.reshape(-1, 128)), EXTRA)
    assert np.array_equal(codes.reshape(-1), w.reshape(-1))
    assert np.array_equal(scales.reshape(-1).view(np.uint32), s.view(np.uint32))


def test_quantizer_special_heads():
    """Zero head -> codes 0 and scale 1e-30/127*extra; f16::MAX head -> H(65504*1) = 128*65504
    in element 0 only, code 127 there."""
    x, mean = reference_case(3, 56)
    codes, scales = O.prepare_qk(x, O.F16, mean, 3, 56 * 128, 0, 56, EXTRA)
    c = O.unpack(codes).reshape(3, 56, 128)
    assert (c[:, 0] == 0).all()
    assert np.array_equal(scales[:, 0], np.full(3, np.float32(np.float32(1e-30) / np.float32(127)) * np.float32(EXTRA), np.float32))
    # head 1: x = 65504 on every channel minus mean of head 1
    y = np.float32(65504.0) - mean[128:256]
    r = np_hadamard_butterfly(y[None, :])[0]
    assert c[0, 1, int(np.argmax(np.abs(r)))] in (127, -127)


def test_butterfly_equals_dense_sylvester_product_where_sums_are_exact():
    """For f16 inputs of one binade every fp32 partial sum is exact, so the butterfly must equal
    H_128 y with H[i][j] = (-1)^popcount(i&j) (tests/kernels.rs:1601-1608) bit for bit."""
    rng = np.random.default_rng(7)
    y = (rng.integers(-1024, 1024, size=(64, 128)).astype(np.float32) / np.float32(64.0))
    i = np.arange(128)
    H = np.where(np.vectorize(lambda v: bin(v).count("1") % 2)(i[:, None] & i[None, :]) == 1,
                 -1.0, 1.0)
    dense = y.astype(np.float64) @ H.T
    out = np.zeros(128, np.float32)
    for row in range(64):
        O.lib().h3o_hadamard128_f32(np.ascontiguousarray(y[row]), out)
        assert np.array_equal(out.astype(np.float64), dense[row])
    # H H = 128 I on the same exact inputs
    twice = np.zeros(128, np.float32)
    O.lib().h3o_hadamard128_f32(np.ascontiguousarray(y[0]), out)
    O.lib().h3o_hadamard128_f32(out.copy(), twice)
    assert np.array_equal(twice, y[0] * np.float32(128.0))


def test_head_major_is_a_relayout_of_token_major():
    """tests/kernels.rs:1812-1847."""
    tokens, heads = 37, 4
    x, mean = reference_case(tokens, heads)
    cap = -(-tokens // 32) * 32
    tw, ts = O.prepare_qk(x, O.F16, mean, tokens, heads * 128, 0, heads, EXTRA)
    hw, hs = O.prepare_qk(x, O.F16, mean, tokens, heads * 128, 0, heads, EXTRA, True, cap)
    hw = hw.reshape(heads, cap, 32)
    for h in range(heads):
        assert np.array_equal(hw[h, :tokens], tw.reshape(tokens, heads, 32)[:, h])
        assert np.array_equal(hs[h, :tokens], ts[:, h])
        assert (hw[h, tokens:] == 0).all() and (hs[h, tokens:] == 0).all()


def test_bf16_input_widens_exactly():
    rng = np.random.default_rng(3)
    f = rng.standard_normal((5, 256)).astype(np.float32)
    bits = O.bf16_bits(f)
    codes, scales = O.prepare_qk(bits, O.BF16, None, 5, 256, 0, 2, 1.0)
    y = O.widen(bits, O.BF16).reshape(-1, 128)
    w, s = np_quantize(np_hadamard_butterfly(y), 1.0)
    assert np.array_equal(codes.reshape(-1), w.reshape(-1))
    assert np.array_equal(scales.reshape(-1), s)


@pytest.mark.parametrize("mistake", ["sign", "order", "truncate", "scale", "lane"])
def test_planted_quantizer_mistakes_are_caught(mistake):
    """A copy of the quantizer with one plausible mistake fails the f64 pin or the numpy pin."""
    tokens, heads = 37, 4
    x, mean = reference_case(tokens, heads)
    y = (O.widen(x, O.F16).reshape(tokens, heads * 128) - mean[None, :]).astype(np.float32)
    y = y.reshape(-1, 128)
    rounding, scale_div = np.rint, np.float32(127.0)
    if mistake == "sign":      # lane with bit k set keeps s - partner instead of partner - s
        yy = y.reshape(-1, 32, 4)
        a, b, c, d = yy[..., 0], yy[..., 1], yy[..., 2], yy[..., 3]
        s = np.stack([a + b + c + d, a - b + c - d, a + b - c - d, a - b - c + d], -1)
        lanes = np.arange(32)
        for k in (1, 2, 4, 8, 16):
            p = s[:, lanes ^ k, :]
            s = np.where(((lanes & k) != 0)[None, :, None], s - p, s + p)
        r = s.reshape(-1, 128)
    elif mistake == "order":   # elements taken channel-transposed (e = l + 32 j)
        r = np_hadamard_butterfly(y.reshape(-1, 4, 32).transpose(0, 2, 1).reshape(-1, 128))
    elif mistake == "lane":    # butterflies applied in reverse lane order: same maths, other bits
        r = np_hadamard_butterfly(y)
        r = r.reshape(-1, 32, 4)[:, ::-1, :].reshape(-1, 128)
    else:
        r = np_hadamard_butterfly(y)
        if mistake == "truncate":
            rounding = np.trunc
        else:
            scale_div = np.float32(128.0)
    w, s = np_quantize(r, EXTRA, rounding, scale_div)
    want_w, want_s, _ = O.prepared_qk_f64(x, mean, tokens, heads, O.EXTRA_Q_F64)
    words_ok = int((w.reshape(-1) != want_w.reshape(-1)).sum()) * 500 < w.size
    scales_ok = np.allclose(s.astype(np.float64), want_s.reshape(-1).astype(np.float64),
                            rtol=1e-4, atol=1e-7)
    assert not (words_ok and scales_ok), f"planted mistake '{mistake}' passed the pins"


# --------------------------------------------------------------------- colmean

def test_colmean_is_the_sequential_f32_sum():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((300, 256)).astype(np.float16)
    bits = np.ascontiguousarray(x).view(np.uint16)
    got = O.colmean(bits, O.F16, 300, 256, 256)
    acc = np.add.accumulate(x.astype(np.float32), axis=0, dtype=np.float32)[-1]
    assert np.array_equal(got, (acc / np.float32(300)).astype(np.float32))


def test_colmean_exact_on_integers():
    x = (np.arange(64 * 256) % 17).astype(np.float16).reshape(64, 256)
    got = O.colmean(np.ascontiguousarray(x).view(np.uint16), O.F16, 64, 256, 256)
    want = (x.astype(np.float64).sum(0) / 64).astype(np.float32)
    assert np.array_equal(got, want)


# --------------------------------------------------------------------- RMSNorm + RoPE

def rope_inputs(tokens, heads, kv):
    """tests/kernels.rs:1135-1146."""
    stride = (heads + 2 * kv) * 128
    fused = O.values(tokens * stride, 0.7).astype(np.float16).reshape(tokens, stride)
    qw = (1.0 + O.values(128, 0.1)).astype(np.float32)
    kw = (qw + np.float32(0.05)).astype(np.float32)
    angles = O.values(tokens * 48, 3.0)
    return (np.ascontiguousarray(fused).view(np.uint16), qw, kw,
            np.cos(angles).astype(np.float32), np.sin(angles).astype(np.float32), stride)


def np_rope_f32(x_bits, fmt, tokens, row_stride, head_offset, heads, w, cos_t, sin_t, eps):
    """Independent numpy restatement of the fixed fp32 order of h3o_rope_qknorm_f16."""
    f32 = np.float32
    v = O.widen(x_bits, fmt).reshape(tokens, row_stride)[:, head_offset:head_offset + heads * 128]
    v = v.reshape(tokens, heads, 32, 4).astype(f32)
    sq = v * v
    part = ((sq[..., 0] + sq[..., 1]) + sq[..., 2]) + sq[..., 3]
    lanes = np.arange(32)
    for k in (1, 2, 4, 8, 16):
        part = part + part[..., lanes ^ k]
    ms = part[..., 0] * f32(0.0078125)
    r = (f32(1.0) / np.sqrt(ms + f32(eps))).astype(f32)
    xn = (v.reshape(tokens, heads, 128) * r[..., None]) * w[None, None, :]
    c = cos_t.reshape(tokens, 1, 48)
    s = sin_t.reshape(tokens, 1, 48)
    out = xn.copy()
    out[..., :48] = xn[..., :48] * c - xn[..., 48:96] * s
    out[..., 48:96] = xn[..., 48:96] * c + xn[..., :48] * s
    return out.astype(np.float16).view(np.uint16).reshape(tokens, heads * 128)


@pytest.mark.parametrize("heads,kv", [(4, 2), (56, 56), (12, 3)])
def test_rope_matches_reference_f64_oracle(heads, kv):
    """tests/kernels.rs:1125-1222: 2e-2 abs + 2e-2 rel against the f64 RMSNorm+RoPE."""
    tokens = 3
    fused, qw, kw, cos_t, sin_t, stride = rope_inputs(tokens, heads, kv)
    for off, count, w in ((0, heads, qw), (heads * 128, kv, kw)):
        got = O.rope_qknorm_f16(fused, O.F16, tokens, stride, off, count, w, cos_t, sin_t, 1e-5)
        want = O.rope_qknorm_f64(fused, O.F16, tokens, stride, off, count, w, cos_t, sin_t, 1e-5)
        g = got.view(np.float16).astype(np.float64).reshape(want.shape)
        assert np.all(np.abs(g - want) <= 2e-2 + 2e-2 * np.abs(want))
        mine = np_rope_f32(fused, O.F16, tokens, stride, off, count, w, cos_t, sin_t, 1e-5)
        assert np.array_equal(got, mine)


def test_rope_identity_rotation_is_rmsnorm():
    tokens, heads = 5, 2
    rng = np.random.default_rng(11)
    x = rng.standard_normal((tokens, heads * 128)).astype(np.float16)
    bits = np.ascontiguousarray(x).view(np.uint16)
    ones = np.ones(128, np.float32)
    cos_t = np.ones((tokens, 48), np.float32)
    sin_t = np.zeros((tokens, 48), np.float32)
    got = O.rope_qknorm_f16(bits, O.F16, tokens, heads * 128, 0, heads, ones, cos_t, sin_t, 1e-5)
    xf = x.astype(np.float64).reshape(tokens, heads, 128)
    want = xf / np.sqrt((xf ** 2).mean(-1, keepdims=True) + 1e-5)
    g = got.view(np.float16).astype(np.float64).reshape(tokens, heads, 128)
    assert np.all(np.abs(g - want) <= 1e-3 + 1e-3 * np.abs(want))


# --------------------------------------------------------------------- transpose

def test_transpose_moves_raw_bits_and_clears_the_tail():
    """tests/kernels.rs:3373-3444: raw half bits incl. NaN/Inf, zeroed tail, untouched beyond."""
    width, tokens, cap = 96, 33, 64
    inp = (np.arange(tokens * width, dtype=np.uint32) * 37).astype(np.uint16).reshape(tokens, width)
    out = np.full((width, cap), 0xFFFF, np.uint16)
    O.transpose(inp, O.F16, tokens, width, 0, width, cap, 48, out)
    assert np.array_equal(out[:, :tokens], inp.T)
    assert (out[:, tokens:48] == 0).all()
    assert (out[:, 48:] == 0xFFFF).all()


# --------------------------------------------------------------------- attention

def np_attention(qc, qs, kc, ks, vt, tokens, rows):
    """Brute force in numpy f64 (one head)."""
    s = (qc[rows].astype(np.float64) @ kc[:tokens].astype(np.float64).T)
    s = s * qs[rows, None].astype(np.float64) * ks[None, :tokens].astype(np.float64)
    p = np.exp(s - s.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    return p @ vt[:, :tokens].view(np.float16).astype(np.float64).T


def random_operands(rng, heads, tokens, cap):
    qc = np.zeros((heads, cap, 128), np.int8)
    kc = np.zeros((heads, cap, 128), np.int8)
    qc[:, :tokens] = np.clip(np.round(rng.standard_normal((heads, tokens, 128)) * 24), -127, 127)
    kc[:, :tokens] = np.clip(np.round(rng.standard_normal((heads, tokens, 128)) * 24), -127, 127)
    t = np.arange(cap)
    qs = np.tile(((1 + t % 7) / 512.0).astype(np.float32), (heads, 1))
    ks = np.tile(((1 + t % 3) / 128.0).astype(np.float32), (heads, 1))
    vt = np.zeros((heads * 128, cap), np.float16)
    vt[:, :tokens] = (rng.standard_normal((heads * 128, tokens)) * 0.3).astype(np.float16)
    return qc, qs, kc, ks, vt.view(np.uint16)


def test_attention_oracle_matches_numpy_brute_force():
    rng = np.random.default_rng(2)
    heads, tokens, cap = 2, 97, 128
    qc, qs, kc, ks, vt = random_operands(rng, heads, tokens, cap)
    rows = np.array([0, 5, 63, 96], np.int32)
    got = O.attention_f64(qc, qs, kc, ks, vt, tokens, cap, heads, rows)
    for h in range(heads):
        want = np_attention(qc[h], qs[h], kc[h], ks[h], vt[h * 128:(h + 1) * 128], tokens, rows)
        np.testing.assert_allclose(got[:, h], want, rtol=1e-12, atol=1e-12)


def test_attention_oracle_closed_forms():
    heads, tokens, cap = 1, 50, 64
    rng = np.random.default_rng(4)
    qc, qs, kc, ks, vt = random_operands(rng, heads, tokens, cap)
    v = vt[:, :tokens].view(np.float16).astype(np.float64)
    # identical keys and scales: uniform weights, output is the mean of V
    kc2 = np.repeat(kc[:, :1], cap, axis=1)
    ks2 = np.full_like(ks, 0.01)
    out = O.attention_f64(qc, qs, kc2, ks2, vt, tokens, cap, heads, np.arange(3, dtype=np.int32))
    np.testing.assert_allclose(out[:, 0], np.tile(v.mean(1), (3, 1)), rtol=1e-12, atol=1e-12)
    # one dominant key: the output is that key's V column
    kc3 = np.zeros_like(kc)
    qc3 = np.zeros_like(qc)
    qc3[0, 0] = 127
    kc3[0, 17] = 127
    qs3 = np.ones_like(qs)
    ks3 = np.ones_like(ks)
    out = O.attention_f64(qc3, qs3, kc3, ks3, vt, tokens, cap, heads, np.array([0], np.int32))
    np.testing.assert_allclose(out[0, 0], v[:, 17], rtol=0, atol=1e-12)


def test_capacity_formula():
    """src/stack.rs:299-302 at the BASELINE configs."""
    assert [O.capacity(t) for t in (1024, 31104, 129024, 130272)] == [1056, 31232, 129056, 130304]
    assert O.capacity(1) == 256 and O.capacity(4095) == 4128 and O.capacity(4096) == 4128
