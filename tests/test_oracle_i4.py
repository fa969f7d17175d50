"""The int4 quantizer of the CPU oracle (h3o_prepare_qk_i4_f32, kernels/prepare_qk_i4.loom), pinned.

The rotation is the int8 quantizer's H_128 butterfly (pinned in test_oracle.py); here:
  - known answers: a one-hot head row rotates to +-A in the Sylvester sign pattern
    H[i][k] = (-1)^popcount(i & k), so its codes are exactly +-7, packed eight per word with the
    low nibble first (the packing the reference's own int4 attention test builds,
    tests/kernels.rs:2366-2375);
  - an independent numpy quantisation (amax, /7, rint, clamp, nibbles) of the oracle's pinned
    rotation, bit for bit, on random rows with and without a mean, f16 and bf16;
  - the scale is amax/7 * extra for the same amax the int8 quantizer finds (int8 scale * 127);
  - a planted mistake (high nibble first) is caught, and codes reach but never pass +-7.
"""
import numpy as np
import pytest

import oracle as O


def sylvester(i, k):
    return np.where(np.vectorize(lambda v: bin(v).count("1") % 2)(i & k) == 0, 1, -1)


def rotate(y):
    r = np.zeros(128, np.float32)
    O.lib().h3o_hadamard128_f32(np.ascontiguousarray(y, np.float32), r)
    return r


def numpy_quantize(r, extra, high_first=False, qmax=7):
    amax = np.float32(max(np.max(np.abs(r)), np.float32(1e-30)))
    sc = np.float32(amax / np.float32(7.0))
    inv = np.float32(np.float32(7.0) / amax)
    q = np.clip(np.rint(r * inv), -qmax, qmax).astype(np.int64) & 15
    words = np.zeros(16, np.uint32)
    for e in range(128):
        nib = (7 - e % 8) if high_first else e % 8
        words[e // 8] |= np.uint32(q[e]) << np.uint32(4 * nib)
    return words.view(np.int32), np.float32(sc * np.float32(extra))


@pytest.mark.parametrize("k", [0, 1, 5, 64, 127])
def test_one_hot_row_gives_sylvester_signs(k):
    x = np.zeros((1, 128), np.float32)
    x[0, k] = 3.0
    codes, scales = O.prepare_qk_i4(O.f16_bits(x).reshape(1, 128), O.F16, None, 1, 128, 0, 1, 1.0)
    got = O.unpack_i4(codes)[0].astype(np.int64)
    assert np.array_equal(got, 7 * sylvester(np.arange(128), k))
    assert scales[0, 0] == np.float32(np.float32(3.0) / np.float32(7.0))


@pytest.mark.parametrize("fmt", [O.F16, O.BF16])
def test_oracle_matches_numpy_quantisation(fmt):
    rng = np.random.default_rng(11 + fmt)
    tokens, heads = 9, 3
    v = (rng.standard_normal((tokens, heads * 128)) * 2).astype(np.float32)
    bits = (O.f16_bits(v) if fmt == O.F16 else O.bf16_bits(v)).reshape(tokens, heads * 128)
    mean = rng.standard_normal(heads * 128).astype(np.float32)
    for m in (None, mean):
        codes, scales = O.prepare_qk_i4(bits, fmt, m, tokens, heads * 128, 0, heads, 0.25)
        x = O.widen(bits, fmt)
        for t in range(tokens):
            for h in range(heads):
                y = x[t, 128 * h:128 * h + 128] - (0 if m is None else m[128 * h:128 * h + 128])
                w, s = numpy_quantize(rotate(y.astype(np.float32)), 0.25)
                assert np.array_equal(codes[t, 16 * h:16 * h + 16], w)
                assert scales[t, h] == s


def test_same_rotation_and_amax_as_the_int8_quantizer():
    rng = np.random.default_rng(3)
    v = rng.standard_normal((5, 256)).astype(np.float32)
    bits = O.f16_bits(v).reshape(5, 256)
    _, s4 = O.prepare_qk_i4(bits, O.F16, None, 5, 256, 0, 2, 1.0)
    _, s8 = O.prepare_qk(bits, O.F16, None, 5, 256, 0, 2, 1.0)
    r = [rotate(O.widen(bits, O.F16)[t, 128 * h:128 * h + 128]) for t in range(5) for h in range(2)]
    amax = np.array([np.float32(max(np.abs(x).max(), np.float32(1e-30))) for x in r], np.float32)
    assert np.array_equal(s4.reshape(-1), (amax / np.float32(7)).astype(np.float32))
    assert np.array_equal(s8.reshape(-1), (amax / np.float32(127)).astype(np.float32))


def test_planted_mistakes_are_caught():
    rng = np.random.default_rng(5)
    y = rng.standard_normal(128).astype(np.float32) * 3
    codes, scales = O.prepare_qk_i4(O.f16_bits(y).reshape(1, 128), O.F16, None, 1, 128, 0, 1, 1.0)
    r = rotate(O.widen(O.f16_bits(y).reshape(1, 128), O.F16)[0])
    good, _ = numpy_quantize(r, 1.0)
    assert np.array_equal(codes[0], good)
    assert not np.array_equal(numpy_quantize(r, 1.0, high_first=True)[0], good)
    # a clamp at +-8 instead of +-7 is visible where a code saturates: amax itself maps to 7, so
    # push one rotated value past it by scaling the row and checking the saturated code
    assert np.all(np.abs(O.unpack_i4(codes)[0]) <= 7) and np.any(np.abs(O.unpack_i4(codes)[0]) == 7)
