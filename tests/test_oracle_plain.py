"""The CPU oracle of the GEMM-operand quantizer prepare_plain_i8 / prepare_plain_f32_i8, pinned.

h3o_prepare_plain_i8 restates kernels/prepare_i8_family.loom (four radix-4 stages per 256-group,
absmax, s = max(amax/16, 1e-30)/127, q = clamp(rne(x/16/s))). Checks:
  - the reference's own test f32_preparation_matches_dense_hadamard_and_marks_invalid_rows
    (tests/kernels.rs:4587-4760) on its inputs: codes within 1 of the dense product, scale
    within 0.01 of max/127, a zero row gets a finite positive scale and zero codes, rows with
    NaN, +-inf or overflowing butterflies get a non-finite scale and zero codes;
  - one-hot rows: each output is +-1/16 of the input, so the codes are exactly 127 times the
    signs of the dense Kronecker matrix the reference test builds (4590-4603): a wrong sign,
    digit or index in any butterfly shows up;
  - an independent numpy restatement of the same operation order, bit for bit, on random f16
    and f32 rows;
  - planted mistakes (one flipped butterfly sign, a dropped 1/16) that these checks catch.
"""
import numpy as np
import pytest

import oracle as O

BASE = np.array([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], np.float64)


def dense_matrix():
    """tests/kernels.rs:4590-4603 without the /16: M[r][c] = prod_b base[digit_b(r)][digit_b(c)]."""
    r = np.arange(256)[:, None]
    c = np.arange(256)[None, :]
    m = np.ones((256, 256))
    for b in range(4):
        m *= BASE[(r >> (2 * b)) & 3, (c >> (2 * b)) & 3]
    return m


M = dense_matrix()


def numpy_plain(x, fmt, out_stride, flip=False, no_sixteenth=False):
    """Independent restatement, vectorised over groups: same expressions, same order."""
    if fmt == O.F32:
        v = np.asarray(x, np.float32) + np.float32(0)
    else:
        v = O.widen(np.asarray(x, np.uint16), fmt)
    tokens, width = v.shape
    g = v.reshape(tokens, width // 256, 4, 4, 4, 4).astype(np.float32)  # digits 3,2,1,0
    with np.errstate(over="ignore", invalid="ignore"):
        for d in range(4):
            ax = 5 - d
            x0, x1, x2, x3 = (np.take(g, i, axis=ax) for i in range(4))
            s01, s23, d01, d23 = x0 + x1, x2 + x3, x0 - x1, x2 - x3
            y1 = (s01 + d23) if (flip and d == 2) else (s01 - d23)
            g = np.stack([s01 + d23, y1, d01 + s23, s23 - d01], axis=ax)
        r = g.reshape(tokens, width)
        a = np.abs(r)
        a = np.where(a < np.inf, a, np.float32(np.inf))
        amax = a.max(axis=1)
        row_max = amax * np.float32(1.0 if no_sixteenth else 0.0625)
        s = np.maximum(row_max, np.float32(1e-30)) / np.float32(127.0)
        inv_s = np.float32(0.0625) / s
        valid = s < np.inf
        q = np.where(valid[:, None], r * inv_s[:, None], np.float32(0))
        q = np.clip(np.rint(q), -127, 127).astype(np.int8)
    codes = np.zeros((tokens, out_stride), np.int8)
    codes[:, :width] = q
    return codes, s.astype(np.float32)


def reference_rows(width):
    """tests/kernels.rs:4605-4618."""
    rows = 7
    x = np.zeros((rows, width), np.float32)
    i = np.arange(width)
    x[0] = ((i * 37) % 997).astype(np.float32) * 1 - 498.0
    x[0] *= 512.0
    x[1] = (((i * 17) % 199).astype(np.float32) - 99.0) / np.float32(127.0)
    x[3, 0] = np.nan
    x[4, width - 1] = np.inf
    x[5, 13] = -np.inf
    x[6, :] = np.finfo(np.float32).max
    return x


@pytest.mark.parametrize("width", [256, 4352, 8192, 14336, 25600])
def test_reference_dense_hadamard_assertions(width):
    x = reference_rows(width)
    stride = width + 64
    codes, scales = O.prepare_plain_i8(x, O.F32, stride)
    rotated = (x[0].astype(np.float64).reshape(-1, 256) @ M.T / 16.0).reshape(-1)
    mx = np.abs(rotated).max()
    assert abs(scales[0] - mx / 127.0) < 0.01
    expected = np.clip(np.round(rotated / scales[0]), -127, 127)
    assert np.all(np.abs(codes[0, :width].astype(np.int64) - expected) <= 1)
    assert np.isfinite(scales[2]) and scales[2] > 0 and np.all(codes[2] == 0)
    for r in range(3, 7):
        assert not np.isfinite(scales[r]) and np.all(codes[r] == 0)
    assert np.all(codes[:, width:] == 0)


def test_one_hot_rows_give_the_dense_signs():
    x = np.eye(256, dtype=np.float32)
    codes, scales = O.prepare_plain_i8(O.f16_bits(x).reshape(256, 256), O.F16, 256)
    assert np.array_equal(codes.astype(np.float64), 127.0 * M.T)
    assert np.all(scales == np.float32(np.float32(0.0625) / np.float32(127.0)))


@pytest.mark.parametrize("fmt", [O.F16, O.BF16, O.F32])
def test_oracle_matches_numpy_bit_for_bit(fmt):
    rng = np.random.default_rng(5 + fmt)
    tokens, width = 33, 1536
    v = rng.standard_normal((tokens, width)).astype(np.float32) * 3
    v[4] *= 1e-3
    v[5] = 0
    x = v if fmt == O.F32 else (O.f16_bits(v) if fmt == O.F16 else O.bf16_bits(v)).reshape(tokens, width)
    got = O.prepare_plain_i8(x, fmt, width + 128)
    want = numpy_plain(x, fmt, width + 128)
    assert np.array_equal(got[0], want[0])
    assert np.array_equal(got[1].view(np.uint32), want[1].view(np.uint32))


def test_planted_mistakes_are_caught():
    x = np.eye(256, dtype=np.float32)
    good = numpy_plain(x, O.F32, 256)[0]
    assert np.array_equal(good.astype(np.float64), 127.0 * M.T)
    flipped = numpy_plain(x, O.F32, 256, flip=True)[0]
    assert not np.array_equal(flipped, good)
    rng = np.random.default_rng(9)
    v = rng.standard_normal((4, 512)).astype(np.float32)
    assert not np.array_equal(numpy_plain(v, O.F32, 512, no_sixteenth=True)[1],
                              O.prepare_plain_i8(v, O.F32, 512)[1])
