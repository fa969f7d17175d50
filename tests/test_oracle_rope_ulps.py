"""How far the RoPE route's quantized operands move with the RMS reciprocal's last bit.

The reference computes r = scalar.rsqrtf(mean + eps) (prepare_qk_rope_i8hm.loom:117,
rope_qknorm_f16.loom:134), whose bits are whatever its absent compiler lowers that to; this build
computes 1 / sqrtf(mean + eps), correctly rounded twice, which the oracle reproduces bit for bit.
A rsqrt within one ulp can differ from it by one unit in the last place either way, so the
reference's own bars are met whatever it lowers to if moving r by one ulp keeps:
  - the f16 RoPE outputs within the route's tolerance, 2e-2 abs + 2e-2 rel of the f64 oracle
    (tests/kernels.rs:1146-1222);
  - the int8 codes within the quantizer's bar: fewer than 1 in 500 packed words differ
    (tests/kernels.rs:1797-1802), every code by at most one step;
  - the scales within 1e-7 abs + 1e-4 rel (tests/kernels.rs:1803-1810).
Inputs: 4,096 tokens x 8 heads of N(0, 0.7^2) f16 activations, per-token random rotations.
"""
import math

import numpy as np
import pytest

import oracle as O


def rope_inputs(seed=11, tokens=4096, heads=8):
    rng = np.random.default_rng(seed)
    width = heads * 128
    x = O.f16_bits(rng.standard_normal((tokens, width), np.float32) * 0.7)
    ang = rng.uniform(-math.pi, math.pi, (tokens, 48)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    return x, w, np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


@pytest.mark.parametrize("ulps", [-1, 1])
def test_one_ulp_of_the_rms_reciprocal_stays_inside_the_reference_bars(ulps):
    tokens, heads = 4096, 8
    width = heads * 128
    x, w, cos_t, sin_t = rope_inputs()
    base = O.rope_qknorm_f16(x, O.F16, tokens, width, 0, heads, w, cos_t, sin_t, 1e-5)
    moved = O.rope_qknorm_f16(x, O.F16, tokens, width, 0, heads, w, cos_t, sin_t, 1e-5,
                              r_ulps=ulps)
    f64 = O.rope_qknorm_f64(x, O.F16, tokens, width, 0, heads, w, cos_t, sin_t, 1e-5)
    got = moved.view(np.float16).astype(np.float64).reshape(tokens, heads, 128)
    assert np.all(np.abs(got - f64) <= 2e-2 + 2e-2 * np.abs(f64))
    # the perturbation reaches the f16 outputs, but rarely, and each by one rounding step of its
    # magnitude (2^-10 relative), plus, where the rotation's two terms cancel, the terms' own
    # change: one ulp of r moves each term by at most |xn| * 2^-23 with |xn| < 8, so 2^-19
    changed = base != moved
    assert 0 < changed.mean() < 1e-3, changed.mean()
    a = base.view(np.float16).astype(np.float64)
    b = moved.view(np.float16).astype(np.float64)
    assert np.all(np.abs(a - b) <= 2.0 ** -10 * np.maximum(np.abs(a), np.abs(b)) + 2.0 ** -19)
    cap = O.capacity(tokens)
    extra = O.config_f32(O.EXTRA_Q_F64)
    qa, sa = O.prepare_qk(base, O.F16, None, tokens, width, 0, heads, extra, True, cap)
    qb, sb = O.prepare_qk(moved, O.F16, None, tokens, width, 0, heads, extra, True, cap)
    words_differ = (qa != qb).mean()
    assert words_differ * 500 < 1, words_differ
    ca = O.unpack(qa).astype(np.int32)
    cb = O.unpack(qb).astype(np.int32)
    assert np.abs(ca - cb).max() <= 1
    sa64, sb64 = sa.astype(np.float64), sb.astype(np.float64)
    assert np.all(np.abs(sb64 - sa64) <= 1e-7 + 1e-4 * np.abs(sa64))


def test_the_probe_moves_r():
    """A planted change the test must see: eight ulps move far more outputs than one."""
    tokens, heads = 512, 8
    width = heads * 128
    x, w, cos_t, sin_t = rope_inputs(tokens=tokens)
    base = O.rope_qknorm_f16(x, O.F16, tokens, width, 0, heads, w, cos_t, sin_t, 1e-5)
    one = O.rope_qknorm_f16(x, O.F16, tokens, width, 0, heads, w, cos_t, sin_t, 1e-5, r_ulps=1)
    eight = O.rope_qknorm_f16(x, O.F16, tokens, width, 0, heads, w, cos_t, sin_t, 1e-5, r_ulps=8)
    assert (base != eight).mean() > 4 * (base != one).mean() > 0
