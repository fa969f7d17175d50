"""The committed golden vectors (tests/golden/*.npz) against the CPU oracle — CPU only.

The vectors are the oracle's outputs on the reference's closed-form inputs, written by
tests/golden/make_golden.py. Recomputing them here pins the oracle against drift; the GPU tests
in test_gpu_golden.py compare the kernels against the same files.
"""
import pathlib
import sys

import numpy as np
import pytest

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))
import make_golden as G  # noqa: E402
import oracle as O  # noqa: E402


@pytest.mark.parametrize("tokens,heads", [(37, 4), (3, 9), (3, 56)])
def test_quantizer_vectors(tokens, heads):
    g = np.load(GOLDEN / f"prepare_qk_i8_t{tokens}_h{heads}.npz")
    x, mean = G.quantizer_case(tokens, heads)
    codes, scales = O.prepare_qk(x, O.F16, mean, tokens, heads * 128, 0, heads, G.EXTRA)
    assert np.array_equal(codes, g["codes"])
    assert np.array_equal(scales.view(np.uint32), g["scales"].view(np.uint32))


@pytest.mark.parametrize("tokens,heads", [(3, 2), (129, 4)])
def test_rope_vectors(tokens, heads):
    g = np.load(GOLDEN / f"rope_t{tokens}_h{heads}.npz")
    fused, w, cos_t, sin_t = G.rope_case(tokens, heads)
    width = heads * 128
    q16 = O.rope_qknorm_f16(fused, O.F16, tokens, 3 * width, 0, heads, w, cos_t, sin_t, 1e-5)
    assert np.array_equal(q16, g["q"])
    cap = int(g["capacity"])
    qw, qs = O.prepare_qk(q16, O.F16, None, tokens, width, 0, heads, G.EXTRA, 1, cap)
    assert np.array_equal(qw, g["qcodes"]) and np.array_equal(qs.view(np.uint32),
                                                               g["qscales"].view(np.uint32))
    # and the rotated rows stay within the reference f64 oracle's tolerance (kernels.rs:1146-1222)
    want = O.rope_qknorm_f64(fused, O.F16, tokens, 3 * width, 0, heads, w, cos_t, sin_t, 1e-5)
    got = g["q"].view(np.float16).astype(np.float64).reshape(tokens, heads, 128)
    assert np.all(np.abs(got - want) <= 2e-2 + 2e-2 * np.abs(want))


@pytest.mark.parametrize("tokens,heads,seed", [(23, 2, 3), (97, 2, 4)])
def test_attention_vectors(tokens, heads, seed):
    g = np.load(GOLDEN / f"attention_i8qkhm_t{tokens}_h{heads}.npz")
    qc, qs, kc, ks, vt, cap = G.attention_case(tokens, heads, seed)
    out = O.attention_f64(qc, qs, kc, ks, vt, tokens, cap, heads, np.arange(tokens))
    assert np.array_equal(out.astype(np.float32), g["out"])
