"""Writes the golden vectors of this directory from the CPU oracle (oracle/h3oracle.c).

The reference checks in no vectors for this path (its tests build inputs in closed form), so the
fixtures here are the oracle's outputs on the reference's own closed-form inputs
(tests/kernels.rs:190-194 `values()`, :1758-1769 special heads, :2352-2362 fused RoPE inputs)
and on small seeded attention operands. The oracle functions are pinned in tests/test_oracle.py
(against the reference's f64 oracle, closed forms and numpy restatements); these files freeze
their outputs so that a later change of the oracle or of a kernel shows up as a diff.

Run from the repository root:  python tests/golden/make_golden.py
"""
import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent / "oracle"))
import oracle as O  # noqa: E402

EXTRA = O.config_f32(O.EXTRA_Q_F64)


def quantizer_case(tokens, heads):
    """tests/kernels.rs:1758-1769: values() inputs, a mean with head 0 zeroed, head 0 all zeros,
    head 1 all f16::MAX when heads == 56."""
    d = 128
    stride = heads * d
    x = O.values(tokens * stride, 0.7).astype(np.float16).reshape(tokens, stride)
    mean = O.values(stride, 0.1)
    mean[:d] = 0.0
    x[:, :d] = 0
    if heads == 56:
        x[:, d:2 * d] = np.float16(65504.0)
    return np.ascontiguousarray(x).view(np.uint16), mean.astype(np.float32)


def rope_case(tokens, heads):
    """Fused QKV rows from ((i*37 + seed) % 7) - 3 (tests/kernels.rs:2352-2362), norm weights and a
    rotary table of the same closed form."""
    d = 128
    width = heads * d
    i = np.arange(tokens * 3 * width)
    fused = ((((i * 37 + 5) % 7) - 3) * 0.25).astype(np.float16).reshape(tokens, 3 * width)
    w = (1.0 + ((np.arange(d) * 13 + 1) % 5 - 2) * 0.125).astype(np.float32)
    ang = (np.arange(tokens)[:, None] * (0.37 ** (np.arange(48)[None, :] / 16.0))).astype(np.float32)
    return np.ascontiguousarray(fused).view(np.uint16), w, np.cos(ang).astype(np.float32), \
        np.sin(ang).astype(np.float32)


def attention_case(tokens, heads, seed):
    """Seeded head-major operands with the reference's scale pattern and late match
    (tests/kernels.rs:2021-2046)."""
    rng = np.random.default_rng(seed)
    cap = -(-(tokens + 16) // 256) * 256
    qc = np.zeros((heads, cap, 128), np.int8)
    kc = np.zeros((heads, cap, 128), np.int8)
    qs = np.zeros((heads, cap), np.float32)
    ks = np.zeros((heads, cap), np.float32)
    vt = np.zeros((heads * 128, cap), np.float16)
    t = np.arange(tokens)
    qs[:, :tokens] = ((1 + t % 7) / 512.0).astype(np.float32)
    ks[:, :tokens] = ((1 + t % 3) / 128.0).astype(np.float32)
    qc[:, :tokens] = np.clip(np.round(rng.standard_normal((heads, tokens, 128)) * 24), -127, 127)
    kc[:, :tokens] = np.clip(np.round(rng.standard_normal((heads, tokens, 128)) * 24), -127, 127)
    vt[:, :tokens] = (rng.standard_normal((heads * 128, tokens)) * 0.3).astype(np.float16)
    for h in range(heads):
        kc[h, tokens - 1] = qc[h, 31 % tokens]
    return qc, qs, kc, ks, vt.view(np.uint16), cap


def main():
    for tokens, heads in [(37, 4), (3, 9), (3, 56)]:
        x, mean = quantizer_case(tokens, heads)
        codes, scales = O.prepare_qk(x, O.F16, mean, tokens, heads * 128, 0, heads, EXTRA)
        np.savez_compressed(HERE / f"prepare_qk_i8_t{tokens}_h{heads}.npz", codes=codes,
                            scales=scales)
    for tokens, heads in [(3, 2), (129, 4)]:
        fused, w, cos_t, sin_t = rope_case(tokens, heads)
        width = heads * 128
        q16 = O.rope_qknorm_f16(fused, O.F16, tokens, 3 * width, 0, heads, w, cos_t, sin_t, 1e-5)
        k16 = O.rope_qknorm_f16(fused, O.F16, tokens, 3 * width, width, heads, w, cos_t, sin_t,
                                1e-5)
        # the fused RoPE quantizer = rotated f16 rows through the quantizer with zero mean
        cap = O.capacity(tokens)
        qw, qsc = O.prepare_qk(q16, O.F16, None, tokens, width, 0, heads, EXTRA, 1, cap)
        kw, ksc = O.prepare_qk(k16, O.F16, None, tokens, width, 0, heads, 1.0, 1, cap)
        np.savez_compressed(HERE / f"rope_t{tokens}_h{heads}.npz", q=q16, k=k16, qcodes=qw,
                            qscales=qsc, kcodes=kw, kscales=ksc, capacity=np.int64(cap))
    for tokens, heads, seed in [(23, 2, 3), (97, 2, 4)]:
        qc, qs, kc, ks, vt, cap = attention_case(tokens, heads, seed)
        out = O.attention_f64(qc, qs, kc, ks, vt, tokens, cap, heads, np.arange(tokens))
        np.savez_compressed(HERE / f"attention_i8qkhm_t{tokens}_h{heads}.npz", out=out.astype(np.float32))
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))


if __name__ == "__main__":
    main()
