"""The CPU oracle of the cross-attention extension (h3o_cross_attention_f64), pinned.

The reference has no cross-attention kernel with grouped heads and a key mask (BASELINE config
4's text part is this build's extension), so the oracle is fixed by what the mathematics fixes:
  - with queries and keys from one sequence, ungrouped heads and no masked key it equals the
    pinned dense oracle h3o_attention_f64 on the same operands;
  - uniform scores (zero query codes) give the mean of the attended V rows of the query's group;
  - brute-force numpy (float64 softmax over the unmasked keys) on a small grouped shape;
  - planted mistakes (the wrong group, a masked key attended) change the answer.
"""
import numpy as np

import oracle as O


def operands(rng, qh, kh, q_tokens, kv_tokens, q_cap, kv_cap):
    qc = np.zeros((qh, q_cap, 128), np.int8)
    kc = np.zeros((kh, kv_cap, 128), np.int8)
    qc[:, :q_tokens] = np.clip(np.round(rng.standard_normal((qh, q_tokens, 128)) * 24), -127, 127)
    kc[:, :kv_tokens] = np.clip(np.round(rng.standard_normal((kh, kv_tokens, 128)) * 24), -127, 127)
    qs = np.zeros((qh, q_cap), np.float32)
    ks = np.zeros((kh, kv_cap), np.float32)
    qs[:, :q_tokens] = ((1 + np.arange(q_tokens) % 7) / 512.0)
    ks[:, :kv_tokens] = ((1 + np.arange(kv_tokens) % 3) / 128.0)
    vt = np.zeros((kh * 128, kv_cap), np.uint16)
    vt[:, :kv_tokens] = O.f16_bits(rng.standard_normal((kh * 128, kv_tokens)) * 0.3).reshape(kh * 128, kv_tokens)
    return qc, qs, kc, ks, vt


def numpy_cross(qc, qs, kc, ks, vt, mask, kv_tokens, rows, group_of=lambda h, g: h // g):
    qh, kh = qc.shape[0], kc.shape[0]
    g = qh // kh
    out = np.zeros((len(rows), qh, 128))
    keys = np.flatnonzero(mask[:kv_tokens])
    v = vt.view(np.float16).astype(np.float64)
    for i, r in enumerate(rows):
        for h in range(qh):
            kv = group_of(h, g)
            s = (kc[kv, keys].astype(np.int64) @ qc[h, r].astype(np.int64)).astype(np.float64)
            s *= float(qs[h, r]) * ks[kv, keys].astype(np.float64)
            p = np.exp(s - s.max())
            out[i, h] = (v[kv * 128:(kv + 1) * 128][:, keys] @ p) / p.sum()
    return out


def test_equals_the_dense_oracle_without_groups_or_mask():
    rng = np.random.default_rng(1)
    qc, qs, kc, ks, vt = operands(rng, 2, 2, 97, 97, 128, 128)
    kc[:, :97] = np.clip(np.round(rng.standard_normal((2, 97, 128)) * 24), -127, 127)
    rows = np.arange(0, 97, 7, dtype=np.int32)
    got = O.cross_attention_f64(qc, qs, kc, ks, vt, np.ones(97, np.uint8), 97, rows)
    want = O.attention_f64(qc, qs, kc, ks, vt, 97, 128, 2, rows)
    assert np.allclose(got, want, atol=1e-13)


def test_uniform_scores_average_the_attended_values():
    rng = np.random.default_rng(2)
    qc, qs, kc, ks, vt = operands(rng, 4, 2, 10, 50, 32, 64)
    qc[:] = 0
    mask = (rng.random(50) > 0.3).astype(np.uint8)
    got = O.cross_attention_f64(qc, qs, kc, ks, vt, mask, 50, np.array([0, 9], np.int32))
    v = vt.view(np.float16).astype(np.float64)
    for h in range(4):
        g = h // 2
        want = v[g * 128:(g + 1) * 128][:, np.flatnonzero(mask)].mean(1)
        assert np.allclose(got[:, h], want[None, :], atol=1e-12)


def test_matches_numpy_and_catches_planted_mistakes():
    rng = np.random.default_rng(3)
    qc, qs, kc, ks, vt = operands(rng, 8, 2, 40, 77, 64, 96)
    mask = (rng.random(77) > 0.2).astype(np.uint8)
    rows = np.array([0, 5, 39], np.int32)
    got = O.cross_attention_f64(qc, qs, kc, ks, vt, mask, 77, rows)
    assert np.allclose(got, numpy_cross(qc, qs, kc, ks, vt, mask, 77, rows), atol=1e-12)
    wrong_group = numpy_cross(qc, qs, kc, ks, vt, mask, 77, rows, group_of=lambda h, g: h % 2)
    assert not np.allclose(got, wrong_group, atol=1e-3)
    leaky = numpy_cross(qc, qs, kc, ks, vt, np.ones(77, np.uint8), 77, rows)
    assert not np.allclose(got, leaky, atol=1e-3)
