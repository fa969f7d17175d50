"""The cross-attention extension on the GPU (h3_attention_i8qkhm_cross): grouped heads and a
key-padding mask, against the f64 oracle at the north-star tolerance (max-abs 2e-2, mean-abs
2e-3), for groups that divide a workgroup's eight waves (the head-major kernel, all query heads
of a key/value head in one workgroup) and for groups that do not (the token-major cross kernel),
with leading key tiles entirely masked; bit-identical to attention_i8qkhm (the same kernel code)
when queries and keys are one sequence, ungrouped heads and no mask; BASELINE config 4's text
shape (130,272 queries,
32 query heads over 8 key/value heads, 512 text tokens, the last 20 % padding) on sampled rows.
"""
import numpy as np
import pytest

import h3attn as H
import oracle as O
from helpers import from_dev, north_star_ok, pack_codes, to_dev
from test_oracle_cross import operands

pytestmark = pytest.mark.gpu


def run_cross(dev, qc, qs, kc, ks, vt, mask, q_tokens, kv_tokens, out_stride=None):
    import torch

    qh, q_cap, _ = qc.shape
    kh, kv_cap, _ = kc.shape
    out_stride = out_stride or qh * 128
    cfg = H.CrossCfg(qh, kh, q_tokens, q_cap, kv_tokens, kv_cap, out_stride)
    out = torch.full((q_tokens * out_stride,), 0x7E00, dtype=torch.int16, device=dev)
    H.attention_i8qkhm_cross(cfg, to_dev(pack_codes(qc), dev), to_dev(qs, dev),
                             to_dev(pack_codes(kc), dev), to_dev(ks, dev), to_dev(vt, dev),
                             to_dev(mask, dev), out)
    return from_dev(out).reshape(q_tokens, out_stride)


@pytest.mark.parametrize("qh,kh,q_tokens,kv_tokens,dead_head", [
    (8, 2, 300, 77, 0), (4, 4, 129, 64, 0), (32, 8, 257, 512, 0), (2, 1, 33, 1, 0),
    (6, 3, 1000, 200, 0), (16, 2, 700, 1000, 0),
    # leading tiles with every key masked (the running max starts from a dead tile)
    (32, 8, 257, 512, 150), (8, 1, 100, 300, 64),
    # a group that does not divide the eight waves of a workgroup (the token-major cross kernel)
    (6, 2, 500, 300, 0), (9, 3, 65, 129, 70)])
def test_cross_attention_matches_the_oracle(dev, qh, kh, q_tokens, kv_tokens, dead_head):
    rng = np.random.default_rng(q_tokens + kv_tokens)
    q_cap = -(-q_tokens // 32) * 32
    kv_cap = -(-kv_tokens // 32) * 32 + 32
    qc, qs, kc, ks, vt = operands(rng, qh, kh, q_tokens, kv_tokens, q_cap, kv_cap)
    mask = (rng.random(kv_tokens) > 0.2).astype(np.uint8)
    mask[:dead_head] = 0
    mask[min(dead_head, kv_tokens - 1)] = 1
    print(f"cross qh={qh} kh={kh} q={q_tokens} kv={kv_tokens} dead={dead_head}", flush=True)
    got = run_cross(dev, qc, qs, kc, ks, vt, mask, q_tokens, kv_tokens)
    rows = np.arange(q_tokens, dtype=np.int32)
    want = O.cross_attention_f64(qc, qs, kc, ks, vt, mask, kv_tokens, rows).reshape(q_tokens, -1)
    mx, mean = north_star_ok(got.view(np.float16).astype(np.float32), want)
    assert mx < 2e-2 and mean < 2e-3, (mx, mean)


def test_one_sequence_unmasked_is_the_dense_kernel(dev):
    import torch

    rng = np.random.default_rng(7)
    heads, tokens, cap = 2, 256, 256
    qc, qs, kc, ks, vt = operands(rng, heads, heads, tokens, tokens, cap, cap)
    got = run_cross(dev, qc, qs, kc, ks, vt, np.ones(tokens, np.uint8), tokens, tokens)
    cfg = H.AttentionCfg(heads * 128, heads * 128, heads * 128, tokens, cap, 1.0)
    out = torch.zeros((tokens * heads * 128,), dtype=torch.int16, device=dev)
    H.attention_i8qkhm(cfg, tokens, heads, to_dev(pack_codes(qc), dev), to_dev(qs, dev),
                       to_dev(pack_codes(kc), dev), to_dev(ks, dev), to_dev(vt, dev), out)
    dense = from_dev(out).reshape(tokens, -1)
    rows = np.arange(tokens, dtype=np.int32)
    want = O.cross_attention_f64(qc, qs, kc, ks, vt, np.ones(tokens, np.uint8), tokens,
                                 rows).reshape(tokens, -1)
    for name, o in (("cross", got), ("dense", dense)):
        mx, mean = north_star_ok(o.view(np.float16).astype(np.float32), want)
        assert mx < 2e-2 and mean < 2e-3, (name, mx, mean)
    # The two forms share the kernel but not the last rounding of every score: cross-attention
    # removes the QK bias with each key's constant (c = -1.5*2^23*ks, -inf for a masked key),
    # the dense form does so on tiles without dead keys with the query's (-1.5*2^23*qs*log2 e).
    # Both put a score within 0.75 units of S of its exact value, so the outputs agree to within
    # a few f16 steps, far inside the oracle's bar.
    a = got.view(np.float16).astype(np.float64)
    b = dense.view(np.float16).astype(np.float64)
    assert np.abs(a - b).max() <= 1e-3 + 2e-3 * np.abs(want).max(), np.abs(a - b).max()


def test_config4_text_shape_on_sampled_rows(dev):
    """130,272 queries (video + audio), 32 query heads over 8 text key/value heads, 512 text
    tokens of which the last 20 % are padding."""
    import torch

    qh, kh, q_tokens, kv_tokens = 32, 8, 130272, 512
    q_cap, kv_cap = H.capacity(q_tokens), 512
    rng = np.random.default_rng(4)
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    qi = torch.randint(-127, 128, (qh * q_cap * 128,), dtype=torch.int8, device=dev, generator=g)
    qs = torch.rand((qh * q_cap,), device=dev, generator=g) * 1e-3 + 1e-4
    qc_s, qs_s, kc, ks, vt = operands(rng, 1, kh, 1, kv_tokens, 32, kv_cap)
    mask = np.ones(kv_tokens, np.uint8)
    mask[int(kv_tokens * 0.8):] = 0
    cfg = H.CrossCfg(qh, kh, q_tokens, q_cap, kv_tokens, kv_cap, qh * 128)
    out = torch.empty((q_tokens * qh * 128,), dtype=torch.int16, device=dev)
    print("cross config 4 text shape", flush=True)
    H.attention_i8qkhm_cross(cfg, qi, qs, to_dev(pack_codes(kc), dev), to_dev(ks, dev),
                             to_dev(vt, dev), to_dev(mask, dev), out)
    rows = np.array([0, 31, 4097, 100000, q_tokens - 1], np.int32)
    qc = from_dev(qi).view(np.int8).reshape(qh, q_cap, 128)[:, rows]
    qsr = from_dev(qs).reshape(qh, q_cap)[:, rows]
    want = O.cross_attention_f64(np.ascontiguousarray(qc), np.ascontiguousarray(qsr), kc, ks, vt,
                                 mask, kv_tokens, np.arange(len(rows), dtype=np.int32))
    got = from_dev(out).reshape(q_tokens, -1)[rows].view(np.float16).astype(np.float32)
    mx, mean = north_star_ok(got, want.reshape(len(rows), -1))
    assert mx < 2e-2 and mean < 2e-3, (mx, mean)
