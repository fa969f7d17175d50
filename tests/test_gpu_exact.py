"""The exact path of the head-major kernels at every key tile.

The kernels keep a running max from earlier key tiles; a 32-key tile whose probabilities could
exceed 2^8 takes the exact path: its max, a raised running max, the output accumulators (pinned
registers, rescaled by hand-scheduled inline assembly) and the row sum rescaled, its
probabilities recomputed. Random inputs take that path at a block's first tile and rarely after.
Here the scores rise at every 32-key tile (helpers.rank1_operands: rank-one codes whose scales
set each score exactly), so the path runs at every tile position: both sub-steps of a 64-key
step, every phase of the four-stage rings, and the partial last tile. Checked against the f64
oracle at 1e-3 abs + 2e-3 rel (check_head_major_attention's bar, tests/kernels.rs:2013-2118), with
two bit-identical runs, for:
  - h3_attention_i8qkhm: the chained build (at most 64 key stages) without and with blocks
    staged across (one key/value head under 64 workload rows, so every workgroup's next block
    reads the same keys) and the unchained build (8,193 keys, a one-key last tile);
  - h3_attention_i8qk (the token-major kernel) at both lengths;
  - h3_attention_i8qkhm_cross (grouped heads, 20 % of the keys masked), chained across blocks;
  - h3_attention_i4qk_fp6 (QK on the FP6 MFMA) at both lengths, and with kv_stride < q_stride.
tests/test_exact_inputs.py shows on the CPU that these inputs force the path and that a
missing or stale rescale would fail this bar.
"""
import numpy as np
import pytest

import h3attn as H
import oracle as O
from helpers import from_dev, pack_codes, rank1_operands, to_dev
from test_gpu_i4 import pack_i4

pytestmark = pytest.mark.gpu


def assert_close(got, want, what):
    err = np.abs(got - want)
    print(f"  {what}: max-abs {err.max():.3e} mean-abs {err.mean():.3e}", flush=True)
    bad = err > 1e-3 + 2e-3 * np.abs(want)
    assert not bad.any(), (what, float(err.max()), np.argwhere(bad)[:4].tolist())


def sample_rows(tokens, extra=()):
    rows = {0, 1, 31, 32, 63, 64, 255, 256, tokens // 2, tokens - 1, *extra}
    return np.array(sorted(r for r in rows if 0 <= r < tokens), np.int32)


def run_twice(fn):
    a = fn()
    b = fn()
    assert np.array_equal(a, b), "unstable output"
    return a


@pytest.mark.parametrize("tokens,heads,kv_heads", [(4096, 3, 3), (4096, 64, 1), (8193, 3, 3)])
def test_head_major_exact_path_at_every_tile(dev, tokens, heads, kv_heads):
    """(4096, 64, 1): every workload row maps to key/value head 0 and query head 0
    (kv_stride = out_stride = 128; attention_i8qkhm...loom:300-340), 1,024 blocks over the
    persistent workgroups, each staging its next block's first key tiles."""
    import torch

    cap = O.capacity(tokens)
    rng = np.random.default_rng(tokens + heads)
    qh = min(heads, kv_heads) if kv_heads == 1 else heads
    qc, qs, kc, ks, vt = rank1_operands(rng, qh, tokens, cap, kv_heads, tokens, cap)
    cfg = H.AttentionCfg(qh * 128, kv_heads * 128, qh * 128, tokens, cap, 1.0)
    args = [to_dev(pack_codes(qc).reshape(qh * cap, 32), dev), to_dev(qs, dev),
            to_dev(pack_codes(kc).reshape(kv_heads * cap, 32), dev), to_dev(ks, dev),
            to_dev(vt, dev)]
    print(f"exact path, head-major: S={tokens} rows={heads} kv_heads={kv_heads}", flush=True)

    def run():
        out = torch.full((tokens, qh * 128), float("nan"), dtype=torch.float16, device=dev)
        H.attention_i8qkhm(cfg, tokens, heads, *args, out)
        torch.cuda.synchronize()
        return from_dev(out)

    got = run_twice(run).view(np.float16).astype(np.float64).reshape(tokens, qh, 128)
    rows = sample_rows(tokens, range(4064, 4100))
    want = O.attention_f64(qc, qs, kc, ks, vt, tokens, cap, qh, rows)
    assert_close(got[rows], want, ("head-major", tokens, heads))


@pytest.mark.parametrize("tokens", [4096, 8193])
def test_token_major_exact_path_at_every_tile(dev, tokens):
    import torch

    heads = 3
    cap = O.capacity(tokens)
    rng = np.random.default_rng(tokens + 11)
    qc, qs, kc, ks, vt = rank1_operands(rng, heads, tokens, cap, heads, tokens, cap)
    tm = lambda c: pack_codes(c.transpose(1, 0, 2)).reshape(cap, heads * 32)
    cfg = H.AttentionCfg(heads * 128, heads * 128, heads * 128, tokens, cap, 1.0)
    args = [to_dev(tm(qc), dev), to_dev(qs.T.copy(), dev), to_dev(tm(kc), dev),
            to_dev(ks.T.copy(), dev), to_dev(vt, dev)]
    print(f"exact path, token-major: S={tokens}", flush=True)

    def run():
        out = torch.full((tokens, heads * 128), float("nan"), dtype=torch.float16, device=dev)
        H.attention_i8qk(cfg, tokens, heads, *args, out)
        torch.cuda.synchronize()
        return from_dev(out)

    got = run_twice(run).view(np.float16).astype(np.float64).reshape(tokens, heads, 128)
    rows = sample_rows(tokens)
    want = O.attention_f64(qc, qs, kc, ks, vt, tokens, cap, heads, rows)
    assert_close(got[rows], want, ("token-major", tokens))


@pytest.mark.parametrize("q_tokens,kv_tokens", [(5000, 512), (700, 1000)])
def test_cross_attention_exact_path_at_every_tile(dev, q_tokens, kv_tokens):
    """32 query heads over 8 key/value heads; (5000, 512): consecutive blocks of a key/value
    head chain through the persistent workgroups (8 key stages, a multiple of the ring)."""
    import torch

    qh, kh = 32, 8
    q_cap = -(-q_tokens // 32) * 32
    kv_cap = -(-kv_tokens // 32) * 32
    rng = np.random.default_rng(q_tokens + kv_tokens)
    qc, qs, kc, ks, vt = rank1_operands(rng, qh, q_tokens, q_cap, kh, kv_tokens, kv_cap)
    mask = (rng.random(kv_tokens) > 0.2).astype(np.uint8)
    cfg = H.CrossCfg(qh, kh, q_tokens, q_cap, kv_tokens, kv_cap, qh * 128)
    args = [to_dev(pack_codes(qc), dev), to_dev(qs, dev), to_dev(pack_codes(kc), dev),
            to_dev(ks, dev), to_dev(vt, dev), to_dev(mask, dev)]
    print(f"exact path, cross: q={q_tokens} kv={kv_tokens}", flush=True)

    def run():
        out = torch.full((q_tokens, qh * 128), float("nan"), dtype=torch.float16, device=dev)
        H.attention_i8qkhm_cross(cfg, *args, out)
        torch.cuda.synchronize()
        return from_dev(out)

    got = run_twice(run).view(np.float16).astype(np.float64).reshape(q_tokens, qh, 128)
    rows = sample_rows(q_tokens)
    want = O.cross_attention_f64(qc, qs, kc, ks, vt, mask, kv_tokens, rows)
    assert_close(got[rows], want, ("cross", q_tokens, kv_tokens))


@pytest.mark.parametrize("tokens,heads,kv_heads", [(4096, 3, 3), (8193, 3, 3), (4096, 4, 2)])
def test_fp6_exact_path_at_every_tile(dev, tokens, heads, kv_heads):
    """The FP6 form moves QK to two MFMAs per sub-step ahead of the same rescale. (4096, 4, 2):
    kv_stride = 256 < q_stride = out_stride = 512, so workload rows 0-3 read key/value heads
    0, 1, 0, 1 and query heads 0, 1, 0, 1 (heads 2 and 3 of the output are never written)."""
    import torch

    cap = H.capacity(tokens)
    rng = np.random.default_rng(tokens + 6)
    # int4 codes: |u| in [2, 3], multipliers 1-2 (codes -6..6); the FP6 form accumulates S/4
    # exactly in f32 from zero, so its dequantisation has no bias error to bound
    qc, qs, kc, ks, vt = rank1_operands(rng, heads, tokens, cap, kv_heads, tokens, cap,
                                        code_min=2, code_max=3, mult_max=(2, 2))
    # token-major int4 operands: [cap][heads*128] codes, [cap][heads] scales
    q_tm = np.ascontiguousarray(qc.transpose(1, 0, 2)).reshape(cap, heads * 128)
    k_tm = np.ascontiguousarray(kc.transpose(1, 0, 2)).reshape(cap, kv_heads * 128)
    cfg = H.AttentionCfg(heads * 128, kv_heads * 128, heads * 128, tokens, cap, 1.0)
    args = [to_dev(pack_i4(q_tm), dev), to_dev(qs.T.copy(), dev), to_dev(pack_i4(k_tm), dev),
            to_dev(ks.T.copy(), dev), to_dev(vt, dev)]
    ws = torch.zeros((H.fp6_workspace_bytes(cfg),), dtype=torch.uint8, device=dev)
    print(f"exact path, fp6: S={tokens} heads={heads} kv_heads={kv_heads}", flush=True)

    def run():
        out = torch.full((tokens, heads * 128), float("nan"), dtype=torch.float16, device=dev)
        H.attention_i4qk_fp6(cfg, tokens, heads, *args, out, ws)
        torch.cuda.synchronize()
        return from_dev(out)

    raw = run_twice(run)
    got = raw.view(np.float16).astype(np.float64).reshape(tokens, heads, 128)
    touched = min(heads, kv_heads)
    rows = sample_rows(tokens)
    # query head h reads key/value head h (h < touched)
    want = O.attention_f64(qc[:touched], qs[:touched], kc[:touched], ks[:touched],
                           vt[:touched * 128], tokens, cap, touched, rows)
    assert_close(got[rows][:, :touched], want, ("fp6", tokens, heads, kv_heads))
    assert np.isnan(got[:, touched:]).all(), "heads no workload row reads were written"
