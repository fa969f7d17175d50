"""The inputs of the every-tile exact-path GPU tests, checked on the CPU.

The head-major kernels take a running max from earlier key tiles and recompute a 32-key tile
exactly (its max, a raised running max, the output accumulators and the row sum rescaled by
alpha = 2^(m_old - m_new)) when a lane's 16 probabilities sum past 2^8. The GPU tests feed scores
that rise at every tile (helpers.rank1_operands), so that this path runs at every tile position.
Here, on the CPU:
  - the codes and scales give the intended scores: S = a_q b_j (u.w) exactly, and
    S * qs * ks * log2(e) = g_q * target_j to f32 accuracy; the int8 codes span most of the
    range, so the kernels' dequantisation error (under 0.75 units of S) stays far below the bar;
  - every tile after the first lifts every lane over the limit: each probability of tile t
    against the max of the keys before it exceeds 2^4, so any 16 of them pass 2^8;
  - a tile-by-tile online softmax in f64 with the rescale reproduces the f64 oracle, and the
    same walk with planted mistakes (no rescale of the accumulators, or the previous tile's
    alpha) misses the GPU tests' bar (1e-3 abs + 2e-3 rel), so those tests would catch them.
"""
import numpy as np

import oracle as O
from helpers import LOG2E, rank1_operands


def online_softmax(qc, qs, kc, ks, vt, tokens, head, row, mistake=None):
    """f64 attention of one query row in 32-key tiles with a running max, the way the kernels
    walk it; `mistake` plants an error in the rescale of the accumulators."""
    s = (kc[head, :tokens].astype(np.int64) @ qc[head, row].astype(np.int64)).astype(np.float64)
    y = s * float(qs[head, row]) * ks[head, :tokens].astype(np.float64) * LOG2E
    v = vt.view(np.float16)[head * 128:(head + 1) * 128, :tokens].astype(np.float64)
    m, l, o, prev_alpha = -np.inf, 0.0, np.zeros(128), 1.0
    for t0 in range(0, tokens, 32):
        yt = y[t0:t0 + 32]
        m_new = max(m, yt.max())
        alpha = 2.0 ** (m - m_new) if np.isfinite(m) else 0.0
        p = 2.0 ** (yt - m_new)
        a_o = {None: alpha, "no_rescale": 1.0, "stale_alpha": prev_alpha}[mistake]
        o = o * a_o + v[:, t0:t0 + 32] @ p
        l = l * alpha + p.sum()
        m, prev_alpha = m_new, alpha
    return o / l


def test_rising_scores_force_the_exact_path_and_planted_mistakes_show():
    rng = np.random.default_rng(5)
    heads, tokens = 2, 8193
    cap = O.capacity(tokens)
    qc, qs, kc, ks, vt = rank1_operands(rng, heads, tokens, cap, heads, tokens, cap)
    rows = np.array([0, 1, 31, 32, 4096, tokens - 1], np.int32)
    want = O.attention_f64(qc, qs, kc, ks, vt, tokens, cap, heads, rows)
    for h in range(heads):
        for i, r in enumerate(rows):
            s = kc[h, :tokens].astype(np.int64) @ qc[h, r].astype(np.int64)
            y = s * float(qs[h, r]) * ks[h, :tokens].astype(np.float64) * LOG2E
            # every tile rises: min of tile t minus max of all keys before it > 4 (log2 units)
            tiles = [y[t0:t0 + 32] for t0 in range(0, tokens, 32)]
            run_max = np.maximum.accumulate([t.max() for t in tiles])
            lift = np.array([tiles[t].min() - run_max[t - 1] for t in range(1, len(tiles))])
            assert lift.min() > 4.0, (h, r, lift.min())
            # the kernels' dequantisation (within 0.75 units of S) moves a score by at most this
            assert 0.75 * np.abs(y).max() / np.abs(s).min() < 4e-3
            got = online_softmax(qc, qs, kc, ks, vt, tokens, h, r)
            assert np.allclose(got, want[i, h], rtol=1e-12, atol=1e-12)
            bar = 1e-3 + 2e-3 * np.abs(want[i, h])
            for mistake in ("no_rescale", "stale_alpha"):
                bad = online_softmax(qc, qs, kc, ks, vt, tokens, h, r, mistake)
                assert (np.abs(bad - want[i, h]) > bar).any(), (mistake, h, r)


def test_rank1_codes_give_the_intended_scores():
    rng = np.random.default_rng(6)
    qh, kh, qt, kt = 8, 2, 300, 512
    qc, qs, kc, ks, vt = rank1_operands(rng, qh, qt, 320, kh, kt, 512)
    assert np.abs(qc.astype(np.int32)).max() <= 127 and np.abs(kc.astype(np.int32)).max() <= 127
    # rank one: every Q row of a head is a multiple of one vector, every K row of another
    q = qc[0, :qt].astype(np.int64)
    k = kc[0, :kt].astype(np.int64)
    assert np.linalg.matrix_rank(q.astype(np.float64)) == 1
    assert np.linalg.matrix_rank(k.astype(np.float64)) == 1
    s = q @ k.T
    y = s * qs[0, :qt, None].astype(np.float64) * ks[0, None, :kt].astype(np.float64) * LOG2E
    ratio = y / y[:, :1]  # g_q cancels: every row is the same target profile
    assert np.allclose(ratio, ratio[:1], rtol=1e-6)
    # one unit of S in log2 units, at the largest score: well below the bar's reach
    per_unit = np.abs(y).max() / np.abs(s).min()
    assert np.abs(s).min() >= 3e5 and 0.75 * per_unit < 2e-3, (np.abs(s).min(), per_unit)
