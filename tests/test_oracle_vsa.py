"""Pins of the VSA part of the CPU oracle (oracle/h3oracle_vsa.c), CPU only.

What fixes each function:
  - the plan and the budget: the reference's own unit tests (src/vsa.rs:145-225): prefix tiles
    [64, 1, 6] for Layout::new(65, 5, 10, 14, 3) (text 65 rows, audio 2*3 rows, a 5 x 5 x 7
    video grid), a bijective inverse, live rows first in each tile, prefix rows in prefix tiles
    only; topk(25) = 2, topk(35) = 4 (a tie rounds to even), topk(1) = 0; its sigma-window cases;
  - the route: the independent oracle of the reference's device test (src/vsa/device.rs:
    571-590) restated in numpy — the topk-th largest non-prefix score as a threshold, kept when
    >= it, or forced for prefix and neighbouring blocks — on random, tied and NaN-holding scores;
    all-equal scores keep every block (device.rs:728-756);
  - pool, kmean: sequential float32 sums (np.add.accumulate) and exact integer-valued means;
  - scores: exact on integer inputs, and within float rounding of a float64 dot otherwise;
  - gather / scatter / gated scatter: a round trip, zero padding rows, and float32-exact gates;
  - coarse and attention (f64): closed forms and agreement with the dense attention oracle;
  - the whole pipeline (gather, pool, scores, route, int8 operands, attention, scatter) against
    the reference device test's independent f32 masked attention on its closed-form inputs:
    normalised RMSE below 0.03 (device.rs:681, the int8 gate), plain and gated;
  - planted mistakes (>= for >, a dropped neighbour rule, an off-by-one length) that these catch.
"""
import math

import numpy as np
import pytest

import oracle as O

EXTRA_Q = O.config_f32(1.0 / 128.0 / math.sqrt(128.0))


# --------------------------------------------------------------------- plan and budget

def check_plan(src, inverse, lengths, prefix, prefix_rows):
    for row, i in enumerate(inverse):
        assert src[i] == row
    for b, ln in enumerate(lengths):
        tile = src[64 * b:64 * b + 64]
        assert np.all(tile[:ln] >= 0) and np.all(tile[ln:] == -1)
    pre = src[:64 * prefix]
    assert np.all(pre[pre >= 0] < prefix_rows)
    assert int(lengths[:prefix].sum()) == prefix_rows


def test_plan_matches_the_reference_cube_layout_test():
    # Layout::new(65, 5, 10, 14, 3, &[], &[]): text 65, audio 6, video 5 x (10/2) x (14/2)
    seq = 65 + 6 + 5 * 5 * 7
    src, inverse, lengths, prefix = O.vsa_plan([(0, 65), (65, 6)], seq, 5, 5, 7)
    assert prefix == 3
    assert list(lengths[:3]) == [64, 1, 6]
    check_plan(src, inverse, lengths, prefix, 71)
    # video cubes: 2 x 2 x 2 of them, the full one first (4*4*4), clipped at t, h and w
    assert list(lengths[3:]) == [64, 48, 16, 12, 16, 12, 4, 3]
    assert src[3 * 64 + 1] == 71 + 1 and src[3 * 64 + 4] == 71 + 7  # (0,0,1) and (0,1,0)


def test_plan_keeps_reference_segments_separate():
    # the shape of src/vsa.rs:162-205: text, several reference segments and audio, each its own
    # run of tiles, then the video cubes
    segs = [(0, 11), (11, 15), (26, 14), (40, 130), (170, 8), (178, 10)]
    prefix_rows = 188
    seq = prefix_rows + 3 * 5 * 7
    src, inverse, lengths, prefix = O.vsa_plan(segs, seq, 3, 5, 7)
    assert prefix == 1 + 1 + 1 + 3 + 1 + 1
    check_plan(src, inverse, lengths, prefix, prefix_rows)
    # no prefix tile mixes two segments
    for b in range(prefix):
        tile = src[64 * b:64 * b + lengths[b]]
        r0, rows = max((s for s in segs if s[0] <= tile[0]), key=lambda s: s[0])
        assert (tile[0] - r0) % 64 == 0 and tile[-1] < r0 + rows


def test_topk_budget_and_sigma_window():
    assert O.vsa_topk(10.0, 25) == 2
    assert O.vsa_topk(10.0, 35) == 4   # 3.5 rounds to even
    assert O.vsa_topk(10.0, 45) == 4   # 4.5 rounds to even
    assert O.vsa_topk(10.0, 1) == 0
    assert O.vsa_topk(100.0, 20) == 19
    assert O.vsa_topk(0.001, 20) == 1
    assert O.vsa_topk(30.0, 5) == 2    # 1.5 -> 2
    args = (0.2, 1.0, 12288)
    assert O.vsa_dense_reason(*args, 12288, 1.0, 10.0) == "outside_sigma_window"
    assert O.vsa_dense_reason(*args, 12288, 0.9, 10.0) is None
    assert O.vsa_dense_reason(*args, 12287, 0.5, 10.0) == "below_min_tokens"


# --------------------------------------------------------------------- route

def numpy_route(scores, prefix, topk, ge=True, near=True):
    """device.rs:571-590: threshold = the topk-th largest non-prefix score (sorted descending,
    NaN never counted as greater); kept when forced or own >= threshold."""
    heads, blocks, _ = scores.shape
    out = np.zeros_like(scores, dtype=np.int32)
    for h in range(heads):
        for q in range(blocks):
            row = scores[h, q]
            ranked = np.sort(row[prefix:][~np.isnan(row[prefix:])])[::-1]
            for j in range(blocks):
                forced = q < prefix or j < prefix or (near and abs(q - j) <= 1)
                if forced:
                    out[h, q, j] = 1
                elif topk == 0:
                    out[h, q, j] = 0
                elif np.isnan(row[j]) or len(ranked) < topk:
                    out[h, q, j] = 1
                else:
                    t = ranked[topk - 1]
                    out[h, q, j] = int(row[j] >= t) if ge else int(row[j] > t)
    return out


@pytest.mark.parametrize("prefix,topk", [(0, 1), (1, 3), (2, 7), (3, 0)])
def test_route_matches_the_threshold_oracle(prefix, topk):
    rng = np.random.default_rng(11 + prefix)
    heads, blocks = 2, 19
    scores = rng.standard_normal((heads, blocks, blocks)).astype(np.float32)
    scores[0, 3] = np.round(scores[0, 3])            # heavy ties
    scores[1, 5, 7] = np.nan
    scores[1, 6, :] = np.float32(0.0)
    scores[1, 6, 9] = np.float32(-0.0)               # -0 equals +0
    got = O.vsa_route(scores, prefix, topk)
    assert np.array_equal(got, numpy_route(scores, prefix, topk))


def test_route_keeps_every_tied_block():
    scores = np.zeros((2, 9, 9), np.float32)
    assert np.all(O.vsa_route(scores, 1, 2) == 1)


def test_route_planted_mistakes_are_caught():
    rng = np.random.default_rng(3)
    scores = np.round(rng.standard_normal((1, 16, 16)) * 2).astype(np.float32)  # ties
    good = O.vsa_route(scores, 1, 3)
    assert not np.array_equal(good, numpy_route(scores, 1, 3, ge=False))
    assert not np.array_equal(good, numpy_route(scores, 1, 3, near=False))
    assert not np.array_equal(good, numpy_route(scores, 0, 3))


# --------------------------------------------------------------------- pool, scores, kmean

def test_pool_is_a_sequential_f32_mean():
    rng = np.random.default_rng(4)
    lengths = np.array([3, 64, 1, 40], np.int32)
    x = rng.standard_normal((256, 256)).astype(np.float32) * 3
    bits = O.f16_bits(x).reshape(256, 256)
    got = O.vsa_pool(lengths, bits)
    xf = bits.view(np.float16).astype(np.float32)
    for b, ln in enumerate(lengths):
        acc = np.add.accumulate(xf[64 * b:64 * b + ln], axis=0, dtype=np.float32)[-1]
        assert np.array_equal(got[b].view(np.uint32), (acc / np.float32(ln)).view(np.uint32))
    ints = O.f16_bits(np.tile(np.arange(64, dtype=np.float32)[:, None], (1, 128))).reshape(64, 128)
    assert np.all(O.vsa_pool(np.array([64], np.int32), ints) == 31.5)
    # the planted off-by-one (one row too many) differs
    assert not np.allclose(O.vsa_pool(lengths + np.array([1, 0, 1, 1], np.int32), bits)[0], got[0])


def test_scores_are_per_head_dot_products():
    rng = np.random.default_rng(5)
    heads, blocks = 3, 7
    qi = rng.integers(-8, 8, (blocks, heads * 128)).astype(np.float32)
    ki = rng.integers(-8, 8, (blocks, heads * 128)).astype(np.float32)
    got = O.vsa_scores(qi, ki, heads)
    want = np.einsum("qhd,khd->hqk", qi.reshape(blocks, heads, 128).astype(np.int64),
                     ki.reshape(blocks, heads, 128).astype(np.int64))
    assert np.array_equal(got, want.astype(np.float32))
    qf = rng.standard_normal((blocks, heads * 128)).astype(np.float32)
    kf = rng.standard_normal((blocks, heads * 128)).astype(np.float32)
    want = np.einsum("qhd,khd->hqk", qf.reshape(blocks, heads, 128).astype(np.float64),
                     kf.reshape(blocks, heads, 128).astype(np.float64))
    assert np.allclose(O.vsa_scores(qf, kf, heads), want, rtol=0, atol=1e-4)


def test_kmean_is_a_sequential_f32_mean():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((37, 256)).astype(np.float32)
    want = np.add.accumulate(x, axis=0, dtype=np.float32)[-1] / np.float32(37)
    assert np.array_equal(O.vsa_kmean(x).view(np.uint32), want.view(np.uint32))


# --------------------------------------------------------------------- data movement

def test_gather_scatter_round_trip_and_gated_scatter():
    rng = np.random.default_rng(7)
    seq = 65 + 6 + 5 * 5 * 7
    src, inverse, lengths, prefix = O.vsa_plan([(0, 65), (65, 6)], seq, 5, 5, 7)
    x = O.f16_bits(rng.standard_normal((seq, 256)).astype(np.float32)).reshape(seq, 256)
    y = O.vsa_gather(src, seq, x)
    assert np.all(y[src < 0] == 0)
    assert np.array_equal(O.vsa_scatter(inverse, y), x)
    coarse = (rng.integers(-64, 64, (len(lengths), 256)) / 32).astype(np.float32)
    gate = O.f16_bits(np.where(np.arange(seq * 256) % 3 == 0, -1.25, 0.75).astype(np.float32)
                      ).reshape(seq, 256)
    got = O.vsa_gated_scatter(inverse, y, gate, coarse)
    g = gate.view(np.float16).astype(np.float64)
    f = x.view(np.float16).astype(np.float64)
    c = coarse[inverse // 64].astype(np.float64)
    want = (g * c + f).astype(np.float32).astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


# --------------------------------------------------------------------- coarse and attention

def test_coarse_closed_forms():
    rng = np.random.default_rng(8)
    heads, blocks = 2, 6
    vm = rng.standard_normal((blocks, heads * 128)).astype(np.float32)
    flat = np.zeros((heads, blocks, blocks), np.float32)
    got = O.vsa_coarse_f64(flat, vm)
    assert np.allclose(got, np.broadcast_to(vm.astype(np.float64).mean(0), got.shape), atol=1e-12)
    scores = rng.standard_normal((heads, blocks, blocks)).astype(np.float32) * 20
    got = O.vsa_coarse_f64(scores, vm)
    s = scores.astype(np.float32) * np.float32(0.08838834764831845)
    p = np.exp(s.astype(np.float64) - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    want = np.einsum("hqk,khd->qhd", p, vm.reshape(blocks, heads, 128).astype(np.float64))
    assert np.allclose(got, want.reshape(blocks, -1), atol=1e-12)


def token_major_operands(rng, heads, n):
    qc = np.clip(np.round(rng.standard_normal((n, heads * 128)) * 24), -127, 127).astype(np.int8)
    kc = np.clip(np.round(rng.standard_normal((n, heads * 128)) * 24), -127, 127).astype(np.int8)
    qs = ((1 + np.arange(n)[:, None] % 7) / 512.0 * np.ones(heads)).astype(np.float32)
    ks = ((1 + np.arange(n)[:, None] % 3) / 128.0 * np.ones(heads)).astype(np.float32)
    vt = O.f16_bits(rng.standard_normal((heads * 128, n)) * 0.3).reshape(heads * 128, n)
    return qc, qs, kc, ks, vt


def test_sparse_attention_with_every_block_routed_is_dense_attention():
    rng = np.random.default_rng(9)
    heads, blocks = 2, 4
    n = 64 * blocks
    qc, qs, kc, ks, vt = token_major_operands(rng, heads, n)
    routes = np.ones((heads, blocks, blocks), np.int32)
    lengths = np.full(blocks, 64, np.int32)
    rows = np.arange(0, n, 5, dtype=np.int32)
    got = O.vsa_attention_f64(qc, qs, kc, ks, vt, n, n, heads, routes, lengths, rows)
    hm = lambda c: np.ascontiguousarray(c.reshape(n, heads, 128).transpose(1, 0, 2))
    want = O.attention_f64(hm(qc), np.ascontiguousarray(qs.T), hm(kc), np.ascontiguousarray(ks.T),
                           vt, n, n, heads, rows)
    assert np.allclose(got, want, atol=1e-12)


def test_sparse_attention_masks_unrouted_blocks_and_dead_keys():
    rng = np.random.default_rng(10)
    heads, blocks = 1, 5
    n = 64 * blocks
    qc, qs, kc, ks, vt = token_major_operands(rng, heads, n)
    qc[:] = 0  # uniform weights over the kept keys
    routes = np.zeros((heads, blocks, blocks), np.int32)
    routes[0, 2, [0, 3]] = 1
    lengths = np.array([10, 64, 64, 33, 64], np.int32)
    got = O.vsa_attention_f64(qc, qs, kc, ks, vt, n, n, heads, routes, lengths,
                              np.array([130, 140], np.int32))
    keys = np.r_[np.arange(0, 10), np.arange(192, 225)]
    want = vt.view(np.float16).astype(np.float64)[:, keys].mean(1)
    assert np.allclose(got[0, 0], want, atol=1e-12) and np.allclose(got[1, 0], want, atol=1e-12)
    # a planted off-by-one in the live length changes the answer
    keys_bad = np.r_[np.arange(0, 11), np.arange(192, 225)]
    assert not np.allclose(got[0, 0], vt.view(np.float16).astype(np.float64)[:, keys_bad].mean(1))


def f16_operands(rng, heads, n, scale=1.0):
    q, k, v = (O.f16_bits(rng.standard_normal((n, heads * 128)) * scale).reshape(n, heads * 128)
               for _ in range(3))
    return q, k, v


def test_f16_sparse_attention_with_every_block_routed_is_dense_softmax_attention():
    """With every cube kept and full, the f16 form is plain softmax attention, computed here
    independently with numpy matrix products on the same f16 values."""
    rng = np.random.default_rng(31)
    heads, blocks = 2, 4
    n = 64 * blocks
    q, k, v = f16_operands(rng, heads, n)
    routes = np.ones((heads, blocks, blocks), np.int32)
    lengths = np.full(blocks, 64, np.int32)
    rows = np.arange(0, n, 3, dtype=np.int32)
    scale = 1 / math.sqrt(128)
    got = O.vsa_attention_f16_f64(q, k, v, n, heads, scale, routes, lengths, rows)
    f = lambda x: x.view(np.float16).astype(np.float64).reshape(n, heads, 128)
    qf, kf, vf = f(q), f(k), f(v)
    for h in range(heads):
        lg = qf[rows, h] @ kf[:, h].T * scale
        pr = np.exp(lg - lg.max(1, keepdims=True))
        pr /= pr.sum(1, keepdims=True)
        assert np.allclose(got[:, h], pr @ vf[:, h], atol=1e-12)
    # a planted scale mistake (the 1/sqrt(128) dropped) is far outside that agreement
    bad = O.vsa_attention_f16_f64(q, k, v, n, heads, 1.0, routes, lengths, rows)
    assert np.abs(bad - got).max() > 1e-2


def test_f16_sparse_attention_masks_unrouted_blocks_and_dead_keys():
    rng = np.random.default_rng(32)
    heads, blocks = 1, 5
    n = 64 * blocks
    q, k, v = f16_operands(rng, heads, n)
    q[:] = 0  # every logit 0: uniform weights over the kept live keys
    routes = np.zeros((heads, blocks, blocks), np.int32)
    routes[0, 2, [0, 3]] = 1
    lengths = np.array([10, 64, 64, 33, 64], np.int32)
    got = O.vsa_attention_f16_f64(q, k, v, n, heads, 0.09, routes, lengths,
                                  np.array([130, 140], np.int32))
    keys = np.r_[np.arange(0, 10), np.arange(192, 225)]
    want = v.view(np.float16).astype(np.float64)[keys].mean(0)
    assert np.allclose(got[0, 0], want, atol=1e-12) and np.allclose(got[1, 0], want, atol=1e-12)
    keys_bad = np.r_[np.arange(0, 11), np.arange(192, 225)]
    assert not np.allclose(got[0, 0], v.view(np.float16).astype(np.float64)[keys_bad].mean(0))
    # one live key in the only kept cube: the output is that key's V row exactly
    routes[:] = 0
    routes[0, 2, 4] = 1
    lengths[4] = 1
    q2, k2, _ = f16_operands(rng, heads, n, 3.0)
    one = O.vsa_attention_f16_f64(q2, k2, v, n, heads, 0.09, routes, lengths,
                                  np.array([128, 191], np.int32))
    assert np.array_equal(one[:, 0], np.repeat(v.view(np.float16).astype(np.float64)[256][None],
                                               2, 0))


# --------------------------------------------------------------------- whole pipeline

def reference_device_inputs():
    """src/vsa/device.rs:513-547: two heads, cubes of [3, 64, 49, 64, 8, 22] live rows, one
    prefix block, keep 30%; q, k, v closed forms rounded to f16."""
    heads = 2
    width = heads * 128
    lengths = np.array([3, 64, 49, 64, 8, 22], np.int32)
    src, inverse = [], []
    for ln in lengths:
        for _ in range(ln):
            inverse.append(len(src))
            src.append(len(inverse) - 1)
        src += [-1] * (64 - ln)
    src = np.array(src, np.int32)
    inverse = np.array(inverse, np.int32)
    t = len(inverse)
    i = np.arange(t * width)
    data = []
    for which in range(3):
        a = ((i * 37 + which * 113).astype(np.float32) * np.float32(0.017))
        b = ((i // width + which * 3).astype(np.float32) * np.float32(0.19))
        v = np.sin(a) * np.float32(0.8) + np.cos(b) * np.float32(0.3)
        data.append(O.f16_bits(v.astype(np.float32)).reshape(t, width))
    gates = O.f16_bits(np.where(i % 3 == 0, -1.25, 0.75).astype(np.float32)).reshape(t, width)
    return heads, src, inverse, lengths, 1, 30.0, data, gates


def independent_expected(heads, src, lengths, prefix, keep, data, gates):
    """device.rs:549-666 in numpy: f32 block means, f32 scores, the sorted threshold, natural
    f32-math attention on the raw f16 inputs; and the gated coarse branch."""
    width = heads * 128
    nb = len(lengths)
    t = data[0].shape[0]
    xs = [d.view(np.float16).astype(np.float32) for d in data]
    means = []
    for x in xs:
        m = np.zeros((nb, width), np.float32)
        for b, ln in enumerate(lengths):
            rows = src[64 * b:64 * b + ln]
            m[b] = x[rows].sum(0) / np.float32(ln)
        means.append(m)
    topk = O.vsa_topk(keep, nb - prefix)
    expected = np.zeros((t, width), np.float64)
    gated = np.zeros((t, width), np.float64)
    routes = np.zeros((heads, nb, nb), np.int32)
    g = gates.view(np.float16).astype(np.float64)
    for h in range(heads):
        sl = slice(128 * h, 128 * h + 128)
        sc = means[0][:, sl] @ means[1][:, sl].T
        for qb in range(nb):
            ranked = np.sort(sc[qb, prefix:])[::-1]
            thr = ranked[topk - 1]
            kept = [kb for kb in range(nb)
                    if qb < prefix or kb < prefix or abs(qb - kb) <= 1 or sc[qb, kb] >= thr]
            routes[h, qb, kept] = 1
            keys = [src[64 * kb + j] for kb in kept for j in range(lengths[kb])]
            keys = np.array(keys)
            qrows = src[64 * qb:64 * qb + lengths[qb]]
            lg = xs[0][qrows][:, sl].astype(np.float64) @ xs[1][keys][:, sl].T.astype(np.float64)
            lg /= math.sqrt(128)
            p = np.exp(lg - lg.max(1, keepdims=True))
            p /= p.sum(1, keepdims=True)
            expected[qrows, sl] = p @ xs[2][keys][:, sl].astype(np.float64)
            cl = sc[qb].astype(np.float64) / math.sqrt(128)
            cp = np.exp(cl - cl.max())
            cp /= cp.sum()
            coarse = cp @ means[2][:, sl].astype(np.float64)
            gated[qrows, sl] = g[qrows, sl] * coarse[None, :]
    return expected, expected + gated, routes


def oracle_pipeline(heads, src, inverse, lengths, prefix, keep, data, gates, kmean=None):
    """The VSA runtime sequence (src/vsa/device.rs:200-430) on the oracle."""
    t = len(inverse)
    n = len(src)
    width = heads * 128
    nb = len(lengths)
    q, k, v = (O.vsa_gather(src, t, d) for d in data)
    qm, km = O.vsa_pool(lengths, q), O.vsa_pool(lengths, k)
    scores = O.vsa_scores(qm, km, heads)
    routes = O.vsa_route(scores, prefix, O.vsa_topk(keep, nb - prefix))
    qw, qs = O.prepare_qk(q, O.F16, None, n, width, 0, heads, EXTRA_Q)
    mean = np.zeros(width, np.float32) if kmean is None else kmean
    kw, ks = O.prepare_qk(k, O.F16, mean, n, width, 0, heads, 1.0)
    vt = O.transpose(v, O.F16, n, width, 0, width, n, n)
    rows = np.arange(n, dtype=np.int32)
    att = O.vsa_attention_f64(O.unpack(qw), qs, O.unpack(kw), ks, vt, n, n, heads, routes,
                              lengths, rows)
    fine = O.f16_bits(att.reshape(n, width).astype(np.float32)).reshape(n, width)
    out = O.vsa_scatter(inverse, fine)
    vm = O.vsa_pool(lengths, v)
    coarse = O.vsa_coarse_f64(scores, vm).astype(np.float32)
    gated = O.vsa_gated_scatter(inverse, fine, gates, coarse)
    return out, gated, routes, O.vsa_kmean(km)


def oracle_pipeline_f16(heads, src, inverse, lengths, prefix, keep, data, gates):
    """The bits-16 runtime sequence (src/vsa/device.rs:200-263, 362-446): gather, routes, the f16
    attention on the gathered q, k, v, (gated) scatter."""
    t = len(inverse)
    n = len(src)
    width = heads * 128
    nb = len(lengths)
    q, k, v = (O.vsa_gather(src, t, d) for d in data)
    qm, km = O.vsa_pool(lengths, q), O.vsa_pool(lengths, k)
    scores = O.vsa_scores(qm, km, heads)
    routes = O.vsa_route(scores, prefix, O.vsa_topk(keep, nb - prefix))
    att = O.vsa_attention_f16_f64(q, k, v, n, heads, O.config_f32(1 / math.sqrt(128)), routes,
                                  lengths, np.arange(n, dtype=np.int32))
    fine = O.f16_bits(att.reshape(n, width).astype(np.float32)).reshape(n, width)
    out = O.vsa_scatter(inverse, fine)
    coarse = O.vsa_coarse_f64(scores, O.vsa_pool(lengths, v)).astype(np.float32)
    gated = O.vsa_gated_scatter(inverse, fine, gates, coarse)
    return out, gated, routes


def nrmse(actual_bits, expected):
    a = actual_bits.view(np.float16).astype(np.float64)
    return math.sqrt(((a - expected) ** 2).sum() / (expected ** 2).sum())


def test_pipeline_matches_the_reference_device_oracle():
    heads, src, inverse, lengths, prefix, keep, data, gates = reference_device_inputs()
    expected, gated_expected, want_routes = independent_expected(heads, src, lengths, prefix, keep,
                                                                 data, gates)
    out, gated, routes, _ = oracle_pipeline(heads, src, inverse, lengths, prefix, keep, data, gates)
    assert np.array_equal(routes, want_routes)
    assert 0 < routes.sum() < routes.size   # the case is sparse
    assert nrmse(out, expected) < 0.03
    assert nrmse(gated, gated_expected) < 0.03
    # zero queries: every score ties at zero and every block is kept (device.rs:728-756)
    zero = [np.zeros_like(data[0])] + data[1:]
    *_, routes0 = oracle_pipeline(heads, src, inverse, lengths, prefix, keep, zero, gates)[:3]
    assert np.all(routes0 == 1)


def test_f16_pipeline_matches_the_reference_device_oracle():
    """The reference's device test with bits 16 (src/vsa/device.rs:672-700): normalised RMSE
    against its masked f32-math attention below 0.01, plain and gated."""
    heads, src, inverse, lengths, prefix, keep, data, gates = reference_device_inputs()
    expected, gated_expected, want_routes = independent_expected(heads, src, lengths, prefix, keep,
                                                                 data, gates)
    out, gated, routes = oracle_pipeline_f16(heads, src, inverse, lengths, prefix, keep, data,
                                             gates)
    assert np.array_equal(routes, want_routes)
    assert nrmse(out, expected) < 0.01
    assert nrmse(gated, gated_expected) < 0.01


def test_pipeline_planted_route_mistake_is_caught():
    """Dense attention (every block kept) is off the sparse expectation by many times the
    pipeline's own error, and a budget off by one changes the routes."""
    heads, src, inverse, lengths, prefix, keep, data, gates = reference_device_inputs()
    expected, _, want_routes = independent_expected(heads, src, lengths, prefix, keep, data, gates)
    out, *_ = oracle_pipeline(heads, src, inverse, lengths, prefix, keep, data, gates)
    own = nrmse(out, expected)
    width = heads * 128
    xs = [d.view(np.float16).astype(np.float64) for d in data]
    dense = np.zeros_like(expected)
    for h in range(heads):
        sl = slice(128 * h, 128 * h + 128)
        lg = xs[0][:, sl] @ xs[1][:, sl].T / math.sqrt(128)
        p = np.exp(lg - lg.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        dense[:, sl] = p @ xs[2][:, sl]
    assert nrmse(O.f16_bits(dense.astype(np.float32)).reshape(-1, width), expected) > 5 * own
    qm = O.vsa_pool(lengths, O.vsa_gather(src, len(inverse), data[0]))
    km = O.vsa_pool(lengths, O.vsa_gather(src, len(inverse), data[1]))
    topk = O.vsa_topk(keep, len(lengths) - prefix)
    off = O.vsa_route(O.vsa_scores(qm, km, heads), prefix, topk + 1)
    assert not np.array_equal(off, want_routes)


def route_rows_by_rank(scores_row, q, prefix, topk):
    """routes[q][j] of one row by the reference's rank rule (vsa_ops.loom h3_vsa_route), with
    the ranks from a sort: rank(j) = #{k >= prefix, not NaN : score_k > score_j}, NaN ranks 0."""
    blocks = scores_row.shape[0]
    cand = scores_row[prefix:]
    valid = np.sort(cand[~np.isnan(cand)])
    own = scores_row
    rank = np.where(np.isnan(own), 0, len(valid) - np.searchsorted(valid, own, side="right"))
    j = np.arange(blocks)
    forced = (np.abs(j - q) <= 1) | (q < prefix) | (j < prefix)
    return np.where(forced, 1, (rank < topk).astype(np.int32)).astype(np.int32)


def test_sorted_rank_route_equals_the_oracle():
    """The sort-based route rule the long-row GPU test checks with equals the oracle's rank
    count row by row, with ties, NaN scores, prefixes and every budget."""
    rng = np.random.default_rng(0)
    for blocks, prefix in [(9, 0), (23, 2), (40, 5)]:
        s = rng.integers(-3, 4, (1, blocks, blocks)).astype(np.float32)
        s[0, 3, 5] = np.nan
        s[0, 4, 1] = np.nan
        for topk in range(0, blocks - prefix + 2):
            want = O.vsa_route(s, prefix, topk)
            for q in range(blocks):
                assert np.array_equal(route_rows_by_rank(s[0, q], q, prefix, topk), want[0, q])
