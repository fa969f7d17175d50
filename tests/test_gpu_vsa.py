"""The VSA path on the GPU through the C ABI (h3_vsa_*), against the oracle.

  - gather, scatter, pool, block scores, route, kmean and the gated scatter are bit-exact
    against their restatements (h3oracle_vsa.c), on plans with prefix segments and clipped
    cubes, on tied, NaN and signed-zero scores, and for every routing budget from 0 to blocks-1;
  - the coarse branch is within float rounding of its f64 statement (hardware exp);
  - the block-sparse attention matches the f64 attention of its operands over the kept keys at
    the north-star tolerance (max-abs 2e-2, mean-abs 2e-3), with partial cubes (live lengths
    on both sides of the 32-key tile boundary), odd block counts and routes that differ
    between query cubes; with every block routed and full cubes it agrees with the dense
    token-major attention to within f16 rounding (max-abs 2e-3; the two walk the keys in tiles
    of 32 and 64, so their lazy running maxima and f16 partial sums round differently); and
    past one list run (more than 512 listed half-cubes) it still matches the oracle. Each case
    runs both forms: token-major key scales (h3_vsa_attention_i8) and scales transposed
    head-major into a NaN-filled workspace (h3_vsa_attention_i8_ws), whose outputs are also
    bit-identical to each other;
  - the runtime (Runtime::emit) reproduces the reference's device test
    (src/vsa/device.rs:503-760): its intermediate buffers equal the oracle's bit for bit, the
    output's normalised RMSE against the independent masked attention is below 0.03 plain and
    gated, a replay is bit-identical, all-zero queries keep every block, and the per-layer K mean
    carried to the next call is the oracle's;
  - at BASELINE config 3's video grid (32 x 42 x 96 cells, 32 heads) the runtime's routes are
    exact on sampled rows and its attention matches the oracle on sampled queries.
"""
import math

import numpy as np
import pytest

import h3attn as H
import oracle as O
from helpers import from_dev, north_star_ok, pack_codes, to_dev
from test_oracle_vsa import (EXTRA_Q, independent_expected, nrmse, oracle_pipeline,
                             reference_device_inputs, route_rows_by_rank)

pytestmark = pytest.mark.gpu


def vsa_cfg(tokens, lengths, heads, prefix, topk):
    return H.VsaCfg(tokens, 64 * len(lengths), heads * 128, len(lengths), heads, prefix, topk)


def mixed_plan():
    """A prefix of text (70 rows) and audio (6 rows), then a 5 x 6 x 9 video grid."""
    seq = 76 + 5 * 6 * 9
    return O.vsa_plan([(0, 70), (70, 6)], seq, 5, 6, 9), seq


def dev_zeros(shape, dtype, dev):
    import torch

    return torch.zeros(shape, dtype=dtype, device=dev)


def test_gather_scatter_pool_are_exact(dev):
    import torch

    (src, inverse, lengths, prefix), seq = mixed_plan()
    heads = 3
    rng = np.random.default_rng(1)
    x = O.f16_bits(rng.standard_normal((seq, heads * 128)).astype(np.float32) * 2
                   ).reshape(seq, heads * 128)
    cfg = vsa_cfg(seq, lengths, heads, prefix, 3)
    n, w = cfg.padded, cfg.width
    y = torch.full((n * w,), -1, dtype=torch.int16, device=dev)
    print("vsa gather/scatter/pool", flush=True)
    H.vsa_gather(cfg, to_dev(src, dev), to_dev(x, dev), y)
    gy = from_dev(y).reshape(n, w)
    assert np.array_equal(gy, O.vsa_gather(src, seq, x))
    back = torch.full((seq * w,), -1, dtype=torch.int16, device=dev)
    H.vsa_scatter(cfg, to_dev(inverse, dev), y, back)
    assert np.array_equal(from_dev(back).reshape(seq, w), x)
    means = dev_zeros((len(lengths) * w,), torch.float32, dev)
    H.vsa_pool(cfg, to_dev(lengths, dev), y, means)
    want = O.vsa_pool(lengths, gy)
    assert np.array_equal(from_dev(means).reshape(-1, w).view(np.uint32), want.view(np.uint32))


def gpu_scores_routes(dev, qm, km, heads, prefix, topk, lengths_count):
    import torch

    blocks = qm.shape[0]
    cfg = H.VsaCfg(64 * blocks, 64 * blocks, heads * 128, blocks, heads, prefix, topk)
    scores = dev_zeros((heads * blocks * blocks,), torch.float32, dev)
    routes = torch.full((heads * blocks * blocks,), 7, dtype=torch.int32, device=dev)
    H.vsa_scores(cfg, to_dev(qm, dev), to_dev(km, dev), scores)
    H.vsa_route(cfg, scores, routes)
    return (from_dev(scores).reshape(heads, blocks, blocks),
            from_dev(routes).reshape(heads, blocks, blocks))


@pytest.mark.parametrize("blocks,prefix", [(1, 0), (7, 0), (23, 2), (130, 3), (301, 1)])
def test_scores_and_routes_are_exact(dev, blocks, prefix):
    rng = np.random.default_rng(blocks)
    heads = 2
    qm = rng.standard_normal((blocks, heads * 128)).astype(np.float32)
    km = rng.standard_normal((blocks, heads * 128)).astype(np.float32)
    km[blocks // 2] = km[0]  # exact ties between two key blocks
    print(f"vsa scores/route blocks={blocks}", flush=True)
    nonprefix = blocks - prefix
    scores, _ = gpu_scores_routes(dev, qm, km, heads, prefix, 0, blocks)
    want = O.vsa_scores(qm, km, heads)
    assert np.array_equal(scores.view(np.uint32), want.view(np.uint32))
    for topk in sorted({0, 1, min(2, max(nonprefix - 1, 0)), O.vsa_topk(10.0, nonprefix),
                        max(nonprefix - 1, 0), nonprefix + 3}):
        _, routes = gpu_scores_routes(dev, qm, km, heads, prefix, topk, blocks)
        assert np.array_equal(routes, O.vsa_route(want, prefix, topk)), f"topk={topk}"


@pytest.mark.parametrize("blocks,prefix", [(4098, 2), (4099, 2), (5003, 5)])
def test_routes_of_long_rows_are_exact(dev, blocks, prefix):
    """Rows of up to 4,096 candidates are kept in registers by the route kernel, longer ones are
    re-read per radix pass: both sides of that boundary, on sampled rows with ties."""
    rng = np.random.default_rng(blocks)
    heads = 1
    qm = rng.standard_normal((blocks, 128)).astype(np.float32)
    km = rng.standard_normal((blocks, 128)).astype(np.float32)
    km[blocks // 3] = km[7]  # exact ties
    nonprefix = blocks - prefix
    print(f"vsa long-row routes blocks={blocks}", flush=True)
    for topk in (1, O.vsa_topk(10.0, nonprefix), nonprefix - 1):
        scores, routes = gpu_scores_routes(dev, qm, km, heads, prefix, topk, blocks)
        for q in (0, 1, prefix, 7, blocks // 3, blocks // 2, blocks - 1):
            want = route_rows_by_rank(scores[0, q], q, prefix, topk)
            assert np.array_equal(routes[0, q], want), (topk, q)


def test_route_on_special_scores_is_exact(dev):
    import torch

    rng = np.random.default_rng(5)
    heads, blocks, prefix = 3, 41, 2
    scores = np.round(rng.standard_normal((heads, blocks, blocks)) * 3).astype(np.float32)
    scores[0, 4, 9] = np.nan
    scores[0, 5, :] = np.nan
    scores[1, 7, :] = 0.0
    scores[1, 7, ::3] = -0.0
    scores[2, 8, 10] = np.inf
    scores[2, 8, 11] = -np.inf
    scores[2, 9, :] = np.float32(1e-45)  # subnormal ties
    cfg_routes = torch.full((heads * blocks * blocks,), 7, dtype=torch.int32, device=dev)
    sc = to_dev(scores.reshape(-1), dev)
    print("vsa route special scores", flush=True)
    for topk in (0, 1, 4, 38, 39, 60):
        cfg = H.VsaCfg(64 * blocks, 64 * blocks, heads * 128, blocks, heads, prefix, topk)
        H.vsa_route(cfg, sc, cfg_routes)
        got = from_dev(cfg_routes).reshape(heads, blocks, blocks)
        assert np.array_equal(got, O.vsa_route(scores, prefix, topk)), f"topk={topk}"


def test_kmean_and_gated_scatter_are_exact(dev):
    import torch

    (src, inverse, lengths, prefix), seq = mixed_plan()
    heads = 2
    rng = np.random.default_rng(8)
    w = heads * 128
    km = rng.standard_normal((len(lengths), w)).astype(np.float32)
    mean = dev_zeros((w,), torch.float32, dev)
    print("vsa kmean/gated scatter", flush=True)
    H.vsa_kmean(w, len(lengths), to_dev(km, dev), mean)
    assert np.array_equal(from_dev(mean).view(np.uint32), O.vsa_kmean(km).view(np.uint32))
    cfg = vsa_cfg(seq, lengths, heads, prefix, 2)
    fine = O.f16_bits(rng.standard_normal((cfg.padded, w)).astype(np.float32)).reshape(-1, w)
    gate = O.f16_bits(rng.standard_normal((seq, w)).astype(np.float32)).reshape(-1, w)
    coarse = rng.standard_normal((len(lengths), w)).astype(np.float32)
    out = torch.full((seq * w,), -1, dtype=torch.int16, device=dev)
    H.vsa_gated_scatter(cfg, to_dev(inverse, dev), to_dev(fine, dev), to_dev(gate, dev),
                        to_dev(coarse, dev), out)
    want = O.vsa_gated_scatter(inverse, fine, gate, coarse)
    assert np.array_equal(from_dev(out).reshape(seq, w), want)


def test_coarse_matches_its_f64_statement(dev):
    import torch

    rng = np.random.default_rng(9)
    heads, blocks = 2, 77
    scores = (rng.standard_normal((heads, blocks, blocks)) * 30).astype(np.float32)
    vm = rng.standard_normal((blocks, heads * 128)).astype(np.float32)
    cfg = H.VsaCfg(64 * blocks, 64 * blocks, heads * 128, blocks, heads, 0, 1)
    out = dev_zeros((blocks * heads * 128,), torch.float32, dev)
    print("vsa coarse", flush=True)
    H.vsa_coarse(cfg, to_dev(scores, dev), to_dev(vm, dev), out)
    got = from_dev(out).reshape(blocks, -1)
    want = O.vsa_coarse_f64(scores, vm)
    assert np.abs(got - want).max() < 2e-5 * max(1.0, np.abs(want).max())


# --------------------------------------------------------------------- attention

def sparse_operands(rng, heads, lengths):
    """Token-major int8 operands of a gathered layout (dead rows zero, as the quantizer leaves
    them for zero rows), check_head_major_attention-style codes and scales."""
    blocks = len(lengths)
    n = 64 * blocks
    w = heads * 128
    live = np.zeros(n, bool)
    for b, ln in enumerate(lengths):
        live[64 * b:64 * b + ln] = True
    qc = np.clip(np.round(rng.standard_normal((n, w)) * 24), -127, 127).astype(np.int8)
    kc = np.clip(np.round(rng.standard_normal((n, w)) * 24), -127, 127).astype(np.int8)
    t = np.arange(n)
    qs = np.repeat(((1 + t % 7) / 512.0).astype(np.float32)[:, None], heads, 1)
    ks = np.repeat(((1 + t % 3) / 128.0).astype(np.float32)[:, None], heads, 1)
    v = (rng.standard_normal((n, w)) * 0.3).astype(np.float32)
    v[~live] = 0.0
    kc[~live] = 0
    vt = O.f16_bits(np.ascontiguousarray(v.T)).reshape(w, n)
    return qc, qs, kc, ks, vt


def random_routes(rng, heads, blocks, prefix, p):
    r = (rng.random((heads, blocks, blocks)) < p).astype(np.int32)
    for q in range(blocks):
        for j in range(blocks):
            if q < prefix or j < prefix or abs(q - j) <= 1:
                r[:, q, j] = 1
    return r


def run_vsa_attention(dev, qc, qs, kc, ks, vt, routes, lengths, heads, token_count=None,
                      lent=False):
    """h3_vsa_attention_i8 (token-major key scales) or, lent, h3_vsa_attention_i8_ws (the
    scales transposed head-major into a workspace filled with NaN beforehand)."""
    import torch

    n = qc.shape[0]
    w = heads * 128
    token_count = n if token_count is None else token_count
    cfg = H.AttentionCfg(w, w, w, n, n, H.config_f32(1 / math.sqrt(128)))
    out = torch.full((token_count * w,), 0x7E00, dtype=torch.int16, device=dev)
    args = (cfg, token_count, heads, to_dev(pack_codes(qc), dev), to_dev(qs, dev),
            to_dev(pack_codes(kc), dev), to_dev(ks, dev), to_dev(vt, dev), out,
            to_dev(routes, dev), to_dev(lengths, dev))
    if lent:
        nbytes = H.scales_workspace_bytes(cfg)
        assert nbytes == heads * n * 4
        ws = torch.full((nbytes // 2,), 0x7E00, dtype=torch.int16, device=dev)
        H.vsa_attention_i8_ws(*args, ws)
    else:
        H.vsa_attention_i8(*args)
    return from_dev(out).reshape(token_count, w)


LENT = pytest.mark.parametrize("lent", [False, True], ids=["plain", "workspace"])


@pytest.mark.parametrize("lengths,prefix,p", [
    ([64, 64], 0, 0.0),
    ([3, 64, 49, 64, 8, 22], 1, 0.3),
    ([64] * 9, 2, 0.4),
    ([64, 17, 64, 64, 1, 64, 40, 64, 64, 33, 64], 0, 0.25),
    ([32, 64, 33, 31, 64, 64, 2], 1, 0.3),
])
@LENT
def test_sparse_attention_matches_the_oracle(dev, lengths, prefix, p, lent):
    rng = np.random.default_rng(len(lengths) * 13 + prefix)
    heads = 2
    lengths = np.array(lengths, np.int32)
    blocks = len(lengths)
    qc, qs, kc, ks, vt = sparse_operands(rng, heads, lengths)
    routes = random_routes(rng, heads, blocks, prefix, p)
    print(f"vsa attention blocks={blocks} prefix={prefix} p={p} lent={lent}", flush=True)
    got = run_vsa_attention(dev, qc, qs, kc, ks, vt, routes, lengths, heads, lent=lent)
    n = 64 * blocks
    want = O.vsa_attention_f64(qc, qs, kc, ks, vt, n, n, heads, routes, lengths,
                               np.arange(n, dtype=np.int32)).reshape(n, -1)
    mx, mean = north_star_ok(got.view(np.float16).astype(np.float32), want)
    assert mx < 2e-2 and mean < 2e-3, (mx, mean)


@LENT
def test_token_count_limits_the_rows_written(dev, lent):
    rng = np.random.default_rng(3)
    heads, lengths = 1, np.array([64, 64, 64], np.int32)
    qc, qs, kc, ks, vt = sparse_operands(rng, heads, lengths)
    routes = random_routes(rng, heads, 3, 0, 0.5)
    full = run_vsa_attention(dev, qc, qs, kc, ks, vt, routes, lengths, heads, lent=lent)
    part = run_vsa_attention(dev, qc, qs, kc, ks, vt, routes, lengths, heads, token_count=100,
                             lent=lent)
    assert np.array_equal(part, full[:100])


def test_plain_and_workspace_forms_are_identical(dev):
    """The two forms read the same scales from different layouts: bit-identical outputs."""
    rng = np.random.default_rng(21)
    heads, lengths = 3, np.array([64, 40, 64, 64, 7, 64, 64, 64, 33, 64, 64, 64, 64, 1, 64, 64,
                                  64, 64, 64], np.int32)
    qc, qs, kc, ks, vt = sparse_operands(rng, heads, lengths)
    routes = random_routes(rng, heads, len(lengths), 1, 0.35)
    a = run_vsa_attention(dev, qc, qs, kc, ks, vt, routes, lengths, heads)
    b = run_vsa_attention(dev, qc, qs, kc, ks, vt, routes, lengths, heads, lent=True)
    assert np.isfinite(b.view(np.float16)).all()
    assert np.array_equal(a, b)


@pytest.mark.parametrize("blocks,heads", [(5, 2), (16, 3)])
@LENT
def test_every_block_routed_is_the_dense_attention(dev, blocks, heads, lent):
    import torch

    rng = np.random.default_rng(blocks)
    lengths = np.full(blocks, 64, np.int32)
    qc, qs, kc, ks, vt = sparse_operands(rng, heads, lengths)
    routes = np.ones((heads, blocks, blocks), np.int32)
    print(f"vsa dense equivalence blocks={blocks} lent={lent}", flush=True)
    got = run_vsa_attention(dev, qc, qs, kc, ks, vt, routes, lengths, heads, lent=lent)
    n, w = 64 * blocks, heads * 128
    cfg = H.AttentionCfg(w, w, w, n, n, H.config_f32(1 / math.sqrt(128)))
    out = torch.zeros((n * w,), dtype=torch.int16, device=dev)
    H.attention_i8qk(cfg, n, heads, to_dev(pack_codes(qc), dev), to_dev(qs, dev),
                     to_dev(pack_codes(kc), dev), to_dev(ks, dev), to_dev(vt, dev), out)
    dense = from_dev(out).reshape(n, w).view(np.float16).astype(np.float32)
    sparse = got.view(np.float16).astype(np.float32)
    assert np.isfinite(sparse).all()
    assert np.abs(sparse - dense).max() < 2e-3, np.abs(sparse - dense).max()
    want = O.vsa_attention_f64(qc, qs, kc, ks, vt, n, n, heads, routes, lengths,
                               np.arange(n, dtype=np.int32)).reshape(n, -1)
    mx, mean = north_star_ok(sparse, want)
    assert mx < 2e-2 and mean < 2e-3, (mx, mean)


@LENT
def test_more_cubes_than_one_list_run(dev, lent):
    """1100 cubes, nearly all routed: 2,197 or 2,199 live half-cubes per query cube, so the key
    loop runs five times (512 listed half-cubes per run) and must still match the oracle."""
    rng = np.random.default_rng(11)
    heads, blocks = 1, 1100
    lengths = np.full(blocks, 64, np.int32)
    lengths[1050] = 9
    qc, qs, kc, ks, vt = sparse_operands(rng, heads, lengths)
    routes = np.ones((heads, blocks, blocks), np.int32)
    routes[0, :, 3] = 0
    for q in (2, 3, 4):
        routes[0, q, 3] = 1  # the neighbours keep block 3
    print(f"vsa several list runs lent={lent}", flush=True)
    got = run_vsa_attention(dev, qc, qs, kc, ks, vt, routes, lengths, heads, lent=lent)
    n = 64 * blocks
    rows = np.array([0, 1, 200, 230, 64 * 1050 + 3, 64 * 1099 + 63, 64 * 3 + 5], np.int32)
    want = O.vsa_attention_f64(qc, qs, kc, ks, vt, n, n, heads, routes, lengths, rows)
    mx, mean = north_star_ok(got[rows].view(np.float16).astype(np.float32),
                             want.reshape(len(rows), -1))
    assert mx < 2e-2 and mean < 2e-3, (mx, mean)


# --------------------------------------------------------------------- runtime

def torch_f16(bits, dev):
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(dev)


def read(view, dtype, shape):
    from helpers import read_device

    return read_device(view).view(dtype).reshape(shape)


def test_runtime_reproduces_the_reference_device_test(dev):
    import torch

    heads, src, inverse, lengths, prefix, keep, data, gates = reference_device_inputs()
    t = len(inverse)
    w = heads * 128
    n = len(src)
    nb = len(lengths)
    expected, gated_expected, want_routes = independent_expected(heads, src, lengths, prefix,
                                                                 keep, data, gates)
    vsa = H.Vsa(src, inverse, lengths, prefix, heads, H.VsaOptions(keep_percent=keep))
    q, k, v = (torch_f16(d, dev) for d in data)
    out = torch.zeros((t * w,), dtype=torch.int16, device=dev)
    print("vsa runtime reference case", flush=True)
    vsa.attend(0, q, k, v, out)
    got = from_dev(out).reshape(t, w)
    err = nrmse(got, expected)
    print(f"VSA 8: normalized RMSE={err}", flush=True)
    assert err < 0.03
    # the intermediate buffers against the oracle pipeline, bit for bit
    b = vsa.buffers(0)
    gq = read(b.q, np.uint16, (n, w))
    assert np.array_equal(gq, O.vsa_gather(src, t, data[0]))
    gk0 = read(b.k, np.uint16, (n, w))
    assert np.array_equal(gk0, O.vsa_gather(src, t, data[1]))
    gv = O.vsa_gather(src, t, data[2])
    assert np.array_equal(read(b.v, np.uint16, (n, w)), gv)
    assert np.array_equal(read(b.vt, np.uint16, (w, n)), np.ascontiguousarray(gv.T))
    qm = read(b.qm, np.float32, (nb, w))
    km = read(b.km, np.float32, (nb, w))
    assert np.array_equal(qm.view(np.uint32), O.vsa_pool(lengths, gq).view(np.uint32))
    assert np.array_equal(km.view(np.uint32), O.vsa_pool(lengths, gk0).view(np.uint32))
    scores = read(b.scores, np.float32, (heads, nb, nb))
    assert np.array_equal(scores.view(np.uint32), O.vsa_scores(qm, km, heads).view(np.uint32))
    routes = read(b.routes, np.int32, (heads, nb, nb))
    assert np.array_equal(routes, want_routes)
    qw, qsc = O.prepare_qk(gq, O.F16, None, n, w, 0, heads, EXTRA_Q)
    assert np.array_equal(read(b.qi, np.int32, (n, heads * 32)), qw)
    assert np.array_equal(read(b.qs, np.float32, (n, heads)).view(np.uint32), qsc.view(np.uint32))
    mean1 = read(b.kmean, np.float32, (w,))
    assert np.array_equal(mean1.view(np.uint32), O.vsa_kmean(km).view(np.uint32))
    # replay after reset: bit-identical
    vsa.reset()
    out2 = torch.zeros_like(out)
    vsa.attend(0, q, k, v, out2)
    assert torch.equal(out, out2)
    # a second call centres K on the first call's mean
    vsa.attend(0, q, k, v, out2)
    gk = read(b.k, np.uint16, (n, w))
    kw, ksc = O.prepare_qk(gk, O.F16, mean1, n, w, 0, heads, 1.0)
    assert np.array_equal(read(b.ki, np.int32, (n, heads * 32)), kw)
    assert np.array_equal(read(b.ks, np.float32, (n, heads)).view(np.uint32), ksc.view(np.uint32))
    assert nrmse(from_dev(out2).reshape(t, w), expected) < 0.03
    # gated
    vsa.reset()
    gout = torch.zeros_like(out)
    vsa.attend(0, q, k, v, gout, gate=torch_f16(gates, dev))
    gerr = nrmse(from_dev(gout).reshape(t, w), gated_expected)
    print(f"VSA gated 8: normalized RMSE={gerr}", flush=True)
    assert gerr < 0.03
    # all-zero queries: every score ties and every block is kept
    vsa.attend(0, torch.zeros_like(q), k, v, out)
    assert np.all(read(b.routes, np.int32, (heads, nb, nb)) == 1)
    vsa.close()


def test_runtime_at_config3_grid_on_sampled_rows(dev):
    """BASELINE config 3's video grid (32 latent frames x 42 x 96 cells = 129,024 tokens,
    32 heads), default options (keep 10%): routes exact on sampled rows, attention within the
    north-star tolerance of the oracle on sampled queries (over the runtime's own operands)."""
    import torch

    nt, nh, nw, heads = 32, 42, 96, 32
    seq = nt * nh * nw
    src, inverse, lengths, prefix = H.vsa_plan([], seq, nt, nh, nw)
    nb, n, w = len(lengths), len(src), heads * 128
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    q = torch.randn((seq, w), generator=g, device=dev).half()
    k = torch.randn((seq, w), generator=g, device=dev).half()
    v = torch.randn((seq, w), generator=g, device=dev).half()
    out = torch.zeros((seq, w), dtype=torch.float16, device=dev)
    vsa = H.Vsa(src, inverse, lengths, prefix, heads)
    print(f"vsa runtime config-3 grid blocks={nb}", flush=True)
    vsa.attend(0, q, k, v, out)
    torch.cuda.synchronize()
    b = vsa.buffers(0)
    rows = np.array([0, 1, 777, 1500, nb - 1], np.int64)
    scores = read(b.scores, np.float32, (heads, nb, nb))
    routes = read(b.routes, np.int32, (heads, nb, nb))
    topk = H.VsaOptions().topk(nb - prefix)
    j = np.arange(nb)
    for h in (0, 31):
        for r in rows:
            row = scores[h, r]
            cand = row[prefix:][~np.isnan(row[prefix:])]
            thr = np.sort(cand)[::-1][topk - 1]
            want = (row >= thr) | np.isnan(row) | (np.abs(j - r) <= 1) | (j < prefix)
            assert np.array_equal(routes[h, r], want.astype(np.int32)), (h, r)
    qi = read(b.qi, np.int8, (n, w))
    ki = read(b.ki, np.int8, (n, w))
    qs = read(b.qs, np.float32, (n, heads))
    ks = read(b.ks, np.float32, (n, heads))
    vt = read(b.vt, np.uint16, (w, n))
    gathered = read(b.out, np.uint16, (n, w))
    qrows = np.array([0, 63, 64 * 700 + 5, 64 * (nb - 1) + lengths[-1] - 1], np.int32)
    want = O.vsa_attention_f64(qi, qs, ki, ks, vt, n, n, heads, routes, lengths, qrows)
    mx, mean = north_star_ok(gathered[qrows].view(np.float16).astype(np.float32),
                             want.reshape(len(qrows), -1))
    print(f"config-3 grid sampled rows: max {mx:.3e} mean {mean:.3e}", flush=True)
    assert mx < 2e-2 and mean < 2e-3
    # the scatter puts each gathered row back at its token
    tok = src[qrows]
    assert np.array_equal(from_dev(out.view(-1)).reshape(seq, w)[tok], gathered[qrows])
    vsa.close()


def test_runtime_with_prefix_segments_layers_and_gate(dev):
    """A DiT-like layout: 300 text rows and 20 audio rows as prefix segments, then an 8 x 10 x 12
    video grid (clipped cubes at h), two heads, two layers with their own K means, keep 25 %.
    Every buffer of the runtime equals the oracle pipeline's bit for bit where the reference's
    arithmetic is fixed (gathered rows, means, scores, routes, operands, K means); the output is
    within the north-star tolerance of the f64 attention of the runtime's own operands, plain
    and gated."""
    import torch

    heads = 2
    w = heads * 128
    segs = [(0, 300), (300, 20)]
    nt, nh, nw = 8, 10, 12
    seq = 320 + nt * nh * nw
    src, inverse, lengths, prefix = H.vsa_plan(segs, seq, nt, nh, nw)
    n, nb = len(src), len(lengths)
    rng = np.random.default_rng(21)
    data = [O.f16_bits(rng.standard_normal((seq, w)).astype(np.float32)).reshape(seq, w)
            for _ in range(3)]
    data[1] = O.f16_bits((data[1].view(np.float16).astype(np.float32)
                          + rng.standard_normal(w).astype(np.float32) * 1.4)).reshape(seq, w)
    gates = O.f16_bits(rng.standard_normal((seq, w)).astype(np.float32) * 0.5).reshape(seq, w)
    opts = H.VsaOptions(keep_percent=25.0)
    vsa = H.Vsa(src, inverse, lengths, prefix, heads, opts, layers=2)
    q, k, v = (torch_f16(d, dev) for d in data)
    out = torch.zeros((seq * w,), dtype=torch.int16, device=dev)
    print(f"vsa runtime prefix={prefix} blocks={nb}", flush=True)
    means = [np.zeros(w, np.float32), np.zeros(w, np.float32)]
    topk = O.vsa_topk(25.0, nb - prefix)
    for call, layer in enumerate([0, 1, 0]):
        gate = torch_f16(gates, dev) if call == 2 else None
        vsa.attend(layer, q, k, v, out, gate=gate)
        b = vsa.buffers(layer)
        gq = read(b.q, np.uint16, (n, w))
        gk = read(b.k, np.uint16, (n, w))
        assert np.array_equal(gq, O.vsa_gather(src, seq, data[0]))
        km = read(b.km, np.float32, (nb, w))
        qm = read(b.qm, np.float32, (nb, w))
        assert np.array_equal(km.view(np.uint32), O.vsa_pool(lengths, gk).view(np.uint32))
        scores = read(b.scores, np.float32, (heads, nb, nb))
        assert np.array_equal(scores.view(np.uint32), O.vsa_scores(qm, km, heads).view(np.uint32))
        routes = read(b.routes, np.int32, (heads, nb, nb))
        assert np.array_equal(routes, O.vsa_route(scores, prefix, topk))
        kw, ksc = O.prepare_qk(gk, O.F16, means[layer], n, w, 0, heads, 1.0)
        assert np.array_equal(read(b.ki, np.int32, (n, heads * 32)), kw)
        assert np.array_equal(read(b.ks, np.float32, (n, heads)).view(np.uint32),
                              ksc.view(np.uint32))
        means[layer] = O.vsa_kmean(km)
        assert np.array_equal(read(b.kmean, np.float32, (w,)).view(np.uint32),
                              means[layer].view(np.uint32))
        rows = np.arange(n, dtype=np.int32)
        att = O.vsa_attention_f64(read(b.qi, np.int8, (n, w)), read(b.qs, np.float32, (n, heads)),
                                  read(b.ki, np.int8, (n, w)), read(b.ks, np.float32, (n, heads)),
                                  read(b.vt, np.uint16, (w, n)), n, n, heads, routes, lengths,
                                  rows).reshape(n, w)
        fine = read(b.out, np.uint16, (n, w))
        live = src >= 0
        mx, mean = north_star_ok(fine[live].view(np.float16).astype(np.float32), att[live])
        assert mx < 2e-2 and mean < 2e-3, (call, mx, mean)
        got = from_dev(out).reshape(seq, w)
        if gate is None:
            assert np.array_equal(got, fine[inverse])
        else:
            vm = O.vsa_pool(lengths, read(b.v, np.uint16, (n, w)))
            coarse = O.vsa_coarse_f64(scores, vm).astype(np.float32)
            want = O.vsa_gated_scatter(inverse, fine, gates, coarse)
            diff = np.abs(got.view(np.float16).astype(np.float32) - want.view(np.float16).astype(np.float32))
            assert diff.max() < 1e-2, diff.max()
    vsa.close()
