"""The f16 VSA attention (h3_vsa_attention_f16, kernels/vsa_attention_16.loom) and the bits-16 VSA
runtime on the GPU, against the oracle (h3o_vsa_attention_f16_f64) and the reference's own test.

  - on gathered layouts with partial cubes (live lengths on both sides of the 32-key tile
    boundary), prefix blocks and routes that differ between query cubes and heads, the kernel is
    within max-abs 1e-2 and mean-abs 1e-3 of the f64 attention over the kept live keys; the
    dead rows of k and v hold NaN, so a dead key that were read would show;
  - rows at or past token_count are not written;
  - with every block routed and full cubes it is the dense softmax attention (a float32
    PyTorch reference on the CPU), to the same tolerance;
  - the bits-16 runtime reproduces the reference's device test (src/vsa/device.rs:672-700):
    routes exact, normalised RMSE below 0.01 plain and gated, a replay bit-identical;
  - at BASELINE config 3's video grid (129,024 tokens, 32 heads) the runtime's attention matches
    the oracle on sampled queries.
"""
import math

import numpy as np
import pytest

import h3attn as H
import oracle as O
from helpers import from_dev, north_star_ok, to_dev
from test_gpu_vsa import random_routes, read, torch_f16
from test_oracle_vsa import independent_expected, nrmse, reference_device_inputs

pytestmark = pytest.mark.gpu

NAN16 = 0x7E00


def f16_sparse_operands(rng, heads, lengths):
    """Gathered f16 q, k, v [64*blocks][heads*128]: dead query rows zero (as the gather leaves
    them), dead key and value rows NaN."""
    n = 64 * len(lengths)
    w = heads * 128
    live = np.zeros(n, bool)
    for b, ln in enumerate(lengths):
        live[64 * b:64 * b + ln] = True
    q, k, v = (O.f16_bits(rng.standard_normal((n, w))).reshape(n, w) for _ in range(3))
    q[~live] = 0
    k[~live] = NAN16
    v[~live] = NAN16
    return q, k, v


def run_f16(dev, q, k, v, routes, lengths, heads, token_count=None, scale=None):
    import torch

    n = q.shape[0]
    w = heads * 128
    token_count = n if token_count is None else token_count
    scale = H.config_f32(1 / math.sqrt(128)) if scale is None else scale
    cfg = H.AttentionCfg(w, w, w, n, n, scale)
    out = torch.full((token_count * w,), NAN16, dtype=torch.int16, device=dev)
    H.vsa_attention_f16(cfg, token_count, heads, to_dev(q, dev), to_dev(k, dev), to_dev(v, dev),
                        out, to_dev(routes, dev), to_dev(lengths, dev))
    return from_dev(out).reshape(token_count, w)


@pytest.mark.parametrize("lengths,prefix,p", [
    ([64, 64], 0, 0.0),
    ([3, 64, 49, 64, 8, 22], 1, 0.3),
    ([64] * 9, 2, 0.4),
    ([64, 17, 64, 64, 1, 64, 40, 64, 64, 33, 64], 0, 0.25),
    ([32, 64, 33, 31, 64, 64, 2], 1, 0.3),
])
def test_f16_sparse_attention_matches_the_oracle(dev, lengths, prefix, p):
    rng = np.random.default_rng(len(lengths) * 17 + prefix)
    heads = 2
    lengths = np.array(lengths, np.int32)
    blocks = len(lengths)
    q, k, v = f16_sparse_operands(rng, heads, lengths)
    routes = random_routes(rng, heads, blocks, prefix, p)
    print(f"vsa f16 attention blocks={blocks} prefix={prefix} p={p}", flush=True)
    got = run_f16(dev, q, k, v, routes, lengths, heads)
    n = 64 * blocks
    scale = H.config_f32(1 / math.sqrt(128))
    want = O.vsa_attention_f16_f64(q, k, v, n, heads, scale, routes, lengths,
                                   np.arange(n, dtype=np.int32)).reshape(n, -1)
    mx, mean = north_star_ok(got.view(np.float16).astype(np.float32), want)
    print(f"  max {mx:.3e} mean {mean:.3e}", flush=True)
    assert mx < 1e-2 and mean < 1e-3, (mx, mean)


def test_f16_token_count_limits_the_rows_written(dev):
    rng = np.random.default_rng(5)
    heads, lengths = 1, np.array([64, 64, 64], np.int32)
    q, k, v = f16_sparse_operands(rng, heads, lengths)
    routes = random_routes(rng, heads, 3, 0, 0.5)
    full = run_f16(dev, q, k, v, routes, lengths, heads)
    part = run_f16(dev, q, k, v, routes, lengths, heads, token_count=100)
    assert np.isfinite(full.view(np.float16)).all()
    assert np.array_equal(part, full[:100])


@pytest.mark.parametrize("blocks,heads", [(5, 2), (16, 3)])
def test_f16_every_block_routed_is_dense_attention(dev, blocks, heads):
    import torch

    rng = np.random.default_rng(blocks + heads)
    n, w = 64 * blocks, heads * 128
    q, k, v = f16_sparse_operands(rng, heads, np.full(blocks, 64, np.int32))
    routes = np.ones((heads, blocks, blocks), np.int32)
    scale = H.config_f32(0.125)
    got = run_f16(dev, q, k, v, routes, np.full(blocks, 64, np.int32), heads, scale=scale)
    f = lambda x: torch.from_numpy(x.view(np.float16).astype(np.float32)).view(n, heads, 128)
    qt, kt, vt = f(q).transpose(0, 1), f(k).transpose(0, 1), f(v).transpose(0, 1)
    p = torch.softmax(torch.matmul(qt, kt.transpose(1, 2).contiguous()) * scale, dim=-1)
    want = torch.matmul(p, vt).transpose(0, 1).reshape(n, w).numpy()
    mx, mean = north_star_ok(got.view(np.float16).astype(np.float32), want.astype(np.float64))
    assert mx < 1e-2 and mean < 1e-3, (mx, mean)


def test_f16_runtime_reproduces_the_reference_device_test(dev):
    import torch

    heads, src, inverse, lengths, prefix, keep, data, gates = reference_device_inputs()
    t = len(inverse)
    w = heads * 128
    nb = len(lengths)
    expected, gated_expected, want_routes = independent_expected(heads, src, lengths, prefix,
                                                                 keep, data, gates)
    vsa = H.Vsa(src, inverse, lengths, prefix, heads, H.VsaOptions(keep_percent=keep), bits=16)
    q, k, v = (torch_f16(d, dev) for d in data)
    out = torch.zeros((t * w,), dtype=torch.int16, device=dev)
    print("vsa f16 runtime reference case", flush=True)
    vsa.attend(0, q, k, v, out)
    err = nrmse(from_dev(out).reshape(t, w), expected)
    print(f"VSA 16: normalized RMSE={err}", flush=True)
    assert err < 0.01
    b = vsa.buffers(0)
    assert np.array_equal(read(b.routes, np.int32, (heads, nb, nb)), want_routes)
    assert not b.qi.ptr and not b.vt.ptr and not b.kmean.ptr  # no INT8 operands at bits 16
    vsa.reset()
    out2 = torch.zeros_like(out)
    vsa.attend(0, q, k, v, out2)
    assert torch.equal(out, out2)
    gout = torch.zeros_like(out)
    vsa.attend(0, q, k, v, gout, gate=torch_f16(gates, dev))
    gerr = nrmse(from_dev(gout).reshape(t, w), gated_expected)
    print(f"VSA gated 16: normalized RMSE={gerr}", flush=True)
    assert gerr < 0.01
    vsa.close()


def test_f16_runtime_at_config3_grid_on_sampled_rows(dev):
    import torch

    nt, nh, nw, heads = 32, 42, 96, 32
    seq = nt * nh * nw
    src, inverse, lengths, prefix = H.vsa_plan([], seq, nt, nh, nw)
    nb, n, w = len(lengths), len(src), heads * 128
    g = torch.Generator(device=dev)
    g.manual_seed(4)
    q = torch.randn((seq, w), generator=g, device=dev).half()
    k = torch.randn((seq, w), generator=g, device=dev).half()
    v = torch.randn((seq, w), generator=g, device=dev).half()
    out = torch.zeros((seq, w), dtype=torch.float16, device=dev)
    vsa = H.Vsa(src, inverse, lengths, prefix, heads, bits=16)
    print(f"vsa f16 runtime config-3 grid blocks={nb}", flush=True)
    vsa.attend(0, q, k, v, out)
    torch.cuda.synchronize()
    b = vsa.buffers(0)
    routes = read(b.routes, np.int32, (heads, nb, nb))
    gq, gk, gv = (read(x, np.uint16, (n, w)) for x in (b.q, b.k, b.v))
    gathered = read(b.out, np.uint16, (n, w))
    qrows = np.array([0, 63, 64 * 700 + 5, 64 * (nb - 1) + lengths[-1] - 1], np.int32)
    want = O.vsa_attention_f16_f64(gq, gk, gv, n, heads, H.config_f32(1 / math.sqrt(128)), routes,
                                   lengths, qrows)
    mx, mean = north_star_ok(gathered[qrows].view(np.float16).astype(np.float32),
                             want.reshape(len(qrows), -1))
    print(f"config-3 grid f16 sampled rows: max {mx:.3e} mean {mean:.3e}", flush=True)
    assert mx < 1e-2 and mean < 1e-3
    tok = src[qrows]
    assert np.array_equal(from_dev(out.view(-1)).reshape(seq, w)[tok], gathered[qrows])
    vsa.close()
