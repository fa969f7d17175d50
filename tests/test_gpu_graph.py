"""The entry points are stream-ordered and capturable (the reference records its dispatch calls
into graphs and replays them with fixed addresses, docs/shared-hrx.md:102-104): a HIP graph
captured through torch.cuda.graph around the step's kernels (the fused RoPE quantizers of Q and
K, the V transpose and the head-major attention), a _ws attention (scale transpose + attention),
the FP6 int4 attention (conversion + attention), the VSA attention with a lent workspace and
the f16 VSA attention and runtime, replayed three times with eager work and
synchronisations between the replays, gives the eager result bit for bit on every replay. The
captured regions hold only this library's kernels (no memset or library reduction nodes)."""
import math

import numpy as np
import pytest

import h3attn as H
import oracle as O
from helpers import from_dev, pack_codes, to_dev

pytestmark = pytest.mark.gpu


def replay_matches(torch, dev, run, outs):
    """Eager result of `run`, then a graph of it replayed three times: every replay equal."""
    run()
    torch.cuda.synchronize()
    eager = [from_dev(o).copy() for o in outs]
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):  # warm the capture stream as torch recommends
        run()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    noise = torch.randn(1 << 20, device=dev)
    for rep in range(3):
        for o in outs:
            o.zero_()  # a fill kernel between the replays, then eager work
        noise.mul_(1.0001).add_(0.5)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for o, want in zip(outs, eager):
            assert np.array_equal(from_dev(o), want), f"replay {rep}"
    del g


def test_step_kernels_replay_from_a_graph(dev):
    import torch

    tokens, heads = 700, 2
    width = heads * 128
    cap = H.capacity(tokens)
    g = torch.Generator(device=dev).manual_seed(4)
    fused = (torch.randn((tokens, 3 * width), generator=g, device=dev)).to(torch.float16)
    w = torch.ones(128, dtype=torch.float32, device=dev)
    cos = torch.rand((tokens, 48), generator=g, device=dev)
    sin = torch.rand((tokens, 48), generator=g, device=dev)
    qi = torch.zeros((heads * cap, 32), dtype=torch.int32, device=dev)
    ki = torch.zeros_like(qi)
    qs = torch.zeros((heads, cap), dtype=torch.float32, device=dev)
    ks = torch.zeros_like(qs)
    vt = torch.zeros((width, cap), dtype=torch.float16, device=dev)
    out = torch.zeros((tokens, width), dtype=torch.float16, device=dev)
    pq = H.PrepareCfg(3 * width, 0, heads, H.EXTRA_Q, cap, 1e-5, H.H3_ELEM_F16)
    pk = H.PrepareCfg(3 * width, width, heads, 1.0, cap, 1e-5, H.H3_ELEM_F16)
    tc = H.TransposeCfg(width, cap, H.H3_ELEM_F16)
    ac = H.AttentionCfg(width, width, width, tokens, cap, H.config_f32(1 / math.sqrt(128)))

    def run():
        H.prepare_qk_rope_i8hm(pq, tokens, fused, w, cos, sin, qi, qs)
        H.prepare_qk_rope_i8hm(pk, tokens, fused, w, cos, sin, ki, ks)
        H.transpose_qkv_v_f16(tc, tokens, tokens, fused, vt)
        H.attention_i8qkhm(ac, tokens, heads, qi, qs, ki, ks, vt, out)

    print("graph: step kernels", flush=True)
    replay_matches(torch, dev, run, [qi, qs, ki, ks, vt, out])


def test_workspace_forms_replay_from_a_graph(dev):
    import torch

    tokens, heads = 900, 2
    stride = heads * 128
    cap = H.capacity(tokens)
    rng = np.random.default_rng(8)
    q = rng.integers(-7, 8, (cap, stride)).astype(np.int8)
    k = rng.integers(-7, 8, (cap, stride)).astype(np.int8)
    q[tokens:] = 0
    k[tokens:] = 0
    qs = to_dev(rng.uniform(0.005, 0.05, (cap, heads)).astype(np.float32), dev)
    ks = to_dev(rng.uniform(0.005, 0.05, (cap, heads)).astype(np.float32), dev)
    v = O.f16_bits(rng.standard_normal((tokens, stride)).astype(np.float32)).reshape(tokens, stride)
    vt = to_dev(O.transpose(v, O.F16, tokens, stride, 0, stride, cap, cap), dev)
    qi, ki = to_dev(q.view(np.int32), dev), to_dev(k.view(np.int32), dev)
    cfg = H.AttentionCfg(stride, stride, stride, tokens, cap, 1.0)
    ws = torch.zeros(H.scales_workspace_bytes(cfg), dtype=torch.uint8, device=dev)
    out = torch.zeros((tokens, stride), dtype=torch.float16, device=dev)
    print("graph: attention_i8qk_ws", flush=True)
    replay_matches(torch, dev,
                   lambda: H.attention_i8qk_ws(cfg, tokens, heads, qi, qs, ki, ks, vt, out, ws),
                   [out, ws])


def test_fp6_int4_attention_replays_from_a_graph(dev):
    """h3_attention_i4qk_fp6: the conversion into the workspace and the FP6 attention."""
    import torch

    from test_gpu_fp6 import operands
    from test_gpu_i4 import pack_i4

    tokens, heads = 900, 2
    stride = heads * 128
    cap = H.capacity(tokens)
    q, k, qs, ks, vt = operands(np.random.default_rng(14), tokens, heads, cap)
    cfg = H.AttentionCfg(stride, stride, stride, tokens, cap, 1.0)
    args = [to_dev(pack_i4(q), dev), to_dev(qs, dev), to_dev(pack_i4(k), dev), to_dev(ks, dev),
            to_dev(vt, dev)]
    ws = torch.zeros(H.fp6_workspace_bytes(cfg), dtype=torch.uint8, device=dev)
    out = torch.zeros((tokens, stride), dtype=torch.float16, device=dev)
    print("graph: attention_i4qk_fp6", flush=True)
    replay_matches(torch, dev, lambda: H.attention_i4qk_fp6(cfg, tokens, heads, *args, out, ws),
                   [out])


def test_vsa_attention_replays_from_a_graph(dev):
    import torch

    from test_gpu_vsa import random_routes, sparse_operands

    rng = np.random.default_rng(12)
    heads = 2
    lengths = np.array([64, 40, 64, 64, 9, 64, 64, 33, 64], np.int32)
    blocks = len(lengths)
    n, w = 64 * blocks, heads * 128
    qc, qs, kc, ks, vt = sparse_operands(rng, heads, lengths)
    routes = random_routes(rng, heads, blocks, 1, 0.4)
    cfg = H.AttentionCfg(w, w, w, n, n, H.config_f32(1 / math.sqrt(128)))
    args = [to_dev(pack_codes(qc), dev), to_dev(qs, dev), to_dev(pack_codes(kc), dev),
            to_dev(ks, dev), to_dev(vt, dev)]
    out = torch.zeros((n, w), dtype=torch.float16, device=dev)
    out_ws = torch.zeros_like(out)
    rt, ln = to_dev(routes, dev), to_dev(lengths, dev)
    ws = torch.zeros(H.scales_workspace_bytes(cfg), dtype=torch.uint8, device=dev)

    def run():
        H.vsa_attention_i8(cfg, n, heads, *args, out, rt, ln)
        H.vsa_attention_i8_ws(cfg, n, heads, *args, out_ws, rt, ln, ws)

    print("graph: vsa attention, both forms", flush=True)
    replay_matches(torch, dev, run, [out, out_ws])
    assert np.array_equal(from_dev(out), from_dev(out_ws))


def test_f16_vsa_attention_and_runtime_replay_from_a_graph(dev):
    """The f16 VSA attention alone, and the bits-16 runtime (gather, pool, scores, route, the f16
    attention, gated scatter) on the reference's device-test inputs, as the reference's test
    replays its graph (src/vsa/device.rs:701-719)."""
    import torch

    from test_gpu_vsa import random_routes, torch_f16
    from test_gpu_vsa_f16 import f16_sparse_operands
    from test_oracle_vsa import reference_device_inputs

    rng = np.random.default_rng(13)
    heads = 2
    lengths = np.array([64, 40, 64, 64, 9, 64, 64, 33, 64], np.int32)
    blocks = len(lengths)
    n, w = 64 * blocks, heads * 128
    q, k, v = (to_dev(x, dev) for x in f16_sparse_operands(rng, heads, lengths))
    routes = to_dev(random_routes(rng, heads, blocks, 1, 0.4), dev)
    ln = to_dev(lengths, dev)
    cfg = H.AttentionCfg(w, w, w, n, n, H.config_f32(1 / math.sqrt(128)))
    out = torch.zeros((n, w), dtype=torch.float16, device=dev)
    print("graph: f16 vsa attention", flush=True)
    replay_matches(torch, dev, lambda: H.vsa_attention_f16(cfg, n, heads, q, k, v, out, routes, ln),
                   [out])

    heads, src, inverse, lengths, prefix, keep, data, gates = reference_device_inputs()
    t, w = len(inverse), heads * 128
    vsa = H.Vsa(src, inverse, lengths, prefix, heads, H.VsaOptions(keep_percent=keep), bits=16)
    qd, kd, vd = (torch_f16(d, dev) for d in data)
    gate = torch_f16(gates, dev)
    rout = torch.zeros((t * w,), dtype=torch.int16, device=dev)
    gout = torch.zeros_like(rout)

    def run():
        vsa.attend(0, qd, kd, vd, rout)
        vsa.attend(0, qd, kd, vd, gout, gate=gate)

    print("graph: bits-16 vsa runtime", flush=True)
    replay_matches(torch, dev, run, [rout, gout])
    vsa.close()


@pytest.mark.parametrize("smooth", [False, True])
def test_stack_fused_route_branches_replay_from_a_graph(dev, smooth):
    """h3_stack_attend_fused forks the Q, K and V preparations onto the stack's side streams and
    joins them before the attention; captured from the caller's stream, the branches join the
    graph and every replay gives the eager output bit for bit."""
    import torch

    from test_gpu_stack import fused_inputs

    tokens, heads = 4100, 2
    rng = np.random.default_rng(41)
    fused, qw, kw, cos_t, sin_t = fused_inputs(rng, tokens, heads)
    st = H.Stack(heads, tokens, ksmooth=smooth, fused=True)
    args = [to_dev(a, dev) for a in (fused, qw, kw, cos_t, sin_t)]
    out = torch.zeros((tokens, heads * 128), dtype=torch.float16, device=dev)
    print(f"graph: stack fused route, smooth={smooth}", flush=True)
    replay_matches(torch, dev, lambda: st.attend_fused(tokens, *args, out), [out])
    st.close()
