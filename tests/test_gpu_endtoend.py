"""Full-size paths end to end on sampled rows, and the token-major kernels past one launch.

- BASELINE config 3 as bench.py times it: bf16 fused QKV (N(0,1), K offset N(0,2) per channel,
  3D RoPE) -> prepare_qk_rope_i8hm(Q), prepare_qk_rope_i8hm(K), transpose_qkv_v_f16,
  attention_i8qkhm. On sampled rows the Q and K operands equal the oracle's RoPE + quantizer
  (rope_qknorm_f16 then prepare_qk head-major, the route the fused kernel restates) bit for bit
  and the V^T columns the oracle's transpose; sampled output rows match the f64 attention of the
  operands (the oracle's Q rows over the GPU's K and V^T, which the row checks pin) at the north
  star's max-abs 2e-2 / mean-abs 2e-3.
- BASELINE config 5(a), int4 QK at S = 129,024, H = 32: prepare_qk_i4 of Q and K from the same
  fused rows (codes and scales of sampled rows equal the oracle's), attention_i4qk and its _ws
  form (bit-identical), the skip twin at tau = 1000 (bit-identical to attention_i4qk) and at
  tau = 2 (finite), and sampled rows of attention_i4qk against the f64 attention of the read-back
  codes (tests/kernels.rs:1994-2019 style sampled-row checks); the FP6 form
  (h3_attention_i4qk_fp6, NaN-filled workspace) finite and on the same sampled rows within the
  same tolerance.
- The token-major kernels (i8qk, i4qk, i4qks; plain and _ws) split their work into launches of
  16 * CUs items; 1100 workload heads over 1000 tokens (128-query blocks) make three launches
  on 256 CUs, the last one partial. Heads wrap
  onto the two key/value and output heads, so every launch rewrites the same rows with the same
  values and the last launch's writes are what remains: all rows are checked against the oracle.
"""
import math

import numpy as np
import pytest

import bench as B
import h3attn as H
import oracle as O
from helpers import from_dev, north_star_ok, to_dev

pytestmark = pytest.mark.gpu


def fused_qkv(torch, dev, tokens, width, seed):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    fused = torch.randn((tokens, 3 * width), generator=g, device=dev, dtype=torch.float32)
    fused[:, width:2 * width] += torch.randn((width,), generator=g, device=dev) * math.sqrt(2.0)
    return fused.to(torch.bfloat16)


def sample_rows(rng, tokens):
    edges = [0, 1, 31, 32, 255, 256, tokens // 2, tokens - 2, tokens - 1]
    return np.unique(np.concatenate([edges, rng.integers(0, tokens, 7)])).astype(np.int32)


def test_config3_bench_step_end_to_end(dev):
    import torch

    tokens, heads, grid = B.WORKLOADS["c3"]
    width = heads * 128
    cap = H.capacity(tokens)
    fused = fused_qkv(torch, dev, tokens, width, 1234)
    cos_t, sin_t = B.rope_tables(torch, dev, tokens, grid)
    one = torch.ones(128, device=dev)
    qi = torch.zeros(heads * cap * 32, dtype=torch.int32, device=dev)
    ki = torch.zeros_like(qi)
    qs = torch.zeros(heads * cap, dtype=torch.float32, device=dev)
    ks = torch.zeros_like(qs)
    vt = torch.zeros(width * cap, dtype=torch.float16, device=dev)
    out = torch.zeros((tokens, width), dtype=torch.float16, device=dev)
    elem = H.H3_ELEM_BF16
    print("C3 step: prepare Q, K, V^T, attention", flush=True)
    H.prepare_qk_rope_i8hm(H.PrepareCfg(3 * width, 0, heads, H.EXTRA_Q, cap, 1e-5, elem), tokens,
                           fused, one, cos_t, sin_t, qi, qs)
    H.prepare_qk_rope_i8hm(H.PrepareCfg(3 * width, width, heads, 1.0, cap, 1e-5, elem), tokens,
                           fused, one, cos_t, sin_t, ki, ks)
    H.transpose_qkv_v_f16(H.TransposeCfg(width, cap, elem), tokens, tokens, fused, vt)
    cfg = H.AttentionCfg(width, width, width, tokens, cap, H.config_f32(1.0 / math.sqrt(128.0)))
    H.attention_i8qkhm(cfg, tokens, heads, qi, qs, ki, ks, vt, out)
    torch.cuda.synchronize()

    rng = np.random.default_rng(3)
    rows = sample_rows(rng, tokens)
    n = len(rows)
    x = from_dev(fused[torch.from_numpy(rows).long().to(dev)].contiguous().view(torch.int16))
    ct, st = cos_t.cpu().numpy()[rows], sin_t.cpu().numpy()[rows]
    w1 = np.ones(128, np.float32)
    extra = O.config_f32(O.EXTRA_Q_F64)
    gq = O.unpack(from_dev(qi).reshape(heads, cap, 32))
    gk = O.unpack(from_dev(ki).reshape(heads, cap, 32))
    gqs, gks = qs.cpu().numpy().reshape(heads, cap), ks.cpu().numpy().reshape(heads, cap)
    for part, offset, ex, codes, scales in (("Q", 0, extra, gq, gqs), ("K", width, 1.0, gk, gks)):
        r16 = O.rope_qknorm_f16(x, O.BF16, n, 3 * width, offset, heads, w1, ct, st, 1e-5)
        wc, wsc = O.prepare_qk(r16, O.F16, np.zeros(width, np.float32), n, width, 0, heads, ex,
                               True, n)
        wc = O.unpack(wc.reshape(heads, n, 32))
        assert np.array_equal(codes[:, rows], wc), f"{part} codes differ from the oracle's"
        assert np.array_equal(scales[:, rows].view(np.uint32), wsc.view(np.uint32)), part
    gvt = from_dev(vt.view(torch.int16)).reshape(width, cap)
    wvt = O.transpose(x, O.BF16, n, 3 * width, 2 * width, width, n, n)
    assert np.array_equal(gvt[:, rows], wvt)
    assert not gvt[:, tokens:].any()
    # the f64 attention of the operands: the oracle's Q rows (equal to the GPU's) over all keys
    qc = np.zeros((heads, cap, 128), np.int8)
    qsc = np.zeros((heads, cap), np.float32)
    qc[:, rows], qsc[:, rows] = gq[:, rows], gqs[:, rows]
    want = O.attention_f64(qc, qsc, gk, gks, gvt, tokens, cap, heads, rows)
    got = from_dev(out).view(np.float16).astype(np.float64).reshape(tokens, heads, 128)[rows]
    mx, mean = north_star_ok(got, want)
    assert mx < 2e-2 and mean < 2e-3, (mx, mean)
    assert bool(torch.isfinite(out).all())


def test_config5a_int4_at_full_size(dev):
    import torch

    tokens, heads, _ = B.WORKLOADS["c3"]
    width = heads * 128
    cap = H.capacity(tokens)
    fused = fused_qkv(torch, dev, tokens, width, 55)
    qi = torch.zeros((cap, width // 8), dtype=torch.int32, device=dev)
    ki = torch.zeros_like(qi)
    qs = torch.zeros((cap, heads), dtype=torch.float32, device=dev)
    ks = torch.zeros_like(qs)
    elem = H.H3_ELEM_BF16
    print("5a: int4 operands", flush=True)
    H.prepare_qk_i4(H.PrepareCfg(3 * width, 0, heads, H.EXTRA_Q, cap, 1e-5, elem), tokens, fused,
                    None, qi, qs)
    H.prepare_qk_i4(H.PrepareCfg(3 * width, width, heads, 1.0, cap, 1e-5, elem), tokens, fused,
                    None, ki, ks)
    vt = torch.zeros(width * cap, dtype=torch.float16, device=dev)
    H.transpose_qkv_v_f16(H.TransposeCfg(width, cap, elem), tokens, tokens, fused, vt)
    cfg = H.AttentionCfg(width, width, width, tokens, cap, 1.0)
    args = (cfg, tokens, heads, qi, qs, ki, ks, vt)
    outs = {}
    for name in ("plain", "ws", "tau1000", "tau2"):
        outs[name] = torch.full((tokens, width), float("nan"), dtype=torch.float16, device=dev)
    ws = torch.full((H.scales_workspace_bytes(cfg) // 4,), float("nan"), dtype=torch.float32,
                    device=dev)
    print("5a: attention_i4qk, _ws, skip twin tau=1000 and tau=2", flush=True)
    H.attention_i4qk(*args, outs["plain"])
    H.attention_i4qk_ws(*args, outs["ws"], ws)
    for tau, name in ((1000.0, "tau1000"), (2.0, "tau2")):
        sc = H.AttentionSkipCfg(width, width, width, tokens, cap, 1.0, tau)
        H.attention_i4qks_ws(sc, tokens, heads, qi, qs, ki, ks, vt, outs[name], ws)
    print("5a: attention_i4qk_fp6", flush=True)
    outs["fp6"] = torch.full((tokens, width), float("nan"), dtype=torch.float16, device=dev)
    ws6 = torch.full((H.fp6_workspace_bytes(cfg) // 4,), float("nan"), dtype=torch.float32,
                     device=dev)
    H.attention_i4qk_fp6(*args, outs["fp6"], ws6)
    torch.cuda.synchronize()
    del ws6
    plain = from_dev(outs["plain"])
    assert np.array_equal(from_dev(outs["ws"]), plain)
    assert np.array_equal(from_dev(outs["tau1000"]), plain)
    assert bool(torch.isfinite(outs["tau2"]).all()) and bool(torch.isfinite(outs["plain"]).all())

    rng = np.random.default_rng(5)
    rows = sample_rows(rng, tokens)
    x = from_dev(fused[torch.from_numpy(rows).long().to(dev)].contiguous().view(torch.int16))
    gqi, gki = from_dev(qi), from_dev(ki)
    gqs, gks = qs.cpu().numpy(), ks.cpu().numpy()
    for part, offset, ex, codes, scales in (("Q", 0, H.EXTRA_Q, gqi, gqs),
                                             ("K", width, 1.0, gki, gks)):
        wc, wsc = O.prepare_qk_i4(x, O.BF16, None, len(rows), 3 * width, offset, heads, ex)
        assert np.array_equal(codes[rows], wc), f"{part} int4 codes differ from the oracle's"
        assert np.array_equal(scales[rows].view(np.uint32), wsc.view(np.uint32)), part
    qc = O.unpack_i4(gqi).reshape(cap, heads, 128).transpose(1, 0, 2).copy()
    kc = O.unpack_i4(gki).reshape(cap, heads, 128).transpose(1, 0, 2).copy()
    gvt = from_dev(vt.view(torch.int16)).reshape(width, cap)
    want = O.attention_f64(qc, gqs.T.copy(), kc, gks.T.copy(), gvt, tokens, cap, heads, rows)
    got = plain.view(np.float16).astype(np.float64).reshape(tokens, heads, 128)[rows]
    mx, mean = north_star_ok(got, want)
    assert mx < 2e-2 and mean < 2e-3, (mx, mean)
    got6 = from_dev(outs["fp6"]).view(np.float16).astype(np.float64).reshape(tokens, heads, 128)
    mx, mean = north_star_ok(got6[rows], want)
    print(f"5a fp6 sampled rows: max {mx:.3e} mean {mean:.3e}", flush=True)
    assert mx < 2e-2 and mean < 2e-3, (mx, mean)
    assert np.isfinite(got6).all()


def test_token_major_kernels_past_one_launch(dev):
    import torch

    tokens, heads, kv_heads = 1000, 1100, 2
    stride = kv_heads * 128
    cap = H.capacity(tokens)
    rng = np.random.default_rng(1024)
    q = rng.integers(-7, 8, (cap, stride)).astype(np.int8)
    k = rng.integers(-7, 8, (cap, stride)).astype(np.int8)
    q[tokens:] = 0
    k[tokens:] = 0
    qs = rng.uniform(0.005, 0.05, (cap, kv_heads)).astype(np.float32)
    ks = rng.uniform(0.005, 0.05, (cap, kv_heads)).astype(np.float32)
    v = O.f16_bits(rng.standard_normal((tokens, stride)).astype(np.float32)).reshape(tokens, stride)
    vt = O.transpose(v, O.F16, tokens, stride, 0, stride, cap, cap)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    items = -(-tokens // 128) * heads  # 128-query blocks x heads
    gen = 16 * cus
    assert items > 2 * gen and items % gen != 0  # three launches or more, the last one partial
    cfg = H.AttentionCfg(stride, stride, stride, tokens, cap, 1.0)
    scfg = H.AttentionSkipCfg(stride, stride, stride, tokens, cap, 1.0, 1000.0)
    rows = np.arange(tokens, dtype=np.int32)
    qc = q.reshape(cap, kv_heads, 128).transpose(1, 0, 2).copy()
    kc = k.reshape(cap, kv_heads, 128).transpose(1, 0, 2).copy()
    want = O.attention_f64(qc, qs.T.copy(), kc, ks.T.copy(), vt, tokens, cap, kv_heads, rows)
    from test_gpu_i4 import pack_i4

    dv = {name: to_dev(a, dev) for name, a in (("qs", qs), ("ks", ks), ("vt", vt))}
    ws = torch.full((H.scales_workspace_bytes(cfg) // 4,), float("nan"), dtype=torch.float32,
                    device=dev)
    forms = [("i8qk", cfg, q.view(np.int32), k.view(np.int32), H.attention_i8qk, H.attention_i8qk_ws),
             ("i4qk", cfg, pack_i4(q), pack_i4(k), H.attention_i4qk, H.attention_i4qk_ws),
             ("i4qks", scfg, pack_i4(q), pack_i4(k), H.attention_i4qks, H.attention_i4qks_ws)]
    for name, c, qq, kk, plain, lent in forms:
        for form, fn, extra in (("plain", plain, ()), ("ws", lent, (ws,))):
            print(f"past one launch: {name} {form} heads={heads}", flush=True)
            out = torch.full((tokens, stride), float("nan"), dtype=torch.float16, device=dev)
            fn(c, tokens, heads, to_dev(qq, dev), dv["qs"], to_dev(kk, dev), dv["ks"], dv["vt"],
               out, *extra)
            torch.cuda.synchronize()
            got = from_dev(out).view(np.float16).astype(np.float64).reshape(tokens, kv_heads, 128)
            mx, mean = north_star_ok(got, want)
            assert mx < 2e-2 and mean < 2e-3, (name, form, mx, mean)
