"""The reference's direct-attention output pitch on the GPU.

With f16 GEMM activations the reference's Stack::build compiles its attention with
out_stride = gemm_pitch(inner, 16) (src/stack.rs:408, 751-758; src/model.rs:74-85), so the
attention writes the out projection's operand directly at a padded pitch, and it qualifies
exactly that config for the head-major kernel (tests/compiler.rs:43-45: q/kv 7168, out 7296,
56 heads). The operands are sized by the workload's heads (src/stack.rs:1830-1837), the output
by the pitch (src/stack.rs:1683). Each test binds exactly those sizes, fills the output with
guard bytes, and checks sampled rows against the f64 oracle to the north star's tolerance and
that the 128 pad columns of every row and the bytes past the output are untouched.
"""
import math

import numpy as np
import pytest

import h3attn as H
import oracle as O
from helpers import filled, from_dev, north_star_ok, pack_codes, read_device, to_dev

pytestmark = pytest.mark.gpu

GUARD = 64


def gemm_pitch16(k):
    """gemm_pitch(k, 16) (src/model.rs:74-85)."""
    return k + 128 if (2 * k) % 1024 == 0 else k


def int_operands(rng, heads, tokens, cap):
    """Head-major int8 codes (uniform in [-64, 64]), scales as check_head_major_attention's
    pattern (tests/kernels.rs:2021-2038), V^T N(0,1)*0.3 f16; capacity rows zero."""
    qc = np.zeros((heads, cap, 128), np.int8)
    kc = np.zeros((heads, cap, 128), np.int8)
    qc[:, :tokens] = rng.integers(-64, 65, (heads, tokens, 128), dtype=np.int8)
    kc[:, :tokens] = rng.integers(-64, 65, (heads, tokens, 128), dtype=np.int8)
    t = np.arange(tokens)
    qs = np.zeros((heads, cap), np.float32)
    ks = np.zeros((heads, cap), np.float32)
    qs[:, :tokens] = ((1 + t % 7) / 1024.0).astype(np.float32)
    ks[:, :tokens] = ((1 + t % 3) / 256.0).astype(np.float32)
    vt = np.zeros((heads * 128, cap), np.float16)
    vt[:, :tokens] = (rng.standard_normal((heads * 128, tokens), np.float32) * 0.3).astype(
        np.float16)
    return qc, qs, kc, ks, vt.view(np.uint16)


def check_padded_output(raw, tokens, pitch, inner, rows, want):
    body = tokens * pitch * 2
    assert (raw[body:] == 0xFF).all(), "attention wrote past the output"
    out = raw[:body].view(np.uint16).reshape(tokens, pitch)
    assert (out[:, inner:] == 0xFFFF).all(), "attention wrote into the pad columns"
    got = out[:, :inner].view(np.float16).astype(np.float64).reshape(tokens, -1, 128)
    assert np.all(np.isfinite(got))
    mx, mean = north_star_ok(got[rows], want)
    assert mx <= 2e-2 and mean <= 2e-3, (mx, mean)


@pytest.mark.parametrize("tokens", [4000, 37977])
def test_head_major_attention_at_the_reference_direct_pitch(dev, tokens):
    """56 heads, q/kv 7168, out 7296 (tests/compiler.rs:43-45), with reference-sized bindings;
    4,000 tokens run the chained kernel (at most 64 key tiles), 37,977 the unchained one."""
    import torch

    heads = 56
    inner = heads * 128
    pitch = gemm_pitch16(inner)
    assert pitch == 7296
    cap = O.capacity(tokens)
    rng = np.random.default_rng(tokens + 56)
    qc, qs, kc, ks, vt = int_operands(rng, heads, tokens, cap)
    cfg = H.AttentionCfg(inner, inner, pitch, tokens, cap, 1.0)
    out = filled((tokens * pitch * 2 + GUARD,), 0xFF, np.uint8, dev)
    print(f"head-major attention at the direct pitch: S={tokens} H={heads} out_stride={pitch}",
          flush=True)
    H.attention_i8qkhm(cfg, tokens, heads, to_dev(pack_codes(qc).reshape(heads * cap, 32), dev),
                       to_dev(qs, dev), to_dev(pack_codes(kc).reshape(heads * cap, 32), dev),
                       to_dev(ks, dev), to_dev(vt, dev), out[: tokens * pitch * 2])
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([[0, 31, 32, 255, 256, tokens - 1],
                                     rng.integers(0, tokens, 4)])).astype(np.int32)
    want = O.attention_f64(qc, qs, kc, ks, vt, tokens, cap, heads, rows)
    check_padded_output(out.cpu().numpy(), tokens, pitch, inner, rows, want)


def test_token_major_attention_at_a_direct_pitch(dev):
    """The token-major kernel under a padded output pitch: 8 heads (inner 1024, pitch 1152),
    Q scales [capacity][8] as the quantizer writes them."""
    import torch

    heads, tokens = 8, 1000
    inner = heads * 128
    pitch = gemm_pitch16(inner)
    assert pitch == 1152
    cap = max(-(-(tokens + 16) // 32) * 32, -(-tokens // 64) * 64)
    rng = np.random.default_rng(1152)
    qc, qs, kc, ks, vt = int_operands(rng, heads, tokens, cap)
    tm = lambda c: pack_codes(c.transpose(1, 0, 2)).reshape(cap, heads * 32)
    cfg = H.AttentionCfg(inner, inner, pitch, tokens, cap, 1.0)
    out = filled((tokens * pitch * 2 + GUARD,), 0xFF, np.uint8, dev)
    H.attention_i8qk(cfg, tokens, heads, to_dev(tm(qc), dev), to_dev(qs.T.copy(), dev),
                     to_dev(tm(kc), dev), to_dev(ks.T.copy(), dev), to_dev(vt, dev),
                     out[: tokens * pitch * 2])
    torch.cuda.synchronize()
    rows = np.array([0, 15, 16, 31, 32, 500, tokens - 1], np.int32)
    want = O.attention_f64(qc, qs, kc, ks, vt, tokens, cap, heads, rows)
    check_padded_output(out.cpu().numpy(), tokens, pitch, inner, rows, want)


@pytest.mark.parametrize("tokens", [1024, 4500])
def test_stack_direct_attention_route(dev, tokens):
    """Stack::build with direct_attn (f16 GEMM activations): the attention output at
    gemm_pitch(inner, 16), pad columns untouched, against the oracle's composition of the fused
    route (1,024 tokens: the separate token-major route; 4,500: the fused head-major one)."""
    import torch

    heads = 8
    inner = heads * 128
    pitch = gemm_pitch16(inner)
    rng = np.random.default_rng(tokens + 7)
    f = rng.standard_normal((tokens, 3 * inner), np.float32)
    f[:, inner:2 * inner] += (rng.standard_normal(inner) * math.sqrt(2.0)).astype(np.float32)
    fused = O.f16_bits(f)
    ones = np.ones(128, np.float32)
    ang = rng.uniform(-math.pi, math.pi, (tokens, 48)).astype(np.float32)
    cos_t, sin_t = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    head_major = tokens >= 4096
    st = H.Stack(heads, tokens, fused=head_major, direct_attn=True)
    cap = st.capacity
    out = filled((tokens * pitch * 2 + GUARD,), 0xFF, np.uint8, dev)
    body = out[: tokens * pitch * 2]
    q = O.rope_qknorm_f16(fused, O.F16, tokens, 3 * inner, 0, heads, ones, cos_t, sin_t, 1e-5)
    k = O.rope_qknorm_f16(fused, O.F16, tokens, 3 * inner, inner, heads, ones, cos_t, sin_t, 1e-5)
    if head_major:
        st.attend_fused(tokens, to_dev(fused, dev), to_dev(ones, dev), to_dev(ones, dev),
                        to_dev(cos_t, dev), to_dev(sin_t, dev), body)
    else:
        v = np.ascontiguousarray(fused.reshape(tokens, 3 * inner)[:, 2 * inner:])
        st.attend(tokens, to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), body)
    torch.cuda.synchronize()
    assert st.operands().head_major == int(head_major)
    st.close()
    extra = O.config_f32(O.EXTRA_Q_F64)
    qw, qs = O.prepare_qk(q, O.F16, None, tokens, inner, 0, heads, extra, True, cap)
    kw, ks = O.prepare_qk(k, O.F16, None, tokens, inner, 0, heads, 1.0, True, cap)
    vt = O.transpose(fused, O.F16, tokens, 3 * inner, 2 * inner, inner, cap, cap)
    rows = np.array([0, 63, 64, tokens // 2, tokens - 1], np.int32)
    want = O.attention_f64(O.unpack(qw).reshape(heads, cap, 128), qs,
                           O.unpack(kw).reshape(heads, cap, 128), ks, vt, tokens, cap, heads,
                           rows)
    check_padded_output(out.cpu().numpy(), tokens, pitch, inner, rows, want)


@pytest.mark.parametrize("tokens", [1000, 5000])
def test_fp6_attention_at_a_direct_pitch(dev, tokens):
    """h3_attention_i4qk_fp6 (int4 operands converted to FP6, the head-major kernel's FP6 form)
    under a padded output pitch: 4 heads (inner 512, pitch 640); 1,000 tokens run the chained
    kernel, 5,000 the unchained one."""
    import torch

    from test_gpu_i4 import pack_i4

    heads = 4
    inner = heads * 128
    pitch = gemm_pitch16(inner)
    assert pitch == 640
    cap = H.capacity(tokens)
    rng = np.random.default_rng(tokens + 640)
    qc, qs, kc, ks, vt = int_operands(rng, heads, tokens, cap)
    # int4 codes in [-7, 7] in place of the int8 ones (capacity rows stay zero)
    qc[:, :tokens] = rng.integers(-7, 8, (heads, tokens, 128), dtype=np.int8)
    kc[:, :tokens] = rng.integers(-7, 8, (heads, tokens, 128), dtype=np.int8)
    tm = lambda c: pack_i4(np.ascontiguousarray(c.transpose(1, 0, 2)).reshape(cap, inner))
    cfg = H.AttentionCfg(inner, inner, pitch, tokens, cap, 1.0)
    ws = torch.zeros((H.fp6_workspace_bytes(cfg),), dtype=torch.uint8, device=dev)
    out = filled((tokens * pitch * 2 + GUARD,), 0xFF, np.uint8, dev)
    print(f"fp6 attention at a direct pitch: S={tokens} H={heads} out_stride={pitch}", flush=True)
    H.attention_i4qk_fp6(cfg, tokens, heads, to_dev(tm(qc), dev), to_dev(qs.T.copy(), dev),
                         to_dev(tm(kc), dev), to_dev(ks.T.copy(), dev), to_dev(vt, dev),
                         out[: tokens * pitch * 2], ws)
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([[0, 31, 32, 255, 256, tokens - 1],
                                     rng.integers(0, tokens, 4)])).astype(np.int32)
    want = O.attention_f64(qc, qs, kc, ks, vt, tokens, cap, heads, rows)
    check_padded_output(out.cpu().numpy(), tokens, pitch, inner, rows, want)
