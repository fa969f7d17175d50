"""The host mirror of the reference's Stack (src/stack.rs) end to end on the GPU: route selection,
operand buffers and the attention output against the oracle's composition of the same steps."""
import math

import numpy as np
import pytest

import h3attn as H
import oracle as O
from helpers import from_dev, north_star_ok, read_device, to_dev

pytestmark = pytest.mark.gpu


def fused_inputs(rng, tokens, heads, k_offset_sigma=math.sqrt(2.0)):
    """BASELINE-style inputs: N(0,1) Q/K/V, K with a per-channel offset of variance 2."""
    width = heads * 128
    f = rng.standard_normal((tokens, 3 * width), np.float32)
    f[:, width:2 * width] += (rng.standard_normal(width) * k_offset_sigma).astype(np.float32)
    angles = rng.uniform(-math.pi, math.pi, (tokens, 48)).astype(np.float32)
    return (O.f16_bits(f), np.ones(128, np.float32), np.ones(128, np.float32),
            np.cos(angles).astype(np.float32), np.sin(angles).astype(np.float32))


def oracle_attention(fused, qw, kw, cos_t, sin_t, tokens, heads, cap, smooth, rows):
    width = heads * 128
    q = O.rope_qknorm_f16(fused, O.F16, tokens, 3 * width, 0, heads, qw, cos_t, sin_t, 1e-5)
    k = O.rope_qknorm_f16(fused, O.F16, tokens, 3 * width, width, heads, kw, cos_t, sin_t, 1e-5)
    mean = O.colmean(k, O.F16, tokens, width, width) if smooth else None
    extra = O.config_f32(O.EXTRA_Q_F64)
    qw_, qs = O.prepare_qk(q, O.F16, None, tokens, width, 0, heads, extra, True, cap)
    kw_, ks = O.prepare_qk(k, O.F16, mean, tokens, width, 0, heads, 1.0, True, cap)
    vt = O.transpose(fused, O.F16, tokens, 3 * width, 2 * width, width, cap, cap)
    qc = O.unpack(qw_).reshape(heads, cap, 128)
    kc = O.unpack(kw_).reshape(heads, cap, 128)
    return O.attention_f64(qc, qs, kc, ks, vt, tokens, cap, heads, rows), (qw_, qs, kw_, ks, vt)


@pytest.mark.parametrize("tokens,heads,smooth", [(4096, 4, False), (5000, 2, True)])
def test_stack_fused_route_matches_oracle(dev, tokens, heads, smooth):
    import torch

    rng = np.random.default_rng(tokens)
    fused, qw, kw, cos_t, sin_t = fused_inputs(rng, tokens, heads)
    st = H.Stack(heads, tokens, ksmooth=smooth, fused=True)
    cap = st.capacity
    assert cap == O.capacity(tokens)
    out = torch.zeros((tokens, heads * 128), dtype=torch.float16, device=dev)
    st.attend_fused(tokens, to_dev(fused, dev), to_dev(qw, dev), to_dev(kw, dev),
                    to_dev(cos_t, dev), to_dev(sin_t, dev), out)
    torch.cuda.synchronize()
    rows = np.array([0, 1, 127, 128, tokens // 2, tokens - 1], np.int32)
    want, (qw_, qs, kw_, ks, vt) = oracle_attention(fused, qw, kw, cos_t, sin_t, tokens, heads,
                                                    cap, smooth, rows)
    ops = st.operands()
    assert ops.head_major == 1
    # the operands the stack prepared are bit-exact with the oracle's
    for view, want_arr in ((ops.qi, qw_), (ops.qs, qs), (ops.ki, kw_), (ops.ks, ks)):
        got_b = read_device(view)
        w = np.ascontiguousarray(want_arr).view(np.uint8).reshape(-1)
        assert np.array_equal(got_b[:w.size], w)
    got_vt = read_device(ops.vt).view(np.uint16).reshape(heads * 128, cap)
    assert np.array_equal(got_vt[:, :tokens], vt[:, :tokens]) and (got_vt[:, tokens:] == 0).all()
    got = from_dev(out).view(np.float16).astype(np.float64).reshape(tokens, heads, 128)
    mx, mean = north_star_ok(got[rows], want)
    assert mx <= 2e-2 and mean <= 2e-3, (mx, mean)
    assert np.all(np.isfinite(got))
    st.close()


@pytest.mark.parametrize("tokens,heads,smooth", [(1024, 8, True), (1024, 8, False),
                                                 (4500, 2, True)])
def test_stack_separate_route_matches_oracle(dev, tokens, heads, smooth):
    """Stack::attend on post-RoPE Q/K and V: token-major below 4096 tokens, head-major above."""
    import torch

    rng = np.random.default_rng(tokens + 1)
    width = heads * 128
    fused, qw, kw, cos_t, sin_t = fused_inputs(rng, tokens, heads)
    q = O.rope_qknorm_f16(fused, O.F16, tokens, 3 * width, 0, heads, qw, cos_t, sin_t, 1e-5)
    k = O.rope_qknorm_f16(fused, O.F16, tokens, 3 * width, width, heads, kw, cos_t, sin_t, 1e-5)
    v = np.ascontiguousarray(fused.reshape(tokens, 3 * width)[:, 2 * width:])
    st = H.Stack(heads, tokens, ksmooth=smooth, fused=False)
    cap = st.capacity
    out = torch.zeros((tokens, width), dtype=torch.float16, device=dev)
    st.attend(tokens, to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), out)
    torch.cuda.synchronize()
    rows = np.array([0, 63, 64, tokens - 1], np.int32)
    want, _ = oracle_attention(fused, qw, kw, cos_t, sin_t, tokens, heads, cap, smooth, rows)
    got = from_dev(out).view(np.float16).astype(np.float64).reshape(tokens, heads, 128)
    mx, mean = north_star_ok(got[rows], want)
    assert mx <= 2e-2 and mean <= 2e-3, (mx, mean)
    st.close()


def test_stack_refuses_short_output(dev):
    import torch

    st = H.Stack(2, 4096, fused=True)
    small = torch.zeros(10, dtype=torch.float16, device=dev)
    with pytest.raises(H.H3Error) as e:
        st.attend_fused(4096, small, small, small, small, small, small)
    assert e.value.status == H.H3_ERR_BINDING
    st.close()
