"""The compact route end to end on the GPU: the INT8 QKV projection writes Q/K rows and V^T
(h3_gemm_i8_qkv_256), Stack::prepare_fused_operands reads them in place
(h3_stack_attend_compact, src/stack.rs:634-661, 1034-1040, 1561-1600), and the attention output
is byte-identical to the fused route run on the same projection laid out as [t][3*inner] rows
(h3_stack_attend_fused: RoPE quantizers over 3*inner rows plus the V transpose). The output is
also checked against the oracle's attention of those operands at the north-star tolerance."""
import math

import numpy as np
import pytest

import h3attn as H
import oracle as O
from helpers import from_dev, north_star_ok, to_dev
from test_gpu_stack import oracle_attention

pytestmark = pytest.mark.gpu


def projection_inputs(rng, tokens, hidden, n):
    a = rng.integers(-128, 128, (tokens, hidden), dtype=np.int8)
    w = rng.integers(-128, 128, (n, hidden), dtype=np.int8)
    # scales that give Q/K/V entries of order one, like normalised activations
    ws = np.full(n, 1.0 / (128.0 * math.sqrt(hidden)), np.float32) * rng.uniform(0.5, 2.0, n).astype(np.float32)
    as_ = rng.uniform(0.5, 1.5, tokens).astype(np.float32) / 128.0 * 1.7
    return a, w, ws, as_


@pytest.mark.parametrize("tokens,heads,smooth", [(5000, 2, False), (5000, 2, True),
                                                 (31104, 1, False)])
def test_compact_route_is_byte_identical_to_the_fused_route(dev, tokens, heads, smooth):
    import torch

    inner = heads * 128
    n, hidden = 3 * inner, 256
    rng = np.random.default_rng(tokens + heads)
    a, w, ws, as_ = projection_inputs(rng, tokens, hidden, n)
    angles = rng.uniform(-math.pi, math.pi, (tokens, 48)).astype(np.float32)
    cos_t, sin_t = np.cos(angles).astype(np.float32), np.sin(angles).astype(np.float32)
    qw = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    kw = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    print(f"compact route tokens={tokens} heads={heads} smooth={smooth}", flush=True)

    compact = torch.empty(H.compact_qkv_elements(tokens, n), dtype=torch.int16, device=dev)
    H.gemm_i8_qkv_256(H.GemmCfg(hidden, n, hidden, 1), tokens, to_dev(a, dev), to_dev(w, dev),
                      to_dev(ws, dev), to_dev(as_, dev), compact)
    d = {k: to_dev(v, dev) for k, v in dict(qw=qw, kw=kw, cos=cos_t, sin=sin_t).items()}

    st = H.Stack(heads, tokens, ksmooth=smooth, fused=True)
    cap = st.capacity
    assert cap == -(-tokens // 256) * 256
    out_c = torch.zeros((tokens, inner), dtype=torch.float16, device=dev)
    st.attend_compact(tokens, compact, d["qw"], d["kw"], d["cos"], d["sin"], out_c)

    # the same projection as fused [t][3*inner] rows: Q|K rows, then V = (V^T)^T
    host = from_dev(compact)
    qk = host[:tokens * 2 * inner].reshape(tokens, 2 * inner)
    vt = host[tokens * 2 * inner:].reshape(inner, cap)
    assert np.all(vt[:, tokens:] == 0)
    fused = np.ascontiguousarray(np.concatenate([qk, vt[:, :tokens].T], axis=1))
    st2 = H.Stack(heads, tokens, ksmooth=smooth, fused=True)
    out_f = torch.zeros((tokens, inner), dtype=torch.float16, device=dev)
    st2.attend_fused(tokens, to_dev(fused, dev), d["qw"], d["kw"], d["cos"], d["sin"], out_f)
    torch.cuda.synchronize()
    got_c, got_f = from_dev(out_c), from_dev(out_f)
    assert np.array_equal(got_c, got_f)

    rows = np.array([0, 1, 255, 256, tokens // 2, tokens - 1], np.int32)
    want, _ = oracle_attention(fused, qw, kw, cos_t, sin_t, tokens, heads, cap, smooth, rows)
    got = got_c.view(np.float16).astype(np.float64).reshape(tokens, heads, 128)
    mx, mean = north_star_ok(got[rows], want)
    assert mx <= 2e-2 and mean <= 2e-3, (mx, mean)
    st.close()
    st2.close()


def test_compact_route_preconditions(dev):
    import torch

    small = torch.zeros(16, dtype=torch.float16, device=dev)
    st = H.Stack(2, 4096, fused=True)  # capacity 4128 != 4096: no compact route
    with pytest.raises(H.H3Error) as e:
        st.attend_compact(4096, small, small, small, small, small, small)
    assert e.value.status == H.H3_ERR_ARGUMENT
    st.close()
    st = H.Stack(2, 5000, fused=True)
    with pytest.raises(H.H3Error) as e:
        st.attend_compact(4999, small, small, small, small, small, small)
    assert e.value.status == H.H3_ERR_ARGUMENT
    with pytest.raises(H.H3Error) as e:
        st.attend_compact(5000, small, small, small, small, small, small)
    assert e.value.status == H.H3_ERR_BINDING
    st.close()
