"""h3_attention_i8qk_static, the allocation-free form of h3_attention_i8qk_ws, through the C ABI.

The static form takes no workspace: the library's 8 MiB device array stands in for it. Two calls
in a row (the second with fewer tokens and heads, after a larger one has filled the array) must
equal h3_attention_i8qk_ws with a lent NaN-filled workspace bit for bit, and h3_attention_i8qk
as well (the _ws forms are bit-identical to the plain ones). A config whose head-major scale
copy exceeds 8 MiB is refused before any device work.
"""
import ctypes

import numpy as np
import pytest

import h3attn as H
import oracle as O
from helpers import from_dev, to_dev

SCRATCH_BYTES = 8 << 20


def test_static_form_refuses_more_than_its_scratch():
    heads, tokens = 32, 65537  # 32 * 65537 * 4 bytes of key scales: just past 8 MiB
    w = heads * 128
    cfg = H.AttentionCfg(w, w, w, tokens, H.capacity(tokens), 1.0)
    need = H.scales_workspace_bytes(cfg)
    assert need == heads * tokens * 4 > SCRATCH_BYTES
    big = H.raw_view(0x1000, 1 << 40)  # never dereferenced: the call fails first
    st = H.lib().h3_attention_i8qk_static(ctypes.byref(cfg), tokens, heads, big, big, big, big,
                                          big, big, None)
    assert st == H.H3_ERR_CONFIG
    assert H.last_error() == (
        f"attention_i8qk_static: (kv_stride/128) * tokens * 4 = {need} bytes of key scales exceed "
        f"the {SCRATCH_BYTES}-byte static scratch (use h3_attention_i8qk_ws with a lent workspace)")
    st = H.lib().h3_attention_i8qk_static(None, tokens, heads, big, big, big, big, big, big, None)
    assert st == H.H3_ERR_ARGUMENT


def _operands(rng, tokens, heads):
    stride = heads * 128
    cap = H.capacity(tokens)
    q = rng.integers(-7, 8, (cap, stride)).astype(np.int8)
    k = rng.integers(-7, 8, (cap, stride)).astype(np.int8)
    q[tokens:] = 0
    k[tokens:] = 0
    qs = rng.uniform(0.005, 0.05, (cap, heads)).astype(np.float32)
    ks = rng.uniform(0.005, 0.05, (cap, heads)).astype(np.float32)
    v = O.f16_bits(rng.standard_normal((tokens, stride)).astype(np.float32)).reshape(tokens, stride)
    vt = O.transpose(v, O.F16, tokens, stride, 0, stride, cap, cap)
    cfg = H.AttentionCfg(stride, stride, stride, tokens, cap, 1.0)
    return cfg, q.view(np.int32), qs, k.view(np.int32), ks, vt


@pytest.mark.gpu
def test_static_form_equals_the_workspace_form_on_two_calls(dev):
    import torch

    lib = H.lib()
    for tokens, heads in [(16000, 32), (1500, 3)]:  # 2 MB then 18 KB of scales
        print(f"static form tokens={tokens} heads={heads}", flush=True)
        rng = np.random.default_rng(tokens + heads)
        cfg, qi, qs, ki, ks, vt = _operands(rng, tokens, heads)
        assert H.scales_workspace_bytes(cfg) <= SCRATCH_BYTES
        args = [to_dev(x, dev) for x in (qi, qs, ki, ks, vt)]
        stride = heads * 128
        ws_out = torch.full((tokens * stride,), 0x7E00, dtype=torch.int16, device=dev)
        st_out = torch.full_like(ws_out, 0x7E00)
        plain_out = torch.full_like(ws_out, 0x7E00)
        ws = torch.full((H.scales_workspace_bytes(cfg) // 2,), 0x7E00, dtype=torch.int16,
                        device=dev)
        H.attention_i8qk_ws(cfg, tokens, heads, *args, ws_out, ws)
        H.attention_i8qk(cfg, tokens, heads, *args, plain_out)
        st = lib.h3_attention_i8qk_static(ctypes.byref(cfg), tokens, heads,
                                          *[H.view(a) for a in args], H.view(st_out),
                                          H.stream_ptr(None))
        assert st == H.H3_OK, H.last_error()
        torch.cuda.synchronize()
        got = from_dev(st_out)
        assert np.isfinite(got.view(np.float16)).all()
        assert np.array_equal(got, from_dev(ws_out))
        assert np.array_equal(got, from_dev(plain_out))
