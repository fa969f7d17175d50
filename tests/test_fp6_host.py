"""The FP6 form of the int4 attention on a CPU host: the code table maps every signed nibble c
(-8..7) to the FP6 E2M3 code of c/2 exactly (checked against the format's definition, and a
planted c-for-c/2 mapping fails), the restated workspace rows decode to the codes' halves with
-8 included, and the entry point refuses short or null workspaces with the binding errors of the
_ws forms before touching a device."""
import ctypes

import numpy as np

import h3attn as H
import oracle as O
from helpers import FP6_HALF_CODES, e2m3_value, fp6_decode_rows, fp6_rows


def test_code_table_is_half_the_nibble_in_e2m3():
    nib = np.arange(16)
    c = np.where(nib < 8, nib, nib - 16)
    assert np.array_equal(e2m3_value(FP6_HALF_CODES), c / 2.0)
    # every representable half-integer in [-4, 3.5] and no other code gives it
    vals = e2m3_value(np.arange(64))
    for v in c / 2.0:
        assert np.count_nonzero(vals == v) == (2 if v == 0 else 1)  # +0 and -0
    # a planted mapping of c itself: 5 and 7 have no E2M3 code, -8 is out of range
    assert not np.isin(np.array([5.0, 7.0, -8.0]) * 2, vals).all()


def test_restated_rows_decode_to_the_halves_of_the_codes():
    rng = np.random.default_rng(3)
    tokens, heads, cap = 37, 3, 64
    codes = rng.integers(-8, 8, (tokens, heads * 128)).astype(np.int8)
    codes[0, :128] = -8
    codes[1, :128] = 7
    from test_gpu_i4 import pack_i4
    words = pack_i4(codes)
    rows = fp6_rows(words, heads, tokens, cap)
    got = fp6_decode_rows(rows).reshape(heads, cap, 128)[:, :tokens]
    want = codes.reshape(tokens, heads, 128).transpose(1, 0, 2) / 2.0
    assert np.array_equal(got, want)
    assert np.array_equal(O.unpack_i4(words).reshape(tokens, heads, 128).transpose(1, 0, 2) / 2.0,
                          want)
    pad = rows.reshape(heads, cap, 4, 32)[:, :, :, 24:]
    assert not pad.any()


def test_fp6_workspace_is_checked():
    heads, tokens = 3, 500
    cap = H.capacity(tokens)
    w = heads * 128
    a = H.AttentionCfg(w, w, w, tokens, cap, 1.0)
    r = lambda x: (x + 255) // 256 * 256
    need = 2 * r(heads * cap * 128) + 2 * r(heads * cap * 4)
    assert H.fp6_workspace_bytes(a) == need
    big = H.raw_view(0x1000, 1 << 28)
    L = H.lib()
    st = L.h3_attention_i4qk_fp6(ctypes.byref(a), tokens, heads, big, big, big, big, big, big,
                                 H.raw_view(0x1000, need - 4), None)
    assert st == H.H3_ERR_BINDING
    assert H.last_error() == (f"attention_i4qk_fp6: workspace is {need - 4} bytes, the kernel "
                              f"addresses {need}")
    st = L.h3_attention_i4qk_fp6(ctypes.byref(a), tokens, heads, big, big, big, big, big, big,
                                 H.raw_view(0, need), None)
    assert st == H.H3_ERR_ARGUMENT and "null workspace" in H.last_error()
    # the int4 operands' extents: q codes [cap][q_stride/2 bytes]
    st = L.h3_attention_i4qk_fp6(ctypes.byref(a), tokens, heads, H.raw_view(0x1000, cap * w // 2 - 1),
                                 big, big, big, big, big, H.raw_view(0x1000, need), None)
    assert st == H.H3_ERR_BINDING and "binding 0" in H.last_error()


def test_fp6_and_f16_vsa_refuse_misaligned_rows():
    heads, tokens = 2, 256
    cap = H.capacity(tokens)
    w = heads * 128
    a = H.AttentionCfg(w, w, w, tokens, cap, 1.0)
    big, odd = H.raw_view(0x1000, 1 << 28), H.raw_view(0x1008, 1 << 28)
    L = H.lib()
    st = L.h3_attention_i4qk_fp6(ctypes.byref(a), tokens, heads, odd, big, big, big, big, big,
                                 big, None)
    assert st == H.H3_ERR_ARGUMENT and "not 16-byte aligned" in H.last_error()
    st = L.h3_attention_i4qk_fp6(ctypes.byref(a), tokens, heads, big, big, big, big, big, big,
                                 odd, None)
    assert st == H.H3_ERR_ARGUMENT and "binding 2 is not 16-byte aligned" in H.last_error()
    v = H.AttentionCfg(w, w, w, 256, 256, 0.088)
    st = L.h3_vsa_attention_f16(ctypes.byref(v), 256, heads, big, big, odd, big, big, big, None)
    assert st == H.H3_ERR_ARGUMENT and "binding 2 is not 16-byte aligned" in H.last_error()
