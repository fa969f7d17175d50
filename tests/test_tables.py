"""rope::dit on the host (h3_rope_dit_tables), against the reference's own checks of it
(src/rope.rs:325-351 assert_dit_matches_scalar, 353-403, 405-418, 420-425): every entry equals,
bit for bit, cosf/sinf of the float angle (float)pos * inv_freq[j], for media grids, repeated
coordinates, signed zeros, doubles that narrow to one float, huge and tiny positions, and
negative or zero frequencies. The scalar side calls the C library's cosf/sinf through ctypes,
the functions the reference's f32::cos/f32::sin reach on this platform. Host only: no GPU."""
import ctypes
import ctypes.util

import numpy as np
import pytest

import h3attn as H

_libm = ctypes.CDLL(ctypes.util.find_library("m"))
_libm.cosf.argtypes = [ctypes.c_float]
_libm.cosf.restype = ctypes.c_float
_libm.sinf.argtypes = [ctypes.c_float]
_libm.sinf.restype = ctypes.c_float


def scalar_tables(pos, inv):
    rows = len(pos) // 3
    c = np.empty((rows, 48), np.float32)
    s = np.empty((rows, 48), np.float32)
    for r in range(rows):
        for ax in range(3):
            p = np.float32(pos[3 * r + ax])
            for j in range(16):
                angle = float(np.float32(p * np.float32(inv[j])))
                c[r, 16 * ax + j] = _libm.cosf(angle)
                s[r, 16 * ax + j] = _libm.sinf(angle)
    return c, s


def assert_matches_scalar(pos, inv):
    pos = np.asarray(pos, np.float64)
    inv = np.asarray(inv, np.float32)
    c, s = H.rope_dit_tables(pos.reshape(-1, 3), inv)
    wc, wsn = scalar_tables(pos, inv)
    assert np.array_equal(c.view(np.uint32), wc.view(np.uint32))
    assert np.array_equal(s.view(np.uint32), wsn.view(np.uint32))


def grid_positions(frames, h, w, t_scale=1.0, s_scale=0.0625):
    t, y, x = np.meshgrid(np.arange(frames) * t_scale, np.arange(h) * s_scale,
                          np.arange(w) * s_scale, indexing="ij")
    return np.stack([t, y, x], -1).reshape(-1)


@pytest.mark.parametrize("frames,h,w", [(2, 4, 4), (7, 12, 20), (3, 42, 96)])
def test_tables_match_scalar_for_media_grids(frames, h, w):
    inv = np.array([np.float32(10000.0) ** np.float32(-np.float32(j) / np.float32(16.0))
                    for j in range(16)], np.float32)
    assert_matches_scalar(grid_positions(frames, h, w), inv)


def test_tables_preserve_float_rounding_and_signed_zero():
    pos = []
    for p in [0.0, -0.0, 1.0, 1.0 + np.finfo(np.float64).eps, -0.125, 1e7, 1e20, 1e-40]:
        pos += [p, p, p]
    pos += list(np.arange(4096 * 3) * 0.123456789)
    for freq in [1.0 / 3.0, -0.25, 0.0]:
        assert_matches_scalar(pos, [freq] * 16)
    c, s = H.rope_dit_tables(np.zeros((0, 3)), np.full(16, 0.5, np.float32))
    assert c.shape == (0, 48) and s.shape == (0, 48)


def test_signed_zero_position_keeps_the_sign_of_the_sine():
    c, s = H.rope_dit_tables(np.array([[0.0, -0.0, 0.0]]), np.full(16, 0.5, np.float32))
    assert np.all(c == 1.0)
    assert np.all(np.signbit(s[0, 16:32])) and not np.any(np.signbit(s[0, :16]))


def test_every_table_starts_at_the_identity_rotation():
    c, s = H.rope_dit_tables(np.zeros((1, 3)), np.full(16, 0.5, np.float32))
    assert np.all(c == 1.0) and np.all(s == 0.0)


def test_bad_arguments_are_refused():
    lib = H.lib()
    assert lib.h3_rope_dit_tables(None, 3, None, None, None) == H.H3_ERR_ARGUMENT
    with pytest.raises(ValueError):
        H.rope_dit_tables(np.zeros((2, 3)), np.zeros(8, np.float32))
