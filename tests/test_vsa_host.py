"""The VSA host side on a CPU host: the library's plan, budget, options checks and sigma window
(src/vsa.rs) equal the oracle's restatement, and every VSA entry point refuses bad configs and
short bindings with the reference's extents (src/vsa/device.rs:200-446) before touching a
device. No kernel is launched here."""
import ctypes

import numpy as np
import pytest

import h3attn as H
import oracle as O


def fake(nbytes):
    """A 16-byte aligned binding that is never dereferenced."""
    return H.raw_view(0x1000, nbytes)


@pytest.mark.parametrize("segs,grid", [
    ([(0, 65), (65, 6)], (5, 5, 7)),            # the reference's plan test layout
    ([], (8, 11, 24)),                           # BASELINE config 3's cube grid
    ([(0, 11), (11, 130), (141, 1)], (3, 2, 13)),
    ([(0, 64), (64, 128)], (4, 4, 4)),
    ([(0, 1)], (1, 1, 1)),
])
def test_host_plan_equals_the_oracle(segs, grid):
    seq = (segs[-1][0] + segs[-1][1] if segs else 0) + grid[0] * grid[1] * grid[2]
    got = H.vsa_plan(segs, seq, *grid)
    want = O.vsa_plan(segs, seq, *grid)
    for g, w in zip(got, want):
        assert np.array_equal(np.asarray(g), np.asarray(w))


def test_plan_refuses_uncovered_rows():
    with pytest.raises(H.H3Error, match="cover every live token"):
        H.vsa_plan([(0, 10)], 10 + 4 * 4 * 4 + 1, 4, 4, 4)   # row 10 belongs to no segment


def test_topk_and_dense_reason_equal_the_oracle():
    for kp in (0.5, 10.0, 12.5, 30.0, 50.0, 99.9, 100.0):
        for nonprefix in (0, 1, 2, 3, 5, 25, 35, 45, 2112, 16384):
            assert H.VsaOptions(keep_percent=kp).topk(nonprefix) == O.vsa_topk(kp, nonprefix)
    opt = H.VsaOptions()
    for tokens in (12287, 12288, 129024):
        for sigma in (0.0, 0.1, 0.5, 0.9, 0.95, 1.0):
            for shift in (1.0, 3.0, 10.0):
                want = O.vsa_dense_reason(opt.start, opt.end, opt.min_tokens, tokens, sigma, shift)
                assert opt.dense_reason(tokens, sigma, shift) == want


@pytest.mark.parametrize("kwargs,bits,message", [
    (dict(keep_percent=0.0), 8, "keep_percent"),
    (dict(keep_percent=100.5), 8, "keep_percent"),
    (dict(keep_percent=float("nan")), 8, "keep_percent"),
    (dict(start=0.5, end=0.4), 8, "start <= end"),
    (dict(end=1.5), 8, "start <= end"),
    (dict(min_tokens=(1 << 20) + 1), 8, "out of range"),
    (dict(dense_blocks=[50]), 8, "out of range"),
    (dict(), 4, "not i4"),
])
def test_options_validation_matches_the_reference(kwargs, bits, message):
    with pytest.raises(H.H3Error, match=message):
        H.VsaOptions(**kwargs).validate(bits)
    H.VsaOptions(dense_blocks=[0, 49]).validate(8)
    H.VsaOptions(keep_percent=100.0, start=0.0, end=0.0).validate(16)


def cfg(tokens=300, blocks=6, heads=2, prefix=1, topk=2):
    return H.VsaCfg(tokens, 64 * blocks, 128 * heads, blocks, heads, prefix, topk)


def test_vsa_bindings_follow_the_reference_extents():
    c = cfg()
    n, t, w, b, h = 384, 300, 256, 6, 2
    L = H.lib()
    cases = [
        (L.h3_vsa_gather, [n * 4, t * w * 2, n * w * 2]),
        (L.h3_vsa_scatter, [t * 4, n * w * 2, t * w * 2]),
        (L.h3_vsa_pool, [b * 4, n * w * 2, b * w * 4]),
        (L.h3_vsa_scores, [b * w * 4, b * w * 4, h * b * b * 4]),
        (L.h3_vsa_route, [h * b * b * 4, h * b * b * 4]),
        (L.h3_vsa_coarse, [h * b * b * 4, b * w * 4, b * w * 4]),
        (L.h3_vsa_gated_scatter, [t * 4, n * w * 2, t * w * 2, b * w * 4, t * w * 2]),
    ]
    for fn, need in cases:
        for i in range(len(need)):
            views = [fake(x) for x in need]
            views[i] = fake(need[i] - 1)
            st = fn(ctypes.byref(c), *views, None)
            assert st == H.H3_ERR_BINDING, (fn.__name__, i, H.last_error())
            assert f"binding {i} is {need[i] - 1} bytes, the kernel addresses {need[i]}" in H.last_error()
    st = L.h3_vsa_kmean(w, b, fake(b * w * 4 - 4), fake(w * 4), None)
    assert st == H.H3_ERR_BINDING


@pytest.mark.parametrize("field,value", [("padded", 320), ("padded", 100), ("width", 200),
                                         ("heads", 3), ("blocks", 0), ("prefix", 7),
                                         ("topk", 20000), ("tokens", 0)])
def test_vsa_config_outside_declared_ranges_is_refused(field, value):
    c = cfg()
    setattr(c, field, value)
    big = fake(1 << 30)
    st = H.lib().h3_vsa_gather(ctypes.byref(c), big, big, big, None)
    assert st == H.H3_ERR_CONFIG, H.last_error()


def test_vsa_attention_checks_routes_and_lengths():
    heads, blocks = 2, 5
    n, w = 64 * blocks, 256
    a = H.AttentionCfg(w, w, w, n, n, 0.088)
    big = fake(1 << 28)
    L = H.lib()
    st = L.h3_vsa_attention_i8(ctypes.byref(a), n, heads, big, big, big, big, big, big,
                               fake(heads * blocks * blocks * 4 - 1), fake(blocks * 4), None)
    assert st == H.H3_ERR_BINDING and "binding 0" in H.last_error()
    st = L.h3_vsa_attention_i8(ctypes.byref(a), n, heads, big, big, big, big, big, big,
                               fake(heads * blocks * blocks * 4), fake(blocks * 4 - 4), None)
    assert st == H.H3_ERR_BINDING and "binding 1" in H.last_error()
    a.tokens = n - 1  # not whole cubes
    st = L.h3_vsa_attention_i8(ctypes.byref(a), n - 1, heads, big, big, big, big, big, big, big,
                               big, None)
    assert st == H.H3_ERR_CONFIG, H.last_error()


def test_workspace_forms_check_their_workspace():
    """The dense _ws forms: a head-major scale copy of (kv_stride/128) x tokens f32."""
    heads, tokens = 3, 500
    cap = H.capacity(tokens)
    w = heads * 128
    a = H.AttentionCfg(w, w, w, tokens, cap, 1.0)
    s = H.AttentionSkipCfg(w, w, w, tokens, cap, 1.0, 1.0)
    big = fake(1 << 28)
    need = heads * tokens * 4
    assert H.scales_workspace_bytes(a) == need
    L = H.lib()
    for fn, c, stage in [(L.h3_attention_i8qk_ws, a, "attention_i8qk"),
                         (L.h3_attention_i4qk_ws, a, "attention_i4qk"),
                         (L.h3_attention_i4qks_ws, s, "attention_i4qks")]:
        st = fn(ctypes.byref(c), tokens, heads, big, big, big, big, big, big, fake(need - 4), None)
        assert st == H.H3_ERR_BINDING
        assert H.last_error() == f"{stage}: workspace is {need - 4} bytes, the kernel addresses {need}"
        st = fn(ctypes.byref(c), tokens, heads, big, big, big, big, big, big, H.raw_view(0, need),
                None)
        assert st == H.H3_ERR_ARGUMENT and "null workspace" in H.last_error()


def test_vsa_attention_workspace_is_checked():
    """h3_vsa_attention_i8_ws: a head-major copy of the key scales, (kv_stride/128) x tokens
    f32; a short or null workspace refused."""
    heads, blocks = 2, 5
    n, w = 64 * blocks, 256
    a = H.AttentionCfg(w, w, w, n, n, 0.088)
    big = fake(1 << 28)
    L = H.lib()
    need = (w // 128) * n * 4
    assert H.scales_workspace_bytes(a) == need
    st = L.h3_vsa_attention_i8_ws(ctypes.byref(a), n, heads, big, big, big, big, big, big, big,
                                  big, fake(need - 1), None)
    assert st == H.H3_ERR_BINDING
    assert H.last_error() == f"VSA attention: workspace is {need - 1} bytes, the kernel addresses {need}"
    st = L.h3_vsa_attention_i8_ws(ctypes.byref(a), n, heads, big, big, big, big, big, big, big,
                                  big, H.raw_view(0, need), None)
    assert st == H.H3_ERR_ARGUMENT and "null workspace" in H.last_error()


def test_runtime_build_refuses_bad_options_without_allocating():
    src, inverse, lengths, prefix = H.vsa_plan([(0, 65), (65, 6)], 246, 5, 5, 7)
    with pytest.raises(H.H3Error, match="keep_percent"):
        H.Vsa(src, inverse, lengths, prefix, 2, H.VsaOptions(keep_percent=0.0))


def test_f16_vsa_attention_checks_its_bindings():
    """h3_vsa_attention_f16 (vsa_attention_16.loom): q [cap][q_stride], k and v
    [cap][kv_stride] f16, out [token_count][out_stride], routes [heads][blocks][blocks],
    lengths [blocks]; whole cubes only."""
    heads, blocks = 2, 5
    n, w = 64 * blocks, 256
    a = H.AttentionCfg(w, w, w, n, n, 0.088)
    L = H.lib()
    need = [n * w * 2, n * w * 2, n * w * 2, n * w * 2, heads * blocks * blocks * 4, blocks * 4]
    for i in range(6):
        views = [fake(x - (4 if j == i else 0)) for j, x in enumerate(need)]
        st = L.h3_vsa_attention_f16(ctypes.byref(a), n, heads, *views, None)
        assert st == H.H3_ERR_BINDING and f"binding {i} " in H.last_error(), H.last_error()
    a.tokens = n - 1
    st = L.h3_vsa_attention_f16(ctypes.byref(a), n - 1, heads, *[fake(x) for x in need], None)
    assert st == H.H3_ERR_CONFIG, H.last_error()
