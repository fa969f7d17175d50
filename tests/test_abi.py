"""The C ABI on a CPU host: libh3attn.so loads, exports every symbol include/h3attn.h declares,
and refuses bad configs and short bindings before touching a device (src/dispatch.rs:264-276).
No kernel is launched here."""
import ctypes
import pathlib
import re
import subprocess

import pytest

import h3attn as H

ROOT = pathlib.Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "h3attn.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(h3_\w+)\s*\(", text)))


def test_library_exports_every_declared_function():
    names = declared_functions()
    assert len(names) >= 19
    out = subprocess.run(["nm", "-D", "--defined-only", str(H.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (h3_\w+)", out))
    missing = [n for n in names if n not in exported]
    assert not missing, f"declared but not exported: {missing}"
    lib = H.lib()
    for n in names:
        assert getattr(lib, n) is not None
    assert set(H.SIGNATURES) <= set(names)


def test_capacity_matches_the_reference_formula():
    import oracle as O

    for t in [1, 23, 63, 64, 65, 129, 1024, 4095, 4096, 4097, 31104, 129024, 130272, 1048544]:
        assert H.capacity(t) == O.capacity(t), t


def fake(nbytes):
    """A binding that is never dereferenced: the checks reject the call before any launch."""
    return H.raw_view(0x1000, nbytes)


def prep_cfg(heads=4, cap=64):
    return H.PrepareCfg(heads * 128, 0, heads, 1.0, cap, 1e-5, H.H3_ELEM_F16)


def call_prepare(cfg, tokens, x, mean, codes, scales):
    return H.lib().h3_prepare_qk_i8hm(ctypes.byref(cfg), tokens, x, mean, codes, scales, None)


def test_short_binding_is_refused_with_the_reference_message():
    cfg = prep_cfg()
    tokens = 37
    need_x = tokens * 512 * 2
    st = call_prepare(cfg, tokens, fake(need_x - 2), fake(2048), fake(4 * 64 * 128),
                      fake(4 * 64 * 4))
    assert st == H.H3_ERR_BINDING
    assert H.last_error() == (
        f"prepare_qk_i8hm: binding 0 is {need_x - 2} bytes, the kernel addresses {need_x}")
    st = call_prepare(cfg, tokens, fake(need_x), fake(2048), fake(4 * 64 * 128 - 1),
                      fake(4 * 64 * 4))
    assert st == H.H3_ERR_BINDING and "binding 2" in H.last_error()


@pytest.mark.parametrize("field,value", [("row_stride", 100), ("row_stride", 0),
                                         ("heads", 0), ("heads", 300), ("head_offset", 64),
                                         ("token_capacity", 48), ("elem", 7)])
def test_prepare_config_outside_declared_ranges_is_refused(field, value):
    cfg = prep_cfg()
    setattr(cfg, field, value)
    st = call_prepare(cfg, 37, fake(1 << 30), fake(1 << 20), fake(1 << 30), fake(1 << 30))
    assert st == H.H3_ERR_CONFIG, H.last_error()


def test_tokens_beyond_capacity_are_refused():
    st = call_prepare(prep_cfg(cap=32), 37, fake(1 << 30), fake(1 << 20), fake(1 << 30),
                      fake(1 << 30))
    assert st == H.H3_ERR_ARGUMENT and "exceed token_capacity" in H.last_error()


def att_cfg(tokens=97, cap=128, heads=4):
    w = heads * 128
    return H.AttentionCfg(w, w, w, tokens, cap, 1.0)


def call_attention(cfg, token_count, heads, sizes):
    views = [fake(n) for n in sizes]
    return H.lib().h3_attention_i8qkhm(ctypes.byref(cfg), token_count, heads, *views, None)


def test_attention_checks_every_binding():
    heads, tokens, cap = 4, 97, 128
    need = [heads * cap * 128, heads * cap * 4, heads * cap * 128, heads * cap * 4,
            heads * 128 * cap * 2, tokens * heads * 128 * 2]
    for i in range(6):
        sizes = list(need)
        sizes[i] -= 1
        st = call_attention(att_cfg(tokens, cap, heads), tokens, heads, sizes)
        assert st == H.H3_ERR_BINDING and f"binding {i} " in H.last_error()


@pytest.mark.parametrize("field,value", [("q_stride", 100), ("kv_stride", 0),
                                         ("out_stride", 40000), ("tokens", 0),
                                         ("token_capacity", 24), ("tokens", 200)])
def test_attention_config_outside_declared_ranges_is_refused(field, value):
    cfg = att_cfg()
    setattr(cfg, field, value)
    st = call_attention(cfg, 1, 4, [1 << 40] * 6)
    assert st == H.H3_ERR_CONFIG, H.last_error()


def test_attention_token_count_must_lie_in_the_sequence():
    st = call_attention(att_cfg(), 98, 4, [1 << 40] * 6)
    assert st == H.H3_ERR_ARGUMENT and "token_count" in H.last_error()


def test_transpose_checks_rows_and_bindings():
    cfg = H.TransposeCfg(256, 128, H.H3_ELEM_F16)
    lib = H.lib()
    assert lib.h3_transpose_f16(ctypes.byref(cfg), 200, 100, fake(1 << 30), fake(1 << 30),
                                None) == H.H3_ERR_ARGUMENT
    st = lib.h3_transpose_qkv_v_f16(ctypes.byref(cfg), 100, 100, fake(100 * 768 * 2 - 1),
                                    fake(1 << 30), None)
    assert st == H.H3_ERR_BINDING and "binding 0" in H.last_error()
    cfg.width = 48
    assert lib.h3_transpose_f16(ctypes.byref(cfg), 10, 10, fake(1 << 30), fake(1 << 30),
                                None) == H.H3_ERR_CONFIG


def test_colmean_width_range():
    lib = H.lib()
    assert lib.h3_colmean_f32(128, 0, 10, fake(1 << 20), fake(1 << 20), None) == H.H3_ERR_CONFIG
    assert lib.h3_colmean_f32(512, 0, 10, fake(10 * 512 * 2 - 2), fake(2048),
                              None) == H.H3_ERR_BINDING


def test_rope_config_checks():
    lib = H.lib()
    cfg = H.RopeCfg(128 * 12, 4, 4, 512, 1e-5, 1, H.H3_ELEM_F16)
    ok_sizes = [3 * 1536 * 2, 512, 512, 3 * 48 * 4, 3 * 48 * 4, 3 * 512 * 2, 3 * 512 * 2,
                3 * 512 * 2]
    sizes = list(ok_sizes)
    sizes[3] -= 4
    st = lib.h3_rope_qknorm_f16(ctypes.byref(cfg), 3, *[fake(n) for n in sizes], None)
    assert st == H.H3_ERR_BINDING and "binding 3" in H.last_error()
    cfg.k_offset = 256  # K would overlap Q
    st = lib.h3_rope_qknorm_f16(ctypes.byref(cfg), 3, *[fake(n) for n in ok_sizes], None)
    assert st == H.H3_ERR_CONFIG


def test_python_layer_raises_with_status():
    with pytest.raises(H.H3Error) as e:
        H.check(H.lib().h3_colmean_f32(128, 0, 10, fake(1), fake(1), None))
    assert e.value.status == H.H3_ERR_CONFIG


def call_gemm(cfg, tokens, sizes):
    return H.lib().h3_gemm_i8_qkv_256(ctypes.byref(cfg), tokens, *[fake(n) for n in sizes], None)


def test_gemm_bindings_follow_the_reference_extents():
    """src/dispatch.rs:1025-1045: a t*k_stride, w n*k_stride, scales, and the compact output
    t*n + (ceil(t/256)*256 - t)*n/3 f16 elements."""
    t, k, n = 300, 128, 768
    cfg = H.GemmCfg(k, n, k, 2)
    need = [t * k, n * k, n * 4, t * 4, (t * n + (512 - t) * (n // 3)) * 2]
    for i in range(5):
        sizes = list(need)
        sizes[i] -= 1
        st = call_gemm(cfg, t, sizes)
        assert st == H.H3_ERR_BINDING and H.last_error() == (
            f"gemm_i8_qkv_256: binding {i} is {sizes[i]} bytes, the kernel addresses {need[i]}")


@pytest.mark.parametrize("field,value", [("k_size", 96), ("k_size", 0), ("n_size", 512),
                                         ("n_size", 65664), ("k_stride", 64), ("m_group", 0),
                                         ("m_group", 5)])
def test_gemm_config_outside_declared_ranges_is_refused(field, value):
    cfg = H.GemmCfg(128, 768, 128, 1)
    setattr(cfg, field, value)
    assert call_gemm(cfg, 16, [1 << 40] * 5) == H.H3_ERR_CONFIG, H.last_error()


def test_gemm_rejects_misaligned_output_and_bad_token_counts():
    cfg = H.GemmCfg(128, 768, 128, 1)
    lib = H.lib()
    views = [fake(1 << 40)] * 4 + [H.raw_view(0x1004, 1 << 40)]
    assert lib.h3_gemm_i8_qkv_256(ctypes.byref(cfg), 16, *views, None) == H.H3_ERR_ARGUMENT
    assert call_gemm(cfg, 0, [1 << 40] * 5) == H.H3_ERR_ARGUMENT


def call_plain(cfg, tokens, sizes, x_ptr=0x1000):
    views = [H.raw_view(x_ptr, sizes[0])] + [fake(n) for n in sizes[1:]]
    return H.lib().h3_prepare_plain_i8(ctypes.byref(cfg), tokens, *views, None)


def test_prepare_plain_bindings_and_configs():
    t = 7
    cfg = H.PreparePlainCfg(4096, 448, 4160, H.H3_ELEM_F16)
    need = [t * 4096 * 2, t * 4160, t * 4]
    for i in range(3):
        sizes = list(need)
        sizes[i] -= 1
        assert call_plain(cfg, t, sizes) == H.H3_ERR_BINDING and f"binding {i}" in H.last_error()
    f32 = H.PreparePlainCfg(4096, 448, 4160, H.H3_ELEM_F32)
    sizes = [t * 4096 * 4 - 1, t * 4160, t * 4]
    assert call_plain(f32, t, sizes) == H.H3_ERR_BINDING
    for field, value in [("width", 100), ("width", 33024), ("lanes", 16), ("lanes", 48),
                         ("out_stride", 4032), ("out_stride", 4100), ("elem", 3)]:
        bad = H.PreparePlainCfg(4096, 448, 4160, H.H3_ELEM_F16)
        setattr(bad, field, value)
        assert call_plain(bad, t, [1 << 40] * 3) == H.H3_ERR_CONFIG, (field, value)
    assert call_plain(cfg, t, [1 << 40] * 3, x_ptr=0x1008) == H.H3_ERR_ARGUMENT
    assert call_plain(cfg, 0, [1 << 40] * 3) == H.H3_ERR_ARGUMENT


def test_int4_bindings_are_half_the_int8_extents():
    """prepare_qk_i4 writes 64 code bytes per (token, head); attention_i4qk reads capacity rows
    of q_stride/2 and kv_stride/2 code bytes (src/stack.rs:846, 1725-1750)."""
    lib = H.lib()
    cfg = H.PrepareCfg(512, 0, 4, 1.0, 64, 1e-5, H.H3_ELEM_F16)
    t = 37
    need = [t * 512 * 2, 2048, t * 4 * 64, t * 4 * 4]
    sizes = list(need)
    sizes[2] -= 1
    st = lib.h3_prepare_qk_i4(ctypes.byref(cfg), t, *[fake(n) for n in sizes], None)
    assert st == H.H3_ERR_BINDING and H.last_error() == (
        f"prepare_qk_i4: binding 2 is {need[2] - 1} bytes, the kernel addresses {need[2]}")
    acfg = att_cfg(97, 128, 4)
    stride = 4 * 128
    need = [128 * stride // 2, 128 * 4 * 4, 128 * stride // 2, 128 * 4 * 4, stride * 128 * 2,
            97 * stride * 2]
    for i in (0, 2):
        sizes = list(need)
        sizes[i] -= 1
        st = lib.h3_attention_i4qk(ctypes.byref(acfg), 97, 4, *[fake(n) for n in sizes], None)
        assert st == H.H3_ERR_BINDING and f"binding {i} " in H.last_error()


def test_skip_twin_checks_tau_and_bindings():
    lib = H.lib()
    stride = 4 * 128
    cfg = H.AttentionSkipCfg(stride, stride, stride, 97, 128, 1.0, float("nan"))
    sizes = [1 << 30] * 6
    assert lib.h3_attention_i4qks(ctypes.byref(cfg), 97, 4, *[fake(n) for n in sizes],
                                  None) == H.H3_ERR_CONFIG
    cfg.skip_tau = 2.0
    need = [128 * stride // 2, 128 * 4 * 4, 128 * stride // 2, 128 * 4 * 4, stride * 128 * 2,
            97 * stride * 2]
    sizes = list(need)
    sizes[5] -= 2
    st = lib.h3_attention_i4qks(ctypes.byref(cfg), 97, 4, *[fake(n) for n in sizes], None)
    assert st == H.H3_ERR_BINDING and H.last_error().startswith("attention_i4qks: binding 5")


def test_cross_attention_checks_groups_capacities_and_bindings():
    L = H.lib()
    qh, kh, qt, kt, qc, kc = 8, 2, 300, 77, 320, 96
    need = [qh * qc * 128, qh * qc * 4, kh * kc * 128, kh * kc * 4, kh * 128 * kc * 2, kt,
            qt * qh * 128 * 2]
    cfg = H.CrossCfg(qh, kh, qt, qc, kt, kc, qh * 128)
    for i in range(len(need)):
        views = [fake(x) for x in need]
        views[i] = fake(need[i] - 1)
        st = L.h3_attention_i8qkhm_cross(ctypes.byref(cfg), *views, None)
        assert st == H.H3_ERR_BINDING and f"binding {i} is" in H.last_error(), H.last_error()
    for field, value in [("kv_heads", 3), ("q_capacity", 310), ("kv_capacity", 64),
                         ("out_stride", 512), ("kv_tokens", 0)]:
        bad = H.CrossCfg(qh, kh, qt, qc, kt, kc, qh * 128)
        setattr(bad, field, value)
        st = L.h3_attention_i8qkhm_cross(ctypes.byref(bad), *[fake(1 << 30)] * 7, None)
        assert st == H.H3_ERR_CONFIG, (field, H.last_error())


def gemm_pitch16(k):
    """gemm_pitch(k, 16) (src/model.rs:74-85)."""
    return k + 128 if (2 * k) % 1024 == 0 else k


def direct_pitch_bindings(heads, tokens, cap):
    """The byte lengths the reference's Stack::attend passes as `required` for its attention
    (src/stack.rs:1815-1838): operands sized by the workload's heads, the output at the
    direct-attention pitch (src/stack.rs:1683, 817-822)."""
    inner = heads * 128
    return [cap * heads * 128, cap * heads * 4, cap * heads * 128, cap * heads * 4,
            inner * cap * 2, tokens * gemm_pitch16(inner) * 2]


def no_device_reached():
    """Fake bindings pass every host check and stop at the device query on a CPU host."""
    return H.H3_ERR_NO_DEVICE


@pytest.mark.parametrize("entry", ["h3_attention_i8qkhm", "h3_attention_i8qk"])
def test_attention_accepts_the_reference_direct_attention_pitch(entry):
    """tests/compiler.rs:43-45 qualifies q/kv 7168, out 7296 (56 heads, gemm_pitch(7168, 16));
    the reference's caller binds operands of cap*56*... bytes and an output of t*7296*2
    (src/stack.rs:1683, 1830-1837). Every binding one byte short is refused with the reference's
    message; the exact sizes pass every check."""
    heads, tokens = 56, 37977
    inner = heads * 128
    cap = H.capacity(tokens)
    assert gemm_pitch16(inner) == 7296
    cfg = H.AttentionCfg(inner, inner, 7296, tokens, cap, 1.0)
    need = direct_pitch_bindings(heads, tokens, cap)
    fn = getattr(H.lib(), entry)
    st = fn(ctypes.byref(cfg), tokens, heads, *[fake(n) for n in need], None)
    assert st == no_device_reached(), H.last_error()
    # the output extent the kernel addresses ends at the last touched head's columns
    need[5] = ((tokens - 1) * 7296 + inner) * 2
    st = fn(ctypes.byref(cfg), tokens, heads, *[fake(n) for n in need], None)
    assert st == no_device_reached(), H.last_error()
    for i in range(6):
        sizes = list(need)
        sizes[i] -= 1
        st = fn(ctypes.byref(cfg), tokens, heads, *[fake(n) for n in sizes], None)
        assert st == H.H3_ERR_BINDING, (i, H.last_error())
        assert H.last_error().endswith(f"binding {i} is {sizes[i]} bytes, the kernel addresses "
                                       f"{need[i]}")


def test_attention_extents_follow_the_touched_heads():
    """A launch of `heads` rows reads key/value heads < min(heads, kv_stride/128) and query
    heads < min(that, out_stride/128) (attention_i8qkhm_mha8_k64_lds_f16_wmma.loom:300-340):
    fewer heads than the strides hold need smaller bindings; a token-major launch whose query
    heads lie past a q_stride row is refused."""
    lib = H.lib()
    tokens, cap = 97, 128
    cfg = H.AttentionCfg(8 * 128, 8 * 128, 8 * 128, tokens, cap, 1.0)
    heads = 3
    need = [heads * cap * 128, heads * cap * 4, heads * cap * 128, heads * cap * 4,
            heads * 128 * cap * 2, ((tokens - 1) * 1024 + heads * 128) * 2]
    assert lib.h3_attention_i8qkhm(ctypes.byref(cfg), tokens, heads, *[fake(n) for n in need],
                                   None) == no_device_reached(), H.last_error()
    for i in range(6):
        sizes = list(need)
        sizes[i] -= 1
        st = lib.h3_attention_i8qkhm(ctypes.byref(cfg), tokens, heads,
                                     *[fake(n) for n in sizes], None)
        assert st == H.H3_ERR_BINDING and f"binding {i} " in H.last_error()
    # GQA-style wrap: 8 workload rows over 2 key/value heads read 2 query heads
    gqa = H.AttentionCfg(8 * 128, 2 * 128, 8 * 128, tokens, cap, 1.0)
    need = [2 * cap * 128, 2 * cap * 4, 2 * cap * 128, 2 * cap * 4, 2 * 128 * cap * 2,
            ((tokens - 1) * 1024 + 2 * 128) * 2]
    assert lib.h3_attention_i8qkhm(ctypes.byref(gqa), tokens, 8, *[fake(n) for n in need],
                                   None) == no_device_reached(), H.last_error()
    # head-major does not address Q through q_stride; token-major rows must hold the heads
    narrow = H.AttentionCfg(128, 4 * 128, 4 * 128, tokens, cap, 1.0)
    assert lib.h3_attention_i8qkhm(ctypes.byref(narrow), tokens, 4, *[fake(1 << 40)] * 6,
                                   None) == no_device_reached(), H.last_error()
    st = lib.h3_attention_i8qk(ctypes.byref(narrow), tokens, 4, *[fake(1 << 40)] * 6, None)
    assert st == H.H3_ERR_CONFIG and "holds 1 query heads, the launch reads 4" in H.last_error()


def test_lent_workspace_is_checked_like_a_binding():
    """The _ws forms check the workspace's size before any launch."""
    lib = H.lib()
    stride = 4 * 128
    cfg = H.AttentionCfg(stride, stride, stride, 97, 128, 1.0)
    ws = lib.h3_scales_workspace_bytes(ctypes.byref(cfg))
    assert ws == 4 * 97 * 4
    need = [128 * stride, 128 * 4 * 4, 128 * stride, 128 * 4 * 4, stride * 128 * 2,
            97 * stride * 2]
    st = lib.h3_attention_i8qk_ws(ctypes.byref(cfg), 97, 4, *[fake(n) for n in need],
                                  fake(ws - 1), None)
    assert st == H.H3_ERR_BINDING and H.last_error() == (
        f"attention_i8qk: workspace is {ws - 1} bytes, the kernel addresses {ws}")
    st = lib.h3_attention_i8qk_ws(ctypes.byref(cfg), 97, 4, *[fake(n) for n in need], fake(ws),
                                  None)
    assert st == no_device_reached(), H.last_error()
