"""Python binding of libh3attn (the C ABI in include/h3attn.h) over torch device tensors.

This is the host-side mirror used by the tests and the benchmark: each function takes torch
tensors already resident on the GPU, passes their device pointers and byte lengths to the C ABI,
and enqueues on torch's current stream. The library is required: importing works without a
GPU, but every call needs the built libh3attn.so and fails loudly without it; there is no CPU
fallback anywhere in this package.

Function names and arguments follow the reference's kernels (kernels/*.loom in h3-hrx) and
their host call sites (src/stack.rs), e.g. prepare_qk_i8hm(cfg, tokens, x, mean, codes, scales).
"""
from __future__ import annotations

import ctypes
import math
import pathlib
from typing import Optional

_HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = _HERE.parent / "libh3attn.so"

H3_OK, H3_ERR_BINDING, H3_ERR_CONFIG, H3_ERR_ARGUMENT, H3_ERR_LAUNCH, H3_ERR_NO_DEVICE = range(6)
H3_ELEM_F16, H3_ELEM_BF16, H3_ELEM_F32 = 0, 1, 2
STATUS_NAMES = {0: "ok", 1: "binding", 2: "config", 3: "argument", 4: "launch", 5: "no device"}


class H3Error(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"[{STATUS_NAMES.get(status, status)}] {message}")
        self.status = status
        self.message = message


class View(ctypes.Structure):
    _fields_ = [("ptr", ctypes.c_void_p), ("bytes", ctypes.c_size_t)]


class PrepareCfg(ctypes.Structure):
    _fields_ = [
        ("row_stride", ctypes.c_uint32),
        ("head_offset", ctypes.c_uint32),
        ("heads", ctypes.c_uint32),
        ("extra_scale", ctypes.c_float),
        ("token_capacity", ctypes.c_uint32),
        ("eps", ctypes.c_float),
        ("elem", ctypes.c_uint32),
    ]


class RopeCfg(ctypes.Structure):
    _fields_ = [
        ("row_stride", ctypes.c_uint32),
        ("heads", ctypes.c_uint32),
        ("kv_heads", ctypes.c_uint32),
        ("k_offset", ctypes.c_uint32),
        ("eps", ctypes.c_float),
        ("copy_v", ctypes.c_uint32),
        ("elem", ctypes.c_uint32),
    ]


class TransposeCfg(ctypes.Structure):
    _fields_ = [
        ("width", ctypes.c_uint32),
        ("row_capacity", ctypes.c_uint32),
        ("elem", ctypes.c_uint32),
    ]


class AttentionCfg(ctypes.Structure):
    _fields_ = [
        ("q_stride", ctypes.c_uint32),
        ("kv_stride", ctypes.c_uint32),
        ("out_stride", ctypes.c_uint32),
        ("tokens", ctypes.c_uint32),
        ("token_capacity", ctypes.c_uint32),
        ("scale", ctypes.c_float),
    ]


class GemmCfg(ctypes.Structure):
    _fields_ = [
        ("k_size", ctypes.c_uint32),
        ("n_size", ctypes.c_uint32),
        ("k_stride", ctypes.c_uint32),
        ("m_group", ctypes.c_uint32),
    ]


class PreparePlainCfg(ctypes.Structure):
    _fields_ = [
        ("width", ctypes.c_uint32),
        ("lanes", ctypes.c_uint32),
        ("out_stride", ctypes.c_uint32),
        ("elem", ctypes.c_uint32),
    ]


class AttentionSkipCfg(ctypes.Structure):
    _fields_ = [
        ("q_stride", ctypes.c_uint32),
        ("kv_stride", ctypes.c_uint32),
        ("out_stride", ctypes.c_uint32),
        ("tokens", ctypes.c_uint32),
        ("token_capacity", ctypes.c_uint32),
        ("scale", ctypes.c_float),
        ("skip_tau", ctypes.c_float),
    ]


class StackDims(ctypes.Structure):
    _fields_ = [
        ("heads", ctypes.c_uint32),
        ("tokens", ctypes.c_uint32),
        ("eps", ctypes.c_float),
        ("elem", ctypes.c_uint32),
        ("ksmooth", ctypes.c_int),
        ("fused", ctypes.c_int),
        ("direct_attn", ctypes.c_int),
    ]


class IntQk(ctypes.Structure):
    _fields_ = [
        ("qi", View), ("ki", View), ("qs", View), ("ks", View),
        ("kmean", View), ("zmean", View), ("vt", View), ("head_major", ctypes.c_int),
    ]


class CrossCfg(ctypes.Structure):
    _fields_ = [(name, ctypes.c_uint32) for name in (
        "q_heads", "kv_heads", "q_tokens", "q_capacity", "kv_tokens", "kv_capacity",
        "out_stride")]


class VsaCfg(ctypes.Structure):
    """h3.vsa.* (kernels/vsa_ops.loom:3-9)."""
    _fields_ = [
        ("tokens", ctypes.c_uint32),
        ("padded", ctypes.c_uint32),
        ("width", ctypes.c_uint32),
        ("blocks", ctypes.c_uint32),
        ("heads", ctypes.c_uint32),
        ("prefix", ctypes.c_uint32),
        ("topk", ctypes.c_uint32),
    ]


class VsaSegment(ctypes.Structure):
    _fields_ = [("row0", ctypes.c_uint32), ("rows", ctypes.c_uint32)]


class VsaOptionsC(ctypes.Structure):
    _fields_ = [
        ("keep_percent", ctypes.c_double),
        ("start", ctypes.c_double),
        ("end", ctypes.c_double),
        ("min_tokens", ctypes.c_uint32),
        ("dense_blocks", ctypes.POINTER(ctypes.c_uint32)),
        ("n_dense_blocks", ctypes.c_uint32),
    ]


class VsaBuffers(ctypes.Structure):
    _fields_ = [(name, View) for name in (
        "src", "inverse", "lengths", "q", "k", "v", "qm", "km", "scores", "routes", "qi", "ki",
        "qs", "ks", "vt", "out", "kmean")] + [("cfg", VsaCfg), ("attention", AttentionCfg)]


# (name, argtypes) of every exported entry point; restype is int unless noted.
_P = ctypes.POINTER
_S = ctypes.c_void_p
SIGNATURES = {
    "h3_last_error": ([], ctypes.c_char_p),
    "h3_version": ([], ctypes.c_char_p),
    "h3_prepare_qk_i8": ([_P(PrepareCfg), ctypes.c_uint32, View, View, View, View, _S], ctypes.c_int),
    "h3_prepare_qk_i8hm": ([_P(PrepareCfg), ctypes.c_uint32, View, View, View, View, _S], ctypes.c_int),
    "h3_prepare_qk_i4": ([_P(PrepareCfg), ctypes.c_uint32, View, View, View, View, _S], ctypes.c_int),
    "h3_prepare_qk_rope_i8hm": (
        [_P(PrepareCfg), ctypes.c_uint32, View, View, View, View, View, View, _S], ctypes.c_int),
    "h3_prepare_k_rope_smooth_i8hm": (
        [_P(PrepareCfg), ctypes.c_uint32, View, View, View, View, View, View, View, _S], ctypes.c_int),
    "h3_rope_qknorm_f16": (
        [_P(RopeCfg), ctypes.c_uint32, View, View, View, View, View, View, View, View, _S], ctypes.c_int),
    "h3_colmean_f32": ([ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, View, View, _S], ctypes.c_int),
    "h3_transpose_f16": ([_P(TransposeCfg), ctypes.c_uint32, ctypes.c_uint32, View, View, _S], ctypes.c_int),
    "h3_transpose_qkv_v_f16": (
        [_P(TransposeCfg), ctypes.c_uint32, ctypes.c_uint32, View, View, _S], ctypes.c_int),
    "h3_attention_i8qkhm": (
        [_P(AttentionCfg), ctypes.c_uint32, ctypes.c_uint32, View, View, View, View, View, View, _S],
        ctypes.c_int),
    "h3_attention_i8qk": (
        [_P(AttentionCfg), ctypes.c_uint32, ctypes.c_uint32, View, View, View, View, View, View, _S],
        ctypes.c_int),
    "h3_prepare_plain_i8": (
        [_P(PreparePlainCfg), ctypes.c_uint32, View, View, View, _S], ctypes.c_int),
    "h3_gemm_i8_qkv_256": (
        [_P(GemmCfg), ctypes.c_uint32, View, View, View, View, View, _S], ctypes.c_int),
    "h3_rope_dit_tables": (
        [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p],
        ctypes.c_int),
    "h3_attention_i4qk": (
        [_P(AttentionCfg), ctypes.c_uint32, ctypes.c_uint32, View, View, View, View, View, View, _S],
        ctypes.c_int),
    "h3_attention_i4qks": (
        [_P(AttentionSkipCfg), ctypes.c_uint32, ctypes.c_uint32, View, View, View, View, View, View,
         _S], ctypes.c_int),
    "h3_attention_i8qkhm_cross": (
        [_P(CrossCfg), View, View, View, View, View, View, View, _S], ctypes.c_int),
    "h3_vsa_gather": ([_P(VsaCfg), View, View, View, _S], ctypes.c_int),
    "h3_vsa_scatter": ([_P(VsaCfg), View, View, View, _S], ctypes.c_int),
    "h3_vsa_pool": ([_P(VsaCfg), View, View, View, _S], ctypes.c_int),
    "h3_vsa_scores": ([_P(VsaCfg), View, View, View, _S], ctypes.c_int),
    "h3_vsa_route": ([_P(VsaCfg), View, View, _S], ctypes.c_int),
    "h3_vsa_coarse": ([_P(VsaCfg), View, View, View, _S], ctypes.c_int),
    "h3_vsa_gated_scatter": ([_P(VsaCfg), View, View, View, View, View, _S], ctypes.c_int),
    "h3_vsa_kmean": ([ctypes.c_uint32, ctypes.c_uint32, View, View, _S], ctypes.c_int),
    "h3_vsa_attention_i8": (
        [_P(AttentionCfg), ctypes.c_uint32, ctypes.c_uint32, View, View, View, View, View, View,
         View, View, _S], ctypes.c_int),
    "h3_vsa_attention_f16": (
        [_P(AttentionCfg), ctypes.c_uint32, ctypes.c_uint32, View, View, View, View, View, View,
         _S], ctypes.c_int),
    "h3_vsa_attention_i8_ws": (
        [_P(AttentionCfg), ctypes.c_uint32, ctypes.c_uint32, View, View, View, View, View, View,
         View, View, View, _S], ctypes.c_int),
    "h3_scales_workspace_bytes": ([_P(AttentionCfg)], ctypes.c_size_t),
    "h3_fp6_workspace_bytes": ([_P(AttentionCfg)], ctypes.c_size_t),
    "h3_attention_i4qk_fp6": (
        [_P(AttentionCfg), ctypes.c_uint32, ctypes.c_uint32, View, View, View, View, View, View,
         View, _S], ctypes.c_int),
    "h3_attention_i8qk_ws": (
        [_P(AttentionCfg), ctypes.c_uint32, ctypes.c_uint32, View, View, View, View, View, View,
         View, _S], ctypes.c_int),
    "h3_attention_i4qk_ws": (
        [_P(AttentionCfg), ctypes.c_uint32, ctypes.c_uint32, View, View, View, View, View, View,
         View, _S], ctypes.c_int),
    "h3_attention_i8qk_static": (
        [_P(AttentionCfg), ctypes.c_uint32, ctypes.c_uint32, View, View, View, View, View, View,
         _S], ctypes.c_int),
    "h3_attention_i4qks_ws": (
        [_P(AttentionSkipCfg), ctypes.c_uint32, ctypes.c_uint32, View, View, View, View, View,
         View, View, _S], ctypes.c_int),
    "h3_vsa_plan_blocks": (
        [_P(VsaSegment), ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
         _P(ctypes.c_uint32)], ctypes.c_int),
    "h3_vsa_plan": (
        [_P(VsaSegment), ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
         ctypes.c_uint32, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, _P(ctypes.c_uint32)],
        ctypes.c_int),
    "h3_vsa_validate": ([_P(VsaOptionsC), ctypes.c_uint32], ctypes.c_int),
    "h3_vsa_topk": ([ctypes.c_double, ctypes.c_uint32], ctypes.c_uint32),
    "h3_vsa_dense_reason": (
        [_P(VsaOptionsC), ctypes.c_uint32, ctypes.c_float, ctypes.c_double], ctypes.c_char_p),
    "h3_vsa_build": (
        [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32,
         ctypes.c_uint32, _P(VsaOptionsC), ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p],
        ctypes.c_int),
    "h3_vsa_build_bits": (
        [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32,
         ctypes.c_uint32, _P(VsaOptionsC), ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
         ctypes.c_void_p], ctypes.c_int),
    "h3_vsa_destroy": ([ctypes.c_void_p], None),
    "h3_vsa_reset": ([ctypes.c_void_p, _S], ctypes.c_int),
    "h3_vsa_attend": (
        [ctypes.c_void_p, ctypes.c_uint32, View, View, View, View, View, _S], ctypes.c_int),
    "h3_vsa_inspect": ([ctypes.c_void_p, ctypes.c_uint32, _P(VsaBuffers)], ctypes.c_int),
    "h3_capacity": ([ctypes.c_uint32, ctypes.c_int], ctypes.c_uint32),
    "h3_stack_build": ([_P(StackDims), ctypes.c_void_p], ctypes.c_int),
    "h3_stack_destroy": ([ctypes.c_void_p], None),
    "h3_stack_capacity": ([ctypes.c_void_p], ctypes.c_uint32),
    "h3_stack_attend_fused": (
        [ctypes.c_void_p, ctypes.c_uint32, View, View, View, View, View, View, _S], ctypes.c_int),
    "h3_stack_attend_compact": (
        [ctypes.c_void_p, ctypes.c_uint32, View, View, View, View, View, View, _S], ctypes.c_int),
    "h3_stack_attend": ([ctypes.c_void_p, ctypes.c_uint32, View, View, View, View, _S], ctypes.c_int),
    "h3_stack_operands": ([ctypes.c_void_p, _P(IntQk)], ctypes.c_int),
}

_lib: Optional[ctypes.CDLL] = None


def lib() -> ctypes.CDLL:
    """Load libh3attn.so (built in-tree by h3-hrx_amd/build.py). Raises if it is missing."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: build it with __graft_entry__.build()")
        # torch ships its own libamdhip64 (same soname, but its libraries ask for the unversioned
        # file name), so a process that loaded this library first would end up with two HIP
        # runtimes once torch is imported, and this library's would find no device. Loaded after
        # torch, the library binds to torch's runtime.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = res
        _lib = handle
    return _lib


def last_error() -> str:
    return lib().h3_last_error().decode()


def check(status: int) -> None:
    if status != H3_OK:
        raise H3Error(status, last_error())


def config_f32(v: float) -> float:
    """compile::num's %.17g spelling parsed as f32 (src/compile.rs:38-83)."""
    import numpy as np

    return float(np.float32(float("%.17g" % v)))


EXTRA_Q = config_f32(1.0 / math.sqrt(128.0) / 128.0)  # src/stack.rs:622-625


# ------------------------------------------------------------------------- tensor plumbing

def view(t) -> View:
    """A binding of a torch tensor (any dtype): device pointer and byte length. The tensor must
    live on the current GPU: a host or other-device pointer handed to a kernel faults the GPU."""
    if t is None:
        return View(None, 0)
    if hasattr(t, "data_ptr"):
        if not t.is_contiguous():
            raise ValueError("bindings must be contiguous")
        if not t.is_cuda:
            raise ValueError(f"bindings must be GPU tensors, got one on {t.device}")
        import torch

        if t.device.index != torch.cuda.current_device():
            raise ValueError(f"binding on {t.device}, the current device is "
                             f"cuda:{torch.cuda.current_device()}")
        return View(t.data_ptr(), t.numel() * t.element_size())
    if isinstance(t, View):
        return t
    raise TypeError(f"cannot bind {type(t)}")


def raw_view(ptr: int, nbytes: int) -> View:
    return View(ptr, nbytes)


def stream_ptr(stream=None) -> int:
    import torch

    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def elem_of(t) -> int:
    import torch

    if t.dtype == torch.bfloat16:
        return H3_ELEM_BF16
    if t.dtype in (torch.float16, torch.int16, torch.uint16):
        return H3_ELEM_F16
    raise TypeError(f"activations must be f16 or bf16, not {t.dtype}")


# ------------------------------------------------------------------------- entry points

def prepare_qk_i8(cfg: PrepareCfg, tokens: int, x, mean, codes, scales, stream=None) -> None:
    check(lib().h3_prepare_qk_i8(ctypes.byref(cfg), tokens, view(x), view(mean), view(codes),
                                 view(scales), stream_ptr(stream)))


def prepare_qk_i8hm(cfg: PrepareCfg, tokens: int, x, mean, codes, scales, stream=None) -> None:
    check(lib().h3_prepare_qk_i8hm(ctypes.byref(cfg), tokens, view(x), view(mean), view(codes),
                                   view(scales), stream_ptr(stream)))


def prepare_qk_i4(cfg: PrepareCfg, tokens: int, x, mean, codes, scales, stream=None) -> None:
    check(lib().h3_prepare_qk_i4(ctypes.byref(cfg), tokens, view(x), view(mean), view(codes),
                                 view(scales), stream_ptr(stream)))


def prepare_qk_rope_i8hm(cfg: PrepareCfg, tokens: int, x, weight, cos_t, sin_t, codes, scales,
                         stream=None) -> None:
    check(lib().h3_prepare_qk_rope_i8hm(ctypes.byref(cfg), tokens, view(x), view(weight),
                                        view(cos_t), view(sin_t), view(codes), view(scales),
                                        stream_ptr(stream)))


def prepare_k_rope_smooth_i8hm(cfg: PrepareCfg, tokens: int, x, weight, cos_t, sin_t, mean,
                               codes, scales, stream=None) -> None:
    check(lib().h3_prepare_k_rope_smooth_i8hm(ctypes.byref(cfg), tokens, view(x), view(weight),
                                              view(cos_t), view(sin_t), view(mean), view(codes),
                                              view(scales), stream_ptr(stream)))


def rope_qknorm_f16(cfg: RopeCfg, tokens: int, x, qweight, kweight, cos_t, sin_t, q_out, k_out,
                    v_out=None, stream=None) -> None:
    check(lib().h3_rope_qknorm_f16(ctypes.byref(cfg), tokens, view(x), view(qweight),
                                   view(kweight), view(cos_t), view(sin_t), view(q_out),
                                   view(k_out), view(v_out), stream_ptr(stream)))


def colmean_f32(width: int, tokens: int, x, mean, elem: int = H3_ELEM_F16, stream=None) -> None:
    check(lib().h3_colmean_f32(width, elem, tokens, view(x), view(mean), stream_ptr(stream)))


def transpose_f16(cfg: TransposeCfg, launch_rows: int, rows: int, x, out, stream=None) -> None:
    check(lib().h3_transpose_f16(ctypes.byref(cfg), launch_rows, rows, view(x), view(out),
                                 stream_ptr(stream)))


def transpose_qkv_v_f16(cfg: TransposeCfg, launch_rows: int, rows: int, x, out,
                        stream=None) -> None:
    check(lib().h3_transpose_qkv_v_f16(ctypes.byref(cfg), launch_rows, rows, view(x), view(out),
                                       stream_ptr(stream)))


def attention_i8qkhm(cfg: AttentionCfg, token_count: int, heads: int, qi, qs, ki, ks, vt, out,
                     stream=None) -> None:
    check(lib().h3_attention_i8qkhm(ctypes.byref(cfg), token_count, heads, view(qi), view(qs),
                                    view(ki), view(ks), view(vt), view(out), stream_ptr(stream)))


def attention_i8qk(cfg: AttentionCfg, token_count: int, heads: int, qi, qs, ki, ks, vt, out,
                   stream=None) -> None:
    check(lib().h3_attention_i8qk(ctypes.byref(cfg), token_count, heads, view(qi), view(qs),
                                  view(ki), view(ks), view(vt), view(out), stream_ptr(stream)))


def prepare_plain_i8(cfg: PreparePlainCfg, tokens: int, x, codes, scales, stream=None) -> None:
    check(lib().h3_prepare_plain_i8(ctypes.byref(cfg), tokens, view(x), view(codes), view(scales),
                                    stream_ptr(stream)))


def gemm_i8_qkv_256(cfg: GemmCfg, tokens: int, a, w, w_scale, a_scale, out, stream=None) -> None:
    check(lib().h3_gemm_i8_qkv_256(ctypes.byref(cfg), tokens, view(a), view(w), view(w_scale),
                                   view(a_scale), view(out), stream_ptr(stream)))


def compact_qkv_elements(tokens: int, n: int) -> int:
    """f16 elements of the compact QKV output (src/dispatch.rs:1038-1043)."""
    cap = -(-tokens // 256) * 256
    return tokens * n + (cap - tokens) * (n // 3)


def rope_dit_tables(pos, inv_freq):
    """rope::dit on the host: pos [rows][3] float64, inv_freq [16] float32 (numpy arrays);
    returns (cos, sin) float32 [rows][48]."""
    import numpy as np

    pos = np.ascontiguousarray(pos, np.float64).reshape(-1)
    inv = np.ascontiguousarray(inv_freq, np.float32)
    if inv.size != 16 or pos.size % 3:
        raise ValueError("pos must hold [rows][3] coordinates and inv_freq 16 frequencies")
    rows = pos.size // 3
    cos = np.empty((rows, 48), np.float32)
    sin = np.empty((rows, 48), np.float32)
    check(lib().h3_rope_dit_tables(pos.ctypes.data, rows, inv.ctypes.data, cos.ctypes.data,
                                   sin.ctypes.data))
    return cos, sin


def attention_i4qk(cfg: AttentionCfg, token_count: int, heads: int, qi, qs, ki, ks, vt, out,
                   stream=None) -> None:
    check(lib().h3_attention_i4qk(ctypes.byref(cfg), token_count, heads, view(qi), view(qs),
                                  view(ki), view(ks), view(vt), view(out), stream_ptr(stream)))


def attention_i4qks(cfg: AttentionSkipCfg, token_count: int, heads: int, qi, qs, ki, ks, vt, out,
                    stream=None) -> None:
    check(lib().h3_attention_i4qks(ctypes.byref(cfg), token_count, heads, view(qi), view(qs),
                                   view(ki), view(ks), view(vt), view(out), stream_ptr(stream)))


def capacity(tokens: int, causal: bool = False) -> int:
    """src/stack.rs:299-302."""
    return lib().h3_capacity(tokens, int(causal))


class Stack:
    """The INT8 attention block of the reference's Stack (src/stack.rs): build once, then
    attend_fused (prepare_fused_operands + attention) or attend (the separate route)."""

    def __init__(self, heads: int, tokens: int, eps: float = 1e-5, elem: int = H3_ELEM_F16,
                 ksmooth: bool = False, fused: bool = True, direct_attn: bool = False):
        self.dims = StackDims(heads, tokens, eps, elem, int(ksmooth), int(fused),
                              int(direct_attn))
        handle = ctypes.c_void_p()
        check(lib().h3_stack_build(ctypes.byref(self.dims), ctypes.byref(handle)))
        self.handle = handle
        self.capacity = lib().h3_stack_capacity(handle)

    def close(self) -> None:
        if self.handle:
            lib().h3_stack_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def attend_fused(self, t, fused, qnorm, knorm, cos_t, sin_t, out, stream=None) -> None:
        check(lib().h3_stack_attend_fused(self.handle, t, view(fused), view(qnorm), view(knorm),
                                          view(cos_t), view(sin_t), view(out), stream_ptr(stream)))

    def attend_compact(self, t, compact, qnorm, knorm, cos_t, sin_t, out, stream=None) -> None:
        check(lib().h3_stack_attend_compact(self.handle, t, view(compact), view(qnorm),
                                            view(knorm), view(cos_t), view(sin_t), view(out),
                                            stream_ptr(stream)))

    def attend(self, t, q, k, v, out, stream=None) -> None:
        check(lib().h3_stack_attend(self.handle, t, view(q), view(k), view(v), view(out),
                                    stream_ptr(stream)))

    def operands(self) -> IntQk:
        ops = IntQk()
        check(lib().h3_stack_operands(self.handle, ctypes.byref(ops)))
        return ops


def attention_i8qkhm_cross(cfg: CrossCfg, qi, qs, ki, ks, vt, key_mask, out, stream=None) -> None:
    """Cross-attention with grouped heads and a key-padding mask (an extension)."""
    check(lib().h3_attention_i8qkhm_cross(ctypes.byref(cfg), view(qi), view(qs), view(ki),
                                          view(ks), view(vt), view(key_mask), view(out),
                                          stream_ptr(stream)))


# ------------------------------------------------------------------------- VSA (src/vsa.rs)

def vsa_gather(cfg: VsaCfg, src, x, y, stream=None) -> None:
    check(lib().h3_vsa_gather(ctypes.byref(cfg), view(src), view(x), view(y), stream_ptr(stream)))


def vsa_scatter(cfg: VsaCfg, inverse, x, y, stream=None) -> None:
    check(lib().h3_vsa_scatter(ctypes.byref(cfg), view(inverse), view(x), view(y),
                               stream_ptr(stream)))


def vsa_pool(cfg: VsaCfg, lengths, x, means, stream=None) -> None:
    check(lib().h3_vsa_pool(ctypes.byref(cfg), view(lengths), view(x), view(means),
                            stream_ptr(stream)))


def vsa_scores(cfg: VsaCfg, qm, km, scores, stream=None) -> None:
    check(lib().h3_vsa_scores(ctypes.byref(cfg), view(qm), view(km), view(scores),
                              stream_ptr(stream)))


def vsa_route(cfg: VsaCfg, scores, routes, stream=None) -> None:
    check(lib().h3_vsa_route(ctypes.byref(cfg), view(scores), view(routes), stream_ptr(stream)))


def vsa_coarse(cfg: VsaCfg, scores, vm, coarse, stream=None) -> None:
    check(lib().h3_vsa_coarse(ctypes.byref(cfg), view(scores), view(vm), view(coarse),
                              stream_ptr(stream)))


def vsa_gated_scatter(cfg: VsaCfg, inverse, fine, gate, coarse, out, stream=None) -> None:
    check(lib().h3_vsa_gated_scatter(ctypes.byref(cfg), view(inverse), view(fine), view(gate),
                                     view(coarse), view(out), stream_ptr(stream)))


def vsa_kmean(width: int, tokens: int, x, mean, stream=None) -> None:
    check(lib().h3_vsa_kmean(width, tokens, view(x), view(mean), stream_ptr(stream)))


def vsa_attention_i8(cfg: AttentionCfg, token_count: int, heads: int, qi, qs, ki, ks, vt, out,
                     routes, lengths, stream=None) -> None:
    check(lib().h3_vsa_attention_i8(ctypes.byref(cfg), token_count, heads, view(qi), view(qs),
                                    view(ki), view(ks), view(vt), view(out), view(routes),
                                    view(lengths), stream_ptr(stream)))


def vsa_attention_f16(cfg: AttentionCfg, token_count: int, heads: int, q, k, v, out, routes,
                      lengths, stream=None) -> None:
    """h3_vsa_attention_16 (kernels/vsa_attention_16.loom): token-major f16 q, k, v; scores
    (q . k) * cfg.scale over the kept cubes' live keys."""
    check(lib().h3_vsa_attention_f16(ctypes.byref(cfg), token_count, heads, view(q), view(k),
                                     view(v), view(out), view(routes), view(lengths),
                                     stream_ptr(stream)))


def fp6_workspace_bytes(cfg: AttentionCfg) -> int:
    """Bytes of the workspace h3_attention_i4qk_fp6 converts the int4 operands into."""
    return lib().h3_fp6_workspace_bytes(ctypes.byref(cfg))


def attention_i4qk_fp6(cfg: AttentionCfg, token_count: int, heads: int, qi, qs, ki, ks, vt, out,
                       workspace, stream=None) -> None:
    """h3_attention_i4qk on the FP6 MFMA: the int4 operands converted into `workspace`
    (fp6_workspace_bytes(cfg) bytes), then the head-major kernel's FP6 form."""
    check(lib().h3_attention_i4qk_fp6(ctypes.byref(cfg), token_count, heads, view(qi), view(qs),
                                      view(ki), view(ks), view(vt), view(out), view(workspace),
                                      stream_ptr(stream)))


def scales_workspace_bytes(cfg) -> int:
    """Bytes of the head-major key-scale copy the _ws attention forms need for `cfg`."""
    if isinstance(cfg, AttentionSkipCfg):
        cfg = AttentionCfg(cfg.q_stride, cfg.kv_stride, cfg.out_stride, cfg.tokens,
                           cfg.token_capacity, cfg.scale)
    return int(lib().h3_scales_workspace_bytes(ctypes.byref(cfg)))


def attention_i8qk_ws(cfg: AttentionCfg, token_count: int, heads: int, qi, qs, ki, ks, vt, out,
                      workspace, stream=None) -> None:
    check(lib().h3_attention_i8qk_ws(ctypes.byref(cfg), token_count, heads, view(qi), view(qs),
                                     view(ki), view(ks), view(vt), view(out), view(workspace),
                                     stream_ptr(stream)))


def attention_i8qk_static(cfg: AttentionCfg, token_count: int, heads: int, qi, qs, ki, ks, vt,
                          out, stream=None) -> None:
    """h3_attention_i8qk_static: the _ws form with the library's static scratch array."""
    check(lib().h3_attention_i8qk_static(ctypes.byref(cfg), token_count, heads, view(qi),
                                         view(qs), view(ki), view(ks), view(vt), view(out),
                                         stream_ptr(stream)))


def attention_i4qk_ws(cfg: AttentionCfg, token_count: int, heads: int, qi, qs, ki, ks, vt, out,
                      workspace, stream=None) -> None:
    check(lib().h3_attention_i4qk_ws(ctypes.byref(cfg), token_count, heads, view(qi), view(qs),
                                     view(ki), view(ks), view(vt), view(out), view(workspace),
                                     stream_ptr(stream)))


def attention_i4qks_ws(cfg: AttentionSkipCfg, token_count: int, heads: int, qi, qs, ki, ks, vt,
                       out, workspace, stream=None) -> None:
    check(lib().h3_attention_i4qks_ws(ctypes.byref(cfg), token_count, heads, view(qi), view(qs),
                                      view(ki), view(ks), view(vt), view(out), view(workspace),
                                      stream_ptr(stream)))


def vsa_attention_i8_ws(cfg: AttentionCfg, token_count: int, heads: int, qi, qs, ki, ks, vt, out,
                        routes, lengths, workspace, stream=None) -> None:
    check(lib().h3_vsa_attention_i8_ws(ctypes.byref(cfg), token_count, heads, view(qi), view(qs),
                                       view(ki), view(ks), view(vt), view(out), view(routes),
                                       view(lengths), view(workspace), stream_ptr(stream)))


class VsaOptions:
    """VsaOptions (src/vsa.rs:11-31) with its defaults."""

    def __init__(self, keep_percent=10.0, start=0.2, end=1.0, min_tokens=12288, dense_blocks=()):
        self.keep_percent, self.start, self.end = float(keep_percent), float(start), float(end)
        self.min_tokens = int(min_tokens)
        self.dense_blocks = [int(b) for b in dense_blocks]

    def c(self) -> VsaOptionsC:
        arr = (ctypes.c_uint32 * max(1, len(self.dense_blocks)))(*self.dense_blocks)
        opt = VsaOptionsC(self.keep_percent, self.start, self.end, self.min_tokens,
                          ctypes.cast(arr, ctypes.POINTER(ctypes.c_uint32)), len(self.dense_blocks))
        opt._keep = arr
        return opt

    def validate(self, attention_bits: int = 8) -> None:
        check(lib().h3_vsa_validate(ctypes.byref(self.c()), attention_bits))

    def topk(self, nonprefix: int) -> int:
        return int(lib().h3_vsa_topk(self.keep_percent, nonprefix))

    def dense_reason(self, tokens: int, sigma: float, shift: float):
        r = lib().h3_vsa_dense_reason(ctypes.byref(self.c()), tokens, sigma, shift)
        return None if r is None else r.decode()


def vsa_plan(segments, seq_len: int, nt: int, nh: int, nw: int):
    """Plan::new (src/vsa.rs:94-143): segments [(row0, rows)] of the prefix in order, then the
    nt x nh x nw video grid at the end of the sequence. Returns numpy (src, inverse, lengths,
    prefix_blocks)."""
    import numpy as np

    segs = (VsaSegment * max(1, len(segments)))(*[VsaSegment(a, b) for a, b in segments])
    blocks = ctypes.c_uint32()
    check(lib().h3_vsa_plan_blocks(segs, len(segments), nt, nh, nw, ctypes.byref(blocks)))
    src = np.zeros(64 * blocks.value, np.int32)
    inverse = np.zeros(max(1, seq_len), np.int32)
    lengths = np.zeros(blocks.value, np.int32)
    prefix = ctypes.c_uint32()
    check(lib().h3_vsa_plan(segs, len(segments), seq_len, nt, nh, nw, src.ctypes.data,
                            inverse.ctypes.data, lengths.ctypes.data, ctypes.byref(prefix)))
    return src, inverse[:seq_len], lengths, prefix.value


class Vsa:
    """vsa::device::Runtime (src/vsa/device.rs): build once per plan, then
    attend(layer, q, k, v, out, gate=None) per DiT block; reset() clears the per-layer K means.
    bits 8: INT8 attention (the K means centre the K operand); bits 16: f16 attention."""

    def __init__(self, src, inverse, lengths, prefix_blocks: int, heads: int,
                 options: Optional[VsaOptions] = None, layers: int = 1, bits: int = 8):
        import numpy as np

        self.options = options or VsaOptions()
        src = np.ascontiguousarray(src, np.int32)
        inverse = np.ascontiguousarray(inverse, np.int32)
        lengths = np.ascontiguousarray(lengths, np.int32)
        handle = ctypes.c_void_p()
        opt = self.options.c()
        check(lib().h3_vsa_build_bits(src.ctypes.data, inverse.ctypes.data, lengths.ctypes.data,
                                      len(lengths), len(inverse), prefix_blocks,
                                      ctypes.byref(opt), heads, bits, layers,
                                      ctypes.byref(handle)))
        self.bits = bits
        self.handle = handle
        self.layers = layers

    def close(self) -> None:
        if self.handle:
            lib().h3_vsa_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset(self, stream=None) -> None:
        check(lib().h3_vsa_reset(self.handle, stream_ptr(stream)))

    def attend(self, layer: int, q, k, v, out, gate=None, stream=None) -> None:
        check(lib().h3_vsa_attend(self.handle, layer, view(q), view(k), view(v), view(out),
                                  view(gate), stream_ptr(stream)))

    def buffers(self, layer: int = 0) -> VsaBuffers:
        b = VsaBuffers()
        check(lib().h3_vsa_inspect(self.handle, layer, ctypes.byref(b)))
        return b
