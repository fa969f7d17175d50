"""numpy front end of the CPU oracle (oracle/h3oracle.c) — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module, and
only as the checker or the timed CPU baseline; the shipped library (h3-hrx_amd/) never does.
Besides wrapping the C restatement, it holds the reference's closed-form test inputs
(tests/kernels.rs:190-194 `values`) and small numpy helpers.
"""
from __future__ import annotations

import ctypes
import math
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB = HERE / "_build" / "libh3oracle.so"
F16, BF16 = 0, 1

_P = np.ctypeslib.ndpointer
_lib = None


def build() -> pathlib.Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = ctypes.CDLL(str(LIB))
        u16 = _P(np.uint16, flags="C")
        f32 = _P(np.float32, flags="C")
        f64 = _P(np.float64, flags="C")
        i32 = _P(np.int32, flags="C")
        i8 = _P(np.int8, flags="C")
        c_int, c_float, c_double = ctypes.c_int, ctypes.c_float, ctypes.c_double
        L.h3o_half_to_float.argtypes = [ctypes.c_uint16]
        L.h3o_half_to_float.restype = c_float
        L.h3o_float_to_half.argtypes = [c_float]
        L.h3o_float_to_half.restype = ctypes.c_uint16
        L.h3o_config_f32.argtypes = [c_double]
        L.h3o_config_f32.restype = c_float
        L.h3o_prepare_qk_f32.argtypes = [u16, c_int, ctypes.c_void_p, c_int, c_int, c_int, c_int,
                                         c_float, c_int, c_int, i32, f32]
        L.h3o_prepare_qk_f32.restype = None
        L.h3o_quantize_row.argtypes = [f32, c_float, i32, f32]
        L.h3o_quantize_row.restype = None
        L.h3o_hadamard128_f32.argtypes = [f32, f32]
        L.h3o_hadamard128_f32.restype = None
        L.h3o_prepared_qk_f64.argtypes = [u16, f32, c_int, c_int, c_double, i32, f32,
                                          ctypes.c_void_p]
        L.h3o_prepared_qk_f64.restype = None
        L.h3o_colmean_f32.argtypes = [u16, c_int, c_int, c_int, c_int, f32]
        L.h3o_colmean_f32.restype = None
        L.h3o_rope_qknorm_f16.argtypes = [u16, c_int, c_int, c_int, c_int, c_int, f32, f32, f32,
                                          c_float, u16, c_int]
        L.h3o_rope_qknorm_f16.restype = None
        L.h3o_rope_qknorm_f16_ulps.argtypes = [u16, c_int, c_int, c_int, c_int, c_int, f32, f32,
                                               f32, c_float, u16, c_int, c_int]
        L.h3o_rope_qknorm_f16_ulps.restype = None
        L.h3o_rope_qknorm_f64.argtypes = [u16, c_int, c_int, c_int, c_int, c_int, f32, f32, f32,
                                          c_double, f64]
        L.h3o_rope_qknorm_f64.restype = None
        L.h3o_transpose_f16.argtypes = [u16, c_int, c_int, c_int, c_int, c_int, c_int, c_int, u16]
        L.h3o_transpose_f16.restype = None
        L.h3o_attention_f64.argtypes = [i8, f32, i8, f32, u16, c_int, c_int, c_int,
                                        _P(np.int32, flags="C"), c_int, f64, c_int]
        L.h3o_attention_f64.restype = c_int
        L.h3o_unpack_codes.argtypes = [i32, ctypes.c_size_t, i8]
        L.h3o_unpack_codes.restype = None
        L.h3o_cpu_baseline.argtypes = [u16, u16, u16, c_int, c_int, _P(np.int32, flags="C"),
                                       c_int, c_int, f64, ctypes.POINTER(c_double)]
        L.h3o_cpu_baseline.restype = c_double
        L.h3o_gemm_i8_qkv.argtypes = [i8, i8, f32, f32, c_int, c_int, c_int, c_int, u16, c_int]
        L.h3o_gemm_i8_qkv.restype = None
        L.h3o_prepare_plain_i8.argtypes = [ctypes.c_void_p, c_int, c_int, c_int, c_int, i8, f32]
        L.h3o_prepare_plain_i8.restype = None
        L.h3o_prepare_qk_i4_f32.argtypes = [u16, c_int, ctypes.c_void_p, c_int, c_int, c_int, c_int,
                                            c_float, i32, f32]
        L.h3o_prepare_qk_i4_f32.restype = None
        ip = _P(np.int32, flags="C")
        L.h3o_cross_attention_f64.argtypes = [i8, f32, i8, f32, u16, _P(np.uint8, flags="C"),
                                              c_int, c_int, c_int, c_int, c_int, ip, c_int, f64,
                                              c_int]
        L.h3o_cross_attention_f64.restype = c_int
        L.h3o_vsa_plan_blocks.argtypes = [ip, c_int, c_int, c_int, c_int]
        L.h3o_vsa_plan_blocks.restype = c_int
        L.h3o_vsa_plan.argtypes = [ip, ip, c_int, c_int, c_int, c_int, c_int, i32, i32, i32,
                                   ctypes.POINTER(c_int)]
        L.h3o_vsa_plan.restype = c_int
        L.h3o_vsa_topk.argtypes = [c_double, c_int]
        L.h3o_vsa_topk.restype = c_int
        L.h3o_vsa_dense_reason.argtypes = [c_double, c_double, ctypes.c_long, ctypes.c_long,
                                           c_float, c_double]
        L.h3o_vsa_dense_reason.restype = c_int
        L.h3o_vsa_gather.argtypes = [i32, c_int, c_int, c_int, u16, u16]
        L.h3o_vsa_gather.restype = None
        L.h3o_vsa_scatter.argtypes = [i32, c_int, c_int, u16, u16]
        L.h3o_vsa_scatter.restype = None
        L.h3o_vsa_pool.argtypes = [i32, c_int, c_int, u16, f32]
        L.h3o_vsa_pool.restype = None
        L.h3o_vsa_scores.argtypes = [f32, f32, c_int, c_int, f32]
        L.h3o_vsa_scores.restype = None
        L.h3o_vsa_route.argtypes = [f32, c_int, c_int, c_int, c_int, i32]
        L.h3o_vsa_route.restype = None
        L.h3o_vsa_coarse_f64.argtypes = [f32, f32, c_int, c_int, f64]
        L.h3o_vsa_coarse_f64.restype = None
        L.h3o_vsa_gated_scatter.argtypes = [i32, c_int, c_int, u16, u16, f32, u16]
        L.h3o_vsa_gated_scatter.restype = None
        L.h3o_vsa_kmean.argtypes = [f32, c_int, c_int, f32]
        L.h3o_vsa_kmean.restype = None
        L.h3o_vsa_attention_f64.argtypes = [i8, f32, i8, f32, u16, c_int, c_int, c_int, i32, i32,
                                            ip, c_int, f64, c_int]
        L.h3o_vsa_attention_f64.restype = c_int
        L.h3o_vsa_attention_f16_f64.argtypes = [u16, u16, u16, c_int, c_int, ctypes.c_double,
                                                i32, i32, ip, c_int, f64, c_int]
        L.h3o_vsa_attention_f16_f64.restype = c_int
        L.h3o_max_threads.argtypes = []
        L.h3o_max_threads.restype = c_int
        _lib = L
    return _lib


# --------------------------------------------------------------------- reference test inputs

def values(n: int, scale: float) -> np.ndarray:
    """tests/kernels.rs:190-194: ((i*37 % 101) - 50) * scale / 50 in f32."""
    i = np.arange(n, dtype=np.int64)
    return ((((i * 37) % 101).astype(np.float32) - np.float32(50.0)) * np.float32(scale)
            / np.float32(50.0)).astype(np.float32)


def f16_bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32).astype(np.float16)).view(np.uint16)


def bf16_bits(a: np.ndarray) -> np.ndarray:
    """Round f32 to bf16 (nearest even) and return the bit patterns."""
    u = np.ascontiguousarray(np.asarray(a, dtype=np.float32)).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def widen(bits: np.ndarray, fmt: int) -> np.ndarray:
    if fmt == BF16:
        return (bits.astype(np.uint32) << 16).view(np.float32)
    return bits.view(np.float16).astype(np.float32)


def capacity(tokens: int, causal: bool = False) -> int:
    """src/stack.rs:299-302."""
    waves = 8 if (causal or tokens >= 4096) else 4
    cap = -(-(tokens + 16) // 32) * 32
    cap = max(cap, -(-tokens // (16 * waves)) * 16 * waves)
    return max(cap, -(-tokens // 256) * 256)


EXTRA_Q_F64 = 1.0 / math.sqrt(128.0) / 128.0


def config_f32(v: float) -> float:
    return float(lib().h3o_config_f32(v))


# --------------------------------------------------------------------- oracle calls

def prepare_qk(x_bits: np.ndarray, fmt: int, mean, tokens: int, row_stride: int, head_offset: int,
               heads: int, extra: float, head_major: bool = False, cap: int = 0):
    """fp32 restatement of the quantizer; returns (codes i32, scales f32)."""
    if head_major:
        codes = np.zeros((heads * cap, 32), np.int32)
        scales = np.zeros((heads, cap), np.float32)
    else:
        codes = np.zeros((tokens, heads * 32), np.int32)
        scales = np.zeros((tokens, heads), np.float32)
    m = None
    if mean is not None:
        m = np.ascontiguousarray(mean, dtype=np.float32)
    lib().h3o_prepare_qk_f32(np.ascontiguousarray(x_bits, np.uint16), fmt,
                             None if m is None else m.ctypes.data, tokens, row_stride,
                             head_offset, heads, extra, int(head_major), cap, codes, scales)
    return codes, scales


def prepared_qk_f64(x_bits: np.ndarray, mean: np.ndarray, tokens: int, heads: int, extra: float):
    """tests/kernels.rs:1704-1741; returns (words, scales, codes f64)."""
    words = np.zeros((tokens, heads * 32), np.int32)
    scales = np.zeros((tokens, heads), np.float32)
    codes = np.zeros((tokens, heads * 128), np.float64)
    lib().h3o_prepared_qk_f64(np.ascontiguousarray(x_bits, np.uint16),
                              np.ascontiguousarray(mean, np.float32), tokens, heads, extra, words,
                              scales, codes.ctypes.data)
    return words, scales, codes


def colmean(x_bits: np.ndarray, fmt: int, tokens: int, width: int, row_stride: int) -> np.ndarray:
    out = np.zeros(width, np.float32)
    lib().h3o_colmean_f32(np.ascontiguousarray(x_bits, np.uint16), fmt, tokens, width,
                          row_stride, out)
    return out


def rope_qknorm_f16(x_bits, fmt, tokens, row_stride, head_offset, heads, weight, cos_t, sin_t,
                    eps, r_ulps: int = 0) -> np.ndarray:
    """RMSNorm + RoPE to f16 in this build's fixed fp32 order; r_ulps moves the RMS reciprocal
    by that many units in the last place (a sensitivity probe for an rsqrt that is not correctly
    rounded)."""
    out = np.zeros((tokens, heads * 128), np.uint16)
    lib().h3o_rope_qknorm_f16_ulps(np.ascontiguousarray(x_bits, np.uint16), fmt, tokens,
                                   row_stride, head_offset, heads,
                                   np.ascontiguousarray(weight, np.float32),
                                   np.ascontiguousarray(cos_t, np.float32),
                                   np.ascontiguousarray(sin_t, np.float32), eps, out, heads * 128,
                                   int(r_ulps))
    return out


def rope_qknorm_f64(x_bits, fmt, tokens, row_stride, head_offset, heads, weight, cos_t, sin_t,
                    eps) -> np.ndarray:
    out = np.zeros((tokens, heads, 128), np.float64)
    lib().h3o_rope_qknorm_f64(np.ascontiguousarray(x_bits, np.uint16), fmt, tokens, row_stride,
                              head_offset, heads, np.ascontiguousarray(weight, np.float32),
                              np.ascontiguousarray(cos_t, np.float32),
                              np.ascontiguousarray(sin_t, np.float32), eps, out)
    return out


def transpose(x_bits, fmt, rows, row_stride, col_offset, width, cap, clear_to, out=None):
    if out is None:
        out = np.zeros((width, cap), np.uint16)
    lib().h3o_transpose_f16(np.ascontiguousarray(x_bits, np.uint16), fmt, rows, row_stride,
                            col_offset, width, cap, clear_to, out)
    return out


def unpack(words: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(words, np.int32)
    return w.view(np.int8).reshape(*w.shape[:-1], w.shape[-1] * 4)


def attention_f64(qc, qs, kc, ks, vt, tokens, cap, heads, rows, threads=0) -> np.ndarray:
    """Head-major int8 codes qc/kc [heads][cap][128], scales [heads][cap], vt [heads*128][cap]
    f16 bits; returns f64 [len(rows)][heads][128]."""
    rows = np.ascontiguousarray(rows, np.int32)
    out = np.zeros((len(rows), heads, 128), np.float64)
    lib().h3o_attention_f64(np.ascontiguousarray(qc, np.int8), np.ascontiguousarray(qs, np.float32),
                            np.ascontiguousarray(kc, np.int8), np.ascontiguousarray(ks, np.float32),
                            np.ascontiguousarray(vt, np.uint16), tokens, cap, heads, rows,
                            len(rows), out, threads)
    return out


def cpu_baseline(q_bits, k_bits, v_bits, tokens, heads, rows, threads=0):
    """Times the reference's CPU path; returns (per_row_seconds, fixed_seconds, out)."""
    rows = np.ascontiguousarray(rows, np.int32)
    out = np.zeros((len(rows), heads, 128), np.float64)
    fixed = ctypes.c_double(0.0)
    per_row = lib().h3o_cpu_baseline(np.ascontiguousarray(q_bits, np.uint16),
                                     np.ascontiguousarray(k_bits, np.uint16),
                                     np.ascontiguousarray(v_bits, np.uint16), tokens, heads, rows,
                                     len(rows), threads, out, ctypes.byref(fixed))
    return per_row, fixed.value, out


def max_threads() -> int:
    return int(lib().h3o_max_threads())


def gemm_i8_qkv(a: np.ndarray, w: np.ndarray, ws: np.ndarray, as_: np.ndarray, k: int,
                threads: int = 0) -> np.ndarray:
    """Compact INT8 QKV projection; a [m][k_stride] int8, w [n][k_stride] int8. Returns the f16
    bits of the whole output: m*n + (cap - m)*n/3 elements (Q/K rows, then V^T)."""
    a = np.ascontiguousarray(a, np.int8)
    w = np.ascontiguousarray(w, np.int8)
    m, k_stride = a.shape
    n = w.shape[0]
    cap = -(-m // 256) * 256
    out = np.zeros(m * n + (cap - m) * (n // 3), np.uint16)
    lib().h3o_gemm_i8_qkv(a.reshape(-1), w.reshape(-1), np.ascontiguousarray(ws, np.float32),
                          np.ascontiguousarray(as_, np.float32), m, n, k, k_stride, out, threads)
    return out


F32 = 2


def prepare_plain_i8(x: np.ndarray, fmt: int, out_stride: int):
    """prepare_plain_i8 (fmt F16/BF16: x holds 16-bit patterns) or prepare_plain_f32_i8 (fmt F32:
    x float32), x [tokens][width]. Returns (codes int8 [tokens][out_stride], scales f32)."""
    x = np.ascontiguousarray(x, np.float32 if fmt == F32 else np.uint16)
    tokens, width = x.shape
    codes = np.zeros((tokens, out_stride), np.int8)
    scales = np.zeros(tokens, np.float32)
    lib().h3o_prepare_plain_i8(x.ctypes.data, fmt, tokens, width, out_stride, codes.reshape(-1),
                               scales)
    return codes, scales


def prepare_qk_i4(x_bits: np.ndarray, fmt: int, mean, tokens: int, row_stride: int,
                  head_offset: int, heads: int, extra: float):
    """int4 quantizer, token-major; returns (codes i32 [tokens][heads*16], scales f32)."""
    codes = np.zeros((tokens, heads * 16), np.int32)
    scales = np.zeros((tokens, heads), np.float32)
    m = None if mean is None else np.ascontiguousarray(mean, np.float32)
    lib().h3o_prepare_qk_i4_f32(np.ascontiguousarray(x_bits, np.uint16), fmt,
                                None if m is None else m.ctypes.data, tokens, row_stride,
                                head_offset, heads, extra, codes, scales)
    return codes, scales


def unpack_i4(words: np.ndarray) -> np.ndarray:
    """Words of eight 4-bit codes (low nibble first) -> int8 codes, last axis x8."""
    w = np.ascontiguousarray(words, np.int32).view(np.uint32)
    sh = (np.arange(8, dtype=np.uint32) * 4)
    nib = ((w[..., None] >> sh) & 15).astype(np.int8)
    nib = np.where(nib >= 8, nib - 16, nib).astype(np.int8)
    return nib.reshape(*w.shape[:-1], w.shape[-1] * 8)


# --------------------------------------------------------------------- VSA (h3oracle_vsa.c)

DENSE_REASONS = {0: None, 1: "below_min_tokens", 2: "outside_sigma_window"}


def vsa_plan(segments, seq_len: int, nt: int, nh: int, nw: int):
    """src/vsa.rs:94-143. segments: [(row0, rows)] of the prefix (text, references, audio) in
    order; the video grid nt x nh x nw ends the sequence. Returns (src, inverse, lengths,
    prefix_blocks)."""
    row0 = np.ascontiguousarray([s[0] for s in segments] or [0], np.int32)
    rows = np.ascontiguousarray([s[1] for s in segments] or [0], np.int32)
    n_segs = len(segments)
    blocks = lib().h3o_vsa_plan_blocks(rows, n_segs, nt, nh, nw)
    src = np.zeros(64 * blocks, np.int32)
    inverse = np.zeros(max(seq_len, 1), np.int32)
    lengths = np.zeros(max(blocks, 1), np.int32)
    prefix = ctypes.c_int(0)
    got = lib().h3o_vsa_plan(row0, rows, n_segs, seq_len, nt, nh, nw, src, inverse, lengths,
                             ctypes.byref(prefix))
    if got < 0:
        raise ValueError("VSA layout must cover every live token")
    return src, inverse[:seq_len], lengths[:blocks], prefix.value


def vsa_topk(keep_percent: float, nonprefix: int) -> int:
    return int(lib().h3o_vsa_topk(keep_percent, nonprefix))


def vsa_dense_reason(start, end, min_tokens, tokens, sigma, shift):
    return DENSE_REASONS[lib().h3o_vsa_dense_reason(start, end, min_tokens, tokens, sigma, shift)]


def vsa_gather(src, tokens, x_bits):
    x = np.ascontiguousarray(x_bits, np.uint16)
    width = x.shape[1]
    src = np.ascontiguousarray(src, np.int32)
    y = np.zeros((len(src), width), np.uint16)
    lib().h3o_vsa_gather(src, len(src), tokens, width, x, y)
    return y


def vsa_scatter(inverse, x_bits):
    x = np.ascontiguousarray(x_bits, np.uint16)
    inverse = np.ascontiguousarray(inverse, np.int32)
    y = np.zeros((len(inverse), x.shape[1]), np.uint16)
    lib().h3o_vsa_scatter(inverse, len(inverse), x.shape[1], x, y)
    return y


def vsa_pool(lengths, x_bits):
    x = np.ascontiguousarray(x_bits, np.uint16)
    lengths = np.ascontiguousarray(lengths, np.int32)
    means = np.zeros((len(lengths), x.shape[1]), np.float32)
    lib().h3o_vsa_pool(lengths, len(lengths), x.shape[1], x, means)
    return means


def vsa_scores(qm, km, heads):
    qm = np.ascontiguousarray(qm, np.float32)
    km = np.ascontiguousarray(km, np.float32)
    blocks = qm.shape[0]
    out = np.zeros((heads, blocks, blocks), np.float32)
    lib().h3o_vsa_scores(qm, km, blocks, heads, out)
    return out


def vsa_route(scores, prefix, topk):
    scores = np.ascontiguousarray(scores, np.float32)
    heads, blocks, _ = scores.shape
    routes = np.zeros((heads, blocks, blocks), np.int32)
    lib().h3o_vsa_route(scores, blocks, heads, prefix, topk, routes)
    return routes


def vsa_coarse_f64(scores, vm):
    scores = np.ascontiguousarray(scores, np.float32)
    vm = np.ascontiguousarray(vm, np.float32)
    heads, blocks, _ = scores.shape
    out = np.zeros((blocks, heads * 128), np.float64)
    lib().h3o_vsa_coarse_f64(scores, vm, blocks, heads, out)
    return out


def vsa_gated_scatter(inverse, fine_bits, gate_bits, coarse):
    inverse = np.ascontiguousarray(inverse, np.int32)
    fine = np.ascontiguousarray(fine_bits, np.uint16)
    gate = np.ascontiguousarray(gate_bits, np.uint16)
    width = fine.shape[1]
    out = np.zeros((len(inverse), width), np.uint16)
    lib().h3o_vsa_gated_scatter(inverse, len(inverse), width, fine, gate,
                                np.ascontiguousarray(coarse, np.float32), out)
    return out


def vsa_kmean(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(x.shape[1], np.float32)
    lib().h3o_vsa_kmean(x, x.shape[0], x.shape[1], out)
    return out


def vsa_attention_f16_f64(q, k, v, tokens, heads, scale, routes, lengths, rows, threads=0):
    """f16 bits q, k, v token-major [>= tokens][heads*128], logits (q . k) * scale, routes
    [heads][blocks][blocks], lengths [blocks]; f64 [len(rows)][heads][128]."""
    rows = np.ascontiguousarray(rows, np.int32)
    out = np.zeros((len(rows), heads, 128), np.float64)
    lib().h3o_vsa_attention_f16_f64(np.ascontiguousarray(q, np.uint16).reshape(-1),
                                    np.ascontiguousarray(k, np.uint16).reshape(-1),
                                    np.ascontiguousarray(v, np.uint16).reshape(-1), tokens, heads,
                                    float(scale),
                                    np.ascontiguousarray(routes, np.int32).reshape(-1),
                                    np.ascontiguousarray(lengths, np.int32), rows, len(rows), out,
                                    threads)
    return out


def vsa_attention_f64(qc, qs, kc, ks, vt, tokens, cap, heads, routes, lengths, rows, threads=0):
    """Token-major int8 codes qc/kc [cap][heads*128], scales [cap][heads], vt [heads*128][cap] f16
    bits, routes [heads][blocks][blocks], lengths [blocks]; f64 [len(rows)][heads][128]."""
    rows = np.ascontiguousarray(rows, np.int32)
    out = np.zeros((len(rows), heads, 128), np.float64)
    lib().h3o_vsa_attention_f64(np.ascontiguousarray(qc, np.int8).reshape(-1),
                                np.ascontiguousarray(qs, np.float32).reshape(-1),
                                np.ascontiguousarray(kc, np.int8).reshape(-1),
                                np.ascontiguousarray(ks, np.float32).reshape(-1),
                                np.ascontiguousarray(vt, np.uint16).reshape(-1), tokens, cap,
                                heads, np.ascontiguousarray(routes, np.int32).reshape(-1),
                                np.ascontiguousarray(lengths, np.int32), rows, len(rows), out,
                                threads)
    return out


def cross_attention_f64(qc, qs, kc, ks, vt, mask, kv_tokens, rows, threads=0):
    """Head-major codes qc [qh][q_cap][128], kc [kh][kv_cap][128], scales [heads][cap], vt
    [kh*128][kv_cap] f16 bits, mask [kv_tokens] u8; f64 [len(rows)][qh][128]."""
    qc = np.ascontiguousarray(qc, np.int8)
    kc = np.ascontiguousarray(kc, np.int8)
    qh, q_cap, _ = qc.shape
    kh, kv_cap, _ = kc.shape
    rows = np.ascontiguousarray(rows, np.int32)
    out = np.zeros((len(rows), qh, 128), np.float64)
    lib().h3o_cross_attention_f64(qc.reshape(-1), np.ascontiguousarray(qs, np.float32).reshape(-1),
                                  kc.reshape(-1), np.ascontiguousarray(ks, np.float32).reshape(-1),
                                  np.ascontiguousarray(vt, np.uint16).reshape(-1),
                                  np.ascontiguousarray(mask, np.uint8), q_cap, kv_tokens, kv_cap,
                                  qh, kh, rows, len(rows), out, threads)
    return out
