"""Shared helpers for the GPU parity tests: host<->device copies and operand builders."""
from __future__ import annotations

import numpy as np

import oracle as O


def to_dev(a: np.ndarray, dev):
    import torch

    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        t = torch.from_numpy(a.view(np.int16))
    elif a.dtype == np.uint8:
        t = torch.from_numpy(a)
    else:
        t = torch.from_numpy(a)
    return t.to(dev)


def from_dev(t) -> np.ndarray:
    import torch

    t = t.detach().cpu()
    if t.dtype == torch.int16:
        return t.numpy().view(np.uint16)
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def read_device(view) -> np.ndarray:
    """Copy a device binding (an h3attn View) to host bytes with hipMemcpy."""
    import ctypes

    import torch

    torch.cuda.synchronize()
    hip = ctypes.CDLL("libamdhip64.so")
    out = np.empty(view.bytes, np.uint8)
    rc = hip.hipMemcpy(ctypes.c_void_p(out.ctypes.data), ctypes.c_void_p(view.ptr),
                       ctypes.c_size_t(view.bytes), 2)  # hipMemcpyDeviceToHost
    assert rc == 0, f"hipMemcpy failed: {rc}"
    return out


def filled(shape, fill_byte: int, dtype, dev):
    """A device buffer whose every byte is fill_byte (poisoned capacity / guard bytes)."""
    import torch

    n = int(np.prod(shape)) * np.dtype(dtype).itemsize
    t = torch.full((n,), fill_byte, dtype=torch.uint8, device=dev)
    return t


def head_major_operands(rng, heads, tokens, cap, late_match=True):
    """check_head_major_attention inputs (tests/kernels.rs:2021-2046) from numpy's generator:
    int8 codes N(0,1)*24 rounded and clamped, qs = (1+t%7)/512, ks = (1+t%3)/128,
    V^T N(0,1)*0.3 in f16, K row tokens-1 = Q row 31 (a strong late match)."""
    qc = np.zeros((heads, cap, 128), np.int8)
    kc = np.zeros((heads, cap, 128), np.int8)
    qs = np.zeros((heads, cap), np.float32)
    ks = np.zeros((heads, cap), np.float32)
    vt = np.zeros((heads * 128, cap), np.float16)
    t = np.arange(tokens)
    qs[:, :tokens] = ((1 + t % 7) / 512.0).astype(np.float32)
    ks[:, :tokens] = ((1 + t % 3) / 128.0).astype(np.float32)
    qc[:, :tokens] = np.clip(np.round(rng.standard_normal((heads, tokens, 128), np.float32) * 24),
                             -127, 127)
    kc[:, :tokens] = np.clip(np.round(rng.standard_normal((heads, tokens, 128), np.float32) * 24),
                             -127, 127)
    vt[:, :tokens] = (rng.standard_normal((heads * 128, tokens), np.float32) * 0.3).astype(np.float16)
    if late_match:
        for h in range(heads):
            kc[h, tokens - 1] = qc[h, 31]
    return qc, qs, kc, ks, vt.view(np.uint16)


def pack_codes(codes: np.ndarray) -> np.ndarray:
    """int8 [..., 128] -> i32 words [..., 32], low byte first."""
    c = np.ascontiguousarray(codes, np.int8)
    return c.view(np.int32)


def north_star_ok(got: np.ndarray, want: np.ndarray):
    """max-abs 2e-2 and mean-abs 2e-3 on f16 outputs."""
    err = np.abs(got.astype(np.float64) - want)
    return float(err.max()), float(err.mean())
