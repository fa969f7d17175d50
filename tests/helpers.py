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


# ---- the FP6 form of the int4 attention (h3_attention_i4qk_fp6): its workspace layout, restated

def e2m3_value(code):
    """The OCP FP6 E2M3 value of a 6-bit code: sign bit 5, exponent bits 4-3 (bias 1), mantissa
    bits 2-0, subnormal at exponent 0; no infinities or NaNs."""
    code = np.asarray(code, np.int64)
    s = np.where(code & 32, -1.0, 1.0)
    e = (code >> 3) & 3
    m = (code & 7).astype(np.float64)
    return s * np.where(e == 0, m / 8.0, (1.0 + m / 8.0) * np.exp2(e - 1.0))


# e2m3 code of c/2 for the signed nibble c = 0..7, -8..-1 (index = the nibble's 4 bits)
FP6_HALF_CODES = np.array([0, 4, 8, 12, 16, 18, 20, 22, 56, 54, 52, 50, 48, 44, 40, 36], np.uint8)


def fp6_rows(words, heads, tokens, cap):
    """Token-major int4 words [rows][heads*16] (low nibble first) -> the FP6 head-major rows
    [heads*cap][128] bytes of the workspace for rows < tokens (other rows left 0): block b of a
    row holds channels 32b..32b+31 as six-bit codes, code i in bits 6i.. of its first 24 bytes,
    then 8 zero bytes."""
    w = np.ascontiguousarray(words, np.int32).view(np.uint32)[:tokens].reshape(tokens, heads, 16)
    nib = np.stack([(w >> np.uint32(4 * j)) & np.uint32(15) for j in range(8)], -1)
    codes = FP6_HALF_CODES[nib.reshape(tokens, heads, 128)].astype(np.uint64)  # [t][h][ch]
    out = np.zeros((heads, cap, 4, 32), np.uint8)
    for b in range(4):
        blk = codes[:, :, 32 * b:32 * b + 32]
        acc = np.zeros((tokens, heads, 3), np.uint64)  # 192 bits as three u64
        for i in range(32):
            bit = 6 * i
            acc[..., bit // 64] |= blk[..., i] << np.uint64(bit % 64)
            if bit % 64 > 58:
                acc[..., bit // 64 + 1] |= blk[..., i] >> np.uint64(64 - bit % 64)
        out[:, :tokens, b, :24] = acc.astype("<u8").view(np.uint8).reshape(tokens, heads, 24).transpose(1, 0, 2)
    return out.reshape(heads * cap, 128)


def fp6_decode_rows(rows):
    """The values of FP6 rows [n][128] bytes: [n][128] channel values."""
    r = np.ascontiguousarray(rows, np.uint8).reshape(-1, 4, 32)[:, :, :24]
    q = r.reshape(-1, 4, 3, 8).copy().view("<u8")[..., 0]  # [n][4][3] u64
    vals = np.zeros((r.shape[0], 4, 32), np.float64)
    for i in range(32):
        bit = 6 * i
        c = (q[..., bit // 64] >> np.uint64(bit % 64)) & np.uint64(63)
        if bit % 64 > 58:
            c |= (q[..., bit // 64 + 1] << np.uint64(64 - bit % 64)) & np.uint64(63)
        vals[..., i] = e2m3_value(c.astype(np.int64))
    return vals.reshape(-1, 128)


# ---- inputs whose scores rise at every 32-key tile (the exact path at every tile)

LOG2E = 1.4426950408889634


def rising_scores(rng, tokens, rise=(4.7, 5.7), spread=0.4):
    """Score targets in log2 units: key j gets base(j // 32) + e_j, e_j in [0, spread), where
    the bases of consecutive 32-key tiles step up by rise[0]..rise[1] (a different step each
    tile). With rise[0] - spread > 4, each of a tile's probabilities against the max of all
    earlier keys exceeds 2^4, so any 16 of them sum past 2^8."""
    tiles = (tokens + 31) // 32
    steps = rng.uniform(rise[0], rise[1], tiles)
    base = 1.0 + np.concatenate([[0.0], np.cumsum(steps)[:-1]])
    return base[np.arange(tokens) // 32] + rng.uniform(0.0, spread, tokens)


def rank1_operands(rng, q_heads, q_tokens, q_cap, kv_heads, kv_tokens, kv_cap, code_min=48,
                   code_max=63, mult_max=(2, 2), gain=(1.0, 1.25)):
    """Codes of rank one, Q rows a_q * u and K rows b_j * w (u random with |u_c| in
    [code_min, code_max] and random signs, w = u moved by at most 2 per channel, integer
    multipliers a, b >= 1), so S_qj = a_q b_j (u.w) exactly, and scales that set the score of
    query q and key j (log2 units) to g_q * rising_scores[j]: ks_j = target_j / (b_j u.w),
    qs_q = g_q / (a_q log2 e). The codes span most of the int8 range, as absmax-quantised rows
    do, so |S| >= u.w (about 4e5 with the defaults): the head-major kernels dequantise S to
    within 0.75 units of S (a bias added in the accumulator, removed by one FMA), which at the
    ~1,700 log2 units these scores reach over 8,193 keys stays below 0.004 log2 units. Head-major
    codes [heads][cap][128] int8, scales [heads][cap] f32, V^T [kv_heads*128][kv_cap] f16 bits
    N(0,1)*0.3; capacity rows zero."""
    u = rng.integers(code_min, code_max + 1, 128) * rng.choice([-1, 1], 128)
    w = np.clip(u + rng.integers(-2, 3, 128), -code_max, code_max)
    uw = int(u @ w)
    assert uw > 0
    qc = np.zeros((q_heads, q_cap, 128), np.int8)
    kc = np.zeros((kv_heads, kv_cap, 128), np.int8)
    a = rng.integers(1, mult_max[0] + 1, (q_heads, q_tokens))
    b = rng.integers(1, mult_max[1] + 1, (kv_heads, kv_tokens))
    assert code_max * max(mult_max) <= 127
    qc[:, :q_tokens] = (a[..., None] * u).astype(np.int8)
    kc[:, :kv_tokens] = (b[..., None] * w).astype(np.int8)
    target = np.stack([rising_scores(rng, kv_tokens) for _ in range(kv_heads)])
    g = rng.uniform(gain[0], gain[1], (q_heads, q_tokens))
    qs = np.zeros((q_heads, q_cap), np.float32)
    ks = np.zeros((kv_heads, kv_cap), np.float32)
    qs[:, :q_tokens] = (g / (a * LOG2E)).astype(np.float32)
    ks[:, :kv_tokens] = (target / (b * uw)).astype(np.float32)
    vt = np.zeros((kv_heads * 128, kv_cap), np.float16)
    vt[:, :kv_tokens] = (rng.standard_normal((kv_heads * 128, kv_tokens), np.float32) *
                         0.3).astype(np.float16)
    return qc, qs, kc, ks, vt.view(np.uint16)
