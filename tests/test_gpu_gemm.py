"""The compact INT8 QKV projection (h3_gemm_i8_qkv_256) on the GPU, through the C ABI.

Mirrors the reference's tests of h3_gemm_i8_qkv_256:
  - compact_qkv_matches_scalar_projection_and_zeroes_v_padding (tests/kernels.rs:4392-4460):
    k=64, n=384, rows 1/17/255/256/257/513, non-finite and saturating scales, V^T padding
    zeroed, 64 guard bytes past the output untouched;
  - compact_qkv_dispatch_crosses_specialized_row_bound (5365-5420): rows 65535/65536/65537/17;
plus a K that is not a multiple of 128 with padded rows, and the DiT projection shape
(K=4096, N=12288) checked on sampled tokens. Bit-exact against the oracle everywhere.
"""
import numpy as np
import pytest

import h3attn as H
import oracle as O
from helpers import from_dev, to_dev
from test_oracle_gemm import reference_inputs, same_bits

pytestmark = pytest.mark.gpu


def run_gemm(dev, a, w, ws, as_, k, guard=True, m_group=3):
    import torch

    m, stride = a.shape
    n = w.shape[0]
    elems = H.compact_qkv_elements(m, n)
    out = torch.full((elems * 2 + (64 if guard else 0),), 0x7F, dtype=torch.uint8, device=dev)
    if guard:
        out[elems * 2:] = 0xA5
    cfg = H.GemmCfg(k, n, stride, m_group)
    H.gemm_i8_qkv_256(cfg, m, to_dev(a, dev), to_dev(w, dev), to_dev(ws, dev), to_dev(as_, dev),
                      out)
    host = from_dev(out)
    if guard:
        assert np.all(host[elems * 2:] == 0xA5), "wrote past the output binding"
    return host[:elems * 2].view(np.uint16)


@pytest.mark.parametrize("rows", [1, 17, 255, 256, 257, 513])
def test_compact_qkv_matches_the_scalar_projection(dev, rows):
    a, w, ws, scales = reference_inputs(rows)
    print(f"gemm reference case rows={rows}", flush=True)
    same_bits(run_gemm(dev, a, w, ws, scales, 64), O.gemm_i8_qkv(a, w, ws, scales, 64))


@pytest.mark.parametrize("rows", [65535, 65536, 65537, 17])
def test_compact_qkv_across_the_row_bound(dev, rows):
    """tests/kernels.rs:5365-5420 inputs: w = (i/k % 5) - 2, a = (i/k % 7) - 3, ws = 1/k, as = 1."""
    k, n = 64, 384
    w = ((np.arange(n * k) // k % 5) - 2).astype(np.int8).reshape(n, k)
    a = ((np.arange(rows * k) // k % 7) - 3).astype(np.int8).reshape(rows, k)
    ws = np.full(n, 1.0 / k, np.float32)
    as_ = np.ones(rows, np.float32)
    print(f"gemm row-bound case rows={rows}", flush=True)
    same_bits(run_gemm(dev, a, w, ws, as_, k), O.gemm_i8_qkv(a, w, ws, as_, k))


def test_compact_qkv_half_step_and_row_padding(dev):
    """K = 192 (one full 128-byte step and a 64-byte one), rows padded to 256 bytes with
    garbage past K, N = 1152 (a partial last V tile), M = 700."""
    rng = np.random.default_rng(3)
    m, n, k, stride = 700, 1152, 192, 256
    a = rng.integers(-128, 128, (m, stride), dtype=np.int8)
    w = rng.integers(-128, 128, (n, stride), dtype=np.int8)
    ws = rng.uniform(1e-3, 2e-2, n).astype(np.float32)
    as_ = rng.uniform(1e-3, 5e-2, m).astype(np.float32)
    print("gemm half-step case", flush=True)
    same_bits(run_gemm(dev, a, w, ws, as_, k), O.gemm_i8_qkv(a, w, ws, as_, k))


@pytest.mark.parametrize("k", [256, 320, 384, 448, 576])
def test_compact_qkv_step_counts(dev, k):
    """K advances 128 bytes a step through two LDS stages: 256-576 bytes are even and odd step
    counts (2-5), with and without a final 64-byte half step (320, 448, 576), rows padded past K
    by garbage and a partial last tile in M and in V, bit-exact."""
    rng = np.random.default_rng(k)
    m, n, stride = 300, 768, k + 64
    a = rng.integers(-128, 128, (m, stride), dtype=np.int8)
    w = rng.integers(-128, 128, (n, stride), dtype=np.int8)
    ws = rng.uniform(1e-3, 2e-2, n).astype(np.float32)
    as_ = rng.uniform(1e-3, 5e-2, m).astype(np.float32)
    print(f"gemm step-count case k={k}", flush=True)
    same_bits(run_gemm(dev, a, w, ws, as_, k), O.gemm_i8_qkv(a, w, ws, as_, k))


@pytest.mark.parametrize("m", [31104, 129024])
def test_dit_projection_shape_on_sampled_tokens(dev, m):
    """K = 4096, N = 3*4096 at the BASELINE token counts; every column of 48 sampled tokens
    (and the V^T padding) against exact products computed in float64."""
    import torch

    k, n = 4096, 12288
    g = torch.Generator(device=dev).manual_seed(m)
    a = torch.randint(-128, 128, (m, k), dtype=torch.int8, device=dev, generator=g)
    w = torch.randint(-128, 128, (n, k), dtype=torch.int8, device=dev, generator=g)
    ws = (torch.rand(n, device=dev, generator=g) * 2e-4 + 1e-5).float()
    as_ = (torch.rand(m, device=dev, generator=g) * 2e-2 + 1e-3).float()
    elems = H.compact_qkv_elements(m, n)
    out = torch.empty(elems, dtype=torch.int16, device=dev)
    print(f"gemm DiT shape m={m}", flush=True)
    H.gemm_i8_qkv_256(H.GemmCfg(k, n, k, 1), m, a, w, ws, as_, out)
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([[0, 1, 255, 256, m - 1],
                                     np.random.default_rng(m).integers(0, m, 43)]))
    a_s = a[torch.from_numpy(rows).to(dev)].cpu().numpy().astype(np.float64)
    w_h = w.cpu().numpy().astype(np.float64)
    dot = (a_s @ w_h.T).astype(np.int64)  # exact: |sum| < 2^26
    wsh, ash = ws.cpu().numpy(), as_.cpu().numpy()[rows]
    raw = (dot.astype(np.float32) * wsh[None, :]) * ash[:, None] + np.float32(0)
    raw = np.clip(raw, np.float32(-65472), np.float32(65472))
    want = raw.astype(np.float16).view(np.uint16)
    host = from_dev(out)
    qk = 2 * n // 3
    cap = -(-m // 256) * 256
    got_qk = host[:m * qk].reshape(m, qk)[rows]
    vt = host[m * qk:].reshape(n // 3, cap)
    assert np.array_equal(got_qk, want[:, :qk])
    assert np.array_equal(vt[:, rows].T, want[:, qk:])
    assert np.all(vt[:, m:] == 0)
