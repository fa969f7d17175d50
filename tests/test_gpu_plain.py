"""The GEMM-operand quantizer (h3_prepare_plain_i8) on the GPU through the C ABI, bit-exact
against the oracle. Mirrors the reference's tests of prepare_plain_i8 / prepare_plain_f32_i8:
  - f32_preparation_matches_dense_hadamard_and_marks_invalid_rows (tests/kernels.rs:4587-4760):
    widths 256..25600, a NaN / +inf / -inf / overflowing row, guard bytes after the codes and
    the scales, and the same row repeated over 1, 31, 32, 33 tokens;
  - tiled_preparation_matches_single_pass_across_formats (4279-4353): widths 4352 and 14336,
    f16 and f32 inputs, the largest values in the last group;
plus the attention-output shape of the DiT (width 4096, f16) at the BASELINE token counts on
sampled rows, and bf16 input (this build's extension)."""
import numpy as np
import pytest

import h3attn as H
import oracle as O
from helpers import from_dev, to_dev
from test_oracle_plain import reference_rows

pytestmark = pytest.mark.gpu


def run_plain(dev, x, elem, width, stride, tokens=None):
    import torch

    tokens = x.shape[0] if tokens is None else tokens
    codes = torch.full((tokens * stride + 19,), 0x55, dtype=torch.uint8, device=dev)
    scales = torch.full((tokens * 4 + 20,), 0x55, dtype=torch.uint8, device=dev)
    cfg = H.PreparePlainCfg(width, 256, stride, elem)
    H.prepare_plain_i8(cfg, tokens, to_dev(x, dev), codes[:tokens * stride], scales[:tokens * 4])
    c, s = from_dev(codes), from_dev(scales)
    assert np.all(c[tokens * stride:] == 0x55) and np.all(s[tokens * 4:] == 0x55), "guard bytes"
    return c[:tokens * stride].view(np.int8).reshape(tokens, stride), s[:tokens * 4].view(np.float32)


def check_rows(got_c, got_s, want_c, want_s, width):
    assert np.array_equal(got_c[:, :width], want_c[:, :width])
    assert np.all(got_c[:, width:].view(np.uint8) == 0x55), "bytes past the width untouched"
    assert np.array_equal(got_s.view(np.uint32), want_s.view(np.uint32))


@pytest.mark.parametrize("width", [256, 4352, 8192, 14336, 25600])
def test_f32_rows_match_the_oracle_and_mark_invalid_rows(dev, width):
    x = reference_rows(width)
    stride = width + 64
    print(f"prepare_plain f32 width={width}", flush=True)
    c, s = run_plain(dev, x, H.H3_ELEM_F32, width, stride)
    wc, ws = O.prepare_plain_i8(x, O.F32, stride)
    check_rows(c, s, wc, ws, width)
    for r in range(3, 7):
        assert not np.isfinite(s[r]) and np.all(c[r, :width] == 0)


def test_repeated_row_gives_repeated_codes(dev):
    width, stride = 14336, 14400
    row = reference_rows(width)[:1]
    first = None
    for tokens in [1, 31, 32, 33]:
        c, s = run_plain(dev, np.repeat(row, tokens, axis=0), H.H3_ELEM_F32, width, stride)
        if first is None:
            first = (c[0].copy(), s[0])
        assert all(np.array_equal(c[t], first[0]) for t in range(tokens))
        assert np.all(s == first[1])


@pytest.mark.parametrize("width", [4352, 14336])
@pytest.mark.parametrize("elem", [H.H3_ELEM_F16, H.H3_ELEM_F32, H.H3_ELEM_BF16])
def test_tiled_inputs_match_the_oracle(dev, width, elem):
    rows, stride = 5, width + 64
    v = np.zeros((rows, width), np.float32)
    i = np.arange(width)
    v[0] = (((i * 37) % 101).astype(np.float32) - 50.0) * 128.0
    v[0, width - 256:] *= 4.0  # the largest values in the last group
    v[2, 0] = np.nan
    v[3, width - 1] = np.inf
    v[4, 13] = -np.inf
    fmt = {H.H3_ELEM_F16: O.F16, H.H3_ELEM_F32: O.F32, H.H3_ELEM_BF16: O.BF16}[elem]
    x = v if fmt == O.F32 else (O.f16_bits(v) if fmt == O.F16 else O.bf16_bits(v)).reshape(rows, width)
    print(f"prepare_plain tiled inputs width={width} elem={elem}", flush=True)
    c, s = run_plain(dev, x, elem, width, stride)
    wc, ws = O.prepare_plain_i8(x, fmt, stride)
    check_rows(c, s, wc, ws, width)


@pytest.mark.parametrize("width", [256, 768, 4096, 32768])
def test_random_rows_all_widths(dev, width):
    rng = np.random.default_rng(width)
    rows = 67
    v = (rng.standard_normal((rows, width)) * rng.uniform(0.01, 100, (rows, 1))).astype(np.float32)
    x = O.f16_bits(v).reshape(rows, width)
    print(f"prepare_plain random width={width}", flush=True)
    c, s = run_plain(dev, x, H.H3_ELEM_F16, width, width + 128)
    wc, ws = O.prepare_plain_i8(x, O.F16, width + 128)
    check_rows(c, s, wc, ws, width)


@pytest.mark.parametrize("tokens", [31104, 129024])
def test_attention_output_shape_on_sampled_rows(dev, tokens):
    """width INNER = 4096, f16: the attention output feeding the out-projection."""
    import torch

    width = 4096
    g = torch.Generator(device=dev).manual_seed(tokens)
    x = (torch.randn((tokens, width), generator=g, device=dev) * 0.5).half()
    codes = torch.empty((tokens, width), dtype=torch.int8, device=dev)
    scales = torch.empty(tokens, dtype=torch.float32, device=dev)
    print(f"prepare_plain DiT shape tokens={tokens}", flush=True)
    H.prepare_plain_i8(H.PreparePlainCfg(width, 448, width, H.H3_ELEM_F16), tokens, x, codes,
                       scales)
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([[0, 1, tokens - 1],
                                     np.random.default_rng(tokens).integers(0, tokens, 61)]))
    xs = from_dev(x)[rows]
    wc, ws = O.prepare_plain_i8(xs, O.F16, width)
    got_c = codes.cpu().numpy()[rows]
    got_s = scales.cpu().numpy()[rows]
    assert np.array_equal(got_c, wc)
    assert np.array_equal(got_s.view(np.uint32), ws.view(np.uint32))
    assert np.all(np.isfinite(scales.cpu().numpy()))
