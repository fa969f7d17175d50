"""Operand preparation kernels on the GPU: bit-exact against the oracle.

Mirrors the reference's tests:
  - prepare_qk_int8_rotates_quantises_and_packs_the_attention_operands (tests/kernels.rs:1752-1849)
  - subgroup_shuffle_preparation_matches_lds_repeatedly (3278-3371): offsets, partial head
    rounds, 256 heads, poisoned capacity, repeated launches byte-identical
  - rotary_qk_norm_matches_cpu_for_all_head_layouts_and_copies_v (1125-1241)
  - fused_qkv_operands_are_byte_identical_to_separate_preparation (3153-3276)
  - transposed_values_clear_reused_capacity (3373-3444)
All through the C ABI.
"""
import math

import numpy as np
import pytest

import h3attn as H
import oracle as O
from helpers import filled, from_dev, to_dev

pytestmark = pytest.mark.gpu

EXTRA = O.config_f32(O.EXTRA_Q_F64)


def prepare_inputs(tokens, heads, offset, stride_extra=128):
    """subgroup_shuffle_preparation inputs (tests/kernels.rs:3291-3304)."""
    width = heads * 128
    stride = offset + width + stride_extra
    x = O.values(tokens * stride, 0.7).astype(np.float16).reshape(tokens, stride)
    mean = O.values(stride, 0.1)
    mean[offset:offset + 128] = 0.0
    x[:, offset:offset + 128] = 0
    if heads > 1:
        x[:, offset + 128:offset + 256] = np.float16(65504.0)
    return np.ascontiguousarray(x).view(np.uint16), mean, stride


CASES = [(1, 1, 0, 1.0), (257, 17, 128, EXTRA), (3, 256, 128, 1.0), (2049, 56, 128, EXTRA),
         (4097, 56, 0, 1.0), (37, 4, 0, EXTRA), (3, 9, 0, EXTRA)]


@pytest.mark.parametrize("tokens,heads,offset,extra", CASES)
def test_prepare_qk_is_bit_exact_in_both_layouts(dev, tokens, heads, offset, extra):
    import torch

    x, mean, stride = prepare_inputs(tokens, heads, offset)
    cap = -(-tokens // 256) * 256
    width = heads * 128
    want_hw, want_hs = O.prepare_qk(x, O.F16, mean, tokens, stride, offset, heads, extra, True, cap)
    want_tw, want_ts = O.prepare_qk(x, O.F16, mean, tokens, stride, offset, heads, extra)
    x_d, m_d = to_dev(x, dev), to_dev(mean, dev)
    cfg = H.PrepareCfg(stride, offset, heads, extra, cap, 1e-5, H.H3_ELEM_F16)
    for rep in range(4):
        codes = filled((cap * width,), 0x55, np.uint8, dev)
        scales = filled((cap * heads * 4,), 0x55, np.uint8, dev)
        H.prepare_qk_i8hm(cfg, tokens, x_d, m_d, codes, scales)
        tcodes = filled((tokens * width,), 0x55, np.uint8, dev)
        tscales = filled((tokens * heads * 4,), 0x55, np.uint8, dev)
        H.prepare_qk_i8(cfg, tokens, x_d, m_d, tcodes, tscales)
        torch.cuda.synchronize()
        hw = codes.cpu().numpy().view(np.int32).reshape(heads, cap, 32)
        hs = scales.cpu().numpy().view(np.float32).reshape(heads, cap)
        ref_hw = want_hw.reshape(heads, cap, 32)
        assert np.array_equal(hw[:, :tokens], ref_hw[:, :tokens]), f"codes rep {rep}"
        assert np.array_equal(hs[:, :tokens].view(np.uint32), want_hs[:, :tokens].view(np.uint32))
        # rows past tokens keep the poison: the kernel never writes them
        assert (codes.cpu().numpy().reshape(heads, cap, 128)[:, tokens:] == 0x55).all()
        assert np.array_equal(tcodes.cpu().numpy().view(np.int32).reshape(tokens, -1), want_tw)
        assert np.array_equal(tscales.cpu().numpy().view(np.uint32).reshape(tokens, heads),
                              want_ts.view(np.uint32))


def test_prepare_qk_against_reference_f64_oracle(dev):
    """tests/kernels.rs:1797-1810 directly on the GPU output."""
    import torch

    for tokens, heads in [(37, 4), (3, 9), (3, 56)]:
        x, mean, stride = prepare_inputs(tokens, heads, 0, stride_extra=0)
        if heads != 56:  # the reference test only writes f16::MAX into head 1 when heads == 56
            x = x.copy()
            x.view(np.float16)[:, 128:256] = O.values(tokens * stride, 0.7).astype(
                np.float16).reshape(tokens, stride)[:, 128:256]
        cfg = H.PrepareCfg(stride, 0, heads, EXTRA, 0, 1e-5, H.H3_ELEM_F16)
        codes = torch.zeros(tokens * heads * 32, dtype=torch.int32, device=dev)
        scales = torch.zeros(tokens * heads, dtype=torch.float32, device=dev)
        H.prepare_qk_i8(cfg, tokens, to_dev(x, dev), to_dev(mean, dev), codes, scales)
        torch.cuda.synchronize()
        want_w, want_s, _ = O.prepared_qk_f64(x, mean, tokens, heads, O.EXTRA_Q_F64)
        words = codes.cpu().numpy()
        differing = int((words != want_w.reshape(-1)).sum())
        assert differing * 500 < words.size
        np.testing.assert_allclose(scales.cpu().numpy().astype(np.float64),
                                   want_s.reshape(-1).astype(np.float64), rtol=1e-4, atol=1e-7)


def test_prepare_qk_bf16_input_is_bit_exact(dev):
    import torch

    tokens, heads = 129, 8
    rng = np.random.default_rng(12)
    f = rng.standard_normal((tokens, heads * 128)).astype(np.float32)
    f += rng.standard_normal(heads * 128).astype(np.float32) * np.float32(np.sqrt(2.0))
    x = O.bf16_bits(f)
    mean = O.colmean(x, O.BF16, tokens, heads * 128, heads * 128)
    cap = 256
    want_w, want_s = O.prepare_qk(x, O.BF16, mean, tokens, heads * 128, 0, heads, 1.0, True, cap)
    cfg = H.PrepareCfg(heads * 128, 0, heads, 1.0, cap, 1e-5, H.H3_ELEM_BF16)
    codes = torch.zeros(heads * cap * 32, dtype=torch.int32, device=dev)
    scales = torch.zeros(heads * cap, dtype=torch.float32, device=dev)
    m_d = torch.zeros(heads * 128, dtype=torch.float32, device=dev)
    x_d = to_dev(x, dev)
    H.colmean_f32(heads * 128, tokens, x_d, m_d, elem=H.H3_ELEM_BF16)
    H.prepare_qk_i8hm(cfg, tokens, x_d, m_d, codes, scales)
    torch.cuda.synchronize()
    assert np.array_equal(m_d.cpu().numpy().view(np.uint32), mean.view(np.uint32))
    assert np.array_equal(codes.cpu().numpy(), want_w.reshape(-1))
    assert np.array_equal(scales.cpu().numpy().view(np.uint32), want_s.reshape(-1).view(np.uint32))


@pytest.mark.parametrize("tokens,width", [(1, 256), (300, 256), (4097, 7168), (31104, 4096)])
def test_colmean_is_bit_exact(dev, tokens, width):
    import torch

    rng = np.random.default_rng(tokens)
    x = (rng.standard_normal((tokens, width), np.float32) + np.float32(1.5)).astype(np.float16)
    bits = np.ascontiguousarray(x).view(np.uint16)
    want = O.colmean(bits, O.F16, tokens, width, width)
    got = torch.zeros(width, dtype=torch.float32, device=dev)
    H.colmean_f32(width, tokens, to_dev(bits, dev), got)
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy().view(np.uint32), want.view(np.uint32))


def rope_case(tokens, heads, kv):
    stride = (heads + 2 * kv) * 128
    fused = O.f16_bits(O.values(tokens * stride, 0.7)).reshape(tokens, stride)
    qw = (1.0 + O.values(128, 0.1)).astype(np.float32)
    kw = (qw + np.float32(0.05)).astype(np.float32)
    angles = O.values(tokens * 48, 3.0)
    return fused, qw, kw, np.cos(angles).astype(np.float32), np.sin(angles).astype(np.float32), stride


@pytest.mark.parametrize("heads,kv", [(4, 2), (56, 56), (12, 3)])
def test_rope_qknorm_is_bit_exact_and_copies_v(dev, heads, kv):
    import torch

    tokens = 3
    fused, qw, kw, cos_t, sin_t, stride = rope_case(tokens, heads, kv)
    off = heads * 128
    want_q = O.rope_qknorm_f16(fused, O.F16, tokens, stride, 0, heads, qw, cos_t, sin_t, 1e-5)
    want_k = O.rope_qknorm_f16(fused, O.F16, tokens, stride, off, kv, kw, cos_t, sin_t, 1e-5)
    f_d = to_dev(fused, dev)
    args = [to_dev(a, dev) for a in (qw, kw, cos_t, sin_t)]
    q_out = torch.zeros(tokens * heads * 128, dtype=torch.int16, device=dev)
    k_out = torch.zeros(tokens * kv * 128, dtype=torch.int16, device=dev)
    v_out = torch.zeros(tokens * kv * 128, dtype=torch.int16, device=dev)
    cfg = H.RopeCfg(stride, heads, kv, off, 1e-5, 1, H.H3_ELEM_F16)
    H.rope_qknorm_f16(cfg, tokens, f_d, *args, q_out, k_out, v_out)
    torch.cuda.synchronize()
    assert np.array_equal(from_dev(q_out).reshape(tokens, -1), want_q)
    assert np.array_equal(from_dev(k_out).reshape(tokens, -1), want_k)
    assert np.array_equal(from_dev(v_out).reshape(tokens, -1), fused[:, off + kv * 128:])
    # copy_v = 0 leaves V alone and Q/K unchanged (tests/kernels.rs:1225-1240)
    v_poison = torch.full_like(v_out, 0x5555)
    q2, k2 = torch.full_like(q_out, -1), torch.full_like(k_out, -1)
    cfg.copy_v = 0
    H.rope_qknorm_f16(cfg, tokens, f_d, *args, q2, k2, v_poison)
    torch.cuda.synchronize()
    assert torch.equal(q2, q_out) and torch.equal(k2, k_out)
    assert (v_poison == 0x5555).all()
    # and the f64 RMSNorm+RoPE oracle, 2e-2 abs + 2e-2 rel
    want64 = O.rope_qknorm_f64(fused, O.F16, tokens, stride, 0, heads, qw, cos_t, sin_t, 1e-5)
    g = from_dev(q_out).view(np.float16).astype(np.float64).reshape(want64.shape)
    assert np.all(np.abs(g - want64) <= 2e-2 + 2e-2 * np.abs(want64))


@pytest.mark.parametrize("tokens,heads", [(3, 2), (129, 56), (257, 17), (4097, 56)])
def test_fused_operands_are_byte_identical_to_separate_preparation(dev, tokens, heads):
    """tests/kernels.rs:3153-3276, plus bit-exactness against the oracle."""
    import torch

    width = heads * 128
    cap = -(-tokens // 256) * 256
    fused = O.values(tokens * width * 3, 0.7).astype(np.float16).reshape(tokens, 3 * width)
    for off in (0, width):
        fused[:, off:off + 128] = 0
        fused[:, off + 128:off + 256] = np.float16(65504.0)
    fused = np.ascontiguousarray(fused).view(np.uint16)
    qw = (1.0 + O.values(128, 0.1)).astype(np.float32)
    kw = (qw + np.float32(0.05)).astype(np.float32)
    angles = O.values(tokens * 48, 3.0)
    cos_t, sin_t = np.cos(angles).astype(np.float32), np.sin(angles).astype(np.float32)
    f_d = to_dev(fused, dev)
    qw_d, kw_d, c_d, s_d = (to_dev(a, dev) for a in (qw, kw, cos_t, sin_t))
    split = [torch.zeros(tokens * width, dtype=torch.int16, device=dev) for _ in range(3)]
    H.rope_qknorm_f16(H.RopeCfg(3 * width, heads, heads, width, 1e-5, 1, H.H3_ELEM_F16), tokens,
                      f_d, qw_d, kw_d, c_d, s_d, *split)
    zero_mean = torch.zeros(width, dtype=torch.float32, device=dev)
    for i, (w_d, extra) in enumerate(((qw_d, EXTRA), (kw_d, 1.0))):
        cfg = H.PrepareCfg(width, 0, heads, extra, cap, 1e-5, H.H3_ELEM_F16)
        old_c = filled((cap * width,), 0x55, np.uint8, dev)
        old_s = filled((cap * heads * 4,), 0x55, np.uint8, dev)
        H.prepare_qk_i8hm(cfg, tokens, split[i], zero_mean, old_c, old_s)
        cfg.row_stride, cfg.head_offset = 3 * width, i * width
        for rep in range(8):
            new_c = filled((cap * width,), 0x55, np.uint8, dev)
            new_s = filled((cap * heads * 4,), 0x55, np.uint8, dev)
            H.prepare_qk_rope_i8hm(cfg, tokens, f_d, w_d, c_d, s_d, new_c, new_s)
            torch.cuda.synchronize()
            assert torch.equal(old_c, new_c), f"codes differ: tokens={tokens} head={i} rep={rep}"
            assert torch.equal(old_s, new_s), f"scales differ: tokens={tokens} head={i} rep={rep}"
        # against the oracle: RoPE (fixed fp32 order) then the quantizer
        roped = O.rope_qknorm_f16(fused, O.F16, tokens, 3 * width, i * width, heads,
                                  qw if i == 0 else kw, cos_t, sin_t, 1e-5)
        want_w, want_s = O.prepare_qk(roped, O.F16, None, tokens, width, 0, heads, extra, True, cap)
        got_w = new_c.cpu().numpy().view(np.int32).reshape(heads, cap, 32)[:, :tokens]
        assert np.array_equal(got_w, want_w.reshape(heads, cap, 32)[:, :tokens])
        got_s = new_s.cpu().numpy().view(np.uint32).reshape(heads, cap)[:, :tokens]
        assert np.array_equal(got_s, want_s.view(np.uint32)[:, :tokens])
    # V transpose: transpose_f16 of the split V == transpose_qkv_v_f16 of the fused rows
    tcfg = H.TransposeCfg(width, cap, H.H3_ELEM_F16)
    old = torch.zeros(cap * width, dtype=torch.int16, device=dev)
    new = torch.zeros(cap * width, dtype=torch.int16, device=dev)
    H.transpose_f16(tcfg, tokens, tokens, split[2], old)
    H.transpose_qkv_v_f16(tcfg, tokens, tokens, f_d, new)
    torch.cuda.synchronize()
    assert torch.equal(old, new)


@pytest.mark.parametrize("tokens,heads,bf16", [(1, 2, False), (257, 4, False), (383, 2, True),
                                               (384, 4, False), (385, 2, False), (769, 2, True),
                                               (4097, 8, False), (129024, 32, True)])
def test_fused_k_smoothing_is_byte_identical_to_the_separate_route(dev, tokens, heads, bf16):
    """This build's fused K-mean + RoPE + quantize == rope_qknorm_f16 -> colmean_f32 ->
    prepare_qk_i8hm(mean), the reference's smoothed route (src/stack.rs:1306-1326, 1727-1791).
    Lengths around the column-mean kernel's 384-token chunks, both input formats, and BASELINE
    config 3's K (129,024 tokens x 32 heads) at full size; the oracle composition is checked up
    to 4,097 tokens."""
    import torch

    print(f"fused K smoothing tokens={tokens} heads={heads} bf16={bf16}", flush=True)
    width = heads * 128
    cap = O.capacity(tokens)
    rng = np.random.default_rng(tokens)
    fmt, elem = (O.BF16, H.H3_ELEM_BF16) if bf16 else (O.F16, H.H3_ELEM_F16)
    kw = (1.0 + O.values(128, 0.1)).astype(np.float32)
    angles = rng.uniform(-3, 3, (tokens, 48)).astype(np.float32)
    cos_t, sin_t = np.cos(angles).astype(np.float32), np.sin(angles).astype(np.float32)
    kw_d, c_d, s_d = (to_dev(a, dev) for a in (kw, cos_t, sin_t))
    if tokens <= 4097:
        f = rng.standard_normal((tokens, 3 * width), np.float32)
        f[:, width:2 * width] += (rng.standard_normal(width).astype(np.float32)
                                  * np.float32(np.sqrt(2)))
        fused = O.bf16_bits(f) if bf16 else O.f16_bits(f)
        f_d = to_dev(fused, dev)
    else:  # full size: generated on the device (the oracle composition is not run)
        g = torch.Generator(device=dev)
        g.manual_seed(tokens)
        f = torch.randn((tokens, 3 * width), generator=g, device=dev)
        f[:, width:2 * width] += torch.randn((width,), generator=g, device=dev) * math.sqrt(2.0)
        f_d = f.to(torch.bfloat16 if bf16 else torch.float16).view(torch.int16)
        del f
    # separate route
    k_rot = torch.zeros(tokens * width, dtype=torch.int16, device=dev)
    q_rot = torch.zeros(tokens * width, dtype=torch.int16, device=dev)
    H.rope_qknorm_f16(H.RopeCfg(3 * width, heads, heads, width, 1e-5, 0, elem), tokens,
                      f_d, kw_d, kw_d, c_d, s_d, q_rot, k_rot, None)
    del q_rot
    mean_sep = torch.zeros(width, dtype=torch.float32, device=dev)
    H.colmean_f32(width, tokens, k_rot, mean_sep)
    cfg = H.PrepareCfg(width, 0, heads, 1.0, cap, 1e-5, H.H3_ELEM_F16)
    sep_c = torch.zeros(cap * width, dtype=torch.uint8, device=dev)
    sep_s = torch.zeros(cap * heads, dtype=torch.float32, device=dev)
    H.prepare_qk_i8hm(cfg, tokens, k_rot, mean_sep, sep_c, sep_s)
    # fused route
    cfg2 = H.PrepareCfg(3 * width, width, heads, 1.0, cap, 1e-5, elem)
    mean_f = torch.zeros(width, dtype=torch.float32, device=dev)
    fus_c = torch.zeros(cap * width, dtype=torch.uint8, device=dev)
    fus_s = torch.zeros(cap * heads, dtype=torch.float32, device=dev)
    H.prepare_k_rope_smooth_i8hm(cfg2, tokens, f_d, kw_d, c_d, s_d, mean_f, fus_c, fus_s)
    torch.cuda.synchronize()
    assert torch.equal(mean_sep.view(torch.int32), mean_f.view(torch.int32))
    assert torch.equal(sep_c, fus_c) and torch.equal(sep_s.view(torch.int32), fus_s.view(torch.int32))
    if tokens > 4097:
        return
    # and the oracle composition
    roped = O.rope_qknorm_f16(fused, fmt, tokens, 3 * width, width, heads, kw, cos_t, sin_t, 1e-5)
    mean = O.colmean(roped, O.F16, tokens, width, width)
    assert np.array_equal(mean_f.cpu().numpy().view(np.uint32), mean.view(np.uint32))
    want_w, _ = O.prepare_qk(roped, O.F16, mean, tokens, width, 0, heads, 1.0, True, cap)
    assert np.array_equal(fus_c.cpu().numpy().view(np.int32), want_w.reshape(-1))


@pytest.mark.parametrize("width", [32, 96, 256, 7168])
def test_transposed_values_clear_reused_capacity(dev, width):
    """tests/kernels.rs:3373-3444 (7168 on a subset of lengths)."""
    import torch

    token_list = [1, 31, 32, 33, 63, 64, 65, 129, 4096, 4097, 8193] if width <= 256 else [33, 4097]
    for tokens in token_list:
        for cap in (-(-tokens // 32) * 32, -(-(tokens + 32) // 256) * 256):
            out_bytes = cap * width * 2
            inp = (np.arange(tokens * width, dtype=np.uint64) * 37 % 65536).astype(np.uint16)
            inp = inp.reshape(tokens, width)
            base = np.concatenate([np.full(out_bytes, 0xFF, np.uint8), np.full(19, 0xA5, np.uint8)])
            cfg = H.TransposeCfg(width, cap, H.H3_ELEM_F16)
            a = to_dev(base, dev)
            H.transpose_f16(cfg, cap, tokens, to_dev(inp, dev), a[:out_bytes])
            fused = np.full((tokens, 3 * width), 0xFFFF, np.uint16)
            fused[:, 2 * width:] = inp
            b = to_dev(base, dev)
            H.transpose_qkv_v_f16(cfg, cap, tokens, to_dev(fused, dev), b[:out_bytes])
            torch.cuda.synchronize()
            a, b = a.cpu().numpy(), b.cpu().numpy()
            assert np.array_equal(a, b), "direct V transpose changed bits or padding"
            assert (a[out_bytes:] == 0xA5).all()
            want = np.zeros((width, cap), np.uint16)
            want[:, :tokens] = inp.T
            assert np.array_equal(a[:out_bytes].view(np.uint16).reshape(width, cap), want), (
                f"tokens={tokens} cap={cap}")


def test_transpose_bf16_rounds_to_f16(dev):
    import torch

    tokens, width, cap = 77, 256, 96
    rng = np.random.default_rng(8)
    f = rng.standard_normal((tokens, width)).astype(np.float32)
    bits = O.bf16_bits(f)
    want = O.transpose(bits, O.BF16, tokens, width, 0, width, cap, cap)
    out = torch.zeros(width * cap, dtype=torch.int16, device=dev)
    H.transpose_f16(H.TransposeCfg(width, cap, H.H3_ELEM_BF16), cap, tokens, to_dev(bits, dev), out)
    torch.cuda.synchronize()
    assert np.array_equal(from_dev(out).reshape(width, cap), want)


@pytest.mark.parametrize("elem", [H.H3_ELEM_F16, H.H3_ELEM_BF16])
def test_quantizers_on_non_finite_and_extreme_rows(dev, elem):
    """Rows holding NaN, +inf, -inf, the format's largest finite values, subnormals or zeros
    through every quantizer kernel (prepare_qk_i8, _i8hm, _i4, prepare_qk_rope_i8hm, with and
    without a mean), bit for bit against the oracle's fp32 restatement. The kernels form the
    code clamp(rne(p), +-127) as rne(clamp(p, +-127)) with a rounding add; for a NaN product
    both give -127 (the clamp's max returns the number), which these rows exercise."""
    import torch

    tokens, heads = 67, 3
    width = heads * 128
    stride = 3 * width
    fmt = O.F16 if elem == H.H3_ELEM_F16 else O.BF16
    big = 65504.0 if elem == H.H3_ELEM_F16 else 3.0e38
    rng = np.random.default_rng(21 + elem)
    f = rng.standard_normal((tokens, stride)).astype(np.float32)
    f[1, 5] = np.nan
    f[2, 130] = np.inf
    f[3, 300] = -np.inf
    f[4, :] = big
    f[5, 0:128] = -big
    f[6, :] = 0.0
    f[7, 128:256] = 1e-7  # subnormal in f16, tiny in bf16
    f[8, 7] = np.nan
    f[8, 9] = np.inf
    f[9, 256:384] = np.nan
    f[10, 128:256:2] = big
    x = O.f16_bits(f) if fmt == O.F16 else O.bf16_bits(f)
    x_d = to_dev(x, dev)
    mean = O.values(stride, 0.3)
    m_d = to_dev(mean, dev)
    cap = 96
    print(f"non-finite quantizer rows, elem={elem}", flush=True)
    for offset, m, m_host in ((0, None, None), (width, m_d, mean)):
        cfg = H.PrepareCfg(stride, offset, heads, EXTRA, cap, 1e-5, elem)
        want_hw, want_hs = O.prepare_qk(x, fmt, m_host, tokens, stride, offset, heads, EXTRA, True,
                                        cap)
        want_tw, want_ts = O.prepare_qk(x, fmt, m_host, tokens, stride, offset, heads, EXTRA)
        want_iw, want_is = O.prepare_qk_i4(x, fmt, m_host, tokens, stride, offset, heads, EXTRA)
        codes = filled((cap * width,), 0x55, np.uint8, dev)
        scales = filled((cap * heads * 4,), 0x55, np.uint8, dev)
        H.prepare_qk_i8hm(cfg, tokens, x_d, m, codes, scales)
        tcodes = torch.zeros(tokens * heads * 32, dtype=torch.int32, device=dev)
        tscales = torch.zeros(tokens * heads, dtype=torch.float32, device=dev)
        H.prepare_qk_i8(cfg, tokens, x_d, m, tcodes, tscales)
        icodes = torch.zeros(tokens * heads * 16, dtype=torch.int32, device=dev)
        iscales = torch.zeros(tokens * heads, dtype=torch.float32, device=dev)
        H.prepare_qk_i4(cfg, tokens, x_d, m, icodes, iscales)
        torch.cuda.synchronize()
        hw = codes.cpu().numpy().view(np.int32).reshape(heads, cap, 32)[:, :tokens]
        hs = scales.cpu().numpy().view(np.uint32).reshape(heads, cap)[:, :tokens]
        assert np.array_equal(hw, want_hw.reshape(heads, cap, 32)[:, :tokens]), offset
        assert np.array_equal(hs, want_hs.view(np.uint32)[:, :tokens]), offset
        assert np.array_equal(tcodes.cpu().numpy(), want_tw.reshape(-1)), offset
        assert np.array_equal(tscales.cpu().numpy().view(np.uint32), want_ts.view(np.uint32).reshape(-1))
        assert np.array_equal(icodes.cpu().numpy(), want_iw.reshape(-1)), offset
        assert np.array_equal(iscales.cpu().numpy().view(np.uint32), want_is.view(np.uint32).reshape(-1))
    # the RoPE quantizer: RMSNorm + RoPE of the same rows (their non-finite values spread over
    # the row through the norm), then the quantizer
    w = (1.0 + O.values(128, 0.1)).astype(np.float32)
    angles = O.values(tokens * 48, 3.0)
    cos_t, sin_t = np.cos(angles).astype(np.float32), np.sin(angles).astype(np.float32)
    for offset in (0, width):
        cfg = H.PrepareCfg(stride, offset, heads, EXTRA, cap, 1e-5, elem)
        roped = O.rope_qknorm_f16(x, fmt, tokens, stride, offset, heads, w, cos_t, sin_t, 1e-5)
        want_w, want_s = O.prepare_qk(roped, O.F16, None, tokens, width, 0, heads, EXTRA, True, cap)
        codes = filled((cap * width,), 0x55, np.uint8, dev)
        scales = filled((cap * heads * 4,), 0x55, np.uint8, dev)
        H.prepare_qk_rope_i8hm(cfg, tokens, x_d, to_dev(w, dev), to_dev(cos_t, dev),
                               to_dev(sin_t, dev), codes, scales)
        torch.cuda.synchronize()
        got_w = codes.cpu().numpy().view(np.int32).reshape(heads, cap, 32)[:, :tokens]
        got_s = scales.cpu().numpy().view(np.uint32).reshape(heads, cap)[:, :tokens]
        assert np.array_equal(got_w, want_w.reshape(heads, cap, 32)[:, :tokens]), offset
        assert np.array_equal(got_s, want_s.view(np.uint32)[:, :tokens]), offset
