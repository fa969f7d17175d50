"""INT8-QK attention kernels on the GPU against the f64 oracle of their operands.

Mirrors the reference's kernel tests:
  - int8_qk_attention_matches_the_attention_its_operands_define (tests/kernels.rs:1859-1990):
    token-major and head-major, tokens 23/64/97/129, 4 heads, full prepare pipeline from
    values() inputs; 2e-2 abs + 2e-2 rel, plus the north star's max-abs 2e-2 / mean-abs 2e-3;
  - check_head_major_attention (tests/kernels.rs:2013-2118): short sequences and partial tiles
    in full, long sequences on sampled query rows, a strong match in the final key tile, guard
    bytes past the output, three bit-identical replays; 1e-3 abs + 2e-3 rel.
All calls go through the C ABI (h3attn -> libh3attn.so).
"""
import math

import numpy as np
import pytest

import h3attn as H
import oracle as O
from helpers import filled, from_dev, head_major_operands, north_star_ok, pack_codes, to_dev

pytestmark = pytest.mark.gpu


def run_attention(dev, head_major, qw, qs, kw, ks, vt, tokens, cap, heads, token_count,
                  guard=0, repeats=1):
    import torch

    stride = heads * 128
    cfg = H.AttentionCfg(stride, stride, stride, tokens, cap, 1.0)
    qi_d, qs_d, ki_d, ks_d, vt_d = (to_dev(a, dev) for a in (qw, qs, kw, ks, vt))
    outs = []
    for _ in range(repeats):
        out = filled((token_count * stride * 2 + guard * 2,), 0xFF, np.uint8, dev)
        body = out[: token_count * stride * 2]
        fn = H.attention_i8qkhm if head_major else H.attention_i8qk
        fn(cfg, token_count, heads, qi_d, qs_d, ki_d, ks_d, vt_d, body)
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
    return outs


@pytest.mark.parametrize("head_major", [False, True])
@pytest.mark.parametrize("tokens", [23, 64, 97, 129])
def test_int8_attention_matches_the_attention_its_operands_define(dev, head_major, tokens):
    heads, d = 4, 128
    stride = heads * d
    waves = 8 if head_major else 4
    block = 16 * waves
    cap = max(-(-(tokens + 16) // 32) * 32, -(-tokens // block) * block)
    q = O.f16_bits(O.values(tokens * stride, 0.7)).reshape(tokens, stride)
    k = O.f16_bits(O.values(tokens * stride, 0.65)).reshape(tokens, stride)
    v = O.f16_bits(O.values(tokens * stride, 0.5)).reshape(tokens, stride)
    extra = O.config_f32(O.EXTRA_Q_F64)
    kmean = O.colmean(k, O.F16, tokens, stride, stride)
    # operands from the bit-exact quantizer restatement, laid out as the kernel reads them
    qw, qsc = O.prepare_qk(q, O.F16, None, tokens, stride, 0, heads, extra, head_major, cap)
    kw, ksc = O.prepare_qk(k, O.F16, kmean, tokens, stride, 0, heads, 1.0, head_major, cap)
    if not head_major:  # token-major, padded to capacity
        qw = np.vstack([qw, np.zeros((cap - tokens, stride // 4), np.int32)])
        kw = np.vstack([kw, np.zeros((cap - tokens, stride // 4), np.int32)])
        qsc = np.vstack([qsc, np.zeros((cap - tokens, heads), np.float32)])
        ksc = np.vstack([ksc, np.zeros((cap - tokens, heads), np.float32)])
    vt = O.transpose(v, O.F16, tokens, stride, 0, stride, cap, cap)
    got = run_attention(dev, head_major, qw, qsc, kw, ksc, vt, tokens, cap, heads, tokens)[0]
    got = got.view(np.float16).astype(np.float64).reshape(tokens, heads, d)
    # f64 oracle on head-major unpacked codes
    if head_major:
        qc = O.unpack(qw).reshape(heads, cap, 128)
        kc = O.unpack(kw).reshape(heads, cap, 128)
        qs_h, ks_h = qsc, ksc
    else:
        qc = O.unpack(qw).reshape(cap, heads, 128).transpose(1, 0, 2).copy()
        kc = O.unpack(kw).reshape(cap, heads, 128).transpose(1, 0, 2).copy()
        qs_h, ks_h = qsc.T.copy(), ksc.T.copy()
    want = O.attention_f64(qc, qs_h, kc, ks_h, vt, tokens, cap, heads, np.arange(tokens))
    assert np.all(np.isfinite(got))
    assert np.all(np.abs(got - want) <= 2e-2 + 2e-2 * np.abs(want))
    mx, mean = north_star_ok(got, want)
    assert mx <= 2e-2 and mean <= 2e-3, (mx, mean)


def check_head_major(dev, token_counts, query_limit, heads=3, seed_base=0):
    d = 128
    stride = heads * d
    for tokens in token_counts:
        queries = query_limit if tokens > 65536 else tokens
        cap = -(-(tokens + 16) // 256) * 256
        rng = np.random.default_rng(seed_base + tokens)
        qc, qs, kc, ks, vt = head_major_operands(rng, heads, tokens, cap)
        print(f"head-major attention tokens={tokens} queries={queries}", flush=True)
        outs = run_attention(dev, True, pack_codes(qc).reshape(heads * cap, 32), qs,
                             pack_codes(kc).reshape(heads * cap, 32), ks, vt, tokens, cap, heads,
                             queries, guard=19, repeats=3)
        body = queries * stride * 2
        for o in outs:
            assert (o[body:] == 0xFF).all(), f"attention wrote past the output at {tokens} tokens"
            assert np.array_equal(o, outs[0]), f"unstable attention at {tokens} tokens"
        got = outs[0][:body].view(np.float16).astype(np.float64).reshape(queries, heads, d)
        assert np.all(np.isfinite(got)), f"tokens={tokens}"
        rows = sorted({r for r in (0, 15, 16, 31, 63, 64, 127, 128, 4095, queries - 1)
                       if r < queries})
        want = O.attention_f64(qc, qs, kc, ks, vt, tokens, cap, heads, np.array(rows, np.int32))
        for i, r in enumerate(rows):
            err = np.abs(got[r] - want[i])
            bad = err > 1e-3 + 2e-3 * np.abs(want[i])
            assert not bad.any(), (tokens, r, float(err.max()))


def test_head_major_attention_handles_short_sequences_and_partial_tiles(dev):
    check_head_major(dev, [1, 63, 64, 65, 127, 128, 129, 255, 256, 257, 1024, 1025, 2048, 2049,
                           4095], 1 << 30)


def test_head_major_attention_handles_long_reference_sequences(dev):
    """head_major_int8_attention_handles_long_reference_sequences (tests/kernels.rs:1994-1996):
    the same lengths, 478,340 included, 129 query rows; 65,537 again with 127."""
    check_head_major(dev, [4096, 4097, 8193, 65537, 119585, 478340], 129)
    check_head_major(dev, [65537], 127, seed_base=1)


def test_head_major_attention_at_the_qualified_maximum_length(dev):
    """tests/compiler.rs:34-45 qualifies the head-major kernel at 1,048,544 tokens (capacity
    1,048,576, the largest the config allows): one head, 129 query rows over every key, guard
    bytes and three bit-identical runs as check_head_major_attention."""
    check_head_major(dev, [1048544], 129, heads=1)


def test_token_count_below_tokens_writes_only_those_rows(dev):
    """The long-sequence form of the reference test: token_count (rows written) < tokens."""
    heads, tokens = 2, 3000
    cap = -(-(tokens + 16) // 256) * 256
    rng = np.random.default_rng(9)
    qc, qs, kc, ks, vt = head_major_operands(rng, heads, tokens, cap)
    q_rows = 200
    outs = run_attention(dev, True, pack_codes(qc).reshape(heads * cap, 32), qs,
                         pack_codes(kc).reshape(heads * cap, 32), ks, vt, tokens, cap, heads,
                         q_rows, guard=64)
    body = q_rows * heads * 128 * 2
    assert (outs[0][body:] == 0xFF).all()
    got = outs[0][:body].view(np.float16).astype(np.float64).reshape(q_rows, heads, 128)
    rows = np.array([0, 99, 199], np.int32)
    want = O.attention_f64(qc, qs, kc, ks, vt, tokens, cap, heads, rows)
    assert np.all(np.abs(got[rows] - want) <= 1e-3 + 2e-3 * np.abs(want))


@pytest.mark.parametrize("tokens,heads", [(31104, 32), (129024, 32), (130272, 32)])
def test_baseline_shapes_on_sampled_rows(dev, tokens, heads):
    """BASELINE configs 2, 3 and 4 (the joint 129,024 + 1,248-token sequence) at full size: every
    query row is computed by the kernel, a
    sample of rows (first, last, tile edges, random) is checked against the f64 oracle to the
    north star's tolerance."""
    import torch

    cap = O.capacity(tokens)
    rng = np.random.default_rng(tokens)
    qc, qs, kc, ks, vt = head_major_operands(rng, heads, tokens, cap, late_match=False)
    stride = heads * 128
    cfg = H.AttentionCfg(stride, stride, stride, tokens, cap, 1.0)
    out = torch.empty((tokens, stride), dtype=torch.float16, device=dev)
    print(f"attention at S={tokens} H={heads}", flush=True)
    H.attention_i8qkhm(cfg, tokens, heads, to_dev(pack_codes(qc).reshape(heads * cap, 32), dev),
                       to_dev(qs, dev), to_dev(pack_codes(kc).reshape(heads * cap, 32), dev),
                       to_dev(ks, dev), to_dev(vt, dev), out)
    torch.cuda.synchronize()
    got = from_dev(out).view(np.float16).astype(np.float64).reshape(tokens, heads, 128)
    rows = np.unique(np.concatenate([[0, 31, 32, 127, 128, tokens - 1],
                                     rng.integers(0, tokens, 10)])).astype(np.int32)
    want = O.attention_f64(qc, qs, kc, ks, vt, tokens, cap, heads, rows)
    mx, mean = north_star_ok(got[rows], want)
    assert mx <= 2e-2 and mean <= 2e-3, (mx, mean)
    assert np.all(np.isfinite(got))


@pytest.mark.parametrize("head_major", [True, False])
@pytest.mark.parametrize("flat", ["exact", "near"])
def test_row_sum_error_is_bounded_on_long_flat_rows_with_large_values(dev, flat, head_major):
    """The output is O / l with both O (the PV accumulators) and the row sum l built from the
    same f16-rounded probabilities p~ = p(1 + d), |d| <= 2^-11, summed in f32. It is therefore
    the exact weighted mean of V under the weights p~ / sum p~, each within a relative
    2^-10 / (1 - 2^-11) of the exact softmax weight, so |out - exact| <= ~2^-10 max|V| plus f32
    accumulation and the f16 output rounding. Long rows (BASELINE config 3's 129,024 keys) with
    |V| up to ~1,500 and either exactly flat scores (every p = 1, out = mean of V) or nearly
    flat ones (every p a distinct value near 1, each rounded) check that bound at scale.
    Both layouts run the head-major kernel (the token-major one through its row strides), so
    both take the same bound."""
    import torch

    heads, tokens = 2, 129024
    cap = O.capacity(tokens)
    rng = np.random.default_rng(77 if flat == "near" else 78)
    qc, qs, kc, ks, vt = head_major_operands(rng, heads, tokens, cap, late_match=False)
    if flat == "exact":
        qc[:] = 0
    else:
        qs[:, :tokens] = np.float32(1.0 / 2048.0)
    vt = (rng.standard_normal((heads * 128, cap), np.float32) * 300.0).astype(np.float16)
    vt[:, tokens:] = 0
    vmax = float(np.abs(vt.astype(np.float64)).max())
    vt = vt.view(np.uint16)
    stride = heads * 128
    cfg = H.AttentionCfg(stride, stride, stride, tokens, cap, 1.0)
    out = torch.empty((tokens, stride), dtype=torch.float16, device=dev)
    print(f"row-sum bound, {flat} flat rows, S={tokens} H={heads} head_major={head_major}",
          flush=True)
    if head_major:
        H.attention_i8qkhm(cfg, tokens, heads,
                           to_dev(pack_codes(qc).reshape(heads * cap, 32), dev), to_dev(qs, dev),
                           to_dev(pack_codes(kc).reshape(heads * cap, 32), dev), to_dev(ks, dev),
                           to_dev(vt, dev), out)
    else:  # the same operands in the token-major layout: [cap][heads] rows of codes and scales
        tm = lambda c: pack_codes(c.transpose(1, 0, 2)).reshape(cap, heads * 32)
        H.attention_i8qk(cfg, tokens, heads, to_dev(tm(qc), dev), to_dev(qs.T.copy(), dev),
                         to_dev(tm(kc), dev), to_dev(ks.T.copy(), dev), to_dev(vt, dev), out)
    torch.cuda.synchronize()
    got = from_dev(out).view(np.float16).astype(np.float64).reshape(tokens, heads, 128)
    rows = np.unique(np.concatenate([[0, 31, 32, 255, 256, tokens - 1],
                                     rng.integers(0, tokens, 6)])).astype(np.int32)
    want = O.attention_f64(qc, qs, kc, ks, vt, tokens, cap, heads, rows)
    if flat == "exact":  # closed form: every key weighs the same
        mean_v = vt[:, :tokens].view(np.float16).astype(np.float64).mean(1).reshape(heads, 128)
        assert np.allclose(want, mean_v[None], rtol=0, atol=1e-9 * vmax)
    err = np.abs(got[rows] - want)
    rel = 2.0 ** -10 + 2.0 ** -12
    bound = rel * vmax + 2.0 ** -11 * np.abs(want)
    assert np.all(err <= bound), (flat, float(err.max()), vmax)
    assert float(err.mean()) <= 5e-5 * vmax, (flat, float(err.mean()), vmax)
    assert np.all(np.isfinite(got))


@pytest.mark.parametrize("tokens,q_heads,kv_heads,pad", [(1025, 3, 3, 0), (4096, 4, 2, 128),
                                                         (4097, 2, 2, 0), (9000, 2, 1, 128)])
def test_token_major_layout_gives_the_head_major_bits(dev, tokens, q_heads, kv_heads, pad):
    """h3_attention_i8qk runs the head-major kernel with row strides (K and Q rows kv_stride and
    q_stride bytes apart, key scales [token][kv heads], query scales [token][q_stride/128]): on
    the same operands laid out both ways, its output equals h3_attention_i8qkhm's bit for bit.
    Short and long sequences (the head-major entry chains blocks up to 4,096 keys, the
    token-major one never does), GQA head wrap (kv_stride < q_stride) and a padded output pitch
    whose pad columns stay untouched; sampled rows against the f64 oracle at 1e-3 + 2e-3 rel."""
    import torch

    cap = O.capacity(tokens)
    rng = np.random.default_rng(tokens + 17 * q_heads)
    qc, qs, _, _, _ = head_major_operands(rng, q_heads, tokens, cap, late_match=False)
    _, _, kc, ks, vt = head_major_operands(rng, kv_heads, tokens, cap, late_match=False)
    kc[:, tokens - 1] = qc[:kv_heads, 31]  # a strong match in the last key tile
    q_stride, kv_stride, out_stride = q_heads * 128, kv_heads * 128, q_heads * 128 + pad
    cfg = H.AttentionCfg(q_stride, kv_stride, out_stride, tokens, cap, 1.0)
    hm = [to_dev(pack_codes(qc).reshape(q_heads * cap, 32), dev), to_dev(qs, dev),
          to_dev(pack_codes(kc).reshape(kv_heads * cap, 32), dev), to_dev(ks, dev)]
    tm = [to_dev(pack_codes(qc.transpose(1, 0, 2)).reshape(cap, q_heads * 32), dev),
          to_dev(qs.T.copy(), dev),
          to_dev(pack_codes(kc.transpose(1, 0, 2)).reshape(cap, kv_heads * 32), dev),
          to_dev(ks.T.copy(), dev)]
    vt_d = to_dev(vt, dev)
    nbytes = tokens * out_stride * 2
    outs = []
    print(f"token-major vs head-major: S={tokens} heads={q_heads}/{kv_heads} pad={pad}", flush=True)
    for fn, ops in ((H.attention_i8qkhm, hm), (H.attention_i8qk, tm)):
        out = filled((nbytes,), 0xA5, np.uint8, dev)
        fn(cfg, tokens, q_heads, *ops, vt_d, out)
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
    assert np.array_equal(outs[0], outs[1]), "token-major and head-major outputs differ"
    # the reference's head wrap: workload row h reads key/value head h mod kv and query and
    # output head h mod min(kv, out_stride/128), so only the first kv output heads are written
    touched = min(kv_heads, out_stride // 128)
    rows_out = outs[1].view(np.uint16).reshape(tokens, out_stride)
    assert (rows_out[:, touched * 128:] == 0xA5A5).all(), "untouched heads or pad columns written"
    got = rows_out[:, :touched * 128].reshape(tokens, touched, 128)
    rows = np.unique(np.concatenate([[0, 31, 255, 256, tokens - 1],
                                     rng.integers(0, tokens, 5)])).astype(np.int32)
    want = O.attention_f64(qc[:touched], qs[:touched], kc[:touched], ks[:touched],
                           vt.reshape(kv_heads, 128, cap)[:touched].reshape(touched * 128, cap),
                           tokens, cap, touched, rows)
    err = np.abs(got[rows].view(np.float16).astype(np.float64) - want)
    assert np.all(err <= 1e-3 + 2e-3 * np.abs(want)), float(err.max())
