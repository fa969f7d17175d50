/*
 * h3oracle — CPU restatement of h3-hrx's INT8 (SageAttention-style) attention path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the shipped library links, loads or calls this code.
 * It is the checker for the HIP kernels (tests/, __graft_entry__.smoke()) and the timed CPU
 * baseline in bench.py. Every function cites the reference file:line it restates
 * (paths relative to the zacharydenton/h3-hrx source tree).
 *
 * Pinning status (what checks each function, besides the HIP kernels it judges):
 *   h3o_prepare_qk_f32      fp32 op-order restatement of kernels/prepare_qk_i8.loom:63-188.
 *                           Pinned by the reference's own f64 oracle (tests/kernels.rs:1704-1741)
 *                           on its closed-form inputs: codes may differ only at rounding ties
 *                           (< 1/500 words, tests/kernels.rs:1797-1802), scales within
 *                           1e-7 + 1e-4 rel (1803-1810); by the zero-head and f16::MAX-head
 *                           special cases; by exactness of the butterfly against the dense
 *                           Sylvester product where fp32 sums are exact; and by an independent
 *                           numpy restatement (tests/test_oracle.py).
 *   h3o_prepared_qk_f64     restatement of the reference test oracle tests/kernels.rs:1704-1741.
 *   h3o_prepare_qk_i4_f32   kernels/prepare_qk_i4.loom:73-214: the pinned H_128 above with
 *                           amax/7 scales and nibble packing. The reference holds no int4
 *                           quantizer test; pinned by known answers (a one-hot row gives +-7
 *                           in the Sylvester sign pattern, packed low nibble first as the
 *                           reference's own attention test packs codes, tests/kernels.rs:2366-
 *                           2375), by an independent numpy quantisation of the pinned rotation,
 *                           and by consistency with the int8 quantizer's rotation.
 *   h3o_colmean_f32         kernels/colmean_f32.loom (in-file 30-40): sequential fp32 sum.
 *                           Pinned by exact integer-valued sums and by numpy cumulative float32.
 *   h3o_rope_qknorm_f16     this build's RMSNorm + rotate-half RoPE in a fixed fp32 order
 *                           (kernels/prepare_qk_rope_i8hm.loom:110-130 defines the maths; its
 *                           reduction order and rsqrt are not pinned by the reference). Pinned
 *                           to the reference's f64 oracle (tests/kernels.rs:1146-1180) within
 *                           2e-2 abs + 2e-2 rel, and by the identity-rotation special case.
 *   h3o_transpose_f16       kernels/transpose_f16.loom: bit permutation plus zero tail.
 *   h3o_gemm_i8_qkv         the compact INT8 QKV projection, kernels/gemm_packed_256.loom:
 *                           14-412 as h3_gemm_i8_qkv_256 (3429-3471), in the scalar form of the
 *                           reference test tests/kernels.rs:4392-4460. Pinned by that test's
 *                           closed-form inputs and assertions (non-finite weight scales, a 100x
 *                           scale that saturates to 65472, zero V padding), by exact int64 dot
 *                           products, and by an independent numpy restatement (float32 ops,
 *                           astype(float16)) in tests/test_oracle_gemm.py.
 *   h3o_prepare_plain_i8    the GEMM-operand quantizer prepare_plain_i8 / prepare_plain_f32_i8
 *                           (kernels/prepare_i8_family.loom:4-72, 80-193, 200-294, 598-689):
 *                           per 256-group, four radix-4 stages (strides 1, 4, 16, 64) in the
 *                           reference's fp32 operation order, absmax with non-finite -> inf,
 *                           s = max(amax/16, 1e-30)/127, q = clamp(rne(x*(1/16)/s)). Pinned by
 *                           the reference test f32_preparation_matches_dense_hadamard_and_marks_
 *                           invalid_rows (tests/kernels.rs:4587-4760: codes within 1 of the
 *                           dense product, scale within 0.01, non-finite rows -> zero codes and
 *                           a non-finite scale) on its inputs, by exactness against the dense
 *                           Kronecker product on integer inputs whose sums are exact in fp32,
 *                           and by an independent numpy restatement. The rounding order of the
 *                           butterflies follows the .loom text; no reference vector pins it
 *                           beyond those checks.
 *   h3o_vsa_*               the VSA path (h3oracle_vsa.c): the cube plan and top-k budget of
 *                           src/vsa.rs:54-143 and the vsa_ops / vsa_kmean kernels as literal
 *                           restatements (route by the reference's rank count). Pinned by the
 *                           reference's own tests: the plan tests of src/vsa.rs:145-225 (prefix
 *                           tiles [64, 1, 6], bijection, prefix rows first), its budget cases
 *                           topk(25) = 2, topk(35) = 4, topk(1) = 0 and its sigma-window cases,
 *                           and the independent masked oracle of src/vsa/device.rs:513-620
 *                           (f32 block means, scores, a sort-based top-k threshold, the neighbour
 *                           and prefix rule, all-tie rows keeping every block), restated in numpy
 *                           in tests/test_oracle_vsa.py; by brute-force closed forms (integer
 *                           means, one-hot scores) and planted mistakes. h3o_vsa_coarse_f64 and
 *                           h3o_vsa_attention_f64 are exact-arithmetic statements of what the
 *                           reference approximates (expf<afn>, f16 probabilities): pinned by
 *                           closed forms (uniform scores give the mean of the routed values, a
 *                           route to one block gives that block's attention) and by the dense
 *                           h3o_attention_f64 when every block is routed.
 *   h3o_cross_attention_f64 the cross-attention extension (grouped heads, key mask): the formula
 *                           of h3o_attention_f64 over the attended keys. Pinned by equality with
 *                           h3o_attention_f64 when queries and keys are one sequence, the heads
 *                           are not grouped and no key is masked; by the mean of the attended V
 *                           rows for uniform scores; and by brute-force numpy on small shapes.
 *   h3o_attention_f64       the attention the operands define, tests/kernels.rs:1891-1913 and
 *                           2084-2111: softmax_j(sum(qc*kc) * qs * ks) . V in f64. Pinned by
 *                           closed forms: uniform keys give the mean of V, a single dominant key
 *                           returns its V row, and brute-force numpy on small shapes.
 */
#ifndef H3ORACLE_H
#define H3ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element formats of activations: raw 16-bit patterns */
enum { H3O_F16 = 0, H3O_BF16 = 1 };

float h3o_half_to_float(uint16_t h);
uint16_t h3o_float_to_half(float f); /* IEEE binary16, round to nearest even */
float h3o_bf16_to_float(uint16_t h);

/* %.17g spelling of a double parsed back as f32, as compile::num + the Loom config parse do
 * (src/compile.rs:38-83). */
float h3o_config_f32(double v);

/* Quantizer, bit-exact fp32 order of kernels/prepare_qk_i8.loom:63-188.
 *   x      [tokens][row_stride] 16-bit elements (fmt H3O_F16 or H3O_BF16)
 *   mean   [row_stride] f32 (may be NULL: zero mean)
 *   head_major == 0: codes [tokens][heads*32] i32, scales [tokens][heads]
 *   head_major != 0: codes [heads*capacity][32] i32, scales [heads][capacity]
 * Rows >= tokens are not written. */
void h3o_prepare_qk_f32(const uint16_t *x, int fmt, const float *mean, int tokens, int row_stride,
                        int head_offset, int heads, float extra, int head_major, int capacity,
                        int32_t *codes, float *scales);

/* int4 quantizer (kernels/prepare_qk_i4.loom:73-214), token-major: codes [tokens][heads*16]
 * i32 (eight 4-bit codes per word, low nibble first), scales [tokens][heads] = amax/7 * extra. */
void h3o_prepare_qk_i4_f32(const uint16_t *x, int fmt, const float *mean, int tokens,
                           int row_stride, int head_offset, int heads, float extra,
                           int32_t *codes, float *scales);
void h3o_quantize_row_i4(const float *y, float extra, int32_t *words, float *scale);

/* One head row: y[128] f32 (already mean-subtracted) -> 32 packed words + scale. */
void h3o_quantize_row(const float *y, float extra, int32_t *words, float *scale);

/* Unnormalised Sylvester H_128 in the reference's fp32 butterfly order. */
void h3o_hadamard128_f32(const float *y, float *r);

/* The reference test oracle tests/kernels.rs:1704-1741 (f64, ties away from zero).
 * x f16 [tokens][heads*128], mean [heads*128]; codes_out f64 [tokens][heads*128] (may be NULL). */
void h3o_prepared_qk_f64(const uint16_t *x, const float *mean, int tokens, int heads, double extra,
                         int32_t *words, float *scales, double *codes_out);

/* kernels/colmean_f32.loom: mean[c] = (sum_t f32(x[t][c])) / f32(tokens), sequential. */
void h3o_colmean_f32(const uint16_t *x, int fmt, int tokens, int width, int row_stride,
                     float *mean);

/* RMSNorm(weight, eps) + rotate-half RoPE on channels < 96 (pairs c <-> c+48), rounded to f16.
 * x [tokens][row_stride] (heads x 128 at head_offset), weight[128], cos/sin [tokens][48].
 * out f16 bits [tokens][out_stride] at column h*128. Fixed fp32 order of this build's kernel. */
void h3o_rope_qknorm_f16(const uint16_t *x, int fmt, int tokens, int row_stride, int head_offset,
                         int heads, const float *weight, const float *cos_t, const float *sin_t,
                         float eps, uint16_t *out, int out_stride);
void h3o_rope_qknorm_f16_ulps(const uint16_t *x, int fmt, int tokens, int row_stride,
                              int head_offset, int heads, const float *weight, const float *cos_t,
                              const float *sin_t, float eps, uint16_t *out, int out_stride,
                              int r_ulps);

/* The reference's f64 RMSNorm+RoPE oracle (tests/kernels.rs:1146-1180), f64 out. */
void h3o_rope_qknorm_f64(const uint16_t *x, int fmt, int tokens, int row_stride, int head_offset,
                         int heads, const float *weight, const float *cos_t, const float *sin_t,
                         double eps, double *out);

/* V transpose: x [rows][row_stride] (width columns at col_offset) -> out [width][capacity],
 * columns [rows, clear_to) zeroed, columns >= clear_to untouched. bf16 input is rounded to f16. */
void h3o_transpose_f16(const uint16_t *x, int fmt, int rows, int row_stride, int col_offset,
                       int width, int capacity, int clear_to, uint16_t *out);

/* Attention of the operands, f64 (tests/kernels.rs:1891-1913, 2084-2111).
 *   codes  int8 [heads][capacity][128] (head-major, unpacked) for q and k
 *   qs, ks [heads][capacity]; vt f16 [heads*128][capacity]
 *   rows: the query rows to evaluate (n_rows of them); out f64 [n_rows][heads][128]
 * threads: OpenMP threads (<= 0: all). Returns 0. */
int h3o_attention_f64(const int8_t *qc, const float *qs, const int8_t *kc, const float *ks,
                      const uint16_t *vt, int tokens, int capacity, int heads, const int *rows,
                      int n_rows, double *out, int threads);

/* Unpack codes: head-major packed words [heads*capacity][32] -> int8 [heads*capacity][128]. */
void h3o_unpack_codes(const int32_t *words, size_t n_rows, int8_t *codes);

/* CPU baseline: the reference's CPU path for one call on sampled query rows — f64 prepared_qk
 * of Q (rows sampled) and K (all tokens), then f64 attention of those operands. Returns the
 * seconds of the per-row part; *fixed_seconds gets the per-call part. threads as above. */
double h3o_cpu_baseline(const uint16_t *q, const uint16_t *k, const uint16_t *v, int tokens,
                        int heads, const int *rows, int n_rows, int threads, double *out,
                        double *fixed_seconds);

/* Compact INT8 QKV projection (kernels/gemm_packed_256.loom:14-412, 3429-3471;
 * tests/kernels.rs:4392-4460): a [m][k_stride] int8, w [n][k_stride] int8 (first k bytes of each
 * row used), ws [n], as [m] f32; out f16 bits, m*n + (cap-m)*n/3 elements, cap = ceil(m/256)*256:
 * Q/K rows [m][2n/3], then V^T [n/3][cap] with zero columns m..cap-1.
 * threads: OpenMP threads (<= 0: all). */
void h3o_gemm_i8_qkv(const int8_t *a, const int8_t *w, const float *ws, const float *as, int m,
                     int n, int k, int k_stride, uint16_t *out, int threads);

/* prepare_plain_i8 (fmt H3O_F16 / H3O_BF16, 16-bit x) and prepare_plain_f32_i8 (fmt 2, f32 x):
 * x [tokens][width]; codes int8 [tokens][out_stride] (first width bytes written); scales
 * [tokens] f32. */
void h3o_prepare_plain_i8(const void *x, int fmt, int tokens, int width, int out_stride,
                          int8_t *codes, float *scales);

/* Cross-attention with grouped heads and a key mask (this build's extension), f64. */
int h3o_cross_attention_f64(const int8_t *qc, const float *qs, const int8_t *kc, const float *ks,
                            const uint16_t *vt, const uint8_t *mask, int q_cap, int kv_tokens,
                            int kv_cap, int qh, int kh, const int *rows, int n_rows, double *out,
                            int threads);

/* ---- VSA (h3oracle_vsa.c; src/vsa.rs, kernels/vsa_ops.loom, vsa_kmean.loom, vsa_attention_8) */
/* Blocks of the plan: 64-row tiles of each prefix segment plus 4x4x4 video cubes. */
int h3o_vsa_plan_blocks(const int *seg_rows, int n_segs, int nt, int nh, int nw);
/* src/vsa.rs:94-143. segments (row0, rows) in order; video cells (t, h, w) at rows
 * seq_len - nt*nh*nw + (t*nh + h)*nw + w. src [64*blocks], inverse [seq_len], lengths [blocks].
 * Returns the block count, or -1 when some row is not covered. */
int h3o_vsa_plan(const int *seg_row0, const int *seg_rows, int n_segs, int seq_len, int nt,
                 int nh, int nw, int32_t *src, int32_t *inverse, int32_t *lengths,
                 int *prefix_blocks);
int h3o_vsa_topk(double keep_percent, int nonprefix);
int h3o_vsa_dense_reason(double start, double end, long min_tokens, long tokens, float sigma,
                         double shift);
void h3o_vsa_gather(const int32_t *src, int padded, int tokens, int width, const uint16_t *x,
                    uint16_t *y);
void h3o_vsa_scatter(const int32_t *inverse, int tokens, int width, const uint16_t *x,
                     uint16_t *y);
void h3o_vsa_pool(const int32_t *lengths, int blocks, int width, const uint16_t *x,
                  float *means);
void h3o_vsa_scores(const float *qm, const float *km, int blocks, int heads, float *scores);
void h3o_vsa_route(const float *scores, int blocks, int heads, int prefix, int topk,
                   int32_t *routes);
void h3o_vsa_coarse_f64(const float *scores, const float *vm, int blocks, int heads,
                        double *coarse);
void h3o_vsa_gated_scatter(const int32_t *inverse, int tokens, int width, const uint16_t *fine,
                           const uint16_t *gate, const float *coarse, uint16_t *out);
void h3o_vsa_kmean(const float *x, int tokens, int width, float *mean);
int h3o_vsa_attention_f64(const int8_t *qc, const float *qs, const int8_t *kc, const float *ks,
                          const uint16_t *vt, int tokens, int capacity, int heads,
                          const int32_t *routes, const int32_t *lengths, const int *rows,
                          int n_rows, double *out, int threads);
/* kernels/vsa_attention_16.loom in f64: f16 q, k, v token-major [capacity][heads*128], logits
 * (q . k) * scale, natural softmax over the kept cubes' live keys. */
int h3o_vsa_attention_f16_f64(const uint16_t *q, const uint16_t *k, const uint16_t *v, int tokens,
                              int heads, double scale, const int32_t *routes,
                              const int32_t *lengths, const int *rows, int n_rows, double *out,
                              int threads);

int h3o_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
