/*
 * h3attn.h — C ABI of libh3attn: the MI355X (gfx950) INT8 attention path of h3-hrx.
 *
 * Each entry point replaces one reference kernel launch made through
 * `dispatch::emit(sink, kernel, profile, stage, workload, scalars, bindings, required)`
 * (reference src/dispatch.rs:254-316) on a kernel obtained from `Compiler::get`
 * (src/compile.rs:320-326). A reference launch carries
 *   - the kernel's config map (src/compile.rs:19-22)  -> the cfg struct of each entry point,
 *   - the workload and device scalars                  -> the uint32_t arguments,
 *   - bindings (buffer views) with required lengths    -> h3_view {pointer, bytes} arguments.
 *
 * Conventions, all mirroring the reference's contract:
 *   - Pointers are device pointers. The library never allocates and never synchronises: work
 *     is enqueued on `stream` in order (src/dispatch.rs:86-133) and may be captured in a graph.
 *   - Before any launch every binding's byte length is checked against the extent the kernel
 *     addresses; a short binding returns H3_ERR_BINDING and launches nothing
 *     (src/dispatch.rs:264-276). h3_last_error() then reads
 *     "{stage}: binding {i} is {n} bytes, the kernel addresses {need}".
 *   - Config values outside the ranges the reference declares (`config.decl ... where [...]`
 *     in each kernel .loom file) return H3_ERR_CONFIG and launch nothing.
 *   - Activations are 16-bit: H3_ELEM_F16 as in the reference, or H3_ELEM_BF16 (an extension:
 *     widened to f32 exactly, so the quantizer arithmetic is unchanged).
 *   - Head-major operands: codes [heads][capacity][32] i32 (four int8 codes per word, low byte
 *     first), scales [heads][capacity] f32. Token-major: codes [tokens][heads*32], scales
 *     [tokens][heads]. Values: one fp32 scale per (token, head) = absmax/127 * extra_scale.
 *   - V^T: [width][row_capacity] f16. Rows of the output past the token count are not written.
 */
#ifndef H3ATTN_H
#define H3ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t *h3_stream; /* hipStream_t; NULL is the default stream */

/* A binding: a device buffer and its length in bytes (reference `View`, src/stack.rs:204-213). */
typedef struct {
  void *ptr;
  size_t bytes;
} h3_view;

enum {
  H3_OK = 0,
  H3_ERR_BINDING = 1,  /* a binding is shorter than the extent the kernel addresses */
  H3_ERR_CONFIG = 2,   /* a config value outside its declared range */
  H3_ERR_ARGUMENT = 3, /* a workload/scalar argument outside its range, or a null pointer */
  H3_ERR_LAUNCH = 4,   /* the HIP runtime refused the launch */
  H3_ERR_NO_DEVICE = 5 /* no usable gfx950 device */
};

enum { H3_ELEM_F16 = 0, H3_ELEM_BF16 = 1, H3_ELEM_F32 = 2 /* h3_prepare_plain_i8 only */ };

/* Message of the last failing call on this thread ("" after success). */
const char *h3_last_error(void);
/* Library version string. */
const char *h3_version(void);

/* ------------------------------------------------------------------ operand preparation */

/* Config of h3.prepare_qk_i8 / prepare_qk_i8hm / prepare_qk_rope_i8hm
 * (kernels/prepare_qk_i8.loom:9-15, prepare_qk_i8hm.loom:5-13, prepare_qk_rope_i8hm.loom:7-17):
 *   row_stride   multiple of 128 in [128, 65536): elements per input row
 *   head_offset  multiple of 128 in [0, 65536): first channel of head 0
 *   heads        [1, 256)
 *   extra_scale  multiplies absmax/127 into the stored scale (Q: 1/sqrt(128)/128, K: 1)
 *   token_capacity  head-major row capacity, multiple of 32 in [32, 1048576)
 *   eps          RMSNorm epsilon (RoPE variants only)
 *   elem         H3_ELEM_F16 or H3_ELEM_BF16 */
typedef struct {
  uint32_t row_stride;
  uint32_t head_offset;
  uint32_t heads;
  float extra_scale;
  uint32_t token_capacity;
  float eps;
  uint32_t elem;
} h3_prepare_cfg;

/* h3_prepare_qk_i8 (kernels/prepare_qk_i8.loom:17-192; token-major).
 * Per (token, head): y = x - mean; r = H_128 y (unnormalised Sylvester Hadamard, the
 * reference's fp32 butterfly order); amax = max(max|r|, 1e-30); codes = clamp(rne(r*127/amax),
 * +-127) packed four per i32; scale = amax/127 * extra_scale.
 *   x [tokens][row_stride] 16-bit, mean [row_stride] f32 -> codes [tokens][heads*32] i32,
 *   scales [tokens][heads] f32. tokens in [1, 1048576). */
int h3_prepare_qk_i8(const h3_prepare_cfg *cfg, uint32_t tokens, h3_view x, h3_view mean,
                     h3_view codes, h3_view scales, h3_stream stream);

/* h3_prepare_qk_i8hm (kernels/prepare_qk_i8hm.loom:13-196): as above, written head-major:
 * codes [heads][token_capacity][32], scales [heads][token_capacity]. Requires
 * tokens <= token_capacity; rows past tokens are untouched (the caller zeroes them once). */
int h3_prepare_qk_i8hm(const h3_prepare_cfg *cfg, uint32_t tokens, h3_view x, h3_view mean,
                       h3_view codes, h3_view scales, h3_stream stream);

/* h3_prepare_qk_i4 (kernels/prepare_qk_i4.loom:1-244): the int4 operands of attention_i4qk*,
 * token-major. The same rotation; amax = max(max|r|, 1e-30); scale = amax/7 * extra_scale;
 * codes = clamp(rne(r*7/amax), +-7), eight 4-bit codes per i32 word, low nibble first.
 *   x [tokens][row_stride] 16-bit, mean [row_stride] f32 (may be null) -> codes
 *   [tokens][heads*16] i32, scales [tokens][heads] f32. token_capacity is not read. */
int h3_prepare_qk_i4(const h3_prepare_cfg *cfg, uint32_t tokens, h3_view x, h3_view mean,
                     h3_view codes, h3_view scales, h3_stream stream);

/* h3_prepare_qk_rope_i8hm (kernels/prepare_qk_rope_i8hm.loom:19-243): per-head RMSNorm
 * (weight[128], eps), rotate-half RoPE on channels < 96 (pairs c <-> c+48, tables cos/sin
 * [tokens][48] f32), f16 rounding, then the quantizer with zero mean; head-major output.
 * x is the fused QKV row [tokens][row_stride]; head_offset selects Q (0) or K (inner). */
int h3_prepare_qk_rope_i8hm(const h3_prepare_cfg *cfg, uint32_t tokens, h3_view x,
                            h3_view weight, h3_view cos_t, h3_view sin_t, h3_view codes,
                            h3_view scales, h3_stream stream);

/* K-mean smoothing fused with RMSNorm + RoPE + quantize (no reference counterpart: the reference
 * keeps rope_qknorm_f16 -> colmean_f32 -> prepare_qk_i8hm(mean) for smoothing,
 * src/stack.rs:1306-1326, 1727-1791). Two passes on `stream`: the column mean of the rotated f16
 * K over all tokens into `mean` ([heads*128] f32, sequential fp32 order), then the quantizer on
 * rotated K minus that mean. Byte-identical to the separate route. */
int h3_prepare_k_rope_smooth_i8hm(const h3_prepare_cfg *cfg, uint32_t tokens, h3_view x,
                                  h3_view weight, h3_view cos_t, h3_view sin_t, h3_view mean,
                                  h3_view codes, h3_view scales, h3_stream stream);

/* Config of h3.rope_qknorm_f16 (kernels/rope_qknorm_f16.loom; src/stack.rs:563-577). */
typedef struct {
  uint32_t row_stride; /* elements per fused QKV row */
  uint32_t heads;      /* query heads */
  uint32_t kv_heads;   /* key/value heads */
  uint32_t k_offset;   /* first K channel (heads*128) */
  float eps;
  uint32_t copy_v; /* 1: also copy the V slice into v_out [tokens][kv_heads*128] */
  uint32_t elem;
} h3_rope_cfg;

/* h3_rope_qknorm_f16 (kernels/rope_qknorm_f16.loom:1-173): RMSNorm + RoPE of Q and K to f16
 * q_out [tokens][heads*128], k_out [tokens][kv_heads*128]; V copied when copy_v. The same
 * device arithmetic as h3_prepare_qk_rope_i8hm, so the fused and separate routes agree
 * byte-for-byte (tests/kernels.rs:3153-3276). */
int h3_rope_qknorm_f16(const h3_rope_cfg *cfg, uint32_t tokens, h3_view x, h3_view qweight,
                       h3_view kweight, h3_view cos_t, h3_view sin_t, h3_view q_out,
                       h3_view k_out, h3_view v_out, h3_stream stream);

/* h3_colmean_f32 (kernels/colmean_f32.loom): mean[c] = (sum_t x[t][c]) / tokens in sequential
 * fp32 order. width: multiple of 256 in [256, 65536); x [tokens][width] 16-bit. */
int h3_colmean_f32(uint32_t width, uint32_t elem, uint32_t tokens, h3_view x, h3_view mean,
                   h3_stream stream);

/* Config of h3.transpose_f16 / transpose_qkv_v_f16 (kernels/transpose_f16.loom:7-9). */
typedef struct {
  uint32_t width;        /* multiple of 32 in [32, 65536) */
  uint32_t row_capacity; /* multiple of 32 in [32, 1048576) */
  uint32_t elem;         /* bf16 input is rounded to f16 */
} h3_transpose_cfg;

/* h3_transpose_f16 (kernels/transpose_f16.loom): x [rows][width] -> out [width][row_capacity]
 * f16. The launch covers ceil(launch_rows/32) tiles of 32 columns: columns >= rows inside them
 * are zeroed (launch over the whole capacity to clear reused storage, src/stack.rs:1804-1811).
 * rows <= launch_rows; both <= row_capacity. */
int h3_transpose_f16(const h3_transpose_cfg *cfg, uint32_t launch_rows, uint32_t rows, h3_view x,
                     h3_view out, h3_stream stream);

/* h3_transpose_qkv_v_f16 (kernels/transpose_qkv_v_f16.loom): as above, reading the V third of
 * a fused [rows][3*width] QKV projection; tiles of 64 columns when width % 64 == 0, else 32. */
int h3_transpose_qkv_v_f16(const h3_transpose_cfg *cfg, uint32_t launch_rows, uint32_t rows,
                           h3_view x, h3_view out, h3_stream stream);

/* ------------------------------------------------------------------ producers of the operands */

/* Config of h3.gemm_i8_qkv_256 (kernels/gemm_packed_256.loom:3432-3440; src/dispatch.rs:758-790):
 *   k_size    multiple of 64 in [64, 65536]: reduction length
 *   n_size    multiple of 384 in [384, 65536]: output channels (Q, K, V thirds)
 *   k_stride  multiple of 64 in [64, 65536], >= k_size: bytes per operand row
 *   m_group   [1, 4]: the reference's raster grouping; accepted and validated, the raster here
 *             is fixed by the kernel. */
typedef struct {
  uint32_t k_size;
  uint32_t n_size;
  uint32_t k_stride;
  uint32_t m_group;
} h3_gemm_cfg;

/* h3_gemm_i8_qkv_256 (kernels/gemm_packed_256.loom:3429-3471, the packed_256 template at
 * 14-412; bindings src/dispatch.rs:1025-1045): the compact INT8 QKV projection.
 *   acc = sum_k a[m][k] * w[n][k] (int8, exact int32);
 *   v = ((float)acc * w_scale[n]) * a_scale[m] + 0.0, clamped to +-65472 when finite;
 *   n < 2N/3: out[m][n] f16 with row pitch 2N/3 (Q and K rows);
 *   n >= 2N/3: V^T, out[M*2N/3 + (n - 2N/3)*cap + m] f16, cap = ceil(M/256)*256, zero for
 *   M <= m < cap.
 *   a [tokens][k_stride] int8, w [n_size][k_stride] int8, w_scale [n_size] f32,
 *   a_scale [tokens] f32, out (tokens*n_size + (cap - tokens)*n_size/3) f16 (8-byte aligned).
 *   tokens in [1, 16777216]. */
int h3_gemm_i8_qkv_256(const h3_gemm_cfg *cfg, uint32_t tokens, h3_view a, h3_view w,
                       h3_view w_scale, h3_view a_scale, h3_view out, h3_stream stream);

/* Config of h3.prepare_plain_i8 / prepare_plain_f32_i8
 * (kernels/prepare_i8_family.loom:202-206, 598-602; src/dispatch.rs:570-600):
 *   width       multiple of 256 in [256, 32768]: channels per token row
 *   lanes       multiple of 32 in [32, 1024]: the reference's launch width; accepted and
 *               validated, the launch shape here is fixed by the kernel
 *   out_stride  multiple of 64 in [256, 65536], >= width: bytes per code row (the GEMM's
 *               k_stride)
 *   elem        H3_ELEM_F16 (prepare_plain_i8), H3_ELEM_F32 (prepare_plain_f32_i8) or
 *               H3_ELEM_BF16 (an extension) */
typedef struct {
  uint32_t width;
  uint32_t lanes;
  uint32_t out_stride;
  uint32_t elem;
} h3_prepare_plain_cfg;

/* h3_prepare_plain_i8 (kernels/prepare_i8_family.loom:200-294, f32 input 598-689): the INT8
 * GEMM A operand. Per token row: each 256-channel group rotated by H4 (x) H4 (x) H4 (x) H4 with
 * H4 = [[1,1,1,-1],[1,1,-1,1],[1,-1,1,1],[-1,1,1,1]] (radix-4 stages of strides 1, 4, 16, 64 in
 * the reference's fp32 order), amax over the row (non-finite counts as inf),
 * s = max(amax/16, 1e-30)/127, codes = clamp(rne(y*(1/16)/s), +-127), zero codes when s is not
 * finite.
 *   x [tokens][width] (elem), codes [tokens][out_stride] int8 (bytes >= width untouched),
 *   scales [tokens] f32. x and codes 16-byte aligned. tokens in [1, 1048576]. */
int h3_prepare_plain_i8(const h3_prepare_plain_cfg *cfg, uint32_t tokens, h3_view x,
                        h3_view codes, h3_view scales, h3_stream stream);

/* rope::dit (src/rope.rs:11-37), on the host: the DiT's cos/sin tables [rows][48] f32 for
 * h3_prepare_qk_rope_i8hm and h3_rope_qknorm_f16. For row r and axis a in 0..2, with
 * p = (float)pos[3r + a] and angle = p * inv_freq[j] in f32 (j in 0..15):
 * cos_t[48r + 16a + j] = cosf(angle), sin_t[...] = sinf(angle).
 * pos [rows][3] f64, inv_freq [16] f32, cos_t/sin_t [rows][48] f32: HOST pointers. No device
 * work; safe to call without a GPU. */
int h3_rope_dit_tables(const double *pos, size_t rows, const float *inv_freq, float *cos_t,
                       float *sin_t);

/* ------------------------------------------------------------------ attention */

/* Config of h3.attention_i8qk_* / attention_i8qkhm_mha8_k64_lds_f16_wmma
 * (kernels/attention_i8qkhm_mha8_k64_lds_f16_wmma.loom:7-17):
 *   q_stride, kv_stride, out_stride  multiples of 128 in [128, 32768): channels per token
 *   tokens          [1, 1048576): keys (and query rows) of the sequence
 *   token_capacity  multiple of 16 in [32, 1048576), >= tokens
 *   scale           declared and unused, as in the reference (the softmax scale rides in
 *                   Q's extra_scale, src/stack.rs:622-625).
 * Heads: the launch's `heads` rows take key/value head y % (kv_stride/128) and query head
 * kv_head % (out_stride/128) (attention_i8qkhm_mha8_k64_lds_f16_wmma.loom:300-340), so it reads
 * kv = min(heads, kv_stride/128) key/value heads and q = min(kv, out_stride/128) query heads.
 * out_stride may exceed heads*128: the reference's direct-attention pitch (src/stack.rs:751-758,
 * gemm_pitch in src/model.rs:74-85, e.g. q/kv 7168, out 7296 at 56 heads) leaves the columns
 * past the touched heads unwritten. Bindings are checked against what the launch addresses:
 * head-major Q codes/scales q*token_capacity rows, K kv*token_capacity rows; token-major whole
 * rows of token_capacity; V^T kv*128 rows of token_capacity; out (token_count-1)*out_stride +
 * q*128 elements. Token-major launches need q <= q_stride/128. */
typedef struct {
  uint32_t q_stride;
  uint32_t kv_stride;
  uint32_t out_stride;
  uint32_t tokens;
  uint32_t token_capacity;
  float scale;
} h3_attention_cfg;

/* h3_attention_i8qkhm (kernels/attention_i8qkhm_mha8_k64_lds_f16_wmma.loom): non-causal MHA
 * over head-major INT8 operands.
 *   out[t][h*128 + c] = sum_j softmax_j(S_tj * qs_t * ks_j) vt[h*128 + c][j],
 *   S_tj = sum_e qcode_te * kcode_je (exact int32), for t < token_count, h < heads.
 *   qi, ki [heads][token_capacity][32] i32; qs, ks [heads][token_capacity] f32;
 *   vt [kv_stride][token_capacity] f16 (columns >= tokens must be finite, the transposes
 *   zero them); out [token_count][out_stride] f16. token_count in [1, tokens]. */
int h3_attention_i8qkhm(const h3_attention_cfg *cfg, uint32_t token_count, uint32_t heads,
                        h3_view qi, h3_view qs, h3_view ki, h3_view ks, h3_view vt, h3_view out,
                        h3_stream stream);

/* h3_attention_i8qk (kernels/attention_i8qk_family.loom: attention_i8qk_mha_lds_f16_wmma): the
 * same attention over token-major operands: qi [capacity][q_stride/4] i32,
 * qs [capacity][q_stride/128], ki [capacity][kv_stride/4], ks [capacity][kv_stride/128]. The Q
 * scales are read at the pitch the quantizer writes them, q_stride/128 heads per token; the
 * reference's kernel reads them at out_stride/128 (attention_i8qk_family.loom:87, 112, 197),
 * which differs only under a padded output pitch, where it would read another row's scale. */
int h3_attention_i8qk(const h3_attention_cfg *cfg, uint32_t token_count, uint32_t heads,
                      h3_view qi, h3_view qs, h3_view ki, h3_view ks, h3_view vt, h3_view out,
                      h3_stream stream);

/* h3_attention_i4qk (kernels/attention_i4qk_family.loom: attention_i4qk_mha_lds_f16_wmma and
 * attention_i4qk_mha8_lds_f16_wmma; kernels/attention_i4qkl_mha8_lds_f16_wmma.loom for long
 * sequences, src/stack.rs:712-722): the same attention over int4 operands from
 * h3_prepare_qk_i4: qi [capacity][q_stride/2] bytes and ki [capacity][kv_stride/2] bytes (eight
 * 4-bit codes per word, low nibble first), qs/ks [capacity][heads] f32. The reference's three
 * launch shapes are one kernel here. */
int h3_attention_i4qk(const h3_attention_cfg *cfg, uint32_t token_count, uint32_t heads,
                      h3_view qi, h3_view qs, h3_view ki, h3_view ks, h3_view vt, h3_view out,
                      h3_stream stream);

/* Config of the skip twins h3.attention_i4qks_* (kernels/attention_i4qks_family.loom:
 * 487-534): the attention config plus skip_tau (finite; the reference's Stack selects the twins
 * for tau > 0, src/stack.rs:727-745). */
typedef struct {
  uint32_t q_stride;
  uint32_t kv_stride;
  uint32_t out_stride;
  uint32_t tokens;
  uint32_t token_capacity;
  float scale;
  float skip_tau;
} h3_attention_skip_cfg;

/* h3_attention_i4qks (kernels/attention_i4qks_family.loom, attention_i4qksl_mha8_lds_f16_wmma
 * .loom): h3_attention_i4qk with the reference's tile skip. For each key tile and each wave of
 * queries, gap = max over the wave's queries of (the tile's max score - the running max before
 * the tile), in the natural-log units of the scores; a tile with gap < -skip_tau adds nothing
 * (no probabilities, no PV; loom:318-324). Tiles here are 64 keys x 32 queries (the reference's
 * 16 x 16), and the running max is the kernel's lazily raised one (never above the exact max),
 * so this kernel never skips a tile the exact rule would keep at this granularity. */
int h3_attention_i4qks(const h3_attention_skip_cfg *cfg, uint32_t token_count, uint32_t heads,
                       h3_view qi, h3_view qs, h3_view ki, h3_view ks, h3_view vt, h3_view out,
                       h3_stream stream);

/* The _ws forms of the token-major attention entries (h3_attention_i8qk, h3_attention_i4qk,
 * h3_attention_i4qks; h3_vsa_attention_i8_ws below) have no counterpart in the reference; they
 * are for callers that can lend device memory. Token-major key scales ([token][heads] f32, the
 * reference's layout) put every (key, head) scale in its own 128-byte line shared with the other
 * heads, so each key tile pulls one line per key. A _ws form first transposes the scales
 * head-major into `workspace`, at least h3_scales_workspace_bytes(cfg) = (kv_stride/128) *
 * tokens * 4 bytes, and the kernel reads them from there (measured at 129k tokens and 32 heads:
 * 7-8 % faster dense, 28 % faster VSA attention). Results are bit-identical to the form without
 * _ws. Calls that share a workspace must not overlap. A short workspace fails with
 * H3_ERR_BINDING, a null one with H3_ERR_ARGUMENT. */
size_t h3_scales_workspace_bytes(const h3_attention_cfg *cfg);
int h3_attention_i8qk_ws(const h3_attention_cfg *cfg, uint32_t token_count, uint32_t heads,
                         h3_view qi, h3_view qs, h3_view ki, h3_view ks, h3_view vt, h3_view out,
                         h3_view workspace, h3_stream stream);
int h3_attention_i4qk_ws(const h3_attention_cfg *cfg, uint32_t token_count, uint32_t heads,
                         h3_view qi, h3_view qs, h3_view ki, h3_view ks, h3_view vt, h3_view out,
                         h3_view workspace, h3_stream stream);
int h3_attention_i4qks_ws(const h3_attention_skip_cfg *cfg, uint32_t token_count, uint32_t heads,
                          h3_view qi, h3_view qs, h3_view ki, h3_view ks, h3_view vt,
                          h3_view out, h3_view workspace, h3_stream stream);

/* h3_attention_i4qk_fp6: h3_attention_i4qk (the same bindings, token-major int4 operands and
 * scales as h3_prepare_qk_i4 writes them) computed on gfx950's FP6 matrix instructions, with a
 * lent workspace of h3_fp6_workspace_bytes(cfg) bytes (1.09 GB at 129,024 tokens and 32 heads).
 * No counterpart in the reference: every int4 code c (-8..7) is converted into the workspace as
 * the FP6 e2m3 value c/2 (exact), in head-major rows laid out for v_mfma_f32_32x32x64_f8f6f4, and
 * the scales head-major (the key scales times 4); the head-major attention kernel then runs QK
 * on that MFMA, 64 channels per instruction at the cost of the int8 one's 32, with exact f32
 * scores. Allocates nothing. */
int h3_attention_i4qk_fp6(const h3_attention_cfg *cfg, uint32_t token_count, uint32_t heads,
                          h3_view qi, h3_view qs, h3_view ki, h3_view ks, h3_view vt, h3_view out,
                          h3_view workspace, h3_stream stream);
size_t h3_fp6_workspace_bytes(const h3_attention_cfg *cfg);

/* h3_attention_i8qk_static has no counterpart in the reference. It is for callers that cannot
 * allocate device memory and have none to lend (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc): h3_attention_i8qk_ws with the workspace in a static
 * device array of 8 MiB that the library holds on each GPU it runs on until the process ends.
 * Same arguments as h3_attention_i8qk and results bit-identical to h3_attention_i8qk_ws; it
 * allocates nothing (the first call on a device looks up that device's array with
 * hipGetSymbolAddress). Limit: h3_scales_workspace_bytes(cfg) <= 8 MiB, i.e. (kv_stride/128) *
 * tokens <= 2,097,152 (32 heads up to 65,536 tokens); beyond it the call fails with
 * H3_ERR_CONFIG and launches nothing. Calls on one device share the array: calls that overlap on
 * one device (unordered streams) race. */
int h3_attention_i8qk_static(const h3_attention_cfg *cfg, uint32_t token_count, uint32_t heads,
                             h3_view qi, h3_view qs, h3_view ki, h3_view ks, h3_view vt,
                             h3_view out, h3_stream stream);

/* Cross-attention with grouped heads and a key-padding mask: BASELINE config 4's text
 * cross-attention (32 query heads over 8 key/value heads, 512 text tokens, padded positions
 * masked). An extension: the reference has no such kernel.
 *   q_heads   [1, 256]; kv_heads divides q_heads; query head h reads key/value head
 *             h / (q_heads / kv_heads)
 *   q_tokens  [1, 1048576] query rows; q_capacity multiple of 32, >= q_tokens
 *   kv_tokens [1, 1048576] key rows;   kv_capacity multiple of 32, >= kv_tokens
 *   out_stride multiple of 128 in [128 * q_heads, 32768] */
typedef struct {
  uint32_t q_heads;
  uint32_t kv_heads;
  uint32_t q_tokens;
  uint32_t q_capacity;
  uint32_t kv_tokens;
  uint32_t kv_capacity;
  uint32_t out_stride;
} h3_cross_cfg;

/* h3_attention_i8qkhm_cross: out[t][h*128 + c] = sum_j softmax_j(S_tj * qs_t * ks_j) vt[g*128 +
 * c][j] over the keys j < kv_tokens with key_mask[j] != 0, g = h / (q_heads / kv_heads).
 * Head-major operands as h3_attention_i8qkhm: qi [q_heads][q_capacity][32] i32, qs
 * [q_heads][q_capacity] f32, ki [kv_heads][kv_capacity][32], ks [kv_heads][kv_capacity],
 * vt [kv_heads*128][kv_capacity] f16 (columns >= kv_tokens finite), key_mask [kv_tokens] u8,
 * out [q_tokens][out_stride] f16. A query whose keys are all masked gets a non-finite row. qs
 * must be positive (the quantizer's are): masked keys are dropped through a -inf
 * dequantisation offset. */
int h3_attention_i8qkhm_cross(const h3_cross_cfg *cfg, h3_view qi, h3_view qs, h3_view ki,
                              h3_view ks, h3_view vt, h3_view key_mask, h3_view out,
                              h3_stream stream);

/* ------------------------------------------------------------------ VSA (video sparse attention) */

/* Config of h3.vsa.* (kernels/vsa_ops.loom:3-9), as src/vsa/device.rs:63-77 builds it:
 *   tokens  [1, 1048576]: rows of the activations in sequence order
 *   padded  multiple of 64 in [64, 1048576]: rows of the gathered layout, 64 * blocks
 *   width   multiple of 128 in [128, 32768]: heads * 128
 *   blocks  [1, 16384]: 64-row blocks of the plan (prefix tiles, then 4x4x4 video cubes)
 *   heads   [1, 256]
 *   prefix  [0, blocks]: the prefix blocks (text, references, audio), always attended
 *   topk    [0, 16384]: non-prefix blocks each query block keeps beyond the forced ones
 * The gathered layout holds block b in rows 64b..64b+63, its lengths[b] live rows first. f16
 * activations, block means (f32) and the gated scatter's operands must be 16-byte aligned. */
typedef struct {
  uint32_t tokens;
  uint32_t padded;
  uint32_t width;
  uint32_t blocks;
  uint32_t heads;
  uint32_t prefix;
  uint32_t topk;
} h3_vsa_cfg;

/* h3_vsa_gather (vsa_ops.loom h3_vsa_gather): y[i] = x[src[i]] for 0 <= src[i] < tokens, else a
 * zero row. src [padded] i32, x [tokens][width] f16, y [padded][width] f16. */
int h3_vsa_gather(const h3_vsa_cfg *cfg, h3_view src, h3_view x, h3_view y, h3_stream stream);
/* h3_vsa_scatter (vsa_ops.loom h3_vsa_scatter): y[r] = x[inverse[r]]. inverse [tokens] i32 (a
 * value outside [0, padded) writes a zero row), x [padded][width], y [tokens][width] f16. */
int h3_vsa_scatter(const h3_vsa_cfg *cfg, h3_view inverse, h3_view x, h3_view y,
                   h3_stream stream);
/* h3_vsa_pool (vsa_ops.loom h3_vsa_pool): means[b][c] = (sum_{j < lengths[b]} x[64b+j][c]) /
 * lengths[b], a running f32 sum over the rows (bit-identical to the reference). lengths
 * [blocks] i32 in [1, 64], x [padded][width] f16, means [blocks][width] f32. */
int h3_vsa_pool(const h3_vsa_cfg *cfg, h3_view lengths, h3_view x, h3_view means,
                h3_stream stream);
/* h3_vsa_scores (vsa_ops.loom h3_vsa_scores): scores[h][q][j] = fma chain over d = 0..127 of
 * qm[q][128h+d] * km[j][128h+d] (bit-identical). qm, km [blocks][width] f32, scores
 * [heads][blocks][blocks] f32. */
int h3_vsa_scores(const h3_vsa_cfg *cfg, h3_view qm, h3_view km, h3_view scores,
                  h3_stream stream);
/* h3_vsa_route (vsa_ops.loom h3_vsa_route): routes[h][q][j] = 1 when q < prefix, j < prefix or
 * |q - j| <= 1; otherwise 1 when fewer than topk of the non-prefix scores of row q are strictly
 * greater than scores[h][q][j], else 0. Exact (integer) result; computed per row by a radix
 * select of the topk-th largest score instead of the reference's count per entry. */
int h3_vsa_route(const h3_vsa_cfg *cfg, h3_view scores, h3_view routes, h3_stream stream);
/* h3_vsa_coarse (vsa_ops.loom h3_vsa_coarse): coarse[q][128h+c] = sum_j softmax_j(scores[h][q]
 * [j] / sqrt(128)) vm[j][128h+c], with the hardware exp (the reference's expf<afn>). scores
 * [heads][blocks][blocks], vm and coarse [blocks][width] f32. */
int h3_vsa_coarse(const h3_vsa_cfg *cfg, h3_view scores, h3_view vm, h3_view coarse,
                  h3_stream stream);
/* h3_vsa_gated_scatter (vsa_ops.loom h3_vsa_gated_scatter): out[r][c] = f16(fma(gate[r][c],
 * coarse[inverse[r]/64][c], fine[inverse[r]][c])) (bit-identical). inverse [tokens], fine
 * [padded][width] f16, gate [tokens][width] f16, coarse [blocks][width] f32, out [tokens][width]. */
int h3_vsa_gated_scatter(const h3_vsa_cfg *cfg, h3_view inverse, h3_view fine, h3_view gate,
                         h3_view coarse, h3_view out, h3_stream stream);
/* h3_vsa_kmean (kernels/vsa_kmean.loom): mean[c] = (sum_t x[t][c]) / tokens, a running f32 sum
 * (bit-identical). width multiple of 128 in [128, 65536]; x [tokens][width] f32, mean [width]. */
int h3_vsa_kmean(uint32_t width, uint32_t tokens, h3_view x, h3_view mean, h3_stream stream);
/* h3_vsa_attention_i8 (kernels/vsa_attention_8.loom, h3_vsa_attention_8): h3_attention_i8qk over
 * the gathered layout, where query row t (block t/64) of head h attends only to the keys
 * 64kb + j with routes[h][t/64][kb] != 0 and j < lengths[kb]. cfg->tokens = padded (a multiple
 * of 64, blocks = tokens/64 <= 16384), token operands as h3_attention_i8qk; routes
 * [out_stride/128][blocks][blocks] i32, lengths [blocks] i32. qs must be positive (the quantizer's
 * scales are). Allocates nothing. h3_vsa_attention_i8_ws is the faster form for callers that
 * can lend a workspace. */
int h3_vsa_attention_i8(const h3_attention_cfg *cfg, uint32_t token_count, uint32_t heads,
                        h3_view qi, h3_view qs, h3_view ki, h3_view ks, h3_view vt, h3_view out,
                        h3_view routes, h3_view lengths, h3_stream stream);
/* h3_vsa_attention_i8_ws: h3_vsa_attention_i8 with the key scales read from a head-major copy in
 * a lent workspace of h3_scales_workspace_bytes(cfg) bytes (16.5 MB at 129k tokens and 32
 * heads), as the _ws forms above; no counterpart in the reference. The VSA runtime
 * (h3_vsa_attend) lends its own. */
int h3_vsa_attention_i8_ws(const h3_attention_cfg *cfg, uint32_t token_count, uint32_t heads,
                           h3_view qi, h3_view qs, h3_view ki, h3_view ks, h3_view vt,
                           h3_view out, h3_view routes, h3_view lengths, h3_view workspace,
                           h3_stream stream);


/* h3_vsa_attention_f16 (kernels/vsa_attention_16.loom, h3_vsa_attention_16): the f16 form over
 * the same gathered layout: query row t of head h attends to the keys 64kb + j with
 * routes[h][t/64][kb] != 0 and j < lengths[kb], with scores (q . k) * cfg->scale in f32, a
 * softmax, and f16 probabilities times f16 V. q [token_capacity][q_stride], k and v
 * [token_capacity][kv_stride] f16 token-major (V is not transposed), out [token_count][out_stride]
 * f16; cfg->tokens = padded (a multiple of 64, blocks <= 16384). Allocates nothing. */
int h3_vsa_attention_f16(const h3_attention_cfg *cfg, uint32_t token_count, uint32_t heads,
                         h3_view q, h3_view k, h3_view v, h3_view out, h3_view routes,
                         h3_view lengths, h3_stream stream);

/* ---- VSA host policy (src/vsa.rs), no device work */

/* A prefix segment of the sequence: rows row0 .. row0+rows-1 (text, a reference, audio). */
typedef struct {
  uint32_t row0;
  uint32_t rows;
} h3_vsa_segment;

/* Plan::new (src/vsa.rs:94-143) on a layout given as its prefix segments, in order, and its
 * video grid of nt x nh x nw latent cells (nh = lat_h/2, nw = lat_w/2), which fills rows
 * seq_len - nt*nh*nw + (t*nh + h)*nw + w. Each segment is cut into 64-row tiles (the last one
 * padded with -1); the grid into 4x4x4 cubes in (t, h, w) order, row-major inside a cube.
 * h3_vsa_plan_blocks gives the block count; h3_vsa_plan fills HOST arrays src [64*blocks],
 * inverse [seq_len], lengths [blocks] and *prefix_blocks, and fails (H3_ERR_ARGUMENT) unless
 * every row is covered exactly once (src/vsa.rs:137-140). */
int h3_vsa_plan_blocks(const h3_vsa_segment *segments, uint32_t n_segments, uint32_t nt,
                       uint32_t nh, uint32_t nw, uint32_t *blocks);
int h3_vsa_plan(const h3_vsa_segment *segments, uint32_t n_segments, uint32_t seq_len,
                uint32_t nt, uint32_t nh, uint32_t nw, int32_t *src, int32_t *inverse,
                int32_t *lengths, uint32_t *prefix_blocks);

/* VsaOptions (src/vsa.rs:11-31): keep_percent in (0, 100], 0 <= start <= end <= 1,
 * min_tokens <= 2^20, dense_blocks: global DiT block indices (< 50) that always run dense. */
typedef struct {
  double keep_percent;
  double start;
  double end;
  uint32_t min_tokens;
  const uint32_t *dense_blocks;
  uint32_t n_dense_blocks;
} h3_vsa_options;

/* VsaOptions::validate and AttentionPattern::validate (src/vsa.rs:33-52, 76-85): also refuses
 * attention_bits == 4 ("VSA supports f16 or i8 attention, not i4"). */
int h3_vsa_validate(const h3_vsa_options *options, uint32_t attention_bits);
/* VsaOptions::topk (src/vsa.rs:54-59): round-half-even(keep_percent/100 * nonprefix), at least
 * 1, at most nonprefix - 1 (0 when nonprefix <= 1). */
uint32_t h3_vsa_topk(double keep_percent, uint32_t nonprefix);
/* VsaOptions::dense_reason (src/vsa.rs:60-72): NULL when the step runs sparse, else
 * "below_min_tokens" or "outside_sigma_window". */
const char *h3_vsa_dense_reason(const h3_vsa_options *options, uint32_t tokens, float sigma,
                                double shift);

/* ---- VSA runtime (src/vsa/device.rs: Runtime::new, emit, reset) */

typedef struct h3_vsa h3_vsa;

/* Runtime::new (src/vsa/device.rs:49-188) for the INT8 attention (bits 8): uploads the plan
 * (HOST arrays as h3_vsa_plan fills them), derives the h3.vsa.* and attention configs, and
 * allocates the gathered q/k/v, block means, scores, routes, operand and output buffers and
 * one zeroed K-mean vector per layer. The only allocating VSA call. */
int h3_vsa_build(const int32_t *src, const int32_t *inverse, const int32_t *lengths,
                 uint32_t blocks, uint32_t seq_len, uint32_t prefix_blocks,
                 const h3_vsa_options *options, uint32_t heads, uint32_t layers, h3_vsa **out);
/* Runtime::new with its `bits` argument (device.rs:49-58, 86): 8 as h3_vsa_build, or 16 for the
 * f16 attention (h3_vsa_attention_f16 on the gathered q, k, v): no INT8 operands, V^T or K means
 * are allocated, and h3_vsa_attend runs gather, pool, scores, route, the f16 attention and the
 * (gated) scatter (device.rs:362-386). */
int h3_vsa_build_bits(const int32_t *src, const int32_t *inverse, const int32_t *lengths,
                      uint32_t blocks, uint32_t seq_len, uint32_t prefix_blocks,
                      const h3_vsa_options *options, uint32_t heads, uint32_t bits,
                      uint32_t layers, h3_vsa **out);
void h3_vsa_destroy(h3_vsa *vsa);
/* Runtime::reset (device.rs:189-196): zero every layer's K-mean vector. */
int h3_vsa_reset(h3_vsa *vsa, h3_stream stream);
/* Runtime::emit (device.rs:197-446) for layer `layer`: gather q, k, v [seq_len][heads*128] f16
 * -> pool q, k -> block scores -> route -> Q operand (zero mean), K operand centred on the
 * layer's K mean from the previous call || V transpose -> sparse attention -> the layer's K
 * mean from this call's block means -> scatter into out [seq_len][heads*128] f16, or, with a
 * gate [seq_len][heads*128] f16 (gate.ptr non-NULL), pool v -> coarse attention -> gated
 * scatter. */
int h3_vsa_attend(h3_vsa *vsa, uint32_t layer, h3_view q, h3_view k, h3_view v, h3_view out,
                  h3_view gate, h3_stream stream);
/* Device buffers of the runtime, for inspection: the plan, gathered q/k/v, block means,
 * scores and routes, the INT8 operands, V^T, the gathered output, and layer `layer`'s K mean
 * (the INT8 operands, V^T and the K mean are empty views in a bits-16 runtime). */
typedef struct {
  h3_view src, inverse, lengths, q, k, v, qm, km, scores, routes, qi, ki, qs, ks, vt, out,
      kmean;
  h3_vsa_cfg cfg;
  h3_attention_cfg attention;
} h3_vsa_buffers;
int h3_vsa_inspect(const h3_vsa *vsa, uint32_t layer, h3_vsa_buffers *out);

/* ------------------------------------------------------------------ stack (host mirror) */

/* Row capacity the reference allocates for a sequence of `tokens` (src/stack.rs:299-302):
 * waves = (causal || tokens >= 4096) ? 8 : 4;
 * max(ceil((t+16)/32)*32, ceil(t/(16*waves))*16*waves, ceil(t/256)*256). */
uint32_t h3_capacity(uint32_t tokens, int causal);

/* Attention block dimensions (the subset of the reference's StackDims, src/stack.rs, this path
 * reads). heads == kv_heads, head_dim 128, rope_dim 96. */
typedef struct {
  uint32_t heads;
  uint32_t tokens;
  float eps;      /* RMSNorm epsilon */
  uint32_t elem;  /* element format of the fused QKV projection */
  int ksmooth;    /* H3_KSMOOTH=1: K-mean smoothing on (separate, unfused route) */
  int fused;      /* H3_FUSED_OPERANDS != 0: fused RoPE+quantize operands */
  int direct_attn; /* f16 GEMM activations: the attention writes the out projection's operand
                    * directly, at the padded pitch gemm_pitch(inner, 16) = inner + 128 when
                    * inner*2 is a multiple of 1024, else inner (src/stack.rs:408, 751-758,
                    * 817-822; src/model.rs:74-85). The output binding of the attend calls is
                    * then [t][pitch] f16, and the pad columns are never written. */
} h3_stack_dims;

typedef struct h3_stack h3_stack;

/* Stack::build (src/stack.rs:260-987, INT8 branch): chooses the route (fused head-major operands,
 * head-major separate, or token-major below 4096 tokens), derives every kernel config
 * (src/stack.rs:597-766), and allocates the zero-filled IntQk operand buffers
 * (src/stack.rs:845-908); on the fused route it also creates two side streams (default
 * priority) and three events for the branch fan-out below. The only allocating call;
 * attend/prepare never allocate. */
int h3_stack_build(const h3_stack_dims *dims, h3_stack **out);
void h3_stack_destroy(h3_stack *stack);
uint32_t h3_stack_capacity(const h3_stack *stack);

/* Stack::prepare_fused_operands (src/stack.rs:1541-1616) followed by attention: reads the fused
 * QKV projection [t][3*heads*128], per-head norm weights, cos/sin [t][48]; writes the attention
 * output [t][heads*128] f16. The Q quantizer, the K quantizer (smoothed or not) and the V
 * transpose are three independent branches, as the reference records them
 * (src/stack.rs:1751-1813): forked from `stream` onto the stack's side streams with an event and
 * joined back before the attention, so the call stays ordered on `stream` and capturable. Calls
 * on one stack must not overlap (they share its side streams and operand buffers). */
int h3_stack_attend_fused(h3_stack *stack, uint32_t t, h3_view fused, h3_view qnorm,
                          h3_view knorm, h3_view cos_t, h3_view sin_t, h3_view out,
                          h3_stream stream);

/* Stack::prepare_fused_operands on the compact route (src/stack.rs:634-661, 1034-1040,
 * 1561-1600) followed by attention: `compact` is the output of h3_gemm_i8_qkv_256 for the
 * stack's token count, i.e. Q/K rows [t][2*heads*128] f16 then V^T [heads*128][capacity]. Q and
 * K are prepared from the rows (row stride 2*inner); V^T is read in place, no transpose. Needs
 * the fused route, capacity == ceil(tokens/256)*256 (the reference's condition for this route)
 * and t == the stack's tokens. */
int h3_stack_attend_compact(h3_stack *stack, uint32_t t, h3_view compact, h3_view qnorm,
                            h3_view knorm, h3_view cos_t, h3_view sin_t, h3_view out,
                            h3_stream stream);

/* Stack::attend (src/stack.rs:1669-1839) on post-RoPE f16 q, k, v [t][heads*128]
 * (the unfused route): [colmean(K) when smoothing] -> prep_q || prep_k || transpose(V) ->
 * attention. */
int h3_stack_attend(h3_stack *stack, uint32_t t, h3_view q, h3_view k, h3_view v, h3_view out,
                    h3_stream stream);

/* Operand buffers of the stack (IntQk, src/stack.rs:229-238), for inspection by tests. */
typedef struct {
  h3_view qi, ki, qs, ks, kmean, zmean, vt;
  int head_major;
} h3_int_qk;
int h3_stack_operands(const h3_stack *stack, h3_int_qk *out);

#ifdef __cplusplus
}
#endif
#endif
