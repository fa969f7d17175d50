// Internal declarations shared by the HIP translation units of libh3attn.
// Device helpers for 16-bit activations and the launchers behind the C ABI in include/h3attn.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/h3attn.h"

namespace h3 {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

// Widen four 16-bit activations (f16 or bf16 bit patterns held in two dwords) to f32 exactly.
__device__ __forceinline__ v4f widen4(uint2 bits, int elem) {
  v4f out;
  if (elem == H3_ELEM_BF16) {
    out[0] = __uint_as_float(bits.x << 16);
    out[1] = __uint_as_float(bits.x & 0xffff0000u);
    out[2] = __uint_as_float(bits.y << 16);
    out[3] = __uint_as_float(bits.y & 0xffff0000u);
  } else {
    v4h h = __builtin_bit_cast(v4h, bits);
    out[0] = (float)h[0];
    out[1] = (float)h[1];
    out[2] = (float)h[2];
    out[3] = (float)h[3];
  }
  return out;
}

// Records `msg` for h3_last_error() and returns `status` (abi.cpp).
int set_error(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Launchers (host). Shapes and bindings are validated by the caller (abi.cpp).
hipError_t launch_prepare_qk(const h3_prepare_cfg& cfg, uint32_t tokens, int head_major,
                             const void* x, const float* mean, int32_t* codes, float* scales,
                             hipStream_t stream);
hipError_t launch_prepare_qk_i4(const h3_prepare_cfg& cfg, uint32_t tokens, const void* x,
                                const float* mean, int32_t* codes, float* scales,
                                hipStream_t stream);
hipError_t launch_prepare_qk_rope(const h3_prepare_cfg& cfg, uint32_t tokens, const void* x,
                                  const float* weight, const float* cos_t, const float* sin_t,
                                  int32_t* codes, float* scales, hipStream_t stream);
hipError_t launch_rope_qknorm(const h3_rope_cfg& cfg, uint32_t tokens, const void* x,
                              const float* qweight, const float* kweight, const float* cos_t,
                              const float* sin_t, uint16_t* q_out, uint16_t* k_out,
                              uint16_t* v_out, hipStream_t stream);
hipError_t launch_colmean(uint32_t width, uint32_t row_stride, uint32_t elem, uint32_t tokens,
                          const void* x, float* mean, hipStream_t stream);
// Two launches: r of every K row into r_scratch ([heads][capacity] floats), then the column
// chains; r_scratch may be the quantizer's scales binding, which the next pass overwrites.
hipError_t launch_rope_colmean(const h3_prepare_cfg& cfg, uint32_t tokens, const void* x,
                               const float* weight, const float* cos_t, const float* sin_t,
                               float* r_scratch, float* mean, hipStream_t stream);
hipError_t launch_prepare_qk_rope_mean(const h3_prepare_cfg& cfg, uint32_t tokens, const void* x,
                                       const float* weight, const float* cos_t,
                                       const float* sin_t, const float* mean, int32_t* codes,
                                       float* scales, hipStream_t stream);
hipError_t launch_transpose(uint32_t width, uint32_t row_capacity, uint32_t row_stride,
                            uint32_t col_offset, uint32_t elem, uint32_t tile, uint32_t launch_rows,
                            uint32_t rows, const void* x, uint16_t* out, hipStream_t stream);
hipError_t launch_gemm_i8_qkv(uint32_t m, uint32_t n, uint32_t k, uint32_t k_stride,
                              const int8_t* a, const int8_t* w, const float* ws, const float* as,
                              uint16_t* out, hipStream_t stream);
hipError_t launch_prepare_plain(uint32_t width, uint32_t out_stride, uint32_t elem,
                                uint32_t tokens, const void* x, uint8_t* codes, float* scales,
                                hipStream_t stream);
// mode: 0 int8 token-major, 1 int8 head-major, 2 int4 token-major, 3 int4 with tile skip
// (skip_tau is read in mode 3 only)
hipError_t launch_attention(const h3_attention_cfg& cfg, int mode, float skip_tau,
                            uint32_t token_count,
                            uint32_t heads, const int32_t* qi, const float* qs, const int32_t* ki,
                            const float* ks, const uint16_t* vt, uint16_t* out, void* workspace,
                            hipStream_t stream);
// The FP6 form of the int4 attention (fp6.hip): byte offsets in its lent workspace of the FP6
// Q and K rows ([heads][capacity][128 B]) and the head-major scales (the key scales times 4).
struct Fp6Layout {
  size_t q, k, qs, ks, bytes;
};
Fp6Layout fp6_layout(const h3_attention_cfg& cfg);
// Converts the token-major int4 operands into the workspace, then runs the head-major kernel's
// FP6 form (launch_attention_hm_fp6) on them.
hipError_t launch_attention_i4_fp6(const h3_attention_cfg& cfg, uint32_t token_count,
                                   uint32_t heads, const int32_t* qi, const float* qs,
                                   const int32_t* ki, const float* ks, const uint16_t* vt,
                                   uint16_t* out, void* workspace, hipStream_t stream);
hipError_t launch_attention_hm_fp6(const h3_attention_cfg& cfg, uint32_t token_count,
                                   uint32_t heads, const void* qf, const float* qs, const void* kf,
                                   const float* ks, const uint16_t* vt, uint16_t* out,
                                   hipStream_t stream);
// Compute units of the current device (cached per device; 256 if the query fails).
uint32_t device_cus();
// attention_i8qkhm: the head-major INT8 kernel of attention_hm.hip (eight waves of 32 queries,
// two per SIMD). Shapes are validated by the caller.
hipError_t launch_attention_hm(const h3_attention_cfg& cfg, uint32_t token_count, uint32_t heads,
                               const int32_t* qi, const float* qs, const int32_t* ki,
                               const float* ks, const uint16_t* vt, uint16_t* out,
                               hipStream_t stream);
// The same kernel on attention_i8qk_family's token-major operands: codes [token][stride], query
// scales [token][q_stride/128], key scales [token][kv_stride/128] or (ks_head_major) the lent
// head-major copy [kv_head][tokens].
hipError_t launch_attention_hm_tm(const h3_attention_cfg& cfg, uint32_t token_count,
                                  uint32_t heads, const int32_t* qi, const float* qs,
                                  const int32_t* ki, const float* ks, bool ks_head_major,
                                  const uint16_t* vt, uint16_t* out, hipStream_t stream);
// The same kernel as cross-attention with a key mask and grouped heads; q_heads / kv_heads must
// divide 8 (each workgroup holds all query heads of one key/value head).
hipError_t launch_attention_hm_cross(const h3_cross_cfg& cfg, const int32_t* qi, const float* qs,
                                     const int32_t* ki, const float* ks, const uint16_t* vt,
                                     const uint8_t* key_mask, uint16_t* out, hipStream_t stream);
// Bytes of the head-major key-scale copy the token-major attention kernels read when a caller
// lends a workspace: (kv_stride / 128) * tokens f32.
size_t scales_workspace_bytes(const h3_attention_cfg& cfg);

// Cross-attention with grouped heads and a key-padding mask (attention.hip)
hipError_t launch_attention_cross(const h3_cross_cfg& cfg, const int32_t* qi, const float* qs,
                                  const int32_t* ki, const float* ks, const uint16_t* vt,
                                  const uint8_t* key_mask, uint16_t* out, hipStream_t stream);
// The int8 token-major attention over the cubes `routes` keeps (attention.hip). With a
// `workspace` of scales_workspace_bytes(cfg) bytes the key scales are first transposed into it
// (head-major) and the kernel reads them from there; with nullptr it reads the token-major
// scales (one 128-byte line per key and head).
hipError_t launch_attention_vsa(const h3_attention_cfg& cfg, uint32_t token_count,
                                uint32_t heads, const int32_t* qi, const float* qs,
                                const int32_t* ki, const float* ks, const uint16_t* vt,
                                uint16_t* out, const int32_t* routes, const int32_t* lengths,
                                void* workspace, hipStream_t stream);
// The f16 VSA attention (attention.hip): token-major f16 q, k, v; scores times cfg.scale.
hipError_t launch_attention_vsa_f16(const h3_attention_cfg& cfg, uint32_t token_count,
                                    uint32_t heads, const uint16_t* q, const uint16_t* k,
                                    const uint16_t* v, uint16_t* out, const int32_t* routes,
                                    const int32_t* lengths, hipStream_t stream);
// h3_vsa_attention_i8 with a caller's workspace of at least scales_workspace_bytes(*cfg) bytes
// (abi.cpp); with an empty view it reads the token-major scales as the public entry point does.
int vsa_attention_i8_ws(const h3_attention_cfg* cfg, uint32_t token_count, uint32_t heads,
                        h3_view qi, h3_view qs, h3_view ki, h3_view ks, h3_view vt, h3_view out,
                        h3_view routes, h3_view lengths, h3_view workspace, hipStream_t stream);
// h3_attention_i8qk_ws on the library's own static scratch array (noalloc.hip): the same
// checks, except that the workspace, a device symbol's address, skips the runtime's pointer
// query.
int attention_i8qk_static_ws(const h3_attention_cfg* cfg, uint32_t token_count, uint32_t heads,
                             h3_view qi, h3_view qs, h3_view ki, h3_view ks, h3_view vt,
                             h3_view out, h3_view workspace, hipStream_t stream);
// VSA operations (vsa.hip)
hipError_t launch_vsa_gather(uint32_t tokens, uint32_t padded, uint32_t width, const int32_t* src,
                             const uint16_t* x, uint16_t* y, hipStream_t stream);
hipError_t launch_vsa_scatter(uint32_t tokens, uint32_t padded, uint32_t width,
                              const int32_t* inverse, const uint16_t* x, uint16_t* y,
                              hipStream_t stream);
hipError_t launch_vsa_pool(uint32_t blocks, uint32_t width, const int32_t* lengths,
                           const uint16_t* x, float* means, hipStream_t stream);
// launch_vsa_gather then launch_vsa_pool on its output, in one kernel (padded = 64 * blocks).
hipError_t launch_vsa_gather_pool(uint32_t tokens, uint32_t blocks, uint32_t width,
                                  const int32_t* src, const int32_t* lengths, const uint16_t* x,
                                  uint16_t* y, float* means, hipStream_t stream);
// h3_vsa_gather(cfg, src, x, y) then h3_vsa_pool(cfg, lengths, y, means), with the checks of
// both, in one kernel (abi.cpp).
int vsa_gather_pool(const h3_vsa_cfg* cfg, h3_view src, h3_view lengths, h3_view x, h3_view y,
                    h3_view means, h3_stream stream);
// The VSA gather of f16 rows x -> gathered ([rows][width], rows a multiple of 64) and the V^T
// transpose of the gathered rows -> out ([width][rows] f16) from one read of x (prepare.hip).
hipError_t launch_gather_transpose(uint32_t width, uint32_t rows, const int32_t* src,
                                   uint32_t src_rows, const uint16_t* x, uint16_t* gathered,
                                   uint16_t* out, hipStream_t stream);
// h3_vsa_gather(cfg, src, x, y) then h3_transpose_f16 of y into vt ([width][padded]), with the
// checks of both, in one kernel (abi.cpp).
int vsa_gather_transpose(const h3_vsa_cfg* cfg, h3_view src, h3_view x, h3_view y, h3_view vt,
                         h3_stream stream);
hipError_t launch_vsa_scores(uint32_t blocks, uint32_t heads, const float* qm, const float* km,
                             float* scores, hipStream_t stream);
hipError_t launch_vsa_route(uint32_t blocks, uint32_t heads, uint32_t prefix, uint32_t topk,
                            const float* scores, int32_t* routes, hipStream_t stream);
hipError_t launch_vsa_coarse(uint32_t blocks, uint32_t heads, const float* scores,
                             const float* vm, float* coarse, hipStream_t stream);
hipError_t launch_vsa_gated_scatter(uint32_t tokens, uint32_t padded, uint32_t width,
                                    const int32_t* inverse, const uint16_t* fine,
                                    const uint16_t* gate, const float* coarse, uint16_t* out,
                                    hipStream_t stream);
hipError_t launch_vsa_kmean(uint32_t tokens, uint32_t width, const float* x, float* mean,
                            hipStream_t stream);

}  // namespace h3
