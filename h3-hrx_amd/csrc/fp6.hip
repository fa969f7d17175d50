// The FP6 form of the int4 attention (h3_attention_i4qk_fp6; this build's extension of
// kernels/attention_i4qk_family.loom): the int4 operands the quantizer writes (token-major, eight
// signed nibbles per word, low nibble first; token-major f32 scales) are converted into a lent
// workspace for the head-major kernel's FP6 QK (attention_hm.hip, kFp6):
//   - codes: every nibble c (-8..7) becomes the FP6 e2m3 code of c/2, which that format holds
//     exactly (0, 0.5, 1, 1.5, 2, 2.5, 3, 3.5 and -4 .. -0.5); a head's 128 channels become a
//     128-byte row [head * capacity + token] of four 32-byte blocks, block b holding channels
//     32b .. 32b+31 as 32 six-bit codes, code i in bits 6i .. 6i+5 of the block's first 24
//     bytes (little-endian), then 8 zero bytes. That is the operand layout of
//     v_mfma_f32_32x32x64_f8f6f4 with FP6 sources: lane l gives 32 consecutive K elements, the
//     first in the low bits.
//   - scales: transposed head-major, [head][capacity]; the key scales times 4, since the FP6
//     dot products are of c/2 values and so come out as S/4 (a power of two: exact).
// Rows at or past `tokens` are not written; the attention kernel reads none of them.
#include <algorithm>

#include "internal.hpp"

namespace h3 {
namespace {

// e2m3 code of |c|/2 for |c| = 0..8 in 6-bit fields: 0, 0.5 (4), 1 (8), 1.5 (12), 2 (16),
// 2.5 (18), 3 (20), 3.5 (22), 4 (24).
constexpr uint64_t kHalfCodes = 0ull | (4ull << 6) | (8ull << 12) | (12ull << 18) | (16ull << 24) |
                                (18ull << 30) | (20ull << 36) | (22ull << 42) | (24ull << 48);

__device__ __forceinline__ uint32_t fp6_half_code(uint32_t nib) {
  const int c = (int)(nib << 28) >> 28;  // the signed nibble
  const uint32_t a = (uint32_t)(c < 0 ? -c : c);
  return ((uint32_t)(kHalfCodes >> (6 * a)) & 63u) | (c < 0 ? 32u : 0u);
}

// One thread per (token, head, block): four code words in, a 32-byte block out.
__global__ __launch_bounds__(256) void k_i4_fp6_rows(const uint4* __restrict__ codes,
                                                     uint32_t row_quads, uint32_t heads,
                                                     uint32_t tokens, uint32_t capacity,
                                                     uint4* __restrict__ rows) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)tokens * heads * 4) return;
  const uint32_t b = (uint32_t)(i & 3);
  const size_t th = i >> 2;
  const uint32_t h = (uint32_t)(th % heads), t = (uint32_t)(th / heads);
  const uint4 q = codes[(size_t)t * row_quads + 4 * h + b];
  const uint32_t word[4] = {q.x, q.y, q.z, q.w};
  uint32_t w[6] = {0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int e = 0; e < 32; ++e) {
    const uint32_t code = fp6_half_code((word[e >> 3] >> (4 * (e & 7))) & 15u);
    const int bit = 6 * e;
    w[bit >> 5] |= code << (bit & 31);
    if ((bit & 31) > 26) w[(bit >> 5) + 1] |= code >> (32 - (bit & 31));
  }
  uint4* dst = rows + ((size_t)h * capacity + t) * 8 + 2 * b;
  dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
  dst[1] = make_uint4(w[4], w[5], 0u, 0u);
}

// [tokens][heads] -> [heads][capacity] f32, times `mult`, through a 64 x 64 LDS tile.
__global__ __launch_bounds__(256) void k_fp6_scales(const float* __restrict__ s, float* __restrict__ out,
                                                    uint32_t tokens, uint32_t heads,
                                                    uint32_t capacity, float mult) {
  __shared__ float tile[64][65];
  const uint32_t t0 = blockIdx.x * 64, h0 = blockIdx.y * 64;
  const uint32_t x = threadIdx.x & 63, y = threadIdx.x >> 6;
  for (uint32_t r = y; r < 64; r += 4) {
    const uint32_t t = t0 + r, h = h0 + x;
    if (t < tokens && h < heads) tile[r][x] = s[(size_t)t * heads + h];
  }
  __syncthreads();
  for (uint32_t r = y; r < 64; r += 4) {
    const uint32_t h = h0 + r, t = t0 + x;
    if (t < tokens && h < heads) out[(size_t)h * capacity + t] = tile[x][r] * mult;
  }
}

size_t round256(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace

Fp6Layout fp6_layout(const h3_attention_cfg& cfg) {
  const size_t cap = cfg.token_capacity;
  // Every head of a code row is converted: q_stride/128 query heads, kv_stride/128 key heads
  // (the launch reads a subset of them, checked by the caller).
  const size_t hq = cfg.q_stride / 128, hk = cfg.kv_stride / 128;
  Fp6Layout L;
  L.q = 0;
  L.k = L.q + round256(hq * cap * 128);
  L.qs = L.k + round256(hk * cap * 128);
  L.ks = L.qs + round256(hq * cap * 4);
  L.bytes = L.ks + round256(hk * cap * 4);
  return L;
}

hipError_t launch_attention_i4_fp6(const h3_attention_cfg& cfg, uint32_t token_count,
                                   uint32_t heads, const int32_t* qi, const float* qs,
                                   const int32_t* ki, const float* ks, const uint16_t* vt,
                                   uint16_t* out, void* workspace, hipStream_t stream) {
  const Fp6Layout L = fp6_layout(cfg);
  char* ws = static_cast<char*>(workspace);
  const uint32_t hq = cfg.q_stride / 128, hk = cfg.kv_stride / 128;
  const uint32_t tokens = cfg.tokens, cap = cfg.token_capacity;
  // Q rows: every query head of the q_stride-wide rows (q_stride/2 bytes each), with the Q
  // scales [tokens][q_stride/128] the quantizer writes
  const size_t nq = (size_t)tokens * hq * 4, nk = (size_t)tokens * hk * 4;
  hipLaunchKernelGGL(k_i4_fp6_rows, dim3((unsigned)((nq + 255) / 256)), dim3(256), 0, stream,
                     reinterpret_cast<const uint4*>(qi), cfg.q_stride / 32, hq, tokens, cap,
                     reinterpret_cast<uint4*>(ws + L.q));
  hipLaunchKernelGGL(k_i4_fp6_rows, dim3((unsigned)((nk + 255) / 256)), dim3(256), 0, stream,
                     reinterpret_cast<const uint4*>(ki), cfg.kv_stride / 32, hk, tokens, cap,
                     reinterpret_cast<uint4*>(ws + L.k));
  hipLaunchKernelGGL(k_fp6_scales, dim3((tokens + 63) / 64, (hq + 63) / 64), dim3(256), 0, stream,
                     qs, reinterpret_cast<float*>(ws + L.qs), tokens, hq, cap, 1.0f);
  hipLaunchKernelGGL(k_fp6_scales, dim3((tokens + 63) / 64, (hk + 63) / 64), dim3(256), 0, stream,
                     ks, reinterpret_cast<float*>(ws + L.ks), tokens, hk, cap, 4.0f);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_attention_hm_fp6(cfg, token_count, heads, ws + L.q,
                                 reinterpret_cast<const float*>(ws + L.qs), ws + L.k,
                                 reinterpret_cast<const float*>(ws + L.ks), vt, out, stream);
}

}  // namespace h3
