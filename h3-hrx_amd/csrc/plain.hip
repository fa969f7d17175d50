// GEMM-operand INT8 preparation on gfx950: prepare_plain_i8 / prepare_plain_f32_i8
// (kernels/prepare_i8_family.loom:4-72, 80-193, 200-294, 598-689). Per token row of `width`
// channels: rotate every 256-channel group by H4 (x) H4 (x) H4 (x) H4 (four radix-4 stages of
// strides 1, 4, 16, 64, the 1/16 normalisation folded into the scale), take the row's absmax
// (non-finite values count as +inf), and write symmetric int8 codes
//   s = max(amax/16, 1e-30)/127,  q = clamp(rne(x * (1/16)/s), +-127)
// with s beside them; a row whose s is not finite gets zero codes. This is the A operand of the
// INT8 GEMMs, e.g. the attention output before the out-projection (src/dispatch.rs:589-595).
//
// Layout on the GPU: lane g of a row holds channels 64g..64g+63 in registers, so the radix-4
// stages on index digits 0-2 (strides 1, 4, 16) run inside the lane, and the stage on digit 3
// (stride 64) runs across the four lanes of a quad with DPP moves. Every butterfly evaluates the
// reference's four expressions y0 = s01+d23, y1 = s01-d23, y2 = d01+s23, y3 = s23-d01 exactly
// (-ffp-contract=off; the cross-lane form below rewrites them only with exact identities).
// Rows of up to 4096 channels take one wave each (four rows per 256-thread workgroup); wider
// rows take one workgroup of width/64 lanes with the absmax combined through LDS.
#include "internal.hpp"

namespace h3 {
namespace {

constexpr int kGroup = 64;  // channels per lane

__device__ __forceinline__ float quad_dpp_xor1(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true));
}
__device__ __forceinline__ float quad_dpp_xor2(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true));
}

// Radix-4 butterfly on digit d of the lane's 64 values, in the reference's operation order.
template <int kStride>
__device__ __forceinline__ void radix4_in_lane(float (&v)[kGroup]) {
#pragma unroll
  for (int base = 0; base < kGroup; ++base) {
    if ((base / kStride) % 4 != 0) continue;
    const float x0 = v[base], x1 = v[base + kStride], x2 = v[base + 2 * kStride],
                x3 = v[base + 3 * kStride];
    const float s01 = x0 + x1, s23 = x2 + x3, d01 = x0 - x1, d23 = x2 - x3;
    v[base] = s01 + d23;
    v[base + kStride] = s01 - d23;
    v[base + 2 * kStride] = d01 + s23;
    v[base + 3 * kStride] = s23 - d01;
  }
}

// The stride-64 stage across lane digit d = lane % 4, per value x (x_d in lane d):
//   S = x_{d^1} + x_d,  T = x_{d^1} - x_d,  y = S - T_{d^2}.
// Lane 0: (x1+x0) - (x3-x2) = s01 + d23;  lane 1: (x0+x1) - (x2-x3) = s01 - d23;
// lane 2: (x3+x2) - (x1-x0) = d01 + s23;  lane 3: (x2+x3) - (x0-x1) = s23 - d01;
// equal bit for bit to the reference's expressions (a+b = b+a and a-(c-b) = a+(b-c) exactly).
__device__ __forceinline__ float radix4_across_quad(float x) {
  const float xp = quad_dpp_xor1(x);
  const float s = xp + x;
  const float t = xp - x;
  return s - quad_dpp_xor2(t);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int k = 32; k >= 1; k >>= 1) v = fmaxf(v, __shfl_xor(v, k));
  return v;
}

// Load the lane's 64 channels of `row` as f32 (elem: f16, bf16 or f32).
__device__ __forceinline__ void load_group(const void* x, size_t first, int elem,
                                           float (&v)[kGroup]) {
  if (elem == H3_ELEM_F32) {
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(x) + first);
#pragma unroll
    for (int i = 0; i < kGroup / 4; ++i) {
      const float4 f = p[i];
      v[4 * i + 0] = f.x + 0.0f;  // loom:641 adds zero to the f32 input
      v[4 * i + 1] = f.y + 0.0f;
      v[4 * i + 2] = f.z + 0.0f;
      v[4 * i + 3] = f.w + 0.0f;
    }
  } else {
    const uint4* p = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + first);
#pragma unroll
    for (int i = 0; i < kGroup / 8; ++i) {
      const uint4 b = p[i];
      const v4f lo = widen4(make_uint2(b.x, b.y), elem), hi = widen4(make_uint2(b.z, b.w), elem);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[8 * i + j] = lo[j];
        v[8 * i + 4 + j] = hi[j];
      }
    }
  }
}

// Four codes clamp(rne(y * inv_s), +-127) as one word, low byte first. Formed as
// rne(clamp(y * inv_s, +-127)) (the same integer for every finite product; the caller only
// quantises rows whose values are all finite) by adding 1.5 * 2^23: the sum is rounded to an
// integer, ties to even, and the low byte of its bits is the code in two's complement.
__device__ __forceinline__ uint32_t code_bits(float y, float inv_s) {
  return __float_as_uint(fminf(fmaxf(y * inv_s, -127.0f), 127.0f) + 12582912.0f);
}
__device__ __forceinline__ uint32_t code4(const float* y, float inv_s) {
  const uint32_t lo = __builtin_amdgcn_perm(code_bits(y[1], inv_s), code_bits(y[0], inv_s),
                                            0x0c0c0400u);
  const uint32_t hi = __builtin_amdgcn_perm(code_bits(y[3], inv_s), code_bits(y[2], inv_s),
                                            0x04000c0cu);
  return lo | hi;
}

// Transform of the lane's 64 channels (the four radix-4 stages), the row's absmax (over the wave,
// and through `wave_amax` over the workgroup when kWide), and the codes and scale of the row.
template <bool kWide>
__device__ __forceinline__ void transform_store(float (&v)[kGroup], float* wave_amax,
                                                uint32_t wave, uint32_t lane, uint32_t row,
                                                uint32_t g, bool active, uint32_t out_stride,
                                                uint8_t* __restrict__ codes,
                                                float* __restrict__ scales) {
  radix4_in_lane<1>(v);
  radix4_in_lane<4>(v);
  radix4_in_lane<16>(v);
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < kGroup; ++i) {
    v[i] = radix4_across_quad(v[i]);
    const float a = __builtin_fabsf(v[i]);
    amax = fmaxf(amax, a < __builtin_inff() ? a : __builtin_inff());
  }
  amax = wave_max(amax);
  if (kWide) {
    if (lane == 0) wave_amax[wave] = amax;
    __syncthreads();
    amax = 0.0f;
    for (uint32_t w = 0; w < (blockDim.x >> 6); ++w) amax = fmaxf(amax, wave_amax[w]);
  }
  // loom:155-163
  const float row_max = amax * 0.0625f;
  const float safe = fmaxf(row_max, 1.0000000000000001e-30f);
  const float s = safe / 127.0f;
  const float inv_s = 0.0625f / s;
  const bool valid = s < __builtin_inff();
  if (!active) return;
  uint32_t words[kGroup / 4];
  if (valid) {
#pragma unroll
    for (int i = 0; i < kGroup / 4; ++i) words[i] = code4(v + 4 * i, inv_s);
  } else {
#pragma unroll
    for (int i = 0; i < kGroup / 4; ++i) words[i] = 0;
  }
  uint4* dst = reinterpret_cast<uint4*>(codes + (size_t)row * out_stride + (size_t)g * kGroup);
#pragma unroll
  for (int i = 0; i < kGroup / 16; ++i)
    dst[i] = make_uint4(words[4 * i], words[4 * i + 1], words[4 * i + 2], words[4 * i + 3]);
  if (g == 0) scales[row] = s;
}

// One token row per wave (kWide == false, width <= 4096: lanes >= width/64 idle) or per
// workgroup of width/64 lanes (kWide).
template <bool kWide>
__global__ __launch_bounds__(kWide ? 512 : 256) void k_prepare_plain(
    const void* __restrict__ x, uint32_t tokens, uint32_t width, uint32_t out_stride, int elem,
    uint8_t* __restrict__ codes, float* __restrict__ scales) {
  __shared__ float wave_amax[8];
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t row = kWide ? blockIdx.x : blockIdx.x * 4 + wave;
  const uint32_t g = kWide ? threadIdx.x : lane;  // channel group of this lane
  const uint32_t groups = width / kGroup;
  const bool active = row < tokens && g < groups;
  if (!kWide && row >= tokens) return;  // whole wave past the rows

  float v[kGroup];
  if (active) {
    load_group(x, (size_t)row * width + (size_t)g * kGroup, elem, v);
  } else {
#pragma unroll
    for (int i = 0; i < kGroup; ++i) v[i] = 0.0f;
  }
  transform_store<kWide>(v, wave_amax, wave, lane, row, g, active, out_stride, codes, scales);
}

// 16-bit rows of up to 4,096 channels: one wave per row as k_prepare_plain<false>, but each wave
// walks kRowsPerWave rows (row0, row0 + stride, ...) and loads the next row's inputs (8 x 16
// bytes per lane) while it transforms the current one, so a row's loads are in flight under the
// arithmetic of the previous row.
#ifndef H3_PLAIN_ROWS_PER_WAVE
#define H3_PLAIN_ROWS_PER_WAVE 8
#endif
constexpr uint32_t kRowsPerWave = H3_PLAIN_ROWS_PER_WAVE;

__global__ __launch_bounds__(256) void k_prepare_plain_rows(const uint16_t* __restrict__ x,
                                                            uint32_t tokens, uint32_t width,
                                                            uint32_t out_stride, int elem,
                                                            uint8_t* __restrict__ codes,
                                                            float* __restrict__ scales) {
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t g = lane;
  const bool active = g < width / kGroup;
  const uint32_t stride = gridDim.x * 4;
  uint32_t row = blockIdx.x * 4 + wave;
  if (row >= tokens) return;  // whole wave
  uint4 cur[kGroup / 8], nxt[kGroup / 8];
  auto load = [&](uint32_t r, uint4 (&dst)[kGroup / 8]) {
    const uint4* p = reinterpret_cast<const uint4*>(x + (size_t)r * width + (size_t)g * kGroup);
#pragma unroll
    for (int i = 0; i < kGroup / 8; ++i) dst[i] = active ? p[i] : make_uint4(0, 0, 0, 0);
  };
  load(row, cur);
  for (; row < tokens; row += stride) {
    const bool more = row + stride < tokens;  // wave-uniform
    if (more) load(row + stride, nxt);
    float v[kGroup];
#pragma unroll
    for (int i = 0; i < kGroup / 8; ++i) {
      const v4f lo = widen4(make_uint2(cur[i].x, cur[i].y), elem);
      const v4f hi = widen4(make_uint2(cur[i].z, cur[i].w), elem);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[8 * i + j] = lo[j];
        v[8 * i + 4 + j] = hi[j];
      }
    }
    transform_store<false>(v, nullptr, wave, lane, row, g, active, out_stride, codes, scales);
    if (more) {
#pragma unroll
      for (int i = 0; i < kGroup / 8; ++i) cur[i] = nxt[i];
    }
  }
}

}  // namespace

hipError_t launch_prepare_plain(uint32_t width, uint32_t out_stride, uint32_t elem,
                                uint32_t tokens, const void* x, uint8_t* codes, float* scales,
                                hipStream_t stream) {
  const uint32_t groups = width / kGroup;
  if (groups <= 64 && elem != H3_ELEM_F32) {
    const uint32_t waves = (tokens + kRowsPerWave - 1) / kRowsPerWave;
    hipLaunchKernelGGL(k_prepare_plain_rows, dim3((waves + 3) / 4), dim3(256), 0, stream,
                       static_cast<const uint16_t*>(x), tokens, width, out_stride, (int)elem,
                       codes, scales);
  } else if (groups <= 64) {
    hipLaunchKernelGGL(k_prepare_plain<false>, dim3((tokens + 3) / 4), dim3(256), 0, stream, x,
                       tokens, width, out_stride, (int)elem, codes, scales);
  } else {
    const uint32_t threads = (groups + 63) / 64 * 64;
    hipLaunchKernelGGL(k_prepare_plain<true>, dim3(tokens), dim3(threads), 0, stream, x, tokens,
                       width, out_stride, (int)elem, codes, scales);
  }
  return hipGetLastError();
}

}  // namespace h3
