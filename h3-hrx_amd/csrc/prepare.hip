// Operand preparation for INT8 attention on gfx950: Hadamard-rotated per-(token, head) INT8
// quantisation, the fused RMSNorm + RoPE variant, the f16 RoPE kernel, K column means and the
// V transposes: byte work at HBM rates, the quantizers bounded by their vector issue (each row
// takes a norm, a 128-point Hadamard butterfly and a quantisation). In the quantizers each
// (token, head) row of 128 channels is held by an 8-lane group (sixteen channels per lane, two
// 16-byte loads per lane), a 256-thread workgroup holds 32 rows at a time and every global
// access covers whole 256-byte rows; several rows per group are loaded before any is processed,
// to keep enough bytes in flight. The row-norm pass of the fused K smoothing uses 16-lane groups
// (eight channels per lane), the f16 RoPE kernel and the column means 32-lane halves (four
// channels per lane), all with the same arithmetic.
//
// The arithmetic is built with -ffp-contract=off: every float operation below is one IEEE
// operation in the order written, which is what makes the quantizer bit-exact with the
// reference's fp32 op order (kernels/prepare_qk_i8.loom:63-188).
#include <algorithm>
#include <type_traits>

#include "internal.hpp"

namespace h3 {
namespace {

constexpr int kRowsPerBlock = 8;  // 256 threads = 8 half-waves = 8 (token, head) rows
// Rows per 8-lane group in the quantizers: their loads are issued together before any row is
// processed, so each group keeps kRowsAhead 256-byte rows in flight (one row is far too few
// bytes in flight to cover HBM latency at these kernels' occupancy).
constexpr int kRowsAhead = 4;

// Butterfly partner exchange inside a 32-lane half-wave, on the vector pipe: lane masks 1, 2 and
// 8 are one DPP move (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_ror:8), mask 4 is two
// (row_half_mirror then quad_perm [3,2,1,0]); mask 16 is v_permlane16_swap, which yields the
// values of both members of each lane pair at once (the lane with bit 4 clear first).
__device__ __forceinline__ float dpp(float v, int ctrl) {
  switch (ctrl) {  // the control must be an immediate
    case 0xB1: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true));
    case 0x4E: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true));
    case 0x141: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, true));
    case 0x1B: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x1B, 0xF, 0xF, true));
    default: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xF, 0xF, true));
  }
}
__device__ __forceinline__ float xor_partner(float v, int k) {  // k in {1, 2, 4, 8}
  if (k == 1) return dpp(v, 0xB1);
  if (k == 2) return dpp(v, 0x4E);
  if (k == 4) return dpp(dpp(v, 0x141), 0x1B);
  return dpp(v, 0x128);
}
__device__ __forceinline__ void pair16(float v, float& lo, float& hi) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  lo = __uint_as_float(r[0]);
  hi = __uint_as_float(r[1]);
}
// Sum over the 32 lanes of a half-wave in the order k = 1, 2, 4, 8, 16; every lane gets it.
__device__ __forceinline__ float half_sum(float v) {
#pragma unroll
  for (int k = 1; k < 16; k <<= 1) v = v + xor_partner(v, k);
  float lo, hi;
  pair16(v, lo, hi);
  return lo + hi;
}

// ---------------------------------------------------------------- 16-lane row groups
// The row-norm pass of the fused K smoothing holds one 128-channel row in a 16-lane group (a DPP
// row), eight channels per lane, read with one 16-byte load per lane. Partner exchanges k = 1, 2,
// 4, 8 are the DPP moves of xor_partner, which stay inside a DPP row.
__device__ __forceinline__ float row16_sum(float v) {  // order k = 1, 2, 4, 8
#pragma unroll
  for (int k = 1; k < 16; k <<= 1) v = v + xor_partner(v, k);
  return v;
}

// r = 1/sqrt(mean(v^2) + eps) of the row held by a 16-lane group, eight channels per lane: the
// 32-lane layout's operations in its order (the lane partial is that layout's first butterfly
// sum, k = 1, 2, 4, 8 here are its k = 2, 4, 8, 16).
__device__ __forceinline__ float rms_inverse8(const float (&v)[8], float eps) {
  const float p0 = ((v[0] * v[0] + v[1] * v[1]) + v[2] * v[2]) + v[3] * v[3];
  const float p1 = ((v[4] * v[4] + v[5] * v[5]) + v[6] * v[6]) + v[7] * v[7];
  const float part = row16_sum(p0 + p1);
  const float ms = part * 0.0078125f;
  const float me = ms + eps;
  return 1.0f / __builtin_sqrtf(me);
}

// Eight 16-bit activations (f16 or bf16 bit patterns) widened to f32 exactly.
__device__ __forceinline__ void widen8(uint4 b, int elem, float (&v)[8]) {
  const v4f lo = widen4(make_uint2(b.x, b.y), elem), hi = widen4(make_uint2(b.z, b.w), elem);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[j] = lo[j];
    v[4 + j] = hi[j];
  }
}

__device__ __forceinline__ uint2 load4(const void* base, size_t elem_index) {
  return *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(base) + elem_index);
}

// Per-head RMSNorm(weight, eps) + rotate-half RoPE on channels < 96, rounded to f16 and widened
// back, in this build's fixed fp32 order: lane partial ((v0^2 + v1^2) + v2^2) + v3^2, butterfly
// sum over lanes k = 1..16, mean = ss/128, r = 1/sqrt(mean + eps) (two correctly rounded
// operations), xn = (v*r)*w, then lanes 0-11 (channels 0-47) out = xn*cos - xn_{+48}*sin,
// lanes 12-23 (channels 48-95) out = xn*cos + xn_{-48}*sin, lanes 24-31 out = xn.
// The maths is the reference's (kernels/prepare_qk_rope_i8hm.loom:110-130,
// kernels/rope_qknorm_f16.loom); the device code is shared by every kernel that needs it, so
// fused and separate routes produce identical bits.
// The table values one lane needs for its four channels: norm weights, cos and sin.
struct RopeLane {
  float4 w, c, s;
};

__device__ __forceinline__ RopeLane rope_lane(int lane, const float* weight, const float* cos_row,
                                              const float* sin_row) {
  const int pairlane = lane < 12 ? lane : (lane < 24 ? lane - 12 : 0);
  RopeLane t;
  t.w = *reinterpret_cast<const float4*>(weight + 4 * lane);
  t.c = *reinterpret_cast<const float4*>(cos_row + 4 * pairlane);
  t.s = *reinterpret_cast<const float4*>(sin_row + 4 * pairlane);
  return t;
}

// o rounded to f16 (round to nearest even) and widened back. The empty asm keeps o a rounded f32
// value first: without it the compiler may fold the multiply that produced o into a
// mixed-precision FMA that rounds the exact product once, straight to f16 (v_fma_mixlo_f16),
// which differs from rounding to f32 and then to f16 whenever the two roundings interact.
__device__ __forceinline__ float f16_round(float o) {
  asm("" : "+v"(o));
  return (float)(_Float16)o;
}

// r = 1/sqrt(mean(v^2) + eps) of the 128-channel row held by a half-wave (four channels per lane).
__device__ __forceinline__ float rms_inverse(v4f v, float eps) {
  float part = ((v[0] * v[0] + v[1] * v[1]) + v[2] * v[2]) + v[3] * v[3];
  part = half_sum(part);
  float ms = part * 0.0078125f;
  float me = ms + eps;
  return 1.0f / __builtin_sqrtf(me);
}

// One channel of rmsnorm_rope_f16 given its row's r: the same operations in the same order
// (xn = (v*r)*w for the channel and for its rotation partner, then xn*cos -/+ partner*sin or xn
// itself), rounded to f16 and widened, so the same bits.
__device__ __forceinline__ float rope_channel(float v, float pv, float r, float w, float pw,
                                              float c, float s, bool lo, bool pair) {
  const float xn = (v * r) * w;
  const float px = (pv * r) * pw;
  const float a = xn * c;
  const float b = px * s;
  float o = lo ? (a - b) : (a + b);
  o = pair ? o : xn;
  return f16_round(o);
}

__device__ __forceinline__ v4f rmsnorm_rope_f16(v4f v, int lane, const RopeLane& tab, float eps) {
  const float r = rms_inverse(v, eps);
  const float4 w = tab.w;
  v4f xn;
  xn[0] = (v[0] * r) * w.x;
  xn[1] = (v[1] * r) * w.y;
  xn[2] = (v[2] * r) * w.z;
  xn[3] = (v[3] * r) * w.w;
  const bool lo = lane < 12, pair = lane < 24;
  const int partner = lo ? lane + 12 : (pair ? lane - 12 : lane);
  v4f px;
#pragma unroll
  for (int j = 0; j < 4; ++j) px[j] = __shfl(xn[j], partner, 32);
  const float cc[4] = {tab.c.x, tab.c.y, tab.c.z, tab.c.w};
  const float ss[4] = {tab.s.x, tab.s.y, tab.s.z, tab.s.w};
  v4f out;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float a = xn[j] * cc[j];
    float b = px[j] * ss[j];
    float o = lo ? (a - b) : (a + b);
    o = pair ? o : xn[j];
    out[j] = f16_round(o);
  }
  return out;
}

__device__ __forceinline__ v4f rmsnorm_rope_f16(v4f v, int lane, const float* weight,
                                                const float* cos_row, const float* sin_row,
                                                float eps) {
  return rmsnorm_rope_f16(v, lane, rope_lane(lane, weight, cos_row, sin_row), eps);
}

// ---------------------------------------------------------------- quantizer kernels

constexpr int kGroupsPerBlock = 16;  // the row-norm pass: 256 threads = 16 groups of 16 lanes

__device__ __forceinline__ uint4 load8(const void* base, size_t elem_index) {
  return *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(base) + elem_index);
}
// The same load marked non-temporal: for inputs a kernel reads exactly once, so that they do not
// push out of the caches what the neighbouring kernels will read again.
__device__ __forceinline__ uint4 load8_nt(const void* base, size_t elem_index) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  return __builtin_bit_cast(uint4, __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
                                       reinterpret_cast<const uint16_t*>(base) + elem_index)));
}

// ---------------------------------------------------------------- 8-lane row groups
// The RoPE quantizer holds one 128-channel row in an 8-lane group, sixteen channels per lane
// (two 16-byte loads): a wave then works on eight rows at once, so the per-row work (the norm's
// square root and division, the quantizer's two divisions, the reductions) is spread over twice
// as many rows as in the 16-lane layout, and one more Hadamard stage runs inside the lane. The
// lane of local index i holds channels 16i..16i+15, i.e. the four-channel lanes 4i..4i+3 of the
// 32-lane layout; every sum below is formed from the same two operands in the same order as
// there, so the bits are the same. A group's lanes are those that differ in lane bits 0, 1 and
// 3 (local bits 0, 1, 2), so its three partner exchanges are single DPP moves (quad_perm,
// quad_perm, row_ror:8), where lane bit 2 would need two.
__device__ __forceinline__ int local8(int lane) { return (lane & 3) | ((lane >> 1) & 4); }
__device__ __forceinline__ int group8(int lane) { return ((lane >> 2) & 1) | ((lane >> 3) & 6); }
// The lane of local index i in the group of `lane`.
__device__ __forceinline__ int lane8(int lane, int i) { return (lane & 0x34) | (i & 3) | ((i & 4) << 1); }
constexpr int kLane8Xor[3] = {1, 2, 8};  // lane exchange of local bit 0, 1, 2
constexpr int kRopeGroups = 32;  // 256 threads = 32 groups of 8 lanes
__device__ __forceinline__ float row8_sum(float v) {  // local order 1, 2, 4
#pragma unroll
  for (int b = 0; b < 3; ++b) v = v + xor_partner(v, kLane8Xor[b]);
  return v;
}
__device__ __forceinline__ float row8_max(float v) {
#pragma unroll
  for (int b = 2; b >= 0; --b) v = fmaxf(v, xor_partner(v, kLane8Xor[b]));
  return v;
}

struct RopeLane16 {
  float w[16], c[16], s[16];
};

// Norm weights of the lane's channels and, for lanes 0-5 (channels 0-95), the cos/sin columns
// of their rotation pairs: channel c < 48 and c + 48 share column c. Lanes 0-2 keep -sin, so that
// both halves of the rotation are one addition (a + (-b) is a - b exactly; -(px*sin) is
// px*(-sin) exactly).
__device__ __forceinline__ RopeLane16 rope_lane16(int l, const float* weight, const float* cos_row,
                                                  const float* sin_row) {
  const int pairlane = l < 3 ? l : (l < 6 ? l - 3 : 0);
  RopeLane16 t;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float4 w = *reinterpret_cast<const float4*>(weight + 16 * l + 4 * q);
    const float4 c = *reinterpret_cast<const float4*>(cos_row + 16 * pairlane + 4 * q);
    const float4 sn = *reinterpret_cast<const float4*>(sin_row + 16 * pairlane + 4 * q);
    t.w[4 * q] = w.x; t.w[4 * q + 1] = w.y; t.w[4 * q + 2] = w.z; t.w[4 * q + 3] = w.w;
    t.c[4 * q] = c.x; t.c[4 * q + 1] = c.y; t.c[4 * q + 2] = c.z; t.c[4 * q + 3] = c.w;
    t.s[4 * q] = sn.x; t.s[4 * q + 1] = sn.y; t.s[4 * q + 2] = sn.z; t.s[4 * q + 3] = sn.w;
  }
  if (l < 3) {
#pragma unroll
    for (int j = 0; j < 16; ++j) t.s[j] = -t.s[j];
  }
  return t;
}

// rmsnorm_rope_f16 for a row held sixteen channels per lane: the four-channel partials p0..p3
// of the 32-lane layout's lanes 4l..4l+3, its butterflies k = 1, 2 in the lane ((p0 + p1) +
// (p2 + p3)), its k = 4, 8, 16 as the exchanges of local bits 0, 1, 2; the rotation partner is
// local index l +- 3. `lane` is the wave lane, l its local index.
__device__ __forceinline__ void rmsnorm_rope16(float (&v)[16], int lane, int l,
                                               const RopeLane16& tab, float eps) {
  float p[4];
#pragma unroll
  for (int k = 0; k < 4; ++k)
    p[k] = ((v[4 * k] * v[4 * k] + v[4 * k + 1] * v[4 * k + 1]) + v[4 * k + 2] * v[4 * k + 2]) +
           v[4 * k + 3] * v[4 * k + 3];
  const float part = row8_sum((p[0] + p[1]) + (p[2] + p[3]));
  const float ms = part * 0.0078125f;
  const float me = ms + eps;
  const float r = 1.0f / __builtin_sqrtf(me);
  float xn[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) xn[j] = (v[j] * r) * tab.w[j];
  const bool pair = l < 6;
  const int partner = lane8(lane, l < 3 ? l + 3 : (pair ? l - 3 : l));
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const float px = __shfl(xn[j], partner);
    const float a = xn[j] * tab.c[j];
    const float b = px * tab.s[j];  // tab.s is -sin on lanes 0-2: a + b is a - px*sin there
    const float o = pair ? a + b : xn[j];
    v[j] = f16_round(o);
  }
}

// hadamard128 for sixteen elements per lane: element bits 0-1 (the radix-4 stage), 2 and 3 in
// the lane, bits 4-6 across local bits 0, 1, 2; each stage keeps s + partner (bit clear) and
// partner - s (bit set), the reference's operands in the reference's order. l: local index.
__device__ __forceinline__ void hadamard128_16(float (&s)[16], int l) {
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const float ab_p = s[4 * g] + s[4 * g + 1], ab_m = s[4 * g] - s[4 * g + 1];
    const float cd_p = s[4 * g + 2] + s[4 * g + 3], cd_m = s[4 * g + 2] - s[4 * g + 3];
    s[4 * g] = ab_p + cd_p;
    s[4 * g + 1] = ab_m + cd_m;
    s[4 * g + 2] = ab_p - cd_p;
    s[4 * g + 3] = ab_m - cd_m;
  }
#pragma unroll
  for (int b = 4; b <= 8; b <<= 1) {  // element bits 2 and 3
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      if (j & b) continue;
      const float p = s[j] + s[j + b], m = s[j] - s[j + b];
      s[j] = p;
      s[j + b] = m;
    }
  }
#pragma unroll
  for (int b = 0; b < 3; ++b) {  // element bits 4-6; fma(s, -1, p) is p - s exactly
    const float sign = (l & (1 << b)) ? -1.0f : 1.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) s[j] = __builtin_fmaf(s[j], sign, xor_partner(s[j], kLane8Xor[b]));
  }
}

// quantize_row for sixteen elements per lane; returns the lane's four words (elements
// 16l..16l+15, low byte first). The code is clamp(rne(p), +-127) with p = r * inv, formed as
// rne(clamp(p, +-127)) (the same integer for every p, NaN included: both give -127) by adding
// 1.5 * 2^23: the sum is rounded to an integer, ties to even, and the low byte of its bits is
// the code in two's complement.
__device__ __forceinline__ uint4 quantize_row16(const float (&r)[16], float extra, float* scale) {
  float m = 0.0f;
#pragma unroll
  for (int j = 0; j < 16; ++j) m = fmaxf(m, fabsf(r[j]));
  m = row8_max(m);
  const float amax = fmaxf(m, 1.0000000000000001e-30f);
  const float sc = amax / 127.0f;
  const float inv = 127.0f / amax;
  uint32_t b[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const float q = fminf(fmaxf(r[j] * inv, -127.0f), 127.0f);
    b[j] = __float_as_uint(q + 12582912.0f);
  }
  uint32_t w[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t lo = __builtin_amdgcn_perm(b[4 * k + 1], b[4 * k], 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm(b[4 * k + 3], b[4 * k + 2], 0x04000c0cu);
    w[k] = lo | hi;
  }
  *scale = sc * extra;
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// The int4 form (kernels/prepare_qk_i4.loom:174-214) for sixteen elements per lane: amax/7
// scales, codes clamp(rne(r*7/amax), +-7) formed as quantize_row16 forms its bytes; returns the
// lane's two words of nibbles (elements 16l..16l+7 and 16l+8..16l+15, low nibble first).
__device__ __forceinline__ uint2 quantize_row16_i4(const float (&r)[16], float extra,
                                                   float* scale) {
  float m = 0.0f;
#pragma unroll
  for (int j = 0; j < 16; ++j) m = fmaxf(m, fabsf(r[j]));
  m = row8_max(m);
  const float amax = fmaxf(m, 1.0000000000000001e-30f);
  const float sc = amax / 7.0f;
  const float inv = 7.0f / amax;
  uint32_t w[2] = {0u, 0u};
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const float q = fminf(fmaxf(r[j] * inv, -7.0f), 7.0f);
    w[j / 8] |= (__float_as_uint(q + 12582912.0f) & 0xfu) << (4 * (j % 8));
  }
  *scale = sc * extra;
  return make_uint2(w[0], w[1]);
}

// (token, head) rows (kernels/prepare_qk_i8.loom, prepare_qk_i8hm.loom; with kI4 the token-major
// int4 operands of kernels/prepare_qk_i4.loom, codes [tokens][heads*16] i32), one per 8-lane
// group; group g of block b takes rows b*32*kRowsAhead + 32i + g, i < kRowsAhead, all loads
// issued before the first row is processed. Head-major rows walk tokens fastest (contiguous code
// stores), token-major rows walk heads.
template <bool kHeadMajor, int kElem, bool kMean, bool kI4 = false>
__global__ __launch_bounds__(256) void k_prepare_qk(const void* __restrict__ x,
                                                    const float* __restrict__ mean,
                                                    int32_t* __restrict__ codes,
                                                    float* __restrict__ scales, uint32_t tokens,
                                                    uint32_t row_stride, uint32_t head_offset,
                                                    uint32_t heads, uint32_t capacity,
                                                    float extra) {
  const int lane = threadIdx.x & 63;
  const int l = local8(lane);
  const uint32_t first =
      blockIdx.x * kRopeGroups * kRowsAhead + 8 * (threadIdx.x >> 6) + group8(lane);
  const uint32_t total = tokens * heads;
  uint4 in[kRowsAhead][2];
#pragma unroll
  for (int i = 0; i < kRowsAhead; ++i) {
    const uint32_t row = first + kRopeGroups * i;
    if (row >= total) break;
    const uint32_t t = kHeadMajor ? row % tokens : row / heads;
    const uint32_t h = kHeadMajor ? row / tokens : row % heads;
    const size_t at = (size_t)t * row_stride + head_offset + 128u * h + 16u * l;
    in[i][0] = load8(x, at);
    in[i][1] = load8(x, at + 8);
  }
#pragma unroll
  for (int i = 0; i < kRowsAhead; ++i) {
    const uint32_t row = first + kRopeGroups * i;
    if (row >= total) break;
    const uint32_t t = kHeadMajor ? row % tokens : row / heads;
    const uint32_t h = kHeadMajor ? row / tokens : row % heads;
    float y[16];
    {
      float lo8[8], hi8[8];
      widen8(in[i][0], kElem, lo8);
      widen8(in[i][1], kElem, hi8);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        y[j] = lo8[j];
        y[8 + j] = hi8[j];
      }
    }
    if (kMean) {
      const float* mc = mean + head_offset + 128u * h + 16u * l;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 m4 = *reinterpret_cast<const float4*>(mc + 4 * q);
        y[4 * q] = y[4 * q] - m4.x;
        y[4 * q + 1] = y[4 * q + 1] - m4.y;
        y[4 * q + 2] = y[4 * q + 2] - m4.z;
        y[4 * q + 3] = y[4 * q + 3] - m4.w;
      }
    }
    hadamard128_16(y, l);
    float scale;
    const size_t out_row = kHeadMajor ? (size_t)h * capacity + t : (size_t)t * heads + h;
    if constexpr (kI4) {
      reinterpret_cast<uint2*>(codes + out_row * 16)[l] = quantize_row16_i4(y, extra, &scale);
    } else {
      reinterpret_cast<uint4*>(codes + out_row * 32)[l] = quantize_row16(y, extra, &scale);
    }
    if (l == 0) scales[out_row] = scale;
  }
}

// RMSNorm + RoPE + f16 rounding + (optional mean subtraction) + quantizer, head-major output
// (kernels/prepare_qk_rope_i8hm.loom:94-239; mean == nullptr is the reference's unsmoothed
// kernel, a mean is this build's fused K-smoothing second pass). One 8-lane group owns one token
// and walks its heads with kRowsAhead heads in flight: the token's RoPE tables are read once
// (not once per head), its heads' inputs are one contiguous run of the fused row, and the 32
// groups of a workgroup write 32 consecutive head-major rows (4 KiB) per head. Group g of wave w
// takes token 32 * block + 8w + g.
template <int kElem, bool kMean>
__global__ __launch_bounds__(256) void k_prepare_qk_rope(
    const void* __restrict__ x, const float* __restrict__ weight, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, const float* __restrict__ mean, int32_t* __restrict__ codes,
    float* __restrict__ scales, uint32_t tokens, uint32_t row_stride, uint32_t head_offset,
    uint32_t heads, uint32_t capacity, float extra, float eps) {
  const int lane = threadIdx.x & 63;
  const uint32_t t = blockIdx.x * kRopeGroups + 8 * (threadIdx.x >> 6) + group8(lane);
  const int l = local8(lane);
  if (t >= tokens) return;
  const RopeLane16 tab = rope_lane16(l, weight, cos_t + (size_t)t * 48, sin_t + (size_t)t * 48);
  const size_t row0 = (size_t)t * row_stride + head_offset + 16u * l;
  uint4 ring[kRowsAhead][2];  // heads h .. h + kRowsAhead - 1 in flight
#pragma unroll
  for (int i = 0; i < kRowsAhead; ++i)
    if ((uint32_t)i < heads) {
      ring[i][0] = load8(x, row0 + 128u * i);
      ring[i][1] = load8(x, row0 + 128u * i + 8);
    }
  for (uint32_t h0 = 0; h0 < heads; h0 += kRowsAhead) {
#pragma unroll
    for (int i = 0; i < kRowsAhead; ++i) {
      const uint32_t h = h0 + i;
      if (h >= heads) break;
      float y[16];
      {
        float lo8[8], hi8[8];
        widen8(ring[i][0], kElem, lo8);
        widen8(ring[i][1], kElem, hi8);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          y[j] = lo8[j];
          y[8 + j] = hi8[j];
        }
      }
      if (h + kRowsAhead < heads) {
        ring[i][0] = load8(x, row0 + 128u * (h + kRowsAhead));
        ring[i][1] = load8(x, row0 + 128u * (h + kRowsAhead) + 8);
      }
      float4 mu[4];  // the column means, loaded before the norm so that they land under it
      if (kMean) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          mu[q] = *reinterpret_cast<const float4*>(mean + 128u * h + 16u * l + 4 * q);
      }
      rmsnorm_rope16(y, lane, l, tab, eps);
      if (kMean) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          y[4 * q] = y[4 * q] - mu[q].x;
          y[4 * q + 1] = y[4 * q + 1] - mu[q].y;
          y[4 * q + 2] = y[4 * q + 2] - mu[q].z;
          y[4 * q + 3] = y[4 * q + 3] - mu[q].w;
        }
      }
      hadamard128_16(y, l);
      float scale;
      const uint4 w = quantize_row16(y, extra, &scale);
      const size_t out_row = (size_t)h * capacity + t;
      reinterpret_cast<uint4*>(codes + out_row * 32)[l] = w;
      if (l == 0) scales[out_row] = scale;
    }
  }
}

// RMSNorm + RoPE of Q and K heads to f16, V optionally copied (kernels/rope_qknorm_f16.loom).
// Rows are (token, head) over heads + kv_heads (+ kv_heads copy rows).
__global__ __launch_bounds__(256) void k_rope_qknorm(
    const void* __restrict__ x, const float* __restrict__ qweight,
    const float* __restrict__ kweight, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_out,
    uint16_t* __restrict__ v_out, uint32_t tokens, uint32_t row_stride, uint32_t heads,
    uint32_t kv_heads, uint32_t k_offset, float eps, uint32_t elem, uint32_t copy_v) {
  const uint32_t per_token = heads + kv_heads + (copy_v ? kv_heads : 0);
  const uint32_t row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 5);
  const int lane = threadIdx.x & 31;
  if (row >= tokens * per_token) return;
  const uint32_t t = row / per_token;
  const uint32_t j = row % per_token;
  if (j >= heads + kv_heads) {  // V copy: bits unchanged (bf16 input is rounded to f16)
    const uint32_t vh = j - heads - kv_heads;
    const uint32_t col = k_offset + 128u * kv_heads + 128u * vh + 4u * lane;
    uint2 bits = load4(x, (size_t)t * row_stride + col);
    if (elem == H3_ELEM_BF16) {
      v4f f = widen4(bits, elem);
      v4h hv = {(_Float16)f[0], (_Float16)f[1], (_Float16)f[2], (_Float16)f[3]};
      bits = __builtin_bit_cast(uint2, hv);
    }
    *reinterpret_cast<uint2*>(v_out + (size_t)t * kv_heads * 128 + 128u * vh + 4u * lane) = bits;
    return;
  }
  const bool is_q = j < heads;
  const uint32_t h = is_q ? j : j - heads;
  const uint32_t col = (is_q ? 0u : k_offset) + 128u * h + 4u * lane;
  v4f v = widen4(load4(x, (size_t)t * row_stride + col), elem);
  v4f o = rmsnorm_rope_f16(v, lane, is_q ? qweight : kweight, cos_t + (size_t)t * 48,
                           sin_t + (size_t)t * 48, eps);
  v4h hv = {(_Float16)o[0], (_Float16)o[1], (_Float16)o[2], (_Float16)o[3]};
  uint16_t* dst = is_q ? q_out + (size_t)t * heads * 128 : k_out + (size_t)t * kv_heads * 128;
  *reinterpret_cast<v4h*>(dst + 128u * h + 4u * lane) = hv;
}

// ---------------------------------------------------------------- column means

// mean[c] = (sum_t x[t][c]) / tokens, one lane per column summing tokens in order
// (kernels/colmean_f32.loom in-file 30-40). Eight loads are issued ahead of the dependent adds.
__global__ __launch_bounds__(64) void k_colmean(const void* __restrict__ x,
                                                float* __restrict__ mean, uint32_t tokens,
                                                uint32_t width, uint32_t row_stride,
                                                uint32_t elem) {
  const uint32_t c = blockIdx.x * 64 + threadIdx.x;
  if (c >= width) return;
  const uint16_t* p = reinterpret_cast<const uint16_t*>(x) + c;
  float acc = 0.0f;
  uint32_t t = 0;
  constexpr int kAhead = 16;
  for (; t + kAhead <= tokens; t += kAhead) {
    uint16_t v[kAhead];
#pragma unroll
    for (int i = 0; i < kAhead; ++i) v[i] = p[(size_t)(t + i) * row_stride];
#pragma unroll
    for (int i = 0; i < kAhead; ++i)
      acc = acc + (elem == H3_ELEM_BF16 ? __uint_as_float((uint32_t)v[i] << 16)
                                        : (float)__builtin_bit_cast(_Float16, v[i]));
  }
  for (; t < tokens; ++t) {
    uint16_t v = p[(size_t)t * row_stride];
    acc = acc + (elem == H3_ELEM_BF16 ? __uint_as_float((uint32_t)v << 16)
                                      : (float)__builtin_bit_cast(_Float16, v));
  }
  mean[c] = acc / (float)tokens;
}

// The fused K smoothing's column mean: mean[c] = (sum_t rope(K)[t][c]) / tokens, where rope(K) is
// RMSNorm+RoPE of K rounded to f16 (exactly what h3_rope_qknorm_f16 writes) and the sum runs in
// token order in fp32, one dependent add per token (kernels/colmean_f32.loom in-file 30-40). The
// add chain of each column is inherently sequential; everything feeding it is spread out.
//
// Pass 1 (k_rope_rms): r of every (token, head) row into a float buffer [heads][capacity] (the
// scales binding, which the quantizer pass then overwrites). One row per 16-lane group, eight
// channels per lane (rms_inverse8, the same bits as the four-channel layout). A workgroup takes
// kRmsTokens consecutive tokens; group g walks heads g, g + 16, ... and for each loads that
// head's row of all kRmsTokens tokens before reducing any (16 rows, 64 KiB per workgroup in
// flight), so the 16 groups read whole contiguous runs of the fused rows. Lane i of the group
// then stores token i's r: one 64-byte store per head.
constexpr int kRmsTokens = 16;
template <int kElem>
__global__ __launch_bounds__(256) void k_rope_rms(const void* __restrict__ x,
                                                  float* __restrict__ r_out, uint32_t tokens,
                                                  uint32_t heads, uint32_t row_stride,
                                                  uint32_t head_offset, uint32_t capacity,
                                                  float eps) {
  const int g = threadIdx.x >> 4, l = threadIdx.x & 15;
  const uint32_t t0 = blockIdx.x * kRmsTokens;
  for (uint32_t h = g; h < heads; h += kGroupsPerBlock) {
    uint4 raw[kRmsTokens];
#pragma unroll
    for (int i = 0; i < kRmsTokens; ++i) {
      const uint32_t t = min(t0 + i, tokens - 1);  // every lane stays in the butterfly
      raw[i] = load8_nt(x, (size_t)t * row_stride + head_offset + 128u * h + 8u * l);
    }
    float mine = 0.0f;
#pragma unroll
    for (int i = 0; i < kRmsTokens; ++i) {
      float v[8];
      widen8(raw[i], kElem, v);
      const float r = rms_inverse8(v, eps);
      mine = l == i ? r : mine;
    }
    if (t0 + l < tokens) r_out[(size_t)h * capacity + t0 + l] = mine;
  }
}

// Pass 2 (k_rope_colmean): one workgroup per 16 channels of one head (8 per head, 256 at 32
// heads). Workgroups 0-5 of a head own rotation pairs: channels 8k..8k+7 and 48+8k..48+8k+7,
// which are each other's RoPE partners and share cos/sin columns 8k..8k+7, so every input byte is
// loaded once; workgroups 6 and 7 own channels 96-111 and 112-127 (not rotated). Eight waves:
// lanes 0-15 of wave 0 each run one channel's add chain over an LDS tile; wave 4 (the other wave
// on wave 0's SIMD) only joins the barriers, so the chain has its SIMD to itself; the six other
// waves (384 producer threads, one token each per 384-token chunk) compute the f16 RoPE values
// into the double-buffered tile. Producers keep three chunks of raw inputs in registers and load
// each chunk two chunks ahead, so the chain (tokens dependent adds) stays the critical path. The
// eight workgroups of a head are placed on one XCD so that the rows they read share an L2.
constexpr int kSlab = 16;                        // channels per workgroup
constexpr int kSlabs = 128 / kSlab;              // workgroups per head
constexpr int kColmeanThreads = 512;
constexpr int kChunk = 384;                      // tokens per chunk = producer threads
constexpr int kChunkPad = kChunk + 4;            // floats per LDS column (a 16-byte multiple)
constexpr int kRing = 3;                         // chunks of raw inputs held per producer

struct PairToken {  // the raw inputs of one token for a workgroup's 16 channels
  uint4 a, b;       // channels of the first and second group of eight (16-bit bit patterns)
  float4 c[2], s[2];  // cos/sin of the pair's eight table columns (rotated workgroups only)
  float r;
};

__device__ __forceinline__ void load_pair_token(PairToken& in, const void* x, const float* r_in,
                                                const float* cos_t, const float* sin_t,
                                                uint32_t t, uint32_t tokens, size_t col_a,
                                                size_t col_b, uint32_t row_stride,
                                                size_t r_base, uint32_t tab0, bool rotated) {
  if (t >= tokens) return;  // past the sequence: never consumed
  const uint16_t* row = reinterpret_cast<const uint16_t*>(x) + (size_t)t * row_stride;
  in.a = *reinterpret_cast<const uint4*>(row + col_a);
  in.b = *reinterpret_cast<const uint4*>(row + col_b);
  in.r = r_in[r_base + t];
  if (rotated) {
    const float* ct = cos_t + (size_t)t * 48 + tab0;
    const float* st = sin_t + (size_t)t * 48 + tab0;
    in.c[0] = *reinterpret_cast<const float4*>(ct);
    in.c[1] = *reinterpret_cast<const float4*>(ct + 4);
    in.s[0] = *reinterpret_cast<const float4*>(st);
    in.s[1] = *reinterpret_cast<const float4*>(st + 4);
  }
}

__device__ __forceinline__ void unpack8(uint4 b, uint32_t elem, float (&v)[8]) {
  const v4f lo = widen4(make_uint2(b.x, b.y), elem), hi = widen4(make_uint2(b.z, b.w), elem);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[j] = lo[j];
    v[4 + j] = hi[j];
  }
}

__global__ __launch_bounds__(kColmeanThreads) void k_rope_colmean(
    const void* __restrict__ x, const float* __restrict__ weight, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, const float* __restrict__ r_in, float* __restrict__ mean,
    uint32_t tokens, uint32_t row_stride, uint32_t head_offset, uint32_t capacity,
    uint32_t total, uint32_t per_xcd, uint32_t elem) {
  __shared__ __align__(16) float tile[2][kSlab][kChunkPad];
  const uint32_t b = blockIdx.x;
  const uint32_t logical = (b % 8) * per_xcd + b / 8;  // workgroup b runs on XCD b % 8
  if (logical >= total) return;                       // whole workgroup, before any barrier
  const uint32_t h = logical / kSlabs, k = logical % kSlabs;
  const bool rotated = k < 6;
  // channels of tile rows 0-7 and 8-15
  const uint32_t ca = rotated ? 8 * k : 96 + 16 * (k - 6);
  const uint32_t cb = rotated ? ca + 48 : ca + 8;
  const size_t col_a = head_offset + 128u * h + ca, col_b = head_offset + 128u * h + cb;
  const size_t r_base = (size_t)h * capacity;
  const uint32_t chunks = (tokens + kChunk - 1) / kChunk;
  const int wave = threadIdx.x >> 6;
  const bool producer = wave != 0 && wave != 4;
  const int p = (wave < 4 ? wave - 1 : wave - 2) * 64 + (threadIdx.x & 63);  // 0..383

  float wa[8], wb[8];
  PairToken ring[kRing];
  auto load = [&](PairToken& in, uint32_t j) {
    load_pair_token(in, x, r_in, cos_t, sin_t, j * kChunk + p, tokens, col_a, col_b, row_stride,
                    r_base, 8 * k, rotated);
  };
  // Chunk j's values into tile buffer j % 2: the operations of rmsnorm_rope_f16, channel by
  // channel (rope_channel), so the values are bit-identical to h3_rope_qknorm_f16's output.
  auto store = [&](const PairToken& in, uint32_t j) {
    if (j * kChunk + p >= tokens) return;
    float (*dst)[kChunkPad] = tile[j & 1];
    float va[8], vb[8];
    unpack8(in.a, elem, va);
    unpack8(in.b, elem, vb);
    if (rotated) {
      const float cc[8] = {in.c[0].x, in.c[0].y, in.c[0].z, in.c[0].w,
                           in.c[1].x, in.c[1].y, in.c[1].z, in.c[1].w};
      const float ss[8] = {in.s[0].x, in.s[0].y, in.s[0].z, in.s[0].w,
                           in.s[1].x, in.s[1].y, in.s[1].z, in.s[1].w};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        dst[i][p] = rope_channel(va[i], vb[i], in.r, wa[i], wb[i], cc[i], ss[i], true, true);
        dst[8 + i][p] = rope_channel(vb[i], va[i], in.r, wb[i], wa[i], cc[i], ss[i], false, true);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        dst[i][p] = rope_channel(va[i], 0.0f, in.r, wa[i], 0.0f, 0.0f, 0.0f, false, false);
        dst[8 + i][p] = rope_channel(vb[i], 0.0f, in.r, wb[i], 0.0f, 0.0f, 0.0f, false, false);
      }
    }
  };

  if (producer) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      wa[i] = weight[ca + i];
      wb[i] = weight[cb + i];
    }
#pragma unroll
    for (int i = 0; i < kRing; ++i)
      if ((uint32_t)i < chunks) load(ring[i], i);
    store(ring[0], 0);
  }
  __syncthreads();

  float acc = 0.0f;
  const int lane = threadIdx.x;  // the chain lanes (wave 0, lanes 0-15)
  // One chunk: producers store chunk j + 1 and load chunk j + 3 into the ring slot chunk j
  // left; lanes 0-15 add chunk j. Slot indices are compile-time (the loop is unrolled by kRing).
  auto chunk = [&](uint32_t j, auto slot) {
    constexpr int kNext = (decltype(slot)::value + 1) % kRing;
    if (producer && j + 1 < chunks) {
      store(ring[kNext], j + 1);
      if (j + kRing < chunks) load(ring[decltype(slot)::value], j + kRing);
    }
    if (threadIdx.x < kSlab) {
      const float* col = tile[j & 1][lane];
      const uint32_t n = min((uint32_t)kChunk, tokens - j * kChunk);
      if (n == kChunk) {
        float4 cur[8], nxt[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) cur[i] = *reinterpret_cast<const float4*>(col + 4 * i);
        for (int g = 0; g < kChunk / 32; ++g) {
          if (g + 1 < kChunk / 32) {
#pragma unroll
            for (int i = 0; i < 8; ++i)
              nxt[i] = *reinterpret_cast<const float4*>(col + 32 * (g + 1) + 4 * i);
          }
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            acc = acc + cur[i].x;
            acc = acc + cur[i].y;
            acc = acc + cur[i].z;
            acc = acc + cur[i].w;
          }
#pragma unroll
          for (int i = 0; i < 8; ++i) cur[i] = nxt[i];
        }
      } else {
        for (uint32_t i = 0; i < n; ++i) acc = acc + col[i];
      }
    }
    __syncthreads();
  };
  uint32_t j = 0;
  for (; j + kRing <= chunks; j += kRing) {
    chunk(j, std::integral_constant<int, 0>{});
    chunk(j + 1, std::integral_constant<int, 1>{});
    chunk(j + 2, std::integral_constant<int, 2>{});
  }
  if (j < chunks) chunk(j, std::integral_constant<int, 0>{});
  if (j + 1 < chunks) chunk(j + 1, std::integral_constant<int, 1>{});
  if (threadIdx.x < kSlab) {
    const uint32_t c = lane < 8 ? ca + lane : cb + (lane - 8);
    mean[128u * h + c] = acc / (float)tokens;
  }
}

// ---------------------------------------------------------------- transposes

// x [rows][row_stride] (width columns at col_offset) -> out [width][capacity] f16 through a
// 64x64 LDS tile (rows padded to 66 halves). Output columns [rows, clear_to) are zeroed,
// columns >= clear_to are left alone (kernels/transpose_f16.loom, transpose_qkv_v_f16.loom).
// kGather: row r of the input is row src[r] of x (a zero row where src[r] >= src_rows), and each
// loaded piece is also written, as loaded, to gathered[r][c] (the VSA runtime's gathered v,
// [rows][width], and its V^T from one read of x).
template <bool kGather>
__global__ __launch_bounds__(256) void k_transpose(const uint16_t* __restrict__ x,
                                                   uint16_t* __restrict__ out, uint32_t rows,
                                                   uint32_t clear_to, uint32_t width,
                                                   uint32_t capacity, uint32_t row_stride,
                                                   uint32_t col_offset, uint32_t elem,
                                                   const int32_t* __restrict__ src,
                                                   uint32_t src_rows,
                                                   uint16_t* __restrict__ gathered) {
  __shared__ uint16_t tile[64][64 + 2];
  const uint32_t c0 = blockIdx.x * 64, r0 = blockIdx.y * 64;
  // load: 64 rows x 64 columns, lane -> row i/16 (+16k), columns 4*(i%16)..+3
  const int lr = threadIdx.x >> 4, lc = (threadIdx.x & 15) * 4;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t r = r0 + lr + 16 * k;
    const uint32_t c = c0 + lc;
    uint16_t v[4] = {0, 0, 0, 0};
    if (r < rows && c < width) {
      uint2 bits;
      if (kGather) {
        const uint32_t sr = (uint32_t)src[r];
        bits = sr < src_rows
                   ? *reinterpret_cast<const uint2*>(x + (size_t)sr * row_stride + col_offset + c)
                   : make_uint2(0u, 0u);
        *reinterpret_cast<uint2*>(gathered + (size_t)r * width + c) = bits;
      } else {
        bits = *reinterpret_cast<const uint2*>(x + (size_t)r * row_stride + col_offset + c);
      }
      if (elem == H3_ELEM_BF16) {
        v4f f = widen4(bits, elem);
        v4h hv = {(_Float16)f[0], (_Float16)f[1], (_Float16)f[2], (_Float16)f[3]};
        bits = __builtin_bit_cast(uint2, hv);
      }
      v[0] = bits.x & 0xffff;
      v[1] = bits.x >> 16;
      v[2] = bits.y & 0xffff;
      v[3] = bits.y >> 16;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) tile[lr + 16 * k][lc + j] = v[j];
  }
  __syncthreads();
  // store: output row (channel) c0 + i/16 (+16k), output columns r0 + 4*(i%16)..+3
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t oc = c0 + lr + 16 * k;
    const uint32_t orow = r0 + lc;
    if (oc >= width) continue;
    uint16_t v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = tile[lc + j][lr + 16 * k];
    uint16_t* dst = out + (size_t)oc * capacity + orow;
    if (orow + 4 <= clear_to) {
      *reinterpret_cast<uint2*>(dst) =
          make_uint2((uint32_t)v[0] | ((uint32_t)v[1] << 16), (uint32_t)v[2] | ((uint32_t)v[3] << 16));
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (orow + j < clear_to) dst[j] = v[j];
    }
  }
}

inline uint32_t div_up(uint32_t a, uint32_t b) { return (a + b - 1) / b; }

}  // namespace

hipError_t launch_prepare_qk(const h3_prepare_cfg& cfg, uint32_t tokens, int head_major,
                             const void* x, const float* mean, int32_t* codes, float* scales,
                             hipStream_t stream) {
  const uint32_t rows = tokens * cfg.heads;
  const dim3 grid(div_up(rows, kRopeGroups * kRowsAhead));
  const uint32_t cap = head_major ? cfg.token_capacity : 0u;
  auto launch = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid, dim3(256), 0, stream, x, mean, codes, scales, tokens,
                       cfg.row_stride, cfg.head_offset, cfg.heads, cap, cfg.extra_scale);
  };
  // every (layout, element, mean) combination as its own kernel
  const int pick = (head_major ? 4 : 0) | (cfg.elem == H3_ELEM_BF16 ? 2 : 0) | (mean ? 1 : 0);
  switch (pick) {
    case 0: launch(k_prepare_qk<false, H3_ELEM_F16, false>); break;
    case 1: launch(k_prepare_qk<false, H3_ELEM_F16, true>); break;
    case 2: launch(k_prepare_qk<false, H3_ELEM_BF16, false>); break;
    case 3: launch(k_prepare_qk<false, H3_ELEM_BF16, true>); break;
    case 4: launch(k_prepare_qk<true, H3_ELEM_F16, false>); break;
    case 5: launch(k_prepare_qk<true, H3_ELEM_F16, true>); break;
    case 6: launch(k_prepare_qk<true, H3_ELEM_BF16, false>); break;
    default: launch(k_prepare_qk<true, H3_ELEM_BF16, true>); break;
  }
  return hipGetLastError();
}

hipError_t launch_prepare_qk_i4(const h3_prepare_cfg& cfg, uint32_t tokens, const void* x,
                                const float* mean, int32_t* codes, float* scales,
                                hipStream_t stream) {
  const uint32_t rows = tokens * cfg.heads;
  const dim3 grid(div_up(rows, kRopeGroups * kRowsAhead));
  auto launch = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid, dim3(256), 0, stream, x, mean, codes, scales, tokens,
                       cfg.row_stride, cfg.head_offset, cfg.heads, 0u, cfg.extra_scale);
  };
  const int pick = (cfg.elem == H3_ELEM_BF16 ? 2 : 0) | (mean ? 1 : 0);
  switch (pick) {
    case 0: launch(k_prepare_qk<false, H3_ELEM_F16, false, true>); break;
    case 1: launch(k_prepare_qk<false, H3_ELEM_F16, true, true>); break;
    case 2: launch(k_prepare_qk<false, H3_ELEM_BF16, false, true>); break;
    default: launch(k_prepare_qk<false, H3_ELEM_BF16, true, true>); break;
  }
  return hipGetLastError();
}

hipError_t launch_prepare_qk_rope(const h3_prepare_cfg& cfg, uint32_t tokens, const void* x,
                                  const float* weight, const float* cos_t, const float* sin_t,
                                  int32_t* codes, float* scales, hipStream_t stream) {
  return launch_prepare_qk_rope_mean(cfg, tokens, x, weight, cos_t, sin_t, nullptr, codes, scales,
                                     stream);
}

hipError_t launch_prepare_qk_rope_mean(const h3_prepare_cfg& cfg, uint32_t tokens, const void* x,
                                       const float* weight, const float* cos_t,
                                       const float* sin_t, const float* mean, int32_t* codes,
                                       float* scales, hipStream_t stream) {
  const dim3 grid(div_up(tokens, kRopeGroups));
  auto launch = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid, dim3(256), 0, stream, x, weight, cos_t, sin_t, mean, codes,
                       scales, tokens, cfg.row_stride, cfg.head_offset, cfg.heads,
                       cfg.token_capacity, cfg.extra_scale, cfg.eps);
  };
  const bool bf16 = cfg.elem == H3_ELEM_BF16;
  if (mean)
    bf16 ? launch(k_prepare_qk_rope<H3_ELEM_BF16, true>) : launch(k_prepare_qk_rope<H3_ELEM_F16, true>);
  else
    bf16 ? launch(k_prepare_qk_rope<H3_ELEM_BF16, false>) : launch(k_prepare_qk_rope<H3_ELEM_F16, false>);
  return hipGetLastError();
}

hipError_t launch_rope_qknorm(const h3_rope_cfg& cfg, uint32_t tokens, const void* x,
                              const float* qweight, const float* kweight, const float* cos_t,
                              const float* sin_t, uint16_t* q_out, uint16_t* k_out,
                              uint16_t* v_out, hipStream_t stream) {
  const uint32_t per_token = cfg.heads + cfg.kv_heads + (cfg.copy_v ? cfg.kv_heads : 0);
  hipLaunchKernelGGL(k_rope_qknorm, dim3(div_up(tokens * per_token, kRowsPerBlock)), dim3(256), 0,
                     stream, x, qweight, kweight, cos_t, sin_t, q_out, k_out, v_out, tokens,
                     cfg.row_stride, cfg.heads, cfg.kv_heads, cfg.k_offset, cfg.eps, cfg.elem,
                     cfg.copy_v);
  return hipGetLastError();
}

hipError_t launch_colmean(uint32_t width, uint32_t row_stride, uint32_t elem, uint32_t tokens,
                          const void* x, float* mean, hipStream_t stream) {
  hipLaunchKernelGGL(k_colmean, dim3(div_up(width, 64)), dim3(64), 0, stream, x, mean, tokens,
                     width, row_stride, elem);
  return hipGetLastError();
}

hipError_t launch_rope_colmean(const h3_prepare_cfg& cfg, uint32_t tokens, const void* x,
                               const float* weight, const float* cos_t, const float* sin_t,
                               float* r_scratch, float* mean, hipStream_t stream) {
  const dim3 rms_grid(div_up(tokens, kRmsTokens));
  if (cfg.elem == H3_ELEM_BF16)
    hipLaunchKernelGGL(k_rope_rms<H3_ELEM_BF16>, rms_grid, dim3(256), 0, stream, x, r_scratch,
                       tokens, cfg.heads, cfg.row_stride, cfg.head_offset, cfg.token_capacity,
                       cfg.eps);
  else
    hipLaunchKernelGGL(k_rope_rms<H3_ELEM_F16>, rms_grid, dim3(256), 0, stream, x, r_scratch,
                       tokens, cfg.heads, cfg.row_stride, cfg.head_offset, cfg.token_capacity,
                       cfg.eps);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const uint32_t total = cfg.heads * kSlabs, per_xcd = div_up(total, 8);
  hipLaunchKernelGGL(k_rope_colmean, dim3(8 * per_xcd), dim3(kColmeanThreads), 0, stream, x,
                     weight, cos_t,
                     sin_t, r_scratch, mean, tokens, cfg.row_stride, cfg.head_offset,
                     cfg.token_capacity, total, per_xcd, cfg.elem);
  return hipGetLastError();
}

hipError_t launch_transpose(uint32_t width, uint32_t row_capacity, uint32_t row_stride,
                            uint32_t col_offset, uint32_t elem, uint32_t tile, uint32_t launch_rows,
                            uint32_t rows, const void* x, uint16_t* out, hipStream_t stream) {
  uint32_t clear_to = div_up(launch_rows, tile) * tile;
  if (clear_to > row_capacity) clear_to = row_capacity;
  if (clear_to == 0) return hipSuccess;
  dim3 grid(div_up(width, 64), div_up(clear_to, 64));
  hipLaunchKernelGGL(k_transpose<false>, grid, dim3(256), 0, stream,
                     reinterpret_cast<const uint16_t*>(x), out, rows, clear_to, width,
                     row_capacity, row_stride, col_offset, elem, nullptr, 0u, nullptr);
  return hipGetLastError();
}

hipError_t launch_gather_transpose(uint32_t width, uint32_t rows, const int32_t* src,
                                   uint32_t src_rows, const uint16_t* x, uint16_t* gathered,
                                   uint16_t* out, hipStream_t stream) {
  // rows is a multiple of 64 (the VSA layout's padded row count), so every row is loaded
  dim3 grid(div_up(width, 64), div_up(rows, 64));
  hipLaunchKernelGGL(k_transpose<true>, grid, dim3(256), 0, stream, x, out, rows, rows, width,
                     rows, width, 0u, (uint32_t)H3_ELEM_F16, src, src_rows, gathered);
  return hipGetLastError();
}

}  // namespace h3
