// INT8 QKV projection with the compact Q/K-rows + V^T epilogue, on gfx950 int8 MFMA.
//
// Semantics follow kernels/gemm_packed_256.loom:14-412 instantiated as h3_gemm_i8_qkv_256
// (kernels/gemm_packed_256.loom:3429-3471; dispatch src/dispatch.rs:756-790 and 1025-1060):
//   acc[m][n]  = sum_k a[m][k] * w[n][k]                       (int8 x int8, exact int32)
//   v          = ((float)acc * w_scale[n]) * a_scale[m] + 0.0   (three IEEE f32 operations)
//   v          = clamp(v, -65472, 65472) when v is finite; inf and NaN pass unchanged
//   columns n < 2N/3 (Q and K): out[m][n], row pitch 2N/3 f16
//   columns n >= 2N/3 (V):      vt[n - 2N/3][m] at element offset M*2N/3, row pitch
//                               cap = ceil(M/256)*256; rows M <= m < cap are written as zero.
// That layout is what Stack::prepare_fused_operands reads on the compact route
// (src/stack.rs:634-661, 1034-1040, 1561-1600): Q/K rows for the RoPE quantizer with a row
// stride of 2*inner, V^T already in the attention's operand layout, no transpose pass.
//
// Design. A workgroup computes a 256 x 256 tile with 8 waves (2 along M x 4 along N, 128 x 64
// each: 4 x 2 blocks of v_mfma_i32_32x32x32_i8). K advances 128 bytes per step through two
// LDS stages of 64 KiB (256 A rows + 256 W rows of 128 bytes), filled by LDS-DMA
// (buffer_load ... lds) one step ahead; rows are 16-byte chunks XOR-swizzled by (row/2)%8 so the
// 32 rows a half-wave reads hit distinct banks. Buffer descriptors end at the last valid row,
// so rows past M (or past N) load as zero. The operand order of the MFMA is chosen per region
// so each lane ends up holding four consecutive output elements along the stored direction:
// W.A^T for Q/K tiles (4 consecutive channels of one token) and A.W^T for V tiles (4
// consecutive tokens of one channel), each written as one 8-byte store.
#include "internal.hpp"

namespace h3 {
namespace {

constexpr int kBM = 256;                       // tile rows (tokens)
constexpr int kBN = 256;                       // tile columns (output channels)
constexpr int kBK = 128;                       // K bytes per step
constexpr int kWaves = 8;                      // 2 (M) x 4 (N)
constexpr int kThreads = 64 * kWaves;
constexpr int kMB = 4;                         // 32-row blocks per wave along M (128 rows)
constexpr int kNB = 2;                         // 32-column blocks per wave along N (64 columns)
constexpr int kStage = (kBM + kBN) * kBK;      // 65536 bytes: A rows, then W rows
constexpr int kLoads = kStage / 1024 / kWaves;  // 1 KiB DMA loads per wave per step: 8
constexpr int kGroupM = 4;                     // m-tiles that share one sweep over the n-tiles
constexpr int kRsrcWord3 = 0x00020000;         // raw buffer, 32-bit data format, no swizzle

typedef __attribute__((address_space(3))) void lds_void;

struct Args {
  const int8_t* a;
  const int8_t* w;
  const float* ws;
  const float* as;
  uint16_t* out;
  uint32_t m;         // tokens
  uint32_t n;         // output channels (3 * inner)
  uint32_t k;         // reduction length (multiple of 64)
  uint32_t k_stride;  // bytes per operand row
  uint32_t qk_width;  // 2N/3: row pitch of the Q/K rows, first V channel
  uint32_t cap;       // ceil(M/256)*256: row pitch of V^T
  uint32_t tiles_m, tiles_n_qk, tiles_n, total, per_xcd;
};

// A buffer descriptor from wave-uniform values, read back from the first lane so that the
// compiler keeps it in scalar registers.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
  const uint64_t v = reinterpret_cast<uint64_t>(base);
  const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(lo | (hi << 32)), (short)0,
                                           __builtin_amdgcn_readfirstlane((int)bytes), kRsrcWord3);
}

// LDS byte offset, inside a 128-byte row, of logical 16-byte chunk c for swizzle sw.
__device__ __forceinline__ uint32_t chunk_off(uint32_t c, uint32_t sw) { return 16 * (c ^ sw); }

// f32 epilogue of one accumulator (kernels/gemm_packed_256.loom:370-397).
__device__ __forceinline__ _Float16 finish(int acc, float ws, float as) {
  float v = (float)acc * ws;
  v = v * as;
  v = v + 0.0f;
  if (__builtin_fabsf(v) < __builtin_inff()) v = __builtin_fminf(__builtin_fmaxf(v, -65472.0f), 65472.0f);
  return (_Float16)v;
}

// One K step on the stage `st`: kSteps MFMA substeps of 32 bytes each (4, or 2 for a final
// 64-byte remainder). Operands of substep s+1 are read while the MFMAs of substep s run.
template <bool kTrans, int kSteps>
__device__ __forceinline__ void mma_stage(const char* st, uint32_t arow, uint32_t wrow,
                                          uint32_t half, uint32_t sw, v16i (&acc)[kMB][kNB]) {
  v4i af[2][kMB], wf[2][kNB];
  auto load = [&](int buf, int ks) {
#pragma unroll
    for (int mb = 0; mb < kMB; ++mb)
      af[buf][mb] = *reinterpret_cast<const v4i*>(st + (arow + 32 * mb) * kBK +
                                                   chunk_off(2 * ks + half, sw));
#pragma unroll
    for (int nb = 0; nb < kNB; ++nb)
      wf[buf][nb] = *reinterpret_cast<const v4i*>(st + (kBM + wrow + 32 * nb) * kBK +
                                                   chunk_off(2 * ks + half, sw));
  };
  load(0, 0);
#pragma unroll
  for (int ks = 0; ks < kSteps; ++ks) {
    const int cur = ks & 1;
    if (ks + 1 < kSteps) load(cur ^ 1, ks + 1);
    __builtin_amdgcn_sched_barrier(0);  // the next substep's reads go out before these MFMAs
#pragma unroll
    for (int mb = 0; mb < kMB; ++mb)
#pragma unroll
      for (int nb = 0; nb < kNB; ++nb)
        acc[mb][nb] = kTrans ? __builtin_amdgcn_mfma_i32_32x32x32_i8(wf[cur][nb], af[cur][mb],
                                                                     acc[mb][nb], 0, 0, 0)
                             : __builtin_amdgcn_mfma_i32_32x32x32_i8(af[cur][mb], wf[cur][nb],
                                                                     acc[mb][nb], 0, 0, 0);
  }
}

template <bool kTrans>
__device__ __forceinline__ void tile(const Args& a, uint32_t m0, uint32_t n0, char* s0, char* s1) {
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t wave_m = wave >> 2, wave_n = wave & 3;
  const uint32_t half = lane >> 5;
  const uint32_t arow = wave_m * 128 + (lane & 31);  // A row of block 0 (stage row)
  const uint32_t wrow = wave_n * 64 + (lane & 31);   // W row of block 0 (stage row - 256)
  const uint32_t sw = (lane >> 1) & 7;               // (row/2)%8, the same for every block

  // DMA map: wave w fills stage rows 64w..64w+63 (waves 0-3: A, waves 4-7: W); lane l of load
  // t writes stage bytes (8w + t)*1024 + 16l, i.e. row r = (8w+t)*8 + l/8, position l%8, which
  // holds logical chunk (l%8) ^ ((r/2)%8).
  const bool is_a = wave < 4;
  const uint32_t rows_left = is_a ? (a.m > m0 ? min(a.m - m0, (uint32_t)kBM) : 0u)
                                  : (a.n > n0 ? min(a.n - n0, (uint32_t)kBN) : 0u);
  const int8_t* base = is_a ? a.a + (size_t)m0 * a.k_stride : a.w + (size_t)n0 * a.k_stride;
  const uint32_t bytes = rows_left * a.k_stride;
  uint32_t voff[kLoads];
#pragma unroll
  for (int t = 0; t < kLoads; ++t) {
    const uint32_t r = (8 * wave + t) * 8 + (lane >> 3);
    const uint32_t row = r & (kBM - 1);
    voff[t] = row * a.k_stride + 16 * ((lane & 7) ^ ((r >> 1) & 7));
  }
  // Step at K byte k0: the descriptor starts at k0 and ends at the last valid row's end, so
  // rows past the tile's valid ones read zero and nothing past the operand is addressed. In a
  // final 64-byte step the lanes of logical chunks 4..7 (bytes k0+64..k0+127, past K) are sent
  // out of range and write zeros.
  auto stage = [&](char* st, uint32_t k0, bool half_step) {
    const __amdgpu_buffer_rsrc_t rs = rsrc(base + k0, bytes > k0 ? bytes - k0 : 0u);
#pragma unroll
    for (int t = 0; t < kLoads; ++t) {
      const uint32_t r = (8 * wave + t) * 8 + (lane >> 3);
      const bool past_k = half_step && (((lane & 7) ^ ((r >> 1) & 7)) >= 4);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(st + (8 * wave + t) * 1024), 16,
                                               past_k ? 0x80000000u : voff[t], 0, 0, 0);
    }
  };

  v16i acc[kMB][kNB];
#pragma unroll
  for (int mb = 0; mb < kMB; ++mb)
#pragma unroll
    for (int nb = 0; nb < kNB; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mb][nb][r] = 0;

  // K steps of 128 bytes; K is a multiple of 64, so the last step may hold only 64 bytes (its
  // other half loads as zero). Step i sits in stage s0 when i is even, s1 when odd. Before each
  // step's reads: this wave's loads of it are complete (vmcnt 0), the barrier covers the other
  // waves' loads and tells that every wave is done reading the stage the next loads overwrite.
  const uint32_t steps = (a.k + kBK - 1) / kBK;
  const bool tail = a.k % kBK != 0;
  stage(s0, 0, tail && steps == 1);
  uint32_t i = 0;
  // The scheduling fences keep each step's staging loads at its top, a whole step ahead of
  // their use, where the scheduler would otherwise sink them below the MFMAs.
  for (; i + 2 <= steps; i += 2) {  // pairs of steps: i in s0, i+1 in s1
    __syncthreads();
    stage(s1, (i + 1) * kBK, tail && i + 2 == steps);
    __builtin_amdgcn_sched_barrier(0);
    mma_stage<kTrans, 4>(s0, arow, wrow, half, sw, acc);
    __syncthreads();
    if (i + 2 < steps) stage(s0, (i + 2) * kBK, tail && i + 3 == steps);
    __builtin_amdgcn_sched_barrier(0);
    mma_stage<kTrans, 4>(s1, arow, wrow, half, sw, acc);
  }
  if (i < steps) {  // an odd step count ends with one step in s0
    __syncthreads();
    mma_stage<kTrans, 4>(s0, arow, wrow, half, sw, acc);
  }

  if (kTrans) {
    // Q/K tile: block (mb, nb) holds C^T: lane column = token, registers 4g+i = channels
    // 8g + 4*half + i of the block.
#pragma unroll
    for (int mb = 0; mb < kMB; ++mb) {
      const uint32_t m = m0 + arow + 32 * mb;
      if (m >= a.m) continue;
      const float asv = a.as[m];
      uint16_t* dst = a.out + (size_t)m * a.qk_width;
#pragma unroll
      for (int nb = 0; nb < kNB; ++nb) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const uint32_t n = n0 + wave_n * 64 + 32 * nb + 8 * g + 4 * half;
          v4h o;
#pragma unroll
          for (int i = 0; i < 4; ++i) o[i] = finish(acc[mb][nb][4 * g + i], a.ws[n + i], asv);
          *reinterpret_cast<v4h*>(dst + n) = o;
        }
      }
    }
  } else {
    // V tile: block (mb, nb) holds C: lane column = channel, registers 4g+i = tokens
    // 8g + 4*half + i of the block; tokens >= M are stored as zero up to the capacity.
    uint16_t* vt = a.out + (size_t)a.m * a.qk_width;
#pragma unroll
    for (int nb = 0; nb < kNB; ++nb) {
      const uint32_t n = n0 + wave_n * 64 + 32 * nb + (lane & 31);
      if (n >= a.n) continue;
      const float wsv = a.ws[n];
      uint16_t* dst = vt + (size_t)(n - a.qk_width) * a.cap;
#pragma unroll
      for (int mb = 0; mb < kMB; ++mb) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const uint32_t m = m0 + wave_m * 128 + 32 * mb + 8 * g + 4 * half;
          v4h o;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t mi = m + i;
            const float asv = a.as[mi < a.m ? mi : a.m - 1];
            o[i] = mi < a.m ? finish(acc[mb][nb][4 * g + i], wsv, asv) : (_Float16)0.0f;
          }
          *reinterpret_cast<v4h*>(dst + m) = o;
        }
      }
    }
  }
}

__global__ __launch_bounds__(kThreads) void k_gemm_i8_qkv(Args a) {
  __shared__ __attribute__((aligned(16))) char s0[kStage];
  __shared__ __attribute__((aligned(16))) char s1[kStage];
  // XCD-aware remap (block b runs on XCD b % 8): each XCD takes a contiguous range of the
  // rasterised tiles, so the tiles resident on one XCD share A and W rows in its L2.
  const uint32_t b = blockIdx.x;
  const uint32_t w = (b & 7u) * a.per_xcd + (b >> 3);
  if (w >= a.total) return;
  const uint32_t span = kGroupM * a.tiles_n;
  const uint32_t gm = w / span, r = w % span;
  const uint32_t m_in = min((uint32_t)kGroupM, a.tiles_m - gm * kGroupM);
  const uint32_t m_tile = gm * kGroupM + r % m_in;
  const uint32_t n_tile = r / m_in;
  const uint32_t m0 = m_tile * kBM;
  if (n_tile < a.tiles_n_qk)
    tile<true>(a, m0, n_tile * kBN, s0, s1);
  else
    tile<false>(a, m0, a.qk_width + (n_tile - a.tiles_n_qk) * kBN, s0, s1);
}

}  // namespace

hipError_t launch_gemm_i8_qkv(uint32_t m, uint32_t n, uint32_t k, uint32_t k_stride,
                              const int8_t* a, const int8_t* w, const float* ws, const float* as,
                              uint16_t* out, hipStream_t stream) {
  Args g;
  g.a = a;
  g.w = w;
  g.ws = ws;
  g.as = as;
  g.out = out;
  g.m = m;
  g.n = n;
  g.k = k;
  g.k_stride = k_stride;
  g.qk_width = n / 3 * 2;
  g.cap = (m + kBM - 1) / kBM * kBM;
  g.tiles_m = (m + kBM - 1) / kBM;
  g.tiles_n_qk = g.qk_width / kBN;
  g.tiles_n = g.tiles_n_qk + (n / 3 + kBN - 1) / kBN;
  g.total = g.tiles_m * g.tiles_n;
  g.per_xcd = (g.total + 7) / 8;
  hipLaunchKernelGGL(k_gemm_i8_qkv, dim3(g.per_xcd * 8), dim3(kThreads), 0, stream, g);
  return hipGetLastError();
}

}  // namespace h3
