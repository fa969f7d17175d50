// VSA (video sparse attention) device operations on gfx950: the kernels of
// kernels/vsa_ops.loom (gather, scatter, pool, block scores, route, coarse, gated scatter) and
// kernels/vsa_kmean.loom. The block-sparse attention itself is k_attention_vsa (attention.hip).
//
// Layout: activations are f16 rows of `width` = heads*128 channels. The gathered ("padded")
// layout holds 64 rows per block (a prefix tile or a 4x4x4 video cube), live rows first, dead
// rows zero. Block means are f32 [blocks][width]; scores f32 and routes i32
// [heads][blocks][blocks].
//
// Exactness: gather/scatter are bit copies; pool, kmean and the block scores keep the
// reference's sequential f32 order per output (a running sum over rows; an fma chain over the
// 128 channels of a head), so they are bit-identical to it. The route is an exact integer
// function of the scores: the reference counts, for each (head, q, j), the non-prefix scores of
// row q strictly greater than scores[q][j] (O(blocks) per entry); here one radix select per row
// finds T, the topk-th largest non-NaN non-prefix score, and `count < topk` is evaluated as
// `score >= T` (equivalent for non-NaN scores once -0 and +0 share a key; a NaN score has count
// 0; fewer than topk candidates keeps every non-NaN score). The coarse branch uses the hardware
// exp, as the reference's expf<afn> does.
#include "internal.hpp"

namespace h3 {
namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerBlock = kThreads / 64;  // row copies: one wave per row

__device__ __forceinline__ uint4 zero4() { return make_uint4(0u, 0u, 0u, 0u); }

// h3_vsa_gather: y[i] = x[src[i]] for src[i] < tokens (unsigned), else a zero row.
__global__ __launch_bounds__(kThreads) void k_vsa_gather(const int32_t* __restrict__ src,
                                                         const uint4* __restrict__ x,
                                                         uint4* __restrict__ y, uint32_t tokens,
                                                         uint32_t padded, uint32_t chunks) {
  const uint32_t row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= padded) return;
  const uint32_t s = (uint32_t)src[row];
  const bool live = s < tokens;
  const uint4* xr = x + (size_t)(live ? s : 0u) * chunks;
  uint4* yr = y + (size_t)row * chunks;
#pragma unroll 4
  for (uint32_t c = threadIdx.x & 63; c < chunks; c += 64) yr[c] = live ? xr[c] : zero4();
}

// h3_vsa_scatter: y[r] = x[inverse[r]] (inverse[r] >= padded, which a valid plan never holds,
// writes a zero row instead of reading out of range).
__global__ __launch_bounds__(kThreads) void k_vsa_scatter(const int32_t* __restrict__ inverse,
                                                          const uint4* __restrict__ x,
                                                          uint4* __restrict__ y, uint32_t tokens,
                                                          uint32_t padded, uint32_t chunks) {
  const uint32_t row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= tokens) return;
  const uint32_t s = (uint32_t)inverse[row];
  const bool live = s < padded;
  const uint4* xr = x + (size_t)(live ? s : 0u) * chunks;
  uint4* yr = y + (size_t)row * chunks;
#pragma unroll 4
  for (uint32_t c = threadIdx.x & 63; c < chunks; c += 64) yr[c] = live ? xr[c] : zero4();
}

// h3_vsa_pool: means[b][c] = (sum_{j < len} f32(x[64b + j][c])) / f32(len), a running f32 sum
// over the rows in order. A thread owns eight consecutive channels.
__global__ __launch_bounds__(kThreads) void k_vsa_pool(const int32_t* __restrict__ lengths,
                                                       const uint4* __restrict__ x,
                                                       float4* __restrict__ means,
                                                       uint32_t chunks) {
  const uint32_t b = blockIdx.x;
  const uint32_t c = blockIdx.y * kThreads + threadIdx.x;
  if (c >= chunks) return;
  const int len_raw = lengths[b];
  const int len = len_raw < 0 ? 0 : len_raw > 64 ? 64 : len_raw;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const uint4* xr = x + (size_t)64 * b * chunks + c;
  for (int j = 0; j < len; ++j) {
    const uint4 v = xr[(size_t)j * chunks];
    const v4f lo = widen4(make_uint2(v.x, v.y), H3_ELEM_F16);
    const v4f hi = widen4(make_uint2(v.z, v.w), H3_ELEM_F16);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[i] = acc[i] + lo[i];
      acc[4 + i] = acc[4 + i] + hi[i];
    }
  }
  const float lf = (float)len;
  float4* out = means + ((size_t)b * chunks + c) * 2;
  out[0] = make_float4(acc[0] / lf, acc[1] / lf, acc[2] / lf, acc[3] / lf);
  out[1] = make_float4(acc[4] / lf, acc[5] / lf, acc[6] / lf, acc[7] / lf);
}

// h3_vsa_gather, then h3_vsa_pool of the gathered rows, in one pass (the runtime's q and k): a
// thread owns eight consecutive channels of one cube, copies the cube's 64 rows (a zero row
// where src[i] >= tokens) and sums the first `len` of the values it wrote, in row order. The
// rows and the means are those of the two kernels run one after the other, bit for bit, and the
// gathered rows are not read back.
__global__ __launch_bounds__(kThreads) void k_vsa_gather_pool(const int32_t* __restrict__ src,
                                                              const int32_t* __restrict__ lengths,
                                                              const uint4* __restrict__ x,
                                                              uint4* __restrict__ y,
                                                              float4* __restrict__ means,
                                                              uint32_t tokens, uint32_t chunks) {
  const uint32_t b = blockIdx.x;
  const uint32_t c = blockIdx.y * kThreads + threadIdx.x;
  if (c >= chunks) return;
  const int len_raw = lengths[b];
  const int len = len_raw < 0 ? 0 : len_raw > 64 ? 64 : len_raw;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const int32_t* sb = src + (size_t)64 * b;
  uint4* yb = y + (size_t)64 * b * chunks + c;
#pragma unroll 8
  for (int j = 0; j < 64; ++j) {
    const uint32_t s = (uint32_t)sb[j];
    const uint4 v = s < tokens ? x[(size_t)s * chunks + c] : zero4();
    yb[(size_t)j * chunks] = v;
    if (j < len) {
      const v4f lo = widen4(make_uint2(v.x, v.y), H3_ELEM_F16);
      const v4f hi = widen4(make_uint2(v.z, v.w), H3_ELEM_F16);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[i] = acc[i] + lo[i];
        acc[4 + i] = acc[4 + i] + hi[i];
      }
    }
  }
  const float lf = (float)len;
  float4* out = means + ((size_t)b * chunks + c) * 2;
  out[0] = make_float4(acc[0] / lf, acc[1] / lf, acc[2] / lf, acc[3] / lf);
  out[1] = make_float4(acc[4] / lf, acc[5] / lf, acc[6] / lf, acc[7] / lf);
}

// h3_vsa_scores: scores[h][q][j] = fma chain over d = 0..127 of qm[q][128h+d] * km[j][128h+d].
// A workgroup computes a 64 x 64 tile of one head, a thread 4 x 4 outputs, with the channels
// staged through LDS 32 at a time (transposed, so a thread reads 4 q or 4 j values per load).
constexpr int kScoreTile = 64;
constexpr int kScoreSlice = 32;
__global__ __launch_bounds__(kThreads) void k_vsa_scores(const float* __restrict__ qm,
                                                         const float* __restrict__ km,
                                                         float* __restrict__ scores,
                                                         uint32_t blocks, uint32_t width) {
  __shared__ __attribute__((aligned(16))) float qt[kScoreSlice][kScoreTile + 4];
  __shared__ __attribute__((aligned(16))) float kt[kScoreSlice][kScoreTile + 4];
  const uint32_t h = blockIdx.z;
  const uint32_t q0 = blockIdx.y * kScoreTile, j0 = blockIdx.x * kScoreTile;
  const int tq = threadIdx.x >> 4, tj = threadIdx.x & 15;
  float acc[4][4] = {};
  for (int d0 = 0; d0 < 128; d0 += kScoreSlice) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {  // 64 rows x 32 channels = 512 float4 per operand
      const int idx = threadIdx.x + kThreads * i;
      const int r = idx >> 3, c4 = idx & 7;
      const size_t col = (size_t)h * 128 + d0 + 4 * c4;
      float4 qv = make_float4(0.f, 0.f, 0.f, 0.f), kv = qv;
      if (q0 + r < blocks) qv = *reinterpret_cast<const float4*>(qm + (size_t)(q0 + r) * width + col);
      if (j0 + r < blocks) kv = *reinterpret_cast<const float4*>(km + (size_t)(j0 + r) * width + col);
      qt[4 * c4 + 0][r] = qv.x;
      qt[4 * c4 + 1][r] = qv.y;
      qt[4 * c4 + 2][r] = qv.z;
      qt[4 * c4 + 3][r] = qv.w;
      kt[4 * c4 + 0][r] = kv.x;
      kt[4 * c4 + 1][r] = kv.y;
      kt[4 * c4 + 2][r] = kv.z;
      kt[4 * c4 + 3][r] = kv.w;
    }
    __syncthreads();
#pragma unroll 8
    for (int d = 0; d < kScoreSlice; ++d) {
      const float4 a = *reinterpret_cast<const float4*>(&qt[d][4 * tq]);
      const float4 b = *reinterpret_cast<const float4*>(&kt[d][4 * tj]);
      const float av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int k = 0; k < 4; ++k) acc[i][k] = __builtin_fmaf(av[i], bv[k], acc[i][k]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t q = q0 + 4 * tq + i;
    if (q >= blocks) continue;
    float* row = scores + ((size_t)h * blocks + q) * blocks;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (j0 + 4 * tj + k < blocks) row[j0 + 4 * tj + k] = acc[i][k];
  }
}

// Order-preserving key of a float (unsigned order = float order), -0 and +0 sharing one key.
__device__ __forceinline__ uint32_t order_key(float f) {
  uint32_t b = __float_as_uint(f);
  if ((b & 0x7fffffffu) == 0) b = 0;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
// NaN patterns map below the key of -inf (0x007fffff) or above the key of +inf (0xff800000).
__device__ __forceinline__ bool key_is_nan(uint32_t k) { return k < 0x007fffffu || k > 0xff800000u; }

// h3_vsa_route: one workgroup per (q, head) row. Four 8-bit radix passes find the topk-th
// largest candidate key (candidates: j >= prefix, not NaN); the row is then written. kPer > 0:
// each thread keeps the keys of its candidates j = prefix + tid + kThreads*i (i < kPer) in
// registers, so the row is read from memory once instead of once per pass.
template <int kPer>
__global__ __launch_bounds__(kThreads) void k_vsa_route(const float* __restrict__ scores,
                                                        int32_t* __restrict__ routes,
                                                        uint32_t blocks, uint32_t prefix,
                                                        uint32_t topk) {
  __shared__ uint32_t hist[256];
  __shared__ uint32_t sel[3];  // chosen digit, rank left inside it, candidates (pass 0)
  const uint32_t q = blockIdx.x, h = blockIdx.y;
  const float* row = scores + ((size_t)h * blocks + q) * blocks;
  int32_t* out = routes + ((size_t)h * blocks + q) * blocks;
  const uint32_t tid = threadIdx.x, lane = tid & 63;
  const bool select = topk > 0 && q >= prefix;  // a prefix row keeps everything
  uint32_t want = topk, bits = 0, mask = 0, candidates = 0;
  uint32_t cache[kPer > 0 ? kPer : 1];  // order keys of this thread's candidates (0: a NaN key)
  if constexpr (kPer > 0) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const uint32_t j = prefix + tid + kThreads * i;
      cache[i] = j < blocks ? order_key(row[j]) : 0u;
    }
  }
  for (int pass = 0; pass < 4 && select; ++pass) {
    const int shift = 24 - 8 * pass;
    hist[tid] = 0;
    __syncthreads();
    if constexpr (kPer > 0) {
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const uint32_t k = cache[i];
        if (!key_is_nan(k) && (k & mask) == bits) atomicAdd(&hist[(k >> shift) & 255u], 1u);
      }
    } else {
      for (uint32_t j = prefix + tid; j < blocks; j += kThreads) {
        const uint32_t k = order_key(row[j]);
        if (!key_is_nan(k) && (k & mask) == bits) atomicAdd(&hist[(k >> shift) & 255u], 1u);
      }
    }
    __syncthreads();
    if (tid < 64) {  // lane l scans bins 255-4l, 254-4l, 253-4l, 252-4l (descending)
      uint32_t c[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) c[i] = hist[255 - 4 * lane - i];
      const uint32_t own = c[0] + c[1] + c[2] + c[3];
      uint32_t incl = own;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t up = __shfl_up(incl, o);
        if ((int)lane >= o) incl += up;
      }
      const uint32_t excl = incl - own;
      const uint32_t total = __shfl(incl, 63);
      if (lane == 0 && pass == 0) sel[2] = total;
      if (excl < want && want <= incl) {
        uint32_t acc = excl;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (acc + c[i] >= want) {
            sel[0] = 255 - 4 * lane - i;
            sel[1] = want - acc;
            break;
          }
          acc += c[i];
        }
      }
    }
    __syncthreads();
    if (pass == 0) {
      candidates = sel[2];
      if (candidates < want) {  // fewer candidates than the budget: every non-NaN score stays
        __syncthreads();
        break;
      }
    }
    bits |= sel[0] << shift;
    mask |= 255u << shift;
    want = sel[1];
    __syncthreads();
  }
  const bool all = select && candidates < topk;
  // routes[q][j]: 1 when forced (a prefix row or column, |q - j| <= 1); else 0 without a budget,
  // 1 when there are fewer candidates than the budget, else NaN or at least the threshold key.
  auto keep_of = [&](uint32_t j, uint32_t k) -> int32_t {
    if (q < prefix || j < prefix || (j <= q + 1 && q <= j + 1)) return 1;
    if (topk == 0) return 0;
    return all || key_is_nan(k) || k >= bits ? 1 : 0;
  };
  if constexpr (kPer > 0) {
    for (uint32_t j = tid; j < prefix && j < blocks; j += kThreads) out[j] = 1;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const uint32_t j = prefix + tid + kThreads * i;
      if (j < blocks) out[j] = keep_of(j, cache[i]);
    }
  } else {
    for (uint32_t j = tid; j < blocks; j += kThreads) out[j] = keep_of(j, order_key(row[j]));
  }
}

// h3_vsa_coarse: coarse[q][128h+c] = sum_j w_qj vm[j][128h+c] / sum_j w_qj with
// w_qj = exp(scores[h][q][j]*scale - max_j(scores[h][q][j]*scale)), the max starting at -1e9.
// A workgroup takes 32 query blocks of one head; thread (c, g) owns channel c of 16 of them.
constexpr int kCoarseRows = 32;
constexpr int kCoarseCols = 64;  // key blocks per LDS slice
__global__ __launch_bounds__(kThreads) void k_vsa_coarse(const float* __restrict__ scores,
                                                         const float* __restrict__ vm,
                                                         float* __restrict__ coarse,
                                                         uint32_t blocks, uint32_t width) {
  __shared__ float w[kCoarseRows][kCoarseCols + 1];
  __shared__ float row_max[kCoarseRows];
  __shared__ float row_sum[kCoarseRows];
  const float scale = 0.08838834764831845f;
  const uint32_t h = blockIdx.y, q0 = blockIdx.x * kCoarseRows;
  const uint32_t tid = threadIdx.x;
  // max: 8 threads per row
  const uint32_t r8 = tid >> 3, p8 = tid & 7;
  const float* srow = scores + ((size_t)h * blocks + q0 + r8) * blocks;
  const bool row_live = q0 + r8 < blocks;
  float m = -1.0e9f;
  if (row_live)
    for (uint32_t j = p8; j < blocks; j += 8) m = fmaxf(srow[j] * scale, m);
#pragma unroll
  for (int o = 1; o < 8; o <<= 1) m = fmaxf(m, __shfl_xor(m, o));
  float part = 0.0f;  // this thread's share of the row sum
  const uint32_t c = tid & 127, g = tid >> 7;
  float acc[16] = {};
  const float* vcol = vm + (size_t)h * 128 + c;
  for (uint32_t j0 = 0; j0 < blocks; j0 += kCoarseCols) {
    // weights of the slice: 8 threads per row, 8 key blocks each
#pragma unroll
    for (int i = 0; i < kCoarseCols / 8; ++i) {
      const uint32_t jj = p8 * (kCoarseCols / 8) + i, j = j0 + jj;
      float wv = 0.0f;
      if (row_live && j < blocks) wv = __expf(srow[j] * scale - m);
      part += wv;
      w[r8][jj] = wv;
    }
    __syncthreads();
    const uint32_t jn = blocks - j0 < (uint32_t)kCoarseCols ? blocks - j0 : kCoarseCols;
    for (uint32_t jj = 0; jj < jn; ++jj) {
      const float v = vcol[(size_t)(j0 + jj) * width];
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[i] = __builtin_fmaf(w[16 * g + i][jj], v, acc[i]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int o = 1; o < 8; o <<= 1) part += __shfl_xor(part, o);
  if (p8 == 0) {
    row_max[r8] = m;
    row_sum[r8] = part;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t q = q0 + 16 * g + i;
    if (q < blocks) coarse[(size_t)q * width + (size_t)h * 128 + c] = acc[i] / row_sum[16 * g + i];
  }
}

// h3_vsa_gated_scatter: out[r][c] = f16(fma(f32(gate[r][c]), coarse[inverse[r]/64][c],
// f32(fine[inverse[r]][c]))), round to nearest even. A wave per output row, 8 channels a lane.
__global__ __launch_bounds__(kThreads) void k_vsa_gated_scatter(
    const int32_t* __restrict__ inverse, const uint4* __restrict__ fine,
    const uint4* __restrict__ gate, const float4* __restrict__ coarse, uint4* __restrict__ out,
    uint32_t tokens, uint32_t padded, uint32_t chunks) {
  const uint32_t row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= tokens) return;
  const uint32_t s = (uint32_t)inverse[row];
  const bool live = s < padded;
  const uint32_t sr = live ? s : 0u, b = sr / 64;
#pragma unroll 2
  for (uint32_t c = threadIdx.x & 63; c < chunks; c += 64) {
    const uint4 f = fine[(size_t)sr * chunks + c];
    const uint4 g = gate[(size_t)row * chunks + c];
    const float4 c0 = coarse[((size_t)b * chunks + c) * 2];
    const float4 c1 = coarse[((size_t)b * chunks + c) * 2 + 1];
    const v4f f0 = widen4(make_uint2(f.x, f.y), H3_ELEM_F16), f1 = widen4(make_uint2(f.z, f.w), H3_ELEM_F16);
    const v4f g0 = widen4(make_uint2(g.x, g.y), H3_ELEM_F16), g1 = widen4(make_uint2(g.z, g.w), H3_ELEM_F16);
    const float cv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
    v8h o;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[i] = (_Float16)__builtin_fmaf(g0[i], cv[i], f0[i]);
      o[4 + i] = (_Float16)__builtin_fmaf(g1[i], cv[4 + i], f1[i]);
    }
    out[(size_t)row * chunks + c] = live ? __builtin_bit_cast(uint4, o) : zero4();
  }
}

// h3_vsa_kmean: mean[c] = (sum_t x[t][c]) / f32(tokens), a running f32 sum over the rows.
__global__ __launch_bounds__(kThreads) void k_vsa_kmean(const float* __restrict__ x,
                                                        float* __restrict__ mean,
                                                        uint32_t tokens, uint32_t width) {
  const uint32_t c = blockIdx.x * kThreads + threadIdx.x;
  if (c >= width) return;
  float acc = 0.0f;
#pragma unroll 8
  for (uint32_t t = 0; t < tokens; ++t) acc = acc + x[(size_t)t * width + c];
  mean[c] = acc / (float)tokens;
}

}  // namespace

hipError_t launch_vsa_gather(uint32_t tokens, uint32_t padded, uint32_t width, const int32_t* src,
                             const uint16_t* x, uint16_t* y, hipStream_t stream) {
  hipLaunchKernelGGL(k_vsa_gather, dim3((padded + kRowsPerBlock - 1) / kRowsPerBlock),
                     dim3(kThreads), 0, stream, src, reinterpret_cast<const uint4*>(x),
                     reinterpret_cast<uint4*>(y), tokens, padded, width / 8);
  return hipGetLastError();
}

hipError_t launch_vsa_scatter(uint32_t tokens, uint32_t padded, uint32_t width,
                              const int32_t* inverse, const uint16_t* x, uint16_t* y,
                              hipStream_t stream) {
  hipLaunchKernelGGL(k_vsa_scatter, dim3((tokens + kRowsPerBlock - 1) / kRowsPerBlock),
                     dim3(kThreads), 0, stream, inverse, reinterpret_cast<const uint4*>(x),
                     reinterpret_cast<uint4*>(y), tokens, padded, width / 8);
  return hipGetLastError();
}

hipError_t launch_vsa_pool(uint32_t blocks, uint32_t width, const int32_t* lengths,
                           const uint16_t* x, float* means, hipStream_t stream) {
  const uint32_t chunks = width / 8;
  hipLaunchKernelGGL(k_vsa_pool, dim3(blocks, (chunks + kThreads - 1) / kThreads), dim3(kThreads),
                     0, stream, lengths, reinterpret_cast<const uint4*>(x),
                     reinterpret_cast<float4*>(means), chunks);
  return hipGetLastError();
}

hipError_t launch_vsa_gather_pool(uint32_t tokens, uint32_t blocks, uint32_t width,
                                  const int32_t* src, const int32_t* lengths, const uint16_t* x,
                                  uint16_t* y, float* means, hipStream_t stream) {
  const uint32_t chunks = width / 8;
  hipLaunchKernelGGL(k_vsa_gather_pool, dim3(blocks, (chunks + kThreads - 1) / kThreads),
                     dim3(kThreads), 0, stream, src, lengths, reinterpret_cast<const uint4*>(x),
                     reinterpret_cast<uint4*>(y), reinterpret_cast<float4*>(means), tokens,
                     chunks);
  return hipGetLastError();
}

hipError_t launch_vsa_scores(uint32_t blocks, uint32_t heads, const float* qm, const float* km,
                             float* scores, hipStream_t stream) {
  const uint32_t tiles = (blocks + kScoreTile - 1) / kScoreTile;
  hipLaunchKernelGGL(k_vsa_scores, dim3(tiles, tiles, heads), dim3(kThreads), 0, stream, qm, km,
                     scores, blocks, heads * 128);
  return hipGetLastError();
}

hipError_t launch_vsa_route(uint32_t blocks, uint32_t heads, uint32_t prefix, uint32_t topk,
                            const float* scores, int32_t* routes, hipStream_t stream) {
  constexpr int kPer = 16;  // rows of up to 4,096 candidates stay in registers
  if (blocks <= prefix + (uint32_t)kPer * kThreads)
    hipLaunchKernelGGL(k_vsa_route<kPer>, dim3(blocks, heads), dim3(kThreads), 0, stream, scores,
                       routes, blocks, prefix, topk);
  else
    hipLaunchKernelGGL(k_vsa_route<0>, dim3(blocks, heads), dim3(kThreads), 0, stream, scores,
                       routes, blocks, prefix, topk);
  return hipGetLastError();
}

hipError_t launch_vsa_coarse(uint32_t blocks, uint32_t heads, const float* scores,
                             const float* vm, float* coarse, hipStream_t stream) {
  hipLaunchKernelGGL(k_vsa_coarse, dim3((blocks + kCoarseRows - 1) / kCoarseRows, heads),
                     dim3(kThreads), 0, stream, scores, vm, coarse, blocks, heads * 128);
  return hipGetLastError();
}

hipError_t launch_vsa_gated_scatter(uint32_t tokens, uint32_t padded, uint32_t width,
                                    const int32_t* inverse, const uint16_t* fine,
                                    const uint16_t* gate, const float* coarse, uint16_t* out,
                                    hipStream_t stream) {
  hipLaunchKernelGGL(k_vsa_gated_scatter, dim3((tokens + kRowsPerBlock - 1) / kRowsPerBlock),
                     dim3(kThreads), 0, stream, inverse, reinterpret_cast<const uint4*>(fine),
                     reinterpret_cast<const uint4*>(gate), reinterpret_cast<const float4*>(coarse),
                     reinterpret_cast<uint4*>(out), tokens, padded, width / 8);
  return hipGetLastError();
}

hipError_t launch_vsa_kmean(uint32_t tokens, uint32_t width, const float* x, float* mean,
                            hipStream_t stream) {
  hipLaunchKernelGGL(k_vsa_kmean, dim3((width + kThreads - 1) / kThreads), dim3(kThreads), 0,
                     stream, x, mean, tokens, width);
  return hipGetLastError();
}

}  // namespace h3
