// INT8-QK flash attention for gfx950 (CDNA4).
//
// One workgroup = 4 wave64s x 32 queries of one head; keys stream through double-buffered
// 64-key LDS tiles. Per wave and key tile:
//   QK   S^T (64 keys x 32 queries) = K (64 x 128 i8) . Q^T on v_mfma_i32_32x32x32_i8, exact
//        int32. With keys as the MFMA rows, lane l owns query l%32 and 32 of the tile's keys:
//        key(b, r, l) = 32b + 8(r/4) + 4(l/32) + r%4 for block b in {0,1}, accumulator reg r.
//        Every softmax statistic (running max, sum, Q scale) is a per-lane scalar; only the max
//        is exchanged, once per tile, with the lane's partner in the other half-wave.
//   softmax  u = f32(S) * ks_key; online max in u units; p = exp2(u*qs*log2e - m*qs*log2e).
//   PV   O^T (128 ch x 32 queries) += V^T . P^T on v_mfma_f32_32x32x16_f16. The B operand of a
//        16-key MFMA step is eight consecutive accumulator registers of one S^T block, converted
//        to f16 in place: no cross-lane shuffle. The matching A operand needs, in lane half h,
//        keys {8(j/4) + 4h + j%4 : j < 8} of each 16-key group; the V^T tile is therefore
//        stored in LDS with key bits 2 and 3 swapped inside every 16-key group, which turns each
//        A operand into one aligned 16-byte LDS read.
// LDS rows are padded to 144 bytes so the 32 rows a half-wave reads land on distinct banks.
// Workgroups are remapped so consecutive query blocks of one head run on the same XCD and
// share its L2 while they walk the same K/V stream.
//
// Semantics follow kernels/attention_i8qkhm_mha8_k64_lds_f16_wmma.loom:437-1067 (head-major)
// and kernels/attention_i8qk_family.loom:193-424 (token-major): non-causal MHA, keys >= tokens
// masked, rows >= token_count not written, f16 output [token_count][out_stride].
#include "internal.hpp"

namespace h3 {
namespace {

constexpr int kWaves = 4;
constexpr int kQueriesPerWave = 32;
constexpr int kQueriesPerBlock = kWaves * kQueriesPerWave;  // 128
constexpr int kKeys = 64;                                   // keys per LDS tile
constexpr int kRowBytes = 144;                              // 128 data bytes + 16 pad
constexpr int kKBytes = kKeys * kRowBytes;                  // 9216
constexpr int kVBytes = 128 * kRowBytes;                    // 18432
constexpr int kStageBytes = kKBytes + kVBytes + kKeys * 4;  // 27904
constexpr float kLog2e = 1.4426950408889634f;

struct Args {
  const int32_t* qi;
  const float* qs;
  const int32_t* ki;
  const float* ks;
  const uint16_t* vt;
  uint16_t* out;
  uint32_t tokens;
  uint32_t token_count;
  uint32_t capacity;
  uint32_t q_words;   // q_stride / 4 (token-major row pitch of qi, in words)
  uint32_t kv_words;  // kv_stride / 4
  uint32_t out_stride;
  uint32_t q_blocks;  // ceil(token_count / 128)
  uint32_t heads;     // workload heads (grid y of the reference)
  uint32_t kv_head_limit;
  uint32_t head_limit;
  uint32_t total;      // q_blocks * heads
  uint32_t per_xcd;    // ceil(total / 8)
};

// Registers holding one key tile on its way from global memory to LDS.
struct Prefetch {
  v4i k[2];
  v4i v[4];
  float ks;
};

template <bool kHeadMajor>
__device__ __forceinline__ void load_tile(const Args& a, uint32_t kv_head, uint32_t k0,
                                          Prefetch& pf) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = tid + 256 * i;  // 512 chunks of 16 bytes: key c/8, part c%8
    const uint32_t key = k0 + (c >> 3);
    const int part = c & 7;
    v4i val = {0, 0, 0, 0};
    if (key < a.tokens) {
      const int32_t* src =
          kHeadMajor ? a.ki + ((size_t)kv_head * a.capacity + key) * 32 + part * 4
                     : a.ki + (size_t)key * a.kv_words + kv_head * 32 + part * 4;
      val = *reinterpret_cast<const v4i*>(src);
    }
    pf.k[i] = val;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = tid + 256 * i;  // 1024 chunks: channel c/8, keys 8*(c%8)..+7
    const int d = c >> 3, part = c & 7;
    const uint32_t key = k0 + 8 * part;
    const uint16_t* src = a.vt + ((size_t)kv_head * 128 + d) * a.capacity + key;
    v4i val;
    if (key + 8 <= a.tokens) {
      val = *reinterpret_cast<const v4i*>(src);
    } else {
      uint16_t h[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) h[j] = (key + j < a.tokens) ? src[j] : (uint16_t)0;
      val = __builtin_bit_cast(v4i, h);
    }
    pf.v[i] = val;
  }
  if (tid < kKeys) {
    const uint32_t key = k0 + tid;
    float s = 0.0f;
    if (key < a.tokens)
      s = kHeadMajor ? a.ks[(size_t)kv_head * a.capacity + key]
                     : a.ks[(size_t)key * a.kv_head_limit + kv_head];
    pf.ks = s;
  }
}

__device__ __forceinline__ void store_tile(char* stage, const Prefetch& pf) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = tid + 256 * i;
    *reinterpret_cast<v4i*>(stage + (c >> 3) * kRowBytes + (c & 7) * 16) = pf.k[i];
  }
  char* vbase = stage + kKBytes;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = tid + 256 * i;
    const int d = c >> 3, part = c & 7;
    // keys 8*part..+3 and +4..+7 of 16-key group part/2, placed with key bits 2 and 3 swapped
    const int group = part >> 1, odd = part & 1;
    char* row = vbase + d * kRowBytes + group * 32;
    int2 lo = {pf.v[i][0], pf.v[i][1]};
    int2 hi = {pf.v[i][2], pf.v[i][3]};
    *reinterpret_cast<int2*>(row + (4 * odd) * 2) = lo;
    *reinterpret_cast<int2*>(row + (8 + 4 * odd) * 2) = hi;
  }
  if (tid < kKeys) reinterpret_cast<float*>(stage + kKBytes + kVBytes)[tid] = pf.ks;
}

template <bool kHeadMajor>
__global__ __launch_bounds__(256) void k_attention(Args a) {
  __shared__ __attribute__((aligned(16))) char smem[2 * kStageBytes];

  // XCD-aware remap: hardware hands block b to XCD b % 8; give each XCD a contiguous range of
  // (head, query block) work so its resident blocks share one head's K/V stream in L2.
  const uint32_t b = blockIdx.x;
  const uint32_t logical = (b & 7u) * a.per_xcd + (b >> 3);
  if (logical >= a.total) return;
  const uint32_t head_y = logical / a.q_blocks;
  const uint32_t qb = logical % a.q_blocks;
  const uint32_t kv_head = head_y % a.kv_head_limit;
  const uint32_t head = kv_head % a.head_limit;

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int n = lane & 31;      // query within the wave's tile
  const int half = lane >> 5;   // which 16 key-bytes / key slots this lane holds

  const uint32_t tiles32 = (a.tokens + 31) / 32;
  const uint32_t q_tile = qb * kWaves + wave;
  const uint32_t q_tile_c = q_tile < tiles32 ? q_tile : tiles32 - 1;
  const uint32_t q = q_tile_c * kQueriesPerWave + n;
  const uint32_t q_read = q < a.tokens ? q : a.tokens - 1;

  // Q^T operand, held for the whole key loop: 4 chunks of 32 channels, 16 bytes per lane.
  v4i qop[4];
  {
    const int32_t* src = kHeadMajor ? a.qi + ((size_t)head * a.capacity + q_read) * 32
                                    : a.qi + (size_t)q_read * a.q_words + head * 32;
#pragma unroll
    for (int dc = 0; dc < 4; ++dc) qop[dc] = *reinterpret_cast<const v4i*>(src + 8 * dc + 4 * half);
  }
  const float qsv = kHeadMajor ? a.qs[(size_t)head * a.capacity + q_read]
                               : a.qs[(size_t)q_read * a.head_limit + head];
  const float qsl = qsv * kLog2e;

  v16f acc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[db][r] = 0.0f;
  float m_run = -1.0e30f;  // running max in u units (f32(S) * ks)
  float l_run = 0.0f;      // this lane's partial sum over its key slots

  const uint32_t n_tiles = (a.tokens + kKeys - 1) / kKeys;
  Prefetch pf;
  load_tile<kHeadMajor>(a, kv_head, 0, pf);
  store_tile(smem, pf);
  __syncthreads();

  for (uint32_t kt = 0; kt < n_tiles; ++kt) {
    const bool more = kt + 1 < n_tiles;
    if (more) load_tile<kHeadMajor>(a, kv_head, (kt + 1) * kKeys, pf);
    const char* stage = smem + (kt & 1) * kStageBytes;
    const char* kst = stage;
    const char* vst = stage + kKBytes;
    const float* kss = reinterpret_cast<const float*>(stage + kKBytes + kVBytes);

    // ---- S^T = K . Q^T
    v16i s[2];
#pragma unroll
    for (int bb = 0; bb < 2; ++bb)
#pragma unroll
      for (int r = 0; r < 16; ++r) s[bb][r] = 0;
#pragma unroll
    for (int dc = 0; dc < 4; ++dc) {
#pragma unroll
      for (int bb = 0; bb < 2; ++bb) {
        v4i kop = *reinterpret_cast<const v4i*>(kst + (32 * bb + n) * kRowBytes + 32 * dc + 16 * half);
        s[bb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(kop, qop[dc], s[bb], 0, 0, 0);
      }
    }

    // ---- scores in u units, tile max
    float u[2][16];
    float tmax = -INFINITY;
    const uint32_t k0 = kt * kKeys;
    const bool partial = k0 + kKeys > a.tokens;
#pragma unroll
    for (int bb = 0; bb < 2; ++bb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kb = 32 * bb + 8 * i + 4 * half;
        const float4 k4 = *reinterpret_cast<const float4*>(kss + kb);
        const float kv[4] = {k4.x, k4.y, k4.z, k4.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float v = (float)s[bb][4 * i + j] * kv[j];
          if (partial && k0 + kb + j >= a.tokens) v = -INFINITY;
          u[bb][4 * i + j] = v;
        }
      }
    }
#pragma unroll
    for (int bb = 0; bb < 2; ++bb)
#pragma unroll
      for (int r = 0; r < 16; r += 2) tmax = fmaxf(tmax, fmaxf(u[bb][r], u[bb][r + 1]));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
    const float m_new = fmaxf(m_run, tmax);
    const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * qsl);
    const float neg = -(m_new * qsl);
    m_run = m_new;

    // ---- probabilities, packed to f16 B operands
    v8h pb[4];
    float psum = 0.0f;
#pragma unroll
    for (int bb = 0; bb < 2; ++bb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float p = __builtin_amdgcn_exp2f(__builtin_fmaf(u[bb][r], qsl, neg));
        if (partial && u[bb][r] == -INFINITY) p = 0.0f;
        psum += p;
        pb[2 * bb + r / 8][r % 8] = (_Float16)p;
      }
    }
    l_run = l_run * alpha + psum;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[db][r] *= alpha;

    // ---- O^T += V^T . P^T
#pragma unroll
    for (int g = 0; g < 4; ++g) {
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        v8h vop = *reinterpret_cast<const v8h*>(vst + (32 * db + n) * kRowBytes + (16 * g + 8 * half) * 2);
        acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vop, pb[g], acc[db], 0, 0, 0);
      }
    }

    if (more) store_tile(smem + ((kt + 1) & 1) * kStageBytes, pf);
    __syncthreads();
  }

  // ---- normalise and store rows < token_count
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const float inv = 1.0f / l_tot;
  if (q_tile < tiles32 && q < a.token_count && q < a.tokens) {
    uint16_t* dst = a.out + (size_t)q * a.out_stride + head * 128;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v4h o = {(_Float16)(acc[db][4 * i + 0] * inv), (_Float16)(acc[db][4 * i + 1] * inv),
                 (_Float16)(acc[db][4 * i + 2] * inv), (_Float16)(acc[db][4 * i + 3] * inv)};
        *reinterpret_cast<v4h*>(dst + 32 * db + 8 * i + 4 * half) = o;
      }
    }
  }
}

}  // namespace

hipError_t launch_attention(const h3_attention_cfg& cfg, int head_major, uint32_t token_count,
                            uint32_t heads, const int32_t* qi, const float* qs, const int32_t* ki,
                            const float* ks, const uint16_t* vt, uint16_t* out,
                            hipStream_t stream) {
  Args a;
  a.qi = qi;
  a.qs = qs;
  a.ki = ki;
  a.ks = ks;
  a.vt = vt;
  a.out = out;
  a.tokens = cfg.tokens;
  a.token_count = token_count;
  a.capacity = cfg.token_capacity;
  a.q_words = cfg.q_stride / 4;
  a.kv_words = cfg.kv_stride / 4;
  a.out_stride = cfg.out_stride;
  a.q_blocks = (token_count + kQueriesPerBlock - 1) / kQueriesPerBlock;
  a.heads = heads;
  a.kv_head_limit = cfg.kv_stride / 128;
  a.head_limit = cfg.out_stride / 128;
  a.total = a.q_blocks * heads;
  a.per_xcd = (a.total + 7) / 8;
  dim3 grid(a.per_xcd * 8);
  if (head_major)
    hipLaunchKernelGGL(k_attention<true>, grid, dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL(k_attention<false>, grid, dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace h3
