// INT8-QK flash attention for gfx950 (CDNA4).
//
// One workgroup = 4 wave64s x 32 queries of one head; keys stream through double-buffered
// 64-key LDS tiles; two workgroups share a CU (two waves per SIMD), so one wave's softmax
// overlaps the other's matrix work. Per wave and key tile:
//   QK   S^T (64 keys x 32 queries) = K (64 x 128 i8) . Q^T on v_mfma_i32_32x32x32_i8, exact
//        int32. With keys as the MFMA rows, lane l owns query l%32 and 32 of the tile's keys:
//        key(b, r, l) = 32b + 8(r/4) + 4(l/32) + r%4 for block b in {0,1}, accumulator reg r.
//        Every softmax statistic (running max, sum, Q scale) is a per-lane scalar; only the
//        tile max is exchanged, once per tile, with the lane's partner in the other half-wave.
//   dequant  The accumulators start from the bit pattern of 1.5*2^23 instead of 0, so after
//        the MFMA each holds the float 1.5*2^23 + S exactly (|S| <= 128*128*128 < 2^22). One
//        FMA per score then gives u = S*ks: u = acc*ks + (-1.5*2^23*ks), the second term
//        precomputed per key when the tile is staged. No int->float conversion is issued.
//   softmax  online, base 2, in units of u: p = exp2(u*qs*log2e - m). The running max m is
//        raised only when a tile's max exceeds it by more than 8 (p <= 2^8 stays exact enough
//        in f16 and in the f32 sums); only then are the output accumulators rescaled, so in
//        the steady state the O accumulators are touched by nothing but the MFMAs.
//   PV   O^T (128 ch x 32 queries) += V^T . P^T on v_mfma_f32_32x32x16_f16. The B operand of a
//        16-key MFMA step is eight consecutive accumulator registers of one S^T block, converted
//        to f16 in place: no cross-lane shuffle. The matching A operand needs, in lane half h,
//        keys {8(j/4) + 4h + j%4 : j < 8} of each 16-key group; the V^T tile is therefore
//        stored in LDS with key bits 2 and 3 swapped inside every 16-key group, which turns each
//        A operand into one aligned 16-byte LDS read. The row sum is accumulated from the same
//        packed f16 probabilities with v_dot2 (two per instruction).
// LDS rows are padded to 144 bytes so the 32 rows a half-wave reads land on distinct banks.
// Full key tiles run without any masking; only the final partial tile is masked.
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
constexpr int kScaleOffset = kKBytes + kVBytes;             // ks[64] then -M*ks[64]
constexpr int kStageBytes = kScaleOffset + 2 * kKeys * 4;   // 28160
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kMagicBits = 0x4B400000;  // float 12582912 = 1.5 * 2^23
constexpr float kMagic = 12582912.0f;
constexpr float kRescaleSlack = 8.0f;   // raise the running max only past 2^8 growth

typedef int v2i __attribute__((ext_vector_type(2)));

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

// Global -> registers. kMasked: keys >= tokens read as zero (only the final tile).
template <bool kHeadMajor, bool kMasked>
__device__ __forceinline__ void load_tile(const Args& a, uint32_t kv_head, uint32_t k0,
                                          Prefetch& pf) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = tid + 256 * i;  // 512 chunks of 16 bytes: key c/8, part c%8
    const uint32_t key = k0 + (c >> 3);
    const int part = c & 7;
    const int32_t* src = kHeadMajor ? a.ki + ((size_t)kv_head * a.capacity + key) * 32 + part * 4
                                    : a.ki + (size_t)key * a.kv_words + kv_head * 32 + part * 4;
    if (!kMasked || key < a.tokens) {
      pf.k[i] = *reinterpret_cast<const v4i*>(src);
    } else {
      pf.k[i] = v4i{0, 0, 0, 0};
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = tid + 256 * i;  // 1024 chunks: channel c/8, keys 8*(c%8)..+7
    const int d = c >> 3, part = c & 7;
    const uint32_t key = k0 + 8 * part;
    const uint16_t* src = a.vt + ((size_t)kv_head * 128 + d) * a.capacity + key;
    if (!kMasked || key + 8 <= a.tokens) {
      pf.v[i] = *reinterpret_cast<const v4i*>(src);
    } else {
      uint16_t h[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) h[j] = (key + j < a.tokens) ? src[j] : (uint16_t)0;
      pf.v[i] = __builtin_bit_cast(v4i, h);
    }
  }
  if (tid < kKeys) {
    const uint32_t key = k0 + tid;
    float s = 0.0f;
    if (!kMasked || key < a.tokens)
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
    *reinterpret_cast<v2i*>(row + (4 * odd) * 2) = v2i{pf.v[i][0], pf.v[i][1]};
    *reinterpret_cast<v2i*>(row + (8 + 4 * odd) * 2) = v2i{pf.v[i][2], pf.v[i][3]};
  }
  if (tid < kKeys) {
    float* sc = reinterpret_cast<float*>(stage + kScaleOffset);
    sc[tid] = pf.ks;
    sc[kKeys + tid] = -(kMagic * pf.ks);
  }
}

// Per-wave state carried across key tiles.
struct State {
  v16f acc[4];   // O^T, 4 blocks of 32 channels
  float m;       // running max in log2 units (u * qs * log2e)
  float l;       // this lane's partial row sum over its key slots
};

// One 64-key tile from LDS stage `stage`. kMasked: keys >= tokens get probability 0.
template <bool kMasked>
__device__ __forceinline__ void tile_step(const char* stage, const v4i (&qop)[4], float qsl,
                                          State& st, int n, int half, uint32_t k0,
                                          uint32_t tokens) {
  const char* kst = stage;
  const char* vst = stage + kKBytes;
  const float* kss = reinterpret_cast<const float*>(stage + kScaleOffset);

  // ---- S^T = K . Q^T, accumulated on top of the 1.5*2^23 float bias
  const v16i magic = {kMagicBits, kMagicBits, kMagicBits, kMagicBits, kMagicBits, kMagicBits,
                      kMagicBits, kMagicBits, kMagicBits, kMagicBits, kMagicBits, kMagicBits,
                      kMagicBits, kMagicBits, kMagicBits, kMagicBits};
  v16i s[2];
#pragma unroll
  for (int bb = 0; bb < 2; ++bb) {
    v4i kop = *reinterpret_cast<const v4i*>(kst + (32 * bb + n) * kRowBytes + 16 * half);
    s[bb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(kop, qop[0], magic, 0, 0, 0);
  }
#pragma unroll
  for (int dc = 1; dc < 4; ++dc) {
#pragma unroll
    for (int bb = 0; bb < 2; ++bb) {
      v4i kop = *reinterpret_cast<const v4i*>(kst + (32 * bb + n) * kRowBytes + 32 * dc + 16 * half);
      s[bb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(kop, qop[dc], s[bb], 0, 0, 0);
    }
  }

  // ---- u = S * ks in one FMA per score; tile max
  float u[2][16];
#pragma unroll
  for (int bb = 0; bb < 2; ++bb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int kb = 32 * bb + 8 * i + 4 * half;
      const float4 k4 = *reinterpret_cast<const float4*>(kss + kb);
      const float4 c4 = *reinterpret_cast<const float4*>(kss + kKeys + kb);
      const float kv[4] = {k4.x, k4.y, k4.z, k4.w};
      const float cv[4] = {c4.x, c4.y, c4.z, c4.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float v = __builtin_fmaf(__int_as_float(s[bb][4 * i + j]), kv[j], cv[j]);
        if (kMasked && k0 + kb + j >= tokens) v = -INFINITY;
        u[bb][4 * i + j] = v;
      }
    }
  }
  float tmax = -INFINITY;
#pragma unroll
  for (int bb = 0; bb < 2; ++bb)
#pragma unroll
    for (int r = 0; r < 16; r += 2) tmax = fmaxf(tmax, fmaxf(u[bb][r], u[bb][r + 1]));
  tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
  const float mt = tmax * qsl;

  // ---- lazy rescale: only when some row's max grew past the slack
  if (__any(mt > st.m + kRescaleSlack)) {
    const float mn = fmaxf(st.m, mt);
    const float alpha = __builtin_amdgcn_exp2f(st.m - mn);
    st.m = mn;
    st.l *= alpha;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) st.acc[db][r] *= alpha;
  }

  // ---- probabilities, packed to f16 B operands, row sum by v_dot2
  const float neg = -st.m;
  v8h pb[4];
#pragma unroll
  for (int bb = 0; bb < 2; ++bb) {
#pragma unroll
    for (int r = 0; r < 16; r += 2) {
      float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(u[bb][r], qsl, neg));
      float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(u[bb][r + 1], qsl, neg));
      if (kMasked) {
        if (u[bb][r] == -INFINITY) p0 = 0.0f;
        if (u[bb][r + 1] == -INFINITY) p1 = 0.0f;
      }
      v2h pair = {(_Float16)p0, (_Float16)p1};
      st.l = __builtin_amdgcn_fdot2(pair, v2h{(_Float16)1.0f, (_Float16)1.0f}, st.l, false);
      pb[2 * bb + r / 8][r % 8] = pair[0];
      pb[2 * bb + r / 8][r % 8 + 1] = pair[1];
    }
  }

  // ---- O^T += V^T . P^T
#pragma unroll
  for (int g = 0; g < 4; ++g) {
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      v8h vop = *reinterpret_cast<const v8h*>(vst + (32 * db + n) * kRowBytes + (16 * g + 8 * half) * 2);
      st.acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vop, pb[g], st.acc[db], 0, 0, 0);
    }
  }
}

template <bool kHeadMajor>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void k_attention(Args a) {
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

  State st;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) st.acc[db][r] = 0.0f;
  st.m = -1.0e30f;
  st.l = 0.0f;

  const uint32_t full = a.tokens / kKeys;             // unmasked tiles
  const uint32_t n_tiles = (a.tokens + kKeys - 1) / kKeys;
  Prefetch pf;
  if (full > 0)
    load_tile<kHeadMajor, false>(a, kv_head, 0, pf);
  else
    load_tile<kHeadMajor, true>(a, kv_head, 0, pf);
  store_tile(smem, pf);
  __syncthreads();

  for (uint32_t kt = 0; kt < full; ++kt) {
    const uint32_t next = kt + 1;
    if (next < full)
      load_tile<kHeadMajor, false>(a, kv_head, next * kKeys, pf);
    else if (next < n_tiles)
      load_tile<kHeadMajor, true>(a, kv_head, next * kKeys, pf);
    tile_step<false>(smem + (kt & 1) * kStageBytes, qop, qsl, st, n, half, kt * kKeys, a.tokens);
    if (next < n_tiles) store_tile(smem + (next & 1) * kStageBytes, pf);
    __syncthreads();
  }
  if (full < n_tiles)
    tile_step<true>(smem + (full & 1) * kStageBytes, qop, qsl, st, n, half, full * kKeys,
                    a.tokens);

  // ---- normalise and store rows < token_count
  const float l_tot = st.l + __shfl_xor(st.l, 32);
  const float inv = 1.0f / l_tot;
  if (q_tile < tiles32 && q < a.token_count && q < a.tokens) {
    uint16_t* dst = a.out + (size_t)q * a.out_stride + head * 128;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v4h o = {(_Float16)(st.acc[db][4 * i + 0] * inv), (_Float16)(st.acc[db][4 * i + 1] * inv),
                 (_Float16)(st.acc[db][4 * i + 2] * inv), (_Float16)(st.acc[db][4 * i + 3] * inv)};
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
