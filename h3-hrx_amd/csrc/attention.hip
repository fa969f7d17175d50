// INT8-QK flash attention for gfx950 (CDNA4): the kernel of the INT4 token-major family (codes
// widened to int8 in registers), its skip twin, the VSA attention and the cross-attention groups
// that do not divide eight. The INT8 entries, head-major and token-major, run on the eight-wave
// kernel of attention_hm.hip.
//
// One workgroup = 4 wave64s x 32 queries of one head; keys stream through 64-key LDS tiles;
// two workgroups share a CU (two waves per SIMD). Per wave and key tile:
//   QK   S^T (64 keys x 32 queries) = K (64 x 128 i8) . Q^T on v_mfma_i32_32x32x32_i8, exact
//        int32. With keys as the MFMA rows, lane l owns query l%32; accumulator register r of
//        block b holds MFMA row m = 32b + 8(r/4) + 4(l/32) + r%4. Every softmax statistic
//        (running max, sum, Q scale) is a per-lane scalar; only the tile max is exchanged, once
//        per tile, with the lane's partner in the other half-wave (v_permlane32_swap).
//   K row order  LDS row m of a K tile holds key swap23(m) (bits 2 and 3 exchanged), so the
//        eight accumulator registers 8(g%2)..+7 of block g/2 hold keys 16g + 8(l/32) + 0..7 in
//        order: exactly the B operand layout of a 16-key f16 MFMA step, with V^T in natural key
//        order. P never leaves its registers.
//   dequant  The accumulators start from the bit pattern of 1.5*2^23 instead of 0, so after
//        the MFMA each holds the float 1.5*2^23 + S exactly (|S| <= 128*128*128 < 2^22). One
//        FMA per score then gives u = S*ks: u = acc*ks + (-1.5*2^23*ks), the second term
//        precomputed per key when the tile is staged. No int->float conversion is issued.
//   softmax  online, base 2, in units of u: p = exp2(u*qs*log2e - m). The running max m is
//        raised only when a tile's max exceeds it by more than 8 (p <= 2^8 stays exact enough
//        in f16 and in the f32 sums); only then are the output accumulators rescaled, so in
//        the steady state the O accumulators are touched by nothing but the MFMAs.
//   PV   O^T (128 ch x 32 queries) += V^T . P^T on v_mfma_f32_32x32x16_f16; the row sum is
//        accumulated from the same packed f16 probabilities (a packed f16 add tree per tile).
//
// Software pipeline (one wave, step j): the matrix work of two tiles runs under the vector work
// of one, in a fixed issue order:
//   phase A  QK(j+1): 8 int8 MFMAs   with  exp/pack/sum of tile j's first 16 key slots
//   phase B  PV(j):  16 f16 MFMAs     with  exp/pack/sum of its last 16 slots (feeding PV(j)'s
//                                          later MFMAs), then dequant + max of tile j+1 and the
//                                          raise of the running max
// so every MFMA has independent VALU work to co-issue with. LDS operands are read a few MFMAs
// ahead (H3_ATTN_PF).
//
// Staging: K and V^T tiles go from HBM straight into LDS with buffer_load ... lds (LDS-DMA; no
// registers, no LDS store instructions), through rings of three stages each. Step j reads
// K(j+1) and V(j) and issues the loads of K(j+3) and V(j+2), so every load has two steps to
// land. A wave waits only for its own loads of the previous step before the step's barrier
// (s_waitcnt vmcnt(7)), never for the ones it has just issued. LDS rows are 128 bytes with
// their 16-byte chunks XOR-swizzled by (row/2)%8, so the 32 rows a half-wave reads fall on
// distinct banks. The key scales ks and -1.5*2^23*ks go through registers (one small load per
// wave per step, stored a step later) since the second is computed.
// Global loads use buffer descriptors whose range ends at the last valid key, so keys past the
// sequence read as zero with no per-element test; only the final partial tile is masked.
// Workgroups are remapped so consecutive query blocks of one head run on the same XCD and
// share its L2 while they walk the same K/V stream.
//
// Semantics follow kernels/attention_i8qkhm_mha8_k64_lds_f16_wmma.loom:437-1067 (head-major)
// and kernels/attention_i8qk_family.loom:193-424 (token-major): non-causal MHA, keys >= tokens
// masked, rows >= token_count not written, f16 output [token_count][out_stride].
#include <algorithm>

#include <atomic>
#include <type_traits>

#include "internal.hpp"

namespace h3 {
namespace {

#ifndef H3_ATTN_WAVES
#define H3_ATTN_WAVES 4
#endif
constexpr int kWaves = H3_ATTN_WAVES;  // waves per workgroup, all on one K/V stream
constexpr int kThreads = 64 * kWaves;
constexpr int kQueriesPerWave = 32;
constexpr int kQueriesPerBlock = kWaves * kQueriesPerWave;
constexpr int kKeys = 64;                                   // keys per LDS tile
constexpr int kRowBytes = 128;                              // unpadded, chunks swizzled
constexpr int kKRows = kKeys * kRowBytes;                   // 8192
constexpr int kKStage = kKRows + 2 * kKeys * 4;             // + ks[64], -M*ks[64]: 8704
constexpr int kVStage = 128 * kRowBytes;                    // 16384
constexpr int kKLoads = 8 / kWaves;                         // 1 KiB LDS-DMA loads per wave
constexpr int kVLoads = 16 / kWaves;
constexpr int kSRows = kKeys / kWaves;                      // scale rows stored per wave
// Operand layouts: int8 codes token-major (attention_i8qk_*) or head-major (attention_i8qkhm_*),
// and int4 codes token-major (attention_i4qk_*, eight codes per word, low nibble first).
// kTokenI4Skip is the int4 kernel with the tile skip of attention_i4qks_* (a threshold tau).
// The int8 token-major layout is also that of the VSA kernel (k_attention_vsa).
enum Mode { kTokenI8 = 0, kHeadI8 = 1, kTokenI4 = 2, kTokenI4Skip = 3 };
constexpr bool isI4(int mode) { return mode == kTokenI4 || mode == kTokenI4Skip; }
constexpr int kI4RowBytes = 64;                             // int4 K tile rows in LDS
constexpr int kKRowsOf(int mode) { return isI4(mode) ? kKeys * kI4RowBytes : kKRows; }
constexpr int kKLoadsOf(int mode) { return isI4(mode) ? 4 / kWaves : kKLoads; }
// s_waitcnt fields (gfx9 layout): vmcnt <= the loads one step issues (K tile, V^T tile, the
// scale load), lgkmcnt 0, expcnt untouched; or vmcnt 0.
constexpr int kWaitPrevStepOf(int mode) {
  return (kKLoadsOf(mode) + kVLoads + 1) | (7 << 4) | (0 << 8);
}
#ifndef H3_ATTN_PF
#define H3_ATTN_PF 2
#endif
constexpr int kPf = H3_ATTN_PF;    // MFMA operands are read from LDS this many MFMAs ahead
constexpr int kSPf = H3_ATTN_PF;   // and the key scales this many chunks ahead
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kMagicBits = 0x4B400000;  // float 12582912 = 1.5 * 2^23
constexpr float kMagic = 12582912.0f;
constexpr float kRescaleSlack = 8.0f;   // raise the running max only past 2^8 growth
constexpr int kRsrcWord3 = 0x00020000;  // gfx9 raw buffer: 32-bit data format, no swizzle
constexpr int kWaitAll = 0 | (7 << 4) | (0 << 8);

typedef __attribute__((address_space(3))) void lds_void;

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
  uint32_t q_row;     // token-major row pitch of qi in bytes (q_stride, or q_stride/2 for int4)
  uint32_t kv_bytes;  // token-major row pitch of ki in bytes (kv_stride, or kv_stride/2)
  uint32_t out_stride;
  uint32_t q_blocks;  // ceil(token_count / 128)
  uint32_t heads;     // workload heads (grid y of the reference)
  uint32_t kv_head_limit;
  uint32_t head_limit;
  // Token-major Q scales [capacity][q_scale_pitch]: the heads a q_stride-wide code row holds
  // (q_stride/128), which is what the quantizer writes per token. The reference's token-major
  // kernel reads them at out_stride/128 instead (attention_i8qk_family.loom:87, 112, 197); the
  // two agree unless the output pitch is padded (src/stack.rs:751-758), where its reading would
  // take another (token, head)'s scale.
  uint32_t q_scale_pitch;
  uint32_t total;      // q_blocks * heads
  uint32_t per_xcd;    // ceil(total / 8)
  float neg_tau;       // tile skip (kTokenI4Skip): -tau * log2(e)
  const uint8_t* key_mask;  // k_attention_cross: [tokens], nonzero = key attended
  uint32_t q_tokens;        // k_attention_cross: query rows (tokens counts the keys)
  uint32_t q_capacity;      // k_attention_cross: head-major row capacity of qi / qs
  uint32_t kv_group;        // k_attention_cross: query heads per key/value head
  const int32_t* routes;   // k_attention_vsa: [head_limit][blocks][blocks], nonzero = kept
  const int32_t* lengths;  // k_attention_vsa: live keys of each 64-key cube
  uint32_t blocks;         // k_attention_vsa: tokens / 64
  uint32_t base;           // k_attention_vsa: first (head, cube) item of this launch
  float scale;             // k_attention_vsa<·, true>: the score scale of the f16 operands
};

__device__ __forceinline__ uint32_t swap23(uint32_t m) {
  return (m & ~12u) | ((m & 4u) << 1) | ((m & 8u) >> 1);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           kRsrcWord3);
}

// Per-thread constants of the staging loads.
struct Stager {
  uint32_t koff[kKLoads];  // byte offset inside a K tile of this lane's 16 bytes, per DMA load
  uint32_t voff[kVLoads];  // byte offset inside a V^T tile (from the head block base + 2*k0)
  uint32_t soff;     // ks element offset (bytes) of this lane's scale row
  uint32_t srow;     // MFMA row whose scales this lane stores (lanes below kSRows)
  int wave;
};

// LDS byte o of a K/V^T stage holds row o/128, logical chunk ((o/16)%8) ^ ((row/2)%8). An int4
// K stage has 64-byte rows: byte o holds row o/64, logical chunk ((o/16)%4) ^ ((row/4)%4), so the
// sixteen rows a quarter-wave reads with one 16-byte load each fall on distinct banks.
// kHmScales (token-major modes): the key scales are read from a head-major copy,
// [kv_head_limit][tokens], instead of the token-major [token][kv_head_limit] array.
template <int kMode, bool kHmScales = false>
__device__ __forceinline__ Stager make_stager(const Args& a, int wave, int lane) {
  constexpr bool kHeadMajor = kMode == kHeadI8;
  Stager s;
  s.wave = wave;
  if constexpr (isI4(kMode)) {
#pragma unroll
    for (int t = 0; t < kKLoadsOf(kMode); ++t) {
      const uint32_t o = (wave * kKLoadsOf(kMode) + t) * 1024 + 16 * lane;
      const uint32_t row = o >> 6, chunk = ((o >> 4) & 3) ^ ((row >> 2) & 3);
      s.koff[t] = swap23(row) * a.kv_bytes + 16 * chunk;
    }
  } else {
#pragma unroll
    for (int t = 0; t < kKLoads; ++t) {
      const uint32_t o = (wave * kKLoads + t) * 1024 + 16 * lane;
      const uint32_t row = o >> 7, chunk = ((o >> 4) & 7) ^ ((row >> 1) & 7);
      const uint32_t key = swap23(row);
      s.koff[t] = (kHeadMajor ? key * 128 : key * a.kv_bytes) + 16 * chunk;
    }
  }
#pragma unroll
  for (int t = 0; t < kVLoads; ++t) {
    const uint32_t o = (wave * kVLoads + t) * 1024 + 16 * lane;
    const uint32_t row = o >> 7, chunk = ((o >> 4) & 7) ^ ((row >> 1) & 7);
    s.voff[t] = row * a.capacity * 2 + 16 * chunk;
  }
  s.srow = kSRows * wave + (lane & (kSRows - 1));
  const uint32_t skey = swap23(s.srow);
  s.soff = kHeadMajor || kHmScales ? skey * 4 : skey * a.kv_head_limit * 4;
  return s;
}

// LDS-DMA of K tile k0 (rows past the sequence load as zero) into stage `kst`, and the load of
// its scales into a register.
template <int kMode, bool kHmScales = false>
__device__ __forceinline__ float stage_k(const Args& a, const Stager& sg, uint32_t kv_head,
                                         uint32_t k0, char* kst) {
  constexpr bool kHeadMajor = kMode == kHeadI8;
  constexpr uint32_t kCodeBytes = isI4(kMode) ? 64 : 128;  // code bytes per (key, head)
  const uint32_t live = a.tokens > k0 ? min(a.tokens - k0, (uint32_t)kKeys) : 0u;
  const char* base;
  uint32_t bytes;
  const float* sbase;
  uint32_t sbytes;
  if (kHeadMajor) {
    base = reinterpret_cast<const char*>(a.ki) + ((size_t)kv_head * a.capacity + k0) * 128;
    bytes = live * 128;
    sbase = a.ks + (size_t)kv_head * a.capacity + k0;
    sbytes = live * 4;
  } else {
    base = reinterpret_cast<const char*>(a.ki) + (size_t)k0 * a.kv_bytes + kv_head * kCodeBytes;
    bytes = live ? (live - 1) * a.kv_bytes + kCodeBytes : 0;
    if (kHmScales) {
      sbase = a.ks + (size_t)kv_head * a.tokens + k0;
      sbytes = live * 4;
    } else {
      sbase = a.ks + (size_t)k0 * a.kv_head_limit + kv_head;
      sbytes = live ? ((live - 1) * a.kv_head_limit + 1) * 4 : 0;
    }
  }
  const __amdgpu_buffer_rsrc_t rk = rsrc(base, bytes);
#pragma unroll
  for (int t = 0; t < kKLoadsOf(kMode); ++t)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rk, (lds_void*)(kst + (sg.wave * kKLoadsOf(kMode) + t) * 1024), 16, sg.koff[t], 0, 0, 0);
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsrc(sbase, sbytes),
                                                                         sg.soff, 0, 0));
}

// LDS-DMA of V^T tile k0 into stage `vst`. The range ends at the end of this head's V^T block;
// columns past `tokens` inside it are zero (the transposes clear them) or belong to the next
// row, and are multiplied by probability 0.
__device__ __forceinline__ void stage_v(const Args& a, const Stager& sg, uint32_t kv_head,
                                        uint32_t k0, char* vst) {
  const uint32_t blk = 128 * a.capacity;  // elements of this head's V^T block
  const char* base = reinterpret_cast<const char*>(a.vt) + ((size_t)kv_head * blk + k0) * 2;
  const __amdgpu_buffer_rsrc_t rv = rsrc(base, k0 < blk ? (blk - k0) * 2 : 0u);
#pragma unroll
  for (int t = 0; t < kVLoads; ++t)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rv, (lds_void*)(vst + (sg.wave * kVLoads + t) * 1024), 16, sg.voff[t], 0, 0, 0);
}

// Scales of a staged K tile: ks and -1.5*2^23*ks at its MFMA-row index.
template <int kMode>
__device__ __forceinline__ void store_scales(char* kst, const Stager& sg, float ks) {
  if ((threadIdx.x & 63) < kSRows) {
    float* sc = reinterpret_cast<float*>(kst + kKRowsOf(kMode));
    sc[sg.srow] = ks;
    sc[kKeys + sg.srow] = -(kMagic * ks);
  }
}


// Barrier between pipeline steps: this wave's LDS writes, and its staging loads from before the
// current step, are complete; the loads issued in this step stay in flight.
template <int kWait>
__device__ __forceinline__ void step_barrier() {
  __builtin_amdgcn_s_waitcnt(kWait);
  asm volatile("s_barrier" ::: "memory");
}

// Per-wave state carried across key tiles.
struct State {
  v16f acc[4];   // O^T, 4 blocks of 32 channels
  float m;       // running max in log2 units (u * qs * log2e)
  float l;       // this lane's partial row sum over its key slots
  float alpha;   // rescale of acc still owed for the last raise of m (1: none)
  float gap;     // last tile's max minus the running max before it (log2 units; tile skip)
};

// Issue-order fence: the scheduler keeps each chunk's MFMA, LDS reads and VALU work together.
#define H3_CHUNK_END() __builtin_amdgcn_sched_barrier(0)

// Probabilities of key slots r, r+1 of S^T block bb: exp2, pack to f16 (B operand of PV).
template <bool kMasked>
__device__ __forceinline__ void exp_pair(const float (&u)[2][16], int bb, int r, float qsl,
                                         float negm, v8h (&pb)[4]) {
  float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(u[bb][r], qsl, negm));
  float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(u[bb][r + 1], qsl, negm));
  if (kMasked) {
    if (u[bb][r] == -INFINITY) p0 = 0.0f;
    if (u[bb][r + 1] == -INFINITY) p1 = 0.0f;
  }
  const v2h pair = {(_Float16)p0, (_Float16)p1};
  pb[2 * bb + r / 8][r % 8] = pair[0];
  pb[2 * bb + r / 8][r % 8 + 1] = pair[1];
}

// This lane's sum of a tile's 32 packed f16 probabilities: a tree of packed f16 adds (15 full-rate
// v_pk_add_f16) and one v_dot2 into f32, instead of a v_dot2 (two VALU slots each) per pair. The
// partial sums stay below 2^13 (p <= 2^8 under the lazy max), well inside f16's range.
__device__ __forceinline__ float tile_sum(const v8h (&pb)[4]) {
  const v8h t8 = (pb[0] + pb[1]) + (pb[2] + pb[3]);
  const v4h t4 = v4h{t8[0], t8[1], t8[2], t8[3]} + v4h{t8[4], t8[5], t8[6], t8[7]};
  const v2h t2 = v2h{t4[0], t4[1]} + v2h{t4[2], t4[3]};
  return __builtin_amdgcn_fdot2(t2, v2h{(_Float16)1.0f, (_Float16)1.0f}, 0.0f, false);
}

// max3 kept where it is written: as an opaque instruction it is neither reassociated into one
// tree at the end of the step nor moved out of its issue chunk.
__device__ __forceinline__ float max3(float a, float b, float c) {
  float r;
  asm volatile("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// Dequantize four key slots (S^T block bb, registers 4i..4i+3) of a fresh tile into u. key0 is
// the key of the first of them; the other three follow it.
template <bool kMasked>
__device__ __forceinline__ void dequant4(const v16i (&s)[2], int bb, int i, float4 k4, float4 c4,
                                         float (&u)[2][16], float& tmax, uint32_t key0,
                                         uint32_t tokens) {
  const float kv[4] = {k4.x, k4.y, k4.z, k4.w};
  const float cv[4] = {c4.x, c4.y, c4.z, c4.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float v = __builtin_fmaf(__int_as_float(s[bb][4 * i + j]), kv[j], cv[j]);
    if (kMasked && key0 + j >= tokens) v = -INFINITY;
    u[bb][4 * i + j] = v;
  }
  tmax = max3(tmax, max3(u[bb][4 * i], u[bb][4 * i + 1], u[bb][4 * i + 2]), u[bb][4 * i + 3]);
}

// Key of the first of the four slots (bb, 4i..4i+3) in lane half `half`: swap23 of the MFMA row.
__device__ __forceinline__ uint32_t slot_key(int bb, int i, int half) {
  return 32 * bb + 16 * (i >> 1) + 8 * half + 4 * (i & 1);
}

// The tile max of both half-waves: v_permlane32_swap exchanges lanes l and l+32 on the vector
// pipe (no LDS round trip).
__device__ __forceinline__ float half_swap_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Tile max -> lazy raise of the running max; the accumulator rescale is owed to the next step.
__device__ __forceinline__ void raise_max(float tmax, float qsl, State& st) {
  tmax = half_swap_max(tmax);
  const float mt = tmax * qsl;
  st.gap = mt - st.m;
  const float m_new = mt > st.m + kRescaleSlack ? mt : st.m;
  const float alpha = __builtin_amdgcn_exp2f(st.m - m_new);
  st.l *= alpha;
  st.alpha *= alpha;
  st.m = m_new;
}

// max(v, v of the lane the DPP control selects): quad_perm [1,0,3,2] (0xB1) and [2,3,0,1]
// (0x4E), row_half_mirror (0x141, lane i <-> 7-i of each 8) and row_mirror (0x140, i <-> 15-i of
// each 16) reduce over 16 lanes on the vector pipe, with no LDS round trip.
template <int kCtrl>
__device__ __forceinline__ float dpp_max(float v) {
  const int o = __builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), kCtrl, 0xF, 0xF,
                                            false);
  return fmaxf(v, __int_as_float(o));
}

// Tile skip decision (kernels/attention_i4qks_family.loom:318-324): the largest gap between a
// tile's max and the running max before it over the wave's 32 queries (lanes 0-31; lanes 32-63
// hold the same queries), wave-uniform.
__device__ __forceinline__ float wave_gap(float gap) {
  gap = dpp_max<0xB1>(gap);
  gap = dpp_max<0x4E>(gap);
  gap = dpp_max<0x141>(gap);
  gap = dpp_max<0x140>(gap);
  const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gap), 0));
  const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gap), 16));
  return fmaxf(a, b);
}

// LDS byte offset, inside a row, of logical 16-byte chunk 2x + half for rows with (row/2)%8 = sw.
__device__ __forceinline__ uint32_t chunk_off(int x, int half, uint32_t sw) {
  return 16 * ((2 * x + half) ^ sw);
}

// int4 operands: eight 4-bit codes of a word become int8 lanes holding 16x the code,
// ((w << 4) & 0xF0F0F0F0) for the low nibbles and (w & 0xF0F0F0F0) for the high ones, so the
// int8 MFMA computes 256x the int4 dot product exactly (|256 S| < 2^21). The same byte order is
// used for Q and K, so the permutation of dimensions it implies cancels in the dot product.
// The 16 bytes at int4 row offset 16(2p + half) hold the operands of MFMA chunks 2p and 2p + 1.
__device__ __forceinline__ v4i widen_i4(uint32_t x0, uint32_t x1) {
  const v4i r = {(int)((x0 << 4) & 0xF0F0F0F0u), (int)(x0 & 0xF0F0F0F0u),
                 (int)((x1 << 4) & 0xF0F0F0F0u), (int)(x1 & 0xF0F0F0F0u)};
  return r;
}
// The packed int4 codes of MFMA chunks (bb, 2p) (words x, y) and (bb, 2p + 1) (words z, w) from
// an int4 stage (64-byte rows, chunks swizzled by (row/4)%4; row 32bb + n, with (n/4)%4 = g).
__device__ __forceinline__ uint4 k_raw_i4(const char* kst, int n, int half, uint32_t g, int bb,
                                          int p) {
  return *reinterpret_cast<const uint4*>(kst + (32 * bb + n) * kI4RowBytes +
                                         16 * ((2 * p + half) ^ g));
}
// K operands of MFMA chunks (bb, 2p) and (bb, 2p + 1) from an int4 stage, widened.
__device__ __forceinline__ void k_pair_i4(const char* kst, int n, int half, uint32_t g, int bb,
                                          int p, v4i& even, v4i& odd) {
  const uint4 w = *reinterpret_cast<const uint4*>(kst + (32 * bb + n) * kI4RowBytes +
                                                  16 * ((2 * p + half) ^ g));
  even = widen_i4(w.x, w.y);
  odd = widen_i4(w.z, w.w);
}

// The first tile's QK and dequant (no softmax work to overlap yet).
template <int kMode, bool kMasked>
__device__ __forceinline__ void first_tile(const char* kst, const v4i (&qop)[4], float qsl,
                                           State& st, float (&u)[2][16], int n, int half,
                                           uint32_t tokens) {
  const v16i magic = {kMagicBits, kMagicBits, kMagicBits, kMagicBits, kMagicBits, kMagicBits,
                      kMagicBits, kMagicBits, kMagicBits, kMagicBits, kMagicBits, kMagicBits,
                      kMagicBits, kMagicBits, kMagicBits, kMagicBits};
  const uint32_t sw = (n >> 1) & 7;
  const char* krow = kst + n * kRowBytes;
  const float* kss = reinterpret_cast<const float*>(kst + kKRowsOf(kMode));
  v16i s[2];
  if constexpr (isI4(kMode)) {
    v4i kop[8];
#pragma unroll
    for (int q = 0; q < 4; ++q)
      k_pair_i4(kst, n, half, (n >> 2) & 3, q & 1, q >> 1, kop[4 * (q >> 1) + (q & 1)],
                kop[4 * (q >> 1) + 2 + (q & 1)]);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int bb = c & 1, dc = c >> 1;
      s[bb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(kop[c], qop[dc], dc == 0 ? magic : s[bb], 0, 0, 0);
    }
  } else {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int bb = c & 1, dc = c >> 1;
      const v4i kop = *reinterpret_cast<const v4i*>(krow + bb * 32 * kRowBytes + chunk_off(dc, half, sw));
      s[bb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(kop, qop[dc], dc == 0 ? magic : s[bb], 0, 0, 0);
    }
  }
  float tmax = -INFINITY;
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int bb = q >> 2, i = q & 3;
    const int kb = 32 * bb + 8 * i + 4 * half;
    dequant4<kMasked>(s, bb, i, *reinterpret_cast<const float4*>(kss + kb),
                      *reinterpret_cast<const float4*>(kss + kKeys + kb), u, tmax,
                      slot_key(bb, i, half), tokens);
  }
  raise_max(tmax, qsl, st);
}

// One pipeline step: QK(j+1) and PV(j) under tile j's softmax and tile j+1's dequant.
//   kst    LDS stage of K(j+1) (unused when !kNext), vst  LDS stage of V(j)
//   u      in: tile j's dequantized scores; out: tile j+1's
//   knext0 first key of tile j+1
//   skip   (kTokenI4Skip only, wave-uniform) tile j is skipped: no probabilities and no PV;
//          tile j+1 is still prepared
template <int kMode, bool kNext, bool kMaskNext, bool kMaskCur>
__device__ __forceinline__ void step(const char* kst, const char* vst, const v4i (&qop)[4],
                                     float qsl, State& st, float (&u)[2][16], int n, int half,
                                     uint32_t knext0, uint32_t tokens, bool skip = false) {
  const bool do_pv = kMode != kTokenI4Skip || !skip;
  constexpr bool do_qk = kNext;
  // The rescale owed by the last raise of m, now that PV(j-1) has accumulated.
  if (__any(st.alpha != 1.0f)) {
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) st.acc[db][r] *= st.alpha;
    st.alpha = 1.0f;
  }
  const v16i magic = {kMagicBits, kMagicBits, kMagicBits, kMagicBits, kMagicBits, kMagicBits,
                      kMagicBits, kMagicBits, kMagicBits, kMagicBits, kMagicBits, kMagicBits,
                      kMagicBits, kMagicBits, kMagicBits, kMagicBits};
  const float negm = -st.m;
  const uint32_t sw = (n >> 1) & 7;
  const char* krow = kst + n * kRowBytes;  // + 32*bb rows + chunk_off(dc)
  const char* vrow = vst + n * kRowBytes;  // + 32*db rows + chunk_off(g)
  const float* kss = reinterpret_cast<const float*>(kst + kKRowsOf(kMode));
  v16i s[2];
  v8h pb[4];
  v4i kop[8];
  uint4 kraw[4];  // int4: the packed codes of MFMA chunks (bb, 2p) and (bb, 2p + 1), p = i / 2
  v8h vop[16];
  float4 k4[8], c4[8];

  // ---- phase A: QK(j+1) || probabilities of slots 0..15 (block 0)
  constexpr bool kI4 = isI4(kMode);
  if (do_qk) {
    if constexpr (kI4) {  // codes of chunks 0..3 now, 4..7 two MFMAs ahead of their use; each
                          // chunk is widened just before its MFMA (half the registers held)
      kraw[0] = k_raw_i4(kst, n, half, (n >> 2) & 3, 0, 0);
      kraw[1] = k_raw_i4(kst, n, half, (n >> 2) & 3, 1, 0);
    } else {
#pragma unroll
      for (int w = 0; w < kPf; ++w)
        kop[w] = *reinterpret_cast<const v4i*>(krow + (w & 1) * 32 * kRowBytes + chunk_off(w >> 1, half, sw));
    }
  }
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const int bb = c & 1, dc = c >> 1;
    if constexpr (kI4) {
      if (do_qk && c == 2) {
        kraw[2] = k_raw_i4(kst, n, half, (n >> 2) & 3, 0, 1);
        kraw[3] = k_raw_i4(kst, n, half, (n >> 2) & 3, 1, 1);
      }
      if (do_qk) {
        const uint4 w = kraw[(c >> 2) * 2 + (c & 1)];
        kop[c] = (c >> 1) & 1 ? widen_i4(w.z, w.w) : widen_i4(w.x, w.y);
      }
    } else if (do_qk && c + kPf < 8) {
      const int w = c + kPf;
      kop[w] = *reinterpret_cast<const v4i*>(krow + (w & 1) * 32 * kRowBytes + chunk_off(w >> 1, half, sw));
    }
    if (do_pv && c >= 8 - kPf) {
      const int w = c - (8 - kPf);
      vop[w] = *reinterpret_cast<const v8h*>(vrow + (w & 3) * 32 * kRowBytes + chunk_off(w >> 2, half, sw));
    }
    if (do_qk)
      s[bb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(kop[c], qop[dc], dc == 0 ? magic : s[bb], 0, 0, 0);
    if (do_pv) exp_pair<kMaskCur>(u, 0, 2 * c, qsl, negm, pb);
    H3_CHUNK_END();
  }

  // ---- phase B: PV(j) || probabilities of slots 16..31, then dequant + max of tile j+1
  float tmax = -INFINITY;
#pragma unroll
  for (int c = 0; c < 16; ++c) {
    const int g = c >> 2, db = c & 3;
    if (do_pv && c + kPf < 16) {
      const int w = c + kPf;
      vop[w] = *reinterpret_cast<const v8h*>(vrow + (w & 3) * 32 * kRowBytes + chunk_off(w >> 2, half, sw));
    }
    if (do_qk && c >= 6 - kSPf && c < 14 - kSPf) {  // scales of dequant quarter q, kSPf ahead
      const int q = c - (6 - kSPf), kb = 32 * (q >> 2) + 8 * (q & 3) + 4 * half;
      k4[q] = *reinterpret_cast<const float4*>(kss + kb);
      c4[q] = *reinterpret_cast<const float4*>(kss + kKeys + kb);
    }
    if (do_pv) {
      st.acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vop[c], pb[g], st.acc[db], 0, 0, 0);
      if (c < 8) exp_pair<kMaskCur>(u, 1, 2 * c, qsl, negm, pb);
    }
    if (do_qk && c >= 6 && c < 14) {
      const int q = c - 6, bb = q >> 2, i = q & 3;
      dequant4<kMaskNext>(s, bb, i, k4[q], c4[q], u, tmax, knext0 + slot_key(bb, i, half),
                          tokens);
    }
    if (do_qk && c == 14) {  // under the last MFMAs: tile j's probabilities are complete
      if (do_pv) st.l += tile_sum(pb);
      raise_max(tmax, qsl, st);
    }
    H3_CHUNK_END();
  }
  if (!do_qk && do_pv) st.l += tile_sum(pb);
}

template <int kMode, bool kHmScales = false>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void k_attention(Args a) {
  constexpr bool kHeadMajor = kMode == kHeadI8;
  constexpr bool kSkip = kMode == kTokenI4Skip;
  constexpr int kWaitPrevStep = kWaitPrevStepOf(kMode);
  // Three K stages and three V^T stages, each its own array so that the compiler can tell an
  // LDS-DMA into one stage from the reads of another.
  __shared__ __attribute__((aligned(16))) char k0s[kKStage];
  __shared__ __attribute__((aligned(16))) char k1s[kKStage];
  __shared__ __attribute__((aligned(16))) char k2s[kKStage];
  __shared__ __attribute__((aligned(16))) char v0s[kVStage];
  __shared__ __attribute__((aligned(16))) char v1s[kVStage];
  __shared__ __attribute__((aligned(16))) char v2s[kVStage];

  // XCD-aware remap: hardware hands block b to XCD b % 8; give each XCD a contiguous range of
  // the launch's (head, query block) work [base, base + total) so its resident blocks share one
  // head's K/V stream in L2.
  const uint32_t b = blockIdx.x;
  const uint32_t local = (b & 7u) * a.per_xcd + (b >> 3);
  if (local >= a.total) return;
  const uint32_t logical = a.base + local;
  const uint32_t head_y = logical / a.q_blocks;
  const uint32_t qb = logical % a.q_blocks;
  const uint32_t kv_head = head_y % a.kv_head_limit;
  const uint32_t head = kv_head % a.head_limit;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int n = lane & 31;      // query within the wave's tile
  const int half = lane >> 5;   // which 16 key-bytes / key slots this lane holds

  const uint32_t tiles32 = (a.tokens + 31) / 32;
  const uint32_t q_tile = qb * kWaves + wave;
  const uint32_t q_tile_c = q_tile < tiles32 ? q_tile : tiles32 - 1;
  const uint32_t q = q_tile_c * kQueriesPerWave + n;
  const uint32_t q_read = q < a.tokens ? q : a.tokens - 1;

  const Stager sg = make_stager<kMode, kHmScales>(a, wave, lane);
  const uint32_t n_tiles = (a.tokens + kKeys - 1) / kKeys;
  const uint32_t full = a.tokens / kKeys;  // tiles with no key past the sequence

  // ---- prologue: K(0..2) and V(0..1) in flight, scales of K(0), K(1) stored, K(2)'s held
  float ks0 = stage_k<kMode, kHmScales>(a, sg, kv_head, 0, k0s);
  float ks1 = stage_k<kMode, kHmScales>(a, sg, kv_head, kKeys, k1s);
  float ks_held = stage_k<kMode, kHmScales>(a, sg, kv_head, 2 * kKeys, k2s);
  stage_v(a, sg, kv_head, 0, v0s);
  stage_v(a, sg, kv_head, kKeys, v1s);

  // Q^T operand, held for the whole key loop: 4 chunks of 32 channels, 16 bytes per lane.
  v4i qop[4];
  if constexpr (isI4(kMode)) {  // 64 code bytes per (token, head), widened like K
    const char* src = reinterpret_cast<const char*>(a.qi) + (size_t)q_read * a.q_row + head * 64;
    const uint4 w0 = *reinterpret_cast<const uint4*>(src + 16 * half);
    const uint4 w1 = *reinterpret_cast<const uint4*>(src + 16 * (2 + half));
    qop[0] = widen_i4(w0.x, w0.y);
    qop[1] = widen_i4(w0.z, w0.w);
    qop[2] = widen_i4(w1.x, w1.y);
    qop[3] = widen_i4(w1.z, w1.w);
  } else {
    const int32_t* src = kHeadMajor ? a.qi + ((size_t)head * a.capacity + q_read) * 32
                                    : a.qi + (size_t)q_read * (a.q_row / 4) + head * 32;
#pragma unroll
    for (int dc = 0; dc < 4; ++dc) qop[dc] = *reinterpret_cast<const v4i*>(src + 8 * dc + 4 * half);
  }
  const float qsv = kHeadMajor ? a.qs[(size_t)head * a.capacity + q_read]
                               : a.qs[(size_t)q_read * a.q_scale_pitch + head];
  // log2 units; int4 scores arrive 256x (the widened codes are 16x each)
  const float qsl = isI4(kMode) ? qsv * kLog2e * (1.0f / 256.0f) : qsv * kLog2e;

  State st;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) st.acc[db][r] = 0.0f;
  st.m = -1.0e30f;
  st.l = 0.0f;
  st.alpha = 1.0f;

  store_scales<kMode>(k0s, sg, ks0);
  store_scales<kMode>(k1s, sg, ks1);
  step_barrier<kWaitAll>();
  float u[2][16];
  if (full == 0)
    first_tile<kMode, true>(k0s, qop, qsl, st, u, n, half, a.tokens);
  else
    first_tile<kMode, false>(k0s, qop, qsl, st, u, n, half, a.tokens);
  step_barrier<kWaitAll>();  // K(0)'s stage is refilled by step 0
  // Tile skip: whether tile j's probabilities and PV are dropped, decided from its max once it is
  // dequantized (the first tile always stays: the running max before it is -1e30).
  bool skip = false;
  if constexpr (kSkip) skip = wave_gap(st.gap) < a.neg_tau;
#define H3_STEP(KN, KMN, KMC, KST, VST, KNEXT0)                                                \
  {                                                                                          \
    step<kMode, KN, KMN, KMC>(KST, VST, qop, qsl, st, u, n, half, KNEXT0, a.tokens, skip);   \
    if (kSkip && KN) skip = wave_gap(st.gap) < a.neg_tau;                                    \
  }

  // One steady step j (tile j+1 full) on compile-time stages: reads K(j+1) from kn, V(j) from
  // vc; stages K(j+3) into kc (K(j)'s stage) and V(j+2) into vn2 (V(j-1)'s stage); stores the
  // scales of K(j+2) (stage kn2) loaded one step earlier.
#define H3_STEADY(kc, kn, kn2, vc, vn2)                                                       \
  {                                                                                          \
    const float ks_new = stage_k<kMode, kHmScales>(a, sg, kv_head, (j + 3) * kKeys, kc);           \
    stage_v(a, sg, kv_head, (j + 2) * kKeys, vn2);                                           \
    H3_STEP(true, false, false, kn, vc, (j + 1) * kKeys)                                     \
    store_scales<kMode>(kn2, sg, ks_held);                                                   \
    ks_held = ks_new;                                                                        \
    step_barrier<kWaitPrevStep>();                                                           \
    ++j;                                                                                     \
  }

  // ---- steady steps, three per iteration so every stage is a fixed array
  const uint32_t steady = full > 0 ? full - 1 : 0;  // steps j with tile j+1 full
  uint32_t j = 0;
  for (; j + 3 <= steady;) {
    H3_STEADY(k0s, k1s, k2s, v0s, v2s)
    H3_STEADY(k1s, k2s, k0s, v1s, v0s)
    H3_STEADY(k2s, k0s, k1s, v2s, v1s)
  }
  if (j < steady) H3_STEADY(k0s, k1s, k2s, v0s, v2s)
  if (j < steady) H3_STEADY(k1s, k2s, k0s, v1s, v0s)
#undef H3_STEADY

  // ---- tail (stages chosen at run time): the step into the partial tile, then the last step
  auto kst = [&](uint32_t t) { const uint32_t r = t % 3; return r == 0 ? k0s : r == 1 ? k1s : k2s; };
  auto vst = [&](uint32_t t) { const uint32_t r = t % 3; return r == 0 ? v0s : r == 1 ? v1s : v2s; };
  if (n_tiles > full && full > 0) {  // j == full - 1: tile j+1 is the partial tile
    H3_STEP(true, true, false, kst(j + 1), vst(j), (j + 1) * kKeys)
    step_barrier<kWaitAll>();
    ++j;
  }
  if (n_tiles > full)
    H3_STEP(false, false, true, nullptr, vst(j), 0)
  else
    H3_STEP(false, false, false, nullptr, vst(j), 0)
#undef H3_STEP
  // The last step raises no max, so no rescale is owed after its PV.
  step_barrier<kWaitAll>();  // no staging load outlives the workgroup

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

// ---------------------------------------------------------------- VSA block-sparse attention
//
// kernels/vsa_attention_8.loom: query cube b (64 queries in the gathered layout) attends to the
// keys of every key cube kb with routes[head][b][kb] != 0, and within a cube only to its first
// lengths[kb] keys. Each query cube keeps its own set of key cubes, so a workgroup here holds
// one query cube (two waves of 32 queries) and walks only that cube's keys: no wave ever waits
// on tiles another query cube keeps. To run two waves per SIMD with a K/V^T stream per
// workgroup, four workgroups share a CU, and the three-stage rings hold 32-key tiles (half a
// cube): 3 x (4,352 + 8,192) bytes per workgroup.
//
// Memory: a kept cube costs 24.5 KB of K and V^T, and the kept sets of different query cubes
// are unrelated, so the tiles mostly come from beyond L2. Two things keep that traffic down:
// one launch per generation of resident workgroups (they start together and walk their
// ascending key lists at about the same pace, so more shared tiles are still in L2), and key
// scales in head-major order when the caller lends a workspace: token-major scales
// ([token][head] f32) put each key's scale in its own 128-byte line shared with the other heads,
// so a 32-key tile would pull 4 KB of lines for 128 bytes of scales (kHmScales: the launcher
// first transposes them into the workspace).
//
// Per run of the key loop the workgroup scans its route row into an LDS list
// of the live half-cubes it keeps (ascending keys, up to kVsaListMax per run; more runs continue
// the same online softmax). Keys past a cube's live length are masked through their staged scale
// pair (ks, -inf), so the loop has no masked variant. The per-tile work is that of k_attention on
// a 32-key tile: S^T is one 32 x 32 block, whose sixteen accumulator registers hold keys
// 8h + 0..7 (registers 0..7, h = lane / 32) and 16 + 8h + 0..7 (registers 8..15) under the same
// K row permutation, i.e. the B operands of two 16-key f16 MFMA steps.
constexpr int kVsaWaves = 2;
constexpr int kVsaThreads = 64 * kVsaWaves;
constexpr int kVsaKeys = 32;                              // keys per tile: half a cube
constexpr int kVsaKRows = kVsaKeys * kRowBytes;           // 4096
constexpr int kVsaKStage = kVsaKRows + 2 * kVsaKeys * 4;  // + ks[32], -M*ks[32]: 4352
constexpr int kVsaVRowBytes = 2 * kVsaKeys;               // a V^T row: 32 keys of f16
constexpr int kVsaVStage = 128 * kVsaVRowBytes;           // 8192
constexpr int kVsaKLoads = kVsaKRows / 1024 / kVsaWaves;  // 1 KiB LDS-DMA loads per wave: 2
constexpr int kVsaVLoads = kVsaVStage / 1024 / kVsaWaves; // 4
constexpr int kVsaSRows = kVsaKeys / kVsaWaves;           // scale rows stored per wave: 16
constexpr int kVsaWaitPrevStep = (kVsaKLoads + kVsaVLoads + 1) | (7 << 4) | (0 << 8);
constexpr int kVsaListMax = 512;                          // list entries per run of the key loop
// The f16 form (kernels/vsa_attention_16.loom): K and V token-major f16, [tokens][kv_stride].
// A K stage holds 32 rows of 256 bytes (one head's 128 channels) and the keys' masks c (0 for a
// live key, -inf for a dead one); a V stage holds the 32 keys' rows of V as they lie in memory,
// and the PV operand is read from it with the LDS transposed read (ds_read_b64_tr_b16).
constexpr int kVsaF16RowBytes = 256;
constexpr int kVsaF16KRows = kVsaKeys * kVsaF16RowBytes;          // 8192
constexpr int kVsaF16KStage = kVsaF16KRows + kVsaKeys * 4;        // + c[32]: 8320
constexpr int kVsaF16VStage = kVsaKeys * kVsaF16RowBytes;         // 8192
constexpr int kVsaF16KLoads = kVsaF16KRows / 1024 / kVsaWaves;    // 4
constexpr int kVsaF16VLoads = kVsaF16VStage / 1024 / kVsaWaves;   // 4
static_assert(kVsaF16VStage == kVsaVStage, "the V stages of both forms are 8 KiB");
constexpr int kVsaKLoadsMax = kVsaF16KLoads > kVsaKLoads ? kVsaF16KLoads : kVsaKLoads;
constexpr int kVsaVLoadsMax = kVsaF16VLoads > kVsaVLoads ? kVsaF16VLoads : kVsaVLoads;
template <bool kF16> constexpr int vsa_kstage() { return kF16 ? kVsaF16KStage : kVsaKStage; }
constexpr int kVsaPf = 1;  // MFMA operands and key scales read from LDS one chunk ahead (2: +1 %)
// entry: cube (14 bits) | half << 14 | live keys of the half (1..32) << 16
constexpr uint32_t kEntryCube = 0x3fffu;
static_assert(kVsaSRows <= 64 && (kVsaSRows & (kVsaSRows - 1)) == 0, "scale rows per wave");

struct VsaStager {
  uint32_t koff[kVsaKLoadsMax];  // byte offset inside a K tile of this lane's 16 bytes, per load
  uint32_t voff[kVsaVLoadsMax];  // byte offset inside a V^T tile (from the head block base + 2*k0)
                                 // or, f16, inside a V tile (from the tile's first row)
  uint32_t soff;              // ks element offset (bytes) of this lane's scale row
  uint32_t srow;              // MFMA row whose scales this lane stores (lanes below kVsaSRows)
  int wave;
};

// K stage: as in k_attention (128-byte rows, chunks swizzled by (row/2)%8, row m holds key
// swap23(m)). V^T stage: 64-byte rows (one channel, 32 keys), byte o holds row o/64, logical
// chunk ((o/16)%4) ^ ((row/4)%4), so the sixteen rows a quarter-wave reads fall on distinct banks.
//
// f16 stages (kF16): K byte o holds row o/256, logical chunk ((o/16)%16) ^ (row%16), row m holding
// key swap23(m) as above, so the sixteen rows a quarter-wave reads with one 16-byte load fall on
// distinct banks. V byte o holds key o/256 (natural order), logical chunk ((o/16)%16) ^
// (4*(key%4)): a transposed read takes 4 keys x 32 bytes per 16 lanes and 8 keys x 64 bytes per
// 32 lanes (one LDS cycle), and the swizzle puts those 16 chunks on distinct banks.
template <bool kHmScales, bool kF16 = false>
__device__ __forceinline__ VsaStager make_vsa_stager(const Args& a, int wave, int lane) {
  VsaStager s;
  s.wave = wave;
  if constexpr (kF16) {
#pragma unroll
    for (int t = 0; t < kVsaF16KLoads; ++t) {
      const uint32_t o = (wave * kVsaF16KLoads + t) * 1024 + 16 * lane;
      const uint32_t row = o >> 8, chunk = ((o >> 4) & 15) ^ (row & 15);
      s.koff[t] = swap23(row) * a.kv_bytes + 16 * chunk;
    }
#pragma unroll
    for (int t = 0; t < kVsaF16VLoads; ++t) {
      const uint32_t o = (wave * kVsaF16VLoads + t) * 1024 + 16 * lane;
      const uint32_t key = o >> 8, chunk = ((o >> 4) & 15) ^ (4 * (key & 3));
      s.voff[t] = key * a.kv_bytes + 16 * chunk;
    }
    s.srow = kVsaSRows * wave + (lane & (kVsaSRows - 1));
    s.soff = 0;
    return s;
  }
#pragma unroll
  for (int t = 0; t < kVsaKLoads; ++t) {
    const uint32_t o = (wave * kVsaKLoads + t) * 1024 + 16 * lane;
    const uint32_t row = o >> 7, chunk = ((o >> 4) & 7) ^ ((row >> 1) & 7);
    s.koff[t] = swap23(row) * a.kv_bytes + 16 * chunk;
  }
#pragma unroll
  for (int t = 0; t < kVsaVLoads; ++t) {
    const uint32_t o = (wave * kVsaVLoads + t) * 1024 + 16 * lane;
    const uint32_t row = o >> 6, chunk = ((o >> 4) & 3) ^ ((row >> 2) & 3);
    s.voff[t] = row * a.capacity * 2 + 16 * chunk;
  }
  s.srow = kVsaSRows * wave + (lane & (kVsaSRows - 1));
  s.soff = swap23(s.srow) * (kHmScales ? 4u : a.kv_head_limit * 4);
  return s;
}

// LDS-DMA of the `live` keys of K tile k0 into stage `kst` (rows from `live` on load as zero),
// and the load of this lane's key scale (head-major or token-major scales).
template <bool kHmScales, bool kF16 = false>
__device__ __forceinline__ float stage_k_vsa(const Args& a, const VsaStager& sg, uint32_t kv_head,
                                             uint32_t k0, uint32_t live, char* kst) {
  if constexpr (kF16) {  // f16 rows: no scales
    const char* base = reinterpret_cast<const char*>(a.ki) + (size_t)k0 * a.kv_bytes +
                       kv_head * kVsaF16RowBytes;
    const __amdgpu_buffer_rsrc_t rk =
        rsrc(base, live ? (live - 1) * a.kv_bytes + kVsaF16RowBytes : 0u);
#pragma unroll
    for (int t = 0; t < kVsaF16KLoads; ++t)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rk, (lds_void*)(kst + (sg.wave * kVsaF16KLoads + t) * 1024), 16, sg.koff[t], 0, 0, 0);
    return 1.0f;
  }
  const char* base = reinterpret_cast<const char*>(a.ki) + (size_t)k0 * a.kv_bytes + kv_head * 128;
  const __amdgpu_buffer_rsrc_t rk = rsrc(base, live ? (live - 1) * a.kv_bytes + 128 : 0u);
#pragma unroll
  for (int t = 0; t < kVsaKLoads; ++t)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rk, (lds_void*)(kst + (sg.wave * kVsaKLoads + t) * 1024), 16, sg.koff[t], 0, 0, 0);
  const float* sbase = kHmScales ? a.ks + (size_t)kv_head * a.tokens + k0
                                 : a.ks + (size_t)k0 * a.kv_head_limit + kv_head;
  const uint32_t sbytes = kHmScales ? live * 4
                                    : live ? ((live - 1) * a.kv_head_limit + 1) * 4 : 0u;
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsrc(sbase, sbytes),
                                                                         sg.soff, 0, 0));
}

// LDS-DMA of V^T tile k0 (32 columns of every channel row of this head's block); f16: the `live`
// rows of V from key k0 (rows from `live` on load as zero, so a dead key's V is finite).
template <bool kF16 = false>
__device__ __forceinline__ void stage_v_vsa(const Args& a, const VsaStager& sg, uint32_t kv_head,
                                            uint32_t k0, uint32_t live, char* vst) {
  if constexpr (kF16) {
    const char* base = reinterpret_cast<const char*>(a.vt) + (size_t)k0 * a.kv_bytes +
                       kv_head * kVsaF16RowBytes;
    const __amdgpu_buffer_rsrc_t rv =
        rsrc(base, live ? (live - 1) * a.kv_bytes + kVsaF16RowBytes : 0u);
#pragma unroll
    for (int t = 0; t < kVsaF16VLoads; ++t)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rv, (lds_void*)(vst + (sg.wave * kVsaF16VLoads + t) * 1024), 16, sg.voff[t], 0, 0, 0);
    return;
  }
  (void)live;
  const uint32_t blk = 128 * a.capacity;
  const char* base = reinterpret_cast<const char*>(a.vt) + ((size_t)kv_head * blk + k0) * 2;
  const __amdgpu_buffer_rsrc_t rv = rsrc(base, k0 < blk ? (blk - k0) * 2 : 0u);
#pragma unroll
  for (int t = 0; t < kVsaVLoads; ++t)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rv, (lds_void*)(vst + (sg.wave * kVsaVLoads + t) * 1024), 16, sg.voff[t], 0, 0, 0);
}

// Scales of a staged tile: (ks, -1.5*2^23*ks) for a live key, (ks, -inf) for a dead one; f16:
// the mask c alone (0 live, -inf dead).
template <bool kF16 = false>
__device__ __forceinline__ void store_scales_vsa(char* kst, const VsaStager& sg, float ks,
                                                 uint32_t live) {
  if constexpr (kF16) {
    if ((threadIdx.x & 63) < kVsaSRows)
      reinterpret_cast<float*>(kst + kVsaF16KRows)[sg.srow] =
          swap23(sg.srow) < live ? 0.0f : -INFINITY;
    return;
  }
  if ((threadIdx.x & 63) < kVsaSRows) {
    float* sc = reinterpret_cast<float*>(kst + kVsaKRows);
    sc[sg.srow] = ks;
    sc[kVsaKeys + sg.srow] = swap23(sg.srow) < live ? -(kMagic * ks) : -INFINITY;
  }
}

// Probabilities of slots r, r+1 of a 32-key tile into pb[r/8].
__device__ __forceinline__ void exp_pair_vsa(const float (&u)[16], int r, float qsl, float negm,
                                             v8h (&pb)[2]) {
  const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(u[r], qsl, negm));
  const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(u[r + 1], qsl, negm));
  pb[r / 8][r % 8] = (_Float16)p0;
  pb[r / 8][r % 8 + 1] = (_Float16)p1;
}

// Dequantize slots 4i..4i+3 of a fresh 32-key tile into u and fold them into the tile max.
__device__ __forceinline__ void dequant_vsa(const v16i& s, int i, float4 k4, float4 c4,
                                            float (&u)[16], float& tmax) {
  u[4 * i + 0] = __builtin_fmaf(__int_as_float(s[4 * i + 0]), k4.x, c4.x);
  u[4 * i + 1] = __builtin_fmaf(__int_as_float(s[4 * i + 1]), k4.y, c4.y);
  u[4 * i + 2] = __builtin_fmaf(__int_as_float(s[4 * i + 2]), k4.z, c4.z);
  u[4 * i + 3] = __builtin_fmaf(__int_as_float(s[4 * i + 3]), k4.w, c4.w);
  tmax = max3(tmax, max3(u[4 * i], u[4 * i + 1], u[4 * i + 2]), u[4 * i + 3]);
}

// This lane's sum of a 32-key tile's 16 packed f16 probabilities.
__device__ __forceinline__ float tile_sum_vsa(const v8h (&pb)[2]) {
  const v8h t8 = pb[0] + pb[1];
  const v4h t4 = v4h{t8[0], t8[1], t8[2], t8[3]} + v4h{t8[4], t8[5], t8[6], t8[7]};
  const v2h t2 = v2h{t4[0], t4[1]} + v2h{t4[2], t4[3]};
  return __builtin_amdgcn_fdot2(t2, v2h{(_Float16)1.0f, (_Float16)1.0f}, 0.0f, false);
}

// K operand of QK chunk dc (32 channels) and V^T operand of PV chunk w (channel block w%4,
// key half w/4) for this lane.
__device__ __forceinline__ v4i k_op_vsa(const char* kst, int n, int half, int dc) {
  return *reinterpret_cast<const v4i*>(kst + n * kRowBytes + chunk_off(dc, half, (n >> 1) & 7));
}
__device__ __forceinline__ v8h v_op_vsa(const char* vst, int n, int half, int w) {
  const int db = w & 3, g = w >> 2;
  return *reinterpret_cast<const v8h*>(vst + (32 * db + n) * kVsaVRowBytes +
                                       16 * ((2 * g + half) ^ ((n >> 2) & 3)));
}

// A QK MFMA that starts from the bias `magic` and writes its own registers, so the bias stays in
// place from tile to tile (a builtin MFMA onto a copy of the bias costs 16 moves a tile).
__device__ __forceinline__ v16i qk_onto_vsa(v4i k, v4i q, const v16i& magic) {
  v16i d;
  asm volatile("v_mfma_i32_32x32x32_i8 %0, %1, %2, %3" : "=&v"(d) : "v"(k), "v"(q), "v"(magic));
  return d;
}

// The first tile's QK and dequant.
__device__ __forceinline__ void first_tile_vsa(const char* kst, const v4i (&qop)[4], float qsl,
                                               State& st, float (&u)[16], int n, int half) {
  const v16i magic = {kMagicBits, kMagicBits, kMagicBits, kMagicBits, kMagicBits, kMagicBits,
                      kMagicBits, kMagicBits, kMagicBits, kMagicBits, kMagicBits, kMagicBits,
                      kMagicBits, kMagicBits, kMagicBits, kMagicBits};
  const float* kss = reinterpret_cast<const float*>(kst + kVsaKRows);
  v16i s = magic;
#pragma unroll
  for (int dc = 0; dc < 4; ++dc)
    s = __builtin_amdgcn_mfma_i32_32x32x32_i8(k_op_vsa(kst, n, half, dc), qop[dc], s, 0, 0, 0);
  float tmax = -INFINITY;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int kb = 8 * i + 4 * half;
    dequant_vsa(s, i, *reinterpret_cast<const float4*>(kss + kb),
                *reinterpret_cast<const float4*>(kss + kVsaKeys + kb), u, tmax);
  }
  raise_max(tmax, qsl, st);
}

// One pipeline step on 32-key tiles: QK(j+1) and PV(j) under tile j's softmax and tile j+1's
// dequant, in the issue order of step():
//   phase A  QK(j+1): 4 int8 MFMAs  with  the probabilities of tile j's slots 0..7
//   phase B  PV(j):   8 f16 MFMAs   with  slots 8..15 (feeding PV(j)'s second key half), then
//                                         the dequant + max of tile j+1 and the raise of m
template <bool kNext>
__device__ __forceinline__ void step_vsa(const char* kst, const char* vst, const v4i (&qop)[4],
                                         float qsl, State& st, float (&u)[16], int n, int half,
                                         const v16i& magic) {
  if (__any(st.alpha != 1.0f)) {  // the rescale owed by the last raise of m
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) st.acc[db][r] *= st.alpha;
    st.alpha = 1.0f;
  }
  const float negm = -st.m;
  const float* kss = reinterpret_cast<const float*>(kst + kVsaKRows);
  v16i s;
  v8h pb[2];
  v4i kop[4];
  v8h vop[8];
  float4 k4[4], c4[4];

  // ---- phase A: QK(j+1) || probabilities of slots 0..7
  if (kNext) {
#pragma unroll
    for (int w = 0; w < kVsaPf; ++w) kop[w] = k_op_vsa(kst, n, half, w);
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    if (kNext && c + kVsaPf < 4) kop[c + kVsaPf] = k_op_vsa(kst, n, half, c + kVsaPf);
    if (c >= 4 - kVsaPf) vop[c - (4 - kVsaPf)] = v_op_vsa(vst, n, half, c - (4 - kVsaPf));
    if (kNext) {
      if (c == 0)
        s = qk_onto_vsa(kop[0], qop[0], magic);
      else
        s = __builtin_amdgcn_mfma_i32_32x32x32_i8(kop[c], qop[c], s, 0, 0, 0);
    }
    exp_pair_vsa(u, 2 * c, qsl, negm, pb);
    H3_CHUNK_END();
  }

  // ---- phase B: PV(j) || probabilities of slots 8..15, then dequant + max of tile j+1
  float tmax = -INFINITY;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    if (c + kVsaPf < 8) vop[c + kVsaPf] = v_op_vsa(vst, n, half, c + kVsaPf);
    if (kNext && c >= 3 - kVsaPf && c < 7 - kVsaPf) {  // scales of dequant quarter q, kVsaPf ahead
      const int q = c - (3 - kVsaPf), kb = 8 * q + 4 * half;
      k4[q] = *reinterpret_cast<const float4*>(kss + kb);
      c4[q] = *reinterpret_cast<const float4*>(kss + kVsaKeys + kb);
    }
    st.acc[c & 3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vop[c], pb[c >> 2], st.acc[c & 3], 0, 0, 0);
    if (c < 4) exp_pair_vsa(u, 8 + 2 * c, qsl, negm, pb);
    if (kNext && c >= 3 && c < 7) dequant_vsa(s, c - 3, k4[c - 3], c4[c - 3], u, tmax);
    if (kNext && c == 7) {
      st.l += tile_sum_vsa(pb);
      raise_max(tmax, qsl, st);
    }
    H3_CHUNK_END();
  }
  if (!kNext) st.l += tile_sum_vsa(pb);
}

// ---- the f16 form's per-tile work (kernels/vsa_attention_16.loom: f16 QK in f32, times the
// config scale, softmax, f16 PV): S^T = K Q^T on v_mfma_f32_32x32x16_f16, eight MFMAs per 32-key
// tile, Q (32 queries x 128 channels) held as the B operands; the scores need no dequantisation,
// only the dead-key mask c, so u = S + c; the softmax and PV are those of the int8 form.
typedef short v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s lds_v4s;

// K operand of QK chunk c (channels 16c .. 16c+15): row n, logical chunk 2c + half.
__device__ __forceinline__ v8h k_op_f16(const char* kst, int n, int half, int c) {
  return *reinterpret_cast<const v8h*>(kst + n * kVsaF16RowBytes + 16 * ((2 * c + half) ^ (n & 15)));
}

// PV operand w (channel block w%4, key half w/4) from a V stage: lane l needs
// V[16*(w/4) + 8*(l/32) + i][32*(w%4) + l%32] for i = 0..7 (the A operand of
// v_mfma_f32_32x32x16_f16). The transposed read gives, in each group of 16 lanes, lane i element e
// of the 8-byte piece lane 4e + i/4 points at, element i%4; with lane j pointing at key k0 + j/4,
// channels c0 + 4*(j%4) .. +3, lane i receives V[k0 + e][c0 + i], e = 0..3. Two reads (keys k0 and
// k0 + 4) make the eight keys.
__device__ __forceinline__ v8h v_op_f16(const char* vst, int lane, int w) {
  const int db = w & 3, kh = w >> 2;
  const int g = lane >> 4, j = lane & 15;
  const int key = 16 * kh + 8 * (g >> 1) + (j >> 2);               // key % 4 == j / 4
  const int chunk = 4 * db + 2 * (g & 1) + ((j & 3) >> 1);
  const int off = key * kVsaF16RowBytes + 16 * (chunk ^ (4 * (j >> 2))) + 8 * (j & 1);
  const v4h lo = __builtin_bit_cast(
      v4h, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(vst + off)));
  const v4h hi = __builtin_bit_cast(
      v4h, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(vst + off + 4 * kVsaF16RowBytes)));
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Slots 4i..4i+3 of a fresh tile: u = S + c (c = 0 live, -inf dead), folded into the tile max.
__device__ __forceinline__ void dequant_f16(const v16f& s, int i, float4 c4, float (&u)[16],
                                            float& tmax) {
  u[4 * i + 0] = s[4 * i + 0] + c4.x;
  u[4 * i + 1] = s[4 * i + 1] + c4.y;
  u[4 * i + 2] = s[4 * i + 2] + c4.z;
  u[4 * i + 3] = s[4 * i + 3] + c4.w;
  tmax = max3(tmax, max3(u[4 * i], u[4 * i + 1], u[4 * i + 2]), u[4 * i + 3]);
}

// The probability of slot r into pb[r/8].
__device__ __forceinline__ void exp_one_vsa(const float (&u)[16], int r, float qsl, float negm,
                                            v8h (&pb)[2]) {
  pb[r / 8][r % 8] = (_Float16)__builtin_amdgcn_exp2f(__builtin_fmaf(u[r], qsl, negm));
}

__device__ __forceinline__ void first_tile_f16(const char* kst, const v8h (&qop)[8], float qsl,
                                               State& st, float (&u)[16], int n, int half) {
  const float* kc = reinterpret_cast<const float*>(kst + kVsaF16KRows);
  v16f s = {};
#pragma unroll
  for (int c = 0; c < 8; ++c)
    s = __builtin_amdgcn_mfma_f32_32x32x16_f16(k_op_f16(kst, n, half, c), qop[c], s, 0, 0, 0);
  float tmax = -INFINITY;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    dequant_f16(s, i, *reinterpret_cast<const float4*>(kc + 8 * i + 4 * half), u, tmax);
  raise_max(tmax, qsl, st);
}

// One pipeline step of the f16 form, in the order of step_vsa:
//   phase A  QK(j+1): 8 f16 MFMAs  with  the probabilities of tile j's slots 0..7 (one a chunk)
//   phase B  PV(j):   8 f16 MFMAs  with  slots 8..15, then the mask + max of tile j+1 and the
//                                        raise of m
template <bool kNext>
__device__ __forceinline__ void step_f16(const char* kst, const char* vst, const v8h (&qop)[8],
                                         float qsl, State& st, float (&u)[16], int lane) {
  const int n = lane & 31, half = lane >> 5;
  if (__any(st.alpha != 1.0f)) {  // the rescale owed by the last raise of m
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) st.acc[db][r] *= st.alpha;
    st.alpha = 1.0f;
  }
  const float negm = -st.m;
  const float* kc = reinterpret_cast<const float*>(kst + kVsaF16KRows);
  v16f s = {};
  v8h pb[2];
  v8h kop[8];
  v8h vop[8];
  float4 c4[4];

  // ---- phase A: QK(j+1) || probabilities of slots 0..7
  if (kNext) kop[0] = k_op_f16(kst, n, half, 0);
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    if (kNext && c + 1 < 8) kop[c + 1] = k_op_f16(kst, n, half, c + 1);
    if (c == 7) vop[0] = v_op_f16(vst, lane, 0);
    if (kNext) s = __builtin_amdgcn_mfma_f32_32x32x16_f16(kop[c], qop[c], s, 0, 0, 0);
    exp_one_vsa(u, c, qsl, negm, pb);
    H3_CHUNK_END();
  }

  // ---- phase B: PV(j) || probabilities of slots 8..15, then mask + max of tile j+1
  float tmax = -INFINITY;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    if (c + 1 < 8) vop[c + 1] = v_op_f16(vst, lane, c + 1);
    if (kNext && c >= 2 && c < 6) c4[c - 2] = *reinterpret_cast<const float4*>(kc + 8 * (c - 2) + 4 * half);
    st.acc[c & 3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vop[c], pb[c >> 2], st.acc[c & 3], 0, 0, 0);
    if (c < 4) exp_pair_vsa(u, 8 + 2 * c, qsl, negm, pb);
    if (kNext && c >= 3 && c < 7) dequant_f16(s, c - 3, c4[c - 3], u, tmax);
    if (kNext && c == 7) {
      st.l += tile_sum_vsa(pb);
      raise_max(tmax, qsl, st);
    }
    H3_CHUNK_END();
  }
  if (!kNext) st.l += tile_sum_vsa(pb);
}

template <bool kF16, bool kNext, class QOp>
__device__ __forceinline__ void vsa_step(const char* kst, const char* vst, const QOp& qop,
                                         float qsl, State& st, float (&u)[16], int lane,
                                         const v16i& magic) {
  if constexpr (kF16)
    step_f16<kNext>(kst, vst, qop, qsl, st, u, lane);
  else
    step_vsa<kNext>(kst, vst, qop, qsl, st, u, lane & 31, lane >> 5, magic);
}

__device__ __forceinline__ uint32_t rfl(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }

// kHmScales: a.ks is head-major, [kv_head_limit][tokens]; otherwise token-major as the
// operands' producer writes it, [tokens][kv_head_limit]. kF16: the f16 form (a.qi, a.ki, a.vt
// are the token-major f16 q, k, v; a.q_row and a.kv_bytes their row pitches in bytes; scores
// times a.scale), on two-stage rings so that four workgroups share a CU (35.1 KB of LDS each).
template <bool kHmScales, bool kF16 = false>
__global__ __launch_bounds__(kVsaThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void k_attention_vsa(Args a) {
  __shared__ __attribute__((aligned(16))) char k0s[vsa_kstage<kF16>()];
  __shared__ __attribute__((aligned(16))) char k1s[vsa_kstage<kF16>()];
  __shared__ __attribute__((aligned(16))) char k2s[kF16 ? 16 : kVsaKStage];  // int8: 3 stages
  __shared__ __attribute__((aligned(16))) char v0s[kVsaVStage];
  __shared__ __attribute__((aligned(16))) char v1s[kVsaVStage];
  __shared__ __attribute__((aligned(16))) char v2s[kF16 ? 16 : kVsaVStage];
  __shared__ uint32_t list[kVsaListMax];
  __shared__ uint32_t wave_counts[kVsaWaves];

  // XCD-aware remap of k_attention over the launch's items [base, base + total): each XCD runs
  // a contiguous range of (head, cube) work.
  const uint32_t b = blockIdx.x;
  const uint32_t local = (b & 7u) * a.per_xcd + (b >> 3);
  if (local >= a.total) return;
  const uint32_t logical = a.base + local;
  const uint32_t head_y = logical / a.q_blocks;
  const uint32_t cube = logical % a.q_blocks;  // this workgroup's query cube
  const uint32_t kv_head = head_y % a.kv_head_limit;
  const uint32_t head = kv_head % a.head_limit;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int n = lane & 31;
  const int half = lane >> 5;
  const uint32_t q = cube * 64 + wave * kQueriesPerWave + n;
  const uint32_t q_read = q < a.tokens ? q : a.tokens - 1;

  const VsaStager sg = make_vsa_stager<kHmScales, kF16>(a, wave, lane);
  std::conditional_t<kF16, v8h[8], v4i[4]> qop;
  float qsl;
  if constexpr (kF16) {
    const char* src = reinterpret_cast<const char*>(a.qi) + (size_t)q_read * a.q_row +
                      head * kVsaF16RowBytes;
#pragma unroll
    for (int c = 0; c < 8; ++c) qop[c] = *reinterpret_cast<const v8h*>(src + 32 * c + 16 * half);
    qsl = a.scale * kLog2e;
  } else {
    const int32_t* src = a.qi + (size_t)q_read * (a.q_row / 4) + head * 32;
#pragma unroll
    for (int dc = 0; dc < 4; ++dc) qop[dc] = *reinterpret_cast<const v4i*>(src + 8 * dc + 4 * half);
    qsl = a.qs[(size_t)q_read * a.q_scale_pitch + head] * kLog2e;
  }

  State st;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) st.acc[db][r] = 0.0f;
  st.m = -1.0e30f;
  st.l = 0.0f;
  st.alpha = 1.0f;
  float u[16] = {};
  v16i magic = {};  // the int8 form's QK accumulator bias, kept in registers for the whole walk
  if constexpr (!kF16) {
#pragma unroll
    for (int r = 0; r < 16; ++r) magic[r] = kMagicBits;
    asm volatile("" : "+v"(magic));
  }

  const int32_t* route = a.routes + ((size_t)head * a.blocks + cube) * a.blocks;
  auto k0_of = [](uint32_t e) { return (e & kEntryCube) * 64 + ((e >> 14) & 1u) * kVsaKeys; };
  auto live_of = [](uint32_t e) { return e >> 16; };

  // Route flag and length of this thread's cube in the pass at `at`, loaded together (one round
  // trip) and one pass ahead of their use.
  auto fetch = [&](uint32_t at, int32_t& keep, int32_t& len) {
    const uint32_t kb = at + threadIdx.x;
    keep = 0;
    len = 0;
    if (kb < a.blocks) {
      keep = route[kb];
      len = a.lengths[kb];
    }
  };
  uint32_t scan = 0;  // first key cube not yet listed
  while (scan < a.blocks) {
    // ---- list the live halves of the kept cubes from `scan` on, kVsaThreads cubes per pass
    uint32_t count = 0;
    int32_t keep_next, len_next;
    fetch(scan, keep_next, len_next);
    while (scan < a.blocks) {
      const uint32_t kb = scan + threadIdx.x;
      const int32_t keep = keep_next, len = len_next;
      if (scan + kVsaThreads < a.blocks) fetch(scan + kVsaThreads, keep_next, len_next);
      const uint32_t live = keep == 0 ? 0u : len < 0 ? 0u : len > 64 ? 64u : (uint32_t)len;
      const uint64_t ball0 = __ballot(live > 0);
      const uint64_t ball1 = __ballot(live > (uint32_t)kVsaKeys);
      if (lane == 0) wave_counts[wave] = (uint32_t)(__popcll(ball0) + __popcll(ball1));
      __syncthreads();
      uint32_t before = 0, pass_total = 0;
#pragma unroll
      for (int w = 0; w < kVsaWaves; ++w) {
        const uint32_t c = wave_counts[w];
        before += w < wave ? c : 0u;
        pass_total += c;
      }
      if (count + pass_total > (uint32_t)kVsaListMax) {  // the same decision in every wave
        __syncthreads();
        break;
      }
      if (live > 0) {
        const uint32_t rank =
            __builtin_amdgcn_mbcnt_hi((uint32_t)(ball0 >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)ball0, 0u)) +
            __builtin_amdgcn_mbcnt_hi((uint32_t)(ball1 >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)ball1, 0u));
        const uint32_t at = count + before + rank;
        list[at] = kb | (min(live, (uint32_t)kVsaKeys) << 16);
        if (live > (uint32_t)kVsaKeys) list[at + 1] = kb | (1u << 14) | ((live - kVsaKeys) << 16);
      }
      count += pass_total;
      scan += kVsaThreads;
      __syncthreads();
    }
    if (count == 0) continue;

    auto entry = [&](uint32_t t) { return t < count ? rfl(list[t]) : 0u; };
    if constexpr (kF16) {
      // ---- the f16 form on two-stage rings (35 KB of LDS, four workgroups per CU): step j
      // stages K(j+2) into K(j)'s stage and V(j+1) into V(j-1)'s, with K(j+2)'s key mask (known
      // from the list, no load), while QK(j+1) and PV(j) run; its barrier waits for all of its
      // loads, which the next step reads.
      {
        const uint32_t e0 = entry(0), e1 = entry(1);
        stage_k_vsa<kHmScales, kF16>(a, sg, kv_head, k0_of(e0), live_of(e0), k0s);
        stage_k_vsa<kHmScales, kF16>(a, sg, kv_head, k0_of(e1), live_of(e1), k1s);
        stage_v_vsa<kF16>(a, sg, kv_head, k0_of(e0), live_of(e0), v0s);
        store_scales_vsa<kF16>(k0s, sg, 1.0f, live_of(e0));
        store_scales_vsa<kF16>(k1s, sg, 1.0f, live_of(e1));
      }
      step_barrier<kWaitAll>();
      first_tile_f16(k0s, qop, qsl, st, u, n, half);
      step_barrier<kWaitAll>();
#define H3_VSA_F16_STEP(ka, kb, va, vb)                                                        \
  {                                                                                          \
    const uint32_t ek = entry(j + 2), ev = entry(j + 1);                                     \
    stage_k_vsa<kHmScales, kF16>(a, sg, kv_head, k0_of(ek), live_of(ek), ka);                \
    stage_v_vsa<kF16>(a, sg, kv_head, k0_of(ev), live_of(ev), vb);                           \
    store_scales_vsa<kF16>(ka, sg, 1.0f, live_of(ek));                                       \
    vsa_step<kF16, true>(kb, va, qop, qsl, st, u, lane, magic);                              \
    step_barrier<kWaitAll>();                                                                \
    ++j;                                                                                     \
  }
      const uint32_t steady = count - 1;
      uint32_t j = 0;
      for (; j + 2 <= steady;) {
        H3_VSA_F16_STEP(k0s, k1s, v0s, v1s)
        H3_VSA_F16_STEP(k1s, k0s, v1s, v0s)
      }
      if (j < steady) H3_VSA_F16_STEP(k0s, k1s, v0s, v1s)
#undef H3_VSA_F16_STEP
      vsa_step<kF16, false>(nullptr, (j & 1) ? v1s : v0s, qop, qsl, st, u, lane, magic);
    } else {
      // ---- the pipeline of k_attention over list[0 .. count): tile t is the half-cube list[t]
      uint32_t e2 = entry(2), e3 = entry(3);
      {
        const uint32_t e0 = entry(0), e1 = entry(1);
        const float ks0 = stage_k_vsa<kHmScales, kF16>(a, sg, kv_head, k0_of(e0), live_of(e0), k0s);
        const float ks1 = stage_k_vsa<kHmScales, kF16>(a, sg, kv_head, k0_of(e1), live_of(e1), k1s);
        stage_v_vsa<kF16>(a, sg, kv_head, k0_of(e0), live_of(e0), v0s);
        stage_v_vsa<kF16>(a, sg, kv_head, k0_of(e1), live_of(e1), v1s);
        store_scales_vsa<kF16>(k0s, sg, ks0, live_of(e0));
        store_scales_vsa<kF16>(k1s, sg, ks1, live_of(e1));
      }
      float ks_held = stage_k_vsa<kHmScales, kF16>(a, sg, kv_head, k0_of(e2), live_of(e2), k2s);
      step_barrier<kWaitAll>();
      first_tile_vsa(k0s, qop, qsl, st, u, n, half);
      step_barrier<kWaitAll>();

      // One step j: K(j+3) -> kc, V(j+2) -> vn2; QK(j+1) from kn, PV(j) from vc; then the scales
      // of K(j+2) into kn2.
#define H3_VSA_STEP(kc, kn, kn2, vc, vn2)                                                      \
  {                                                                                          \
    const float ks_new = stage_k_vsa<kHmScales, false>(a, sg, kv_head, k0_of(e3), live_of(e3), \
                                                       kc);                                  \
    stage_v_vsa<false>(a, sg, kv_head, k0_of(e2), live_of(e2), vn2);                         \
    const uint32_t e4 = entry(j + 4);                                                        \
    vsa_step<false, true>(kn, vc, qop, qsl, st, u, lane, magic);                             \
    store_scales_vsa<false>(kn2, sg, ks_held, live_of(e2));                                  \
    ks_held = ks_new;                                                                        \
    e2 = e3;                                                                                 \
    e3 = e4;                                                                                 \
    step_barrier<kVsaWaitPrevStep>();                                                        \
    ++j;                                                                                     \
  }
      const uint32_t steady = count - 1;
      uint32_t j = 0;
      for (; j + 3 <= steady;) {
        H3_VSA_STEP(k0s, k1s, k2s, v0s, v2s)
        H3_VSA_STEP(k1s, k2s, k0s, v1s, v0s)
        H3_VSA_STEP(k2s, k0s, k1s, v2s, v1s)
      }
      if (j < steady) H3_VSA_STEP(k0s, k1s, k2s, v0s, v2s)
      if (j < steady) H3_VSA_STEP(k1s, k2s, k0s, v1s, v0s)
#undef H3_VSA_STEP
      {  // the last tile's PV (stage j % 3)
        const uint32_t r = j % 3;
        vsa_step<kF16, false>(nullptr, r == 0 ? v0s : r == 1 ? v1s : v2s, qop, qsl, st, u, lane,
                              magic);
      }
    }
    step_barrier<kWaitAll>();  // no staging load outlives the run; the stages are reused
  }

  // ---- normalise and store rows < token_count
  const float l_tot = st.l + __shfl_xor(st.l, 32);
  const float inv = 1.0f / l_tot;
  if (q < a.token_count && q < a.tokens) {
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

// Transpose of the key scales of the VSA attention, [tokens][heads] -> [heads][tokens] f32,
// through a 64 x 64 LDS tile (coalesced reads and writes).
__global__ __launch_bounds__(256) void k_scales_head_major(const float* __restrict__ ks,
                                                           float* __restrict__ out,
                                                           uint32_t tokens, uint32_t heads) {
  __shared__ float tile[64][65];
  const uint32_t t0 = blockIdx.x * 64, h0 = blockIdx.y * 64;
  const uint32_t x = threadIdx.x & 63, y = threadIdx.x >> 6;  // 64 x 4 threads
  for (uint32_t r = y; r < 64; r += 4) {
    const uint32_t t = t0 + r, h = h0 + x;
    if (t < tokens && h < heads) tile[r][x] = ks[(size_t)t * heads + h];
  }
  __syncthreads();
  for (uint32_t r = y; r < 64; r += 4) {
    const uint32_t h = h0 + r, t = t0 + x;
    if (t < tokens && h < heads) out[(size_t)h * tokens + t] = tile[x][r];
  }
}

// ---------------------------------------------------------------- cross-attention (GQA, key mask)
//
// An extension with no counterpart in the reference: queries of one sequence (the video + audio
// rows) attend to the keys of another (the text), with grouped heads (query head h reads key /
// value head h / kv_group) and a key-padding mask (keys with key_mask == 0, and keys past the
// key count, get probability 0). Head-major int8 operands as attention_i8qkhm, separate row
// capacities for Q and K. The key loop is the pipeline of k_attention; every tile is masked
// through its staged scale pairs (ks, -inf for a dead key), so no tile needs the masked step.

// Whether key k0 + (this lane's scale row) is attended; read by the lanes that store scales.
__device__ __forceinline__ bool key_live(const Args& a, const Stager& sg, uint32_t k0) {
  const uint32_t key = k0 + swap23(sg.srow);
  return key < a.tokens && a.key_mask[key] != 0;
}

__device__ __forceinline__ void store_scales_mask(char* kst, const Stager& sg, float ks,
                                                  bool live) {
  if ((threadIdx.x & 63) < kSRows) {
    float* sc = reinterpret_cast<float*>(kst + kKRows);
    sc[sg.srow] = ks;
    sc[kKeys + sg.srow] = live ? -(kMagic * ks) : -INFINITY;
  }
}

__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void k_attention_cross(Args a) {
  constexpr int kMode = kHeadI8;
  constexpr int kWaitPrevStep = kWaitPrevStepOf(kMode);
  __shared__ __attribute__((aligned(16))) char k0s[kKStage];
  __shared__ __attribute__((aligned(16))) char k1s[kKStage];
  __shared__ __attribute__((aligned(16))) char k2s[kKStage];
  __shared__ __attribute__((aligned(16))) char v0s[kVStage];
  __shared__ __attribute__((aligned(16))) char v1s[kVStage];
  __shared__ __attribute__((aligned(16))) char v2s[kVStage];

  const uint32_t b = blockIdx.x;
  const uint32_t logical = (b & 7u) * a.per_xcd + (b >> 3);
  if (logical >= a.total) return;
  const uint32_t head = logical / a.q_blocks;  // query head
  const uint32_t qb = logical % a.q_blocks;
  const uint32_t kv_head = head / a.kv_group;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int n = lane & 31;
  const int half = lane >> 5;
  const uint32_t tiles32 = (a.q_tokens + 31) / 32;
  const uint32_t q_tile = qb * kWaves + wave;
  const uint32_t q_tile_c = q_tile < tiles32 ? q_tile : tiles32 - 1;
  const uint32_t q = q_tile_c * kQueriesPerWave + n;
  const uint32_t q_read = q < a.q_tokens ? q : a.q_tokens - 1;

  const Stager sg = make_stager<kMode>(a, wave, lane);
  const uint32_t n_tiles = (a.tokens + kKeys - 1) / kKeys;

  float ks0 = stage_k<kMode>(a, sg, kv_head, 0, k0s);
  const bool m0 = key_live(a, sg, 0);
  float ks1 = stage_k<kMode>(a, sg, kv_head, kKeys, k1s);
  const bool m1 = key_live(a, sg, kKeys);
  float ks_held = stage_k<kMode>(a, sg, kv_head, 2 * kKeys, k2s);
  bool m_held = key_live(a, sg, 2 * kKeys);
  stage_v(a, sg, kv_head, 0, v0s);
  stage_v(a, sg, kv_head, kKeys, v1s);

  v4i qop[4];
  {
    const int32_t* src = a.qi + ((size_t)head * a.q_capacity + q_read) * 32;
#pragma unroll
    for (int dc = 0; dc < 4; ++dc) qop[dc] = *reinterpret_cast<const v4i*>(src + 8 * dc + 4 * half);
  }
  const float qsl = a.qs[(size_t)head * a.q_capacity + q_read] * kLog2e;

  State st;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) st.acc[db][r] = 0.0f;
  st.m = -1.0e30f;
  st.l = 0.0f;
  st.alpha = 1.0f;

  store_scales_mask(k0s, sg, ks0, m0);
  store_scales_mask(k1s, sg, ks1, m1);
  step_barrier<kWaitAll>();
  float u[2][16];
  first_tile<kMode, false>(k0s, qop, qsl, st, u, n, half, a.tokens);
  step_barrier<kWaitAll>();

#define H3_CROSS_STEP(kc, kn, kn2, vc, vn2)                                                   \
  {                                                                                          \
    const float ks_new = stage_k<kMode>(a, sg, kv_head, (j + 3) * kKeys, kc);                \
    const bool m_new = key_live(a, sg, (j + 3) * kKeys);                                     \
    stage_v(a, sg, kv_head, (j + 2) * kKeys, vn2);                                           \
    step<kMode, true, false, false>(kn, vc, qop, qsl, st, u, n, half, 0, a.tokens);          \
    store_scales_mask(kn2, sg, ks_held, m_held);                                             \
    ks_held = ks_new;                                                                        \
    m_held = m_new;                                                                          \
    step_barrier<kWaitPrevStep>();                                                           \
    ++j;                                                                                     \
  }
  const uint32_t steady = n_tiles - 1;
  uint32_t j = 0;
  for (; j + 3 <= steady;) {
    H3_CROSS_STEP(k0s, k1s, k2s, v0s, v2s)
    H3_CROSS_STEP(k1s, k2s, k0s, v1s, v0s)
    H3_CROSS_STEP(k2s, k0s, k1s, v2s, v1s)
  }
  if (j < steady) H3_CROSS_STEP(k0s, k1s, k2s, v0s, v2s)
  if (j < steady) H3_CROSS_STEP(k1s, k2s, k0s, v1s, v0s)
#undef H3_CROSS_STEP
  {
    const uint32_t r = j % 3;
    const char* vlast = r == 0 ? v0s : r == 1 ? v1s : v2s;
    step<kMode, false, false, false>(nullptr, vlast, qop, qsl, st, u, n, half, 0, a.tokens);
  }
  step_barrier<kWaitAll>();

  const float l_tot = st.l + __shfl_xor(st.l, 32);
  const float inv = 1.0f / l_tot;
  if (q_tile < tiles32 && q < a.q_tokens) {
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

// CUs of the current device (cached per device).
uint32_t device_cus() {
  static std::atomic<int> cus[64] = {};  // per device, once known (host threads may race to fill)
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      return 256;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return (uint32_t)n;
}

hipError_t launch_attention(const h3_attention_cfg& cfg, int mode, float skip_tau,
                            uint32_t token_count,
                            uint32_t heads, const int32_t* qi, const float* qs, const int32_t* ki,
                            const float* ks, const uint16_t* vt, uint16_t* out, void* workspace,
                            hipStream_t stream) {
  if (mode == kHeadI8)
    return launch_attention_hm(cfg, token_count, heads, qi, qs, ki, ks, vt, out, stream);
  Args a{};
  a.qi = qi;
  a.qs = qs;
  a.ki = ki;
  a.ks = ks;
  a.vt = vt;
  a.out = out;
  a.tokens = cfg.tokens;
  a.token_count = token_count;
  a.capacity = cfg.token_capacity;
  a.q_row = isI4(mode) ? cfg.q_stride / 2 : cfg.q_stride;
  a.kv_bytes = isI4(mode) ? cfg.kv_stride / 2 : cfg.kv_stride;
  a.neg_tau = -skip_tau * kLog2e;
  a.out_stride = cfg.out_stride;
  a.q_blocks = (token_count + kQueriesPerBlock - 1) / kQueriesPerBlock;
  a.heads = heads;
  a.kv_head_limit = cfg.kv_stride / 128;
  a.head_limit = cfg.out_stride / 128;
  a.q_scale_pitch = cfg.q_stride / 128;
  const bool hm_scales = workspace != nullptr;
  if (hm_scales) {  // token-major codes, head-major copy of the key scales
    float* ks_hm = static_cast<float*>(workspace);
    hipLaunchKernelGGL(k_scales_head_major, dim3((a.tokens + 63) / 64, (a.kv_head_limit + 63) / 64),
                       dim3(256), 0, stream, ks, ks_hm, a.tokens, a.kv_head_limit);
    a.ks = ks_hm;
  }
  // INT8 token-major operands run on the head-major kernel, which reads the token-major rows and
  // scales through its row strides (eight waves share every staged K/V^T tile there).
  if (mode == kTokenI8)
    return launch_attention_hm_tm(cfg, token_count, heads, qi, qs, ki, a.ks, hm_scales, vt, out,
                                  stream);
  // One launch per eight generations of resident workgroups (two per CU), so the workgroups of
  // a launch start together and stay closer in the key stream, whose K rows and scales they
  // share in L2 with fewer heads' neighbours (measured at C3: -5.5 % int4, -2.7 % int4 with
  // head-major scales).
  const uint32_t items = a.q_blocks * heads;
  const uint32_t gen = std::max(1u, 16u * device_cus());
  for (uint32_t base = 0; base < items; base += gen) {
    a.base = base;
    a.total = std::min(gen, items - base);
    a.per_xcd = (a.total + 7) / 8;
    const dim3 grid(a.per_xcd * 8);
    if (mode == kTokenI4) {
      if (hm_scales)
        hipLaunchKernelGGL((k_attention<kTokenI4, true>), grid, dim3(kThreads), 0, stream, a);
      else
        hipLaunchKernelGGL(k_attention<kTokenI4>, grid, dim3(kThreads), 0, stream, a);
    } else if (mode == kTokenI4Skip) {
      if (hm_scales)
        hipLaunchKernelGGL((k_attention<kTokenI4Skip, true>), grid, dim3(kThreads), 0, stream, a);
      else
        hipLaunchKernelGGL(k_attention<kTokenI4Skip>, grid, dim3(kThreads), 0, stream, a);
    }
  }
  return hipGetLastError();
}

hipError_t launch_attention_cross(const h3_cross_cfg& cfg, const int32_t* qi, const float* qs,
                                  const int32_t* ki, const float* ks, const uint16_t* vt,
                                  const uint8_t* key_mask, uint16_t* out, hipStream_t stream) {
  // Groups that divide a workgroup's eight waves run on the head-major kernel, whose workgroups
  // hold every query head of one key/value head over the same staged K/V^T tiles.
  const uint32_t group = cfg.q_heads / cfg.kv_heads;
  if (8 % group == 0)
    return launch_attention_hm_cross(cfg, qi, qs, ki, ks, vt, key_mask, out, stream);
  Args a{};
  a.qi = qi;
  a.qs = qs;
  a.ki = ki;
  a.ks = ks;
  a.vt = vt;
  a.out = out;
  a.key_mask = key_mask;
  a.tokens = cfg.kv_tokens;
  a.capacity = cfg.kv_capacity;
  a.q_tokens = cfg.q_tokens;
  a.q_capacity = cfg.q_capacity;
  a.token_count = cfg.q_tokens;
  a.kv_group = cfg.q_heads / cfg.kv_heads;
  a.out_stride = cfg.out_stride;
  a.q_blocks = (cfg.q_tokens + kQueriesPerBlock - 1) / kQueriesPerBlock;
  a.heads = cfg.q_heads;
  a.kv_head_limit = cfg.kv_heads;
  a.head_limit = cfg.q_heads;
  a.q_scale_pitch = cfg.q_heads;
  a.total = a.q_blocks * cfg.q_heads;
  a.per_xcd = (a.total + 7) / 8;
  hipLaunchKernelGGL(k_attention_cross, dim3(a.per_xcd * 8), dim3(kThreads), 0, stream, a);
  return hipGetLastError();
}

size_t scales_workspace_bytes(const h3_attention_cfg& cfg) {
  return (size_t)(cfg.kv_stride / 128) * cfg.tokens * 4;
}

hipError_t launch_attention_vsa(const h3_attention_cfg& cfg, uint32_t token_count,
                                uint32_t heads, const int32_t* qi, const float* qs,
                                const int32_t* ki, const float* ks, const uint16_t* vt,
                                uint16_t* out, const int32_t* routes, const int32_t* lengths,
                                void* workspace, hipStream_t stream) {
  Args a{};
  a.qi = qi;
  a.qs = qs;
  a.ki = ki;
  a.ks = ks;
  a.vt = vt;
  a.out = out;
  a.tokens = cfg.tokens;
  a.token_count = token_count;
  a.capacity = cfg.token_capacity;
  a.q_row = cfg.q_stride;
  a.kv_bytes = cfg.kv_stride;
  a.out_stride = cfg.out_stride;
  a.q_blocks = (token_count + 63) / 64;  // one query cube per workgroup
  a.heads = heads;
  a.kv_head_limit = cfg.kv_stride / 128;
  a.head_limit = cfg.out_stride / 128;
  a.q_scale_pitch = cfg.q_stride / 128;
  a.routes = routes;
  a.lengths = lengths;
  a.blocks = cfg.tokens / 64;
  if (workspace) {  // head-major key scales for the kernel
    float* ks_hm = static_cast<float*>(workspace);
    hipLaunchKernelGGL(k_scales_head_major, dim3((a.tokens + 63) / 64, (a.kv_head_limit + 63) / 64),
                       dim3(256), 0, stream, ks, ks_hm, a.tokens, a.kv_head_limit);
    a.ks = ks_hm;
  }
  // One launch per generation of resident workgroups (four per CU): its workgroups start
  // together and walk their ascending key lists at about the same pace, so more of the tiles
  // they share are still in L2 (measured at 129k tokens with token-major scales: 45.9 ms against
  // 56.5 ms for one launch of all the work).
  const uint32_t items = a.q_blocks * heads;
  const uint32_t gen = std::max(1u, 4u * device_cus());
  for (uint32_t base = 0; base < items; base += gen) {
    a.base = base;
    a.total = std::min(gen, items - base);
    a.per_xcd = (a.total + 7) / 8;
    if (workspace)
      hipLaunchKernelGGL(k_attention_vsa<true>, dim3(a.per_xcd * 8), dim3(kVsaThreads), 0, stream, a);
    else
      hipLaunchKernelGGL(k_attention_vsa<false>, dim3(a.per_xcd * 8), dim3(kVsaThreads), 0, stream, a);
  }
  return hipGetLastError();
}

hipError_t launch_attention_vsa_f16(const h3_attention_cfg& cfg, uint32_t token_count,
                                    uint32_t heads, const uint16_t* q, const uint16_t* k,
                                    const uint16_t* v, uint16_t* out, const int32_t* routes,
                                    const int32_t* lengths, hipStream_t stream) {
  Args a{};
  a.qi = reinterpret_cast<const int32_t*>(q);
  a.ki = reinterpret_cast<const int32_t*>(k);
  a.vt = v;
  a.out = out;
  a.tokens = cfg.tokens;
  a.token_count = token_count;
  a.capacity = cfg.token_capacity;
  a.q_row = cfg.q_stride * 2;
  a.kv_bytes = cfg.kv_stride * 2;
  a.out_stride = cfg.out_stride;
  a.q_blocks = (token_count + 63) / 64;
  a.heads = heads;
  a.kv_head_limit = cfg.kv_stride / 128;
  a.head_limit = cfg.out_stride / 128;
  a.q_scale_pitch = cfg.q_stride / 128;
  a.routes = routes;
  a.lengths = lengths;
  a.blocks = cfg.tokens / 64;
  a.scale = cfg.scale;
  // Generations of resident workgroups as in launch_attention_vsa (four per CU).
  const uint32_t items = a.q_blocks * heads;
  const uint32_t gen = std::max(1u, 4u * device_cus());
  for (uint32_t base = 0; base < items; base += gen) {
    a.base = base;
    a.total = std::min(gen, items - base);
    a.per_xcd = (a.total + 7) / 8;
    hipLaunchKernelGGL((k_attention_vsa<false, true>), dim3(a.per_xcd * 8), dim3(kVsaThreads), 0,
                       stream, a);
  }
  return hipGetLastError();
}

}  // namespace h3
