// Head-major INT8-QK flash attention for gfx950 (CDNA4): attention_i8qkhm_mha8_k64_lds_f16_wmma
// (kernels/attention_i8qkhm_mha8_k64_lds_f16_wmma.loom:437-1067): non-causal MHA over head-major
// operands, keys >= tokens masked, rows >= token_count not written, f16 output
// [token_count][out_stride].
//
// Shape of the work. One wave per SIMD (four per workgroup, one workgroup per CU), each wave
// owning two tiles of 32 queries (A and B) of one head; 64-key K / V^T tiles stream through LDS
// and are consumed in two sub-steps of 32 keys. Sub-step t issues, for both query tiles, QK of
// key tile t+2 and PV of key tile t on the matrix cores, while the vector ALU turns the scores of
// key tile t+1 into probabilities: every MFMA has independent vector work beside it, no second
// wave is needed to hide the softmax, and each K, V^T and key-scale read from LDS feeds both
// query tiles. Per 32 keys and query tile:
//   QK   S^T (32 keys x 32 queries) = K . Q^T on v_mfma_i32_32x32x32_i8, exact int32; lane l owns
//        query l%32, accumulator register r holds MFMA row 8(r/4) + 4(l/32) + r%4 of the key
//        block. LDS row m of a K tile holds key swap23(m) (bits 2 and 3 exchanged), so registers
//        8g..8g+7 are keys 16g + 8(l/32) + 0..7 of the block: the B operand of a 16-key f16 MFMA
//        step with V^T in natural key order, and P never leaves its registers.
//   dequant  accumulators start from the bit pattern of 1.5*2^23, so each ends as the float
//        1.5*2^23 + S exactly and one FMA gives u = S*ks: u = acc*ks + c with c = -1.5*2^23*ks
//        staged per key, or c = -inf for a key past the sequence (masking costs nothing).
//   softmax  base 2 on y = u*qs*log2e - m with no per-tile max: the running max m is kept from
//        earlier tiles and a tile whose probabilities could exceed 2^8 is caught by its row sum
//        (every p >= 0, so the sum of a lane's 16 probabilities bounds each of them; f16
//        overflow shows as inf). Such a tile takes the exact path: its max is computed, m is
//        raised, the output accumulators and the sum are rescaled and its probabilities
//        recomputed. The first key tile of each query tile always takes it (m starts at -1e30).
//   PV   O^T (128 ch x 32 queries) += V^T . P^T on v_mfma_f32_32x32x16_f16, f32 accumulators;
//        the row sum is a packed f16 add tree of the same probabilities per tile, added in f32.
// S^T and P are double-buffered by key-tile parity, so every dependence between the matrix and
// the vector work is a whole sub-step long.
//
// Staging: K, V^T and key-scale tiles go through three-stage rings. K and V^T go from HBM into
// LDS with buffer_load ... lds (no registers, no LDS store instructions); the key scale takes a
// register (one load per lane for 16 lanes of each wave), stored with its c a step later. Step j
// (64 keys, two sub-steps) reads K(j+1), V(j) and the scales of tiles j and j+1, and issues
// K(j+3), V(j+2) and the scale load of tile j+3, so every load has two steps to land; before the
// step's barrier a wave waits only for its own loads of the step before. LDS rows are 128 bytes
// with their 16-byte chunks XOR-swizzled by (row/2)%8, so the 32 rows a half-wave reads fall on
// distinct banks. Buffer descriptors end at the last valid key, so keys past the sequence read
// as zero.
// Workgroups are remapped so each XCD runs a contiguous range of (head, query block) work and its
// resident workgroups stream the same head's K/V^T through their shared L2.
#include <algorithm>
#include <type_traits>
#include <utility>

#include "internal.hpp"

namespace h3 {
namespace {

constexpr int kWaves = 4;                         // one per SIMD
constexpr int kThreads = 64 * kWaves;
constexpr int kTileQ = 32;                        // queries per tile, two tiles per wave
constexpr int kBlockQ = kWaves * 2 * kTileQ;      // 256 queries per workgroup
constexpr int kKeys = 64;                         // keys per LDS tile
constexpr int kRowBytes = 128;
constexpr int kKStage = kKeys * kRowBytes;        // 8192: int8 codes of 64 keys
constexpr int kVStage = 128 * kRowBytes;          // 16384: 128 channels x 64 keys of f16
constexpr int kSStage = 2 * kKeys * 4;            // 512: ks[64], c[64] at MFMA-row index
constexpr int kKLoads = kKStage / 1024 / kWaves;  // 1 KiB LDS-DMA loads per wave per tile: 2
constexpr int kVLoads = kVStage / 1024 / kWaves;  // 4
constexpr int kSRows = kKeys / kWaves;            // scale rows stored per wave: 16
// s_waitcnt fields (gfx9 layout): vmcnt <= the loads one step issues (K, V^T, scale), expcnt
// untouched, lgkmcnt 0; or vmcnt 0.
constexpr int kStages = 4;                        // ring depth of K, V^T and scale tiles
constexpr int kLoadsPerStep = kKLoads + kVLoads + 1;
constexpr int kWaitPrevStep = kLoadsPerStep | (7 << 4) | (0 << 8);
constexpr int kWaitTwoSteps = (2 * kLoadsPerStep) | (7 << 4) | (0 << 8);
constexpr int kWaitAll = 0 | (7 << 4) | (0 << 8);
constexpr int kPf = 4;                            // LDS operands read this many ahead (of 12)
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kMagicBits = 0x4B400000;            // float 12582912 = 1.5 * 2^23
constexpr float kMagic = 12582912.0f;
constexpr float kSumLimit = 256.0f;               // a lane's tile sum above this: exact path
constexpr int kRsrcWord3 = 0x00020000;            // gfx9 raw buffer: 32-bit data, no swizzle

typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ uint32_t swap23(uint32_t m) {
  return (m & ~12u) | ((m & 4u) << 1) | ((m & 8u) >> 1);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           kRsrcWord3);
}

struct Geometry {
  const int32_t* qi;
  const float* qs;
  const int32_t* ki;
  const float* ks;
  const uint16_t* vt;
  uint16_t* out;
  uint32_t tokens;       // keys (and readable query rows)
  uint32_t rows;         // query rows written: min(token_count, tokens)
  uint32_t capacity;
  uint32_t out_stride;
  uint32_t q_blocks;     // ceil(token_count / 256)
  uint32_t kv_head_limit;
  uint32_t head_limit;
  uint32_t total;        // q_blocks * heads
  uint32_t per_xcd;      // ceil(total / 8)
};

// Per-lane constants of the staging loads (the wave's share of each tile).
struct Stager {
  uint32_t koff[kKLoads];  // byte offset in the head's K rows of this lane's 16 bytes, per load
  uint32_t voff[kVLoads];  // byte offset in the head's V^T block (from column k0) per load
  uint32_t srow;           // MFMA row whose key scale this lane stores (lanes below kSRows)
  uint32_t skey;           // its key within the tile: swap23(srow)
  int wave;
};

// LDS byte o of a K or V^T stage holds row o/128, logical 16-byte chunk ((o/16)%8) ^ ((row/2)%8);
// K row m holds key swap23(m).
__device__ __forceinline__ Stager make_stager(const Geometry& g, int wave, int lane) {
  Stager s;
  s.wave = wave;
#pragma unroll
  for (int t = 0; t < kKLoads; ++t) {
    const uint32_t o = (wave * kKLoads + t) * 1024 + 16 * lane;
    const uint32_t row = o >> 7, chunk = ((o >> 4) & 7) ^ ((row >> 1) & 7);
    s.koff[t] = swap23(row) * kRowBytes + 16 * chunk;
  }
#pragma unroll
  for (int t = 0; t < kVLoads; ++t) {
    const uint32_t o = (wave * kVLoads + t) * 1024 + 16 * lane;
    const uint32_t row = o >> 7, chunk = ((o >> 4) & 7) ^ ((row >> 1) & 7);
    s.voff[t] = row * g.capacity * 2 + 16 * chunk;
  }
  s.srow = kSRows * wave + (lane & (kSRows - 1));
  s.skey = swap23(s.srow);
  return s;
}

// LDS-DMA of K tile k0 into `kst` (rows past the sequence load as zero) and the load of this
// lane's key scale into a register.
__device__ __forceinline__ float stage_k(const Geometry& g, const Stager& sg, uint32_t kv_head,
                                         uint32_t k0, char* kst) {
  const uint32_t live = g.tokens > k0 ? min(g.tokens - k0, (uint32_t)kKeys) : 0u;
  const float* sbase = g.ks + (size_t)kv_head * g.capacity + k0;
  const float ks = __builtin_bit_cast(
      float, __builtin_amdgcn_raw_buffer_load_b32(rsrc(sbase, live * 4), sg.skey * 4, 0, 0));
  const char* base = reinterpret_cast<const char*>(g.ki) + ((size_t)kv_head * g.capacity + k0) * 128;
  const __amdgpu_buffer_rsrc_t rk = rsrc(base, live * 128);
#pragma unroll
  for (int t = 0; t < kKLoads; ++t)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rk, (lds_void*)(kst + (sg.wave * kKLoads + t) * 1024), 16, sg.koff[t], 0, 0, 0);
  return ks;
}

// LDS-DMA of V^T tile k0 into `vst`. The range ends at the end of this head's V^T block; columns
// past `tokens` inside it are zero or belong to the next channel row, and meet probability 0.
__device__ __forceinline__ void stage_v(const Geometry& g, const Stager& sg, uint32_t kv_head,
                                        uint32_t k0, char* vst) {
  const uint32_t blk = 128 * g.capacity;
  const char* base = reinterpret_cast<const char*>(g.vt) + ((size_t)kv_head * blk + k0) * 2;
  const __amdgpu_buffer_rsrc_t rv = rsrc(base, k0 < blk ? (blk - k0) * 2 : 0u);
#pragma unroll
  for (int t = 0; t < kVLoads; ++t)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rv, (lds_void*)(vst + (sg.wave * kVLoads + t) * 1024), 16, sg.voff[t], 0, 0, 0);
}

// Scales of K tile k0 at their MFMA rows: ks, and c = -1.5*2^23*ks for a key inside the
// sequence or -inf for one past it.
__device__ __forceinline__ void store_scales(char* sst, const Stager& sg, float ks, uint32_t k0,
                                             uint32_t tokens) {
  if ((threadIdx.x & 63) < kSRows) {
    float* sc = reinterpret_cast<float*>(sst);
    sc[sg.srow] = ks;
    sc[kKeys + sg.srow] = k0 + sg.skey < tokens ? -(kMagic * ks) : -INFINITY;
  }
}

// Barrier between steps: this wave's LDS writes, and its staging loads from before the current
// step, are complete; the loads issued in this step stay in flight.
template <int kWait>
__device__ __forceinline__ void step_barrier() {
  __builtin_amdgcn_s_waitcnt(kWait);
  asm volatile("s_barrier" ::: "memory");
}

// One 32-query tile of a wave (its O^T accumulators live in fixed AGPRs, see below). S^T and P
// are double-buffered by the parity of the 32-key tile they belong to.
struct Tile {
  v16i s[2];    // S^T of the 32-key tiles of each parity
  v8h p[2][2];  // probabilities of the 32-key tiles of each parity, packed f16 (16 keys each)
  v4i q[4];     // Q^T operand: 4 chunks of 32 channels
  float qsl;    // qs * log2(e)
  float negm;   // minus the running max (log2 units)
  float l;      // this lane's share of the row sum
};

// Issue-order fence: the scheduler keeps each chunk's MFMA, LDS reads and vector work together.
#define H3_CHUNK_END() __builtin_amdgcn_sched_barrier(0)

__device__ __forceinline__ uint32_t chunk_off(int x, int half, uint32_t sw) {
  return 16 * ((2 * x + half) ^ sw);
}

// The MFMAs are written as inline assembly, and the output accumulators O^T of the two tiles
// live in fixed AGPRs: tile t's block db (32 channels x 32 queries, f32) in a[64t + 16db ..
// +15], a0-a127 in all. With one wave per SIMD the compiler would give builtin MFMAs the AGPR
// form, so S^T would need a v_accvgpr_read per score, and it copies AGPR accumulators between
// register sets wherever a conditional rescale rejoins the fast path. Here S^T lives in VGPRs,
// O^T never moves, and the compiler keeps no value of its own in a0-a127 (every asm that touches
// them names them as clobbered; nothing else of the kernel uses AGPRs). Hazards are covered by
// the schedule: an accumulator chain is the same opcode on exactly the same registers, which the
// hardware forwards with no wait states; the vector ALU reads S^T only in the next half step
// (more than a hundred instructions later) or after explicit waits (half steps without PV),
// writes P a half step before PV reads it, and touches O^T only in the exact path and the
// epilogue, both behind explicit waits.
#define H3_A16(b) "a" #b "0", "a" #b "1", "a" #b "2", "a" #b "3", "a" #b "4", "a" #b "5", "a" #b "6", \
                  "a" #b "7", "a" #b "8", "a" #b "9"
#define H3_O_CLOBBERS                                                                          \
  "a0", "a1", "a2", "a3", "a4", "a5", "a6", "a7", "a8", "a9", H3_A16(1), H3_A16(2), H3_A16(3),  \
      H3_A16(4), H3_A16(5), H3_A16(6), H3_A16(7), H3_A16(8), H3_A16(9), H3_A16(10), H3_A16(11), \
      H3_A16(12), "a120", "a121", "a122", "a123", "a124", "a125", "a126", "a127"

__device__ __forceinline__ v16i qk_first(v4i k, v4i q, const v16i& magic) {
  v16i d;
  asm volatile("v_mfma_i32_32x32x32_i8 %0, %1, %2, %3" : "=&v"(d) : "v"(k), "a"(q), "v"(magic));
  return d;
}
__device__ __forceinline__ void qk_next(v16i& d, v4i k, v4i q) {
  asm volatile("v_mfma_i32_32x32x32_i8 %0, %1, %2, %0" : "+v"(d) : "v"(k), "a"(q));
}
// O^T block (tile, db) += V^T . P^T
template <int kBase>
__device__ __forceinline__ void pv_block(v8h v, v8h p) {
  asm volatile("v_mfma_f32_32x32x16_f16 a[%2:%3], %0, %1, a[%2:%3]"
               :: "v"(v), "v"(p), "n"(kBase), "n"(kBase + 15) : H3_O_CLOBBERS);
}
template <int kTile>
__device__ __forceinline__ void pv_mfma(int db, v8h v, v8h p) {
  switch (db) {  // db is a constant once the chunk loop is unrolled
    case 0: pv_block<64 * kTile + 0>(v, p); break;
    case 1: pv_block<64 * kTile + 16>(v, p); break;
    case 2: pv_block<64 * kTile + 32>(v, p); break;
    default: pv_block<64 * kTile + 48>(v, p); break;
  }
}
// Accumulator register kReg *= alpha, and its read for the epilogue.
template <int kReg>
__device__ __forceinline__ void scale_acc(float alpha) {
  float t;
  asm volatile("v_accvgpr_read_b32 %0, a[%2]\n\tv_mul_f32 %0, %0, %1\n\tv_accvgpr_write_b32 a[%2], %0"
               : "=&v"(t) : "v"(alpha), "n"(kReg) : H3_O_CLOBBERS);
}
template <int kReg>
__device__ __forceinline__ float read_acc() {
  float t;
  asm volatile("v_accvgpr_read_b32 %0, a[%1]" : "=v"(t) : "n"(kReg));
  return t;
}
template <int kTile, int... kR>
__device__ __forceinline__ void scale_tile(float alpha, std::integer_sequence<int, kR...>) {
  (scale_acc<64 * kTile + kR>(alpha), ...);
}
template <int kTile, int... kR>
__device__ __forceinline__ void read_tile(float (&o)[64], std::integer_sequence<int, kR...>) {
  ((o[kR] = read_acc<64 * kTile + kR>()), ...);
}
template <int kReg>
__device__ __forceinline__ void zero_acc() {
  asm volatile("v_accvgpr_write_b32 a[%0], 0" :: "n"(kReg) : H3_O_CLOBBERS);
}
template <int... kR>
__device__ __forceinline__ void zero_accumulators(std::integer_sequence<int, kR...>) {
  (zero_acc<kR>(), ...);
}

__device__ __forceinline__ float half_swap_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// A lane's sum of a tile's 32 packed probabilities: a packed f16 add tree and one dot2 into f32.
__device__ __forceinline__ float fold_sum(v8h t8) {
  const v4h t4 = v4h{t8[0], t8[1], t8[2], t8[3]} + v4h{t8[4], t8[5], t8[6], t8[7]};
  const v2h t2 = v2h{t4[0], t4[1]} + v2h{t4[2], t4[3]};
  return __builtin_amdgcn_fdot2(t2, v2h{(_Float16)1.0f, (_Float16)1.0f}, 0.0f, false);
}

// Scales of quarter i (slots 4i..4i+3) of key block b: ks at kss[32b + 8i + 4h .. +3] for lane
// half h, c 64 floats further.
__device__ __forceinline__ float4 scale4(const float* kss, int b, int i, int half) {
  return *reinterpret_cast<const float4*>(kss + 32 * b + 8 * i + 4 * half);
}

// Dequantized scores of quarter i of a tile's S^T: u = acc*ks + c.
__device__ __forceinline__ void dequant_quarter(const v16i& s, int i, float4 k4, float4 c4,
                                                float (&u)[4]) {
  const float kv[4] = {k4.x, k4.y, k4.z, k4.w}, cv[4] = {c4.x, c4.y, c4.z, c4.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    u[j] = __builtin_fmaf(__int_as_float(s[4 * i + j]), kv[j], cv[j]);
    asm volatile("" : "+v"(u[j]));  // keeps the work in this chunk (no sinking or hoisting)
  }
}

// Exponent arguments y = u*qsl - m of a quarter, computed in f32 and rounded once to f16 into the
// low and high halves of two words (v_fma_mixlo/mixhi_f16). Then p = 2^y in place with the f16
// exponential on each half (SDWA, the other half preserved): the probabilities come out packed
// as PV's B operand with no separate conversion. Each exponential's result is read two
// instructions later at the earliest, and the trailing nop covers the first read after the block.
__device__ __forceinline__ void exparg_quarter(const float (&u)[4], float qsl, float negm,
                                               uint32_t (&w)[2]) {
  asm volatile("v_fma_mixlo_f16 %0, %2, %6, %7\n\t"
               "v_fma_mixlo_f16 %1, %4, %6, %7\n\t"
               "v_fma_mixhi_f16 %0, %3, %6, %7\n\t"
               "v_fma_mixhi_f16 %1, %5, %6, %7"
               : "=&v"(w[0]), "=&v"(w[1])
               : "v"(u[0]), "v"(u[1]), "v"(u[2]), "v"(u[3]), "v"(qsl), "v"(negm));
}
__device__ __forceinline__ void exp2_quarter(uint32_t (&w)[2]) {
  asm volatile("v_exp_f16_sdwa %0, %0 dst_sel:WORD_0 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0\n\t"
               "v_exp_f16_sdwa %1, %1 dst_sel:WORD_0 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0\n\t"
               "v_exp_f16_sdwa %0, %0 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_1\n\t"
               "v_exp_f16_sdwa %1, %1 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_1\n\t"
               "s_nop 0"
               : "+v"(w[0]), "+v"(w[1]));
}
// The words of quarter i go to group i/2 (16 keys), elements 4(i%2)..+3.
__device__ __forceinline__ void put_quarter(v8h (&p)[2], int i, const uint32_t (&w)[2]) {
  const v2h a = __builtin_bit_cast(v2h, w[0]), b = __builtin_bit_cast(v2h, w[1]);
  const int g = i >> 1, e = 4 * (i & 1);
  p[g][e + 0] = a[0];
  p[g][e + 1] = a[1];
  p[g][e + 2] = b[0];
  p[g][e + 3] = b[1];
}

// The exact path for a tile whose probabilities of key tile `par` (computed against the running
// max) may exceed 2^8: take the tile's max, raise m, rescale the accumulators and the row sum,
// recompute the probabilities. `kss` and `b` locate the key tile's scales.
template <int kTile>
__device__ __forceinline__ void raise_exact(Tile& T, int par, const float* kss, int b, int half) {
  float u[16];
  float tmax = -INFINITY;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float4 k4 = scale4(kss, b, i, half), c4 = scale4(kss + kKeys, b, i, half);
    const float kv[4] = {k4.x, k4.y, k4.z, k4.w}, cv[4] = {c4.x, c4.y, c4.z, c4.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      u[4 * i + j] = __builtin_fmaf(__int_as_float(T.s[par][4 * i + j]), kv[j], cv[j]);
      tmax = fmaxf(tmax, u[4 * i + j]);
    }
  }
  tmax = half_swap_max(tmax);
  const float m_old = -T.negm;
  const float m_new = fmaxf(m_old, tmax * T.qsl);
  const float alpha = __builtin_amdgcn_exp2f(m_old - m_new);
  // The tile's PV MFMAs of this sub-step were issued before; the waits on both sides of the
  // rescale cover them and the next MFMA that reads the accumulators.
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  scale_tile<kTile>(alpha, std::make_integer_sequence<int, 64>{});
  asm volatile("s_nop 7\n\ts_nop 7" ::: "memory");
  T.negm = -m_new;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float uq[4] = {u[4 * i], u[4 * i + 1], u[4 * i + 2], u[4 * i + 3]};
    uint32_t w[2];
    exparg_quarter(uq, T.qsl, T.negm, w);
    exp2_quarter(w);
    put_quarter(T.p[par], i, w);
  }
  T.l = T.l * alpha + fold_sum(T.p[par][0] + T.p[par][1]);
  asm volatile("s_nop 7" ::: "memory");  // fresh P before the next MFMA reads it
}

// The overflow check of both tiles' fresh probabilities (key tile parity `par`; `ta`, `tb` their
// lane sums), then their row sums. One wave-uniform branch for both, so that no work of either
// is moved behind it.
__device__ __forceinline__ void check_tiles(Tile& A, Tile& B, float ta, float tb, int par,
                                            const float* kss, int b, int half) {
  const bool oa = !(ta <= kSumLimit), ob = !(tb <= kSumLimit);
  if (__builtin_expect(__any(oa || ob), 0)) {
    if (__any(oa))
      raise_exact<0>(A, par, kss, b, half);
    else
      A.l += ta;
    if (__any(ob))
      raise_exact<1>(B, par, kss, b, half);
    else
      B.l += tb;
  } else {
    A.l += ta;
    B.l += tb;
  }
}

// Packed f16 partial sum of a 16-key group (4 words) of probabilities.
__device__ __forceinline__ v2h group_sum(const v8h& g) {
  const v4h t4 = v4h{g[0], g[1], g[2], g[3]} + v4h{g[4], g[5], g[6], g[7]};
  return v2h{t4[0], t4[1]} + v2h{t4[2], t4[3]};
}

// Sub-step t (kPar = t % 2) for both query tiles, in 24 chunks of one MFMA each:
//   kQK  QK of key tile t+2 (block kPar of K stage `kst`) into S^T[kPar]
//   kPV  PV of key tile t (block kPar of V^T stage `vst`) from P[kPar]
//   kSM  probabilities of key tile t+1 (block `sb` of scale stage `sst`) from S^T[1-kPar] into
//        P[1-kPar], then the overflow checks.
// The 12 LDS operands (4 K chunks, then 8 V^T chunks, each feeding an MFMA of A then one of B) are
// read kPf operands ahead. QK comes first, so the S^T it writes is read by the vector ALU only in
// the next sub-step, after this one's 16 PV MFMAs. The softmax runs as 8 units (quarter, tile)
// in the order A0 A1 B0 B1 A2 A3 B2 B3, three chunks each (dequantisation, exponent arguments,
// exponentials), so each quarter's scales (read two quarters ahead) serve both tiles while in
// registers and a 16-key group's partial row sum is taken as soon as its two quarters are done.
template <int kPar, bool kQK, bool kPV, bool kSM>
__device__ __forceinline__ void sub_step(const char* kst, const char* vst, const char* sst, int sb,
                                         Tile& A, Tile& B, int n, int half, const v16i& magic) {
  constexpr int kSm = 1 - kPar;  // parity of the tile whose probabilities are computed
  const uint32_t sw = (n >> 1) & 7;
  const float* kss = reinterpret_cast<const float*>(sst);
  v4i kop[4];
  v8h vop[8];
  float4 k4[4], c4[4];
  float u[4];
  uint32_t w[2];
  v2h gs[2][2];  // partial row sums of the groups of A and B
  constexpr int kIsK[12] = {1, 1, 1, 1, 0, 0, 0, 0, 0, 0, 0, 0};
  constexpr int kIdx[12] = {0, 1, 2, 3, 0, 1, 2, 3, 4, 5, 6, 7};
  // unit u: quarter kUnitQ[u] of tile kUnitT[u]
  constexpr int kUnitQ[8] = {0, 1, 0, 1, 2, 3, 2, 3};
  constexpr int kUnitT[8] = {0, 0, 1, 1, 0, 0, 1, 1};
  auto read_op = [&](int o) {
    if (kIsK[o]) {
      if (kQK)
        kop[kIdx[o]] = *reinterpret_cast<const v4i*>(kst + (32 * kPar + n) * kRowBytes +
                                                     chunk_off(kIdx[o], half, sw));
    } else if (kPV) {
      // V^T chunk v: channel block db = v % 4, key group 2*kPar + v / 4 of the stage
      const int v = kIdx[o], db = v & 3, g = 2 * kPar + (v >> 2);
      vop[v] = *reinterpret_cast<const v8h*>(vst + (32 * db + n) * kRowBytes +
                                             chunk_off(g, half, sw));
    }
  };
  auto read_scales = [&](int i) {
    k4[i] = scale4(kss, sb, i, half);
    c4[i] = scale4(kss + kKeys, sb, i, half);
  };
#pragma unroll
  for (int o = 0; o < kPf; ++o) read_op(o);
  if (kSM) {
    read_scales(0);
    read_scales(1);
  }
#pragma unroll
  for (int c = 0; c < 24; ++c) {
    const int o = c >> 1;        // operand of this chunk's MFMA
    Tile& X = (c & 1) ? B : A;   // the query tile it is for
    if ((c & 1) && o + kPf < 12) read_op(o + kPf);
    if (kIsK[o]) {
      if (kQK) {
        const int dc = kIdx[o];
        if (dc == 0)
          X.s[kPar] = qk_first(kop[dc], X.q[dc], magic);
        else
          qk_next(X.s[kPar], kop[dc], X.q[dc]);
      }
    } else if (kPV) {
      const int v = kIdx[o];
      if (c & 1)
        pv_mfma<1>(v & 3, vop[v], B.p[kPar][v >> 2]);
      else
        pv_mfma<0>(v & 3, vop[v], A.p[kPar][v >> 2]);
    }
    if (kSM) {
      const int unit = c / 3, phase = c % 3, i = kUnitQ[unit], t = kUnitT[unit];
      Tile& Y = t ? B : A;
      if (phase == 0) {
        if (unit == 1) read_scales(2);
        if (unit == 3) read_scales(3);
        dequant_quarter(Y.s[kSm], i, k4[i], c4[i], u);
      } else if (phase == 1) {
        exparg_quarter(u, Y.qsl, Y.negm, w);
      } else {
        exp2_quarter(w);
        put_quarter(Y.p[kSm], i, w);
        if (i & 1) gs[t][i >> 1] = group_sum(Y.p[kSm][i >> 1]);  // the group is complete
      }
    }
    H3_CHUNK_END();
  }
  if (kQK && !kPV)  // the next sub-step's vector ALU reads this S^T at once: cover the latency
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  if (kSM) {
    const v2h one = {(_Float16)1.0f, (_Float16)1.0f};
    const float ta = __builtin_amdgcn_fdot2(gs[0][0] + gs[0][1], one, 0.0f, false);
    const float tb = __builtin_amdgcn_fdot2(gs[1][0] + gs[1][1], one, 0.0f, false);
    check_tiles(A, B, ta, tb, kSm, kss, sb, half);
  }
}

// Stage `i` of a ring of separately declared arrays (i is a constant after unrolling, so the
// compiler still sees which array every access and LDS-DMA goes to).
__device__ __forceinline__ char* ring(int i, char* a0, char* a1, char* a2, char* a3) {
  return i == 0 ? a0 : i == 1 ? a1 : i == 2 ? a2 : a3;
}

__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void k_attention_hm(Geometry g) {
  // Four-stage rings, each stage its own array so that the compiler can tell an LDS-DMA into one
  // stage from the reads of another.
  __shared__ __attribute__((aligned(16))) char k0s[kKStage], k1s[kKStage], k2s[kKStage], k3s[kKStage];
  __shared__ __attribute__((aligned(16))) char v0s[kVStage], v1s[kVStage], v2s[kVStage], v3s[kVStage];
  __shared__ __attribute__((aligned(16))) char s0s[kSStage], s1s[kSStage], s2s[kSStage], s3s[kSStage];
  auto kr = [&](int i) { return ring(i & 3, k0s, k1s, k2s, k3s); };
  auto vr = [&](int i) { return ring(i & 3, v0s, v1s, v2s, v3s); };
  auto sr = [&](int i) { return ring(i & 3, s0s, s1s, s2s, s3s); };

  // XCD-aware remap: hardware hands block b to XCD b % 8; give each XCD a contiguous range of
  // (head, query block) work so its resident blocks share one head's K/V^T stream in L2.
  const uint32_t b = blockIdx.x;
  const uint32_t logical = (b & 7u) * g.per_xcd + (b >> 3);
  if (logical >= g.total) return;
  const uint32_t head_y = logical / g.q_blocks;
  const uint32_t qb = logical % g.q_blocks;
  const uint32_t kv_head = head_y % g.kv_head_limit;
  const uint32_t head = kv_head % g.head_limit;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int n = lane & 31;
  const int half = lane >> 5;
  const Stager sg = make_stager(g, wave, lane);
  const uint32_t n_stages = (g.tokens + kKeys - 1) / kKeys;  // 64-key stages; 32-key tiles 2x

  // ---- prologue: K(0..2), V(0..1) and the scales of stages 0..2 in flight
  const float ks0 = stage_k(g, sg, kv_head, 0, k0s);
  const float ks1 = stage_k(g, sg, kv_head, kKeys, k1s);
  const float ks2 = stage_k(g, sg, kv_head, 2 * kKeys, k2s);
  stage_v(g, sg, kv_head, 0, v0s);
  stage_v(g, sg, kv_head, kKeys, v1s);

  // The QK bias 1.5*2^23, made opaque so that it stays in registers for the whole loop.
  v16i magic;
#pragma unroll
  for (int r = 0; r < 16; ++r) magic[r] = kMagicBits;
  asm volatile("" : "+v"(magic));
  Tile A, B;
  const uint32_t q0 = qb * kBlockQ + wave * 2 * kTileQ + n;  // tile A's query; tile B's is +32
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    Tile& T = t == 0 ? A : B;
    const uint32_t q = q0 + t * kTileQ;
    const uint32_t q_read = q < g.tokens ? q : g.tokens - 1;
    const int32_t* src = g.qi + ((size_t)head * g.capacity + q_read) * 32;
#pragma unroll
    for (int dc = 0; dc < 4; ++dc) T.q[dc] = *reinterpret_cast<const v4i*>(src + 8 * dc + 4 * half);
    T.qsl = g.qs[(size_t)head * g.capacity + q_read] * kLog2e;
    T.negm = 1.0e30f;
    T.l = 0.0f;
  }
  zero_accumulators(std::make_integer_sequence<int, 128>{});
  store_scales(s0s, sg, ks0, 0, g.tokens);
  store_scales(s1s, sg, ks1, kKeys, g.tokens);
  step_barrier<kWaitAll>();

  // ---- step -1: QK of key tiles 0 and 1, the probabilities of tile 0
  float ks_held = stage_k(g, sg, kv_head, 3 * kKeys, k3s);
  stage_v(g, sg, kv_head, 2 * kKeys, v2s);
  sub_step<0, true, false, false>(k0s, nullptr, nullptr, 0, A, B, n, half, magic);
  sub_step<1, true, false, true>(k0s, nullptr, s0s, 0, A, B, n, half, magic);
  store_scales(s2s, sg, ks2, 2 * kKeys, g.tokens);
  step_barrier<kWaitPrevStep>();

  // Steady step j (stage j+1 exists), J = j % 4: sub-steps 2j and 2j+1 read K(j+1), V(j) and the
  // scales of tiles 2j+1 (stage j, block 1) and 2j+2 (stage j+1, block 0); the step stages K(j+4)
  // into K(j)'s array, V(j+3) into V(j-1)'s, and stores the scales of stage j+3 (loaded one step
  // earlier) into S(j-1)'s. Every load has three steps to land; a step waits for its own loads of
  // two steps before.
  uint32_t j = 0;
  auto steady = [&](auto J_) {
    constexpr int J = decltype(J_)::value;
    const float ks_new = stage_k(g, sg, kv_head, (j + 4) * kKeys, kr(J));
    stage_v(g, sg, kv_head, (j + 3) * kKeys, vr(J + 3));
    sub_step<0, true, true, true>(kr(J + 1), vr(J), sr(J), 1, A, B, n, half, magic);
    sub_step<1, true, true, true>(kr(J + 1), vr(J), sr(J + 1), 0, A, B, n, half, magic);
    store_scales(sr(J + 3), sg, ks_held, (j + 3) * kKeys, g.tokens);
    ks_held = ks_new;
    step_barrier<kWaitTwoSteps>();
    ++j;
  };
  const uint32_t n_steady = n_stages - 1;  // steps j with stage j+1
  for (; j + 4 <= n_steady;) {
    steady(std::integral_constant<int, 0>{});
    steady(std::integral_constant<int, 1>{});
    steady(std::integral_constant<int, 2>{});
    steady(std::integral_constant<int, 3>{});
  }
  if (j < n_steady) steady(std::integral_constant<int, 0>{});
  if (j < n_steady) steady(std::integral_constant<int, 1>{});
  if (j < n_steady) steady(std::integral_constant<int, 2>{});

  // ---- last step (j = n_stages - 1): PV of tiles 2j and 2j+1, the probabilities of 2j+1 between
  sub_step<0, false, true, true>(nullptr, vr(j), sr(j), 1, A, B, n, half, magic);
  sub_step<1, false, true, false>(nullptr, vr(j), nullptr, 0, A, B, n, half, magic);
  step_barrier<kWaitAll>();  // no staging load outlives the workgroup
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");  // the last PV MFMAs have landed

  // ---- normalise and store rows < min(token_count, tokens)
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const Tile& T = t == 0 ? A : B;
    float o[64];
    if (t == 0)
      read_tile<0>(o, std::make_integer_sequence<int, 64>{});
    else
      read_tile<1>(o, std::make_integer_sequence<int, 64>{});
    const float l_tot = T.l + __shfl_xor(T.l, 32);
    const float inv = 1.0f / l_tot;
    const uint32_t q = q0 + t * kTileQ;
    if (q < g.rows) {
      uint16_t* dst = g.out + (size_t)q * g.out_stride + head * 128;
#pragma unroll
      for (int db = 0; db < 4; ++db) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float* r = o + 16 * db + 4 * i;
          v4h h = {(_Float16)(r[0] * inv), (_Float16)(r[1] * inv), (_Float16)(r[2] * inv),
                   (_Float16)(r[3] * inv)};
          *reinterpret_cast<v4h*>(dst + 32 * db + 8 * i + 4 * half) = h;
        }
      }
    }
  }
}

}  // namespace

hipError_t launch_attention_hm(const h3_attention_cfg& cfg, uint32_t token_count, uint32_t heads,
                               const int32_t* qi, const float* qs, const int32_t* ki,
                               const float* ks, const uint16_t* vt, uint16_t* out,
                               hipStream_t stream) {
  Geometry g{};
  g.qi = qi;
  g.qs = qs;
  g.ki = ki;
  g.ks = ks;
  g.vt = vt;
  g.out = out;
  g.tokens = cfg.tokens;
  g.rows = std::min(token_count, cfg.tokens);
  g.capacity = cfg.token_capacity;
  g.out_stride = cfg.out_stride;
  g.q_blocks = (token_count + kBlockQ - 1) / kBlockQ;
  g.kv_head_limit = cfg.kv_stride / 128;
  g.head_limit = cfg.out_stride / 128;
  g.total = g.q_blocks * heads;
  g.per_xcd = (g.total + 7) / 8;
  hipLaunchKernelGGL(k_attention_hm, dim3(g.per_xcd * 8), dim3(kThreads), 0, stream, g);
  return hipGetLastError();
}

}  // namespace h3
