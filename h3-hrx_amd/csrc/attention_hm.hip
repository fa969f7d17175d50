// Head-major INT8-QK flash attention for gfx950 (CDNA4): attention_i8qkhm_mha8_k64_lds_f16_wmma
// (kernels/attention_i8qkhm_mha8_k64_lds_f16_wmma.loom:437-1067): non-causal MHA over head-major
// operands, keys >= tokens masked, rows >= token_count not written, f16 output
// [token_count][out_stride].
//
// Shape of the work. Eight waves per workgroup, two per SIMD, each owning one tile of 32 queries
// of one head; 64-key K / V^T tiles stream through LDS and are consumed in two sub-steps of 32
// keys. Sub-step t issues QK of key tile t+2 and PV of key tile t on the matrix cores while the
// vector ALU turns the scores of key tile t+1 into probabilities, so every MFMA has independent
// vector work beside it. A single wave issues vector instructions at half the SIMD's rate, which
// left the softmax as long as the MFMAs; with two waves per SIMD their vector work interleaves
// and each covers the other's waits. (Sustained dense MFMA work is power-limited on this part:
// the engine clock falls as the matrix cores' duty rises, so wall time, not cycles, is the
// measure of a schedule.) Per 32 keys:
//   QK   S^T (32 keys x 32 queries) = K . Q^T on v_mfma_i32_32x32x32_i8, exact int32; lane l owns
//        query l%32, accumulator register r holds MFMA row 8(r/4) + 4(l/32) + r%4 of the key
//        block. LDS row m of a K tile holds key swap23(m) (bits 2 and 3 exchanged), so registers
//        8g..8g+7 are keys 16g + 8(l/32) + 0..7 of the block: the B operand of a 16-key f16 MFMA
//        step with V^T in natural key order, and P never leaves its registers.
//   dequant  accumulators start from the bit pattern of 1.5*2^23, so each ends as the float
//        1.5*2^23 + S exactly and one FMA gives u = acc*ks + c with c = -1.5*2^23*ks staged per
//        key (rounded to f32, so u is S*ks to within 0.75*ks plus the FMA's rounding: less than
//        one unit of S), or c = -inf for a key past the sequence (masking costs nothing).
//   FP6 form (kFp6, h3_attention_i4qk_fp6): int4 codes c, converted beforehand to the FP6 e2m3
//        values c/2 (exact for every signed nibble, -8 included) in head-major rows laid out
//        for the f8f6f4 MFMA, and the key scales folded with the factor 4. QK is two
//        v_mfma_f32_32x32x64_f8f6f4 per 32 keys (64 channels each, at the int8 instruction's
//        cost), accumulating S/4 exactly in f32 from zero, so u = acc*(4ks) + c with c = 0 is
//        S*ks rounded once.
//   softmax  base 2 on y = u*qs*log2e - m with no per-tile max: the running max m is kept from
//        earlier tiles and a tile whose probabilities could exceed 2^8 is caught by its row sum
//        (every p >= 0, so the sum of a lane's 16 probabilities bounds each of them; f16
//        overflow shows as inf). Such a tile takes the exact path: its max is computed, m is
//        raised, the output accumulators and the sum are rescaled and its probabilities
//        recomputed. The first key tile always takes it (m starts at -1e30); in cross-
//        attention it computes its max before its probabilities instead, since O^T and the sum
//        are still zero and there is nothing to rescale.
//   PV   O^T (128 ch x 32 queries) += V^T . P^T on v_mfma_f32_32x32x16_f16, f32 accumulators;
//        the row sum adds the same f16 probabilities in f32, two at a time (v_dot2 with 1).
// S^T and P are double-buffered by key-tile parity, so every dependence between the matrix and
// the vector work is a whole sub-step long.
//
// Staging: K, V^T and key-scale tiles go through four-stage rings. K and V^T go from HBM into LDS
// with buffer_load ... lds (no registers, no LDS store instructions); the key scale takes a
// register (one load per lane for 8 lanes of each wave), stored with its c a step later. Step j
// (64 keys, two sub-steps) reads K(j+1), V(j) and the scales of stages j and j+1, and issues
// K(j+4), V(j+3) and the scale load of stage j+4, spread over the step, so every load has three
// steps to land; before the step's barrier a wave waits only for its own loads of two steps
// before. LDS rows are 128 bytes with their 16-byte chunks XOR-swizzled by (row/2)%8, so the 32
// rows a half-wave reads fall on distinct banks. Buffer descriptors end at the last valid key, so
// keys past the sequence read as zero.
// Workgroups are remapped so each XCD runs a contiguous range of (head, query block) work and its
// resident workgroups stream the same head's K/V^T through their shared L2.
#include <algorithm>
#include <type_traits>
#include <utility>

#include "internal.hpp"

namespace h3 {
namespace {

constexpr int kWaves = 8;                         // two per SIMD
constexpr int kThreads = 64 * kWaves;
constexpr int kTileQ = 32;                        // queries per wave
constexpr int kBlockQ = kWaves * kTileQ;          // 256 queries per workgroup
constexpr int kKeys = 64;                         // keys per LDS tile
constexpr int kRowBytes = 128;
constexpr int kKStage = kKeys * kRowBytes;        // 8192: int8 codes of 64 keys
constexpr int kVStage = 128 * kRowBytes;          // 16384: 128 channels x 64 keys of f16
constexpr int kSStage = 2 * kKeys * 4;            // 512: ks[64], c[64] at MFMA-row index
constexpr int kTabStages = 64;  // key tiles of a chained sequence (kPersistMaxStages)
constexpr int kKLoads = kKStage / 1024 / kWaves;  // 1 KiB LDS-DMA loads per wave per tile: 1
constexpr int kVLoads = kVStage / 1024 / kWaves;  // 2
constexpr int kSRows = kKeys / kWaves;            // scale rows stored per wave: 8
constexpr int kLoadsPerStep = kKLoads + kVLoads + 1;
constexpr int kLoadGap = 6;                       // chunks between a step's staging loads
// s_waitcnt fields (gfx9 layout): vmcnt <= the loads of one or two steps, expcnt untouched,
// lgkmcnt 0; or vmcnt 0.
// Memory loads a wave issues per step: the key scale, its K and V^T LDS-DMA loads, and with
// cross-attention also the key's mask byte (a second load in the scale's slot).
template <bool kCross>
constexpr int kVmemPerStep = kLoadsPerStep + (kCross ? 1 : 0);
// With the scales resident in LDS (kTab: chained cross-attention) a step loads no scale or mask.
template <bool kCross, bool kTab = false>
constexpr int kVmemStep = kTab ? kLoadsPerStep - 1 : kVmemPerStep<kCross>;
template <bool kCross, bool kTab = false>
constexpr int kWaitPrevStep = kVmemStep<kCross, kTab> | (7 << 4) | (0 << 8);
template <bool kCross, bool kTab = false>
constexpr int kWaitTwoSteps = (2 * kVmemStep<kCross, kTab>) | (7 << 4) | (0 << 8);
constexpr int kWaitAll = 0 | (7 << 4) | (0 << 8);
// LDS work only: vmcnt at its maximum (63: low bits 3:0 and high bits 15:14), lgkmcnt 0.
constexpr int kWaitLds = 0xF | (7 << 4) | (0 << 8) | (3 << 14);
constexpr int kWaitLdsWrites = kWaitLds;  // the same wait, named for its use in the epilogue
static_assert(2 * kVmemPerStep<true> < 16, "the vmcnt field's low four bits hold the count");
// V^T operands are read kPf chunks ahead of their MFMA, and a step's barrier comes right after
// the last operand read of its second sub-step, at chunk 12 - kPf. The unchained INT8 kernel
// reads 5 ahead (0.5 % faster at C3 than 4, with the priority scheme below); the chained ones
// keep 4, where 5 makes the compiler spill 4-12 dwords, and so does the FP6 form, which 5 made
// 0.7 % slower.
template <bool kChain, bool kFp6>
constexpr int kPf = kChain || kFp6 ? 4 : 5;
template <bool kChain, bool kFp6>
constexpr int kBarrierChunk = 12 - kPf<kChain, kFp6>;
constexpr int kKBias = 65536;                     // see Lanes
constexpr int kOStage = kTileQ * 64 * 2;          // 4 KiB: 32 output rows x 64 channels of f16
static_assert(4 * kOStage == kVStage, "four waves' output stages fill one V^T stage");
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kMagic = 12582912.0f;             // 1.5 * 2^23, the QK accumulators' bias
constexpr int kMagicBits = 0x4B400000;            // its bit pattern
constexpr float kSumLimit = 256.0f;               // a lane's tile sum above this: exact path
constexpr int kCpolNt = 2;                        // buffer store cache policy: non-temporal
constexpr int kRsrcWord3 = 0x00020000;            // gfx9 raw buffer: 32-bit data, no swizzle

typedef __attribute__((address_space(3))) void lds_void;
typedef unsigned int v4u __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v6i __attribute__((ext_vector_type(6)));  // an FP6 MFMA operand: 32 six-bit codes

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
  uint32_t tokens;       // keys (and, self-attention, readable query rows)
  uint32_t rows;         // query rows written: min(token_count, tokens); cross: query tokens
  uint32_t capacity;     // head-major row capacity of K / V^T (and, self-attention, of Q)
  uint32_t out_stride;
  uint32_t q_blocks;     // self: ceil(token_count / 256); cross: ceil(q_tokens / queries per head)
  uint32_t kv_head_limit;
  uint32_t head_limit;
  uint32_t total;        // q_blocks * heads (cross: * kv_heads)
  uint32_t per_xcd;      // ceil(total / 8): blocks per XCD
  uint32_t wpx;          // persistent workgroups per XCD (at most per_xcd)
  // cross-attention only: keys with key_mask == 0 are dead; the kv_group query heads of a key /
  // value head share a workgroup, waves_per_head = 8 / kv_group waves each
  const uint8_t* key_mask;
  uint32_t q_tokens;
  uint32_t q_capacity;
  uint32_t kv_group;
  uint32_t waves_per_head;
  // token-major operands (kTm; attention_i8qk_family's layouts): codes [token][stride] int8, key
  // scales at ks[key * ks_key + kv_head * ks_head] ([token][kv_heads] f32, or the lent head-major
  // copy [kv_head][tokens]), query scales at qs[query * qs_row + head]
  uint32_t k_row;    // bytes from one key's row of K to the next (kv_stride)
  uint32_t q_row;    // bytes from one query's row of Q to the next (q_stride)
  uint32_t ks_key;
  uint32_t ks_head;
  uint32_t qs_row;   // q_stride / 128
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
// K row m holds key swap23(m). With token-major operands (kTm) a key's 128 bytes are one piece of
// its token's row, k_row bytes after the previous key's.
template <bool kTm = false>
__device__ __forceinline__ Stager make_stager(const Geometry& g, int wave, int lane) {
  Stager s;
  s.wave = wave;
#pragma unroll
  for (int t = 0; t < kKLoads; ++t) {
    const uint32_t o = (wave * kKLoads + t) * 1024 + 16 * lane;
    const uint32_t row = o >> 7, chunk = ((o >> 4) & 7) ^ ((row >> 1) & 7);
    s.koff[t] = swap23(row) * (kTm ? g.k_row : kRowBytes) + 16 * chunk;
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

// Staging loads of one step (K tile at key kk0, V^T tile at key vk0, the key scales of the tile at
// key sk0): buffer descriptors that end at the last valid key (K, scales) or at the end of the
// head's V^T block.
struct StepLoads {
  __amdgpu_buffer_rsrc_t rk, rv, rs, rm;
  char* kst;
  char* vst;
  float ks;
  uint32_t keep;    // cross-attention: the key's mask byte (0 past the sequence)
  uint32_t sbytes;  // token-major operands: bytes from one key's scale to the next
};
template <bool kCross, bool kTm = false>
__device__ __forceinline__ StepLoads plan_step(const Geometry& g, uint32_t kv_head, uint32_t kk0,
                                               char* kst, uint32_t vk0, char* vst, uint32_t sk0) {
  StepLoads L;
  const uint32_t live = g.tokens > kk0 ? min(g.tokens - kk0, (uint32_t)kKeys) : 0u;
  const uint32_t slive = g.tokens > sk0 ? min(g.tokens - sk0, (uint32_t)kKeys) : 0u;
  if (kTm) {  // the descriptors end at the last valid key's scale and row
    L.rs = rsrc(g.ks + (size_t)sk0 * g.ks_key + (size_t)kv_head * g.ks_head,
                slive ? ((slive - 1) * g.ks_key + 1) * 4 : 0u);
    L.rk = rsrc(reinterpret_cast<const char*>(g.ki) + (size_t)kk0 * g.k_row + kv_head * 128,
                live ? (live - 1) * g.k_row + 128 : 0u);
  } else {
    L.rs = rsrc(g.ks + (size_t)kv_head * g.capacity + sk0, slive * 4);
    L.rk = rsrc(reinterpret_cast<const char*>(g.ki) + ((size_t)kv_head * g.capacity + kk0) * 128,
                live * 128);
  }
  if (kCross) L.rm = rsrc(g.key_mask + sk0, slive);
  L.keep = 0;
  L.sbytes = kTm ? g.ks_key * 4 : 4u;
  // V^T: columns past `tokens` inside the head's block are zero or belong to the next channel
  // row, and meet probability 0
  const uint32_t blk = 128 * g.capacity;
  L.rv = rsrc(reinterpret_cast<const char*>(g.vt) + ((size_t)kv_head * blk + vk0) * 2,
              vk0 < blk ? (blk - vk0) * 2 : 0u);
  L.kst = kst;
  L.vst = vst;
  L.ks = 0.0f;
  return L;
}
// Load `slot` of a step: 0 the key scale (into a register; with cross-attention also the key's
// mask byte), then the K tile's LDS-DMA loads, then the V^T tile's. The scale is of the stage
// after the step's K tile, so that it has two steps to land before it is stored.
template <bool kCross, bool kTm = false, bool kTab = false>
__device__ __forceinline__ void issue_load(StepLoads& L, const Stager& sg, int slot) {
  if (slot == 0) {
    if (kTab) return;  // the scales and mask bytes are resident in LDS
    L.ks = __builtin_bit_cast(
        float, __builtin_amdgcn_raw_buffer_load_b32(L.rs, sg.skey * (kTm ? L.sbytes : 4u), 0, 0));
    if (kCross) L.keep = __builtin_amdgcn_raw_buffer_load_b8(L.rm, sg.skey, 0, 0);
  } else if (slot <= kKLoads) {
    const int t = slot - 1;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        L.rk, (lds_void*)(L.kst + (sg.wave * kKLoads + t) * 1024), 16, sg.koff[t], 0, 0, 0);
  } else {
    const int t = slot - 1 - kKLoads;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        L.rv, (lds_void*)(L.vst + (sg.wave * kVLoads + t) * 1024), 16, sg.voff[t], 0, 0, 0);
  }
}
template <bool kCross, bool kTm = false, bool kTab = false>
__device__ __forceinline__ void issue_k(StepLoads& L, const Stager& sg) {
#pragma unroll
  for (int s = 0; s <= kKLoads; ++s) issue_load<kCross, kTm, kTab>(L, sg, s);
}
template <bool kCross, bool kTm = false>
__device__ __forceinline__ void issue_v(StepLoads& L, const Stager& sg) {
#pragma unroll
  for (int s = kKLoads + 1; s < kLoadsPerStep; ++s) issue_load<kCross, kTm>(L, sg, s);
}

// Scales of K tile k0 at their MFMA rows: ks, and c = -1.5*2^23*ks for a key inside the
// sequence or -inf for one past it. Within each aligned group of 4 rows (one lane half's keys of
// a quarter), ks is stored rotated by one slot and c by two, so that in the dequantisation FMA
// of row j the score (register 4i+j of S^T), its ks (slot j+1 of a 4-register load) and its c
// (slot j+2) lie in three different VGPR banks; unrotated, all three share bank j and every FMA
// waits on bank conflicts.
__device__ __forceinline__ uint32_t rot(uint32_t r, uint32_t by) {
  return (r & ~3u) | ((r + by) & 3u);
}
template <bool kFp6 = false>
__device__ __forceinline__ void store_scales(char* sst, const Stager& sg, float ks, uint32_t k0,
                                             uint32_t tokens) {
  if ((threadIdx.x & 63) < kSRows) {
    float* sc = reinterpret_cast<float*>(sst);
    sc[rot(sg.srow, 1)] = ks;
    sc[kKeys + rot(sg.srow, 2)] = k0 + sg.skey < tokens ? (kFp6 ? 0.0f : -(kMagic * ks)) : -INFINITY;
  }
}
// Cross-attention: a key is live when its mask byte is nonzero (the mask's descriptor ends at the
// last key, so keys past the sequence read 0).
__device__ __forceinline__ void store_scales_masked(char* sst, const Stager& sg, float ks,
                                                    uint32_t keep) {
  if ((threadIdx.x & 63) < kSRows) {
    float* sc = reinterpret_cast<float*>(sst);
    sc[rot(sg.srow, 1)] = ks;
    sc[kKeys + rot(sg.srow, 2)] = keep != 0 ? -(kMagic * ks) : -INFINITY;
  }
}
template <bool kCross, bool kFp6 = false>
__device__ __forceinline__ void store_stage_scales(char* sst, const Stager& sg, float ks,
                                                   uint32_t keep, uint32_t k0, uint32_t tokens) {
  if (kCross)
    store_scales_masked(sst, sg, ks, keep);
  else
    store_scales<kFp6>(sst, sg, ks, k0, tokens);
}

// Barrier between steps: this wave's LDS writes, and its staging loads from before the current
// step (or the two current steps), are complete; the later loads stay in flight.
template <int kWait>
__device__ __forceinline__ void step_barrier() {
  __builtin_amdgcn_s_waitcnt(kWait);
  asm volatile("s_barrier" ::: "memory");
}

// Issue priority of the two waves of a SIMD. The matrix pipe serves the older wave (waves 0-3)
// first when both have an MFMA ready, so with equal priorities waves 0-3 finished a step's first
// sub-step in ~1,160 cycles and waves 4-7 in ~1,780, and waves 0-3 then idled ~870 cycles of a
// ~3,020-cycle step at the barrier while waves 4-7 ran alone (s_memtime stamps at C3). Waves 4-7
// take priority 1 for the first sub-step of every steady step and all waves return to 0 for the
// second: the barrier wait falls to ~240 cycles and a step to ~2,840 (-2.4 to -3.1 % at C3).
// Longer or shorter windows measured worse. The choice between the two values is made inside
// the asm (a scalar branch the compiler does not see), so the steady loop's control flow, and
// the register allocation around its inline-asm MFMAs, stay as they are.
__device__ __forceinline__ void prio_late_waves_first(uint32_t wave) {
  asm volatile(
      "s_cmp_lt_u32 %0, 4\n\t"
      "s_cbranch_scc1 1f\n\t"
      "s_setprio 1\n\t"
      "s_branch 2f\n"
      "1:\n\t"
      "s_setprio 0\n"
      "2:" ::"s"(wave)
      : "scc");
}
__device__ __forceinline__ void prio_equal() { asm volatile("s_setprio 0"); }

// The wave's 32-query tile. S^T and P are double-buffered by the parity of the 32-key tile they
// belong to.
struct Tile {
  v16i s[2];    // S^T of the 32-key tiles of each parity
  v4i q[4];     // Q^T operand: 4 chunks of 32 channels
  v6i qf[2];    // FP6 form: the Q^T operand, 2 chunks of 64 channels
  float qsl;    // qs * log2(e)
  float cq;     // -1.5*2^23 * qsl: removes the QK accumulators' bias (0 in the FP6 form)
  float negm;   // minus the running max (log2 units)
  float l;      // this lane's share of the row sum
};

// Issue-order fence: the scheduler keeps each chunk's MFMA, LDS reads and vector work together.
#define H3_CHUNK_END() __builtin_amdgcn_sched_barrier(0)

__device__ __forceinline__ uint32_t chunk_off(int x, int half, uint32_t sw) {
  return 16 * ((2 * x + half) ^ sw);
}

// This lane's byte offsets in the LDS stages, computed once: row n of a 32-row block with the
// chunk swizzle applied, for K chunk x (4 per row) and V^T key group g (4 per 64-key row), and
// its lane half's first scale. Every LDS read is one of these plus a constant, which the
// instruction's 16-bit offset field takes; the K offsets carry 64 KiB of their own, since the K
// stages lie above the V^T stages (a K stage's constant is then its address less 64 KiB).
struct Lanes {
  uint32_t k[4];
  uint32_t v[4];
  uint32_t s;
};
// FP6 form: a 128-byte K row holds 32-byte blocks b (channels 32b .. 32b+31, 24 bytes of codes
// and 8 of padding), so the operand of QK chunk x (channels 64x ..) for lane half h is block
// 2x + h: 16-byte chunks 4x + 2h (k[2x]) and 4x + 2h + 1 (first 8 bytes, k[2x+1]).
template <bool kFp6 = false>
__device__ __forceinline__ Lanes make_lanes(int n, int half) {
  Lanes L;
  const uint32_t sw = (n >> 1) & 7;
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    L.k[x] = kKBias + n * kRowBytes +
             (kFp6 ? 16 * ((4 * (x >> 1) + 2 * half + (x & 1)) ^ sw) : chunk_off(x, half, sw));
    L.v[x] = n * kRowBytes + chunk_off(x, half, sw);
    asm volatile("" : "+v"(L.k[x]));
    asm volatile("" : "+v"(L.v[x]));
  }
  L.s = 16 * half;
  asm volatile("" : "+v"(L.s));
  return L;
}

// The MFMAs are written as inline assembly on VGPRs only, and the output accumulators O^T live
// in fixed VGPRs: block db (32 channels x 32 queries, f32) in v[192 + 16db .. +15], v192-v255 in
// all. The compiler allocates only v0-v191 (amdgpu_num_vgpr), so nothing of its own ever lands
// there, and every asm that touches them names them as clobbered (which also counts them in the
// kernel's register total: 256, two waves per SIMD). The kernel uses no AGPRs: a kernel that does
// gets only half of that budget as VGPRs. S^T stays in VGPRs for the vector ALU, and O^T never
// moves (a compiler-managed O^T is copied between register sets wherever the exact path rejoins
// the fast one). Hazards are covered by the schedule: an accumulator chain is the same opcode on
// exactly the same registers, which the hardware forwards with no wait states; the vector ALU
// reads S^T only in the next sub-step or after explicit waits (sub-steps without PV), writes P a
// sub-step before PV reads it, and touches O^T only in the exact path and the epilogue, both
// behind explicit waits.
constexpr int kOReg = 192;  // first VGPR of O^T
// P, PV's B operand: the probabilities of the 32-key tile of parity `par` as packed f16, 16 keys
// per MFMA group g, in v[kPReg + 8 par + 4 g .. +3] (four words: quarters 2g and 2g+1, two words
// each). Written by the softmax's conversions and read by the PV MFMAs in place, so no copies sit
// between them; the compiler's share ends below kPReg.
constexpr int kPReg = 176;
#define H3_V16(b) "v" #b "0", "v" #b "1", "v" #b "2", "v" #b "3", "v" #b "4", "v" #b "5", \
                  "v" #b "6", "v" #b "7", "v" #b "8", "v" #b "9"
#define H3_P_CLOBBERS "v176", "v177", "v178", "v179", "v180", "v181", "v182", "v183", "v184", \
    "v185", "v186", "v187", "v188", "v189", "v190", "v191"
#define H3_O_CLOBBERS "v192", "v193", "v194", "v195", "v196", "v197", "v198", "v199", H3_V16(20), \
    H3_V16(21), H3_V16(22), H3_V16(23), H3_V16(24), "v250", "v251", "v252", "v253", "v254", "v255"

// O^T block at VGPR kBase += V^T . P^T, P group at VGPR kP
template <int kBase, int kP>
__device__ __forceinline__ void pv_block(v8h v) {
  asm volatile("v_mfma_f32_32x32x16_f16 v[%1:%2], %0, v[%3:%4], v[%1:%2]"
               :: "v"(v), "n"(kBase), "n"(kBase + 15), "n"(kP), "n"(kP + 3) : H3_O_CLOBBERS);
}
template <int kP>
__device__ __forceinline__ void pv_group(int db, v8h v) {
  switch (db) {  // db is a constant once the chunk loop is unrolled
    case 0: pv_block<kOReg, kP>(v); break;
    case 1: pv_block<kOReg + 16, kP>(v); break;
    case 2: pv_block<kOReg + 32, kP>(v); break;
    default: pv_block<kOReg + 48, kP>(v); break;
  }
}
// PV for channel block db with P group g of parity par (all constants once unrolled).
__device__ __forceinline__ void pv_mfma(int db, v8h v, int par, int g) {
  switch (2 * par + g) {
    case 0: pv_group<kPReg>(db, v); break;
    case 1: pv_group<kPReg + 4>(db, v); break;
    case 2: pv_group<kPReg + 8>(db, v); break;
    default: pv_group<kPReg + 12>(db, v); break;
  }
}
// Accumulator register kOReg + kR *= alpha, its read for the epilogue, and its clearing.
template <int kR>
__device__ __forceinline__ void scale_acc(float alpha) {
  asm volatile("v_mul_f32 v[%1], v[%1], %0" :: "v"(alpha), "n"(kOReg + kR) : H3_O_CLOBBERS);
}
template <int kR>
__device__ __forceinline__ float read_acc() {
  float t;
  asm volatile("v_mov_b32 %0, v[%1]" : "=v"(t) : "n"(kOReg + kR));
  return t;
}
template <int kR>
__device__ __forceinline__ void zero_acc() {
  asm volatile("v_mov_b32 v[%0], 0" :: "n"(kOReg + kR) : H3_O_CLOBBERS);
}
template <int... kR>
__device__ __forceinline__ void scale_all(float alpha, std::integer_sequence<int, kR...>) {
  (scale_acc<kR>(alpha), ...);
}
template <int... kR>
__device__ __forceinline__ void read_all(float (&o)[64], std::integer_sequence<int, kR...>) {
  ((o[kR] = read_acc<kR>()), ...);
}
template <int... kR>
__device__ __forceinline__ void zero_all(std::integer_sequence<int, kR...>) {
  (zero_acc<kR>(), ...);
}

// FP6 form: QK chunk x of a tile on the f8f6f4 MFMA (both operands FP6 e2m3), from zero or
// accumulating.
__device__ __forceinline__ v16i qk_fp6_first(v6i k, v6i q) {
  v16i d;
  asm volatile("v_mfma_f32_32x32x64_f8f6f4 %0, %1, %2, 0 cbsz:2 blgp:2" : "=&v"(d) : "v"(k), "v"(q));
  return d;
}
__device__ __forceinline__ void qk_fp6_next(v16i& d, v6i k, v6i q) {
  asm volatile("v_mfma_f32_32x32x64_f8f6f4 %0, %1, %2, %0 cbsz:2 blgp:2" : "+v"(d) : "v"(k), "v"(q));
}

// The first QK MFMA of a tile accumulates onto the bias 1.5*2^23 (`magic`, kept in registers).
__device__ __forceinline__ v16i qk_first(v4i k, v4i q, const v16i& magic) {
  v16i d;
  asm volatile("v_mfma_i32_32x32x32_i8 %0, %1, %2, %3" : "=&v"(d) : "v"(k), "v"(q), "v"(magic));
  return d;
}
__device__ __forceinline__ void qk_next(v16i& d, v4i k, v4i q) {
  asm volatile("v_mfma_i32_32x32x32_i8 %0, %1, %2, %0" : "+v"(d) : "v"(k), "v"(q));
}


__device__ __forceinline__ float half_swap_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Scales of quarter i (slots 4i..4i+3) of key block b: ks at kss[32b + 8i + 4h .. +3] for lane
// half h (byte offset `soff` = 16h), c 64 floats further.
__device__ __forceinline__ float4 scale4(const float* kss, int b, int i, uint32_t soff) {
  return *reinterpret_cast<const float4*>(reinterpret_cast<const char*>(kss + 32 * b + 8 * i) +
                                          soff);
}

// Dequantized scores of quarter i of the tile's S^T on the masked path (a key's c is -inf when
// it is dead): u = acc*ks + c, with the scales of row j in slot j+1 of k4 and j+2 of c4 (stored
// rotated, so the three operands of each FMA lie in different VGPR banks).
__device__ __forceinline__ void dequant_quarter(const v16i& s, int i, float4 k4, float4 c4,
                                                float (&u)[4]) {
  asm volatile("v_fma_f32 %0, %4, %8, %12\n\t"
               "v_fma_f32 %1, %5, %9, %13\n\t"
               "v_fma_f32 %2, %6, %10, %14\n\t"
               "v_fma_f32 %3, %7, %11, %15"
               : "=&v"(u[0]), "=&v"(u[1]), "=&v"(u[2]), "=&v"(u[3])
               : "v"(s[4 * i]), "v"(s[4 * i + 1]), "v"(s[4 * i + 2]), "v"(s[4 * i + 3]),
                 "v"(k4.y), "v"(k4.z), "v"(k4.w), "v"(k4.x),
                 "v"(c4.z), "v"(c4.w), "v"(c4.x), "v"(c4.y));
}
// y = u*qsl + negm for the four dequantized scores.
__device__ __forceinline__ void exparg_quarter(float (&y)[4], float qsl, float negm) {
  asm volatile("v_fma_f32 %0, %0, %4, %5\n\t"
               "v_fma_f32 %1, %1, %4, %5\n\t"
               "v_fma_f32 %2, %2, %4, %5\n\t"
               "v_fma_f32 %3, %3, %4, %5"
               : "+v"(y[0]), "+v"(y[1]), "+v"(y[2]), "+v"(y[3])
               : "v"(qsl), "v"(negm));
}

// Exponent arguments y (log2 units, less the running max) of quarter i, on a tile whose keys all
// lie inside the sequence: t = acc*qsl + cq with the lane's own constants (cq removes the
// accumulators' bias, so t is S*qs*log2(e) to within 0.75*qsl, less than one unit of S), then
// y = t*ks + negm. Only the key scales come from LDS (row j's in slot j+1 of k4). Both FMAs are
// full-rate vector instructions; the masked path below needs the c values as well.
__device__ __forceinline__ void scores_quarter(const v16i& s, int i, float4 k4, float qsl,
                                               float cq, float negm, float (&y)[4]) {
  asm volatile("v_fma_f32 %0, %4, %8, %9\n\t"
               "v_fma_f32 %1, %5, %8, %9\n\t"
               "v_fma_f32 %2, %6, %8, %9\n\t"
               "v_fma_f32 %3, %7, %8, %9\n\t"
               "v_fma_f32 %0, %0, %10, %14\n\t"
               "v_fma_f32 %1, %1, %11, %14\n\t"
               "v_fma_f32 %2, %2, %12, %14\n\t"
               "v_fma_f32 %3, %3, %13, %14"
               : "=&v"(y[0]), "=&v"(y[1]), "=&v"(y[2]), "=&v"(y[3])
               : "v"(s[4 * i]), "v"(s[4 * i + 1]), "v"(s[4 * i + 2]), "v"(s[4 * i + 3]),
                 "v"(qsl), "v"(cq), "v"(k4.y), "v"(k4.z), "v"(k4.w), "v"(k4.x), "v"(negm));
}
// The same on a tile that holds dead keys (past the sequence, or masked in cross-attention):
// u = acc*ks + c with c = -inf for a dead key, then y = u*qsl + negm (-inf: probability 0).
__device__ __forceinline__ void scores_quarter_masked(const v16i& s, int i, float4 k4, float4 c4,
                                                      float qsl, float negm, float (&y)[4]) {
  dequant_quarter(s, i, k4, c4, y);
  exparg_quarter(y, qsl, negm);
}
// The exponent arguments of quarter i: on a tile that may hold dead keys (kMasked) through their
// staged c values, else from the key scales alone.
template <bool kMasked>
__device__ __forceinline__ void scores(const v16i& s, int i, float4 k4, float4 c4, float qsl,
                                       float cq, float negm, float (&y)[4]) {
  if constexpr (kMasked)
    scores_quarter_masked(s, i, k4, c4, qsl, negm, y);
  else
    scores_quarter(s, i, k4, qsl, cq, negm, y);
}

// p = 2^y in f32, in place, in two parts: three of the quarter's exponentials with the sum of
// the first two (`a`), then the fourth with the f16 packing (v_cvt_pk_f16_f32, round to nearest
// even) of (p0, p1) and (p2, p3) as PV's B operand and the rest of the quarter's sum into the
// tile sum `ts`. The row sum adds the unrounded f32 probabilities, as the reference does; f32
// adds run beside the matrix pipe, where dot-product instructions would occupy it. A
// transcendental's result is read only after one wait state: p0 and p1 two and one
// instructions after their exponentials in the first part, p3 after the first conversion.
__device__ __forceinline__ void exp3_quarter(float (&y)[4], float& a) {
  asm volatile("v_exp_f32 %0, %0\n\t"
               "v_exp_f32 %1, %1\n\t"
               "v_exp_f32 %2, %2\n\t"
               "v_add_f32 %3, %0, %1"
               : "+v"(y[0]), "+v"(y[1]), "+v"(y[2]), "=&v"(a));
}
template <int kW>
__device__ __forceinline__ void exp_pack_to(float (&y)[4], float& a, float& ts) {
  float b;
  asm volatile("v_exp_f32 %1, %1\n\t"
               "v_cvt_pk_f16_f32 v[%4], %6, %7\n\t"
               "v_cvt_pk_f16_f32 v[%5], %8, %1\n\t"
               "v_add_f32 %0, %8, %1\n\t"
               "v_add_f32 %2, %2, %0\n\t"
               "v_add_f32 %3, %3, %2"
               : "=&v"(b), "+v"(y[3]), "+v"(a), "+v"(ts)
               : "n"(kW), "n"(kW + 1), "v"(y[0]), "v"(y[1]), "v"(y[2])
               : H3_P_CLOBBERS);
}
// The fourth exponential of quarter i, the f16 packing of (p0, p1) and (p2, p3) into the P words
// of parity par (group i/2, words 2(i%2) and +1) and the rest of the quarter's sum into `ts`.
__device__ __forceinline__ void exp_pack_quarter(float (&y)[4], float& a, float& ts, int par,
                                                 int i) {
  switch (8 * par + 2 * i) {  // constants once unrolled
    case 0: exp_pack_to<kPReg + 0>(y, a, ts); break;
    case 2: exp_pack_to<kPReg + 2>(y, a, ts); break;
    case 4: exp_pack_to<kPReg + 4>(y, a, ts); break;
    case 6: exp_pack_to<kPReg + 6>(y, a, ts); break;
    case 8: exp_pack_to<kPReg + 8>(y, a, ts); break;
    case 10: exp_pack_to<kPReg + 10>(y, a, ts); break;
    case 12: exp_pack_to<kPReg + 12>(y, a, ts); break;
    default: exp_pack_to<kPReg + 14>(y, a, ts); break;
  }
}

// The probabilities of quarter i against negm: y, then p = 2^y packed as PV's operand into the P
// words of parity par, and its share of the tile sum.
template <bool kMasked>
__device__ __forceinline__ float probs_quarter(Tile& T, int par, int i, float4 k4, float4 c4,
                                               float ts) {
  float y[4];
  float a;
  scores<kMasked>(T.s[par], i, k4, c4, T.qsl, T.cq, T.negm, y);
  exp3_quarter(y, a);
  exp_pack_quarter(y, a, ts, par, i);
  return ts;
}

// The exact path for probabilities of key tile `par` (computed against the running max) that may
// exceed 2^8: take the tile's max, raise m, rescale the accumulators and the row sum, recompute
// the probabilities. `kss` and `b` locate the key tile's scales. It works quarter by quarter,
// re-reading the scales, so that few registers are live beside the loop's own. The max is of the
// scores as the probabilities compute them, with negm = 0 (log2 units).
template <bool kMasked>
__device__ __forceinline__ void raise_exact(Tile& T, int par, const float* kss, int b,
                                            uint32_t soff, int half) {
  float tmax = -INFINITY;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float4 k4 = scale4(kss, b, i, soff);
    const float4 c4 = kMasked ? scale4(kss + kKeys, b, i, soff) : k4;
    float y[4];
    scores<kMasked>(T.s[par], i, k4, c4, T.qsl, T.cq, 0.0f, y);
#pragma unroll
    for (int j = 0; j < 4; ++j) tmax = fmaxf(tmax, y[j]);
  }
  tmax = half_swap_max(tmax);
  const float m_old = -T.negm;
  const float m_new = fmaxf(m_old, tmax);
  const float alpha = __builtin_amdgcn_exp2f(m_old - m_new);
  // The tile's PV MFMAs of this sub-step were issued before; the waits on both sides of the
  // rescale cover them and the next MFMA that reads the accumulators. alpha is an input of the
  // first wait, so it (a transcendental result, which a dependent instruction may read only after
  // a wait state) is complete before the waits begin; the compiler does not see the rescale's
  // inline-asm reads of it and would otherwise place the exponential right before them.
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" :: "v"(alpha)
               : "memory");
  scale_all(alpha, std::make_integer_sequence<int, 64>{});
  asm volatile("s_nop 7\n\ts_nop 7" ::: "memory");
  T.negm = -m_new;
  float ts = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float4 k4 = scale4(kss, b, i, soff);
    const float4 c4 = kMasked ? scale4(kss + kKeys, b, i, soff) : k4;
    ts = probs_quarter<kMasked>(T, par, i, k4, c4, ts);
  }
  T.l = T.l * alpha + ts;
  asm volatile("s_nop 7" ::: "memory");  // fresh P before the next MFMA reads it
}

// The probabilities of a block's first key tile in cross-attention: the exact path with nothing
// to rescale. The running max is still -1e30 (negm 1e30) and O^T and the row sum are zero, so the
// rescale of raise_exact multiplies zeros and 0*alpha + sum is the sum: the max is taken first
// and the probabilities computed once, from the same dequantised scores, with the results of the
// general path bit for bit and none of its overflowing first pass.
__device__ __forceinline__ void first_tile(Tile& T, int par, const float* kss, int b,
                                           uint32_t soff) {
  float u[4][4];
  float tmax = -INFINITY;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    dequant_quarter(T.s[par], i, scale4(kss, b, i, soff), scale4(kss + kKeys, b, i, soff), u[i]);
    float y[4] = {u[i][0], u[i][1], u[i][2], u[i][3]};
    exparg_quarter(y, T.qsl, 0.0f);
#pragma unroll
    for (int j = 0; j < 4; ++j) tmax = fmaxf(tmax, y[j]);
  }
  tmax = half_swap_max(tmax);
  T.negm = -fmaxf(-1.0e30f, tmax);
  float ts = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float a;
    exparg_quarter(u[i], T.qsl, T.negm);
    exp3_quarter(u[i], a);
    exp_pack_quarter(u[i], a, ts, par, i);
  }
  T.l = ts;
  asm volatile("s_nop 7" ::: "memory");  // fresh P before the next MFMA reads it
}

// The first LDS operands of a sub-step, read during the sub-step before it: the four K chunks of
// its QK and the scales of its first two quarters.
struct Pre {
  v4i k[4];
  v6i kf[2];  // FP6 form: the two K chunks
  float4 k4[2];  // key scales of quarters 0 and 1 (a masked sub-step reads their c itself)
};
// Part `part` (0-5) of the reads of `pre` for a sub-step that reads block `kb` of K stage `kst`
// and block `sb` of scale stage `sst`: parts 0-3 the K chunks, 4-5 the scales of quarters 0-1.
// FP6 form: parts 0-3 are the 16-byte and 8-byte halves of the two K chunks.
template <bool kFp6 = false>
__device__ __forceinline__ void prefetch(Pre& pre, int part, const char* kst, int kb,
                                         const char* sst, int sb, const Lanes& ln) {
  if (part < 4) {
    const char* a = kst + (32 * kb * kRowBytes - kKBias) + ln.k[part];
    if constexpr (kFp6) {
      v6i& d = pre.kf[part >> 1];
      if ((part & 1) == 0) {
        const v4i lo = *reinterpret_cast<const v4i*>(a), hi = __builtin_shufflevector(d, d, 4, 5, -1, -1);
        d = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5);
      } else {
        const v2i h2 = *reinterpret_cast<const v2i*>(a);
        const v4i lo = __builtin_shufflevector(d, d, 0, 1, 2, 3),
                  hi = __builtin_shufflevector(h2, h2, 0, 1, -1, -1);
        d = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5);
      }
    } else {
      pre.k[part] = *reinterpret_cast<const v4i*>(a);
    }
  } else {
    const float* kss = reinterpret_cast<const float*>(sst);
    pre.k4[part - 4] = scale4(kss, sb, part - 4, ln.s);
  }
}

// Sub-step t (kPar = t % 2), in 12 chunks of one MFMA each:
//   kQK  QK of key tile t+2 (its K chunks in `pre`) into S^T[kPar]
//   kPV  PV of key tile t (block kPar of V^T stage `vst`) from P[kPar]
//   kSM  probabilities of key tile t+1 (block `sb` of scale stage `sst`) from S^T[1-kPar] into
//        P[1-kPar], then the overflow check. kMasked: the tile may hold dead keys (past the
//        sequence, or masked in cross-attention), so its scores take the masked path, which
//        reads each key's c (-inf for a dead key) beside its scale.
// Every chunk issues its MFMA first and its vector work right behind it (all of it inline
// assembly, whose order the compiler keeps); then its LDS reads and whatever `stage(c, next)`
// issues (staging loads, the step barrier, the reads of the next sub-step's `Pre`). The K chunks
// and the first two quarters' key scales come in `pre`, read during the sub-step before; the 8
// V^T chunks are read kPfT chunks ahead. QK comes first, so the S^T it writes is read by the
// vector ALU only in the next sub-step, after this one's 8 PV MFMAs. The softmax runs quarter by
// quarter (4 keys of each lane half), three chunks each (the exponent arguments, three
// exponentials, the last one with the f16 packing and the quarter's share of the tile sum), with
// the scales of quarters 2 and 3 read two quarters ahead. Each quarter adds its probabilities to
// the lane's tile sum right away (f32 adds), so the overflow check after the last chunk waits on
// a few instructions only.
template <int kPar, bool kQK, bool kPV, bool kSM, bool kFp6, bool kFirst = false,
          bool kMasked = false, int kPfT = 4, typename Stage>
__device__ __forceinline__ void sub_step(const char* vst, const char* sst, int sb, Tile& T,
                                         const Lanes& ln, int half, const v16i& magic, Pre& pre,
                                         Stage&& stage) {
  constexpr int kSm = 1 - kPar;  // parity of the tile whose probabilities are computed
  const float* kss = reinterpret_cast<const float*>(sst);
  v4i kop[4];
  v6i kopf[2];
  v8h vop[8];
  float4 k4[4], c4[4];
  float y[4], ysum;
  float ts = 0.0f;  // the lane's tile sum
  auto read_op = [&](int o) {
    if (o >= 4 && kPV) {
      // V^T chunk v: channel block db = v % 4, key group 2*kPar + v / 4 of the stage
      const int v = o - 4, db = v & 3, g = 2 * kPar + (v >> 2);
      vop[v] = *reinterpret_cast<const v8h*>(vst + 32 * db * kRowBytes + ln.v[g]);
    }
  };
  auto read_scales = [&](int i) {
    k4[i] = scale4(kss, sb, i, ln.s);
    if (kMasked) c4[i] = scale4(kss + kKeys, sb, i, ln.s);
  };
  if constexpr (kFp6) {
    kopf[0] = pre.kf[0];
    kopf[1] = pre.kf[1];
  } else {
#pragma unroll
    for (int o = 0; o < 4; ++o) kop[o] = pre.k[o];
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    k4[i] = pre.k4[i];
    c4[i] = kMasked && kSM && !kFirst ? scale4(kss + kKeys, sb, i, ln.s) : k4[i];
  }
#pragma unroll
  for (int i = 2; i < 4; ++i) c4[i] = k4[0];  // defined before read_scales fills them
#pragma unroll
  for (int o = 4; o < 4 + kPfT; ++o) read_op(o);
#pragma unroll
  for (int c = 0; c < 12; ++c) {
    if (c < 4) {
      if (kQK) {
        if constexpr (kFp6) {  // chunks 1 and 3 carry no MFMA: their vector work stays
          if (c == 0)
            T.s[kPar] = qk_fp6_first(kopf[0], T.qf[0]);
          else if (c == 2)
            qk_fp6_next(T.s[kPar], kopf[1], T.qf[1]);
        } else if (c == 0) {
          T.s[kPar] = qk_first(kop[0], T.q[0], magic);
        } else {
          qk_next(T.s[kPar], kop[c], T.q[c]);
        }
      }
    } else if (kPV) {
      const int v = c - 4;
      pv_mfma(v & 3, vop[v], kPar, v >> 2);
    }
    if (kSM && !kFirst) {
      // quarter c/3: exponent arguments; three exponentials; the fourth with the packing and
      // the quarter's share of the tile sum
      const int i = c / 3, phase = c % 3;
      if (phase == 0) {
        scores<kMasked>(T.s[kSm], i, k4[i], c4[i], T.qsl, T.cq, T.negm, y);
      } else if (phase == 1) {
        exp3_quarter(y, ysum);
      } else {
        exp_pack_quarter(y, ysum, ts, kSm, i);
        if (i == 0 || i == 1) read_scales(i + 2);
      }
    }
    if (c >= 4 && c + kPfT < 12) read_op(c + kPfT);
    stage(c, pre);
    H3_CHUNK_END();
  }
  if (kQK && !kPV)  // the next sub-step's vector ALU reads this S^T at once: cover the latency
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  if constexpr (kSM && kFirst) {
    first_tile(T, kSm, kss, sb, ln.s);
  } else if (kSM) {
    if (__builtin_expect(__any(!(ts <= kSumLimit)), 0))
      raise_exact<kMasked>(T, kSm, kss, sb, ln.s, half);
    else
      T.l += ts;
  }
}

// The reads of the next step's first `Pre` (K stage `kst` block 0, scale stage `sst` block 1) in
// the chunks after the step barrier of a step's second sub-step.
template <bool kFp6, int kBar>
__device__ __forceinline__ void next_step_reads(int c, Pre& next, const char* kst, const char* sst,
                                                const Lanes& ln) {
  if (c == kBar + 1) {
    prefetch<kFp6>(next, 0, kst, 0, sst, 1, ln);
    prefetch<kFp6>(next, 4, kst, 0, sst, 1, ln);
  } else if (c == kBar + 2) {
    prefetch<kFp6>(next, 1, kst, 0, sst, 1, ln);
    prefetch<kFp6>(next, 5, kst, 0, sst, 1, ln);
  } else if (c == kBar + 3) {
    prefetch<kFp6>(next, 2, kst, 0, sst, 1, ln);
    prefetch<kFp6>(next, 3, kst, 0, sst, 1, ln);
  }
}

// Stage `i` of a ring of separately declared arrays (i is a constant after unrolling, so the
// compiler still sees which array every access and LDS-DMA goes to).
__device__ __forceinline__ char* ring(int i, char* a0, char* a1, char* a2, char* a3) {
  return i == 0 ? a0 : i == 1 ? a1 : i == 2 ? a2 : a3;
}

template <bool kCross, bool kChain, bool kFp6 = false, bool kTm = false>
__global__ __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(2, 2), amdgpu_num_vgpr(kPReg)))
void k_attention_hm(Geometry g) {
  static_assert(!kTm || (!kCross && !kFp6), "token-major operands: INT8 self-attention only");
  // Four-stage rings, each stage its own array so that the compiler can tell an LDS-DMA into one
  // stage from the reads of another.
  __shared__ __attribute__((aligned(16))) char k0s[kKStage], k1s[kKStage], k2s[kKStage], k3s[kKStage];
  __shared__ __attribute__((aligned(16))) char v0s[kVStage], v1s[kVStage], v2s[kVStage], v3s[kVStage];
  __shared__ __attribute__((aligned(16))) char s0s[kSStage], s1s[kSStage], s2s[kSStage], s3s[kSStage];
  auto kr = [&](int i) { return ring(i & 3, k0s, k1s, k2s, k3s); };
  auto vr = [&](int i) { return ring(i & 3, v0s, v1s, v2s, v3s); };
  auto sr = [&](int i) { return ring(i & 3, s0s, s1s, s2s, s3s); };
  // Chained cross-attention keeps the scale pairs (ks, c) of all its key tiles in LDS for as long
  // as its workgroup stays on one key/value head: the text keys are few (at most
  // kPersistMaxStages tiles here) and every block of the head walks the same ones, so the steps
  // load no scale or mask byte and store nothing, and no wait of theirs lands behind the previous
  // block's output stores. Stage `st`'s pairs sit at stab + st * kSStage in the ring layout.
  constexpr bool kTab = kCross && kChain;
  __shared__ __attribute__((aligned(16))) char stab[kTab ? kTabStages * kSStage : 16];
  // the scale stage of stage `st`, ring slot i
  auto ss = [&](int i, uint32_t st) -> char* { return kTab ? stab + st * kSStage : sr(i); };
  constexpr int kPfK = kPf<kChain, kFp6>;
  constexpr int kBarK = kBarrierChunk<kChain, kFp6>;

  // Persistent workgroups, XCD-aware: the hardware hands workgroup b to XCD b % 8, and each XCD
  // owns a contiguous range of per_xcd (head, query block) blocks, which its wpx workgroups take
  // in turn (workgroup i of the XCD: blocks i, i + wpx, i + 2 wpx, ...). At any moment the
  // XCD's resident workgroups hold wpx consecutive blocks, which share one head's K/V^T stream
  // through the XCD's L2, and a workgroup's next block is usually of the same key/value head.
  const uint32_t xcd = blockIdx.x & 7u;
  uint32_t local = blockIdx.x >> 3;
  if (local >= g.per_xcd || xcd * g.per_xcd + local >= g.total) return;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int n = lane & 31;
  const int half = lane >> 5;
  const Stager sg = make_stager<kTm>(g, wave, lane);
  const Lanes ln = make_lanes<kFp6>(n, half);
  // The QK bias 1.5*2^23, made opaque so that it stays in registers for the whole loop.
  v16i magic = {};  // the int8 form's accumulator bias (the FP6 form starts QK from zero)
  if constexpr (!kFp6) {
#pragma unroll
    for (int r = 0; r < 16; ++r) magic[r] = kMagicBits;
    asm volatile("" : "+v"(magic));
  }
  const uint32_t n_stages = (g.tokens + kKeys - 1) / kKeys;  // 64-key stages; 32-key tiles 2x
  // Chaining: when the next block reads the same K/V^T stream and the stage count is a multiple
  // of the ring length, this block's last steady steps stage the next block's first stages
  // (K 0-2, V^T 0-1 and their scales) into the ring slots they would have had anyway, so the
  // next block starts without a prologue.
  const bool chain_ok = kChain && n_stages % 4 == 0;
  auto kv_head_of = [&](uint32_t logical) {
    const uint32_t head_y = logical / g.q_blocks;
    return kCross ? head_y : head_y % g.kv_head_limit;
  };
  // This wave's part of block `logical`: key/value head, query head, first query row of its tile.
  struct WaveBlock {
    uint32_t kv_head, head, q0;
  };
  auto wave_block = [&](uint32_t logical) {
    const uint32_t head_y = logical / g.q_blocks;
    const uint32_t qb = logical % g.q_blocks;
    WaveBlock w;
    if (kCross) {  // block = (key/value head, query block); its kv_group query heads share it
      w.kv_head = head_y;
      w.head = w.kv_head * g.kv_group + (uint32_t)wave / g.waves_per_head;
      w.q0 = (qb * g.waves_per_head + (uint32_t)wave % g.waves_per_head) * kTileQ;
    } else {
      w.kv_head = head_y % g.kv_head_limit;
      w.head = w.kv_head % g.head_limit;
      w.q0 = qb * kBlockQ + wave * kTileQ;
    }
    return w;
  };
  const uint32_t q_limit = kCross ? g.q_tokens : g.tokens;  // readable query rows
  const uint32_t q_cap = kCross ? g.q_capacity : g.capacity;
  // The Q^T operand and scale of this lane's query in block `w`.
  // The Q^T operand of this lane's query in block `w`; returns the query's scale.
  auto load_q_codes = [&](Tile& T, const WaveBlock& w) -> float {
    const uint32_t qq = w.q0 + n;
    const uint32_t q_read = qq < q_limit ? qq : q_limit - 1;
    const int32_t* src =
        kTm ? reinterpret_cast<const int32_t*>(reinterpret_cast<const char*>(g.qi) +
                                               (size_t)q_read * g.q_row + w.head * 128)
            : g.qi + ((size_t)w.head * q_cap + q_read) * 32;
    if constexpr (kFp6) {  // blocks 2x + half of the row: 24 bytes of codes each
      const char* b = reinterpret_cast<const char*>(src) + 32 * half;
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        const v2i h2 = *reinterpret_cast<const v2i*>(b + 64 * x + 16);
        T.qf[x] = __builtin_shufflevector(*reinterpret_cast<const v4i*>(b + 64 * x),
                                          __builtin_shufflevector(h2, h2, 0, 1, -1, -1), 0, 1, 2,
                                          3, 4, 5);
      }
    } else {
#pragma unroll
      for (int dc = 0; dc < 4; ++dc) T.q[dc] = *reinterpret_cast<const v4i*>(src + 8 * dc + 4 * half);
    }
    return kTm ? g.qs[(size_t)q_read * g.qs_row + w.head] : g.qs[(size_t)w.head * q_cap + q_read];
  };
  auto set_q_scale = [&](Tile& T, float qs) {
    T.qsl = qs * kLog2e;
    T.cq = kFp6 ? 0.0f : -(kMagic * T.qsl);
  };
  auto load_q = [&](Tile& T, const WaveBlock& w) { set_q_scale(T, load_q_codes(T, w)); };

  bool chained = false;  // this block's first stages were staged by the previous block
  bool have_q = false;   // this block's Q was loaded by the previous block
  // The next block's stage-2 and stage-3 key scales (and mask bytes), loaded by a block that
  // chains into it.
  float ks_carry[2] = {0.0f, 0.0f};
  uint32_t keep_carry[2] = {0u, 0u};
  uint32_t tab_head = ~0u;  // the key/value head whose scale pairs fill stab
  Tile T;
  if constexpr (kTab) {
    // Every block's Q is loaded before the last barrier of the block before it (the first
    // block's here, waited for at once), so no wait for Q stands in step -1, where it would also
    // wait for the previous block's output stores (vmcnt counts both, in order).
    load_q(T, wave_block(xcd * g.per_xcd + local));
    __builtin_amdgcn_s_waitcnt(kWaitAll);
  }

  for (;;) {
  const uint32_t logical = xcd * g.per_xcd + local;
  const uint32_t next_local = local + g.wpx;
  const bool has_next =
      kChain && next_local < g.per_xcd && xcd * g.per_xcd + next_local < g.total;
  const WaveBlock wb = wave_block(logical);
  const uint32_t kv_head = wb.kv_head, head = wb.head;
  const bool wrap = chain_ok && has_next && kv_head_of(xcd * g.per_xcd + next_local) == kv_head;
  // stage index of a load: past the last stage it is the next block's (chained) or out of range
  auto stage_of = [&](uint32_t st) { return wrap && st >= n_stages ? st - n_stages : st; };

  // ---- prologue: K and scales of stages 0..2, V^T of stages 0 and 1 and the scales of stage 3
  // in flight (unless chained)
  StepLoads L0 = plan_step<kCross, kTm>(g, kv_head, 0, k0s, 0, v0s, 0);
  StepLoads L1 = plan_step<kCross, kTm>(g, kv_head, kKeys, k1s, kKeys, v1s, kKeys);
  StepLoads L2 = plan_step<kCross, kTm>(g, kv_head, 2 * kKeys, k2s, 0, nullptr, 2 * kKeys);
  StepLoads L3 = plan_step<kCross, kTm>(g, kv_head, 0, nullptr, 0, nullptr, stage_of(3) * kKeys);
  if (kTab && kv_head != tab_head) {
    // Every wave is past the previous block's last barrier, after which nothing reads stab; the
    // prologue's barrier below publishes the new pairs.
    for (uint32_t k = threadIdx.x; k < n_stages * kKeys; k += kThreads) {
      const uint32_t m = swap23(k % kKeys);  // the MFMA row of key k % kKeys
      const bool in = k < g.tokens;
      const float ks = in ? g.ks[(size_t)kv_head * g.capacity + k] : 0.0f;
      const bool live = in && g.key_mask[k] != 0;
      float* sc = reinterpret_cast<float*>(stab + (k / kKeys) * kSStage);
      sc[rot(m, 1)] = ks;
      sc[kKeys + rot(m, 2)] = live ? -(kMagic * ks) : -INFINITY;
    }
    tab_head = kv_head;
  }
  if (!chained) {
    issue_k<kCross, kTm, kTab>(L0, sg);
    issue_v<kCross, kTm>(L0, sg);
    issue_k<kCross, kTm, kTab>(L1, sg);
    issue_v<kCross, kTm>(L1, sg);
    issue_k<kCross, kTm, kTab>(L2, sg);
    issue_load<kCross, kTm, kTab>(L3, sg, 0);
  } else {
    L2.ks = ks_carry[0];
    L2.keep = keep_carry[0];
    L3.ks = ks_carry[1];
    L3.keep = keep_carry[1];
  }

  if (!kTab && !have_q) load_q(T, wb);
  T.negm = 1.0e30f;
  T.l = 0.0f;
  zero_all(std::make_integer_sequence<int, 64>{});
  if (!chained) {
    if (!kTab) {
      store_stage_scales<kCross, kFp6>(s0s, sg, L0.ks, L0.keep, 0, g.tokens);
      store_stage_scales<kCross, kFp6>(s1s, sg, L1.ks, L1.keep, kKeys, g.tokens);
    }
    step_barrier<kWaitAll>();
  } else {
    // The first stages landed before the previous block's last barrier; the previous block's
    // output stores stay in flight (only LDS work is waited for).
    step_barrier<kWaitLds>();
  }

  // ---- step -1: QK of key tiles 0 and 1, the probabilities of tile 0; K(3), V(2) and the scales
  // of stage 4 in flight
  StepLoads Lm = plan_step<kCross, kTm>(g, kv_head, stage_of(3) * kKeys, k3s, 2 * kKeys, v2s,
                                   stage_of(4) * kKeys);
  issue_k<kCross, kTm, kTab>(Lm, sg);
  issue_v<kCross, kTm>(Lm, sg);
  Pre pre;
#pragma unroll
  for (int part = 0; part < 4; ++part) prefetch<kFp6>(pre, part, k0s, 0, ss(0, 0), 0, ln);
  sub_step<0, true, false, false, kFp6>(nullptr, nullptr, 0, T, ln, half, magic, pre,
                                  [&](int c, Pre& next) {
    if (c >= 4 && c < 10) prefetch<kFp6>(next, c - 4, k0s, 1, ss(0, 0), 0, ln);
  });
  // The first tile's own path pays where blocks are short (cross-attention's few key tiles);
  // self-attention keeps the general path, whose code measured marginally faster at long
  // sequences. The results are the same bits either way. Tile 0 is the last one of a sequence of
  // at most 32 keys, so it takes the masked path.
  sub_step<1, true, false, true, kFp6, kCross, true>(nullptr, ss(0, 0), 0, T, ln, half, magic, pre,
                                                      [&](int c, Pre& next) {
    if (!kTab && c == 0)
      store_stage_scales<kCross, kFp6>(s2s, sg, L2.ks, L2.keep, 2 * kKeys, g.tokens);
    // with the scales resident, every staging load older than step -1's has landed (the
    // prologue's barrier, or the previous block's last one, waited for them all): LDS work only
    if (c == kBarK) step_barrier<kTab ? kWaitLds : kWaitPrevStep<kCross, kTab>>();
    next_step_reads<kFp6, kBarK>(c, next, k1s, ss(0, 0), ln);
  });
  // Key scales (and mask bytes) in registers until their store: those loaded in step j (stage
  // j+5) wait in hold[j % 2] for step j+2; the prologue's (stage 3) count as step -2's.
  float ks_hold[2] = {L3.ks, Lm.ks};
  uint32_t keep_hold[2] = {L3.keep, Lm.keep};

  // Steady step j (stage j+1 exists), J = j % 4: sub-steps 2j and 2j+1 read K(j+1), V(j) and the
  // scales of tiles 2j+1 (stage j, block 1) and 2j+2 (stage j+1, block 0); the step stages K(j+4)
  // into K(j)'s array and V(j+3) into V(j-1)'s, loads the scale of stage j+5, and stores the
  // scales of stage j+3 (loaded two steps earlier) into S(j-1)'s. Every K and V^T load has three
  // steps to land, every scale two. The step's barrier comes once its last read of K(j+1) and
  // V(j) is issued (chunk kBarK of its second sub-step), after a wait for this wave's loads of
  // two steps before; the reads for the next step's first sub-step follow it. Stages past the
  // last are the next block's first ones when the blocks chain.
  uint32_t j = 0;
  auto steady = [&](auto J_) {
    constexpr int J = decltype(J_)::value;
    StepLoads L = plan_step<kCross, kTm>(g, kv_head, stage_of(j + 4) * kKeys, kr(J),
                                    stage_of(j + 3) * kKeys, vr(J + 3), stage_of(j + 5) * kKeys);
    // one staging load every kLoadGap chunks: the scale first, then K and V^T
    sub_step<0, true, true, true, kFp6, false, kCross, kPfK>(
        vr(J), ss(J, j), 1, T, ln, half, magic, pre, [&](int c, Pre& next) {
      if (c == 0) prio_late_waves_first(wave);
      if (!kTab && c == 0)
        store_stage_scales<kCross, kFp6>(sr(J + 3), sg, ks_hold[J & 1], keep_hold[J & 1],
                                         stage_of(j + 3) * kKeys, g.tokens);
      if (c % kLoadGap == 0 && c / kLoadGap < kLoadsPerStep)
        issue_load<kCross, kTm, kTab>(L, sg, c / kLoadGap);
      if (c >= 4 && c < 10) prefetch<kFp6>(next, c - 4, kr(J + 1), 1, ss(J + 1, j + 1), 0, ln);
    });
    auto stage1 = [&](int c, Pre& next) {
      if (c == 0) prio_equal();
      const int slot = (c + 12) / kLoadGap;
      if ((c + 12) % kLoadGap == 0 && slot < kLoadsPerStep)
        issue_load<kCross, kTm, kTab>(L, sg, slot);
      if (c == kBarK) step_barrier<kWaitTwoSteps<kCross, kTab>>();
      next_step_reads<kFp6, kBarK>(c, next, kr(J + 2), ss(J + 1, j + 1), ln);
    };
    // Tile 2j+2 (keys 64(j+1) ..) holds keys past the sequence in the last steady step when the
    // sequence ends inside its 32 keys: this sub-step always takes the masked path. (A branch
    // between the two paths here puts register copies at its join that the inline-assembly
    // MFMAs after it may read before they land, which the compiler does not guard against.)
    sub_step<1, true, true, true, kFp6, false, true, kPfK>(vr(J), ss(J + 1, j + 1), 0, T, ln, half,
                                                           magic, pre, stage1);
    ks_hold[J & 1] = L.ks;
    keep_hold[J & 1] = L.keep;
    ++j;
  };
  const uint32_t n_steady = n_stages - 1;  // steps j with stage j+1
  for (uint32_t quads = n_steady / 4; quads > 0; --quads) {
    steady(std::integral_constant<int, 0>{});
    steady(std::integral_constant<int, 1>{});
    steady(std::integral_constant<int, 2>{});
    steady(std::integral_constant<int, 3>{});
  }
  const uint32_t rest = n_steady % 4;
  if (rest > 0) steady(std::integral_constant<int, 0>{});
  if (rest > 1) steady(std::integral_constant<int, 1>{});
  if (rest > 2) steady(std::integral_constant<int, 2>{});

  // ---- last step (j = n_stages - 1): PV of tiles 2j and 2j+1, the probabilities of 2j+1 between
  // (its scales came in `pre`; its K reads there are unused). Tile 2j+1 may hold keys past the
  // sequence: the masked path. With the scales resident, the next block's Q codes are loaded
  // first (no QK is left in this block), so that this step's last barrier covers them.
  float qs_next = 0.0f;
  if (kTab && has_next) qs_next = load_q_codes(T, wave_block(xcd * g.per_xcd + next_local));
  sub_step<0, false, true, true, kFp6, false, true, kPfK>(vr(j), ss(j, j), 1, T, ln, half, magic,
                                                          pre, [](int, Pre&) {});
  sub_step<1, false, true, false, kFp6, false, false, kPfK>(vr(j), nullptr, 0, T, ln, half,
                                                            magic, pre, [](int, Pre&) {});
  step_barrier<kWaitAll>();  // no staging load outlives the block (chained ones have landed)
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");  // the last PV MFMAs have landed

  // The next block's Q, loaded now (this block's QK is done) so that it lands during the
  // epilogue and ahead of the stores below.
  const float l_here = T.l;
  if (kTab && has_next) set_q_scale(T, qs_next);
  if (!kTab && has_next) load_q(T, wave_block(xcd * g.per_xcd + next_local));

  // ---- normalise and store rows < min(token_count, tokens). O^T gives each lane one query and
  // 8-byte pieces of its channels, so the rows are first transposed through the wave's LDS stage
  // (64 channels at a time, 16-byte chunks XOR-swizzled by row % 8): each store then writes 128
  // contiguous bytes of eight rows instead of 16 bytes of 32 rows. The stores go through a buffer
  // descriptor that ends at the last valid row of the wave's tile (the hardware drops stores past
  // it), so they are the same instructions for every wave and nothing waits for them.
  {
    float o[64];
    read_all(o, std::make_integer_sequence<int, 64>{});
    const float l_tot = l_here + __shfl_xor(l_here, 32);
    const float inv = 1.0f / l_tot;
    const uint32_t live = g.rows > wb.q0 ? min(g.rows - wb.q0, (uint32_t)kTileQ) : 0u;
    const __amdgpu_buffer_rsrc_t ro =
        rsrc(g.out + (size_t)wb.q0 * g.out_stride, live * g.out_stride * 2);
    // The stage: a quarter of V^T stage 2 or 3. Neither holds anything live between the last
    // step's barrier (after which no wave reads them) and the next block's first barrier (before
    // which nothing is staged into them; a chained block's early stages are K 0-2 and V^T 0-1).
    char* ow = (wave < 4 ? v2s : v3s) + (wave & 3) * kOStage;
    const uint32_t sr = lane >> 3, sj = lane & 7;  // store: rows 8k + sr, chunk sj
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
#pragma unroll
      for (int dbl = 0; dbl < 2; ++dbl) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float* r = o + 16 * (2 * pass + dbl) + 4 * i;
          const v4h h = {(_Float16)(r[0] * inv), (_Float16)(r[1] * inv), (_Float16)(r[2] * inv),
                         (_Float16)(r[3] * inv)};
          const int chunk = 4 * dbl + i;  // channel 64 pass + 8 chunk + 4 half
          *reinterpret_cast<v4h*>(ow + n * 128 + 16 * (chunk ^ (n & 7)) + 8 * half) = h;
        }
      }
      __builtin_amdgcn_s_waitcnt(kWaitLdsWrites);  // this wave's pieces are in the stage
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t row = 8 * k + sr;
        const v4u v = *reinterpret_cast<const v4u*>(ow + row * 128 + 16 * (sj ^ (row & 7)));
        // non-temporal (cache policy nt): the output streams past L2, which it could not stay
        // in anyway, and a chained block's next waits on the shared vmcnt find the burst done
        // sooner (cross-attention at config 4: 1.040-1.045 ms against 1.051-1.059 ms)
        __builtin_amdgcn_raw_buffer_store_b128(
            v, ro, (row * g.out_stride + head * 128 + 64 * pass + 8 * sj) * 2, 0, kCpolNt);
      }
      __builtin_amdgcn_s_waitcnt(kWaitLdsWrites);  // the stage is read before it is rewritten
      __builtin_amdgcn_wave_barrier();
    }
  }
  if (!has_next) break;
  have_q = true;
  chained = wrap;
  // after the last steady step (j - 1): hold[j % 2] holds stage n_stages + 2, the other
  // n_stages + 3, i.e. the next block's stages 2 and 3 when it chains
  ks_carry[0] = (j & 1) ? ks_hold[1] : ks_hold[0];
  ks_carry[1] = (j & 1) ? ks_hold[0] : ks_hold[1];
  keep_carry[0] = (j & 1) ? keep_hold[1] : keep_hold[0];
  keep_carry[1] = (j & 1) ? keep_hold[0] : keep_hold[1];
  local = next_local;
  }
}

// Short key sequences (at most kPersistMaxStages 64-key stages) run one persistent workgroup per
// CU that chains its blocks, since their per-block fill and drain is a large share of a block;
// long ones run one workgroup per block (the loop compiled out), so that the hardware's dispatch
// hands blocks to whichever CU is free. At 129,024 keys the chaining build was 5-6 % slower, from
// a static split of the blocks over CUs that run at different speeds and from the extra
// per-step work of the stage wrap.
constexpr uint32_t kPersistMaxStages = kTabStages;
bool chain_blocks(const Geometry& g) {
  return (g.tokens + kKeys - 1) / kKeys <= kPersistMaxStages;
}
uint32_t workgroups_per_xcd(const Geometry& g) {
  if (!chain_blocks(g)) return g.per_xcd;
  return std::min(g.per_xcd, std::max(1u, device_cus() / 8));  // one workgroup per CU
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
  g.wpx = workgroups_per_xcd(g);
  if (chain_blocks(g))
    hipLaunchKernelGGL((k_attention_hm<false, true>), dim3(g.wpx * 8), dim3(kThreads), 0, stream, g);
  else
    hipLaunchKernelGGL((k_attention_hm<false, false>), dim3(g.wpx * 8), dim3(kThreads), 0, stream, g);
  return hipGetLastError();
}

// attention_i8qk_family's token-major operands on this kernel: Q and K codes [token][stride],
// query scales [token][q_stride / 128], key scales [token][kv_stride / 128] or, when
// `ks_head_major`, the lent head-major copy [kv_head][tokens]; V^T and the output as above.
hipError_t launch_attention_hm_tm(const h3_attention_cfg& cfg, uint32_t token_count,
                                  uint32_t heads, const int32_t* qi, const float* qs,
                                  const int32_t* ki, const float* ks, bool ks_head_major,
                                  const uint16_t* vt, uint16_t* out, hipStream_t stream) {
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
  g.k_row = cfg.kv_stride;
  g.q_row = cfg.q_stride;
  g.qs_row = cfg.q_stride / 128;
  g.ks_key = ks_head_major ? 1u : g.kv_head_limit;
  g.ks_head = ks_head_major ? cfg.tokens : 1u;
  g.total = g.q_blocks * heads;
  g.per_xcd = (g.total + 7) / 8;
  g.wpx = g.per_xcd;  // one workgroup per block at every length (the chained form would spill)
  hipLaunchKernelGGL((k_attention_hm<false, false, false, true>), dim3(g.wpx * 8), dim3(kThreads),
                     0, stream, g);
  return hipGetLastError();
}

hipError_t launch_attention_hm_fp6(const h3_attention_cfg& cfg, uint32_t token_count,
                                   uint32_t heads, const void* qf, const float* qs, const void* kf,
                                   const float* ks, const uint16_t* vt, uint16_t* out,
                                   hipStream_t stream) {
  Geometry g{};
  g.qi = static_cast<const int32_t*>(qf);
  g.qs = qs;
  g.ki = static_cast<const int32_t*>(kf);
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
  g.wpx = workgroups_per_xcd(g);
  if (chain_blocks(g))
    hipLaunchKernelGGL((k_attention_hm<false, true, true>), dim3(g.wpx * 8), dim3(kThreads), 0,
                       stream, g);
  else
    hipLaunchKernelGGL((k_attention_hm<false, false, true>), dim3(g.wpx * 8), dim3(kThreads), 0,
                       stream, g);
  return hipGetLastError();
}

hipError_t launch_attention_hm_cross(const h3_cross_cfg& cfg, const int32_t* qi, const float* qs,
                                     const int32_t* ki, const float* ks, const uint16_t* vt,
                                     const uint8_t* key_mask, uint16_t* out, hipStream_t stream) {
  Geometry g{};
  g.qi = qi;
  g.qs = qs;
  g.ki = ki;
  g.ks = ks;
  g.vt = vt;
  g.out = out;
  g.tokens = cfg.kv_tokens;
  g.rows = cfg.q_tokens;
  g.capacity = cfg.kv_capacity;
  g.out_stride = cfg.out_stride;
  g.key_mask = key_mask;
  g.q_tokens = cfg.q_tokens;
  g.q_capacity = cfg.q_capacity;
  g.kv_group = cfg.q_heads / cfg.kv_heads;
  g.waves_per_head = kWaves / g.kv_group;
  const uint32_t per_block = g.waves_per_head * kTileQ;  // queries of each head per block
  g.q_blocks = (cfg.q_tokens + per_block - 1) / per_block;
  g.kv_head_limit = cfg.kv_heads;
  g.head_limit = cfg.q_heads;
  g.total = g.q_blocks * cfg.kv_heads;
  g.per_xcd = (g.total + 7) / 8;
  g.wpx = workgroups_per_xcd(g);
  if (chain_blocks(g))
    hipLaunchKernelGGL((k_attention_hm<true, true>), dim3(g.wpx * 8), dim3(kThreads), 0, stream, g);
  else
    hipLaunchKernelGGL((k_attention_hm<true, false>), dim3(g.wpx * 8), dim3(kThreads), 0, stream, g);
  return hipGetLastError();
}

}  // namespace h3
