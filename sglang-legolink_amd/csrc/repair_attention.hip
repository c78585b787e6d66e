// Sparse repair attention on gfx950 (MI355X): the repair pass's attention of
// repair rows over the linked KV, read through each request's slot list.
//
// Work decomposition (planned on the host by ll_repair_attention_plan):
//   The 16-query tiles of one request (consecutive repair rows) form a run;
//   G query heads share one KV head, so a run of n tiles has n * G (query
//   tile, query head) pairs, numbered tile-major: pair f is tile f / G, query
//   head f % G of the KV head.  The run's pairs are cut into windows of 16
//   consecutive pairs (the last may be shorter), so a window may start or end
//   inside a tile: with G = 7, windows of 16 pairs keep every wave busy where
//   whole tiles (2 x 7 = 14 pairs) would leave one of eight waves idle.
//   item = one window (its tiles, at most 16, and its first pair's head) and
//   a KV range [kv_begin, kv_end) of logical positions; long ranges are
//   split and the partial results merged by a combine pass.
//   workgroup = (item, KV head); the window's pairs are spread over its
//   waves, so each K/V tile staged in LDS serves every pair of the window.
//   A workgroup holds P = 16 pairs (8 for head dim 256, whose windows take
//   two workgroups per KV head).
//
// Per 64-token KV tile:
//   1. gather the tile's K and V rows of this KV head into LDS by slot;
//   2. S^T = K Q^T on MFMAs: A = K rows from LDS, B = the queries (kept in
//      registers);
//   3. masking (causal by logical position, split range, invalid slots),
//      online softmax in fp32 with exp2 (row statistics reduced across the
//      lanes of a query with permlane swaps);
//   4. O^T += V^T P^T: B = the probabilities straight from the S^T
//      accumulators (the token order inside the K step is free, as long as
//      A uses the same one), A = V^T from transposed LDS reads.
//
// Every head dim (64, 128, 256) runs repair_attention_m32_kernel: two pairs
// per wave on v_mfma_f32_32x32x16, rows gathered into an LDS ring by
// LDS-DMA loads (buffer_load ... lds with 32-bit row offsets where the pool
// fits them, else global_load_lds).
//
// Roofline: MFMA-bound in principle.  Algorithmic work per (query, visible
// key) pair and query head: 4 * head_dim flops (QK and PV); KV bytes are read
// once per item and KV head.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <functional>
#include <mutex>
#include <type_traits>
#include <vector>

#include "legolink_kv.h"
#include "ll_internal.h"

namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) short i16x4;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2;

constexpr int kWave = 64;
constexpr int kQueries = 16;  // queries per item: one MFMA column tile
constexpr int kTile = 64;     // KV tokens per LDS tile
constexpr int kMaxPairs = 16;  // (query tile, query head) pairs per window (and per workgroup at head dims 64, 128)
// 16-query tiles a window touches: 16 for one query head per KV head (MHA),
// at most 9 for larger groups.
constexpr int kMaxTiles = 16;
// kv_offset, kv_begin, kv_end, tiles, the window's first pair (its head in
// the first tile, 0 .. G - 1) and its pair count (1 .. 16), then per tile
// (first query, lowest position, query count (0: absent), partial slot (-1:
// none), key end).
constexpr int kItemHeader = 6;
constexpr int kTileInts = 5;
constexpr int kItemInts = kItemHeader + kTileInts * kMaxTiles;  // 86
constexpr int kCombineInts = 4;

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  const int rc = ll_record_error(code, fmt, ap);
  va_end(ap);
  return rc;
}

struct AttnParams {
  const uint16_t *q;
  uint16_t *out;
  const uint16_t *k;
  const uint16_t *v;
  const void *slots;
  const int *items;
  const int *combine;
  const int *positions;  // logical position of every query
  float *ws;
  long long num_queries;
  long long num_slots;
  long long slots_len;
  long long ws_items;
  int hq;
  int hkv;
  int group;
  int pair_chunks;   // workgroups per (item, KV head): 16 / (pairs per workgroup)
  int slots64;
  unsigned pool_bytes;  // bytes of the K (and of the V) buffer, when they fit 32-bit offsets; else 0
  float scale_log2;
};

// The 16-bit element types of queries, keys, values and outputs: the MFMA
// that takes them (fp32 accumulation) and the rounding of fp32 results back
// to them (two at a time, round to nearest even).
struct Bf16 {
  typedef bf16x8 frag;
  static constexpr uint32_t kOnes = 0x3F803F80u;  // two 1.0s
  __device__ static uint32_t pack(float lo, float hi) {  // one v_cvt_pk_bf16_f32
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
  }
  __device__ static f32x16 mfma32(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  __device__ static float dot2_ones(uint32_t pair, float acc) {  // acc + lo + hi, one v_dot2_f32_bf16
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pair), __builtin_bit_cast(bf16x2, kOnes),
                                           acc, false);
  }
  __device__ static f32x2 unpack(uint32_t pair) {  // exact
    return f32x2{__uint_as_float(pair << 16), __uint_as_float(pair & 0xffff0000u)};
  }
};

struct F16 {
  typedef f16x8 frag;
  static constexpr uint32_t kOnes = 0x3C003C00u;
  __device__ static uint32_t pack(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, f16x2));
  }
  __device__ static f32x16 mfma32(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  __device__ static float dot2_ones(uint32_t pair, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, pair), __builtin_bit_cast(f16x2, kOnes), acc, false);
  }
  __device__ static f32x2 unpack(uint32_t pair) {  // exact
    return __builtin_convertvector(__builtin_bit_cast(f16x2, pair), f32x2);
  }
};

__device__ inline long long slot_at(const AttnParams &p, long long i) {
  return p.slots64 ? static_cast<const long long *>(p.slots)[i]
                   : static_cast<long long>(static_cast<const int *>(p.slots)[i]);
}

// Partial result of item `partial`, query head h: the 16 queries' outputs
// over the item's keys, normalised by their own sums (O / l) and rounded to
// the KV dtype, [16][D] 16-bit values, then (m, l) [16][2] in fp32: 8 D + 32
// floats.  Rounding O / l adds at most 2^-9 of the softmax-weighted |V| to
// the merged output (a convex combination of the partials), half of what
// rounding the probabilities to the KV dtype already allows.
template <int D>
__host__ __device__ constexpr int partial_floats() { return kQueries * D / 2 + 2 * kQueries; }
template <int D>
__device__ inline float *partial_block(const AttnParams &p, int partial, int h) {
  return p.ws + (static_cast<long long>(partial) * p.hq + h) * partial_floats<D>();
}

// v_permlane32_swap a, b exchanges the upper half of a with the lower half of
// b: from two copies of x it leaves (x[l], x[l ^ 32]) in the lane, up to
// order -- the operands of an xor shuffle 32.  (Inline assembly: the compiler
// builtin loses the second result when both operands hold the same value.)
// The s_nop covers the wait states between a VALU write of an operand and the
// permute.
__device__ inline void permlane32_swap(unsigned &a, unsigned &b) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}

// v_max_f32 straight from assembly: fmaxf would first quiet its operands
// (which come out of inline assembly) with two more instructions.  Scores
// reaching here are never NaN (masked ones are -inf).
__device__ inline float max_f32(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

constexpr float kSlack = 8.f;  // log2 headroom of the lazily updated softmax maximum
constexpr float kScoreFloor = -1e30f;  // initial softmax maximum (raw score units)

// (Query tile, query head) pairs per workgroup, two per wave: head dim 256
// needs twice the registers and LDS per wave, so its workgroups hold 4 waves.
__host__ __device__ constexpr int max_pairs(int d) { return d == 256 ? kMaxPairs / 2 : kMaxPairs; }

// K and V rows are gathered straight into an LDS ring with LDS-DMA loads,
// up to three tiles ahead of the MFMAs, so no registers stage them.  Rows are
// stored token-major with their 16-byte chunks XOR-swizzled by token, which keeps the fragment reads free of bank conflicts.  V^T
// fragments come from ds_read_b64_tr_b16: within a group of 16 lanes it
// returns to lane i, element e, element i % 4 of the 8 bytes that lane
// 4 e + i / 4 addressed (checked on the device), so lanes addressing 4 dims of
// 4 tokens receive 4 tokens of one dim -- the MFMA's A layout.  The item's
// slots are read into LDS kDmaMaxRange at a time.
constexpr int kDmaStages = 4;
// KV tokens per slot-list refill: the slots fill the LDS the ring leaves (the
// 4 x 32 KB ring at head dims 128 and 256, 159 KB in all).
constexpr int kDmaMaxRange = 7680;
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// Two 16-byte-per-lane gathers into LDS (global_load_lds_dwordx4: lane l's
// bytes land at the LDS base in M0 + 16 l).  They are issued from inline
// assembly so that the compiler, which cannot tell the ring's stages apart,
// does not add waits for every outstanding gather before each LDS access:
// the loop below orders the stages itself with explicit vmcnt waits and
// barriers.  M0 is saved and restored around them.
__device__ inline void dma_pair(const void *src0, void *lds0, const void *src1, void *lds1) {
  const unsigned base0 = __builtin_amdgcn_readfirstlane(
      static_cast<unsigned>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) void *)lds0)));
  const unsigned base1 = __builtin_amdgcn_readfirstlane(
      static_cast<unsigned>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) void *)lds1)));
  unsigned saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off\n\t"
      "s_mov_b32 m0, %4\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %2, off\n\t"
      "s_nop 0\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(src0), "v"(src1), "s"(base0), "s"(base1)
      : "memory");
}

// The same with 32-bit byte offsets into the K and V buffers (buffer loads:
// one multiply-add per address instead of 64-bit address arithmetic), for
// pools whose K and V buffers each fit in 4 GiB.  The resources hold the
// buffer's base and size (loads past it would read zeros; the offsets used
// stay inside).
typedef int i32x4r __attribute__((ext_vector_type(4)));
__device__ inline i32x4r buffer_resource(const void *base, unsigned bytes) {
  const unsigned long long address = reinterpret_cast<unsigned long long>(base);
  i32x4r r;
  r[0] = static_cast<int>(static_cast<unsigned>(address));
  r[1] = static_cast<int>(static_cast<unsigned>(address >> 32) & 0xffffu);  // stride 0
  r[2] = static_cast<int>(bytes);
  r[3] = 0x00020000;  // raw 32-bit dwords
  return r;
}

__device__ inline void dma_pair_buffer(unsigned off0, void *lds0, i32x4r res0, unsigned off1, void *lds1,
                                       i32x4r res1) {
  const unsigned base0 = __builtin_amdgcn_readfirstlane(
      static_cast<unsigned>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) void *)lds0)));
  const unsigned base1 = __builtin_amdgcn_readfirstlane(
      static_cast<unsigned>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) void *)lds1)));
  unsigned saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %1, %5, 0 offen lds\n\t"
      "s_mov_b32 m0, %4\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %2, %6, 0 offen lds\n\t"
      "s_nop 0\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(off0), "v"(off1), "s"(base0), "s"(base1), "s"(res0), "s"(res1)
      : "memory");
}

// s_barrier without __syncthreads()'s wait for all outstanding memory
// operations (which would drain the gathers in flight); the empty asm keeps
// the compiler from moving LDS accesses across it.
__device__ inline void workgroup_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}


// Attention on v_mfma_f32_32x32x16 (issues at ~34 cycles for twice the work
// of a 16x16x32 at ~20, and hides about four VALU instructions in the wave
// that issued it, against two).  Each wave owns two (query tile, head) pairs,
// 32 MFMA columns: column n = 16 (pair - 2 wave) + query.  Lane layouts
// (checked on the device with integer matrices): A and B lane l element e ->
// row / column l % 32, k = 8 (l / 32) + e; accumulator register r -> row
// 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32.
//   S^T = K Q^T per 32-token block: A = K rows from LDS (token l % 32, dims
//   16 ks + 8 (l / 32) + e: one 16-byte chunk), B = the lane's query (held).
//   O^T += V^T P^T per 16-token step s of a block: B = accumulator registers
//   8 s .. 8 s + 7 rounded in place, which puts token 16 s + 8 (e / 4) +
//   4 (l / 32) + e % 4 at k = 8 (l / 32) + e; A = V^T through two transposed
//   reads giving each lane one dim of that token order.
// Each lane sums its bf16/fp16 probabilities with v_dot2 against ones (the
// values the value product sees); the two lanes of a column add at the end.
// Chunk swizzles (chunk c of token t is stored at c ^ swizzle(t)), chosen so
// that the 16 lanes of a K read (16 tokens, one chunk each) and the 32 lanes
// of a transposed V read (4 tokens x 64 bytes) each cover the 64 banks once:
//   head dims 128 and 256 (256- and 512-byte rows, each starting a bank
//   row): K c ^ (t % 16), V c ^ 4 (t % 4);
//   head dim 64 (128-byte rows, two per bank row): K c ^ ((t / 2) % 8),
//   V c ^ 4 ((t / 2) % 2).
// Each wave issues an equal share of a tile's K and V gathers, during the
// tile kLead earlier, after that tile's score batch w % 4 (so that the
// workgroup's loads do not all queue at once).
// Head dims 64 and 128: 8 waves and a four-stage ring; head dim 256 (twice the
// registers and LDS per tile): 4 waves, one per SIMD, and a two-stage ring.
template <int D>
__host__ __device__ constexpr int m32_threads() { return D == 256 ? 256 : 512; }
template <int D>
__host__ __device__ constexpr int m32_stages() { return D == 256 ? 2 : kDmaStages; }

template <int D>
__host__ __device__ constexpr int m32_k_swizzle(int t) { return D >= 128 ? t % 16 : (t / 2) % 8; }
template <int D>
__host__ __device__ constexpr int m32_v_swizzle(int t) { return D >= 128 ? 4 * (t % 4) : 4 * ((t / 2) % 2); }

template <int D, typename E, bool kOffsets>
__global__ void __launch_bounds__(m32_threads<D>()) repair_attention_m32_kernel(const AttnParams p) {
  typedef typename E::frag frag;
  static_assert(D == 64 || D == 128 || D == 256, "head dims 64, 128 and 256");
  constexpr int kM32Threads = m32_threads<D>();
  constexpr int kStages = m32_stages<D>();
  constexpr int kLead = kStages - 1;  // tiles gathered ahead of the one computed
  constexpr int kKSteps = D / 16;                        // 16-dim steps of the score MFMAs
  constexpr int kDimBlocks = D / 32;                     // 32-dim blocks of O^T
  constexpr int kChunksPerRow = D / 8;                   // 16-byte chunks per row
  constexpr int kGathers = kChunksPerRow / (kM32Threads / kWave);  // per wave, per tile, of K and of V
  constexpr int kRowBytes = D * 2;
  constexpr int kStageBytes = kTile * kRowBytes;         // one K or V tile
  constexpr int kRangeTiles = kDmaMaxRange / kTile;
  static_assert(kM32Threads / kWave * 2 == max_pairs(D), "two (tile, head) pairs per wave");
  __shared__ __attribute__((aligned(16))) unsigned char k_ring[kStages * kStageBytes];
  __shared__ __attribute__((aligned(16))) unsigned char v_ring[kStages * kStageBytes];
  __shared__ int slot_lds[kDmaMaxRange];
  __shared__ unsigned long long tile_valid[kRangeTiles];

  constexpr int kPairs = max_pairs(D);
  const int *it = p.items + static_cast<long long>(blockIdx.x) * kItemInts;
  const int kv_off = it[0], kv_begin = it[1], kv_end = it[2], n_tiles = it[3];
  const int pair_first = it[4], pair_count = it[5];
  // blockIdx.y = (KV head, pair chunk): this workgroup's pairs of the window
  // are [wg_first, wg_end), counted from the item's first tile.
  const int hk = blockIdx.y / p.pair_chunks;
  const int wg_first = pair_first + static_cast<int>(blockIdx.y % p.pair_chunks) * kPairs;
  const int wg_end = min(pair_first + pair_count, wg_first + kPairs);
  if (n_tiles < 1 || n_tiles > kMaxTiles || kv_off < 0 || kv_begin < 0 || kv_begin > kv_end ||
      static_cast<long long>(kv_off) + kv_end > p.slots_len ||
      hk >= p.hkv || pair_first < 0 || pair_first >= p.group || pair_count < 1 || pair_count > kMaxPairs ||
      wg_first >= wg_end || (wg_end - 1) / p.group >= n_tiles)
    return;

  const int tid = threadIdx.x;
  // Wave-uniform values are made visibly uniform (readfirstlane), so that
  // branches on them are scalar branches: otherwise the compiler evaluates
  // both sides of the per-tile mask branch below on every tile.
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int lane = tid % kWave;
  const int h = lane / 32;   // k half of the A/B operands, row group of the accumulators
  const int col = lane % 32;  // MFMA column of this lane
  const int qc = col % 16;    // query within the column's pair

  // The wave's two pairs; a pair computes when its tile and head exist and its
  // table entry is sane.
  struct PairInfo {
    bool computes;
    int q_index, q_pos, q_count, partial, stop, hq;
  };
  auto pair_info = [&](int pair) {
    PairInfo r;
    const int flat = wg_first + pair;  // pair index in the window's tiles
    const int tile = flat / p.group;
    const int head = flat - tile * p.group;
    const bool in_window = flat < wg_end;  // and so tile < n_tiles (checked above)
    const int *e = it + kItemHeader + kTileInts * (in_window ? tile : 0);
    r.q_index = e[0];
    r.q_pos = e[1];
    r.q_count = e[2];
    r.partial = e[3];
    const int needed = e[4];
    r.hq = hk * p.group + head;
    r.computes = in_window && r.q_count >= 1 && r.q_count <= kQueries && r.q_index >= 0 &&
                 static_cast<long long>(r.q_index) + r.q_count <= p.num_queries && r.q_pos >= 0 &&
                 needed > r.q_pos && (r.partial == -1 || (r.partial >= 0 && r.partial < p.ws_items));
    r.stop = r.computes ? min(kv_end, needed) : kv_begin;
    return r;
  };
  const PairInfo pair0 = pair_info(2 * wave), pair1 = pair_info(2 * wave + 1);
  const PairInfo &mine = col < 16 ? pair0 : pair1;
  const bool wave_computes = pair0.computes || pair1.computes;
  const int wave_stop = max(pair0.stop, pair1.stop);
  // Keys below both pairs' lowest query position and stop need no causal mask.
  int wave_unmasked = kv_end;
  if (pair0.computes) wave_unmasked = min(wave_unmasked, min(pair0.q_pos, pair0.stop));
  if (pair1.computes) wave_unmasked = min(wave_unmasked, min(pair1.q_pos, pair1.stop));
  const bool q_ok = mine.computes && qc < mine.q_count;
  const int my_pos = q_ok ? p.positions[mine.q_index + qc] : 0;
  const int my_stop = mine.stop;

  // Keys this workgroup's tiles need.
  int load_stop = kv_begin;
  for (int t = wg_first / p.group; t <= (wg_end - 1) / p.group; ++t) {
    const int *e = it + kItemHeader + kTileInts * t;
    if (e[2] >= 1) load_stop = max(load_stop, min(kv_end, e[4]));
  }
  // B operand of the score MFMAs: the lane's query, dims 16 ks + 8 h .. + 7.
  frag qf[kKSteps];
  {
    const uint16_t *qrow = p.q + (static_cast<long long>(mine.q_index + qc) * p.hq + mine.hq) * D + 8 * h;
#pragma unroll
    for (int ks = 0; ks < kKSteps; ++ks) {
      u32x4 bits = {0u, 0u, 0u, 0u};
      if (q_ok) bits = *reinterpret_cast<const u32x4 *>(qrow + 16 * ks);
      qf[ks] = __builtin_bit_cast(frag, bits);
    }
  }

  // Gather of tile t: D / 8 K and D / 8 V instructions of 64 lanes; wave w
  // issues instructions kGathers w .. kGathers w + kGathers - 1 of each.
  // Instruction k fills stage chunks 64 k .. 64 k + 63: chunk P holds token
  // P / kChunksPerRow and, of its row, chunk (P % kChunksPerRow) ^
  // swizzle(token) (each swizzle is its own inverse).
  const long long row_stride = static_cast<long long>(p.hkv) * D;
  const bool have_slots = p.num_slots > 0;
  int g_token[kGathers], g_kchunk[kGathers], g_vchunk[kGathers];
  unsigned g_koff[kGathers], g_voff[kGathers];  // kOffsets: the lane's bytes within a token's row
#pragma unroll
  for (int j = 0; j < kGathers; ++j) {
    const int chunk_index = (kGathers * wave + j) * kWave + lane;
    g_token[j] = chunk_index / kChunksPerRow;
    g_kchunk[j] = (chunk_index % kChunksPerRow) ^ m32_k_swizzle<D>(g_token[j]);
    g_vchunk[j] = (chunk_index % kChunksPerRow) ^ m32_v_swizzle<D>(g_token[j]);
    g_koff[j] = static_cast<unsigned>(hk * D * 2 + g_kchunk[j] * 16);
    g_voff[j] = static_cast<unsigned>(hk * D * 2 + g_vchunk[j] * 16);
  }
  const i32x4r k_res = buffer_resource(p.k, p.pool_bytes);
  const i32x4r v_res = buffer_resource(p.v, p.pool_bytes);
  auto gather_slots = [&](int t, int *slots) {
#pragma unroll
    for (int j = 0; j < kGathers; ++j) slots[j] = slot_lds[t * kTile + g_token[j]];
  };
  // The slot list holds slots, or with kOffsets the byte offset of each
  // token's row (row 0 for a token without a valid slot).
  auto gather_from = [&](const int *slots, unsigned char *k_dst, unsigned char *v_dst) {
    if (!have_slots) return;
#pragma unroll
    for (int j = 0; j < kGathers; ++j) {
      const int offset = (kGathers * wave + j) * kWave * 16;
      if constexpr (kOffsets) {
        const unsigned row = static_cast<unsigned>(slots[j]);
        dma_pair_buffer(row + g_koff[j], k_dst + offset, k_res, row + g_voff[j], v_dst + offset, v_res);
      } else {
        const int slot = max(slots[j], 0);
        const long long row = slot * row_stride + hk * D;
        dma_pair(p.k + row + g_kchunk[j] * 8, k_dst + offset, p.v + row + g_vchunk[j] * 8, v_dst + offset);
      }
    }
  };
  auto gather = [&](int t, unsigned char *k_dst, unsigned char *v_dst) {
    int slots[kGathers];
    gather_slots(t, slots);
    gather_from(slots, k_dst, v_dst);
  };

  float m = kScoreFloor;
  float l = 0.f;
  f32x16 o[kDimBlocks];
#pragma unroll
  for (int b = 0; b < kDimBlocks; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[b][r] = 0.f;
  const float scale_log2 = p.scale_log2;
  const float slack = kSlack / scale_log2;

  // Per-lane LDS offsets.  K: token col of a 32-token block, chunk
  // (2 ks + h) ^ (col % 16).  V (transposed reads): lane i of 16-lane group q
  // addresses token 4 h + i / 4 (+ the step's base) and the 8 bytes of dims
  // 32 b + 16 (q % 2) + 4 (i % 4); that dim chunk sits at chunk position
  // (4 b + 2 (q % 2) + (i % 4) / 2) ^ 4 (i / 4) = 4 (b ^ (i / 4)) + ...
  const int li = lane % 16;
  const int vu = li / 4;
  const int v_lane = (4 * h + vu) * kRowBytes + (2 * ((lane / 16) % 2) + (li % 4) / 2) * 16 + 8 * (li % 2);
  const int k_lane = col * kRowBytes;
  // The lane's byte offsets within a stage: K per 16-dim step ks (its
  // swizzled chunk), V per 32-dim block b.  Kept in registers (the empty asm
  // stops the compiler from recomputing them per tile), so that with the
  // stage a constant every fragment read is one register plus an immediate.
  int k_off[kKSteps];
#pragma unroll
  for (int ks = 0; ks < kKSteps; ++ks) {
    k_off[ks] = k_lane + ((2 * ks + h) ^ m32_k_swizzle<D>(col)) * 16;
    asm volatile("" : "+v"(k_off[ks]));
  }
  // V offsets carry the V ring's LDS address (beyond the 16-bit immediate
  // of the reads), so that the stage and step offsets stay immediates.
  const unsigned v_ring_lds =
      static_cast<unsigned>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) unsigned char *)v_ring));
  unsigned v_off[kDimBlocks];
#pragma unroll
  for (int b = 0; b < kDimBlocks; ++b) {
    v_off[b] = v_ring_lds + v_lane + ((b ^ (m32_v_swizzle<D>(vu) / 4)) << 6);
    asm volatile("" : "+v"(v_off[b]));
  }

  // Tiles are gathered kLead ahead: tile t + kLead goes into the stage of
  // tile t - 1 once every wave is past it (the barrier at the top of tile t).
  // A wave's 2 kGathers loads of tile t are complete when at most those of
  // tiles t + 1 .. t + kLead - 1 are outstanding (loads count down in issue
  // order).
  // The keys go in chunks of at most kDmaMaxRange, the slot list's capacity:
  // per chunk the slot list is refilled (the ring drained at the chunk's end
  // and restarted), while the softmax state carries over, so one workgroup
  // takes a key range of any length.
  for (int chunk_begin = kv_begin; chunk_begin < load_stop; chunk_begin += kDmaMaxRange) {
  const int range = min(load_stop - chunk_begin, kDmaMaxRange);
  const int tiles = (range + kTile - 1) / kTile;
  if (chunk_begin != kv_begin) __syncthreads();  // every wave is done with the previous chunk's slots and stages
  // Each wave takes whole 64-token tiles (the workgroup is a whole number of
  // waves), so a tile's valid-slot bits are one ballot.
  for (int i = tid; i < tiles * kTile; i += kM32Threads) {
    int slot = -1;
    if (i < range) {
      const long long s = slot_at(p, static_cast<long long>(kv_off) + chunk_begin + i);
      if (s >= 0 && s < p.num_slots) slot = static_cast<int>(s);
    }
    if constexpr (kOffsets)
      slot_lds[i] = static_cast<int>(static_cast<unsigned>(slot >= 0 ? slot : 0) * static_cast<unsigned>(2 * row_stride));
    else
      slot_lds[i] = slot;
    const unsigned long long bits = __builtin_amdgcn_ballot_w64(slot >= 0);
    if (lane == 0) tile_valid[i / kTile] = bits;
  }
  __builtin_amdgcn_s_waitcnt(0xF70);  // vmcnt(0): the slots (and, in the first chunk, the queries) are in
  __syncthreads();
#pragma unroll
  for (int t = 0; t < kLead; ++t)
    if (t < tiles) gather(t, k_ring + t * kStageBytes, v_ring + t * kStageBytes);
  static_assert(kStages == 2 || kStages == 4, "the tile loop is unrolled over the ring's stages");
  // One tile; the ring stage (t % kStages) is a compile-time constant, so
  // that the stage offsets of the LDS reads are immediates.
  auto tile_step = [&](const int t, auto stage_tag) __attribute__((always_inline)) {
    constexpr int stage = decltype(stage_tag)::value;  // t % kStages
    constexpr int lead_stage = (stage + kLead) % kStages;
    const unsigned char *k_stage = k_ring + stage * kStageBytes;
    unsigned char *v_stage = v_ring + stage * kStageBytes;
    // The slots of the gather issued after the barrier and the tile's
    // validity bits are read before it, so that their LDS latency passes
    // while the waves meet (both tables are written only before the loop).
    int next_slots[kGathers];
    if (t + kLead < tiles) gather_slots(t + kLead, next_slots);
    const unsigned long long valid_bits_lds = tile_valid[t];
    if (kLead >= 3 && t + 2 < tiles) __builtin_amdgcn_s_waitcnt(0xF70 | (4 * kGathers));
    else if (kLead >= 2 && t + 1 < tiles) __builtin_amdgcn_s_waitcnt(0xF70 | (2 * kGathers));
    else __builtin_amdgcn_s_waitcnt(0xF70);  // vmcnt(0)
    workgroup_barrier();
    // The gathers of tile t + kLead go to the stage every wave left before
    // this barrier.  Waves issue them at different points of the tile (wave w
    // after score batch w % 4), so that the workgroup's 32 loads do not all
    // queue for the texture unit at once while every wave waits in order
    // behind its own.
    const bool gather_due = t + kLead < tiles;
    auto issue_gathers = [&]() {
      gather_from(next_slots, k_ring + lead_stage * kStageBytes, v_ring + lead_stage * kStageBytes);
    };
    constexpr int kIssuePoints = kKSteps / 2;  // score batches of a tile
    const int issue_point = wave % kIssuePoints;
    // readfirstlane returns int: each half goes through unsigned so that the
    // low half is not sign-extended into the high one.
    const unsigned valid_lo =
        static_cast<unsigned>(__builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<unsigned>(valid_bits_lds))));
    const unsigned valid_hi = static_cast<unsigned>(
        __builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<unsigned>(valid_bits_lds >> 32))));
    const unsigned long long valid_bits = (static_cast<unsigned long long>(valid_hi) << 32) | valid_lo;
    if (valid_bits != ~0ull) {
      // Zero the V rows of tokens without a valid slot (0 * Inf would be NaN).
      for (int c = tid; c < kTile * kChunksPerRow; c += kM32Threads)
        if (((valid_bits >> (c / kChunksPerRow)) & 1ull) == 0)
          *reinterpret_cast<u32x4 *>(v_stage + c * 16) = u32x4{0u, 0u, 0u, 0u};
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
      workgroup_barrier();
    }
    const int t0 = chunk_begin + t * kTile;
    if (!wave_computes || t0 >= wave_stop) {
      if (gather_due) issue_gathers();
      return;
    }

    f32x16 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kb][r] = 0.f;
    // K fragments in batches of two 16-dim steps (both 32-token blocks), the
    // next batch's reads issued before this batch's MFMAs so that the LDS
    // latency hides under them.
    frag kf[2][4];
    auto load_k = [&](int batch, frag *dst) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
          dst[2 * j + kb] = *reinterpret_cast<const frag *>(k_stage + k_off[2 * batch + j] + kb * 32 * kRowBytes);
      }
    };
    load_k(0, kf[0]);
#pragma unroll
    for (int batch = 0; batch < kKSteps / 2; ++batch) {
      if (batch + 1 < kKSteps / 2) load_k(batch + 1, kf[(batch + 1) % 2]);
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) s[kb] = E::mfma32(kf[batch % 2][2 * j + kb], qf[2 * batch + j], s[kb]);
      if (gather_due && issue_point == batch) issue_gathers();
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // the first batch's 4 LDS reads
#pragma unroll
    for (int batch = 0; batch < kKSteps / 2; ++batch) {
      if (batch + 1 < kKSteps / 2) __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // next batch's reads
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);  // this batch's MFMAs
    }
    // Tiles that every query of the wave sees whole (the common case) skip the
    // mask: a scalar branch, since `whole` is wave-uniform.
    const bool whole = valid_bits == ~0ull && t0 + kTile <= wave_unmasked;
    if (!whole) {
      // Register r of block kb holds token 32 kb + 8 (r / 4) + 4 h + r % 4:
      // visible iff at or below the lane's limit and its slot is valid.
      const int limit = q_ok ? min(my_stop - 1, my_pos) - t0 - 4 * h : -1;
      const unsigned long long lane_bits = valid_bits >> (4 * h);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int rel = 32 * kb + 8 * (r / 4) + r % 4;
          const bool visible = rel <= limit && ((lane_bits >> rel) & 1ull) != 0;
          s[kb][r] = visible ? s[kb][r] : -INFINITY;
        }
      }
    }
    float tile_max = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) tile_max = fmaxf(tile_max, s[kb][r]);
    if (!q_ok) tile_max = -INFINITY;
    {
      unsigned a = __builtin_bit_cast(unsigned, tile_max), b = a;
      permlane32_swap(a, b);
      tile_max = max_f32(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
    }
    const bool raise = tile_max > m + slack;
    const float m_new = raise ? tile_max : m;
    const float bias = -m_new * scale_log2;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kb][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][r], scale_log2, bias));
    if (__builtin_amdgcn_ballot_w64(raise) != 0) {  // wave-uniform
      const float alpha = __builtin_amdgcn_exp2f((m - m_new) * scale_log2);
      l *= alpha;
#pragma unroll
      for (int b = 0; b < kDimBlocks; ++b) o[b] *= alpha;
    }
    m = m_new;
    // P^T operands of the four 16-token steps (step 2 kb + st), and their sums.
    frag pb[4];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        u32x4 bits;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          bits[j] = E::pack(s[kb][8 * st + 2 * j], s[kb][8 * st + 2 * j + 1]);
          l = E::dot2_ones(bits[j], l);
        }
        pb[2 * kb + st] = __builtin_bit_cast(frag, bits);
      }
    }
    // V^T fragments of one step (every dim block, two transposed reads each),
    // the next step's reads issued before this step's MFMAs.  Step 2 kb + st
    // covers tokens 32 kb + 16 st + 4 h + (0..3) and, 8 further, the second read.
    frag vf[2][kDimBlocks];
    auto load_v = [&](int step, frag *dst) {
      const int token_base = 16 * step * kRowBytes;
#pragma unroll
      for (int b = 0; b < kDimBlocks; ++b) {
        const unsigned lo = v_off[b] + stage * kStageBytes + token_base;
        const i16x4 a_lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(reinterpret_cast<lds_i16x4 *>(static_cast<uintptr_t>(lo)));
        const i16x4 a_hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            reinterpret_cast<lds_i16x4 *>(static_cast<uintptr_t>(lo + 8 * kRowBytes)));
        u32x4 va;
        va[0] = __builtin_bit_cast(u32x2, a_lo)[0];
        va[1] = __builtin_bit_cast(u32x2, a_lo)[1];
        va[2] = __builtin_bit_cast(u32x2, a_hi)[0];
        va[3] = __builtin_bit_cast(u32x2, a_hi)[1];
        dst[b] = __builtin_bit_cast(frag, va);
      }
    };
    load_v(0, vf[0]);
#pragma unroll
    for (int step = 0; step < 4; ++step) {
      if (step + 1 < 4) load_v(step + 1, vf[(step + 1) % 2]);
#pragma unroll
      for (int b = 0; b < kDimBlocks; ++b) o[b] = E::mfma32(vf[step % 2][b], pb[step], o[b]);
    }
  };
  for (int tb = 0; tb < tiles; tb += kStages) {
    tile_step(tb, std::integral_constant<int, 0>{});
    if (tb + 1 < tiles) tile_step(tb + 1, std::integral_constant<int, 1>{});
    if constexpr (kStages == 4) {
      if (tb + 2 < tiles) tile_step(tb + 2, std::integral_constant<int, 2>{});
      if (tb + 3 < tiles) tile_step(tb + 3, std::integral_constant<int, 3>{});
    }
  }
  }  // key chunks
  // The column's other half (lane l ^ 32) summed the other tokens.
  {
    unsigned a = __builtin_bit_cast(unsigned, l), b = a;
    permlane32_swap(a, b);
    l = __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
  }
  if (!mine.computes) return;
  // The output row, or the partial result's row: O / l in the KV dtype.
  // Register r of dim block b holds dim 32 b + 8 (r / 4) + 4 h + r % 4.
  if (!q_ok) return;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  float *block = mine.partial < 0 ? nullptr : partial_block<D>(p, mine.partial, mine.hq);
  uint16_t *dst = block == nullptr
                      ? p.out + (static_cast<long long>(mine.q_index + qc) * p.hq + mine.hq) * D + 4 * h
                      : reinterpret_cast<uint16_t *>(block) + qc * D + 4 * h;
#pragma unroll
  for (int b = 0; b < kDimBlocks; ++b)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      u32x2 packed;
      packed[0] = E::pack(o[b][4 * rr] * inv, o[b][4 * rr + 1] * inv);
      packed[1] = E::pack(o[b][4 * rr + 2] * inv, o[b][4 * rr + 3] * inv);
      *reinterpret_cast<u32x2 *>(dst + 32 * b + 8 * rr) = packed;
    }
  if (block != nullptr && h == 0) {
    block[kQueries * D / 2 + 2 * qc] = m * scale_log2;
    block[kQueries * D / 2 + 2 * qc + 1] = l;
  }
}

// Merges the split partial results of one 16-query tile: workgroup (combine
// item, query head); thread = (query, 1/16 of the dims).
template <int D, typename E>
__global__ void __launch_bounds__(256) repair_combine_kernel(const AttnParams p) {
  constexpr int kPer = D / 16;
  const int *ci = p.combine + static_cast<long long>(blockIdx.x) * kCombineInts;
  const int q_index = ci[0], q_count = ci[1], first = ci[2], count = ci[3];
  if (q_count < 1 || q_count > kQueries || q_index < 0 ||
      static_cast<long long>(q_index) + q_count > p.num_queries || first < 0 || count < 1 ||
      static_cast<long long>(first) + count > p.ws_items)
    return;
  const int h = blockIdx.y;
  const int c = threadIdx.x / 16;
  const int part = threadIdx.x % 16;
  if (c >= q_count) return;
  // One pass in batches of kBatch partials whose loads are all in flight
  // together; the running maximum rescales what is summed when a batch
  // raises it.  A partial's weight is its sum l times 2^(m - max): its
  // normalised output O / l then contributes exactly O.
  constexpr int kBatch = 8;
  float run_max = -INFINITY;
  float total = 0.f;
  f32x4 acc[kPer / 4];
#pragma unroll
  for (int d = 0; d < kPer / 4; ++d) acc[d] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < count; s0 += kBatch) {
    float ms[kBatch], ls[kBatch];
    u32x2 rows[kBatch][kPer / 4];  // kPer 16-bit values: kPer / 4 pairs of words
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int s = min(s0 + i, count - 1);  // past the end: the last partial again, unused
      const float *block = partial_block<D>(p, first + s, h);
      ms[i] = block[kQueries * D / 2 + 2 * c];
      ls[i] = block[kQueries * D / 2 + 2 * c + 1];
      const u32x2 *row = reinterpret_cast<const u32x2 *>(reinterpret_cast<const uint16_t *>(block) + c * D +
                                                         part * kPer);
#pragma unroll
      for (int d = 0; d < kPer / 4; ++d) rows[i][d] = row[d];
    }
    float batch_max = run_max;
#pragma unroll
    for (int i = 0; i < kBatch; ++i)
      if (s0 + i < count) batch_max = fmaxf(batch_max, ms[i]);
    if (batch_max > run_max) {
      const float scale = run_max == -INFINITY ? 0.f : exp2f(run_max - batch_max);
      total *= scale;
#pragma unroll
      for (int d = 0; d < kPer / 4; ++d) acc[d] *= scale;
      run_max = batch_max;
    }
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const float w = s0 + i >= count || ms[i] == -INFINITY ? 0.f : exp2f(ms[i] - run_max) * ls[i];
      total += w;
#pragma unroll
      for (int d = 0; d < kPer / 4; ++d) {  // values 4 d .. 4 d + 3
        const f32x2 v0 = E::unpack(rows[i][d][0]);
        const f32x2 v1 = E::unpack(rows[i][d][1]);
        acc[d] += w * f32x4{v0[0], v0[1], v1[0], v1[1]};
      }
    }
  }
  const float inv = total > 0.f ? 1.f / total : 0.f;
  uint16_t *dst = p.out + (static_cast<long long>(q_index + c) * p.hq + h) * D + part * kPer;
  uint32_t packed[kPer / 2];
#pragma unroll
  for (int d = 0; d < kPer / 4; ++d) {
    packed[2 * d] = E::pack(acc[d][0] * inv, acc[d][1] * inv);
    packed[2 * d + 1] = E::pack(acc[d][2] * inv, acc[d][3] * inv);
  }
#pragma unroll
  for (int d = 0; d < kPer / 4; ++d)  // the output is 8-byte aligned
    *reinterpret_cast<u32x2 *>(dst + 4 * d) = u32x2{packed[2 * d], packed[2 * d + 1]};
}

// Modelled run time of a plan in units of one 64-token key tile of a work
// item (about 2.4 us for Qwen's 28/4 heads on MI355X).  `groups` calls its
// argument with (key tokens, partial results) of every group of query tiles.
constexpr int kComputeUnits = 256;          // MI355X
constexpr double kItemOverheadTiles = 3.0;  // slots, queries, write-out
constexpr double kPartialBytesPerTile = 12e6;  // partial results the combine reads in one tile's time
constexpr double kCombineLaunchTiles = 2.0;
constexpr int64_t kRefillTiles = 2;  // an item's slot-list refill (every kDmaMaxRange keys): drain and restart
// A plan whose cost provably exceeds `beat` returns early with a lower bound
// of its cost (still above `beat`).
template <typename Groups>
double plan_cost_estimate(int64_t split, int64_t num_kv_heads, int64_t num_q_heads, double beat,
                          Groups &&groups) {
  // A group of `needed` keys makes needed / split full chunks and one shorter
  // one.  Costs are whole numbers of tiles, so their sums are exact in double
  // and do not depend on the order they are added in.
  auto tiles_of = [](int64_t keys) {  // an item's cost in whole tiles
    return (keys + kTile - 1) / kTile + static_cast<int64_t>(kItemOverheadTiles) +
           kRefillTiles * ((keys - 1) / kDmaMaxRange);
  };
  const double full_cost = static_cast<double>(tiles_of(split));
  int64_t partials = 0, count = 0;
  double total = 0.0, longest = 0.0;
  groups([&](int64_t needed, int64_t group_partials) {
    const int64_t full = needed / split, rest = needed - full * split;
    count += full + (rest > 0);
    total += static_cast<double>(full) * full_cost;
    if (full > 0) longest = full_cost > longest ? full_cost : longest;
    if (rest > 0) {
      const double cost = static_cast<double>(tiles_of(rest));
      total += cost;
      longest = cost > longest ? cost : longest;
    }
    partials += group_partials;
  });
  double combine_cost = 0.0;
  if (partials > 0)  // 16 queries' 16-bit outputs (head dim 128) and fp32 (max, sum) per partial and head
    combine_cost = kCombineLaunchTiles + static_cast<double>(partials) * num_q_heads *
                                             (kQueries * 128 * 2 + 2 * kQueries * 4) / kPartialBytesPerTile;
  if (count == 0) return combine_cost;
  if (count * num_kv_heads > 8 * kComputeUnits) {
    // Many rounds: the last one's imbalance is small against the total; it
    // leaves about half of the longest item to run alone.
    return total * num_kv_heads / kComputeUnits + 0.5 * longest + combine_cost;
  }
  // No schedule ends before its longest item or before the CUs have run
  // every item's work.
  const double spread = total * static_cast<double>(num_kv_heads) / kComputeUnits;
  const double bound = (longest > spread ? longest : spread) + combine_cost;
  if (bound > beat) return bound;
  double makespan = 0.0;
  // Item costs in whole tiles, longest first (the order the plan dispatches
  // its items in, see the ordering below): counted by value, then listed.
  static_assert(kItemOverheadTiles == 3.0, "the schedule counts whole tiles");
  const int64_t max_cost = tiles_of(split);
  std::vector<int64_t> cost_count(static_cast<size_t>(max_cost + 1), 0);
  groups([&](int64_t needed, int64_t) {
    const int64_t full = needed / split, rest = needed - full * split;
    cost_count[static_cast<size_t>(max_cost)] += full;
    if (rest > 0) ++cost_count[static_cast<size_t>(tiles_of(rest))];
  });
  std::vector<int64_t> item_cost;
  item_cost.reserve(static_cast<size_t>(count));
  for (int64_t c = max_cost; c > 0; --c) item_cost.insert(item_cost.end(), static_cast<size_t>(cost_count[c]), c);
  const int64_t n = static_cast<int64_t>(item_cost.size());
  if (n * num_kv_heads <= 2 * kComputeUnits) {
    // At most two rounds: the workgroups beyond the first 256 start when the
    // first round has ended (measured on c2: its 4 extra workgroups started
    // 72 us into an 82 us kernel, not when the first short items freed their
    // CUs), so the rounds' longest items add up.
    int64_t second = 0;
    for (int64_t g = kComputeUnits; g < n * num_kv_heads; ++g) {
      const int64_t cost = item_cost[static_cast<size_t>(g % n)];  // grid order: items, then KV heads
      second = cost > second ? cost : second;
    }
    makespan = static_cast<double>(item_cost.front() + second);
  } else {
    // Each workgroup starts on the CU that frees first.  Free times are
    // whole tiles and never earlier than the last start, so the CUs are
    // counted by free time and the earliest is found by moving forward.
    std::vector<int32_t> free_from(1, kComputeUnits);
    int64_t now = 0, last_end = 0;
    for (int64_t h = 0; h < num_kv_heads; ++h) {
      for (const int64_t cost : item_cost) {
        while (free_from[static_cast<size_t>(now)] == 0) ++now;
        --free_from[static_cast<size_t>(now)];
        const int64_t end = now + cost;
        if (end >= static_cast<int64_t>(free_from.size())) free_from.resize(static_cast<size_t>(end + 1), 0);
        ++free_from[static_cast<size_t>(end)];
        last_end = end > last_end ? end : last_end;
      }
    }
    makespan = static_cast<double>(last_end);
  }
  return makespan + combine_cost;
}

bool aligned(const void *ptr, uintptr_t bytes) {
  return (reinterpret_cast<uintptr_t>(ptr) & (bytes - 1)) == 0;
}

// Split partial results of ll_repair_attention_noalloc: one array per device,
// held from the library's load on that device until the process ends.  Host
// code must not use the array's name as a device address (it is a host-side
// stand-in); scratch_on() returns the device's own address of it.
constexpr long long kScratchBytes = LL_REPAIR_SCRATCH_BYTES;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
float *g_scratch_ptr[kMaxDevices];

// The scratch array's address on `device`, looked up once per device with that
// device current.  Returns nullptr (and records the error) on failure.
float *scratch_on(int device) {
  if (device < 0 || device >= kMaxDevices) {
    fail(LL_ERR_INVALID_ARGUMENT, "device %d is outside the %d devices the scratch table covers", device,
         kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[device] != nullptr) return g_scratch_ptr[device];
  int current = -1;
  hipError_t err = hipGetDevice(&current);
  if (err == hipSuccess && current != device) err = hipSetDevice(device);
  void *ptr = nullptr;
  if (err == hipSuccess) err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (current >= 0 && current != device) {
    const hipError_t restore = hipSetDevice(current);
    if (err == hipSuccess) err = restore;
  }
  if (err != hipSuccess || ptr == nullptr) {
    fail(LL_ERR_HIP, "scratch address on device %d: %s", device,
         err != hipSuccess ? hipGetErrorString(err) : "null address");
    return nullptr;
  }
  g_scratch_ptr[device] = static_cast<float *>(ptr);
  return g_scratch_ptr[device];
}

// Checks of the repair attention's arguments other than the workspace.
int check_attention_args(const ll_repair_attention_args *a) {
  if (a == nullptr) return fail(LL_ERR_INVALID_ARGUMENT, "args is NULL");
  if (a->struct_size != static_cast<int64_t>(sizeof(ll_repair_attention_args)))
    return fail(LL_ERR_INVALID_ARGUMENT, "struct_size %lld != %zu",
                static_cast<long long>(a->struct_size), sizeof(ll_repair_attention_args));
  if (a->kv_dtype != LL_DTYPE_BFLOAT16 && a->kv_dtype != LL_DTYPE_FLOAT16)
    return fail(LL_ERR_FP16_OR_BF16_REQUIRED, "repair attention takes fp16 or bf16 queries and KV");
  if (a->head_dim != 64 && a->head_dim != 128 && a->head_dim != 256)
    return fail(LL_ERR_HEAD_DIMENSION_OUT_OF_RANGE, "head_dim must be 64, 128 or 256");
  if (a->num_kv_heads < 1 || a->num_q_heads < 1 || a->num_q_heads % a->num_kv_heads != 0 ||
      a->num_q_heads > 65535)
    return fail(LL_ERR_KV_HEAD_LAYOUT_MISMATCH,
                "num_q_heads must be a multiple of num_kv_heads, at most 65535");
  if (a->num_queries < 0 || a->num_slots < 0 || a->kv_slots_len < 0 || a->num_items < 0 ||
      a->num_combine < 0 || a->workspace_items < 0)
    return fail(LL_ERR_INVALID_ARGUMENT, "counts must be >= 0");
  if (a->num_slots > 0x7fffffff) return fail(LL_ERR_INVALID_ARGUMENT, "num_slots must be below 2^31");
  if (!(a->softmax_scale > 0.0) || !isfinite(a->softmax_scale))
    return fail(LL_ERR_INVALID_ARGUMENT, "softmax_scale must be finite and > 0");
  if (a->num_items == 0) return LL_OK;
  if (a->num_items > 0x7fffffff || a->num_combine > 0x7fffffff)
    return fail(LL_ERR_INVALID_ARGUMENT, "too many items");
  if (a->query == nullptr || a->output == nullptr || a->key_buffer == nullptr ||
      a->value_buffer == nullptr || a->kv_slots == nullptr || a->items == nullptr ||
      a->query_positions == nullptr)
    return fail(LL_ERR_INVALID_ARGUMENT, "query/output/key/value/kv_slots/items/query_positions pointer is NULL");
  if (a->kv_slots_dtype != LL_DTYPE_INT32 && a->kv_slots_dtype != LL_DTYPE_INT64)
    return fail(LL_ERR_INTEGER_TOKEN_MAPS_REQUIRED, "kv_slots must be int32 or int64");
  if (a->num_combine > 0 && a->combine == nullptr)
    return fail(LL_ERR_INVALID_ARGUMENT, "split items need the combine table");
  if (!aligned(a->query, 16) || !aligned(a->key_buffer, 16) || !aligned(a->value_buffer, 16) ||
      !aligned(a->output, 8))
    return fail(LL_ERR_INVALID_ARGUMENT, "query/key/value (16-byte) and output (8-byte) must be aligned");
  return LL_OK;
}

template <int D, bool kOffsets>
void launch_m32(bool f16, dim3 grid, hipStream_t s, const AttnParams &p) {
  if (f16) repair_attention_m32_kernel<D, F16, kOffsets><<<grid, dim3(m32_threads<D>()), 0, s>>>(p);
  else repair_attention_m32_kernel<D, Bf16, kOffsets><<<grid, dim3(m32_threads<D>()), 0, s>>>(p);
}

// Launches the attention (and the combine of split items) with the partial
// results in `ws` (ws_items partial slots); the arguments are checked.
int launch_attention(const ll_repair_attention_args *a, float *ws, long long ws_items, hipStream_t s) {
  AttnParams p;
  memset(&p, 0, sizeof(p));
  p.q = static_cast<const uint16_t *>(a->query);
  p.out = static_cast<uint16_t *>(a->output);
  p.k = static_cast<const uint16_t *>(a->key_buffer);
  p.v = static_cast<const uint16_t *>(a->value_buffer);
  p.slots = a->kv_slots;
  p.items = a->items;
  p.combine = a->combine;
  p.positions = a->query_positions;
  p.ws = ws;
  p.num_queries = a->num_queries;
  p.num_slots = a->num_slots;
  p.slots_len = a->kv_slots_len;
  p.ws_items = ws != nullptr ? ws_items : 0;
  p.hq = static_cast<int>(a->num_q_heads);
  p.hkv = static_cast<int>(a->num_kv_heads);
  p.group = static_cast<int>(a->num_q_heads / a->num_kv_heads);
  // A workgroup holds a whole window of 16 pairs, or half of it at head dim
  // 256 (two workgroups per item and KV head).
  p.pair_chunks = kMaxPairs / max_pairs(static_cast<int>(a->head_dim));
  p.slots64 = a->kv_slots_dtype == LL_DTYPE_INT64 ? 1 : 0;
  p.scale_log2 = static_cast<float>(a->softmax_scale * 1.4426950408889634);  // log2(e)

  if (a->num_kv_heads * p.pair_chunks > 65535)
    return fail(LL_ERR_KV_HEAD_LAYOUT_MISMATCH, "too many KV heads for the grid");
  const dim3 grid(static_cast<unsigned>(a->num_items), static_cast<unsigned>(a->num_kv_heads * p.pair_chunks));
  const bool f16 = a->kv_dtype == LL_DTYPE_FLOAT16;
  // 32-bit row offsets where every row of the K (and V) buffer is below 4 GiB.
  const unsigned long long pool_bytes =
      static_cast<unsigned long long>(a->num_slots) * a->num_kv_heads * a->head_dim * 2;
  p.pool_bytes = pool_bytes <= 0xffffffffull ? static_cast<unsigned>(pool_bytes) : 0u;
  if (p.pool_bytes != 0 || a->num_slots == 0) {
    if (a->head_dim == 128) launch_m32<128, true>(f16, grid, s, p);
    else if (a->head_dim == 64) launch_m32<64, true>(f16, grid, s, p);
    else launch_m32<256, true>(f16, grid, s, p);
  } else {
    if (a->head_dim == 128) launch_m32<128, false>(f16, grid, s, p);
    else if (a->head_dim == 64) launch_m32<64, false>(f16, grid, s, p);
    else launch_m32<256, false>(f16, grid, s, p);
  }
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(LL_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(err));
  if (a->num_combine > 0) {
    const dim3 cgrid(static_cast<unsigned>(a->num_combine), static_cast<unsigned>(a->num_q_heads));
    if (a->head_dim == 128) {
      if (f16) repair_combine_kernel<128, F16><<<cgrid, dim3(256), 0, s>>>(p);
      else repair_combine_kernel<128, Bf16><<<cgrid, dim3(256), 0, s>>>(p);
    } else if (a->head_dim == 64) {
      if (f16) repair_combine_kernel<64, F16><<<cgrid, dim3(256), 0, s>>>(p);
      else repair_combine_kernel<64, Bf16><<<cgrid, dim3(256), 0, s>>>(p);
    } else {
      if (f16) repair_combine_kernel<256, F16><<<cgrid, dim3(256), 0, s>>>(p);
      else repair_combine_kernel<256, Bf16><<<cgrid, dim3(256), 0, s>>>(p);
    }
    err = hipGetLastError();
    if (err != hipSuccess) return fail(LL_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(err));
  }
  return LL_OK;
}

}  // namespace

extern "C" {

int64_t ll_repair_attention_args_size(void) {
  return static_cast<int64_t>(sizeof(ll_repair_attention_args));
}

}  // extern "C"

namespace {

// A plan computed into its own tables.  The last one is kept per thread:
// the table-sizing call and the table-filling call that follows it with the
// same rows and heads then compute it once.
struct RepairPlan {
  std::vector<ll_repair_row> rows;
  int64_t num_q_heads = -1, num_kv_heads = -1, split_in = -1;
  std::vector<int32_t> items, combine, positions;
  std::vector<int32_t> sorted;  // reordering space for the items
  ll_repair_attention_plan_info info{};
};

int compute_plan(const ll_repair_row *rows, int64_t num_rows, int64_t num_q_heads, int64_t num_kv_heads,
                 int64_t split_tokens, RepairPlan &out) {
  constexpr int64_t kIntMax = 0x7fffffff;
  const int64_t group = num_q_heads / num_kv_heads;
  // 16-query tiles in row order.  Consecutive rows of one request (the next
  // row's queries follow the last one's, same kv_offset) share a tile, so
  // short repair spans fill it; a tile records its lowest position and its
  // key end (highest position + 1).
  struct Tile { int64_t q_index, pos, count, kv_offset, needed; };
  int64_t num_queries = 0;
  for (int64_t r = 0; r < num_rows; ++r) {
    const ll_repair_row &row = rows[r];
    if (row.query_count < 1 || row.query_start < 0 || row.query_index < 0 || row.kv_offset < 0 ||
        row.query_start + row.query_count > kIntMax || row.query_index + row.query_count > kIntMax ||
        row.kv_offset + row.query_start + row.query_count > kIntMax)
      return fail(LL_ERR_INVALID_ARGUMENT, "row %lld: counts, positions and offsets must be >= 0 "
                  "(query_count >= 1) and fit in int32", static_cast<long long>(r));
    if (row.query_index + row.query_count > num_queries) num_queries = row.query_index + row.query_count;
  }
  out.positions.assign(static_cast<size_t>(num_queries), 0);
  int32_t *positions = out.positions.data();
  std::vector<Tile> tiles;
  int64_t fill = 0;  // queries in the open tile
  for (int64_t r = 0; r < num_rows; ++r) {
    const ll_repair_row &row = rows[r];
    for (int64_t i = 0; i < row.query_count; ++i)
      positions[row.query_index + i] = static_cast<int32_t>(row.query_start + i);
    const bool continues = fill > 0 && row.kv_offset == tiles.back().kv_offset &&
                           row.query_index == tiles.back().q_index + tiles.back().count;
    if (!continues) fill = 0;
    for (int64_t i = 0; i < row.query_count;) {
      if (fill == 0) tiles.push_back(Tile{row.query_index + i, kIntMax, 0, row.kv_offset, 0});
      Tile &tile = tiles.back();
      const int64_t take = row.query_count - i < kQueries - fill ? row.query_count - i : kQueries - fill;
      if (row.query_start + i < tile.pos) tile.pos = row.query_start + i;
      if (row.query_start + i + take > tile.needed) tile.needed = row.query_start + i + take;
      tile.count += take;
      fill = fill + take == kQueries ? 0 : fill + take;
      i += take;
    }
  }
  const int64_t n_tiles = static_cast<int64_t>(tiles.size());
  // Windows: the (tile, query head) pairs of each run of consecutive tiles of
  // one request, tile-major, cut into windows of at most kMaxPairs.  A window
  // covers tiles [first, last), from head pair_first of its first tile,
  // pair_count pairs, and costs its workgroup the keys of its furthest tile.
  // Below 16 query heads per KV head the cut points are chosen by dynamic
  // programming over the run's pairs, minimising the summed cost (key tiles
  // of each window's furthest tile plus a per-item overhead), so windows
  // cross tile boundaries freely: 16 pairs per workgroup where whole tiles of
  // 7 heads would fill 14.  From 16 heads up every tile is cut on its own.
  struct Window { int64_t first, last, pair_first, pair_count; };
  std::vector<Window> windows;
  std::vector<double> cost;
  std::vector<int64_t> from, pair_tiles;
  for (int64_t run = 0; run < n_tiles;) {
    int64_t run_end = run + 1;
    while (run_end < n_tiles && tiles[run_end].kv_offset == tiles[run].kv_offset) ++run_end;
    if (group >= kMaxPairs) {
      for (int64_t t = run; t < run_end; ++t)
        for (int64_t f = 0; f < group; f += kMaxPairs)
          windows.push_back(Window{t, t + 1, f, group - f < kMaxPairs ? group - f : kMaxPairs});
    } else {
      const int64_t n = (run_end - run) * group;  // pairs of the run, below 16 per tile
      cost.assign(static_cast<size_t>(n + 1), 0.0);
      from.assign(static_cast<size_t>(n + 1), 0);
      // Key tiles of each pair's tile (the ceiling of the maximum is the
      // maximum of the ceilings).
      pair_tiles.resize(static_cast<size_t>(n));
      for (int64_t t = run, j = 0; t < run_end; ++t)
        for (int64_t h = 0; h < group; ++h, ++j) pair_tiles[j] = (tiles[t].needed + kTile - 1) / kTile;
      for (int64_t i = 1; i <= n; ++i) {
        double best = -1.0;
        int64_t furthest = 0;
        for (int64_t j = i - 1; j >= 0 && j >= i - kMaxPairs; --j) {  // window [j, i)
          furthest = pair_tiles[j] > furthest ? pair_tiles[j] : furthest;
          const double c = cost[j] + static_cast<double>(furthest) + kItemOverheadTiles;
          if (best < 0.0 || c <= best) {  // ties: the longer window
            best = c;
            from[i] = j;
          }
        }
        cost[i] = best;
      }
      const size_t run_first = windows.size();
      for (int64_t i = n; i > 0; i = from[i]) {
        const int64_t j = from[i];
        windows.push_back(Window{run + j / group, run + (i - 1) / group + 1, j % group, i - j});
      }
      std::reverse(windows.begin() + static_cast<std::ptrdiff_t>(run_first), windows.end());
    }
    run = run_end;
  }
  std::vector<int64_t> window_keys(windows.size());  // keys of each window's furthest tile
  for (size_t k = 0; k < windows.size(); ++k) {
    int64_t needed = 0;
    for (int64_t t = windows[k].first; t < windows[k].last; ++t)
      needed = tiles[t].needed > needed ? tiles[t].needed : needed;
    window_keys[k] = needed;
  }
  int64_t split = split_tokens;
  if (split == 0) {
    // Pick the chunk length whose plan finishes first on a model of the
    // device: one workgroup per CU at a time (its LDS allows no more),
    // workgroups dispatched in grid order to the first free CU, each costing
    // its key tiles plus a fixed overhead, then the combine pass reading every
    // partial result.  Few long chunks leave CUs idle in the last round; many
    // short ones add overhead and partials.  A coarse pass over lengths from
    // 512 to the maximum, then every multiple of the key tile within 256 of
    // the best: one tile more per item can save a round (c2: 2,112 keys make
    // 64 items, one round of 4 KV heads on 256 CUs, where 2,048 make 65).
    double best = -1.0;
    auto estimate = [&](int64_t candidate) {
      const double beat = best < 0.0 ? HUGE_VAL : best;
      return plan_cost_estimate(candidate, num_kv_heads, num_q_heads, beat, [&](auto &&visit) {
        int64_t next_tile = 0;  // a tile's partials count with the first window that holds it
        for (size_t k = 0; k < windows.size(); ++k) {
          const Window &w = windows[k];
          int64_t partials = 0;
          for (int64_t t = w.first > next_tile ? w.first : next_tile; t < w.last; ++t) {
            const int64_t chunks = (tiles[t].needed + candidate - 1) / candidate;
            partials += chunks > 1 ? chunks : 0;
          }
          next_tile = w.last > next_tile ? w.last : next_tile;
          visit(window_keys[k], partials);
        }
      });
    };
    // Beyond 7,680 keys the lengths grow by half up to the longest window's
    // keys, which leaves every window whole (no partials, no combine).
    static const int64_t kCoarse[] = {512,  640,  768,  1024, 1280, 1536, 1792, 2048, 2304,
                                      2560, 3072, 3584, 4096, 4608, 5120, 6144, 7680};
    int64_t longest = kTile;
    for (const int64_t keys : window_keys) longest = keys > longest ? keys : longest;
    longest = (longest + kTile - 1) / kTile * kTile;
    std::vector<int64_t> candidates(std::begin(kCoarse), std::end(kCoarse));
    for (int64_t c = kCoarse[16] * 3 / 2 / kTile * kTile; c < longest; c = c * 3 / 2 / kTile * kTile)
      candidates.push_back(c);
    if (longest > kCoarse[16]) candidates.push_back(longest);
    for (const int64_t candidate : candidates) {
      const double cost = estimate(candidate);
      if (best < 0.0 || cost <= best) {
        best = cost;
        split = candidate;
      }
    }
    const int64_t coarse = split;
    for (int64_t candidate = coarse - 256; candidate <= coarse + 256; candidate += kTile) {
      if (candidate < 512 || candidate == coarse) continue;
      const double cost = estimate(candidate);
      if (cost < best || (cost == best && candidate > split)) {
        best = cost;
        split = candidate;
      }
    }
  }
  // Each tile's key chunks, and the partial slots and combine item of a tile
  // with more than one.
  int64_t n_items = 0, n_combine = 0, n_partial = 0;
  std::vector<int64_t> chunks(static_cast<size_t>(n_tiles)), base(static_cast<size_t>(n_tiles), -1);
  out.combine.clear();
  for (int64_t t = 0; t < n_tiles; ++t) {
    chunks[t] = (tiles[t].needed + split - 1) / split;
    if (chunks[t] < 2) continue;
    out.combine.push_back(static_cast<int32_t>(tiles[t].q_index));
    out.combine.push_back(static_cast<int32_t>(tiles[t].count));
    out.combine.push_back(static_cast<int32_t>(n_partial));
    out.combine.push_back(static_cast<int32_t>(chunks[t]));
    base[t] = n_partial;
    n_partial += chunks[t];
    ++n_combine;
  }
  for (const int64_t needed : window_keys) n_items += (needed + split - 1) / split;
  if (n_items > kIntMax || n_partial > kIntMax) return fail(LL_ERR_INVALID_ARGUMENT, "too many work items");
  out.items.assign(static_cast<size_t>(n_items * kItemInts), 0);
  int32_t *items = out.items.data();
  n_items = 0;
  for (size_t k = 0; k < windows.size(); ++k) {
    const Window &w = windows[k];
    const int64_t needed = window_keys[k];
    const int64_t window_chunks = (needed + split - 1) / split;
    for (int64_t s = 0; s < window_chunks; ++s, ++n_items) {
      int32_t *it = items + n_items * kItemInts;  // zeroed by the assign above
      it[0] = static_cast<int32_t>(tiles[w.first].kv_offset);
      it[1] = static_cast<int32_t>(s * split);
      it[2] = static_cast<int32_t>((s + 1) * split < needed ? (s + 1) * split : needed);
      it[3] = static_cast<int32_t>(w.last - w.first);
      it[4] = static_cast<int32_t>(w.pair_first);
      it[5] = static_cast<int32_t>(w.pair_count);
      for (int64_t t = w.first; t < w.last; ++t) {
        int32_t *e = it + kItemHeader + kTileInts * (t - w.first);
        e[0] = static_cast<int32_t>(tiles[t].q_index);
        e[1] = static_cast<int32_t>(tiles[t].pos);
        const bool present = s < chunks[t];  // this chunk holds keys the tile sees
        e[2] = present ? static_cast<int32_t>(tiles[t].count) : 0;
        e[3] = !present || chunks[t] == 1 ? -1 : static_cast<int32_t>(base[t] + s);
        e[4] = static_cast<int32_t>(tiles[t].needed);
      }
    }
  }
  if (n_items > 1) {
    // Longest key chunks first (the last round then holds the short ones),
    // and among equals the chunks in key order, so that the items running
    // together read the same keys: c5 +7 %, c3 +9 % over plan order.  The
    // order is free: every item names its own queries and partial slots.
    // Keys (longer first, then key begin, then plan order) are distinct, so
    // an unstable sort of them gives the stable order.
    struct Key { int32_t neg_len, begin, index; };
    std::vector<Key> order(static_cast<size_t>(n_items));
    for (int64_t i = 0; i < n_items; ++i) {
      const int32_t *x = items + i * kItemInts;
      order[static_cast<size_t>(i)] = Key{x[1] - x[2], x[1], static_cast<int32_t>(i)};
    }
    std::sort(order.begin(), order.end(), [](const Key &a, const Key &b) {
      return a.neg_len != b.neg_len ? a.neg_len < b.neg_len : a.begin != b.begin ? a.begin < b.begin
                                                                                 : a.index < b.index;
    });
    out.sorted.resize(static_cast<size_t>(n_items * kItemInts));
    for (int64_t i = 0; i < n_items; ++i)
      memcpy(&out.sorted[static_cast<size_t>(i * kItemInts)], items + order[static_cast<size_t>(i)].index * kItemInts,
             kItemInts * sizeof(int32_t));
    out.items.swap(out.sorted);
  }
  out.info.num_items = n_items;
  out.info.num_combine = n_combine;
  out.info.workspace_items = n_partial;
  out.info.split_tokens = split;
  out.info.num_queries = num_queries;
  return LL_OK;
}


}  // namespace

extern "C" {

int ll_repair_attention_plan(const ll_repair_row *rows, int64_t num_rows, int64_t num_q_heads,
                             int64_t num_kv_heads, int64_t split_tokens, int32_t *items,
                             int64_t items_capacity, int32_t *combine, int64_t combine_capacity,
                             int32_t *positions, int64_t positions_capacity,
                             ll_repair_attention_plan_info *info) {
  if (info == nullptr) return fail(LL_ERR_INVALID_ARGUMENT, "info is NULL");
  if (num_rows < 0 || (num_rows > 0 && rows == nullptr))
    return fail(LL_ERR_INVALID_ARGUMENT, "rows must be a host array of num_rows >= 0 entries");
  if (num_kv_heads < 1 || num_q_heads < 1 || num_q_heads % num_kv_heads != 0)
    return fail(LL_ERR_KV_HEAD_LAYOUT_MISMATCH, "num_q_heads must be a multiple of num_kv_heads");
  if (split_tokens < 0 || split_tokens % kTile != 0 || split_tokens > 0x7fffffc0)
    return fail(LL_ERR_INVALID_ARGUMENT, "split_tokens must be 0 or a positive multiple of %d below 2^31",
                kTile);
  if (num_q_heads > 65535)
    return fail(LL_ERR_KV_HEAD_LAYOUT_MISMATCH, "num_q_heads must be at most 65535");
  thread_local RepairPlan kept;
  const bool same_rows =
      static_cast<int64_t>(kept.rows.size()) == num_rows && kept.num_q_heads == num_q_heads &&
      kept.num_kv_heads == num_kv_heads &&
      (split_tokens == kept.split_in || split_tokens == kept.info.split_tokens) &&
      (num_rows == 0 || memcmp(kept.rows.data(), rows, static_cast<size_t>(num_rows) * sizeof(ll_repair_row)) == 0);
  if (!same_rows) {
    kept.num_q_heads = -1;  // invalid until computed
    const int rc = compute_plan(rows, num_rows, num_q_heads, num_kv_heads, split_tokens, kept);
    if (rc != LL_OK) return rc;
    kept.rows.assign(rows, rows + num_rows);
    kept.num_q_heads = num_q_heads;
    kept.num_kv_heads = num_kv_heads;
    kept.split_in = split_tokens;
  }
  const ll_repair_attention_plan_info &plan = kept.info;
  if (positions != nullptr && positions_capacity < plan.num_queries)
    return fail(LL_ERR_INVALID_ARGUMENT, "positions_capacity %lld is below the %lld queries",
                static_cast<long long>(positions_capacity), static_cast<long long>(plan.num_queries));
  if (combine != nullptr && combine_capacity < plan.num_combine)
    return fail(LL_ERR_INVALID_ARGUMENT, "combine_capacity %lld is too small",
                static_cast<long long>(combine_capacity));
  if (items != nullptr && items_capacity < plan.num_items)
    return fail(LL_ERR_INVALID_ARGUMENT, "items_capacity %lld is too small",
                static_cast<long long>(items_capacity));
  if (positions != nullptr && !kept.positions.empty())
    memcpy(positions, kept.positions.data(), kept.positions.size() * sizeof(int32_t));
  if (combine != nullptr && !kept.combine.empty())
    memcpy(combine, kept.combine.data(), kept.combine.size() * sizeof(int32_t));
  if (items != nullptr && !kept.items.empty())
    memcpy(items, kept.items.data(), kept.items.size() * sizeof(int32_t));
  *info = plan;
  return LL_OK;
}

int ll_repair_attention(const ll_repair_attention_args *a, ll_stream_t stream) {
  int rc = check_attention_args(a);
  if (rc != LL_OK || a->num_items == 0) return rc;
  if (a->num_combine > 0 && (a->workspace == nullptr || a->workspace_items < 1))
    return fail(LL_ERR_INVALID_ARGUMENT, "split items need the combine table and a workspace");
  if (!aligned(a->workspace, 16)) return fail(LL_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
  return launch_attention(a, a->workspace, a->workspace_items, reinterpret_cast<hipStream_t>(stream));
}

int ll_repair_attention_noalloc(const ll_repair_attention_args *a, ll_stream_t stream) {
  int rc = check_attention_args(a);
  if (rc != LL_OK) return rc;
  if (a->workspace != nullptr)
    return fail(LL_ERR_INVALID_ARGUMENT, "workspace must be NULL: the partial results go to the "
                "library's scratch array");
  if (a->num_items == 0) return LL_OK;
  // Every (partial, query head) block holds 16 queries x head_dim 16-bit
  // outputs and an fp32 (maximum, sum) pair per query: 8 head_dim + 32 floats.
  // workspace_items is bounded before the product, which then stays below
  // 2^56 (num_q_heads <= 65535 and head_dim <= 256 were checked).
  const long long block_floats = 8 * a->head_dim + 32;
  if (a->workspace_items > kScratchBytes ||
      a->workspace_items * a->num_q_heads * block_floats * 4 > kScratchBytes)
    return fail(LL_ERR_INVALID_ARGUMENT, "the plan's %lld split partials (%lld query heads, %lld bytes each) "
                "exceed what the scratch array holds: %lld bytes (LL_REPAIR_SCRATCH_BYTES)",
                static_cast<long long>(a->workspace_items), static_cast<long long>(a->num_q_heads),
                block_floats * 4, kScratchBytes);
  if (a->num_combine > 0 && a->workspace_items < 1)
    return fail(LL_ERR_INVALID_ARGUMENT, "split items need workspace_items partial slots");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  int device = -1;
  const hipError_t err = s != nullptr ? hipStreamGetDevice(s, &device) : hipGetDevice(&device);
  if (err != hipSuccess) return fail(LL_ERR_HIP, "stream device: %s", hipGetErrorString(err));
  float *ws = nullptr;
  if (a->num_combine > 0) {
    ws = scratch_on(device);
    if (ws == nullptr) return LL_ERR_HIP;
  }
  return launch_attention(a, ws, a->workspace_items, s);
}

int64_t ll_repair_scratch_bytes(void) { return kScratchBytes; }

}  // extern "C"
