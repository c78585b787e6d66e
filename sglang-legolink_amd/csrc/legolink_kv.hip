// LegoLink KV link kernels for MI355X (gfx950) and their C ABI.
//
// Two kernels implement the link (gather -> RoPE delta re-rotation -> scatter):
//
//   kv_link_vec_kernel      the production kernel.  The per-layer K/V rows of
//                           all tokens are flattened into 16-byte chunks; one
//                           lane owns one chunk of one token's row and walks
//                           that chunk through a run of layers.  The token's
//                           fp32 RoPE delta is computed once per lane and
//                           reused for every layer (and both V/K moves use one
//                           global_load_dwordx4 / global_store_dwordx4 per lane
//                           per layer).  Neox pairs (i, i + D/2) sit in lanes
//                           q and q ^ (D/16) of the same head, so the partner
//                           half arrives by a DPP row rotation (D = 128) or a
//                           lane swizzle (other D) instead of a second load.
//   kv_link_generic_kernel  one thread per rotary pair / pass-through element /
//                           V element; every shape the operator accepts
//                           (partial rotary, K/V head dims that differ,
//                           bf16/fp16 caches, strided caches).
//
// kv_scatter_kernel writes repaired boundary rows into the pool.
//
// Two rounding semantics, both with separate round-to-nearest-even multiplies
// and adds (the file is compiled with contraction off, so no FMA is formed):
//   fused  the reference's fused kernel, patched_sglang_files/python/sglang/srt/
//          legolink_triton.py:413-470: the delta and the rotation in fp32 and K
//          rounded once at the store (bf16 K with a bf16/fp16 cache: every
//          product and sum rounded to bf16);
//   eager  the reference's torch path, pic_runtime.py:6025-6058 and :1868-1885:
//          the delta computed in the cache's dtype and cast to the key dtype,
//          then every product and sum of the rotation rounded to the key dtype.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <vector>

#include "legolink_kv.h"
#include "ll_internal.h"

#pragma clang fp contract(off)

namespace {

// Layers whose loads one lane issues before it stores.  Random 1 KB rows are
// DRAM-page bound rather than latency bound: 2 measured best on gfx950.
#ifndef LL_LAYER_UNROLL
#define LL_LAYER_UNROLL 2
#endif
// 1: destination rows are written with non-temporal stores (the link never
// re-reads them); measured 1-3 % faster than plain stores on gfx950.
#ifndef LL_NT_STORE
#define LL_NT_STORE 1
#endif

constexpr int kMaxLayersPerLaunch = 64;
constexpr int kWave = 64;
// Workgroup-staged deltas: tokens whose deltas one workgroup stages in LDS.
constexpr int kMaxStagedTokens = 18;
constexpr int kMaxWavesPerBlock = 16;
constexpr int kLayerUnroll = LL_LAYER_UNROLL;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// Kernel parameters (passed by value in the kernarg segment; the per-layer
// pointer tables make one launch cover up to kMaxLayersPerLaunch layers
// without a device-side table allocation).
// ---------------------------------------------------------------------------
struct LinkParams {
  char *k_layers[kMaxLayersPerLaunch];   // destination rows
  char *v_layers[kMaxLayersPerLaunch];
  const char *sk_layers[kMaxLayersPerLaunch];  // source rows (the same buffers, or another pool)
  const char *sv_layers[kMaxLayersPerLaunch];
  const void *src;
  const void *dst;
  const void *lpos;
  const void *gpos;
  const unsigned char *mask;
  const void *cs;
  long long num_tokens;
  long long num_slots;       // destination rows per layer
  long long src_num_slots;   // source rows per layer
  long long cs_rows;
  long long cs_stride_row;
  long long cs_stride_col;
  long long prefix;
  long long k_row_bytes;
  long long v_row_bytes;
  long long chunks_per_row;  // vector kernel: 16-byte chunks per K row (== per V row)
  int num_layers;            // layers in this launch
  int layers_per_wave;
  int layer_groups_per_block;  // vector kernel: waves of a block that share a token
  int num_heads;
  int kdim;
  int vdim;
  int rotary_dim;
  int idx64;                 // bit0 src, bit1 dst, bit2 local, bit3 global are int64
  int neox;
  int stream_rows;           // vector kernel: non-temporal row loads (rows read once)
  int eager;                 // LL_ROUNDING_EAGER: the torch path's rounding points
  int staged;                // vector kernel: deltas staged once per workgroup in LDS
  unsigned long long *skipped;  // tokens skipped for an out-of-range index, or NULL
  f32x2 *delta_table;        // layer-major kernel: per token and rotary pair (dc, ds)
  int write_table;           // layer-major value pass: layer 0 writes the delta table
};

struct ScatterParams {
  char *k_layers[kMaxLayersPerLaunch];
  char *v_layers[kMaxLayersPerLaunch];
  const void *dst;
  const char *rk;
  const char *rv;
  long long num_rows;
  long long num_slots;
  long long rk_layer_stride_bytes;
  long long rv_layer_stride_bytes;
  long long k_row_bytes;
  long long v_row_bytes;
  int idx64;
};

// ---------------------------------------------------------------------------
// Element conversions.
// ---------------------------------------------------------------------------
__device__ __forceinline__ long long load_index(const void *p, bool is64, long long i) {
  return is64 ? static_cast<const long long *>(p)[i]
              : static_cast<long long>(static_cast<const int *>(p)[i]);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits) {
  return __uint_as_float(bits << 16);
}

// float -> bf16 bits, round to nearest even; NaN becomes the quiet NaN 0x7fc0.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits) {
  return __half2float(__ushort_as_half(static_cast<unsigned short>(bits)));
}

__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  return __half_as_ushort(__float2half_rn(f));
}

// Round an fp32 value to the nearest bf16 / fp16 and widen it back.
__device__ __forceinline__ float round_bf16(float f) {
  return bf16_bits_to_f32(f32_to_bf16_bits(f));
}

__device__ __forceinline__ float round_f16(float f) {
  return f16_bits_to_f32(f32_to_f16_bits(f));
}

// Storage-type codes of the rounding helpers (the kernels' kCache / kKey
// codes): 1 = fp16, 2 = bf16, 3 = fp32 (an fp32 op result is already rounded).
template <int kTo>
__device__ __forceinline__ float round_to(float f) {
  if constexpr (kTo == 2) return round_bf16(f);
  else if constexpr (kTo == 1) return round_f16(f);
  else return f;
}

template <bool kBF16>
__device__ __forceinline__ float lo_elem(uint32_t w) {
  if constexpr (kBF16) return __uint_as_float(w << 16);
  else return f16_bits_to_f32(w & 0xffffu);
}

template <bool kBF16>
__device__ __forceinline__ float hi_elem(uint32_t w) {
  if constexpr (kBF16) return __uint_as_float(w & 0xffff0000u);
  else return f16_bits_to_f32(w >> 16);
}

template <bool kBF16>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  if constexpr (kBF16) return f32_to_bf16_bits(a) | (f32_to_bf16_bits(b) << 16);
  else return f32_to_f16_bits(a) | (f32_to_f16_bits(b) << 16);
}

// ---------------------------------------------------------------------------
// Cross-lane partner exchange: lane i receives lane i ^ kXor (kXor < 64).
// ---------------------------------------------------------------------------
template <int kXor>
__device__ __forceinline__ uint32_t xor_lane(uint32_t v) {
  if constexpr (kXor == 8) {
    // DPP row_ror:8 rotates each 16-lane row by 8, i.e. lane i <- lane i ^ 8.
    return static_cast<uint32_t>(
        __builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x128, 0xf, 0xf, false));
  } else {
    return static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), kXor, kWave));
  }
}

template <int kXor>
__device__ __forceinline__ u32x4 xor_lane4(u32x4 v) {
  u32x4 r;
  r.x = xor_lane<kXor>(v.x);
  r.y = xor_lane<kXor>(v.y);
  r.z = xor_lane<kXor>(v.z);
  r.w = xor_lane<kXor>(v.w);
  return r;
}

// A row chunk of the source pool; non-temporal when each row is read once.
// (A compile-time choice: with a runtime one the compiler merges both loads
// into one plain load.)
template <bool kStream>
__device__ __forceinline__ u32x4 load_row(const char *address) {
  const u32x4 *chunk = reinterpret_cast<const u32x4 *>(address);
  if constexpr (kStream) return __builtin_nontemporal_load(chunk);
  else return *chunk;
}

__device__ __forceinline__ void store_row_chunk(char *address, u32x4 value) {
#if LL_NT_STORE
  __builtin_nontemporal_store(value, reinterpret_cast<u32x4 *>(address));
#else
  *reinterpret_cast<u32x4 *>(address) = value;
#endif
}

// Neox: x holds 8 elements of this lane's half, y the same 8 dims of the other
// half.  out = x*dc + y*dsn, with dsn = -ds in the first half and +ds in the
// second half:  first' = first*dc - second*ds,  second' = second*dc + first*ds.
// kProd rounds each product before the sum (round_to codes): to bf16 for the
// fused bf16 chain (bf16 K with a bf16/fp16 cache) and to the key dtype for
// the eager semantics; 3 keeps fp32.  The sum is rounded to the key dtype when
// packed.  RNE is symmetric under negation, so rounding y * dsn equals
// negating the rounded y * ds.
template <int kProd>
__device__ __forceinline__ float rot_term(float a, float b) {
  return round_to<kProd>(a * b);
}

template <bool kBF16, int kProd>
__device__ __forceinline__ u32x4 rotate_neox(u32x4 x, u32x4 y, const float *dc,
                                             const float *dsn) {
  u32x4 out;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float x0 = lo_elem<kBF16>(x[w]);
    const float x1 = hi_elem<kBF16>(x[w]);
    const float y0 = lo_elem<kBF16>(y[w]);
    const float y1 = hi_elem<kBF16>(y[w]);
    const float r0 = rot_term<kProd>(x0, dc[2 * w]) + rot_term<kProd>(y0, dsn[2 * w]);
    const float r1 = rot_term<kProd>(x1, dc[2 * w + 1]) + rot_term<kProd>(y1, dsn[2 * w + 1]);
    out[w] = pack2<kBF16>(r0, r1);
  }
  return out;
}

// GPT-J style: every 32-bit word holds one (first, second) pair.
template <bool kBF16, int kProd>
__device__ __forceinline__ u32x4 rotate_gptj(u32x4 x, const float *dc, const float *ds) {
  u32x4 out;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float a = lo_elem<kBF16>(x[w]);
    const float b = hi_elem<kBF16>(x[w]);
    const float r0 = rot_term<kProd>(a, dc[w]) - rot_term<kProd>(b, ds[w]);
    const float r1 = rot_term<kProd>(b, dc[w]) + rot_term<kProd>(a, ds[w]);
    out[w] = pack2<kBF16>(r0, r1);
  }
  return out;
}

// Rounding points of one rounding semantics (round_to codes).  The delta's
// products and sums round to kDelta, the delta is then cast to kCast, and the
// rotation's products round to kProd.
template <bool kBF16, int kCache, bool kEager>
struct Rounding {
  static constexpr int kKey = kBF16 ? 2 : 1;
  // Fused: bf16 K with a 16-bit cache follows the reference's bf16 chain
  // (legolink_triton.py:437-468), everything else stays fp32 (:413-436, :469-470).
  static constexpr bool kFusedChain = kBF16 && kCache != 3;
  static constexpr int kDelta = kEager ? kCache : (kFusedChain ? 2 : 3);
  static constexpr int kCast = kEager ? (kCache == kKey ? 3 : kKey) : 3;
  static constexpr int kProd = kEager ? kKey : (kFusedChain ? 2 : 3);
};

// The delta rotation of one pair: dc = gc*lc + gs*ls, ds = gs*lc - gc*ls.
template <int kDelta, int kCast>
__device__ __forceinline__ void delta_pair(float lc, float ls, float gc, float gs, float &dc,
                                           float &ds) {
  dc = round_to<kCast>(round_to<kDelta>(round_to<kDelta>(gc * lc) + round_to<kDelta>(gs * ls)));
  ds = round_to<kCast>(round_to<kDelta>(round_to<kDelta>(gs * lc) - round_to<kDelta>(gc * ls)));
}

// N consecutive cos/sin table entries from element `offset`, widened to fp32
// (exactly: bf16 and fp16 values are fp32 values).  kCache: 1 = fp16,
// 2 = bf16, 3 = fp32.  The address is 16-byte aligned (8-byte for four
// 16-bit entries).
template <int kCache, int N>
__device__ __forceinline__ void load_table(const void *cs, long long offset, float *out) {
  if constexpr (kCache == 3) {
#pragma unroll
    for (int e = 0; e < N; e += 4) {
      const f32x4 v = *reinterpret_cast<const f32x4 *>(static_cast<const float *>(cs) + offset + e);
#pragma unroll
      for (int k = 0; k < 4; ++k) out[e + k] = v[k];
    }
  } else {
    const uint16_t *base = static_cast<const uint16_t *>(cs) + offset;
    uint32_t w[N / 2];
    if constexpr (N == 8) {
      const u32x4 v = *reinterpret_cast<const u32x4 *>(base);
#pragma unroll
      for (int k = 0; k < 4; ++k) w[k] = v[k];
    } else {
      static_assert(N == 4, "four or eight entries");
      const u32x2 v = *reinterpret_cast<const u32x2 *>(base);
      w[0] = v[0];
      w[1] = v[1];
    }
#pragma unroll
    for (int k = 0; k < N / 2; ++k) {
      out[2 * k] = lo_elem<kCache == 2>(w[k]);
      out[2 * k + 1] = hi_elem<kCache == 2>(w[k]);
    }
  }
}

// ---------------------------------------------------------------------------
// Vectorised link kernel.
//   Waves cover num_tokens * chunks_per_row chunks, 64 per wave; the launch's
//   layers are split into groups of layers_per_wave.  A block of W waves holds
//   W / G chunk-waves x G layer groups (G = layer_groups_per_block).
//   grid.x = chunk-waves / (W / G), grid.y = layer groups / G.
//   Deltas: per wave (each lane reads its token's cos/sin entries and computes
//   its 8 pairs' delta itself), or, with kStaged, once per workgroup: G covers
//   every layer group of the launch, the workgroup computes each of its tokens'
//   deltas once into LDS (every table entry read once per token), and every
//   wave reads its lanes' pairs from there.
// Requirements (checked on the host): key_head_dim == value_head_dim ==
// rotary_dim == kD, an fp32, bf16 or fp16 cos/sin cache (kCache) with unit
// column stride and 16-byte aligned rows, 16-byte aligned layer buffers; for
// kStaged also an fp32 cache and at most kMaxStagedTokens tokens per block.
// ---------------------------------------------------------------------------
template <bool kBF16, int kD, int kR, bool kNeox, typename Index, int kCache, bool kStream,
          bool kEager, bool kStaged>
__global__ void __launch_bounds__(kStaged ? kMaxWavesPerBlock * kWave : 512)
kv_link_vec_kernel(const LinkParams p) {
  constexpr int kChunksPerHead = kD / 8;
  constexpr int kRotChunks = kR / 8;     // chunks of a head that rotate; the rest are copied
  constexpr int kPairs = kNeox ? 8 : 4;  // rotary pairs touched by one lane
  using Round = Rounding<kBF16, kCache, kEager>;
  constexpr int kHalf = kR / 2;
  static_assert(kR == kD || kR * 2 == kD, "full or half rotary");

  const int lane = threadIdx.x & (kWave - 1);
  // Wave-uniform by construction; readfirstlane lets the compiler keep the
  // layer range in scalar registers, so the per-layer row pointers are read
  // from the kernel arguments with scalar loads.
  const int wave_in_block = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
  const int groups = p.layer_groups_per_block;
  const long long wave =
      static_cast<long long>(blockIdx.x) * (blockDim.x / kWave / groups) + wave_in_block / groups;
  const int layer_group = blockIdx.y * groups + wave_in_block % groups;
  const int l0 = layer_group * p.layers_per_wave;
  const int l1 = min(l0 + p.layers_per_wave, p.num_layers);
  // A whole wave whose layer group lies past the last layer has no rows; with
  // staged deltas it still helps stage and meets the barrier.
  if constexpr (!kStaged) {
    if (l0 >= l1) return;
  }
  const bool has_layers = l0 < l1;
  const long long g = wave * kWave + lane;
  const long long C = p.chunks_per_row;
  const bool in_range = g < p.num_tokens * C;
  const long long t = in_range ? g / C : 0;
  const long long c = in_range ? g - t * C : 0;
  // Chunk index inside the head; chunks_per_row is a multiple of
  // kChunksPerHead and kChunksPerHead divides 64, so this is lane-aligned.
  const int q = lane % kChunksPerHead;
  const bool rotating = kR == kD || q < kRotChunks;

  // The token's maps: five independent loads with no branch between them, so
  // they are in flight together (t < num_tokens always holds).  Without a
  // mask the mask byte is read from the source map and ignored.
  const Index *maps_src = static_cast<const Index *>(p.src);
  const long long src = static_cast<long long>(maps_src[t]);
  const long long dst = static_cast<long long>(static_cast<const Index *>(p.dst)[t]);
  const long long lp = static_cast<long long>(static_cast<const Index *>(p.lpos)[t]);
  const long long gp = static_cast<long long>(static_cast<const Index *>(p.gpos)[t]);
  const unsigned char *mask_bytes =
      p.mask != nullptr ? p.mask : reinterpret_cast<const unsigned char *>(maps_src);
  const unsigned char mask_byte = mask_bytes[t];
  const bool remap = t >= p.prefix;
  const bool positions_ok = lp >= 0 && lp < p.cs_rows && gp >= 0 && gp < p.cs_rows;
  const bool masked = p.mask != nullptr && mask_byte != 0;
  const bool ok = in_range && !masked && src >= 0 && src < p.src_num_slots && dst >= 0 &&
                  dst < p.num_slots && (!remap || positions_ok);
  // An unmasked token skipped for an out-of-range index is counted once, by
  // its first chunk's lane in layer group 0 (an ordinary global atomic).
  if (p.skipped != nullptr && in_range && !ok && !masked && c == 0 && layer_group == 0)
    atomicAdd(p.skipped, 1ull);

  // Row loads are unconditional so that no wait separates one layer's loads
  // from the next: a lane without a valid source reads row 0 (the host
  // launches only when the source pool has rows) and stores nothing.
  const long long src_row = (src >= 0 && src < p.src_num_slots) ? src : 0;
  const long long k_src = src_row * p.k_row_bytes + c * 16;
  const long long k_dst = dst * p.k_row_bytes + c * 16;
  const long long v_src = src_row * p.v_row_bytes + c * 16;
  const long long v_dst = dst * p.v_row_bytes + c * 16;

  // Rows of the first layers are requested before the cos/sin reads, so both
  // are in flight while the delta is computed.  Past l1 the last layer is
  // read again (uniform clamp) and not stored.
  u32x4 kin[kLayerUnroll];
  u32x4 vin[kLayerUnroll];
  if (has_layers) {
#pragma unroll
    for (int u = 0; u < kLayerUnroll; ++u) {
      const int lu = min(l0 + u, l1 - 1);
      kin[u] = load_row<kStream>(p.sk_layers[lu] + k_src);
      vin[u] = load_row<kStream>(p.sv_layers[lu] + v_src);
    }
  }

  // fp32 delta of this lane's rotary pairs.  Rows are clamped to 0 where the
  // delta is not used (prefix tokens, invalid positions), so the reads stay in
  // bounds without a branch; a table without rows is never read.
  float dc[kPairs];
  float ds[kPairs];
#pragma unroll
  for (int e = 0; e < kPairs; ++e) {
    dc[e] = 1.0f;
    ds[e] = 0.0f;
  }
  if constexpr (kStaged) {
    // The workgroup's tokens [t_first, t_end): entry (token, pair) of the LDS
    // table holds that token's (dc, ds) for the pair; identity where the delta
    // is not used.  Consecutive threads take consecutive pairs of a token, so
    // the table reads are coalesced.
    constexpr int kTokenPairs = kR / 2;
    __shared__ float staged_cos[kMaxStagedTokens * kTokenPairs];
    __shared__ float staged_sin[kMaxStagedTokens * kTokenPairs];
    const long long block_chunks = static_cast<long long>(blockDim.x / kWave / groups) * kWave;
    const long long first_chunk = static_cast<long long>(blockIdx.x) * block_chunks;
    const long long t_first = first_chunk / C;
    const long long t_end = min((first_chunk + block_chunks + C - 1) / C, p.num_tokens);
    const int entries = static_cast<int>(t_end - t_first) * kTokenPairs;
    const float *table = static_cast<const float *>(p.cs);
    for (int e = threadIdx.x; e < entries; e += blockDim.x) {
      const int token = e / kTokenPairs;
      const int i = e - token * kTokenPairs;
      const long long tt = t_first + token;
      float sc = 1.0f, ss = 0.0f;
      if (tt >= p.prefix) {
        const long long lpe = static_cast<long long>(static_cast<const Index *>(p.lpos)[tt]);
        const long long gpe = static_cast<long long>(static_cast<const Index *>(p.gpos)[tt]);
        if (lpe >= 0 && lpe < p.cs_rows && gpe >= 0 && gpe < p.cs_rows) {
          const float lc = table[lpe * p.cs_stride_row + i];
          const float ls = table[lpe * p.cs_stride_row + i + kHalf];
          const float gc = table[gpe * p.cs_stride_row + i];
          const float gs = table[gpe * p.cs_stride_row + i + kHalf];
          delta_pair<Round::kDelta, Round::kCast>(lc, ls, gc, gs, sc, ss);
        }
      }
      staged_cos[e] = sc;
      staged_sin[e] = ss;
    }
    __syncthreads();
    if (!has_layers) return;
    const int token = in_range ? static_cast<int>(t - t_first) : 0;
    const int pb = kNeox ? (q % (kRotChunks / 2)) * 8 : (rotating ? q : 0) * 4;
#pragma unroll
    for (int e = 0; e < kPairs; ++e) {
      dc[e] = staged_cos[token * kTokenPairs + pb + e];
      ds[e] = staged_sin[token * kTokenPairs + pb + e];
    }
  } else if (p.cs_rows > 0) {
    const bool use = remap && positions_ok;
    const long long lrow_index = use ? lp : 0;
    const long long grow_index = use ? gp : 0;
    // Lanes past the rotary dims read the first pairs' entries (unused), so
    // the reads stay inside the row.
    const int pb = kNeox ? (q % (kRotChunks / 2)) * 8 : (rotating ? q : 0) * 4;
    const long long lrow = lrow_index * p.cs_stride_row + pb;
    const long long grow = grow_index * p.cs_stride_row + pb;
    float lc[kPairs], ls[kPairs], gc[kPairs], gs[kPairs];
    load_table<kCache, kPairs>(p.cs, lrow, lc);
    load_table<kCache, kPairs>(p.cs, lrow + kHalf, ls);
    load_table<kCache, kPairs>(p.cs, grow, gc);
    load_table<kCache, kPairs>(p.cs, grow + kHalf, gs);
#pragma unroll
    for (int e = 0; e < kPairs; ++e)
      delta_pair<Round::kDelta, Round::kCast>(lc[e], ls[e], gc[e], gs[e], dc[e], ds[e]);
  }
  float dsn[kPairs];
  if constexpr (kNeox) {
    const bool second_half = q >= kRotChunks / 2;
#pragma unroll
    for (int e = 0; e < kPairs; ++e) dsn[e] = second_half ? ds[e] : -ds[e];
  }

  for (int l = l0; l < l1; l += kLayerUnroll) {
    if (l != l0) {
#pragma unroll
      for (int u = 0; u < kLayerUnroll; ++u) {
        const int lu = min(l + u, l1 - 1);
        kin[u] = load_row<kStream>(p.sk_layers[lu] + k_src);
        vin[u] = load_row<kStream>(p.sv_layers[lu] + v_src);
      }
    }
#pragma unroll
    for (int u = 0; u < kLayerUnroll; ++u) {
      u32x4 kout = kin[u];
      if constexpr (kNeox) {
        // Every lane takes part in the exchange (uniform control flow here).
        const u32x4 partner = xor_lane4<kRotChunks / 2>(kin[u]);
        if (remap && rotating) kout = rotate_neox<kBF16, Round::kProd>(kin[u], partner, dc, dsn);
      } else {
        if (remap && rotating) kout = rotate_gptj<kBF16, Round::kProd>(kin[u], dc, ds);
      }
      if (ok && l + u < l1) {
        store_row_chunk(p.k_layers[l + u] + k_dst, kout);
        store_row_chunk(p.v_layers[l + u] + v_dst, vin[u]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Layer-major link (LL_DELTA_TABLE).  Two launches of kv_link_layer_kernel,
// each a walk of the layers one after another (wave w moves two consecutive
// tokens of one layer, one 1 KiB chunk of their rows per lane group), so that
// at any time the GPU reads and writes about one buffer of one layer:
//
//   value pass  the V rows (bit copies); with write_table, the waves of
//               layer 0 also write the delta table: entry [t][i] = (dc, ds)
//               of rotary pair i of token t (consecutive lanes on
//               consecutive pairs, so the cos/sin rows are read coalesced,
//               once per token), (1, 0) where the token keeps its rotation
//               (the identity prefix) or a position is out of range;
//   key pass    the K rows, each lane rotating its chunk with its 8 pairs'
//               deltas read back from the table (the table is small and
//               stays in the caches).
// The second launch is ordered after the first on the stream, so the table
// is complete when the key pass reads it.  The arithmetic is the vector
// kernel's: same delta_pair rounding points, same rotate_neox, same bounds
// checks, skips and skipped-token count (counted by the value pass).
// Requirements (checked on the host): neox, rotary_dim == key_head_dim ==
// value_head_dim == kD, an fp32 table with unit column stride and 16-byte
// aligned rows, chunks_per_row a multiple of 64, 16-byte aligned buffers.
// ---------------------------------------------------------------------------
constexpr int kLayerMajorWaves = 4;  // waves per workgroup of the layer-major kernel

template <bool kBF16, int kD, typename Index, bool kStream, bool kEager, bool kKeys>
__global__ void __launch_bounds__(kLayerMajorWaves * kWave) kv_link_layer_kernel(const LinkParams p) {
  constexpr bool kValues = !kKeys;
  constexpr int kChunksPerHead = kD / 8;
  constexpr int kHalfChunks = kChunksPerHead / 2;  // chunks of a head's first rotate half
  constexpr int kPairs = kD / 2;                   // rotary pairs of a token (full rotary)
  using Round = Rounding<kBF16, 3, kEager>;

  const int lane = threadIdx.x & (kWave - 1);
  // Wave-uniform: the wave's layer, token pair and row part (scalar registers).
  const long long wave = static_cast<long long>(blockIdx.x) * kLayerMajorWaves +
                         __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
  const long long parts = p.chunks_per_row / kWave;
  const long long pairs = (p.num_tokens + 1) / 2;
  const long long per_layer = pairs * parts;
  if (wave >= per_layer * p.num_layers) return;
  const int layer = static_cast<int>(wave / per_layer);
  const long long rest = wave - static_cast<long long>(layer) * per_layer;
  const long long pair = rest / parts;
  const long long part = rest - pair * parts;
  const long long c = part * kWave + lane;  // the lane's 16-byte chunk of the row
  const int q = lane % kChunksPerHead;
  const bool second_half = q >= kHalfChunks;
  const int pb = (q % kHalfChunks) * 8;     // the lane's first rotary pair

  u32x4 kin[2], vin[2];
  long long k_dst[2], v_dst[2], token[2], lpos[2], gpos[2];
  bool ok[2], remap[2], use[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const long long t = 2 * pair + u;
    const bool in_range = t < p.num_tokens;
    token[u] = in_range ? t : 2 * pair;
    const long long tt = token[u];
    const long long src = static_cast<long long>(static_cast<const Index *>(p.src)[tt]);
    const long long dst = static_cast<long long>(static_cast<const Index *>(p.dst)[tt]);
    const long long lp = static_cast<long long>(static_cast<const Index *>(p.lpos)[tt]);
    const long long gp = static_cast<long long>(static_cast<const Index *>(p.gpos)[tt]);
    const bool masked = p.mask != nullptr && p.mask[tt] != 0;
    remap[u] = tt >= p.prefix;
    const bool positions_ok = lp >= 0 && lp < p.cs_rows && gp >= 0 && gp < p.cs_rows;
    ok[u] = in_range && !masked && src >= 0 && src < p.src_num_slots && dst >= 0 && dst < p.num_slots &&
            (!remap[u] || positions_ok);
    use[u] = remap[u] && positions_ok;
    lpos[u] = use[u] ? lp : 0;
    gpos[u] = use[u] ? gp : 0;
    // An unmasked token skipped for an out-of-range index is counted once:
    // by lane 0 of its first row part in layer 0.
    if (kValues && p.skipped != nullptr && in_range && !ok[u] && !masked && layer == 0 && part == 0 &&
        lane == 0)
      atomicAdd(p.skipped, 1ull);
    // Unconditional row loads: a token without a valid source reads row 0
    // (the host launches only when the source pool has rows) and stores nothing.
    const long long src_row = (src >= 0 && src < p.src_num_slots) ? src : 0;
    if constexpr (kKeys) {
      kin[u] = load_row<kStream>(p.sk_layers[layer] + src_row * p.k_row_bytes + c * 16);
      k_dst[u] = dst * p.k_row_bytes + c * 16;
    } else {
      vin[u] = load_row<kStream>(p.sv_layers[layer] + src_row * p.v_row_bytes + c * 16);
      v_dst[u] = dst * p.v_row_bytes + c * 16;
    }
  }
  if constexpr (!kKeys) {
    // Layer 0 of the value pass writes the delta table: entry (token, pair)
    // = (dc, ds), identity where the token keeps its rotation.
    if (p.write_table && layer == 0 && part == 0) {
      const float *cs = static_cast<const float *>(p.cs);
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        if (2 * pair + u >= p.num_tokens) continue;
        for (int i = lane; i < kPairs; i += kWave) {
          float dc = 1.0f, ds = 0.0f;
          if (use[u]) {
            const float lc = cs[lpos[u] * p.cs_stride_row + i];
            const float ls = cs[lpos[u] * p.cs_stride_row + i + kPairs];
            const float gc = cs[gpos[u] * p.cs_stride_row + i];
            const float gs = cs[gpos[u] * p.cs_stride_row + i + kPairs];
            delta_pair<Round::kDelta, Round::kCast>(lc, ls, gc, gs, dc, ds);
          }
          f32x2 entry;
          entry.x = dc;
          entry.y = ds;
          p.delta_table[token[u] * kPairs + i] = entry;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u)
      if (ok[u]) store_row_chunk(p.v_layers[layer] + v_dst[u], vin[u]);
    return;
  }
  // The lanes' deltas: 8 consecutive (dc, ds) entries of the token's row of
  // the table, identity where the token keeps its rotation.
  f32x4 entries[2][4];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const f32x4 *row = reinterpret_cast<const f32x4 *>(p.delta_table + token[u] * kPairs + pb);
#pragma unroll
    for (int k = 0; k < 4; ++k) entries[u][k] = row[k];
  }
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    float dc[8], dsn[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      dc[2 * k] = entries[u][k][0];
      dc[2 * k + 1] = entries[u][k][2];
      const float s0 = entries[u][k][1];
      const float s1 = entries[u][k][3];
      dsn[2 * k] = second_half ? s0 : -s0;
      dsn[2 * k + 1] = second_half ? s1 : -s1;
    }
    // Every lane takes part in the exchange (uniform control flow here).
    const u32x4 partner = xor_lane4<kHalfChunks>(kin[u]);
    u32x4 kout = kin[u];
    if (remap[u]) kout = rotate_neox<kBF16, Round::kProd>(kin[u], partner, dc, dsn);
    if (ok[u]) store_row_chunk(p.k_layers[layer] + k_dst[u], kout);
  }
}

// ---------------------------------------------------------------------------
// Generic link kernel: grid.y = layer, blocks stride over tokens, threads over
// the token's work items (rotary pairs, pass-through K dims, V dims).
// kKey: 1 = fp16, 2 = bf16.  kCache: 1 = fp16, 2 = bf16, 3 = fp32.
// ---------------------------------------------------------------------------
template <int kCache>
__device__ __forceinline__ float load_cache(const void *cs, long long offset) {
  if constexpr (kCache == 3) return static_cast<const float *>(cs)[offset];
  else if constexpr (kCache == 2)
    return bf16_bits_to_f32(static_cast<const uint16_t *>(cs)[offset]);
  else return f16_bits_to_f32(static_cast<const uint16_t *>(cs)[offset]);
}

template <int kKey>
__device__ __forceinline__ float key_to_f32(uint16_t bits) {
  if constexpr (kKey == 2) return bf16_bits_to_f32(bits);
  else return f16_bits_to_f32(bits);
}

template <int kKey>
__device__ __forceinline__ uint16_t f32_to_key(float f) {
  if constexpr (kKey == 2) return static_cast<uint16_t>(f32_to_bf16_bits(f));
  else return static_cast<uint16_t>(f32_to_f16_bits(f));
}

template <int kKey, int kCache, bool kEager>
__global__ void __launch_bounds__(512) kv_link_generic_kernel(const LinkParams p) {
  using Round = Rounding<kKey == 2, kCache, kEager>;
  const int layer = blockIdx.y;
  const uint16_t *kbase = reinterpret_cast<const uint16_t *>(p.sk_layers[layer]);
  uint16_t *kout = reinterpret_cast<uint16_t *>(p.k_layers[layer]);
  const uint16_t *vbase = reinterpret_cast<const uint16_t *>(p.sv_layers[layer]);
  uint16_t *vout = reinterpret_cast<uint16_t *>(p.v_layers[layer]);
  const int half = p.rotary_dim / 2;
  const int rot_items = p.num_heads * half;
  const int pass_dims = p.kdim - p.rotary_dim;
  const int pass_items = p.num_heads * pass_dims;
  const int v_items = p.num_heads * p.vdim;
  const int items = rot_items + pass_items + v_items;
  const long long k_row = static_cast<long long>(p.num_heads) * p.kdim;
  const long long v_row = static_cast<long long>(p.num_heads) * p.vdim;

  for (long long t = blockIdx.x; t < p.num_tokens; t += gridDim.x) {
    if (p.mask != nullptr && p.mask[t] != 0) continue;
    const long long src = load_index(p.src, p.idx64 & 1, t);
    const long long dst = load_index(p.dst, p.idx64 & 2, t);
    bool bad = src < 0 || src >= p.src_num_slots || dst < 0 || dst >= p.num_slots;
    const bool remap = t >= p.prefix;
    long long lp = 0, gp = 0;
    if (remap && !bad) {
      lp = load_index(p.lpos, p.idx64 & 4, t);
      gp = load_index(p.gpos, p.idx64 & 8, t);
      bad = lp < 0 || lp >= p.cs_rows || gp < 0 || gp >= p.cs_rows;
    }
    if (bad) {
      // Counted once per token: by thread 0 of the first layer's workgroup.
      if (p.skipped != nullptr && blockIdx.y == 0 && threadIdx.x == 0) atomicAdd(p.skipped, 1ull);
      continue;
    }
    const uint16_t *ks = kbase + src * k_row;
    uint16_t *kd = kout + dst * k_row;
    for (int w = threadIdx.x; w < items; w += blockDim.x) {
      if (w < rot_items) {
        const int h = w / half;
        const int i = w - h * half;
        const int d1 = p.neox ? i : 2 * i;
        const int d2 = p.neox ? i + half : 2 * i + 1;
        const uint16_t b1 = ks[h * p.kdim + d1];
        const uint16_t b2 = ks[h * p.kdim + d2];
        uint16_t o1 = b1, o2 = b2;
        if (remap) {
          const float lc = load_cache<kCache>(p.cs, lp * p.cs_stride_row + i * p.cs_stride_col);
          const float ls =
              load_cache<kCache>(p.cs, lp * p.cs_stride_row + (i + half) * p.cs_stride_col);
          const float gc = load_cache<kCache>(p.cs, gp * p.cs_stride_row + i * p.cs_stride_col);
          const float gs =
              load_cache<kCache>(p.cs, gp * p.cs_stride_row + (i + half) * p.cs_stride_col);
          const float x1 = key_to_f32<kKey>(b1);
          const float x2 = key_to_f32<kKey>(b2);
          float dc, ds;
          delta_pair<Round::kDelta, Round::kCast>(lc, ls, gc, gs, dc, ds);
          const float first_cos = round_to<Round::kProd>(x1 * dc);
          const float second_sin = round_to<Round::kProd>(x2 * ds);
          const float second_cos = round_to<Round::kProd>(x2 * dc);
          const float first_sin = round_to<Round::kProd>(x1 * ds);
          o1 = f32_to_key<kKey>(first_cos - second_sin);
          o2 = f32_to_key<kKey>(second_cos + first_sin);
        }
        kd[h * p.kdim + d1] = o1;
        kd[h * p.kdim + d2] = o2;
      } else if (w < rot_items + pass_items) {
        const int j = w - rot_items;
        const int h = j / pass_dims;
        const int d = p.rotary_dim + (j - h * pass_dims);
        kd[h * p.kdim + d] = ks[h * p.kdim + d];
      } else {
        const long long j = w - rot_items - pass_items;
        vout[dst * v_row + j] = vbase[src * v_row + j];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Repaired-row scatter: grid.y = layer; threads stride over the layer's
// (row, chunk) items, K rows first, then V rows.
// ---------------------------------------------------------------------------
template <typename Chunk>
__global__ void __launch_bounds__(512) kv_scatter_kernel(const ScatterParams p) {
  const int layer = blockIdx.y;
  constexpr int kBytes = sizeof(Chunk);
  const long long kc = p.k_row_bytes / kBytes;
  const long long vc = p.v_row_bytes / kBytes;
  const long long k_items = p.num_rows * kc;
  const long long total = k_items + p.num_rows * vc;
  const long long stride = static_cast<long long>(gridDim.x) * blockDim.x;
  for (long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += stride) {
    const bool is_k = i < k_items;
    const long long j = is_k ? i : i - k_items;
    const long long per_row = is_k ? kc : vc;
    const long long r = j / per_row;
    const long long c = j - r * per_row;
    const long long slot = load_index(p.dst, p.idx64 & 2, r);
    if (slot < 0 || slot >= p.num_slots) continue;
    if (is_k) {
      const Chunk v = *reinterpret_cast<const Chunk *>(
          p.rk + layer * p.rk_layer_stride_bytes + r * p.k_row_bytes + c * kBytes);
      *reinterpret_cast<Chunk *>(p.k_layers[layer] + slot * p.k_row_bytes + c * kBytes) = v;
    } else {
      const Chunk v = *reinterpret_cast<const Chunk *>(
          p.rv + layer * p.rv_layer_stride_bytes + r * p.v_row_bytes + c * kBytes);
      *reinterpret_cast<Chunk *>(p.v_layers[layer] + slot * p.v_row_bytes + c * kBytes) = v;
    }
  }
}

// ---------------------------------------------------------------------------
// Map builder: writes a link's token maps from a plan's runs.  Workgroup
// (x, y) takes tokens [y * kMapTokensPerBlock, (y + 1) * kMapTokensPerBlock)
// of run x; the runs of one launch travel in the kernel arguments (validated
// on the host, so every index below is in range).  The work is a few int64
// reads and writes per token: a latency-bound pass far below HBM bandwidth.
// ---------------------------------------------------------------------------
// 56 runs x 64 B keep the kernel arguments under 4 KB (hidden arguments included).
constexpr int kMaxSegmentsPerLaunch = 56;
constexpr int kMapTokensPerBlock = 1024;

struct MapSegment {
  const long long *src;
  const long long *local;  // nullptr: local_start + i
  long long start;         // global position of token 0
  long long dst_start;     // index of token 0's slot in the destination slots
  long long local_start;
  int count;
  int map_offset;
  int repair_begin;
  int repair_end;
  int repair_offset;  // < 0: repair rows not recorded
  int set;
};

// Where the maps go (shared by every run of a launch).
struct MapTargets {
  const void *dst;
  long long *maps[2];
  long long cap[2];
  unsigned char *mask[2];
  long long *repair_dst;
  int dst64;
};

struct MapParams {
  MapSegment seg[kMaxSegmentsPerLaunch];
  MapTargets t;
};

__device__ __forceinline__ void map_run_tokens(const MapSegment &sg, const MapTargets &p) {
  const int first = static_cast<int>(blockIdx.y) * kMapTokensPerBlock;
  const int end = min(sg.count, first + kMapTokensPerBlock);
  unsigned char *mask = p.mask[sg.set];
  long long *m = p.maps[sg.set];
  const long long cap = p.cap[sg.set];
  const int repair_rows = sg.repair_end - sg.repair_begin;
  for (int i = first + static_cast<int>(threadIdx.x); i < end; i += blockDim.x) {
    const long long pos = sg.start + i;
    const long long di = sg.dst_start + i;
    const long long d = p.dst64 ? static_cast<const long long *>(p.dst)[di]
                                : static_cast<long long>(static_cast<const int *>(p.dst)[di]);
    const bool repair = i >= sg.repair_begin && i < sg.repair_end;
    if (repair && sg.repair_offset >= 0) p.repair_dst[sg.repair_offset + (i - sg.repair_begin)] = d;
    if (repair && mask == nullptr) continue;  // compacted set: repair rows take no entry
    const int o = sg.map_offset + ((mask == nullptr && i >= sg.repair_end) ? i - repair_rows : i);
    m[o] = sg.src[i];
    m[cap + o] = d;
    m[2 * cap + o] = sg.local != nullptr ? sg.local[i] : sg.local_start + i;
    m[3 * cap + o] = pos;
    if (mask != nullptr) mask[o] = repair ? 1 : 0;
  }
}

__global__ void __launch_bounds__(256) build_link_maps_kernel(const MapParams p) {
  map_run_tokens(p.seg[blockIdx.x], p.t);
}

// The same, with the runs read from a device copy of the run table: one
// launch for any number of runs.  The host validated its own copy of the
// table; each block checks its run again against the launch's bounds (the
// checks of ll_kv_build_link_maps), so a device table that differs from the
// host's cannot send a write out of range: such a run is left out.
__global__ void __launch_bounds__(256) build_link_maps_table_kernel(const MapTargets p,
                                                                    const ll_link_segment *runs,
                                                                    long long num_destination_slots,
                                                                    long long repair_capacity) {
  const ll_link_segment g = runs[blockIdx.x];
  constexpr long long kIntMax = 0x7fffffff;
  if (g.token_count <= 0 || g.token_count > kIntMax || g.source_slots == nullptr) return;
  if (g.map_set != 0 && g.map_set != 1) return;
  if (g.destination_start < 0 || g.destination_start > num_destination_slots - g.token_count) return;
  if (g.repair_begin < 0 || g.repair_begin > g.repair_end || g.repair_end > g.token_count) return;
  const int set = static_cast<int>(g.map_set);
  const long long repair_rows = g.repair_end - g.repair_begin;
  const long long entries = g.token_count - (p.mask[set] == nullptr ? repair_rows : 0);
  if (entries > 0 && (p.maps[set] == nullptr || g.map_offset < 0 || g.map_offset > p.cap[set] - entries)) return;
  if (g.repair_offset < -1) return;
  const bool record = repair_rows > 0 && g.repair_offset >= 0;
  if (record && (p.repair_dst == nullptr || g.repair_offset > repair_capacity - repair_rows)) return;
  MapSegment sg;
  sg.src = reinterpret_cast<const long long *>(g.source_slots);
  sg.local = reinterpret_cast<const long long *>(g.local_positions);
  sg.start = g.start_token;
  sg.dst_start = g.destination_start;
  sg.local_start = g.local_start;
  sg.count = static_cast<int>(g.token_count);
  sg.map_offset = static_cast<int>(g.map_offset);
  sg.repair_begin = static_cast<int>(g.repair_begin);
  sg.repair_end = static_cast<int>(g.repair_end);
  sg.repair_offset = record ? static_cast<int>(g.repair_offset) : -1;
  sg.set = set;
  map_run_tokens(sg, p);
}

// ---------------------------------------------------------------------------
// Visit order of a map set: a counting sort over buckets of 2^shift
// consecutive slots of one map row (source or destination), in three launches.  The count adds every
// entry to its bucket's counter (atomics); one workgroup turns the counts
// into exclusive offsets and clears the counters for the next call; the
// scatter takes each entry's place with an atomic increment of its bucket's
// offset.  The launches' boundaries order them: no fences, and no workgroup
// waits for another.
// ---------------------------------------------------------------------------
constexpr int kOrderBuckets = LL_ORDER_BUCKETS;
constexpr int kOrderThreads = 1024;
static_assert(kOrderBuckets % kOrderThreads == 0, "whole bucket runs per thread");

struct OrderParams {
  const long long *maps;
  const long long *key;  // the map row ordered by: maps + key_row * cap
  const unsigned char *mask;
  long long cap, count, prefix, num_slots;
  int shift;
  long long *out;
  unsigned char *out_mask;
  int *counts;   // [kOrderBuckets]: zero between calls
  int *offsets;  // [kOrderBuckets]
};

__device__ __forceinline__ int order_bucket(long long slot, const OrderParams &p) {
  if (slot < 0) return 0;
  if (slot >= p.num_slots) return kOrderBuckets - 1;
  return static_cast<int>(slot >> p.shift);  // below kOrderBuckets by the choice of shift
}

__global__ void __launch_bounds__(256) order_count_kernel(const OrderParams p) {
  const long long n = p.count - p.prefix;
  const long long *dst = p.key + p.prefix;
  for (long long i = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += static_cast<long long>(gridDim.x) * 256)
    atomicAdd(&p.counts[order_bucket(dst[i], p)], 1);
}

__global__ void __launch_bounds__(kOrderThreads) order_offsets_kernel(const OrderParams p) {
  // Thread t owns buckets [16 t, 16 t + 16): 64 contiguous bytes, read and
  // written as four 16-byte vectors.  Scan: within each wave by shuffles,
  // then across the 16 waves through LDS.
  typedef int i32x4 __attribute__((ext_vector_type(4)));
  constexpr int kPer = kOrderBuckets / kOrderThreads;
  static_assert(kPer == 16, "four 16-byte vectors per thread");
  __shared__ int wave_totals[kOrderThreads / 64];
  i32x4 *counts = reinterpret_cast<i32x4 *>(p.counts) + threadIdx.x * (kPer / 4);
  i32x4 *offsets = reinterpret_cast<i32x4 *>(p.offsets) + threadIdx.x * (kPer / 4);
  i32x4 own[kPer / 4];
  int total = 0;
#pragma unroll
  for (int k = 0; k < kPer / 4; ++k) {
    own[k] = counts[k];
    total += own[k][0] + own[k][1] + own[k][2] + own[k][3];
  }
  const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  int inclusive = total;
#pragma unroll
  for (int step = 1; step < 64; step <<= 1) {
    const int up = __shfl_up(inclusive, step, 64);
    if (lane >= step) inclusive += up;
  }
  if (lane == 63) wave_totals[wave] = inclusive;
  __syncthreads();
  int before = 0;
  for (int w = 0; w < wave; ++w) before += wave_totals[w];
  int offset = before + inclusive - total;
  const i32x4 zero = {0, 0, 0, 0};
#pragma unroll
  for (int k = 0; k < kPer / 4; ++k) {
    i32x4 out;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      out[e] = offset;
      offset += own[k][e];
    }
    offsets[k] = out;
    counts[k] = zero;
  }
}

__global__ void __launch_bounds__(256) order_scatter_kernel(const OrderParams p) {
  const long long n = p.count - p.prefix;
  for (long long i = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x; i < p.count;
       i += static_cast<long long>(gridDim.x) * 256) {
    long long o = i;
    if (i >= p.prefix) {
      const long long place = atomicAdd(&p.offsets[order_bucket(p.key[i], p)], 1);
      if (place < 0 || place >= n) continue;  // only if the workspace was shared by overlapping calls
      o = p.prefix + place;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) p.out[r * p.cap + o] = p.maps[r * p.cap + i];
    if (p.mask != nullptr) p.out_mask[o] = p.mask[i];
  }
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
thread_local std::string g_last_error;

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  const int rc = ll_record_error(code, fmt, ap);
  va_end(ap);
  return rc;
}

bool is_index_dtype(int64_t dt) { return dt == LL_DTYPE_INT32 || dt == LL_DTYPE_INT64; }

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int validate_link(const ll_kv_link_args *a) {
  if (a == nullptr) return fail(LL_ERR_INVALID_ARGUMENT, "args is NULL");
  if (a->struct_size != static_cast<int64_t>(sizeof(ll_kv_link_args)))
    return fail(LL_ERR_INVALID_ARGUMENT, "struct_size %lld != %zu",
                static_cast<long long>(a->struct_size), sizeof(ll_kv_link_args));
  if (a->num_layers < 1 || a->key_layers == nullptr || a->value_layers == nullptr)
    return fail(LL_ERR_INVALID_ARGUMENT, "num_layers must be >= 1 with key/value layer tables");
  for (int64_t l = 0; l < a->num_layers; ++l)
    if (a->key_layers[l] == nullptr || a->value_layers[l] == nullptr)
      return fail(LL_ERR_INVALID_ARGUMENT, "layer %lld buffer is NULL", static_cast<long long>(l));
  if ((a->source_key_layers == nullptr) != (a->source_value_layers == nullptr))
    return fail(LL_ERR_INVALID_ARGUMENT, "source key and value layer tables must both be set or both NULL");
  if (a->source_key_layers != nullptr) {
    for (int64_t l = 0; l < a->num_layers; ++l)
      if (a->source_key_layers[l] == nullptr || a->source_value_layers[l] == nullptr)
        return fail(LL_ERR_INVALID_ARGUMENT, "source layer %lld buffer is NULL",
                    static_cast<long long>(l));
    if (a->source_num_slots < 0)
      return fail(LL_ERR_INVALID_ARGUMENT, "source_num_slots is negative");
  }
  if (a->num_slots < 0) return fail(LL_ERR_INVALID_ARGUMENT, "num_slots is negative");
  if (a->num_heads < 1)
    return fail(LL_ERR_MHA_3D_KV_BUFFERS_REQUIRED, "num_heads must be >= 1");
  if (a->kv_dtype != LL_DTYPE_BFLOAT16 && a->kv_dtype != LL_DTYPE_FLOAT16)
    return fail(LL_ERR_FP16_OR_BF16_REQUIRED, "kv_dtype must be fp16 or bf16");
  if (a->key_head_dim < 1 || a->value_head_dim < 1 || a->key_head_dim > 256 ||
      a->value_head_dim > 256)
    return fail(LL_ERR_HEAD_DIMENSION_OUT_OF_RANGE, "head dims must be in 1..256");
  if (a->num_tokens < 0) return fail(LL_ERR_INVALID_ARGUMENT, "num_tokens is negative");
  if (a->num_tokens == 0) return fail(LL_ERR_EMPTY_LINK, "no tokens to link");
  if (a->source_slots == nullptr || a->destination_slots == nullptr ||
      a->local_positions == nullptr || a->global_positions == nullptr)
    return fail(LL_ERR_INVALID_ARGUMENT, "token map pointer is NULL");
  if (a->repair_mask != nullptr && a->repair_mask_dtype != LL_DTYPE_UINT8)
    return fail(LL_ERR_BOOLEAN_REPAIR_MASK_REQUIRED, "repair mask must be uint8/bool");
  if (!is_index_dtype(a->source_slots_dtype) || !is_index_dtype(a->destination_slots_dtype) ||
      !is_index_dtype(a->local_positions_dtype) || !is_index_dtype(a->global_positions_dtype))
    return fail(LL_ERR_INTEGER_TOKEN_MAPS_REQUIRED, "token maps must be int32 or int64");
  if (a->rotary_dim <= 0 || (a->rotary_dim % 2) != 0)
    return fail(LL_ERR_EVEN_ROTARY_DIM_REQUIRED, "rotary_dim must be positive and even");
  if (a->rotary_dim > a->key_head_dim)
    return fail(LL_ERR_ROTARY_DIM_EXCEEDS_HEAD_DIM, "rotary_dim exceeds key_head_dim");
  if (a->cos_sin_cache == nullptr || a->cos_sin_rows < 0 || a->cos_sin_cols < a->rotary_dim)
    return fail(LL_ERR_UNSUPPORTED_COS_SIN_CACHE, "cos/sin cache must hold >= rotary_dim columns");
  if (a->cos_sin_dtype != LL_DTYPE_FLOAT32 && a->cos_sin_dtype != LL_DTYPE_BFLOAT16 &&
      a->cos_sin_dtype != LL_DTYPE_FLOAT16)
    return fail(LL_ERR_UNSUPPORTED_COS_SIN_DTYPE, "cos/sin cache must be fp32, bf16 or fp16");
  if (a->prefix_token_count < 0 || a->prefix_token_count > a->num_tokens)
    return fail(LL_ERR_PREFIX_OUT_OF_RANGE, "prefix_token_count is outside the linked token range");
  if (a->kernel < LL_KERNEL_AUTO || a->kernel > LL_KERNEL_GENERIC)
    return fail(LL_ERR_LAUNCH_CONFIG, "unknown kernel selector %lld",
                static_cast<long long>(a->kernel));
  if (a->delta_staging < LL_DELTA_AUTO || a->delta_staging > LL_DELTA_TABLE)
    return fail(LL_ERR_LAUNCH_CONFIG, "unknown delta_staging %lld", static_cast<long long>(a->delta_staging));
  if (a->delta_workspace_bytes < 0) return fail(LL_ERR_INVALID_ARGUMENT, "delta_workspace_bytes is negative");
  if (a->delta_staging == LL_DELTA_WORKGROUP) {
    if (a->waves_per_block < 0 || a->waves_per_block > kMaxWavesPerBlock)
      return fail(LL_ERR_LAUNCH_CONFIG, "waves_per_block must be 0..16 with workgroup-staged deltas");
    if (a->layer_groups_per_block != 0)
      return fail(LL_ERR_LAUNCH_CONFIG, "workgroup-staged deltas choose layer_groups_per_block themselves");
  } else if (a->waves_per_block != 0 && a->waves_per_block != 1 && a->waves_per_block != 2 &&
             a->waves_per_block != 4 && a->waves_per_block != 8) {
    return fail(LL_ERR_LAUNCH_CONFIG, "waves_per_block must be 0, 1, 2, 4 or 8");
  }
  if (a->layers_per_wave < 0) return fail(LL_ERR_LAUNCH_CONFIG, "layers_per_wave is negative");
  if (a->rounding != LL_ROUNDING_FUSED && a->rounding != LL_ROUNDING_EAGER)
    return fail(LL_ERR_INVALID_ARGUMENT, "unknown rounding %lld", static_cast<long long>(a->rounding));
  if (reinterpret_cast<uintptr_t>(a->skipped_rows) % alignof(uint64_t) != 0)
    return fail(LL_ERR_INVALID_ARGUMENT, "skipped_rows must be 8-byte aligned");
  if (a->layer_groups_per_block < 0 ||
      (a->layer_groups_per_block > 0 &&
       ((a->waves_per_block ? a->waves_per_block : 4) % a->layer_groups_per_block) != 0))
    return fail(LL_ERR_LAUNCH_CONFIG, "layer_groups_per_block must divide waves_per_block");
  return LL_OK;
}

bool vector_kernel_fits(const ll_kv_link_args *a) {
  const int64_t d = a->key_head_dim;
  // One index type for all four token maps.
  if (a->destination_slots_dtype != a->source_slots_dtype ||
      a->local_positions_dtype != a->source_slots_dtype ||
      a->global_positions_dtype != a->source_slots_dtype)
    return false;
  if (!(d == 32 || d == 64 || d == 128 || d == 256)) return false;
  if (a->value_head_dim != d) return false;
  if (a->rotary_dim != d && !(a->rotary_dim * 2 == d && d >= 32)) return false;
  if (a->cos_sin_stride_col != 1 || !aligned16(a->cos_sin_cache)) return false;
  // Rows 16-byte aligned: 4 fp32 or 8 16-bit entries per 16 bytes.
  if ((a->cos_sin_stride_row % (a->cos_sin_dtype == LL_DTYPE_FLOAT32 ? 4 : 8)) != 0) return false;
  for (int64_t l = 0; l < a->num_layers; ++l)
    if (!aligned16(a->key_layers[l]) || !aligned16(a->value_layers[l])) return false;
  if (a->source_key_layers != nullptr)
    for (int64_t l = 0; l < a->num_layers; ++l)
      if (!aligned16(a->source_key_layers[l]) || !aligned16(a->source_value_layers[l])) return false;
  return true;
}

struct LinkPlan {
  int kernel;  // LL_KERNEL_VECTOR / LL_KERNEL_GENERIC
  int block_threads;
  long long grid_x;
  int layers_per_wave;  // vector kernel
  int layer_groups_per_block;  // vector kernel
  int launches;
  bool staged;  // vector kernel: workgroup-staged deltas
  bool layer_major;  // delta table + layer-major kernel
};

// Workgroup-staged deltas need the production shape (neox, full rotary, fp32
// table) on the vector kernel.
bool staging_fits(const ll_kv_link_args *a) {
  return a->is_neox_style && a->rotary_dim == a->key_head_dim && a->cos_sin_dtype == LL_DTYPE_FLOAT32;
}

// The layer-major kernel moves rows in whole 1 KiB chunks per wave and reads
// each token's deltas from the caller's workspace.
bool table_fits(const ll_kv_link_args *a) {
  return staging_fits(a) && (a->num_heads * a->key_head_dim) % 512 == 0 && a->delta_workspace != nullptr &&
         aligned16(a->delta_workspace) && a->delta_workspace_bytes / 4 / a->rotary_dim >= a->num_tokens;
}

// Launch shape of the vector kernel.  Short runs of layers per wave keep the
// GPU's in-flight rows within few layer buffers at a time.  Measured on gfx950
// (random 1 KB rows, interleaved A/B in one process): 4 layers per wave beats
// one wave walking all 28 layers by 2-8 % and 2 layers per wave by 1-3 %, and
// by 12 % when links share source blocks; on one of the boxes measured, 2 was
// 1.8 % ahead of 4 on the 32k-token link.  Links too small to fill the GPU
// with such waves are split to about kTargetWaves waves instead.
constexpr long long kTargetWaves = 16384;  // 64 waves per CU on 256 CUs
constexpr int kDefaultLayersPerWave = 4;

int plan_link(const ll_kv_link_args *a, LinkPlan *plan) {
  const bool fits = vector_kernel_fits(a);
  if (a->kernel == LL_KERNEL_VECTOR && !fits)
    return fail(LL_ERR_UNSUPPORTED_KERNEL,
                "vector kernel needs key_head_dim == value_head_dim in {32,64,128,256}, "
                "rotary_dim equal to it or half of it, one index type for the four token maps, a unit-stride "
                "cache with 16-byte aligned rows and 16-byte aligned buffers");
  plan->kernel = (a->kernel == LL_KERNEL_GENERIC || !fits) ? LL_KERNEL_GENERIC : LL_KERNEL_VECTOR;
  const int waves_per_block =
      a->waves_per_block && a->delta_staging != LL_DELTA_WORKGROUP ? static_cast<int>(a->waves_per_block) : 4;
  plan->block_threads = waves_per_block * kWave;
  const int layers_first = static_cast<int>(
      a->num_layers < kMaxLayersPerLaunch ? a->num_layers : kMaxLayersPerLaunch);
  plan->launches = static_cast<int>((a->num_layers + kMaxLayersPerLaunch - 1) / kMaxLayersPerLaunch);
  if (plan->kernel == LL_KERNEL_VECTOR) {
    const long long chunks = a->num_heads * a->key_head_dim / 8;
    const long long waves_x = (a->num_tokens * chunks + kWave - 1) / kWave;
    const int groups_per_block =
        a->layer_groups_per_block ? static_cast<int>(a->layer_groups_per_block) : 1;
    plan->layer_groups_per_block = groups_per_block;
    const int chunk_waves_per_block = waves_per_block / groups_per_block;
    plan->grid_x = (waves_x + chunk_waves_per_block - 1) / chunk_waves_per_block;
    int lpw = static_cast<int>(a->layers_per_wave);
    if (lpw == 0) {
      if (waves_x * ((layers_first + kDefaultLayersPerWave - 1) / kDefaultLayersPerWave) >=
          kTargetWaves) {
        lpw = kDefaultLayersPerWave;
      } else {
        long long groups = (kTargetWaves + waves_x - 1) / waves_x;
        if (groups > layers_first) groups = layers_first;
        lpw = static_cast<int>((layers_first + groups - 1) / groups);
      }
    }
    if (lpw > layers_first) lpw = layers_first;
    plan->layers_per_wave = lpw;
    plan->staged = false;
    plan->layer_major = false;
    // The delta table and the layer-major passes on request only: against
    // the staged workgroups they gain 12 % on contiguous rows, but lose
    // 1.4-2.0 % on the executor's own c2, c4 and c5 maps and 0.3-2.1 % on
    // rows in runs of 4-64 slots.
    if (a->delta_staging == LL_DELTA_TABLE && table_fits(a)) {
      const long long pairs = (a->num_tokens + 1) / 2;
      const long long waves = pairs * (chunks / kWave) * layers_first;
      plan->layer_major = true;
      plan->block_threads = kLayerMajorWaves * kWave;
      plan->grid_x = (waves + kLayerMajorWaves - 1) / kLayerMajorWaves;
      plan->layers_per_wave = 1;
      plan->layer_groups_per_block = 1;
      return plan->grid_x > 0x7fffffffLL ? fail(LL_ERR_LAUNCH_CONFIG, "link too large for one grid") : LL_OK;
    }
    // By default, staged deltas where they fit and the source rows are
    // streamed (read once, beyond the caches): there they cut the table reads
    // from one per token and layer group to one per token (c2 reads 1.094x ->
    // 1.018x the row bytes) and the DRAM-bound link gains 0.4-2 % (c2, c4, c5).
    // Links whose rows come partly from cache (batched requests sharing
    // blocks) run faster with per-wave deltas (c3: 8.34 against 8.91 ms).  An
    // explicit layer_groups_per_block asks for per-wave deltas.
    const bool want_staged =
        a->delta_staging == LL_DELTA_WORKGROUP ||
        ((a->delta_staging == LL_DELTA_AUTO || a->delta_staging == LL_DELTA_TABLE) &&
         a->layer_groups_per_block == 0 && a->stream_source_rows != 0);
    if (want_staged && staging_fits(a)) {
      // Every layer group of a token in one workgroup: G groups of
      // layers_per_wave layers (at most 16, so lpw grows for deep models),
      // times as many chunk-waves as fit in the wave budget and the LDS table.
      int groups = (layers_first + lpw - 1) / lpw;
      if (groups > kMaxWavesPerBlock) {
        lpw = (layers_first + kMaxWavesPerBlock - 1) / kMaxWavesPerBlock;
        plan->layers_per_wave = lpw;
        groups = (layers_first + lpw - 1) / lpw;
      }
      const int budget = a->delta_staging == LL_DELTA_WORKGROUP && a->waves_per_block
                             ? static_cast<int>(a->waves_per_block) : kMaxWavesPerBlock;
      int chunk_waves = budget / groups;
      const long long row_chunks = chunks;
      while (chunk_waves > 1 &&
             (chunk_waves * kWave + row_chunks - 1) / row_chunks + 1 > kMaxStagedTokens)
        --chunk_waves;
      if (chunk_waves >= 1 && (chunk_waves * kWave + row_chunks - 1) / row_chunks + 1 <= kMaxStagedTokens) {
        plan->staged = true;
        plan->layer_groups_per_block = groups;
        plan->block_threads = chunk_waves * groups * kWave;
        plan->grid_x = (waves_x + chunk_waves - 1) / chunk_waves;
      }
    }
  } else {
    plan->grid_x = a->num_tokens < 65536 ? a->num_tokens : 65536;
    plan->layers_per_wave = 1;
    plan->layer_groups_per_block = 1;
    plan->staged = false;
    plan->layer_major = false;
  }
  if (plan->grid_x > 0x7fffffffLL) return fail(LL_ERR_LAUNCH_CONFIG, "link too large for one grid");
  return LL_OK;
}

template <bool kBF16, int kD, int kR, int kCache, bool kStream, bool kEager, bool kStaged>
void launch_vec_index(dim3 grid, dim3 block, hipStream_t s, const LinkParams &p, bool neox) {
  const bool index64 = (p.idx64 & 15) == 15;  // the vector kernel needs one index type
  if constexpr (kStaged) {  // neox only (the plan checks)
    if (index64)
      kv_link_vec_kernel<kBF16, kD, kR, true, long long, kCache, kStream, kEager, true><<<grid, block, 0, s>>>(p);
    else
      kv_link_vec_kernel<kBF16, kD, kR, true, int, kCache, kStream, kEager, true><<<grid, block, 0, s>>>(p);
  } else if (neox) {
    if (index64)
      kv_link_vec_kernel<kBF16, kD, kR, true, long long, kCache, kStream, kEager, false><<<grid, block, 0, s>>>(p);
    else
      kv_link_vec_kernel<kBF16, kD, kR, true, int, kCache, kStream, kEager, false><<<grid, block, 0, s>>>(p);
  } else {
    if (index64)
      kv_link_vec_kernel<kBF16, kD, kR, false, long long, kCache, kStream, kEager, false><<<grid, block, 0, s>>>(p);
    else
      kv_link_vec_kernel<kBF16, kD, kR, false, int, kCache, kStream, kEager, false><<<grid, block, 0, s>>>(p);
  }
}

// Streamed (non-temporal) row loads and workgroup-staged deltas are built for
// the full-rotary fp32-table kernels only, the production shape; other shapes
// load rows as usual and compute deltas per wave.
template <bool kBF16, int kD, int kR, int kCache, bool kEager>
void launch_vec_neox(dim3 grid, dim3 block, hipStream_t s, const LinkParams &p, bool neox) {
  if constexpr (kR == kD && kCache == 3) {
    if (p.staged) {
      if (p.stream_rows) launch_vec_index<kBF16, kD, kR, kCache, true, kEager, true>(grid, block, s, p, neox);
      else launch_vec_index<kBF16, kD, kR, kCache, false, kEager, true>(grid, block, s, p, neox);
      return;
    }
    if (p.stream_rows) {
      launch_vec_index<kBF16, kD, kR, kCache, true, kEager, false>(grid, block, s, p, neox);
      return;
    }
  }
  launch_vec_index<kBF16, kD, kR, kCache, false, kEager, false>(grid, block, s, p, neox);
}

template <bool kBF16, int kD, int kCache, bool kEager>
void launch_vec_rotary(dim3 grid, dim3 block, hipStream_t s, const LinkParams &p, bool neox) {
  if (p.rotary_dim == kD) launch_vec_neox<kBF16, kD, kD, kCache, kEager>(grid, block, s, p, neox);
  else launch_vec_neox<kBF16, kD, kD / 2, kCache, kEager>(grid, block, s, p, neox);
}

template <bool kBF16, int kCache, bool kEager>
void launch_vec_dim(int d, dim3 grid, dim3 block, hipStream_t s, const LinkParams &p, bool neox) {
  switch (d) {
    case 32: launch_vec_rotary<kBF16, 32, kCache, kEager>(grid, block, s, p, neox); break;
    case 64: launch_vec_rotary<kBF16, 64, kCache, kEager>(grid, block, s, p, neox); break;
    case 128: launch_vec_rotary<kBF16, 128, kCache, kEager>(grid, block, s, p, neox); break;
    default: launch_vec_rotary<kBF16, 256, kCache, kEager>(grid, block, s, p, neox); break;
  }
}

template <bool kBF16, bool kEager>
void launch_vec_cache(int cache_dtype, int d, dim3 grid, dim3 block, hipStream_t s,
                      const LinkParams &p, bool neox) {
  switch (cache_dtype) {
    case LL_DTYPE_FLOAT32: launch_vec_dim<kBF16, 3, kEager>(d, grid, block, s, p, neox); break;
    case LL_DTYPE_BFLOAT16: launch_vec_dim<kBF16, 2, kEager>(d, grid, block, s, p, neox); break;
    default: launch_vec_dim<kBF16, 1, kEager>(d, grid, block, s, p, neox); break;
  }
}

template <bool kBF16>
void launch_vec(int cache_dtype, int d, dim3 grid, dim3 block, hipStream_t s, const LinkParams &p,
                bool neox) {
  if (p.eager) launch_vec_cache<kBF16, true>(cache_dtype, d, grid, block, s, p, neox);
  else launch_vec_cache<kBF16, false>(cache_dtype, d, grid, block, s, p, neox);
}

// Layer-major link: per launch of <= 64 layers, the value pass (the first
// one also writing the delta table) and then the key pass.
template <bool kBF16, int kD, typename Index, bool kEager>
void launch_layer_major_typed(dim3 grid, hipStream_t s, const LinkParams &p) {
  const dim3 block(kLayerMajorWaves * kWave);
  if (p.stream_rows) {
    kv_link_layer_kernel<kBF16, kD, Index, true, kEager, false><<<grid, block, 0, s>>>(p);
    kv_link_layer_kernel<kBF16, kD, Index, true, kEager, true><<<grid, block, 0, s>>>(p);
  } else {
    kv_link_layer_kernel<kBF16, kD, Index, false, kEager, false><<<grid, block, 0, s>>>(p);
    kv_link_layer_kernel<kBF16, kD, Index, false, kEager, true><<<grid, block, 0, s>>>(p);
  }
}

template <bool kBF16, int kD, bool kEager>
void launch_layer_major_index(dim3 grid, hipStream_t s, const LinkParams &p) {
  const bool index64 = (p.idx64 & 15) == 15;  // one index type for the four maps (the plan checks)
  if (index64) launch_layer_major_typed<kBF16, kD, long long, kEager>(grid, s, p);
  else launch_layer_major_typed<kBF16, kD, int, kEager>(grid, s, p);
}

template <bool kBF16, bool kEager>
void launch_layer_major_dim(dim3 grid, hipStream_t s, const LinkParams &p) {
  switch (p.kdim) {
    case 32: launch_layer_major_index<kBF16, 32, kEager>(grid, s, p); break;
    case 64: launch_layer_major_index<kBF16, 64, kEager>(grid, s, p); break;
    case 128: launch_layer_major_index<kBF16, 128, kEager>(grid, s, p); break;
    default: launch_layer_major_index<kBF16, 256, kEager>(grid, s, p); break;
  }
}

void launch_layer_major(bool bf16, dim3 grid, hipStream_t s, const LinkParams &p) {
  if (bf16) {
    if (p.eager) launch_layer_major_dim<true, true>(grid, s, p);
    else launch_layer_major_dim<true, false>(grid, s, p);
  } else {
    if (p.eager) launch_layer_major_dim<false, true>(grid, s, p);
    else launch_layer_major_dim<false, false>(grid, s, p);
  }
}

template <int kKey, bool kEager>
void launch_generic_cache(int cache_dtype, dim3 grid, dim3 block, hipStream_t s,
                          const LinkParams &p) {
  switch (cache_dtype) {
    case LL_DTYPE_FLOAT32: kv_link_generic_kernel<kKey, 3, kEager><<<grid, block, 0, s>>>(p); break;
    case LL_DTYPE_BFLOAT16: kv_link_generic_kernel<kKey, 2, kEager><<<grid, block, 0, s>>>(p); break;
    default: kv_link_generic_kernel<kKey, 1, kEager><<<grid, block, 0, s>>>(p); break;
  }
}

template <int kKey>
void launch_generic(int cache_dtype, dim3 grid, dim3 block, hipStream_t s, const LinkParams &p) {
  if (p.eager) launch_generic_cache<kKey, true>(cache_dtype, grid, block, s, p);
  else launch_generic_cache<kKey, false>(cache_dtype, grid, block, s, p);
}

// Host scratch of the run planner, kept per thread so that repeated plans
// reuse its capacity instead of mapping fresh pages on every call.
struct PlanScratch {
  struct Seg { int64_t block, a, b, rb, re; };
  struct Run { int64_t first, last; };  // consecutive repair positions, inclusive
  struct Hit { int64_t begin, end; };   // a block's repair offsets [begin, end)
  std::vector<int64_t> dstart, offset, positions, by_start, hit_block, bucket, fill, map_offset;
  std::vector<Run> runs;
  std::vector<Hit> hits, block_hits;
  std::vector<Seg> segs;
};

PlanScratch &plan_scratch() {
  thread_local PlanScratch scratch_space;
  return scratch_space;
}

}  // namespace

int ll_record_error(int code, const char *fmt, va_list ap) {
  char buf[512];
  vsnprintf(buf, sizeof(buf), fmt, ap);
  g_last_error = buf;
  return code;
}

extern "C" {

int ll_abi_version(void) { return LL_ABI_VERSION; }
int64_t ll_kv_link_args_size(void) { return static_cast<int64_t>(sizeof(ll_kv_link_args)); }
int64_t ll_kv_scatter_args_size(void) { return static_cast<int64_t>(sizeof(ll_kv_scatter_args)); }
int64_t ll_link_maps_args_size(void) { return static_cast<int64_t>(sizeof(ll_link_maps_args)); }
const char *ll_last_error(void) { return g_last_error.c_str(); }

const char *ll_status_reason(int status) {
  switch (status) {
    case LL_OK: return "supported";
    case LL_ERR_INVALID_ARGUMENT: return "invalid_argument";
    case LL_ERR_MHA_3D_KV_BUFFERS_REQUIRED: return "mha_3d_kv_buffers_required";
    case LL_ERR_KV_HEAD_LAYOUT_MISMATCH: return "kv_head_layout_mismatch";
    case LL_ERR_KV_DTYPE_MISMATCH: return "kv_dtype_mismatch";
    case LL_ERR_FP16_OR_BF16_REQUIRED: return "fp16_or_bf16_required";
    case LL_ERR_CONTIGUOUS_KV_BUFFERS_REQUIRED: return "contiguous_kv_buffers_required";
    case LL_ERR_HEAD_DIMENSION_OUT_OF_RANGE: return "head_dimension_out_of_range";
    case LL_ERR_EMPTY_LINK: return "empty_link";
    case LL_ERR_TOKEN_MAP_LENGTH_MISMATCH: return "token_map_length_mismatch";
    case LL_ERR_REPAIR_MASK_LENGTH_MISMATCH: return "repair_mask_length_mismatch";
    case LL_ERR_BOOLEAN_REPAIR_MASK_REQUIRED: return "boolean_repair_mask_required";
    case LL_ERR_INTEGER_TOKEN_MAPS_REQUIRED: return "integer_token_maps_required";
    case LL_ERR_EVEN_ROTARY_DIM_REQUIRED: return "even_rotary_dim_required";
    case LL_ERR_ROTARY_DIM_EXCEEDS_HEAD_DIM: return "rotary_dim_exceeds_head_dim";
    case LL_ERR_UNSUPPORTED_COS_SIN_CACHE: return "unsupported_cos_sin_cache";
    case LL_ERR_UNSUPPORTED_COS_SIN_DTYPE: return "unsupported_cos_sin_dtype";
    case LL_ERR_PREFIX_OUT_OF_RANGE: return "prefix_token_count_out_of_range";
    case LL_ERR_LAUNCH_CONFIG: return "invalid_launch_config";
    case LL_ERR_UNSUPPORTED_KERNEL: return "unsupported_kernel_for_shape";
    case LL_ERR_HIP: return "hip_error";
    default: return "unknown_status";
  }
}

int ll_kv_link_describe(const ll_kv_link_args *args, ll_launch_info *info) {
  int rc = validate_link(args);
  if (rc != LL_OK) return rc;
  if (info == nullptr) return fail(LL_ERR_INVALID_ARGUMENT, "info is NULL");
  LinkPlan plan;
  rc = plan_link(args, &plan);
  if (rc != LL_OK) return rc;
  const int layers_first = static_cast<int>(
      args->num_layers < kMaxLayersPerLaunch ? args->num_layers : kMaxLayersPerLaunch);
  info->kernel = plan.kernel;
  info->launches = plan.launches;
  info->grid_x = plan.grid_x;
  const int layer_groups = (layers_first + plan.layers_per_wave - 1) / plan.layers_per_wave;
  info->grid_y = plan.kernel == LL_KERNEL_VECTOR
                     ? (layer_groups + plan.layer_groups_per_block - 1) / plan.layer_groups_per_block
                     : layers_first;
  info->block_threads = plan.block_threads;
  info->layers_per_wave = plan.layers_per_wave;
  info->layer_groups_per_block = plan.layer_groups_per_block;
  info->delta_staging = plan.kernel != LL_KERNEL_VECTOR
                            ? 0
                            : (plan.layer_major ? LL_DELTA_TABLE : (plan.staged ? LL_DELTA_WORKGROUP : LL_DELTA_PER_WAVE));
  if (plan.layer_major) info->grid_y = 1;
  return LL_OK;
}

int ll_kv_link(const ll_kv_link_args *a, ll_stream_t stream) {
  int rc = validate_link(a);
  if (rc != LL_OK) return rc;
  LinkPlan plan;
  rc = plan_link(a, &plan);
  if (rc != LL_OK) return rc;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);

  LinkParams p;
  memset(&p, 0, sizeof(p));
  p.src = a->source_slots;
  p.dst = a->destination_slots;
  p.lpos = a->local_positions;
  p.gpos = a->global_positions;
  p.mask = static_cast<const unsigned char *>(a->repair_mask);
  p.cs = a->cos_sin_cache;
  p.num_tokens = a->num_tokens;
  p.num_slots = a->num_slots;
  p.src_num_slots = a->source_key_layers != nullptr ? a->source_num_slots : a->num_slots;
  p.stream_rows = a->stream_source_rows != 0 ? 1 : 0;
  p.eager = a->rounding == LL_ROUNDING_EAGER ? 1 : 0;
  p.staged = plan.staged ? 1 : 0;
  p.skipped = reinterpret_cast<unsigned long long *>(a->skipped_rows);
  p.delta_table = plan.layer_major ? static_cast<f32x2 *>(a->delta_workspace) : nullptr;
  p.cs_rows = a->cos_sin_rows;
  p.cs_stride_row = a->cos_sin_stride_row;
  p.cs_stride_col = a->cos_sin_stride_col;
  p.prefix = a->prefix_token_count;
  p.k_row_bytes = a->num_heads * a->key_head_dim * 2;
  p.v_row_bytes = a->num_heads * a->value_head_dim * 2;
  p.chunks_per_row = a->num_heads * a->key_head_dim / 8;
  p.num_heads = static_cast<int>(a->num_heads);
  p.kdim = static_cast<int>(a->key_head_dim);
  p.vdim = static_cast<int>(a->value_head_dim);
  p.rotary_dim = static_cast<int>(a->rotary_dim);
  p.idx64 = (a->source_slots_dtype == LL_DTYPE_INT64 ? 1 : 0) |
            (a->destination_slots_dtype == LL_DTYPE_INT64 ? 2 : 0) |
            (a->local_positions_dtype == LL_DTYPE_INT64 ? 4 : 0) |
            (a->global_positions_dtype == LL_DTYPE_INT64 ? 8 : 0);
  p.neox = a->is_neox_style ? 1 : 0;
  const bool bf16 = a->kv_dtype == LL_DTYPE_BFLOAT16;
  const dim3 block(plan.block_threads);
  // Every slot index is out of range for an empty pool: every token is
  // skipped, and no kernel runs (the vector kernel reads row 0 of the source
  // pool unconditionally), so none could be counted.
  if (p.src_num_slots == 0 || p.num_slots == 0) {
    if (a->skipped_rows != nullptr)
      return fail(LL_ERR_INVALID_ARGUMENT, "skipped_rows is set and a pool has no rows");
    return LL_OK;
  }

  p.write_table = plan.layer_major ? 1 : 0;
  for (int64_t base = 0; base < a->num_layers; base += kMaxLayersPerLaunch) {
    const int n = static_cast<int>(a->num_layers - base < kMaxLayersPerLaunch
                                       ? a->num_layers - base
                                       : kMaxLayersPerLaunch);
    for (int l = 0; l < n; ++l) {
      p.k_layers[l] = static_cast<char *>(a->key_layers[base + l]);
      p.v_layers[l] = static_cast<char *>(a->value_layers[base + l]);
      const bool own = a->source_key_layers == nullptr;
      p.sk_layers[l] = static_cast<const char *>(own ? a->key_layers[base + l]
                                                      : a->source_key_layers[base + l]);
      p.sv_layers[l] = static_cast<const char *>(own ? a->value_layers[base + l]
                                                      : a->source_value_layers[base + l]);
    }
    p.num_layers = n;
    if (plan.layer_major) {
      const long long pairs = (p.num_tokens + 1) / 2;
      const long long waves = pairs * (p.chunks_per_row / kWave) * n;
      const dim3 grid(static_cast<unsigned>((waves + kLayerMajorWaves - 1) / kLayerMajorWaves));
      launch_layer_major(bf16, grid, s, p);
      p.write_table = 0;  // the first launch's value pass wrote it
    } else if (plan.kernel == LL_KERNEL_VECTOR) {
      const int lpw = plan.layers_per_wave < n ? plan.layers_per_wave : n;
      p.layers_per_wave = lpw;
      p.layer_groups_per_block = plan.layer_groups_per_block;
      const int layer_groups = (n + lpw - 1) / lpw;
      const dim3 grid(static_cast<unsigned>(plan.grid_x),
                      static_cast<unsigned>((layer_groups + plan.layer_groups_per_block - 1) /
                                            plan.layer_groups_per_block));
      const int cache = static_cast<int>(a->cos_sin_dtype);
      if (bf16) launch_vec<true>(cache, p.kdim, grid, block, s, p, p.neox != 0);
      else launch_vec<false>(cache, p.kdim, grid, block, s, p, p.neox != 0);
    } else {
      p.layers_per_wave = 1;
      p.layer_groups_per_block = 1;
      const dim3 grid(static_cast<unsigned>(plan.grid_x), static_cast<unsigned>(n));
      if (bf16) launch_generic<2>(static_cast<int>(a->cos_sin_dtype), grid, block, s, p);
      else launch_generic<1>(static_cast<int>(a->cos_sin_dtype), grid, block, s, p);
    }
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess)
      return fail(LL_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(err));
    p.skipped = nullptr;  // later launches see the same tokens: count them once
  }
  return LL_OK;
}

int ll_kv_scatter_rows(const ll_kv_scatter_args *a, ll_stream_t stream) {
  if (a == nullptr) return fail(LL_ERR_INVALID_ARGUMENT, "args is NULL");
  if (a->struct_size != static_cast<int64_t>(sizeof(ll_kv_scatter_args)))
    return fail(LL_ERR_INVALID_ARGUMENT, "struct_size %lld != %zu",
                static_cast<long long>(a->struct_size), sizeof(ll_kv_scatter_args));
  if (a->num_layers < 1 || a->key_layers == nullptr || a->value_layers == nullptr)
    return fail(LL_ERR_INVALID_ARGUMENT, "num_layers must be >= 1 with key/value layer tables");
  for (int64_t l = 0; l < a->num_layers; ++l)
    if (a->key_layers[l] == nullptr || a->value_layers[l] == nullptr)
      return fail(LL_ERR_INVALID_ARGUMENT, "layer %lld buffer is NULL", static_cast<long long>(l));
  if (a->num_slots < 0 || a->num_rows < 0)
    return fail(LL_ERR_INVALID_ARGUMENT, "num_slots and num_rows must be >= 0");
  if (a->num_heads < 1)
    return fail(LL_ERR_MHA_3D_KV_BUFFERS_REQUIRED, "num_heads must be >= 1");
  if (a->kv_dtype != LL_DTYPE_BFLOAT16 && a->kv_dtype != LL_DTYPE_FLOAT16)
    return fail(LL_ERR_FP16_OR_BF16_REQUIRED, "kv_dtype must be fp16 or bf16");
  if (a->key_head_dim < 1 || a->value_head_dim < 1 || a->key_head_dim > 256 ||
      a->value_head_dim > 256)
    return fail(LL_ERR_HEAD_DIMENSION_OUT_OF_RANGE, "head dims must be in 1..256");
  if (a->waves_per_block != 0 && a->waves_per_block != 1 && a->waves_per_block != 2 &&
      a->waves_per_block != 4 && a->waves_per_block != 8)
    return fail(LL_ERR_LAUNCH_CONFIG, "waves_per_block must be 0, 1, 2, 4 or 8");
  if (a->num_rows == 0) return LL_OK;
  if (a->destination_slots == nullptr || a->repaired_key == nullptr ||
      a->repaired_value == nullptr)
    return fail(LL_ERR_INVALID_ARGUMENT, "destination_slots / repaired rows pointer is NULL");
  if (!is_index_dtype(a->destination_slots_dtype))
    return fail(LL_ERR_INTEGER_TOKEN_MAPS_REQUIRED, "destination slots must be int32 or int64");
  if (a->repaired_key_layer_stride < 0 || a->repaired_value_layer_stride < 0)
    return fail(LL_ERR_INVALID_ARGUMENT, "repaired layer strides must be >= 0");

  ScatterParams p;
  memset(&p, 0, sizeof(p));
  p.dst = a->destination_slots;
  p.rk = static_cast<const char *>(a->repaired_key);
  p.rv = static_cast<const char *>(a->repaired_value);
  p.num_rows = a->num_rows;
  p.num_slots = a->num_slots;
  p.rk_layer_stride_bytes = a->repaired_key_layer_stride * 2;
  p.rv_layer_stride_bytes = a->repaired_value_layer_stride * 2;
  p.k_row_bytes = a->num_heads * a->key_head_dim * 2;
  p.v_row_bytes = a->num_heads * a->value_head_dim * 2;
  p.idx64 = a->destination_slots_dtype == LL_DTYPE_INT64 ? 2 : 0;

  bool vec = (p.k_row_bytes % 16) == 0 && (p.v_row_bytes % 16) == 0 &&
             (p.rk_layer_stride_bytes % 16) == 0 && (p.rv_layer_stride_bytes % 16) == 0 &&
             aligned16(p.rk) && aligned16(p.rv);
  for (int64_t l = 0; l < a->num_layers && vec; ++l)
    vec = aligned16(a->key_layers[l]) && aligned16(a->value_layers[l]);
  const long long chunk = vec ? 16 : 2;
  const long long items = a->num_rows * (p.k_row_bytes + p.v_row_bytes) / chunk;
  const int waves_per_block = a->waves_per_block ? static_cast<int>(a->waves_per_block) : 4;
  const int threads = waves_per_block * kWave;
  long long gx = (items + threads - 1) / threads;
  if (gx > 65536) gx = 65536;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);

  for (int64_t base = 0; base < a->num_layers; base += kMaxLayersPerLaunch) {
    const int n = static_cast<int>(a->num_layers - base < kMaxLayersPerLaunch
                                       ? a->num_layers - base
                                       : kMaxLayersPerLaunch);
    for (int l = 0; l < n; ++l) {
      p.k_layers[l] = static_cast<char *>(a->key_layers[base + l]);
      p.v_layers[l] = static_cast<char *>(a->value_layers[base + l]);
    }
    // Staged rows of layer base + l start at (base + l) * stride.
    ScatterParams q = p;
    q.rk = p.rk + base * p.rk_layer_stride_bytes;
    q.rv = p.rv + base * p.rv_layer_stride_bytes;
    const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(n));
    if (vec) kv_scatter_kernel<u32x4><<<grid, dim3(threads), 0, s>>>(q);
    else kv_scatter_kernel<uint16_t><<<grid, dim3(threads), 0, s>>>(q);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess)
      return fail(LL_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(err));
  }
  return LL_OK;
}

int ll_plan_link_runs(const ll_link_block *blocks, int64_t num_blocks, const int64_t *repair_positions,
                      int64_t num_repair_positions, int64_t compact, ll_link_segment *segments,
                      int64_t segment_capacity, int64_t *segment_blocks, int64_t *repair_offsets,
                      int64_t repair_offsets_capacity, ll_link_run_plan_info *info) {
  if (info == nullptr) return fail(LL_ERR_INVALID_ARGUMENT, "info is NULL");
  if (num_blocks < 0 || (num_blocks > 0 && blocks == nullptr))
    return fail(LL_ERR_INVALID_ARGUMENT, "blocks must be a host array of num_blocks >= 0 entries");
  if (num_repair_positions < 0 || (num_repair_positions > 0 && repair_positions == nullptr))
    return fail(LL_ERR_INVALID_ARGUMENT, "repair_positions must be a host array of >= 0 entries");
  if (segment_capacity < 0 || repair_offsets_capacity < 0)
    return fail(LL_ERR_INVALID_ARGUMENT, "capacities must be >= 0");
  constexpr int64_t kLimit = static_cast<int64_t>(1) << 62;
  PlanScratch &w = plan_scratch();
  // Destination index of every block's first token, and its concatenation
  // offset (blocks back to back in plan order).
  std::vector<int64_t> &dstart = w.dstart, &offset = w.offset;
  dstart.resize(static_cast<size_t>(num_blocks));
  offset.resize(static_cast<size_t>(num_blocks));
  int64_t total = 0;
  for (int64_t b = 0; b < num_blocks; ++b) {
    const ll_link_block &k = blocks[b];
    // Both starts below 2^62 keep their sum, and every position difference
    // taken from it, inside int64.
    if (k.token_count < 0 || k.token_count > 0x7fffffff || k.start_token < 0 || k.start_token >= kLimit ||
        k.destination_base < 0 || k.destination_base >= kLimit || (k.map_set != 0 && k.map_set != 1) ||
        total > kLimit - k.token_count)
      return fail(LL_ERR_INVALID_ARGUMENT, "block %lld: token_count in [0, 2^31), start_token and "
                  "destination_base in [0, 2^62), map_set 0 or 1", static_cast<long long>(b));
    dstart[static_cast<size_t>(b)] = k.start_token + k.destination_base;
    offset[static_cast<size_t>(b)] = total;
    total += k.token_count;
  }
  // Repair positions as runs of consecutive positions [first, last], sorted
  // and without duplicates.  Plans list them in increasing order, in runs
  // (a seam's imp_indices); other inputs are sorted first.
  std::vector<PlanScratch::Run> &runs = w.runs;
  auto find_runs = [&runs](const int64_t *p, int64_t n) {  // false where p is not increasing
    runs.clear();
    for (int64_t i = 0; i < n;) {
      int64_t j = i;
      while (j + 1 < n && p[j] != INT64_MAX && p[j + 1] == p[j] + 1) ++j;
      if (j + 1 < n && p[j + 1] <= p[j]) return false;
      runs.push_back(PlanScratch::Run{p[i], p[j]});
      i = j + 1;
    }
    return true;
  };
  if (!find_runs(repair_positions, num_repair_positions)) {
    std::vector<int64_t> &positions = w.positions;
    positions.assign(repair_positions, repair_positions + num_repair_positions);
    std::sort(positions.begin(), positions.end());
    positions.erase(std::unique(positions.begin(), positions.end()), positions.end());
    find_runs(positions.data(), static_cast<int64_t>(positions.size()));
  }
  std::vector<int64_t> &by_start = w.by_start;
  by_start.resize(static_cast<size_t>(num_blocks));
  for (int64_t b = 0; b < num_blocks; ++b) by_start[static_cast<size_t>(b)] = b;
  // Plans lay their blocks out in position order; sort only when they do not.
  const bool in_order = std::is_sorted(dstart.begin(), dstart.end());
  if (!in_order)
    std::stable_sort(by_start.begin(), by_start.end(), [&](int64_t x, int64_t y) {
      return dstart[static_cast<size_t>(x)] < dstart[static_cast<size_t>(y)];
    });
  // Each position belongs to the last block starting at or before it, if it
  // lies inside that block: block by_start[k] holds the positions of
  // [its start, min(its end, the next block's start)).  One walk over the
  // blocks in start order and the runs gives each block's repair runs as
  // offset ranges [begin, end), increasing.  They are then bucketed by block
  // (counting sort) when the blocks are not in start order.
  std::vector<PlanScratch::Hit> &hits = w.hits;
  std::vector<int64_t> &hit_block = w.hit_block;
  hits.clear();
  hit_block.clear();
  size_t r = 0;
  for (size_t k = 0; k < by_start.size() && r < runs.size(); ++k) {
    const int64_t b = by_start[k];
    const int64_t first = dstart[static_cast<size_t>(b)];
    int64_t owned_end = first + blocks[b].token_count;
    if (k + 1 < by_start.size()) {
      const int64_t next = dstart[static_cast<size_t>(by_start[k + 1])];
      owned_end = next < owned_end ? next : owned_end;
    }
    while (r < runs.size() && runs[r].last < first) ++r;
    for (size_t q = r; q < runs.size() && runs[q].first < owned_end; ++q) {
      const int64_t lo = runs[q].first > first ? runs[q].first : first;
      const int64_t hi = runs[q].last < owned_end - 1 ? runs[q].last : owned_end - 1;
      if (lo > hi) continue;
      hits.push_back(PlanScratch::Hit{lo - first, hi - first + 1});
      hit_block.push_back(b);
    }
  }
  std::vector<int64_t> &bucket = w.bucket, &fill = w.fill;
  bucket.assign(static_cast<size_t>(num_blocks) + 1, 0);
  for (const int64_t b : hit_block) ++bucket[static_cast<size_t>(b) + 1];
  for (size_t b = 0; b < static_cast<size_t>(num_blocks); ++b) bucket[b + 1] += bucket[b];
  std::vector<PlanScratch::Hit> &block_hits = w.block_hits;
  if (in_order) {
    block_hits.swap(hits);  // hits of blocks in position order come grouped by block
  } else {
    block_hits.resize(hits.size());  // grouped by block, increasing within each
    fill.assign(bucket.begin(), bucket.end() - 1);
    for (size_t i = 0; i < hits.size(); ++i)
      block_hits[static_cast<size_t>(fill[static_cast<size_t>(hit_block[i])]++)] = hits[i];
  }
  // Segments in plan order: a block's repair runs cut it; segment j of a
  // block spans [first ? 0 : begin_j, last ? count : begin_{j+1}) and holds
  // repair run j.
  std::vector<PlanScratch::Seg> &segs = w.segs;
  segs.clear();
  for (int64_t b = 0; b < num_blocks; ++b) {
    const PlanScratch::Hit *h = block_hits.data() + bucket[static_cast<size_t>(b)];
    const int64_t count_hits = bucket[static_cast<size_t>(b) + 1] - bucket[static_cast<size_t>(b)];
    const int64_t count = blocks[b].token_count;
    if (count_hits == 0) {
      if (count > 0) segs.push_back(PlanScratch::Seg{b, 0, count, 0, 0});
      continue;
    }
    for (int64_t i = 0; i < count_hits; ++i) {
      const int64_t a = i == 0 ? 0 : h[i].begin;
      const int64_t e = i + 1 == count_hits ? count : h[i + 1].begin;
      segs.push_back(PlanScratch::Seg{b, a, e, h[i].begin - a, h[i].end - a});
    }
  }
  const int64_t n = static_cast<int64_t>(segs.size());
  // Map offsets per set: the identity (leading) blocks' runs first, then the
  // others, each in plan order.  Repair rows are numbered in plan order.
  int64_t map_count[2] = {0, 0}, set_repair[2] = {0, 0}, set_prefix[2] = {0, 0};
  std::vector<int64_t> &map_offset = w.map_offset;
  map_offset.resize(static_cast<size_t>(n));
  for (int pass = 0; pass < 2; ++pass) {
    for (int64_t i = 0; i < n; ++i) {
      const PlanScratch::Seg &g = segs[static_cast<size_t>(i)];
      const bool lead = blocks[g.block].leading != 0;
      if (lead != (pass == 0)) continue;
      const int set = static_cast<int>(blocks[g.block].map_set);
      const int64_t entries = (g.b - g.a) - (compact ? g.re - g.rb : 0);
      map_offset[static_cast<size_t>(i)] = map_count[set];
      map_count[set] += entries;
      set_repair[set] += g.re - g.rb;
      if (lead) set_prefix[set] += entries;
    }
  }
  int64_t repair_count = 0;
  for (const PlanScratch::Seg &g : segs) repair_count += g.re - g.rb;
  info->num_segments = n;
  info->map_count[0] = map_count[0];
  info->map_count[1] = map_count[1];
  info->set_repair_rows[0] = set_repair[0];
  info->set_repair_rows[1] = set_repair[1];
  info->set_prefix[0] = set_prefix[0];
  info->set_prefix[1] = set_prefix[1];
  info->repair_count = repair_count;
  if (segments == nullptr && segment_blocks == nullptr && repair_offsets == nullptr) return LL_OK;
  if (n > segment_capacity)
    return fail(LL_ERR_INVALID_ARGUMENT, "segment_capacity %lld is below the %lld runs",
                static_cast<long long>(segment_capacity), static_cast<long long>(n));
  if (repair_offsets != nullptr && repair_count > repair_offsets_capacity)
    return fail(LL_ERR_INVALID_ARGUMENT, "repair_offsets_capacity %lld is below the %lld repair rows",
                static_cast<long long>(repair_offsets_capacity), static_cast<long long>(repair_count));
  int64_t repair_seen = 0;
  for (int64_t i = 0; i < n; ++i) {
    const PlanScratch::Seg &g = segs[static_cast<size_t>(i)];
    const ll_link_block &k = blocks[g.block];
    if (segments != nullptr) {
      ll_link_segment &out = segments[i];
      out.source_slots = k.source_slots + g.a;
      out.local_positions = k.local_positions != nullptr ? k.local_positions + g.a : nullptr;
      out.token_count = g.b - g.a;
      out.start_token = k.start_token + g.a;
      out.destination_start = dstart[static_cast<size_t>(g.block)] + g.a;
      out.local_start = k.local_start + g.a;
      out.repair_begin = g.rb;
      out.repair_end = g.re;
      out.map_set = k.map_set;
      out.map_offset = map_offset[static_cast<size_t>(i)];
      out.repair_offset = repair_seen;
    }
    if (segment_blocks != nullptr) segment_blocks[i] = g.block;
    if (repair_offsets != nullptr)
      for (int64_t r = g.rb; r < g.re; ++r)
        repair_offsets[repair_seen + (r - g.rb)] = offset[static_cast<size_t>(g.block)] + g.a + r;
    repair_seen += g.re - g.rb;
  }
  return LL_OK;
}

int ll_kv_build_link_maps(const ll_link_maps_args *a, ll_stream_t stream) {
  if (a == nullptr) return fail(LL_ERR_INVALID_ARGUMENT, "args is NULL");
  if (a->struct_size != static_cast<int64_t>(sizeof(ll_link_maps_args)))
    return fail(LL_ERR_INVALID_ARGUMENT, "struct_size %lld != %zu",
                static_cast<long long>(a->struct_size), sizeof(ll_link_maps_args));
  if (a->num_segments < 0) return fail(LL_ERR_INVALID_ARGUMENT, "num_segments is negative");
  if (a->num_segments == 0) return LL_OK;
  if (a->segments == nullptr) return fail(LL_ERR_INVALID_ARGUMENT, "segments is NULL");
  if (!is_index_dtype(a->destination_slots_dtype))
    return fail(LL_ERR_INTEGER_TOKEN_MAPS_REQUIRED, "destination slots must be int32 or int64");
  if (a->num_destination_slots < 0)
    return fail(LL_ERR_INVALID_ARGUMENT, "num_destination_slots is negative");
  constexpr int64_t kIntMax = 0x7fffffff;
  for (int s = 0; s < 2; ++s)
    if (a->map_capacity[s] < 0 || a->map_capacity[s] > kIntMax)
      return fail(LL_ERR_INVALID_ARGUMENT, "map_capacity[%d] must be in [0, 2^31)", s);
  if (a->repair_capacity < 0) return fail(LL_ERR_INVALID_ARGUMENT, "repair_capacity is negative");

  // Validate every run before the first launch.
  for (int64_t k = 0; k < a->num_segments; ++k) {
    const ll_link_segment &g = a->segments[k];
    const long long kk = static_cast<long long>(k);
    if (g.token_count < 0 || g.token_count > kIntMax)
      return fail(LL_ERR_INVALID_ARGUMENT, "segment %lld: token_count out of range", kk);
    if (g.token_count == 0) continue;
    if (g.source_slots == nullptr)
      return fail(LL_ERR_INVALID_ARGUMENT, "segment %lld: source_slots is NULL", kk);
    if (a->destination_slots == nullptr)
      return fail(LL_ERR_INVALID_ARGUMENT, "destination_slots is NULL");
    if (g.destination_start < 0 || g.destination_start > a->num_destination_slots - g.token_count)
      return fail(LL_ERR_INVALID_ARGUMENT,
                  "segment %lld: destination indices [%lld, %lld) outside the %lld destination slots",
                  kk, static_cast<long long>(g.destination_start),
                  static_cast<long long>(g.destination_start + g.token_count),
                  static_cast<long long>(a->num_destination_slots));
    if (g.start_token < 0 || g.start_token > (static_cast<int64_t>(1) << 62))
      return fail(LL_ERR_INVALID_ARGUMENT, "segment %lld: start_token out of range", kk);
    if (g.repair_begin < 0 || g.repair_begin > g.repair_end || g.repair_end > g.token_count)
      return fail(LL_ERR_INVALID_ARGUMENT, "segment %lld: repair rows outside the run", kk);
    if (g.map_set != 0 && g.map_set != 1)
      return fail(LL_ERR_INVALID_ARGUMENT, "segment %lld: map_set must be 0 or 1", kk);
    const int set = static_cast<int>(g.map_set);
    const int64_t repair_rows = g.repair_end - g.repair_begin;
    const int64_t entries = g.token_count - (a->repair_mask[set] == nullptr ? repair_rows : 0);
    if (entries > 0) {
      if (a->maps[set] == nullptr)
        return fail(LL_ERR_INVALID_ARGUMENT, "segment %lld: maps[%d] is NULL", kk, set);
      if (g.map_offset < 0 || g.map_offset > a->map_capacity[set] - entries)
        return fail(LL_ERR_INVALID_ARGUMENT,
                    "segment %lld: map entries [%lld, %lld) outside capacity %lld", kk,
                    static_cast<long long>(g.map_offset),
                    static_cast<long long>(g.map_offset + entries),
                    static_cast<long long>(a->map_capacity[set]));
    }
    if (g.repair_offset < -1)
      return fail(LL_ERR_INVALID_ARGUMENT, "segment %lld: repair_offset must be >= -1", kk);
    if (repair_rows > 0 && g.repair_offset >= 0) {
      if (a->repair_destination_slots == nullptr)
        return fail(LL_ERR_INVALID_ARGUMENT, "repair_destination_slots is NULL");
      if (g.repair_offset > a->repair_capacity - repair_rows)
        return fail(LL_ERR_INVALID_ARGUMENT,
                    "segment %lld: repair rows [%lld, %lld) outside capacity %lld", kk,
                    static_cast<long long>(g.repair_offset),
                    static_cast<long long>(g.repair_offset + repair_rows),
                    static_cast<long long>(a->repair_capacity));
    }
  }

  MapParams p;
  memset(&p, 0, sizeof(p));
  p.t.dst = a->destination_slots;
  p.t.dst64 = a->destination_slots_dtype == LL_DTYPE_INT64 ? 1 : 0;
  for (int s = 0; s < 2; ++s) {
    p.t.maps[s] = reinterpret_cast<long long *>(a->maps[s]);
    p.t.cap[s] = a->map_capacity[s];
    p.t.mask[s] = a->repair_mask[s];
  }
  p.t.repair_dst = reinterpret_cast<long long *>(a->repair_destination_slots);
  hipStream_t stream_h = reinterpret_cast<hipStream_t>(stream);
  if (a->device_segments != nullptr) {
    // One launch over the device copy of the runs.
    int64_t longest = 0;
    for (int64_t k = 0; k < a->num_segments; ++k)
      longest = a->segments[k].token_count > longest ? a->segments[k].token_count : longest;
    if (longest == 0) return LL_OK;
    if (a->num_segments > kIntMax)
      return fail(LL_ERR_INVALID_ARGUMENT, "num_segments must be below 2^31 with device_segments");
    const dim3 grid(static_cast<unsigned>(a->num_segments),
                    static_cast<unsigned>((longest + kMapTokensPerBlock - 1) / kMapTokensPerBlock));
    build_link_maps_table_kernel<<<grid, dim3(256), 0, stream_h>>>(p.t, a->device_segments,
                                                                    a->num_destination_slots, a->repair_capacity);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return fail(LL_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(err));
    return LL_OK;
  }
  int n = 0;
  int64_t longest = 0;
  auto launch = [&]() -> int {
    if (n == 0) return LL_OK;
    const dim3 grid(static_cast<unsigned>(n),
                    static_cast<unsigned>((longest + kMapTokensPerBlock - 1) / kMapTokensPerBlock));
    build_link_maps_kernel<<<grid, dim3(256), 0, stream_h>>>(p);
    n = 0;
    longest = 0;
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess)
      return fail(LL_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(err));
    return LL_OK;
  };
  for (int64_t k = 0; k < a->num_segments; ++k) {
    const ll_link_segment &g = a->segments[k];
    if (g.token_count == 0) continue;
    MapSegment &m = p.seg[n++];
    m.src = reinterpret_cast<const long long *>(g.source_slots);
    m.local = reinterpret_cast<const long long *>(g.local_positions);
    m.start = g.start_token;
    m.dst_start = g.destination_start;
    m.local_start = g.local_start;
    m.count = static_cast<int>(g.token_count);
    m.map_offset = static_cast<int>(g.map_offset);
    m.repair_begin = static_cast<int>(g.repair_begin);
    m.repair_end = static_cast<int>(g.repair_end);
    m.repair_offset = g.repair_offset >= 0 && g.repair_end > g.repair_begin
                          ? static_cast<int>(g.repair_offset) : -1;
    m.set = static_cast<int>(g.map_set);
    if (g.token_count > longest) longest = g.token_count;
    if (n == kMaxSegmentsPerLaunch) {
      const int rc = launch();
      if (rc != LL_OK) return rc;
    }
  }
  return launch();
}

int64_t ll_order_maps_args_size(void) { return static_cast<int64_t>(sizeof(ll_order_maps_args)); }

int ll_order_link_maps(const ll_order_maps_args *a, ll_stream_t stream) {
  if (a == nullptr) return fail(LL_ERR_INVALID_ARGUMENT, "args is NULL");
  if (a->struct_size != static_cast<int64_t>(sizeof(ll_order_maps_args)))
    return fail(LL_ERR_INVALID_ARGUMENT, "struct_size %lld != %zu",
                static_cast<long long>(a->struct_size), sizeof(ll_order_maps_args));
  constexpr int64_t kIntMax = 0x7fffffff;
  if (a->capacity < 0 || a->capacity > kIntMax || a->count < 0 || a->count > a->capacity || a->prefix < 0 ||
      a->prefix > a->count)
    return fail(LL_ERR_INVALID_ARGUMENT, "need 0 <= prefix <= count <= capacity < 2^31");
  if (a->num_slots < 1) return fail(LL_ERR_INVALID_ARGUMENT, "num_slots must be >= 1");
  if (a->key_row != 0 && a->key_row != 1)
    return fail(LL_ERR_INVALID_ARGUMENT, "key_row must be 0 (source slots) or 1 (destination slots)");
  if (a->count == 0) return LL_OK;
  if (a->maps == nullptr || a->out_maps == nullptr)
    return fail(LL_ERR_INVALID_ARGUMENT, "maps and out_maps must be device arrays");
  if ((a->mask == nullptr) != (a->out_mask == nullptr))
    return fail(LL_ERR_INVALID_ARGUMENT, "mask and out_mask must both be given or both be NULL");
  const uintptr_t in_begin = reinterpret_cast<uintptr_t>(a->maps);
  const uintptr_t out_begin = reinterpret_cast<uintptr_t>(a->out_maps);
  const uintptr_t bytes = static_cast<uintptr_t>(4 * a->capacity) * sizeof(int64_t);
  if ((in_begin & 7u) != 0 || (out_begin & 7u) != 0)
    return fail(LL_ERR_INVALID_ARGUMENT, "maps and out_maps must be 8-byte aligned");
  if (in_begin < out_begin + bytes && out_begin < in_begin + bytes)
    return fail(LL_ERR_INVALID_ARGUMENT, "out_maps overlaps maps");
  if (a->mask != nullptr) {
    const uintptr_t m = reinterpret_cast<uintptr_t>(a->mask), o = reinterpret_cast<uintptr_t>(a->out_mask);
    if (m < o + static_cast<uintptr_t>(a->capacity) && o < m + static_cast<uintptr_t>(a->capacity))
      return fail(LL_ERR_INVALID_ARGUMENT, "out_mask overlaps mask");
  }
  if (a->workspace == nullptr || a->workspace_bytes < LL_ORDER_WORKSPACE_BYTES ||
      (reinterpret_cast<uintptr_t>(a->workspace) & 15u) != 0)
    return fail(LL_ERR_INVALID_ARGUMENT, "workspace must be a 16-byte aligned device array of at least %d bytes",
                LL_ORDER_WORKSPACE_BYTES);
  OrderParams p;
  p.maps = reinterpret_cast<const long long *>(a->maps);
  p.key = p.maps + a->key_row * a->capacity;
  p.mask = a->mask;
  p.cap = a->capacity;
  p.count = a->count;
  p.prefix = a->prefix;
  p.num_slots = a->num_slots;
  p.shift = 0;
  while (((a->num_slots - 1) >> p.shift) >= kOrderBuckets) ++p.shift;
  p.out = reinterpret_cast<long long *>(a->out_maps);
  p.out_mask = a->out_mask;
  p.counts = static_cast<int *>(a->workspace);
  p.offsets = p.counts + kOrderBuckets;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t tail = a->count - a->prefix;
  if (tail > 0) {
    const int64_t blocks = (tail + 255) / 256;
    order_count_kernel<<<dim3(static_cast<unsigned>(blocks < 4096 ? blocks : 4096)), dim3(256), 0, s>>>(p);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return fail(LL_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(err));
    order_offsets_kernel<<<dim3(1), dim3(kOrderThreads), 0, s>>>(p);
    err = hipGetLastError();
    if (err != hipSuccess) return fail(LL_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(err));
  }
  const int64_t blocks = (a->count + 255) / 256;
  order_scatter_kernel<<<dim3(static_cast<unsigned>(blocks < 4096 ? blocks : 4096)), dim3(256), 0, s>>>(p);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(LL_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(err));
  return LL_OK;
}

}  // extern "C"
