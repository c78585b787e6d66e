// Row-access calibration kernels for the link's measurements (bench.py
// --run-sweep): the link's own row traffic -- one 1 KiB-multiple row of K and
// one of V per (token, layer), at the link's source and destination slots --
// moved without the RoPE arithmetic, and split into its halves:
//
//   copy        read the source rows, write them to the destination rows;
//   read only   read the source rows (nothing is written back);
//   write only  write the destination rows (nothing is read).
//
// The time of the two halves bounds what any copy of these rows can reach if
// its reads and writes did not slow each other down; the copy is an
// independent implementation of the link's data movement.  Two work orders:
// token-major (a wave walks `layers_per_wave` layers of one token, the link
// kernel's order) and layer-major (a wave moves `tokens_per_wave` tokens of
// one layer; the grid walks the layers one after another).  A dynamic LDS
// allocation per workgroup limits how many workgroups share a CU.  A launch
// may move the K rows only or the V rows only (two such launches: a copy in
// two passes, one buffer of one layer at a time).
//
// Built as liblegolink_calibration.so, separate from the link library: it is
// measurement infrastructure and no part of the link's C ABI.
#include <hip/hip_runtime.h>

#include <stdint.h>
#include <stdio.h>

#include <string>

extern "C" {

typedef struct llc_row_args {
  int64_t struct_size;           // sizeof(llc_row_args)
  int64_t num_layers;            // 1..64
  void *const *key_layers;       // host array [num_layers] of device pointers
  void *const *value_layers;     // host array [num_layers] of device pointers
  int64_t num_slots;             // rows of every buffer
  int64_t row_bytes;             // bytes of one K (and one V) row: a positive multiple of 1024
  int64_t num_tokens;            // >= 1
  const int64_t *source_slots;   // device [num_tokens]
  const int64_t *destination_slots;  // device [num_tokens]
  int64_t mode;                  // 0 copy, 1 read only, 2 write only
  int64_t layer_major;           // 0 token-major, 1 layer-major
  int64_t layers_per_wave;       // token-major: divides num_layers, even layers_per_wave * tokens_per_wave
  int64_t tokens_per_wave;       // layer-major: divides num_tokens
  int64_t lds_bytes;             // dynamic LDS per 256-thread workgroup, 0..65536 (occupancy limit)
  uint32_t *sink;                // device [4 * 65536] words: read-only mode's (never taken) output
  int64_t buffers;               // 1 K rows only, 2 V rows only, 3 (or 0) both
} llc_row_args;

int llc_rows(const llc_row_args *args, hipStream_t stream);
int64_t llc_row_args_size(void);
const char *llc_last_error(void);

}  // extern "C"

namespace {

constexpr int kMaxLayers = 64;
constexpr int kWave = 64;
constexpr int kWavesPerBlock = 4;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct RowParams {
  char *k[kMaxLayers];
  char *v[kMaxLayers];
  const int64_t *src;
  const int64_t *dst;
  u32x4 *sink;
  long long num_slots;
  long long row_bytes;
  long long chunks;       // 1 KiB chunks per row
  long long num_tokens;
  long long waves;
  int num_layers;
  int layer_major;
  int per_wave;           // layers (token-major) or tokens (layer-major) per wave
  int buffers;            // bit 0 K rows, bit 1 V rows
};

thread_local std::string g_error;

int fail(const char *message) {
  g_error = message;
  return -1;
}

// Item i of a wave: (token, layer, 1 KiB chunk of the row).
__device__ __forceinline__ void item_of(const RowParams &p, long long w, int i, long long &token, int &layer,
                                        long long &chunk) {
  // A wave covers one chunk column of per_wave rows; chunk-waves of one row
  // group are consecutive.
  const long long group = w / p.chunks;
  chunk = w - group * p.chunks;
  if (p.layer_major) {
    const long long token_groups = p.num_tokens / p.per_wave;
    layer = static_cast<int>(group / token_groups);
    token = (group - static_cast<long long>(layer) * token_groups) * p.per_wave + i;
  } else {
    const int layer_groups = p.num_layers / p.per_wave;
    token = group / layer_groups;
    layer = static_cast<int>(group - token * layer_groups) * p.per_wave + i;
  }
}

template <int kMode, int kBuffers>
__global__ void __launch_bounds__(kWavesPerBlock * kWave) row_calibration_kernel(const RowParams p) {
  constexpr bool kK = (kBuffers & 1) != 0, kV = (kBuffers & 2) != 0;
  extern __shared__ char occupancy[];
  const int lane = threadIdx.x & (kWave - 1);
  const long long w = static_cast<long long>(blockIdx.x) * kWavesPerBlock + threadIdx.x / kWave;
  if (w >= p.waves) return;
  if (p.waves < 0) occupancy[threadIdx.x] = 0;  // never taken: keeps the LDS allocation in use
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (int i = 0; i < p.per_wave; i += 2) {
    u32x4 kin[2], vin[2];
    long long d[2];
    int layer[2];
    bool ok[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      long long token, chunk;
      item_of(p, w, i + u, token, layer[u], chunk);
      const long long s = p.src[token];
      const long long t = p.dst[token];
      ok[u] = s >= 0 && s < p.num_slots && t >= 0 && t < p.num_slots;
      const long long offset = chunk * 1024 + lane * 16;
      const long long so = (ok[u] ? s : 0) * p.row_bytes + offset;
      d[u] = (ok[u] ? t : 0) * p.row_bytes + offset;
      if constexpr (kMode != 2) {
        kin[u] = vin[u] = u32x4{0u, 0u, 0u, 0u};
        if constexpr (kK) kin[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p.k[layer[u]] + so));
        if constexpr (kV) vin[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p.v[layer[u]] + so));
      } else {
        kin[u] = u32x4{static_cast<uint32_t>(token), static_cast<uint32_t>(layer[u]), static_cast<uint32_t>(lane), 1u};
        vin[u] = u32x4{static_cast<uint32_t>(token), static_cast<uint32_t>(layer[u]), static_cast<uint32_t>(lane), 2u};
      }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      if constexpr (kMode == 1) {
        acc ^= kin[u];
        acc ^= vin[u];
      } else if (ok[u]) {
        if constexpr (kK) __builtin_nontemporal_store(kin[u], reinterpret_cast<u32x4 *>(p.k[layer[u]] + d[u]));
        if constexpr (kV) __builtin_nontemporal_store(vin[u], reinterpret_cast<u32x4 *>(p.v[layer[u]] + d[u]));
      }
    }
  }
  // Read only: the loaded words must reach a use; this store is taken only
  // for one specific XOR of every row word the lane read.
  if constexpr (kMode == 1) {
    if (acc.x == 0x9e3779b9u && acc.y == 0x7f4a7c15u && acc.z == 0x2545f491u)
      p.sink[(w * kWave + lane) & 65535] = acc;
  }
}

}  // namespace

extern "C" int64_t llc_row_args_size(void) { return static_cast<int64_t>(sizeof(llc_row_args)); }

extern "C" const char *llc_last_error(void) { return g_error.c_str(); }

extern "C" int llc_rows(const llc_row_args *a, hipStream_t stream) {
  if (a == nullptr || a->struct_size != static_cast<int64_t>(sizeof(llc_row_args)))
    return fail("args is NULL or struct_size differs");
  if (a->num_layers < 1 || a->num_layers > kMaxLayers) return fail("num_layers must be 1..64");
  if (a->key_layers == nullptr || a->value_layers == nullptr) return fail("layer tables are NULL");
  if (a->row_bytes < 1024 || a->row_bytes % 1024 != 0) return fail("row_bytes must be a positive multiple of 1024");
  if (a->num_slots < 1 || a->num_tokens < 1) return fail("num_slots and num_tokens must be positive");
  if (a->source_slots == nullptr || a->destination_slots == nullptr) return fail("slot maps are NULL");
  if (a->mode < 0 || a->mode > 2) return fail("mode must be 0 (copy), 1 (read only) or 2 (write only)");
  if (a->mode == 1 && a->sink == nullptr) return fail("read only needs a sink of 65536 16-byte words");
  if (a->lds_bytes < 0 || a->lds_bytes > 65536) return fail("lds_bytes must be 0..65536");
  RowParams p{};
  for (int64_t l = 0; l < a->num_layers; ++l) {
    if (a->key_layers[l] == nullptr || a->value_layers[l] == nullptr) return fail("a layer pointer is NULL");
    p.k[l] = static_cast<char *>(a->key_layers[l]);
    p.v[l] = static_cast<char *>(a->value_layers[l]);
  }
  int per_wave;
  long long groups;
  if (a->layer_major) {
    if (a->tokens_per_wave < 2 || a->tokens_per_wave % 2 || a->num_tokens % a->tokens_per_wave)
      return fail("tokens_per_wave must be even and divide num_tokens");
    per_wave = static_cast<int>(a->tokens_per_wave);
    groups = a->num_layers * (a->num_tokens / a->tokens_per_wave);
  } else {
    if (a->layers_per_wave < 2 || a->layers_per_wave % 2 || a->num_layers % a->layers_per_wave)
      return fail("layers_per_wave must be even and divide num_layers");
    per_wave = static_cast<int>(a->layers_per_wave);
    groups = a->num_tokens * (a->num_layers / a->layers_per_wave);
  }
  p.src = a->source_slots;
  p.dst = a->destination_slots;
  p.sink = reinterpret_cast<u32x4 *>(a->sink);
  p.num_slots = a->num_slots;
  p.row_bytes = a->row_bytes;
  p.chunks = a->row_bytes / 1024;
  p.num_tokens = a->num_tokens;
  p.num_layers = static_cast<int>(a->num_layers);
  p.layer_major = a->layer_major ? 1 : 0;
  if (a->buffers < 0 || a->buffers > 3) return fail("buffers must be 0..3");
  p.buffers = a->buffers == 0 ? 3 : static_cast<int>(a->buffers);
  p.per_wave = per_wave;
  p.waves = groups * p.chunks;
  const long long blocks = (p.waves + kWavesPerBlock - 1) / kWavesPerBlock;
  if (blocks > 0x7fffffffLL) return fail("too many rows for one grid");
  const dim3 grid(static_cast<unsigned>(blocks)), block(kWavesPerBlock * kWave);
  const size_t lds = static_cast<size_t>(a->lds_bytes);
  if (a->mode == 0) {
    if (p.buffers == 1) row_calibration_kernel<0, 1><<<grid, block, lds, stream>>>(p);
    else if (p.buffers == 2) row_calibration_kernel<0, 2><<<grid, block, lds, stream>>>(p);
    else row_calibration_kernel<0, 3><<<grid, block, lds, stream>>>(p);
  } else if (a->mode == 1) {
    if (p.buffers != 3) return fail("read only moves both buffers");
    row_calibration_kernel<1, 3><<<grid, block, lds, stream>>>(p);
  } else {
    if (p.buffers != 3) return fail("write only moves both buffers");
    row_calibration_kernel<2, 3><<<grid, block, lds, stream>>>(p);
  }
  const hipError_t error = hipGetLastError();
  if (error != hipSuccess) {
    g_error = std::string("launch failed: ") + hipGetErrorString(error);
    return -2;
  }
  return 0;
}
