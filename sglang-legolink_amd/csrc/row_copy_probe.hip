// Memory-ceiling probes for bench.py --ceiling (measurement only, not part of
// the link library's ABI).
//
//   llp_stream_copy  contiguous copy, one 16-byte element per thread over a
//                    grid that covers the buffer once: the streaming copy
//                    bandwidth of the device.
//   llp_row_copy     the link's access pattern without arithmetic: for every
//                    buffer b and token t, copy row src[t] to row dst[t]
//                    (rows of row_bytes, 16-byte aligned).  One wave per
//                    (buffer, token) row, buffer-major block order.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kMaxBuffers = 256;

struct RowCopyParams {
  char *buffers[kMaxBuffers];
  const long long *src;
  const long long *dst;
  long long tokens;
  long long slots;
  long long row_chunks;  // 16-byte chunks per row
  int num_buffers;
};

__global__ void __launch_bounds__(256) stream_copy_kernel(const u32x4 *__restrict__ src,
                                                          u32x4 *__restrict__ dst, long long n) {
  const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = src[i];
}

// grid.x = num_buffers * rows_per_buffer_blocks; each block covers 256 chunks
// of consecutive tokens' rows in one buffer.
__global__ void __launch_bounds__(256) row_copy_kernel(const RowCopyParams p, long long blocks_per_buffer) {
  const long long buffer = blockIdx.x / blocks_per_buffer;
  const long long chunk = (blockIdx.x % blocks_per_buffer) * 256 + threadIdx.x;
  if (buffer >= p.num_buffers || chunk >= p.tokens * p.row_chunks) return;
  const long long t = chunk / p.row_chunks;
  const long long c = chunk - t * p.row_chunks;
  const long long s = p.src[t];
  const long long d = p.dst[t];
  if (s < 0 || s >= p.slots || d < 0 || d >= p.slots) return;
  char *base = p.buffers[buffer];
  const u32x4 v = *reinterpret_cast<const u32x4 *>(base + (s * p.row_chunks + c) * 16);
  *reinterpret_cast<u32x4 *>(base + (d * p.row_chunks + c) * 16) = v;
}

}  // namespace

extern "C" {

// bytes must be a multiple of 16; src/dst device pointers, 16-byte aligned.
int llp_stream_copy(const void *src, void *dst, long long bytes, hipStream_t stream) {
  if (src == nullptr || dst == nullptr || bytes <= 0 || (bytes % 16) != 0) return -1;
  const long long n = bytes / 16;
  const long long blocks = (n + 255) / 256;
  if (blocks > 0x7fffffffLL) return -1;
  stream_copy_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream>>>(
      static_cast<const u32x4 *>(src), static_cast<u32x4 *>(dst), n);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

// buffers: host array of num_buffers device pointers, each [slots, row_bytes].
int llp_row_copy(void *const *buffers, int num_buffers, const long long *src, const long long *dst,
                 long long tokens, long long slots, long long row_bytes, hipStream_t stream) {
  if (buffers == nullptr || num_buffers < 1 || num_buffers > kMaxBuffers || src == nullptr ||
      dst == nullptr || tokens < 1 || slots < 1 || row_bytes < 16 || (row_bytes % 16) != 0)
    return -1;
  RowCopyParams p;
  for (int b = 0; b < num_buffers; ++b) {
    if (buffers[b] == nullptr) return -1;
    p.buffers[b] = static_cast<char *>(buffers[b]);
  }
  p.src = src;
  p.dst = dst;
  p.tokens = tokens;
  p.slots = slots;
  p.row_chunks = row_bytes / 16;
  p.num_buffers = num_buffers;
  const long long blocks_per_buffer = (tokens * p.row_chunks + 255) / 256;
  const long long blocks = blocks_per_buffer * num_buffers;
  if (blocks > 0x7fffffffLL) return -1;
  row_copy_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream>>>(p, blocks_per_buffer);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // extern "C"
