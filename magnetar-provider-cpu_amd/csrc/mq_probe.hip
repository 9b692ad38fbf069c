// Streaming-read probe (libmagnetar_probe.so): a measurement aid for the
// benchmark, not part of the matmul path. It reads a device buffer once
// with 16-byte loads and nothing else, so its rate is the practical HBM
// read ceiling the decode GEMV is compared with at the same size.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

// Work-group w reads the `per_group` 16-byte words starting at
// w * per_group, `U` per lane in flight, lane-contiguous (each load
// instruction covers 64 consecutive words of a wave). The words are folded
// with xor and the fold is stored only when it equals `never`, which the
// compiler cannot rule out, so every load stays.
template <int U>
__global__ void stream_read_kernel(const uint4* __restrict__ src, uint64_t words, uint32_t never,
                                   uint32_t* __restrict__ sink) {
  const uint64_t per_group = static_cast<uint64_t>(blockDim.x) * U;
  const uint64_t base = blockIdx.x * per_group + threadIdx.x;
  uint4 v[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint64_t i = base + static_cast<uint64_t>(u) * blockDim.x;
    v[u] = i < words ? src[i] : make_uint4(0, 0, 0, 0);
  }
  uint32_t acc = 0;
#pragma unroll
  for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  if (acc == never) sink[blockIdx.x] = acc;
}

}  // namespace

extern "C" {

// Reads `bytes` (a multiple of 16) at `src` on `stream` (a hipStream_t):
// `loads` 16-byte loads per lane (1, 2, 4 or 8), `block` threads per
// work-group (64..1024, a multiple of 64). `sink` must hold one u32 per
// work-group: ceil(bytes / (16 * loads * block)). Returns 0, or -1 for a
// shape outside those bounds.
int mqp_stream_read(const void* src, uint64_t bytes, int loads, int block, uint32_t* sink, void* stream) {
  if (!src || !sink || bytes % 16 || block < 64 || block > 1024 || block % 64) return -1;
  const uint64_t words = bytes / 16;
  const uint64_t per_group = static_cast<uint64_t>(block) * loads;
  const dim3 grid(static_cast<unsigned>((words + per_group - 1) / per_group));
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const uint4* p = static_cast<const uint4*>(src);
  switch (loads) {
    case 1: hipLaunchKernelGGL(stream_read_kernel<1>, grid, dim3(block), 0, s, p, words, 0x9E3779B9u, sink); break;
    case 2: hipLaunchKernelGGL(stream_read_kernel<2>, grid, dim3(block), 0, s, p, words, 0x9E3779B9u, sink); break;
    case 4: hipLaunchKernelGGL(stream_read_kernel<4>, grid, dim3(block), 0, s, p, words, 0x9E3779B9u, sink); break;
    case 8: hipLaunchKernelGGL(stream_read_kernel<8>, grid, dim3(block), 0, s, p, words, 0x9E3779B9u, sink); break;
    default: return -1;
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// Work-groups a call of that shape launches (the sink's length).
uint64_t mqp_stream_groups(uint64_t bytes, int loads, int block) {
  const uint64_t per_group = static_cast<uint64_t>(block) * (loads > 0 ? loads : 1);
  return (bytes / 16 + per_group - 1) / per_group;
}

}  // extern "C"
