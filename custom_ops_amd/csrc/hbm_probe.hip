// HBM read-bandwidth probe: measurement tooling behind profiles/ (the cold
// streaming ceiling that the split-KV shapes are compared with), not part of
// the attention operator or its C ABI.
//
// One pass reads `bytes` once, 16 bytes per lane per load, eight independent
// loads in flight per lane, and writes nothing but one word per workgroup
// (kept only so the loads cannot be dropped). The caller flushes the caches
// (a 512 MiB write) before each pass so every byte comes from HBM.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

namespace {
constexpr int kThreads = 256;
constexpr int kUnroll = 8;

__global__ __launch_bounds__(kThreads) void hbm_read_kernel(const u32x4* __restrict__ src, uint64_t n16,
                                                            uint32_t* __restrict__ sink) {
  const uint64_t stride = (uint64_t)gridDim.x * kThreads;
  uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (; i + (kUnroll - 1) * stride < n16; i += kUnroll * stride) {
    u32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) v[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc ^= v[u];
  }
  for (; i < n16; i += stride) acc ^= src[i];
  const uint32_t x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
  if (x == 0x9e3779b9u) sink[blockIdx.x] = x;   // practically never: the loads must stay
}
}  // namespace

// Read `bytes` (a multiple of 16) at `src` once on `stream`; `sink` needs one
// word per workgroup (the grid is 2048 workgroups). Returns a hipError_t.
extern "C" int mi355_probe_read(const void* src, size_t bytes, void* sink, void* stream) {
  if (!src || !sink || bytes % 16) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(hbm_read_kernel, dim3(2048), dim3(kThreads), 0, (hipStream_t)stream,
                     (const u32x4*)src, (uint64_t)(bytes / 16), (uint32_t*)sink);
  return (int)hipGetLastError();
}
