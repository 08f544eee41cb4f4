// Measurement probes behind profiles/, not part of the attention operator or
// its C ABI: the cold HBM read ceiling (the split-KV shapes are compared with
// it) and the matrix core's sustained bf16 rate with random or constant
// operands (the clock and socket power it runs at bound the MFMA-heavy shapes).
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

namespace {
constexpr int kThreads = 256;
constexpr int kUnroll = 8;

// One pass reads `bytes` once, 16 bytes per lane per load, eight independent
// loads in flight per lane, and writes nothing but one word per workgroup
// (kept only so the loads cannot be dropped). The caller flushes the caches
// (a 512 MiB write) before each pass so every byte comes from HBM.
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

// 8 waves per CU of back-to-back 32x32x16 bf16 MFMAs, 4 accumulator chains per
// wave, one operand pair per wave. pattern 0: operands from a per-lane LCG,
// about N(0,1) (sum of four uniforms); 1: constant operands (0.5 + i/100,
// 0.25). Each MFMA is 32768 flops.
__global__ __launch_bounds__(512) void mfma_probe_kernel(int iters, int pattern, float* __restrict__ sink) {
  uint32_t x = 0x9e3779b9u ^ (threadIdx.x * 2654435761u) ^ (blockIdx.x * 40503u);
  auto uni = [&]() {
    x = x * 1664525u + 1013904223u;
    return (float)(int)(x >> 8) * (1.f / 8388608.f) - 1.f;
  };
  bf16x8 a, b;
  for (int i = 0; i < 8; ++i) {
    float fa = 0.5f + 0.01f * i, fb = 0.25f;
    if (pattern == 0) {
      fa = (uni() + uni() + uni() + uni()) * 0.87f;
      fb = (uni() + uni() + uni() + uni()) * 0.87f;
    }
    a[i] = (__bf16)fa;
    b[i] = (__bf16)fb;
  }
  f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
  for (int it = 0; it < iters; ++it) {
    c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c1, 0, 0, 0);
    c2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c2, 0, 0, 0);
    c3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c3, 0, 0, 0);
  }
  const float acc = c0[0] + c1[3] + c2[5] + c3[7];
  if (acc == 12345.f) sink[blockIdx.x] = acc;   // practically never: the MFMAs must stay
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

// One launch of the MFMA probe on `stream`: `ctas` workgroups (one per CU) of
// 512 threads, `iters` x 4 MFMAs per wave; `sink` needs one float per
// workgroup. Returns a hipError_t.
extern "C" int mi355_probe_mfma(int ctas, int iters, int pattern, void* sink, void* stream) {
  if (ctas <= 0 || iters <= 0 || !sink || (pattern != 0 && pattern != 1)) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(mfma_probe_kernel, dim3(ctas), dim3(512), 0, (hipStream_t)stream, iters, pattern,
                     (float*)sink);
  return (int)hipGetLastError();
}
