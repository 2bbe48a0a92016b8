// Plain HBM read of a device buffer: the bandwidth floor the weight-streaming
// kernels are measured against (a decode GEMM cannot read its weights faster
// than a kernel that only reads them). Each lane issues four 16-byte loads
// per pass, grid-strided, and folds them into one dword that is stored only
// when it equals a constant no input is meant to hit, so the loads stay live
// without a store per workgroup.

#include <hip/hip_runtime.h>

#include "qmoe.h"
#include "qmoe_common.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kUnroll = 4;

__global__ __launch_bounds__(kThreads) void stream_read_kernel(const u32x4* __restrict__ src, int64_t n16,
                                                               uint32_t* __restrict__ sink) {
  uint32_t acc = 0;
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  for (; i + (kUnroll - 1) * stride < n16; i += kUnroll * stride) {
    u32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) v[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (; i < n16; i += stride) {
    const u32x4 v = __builtin_nontemporal_load(src + i);
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == 0x9e3779b9u) sink[blockIdx.x] = acc;
}

}  // namespace

extern "C" int qmoe_stream_read(const void* src, int64_t bytes, int32_t workgroups, void* sink,
                                qmoe_stream_t stream) {
  if (!src || !sink || bytes <= 0 || (bytes % 16) != 0 || (reinterpret_cast<uintptr_t>(src) & 15) ||
      workgroups <= 0)
    return QMOE_ERR_ARG;
  const int64_t n16 = bytes / 16;
  const int64_t need = (n16 + (int64_t)kThreads * kUnroll - 1) / ((int64_t)kThreads * kUnroll);
  const unsigned grid = (unsigned)(need < workgroups ? need : workgroups);
  hipLaunchKernelGGL(stream_read_kernel, dim3(grid), dim3(kThreads), 0, reinterpret_cast<hipStream_t>(stream),
                     static_cast<const u32x4*>(src), n16, static_cast<uint32_t*>(sink));
  return hipGetLastError() == hipSuccess ? QMOE_OK : QMOE_ERR_LAUNCH;
}
