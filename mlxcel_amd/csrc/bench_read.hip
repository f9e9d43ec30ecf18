// bench_read.hip — streaming-read ceiling for bench.py (not part of the
// quantized-matmul library or its C-ABI; built into libmlxq_bench.so).
//
// A workgroup reads a contiguous slice of the buffer with 16-byte loads,
// four in flight per lane, and folds them with xor; the result is stored only
// when it equals a value no test buffer produces, so the loads stay live
// without a write stream.  Timed at the decode kernels' bytes per launch, it
// gives the fastest any kernel on the device streams that many bytes once,
// which is the practical bound for a decode projection of that size.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace {

__global__ __launch_bounds__(512) void read_fold_kernel(const uint4* __restrict__ p, size_t n16, int per_wg,
                                                        uint32_t* __restrict__ sink) {
  const size_t base = (size_t)blockIdx.x * (size_t)per_wg;
  uint32_t acc = 0;
  for (int i = threadIdx.x; i < per_wg; i += 4 * (int)blockDim.x) {
    uint4 v[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int o = i + u * (int)blockDim.x;
      const size_t j = base + (size_t)o;
      v[u] = (o < per_wg && j < n16) ? p[j] : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int u = 0; u < 4; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == 0x9E3779B9u) sink[blockIdx.x] = acc;
}

}  // namespace

extern "C" int mlxq_bench_read(const void* buf, size_t bytes, uint32_t* sink, int workgroups, int threads,
                               void* stream) {
  if (!buf || !sink || workgroups <= 0 || threads <= 0 || threads > 512 || (threads & 63) != 0 || bytes < 16)
    return (int)hipErrorInvalidValue;
  const size_t n16 = bytes / 16;
  const size_t per = (n16 + (size_t)workgroups - 1) / (size_t)workgroups;
  if (per > (size_t)0x7FFFFFFF) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(read_fold_kernel, dim3((unsigned)workgroups), dim3((unsigned)threads), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<const uint4*>(buf), n16, (int)per, sink);
  return (int)hipGetLastError();
}
