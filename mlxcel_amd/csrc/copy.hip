// copy.hip — strided <-> row-contiguous copies for gfx950.
//
// The reference's quantized matmul copies inputs that are not row-contiguous
// before its kernels run (overlays/rocm/mlx/backend/rocm/quantized/qmm.hip:
// 3557-3564, `ensure_row_contiguous`); the library does the same for x, w,
// scales and biases, and writes a result into a strided `out` through a
// contiguous staging buffer.  One thread per element (elements of 1, 2, 4 or
// 8 bytes); the index is decomposed over the view's shape, so any strides
// (broadcast zeros included) work in either direction.
#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"

namespace mlxq {

__global__ __launch_bounds__(256) void strided_copy_kernel(const CopyArgs a) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.n; i += stride) {
    int64_t r = i, so = 0, dof = 0;
    for (int d = a.ndim - 1; d >= 0; d--) {
      const int64_t c = r % a.shape[d];
      r /= a.shape[d];
      so += c * a.src_strides[d];
      dof += c * a.dst_strides[d];
    }
    switch (a.esz) {
      case 1: static_cast<uint8_t*>(a.dst)[dof] = static_cast<const uint8_t*>(a.src)[so]; break;
      case 2: static_cast<uint16_t*>(a.dst)[dof] = static_cast<const uint16_t*>(a.src)[so]; break;
      case 4: static_cast<uint32_t*>(a.dst)[dof] = static_cast<const uint32_t*>(a.src)[so]; break;
      default: static_cast<uint64_t*>(a.dst)[dof] = static_cast<const uint64_t*>(a.src)[so]; break;
    }
  }
}

hipError_t launch_strided_copy(const CopyArgs& a, hipStream_t stream) {
  if (a.n <= 0) return hipSuccess;
  if (a.ndim < 0 || a.ndim > MLXQ_MAX_DIMS || (a.esz != 1 && a.esz != 2 && a.esz != 4 && a.esz != 8))
    return hipErrorInvalidValue;
  const int64_t blocks = std::min<int64_t>((a.n + 255) / 256, 65536);
  hipLaunchKernelGGL(strided_copy_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace mlxq
