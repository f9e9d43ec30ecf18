// bias.hip — the linear bias of a quantized linear layer on gfx950.
//
// out[r][n] = T(out[r][n] + bias[n]) (or bias[r][n] for a full-shape bias):
// MLX's `add` of two arrays of the output type T, computed in fp32 and rounded
// to nearest even once, as quantized_linear_forward applies it after quantized_matmul
// (src/lib/mlxcel-core/cpp/mlx_cxx_bridge.cpp:1707-1746).  HBM-bound: one
// read and one write of the output, one read of the bias; 8 elements a lane.
#include "common.hpp"
#include "kernels.hpp"

namespace mlxq {

// vec: out and bias 16-byte aligned and bias_n a multiple of 8 (16-byte
// accesses), else one element at a time.
__global__ __launch_bounds__(256) void bias_add_kernel(uint16_t* __restrict__ out, const uint16_t* __restrict__ bias,
                                                       int64_t n, int64_t bias_n, int vec) {
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (i >= n) return;
  if (vec && i + 8 <= n) {
    u32x4 o = *reinterpret_cast<const u32x4*>(out + i);
    const u32x4 b = *reinterpret_cast<const u32x4*>(bias + i % bias_n);
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const uint32_t lo = f32_to_bf16_bits(bf16_bits_to_f32(o[q] & 0xFFFFu) + bf16_bits_to_f32(b[q] & 0xFFFFu));
      const uint32_t hi = f32_to_bf16_bits(bf16_bits_to_f32(o[q] >> 16) + bf16_bits_to_f32(b[q] >> 16));
      o[q] = lo | (hi << 16);
    }
    *reinterpret_cast<u32x4*>(out + i) = o;
  } else {
    for (int64_t j = i; j < n && j < i + 8; j++)
      out[j] = (uint16_t)f32_to_bf16_bits(bf16_bits_to_f32(out[j]) + bf16_bits_to_f32(bias[j % bias_n]));
  }
}

// float16 / float32 outputs: the same add in fp32, one element a thread
template <typename T>
__global__ __launch_bounds__(256) void bias_add_any_kernel(T* __restrict__ out, const T* __restrict__ bias, int64_t n,
                                                           int64_t bias_n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  out[i] = (T)((float)out[i] + (float)bias[i % bias_n]);
}

hipError_t launch_bias_add(void* out_, const void* bias_, int64_t n, int64_t bias_n, int tc, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  if (bias_n <= 0) return hipErrorInvalidValue;
  if (tc == GEN_F16 || tc == GEN_F32) {
    const unsigned blocks = (unsigned)((n + 255) / 256);
    if (tc == GEN_F16)
      hipLaunchKernelGGL(bias_add_any_kernel<_Float16>, dim3(blocks), dim3(256), 0, stream,
                         static_cast<_Float16*>(out_), static_cast<const _Float16*>(bias_), n, bias_n);
    else
      hipLaunchKernelGGL(bias_add_any_kernel<float>, dim3(blocks), dim3(256), 0, stream, static_cast<float*>(out_),
                         static_cast<const float*>(bias_), n, bias_n);
    return hipGetLastError();
  }
  if (tc != GEN_BF16) return hipErrorInvalidValue;
  uint16_t* out = static_cast<uint16_t*>(out_);
  const uint16_t* bias = static_cast<const uint16_t*>(bias_);
  const int64_t lanes = (n + 7) / 8;
  const int vec = ((reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(bias)) & 15u) == 0 &&
                  bias_n % 8 == 0;
  hipLaunchKernelGGL(bias_add_kernel, dim3((unsigned)((lanes + 255) / 256)), dim3(256), 0, stream, out, bias, n,
                     bias_n, vec);
  return hipGetLastError();
}

}  // namespace mlxq
