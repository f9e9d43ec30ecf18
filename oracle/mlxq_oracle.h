/*
 * mlxq_oracle.h — CPU restatement of MLX's quantized-matmul semantics.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the GPU path is
 * compared against (and the timed single-core CPU baseline in bench.py).  It
 * is never linked into, loaded by, or called from the product library
 * (mlxcel_amd/, include/mlxq.h).
 *
 * bf16 values are passed as their raw uint16_t bit patterns.  Every function
 * names the reference file:line it restates; abbreviations:
 *   CPUQ = src/lib/mlxcelverse/overlays/cpu/mlx/backend/cpu/quantized.cpp
 *   ROPS = src/lib/mlxcelverse/overlays/rocm/mlx/ops.cpp
 *   QAFF = src/lib/mlxcelverse/overlays/rocm/mlx/backend/rocm/quantized/affine_quantize.hip
 */
#ifndef MLXQ_ORACLE_H
#define MLXQ_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* float <-> bf16 with MLX's conversion (round to nearest even, NaN -> 0x7FC0). */
uint16_t oracle_f32_to_bf16(float f);
float oracle_bf16_to_f32(uint16_t h);
uint16_t oracle_f32_to_f16(float f);
float oracle_f16_to_f32(uint16_t h);
void oracle_f32_to_bf16_n(const float* in, uint16_t* out, int64_t n);
void oracle_bf16_to_f32_n(const uint16_t* in, float* out, int64_t n);

/* Affine quantize, CPUQ:1233-1305 (`quantize<bfloat16_t, uint32_t>`).
 * w: [rows, K] bf16.  wq: [rows, K*bits/32] u32.  scales/biases: [rows, K/gs] bf16.
 * bits in {1, 2, 4, 8}; returns 0 on success, -1 on unsupported arguments. */
/* MLX's CPU affine quantizer for dtype 0 = bfloat16, 1 = float16, 2 = float32
 * weights (scales and biases written in the same dtype) and bits 1-6 or 8. */
int oracle_affine_quantize_t(const void* w, int dtype, int64_t rows, int64_t K, int group_size, int bits,
                             uint32_t* wq, void* scales, void* biases);
int oracle_affine_quantize(const uint16_t* w, int64_t rows, int64_t K, int group_size,
                           int bits, uint32_t* wq, uint16_t* scales, uint16_t* biases);

/* Affine dequantize.
 * rounding == 2: MLX CPU graph fallback, ROPS:5531-5573 — `multiply(w, scales)`
 *                then `add(.., biases)` in bf16: bf16(bf16(q*s) + b).
 * rounding == 1: ROCm GPU kernel, QAFF:164 — bf16(s*q + b) computed in float. */
int oracle_affine_dequantize(const uint32_t* wq, const uint16_t* scales,
                             const uint16_t* biases, int64_t rows, int64_t K,
                             int group_size, int bits, int rounding, uint16_t* out);

/* mxfp4 scale decode, CPUQ:89-105 `dequantize_scale<T, 32>` (bf16 bits). */
uint16_t oracle_e8m0_to_bf16(uint8_t s);

/* mxfp4 quantize, the graph fallback of ROPS:5364-5431 evaluated in bf16.
 * w: [rows, K] bf16, K % 32 == 0.  wq: [rows, K/8] u32.  scales: [rows, K/32] u8. */
int oracle_mxfp4_quantize(const uint16_t* w, int64_t rows, int64_t K, uint32_t* wq,
                          uint8_t* scales);

/* mxfp4 dequantize, ROPS:5646-5695 (LUT[nibble] * 2^(s-127); s == 0xFF -> NaN). */
int oracle_mxfp4_dequantize(const uint32_t* wq, const uint8_t* scales, int64_t rows,
                            int64_t K, uint16_t* out);

/* fp8 e4m3 as MLX's to_fp8 / from_fp8 on the ROCm backend
 * (overlays/rocm/mlx/backend/rocm/quantized/convert_fp8.hip:18-90). */
uint8_t oracle_e4m3_encode(float f);
float oracle_e4m3_decode(uint8_t c);
void oracle_e4m3_encode_n(const float* in, uint8_t* out, int64_t n);
void oracle_e4m3_decode_n(const uint8_t* in, float* out, int64_t n);

/* mxfp8 (e4m3 codes, group 32, e8m0 scales) and nvfp4 (e2m1 codes, group 16,
 * e4m3 scales, no global scale): the graph quantizer ROPS:5364-5431 and
 * dequantizer ROPS:5646-5695.  wq: [rows, K*bits/32] u32, scales [rows, K/gs] u8. */
int oracle_mxfp8_quantize(const uint16_t* w, int64_t rows, int64_t K, uint32_t* wq, uint8_t* scales);
int oracle_mxfp8_dequantize(const uint32_t* wq, const uint8_t* scales, int64_t rows, int64_t K,
                            uint16_t* out);
int oracle_nvfp4_quantize(const uint16_t* w, int64_t rows, int64_t K, uint32_t* wq, uint8_t* scales);
int oracle_nvfp4_dequantize(const uint32_t* wq, const uint8_t* scales, int64_t rows, int64_t K,
                            uint16_t* out);

/* `_qmm_t<bfloat16_t, bits, gs>`, CPUQ:199-257: y[m, n] = bf16(sum_k x*(s*q+b)),
 * float accumulation in MLX's loop order.  x: [M, K], w: [N, K*bits/32]. */
int oracle_qmm_t_affine(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                        const uint16_t* biases, int64_t M, int64_t N, int64_t K,
                        int group_size, int bits, uint16_t* out);

/* `_qmm<bfloat16_t, bits, gs>` (transpose=false), CPUQ:139-197:
 * w: [K, N*bits/32], scales/biases: [K, N/gs]; y[m, n] accumulated over k. */
int oracle_qmm_affine(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                      const uint16_t* biases, int64_t M, int64_t N, int64_t K,
                      int group_size, int bits, uint16_t* out);

/* `fp_qmm_t<bfloat16_t, 32, 4>` (mxfp4), CPUQ:550-597. */
int oracle_fp_qmm_t_mxfp4(const uint16_t* x, const uint32_t* wq, const uint8_t* scales,
                          int64_t M, int64_t N, int64_t K, uint16_t* out);

/* `_bs_qmm_dispatch_typed` / `fp_bs_qmm_dispatch_mode`, CPUQ:764-813, 875-914:
 * for each i < B: out[i] = x[lhs[i]] @ dequant(w[rhs[i]])^T.
 * x: [*, M, K] (lhs indexes its flattened batch), w: [E, N, K*bits/32],
 * scales/biases: [E, N, K/gs]; mode 0 = affine, 1 = mxfp4 (biases ignored). */
int oracle_gather_qmm_t(const uint16_t* x, const uint32_t* wq, const void* scales,
                        const uint16_t* biases, const uint32_t* lhs,
                        const uint32_t* rhs, int64_t B, int64_t M, int64_t N,
                        int64_t K, int group_size, int bits, int mode, uint16_t* out);

int oracle_affine_dequantize_f32(const uint32_t* wq, const uint16_t* scales, const uint16_t* biases,
                                 int64_t rows, int64_t K, int group_size, int bits, float* out);
int oracle_fused_moe(const uint16_t* x, const uint32_t* idx, const float* scores, const uint32_t* gate_w,
                     const uint16_t* gate_s, const uint16_t* gate_b, const uint32_t* up_w,
                     const uint16_t* up_s, const uint16_t* up_b, const uint32_t* down_w,
                     const uint16_t* down_s, const uint16_t* down_b, int64_t din, int64_t dff, int64_t k,
                     int64_t E, int group_size, int gu_bits, int d_bits, int act, float* out);

#ifdef __cplusplus
}
#endif

#endif
