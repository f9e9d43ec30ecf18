/*
 * mlxq.h — C ABI of the MI355X (gfx950) quantized-matmul library.
 *
 * Drop-in replacement for the MLX primitives behind mlxcel's quantized
 * linear layers and MoE experts:
 *   mlxq_quantized_matmul  <- ffi::quantized_matmul   (src/lib/mlxcel-core/src/lib.rs:1391-1400,
 *                             cpp/mlx_cxx_bridge.cpp:3782-3814 -> mlx::core::quantized_matmul,
 *                             overlays/rocm/mlx/ops.cpp:4955-5008)
 *   mlxq_gather_qmm        <- ffi::gather_qmm         (lib.rs:1374-1388, mlx_cxx_bridge.cpp:3745-3780
 *                             -> mlx::core::gather_qmm, ops.cpp:5841-5948)
 *   mlxq_dequantize        <- ffi::dequantize         (lib.rs:1409-1416, mlx_cxx_bridge.cpp:3816-3878
 *                             -> mlx::core::dequantize, ops.cpp:5753-5805)
 *   mlxq_quantize          <- ffi::quantize_weights_* (mlx_cxx_bridge.cpp:7867-7900
 *                             -> mlx::core::quantize, ops.cpp:5454-5492)
 *   mlxq_quantized_linear  <- ffi::quantized_linear_forward (lib.rs:697-707,
 *                             mlx_cxx_bridge.cpp:1707-1746)
 *   mlxq_quantized_matmul_matches_dense_gemm <- ffi::quantized_matmul_matches_dense_gemm
 *                             (lib.rs:2925-2940)
 *   mlxq_quantized_matmul_multi <- the fused q/k/v and gate/up GEMVs of mlxcel-xla
 *                             (src/lib/mlxcel-xla/csrc/qmv4.hip:265-387)
 *   mlxq_fused_moe_expert  <- ffi::fused_moe_expert_kernel (lib.rs:2336-2356,
 *                             mlx_cxx_bridge.h:2061-2070, mlx_cxx_kernels.cpp:4078-4094)
 *   mlxq_fused_moe_geglu   <- ffi::fused_moe_geglu_kernel  (lib.rs:2357-2380,
 *                             mlx_cxx_bridge.h:2072-2084, mlx_cxx_kernels.cpp:4096-4112)
 *
 * Conventions (differences from the reference are deliberate and listed):
 *   - Eager and stream-ordered: work is enqueued on `stream` (a hipStream_t,
 *     NULL = the default stream) and the call returns without waiting.  The
 *     reference builds a lazy graph node; the node's eval is what this does.
 *   - Caller-allocated output: `out` must already have the shape and dtype
 *     the reference would give the result (query it with the *_shape
 *     functions).  All `data` pointers are device pointers.
 *   - Errors are status codes, never exceptions.  Argument errors return
 *     MLXQ_EINVAL with the reference's exception text in mlxq_last_error();
 *     valid combinations this library does not implement return
 *     MLXQ_EUNSUPPORTED so the caller can fall back.
 *   - group_size / bits <= 0 select the mode's default (the reference's
 *     std::nullopt), as in quantization_params_from_mode (ops.cpp:4846-4870).
 *   - Thread-safe and re-entrant.  Index values outside the expert or batch
 *     range are clamped to the last valid entry instead of reading out of
 *     bounds.
 */
#ifndef MLXQ_H
#define MLXQ_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MLXQ_MAX_DIMS 8

typedef enum mlxq_status {
  MLXQ_OK = 0,
  MLXQ_EINVAL = 1,       /* argument rejected; message = the reference's std::invalid_argument text */
  MLXQ_EUNSUPPORTED = 2, /* valid for MLX but not implemented here (caller falls back) */
  MLXQ_EHIP = 3,         /* HIP runtime error (launch failure, no device) */
  MLXQ_ENOMEM = 4        /* device workspace allocation failed */
} mlxq_status;

/* Same order as mlx::core::Dtype::Val. */
typedef enum mlxq_dtype {
  MLXQ_BOOL = 0,
  MLXQ_UINT8 = 1,
  MLXQ_UINT16 = 2,
  MLXQ_UINT32 = 3,
  MLXQ_UINT64 = 4,
  MLXQ_INT8 = 5,
  MLXQ_INT16 = 6,
  MLXQ_INT32 = 7,
  MLXQ_INT64 = 8,
  MLXQ_FLOAT16 = 9,
  MLXQ_FLOAT32 = 10,
  MLXQ_FLOAT64 = 11,
  MLXQ_BFLOAT16 = 12,
  MLXQ_COMPLEX64 = 13
} mlxq_dtype;

/* A strided view of device memory (strides in elements, like mlx::core::array). */
typedef struct mlxq_array {
  void* data;
  int32_t dtype; /* mlxq_dtype */
  int32_t ndim;  /* 0 .. MLXQ_MAX_DIMS */
  int64_t shape[MLXQ_MAX_DIMS];
  int64_t strides[MLXQ_MAX_DIMS];
} mlxq_array;

/* Device scratch.  Calls that need scratch (split-K partials of the 5-16-row
 * decode kernel and of the prefill GEMM, gather index lists, the fused MoE's
 * activations) use a per-(device, stream) workspace that grows on demand.  A
 * grown workspace never frees the buffer it replaces (a HIP graph captured
 * earlier may still use it); no call synchronizes a stream, and a call that
 * would have to grow the workspace of a stream under capture returns
 * MLXQ_ENOMEM instead of allocating.  Callers that capture either run each
 * call shape once before the capture or reserve the workspace up front. */

/* Grows `stream`'s workspace on the current device to at least `bytes`, both
 * the kernel scratch and the staging buffer that holds row-contiguous copies
 * of strided or misaligned operands (each at least `bytes`), so a capture of
 * calls needing at most that much of either allocates nothing.  Also
 * allocates the stream's stream-K counters (1 MiB) and resolves the device
 * address of mlxq_quantized_matmul_noalloc's fixed scratch.  A captured
 * prefill call whose stream-K plan needs more scratch than the stream holds
 * (2 x CUs x 256 KiB, 128 MiB on MI355X) takes the plan without stream-K
 * instead of allocating; its result then equals the eager call's within
 * rounding, not bit for bit (stream-K adds a cut tile's two K pieces in
 * fp32).  No counterpart in the reference (MLX allocates inside each
 * eval). */
mlxq_status mlxq_workspace_reserve(size_t bytes, void* stream);

/* Bytes of device memory held by the workspaces (current and replaced
 * buffers), like the reference's get_cache_memory (lib.rs:2720). */
size_t mlxq_get_cache_memory(void);

/* Synchronizes every device that holds a workspace and frees all workspace
 * buffers, like the reference's clear_memory_cache (lib.rs:2666).  HIP graphs
 * captured earlier that ran library calls must not be replayed afterwards. */
mlxq_status mlxq_clear_cache(void);

/* The MLXQ_* environment switches (forced kernels, tile shapes: A/B
 * measurement and tests only) are read once, at the first call; this re-reads
 * them.  No counterpart in the reference, which latches its knobs in function
 * statics (rocm/quantized/qmm.hip:392-452). */
void mlxq_reload_options(void);

/* Message of the last failing call on this thread ("" if none). */
const char* mlxq_last_error(void);

/* Library version string, e.g. "mlxq 0.1.0 gfx950". */
const char* mlxq_version(void);

/* y = x @ dequantize(w, scales, biases)^T  (transpose=true), or without the
 * transpose.  Shapes/dtypes exactly as mlx::core::quantized_matmul
 * (ops.cpp:4955-5008): out.shape = x.shape[:-1] + [N], out dtype =
 * promote(x, scales, biases) for affine and x.dtype for fp modes.
 * Implemented: both transposes; mode "affine" with bits 1, 2, 3, 4, 5, 6 or 8
 * and group_size 32/64/128; mode "mxfp4"; bfloat16, float16 and float32
 * activations, scales and biases (computed in the promoted type, fp32
 * accumulation); w 2-D, or batched with batch dims that broadcast against
 * x's.  Operands of any strides: ones that are not row-contiguous and
 * 16-byte aligned are first copied into a per-stream staging workspace, as
 * the reference copies them (rocm/quantized/qmm.hip:3557-3564), and a
 * strided `out` is written through it.  bfloat16 4/8-bit affine and mxfp4
 * with transpose=true run the specialised kernels, and so does float16
 * (x, scales, biases and result) 4/8-bit affine with transpose=true (decode
 * and prefill; its prefill dequantizes the weights to float16, as the
 * reference's dequantize + GEMM route does); every other combination runs
 * the general path: affine calls of 1-4 rows per matrix with transpose=true
 * (1-2 with transpose=false) on its row-streaming decode kernels (fp32
 * products, no weight rounding), the rest on its tile kernel (float16
 * results there also round the dequantized weights to float16).  Operands
 * of 2 GiB and more: with 2-D weights, x and
 * the result run as row chunks below 2 GiB on the same kernels; a weight
 * matrix (or its scales) of 2 GiB or more runs on the general kernel.
 * Batched weights take any rows per batch. */
mlxq_status mlxq_quantized_matmul(const mlxq_array* x, const mlxq_array* w,
                                  const mlxq_array* scales, const mlxq_array* biases,
                                  bool transpose, int32_t group_size, int32_t bits,
                                  const char* mode, mlxq_array* out, void* stream);

/* quantized_matmul without any allocation: the same validation, kernels and
 * result bits as mlxq_quantized_matmul (except at the prefill shapes that
 * take the stream-K plan, whose partials do not fit the fixed scratch: the
 * plan without it gives the same result within rounding), but the scratch
 * some routes need (split-K partials of the 5-16-row decode kernel and of
 * the prefill GEMM) lives in a fixed 64 MiB device array of the library (one
 * per GPU, held until the process ends) instead of the per-stream
 * workspace.  Calls that
 * would need more return MLXQ_ENOMEM with the size in mlxq_last_error().
 * Every call on one GPU shares that array: calls that overlap in time on one
 * GPU (several streams, threads or replays of graphs in flight together) race.
 * Operands must be row-contiguous and 16-byte aligned (no staging copies).
 * No counterpart in the reference; it is for callers that cannot allocate
 * (code under HIP-graph capture, tight serving loops). */
mlxq_status mlxq_quantized_matmul_noalloc(const mlxq_array* x, const mlxq_array* w,
                                          const mlxq_array* scales, const mlxq_array* biases,
                                          bool transpose, int32_t group_size, int32_t bits,
                                          const char* mode, mlxq_array* out, void* stream);

/* A quantized linear layer, as the reference's quantized_linear_forward
 * (lib.rs:697-707, mlx_cxx_bridge.cpp:1707-1746): quantized_matmul with
 * transpose = true, then `+ linear_bias` as MLX adds two bf16 arrays (fp32
 * sum, one rounding; float16 / float32 results likewise in their type).
 * `linear_bias` may be NULL; otherwise row-contiguous, of shape (N) (or
 * (1, ..., N)) or the output's shape, in the output's dtype (other layouts
 * return MLXQ_EUNSUPPORTED). */
mlxq_status mlxq_quantized_linear(const mlxq_array* x, const mlxq_array* w, const mlxq_array* scales,
                                  const mlxq_array* biases, const mlxq_array* linear_bias,
                                  int32_t group_size, int32_t bits, const char* mode,
                                  mlxq_array* out, void* stream);

/* Whether quantized_matmul on these inputs returns the bytes of dequantize +
 * a dense GEMM, as the reference's quantized_matmul_matches_dense_gemm
 * (lib.rs:2925-2940, rocm qmm.hip:3493-3542) answers for its routes.  Always
 * 0 here: every route dequantizes inside the matmul kernel.  No device work. */
int32_t mlxq_quantized_matmul_matches_dense_gemm(const mlxq_array* x, const mlxq_array* w,
                                                 const mlxq_array* scales,
                                                 const mlxq_array* biases, int32_t group_size,
                                                 int32_t bits);

/* Several projections of one activation in one call (q/k/v, gate/up):
 * out[i] = quantized_matmul(x, w[i], scales[i], biases[i], transpose = true,
 * group_size, bits, mode) for i < n, 1 <= n <= 4, every w[i] 2-D and of the
 * same format.  Results are bit for bit those of n mlxq_quantized_matmul
 * calls; at decode row counts the n projections run as one launch that reads
 * x once.  One exception: at 5-16 rows, where the projections' 64-row
 * blocks together exceed one round of the CUs while each alone fits (gate +
 * up of 2 x 12288 rows with 4-bit codes on MI355X), the one launch takes
 * the split-K kernel and the separate calls the whole-row kernel, so the
 * results agree within rounding, not bit for bit.  `biases` (the array of
 * pointers) may be NULL for mxfp4.  No counterpart in the MLX op layer: it
 * replaces the fused q/k/v and gate/up GEMV launches of the reference's
 * native decode path
 * (src/lib/mlxcel-xla/csrc/qmv4.hip:265-387, src/native_qmv.rs:250-330). */
mlxq_status mlxq_quantized_matmul_multi(const mlxq_array* x, int32_t n, const mlxq_array* const* w,
                                        const mlxq_array* const* scales,
                                        const mlxq_array* const* biases, int32_t group_size,
                                        int32_t bits, const char* mode, mlxq_array* const* out,
                                        void* stream);

/* Output shape/dtype the reference would give quantized_matmul, after the same
 * validation (no device work). */
mlxq_status mlxq_quantized_matmul_shape(const mlxq_array* x, const mlxq_array* w,
                                        const mlxq_array* scales, const mlxq_array* biases,
                                        bool transpose, int32_t group_size, int32_t bits,
                                        const char* mode, int32_t* out_ndim,
                                        int64_t* out_shape, int32_t* out_dtype);

/* out[i] = x[lhs[i]] @ dequantize(w[rhs[i]])^T over the broadcast index
 * shape, as mlx::core::gather_qmm (ops.cpp:5841-5948): out.shape =
 * broadcast(lhs, rhs).shape + [x.shape[-2], N].  NULL lhs/rhs default to
 * arange over the batch dims of x/w; both NULL is quantized_matmul.
 * `sorted_indices` is the reference's promise that rhs, cast to uint32 as
 * the reference casts indices (ops.cpp:100), is non-decreasing in the flat
 * order of the broadcast batch; as in the reference's expert-run kernels
 * (rocm/quantized/qmm.hip:4705-4740, found by binary search) the result is
 * unspecified when the promise is false (the sorted routes for one
 * activation row per entry then leave some output rows unwritten: negative
 * int32 values, for instance, are not sorted after the cast).  Sorted and
 * unsorted routes differ only in summation order (same tolerance).
 * `global_scale` (nvfp4 only in the reference) must be
 * NULL.  Index arrays may be any integer dtype and any strides
 * (broadcasting included).  Types, code widths, transposes and strides as
 * for mlxq_quantized_matmul; any rows per gathered matrix.  Any number of
 * index entries: more than 65528 run as chunks of 65528 entries over flat
 * copies of the indices in the stream's workspace. */
mlxq_status mlxq_gather_qmm(const mlxq_array* x, const mlxq_array* w,
                            const mlxq_array* scales, const mlxq_array* biases,
                            const mlxq_array* lhs_indices, const mlxq_array* rhs_indices,
                            bool transpose, int32_t group_size, int32_t bits,
                            bool sorted_indices, const char* mode,
                            const mlxq_array* global_scale, mlxq_array* out, void* stream);

mlxq_status mlxq_gather_qmm_shape(const mlxq_array* x, const mlxq_array* w,
                                  const mlxq_array* scales, const mlxq_array* biases,
                                  const mlxq_array* lhs_indices,
                                  const mlxq_array* rhs_indices, bool transpose,
                                  int32_t group_size, int32_t bits, const char* mode,
                                  int32_t* out_ndim, int64_t* out_shape,
                                  int32_t* out_dtype);

/* w_hat = dequantize(w, scales, biases), as mlx::core::dequantize
 * (ops.cpp:5753-5805).  Affine output is bit-exact to the MLX CPU graph
 * (ops.cpp:5531-5573): bf16(bf16(q*s) + b).  mxfp4 output is
 * LUT[q] * 2^(s-127) (exact; s == 255 gives NaN, ops.cpp:5692-5695); mxfp8
 * is from_fp8(q) * 2^(s-127) rounded once to bf16; nvfp4 (no global scale)
 * LUT[q] * from_fp8(s) (exact) (ops.cpp:5661-5695; e4m3 decoding as
 * rocm/quantized/convert_fp8.hip:68-90).
 * `dtype` < 0 selects the reference default (scales' dtype for affine,
 * bfloat16 for fp modes).  Affine: bits 1-6 and 8 with scales/biases
 * of one type T in {bfloat16, float16, float32} and any of those outputs,
 * To(T(T(q*s) + b)) bit-exactly (ops.cpp:5494-5586 then astype).  mxfp4
 * also to float16/float32 (the scale 2^(s-127) formed in the output type,
 * ops.cpp:5680-5690); mxfp8 and nvfp4 to bfloat16.  Any strides. */
mlxq_status mlxq_dequantize(const mlxq_array* w, const mlxq_array* scales,
                            const mlxq_array* biases, int32_t group_size, int32_t bits,
                            const char* mode, int32_t dtype, mlxq_array* out, void* stream);

/* (wq, scales[, biases]) = quantize(w), as mlx::core::quantize
 * (ops.cpp:5454-5492).  Affine follows the MLX CPU quantizer
 * (overlays/cpu/.../quantized.cpp:1233-1305) bit-exactly; mxfp4, mxfp8 and
 * nvfp4 (without a global scale) follow the graph quantizer
 * (ops.cpp:5364-5431) as the ROCm backend evaluates it, to_fp8 included
 * (rocm/quantized/convert_fp8.hip:18-66).  `biases_out` is ignored for fp
 * modes.  Affine: bfloat16, float16 or float32 w (scales and biases in w's
 * type), bits 1-6 and 8 (8 codes per `bits` bytes, the little-endian bit
 * stream of CPUQ:1283-1297); fp modes: bfloat16 w.  w row-contiguous and
 * 16-byte aligned. */
mlxq_status mlxq_quantize(const mlxq_array* w, int32_t group_size, int32_t bits,
                          const char* mode, mlxq_array* wq_out, mlxq_array* scales_out,
                          mlxq_array* biases_out, void* stream);

/* Fused single-token decode MoE with SwiGLU experts, as the reference's
 * fused_moe_expert_kernel:
 *   out[h] = sum_j scores[j] * down_e(silu(gate_e(x)) * up_e(x))[h],  e = indices[j]
 * x: bfloat16, din elements.  indices, scores: k elements (32/64-bit
 * integers; float32, bfloat16 or float16).  gate_w/up_w: uint32
 * (E, dff, din*gu_bits/32) with bfloat16 scales/biases (E, dff, din/group_size);
 * down_w: uint32 (E, din, dff*d_bits/32) with bfloat16 scales/biases
 * (E, din, dff/group_size); affine quantization.  out: bfloat16 (din).
 * Gate/up, the activation and every per-expert product are fp32; the sum over
 * the k experts is fp32 in a fixed order and rounded to bfloat16 once
 * (mlx_cxx_kernels.cpp:3886-3899).  Implemented: gu_bits 4/8, d_bits 4/6/8,
 * group_size 32/64/128; other valid configurations return MLXQ_EUNSUPPORTED
 * (the reference's callers then take their gather_qmm path).  Index values
 * past the expert count are clamped to E-1.  Uses the per-stream workspace
 * (k*dff fp32). */
mlxq_status mlxq_fused_moe_expert(const mlxq_array* x, const mlxq_array* indices,
                                  const mlxq_array* gate_w, const mlxq_array* gate_s,
                                  const mlxq_array* gate_b, const mlxq_array* up_w,
                                  const mlxq_array* up_s, const mlxq_array* up_b,
                                  const mlxq_array* down_w, const mlxq_array* down_s,
                                  const mlxq_array* down_b, const mlxq_array* scores, int32_t din,
                                  int32_t dff, int32_t k, int32_t gu_bits, int32_t d_bits,
                                  int32_t group_size, mlxq_array* out, void* stream);

/* Same with GeGLU experts (gemma4): gelu_tanh(gate) * up, as the reference's
 * fused_moe_geglu_kernel. */
mlxq_status mlxq_fused_moe_geglu(const mlxq_array* x, const mlxq_array* indices,
                                 const mlxq_array* gate_w, const mlxq_array* gate_s,
                                 const mlxq_array* gate_b, const mlxq_array* up_w,
                                 const mlxq_array* up_s, const mlxq_array* up_b,
                                 const mlxq_array* down_w, const mlxq_array* down_s,
                                 const mlxq_array* down_b, const mlxq_array* scores, int32_t din,
                                 int32_t dff, int32_t k, int32_t gu_bits, int32_t d_bits,
                                 int32_t group_size, mlxq_array* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MLXQ_H */
