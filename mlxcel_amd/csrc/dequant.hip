// dequant.hip — load-time conversions on gfx950: dequantize and quantize.
//
// Bit-exact to the MLX CPU definitions (built with -ffp-contract=off):
//  * affine dequantize: the CPU graph fallback, overlays/rocm/mlx/ops.cpp:5531-5573,
//    where uint32 x bf16 promotes to bf16 so each op rounds: bf16(bf16(q*s) + b).
//  * mxfp4 dequantize: ops.cpp:5646-5695, LUT[q] * 2^(s-127), s == 255 -> NaN;
//    built from integer fields so bf16 subnormal results are exact whatever the
//    hardware's float denormal mode.
//  * affine quantize: overlays/cpu/mlx/backend/cpu/quantized.cpp:1233-1305
//    (`quantize<bfloat16_t, uint32_t>`), including the edge snapping and the
//    codes computed with the unrounded float scale/bias; bits 2, 4, 6 and 8
//    (6-bit codes go out as 3-byte packs of 4, the bit stream of the codes).
//  * mxfp4 quantize: the graph fallback ops.cpp:5364-5431, every op rounded to
//    bf16 as MLX evaluates it; the shared exponent is the smallest e with
//    2^e >= bf16(max|w| / 6), which is what round(log2) + the round-up step
//    produce for every normal scale.
//  * mxfp8 / nvfp4 (e4m3 codes with e8m0 scales per 32 / e2m1 codes with e4m3
//    scales per 16, no global scale): the same graph fallbacks, with MLX's
//    to_fp8 as the ROCm backend evaluates it
//    (overlays/rocm/mlx/backend/rocm/quantized/convert_fp8.hip:18-90: half-up
//    mantissa rounding, saturation to 448 except the NaN code for [464, 496),
//    zero below 2^-9, truncated subnormals) and from_fp8's exact decode.
// All are HBM-bound streaming kernels (one word or one group per lane group).
#include "common.hpp"
#include "kernels.hpp"

namespace mlxq {

__device__ __forceinline__ float bfr(float f) { return bf16_bits_to_f32(f32_to_bf16_bits(f)); }

// ---- affine dequantize ------------------------------------------------------

template <int BITS>
__global__ __launch_bounds__(256) void affine_dequant_kernel(const uint32_t* __restrict__ w,
                                                             const uint16_t* __restrict__ scales,
                                                             const uint16_t* __restrict__ biases,
                                                             uint16_t* __restrict__ out,
                                                             int64_t nwords, int64_t Kw, int gs) {
  constexpr int PER = 32 / BITS;  // codes per word
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nwords) return;
  const int64_t row = i / Kw;
  const int64_t col = i - row * Kw;
  const int64_t k0 = col * PER;
  const int64_t G = Kw * PER / gs;
  const int64_t gi = row * G + k0 / gs;
  const float s = bf16_bits_to_f32(scales[gi]);
  const float b = bf16_bits_to_f32(biases[gi]);
  const uint32_t word = __builtin_nontemporal_load(w + i);
  uint32_t packed[PER / 2];
#pragma unroll
  for (int p = 0; p < PER; p += 2) {
    const float q0 = (float)((word >> (p * BITS)) & ((1u << BITS) - 1u));
    const float q1 = (float)((word >> ((p + 1) * BITS)) & ((1u << BITS) - 1u));
    const uint32_t h0 = f32_to_bf16_bits(bfr(q0 * s) + b);
    const uint32_t h1 = f32_to_bf16_bits(bfr(q1 * s) + b);
    packed[p / 2] = h0 | (h1 << 16);
  }
  uint32_t* dst = reinterpret_cast<uint32_t*>(out + row * (Kw * PER) + k0);
#pragma unroll
  for (int p = 0; p < PER / 2; p++) dst[p] = packed[p];
}

// 6-bit: one lane per 12-byte unit of 16 codes (four 3-byte packs; code j is
// bits 6j .. 6j+5 of the little-endian unit, quantized.cpp:1283-1297).
__global__ __launch_bounds__(256) void affine_dequant6_kernel(const uint32_t* __restrict__ w,
                                                              const uint16_t* __restrict__ scales,
                                                              const uint16_t* __restrict__ biases,
                                                              uint16_t* __restrict__ out, int64_t nunits,
                                                              int64_t upr, int gs) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nunits) return;
  const int64_t row = i / upr;
  const int64_t k0 = (i - row * upr) * 16;
  const int64_t gi = row * (upr * 16 / gs) + k0 / gs;
  const float s = bf16_bits_to_f32(scales[gi]);
  const float b = bf16_bits_to_f32(biases[gi]);
  const uint32_t u[3] = {w[3 * i], w[3 * i + 1], w[3 * i + 2]};
  u32x4 o[2];
#pragma unroll
  for (int p = 0; p < 16; p += 2) {
    uint32_t h[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int bit = 6 * (p + j), wi = bit >> 5, sh = bit & 31;
      const uint32_t c = sh <= 26 ? (u[wi] >> sh) & 63u : ((u[wi] >> sh) | (u[wi + 1] << (32 - sh))) & 63u;
      h[j] = f32_to_bf16_bits(bfr((float)c * s) + b);
    }
    o[p / 8][(p / 2) % 4] = h[0] | (h[1] << 16);
  }
  u32x4* dst = reinterpret_cast<u32x4*>(out + row * (upr * 16) + k0);
  dst[0] = o[0];
  dst[1] = o[1];
}

hipError_t launch_affine_dequantize(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                                    uint16_t* out, int64_t rows, int64_t K, int gs, int bits,
                                    hipStream_t stream) {
  if (bits == 6) {
    const int64_t nunits = rows * (K / 16);
    if (nunits == 0) return hipSuccess;
    hipLaunchKernelGGL(affine_dequant6_kernel, dim3((unsigned)((nunits + 255) / 256)), dim3(256), 0, stream, w,
                       scales, biases, out, nunits, K / 16, gs);
    return hipGetLastError();
  }
  const int64_t Kw = K * bits / 32;
  const int64_t nwords = rows * Kw;
  if (nwords == 0) return hipSuccess;
  const unsigned blocks = (unsigned)((nwords + 255) / 256);
  switch (bits) {
    case 2:
      hipLaunchKernelGGL(affine_dequant_kernel<2>, dim3(blocks), dim3(256), 0, stream, w, scales, biases,
                         out, nwords, Kw, gs);
      break;
    case 4:
      hipLaunchKernelGGL(affine_dequant_kernel<4>, dim3(blocks), dim3(256), 0, stream, w, scales, biases,
                         out, nwords, Kw, gs);
      break;
    default:
      hipLaunchKernelGGL(affine_dequant_kernel<8>, dim3(blocks), dim3(256), 0, stream, w, scales, biases,
                         out, nwords, Kw, gs);
      break;
  }
  return hipGetLastError();
}

// ---- mxfp4 dequantize -------------------------------------------------------

// bf16 bits of LUT[code] * 2^(s-127), exact (see file header).
__device__ __forceinline__ uint32_t mxfp4_value_bits(uint32_t code, uint32_t s) {
  if (s == 255u) return 0x7FC0u;
  const uint32_t sign = (code & 8u) << 12;
  const uint32_t mag = code & 7u;
  if (mag == 0u) return sign;
  // mag 1..7 -> 0.5, 1, 1.5, 2, 3, 4, 6 = m * 2^ex with m in {1, 1.5}
  const int ex = (mag == 1u) ? -1 : (int)((mag - 2u) >> 1);
  const uint32_t half = (mag >= 3u && (mag & 1u)) ? 1u : 0u;  // m == 1.5
  const int E = ex + (int)s;                                   // biased bf16 exponent
  if (E >= 255) return sign | 0x7F80u;                         // overflow to inf
  if (E >= 1) return sign | ((uint32_t)E << 7) | (half << 6);
  // subnormal: value = m * 2^(E-127) = mant * 2^-133
  const uint32_t mant = (half ? 3u : 2u) << (E + 5);           // (2 or 3) * 2^(E+6) / 2
  return sign | mant;
}

__global__ __launch_bounds__(256) void mxfp4_dequant_kernel(const uint32_t* __restrict__ w,
                                                            const uint8_t* __restrict__ scales,
                                                            uint16_t* __restrict__ out,
                                                            int64_t nwords) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nwords) return;
  const uint32_t word = __builtin_nontemporal_load(w + i);
  const uint32_t s = scales[i >> 2];  // 4 words (32 codes) per scale
  u32x4 o;
#pragma unroll
  for (int p = 0; p < 4; p++) {
    const uint32_t lo = mxfp4_value_bits((word >> (8 * p)) & 15u, s);
    const uint32_t hi = mxfp4_value_bits((word >> (8 * p + 4)) & 15u, s);
    o[p] = lo | (hi << 16);
  }
  *reinterpret_cast<u32x4*>(out + i * 8) = o;
}

hipError_t launch_mxfp4_dequantize(const uint32_t* w, const uint8_t* scales, uint16_t* out,
                                   int64_t rows, int64_t K, hipStream_t stream) {
  const int64_t nwords = rows * (K / 8);
  if (nwords == 0) return hipSuccess;
  hipLaunchKernelGGL(mxfp4_dequant_kernel, dim3((unsigned)((nwords + 255) / 256)), dim3(256), 0, stream, w,
                     scales, out, nwords);
  return hipGetLastError();
}

// ---- affine quantize --------------------------------------------------------
// GS/8 consecutive lanes own one group; each lane converts 8 consecutive
// values.  TI: element type of the weights and of the scales / biases written
// (GEN_BF16, GEN_F16, GEN_F32; MLX writes them in the weights' type).  The
// arithmetic is the reference CPU quantizer's (quantized.cpp:1251-1303) in
// float32, values widened exactly from TI.

template <int TI>
__device__ __forceinline__ float widen16(uint32_t h) {
  if constexpr (TI == GEN_F16) return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
  return bf16_bits_to_f32(h);
}

// static_cast<T>(v): round to nearest even
template <int TI>
__device__ __forceinline__ void store_typed(void* p, int64_t i, float v) {
  if constexpr (TI == GEN_F32) reinterpret_cast<float*>(p)[i] = v;
  else if constexpr (TI == GEN_F16) reinterpret_cast<_Float16*>(p)[i] = (_Float16)v;
  else reinterpret_cast<uint16_t*>(p)[i] = (uint16_t)f32_to_bf16_bits(v);
}

template <int TI, int BITS, int GS>
__global__ __launch_bounds__(256) void affine_quant_kernel(const void* __restrict__ w, uint32_t* __restrict__ wq,
                                                           void* __restrict__ scales, void* __restrict__ biases,
                                                           int64_t n_pieces) {
  constexpr int L = GS / 8;  // lanes per group
  const int64_t piece = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // 8 values each
  const bool live = piece < n_pieces;
  float vals[8];
  if constexpr (TI == GEN_F32) {
    u32x4 a = {0u, 0u, 0u, 0u}, b = {0u, 0u, 0u, 0u};
    if (live) {
      a = reinterpret_cast<const u32x4*>(w)[2 * piece];
      b = reinterpret_cast<const u32x4*>(w)[2 * piece + 1];
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      vals[i] = __uint_as_float(a[i]);
      vals[4 + i] = __uint_as_float(b[i]);
    }
  } else {
    u32x4 v = {0u, 0u, 0u, 0u};
    if (live) v = reinterpret_cast<const u32x4*>(w)[piece];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      vals[2 * i] = widen16<TI>(v[i] & 0xFFFFu);
      vals[2 * i + 1] = widen16<TI>(v[i] >> 16);
    }
  }
  // (a < b) ? b : a  /  (b < a) ? b : a  as std::max / std::min
  float w_max = -INFINITY, w_min = INFINITY;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    w_max = (w_max < vals[i]) ? vals[i] : w_max;
    w_min = (vals[i] < w_min) ? vals[i] : w_min;
  }
#pragma unroll
  for (int off = 1; off < L; off <<= 1) {
    const float omax = __shfl_xor(w_max, off);
    const float omin = __shfl_xor(w_min, off);
    w_max = (w_max < omax) ? omax : w_max;
    w_min = (omin < w_min) ? omin : w_min;
  }
  const float n_bins = (float)((1 << BITS) - 1);
  const float eps = 1e-7f;
  float scale, bias;
  if constexpr (BITS == 1) {
    // code 0 -> w_min, code 1 -> w_max (quantized.cpp:1261-1264)
    scale = w_max - w_min;
    scale = (scale < eps) ? eps : scale;
    bias = w_min;
  } else {
    const bool mask = fabsf(w_min) > fabsf(w_max);
    scale = (w_max - w_min) / n_bins;
    scale = (scale < eps) ? eps : scale;
    scale = mask ? scale : -scale;
    const float edge = mask ? w_min : w_max;
    const float q0 = rintf(edge / scale);
    bias = 0.0f;
    if (q0 != 0.0f) {
      scale = edge / q0;
      bias = edge;
    }
  }
  // 8 codes of BITS bits, low bits first: BITS bytes of the row's stream
  uint64_t all = 0;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    float q = rintf((vals[i] - bias) / scale);
    q = (q < 0.0f) ? 0.0f : q;
    q = (n_bins < q) ? n_bins : q;
    all |= (uint64_t)(uint32_t)q << (BITS * i);
  }
  if (live) {
    if constexpr (BITS == 4) {
      wq[piece] = (uint32_t)all;
    } else if constexpr (BITS == 8) {
      *reinterpret_cast<u32x2*>(wq + piece * 2) = u32x2{(uint32_t)all, (uint32_t)(all >> 32)};
    } else {
      uint8_t* d = reinterpret_cast<uint8_t*>(wq) + piece * BITS;
#pragma unroll
      for (int b = 0; b < BITS; b++) d[b] = (uint8_t)(all >> (8 * b));
    }
    if ((piece % L) == 0) {
      store_typed<TI>(scales, piece / L, scale);
      store_typed<TI>(biases, piece / L, bias);
    }
  }
}

template <int TI, int BITS>
static void launch_aq_bits(const void* w, uint32_t* wq, void* s, void* b, int64_t pieces, int gs,
                           hipStream_t stream) {
  const dim3 grid((unsigned)((pieces + 255) / 256));
  if (gs == 32)
    hipLaunchKernelGGL((affine_quant_kernel<TI, BITS, 32>), grid, dim3(256), 0, stream, w, wq, s, b, pieces);
  else if (gs == 64)
    hipLaunchKernelGGL((affine_quant_kernel<TI, BITS, 64>), grid, dim3(256), 0, stream, w, wq, s, b, pieces);
  else
    hipLaunchKernelGGL((affine_quant_kernel<TI, BITS, 128>), grid, dim3(256), 0, stream, w, wq, s, b, pieces);
}

template <int TI>
static void launch_aq_type(const void* w, uint32_t* wq, void* s, void* b, int64_t pieces, int gs, int bits,
                           hipStream_t stream) {
  switch (bits) {
    case 1: launch_aq_bits<TI, 1>(w, wq, s, b, pieces, gs, stream); break;
    case 2: launch_aq_bits<TI, 2>(w, wq, s, b, pieces, gs, stream); break;
    case 3: launch_aq_bits<TI, 3>(w, wq, s, b, pieces, gs, stream); break;
    case 4: launch_aq_bits<TI, 4>(w, wq, s, b, pieces, gs, stream); break;
    case 5: launch_aq_bits<TI, 5>(w, wq, s, b, pieces, gs, stream); break;
    case 6: launch_aq_bits<TI, 6>(w, wq, s, b, pieces, gs, stream); break;
    default: launch_aq_bits<TI, 8>(w, wq, s, b, pieces, gs, stream); break;
  }
}

hipError_t launch_affine_quantize(const void* w, int ti, uint32_t* wq, void* scales, void* biases, int64_t rows,
                                  int64_t K, int gs, int bits, hipStream_t stream) {
  const int64_t pieces = rows * K / 8;
  if (pieces == 0) return hipSuccess;
  if ((bits < 1 || bits > 8 || bits == 7) || (gs != 32 && gs != 64 && gs != 128) || ti < 0 || ti > 2)
    return hipErrorInvalidValue;
  if (ti == GEN_F32) launch_aq_type<GEN_F32>(w, wq, scales, biases, pieces, gs, bits, stream);
  else if (ti == GEN_F16) launch_aq_type<GEN_F16>(w, wq, scales, biases, pieces, gs, bits, stream);
  else launch_aq_type<GEN_BF16>(w, wq, scales, biases, pieces, gs, bits, stream);
  return hipGetLastError();
}

// ---- mxfp4 quantize ---------------------------------------------------------
// 4 lanes per group of 32 values, 8 values (one output word) per lane.

__device__ __forceinline__ int ceil_log2_pos(float s) {
  const uint32_t u = __float_as_uint(s);
  const int e = (int)(u >> 23);
  const uint32_t mant = u & 0x7FFFFFu;
  if (e != 0) return (e - 127) + (mant != 0u ? 1 : 0);
  // subnormal: s = mant * 2^-149
  return (32 - __clz((int)(mant - 1u))) - 149;
}

__global__ __launch_bounds__(256) void mxfp4_quant_kernel(const uint16_t* __restrict__ w,
                                                          uint32_t* __restrict__ wq,
                                                          uint8_t* __restrict__ scales,
                                                          int64_t n_pieces) {
  const float lut[16] = {+0.0f, +0.5f, +1.0f, +1.5f, +2.0f, +3.0f, +4.0f, +6.0f,
                         -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};
  const int64_t piece = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const bool live = piece < n_pieces;
  u32x4 v = {0u, 0u, 0u, 0u};
  if (live) v = *reinterpret_cast<const u32x4*>(w + piece * 8);
  float vals[8];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    vals[2 * i] = bf16_bits_to_f32(v[i] & 0xFFFFu);
    vals[2 * i + 1] = bf16_bits_to_f32(v[i] >> 16);
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const float a = fabsf(vals[i]);
    amax = (amax < a) ? a : amax;
  }
#pragma unroll
  for (int off = 1; off < 4; off <<= 1) {
    const float o = __shfl_xor(amax, off);
    amax = (amax < o) ? o : amax;
  }
  const float s = bfr(amax / 6.0f);
  const int e = (s == 0.0f) ? 0 : ceil_log2_pos(s);
  // power(bf16(2), e) in bf16: 2^e is exact in bf16 for e >= -133
  const float p = bf16_bits_to_f32(e >= -126 ? (uint32_t)(e + 127) << 7 : (0x40u >> (-127 - e)));
  uint32_t word = 0;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const float x = bfr(vals[i] / p);
    int best = 0;
    float best_d = INFINITY;
#pragma unroll
    for (int c = 0; c < 16; c++) {
      const float d = fabsf(bfr(x - lut[c]));
      if (d < best_d) {
        best_d = d;
        best = c;
      }
    }
    word |= (uint32_t)best << (4 * i);
  }
  if (live) wq[piece] = word;
  if (live && (piece & 3) == 0) scales[piece >> 2] = (uint8_t)(e + 127);
}

hipError_t launch_mxfp4_quantize(const uint16_t* w, uint32_t* wq, uint8_t* scales, int64_t rows,
                                 int64_t K, hipStream_t stream) {
  const int64_t pieces = rows * K / 8;
  if (pieces == 0) return hipSuccess;
  hipLaunchKernelGGL(mxfp4_quant_kernel, dim3((unsigned)((pieces + 255) / 256)), dim3(256), 0, stream, w,
                     wq, scales, pieces);
  return hipGetLastError();
}

// ---- fp8 e4m3 ----------------------------------------------------------------

// MLX to_fp8 on the ROCm backend (convert_fp8.hip:18-66), integer steps.
__device__ __forceinline__ uint32_t e4m3_encode(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7Fu;  // NaN
  const uint32_t sign = (u >> 24) & 0x80u;
  const int e = (int)((u >> 23) & 0xFFu) - 127;
  const uint32_t frac = u & 0x7FFFFFu;
  if (e < -9) return sign;
  if (e > 8) return sign | 0x7Eu;
  int be = e + 7;
  uint32_t m = (frac + 0x80000u) >> 20;
  if (m > 7u) {
    m = 0u;
    if (++be > 15) return sign | 0x7Eu;
  }
  if (be <= 0) {
    m = (frac | 0x800000u) >> (20 + (1 - be));
    be = 0;
  }
  return sign | ((uint32_t)be << 3) | (m & 7u);
}

// e4m3 code c as sign * M * 2^E (M < 16); false for the NaN codes
__device__ __forceinline__ bool e4m3_fields(uint32_t c, uint32_t& sign, uint32_t& M, int& E) {
  const uint32_t e = (c >> 3) & 15u, m = c & 7u;
  sign = (c & 0x80u) << 8;
  if (e == 15u && m == 7u) return false;
  if (e == 0u) {
    M = m;
    E = -9;
  } else {
    M = 8u + m;
    E = (int)e - 10;
  }
  return true;
}

__device__ __forceinline__ float e4m3_decode(uint32_t c) {
  uint32_t sign, M;
  int E;
  if (!e4m3_fields(c, sign, M, E)) return __uint_as_float(0x7FC00000u);
  const float v = __builtin_ldexpf((float)M, E);  // >= 2^-9: a normal float
  return sign ? -v : v;
}

// bf16 bits of sign * M * 2^E (M < 16), rounded to nearest even; integer
// arithmetic, so bf16 subnormal results do not depend on the float denormal mode
__device__ __forceinline__ uint32_t bf16_scaled(uint32_t sign, uint32_t M, int E) {
  if (M == 0u) return sign;
  const int p = 31 - __clz((int)M);  // M = 1.f * 2^p
  const int ex = E + p;
  if (ex > 127) return sign | 0x7F80u;
  if (ex >= -126) return sign | ((uint32_t)(ex + 127) << 7) | ((M - (1u << p)) << (7 - p));
  const int sh = E + 133;  // subnormal: value / 2^-133 = M * 2^sh
  if (sh >= 0) return sign | (M << sh);
  const int r = -sh;
  if (r > 5) return sign;  // below half the smallest subnormal
  uint32_t q = M >> r;
  const uint32_t rem = M & ((1u << r) - 1u), half = 1u << (r - 1);
  if (rem > half || (rem == half && (q & 1u))) q++;
  return sign | q;
}

// ---- mxfp8 dequantize: from_fp8(code) * 2^(s-127), one bf16 rounding ---------

__global__ __launch_bounds__(256) void mxfp8_dequant_kernel(const uint32_t* __restrict__ w,
                                                            const uint8_t* __restrict__ scales,
                                                            uint16_t* __restrict__ out, int64_t npairs) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // 8 codes (2 words)
  if (i >= npairs) return;
  const u32x2 wd = *reinterpret_cast<const u32x2*>(w + 2 * i);
  const uint32_t s = scales[i >> 2];  // 32 codes per scale
  u32x4 o;
#pragma unroll
  for (int q = 0; q < 8; q++) {
    const uint32_t c = (wd[q >> 2] >> (8 * (q & 3))) & 0xFFu;
    uint32_t sign, M, bits;
    int E;
    if (s == 255u || !e4m3_fields(c, sign, M, E)) bits = 0x7FC0u;
    else bits = bf16_scaled(sign, M, E + (int)s - 127);
    if (q & 1) o[q >> 1] |= bits << 16;
    else o[q >> 1] = bits;
  }
  *reinterpret_cast<u32x4*>(out + 8 * i) = o;
}

// ---- nvfp4 dequantize: LUT[code] * from_fp8(scale), exact in bf16 ------------

__global__ __launch_bounds__(256) void nvfp4_dequant_kernel(const uint32_t* __restrict__ w,
                                                            const uint8_t* __restrict__ scales,
                                                            uint16_t* __restrict__ out, int64_t nwords) {
  const float lut[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nwords) return;
  const uint32_t word = w[i];
  const float sc = e4m3_decode(scales[i >> 1]);  // 16 codes per scale
  u32x4 o;
#pragma unroll
  for (int q = 0; q < 8; q++) {
    const uint32_t c = (word >> (4 * q)) & 15u;
    float v = lut[c & 7u] * sc;  // products of <= 6 significant bits: exact
    if (c & 8u) v = -v;
    const uint32_t bits = f32_to_bf16_bits(v);
    if (q & 1) o[q >> 1] |= bits << 16;
    else o[q >> 1] = bits;
  }
  *reinterpret_cast<u32x4*>(out + 8 * i) = o;
}

hipError_t launch_fp_dequantize(int mode, const uint32_t* w, const uint8_t* scales, uint16_t* out, int64_t rows,
                                int64_t K, hipStream_t stream) {
  if (mode == FP_MXFP8) {
    const int64_t n = rows * K / 8;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(mxfp8_dequant_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, w, scales,
                       out, n);
  } else {
    const int64_t n = rows * K / 8;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(nvfp4_dequant_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, w, scales,
                       out, n);
  }
  return hipGetLastError();
}

// ---- mxfp8 quantize: 4 lanes per group of 32, 8 values (2 words) per lane ----

__global__ __launch_bounds__(256) void mxfp8_quant_kernel(const uint16_t* __restrict__ w,
                                                          uint32_t* __restrict__ wq,
                                                          uint8_t* __restrict__ scales, int64_t n_pieces) {
  const int64_t piece = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const bool live = piece < n_pieces;
  u32x4 v = {0u, 0u, 0u, 0u};
  if (live) v = *reinterpret_cast<const u32x4*>(w + piece * 8);
  float vals[8];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    vals[2 * i] = bf16_bits_to_f32(v[i] & 0xFFFFu);
    vals[2 * i + 1] = bf16_bits_to_f32(v[i] >> 16);
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const float a = fabsf(vals[i]);
    amax = (amax < a) ? a : amax;
  }
#pragma unroll
  for (int off = 1; off < 4; off <<= 1) {
    const float o = __shfl_xor(amax, off);
    amax = (amax < o) ? o : amax;
  }
  const float s = bfr(amax / 448.0f);
  const int e = (s == 0.0f) ? 0 : ceil_log2_pos(s);
  const float p = bf16_bits_to_f32(e >= -126 ? (uint32_t)(e + 127) << 7 : (0x40u >> (-127 - e)));
  u32x2 out = {0u, 0u};
#pragma unroll
  for (int i = 0; i < 8; i++) out[i >> 2] |= e4m3_encode(bfr(vals[i] / p)) << (8 * (i & 3));
  if (live) *reinterpret_cast<u32x2*>(wq + 2 * piece) = out;
  if (live && (piece & 3) == 0) scales[piece >> 2] = (uint8_t)(e + 127);
}

// ---- nvfp4 quantize: 2 lanes per group of 16, 8 values (1 word) per lane ----

__global__ __launch_bounds__(256) void nvfp4_quant_kernel(const uint16_t* __restrict__ w,
                                                          uint32_t* __restrict__ wq,
                                                          uint8_t* __restrict__ scales, int64_t n_pieces) {
  const float lut[16] = {+0.0f, +0.5f, +1.0f, +1.5f, +2.0f, +3.0f, +4.0f, +6.0f,
                         -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};
  const int64_t piece = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const bool live = piece < n_pieces;
  u32x4 v = {0u, 0u, 0u, 0u};
  if (live) v = *reinterpret_cast<const u32x4*>(w + piece * 8);
  float vals[8];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    vals[2 * i] = bf16_bits_to_f32(v[i] & 0xFFFFu);
    vals[2 * i + 1] = bf16_bits_to_f32(v[i] >> 16);
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const float a = fabsf(vals[i]);
    amax = (amax < a) ? a : amax;
  }
  const float o = __shfl_xor(amax, 1);
  amax = (amax < o) ? o : amax;
  const uint32_t sc = e4m3_encode(bfr(amax / 6.0f));
  const float d = e4m3_decode(sc);
  uint32_t word = 0;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    // bf16 quotient; float32 distances (exact); the first minimum wins, and a
    // NaN or infinite quotient (zero scale) keeps code 0
    const float x = bfr(vals[i] / d);
    int best = 0;
    float best_d = INFINITY;
#pragma unroll
    for (int c = 0; c < 16; c++) {
      const float dist = fabsf(x - lut[c]);
      if (dist < best_d) {
        best_d = dist;
        best = c;
      }
    }
    word |= (uint32_t)best << (4 * i);
  }
  if (live) wq[piece] = word;
  if (live && (piece & 1) == 0) scales[piece >> 1] = (uint8_t)sc;
}

hipError_t launch_fp_quantize(int mode, const uint16_t* w, uint32_t* wq, uint8_t* scales, int64_t rows, int64_t K,
                              hipStream_t stream) {
  const int64_t pieces = rows * K / 8;
  if (pieces == 0) return hipSuccess;
  if (mode == FP_MXFP8)
    hipLaunchKernelGGL(mxfp8_quant_kernel, dim3((unsigned)((pieces + 255) / 256)), dim3(256), 0, stream, w, wq,
                       scales, pieces);
  else
    hipLaunchKernelGGL(nvfp4_quant_kernel, dim3((unsigned)((pieces + 255) / 256)), dim3(256), 0, stream, w, wq,
                       scales, pieces);
  return hipGetLastError();
}

// ---- dequantize for every element type and code width -------------------
// Affine (ops.cpp:5494-5586, then astype to the requested type at 5788-5793):
// the graph multiplies the codes by the scales in the scales' type T and adds
// the biases in T, each op rounded to T, then casts to the output type:
//   out = To(T(T(q * s) + b))   (T, To in {bfloat16, float16, float32}).
// mxfp4 to float16 / float32 (ops.cpp:5646-5695 with out_type): the scale
// 2^(s-127) is formed in the output type (float16: rounded, so it is 0 below
// 2^-25 and inf from 2^16), times the LUT value, rounded once; s == 255 -> NaN.
// One thread per 32-code piece (`bits` words), codes read as the little-endian
// bit stream of the packed row (quantized.cpp:107-137).

namespace {

template <int T>
__device__ __forceinline__ float round_to(float f) {
  if constexpr (T == GEN_BF16) return bfr(f);
  else if constexpr (T == GEN_F16) return (float)(_Float16)f;
  else return f;
}

template <int T>
__device__ __forceinline__ float load_t(const void* p, int64_t i) {
  if constexpr (T == GEN_F32) return static_cast<const float*>(p)[i];
  else if constexpr (T == GEN_BF16) return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  else return (float)__builtin_bit_cast(_Float16, static_cast<const uint16_t*>(p)[i]);
}

template <int T>
__device__ __forceinline__ void store_t(void* p, int64_t i, float v) {
  if constexpr (T == GEN_F32) static_cast<float*>(p)[i] = v;
  else if constexpr (T == GEN_BF16) static_cast<uint16_t*>(p)[i] = (uint16_t)f32_to_bf16_bits(v);
  else static_cast<uint16_t*>(p)[i] = __builtin_bit_cast(uint16_t, (_Float16)v);
}

__device__ __forceinline__ uint32_t piece_code(const uint32_t* wp, int j, int bits) {
  const int sb = j * bits, d = sb >> 5, sh = sb & 31;
  uint64_t v = wp[d];
  if (sh + bits > 32) v |= (uint64_t)wp[d + 1] << 32;
  return (uint32_t)(v >> sh) & ((1u << bits) - 1u);
}

}  // namespace

template <int TS, int TO>
__global__ __launch_bounds__(256) void gen_affine_dequant_kernel(const uint32_t* __restrict__ w, const void* scales,
                                                                 const void* biases, void* out, int64_t npieces,
                                                                 int64_t ppr, int gs_shift, int bits) {
  const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= npieces) return;
  const int64_t row = p / ppr, c = p - row * ppr;
  const int64_t K = ppr * 32;
  const int64_t g = row * (K >> gs_shift) + ((c * 32) >> gs_shift);
  const float sc = load_t<TS>(scales, g), bi = load_t<TS>(biases, g);
  const uint32_t* wp = w + p * bits;
  for (int j = 0; j < 32; j++) {
    const float q = (float)piece_code(wp, j, bits);
    store_t<TO>(out, row * K + c * 32 + j, round_to<TS>(round_to<TS>(q * sc) + bi));
  }
}

template <int TO>
__global__ __launch_bounds__(256) void gen_mxfp4_dequant_kernel(const uint32_t* __restrict__ w,
                                                                const uint8_t* __restrict__ scales, void* out,
                                                                int64_t npieces) {
  const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= npieces) return;
  const uint32_t s = scales[p];
  // 2^(s-127) in the output type (exact in float32, whose subnormals reach 2^-149)
  float scale = s == 255u ? __builtin_nanf("") : __builtin_ldexpf(1.0f, (int)s - 127);
  scale = round_to<TO>(scale);
  const uint32_t* wp = w + p * 4;
  for (int j = 0; j < 32; j++) {
    const uint32_t code = (wp[j >> 3] >> (4 * (j & 7))) & 15u;
    const float mag = (code & 6u) == 0 ? 0.5f * (float)(code & 1u)
                                       : (1.0f + 0.5f * (float)(code & 1u)) * (float)(1u << (((code >> 1) & 3u) - 1u));
    store_t<TO>(out, p * 32 + j, ((code & 8u) ? -mag : mag) * scale);
  }
}

hipError_t launch_gen_dequantize(int mode, const uint32_t* w, const void* scales, const void* biases, void* out,
                                 int64_t rows, int64_t K, int gs, int bits, int ts, int to, hipStream_t stream) {
  if (K % 32 != 0) return hipErrorInvalidValue;
  const int64_t npieces = rows * (K / 32);
  if (npieces == 0) return hipSuccess;
  const dim3 grid((unsigned)((npieces + 255) / 256)), block(256);
  if (mode == GEN_MXFP4) {
    if (to == GEN_F32) hipLaunchKernelGGL(gen_mxfp4_dequant_kernel<GEN_F32>, grid, block, 0, stream, w,
                                          static_cast<const uint8_t*>(scales), out, npieces);
    else if (to == GEN_F16) hipLaunchKernelGGL(gen_mxfp4_dequant_kernel<GEN_F16>, grid, block, 0, stream, w,
                                               static_cast<const uint8_t*>(scales), out, npieces);
    else return hipErrorInvalidValue;
    return hipGetLastError();
  }
  int shift = 0;
  while ((1 << shift) < gs) shift++;
#define GDQ(TS_, TO_)                                                                                          \
  if (ts == TS_ && to == TO_) {                                                                                \
    hipLaunchKernelGGL((gen_affine_dequant_kernel<TS_, TO_>), grid, block, 0, stream, w, scales, biases, out, \
                       npieces, K / 32, shift, bits);                                                          \
    return hipGetLastError();                                                                                  \
  }
  GDQ(GEN_BF16, GEN_BF16) GDQ(GEN_BF16, GEN_F16) GDQ(GEN_BF16, GEN_F32)
  GDQ(GEN_F16, GEN_BF16) GDQ(GEN_F16, GEN_F16) GDQ(GEN_F16, GEN_F32)
  GDQ(GEN_F32, GEN_BF16) GDQ(GEN_F32, GEN_F16) GDQ(GEN_F32, GEN_F32)
#undef GDQ
  return hipErrorInvalidValue;
}

}  // namespace mlxq
