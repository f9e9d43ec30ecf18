/*
 * mlxq_oracle.c — CPU restatement of MLX's quantized matmul, quantize and
 * dequantize, as built into mlxcel.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the GPU path and the timed
 * single-core CPU baseline.  The product library never links or calls it.
 *
 * Built with -ffp-contract=off so float expressions round exactly as the
 * reference's scalar loops do on an x86 host without FMA contraction.
 * Citations: CPUQ = src/lib/mlxcelverse/overlays/cpu/mlx/backend/cpu/quantized.cpp,
 * ROPS = src/lib/mlxcelverse/overlays/rocm/mlx/ops.cpp,
 * QAFF = src/lib/mlxcelverse/overlays/rocm/mlx/backend/rocm/quantized/affine_quantize.hip,
 * FP8C = src/lib/mlxcelverse/overlays/rocm/mlx/backend/rocm/quantized/convert_fp8.hip.
 *
 * Parity pins (tests/test_oracle.py): hand-computed known answers, torch's
 * independent bf16 arithmetic for both dequantize roundings, exhaustive
 * mxfp4 table vs ldexp, f64 matmul of the dequantized weights (the
 * reference's own test method, cpu_qmm_accum_tests.rs:237-287), one-hot and
 * all-ones activations with exact closed forms, and quantizer invariants.
 * The affine quantizer is pinned by hand-worked groups (bf16-unrepresentable
 * scales, rint ties of both parities in the codes and in q0, the
 * |w_min| == |w_max| branch, a clamped extreme) and by an independent numpy
 * float32 restatement on random data; the mxfp4 quantizer by hand-worked
 * groups (exponent round-up, first-minimum ties) and an exact argmin check.
 * tests/test_oracle_mutants.py plants one mistake at a time in a copy of this
 * file (bf16 scale in the codes, roundf for rint, >= for >, no clamp, no
 * snap, last-minimum ties, no exponent round-up) and requires the pins to
 * reject each.  Unpinned beyond invariants: the exact bits of MLX's bf16 log2 inside the
 * mxfp4 graph quantizer (shown not to change the chosen exponent for normal
 * scales), and MLX's NaN sign on conversion.
 */
#include "mlxq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---- bf16 (MLX `_MLX_BFloat16`: RNE, NaN -> 0x7FC0) ------------------------ */

uint16_t oracle_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if (isnan(f)) return 0x7FC0;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float oracle_bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

void oracle_f32_to_bf16_n(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; i++) out[i] = oracle_f32_to_bf16(in[i]);
}

void oracle_bf16_to_f32_n(const uint16_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; i++) out[i] = oracle_bf16_to_f32(in[i]);
}

/* ---- float16 (IEEE binary16: 1 sign, 5 exponent, 10 mantissa bits) -------- */

float oracle_f16_to_f32(uint16_t h) {
  const int sign = h >> 15, e = (h >> 10) & 31, m = h & 1023;
  float v;
  if (e == 0) v = ldexpf((float)m, -24);                     /* zero, subnormal */
  else if (e == 31) v = m ? NAN : INFINITY;
  else v = ldexpf((float)(1024 + m), e - 25);
  return sign ? -v : v;
}

/* round to nearest, ties to even; overflow to infinity; NaN -> 0x7E00 */
uint16_t oracle_f32_to_f16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return sign | 0x7E00u;
  if (a >= 0x477FF000u) return sign | 0x7C00u;  /* >= 65520: rounds past 65504 */
  if (a >= 0x38800000u) {                        /* >= 2^-14: normal */
    uint32_t r = ((((a >> 23) - 112u) << 10) | ((a >> 13) & 1023u));
    const uint32_t rem = a & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
    return sign | (uint16_t)r;
  }
  float av;
  memcpy(&av, &a, 4);
  return sign | (uint16_t)rintf(av * 16777216.0f); /* subnormal: units of 2^-24 */
}

/* bf16 binary op as MLX evaluates it on the CPU: widen, operate in float,
 * round the float result to bf16. */
static inline float bf(float f) { return oracle_bf16_to_f32(oracle_f32_to_bf16(f)); }

/* std::max / std::min on floats: (a < b) ? b : a  and  (b < a) ? b : a. */
static inline float std_max(float a, float b) { return (a < b) ? b : a; }
static inline float std_min(float a, float b) { return (b < a) ? b : a; }

static int pow2_bits(int bits) { return bits == 1 || bits == 2 || bits == 4 || bits == 8; }
/* widths with an affine packing here: the power-of-two ones and 6 */
static int affine_bits(int bits) { return pow2_bits(bits) || bits == 6; }
static int valid_gs(int gs) { return gs == 32 || gs == 64 || gs == 128; }

/* Code i of a packed row.  Power-of-two widths pack 32/bits codes per uint32,
 * low bits first (CPUQ:1283-1290; ROPS:5231-5238); 6-bit packs 4 codes per 3
 * bytes, little-endian, code k at bit 6k of the 24-bit pack (CPUQ:1238-1240,
 * 1283-1297: pack factor 4, 3 bytes per pack). */
static inline uint32_t code_at(const uint32_t* row, int bits, int64_t i) {
  if (bits == 6) {
    const uint8_t* b = (const uint8_t*)row + (i / 4) * 3;
    uint32_t pack = (uint32_t)b[0] | ((uint32_t)b[1] << 8) | ((uint32_t)b[2] << 16);
    return (pack >> ((i % 4) * 6)) & 63u;
  }
  int per = 32 / bits;
  return (row[i / per] >> ((i % per) * bits)) & ((1u << bits) - 1u);
}

/* ---- affine quantize: CPUQ:1233-1305 ------------------------------------ */

/* element i of an array of dtype 0 = bfloat16, 1 = float16, 2 = float32, as
 * float (exact for all three) */
static inline float load_as_f32(const void* a, int dtype, int64_t i) {
  if (dtype == 2) return ((const float*)a)[i];
  const uint16_t h = ((const uint16_t*)a)[i];
  return dtype == 1 ? oracle_f16_to_f32(h) : oracle_bf16_to_f32(h);
}

/* static_cast<T>(f) for the scale and bias outputs */
static inline void store_from_f32(void* a, int dtype, int64_t i, float f) {
  if (dtype == 2) ((float*)a)[i] = f;
  else ((uint16_t*)a)[i] = dtype == 1 ? oracle_f32_to_f16(f) : oracle_f32_to_bf16(f);
}

/* Any width of 1-6 or 8 bits: the reference packs power-of-two widths
 * 32/bits codes per uint32 (CPUQ:1283-1285) and 3/5/6 bits as 8, 8 and 4
 * codes per 3, 5 and 3 bytes (CPUQ:1286-1297), low bits first; both are the
 * one little-endian bit stream, written here as 8 codes per `bits` bytes. */
int oracle_affine_quantize_t(const void* w, int dtype, int64_t rows, int64_t K, int group_size, int bits,
                             uint32_t* wq, void* scales, void* biases) {
  if (bits < 1 || bits > 8 || bits == 7 || !valid_gs(group_size) || K % group_size || dtype < 0 || dtype > 2)
    return -1;
  const float n_bins = (float)((1 << bits) - 1);
  const float eps = 1e-7f;
  const int el_per_int = 8;                 /* codes per pack */
  const int bytes_per_pack = bits;
  const int64_t int_per_group = (int64_t)group_size / el_per_int;
  const int64_t n_groups = rows * (K / group_size);

  for (int64_t i = 0; i < n_groups; ++i) {
    const int64_t g = i * group_size;
    float w_min = INFINITY;
    float w_max = -w_min;
    for (int j = 0; j < group_size; ++j) {
      float v = load_as_f32(w, dtype, g + j);
      w_max = std_max(w_max, v);
      w_min = std_min(w_min, v);
    }
    int mask = fabsf(w_min) > fabsf(w_max);
    float scale, bias;
    if (bits == 1) {
      scale = std_max(w_max - w_min, eps);
      bias = w_min;
    } else {
      scale = std_max((w_max - w_min) / n_bins, eps);
      scale = mask ? scale : -scale;
      float edge = mask ? w_min : w_max;
      float q0 = rintf(edge / scale);
      bias = 0;
      if (q0 != 0) {
        scale = edge / q0;
        bias = edge;
      }
    }
    uint8_t* out = (uint8_t*)wq + i * int_per_group * bytes_per_pack;
    for (int64_t j = 0; j < int_per_group; ++j) {
      uint64_t out_el = 0;
      for (int k = 0; k < el_per_int; ++k) {
        float w_el = load_as_f32(w, dtype, g + j * el_per_int + k);
        w_el = rintf((w_el - bias) / scale);
        w_el = std_min(std_max(w_el, 0.0f), n_bins);
        out_el |= (uint64_t)w_el << (k * bits);
      }
      for (int b = 0; b < bytes_per_pack; ++b) out[j * bytes_per_pack + b] = (uint8_t)(out_el >> (8 * b));
    }
    store_from_f32(scales, dtype, i, scale);
    store_from_f32(biases, dtype, i, bias);
  }
  return 0;
}

int oracle_affine_quantize(const uint16_t* w, int64_t rows, int64_t K, int group_size,
                           int bits, uint32_t* wq, uint16_t* scales, uint16_t* biases) {
  if (!affine_bits(bits)) return -1;
  return oracle_affine_quantize_t(w, 0, rows, K, group_size, bits, wq, scales, biases);
}

/* ---- affine dequantize: ROPS:5531-5573 (graph) and QAFF:164 (GPU) -------- */

int oracle_affine_dequantize(const uint32_t* wq, const uint16_t* scales,
                             const uint16_t* biases, int64_t rows, int64_t K,
                             int group_size, int bits, int rounding, uint16_t* out) {
  if (!affine_bits(bits) || group_size <= 0 || K % group_size || (K * bits) % 32) return -1;
  const int64_t wcols = K * bits / 32;
  const int64_t G = K / group_size;
  for (int64_t r = 0; r < rows; r++) {
    const uint32_t* row = wq + r * wcols;
    for (int64_t k = 0; k < K; k++) {
      float q = (float)code_at(row, bits, k);
      float s = oracle_bf16_to_f32(scales[r * G + k / group_size]);
      float b = oracle_bf16_to_f32(biases[r * G + k / group_size]);
      float v;
      if (rounding == 2) {
        /* uint32 x bf16 promotes to bf16 (upstream type_rules), so the
         * product is stored as bf16 before the bf16 add. */
        v = bf(bf(q * s) + b);
      } else {
        v = s * q + b;
      }
      out[r * K + k] = oracle_f32_to_bf16(v);
    }
  }
  return 0;
}

/* ---- mxfp4 -------------------------------------------------------------- */

/* CPUQ:73-90 */
static const float FP4_LUT[16] = {+0.0f, +0.5f, +1.0f, +1.5f, +2.0f, +3.0f, +4.0f, +6.0f,
                                  -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

/* CPUQ:91-105 */
uint16_t oracle_e8m0_to_bf16(uint8_t s) {
  return (s == 0) ? 0x40 : (s == 0xFF ? 0x7FC0 : (uint16_t)((uint16_t)s << 7));
}

/* ROPS:5364-5431, e8m0 branch, every op on bf16 arrays rounded as MLX does. */
int oracle_mxfp4_quantize(const uint16_t* w, int64_t rows, int64_t K, uint32_t* wq,
                          uint8_t* scales) {
  if (K % 32) return -1;
  const int64_t n_groups = rows * (K / 32);
  for (int64_t i = 0; i < n_groups; i++) {
    const uint16_t* g = w + i * 32;
    /* scales = max(abs(wq)) / bf16(6.0) */
    float amax = 0.0f;
    for (int j = 0; j < 32; j++) amax = std_max(amax, fabsf(oracle_bf16_to_f32(g[j])));
    float s = bf(amax / 6.0f);
    float e_bf; /* `scales` after the where(): bf16 holding the exponent */
    if (s == 0.0f) {
      e_bf = 0.0f;
    } else {
      /* exponent = int32(round(log2(scales))) in bf16 */
      int e = (int)rintf(bf(log2f(s)));
      /* decoded = 2^exponent in float32; round up if it is below the scale */
      float decoded = ldexpf(1.0f, e);
      if (decoded < s) e += 1;
      e_bf = bf((float)e);
    }
    /* wq = wq / power(bf16(2), scales) in bf16 */
    float p = bf(powf(2.0f, e_bf));
    uint32_t words[4] = {0, 0, 0, 0};
    for (int j = 0; j < 32; j++) {
      float v = bf(oracle_bf16_to_f32(g[j]) / p);
      /* argmin(|bf16(v - lut)|), first minimum wins */
      int best = 0;
      float best_d = INFINITY;
      for (int c = 0; c < 16; c++) {
        float d = fabsf(bf(v - FP4_LUT[c]));
        if (d < best_d) {
          best_d = d;
          best = c;
        }
      }
      words[j / 8] |= (uint32_t)best << (4 * (j % 8));
    }
    memcpy(wq + i * 4, words, sizeof(words));
    /* scales = uint8(bf16(scales + 127)) */
    scales[i] = (uint8_t)bf(e_bf + 127.0f);
  }
  return 0;
}

/* ROPS:5646-5695: LUT in the output dtype, scale 2^(s-127) in bf16, 0xFF -> NaN. */
int oracle_mxfp4_dequantize(const uint32_t* wq, const uint8_t* scales, int64_t rows,
                            int64_t K, uint16_t* out) {
  if (K % 32) return -1;
  const int64_t G = K / 32;
  for (int64_t r = 0; r < rows; r++) {
    const uint32_t* row = wq + r * (K / 8);
    for (int64_t k = 0; k < K; k++) {
      uint8_t s = scales[r * G + k / 32];
      float v;
      if (s == 0xFF) {
        v = NAN;
      } else {
        float sc = bf(powf(2.0f, bf((float)s - 127.0f)));
        v = bf(FP4_LUT[code_at(row, 4, k)] * sc);
      }
      out[r * K + k] = oracle_f32_to_bf16(v);
    }
  }
  return 0;
}

/* ---- fp8 e4m3 (MLX to_fp8 / from_fp8) ------------------------------------- */

/* The ROCm backend's to_fp8 encoder, FP8C:18-66 (float_to_fp8_e4m3): NaN ->
 * 0x7F; exponents below -9 -> signed zero; above 8 -> 0x7E (448); the 23-bit
 * mantissa rounded to 3 bits by adding half a unit and truncating (ties away
 * from zero); a carry into the exponent past 15 -> 0x7E; results below the
 * normal range keep (1.mant) >> (1 - exponent) truncated. */
uint8_t oracle_e4m3_encode(float f) {
  if (isnan(f)) return 0x7F;
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint8_t sign = (uint8_t)((u >> 31) << 7);
  const int e = (int)((u >> 23) & 0xFFu) - 127;
  const uint32_t frac = u & 0x7FFFFFu;
  if (e < -9) return sign;
  if (e > 8) return sign | 0x7E;
  int be = e + 7;                      /* biased e4m3 exponent */
  uint32_t m = (frac + 0x80000u) >> 20; /* 3 mantissa bits, half-up */
  if (m > 7) {
    m = 0;
    if (++be > 15) return sign | 0x7E;
  }
  if (be <= 0) {
    m = (frac | 0x800000u) >> (20 + (1 - be));
    be = 0;
  }
  return sign | (uint8_t)((be & 0xF) << 3) | (uint8_t)(m & 7u);
}

/* FP8C:68-90 (fp8_e4m3_to_float): e4m3fn, exponent bias 7, no infinities,
 * 0x7F / 0xFF NaN, subnormals m * 2^-9. */
float oracle_e4m3_decode(uint8_t c) {
  const int e = (c >> 3) & 0xF, m = c & 7;
  float v;
  if (e == 15 && m == 7) return NAN;
  if (e == 0) v = ldexpf((float)m, -9);
  else v = ldexpf((float)(8 + m), e - 10);
  return (c & 0x80) ? -v : v;
}

void oracle_e4m3_encode_n(const float* in, uint8_t* out, int64_t n) {
  for (int64_t i = 0; i < n; i++) out[i] = oracle_e4m3_encode(in[i]);
}

void oracle_e4m3_decode_n(const uint8_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; i++) out[i] = oracle_e4m3_decode(in[i]);
}

/* The e8m0 exponent of the mx graph quantizers (ROPS:5384-5396) for the bf16
 * scale s: round(log2(s)) in bf16, plus one when 2^that is below s; 0 for s == 0. */
static int mx_exponent(float s) {
  if (s == 0.0f) return 0;
  int e = (int)rintf(bf(log2f(s)));
  if (ldexpf(1.0f, e) < s) e += 1;
  return e;
}

/* mxfp8 quantize, the graph fallback of ROPS:5364-5431 with bits 8, group 32:
 * scale = bf16(max|w| / 448), e8m0 exponent as for mxfp4, codes =
 * to_fp8(bf16(w / 2^e)) (FP8C encoder), 4 codes per uint32 low byte first
 * (view as uint32). */
int oracle_mxfp8_quantize(const uint16_t* w, int64_t rows, int64_t K, uint32_t* wq, uint8_t* scales) {
  if (K % 32) return -1;
  const int64_t n_groups = rows * (K / 32);
  uint8_t* out = (uint8_t*)wq;
  for (int64_t i = 0; i < n_groups; i++) {
    const uint16_t* g = w + i * 32;
    float amax = 0.0f;
    for (int j = 0; j < 32; j++) amax = std_max(amax, fabsf(oracle_bf16_to_f32(g[j])));
    const int e = mx_exponent(bf(amax / 448.0f));
    const float p = bf(powf(2.0f, (float)e));
    for (int j = 0; j < 32; j++) out[i * 32 + j] = oracle_e4m3_encode(bf(oracle_bf16_to_f32(g[j]) / p));
    scales[i] = (uint8_t)(e + 127);
  }
  return 0;
}

/* mxfp8 dequantize, ROPS:5682, 5692-5695: from_fp8(byte) * 2^(s-127) in bf16,
 * s == 0xFF -> NaN. */
int oracle_mxfp8_dequantize(const uint32_t* wq, const uint8_t* scales, int64_t rows, int64_t K,
                            uint16_t* out) {
  if (K % 32) return -1;
  const uint8_t* codes = (const uint8_t*)wq;
  for (int64_t i = 0; i < rows * K; i++) {
    const uint8_t s = scales[i / 32];
    float v;
    if (s == 0xFF) {
      v = NAN;
    } else {
      const float sc = bf(powf(2.0f, bf((float)s - 127.0f)));
      v = bf(bf(oracle_e4m3_decode(codes[i])) * sc);
    }
    out[i] = oracle_f32_to_bf16(v);
  }
  return 0;
}

/* nvfp4 quantize without a global scale, the graph fallback of
 * ROPS:5364-5382, 5402-5424 with group 16: scale = bf16(max|w| / 6) (bf16
 * divide), times the float32 1.0 of scale_encode (the product is float32),
 * to_fp8 (FP8C encoder); w / from_fp8(scale) in bf16, times that float32 1.0
 * (float32), so the LUT distances are float32 (exact); argmin keeps the first
 * minimum (a zero scale gives NaN or infinite quotients whose distances never
 * compare smaller: code 0). */
int oracle_nvfp4_quantize(const uint16_t* w, int64_t rows, int64_t K, uint32_t* wq, uint8_t* scales) {
  if (K % 16) return -1;
  const int64_t n_groups = rows * (K / 16);
  for (int64_t i = 0; i < n_groups; i++) {
    const uint16_t* g = w + i * 16;
    float amax = 0.0f;
    for (int j = 0; j < 16; j++) amax = std_max(amax, fabsf(oracle_bf16_to_f32(g[j])));
    const uint8_t sc = oracle_e4m3_encode(bf(amax / 6.0f));
    const float d = bf(oracle_e4m3_decode(sc));
    uint32_t words[2] = {0, 0};
    for (int j = 0; j < 16; j++) {
      const float v = bf(oracle_bf16_to_f32(g[j]) / d);
      int best = 0;
      float best_d = INFINITY;
      for (int c = 0; c < 16; c++) {
        const float dist = fabsf(v - FP4_LUT[c]);
        if (dist < best_d) {
          best_d = dist;
          best = c;
        }
      }
      words[j / 8] |= (uint32_t)best << (4 * (j % 8));
    }
    memcpy(wq + i * 2, words, sizeof(words));
    scales[i] = sc;
  }
  return 0;
}

/* nvfp4 dequantize without a global scale, ROPS:5661-5690: LUT[nibble] *
 * from_fp8(scale) in bf16 (exact). */
int oracle_nvfp4_dequantize(const uint32_t* wq, const uint8_t* scales, int64_t rows, int64_t K,
                            uint16_t* out) {
  if (K % 16) return -1;
  for (int64_t r = 0; r < rows; r++) {
    const uint32_t* row = wq + r * (K / 8);
    for (int64_t k = 0; k < K; k++) {
      const float sc = bf(oracle_e4m3_decode(scales[r * (K / 16) + k / 16]));
      out[r * K + k] = oracle_f32_to_bf16(bf(FP4_LUT[code_at(row, 4, k)] * sc));
    }
  }
  return 0;
}

/* ---- quantized matmul: CPUQ:139-257, 550-597 ---------------------------- */

int oracle_qmm_t_affine(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                        const uint16_t* biases, int64_t M, int64_t N, int64_t K,
                        int group_size, int bits, uint16_t* out) {
  if (!pow2_bits(bits) || !valid_gs(group_size) || K % group_size) return -1;
  const int bitmask = (1 << bits) - 1;
  const int pack_factor = 8 / bits; /* codes per byte */
  const int packs_in_group = group_size / pack_factor;
  for (int64_t m = 0; m < M; m++) {
    const uint8_t* w_local = (const uint8_t*)wq;
    const uint16_t* scales_local = scales;
    const uint16_t* biases_local = biases;
    for (int64_t n = 0; n < N; n++) {
      const uint16_t* x_local = x + m * K;
      float sum = 0;
      for (int64_t k = 0; k < K; k += group_size) {
        float scale = oracle_bf16_to_f32(*scales_local++);
        float bias = oracle_bf16_to_f32(*biases_local++);
        for (int kw = 0; kw < packs_in_group; kw++) {
          uint8_t wi = *w_local++;
          for (int p = 0; p < pack_factor; p++) {
            /* T(q) is exact; scale*T(q)+bias in float; x (bf16) * float */
            sum += oracle_bf16_to_f32(*x_local++) * (scale * (float)(wi & bitmask) + bias);
            if (bits != 8) wi >>= bits;
          }
        }
      }
      out[m * N + n] = oracle_f32_to_bf16(sum);
    }
  }
  return 0;
}

int oracle_qmm_affine(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                      const uint16_t* biases, int64_t M, int64_t N, int64_t K,
                      int group_size, int bits, uint16_t* out) {
  if (!pow2_bits(bits) || !valid_gs(group_size) || N % group_size) return -1;
  const int bitmask = (1 << bits) - 1;
  const int pack_factor = 8 / bits;
  const int packs_in_group = group_size / pack_factor;
  float* acc = (float*)malloc(sizeof(float) * (size_t)N);
  if (!acc) return -1;
  for (int64_t m = 0; m < M; m++) {
    const uint8_t* w_local = (const uint8_t*)wq;
    const uint16_t* scales_local = scales;
    const uint16_t* biases_local = biases;
    for (int64_t n = 0; n < N; n++) acc[n] = 0.0f;
    for (int64_t k = 0; k < K; k++) {
      float* result_local = acc;
      float xi = oracle_bf16_to_f32(x[m * K + k]);
      for (int64_t n = 0; n < N; n += group_size) {
        float scale = oracle_bf16_to_f32(*scales_local++);
        float bias = oracle_bf16_to_f32(*biases_local++);
        for (int ng = 0; ng < packs_in_group; ng++) {
          uint8_t wi = *w_local++;
          for (int p = 0; p < pack_factor; p++) {
            (*result_local++) += xi * (scale * (float)(wi & bitmask) + bias);
            if (bits != 8) wi >>= bits;
          }
        }
      }
    }
    for (int64_t n = 0; n < N; n++) out[m * N + n] = oracle_f32_to_bf16(acc[n]);
  }
  free(acc);
  return 0;
}

int oracle_fp_qmm_t_mxfp4(const uint16_t* x, const uint32_t* wq, const uint8_t* scales,
                          int64_t M, int64_t N, int64_t K, uint16_t* out) {
  if (K % 32) return -1;
  float* x_row = (float*)malloc(sizeof(float) * (size_t)K);
  if (!x_row) return -1;
  for (int64_t m = 0; m < M; m++) {
    const uint8_t* w_local = (const uint8_t*)wq;
    const uint8_t* scales_local = scales;
    for (int64_t k = 0; k < K; k++) x_row[k] = oracle_bf16_to_f32(x[m * K + k]);
    for (int64_t n = 0; n < N; n++) {
      const float* x_local = x_row;
      float sum = 0;
      for (int64_t k = 0; k < K; k += 32) {
        float scale = oracle_bf16_to_f32(oracle_e8m0_to_bf16(*scales_local++));
        float gsum = 0;
        for (int kw = 0; kw < 16; kw++) {
          gsum += (*x_local++) * FP4_LUT[w_local[0] & 0xf];
          gsum += (*x_local++) * FP4_LUT[(w_local[0] >> 4) & 0xf];
          w_local++;
        }
        sum += scale * gsum;
      }
      out[m * N + n] = oracle_f32_to_bf16(sum);
    }
  }
  free(x_row);
  return 0;
}

int oracle_gather_qmm_t(const uint16_t* x, const uint32_t* wq, const void* scales,
                        const uint16_t* biases, const uint32_t* lhs,
                        const uint32_t* rhs, int64_t B, int64_t M, int64_t N,
                        int64_t K, int group_size, int bits, int mode, uint16_t* out) {
  const int64_t w_els = N * (K * bits / 32);
  const int64_t g_els = N * (K / group_size);
  for (int64_t i = 0; i < B; i++) {
    int64_t xi = lhs[i], wi = rhs[i];
    int rc;
    if (mode == 0) {
      rc = oracle_qmm_t_affine(x + xi * M * K, wq + wi * w_els,
                               (const uint16_t*)scales + wi * g_els, biases + wi * g_els,
                               M, N, K, group_size, bits, out + i * M * N);
    } else {
      rc = oracle_fp_qmm_t_mxfp4(x + xi * M * K, wq + wi * w_els,
                                 (const uint8_t*)scales + wi * g_els, M, N, K,
                                 out + i * M * N);
    }
    if (rc) return rc;
  }
  return 0;
}

/* ---- affine dequantize to fp32 -------------------------------------------
 * s * q + b in float from the bf16 scale and bias: the weights of the
 * reference's all-f32 ground truth for the fused decode MoE, whose scales and
 * biases are cast to f32 before MLX's dequantize (fused_moe_parity_tests.rs:
 * 241-282, mlx_cxx_kernels.cpp:4003-4011). */
int oracle_affine_dequantize_f32(const uint32_t* wq, const uint16_t* scales, const uint16_t* biases,
                                 int64_t rows, int64_t K, int group_size, int bits, float* out) {
  if (!affine_bits(bits) || group_size <= 0 || K % group_size || (K * bits) % 32) return -1;
  const int64_t wcols = K * bits / 32;
  const int64_t G = K / group_size;
  for (int64_t r = 0; r < rows; r++) {
    const uint32_t* row = wq + r * wcols;
    for (int64_t k = 0; k < K; k++) {
      float s = oracle_bf16_to_f32(scales[r * G + k / group_size]);
      float b = oracle_bf16_to_f32(biases[r * G + k / group_size]);
      out[r * K + k] = s * (float)code_at(row, bits, k) + b;
    }
  }
  return 0;
}

/* ---- fused single-token decode MoE (dense, fp64) --------------------------
 * out[h] = sum_j score[j] * sum_f A(g_j[f]) u_j[f] Wd[e_j][h][f],
 * g_j[f] = sum_i x[i] Wg[e_j][f][i] (u_j with Wu), e_j = min(idx[j], E-1),
 * A = SiLU (act 0) or tanh-approximated GELU (act 1): the math of the
 * reference's fused kernels (mlx_cxx_kernels.cpp:3032-3170) and of its
 * all-f32 ground truth (fused_moe_parity_tests.rs:241-282), carried in fp64
 * over the fp32 dequantized weights.  Result in fp32 (not rounded). */
static double act_fn(int act, double g, double u) {
  if (act == 1) return 0.5 * g * (1.0 + tanh(0.7978845608028654 * (g + 0.044715 * g * g * g))) * u;
  return g / (1.0 + exp(-g)) * u;
}

int oracle_fused_moe(const uint16_t* x, const uint32_t* idx, const float* scores, const uint32_t* gate_w,
                     const uint16_t* gate_s, const uint16_t* gate_b, const uint32_t* up_w,
                     const uint16_t* up_s, const uint16_t* up_b, const uint32_t* down_w,
                     const uint16_t* down_s, const uint16_t* down_b, int64_t din, int64_t dff, int64_t k,
                     int64_t E, int group_size, int gu_bits, int d_bits, int act, float* out) {
  if (!affine_bits(gu_bits) || !affine_bits(d_bits) || din % group_size || dff % group_size) return -1;
  float* wg = malloc(sizeof(float) * dff * din);
  float* wu = malloc(sizeof(float) * dff * din);
  float* wd = malloc(sizeof(float) * din * dff);
  double* a = malloc(sizeof(double) * dff);
  double* y = calloc((size_t)din, sizeof(double));
  int rc = (wg && wu && wd && a && y) ? 0 : -2;
  const int64_t gcols = din * gu_bits / 32, dcols = dff * d_bits / 32;
  for (int64_t j = 0; j < k && rc == 0; j++) {
    const int64_t e = idx[j] < (uint32_t)E ? (int64_t)idx[j] : E - 1;
    oracle_affine_dequantize_f32(gate_w + e * dff * gcols, gate_s + e * dff * (din / group_size),
                                 gate_b + e * dff * (din / group_size), dff, din, group_size, gu_bits, wg);
    oracle_affine_dequantize_f32(up_w + e * dff * gcols, up_s + e * dff * (din / group_size),
                                 up_b + e * dff * (din / group_size), dff, din, group_size, gu_bits, wu);
    oracle_affine_dequantize_f32(down_w + e * din * dcols, down_s + e * din * (dff / group_size),
                                 down_b + e * din * (dff / group_size), din, dff, group_size, d_bits, wd);
    for (int64_t f = 0; f < dff; f++) {
      double g = 0.0, u = 0.0;
      for (int64_t i = 0; i < din; i++) {
        const double xv = oracle_bf16_to_f32(x[i]);
        g += xv * wg[f * din + i];
        u += xv * wu[f * din + i];
      }
      a[f] = act_fn(act, g, u);
    }
    for (int64_t h = 0; h < din; h++) {
      double d = 0.0;
      for (int64_t f = 0; f < dff; f++) d += a[f] * wd[h * dff + f];
      y[h] += (double)scores[j] * d;
    }
  }
  if (rc == 0)
    for (int64_t h = 0; h < din; h++) out[h] = (float)y[h];
  free(wg);
  free(wu);
  free(wd);
  free(a);
  free(y);
  return rc;
}
