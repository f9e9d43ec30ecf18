// qmm_gen.hip — the general quantized matmul for gfx950: every combination
// the specialised kernels do not take.
//
// Reference semantics: quantized_matmul / gather_qmm (overlays/rocm/mlx/
// ops.cpp:4955-5008, 5841-5948) cast x, scales and biases to the promoted
// type T (affine) or keep x's type (fp modes) and evaluate
//   transpose=true : y[m][n] = sum_k x[m][k] * (s[n][k/gs] * q[n][k] + b[n][k/gs])
//   transpose=false: y[m][n] = sum_k x[m][k] * (s[k][n/gs] * q[k][n] + b[k][n/gs])
// in fp32 and round y to T (CPU: overlays/cpu/mlx/backend/cpu/quantized.cpp:
// 139-197 `_qmm`, 199-257 `_qmm_t`, 550-597 `fp_qmm_t`; codes of 3, 5 and 6
// bits are read as a little-endian bit stream, quantized.cpp:107-137).
//
// Covered here: T in {bfloat16, float16, float32} (x and scales may each be
// any of them; the cast to T is exact), affine codes of 1, 2, 3, 4, 5, 6 and
// 8 bits with groups of 32, 64 or 128, mxfp4, both transposes, any rows per
// matrix, and the segment tables of gather_qmm.
//
// Design.  One workgroup computes a BM x 64 output tile of one segment over
// a K range, 32 K positions per step.  Each step stages the activations
// (converted to T) and the dequantized weights (fp32 s * q + b, rounded to
// T, as the reference's GPU route rounds its dequantized matrix before the
// GEMM) in LDS; four waves each own 16 output columns and run
// v_mfma_f32_16x16x32_{bf16,f16} (T 16-bit) or v_mfma_f32_16x16x4_f32 (T
// float32) over BM / 16 row blocks with fp32 accumulation.  The global
// loads of step i + 1 are issued before the MFMAs of step i.  Small row
// counts split K over workgroups (fp32 partials summed by gen_reduce_kernel
// in a fixed order), so decode shapes still fill the chip.
//
// A 32-position piece of one quantized row (or of one quantized column
// block for transpose=false) lies in a single quantization group (group
// sizes are multiples of 32); its codes occupy `bits` consecutive words, and
// each of the 4 threads that unpack it reads the <= 2 words holding its 8
// codes.
#include <hip/hip_fp16.h>

#include "common.hpp"
#include "kernels.hpp"

namespace mlxq {

namespace {

constexpr int kGenBN = 64;
constexpr int kGenBK = 32;

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ float load_as_f32(const void* p, int64_t i, int dt) {
  if (dt == GEN_F32) return static_cast<const float*>(p)[i];
  const uint16_t h = static_cast<const uint16_t*>(p)[i];
  if (dt == GEN_BF16) return bf16_bits_to_f32(h);
  return (float)__builtin_bit_cast(_Float16, h);
}

// 8 consecutive elements of a row of x (16 or 32 bytes, aligned)
__device__ __forceinline__ void load8_as_f32(const void* p, int64_t i, int dt, float (&v)[8]) {
  if (dt == GEN_F32) {
    const float4* q = reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
    const float4 a = q[0], b = q[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    return;
  }
  const u32x4 u = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(p) + i);
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const uint32_t lo = u[j] & 0xFFFFu, hi = u[j] >> 16;
    if (dt == GEN_BF16) {
      v[2 * j] = bf16_bits_to_f32(lo);
      v[2 * j + 1] = bf16_bits_to_f32(hi);
    } else {
      v[2 * j] = (float)__builtin_bit_cast(_Float16, (uint16_t)lo);
      v[2 * j + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)hi);
    }
  }
}

// fp32 -> element of T (round to nearest even), as raw bits in the low half
// for 16-bit T
template <int TC>
__device__ __forceinline__ uint32_t to_tc_bits(float f) {
  if constexpr (TC == GEN_BF16) return f32_to_bf16_bits(f);
  else if constexpr (TC == GEN_F16) return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
  else return __float_as_uint(f);
}

__device__ __forceinline__ float e2m1_value(uint32_t c) {
  // e2m1: sign, 2-bit exponent, 1-bit mantissa; 0 .5 1 1.5 2 3 4 6
  const float mag = (c & 6u) == 0 ? 0.5f * (float)(c & 1u)
                                  : (1.0f + 0.5f * (float)(c & 1u)) * (float)(1u << (((c >> 1) & 3u) - 1u));
  return (c & 8u) ? -mag : mag;
}

// Staged operands of one K step for one thread: 8 activations and the 8
// codes (with their group's scale and bias) of the thread's weight piece.
struct GenStage {
  float xv[8];
  uint32_t lo, hi;  // code words (hi only when the 8 codes cross a word)
  float s, b;
};

}  // namespace

// TC: compute type of the MFMA (and of the result); BM: rows per tile (16 or
// 64); TRANS: the reference's `transpose`.
template <int TC, int BM, bool TRANS>
__global__ __launch_bounds__(256) void qmm_gen_kernel(const GenArgs a) {
  constexpr int TB = TC == GEN_F32 ? 4 : 2;                     // bytes per staged element
  constexpr int LDK = TC == GEN_F32 ? kGenBK + 1 : kGenBK + 8;  // padded row (elements)
  __shared__ __align__(16) unsigned char lds[(BM + kGenBN) * LDK * TB];
  unsigned char* xs = lds;                     // [BM][LDK]
  unsigned char* wsm = lds + BM * LDK * TB;    // [BN][LDK]

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int seg = blockIdx.z;
  const int mt = blockIdx.y % a.tiles_m, kz = blockIdx.y / a.tiles_m;
  const int n0 = blockIdx.x * kGenBN;
  const int m0 = mt * BM;
  const int N = a.N, K = a.K, M = a.M;
  const int bits = a.bits;
  const uint32_t mask = (1u << bits) - 1u;

  // segment -> x batch and weight matrix (clamped as the reference's
  // indices are, ops.cpp:100)
  const int xb = a.lhs ? (int)min(a.lhs[seg], (uint32_t)(a.X - 1)) : (a.X > 1 ? seg : 0);
  const int eb = a.rhs ? (int)min(a.rhs[seg], (uint32_t)(a.E - 1)) : (a.E > 1 ? seg : 0);
  const uint32_t* W = a.w + (int64_t)eb * a.w_expert_stride;
  const int64_t sofs = (int64_t)eb * a.s_expert_stride;

  const int ksteps = (K + kGenBK - 1) / kGenBK;
  const int kst0 = kz * a.ksteps_per_split;
  const int kst1 = min(ksteps, kst0 + a.ksteps_per_split);

  // this thread's activation piece: row m0 + tid/4, K positions 8*(tid%4)..
  const int xr = tid >> 2, xp = tid & 3;
  const bool x_live = xr < BM && m0 + xr < M;
  const int64_t xrow = ((int64_t)xb * M + m0 + xr) * K;
  // this thread's weight piece: 4 threads per 32-code piece
  const int sp = tid >> 2, part = tid & 3;
  const int sbit = part * 8 * bits;  // first bit of its 8 codes inside the piece
  const int wd = sbit >> 5, wsh = sbit & 31;
  const bool two = wsh + 8 * bits > 32;
  int wn, wk;  // the piece's weight row n (TRANS) / code row k (!TRANS) and offsets
  bool w_live;
  int64_t wrow_words, srow;
  if constexpr (TRANS) {
    wn = n0 + sp;  // row n, K positions k0 + 8*part ..
    wk = 0;
    w_live = wn < N;
    wrow_words = (int64_t)wn * ((int64_t)K * bits / 32);
    srow = sofs + (int64_t)wn * (K >> a.gs_shift);
  } else {
    wk = sp >> 1;  // code row k0 + sp/2, columns n0 + 32*(sp&1) + 8*part ..
    wn = n0 + 32 * (sp & 1);
    w_live = wn < N;
    wrow_words = 0;
    srow = 0;
  }

  auto fetch = [&](int kst, GenStage& st) {
    const int k0 = kst * kGenBK;
    const int kx = k0 + 8 * xp;
    if (x_live && a.x_vec && kx < K) {
      load8_as_f32(a.x, xrow + kx, a.x_dtype, st.xv);  // K % 8 == 0: the 8 lie inside the row
    } else {
#pragma unroll
      for (int j = 0; j < 8; j++) st.xv[j] = (x_live && kx + j < K) ? load_as_f32(a.x, xrow + kx + j, a.x_dtype) : 0.f;
    }
    st.lo = st.hi = 0u;
    st.s = st.b = 0.f;
    int64_t wbase, sidx;
    bool live = w_live;
    if constexpr (TRANS) {
      wbase = wrow_words + (int64_t)k0 * bits / 32;
      sidx = srow + (k0 >> a.gs_shift);
    } else {
      const int k = k0 + wk;
      live = live && k < K;
      wbase = (int64_t)k * ((int64_t)N * bits / 32) + (int64_t)wn * bits / 32;
      sidx = sofs + (int64_t)k * (N >> a.gs_shift) + (wn >> a.gs_shift);
    }
    if (live) {
      st.lo = W[wbase + wd];
      if (two) st.hi = W[wbase + wd + 1];
      if (a.mode == GEN_MXFP4) {
        st.s = e8m0_to_f32(static_cast<const uint8_t*>(a.scales)[sidx]);
      } else {
        st.s = load_as_f32(a.scales, sidx, a.s_dtype);
        st.b = load_as_f32(a.biases, sidx, a.b_dtype);
      }
    }
  };

  auto stage = [&](const GenStage& st) {
    // activations -> xs[xr][8*xp ..]
    if (xr < BM) {
      unsigned char* d = xs + (xr * LDK + 8 * xp) * TB;
      if constexpr (TC == GEN_F32) {
        float* f = reinterpret_cast<float*>(d);
#pragma unroll
        for (int j = 0; j < 8; j++) f[j] = st.xv[j];
      } else {
        u32x4 u;
#pragma unroll
        for (int j = 0; j < 4; j++) u[j] = to_tc_bits<TC>(st.xv[2 * j]) | (to_tc_bits<TC>(st.xv[2 * j + 1]) << 16);
        *reinterpret_cast<u32x4*>(d) = u;
      }
    }
    // 8 codes -> dequantized weights
    const uint64_t v = ((uint64_t)st.hi << 32) | st.lo;
    float w8[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const uint32_t c = (uint32_t)(v >> (wsh + j * bits)) & mask;
      w8[j] = a.mode == GEN_MXFP4 ? e2m1_value(c) * st.s : __builtin_fmaf(st.s, (float)c, st.b);
    }
    if constexpr (TRANS) {
      unsigned char* d = wsm + (sp * LDK + 8 * part) * TB;
      if constexpr (TC == GEN_F32) {
        float* f = reinterpret_cast<float*>(d);
#pragma unroll
        for (int j = 0; j < 8; j++) f[j] = w8[j];
      } else {
        u32x4 u;
#pragma unroll
        for (int j = 0; j < 4; j++) u[j] = to_tc_bits<TC>(w8[2 * j]) | (to_tc_bits<TC>(w8[2 * j + 1]) << 16);
        *reinterpret_cast<u32x4*>(d) = u;
      }
    } else {
      // codes run along N: column (wn - n0) + 8*part + j, K position wk
      const int c0 = wn - n0 + 8 * part;
#pragma unroll
      for (int j = 0; j < 8; j++) {
        unsigned char* d = wsm + ((c0 + j) * LDK + wk) * TB;
        if constexpr (TC == GEN_F32) *reinterpret_cast<float*>(d) = w8[j];
        else *reinterpret_cast<uint16_t*>(d) = (uint16_t)to_tc_bits<TC>(w8[j]);
      }
    }
  };

  f32x4 acc[BM / 16];
#pragma unroll
  for (int b = 0; b < BM / 16; b++) acc[b] = f32x4{0.f, 0.f, 0.f, 0.f};

  GenStage cur;
  if (kst0 < kst1) fetch(kst0, cur);
  for (int kst = kst0; kst < kst1; kst++) {
    stage(cur);
    __syncthreads();
    if (kst + 1 < kst1) fetch(kst + 1, cur);  // in flight during the MFMAs
    const int col = wave * 16 + (lane & 15);
    if constexpr (TC == GEN_F32) {
#pragma unroll
      for (int kk = 0; kk < kGenBK / 4; kk++) {
        const float bw = reinterpret_cast<const float*>(wsm)[col * LDK + 4 * kk + (lane >> 4)];
#pragma unroll
        for (int b = 0; b < BM / 16; b++) {
          const float ax = reinterpret_cast<const float*>(xs)[(b * 16 + (lane & 15)) * LDK + 4 * kk + (lane >> 4)];
          acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(ax, bw, acc[b], 0, 0, 0);
        }
      }
    } else {
      const u32x4 bw = *reinterpret_cast<const u32x4*>(wsm + (col * LDK + 8 * (lane >> 4)) * TB);
#pragma unroll
      for (int b = 0; b < BM / 16; b++) {
        const u32x4 ax = *reinterpret_cast<const u32x4*>(xs + ((b * 16 + (lane & 15)) * LDK + 8 * (lane >> 4)) * TB);
        if constexpr (TC == GEN_BF16)
          acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ax), __builtin_bit_cast(bf16x8, bw),
                                                           acc[b], 0, 0, 0);
        else
          acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, ax), __builtin_bit_cast(f16x8, bw),
                                                          acc[b], 0, 0, 0);
      }
    }
    __syncthreads();
  }

  // D of a 16x16 block: lane holds column lane%16, rows 4*(lane/16) .. +3
  const int n = n0 + wave * 16 + (lane & 15);
  if (n >= N) return;
#pragma unroll
  for (int b = 0; b < BM / 16; b++) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int m = m0 + b * 16 + 4 * (lane >> 4) + r;
      if (m >= M) continue;
      const int64_t o = ((int64_t)seg * M + m) * N + n;
      if (a.ks > 1) {
        a.ws[(int64_t)kz * a.out_elems + o] = acc[b][r];
      } else if constexpr (TC == GEN_F32) {
        static_cast<float*>(a.out)[o] = acc[b][r];
      } else {
        static_cast<uint16_t*>(a.out)[o] = (uint16_t)to_tc_bits<TC>(acc[b][r]);
      }
    }
  }
}

// out[i] = sum over z < ks of ws[z][i] (in order), rounded to the output type;
// the partials are loaded 8 at a time so their latencies overlap, and
// 64-thread workgroups spread small outputs over the CUs
__global__ __launch_bounds__(64) void gen_reduce_kernel(const float* ws, void* out, int64_t n, int ks, int tc) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float s = 0.f;
  int z = 0;
  for (; z + 8 <= ks; z += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; u++) v[u] = ws[(int64_t)(z + u) * n + i];
#pragma unroll
    for (int u = 0; u < 8; u++) s += v[u];
  }
  for (; z < ks; z++) s += ws[(int64_t)z * n + i];
  if (tc == GEN_F32) static_cast<float*>(out)[i] = s;
  else if (tc == GEN_BF16) static_cast<uint16_t*>(out)[i] = (uint16_t)f32_to_bf16_bits(s);
  else static_cast<uint16_t*>(out)[i] = __builtin_bit_cast(uint16_t, (_Float16)s);
}

// ---- decode: 1-2 rows, transpose=true, affine ------------------------------
//
// The general path's decode shapes (codes of 1-8 bits, or float32
// activations) as a row-streaming GEMV instead of the tile kernel: a wave
// owns R weight rows; lane l takes the 32-position pieces l, l + 64, ... of
// every row.  A piece is BITS consecutive words (the reference's
// little-endian bit stream, quantized.cpp:107-137) inside one quantization
// group, so per piece and row
//   y += s * sum_j q_j x_j + b * sum_j x_j
// with the codes widened exactly to fp32 and every product and sum in fp32
// (the reference's qmv formulation, qmv_tiled_kernel.hip:29-128).  The
// activation piece (32 values per row) is converted once and serves the R
// rows.  Lane partials meet in a butterfly over the wave; no LDS, no
// barriers, one launch.
constexpr int kGenQmvRows = 4;  // weight rows per wave
constexpr int kGenQmvWaves = 4;

template <int XT>
__device__ __forceinline__ void load32_as_f32(const void* p, int64_t i, float (&v)[32]) {
#pragma unroll
  for (int q = 0; q < 4; q++) {
    float t[8];
    load8_as_f32(p, i + 8 * q, XT, t);
#pragma unroll
    for (int j = 0; j < 8; j++) v[8 * q + j] = t[j];
  }
}

// load_as_f32 without branches on the element type (two 16-bit loads, the
// second one repeating the first for 16-bit types), so that the loads of
// several rows can be issued together
__device__ __forceinline__ float load_as_f32_flat(const void* p, int64_t i, int dt) {
  const uint16_t* h = static_cast<const uint16_t*>(p);
  const bool wide = dt == GEN_F32;
  const uint32_t lo = h[wide ? 2 * i : i], hi = h[wide ? 2 * i + 1 : i];
  const float f16v = (float)__builtin_bit_cast(_Float16, (uint16_t)lo);
  const float v16 = dt == GEN_BF16 ? __uint_as_float(lo << 16) : f16v;
  return wide ? __uint_as_float(lo | (hi << 16)) : v16;
}

// code j of a piece held in w[0 .. BITS-1]
template <int BITS>
__device__ __forceinline__ uint32_t piece_code(const uint32_t (&w)[BITS], int j) {
  const int o = j * BITS, i = o >> 5, sh = o & 31;
  uint32_t v = w[i] >> sh;
  if (sh + BITS > 32) v |= w[i + 1] << (32 - sh);
  return v & ((1u << BITS) - 1u);
}

template <int BITS, int XT, int MR>
__global__ __launch_bounds__(256) void qmv_gen_kernel(const GenArgs a, int tc) {
  constexpr int R = kGenQmvRows;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int seg = blockIdx.y;
  const int n0 = (blockIdx.x * kGenQmvWaves + wave) * R;
  if (n0 >= a.N) return;  // wave-uniform; the kernel has no barriers
  const int N = a.N, K = a.K, M = a.M;
  const int xb = a.lhs ? (int)min(a.lhs[seg], (uint32_t)(a.X - 1)) : (a.X > 1 ? seg : 0);
  const int eb = a.rhs ? (int)min(a.rhs[seg], (uint32_t)(a.E - 1)) : (a.E > 1 ? seg : 0);
  const uint32_t* W = a.w + (int64_t)eb * a.w_expert_stride;
  const int64_t sofs = (int64_t)eb * a.s_expert_stride;
  const int64_t rw = (int64_t)(K >> 5) * BITS;  // words per weight row
  const int G = K >> a.gs_shift;
  const int nch = K >> 5;

  float acc[MR][R];
#pragma unroll
  for (int m = 0; m < MR; m++)
#pragma unroll
    for (int r = 0; r < R; r++) acc[m][r] = 0.f;

  for (int c = lane; c < nch; c += 64) {
    float xv[MR][32], sx[MR];
#pragma unroll
    for (int m = 0; m < MR; m++) {
      if (m < M) {
        load32_as_f32<XT>(a.x, ((int64_t)xb * M + m) * K + (int64_t)c * 32, xv[m]);
      } else {
#pragma unroll
        for (int j = 0; j < 32; j++) xv[m][j] = 0.f;
      }
      float t = 0.f;
#pragma unroll
      for (int j = 0; j < 32; j++) t += xv[m][j];
      sx[m] = t;
    }
    // all R rows' loads first (rows past N read row N-1 and are not
    // stored), so their latencies overlap
    const int g = (c * 32) >> a.gs_shift;
    uint32_t w[R][BITS];
    float sv[R], bv[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
      const int n = min(n0 + r, N - 1);
      const uint32_t* wp = W + (int64_t)n * rw + (int64_t)c * BITS;
#pragma unroll
      for (int t = 0; t < BITS; t++) w[r][t] = wp[t];
      sv[r] = load_as_f32_flat(a.scales, sofs + (int64_t)n * G + g, a.s_dtype);
      bv[r] = load_as_f32_flat(a.biases, sofs + (int64_t)n * G + g, a.b_dtype);
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
      float qx[MR];
#pragma unroll
      for (int m = 0; m < MR; m++) qx[m] = 0.f;
#pragma unroll
      for (int j = 0; j < 32; j++) {
        const float q = (float)piece_code<BITS>(w[r], j);
#pragma unroll
        for (int m = 0; m < MR; m++) qx[m] = __builtin_fmaf(q, xv[m][j], qx[m]);
      }
#pragma unroll
      for (int m = 0; m < MR; m++) acc[m][r] = __builtin_fmaf(sv[r], qx[m], __builtin_fmaf(bv[r], sx[m], acc[m][r]));
    }
  }

#pragma unroll
  for (int m = 0; m < MR; m++) {
#pragma unroll
    for (int r = 0; r < R; r++) {
      float v = acc[m][r];
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
      const int n = n0 + r;
      if (lane == 0 && m < M && n < N) {
        const int64_t o = ((int64_t)seg * M + m) * N + n;
        if (tc == GEN_F32) static_cast<float*>(a.out)[o] = v;
        else if (tc == GEN_BF16) static_cast<uint16_t*>(a.out)[o] = (uint16_t)f32_to_bf16_bits(v);
        else static_cast<uint16_t*>(a.out)[o] = __builtin_bit_cast(uint16_t, (_Float16)v);
      }
    }
  }
}

// transpose=false decode (W is [K][N], codes packed along N): lane l of a
// workgroup owns the 32-column piece blockIdx.x * 64 + l, i.e. 32 fp32 sums
// per activation row, over the code rows k of the workgroup's K range; the 8
// waves take every 8th row, kGenQmvtRows rows at a time with all their loads
// issued first (rows past the range read the range's last row and count with
// x = 0).  Per row and piece: s * x_k and b * x_k once, then 32 FMAs; the
// bias part is one running sum per piece.  The waves' sums meet in LDS in a
// fixed order; several K ranges leave fp32 partials for gen_reduce_kernel.
constexpr int kGenQmvtWaves = 8;
constexpr int kGenQmvtRows = 4;

template <int BITS, int XT, int MR>
__global__ __launch_bounds__(512) void qmv_gen_t_kernel(const GenArgs a, int tc, int kper) {
  __shared__ float red[kGenQmvtWaves][32][64];
  constexpr int U = kGenQmvtRows;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int seg = blockIdx.z, kz = blockIdx.y;
  const int N = a.N, K = a.K, M = a.M;
  const int npc = N >> 5;
  const int pc = blockIdx.x * 64 + lane;
  const int pcl = min(pc, npc - 1);
  const int xb = a.lhs ? (int)min(a.lhs[seg], (uint32_t)(a.X - 1)) : (a.X > 1 ? seg : 0);
  const int eb = a.rhs ? (int)min(a.rhs[seg], (uint32_t)(a.E - 1)) : (a.E > 1 ? seg : 0);
  const uint32_t* W = a.w + (int64_t)eb * a.w_expert_stride;
  const int64_t sofs = (int64_t)eb * a.s_expert_stride;
  const int64_t rw = (int64_t)npc * BITS;  // words per code row
  const int Gn = N >> a.gs_shift;
  const int g = (pcl * 32) >> a.gs_shift;
  const int k0 = kz * kper, k1 = min(K, k0 + kper);

  float acc[MR][32], bsum[MR];
#pragma unroll
  for (int m = 0; m < MR; m++) {
    bsum[m] = 0.f;
#pragma unroll
    for (int j = 0; j < 32; j++) acc[m][j] = 0.f;
  }
  for (int kb = k0 + wave * U; kb < k1; kb += kGenQmvtWaves * U) {  // wave-uniform
    uint32_t w[U][BITS];
    float sv[U], bv[U], xk[U][MR];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int k = min(kb + u, k1 - 1);
      const uint32_t* wp = W + (int64_t)k * rw + (int64_t)pcl * BITS;
#pragma unroll
      for (int t = 0; t < BITS; t++) w[u][t] = wp[t];
      sv[u] = load_as_f32_flat(a.scales, sofs + (int64_t)k * Gn + g, a.s_dtype);
      bv[u] = load_as_f32_flat(a.biases, sofs + (int64_t)k * Gn + g, a.b_dtype);
#pragma unroll
      for (int m = 0; m < MR; m++) {
        const float xv = load_as_f32(a.x, ((int64_t)xb * M + min(m, M - 1)) * K + k, XT);
        xk[u][m] = kb + u < k1 ? xv : 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
      float xs[MR];
#pragma unroll
      for (int m = 0; m < MR; m++) {
        xs[m] = xk[u][m] * sv[u];
        bsum[m] = __builtin_fmaf(xk[u][m], bv[u], bsum[m]);
      }
#pragma unroll
      for (int j = 0; j < 32; j++) {
        const float q = (float)piece_code<BITS>(w[u], j);
#pragma unroll
        for (int m = 0; m < MR; m++) acc[m][j] = __builtin_fmaf(xs[m], q, acc[m][j]);
      }
    }
  }

  const int64_t n_out = (int64_t)seg * M * N;
#pragma unroll
  for (int m = 0; m < MR; m++) {
    if (m > 0) __syncthreads();  // the previous row's sums have been read
#pragma unroll
    for (int j = 0; j < 32; j++) red[wave][j][lane ^ j] = acc[m][j] + bsum[m];  // lane ^ j: no bank conflicts below
    __syncthreads();
    // 512 threads x 4 of the workgroup's 2048 (piece, column) sums
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int e = threadIdx.x + 512 * i;
      const int l = e >> 5, j = e & 31;  // consecutive threads: one piece's columns
      float t = 0.f;
#pragma unroll
      for (int v = 0; v < kGenQmvtWaves; v++) t += red[v][j][l ^ j];
      const int p = blockIdx.x * 64 + l;
      if (p < npc && m < M) {
        const int64_t o = n_out + (int64_t)m * N + p * 32 + j;
        if (a.ws) a.ws[(int64_t)kz * a.out_elems + o] = t;
        else if (tc == GEN_F32) static_cast<float*>(a.out)[o] = t;
        else if (tc == GEN_BF16) static_cast<uint16_t*>(a.out)[o] = (uint16_t)f32_to_bf16_bits(t);
        else static_cast<uint16_t*>(a.out)[o] = __builtin_bit_cast(uint16_t, (_Float16)t);
      }
    }
  }
}

// ---- host ------------------------------------------------------------------

GenPlan gen_plan(int64_t M, int64_t N, int64_t K, int64_t nseg, int cus, int ks_req) {
  GenPlan p;
  p.bm = M <= 16 ? 16 : 64;
  p.tiles_m = (int)((M + p.bm - 1) / p.bm);
  p.tiles_n = (int)((N + kGenBN - 1) / kGenBN);
  const int ksteps = (int)((K + kGenBK - 1) / kGenBK);
  int ks = 1;
  const int64_t wgs = (int64_t)p.tiles_n * p.tiles_m * nseg;
  if (ks_req > 0) {
    ks = ks_req;
  } else {
    // split K until about two workgroups per CU, keeping >= 4 steps each
    while (wgs * ks < 2LL * cus && ks < 32 && ksteps / (ks * 2) >= 4) ks *= 2;
  }
  ks = std::max(1, std::min(ks, ksteps));
  p.ksteps_per_split = (ksteps + ks - 1) / ks;
  p.ks = (ksteps + p.ksteps_per_split - 1) / p.ksteps_per_split;
  p.ok = (int64_t)p.tiles_m * p.ks <= 65535 && nseg <= 65535 && p.tiles_n <= (1 << 30);
  return p;
}

hipError_t qmm_gen_launch(const GenArgs& a0, const GenPlan& p, int tc, bool transpose, int64_t nseg,
                          hipStream_t stream) {
  if (!p.ok) return hipErrorInvalidValue;
  GenArgs a = a0;
  a.tiles_m = p.tiles_m;
  a.ks = p.ks;
  a.ksteps_per_split = p.ksteps_per_split;
  const dim3 grid((unsigned)p.tiles_n, (unsigned)(p.tiles_m * p.ks), (unsigned)nseg), block(256);
#define GEN_CASE(TC_, BM_, TR_)                                                       \
  if (tc == TC_ && p.bm == BM_ && transpose == TR_) {                                 \
    hipLaunchKernelGGL((qmm_gen_kernel<TC_, BM_, TR_>), grid, block, 0, stream, a);   \
    return hipGetLastError();                                                         \
  }
  GEN_CASE(GEN_BF16, 16, true)
  GEN_CASE(GEN_BF16, 64, true)
  GEN_CASE(GEN_BF16, 16, false)
  GEN_CASE(GEN_BF16, 64, false)
  GEN_CASE(GEN_F16, 16, true)
  GEN_CASE(GEN_F16, 64, true)
  GEN_CASE(GEN_F16, 16, false)
  GEN_CASE(GEN_F16, 64, false)
  GEN_CASE(GEN_F32, 16, true)
  GEN_CASE(GEN_F32, 64, true)
  GEN_CASE(GEN_F32, 16, false)
  GEN_CASE(GEN_F32, 64, false)
#undef GEN_CASE
  return hipErrorInvalidValue;
}

bool qmv_gen_fits(int mode, bool transpose, int64_t M, int64_t N, int64_t K, int64_t nseg, int bits) {
  return mode == GEN_AFFINE && transpose && M >= 1 && M <= 4 && K % 32 == 0 && K > 0 && nseg <= 65535 &&
         (N + kGenQmvRows * kGenQmvWaves - 1) / (kGenQmvRows * kGenQmvWaves) <= 0x7FFFFFFF &&
         ((bits >= 1 && bits <= 6) || bits == 8);
}

hipError_t qmv_gen_launch(const GenArgs& a, int tc, int64_t nseg, hipStream_t stream) {
  if (!qmv_gen_fits(a.mode, true, a.M, a.N, a.K, nseg, a.bits)) return hipErrorInvalidValue;
  const int64_t per_wg = kGenQmvRows * kGenQmvWaves;
  const dim3 grid((unsigned)((a.N + per_wg - 1) / per_wg), (unsigned)nseg), block(64 * kGenQmvWaves);
  const int mr = a.M <= 1 ? 1 : a.M <= 2 ? 2 : 4;  // 3 rows run as 4 (the 4th is zeros, not stored)
#define QG_CASE(B_, X_, MR_)                                                                  \
  if (a.bits == B_ && a.x_dtype == X_ && mr == MR_) {                                         \
    hipLaunchKernelGGL((qmv_gen_kernel<B_, X_, MR_>), grid, block, 0, stream, a, tc);         \
    return hipGetLastError();                                                                 \
  }
#define QG_BITS(X_, MR_) \
  QG_CASE(1, X_, MR_) QG_CASE(2, X_, MR_) QG_CASE(3, X_, MR_) QG_CASE(4, X_, MR_) \
  QG_CASE(5, X_, MR_) QG_CASE(6, X_, MR_) QG_CASE(8, X_, MR_)
  QG_BITS(GEN_BF16, 1)
  QG_BITS(GEN_BF16, 2)
  QG_BITS(GEN_BF16, 4)
  QG_BITS(GEN_F16, 1)
  QG_BITS(GEN_F16, 2)
  QG_BITS(GEN_F16, 4)
  QG_BITS(GEN_F32, 1)
  QG_BITS(GEN_F32, 2)
  QG_BITS(GEN_F32, 4)
#undef QG_BITS
#undef QG_CASE
  return hipErrorInvalidValue;
}

GenTPlan qmv_gen_t_plan(int64_t M, int64_t N, int64_t K, int64_t nseg, int bits, int mode, int cus) {
  GenTPlan p;
  if (mode != GEN_AFFINE || M < 1 || M > 2 || N % 32 != 0 || N <= 0 || K <= 0 || nseg > 65535 ||
      !((bits >= 1 && bits <= 6) || bits == 8))
    return p;
  p.blocks = (int)((N / 32 + 63) / 64);
  // about two workgroups per CU, each K range a whole number of the 8
  // waves' 4-row steps
  const int64_t step = kGenQmvtWaves * kGenQmvtRows;
  int64_t ks = std::max<int64_t>(1, (2LL * cus + p.blocks * nseg - 1) / (p.blocks * nseg));
  int64_t kper = (K + ks - 1) / ks;
  kper = std::max<int64_t>(step, (kper + step - 1) / step * step);
  p.kper = (int)kper;
  p.ks = (int)((K + kper - 1) / kper);
  p.ok = p.ks <= 65535;
  return p;
}

hipError_t qmv_gen_t_launch(const GenArgs& a, const GenTPlan& p, int tc, int64_t nseg, hipStream_t stream) {
  if (!p.ok || (p.ks > 1) != (a.ws != nullptr)) return hipErrorInvalidValue;
  const dim3 grid((unsigned)p.blocks, (unsigned)p.ks, (unsigned)nseg), block(64 * kGenQmvtWaves);
#define QT_CASE(B_, X_, MR_)                                                                       \
  if (a.bits == B_ && a.x_dtype == X_ && (a.M <= 1) == (MR_ == 1)) {                               \
    hipLaunchKernelGGL((qmv_gen_t_kernel<B_, X_, MR_>), grid, block, 0, stream, a, tc, p.kper);    \
    return hipGetLastError();                                                                      \
  }
#define QT_BITS(X_, MR_) \
  QT_CASE(1, X_, MR_) QT_CASE(2, X_, MR_) QT_CASE(3, X_, MR_) QT_CASE(4, X_, MR_) \
  QT_CASE(5, X_, MR_) QT_CASE(6, X_, MR_) QT_CASE(8, X_, MR_)
  QT_BITS(GEN_BF16, 1)
  QT_BITS(GEN_BF16, 2)
  QT_BITS(GEN_F16, 1)
  QT_BITS(GEN_F16, 2)
  QT_BITS(GEN_F32, 1)
  QT_BITS(GEN_F32, 2)
#undef QT_BITS
#undef QT_CASE
  return hipErrorInvalidValue;
}

hipError_t launch_gen_reduce(const float* ws, void* out, int64_t n, int ks, int tc, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  const int64_t blocks = (n + 63) / 64;
  if (blocks > 0x7FFFFFFF) return hipErrorInvalidValue;
  hipLaunchKernelGGL(gen_reduce_kernel, dim3((unsigned)blocks), dim3(64), 0, stream, ws, out, n, ks, tc);
  return hipGetLastError();
}

}  // namespace mlxq
