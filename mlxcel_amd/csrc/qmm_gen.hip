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

// out[i] = sum over z < ks of ws[z][i] (in order), rounded to the output type
__global__ __launch_bounds__(256) void gen_reduce_kernel(const float* ws, void* out, int64_t n, int ks, int tc) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float s = 0.f;
  for (int z = 0; z < ks; z++) s += ws[(int64_t)z * n + i];
  if (tc == GEN_F32) static_cast<float*>(out)[i] = s;
  else if (tc == GEN_BF16) static_cast<uint16_t*>(out)[i] = (uint16_t)f32_to_bf16_bits(s);
  else static_cast<uint16_t*>(out)[i] = __builtin_bit_cast(uint16_t, (_Float16)s);
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

hipError_t launch_gen_reduce(const float* ws, void* out, int64_t n, int ks, int tc, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  const int64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(gen_reduce_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, ws, out, n, ks, tc);
  return hipGetLastError();
}

}  // namespace mlxq
