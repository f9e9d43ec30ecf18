// qmm.hip — prefill quantized matmul (many activation rows) for gfx950.
//
// Replaces the reference's prefill route: affine dequantize to a bf16
// temporary and a hipBLASLt GEMM (overlays/rocm/mlx/backend/rocm/quantized/
// affine_quantize.hip:127-167 + qmm.hip:1376-1617, 3689-3892).  Here the
// dequantization happens on the way into LDS, so the bf16 weights never
// touch HBM: y = x @ W^T with W = bf16(s*q + b) (affine; the reference GPU
// dequantizer's rounding, affine_quantize.hip:164) or fp4(q) * 2^(e-127)
// (mxfp4, exact), fp32 accumulation, one bf16 rounding on store.
//
// Tiling (MI355X-first):
//  * workgroup = 4 waves (2 x 2) computing a 256 x 128 tile of y; each wave
//    owns 128 x 64 = 8 x 4 tiles of v_mfma_f32_16x16x32_bf16 (128 fp32
//    accumulators per lane);
//  * K advances 64 at a time through double-buffered LDS: activation tile
//    [256][64 + 8] and dequantized weight tile [128][64 + 8] bf16 (the 8-element
//    pad puts the 16 rows a fragment read touches on distinct banks);
//  * the next K-step's global loads are issued before the current step's
//    MFMAs, so HBM/L2 latency hides behind the matrix cores; one barrier per
//    K-step;
//  * when the grid would leave CUs idle (short M), K is split across
//    workgroups and fp32 partials are summed by a second kernel in a fixed
//    order (bitwise reproducible).
#include "common.hpp"
#include "kernels.hpp"

namespace mlxq {

namespace {

constexpr int BK = 64;
constexpr int LDSK = BK + 8;  // padded row length (bf16)
constexpr int NT = 256;       // threads per workgroup (4 waves, 2 x 2)
constexpr uint32_t kDeadQ = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t qrsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

typedef float f32x2 __attribute__((ext_vector_type(2)));

// Two floats -> a bf16 pair, round to nearest even (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}

// Byte j of w as a float (v_cvt_f32_ubyte<j>).
__device__ __forceinline__ float ubyte(uint32_t w, int j) { return (float)((w >> (8 * j)) & 0xFFu); }

}  // namespace

// BM x BN output tile per workgroup; each wave owns (BM/2) x (BN/2).
template <int FMT, int BM, int BN>
__global__ __launch_bounds__(NT) void qmm_kernel(const QmmArgs a) {
  constexpr int TM = BM / 2, TN = BN / 2;  // wave tile
  constexpr int FM = TM / 16, FN = TN / 16;  // 16 x 16 MFMA tiles per wave
  constexpr bool AFF = FMT != MXFP4;
  constexpr int BITS = FMT == AFF8 ? 8 : 4;
  constexpr int WT = BK * BITS / 8 / 16;   // threads per weight row per K-step (16 bytes each)
  constexpr int WROWS = NT / WT;           // weight rows loaded per pass
  constexpr int WPASS = BN / WROWS;        // passes per K-step
  constexpr int VPL = 128 / BITS;          // values per 16-byte load
  constexpr int XPASS = BM * BK * 2 / 16 / NT;  // 16-byte activation loads per thread per K-step

  __shared__ __align__(16) uint16_t xs[2][BM * LDSK];
  __shared__ __align__(16) uint16_t wsm[2][BN * LDSK];

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;  // wave position in the 2 x 2 grid
  static_assert(BN % WROWS == 0, "weight rows per pass must divide BN");
  const int n0 = blockIdx.x * BN;
  const int M = a.M, N = a.N, K = a.K;
  const int nks = a.ksteps_per_split;
  const int ks0 = blockIdx.z * nks;
  const int ks1 = min(ks0 + nks, K / BK);

  // Rows of this tile: rows m0 .. m0+rows-1 of x / y, or (gathers grouped by
  // expert) table entry blockIdx.y: grouped rows r0 .. r0+rows-1 of one
  // expert, read and written through xrows / orows.
  int m0 = blockIdx.y * BM, rows = min(BM, M - m0), r0 = 0;
  int64_t wbase = 0, sbase = 0;
  if (a.seg) {
    if ((int)blockIdx.y >= (int)a.nseg_dev[0]) return;
    const int expert = (int)a.seg[3 * blockIdx.y];
    r0 = (int)a.seg[3 * blockIdx.y + 1];
    rows = (int)a.seg[3 * blockIdx.y + 2];
    m0 = 0;
    wbase = (int64_t)expert * a.w_expert_stride;
    sbase = (int64_t)expert * a.s_expert_stride;
  }

  const __amdgpu_buffer_rsrc_t xr = qrsrc(a.x, (uint32_t)((int64_t)a.x_rows * K * 2));
  const uint32_t RB = (uint32_t)(K * BITS / 8);  // bytes per weight row
  const __amdgpu_buffer_rsrc_t wr = qrsrc(a.w + wbase, (uint32_t)((int64_t)N * RB));
  const int G = K >> a.gs_shift;
  const __amdgpu_buffer_rsrc_t sr =
      qrsrc(reinterpret_cast<const uint8_t*>(a.scales) + sbase * (AFF ? 2 : 1), (uint32_t)((int64_t)N * G * (AFF ? 2 : 1)));
  const __amdgpu_buffer_rsrc_t br =
      qrsrc(AFF ? (const void*)(a.biases + sbase) : a.scales, (uint32_t)(AFF ? (int64_t)N * G * 2 : 0));

  // ---- global -> register staging of one K-step ----------------------------
  // activations: thread t loads row (t / 8) + 32 i, 16-byte chunk t % 8
  const int xrow = t >> 3, xch = t & 7;
  // weights: thread t loads row (t / WT) + WROWS p, 16-byte piece t % WT
  const int wrow = t / WT, wpc = t % WT;
  uint32_t xbase[XPASS];  // byte offset of each staged x row (tile rows past `rows` read 0)
#pragma unroll
  for (int i = 0; i < XPASS; i++) {
    const int tr = xrow + 32 * i;
    const uint32_t xrw = a.seg ? (tr < rows ? a.xrows[r0 + tr] : 0u) : (uint32_t)(m0 + tr);
    xbase[i] = tr < rows ? xrw * (uint32_t)K * 2u + (uint32_t)xch * 16u : kDeadQ;
  }
  u32x4 xreg[XPASS];
  u32x4 wreg[WPASS];
  uint32_t sreg[WPASS], breg[WPASS];
  auto load_step = [&](int ks) {
    const int k0 = ks * BK;
#pragma unroll
    for (int i = 0; i < XPASS; i++)
      xreg[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, xbase[i] + (uint32_t)k0 * 2u, 0, 0));
#pragma unroll
    for (int p = 0; p < WPASS; p++) {
      const int n = n0 + wrow + WROWS * p;
      const bool live = n < N;
      const uint32_t off = live ? (uint32_t)n * RB + (uint32_t)(k0 * BITS / 8 + wpc * 16) : kDeadQ;
      wreg[p] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, off, 0, 2 /* nt */));
      const int g = (k0 + wpc * VPL) >> a.gs_shift;
      const uint32_t so = live ? (uint32_t)(n * G + g) : kDeadQ;
      if constexpr (AFF) {
        sreg[p] = __builtin_amdgcn_raw_buffer_load_b16(sr, so * 2u, 0, 0);
        breg[p] = __builtin_amdgcn_raw_buffer_load_b16(br, so * 2u, 0, 0);
      } else {
        sreg[p] = __builtin_amdgcn_raw_buffer_load_b8(sr, so, 0, 0);
        breg[p] = 0u;
      }
    }
  };

  // ---- register -> LDS (activations as is, weights dequantized) ------------
  auto store_step = [&](int buf) {
#pragma unroll
    for (int i = 0; i < XPASS; i++)
      *reinterpret_cast<u32x4*>(&xs[buf][(xrow + 32 * i) * LDSK + xch * 8]) = xreg[i];
#pragma unroll
    for (int p = 0; p < WPASS; p++) {
      const u32x4 w = wreg[p];
      uint32_t o[VPL / 2];
      if constexpr (AFF) {
        const float sc = bf16_bits_to_f32(sreg[p]);
        const float bi = bf16_bits_to_f32(breg[p]);
        if constexpr (BITS == 4) {
          // nibbles 2j (low half of byte j) and 2j+1 (high half)
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const uint32_t lo = w[e] & 0x0F0F0F0Fu, hi = (w[e] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int j = 0; j < 4; j++)
              o[e * 4 + j] = pack_bf16x2(__builtin_fmaf(sc, ubyte(lo, j), bi), __builtin_fmaf(sc, ubyte(hi, j), bi));
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; e++)
#pragma unroll
            for (int j = 0; j < 4; j += 2)
              o[e * 2 + j / 2] =
                  pack_bf16x2(__builtin_fmaf(sc, ubyte(w[e], j), bi), __builtin_fmaf(sc, ubyte(w[e], j + 1), bi));
        }
      } else {
        // fp4 code points times a power of two are exact in bf16: for normal
        // scales (e8m0 1..254) the gfx950 scaled conversion does it in one
        // instruction per pair; 2^-127 and NaN take the explicit product.
        const float sc = e8m0_to_f32(sreg[p]);
        if (sreg[p] - 1u < 254u) {
#pragma unroll
          for (int e = 0; e < 4; e++) unpack_mxfp4_scaled(w[e], sc, &o[e * 4]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; e++) {
            uint32_t v[4];
            unpack_mxfp4(w[e], v);  // pairs (2h, 2h+1) of the code points
#pragma unroll
            for (int h = 0; h < 4; h++)
              o[e * 4 + h] = pack_bf16x2(bf16_bits_to_f32(v[h] & 0xFFFFu) * sc, bf16_bits_to_f32(v[h] >> 16) * sc);
          }
        }
      }
      uint16_t* dst = &wsm[buf][(wrow + WROWS * p) * LDSK + wpc * VPL];
#pragma unroll
      for (int c = 0; c < VPL / 8; c++)
        *reinterpret_cast<u32x4*>(dst + 8 * c) = u32x4{o[4 * c], o[4 * c + 1], o[4 * c + 2], o[4 * c + 3]};
    }
  };

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int j = 0; j < FN; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int fr = lane & 15;         // fragment row (A) / column (B)
  const int fk = (lane >> 4) * 8;   // fragment k offset within 32

  if (ks0 < ks1) {
    load_step(ks0);
    store_step(0);
    __syncthreads();
    for (int ks = ks0; ks < ks1; ks++) {
      const int buf = (ks - ks0) & 1;
      if (ks + 1 < ks1) load_step(ks + 1);
#pragma unroll
      for (int kk = 0; kk < BK; kk += 32) {
        bf16x8 af[FM], bfr[FN];
#pragma unroll
        for (int i = 0; i < FM; i++)
          af[i] = *reinterpret_cast<const bf16x8*>(&xs[buf][(wm * TM + i * 16 + fr) * LDSK + kk + fk]);
#pragma unroll
        for (int j = 0; j < FN; j++)
          bfr[j] = *reinterpret_cast<const bf16x8*>(&wsm[buf][(wn * TN + j * 16 + fr) * LDSK + kk + fk]);
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
          for (int j = 0; j < FN; j++) acc[i][j] = mfma16x16x32(af[i], bfr[j], acc[i][j]);
      }
      if (ks + 1 < ks1) store_step(buf ^ 1);
      __syncthreads();
    }
  }

  // ---- epilogue: lane holds rows 4 (lane / 16) + q of each 16 x 16 tile ------
  const bool split = a.ksplit > 1;
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int j = 0; j < FN; j++)
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int tr = wm * TM + i * 16 + 4 * (lane >> 4) + q;
        const int c = n0 + wn * TN + j * 16 + fr;
        if (tr < rows && c < N) {
          const int64_t r = a.seg ? (int64_t)a.orows[r0 + tr] : (int64_t)(m0 + tr);
          if (split) a.ws[((int64_t)blockIdx.z * M + r) * N + c] = acc[i][j][q];
          else a.out[r * N + c] = (uint16_t)f32_to_bf16_bits(acc[i][j][q]);
        }
      }
}

// ---- host ------------------------------------------------------------------

// Tile shapes (BM x BN): 0 = 256 x 128, 1 = 256 x 256, 2 = 128 x 128, 3 = 64 x 128.
QmmPlan qmm_plan(int fmt, int gs, int64_t M, int64_t N, int64_t K, int num_cus, int tile_req, int ksplit_req) {
  QmmPlan p;
  const int bits = fmt == AFF8 ? 8 : 4;
  if (K % BK != 0 || K % gs != 0 || M <= 0 || N <= 0) return p;
  if (M * K * 2 >= ((int64_t)1 << 31) || N * K * bits / 8 >= ((int64_t)1 << 31)) return p;
  static const int kBM[4] = {256, 256, 128, 64}, kBN[4] = {128, 256, 128, 128};
  const int nks = (int)(K / BK);
  auto tiles_of = [&](int t) { return ((M + kBM[t] - 1) / kBM[t]) * ((N + kBN[t] - 1) / kBN[t]); };
  int tile = 0;
  if (tile_req >= 0 && tile_req <= 3) {
    tile = tile_req;
  } else {
    // the largest tile that still gives every CU a workgroup without a K split
    tile = tiles_of(1) >= num_cus ? 1 : (tiles_of(0) >= (num_cus * 3) / 4 ? 0 : 2);
  }
  p.tile = tile;
  p.tiles_n = (int)((N + kBN[tile] - 1) / kBN[tile]);
  p.tiles_m = (int)((M + kBM[tile] - 1) / kBM[tile]);
  const int64_t tiles = (int64_t)p.tiles_n * p.tiles_m;
  int ks = 1;
  if (ksplit_req > 0) {
    ks = ksplit_req;
  } else {
    // split K while the grid covers less than the CUs and each split keeps >= 8 K-steps
    while (tiles * ks * 2 <= num_cus && nks / (ks * 2) >= 8) ks *= 2;
  }
  p.ksteps_per_split = (nks + ks - 1) / ks;
  p.ksplit = (nks + p.ksteps_per_split - 1) / p.ksteps_per_split;
  p.ok = true;
  return p;
}

namespace {
template <int FMT>
void qmm_launch_fmt(const QmmArgs& a, const QmmPlan& p, dim3 grid, hipStream_t stream) {
  switch (p.tile) {
    case 1: hipLaunchKernelGGL((qmm_kernel<FMT, 256, 256>), grid, dim3(NT), 0, stream, a); break;
    case 2: hipLaunchKernelGGL((qmm_kernel<FMT, 128, 128>), grid, dim3(NT), 0, stream, a); break;
    case 3: hipLaunchKernelGGL((qmm_kernel<FMT, 64, 128>), grid, dim3(NT), 0, stream, a); break;
    default: hipLaunchKernelGGL((qmm_kernel<FMT, 256, 128>), grid, dim3(NT), 0, stream, a); break;
  }
}
}  // namespace

QmmPlan qmm_plan_grouped(int fmt, int gs, int64_t N, int64_t K, int tile) {
  QmmPlan p;
  const int bits = fmt == AFF8 ? 8 : 4;
  if (K % BK != 0 || K % gs != 0 || N <= 0 || tile < 0 || tile > 3) return p;
  if (N * K * bits / 8 >= ((int64_t)1 << 31)) return p;
  static const int kBM[4] = {256, 256, 128, 64}, kBN[4] = {128, 256, 128, 128};
  p.tile = tile;
  p.rows_per_tile = kBM[tile];
  p.tiles_n = (int)((N + kBN[tile] - 1) / kBN[tile]);
  p.tiles_m = 0;  // the caller sets the segment count
  p.ksplit = 1;
  p.ksteps_per_split = (int)(K / BK);
  p.ok = true;
  return p;
}

hipError_t qmm_launch(int fmt, const QmmArgs& a, const QmmPlan& p, hipStream_t stream) {
  if (!p.ok) return hipErrorInvalidValue;
  const dim3 grid((unsigned)p.tiles_n, (unsigned)p.tiles_m, (unsigned)p.ksplit);
  switch (fmt) {
    case AFF4: qmm_launch_fmt<AFF4>(a, p, grid, stream); break;
    case AFF8: qmm_launch_fmt<AFF8>(a, p, grid, stream); break;
    default: qmm_launch_fmt<MXFP4>(a, p, grid, stream); break;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.ksplit == 1) return e;
  return launch_splitk_reduce(a.ws, a.out, (int64_t)a.M * a.N, p.ksplit, stream);
}

}  // namespace mlxq
