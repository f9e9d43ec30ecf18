// qmv.hip — skinny quantized matmul (decode: M <= 16 rows per segment) for gfx950.
//
// Replaces the reference's decode route (overlays/rocm/mlx/backend/rocm/quantized/
// qmv_tiled_kernel.hip:29-128 on wave64, qmm.hip:3280-3360 on wave32) and the
// MoE decode gather kernels (qmm.hip:5578-6054, 4741-4915).  Same math as the
// CPU loop it is checked against (overlays/cpu/mlx/backend/cpu/quantized.cpp:
// 199-257 affine, 550-597 mxfp4): y[m,n] = sum_g s[n,g] * sum_{k in g} x[m,k] q[n,k]
// (+ b[n,g] * sum_{k in g} x[m,k]) in fp32, one bf16 rounding on store.
//
// Design (MI355X-first, not a port):
//  * Work unit = 16 output columns x one K range.  One wavefront streams the
//    packed weights of its 16 columns with one 128-bit nontemporal load per
//    lane per K-step (lane = column (i%16) x 16-byte chunk (i/16)), so each
//    load instruction moves 1 KiB of HBM.  Every load of the wave's K range is
//    issued before any arithmetic.
//  * The codes are widened in registers into bf16 MFMA fragments
//    (AFF4: one and-or per pair, "128+q" trick; MXFP4: the gfx950 fp4
//    conversion; AFF8: byte -> f32 -> bf16) and multiplied on
//    v_mfma_f32_16x16x32_bf16 against the activations held in LDS.
//  * Quantization groups never mix inside an MFMA row: A-operand row
//    R = m*S + slot only carries the activations of the lane-chunks that fall
//    in group slot `slot` of the K-step (S = groups per K-step).  After each
//    K-step the fp32 tile is folded with the per-group scale (and the bias
//    times the group's activation sum), so scale/bias cost one FMA per
//    output per group instead of one per weight.
//  * The waves of a workgroup split K and reduce through LDS; larger K is
//    split across workgroups (gridDim.z) and the last workgroup of a column
//    tile to finish sums the fp32 partials in a fixed order, so results are
//    bitwise reproducible run to run.
//  * Segments (gridDim.y) generalise the kernel to batched and gathered
//    (MoE) products: each segment is a run of rows that share one weight
//    matrix (expert).
#include "common.hpp"
#include "kernels.hpp"

namespace mlxq {

template <int FMT>
struct Fmt_traits;
template <>
struct Fmt_traits<AFF4> {
  static constexpr int CK = 32;  // K values per 16-byte chunk
};
template <>
struct Fmt_traits<AFF8> {
  static constexpr int CK = 16;
};
template <>
struct Fmt_traits<MXFP4> {
  static constexpr int CK = 32;
};

__device__ __forceinline__ u32x4 lds_read16(const unsigned char* base, uint32_t off) {
  return *reinterpret_cast<const u32x4*>(base + off);
}

template <int FMT, int GS, int MT, int NW, int TK>
__global__ __launch_bounds__(NW * 64) void qmv_kernel(const QmvArgs a) {
  constexpr int CK = Fmt_traits<FMT>::CK;
  constexpr int KSTEP = 4 * CK;             // K values per K-step (4 lane groups)
  constexpr int NJ = CK / 8;                // MFMAs per K-step
  constexpr int S = (KSTEP + GS - 1) / GS;  // quantization groups per K-step
  constexpr bool AFF = FMT != MXFP4;
  constexpr int BITS = FMT == AFF8 ? 8 : 4;

  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int s_is_last;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nl = lane & 15;
  const int kq = lane >> 4;
  const int tile = blockIdx.x;
  const int sidx = blockIdx.y;
  const int kz = blockIdx.z;

  // ---- segment: rows sharing one weight matrix ----------------------------
  int expert, count, row_begin = 0, xbatch = 0;
  if (a.seg) {
    if (sidx >= *a.nseg) return;
    expert = a.seg[3 * sidx + 0];
    row_begin = a.seg[3 * sidx + 1];
    count = a.seg[3 * sidx + 2];
  } else {
    count = min(a.rps, a.total_rows - sidx * a.rps);
    expert = a.rhs ? (int)min(a.rhs[sidx], (uint32_t)(a.E - 1)) : (a.w_expert_stride ? sidx : 0);
    xbatch = a.lhs ? (int)min(a.lhs[sidx], (uint32_t)(a.X - 1)) : sidx;
  }
  if (count <= 0) return;

  const int N = a.N;
  const int K = a.K;
  const int n0 = tile * 16;
  const int n = min(n0 + nl, N - 1);
  const int Kw = K / (32 / BITS);  // uint32 words per weight row
  const int G = K / GS;            // groups per row
  const int nchunks = K / CK;
  const uint32_t* wrow = a.w + (int64_t)expert * a.w_expert_stride + (int64_t)n * Kw;
  const int64_t srow = (int64_t)expert * a.s_expert_stride + (int64_t)n * G;

  const int nkst = (K + KSTEP - 1) / KSTEP;
  const int kst0 = kz * a.kst_per_wg;
  const int kst1 = min(nkst, kst0 + a.kst_per_wg);
  const int kb = kst0 * KSTEP;
  const int KC = a.kst_per_wg * KSTEP;  // LDS row length (K values)
  const int per = (a.kst_per_wg + NW - 1) / NW;
  const int wk0 = kst0 + wave * per;
  const int nst = max(0, min(kst1, wk0 + per) - wk0);

  // ---- 1. issue every weight / scale / bias load of this wave -------------
  u32x4 wv[TK];
  uint32_t sraw[TK][S];
  uint32_t braw[TK][S];
#pragma unroll
  for (int i = 0; i < TK; i++) {
    if (i < nst) {
      const int t = wk0 + i;
      const int c = t * 4 + kq;
      wv[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow) + (c < nchunks ? c : 0));
      const int gt = (t * KSTEP) / GS;
#pragma unroll
      for (int sl = 0; sl < S; sl++) {
        const int g = min(gt + sl, G - 1);
        if constexpr (AFF) {
          sraw[i][sl] = reinterpret_cast<const uint16_t*>(a.scales)[srow + g];
          braw[i][sl] = a.biases[srow + g];
        } else {
          sraw[i][sl] = reinterpret_cast<const uint8_t*>(a.scales)[srow + g];
        }
      }
    }
  }

  // ---- 2. stage this workgroup's activations (and group sums) in LDS ------
  // Layout: x[m][KC] bf16 (AFF4 fragments pre-permuted), 16 zero bytes,
  // then xsum[m][KC/GS] fp32.
  const int rows_lds = a.rows_lds;
  const uint32_t zpad = (uint32_t)rows_lds * KC * 2;
  float* xsum = reinterpret_cast<float*>(smem + zpad + 16);
  const int GPW = KC / GS;  // groups per workgroup K range
  {
    const int per_row8 = KC / 8;
    const int total8 = rows_lds * per_row8;
    for (int idx = threadIdx.x; idx < total8; idx += NW * 64) {
      const int m = idx / per_row8;
      const int k8 = idx - m * per_row8;
      const int k = kb + k8 * 8;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (m < count && k < K) {
        int64_t xr;
        if (a.seg) {
          xr = a.rowmap[2 * (row_begin + m)];
        } else {
          xr = (int64_t)xbatch * a.rps + m;
        }
        v = *reinterpret_cast<const u32x4*>(a.x + xr * K + k);
      }
      if constexpr (AFF) {
        float s = sum_bf16x8(v);
#pragma unroll
        for (int off = 1; off < GS / 8; off <<= 1) s += __shfl_xor(s, off);
        if ((k8 % (GS / 8)) == 0) xsum[m * GPW + (k8 * 8) / GS] = s;
      }
      if constexpr (FMT == AFF4) v = perm_aff4(v);
      *reinterpret_cast<u32x4*>(smem + ((uint32_t)m * KC + k8 * 8) * 2) = v;
    }
    if (threadIdx.x == 0) *reinterpret_cast<u32x4*>(smem + zpad) = u32x4{0u, 0u, 0u, 0u};
  }
  __syncthreads();

  // ---- 3. MFMA over the K-steps, fold per group ----------------------------
  const int slot_kq = (kq * CK) / GS < S ? (kq * CK) / GS : 0;
  uint32_t xoff[MT];
  bool aact[MT];
#pragma unroll
  for (int mt = 0; mt < MT; mt++) {
    const int R = 16 * mt + nl;
    const int mA = R / S;
    aact[mt] = (mA < count) && ((R % S) == slot_kq);
    xoff[mt] = ((uint32_t)mA * KC + kq * CK) * 2;
  }
  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; mt++) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int i = 0; i < TK; i++) {
    if (i < nst) {
      const int t = wk0 + i;
      const bool cvalid = (t * 4 + kq) < nchunks;
      const uint32_t kloc2 = (uint32_t)(t - kst0) * KSTEP * 2;
      f32x4 d[MT];
#pragma unroll
      for (int j = 0; j < NJ; j++) {
        uint32_t bv[4];
        if constexpr (FMT == AFF4) unpack_aff4(wv[i][j], bv);
        if constexpr (FMT == MXFP4) unpack_mxfp4(wv[i][j], bv);
        if constexpr (FMT == AFF8) unpack_aff8(wv[i][2 * j], wv[i][2 * j + 1], bv);
        const bf16x8 b = as_bf16x8(bv);
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
          const uint32_t off = (aact[mt] && cvalid) ? xoff[mt] + kloc2 + 16u * j : zpad;
          const bf16x8 av = __builtin_bit_cast(bf16x8, lds_read16(smem, off));
          d[mt] = mfma16x16x32(av, b, j == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : d[mt]);
        }
      }
      // fold: acc += s * D (+ b' * xsum)
      const int gl0 = (t - kst0) * KSTEP / GS;
#pragma unroll
      for (int mt = 0; mt < MT; mt++) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const int sl = q % S;
          float sc;
          if constexpr (AFF) {
            sc = bf16_bits_to_f32(sraw[i][sl]);
          } else {
            sc = e8m0_to_f32(sraw[i][sl]);
          }
          float v = acc[mt][q];
          if constexpr (AFF) {
            const float bi = bf16_bits_to_f32(braw[i][sl]);
            const float bp = (FMT == AFF4) ? __builtin_fmaf(-128.0f, sc, bi) : bi;
            const int mD = min((16 * mt + 4 * kq + q) / S, rows_lds - 1);
            v = __builtin_fmaf(bp, xsum[mD * GPW + gl0 + sl], v);
          }
          acc[mt][q] = __builtin_fmaf(sc, d[mt][q], v);
        }
      }
    }
  }

  // ---- 4. reduce the waves of this workgroup through LDS -------------------
  __syncthreads();  // every wave is done reading the activations
  float* red = reinterpret_cast<float*>(smem);
#pragma unroll
  for (int mt = 0; mt < MT; mt++)
#pragma unroll
    for (int q = 0; q < 4; q++) red[((wave * MT + mt) * 4 + q) * 64 + lane] = acc[mt][q];
  __syncthreads();

  const bool split = a.ks > 1;
  if (wave == 0) {
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
      float tot[4];
#pragma unroll
      for (int q = 0; q < 4; q++) {
        float s = 0.f;
        for (int w = 0; w < NW; w++) s += red[((w * MT + mt) * 4 + q) * 64 + lane];
        tot[q] = s;
      }
      // rows 16mt+4kq+q hold (m = R / S, slot = R % S): sum the S slots of each m
#pragma unroll
      for (int u = 0; u < 4 / S; u++) {
        float y = 0.f;
#pragma unroll
        for (int sl = 0; sl < S; sl++) y += tot[u * S + sl];
        const int m = (16 * mt + 4 * kq) / S + u;
        if (m < count && n0 + nl < N) {
          const int64_t orow = a.seg ? (int64_t)a.rowmap[2 * (row_begin + m) + 1]
                                     : (int64_t)sidx * a.rps + m;
          if (split) {
            a.ws[((int64_t)kz * a.out_rows + orow) * N + n0 + nl] = y;
          } else {
            a.out[orow * N + n0 + nl] = (uint16_t)f32_to_bf16_bits(y);
          }
        }
      }
    }
  }
  if (!split) return;

  // ---- 5. split-K: the last workgroup of this tile sums the partials --------
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned prev = atomicAdd(&a.counters[sidx * gridDim.x + tile], 1u);
    s_is_last = (prev == (unsigned)(a.ks - 1));
  }
  __syncthreads();
  if (!s_is_last) return;
  __threadfence();
  if (wave == 0) {
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
#pragma unroll
      for (int u = 0; u < 4 / S; u++) {
        const int m = (16 * mt + 4 * kq) / S + u;
        if (m < count && n0 + nl < N) {
          const int64_t orow = a.seg ? (int64_t)a.rowmap[2 * (row_begin + m) + 1]
                                     : (int64_t)sidx * a.rps + m;
          float y = 0.f;
          for (int z = 0; z < a.ks; z++) y += a.ws[((int64_t)z * a.out_rows + orow) * N + n0 + nl];
          a.out[orow * N + n0 + nl] = (uint16_t)f32_to_bf16_bits(y);
        }
      }
    }
  }
  if (threadIdx.x == 0) a.counters[sidx * gridDim.x + tile] = 0u;
}

// ---- gather index preparation ----------------------------------------------

__device__ __forceinline__ int64_t load_index(const void* p, int dtype, int64_t loc) {
  switch (dtype) {
    case MLXQ_BOOL:
    case MLXQ_UINT8: return reinterpret_cast<const uint8_t*>(p)[loc];
    case MLXQ_UINT16: return reinterpret_cast<const uint16_t*>(p)[loc];
    case MLXQ_UINT32: return reinterpret_cast<const uint32_t*>(p)[loc];
    case MLXQ_UINT64: return (int64_t)reinterpret_cast<const uint64_t*>(p)[loc];
    case MLXQ_INT8: return reinterpret_cast<const int8_t*>(p)[loc];
    case MLXQ_INT16: return reinterpret_cast<const int16_t*>(p)[loc];
    case MLXQ_INT32: return reinterpret_cast<const int32_t*>(p)[loc];
    default: return reinterpret_cast<const int64_t*>(p)[loc];
  }
}

__global__ __launch_bounds__(256) void index_prep_kernel(const IdxPrepArgs a) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= a.B) return;
#pragma unroll
  for (int s = 0; s < 2; s++) {
    int64_t rem = i, loc = 0;
    for (int d = a.bnd - 1; d >= 0; d--) {
      const int64_t c = rem % a.bshape[d];
      rem /= a.bshape[d];
      loc += c * a.bstrides[s][d];
    }
    int64_t v = a.data[s] ? (int64_t)(uint32_t)load_index(a.data[s], a.dtype[s], loc) : loc;
    if (v >= a.clamp[s]) v = a.clamp[s] - 1;
    a.out[s][i] = (uint32_t)v;
  }
}

hipError_t launch_index_prep(const IdxPrepArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL(index_prep_kernel, dim3((unsigned)((a.B + 255) / 256)), dim3(256), 0, stream, a);
  return hipGetLastError();
}

// ---- host launch -----------------------------------------------------------

namespace {
constexpr int kNW = 4;
constexpr int kTK = 8;

template <int FMT, int GS, int MT>
hipError_t launch_t(const QmvArgs& a, dim3 grid, size_t lds, hipStream_t stream) {
  hipLaunchKernelGGL((qmv_kernel<FMT, GS, MT, kNW, kTK>), grid, dim3(kNW * 64), lds, stream, a);
  return hipGetLastError();
}

template <int FMT, int GS>
hipError_t launch_mt(int mt, const QmvArgs& a, dim3 grid, size_t lds, hipStream_t stream) {
  switch (mt) {
    case 1: return launch_t<FMT, GS, 1>(a, grid, lds, stream);
    case 2: return launch_t<FMT, GS, 2>(a, grid, lds, stream);
    default: return launch_t<FMT, GS, 4>(a, grid, lds, stream);
  }
}
}  // namespace

int qmv_ck(int fmt) { return fmt == AFF8 ? 16 : 32; }

int qmv_slots(int fmt, int gs) {
  const int kstep = 4 * qmv_ck(fmt);
  return (kstep + gs - 1) / gs;
}

int qmv_tile_mt(int fmt, int gs, int rows) {
  const int s = qmv_slots(fmt, gs);
  const int need = (rows * s + 15) / 16;
  return need <= 1 ? 1 : (need <= 2 ? 2 : 4);
}

int qmv_max_rows(int fmt, int gs) { return 16 * 4 / qmv_slots(fmt, gs); }

QmvPlan qmv_plan(int fmt, int gs, int64_t N, int64_t K, int rows_lds, int nseg, int num_cus) {
  QmvPlan p;
  const int kstep = 4 * qmv_ck(fmt);
  const int nkst = (int)((K + kstep - 1) / kstep);
  const int tiles = (int)((N + 15) / 16);
  // K-steps per workgroup: at most kNW * kTK (every wave holds <= kTK loads in
  // registers), rounded so that the workgroup K range is a multiple of 128.
  const int step_align = 128 / kstep;  // K-steps per 128 K values
  int max_kst = kNW * kTK;
  // Split K across workgroups until there are enough workgroups to cover the
  // chip twice or the per-workgroup range gets short.
  int ks = (nkst + max_kst - 1) / max_kst;
  while ((int64_t)tiles * nseg * ks < 2LL * num_cus && (nkst + ks) / (ks + 1) >= 4 * step_align * 2) ks++;
  int kst_per = (nkst + ks - 1) / ks;
  kst_per = ((kst_per + step_align - 1) / step_align) * step_align;
  ks = (nkst + kst_per - 1) / kst_per;
  // Dynamic LDS: activations rows x KC bf16, a 16-byte zero pad, group sums
  // rows x KC/gs fp32; the same bytes later hold the cross-wave reduction.
  auto lds_bytes = [&](int kp) {
    const int KC = kp * kstep;
    const size_t x = (size_t)rows_lds * KC * 2 + 16 + (size_t)rows_lds * (KC / gs) * 4;
    const size_t red = (size_t)kNW * 4 * 4 * 64 * 4;  // NW x MT(<=4) x 4 x 64 floats
    return x > red ? x : red;
  };
  while (lds_bytes(kst_per) > 64 * 1024 && kst_per > step_align) {
    kst_per = ((kst_per / 2 + step_align - 1) / step_align) * step_align;
    ks = (nkst + kst_per - 1) / kst_per;
  }
  p.ks = ks;
  p.kst_per_wg = kst_per;
  p.tiles = tiles;
  p.lds = lds_bytes(kst_per);
  return p;
}

hipError_t qmv_launch(int fmt, int gs, int mt, const QmvArgs& a, int nseg_slots, const QmvPlan& p,
                      hipStream_t stream) {
  dim3 grid((unsigned)p.tiles, (unsigned)nseg_slots, (unsigned)p.ks);
  switch (fmt) {
    case AFF4:
      if (gs == 32) return launch_mt<AFF4, 32>(mt, a, grid, p.lds, stream);
      if (gs == 64) return launch_mt<AFF4, 64>(mt, a, grid, p.lds, stream);
      return launch_mt<AFF4, 128>(mt, a, grid, p.lds, stream);
    case AFF8:
      if (gs == 32) return launch_mt<AFF8, 32>(mt, a, grid, p.lds, stream);
      if (gs == 64) return launch_mt<AFF8, 64>(mt, a, grid, p.lds, stream);
      return launch_mt<AFF8, 128>(mt, a, grid, p.lds, stream);
    default:
      return launch_mt<MXFP4, 32>(mt, a, grid, p.lds, stream);
  }
}

}  // namespace mlxq
