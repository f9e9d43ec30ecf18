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
//    (AFF4: one byte permute per pair, "128+q" trick; MXFP4: the gfx950 fp4
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
//    (MoE) products: segment s is the x.shape[-2] rows of batch lhs[s]
//    multiplied by weight matrix rhs[s] (expert).
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

// LDS layout.  The workgroup shares
//   [sb]  16 x (GW + 1) x {scale, bias - 128*scale | bias} fp32 (affine) or
//         16 x (GW + 1) scale fp32 (mxfp4): the scales of the 16 rows over the
//         workgroup's K range, staged with coalesced loads (one row per
//         instruction) instead of one scattered load per lane and K-step;
// and every wave owns a region holding what its K-steps
// t = kst0 + wave + NW * i (i < TK) need:
//   [x]   rows_lds x TK x KSTEP bf16 activations (AFF4 fragments pre-permuted
//         to [x0,x4,x1,x5,x2,x6,x3,x7]); K outside the matrix is zero
//   [xs]  TK x (KSTEP / XG) x CAP fp32 activation sums ([i][sum][row]; for
//         S == 4 [i][row][sum]), CAP = 16 * MT / S; absent rows are zero
//   [zero] 64 zero bytes: the A operand of lanes with no activation row.
// After the K loop the bytes are reused for the cross-wave reduction.
struct QmvLds {
  uint32_t sb, w0, x, xs, zpad, wreg, total;  // x/xs/zpad relative to a wave region
};

__host__ __device__ inline QmvLds qmv_lds_layout(int fmt, int gs, int rows_lds, int tk, int nw, int mt, int gw) {
  const int ck = fmt == AFF8 ? 16 : 32;
  const int kstep = 4 * ck;
  const int xg = gs < kstep ? gs : kstep;
  const int s = (kstep + gs - 1) / gs;
  const int cap = 16 * mt / s;
  QmvLds l;
  l.sb = 0;
  l.w0 = ((uint32_t)16 * (gw + 1) * (fmt != MXFP4 ? 8 : 4) + 15u) & ~15u;  // row pitch gw + 1: no bank conflicts
  l.x = 0;
  l.xs = (uint32_t)rows_lds * tk * kstep * 2;
  l.zpad = (l.xs + (fmt != MXFP4 ? (uint32_t)tk * (kstep / xg) * cap * 4 : 0) + 15u) & ~15u;
  l.wreg = l.zpad + 64;
  l.total = l.w0 + (uint32_t)nw * l.wreg;
  const uint32_t red = (uint32_t)nw * mt * 4 * 64 * 4;
  if (l.total < red) l.total = red;
  return l;
}

template <int FMT, int GS, int MT, int NW, int TK>
__global__ __launch_bounds__(NW * 64) void qmv_kernel(const QmvArgs a) {
  constexpr int CK = Fmt_traits<FMT>::CK;
  constexpr int KSTEP = 4 * CK;                // K values per K-step (4 lane groups)
  constexpr int NJ = CK / 8;                   // MFMAs per K-step
  constexpr int S = (KSTEP + GS - 1) / GS;     // quantization groups per K-step
  constexpr int XG = GS < KSTEP ? GS : KSTEP;  // K values per activation sum
  constexpr int XSK = KSTEP / XG;              // activation sums per K-step
  constexpr int CAP = 16 * MT / S;             // activation rows per segment
  constexpr bool AFF = FMT != MXFP4;
  constexpr int BITS = FMT == AFF8 ? 8 : 4;
  constexpr int PPK = KSTEP / 8;               // 16-byte activation pieces per K-step
  constexpr int KPL = 64 / PPK;                // K-steps covered by one wave-wide load
  constexpr int XL = (TK + KPL - 1) / KPL;     // activation loads per row per lane
  constexpr int XEARLY = 4;                    // activation loads issued before the weights

  extern __shared__ __align__(16) unsigned char smem[];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nl = lane & 15;
  const int kq = lane >> 4;
  const int tile = blockIdx.x;
  const int sidx = blockIdx.y;

  // ---- segment (wave-uniform) ---------------------------------------------
  // Either segment sidx of `rps` consecutive rows (batch lhs[sidx], expert
  // rhs[sidx]), or, for gathers grouped by expert, table entry sidx: rows
  // r0 .. r0+count-1 of the grouped order, read and written through
  // xrows / orows.
  int count, expert, r0 = 0, xbatch = 0;
  if (a.seg) {
    if (sidx >= (int)a.nseg_dev[0]) return;
    expert = (int)a.seg[3 * sidx];
    r0 = (int)a.seg[3 * sidx + 1];
    count = (int)a.seg[3 * sidx + 2];
  } else {
    count = min(a.rps, a.total_rows - sidx * a.rps);
    if (count <= 0) return;
    expert = seg_index(a.rhs, a.rhs_stride, sidx, a.E, a.w_expert_stride ? sidx : 0);
    xbatch = seg_index(a.lhs, a.lhs_stride, sidx, a.X, a.lhs_div > 1 ? sidx / a.lhs_div : sidx);
  }

  const int N = a.N;
  const int K = a.K;
  const int n0 = tile * 16;
  const int nchunks = K / CK;
  const int G = K / GS;
  const int kst0 = blockIdx.z * a.kst_per_wg;
  const int nkst = (K + KSTEP - 1) / KSTEP;
  const int kst1 = min(nkst, kst0 + a.kst_per_wg);
  const int t0 = kst0 + wave;  // this wave's K-steps: t0 + NW * i
  const int nst = min(TK, max(0, (kst1 - t0 + NW - 1) / NW));
  const int rows_lds = a.rows_lds;
  const int KC = a.kst_per_wg * KSTEP;  // the workgroup's K range
  const int GW = KC / GS;                // groups of that range per row (>= 1)
  const int GWP = GW + 1;                // LDS row pitch of the scales
  const int g0 = (kst0 * KSTEP) / GS;
  const QmvLds L = qmv_lds_layout(FMT, GS, rows_lds, TK, NW, MT, GW);
  unsigned char* wr = smem + L.w0 + wave * L.wreg;  // this wave's region

  // ---- 1. loads: activations and scales of this wave, then its weights ----
  // vmcnt retires in order, so the small staged loads can be consumed while
  // the weight loads (issued last) are still in flight.
  const uint16_t* xrow0 = a.x + ((int64_t)xbatch * a.rps) * K;
  auto x_item = [&](int e, int& m, int& i, int& piece) {  // e-th activation load of this lane
    m = e / XL;
    i = lane / PPK + KPL * (e - m * XL);
    piece = lane % PPK;
  };
  auto x_load = [&](int e) -> u32x4 {
    int m, i, piece;
    x_item(e, m, i, piece);
    const int t = t0 + NW * i;
    const int k = t * KSTEP + piece * 8;
    const bool live = m < count && i < nst && k < K;
    const uint16_t* xr = a.seg ? a.x + (int64_t)a.xrows[r0 + min(m, count - 1)] * K : xrow0 + (int64_t)m * K;
    return live ? *reinterpret_cast<const u32x4*>(xr + k) : u32x4{0u, 0u, 0u, 0u};
  };
  const int nx = rows_lds * XL;
  u32x4 xv[XEARLY];
#pragma unroll
  for (int e = 0; e < XEARLY; e++)
    if (e < nx) xv[e] = x_load(e);

  // Scales: wave w stages rows w, w + NW, ...; lane j of a load takes group
  // g0 + j + 64 v, so one instruction reads one row's groups contiguously.
  constexpr int RPW = 16 / NW;  // rows per wave
  const int64_t sbase = (int64_t)expert * a.s_expert_stride;
  const int nsv = (GW + 63) / 64;  // loads per row
  auto sb_idx = [&](int u, int v, int& r, int& j) -> int64_t {
    r = wave + NW * u;
    j = lane + 64 * v;
    return sbase + (int64_t)min(n0 + r, N - 1) * G + min(g0 + j, G - 1);
  };
  constexpr int SBE = 8;  // loads per lane issued before the weights; e -> (u, v) = (e % RPW, e / RPW)
  uint32_t s_raw[SBE], b_raw[SBE];
#pragma unroll
  for (int e = 0; e < SBE; e++) {
    s_raw[e] = b_raw[e] = 0u;
    if (e < RPW * nsv) {
      int r, j;
      const int64_t o = sb_idx(e % RPW, e / RPW, r, j);
      if constexpr (AFF) {
        s_raw[e] = reinterpret_cast<const uint16_t*>(a.scales)[o];
        b_raw[e] = a.biases[o];
      } else {
        s_raw[e] = reinterpret_cast<const uint8_t*>(a.scales)[o];
      }
    }
  }

  // Weight loads: unconditional (clamped indices; a clamped chunk meets zero
  // activations) so they go out back to back.
  const u32x4* wrow = reinterpret_cast<const u32x4*>(a.w + (int64_t)expert * a.w_expert_stride +
                                                     (int64_t)min(n0 + nl, N - 1) * (K / (32 / BITS)));
  u32x4 wv[TK];
#pragma unroll
  for (int i = 0; i < TK; i++) {
    const int c = min((t0 + NW * min(i, max(nst - 1, 0))) * 4 + kq, nchunks - 1);
    wv[i] = __builtin_nontemporal_load(wrow + c);
  }
  __builtin_amdgcn_sched_barrier(0);  // keep uses of staged data below the weight loads

  // ---- 2. stage this wave's operands in its LDS region ---------------------
  float* xsw = reinterpret_cast<float*>(wr + L.xs);
  auto x_put = [&](int e, u32x4 v) {
    int m, i, piece;
    x_item(e, m, i, piece);
    if constexpr (AFF) {
      float s = sum_bf16x8(v);
#pragma unroll
      for (int off = 1; off < XG / 8; off <<= 1) s += __shfl_xor(s, off);
      if (i < TK && (piece % (XG / 8)) == 0) {
        const int sl = piece / (XG / 8);
        xsw[S == 4 ? (i * CAP + m) * XSK + sl : (i * XSK + sl) * CAP + m] = s;
      }
    }
    if (i < TK) {
      if constexpr (FMT == AFF4) v = perm_aff4(v);
      *reinterpret_cast<u32x4*>(wr + L.x + (uint32_t)((m * TK + i) * KSTEP + piece * 8) * 2) = v;
    }
  };
#pragma unroll
  for (int e = 0; e < XEARLY; e++)
    if (e < nx) x_put(e, xv[e]);
  for (int e = XEARLY; e < nx; e++) x_put(e, x_load(e));
  if constexpr (AFF) {  // sums of rows this segment does not have
    for (int e = lane; e < TK * XSK * (CAP - rows_lds); e += 64) {
      const int m = rows_lds + e % (CAP - rows_lds);
      const int r = e / (CAP - rows_lds);  // (i, sl) pair
      const int i = r / XSK, sl = r % XSK;
      xsw[S == 4 ? (i * CAP + m) * XSK + sl : (i * XSK + sl) * CAP + m] = 0.f;
    }
  }
  auto sb_put = [&](int r, int j, uint32_t sr, uint32_t br) {
    if (j >= GW) return;
    if constexpr (AFF) {
      const float sc = bf16_bits_to_f32(sr);
      const float bi = bf16_bits_to_f32(br);
      reinterpret_cast<float2*>(smem + L.sb)[r * GWP + j] =
          float2{sc, (FMT == AFF4) ? __builtin_fmaf(-128.0f, sc, bi) : bi};
    } else {
      reinterpret_cast<float*>(smem + L.sb)[r * GWP + j] = e8m0_to_f32(sr);
    }
  };
#pragma unroll
  for (int e = 0; e < SBE; e++) {
    if (e < RPW * nsv) {
      int r, j;
      sb_idx(e % RPW, e / RPW, r, j);
      sb_put(r, j, s_raw[e], b_raw[e]);
    }
  }
  for (int e = SBE; e < RPW * nsv; e++) {  // wide K ranges: the rest
    int r, j;
    const int64_t o = sb_idx(e % RPW, e / RPW, r, j);
    if constexpr (AFF) {
      sb_put(r, j, reinterpret_cast<const uint16_t*>(a.scales)[o], a.biases[o]);
    } else {
      sb_put(r, j, reinterpret_cast<const uint8_t*>(a.scales)[o], 0u);
    }
  }
  if (lane < 4) reinterpret_cast<u32x4*>(wr + L.zpad)[lane] = u32x4{0u, 0u, 0u, 0u};
  __syncthreads();  // the shared scales (and every wave's own region)

  // ---- 3. MFMA over this wave's K-steps, fold per group --------------------
  const int slot_kq = (kq * CK) / GS < S ? (kq * CK) / GS : 0;
  uint32_t abase[MT];
  bool aact[MT];
#pragma unroll
  for (int mt = 0; mt < MT; mt++) {
    const int R = 16 * mt + nl;
    aact[mt] = R / S < count && (R % S) == slot_kq;
    abase[mt] = (uint32_t)(wr - smem) + L.x + (uint32_t)((R / S) * TK * KSTEP + kq * CK) * 2;
  }
  // scales of K-step i: group (wave + NW i) * S + sl of row nl (GS <= KSTEP),
  // or (wave + NW i) / 2 when a group spans two K-steps (NW is even)
  const uint32_t sbb = L.sb + (uint32_t)(nl * GWP + (GS <= KSTEP ? wave * S : wave / 2)) * (AFF ? 8 : 4);
  constexpr uint32_t SB_STEP = (uint32_t)(GS <= KSTEP ? NW * S : NW / 2) * (AFF ? 8 : 4);
  const uint32_t zp = (uint32_t)(wr - smem) + L.zpad;
  uint32_t xsb[MT];
#pragma unroll
  for (int mt = 0; mt < MT; mt++) {
    const int m0 = (16 * mt + 4 * kq) / S;
    xsb[mt] = (uint32_t)(wr - smem) + L.xs + (uint32_t)(S == 4 ? m0 * XSK : m0) * 4;
  }

  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; mt++) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int i = 0; i < TK; i++) {
    if (i < nst) {  // wave-uniform
      const u32x4 w = wv[i];
      uint32_t ab[MT];
#pragma unroll
      for (int mt = 0; mt < MT; mt++) ab[mt] = aact[mt] ? abase[mt] + (uint32_t)(i * KSTEP) * 2 : zp;
      f32x4 d[MT];
#pragma unroll
      for (int jj = 0; jj < NJ; jj++) {
        uint32_t bv[4];
        if constexpr (FMT == AFF4) unpack_aff4(w[jj], bv);
        if constexpr (FMT == MXFP4) unpack_mxfp4(w[jj], bv);
        if constexpr (FMT == AFF8) unpack_aff8(w[2 * jj], w[2 * jj + 1], bv);
        const bf16x8 b = as_bf16x8(bv);
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
          const bf16x8 av = __builtin_bit_cast(bf16x8, lds_read16(smem, ab[mt] + 16u * jj));
          d[mt] = mfma16x16x32(av, b, jj == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : d[mt]);
        }
      }
      // fold: acc += s * D (+ b' * sum(x)) per output row
      float sc[S], bp[S];
#pragma unroll
      for (int sl = 0; sl < S; sl++) {
        if constexpr (AFF) {
          const float2 v2 = *reinterpret_cast<const float2*>(smem + sbb + i * SB_STEP + sl * 8);
          sc[sl] = v2.x;
          bp[sl] = v2.y;
        } else {
          sc[sl] = *reinterpret_cast<const float*>(smem + sbb + i * SB_STEP + sl * 4);
          bp[sl] = 0.f;
        }
      }
#pragma unroll
      for (int mt = 0; mt < MT; mt++) {
        float xs[4];
        if constexpr (AFF) {
#pragma unroll
          for (int q = 0; q < 4; q++) {
            // D row (16mt + 4kq + q) is activation row m0 + q / S, sum slot q % S
            const int dm = q / S, sl = q % S;
            const uint32_t off = S == 4 ? (uint32_t)((i * CAP) * XSK + sl) * 4
                                        : (uint32_t)((i * XSK + sl) * CAP + dm) * 4;
            xs[q] = *reinterpret_cast<const float*>(smem + xsb[mt] + off);
          }
        }
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const int sl = q % S;
          float v = acc[mt][q];
          if constexpr (AFF) v = __builtin_fmaf(bp[sl], xs[q], v);
          acc[mt][q] = __builtin_fmaf(sc[sl], d[mt][q], v);
        }
      }
    }
  }

  // ---- 4. reduce the waves of this workgroup through LDS -------------------
  __syncthreads();  // every wave is done reading LDS
  float* red = reinterpret_cast<float*>(smem);
#pragma unroll
  for (int mt = 0; mt < MT; mt++)
#pragma unroll
    for (int q = 0; q < 4; q++) red[((wave * MT + mt) * 4 + q) * 64 + lane] = acc[mt][q];
  __syncthreads();

  const bool split = a.ks > 1;
  for (int e = threadIdx.x; e < MT * 64; e += NW * 64) {
    const int mt = e >> 6;
    const int ln = e & 63;
    const int lq = ln >> 4;
    const int lnl = ln & 15;
    float tot[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
      float s = 0.f;
      for (int w = 0; w < NW; w++) s += red[((w * MT + mt) * 4 + q) * 64 + ln];
      tot[q] = s;
    }
#pragma unroll
    for (int u = 0; u < 4 / S; u++) {
      float y = 0.f;
#pragma unroll
      for (int sl = 0; sl < S; sl++) y += tot[u * S + sl];
      const int m = (16 * mt + 4 * lq) / S + u;
      if (m < count && n0 + lnl < N) {
        const int64_t orow = a.seg ? (int64_t)a.orows[r0 + m] : (int64_t)sidx * a.rps + m;
        if (split) {
          a.ws[((int64_t)blockIdx.z * a.out_rows + orow) * N + n0 + lnl] = y;
        } else {
          a.out[orow * N + n0 + lnl] = (uint16_t)f32_to_bf16_bits(y);
        }
      }
    }
  }
}

// Second pass of a K split: out = bf16(sum over z of the fp32 partials), in a
// fixed order (bitwise reproducible; no cross-workgroup fences needed).
// XT: 16-bit result type (0 bfloat16, 1 float16)
template <int XT>
__global__ __launch_bounds__(256) void qmv_splitk_reduce(const float* __restrict__ ws, uint16_t* __restrict__ out,
                                                         int64_t n, int ks) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float y = 0.f;
  for (int z = 0; z < ks; z++) y += ws[(int64_t)z * n + i];
  out[i] = (uint16_t)f32_to_xt<XT>(y);
}

// The same sum, 4 outputs per thread: 16-byte partial loads, up to 16
// splits' loads in flight before their adds (one memory round trip for the
// mid-size decode kernel's 14 K ranges instead of four; the split order of
// the sum is unchanged).
template <int XT>
__global__ __launch_bounds__(256) void qmv_splitk_reduce4(const float4* __restrict__ ws, uint2* __restrict__ out,
                                                          int64_t n4, int ks) {
  constexpr int ZB = 16;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n4) return;
  float4 y = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int z = 0; z < ks; z += ZB) {  // uniform
    float4 v[ZB];
#pragma unroll
    for (int u = 0; u < ZB; u++)
      if (z + u < ks) v[u] = ws[(int64_t)(z + u) * n4 + i];
#pragma unroll
    for (int u = 0; u < ZB; u++) {
      if (z + u < ks) {
        y.x += v[u].x;
        y.y += v[u].y;
        y.z += v[u].z;
        y.w += v[u].w;
      }
    }
  }
  out[i] = make_uint2(f32_to_xt<XT>(y.x) | (f32_to_xt<XT>(y.y) << 16),
                      f32_to_xt<XT>(y.z) | (f32_to_xt<XT>(y.w) << 16));
}

template <int XT>
static void splitk_reduce_xt(const float* ws, uint16_t* out, int64_t n, int ks, hipStream_t stream) {
  if (n % 4 == 0 && (reinterpret_cast<uintptr_t>(out) & 7) == 0 && (reinterpret_cast<uintptr_t>(ws) & 15) == 0) {
    const int64_t n4 = n / 4;
    hipLaunchKernelGGL(qmv_splitk_reduce4<XT>, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, stream,
                       reinterpret_cast<const float4*>(ws), reinterpret_cast<uint2*>(out), n4, ks);
  } else {
    hipLaunchKernelGGL(qmv_splitk_reduce<XT>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, ws, out, n,
                       ks);
  }
}

hipError_t launch_splitk_reduce(const float* ws, uint16_t* out, int64_t n, int ks, hipStream_t stream, int xt) {
  if (xt == 1) splitk_reduce_xt<1>(ws, out, n, ks, stream);
  else splitk_reduce_xt<0>(ws, out, n, ks, stream);
  return hipGetLastError();
}

// The sum over the partials [ks][M][t.ntot] of several matrices: thread i
// takes VEC consecutive columns of one row (a matrix's columns start at a
// multiple of VEC), finds their matrix and writes its output; the same split
// order as qmv_splitk_reduce4, so the bits are those of one reduction per
// matrix.
template <int XT, int VEC>
__global__ __launch_bounds__(256) void qmv_splitk_reduce_multi(const float* __restrict__ ws, const QmvMatTable t,
                                                              int M, int ks) {
  constexpr int ZB = 16;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int cq = t.ntot / VEC;
  if (i >= (int64_t)M * cq) return;
  const int m = (int)(i / cq), c = (int)(i % cq) * VEC;
  int p = 0;
#pragma unroll
  for (int j = 0; j < kQmvMultiMax - 1; j++) p += (j < t.n - 1 && c >= t.noff[j + 1]) ? 1 : 0;
  const int64_t MN = (int64_t)M * t.ntot;
  const float* src = ws + (int64_t)m * t.ntot + c;
  float y[VEC];
#pragma unroll
  for (int e = 0; e < VEC; e++) y[e] = 0.f;
  for (int z = 0; z < ks; z += ZB) {  // uniform
    float v[ZB][VEC];
#pragma unroll
    for (int u = 0; u < ZB; u++) {
      if (z + u < ks) {
        if constexpr (VEC == 4) {
          const float4 q = *reinterpret_cast<const float4*>(src + (int64_t)(z + u) * MN);
          v[u][0] = q.x;
          v[u][1] = q.y;
          v[u][2] = q.z;
          v[u][3] = q.w;
        } else if constexpr (VEC == 2) {
          const float2 q = *reinterpret_cast<const float2*>(src + (int64_t)(z + u) * MN);
          v[u][0] = q.x;
          v[u][1] = q.y;
        } else {
          v[u][0] = src[(int64_t)(z + u) * MN];
        }
      }
    }
#pragma unroll
    for (int u = 0; u < ZB; u++)
      if (z + u < ks)
#pragma unroll
        for (int e = 0; e < VEC; e++) y[e] += v[u][e];
  }
  uint16_t* dst = t.out[0];
  int Np = t.N[0], off = 0;
#pragma unroll
  for (int j = 1; j < kQmvMultiMax; j++) {
    const bool on = p == j;
    dst = on ? t.out[j] : dst;
    Np = on ? t.N[j] : Np;
    off = on ? t.noff[j] : off;
  }
#pragma unroll
  for (int e = 0; e < VEC; e++) dst[(int64_t)m * Np + (c - off) + e] = (uint16_t)f32_to_xt<XT>(y[e]);
}

hipError_t launch_splitk_reduce_multi(const float* ws, const QmvMatTable& t, int M, int ks, hipStream_t stream,
                                      int xt, int vec_req) {
  // one output per thread for long K (many splits: the Llama-3-8B down shape
  // at 5-16 rows, 14 splits, 0.2-0.6 us faster on MI355X), else four
  int vec = vec_req == 1 || vec_req == 2 || vec_req == 4 ? vec_req : (ks >= 8 ? 1 : 4);
  auto fits = [&](int v) {
    bool ok = (reinterpret_cast<uintptr_t>(ws) & (4 * v - 1)) == 0 && t.ntot % v == 0;
    for (int j = 0; j < t.n; j++) ok = ok && t.N[j] % v == 0 && t.noff[j] % v == 0;
    return ok;
  };
  while (vec > 1 && !fits(vec)) vec /= 2;
  const int64_t n = (int64_t)M * t.ntot / vec;
  const dim3 grid((unsigned)((n + 255) / 256)), block(256);
#define RM_CASE(V)                                                                                          \
  if (vec == V) {                                                                                           \
    if (xt == 1) hipLaunchKernelGGL((qmv_splitk_reduce_multi<1, V>), grid, block, 0, stream, ws, t, M, ks); \
    else hipLaunchKernelGGL((qmv_splitk_reduce_multi<0, V>), grid, block, 0, stream, ws, t, M, ks);         \
  }
  RM_CASE(1)
  RM_CASE(2)
  RM_CASE(4)
#undef RM_CASE
  return hipGetLastError();
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

// ---- gather grouping by expert (one workgroup) ------------------------------
// Counting sort of the B index entries by expert (rhs), then segments of at
// most `cap` rows of one expert.  Entry b contributes output rows b*M + m
// (m < M) computed from x rows lhs[b]*M + m.  Rows of one expert are
// contiguous in xrows/orows; their order inside the expert follows LDS
// atomics and does not affect any result (each output row is computed on its
// own).  seg[s] = {expert, first grouped row, rows}; nseg[0] = segment count.

namespace {
constexpr int kGroupThreads = 1024;

// exclusive scan of one value per thread over the workgroup (Hillis-Steele in LDS)
__device__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* tmp) {
  const int t = threadIdx.x;
  tmp[t] = v;
  __syncthreads();
  for (int off = 1; off < kGroupThreads; off <<= 1) {
    const uint32_t add = t >= off ? tmp[t - off] : 0u;
    __syncthreads();
    tmp[t] += add;
    __syncthreads();
  }
  const uint32_t incl = tmp[t];
  __syncthreads();
  return incl - v;
}
}  // namespace

__global__ __launch_bounds__(kGroupThreads) void group_by_expert_kernel(GroupArgs a) {
  extern __shared__ uint32_t gsh[];
  uint32_t* cnt = gsh;                 // [E] entries per expert
  uint32_t* start = gsh + a.E;         // [E] first grouped entry
  uint32_t* sstart = gsh + 2 * a.E;    // [E] first segment
  uint32_t* tmp = gsh + 3 * a.E;       // [kGroupThreads] scan scratch
  const int t = threadIdx.x;
  for (int e = t; e < a.E; e += kGroupThreads) cnt[e] = 0u;
  __syncthreads();
  for (int b = t; b < a.B; b += kGroupThreads) atomicAdd(&cnt[a.rhs[b]], 1u);
  __syncthreads();
  // each thread owns a contiguous run of experts; scan the run totals
  const int per = (a.E + kGroupThreads - 1) / kGroupThreads;
  const int e0 = min(t * per, a.E), e1 = min(e0 + per, a.E);
  uint32_t ent = 0, segs = 0;
  for (int e = e0; e < e1; e++) {
    ent += cnt[e];
    segs += (cnt[e] * (uint32_t)a.M + (uint32_t)a.cap - 1) / (uint32_t)a.cap;
  }
  uint32_t ent0 = block_exclusive_scan(ent, tmp);
  uint32_t seg0 = block_exclusive_scan(segs, tmp);
  for (int e = e0; e < e1; e++) {
    start[e] = ent0;
    sstart[e] = seg0;
    ent0 += cnt[e];
    seg0 += (cnt[e] * (uint32_t)a.M + (uint32_t)a.cap - 1) / (uint32_t)a.cap;
  }
  if (t == kGroupThreads - 1) a.nseg[0] = seg0;
  __syncthreads();
  // segment table: expert e's rows [start*M, (start+cnt)*M) in pieces of cap
  for (int e = t; e < a.E; e += kGroupThreads) {
    const uint32_t rows = cnt[e] * (uint32_t)a.M;
    const uint32_t row0 = start[e] * (uint32_t)a.M;
    for (uint32_t j = 0, s = sstart[e]; j * (uint32_t)a.cap < rows; j++, s++) {
      a.seg[3 * s] = (uint32_t)e;
      a.seg[3 * s + 1] = row0 + j * (uint32_t)a.cap;
      a.seg[3 * s + 2] = min((uint32_t)a.cap, rows - j * (uint32_t)a.cap);
    }
  }
  __syncthreads();
  // scatter rows (cnt is reused as the fill counter)
  for (int e = t; e < a.E; e += kGroupThreads) cnt[e] = 0u;
  __syncthreads();
  for (int b = t; b < a.B; b += kGroupThreads) {
    const uint32_t e = a.rhs[b];
    const uint32_t p = start[e] + atomicAdd(&cnt[e], 1u);
    for (int m = 0; m < a.M; m++) {
      a.xrows[p * a.M + m] = a.lhs[b] * (uint32_t)a.M + (uint32_t)m;
      a.orows[p * a.M + m] = (uint32_t)b * (uint32_t)a.M + (uint32_t)m;
    }
  }
}

hipError_t launch_group_by_expert(const GroupArgs& a, hipStream_t stream) {
  const size_t lds = (size_t)(3 * a.E + kGroupThreads) * sizeof(uint32_t);
  hipLaunchKernelGGL(group_by_expert_kernel, dim3(1), dim3(kGroupThreads), lds, stream, a);
  return hipGetLastError();
}

// ---- host launch -----------------------------------------------------------

namespace {

// (NW, TK) instantiated for every format: waves per workgroup and K-steps
// per wave.  One workgroup covers NW * TK K-steps.
template <int FMT, int GS, int MT>
hipError_t launch_nwt(int nw, int tk, const QmvArgs& a, dim3 grid, size_t lds, hipStream_t stream) {
#define QMV_CASE(NW_, TK_)                                                                             \
  if (nw == NW_ && tk == TK_) {                                                                        \
    hipLaunchKernelGGL((qmv_kernel<FMT, GS, MT, NW_, TK_>), grid, dim3(NW_ * 64), lds, stream, a);    \
    return hipGetLastError();                                                                          \
  }
  QMV_CASE(4, 4)
  QMV_CASE(4, 8)
  QMV_CASE(8, 4)
  QMV_CASE(8, 8)
  QMV_CASE(16, 4)
  QMV_CASE(16, 8)
#undef QMV_CASE
  return hipErrorInvalidValue;
}

template <int FMT, int GS>
hipError_t launch_mt(int mt, int nw, int tk, const QmvArgs& a, dim3 grid, size_t lds, hipStream_t stream) {
  switch (mt) {
    case 1: return launch_nwt<FMT, GS, 1>(nw, tk, a, grid, lds, stream);
    case 2: return launch_nwt<FMT, GS, 2>(nw, tk, a, grid, lds, stream);
    default: return launch_nwt<FMT, GS, 4>(nw, tk, a, grid, lds, stream);
  }
}

bool valid_nwt(int nw, int tk) { return (nw == 4 || nw == 8 || nw == 16) && (tk == 4 || tk == 8); }
}  // namespace

int qmv_ck(int fmt) { return fmt == AFF8 ? 16 : 32; }

const uint32_t kQmvLdsMax = 160 * 1024;  // LDS per workgroup on gfx950

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

QmvPlan qmv_plan(int fmt, int gs, int64_t N, int64_t K, int rows_lds, int nseg, int num_cus, int nw_req,
                 int tk_req) {
  QmvPlan pl;
  const int kstep = 4 * qmv_ck(fmt);
  const int nkst = (int)((K + kstep - 1) / kstep);
  const int tiles = (int)((N + 15) / 16);
  const int mt = qmv_tile_mt(fmt, gs, rows_lds);
  // Workgroup K ranges are whole multiples of 128 K values (the largest
  // group), so activation sums never straddle two workgroups.
  const int step_align = 128 / kstep;
  // Default shape: the first (NW, TK) whose NW * TK covers K, so one
  // workgroup streams whole rows and no second pass is needed.
  int nw = 16 / mt, tk = 8;
  const int opts[5][2] = {{8, 4}, {16, 4}, {16, 8}, {8, 8}, {4, 8}};
  for (auto& o : opts) {
    if (o[0] * mt > 16) continue;
    if (o[0] * o[1] >= nkst) {
      nw = o[0];
      tk = o[1];
      break;
    }
  }
  if (valid_nwt(nw_req, tk_req) && nw_req * mt <= 16) {
    nw = nw_req;
    tk = tk_req;
  }
  auto per_of = [&](int k) {
    int per = (nkst + k - 1) / k;
    per = ((per + step_align - 1) / step_align) * step_align;
    return per;
  };
  // the per-wave regions must fit the LDS of one workgroup (160 KiB on gfx950)
  auto lds_of = [&](int nw_, int tk_) {
    int k = 1;
    while (per_of(k) > nw_ * tk_) k++;
    return qmv_lds_layout(fmt, gs, rows_lds, tk_, nw_, mt, per_of(k) * kstep / gs).total;
  };
  while (lds_of(nw, tk) > kQmvLdsMax && nw > 4) nw /= 2;
  while (lds_of(nw, tk) > kQmvLdsMax && tk > 4) tk = 4;
  int ks = 1;
  while (per_of(ks) > nw * tk) ks++;  // a workgroup holds at most NW * TK K-steps
  const int per = per_of(ks);
  pl.ks = (nkst + per - 1) / per;
  pl.kst_per_wg = per;
  pl.tiles = tiles;
  pl.nw = nw;
  pl.p = tk;
  pl.mt = mt;
  pl.lds = qmv_lds_layout(fmt, gs, rows_lds, tk, nw, mt, per * kstep / gs).total;
  (void)num_cus;
  (void)nseg;
  return pl;
}

hipError_t qmv_launch(int fmt, int gs, const QmvArgs& a, int nseg_slots, const QmvPlan& p, hipStream_t stream) {
  dim3 grid((unsigned)p.tiles, (unsigned)nseg_slots, (unsigned)p.ks);
  hipError_t e;
  switch (fmt) {
    case AFF4:
      e = gs == 32 ? launch_mt<AFF4, 32>(p.mt, p.nw, p.p, a, grid, p.lds, stream)
        : gs == 64 ? launch_mt<AFF4, 64>(p.mt, p.nw, p.p, a, grid, p.lds, stream)
                   : launch_mt<AFF4, 128>(p.mt, p.nw, p.p, a, grid, p.lds, stream);
      break;
    case AFF8:
      e = gs == 32 ? launch_mt<AFF8, 32>(p.mt, p.nw, p.p, a, grid, p.lds, stream)
        : gs == 64 ? launch_mt<AFF8, 64>(p.mt, p.nw, p.p, a, grid, p.lds, stream)
                   : launch_mt<AFF8, 128>(p.mt, p.nw, p.p, a, grid, p.lds, stream);
      break;
    default:
      e = launch_mt<MXFP4, 32>(p.mt, p.nw, p.p, a, grid, p.lds, stream);
      break;
  }
  if (e != hipSuccess || p.ks == 1) return e;
  return launch_splitk_reduce(a.ws, a.out, (int64_t)a.out_rows * a.N, p.ks, stream);
}

}  // namespace mlxq
