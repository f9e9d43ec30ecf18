// qmv_fr.hip — full-row decode kernel (1 or 2 activation rows per weight
// matrix) for gfx950.
//
// Same product as qmv.hip and qmv_rs.hip (reference decode route:
// overlays/rocm/mlx/backend/rocm/quantized/qmv_tiled_kernel.hip:29-128 and the
// MoE decode kernels of qmm.hip:5578-6054; CPU math overlays/cpu/mlx/backend/
// cpu/quantized.cpp:199-257 affine, 550-597 mxfp4).
//
// Layout.  A workgroup of 8 waves owns 8*R consecutive weight rows; wave w
// streams rows w*R .. w*R+R-1 whole, 1 KiB (one load instruction, 16 bytes a
// lane) at a time, so a wave reads R*row_bytes consecutive bytes and the
// chip's loads in flight form dense address ranges.  All of a wave's loads are
// issued before any arithmetic; each later consumer waits only for its own.
//
// The activations are read from HBM/L2 once per workgroup into LDS (bf16,
// 16-byte pieces laid out [row][chunk][piece][lane] so lane reads are
// conflict-free), together with the per-lane activation sums the affine fold
// needs, and the tile's scales ([group][row], fp32).  Lane L of a wave always
// covers the 32 (4-bit) or 16 (8-bit) K positions L of every 1 KiB chunk, so
// its 16 bytes of a row lie in one quantization group:
//   y += s * sum((128 + q) x) + (b - 128 s) * sum(x)        (AFF4)
//   y += s * sum(q x) + b * sum(x)                            (AFF8)
//   y += 2^(e-127) * sum(fp4(q) x)                            (MXFP4)
// with the sums in fp32 via v_dot2_f32_bf16.  Each wave reduces its own rows
// (DPP within 16-lane rows, then two cross-row exchanges), so no workgroup
// barrier follows the loads' arrival; results are bitwise reproducible.
//
// Buffer loads (raw, bounds checked) read zeros past the end of an operand:
// padded chunk lanes and activation rows past the segment's count cost no
// special cases.
#include "common.hpp"
#include "kernels.hpp"

namespace mlxq {

namespace {

constexpr int kWaves = 8;  // waves per workgroup
constexpr int kSPre = 4;   // scale units per thread issued before the weights

}  // namespace

// LDS of one workgroup: activations (MR x C chunks x 64 lanes x 64 or 32
// bytes), their per-lane sums (MR x C x 64 fp32), the tile's scales (G x 8R,
// 8 or 4 bytes each).
struct QmvFrLds {
  uint32_t x, xs, sb, total;
};
__host__ __device__ inline QmvFrLds qmv_fr_lds(int fmt, int mr, int r, int chunks, int64_t G) {
  QmvFrLds l;
  l.x = 0;
  l.xs = (uint32_t)(mr * chunks * (fmt == AFF8 ? 2048 : 4096));
  l.sb = l.xs + (uint32_t)(mr * chunks * 64 * 4);
  l.total = l.sb + (uint32_t)(G * kWaves * r * (fmt != MXFP4 ? 8 : 4));
  return l;
}

// FMT: weight format; MR: activation rows (1 or 2); R: rows per wave;
// CMAX: 1 KiB chunks per row compiled for (a row has `chunks` <= CMAX).
template <int FMT, int MR, int R, int CMAX>
__global__ __launch_bounds__(kWaves * 64) void qmv_fr_kernel(const QmvArgs a, int gs_shift, int chunks) {
  constexpr bool AFF = FMT != MXFP4;
  constexpr int BITS = FMT == AFF8 ? 8 : 4;
  constexpr int KL = 128 / BITS;  // K positions per lane and chunk (16 bytes)
  constexpr int XV = KL / 8;      // 16-byte activation pieces per lane and chunk
  constexpr int NP = KL / 2;      // bf16 pairs per lane and chunk
  constexpr int RW = kWaves * R;  // rows per workgroup
  constexpr int LRW = log2i(RW);
  constexpr int V = R * MR;       // partial sums per lane
  static_assert(V <= 16 && (V & (V - 1)) == 0, "partials per lane must be a power of two <= 16");
  constexpr int VQ = 16 / V;      // lanes holding one partial after the row butterfly
  constexpr int SB = AFF ? 8 : 4; // LDS bytes per staged scale
  constexpr int NT = kWaves * 64;
  constexpr int LXV = log2i(XV);
  constexpr int XPRE = (MR * CMAX * 64 * XV + NT - 1) / NT;  // activation loads per thread

  extern __shared__ __align__(16) unsigned char smem[];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int sidx = blockIdx.y;

  // ---- segment (workgroup-uniform) ----------------------------------------
  const int count = min(a.rps, a.total_rows - sidx * a.rps);
  if (count <= 0) return;
  const int expert = seg_index(a.rhs, a.rhs_stride, sidx, a.E, a.w_expert_stride ? sidx : 0);
  const int xbatch = seg_index(a.lhs, a.lhs_stride, sidx, a.X, a.lhs_div > 1 ? sidx / a.lhs_div : sidx);

  const int N = a.N;
  const int K = a.K;
  const int nlc = K / KL;                  // 16-byte lane chunks per row
  const uint32_t RB = (uint32_t)nlc * 16u; // bytes per weight row
  const int G = K >> gs_shift;
  const int row0 = blockIdx.x * RW;
  const int wrow0 = row0 + wave * R;       // this wave's first row
  const QmvFrLds L = qmv_fr_lds(FMT, MR, R, chunks, G);

  const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(a.w + (int64_t)expert * a.w_expert_stride, (uint32_t)N * RB);
  const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(a.x + (int64_t)xbatch * a.rps * K, (uint32_t)count * (uint32_t)K * 2u);
  const int64_t sb0 = (int64_t)expert * a.s_expert_stride;
  const __amdgpu_buffer_rsrc_t sr =
      buffer_rsrc(reinterpret_cast<const uint8_t*>(a.scales) + sb0 * (AFF ? 2 : 1), (uint32_t)(N * G * (AFF ? 2 : 1)));
  const __amdgpu_buffer_rsrc_t br =
      buffer_rsrc(AFF ? (const void*)(a.biases + sb0) : a.scales, (uint32_t)(AFF ? N * G * 2 : 0));

  // ---- 1. loads: activations, scales, then this wave's rows ----------------
  // activation piece i of row m: 8 bf16 at K = 8 i (pieces past K read 0);
  // a row is padded to whole chunks of 64 * XV pieces
  const int xpieces = chunks * 64 * XV;
  const int kp = K / 8;
  u32x4 xpre[MR][XPRE];
#pragma unroll
  for (int m = 0; m < MR; m++)
#pragma unroll
    for (int u = 0; u < XPRE; u++) {
      const int i = (int)threadIdx.x + NT * u;
      const uint32_t off = i < kp ? (uint32_t)(m * K + 8 * i) * 2u : kDeadOfs;
      xpre[m][u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
    }

  // scales of the G x RW tile: thread t stages row t % RW, units of `upw`
  // groups (a word; a short or byte when rows hold odd counts) t / RW + k NT / RW
  const int upw = AFF ? ((G & 1) ? 1 : 2) : ((G & 3) ? ((G & 1) ? 1 : 2) : 4);
  const int gu = G / upw;
  const int s_row = threadIdx.x & (RW - 1);
  const int s_j0 = threadIdx.x >> LRW;
  constexpr int s_js = NT / RW;
  const uint32_t s_og = (uint32_t)(min(row0 + s_row, N - 1) * G);
  auto load_unit = [&](int jn, uint32_t& s_, uint32_t& b_) {
    const uint32_t og = jn < gu ? s_og + (uint32_t)(jn * upw) : 0u;
    if constexpr (AFF) {
      if (upw == 2) {
        s_ = __builtin_amdgcn_raw_buffer_load_b32(sr, og * 2u, 0, 0);
        b_ = __builtin_amdgcn_raw_buffer_load_b32(br, og * 2u, 0, 0);
      } else {
        s_ = __builtin_amdgcn_raw_buffer_load_b16(sr, og * 2u, 0, 0);
        b_ = __builtin_amdgcn_raw_buffer_load_b16(br, og * 2u, 0, 0);
      }
    } else {
      s_ = upw == 4 ? __builtin_amdgcn_raw_buffer_load_b32(sr, og, 0, 0)
                    : (upw == 2 ? (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(sr, og, 0, 0)
                                : (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(sr, og, 0, 0));
      b_ = 0u;
    }
  };
  uint32_t spre[kSPre], bpre[kSPre];
#pragma unroll
  for (int u = 0; u < kSPre; u++) load_unit(s_j0 + s_js * u, spre[u], bpre[u]);

  // this lane's byte offset in chunk j of a row (padded lanes read 0)
  uint32_t wo[CMAX];
#pragma unroll
  for (int j = 0; j < CMAX; j++) wo[j] = (j < chunks && j * 64 + lane < nlc) ? (uint32_t)(j * 1024 + lane * 16) : kDeadOfs;
  u32x4 wv[R][CMAX];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const uint32_t rowoff = (uint32_t)min(wrow0 + r, N - 1) * RB;  // rows past N: row N-1, never stored
#pragma unroll
    for (int j = 0; j < CMAX; j++)
      wv[r][j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, wo[j], rowoff, 2 /* nt */));
  }
  __builtin_amdgcn_sched_barrier(0);  // keep the arithmetic below the loads

  // ---- 2. stage activations (+ sums) and scales in LDS ---------------------
  // piece i -> chunk i / (64 XV), lane (i / XV) % 64, piece-in-lane i % XV;
  // the XV pieces of a lane chunk sit on XV consecutive threads
  auto put_x = [&](int m, int i, u32x4 v) {
    float s = 0.f;
    if constexpr (AFF) {
#pragma unroll
      for (int e = 0; e < 4; e++) s = dot2(v[e], 0x3F803F80u, s);  // sum of the 8 values
      s += dpp<0xB1>(s);                                           // + the piece on lane ^ 1
      if constexpr (XV == 4) s += dpp<0x4E>(s);                    // + the pieces on lanes ^ 2
    }
    if constexpr (FMT == AFF4) v = perm_aff4_v(v);
    if (i < xpieces) {
      const int j = i >> (6 + LXV), ln = (i >> LXV) & 63, pv = i & (XV - 1);
      *reinterpret_cast<u32x4*>(smem + L.x + (uint32_t)(((m * chunks + j) * XV + pv) * 1024 + ln * 16)) = v;
      if (pv == 0) reinterpret_cast<float*>(smem + L.xs)[(m * chunks + j) * 64 + ln] = s;
    }
  };
#pragma unroll
  for (int m = 0; m < MR; m++)
#pragma unroll
    for (int u = 0; u < XPRE; u++) put_x(m, (int)threadIdx.x + NT * u, xpre[m][u]);

  auto put_unit = [&](int jn, uint32_t s_, uint32_t b_) {
    if (jn >= gu) return;
    for (int h = 0; h < upw; h++) {
      const int idx = (jn * upw + h) * RW + s_row;
      if constexpr (AFF) {
        const float sc = bf16_bits_to_f32((s_ >> (16 * h)) & 0xFFFFu);
        const float bi = bf16_bits_to_f32((b_ >> (16 * h)) & 0xFFFFu);
        reinterpret_cast<float2*>(smem + L.sb)[idx] = float2{sc, FMT == AFF4 ? __builtin_fmaf(-128.0f, sc, bi) : bi};
      } else {
        reinterpret_cast<float*>(smem + L.sb)[idx] = e8m0_to_f32((s_ >> (8 * h)) & 0xFFu);
      }
    }
  };
#pragma unroll
  for (int u = 0; u < kSPre; u++) put_unit(s_j0 + s_js * u, spre[u], bpre[u]);
  for (int jn = s_j0 + s_js * kSPre; jn < gu; jn += s_js) {  // long rows: the rest
    uint32_t s_, b_;
    load_unit(jn, s_, b_);
    put_unit(jn, s_, b_);
  }
  __syncthreads();

  // ---- 3. dot products -----------------------------------------------------
  float y[R][MR];
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int m = 0; m < MR; m++) y[r][m] = 0.f;

#pragma unroll
  for (int j = 0; j < CMAX; j++) {
    if (j < chunks) {  // workgroup-uniform
      u32x4 xv[MR][XV];
      float xs[MR];
#pragma unroll
      for (int m = 0; m < MR; m++) {
#pragma unroll
        for (int v = 0; v < XV; v++)
          xv[m][v] = *reinterpret_cast<const u32x4*>(smem + L.x + (uint32_t)(((m * chunks + j) * XV + v) * 1024 + lane * 16));
        xs[m] = reinterpret_cast<const float*>(smem + L.xs)[(m * chunks + j) * 64 + lane];
      }
      const bool live = j * 64 + lane < nlc;
      const int g = min(((j * 64 + lane) * KL) >> gs_shift, G - 1);
      const uint32_t sbase = L.sb + (uint32_t)(g * RW + wave * R) * SB;
#pragma unroll
      for (int r = 0; r < R; r++) {
        float sc, bp = 0.f;
        if constexpr (AFF) {
          const float2 t = *reinterpret_cast<const float2*>(smem + sbase + r * 8);
          sc = t.x;
          bp = t.y;
        } else {
          sc = *reinterpret_cast<const float*>(smem + sbase + r * 4);
        }
        if (!live) sc = bp = 0.f;  // padded lanes add exactly 0
        uint32_t pr[NP];
        const u32x4 w = wv[r][j];
        if constexpr (FMT == AFF8) {
          uint32_t t[4];
          unpack_aff8(w[0], w[1], t);
#pragma unroll
          for (int e = 0; e < 4; e++) pr[e] = t[e];
          unpack_aff8(w[2], w[3], t);
#pragma unroll
          for (int e = 0; e < 4; e++) pr[4 + e] = t[e];
        } else {
#pragma unroll
          for (int q = 0; q < 4; q++) {
            uint32_t t[4];
            if constexpr (FMT == AFF4) unpack_aff4(w[q], t);
            else unpack_mxfp4(w[q], t);
#pragma unroll
            for (int e = 0; e < 4; e++) pr[4 * q + e] = t[e];
          }
        }
#pragma unroll
        for (int m = 0; m < MR; m++) {
          float d = 0.f;
#pragma unroll
          for (int p = 0; p < NP; p++) d = dot2(pr[p], xv[m][p / 4][p % 4], d);
          float acc = y[r][m];
          if constexpr (AFF) acc = __builtin_fmaf(bp, xs[m], acc);
          y[r][m] = __builtin_fmaf(sc, d, acc);
        }
      }
    }
  }

  // ---- 4. reduce this wave's partials over its 64 lanes and store ----------
  float v[V];
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int m = 0; m < MR; m++) v[r * MR + m] = y[r][m];
  row_butterfly<V, 0>(v, lane);
  float t = v[0];
  t += __shfl_xor(t, 16);
  t += __shfl_xor(t, 32);
  const int li = lane & 15;
  if (lane < 16 && li % VQ == 0) {
    const int idx = li / VQ;
    const int r = idx / MR, m = idx % MR;
    const int row = wrow0 + r;
    if (row < N && m < count) a.out[((int64_t)sidx * a.rps + m) * N + row] = (uint16_t)f32_to_bf16_bits(t);
  }
}

// ---- host ------------------------------------------------------------------

namespace {

template <int FMT, int MR>
hipError_t fr_launch(const QmvFrPlan& p, const QmvArgs& a, int gs_shift, dim3 grid, hipStream_t stream) {
#define FR_CASE(R_, C_)                                                                                       \
  if (p.r == R_ && p.cmax == C_) {                                                                            \
    hipLaunchKernelGGL((qmv_fr_kernel<FMT, MR, R_, C_>), grid, dim3(kWaves * 64), p.lds, stream, a, gs_shift, \
                       p.chunks);                                                                             \
    return hipGetLastError();                                                                                 \
  }
  FR_CASE(8, 1)
  FR_CASE(4, 1)
  FR_CASE(4, 2)
  FR_CASE(2, 2)
  FR_CASE(2, 4)
  FR_CASE(1, 4)
  FR_CASE(1, 8)
  FR_CASE(1, 16)
#undef FR_CASE
  return hipErrorInvalidValue;
}

bool fr_valid(int r, int cmax) {
  return (r == 8 && cmax == 1) || (r == 4 && cmax <= 2) || (r == 2 && (cmax == 2 || cmax == 4)) ||
         (r == 1 && cmax >= 4 && cmax <= 16);
}

}  // namespace

QmvFrPlan qmv_fr_plan(int fmt, int gs, int64_t N, int64_t K, int rows, int r_req) {
  QmvFrPlan p;
  if (rows < 1 || rows > 2) return p;
  const int kl = fmt == AFF8 ? 16 : 32;
  if (K % kl != 0 || K % gs != 0) return p;
  const int64_t nlc = K / kl;
  const int64_t chunks = (nlc + 63) / 64;
  if (chunks > 16) return p;
  p.mr = rows;
  p.chunks = (int)chunks;
  p.cmax = chunks <= 1 ? 1 : (chunks <= 2 ? 2 : (chunks <= 4 ? 4 : (chunks <= 8 ? 8 : 16)));
  p.r = p.cmax == 1 ? 8 : (p.cmax == 2 ? 4 : (p.cmax == 4 ? 2 : 1));
  if (r_req > 0 && fr_valid(r_req, p.cmax)) p.r = r_req;
  const int64_t G = K / gs;
  p.lds = qmv_fr_lds(fmt, p.mr, p.r, p.chunks, G).total;
  p.tiles = (int)((N + (int64_t)kWaves * p.r - 1) / ((int64_t)kWaves * p.r));
  // 32-bit buffer offsets with 0x80000000 as the dead-lane marker
  const int64_t wbytes = N * nlc * 16;
  p.ok = fr_valid(p.r, p.cmax) && p.lds <= kQmvLdsMax && wbytes < ((int64_t)1 << 31) &&
         N * G * 2 < ((int64_t)1 << 31) && (int64_t)2 * K * 2 < ((int64_t)1 << 31);
  return p;
}

hipError_t qmv_fr_launch(int fmt, int gs, const QmvArgs& a, int nseg, const QmvFrPlan& p, hipStream_t stream) {
  if (!p.ok) return hipErrorInvalidValue;
  const int gs_shift = log2i(gs);
  const dim3 grid((unsigned)p.tiles, (unsigned)nseg, 1);
  switch (fmt) {
    case AFF4: return p.mr == 1 ? fr_launch<AFF4, 1>(p, a, gs_shift, grid, stream)
                                : fr_launch<AFF4, 2>(p, a, gs_shift, grid, stream);
    case AFF8: return p.mr == 1 ? fr_launch<AFF8, 1>(p, a, gs_shift, grid, stream)
                                : fr_launch<AFF8, 2>(p, a, gs_shift, grid, stream);
    default: return p.mr == 1 ? fr_launch<MXFP4, 1>(p, a, gs_shift, grid, stream)
                              : fr_launch<MXFP4, 2>(p, a, gs_shift, grid, stream);
  }
}

}  // namespace mlxq
