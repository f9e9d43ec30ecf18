// qmv_rs.hip — row-streaming decode kernel (1 to 4 activation rows per
// weight matrix) for gfx950.
//
// Same product as qmv.hip (reference decode route: overlays/rocm/mlx/backend/
// rocm/quantized/qmv_tiled_kernel.hip:29-128 and the MoE decode kernels of
// qmm.hip:5578-6054; CPU math overlays/cpu/mlx/backend/cpu/quantized.cpp:
// 199-257 affine, 550-597 mxfp4), shaped for how HBM3E wants to be read.
//
// Access pattern.  A packed weight row is cut into 1 KiB chunks; chunk c of
// every row of a workgroup's R-row tile is read by wave c, one 16-byte lane
// per 1/64 of the chunk.  Every load instruction therefore moves 1 KiB of
// consecutive bytes and a workgroup reads R whole rows, so the bytes in
// flight form a few dense address ranges.  (Reading the same bytes as 16 rows
// x 64 B per instruction, the fragment layout an MFMA wants, costs about 25%
// more time on MI355X at these sizes.)
//
// Arithmetic.  A lane always covers the same 32 (4-bit) or 16 (8-bit) K
// positions of its rows, so its activations for those positions are loaded
// once into registers.  The codes are widened to bf16 pairs (AFF4 "128 + q"
// with one byte permute per pair, MXFP4 with the gfx950 fp4 conversion, AFF8 via
// byte -> f32 -> bf16) and multiplied with v_dot2_f32_bf16 in fp32.  A lane's
// 16 bytes lie inside one quantization group, so the scale and bias apply
// once per lane and row:  y += s * sum((128+q) x) + (b - 128 s) * sum(x).
// Partial sums of all (row, activation-row) pairs are reduced across the 64
// lanes with a halving butterfly and across waves through LDS in a fixed
// order, so results are bitwise reproducible.
#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"

namespace mlxq {

// LDS bytes of one workgroup: per wave, the scales of its chunks
// (CPW x groups-per-chunk x R rows, row fastest; (scale, bias - 128 scale |
// bias) fp32 pairs for affine, scale fp32 for mxfp4), then the reduction
// buffer (NW waves x 4 lane rows x R*MR partials).
__host__ __device__ inline uint32_t qmv_rs_wave_lds(int fmt, int r, int cpw, int gs) {
  const int kl = fmt == AFF8 ? 16 : 32;
  return (uint32_t)(cpw * (64 * kl / gs) * r * (fmt != MXFP4 ? 8 : 4));
}
__host__ __device__ inline uint32_t qmv_rs_lds(int fmt, int r, int mr, int nw, int cpw, int gs) {
  return (uint32_t)nw * qmv_rs_wave_lds(fmt, r, cpw, gs) + (uint32_t)(nw * 4 * r * mr * 4);
}


// Compact launch arguments of the dense and multi-projection entries: every
// field a wave needs before its first weight load sits in the first few
// scalar-cache lines and no branch depends on a loaded value before the
// weight stream is issued (each dependent round of kernel-argument loads
// costs a memory latency at the start of every workgroup).
struct RsDenseArgs {
  const uint16_t* x;     // count rows of K
  const uint32_t* w;     // [N][K*bits/32]
  const void* scales;
  const uint16_t* biases;
  uint16_t* out;         // count rows of N
  int N, K, count, gs_shift;
};
struct RsMultiArgs {
  const uint16_t* x;
  int K, count, gs_shift, n;
  int tile_end[kQmvMultiMax];
  int N[kQmvMultiMax];
  const uint32_t* w[kQmvMultiMax];
  const void* scales[kQmvMultiMax];
  const uint16_t* biases[kQmvMultiMax];
  uint16_t* out[kQmvMultiMax];
};

// FMT: weight format; MR: activation rows (>= `count`);
// R: weight rows per workgroup (power of two); CPW: 1 KiB chunks per wave and
// row; UPW: quantization groups per scale load (1, 2 or 4: the widest load
// every row's scales stay aligned for, chosen on the host from K / gs).  The
// load width is a template parameter so the scale loads carry no branches:
// a branch join there makes the compiler wait for the loads before it issues
// the weight stream.
//
// One row tile: output rows [tile*R, tile*R + R) of the `count` activation
// rows at x (row stride K) against the matrix Wm (N rows), written to Om
// (row stride N).
template <int FMT, int MR, int R, int CPW, int UPW, int XT = 0>
__device__ __forceinline__ void rs_tile(const uint16_t* x, int count, const uint32_t* Wm, const void* Sm,
                                        const uint16_t* Bm, uint16_t* Om, int N, int K, int gs_shift, int tile) {
  constexpr bool AFF = FMT != MXFP4;
  constexpr int BITS = FMT == AFF8 ? 8 : 4;
  constexpr int KL = 128 / BITS;  // K positions per lane chunk (16 bytes)
  constexpr int XV = KL / 8;      // 16-byte activation pieces per lane chunk
  constexpr int NP = KL / 2;      // bf16 pairs per lane chunk
  constexpr int V = R * MR;       // partial sums per lane
  static_assert(V <= 64 && (V & (V - 1)) == 0, "partials per lane must be a power of two <= 64");
  static_assert((R & (R - 1)) == 0 && R <= 16, "R must be a power of two <= 16");
  constexpr int LR = log2i(R);
  constexpr int VC = V >= 16 ? V / 16 : 1;  // partials per lane after the row butterfly
  constexpr int VQ = V >= 16 ? 1 : 16 / V;  // lanes per partial after it
  constexpr int SBE = 4;                    // scale loads per lane issued before the weights (at most)
  constexpr int ESZ = AFF ? 2 : 1;          // bytes per stored scale
  // offset of the widened affine codes (bfloat16 8-bit codes convert exactly, no offset)
  constexpr float OFS = XT ? 1024.0f : (FMT == AFF4 ? 128.0f : 0.0f);
  constexpr uint32_t ONES = XT ? 0x3C003C00u : 0x3F803F80u;  // the pair (1, 1)

  extern __shared__ __align__(16) unsigned char smem[];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int NW = blockDim.x >> 6;
  const int row0 = tile * R;
  const int nlc = K / KL;  // lane chunks per row
  const uint32_t RB = (uint32_t)nlc * 16u;  // bytes per weight row
  const int G = K >> gs_shift;
  const int gs = 1 << gs_shift;
  unsigned char* wsl = smem + wave * qmv_rs_wave_lds(FMT, R, CPW, gs);  // this wave's scales
  float* red = reinterpret_cast<float*>(smem + NW * qmv_rs_wave_lds(FMT, R, CPW, gs));

  // Buffer resources: bounds-checked loads return 0 past the end, which
  // covers rows past N, activation rows past `count` and dead lanes.
  const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(Wm, (uint32_t)N * RB);
  const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(x, (uint32_t)count * (uint32_t)K * 2u);
  const __amdgpu_buffer_rsrc_t sr = buffer_rsrc(Sm, (uint32_t)(N * G * ESZ));
  const __amdgpu_buffer_rsrc_t br = buffer_rsrc(AFF ? (const void*)Bm : Sm, (uint32_t)(AFF ? N * G * 2 : 0));

  int kc[CPW];
  bool live[CPW];
  uint32_t wo[CPW], xo[CPW];
#pragma unroll
  for (int j = 0; j < CPW; j++) {
    kc[j] = (wave + NW * j) * 64 + lane;
    live[j] = kc[j] < nlc;
    wo[j] = live[j] ? (uint32_t)kc[j] * 16u : kDeadOfs;
    xo[j] = live[j] ? (uint32_t)kc[j] * (KL * 2) : kDeadOfs;
  }

  // ---- 1. loads: activations, the tile's scales, then weights -------------
  u32x4 xv[MR][CPW][XV];
#pragma unroll
  for (int m = 0; m < MR; m++)
#pragma unroll
    for (int j = 0; j < CPW; j++)
#pragma unroll
      for (int v = 0; v < XV; v++)
        xv[m][j][v] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, xo[j] + (uint32_t)(m * K * 2 + v * 16), 0, 0));

  // Scales of this wave's chunks: for each chunk j (groups gbase[j] ..
  // gbase[j] + gc - 1) and row r, gc / upw units of upw groups (up to four
  // groups per load when every row's scales start at a multiple of four
  // groups, else two or one); lane L loads units
  // L, L + 64, ...  A wave reads only what it wrote itself, so no workgroup
  // barrier stands between the loads and the arithmetic.
  constexpr int upw = UPW;  // groups per unit
  const int gc = (64 * KL) >> gs_shift;               // groups per chunk (>= 8)
  const int upc = gc / upw;                           // units per chunk and row
  const int lupc = __builtin_ctz((unsigned)upc);
  const int nunits = CPW * R * upc;
  const int nld = (nunits + 63) / 64;                 // loads per lane (uniform)
  int gbase[CPW];
#pragma unroll
  for (int j = 0; j < CPW; j++) gbase[j] = ((wave + NW * j) * 64 * KL) >> gs_shift;
  auto unit_of = [&](int u, int& j, int& r, int& gl) {
    r = u & (R - 1);
    const int rest = u >> LR;
    gl = rest & (upc - 1);
    j = min(rest >> lupc, CPW - 1);
  };
  // affine units of 4 groups are 8 bytes: words [i][0] hold groups 0-1,
  // [i][1] groups 2-3
  constexpr int SW = AFF && UPW == 4 ? 2 : 1;
  uint32_t sraw[SBE][SW], braw[SBE][SW];
#pragma unroll
  for (int i = 0; i < SBE; i++) {
#pragma unroll
    for (int h = 0; h < SW; h++) sraw[i][h] = braw[i][h] = 0u;
    if (i < nld) {  // wave-uniform
      int j, r, gl;
      unit_of(lane + 64 * i, j, r, gl);
      const uint32_t og = (uint32_t)((row0 + r) * G + gbase[j] + gl * upw);  // in groups
      if constexpr (AFF) {
        if constexpr (UPW == 4) {
          const u32x2 s2 = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(sr, og * 2u, 0, 0));
          const u32x2 b2 = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(br, og * 2u, 0, 0));
          sraw[i][0] = s2[0];
          sraw[i][SW - 1] = s2[1];
          braw[i][0] = b2[0];
          braw[i][SW - 1] = b2[1];
        } else if constexpr (UPW == 2) {
          sraw[i][0] = __builtin_amdgcn_raw_buffer_load_b32(sr, og * 2u, 0, 0);
          braw[i][0] = __builtin_amdgcn_raw_buffer_load_b32(br, og * 2u, 0, 0);
        } else {
          sraw[i][0] = __builtin_amdgcn_raw_buffer_load_b16(sr, og * 2u, 0, 0);
          braw[i][0] = __builtin_amdgcn_raw_buffer_load_b16(br, og * 2u, 0, 0);
        }
      } else {
        if constexpr (UPW == 4) sraw[i][0] = __builtin_amdgcn_raw_buffer_load_b32(sr, og, 0, 0);
        else if constexpr (UPW == 2) sraw[i][0] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(sr, og, 0, 0);
        else sraw[i][0] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(sr, og, 0, 0);
      }
    }
  }

  u32x4 wv[R][CPW];
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int j = 0; j < CPW; j++)
      wv[r][j] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, wo[j] + (uint32_t)(row0 + r) * RB, 0, 2 /* nt */));
  __builtin_amdgcn_sched_barrier(0);  // keep the arithmetic below the loads

  // ---- 2. stage the scales; activation sums and operand order -------------
#pragma unroll
  for (int i = 0; i < SBE; i++) {
    if (i < nld && lane + 64 * i < nunits) {
      int j, r, gl;
      unit_of(lane + 64 * i, j, r, gl);
#pragma unroll
      for (int h = 0; h < UPW; h++) {
        const int idx = (j * gc + gl * UPW + h) * R + r;
        if constexpr (AFF) {
          const float sc = xt_to_f32<XT>((sraw[i][h >> 1] >> (16 * (h & 1))) & 0xFFFFu);
          const float bi = xt_to_f32<XT>((braw[i][h >> 1] >> (16 * (h & 1))) & 0xFFFFu);
          reinterpret_cast<float2*>(wsl)[idx] = float2{sc, OFS != 0.0f ? __builtin_fmaf(-OFS, sc, bi) : bi};
        } else {
          reinterpret_cast<float*>(wsl)[idx] = e8m0_to_f32((sraw[i][0] >> (8 * h)) & 0xFFu);
        }
      }
    }
  }

  float xs[MR][CPW];
#pragma unroll
  for (int m = 0; m < MR; m++)
#pragma unroll
    for (int j = 0; j < CPW; j++) {
      float s = 0.f;
      if constexpr (AFF) {
#pragma unroll
        for (int v = 0; v < XV; v++)
#pragma unroll
          for (int e = 0; e < 4; e++) s = dotx<XT>(xv[m][j][v][e], ONES, s);  // pairs times (1, 1)
      }
      xs[m][j] = s;
      if constexpr (FMT == AFF4) {
#pragma unroll
        for (int v = 0; v < XV; v++) xv[m][j][v] = perm_aff4_v(xv[m][j][v]);
      }
    }
  // the wave's own LDS writes complete in order before its reads (this also
  // fences the compiler)
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

  // ---- 3. dot products, one scale/bias fold per lane chunk -----------------
  uint32_t sbase[CPW];  // LDS byte offset of this lane's group, row 0
#pragma unroll
  for (int j = 0; j < CPW; j++)
    sbase[j] = (uint32_t)(wsl - smem) + (uint32_t)((j * gc + ((lane * KL) >> gs_shift)) * R) * (AFF ? 8u : 4u);

  float y[R][MR];
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int m = 0; m < MR; m++) y[r][m] = 0.f;

#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int j = 0; j < CPW; j++) {
      float sc, bp = 0.f;
      if constexpr (AFF) {
        const float2 t = *reinterpret_cast<const float2*>(smem + sbase[j] + r * 8);
        sc = t.x;
        bp = t.y;
      } else {
        sc = *reinterpret_cast<const float*>(smem + sbase[j] + r * 4);
      }
      if (!live[j]) sc = bp = 0.f;  // lanes past the end of the row add exactly 0
      uint32_t pr[NP];
      const u32x4 w = wv[r][j];
      if constexpr (FMT == AFF8 && XT == 1) {
        // byte pairs (b0, b1), (b2, b3) of each word as float16 1024 + q
#pragma unroll
        for (int q = 0; q < 4; q++) {
          pr[2 * q] = __builtin_amdgcn_perm(0x64646464u, w[q], 0x04010400u);
          pr[2 * q + 1] = __builtin_amdgcn_perm(0x64646464u, w[q], 0x04030402u);
        }
      } else if constexpr (FMT == AFF8) {
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
          if constexpr (FMT == AFF4) unpack_aff4(w[q], t, XT ? 0x64646464u : 0x43434343u);
          else if constexpr (XT == 1) unpack_mxfp4_f16(w[q], t);
          else unpack_mxfp4(w[q], t);
#pragma unroll
          for (int e = 0; e < 4; e++) pr[4 * q + e] = t[e];
        }
      }
#pragma unroll
      for (int m = 0; m < MR; m++) {
        float d = 0.f;
#pragma unroll
        for (int p = 0; p < NP; p++) {
          // pair p covers lane-chunk K positions 2p, 2p+1 (AFF4: the permuted pair of word p/4)
          d = dotx<XT>(pr[p], xv[m][j][p / 4][p % 4], d);
        }
        float acc = y[r][m];
        if constexpr (AFF) acc = __builtin_fmaf(bp, xs[m][j], acc);
        y[r][m] = __builtin_fmaf(sc, d, acc);
      }
    }

  // ---- 4. reduce: 16-lane rows (DPP), then rows and waves (LDS) ------------
  float v[V];
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int m = 0; m < MR; m++) v[r * MR + m] = y[r][m];
  row_butterfly<V, 0>(v, lane);
  const int li = lane & 15;
  if (li % VQ == 0) {
#pragma unroll
    for (int c = 0; c < VC; c++) red[(wave * 4 + (lane >> 4)) * V + (li / VQ) * VC + c] = v[c];
  }
  __syncthreads();
  if ((int)threadIdx.x < V) {
    const int idx = threadIdx.x;
    float tot = 0.f;
    for (int q = 0; q < NW * 4; q++) tot += red[q * V + idx];
    const int r = idx / MR, m = idx % MR;
    const int row = row0 + r;
    if (row < N && m < count) Om[(int64_t)m * N + row] = (uint16_t)f32_to_xt<XT>(tot);
  }
}

// General entry: segments of a gather or of batched weights (segment
// blockIdx.y: expert rhs[s], x batch lhs[s], runs of a sorted gather), and
// the multi-projection table of QmvMulti.
template <int FMT, int MR, int R, int CPW, int UPW>
__global__ __launch_bounds__(512) void qmv_rs_kernel(const QmvArgs a, int gs_shift, const QmvMulti mp) {
  constexpr bool AFF = FMT != MXFP4;
  constexpr int ESZ = AFF ? 2 : 1;
  const int sidx = blockIdx.y;
  int count = min(a.rps, a.total_rows - sidx * a.rps);
  if (count <= 0) return;
  const int expert = seg_index(a.rhs, a.rhs_stride, sidx, a.E, a.w_expert_stride ? sidx : 0);
  if (a.runs) {
    // Expert runs of a sorted gather (one activation row per entry, MR >= 4):
    // entry sidx starts a segment where the expert changes or at a multiple
    // of 4, and the segment takes the following entries of the same expert
    // up to the next multiple of 4; every other entry's workgroup exits.  So
    // each entry is computed once and each run of an expert streams its
    // weights once per 4 entries instead of once per entry.
    if ((sidx & 3) != 0 && seg_index(a.rhs, a.rhs_stride, sidx - 1, a.E, 0) == expert) return;
    count = 1;
    while (count < 4 && ((sidx + count) & 3) != 0 && sidx + count < a.total_rows &&
           seg_index(a.rhs, a.rhs_stride, sidx + count, a.E, 0) == expert)
      count++;
  }
  const int xbatch = seg_index(a.lhs, a.lhs_stride, sidx, a.X, a.lhs_div > 1 ? sidx / a.lhs_div : sidx);
  const uint32_t* Wm = a.w;
  const void* Sm = a.scales;
  const uint16_t* Bm = a.biases;
  uint16_t* Om = a.out;
  int N = a.N;
  int tile = blockIdx.x;
  if (mp.n > 1) {  // workgroup-uniform
    int p = 0;
    while (p < mp.n - 1 && tile >= mp.tile_end[p]) p++;
    tile -= p > 0 ? mp.tile_end[p - 1] : 0;
    Wm = mp.w[p];
    Sm = mp.scales[p];
    Bm = mp.biases[p];
    Om = mp.out[p];
    N = mp.N[p];
  }
  const int64_t sb0 = (int64_t)expert * a.s_expert_stride;
  rs_tile<FMT, MR, R, CPW, UPW>(a.x + (int64_t)xbatch * a.rps * a.K, count, Wm + (int64_t)expert * a.w_expert_stride,
                                reinterpret_cast<const uint8_t*>(Sm) + sb0 * ESZ, Bm ? Bm + sb0 : Bm,
                                Om + (int64_t)sidx * a.rps * N, N, a.K, gs_shift, tile);
}

// Dense entry: one 2-D matrix, `count` <= MR activation rows; XT: bfloat16
// or float16 elements.
template <int FMT, int MR, int R, int CPW, int UPW, int XT>
__global__ __launch_bounds__(512) void qmv_rs_dense_kernel(const RsDenseArgs a) {
  rs_tile<FMT, MR, R, CPW, UPW, XT>(a.x, a.count, a.w, a.scales, a.biases, a.out, a.N, a.K, a.gs_shift, blockIdx.x);
}

// Several 2-D matrices of the same activations: matrix p owns the row tiles
// [tile_end[p-1], tile_end[p]).  Every table entry is read unconditionally
// and selected, so the kernel-argument loads form one round.
template <int FMT, int MR, int R, int CPW, int UPW>
__global__ __launch_bounds__(512) void qmv_rs_multi_kernel(const RsMultiArgs a) {
  int tile = blockIdx.x;
  int p = 0;
#pragma unroll
  for (int i = 0; i < kQmvMultiMax - 1; i++) p += (i < a.n - 1 && tile >= a.tile_end[i]) ? 1 : 0;
  const uint32_t* Wm = a.w[0];
  const void* Sm = a.scales[0];
  const uint16_t* Bm = a.biases[0];
  uint16_t* Om = a.out[0];
  int N = a.N[0];
  int t0 = 0;
#pragma unroll
  for (int i = 1; i < kQmvMultiMax; i++) {
    const bool on = p == i;
    Wm = on ? a.w[i] : Wm;
    Sm = on ? a.scales[i] : Sm;
    Bm = on ? a.biases[i] : Bm;
    Om = on ? a.out[i] : Om;
    N = on ? a.N[i] : N;
    t0 = on ? a.tile_end[i - 1] : t0;
  }
  rs_tile<FMT, MR, R, CPW, UPW>(a.x, a.count, Wm, Sm, Bm, Om, N, a.K, a.gs_shift, tile - t0);
}

// ---- host ------------------------------------------------------------------

namespace {

enum RsEntry { RS_GENERAL, RS_DENSE, RS_MULTI };

struct RsLaunch {
  RsEntry entry;
  int xt;  // 0 bfloat16, 1 float16 (dense entry only)
  dim3 grid;
  const QmvArgs* a;
  int gs_shift;
  const QmvMulti* mp;
  RsDenseArgs dense;
  RsMultiArgs multi;
};

template <int FMT, int UPW>
hipError_t rs_launch_upw(const QmvRsPlan& p, const RsLaunch& L, hipStream_t stream) {
  const dim3 block((unsigned)(p.nw * 64));
#define RS_CASE(MR_, R_, CPW_)                                                                                     \
  if (p.mr == MR_ && p.r == R_ && p.cpw == CPW_) {                                                                 \
    if (L.entry == RS_DENSE && L.xt == 1)                                                                          \
      hipLaunchKernelGGL((qmv_rs_dense_kernel<FMT, MR_, R_, CPW_, UPW, 1>), L.grid, block, p.lds, stream, L.dense); \
    else if (L.entry == RS_DENSE)                                                                                  \
      hipLaunchKernelGGL((qmv_rs_dense_kernel<FMT, MR_, R_, CPW_, UPW, 0>), L.grid, block, p.lds, stream, L.dense); \
    else if (L.entry == RS_MULTI)                                                                                  \
      hipLaunchKernelGGL((qmv_rs_multi_kernel<FMT, MR_, R_, CPW_, UPW>), L.grid, block, p.lds, stream, L.multi);   \
    else                                                                                                           \
      hipLaunchKernelGGL((qmv_rs_kernel<FMT, MR_, R_, CPW_, UPW>), L.grid, block, p.lds, stream, *L.a, L.gs_shift, \
                         *L.mp);                                                                                   \
    return hipGetLastError();                                                                                      \
  }
  RS_CASE(1, 4, 1)
  RS_CASE(1, 8, 1)
  RS_CASE(1, 16, 1)
  RS_CASE(2, 4, 1)
  RS_CASE(2, 8, 1)
  RS_CASE(4, 4, 1)
  RS_CASE(4, 8, 1)
  RS_CASE(1, 4, 2)
  RS_CASE(1, 8, 2)
  RS_CASE(2, 4, 2)
  RS_CASE(2, 8, 2)
  RS_CASE(4, 4, 2)
#undef RS_CASE
  return hipErrorInvalidValue;
}

// scale groups per load: the widest load every row's scales stay aligned for
int rs_upw(int fmt, int64_t G) {
  (void)fmt;
  return (G & 3) ? ((G & 1) ? 1 : 2) : 4;
}

template <int FMT>
hipError_t rs_launch_fmt(const QmvRsPlan& p, const RsLaunch& L, int K, hipStream_t stream) {
  const int upw = rs_upw(FMT, (int64_t)K >> L.gs_shift);
  if (upw == 1) return rs_launch_upw<FMT, 1>(p, L, stream);
  if (upw == 4) return rs_launch_upw<FMT, 4>(p, L, stream);
  return rs_launch_upw<FMT, 2>(p, L, stream);
}

bool rs_valid(int mr, int r, int cpw) {
  if (cpw == 1) return (mr == 1 && (r == 4 || r == 8 || r == 16)) || ((mr == 2 || mr == 4) && (r == 4 || r == 8));
  if (cpw == 2) return ((mr == 1 || mr == 2) && (r == 4 || r == 8)) || (mr == 4 && r == 4);
  return false;
}

}  // namespace

QmvRsPlan qmv_rs_plan(int fmt, int gs, int64_t N, int64_t K, int rows, int r_req) {
  QmvRsPlan p;
  const int kl = fmt == AFF8 ? 16 : 32;
  const int64_t nlc = K / kl;
  const int64_t chunks = (nlc + 63) / 64;
  p.mr = rows <= 1 ? 1 : (rows <= 2 ? 2 : 4);
  if (rows > 4 || rows < 1) return p;
  // at most 8 waves of up to 256 registers (two per SIMD)
  p.cpw = chunks <= 8 ? 1 : 2;
  if (chunks > 16) return p;
  p.nw = (int)((chunks + p.cpw - 1) / p.cpw);
  p.r = 8;
  if (p.cpw == 2 && p.mr == 4) p.r = 4;
  // 4-bit matrices up to 16 MB (q/o/k/v projections, MoE experts) at 1-2
  // rows: 4 rows per workgroup, twice the workgroups (MI355X: 4096 x 4096
  // 5.26 -> 4.77 us, 1024 x 4096 4.09 -> 3.80, gpt-oss expert down 7.2 -> 6.6;
  // larger matrices and 8-bit codes are as fast or faster at 8)
  if (fmt != AFF8 && p.mr <= 2 && N * K / 2 <= ((int64_t)16 << 20)) p.r = 4;
  // long 4-bit rows at one activation row (Llama-3-8B down, K = 14336: 7
  // waves per workgroup): 16 rows per workgroup (MI355X: 8.70 -> 8.36 us)
  else if (fmt != AFF8 && p.mr == 1 && p.cpw == 1 && p.nw >= 6) p.r = 16;
  if (r_req > 0 && rs_valid(p.mr, r_req, p.cpw)) p.r = r_req;
  p.tiles = (int)((N + p.r - 1) / p.r);
  p.lds = qmv_rs_lds(fmt, p.r, p.mr, p.nw, p.cpw, gs);
  // every scale load of a wave is issued before its weights: at most 4 per lane
  const int64_t G = K / gs;
  const int upw = rs_upw(fmt, G);
  const int gc = 64 * kl / gs;
  const int units = p.cpw * p.r * gc / upw;
  // buffer offsets are 32-bit and 0x80000000 marks a dead lane: every operand
  // of one launch must stay below 2 GiB
  const int64_t wbytes = N * (K / kl) * 16, sbytes = N * G * 2;
  p.ok = rs_valid(p.mr, p.r, p.cpw) && K % kl == 0 && K % gs == 0 && p.lds <= kQmvLdsMax && units <= 4 * 64 &&
         wbytes + (int64_t)p.r * (K / kl) * 16 < ((int64_t)1 << 31) && sbytes < ((int64_t)1 << 31) &&
         (int64_t)4 * K * 2 < ((int64_t)1 << 31);
  return p;
}

hipError_t qmv_rs_launch(int fmt, int gs, const QmvArgs& a, int nseg, const QmvRsPlan& p, hipStream_t stream,
                         const QmvMulti* multi) {
  if (!p.ok) return hipErrorInvalidValue;
  RsLaunch L{};
  L.a = &a;
  L.gs_shift = log2i(gs);
  QmvMulti none{};
  L.mp = &none;
  int tiles = p.tiles;
  if (multi && multi->n > 1) {
    // several 2-D matrices of one activation block (segment 0)
    tiles = multi->tile_end[multi->n - 1];
    L.entry = RS_MULTI;
    RsMultiArgs& m = L.multi;
    m.x = a.x;
    m.K = a.K;
    m.count = std::min(a.rps, a.total_rows);
    m.gs_shift = L.gs_shift;
    m.n = multi->n;
    for (int i = 0; i < kQmvMultiMax; i++) {
      const int j = i < multi->n ? i : multi->n - 1;  // unused entries repeat the last one
      m.tile_end[i] = multi->tile_end[j];
      m.N[i] = multi->N[j];
      m.w[i] = multi->w[j];
      m.scales[i] = multi->scales[j];
      m.biases[i] = multi->biases[j];
      m.out[i] = multi->out[j];
    }
    nseg = 1;
  } else if (nseg == 1 && !a.rhs && !a.lhs && !a.runs && a.w_expert_stride == 0) {
    L.entry = RS_DENSE;
    RsDenseArgs& d = L.dense;
    d.x = a.x;
    d.w = a.w;
    d.scales = a.scales;
    d.biases = a.biases;
    d.out = a.out;
    d.N = a.N;
    d.K = a.K;
    d.count = std::min(a.rps, a.total_rows);
    d.gs_shift = L.gs_shift;
  } else {
    L.entry = RS_GENERAL;
  }
  L.xt = a.xt;
  if (a.xt != 0 && L.entry != RS_DENSE) return hipErrorInvalidValue;  // float16: dense entry only
  L.grid = dim3((unsigned)tiles, (unsigned)nseg, 1);
  switch (fmt) {
    case AFF4: return rs_launch_fmt<AFF4>(p, L, a.K, stream);
    case AFF8: return rs_launch_fmt<AFF8>(p, L, a.K, stream);
    default: return rs_launch_fmt<MXFP4>(p, L, a.K, stream);
  }
}

}  // namespace mlxq
