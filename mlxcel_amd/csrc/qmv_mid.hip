// qmv_mid.hip — decode kernel for 5 to 16 activation rows per weight matrix
// (affine 4/8-bit, bfloat16 or float16) on gfx950.
//
// Same product as the other decode kernels (reference decode route: overlays/
// rocm/mlx/backend/rocm/quantized/qmv_tiled_kernel.hip:29-128; CPU math
// overlays/cpu/mlx/backend/cpu/quantized.cpp:199-257): y[m,n] = sum_g s[n,g] *
// sum_{k in g} x[m,k] q[n,k] + b[n,g] * sum_{k in g} x[m,k], fp32
// accumulation, one rounding to the result type on store.
//
// Why a kernel of its own: at 16 activation rows the activations weigh 32
// bytes per k against 8 bytes per k for 16 rows of 4-bit codes, so a kernel
// that reloads them for every 16 weight rows moves several times more
// activation bytes (L2 -> CU) than weight bytes (HBM -> CU).  Here a
// workgroup owns 128 weight rows and one K range: it stages that range of the
// activations, their group sums and the rows' scales in LDS once, and its
// four waves (two 16-row tiles each) stream the weights past them.
//
// Products: v_mfma_f32_16x16x32_bf16 with the weights as the B operand (lane i
// holds weight row i % 16, 16-byte code chunk i / 16 of a 4-chunk window) and
// the activations as A.  A window holds S quantization groups (S = window /
// group size, at least 1); A row r carries activation row r / S restricted to
// the chunks of group r % S and zeros elsewhere, so an MFMA never mixes groups
// and the fold y += s * D + (b - 128 s) * sum(x) (AFF4 "128 + q" codes; AFF8
// codes are the bytes themselves, so b) runs once per output, window and
// group.  The activations are staged permuted to the AFF4 pair order
// ([x0,x4,x1,x5,x2,x6,x3,x7] per 8) so the codes widen with one byte permute
// per pair.
//
// Each workgroup covers a K range of 8 windows (1024 k for 4-bit, 512 for
// 8-bit; 4 windows on request); every wave keeps 4 windows of weight loads
// in flight per tile.  K ranges
// of one row block write fp32 partials that a second kernel adds in a fixed
// order (bitwise reproducible).  (A last-workgroup-adds-them variant needs a
// device-scope release/acquire per workgroup, which on MI355X writes back and
// invalidates the XCD's L2: it measured ~50 us per launch.)
#include "common.hpp"
#include "kernels.hpp"

namespace mlxq {

namespace {

constexpr int MID_NW = 4;                      // waves per workgroup
constexpr int MID_T = 2;                       // 16-row tiles per wave
constexpr int MID_ROWS = MID_NW * MID_T * 16;  // weight rows per workgroup
constexpr int MID_WIN = 8;                     // windows per workgroup (4 on request)
constexpr int MID_P = 4;                       // windows of weight loads in flight per tile
constexpr int MID_NT = 64 * MID_NW;            // threads per workgroup

// Sum over aligned groups of PG (4, 8 or 16) lanes: quad swaps, then the
// half-row and row mirrors, which pair the partial sums of adjacent groups.
template <int PG>
__device__ __forceinline__ float group_sum(float v) {
  v += dpp<0xB1>(v);  // quad_perm [1,0,3,2]
  v += dpp<0x4E>(v);  // quad_perm [2,3,0,1]
  if constexpr (PG >= 8) v += dpp<0x141>(v);   // row_half_mirror
  if constexpr (PG >= 16) v += dpp<0x140>(v);  // row_mirror
  return v;
}

// [x0..x7] (bf16, 4 words) -> [x0,x4,x1,x5,x2,x6,x3,x7]
__device__ __forceinline__ u32x4 perm_aff4_mid(u32x4 x) {
  return u32x4{__builtin_amdgcn_perm(x[2], x[0], 0x05040100u), __builtin_amdgcn_perm(x[2], x[0], 0x07060302u),
               __builtin_amdgcn_perm(x[3], x[1], 0x05040100u), __builtin_amdgcn_perm(x[3], x[1], 0x07060302u)};
}

}  // namespace

__host__ __device__ inline QmvMidLds qmv_mid_lds(int fmt, int gs, int kr, int na) {
  const int kw = fmt == AFF8 ? 64 : 128;
  QmvMidLds l;
  l.xpitch = kr + 8;  // bf16 per staged activation row (16 bytes of padding shift rows across banks)
  l.xl = 0;
  l.xs = l.xl + 16u * (uint32_t)l.xpitch * 2u;
  l.sc = l.xs + (uint32_t)(kr / kw) * 16u * (uint32_t)na * 4u;
  // scale rows are (kr / gs + 2) pairs apart: the 16 rows a tile's lanes read
  // at once then fall on distinct LDS banks
  l.zero = l.sc + (uint32_t)MID_ROWS * (uint32_t)(kr / gs + 2) * 8u;
  l.total = l.zero + 16u;
  return l;
}

// FMT: AFF4 or AFF8; S: quantization groups per window; NA: 16-row A tiles
// (1 or 2, 16 NA >= rows * S); SW: scale groups per staging load (8 or 2).
// One A tile fits two waves per SIMD without spilling (the register bound
// below makes the allocator pack the accumulators); more A tiles keep their
// own allocation.
// XT: 16-bit type of activations, scales, biases and result (0 bfloat16, 1
// float16: codes widen to float16 1024 + q, products on the float16 MFMA).
// W: windows per workgroup (8, or 4).
template <int FMT, int S, int NA, int SW, int XT, int W>
__global__ __launch_bounds__(MID_NT, NA == 1 ? 2 : 1) void qmv_mid_kernel(const QmvMidArgs a) {
  constexpr int CK = FMT == AFF8 ? 16 : 32;  // k per 16-byte code chunk
  constexpr int KW = 4 * CK;                 // k per window (4 chunks)
  constexpr int NQ = CK / 8;                 // MFMAs per window, tile and A tile
  constexpr int XG = KW / S;                 // k per group slot of a window
  constexpr int YV = 4 / S;                  // activation rows per lane and A tile after the fold
  constexpr int KR = W * KW;                 // k per workgroup
  constexpr int XPMAX = 16 * KR / 8 / MID_NT;  // activation pieces per thread, upper bound
  constexpr int SPMAX = SW == 8 ? 2 : 4;     // scale loads per thread and operand, upper bound (checked on the host)

  extern __shared__ __align__(16) unsigned char smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const QmvMat mat = pick_matrix(a.mt, a.w, a.scales, a.biases, a.out, a.N, blockIdx.x);
  const int M = a.M;
  const int N = mat.N;
  const int K = a.K;
  constexpr int kr = KR;
  const int rb = mat.blk;
  const int sp = blockIdx.y;
  const int k0 = sp * kr;
  constexpr int nwin = W;  // every split is a full K range (K % KR == 0)
  const int G = K >> a.gs_shift;
  const int ngr = kr >> a.gs_shift;  // groups per K range
  const int spitch = ngr + 2;        // scale pairs per staged row
  const int row_wg = rb * MID_ROWS;
  const QmvMidLds L = qmv_mid_lds(FMT, 1 << a.gs_shift, kr, NA);

  const uint32_t RB = (uint32_t)(K / CK) * 16u;  // bytes per weight row
  const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(mat.w, (uint32_t)N * RB);
  const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(a.x, (uint32_t)M * (uint32_t)K * 2u);
  const __amdgpu_buffer_rsrc_t sr = buffer_rsrc(mat.scales, (uint32_t)N * (uint32_t)G * 2u);
  const __amdgpu_buffer_rsrc_t br = buffer_rsrc(mat.biases, (uint32_t)N * (uint32_t)G * 2u);

  // ---- 1. loads: activation range, the block's scales, then the first
  // windows of weights (the staged data is consumed first; loads retire in
  // order) ---------------------------------------------------------------------
  const int xpieces = M * (kr / 8);
  u32x4 xpre[XPMAX];
#pragma unroll
  for (int i = 0; i < XPMAX; i++) {
    const int p = tid + i * MID_NT;
    const int m = p / (kr / 8), c = p % (kr / 8);
    const uint32_t o = p < xpieces ? (uint32_t)(m * K + k0 + 8 * c) * 2u : kDeadOfs;
    xpre[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, o, 0, 0));
  }
  const int sunits = MID_ROWS * ngr / SW;  // per operand
  u32x4 spre[SPMAX], bpre[SPMAX];
#pragma unroll
  for (int i = 0; i < SPMAX; i++) {
    const int u = tid + i * MID_NT;
    const int r = u / (ngr / SW), gl = (u % (ngr / SW)) * SW;
    const int n = row_wg + r;
    const uint32_t o = (u < sunits && n < N) ? (uint32_t)(n * G + (k0 >> a.gs_shift) + gl) * 2u : kDeadOfs;
    if constexpr (SW == 8) {
      spre[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(sr, o, 0, 0));
      bpre[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(br, o, 0, 0));
    } else {
      spre[i] = u32x4{__builtin_amdgcn_raw_buffer_load_b32(sr, o, 0, 0), 0u, 0u, 0u};
      bpre[i] = u32x4{__builtin_amdgcn_raw_buffer_load_b32(br, o, 0, 0), 0u, 0u, 0u};
    }
  }

  // weight tiles of this wave: rows row_wg + wave*32 + t*16 + (lane & 15);
  // lane's chunk in a window: lane >> 4
  const int nl = lane & 15;
  const int g = lane >> 4;
  uint32_t woff[MID_T];
#pragma unroll
  for (int t = 0; t < MID_T; t++) {
    const int n = row_wg + wave * (MID_T * 16) + t * 16 + nl;
    woff[t] = n < N ? (uint32_t)n * RB + (uint32_t)(k0 / CK + g) * 16u : kDeadOfs;
  }
  u32x4 wbuf[MID_P][MID_T];
#pragma unroll
  for (int p = 0; p < MID_P; p++)
#pragma unroll
    for (int t = 0; t < MID_T; t++)
      wbuf[p][t] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, woff[t] == kDeadOfs ? kDeadOfs : woff[t] + p * 64u, 0,
                                                       0 /* default cache policy: faster than nt */));
  __builtin_amdgcn_sched_barrier(0);

  // ---- 2. stage activations (AFF4 pair order), scales, a zero piece ---------
  // Group sums come from the staging registers: a wave's 64 lanes hold 64
  // consecutive 8-value pieces of one activation row, and the XG / 8 pieces
  // of one (window, slot) are adjacent lanes.
  uint16_t* xl = reinterpret_cast<uint16_t*>(smem + L.xl);
  float* xsl = reinterpret_cast<float*>(smem + L.xs);
  constexpr int PG = XG / 8;  // pieces per group slot (4, 8 or 16)
#pragma unroll
  for (int i = 0; i < XPMAX; i++) {
    const int p = tid + i * MID_NT;
    const int m = p / (kr / 8), c = p % (kr / 8);
    if (p < xpieces) {
      const u32x4 v = FMT == AFF4 ? perm_aff4_mid(xpre[i]) : xpre[i];
      *reinterpret_cast<u32x4*>(xl + m * L.xpitch + 8 * c) = v;
    }
    float sum = 0.f;
    constexpr uint32_t ONES = XT ? 0x3C003C00u : 0x3F803F80u;
#pragma unroll
    for (int e = 0; e < 4; e++) sum = dotx<XT>(xpre[i][e], ONES, sum);  // pairs times (1, 1); dead pieces are 0
    sum = group_sum<PG>(sum);
    const int w = (8 * c) / KW, slot = ((8 * c) % KW) / XG;
    const int r = m * S + slot;
    if ((lane & (PG - 1)) == 0 && r < 16 * NA) xsl[w * 16 * NA + r] = sum;
  }
  float2* sl = reinterpret_cast<float2*>(smem + L.sc);
#pragma unroll
  for (int i = 0; i < SPMAX; i++) {
    const int u = tid + i * MID_NT;
    if (u < sunits) {
      const int r = u / (ngr / SW), gl = (u % (ngr / SW)) * SW;
#pragma unroll
      for (int h = 0; h < SW; h++) {
        const uint32_t sb = (spre[i][h >> 1] >> (16 * (h & 1))) & 0xFFFFu;
        const uint32_t bb = (bpre[i][h >> 1] >> (16 * (h & 1))) & 0xFFFFu;
        const float s = xt_to_f32<XT>(sb), b = xt_to_f32<XT>(bb);
        // the codes' offset (bfloat16 4-bit 128, float16 1024) times sum(x)
        // comes off with the bias
        constexpr float OFS = XT ? 1024.0f : (FMT == AFF4 ? 128.0f : 0.0f);
        sl[r * spitch + gl + h] = float2{s, OFS != 0.0f ? __builtin_fmaf(-OFS, s, b) : b};
      }
    }
  }
  if (tid == 0) *reinterpret_cast<u32x4*>(smem + L.zero) = u32x4{0u, 0u, 0u, 0u};
  __syncthreads();

  // ---- 3. windows: A from LDS, B from the weight ring, fold per group -------
  // A operand of lane (row r = lane & 15, chunk g) for A tile a: activation
  // row (16a + r) / S if chunk g belongs to slot (16a + r) % S, else the zero
  // piece.  Addresses advance by wstep per window and qstep per MFMA.
  const int slot_g = (g * CK) / XG;  // slot of this lane's chunk
  uint32_t abase[NA], wstep[NA], qstep[NA];
#pragma unroll
  for (int t = 0; t < NA; t++) {
    const int r = 16 * t + nl;
    const int m = r / S, slot = r % S;
    const bool live = m < M && slot == slot_g;
    abase[t] = live ? L.xl + (uint32_t)(m * L.xpitch + g * CK) * 2u : L.zero;
    wstep[t] = live ? KW * 2u : 0u;
    qstep[t] = live ? 16u : 0u;
  }
  // fold rows of this lane: D row 4 * g + i of A tile a is activation row
  // (16a + 4g + i) / S, slot (16a + 4g + i) % S
  float y[MID_T][NA][YV];
#pragma unroll
  for (int t = 0; t < MID_T; t++)
#pragma unroll
    for (int u = 0; u < NA; u++)
#pragma unroll
      for (int j = 0; j < YV; j++) y[t][u][j] = 0.f;

  const uint32_t srow0 = L.sc + (uint32_t)((wave * MID_T * 16 + nl) * spitch) * 8u;  // this lane's row, tile 0
  const int gsh = a.gs_shift;

  {
#pragma unroll
    for (int w = 0; w < W; w++) {
      u32x4 A[NA][NQ];
#pragma unroll
      for (int t = 0; t < NA; t++)
#pragma unroll
        for (int q = 0; q < NQ; q++)
          A[t][q] = *reinterpret_cast<const u32x4*>(smem + abase[t] + (uint32_t)w * wstep[t] + (uint32_t)q * qstep[t]);
      f32x4 xsv[NA];
#pragma unroll
      for (int t = 0; t < NA; t++) xsv[t] = *reinterpret_cast<const f32x4*>(xsl + w * 16 * NA + 16 * t + 4 * g);
      // first group of this window (groups of one window are consecutive)
      const int grp0 = (w * KW) >> gsh;
#pragma unroll
      for (int t = 0; t < MID_T; t++) {
        // ring slot w % MID_P: take window w, refill it with window w + MID_P
        const u32x4 wv = wbuf[w % MID_P][t];
        if (w + MID_P < W)
          wbuf[w % MID_P][t] = __builtin_bit_cast(
              u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                         wr, woff[t] == kDeadOfs ? kDeadOfs : woff[t] + (uint32_t)(w + MID_P) * 64u, 0, 0));
        u32x4 B[NQ];
        if constexpr (FMT == AFF4) {
#pragma unroll
          for (int q = 0; q < NQ; q++) {
            uint32_t pr[4];
            unpack_aff4(wv[q], pr, XT ? 0x64646464u : 0x43434343u);
            B[q] = u32x4{pr[0], pr[1], pr[2], pr[3]};
          }
        } else if constexpr (XT == 1) {
          // byte pairs (b0, b1), (b2, b3) of each word as float16 1024 + q
#pragma unroll
          for (int q = 0; q < 2; q++)
            B[q] = u32x4{__builtin_amdgcn_perm(0x64646464u, wv[2 * q], 0x04010400u),
                         __builtin_amdgcn_perm(0x64646464u, wv[2 * q], 0x04030402u),
                         __builtin_amdgcn_perm(0x64646464u, wv[2 * q + 1], 0x04010400u),
                         __builtin_amdgcn_perm(0x64646464u, wv[2 * q + 1], 0x04030402u)};
        } else {
          uint32_t pr[4];
          unpack_aff8(wv[0], wv[1], pr);
          B[0] = u32x4{pr[0], pr[1], pr[2], pr[3]};
          unpack_aff8(wv[2], wv[3], pr);
          B[1] = u32x4{pr[0], pr[1], pr[2], pr[3]};
        }
        // scale pairs (s, b') of this lane's weight row for the window's slots
        float2 sc[S];
        const unsigned char* sp0 = smem + srow0 + (uint32_t)((t * 16 * spitch + grp0) * 8);
#pragma unroll
        for (int h = 0; h < S; h++) sc[h] = reinterpret_cast<const float2*>(sp0)[h];
#pragma unroll
        for (int u = 0; u < NA; u++) {
          f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int q = 0; q < NQ; q++) d = mfma16x16x32_xt<XT>(A[u][q], B[q], d);
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const int slot = (4 * g + i) % S;  // 16u is a multiple of S
            y[t][u][i / S] = __builtin_fmaf(sc[slot].x, d[i], __builtin_fmaf(sc[slot].y, xsv[u][i], y[t][u][i / S]));
          }
        }
      }
      // one window at a time: hoisting the operand reads of later windows
      // costs more registers than the overlap gains
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // ---- 4. store: bf16 (one K range) or this range's fp32 partials ----------
  const int ntot = a.mt.n > 1 ? a.mt.ntot : N;  // partials' row length
#pragma unroll
  for (int t = 0; t < MID_T; t++) {
    const int n = row_wg + wave * (MID_T * 16) + t * 16 + nl;
#pragma unroll
    for (int u = 0; u < NA; u++)
#pragma unroll
      for (int j = 0; j < YV; j++) {
        const int m = (16 * u + 4 * g) / S + j;
        if (m < M && n < N) {
          if (a.ks == 1) mat.out[(int64_t)m * N + n] = (uint16_t)f32_to_xt<XT>(y[t][u][j]);
          else a.ws[((int64_t)sp * M + m) * ntot + mat.noff + n] = y[t][u][j];
        }
      }
  }
}

// ---- host ------------------------------------------------------------------

namespace {

template <int FMT, int S, int NA, int XT, int W>
hipError_t mid_launch_w(const QmvMidPlan& p, const QmvMidArgs& a, hipStream_t stream) {
  const dim3 grid((unsigned)p.row_blocks, (unsigned)p.ks, 1);
  if (p.sw == 8) hipLaunchKernelGGL((qmv_mid_kernel<FMT, S, NA, 8, XT, W>), grid, dim3(MID_NT), p.lds, stream, a);
  else hipLaunchKernelGGL((qmv_mid_kernel<FMT, S, NA, 2, XT, W>), grid, dim3(MID_NT), p.lds, stream, a);
  return hipGetLastError();
}

template <int FMT, int S, int NA, int XT>
hipError_t mid_launch_xt(const QmvMidPlan& p, const QmvMidArgs& a, hipStream_t stream) {
  constexpr int kw = FMT == AFF8 ? 64 : 128;
  return p.kr == 4 * kw ? mid_launch_w<FMT, S, NA, XT, 4>(p, a, stream) : mid_launch_w<FMT, S, NA, XT, 8>(p, a, stream);
}

template <int FMT, int S, int NA>
hipError_t mid_launch_sna(const QmvMidPlan& p, const QmvMidArgs& a, hipStream_t stream) {
  return a.xt ? mid_launch_xt<FMT, S, NA, 1>(p, a, stream) : mid_launch_xt<FMT, S, NA, 0>(p, a, stream);
}

template <int FMT, int S>
hipError_t mid_launch_s(const QmvMidPlan& p, const QmvMidArgs& a, hipStream_t stream) {
  switch (p.na) {
    case 1: return mid_launch_sna<FMT, S, 1>(p, a, stream);
    case 2: return mid_launch_sna<FMT, S, 2>(p, a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

QmvMidPlan qmv_mid_plan(int fmt, int gs, int64_t N, int64_t K, int rows, int cus, int win_req) {
  QmvMidPlan p;
  if (fmt != AFF4 && fmt != AFF8) return p;
  if (rows < 1 || rows > 16 || (gs != 32 && gs != 64 && gs != 128) || N < 1 || K < 1) return p;
  const int kw = fmt == AFF8 ? 64 : 128;
  p.s = kw / gs > 1 ? kw / gs : 1;
  const int ar = rows * p.s;
  // more than two A tiles (4-bit g32 above 8 rows) would spill: other kernels
  p.na = ar <= 16 ? 1 : 2;
  if (ar > 32) return p;
  p.row_blocks = (int)((N + MID_ROWS - 1) / MID_ROWS);
  p.kr = MID_WIN * kw;  // K per workgroup (a multiple of every group size)
  if (K % p.kr != 0) return p;
  // Half the K range on request only.  MI355X, Qwen3-8B shapes, 4-bit g64,
  // 16 rows (kernel + reduction): o 4096 x 4096 10.3 -> 9.4 us (256
  // workgroups instead of 128), down 4096 x 12288 17.0 -> 16.1, but q/k/v in
  // one launch 11.4 -> 13.0 (384 instead of 192); a q/k/v launch must give
  // the bits of its single calls, and q has o's shape, so one rule for both.
  (void)cus;
  if (win_req == 4) p.kr = 4 * kw;
  p.ks = (int)(K / p.kr);
  const int64_t G = K / gs;
  const int ngr = p.kr / gs;
  p.sw = (G % 8 == 0 && ngr % 8 == 0) ? 8 : ((G % 2 == 0 && ngr % 2 == 0) ? 2 : 0);
  if (!p.sw) return p;
  // staging loads per thread stay within the kernel's register arrays
  if ((MID_ROWS * ngr / p.sw + MID_NT - 1) / MID_NT > (p.sw == 8 ? 2 : 4)) return p;
  p.lds = qmv_mid_lds(fmt, gs, p.kr, p.na).total;
  // buffer offsets are 32-bit and 0x80000000 marks a dead lane
  const int64_t wbytes = N * K * (fmt == AFF8 ? 8 : 4) / 8;
  p.ok = p.lds <= 80 * 1024 && wbytes < ((int64_t)1 << 31) && N * G * 2 < ((int64_t)1 << 31) &&
         (int64_t)rows * K * 2 < ((int64_t)1 << 31) && p.ks <= 65535 && p.row_blocks <= 65535;
  return p;
}

hipError_t qmv_mid_launch(int fmt, const QmvMidArgs& a, const QmvMidPlan& p, hipStream_t stream) {
  if (!p.ok || (p.ks > 1 && !a.ws)) return hipErrorInvalidValue;
  hipError_t e;
  if (fmt == AFF4) {
    switch (p.s) {
      case 1: e = mid_launch_s<AFF4, 1>(p, a, stream); break;
      case 2: e = mid_launch_s<AFF4, 2>(p, a, stream); break;
      default: e = mid_launch_s<AFF4, 4>(p, a, stream); break;
    }
  } else {
    e = p.s == 2 ? mid_launch_s<AFF8, 2>(p, a, stream) : mid_launch_s<AFF8, 1>(p, a, stream);
  }
  if (e != hipSuccess || p.ks == 1) return e;
  QmvMatTable t = a.mt;
  if (t.n <= 1) {
    t.n = 1;
    t.ntot = a.N;
    t.N[0] = a.N;
    t.noff[0] = 0;
    t.out[0] = a.out;
  }
  return launch_splitk_reduce_multi(a.ws, t, a.M, p.ks, stream, a.xt, a.red_vec);
}

}  // namespace mlxq
