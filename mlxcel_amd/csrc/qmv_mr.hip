// qmv_mr.hip — decode kernel for 3 to 16 activation rows per weight matrix
// (affine 4/8-bit, bfloat16 or float16) on gfx950 for matrices with many rows: each
// wave owns 16 weight rows over the whole of K, so every output is finished
// in one launch.
//
// Same product and arithmetic as qmv_mid.hip (reference decode route:
// overlays/rocm/mlx/backend/rocm/quantized/qmv_tiled_kernel.hip:29-128; CPU
// math overlays/cpu/mlx/backend/cpu/quantized.cpp:199-257):
// v_mfma_f32_16x16x32_bf16 with the weights as the B operand straight from
// registers (lane i: weight row i % 16, 16-byte code chunk i / 16 of a
// 4-chunk window), the activations from LDS as A (A row r = activation row
// r / S restricted to group slot r % S, zeros elsewhere), and the fold
// y += s * D + (b - 128 s) * sum(x) once per output, window and group.
//
// Layout of the work.  A workgroup owns 64 weight rows (four waves, one
// 16-row tile each) and walks K in ranges of 8 windows (1024 positions for
// 4-bit codes, 512 for 8-bit).  The four waves share one staged copy of each
// range's activations, group sums and the 64 rows' scales, double-buffered in
// LDS: while the waves multiply range r, the next range's activations and
// scales are already in registers and a ring of weight loads runs 4-16
// windows ahead (8 by default: deeper rings measured slower, their
// registers cost more than they hide); one barrier per range.  Ranges go two per loop turn so
// every LDS and ring index is a compile-time constant (an odd last turn
// multiplies zeros), and the loads of a range differ only in scalar offsets
// and a scalar choice between a live and an empty buffer resource.  Used when the matrix has enough rows for
// ~one workgroup per CU (Llama-3-8B gate/up: 14336 rows -> 224); a
// matrix with fewer rows needs K split across workgroups (qmv_mid.hip).
#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"

namespace mlxq {

namespace {

constexpr int MR_NW = 4;           // waves per workgroup = 16-row tiles
constexpr int MR_NT = 64 * MR_NW;  // threads per workgroup
constexpr int MR_RW = 16 * MR_NW;  // weight rows per workgroup
constexpr int MR_WIN = 8;          // windows per staged range

// Sum over aligned groups of PG (4, 8 or 16) lanes
template <int PG>
__device__ __forceinline__ float mr_group_sum(float v) {
  v += dpp<0xB1>(v);  // quad_perm [1,0,3,2]
  v += dpp<0x4E>(v);  // quad_perm [2,3,0,1]
  if constexpr (PG >= 8) v += dpp<0x141>(v);   // row_half_mirror
  if constexpr (PG >= 16) v += dpp<0x140>(v);  // row_mirror
  return v;
}

}  // namespace

// LDS of one buffer (byte offsets): activations [XR + 1 rows][RK + 8] bf16
// (row XR stays zero: the A operand of lanes without an activation row),
// group sums [8 windows][16 NA] float, scale pairs [64 rows][RK / GSMIN + 2]
// float2 (GSMIN = the smallest group size of the variant).  Two buffers.
__host__ __device__ constexpr uint32_t mr_buf_bytes(int rk, int xr, int na, int gsmin, uint32_t* xs_off = nullptr,
                                                    uint32_t* sc_off = nullptr) {
  const uint32_t xs = (uint32_t)(xr + 1) * (uint32_t)(rk + 8) * 2u;
  const uint32_t sc = xs + (uint32_t)MR_WIN * 16u * (uint32_t)na * 4u;
  const uint32_t end = sc + (uint32_t)MR_RW * (uint32_t)(rk / gsmin + 2) * 8u;
  if (xs_off) *xs_off = xs;
  if (sc_off) *sc_off = sc;
  return (end + 15u) & ~15u;
}

// FMT: AFF4 / AFF8; S: groups per window; NA: 16-row A tiles; XR: activation
// rows staged (8 or 16, at least M); RING: windows of weight loads in flight;
// XT: 16-bit type of activations, scales, biases and result (0 bfloat16, 1
// float16: codes widen to float16 1024 + q for both widths, and the products
// run on v_mfma_f32_16x16x32_f16).
template <int FMT, int S, int NA, int XR, int RING, int XT>
__global__ __launch_bounds__(MR_NT, 1) void qmv_mr_kernel(const QmvMrArgs a) {
  constexpr int CK = FMT == AFF8 ? 16 : 32;  // k per 16-byte code chunk
  constexpr int KW = 4 * CK;                 // k per window
  constexpr int NQ = CK / 8;                 // MFMAs per window and A tile
  constexpr int XG = KW / S;                 // k per group slot
  constexpr int PG = XG / 8;                 // 8-value pieces per group slot
  constexpr int YV = 4 / S;                  // activation rows per lane and A tile after the fold
  constexpr int RK = MR_WIN * KW;            // k per staged range
  constexpr int XP = RK + 8;                 // bf16 per staged row (16 bytes of padding)
  constexpr int PCS = RK / 8;                // 8-value pieces per row and range
  constexpr int XL = XR * PCS / MR_NT;       // activation loads per thread and range
  constexpr int GSMIN = KW / S;              // smallest group size of this variant
  constexpr int SPITCH = RK / GSMIN + 2;     // scale pairs per staged row
  constexpr uint32_t XSO = (uint32_t)(XR + 1) * XP * 2u;
  constexpr uint32_t SCO = XSO + (uint32_t)MR_WIN * 16u * NA * 4u;
  constexpr uint32_t BUF = mr_buf_bytes(RK, XR, NA, GSMIN);
  constexpr uint32_t ZROW = (uint32_t)XR * XP * 2u;  // the zero row of a buffer
  constexpr int SL = (MR_RW * (RK / GSMIN) / 4 + MR_NT - 1) / MR_NT;  // scale loads per thread, upper bound
  static_assert(XL * MR_NT == XR * PCS, "activation pieces split evenly over the threads");
  static_assert(PCS % 64 == 0, "a wave's pieces lie in one row");
  static_assert(PCS % PG == 0 && PG <= 16, "group slots stay inside a row of 16 lanes");
  static_assert((XP * 2) % 16 == 0, "the zero row is whole 16-byte pieces");

  extern __shared__ __align__(16) unsigned char smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const QmvMat mat = pick_matrix(a.mt, a.w, a.scales, a.biases, a.out, a.N, blockIdx.x);
  const int M = a.M, N = mat.N, K = a.K;
  const int gsh = a.gs_shift;
  const int G = K >> gsh;
  const int ngr = RK >> gsh;  // groups per range
  const int row_wg = mat.blk * MR_RW;
  const int nranges = K / RK;

  const uint32_t RB = (uint32_t)(K / CK) * 16u;  // bytes per weight row
  // live resources and dead ones (no records: every load returns 0), chosen
  // per range with scalar selects; range offsets go in the scalar offset
  const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(mat.w, (uint32_t)N * RB);
  const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(a.x, (uint32_t)M * (uint32_t)K * 2u);
  const __amdgpu_buffer_rsrc_t sr = buffer_rsrc(mat.scales, (uint32_t)N * (uint32_t)G * 2u);
  const __amdgpu_buffer_rsrc_t br = buffer_rsrc(mat.biases, (uint32_t)N * (uint32_t)G * 2u);
  const __amdgpu_buffer_rsrc_t w0 = buffer_rsrc(mat.w, 0u);
  const __amdgpu_buffer_rsrc_t x0 = buffer_rsrc(a.x, 0u);
  const __amdgpu_buffer_rsrc_t s0 = buffer_rsrc(mat.scales, 0u);
  const __amdgpu_buffer_rsrc_t b0 = buffer_rsrc(mat.biases, 0u);

  // Per-thread load offsets inside a range.  Activation piece i: p = tid +
  // 256 i, row p / PCS, piece p % PCS.  Scale unit i: u = tid + 256 i, row
  // u / (ngr / 4), groups (u % (ngr / 4)) * 4 .. + 3.
  const int sunits = MR_RW * ngr / 4;
  uint32_t xoff[XL], soff[SL];
#pragma unroll
  for (int i = 0; i < XL; i++) {
    const int p = tid + MR_NT * i;
    const int m = p / PCS, c = p % PCS;
    xoff[i] = m < M ? (uint32_t)(m * K + 8 * c) * 2u : kDeadOfs;
  }
#pragma unroll
  for (int i = 0; i < SL; i++) {
    const int u = tid + MR_NT * i;
    const int r = u / (ngr / 4), gl = (u % (ngr / 4)) * 4;
    const int n = row_wg + r;
    soff[i] = (u < sunits && n < N) ? (uint32_t)(n * G + gl) * 2u : kDeadOfs;
  }
  u32x4 xpre[XL];
  u32x2 spre[SL], bpre[SL];
  auto issue_range = [&](int range) {
    const bool live = range < nranges;
    const __amdgpu_buffer_rsrc_t xq = live ? xr : x0;
    const __amdgpu_buffer_rsrc_t sq = live ? sr : s0;
    const __amdgpu_buffer_rsrc_t bq = live ? br : b0;
    const int xs = range * RK * 2, ss = range * ngr * 2;
#pragma unroll
    for (int i = 0; i < XL; i++) xpre[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xq, xoff[i], xs, 0));
#pragma unroll
    for (int i = 0; i < SL; i++) {
      spre[i] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(sq, soff[i], ss, 0));
      bpre[i] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(bq, soff[i], ss, 0));
    }
  };
  // registers -> the LDS buffer at byte offset bofs: activations (AFF4 pair
  // order), group sums, scale pairs
  auto stage_range = [&](uint32_t bofs) {
    uint16_t* xl = reinterpret_cast<uint16_t*>(smem + bofs);
    float* xsl = reinterpret_cast<float*>(smem + bofs + XSO);
    float2* sl = reinterpret_cast<float2*>(smem + bofs + SCO);
#pragma unroll
    for (int i = 0; i < XL; i++) {
      const int p = tid + MR_NT * i;
      const int m = p / PCS, c = p % PCS;
      const u32x4 v = FMT == AFF4 ? perm_aff4_v(xpre[i]) : xpre[i];
      *reinterpret_cast<u32x4*>(xl + m * XP + 8 * c) = v;
      float sum = 0.f;
      constexpr uint32_t ONES = XT ? 0x3C003C00u : 0x3F803F80u;
#pragma unroll
      for (int e = 0; e < 4; e++) sum = dotx<XT>(xpre[i][e], ONES, sum);  // rows past M read 0
      sum = mr_group_sum<PG>(sum);
      const int w = (8 * c) / KW, slot = ((8 * c) % KW) / XG;
      const int r = m * S + slot;
      if ((lane & (PG - 1)) == 0 && r < 16 * NA) xsl[w * 16 * NA + r] = sum;
    }
#pragma unroll
    for (int i = 0; i < SL; i++) {
      const int u = tid + MR_NT * i;
      if (u < sunits) {
        const int r = u / (ngr / 4), gl = (u % (ngr / 4)) * 4;
#pragma unroll
        for (int h = 0; h < 4; h++) {
          const float s = xt_to_f32<XT>((spre[i][h >> 1] >> (16 * (h & 1))) & 0xFFFFu);
          const float b = xt_to_f32<XT>((bpre[i][h >> 1] >> (16 * (h & 1))) & 0xFFFFu);
          // the codes' offset (bfloat16 4-bit 128, float16 1024) times sum(x)
          // comes off with the bias
          constexpr float OFS = XT ? 1024.0f : (FMT == AFF4 ? 128.0f : 0.0f);
          sl[r * SPITCH + gl + h] = float2{s, OFS != 0.0f ? __builtin_fmaf(-OFS, s, b) : b};
        }
      }
    }
  };

  // weights: row row_wg + 16 wave + (lane & 15), chunk lane >> 4 of each
  // window; a ring of RING windows keeps that many windows of loads in flight
  const int nl = lane & 15, g = lane >> 4;
  const int nrow = row_wg + wave * 16 + nl;
  const uint32_t woff = nrow < N ? (uint32_t)nrow * RB + (uint32_t)g * 16u : kDeadOfs;
  auto w_load = [&](int range, int w) {
    const __amdgpu_buffer_rsrc_t wq = range < nranges ? wr : w0;
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wq, woff + (uint32_t)w * 64u,
                                                                           range * (MR_WIN * 64), 0));
  };

  // ---- prologue: range 0 staged, range 1 in registers, RING windows of weights
  static_assert(RING == 4 || RING == 8 || RING == 16, "the ring slots repeat every two ranges");
  issue_range(0);
  u32x4 wbuf[RING];
#pragma unroll
  for (int p = 0; p < RING; p++) wbuf[p] = w_load(p / MR_WIN, p % MR_WIN);
  for (int i = tid; i < 2 * (XP * 2 / 16); i += MR_NT)
    *reinterpret_cast<u32x4*>(smem + (uint32_t)(i / (XP * 2 / 16)) * BUF + ZROW + (uint32_t)(i % (XP * 2 / 16)) * 16u) =
        u32x4{0u, 0u, 0u, 0u};
  stage_range(0u);
  issue_range(1);
  __syncthreads();

  // A operand of lane (row nl, chunk g) for A tile u: activation row
  // (16u + nl) / S if chunk g belongs to slot (16u + nl) % S, else the zero
  // row.  Window, MFMA and buffer add constants to this base.
  const int slot_g = (g * CK) / XG;
  uint32_t abase[NA];
#pragma unroll
  for (int u = 0; u < NA; u++) {
    const int r = 16 * u + nl;
    const int m = r / S, slot = r % S;
    abase[u] = (m < M && slot == slot_g ? (uint32_t)m * XP * 2u : ZROW) + (uint32_t)(g * CK) * 2u;
  }

  float y[NA][YV];
#pragma unroll
  for (int u = 0; u < NA; u++)
#pragma unroll
    for (int j = 0; j < YV; j++) y[u][j] = 0.f;

  const uint32_t srow = SCO + (uint32_t)((wave * 16 + nl) * SPITCH) * 8u;  // this lane's scale row

  // two ranges per turn, so the buffer and ring halves are compile-time; a
  // turn past the last range (odd count) multiplies zeros
  for (int r2 = 0; r2 < nranges; r2 += 2) {
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const int range = r2 + h;
      const uint32_t bofs = (uint32_t)h * BUF;
#pragma unroll
      for (int w = 0; w < MR_WIN; w++) {
        u32x4 A[NA][NQ];
#pragma unroll
        for (int u = 0; u < NA; u++)
#pragma unroll
          for (int q = 0; q < NQ; q++)
            A[u][q] = *reinterpret_cast<const u32x4*>(smem + abase[u] + bofs + (uint32_t)(w * KW * 2 + q * 16));
        f32x4 xsv[NA];
#pragma unroll
        for (int u = 0; u < NA; u++)
          xsv[u] = *reinterpret_cast<const f32x4*>(smem + bofs + XSO + (uint32_t)((w * 16 * NA + 16 * u + 4 * g) * 4));
        // ring slot: take this range's window w, refill it with the window
        // RING windows on
        const int rs = (h * MR_WIN + w) % RING;
        const u32x4 wv = wbuf[rs];
        wbuf[rs] = w_load(range + (w + RING) / MR_WIN, (w + RING) % MR_WIN);
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
        const int grp0 = (w * KW) >> gsh;  // first group of this window inside the range
        float2 sc[S];
        const unsigned char* sp0 = smem + bofs + srow + (uint32_t)(grp0 * 8);
#pragma unroll
        for (int hh = 0; hh < S; hh++) sc[hh] = reinterpret_cast<const float2*>(sp0)[hh];
#pragma unroll
        for (int u = 0; u < NA; u++) {
          f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int q = 0; q < NQ; q++) d = mfma16x16x32_xt<XT>(A[u][q], B[q], d);
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const int slot = (4 * g + i) % S;  // 16u is a multiple of S
            y[u][i / S] = __builtin_fmaf(sc[slot].x, d[i], __builtin_fmaf(sc[slot].y, xsv[u][i], y[u][i / S]));
          }
        }
        // one window at a time: hoisting later windows' operand reads costs
        // more registers than it hides
        __builtin_amdgcn_sched_barrier(0);
      }
      // the next range (in registers) goes to the other buffer, whose last
      // readers finished before the previous barrier; the one after it goes out
      stage_range((uint32_t)(h ^ 1) * BUF);
      issue_range(range + 2);
      __syncthreads();
    }
  }

  // ---- store: each wave's outputs are complete ----------------------------
  if (nrow < N) {
#pragma unroll
    for (int u = 0; u < NA; u++)
#pragma unroll
      for (int j = 0; j < YV; j++) {
        const int m = (16 * u + 4 * g) / S + j;
        if (m < M) mat.out[(int64_t)m * N + nrow] = (uint16_t)f32_to_xt<XT>(y[u][j]);
      }
  }
}

// ---- K split over the waves: matrices with few rows -----------------------
//
// The same staged ranges, operands and fold, but a workgroup owns only 16 T
// weight rows (T 16-row tiles, T = 1-4) and its NW waves split every range's
// 8 windows between them (8 waves: wave v takes window v, for all T tiles);
// at the end the waves add their partial sums through LDS in wave order and
// wave 0 stores the finished outputs.  A matrix of 4096 rows (Qwen3-8B o, q)
// then gives 256 workgroups of 16 rows, each over the whole of K, where the
// split-K kernel (qmv_mid.hip) needs a second launch to add its K ranges: a
// launch there is a memory round trip for the staged activations, the
// windows, and a second round trip for the fp32 partials before the
// reduction launch's own.  Each output's sum runs in the same order whatever
// T, so the multi-projection launch gives the bits of single calls.

__host__ __device__ constexpr uint32_t kq_buf_bytes(int rk, int xr, int na, int gsmin, int rw) {
  const uint32_t xs = (uint32_t)(xr + 1) * (uint32_t)(rk + 8) * 2u;
  const uint32_t sc = xs + (uint32_t)MR_WIN * 16u * (uint32_t)na * 4u;
  const uint32_t end = sc + (uint32_t)rw * (uint32_t)(rk / gsmin + 2) * 8u;
  return (end + 15u) & ~15u;
}

// FMT, S, NA, XR, XT as qmv_mr_kernel; T: 16-row tiles per workgroup; NW:
// waves per workgroup (4 or 8; MR_WIN / NW windows per wave and range).
template <int FMT, int S, int NA, int XR, int T, int NW, int XT>
__global__ __launch_bounds__(64 * NW, 1) void qmv_kq_kernel(const QmvMrArgs a) {
  constexpr int NT = 64 * NW;
  constexpr int KQ_WPW = MR_WIN / NW;  // windows per wave and range
  constexpr int KQ_RING = 2 * KQ_WPW;  // ring entries per tile: two ranges of this wave's windows
  constexpr int CK = FMT == AFF8 ? 16 : 32;
  constexpr int KW = 4 * CK;
  constexpr int NQ = CK / 8;
  constexpr int XG = KW / S;
  constexpr int PG = XG / 8;
  constexpr int YV = 4 / S;
  constexpr int RK = MR_WIN * KW;
  constexpr int XP = RK + 8;
  constexpr int PCS = RK / 8;
  constexpr int XL = XR * PCS / NT;
  constexpr int GSMIN = KW / S;
  constexpr int SPITCH = RK / GSMIN + 2;
  constexpr int RW = 16 * T;  // weight rows per workgroup
  constexpr uint32_t XSO = (uint32_t)(XR + 1) * XP * 2u;
  constexpr uint32_t SCO = XSO + (uint32_t)MR_WIN * 16u * NA * 4u;
  constexpr uint32_t BUF = kq_buf_bytes(RK, XR, NA, GSMIN, RW);
  constexpr uint32_t ZROW = (uint32_t)XR * XP * 2u;
  constexpr int SL = (RW * (RK / GSMIN) / 4 + NT - 1) / NT;  // scale loads per thread, upper bound
  constexpr int NY = T * NA * YV;                                   // partial sums per lane
  static_assert(XL * NT == XR * PCS, "activation pieces split evenly over the threads");
  static_assert(PCS % 64 == 0 && PCS % PG == 0 && PG <= 16, "pieces and group slots as in qmv_mr_kernel");
  static_assert((XP * 2) % 16 == 0, "the zero row is whole 16-byte pieces");

  extern __shared__ __align__(16) unsigned char smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const QmvMat mat = pick_matrix(a.mt, a.w, a.scales, a.biases, a.out, a.N, blockIdx.x);
  const int M = a.M, N = mat.N, K = a.K;
  const int gsh = a.gs_shift;
  const int G = K >> gsh;
  const int ngr = RK >> gsh;
  const int row_wg = mat.blk * RW;
  const int nranges = K / RK;

  const uint32_t RB = (uint32_t)(K / CK) * 16u;
  const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(mat.w, (uint32_t)N * RB);
  const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(a.x, (uint32_t)M * (uint32_t)K * 2u);
  const __amdgpu_buffer_rsrc_t sr = buffer_rsrc(mat.scales, (uint32_t)N * (uint32_t)G * 2u);
  const __amdgpu_buffer_rsrc_t br = buffer_rsrc(mat.biases, (uint32_t)N * (uint32_t)G * 2u);
  const __amdgpu_buffer_rsrc_t w0 = buffer_rsrc(mat.w, 0u);
  const __amdgpu_buffer_rsrc_t x0 = buffer_rsrc(a.x, 0u);
  const __amdgpu_buffer_rsrc_t s0 = buffer_rsrc(mat.scales, 0u);
  const __amdgpu_buffer_rsrc_t b0 = buffer_rsrc(mat.biases, 0u);

  const int sunits = RW * ngr / 4;
  uint32_t xoff[XL], soff[SL];
#pragma unroll
  for (int i = 0; i < XL; i++) {
    const int p = tid + NT * i;
    const int m = p / PCS, c = p % PCS;
    xoff[i] = m < M ? (uint32_t)(m * K + 8 * c) * 2u : kDeadOfs;
  }
#pragma unroll
  for (int i = 0; i < SL; i++) {
    const int u = tid + NT * i;
    const int r = u / (ngr / 4), gl = (u % (ngr / 4)) * 4;
    const int n = row_wg + r;
    soff[i] = (u < sunits && n < N) ? (uint32_t)(n * G + gl) * 2u : kDeadOfs;
  }
  u32x4 xpre[XL];
  u32x2 spre[SL], bpre[SL];
  auto issue_range = [&](int range) {
    const bool live = range < nranges;
    const __amdgpu_buffer_rsrc_t xq = live ? xr : x0;
    const __amdgpu_buffer_rsrc_t sq = live ? sr : s0;
    const __amdgpu_buffer_rsrc_t bq = live ? br : b0;
    const int xs = range * RK * 2, ss = range * ngr * 2;
#pragma unroll
    for (int i = 0; i < XL; i++) xpre[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xq, xoff[i], xs, 0));
#pragma unroll
    for (int i = 0; i < SL; i++) {
      spre[i] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(sq, soff[i], ss, 0));
      bpre[i] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(bq, soff[i], ss, 0));
    }
  };
  auto stage_range = [&](uint32_t bofs) {
    uint16_t* xl = reinterpret_cast<uint16_t*>(smem + bofs);
    float* xsl = reinterpret_cast<float*>(smem + bofs + XSO);
    float2* sl = reinterpret_cast<float2*>(smem + bofs + SCO);
#pragma unroll
    for (int i = 0; i < XL; i++) {
      const int p = tid + NT * i;
      const int m = p / PCS, c = p % PCS;
      const u32x4 v = FMT == AFF4 ? perm_aff4_v(xpre[i]) : xpre[i];
      *reinterpret_cast<u32x4*>(xl + m * XP + 8 * c) = v;
      float sum = 0.f;
      constexpr uint32_t ONES = XT ? 0x3C003C00u : 0x3F803F80u;
#pragma unroll
      for (int e = 0; e < 4; e++) sum = dotx<XT>(xpre[i][e], ONES, sum);
      sum = mr_group_sum<PG>(sum);
      const int w = (8 * c) / KW, slot = ((8 * c) % KW) / XG;
      const int r = m * S + slot;
      if ((lane & (PG - 1)) == 0 && r < 16 * NA) xsl[w * 16 * NA + r] = sum;
    }
#pragma unroll
    for (int i = 0; i < SL; i++) {
      const int u = tid + NT * i;
      if (u < sunits) {
        const int r = u / (ngr / 4), gl = (u % (ngr / 4)) * 4;
#pragma unroll
        for (int h = 0; h < 4; h++) {
          const float s = xt_to_f32<XT>((spre[i][h >> 1] >> (16 * (h & 1))) & 0xFFFFu);
          const float b = xt_to_f32<XT>((bpre[i][h >> 1] >> (16 * (h & 1))) & 0xFFFFu);
          constexpr float OFS = XT ? 1024.0f : (FMT == AFF4 ? 128.0f : 0.0f);
          sl[r * SPITCH + gl + h] = float2{s, OFS != 0.0f ? __builtin_fmaf(-OFS, s, b) : b};
        }
      }
    }
  };

  // weights: tile t row row_wg + 16 t + (lane & 15), chunk lane >> 4 of this
  // wave's windows 2 wave + j; a ring of two ranges' worth per tile
  const int nl = lane & 15, g = lane >> 4;
  const int wv0 = __builtin_amdgcn_readfirstlane(wave) * KQ_WPW;  // this wave's first window in a range
  uint32_t woff[T];
#pragma unroll
  for (int t = 0; t < T; t++) {
    const int n = row_wg + 16 * t + nl;
    woff[t] = n < N ? (uint32_t)n * RB + (uint32_t)g * 16u : kDeadOfs;
  }
  auto w_load = [&](int range, int j, int t) {
    const __amdgpu_buffer_rsrc_t wq = range < nranges ? wr : w0;
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wq, woff[t],
                                                                           range * (MR_WIN * 64) + (wv0 + j) * 64, 0));
  };

  // ---- prologue: range 0 staged, range 1 in registers, two ranges of weights
  issue_range(0);
  u32x4 wbuf[KQ_RING][T];
#pragma unroll
  for (int p = 0; p < KQ_RING; p++)
#pragma unroll
    for (int t = 0; t < T; t++) wbuf[p][t] = w_load(p / KQ_WPW, p % KQ_WPW, t);
  for (int i = tid; i < 2 * (XP * 2 / 16); i += NT)
    *reinterpret_cast<u32x4*>(smem + (uint32_t)(i / (XP * 2 / 16)) * BUF + ZROW + (uint32_t)(i % (XP * 2 / 16)) * 16u) =
        u32x4{0u, 0u, 0u, 0u};
  stage_range(0u);
  issue_range(1);
  __syncthreads();

  // per-lane LDS bases of this wave's windows: A operand (as qmv_mr_kernel),
  // group sums and the first scale pair of each window
  const int slot_g = (g * CK) / XG;
  uint32_t abase[KQ_WPW][NA], xsb[KQ_WPW], sgo[KQ_WPW];
#pragma unroll
  for (int j = 0; j < KQ_WPW; j++) {
    const int w = wv0 + j;
#pragma unroll
    for (int u = 0; u < NA; u++) {
      const int r = 16 * u + nl;
      const int m = r / S, slot = r % S;
      abase[j][u] = (m < M && slot == slot_g ? (uint32_t)m * XP * 2u : ZROW) + (uint32_t)(g * CK) * 2u +
                    (uint32_t)(w * KW * 2);
    }
    xsb[j] = XSO + (uint32_t)((w * 16 * NA + 4 * g) * 4);
    sgo[j] = (uint32_t)(((w * KW) >> gsh) * 8);
  }

  float y[T][NA][YV];
#pragma unroll
  for (int t = 0; t < T; t++)
#pragma unroll
    for (int u = 0; u < NA; u++)
#pragma unroll
      for (int j = 0; j < YV; j++) y[t][u][j] = 0.f;

  for (int r2 = 0; r2 < nranges; r2 += 2) {
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const int range = r2 + h;
      const uint32_t bofs = (uint32_t)h * BUF;
#pragma unroll
      for (int j = 0; j < KQ_WPW; j++) {
        u32x4 A[NA][NQ];
#pragma unroll
        for (int u = 0; u < NA; u++)
#pragma unroll
          for (int q = 0; q < NQ; q++)
            A[u][q] = *reinterpret_cast<const u32x4*>(smem + abase[j][u] + bofs + (uint32_t)(q * 16));
        f32x4 xsv[NA];
#pragma unroll
        for (int u = 0; u < NA; u++) xsv[u] = *reinterpret_cast<const f32x4*>(smem + bofs + xsb[j] + (uint32_t)(64 * u));
        const int rs = h * KQ_WPW + j;  // ring slot; refilled with the same window two ranges on
#pragma unroll
        for (int t = 0; t < T; t++) {
          const u32x4 wv = wbuf[rs][t];
          wbuf[rs][t] = w_load(range + 2, j, t);
          u32x4 B[NQ];
          if constexpr (FMT == AFF4) {
#pragma unroll
            for (int q = 0; q < NQ; q++) {
              uint32_t pr[4];
              unpack_aff4(wv[q], pr, XT ? 0x64646464u : 0x43434343u);
              B[q] = u32x4{pr[0], pr[1], pr[2], pr[3]};
            }
          } else if constexpr (XT == 1) {
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
          float2 sc[S];
          const unsigned char* sp0 = smem + bofs + SCO + (uint32_t)((16 * t + nl) * SPITCH) * 8u + sgo[j];
#pragma unroll
          for (int hh = 0; hh < S; hh++) sc[hh] = reinterpret_cast<const float2*>(sp0)[hh];
#pragma unroll
          for (int u = 0; u < NA; u++) {
            f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int q = 0; q < NQ; q++) d = mfma16x16x32_xt<XT>(A[u][q], B[q], d);
#pragma unroll
            for (int i = 0; i < 4; i++) {
              const int slot = (4 * g + i) % S;
              y[t][u][i / S] = __builtin_fmaf(sc[slot].x, d[i], __builtin_fmaf(sc[slot].y, xsv[u][i], y[t][u][i / S]));
            }
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      stage_range((uint32_t)(h ^ 1) * BUF);
      issue_range(range + 2);
      __syncthreads();
    }
  }

  // ---- the waves' partial sums, added in wave order; wave 0 stores ---------
  // (the last barrier above follows every read of the staged ranges; the
  // launch's LDS covers max(2 BUF, NW x NY x 256 bytes))
  float* red = reinterpret_cast<float*>(smem);
#pragma unroll
  for (int t = 0; t < T; t++)
#pragma unroll
    for (int u = 0; u < NA; u++)
#pragma unroll
      for (int j = 0; j < YV; j++) red[((wave * T + t) * NA * YV + u * YV + j) * 64 + lane] = y[t][u][j];
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int t = 0; t < T; t++) {
      const int nrow = row_wg + 16 * t + nl;
#pragma unroll
      for (int u = 0; u < NA; u++)
#pragma unroll
        for (int j = 0; j < YV; j++) {
          float s = y[t][u][j];
#pragma unroll
          for (int v = 1; v < NW; v++) s += red[((v * T + t) * NA * YV + u * YV + j) * 64 + lane];
          const int m = (16 * u + 4 * g) / S + j;
          if (m < M && nrow < N) mat.out[(int64_t)m * N + nrow] = (uint16_t)f32_to_xt<XT>(s);
        }
    }
  }
}

// ---- host ------------------------------------------------------------------

namespace {

template <int FMT, int S, int NA, int XT>
hipError_t mr_launch_xt(const QmvMrPlan& p, const QmvMrArgs& a, hipStream_t stream) {
  const dim3 grid((unsigned)p.row_blocks), block((unsigned)MR_NT);
  if (p.t > 0) {
    // two A tiles come only with 2 or 4 group slots (more than 16 rows x slots)
    if constexpr (NA == 2 && S == 1) return hipErrorInvalidValue;
    else {
#define KQ_CASE(XR_, T_, NW_)                                                                              \
  if (p.xr == XR_ && p.t == T_ && p.nw == NW_) {                                                           \
    hipLaunchKernelGGL((qmv_kq_kernel<FMT, S, NA, XR_, T_, NW_, XT>), dim3((unsigned)p.row_blocks),        \
                       dim3(64 * NW_), p.lds, stream, a);                                                  \
    return hipGetLastError();                                                                              \
  }
      KQ_CASE(8, 1, 8)
      KQ_CASE(8, 2, 8)
      KQ_CASE(8, 3, 8)
      KQ_CASE(8, 4, 8)
      KQ_CASE(16, 1, 8)
      KQ_CASE(16, 2, 8)
      KQ_CASE(16, 3, 8)
      KQ_CASE(16, 4, 8)
#undef KQ_CASE
      return hipErrorInvalidValue;
    }
  }
  if (p.ring == 4) {
    if (p.xr == 8) hipLaunchKernelGGL((qmv_mr_kernel<FMT, S, NA, 8, 4, XT>), grid, block, p.lds, stream, a);
    else hipLaunchKernelGGL((qmv_mr_kernel<FMT, S, NA, 16, 4, XT>), grid, block, p.lds, stream, a);
  } else if (p.ring == 16) {
    if (p.xr == 8) hipLaunchKernelGGL((qmv_mr_kernel<FMT, S, NA, 8, 16, XT>), grid, block, p.lds, stream, a);
    else hipLaunchKernelGGL((qmv_mr_kernel<FMT, S, NA, 16, 16, XT>), grid, block, p.lds, stream, a);
  } else {
    if (p.xr == 8) hipLaunchKernelGGL((qmv_mr_kernel<FMT, S, NA, 8, 8, XT>), grid, block, p.lds, stream, a);
    else hipLaunchKernelGGL((qmv_mr_kernel<FMT, S, NA, 16, 8, XT>), grid, block, p.lds, stream, a);
  }
  return hipGetLastError();
}

template <int FMT, int S, int NA>
hipError_t mr_launch(const QmvMrPlan& p, const QmvMrArgs& a, hipStream_t stream) {
  return a.xt ? mr_launch_xt<FMT, S, NA, 1>(p, a, stream) : mr_launch_xt<FMT, S, NA, 0>(p, a, stream);
}

template <int FMT, int S>
hipError_t mr_launch_s(const QmvMrPlan& p, const QmvMrArgs& a, hipStream_t stream) {
  return p.na == 1 ? mr_launch<FMT, S, 1>(p, a, stream) : mr_launch<FMT, S, 2>(p, a, stream);
}

}  // namespace

QmvMrPlan qmv_mr_plan(int fmt, int gs, int64_t N, int64_t K, int rows, int cus, bool force, int ring_req) {
  QmvMrPlan p;
  if (fmt != AFF4 && fmt != AFF8) return p;
  if (rows < 1 || rows > 16 || (gs != 32 && gs != 64 && gs != 128) || N < 1 || K < 1) return p;
  const int kw = fmt == AFF8 ? 64 : 128;
  p.s = kw / gs > 1 ? kw / gs : 1;
  const int ar = rows * p.s;
  if (ar > 32) return p;
  p.na = ar <= 16 ? 1 : 2;
  p.xr = rows <= 8 ? 8 : 16;
  p.rk = MR_WIN * kw;
  if (K % p.rk != 0) return p;
  const int64_t G = K / gs;
  if ((p.rk / gs) % 4 != 0 || G % 4 != 0) return p;  // scales load 4 groups at a time
  p.row_blocks = (int)((N + MR_RW - 1) / MR_RW);
  // one launch needs ~one workgroup per CU; fewer rows leave CUs idle
  if (!force && (int64_t)p.row_blocks * 4 < (int64_t)cus * 3) return p;
  p.lds = 2u * mr_buf_bytes(p.rk, p.xr, p.na, kw / p.s);
  // weight ring: 8 windows (one range), 4 with two A tiles, whose operands
  // need the registers (MI355X, Llama-3-8B gate/up: 4-bit M=4 10.4 us with 8
  // vs 11.1 with 4 and 11.6 with 16; M=16 15.3 with 4 vs 15.9 with 8)
  p.ring = (ring_req == 4 || ring_req == 8 || ring_req == 16) ? ring_req : (p.na == 2 ? 4 : 8);
  // buffer offsets are 32-bit and 0x80000000 marks a dead lane
  const int64_t wbytes = N * K * (fmt == AFF8 ? 8 : 4) / 8;
  p.ok = p.lds <= 160 * 1024 && wbytes < ((int64_t)1 << 31) && N * G * 2 < ((int64_t)1 << 31) &&
         (int64_t)rows * K * 2 < ((int64_t)1 << 31) && p.row_blocks <= (1 << 30);
  return p;
}

bool kq_tiles_ok(int t) { return t >= 1 && t <= 4; }

QmvMrPlan qmv_kq_plan(int fmt, int gs, int64_t N, int64_t K, int rows, int cus, int t_req, int nw_req) {
  QmvMrPlan p;
  if (fmt != AFF4 && fmt != AFF8) return p;
  if (rows < 1 || rows > 16 || (gs != 32 && gs != 64 && gs != 128) || N < 1 || K < 1 || cus < 1) return p;
  const int kw = fmt == AFF8 ? 64 : 128;
  p.s = kw / gs > 1 ? kw / gs : 1;
  const int ar = rows * p.s;
  if (ar > 32) return p;
  p.na = ar <= 16 ? 1 : 2;
  p.xr = rows <= 8 ? 8 : 16;
  p.rk = MR_WIN * kw;
  if (K % p.rk != 0) return p;
  const int64_t G = K / gs;
  if ((p.rk / gs) % 4 != 0 || G % 4 != 0) return p;
  // the fewest tiles per workgroup that still fit one round of the CUs
  p.t = 0;
  if (kq_tiles_ok(t_req)) p.t = t_req;
  else
    for (int t = 1; t <= 4; t++)
      if (p.t == 0 && (N + 16 * t - 1) / (16 * t) <= cus) p.t = t;
  if (p.t == 0) return p;
  // 8 waves (one window per wave and range, two waves per SIMD) hide more of
  // each window's operand and MFMA latency than 4 (MI355X, Qwen3-8B shapes,
  // 4-bit g64, 16 rows: o 8.95 -> 7.59 us, down 18.7 -> 15.3, q/k/v in one
  // launch 11.4 -> 10.6; 8 rows: 6.16 -> 6.02, 12.4 -> 11.7, 8.34 -> 8.04)
  (void)nw_req;
  p.nw = 8;
  p.row_blocks = (int)((N + 16 * p.t - 1) / (16 * p.t));
  p.lds = std::max<size_t>(2u * kq_buf_bytes(p.rk, p.xr, p.na, kw / p.s, 16 * p.t),
                           (size_t)p.nw * p.t * p.na * (4 / p.s) * 64u * 4u);  // staging, then the waves' sums
  const int64_t wbytes = N * K * (fmt == AFF8 ? 8 : 4) / 8;
  p.ok = p.lds <= 160 * 1024 && wbytes < ((int64_t)1 << 31) && N * G * 2 < ((int64_t)1 << 31) &&
         (int64_t)rows * K * 2 < ((int64_t)1 << 31) && p.row_blocks <= (1 << 30);
  return p;
}

hipError_t qmv_mr_launch(int fmt, const QmvMrArgs& a, const QmvMrPlan& p, hipStream_t stream) {
  if (!p.ok) return hipErrorInvalidValue;
  if (fmt == AFF4) {
    switch (p.s) {
      case 1: return mr_launch_s<AFF4, 1>(p, a, stream);
      case 2: return mr_launch_s<AFF4, 2>(p, a, stream);
      default: return mr_launch_s<AFF4, 4>(p, a, stream);
    }
  }
  return p.s == 2 ? mr_launch_s<AFF8, 2>(p, a, stream) : mr_launch_s<AFF8, 1>(p, a, stream);
}

}  // namespace mlxq
