// qmm_group.hip — gather_qmm over expert-sorted rows (mxfp4 MoE) for gfx950.
//
// The reference's sorted MoE route (overlays/rocm/mlx/backend/rocm/quantized/
// qmm.hip:4741-4915 gather_qmv_expert_batched_kernel + find_sorted_expert_run:
// a block per expert, its run found by binary search in the sorted indices)
// and its CPU math (overlays/cpu/mlx/backend/cpu/quantized.cpp:550-597,
// 875-914): out[b] = x[b] @ dequant(w[rhs[b]])^T for index entries b whose
// experts rhs[b] are sorted, one activation row per entry.
//
// A workgroup owns one expert and 128 of its weight rows over the whole of K,
// and multiplies them with all of that expert's activation rows (in chunks of
// up to 64), so each expert's weights are streamed once per chunk of rows
// instead of once per entry.  It finds its expert's rows [lo, hi) itself: two
// lower-bound searches over the sorted indices, 64 lanes narrowing the range
// 64-fold per step (no preparation launch).
//
// Products: v_mfma_f32_16x16x32_bf16, weights as the B operand straight from
// registers: lane i holds weight row i % 16 and 16-byte code chunk i / 16 of a
// 4-chunk (128 k) window; a chunk is exactly one mxfp4 group (32 codes), so
// the lane widens its codes with the group's e8m0 scale folded into the gfx950
// fp4 conversion (fp4 code points times a power of two are exact in bf16) and
// the MFMAs accumulate over all of K with no per-group fold.  Activations: a
// 256-k block of the chunk's rows is staged in LDS (the next block's loads and
// the next block's weights are in flight while the current one is used).
#include "common.hpp"
#include "kernels.hpp"

namespace mlxq {

namespace {

constexpr int GQ_NW = 4;                     // waves per workgroup
constexpr int GQ_T = 2;                      // 16-row weight tiles per wave
constexpr int GQ_ROWS = GQ_NW * GQ_T * 16;   // weight rows per workgroup (128)
constexpr int GQ_MC = 64;                    // activation rows per chunk (4 A tiles)
constexpr int GQ_KB = 256;                   // k per staged block (2 windows)
constexpr int GQ_NT = 64 * GQ_NW;
constexpr int GQ_XPITCH = GQ_KB + 8;         // bf16 per staged row (16 bytes of padding)
constexpr int GQ_XP = GQ_MC * GQ_KB / 8 / GQ_NT;  // 16-byte activation pieces per thread and block (8)

// First entry whose (clamped) expert is >= v in the sorted index array;
// wave-uniform.  Each step samples 64 evenly spaced entries of [lo, hi).
__device__ __forceinline__ int lower_bound_sorted(const uint32_t* idx, int stride, int n, int clamp, int v,
                                                  int lane) {
  int lo = 0, hi = n;
  while (lo < hi) {
    const int span = hi - lo;
    const int step = (span + 63) / 64;
    const int pos = lo + lane * step;
    const bool in = pos < hi;
    const int val = in ? seg_index(idx, stride, pos, clamp, 0) : 0x7FFFFFFF;
    const uint64_t below = __ballot(in && val < v);
    const uint64_t inside = __ballot(in);
    const int c = __popcll(below);
    const int ns = __popcll(inside);
    const int nlo = c > 0 ? lo + (c - 1) * step + 1 : lo;
    const int nhi = c < ns ? lo + c * step : hi;
    if (step == 1) return c < ns ? lo + c : hi;
    lo = nlo;
    hi = nhi;
  }
  return lo;
}

}  // namespace

__global__ __launch_bounds__(GQ_NT, 2) void qmm_group_mxfp4_kernel(const QmmGroupArgs a) {
  __shared__ __align__(16) uint16_t xl[GQ_MC * GQ_XPITCH];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int N = a.N;
  const int K = a.K;
  const int e = blockIdx.y;
  const int nb0 = blockIdx.x * GQ_ROWS;

  // ---- this expert's rows ----------------------------------------------------
  const int lo = lower_bound_sorted(a.rhs, a.rhs_stride, a.B, a.E, e, lane);
  const int hi = lower_bound_sorted(a.rhs, a.rhs_stride, a.B, a.E, e + 1, lane);
  if (hi <= lo) return;

  const int nchunk = K / 32;                     // 16-byte code chunks (mxfp4 groups) per row
  const uint32_t RB = (uint32_t)nchunk * 16u;    // bytes per weight row
  const int nwin = (nchunk + 3) / 4;             // 128-k windows
  const int nblk = (nwin + 1) / 2;               // 256-k blocks
  const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(a.w + (int64_t)e * N * (nchunk * 4), (uint32_t)N * RB);
  const __amdgpu_buffer_rsrc_t sr = buffer_rsrc(a.scales + (int64_t)e * N * nchunk, (uint32_t)(N * nchunk));

  const int nl = lane & 15;
  const int g = lane >> 4;
  uint32_t wrow[GQ_T], srow[GQ_T];
#pragma unroll
  for (int t = 0; t < GQ_T; t++) {
    const int n = nb0 + wave * (GQ_T * 16) + t * 16 + nl;
    wrow[t] = n < N ? (uint32_t)n * RB : kDeadOfs;
    srow[t] = n < N ? (uint32_t)(n * nchunk) : kDeadOfs;
  }

  // weights + scales of block b for tile t, window v (0/1) of the block
  // Chunks past the end of a row read the next row's codes (or past the
  // matrix: zeros); they meet activations that are zero there, and fp4 codes
  // are finite, so they add exactly 0.  Their scales are not read (dead: 0,
  // a finite 2^-127), since the next row's could be NaN.
  // Blocks past the last are dead offsets: no memory traffic, zeros.
  auto wload = [&](int b, int t, int v) -> u32x4 {
    const uint32_t o = b < nblk ? wrow[t] + (uint32_t)((2 * b + v) * 4 + g) * 16u : kDeadOfs;
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, o, 0, 2 /* nt */));
  };
  auto sload = [&](int b, int t, int v) -> uint32_t {
    const int c = (2 * b + v) * 4 + g;
    const uint32_t o = (srow[t] != kDeadOfs && c < nchunk) ? srow[t] + (uint32_t)c : kDeadOfs;
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(sr, o, 0, 0);
  };

  for (int r0 = lo; r0 < hi; r0 += GQ_MC) {
    const int cnt = min(GQ_MC, hi - r0);
    const int nat = (cnt + 15) / 16;  // live A tiles (uniform)
    const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(a.x + (int64_t)r0 * K, (uint32_t)cnt * (uint32_t)K * 2u);
    auto xload = [&](int b, int i) -> u32x4 {
      const int p = tid + i * GQ_NT;
      const int m = p / (GQ_KB / 8), c = p % (GQ_KB / 8);
      const int k = b * GQ_KB + 8 * c;
      const uint32_t o = (m < cnt && k < K) ? (uint32_t)(m * K + k) * 2u : kDeadOfs;
      return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, o, 0, 0));
    };

    f32x4 acc[4][GQ_T];
#pragma unroll
    for (int u = 0; u < 4; u++)
#pragma unroll
      for (int t = 0; t < GQ_T; t++) acc[u][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    // block 0 loads
    u32x4 xn[GQ_XP];
#pragma unroll
    for (int i = 0; i < GQ_XP; i++) xn[i] = xload(0, i);
    u32x4 wn[GQ_T][2];
    uint32_t sn[GQ_T][2];
#pragma unroll
    for (int t = 0; t < GQ_T; t++)
#pragma unroll
      for (int v = 0; v < 2; v++) {
        wn[t][v] = wload(0, t, v);
        sn[t][v] = sload(0, t, v);
      }

    for (int b = 0; b < nblk; b++) {
      // stage block b's activations (the previous block's readers are done)
      __syncthreads();
#pragma unroll
      for (int i = 0; i < GQ_XP; i++) {
        const int p = tid + i * GQ_NT;
        const int m = p / (GQ_KB / 8), c = p % (GQ_KB / 8);
        *reinterpret_cast<u32x4*>(xl + m * GQ_XPITCH + 8 * c) = xn[i];
      }
      u32x4 wc[GQ_T][2];
      uint32_t sc[GQ_T][2];
#pragma unroll
      for (int t = 0; t < GQ_T; t++)
#pragma unroll
        for (int v = 0; v < 2; v++) {
          wc[t][v] = wn[t][v];
          sc[t][v] = sn[t][v];
        }
      __syncthreads();
      // next block's loads in flight while this one is used (past the last
      // block every offset is dead: no branch, so no wait at a join)
#pragma unroll
      for (int i = 0; i < GQ_XP; i++) xn[i] = xload(b + 1, i);
#pragma unroll
      for (int t = 0; t < GQ_T; t++)
#pragma unroll
        for (int v = 0; v < 2; v++) {
          wn[t][v] = wload(b + 1, t, v);
          sn[t][v] = sload(b + 1, t, v);
        }
#pragma unroll
      for (int v = 0; v < 2; v++) {
        // B operands: the lane's chunk widened with its group scale folded in
        bf16x8 B[GQ_T][4];
#pragma unroll
        for (int t = 0; t < GQ_T; t++) {
          const float s = e8m0_to_f32(sc[t][v]);
#pragma unroll
          for (int q = 0; q < 4; q++) {
            uint32_t pr[4];
            unpack_mxfp4_scaled(wc[t][v][q], s, pr);
            B[t][q] = as_bf16x8(pr);
          }
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
          if (u < nat) {
            // A: activation row 16u + (lane & 15), k = window base + 32 g + 8 q
            const uint16_t* src = xl + (16 * u + nl) * GQ_XPITCH + v * 128 + g * 32;
            bf16x8 A[4];
#pragma unroll
            for (int q = 0; q < 4; q++) A[q] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(src + 8 * q));
#pragma unroll
            for (int t = 0; t < GQ_T; t++)
#pragma unroll
              for (int q = 0; q < 4; q++) acc[u][t] = mfma16x16x32(A[q], B[t][q], acc[u][t]);
          }
        }
      }
    }

    // ---- store: D row 4 g + i of A tile u is activation row 16u + 4g + i ------
#pragma unroll
    for (int u = 0; u < 4; u++) {
      if (u < nat) {
#pragma unroll
        for (int t = 0; t < GQ_T; t++) {
          const int n = nb0 + wave * (GQ_T * 16) + t * 16 + nl;
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const int m = 16 * u + 4 * g + i;
            if (m < cnt && n < N) a.out[(int64_t)(r0 + m) * N + n] = (uint16_t)f32_to_bf16_bits(acc[u][t][i]);
          }
        }
      }
    }
  }
}

QmmGroupPlan qmm_group_plan(int fmt, int64_t N, int64_t K, int64_t E, int64_t B) {
  QmmGroupPlan p;
  if (fmt != MXFP4 || N < 1 || K < 32 || K % 32 != 0 || E < 1 || B < 1) return p;
  p.row_blocks = (int)((N + GQ_ROWS - 1) / GQ_ROWS);
  // buffer offsets are 32-bit and 0x80000000 marks a dead lane
  p.ok = N * (K / 2) < ((int64_t)1 << 31) && (int64_t)GQ_MC * K * 2 < ((int64_t)1 << 31) && E <= 65535 &&
         p.row_blocks <= 65535 && B * K * 2 < ((int64_t)1 << 40);
  return p;
}

hipError_t qmm_group_launch(const QmmGroupArgs& a, const QmmGroupPlan& p, hipStream_t stream) {
  if (!p.ok) return hipErrorInvalidValue;
  hipLaunchKernelGGL(qmm_group_mxfp4_kernel, dim3((unsigned)p.row_blocks, (unsigned)a.E), dim3(GQ_NT), 0, stream,
                     a);
  return hipGetLastError();
}

}  // namespace mlxq
