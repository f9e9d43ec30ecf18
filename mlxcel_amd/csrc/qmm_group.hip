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
// the MFMAs accumulate over all of K with no per-group fold.
//
// Pipelining: K runs in 128-k blocks.  A block's activations (64 rows x 256
// bytes) go straight from memory into one of 4 LDS buffers with
// buffer_load_dwordx4 ... lds (lane L of a load lands at M0 + 16 L, so each
// wave load fills 4 rows; the row's 16-byte chunks are stored XOR-swizzled by
// the row index, which keeps the 16 rows an MFMA operand read touches on
// distinct banks), and its weights and scales into one of 4 register slots;
// both run 3 blocks ahead of the block being multiplied, with no registers
// spent on activations in flight.
//
// Scales: the workgroup's 128 scale rows are one contiguous range of the
// expert's e8m0 bytes; where they fit (K <= 4096) and are aligned, a few
// wide direct-to-LDS loads bring them into an LDS table once, ahead of the
// ring, and each block reads its byte from there.  Otherwise every block
// loads each lane's scale byte with the weights (one 64-lane byte load per
// tile and block, 16 scattered rows: on MI355X 13% of the T=256 gate/up
// gather's time at K=2880).
#include "common.hpp"
#include "kernels.hpp"

namespace mlxq {

namespace {

constexpr int GQ_NW = 4;                     // waves per workgroup
constexpr int GQ_MCMAX = 64;                 // activation rows per chunk, at most
constexpr int GQ_KB = 128;                   // k per block (one 4-group window)
constexpr int GQ_NT = 64 * GQ_NW;
constexpr int GQ_RING = 4;                   // blocks in the activation / weight rings
constexpr int GQ_STB = 128;                  // LDS scale table: up to 128 e8m0 bytes per row (K <= 4096)

}  // namespace

// SCL: 0, scale bytes loaded per block; 4 or 16, the scale table staged in
// LDS by direct loads of that many bytes per lane.  GT: 16-row weight tiles
// per wave: 2 (128 weight rows, chunks of 64 activation rows), or 3 (192
// rows, chunks of 48, with the scale table only: for a launch that needs one
// round of the CUs' workgroup slots where 128-row blocks need two).
template <int SCL, int GT>
__global__ __launch_bounds__(GQ_NT, 2) void qmm_group_mxfp4_kernel(const QmmGroupArgs a) {
  static_assert(GT == 2 || (GT == 3 && SCL != 0), "192-row workgroups take scales from the table");
  constexpr int GQ_T = GT;                       // 16-row weight tiles per wave
  constexpr int GQ_ROWS = GQ_NW * GQ_T * 16;     // weight rows per workgroup
  constexpr int GQ_MC = GT == 3 ? 48 : 64;       // activation rows per chunk
  constexpr int GQ_AT = GQ_MC / 16;              // A tiles per chunk
  constexpr int GQ_XB = GQ_MC * GQ_KB * 2;       // activation bytes per block (256 per row)
  constexpr int GQ_XI = GQ_XB / 1024 / GQ_NW;    // 1 KiB direct-to-LDS loads per wave and block (4 or 3)
  static_assert(GQ_XI * 1024 * GQ_NW == GQ_XB, "whole 1 KiB wave loads");
  // the ring as four LDS objects, so the compiler's wait analysis sees that
  // a buffer being refilled is not the one being read
  __shared__ __align__(16) unsigned char xl0[GQ_XB], xl1[GQ_XB], xl2[GQ_XB], xl3[GQ_XB];
  __shared__ __align__(16) unsigned char stb[SCL ? GQ_ROWS * GQ_STB : 16];
  static_assert(GQ_RING == 4, "four ring buffers");
  auto ring = [&](int slot) -> unsigned char* { return slot == 0 ? xl0 : slot == 1 ? xl1 : slot == 2 ? xl2 : xl3; };

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
  const int nblk = (nchunk + 3) / 4;             // 128-k blocks
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

  // weights + scales of block b for tile t.
  // Chunks past the end of a row read the next row's codes (or past the
  // matrix: zeros); they meet activations that are zero there, and fp4 codes
  // are finite, so they add exactly 0.  Their scales are not read (dead: 0,
  // a finite 2^-127), since the next row's could be NaN.
  // Blocks past the last are dead offsets: no memory traffic, zeros.
  // Default cache policy, not the streaming hint: a block reads 64 bytes of
  // each 128-byte line of a row and the next block the other half, and with
  // the hint the line often left L2 in between (HBM fetch 1.85x the
  // algorithmic bytes, 1.2x without).
  auto wload = [&](int b, int t) -> u32x4 {
    const uint32_t o = b < nblk ? wrow[t] + (uint32_t)(b * 4 + g) * 16u : kDeadOfs;
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, o, 0, 0));
  };
  auto sload = [&](int b, int t) -> uint32_t {
    const int c = b * 4 + g;
    const uint32_t o = (srow[t] != kDeadOfs && c < nchunk) ? srow[t] + (uint32_t)c : kDeadOfs;
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(sr, o, 0, 0);
  };
  // Scale table (SCL != 0): table row r = weight row nb0 + r, nchunk bytes
  // each, read straight from the range that starts at row nb0; loads past
  // the expert's scales read 0.  Issued before the ring, so the ring's first
  // wait covers them.
  if constexpr (SCL != 0) {
    const int tb = min(GQ_ROWS, N - nb0) * nchunk;  // bytes of this row block's scale rows
    constexpr int PER = 64 * SCL;                   // bytes per wave load
    for (int i = wave; i * PER < tb; i += GQ_NW) {
      auto* dst = (__attribute__((address_space(3))) void*)(stb + i * PER);
      const uint32_t o = (uint32_t)(nb0 * nchunk + i * PER + lane * SCL);
      if constexpr (SCL == 16) __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, dst, 16, o, 0, 0, 0);
      else __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, dst, 4, o, 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  bool slive[GQ_T];
#pragma unroll
  for (int t = 0; t < GQ_T; t++) slive[t] = srow[t] != kDeadOfs;
  // the scale byte of tile t, chunk c (SCL != 0): rows past N and chunks
  // past the row are 0 (a finite 2^-127), never another row's byte
  auto sread = [&](int c, int t) -> uint32_t {
    const int r = wave * (GQ_T * 16) + t * 16 + nl;
    return (slive[t] && c < nchunk) ? (uint32_t)stb[r * nchunk + c] : 0u;
  };
  // LDS layout of a block: row r at r * 256 bytes, its logical 16-byte chunk
  // c at position c ^ (r & 15).  Wave load j of wave w fills rows
  // 4 (w GQ_XI + j) .. +3: lane L writes row rr = 4 (w GQ_XI + j) + L / 16,
  // position L % 16, so it fetches logical chunk (L % 16) ^ (rr & 15).
  constexpr int GQ_VMEM = GQ_XI + (SCL ? 1 : 2) * GQ_T;  // vector-memory instructions per block and wave

  for (int r0 = lo; r0 < hi; r0 += GQ_MC) {
    const int cnt = min(GQ_MC, hi - r0);
    const int nat = (cnt + 15) / 16;  // live A tiles (uniform)
    const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(a.x + (int64_t)r0 * K, (uint32_t)cnt * (uint32_t)K * 2u);
    // Per wave load j: the lane's byte offset at block 0 (dead past the
    // chunk's rows), fixed for the whole chunk; block b adds b * 256 bytes
    // through the scalar offset (the range check covers the vector offset
    // only, and every live offset stays inside the chunk's rows: the one
    // block reaching past K kills its chunks past K).  Address registers
    // that are never rewritten keep the compiler from waiting on the ring.
    uint32_t xo[GQ_XI];
    int xk[GQ_XI];
#pragma unroll
    for (int j = 0; j < GQ_XI; j++) {
      const int rr = 4 * (wave * GQ_XI + j) + (lane >> 4);
      xk[j] = 8 * ((lane & 15) ^ (rr & 15));
      xo[j] = rr < cnt ? (uint32_t)(rr * K + xk[j]) * 2u : kDeadOfs;
    }
    auto issue = [&](int b, int slot, u32x4 (&wn)[GQ_RING][GQ_T], uint32_t (&sn)[GQ_RING][GQ_T]) {
      const bool tail = (b + 1) * GQ_KB > K;  // uniform
#pragma unroll
      for (int j = 0; j < GQ_XI; j++) {
        uint32_t o = xo[j];
        if (tail) o = b * GQ_KB + xk[j] < K ? o : kDeadOfs;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            xr, (__attribute__((address_space(3))) void*)(ring(slot) + (wave * GQ_XI + j) * 1024), 16, o,
            b * GQ_KB * 2, 0, 0);
      }
#pragma unroll
      for (int t = 0; t < GQ_T; t++) {
        wn[slot][t] = wload(b, t);
        if constexpr (SCL == 0) sn[slot][t] = sload(b, t);
      }
    };

    f32x4 acc[GQ_AT][GQ_T];
#pragma unroll
    for (int u = 0; u < GQ_AT; u++)
#pragma unroll
      for (int t = 0; t < GQ_T; t++) acc[u][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    u32x4 wn[GQ_RING][GQ_T];
    uint32_t sn[GQ_RING][GQ_T];
#pragma unroll
    for (int d = 0; d < GQ_RING - 1; d++) issue(d, d, wn, sn);

    // Whole ring turns: the blocks past the last (at most GQ_RING - 1) still
    // wait, synchronise and issue (dead offsets: no memory traffic) but skip
    // their MFMAs.  A loop without an early exit keeps every ring slot in the
    // same registers across the back edge; an exit inside the unrolled turn
    // made the compiler copy the slots there, waiting for every load in
    // flight once a turn.
    for (int b0 = 0; b0 < nblk; b0 += GQ_RING) {
#pragma unroll
      for (int d = 0; d < GQ_RING; d++) {
        const int b = b0 + d;
        // block b's loads were issued GQ_RING - 1 blocks ago: wait until at most
        // the GQ_RING - 2 later blocks' instructions are outstanding, then all
        // waves' activations of block b are in LDS and every wave is done
        // with the buffer block b + GQ_RING - 1 refills
        // (one statement: nothing moves between the wait and the barrier, and
        // no LDS read moves across either; a plain barrier, because the
        // workgroup fences of __syncthreads would also wait for the ring's
        // younger activation loads)
        // (mlxcel_amd/build.py checks the emitted assembly for exactly 8, or 6,
        // loads per block)
        if constexpr (SCL == 0) {
          static_assert(SCL != 0 || GQ_VMEM * (GQ_RING - 2) == 16, "the wait below counts 2 blocks of 8");
          asm volatile("s_waitcnt vmcnt(16)\n\ts_barrier" ::: "memory");
        } else {
          static_assert(SCL == 0 || GQ_VMEM * (GQ_RING - 2) == 12, "the wait below counts 2 blocks of 6");
          asm volatile("s_waitcnt vmcnt(12)\n\ts_barrier" ::: "memory");
        }
        issue(b + GQ_RING - 1, (d + GQ_RING - 1) % GQ_RING, wn, sn);
        if (b >= nblk) continue;  // workgroup-uniform
        const unsigned char* xb = ring(d);
        // B operands: the lane's chunk widened with its group scale folded in
        bf16x8 B[GQ_T][4];
#pragma unroll
        for (int t = 0; t < GQ_T; t++) {
          const float sc = e8m0_to_f32(SCL ? sread(b * 4 + g, t) : sn[d][t]);
#pragma unroll
          for (int q = 0; q < 4; q++) {
            uint32_t pr[4];
            unpack_mxfp4_scaled(wn[d][t][q], sc, pr);
            B[t][q] = as_bf16x8(pr);
          }
        }
#pragma unroll
        for (int u = 0; u < GQ_AT; u++) {
          if (u < nat) {
            // A: activation row 16u + nl, logical chunk 4g + q at position (4g + q) ^ nl
            const unsigned char* row = xb + (16 * u + nl) * 256;
            bf16x8 A[4];
#pragma unroll
            for (int q = 0; q < 4; q++)
              A[q] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(row + 16 * ((4 * g + q) ^ nl)));
#pragma unroll
            for (int t = 0; t < GQ_T; t++)
#pragma unroll
              for (int q = 0; q < 4; q++) acc[u][t] = mfma16x16x32(A[q], B[t][q], acc[u][t]);
          }
        }
      }
    }
    // the ring's loads past the last block (dead, zeros) land before the next
    // chunk or the end of the workgroup reuses the buffers
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();

    // ---- store: D row 4 g + i of A tile u is activation row 16u + 4g + i ------
#pragma unroll
    for (int u = 0; u < GQ_AT; u++) {
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

QmmGroupPlan qmm_group_plan(int fmt, int64_t N, int64_t K, int64_t E, int64_t B, int cus, int tiles_req) {
  QmmGroupPlan p;
  if (fmt != MXFP4 || N < 1 || K < 32 || K % 32 != 0 || E < 1 || B < 1) return p;
  p.scale_table = K / 32 <= GQ_STB;
  // 192-row workgroups (scales from the table, chunks of 48 activation
  // rows) unless their rounds of the CUs' two workgroup slots cost more
  // than the 128-row ones' (a 192-row workgroup takes less than 1.5 times as
  // long: each staged activation block serves 192 weight rows), and where an
  // expert has at most ~40 rows on average (more would often take a second
  // chunk, streaming its weights again).  The grid has E workgroups per row
  // block; those of experts without rows exit at once, so this counts the
  // most it can hold.  MI355X, gpt-oss MoE at T=256 (32 experts, 1024
  // entries): gate/up 2880 x 2 rows and down 2880 rows, 152 -> 135 us for
  // both launches (down alone on 192 rows: 142).
  const int64_t slots = 2 * (int64_t)(cus > 1 ? cus : 1);
  auto rounds = [&](int64_t rows) { return (((N + rows - 1) / rows) * E + slots - 1) / slots; };
  p.tiles = 2;
  if (tiles_req == 3 || (tiles_req != 2 && p.scale_table && B <= 40 * E && rounds(192) * 3 <= rounds(128) * 2))
    p.tiles = 3;
  p.row_blocks = (int)((N + 64 * p.tiles - 1) / (64 * p.tiles));
  // buffer offsets are 32-bit and 0x80000000 marks a dead lane
  p.ok = N * (K / 2) < ((int64_t)1 << 31) && (int64_t)GQ_MCMAX * K * 2 < ((int64_t)1 << 31) && E <= 65535 &&
         p.row_blocks <= 65535 && B * K * 2 < ((int64_t)1 << 40);
  return p;
}

hipError_t qmm_group_launch(const QmmGroupArgs& a, const QmmGroupPlan& p, hipStream_t stream) {
  if (!p.ok) return hipErrorInvalidValue;
  // the LDS scale table's direct loads need their source aligned to the
  // load width: the scales' base and every expert's N * K / 32 bytes
  const uintptr_t sb = reinterpret_cast<uintptr_t>(a.scales);
  const int64_t eb = (int64_t)a.N * (a.K / 32);
  const int scl = !p.scale_table ? 0 : (sb % 16 == 0 && eb % 16 == 0) ? 16 : (sb % 4 == 0 && eb % 4 == 0) ? 4 : 0;
  const int tiles = scl ? p.tiles : 2;  // 192-row workgroups need the table
  const dim3 grid((unsigned)((a.N + 64 * tiles - 1) / (64 * tiles)), (unsigned)a.E);
  if (tiles == 3 && scl == 16) hipLaunchKernelGGL((qmm_group_mxfp4_kernel<16, 3>), grid, dim3(GQ_NT), 0, stream, a);
  else if (tiles == 3) hipLaunchKernelGGL((qmm_group_mxfp4_kernel<4, 3>), grid, dim3(GQ_NT), 0, stream, a);
  else if (scl == 16) hipLaunchKernelGGL((qmm_group_mxfp4_kernel<16, 2>), grid, dim3(GQ_NT), 0, stream, a);
  else if (scl == 4) hipLaunchKernelGGL((qmm_group_mxfp4_kernel<4, 2>), grid, dim3(GQ_NT), 0, stream, a);
  else hipLaunchKernelGGL((qmm_group_mxfp4_kernel<0, 2>), grid, dim3(GQ_NT), 0, stream, a);
  return hipGetLastError();
}

}  // namespace mlxq
