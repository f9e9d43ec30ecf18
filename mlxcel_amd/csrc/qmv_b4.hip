// qmv_b4.hip — block-MFMA decode kernel (1 to 16 activation rows per weight
// matrix) for gfx950.
//
// Same product as qmv_rs.hip / qmv.hip (reference decode route: overlays/
// rocm/mlx/backend/rocm/quantized/qmv_tiled_kernel.hip:29-128 and the MoE
// decode kernels of qmm.hip:5578-6054; CPU math overlays/cpu/mlx/backend/cpu/
// quantized.cpp:199-257 affine, 550-597 mxfp4): y[m,n] = sum_g s[n,g] *
// sum_{k in g} x[m,k] q[n,k] (+ b[n,g] * sum_{k in g} x[m,k]), fp32
// accumulation, one bf16 rounding on store.
//
// The products run on v_mfma_f32_4x4x4bf16_1k, the 16-block matrix
// instruction: block b (lanes 4b..4b+3) multiplies 4 activation rows (lane
// 4b+i supplies row i) by 4 weight rows (lane 4b+j supplies column j and gets
// D[0..3][j] back) over 4 k.  So one wave-load instruction is 4 weight rows x
// 256 contiguous bytes (lane 4b+j reads piece b of row j), each lane keeps its
// own row, and the matrix core does the multiply-adds the row-streaming
// kernel spends v_dot2 instructions on.  Per 16-byte piece a lane does:
//   * unpack: AFF4 "128 + q" bf16 pairs (one byte permute per pair, the activations
//     permuted to match), AFF8 byte -> f32 -> bf16, MXFP4 the gfx950 scaled
//     fp4 conversion with the e8m0 scale folded in (exact);
//   * KL/4 MFMAs per set of 4 activation rows, C starting at 0;
//   * fold (affine): y += s * D + (b - 128 s) * sum(x) per activation row —
//     a piece lies inside one quantization group; MXFP4 adds D (the scale is
//     already in the weights) or, for the e8m0 codes 0 and 255, s * D.
// A workgroup owns 4 RG weight rows; its waves split K into chunks of 16
// pieces, issue every load before any arithmetic, and reduce across pieces
// with DPP row rotations and across waves through LDS in a fixed order
// (bitwise reproducible).  Bounds-checked buffer loads return 0 past the end
// of an operand, which covers ragged N, partial chunks and missing
// activation rows without branches.
// gather_qmm runs the same pass (b4_pass) per index entry, per expert
// segment, per run of a sorted index list, or, in qmv_b4_search_kernel, per
// expert (grid.y) over the entries a binary search of the sorted indices
// finds for it.
#include "common.hpp"
#include "kernels.hpp"

namespace mlxq {

namespace {

// The 4x4x4 accumulation chains are written as inline assembly so their
// registers are fixed: the compiler's own allocation of these chains can put
// an instruction's destination partly over its C (or A) operand, and on
// gfx950 that gives wrong sums.  Here the destination is the C operand
// itself (tied), and a chain's first instruction (C = 0) gets an
// early-clobber destination apart from A and B.  The compiler does not see
// an MFMA inside the assembly, so the wait states it would insert are
// spelled out: 2 before every MFMA (operands just written by the VALU) and
// 16 after a chain before the VALU reads its result (mfma4_done).
__device__ __forceinline__ f32x4 mfma4_first(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1) {
  const u32x2 a = {a0, a1}, b = {b0, b1};
  f32x4 d;
  asm("s_nop 1\n\tv_mfma_f32_4x4x4_16b_bf16 %0, %1, %2, 0" : "=&v"(d) : "v"(a), "v"(b));
  return d;
}
__device__ __forceinline__ void mfma4_acc(f32x4& d, uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1) {
  const u32x2 a = {a0, a1}, b = {b0, b1};
  asm("s_nop 1\n\tv_mfma_f32_4x4x4_16b_bf16 %0, %1, %2, %0" : "+v"(d) : "v"(a), "v"(b));
}
__device__ __forceinline__ void mfma4_done(f32x4& d) { asm volatile("s_nop 7\n\ts_nop 7" : "+v"(d)); }

}  // namespace

// A lane's weight pieces and their scale (and bias) codes for one pass.
template <int RG, int CPW>
struct B4Weights {
  u32x4 wv[CPW][RG];
  uint32_t sraw[CPW][RG], braw[CPW][RG];
};

// Issues the scale, bias and weight loads of the workgroup's 4 RG weight rows
// of `expert` (lane pieces as in b4_pass); they do not depend on which
// activation rows the pass takes.
template <int FMT, int RG, int CPW>
__device__ __forceinline__ void b4_load_weights(const QmvArgs& a, int gs_shift, int expert, int tid,
                                                B4Weights<RG, CPW>& W) {
  constexpr bool AFF = FMT != MXFP4;
  constexpr int BITS = FMT == AFF8 ? 8 : 4;
  constexpr int KL = 128 / BITS;
  const int NW = blockDim.x >> 6;
  const int lane = tid & 63, wave = tid >> 6, b = lane >> 2, j = lane & 3;
  const int N = a.N, K = a.K;
  const int row0 = blockIdx.x * (4 * RG);
  const int nlc = K / KL;
  const uint32_t RB = (uint32_t)nlc * 16u;
  const int G = K >> gs_shift;
  constexpr int ESZ = AFF ? 2 : 1;
  const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(a.w + (int64_t)expert * a.w_expert_stride, (uint32_t)N * RB);
  const int64_t sb0 = (int64_t)expert * a.s_expert_stride;
  const __amdgpu_buffer_rsrc_t sr =
      buffer_rsrc(reinterpret_cast<const uint8_t*>(a.scales) + sb0 * ESZ, (uint32_t)(N * G * ESZ));
  const __amdgpu_buffer_rsrc_t br =
      buffer_rsrc(AFF ? (const void*)(a.biases + sb0) : a.scales, (uint32_t)(AFF ? N * G * 2 : 0));
#pragma unroll
  for (int c = 0; c < CPW; c++) {
    const int pc = (wave + NW * c) * 16 + b;
    const bool live = pc < nlc;
#pragma unroll
    for (int g = 0; g < RG; g++) {
      const int n = row0 + 4 * g + j;
      const uint32_t og = (uint32_t)(n * G + ((pc * KL) >> gs_shift));  // in groups
      const uint32_t ob = (live && n < N) ? og * (uint32_t)ESZ : kDeadOfs;
      if constexpr (AFF) {
        W.sraw[c][g] = __builtin_amdgcn_raw_buffer_load_b16(sr, ob, 0, 0);
        W.braw[c][g] = __builtin_amdgcn_raw_buffer_load_b16(br, ob, 0, 0);
      } else {
        W.sraw[c][g] = __builtin_amdgcn_raw_buffer_load_b8(sr, ob, 0, 0);
        W.braw[c][g] = 0u;
      }
    }
  }
#pragma unroll
  for (int c = 0; c < CPW; c++) {
    const int pc = (wave + NW * c) * 16 + b;
    const bool live = pc < nlc;
#pragma unroll
    for (int g = 0; g < RG; g++) {
      const int n = row0 + 4 * g + j;
      const uint32_t o = (live && n < N) ? (uint32_t)n * RB + (uint32_t)pc * 16u : kDeadOfs;
      // default cache policy: measured faster than the streaming hint here
      W.wv[c][g] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, o, 0, 0));
    }
  }
}

// One pass: `count` activation rows starting at index entry / segment sidx
// against the workgroup's 4 RG weight rows of `expert`.  `tid` is
// threadIdx.x (see the expert-search kernel for why it is an argument).
// PRE: W already holds (or has in flight) this pass's weights, loaded by
// b4_load_weights; otherwise the pass loads them after its activations.
template <int FMT, int MS, int RG, int CPW, bool PRE = false>
__device__ __forceinline__ void b4_pass(const QmvArgs& a, int gs_shift, float* red, int sidx, int count,
                                        int expert, int tid, B4Weights<RG, CPW>& W) {
  constexpr bool AFF = FMT != MXFP4;
  constexpr int BITS = FMT == AFF8 ? 8 : 4;
  constexpr int KL = 128 / BITS;  // K values per 16-byte piece
  constexpr int XV = KL / 8;      // 16-byte activation loads per piece and row
  constexpr int NQ = KL / 4;      // MFMAs (4 k each) per piece and row set
  constexpr int V = MS * RG * 4;  // partial sums per lane
  const int NW = blockDim.x >> 6;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int b = lane >> 2;  // piece within the chunk
  const int j = lane & 3;   // weight row within a group / activation row within a set
  const int xbatch = seg_index(a.lhs, a.lhs_stride, sidx, a.X, a.lhs_div > 1 ? sidx / a.lhs_div : sidx);

  const int N = a.N;
  const int K = a.K;
  const int row0 = blockIdx.x * (4 * RG);
  const int nlc = K / KL;                   // pieces per row
  const uint32_t RB = (uint32_t)nlc * 16u;  // bytes per weight row
  const int G = K >> gs_shift;
  constexpr int ESZ = AFF ? 2 : 1;

  const __amdgpu_buffer_rsrc_t xr =
      buffer_rsrc(a.x + (int64_t)xbatch * a.rps * K, (uint32_t)count * (uint32_t)K * 2u);

  // pieces of this lane: chunk (wave + NW c), piece b
  int pc[CPW];
  bool live[CPW];
#pragma unroll
  for (int c = 0; c < CPW; c++) {
    pc[c] = (wave + NW * c) * 16 + b;
    live[c] = pc[c] < nlc;
  }

  // ---- 1. loads: activations, scales, then weights (all before any math) ----
  u32x4 xv[CPW][MS][XV];
#pragma unroll
  for (int c = 0; c < CPW; c++)
#pragma unroll
    for (int s = 0; s < MS; s++)
#pragma unroll
      for (int v = 0; v < XV; v++) {
        const uint32_t o = live[c] ? (uint32_t)((4 * s + j) * K + pc[c] * KL) * 2u + (uint32_t)v * 16u : kDeadOfs;
        xv[c][s][v] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, o, 0, 0));
      }
  if constexpr (!PRE) b4_load_weights<FMT, RG, CPW>(a, gs_shift, expert, tid, W);
  __builtin_amdgcn_sched_barrier(0);  // keep the arithmetic below the loads

  // ---- 2. activation operands and sums ---------------------------------------
  // xs[c][s]: sums of activation rows 4s + 0..3 over this lane's piece (affine)
  f32x4 xs[CPW][MS];
#pragma unroll
  for (int c = 0; c < CPW; c++)
#pragma unroll
    for (int s = 0; s < MS; s++) {
      xs[c][s] = f32x4{0.f, 0.f, 0.f, 0.f};
      if constexpr (AFF) {
        float own = 0.f;
#pragma unroll
        for (int v = 0; v < XV; v++)
#pragma unroll
          for (int e = 0; e < 4; e++) own = dot2(xv[c][s][v][e], 0x3F803F80u, own);  // pairs times (1, 1)
        // the quad's four rows, broadcast from lanes 4b + 0..3
        xs[c][s] = f32x4{dpp<0x00>(own), dpp<0x55>(own), dpp<0xAA>(own), dpp<0xFF>(own)};
      }
      if constexpr (FMT == AFF4) {
#pragma unroll
        for (int v = 0; v < XV; v++) xv[c][s][v] = perm_aff4_v(xv[c][s][v]);
      }
    }

  // ---- 3. products and folds --------------------------------------------------
  f32x4 y[MS][RG];
#pragma unroll
  for (int s = 0; s < MS; s++)
#pragma unroll
    for (int g = 0; g < RG; g++) y[s][g] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int c = 0; c < CPW; c++)
#pragma unroll
    for (int g = 0; g < RG; g++) {
      uint32_t pr[KL / 2];  // bf16 pairs of this piece (AFF4 in "128 + q" pair order)
      const u32x4 w = W.wv[c][g];
      if constexpr (FMT == AFF4) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
          uint32_t t[4];
          unpack_aff4(w[q], t);
#pragma unroll
          for (int e = 0; e < 4; e++) pr[4 * q + e] = t[e];
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
        // A normal e8m0 scale is folded into the conversion (fp4 code points
        // times 2^k are exact in bf16) and the fold adds D.  2^-127 and NaN
        // (e8m0 0 and 255) are applied to D in fp32 instead, as MLX applies
        // the scale to the group sum: the products stay out of bf16's
        // subnormal range.  One conversion either way (scale 1 for those two
        // codes): a per-lane branch between two conversions compiled to
        // exec-masked blocks that kept the scheduler from overlapping pieces.
        const uint32_t sb = W.sraw[c][g];
        const float cs = sb - 1u < 254u ? e8m0_to_f32(sb) : 1.0f;
#pragma unroll
        for (int q = 0; q < 4; q++) unpack_mxfp4_scaled(w[q], cs, &pr[4 * q]);
      }
      float sc = 0.f, bp = 0.f;
      if constexpr (AFF) {
        sc = bf16_bits_to_f32(W.sraw[c][g] & 0xFFFFu);
        const float bi = bf16_bits_to_f32(W.braw[c][g] & 0xFFFFu);
        bp = FMT == AFF4 ? __builtin_fmaf(-128.0f, sc, bi) : bi;
        if (!live[c] || row0 + 4 * g + j >= N) sc = bp = 0.f;  // dead pieces add exactly 0
      } else {
        const uint32_t sb = W.sraw[c][g];
        sc = sb - 1u < 254u ? 1.0f : e8m0_to_f32(sb);  // scale still to apply to D
      }
      // The MS accumulator chains advance together (quad q of every row set
      // before quad q + 1), so all of them are live at once and each keeps
      // its own registers: a chain whose destination is allocated partly
      // over its own C or A operand gives wrong results on gfx950.
      f32x4 d[MS];
#pragma unroll
      for (int q = 0; q < NQ; q++)
#pragma unroll
        for (int s = 0; s < MS; s++) {
          const uint32_t x0 = xv[c][s][q >> 1][(q & 1) * 2], x1 = xv[c][s][q >> 1][(q & 1) * 2 + 1];
          if (q == 0) d[s] = mfma4_first(x0, x1, pr[0], pr[1]);
          else mfma4_acc(d[s], x0, x1, pr[2 * q], pr[2 * q + 1]);
        }
#pragma unroll
      for (int s = 0; s < MS; s++) {
        mfma4_done(d[s]);
#pragma unroll
        for (int r = 0; r < 4; r++) {
          if constexpr (AFF) y[s][g][r] = __builtin_fmaf(sc, d[s][r], __builtin_fmaf(bp, xs[c][s][r], y[s][g][r]));
          else y[s][g][r] = __builtin_fmaf(sc, d[s][r], y[s][g][r]);
        }
      }
    }

  // ---- 4. reduce: the 4 pieces of a 16-lane row (DPP), then rows and waves (LDS)
  // lane 4b + j holds y[s][g][r] = partial of activation row 4s + r, weight row
  // row0 + 4g + j; lanes with equal j in a row of 16 cover pieces b, b+1..b+3
#pragma unroll
  for (int s = 0; s < MS; s++)
#pragma unroll
    for (int g = 0; g < RG; g++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        float v = y[s][g][r];
        v += dpp<0x124>(v);  // row_ror:4
        v += dpp<0x128>(v);  // row_ror:8
        y[s][g][r] = v;
      }
  if ((lane & 15) < 4) {
    float* dst = red + ((wave * 4 + (lane >> 4)) * V) * 4 + j;
#pragma unroll
    for (int s = 0; s < MS; s++)
#pragma unroll
      for (int g = 0; g < RG; g++)
#pragma unroll
        for (int r = 0; r < 4; r++) dst[((s * RG + g) * 4 + r) * 4] = y[s][g][r];
  }
  __syncthreads();
  // entry t < 4 V: value (s, g, r) = t / 4, column j = t % 4
  for (int t = threadIdx.x; t < 4 * V; t += blockDim.x) {
    float tot = 0.f;
    for (int q = 0; q < NW * 4; q++) tot += red[q * V * 4 + t];
    const int col = t & 3, idx = t >> 2;
    const int r = idx & 3, g = (idx >> 2) % RG, s = (idx >> 2) / RG;
    const int m = 4 * s + r, n = row0 + 4 * g + col;
    if (n < N && m < count) a.out[((int64_t)sidx * a.rps + m) * N + n] = (uint16_t)f32_to_bf16_bits(tot);
  }
}

// FMT: weight format; MS: sets of 4 activation rows (1, 2 or 4); RG: groups
// of 4 weight rows per workgroup; CPW: 16-piece K chunks per wave.
template <int FMT, int MS, int RG, int CPW>
__global__ __launch_bounds__(512) void qmv_b4_kernel(const QmvArgs a, int gs_shift) {
  extern __shared__ __align__(16) float red[];  // [wave][row of 16 lanes][V][4 columns]
  const int sidx = blockIdx.y;
  int count = min(a.rps, a.total_rows - sidx * a.rps);
  if (count <= 0) return;
  const int expert = seg_index(a.rhs, a.rhs_stride, sidx, a.E, a.w_expert_stride ? sidx : 0);
  if (a.runs) {
    // Expert runs of a sorted gather (one activation row per entry, 4 MS >=
    // a.runs rows compiled): entry sidx starts a segment where the expert
    // changes or at a multiple of a.runs, and the segment takes the following
    // entries of the same expert up to the next multiple; other workgroups
    // exit.
    const int cap = a.runs;
    if (sidx % cap != 0 && seg_index(a.rhs, a.rhs_stride, sidx - 1, a.E, 0) == expert) return;
    count = 1;
    while (count < cap && (sidx + count) % cap != 0 && sidx + count < a.total_rows &&
           seg_index(a.rhs, a.rhs_stride, sidx + count, a.E, 0) == expert)
      count++;
  }
  B4Weights<RG, CPW> W;
  b4_pass<FMT, MS, RG, CPW>(a, gs_shift, red, sidx, count, expert, threadIdx.x, W);
}

// Sorted gather with one activation row per entry, one workgroup row per
// expert (blockIdx.y): the expert finds its entries [first, end) by binary
// search in the sorted indices (as the reference's find_sorted_expert_run,
// rocm/quantized/qmm.hip:4741-4915) and takes them 4 MS at a time, so its
// weights stream once per 4 MS entries; experts without entries exit.  The
// first pass's weights do not depend on the search: they are issued right
// behind the search's first loads, so their stream overlaps the search and
// the activation loads (for an expert without entries they are read for
// nothing).  Every per-lane value of a later pass is derived from a thread
// index the compiler cannot see through: hoisted out of the pass loop, the
// pass's addresses would stay live across passes and cost a wave per SIMD.
template <int FMT, int MS, int RG, int CPW>
__global__ __launch_bounds__(512) void qmv_b4_search_kernel(const QmvArgs a, int gs_shift) {
  extern __shared__ __align__(16) float red[];
  const int expert = blockIdx.y;
  int first, end;
  B4Weights<RG, CPW> W;
  sorted_run(a.rhs, a.rhs_stride, a.total_rows, a.E, expert, threadIdx.x & 63, first, end,
             [&]() { b4_load_weights<FMT, RG, CPW>(a, gs_shift, expert, threadIdx.x, W); });
  if (first >= end) return;
  b4_pass<FMT, MS, RG, CPW, true>(a, gs_shift, red, first, min(4 * MS, end - first), expert, threadIdx.x, W);
  for (int s = first + 4 * MS; s < end; s += 4 * MS) {  // workgroup-uniform
    __syncthreads();  // the previous pass has read its reduction
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    B4Weights<RG, CPW> Wn;
    b4_pass<FMT, MS, RG, CPW>(a, gs_shift, red, s, min(4 * MS, end - s), expert, tid, Wn);
  }
}

// ---- host ------------------------------------------------------------------

namespace {

// a.runs < 0 (expert search, grid.y = experts): the search kernel, compiled
// for one set of 4 activation rows per pass
template <int FMT, int MS>
hipError_t b4_launch_ms(const QmvB4Plan& p, const QmvArgs& a, int gs_shift, dim3 grid, hipStream_t stream) {
  const dim3 block((unsigned)(p.nw * 64));
  if (MS != 1 && a.runs < 0) return hipErrorInvalidValue;
#define B4_CASE(RG_, CPW_)                                                                                      \
  if (p.rg == RG_ && p.cpw == CPW_) {                                                                           \
    if (MS == 1 && a.runs < 0)                                                                                  \
      hipLaunchKernelGGL((qmv_b4_search_kernel<FMT, 1, RG_, CPW_>), grid, block, p.lds, stream, a, gs_shift); \
    else                                                                                                        \
      hipLaunchKernelGGL((qmv_b4_kernel<FMT, MS, RG_, CPW_>), grid, block, p.lds, stream, a, gs_shift);        \
    return hipGetLastError();                                                                                   \
  }
  B4_CASE(1, 1)
  B4_CASE(2, 1)
  B4_CASE(4, 1)
  B4_CASE(8, 1)
  B4_CASE(1, 2)
  B4_CASE(2, 2)
  B4_CASE(4, 2)
  B4_CASE(1, 4)
  B4_CASE(2, 4)
  B4_CASE(1, 8)
#undef B4_CASE
  return hipErrorInvalidValue;
}

template <int FMT>
hipError_t b4_launch_fmt(const QmvB4Plan& p, const QmvArgs& a, int gs_shift, dim3 grid, hipStream_t stream) {
  switch (p.ms) {
    case 1: return b4_launch_ms<FMT, 1>(p, a, gs_shift, grid, stream);
    case 2: return b4_launch_ms<FMT, 2>(p, a, gs_shift, grid, stream);
    default: return b4_launch_ms<FMT, 4>(p, a, gs_shift, grid, stream);
  }
}

bool b4_valid(int ms, int rg, int cpw) {
  if (ms != 1 && ms != 2 && ms != 4) return false;
  if (ms == 4 && rg == 4 && cpw == 2) return false;  // spills
  if (cpw == 1 && rg == 8) return ms <= 2;
  if (cpw == 1 || cpw == 2) return rg == 1 || rg == 2 || rg == 4;
  if (cpw == 4) return rg == 1 || rg == 2;
  if (cpw == 8) return rg == 1;
  return false;
}

}  // namespace

QmvB4Plan qmv_b4_plan(int fmt, int gs, int64_t N, int64_t K, int rows, int rg_req, int cpw_req) {
  QmvB4Plan p;
  const int kl = fmt == AFF8 ? 16 : 32;
  if (rows < 1 || rows > 16 || K % kl != 0 || K % gs != 0 || gs < kl) return p;
  p.ms = rows <= 4 ? 1 : (rows <= 8 ? 2 : 4);
  const int64_t nlc = K / kl;
  const int64_t chunks = (nlc + 15) / 16;
  // at most 8 waves (256 VGPRs each); a wave holds RG * CPW weight pieces
  // and MS * CPW * (kl / 8) activation pieces in registers
  p.cpw = chunks <= 8 ? 1 : (chunks <= 16 ? 2 : (chunks <= 32 ? 4 : 8));
  if (chunks > 64) return p;
  const int xregs = p.ms * p.cpw * (kl / 8) * 4;
  if (xregs > 128) return p;
  // weight rows per workgroup: each lane's activations are reused across its
  // RG weight pieces, so more rows cut the activation re-reads (L2 -> CU
  // traffic of 64 MS bytes per lane and piece against 16 RG of weights)
  p.rg = p.ms == 4 ? 1 : (p.ms == 2 ? (p.cpw >= 4 ? 1 : 4) : (p.cpw >= 4 ? 8 / p.cpw : (p.cpw == 1 ? 8 : 4)));
  if (cpw_req > 0) p.cpw = cpw_req;
  if (rg_req > 0) p.rg = rg_req;
  p.nw = (int)((chunks + p.cpw - 1) / p.cpw);
  p.tiles = (int)((N + 4 * p.rg - 1) / (4 * p.rg));
  p.lds = (size_t)p.nw * 4 * (p.ms * p.rg * 4) * 4 * sizeof(float);
  // buffer offsets are 32-bit and 0x80000000 marks a dead lane: every operand
  // of one launch must stay below 2 GiB
  const int64_t wbytes = N * nlc * 16, sbytes = N * (K / gs) * 2;
  // registers per lane: activations, weights, activation sums, partials, scales
  const int regs = p.ms * p.cpw * (kl / 8) * 4 + p.rg * p.cpw * 4 + p.ms * p.cpw * 4 + p.ms * p.rg * 4 +
                   p.rg * p.cpw * 2;
  p.ok = b4_valid(p.ms, p.rg, p.cpw) && regs <= 200 && p.nw <= 8 && (int64_t)p.nw * p.cpw * 16 >= nlc &&
         p.lds <= kQmvLdsMax &&
         wbytes + 4 * p.rg * nlc * 16 < ((int64_t)1 << 31) && sbytes < ((int64_t)1 << 31) &&
         (int64_t)16 * K * 2 < ((int64_t)1 << 31);
  return p;
}

hipError_t qmv_b4_launch(int fmt, int gs, const QmvArgs& a, int nseg, const QmvB4Plan& p, hipStream_t stream) {
  if (!p.ok) return hipErrorInvalidValue;
  const int gs_shift = log2i(gs);
  const dim3 grid((unsigned)p.tiles, (unsigned)nseg, 1);
  switch (fmt) {
    case AFF4: return b4_launch_fmt<AFF4>(p, a, gs_shift, grid, stream);
    case AFF8: return b4_launch_fmt<AFF8>(p, a, gs_shift, grid, stream);
    default: return b4_launch_fmt<MXFP4>(p, a, gs_shift, grid, stream);
  }
}

}  // namespace mlxq
