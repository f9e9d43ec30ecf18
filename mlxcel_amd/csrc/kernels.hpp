// kernels.hpp — launch interfaces between the C-ABI host layer (api.cpp) and
// the gfx950 kernels.  Plain data structs; no torch or MLX types.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mlxq.h"

namespace mlxq {

// Skinny (decode) quantized matmul over segments of rows sharing one weight
// matrix: segment s = output rows [s*rps, s*rps + rps), activations from x
// batch lhs[s] (or s), weight matrix rhs[s] (or s when w_expert_stride != 0,
// else 0).
struct QmvArgs {
  const uint16_t* x;        // bf16 activations, rows of K
  const uint32_t* w;        // packed codes [E][N][K*bits/32]
  const void* scales;       // bf16 (affine) or uint8 e8m0 (mxfp4) [E][N][K/gs]
  const uint16_t* biases;   // bf16 [E][N][K/gs] (affine only)
  uint16_t* out;            // bf16 [out_rows][N]
  float* ws;                // split-K partials [ks][out_rows][N] (ks > 1), summed by a second kernel
  const uint32_t* lhs;      // x batch index per segment (nullable)
  const uint32_t* rhs;      // expert per segment (nullable)
  // Index element strides in 32-bit words (1: 32-bit indices, 2: 64-bit,
  // low word read; 0 counts as 1) and, with no lhs, the divisor that maps a
  // segment to its x batch (x batch = segment / lhs_div; 0 counts as 1).
  int lhs_stride, rhs_stride, lhs_div;
  int N;
  int K;
  int64_t w_expert_stride;  // uint32 words per weight matrix (0: one matrix)
  int64_t s_expert_stride;  // scale/bias elements per weight matrix
  int E;                    // weight matrices (index clamp)
  int X;                    // x batches (index clamp)
  int rps;                  // rows per segment
  int total_rows;           // total rows
  int out_rows;             // rows of `out` (split-K workspace stride)
  int rows_lds;             // activation rows staged per workgroup (>= rows of any segment)
  int ks;                   // workgroups splitting K (gridDim.z)
  int kst_per_wg;           // K-steps per workgroup
  // Gathers grouped by expert (qmv.hip MFMA kernel only): segment table and
  // per-row indirection built by launch_group_by_expert; null otherwise.
  const uint32_t* seg;      // [max segments][3] = {expert, first grouped row, rows}
  const uint32_t* nseg_dev; // segments in the table
  const uint32_t* xrows;    // grouped row -> x row (flattened over x's batch)
  const uint32_t* orows;    // grouped row -> output row
  int xt;                   // element type of x / scales / biases / out: 0 bfloat16, 1 float16
                            // (float16: the row-streaming kernel's dense entry only)
  // Sorted gathers (rps == 1): positive = segments are runs of equal experts
  // among consecutive entries, at most `runs` entries each (row-streaming
  // kernel: 4; block-MFMA kernel: up to its 4 MS rows).  -1 (block-MFMA
  // kernel, MS = 1): blockIdx.y is an expert, which finds its entries by
  // binary search in the sorted indices and takes them 4 at a time.
  int runs;
};

struct QmvPlan {
  int ks = 1;          // workgroups splitting K (gridDim.z)
  int kst_per_wg = 1;  // K-steps per workgroup
  int tiles = 1;       // 16-column tiles
  int nw = 4;          // waves per workgroup
  int p = 4;           // K-steps per wave, all loaded up front (TK)
  int mt = 1;          // 16-row MFMA tiles
  size_t lds = 0;      // dynamic LDS bytes
};

extern const uint32_t kQmvLdsMax;  // bytes of LDS one workgroup may use
int qmv_slots(int fmt, int gs);
int qmv_tile_mt(int fmt, int gs, int rows);
int qmv_max_rows(int fmt, int gs);
// nw/tk: requested waves per workgroup and K-steps per wave (invalid -> defaults).
QmvPlan qmv_plan(int fmt, int gs, int64_t N, int64_t K, int rows_lds, int nseg, int num_cus, int nw, int p);
// Launches the kernel (and, when p.ks > 1, the split-K reduction kernel).
hipError_t qmv_launch(int fmt, int gs, const QmvArgs& a, int nseg_slots, const QmvPlan& p, hipStream_t stream);

// Row-streaming decode kernel (qmv_rs.hip) for 1 to 4 activation rows per
// weight matrix: R weight rows per workgroup, one wave per 1 KiB chunk of a
// row (CPW chunks per wave when a row has more than 8).
// Several projections of the same activations in one row-streaming launch
// (q/k/v, gate/up): matrix p owns the workgroups [tile_end[p-1], tile_end[p])
// of the grid's x dimension; n <= 1 means the QmvArgs matrix alone.
constexpr int kQmvMultiMax = 4;
struct QmvMulti {
  int n;
  int tile_end[kQmvMultiMax];
  int N[kQmvMultiMax];
  const uint32_t* w[kQmvMultiMax];
  const void* scales[kQmvMultiMax];
  const uint16_t* biases[kQmvMultiMax];
  uint16_t* out[kQmvMultiMax];
};
struct QmvRsPlan {
  bool ok = false;  // false: use qmv_plan / qmv_launch
  int mr = 1;       // activation rows compiled for (1, 2 or 4)
  int r = 8;        // weight rows per workgroup
  int cpw = 1;      // 1 KiB chunks per wave and row
  int nw = 1;       // waves per workgroup
  int tiles = 1;    // workgroups along N
  size_t lds = 0;   // dynamic LDS bytes (staged scales + reduction)
};
// r_req: requested rows per workgroup (0 or invalid -> default).
QmvRsPlan qmv_rs_plan(int fmt, int gs, int64_t N, int64_t K, int rows, int r_req);
hipError_t qmv_rs_launch(int fmt, int gs, const QmvArgs& a, int nseg, const QmvRsPlan& p, hipStream_t stream,
                         const QmvMulti* multi = nullptr);

// Strided copy (copy.hip): dst[idx] = src[idx] over an N-d view, strides
// in elements on both sides.
struct CopyArgs {
  const void* src;
  void* dst;
  int ndim, esz;
  int64_t n;
  int64_t shape[MLXQ_MAX_DIMS];
  int64_t src_strides[MLXQ_MAX_DIMS];
  int64_t dst_strides[MLXQ_MAX_DIMS];
};
hipError_t launch_strided_copy(const CopyArgs& a, hipStream_t stream);

// General quantized matmul (qmm_gen.hip): float16 / bfloat16 / float32
// activations and scales, affine codes of 2-8 bits, mxfp4, both transposes,
// gather segments.  Element types of x / scales / result:
enum GenType : int { GEN_BF16 = 0, GEN_F16 = 1, GEN_F32 = 2 };
enum GenMode : int { GEN_AFFINE = 0, GEN_MXFP4 = 1 };
struct GenArgs {
  const void* x;            // [X][M][K] of x_dtype
  const uint32_t* w;        // [E][N][K*bits/32] (transpose) or [E][K][N*bits/32]
  const void* scales;       // [E][N][K/gs] or [E][K][N/gs] of s_dtype (uint8 e8m0 for mxfp4)
  const void* biases;       // like scales (affine)
  void* out;                // [nseg][M][N] of the compute type
  float* ws;                // [ks][nseg*M*N] fp32 partials when ks > 1
  const uint32_t* lhs;      // x batch per segment (null: segment s, or 0 when X == 1)
  const uint32_t* rhs;      // weight matrix per segment (null: segment s, or 0 when E == 1)
  int x_dtype, s_dtype, b_dtype;  // GenType
  int mode;                 // GenMode
  int bits, gs_shift;
  int M, N, K;              // rows per segment, output columns, reduction length
  int X, E;                 // index clamps
  int x_vec;                // K % 8 == 0: 8 activations per vector load
  int64_t w_expert_stride;  // words per weight matrix
  int64_t s_expert_stride;  // scale elements per weight matrix
  int64_t out_elems;        // nseg * M * N (partial stride)
  int tiles_m, ks, ksteps_per_split;  // set by qmm_gen_launch from the plan
};
struct GenPlan {
  bool ok = false;
  int bm = 16;              // rows per tile (16 or 64)
  int tiles_m = 1, tiles_n = 1;
  int ks = 1;               // K splits
  int ksteps_per_split = 1; // 32-position steps per split
};
// ks_req > 0 forces the K split (tests)
GenPlan gen_plan(int64_t M, int64_t N, int64_t K, int64_t nseg, int cus, int ks_req);
// tc: GenType of the MFMA inputs and of `out`
hipError_t qmm_gen_launch(const GenArgs& a, const GenPlan& p, int tc, bool transpose, int64_t nseg,
                          hipStream_t stream);
hipError_t launch_gen_reduce(const float* ws, void* out, int64_t n, int ks, int tc, hipStream_t stream);
// Decode form of the general path (qmm_gen.hip): 1-4 rows per segment,
// transpose=true, affine codes of 1-6 or 8 bits, K a multiple of 32; one
// wave per 4 weight rows, no workspace.  x may be any GenType (scales and
// biases too); tc is the result type.
bool qmv_gen_fits(int mode, bool transpose, int64_t M, int64_t N, int64_t K, int64_t nseg, int bits);
hipError_t qmv_gen_launch(const GenArgs& a, int tc, int64_t nseg, hipStream_t stream);
// transpose=false decode (qmm_gen.hip): 1-2 rows, affine codes of 1-6 or 8
// bits, N a multiple of 32; workgroups of 8 waves over 64 column pieces of
// 32 and one K range of `kper` code rows; ks > 1 ranges write fp32 partials
// ([ks][out_elems] in a.ws) for launch_gen_reduce.
struct GenTPlan {
  bool ok = false;
  int blocks = 0;  // workgroups along N
  int ks = 1;      // K ranges
  int kper = 0;    // code rows per range
};
GenTPlan qmv_gen_t_plan(int64_t M, int64_t N, int64_t K, int64_t nseg, int bits, int mode, int cus);
hipError_t qmv_gen_t_launch(const GenArgs& a, const GenTPlan& p, int tc, int64_t nseg, hipStream_t stream);
// dequantize for every element type (dequant.hip): affine codes of 2-8 bits
// with scales/biases of type ts, or mxfp4 (mode GEN_MXFP4) to float16/float32;
// `to` is the output type.  K a multiple of 32.
hipError_t launch_gen_dequantize(int mode, const uint32_t* w, const void* scales, const void* biases, void* out,
                                 int64_t rows, int64_t K, int gs, int bits, int ts, int to, hipStream_t stream);

// Block-MFMA decode kernel (qmv_b4.hip) for 1 to 16 activation rows per
// weight matrix: v_mfma_f32_4x4x4bf16_1k over 4 weight rows x 256-byte pieces
// per wave-load, RG groups of 4 rows per workgroup, waves split K in chunks
// of 16 pieces (CPW chunks per wave).
struct QmvB4Plan {
  bool ok = false;  // false: shape not covered
  int ms = 1;       // sets of 4 activation rows compiled for (1, 2 or 4)
  int rg = 4;       // groups of 4 weight rows per workgroup
  int cpw = 1;      // chunks per wave
  int nw = 1;       // waves per workgroup
  int tiles = 1;    // workgroups along N
  size_t lds = 0;   // dynamic LDS bytes (cross-wave reduction)
};
// rg_req / cpw_req: requested shape (0 -> default)
QmvB4Plan qmv_b4_plan(int fmt, int gs, int64_t N, int64_t K, int rows, int rg_req, int cpw_req);
hipError_t qmv_b4_launch(int fmt, int gs, const QmvArgs& a, int nseg, const QmvB4Plan& p, hipStream_t stream);

// Mid-size decode (qmv_mid.hip): 1-16 activation rows against one affine
// 4/8-bit weight matrix; workgroups of 128 weight rows x one K range of 8
// windows; fp32 partials of several K ranges are added by launch_splitk_reduce.
//
// Several 2-D matrices of one activation block in one launch (q/k/v,
// gate/up; the mid-size and whole-row kernels): matrix p owns the row blocks
// [blk_end[p-1], blk_end[p]) of the grid's x dimension and, in the split-K
// partials, the columns [noff[p], noff[p] + N[p]) of a [ks][M][ntot] array.
// n <= 1: the kernel's own w / scales / biases / out / N fields alone.
struct QmvMatTable {
  int n;
  int ntot;  // sum of N over the matrices (the partials' row length)
  int blk_end[kQmvMultiMax];
  int N[kQmvMultiMax];
  int noff[kQmvMultiMax];
  const uint32_t* w[kQmvMultiMax];
  const uint16_t* scales[kQmvMultiMax];
  const uint16_t* biases[kQmvMultiMax];
  uint16_t* out[kQmvMultiMax];
};
// The matrix that row block `blk` of a launch belongs to (uniform): its
// operands, N, first column in the partials and the block's index inside it.
// Every table entry is read and selected, so the argument loads form one
// round.
struct QmvMat {
  const uint32_t* w;
  const uint16_t* scales;
  const uint16_t* biases;
  uint16_t* out;
  int N, noff, blk;
};
__device__ __forceinline__ QmvMat pick_matrix(const QmvMatTable& t, const uint32_t* w, const uint16_t* scales,
                                              const uint16_t* biases, uint16_t* out, int N, int blk) {
  QmvMat m{w, scales, biases, out, N, 0, blk};
  if (t.n > 1) {
    int p = 0;
#pragma unroll
    for (int i = 0; i < kQmvMultiMax - 1; i++) p += (i < t.n - 1 && blk >= t.blk_end[i]) ? 1 : 0;
#pragma unroll
    for (int i = 0; i < kQmvMultiMax; i++) {
      const bool on = p == i;
      m.w = on ? t.w[i] : m.w;
      m.scales = on ? t.scales[i] : m.scales;
      m.biases = on ? t.biases[i] : m.biases;
      m.out = on ? t.out[i] : m.out;
      m.N = on ? t.N[i] : m.N;
      m.noff = on ? t.noff[i] : m.noff;
      m.blk = on ? blk - (i > 0 ? t.blk_end[i - 1] : 0) : m.blk;
    }
  }
  return m;
}

struct QmvMidArgs {
  const uint16_t* x;       // bf16 [M][K]
  const uint32_t* w;       // packed codes [N][K*bits/32]
  const uint16_t* scales;  // bf16 [N][K/gs]
  const uint16_t* biases;  // bf16 [N][K/gs]
  uint16_t* out;           // bf16 [M][N]
  float* ws;               // fp32 partials [ks][M][N] (ks > 1)
  int M, N, K, gs_shift;
  int ks;                  // K ranges (gridDim.y)
  int xt;                  // 16-bit type of x / scales / biases / out: 0 bfloat16, 1 float16
  QmvMatTable mt;          // several matrices (mt.n > 1)
  int red_vec;             // outputs per thread of the split-K reduction (1, 2, 4; 0: default)
};
struct QmvMidLds {
  int xpitch = 0;  // bf16 per staged activation row
  uint32_t xl = 0, xs = 0, sc = 0, zero = 0, total = 0;  // byte offsets / size
};
struct QmvMidPlan {
  bool ok = false;
  int s = 1;           // quantization groups per 4-chunk window
  int na = 1;          // 16-row MFMA A tiles (activation row x group slot)
  int row_blocks = 0;  // workgroups along N (128 weight rows each)
  int kr = 0;          // K per workgroup
  int ks = 1;          // workgroups along K
  int sw = 8;          // scale groups per staging load
  size_t lds = 0;
};
// win_req 4 halves the K range per workgroup (8 windows otherwise); cus is
// kept for plans that weigh the grid against the CUs.
QmvMidPlan qmv_mid_plan(int fmt, int gs, int64_t N, int64_t K, int rows, int cus = 0, int win_req = 0);
// Launches the kernel and, with several K ranges, the fixed-order reduction.
hipError_t qmv_mid_launch(int fmt, const QmvMidArgs& a, const QmvMidPlan& p, hipStream_t stream);

// Mid-size decode over whole rows (qmv_mr.hip): 1-16 activation rows against
// one affine 4/8-bit weight matrix with enough rows for ~one workgroup of 64
// rows per CU; each wave finishes 16 outputs per activation row over all of K.
struct QmvMrArgs {
  const uint16_t* x;       // [M][K] of type xt
  const uint32_t* w;       // packed codes [N][K*bits/32]
  const uint16_t* scales;  // [N][K/gs] of type xt
  const uint16_t* biases;  // [N][K/gs] of type xt
  uint16_t* out;           // [M][N] of type xt
  int M, N, K, gs_shift;
  int xt;                  // 0 bfloat16, 1 float16
  QmvMatTable mt;          // several matrices (mt.n > 1)
};
struct QmvMrPlan {
  bool ok = false;
  int s = 1;           // quantization groups per 4-chunk window
  int na = 1;          // 16-row MFMA A tiles
  int xr = 8;          // activation rows staged (8 or 16)
  int rk = 1024;       // K positions per staged range
  int ring = 8;        // windows of weight loads in flight (4, 8 or 16)
  int row_blocks = 0;  // workgroups (64 weight rows each; 16 t with t > 0)
  int t = 0;           // 0: qmv_mr_kernel; 1-4: qmv_kq_kernel with t 16-row tiles per workgroup
  int nw = 8;          // qmv_kq_kernel: waves per workgroup
  size_t lds = 0;
};
// force: plan even when the matrix has too few rows to fill the CUs;
// ring_req: 4, 8 or 16 forces the weight ring depth in windows (0: planner)
QmvMrPlan qmv_mr_plan(int fmt, int gs, int64_t N, int64_t K, int rows, int cus, bool force, int ring_req);
// K split over the waves of a workgroup of 16 t rows (qmv_kq_kernel): t_req
// in 1-4 forces the tiles per workgroup; 0 takes the fewest that fit one
// round of the CUs (none: not planned).  Launched by qmv_mr_launch.
bool kq_tiles_ok(int t);
QmvMrPlan qmv_kq_plan(int fmt, int gs, int64_t N, int64_t K, int rows, int cus, int t_req, int nw_req = 0);
hipError_t qmv_mr_launch(int fmt, const QmvMrArgs& a, const QmvMrPlan& p, hipStream_t stream);

// Expert-sorted gather (qmm_group.hip), mxfp4, one activation row per index
// entry: a workgroup per (128 weight rows, expert) finds the expert's rows in
// the sorted indices and streams its weights once per 64 rows.
struct QmmGroupArgs {
  const uint16_t* x;       // bf16 [B][K], row b = entry b
  const uint32_t* w;       // packed codes [E][N][K/8]
  const uint8_t* scales;   // e8m0 [E][N][K/32]
  uint16_t* out;           // bf16 [B][N]
  const uint32_t* rhs;     // sorted expert per entry (32- or 64-bit, low word)
  int rhs_stride;          // 32-bit words per index (1 or 2)
  int N, K, E, B;
};
struct QmmGroupPlan {
  bool ok = false;
  int tiles = 2;       // 16-row weight tiles per wave: workgroups of 64 * tiles rows
  int row_blocks = 0;  // workgroups along N
  bool scale_table = false;  // K / 32 scale bytes per row fit the kernel's LDS table
};
// cus: the device's CUs; tiles_req 2 or 3 forces the workgroup rows (0: planner).
QmmGroupPlan qmm_group_plan(int fmt, int64_t N, int64_t K, int64_t E, int64_t B, int cus, int tiles_req = 0);
hipError_t qmm_group_launch(const QmmGroupArgs& a, const QmmGroupPlan& p, hipStream_t stream);

// Full-row decode kernel (qmv_fr.hip) for 1 or 2 activation rows per weight
// matrix: 8 waves per workgroup, R whole rows per wave, activations staged in
// LDS once per workgroup.
struct QmvFrPlan {
  bool ok = false;  // false: shape not covered
  int mr = 1;       // activation rows compiled for
  int r = 4;        // rows per wave
  int cmax = 2;     // 1 KiB chunks per row compiled for
  int chunks = 1;   // 1 KiB chunks per row
  int tiles = 1;    // workgroups along N
  size_t lds = 0;   // dynamic LDS bytes
};
QmvFrPlan qmv_fr_plan(int fmt, int gs, int64_t N, int64_t K, int rows, int r_req);
hipError_t qmv_fr_launch(int fmt, int gs, const QmvArgs& a, int nseg, const QmvFrPlan& p, hipStream_t stream);

// Prefill GEMM (qmm.hip): y[M, N] = x[M, K] @ dequant(w)[N, K]^T, 256 x 128
// output tiles, K split across workgroups when the grid is short.
// Stream-K counter words a launch may use (the caller's zeroed array holds
// at least this many).
constexpr int kSplitCounters = 1 << 16;

struct QmmArgs {
  const uint16_t* x;       // bf16 [M, K]
  const uint32_t* w;       // packed codes [N, K*bits/32]
  const void* scales;      // bf16 or e8m0 [N, K/gs]
  const uint16_t* biases;  // bf16 [N, K/gs] (affine)
  uint16_t* out;           // bf16 [M, N]
  float* ws;               // fp32 partials [ksplit, M, N] when ksplit > 1
  int M, N, K;
  int gs_shift;            // log2(group size)
  int ksplit;              // workgroups along K
  int ksteps_per_split;    // 64-wide K-steps per workgroup
  int x_rows;              // rows of x addressable (bounds of the x buffer)
  // Gathers grouped by expert: segment table / row indirection from
  // launch_group_by_expert (segments of at most the tile's rows) and the
  // per-expert strides of w (uint32 words) and scales/biases (elements).
  const uint32_t* seg;
  const uint32_t* nseg_dev;
  const uint32_t* xrows;
  const uint32_t* orows;
  int64_t w_expert_stride;
  int64_t s_expert_stride;
  // Tile walk of the 32x32-MFMA kernel (qmm_tile_kernel): output tiles per
  // dimension and whether consecutive tiles advance along M (1) or N (0).
  int tiles_m, tiles_n, m_fast;
  int xt;                  // 16-bit type of x / scales / biases / out: 0 bfloat16, 1 float16 (tile kernel, affine)
  int ldo;                 // row stride of out in elements (0: N); tile kernel without a K split
  // Stream-K (tile kernel, 256 x 256): workgroup b takes K-steps
  // [b sk_len, (b + 1) sk_len) of all tiles' steps laid end to end; a tile
  // split between two workgroups meets through fp32 partials in ws
  // (2 x gridDim.x x 256 x 256) and the per-boundary counters cnt
  // (gridDim.x, zero between launches).  sk_fallback forces the path a head
  // takes when its tail has not arrived (tests).
  int sk_len;
  int sk_fallback;
  uint32_t* cnt;
};
struct QmmPlan {
  bool ok = false;
  // output tile: 0 = 256 x 128, 1 = 256 x 256, 2 = 128 x 128, 3 = 64 x 128
  // (16x16-MFMA kernel); 4 = 256 x 256, 5 = 256 x 128, 6 = 128 x 128
  // (32x32-MFMA tile kernel)
  int tile = 0;
  int rows_per_tile = 256;
  int tiles_n = 1, tiles_m = 1, ksplit = 1, ksteps_per_split = 1;
  int m_fast = 0;  // tile kernel: consecutive workgroups walk along M
  // Two launches (tile2 >= 0): output columns [0, n_first) on `tile` in
  // whole rounds of the CUs, then [n_first, N) on the narrower tile2
  // (tiles_n2 tiles along N) in one round.  tiles_n is the first launch's.
  int tile2 = -1, n_first = 0, tiles_n2 = 0;
  // Stream-K (sk_len > 0): sk_wgs workgroups of sk_len K-steps each.
  int sk_len = 0, sk_wgs = 0;
};
// Counter words and fp32 partial bytes a stream-K plan needs.
inline int64_t qmm_sk_counters(const QmmPlan& p) { return p.sk_len > 0 ? p.sk_wgs : 0; }
inline int64_t qmm_sk_bytes(const QmmPlan& p) { return p.sk_len > 0 ? (int64_t)2 * p.sk_wgs * 256 * 256 * 4 : 0; }
// rows of x per output tile of a tile code (0 if unknown)
int qmm_tile_rows(int tile);
// Grouped gather: tiles along N for `tile`; tiles_m = segments is set by the caller.
QmmPlan qmm_plan_grouped(int fmt, int gs, int64_t N, int64_t K, int tile);
// tile_req / ksplit_req < 0 (or 0 for ksplit) choose by shape.
// mix: allow the two-launch plan (tile2) when neither tile nor split is requested;
// streamk: allow the stream-K plan there (it takes precedence).
QmmPlan qmm_plan(int fmt, int gs, int64_t M, int64_t N, int64_t K, int num_cus, int tile_req, int ksplit_req,
                 int mix = 1, int streamk = 0);
hipError_t qmm_launch(int fmt, const QmmArgs& a, const QmmPlan& p, hipStream_t stream);
// out[i] = bf16(sum over z < ks of ws[z * n + i]) (qmv.hip)
// out (16-bit type xt: 0 bfloat16, 1 float16) = sum over ks fp32 partials, in split order
hipError_t launch_splitk_reduce(const float* ws, uint16_t* out, int64_t n, int ks, hipStream_t stream, int xt = 0);
// The same sum over the partials [ks][M][t.ntot] of several matrices, each
// column written to its matrix's output (the split order as above).
hipError_t launch_splitk_reduce_multi(const float* ws, const QmvMatTable& t, int M, int ks, hipStream_t stream,
                                      int xt = 0, int vec = 0);

// Elementwise conversions (dequant.hip).
hipError_t launch_affine_dequantize(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                                    uint16_t* out, int64_t rows, int64_t K, int gs, int bits,
                                    hipStream_t stream);
hipError_t launch_mxfp4_dequantize(const uint32_t* w, const uint8_t* scales, uint16_t* out,
                                   int64_t rows, int64_t K, hipStream_t stream);
// affine quantize of bfloat16 / float16 / float32 weights (ti: GenType; the
// scales and biases are written in the same type), bits 1-6 or 8
hipError_t launch_affine_quantize(const void* w, int ti, uint32_t* wq, void* scales, void* biases, int64_t rows,
                                  int64_t K, int gs, int bits, hipStream_t stream);
// mxfp8 (e4m3 codes, e8m0 scales per 32) and nvfp4 (e2m1 codes, e4m3 scales per 16)
enum FpMode : int { FP_MXFP8 = 0, FP_NVFP4 = 1 };
hipError_t launch_fp_dequantize(int mode, const uint32_t* w, const uint8_t* scales, uint16_t* out, int64_t rows,
                                int64_t K, hipStream_t stream);
hipError_t launch_fp_quantize(int mode, const uint16_t* w, uint32_t* wq, uint8_t* scales, int64_t rows, int64_t K,
                              hipStream_t stream);
hipError_t launch_mxfp4_quantize(const uint16_t* w, uint32_t* wq, uint8_t* scales, int64_t rows,
                                 int64_t K, hipStream_t stream);

// Flat uint32 index arrays for gather: out[s][i] = index s at broadcast
// position i (data == nullptr: the default arange, value = location), cast to
// uint32 as the reference does (ops.cpp:100) and clamped to [0, clamp-1].
struct IdxPrepArgs {
  const void* data[2];
  int dtype[2];
  int64_t bstrides[2][MLXQ_MAX_DIMS];
  int64_t clamp[2];
  int64_t bshape[MLXQ_MAX_DIMS];
  int bnd;
  int64_t B;
  uint32_t* out[2];
};
hipError_t launch_index_prep(const IdxPrepArgs& a, hipStream_t stream);

// Groups B gather entries (flat uint32 lhs/rhs, rhs < E) by expert; see qmv.hip.
struct GroupArgs {
  const uint32_t* lhs;
  const uint32_t* rhs;
  int B, M, E, cap;
  uint32_t* xrows;  // [B*M]
  uint32_t* orows;  // [B*M]
  uint32_t* seg;    // [B*M/cap + min(E, B) + 1][3]
  uint32_t* nseg;   // [1]
};
constexpr int kGroupMaxExperts = 8192;  // LDS: (3 E + 1024) words
hipError_t launch_group_by_expert(const GroupArgs& a, hipStream_t stream);

// ---- fused single-token decode MoE (moe.hip) -----------------------------------
enum MoeAct : int { MOE_SWIGLU = 0, MOE_GEGLU = 1 };
constexpr int kMoeMaxWaves = 8;     // waves per workgroup (more lane chunks loop)
constexpr int kMoeGateupRows = 4;   // gate/up output rows per workgroup
constexpr int kMoeDownRows = 8;     // down output rows per workgroup
struct MoeArgs {
  const uint16_t* x;        // bf16 [din]
  const uint32_t* idx;      // expert per slot (32- or 64-bit, low word), [k]
  int idx_stride;           // 32-bit words per index (1 or 2)
  const void* scores;       // routing weight per slot, [k]
  int score_dt;             // 0 fp32, 1 bf16, 2 fp16
  const uint32_t* gate_w;   // [E][dff][din * gu_bits / 32]
  const uint16_t* gate_s;   // bf16 [E][dff][din / gs]
  const uint16_t* gate_b;
  const uint32_t* up_w;
  const uint16_t* up_s;
  const uint16_t* up_b;
  const uint32_t* down_w;   // [E][din][dff * d_bits / 32]
  const uint16_t* down_s;   // bf16 [E][din][dff / gs]
  const uint16_t* down_b;
  float* act;               // fp32 [k][dff] workspace
  uint16_t* out;            // bf16 [din]
  int din, dff, k, E, gs_shift;
};
hipError_t moe_launch(const MoeArgs& a, int gu_bits, int d_bits, int act, hipStream_t stream);

// out[i] = bf16(out[i] + bias[i % bias_n]) over n bf16 elements (bias.hip).
hipError_t launch_bias_add(void* out, const void* bias, int64_t n, int64_t bias_n, int tc, hipStream_t stream);

// ---- scratch.hip: the no-allocation entry point's device array ----
size_t static_scratch_bytes();
hipError_t static_scratch(int dev, void** ptr);

}  // namespace mlxq
