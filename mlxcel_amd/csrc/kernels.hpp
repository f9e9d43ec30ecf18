// kernels.hpp — launch interfaces between the C-ABI host layer (api.cpp) and
// the gfx950 kernels.  Plain data structs; no torch or MLX types.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mlxq.h"

namespace mlxq {

// Skinny (decode) quantized matmul over segments of rows sharing one weight
// matrix.  Mode A (seg == nullptr): segment s = rows [s*rps, s*rps + rps) of
// the output, x batch lhs[s] (or s), weight matrix rhs[s] (or s when
// w_expert_stride != 0, else 0).  Mode B: segment table seg[s] =
// {expert, row_begin, row_count} over a row map rowmap[r] = {x_row, out_row}.
struct QmvArgs {
  const uint16_t* x;        // bf16 activations, rows of K
  const uint32_t* w;        // packed codes [E][N][K*bits/32]
  const void* scales;       // bf16 (affine) or uint8 e8m0 (mxfp4) [E][N][K/gs]
  const uint16_t* biases;   // bf16 [E][N][K/gs] (affine only)
  uint16_t* out;            // bf16 [out_rows][N]
  float* ws;                // split-K partials [ks][out_rows][N] (ks > 1)
  unsigned* counters;       // split-K arrival counters, one per (segment, tile); zero on entry and exit
  const uint32_t* lhs;      // mode A: x batch index per segment (nullable)
  const uint32_t* rhs;      // mode A: expert per segment (nullable)
  const int* seg;           // mode B segment table (nullable)
  const int* rowmap;        // mode B row map
  const int* nseg;          // mode B: number of valid segments (device)
  int N;
  int K;
  int64_t w_expert_stride;  // uint32 words per weight matrix (0: one matrix)
  int64_t s_expert_stride;  // scale/bias elements per weight matrix
  int E;                    // weight matrices (index clamp)
  int X;                    // x batches (index clamp)
  int rps;                  // mode A rows per segment
  int total_rows;           // mode A total rows
  int out_rows;             // rows of `out` (split-K workspace stride)
  int rows_lds;             // activation rows staged per workgroup (>= rows of any segment)
  int ks;                   // workgroups splitting K (gridDim.z)
  int kst_per_wg;           // K-steps per workgroup
};

struct QmvPlan {
  int ks = 1;
  int kst_per_wg = 1;
  int tiles = 1;
  size_t lds = 0;
};

int qmv_slots(int fmt, int gs);
int qmv_tile_mt(int fmt, int gs, int rows);
int qmv_max_rows(int fmt, int gs);
QmvPlan qmv_plan(int fmt, int gs, int64_t N, int64_t K, int rows_lds, int nseg, int num_cus);
hipError_t qmv_launch(int fmt, int gs, int mt, const QmvArgs& a, int nseg_slots, const QmvPlan& p,
                      hipStream_t stream);

// Elementwise conversions (dequant.hip).
hipError_t launch_affine_dequantize(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                                    uint16_t* out, int64_t rows, int64_t K, int gs, int bits,
                                    hipStream_t stream);
hipError_t launch_mxfp4_dequantize(const uint32_t* w, const uint8_t* scales, uint16_t* out,
                                   int64_t rows, int64_t K, hipStream_t stream);
hipError_t launch_affine_quantize(const uint16_t* w, uint32_t* wq, uint16_t* scales,
                                  uint16_t* biases, int64_t rows, int64_t K, int gs, int bits,
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

}  // namespace mlxq
