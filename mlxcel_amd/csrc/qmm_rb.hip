// qmm_rb.hip — prefill quantized GEMM with the weights in registers (gfx950).
//
// Replaces the reference's prefill route (dequantize to bf16, then hipBLASLt:
// overlays/rocm/mlx/backend/rocm/quantized/affine_quantize.hip:127-167,
// qmm.hip:1376-1617) with one kernel: y[M, N] = x[M, K] @ dequant(w)[N, K]^T,
// bf16 in, fp32 accumulate on v_mfma_f32_32x32x16_bf16, bf16 out (or fp32
// partials for a K split).  The dequantized weights round as the reference's
// GPU dequantizer does, bf16(s * q + b) (affine_quantize.hip:164); mxfp4 as
// fp4(q) * 2^(e - 127), exact.
//
// Work split.  A workgroup owns a BM x 256 output tile; its 4 waves sit side
// by side along N, each owning BM x 64 (FM x 2 MFMA tiles of 32 x 32).
//  - Weights never touch LDS: each wave reads exactly the 64 weight rows it
//    multiplies (lane i: row i % 32 and i % 32 + 32, one 16-byte piece per row
//    and K-step), dequantizes them into B operands in registers, and reuses
//    each B operand for its FM MFMAs along M.  A weight value is dequantized
//    once per workgroup.
//  - Activations are shared by the 4 waves through LDS: every 64-wide K-step
//    of the BM x 64 activation tile goes straight from memory into one of 4
//    LDS stages with buffer_load_dwordx4 ... lds (lane L of a wave load lands
//    at stage + 16 L, no registers in flight), each wave loading a quarter.
// The k order inside a K-step is permuted so both operands are cheap to
// fetch: the lane half h = lane / 32 of MFMA slice s covers the 8 k of chunk
// 4 h + s, so a lane's weight piece is 16 contiguous bytes (4-bit) and its
// activation fragments are single 16-byte LDS reads.  (The sum over k does
// not depend on the order; A and B use the same one.)
//
// LDS layout of a stage: row r at r * 128 bytes, its 16-byte chunk c at
// position c ^ swz(r), swz(r) = (r ^ (r >> 3)) & 7, so the 16 rows one MFMA
// fragment read touches per LDS cycle hit distinct banks (with 32 or 64
// banks); the direct-to-LDS loads write consecutive positions, so each lane
// fetches the chunk that belongs at its position.
//
// Pipelining: a ring of 4 stages; step b's loads (activations into LDS,
// weights and scales into register slots) are issued 3 steps ahead.  One
// barrier per step, after a wait that leaves the two younger steps' loads in
// flight.  Steps past the workgroup's last issue dead loads (offset past
// every operand: no traffic) and skip their MFMAs, so every turn of the ring
// is whole and the register slots stay put across the loop's back edge.
#include "common.hpp"
#include "kernels.hpp"

namespace mlxq {

namespace {

constexpr int RB_BK = 64;                 // k per step
constexpr int RB_NW = 4;                  // waves per workgroup (along N)
constexpr int RB_BN = RB_NW * 64;         // output columns per workgroup
constexpr int RB_NS = 4;                  // ring stages
constexpr int RB_NT = 64 * RB_NW;

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// two floats -> a bf16 pair, round to nearest even
__device__ __forceinline__ uint32_t bf2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}

// byte J of w as a float: one v_cvt_f32_ubyteJ (the compiler otherwise emits
// a bit-field extract plus a conversion)
template <int J>
__device__ __forceinline__ float ub(uint32_t w) {
  float r;
  if constexpr (J == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(w));
  else if constexpr (J == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(w));
  else if constexpr (J == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(w));
  else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(w));
  return r;
}

__device__ __forceinline__ int swz(int r) { return (r ^ (r >> 3)) & 7; }

// 16 bytes per lane from the buffer straight into LDS at lds + 16 * lane
// (a plain device function: inside a kernel template's lambda the host pass
// would drop the template's launch stub)
__device__ __forceinline__ void load_lds16(__amdgpu_buffer_rsrc_t r, unsigned char* lds, uint32_t voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
}

// wait until at most N vector-memory instructions of this wave are in
// flight, then a workgroup barrier (one statement: nothing moves in between,
// and no LDS access moves across it)
template <int N>
__device__ __forceinline__ void wait_vm_barrier() {
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"i"(N) : "memory");
}

}  // namespace

template <int FMT, int BM>
__global__ __launch_bounds__(RB_NT, 1) void qmm_rb_kernel(const QmmRbArgs a) {
  constexpr bool AFF = FMT != MXFP4;
  constexpr int BITS = FMT == AFF8 ? 8 : 4;
  constexpr int FM = BM / 32;                    // 32-row MFMA tiles per wave
  constexpr int XB = BM * RB_BK * 2;             // activation bytes per stage
  constexpr int XI = XB / 1024 / RB_NW;          // 1 KiB direct-to-LDS loads per wave and step
  constexpr int WL = BITS == 8 ? 2 : 1;          // 16-byte weight loads per row and step
  constexpr int SL = AFF ? 4 : 2;                // scale loads per step (2 rows x (scale, bias))
  constexpr int VM = XI + 2 * WL + SL;           // vector-memory instructions per step and wave
  static_assert(VM * (RB_NS - 2) < 64, "vmcnt range");
  __shared__ __align__(16) unsigned char xl0[XB], xl1[XB], xl2[XB], xl3[XB];
  static_assert(RB_NS == 4, "four ring stages");
  auto ring = [&](int s) -> unsigned char* { return s == 0 ? xl0 : s == 1 ? xl1 : s == 2 ? xl2 : xl3; };

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int M = a.M, N = a.N, K = a.K;

  // ---- workgroup -> (split, tile): each XCD (id mod 8) walks a contiguous
  // run of tiles, so the tiles its CUs share stay in its L2 -----------------
  const int T = a.tiles_m * a.tiles_n;
  const int G = T * a.ksplit;
  int b = blockIdx.x;
  {
    const int q = G >> 3, r = G & 7, xc = b & 7, j = b >> 3;
    b = xc < r ? xc * (q + 1) + j : r * (q + 1) + (xc - r) * q + j;
  }
  const int z = b / T, tt = b - z * T;
  const int tm = a.m_fast ? tt % a.tiles_m : tt / a.tiles_n;
  const int tn = a.m_fast ? tt / a.tiles_m : tt % a.tiles_n;
  const int m0 = tm * BM, n0 = tn * RB_BN;
  const int ks0 = z * a.ksteps_per_split;
  const int nst = min(a.ksteps_per_split, K / RB_BK - ks0);  // steps of this workgroup (>= 1)

  const uint32_t RB = (uint32_t)(K * BITS / 8);  // bytes per weight row
  const int GR = K >> a.gs_shift;                 // groups per row
  const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(a.x, (uint32_t)((int64_t)M * K * 2));
  const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(a.w, (uint32_t)((int64_t)N * RB));
  const __amdgpu_buffer_rsrc_t sr = buffer_rsrc(a.scales, (uint32_t)((int64_t)N * GR * (AFF ? 2 : 1)));
  const __amdgpu_buffer_rsrc_t br = buffer_rsrc(AFF ? (const void*)a.biases : a.scales,
                                                (uint32_t)(AFF ? (int64_t)N * GR * 2 : 0));

  // activations: wave load j fills stage rows 8 (wave XI + j) .. +7; lane L
  // writes row rr = 8 (wave XI + j) + L / 8 at position L % 8, so it fetches
  // chunk (L % 8) ^ swz(rr) of that row.  Step b adds its k offset through
  // the scalar offset (the bounds check covers the vector offset: dead lanes
  // stay dead, and live lanes never leave their row).
  uint32_t xo[XI];
#pragma unroll
  for (int j = 0; j < XI; j++) {
    const int rr = 8 * (wave * XI + j) + (lane >> 3);
    const int c = (lane & 7) ^ swz(rr);
    xo[j] = m0 + rr < M ? (uint32_t)(m0 + rr) * (uint32_t)K * 2u + (uint32_t)c * 16u : kDeadOfs;
  }

  // weights: lane (h, nl) multiplies rows n0 + 64 wave + 32 j + nl (j = 0, 1)
  // with the k of chunks 4h .. 4h+3 of each step: bytes [16 WL h, 16 WL h + 16 WL)
  // of the row's step piece
  const int h = lane >> 5, nl = lane & 31;
  uint32_t wo[2], so[2];
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int n = n0 + 64 * wave + 32 * j + nl;
    wo[j] = n < N ? (uint32_t)n * RB + (uint32_t)(16 * WL * h) : kDeadOfs;
    so[j] = n < N ? (uint32_t)n * (uint32_t)GR * (AFF ? 2u : 1u) : kDeadOfs;  // bytes
  }

  u32x4 wreg[RB_NS][2][WL];
  uint32_t sreg[RB_NS][2], breg[RB_NS][2];

  // Branch-free issue: a step past the workgroup's last ORs the dead bit into
  // every vector offset (a dead offset plus a small step offset stays dead).
  auto issue = [&](int bb, int slot) {
    const uint32_t dead = (uint32_t)(bb >= nst) << 31;  // workgroup-uniform
    const int ks = ks0 + bb;
#pragma unroll
    for (int j = 0; j < XI; j++) {
      load_lds16(xr, ring(slot) + (wave * XI + j) * 1024, xo[j] | dead, ks * RB_BK * 2);
    }
    const uint32_t wstep = (uint32_t)ks * (uint32_t)(RB_BK * BITS / 8);
    const uint32_t g = (uint32_t)((ks * RB_BK + 32 * h) >> a.gs_shift) * (AFF ? 2u : 1u);  // this lane's group, bytes
#pragma unroll
    for (int j = 0; j < 2; j++) {
#pragma unroll
      for (int l = 0; l < WL; l++)
        wreg[slot][j][l] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, (wo[j] + wstep + 16u * l) | dead, 0, 0));
      const uint32_t go = (so[j] + g) | dead;
      if constexpr (AFF) {
        sreg[slot][j] = __builtin_amdgcn_raw_buffer_load_b16(sr, go, 0, 0);
        breg[slot][j] = __builtin_amdgcn_raw_buffer_load_b16(br, go, 0, 0);
      } else {
        sreg[slot][j] = __builtin_amdgcn_raw_buffer_load_b8(sr, go, 0, 0);
        breg[slot][j] = 0u;
      }
    }
  };

  f32x16 acc[FM][2];
#pragma unroll
  for (int f = 0; f < FM; f++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int q = 0; q < 16; q++) acc[f][j][q] = 0.f;

  // A fragment of tile f, slice s: row 32 f + nl, chunk 4 h + s
  uint32_t aoff[FM];
#pragma unroll
  for (int f = 0; f < FM; f++) {
    const int r = 32 * f + nl;
    aoff[f] = (uint32_t)r * 128u;
  }
  auto afrag = [&](const unsigned char* st, int f, int s) -> bf16x8 {
    const int r = 32 * f + nl;
    return __builtin_bit_cast(bf16x8,
                              *reinterpret_cast<const u32x4*>(st + aoff[f] + 16 * ((4 * h + s) ^ swz(r))));
  };

  // B operand of row j, slice s: the 8 k of chunk 4 h + s, natural order
  auto bfrag = [&](int slot, int j, int s) -> bf16x8 {
    uint32_t o[4];
    if constexpr (FMT == AFF4) {
      const float sc = bf16_bits_to_f32(sreg[slot][j]);
      const float bi = bf16_bits_to_f32(breg[slot][j]);
      const uint32_t w = wreg[slot][j][0][s];
      const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
      o[0] = bf2(__builtin_fmaf(sc, ub<0>(lo), bi), __builtin_fmaf(sc, ub<0>(hi), bi));
      o[1] = bf2(__builtin_fmaf(sc, ub<1>(lo), bi), __builtin_fmaf(sc, ub<1>(hi), bi));
      o[2] = bf2(__builtin_fmaf(sc, ub<2>(lo), bi), __builtin_fmaf(sc, ub<2>(hi), bi));
      o[3] = bf2(__builtin_fmaf(sc, ub<3>(lo), bi), __builtin_fmaf(sc, ub<3>(hi), bi));
    } else if constexpr (FMT == AFF8) {
      const float sc = bf16_bits_to_f32(sreg[slot][j]);
      const float bi = bf16_bits_to_f32(breg[slot][j]);
      const uint32_t w0 = wreg[slot][j][s >> 1][2 * (s & 1)], w1 = wreg[slot][j][s >> 1][2 * (s & 1) + 1];
      o[0] = bf2(__builtin_fmaf(sc, ub<0>(w0), bi), __builtin_fmaf(sc, ub<1>(w0), bi));
      o[1] = bf2(__builtin_fmaf(sc, ub<2>(w0), bi), __builtin_fmaf(sc, ub<3>(w0), bi));
      o[2] = bf2(__builtin_fmaf(sc, ub<0>(w1), bi), __builtin_fmaf(sc, ub<1>(w1), bi));
      o[3] = bf2(__builtin_fmaf(sc, ub<2>(w1), bi), __builtin_fmaf(sc, ub<3>(w1), bi));
    } else {
      // fp4 code points times a normal power of two are exact in bf16 (the
      // scale folds into the conversion); 2^-127 and NaN take the product
      const uint32_t e = sreg[slot][j];
      const float sc = e8m0_to_f32(e);
      const uint32_t w = wreg[slot][j][0][s];
      if (e - 1u < 254u) {
        unpack_mxfp4_scaled(w, sc, o);
      } else {
        uint32_t v[4];
        unpack_mxfp4(w, v);
#pragma unroll
        for (int q = 0; q < 4; q++) o[q] = bf2(bf16_bits_to_f32(v[q] & 0xFFFFu) * sc, bf16_bits_to_f32(v[q] >> 16) * sc);
      }
    }
    return as_bf16x8(o);
  };

  // One whole turn of the ring: steps b0 .. b0 + RB_NS - 1.
  auto turn = [&](int b0) {
#pragma unroll
    for (int d = 0; d < RB_NS; d++) {
      const int bb = b0 + d;
      // step bb's loads were issued RB_NS - 1 steps ago: wait until only the
      // RB_NS - 2 younger steps' instructions are outstanding; after the
      // barrier every wave's activations of step bb are in LDS and every wave
      // is done with the stage step bb + RB_NS - 1 refills
      wait_vm_barrier<VM * (RB_NS - 2)>();
      issue(bb + RB_NS - 1, (d + RB_NS - 1) % RB_NS);
      if (bb >= nst) continue;  // workgroup-uniform
      const unsigned char* st = ring(d);
#pragma unroll
      for (int s = 0; s < 4; s++) {
        bf16x8 bv[2];
#pragma unroll
        for (int j = 0; j < 2; j++) bv[j] = bfrag(d, j, s);
#pragma unroll
        for (int f = 0; f < FM; f++) {
          const bf16x8 av = afrag(st, f, s);
          acc[f][0] = mfma32(av, bv[0], acc[f][0]);
          acc[f][1] = mfma32(av, bv[1], acc[f][1]);
        }
      }
    }
  };

#pragma unroll
  for (int d = 0; d < RB_NS - 1; d++) issue(d, d);
  // the first turn outside the loop: the loop header then joins two
  // identical states, so the compiler's own waits on the register slots
  // (loaded a turn earlier) stay as loose as the ring allows
  turn(0);
  for (int b0 = RB_NS; b0 < nst; b0 += RB_NS) turn(b0);
  // the dead loads past the last step land before the workgroup ends
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // ---- epilogue: D of tile (f, j): lane holds column 32 j + nl, rows
  // 32 f + 8 (q / 4) + 4 h + q % 4 -------------------------------------------
  const bool split = a.ksplit > 1;
#pragma unroll
  for (int f = 0; f < FM; f++)
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int c = n0 + 64 * wave + 32 * j + nl;
      if (c >= N) continue;
#pragma unroll
      for (int q = 0; q < 16; q++) {
        const int r = m0 + 32 * f + 8 * (q >> 2) + 4 * h + (q & 3);
        if (r < M) {
          if (split) a.ws[((int64_t)z * M + r) * N + c] = acc[f][j][q];
          else a.out[(int64_t)r * N + c] = (uint16_t)f32_to_bf16_bits(acc[f][j][q]);
        }
      }
    }
}

QmmRbPlan qmm_rb_plan(int fmt, int gs, int64_t M, int64_t N, int64_t K, int num_cus, int bm_req, int ksplit_req) {
  QmmRbPlan p;
  const int bits = fmt == AFF8 ? 8 : 4;
  if (K % RB_BK != 0 || K % gs != 0 || gs < 32 || M <= 0 || N <= 0) return p;
  // 32-bit buffer offsets: every operand below 2 GiB (0x80000000 marks dead lanes)
  if (M * K * 2 >= ((int64_t)1 << 31) || N * K * bits / 8 >= ((int64_t)1 << 31) || M * N * 4 >= ((int64_t)1 << 31))
    return p;
  const int nks = (int)(K / RB_BK);
  p.bm = (bm_req == 128 || bm_req == 256) ? bm_req : (M >= 2048 ? 256 : 128);
  p.tiles_m = (int)((M + p.bm - 1) / p.bm);
  p.tiles_n = (int)((N + RB_BN - 1) / RB_BN);
  const int64_t tiles = (int64_t)p.tiles_m * p.tiles_n;
  int ks = 1;
  if (ksplit_req > 0) {
    ks = ksplit_req;
  } else {
    // split K while fewer than half the CUs have a tile and each split keeps >= 16 steps
    while (tiles * ks * 2 <= num_cus && nks / (ks * 2) >= 16) ks *= 2;
  }
  p.ksteps_per_split = (nks + ks - 1) / ks;
  p.ksplit = (nks + p.ksteps_per_split - 1) / p.ksteps_per_split;
  p.m_fast = M * K * 2 <= N * K * bits / 8 ? 1 : 0;
  p.ok = tiles * p.ksplit < ((int64_t)1 << 31);
  return p;
}

namespace {
template <int FMT>
void rb_launch_fmt(const QmmRbArgs& a, const QmmRbPlan& p, hipStream_t stream) {
  const dim3 grid((unsigned)((int64_t)p.tiles_m * p.tiles_n * p.ksplit));
  if (p.bm == 256) hipLaunchKernelGGL((qmm_rb_kernel<FMT, 256>), grid, dim3(RB_NT), 0, stream, a);
  else hipLaunchKernelGGL((qmm_rb_kernel<FMT, 128>), grid, dim3(RB_NT), 0, stream, a);
}
}  // namespace

hipError_t qmm_rb_launch(int fmt, const QmmRbArgs& a_in, const QmmRbPlan& p, hipStream_t stream) {
  if (!p.ok || (p.ksplit > 1 && !a_in.ws)) return hipErrorInvalidValue;
  QmmRbArgs a = a_in;
  a.tiles_m = p.tiles_m;
  a.tiles_n = p.tiles_n;
  a.ksplit = p.ksplit;
  a.ksteps_per_split = p.ksteps_per_split;
  a.m_fast = p.m_fast;
  switch (fmt) {
    case AFF4: rb_launch_fmt<AFF4>(a, p, stream); break;
    case AFF8: rb_launch_fmt<AFF8>(a, p, stream); break;
    default: rb_launch_fmt<MXFP4>(a, p, stream); break;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.ksplit == 1) return e;
  return launch_splitk_reduce(a.ws, a.out, (int64_t)a.M * a.N, p.ksplit, stream);
}

}  // namespace mlxq
