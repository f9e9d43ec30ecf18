// qmm.hip — prefill quantized matmul (many activation rows) for gfx950.
//
// Replaces the reference's prefill route: affine dequantize to a bf16
// temporary and a hipBLASLt GEMM (overlays/rocm/mlx/backend/rocm/quantized/
// affine_quantize.hip:127-167 + qmm.hip:1376-1617, 3689-3892).  Here the
// dequantization happens on the way into LDS, so the bf16 weights never
// touch HBM: y = x @ W^T with W = bf16(s*q + b) (affine; the reference GPU
// dequantizer's rounding, affine_quantize.hip:164) or fp4(q) * 2^(e-127)
// (mxfp4, exact), fp32 accumulation, one bf16 rounding on store.
//
// Two kernels:
//  * qmm_tile_kernel (dense prefill, and grouped gathers at tiles 4-8): tiles
//    of 128 x 128 to 256 x 256 on 4 or 8 waves of v_mfma_f32_32x32x16_bf16
//    (or _f16), K in steps of 64 through double-buffered, XOR-swizzled LDS;
//    described above the kernel;
//  * qmm_kernel (grouped gathers at tiles 0-3): 4 waves (2 x 2) of
//    v_mfma_f32_16x16x32_bf16 over padded LDS rows [BM][64 + 8] and
//    [BN][64 + 8] (the 8-element pad puts the 16 rows a fragment read
//    touches on distinct banks), the next K-step's loads issued before the
//    current step's MFMAs, one barrier per K-step.
// When the grid would leave CUs idle (short M), K is split across
// workgroups and the fp32 partials are summed by a second kernel in a fixed
// order (bitwise reproducible).
#include "common.hpp"
#include "kernels.hpp"

namespace mlxq {

namespace {

constexpr int BK = 64;
constexpr int LDSK = BK + 8;  // padded row length (bf16)
constexpr int NT = 256;       // threads per workgroup (4 waves, 2 x 2)

typedef float f32x2 __attribute__((ext_vector_type(2)));

// Two floats -> a bf16 pair, round to nearest even (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}

// The same for the 16-bit type XT (0 bfloat16, 1 float16), round to nearest even.
template <int XT>
__device__ __forceinline__ uint32_t pack_xt2(float lo, float hi) {
  if constexpr (XT == 0) return pack_bf16x2(lo, hi);
  else {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, h2));
  }
}

// Byte j of w as a float (v_cvt_f32_ubyte<j>).
__device__ __forceinline__ float ubyte(uint32_t w, int j) { return (float)((w >> (8 * j)) & 0xFFu); }

// Byte J of w as a float, one v_cvt_f32_ubyte<J> (written out: from a masked
// word the compiler otherwise emits a bit-field extract plus a conversion).
template <int J>
__device__ __forceinline__ float cvt_ubyte(uint32_t w) {
  float r;
  if constexpr (J == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(w));
  else if constexpr (J == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(w));
  else if constexpr (J == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(w));
  else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(w));
  return r;
}

__device__ __forceinline__ int swz(int r) { return (r ^ (r >> 3)) & 7; }

}  // namespace

// BM x BN output tile per workgroup; each wave owns (BM/2) x (BN/2).
template <int FMT, int BM, int BN>
__global__ __launch_bounds__(NT) void qmm_kernel(const QmmArgs a) {
  constexpr int TM = BM / 2, TN = BN / 2;  // wave tile
  constexpr int FM = TM / 16, FN = TN / 16;  // 16 x 16 MFMA tiles per wave
  constexpr bool AFF = FMT != MXFP4;
  constexpr int BITS = FMT == AFF8 ? 8 : 4;
  constexpr int WT = BK * BITS / 8 / 16;   // threads per weight row per K-step (16 bytes each)
  constexpr int WROWS = NT / WT;           // weight rows loaded per pass
  constexpr int WPASS = BN / WROWS;        // passes per K-step
  constexpr int VPL = 128 / BITS;          // values per 16-byte load
  constexpr int XPASS = BM * BK * 2 / 16 / NT;  // 16-byte activation loads per thread per K-step

  __shared__ __align__(16) uint16_t xs[2][BM * LDSK];
  __shared__ __align__(16) uint16_t wsm[2][BN * LDSK];

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;  // wave position in the 2 x 2 grid
  static_assert(BN % WROWS == 0, "weight rows per pass must divide BN");
  const int n0 = blockIdx.x * BN;
  const int M = a.M, N = a.N, K = a.K;
  const int nks = a.ksteps_per_split;
  const int ks0 = blockIdx.z * nks;
  const int ks1 = min(ks0 + nks, K / BK);

  // Rows of this tile: rows m0 .. m0+rows-1 of x / y, or (gathers grouped by
  // expert) table entry blockIdx.y: grouped rows r0 .. r0+rows-1 of one
  // expert, read and written through xrows / orows.
  int m0 = blockIdx.y * BM, rows = min(BM, M - m0), r0 = 0;
  int64_t wbase = 0, sbase = 0;
  if (a.seg) {
    if ((int)blockIdx.y >= (int)a.nseg_dev[0]) return;
    const int expert = (int)a.seg[3 * blockIdx.y];
    r0 = (int)a.seg[3 * blockIdx.y + 1];
    rows = (int)a.seg[3 * blockIdx.y + 2];
    m0 = 0;
    wbase = (int64_t)expert * a.w_expert_stride;
    sbase = (int64_t)expert * a.s_expert_stride;
  }

  const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(a.x, (uint32_t)((int64_t)a.x_rows * K * 2));
  const uint32_t RB = (uint32_t)(K * BITS / 8);  // bytes per weight row
  const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(a.w + wbase, (uint32_t)((int64_t)N * RB));
  const int G = K >> a.gs_shift;
  const __amdgpu_buffer_rsrc_t sr =
      buffer_rsrc(reinterpret_cast<const uint8_t*>(a.scales) + sbase * (AFF ? 2 : 1), (uint32_t)((int64_t)N * G * (AFF ? 2 : 1)));
  const __amdgpu_buffer_rsrc_t br =
      buffer_rsrc(AFF ? (const void*)(a.biases + sbase) : a.scales, (uint32_t)(AFF ? (int64_t)N * G * 2 : 0));

  // ---- global -> register staging of one K-step ----------------------------
  // activations: thread t loads row (t / 8) + 32 i, 16-byte chunk t % 8
  const int xrow = t >> 3, xch = t & 7;
  // weights: thread t loads row (t / WT) + WROWS p, 16-byte piece t % WT
  const int wrow = t / WT, wpc = t % WT;
  uint32_t xbase[XPASS];  // byte offset of each staged x row (tile rows past `rows` read 0)
#pragma unroll
  for (int i = 0; i < XPASS; i++) {
    const int tr = xrow + 32 * i;
    const uint32_t xrw = a.seg ? (tr < rows ? a.xrows[r0 + tr] : 0u) : (uint32_t)(m0 + tr);
    xbase[i] = tr < rows ? xrw * (uint32_t)K * 2u + (uint32_t)xch * 16u : kDeadOfs;
  }
  u32x4 xreg[XPASS];
  u32x4 wreg[WPASS];
  uint32_t sreg[WPASS], breg[WPASS];
  auto load_step = [&](int ks) {
    const int k0 = ks * BK;
#pragma unroll
    for (int i = 0; i < XPASS; i++)
      xreg[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, xbase[i] + (uint32_t)k0 * 2u, 0, 0));
#pragma unroll
    for (int p = 0; p < WPASS; p++) {
      const int n = n0 + wrow + WROWS * p;
      const bool live = n < N;
      const uint32_t off = live ? (uint32_t)n * RB + (uint32_t)(k0 * BITS / 8 + wpc * 16) : kDeadOfs;
      wreg[p] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, off, 0, 2 /* nt */));
      const int g = (k0 + wpc * VPL) >> a.gs_shift;
      const uint32_t so = live ? (uint32_t)(n * G + g) : kDeadOfs;
      if constexpr (AFF) {
        sreg[p] = __builtin_amdgcn_raw_buffer_load_b16(sr, so * 2u, 0, 0);
        breg[p] = __builtin_amdgcn_raw_buffer_load_b16(br, so * 2u, 0, 0);
      } else {
        sreg[p] = __builtin_amdgcn_raw_buffer_load_b8(sr, so, 0, 0);
        breg[p] = 0u;
      }
    }
  };

  // ---- register -> LDS (activations as is, weights dequantized) ------------
  auto store_step = [&](int buf) {
#pragma unroll
    for (int i = 0; i < XPASS; i++)
      *reinterpret_cast<u32x4*>(&xs[buf][(xrow + 32 * i) * LDSK + xch * 8]) = xreg[i];
#pragma unroll
    for (int p = 0; p < WPASS; p++) {
      const u32x4 w = wreg[p];
      uint32_t o[VPL / 2];
      if constexpr (AFF) {
        const float sc = bf16_bits_to_f32(sreg[p]);
        const float bi = bf16_bits_to_f32(breg[p]);
        if constexpr (BITS == 4) {
          // nibbles 2j (low half of byte j) and 2j+1 (high half)
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const uint32_t lo = w[e] & 0x0F0F0F0Fu, hi = (w[e] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int j = 0; j < 4; j++)
              o[e * 4 + j] = pack_bf16x2(__builtin_fmaf(sc, ubyte(lo, j), bi), __builtin_fmaf(sc, ubyte(hi, j), bi));
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; e++)
#pragma unroll
            for (int j = 0; j < 4; j += 2)
              o[e * 2 + j / 2] =
                  pack_bf16x2(__builtin_fmaf(sc, ubyte(w[e], j), bi), __builtin_fmaf(sc, ubyte(w[e], j + 1), bi));
        }
      } else {
        // fp4 code points times a power of two are exact in bf16: for normal
        // scales (e8m0 1..254) the gfx950 scaled conversion does it in one
        // instruction per pair; 2^-127 and NaN take the explicit product.
        const float sc = e8m0_to_f32(sreg[p]);
        if (sreg[p] - 1u < 254u) {
#pragma unroll
          for (int e = 0; e < 4; e++) unpack_mxfp4_scaled(w[e], sc, &o[e * 4]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; e++) {
            uint32_t v[4];
            unpack_mxfp4(w[e], v);  // pairs (2h, 2h+1) of the code points
#pragma unroll
            for (int h = 0; h < 4; h++)
              o[e * 4 + h] = pack_bf16x2(bf16_bits_to_f32(v[h] & 0xFFFFu) * sc, bf16_bits_to_f32(v[h] >> 16) * sc);
          }
        }
      }
      uint16_t* dst = &wsm[buf][(wrow + WROWS * p) * LDSK + wpc * VPL];
#pragma unroll
      for (int c = 0; c < VPL / 8; c++)
        *reinterpret_cast<u32x4*>(dst + 8 * c) = u32x4{o[4 * c], o[4 * c + 1], o[4 * c + 2], o[4 * c + 3]};
    }
  };

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int j = 0; j < FN; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int fr = lane & 15;         // fragment row (A) / column (B)
  const int fk = (lane >> 4) * 8;   // fragment k offset within 32

  if (ks0 < ks1) {
    load_step(ks0);
    store_step(0);
    __syncthreads();
    for (int ks = ks0; ks < ks1; ks++) {
      const int buf = (ks - ks0) & 1;
      if (ks + 1 < ks1) load_step(ks + 1);
#pragma unroll
      for (int kk = 0; kk < BK; kk += 32) {
        bf16x8 af[FM], bfr[FN];
#pragma unroll
        for (int i = 0; i < FM; i++)
          af[i] = *reinterpret_cast<const bf16x8*>(&xs[buf][(wm * TM + i * 16 + fr) * LDSK + kk + fk]);
#pragma unroll
        for (int j = 0; j < FN; j++)
          bfr[j] = *reinterpret_cast<const bf16x8*>(&wsm[buf][(wn * TN + j * 16 + fr) * LDSK + kk + fk]);
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
          for (int j = 0; j < FN; j++) acc[i][j] = mfma16x16x32(af[i], bfr[j], acc[i][j]);
      }
      if (ks + 1 < ks1) store_step(buf ^ 1);
      __syncthreads();
    }
  }

  // ---- epilogue: lane holds rows 4 (lane / 16) + q of each 16 x 16 tile ------
  const bool split = a.ksplit > 1;
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int j = 0; j < FN; j++)
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int tr = wm * TM + i * 16 + 4 * (lane >> 4) + q;
        const int c = n0 + wn * TN + j * 16 + fr;
        if (tr < rows && c < N) {
          const int64_t r = a.seg ? (int64_t)a.orows[r0 + tr] : (int64_t)(m0 + tr);
          if (split) a.ws[((int64_t)blockIdx.z * M + r) * N + c] = acc[i][j][q];
          else a.out[r * N + c] = (uint16_t)f32_to_bf16_bits(acc[i][j][q]);
        }
      }
}

// ---- 32x32-MFMA tile kernel -------------------------------------------------
//
// y[BM x BN tile] with NWM x NWN waves (2 x 2, 2 x 4 or 4 x 2); a wave owns
// (BM/NWM) x (BN/NWN) output elements as v_mfma_f32_32x32x16_bf16 tiles of
// 32 x 32 (128 fp32 accumulators per lane at 128 x 64 per wave).
//
// Per 64-wide K-step, activations [BM][64] and dequantized weights [BN][64]
// (bf16) sit in double-buffered LDS.  Rows are 128 bytes with the 16-byte
// chunk c of row r stored at c ^ swz(r), swz(r) = (r ^ (r >> 3)) & 7, so the
// 16 rows that one LDS cycle of a fragment read touches (same chunk) hit
// distinct banks; with c ^ (r & 7) rows r and r + 8 collided (37% of the LDS
// cycles were bank conflicts by SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE).
// While the MFMAs of step ks run from buffer ks&1, the wave dequantizes step
// ks+1 from registers into the other buffer and then issues the global loads
// of step ks+2, a whole K-step ahead of their first use; two barriers per
// K-step (the loop below says which each one publishes).
//
// Memory requests are what the L1/TA sees per instruction, so every load is
// shaped to touch few lines: activations as 8 lanes x 16 B per 128-byte row
// piece; weights as WT lanes x 16 B per row piece (a row's 64 codes of one
// K-step are contiguous); scales and biases as one 16-byte chunk per row
// (8 bf16 groups or 16 e8m0 groups) every few K-steps, staged in a small
// double-buffered LDS table [group][row].
//
// Workgroups are numbered so that each XCD (workgroup id mod 8) walks a
// contiguous run of tiles, keeping the tiles its CUs share in its own L2.
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x16 mfma32x32x16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// on the bit patterns of 16-bit operands of type XT (1: v_mfma_f32_32x32x16_f16)
template <int XT>
__device__ __forceinline__ f32x16 mfma32x32x16_xt(bf16x8 a, bf16x8 b, f32x16 c) {
  if constexpr (XT == 0) return mfma32x32x16(a, b, c);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
}

// Interleave of one slice: after each MFMA, up to this many VALU
// instructions (measured on MI355X: 6 keeps the dequantization under the
// MFMAs at both tile sizes).
constexpr int kValuPerMfma = 6;

// XT: 16-bit type of x, scales, biases and result (0 bfloat16, 1 float16:
// weights dequantized to float16(s * q + b), products on the float16 MFMA;
// affine only).
template <int FMT, int BM, int BN, int NWM, int NWN, int XT, bool SK = false>
__global__ __launch_bounds__(64 * NWM * NWN) void qmm_tile_kernel(const QmmArgs a) {
  constexpr int NT = 64 * NWM * NWN;         // threads
  constexpr int TM = BM / NWM, TN = BN / NWN;  // wave tile
  constexpr int FM = TM / 32, FN = TN / 32;  // 32 x 32 MFMA tiles per wave
  constexpr bool AFF = FMT != MXFP4;
  constexpr int BITS = FMT == AFF8 ? 8 : 4;
  constexpr int RS = BK;                     // LDS row stride (bf16): 128 bytes, swizzled
  constexpr int XL = BM * BK * 2 / 16 / NT;  // 16-byte activation loads per thread and K-step
  // weight piece per thread and load: 16 bytes, or 8 when a K-step of the
  // tile's weights is less than 16 bytes per thread (256 x 128, 8 waves, 4-bit)
  constexpr int PB = BN * BK * BITS / 8 / NT >= 16 ? 16 : 8;
  constexpr int PW = PB / 4;                 // words per piece
  constexpr int WT = BK * BITS / 8 / PB;     // threads per weight row and K-step
  constexpr int WROWS = NT / WT;             // weight rows per pass
  constexpr int WP = BN / WROWS;             // weight loads per thread and K-step
  constexpr int VPL = PB * 8 / BITS;         // values per weight load
  constexpr int CHG = AFF ? 8 : 16;          // groups in a 16-byte scale chunk
  static_assert(WP >= 1 && WROWS * WP == BN && BN <= NT && XL >= 1, "tile shape");
  static_assert(PB == 16 || (BITS == 4 && PB == 8), "8-byte pieces only for 4-bit codes");

  // double-buffered activation and dequantized-weight tiles; after the last
  // K-step the same bytes stage the output tile
  constexpr int XS_BYTES = 2 * BM * RS * 2, WS_BYTES = 2 * BN * RS * 2;
  __shared__ __align__(16) unsigned char stage[XS_BYTES + WS_BYTES];
  uint16_t(*xs)[BM * RS] = reinterpret_cast<uint16_t(*)[BM * RS]>(stage);
  uint16_t(*wsm)[BN * RS] = reinterpret_cast<uint16_t(*)[BN * RS]>(stage + XS_BYTES);
  static_assert(BM * BN * 2 <= XS_BYTES + WS_BYTES && TM * BN * 4 <= XS_BYTES + WS_BYTES,
                "the output tile (16-bit) and a wave row of it (fp32) fit in the staging buffers");
  // per-chunk (scale, bias) table: affine u32 (bf16 scale | bf16 bias << 16)
  // [slot][group][row]; mxfp4 e8m0 bytes [slot][group][row]
  __shared__ __align__(16) uint32_t tbl[2 * 8 * BN];

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int wm = wave / NWN, wn = wave % NWN;
  const int M = a.M, N = a.N, K = a.K;

  // Accumulators and the placement of the piece last run (the epilogues'
  // inputs).
  f32x16 acc[FM][FN];
  const int fr = lane & 31;
  int m0 = 0, rows = 0, r0 = 0, n0 = 0;
  auto zero_acc = [&]() {
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int j = 0; j < FN; j++)
#pragma unroll
        for (int q = 0; q < 16; q++) acc[i][j][q] = 0.f;
  };

  // K-steps [ks0, ks1) of output tile (tm, tn) into acc (from zero).  The LDS
  // buffers are free on entry (the previous piece's epilogue has passed a
  // barrier behind its last LDS read) and after return hold nothing live.
  auto run_piece = [&](int tm, int tn, int ks0, int ks1) __attribute__((always_inline)) {
  n0 = tn * BN;
  m0 = tm * BM;
  rows = min(BM, M - m0);
  r0 = 0;
  int64_t wbase = 0, sbase = 0;
  if (a.seg) {  // the caller has checked tm < nseg
    const int expert = (int)a.seg[3 * tm];
    r0 = (int)a.seg[3 * tm + 1];
    rows = (int)a.seg[3 * tm + 2];
    m0 = 0;
    wbase = (int64_t)expert * a.w_expert_stride;
    sbase = (int64_t)expert * a.s_expert_stride;
  }

  const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(a.x, (uint32_t)((int64_t)a.x_rows * K * 2));
  const uint32_t RB = (uint32_t)(K * BITS / 8);
  const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(a.w + wbase, (uint32_t)((int64_t)N * RB));
  const int GR = K >> a.gs_shift;  // groups per row
  const __amdgpu_buffer_rsrc_t sr = buffer_rsrc(reinterpret_cast<const uint8_t*>(a.scales) + sbase * (AFF ? 2 : 1),
                                          (uint32_t)((int64_t)N * GR * (AFF ? 2 : 1)));
  const __amdgpu_buffer_rsrc_t br =
      buffer_rsrc(AFF ? (const void*)(a.biases + sbase) : a.scales, (uint32_t)(AFF ? (int64_t)N * GR * 2 : 0));
  const int gs_shift = a.gs_shift;
  const int SPC = (CHG << gs_shift) / BK;  // K-steps per scale chunk (4, 8 or 16)

  // activations: thread t stages rows (t / 8) + (NT / 8) i, 16-byte chunk t % 8
  constexpr int XROWS = NT / 8;
  const int xrow = t >> 3, xch = t & 7;
  uint32_t xoff[XL];
#pragma unroll
  for (int i = 0; i < XL; i++) {
    const int tr = xrow + XROWS * i;
    const uint32_t xrw = a.seg ? (tr < rows ? a.xrows[r0 + tr] : 0u) : (uint32_t)(m0 + tr);
    xoff[i] = tr < rows ? xrw * (uint32_t)K * 2u + (uint32_t)xch * 16u : kDeadOfs;
  }
  auto xdst = [&](int i) {  // LDS position of activation load i
    const int r = xrow + XROWS * i;
    return r * RS + ((xch ^ swz(r)) << 3);
  };

  // weights: thread t dequantizes rows wrow + WROWS p, 16-byte piece wpc
  const int wrow = t / WT, wpc = t % WT;
  uint32_t woff[WP];
#pragma unroll
  for (int p = 0; p < WP; p++) {
    const int n = n0 + wrow + WROWS * p;
    woff[p] = n < N ? (uint32_t)n * RB + (uint32_t)(wpc * PB) : kDeadOfs;
  }

  // scale chunks: thread t < BN loads the 16-byte chunk of row n0 + t
  const bool sload = t < BN;
  const uint32_t srow_off = (n0 + t < N && sload) ? (uint32_t)(n0 + t) * (uint32_t)GR * (AFF ? 2u : 1u) : kDeadOfs;
  // Scale rows need not be 16-byte aligned (K / gs groups per row, e.g. 90
  // e8m0 bytes): a chunk is read as 5 dwords from the dword boundary below
  // and realigned by the byte offset in registers.  The buffer's bounds
  // check zeroes a dword that reaches past the end as a whole, so where the
  // scale rows end inside a dword (N x K / gs elements not a multiple of 4
  // bytes) the last row's last chunk is read element by element: only the
  // bytes past the end read 0.
  const uint32_t sal = srow_off & 3u;
  const uint32_t sbytes = (uint32_t)((int64_t)N * GR * (AFF ? 2 : 1));
  u32x4 sc_r = {0u, 0u, 0u, 0u}, bi_r = {0u, 0u, 0u, 0u};
  uint32_t sc_x = 0u, bi_x = 0u;
  auto dword_by_elements = [&](const __amdgpu_buffer_rsrc_t& r, uint32_t o) -> uint32_t {
    if constexpr (AFF)
      return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, o, 0, 0) |
             ((uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, o + 2u, 0, 0) << 16);
    else
      return (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(r, o, 0, 0) |
             ((uint32_t)__builtin_amdgcn_raw_buffer_load_b8(r, o + 1u, 0, 0) << 8) |
             ((uint32_t)__builtin_amdgcn_raw_buffer_load_b8(r, o + 2u, 0, 0) << 16) |
             ((uint32_t)__builtin_amdgcn_raw_buffer_load_b8(r, o + 3u, 0, 0) << 24);
  };
  auto chunk_load = [&](int c) {
    if (sload) {
      const uint32_t o = (srow_off & ~3u) + (uint32_t)c * 16u;
      if (o < sbytes && o + 20u > sbytes) {
        sc_r = u32x4{dword_by_elements(sr, o), dword_by_elements(sr, o + 4u), dword_by_elements(sr, o + 8u),
                     dword_by_elements(sr, o + 12u)};
        sc_x = dword_by_elements(sr, o + 16u);
        if constexpr (AFF) {
          bi_r = u32x4{dword_by_elements(br, o), dword_by_elements(br, o + 4u), dword_by_elements(br, o + 8u),
                       dword_by_elements(br, o + 12u)};
          bi_x = dword_by_elements(br, o + 16u);
        }
      } else {
        sc_r = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(sr, o, 0, 0));
        sc_x = __builtin_amdgcn_raw_buffer_load_b32(sr, o + 16u, 0, 0);
        if constexpr (AFF) {
          bi_r = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(br, o, 0, 0));
          bi_x = __builtin_amdgcn_raw_buffer_load_b32(br, o + 16u, 0, 0);
        }
      }
    }
  };
  auto realign = [&](u32x4& v, uint32_t x) {
    if (sal != 0u) {
      v = u32x4{__builtin_amdgcn_alignbyte(v[1], v[0], sal), __builtin_amdgcn_alignbyte(v[2], v[1], sal),
                __builtin_amdgcn_alignbyte(v[3], v[2], sal), __builtin_amdgcn_alignbyte(x, v[3], sal)};
    }
  };
  auto chunk_write = [&](int c) {
    if (sload) {
      realign(sc_r, sc_x);
      if constexpr (AFF) realign(bi_r, bi_x);
      const int slot = c & 1;
      if constexpr (AFF) {
#pragma unroll
        for (int j = 0; j < 8; j++)
          tbl[(slot * 8 + j) * BN + t] =
              __builtin_amdgcn_perm(bi_r[j >> 1], sc_r[j >> 1], (j & 1) ? 0x07060302u : 0x05040100u);
      } else {
        uint8_t* tb = reinterpret_cast<uint8_t*>(tbl);
#pragma unroll
        for (int j = 0; j < 16; j++) tb[(slot * 16 + j) * BN + t] = (uint8_t)(sc_r[j >> 2] >> (8 * (j & 3)));
      }
    }
  };

  u32x4 xreg[XL], wreg[WP];
  auto load_step = [&](int ks) {
    const int k0 = ks * BK;
#pragma unroll
    for (int p = 0; p < WP; p++) {
      if constexpr (PB == 16) {
        wreg[p] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, woff[p] + (uint32_t)(k0 * BITS / 8), 0, 0));
      } else {
        const u32x2 h = __builtin_bit_cast(
            u32x2, __builtin_amdgcn_raw_buffer_load_b64(wr, woff[p] + (uint32_t)(k0 * BITS / 8), 0, 0));
        wreg[p] = u32x4{h[0], h[1], 0u, 0u};
      }
    }
#pragma unroll
    for (int i = 0; i < XL; i++)
      xreg[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, xoff[i] + (uint32_t)k0 * 2u, 0, 0));
  };

  // Register -> LDS for step ks in NPART parts so each can sit between the
  // MFMAs of one slice: part p stores the activation loads and dequantizes
  // the weight words that fall in the p-th share.
  constexpr int NPART = BK / 16;
  constexpr int NWORD = WP * PW;  // weight words per thread and K-step
  // (8-bit: the part holding the even word of a pair writes both words; the
  // registers hold the whole step until load_step(ks + 2), after the last part)
  // Table word (affine: scale | bias << 16; mxfp4: the e8m0 byte) of each
  // weight row this thread dequantizes, for this thread's group of step ks
  // (one per 16-byte piece: VPL <= group size).  Read once per step, before
  // the step's fragment reads are issued: LDS reads complete in order, so a
  // table read issued behind them would wait for all of them.
  uint32_t sbw[WP];
  auto table_read = [&](int ks) {
    const int g = ((ks * BK + wpc * VPL) >> gs_shift);
    const int gslot = ((g / CHG) & 1) * CHG + g % CHG;
#pragma unroll
    for (int pp = 0; pp < WP; pp++) {
      const int r = wrow + WROWS * pp;
      if constexpr (AFF) sbw[pp] = tbl[gslot * BN + r];
      else sbw[pp] = reinterpret_cast<const uint8_t*>(tbl)[gslot * BN + r];
    }
  };
  auto store_part = [&](int buf, int p) {
#pragma unroll
    for (int i = 0; i < XL; i++)
      if (i * NPART / XL == p) *reinterpret_cast<u32x4*>(&xs[buf][xdst(i)]) = xreg[i];
#pragma unroll
    for (int e = 0; e < NWORD; e++) {
      if (e * NPART / NWORD != p) continue;
      const int pp = e / PW;  // which weight load
      const int r = wrow + WROWS * pp;
      const uint32_t w = wreg[pp][e % PW];
      uint16_t* rowp = &wsm[buf][r * RS];
      const int r7 = swz(r);
      if constexpr (AFF) {
        const uint32_t sb = sbw[pp];
        const float sc = XT ? xt_to_f32<1>(sb & 0xFFFFu) : __uint_as_float(sb << 16);
        const float bi = XT ? xt_to_f32<1>(sb >> 16) : __uint_as_float(sb & 0xFFFF0000u);
        if constexpr (BITS == 4) {
          // 8 codes: natural pair h = (nibble 2h, nibble 2h + 1) = (byte h of lo, byte h of hi)
          const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
          const u32x4 o = {pack_xt2<XT>(__builtin_fmaf(sc, cvt_ubyte<0>(lo), bi), __builtin_fmaf(sc, cvt_ubyte<0>(hi), bi)),
                           pack_xt2<XT>(__builtin_fmaf(sc, cvt_ubyte<1>(lo), bi), __builtin_fmaf(sc, cvt_ubyte<1>(hi), bi)),
                           pack_xt2<XT>(__builtin_fmaf(sc, cvt_ubyte<2>(lo), bi), __builtin_fmaf(sc, cvt_ubyte<2>(hi), bi)),
                           pack_xt2<XT>(__builtin_fmaf(sc, cvt_ubyte<3>(lo), bi), __builtin_fmaf(sc, cvt_ubyte<3>(hi), bi))};
          const int ch = wpc * PW + (e % PW);  // logical 16-byte chunk (8 values)
          *reinterpret_cast<u32x4*>(rowp + ((ch ^ r7) << 3)) = o;
        } else {
          // two words (8 codes) per 16-byte chunk, written with the even word:
          // the same 16-byte LDS stores as the 4-bit path (8-byte stores of
          // one word each conflicted on 16% of the LDS cycles)
          if ((e & 1) == 0) {
            const uint32_t w1 = wreg[pp][(e % PW) + 1];
            const u32x4 o = {pack_xt2<XT>(__builtin_fmaf(sc, cvt_ubyte<0>(w), bi), __builtin_fmaf(sc, cvt_ubyte<1>(w), bi)),
                             pack_xt2<XT>(__builtin_fmaf(sc, cvt_ubyte<2>(w), bi), __builtin_fmaf(sc, cvt_ubyte<3>(w), bi)),
                             pack_xt2<XT>(__builtin_fmaf(sc, cvt_ubyte<0>(w1), bi), __builtin_fmaf(sc, cvt_ubyte<1>(w1), bi)),
                             pack_xt2<XT>(__builtin_fmaf(sc, cvt_ubyte<2>(w1), bi), __builtin_fmaf(sc, cvt_ubyte<3>(w1), bi))};
            const int ch = wpc * (PW / 2) + (e % PW) / 2;  // logical 16-byte chunk (8 values)
            *reinterpret_cast<u32x4*>(rowp + ((ch ^ r7) << 3)) = o;
          }
        }
      } else {
        // fp4 code points times a normal power of two are exact in bf16 (one
        // scaled conversion per pair); 2^-127 and NaN take the explicit product
        const uint32_t sb = sbw[pp];
        const float sc = e8m0_to_f32(sb);
        uint32_t o[4];
        if (sb - 1u < 254u) {
          unpack_mxfp4_scaled(w, sc, o);
        } else {
          uint32_t v[4];
          unpack_mxfp4(w, v);
#pragma unroll
          for (int h = 0; h < 4; h++)
            o[h] = pack_bf16x2(bf16_bits_to_f32(v[h] & 0xFFFFu) * sc, bf16_bits_to_f32(v[h] >> 16) * sc);
        }
        const int ch = wpc * PW + (e % PW);
        *reinterpret_cast<u32x4*>(rowp + ((ch ^ r7) << 3)) = u32x4{o[0], o[1], o[2], o[3]};
      }
    }
  };

  zero_acc();

  // fragment of 32 x 32 x 16: lane holds row/column (lane % 32), k 8 * (lane / 32) .. + 8;
  // slice s reads logical chunk 2 s + lane / 32 of its row, stored at that ^
  // swz(row); fragment tile i's rows are 32 i + fr past a multiple of 64, so
  // swz(row) = (fr & 7) ^ (fr >> 3) ^ 4 (i & 1)
  const int c0 = (lane >> 5) ^ (fr & 7) ^ (fr >> 3);
  const int arow = (wm * TM + fr) * RS, brow = (wn * TN + fr) * RS;
  static_assert(TM % 64 == 0 && TN % 64 == 0, "wave tiles start at multiples of 64 rows");
  int soff2[2][NPART];
#pragma unroll
  for (int s = 0; s < NPART; s++) {
    soff2[0][s] = ((2 * s) ^ c0) << 3;
    soff2[1][s] = ((2 * s) ^ c0 ^ 4) << 3;
  }


  // Steady state: step ks computes from buffer ks&1 while step ks+1 goes to
  // the other buffer (first two slices) and step ks+2 is loaded.  A barrier
  // after those stores publishes the other buffer, so the last slice can
  // already fetch the first fragments of step ks+1; the barrier at the end of
  // the step keeps the next step's stores off the buffer still being read.
  // Steps past ks1 load (bounds-checked) and store into a buffer nobody
  // reads, which keeps the slice code free of branches so the scheduler can
  // interleave it.
  if (ks0 < ks1) {
    {
      const int c = ks0 / SPC;
      chunk_load(c);
      chunk_write(c);
      if ((ks0 + 1) % SPC == 0 && ks0 + 1 < ks1) {
        chunk_load(c + 1);
        chunk_write(c + 1);
      }
      if ((ks0 + 2) % SPC == 0 && ks0 + 2 < ks1) chunk_load((ks0 + 2) / SPC);
    }
    load_step(ks0);
    __syncthreads();
    table_read(ks0);
#pragma unroll
    for (int p = 0; p < NPART; p++) store_part(0, p);
    load_step(ks0 + 1);
    __syncthreads();
    bf16x8 af[2][FM], bv[2][FN];
#pragma unroll
    for (int i = 0; i < FM; i++) af[0][i] = *reinterpret_cast<const bf16x8*>(xs[0] + arow + i * 32 * RS + soff2[i & 1][0]);
#pragma unroll
    for (int j = 0; j < FN; j++) bv[0][j] = *reinterpret_cast<const bf16x8*>(wsm[0] + brow + j * 32 * RS + soff2[j & 1][0]);
    for (int ks = ks0; ks < ks1; ks++) {
      // scale chunks: table of step ks+2 written now (published by this
      // step's barriers), loads for step ks+3 issued a step ahead
      if ((ks + 2) % SPC == 0 && ks + 2 < ks1) chunk_write((ks + 2) / SPC);
      if ((ks + 3) % SPC == 0 && ks + 3 < ks1) chunk_load((ks + 3) / SPC);
      table_read(ks + 1);
      const int buf = (ks - ks0) & 1;
      const uint16_t* xb = xs[buf];
      const uint16_t* wb = wsm[buf];
#pragma unroll
      for (int s = 0; s < NPART; s++) {
        const int cur = s & 1;
        if (s + 1 < NPART) {
#pragma unroll
          for (int i = 0; i < FM; i++)
            af[cur ^ 1][i] = *reinterpret_cast<const bf16x8*>(xb + arow + i * 32 * RS + soff2[i & 1][s + 1]);
#pragma unroll
          for (int j = 0; j < FN; j++)
            bv[cur ^ 1][j] = *reinterpret_cast<const bf16x8*>(wb + brow + j * 32 * RS + soff2[j & 1][s + 1]);
        } else {
          // first fragments of step ks+1 (published by the barrier after slice 1)
          const uint16_t* xn = xs[buf ^ 1];
          const uint16_t* wnx = wsm[buf ^ 1];
#pragma unroll
          for (int i = 0; i < FM; i++)
            af[cur ^ 1][i] = *reinterpret_cast<const bf16x8*>(xn + arow + i * 32 * RS + soff2[i & 1][0]);
#pragma unroll
          for (int j = 0; j < FN; j++)
            bv[cur ^ 1][j] = *reinterpret_cast<const bf16x8*>(wnx + brow + j * 32 * RS + soff2[j & 1][0]);
        }
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
          for (int j = 0; j < FN; j++) acc[i][j] = mfma32x32x16_xt<XT>(bv[cur][j], af[cur][i], acc[i][j]);
        // step ks+1 goes to the other buffer in the first two slices, then
        // the registers take the loads of step ks+2
        if (s == 0) {
          store_part(buf ^ 1, 0);
          store_part(buf ^ 1, 1);
        } else if (s == 1) {
          store_part(buf ^ 1, 2);
          store_part(buf ^ 1, 3);
          load_step(ks + 2);
        }
        // interleave within the slice: one MFMA, then a share of the VALU,
        // LDS and global-load work; slices are scheduled one by one
        constexpr int NMF = FM * FN;
        // the next slice's fragment reads go out first, a whole slice of
        // MFMAs ahead of their use
        __builtin_amdgcn_sched_group_barrier(0x100, FM + FN, 0);  // DS read
#pragma unroll
        for (int q = 0; q < NMF; q++) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);             // MFMA
          __builtin_amdgcn_sched_group_barrier(0x002, kValuPerMfma, 0);  // VALU
          __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);             // DS write
          __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);             // VMEM read
        }
        __builtin_amdgcn_sched_barrier(0);
        if (s == 1) __syncthreads();  // step ks+1's buffer complete
      }
      __syncthreads();  // step ks's buffer no longer read
    }
  }

  };

  // ---- epilogue ---------------------------------------------------------------
  // The products ran as (weights, activations), so block (i, j) of a lane
  // holds activation row m = wm TM + 32 i + (lane % 32) and weight columns
  // n = wn TN + 32 j + 8 t + 4 (lane / 32) + r at acc[i][j][4 t + r]: four
  // consecutive columns.  The tile goes through the (now free) staging LDS,
  // 16-byte chunk c of a row at c ^ (row % chunks per row), and leaves as
  // 16-byte row pieces (per-element stores of the accumulators took ~8%
  // longer at M = 2048).  fp32 split-K partials go one wave row at a time.
  auto out_row = [&](int tr) -> int64_t { return a.seg ? (int64_t)a.orows[r0 + tr] : (int64_t)(m0 + tr); };
  // the tile's result, rounded to the 16-bit type
  auto store_out = [&]() {
    constexpr int CPR = BN / 8;  // 16-byte chunks per row (8 values)
    uint16_t* ot = reinterpret_cast<uint16_t*>(stage);
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int j = 0; j < FN; j++) {
        const int m = wm * TM + i * 32 + fr;
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const int c = (wn * TN + j * 32 + 8 * q) >> 3;
          const u32x2 pr = {pack_xt2<XT>(acc[i][j][4 * q], acc[i][j][4 * q + 1]),
                            pack_xt2<XT>(acc[i][j][4 * q + 2], acc[i][j][4 * q + 3])};
          *reinterpret_cast<u32x2*>(ot + m * BN + ((c ^ (m & (CPR - 1))) << 3) + 4 * (lane >> 5)) = pr;
        }
      }
    __syncthreads();
    const int64_t ldo = a.ldo > 0 ? a.ldo : N;  // output row stride (a column block of a wider result)
    const bool vec = ((N | ldo) & 7) == 0 && (reinterpret_cast<uintptr_t>(a.out) & 15) == 0;
    for (int idx = t; idx < BM * CPR; idx += NT) {
      const int m = idx / CPR, c = idx - m * CPR;
      const int n = n0 + 8 * c;
      if (m >= rows || n >= N) continue;
      const u32x4 v = *reinterpret_cast<const u32x4*>(ot + m * BN + ((c ^ (m & (CPR - 1))) << 3));
      uint16_t* dst = a.out + out_row(m) * ldo + n;
      if (vec) {
        *reinterpret_cast<u32x4*>(dst) = v;
      } else {
        for (int e = 0; e < 8 && n + e < N; e++) dst[e] = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
      }
    }
  };
  // split z's fp32 partials of the tile, [z][M][N] in the workspace
  auto store_partials = [&](int z) {
    constexpr int CPR = BN / 4;  // 16-byte chunks per row (4 fp32)
    float* ot = reinterpret_cast<float*>(stage);
    const bool vec = (N & 3) == 0;
    for (int p = 0; p < NWM; p++) {  // one wave row of the tile per pass
      if (p > 0) __syncthreads();    // the previous pass has been read
      if (wm == p) {
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
          for (int j = 0; j < FN; j++) {
            const int mm = i * 32 + fr;
#pragma unroll
            for (int q = 0; q < 4; q++) {
              const int c = ((wn * TN + j * 32 + 8 * q) >> 2) + (lane >> 5);
              const f32x4 v = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
              *reinterpret_cast<f32x4*>(ot + mm * BN + ((c ^ (mm & (CPR - 1))) << 2)) = v;
            }
          }
      }
      __syncthreads();
      for (int idx = t; idx < TM * CPR; idx += NT) {
        const int mm = idx / CPR, c = idx - mm * CPR;
        const int m = p * TM + mm, n = n0 + 4 * c;
        if (m >= rows || n >= N) continue;
        const f32x4 v = *reinterpret_cast<const f32x4*>(ot + mm * BN + ((c ^ (mm & (CPR - 1))) << 2));
        float* dst = a.ws + ((int64_t)z * M + out_row(m)) * N + n;
        if (vec) {
          *reinterpret_cast<f32x4*>(dst) = v;
        } else {
          for (int e = 0; e < 4 && n + e < N; e++) dst[e] = v[e];
        }
      }
    }
  };

  // ---- stream-K (256 x 256 tiles on 8 waves, affine codes) -----------------
  // Workgroup b (XCD-contiguous runs of b, as below) takes K-steps
  // [b L, (b + 1) L) of the tiles' steps laid end to end, tile by tile, in
  // pieces.  With L at least a tile's K, a run starts with at most one tail
  // (the end of a tile whose head ends the previous run), then whole tiles,
  // then at most one head.  The tail comes first in its run and the head
  // last in the other, so the tail has normally been written long before
  // the head needs it: the tail's workgroup stores its fp32 accumulators
  // (agent scope, written through L2), waits for the stores and adds 1 to
  // the boundary's counter; the head's workgroup adds 1 too and, if the tail
  // was there, adds the saved tail to its accumulators (agent-scope loads)
  // and stores the tile.  If the tail was not there yet (its workgroup has
  // not run), the head saves its own accumulators, computes the tail itself
  // from zero and adds the saved head: the same one fp32 addition per
  // output, so the same bits.  Whoever arrives second puts the counter back
  // to 0.  No workgroup waits for another.
  if constexpr (SK) {
    static_assert(BM == 256 && BN == 256 && NWM * NWN == 8 && AFF, "stream-K: 256 x 256 tiles, 8 waves, affine codes");
    {
      __shared__ uint32_t sk_old;
      const int P = gridDim.x;
      int b = blockIdx.x;
      {
        const int q = P >> 3, r = P & 7, x = b & 7, j = b >> 3;
        b = x < r ? x * (q + 1) + j : r * (q + 1) + (x - r) * q + j;
      }
      const int nks = K / BK;
      const int64_t steps = (int64_t)a.tiles_m * a.tiles_n * nks;
      int64_t g = (int64_t)b * a.sk_len;
      const int64_t g1 = min(steps, g + (int64_t)a.sk_len);
      constexpr int NQ = FM * FN * 4;  // 16-byte accumulator pieces per lane
      // partials: region 0 the tails, region 1 the heads a fallback saves;
      // slot k is the tile cut by the boundary between runs k - 1 and k;
      // piece idx of (wave, lane) at [region][k][wave][idx][lane] (16 bytes)
      const __amdgpu_buffer_rsrc_t pr = buffer_rsrc(a.ws, (uint32_t)((int64_t)2 * P * BM * BN * 4));
      auto piece_off = [&](int region, int k, int idx) -> uint32_t {
        return (uint32_t)((((((int64_t)region * P + k) * (NT / 64) + wave) * NQ + idx) * 64 + lane) * 16);
      };
      auto save = [&](int region, int k) {
#pragma unroll
        for (int idx = 0; idx < NQ; idx++) {
          const int i = idx / (FN * 4), j = (idx / 4) % FN, q = idx % 4;
          const f32x4 v = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), pr, piece_off(region, k, idx), 0,
                                                 kAgentScope);
        }
      };
      auto add_saved = [&](int region, int k) {
        constexpr int HB = NQ / 4;  // a quarter of the pieces' loads in flight at a time
#pragma unroll
        for (int h = 0; h < NQ / HB; h++) {
          f32x4 v[HB];
#pragma unroll
          for (int u = 0; u < HB; u++)
            v[u] = __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(pr, piece_off(region, k, h * HB + u), 0, kAgentScope));
#pragma unroll
          for (int u = 0; u < HB; u++) {
            const int idx = h * HB + u, i = idx / (FN * 4), j = (idx / 4) % FN, q = idx % 4;
#pragma unroll
            for (int e = 0; e < 4; e++) acc[i][j][4 * q + e] += v[u][e];
          }
        }
      };
      auto arrive = [&](int k) -> uint32_t {
        __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores have completed
        __syncthreads();
        if (t == 0) sk_old = __hip_atomic_fetch_add(a.cnt + k, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        return sk_old;
      };
      auto reset = [&](int k) {
        if (t == 0) __hip_atomic_store(a.cnt + k, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      };
      int fb_tile = -1, fb_ks = 0;
      for (;;) {
        int tile, ks0, ks1, mode;  // 0 whole tile, 1 tail, 2 head, 3 a fallback's tail
        if (fb_tile >= 0) {
          tile = fb_tile;
          ks0 = fb_ks;
          ks1 = nks;
          mode = 3;
        } else if (g < g1) {
          tile = (int)(g / nks);
          ks0 = (int)(g - (int64_t)tile * nks);
          ks1 = (int)min((int64_t)nks, ks0 + (g1 - g));
          mode = ks0 > 0 ? 1 : (ks1 < nks ? 2 : 0);
          g += ks1 - ks0;
        } else {
          break;
        }
        const int tm = a.m_fast ? tile % a.tiles_m : tile / a.tiles_n;
        const int tn = a.m_fast ? tile / a.tiles_m : tile % a.tiles_n;
        run_piece(tm, tn, ks0, ks1);
        if (mode == 0) {
          store_out();
        } else if (mode == 1) {
          save(0, b);
          if (arrive(b) == 1u) reset(b);
        } else if (mode == 2) {
          const bool tail_there = arrive(b + 1) == 1u;
          if (tail_there) reset(b + 1);
          if (tail_there && !a.sk_fallback) {
            add_saved(0, b + 1);
            store_out();
          } else {
            save(1, b + 1);
            fb_tile = tile;
            fb_ks = ks1;
          }
        } else {
          __builtin_amdgcn_s_waitcnt(0);  // the saved head has completed
          add_saved(1, b + 1);
          store_out();
          fb_tile = -1;
        }
        __syncthreads();  // the epilogue's LDS reads are done before the next piece stages
      }
      return;
    }
  }

  // ---- workgroup -> (split, tile): XCD-contiguous runs --------------------
  const int T = a.tiles_m * a.tiles_n;
  const int G = T * a.ksplit;
  int b = blockIdx.x;
  {
    const int q = G >> 3, r = G & 7, x = b & 7, j = b >> 3;
    b = x < r ? x * (q + 1) + j : r * (q + 1) + (x - r) * q + j;
  }
  const int z = b / T, tt = b - z * T;
  const int tm = a.m_fast ? tt % a.tiles_m : tt / a.tiles_n;
  const int tn = a.m_fast ? tt / a.tiles_m : tt % a.tiles_n;
  if (a.seg && tm >= (int)a.nseg_dev[0]) return;
  const int nks = a.ksteps_per_split;
  const int ks0 = z * nks;
  run_piece(tm, tn, ks0, min(ks0 + nks, K / BK));
  if (a.ksplit > 1) store_partials(z);
  else store_out();
}

// ---- host ------------------------------------------------------------------

namespace {
// Tile codes: 0 = 256 x 128, 1 = 256 x 256, 2 = 128 x 128, 3 = 64 x 128
// (16x16-MFMA kernel, grid (n, m, split)); 4 = 256 x 256 (8 waves), 5 = 256 x 128,
// 6 = 128 x 128, 7 = 256 x 256 (4 waves), 8 = 256 x 128 (8 waves, 4 x 2)
// (32x32-MFMA tile kernel, 1-D XCD-ordered grid).
constexpr int kTiles = 9;
const int kBM[kTiles] = {256, 256, 128, 64, 256, 256, 128, 256, 256};
const int kBN[kTiles] = {128, 256, 128, 128, 256, 128, 128, 256, 128};
bool is_tile_kernel(int tile) { return tile >= 4; }
}  // namespace

int qmm_tile_rows(int tile) { return tile >= 0 && tile < kTiles ? kBM[tile] : 0; }

QmmPlan qmm_plan(int fmt, int gs, int64_t M, int64_t N, int64_t K, int num_cus, int tile_req, int ksplit_req,
                 int mix, int streamk) {
  QmmPlan p;
  const int bits = fmt == AFF8 ? 8 : 4;
  if (K % BK != 0 || K % gs != 0 || M <= 0 || N <= 0) return p;
  if (M * K * 2 >= ((int64_t)1 << 31) || N * K * bits / 8 >= ((int64_t)1 << 31)) return p;
  const int nks = (int)(K / BK);
  auto tiles_of = [&](int t) { return ((M + kBM[t] - 1) / kBM[t]) * ((N + kBN[t] - 1) / kBN[t]); };
  int tile;
  if (tile_req >= 0 && tile_req < kTiles) {
    tile = tile_req;
  } else {
    // 256 x 256 (8 waves) when there are enough tiles or K is long enough
    // for a K split to fill the CUs; else 128 x 128, two workgroups per CU.
    // Up to ~512 rows, 256 x 128 on 8 waves where it measured faster: long K
    // (split, down projections: 88-89 us vs 91-93 at M=512), 8-bit codes
    // with ~one tile per CU (gate/up M=512: 83 us vs 94) and 4-bit codes
    // with 0.75-1 tile per CU (gate/up M=384-512: 83-85 us vs 95, steady
    // state; at M=768, 1.3 tiles per CU, 162 vs 127).  Measured on MI355X at
    // the Llama-3-8B prefill shapes.
    // At 129-256 rows (less than one 256 x 128 tile per CU) the same tile
    // with a K split measured best too (gate/up M=256: 51.8 us vs 62 on 128 x
    // 128).
    const bool mid_rows = M > 128 && M <= 768;
    const int64_t t8 = tiles_of(8);
    const bool one_round8 = (fmt == AFF8 && t8 * 4 >= (int64_t)num_cus * 3) || (fmt != MXFP4 && t8 <= num_cus);
    if (mid_rows && (K >= 8192 || one_round8)) tile = 8;
    else tile = (M > 128 && (tiles_of(4) >= num_cus / 2 || K >= 8192)) ? 4 : 6;
  }
  p.tile = tile;
  p.rows_per_tile = kBM[tile];
  p.tiles_n = (int)((N + kBN[tile] - 1) / kBN[tile]);
  p.tiles_m = (int)((M + kBM[tile] - 1) / kBM[tile]);
  const int64_t tiles = (int64_t)p.tiles_n * p.tiles_m;
  int ks = 1;
  if (ksplit_req > 0) {
    ks = ksplit_req;
  } else {
    // split K while the grid covers less than the CUs (up to two workgroups
    // per CU for few rows, where each tile is cheap) and each split keeps >= 8
    // K-steps (gate/up M=32-128: 448 workgroups 31-38 us, 896 37-50 us)
    if (M <= 128) {
      while (tiles * ks * 2 <= 2 * num_cus && nks / (ks * 2) >= 8) ks *= 2;
    } else {
      while (tiles * ks * 2 <= num_cus && nks / (ks * 2) >= 8) ks *= 2;
    }
  }
  p.ksteps_per_split = (nks + ks - 1) / ks;
  p.ksplit = (nks + p.ksteps_per_split - 1) / p.ksteps_per_split;
  // consecutive tiles along M share weights, along N share activations: walk
  // along the dimension whose operand is the smaller of the two to re-read
  p.m_fast = M * K * 2 <= N * K * bits / 8 ? 1 : 0;
  p.ok = tiles * p.ksplit < ((int64_t)1 << 31);
  // Part-full last round: more 256 x 256 tiles than CUs, and the columns
  // past the whole rounds fit one round of 256 x 128 tiles.  Whole columns
  // of 256 x 256 tiles fill the full rounds, the rest runs as that one round
  // of the narrower tile, about 0.65 of a 256 x 256 tile's time (MI355X,
  // gate/up K=4096: M=1280-1536 x N=14336 202 us vs 233, M=2048 x N=12288
  // 214 vs 234).  A 256 x 192 tail for M=2048 x N=14336 measured slower
  // than the second 256 x 256 round (246 vs 240), so none is planned there.
  // Stream-K: one workgroup per CU takes an equal run of the 256 x 256
  // tiles' K-steps laid end to end, so a last round holding only a few tiles
  // does not leave the other CUs idle; a tile cut by a run boundary meets
  // through one fp32 partial.  Runs of at least a tile's K plus 8 steps keep
  // a cut tile's tail (the start of the next run) well ahead of its head
  // (the end of this run).  Taken when the last round holds at most 1/8 of
  // the CUs' tiles: the runs start their tiles at different K-steps, so
  // workgroups that share operands no longer read them from L2 at the same
  // time, which costs ~30% per step (MI355X, K=4096, 4-bit: 12288 x 1536
  // rows, 1.125 rounds, 170.5 us vs 196.6 on the two-launch plan; 14336 x
  // 2048 rows, 1.75 rounds, 269 vs 233).  streamk > 1 forces that run length.
  if (streamk && tile_req < 0 && ksplit_req <= 0 && p.tile == 4 && p.ksplit == 1 && tiles > num_cus &&
      fmt != MXFP4 && (streamk > 1 || (tiles < 2 * (int64_t)num_cus && (tiles - num_cus) * 8 <= num_cus))) {
    const int64_t steps = tiles * nks;
    const int64_t len = streamk > 1 ? streamk : (steps + num_cus - 1) / num_cus;
    if (len >= nks + 8 && len < ((int64_t)1 << 30) && (steps + len - 1) / len <= num_cus) {
      p.sk_len = (int)len;
      p.sk_wgs = (int)((steps + len - 1) / len);
      return p;
    }
  }
  if (mix && tile_req < 0 && ksplit_req <= 0 && p.tile == 4 && p.ksplit == 1 && tiles > num_cus) {
    const int64_t nb = (tiles / num_cus) * num_cus / p.tiles_m;  // 256-wide column tiles in whole rounds
    const int64_t n1 = nb * kBN[4];
    const int64_t tn2 = (N - n1 + kBN[8] - 1) / kBN[8];
    if (n1 > 0 && n1 < N && tn2 * p.tiles_m <= num_cus) {
      p.tile2 = 8;
      p.n_first = (int)n1;
      p.tiles_n2 = (int)tn2;
      p.tiles_n = (int)nb;
    }
  }
  return p;
}

namespace {
template <int FMT, int XT>
void qmm_tile_launch1(const QmmArgs& a, int tile, int ksplit, hipStream_t stream) {
  const dim3 grid((unsigned)((int64_t)a.tiles_m * a.tiles_n * ksplit));
  switch (tile) {
    case 4: hipLaunchKernelGGL((qmm_tile_kernel<FMT, 256, 256, 2, 4, XT>), grid, dim3(512), 0, stream, a); break;
    case 5: hipLaunchKernelGGL((qmm_tile_kernel<FMT, 256, 128, 2, 2, XT>), grid, dim3(256), 0, stream, a); break;
    case 7: hipLaunchKernelGGL((qmm_tile_kernel<FMT, 256, 256, 2, 2, XT>), grid, dim3(256), 0, stream, a); break;
    case 8: hipLaunchKernelGGL((qmm_tile_kernel<FMT, 256, 128, 4, 2, XT>), grid, dim3(512), 0, stream, a); break;
    default: hipLaunchKernelGGL((qmm_tile_kernel<FMT, 128, 128, 2, 2, XT>), grid, dim3(256), 0, stream, a); break;
  }
}

template <int FMT, int XT>
void qmm_tile_launch(const QmmArgs& a, const QmmPlan& p, hipStream_t stream) {
  if (p.sk_len > 0) {
    QmmArgs ak = a;
    ak.sk_len = p.sk_len;
    if constexpr (FMT != MXFP4)
      hipLaunchKernelGGL((qmm_tile_kernel<FMT, 256, 256, 2, 4, XT, true>), dim3((unsigned)p.sk_wgs), dim3(512), 0,
                         stream, ak);
    return;
  }
  if (p.tile2 < 0) {
    qmm_tile_launch1<FMT, XT>(a, p.tile, p.ksplit, stream);
    return;
  }
  // columns [0, n_first) on p.tile, then [n_first, N) on p.tile2: the second
  // launch sees the weight rows, scale rows and result columns from n_first
  // on, with the result's full row stride
  QmmArgs a1 = a;
  a1.N = p.n_first;
  a1.ldo = a.N;
  qmm_tile_launch1<FMT, XT>(a1, p.tile, 1, stream);
  constexpr int BITS = FMT == AFF8 ? 8 : 4;
  const int64_t n1 = p.n_first;
  const int64_t groups = (int64_t)a.K >> a.gs_shift;
  QmmArgs a2 = a;
  a2.w = a.w + n1 * ((int64_t)a.K * BITS / 32);
  a2.scales = reinterpret_cast<const uint8_t*>(a.scales) + n1 * groups * (FMT != MXFP4 ? 2 : 1);
  a2.biases = a.biases ? a.biases + n1 * groups : a.biases;
  a2.out = a.out + n1;
  a2.N = a.N - p.n_first;
  a2.ldo = a.N;
  a2.tiles_n = p.tiles_n2;
  qmm_tile_launch1<FMT, XT>(a2, p.tile2, 1, stream);
}

template <int FMT>
void qmm_launch_fmt(const QmmArgs& a, const QmmPlan& p, hipStream_t stream) {
  if (is_tile_kernel(p.tile)) {
    if constexpr (FMT != MXFP4) {
      if (a.xt == 1) {
        qmm_tile_launch<FMT, 1>(a, p, stream);
        return;
      }
    }
    qmm_tile_launch<FMT, 0>(a, p, stream);
    return;
  }
  const dim3 grid((unsigned)p.tiles_n, (unsigned)p.tiles_m, (unsigned)p.ksplit);
  switch (p.tile) {
    case 1: hipLaunchKernelGGL((qmm_kernel<FMT, 256, 256>), grid, dim3(NT), 0, stream, a); break;
    case 2: hipLaunchKernelGGL((qmm_kernel<FMT, 128, 128>), grid, dim3(NT), 0, stream, a); break;
    case 3: hipLaunchKernelGGL((qmm_kernel<FMT, 64, 128>), grid, dim3(NT), 0, stream, a); break;
    default: hipLaunchKernelGGL((qmm_kernel<FMT, 256, 128>), grid, dim3(NT), 0, stream, a); break;
  }
}
}  // namespace

QmmPlan qmm_plan_grouped(int fmt, int gs, int64_t N, int64_t K, int tile) {
  QmmPlan p;
  const int bits = fmt == AFF8 ? 8 : 4;
  if (K % BK != 0 || K % gs != 0 || N <= 0 || tile < 0 || tile >= kTiles) return p;
  if (N * K * bits / 8 >= ((int64_t)1 << 31)) return p;
  p.tile = tile;
  p.rows_per_tile = kBM[tile];
  p.tiles_n = (int)((N + kBN[tile] - 1) / kBN[tile]);
  p.tiles_m = 0;  // the caller sets the segment count
  p.ksplit = 1;
  p.ksteps_per_split = (int)(K / BK);
  p.m_fast = 0;
  p.ok = true;
  return p;
}

hipError_t qmm_launch(int fmt, const QmmArgs& a_in, const QmmPlan& p, hipStream_t stream) {
  if (!p.ok) return hipErrorInvalidValue;
  // float16: affine codes on the 32x32-MFMA tile kernel only
  if (a_in.xt != 0 && (fmt == MXFP4 || !is_tile_kernel(p.tile))) return hipErrorInvalidValue;
  if (p.sk_len > 0 && (p.tile != 4 || !a_in.ws || !a_in.cnt || a_in.seg || fmt == MXFP4)) return hipErrorInvalidValue;
  QmmArgs a = a_in;
  a.tiles_m = p.tiles_m;
  a.tiles_n = p.tiles_n;
  a.m_fast = p.m_fast;
  if (p.sk_len <= 0) a.sk_len = 0;
  switch (fmt) {
    case AFF4: qmm_launch_fmt<AFF4>(a, p, stream); break;
    case AFF8: qmm_launch_fmt<AFF8>(a, p, stream); break;
    default: qmm_launch_fmt<MXFP4>(a, p, stream); break;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.ksplit == 1) return e;
  return launch_splitk_reduce(a.ws, a.out, (int64_t)a.M * a.N, p.ksplit, stream, a.xt);
}

}  // namespace mlxq
