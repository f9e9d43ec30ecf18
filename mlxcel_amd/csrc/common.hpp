// common.hpp — shared device helpers for the gfx950 quantized-matmul kernels.
//
// Weight formats handled by every kernel (MLX packing, low bits first inside
// each uint32, overlays/rocm/mlx/ops.cpp:5231-5238):
//   AFF4  : affine 4-bit codes, 8 per word, bf16 scale and bias per group
//   AFF8  : affine 8-bit codes, 4 per word, bf16 scale and bias per group
//   MXFP4 : e2m1 codes, 8 per word, e8m0 (uint8) scale per group of 32
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mlxq {

enum Fmt : int { AFF4 = 0, AFF8 = 1, MXFP4 = 2 };

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---- bf16 <-> f32 (bit exact; round to nearest even, NaN -> 0x7FC0, which is
// MLX's `_MLX_BFloat16(float)`) ---------------------------------------------

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return u >> 16;
}

// e8m0 scale as float: 2^(s-127); s == 0 -> 2^-127 (float subnormal, as the
// bf16 0x0040 of overlays/cpu/.../quantized.cpp:97-101), s == 255 -> NaN.
__device__ __forceinline__ float e8m0_to_f32(uint32_t s) {
  uint32_t bits = (s == 0u) ? 0x00400000u : (s == 255u ? 0x7FC00000u : (s << 23));
  return __uint_as_float(bits);
}

// ---- gather indices ----------------------------------------------------------
// Segment sidx of a gather reads its expert / x batch from an index array of
// 32- or 64-bit integers (64-bit: the low word, which is the value cast to
// uint32 as the reference casts indices), clamped to the valid range; with no
// index array the expert is sidx (batched weights) or 0, the x batch
// sidx / div.
__device__ __forceinline__ int seg_index(const uint32_t* idx, int stride, int sidx, int clamp, int dflt) {
  if (!idx) return dflt;
  return (int)min(idx[(int64_t)sidx * (stride > 1 ? stride : 1)], (uint32_t)(clamp - 1));
}

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


// ---- MFMA ------------------------------------------------------------------
// v_mfma_f32_16x16x32_bf16: D[16x16] += A[16x32] * B[32x16], fp32 accumulate.
// Lane i holds A row (i % 16), B column (i % 16), both over the 8 k-slots
// 8*(i/16) .. 8*(i/16)+7; D rows 4*(i/16) .. +3 of column (i % 16).
__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
// the same product on the bit patterns of 16-bit operands of type XT
// (0 bfloat16, 1 float16: v_mfma_f32_16x16x32_f16)
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
template <int XT>
__device__ __forceinline__ f32x4 mfma16x16x32_xt(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (XT == 0)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
}

// ---- unpack one 32-bit word of codes into an MFMA bf16 operand fragment ----
//
// AFF4: 8 nibbles -> 8 bf16 "128 + q" (0x4300 | q is exactly 128+q in bf16),
// two per VGPR: VGPR p = (nibble p, nibble p+4).  The matching activation
// fragment is stored permuted the same way ([x0,x4,x1,x5,x2,x6,x3,x7]); the
// caller removes the 128*sum(x) offset.  The nibbles are split into bytes
// (lo: nibbles 0,2,4,6; hi: 1,3,5,7) and each pair is one v_perm_b32 that
// interleaves two of those bytes with 0x43 bytes: 7 instructions per word,
// all of them ordinary VALU operations the compiler schedules and sees.  (A
// hand-written v_and_or_b32 does the same in 7 too, but inline assembly is
// invisible to the compiler's hazard checks: it inserted no wait states
// between such a write and an MFMA reading the result, and the MFMA then read
// stale operands.)
// (`c` = 0x64646464 gives the float16 pairs 1024 + q instead.)
__device__ __forceinline__ void unpack_aff4(uint32_t w, uint32_t (&v)[4], uint32_t c = 0x43434343u) {
  const uint32_t lo = w & 0x0F0F0F0Fu;
  const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;
  v[0] = __builtin_amdgcn_perm(c, lo, 0x04020400u);  // (n0, n4): bytes lo.0, 0x43, lo.2, 0x43
  v[1] = __builtin_amdgcn_perm(c, hi, 0x04020400u);  // (n1, n5)
  v[2] = __builtin_amdgcn_perm(c, lo, 0x04030401u);  // (n2, n6)
  v[3] = __builtin_amdgcn_perm(c, hi, 0x04030401u);  // (n3, n7)
}

// MXFP4: 8 e2m1 codes -> 8 bf16 in natural order using the gfx950 FP4
// conversion (scale 1.0 keeps the code points exact: 0, .5, 1, 1.5, 2, 3, 4, 6).
__device__ __forceinline__ void unpack_mxfp4(uint32_t w, uint32_t (&v)[4]) {
  bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, 0);
  bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, 1);
  bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, 2);
  bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, 3);
  v[0] = __builtin_bit_cast(uint32_t, p0);
  v[1] = __builtin_bit_cast(uint32_t, p1);
  v[2] = __builtin_bit_cast(uint32_t, p2);
  v[3] = __builtin_bit_cast(uint32_t, p3);
}

// The same as float16 pairs (v_cvt_scalef32_pk_f16_fp4; the code points are
// exact in float16 too).
__device__ __forceinline__ void unpack_mxfp4_f16(uint32_t w, uint32_t (&v)[4]) {
  v[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 0));
  v[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 1));
  v[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 2));
  v[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 3));
}

// MXFP4 with its e8m0 scale folded in: v[h] = (code 2h, code 2h+1) * scale as
// bf16, for a normal power-of-two scale (exact: the products are fp4 code
// points times 2^k).
__device__ __forceinline__ void unpack_mxfp4_scaled(uint32_t w, float scale, uint32_t* v) {
  v[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 0));
  v[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 1));
  v[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 2));
  v[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 3));
}

// AFF8: two words = 8 byte codes -> 8 bf16 (exact: codes are < 256), natural
// order.  The f32 of a byte has a zero low half, so its bf16 is the high half;
// v_perm_b32 gathers the two high halves in one instruction.
__device__ __forceinline__ uint32_t pack_bf16x2_exact(float lo, float hi) {
  return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

__device__ __forceinline__ void unpack_aff8(uint32_t w0, uint32_t w1, uint32_t (&v)[4]) {
  v[0] = pack_bf16x2_exact((float)(w0 & 0xFFu), (float)((w0 >> 8) & 0xFFu));
  v[1] = pack_bf16x2_exact((float)((w0 >> 16) & 0xFFu), (float)(w0 >> 24));
  v[2] = pack_bf16x2_exact((float)(w1 & 0xFFu), (float)((w1 >> 8) & 0xFFu));
  v[3] = pack_bf16x2_exact((float)((w1 >> 16) & 0xFFu), (float)(w1 >> 24));
}

__device__ __forceinline__ bf16x8 as_bf16x8(const uint32_t (&v)[4]) {
  u32x4 t = {v[0], v[1], v[2], v[3]};
  return __builtin_bit_cast(bf16x8, t);
}

// Permute 8 consecutive bf16 (4 words, natural order) into the AFF4 operand
// order [x0,x4,x1,x5,x2,x6,x3,x7].
__device__ __forceinline__ u32x4 perm_aff4(u32x4 x) {
  u32x4 r;
  r[0] = (x[0] & 0xFFFFu) | (x[2] << 16);
  r[1] = (x[0] >> 16) | (x[2] & 0xFFFF0000u);
  r[2] = (x[1] & 0xFFFFu) | (x[3] << 16);
  r[3] = (x[1] >> 16) | (x[3] & 0xFFFF0000u);
  return r;
}

__device__ __forceinline__ float sum_bf16x8(u32x4 x) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; i++) s += bf16_bits_to_f32(x[i] & 0xFFFFu) + bf16_bits_to_f32(x[i] >> 16);
  return s;
}

// ---- buffer loads, dot products, cross-lane sums -------------------------------

constexpr int log2i(int v) { return v <= 1 ? 0 : 1 + log2i(v / 2); }

// A buffer offset past every operand (all operands of a launch stay below
// 2 GiB): bounds-checked buffer loads at it return 0.
constexpr uint32_t kDeadOfs = 0x80000000u;

// Cache-policy bit sc1 of buffer loads and stores (agent scope): stores
// write through the XCD's L2 and loads are not served from a stale L2 line
// of another XCD's data; the bits of relaxed agent-scope atomic loads and
// stores, so data shared between workgroups on different XCDs needs no L2
// writeback or invalidate.
constexpr int kAgentScope = 16;

// Raw buffer resource over [base, base + bytes): loads past the end return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// [first entry whose expert is >= v, first entry whose expert is >= v + 1)
// in the sorted index array, the two searches of lower_bound_sorted run in
// lockstep so each step costs one load round; wave-uniform.  The entries are
// read with bounds-checked buffer loads (no branch around a load, so the
// wave waits for them only where it compares).  `issued` runs once, right
// after the first round's loads are issued and before the wave waits for
// them: vector loads complete in order, so loads it issues stay in flight
// while the first round is consumed.
struct NoHook {
  __device__ void operator()() const {}
};
template <class Hook = NoHook>
__device__ __forceinline__ void sorted_run(const uint32_t* idx, int stride, int n, int clamp, int v, int lane,
                                           int& first, int& end, Hook&& issued = Hook{}) {
  if (n <= 0) {
    first = end = 0;
    return;
  }
  const int st = stride > 1 ? stride : 1;
  // n * st * 4 < 2^31: the callers' index arrays hold at most a few million entries
  const __amdgpu_buffer_rsrc_t ir = buffer_rsrc(idx, (uint32_t)((int64_t)n * st * 4));
  int lo[2] = {0, 0}, hi[2] = {n, n}, res[2] = {n, n};
  bool done[2] = {false, false};
  uint32_t raw[2];
  int step[2];
  bool in[2];
  // Lanes past the range read 0 (dead offset) and are masked out of the
  // ballots by `in`; the value itself is used unconditionally, so no branch
  // (and no wait) forms around the load.
  auto load_round = [&]() {
#pragma unroll
    for (int s = 0; s < 2; s++) {  // both loads in flight before either ballot
      step[s] = (hi[s] - lo[s] + 63) / 64;
      const int pos = lo[s] + lane * step[s];
      in[s] = !done[s] && pos < hi[s];
      raw[s] = __builtin_amdgcn_raw_buffer_load_b32(ir, in[s] ? (uint32_t)pos * (uint32_t)(st * 4) : kDeadOfs, 0, 0);
    }
  };
  auto consume = [&](int s) {
    const int val = (int)min(raw[s], (uint32_t)(clamp - 1));  // first use of the load
    const uint64_t below = __ballot(in[s] && val < v + s);
    const int c = __popcll(below), ns = __popcll(__ballot(in[s]));
    if (step[s] == 1) {
      res[s] = c < ns ? lo[s] + c : hi[s];
      done[s] = true;
    } else {
      const int nlo = c > 0 ? lo[s] + (c - 1) * step[s] + 1 : lo[s];
      const int nhi = c < ns ? lo[s] + c * step[s] : hi[s];
      lo[s] = nlo;
      hi[s] = nhi;
      if (lo[s] >= hi[s]) {
        res[s] = lo[s];
        done[s] = true;
      }
    }
  };
  // first round peeled (both searches live), so the hook's loads sit between
  // its loads and its comparisons in straight-line code
  load_round();
  __builtin_amdgcn_sched_barrier(0);
  issued();
  __builtin_amdgcn_sched_barrier(0);
  consume(0);
  consume(1);
  while (!done[0] || !done[1]) {
    load_round();
#pragma unroll
    for (int s = 0; s < 2; s++)
      if (!done[s]) consume(s);
  }
  first = res[0];
  end = res[1];
}


// c + a.lo * b.lo + a.hi * b.hi over bf16 pairs, fp32 accumulate
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
}

// 16-bit element type of activations, scales, biases and result: XT = 0
// bfloat16, XT = 1 float16 (the reference's quantized_matmul in T = float16,
// ops.cpp:4974-4992; same arithmetic: fp32 dot products of exact 16-bit
// products, one rounding of the result).  Affine codes widen to the type's
// "offset + q" pairs with one byte permute per pair: bfloat16 0x43nn =
// 128 + q (q < 128), float16 0x64nn = 1024 + q (q < 256, so 8-bit codes take
// the same route); the offset times sum(x) comes off with the bias.
template <int XT>
__device__ __forceinline__ float dotx(uint32_t a, uint32_t b, float c) {
  if constexpr (XT == 0) return dot2(a, b, c);
  else {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a), __builtin_bit_cast(h2, b), c, false);
  }
}
template <int XT>
__device__ __forceinline__ float xt_to_f32(uint32_t h) {
  if constexpr (XT == 0) return bf16_bits_to_f32(h);
  else return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}
template <int XT>
__device__ __forceinline__ uint32_t f32_to_xt(float f) {
  if constexpr (XT == 0) return f32_to_bf16_bits(f);
  else return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}


template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum CNT values per lane over each row of 16 lanes with DPP exchanges (no
// LDS round trips).  Step s pairs every lane with one whose bit (3 - s)
// differs: row_mirror (i <-> 15-i), row_half_mirror (i <-> 7-i in each half),
// then quad_perm swaps of bit 1 and bit 0; the pairs of successive steps
// never repeat a lane, so after four steps each value has been summed over
// all 16 lanes.  While more than one value is left, a step halves them: the
// lane with the bit set keeps the upper half and sends the lower.  Afterwards
// lane i (of its row) holds values [(i / Q) * C, (i / Q) * C + C) where
// C = max(CNT / 16, 1) and Q = max(16 / CNT, 1).
template <int CNT, int STEP>
__device__ __forceinline__ void row_butterfly(float* v, int lane) {
  if constexpr (STEP < 4) {
    constexpr int BIT = 8 >> STEP;
    constexpr int CTRL = STEP == 0 ? 0x140 : (STEP == 1 ? 0x141 : (STEP == 2 ? 0x4E : 0xB1));
    if constexpr (CNT > 1) {
      constexpr int H = CNT / 2;
      const bool up = (lane & BIT) != 0;
#pragma unroll
      for (int i = 0; i < H; i++) {
        const float keep = up ? v[i + H] : v[i];
        const float send = up ? v[i] : v[i + H];
        v[i] = keep + dpp<CTRL>(send);
      }
      row_butterfly<H, STEP + 1>(v, lane);
    } else {
      v[0] += dpp<CTRL>(v[0]);
      row_butterfly<1, STEP + 1>(v, lane);
    }
  }
}

// [x0,x1,x2,x3,x4,x5,x6,x7] (bf16, 4 words) -> [x0,x4,x1,x5,x2,x6,x3,x7]: the
// pair order of unpack_aff4
__device__ __forceinline__ u32x4 perm_aff4_v(u32x4 x) {
  return u32x4{__builtin_amdgcn_perm(x[2], x[0], 0x05040100u), __builtin_amdgcn_perm(x[2], x[0], 0x07060302u),
               __builtin_amdgcn_perm(x[3], x[1], 0x05040100u), __builtin_amdgcn_perm(x[3], x[1], 0x07060302u)};
}

}  // namespace mlxq
