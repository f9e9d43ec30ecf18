// moe.hip — fused single-token decode MoE for gfx950.
//
// The routed experts of one decode token, with affine-quantized weights:
//   gate_k[f] = sum_i x[i] * Wg[e_k][f][i],  up_k[f] likewise with Wu
//   act_k[f]  = A(gate_k[f]) * up_k[f]       (A = SiLU, or tanh-approximated GELU)
//   out[h]    = sum_k score[k] * sum_f act_k[f] * Wd[e_k][h][f]
// Reference: fused_moe_expert_kernel / fused_moe_geglu_kernel
// (src/lib/mlxcel-core/cpp/mlx_cxx_kernels.cpp:3817-4112; the kernels' math
// :3032-3170).  As there, two launches: the activations go through global
// memory in fp32 between them, every product and the sum over experts stay in
// fp32, and the result is rounded to bf16 once.  Unlike the reference (one
// 32-lane row per output and a separate reduction over the experts), the sum
// over experts happens inside the down kernel in a fixed order, so there is
// no partial buffer and no third launch, and results are bitwise
// reproducible.
//
// moe_gateup_kernel: one workgroup per (R output rows, expert slot).  Wave w
// reads the 16-byte lane chunks w*64 .. w*64+63 of each of its 2R weight rows
// (gate and up rows f0 .. f0+R-1), so one load instruction moves 1 KiB of
// consecutive bytes; the activation pieces of a lane's chunk are loaded once
// and serve all 2R rows.  Codes widen to bf16 pairs (4-bit: "128 + q", one
// byte permute per pair; 8-bit: exact via f32) and meet the bf16 activations
// in v_dot2_f32_bf16; a lane chunk lies in one quantization group, so
// y += s * sum(q' x) + b' * sum(x) once per chunk and row.
//
// moe_down_kernel: one workgroup per R output rows h.  Its lanes cover the
// (expert slot, lane chunk) pairs of those rows, so all slots of a row are
// summed inside one workgroup: per lane in fp32 FMAs of the fp32 activations
// with the codes (v_cvt_f32_ubyte / bit-field extracts), scaled by the slot's
// routing weight, then across lanes (DPP butterfly) and waves (LDS) in a
// fixed order.
#include "common.hpp"
#include "kernels.hpp"

namespace mlxq {

namespace {

__device__ __forceinline__ int moe_expert(const MoeArgs& a, int slot) {
  return seg_index(a.idx, a.idx_stride, slot, a.E, 0);
}

__device__ __forceinline__ float moe_score(const MoeArgs& a, int slot) {
  if (a.score_dt == 0) return reinterpret_cast<const float*>(a.scores)[slot];
  const uint16_t h = reinterpret_cast<const uint16_t*>(a.scores)[slot];
  if (a.score_dt == 1) return bf16_bits_to_f32(h);
  return (float)__builtin_bit_cast(_Float16, h);
}

// gate/up activation of the reference kernels (mlx_cxx_kernels.cpp:3096-3108)
template <int ACT>
__device__ __forceinline__ float moe_act(float g, float u) {
  if constexpr (ACT == MOE_GEGLU) {
    const float inner = 0.7978845608028654f * (g + 0.044715f * g * g * g);
    return 0.5f * g * (1.0f + tanhf(inner)) * u;
  } else {
    return g / (1.0f + expf(-g)) * u;
  }
}

// Stage V partials per lane for the cross-wave sum: the 16-lane rows are
// summed with the DPP butterfly, then each (wave, lane row) writes its V sums
// to red[(wave * 4 + lane row) * V + i] (red holds NW * 4 * V floats).  After
// the barrier that follows, moe_total adds them up in a fixed order.
template <int V>
__device__ __forceinline__ void moe_stage(float (&v)[V], float* red, int lane, int wave) {
  constexpr int VC = V >= 16 ? V / 16 : 1;  // partials per lane after the row butterfly
  constexpr int VQ = V >= 16 ? 1 : 16 / V;  // lanes per partial after it
  row_butterfly<V, 0>(v, lane);
  const int li = lane & 15;
  if (li % VQ == 0) {
#pragma unroll
    for (int c = 0; c < VC; c++) red[(wave * 4 + (lane >> 4)) * V + (li / VQ) * VC + c] = v[c];
  }
}

__device__ __forceinline__ float moe_total(const float* red, int V, int i, int nw) {
  float t = 0.f;
  for (int q = 0; q < nw * 4; q++) t += red[q * V + i];
  return t;
}

}  // namespace

// GB: gate/up bits (4 or 8); ACT: MOE_SWIGLU or MOE_GEGLU; R: output rows per
// workgroup (gate and up rows each).
template <int GB, int ACT, int R>
__global__ __launch_bounds__(512) void moe_gateup_kernel(const MoeArgs a) {
  constexpr int KL = 128 / GB;  // K positions per 16-byte lane chunk
  constexpr int XV = KL / 8;    // 16-byte activation pieces per chunk
  constexpr int NP = KL / 2;    // bf16 pairs per chunk
  constexpr int V = 2 * R;      // partials per lane: gate rows, then up rows
  __shared__ float red[kMoeMaxWaves * 4 * V];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int NW = blockDim.x >> 6;
  const int slot = blockIdx.y;
  const int e = moe_expert(a, slot);
  const int din = a.din, dff = a.dff;
  const int nlc = din / KL;
  const uint32_t RB = (uint32_t)nlc * 16u;  // bytes per weight row
  const int G = din >> a.gs_shift;
  const int f0 = blockIdx.x * R;

  // Rows past dff read as 0 (scale and bias too) and add exactly 0.
  const int64_t wb = (int64_t)e * dff * (RB / 4), sb = (int64_t)e * dff * G;
  const __amdgpu_buffer_rsrc_t gwr = buffer_rsrc(a.gate_w + wb, (uint32_t)dff * RB);
  const __amdgpu_buffer_rsrc_t uwr = buffer_rsrc(a.up_w + wb, (uint32_t)dff * RB);
  const uint32_t sbytes = (uint32_t)(dff * G * 2);
  const __amdgpu_buffer_rsrc_t gsr = buffer_rsrc(a.gate_s + sb, sbytes);
  const __amdgpu_buffer_rsrc_t gbr = buffer_rsrc(a.gate_b + sb, sbytes);
  const __amdgpu_buffer_rsrc_t usr = buffer_rsrc(a.up_s + sb, sbytes);
  const __amdgpu_buffer_rsrc_t ubr = buffer_rsrc(a.up_b + sb, sbytes);
  const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(a.x, (uint32_t)din * 2u);

  float yg[R], yu[R];
#pragma unroll
  for (int r = 0; r < R; r++) yg[r] = yu[r] = 0.f;

  for (int c0 = wave * 64; c0 < nlc; c0 += NW * 64) {  // wave-uniform
    const int c = c0 + lane;
    const bool live = c < nlc;
    const uint32_t xo = live ? (uint32_t)c * (KL * 2) : kDeadOfs;
    u32x4 xv[XV];
#pragma unroll
    for (int v = 0; v < XV; v++)
      xv[v] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, xo + v * 16u, 0, 0));
    const int g = (c * KL) >> a.gs_shift;
    uint32_t gs[R], gbi[R], us[R], ubi[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
      const uint32_t so = live ? (uint32_t)((f0 + r) * G + g) * 2u : kDeadOfs;
      gs[r] = __builtin_amdgcn_raw_buffer_load_b16(gsr, so, 0, 0);
      gbi[r] = __builtin_amdgcn_raw_buffer_load_b16(gbr, so, 0, 0);
      us[r] = __builtin_amdgcn_raw_buffer_load_b16(usr, so, 0, 0);
      ubi[r] = __builtin_amdgcn_raw_buffer_load_b16(ubr, so, 0, 0);
    }
    u32x4 wg[R], wu[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
      const uint32_t wo = live ? (uint32_t)(f0 + r) * RB + (uint32_t)c * 16u : kDeadOfs;
      wg[r] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(gwr, wo, 0, 2 /* nt */));
      wu[r] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(uwr, wo, 0, 2 /* nt */));
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the arithmetic below the loads

    float xs = 0.f;
#pragma unroll
    for (int v = 0; v < XV; v++)
#pragma unroll
      for (int q = 0; q < 4; q++) xs = dot2(xv[v][q], 0x3F803F80u, xs);  // pairs times (1, 1)
    if constexpr (GB == 4) {
#pragma unroll
      for (int v = 0; v < XV; v++) xv[v] = perm_aff4_v(xv[v]);
    }

    auto row_dot = [&](const u32x4 w) -> float {
      uint32_t pr[NP];
      if constexpr (GB == 8) {
        uint32_t t[4];
        unpack_aff8(w[0], w[1], t);
#pragma unroll
        for (int q = 0; q < 4; q++) pr[q] = t[q];
        unpack_aff8(w[2], w[3], t);
#pragma unroll
        for (int q = 0; q < 4; q++) pr[4 + q] = t[q];
      } else {
#pragma unroll
        for (int q = 0; q < 4; q++) {
          uint32_t t[4];
          unpack_aff4(w[q], t);
#pragma unroll
          for (int j = 0; j < 4; j++) pr[4 * q + j] = t[j];
        }
      }
      float d = 0.f;
#pragma unroll
      for (int p = 0; p < NP; p++) d = dot2(pr[p], xv[p / 4][p % 4], d);
      return d;
    };
    // 4-bit codes carry +128 (bf16 0x43xx): b' = b - 128 s removes it
    auto fold = [&](float acc, float d, uint32_t sbits, uint32_t bbits) -> float {
      const float s = bf16_bits_to_f32(sbits & 0xFFFFu), b = bf16_bits_to_f32(bbits & 0xFFFFu);
      const float bp = GB == 4 ? __builtin_fmaf(-128.0f, s, b) : b;
      return __builtin_fmaf(s, d, __builtin_fmaf(bp, xs, acc));
    };
#pragma unroll
    for (int r = 0; r < R; r++) {
      yg[r] = fold(yg[r], row_dot(wg[r]), gs[r], gbi[r]);
      yu[r] = fold(yu[r], row_dot(wu[r]), us[r], ubi[r]);
    }
  }

  float v[V];
#pragma unroll
  for (int r = 0; r < R; r++) {
    v[r] = yg[r];
    v[R + r] = yu[r];
  }
  moe_stage<V>(v, red, lane, wave);
  __syncthreads();
  if ((int)threadIdx.x < R) {
    const int r = threadIdx.x;
    const int f = f0 + r;
    const float gt = moe_total(red, V, r, NW), ut = moe_total(red, V, R + r, NW);
    if (f < dff) a.act[(int64_t)slot * dff + f] = moe_act<ACT>(gt, ut);
  }
}

// Codes of one lane chunk as floats, in K order: 4-bit (16 bytes, 32 codes,
// low nibble first), 8-bit (16 bytes, 16 codes) or 6-bit (12 bytes, 16 codes:
// code j is bits 6j .. 6j+5 of the little-endian 96-bit chunk, MLX's 3-byte
// packs of 4 codes, overlays/cpu/mlx/backend/cpu/quantized.cpp:1285-1297).
template <int DB>
__device__ __forceinline__ void moe_codes(const uint32_t* w, float* q) {
  if constexpr (DB == 4) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t lo = w[i] & 0x0F0F0F0Fu, hi = (w[i] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        q[8 * i + 2 * j] = (float)((lo >> (8 * j)) & 0xFFu);
        q[8 * i + 2 * j + 1] = (float)((hi >> (8 * j)) & 0xFFu);
      }
    }
  } else if constexpr (DB == 8) {
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) q[4 * i + j] = (float)((w[i] >> (8 * j)) & 0xFFu);
  } else {
#pragma unroll
    for (int j = 0; j < 16; j++) {
      const int bit = 6 * j, wi = bit >> 5, sh = bit & 31;
      uint32_t v;
      if (sh <= 26) v = __builtin_amdgcn_ubfe(w[wi], sh, 6);
      else v = __builtin_amdgcn_alignbit(w[wi + 1], w[wi], sh) & 63u;
      q[j] = (float)v;
    }
  }
}

// DB: down bits (4, 6 or 8); R: output rows per workgroup.
template <int DB, int R>
__global__ __launch_bounds__(512) void moe_down_kernel(const MoeArgs a) {
  constexpr int KL = DB == 6 ? 16 : 128 / DB;  // K positions per lane chunk
  constexpr int CW = DB * KL / 32;             // 32-bit words per lane chunk (4, or 3 for 6-bit)
  constexpr int AV = KL / 4;                   // 16-byte fp32 activation pieces per chunk
  __shared__ float red[kMoeMaxWaves * 4 * R];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int NW = blockDim.x >> 6;
  const int din = a.din, dff = a.dff;
  const int nlc = dff / KL;
  const int T = a.k * nlc;                   // (slot, chunk) pairs of a row
  const int RW = nlc * CW;                   // words per weight row
  const int G = dff >> a.gs_shift;
  const int h0 = blockIdx.x * R;
  const __amdgpu_buffer_rsrc_t ar = buffer_rsrc(a.act, (uint32_t)(a.k * dff) * 4u);

  float y[R];
#pragma unroll
  for (int r = 0; r < R; r++) y[r] = 0.f;

  for (int t0 = wave * 64; t0 < T; t0 += NW * 64) {  // wave-uniform
    const int t = t0 + lane;
    const bool live = t < T;
    const int slot = live ? t / nlc : 0;
    const int c = live ? t - slot * nlc : 0;
    const int e = moe_expert(a, slot);
    const float sc = live ? moe_score(a, slot) : 0.f;
    // Rows past din and dead lanes read row din-1 / chunk 0 of a valid
    // expert (in bounds) and their sums are discarded below.
    const int64_t row0 = (int64_t)e * din;
    const int g = (c * KL) >> a.gs_shift;
    uint32_t sraw[R], braw[R];
    uint32_t wv[R][CW];
#pragma unroll
    for (int r = 0; r < R; r++) {
      const int64_t row = row0 + min(h0 + r, din - 1);
      sraw[r] = a.down_s[row * G + g];
      braw[r] = a.down_b[row * G + g];
      const uint32_t* wp = a.down_w + row * RW + c * CW;
      if constexpr (CW == 4) {
        const u32x4 w4 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wp));
#pragma unroll
        for (int i = 0; i < 4; i++) wv[r][i] = w4[i];
      } else {
#pragma unroll
        for (int i = 0; i < CW; i++) wv[r][i] = __builtin_nontemporal_load(wp + i);
      }
    }
    const uint32_t ao = live ? (uint32_t)(slot * dff + c * KL) * 4u : kDeadOfs;
    f32x4 av[AV];
#pragma unroll
    for (int v = 0; v < AV; v++)
      av[v] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(ar, ao + v * 16u, 0, 0));
    __builtin_amdgcn_sched_barrier(0);  // keep the arithmetic below the loads

    float as = 0.f;
#pragma unroll
    for (int v = 0; v < AV; v++)
#pragma unroll
      for (int j = 0; j < 4; j++) as += av[v][j];
#pragma unroll
    for (int r = 0; r < R; r++) {
      float q[KL];
      moe_codes<DB>(wv[r], q);
      float d = 0.f;
#pragma unroll
      for (int j = 0; j < KL; j++) d = __builtin_fmaf(q[j], av[j / 4][j % 4], d);
      const float s = bf16_bits_to_f32(sraw[r]), b = bf16_bits_to_f32(braw[r]);
      const float part = sc * __builtin_fmaf(s, d, b * as);
      y[r] += (live && h0 + r < din) ? part : 0.f;
    }
  }

  moe_stage<R>(y, red, lane, wave);
  __syncthreads();
  if ((int)threadIdx.x < R) {
    const int h = h0 + threadIdx.x;
    const float tot = moe_total(red, R, threadIdx.x, NW);
    if (h < din) a.out[h] = (uint16_t)f32_to_bf16_bits(tot);
  }
}

// ---- host ------------------------------------------------------------------

namespace {

constexpr int kGateupRows = 4;  // gate/up output rows per workgroup
constexpr int kDownRows = 8;    // down output rows per workgroup

int moe_waves(int64_t lane_chunks) { return (int)std::min<int64_t>(kMoeMaxWaves, std::max<int64_t>(1, (lane_chunks + 63) / 64)); }

}  // namespace

hipError_t moe_launch(const MoeArgs& a, int gu_bits, int d_bits, int act, hipStream_t stream) {
  if (a.din <= 0 || a.dff <= 0 || a.k <= 0) return hipSuccess;
  const int klg = 128 / gu_bits;
  const int kld = d_bits == 6 ? 16 : 128 / d_bits;
  const dim3 ga((unsigned)((a.dff + kGateupRows - 1) / kGateupRows), (unsigned)a.k);
  const dim3 ba((unsigned)(64 * moe_waves(a.din / klg)));
  const dim3 gd((unsigned)((a.din + kDownRows - 1) / kDownRows));
  const dim3 bd((unsigned)(64 * moe_waves((int64_t)a.k * (a.dff / kld))));
  if (gu_bits == 4 && act == MOE_SWIGLU) hipLaunchKernelGGL((moe_gateup_kernel<4, MOE_SWIGLU, kGateupRows>), ga, ba, 0, stream, a);
  else if (gu_bits == 4) hipLaunchKernelGGL((moe_gateup_kernel<4, MOE_GEGLU, kGateupRows>), ga, ba, 0, stream, a);
  else if (act == MOE_SWIGLU) hipLaunchKernelGGL((moe_gateup_kernel<8, MOE_SWIGLU, kGateupRows>), ga, ba, 0, stream, a);
  else hipLaunchKernelGGL((moe_gateup_kernel<8, MOE_GEGLU, kGateupRows>), ga, ba, 0, stream, a);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  if (d_bits == 4) hipLaunchKernelGGL((moe_down_kernel<4, kDownRows>), gd, bd, 0, stream, a);
  else if (d_bits == 6) hipLaunchKernelGGL((moe_down_kernel<6, kDownRows>), gd, bd, 0, stream, a);
  else hipLaunchKernelGGL((moe_down_kernel<8, kDownRows>), gd, bd, 0, stream, a);
  return hipGetLastError();
}

}  // namespace mlxq
