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
// y += s * sum(q' x) + b' * sum(x) once per chunk and row.  The scales and
// biases of the wave's rows and chunk range come in with loads of up to 4
// groups and are staged in LDS as (s, b') pairs, one 8-byte read per row.
//
// Latency, not bandwidth, bounds both launches at decode sizes (about 14 MB
// and 7 MB for Qwen3-30B-A3B experts): each waits for the expert ids before
// its weight loads can start, a full memory round trip per launch.
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

// LDS of a gate/up workgroup: per wave, the cross-wave partials (4 lane rows
// x 2R) and the (scale, bias') pairs of its chunk range (2R rows x GC groups).
__host__ __device__ inline uint32_t moe_gateup_lds(int nw, int gc) {
  return (uint32_t)nw * (4 * 2 * kMoeGateupRows * 4 + 2 * kMoeGateupRows * gc * 8);
}

// GB: gate/up bits (4 or 8); ACT: MOE_SWIGLU or MOE_GEGLU; UPW: quantization
// groups per scale load (1, 2 or 4: the widest load every row's scales stay
// aligned for, from din / group_size).
template <int GB, int ACT, int UPW>
__global__ __launch_bounds__(512) void moe_gateup_kernel(const MoeArgs a) {
  constexpr int R = kMoeGateupRows;
  constexpr int KL = 128 / GB;  // K positions per 16-byte lane chunk
  constexpr int XV = KL / 8;    // 16-byte activation pieces per chunk
  constexpr int NP = KL / 2;    // bf16 pairs per chunk
  constexpr int V = 2 * R;      // rows per workgroup: gate rows, then up rows
  constexpr int SW = UPW == 4 ? 2 : 1;  // 32-bit words per scale load
  constexpr int MAXLD = 4 / UPW;        // scale loads per lane and array (at most)
  extern __shared__ __align__(16) unsigned char smem[];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int NW = blockDim.x >> 6;
  const int slot = blockIdx.y;
  const int e = moe_expert(a, slot);
  const int din = a.din, dff = a.dff;
  const int nlc = din / KL;
  const uint32_t RB = (uint32_t)nlc * 16u;  // bytes per weight row
  const int G = din >> a.gs_shift;
  const int GC = (64 * KL) >> a.gs_shift;   // groups per 64-lane chunk range (8 .. 64)
  const int upr = GC / UPW;                 // scale units per row and range
  const int f0 = blockIdx.x * R;
  float* red = reinterpret_cast<float*>(smem);
  float2* scl = reinterpret_cast<float2*>(smem + NW * 4 * V * 4) + wave * V * GC;

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

  float y[V];
#pragma unroll
  for (int r = 0; r < V; r++) y[r] = 0.f;

  for (int c0 = wave * 64; c0 < nlc; c0 += NW * 64) {  // wave-uniform
    const int c = c0 + lane;
    const bool live = c < nlc;
    const uint32_t xo = live ? (uint32_t)c * (KL * 2) : kDeadOfs;
    u32x4 xv[XV];
#pragma unroll
    for (int v = 0; v < XV; v++)
      xv[v] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, xo + v * 16u, 0, 0));

    // Scales and biases of the range's groups for the R gate and R up rows:
    // unit u = (row r = u / upr, groups gl*UPW .. +UPW-1), four loads (gate
    // s, b, up s, b) per unit; lanes past the units load nothing.
    const int gbase = (c0 * KL) >> a.gs_shift;
    uint32_t ld[MAXLD][4][SW];
#pragma unroll
    for (int i = 0; i < MAXLD; i++) {
      const int u = lane + 64 * i;
      const int r = u / upr, gl = u - r * upr;
      const uint32_t so = (u < R * upr) ? (uint32_t)((f0 + r) * G + gbase + gl * UPW) * 2u : kDeadOfs;
      const __amdgpu_buffer_rsrc_t rs[4] = {gsr, gbr, usr, ubr};
#pragma unroll
      for (int q = 0; q < 4; q++) {
        if constexpr (UPW == 4) {
          const u32x2 t = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs[q], so, 0, 0));
          ld[i][q][0] = t[0];
          ld[i][q][SW - 1] = t[1];
        } else if constexpr (UPW == 2) {
          ld[i][q][0] = __builtin_amdgcn_raw_buffer_load_b32(rs[q], so, 0, 0);
        } else {
          ld[i][q][0] = __builtin_amdgcn_raw_buffer_load_b16(rs[q], so, 0, 0);
        }
      }
    }
    u32x4 wv[V];
#pragma unroll
    for (int r = 0; r < R; r++) {
      const uint32_t wo = live ? (uint32_t)(f0 + r) * RB + (uint32_t)c * 16u : kDeadOfs;
      // default cache policy: measured faster than the streaming hint here
      wv[r] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(gwr, wo, 0, 0));
      wv[R + r] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(uwr, wo, 0, 0));
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the arithmetic below the loads

    // stage (s, b') per (row, group); 4-bit codes carry +128: b' = b - 128 s
#pragma unroll
    for (int i = 0; i < MAXLD; i++) {
      const int u = lane + 64 * i;
      if (u < R * upr) {
        const int r = u / upr, gl = u - r * upr;
#pragma unroll
        for (int h = 0; h < UPW; h++) {
#pragma unroll
          for (int half = 0; half < 2; half++) {  // gate, up
            const uint32_t sw = ld[i][2 * half][h >> 1], bw = ld[i][2 * half + 1][h >> 1];
            const float sv = bf16_bits_to_f32((sw >> (16 * (h & 1))) & 0xFFFFu);
            const float bv = bf16_bits_to_f32((bw >> (16 * (h & 1))) & 0xFFFFu);
            scl[(half * R + r) * GC + gl * UPW + h] = float2{sv, GB == 4 ? __builtin_fmaf(-128.0f, sv, bv) : bv};
          }
        }
      }
    }

    float xs = 0.f;
#pragma unroll
    for (int v = 0; v < XV; v++)
#pragma unroll
      for (int q = 0; q < 4; q++) xs = dot2(xv[v][q], 0x3F803F80u, xs);  // pairs times (1, 1)
    if constexpr (GB == 4) {
#pragma unroll
      for (int v = 0; v < XV; v++) xv[v] = perm_aff4_v(xv[v]);
    }
    // the wave reads only what it wrote, and its LDS operations complete in
    // order (this also fences the compiler)
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

    const int gme = (lane * KL) >> a.gs_shift;  // this lane's group within the range
#pragma unroll
    for (int r = 0; r < V; r++) {
      float2 sbp = scl[r * GC + gme];
      if (!live) sbp = float2{0.f, 0.f};  // lanes past the row add exactly 0
      uint32_t pr[NP];
      const u32x4 w = wv[r];
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
      y[r] = __builtin_fmaf(sbp.x, d, __builtin_fmaf(sbp.y, xs, y[r]));
    }
  }

  moe_stage<V>(y, red, lane, wave);
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
    // the activations do not depend on the expert id: in flight first
    const uint32_t ao = live ? (uint32_t)(slot * dff + c * KL) * 4u : kDeadOfs;
    f32x4 av[AV];
#pragma unroll
    for (int v = 0; v < AV; v++)
      av[v] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(ar, ao + v * 16u, 0, 0));
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

int moe_waves(int64_t lane_chunks) {
  return (int)std::min<int64_t>(kMoeMaxWaves, std::max<int64_t>(1, (lane_chunks + 63) / 64));
}

template <int GB, int ACT>
void launch_gateup(const MoeArgs& a, dim3 block, uint32_t lds, hipStream_t stream) {
  const dim3 grid((unsigned)((a.dff + kMoeGateupRows - 1) / kMoeGateupRows), (unsigned)a.k);
  const int64_t G = a.din >> a.gs_shift;
  if (G % 4 == 0) hipLaunchKernelGGL((moe_gateup_kernel<GB, ACT, 4>), grid, block, lds, stream, a);
  else if (G % 2 == 0) hipLaunchKernelGGL((moe_gateup_kernel<GB, ACT, 2>), grid, block, lds, stream, a);
  else hipLaunchKernelGGL((moe_gateup_kernel<GB, ACT, 1>), grid, block, lds, stream, a);
}

}  // namespace

hipError_t moe_launch(const MoeArgs& a, int gu_bits, int d_bits, int act, hipStream_t stream) {
  if (a.din <= 0 || a.dff <= 0 || a.k <= 0) return hipSuccess;
  const int klg = 128 / gu_bits;
  const int kld = d_bits == 6 ? 16 : 128 / d_bits;
  const int nwa = moe_waves(a.din / klg);
  const dim3 ba((unsigned)(64 * nwa));
  const uint32_t lds = moe_gateup_lds(nwa, (64 * klg) >> a.gs_shift);
  const dim3 bd((unsigned)(64 * moe_waves((int64_t)a.k * (a.dff / kld))));
  if (gu_bits == 4 && act == MOE_SWIGLU) launch_gateup<4, MOE_SWIGLU>(a, ba, lds, stream);
  else if (gu_bits == 4) launch_gateup<4, MOE_GEGLU>(a, ba, lds, stream);
  else if (act == MOE_SWIGLU) launch_gateup<8, MOE_SWIGLU>(a, ba, lds, stream);
  else launch_gateup<8, MOE_GEGLU>(a, ba, lds, stream);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  const dim3 gd((unsigned)((a.din + kMoeDownRows - 1) / kMoeDownRows));
  if (d_bits == 4) hipLaunchKernelGGL((moe_down_kernel<4, kMoeDownRows>), gd, bd, 0, stream, a);
  else if (d_bits == 6) hipLaunchKernelGGL((moe_down_kernel<6, kMoeDownRows>), gd, bd, 0, stream, a);
  else hipLaunchKernelGGL((moe_down_kernel<8, kMoeDownRows>), gd, bd, 0, stream, a);
  return hipGetLastError();
}

}  // namespace mlxq
