// Gated DeltaNet step on gfx950: constants and per-column device helpers shared by the
// one-workgroup kernel (gdn.hip) and the split kernels (gdn_split.hip). The two paths run the same
// per-column arithmetic from these helpers, which is what gives them the same bits.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

#include "qe_device.hpp"

namespace qe {

constexpr int GDN_D = 128;      // dk = dv
constexpr int GDN_RING = 16;
constexpr int GDN_MAXN = 8;
constexpr int GDN_THREADS = 1024;                   // one-workgroup kernel: 16 waves per head
constexpr int GDN_SPLIT = 4;                        // workgroups per head in the split kernel
constexpr int GDN_SPLIT_COLS = GDN_D / GDN_SPLIT;
constexpr int GDN_SPLIT_THREADS = 512;
constexpr int GDN_SPLIT_MIN_ROWS = 5;               // fewer rows: the one-workgroup kernel
constexpr int GDN_STAGE_MAX_ROWS = 2;               // up to this many: the state staged in LDS

struct __align__(16) F4 {
  float x, y, z, w;
};

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }

// Sum over the 16 lanes that share lane & 3 (lane bits 2..5): xor 8 and xor 4 by DPP within a
// 16-lane row, then xor 16 and xor 32 by the permlane swaps. Partners add the same two values,
// so all 16 lanes get the same bits.
__device__ __forceinline__ float colquad_sum(float v) {
  v = v + dpp<0x128>(v);             // row_ror:8 = lane ^ 8
  v = v + dpp<0x1B>(dpp<0x141>(v));  // row_half_mirror then quad_perm [3,2,1,0] = lane ^ 4
  return group4_sum(v);              // lane ^ 16, lane ^ 32
}

// One delta-rule update of this lane's 8 x NC block: S = decay S; kv = S^T k; delta =
// beta (v - kv); S += k delta^T. The identical instruction sequence serves replayed and new rows,
// and each column's arithmetic (an 8-term chain over rows 8 rg .. +7, then the 16-lane
// butterfly) does not depend on NC, so both kernels below compute the same state bits.
template <int NC>
__device__ __forceinline__ void delta_step(float (&s)[8][NC], const float (&k)[8],
                                           const float (&v)[NC], float decay, float beta) {
  float kv[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) kv[c] = 0.f;
#pragma unroll
  for (int r = 0; r < 8; ++r)
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      s[r][c] = s[r][c] * decay;
      kv[c] = fmaf(s[r][c], k[r], kv[c]);
    }
  float delta[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) delta[c] = (v[c] - colquad_sum(kv[c])) * beta;
#pragma unroll
  for (int r = 0; r < 8; ++r)
#pragma unroll
    for (int c = 0; c < NC; ++c) s[r][c] = fmaf(k[r], delta[c], s[r][c]);
}

// o = S^T q for this lane's columns, rounded to bf16 (the reference casts core_attn_out).
template <int NC>
__device__ __forceinline__ void read_out(const float (&s)[8][NC], const float (&q)[8],
                                         float (&o)[NC]) {
#pragma unroll
  for (int c = 0; c < NC; ++c) o[c] = 0.f;
#pragma unroll
  for (int r = 0; r < 8; ++r)
#pragma unroll
    for (int c = 0; c < NC; ++c) o[c] = fmaf(s[r][c], q[r], o[c]);
#pragma unroll
  for (int c = 0; c < NC; ++c) o[c] = round_bf16(colquad_sum(o[c]));
}

// Causal conv (4 taps, the HF buffer order [x_{t-3}, x_{t-2}, x_{t-1}, x_t]) and SiLU of row t of
// one channel; xs holds x at positions P-3 .. P+n-1. Rounds to bf16 after the conv and after SiLU.
__device__ __forceinline__ float conv_silu(const float (&cw)[4], const float (&xs)[3 + GDN_MAXN],
                                           int t) {
  float acc = cw[0] * xs[t];
  acc = fmaf(cw[1], xs[t + 1], acc);
  acc = fmaf(cw[2], xs[t + 2], acc);
  acc = fmaf(cw[3], xs[t + 3], acc);
  return round_bf16(silu_f(round_bf16(acc)));
}

// beta = bf16(sigmoid(b)); decay = exp(-exp(A_log) * softplus(a + dt_bias)), threshold 20.
__device__ __forceinline__ float2 gate_values(__bf16 bb, __bf16 ab, __bf16 dtb, __bf16 alb) {
  const float beta = round_bf16(sigmoid_f32(bf16_to_f32(bb)));
  const float x = bf16_to_f32(ab) + bf16_to_f32(dtb);
  const float sp = x > 20.f ? x : log1pf(expf(x));
  return make_float2(expf(-expf(bf16_to_f32(alb)) * sp), beta);
}

__device__ __forceinline__ void lds_read8(const float* p, float (&d)[8]) {
  const F4 a = *reinterpret_cast<const F4*>(p), b = *reinterpret_cast<const F4*>(p + 4);
  d[0] = a.x; d[1] = a.y; d[2] = a.z; d[3] = a.w; d[4] = b.x; d[5] = b.y; d[6] = b.z; d[7] = b.w;
}
__device__ __forceinline__ void lds_read4(const float* p, float (&d)[4]) {
  const F4 a = *reinterpret_cast<const F4*>(p);
  d[0] = a.x; d[1] = a.y; d[2] = a.z; d[3] = a.w;
}
// NC consecutive floats (NC = 1, 2 or 4), LDS or global memory: one vector access for 2 or 4.
template <int NC>
__device__ __forceinline__ void vec_read_n(const float* p, float (&d)[NC]) {
  if constexpr (NC == 4) {
    lds_read4(p, d);
  } else if constexpr (NC == 2) {
    const float2 a = *reinterpret_cast<const float2*>(p);
    d[0] = a.x; d[1] = a.y;
  } else {
#pragma unroll
    for (int c = 0; c < NC; ++c) d[c] = p[c];
  }
}
template <int NC>
__device__ __forceinline__ void vec_write_n(float* p, const float (&d)[NC]) {
  if constexpr (NC == 4) {
    *reinterpret_cast<F4*>(p) = F4{d[0], d[1], d[2], d[3]};
  } else if constexpr (NC == 2) {
    *reinterpret_cast<float2*>(p) = make_float2(d[0], d[1]);
  } else {
#pragma unroll
    for (int c = 0; c < NC; ++c) p[c] = d[c];
  }
}
// This lane's block of a head's state (rows 8 rg .. +7, columns col0 .. col0 + NC - 1 of the
// row-major [128][128] fp32 state): 8 loads of 4 NC bytes, and the write-back.
template <int NC>
__device__ __forceinline__ void load_state_rows(const float* Sj, int rg, int col0,
                                                float (&s)[8][NC]) {
#pragma unroll
  for (int rr = 0; rr < 8; ++rr) vec_read_n(Sj + (size_t)(rg * 8 + rr) * GDN_D + col0, s[rr]);
}
template <int NC>
__device__ __forceinline__ void store_state_rows(float* Sj, int rg, int col0,
                                                 const float (&s)[8][NC]) {
#pragma unroll
  for (int rr = 0; rr < 8; ++rr) vec_write_n(Sj + (size_t)(rg * 8 + rr) * GDN_D + col0, s[rr]);
}

// Gated RMSNorm of one output row of a head (wave-wide; lane holds columns 2 lane, 2 lane + 1):
// out = bf16(bf16(w * bf16(o * r)) * silu(z)), r = 1 / sqrt(sum(o^2) / 128 + eps). The sum of
// squares is four serial 32-column partials added in order, the same in every kernel, so every
// path gives the same bits.
__device__ __forceinline__ void gated_norm_row(const float* __restrict__ o_row, int lane, float nw0,
                                               float nw1, float z0, float z1, float eps,
                                               __bf16* __restrict__ op) {
  const float2 o = *reinterpret_cast<const float2*>(&o_row[2 * lane]);
  float part_ss = 0.f;
  if (lane < GDN_SPLIT) {
#pragma unroll
    for (int cc = 0; cc < GDN_D / GDN_SPLIT; ++cc)
      part_ss = fmaf(o_row[lane * (GDN_D / GDN_SPLIT) + cc], o_row[lane * (GDN_D / GDN_SPLIT) + cc],
                     part_ss);
  }
  float ss = 0.f;
#pragma unroll
  for (int g = 0; g < GDN_SPLIT; ++g)
    ss += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(part_ss), g));
  const float inv = 1.0f / sqrtf(ss / 128.0f + eps);
  const float y0 = round_bf16(nw0 * round_bf16(o.x * inv));  // bf16 weight * bf16 norm
  const float y1 = round_bf16(nw1 * round_bf16(o.y * inv));
  op[2 * lane] = f32_to_bf16(y0 * silu_f(z0));
  op[2 * lane + 1] = f32_to_bf16(y1 * silu_f(z1));
}

// Split path for 5-8 rows (gdn_split.hip): gdn_split_kernel then gdn_finish_kernel.
hipError_t launch_gdn_split(const __bf16* qkv, const __bf16* z, const __bf16* b, const __bf16* a,
                            long ldp, __bf16* ring, const __bf16* conv_w, const __bf16* A_log,
                            const __bf16* dt_bias, const __bf16* norm_w, float* S, float* st_k,
                            float* st_v, float* st_g, const int* ctl, __bf16* out, long ldo,
                            int n, int Hk, int Hv, float eps, hipStream_t stream);

}  // namespace qe
