// Gated DeltaNet step, split path for 5-8 rows: gdn_split_kernel (each value head's 128 state
// columns over 4 workgroups) followed by gdn_finish_kernel (one workgroup per head). Same
// per-column arithmetic as gdn_step_kernel (gdn.hip), so the same bits.
//
// This file is compiled with LLVM's max-ILP machine scheduler; the one-workgroup kernel in
// gdn.hip keeps the default. Same-box A/B of the whole Gated DeltaNet source under max-ILP, us
// per call at Hk 16 / Hv 48: 6 rows 15.36 -> 14.63, 8 rows 17.39 -> 16.48 (this path); 1 / 2 /
// 4 rows 7.92 / 9.51 / 12.68 -> 7.97 / 9.62 / 12.77 (the one-workgroup kernel). Same bits.
#include "gdn_common.hpp"

namespace qe {

// ------------------------------------------------------------------ split kernels
// The same step with each head's 128 state columns split over GDN_SPLIT workgroups of 512
// threads (32 columns each): four times the CUs for the state I/O and the delta-rule VALU work,
// which bound the one-workgroup kernel. Each workgroup holds rows 8 rg .. +7 of its columns per
// lane and runs the same per-column arithmetic, so the state is bit-identical to the
// one-workgroup kernel's. Every workgroup repeats the conv, l2norm and gates of its head's q and
// k (256 channels) and does the v channels of its own columns.
//
// Nothing waits across workgroups. What needs a whole head (the gated RMSNorm sums the squares
// of a row's 128 outputs) or must not overwrite what another part still reads (the staged k rows
// and gates of the previous call, which every part of a head replays) is left to a second
// kernel, gdn_finish_kernel: gdn_split_kernel writes each row's outputs o, already bf16 values,
// into `out` unnormalised, and stages only its own v columns; gdn_finish_kernel (one workgroup
// per head, after every part has finished) recomputes the head's normalised k rows and gates with
// the same arithmetic, stages them, and normalises `out` in place. Block b runs head b % Hv, part
// b / Hv: with Hv a multiple of 8 the parts of a head share an XCD.

// NT = 256: four waves, two columns per lane; NT = 512: eight waves (two per SIMD, so one wave's
// reduction and LDS latencies hide behind the other's), one column per lane, and the v channels
// and gates on threads of their own (256 .. 287, 288 ..) instead of a second role.
template <int NT>
__global__ void __launch_bounds__(NT)
gdn_split_kernel(const __bf16* __restrict__ qkv, const __bf16* __restrict__ b,
                 const __bf16* __restrict__ a, long ldp, __bf16* __restrict__ ring,
                 const __bf16* __restrict__ conv_w, const __bf16* __restrict__ A_log,
                 const __bf16* __restrict__ dt_bias, float* __restrict__ S,
                 float* __restrict__ st_k, float* __restrict__ st_v, float* __restrict__ st_g,
                 const int* __restrict__ ctl, __bf16* __restrict__ out, long ldo, int n, int Hk,
                 int Hv) {
  constexpr int CW = GDN_SPLIT_COLS;
  constexpr int NC = 512 / NT;  // state columns per lane
  __shared__ __align__(16) float sk[GDN_MAXN][GDN_D], sv[GDN_MAXN][CW];  // replayed rows
  __shared__ __align__(16) float qa[GDN_MAXN][GDN_D], ka[GDN_MAXN][GDN_D], va[GDN_MAXN][CW];
  __shared__ __align__(16) float oa[GDN_MAXN][CW];
  __shared__ float sg[GDN_MAXN][2], ga[GDN_MAXN][2], l2p[GDN_MAXN][4];

  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int j = blockIdx.x % Hv, g = blockIdx.x / Hv;
  const int r = Hv / Hk, i = j / r;
  const int C = 2 * Hk * GDN_D + Hv * GDN_D;
  const int cb = g * CW;                              // first state column of this workgroup
  const int rg = lane >> 2, lc = 4 * NC * w + NC * (lane & 3);  // rows 8 rg .., columns lc ..+NC-1
  float* Sj = S + (size_t)j * GDN_D * GDN_D;

  // Loads, all unconditional with in-bounds indices (as in the one-workgroup kernel).
  const int P = ctl[0];
  const int pend = min(max(ctl[1], 0), GDN_MAXN);
  const bool qk_thread = tid < 2 * GDN_D;             // q (part 0) or k (part 1) channel c
  const int part = (tid >> 7) & 1, c = tid & 127;
  const int ch = (part * Hk + i) * GDN_D + c;
  const int v0 = NT == 512 ? 2 * GDN_D : 0;           // v channels: threads v0 .. v0+31
  const bool v_thread = tid >= v0 && tid < v0 + CW;
  const int cv = tid & (CW - 1);
  const int chv = 2 * Hk * GDN_D + j * GDN_D + cb + cv;
  const uint2 wq = *reinterpret_cast<const uint2*>(conv_w + (size_t)ch * 4);
  const uint2 wvv = *reinterpret_cast<const uint2*>(conv_w + (size_t)chv * 4);
  __bf16 xb[GDN_MAXN], xbv[GDN_MAXN];
#pragma unroll
  for (int t = 0; t < GDN_MAXN; ++t) {
    xb[t] = qkv[(size_t)min(t, n - 1) * ldp + ch];
    xbv[t] = qkv[(size_t)min(t, n - 1) * ldp + chv];
  }
  const int gt = tid - (NT == 512 ? 2 * GDN_D + CW : 3 * 64);  // gate row of the next n threads
  const int gtc = min(max(gt, 0), n - 1);
  const __bf16 bb = b[(size_t)gtc * ldp + j], ab = a[(size_t)gtc * ldp + j];
  const __bf16 dtb = dt_bias[j], alb = A_log[j];
  const int ot = (tid >> 5) & 7, oc = tid & (CW - 1);  // output element (row ot, column cb + oc)
  __bf16 hb[3], hbv[3];
#pragma unroll
  for (int q = 0; q < 3; ++q) {
    const size_t slot = (size_t)((P - 3 + q) & (GDN_RING - 1)) * C;
    hb[q] = ring[slot + ch];
    hbv[q] = ring[slot + chv];
  }
  const F4 stk = *reinterpret_cast<const F4*>(st_k + ((size_t)ot * Hv + j) * GDN_D + 4 * oc);
  const int vr = (tid >> 3) & 7, vp = tid & 7;        // staged v: row vr, columns cb + 4 vp ..
  const F4 stv = *reinterpret_cast<const F4*>(st_v + ((size_t)vr * Hv + j) * GDN_D + cb + 4 * vp);
  const float2 stg = *reinterpret_cast<const float2*>(st_g + ((size_t)(tid & 7) * Hv + j) * 2);
  float s[8][NC];
#pragma unroll
  for (int rr = 0; rr < 8; ++rr) {
    const float* src = Sj + (size_t)(rg * 8 + rr) * GDN_D + cb + lc;
    if constexpr (NC == 2) {
      const float2 v = *reinterpret_cast<const float2*>(src);
      s[rr][0] = v.x;
      s[rr][NC - 1] = v.y;
    } else {
      s[rr][0] = *src;
    }
  }

  if (qk_thread) *reinterpret_cast<F4*>(&sk[ot][4 * oc]) = stk;
  if (tid < 64) *reinterpret_cast<F4*>(&sv[vr][4 * vp]) = stv;
  if (tid < GDN_MAXN) {
    sg[tid][0] = stg.x;
    sg[tid][1] = stg.y;
  }
  if (qk_thread) {
    const bool head_writer = g == 0 && j % r == 0;  // one writer of the shared q/k ring slots
    const float cw[4] = {lo_bf16(wq.x), hi_bf16(wq.x), lo_bf16(wq.y), hi_bf16(wq.y)};
    float xs[3 + GDN_MAXN];
#pragma unroll
    for (int q = 0; q < 3; ++q) xs[q] = P - 3 + q >= 0 ? bf16_to_f32(hb[q]) : 0.f;
#pragma unroll
    for (int t = 0; t < GDN_MAXN; ++t) xs[3 + t] = bf16_to_f32(xb[t]);
#pragma unroll
    for (int t = 0; t < GDN_MAXN; ++t) {
      if (t < n) {
        const float y = conv_silu(cw, xs, t);
        (part == 0 ? qa : ka)[t][c] = y;
        if (head_writer) ring[(size_t)((P + t) & (GDN_RING - 1)) * C + ch] = xb[t];
        const float ss = wave_sum_fast(y * y);  // q: waves 0, 1; k: waves 2, 3
        if (lane == 0) l2p[t][w] = ss;
      }
    }
  }
  if (v_thread) {  // the v channels of this workgroup's columns
    const float cw[4] = {lo_bf16(wvv.x), hi_bf16(wvv.x), lo_bf16(wvv.y), hi_bf16(wvv.y)};
    float xs[3 + GDN_MAXN];
#pragma unroll
    for (int q = 0; q < 3; ++q) xs[q] = P - 3 + q >= 0 ? bf16_to_f32(hbv[q]) : 0.f;
#pragma unroll
    for (int t = 0; t < GDN_MAXN; ++t) xs[3 + t] = bf16_to_f32(xbv[t]);
#pragma unroll
    for (int t = 0; t < GDN_MAXN; ++t) {
      if (t < n) {
        va[t][cv] = conv_silu(cw, xs, t);
        ring[(size_t)((P + t) & (GDN_RING - 1)) * C + chv] = xbv[t];
      }
    }
  }
  if (gt >= 0 && gt < n) {
    const float2 gv = gate_values(bb, ab, dtb, alb);
    ga[gt][0] = gv.x;
    ga[gt][1] = gv.y;
  }
  __syncthreads();

  // Stage this call's v columns for the next call (after the barrier: this workgroup's reads of
  // the previous call's rows at the same addresses are in LDS by now; no other workgroup reads
  // these columns). The k rows and gates, which every part of the head reads, are staged by
  // gdn_finish_kernel.
  if (qk_thread && ot < n) st_v[((size_t)ot * Hv + j) * GDN_D + cb + oc] = va[ot][oc];
  if (qk_thread) {
    const float sqrt_dk = 11.313708498984761f;  // sqrt(128) rounded to fp32
    for (int t = 0; t < n; ++t) {
      const float ss = part == 0 ? l2p[t][0] + l2p[t][1] : l2p[t][2] + l2p[t][3];
      const float inv = 1.0f / sqrtf(ss + 1e-6f);
      if (part == 0) {
        qa[t][c] = (qa[t][c] * inv) / sqrt_dk;
      } else {
        ka[t][c] = ka[t][c] * inv;
      }
    }
  }

  // ---- 1. replay, write the committed columns back ----
  for (int t = 0; t < pend; ++t) {
    float k[8], v[NC];
    lds_read8(&sk[t][rg * 8], k);
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) v[cc] = sv[t][lc + cc];
    delta_step(s, k, v, sg[t][0], sg[t][1]);
  }
  if (pend > 0) {
#pragma unroll
    for (int rr = 0; rr < 8; ++rr) {
      float* dst = Sj + (size_t)(rg * 8 + rr) * GDN_D + cb + lc;
      if constexpr (NC == 2) *reinterpret_cast<float2*>(dst) = make_float2(s[rr][0], s[rr][NC - 1]);
      else *dst = s[rr][0];
    }
  }
  __syncthreads();

  // ---- 2. new rows on the register copy ----
  for (int t = 0; t < n; ++t) {
    float k[8], q[8], v[NC], o[NC];
    lds_read8(&ka[t][rg * 8], k);
    lds_read8(&qa[t][rg * 8], q);
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) v[cc] = va[t][lc + cc];
    delta_step(s, k, v, ga[t][0], ga[t][1]);
    read_out(s, q, o);
    if (rg == 0) {
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) oa[t][lc + cc] = o[cc];
    }
  }
  __syncthreads();

  // ---- 3. this workgroup's columns of each row's output, unnormalised (o is a bf16 value, so
  // `out` holds it exactly); gdn_finish_kernel normalises the whole row ----
  if (qk_thread && ot < n) out[(size_t)ot * ldo + j * GDN_D + cb + oc] = f32_to_bf16(oa[ot][oc]);
}

// Second kernel of a split call, one 256-thread workgroup per value head j, after every part of
// gdn_split_kernel has finished (so no part still reads the previous call's staged rows):
//   * threads 0-127 recompute the normalised k channel c of this call's rows (conv + SiLU from
//     the ring history and the input rows, the sum of squares of waves 0 and 1 added in that
//     order, as gdn_split_kernel's waves 2 and 3 add it) and stage it; threads 128 .. 128+n-1
//     stage the gates;
//   * wave w normalises rows w and w + 4 of the head's outputs in place (gated_norm_row).
__global__ void __launch_bounds__(256)
gdn_finish_kernel(const __bf16* __restrict__ qkv, const __bf16* __restrict__ z,
                  const __bf16* __restrict__ b, const __bf16* __restrict__ a, long ldp,
                  const __bf16* __restrict__ ring, const __bf16* __restrict__ conv_w,
                  const __bf16* __restrict__ A_log, const __bf16* __restrict__ dt_bias,
                  const __bf16* __restrict__ norm_w, float* __restrict__ st_k,
                  float* __restrict__ st_g, const int* __restrict__ ctl, __bf16* __restrict__ out,
                  long ldo, int n, int Hk, int Hv, float eps) {
  __shared__ __align__(16) float oa[GDN_MAXN][GDN_D];
  __shared__ float l2p[GDN_MAXN][2];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int j = blockIdx.x, i = j / (Hv / Hk);
  const int C = 2 * Hk * GDN_D + Hv * GDN_D;
  const int P = ctl[0];
  const int c = tid & 127;
  const int ch = (Hk + i) * GDN_D + c;  // k channel c of qk head i
  const uint2 wk = *reinterpret_cast<const uint2*>(conv_w + (size_t)ch * 4);
  __bf16 xb[GDN_MAXN], hb[3];
#pragma unroll
  for (int t = 0; t < GDN_MAXN; ++t) xb[t] = qkv[(size_t)min(t, n - 1) * ldp + ch];
#pragma unroll
  for (int q = 0; q < 3; ++q) hb[q] = ring[(size_t)((P - 3 + q) & (GDN_RING - 1)) * C + ch];
  const int gt = tid - GDN_D;
  const int gtc = min(max(gt, 0), n - 1);
  const __bf16 bb = b[(size_t)gtc * ldp + j], ab = a[(size_t)gtc * ldp + j];
  const __bf16 dtb = dt_bias[j], alb = A_log[j];
  // outputs, z and weights of rows w and w + 4, columns 2 lane, 2 lane + 1
  __bf16 ob[2][2], zb[2][2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int t = min(w + 4 * h, n - 1);
    const __bf16* src = out + (size_t)t * ldo + j * GDN_D + 2 * lane;
    const __bf16* zp = z + (size_t)t * ldp + j * GDN_D + 2 * lane;
    ob[h][0] = src[0];
    ob[h][1] = src[1];
    zb[h][0] = zp[0];
    zb[h][1] = zp[1];
  }
  const float nw0 = bf16_to_f32(norm_w[2 * lane]), nw1 = bf16_to_f32(norm_w[2 * lane + 1]);

  float y[GDN_MAXN];
  if (tid < GDN_D) {
    const float cw[4] = {lo_bf16(wk.x), hi_bf16(wk.x), lo_bf16(wk.y), hi_bf16(wk.y)};
    float xs[3 + GDN_MAXN];
#pragma unroll
    for (int q = 0; q < 3; ++q) xs[q] = P - 3 + q >= 0 ? bf16_to_f32(hb[q]) : 0.f;
#pragma unroll
    for (int t = 0; t < GDN_MAXN; ++t) xs[3 + t] = bf16_to_f32(xb[t]);
#pragma unroll
    for (int t = 0; t < GDN_MAXN; ++t) {
      y[t] = 0.f;
      if (t < n) {
        y[t] = conv_silu(cw, xs, t);
        const float ss = wave_sum_fast(y[t] * y[t]);
        if (lane == 0) l2p[t][w] = ss;
      }
    }
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    oa[w + 4 * h][2 * lane] = bf16_to_f32(ob[h][0]);
    oa[w + 4 * h][2 * lane + 1] = bf16_to_f32(ob[h][1]);
  }
  __syncthreads();
  if (tid < GDN_D) {
#pragma unroll
    for (int t = 0; t < GDN_MAXN; ++t) {
      if (t < n) {
        const float inv = 1.0f / sqrtf((l2p[t][0] + l2p[t][1]) + 1e-6f);
        st_k[((size_t)t * Hv + j) * GDN_D + c] = y[t] * inv;
      }
    }
  }
  if (gt >= 0 && gt < n)
    *reinterpret_cast<float2*>(st_g + ((size_t)gt * Hv + j) * 2) = gate_values(bb, ab, dtb, alb);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int t = w + 4 * h;
    if (t < n)
      gated_norm_row(oa[t], lane, nw0, nw1, bf16_to_f32(zb[h][0]), bf16_to_f32(zb[h][1]), eps,
                     out + (size_t)t * ldo + j * GDN_D);
  }
}

hipError_t launch_gdn_split(const __bf16* qkv, const __bf16* z, const __bf16* b, const __bf16* a,
                            long ldp, __bf16* ring, const __bf16* conv_w, const __bf16* A_log,
                            const __bf16* dt_bias, const __bf16* norm_w, float* S, float* st_k,
                            float* st_v, float* st_g, const int* ctl, __bf16* out, long ldo,
                            int n, int Hk, int Hv, float eps, hipStream_t stream) {
  gdn_split_kernel<GDN_SPLIT_THREADS><<<dim3(Hv * GDN_SPLIT), dim3(GDN_SPLIT_THREADS), 0, stream>>>(
      qkv, b, a, ldp, ring, conv_w, A_log, dt_bias, S, st_k, st_v, st_g, ctl, out, ldo, n, Hk, Hv);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  gdn_finish_kernel<<<dim3(Hv), dim3(256), 0, stream>>>(qkv, z, b, a, ldp, ring, conv_w, A_log,
                                                        dt_bias, norm_w, st_k, st_g, ctl, out,
                                                        ldo, n, Hk, Hv, eps);
  return hipGetLastError();
}

}  // namespace qe
