// Gated DeltaNet decode / verify step on gfx950: n = 1..8 new rows per layer call with lazy
// rollback (reference csrc/gdn.cu:1-25,65-311; math of python/qengine/reference.py:211-242).
//
// Per value head j (qk head i = j / (Hv/Hk)), with the committed fp32 state S_j [128][128] being
// the state after position pos - pending:
//   1. replay: the `pending` rows staged by the previous call (normalised k, v, decay, beta) are
//      applied to S_j, which is written back once;
//   2. new rows t < n at positions pos + t: causal conv (4 taps) + SiLU over the 384 channels of
//      this head, gates, l2norm of q and k, the delta-rule update on a register copy of S_j, and
//      the gated RMSNorm output; their (k, v, decay, beta) are staged for the next call, S_j is
//      not advanced by them.
// The same inline update runs for replayed and new rows, so the committed state after any
// pattern of calls with kept prefixes equals plain one-row decoding bit for bit.
//
// Two paths share the per-column arithmetic and so give the same bits: gdn_step_kernel (one
// workgroup per head, below) for 1-4 rows, and gdn_split_kernel (each head over 4 workgroups)
// followed by gdn_finish_kernel (further down) for 5-8 rows.
//
// gfx950 layout: one 512-thread workgroup (8 waves) per value head. Wave w owns state columns
// 16w .. 16w+15; lane l holds rows 8(l>>2) .. +7 of columns 16w + 4(l&3) .. +3 (32 fp32 registers,
// loaded as eight 16-byte rows). The dot products over the 128 state rows are a per-lane 8-term
// FMA chain followed by a butterfly over the 16 lanes that share a column quad (DPP xor 8 / 4,
// permlane16 / 32 swaps), so the recurrence needs no LDS and no barrier. Each wave therefore holds
// the whole column: kv, delta and o never leave the wave. Three barriers per call: after the
// per-call inputs are in LDS (staged rows, conv outputs, gates, l2 partial sums), after the
// replay (by then q and k are normalised in LDS, once per channel), and before the gated
// RMSNorm, which needs the 128 outputs of a row (wave t normalises row t).
//
// Conv history is a ring of 16 slots [16][C] keyed by absolute position (slot = pos & 15). A call
// reads positions < pos from the ring (negative positions read as 0) and earlier rows of this
// call from its own inputs, and writes the slots of positions pos .. pos+n-1. With n <= 8 the
// read slots (pos-3 .. pos-1) and the written ones never alias, so workgroups sharing a qk head
// need no synchronisation; only the workgroup with j % (Hv/Hk) == 0 writes the q/k channels.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "qe_device.hpp"
#include "qe_gdn.h"

namespace qe {

constexpr int GDN_D = 128;      // dk = dv
constexpr int GDN_RING = 16;
constexpr int GDN_MAXN = 8;
constexpr int GDN_THREADS = 512;
constexpr int GDN_SPLIT = 4;                        // workgroups per head in the split kernel
constexpr int GDN_SPLIT_COLS = GDN_D / GDN_SPLIT;
constexpr int GDN_SPLIT_THREADS = 512;
constexpr int GDN_SPLIT_MIN_ROWS = 5;               // fewer rows: the one-workgroup kernel

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

__global__ void __launch_bounds__(GDN_THREADS)
gdn_step_kernel(const __bf16* __restrict__ qkv, const __bf16* __restrict__ z,
                const __bf16* __restrict__ b, const __bf16* __restrict__ a, long ldp,
                __bf16* __restrict__ ring, const __bf16* __restrict__ conv_w,
                const __bf16* __restrict__ A_log, const __bf16* __restrict__ dt_bias,
                const __bf16* __restrict__ norm_w, float* __restrict__ S,
                float* __restrict__ st_k, float* __restrict__ st_v, float* __restrict__ st_g,
                const int* __restrict__ ctl, __bf16* __restrict__ out, long ldo, int n, int Hk,
                int Hv, float eps) {
  __shared__ __align__(16) float sk[GDN_MAXN][GDN_D], sv[GDN_MAXN][GDN_D];  // replayed rows
  __shared__ __align__(16) float qa[GDN_MAXN][GDN_D], ka[GDN_MAXN][GDN_D], va[GDN_MAXN][GDN_D];
  __shared__ __align__(16) float oa[GDN_MAXN][GDN_D];
  __shared__ float sg[GDN_MAXN][2], ga[GDN_MAXN][2], l2p[GDN_MAXN][4];

  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int rg = lane >> 2, col0 = 16 * w + 4 * (lane & 3);
  const int j = blockIdx.x, r = Hv / Hk, i = j / r;
  const int C = 2 * Hk * GDN_D + Hv * GDN_D;
  float* Sj = S + (size_t)j * GDN_D * GDN_D;

  // Every global load below is unconditional with an in-bounds index (rows t >= n re-read row
  // n - 1, unused staged rows are read anyway, history slots come from position & 15), so they
  // issue back to back and the waits gather at their first uses; loads behind branches would
  // each wait on their own. Order: the call's position, this call's inputs, the history and the
  // staged rows, then the state block, which is needed last.
  const int P = ctl[0];
  const int pend = min(max(ctl[1], 0), GDN_MAXN);
  const int part = tid >> 7, c = tid & 127;  // conv role (tid < 384): 0 = q, 1 = k, 2 = v
  const int ch = part == 0 ? i * GDN_D + c : part == 1 ? (Hk + i) * GDN_D + c
                                                        : 2 * Hk * GDN_D + j * GDN_D + c;
  const int chl = tid < 3 * GDN_D ? ch : c;
  const uint2 wv = *reinterpret_cast<const uint2*>(conv_w + (size_t)chl * 4);
  __bf16 xb[GDN_MAXN];
#pragma unroll
  for (int t = 0; t < GDN_MAXN; ++t) xb[t] = qkv[(size_t)min(t, n - 1) * ldp + chl];
  const int gt = tid - 3 * GDN_D;  // gate row of threads 384 .. 384+n-1
  const int gtc = min(max(gt, 0), n - 1);
  const __bf16 bb = b[(size_t)gtc * ldp + j], ab = a[(size_t)gtc * ldp + j];
  const __bf16 dtb = dt_bias[j], alb = A_log[j];
  const __bf16* zp = z + (size_t)min(w, n - 1) * ldp + j * GDN_D + 2 * lane;
  const __bf16 zb0 = zp[0], zb1 = zp[1], nb0 = norm_w[2 * lane], nb1 = norm_w[2 * lane + 1];
  __bf16 hb[3];  // x at positions P-3 .. P-1
#pragma unroll
  for (int q = 0; q < 3; ++q) hb[q] = ring[(size_t)((P - 3 + q) & (GDN_RING - 1)) * C + chl];
  const int srow = tid >> 6, su = tid & 63;  // staged rows: thread = (row, 16-byte piece of k or v)
  const F4 stv = *reinterpret_cast<const F4*>(
      su < 32 ? st_k + ((size_t)srow * Hv + j) * GDN_D + 4 * su
              : st_v + ((size_t)srow * Hv + j) * GDN_D + 4 * (su - 32));
  const float2 stg = *reinterpret_cast<const float2*>(st_g + ((size_t)(tid & 7) * Hv + j) * 2);
  float s[8][4];
#pragma unroll
  for (int rr = 0; rr < 8; ++rr) {
    const F4 v = *reinterpret_cast<const F4*>(Sj + (size_t)(rg * 8 + rr) * GDN_D + col0);
    s[rr][0] = v.x; s[rr][1] = v.y; s[rr][2] = v.z; s[rr][3] = v.w;
  }

  *reinterpret_cast<F4*>(su < 32 ? &sk[srow][4 * su] : &sv[srow][4 * (su - 32)]) = stv;
  if (tid < GDN_MAXN) {
    sg[tid][0] = stg.x;
    sg[tid][1] = stg.y;
  }
  const float z0 = bf16_to_f32(zb0), z1 = bf16_to_f32(zb1);
  const float nw0 = bf16_to_f32(nb0), nw1 = bf16_to_f32(nb1);
  if (tid < 3 * GDN_D) {
    const float cw[4] = {lo_bf16(wv.x), hi_bf16(wv.x), lo_bf16(wv.y), hi_bf16(wv.y)};
    // x at positions P-3 .. P+n-1: history from the ring (zero before the sequence), then this
    // call's rows
    float xs[3 + GDN_MAXN];
#pragma unroll
    for (int q = 0; q < 3; ++q) xs[q] = P - 3 + q >= 0 ? bf16_to_f32(hb[q]) : 0.f;
#pragma unroll
    for (int t = 0; t < GDN_MAXN; ++t) xs[3 + t] = bf16_to_f32(xb[t]);
    const bool writes_ring = part == 2 || j % r == 0;  // q/k channels are shared by r heads
#pragma unroll
    for (int t = 0; t < GDN_MAXN; ++t) {
      if (t < n) {
        const float y = conv_silu(cw, xs, t);
        if (part == 0) qa[t][c] = y;
        else if (part == 1) ka[t][c] = y;
        else va[t][c] = y;
        if (writes_ring) ring[(size_t)((P + t) & (GDN_RING - 1)) * C + ch] = xb[t];
        if (part < 2) {  // sum of squares of q (waves 0, 1) and k (waves 2, 3)
          const float ss = wave_sum_fast(y * y);
          if (lane == 0) l2p[t][w] = ss;
        }
      }
    }
  }
  if (gt >= 0 && gt < n) {
    const float2 gv = gate_values(bb, ab, dtb, alb);
    ga[gt][0] = gv.x;
    ga[gt][1] = gv.y;
  }
  __syncthreads();

  // Stage this call's v and gates for the next call's replay. Only after the barrier: the staged
  // rows of the previous call (same addresses) have all been read into LDS by then.
  for (int t = tid >> 7; t < n; t += GDN_THREADS / GDN_D)
    st_v[((size_t)t * Hv + j) * GDN_D + c] = va[t][c];
  if (tid < n)
    *reinterpret_cast<float2*>(st_g + ((size_t)tid * Hv + j) * 2) = make_float2(ga[tid][0], ga[tid][1]);

  // Normalise this call's q and k once per channel (threads 0-255 own one q or k channel each)
  // and stage k for the next call. In place: the rows are read again only after the barrier
  // that follows the replay.
  if (tid < 2 * GDN_D) {
    const float sqrt_dk = 11.313708498984761f;  // sqrt(128) rounded to fp32
    for (int t = 0; t < n; ++t) {
      const float ss = tid < GDN_D ? l2p[t][0] + l2p[t][1] : l2p[t][2] + l2p[t][3];
      const float inv = 1.0f / sqrtf(ss + 1e-6f);
      if (tid < GDN_D) {
        qa[t][c] = (qa[t][c] * inv) / sqrt_dk;
      } else {
        const float kn = ka[t][c] * inv;
        ka[t][c] = kn;
        st_k[((size_t)t * Hv + j) * GDN_D + c] = kn;
      }
    }
  }

  // ---- 1. replay the rows kept by the previous call, write the committed state back ----
  for (int t = 0; t < pend; ++t) {
    float k[8], v[4];
    lds_read8(&sk[t][rg * 8], k);
    lds_read4(&sv[t][col0], v);
    delta_step(s, k, v, sg[t][0], sg[t][1]);
  }
  if (pend > 0) {
#pragma unroll
    for (int rr = 0; rr < 8; ++rr)
      *reinterpret_cast<F4*>(Sj + (size_t)(rg * 8 + rr) * GDN_D + col0) =
          F4{s[rr][0], s[rr][1], s[rr][2], s[rr][3]};
  }
  __syncthreads();

  // ---- 2. new rows on the register copy ----
  for (int t = 0; t < n; ++t) {
    float k[8], q[8], v[4];
    lds_read8(&ka[t][rg * 8], k);
    lds_read8(&qa[t][rg * 8], q);
    lds_read4(&va[t][col0], v);
    delta_step(s, k, v, ga[t][0], ga[t][1]);
    float o[4];
    read_out(s, q, o);
    if (rg == 0) *reinterpret_cast<F4*>(&oa[t][col0]) = F4{o[0], o[1], o[2], o[3]};
  }
  __syncthreads();

  // ---- gated RMSNorm: wave t normalises row t ----
  if (w < n) gated_norm_row(oa[w], lane, nw0, nw1, z0, z1, eps, out + (size_t)w * ldo + j * GDN_D);
}

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

}  // namespace qe

using namespace qe;

extern "C" hipError_t qe_gdn_step_n(const void* qkv, const void* z, const void* b, const void* a,
                                    long ldp, void* ring, const void* conv_w, const void* A_log,
                                    const void* dt_bias, const void* norm_w, float* S, float* st_k,
                                    float* st_v, float* st_g, const int* ctl, void* out, long ldo,
                                    int n, int Hk, int Hv, float eps, hipStream_t stream) {
  auto al = [](const void* p, uintptr_t m) { return (reinterpret_cast<uintptr_t>(p) & (m - 1)) == 0; };
  if (!qkv || !z || !b || !a || !ring || !conv_w || !A_log || !dt_bias || !norm_w || !S || !st_k ||
      !st_v || !st_g || !ctl || !out)
    return hipErrorInvalidValue;
  if (n < 1 || n > GDN_MAXN || Hk < 1 || Hv < 1 || Hv % Hk != 0 || Hv > 65535)
    return hipErrorInvalidValue;
  const long C = 2L * Hk * GDN_D + (long)Hv * GDN_D;
  if (C >= (1L << 26) || ldp < C || ldo < (long)Hv * GDN_D) return hipErrorInvalidValue;
  if (!al(S, 16) || !al(st_k, 16) || !al(st_v, 16) || !al(st_g, 8) || !al(conv_w, 8))
    return hipErrorInvalidValue;
  // 5-8 rows: the split kernel and its finish kernel; 1-4 rows: one workgroup per head (below
  // five rows the split's second launch costs more than the spread saves: same-box A/B on
  // MI355X at Hk 16 / Hv 48, 2 rows 11.2 vs 9.5 us, 4 rows 12.9 vs 12.6, 6 rows 15.4 vs 15.7,
  // 8 rows 17.4 vs 18.8). Both paths give the same bits.
  if (n >= GDN_SPLIT_MIN_ROWS) {
    gdn_split_kernel<GDN_SPLIT_THREADS><<<dim3(Hv * GDN_SPLIT), dim3(GDN_SPLIT_THREADS), 0, stream>>>(
        static_cast<const __bf16*>(qkv), static_cast<const __bf16*>(b),
        static_cast<const __bf16*>(a), ldp, static_cast<__bf16*>(ring),
        static_cast<const __bf16*>(conv_w), static_cast<const __bf16*>(A_log),
        static_cast<const __bf16*>(dt_bias), S, st_k, st_v, st_g, ctl, static_cast<__bf16*>(out),
        ldo, n, Hk, Hv);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    gdn_finish_kernel<<<dim3(Hv), dim3(256), 0, stream>>>(
        static_cast<const __bf16*>(qkv), static_cast<const __bf16*>(z),
        static_cast<const __bf16*>(b), static_cast<const __bf16*>(a), ldp,
        static_cast<const __bf16*>(ring), static_cast<const __bf16*>(conv_w),
        static_cast<const __bf16*>(A_log), static_cast<const __bf16*>(dt_bias),
        static_cast<const __bf16*>(norm_w), st_k, st_g, ctl, static_cast<__bf16*>(out), ldo, n,
        Hk, Hv, eps);
    return hipGetLastError();
  }
  gdn_step_kernel<<<dim3(Hv), dim3(GDN_THREADS), 0, stream>>>(
      static_cast<const __bf16*>(qkv), static_cast<const __bf16*>(z), static_cast<const __bf16*>(b),
      static_cast<const __bf16*>(a), ldp, static_cast<__bf16*>(ring),
      static_cast<const __bf16*>(conv_w), static_cast<const __bf16*>(A_log),
      static_cast<const __bf16*>(dt_bias), static_cast<const __bf16*>(norm_w), S, st_k, st_v, st_g,
      ctl, static_cast<__bf16*>(out), ldo, n, Hk, Hv, eps);
  return hipGetLastError();
}
