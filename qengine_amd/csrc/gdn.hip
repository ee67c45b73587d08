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
// Two paths share the per-column arithmetic (gdn_common.hpp) and so give the same bits:
// gdn_step_kernel (one workgroup per head, below) for 1-4 rows, and gdn_split_kernel (each head
// over 4 workgroups) followed by gdn_finish_kernel (gdn_split.hip) for 5-8 rows.
//
// gfx950 layout: one workgroup of NT = 1024 threads (16 waves, four per SIMD) per value head.
// With NC = 2048 / NT state columns per lane, wave w owns columns 4 NC w .. +4 NC - 1 and lane l
// holds rows 8(l>>2) .. +7 of columns 4 NC w + NC (l&3) .. +NC - 1 (16 fp32 registers at NC = 2,
// loaded as eight 8-byte rows, or for 1-2 rows through a 64 KB LDS copy read and written as whole
// rows; NT = 512 gives NC = 4, 32 registers). Per delta-rule step the CU
// runs the same 3 x 16,384 fp32 operations either way; 16 waves hide more of the butterflies'
// and LDS latencies than 8 (same-box A/B on MI355X at Hk 16 / Hv 48, us per call at 1 / 2 / 3 /
// 4 rows: 8.60 / 10.16 / 11.57 / 12.35 with 8 waves (the split path at 4) against 8.44 / 9.50 /
// 10.70 / 12.03; at 6 and 8 rows the split path stays faster, 14.65 / 16.52 against 15.17 /
// 18.05). The dot products over the 128 state rows are a per-lane 8-term
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
#include "gdn_common.hpp"
#include "qe_gdn.h"

namespace qe {

template <int NT, bool SL>
__global__ void __launch_bounds__(NT)
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
  // SL: the state is staged through LDS. It is read and written back as whole 512-byte rows
  // (coalesced, four 16-byte pieces per thread) and moved to and from the register layout in
  // LDS. Float (r, c) sits at r*128 + 8((c/8) ^ (r/8 & 15)) + c%8, so the 16 rows of one
  // register-layout access (stride 8 rows) hit distinct 32-byte groups. Direct loads in the
  // register layout read 32 bytes of each 128-byte line per wave.
  __shared__ __align__(16) float sS[SL ? GDN_D * GDN_D : 4];
  auto sidx = [](int r, int c) { return r * GDN_D + 8 * ((c >> 3) ^ ((r >> 3) & 15)) + (c & 7); };

  static_assert(NT == 512 || NT == 1024, "8 or 16 waves");
  static_assert(!SL || NT == 1024, "the staged state: four 16-byte pieces per thread");
  constexpr int NC = 2048 / NT;  // state columns per lane: 4 (8 waves) or 2 (16 waves)
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int rg = lane >> 2, col0 = 4 * NC * w + NC * (lane & 3);
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
  // staged rows: thread = (row, 16-byte piece of k or v); waves 8-15 of the 16-wave kernel
  // re-read row 7 and store nothing
  const int srow = min(tid >> 6, GDN_MAXN - 1), su = tid & 63;
  const F4 stv = *reinterpret_cast<const F4*>(
      su < 32 ? st_k + ((size_t)srow * Hv + j) * GDN_D + 4 * su
              : st_v + ((size_t)srow * Hv + j) * GDN_D + 4 * (su - 32));
  const float2 stg = *reinterpret_cast<const float2*>(st_g + ((size_t)(tid & 7) * Hv + j) * 2);
  float s[8][NC];
  F4 gS[SL ? 4 : 1];  // SL: pieces f = tid + NT k, row f / 32, columns 4 (f % 32) .. +3
  if constexpr (SL) {
#pragma unroll
    for (int k = 0; k < 4; ++k) gS[k] = reinterpret_cast<const F4*>(Sj)[tid + NT * k];
  } else {
    load_state_rows(Sj, rg, col0, s);
  }

  if (tid < GDN_MAXN * 64)
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
  if constexpr (SL) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int f = tid + NT * k;
      *reinterpret_cast<F4*>(&sS[sidx(f >> 5, 4 * (f & 31))]) = gS[k];
    }
  }
  __syncthreads();
  if constexpr (SL) {  // each lane reads (and later writes) only its own elements
#pragma unroll
    for (int rr = 0; rr < 8; ++rr) {
      const float2 v = *reinterpret_cast<const float2*>(&sS[sidx(rg * 8 + rr, col0)]);
      s[rr][0] = v.x;
      s[rr][NC - 1] = v.y;
    }
  }

  // Stage this call's v and gates for the next call's replay. Only after the barrier: the staged
  // rows of the previous call (same addresses) have all been read into LDS by then.
  for (int t = tid >> 7; t < n; t += NT / GDN_D)
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
    float k[8], v[NC];
    lds_read8(&sk[t][rg * 8], k);
    vec_read_n(&sv[t][col0], v);
    delta_step(s, k, v, sg[t][0], sg[t][1]);
  }
  if constexpr (SL) {
    if (pend > 0) {
#pragma unroll
      for (int rr = 0; rr < 8; ++rr)
        *reinterpret_cast<float2*>(&sS[sidx(rg * 8 + rr, col0)]) = make_float2(s[rr][0], s[rr][NC - 1]);
    }
    __syncthreads();
    if (pend > 0) {  // the copy runs beside the new rows, which do not touch sS
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int f = tid + NT * k;
        reinterpret_cast<F4*>(Sj)[f] = *reinterpret_cast<const F4*>(&sS[sidx(f >> 5, 4 * (f & 31))]);
      }
    }
  } else {
    if (pend > 0) store_state_rows(Sj, rg, col0, s);
    __syncthreads();
  }

  // ---- 2. new rows on the register copy ----
  for (int t = 0; t < n; ++t) {
    float k[8], q[8], v[NC];
    lds_read8(&ka[t][rg * 8], k);
    lds_read8(&qa[t][rg * 8], q);
    vec_read_n(&va[t][col0], v);
    delta_step(s, k, v, ga[t][0], ga[t][1]);
    float o[NC];
    read_out(s, q, o);
    if (rg == 0) vec_write_n(&oa[t][col0], o);
  }
  __syncthreads();

  // ---- gated RMSNorm: wave t normalises row t ----
  if (w < n) gated_norm_row(oa[w], lane, nw0, nw1, z0, z1, eps, out + (size_t)w * ldo + j * GDN_D);
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
  // five rows the split's second launch costs more than the spread saves: same-box A/B on MI355X
  // at Hk 16 / Hv 48, 4 rows 12.03 us one workgroup against 12.35 split; 6 rows 15.17 against
  // 14.65). Both paths give the same bits.
  if (n >= GDN_SPLIT_MIN_ROWS)
    return launch_gdn_split(static_cast<const __bf16*>(qkv), static_cast<const __bf16*>(z),
                            static_cast<const __bf16*>(b), static_cast<const __bf16*>(a), ldp,
                            static_cast<__bf16*>(ring), static_cast<const __bf16*>(conv_w),
                            static_cast<const __bf16*>(A_log), static_cast<const __bf16*>(dt_bias),
                            static_cast<const __bf16*>(norm_w), S, st_k, st_v, st_g, ctl,
                            static_cast<__bf16*>(out), ldo, n, Hk, Hv, eps, stream);
  // 1-2 rows stage the state through LDS (same bits; same-box A/B, us per call at 1 / 2 / 3 / 4
  // rows: 8.41 / 9.44 / 10.65 / 12.01 direct, 7.73 / 9.21 / 10.66 / 12.10 staged)
  auto kern = n <= GDN_STAGE_MAX_ROWS ? gdn_step_kernel<GDN_THREADS, true>
                                      : gdn_step_kernel<GDN_THREADS, false>;
  kern<<<dim3(Hv), dim3(GDN_THREADS), 0, stream>>>(
      static_cast<const __bf16*>(qkv), static_cast<const __bf16*>(z), static_cast<const __bf16*>(b),
      static_cast<const __bf16*>(a), ldp, static_cast<__bf16*>(ring),
      static_cast<const __bf16*>(conv_w), static_cast<const __bf16*>(A_log),
      static_cast<const __bf16*>(dt_bias), static_cast<const __bf16*>(norm_w), S, st_k, st_v, st_g,
      ctl, static_cast<__bf16*>(out), ldo, n, Hk, Hv, eps);
  return hipGetLastError();
}
