// Second launch of the split-KV decode (reference csrc/attn.cu:125-149): the log-sum-exp merge
// of a row's slice partials and the fused sigmoid output gate, out = bf16(bf16(O / L) *
// bf16(sigmoid(gate))).
//
// This file is compiled with LLVM's max-ILP machine scheduler (the partials kernels measured
// slower under it, so they stay in attn_decode.hip): 3.13 -> 3.00 us per combine at 1 row,
// 3.70 -> 3.64 at 5 rows, same bits (same-box A/B, graphs of 16 combines).
#include "attn_split.hpp"
#include "qe_attn.h"

namespace qe {

// Log-sum-exp merge of the slices holding row t's positions + fused sigmoid output gate.
// One wave per (head h, row t, 16-dim chunk z); lane = (slice group g = lane / 4, 4 dims). The
// slices of a batch of 64 fall into the 16 groups (s = s0 + 16b + g, b < 4); each group sums its
// 4 slices in order b = 0..3 and the 16 group sums meet in a fixed tree across lanes (g ^ 8,
// g ^ 4, g ^ 2, g ^ 1). So the result depends only on row t's partials and slice count, never on
// the other rows of the call.
// All loads of a batch are issued before any is used, so up to 64 slices cost one memory round
// trip. A lone wave pays ~4 cycles for every VALU instruction, so the work after the loads sets
// the kernel's length. Per-wave stamps on the box put it at ~1 us of ~3.9 us for an earlier form
// with 64-dim chunks, 16 slices per lane and a branch per slice, and at ~0.6 us with 8 slices per
// lane and no branches. Hence 4 slices per lane, no branches (every slot is loaded, its index
// clamped to NS - 1, and the slots that do not count are selected away: m = -inf, weight 0,
// data 0; adding those +0 leaves L and O unchanged, as neither is ever -0), a tree for the batch
// maximum, and the gate's sigmoid computed while the partials are in flight. Layer-call, 1 row at
// 16k: 17.9 us with the earlier form, 16.8 with this one (32- and 64-dim chunks of the same
// design: 17.0 and 17.6; 16-dim was also the fastest or within 0.3% at 2-8 rows).
constexpr int COMBINE_DIMS = 16;

// Sum / max over the 16 lane groups of 4 lanes: lane ^ 32, ^ 16 (the gfx950 lane swaps), ^ 8
// and ^ 4 (DPP within each 16-lane row) pair group g with g ^ 8, g ^ 4, g ^ 2, g ^ 1. Every lane
// ends with the same bits (a + b == b + a).
__device__ __forceinline__ float group16_sum(float v) {
  v = xor16_pair(xor32_pair(v, true), true);
  v = v + dpp<0x128>(v);                 // row_ror:8 = lane ^ 8 within 16
  return v + dpp<0x1B>(dpp<0x141>(v));   // row_half_mirror, then quad_perm [3,2,1,0]: lane ^ 4
}
__device__ __forceinline__ float group16_max(float v) {
  v = fmaxf(v, dpp<0x128>(v));
  v = fmaxf(v, dpp<0x1B>(dpp<0x141>(v)));
  return xor32_pair(xor16_pair(v, false), false);
}

__global__ void __launch_bounds__(WAVE)
attn_combine_kernel(const float* __restrict__ part_o, const float* __restrict__ part_ml,
                    const int* __restrict__ pos_ptr, const __bf16* __restrict__ qg, long ldp,
                    __bf16* __restrict__ out, long ldo, int Hq, int max_len, int NS,
                    NsDiv nd, float v_scale) {
  constexpr int G = 16, B = 4;  // slice groups, slices per group per batch
  const int h = blockIdx.x, t = blockIdx.y, z = blockIdx.z;
  const int lane = threadIdx.x, cd = lane & 3, g = lane >> 2;
  const size_t base = ((size_t)t * Hq + h) * NS;
  const float* ml = part_ml + base * 2;
  const int dim = z * COMBINE_DIMS + 4 * cd;
  const __bf16* gp = qg + (size_t)t * ldp + (size_t)h * 2 * HD + HD + dim;

  float gate[4];  // qg rows carry no alignment guarantee beyond 2 bytes
#pragma unroll
  for (int i = 0; i < 4; ++i) gate[i] = bf16_to_f32(gp[i]);
  __builtin_amdgcn_sched_barrier(0);  // the gate's load is issued first
  // The first batch of slices is loaded before pos arrives (every slot below NS exists in the
  // caller's buffers); slots past row t's slice count S are discarded by selection, so stale
  // contents never reach the sums.
  f32x4_t po[B];
  float2 mls[B];
  auto load_batch = [&](int s0) {
#pragma unroll
    for (int b = 0; b < B; ++b) {
      const int s = min(s0 + G * b + g, NS - 1);
      po[b] = *reinterpret_cast<const f32x4_t*>(part_o + (base + s) * HD + dim);
      mls[b] = *reinterpret_cast<const float2*>(ml + 2 * s);
    }
  };
  load_batch(0);
  __builtin_amdgcn_sched_barrier(0);  // every load is issued before the wait for the gate
  float sgate[4];  // bf16(sigmoid(gate)), computed while the partials are in flight
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    sgate[i] = round_bf16(sigmoid_f32(gate[i]));
    asm volatile("" : "+v"(sgate[i]));  // here, not sunk to the stores
  }
  const int L_t = min(pos_ptr[0] + t + 1, max_len);
  const int CH = split_size(L_t, nd);  // slice s holds positions iff s * CH < L_t (s < NS)

  f32x4_t O = {0.f, 0.f, 0.f, 0.f};
  float L = 0.f, M = -INFINITY;
  for (int s0 = 0; s0 < NS && s0 * CH < L_t; s0 += G * B) {
    if (s0 > 0) load_batch(s0);
    float mv[B];  // the slot's max, -inf unless the slot counts
#pragma unroll
    for (int b = 0; b < B; ++b) {
      const int sl = s0 + G * b + g;
      mv[b] = sl < NS && sl * CH < L_t ? mls[b].x : -INFINITY;
    }
    // running max over all slices seen so far (every lane group, so M is wave-uniform)
    const float bm =
        group16_max(fmaxf(M, fmaxf(fmaxf(mv[0], mv[2]), fmaxf(mv[1], mv[3]))));
    if (bm != M) {  // rescale what was accumulated under the old max (exact no-op otherwise)
      const float r = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(M - bm);
      O *= r;
      L *= r;
      M = bm;
    }
#pragma unroll
    for (int b = 0; b < B; ++b) {
      const bool use = mv[b] != -INFINITY;
      const float f = use ? __builtin_amdgcn_exp2f(mv[b] - M) : 0.f;
      const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
      L += (use ? mls[b].y : 0.f) * f;
      O += (use ? po[b] : zero) * f;
    }
  }
  L = group16_sum(L);
#pragma unroll
  for (int i = 0; i < 4; ++i) O[i] = group16_sum(O[i]);
  if (g == 0) {
    __bf16* op = out + (size_t)t * ldo + (size_t)h * HD + dim;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // attention output is a bf16 tensor (v_scale: the fp8 cache's V scale, else exactly 1)
      const float o = round_bf16((O[i] / L) * v_scale);
      op[i] = f32_to_bf16(o * sgate[i]);
    }
  }
}

hipError_t launch_combine(const float* part_o, const float* part_ml, const int* pos,
                          const void* qg, long ldp, void* out, long ldo, int n, int Hq,
                          int max_len, int NS, hipStream_t stream, float v_scale) {
  attn_combine_kernel<<<dim3(Hq, n, HD / COMBINE_DIMS), dim3(WAVE), 0, stream>>>(
      part_o, part_ml, pos, static_cast<const __bf16*>(qg), ldp, static_cast<__bf16*>(out), ldo,
      Hq, max_len, NS, ns_div(NS), v_scale);
  return hipGetLastError();
}

}  // namespace qe
