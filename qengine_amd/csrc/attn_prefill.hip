// Chunked-prefill gated attention on gfx950 (MI355X): T query rows at positions pos..pos+T-1,
// row t attends cache positions [0, min(pos+t+1, max_len)), out = bf16(bf16(softmax . V) *
// bf16(sigmoid(gate))). Same per-row semantics as decode (reference csrc/attn.cu:1-2,78,146-148;
// python/qengine/reference.py:263-272). The reference has no prefill kernel: it feeds prompts
// through its n <= 8 row decode path (engine.py:542-573).
//
// Design (compute-bound, MFMA):
//  * Workgroup = 128 consecutive query rows of one q head: 4 waves x 32 rows, each wave's rows are
//    two 16-column MFMA tiles. Workgroups run heaviest (longest attended prefix) first.
//  * K/V tiles of 32 positions are streamed into LDS by LDS DMA (each wave fetches 8 rows), double
//    buffered, and shared by the 4 waves. K is XOR-swizzled for conflict-free operand reads.
//  * Per tile and wave: S^T = K Q^T (32 MFMA 16x16x32), online softmax per column in the log2
//    domain, O^T += V^T P^T with P as bf16 hi + lo terms (64 MFMA): fp32-class accuracy for
//    short rows too. Q lives in registers as the B operand, O^T in accumulation registers.
//  * Epilogue: O / l rounded to bf16, times bf16(sigmoid(gate)), 16-byte stores.
#include "qe_device.hpp"
#include "qe_attn.h"

namespace qe {
namespace prefill {

constexpr int WAVES = 4;
constexpr int ROWS_PER_WAVE = 32;               // two 16-column MFMA tiles
constexpr int NT = ROWS_PER_WAVE / 16;
constexpr int BQ = WAVES * ROWS_PER_WAVE;       // 128 query rows per workgroup
constexpr int BN = 32;                          // cache positions per step
constexpr int ROW_CHUNKS = HD * 2 / 16;         // 32 chunks of 16 B per 512-byte cache row
constexpr int TILE_U4 = BN * ROW_CHUNKS;        // 16-byte slots per K (or V) tile: 1024
constexpr int STAGE_U4 = 2 * TILE_U4;           // K tile then V tile
constexpr int STAGES = 2;

__device__ __forceinline__ int k_slot(int r, int q) { return r * ROW_CHUNKS + (q ^ (r & 15)); }

// Issue this wave's 8 LDS-DMA loads of tile [p0, p0 + 32): rows 8w .. 8w+7 of K (swizzled) and V.
__device__ __forceinline__ void issue_tile(u32x4_t* stage, __amdgpu_buffer_rsrc_t krs,
                                           __amdgpu_buffer_rsrc_t vrs, int p0, int w, int lane) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = 8 * w + 2 * j + (lane >> 5);
    const int q = (lane & 31) ^ (r & 15);
    buffer_load16_to_lds(krs, (uint32_t)(p0 + r) * (HD * 2) + q * 16,
                         stage + (8 * w + 2 * j) * ROW_CHUNKS);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = 8 * w + 2 * j + (lane >> 5);
    buffer_load16_to_lds(vrs, (uint32_t)(p0 + r) * (HD * 2) + (lane & 31) * 16,
                         stage + TILE_U4 + (8 * w + 2 * j) * ROW_CHUNKS);
  }
}

__global__ void __launch_bounds__(WAVES * WAVE)
attn_prefill_kernel(const __bf16* __restrict__ q, const __bf16* __restrict__ kc,
                    const __bf16* __restrict__ vc, const int* __restrict__ pos_ptr,
                    const __bf16* __restrict__ qg, long ldp, __bf16* __restrict__ out, long ldo,
                    int T, int Hq, int Hkv, int max_len, float scale_log2) {
  const int nblk = gridDim.x;
  const int blk = nblk - 1 - blockIdx.x;  // heaviest (latest) row block first
  const int h = blockIdx.y;
  const int g = h / (Hq / Hkv);
  const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
  const int c = lane & 15, g4 = lane >> 4;
  const int pos0 = pos_ptr[0];

  __shared__ __attribute__((aligned(16))) u32x4_t lds[STAGES * STAGE_U4];  // 64 KB

  // Q^T as the MFMA B operand: column ct*16 + c is chunk row r = blk*128 + 32w + 16ct + c.
  bf16x8_t qb[NT][8];
  int Lcol[NT];
#pragma unroll
  for (int ct = 0; ct < NT; ++ct) {
    const int r = blk * BQ + w * ROWS_PER_WAVE + ct * 16 + c;
    if (r < T) {
      Lcol[ct] = min(pos0 + r + 1, max_len);
      const u32x4_t* src = reinterpret_cast<const u32x4_t*>(q + (size_t)r * Hq * HD + (size_t)h * HD);
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) qb[ct][ks] = as_bf16x8(src[4 * ks + g4]);
    } else {
      Lcol[ct] = 0;
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) qb[ct][ks] = as_bf16x8(u32x4_t{0u, 0u, 0u, 0u});
    }
  }
  // Longest attended prefix of this workgroup's rows, and of this wave's rows.
  const int last_row = min(blk * BQ + BQ, T) - 1;
  const int Lwg = min(pos0 + last_row + 1, max_len);
  const int Lwave = min(pos0 + min(blk * BQ + w * ROWS_PER_WAVE + ROWS_PER_WAVE, T), max_len);
  const int ntiles = Lwg > 0 ? (Lwg + BN - 1) / BN : 0;

  const size_t head_off = (size_t)g * max_len * HD;
  const uint32_t bytes = (uint32_t)max(Lwg, 0) * (uint32_t)(HD * 2);  // past Lwg reads 0
  const __amdgpu_buffer_rsrc_t krs = make_rsrc(kc + head_off, bytes);
  const __amdgpu_buffer_rsrc_t vrs = make_rsrc(vc + head_off, bytes);

  float m[NT], l[NT];
  f32x4_t acc[NT][2][8];
#pragma unroll
  for (int ct = 0; ct < NT; ++ct) {
    m[ct] = -INFINITY;
    l[ct] = 0.f;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[ct][hh][i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  issue_tile(lds, krs, vrs, 0, w, lane);
  issue_tile(lds + STAGE_U4, krs, vrs, BN, w, lane);
  for (int j = 0; j < ntiles; ++j) {
    const u32x4_t* kt = lds + (j & 1) * STAGE_U4;
    const u32x4_t* vt = kt + TILE_U4;
    const int p0 = j * BN;
    vmcnt_wait<8>();   // this wave's loads of tile j are done (tile j+1's 8 may be in flight)
    __syncthreads();   // ... and every other wave's
    if (p0 < Lwave) {  // tiles entirely past this wave's rows contribute nothing
      // S^T = K Q^T: lane holds positions p0 + 16T + 4g4 + i of column c.
      f32x4_t sacc[NT][2];
#pragma unroll
      for (int T2 = 0; T2 < 2; ++T2) {
#pragma unroll
        for (int ct = 0; ct < NT; ++ct) sacc[ct][T2] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
          const bf16x8_t kop = as_bf16x8(kt[k_slot(16 * T2 + c, 4 * ks + g4)]);
#pragma unroll
          for (int ct = 0; ct < NT; ++ct) sacc[ct][T2] = mfma16x16x32(kop, qb[ct][ks], sacc[ct][T2]);
        }
      }
      float corr[NT];
      u32x4_t pb_hi[NT], pb_lo[NT];
      bool moved = false;
#pragma unroll
      for (int ct = 0; ct < NT; ++ct) {
        float sv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int p = p0 + 16 * (e >> 2) + 4 * g4 + (e & 3);
          const float x = sacc[ct][e >> 2][e & 3] * scale_log2;
          sv[e] = p < Lcol[ct] ? x : -INFINITY;
        }
        float tmax = sv[0];
#pragma unroll
        for (int e = 1; e < 8; ++e) tmax = fmaxf(tmax, sv[e]);
        tmax = group4_max(tmax);
        const float mnew = fmaxf(m[ct], tmax);
        const float msub = mnew == -INFINITY ? 0.f : mnew;
        corr[ct] = mnew == m[ct] ? 1.f : __builtin_amdgcn_exp2f(m[ct] - msub);
        moved |= corr[ct] != 1.f;
        float pf[8], plo[8];
        float lsum = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          pf[e] = __builtin_amdgcn_exp2f(sv[e] - msub);
          lsum += pf[e];
          plo[e] = pf[e] - round_bf16(pf[e]);
        }
        l[ct] = l[ct] * corr[ct] + lsum;
        m[ct] = mnew;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          pb_hi[ct][d] = pack_bf16x2(pf[2 * d], pf[2 * d + 1]);
          pb_lo[ct][d] = pack_bf16x2(plo[2 * d], plo[2 * d + 1]);
        }
      }
      if (__any(moved)) {
#pragma unroll
        for (int ct = 0; ct < NT; ++ct)
#pragma unroll
          for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[ct][hh][i] *= corr[ct];
      }
      // O^T += V^T P^T: V rows P(g4, e) = p0 + 16(e>>2) + 4g4 + (e&3), dims 128hh + 8c + [0, 8).
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        u32x4_t vr[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
          vr[e] = vt[(16 * (e >> 2) + 4 * g4 + (e & 3)) * ROW_CHUNKS + 16 * hh + c];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          u32x4_t a;
#pragma unroll
          for (int d = 0; d < 4; ++d)
            a[d] = interleave_halves(vr[2 * d][i >> 1], vr[2 * d + 1][i >> 1], i & 1);
#pragma unroll
          for (int ct = 0; ct < NT; ++ct) {
            acc[ct][hh][i] = mfma16x16x32(as_bf16x8(a), as_bf16x8(pb_hi[ct]), acc[ct][hh][i]);
            acc[ct][hh][i] = mfma16x16x32(as_bf16x8(a), as_bf16x8(pb_lo[ct]), acc[ct][hh][i]);
          }
        }
      }
    }
    __syncthreads();  // every wave is done with this stage before it is refilled
    issue_tile(lds + (j & 1) * STAGE_U4, krs, vrs, p0 + 2 * BN, w, lane);
  }
  vmcnt_wait<0>();  // no LDS DMA may still target this workgroup's LDS when it exits

  // Epilogue: rows of this wave, 8 consecutive dims per (ct, hh, ii) per lane.
#pragma unroll
  for (int ct = 0; ct < NT; ++ct) {
    const float L = group4_sum(l[ct]);
    const int r = blk * BQ + w * ROWS_PER_WAVE + ct * 16 + c;
    if (r >= T) continue;
    const __bf16* gp = qg + (size_t)r * ldp + (size_t)h * 2 * HD + HD;
    __bf16* op = out + (size_t)r * ldo + (size_t)h * HD;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int d0 = 128 * hh + 32 * g4 + 8 * ii;
        const u32x4_t gb = *reinterpret_cast<const u32x4_t*>(gp + d0);
        u32x4_t ob;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float o0 = round_bf16(acc[ct][hh][2 * k][ii] / L);
          const float o1 = round_bf16(acc[ct][hh][2 * k + 1][ii] / L);
          const float s0 = round_bf16(sigmoid_f32(lo_bf16(gb[k])));
          const float s1 = round_bf16(sigmoid_f32(hi_bf16(gb[k])));
          ob[k] = pack_bf16x2(o0 * s0, o1 * s1);
        }
        *reinterpret_cast<u32x4_t*>(op + d0) = ob;
      }
  }
}

}  // namespace prefill
}  // namespace qe

using namespace qe;

extern "C" hipError_t qe_attn_prefill(const void* q, const void* kc, const void* vc,
                                      const int* pos, const void* qg, long ldp, void* out,
                                      long ldo, int T, int Hq, int Hkv, int max_len, float scale,
                                      hipStream_t stream) {
  auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (T < 1 || Hq < 1 || Hkv < 1 || Hq % Hkv != 0 || max_len < 1 || !pos)
    return hipErrorInvalidValue;
  if (!a16(q) || !a16(kc) || !a16(vc) || !a16(qg) || !a16(out) || ldp % 8 != 0 || ldo % 8 != 0)
    return hipErrorInvalidValue;
  if ((unsigned long long)(max_len + 3 * prefill::BN) * HD * 2 >= (1ull << 32))
    return hipErrorInvalidValue;
  const int nblk = (T + prefill::BQ - 1) / prefill::BQ;
  if (Hq > 65535) return hipErrorInvalidValue;
  prefill::attn_prefill_kernel<<<dim3(nblk, Hq), dim3(prefill::WAVES * WAVE), 0, stream>>>(
      static_cast<const __bf16*>(q), static_cast<const __bf16*>(kc),
      static_cast<const __bf16*>(vc), pos, static_cast<const __bf16*>(qg), ldp,
      static_cast<__bf16*>(out), ldo, T, Hq, Hkv, max_len, scale * 1.4426950408889634f);
  return hipGetLastError();
}
