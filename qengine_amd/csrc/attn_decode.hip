// Gated flash-decoding over a bf16 KV cache for n = 1..8 query rows on gfx950 (MI355X).
//
// Semantics follow the reference (csrc/attn.cu:1-9,58-149): row t sits at position pos+t and
// attends cache positions [0, min(pos+t+1, max_len)); scores are q.k * scale; the output is
// bf16(bf16(softmax . V) * bf16(sigmoid(gate))).
//
// Design (MI355X-first, not a translation of the reference's warp-per-position loop):
//  * One workgroup per (split-KV slice, KV head). The slice size CH depends only on (max_len,
//    NS), so every row of every call sees the same slices: row t of an n-row call is
//    bit-identical to a 1-row call at position pos+t, and rows can share each K/V tile.
//  * The Hq/Hkv query heads of the GQA group times the n rows form the columns of the MFMA tiles
//    (NT tiles of 16 columns). K and V are read from HBM exactly once per call; Q stays in
//    registers as an MFMA operand.
//  * S^T = K Q^T and O^T += V^T P^T on v_mfma_f32_16x16x32_bf16. K rows are loaded with 16-byte
//    buffer loads straight into the MFMA A layout. V is loaded as 16-byte row pieces of 8
//    positions and regrouped by v_perm into position pairs. With ~6 FLOP per byte, GQA-6 decode
//    would otherwise need ~70% of the non-packed fp32 VALU peak at 8 TB/s.
//  * Online softmax in the log2 domain per column. Row max/sum reductions over the 4 lane groups
//    use cross-lane shuffles. Rescaling of the accumulators is skipped when no column's max
//    moved (an exact no-op).
//  * Buffer resources bound the K/V reads to the attended range: positions past it load as 0.
//  * A second launch merges the slices (log-sum-exp) and applies the sigmoid gate.
#include "qe_device.hpp"
#include "qe_attn.h"

namespace qe {

constexpr int TILE = 32;               // cache positions per wave step (two 16-row MFMA tiles)
constexpr int WAVES = 4;               // waves per workgroup
constexpr int THREADS = WAVES * WAVE;  // 256

__host__ __device__ inline int split_size(int max_len, int NS) {
  long per = ((long)max_len + NS - 1) / NS;
  per = (per + TILE - 1) / TILE * TILE;
  return per < TILE ? TILE : (int)per;
}

// part_o [n][Hq][NS][HD] (unnormalised O), part_ml [n][Hq][NS][2] = (max in log2 units, sum).
template <int NT>
__global__ void __launch_bounds__(THREADS)
attn_partials_kernel(const __bf16* __restrict__ q, const __bf16* __restrict__ kc,
                     const __bf16* __restrict__ vc, const int* __restrict__ pos_ptr,
                     float* __restrict__ part_o, float* __restrict__ part_ml, int n, int Hq,
                     int Hkv, int max_len, int NS, int CH, float scale_log2) {
  const int s = blockIdx.x, g = blockIdx.y;
  const int grp = Hq / Hkv;
  const int pos0 = pos_ptr[0];
  const int Lmax = min(pos0 + n, max_len);  // attended length of the last row
  const int beg = s * CH;
  if (beg >= Lmax) return;  // slice holds no attended position (uniform per workgroup)
  const int end = min(beg + CH, Lmax);

  const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
  const int c = lane & 15, g4 = lane >> 4;
  const int ncols = grp * n;

  // Q^T as the MFMA B operand. Column ct*16+c is (row t, head g*grp+j), col = t*grp + j.
  // Lane group g4 holds dims [32ks + 8g4, +8) of k-step ks (the same dims as the K operand).
  bf16x8_t qb[NT][8];
  int Lcol[NT];
#pragma unroll
  for (int ct = 0; ct < NT; ++ct) {
    const int col = ct * 16 + c;
    if (col < ncols) {
      const int t = col / grp, j = col - t * grp;
      Lcol[ct] = min(pos0 + t + 1, max_len);
      const u32x4_t* src =
          reinterpret_cast<const u32x4_t*>(q + (size_t)t * Hq * HD + (size_t)(g * grp + j) * HD);
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) qb[ct][ks] = as_bf16x8(src[4 * ks + g4]);
    } else {
      Lcol[ct] = 0;  // padding column: every position masked
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) qb[ct][ks] = as_bf16x8(u32x4_t{0u, 0u, 0u, 0u});
    }
  }

  const size_t head_off = (size_t)g * max_len * HD;
  const uint32_t bytes = (uint32_t)Lmax * (uint32_t)(HD * 2);
  const __amdgpu_buffer_rsrc_t krs = make_rsrc(kc + head_off, bytes);
  const __amdgpu_buffer_rsrc_t vrs = make_rsrc(vc + head_off, bytes);

  float m[NT], l[NT];
  f32x4_t acc[NT][2][8];  // O^T: [ct][half h][i] rows = dims 128h + 32g4 + 8ii + i, col c
#pragma unroll
  for (int ct = 0; ct < NT; ++ct) {
    m[ct] = -INFINITY;
    l[ct] = 0.f;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[ct][h][i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  for (int p0 = beg + w * TILE; p0 < end; p0 += WAVES * TILE) {
    // K: A-operand rows p0 + 16T + c, dims [32ks + 8g4, +8).
    u32x4_t kr[2][8];
#pragma unroll
    for (int T = 0; T < 2; ++T)
#pragma unroll
      for (int ks = 0; ks < 8; ++ks)
        kr[T][ks] = buffer_load16(krs, (uint32_t)(p0 + 16 * T + c) * (HD * 2) + (4 * ks + g4) * 16);
    // V: 8 positions per lane, P(g4, e) = p0 + 16(e>>2) + 4g4 + (e&3), dims 128h + 8c + [0,8).
    u32x4_t vr[8][2];
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        vr[e][h] = buffer_load16(
            vrs, (uint32_t)(p0 + 16 * (e >> 2) + 4 * g4 + (e & 3)) * (HD * 2) + (128 * h + 8 * c) * 2);

    // S^T = K Q^T: lane holds positions p0 + 16T + 4g4 + i of column c.
    f32x4_t sacc[NT][2];
#pragma unroll
    for (int ct = 0; ct < NT; ++ct)
#pragma unroll
      for (int T = 0; T < 2; ++T) {
        f32x4_t a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) a = mfma16x16x32(as_bf16x8(kr[T][ks]), qb[ct][ks], a);
        sacc[ct][T] = a;
      }

    // Online softmax per column (log2 domain). P^T goes to the B operand with element e <-> P(g4, e),
    // as two bf16 terms hi + lo (hi = bf16(p), lo = bf16(p - hi)): ~2^-17 relative error, so P.V
    // keeps fp32-class accuracy at the cost of a second MFMA per tile.
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
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[ct][h][i] *= corr[ct];
    }

    // O^T += V^T P^T. A-operand row c of tile (h, i) is dim 128h + 8c + i over the 8 positions.
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        u32x4_t a;
#pragma unroll
        for (int d = 0; d < 4; ++d)
          a[d] = interleave_halves(vr[2 * d][h][i >> 1], vr[2 * d + 1][h][i >> 1], i & 1);
#pragma unroll
        for (int ct = 0; ct < NT; ++ct) {
          acc[ct][h][i] = mfma16x16x32(as_bf16x8(a), as_bf16x8(pb_hi[ct]), acc[ct][h][i]);
          acc[ct][h][i] = mfma16x16x32(as_bf16x8(a), as_bf16x8(pb_lo[ct]), acc[ct][h][i]);
        }
      }
  }

  // ---- merge the waves of this workgroup in a fixed order and write the slice's partial
#pragma unroll
  for (int ct = 0; ct < NT; ++ct) l[ct] = group4_sum(l[ct]);

  __shared__ float s_m[WAVES][16 * NT], s_l[WAVES][16 * NT];
  __shared__ float s_acc[WAVES][32][WAVE];
  if (g4 == 0) {
#pragma unroll
    for (int ct = 0; ct < NT; ++ct) {
      s_m[w][ct * 16 + c] = m[ct];
      s_l[w][ct * 16 + c] = l[ct];
    }
  }
  __syncthreads();

  float wsc[NT][WAVES];
#pragma unroll
  for (int ct = 0; ct < NT; ++ct) {
    const int col = ct * 16 + c;
    float M = -INFINITY;
#pragma unroll
    for (int v = 0; v < WAVES; ++v) M = fmaxf(M, s_m[v][col]);
    float L = 0.f;
#pragma unroll
    for (int v = 0; v < WAVES; ++v) {
      const float mv = s_m[v][col];
      wsc[ct][v] = mv == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mv - M);
      L += s_l[v][col] * wsc[ct][v];
    }
    if (w == 0 && g4 == 0 && col < ncols) {
      const int t = col / grp, head = g * grp + (col - t * grp);
      float* ml = part_ml + (((size_t)t * Hq + head) * NS + s) * 2;
      ml[0] = M;
      ml[1] = L;
    }
  }

#pragma unroll
  for (int ct = 0; ct < NT; ++ct) {
    const int col = ct * 16 + c;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) s_acc[w][i * 4 + ii][lane] = acc[ct][h][i][ii];
      __syncthreads();
      // this thread merges ii = w for i = 0..7: dims 128h + 32g4 + 8w + [0, 8)
      float o[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float sum = 0.f;
#pragma unroll
        for (int v = 0; v < WAVES; ++v) sum += s_acc[v][i * 4 + w][lane] * wsc[ct][v];
        o[i] = sum;
      }
      if (col < ncols) {
        const int t = col / grp, head = g * grp + (col - t * grp);
        float* dst = part_o + (((size_t)t * Hq + head) * NS + s) * HD + 128 * h + 32 * g4 + 8 * w;
        reinterpret_cast<f32x4_t*>(dst)[0] = f32x4_t{o[0], o[1], o[2], o[3]};
        reinterpret_cast<f32x4_t*>(dst)[1] = f32x4_t{o[4], o[5], o[6], o[7]};
      }
      __syncthreads();
    }
  }
}

// Log-sum-exp merge of the slices holding row t's positions + fused sigmoid output gate.
__global__ void __launch_bounds__(HD)
attn_combine_kernel(const float* __restrict__ part_o, const float* __restrict__ part_ml,
                    const int* __restrict__ pos_ptr, const __bf16* __restrict__ qg, long ldp,
                    __bf16* __restrict__ out, long ldo, int Hq, int max_len, int NS, int CH) {
  const int h = blockIdx.x, t = blockIdx.y, c = threadIdx.x;
  const int L_t = min(pos_ptr[0] + t + 1, max_len);
  const int S = L_t > 0 ? (L_t + CH - 1) / CH : 0;
  const size_t base = ((size_t)t * Hq + h) * NS;
  const float* ml = part_ml + base * 2;
  float M = -INFINITY;
  for (int s = 0; s < S; ++s) M = fmaxf(M, ml[2 * s]);
  float L = 0.f, O = 0.f;
  for (int s = 0; s < S; ++s) {
    const float ms = ml[2 * s];
    if (ms == -INFINITY) continue;
    const float f = __builtin_amdgcn_exp2f(ms - M);
    L += ml[2 * s + 1] * f;
    O += part_o[(base + s) * HD + c] * f;
  }
  const float o = round_bf16(O / L);
  const float gate = bf16_to_f32(qg[(size_t)t * ldp + (size_t)h * 2 * HD + HD + c]);
  const float sg = round_bf16(sigmoid_f32(gate));
  out[(size_t)t * ldo + (size_t)h * HD + c] = f32_to_bf16(o * sg);
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

static hipError_t check_decode_shape(int n, int Hq, int Hkv, int max_len, int NS) {
  if (n < 1 || n > 8 || Hq < 1 || Hkv < 1 || Hq % Hkv != 0 || NS < 1 || max_len < 1)
    return hipErrorInvalidValue;
  if ((Hq / Hkv) * n > 64) return hipErrorInvalidValue;            // at most 4 column tiles
  // byte offsets (including the tile overhang past max_len) must fit the 32-bit buffer range
  if ((unsigned long long)(max_len + TILE) * HD * 2 >= (1ull << 32)) return hipErrorInvalidValue;
  return hipSuccess;
}

static hipError_t launch_partials(const void* q, const void* kc, const void* vc, const int* pos,
                                  float* part_o, float* part_ml, int n, int Hq, int Hkv,
                                  int max_len, int NS, float scale, hipStream_t stream) {
  const int CH = split_size(max_len, NS);
  const int slices = (max_len + CH - 1) / CH;  // <= NS; later slices never hold positions
  const dim3 grid(slices, Hkv), block(THREADS);
  const float scale_log2 = scale * 1.4426950408889634f;
  const int NT = ((Hq / Hkv) * n + 15) / 16;
  const auto* Q = static_cast<const __bf16*>(q);
  const auto* K = static_cast<const __bf16*>(kc);
  const auto* V = static_cast<const __bf16*>(vc);
  switch (NT) {
    case 1: attn_partials_kernel<1><<<grid, block, 0, stream>>>(Q, K, V, pos, part_o, part_ml, n, Hq, Hkv, max_len, NS, CH, scale_log2); break;
    case 2: attn_partials_kernel<2><<<grid, block, 0, stream>>>(Q, K, V, pos, part_o, part_ml, n, Hq, Hkv, max_len, NS, CH, scale_log2); break;
    case 3: attn_partials_kernel<3><<<grid, block, 0, stream>>>(Q, K, V, pos, part_o, part_ml, n, Hq, Hkv, max_len, NS, CH, scale_log2); break;
    default: attn_partials_kernel<4><<<grid, block, 0, stream>>>(Q, K, V, pos, part_o, part_ml, n, Hq, Hkv, max_len, NS, CH, scale_log2); break;
  }
  return hipGetLastError();
}

static hipError_t launch_combine(const float* part_o, const float* part_ml, const int* pos,
                                 const void* qg, long ldp, void* out, long ldo, int n, int Hq,
                                 int max_len, int NS, hipStream_t stream) {
  const int CH = split_size(max_len, NS);
  attn_combine_kernel<<<dim3(Hq, n), dim3(HD), 0, stream>>>(
      part_o, part_ml, pos, static_cast<const __bf16*>(qg), ldp, static_cast<__bf16*>(out), ldo,
      Hq, max_len, NS, CH);
  return hipGetLastError();
}

}  // namespace qe

using namespace qe;

extern "C" int qe_attn_split_size(int max_len, int NS) {
  if (max_len < 1 || NS < 1) return 0;
  return split_size(max_len, NS);
}

extern "C" hipError_t qe_attn_decode_partials(const void* q, const void* kc, const void* vc,
                                              const int* pos, float* part_o, float* part_ml,
                                              int n, int Hq, int Hkv, int max_len, int NS,
                                              float scale, hipStream_t stream) {
  hipError_t e = check_decode_shape(n, Hq, Hkv, max_len, NS);
  if (e != hipSuccess) return e;
  if (!aligned16(q) || !aligned16(kc) || !aligned16(vc) || !aligned16(part_o) || !pos || !part_ml)
    return hipErrorInvalidValue;
  return launch_partials(q, kc, vc, pos, part_o, part_ml, n, Hq, Hkv, max_len, NS, scale, stream);
}

extern "C" hipError_t qe_attn_decode_combine(const float* part_o, const float* part_ml,
                                             const int* pos, const void* qg, long ldp, void* out,
                                             long ldo, int n, int Hq, int max_len, int NS,
                                             hipStream_t stream) {
  if (n < 1 || n > 8 || Hq < 1 || NS < 1 || max_len < 1 || !part_o || !part_ml || !pos || !qg ||
      !out)
    return hipErrorInvalidValue;
  return launch_combine(part_o, part_ml, pos, qg, ldp, out, ldo, n, Hq, max_len, NS, stream);
}

extern "C" hipError_t qe_attn_decode(const void* q, const void* kc, const void* vc, const int* pos,
                                     const void* qg, long ldp, float* part_o, float* part_ml,
                                     void* out, long ldo, int n, int Hq, int Hkv, int max_len,
                                     int NS, float scale, hipStream_t stream) {
  hipError_t e = qe_attn_decode_partials(q, kc, vc, pos, part_o, part_ml, n, Hq, Hkv, max_len, NS,
                                         scale, stream);
  if (e != hipSuccess) return e;
  return qe_attn_decode_combine(part_o, part_ml, pos, qg, ldp, out, ldo, n, Hq, max_len, NS,
                                stream);
}

extern "C" const char* qe_attn_version(void) { return "qengine_amd attn 0.1 (gfx950)"; }
extern "C" void qe_set_pdl_trigger(int) {}
extern "C" void qe_set_pdl_launch(int) {}
