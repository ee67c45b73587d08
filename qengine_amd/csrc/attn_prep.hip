// q/k prep for the gated-attention path on gfx950: per (head, row) RMSNorm1p with one bf16
// rounding, then partial rotate-half RoPE with every elementwise op rounded to bf16, then q to
// q_out and k/v to the KV cache (bf16, or the fp8 KV format). Semantics: reference csrc/attn.cu:17-56 and
// python/qengine/reference.py:132-136,158-176,252-260.
//
// One 256-thread workgroup per (head, ROWS consecutive rows): thread c owns dim c of every row
// (qe::prep_dim, shared with the fused prep + decode kernel so both produce the same bits). A
// row is a few KB, so a workgroup's life is one global-load round trip: decode calls (<= 8 rows)
// take one row per workgroup, prefill chunks 8, whose loads are all issued before the first row
// is normalised (2048 rows: 57,344 one-row workgroups ran 51 us).
#include "qe_device.hpp"
#include "qe_attn.h"

namespace qe {

// FP8: the cache is the fp8 KV format (E4M3FN codes, one byte per value): a K or V value x is
// stored as the code of x * inv_scale (fp32 product, round to nearest even, saturated at +-448);
// it dequantizes to code * scale.
template <bool FP8, int ROWS>
__global__ void __launch_bounds__(HD)
attn_prep_kernel(const __bf16* __restrict__ qg, const __bf16* __restrict__ k,
                 const __bf16* __restrict__ v, long ldp, const __bf16* __restrict__ qnw,
                 const __bf16* __restrict__ knw, const float* __restrict__ inv_freq,
                 const int* __restrict__ pos_ptr, __bf16* __restrict__ q_out,
                 void* __restrict__ kc, void* __restrict__ vc, int n, int Hq, int max_len, int rd,
                 float eps, float k_inv, float v_inv) {
  __shared__ float xn[HD];
  __shared__ float red[HD / WAVE];
  const int hb = blockIdx.x, t0 = blockIdx.y * ROWS, c = threadIdx.x;
  const bool is_q = hb < Hq;
  const int h = is_q ? hb : hb - Hq;
  const int pos0 = pos_ptr[0];  // row t is the token at position pos0 + t

  // All loads first, unconditionally (rows past n re-read row n-1, whose results are not stored),
  // so the workgroup pays one memory round trip for its ROWS rows.
  float xs[ROWS];
  __bf16 vs[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; ++r) {
    const size_t row = (size_t)min(t0 + r, n - 1) * ldp;
    xs[r] = bf16_to_f32(is_q ? qg[row + (size_t)h * 2 * HD + c] : k[row + (size_t)h * HD + c]);
    vs[r] = is_q ? __bf16{} : v[row + (size_t)h * HD + c];
  }
  const float wgt = bf16_to_f32(is_q ? qnw[c] : knw[c]);
  // ROWS > 1: the rows' rotary cos/sin (rd/2 frequencies each) are computed once by the whole
  // workgroup, entry (r, f) = rope_cs_f(pos0 + t0 + r, inv_freq[f]), the values thread c < rd would
  // compute for frequency c mod rd/2 (rope_cs), instead of by 64 threads per row.
  constexpr int TAB = ROWS > 1 ? ROWS * (HD / 2) : 1;
  __shared__ float2 rope_tab[TAB];
  const int half = rd >> 1;
  if constexpr (ROWS > 1) {
    for (int i = c; i < ROWS * half; i += HD) {
      const int r = i / half, f = i - r * half;
      const RopeCS cs = rope_cs_f(pos0 + t0 + r, inv_freq[f], rd, f);
      rope_tab[i] = make_float2(cs.cs, cs.sn);
    }
    lds_barrier();
  }
#pragma unroll
  for (int r = 0; r < ROWS; ++r) {
    const int t = t0 + r;
    if (t >= n) break;  // uniform across the workgroup
    const int pos = pos0 + t;
    RopeCS cs;
    if constexpr (ROWS > 1) {
      if (c < rd) {
        const float2 e = rope_tab[r * half + (c < half ? c : c - half)];
        cs = RopeCS{e.x, e.y};
      } else {
        cs = RopeCS{1.f, 0.f};
      }
    } else {
      cs = rope_cs(pos, inv_freq, rd, c);
    }
    const float y = prep_dim(xs[r], wgt, cs, rd, eps, xn, red);
    if (is_q) {
      q_out[(size_t)t * Hq * HD + (size_t)h * HD + c] = f32_to_bf16(y);
    } else if (pos >= 0 && pos < max_len) {  // never write outside the cache
      const size_t dst = ((size_t)h * max_len + pos) * HD + c;
      if constexpr (FP8) {
        static_cast<uint8_t*>(kc)[dst] = f32_to_fp8(round_bf16(y) * k_inv);
        static_cast<uint8_t*>(vc)[dst] = f32_to_fp8(bf16_to_f32(vs[r]) * v_inv);
      } else {
        static_cast<__bf16*>(kc)[dst] = f32_to_bf16(y);
        static_cast<__bf16*>(vc)[dst] = vs[r];
      }
    }
    // xn and red are free for the next row: prep_dim's second barrier follows every read of red,
    // and the next row's first barrier follows every read of xn.
  }
}

// Rows per workgroup: one for decode calls, 8 for prefill chunks.
template <bool FP8>
static void launch_prep(const void* qg, const void* k, const void* v, long ldp, const void* qnw,
                        const void* knw, const float* inv_freq, const int* pos, void* q_out,
                        void* kc, void* vc, int n, int Hq, int Hkv, int max_len, int rd, float eps,
                        float k_inv, float v_inv, hipStream_t stream) {
  const auto* QG = static_cast<const __bf16*>(qg);
  const auto* K = static_cast<const __bf16*>(k);
  const auto* V = static_cast<const __bf16*>(v);
  const auto* QW = static_cast<const __bf16*>(qnw);
  const auto* KW = static_cast<const __bf16*>(knw);
  auto* QO = static_cast<__bf16*>(q_out);
  if (n <= 8)
    attn_prep_kernel<FP8, 1><<<dim3(Hq + Hkv, n), dim3(HD), 0, stream>>>(
        QG, K, V, ldp, QW, KW, inv_freq, pos, QO, kc, vc, n, Hq, max_len, rd, eps, k_inv, v_inv);
  else
    attn_prep_kernel<FP8, 8><<<dim3(Hq + Hkv, (n + 7) / 8), dim3(HD), 0, stream>>>(
        QG, K, V, ldp, QW, KW, inv_freq, pos, QO, kc, vc, n, Hq, max_len, rd, eps, k_inv, v_inv);
}

}  // namespace qe

using namespace qe;

static bool prep_args_ok(const void* qg, const void* k, const void* v, long ldp, const void* qnw,
                         const void* knw, const float* inv_freq, const int* pos, void* q_out,
                         void* kc, void* vc, int n, int Hq, int Hkv, int max_len, int rd) {
  return !(n < 1 || n > 65535 || Hq < 1 || Hkv < 1 || max_len < 1 || rd < 0 || rd > HD ||
           (rd & 1) || ldp < 1 || !qg || !k || !v || !qnw || !knw || !inv_freq || !pos ||
           !q_out || !kc || !vc);
}

extern "C" hipError_t qe_attn_prep(const void* qg, const void* k, const void* v, long ldp,
                                   const void* qnw, const void* knw, const float* inv_freq,
                                   const int* pos, void* q_out, void* kc, void* vc, int n, int Hq,
                                   int Hkv, int max_len, int rd, float eps, hipStream_t stream) {
  if (!prep_args_ok(qg, k, v, ldp, qnw, knw, inv_freq, pos, q_out, kc, vc, n, Hq, Hkv, max_len, rd))
    return hipErrorInvalidValue;
  launch_prep<false>(qg, k, v, ldp, qnw, knw, inv_freq, pos, q_out, kc, vc, n, Hq, Hkv, max_len,
                     rd, eps, 1.f, 1.f, stream);
  return hipGetLastError();
}

extern "C" hipError_t qe_attn_prep_fp8(const void* qg, const void* k, const void* v, long ldp,
                                       const void* qnw, const void* knw, const float* inv_freq,
                                       const int* pos, void* q_out, void* kc8, void* vc8, int n,
                                       int Hq, int Hkv, int max_len, int rd, float eps,
                                       float k_scale, float v_scale, hipStream_t stream) {
  if (!prep_args_ok(qg, k, v, ldp, qnw, knw, inv_freq, pos, q_out, kc8, vc8, n, Hq, Hkv, max_len,
                    rd) ||
      !kv_scale_ok(k_scale) || !kv_scale_ok(v_scale))
    return hipErrorInvalidValue;
  launch_prep<true>(qg, k, v, ldp, qnw, knw, inv_freq, pos, q_out, kc8, vc8, n, Hq, Hkv, max_len,
                    rd, eps, 1.0f / k_scale, 1.0f / v_scale, stream);
  return hipGetLastError();
}
