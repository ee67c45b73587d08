// q/k prep for the gated-attention path on gfx950: per (head, row) RMSNorm1p with one bf16
// rounding, then partial rotate-half RoPE with every elementwise op rounded to bf16, then q to
// q_out and k/v to the KV cache (bf16, or the fp8 KV format). Semantics: reference csrc/attn.cu:17-56 and
// python/qengine/reference.py:132-136,158-176,252-260.
//
// One 256-thread workgroup per (head, row): thread c owns dim c (qe::prep_dim, shared with the
// fused prep + decode kernel so both produce the same bits). The op is a few KB per row and
// launch-latency bound.
#include "qe_device.hpp"
#include "qe_attn.h"

namespace qe {

// FP8: the cache is the fp8 KV format (E4M3FN codes, one byte per value): a K or V value x is
// stored as the code of x * inv_scale (fp32 product, round to nearest even, saturated at +-448);
// it dequantizes to code * scale.
template <bool FP8>
__global__ void __launch_bounds__(HD)
attn_prep_kernel(const __bf16* __restrict__ qg, const __bf16* __restrict__ k,
                 const __bf16* __restrict__ v, long ldp, const __bf16* __restrict__ qnw,
                 const __bf16* __restrict__ knw, const float* __restrict__ inv_freq,
                 const int* __restrict__ pos_ptr, __bf16* __restrict__ q_out,
                 void* __restrict__ kc, void* __restrict__ vc, int Hq, int max_len, int rd,
                 float eps, float k_inv, float v_inv) {
  __shared__ float xn[HD];
  __shared__ float red[HD / WAVE];
  const int hb = blockIdx.x, t = blockIdx.y, c = threadIdx.x;
  const bool is_q = hb < Hq;
  const int h = is_q ? hb : hb - Hq;
  const int pos = pos_ptr[0] + t;  // row t is the token at position pos + t
  const size_t row = (size_t)t * ldp;

  const float x = bf16_to_f32(is_q ? qg[row + (size_t)h * 2 * HD + c] : k[row + (size_t)h * HD + c]);
  const float wgt = bf16_to_f32(is_q ? qnw[c] : knw[c]);
  const float y = prep_dim(x, wgt, rope_cs(pos, inv_freq, rd, c), rd, eps, xn, red);
  if (is_q) {
    q_out[(size_t)t * Hq * HD + (size_t)h * HD + c] = f32_to_bf16(y);
  } else if (pos >= 0 && pos < max_len) {  // never write outside the cache
    const size_t dst = ((size_t)h * max_len + pos) * HD + c;
    const __bf16 vv = v[row + (size_t)h * HD + c];
    if constexpr (FP8) {
      static_cast<uint8_t*>(kc)[dst] = f32_to_fp8(round_bf16(y) * k_inv);
      static_cast<uint8_t*>(vc)[dst] = f32_to_fp8(bf16_to_f32(vv) * v_inv);
    } else {
      static_cast<__bf16*>(kc)[dst] = f32_to_bf16(y);
      static_cast<__bf16*>(vc)[dst] = vv;
    }
  }
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
  attn_prep_kernel<false><<<dim3(Hq + Hkv, n), dim3(HD), 0, stream>>>(
      static_cast<const __bf16*>(qg), static_cast<const __bf16*>(k),
      static_cast<const __bf16*>(v), ldp, static_cast<const __bf16*>(qnw),
      static_cast<const __bf16*>(knw), inv_freq, pos, static_cast<__bf16*>(q_out), kc, vc, Hq,
      max_len, rd, eps, 1.f, 1.f);
  return hipGetLastError();
}

extern "C" hipError_t qe_attn_prep_fp8(const void* qg, const void* k, const void* v, long ldp,
                                       const void* qnw, const void* knw, const float* inv_freq,
                                       const int* pos, void* q_out, void* kc8, void* vc8, int n,
                                       int Hq, int Hkv, int max_len, int rd, float eps,
                                       float k_scale, float v_scale, hipStream_t stream) {
  if (!prep_args_ok(qg, k, v, ldp, qnw, knw, inv_freq, pos, q_out, kc8, vc8, n, Hq, Hkv, max_len,
                    rd) ||
      !(k_scale > 0.f) || !(v_scale > 0.f) || k_scale == INFINITY || v_scale == INFINITY)
    return hipErrorInvalidValue;
  attn_prep_kernel<true><<<dim3(Hq + Hkv, n), dim3(HD), 0, stream>>>(
      static_cast<const __bf16*>(qg), static_cast<const __bf16*>(k),
      static_cast<const __bf16*>(v), ldp, static_cast<const __bf16*>(qnw),
      static_cast<const __bf16*>(knw), inv_freq, pos, static_cast<__bf16*>(q_out), kc8, vc8, Hq,
      max_len, rd, eps, 1.0f / k_scale, 1.0f / v_scale);
  return hipGetLastError();
}
