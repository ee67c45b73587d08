// q/k prep for the gated-attention path on gfx950: per (head, row) RMSNorm1p with one bf16
// rounding, then partial rotate-half RoPE with every elementwise op rounded to bf16, then q to
// q_out and k/v to the KV cache. Semantics: reference csrc/attn.cu:17-56 and
// python/qengine/reference.py:132-136,158-176,252-260.
//
// One 256-thread workgroup per (head, row): thread c owns dim c (qe::prep_dim, shared with the
// fused prep + decode kernel so both produce the same bits). The op is a few KB per row and
// launch-latency bound.
#include "qe_device.hpp"
#include "qe_attn.h"

namespace qe {

__global__ void __launch_bounds__(HD)
attn_prep_kernel(const __bf16* __restrict__ qg, const __bf16* __restrict__ k,
                 const __bf16* __restrict__ v, long ldp, const __bf16* __restrict__ qnw,
                 const __bf16* __restrict__ knw, const float* __restrict__ inv_freq,
                 const int* __restrict__ pos_ptr, __bf16* __restrict__ q_out,
                 __bf16* __restrict__ kc, __bf16* __restrict__ vc, int Hq, int max_len, int rd,
                 float eps) {
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
    kc[dst] = f32_to_bf16(y);
    vc[dst] = v[row + (size_t)h * HD + c];
  }
}

}  // namespace qe

using namespace qe;

extern "C" hipError_t qe_attn_prep(const void* qg, const void* k, const void* v, long ldp,
                                   const void* qnw, const void* knw, const float* inv_freq,
                                   const int* pos, void* q_out, void* kc, void* vc, int n, int Hq,
                                   int Hkv, int max_len, int rd, float eps, hipStream_t stream) {
  if (n < 1 || n > 65535 || Hq < 1 || Hkv < 1 || max_len < 1 || rd < 0 ||
      rd > HD || (rd & 1) || ldp < 1 || !qg || !k || !v || !qnw || !knw || !inv_freq || !pos ||
      !q_out || !kc || !vc)
    return hipErrorInvalidValue;
  attn_prep_kernel<<<dim3(Hq + Hkv, n), dim3(HD), 0, stream>>>(
      static_cast<const __bf16*>(qg), static_cast<const __bf16*>(k),
      static_cast<const __bf16*>(v), ldp, static_cast<const __bf16*>(qnw),
      static_cast<const __bf16*>(knw), inv_freq, pos, static_cast<__bf16*>(q_out),
      static_cast<__bf16*>(kc), static_cast<__bf16*>(vc), Hq, max_len, rd, eps);
  return hipGetLastError();
}
