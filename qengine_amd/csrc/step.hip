// The rest of one decode / verify step around the attention path on gfx950, so that a whole
// step is one hipGraph: embedding gather, RMSNorm1p with the fused residual add, SwiGLU, per-row
// argmax with torch semantics, and the step bookkeeping that stays on the device (speculative
// accept, commit, MTP row select). Semantics: reference csrc/basic.cu:13-98,157-309 (launchers
// :325-381, bindings csrc/bindings.cpp:33-55,68-136, callers python/qengine/engine.py:434-520).
//
// Every kernel computes row r of an n-row pass exactly as a 1-row pass (rows never mix), which
// keeps speculative verify equal to plain greedy decode.
//
// Design notes (MI355X): these are small HBM- or latency-bound kernels. Rows move with 16-byte
// vector loads/stores where alignment allows (scalar fallbacks otherwise); reductions are wave64
// DPP/permlane butterflies plus a fixed-order sum over the waves, so results do not depend on
// timing; argmax reduces (value, index) pairs under a strict total order, which makes any
// partition of the row give torch's answer.
#include "qe_device.hpp"
#include "qe_step.h"

namespace qe {

__device__ __forceinline__ bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15) == 0;
}

// ------------------------------------------------------------------------------ embedding
// out[r] = table[tok[r]]; an id outside [0, V) gives a zero row (no out-of-bounds read).
template <bool VEC>
__global__ void __launch_bounds__(256)
embed_kernel(const __bf16* __restrict__ table, const int* __restrict__ tok,
             __bf16* __restrict__ out, int H, int V, long ldo) {
  const int r = blockIdx.y;
  const int t = tok[r];
  const bool ok = t >= 0 && t < V;
  const int c = blockIdx.x * 256 + threadIdx.x;
  if constexpr (VEC) {
    if (c >= H / 8) return;
    u32x4_t v = {0u, 0u, 0u, 0u};
    if (ok) v = reinterpret_cast<const u32x4_t*>(table + (size_t)t * H)[c];
    reinterpret_cast<u32x4_t*>(out + (size_t)r * ldo)[c] = v;
  } else {
    if (c >= H) return;
    out[(size_t)r * ldo + c] = ok ? table[(size_t)t * H + c] : f32_to_bf16(0.f);
  }
}

// ------------------------------------------------------------------------------ RMSNorm1p
// y = bf16(x * rsqrt(mean(x^2) + eps) * (1 + w)) in fp32, one rounding. With delta, the residual
// add comes first: x = bf16(x + delta) is written back to x, then normalised.
constexpr int NORM_MAX_THREADS = 1024;

// Sum over the workgroup: wave butterflies, then the wave partials in order 0, 1, 2, ...
__device__ __forceinline__ float block_sum_ordered(float v, float* red) {
  const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
  const int nw = (blockDim.x + WAVE - 1) / WAVE;
  v = wave_sum_fast(v);
  if (lane == 0) red[w] = v;
  __syncthreads();
  float s = red[0];
  for (int i = 1; i < nw; ++i) s += red[i];
  return s;
}

// Vector path: thread c8 owns elements 8c8 .. 8c8+7 (H % 8 == 0, H / 8 <= 1024, 16-byte rows),
// read once into registers.
__global__ void __launch_bounds__(NORM_MAX_THREADS)
rmsnorm1p_vec_kernel(__bf16* __restrict__ x, const __bf16* __restrict__ delta,
                     const __bf16* __restrict__ w, __bf16* __restrict__ out, int H, long ldx,
                     long ldd, long ldo, float eps) {
  __shared__ float red[NORM_MAX_THREADS / WAVE];
  const int c8 = threadIdx.x;
  const bool act = c8 < H / 8;
  u32x4_t* xr = reinterpret_cast<u32x4_t*>(x + (size_t)blockIdx.x * ldx) + c8;
  float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (act) {
    const u32x4_t xv = *xr;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = bf16_to_f32(reinterpret_cast<const __bf16*>(&xv)[i]);
    if (delta) {
      const u32x4_t dv = reinterpret_cast<const u32x4_t*>(delta + (size_t)blockIdx.x * ldd)[c8];
      u32x4_t nx;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        v[i] = round_bf16(v[i] + bf16_to_f32(reinterpret_cast<const __bf16*>(&dv)[i]));
        reinterpret_cast<__bf16*>(&nx)[i] = f32_to_bf16(v[i]);
      }
      *xr = nx;  // the residual stream, bf16(x + delta)
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss += v[i] * v[i];
  const float inv = 1.0f / sqrtf(block_sum_ordered(ss, red) / (float)H + eps);
  if (act) {
    const u32x4_t wv = reinterpret_cast<const u32x4_t*>(w)[c8];
    u32x4_t o;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      reinterpret_cast<__bf16*>(&o)[i] =
          f32_to_bf16((v[i] * inv) * (1.0f + bf16_to_f32(reinterpret_cast<const __bf16*>(&wv)[i])));
    reinterpret_cast<u32x4_t*>(out + (size_t)blockIdx.x * ldo)[c8] = o;
  }
}

// Any H and alignment: strided elements, two passes over the row (the second re-reads what this
// thread wrote or read, so no other thread's write is involved).
__global__ void __launch_bounds__(NORM_MAX_THREADS)
rmsnorm1p_kernel(__bf16* __restrict__ x, const __bf16* __restrict__ delta,
                 const __bf16* __restrict__ w, __bf16* __restrict__ out, int H, long ldx,
                 long ldd, long ldo, float eps) {
  __shared__ float red[NORM_MAX_THREADS / WAVE];
  __bf16* xr = x + (size_t)blockIdx.x * ldx;
  float ss = 0.f;
  for (int c = threadIdx.x; c < H; c += blockDim.x) {
    float v = bf16_to_f32(xr[c]);
    if (delta) {
      v = round_bf16(v + bf16_to_f32(delta[(size_t)blockIdx.x * ldd + c]));
      xr[c] = f32_to_bf16(v);
    }
    ss += v * v;
  }
  const float inv = 1.0f / sqrtf(block_sum_ordered(ss, red) / (float)H + eps);
  __bf16* orow = out + (size_t)blockIdx.x * ldo;
  for (int c = threadIdx.x; c < H; c += blockDim.x)
    orow[c] = f32_to_bf16((bf16_to_f32(xr[c]) * inv) * (1.0f + bf16_to_f32(w[c])));
}

// ------------------------------------------------------------------------------ SwiGLU
// gu row = [gate (I) | up (I)]; out = bf16(bf16(silu(g)) * u), silu in fp32 with an accurate exp.
__device__ __forceinline__ float swiglu1(float g, float u) {
  return round_bf16(g / (1.0f + expf(-g))) * u;
}

template <bool VEC>
__global__ void __launch_bounds__(256)
swiglu_kernel(const __bf16* __restrict__ gu, __bf16* __restrict__ out, int I, long ldg,
              long ldo) {
  const int r = blockIdx.y;
  const __bf16* g = gu + (size_t)r * ldg;
  const int c = blockIdx.x * 256 + threadIdx.x;
  if constexpr (VEC) {
    if (c >= I / 8) return;
    const u32x4_t gv = reinterpret_cast<const u32x4_t*>(g)[c];
    const u32x4_t uv = reinterpret_cast<const u32x4_t*>(g + I)[c];
    u32x4_t o;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      reinterpret_cast<__bf16*>(&o)[i] =
          f32_to_bf16(swiglu1(bf16_to_f32(reinterpret_cast<const __bf16*>(&gv)[i]),
                              bf16_to_f32(reinterpret_cast<const __bf16*>(&uv)[i])));
    reinterpret_cast<u32x4_t*>(out + (size_t)r * ldo)[c] = o;
  } else {
    if (c >= I) return;
    out[(size_t)r * ldo + c] = f32_to_bf16(swiglu1(bf16_to_f32(g[c]), bf16_to_f32(g[I + c])));
  }
}

// ------------------------------------------------------------------------------ argmax
// torch semantics: NaN is the maximum, ties go to the lowest index. `better` is a strict total
// order on (value, index), so the winner does not depend on how the row is partitioned.
constexpr int ARGMAX_NONE = 0x7fffffff;  // loses every comparison

__device__ __forceinline__ bool better(float a, int ia, float b, int ib) {
  const bool an = a != a, bn = b != b;
  if (an != bn) return an;
  if (an) return ia < ib;
  if (a != b) return a > b;
  return ia < ib;
}

__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#pragma unroll
  for (int o = WAVE / 2; o > 0; o >>= 1) {
    const float ov = __shfl_xor(v, o);
    const int oi = __shfl_xor(i, o);
    if (better(ov, oi, v, i)) {
      v = ov;
      i = oi;
    }
  }
}

// Workgroup reduction (256 threads); every thread of wave 0 ends with the result.
__device__ __forceinline__ void block_argmax(float& v, int& i) {
  __shared__ float sv[256 / WAVE];
  __shared__ int si[256 / WAVE];
  const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
  wave_argmax(v, i);
  if (lane == 0) {
    sv[w] = v;
    si[w] = i;
  }
  __syncthreads();
  if (w == 0) {
    v = lane < 256 / WAVE ? sv[lane] : -INFINITY;
    i = lane < 256 / WAVE ? si[lane] : ARGMAX_NONE;
    wave_argmax(v, i);
  }
}

// Pass 1: workgroup b of row r reduces the b-th of nb contiguous chunks of the row (8-element
// groups when the row is 16-byte aligned) into pv/pi[r * nb + b].
__global__ void __launch_bounds__(256)
argmax_pass1_kernel(const __bf16* __restrict__ x, int n, long ldx, float* __restrict__ pv,
                    int* __restrict__ pi) {
  const int r = blockIdx.y, b = blockIdx.x, nb = gridDim.x;
  const __bf16* xr = x + (size_t)r * ldx;
  float v = -INFINITY;
  int i = ARGMAX_NONE;
  if (aligned16(xr) && (n & 7) == 0) {
    const int n8 = n >> 3;
    const int per = (n8 + nb - 1) / nb;
    const int beg = b * per, end = min(beg + per, n8);
    for (int k = beg + threadIdx.x; k < end; k += 256) {
      const u32x4_t q = reinterpret_cast<const u32x4_t*>(xr)[k];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float xv = bf16_to_f32(reinterpret_cast<const __bf16*>(&q)[e]);
        if (better(xv, 8 * k + e, v, i)) {
          v = xv;
          i = 8 * k + e;
        }
      }
    }
  } else {
    const int per = (n + nb - 1) / nb;
    const int beg = b * per, end = min(beg + per, n);
    for (int k = beg + threadIdx.x; k < end; k += 256) {
      const float xv = bf16_to_f32(xr[k]);
      if (better(xv, k, v, i)) {
        v = xv;
        i = k;
      }
    }
  }
  block_argmax(v, i);
  if (threadIdx.x == 0) {
    pv[(size_t)r * nb + b] = v;
    pi[(size_t)r * nb + b] = i;
  }
}

// Pass 2: one workgroup per row over its nb partials; out[r] = idmap ? idmap[a] : a. A row of
// -inf only keeps the sentinel index, which maps to 0 (torch's argmax of such a row).
__global__ void __launch_bounds__(256)
argmax_pass2_kernel(const float* __restrict__ pv, const int* __restrict__ pi, int nb,
                    int* __restrict__ out, const int* __restrict__ idmap) {
  const int r = blockIdx.x;
  float v = -INFINITY;
  int i = ARGMAX_NONE;
  for (int k = threadIdx.x; k < nb; k += 256) {
    const float cv = pv[(size_t)r * nb + k];
    const int ci = pi[(size_t)r * nb + k];
    if (better(cv, ci, v, i)) {
      v = cv;
      i = ci;
    }
  }
  block_argmax(v, i);
  if (threadIdx.x == 0) {
    const int a = i == ARGMAX_NONE ? 0 : i;
    out[r] = idmap ? idmap[a] : a;
  }
}

// ------------------------------------------------------------------------------ bookkeeping
// Device control words (int32): ctl[0] pos of in_tok[0], ctl[1] rows pending for the recurrent
// layers' replay, ctl[2] mode (0 prefill: in_tok are given tokens; 1 decode/verify: in_tok =
// [last token, drafts...]), ctl[3] m = last kept row of this pass, ctl[4] cycles, ctl[5]
// accepted drafts, ctl[16 + m] histogram of accepted drafts per cycle. One thread: these are a
// handful of integers, read by the next kernel of the same graph.
__global__ void __launch_bounds__(WAVE)
accept_kernel(const int* __restrict__ in_tok, const int* __restrict__ am, int n,
              int* __restrict__ ctl, int* __restrict__ next_tok, int* __restrict__ log,
              int max_len) {
  if (threadIdx.x != 0) return;
  const int P = ctl[0];
  const bool verify = ctl[2] == 1;
  int m = n - 1;  // prefill keeps every row
  if (verify) {
    // rows 0..m are right: draft i+1 equals the target's argmax after row i; am[m] is the bonus
    m = 0;
    while (m < n - 1 && in_tok[m + 1] == am[m]) ++m;
    for (int i = 0; i <= m; ++i)
      if (P + 1 + i >= 0 && P + 1 + i < max_len) log[P + 1 + i] = am[i];
    ctl[4] += 1;
    ctl[5] += m;
    ctl[16 + m] += 1;
  } else if (in_tok[n] < 0 && P + n >= 0 && P + n < max_len) {
    log[P + n] = am[n - 1];  // last prompt chunk: its last row yields the first new token
  }
  for (int r = 0; r < n; ++r) {
    int nt;
    if (verify)
      nt = am[r];
    else if (r + 1 < n)
      nt = in_tok[r + 1];
    else
      nt = in_tok[n] >= 0 ? in_tok[n] : am[n - 1];
    next_tok[r] = nt;
  }
  ctl[3] = m;
}

// End of a step: advance pos past the kept rows, mark them pending for the recurrent replay and
// set the next pass input to [bonus token, drafts...].
__global__ void __launch_bounds__(WAVE)
commit_kernel(int* __restrict__ ctl, int* __restrict__ in_tok, const int* __restrict__ am,
              const int* __restrict__ drafts, int k) {
  if (threadIdx.x != 0) return;
  const int m = ctl[3];
  ctl[0] += m + 1;
  ctl[1] = m + 1;
  in_tok[0] = am[m];
  for (int j = 0; j < k; ++j) in_tok[1 + j] = drafts[j];
}

// mpos = off < 0 ? pos : pos + m + 1 + off; optionally dst = src row m and draft0 = mtp_am[m].
__global__ void __launch_bounds__(256)
mtp_select_kernel(const int* __restrict__ ctl, int* __restrict__ mpos, int off,
                  const __bf16* __restrict__ src, long lds, __bf16* __restrict__ dst, int H,
                  const int* __restrict__ mtp_am, int* __restrict__ draft0) {
  const int m = ctl[3];
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    mpos[0] = off < 0 ? ctl[0] : ctl[0] + m + 1 + off;
    if (draft0) draft0[0] = mtp_am[m];
  }
  if (src)
    for (int i = blockIdx.x * 256 + threadIdx.x; i < H; i += gridDim.x * 256)
      dst[i] = src[(size_t)m * lds + i];
}

}  // namespace qe

using namespace qe;

static bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

extern "C" hipError_t qe_embed(const void* table, const int* tok, void* out, int n, int H, int V,
                               long ldo, hipStream_t stream) {
  if (!table || !tok || !out || n < 1 || n > 65535 || H < 1 || V < 1 || ldo < H)
    return hipErrorInvalidValue;
  const auto* T = static_cast<const __bf16*>(table);
  auto* O = static_cast<__bf16*>(out);
  if (H % 8 == 0 && ldo % 8 == 0 && al16(table) && al16(out))
    embed_kernel<true><<<dim3((H / 8 + 255) / 256, n), dim3(256), 0, stream>>>(T, tok, O, H, V, ldo);
  else
    embed_kernel<false><<<dim3((H + 255) / 256, n), dim3(256), 0, stream>>>(T, tok, O, H, V, ldo);
  return hipGetLastError();
}

extern "C" hipError_t qe_rmsnorm1p(void* x, const void* delta, const void* w, void* out, int rows,
                                   int H, long ldx, long ldd, long ldo, float eps,
                                   hipStream_t stream) {
  if (!x || !w || !out || rows < 1 || H < 1 || ldx < H || ldo < H || (delta && ldd < H))
    return hipErrorInvalidValue;
  auto* X = static_cast<__bf16*>(x);
  const auto* D = static_cast<const __bf16*>(delta);
  const auto* Wt = static_cast<const __bf16*>(w);
  auto* O = static_cast<__bf16*>(out);
  const bool vec = H % 8 == 0 && H / 8 <= NORM_MAX_THREADS && ldx % 8 == 0 && ldo % 8 == 0 &&
                   (!delta || ldd % 8 == 0) && al16(x) && al16(out) && al16(w) &&
                   (!delta || al16(delta));
  if (vec) {
    const int threads = (H / 8 + WAVE - 1) / WAVE * WAVE;
    rmsnorm1p_vec_kernel<<<dim3(rows), dim3(threads), 0, stream>>>(X, D, Wt, O, H, ldx, ldd, ldo,
                                                                     eps);
  } else {
    const int threads = H >= NORM_MAX_THREADS ? NORM_MAX_THREADS : (H + WAVE - 1) / WAVE * WAVE;
    rmsnorm1p_kernel<<<dim3(rows), dim3(threads), 0, stream>>>(X, D, Wt, O, H, ldx, ldd, ldo, eps);
  }
  return hipGetLastError();
}

extern "C" hipError_t qe_swiglu(const void* gu, void* out, int n, int I, long ldg, long ldo,
                                hipStream_t stream) {
  if (!gu || !out || n < 1 || n > 65535 || I < 1 || ldg < 2L * I || ldo < I)
    return hipErrorInvalidValue;
  const auto* G = static_cast<const __bf16*>(gu);
  auto* O = static_cast<__bf16*>(out);
  if (I % 8 == 0 && ldg % 8 == 0 && ldo % 8 == 0 && al16(gu) && al16(out))
    swiglu_kernel<true><<<dim3((I / 8 + 255) / 256, n), dim3(256), 0, stream>>>(G, O, I, ldg, ldo);
  else
    swiglu_kernel<false><<<dim3((I + 255) / 256, n), dim3(256), 0, stream>>>(G, O, I, ldg, ldo);
  return hipGetLastError();
}

extern "C" hipError_t qe_argmax(const void* x, int rows, int n, long ldx, float* pv, int* pi,
                                int nb, int* out, const int* idmap, hipStream_t stream) {
  if (!x || !pv || !pi || !out || rows < 1 || rows > 65535 || n < 1 || ldx < n || nb < 1)
    return hipErrorInvalidValue;
  argmax_pass1_kernel<<<dim3(nb, rows), dim3(256), 0, stream>>>(static_cast<const __bf16*>(x), n,
                                                                  ldx, pv, pi);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  argmax_pass2_kernel<<<dim3(rows), dim3(256), 0, stream>>>(pv, pi, nb, out, idmap);
  return hipGetLastError();
}

extern "C" hipError_t qe_accept(const int* in_tok, const int* am, int n, int* ctl, int* next_tok,
                                int* log, int max_len, hipStream_t stream) {
  if (!in_tok || !am || !ctl || !next_tok || !log || n < 1 || n > 8 || max_len < 0)
    return hipErrorInvalidValue;
  accept_kernel<<<dim3(1), dim3(WAVE), 0, stream>>>(in_tok, am, n, ctl, next_tok, log, max_len);
  return hipGetLastError();
}

extern "C" hipError_t qe_commit(int* ctl, int* in_tok, const int* am, const int* drafts, int k,
                                hipStream_t stream) {
  if (!ctl || !in_tok || !am || k < 0 || (k > 0 && !drafts)) return hipErrorInvalidValue;
  commit_kernel<<<dim3(1), dim3(WAVE), 0, stream>>>(ctl, in_tok, am, drafts, k);
  return hipGetLastError();
}

extern "C" hipError_t qe_mtp_select(const int* ctl, int* mpos, int off, const void* src, long lds,
                                    void* dst, int H, const int* mtp_am, int* draft0,
                                    hipStream_t stream) {
  if (!ctl || !mpos || (src && (!dst || H < 1 || lds < H)) || (draft0 && !mtp_am))
    return hipErrorInvalidValue;
  const int blocks = src ? (H + 255) / 256 : 1;
  mtp_select_kernel<<<dim3(blocks), dim3(256), 0, stream>>>(
      ctl, mpos, off, static_cast<const __bf16*>(src), lds, static_cast<__bf16*>(dst), H, mtp_am,
      draft0);
  return hipGetLastError();
}

extern "C" hipError_t qe_l2_persist_limit(size_t) { return hipSuccess; }

extern "C" hipError_t qe_stream_access_window(uintptr_t, size_t, float, hipStream_t) {
  return hipSuccess;
}
