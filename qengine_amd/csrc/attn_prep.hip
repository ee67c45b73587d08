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

// One head per half-wave, eight heads of R consecutive rows per 256-thread workgroup: lane L of
// the half-wave owns dims 8L .. 8L+7 of each row (16-byte loads and stores), and all R rows'
// loads are issued before the first row is normalised.
// The arithmetic is prep_dim's, to the bit: the sum of squares of each 64-dim group follows
// wave_sum_fast's butterfly (dims c and c^32, c^16, c^8 sit in lanes L^4, L^2, L^1 at the same
// slot; c^4, c^2, c^1 in slots k^4, k^2, k^1 of the same lane), and the four group sums are added
// in the order ((r0 + r1) + r2) + r3. The rotary cos/sin of the rows' rd/2 frequencies (fp64
// cos/sin, the kernel's most expensive step) are computed once per workgroup into an LDS table
// (one workgroup barrier); the rotate_half partner goes through the half-wave's own LDS row.
// Needs 16-byte aligned rows (checked by the launcher; otherwise attn_prep_kernel runs).
// The rotary lanes read the rotate_half partner and cos/sin as 16-byte vectors (8 consecutive
// dims of one side of rd/2; scalar reads where rd/2 is not a multiple of 8).
// 2048-row chunk at 24 Q / 4 KV heads, same box: 33.4 us for attn_prep_kernel<false, 8>, about
// 18.5 us here (the launcher's R; 20.7 with scalar rotary reads).
template <bool FP8, int R>
__global__ void __launch_bounds__(HD)
attn_prep_rows_kernel(const __bf16* __restrict__ qg, const __bf16* __restrict__ k,
                      const __bf16* __restrict__ v, long ldp, const __bf16* __restrict__ qnw,
                      const __bf16* __restrict__ knw, const float* __restrict__ inv_freq,
                      const int* __restrict__ pos_ptr, __bf16* __restrict__ q_out,
                      void* __restrict__ kc, void* __restrict__ vc, int n, int Hq, int Hkv,
                      int max_len, int rd, float eps, float k_inv, float v_inv) {
  constexpr int HW = 32;                   // lanes per head
  constexpr int UPW = HD / HW;             // heads per workgroup
  constexpr int TE = (R * (HD / 2) + HD - 1) / HD;  // table entries per thread, at most
  __shared__ __attribute__((aligned(16))) float xn_all[UPW][HD];  // per half-wave: normalised row
  __shared__ __attribute__((aligned(16))) float2 cst[R][HD / 2];  // cos/sin of rd/2 frequencies
  const int tid = threadIdx.x, hw = tid / HW, L = tid & (HW - 1);
  const int nh = Hq + Hkv, wpr = (nh + UPW - 1) / UPW;  // workgroups per row group
  const int grp = blockIdx.x / wpr, t0 = grp * R;
  const int hb_raw = (blockIdx.x - grp * wpr) * UPW + hw;
  const int hb = min(hb_raw, nh - 1);  // the last workgroup of a row group may hold fewer heads
  const bool is_q = hb < Hq;
  const int h = is_q ? hb : hb - Hq;
  float* xn = xn_all[hw];
  const int half = rd >> 1;            // <= 128
  // table entry e = tid + HD i: row e / half, frequency e % half. Its frequency is loaded first
  // (vmcnt counts in order), then every row's input, which fly while the table is computed.
  float fr[TE];
#pragma unroll
  for (int i = 0; i < TE; ++i) {
    const int e = tid + HD * i;
    fr[i] = half > 0 ? inv_freq[e < R * half ? e % half : 0] : 0.f;
  }
  u32x4_t xr[R], vr[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const size_t row = (size_t)min(t0 + r, n - 1) * ldp;  // rows past n re-read row n - 1
    xr[r] = *reinterpret_cast<const u32x4_t*>(
        is_q ? qg + row + (size_t)h * 2 * HD + 8 * L : k + row + (size_t)h * HD + 8 * L);
    vr[r] = is_q ? u32x4_t{0u, 0u, 0u, 0u}
                 : *reinterpret_cast<const u32x4_t*>(v + row + (size_t)h * HD + 8 * L);
  }
  const u32x4_t wr = *reinterpret_cast<const u32x4_t*>((is_q ? qnw : knw) + 8 * L);
  const int pos0 = pos_ptr[0] + t0;
#pragma unroll
  for (int i = 0; i < TE; ++i) {
    const int e = tid + HD * i;
    if (e < R * half) {
      const int r = e / half, f = e - r * half;
      const RopeCS c = rope_cs_f(pos0 + r, fr[i], rd, f);
      cst[r][f] = make_float2(c.cs, c.sn);
    }
  }
  lds_barrier();
  if (hb_raw >= nh) return;
  float w[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    w[2 * i] = lo_bf16(wr[i]);
    w[2 * i + 1] = hi_bf16(wr[i]);
  }
  const int base = (tid & ~(HW - 1)) & (WAVE - 1);  // lane 0 of the half-wave
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int t = t0 + r, pos = pos0 + r;
    if (t >= n) break;  // uniform across the workgroup
    float x[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = lo_bf16(xr[r][i]);
      x[2 * i + 1] = hi_bf16(xr[r][i]);
    }
    // sum of squares of the lane's 64-dim group, in wave_sum_fast's order
    float s[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) s[q] = x[q] * x[q];
#pragma unroll
    for (int q = 0; q < 8; ++q) s[q] = s[q] + dpp<0x1B>(dpp<0x141>(s[q]));  // lane ^ 4: dim ^ 32
#pragma unroll
    for (int q = 0; q < 8; ++q) s[q] = s[q] + dpp<0x4E>(s[q]);              // lane ^ 2: dim ^ 16
#pragma unroll
    for (int q = 0; q < 8; ++q) s[q] = s[q] + dpp<0xB1>(s[q]);              // lane ^ 1: dim ^ 8
    float u[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) u[q] = s[q] + s[q + 4];                     // dim ^ 4
    const float gsum = (u[0] + u[2]) + (u[1] + u[3]);                       // dim ^ 2, then ^ 1
    const float r0 = __shfl(gsum, base), r1 = __shfl(gsum, base + 8);
    const float r2 = __shfl(gsum, base + 16), r3 = __shfl(gsum, base + 24);
    const float total = ((r0 + r1) + r2) + r3;
    const float inv = 1.0f / sqrtf(total / (float)HD + eps);
    float xv[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) xv[q] = round_bf16((x[q] * inv) * (1.0f + w[q]));
    // the half-wave's LDS row: the previous row's partner reads are done before it is rewritten
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
    *reinterpret_cast<f32x4_t*>(&xn[8 * L]) = f32x4_t{xv[0], xv[1], xv[2], xv[3]};
    *reinterpret_cast<f32x4_t*>(&xn[8 * L + 4]) = f32x4_t{xv[4], xv[5], xv[6], xv[7]};
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
    float y[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) y[q] = xv[q];
    const int c0 = 8 * L;
    if (c0 < rd) {
      if ((half & 7) == 0) {  // the lane's 8 dims lie on one side of half: 16-byte LDS reads
        const bool lo = c0 < half;
        const float* pp = &xn[lo ? c0 + half : c0 - half];
        const f32x4_t p[2] = {*reinterpret_cast<const f32x4_t*>(pp),
                              *reinterpret_cast<const f32x4_t*>(pp + 4)};
        const f32x4_t* ep = reinterpret_cast<const f32x4_t*>(&cst[r][lo ? c0 : c0 - half]);
        const f32x4_t e[4] = {ep[0], ep[1], ep[2], ep[3]};  // (cos, sin) of 8 frequencies
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const float rot = lo ? -p[q >> 2][q & 3] : p[q >> 2][q & 3];  // rotate_half
          const float cs = e[q >> 1][2 * (q & 1)], sn = e[q >> 1][2 * (q & 1) + 1];
          y[q] = round_bf16(round_bf16(xv[q] * cs) + round_bf16(rot * sn));
        }
      } else {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const int c = c0 + q;
          if (c < rd) {
            const float rot = c < half ? -xn[c + half] : xn[c - half];  // rotate_half
            const float2 e = cst[r][c < half ? c : c - half];
            y[q] = round_bf16(round_bf16(xv[q] * e.x) + round_bf16(rot * e.y));
          }
        }
      }
    }
    u32x4_t yo;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      yo[i] = (uint32_t)__builtin_bit_cast(uint16_t, f32_to_bf16(y[2 * i])) |
              ((uint32_t)__builtin_bit_cast(uint16_t, f32_to_bf16(y[2 * i + 1])) << 16);
    if (is_q) {
      *reinterpret_cast<u32x4_t*>(q_out + (size_t)t * Hq * HD + (size_t)h * HD + 8 * L) = yo;
    } else if (pos >= 0 && pos < max_len) {  // never write outside the cache
      const size_t dst = ((size_t)h * max_len + pos) * HD + 8 * L;
      if constexpr (FP8) {
        uint32_t kw[2], vw[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          kw[i] = 0u;
          vw[i] = 0u;
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            const int q = 4 * i + b;
            const float vf = q & 1 ? hi_bf16(vr[r][q >> 1]) : lo_bf16(vr[r][q >> 1]);
            kw[i] |= (uint32_t)f32_to_fp8(round_bf16(y[q]) * k_inv) << (8 * b);
            vw[i] |= (uint32_t)f32_to_fp8(vf * v_inv) << (8 * b);
          }
        }
        *reinterpret_cast<uint2*>(static_cast<uint8_t*>(kc) + dst) = make_uint2(kw[0], kw[1]);
        *reinterpret_cast<uint2*>(static_cast<uint8_t*>(vc) + dst) = make_uint2(vw[0], vw[1]);
      } else {
        *reinterpret_cast<u32x4_t*>(static_cast<__bf16*>(kc) + dst) = yo;
        *reinterpret_cast<u32x4_t*>(static_cast<__bf16*>(vc) + dst) = vr[r];
      }
    }
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
  // Decode calls (<= 8 rows): one row per workgroup (the rows kernel measured 4.1 against 2.5 us
  // at 1 and 5 rows: its rotary table and barrier sit on a one-row call's critical path).
  // Chunks with 16-byte aligned rows: attn_prep_rows_kernel; otherwise 8 rows per workgroup.
  const auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (n > 8 && a16(qg) && a16(k) && a16(v) && a16(qnw) && a16(knw) && a16(q_out) && a16(kc) &&
      a16(vc) && ldp % 8 == 0) {
    constexpr int R = 2;  // rows per half-wave (2048 rows: 1 / 2 / 3 / 4 measured 18.9 / 18.4 /
                          // 19.3 / 19.1 us)
    const unsigned wpr = (Hq + Hkv + 7) / 8;  // workgroups per row group
    attn_prep_rows_kernel<FP8, R><<<dim3((n + R - 1) / R * wpr), dim3(HD), 0, stream>>>(
        QG, K, V, ldp, QW, KW, inv_freq, pos, QO, kc, vc, n, Hq, Hkv, max_len, rd, eps, k_inv,
        v_inv);
    return;
  }
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
