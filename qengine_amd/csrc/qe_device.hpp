// Device helpers shared by the gfx950 attention kernels: bf16 rounding, wave64 reductions,
// buffer-resource loads and the MFMA operand types.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qe {

constexpr int HD = 256;      // head_dim (fixed, as in the reference: csrc/attn.cu:15)
constexpr int WAVE = 64;     // CDNA wavefront

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------- bf16 rounding
// torch rounds every bf16 op result to nearest-even; these model one such rounding.
__device__ __forceinline__ float bf16_to_f32(__bf16 x) { return static_cast<float>(x); }
__device__ __forceinline__ __bf16 f32_to_bf16(float x) { return static_cast<__bf16>(x); }
__device__ __forceinline__ float round_bf16(float x) { return bf16_to_f32(f32_to_bf16(x)); }

// The high/low bf16 of a packed dword as fp32 (exact).
__device__ __forceinline__ float lo_bf16(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float hi_bf16(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }

// Pack two fp32 into a dword of two bf16 (round to nearest even): a -> low half, b -> high. One
// v_cvt_pk_bf16_f32 on gfx950 (two scalar conversions would need a shift and an or on top).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}

// dword made of the low halves (sel_hi = false) or high halves (true) of x (-> low) and y (-> high)
__device__ __forceinline__ uint32_t interleave_halves(uint32_t x, uint32_t y, bool sel_hi) {
  return __builtin_amdgcn_perm(y, x, sel_hi ? 0x07060302u : 0x05040100u);
}

// sigmoid in fp32, as torch.sigmoid evaluates a bf16 input before rounding the result.
__device__ __forceinline__ float sigmoid_f32(float x) { return 1.0f / (1.0f + expf(-x)); }

// ---------------------------------------------------------------------------- reductions
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// wave_sum with the same pairing (xor 32, 16, 8, 4, 2, 1; each level adds the partner lane's
// value) on VALU lane moves instead of LDS-crossbar permutes, so it returns the same bits at a
// fraction of the latency: xor 32/16 by the gfx950 permlane swaps, xor 8 by DPP row_ror:8, xor 4
// by DPP row_half_mirror then quad_perm [3,2,1,0], xor 2 and 1 by DPP quad_perm.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __uint_as_float(__builtin_amdgcn_mov_dpp(__float_as_uint(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float wave_sum_fast(float v) {
  auto p32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(p32[0]) + __uint_as_float(p32[1]);
  auto p16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(p16[0]) + __uint_as_float(p16[1]);
  v = v + dpp<0x128>(v);              // row_ror:8 = lane ^ 8 within 16
  v = v + dpp<0x1B>(dpp<0x141>(v));   // row_half_mirror, then quad_perm [3,2,1,0]: lane ^ 4
  v = v + dpp<0x4E>(v);               // quad_perm [2,3,0,1]: lane ^ 2
  return v + dpp<0xB1>(v);            // quad_perm [1,0,3,2]: lane ^ 1
}

// Max / sum across the four 16-lane groups of a wave (lanes l, l^16, l^32, l^48) with the gfx950
// VALU lane swaps instead of an LDS-crossbar permute. permlane16_swap(v, v) returns, per lane,
// the values of 16-lane rows (0,0,2,2) and (1,1,3,3); permlane32_swap(v, v) returns the low and
// the high 32 lanes. Combining the pair is the xor-16 (then xor-32) butterfly, and the lower
// row's value is always the first operand, so every lane computes the same sum bit for bit.
__device__ __forceinline__ float xor16_pair(float v, bool sum) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  const float a = __uint_as_float(p[0]), b = __uint_as_float(p[1]);
  return sum ? a + b : fmaxf(a, b);
}
__device__ __forceinline__ float xor32_pair(float v, bool sum) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  const float a = __uint_as_float(p[0]), b = __uint_as_float(p[1]);
  return sum ? a + b : fmaxf(a, b);
}
__device__ __forceinline__ float group4_max(float v) { return xor32_pair(xor16_pair(v, false), false); }
__device__ __forceinline__ float group4_sum(float v) { return xor32_pair(xor16_pair(v, true), true); }

// ---------------------------------------------------------------------------- q/k prep
// RMSNorm1p + partial rotate-half RoPE of one 256-dim row with a 256-thread workgroup, thread c
// owning dim c (reference csrc/attn.cu:37-49, python/qengine/reference.py:132-136,158-176):
// y = bf16(bf16(xn*cos) + bf16(rot(xn)*sin)) on dims < rd, xn = bf16(x * rsqrt(mean x^2 + eps) *
// (1 + w)); cos/sin of the fp32 angle pos*inv_freq rounded to bf16. Shared by the prep kernel and
// the fused prep + decode kernel, so both produce the same bits.

// cos/sin of thread c's rotary angle at position pos ({1, 0} for dims >= rd). Evaluated in fp64
// from the fp32 angle and rounded once: the correctly rounded fp32 value, which is what the
// reference's fp32 cos/sin return in all but rare cases (single-precision device cos/sin can be a
// couple of ulps off, enough to flip a bf16 rounding).
struct RopeCS {
  float cs, sn;
};
// Thread c's rotary frequency (0 for dims >= rd).
__device__ __forceinline__ float rope_freq(const float* __restrict__ inv_freq, int rd, int c) {
  const int half = rd >> 1;
  return c < rd ? inv_freq[c < half ? c : c - half] : 0.f;
}
__device__ __forceinline__ RopeCS rope_cs_f(int pos, float freq, int rd, int c) {
  if (c >= rd) return {1.f, 0.f};
  const double angd = (double)((float)pos * freq);  // the fp32 angle, in fp64
  double sn, cs;
  sincos(angd, &sn, &cs);  // one argument reduction for both
  return {round_bf16((float)cs), round_bf16((float)sn)};
}
__device__ __forceinline__ RopeCS rope_cs(int pos, const float* __restrict__ inv_freq, int rd,
                                          int c) {
  return rope_cs_f(pos, rope_freq(inv_freq, rd, c), rd, c);
}

// Workgroup barrier for LDS data only: this wave's LDS writes have landed (lgkmcnt(0)), then
// s_barrier between compiler fences. Outstanding global loads stay in flight (unlike
// __syncthreads(), whose release waits for every vector-memory operation).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt at their maxima
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The sum of squares is a wave64 butterfly plus a fixed-order sum of the four wave partials. xn
// (256 floats) and red (4 floats) are LDS scratch. Contains two workgroup barriers (LDS only):
// every thread of the workgroup calls it, the same number of times.
__device__ __forceinline__ float prep_dim(float x, float wgt, RopeCS r, int rd, float eps,
                                          float* xn, float* red) {
  const int c = threadIdx.x;
  const float sq = wave_sum_fast(x * x);
  if ((c & (WAVE - 1)) == 0) red[c / WAVE] = sq;
  lds_barrier();
  const float total = ((red[0] + red[1]) + red[2]) + red[3];
  const float inv = 1.0f / sqrtf(total / (float)HD + eps);
  const float xv = round_bf16((x * inv) * (1.0f + wgt));  // RMSNorm1p output is a bf16 tensor
  xn[c] = xv;
  lds_barrier();
  if (c >= rd) return xv;
  const int half = rd >> 1;
  const float rot = c < half ? -xn[c + half] : xn[c - half];  // rotate_half
  return round_bf16(round_bf16(xv * r.cs) + round_bf16(rot * r.sn));
}

// ---------------------------------------------------------------------------- buffer loads
// Raw buffer resource over [base, base + bytes). Loads whose dword lies past `bytes` return 0
// (no fault), which the kernels use to zero-fill positions beyond the attended range.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}
// The same for a base and size that are wave-uniform where the compiler cannot prove it (values
// merged across branches): readfirstlane keeps the resource in SGPRs, since a resource in VGPRs
// turns every buffer load into a waterfall loop.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc_uniform(const void* base,
                                                                    uint32_t bytes) {
  // readfirstlane returns int: go through uint32_t so the low half is zero-extended, not
  // sign-extended into the high half.
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32));
  return make_rsrc(reinterpret_cast<const void*>(((uint64_t)hi << 32) | (uint64_t)lo),
                   (uint32_t)__builtin_amdgcn_readfirstlane((int)bytes));
}
__device__ __forceinline__ u32x4_t buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(u32x4_t,
                            __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_off, 0, 0));
}
// Same, with the non-temporal hint (cache policy NT): data read exactly once, such as the KV
// cache in decode. Measured on MI355X: ~7.2 TB/s streaming reads vs ~6.4 TB/s without it.
constexpr int CPOL_NT = 2;
__device__ __forceinline__ u32x4_t buffer_load16_stream(__amdgpu_buffer_rsrc_t r,
                                                        uint32_t byte_off) {
  return __builtin_bit_cast(
      u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_off, 0, CPOL_NT));
}

// 8 bytes (non-temporal), e.g. eight fp8 cache values.
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ u32x2_t buffer_load8_stream(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(
      u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(r, (int)byte_off, 0, CPOL_NT));
}

// ---------------------------------------------------------------------------- fp8 (OCP E4M3FN)
// The fp8 KV cache stores E4M3FN codes (1 sign, 4 exponent bits with bias 7, 3 mantissa bits;
// S.1111.111 is NaN; largest finite 448). gfx950's v_cvt_pk_f32_fp8 decodes this format
// (checked for all 256 codes on MI355X) and v_cvt_pk_fp8_f32 encodes it with round-to-nearest-
// even and no saturation (|x| >= 480 becomes NaN), so the encoder clamps to +-448 first.

// Eight fp8 codes (little-endian in w) -> eight bf16 (as 4 packed pairs). Every E4M3 value is a
// bf16 value, so the conversion is exact. gfx950's v_cvt_scalef32_pk_bf16_fp8 with scale 1 does
// a pair in one instruction; it gives the same bits as v_cvt_pk_f32_fp8 followed by keeping the
// upper half of each fp32 for all 65,536 code pairs in both halves of the word, NaN codes
// included (checked on MI355X).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t fp8x2_to_bf16x2_lo(uint32_t w) {  // codes in bytes 0, 1
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false));
}
__device__ __forceinline__ uint32_t fp8x2_to_bf16x2_hi(uint32_t w) {  // codes in bytes 2, 3
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true));
}
__device__ __forceinline__ u32x4_t fp8x8_to_bf16x8(u32x2_t w) {
  return u32x4_t{fp8x2_to_bf16x2_lo(w[0]), fp8x2_to_bf16x2_hi(w[0]), fp8x2_to_bf16x2_lo(w[1]),
                 fp8x2_to_bf16x2_hi(w[1])};
}

// A usable per-cache scale: a normal, finite fp32 value (NaN fails both comparisons). Subnormal
// scales are rejected because their fp32 reciprocal, the encoder's multiplier, overflows to inf,
// which would turn zero inputs into NaN codes.
__host__ __device__ inline bool kv_scale_ok(float s) {
  return s >= 1.17549435e-38f && s <= 3.40282347e38f;
}

// x -> fp8 code: round to nearest even, saturate at +-448, NaN stays NaN.
__device__ __forceinline__ uint8_t f32_to_fp8(float x) {
  const float c = x != x ? x : fminf(fmaxf(x, -448.0f), 448.0f);
  return (uint8_t)(__builtin_amdgcn_cvt_pk_fp8_f32(c, 0.0f, 0, false) & 0xff);
}

// 16 bytes per lane from a buffer straight into LDS (gfx950 LDS DMA, non-temporal): lane i of the
// wave writes lds_base + 16*i. lds_base must be wave-uniform. The compiler does not order later
// LDS reads after this write: wait with vmcnt_wait() first.
// CPOL selects the cache policy: CPOL_NT for data read once (decode's KV stream), 0 for data that
// other workgroups read again soon (prefill's K/V tiles).
template <int CPOL = CPOL_NT>
__device__ __forceinline__ void buffer_load16_to_lds(__amdgpu_buffer_rsrc_t r, uint32_t byte_off,
                                                     void* lds_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      r, (__attribute__((address_space(3))) void*)lds_base, 16, (int)byte_off, 0, 0, CPOL);
}
// The same with the LDS destination as a byte address held in scalar registers (M0 is then set
// by scalar moves, not a readfirstlane per load).
__device__ __forceinline__ void buffer_load16_to_lds_at(__amdgpu_buffer_rsrc_t r,
                                                        uint32_t byte_off, uint32_t lds_byte) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      r, (__attribute__((address_space(3))) void*)(uintptr_t)lds_byte, 16, (int)byte_off, 0, 0,
      CPOL_NT);
}
// LDS byte address of an LDS pointer, made wave-uniform (readfirstlane) so the compiler keeps
// it, and the addresses derived from it, in scalar registers.
__device__ __forceinline__ uint32_t lds_byte_uniform(const void* p) {
  return (uint32_t)__builtin_amdgcn_readfirstlane(
      (int)(uint32_t)(uintptr_t)((__attribute__((address_space(3))) const char*)p));
}

// s_waitcnt vmcnt(N): at most N vector-memory loads of this wave still outstanding (gfx9
// encoding: vmcnt low bits [3:0], high bits [15:14]; expcnt and lgkmcnt left at their maxima).
template <int N>
__device__ __forceinline__ void vmcnt_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier for a ring of LDS-DMA stages: s_barrier between compiler-only fences (LDS
// accesses are not moved across it) but without the hardware waits of __syncthreads(), whose
// workgroup-scope release drains every outstanding LDS-DMA load. The caller has already waited
// (vmcnt) for the DMA loads that the other waves must see; its own earlier LDS reads have
// completed because their results were consumed.
__device__ __forceinline__ void barrier_no_drain() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4_t v) { return __builtin_bit_cast(bf16x8_t, v); }

// D = A(16x32) * B(32x16) + C on bf16 inputs with fp32 accumulation. Lane l holds A row l%16 /
// B column l%16 at k = 8*(l/16)+e, and D rows 4*(l/16)+i of column l%16.
__device__ __forceinline__ f32x4_t mfma16x16x32(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

}  // namespace qe
