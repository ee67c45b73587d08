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
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------- bf16 rounding
// torch rounds every bf16 op result to nearest-even; these model one such rounding.
__device__ __forceinline__ float bf16_to_f32(__bf16 x) { return static_cast<float>(x); }
__device__ __forceinline__ __bf16 f32_to_bf16(float x) { return static_cast<__bf16>(x); }
__device__ __forceinline__ float round_bf16(float x) { return bf16_to_f32(f32_to_bf16(x)); }

// The high/low bf16 of a packed dword as fp32 (exact).
__device__ __forceinline__ float lo_bf16(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float hi_bf16(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }

// Pack two fp32 into a dword of two bf16 (round to nearest even): a -> low half, b -> high.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  const uint32_t lo = __builtin_bit_cast(uint16_t, f32_to_bf16(a));
  const uint32_t hi = __builtin_bit_cast(uint16_t, f32_to_bf16(b));
  return lo | (hi << 16);
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

// ---------------------------------------------------------------------------- buffer loads
// Raw buffer resource over [base, base + bytes). Loads whose dword lies past `bytes` return 0
// (no fault), which the kernels use to zero-fill positions beyond the attended range.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
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
