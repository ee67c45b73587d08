// BF16 GEMV, the LDS-staged kernel for 1-2 activation rows (gemv_bf16_kernel; the design is
// described at the top of gemv.hip). This file is compiled with LLVM's max-ILP machine scheduler;
// the register-activation kernel for 3-8 rows (gemv.hip) keeps the default. Same-box A/B of the
// whole GEMV source under max-ILP, us per call: 1 row in_proj 25.22 -> 24.72, o_proj 14.40 ->
// 13.99; 5 rows in_proj 27.34 -> 27.89, o_proj 15.97 -> 16.34. Same bits.
#include <type_traits>

#include "gemv_common.hpp"

namespace qe {

// XI: LDS-DMA instructions of activation rows per block (two rows each, nr <= 2 * XI). RPT: rows
// of W per tile (even, 10..16); MFMA rows RPT..15 of a shorter tile multiply zeros.
template <int S, int XI, int RPT>
__global__ void __launch_bounds__(GEMV_WAVES * WAVE)
gemv_bf16_kernel(const __bf16* __restrict__ W, const __bf16* __restrict__ x,
                 __bf16* __restrict__ out, int nr, int N, int K, long ldx, long ldo) {
  constexpr int RT = GEMV_WAVES / S;  // row tiles per workgroup
  constexpr int WSL = gemv_w_slots<RPT>();
  constexpr int SLOTS = gemv_stage_slots<XI, RPT>();
  constexpr int LPS = RPT / 2 + XI;  // loads per stage
  extern __shared__ __attribute__((aligned(16))) u32x4_t gemv_smem[];
  const int lane = threadIdx.x & (WAVE - 1);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const int i = lane & 15, g4 = lane >> 4;
  const int tile = blockIdx.x * RT + w / S, kp = w % S;
  const int r0 = tile * RPT;
  // A tile past N (only in the last workgroup) loads nothing but still meets the barrier below.
  const bool live = r0 < N;

  const int K8 = K >> 3;                              // 16-byte chunks per row
  const int nblk = (K + GEMV_KB - 1) / GEMV_KB;       // 256-k blocks per row (last may be partial)
  const int b_beg = kp * nblk / S, b_end = live ? (kp + 1) * nblk / S : b_beg;
  const uint32_t tile_bytes = live ? (uint32_t)min(RPT, N - r0) * (uint32_t)K * 2u : 0u;
  const __amdgpu_buffer_rsrc_t wrs = make_rsrc_uniform(W + (size_t)r0 * K, tile_bytes);
  const __amdgpu_buffer_rsrc_t xrs =
      make_rsrc_uniform(x, (uint32_t)(((size_t)(nr - 1) * ldx + K) * 2));
  u32x4_t* ring = gemv_smem + (size_t)w * GEMV_STG * SLOTS;

  // Slot (r, q) of a stage holds chunk q ^ (r & 15) of row r; rows and chunks past the matrix
  // read 0 (buffer bounds) or are zeroed at use (chunks past K in a partial last block).
  auto issue = [&](int blk, int st) {
    u32x4_t* sb = ring + st * SLOTS;
#pragma unroll
    for (int j = 0; j < RPT / 2; ++j) {
      const int r = 2 * j + (lane >> 5), q = lane & 31;
      buffer_load16_to_lds(wrs, (uint32_t)r * (uint32_t)K * 2u +
                                    (uint32_t)(blk * GEMV_KB + (q ^ (r & 15)) * 8) * 2u,
                           sb + 64 * j);
    }
#pragma unroll
    for (int j = 0; j < XI; ++j) {
      const int c = 2 * j + (lane >> 5), q = lane & 31;
      const int cr = c < nr ? c : nr - 1;
      buffer_load16_to_lds<0>(xrs, (uint32_t)(cr * ldx + blk * GEMV_KB + (q ^ (c & 15)) * 8) * 2u,
                              sb + WSL + 64 * j);
    }
  };

  const bool xok = i < nr;
  const bool aok = RPT == 16 || i < RPT;  // this lane's W row is part of the tile
  const int xr = i < 2 * XI ? i : 2 * XI - 1;  // staged activation row this lane reads
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  const int nb = b_end - b_beg;
  if (nb > 0) issue(b_beg, 0);
  for (int t = 0; t < nb; ++t) {
    // the next block goes in flight before this one is waited for
    if (t + 1 < nb) {
      issue(b_beg + t + 1, (t + 1) % GEMV_STG);
      vmcnt_wait<LPS>();
    } else {
      vmcnt_wait<0>();
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
    const u32x4_t* sb = ring + (t % GEMV_STG) * SLOTS;
    const int cbase = (b_beg + t) * (GEMV_KB / 8);    // first chunk of this block
#pragma unroll
    for (int ks = 0; ks < GEMV_KB / 32; ++ks) {
      const int q = 4 * ks + g4;
      const bool ok = cbase + q < K8;
      const u32x4_t z = {0u, 0u, 0u, 0u};
      const u32x4_t a = sb[(aok ? i : 0) * 32 + (q ^ i)];
      const u32x4_t b = sb[WSL + xr * 32 + (q ^ xr)];
      acc = mfma16x16x32(as_bf16x8(ok && aok ? a : z), as_bf16x8(ok && xok ? b : z), acc);
    }
    // this stage's LDS reads are complete (their values fed the MFMAs) before the DMA that
    // refills it is issued in the next iteration
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
  }

  if constexpr (S > 1) {
    __shared__ f32x4_t red[GEMV_WAVES][WAVE];
    red[w][lane] = acc;
    __syncthreads();
    if (kp != 0) return;
#pragma unroll
    for (int v = 1; v < S; ++v) acc += red[w + v][lane];  // ((p0 + p1) + p2) + ...
  }
  // lane (g4, c = i) holds out^T rows r0 + 4g4 + j, column c
  if (i < nr) {
    __bf16* op = out + (size_t)i * ldo;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = r0 + 4 * g4 + j;
      if (4 * g4 + j < RPT && row < N) op[row] = f32_to_bf16(acc[j]);
    }
  }
}

template <int S, int XI, int RPT>
static hipError_t launch_gemv(const __bf16* W, const __bf16* x, __bf16* out, int nr, int N,
                              int K, long ldx, long ldo, hipStream_t stream) {
  constexpr int RT = GEMV_WAVES / S;
  constexpr size_t lds = gemv_lds_bytes<XI, RPT>();
  // above 64 KB of dynamic LDS a kernel must opt in; once per instantiation and process (a
  // function attribute, not stream work, so it is also legal under graph capture)
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&gemv_bf16_kernel<S, XI, RPT>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (attr != hipSuccess) return attr;
  const int tiles = (N + RPT - 1) / RPT;
  gemv_bf16_kernel<S, XI, RPT><<<dim3((tiles + RT - 1) / RT), dim3(GEMV_WAVES * WAVE), lds, stream>>>(
      W, x, out, nr, N, K, ldx, ldo);
  return hipGetLastError();
}

hipError_t launch_gemv_lds(int S, int XI, int RPT, const __bf16* W, const __bf16* x, __bf16* out,
                           int nr, int N, int K, long ldx, long ldo, hipStream_t stream) {
  auto by_s = [&](auto xi) {
    constexpr int X = decltype(xi)::value;
    switch (S) {
      case 1: return launch_gemv<1, X, 16>(W, x, out, nr, N, K, ldx, ldo, stream);
      case 2: return launch_gemv<2, X, 16>(W, x, out, nr, N, K, ldx, ldo, stream);
      default:
        switch (RPT) {
          case 10: return launch_gemv<4, X, 10>(W, x, out, nr, N, K, ldx, ldo, stream);
          case 12: return launch_gemv<4, X, 12>(W, x, out, nr, N, K, ldx, ldo, stream);
          case 14: return launch_gemv<4, X, 14>(W, x, out, nr, N, K, ldx, ldo, stream);
          default: return launch_gemv<4, X, 16>(W, x, out, nr, N, K, ldx, ldo, stream);
        }
    }
  };
  switch (XI) {
    case 1: return by_s(std::integral_constant<int, 1>{});
    case 2: return by_s(std::integral_constant<int, 2>{});
    case 3: return by_s(std::integral_constant<int, 3>{});
    default: return by_s(std::integral_constant<int, 4>{});
  }
}

}  // namespace qe
