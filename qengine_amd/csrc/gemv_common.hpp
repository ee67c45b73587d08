// BF16 GEMV (gemv.hip, gemv_lds.hip): the ring's shape, shared by the two kernels, and the
// launcher of the LDS-staged kernel for 1-2 activation rows.
#pragma once
#include "qe_device.hpp"

namespace qe {

constexpr int GEMV_WAVES = 4;
constexpr int GEMV_STG = 2;       // ring stages per wave
constexpr int GEMV_KB = 256;      // k per block (one stage)
// 16-byte slots of one W block of an RPT-row tile (RPT even, 10..16): 32 per row
template <int RPT>
constexpr int gemv_w_slots() { return RPT * (GEMV_KB / 8); }
template <int XI, int RPT>
constexpr int gemv_stage_slots() { return gemv_w_slots<RPT>() + 64 * XI; }
template <int XI, int RPT>
constexpr size_t gemv_lds_bytes() {
  return (size_t)GEMV_WAVES * GEMV_STG * gemv_stage_slots<XI, RPT>() * 16;
}

// gemv_bf16_kernel<S, XI, RPT> for nr <= 2 * XI activation rows, S k-parts, RPT rows per W tile
// (gemv_lds.hip). RPT below 16 only with S = 4.
hipError_t launch_gemv_lds(int S, int XI, int RPT, const __bf16* W, const __bf16* x, __bf16* out,
                           int nr, int N, int K, long ldx, long ldo, hipStream_t stream);

}  // namespace qe
