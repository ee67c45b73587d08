// BF16 GEMV (gemv.hip, gemv_lds.hip): the ring's shape, shared by the two kernels, and the
// launcher of the LDS-staged kernel for 1-2 activation rows.
#pragma once
#include "qe_device.hpp"

namespace qe {

constexpr int GEMV_WAVES = 4;
constexpr int GEMV_STG = 2;       // ring stages per wave
constexpr int GEMV_KB = 256;      // k per block (one stage)
constexpr int GEMV_W_SLOTS = 16 * (GEMV_KB / 8);  // 16-byte slots of a W block: 512

template <int XI>
constexpr int gemv_stage_slots() { return GEMV_W_SLOTS + 64 * XI; }
template <int XI>
constexpr size_t gemv_lds_bytes() {
  return (size_t)GEMV_WAVES * GEMV_STG * gemv_stage_slots<XI>() * 16;
}

// gemv_bf16_kernel<S, XI> for nr <= 2 * XI activation rows, S k-parts (gemv_lds.hip).
hipError_t launch_gemv_lds(int S, int XI, const __bf16* W, const __bf16* x, __bf16* out, int nr,
                           int N, int K, long ldx, long ldo, hipStream_t stream);

}  // namespace qe
