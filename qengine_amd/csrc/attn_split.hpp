// Split-KV slicing shared by the decode partials and the combine (attn_decode.hip,
// attn_combine.hip): the slice size of a row, the host-side division by NS, and the combine's
// launcher.
#pragma once
#include "qe_device.hpp"

namespace qe {

constexpr int TILE = 32;  // cache positions per wave step (two 16-row MFMA tiles)
// rows of one decode call: the combine's grid has one y index per row (at most 65535)
constexpr int MAX_DECODE_ROWS = 65535;

// Division by NS as a multiply and a shift, computed once on the host (Granlund & Montgomery,
// "Division by invariant integers using multiplication", 1994, Thm 4.2): with l = ceil(log2 NS)
// and m = floor(2^(23+l) / NS) + 1, floor(a / NS) == (a * m) >> (23 + l) for 0 <= a < 2^23.
// Cache lengths stay below 2^23 (the 32-bit buffer range), so every slicing division is exact;
// the kernels do it in a few scalar instructions instead of a reciprocal-based division.
struct NsDiv {
  uint32_t m;
  int sh;
};
inline NsDiv ns_div(int NS) {
  int l = 0;
  while ((1ll << l) < NS) ++l;
  return NsDiv{(uint32_t)((1ull << (23 + l)) / (unsigned long long)NS + 1), 23 + l};
}
constexpr int SPLIT_L_MAX = 1 << 23;  // split_size's range for L

// Slice size for a row attending L positions (1 <= L < 2^23): ceil(L/NS) rounded up to whole
// tiles.
__host__ __device__ inline int split_size(int L, NsDiv d) {
  if (L < 1) return TILE;
  const uint32_t per = (uint32_t)(((unsigned long long)(uint32_t)(L - 1) * d.m) >> d.sh) + 1u;
  return (int)((per + TILE - 1) / TILE * TILE);
}

// Log-sum-exp merge of the slices + fused sigmoid output gate (attn_combine.hip). v_scale
// multiplies O / L before its bf16 rounding (the fp8 cache's V scale; exactly 1 otherwise).
hipError_t launch_combine(const float* part_o, const float* part_ml, const int* pos,
                          const void* qg, long ldp, void* out, long ldo, int n, int Hq,
                          int max_len, int NS, hipStream_t stream, float v_scale = 1.f);

}  // namespace qe
