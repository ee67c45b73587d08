/* BF16 GEMV for 1..8 activation rows on gfx950 (MI355X): the projections on either side of the
 * gated-attention path (in_proj feeding qe_attn_prep, o_proj after qe_attn_decode), plus a
 * streaming-read probe used to report achievable HBM bandwidth.
 *
 * Device pointers, element strides; every entry point enqueues on `stream`, allocates nothing,
 * never synchronises and returns hipErrorInvalidValue (before any launch) for unsupported
 * arguments. */
#ifndef QE_GEMV_H
#define QE_GEMV_H

#include <stddef.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* out[r][n] = bf16(sum_k W[n][k] * x[r][k]) for r < nr, n < N: W [N][K] bf16 row-major
 * (contiguous), x rows [nr][ldx] bf16, out rows [nr][ldo] bf16, fp32 accumulation. Row r is
 * bit-identical to a 1-row call on x[r]; NaN in x[r] reaches every out[r][n].
 * Valid: 1 <= nr <= 8, N >= 1, K >= 8, K % 8 == 0, ldx >= K, ldx % 8 == 0, ldo >= N,
 * 16-byte aligned W and x, 32*K < 2^32, 2*((nr-1)*ldx + K) < 2^32.
 * Replaces launch_gemv_bf16 (reference csrc/ops.h:10-11, csrc/basic.cu:346-356). */
hipError_t qe_gemv_bf16(const void* W, const void* x, void* out, int nr, int N, int K, long ldx,
                        long ldo, hipStream_t stream);

/* k-parts per 16-row tile qe_gemv_bf16 uses for an [N][K] weight (1, 2 or 4; 0 if invalid):
 * the partial sums of a tile are added in order 0..parts-1. No counterpart in the reference. */
int qe_gemv_kparts(int N, int K);

/* Rows of W per tile qe_gemv_bf16 uses for an [N][K] weight on the current device (16, 14, 12
 * or 10; 0 if invalid): 16 unless the grid has one tile per workgroup (4 k-parts) and at most 4
 * workgroups per compute unit, then the height whose grid best fills its last round over the
 * compute units (5120 x 6144: 10, 512 workgroups; 14336 x 5120: 14, 1024 workgroups on 256
 * CUs). Outputs do not depend on it bit for bit. No counterpart in the reference. */
int qe_gemv_tile_rows(int N, int K);

/* Reads `bytes` (a multiple of 16) from 16-byte aligned device memory `buf` once with 16-byte
 * non-temporal loads, one contiguous range per workgroup over 2048 workgroups, to measure
 * achievable streaming-read bandwidth;
 * writes nothing to `sink` (4 bytes of device memory) in practice. Measurement only: no
 * counterpart in the reference (its HBM probe is bench/membw/membw.cu:1-25). */
hipError_t qe_hbm_read_probe(const void* buf, size_t bytes, void* sink, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* QE_GEMV_H */
