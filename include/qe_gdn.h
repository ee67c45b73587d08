/* Gated DeltaNet decode / verify step on gfx950 (MI355X): the recurrent layer of the hybrid model
 * (48 of its 64 layers), n = 1..8 new rows per call with lazy rollback.
 *
 * Device pointers, element row strides; the entry point enqueues on `stream`, allocates nothing,
 * never synchronises, and returns hipErrorInvalidValue (before any launch) for unsupported
 * arguments. Row r of an n-row call is computed exactly as a 1-row call, and replaying kept rows
 * uses the same arithmetic as computing them, so any pattern of calls with kept prefixes leaves
 * the state and outputs of plain one-row decoding, bit for bit. */
#ifndef QE_GDN_H
#define QE_GDN_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* One call of a Gated DeltaNet layer (dk = dv = 128; C = 2 Hk 128 + Hv 128 conv channels).
 *   qkv, z, b, a   rows [n][ldp] bf16: the layer's input projections (widths C, Hv*128, Hv, Hv)
 *   ring           [16][C] bf16 conv history, slot = position & 15 (zero it for a new sequence)
 *   conv_w [C][4], A_log [Hv], dt_bias [Hv], norm_w [128]: bf16 layer weights
 *   S              [Hv][128][128] fp32 committed state (16-byte aligned)
 *   st_k, st_v     [8][Hv][128] fp32, st_g [8][Hv][2] fp32: rows staged by the previous call
 *   ctl            int32: ctl[0] = pos (position of row 0), ctl[1] = pending (rows of the previous
 *                  call to replay first; values outside [0, 8] are clamped)
 *   out            rows [n][ldo] bf16, width Hv*128
 * Per row: causal conv + SiLU, gates beta = sigmoid(b), decay = exp(-exp(A_log) softplus(a +
 * dt_bias)), l2norm q / sqrt(128) and k, S = decay S, S += k (beta (v - S^T k))^T, o = S^T q,
 * out = bf16(w * bf16(norm(o))) * silu(z). The call replays `pending` staged rows into S (and
 * writes S), runs its n rows on a copy, stages them, and writes the ring slots pos .. pos+n-1.
 * The caller then sets pos += kept, pending = kept.
 * Valid: 1 <= n <= 8, Hk >= 1, Hv % Hk == 0, Hv <= 65535, C < 2^26, ldp >= C, ldo >= Hv*128.
 * A call touches no memory but its arguments, so calls on different layers (different state,
 * ring, staging and output buffers) may run concurrently on any streams; calls that share those
 * buffers must be ordered, as in the reference. 5-8 rows run as two launches (each head split over
 * 4 workgroups, then a per-head finish); no workgroup waits for another.
 * Replaces launch_gdn_step_n (reference csrc/ops.h:20-23, csrc/gdn.cu:65-341). The reference's
 * thread-split argument `q` selects a CUDA block shape; it has no counterpart here. */
hipError_t qe_gdn_step_n(const void* qkv, const void* z, const void* b, const void* a, long ldp,
                         void* ring, const void* conv_w, const void* A_log, const void* dt_bias,
                         const void* norm_w, float* S, float* st_k, float* st_v, float* st_g,
                         const int* ctl, void* out, long ldo, int n, int Hk, int Hv, float eps,
                         hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* QE_GDN_H */
