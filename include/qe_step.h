/* The rest of one decode / verify step around the gated-attention path on gfx950 (MI355X):
 * embedding gather, RMSNorm1p (+ fused residual add), SwiGLU, per-row argmax, and the device-side
 * step bookkeeping (speculative accept, commit, MTP row select), so a whole step is one hipGraph.
 *
 * Device pointers, element row strides; every entry point enqueues on `stream`, allocates
 * nothing, never synchronises, and returns hipErrorInvalidValue (before any launch) for
 * unsupported arguments. Row r of an n-row call is computed exactly as a 1-row call. */
#ifndef QE_STEP_H
#define QE_STEP_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* out[r][:H] = table[tok[r]][:H] for r < n (table [V][H] bf16 contiguous, out rows [n][ldo]);
 * an id outside [0, V) gives a zero row. Valid: 1 <= n <= 65535, H >= 1, V >= 1, ldo >= H.
 * Replaces launch_embed (reference csrc/ops.h:6-7, csrc/basic.cu:16-26). */
hipError_t qe_embed(const void* table, const int* tok, void* out, int n, int H, int V, long ldo,
                    hipStream_t stream);

/* Per row: if delta, x = bf16(x + delta) (written back to x); then
 * out = bf16(x * rsqrt(mean(x^2) + eps) * (1 + w)) in fp32. x rows [rows][ldx], delta rows
 * [rows][ldd] or NULL, w [H], out rows [rows][ldo], bf16. Valid: rows >= 1, H >= 1, ldx, ldo
 * (and ldd with delta) >= H.
 * Replaces launch_rmsnorm1p (reference csrc/ops.h:8-9, csrc/basic.cu:34-97). */
hipError_t qe_rmsnorm1p(void* x, const void* delta, const void* w, void* out, int rows, int H,
                        long ldx, long ldd, long ldo, float eps, hipStream_t stream);

/* Per row: gu = [gate (I) | up (I)], out = bf16(bf16(silu(gate)) * up), silu in fp32.
 * Valid: 1 <= n <= 65535, I >= 1, ldg >= 2I, ldo >= I.
 * Replaces launch_swiglu (reference csrc/ops.h:12, csrc/basic.cu:160-170). */
hipError_t qe_swiglu(const void* gu, void* out, int n, int I, long ldg, long ldo,
                     hipStream_t stream);

/* out[r] = argmax(x[r][:n]) with torch semantics (NaN is the maximum, ties go to the lowest
 * index, a row of -inf gives 0); out[r] = idmap[argmax] when idmap is not NULL. pv (fp32) and pi
 * (int32) are caller workspaces of rows * nb entries (nb partial results per row; two launches).
 * Valid: 1 <= rows <= 65535, n >= 1, ldx >= n, nb >= 1.
 * Replaces launch_argmax (reference csrc/ops.h:13-14, csrc/basic.cu:176-239). */
hipError_t qe_argmax(const void* x, int rows, int n, long ldx, float* pv, int* pi, int nb,
                     int* out, const int* idmap, hipStream_t stream);

/* Speculative accept for a pass of n rows (int32 device buffers). ctl[0] = pos of in_tok[0],
 * ctl[2] = mode (1: verify, in_tok = [last token, drafts...]; else prefill). Sets ctl[3] = m, the
 * last kept row (verify: longest prefix with in_tok[i+1] == am[i]; prefill: n - 1), next_tok[r]
 * for r < n, logs generated tokens at their positions in log[0, max_len), and in verify mode
 * counts ctl[4] += 1, ctl[5] += m, ctl[16 + m] += 1. Needs in_tok > n entries, ctl >= 24.
 * Valid: 1 <= n <= 8, max_len >= 0.
 * Replaces launch_accept (reference csrc/ops.h:15-16, csrc/basic.cu:256-281). */
hipError_t qe_accept(const int* in_tok, const int* am, int n, int* ctl, int* next_tok, int* log,
                     int max_len, hipStream_t stream);

/* End of a pass: ctl[0] += m + 1, ctl[1] = m + 1 (m = ctl[3]), in_tok[0] = am[m],
 * in_tok[1 + j] = drafts[j] for j < k. Valid: k >= 0 (drafts may be NULL when k == 0).
 * Replaces launch_commit (reference csrc/ops.h:17, csrc/basic.cu:283-291). */
hipError_t qe_commit(int* ctl, int* in_tok, const int* am, const int* drafts, int k,
                     hipStream_t stream);

/* mpos[0] = off < 0 ? ctl[0] : ctl[0] + ctl[3] + 1 + off; if src: dst[:H] = src row ctl[3]
 * (rows [.][lds] bf16); if draft0: draft0[0] = mtp_am[ctl[3]].
 * Replaces launch_mtp_select (reference csrc/ops.h:18-19, csrc/basic.cu:295-307). */
hipError_t qe_mtp_select(const int* ctl, int* mpos, int off, const void* src, long lds, void* dst,
                         int H, const int* mtp_am, int* draft0, hipStream_t stream);

/* L2 persistence controls of the reference (an NVIDIA set-aside L2 window for the MTP weights).
 * MI355X exposes no persisting-cache control; its 256 MB Infinity Cache keeps recently used data
 * by itself. Both return hipSuccess and change nothing.
 * Replace l2_persist_limit and stream_access_window (reference csrc/ops.h:35-36,
 * csrc/basic.cu:384-398). */
hipError_t qe_l2_persist_limit(size_t bytes);
hipError_t qe_stream_access_window(uintptr_t base, size_t bytes, float hit_ratio,
                                   hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* QE_STEP_H */
