/* qe_attn.h -- C ABI of the MI355X (gfx950) gated-attention decode path.
 *
 * Library: qengine_amd/libqe_attn.so (hand-written HIP kernels for gfx950 + this C ABI).
 * Every entry point takes raw device pointers, row strides in elements and a HIP stream. It
 * enqueues work on that stream and returns without a host sync. It allocates nothing, so calls
 * can be captured in a hipGraph. `pos` is a device int32 scalar (element 0 = position of row 0),
 * read on the device. Tensors are bf16 (`void*`) unless typed otherwise.
 *
 * Return value: hipSuccess, hipErrorInvalidValue for arguments outside the supported ranges
 * (checked on the host before any launch), or the launch error reported by the HIP runtime.
 *
 * Shapes (head_dim D = 256 is fixed, as in the reference):
 *   qg rows   [n][ldp]: per q head h, [q (D) | gate (D)]  -> row width Hq*2*D
 *   k, v rows [n][ldp]: Hkv*D each (same row stride as qg)
 *   q         [n][Hq*D] contiguous rows
 *   kc, vc    [Hkv][max_len][D] (KV cache, updated in place by qe_attn_prep)
 *   part_o    fp32 [>= n][Hq][NS][D], part_ml fp32 [>= n][Hq][NS][2]: caller-owned scratch
 *             whose contents are private to this library
 *   out rows  [n][ldo]: Hq*D
 * Concurrency: part_o/part_ml are scratch. Two calls that share them must not overlap (as in
 * the reference, where every layer reuses one pair).
 */
#ifndef QE_ATTN_H
#define QE_ATTN_H

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* q/k RMSNorm1p (eps, weights qnw/knw, one bf16 rounding) + partial rotate-half RoPE on the first
 * rd = 2*len(inv_freq) dims (fp32 angle pos*inv_freq, bf16 cos/sin, every op rounded to bf16).
 * Writes q_out[t], and kc/vc[h][pos+t] when 0 <= pos+t < max_len. Valid: 1 <= n <= 65535,
 * 0 <= rd <= 256, rd even.
 * Replaces launch_attn_prep (reference csrc/ops.h:25-27, csrc/attn.cu:157-163). */
hipError_t qe_attn_prep(const void* qg, const void* k, const void* v, long ldp, const void* qnw,
                        const void* knw, const float* inv_freq, const int* pos, void* q_out,
                        void* kc, void* vc, int n, int Hq, int Hkv, int max_len, int rd,
                        float eps, hipStream_t stream);

/* Gated flash-decoding: row t attends cache positions [0, min(pos+t+1, max_len)), scores scaled
 * by `scale`, and out[t] = bf16(bf16(softmax . V) * bf16(sigmoid(gate))), gate = qg[t][h][D:2D].
 * Two launches: split-KV partials, row t over slices of qe_attn_split_size(L_t, NS) positions
 * (L_t = min(pos+t+1, max_len), so about NS slices hold work whatever max_len is), then a
 * log-sum-exp combine with the fused sigmoid gate. Row t of an n-row call is bit-identical to a
 * 1-row call at position pos+t. Valid: 1 <= n <= 65535, Hq % Hkv == 0 (any group size),
 * NS >= 1, (max_len+32)*512 < 2^32, 16-byte aligned q/kc/vc/part_o. A call whose query
 * columns ((Hq/Hkv)*n) exceed one launch's 64 runs the partials as several launches (chunks of
 * min(8, 64/(Hq/Hkv)) rows; above 64 q heads per KV head, one row and at most 64 of its q heads
 * per launch), with the same bits.
 * Replaces launch_attn_decode (reference csrc/ops.h:28-30, csrc/attn.cu:165-172). */
hipError_t qe_attn_decode(const void* q, const void* kc, const void* vc, const int* pos,
                          const void* qg, long ldp, float* part_o, float* part_ml, void* out,
                          long ldo, int n, int Hq, int Hkv, int max_len, int NS, float scale,
                          hipStream_t stream);

/* qe_attn_prep followed by qe_attn_decode (same arguments; q_out is also the decode's q), in two
 * launches instead of three: the split-KV kernel computes its q rows and writes the new K/V
 * cache rows itself, then the combine runs. Every output (q_out, the written cache rows, out) is
 * bit-identical to the two calls in sequence. Valid: the union of both ops' ranges (1 <= n <=
 * 65535, ...); more than 8 rows or 16 columns ((Hq/Hkv)*n > 16) run the two ops.
 * No counterpart in the reference, which overlaps the two launches with programmatic dependent
 * launch instead (csrc/attn.cu:155, csrc/common.cuh:12-46; callers python/qengine/engine.py:455-458). */
hipError_t qe_attn_prep_decode(const void* qg, const void* k, const void* v, long ldp,
                               const void* qnw, const void* knw, const float* inv_freq,
                               const int* pos, void* q_out, void* kc, void* vc, float* part_o,
                               float* part_ml, void* out, long ldo, int n, int Hq, int Hkv,
                               int max_len, int rd, int NS, float scale, float eps,
                               hipStream_t stream);

/* First half of qe_attn_decode: the split-KV partials only (part_o/part_ml filled for the slices
 * that hold positions). The pair is exported separately so that a sequence-sharded caller can
 * exchange partials between devices before combining, and so the partials kernel can be timed
 * on its own. No counterpart in the reference (there the pair is one launcher,
 * csrc/attn.cu:165-172). */
hipError_t qe_attn_decode_partials(const void* q, const void* kc, const void* vc, const int* pos,
                                   float* part_o, float* part_ml, int n, int Hq, int Hkv,
                                   int max_len, int NS, float scale, hipStream_t stream);

/* qe_attn_decode without caller scratch: the same kernels and the same bits, with part_o /
 * part_ml in a file-scope device array of the library (QE_NOALLOC_MAX_SLOTS (row, head, slice)
 * triples: 12,288 x 258 fp32 = 12.7 MB, held on every GPU the library runs on until the process
 * ends). The call allocates nothing (no hipMalloc, hipFree or allocating library routine); on its
 * first call on a device it looks the array's address up once (hipGetSymbolAddress, with that
 * device current). Valid as qe_attn_decode, plus n*Hq*NS <= QE_NOALLOC_MAX_SLOTS
 * (hipErrorInvalidValue otherwise). Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (other streams, other host threads) race. Nothing in the array needs to
 * start at zero. No counterpart in the reference: for callers that cannot allocate device
 * memory (code under hipGraph capture, tight serving loops, harnesses that forbid hipMalloc). */
#define QE_NOALLOC_MAX_SLOTS 12288
hipError_t qe_attn_decode_noalloc(const void* q, const void* kc, const void* vc, const int* pos,
                                  const void* qg, long ldp, void* out, long ldo, int n, int Hq,
                                  int Hkv, int max_len, int NS, float scale, hipStream_t stream);

/* Second half of qe_attn_decode: log-sum-exp combine of the partials + sigmoid output gate.
 * No counterpart in the reference (see qe_attn_decode_partials). */
hipError_t qe_attn_decode_combine(const float* part_o, const float* part_ml, const int* pos,
                                  const void* qg, long ldp, void* out, long ldo, int n, int Hq,
                                  int max_len, int NS, hipStream_t stream);

/* Chunked-prefill gated attention: T rows at positions pos..pos+T-1 (q normed and roped, e.g.
 * by qe_attn_prep with n = T; their K/V already in the cache), row t attends cache positions
 * [0, min(pos+t+1, max_len)), out[t] = bf16(bf16(softmax . V) * bf16(sigmoid(gate))) with the
 * gate in qg[t][h][D:2D]. MFMA flash attention with LDS-staged K/V tiles.
 * Valid: T >= 1, Hq % Hkv == 0, 16-byte aligned q/kc/vc/qg/out, ldp % 8 == 0, ldo % 8 == 0,
 * (max_len+160)*512 < 2^32. q rows are contiguous ([T][Hq*D]).
 * No counterpart in the reference: it feeds prompts through the n <= 8 decode path
 * (python/qengine/engine.py:542-573). */
hipError_t qe_attn_prefill(const void* q, const void* kc, const void* vc, const int* pos,
                           const void* qg, long ldp, void* out, long ldo, int T, int Hq, int Hkv,
                           int max_len, float scale, hipStream_t stream);

/* Number of cache positions per split-KV slice for a row attending L positions with NS partial
 * slots: ceil(L/NS) rounded up to a multiple of 32 (at least 32); row t's partial s covers
 * positions [s*size, (s+1)*size) of [0, L). The reference cuts ceil(L/NS) (csrc/attn.cu:78-80);
 * this function has no counterpart there. It runs the kernels' own arithmetic (a host-computed
 * multiply and shift for the division by NS). Returns 0 for L < 1, L >= 2^23 or NS < 1. */
int qe_attn_split_size(int L, int NS);

/* The fp8 KV cache (no counterpart in the reference, whose cache is bf16: python/qengine/
 * engine.py:419): kc8/vc8 are [Hkv][max_len][256] E4M3FN codes (one byte per value, OCP fp8, the
 * format gfx950's cvt instructions use) with one scale per cache: a code c stands for c * scale.
 * Halves the bytes the decode streams. */

/* qe_attn_prep writing the fp8 cache: a K or V value x is stored as the code nearest to
 * x * (1 / scale) (fp32 product, round to nearest even, saturated at +-448; NaN stays NaN).
 * Valid as qe_attn_prep, plus k_scale, v_scale positive and finite. */
hipError_t qe_attn_prep_fp8(const void* qg, const void* k, const void* v, long ldp,
                            const void* qnw, const void* knw, const float* inv_freq,
                            const int* pos, void* q_out, void* kc8, void* vc8, int n, int Hq,
                            int Hkv, int max_len, int rd, float eps, float k_scale, float v_scale,
                            hipStream_t stream);

/* qe_attn_decode over the fp8 cache: the same attention on the dequantized values (k_scale
 * scales every score, v_scale the attention output before its bf16 rounding). Row t of an n-row
 * call is bit-identical to a 1-row call. Valid as qe_attn_decode. */
hipError_t qe_attn_decode_fp8(const void* q, const void* kc8, const void* vc8, const int* pos,
                              const void* qg, long ldp, float* part_o, float* part_ml, void* out,
                              long ldo, int n, int Hq, int Hkv, int max_len, int NS, float scale,
                              float k_scale, float v_scale, hipStream_t stream);

/* qe_attn_prefill over the fp8 cache: the same attention on the dequantized values (k_scale
 * scales every score, v_scale the attention output before its bf16 rounding). With scales of 1
 * it equals qe_attn_prefill on the dequantized cache bit for bit. Valid as qe_attn_prefill, plus
 * k_scale, v_scale positive and finite. */
hipError_t qe_attn_prefill_fp8(const void* q, const void* kc8, const void* vc8, const int* pos,
                               const void* qg, long ldp, void* out, long ldo, int T, int Hq,
                               int Hkv, int max_len, float scale, float k_scale, float v_scale,
                               hipStream_t stream);

/* First half of qe_attn_decode_fp8 (the partials are not yet multiplied by v_scale). */
hipError_t qe_attn_decode_fp8_partials(const void* q, const void* kc8, const void* vc8,
                                       const int* pos, float* part_o, float* part_ml, int n,
                                       int Hq, int Hkv, int max_len, int NS, float scale,
                                       float k_scale, hipStream_t stream);

/* Measurement only (no counterpart in the reference). A streaming read of exactly the K and V
 * bytes a 1-row decode call at position *pos reads (L = min(*pos+1, max_len) positions), with
 * the partials kernel's grid and slicing (slices of qe_attn_split_size(L, NS) positions x Hkv
 * heads, pos read on the device, 256 threads per workgroup, 16-byte non-temporal loads) and no
 * arithmetic: the floor of any kernel that reads those bytes with that grid. `sink` (4 bytes of
 * device memory) is written only if the folded value hits a constant.
 * Valid: max_len >= 1, Hkv >= 1, NS >= 1, (max_len + 64)*512 < 2^32. */
hipError_t qe_kv_stream_probe(const void* kc, const void* vc, const int* pos, int Hkv,
                              int max_len, int NS, void* sink, hipStream_t stream);

/* Measurement only (no counterpart in the reference). The same K and V bytes as
 * qe_kv_stream_probe on any grid: (grid_per_head, Hkv) workgroups of 256 threads, each streaming
 * a 4 KB-aligned 1/grid_per_head share of its KV head's K rows and of its V rows with depth +
 * depth sixteen-byte non-temporal loads in flight per thread, no arithmetic. Swept over the grid
 * and depth, the fastest is the floor of any one-launch read of these bytes on the part.
 * Valid: max_len >= 1, Hkv >= 1, 1 <= grid_per_head <= 65535, depth in {4, 8, 16},
 * (max_len + 64)*512 < 2^32. */
hipError_t qe_kv_stream_sweep(const void* kc, const void* vc, const int* pos, int Hkv,
                              int max_len, int grid_per_head, int depth, void* sink,
                              hipStream_t stream);

/* Measurement only: one empty one-wave kernel. Its time per node in a hipGraph of such launches
 * is the per-launch floor every graph node pays. */
hipError_t qe_launch_probe(hipStream_t stream);

/* Version string of this library. */
const char* qe_attn_version(void);

/* Import-compatibility no-ops for the reference's programmatic-dependent-launch switches
 * (reference csrc/ops.h:34-35, csrc/bindings.cpp:195-196). gfx950 has no equivalent. */
void qe_set_pdl_trigger(int on);
void qe_set_pdl_launch(int on);

#ifdef __cplusplus
}
#endif

#endif /* QE_ATTN_H */
