// One 32-position tile of gated attention on MFMA, shared by the decode and prefill kernels.
//
// Layout (wave64, v_mfma_f32_16x16x32_bf16, lane = 16*g4 + c):
//  * Columns are queries (q head x row); a wave holds NT column tiles of 16 in registers as the
//    B operand qb[ct][ks] (dims [32ks + 8g4, +8) of column ct*16 + c).
//  * S^T = K Q^T: the A operand (16 positions x 32 dims) is read from the wave's or workgroup's
//    LDS K tile (XOR-swizzled, see k_slot). Lane holds positions p0 + 16T + 4g4 + i of column c.
//  * O^T += V^T P^T: P^T is the B operand with element e <-> position P(g4, e) = p0 + 16(e>>2) +
//    4g4 + (e&3). The V^T A operands (which dims a lane holds) are the caller's choice; the
//    softmax only rescales the NACC accumulators of each column tile.
//  * Online softmax per column in the log2 domain with lazy rescaling: a column's reference max
//    only moves when a score exceeds it by more than LAZY_TAU, so p = exp2(s - m_ref) <= 2^TAU
//    and the accumulators are rescaled rarely. O/L is unchanged mathematically, and each column's
//    arithmetic depends on that column alone.
#pragma once
#include "qe_device.hpp"

namespace qe {
namespace tile {

constexpr int BN = 32;                   // positions per tile (two 16-row MFMA tiles)
constexpr int ROW_CHUNKS = HD * 2 / 16;  // 16-byte chunks per 512-byte cache row
constexpr float LAZY_TAU = 8.f;          // log2 headroom before the reference max must move

// LDS slot of (row r, chunk q) in a K tile: chunks XOR-swizzled by r & 15, so the 16 lanes that
// read one chunk column of 16 rows hit 16 different bank groups.
__device__ __forceinline__ int k_slot(int r, int q) { return r * ROW_CHUNKS + (q ^ (r & 15)); }

// S^T for one tile: sacc[ct][T] holds positions p0 + 16T + 4g4 + i of column ct*16 + c.
// Lane (c, g4) reads chunk 4ks + g4 of row 16T + c, at slot k_slot(16T + c, 4ks + g4). Since
// (4ks + g4) ^ c = 4 (ks ^ (c >> 2)) + (g4 ^ (c & 3)) and ks ^ (c >> 2) = 4 (ks >> 2) +
// ((ks & 3) ^ (c >> 2)), the byte offset is kl[ks & 3] + 256 (ks >> 2) + 8192 T with four
// per-lane bases: one address add per base and tile, the rest immediate offsets (about 25 fewer
// VALU instructions per tile). Callers with two or more column tiles per wave sit at the register
// limit and keep the per-read slot arithmetic, which needs no extra live registers.
// XA (NT == 1; the K tile 256-byte aligned in LDS): the four bases are one per-lane base XORed
// with 64 (ks & 3), since 64 (l ^ (c >> 2)) = 64 l ^ 64 (c >> 2) touches address bits 6-7 only:
// the same addresses, formed per tile instead of living across the caller's loop.
// LEAD > 0: the tile's 16 K operand reads and 16 NT MFMAs are scheduled as LEAD reads, then
// (NT MFMAs, 1 read) groups, then the last LEAD NT MFMAs (sched_group_barrier), so LEAD reads
// stay in flight ahead of the MFMAs that need them.
template <int NT, bool XA = false, int LEAD = 0>
__device__ __forceinline__ void qk_tile(const u32x4_t* k_lds, const bf16x8_t (&qb)[NT][8], int c,
                                        int g4, f32x4_t (&sacc)[NT][2]) {
  typedef __attribute__((address_space(3))) const u32x4_t lds_u32x4;
  const char* kb = reinterpret_cast<const char*>(k_lds);
  const char* kl[4];
#pragma unroll
  for (int l = 0; l < 4; ++l)
    kl[l] = kb + c * (ROW_CHUNKS * 16) + 64 * (l ^ (c >> 2)) + 16 * (g4 ^ (c & 3));
  const uint32_t k0 = (uint32_t)(uintptr_t)((__attribute__((address_space(3))) const char*)kb) +
                      c * (ROW_CHUNKS * 16) + 64 * (c >> 2) + 16 * (g4 ^ (c & 3));
#pragma unroll
  for (int T = 0; T < 2; ++T) {
#pragma unroll
    for (int ct = 0; ct < NT; ++ct) sacc[ct][T] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      const int off = 256 * (ks >> 2) + 16 * ROW_CHUNKS * 16 * T;
      const bf16x8_t kop =
          NT == 1 ? (XA ? as_bf16x8(*(lds_u32x4*)(uintptr_t)((k0 ^ (64u * (ks & 3))) + off))
                        : as_bf16x8(*reinterpret_cast<const u32x4_t*>(kl[ks & 3] + off)))
                  : as_bf16x8(k_lds[k_slot(16 * T + c, 4 * ks + g4)]);
#pragma unroll
      for (int ct = 0; ct < NT; ++ct) sacc[ct][T] = mfma16x16x32(kop, qb[ct][ks], sacc[ct][T]);
    }
  }
  if constexpr (LEAD > 0) {
    __builtin_amdgcn_sched_group_barrier(0x100, LEAD, 0);   // LDS reads
#pragma unroll
    for (int i = 0; i < 16 - LEAD; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, NT, 0);   // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, LEAD * NT, 0);
  }
}

// Online softmax of one tile. MASK: positions >= Lcol[ct] are excluded (needed only on tiles that
// reach past the shortest attended length among the real columns). SPLIT: P goes to the PV MFMA
// as bf16 hi + lo terms (~2^-17 relative) instead of one bf16 term (2^-9).
template <int NT, bool MASK, bool SPLIT, int NACC>
__device__ __forceinline__ void softmax_tile(const f32x4_t (&sacc)[NT][2], int p0,
                                             const int (&Lcol)[NT], float scale_log2, int g4,
                                             float (&m)[NT], float (&l)[NT],
                                             f32x4_t (&acc)[NT][NACC], u32x4_t (&pb_hi)[NT],
                                             u32x4_t (&pb_lo)[NT]) {
  float corr[NT];
  bool moved = false;
#pragma unroll
  for (int ct = 0; ct < NT; ++ct) {
    float sv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = sacc[ct][e >> 2][e & 3] * scale_log2;
      if constexpr (MASK) {
        const int p = p0 + 16 * (e >> 2) + 4 * g4 + (e & 3);
        sv[e] = p < Lcol[ct] ? x : -INFINITY;
      } else {
        sv[e] = x;
      }
    }
    float tmax = fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])),
                       fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7])));
    tmax = group4_max(tmax);
    corr[ct] = 1.f;
    if (tmax > m[ct] + LAZY_TAU) {  // also taken on the first finite tile (m = -inf)
      if (m[ct] != -INFINITY) {
        corr[ct] = __builtin_amdgcn_exp2f(m[ct] - tmax);
        moved = true;
      }
      m[ct] = tmax;
    }
    const float msub = m[ct] == -INFINITY ? 0.f : m[ct];
    float pf[8];
    float lsum = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      pf[e] = __builtin_amdgcn_exp2f(sv[e] - msub);
      lsum += pf[e];
    }
    l[ct] = l[ct] * corr[ct] + lsum;
#pragma unroll
    for (int d = 0; d < 4; ++d) pb_hi[ct][d] = pack_bf16x2(pf[2 * d], pf[2 * d + 1]);
    if constexpr (SPLIT) {
#pragma unroll
      for (int d = 0; d < 4; ++d)
        pb_lo[ct][d] = pack_bf16x2(pf[2 * d] - lo_bf16(pb_hi[ct][d]),
                                   pf[2 * d + 1] - hi_bf16(pb_hi[ct][d]));
    }
  }
  if (__any(moved)) {  // a multiply by exactly 1 for columns that did not move
#pragma unroll
    for (int ct = 0; ct < NT; ++ct)
#pragma unroll
      for (int a = 0; a < NACC; ++a) acc[ct][a] *= corr[ct];
  }
}

// O^T += V^T P^T for dims [128hh, 128hh + 128) from V rows in registers (the decode kernels' V
// loads, and the fp8 cache's converted codes): vr[e] = 16 bytes of V row
// P(g4, e), dims 128hh + 8c + [0, 8). M-tile i of the half has row c = dim 128hh + 8c + i, so
// acc[ct][8hh + i][ii] = O^T[dim 128hh + 32g4 + 8ii + i][column c].
template <int NT, bool SPLIT>
__device__ __forceinline__ void pv_half(const u32x4_t (&vr)[8], int hh, const u32x4_t (&pb_hi)[NT],
                                        const u32x4_t (&pb_lo)[NT], f32x4_t (&acc)[NT][16]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    u32x4_t a;
#pragma unroll
    for (int d = 0; d < 4; ++d) a[d] = interleave_halves(vr[2 * d][i >> 1], vr[2 * d + 1][i >> 1], i & 1);
#pragma unroll
    for (int ct = 0; ct < NT; ++ct) {
      acc[ct][8 * hh + i] = mfma16x16x32(as_bf16x8(a), as_bf16x8(pb_hi[ct]), acc[ct][8 * hh + i]);
      if constexpr (SPLIT)
        acc[ct][8 * hh + i] = mfma16x16x32(as_bf16x8(a), as_bf16x8(pb_lo[ct]), acc[ct][8 * hh + i]);
    }
  }
}

// A V tile (32 rows of 256 bf16) in LDS for pv_tile_tr: chunk q of row r sits in 16-byte slot
// r * ROW_CHUNKS + (q ^ v_swz(r)). A transposing read touches 16 rows at the same two chunks; with
// this swizzle every 8 consecutive rows spread them over 16 distinct 16-byte bank groups.
__device__ __forceinline__ int v_swz(int r) { return 2 * (r & 7); }

// O^T += V^T P^T over one tile with the V^T operands read from LDS by gfx950's transposing read.
// M-tile i holds dims 16i .. 16i+15: acc[ct][i][k] = O^T[16i + 4 g4 + k][column c]. The A operand
// of lane (c, g4) is V[P(g4, e)][16i + c] for e = 0..7, P(g4, e) = p0 + 16(e>>2) + 4g4 + (e&3)
// (the positions of P^T's element e, softmax_tile). ds_read_b64_tr_b16 hands lane 4a + b of each
// 16-lane group element b of the 8 bytes addressed by lane a + 4e of the group, as element e
// (lane layout checked on MI355X). So lane (a = lane & 3, lane/4 & 3, g4) addresses V row
// 4g4 + (lane/4 & 3) (+16 for elements 4..7) at dims 16i + 4a .. +3.
// XA (NT == 1; the V tile 256-byte aligned in LDS): the eight bases are one per-lane base XORed
// with 32 (i & 7) (32 (l ^ (r & 7)) = 32 l ^ 32 (r & 7) touches address bits 5-7 only), formed
// per tile instead of living across the caller's loop: 13 fewer registers in the prefill kernel.
// LEAD > 0: the 32 transposing reads and the MFMAs of the 16 M-tiles (NT, or 2 NT with SPLIT,
// each) are scheduled as the reads of LEAD M-tiles, then (one M-tile's MFMAs, 2 reads) groups,
// then the last LEAD M-tiles' MFMAs.
template <int NT, bool SPLIT, bool XA = false, int LEAD = 0>
__device__ __forceinline__ void pv_tile_tr(const u32x4_t* vt, int lane, int g4,
                                           const u32x4_t (&pb_hi)[NT], const u32x4_t (&pb_lo)[NT],
                                           f32x4_t (&acc)[NT][16]) {
  typedef short v4i16 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
  const int a = lane & 3, r = 4 * g4 + ((lane >> 2) & 3);
  // Chunk (2i + (a >> 1)) ^ v_swz(r) = 2 (i ^ (r & 7)) + (a >> 1) = 16 (i >> 3) + 2 ((i & 7) ^
  // (r & 7)) + (a >> 1): eight per-lane bases vl[i & 7], and 256 (i >> 3) as an immediate offset.
  // (The bases cost registers: callers with two or more column tiles per wave compute each
  // address from the swizzle instead.)
  char* vr = const_cast<char*>(reinterpret_cast<const char*>(vt)) + r * (HD * 2) + (a & 1) * 8;
  char* vl[8];
#pragma unroll
  for (int l = 0; l < 8; ++l) vl[l] = vr + 16 * (a >> 1) + 32 * (l ^ (r & 7));
  const uint32_t v0 = (uint32_t)(uintptr_t)((__attribute__((address_space(3))) char*)vr) +
                      16 * (a >> 1) + 32 * (r & 7);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    typedef __attribute__((address_space(3))) char lds_char;
    lds_char* p =
        NT == 1 ? (XA ? (lds_char*)(uintptr_t)((v0 ^ (32u * (i & 7))) + 256 * (i >> 3))
                      : (lds_char*)(vl[i & 7] + 256 * (i >> 3)))  // rows r, r + 16: one swizzle
                : (lds_char*)(vr + ((2 * i + (a >> 1)) ^ v_swz(r)) * 16);
    const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(reinterpret_cast<lds_v4i16*>(p));
    const v4i16 hi =
        __builtin_amdgcn_ds_read_tr16_b64_v4i16(reinterpret_cast<lds_v4i16*>(p + 16 * HD * 2));
    const u32x2_t l2 = __builtin_bit_cast(u32x2_t, lo), h2 = __builtin_bit_cast(u32x2_t, hi);
    const u32x4_t av = {l2[0], l2[1], h2[0], h2[1]};
#pragma unroll
    for (int ct = 0; ct < NT; ++ct) {
      acc[ct][i] = mfma16x16x32(as_bf16x8(av), as_bf16x8(pb_hi[ct]), acc[ct][i]);
      if constexpr (SPLIT)
        acc[ct][i] = mfma16x16x32(as_bf16x8(av), as_bf16x8(pb_lo[ct]), acc[ct][i]);
    }
  }
  if constexpr (LEAD > 0) {
    constexpr int MPT = NT * (SPLIT ? 2 : 1);  // MFMAs per M-tile
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * LEAD, 0);  // LDS reads
#pragma unroll
    for (int i = 0; i < 16 - LEAD; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, MPT, 0);     // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, LEAD * MPT, 0);
  }
}

}  // namespace tile
}  // namespace qe
