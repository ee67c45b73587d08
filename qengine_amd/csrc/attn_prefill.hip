// Chunked-prefill gated attention on gfx950 (MI355X): T query rows at positions pos..pos+T-1,
// row t attends cache positions [0, min(pos+t+1, max_len)), out = bf16(bf16(softmax . V) *
// bf16(sigmoid(gate))). Same per-row semantics as decode (reference csrc/attn.cu:1-2,78,146-148;
// python/qengine/reference.py:263-272). The reference has no prefill kernel: it feeds prompts
// through its n <= 8 row decode path (engine.py:542-573).
//
// Design (compute-bound, MFMA):
//  * Workgroup = 128 consecutive query rows of one q head: 8 waves x 16 rows (one 16-column MFMA
//    tile per wave, two waves per SIMD). Workgroups are dispatched heaviest (longest attended prefix) first
//    over the whole grid, which balances the causal triangle across the CUs, and the workgroups of
//    one KV head are placed on the same XCDs (one L2 per XCD).
//  * K/V tiles of 32 positions are streamed into a 4-stage LDS ring by LDS DMA (each wave fetches
//    4 rows of K and of V, three tiles ahead, one barrier per tile) and shared by the 8 waves. K
//    and V are XOR-swizzled for conflict-free operand reads (rocprofv3: zero LDS bank conflicts).
//  * The V^T operands of PV come straight from LDS through gfx950's transposing read
//    (ds_read_b64_tr_b16), so no VALU permutes assemble them.
//  * Per tile and wave: S^T = K Q^T (16 MFMA 16x16x32), online softmax per column in the log2
//    domain with lazy rescaling, O^T += V^T P^T (16 MFMA). Waves whose rows attend fewer than
//    512 positions pass P as bf16 hi + lo terms (32 MFMA) for fp32-class accuracy; longer rows
//    average the bf16 rounding of P away. Q lives in registers as the B operand, O^T in
//    accumulation registers. The tile math is shared with decode (attn_tile.hpp).
//  * The tile loop body is branch-free: unmasked tiles (below the wave's shortest row) and masked
//    tiles run as two loops, and the hi/lo choice is made once per wave, so the accumulators stay
//    in one register class across iterations.
//  * Epilogue: O / l rounded to bf16, times bf16(sigmoid(gate)), 8-byte stores.
//  * At GQA 6 (bf16 and fp8 caches), attn_prefill_bal_kernel runs the same per-wave code in a
//    layout that balances the causal triangle: 12 waves (three per SIMD) of one KV head own
//    three quads of (16-row block, q head) units, four units of one length per quad, one unit of
//    each quad per SIMD; the quads of a workgroup mix lengths so that every workgroup carries
//    about the same work, and the grid is one round of workgroups (config 5: 256). Same bits as
//    the 8-wave kernel. Its first form (blocks j and nb-1-j, one q head per wave): 222 -> 212 us
//    at config 5 (same-box A/B); on the fp8 cache it replaced the 8-wave kernel: 290 -> 243 us.
//  * The file is compiled with LLVM's max-ILP machine scheduler. Under the default
//    (occupancy-first) scheduler the tile loop kept one LDS operand read in flight and waited
//    for it before every MFMA; max-ILP interleaves the two S^T accumulation chains and keeps two
//    or more reads in flight in the same 168 registers. Same bits; config 5, same-box A/B against
//    the default scheduler: 207.8 -> 189.3 us (bf16 cache), 243.7 -> 224.7 us (fp8 cache).
#include "attn_tile.hpp"
#include "qe_attn.h"

namespace qe {
namespace prefill {

// Two waves per SIMD: one wave's softmax (VALU) overlaps the other's MFMAs. With 16 rows per
// wave the tile loop fits 218 VGPRs. (Measured on MI355X at config 5: 4 waves x 32 rows, one wave
// per SIMD, ran 328 us; 8 waves x 16 rows runs 271 us.)
constexpr int WAVES = 8;
constexpr int ROWS_PER_WAVE = 16;               // one 16-column MFMA tile per wave
constexpr int NT = ROWS_PER_WAVE / 16;
constexpr int BQ = WAVES * ROWS_PER_WAVE;       // 128 query rows per workgroup
using tile::BN;                                 // cache positions per step
using tile::ROW_CHUNKS;
// Rows attending at least this many positions use one bf16 term for P (error ~2^-9/sqrt(N) of
// the output scale); shorter rows use the hi + lo split.
constexpr int SPLIT_BELOW = 512;
constexpr int TILE_U4 = BN * ROW_CHUNKS;        // 16-byte slots per K (or V) tile: 1024
constexpr int STAGE_U4 = 2 * TILE_U4;           // K tile then V tile (32 KB)
constexpr int STAGES = 4;                       // LDS ring of tiles
constexpr int AHEAD = STAGES - 1;               // tiles in flight beyond the one computed
constexpr int LOAD_ROWS = BN / WAVES;            // K and V rows each wave fetches per tile
constexpr int LOAD_INSTR = LOAD_ROWS / 2;        // two 512-byte rows per LDS-DMA instruction
constexpr int LOADS_PER_TILE = 2 * LOAD_INSTR;   // K then V
static_assert(LOAD_ROWS % 2 == 0 && LOADS_PER_TILE * AHEAD < 64, "tile split over the waves");
constexpr int PF_CPOL = 0;                      // cached loads: every row block re-reads its KV head
constexpr int XCDS = 8;                         // MI355X: 8 XCDs, each with its own L2
// Operand reads kept ahead of the MFMAs in a tile's S^T and O^T steps (tile::qk_tile / pv_tile_tr
// LEAD: 4 K reads, the V^T reads of 4 M-tiles). Max-ILP alone measured 172.2 us at config 5
// (balanced kernel, bf16 cache, one-process A/B); leads 2 / 4 / 6 / 8 gave 171.0 / 169.4 /
// 168.4 / 183.8 (bits identical).
constexpr int SG_LEAD = 4;

// Issue this wave's LDS-DMA loads of tile [p0, p0 + 32): rows LOAD_ROWS*w .. +LOAD_ROWS of K
// and of V (both swizzled: lane i fetches the chunk that belongs in slot 64j + i).
__device__ __forceinline__ void issue_tile(u32x4_t* stage, __amdgpu_buffer_rsrc_t krs,
                                           __amdgpu_buffer_rsrc_t vrs, int p0, int w, int lane) {
#pragma unroll
  for (int j = 0; j < LOAD_INSTR; ++j) {
    const int r = LOAD_ROWS * w + 2 * j + (lane >> 5);
    const int q = (lane & 31) ^ (r & 15);
    buffer_load16_to_lds<PF_CPOL>(krs, (uint32_t)(p0 + r) * (HD * 2) + q * 16,
                                  stage + (LOAD_ROWS * w + 2 * j) * ROW_CHUNKS);
  }
#pragma unroll
  for (int j = 0; j < LOAD_INSTR; ++j) {
    const int r = LOAD_ROWS * w + 2 * j + (lane >> 5);
    buffer_load16_to_lds<PF_CPOL>(vrs, (uint32_t)(p0 + r) * (HD * 2) + ((lane & 31) ^ tile::v_swz(r)) * 16,
                                  stage + TILE_U4 + (LOAD_ROWS * w + 2 * j) * ROW_CHUNKS);
  }
}

// Per-wave running softmax state and O^T accumulators.
struct WaveState {
  float m[NT], l[NT];
  f32x4_t acc[NT][16];  // acc[ct][i][k] = O^T[16i + 4 g4 + k][column ct*16 + c] (tile::pv_tile_tr)
};

// Tiles [j0, j1) of the ring with one branch-free body (SPLIT and MASK fixed).
template <bool SPLIT, bool MASK>
__device__ __forceinline__ void run_tiles(int j0, int j1, int Lwave, u32x4_t* lds,
                                          __amdgpu_buffer_rsrc_t krs, __amdgpu_buffer_rsrc_t vrs,
                                          int w, int lane, int c, int g4,
                                          const bf16x8_t (&qb)[NT][8], const int (&Lcol)[NT],
                                          float scale_log2, WaveState& st) {
  for (int j = j0; j < j1; ++j) {
    const u32x4_t* kt = lds + (j % STAGES) * STAGE_U4;
    const u32x4_t* vt = kt + TILE_U4;
    const int p0 = j * BN;
    vmcnt_wait<LOADS_PER_TILE * (AHEAD - 1)>();  // this wave's loads of tile j are done
    __syncthreads();                // ... and every wave's; tile j-1's stage is free
    // the arithmetic on tile j first, then the loads of tile j + AHEAD: GQA 4 / 8 shapes of
    // config 5 231.3 / 145.0 -> 225.6 / 140.0 us against issuing the loads first (same bits)
    if (p0 < Lwave) {  // tiles past this wave's rows contribute nothing
      f32x4_t sacc[NT][2];
      tile::qk_tile<NT, NT == 1, SG_LEAD>(kt, qb, c, g4, sacc);
      u32x4_t pb_hi[NT], pb_lo[NT];
      tile::softmax_tile<NT, MASK, SPLIT>(sacc, p0, Lcol, scale_log2, g4, st.m, st.l, st.acc,
                                          pb_hi, pb_lo);
      tile::pv_tile_tr<NT, SPLIT, NT == 1, SG_LEAD>(vt, lane, g4, pb_hi, pb_lo, st.acc);
    }
    if (w < WAVES)  // the first WAVES waves load the ring
      issue_tile(lds + ((j + AHEAD) % STAGES) * STAGE_U4, krs, vrs, p0 + AHEAD * BN, w, lane);
  }
}

// ---- fp8 KV cache (E4M3FN codes, 256-byte rows). Tiles arrive in a STAGES-deep fp8 ring by LDS
// DMA (each wave fetches its 4 rows of K and of V: one 1 KB instruction each). One tile before
// its turn a tile is converted once by the 8 waves into a double-buffered bf16 K/V tile (the
// swizzled layouts of the bf16 path: every E4M3 value is a bf16 value, so the conversion is
// exact), and the bf16 tile math runs on it unchanged. The fp8 ring and the bf16 pair take 64 KB
// each.
constexpr int TILE8_U4 = BN * ROW_CHUNKS / 2;   // 16-byte slots per fp8 K (or V) tile: 512
constexpr int STAGE8_U4 = 2 * TILE8_U4;         // fp8 K tile then V tile (16 KB)
constexpr int LOADS_PER_TILE8 = 2;              // one K and one V instruction per wave
static_assert(STAGES * STAGE8_U4 + 2 * STAGE_U4 == STAGES * STAGE_U4, "fp8 ring + bf16 pair");

__device__ __forceinline__ void issue_tile8(u32x4_t* stage, __amdgpu_buffer_rsrc_t krs,
                                            __amdgpu_buffer_rsrc_t vrs, int p0, int w, int lane) {
  const int r = LOAD_ROWS * w + (lane >> 4);  // lane i: row 4w + i/16, 16-byte chunk i % 16
  buffer_load16_to_lds<PF_CPOL>(krs, (uint32_t)(p0 + r) * HD + (lane & 15) * 16,
                                stage + LOAD_ROWS * w * (ROW_CHUNKS / 2));
  buffer_load16_to_lds<PF_CPOL>(vrs, (uint32_t)(p0 + r) * HD + (lane & 15) * 16,
                                stage + TILE8_U4 + LOAD_ROWS * w * (ROW_CHUNKS / 2));
}

// Thread i of the workgroup converts the 16 codes of fp8 chunk i (row i/16, dims 16(i%16) ..) of
// the K and the V tile into two bf16 chunks each, at their swizzled bf16 slots. The 16 threads of
// a row write bf16 chunks 2c + p then 2c + 1 - p (c = i % 16, p = bit 2 ^ bit 3 of c), so each
// store's 8 (and 16) consecutive lanes hit distinct 16-byte bank groups: with p = 0 for all, the
// even chunks of the first store fall on half the groups (2-way conflicts). The row swizzles
// XOR a chunk index with a per-row constant, which keeps the groups distinct.
__device__ __forceinline__ void convert_tile8(const u32x4_t* stage, u32x4_t* bf) {
  const int i = threadIdx.x, r = i >> 4, c = i & 15, q = 2 * c;
  const int p = ((c >> 2) ^ (c >> 3)) & 1;
  const u32x4_t kk = stage[i], vv = stage[TILE8_U4 + i];
  // the codes of chunk q + p (first store) and q + 1 - p (second), selected before conversion
  const u32x2_t ka{p ? kk[2] : kk[0], p ? kk[3] : kk[1]}, kb{p ? kk[0] : kk[2], p ? kk[1] : kk[3]};
  const u32x2_t va{p ? vv[2] : vv[0], p ? vv[3] : vv[1]}, vb{p ? vv[0] : vv[2], p ? vv[1] : vv[3]};
  bf[tile::k_slot(r, q + p)] = fp8x8_to_bf16x8(ka);
  bf[tile::k_slot(r, q + 1 - p)] = fp8x8_to_bf16x8(kb);
  bf[TILE_U4 + r * ROW_CHUNKS + ((q + p) ^ tile::v_swz(r))] = fp8x8_to_bf16x8(va);
  bf[TILE_U4 + r * ROW_CHUNKS + ((q + 1 - p) ^ tile::v_swz(r))] = fp8x8_to_bf16x8(vb);
}

// run_tiles for the fp8 cache, converting one tile ahead: iteration j computes tile j from bf16
// pair j % 2, then converts tile j + 1 into pair (j + 1) % 2 (whose previous tile, j - 1, every
// wave finished before this iteration's barrier), so one barrier per tile orders both. Tile j's
// fp8 stage is free once converted, so iteration j refills it with tile j + STAGES and loads
// still run STAGES - 1 iterations ahead of their conversion. Same bits throughout; config 5
// shapes at GQA 4 / 8: converting tile j between two barriers, then computing it, 277.8 / 178.1
// us; one barrier, converting before the arithmetic 264.5 / 169.3 (266.3 / 169.5 on another
// box); after it 257.9 / 163.3.
template <bool SPLIT, bool MASK>
__device__ __forceinline__ void run_tiles8(int j0, int j1, int Lwave, u32x4_t* lds,
                                           __amdgpu_buffer_rsrc_t krs, __amdgpu_buffer_rsrc_t vrs,
                                           int w, int lane, int c, int g4,
                                           const bf16x8_t (&qb)[NT][8], const int (&Lcol)[NT],
                                           float scale_log2, WaveState& st) {
  u32x4_t* bfp = lds + STAGES * STAGE8_U4;
  for (int j = j0; j < j1; ++j) {
    const int p0 = j * BN;
    vmcnt_wait<LOADS_PER_TILE8 * (STAGES - 2)>();  // this wave's loads of tile j + 1 are done
    // ... and every wave's; bf16 tile j is complete, tile j's fp8 stage and pair (j + 1) % 2 free
    __syncthreads();
    issue_tile8(lds + (j % STAGES) * STAGE8_U4, krs, vrs, p0 + STAGES * BN, w, lane);
    if (p0 < Lwave) {
      const u32x4_t* bf = bfp + (j & 1) * STAGE_U4;
      f32x4_t sacc[NT][2];
      tile::qk_tile<NT, NT == 1, SG_LEAD>(bf, qb, c, g4, sacc);
      u32x4_t pb_hi[NT], pb_lo[NT];
      tile::softmax_tile<NT, MASK, SPLIT>(sacc, p0, Lcol, scale_log2, g4, st.m, st.l, st.acc, pb_hi,
                                          pb_lo);
      tile::pv_tile_tr<NT, SPLIT, NT == 1, SG_LEAD>(bf + TILE_U4, lane, g4, pb_hi, pb_lo, st.acc);
    }
    convert_tile8(lds + ((j + 1) % STAGES) * STAGE8_U4, bfp + ((j + 1) & 1) * STAGE_U4);
  }
}

// KV8: kc/vc hold fp8 codes (one byte per value); v_scale multiplies O / l before its bf16
// rounding (exactly 1 for the bf16 cache).
template <bool KV8>
__global__ void __launch_bounds__(WAVES * WAVE)
attn_prefill_kernel(const __bf16* __restrict__ q, const void* __restrict__ kc,
                    const void* __restrict__ vc, const int* __restrict__ pos_ptr,
                    const __bf16* __restrict__ qg, long ldp, __bf16* __restrict__ out, long ldo,
                    int T, int Hq, int Hkv, int max_len, float scale_log2, float v_scale,
                    int xcd_split) {
  const int grp = Hq / Hkv;
  const int nblk = (T + BQ - 1) / BQ;
  int blk, h;
  if (xcd_split > 0) {
    // Workgroups are dispatched round-robin over the XCDs (linear id L -> XCD L % 8). The
    // xcd_split XCDs 8g/Hkv .. serve KV head g only, taking turns along its work list (row block
    // heaviest first, then q head), so the workgroups that read one KV head's cache share an L2
    // and every XCD gets the same mix of heavy and light blocks.
    const int L = blockIdx.x, x = L % XCDS;
    const int i = (L / XCDS) * xcd_split + x % xcd_split;  // index in KV head g's work list
    blk = nblk - 1 - i / grp;
    h = (x / xcd_split) * grp + i % grp;
  } else {
    blk = nblk - 1 - (int)(blockIdx.x / Hq);  // heaviest (latest) row block first
    h = blockIdx.x % Hq;
  }
  const int g = h / grp;
  const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
  const int c = lane & 15, g4 = lane >> 4;
  const int pos0 = pos_ptr[0];

  __shared__ __attribute__((aligned(256))) u32x4_t lds[STAGES * STAGE_U4];  // 128 KB

  // Q^T as the MFMA B operand: column ct*16 + c is chunk row r = blk*128 + 32w + 16ct + c.
  bf16x8_t qb[NT][8];
  int Lcol[NT];
#pragma unroll
  for (int ct = 0; ct < NT; ++ct) {
    const int r = blk * BQ + w * ROWS_PER_WAVE + ct * 16 + c;
    if (r < T) {
      Lcol[ct] = min(pos0 + r + 1, max_len);
      const u32x4_t* src = reinterpret_cast<const u32x4_t*>(q + (size_t)r * Hq * HD + (size_t)h * HD);
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) qb[ct][ks] = as_bf16x8(src[4 * ks + g4]);
    } else {
      Lcol[ct] = 0;
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) qb[ct][ks] = as_bf16x8(u32x4_t{0u, 0u, 0u, 0u});
    }
  }
  // Longest attended prefix of this workgroup's rows and of this wave's rows; shortest among the
  // wave's real rows (its first row): tiles reaching past it need the per-position mask, and it
  // decides whether P is split.
  const int last_row = min(blk * BQ + BQ, T) - 1;
  const int Lwg = min(pos0 + last_row + 1, max_len);
  const int r_first = blk * BQ + w * ROWS_PER_WAVE;
  const int Lwave = min(pos0 + min(r_first + ROWS_PER_WAVE, T), max_len);
  const int Lmin = min(pos0 + r_first + 1, max_len);
  const int ntiles = Lwg > 0 ? (Lwg + BN - 1) / BN : 0;
  const bool split = Lmin < SPLIT_BELOW;

  constexpr int ELEM = KV8 ? 1 : 2;  // bytes per cache value
  const size_t head_off = (size_t)g * max_len * HD * ELEM;  // bytes
  const uint32_t bytes = (uint32_t)max(Lwg, 0) * (uint32_t)(HD * ELEM);  // past Lwg reads 0
  const __amdgpu_buffer_rsrc_t krs = make_rsrc(static_cast<const char*>(kc) + head_off, bytes);
  const __amdgpu_buffer_rsrc_t vrs = make_rsrc(static_cast<const char*>(vc) + head_off, bytes);

  WaveState st;
#pragma unroll
  for (int ct = 0; ct < NT; ++ct) {
    st.m[ct] = -INFINITY;
    st.l[ct] = 0.f;
#pragma unroll
    for (int a = 0; a < 16; ++a) st.acc[ct][a] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  // Ring of STAGES tiles, AHEAD in flight. One barrier per tile: after the barrier of tile j every
  // wave has finished tile j-1, whose stage is the one refilled with tile j+AHEAD.
  // Tiles below jm need no per-position mask (every real row of the wave attends them fully).
  const int jm = min(ntiles, max(Lmin, 0) / BN);
  if constexpr (KV8) {
#pragma unroll
    for (int a = 0; a < STAGES; ++a) issue_tile8(lds + a * STAGE8_U4, krs, vrs, a * BN, w, lane);
    vmcnt_wait<LOADS_PER_TILE8 * (STAGES - 1)>();  // this wave's loads of tile 0 are done
    __syncthreads();                                // ... and every wave's
    convert_tile8(lds, lds + STAGES * STAGE8_U4);  // the loop converts one tile ahead
    if (split) {
      run_tiles8<true, false>(0, jm, Lwave, lds, krs, vrs, w, lane, c, g4, qb, Lcol, scale_log2, st);
      run_tiles8<true, true>(jm, ntiles, Lwave, lds, krs, vrs, w, lane, c, g4, qb, Lcol, scale_log2, st);
    } else {
      run_tiles8<false, false>(0, jm, Lwave, lds, krs, vrs, w, lane, c, g4, qb, Lcol, scale_log2, st);
      run_tiles8<false, true>(jm, ntiles, Lwave, lds, krs, vrs, w, lane, c, g4, qb, Lcol, scale_log2, st);
    }
  } else {
#pragma unroll
  for (int a = 0; a < AHEAD; ++a) issue_tile(lds + a * STAGE_U4, krs, vrs, a * BN, w, lane);
  if (split) {
    run_tiles<true, false>(0, jm, Lwave, lds, krs, vrs, w, lane, c, g4, qb, Lcol, scale_log2, st);
    run_tiles<true, true>(jm, ntiles, Lwave, lds, krs, vrs, w, lane, c, g4, qb, Lcol, scale_log2, st);
  } else {
    run_tiles<false, false>(0, jm, Lwave, lds, krs, vrs, w, lane, c, g4, qb, Lcol, scale_log2, st);
    run_tiles<false, true>(jm, ntiles, Lwave, lds, krs, vrs, w, lane, c, g4, qb, Lcol, scale_log2, st);
  }
  }
  vmcnt_wait<0>();  // no LDS DMA may still target this workgroup's LDS when it exits

  // Epilogue: rows of this wave, 4 consecutive dims 16i + 4 g4 .. +3 per (ct, i) per lane.
#pragma unroll
  for (int ct = 0; ct < NT; ++ct) {
    const float L = group4_sum(st.l[ct]);
    const int r = blk * BQ + w * ROWS_PER_WAVE + ct * 16 + c;
    if (r >= T) continue;
    const __bf16* gp = qg + (size_t)r * ldp + (size_t)h * 2 * HD + HD;
    __bf16* op = out + (size_t)r * ldo + (size_t)h * HD;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int d0 = 16 * i + 4 * g4;
      const u32x2_t gb = *reinterpret_cast<const u32x2_t*>(gp + d0);
      u32x2_t ob;
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const float o0 = round_bf16((st.acc[ct][i][2 * k] / L) * v_scale);
        const float o1 = round_bf16((st.acc[ct][i][2 * k + 1] / L) * v_scale);
        const float s0 = round_bf16(sigmoid_f32(lo_bf16(gb[k])));
        const float s1 = round_bf16(sigmoid_f32(hi_bf16(gb[k])));
        ob[k] = pack_bf16x2(o0 * s0, o1 * s1);
      }
      *reinterpret_cast<u32x2_t*>(op + d0) = ob;
    }
  }
}

// Balanced layout for GQA 6: a workgroup of 12 waves (three per SIMD) owns KV head g and the pair
// of 16-row blocks j and nb-1-j (light and heavy: their attended lengths add up to about the same
// for every j) for all 6 q heads of the group. Waves 0-5 take block j of heads 0-5, waves 6-11
// block nb-1-j. Every workgroup then carries about the same work, and Hkv * nb/2 of them fill the
// CUs in one round (256 at config 5). The first 8 waves load the K/V ring as in the 8-wave kernel,
// 2 tiles ahead in the 4-stage ring (config 5 under the max-ILP scheduler: 189.3 us against 190.5
// with 3 ahead).
constexpr int BAL_WAVES = 12;
constexpr int BAL_GRP = 6;
constexpr int BAL_AHEAD = 2;

// One tile's S^T, softmax and O^T in the balanced layout, with wave priorities: the MFMA
// phases at 2, the softmax at 1, the barrier and the ring loads at 0, so that a SIMD's three waves
// hand the matrix core to a wave with MFMAs ready and fill the gaps with another's softmax.
// One-process A/B at config 5 (bf16 cache, same bits), us: no priorities 171.0; MFMA phases 2,
// softmax 1: 168.8; MFMA 3 / softmax 1 or 2: 168.8; MFMA 2 / softmax 0: 169.5; MFMA 1 /
// softmax 2: 169.2.
template <bool SPLIT, bool MASK>
__device__ __forceinline__ void tile_math_bal(const u32x4_t* kt, const u32x4_t* vt, int p0,
                                              int lane, int c, int g4,
                                              const bf16x8_t (&qb)[NT][8], const int (&Lcol)[NT],
                                              float scale_log2, WaveState& st) {
  f32x4_t sacc[NT][2];
  __builtin_amdgcn_s_setprio(2);
  tile::qk_tile<NT, NT == 1, SG_LEAD>(kt, qb, c, g4, sacc);
  __builtin_amdgcn_s_setprio(1);
  u32x4_t pb_hi[NT], pb_lo[NT];
  tile::softmax_tile<NT, MASK, SPLIT>(sacc, p0, Lcol, scale_log2, g4, st.m, st.l, st.acc, pb_hi,
                                      pb_lo);
  __builtin_amdgcn_s_setprio(2);
  tile::pv_tile_tr<NT, SPLIT, NT == 1, SG_LEAD>(vt, lane, g4, pb_hi, pb_lo, st.acc);
  __builtin_amdgcn_s_setprio(0);
}

// LOAD: this wave is one of the first 8, which fill the ring. The loaders and the other 4 waves
// run separate copies of the loop, so neither carries the other's code (config 5: 212.8 -> 191.9
// us on one box against the same loop with a per-wave branch around the loads, same bits). The
// loaders issue the next tile after their arithmetic on this one (the stage is free from the
// barrier on): 158.2 -> 156.8 us against issuing it first (one-process A/Bs, same bits; in the
// fp8 loop the same move measured 171.5 -> 173.2).
template <bool SPLIT, bool MASK, bool LOAD>
__device__ __forceinline__ void run_tiles_bal(int j0, int j1, int Lwave, u32x4_t* lds,
                                              __amdgpu_buffer_rsrc_t krs,
                                              __amdgpu_buffer_rsrc_t vrs, int w, int lane, int c,
                                              int g4, const bf16x8_t (&qb)[NT][8],
                                              const int (&Lcol)[NT], float scale_log2,
                                              WaveState& st) {
  for (int j = j0; j < j1; ++j) {
    const u32x4_t* kt = lds + (j % STAGES) * STAGE_U4;
    const u32x4_t* vt = kt + TILE_U4;
    const int p0 = j * BN;
    vmcnt_wait<LOADS_PER_TILE * (BAL_AHEAD - 1)>();  // this wave's loads of tile j are done
    __syncthreads();  // ... and every wave's; the stage refilled now (tile j-2's) is free
    if (p0 < Lwave) tile_math_bal<SPLIT, MASK>(kt, vt, p0, lane, c, g4, qb, Lcol, scale_log2, st);
    if (LOAD)
      issue_tile(lds + ((j + BAL_AHEAD) % STAGES) * STAGE_U4, krs, vrs, p0 + BAL_AHEAD * BN, w,
                 lane);
  }
}

// run_tiles_bal on the fp8 cache: the fp8 ring and the double-buffered bf16 pair of
// run_tiles8, loaded and converted by the first 8 waves (LOAD; 512 threads, one 16-byte chunk of
// K and of V each), one tile ahead: iteration j computes tile j from pair j % 2, then the loading
// waves convert tile j + 1 into pair (j + 1) % 2, so one barrier per tile serves both (the tile
// converted before the barrier of iteration j is tile j). Tile j's fp8 stage is free once it has
// been converted, so iteration j refills it with tile j + STAGES: loads still run STAGES - 1
// iterations ahead of their conversion. Same bits; config 5 fp8, one-process A/Bs in us per call:
// converting tile j between two barriers, then computing it, 188.3 (186.5 with this rule);
// converting tile j + 1 before the arithmetic 182.9; after it 169.9 against 180.3 (166.6 against
// 178.2 on another box).
template <bool SPLIT, bool MASK, bool LOAD>
__device__ __forceinline__ void run_tiles_bal8(int j0, int j1, int Lwave, u32x4_t* lds,
                                               __amdgpu_buffer_rsrc_t krs,
                                               __amdgpu_buffer_rsrc_t vrs, int w, int lane, int c,
                                               int g4, const bf16x8_t (&qb)[NT][8],
                                               const int (&Lcol)[NT], float scale_log2,
                                               WaveState& st) {
  u32x4_t* bfp = lds + STAGES * STAGE8_U4;
  for (int j = j0; j < j1; ++j) {
    const int p0 = j * BN;
    vmcnt_wait<LOADS_PER_TILE8 * (STAGES - 2)>();  // this wave's loads of tile j + 1 are done
    // ... and every wave's; bf16 tile j is complete, tile j's fp8 stage and pair (j + 1) % 2 free
    __syncthreads();
    if (LOAD) issue_tile8(lds + (j % STAGES) * STAGE8_U4, krs, vrs, p0 + STAGES * BN, w, lane);
    if (p0 < Lwave) {
      const u32x4_t* bf = bfp + (j & 1) * STAGE_U4;
      tile_math_bal<SPLIT, MASK>(bf, bf + TILE_U4, p0, lane, c, g4, qb, Lcol, scale_log2, st);
    }
    if (LOAD) convert_tile8(lds + ((j + 1) % STAGES) * STAGE8_U4, bfp + ((j + 1) & 1) * STAGE_U4);
  }
}

template <bool KV8>
__global__ void __launch_bounds__(BAL_WAVES * WAVE)
attn_prefill_bal_kernel(const __bf16* __restrict__ q, const void* __restrict__ kc,
                        const void* __restrict__ vc, const int* __restrict__ pos_ptr,
                        const __bf16* __restrict__ qg, long ldp, __bf16* __restrict__ out, long ldo,
                        int T, int Hq, int Hkv, int max_len, float scale_log2, float v_scale,
                        int xcd_split) {
  const int nb = (T + 15) / 16, npairs = (nb + 1) / 2;
  int g, jp;
  if (xcd_split > 0) {
    const int L = blockIdx.x, x = L % XCDS;
    g = x / xcd_split;
    jp = (L / XCDS) * xcd_split + x % xcd_split;
  } else {
    g = blockIdx.x / npairs;
    jp = blockIdx.x % npairs;
  }
  const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
  const int c = lane & 15, g4 = lane >> 4;
  // Units (16-row block, q head) in quads of four of (nearly) the same length: heads 0-3 of block
  // b, and heads 4-5 of blocks 2m and 2m + 1. Quad rank r = 3m + type runs in length order:
  // type 0 = block 2m, 1 = block 2m + 1, 2 = the heads 4-5 quad of both. Each workgroup takes
  // three ranks (P = npairs workgroups per KV head), and wave w = 4k + s runs unit s of its k-th
  // quad. Wave w runs on SIMD w mod 4, so every SIMD holds one unit of each quad: the same
  // lengths on all four at every tile step. (Pairs of blocks j, nb-1-j with one head per wave
  // left the heavy block's six waves 2 / 2 / 1 / 1 on the SIMDs past the light block's end: the
  // workgroups of block 127 ran 13% longer than those of block 64 at config 5.) A tile step
  // costs more, per unit, with fewer waves on the SIMD, so how the lengths are grouped matters
  // beyond their sum; the rule was chosen by measurement. Measured at config 5 (same bits;
  // one-process A/Bs of library builds, us per call): ranks jp, P + p2(jp), 2P + p3(jp) with
  // jp + p2 + p3 within one of a constant took bf16 162.2 -> 158.1 and fp8 193.5 -> 187.4 against
  // the pairs;
  // 2jp, 2jp + 1 and 3P - 1 - jp (two short or two mid-length quads with the longest left) bf16
  // 159.0, fp8 183.6; on another box P - 1 - jp, 2P - 1 - jp, 2P + jp (the tiers matched in
  // opposite order) bf16 158.9 against 161.3 for the first, fp8 188.6 against 183.9 for the second,
  // and jp, 2P - 1 - jp, 2P + jp bf16 162.6, fp8 190.8. So the opposite tiers are taken. (The fp8
  // instance kept the second rule while its loop converted each tile between two barriers;
  // with the conversion one tile ahead the opposite tiers measured 182.9 against 186.5 us.) Each
  // unit's arithmetic is unchanged.
  const int P = npairs;
  auto triple_rank = [&](int k) __attribute__((always_inline)) {
    return k == 0 ? P - 1 - jp : k == 1 ? 2 * P - 1 - jp : 2 * P + jp;
  };
  // the last live block of a quad (-1: none)
  auto quad_top = [&](int rank) __attribute__((always_inline)) {
    const int m = rank / 3, type = rank - 3 * m;
    const int b = type < 2 ? 2 * m + type : 2 * m + 1;
    return min(b, nb - 1) >= 2 * m + (type == 1) ? min(b, nb - 1) : -1;
  };
  const int wu = __builtin_amdgcn_readfirstlane(w);  // the unit is wave-uniform (scalar)
  const int rank = triple_rank(wu >> 2), s = wu & 3;
  const int qm = rank / 3, qtype = rank - 3 * qm;
  const int blk = qtype < 2 ? 2 * qm + qtype : 2 * qm + (s >> 1);
  const int h = g * BAL_GRP + (qtype < 2 ? s : 4 + (s & 1));
  const bool wave_live = blk < nb;
  const int btop = max(quad_top(triple_rank(0)), max(quad_top(triple_rank(1)), quad_top(triple_rank(2))));
  const int pos0 = pos_ptr[0];

  __shared__ __attribute__((aligned(256))) u32x4_t lds[STAGES * STAGE_U4];  // 128 KB

  bf16x8_t qb[NT][8];
  int Lcol[NT];
  const int r = blk * 16 + c;
  if (wave_live && r < T) {
    Lcol[0] = min(pos0 + r + 1, max_len);
    const u32x4_t* src = reinterpret_cast<const u32x4_t*>(q + (size_t)r * Hq * HD + (size_t)h * HD);
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) qb[0][ks] = as_bf16x8(src[4 * ks + g4]);
  } else {
    Lcol[0] = 0;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) qb[0][ks] = as_bf16x8(u32x4_t{0u, 0u, 0u, 0u});
  }
  // the workgroup's longest attended prefix is its last live block's last row
  const int last_row = min(btop * 16 + 16, T) - 1;
  const int Lwg = min(pos0 + last_row + 1, max_len);
  const int Lwave = wave_live ? min(pos0 + min(blk * 16 + 16, T), max_len) : 0;
  const int Lmin = min(pos0 + blk * 16 + 1, max_len);
  const int ntiles = Lwg > 0 ? (Lwg + BN - 1) / BN : 0;
  const bool split = Lmin < SPLIT_BELOW;

  constexpr int ELEM = KV8 ? 1 : 2;  // bytes per cache value
  const size_t head_off = (size_t)g * max_len * HD * ELEM;
  const uint32_t bytes = (uint32_t)max(Lwg, 0) * (uint32_t)(HD * ELEM);
  const __amdgpu_buffer_rsrc_t krs = make_rsrc(static_cast<const char*>(kc) + head_off, bytes);
  const __amdgpu_buffer_rsrc_t vrs = make_rsrc(static_cast<const char*>(vc) + head_off, bytes);

  WaveState st;
  st.m[0] = -INFINITY;
  st.l[0] = 0.f;
#pragma unroll
  for (int a = 0; a < 16; ++a) st.acc[0][a] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int jm = min(ntiles, max(Lmin, 0) / BN);
  if (w < WAVES) {
    if constexpr (KV8) {
#pragma unroll
      for (int a = 0; a < STAGES; ++a)
        issue_tile8(lds + a * STAGE8_U4, krs, vrs, a * BN, w, lane);
      vmcnt_wait<LOADS_PER_TILE8 * (STAGES - 1)>();  // this wave's loads of tile 0 are done
    } else {
#pragma unroll
      for (int a = 0; a < BAL_AHEAD; ++a)
        issue_tile(lds + a * STAGE_U4, krs, vrs, a * BN, w, lane);
    }
  }
  if constexpr (KV8) {  // the fp8 loop converts one tile ahead: tile 0 here
    __syncthreads();     // every wave's loads of tile 0 are done
    if (w < WAVES) convert_tile8(lds, lds + STAGES * STAGE8_U4);
  }
  // one branch-free loop body per (split, mask) case
  auto run = [&](auto sp, auto mk, int j0, int j1) __attribute__((always_inline)) {
    constexpr bool SP = decltype(sp)::value, MK = decltype(mk)::value;
    if constexpr (KV8) {
      if (w < WAVES)
        run_tiles_bal8<SP, MK, true>(j0, j1, Lwave, lds, krs, vrs, w, lane, c, g4, qb, Lcol,
                                     scale_log2, st);
      else
        run_tiles_bal8<SP, MK, false>(j0, j1, Lwave, lds, krs, vrs, w, lane, c, g4, qb, Lcol,
                                      scale_log2, st);
    } else if (w < WAVES)
      run_tiles_bal<SP, MK, true>(j0, j1, Lwave, lds, krs, vrs, w, lane, c, g4, qb, Lcol,
                                  scale_log2, st);
    else
      run_tiles_bal<SP, MK, false>(j0, j1, Lwave, lds, krs, vrs, w, lane, c, g4, qb, Lcol,
                                   scale_log2, st);
  };
  using T_ = std::integral_constant<bool, true>;
  using F_ = std::integral_constant<bool, false>;
  if (split) {
    run(T_{}, F_{}, 0, jm);
    run(T_{}, T_{}, jm, ntiles);
  } else {
    run(F_{}, F_{}, 0, jm);
    run(F_{}, T_{}, jm, ntiles);
  }
  vmcnt_wait<0>();  // no LDS DMA may still target this workgroup's LDS when it exits

  if (!wave_live || r >= T) return;
  const float L = group4_sum(st.l[0]);
  const __bf16* gp = qg + (size_t)r * ldp + (size_t)h * 2 * HD + HD;
  __bf16* op = out + (size_t)r * ldo + (size_t)h * HD;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int d0 = 16 * i + 4 * g4;
    const u32x2_t gb = *reinterpret_cast<const u32x2_t*>(gp + d0);
    u32x2_t ob;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      // v_scale: the fp8 cache's V scale, exactly 1 for the bf16 cache
      const float o0 = round_bf16((st.acc[0][i][2 * k] / L) * v_scale);
      const float o1 = round_bf16((st.acc[0][i][2 * k + 1] / L) * v_scale);
      const float s0 = round_bf16(sigmoid_f32(lo_bf16(gb[k])));
      const float s1 = round_bf16(sigmoid_f32(hi_bf16(gb[k])));
      ob[k] = pack_bf16x2(o0 * s0, o1 * s1);
    }
    *reinterpret_cast<u32x2_t*>(op + d0) = ob;
  }
}

}  // namespace prefill
}  // namespace qe

using namespace qe;

static hipError_t launch_prefill(const void* q, const void* kc, const void* vc, const int* pos,
                                 const void* qg, long ldp, void* out, long ldo, int T, int Hq,
                                 int Hkv, int max_len, float scale, bool kv8, float k_scale,
                                 float v_scale, hipStream_t stream) {
  auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (T < 1 || Hq < 1 || Hkv < 1 || Hq % Hkv != 0 || max_len < 1 || !pos ||
      (long)((T + prefill::BQ - 1) / prefill::BQ) * Hq > 0x7fffffffL)
    return hipErrorInvalidValue;
  if (!a16(q) || !a16(kc) || !a16(vc) || !a16(qg) || !a16(out) || ldp % 8 != 0 || ldo % 8 != 0)
    return hipErrorInvalidValue;
  // byte offsets of the tiles loaded past the last attended row fit the 32-bit buffer range
  if ((unsigned long long)(max_len + (prefill::AHEAD + 2) * prefill::BN) * HD * 2 >= (1ull << 32))
    return hipErrorInvalidValue;
  const int nblk = (T + prefill::BQ - 1) / prefill::BQ;
  // KV-head-per-XCD placement when the heads divide the XCDs evenly and every XCD of a head gets
  // the same number of workgroups; otherwise plain heaviest-first order.
  const int per_head = prefill::XCDS % Hkv == 0 ? prefill::XCDS / Hkv : 0;
  const int xcd_split =
      per_head > 0 && (nblk * (Hq / Hkv)) % per_head == 0 ? per_head : 0;
  const float scale_log2 = scale * 1.4426950408889634f * k_scale;
  const dim3 grid(nblk * Hq), block(prefill::WAVES * WAVE);
  const auto* Q = static_cast<const __bf16*>(q);
  const auto* QG = static_cast<const __bf16*>(qg);
  auto* O = static_cast<__bf16*>(out);
  if (Hq == prefill::BAL_GRP * Hkv) {  // balanced 12-wave layout (GQA 6)
    const int nb = (T + 15) / 16, npairs = (nb + 1) / 2;
    const int xs = per_head > 0 && npairs % per_head == 0 ? per_head : 0;
    const dim3 bgrid(npairs * Hkv), bblock(prefill::BAL_WAVES * WAVE);
    if (kv8)
      prefill::attn_prefill_bal_kernel<true><<<bgrid, bblock, 0, stream>>>(
          Q, kc, vc, pos, QG, ldp, O, ldo, T, Hq, Hkv, max_len, scale_log2, v_scale, xs);
    else
      prefill::attn_prefill_bal_kernel<false><<<bgrid, bblock, 0, stream>>>(
          Q, kc, vc, pos, QG, ldp, O, ldo, T, Hq, Hkv, max_len, scale_log2, 1.f, xs);
    return hipGetLastError();
  }
  if (kv8)
    prefill::attn_prefill_kernel<true><<<grid, block, 0, stream>>>(
        Q, kc, vc, pos, QG, ldp, O, ldo, T, Hq, Hkv, max_len, scale_log2, v_scale, xcd_split);
  else
    prefill::attn_prefill_kernel<false><<<grid, block, 0, stream>>>(
        Q, kc, vc, pos, QG, ldp, O, ldo, T, Hq, Hkv, max_len, scale_log2, 1.f, xcd_split);
  return hipGetLastError();
}

extern "C" hipError_t qe_attn_prefill(const void* q, const void* kc, const void* vc,
                                      const int* pos, const void* qg, long ldp, void* out,
                                      long ldo, int T, int Hq, int Hkv, int max_len, float scale,
                                      hipStream_t stream) {
  return launch_prefill(q, kc, vc, pos, qg, ldp, out, ldo, T, Hq, Hkv, max_len, scale, false, 1.f,
                        1.f, stream);
}

extern "C" hipError_t qe_attn_prefill_fp8(const void* q, const void* kc8, const void* vc8,
                                          const int* pos, const void* qg, long ldp, void* out,
                                          long ldo, int T, int Hq, int Hkv, int max_len,
                                          float scale, float k_scale, float v_scale,
                                          hipStream_t stream) {
  if (!kv_scale_ok(k_scale) || !kv_scale_ok(v_scale))
    return hipErrorInvalidValue;
  return launch_prefill(q, kc8, vc8, pos, qg, ldp, out, ldo, T, Hq, Hkv, max_len, scale, true,
                        k_scale, v_scale, stream);
}
