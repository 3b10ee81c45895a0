// Persistent grouped GEMM for the expert FFN forward on MI355X (gfx950).
//
//   out[q, p] = sum_k act[q, k] * w[e(q), p, k]        (k contiguous in both)
//
// q runs over routed token rows grouped by expert (ragged segments), p over
// weight rows.  Used for the w13 up-projection with SwiGLU fused into the
// epilogue, for the w2 down-projection with the routing-weight scale and the
// un-permute scatter fused into the epilogue, and for the plain grouped GEMM.
//
// Tile: up to 320 token rows (Q) x 256 weight rows (P); k in stages of 64.
//   * 8 waves, two per SIMD, in a 2 x 4 arrangement: wave (wq, wp) owns 64
//     weight rows and the tile's 32-row token blocks wq, wq + 2, ... (up to
//     5 of them, 2 x 5 accumulators of v_mfma_f32_32x32x16_bf16, 160 fp32
//     registers per lane).  The block count follows the tile's height (the
//     k loop is instantiated per count), so a 256-row tile costs 256 rows of
//     MFMA, LDS reads and token-row DMA, not 320.  The MFMA A operand is the
//     weight tile, B the token tile, so a lane holds 4 consecutive output
//     columns per register group.  SWIGLU: a wave's weight rows are 32 gate
//     rows and the 32 matching up rows.
//   * Two LDS stage buffers of 72 KB (32 KB weights + 40 KB tokens, rows of
//     128 bytes = one full cache line per row and stage) filled by
//     global_load_lds_dwordx4 (HBM/L2 -> LDS without VGPR staging).  A DMA
//     instruction moves 8 whole rows; half-line rows (k stages of 32) cost
//     twice the L2 requests per byte and capped the load rate.  The 16-byte
//     chunk c of row r sits at c ^ ((r ^ (r >> 3)) & 7): the 8 (and 16)
//     consecutive rows a fragment read serves per LDS cycle hit distinct
//     banks.  A wave's DMA writes 1 KB of LDS contiguously, so the
//     permutation is applied to the global addresses.
//   * MFMA fragments are read one k16 step ahead; the single barrier of a
//     stage sits before its last k16 step, after the last reads of the stage,
//     and is where the next-but-one stage's weight rows are issued into the
//     freed buffer; its token rows follow one k16 step later.
//   * Per tile, a wave-uniform byte base (SGPRs) plus one 32-bit per-lane
//     offset per DMA instruction; per stage only the k offset changes.
//   * Persistent: one workgroup per CU walks the tile list with stride
//     gridDim.x; the DMA stream runs over the flattened (tile, k-stage)
//     sequence, so the next tile's first stages load during the current
//     tile's epilogue.  Within a round the 32 workgroups of one XCD take 32
//     consecutive tiles (same expert), so the weights are shared in its L2
//     (the SwiGLU kernels walk the token tiles in pairs, see tile_at).
//   * Tail split: for a walk of at most six full rounds, the tiles left
//     over after the last full round are cut along k into up to 8 pieces
//     that run on the otherwise idle workgroups; every piece writes its fp32
//     accumulators to the workspace and counts its arrival (agent-scope
//     release / atomic / acquire, as the XCDs' L2s are not coherent), and
//     the last piece to arrive streams all partials back through LDS in
//     piece order, so the sum does not depend on arrival order, and runs the
//     ordinary epilogue.
//
// Reference semantics (torchtitanturbo/models/common/npu_gmm.py):
//   :17-18, :31, :38  torch._grouped_mm(x, w.transpose(-2, -1), offs)
//   :32-36            optional clamp with swiglu_limit
//   :37               npu_swiglu: silu(gate) * up, gate = first H columns
#include <cstddef>
#include <cstdlib>
#include <type_traits>

#include "common.h"
#include "dma_asm.h"
#include "gemm_common.h"
#include "kernels.h"

namespace ttamd {
namespace {

using namespace dma;

constexpr int TQ = kFwdTileRows;  // 320 token rows
constexpr int TP = 256;           // weight rows
constexpr int WAVES = 8;          // 2 per SIMD
constexpr int WPN = WAVES / 2;    // waves along the weight rows (2 along the token rows)
constexpr int NJ = TQ / 64;       // 32-row token blocks per wave
constexpr int NPB = TP / 32 / WPN;  // 32-row weight blocks per wave
constexpr int TK = 64;            // k per stage: 128-byte rows
constexpr int NSTAGE = 2;
constexpr int FTHREADS = 64 * WAVES;
constexpr int ROW_BYTES = TK * 2;
constexpr int P_BYTES = TP * ROW_BYTES;                // 32 KB
constexpr int STAGE_BYTES = P_BYTES + TQ * ROW_BYTES;  // 72 KB
constexpr int LDS_BYTES = NSTAGE * STAGE_BYTES;        // 144 KB
constexpr int DMA_P = TP / 8 / WAVES;                  // 4 weight-row instructions per wave
constexpr int DMA_Q = TQ / 8 / WAVES;                  // 5 token-row instructions per wave
constexpr int DMA_PER_STAGE = DMA_P + DMA_Q;           // 9 per lane
static_assert(TQ % 64 == 0 && TP == 256 && TQ % (8 * WAVES) == 0 && NPB % 2 == 0, "tile geometry");
// EPI_SCATTER row metadata (destination row, scale) of a tile, DMA'd with
// the tile's first stage into one of three LDS slots (tile round % 3): the
// slot of round r + 3 is written only after round r's epilogue.
constexpr int META_BYTES = TQ * 8;
// Gathered token rows (q_index): the tile's source-row ids, DMA'd one tile
// ahead into one of two LDS slots (tile round % 2).
constexpr int IDX_OFF = LDS_BYTES + 3 * META_BYTES;
constexpr int IDX_BYTES = TQ * 4;
constexpr int LDS_TOTAL = IDX_OFF + 2 * IDX_BYTES;  // 154 KB
// Split tail tiles: whether this workgroup's piece arrived last, in the
// stage buffers (free by then) past the ring the partial sums stream through.
constexpr int FLAG_OFF = 8 * 16 * 1024;
static_assert(FLAG_OFF + 16 <= LDS_BYTES, "flag inside the stage buffers");
static_assert(kSplitPartBytes == (size_t)WAVES * NJ * NPB * 16 * 64 * 4, "partial-sum area of a piece");

typedef short short4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4_t lds_short4_t;
typedef __attribute__((address_space(1))) int gint_t;
typedef __attribute__((address_space(1))) floatx4_t gfloatx4_t;

// Chunk permutation of the 512-byte reduction-major weight rows (PT): the
// 8 rows n0..n0+3, n0+8..n0+11 one transposed read touches land on four
// distinct 64-byte bank groups, two rows each.
__device__ __forceinline__ int ptswz(int n) { return 4 * ((n ^ (n >> 3)) & 3); }

// MFMA fragments of one k16 step: NPB weight blocks, NJ token blocks.
struct Frag {
  bf16x8_t a[NPB];
  bf16x8_t b[NJ];
};

// PT (dgrad): the weight operand is reduction-major, w[e][n][k] with the
// reduction n as rows and the output index k contiguous.  Its stage is 64
// rows of TP * 2 = 512 bytes (n rows of the tile's 256 output columns), the
// 16-byte chunk c of row n stored at c ^ ptswz(n), and the MFMA A fragments
// (8 consecutive n for one output column) come from two
// ds_read_b64_tr_b16 per block: within each 16-lane group, lane i receives
// element i % 4 of the 4 loaded by lane 4c + i / 4, for c = 0..3, so lane
// src points at row n0 + src / 4, columns r0 + 4 (src % 4) .. + 3, and lane
// i receives rows n0 .. n0 + 3 of column r0 + i.
// GATHER (inference w13): token row j is q row q_index[j] / q_div.
template <int EPI, bool PT, bool GATHER>
__global__ __launch_bounds__(FTHREADS, 1) void gg_fwd_kernel(const FwdArgs a) {
  extern __shared__ __attribute__((aligned(1024))) char smem[];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wq = w / WPN;
  const int wp = w % WPN;
  const int l = threadIdx.x & 63;
  const int G = gridDim.x;
  const int b = blockIdx.x;
  // XCD-aware slot: hardware block ids go round-robin over the 8 XCDs; give
  // XCD x the slots [x*G/8, (x+1)*G/8) so that it takes consecutive tiles.
  const int slot = (b & 7) * (G >> 3) + (b >> 3);
  const int nqt = sload_int(a.n_qtiles);
  const int ntiles = nqt * a.np_tiles;
  // (the schedule scalars are pinned to SGPRs: divisions are expanded in
  // VALU, and the stage advance in issue_p must stay scalar)
  auto U = [](int v) { return __builtin_amdgcn_readfirstlane(v); };
  const int ksteps = U(a.kred / TK);
  // Tail split: the walk has R full rounds of G tiles and rt tiles left
  // over.  Unsplit, rt workgroups run one more whole tile while the others
  // idle.  Split, each leftover tile is cut along k into np pieces of
  // consecutive stages, piece j of leftover tile t taken by slot j * rt + t
  // (so one XCD's slots run the same k range of neighbouring tiles), and
  // every slot runs R whole tiles, then at most one piece.
  const int R = U(ntiles / G);
  const int rt = ntiles - R * G;
  int np = 1;
  if (a.part != nullptr && rt > 0 && rt <= kSplitTiles && R <= kSplitMaxRounds) {
    np = max(1, min(min(G / rt, a.split_max), ksteps / kSplitMinStages));
    // the last piece reads np partials: keep np at most sqrt(ksteps / 2),
    // and two pieces only for long reductions
    while (np > 1 && ksteps < 2 * np * np) --np;
    if (np == 2 && ksteps < 64) np = 1;
    np = U(np);
  }
  const bool has_piece = np > 1 && slot < rt * np;
  const int nfull = U(np > 1 ? R : (slot < ntiles ? (ntiles - slot + G - 1) / G : 0));
  const int nmy = nfull + (has_piece ? 1 : 0);
  const int pc_t = has_piece ? slot % rt : 0;  // leftover tile of the piece
  const int pc_j = has_piece ? slot / rt : 0;  // piece index
  const int pc_k0 = U(pc_j * ksteps / np);
  const int pc_k1 = U((pc_j + 1) * ksteps / np);
  const int pc_L = U(R * G + pc_t);  // its walk index
  // np, pc_j and pc_t in one register through the k loop (unpacked after it)
  const int pc_info = U(np | (pc_j << 8) | (pc_t << 16));
  // Persistent order of the SwiGLU (w13) kernels: token tiles in pairs,
  // weight tile major inside a pair, so 32 consecutive slots (one XCD's)
  // take both token tiles of an expert with 16 weight tiles rather than one
  // token tile with 32: each weight tile is shared in the XCD's L2 instead
  // of across XCDs (C3 w13 -6 %; the other epilogues' kernels were slower
  // with it and keep the table order).  Returns the table order's tile id
  // (qt * np_tiles + pt).
  auto tile_at = [&](int r) {
    const int L = r < nfull ? r * G + slot : pc_L;
    if constexpr (EPI != EPI_SWIGLU) return L;
    const int blk = L / (2 * a.np_tiles);
    const int in_blk = L - blk * 2 * a.np_tiles;
    const int gq = min(2, nqt - 2 * blk);
    const int pt = in_blk / gq;
    return (2 * blk + (in_blk - pt * gq)) * a.np_tiles + pt;
  };
  const int total = nfull * ksteps + (has_piece ? pc_k1 - pc_k0 : 0);
  if (total == 0) return;

  const uint32_t lds0 = lds_addr(smem);
  // DMA lane geometry: instruction i of wave w (per operand) writes the 8
  // rows of row block rb = WAVES*i + w, row 8rb + l / 8, physical chunk l % 8,
  // whose logical chunk is l % 8 ^ cswz(row) = l % 8 ^ ((l / 8 ^ rb) & 7).
  const int drow = l >> 3;

  // ---- DMA stream -----------------------------------------------------------
  // Source-row ids of tile round r (gathered rows only): 64-row chunk c of
  // the tile is moved by wave c % WAVES into slot r % 2.
  auto load_ids = [&](int r) {
    const int tile = tile_at(r);
    const int4 ti = sload_int4(a.table + tile / a.np_tiles);
    for (int c = w; c < TQ / 64; c += WAVES) {
      const uint32_t q = (uint32_t)min(64 * c + l, ti.z - ti.y - 1);
      dma4(q * 4, (uint64_t)(a.q_index + ti.y), lds0 + IDX_OFF + (uint32_t)((r & 1) * IDX_BYTES) + c * 256);
    }
  };
  int d_r = -1;  // tile round whose addresses are loaded
  int d_qblk8 = 0;  // 8-row token blocks the MFMA reads: 4 * ceil(rows / 32)
  int d_pmax = 0, d_qmax = 0;  // last valid weight / token row of the tile (tile-relative)
  uint64_t d_pbase = 0, d_qbase = 0;
  // Row-major operands: instruction i of wave w moves rows rr0 + 64 i with
  // the same chunk permutation (row block 8 i + w has (8 i + w) & 7 = w), so
  // its per-lane offset is recomputed at issue from two lane constants and
  // the tile's uniform clamps, instead of occupying a register per
  // instruction through the k loop.  Per-lane offsets that are not affine
  // in i (transposed weights, gathered token rows) are kept per tile.
  static_assert(WAVES == 8, "row block 8 i + w has chunk permutation term w");
  const int rr0 = 8 * w + drow;
  const uint32_t lch16 = (uint32_t)(((l & 7) ^ ((drow ^ w) & 7)) * 16);
  uint32_t d_ptoff[PT ? DMA_P : 1];
  uint32_t d_gqoff[GATHER ? DMA_Q : 1];
  auto dma_tile = [&](int r) {
    const int tile = tile_at(r);
    const int qt = tile / a.np_tiles;
    const int pt = tile - qt * a.np_tiles;
    const int4 ti = sload_int4(a.table + qt);
    const int64_t ldp2 = a.ldp * 2;
    const int qmax = ti.z - ti.y - 1;
    d_qblk8 = 4 * ((ti.z - ti.y + 31) >> 5);
    d_qmax = qmax;
    if constexpr (PT) {
#pragma unroll
      for (int i = 0; i < DMA_P; ++i) {
        // instruction i of wave w: rows 2 (WAVES i + w) and + 1, 32 chunks each
        const int row = 2 * (WAVES * i + w) + (l >> 5);
        const int lc = (l & 31) ^ ptswz(row);
        const int col = min(pt * TP + 8 * lc, a.n_p - 8) - pt * TP;
        d_ptoff[i] = (uint32_t)(row * ldp2 + col * 2);
      }
    } else {
      d_pmax = a.n_p - 1 - pt * (EPI == EPI_SWIGLU ? 128 : TP);
    }
    if constexpr (GATHER) {
      // Gathered rows: tile row rr reads source row q_index[row] / q_div,
      // whose id was DMA'd into LDS while the previous tile was issued.
      const int* ids = (const int*)(smem + IDX_OFF + (r & 1) * IDX_BYTES);
#pragma unroll
      for (int i = 0; i < DMA_Q; ++i) {
        const int src = min(max(ids[min(rr0 + 64 * i, qmax)] / a.q_div, 0), a.n_q_in - 1);
        d_gqoff[i] = (uint32_t)(src * a.ldq * 2) + lch16;
      }
      if (r + 1 < nmy) load_ids(r + 1);
    }
    if constexpr (PT)
      d_pbase = (uint64_t)(a.p + (int64_t)ti.x * a.p_estride + (int64_t)pt * TP);
    else if constexpr (EPI == EPI_SWIGLU)
      d_pbase = (uint64_t)(a.p + (int64_t)ti.x * a.p_estride + (int64_t)pt * 128 * a.ldp);
    else
      d_pbase = (uint64_t)(a.p + (int64_t)ti.x * a.p_estride + (int64_t)pt * TP * a.ldp);
    d_qbase = (uint64_t)(a.q + (GATHER ? 0 : (int64_t)ti.y * a.ldq));
    if constexpr (EPI == EPI_SCATTER) {
      for (int c = w; c < TQ / 64; c += WAVES) {
        const uint32_t q = (uint32_t)min(64 * c + l, qmax);
        const uint32_t m = lds0 + LDS_BYTES + (uint32_t)((r % 3) * META_BYTES) + c * 256;
        if (a.dest) dma4(q * 4, (uint64_t)(a.dest + ti.y), m);
        if (a.row_scale) dma4(q * 4, (uint64_t)(a.row_scale + ti.y), m + TQ * 4);
      }
    }
    d_r = r;
  };
  // A stage's DMA is issued in two parts: the weight rows (P) at the stage
  // barrier that frees their buffer, the token rows (Q) one k16 step later
  // (see the k loop).  issue_p sets the stage's bases, which issue_q reads.
  uint64_t d_spb = 0, d_sqb = 0;
  uint32_t d_sst = 0;
  // issue_p is called for stages 0, 1, 2, ... in order: the (unit, k stage)
  // of the next one is advanced here rather than divided out per call.
  // Past the end the last stage is issued again.
  int n_r = 0, n_ks = nfull > 0 ? 0 : pc_k0, n_kend = nfull > 0 ? ksteps : pc_k1, n_left = total;
  auto issue_p = [&](int s) {
    const int r = n_r, ks = n_ks;
    if (r != d_r) dma_tile(r);
    d_spb = d_pbase + (PT ? (uint64_t)ks * TK * a.ldp * 2 : (uint64_t)ks * ROW_BYTES);
    d_sqb = d_qbase + (uint64_t)ks * ROW_BYTES;
    d_sst = lds0 + (uint32_t)((s & 1) * STAGE_BYTES) + w * 1024;
    const uint32_t ldp2 = (uint32_t)a.ldp * 2u;
#pragma unroll
    for (int i = 0; i < DMA_P; ++i) {
      uint32_t voff;
      if constexpr (PT) {
        voff = d_ptoff[i];
      } else if constexpr (EPI == EPI_SWIGLU) {
        // rows 0..127 gate, 128..255 up: tile row rr is weight row pt * 128 +
        // (rr & 127), of the up half (hidden + ...) for rr >= 128
        const int col = min(rr0 + 64 * (i & 1), d_pmax);
        voff = (uint32_t)(i < 2 ? col : (int)a.hidden + col) * ldp2 + lch16;
      } else {
        voff = (uint32_t)min(rr0 + 64 * i, d_pmax) * ldp2 + lch16;
      }
      dma16(voff, d_spb, d_sst + i * (WAVES * 1024));
    }
    // Advance to the next stage only now: whatever sits between the stage
    // barrier and these DMAs delays every stage (the empty asm keeps the
    // compiler from hoisting the update above them).  Selects, no branches.
    n_left = __builtin_amdgcn_readfirstlane(n_left);
    n_ks = __builtin_amdgcn_readfirstlane(n_ks);
    n_kend = __builtin_amdgcn_readfirstlane(n_kend);
    n_r = __builtin_amdgcn_readfirstlane(n_r);
    asm volatile("" : "+s"(n_left), "+s"(n_ks), "+s"(n_kend), "+s"(n_r));
    const int adv = n_left > 1 ? 1 : 0;
    n_left -= adv;
    const int nk = n_ks + adv;
    const bool wrap = nk == n_kend;
    n_r += wrap ? 1 : 0;
    const bool full = n_r < nfull;
    n_ks = wrap ? (full ? 0 : pc_k0) : nk;
    n_kend = wrap ? (full ? ksteps : pc_k1) : n_kend;
  };
  // Token rows past the tile's last 32-row block are never read: skip
  // their DMA (wave-uniform: instruction i moves row block WAVES * i + w).
  auto issue_q = [&]() {
    const uint32_t ldq2 = (uint32_t)a.ldq * 2u;
#pragma unroll
    for (int i = 0; i < DMA_Q; ++i) {
      if (WAVES * i + w < d_qblk8) {
        const uint32_t voff = GATHER ? d_gqoff[GATHER ? i : 0] : (uint32_t)min(rr0 + 64 * i, d_qmax) * ldq2 + lch16;
        dma16(voff, d_sqb, d_sst + P_BYTES + i * (WAVES * 1024));
      }
    }
  };
  auto issue = [&](int s) {
    issue_p(s);
    issue_q();
  };

  // ---- fragment geometry -------------------------------------------------------
  // Row 32m + r32 has cswz = fa ^ 4 * (m & 1) with fa = cswz(r32); all
  // fragment blocks start at multiples of 32 rows.
  const int r32 = l & 31;
  const int half = l >> 5;
  const int fa = cswz(r32);
  // SWIGLU: blocks pb < NPB/2 are gate rows, pb + NPB/2 the matching up rows.
  int arow[NPB];
#pragma unroll
  for (int pb = 0; pb < NPB; ++pb)
    arow[pb] = (EPI == EPI_SWIGLU)
                   ? (pb < NPB / 2 ? (128 / WPN) * wp + 32 * pb : 128 + (128 / WPN) * wp + 32 * (pb - NPB / 2))
                   : (TP / WPN) * wp + 32 * pb;
  // PT: lane l of 16-lane group g = (l >> 4) & 3 loads row
  // 16 kk + 8 (g >> 1) + 4 t + (l & 15) / 4, columns arow + 16 (g & 1) +
  // 4 (l & 3) .. + 3 (t = 0, 1: the two halves of its 8 reduction values).
  // With n = 16 kk + tr_row + 4 t, ptswz(n) = 4 (bsw ^ 2 (kk & 1)) for a
  // per-lane bsw, so each (block, kk parity) has one per-lane chunk offset
  // and kk, t only move the row by constants.
  const int tr_row = 8 * ((l >> 5) & 1) + ((l & 15) >> 2);
  const int tr_col = 16 * ((l >> 4) & 1) + 4 * (l & 3);
  const int bsw = ((l >> 2) & 3) ^ ((l >> 5) & 1);
  int trx[PT ? NPB : 1][2];
  if constexpr (PT) {
#pragma unroll
    for (int pb = 0; pb < NPB; ++pb)
#pragma unroll
      for (int par = 0; par < 2; ++par)
        trx[pb][par] = tr_row * (TP * 2) + ((tr_col & 4) << 1) +
                       ((((arow[pb] + tr_col) >> 3) ^ (4 * (bsw ^ (2 * par)))) << 4);
  }
  // Token block j of wave wq is the tile's 32-row block m = 2j + wq, so the
  // chunk permutation term 4 * (m & 1) is 4 * wq for every block of a wave.
  // njv (an integral constant) is the wave's block count in this tile.
  auto read_frag = [&](Frag& f, int s, int kk, auto njv) {
    constexpr int NJV = decltype(njv)::value;
    if constexpr (NJV == 0) return;
    const char* st = smem + (s & 1) * STAGE_BYTES;
#pragma unroll
    for (int pb = 0; pb < NPB; ++pb) {
      if constexpr (PT) {
        short4_t v[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int off = trx[pb][kk & 1] + (16 * kk + 4 * t) * (TP * 2);
          v[t] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_t*)(st + off));
        }
        f.a[pb] = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(v[0], v[1], 0, 1, 2, 3, 4, 5, 6, 7));
        continue;
      }
      const int pc = (2 * kk + half) ^ fa ^ (4 * ((arow[pb] >> 5) & 1));
      f.a[pb] = *(const bf16x8_t*)(st + (arow[pb] + r32) * ROW_BYTES + pc * 16);
    }
#pragma unroll
    for (int j = 0; j < NJV; ++j) {
      const int pc = (2 * kk + half) ^ fa ^ (4 * wq);
      f.b[j] = *(const bf16x8_t*)(st + P_BYTES + (64 * j + 32 * wq + r32) * ROW_BYTES + pc * 16);
    }
  };

  // ---- prologue: stages 0 and 1 in flight, stage 0 landed -----------------------
  // (the token-row DMA count of a stage depends on its tile's height, so the
  // wait is for everything issued)
  if constexpr (GATHER) {
    load_ids(0);
    wait_vm_barrier<0>();
  }
  issue(0);
  issue(1);
  wait_vm_barrier<0>();

  int s = 0;
  // nks: the unit's k stages (ksteps for a whole tile); piece: the unit is
  // a piece of a split leftover tile.
  auto run_tile = [&](auto njv, int r, int row0, int row1, int pt, int nks, bool piece) {
    constexpr int NJV = decltype(njv)::value;
    Frag f0, f1;  // per tile: the first fragments are read at the tile's start
    read_frag(f0, s, 0, njv);
    constexpr int NJA = NJV > 0 ? NJV : 1;
    floatx16_t acc[NPB][NJA];
#pragma unroll
    for (int i = 0; i < NPB; ++i)
#pragma unroll
      for (int j = 0; j < NJA; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
    auto mfma = [&](const Frag& f) {
#pragma unroll
      for (int j = 0; j < NJV; ++j)
#pragma unroll
        for (int pb = 0; pb < NPB; ++pb)
          acc[pb][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[pb], f.b[j], acc[pb][j], 0, 0, 0);
    };
    // One stage: k16 steps 0..3, each computed from registers while the next
    // is read.  Before step 3 every wave has read all of stage s; the barrier
    // there also waits for stage s + 1 (the only stage in flight), and the
    // weight rows of stage s + 2 are issued into stage s's buffer at once;
    // its token rows follow one k16 step later, at the start of stage s + 1
    // (both have landed by that stage's barrier).  A tile's last stage
    // issues the whole next-but-one stage at its barrier, before the
    // epilogue.  Every wave runs the same barrier sequence whatever its
    // block count.
    for (int ks = 0; ks + 1 < nks; ++ks, ++s) {
      if (ks > 0) issue_q();
      read_frag(f1, s, 1, njv);
      mfma(f0);
      read_frag(f0, s, 2, njv);
      mfma(f1);
      read_frag(f1, s, 3, njv);
      mfma(f0);
      wait_vm_barrier<0>();
      issue_p(s + 2);
      read_frag(f0, s + 1, 0, njv);
      mfma(f1);
    }
    // Last stage of the tile: the next tile's first fragments are read at
    // the start of that tile, with its block count.
    if (nks > 1) issue_q();
    read_frag(f1, s, 1, njv);
    mfma(f0);
    read_frag(f0, s, 2, njv);
    mfma(f1);
    read_frag(f1, s, 3, njv);
    mfma(f0);
    wait_vm_barrier<0>();
    issue(s + 2);
    mfma(f1);
    ++s;

    // ---- split leftover tile: publish this piece's sums; the last piece
    //      to arrive adds all of them in piece order (the same order
    //      whichever arrives last) and runs the epilogue.  The partials are
    //      written back from this XCD's L2 (release) before the arrival is
    //      counted, and the last piece invalidates its caches (acquire)
    //      before it reads the others'.  The counter is reset for the next
    //      GEMM on this plan.
    if (__builtin_expect(piece, 0)) {  // (laid out away from the tile path)
      // Partial sums of leftover tile pc_t: np * kSplitPartBytes bytes at
      // part + pc_t * np * kSplitPartBytes, wave w's share (NPB * NJ blocks
      // of 4 KB per piece) at w * np * NPB * NJ * 4 KB, laid out block-major,
      // then piece, then the block's four 1 KB groups (lane l: 16 bytes at
      // 16 l).  The last piece then reads one contiguous stream per wave:
      // 1 KB chunk i is block i / (4 np), piece i / 4 % np, group i % 4.
      // The bases are made opaque here so that no address is computed (and
      // kept live) in the k loop.
      constexpr uint32_t BLK = 4 * 1024;
      // (re-read here rather than held through the k loop)
      int info = pc_info;
      asm volatile("" : "+s"(info));
      const int np = info & 0xff, pc_j = (info >> 8) & 0xff, pc_t = info >> 16;
      const int4 pc = sload_int4((const int4*)((const char*)__builtin_amdgcn_kernarg_segment_ptr() +
                                               offsetof(FwdArgs, part)));
      float* const part = (float*)(((uint64_t)(uint32_t)pc.y << 32) | (uint32_t)pc.x);
      // (global address space: global rather than flat atomics and stores)
      gint_t* const split_cnt = (gint_t*)(((uint64_t)(uint32_t)pc.w << 32) | (uint32_t)pc.z);
      uint64_t pw = (uint64_t)part + (uint64_t)pc_t * np * kSplitPartBytes + (uint64_t)w * np * (NPB * NJ * BLK);
      asm volatile("" : "+s"(pw));
      // the lane id re-derived here (mbcnt of an opaque zero, which the
      // compiler cannot hoist), not kept through the k loop
      uint32_t zero = 0;
      asm volatile("" : "+v"(zero));
      uint32_t loff = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, zero)) * 16u;
      asm volatile("" : "+v"(loff));
      const uint32_t bstride = (uint32_t)np * BLK;  // one block of every piece
#pragma unroll
      for (int pb = 0; pb < NPB; ++pb)
#pragma unroll
        for (int j = 0; j < NJV; ++j) {
          const uint64_t dst = pw + (uint64_t)((pb * NJV + j) * bstride + pc_j * BLK);
#pragma unroll
          for (int g = 0; g < 4; ++g)
            *(gfloatx4_t*)(dst + (uint32_t)(g * 1024) + loff) =
                floatx4_t{acc[pb][j][4 * g], acc[pb][j][4 * g + 1], acc[pb][j][4 * g + 2], acc[pb][j][4 * g + 3]};
        }
      wait_vm<0>();  // this wave's partial has reached L2
      __syncthreads();
      int* flag = (int*)(smem + FLAG_OFF);
      if (w == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        int old = 0;
        if (l == 0) old = __hip_atomic_fetch_add(split_cnt + pc_t, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        old = __builtin_amdgcn_readfirstlane(old);
        if (old == np - 1) {
          if (l == 0) __hip_atomic_store(split_cnt + pc_t, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
          // the cache invalidation has completed before the barrier below
          // lets the other waves load the partials
          wait_vm<0>();
        }
        if (l == 0) *flag = (old == np - 1);
      }
      __syncthreads();
      if (__builtin_amdgcn_readfirstlane(*flag) == 0) return;
      // The sum in piece order.  Each wave streams its share through a ring
      // of 16 one-KB LDS slots (the free stage buffers) with LDS DMA, 16 KB
      // in flight and no VGPRs held for it: chunk i goes to slot i % 16, and
      // exactly one DMA is issued per chunk consumed (past the end: the last
      // chunk again, into the slot just read), so "at most 15 in flight"
      // means chunk i has landed.
      if constexpr (NJV > 0) {
#pragma unroll
        for (int pb = 0; pb < NPB; ++pb)
#pragma unroll
          for (int j = 0; j < NJV; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[pb][j][v] = 0.f;
        constexpr int RING = 16;
        const int last = NPB * NJV * 4 * np - 1;
        const uint32_t ring = lds0 + (uint32_t)w * (RING * 1024);
        auto fetch = [&](int i) {
          dma16(loff, pw + (uint32_t)min(i, last) * 1024u, ring + (uint32_t)(i & (RING - 1)) * 1024u);
        };
#pragma unroll
        for (int i = 0; i < RING; ++i) fetch(i);
        const char* rbase = smem + w * (RING * 1024) + 16 * l;
        int i = 0;
#pragma unroll
        for (int pb = 0; pb < NPB; ++pb)
#pragma unroll
          for (int j = 0; j < NJV; ++j)
            for (int q = 0; q < np; ++q) {
#pragma unroll
              for (int g = 0; g < 4; ++g) {
                wait_vm<RING - 1>();
                const float4 v = *(const float4*)(rbase + (i & (RING - 1)) * 1024);
                acc[pb][j][4 * g] += v.x;
                acc[pb][j][4 * g + 1] += v.y;
                acc[pb][j][4 * g + 2] += v.z;
                acc[pb][j][4 * g + 3] += v.w;
                fetch(i + RING);  // after the adds: the slot's read has completed
                ++i;
              }
            }
        wait_vm<0>();
      }
    }

    // ---- epilogue: acc[pb][j][4g + i] is (token row 64j + 32wq + r32,
    //      weight row arow[pb] + 8g + 4 * half + i).  Column validity is
    //      wave-uniform (H % 64 == 0 and N % 128 == 0 are required), row
    //      validity is per lane.  The scheduling barriers keep each block's
    //      accumulator reads next to their use (no 256-register hoist).
    //      The lane row is re-materialised here (opaque copy) so that the
    //      compiler does not keep per-block row offsets live across the k
    //      loop, where every register is taken.
    int er32 = r32;
    asm volatile("" : "+v"(er32));
    int ehalf = half;  // likewise for the lane's column half (store addresses)
    asm volatile("" : "+v"(ehalf));
    // EPI_SWIGLU_BWD: saved pre-activation of token block jj
    auto load_h = [&](int jj, int pb, uint2 (&dst)[4][2]) {
      if constexpr (EPI == EPI_SWIGLU_BWD) {
        const int gq = row0 + 64 * jj + 32 * wq + er32;
        const int qrow = min(gq, row1 - 1);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int col = min(pt * TP + arow[pb], a.n_p - 32) + 8 * g + 4 * half;
          const bf16_t* hrow = a.h_in + (int64_t)qrow * a.ldh + col;
          dst[g][0] = *(const uint2*)hrow;
          dst[g][1] = *(const uint2*)(hrow + a.hidden);
        }
      }
    };
    // EPI_SWIGLU_BWD: the h values of block (j, pb) are loaded one block
    // ahead, into the other half of hbuf (double buffer).
    uint2 hbuf[2][4][2];
    if constexpr (EPI == EPI_SWIGLU_BWD) load_h(0, 0, hbuf[0]);
#pragma unroll
    for (int j = 0; j < NJV; ++j) {
      const int gq = row0 + 64 * j + 32 * wq + er32;
      const bool row_ok = gq < row1;
      if constexpr (EPI == EPI_SWIGLU) {
        const float L = a.limit;
        // The clamp (swiglu_limit) is wave-uniform: one code path each, so
        // that the unclamped SwiGLU carries no min / max / select per value.
        // Per 32-column block: gate and up are rounded to bf16 two at a time
        // (one two-wide conversion each; the bf16 pairs are what h_out
        // stores), then the row's stores share one address and one branch.
        auto swiglu_rows = [&](auto clampc) {
          constexpr bool CLAMP = decltype(clampc)::value;
#pragma unroll
          for (int pb = 0; pb < NPB / 2; ++pb) {
            uint32_t ap[4][2], gp[4][2], up[4][2];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
#pragma unroll
              for (int i2 = 0; i2 < 2; ++i2) {
                // h is materialised in bf16 by the reference; SwiGLU reads it.
                const int v = 4 * g + 2 * i2;
                gp[g][i2] = pack_bf16x2(acc[pb][j][v], acc[pb][j][v + 1]);
                up[g][i2] = pack_bf16x2(acc[pb + NPB / 2][j][v], acc[pb + NPB / 2][j][v + 1]);
                float av[2];
#pragma unroll
                for (int h2 = 0; h2 < 2; ++h2) {
                  float gc = __uint_as_float(h2 ? (gp[g][i2] & 0xffff0000u) : (gp[g][i2] << 16));
                  float uc = __uint_as_float(h2 ? (up[g][i2] & 0xffff0000u) : (up[g][i2] << 16));
                  if constexpr (CLAMP) {
                    gc = clamp_max_nan(gc, L);
                    uc = clamp_nan(uc, L);
                  }
                  av[h2] = silu_f(gc) * uc;
                }
                ap[g][i2] = pack_bf16x2(av[0], av[1]);
              }
            }
            if (row_ok) {
              const int col = pt * 128 + (128 / WPN) * wp + 32 * pb + 4 * half;
              bf16_t* orow = a.out + (int64_t)gq * a.ldo + col;
#pragma unroll
              for (int g = 0; g < 4; ++g) *(uint2*)(orow + 8 * g) = make_uint2(ap[g][0], ap[g][1]);
              if (a.h_out) {
                bf16_t* hrow = a.h_out + (int64_t)gq * a.ldh + col;
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                  *(uint2*)(hrow + 8 * g) = make_uint2(gp[g][0], gp[g][1]);
                  *(uint2*)(hrow + a.hidden + 8 * g) = make_uint2(up[g][0], up[g][1]);
                }
              }
            }
            __builtin_amdgcn_sched_barrier(0);
          }
        };
        if (pt * 128 + (128 / WPN) * wp < a.n_p) {
          if (a.limit == a.limit)
            swiglu_rows(std::true_type{});
          else
            swiglu_rows(std::false_type{});
        }
      } else if constexpr (EPI == EPI_SWIGLU_BWD) {
        // acc = dA = g for output columns p of the activation; with the saved
        // bf16 pre-activation h = [gate | up]: dgate, dup (clamp masks from
        // the bf16 h, as the reference's autograd sees them).  The 8 h values
        // of a 32-column block are loaded before any is used.
        // Without a clamp the limit is +inf: minimum / maximum against it are
        // exact no-ops (NaN included) and the masks are forced true, so the
        // value loop has no branch on the clamp.
        const bool noclamp = !(a.limit == a.limit);
        const float L = noclamp ? __builtin_inff() : a.limit;
#pragma unroll
        for (int pb = 0; pb < NPB; ++pb) {
          const int blk = j * NPB + pb;
          if (blk + 1 < NJV * NPB) load_h((blk + 1) / NPB, (blk + 1) % NPB, hbuf[(blk + 1) & 1]);
          const uint2 (&hv)[4][2] = hbuf[blk & 1];
          if (pt * TP + arow[pb] < a.n_p && row_ok) {
            const int col0 = pt * TP + arow[pb] + 4 * half;
            bf16_t* drow = a.out + (int64_t)gq * a.ldo + col0;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              const uint2 hg = hv[g][0];
              const uint2 hu = hv[g][1];
              const float gate[4] = {bf16_to_f32(hg.x & 0xffff), bf16_to_f32(hg.x >> 16),
                                     bf16_to_f32(hg.y & 0xffff), bf16_to_f32(hg.y >> 16)};
              const float up[4] = {bf16_to_f32(hu.x & 0xffff), bf16_to_f32(hu.x >> 16),
                                   bf16_to_f32(hu.y & 0xffff), bf16_to_f32(hu.y >> 16)};
              float dg[4], du[4], av[4];
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                const float gd = acc[pb][j][4 * g + i];
                float gc = gate[i], uc = up[i];
                // torch.clamp's backward: where(in range, grad, 0), so exactly
                // zero where it clamped and where h is NaN
                const bool kg = noclamp | (gc <= L);
                const bool ku = noclamp | ((uc >= -L) & (uc <= L));
                gc = clamp_max_nan(gc, L);
                uc = clamp_nan(uc, L);
                const float sig = sigmoid_f(gc);
                const float sv = gc * sig;
                const float ds = sig * (1.f + gc * (1.f - sig));
                dg[i] = kg ? gd * uc * ds : 0.f;
                du[i] = ku ? gd * sv : 0.f;
                av[i] = sv * uc;
              }
              *(uint2*)(drow + 8 * g) = make_uint2(pack_bf16x2(dg[0], dg[1]), pack_bf16x2(dg[2], dg[3]));
              *(uint2*)(drow + a.hidden + 8 * g) =
                  make_uint2(pack_bf16x2(du[0], du[1]), pack_bf16x2(du[2], du[3]));
              if (a.a_out) {
                bf16_t* arow_p = a.a_out + (int64_t)gq * a.hidden + col0 + 8 * g;
                *(uint2*)arow_p = make_uint2(pack_bf16x2(av[0], av[1]), pack_bf16x2(av[2], av[3]));
              }
              __builtin_amdgcn_sched_barrier(0);
            }
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {
        float sc = 1.f;
        int orow_idx = gq;
        if constexpr (EPI == EPI_SCATTER) {
          const int* meta = (const int*)(smem + LDS_BYTES + (r % 3) * META_BYTES);
          const int qrow = 64 * j + 32 * wq + er32;
          if (a.dest) orow_idx = min(max(meta[qrow], 0), a.n_dest - 1);
          if (a.row_scale) {
            sc = __int_as_float(meta[TQ + qrow]);
            if (a.scale_sigmoid) sc = sigmoid_f(sc);
          }
        }
        bf16_t* orow = a.out + (int64_t)orow_idx * a.ldo;
#pragma unroll
        for (int pb = 0; pb < NPB; ++pb) {
          if (pt * TP + arow[pb] < a.n_p) {
            const floatx16_t& v = acc[pb][j];
            uint32_t pk[4][2];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              pk[g][0] = pack_bf16x2(v[4 * g] * sc, v[4 * g + 1] * sc);
              pk[g][1] = pack_bf16x2(v[4 * g + 2] * sc, v[4 * g + 3] * sc);
            }
            // Lanes l and l ^ 32 hold the same output row, half h holding
            // columns 8g + 4h .. + 3 of group g.  Swapping one group each
            // way leaves lane half h with columns 16c + 8h .. + 7 (c = 0, 1),
            // so every store is 16 bytes and 32 contiguous bytes per row.
            // v_permlane32_swap(x, y) exchanges x of lanes 32..63 with y of
            // lanes 0..31: with x = group 2c and y = group 2c + 1, the low
            // half ends with {own 2c, partner's 2c} (columns 16c .. + 7) and
            // the high half with {partner's 2c + 1, own 2c + 1}
            // (columns 16c + 8 .. + 15), both in (x, y) order.
#pragma unroll
            for (int c = 0; c < 2; ++c) {
              uint32_t x[2], y[2];
#pragma unroll
              for (int d = 0; d < 2; ++d) {
                const auto sw = __builtin_amdgcn_permlane32_swap(pk[2 * c][d], pk[2 * c + 1][d], false, false);
                x[d] = sw[0];
                y[d] = sw[1];
              }
              const u32x4_t val = u32x4_t{x[0], x[1], y[0], y[1]};
              const int col = pt * TP + arow[pb] + 16 * c + 8 * ehalf;
              if (row_ok) {
                if (a.accumulate) {
                  // add to the row already there (bf16 + bf16, one rounding)
                  const u32x4_t prev = *(const u32x4_t*)(orow + col);
                  u32x4_t sum;
#pragma unroll
                  for (int d = 0; d < 4; ++d)
                    sum[d] = pack_bf16x2(bf16_to_f32(val[d] & 0xffffu) + bf16_to_f32(prev[d] & 0xffffu),
                                         bf16_to_f32(val[d] >> 16) + bf16_to_f32(prev[d] >> 16));
                  *(u32x4_t*)(orow + col) = sum;
                } else {
                  *(u32x4_t*)(orow + col) = val;
                }
              }
            }
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
  };

  for (int r = 0; r < nmy; ++r) {
    const int tile = tile_at(r);
    const int qt = tile / a.np_tiles;
    const int pt = tile - qt * a.np_tiles;
    const int4 ti = sload_int4(a.table + qt);
    // 32-row blocks of the tile (at most TQ / 32), interleaved over the two
    // token-row waves: wave wq takes blocks wq, wq + 2, ...
    const int nj = min((((ti.z - ti.y + 31) >> 5) + 1 - wq) >> 1, NJ);
    const bool piece = r >= nfull;
    const int nks = piece ? pc_k1 - pc_k0 : ksteps;
    switch (nj) {
      case 5: run_tile(std::integral_constant<int, 5>{}, r, ti.y, ti.z, pt, nks, piece); break;
      case 4: run_tile(std::integral_constant<int, 4>{}, r, ti.y, ti.z, pt, nks, piece); break;
      case 3: run_tile(std::integral_constant<int, 3>{}, r, ti.y, ti.z, pt, nks, piece); break;
      case 2: run_tile(std::integral_constant<int, 2>{}, r, ti.y, ti.z, pt, nks, piece); break;
      case 1: run_tile(std::integral_constant<int, 1>{}, r, ti.y, ti.z, pt, nks, piece); break;
      default: run_tile(std::integral_constant<int, 0>{}, r, ti.y, ti.z, pt, nks, piece); break;
    }
  }
  wait_vm<0>();  // DMAs past the end have landed before the workgroup exits
}

template <int EPI, bool PT = false, bool GATHER = false>
hipError_t launch_fwd(FwdArgs a, hipStream_t stream) {
  // set once per process (thread-safe static initialisation)
  static const hipError_t attr_err =
      hipFuncSetAttribute((const void*)gg_fwd_kernel<EPI, PT, GATHER>, hipFuncAttributeMaxDynamicSharedMemorySize, LDS_TOTAL);
  if (attr_err != hipSuccess) return attr_err;
  const int grid = (num_cus() + 7) & ~7;
  return launch_k(true, gg_fwd_kernel<EPI, PT, GATHER>, dim3(grid), dim3(FTHREADS), LDS_TOTAL, stream, a);
}

}  // namespace

// Pieces per split leftover tile at most (TTAMD_GEMM_SPLIT=1 turns the
// split off, for A/B timing).
static int split_max() {
  static const int v = [] {
    const char* e = getenv("TTAMD_GEMM_SPLIT");
    const int n = e ? atoi(e) : kSplitMaxPieces;
    return n < 1 ? 1 : (n > kSplitMaxPieces ? kSplitMaxPieces : n);
  }();
  return v;
}

// CUs of the device current at the first call (thread-safe static
// initialisation; every device of a process is the same part).
int num_cus() {
  static const int cus = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    return n;
  }();
  return cus;
}

hipError_t launch_fwd_gemm(int epi, const FwdGemm& g, hipStream_t stream) {
  FwdArgs a = {};
  a.q = (const bf16_t*)g.act;
  a.ldq = g.kred;
  a.q_index = g.act_index;
  a.q_div = g.act_div > 0 ? g.act_div : 1;
  a.n_q_in = g.n_act;
  a.p = (const bf16_t*)g.w;
  a.kred = g.kred;
  a.ldp = g.kred;
  a.table = g.table;
  a.n_qtiles = g.n_qtiles;
  a.part = g.part;
  a.split_cnt = g.split_cnt;
  a.split_max = split_max();
  a.out = (bf16_t*)g.out;
  if (epi == EPI_SWIGLU) {
    a.p_estride = (int64_t)2 * g.n * g.kred;
    a.n_p = g.n;
    a.np_tiles = (g.n + 127) / 128;
    a.ldo = g.n;
    a.hidden = g.n;
    a.limit = g.limit;
    a.h_out = (bf16_t*)g.h_out;
    a.ldh = 2 * (int64_t)g.n;
    if (a.q_index) return launch_fwd<EPI_SWIGLU, false, true>(a, stream);
    return launch_fwd<EPI_SWIGLU>(a, stream);
  }
  a.p_estride = (int64_t)g.n * g.kred;
  a.n_p = g.n;
  a.np_tiles = (g.n + TP - 1) / TP;
  a.ldo = g.n;
  a.row_scale = g.row_scale;
  a.dest = g.dest;
  a.n_dest = g.n_dest;
  a.accumulate = g.accumulate;
  a.scale_sigmoid = g.scale_sigmoid;
  if (epi == EPI_SCATTER) return launch_fwd<EPI_SCATTER>(a, stream);
  return launch_fwd<EPI_STORE>(a, stream);
}

hipError_t launch_dgrad_gemm(int epi, const DgradGemm& g, hipStream_t stream) {
  // out[m, k] = sum_n dy[m, n] w[e, n, k]: token rows q = dy (reduction n
  // contiguous), weight operand w[e] = [n][k] reduction-major.
  FwdArgs a = {};
  a.q = (const bf16_t*)g.dy;
  a.ldq = g.n_red;
  a.q_div = 1;
  a.p = (const bf16_t*)g.w;
  a.p_estride = (int64_t)g.n_red * g.n_out;
  a.ldp = g.n_out;
  a.kred = g.n_red;
  a.n_p = g.n_out;
  a.np_tiles = (g.n_out + TP - 1) / TP;
  a.table = g.table;
  a.n_qtiles = g.n_qtiles;
  a.part = g.part;
  a.split_cnt = g.split_cnt;
  a.split_max = split_max();
  a.out = (bf16_t*)g.out;
  if (epi == EPI_SWIGLU_BWD) {
    a.ldo = 2 * (int64_t)g.n_out;
    a.hidden = g.n_out;
    a.limit = g.limit;
    a.h_in = (const bf16_t*)g.h;
    a.ldh = 2 * (int64_t)g.n_out;
    a.a_out = (bf16_t*)g.a_out;
    return launch_fwd<EPI_SWIGLU_BWD, true>(a, stream);
  }
  a.ldo = g.n_out;
  return launch_fwd<EPI_STORE, true>(a, stream);
}

}  // namespace ttamd
