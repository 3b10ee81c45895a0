// Persistent grouped weight gradient on MI355X (gfx950):
//
//   dw[e][n][k] = sum_{m in rows(e)} dy[m][n] * x[m][k]
//
// The backward of torch._grouped_mm w.r.t. its weight (npu_gmm.py:31, :38
// under autograd): dw13 = dh^T x, dw2 = dy^T a per expert, reduction over the
// expert's ragged row range.
//
// Both operands are reduction-major (rows m, columns contiguous), so the
// MFMA fragments (8 consecutive m per lane) come from ds_read_b64_tr_b16 on
// the rows exactly as they arrive from HBM:
//   * Tile: 256 output rows n (the MFMA B operand, one n per lane) x 256
//     output columns k (A operand, 4 consecutive k per lane and register
//     group, so fp32 / bf16 results leave as 16- / 8-byte stores).
//   * 8 waves (2 per SIMD), 2 (n) x 4 (k); each wave 128 n x 64 k =
//     2 x 4 accumulators of v_mfma_f32_32x32x16_bf16.
//   * Stages of 64 rows m: x rows (64 x 512 bytes) and dy rows (64 x 512
//     bytes) DMA'd by global_load_lds_dwordx4 into two 64 KB buffers, chunk
//     c of row m stored at c ^ 4 ((m ^ (m >> 3)) & 3) (conflict-free
//     transposed reads); one barrier per stage as in gemm_fwd.hip.
//   * The last stage of an expert reads clamped rows past its end; their
//     products are removed by zeroing those rows in the x fragments.
//   * Persistent over (expert, n tile, k tile), expert-major, the n tiles in
//     strips of 4 with the k tile major inside a strip (see tile_of), with
//     the XCD-aware slot mapping of gemm_fwd.hip; the DMA stream runs over
//     the flattened (tile, stage) sequence, whose stage counts vary per
//     expert.
//     An expert without rows still takes one (fully masked) stage, so its
//     gradient tile is written as zeros.
//   * Tail split (as in gemm_fwd.hip): with a workspace, the tiles left over
//     after the last full round are cut along the expert's rows into pieces
//     of consecutive stages, run on the otherwise idle workgroups; each
//     piece writes its fp32 sums to the workspace and counts its arrival,
//     and the last to arrive adds all of them in piece order (the same sum
//     whichever arrives last) and runs the epilogue.
#include "common.h"
#include "dma_asm.h"
#include "gemm_common.h"
#include "kernels.h"

namespace ttamd {
namespace {

using namespace dma;

constexpr int TQ = 256;  // n per tile
constexpr int TP = 256;  // k per tile
constexpr int TK = 64;   // rows m per stage
constexpr int WAVES = 8;
constexpr int WPN = 4;              // waves along k
constexpr int NJ = TQ / 32 / 2;     // 4 n blocks per wave
constexpr int NPB = TP / 32 / WPN;  // 2 k blocks per wave
constexpr int THREADS = 64 * WAVES;
constexpr int ROW_BYTES = 512;      // 256 bf16 columns of one row m
constexpr int OP_BYTES = TK * ROW_BYTES;  // 32 KB per operand and stage
constexpr int STAGE_BYTES = 2 * OP_BYTES;
constexpr int LDS_BYTES = 2 * STAGE_BYTES;  // 128 KB
constexpr int SLAB_BYTES = 32 * 128;        // per wave: one 32 x 64 bf16 output block
constexpr int LDS_TOTAL = LDS_BYTES + WAVES * SLAB_BYTES;  // 160 KB
constexpr int DMA_OP = OP_BYTES / 1024 / WAVES;  // 4 instructions per operand and wave
constexpr int DMA_PER_STAGE = 2 * DMA_OP;
constexpr int kStripN = 4;  // n tiles per strip of the tile order

typedef short short4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4_t lds_short4_t;
typedef __attribute__((address_space(1))) int gint_t;
typedef __attribute__((address_space(1))) floatx4_t gfloatx4_t;

__device__ __forceinline__ int ptswz(int m) { return 4 * ((m ^ (m >> 3)) & 3); }

struct Frag {
  bf16x8_t a[NPB];  // x: k blocks
  bf16x8_t b[NJ];   // dy: n blocks
};

__global__ __launch_bounds__(THREADS, 1) void gg_wgrad_dma_kernel(const WgradDmaArgs a) {
  extern __shared__ __attribute__((aligned(1024))) char smem[];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wq = w / WPN;
  const int wp = w % WPN;
  const int l = threadIdx.x & 63;
  const int G = gridDim.x;
  const int b = blockIdx.x;
  const int slot = (b & 7) * (G >> 3) + (b >> 3);
  const int per_e = a.n_tiles * a.k_tiles;
  const int ntiles = a.E * per_e;
  // Tail split: R full rounds, rt tiles left over; piece j of leftover tile
  // t runs on slot j * rt + t after the slot's R whole tiles.
  const int R = ntiles / G;
  const int rt = ntiles - R * G;
  const int np = (a.split_np > 1 && rt > 0 && rt <= kSplitTiles && a.split_np * rt <= G) ? a.split_np : 1;
  const bool has_piece = np > 1 && slot < rt * np;
  const int nfull = np > 1 ? R : (slot < ntiles ? (ntiles - slot + G - 1) / G : 0);
  const int nmy = nfull + (has_piece ? 1 : 0);
  if (nmy == 0) return;
  const int pc_t = has_piece ? slot % rt : 0;  // leftover tile of the piece
  const int pc_j = has_piece ? slot / rt : 0;  // piece index
  const uint32_t lds0 = lds_addr(smem);

  // tile round r -> (expert, n tile, k tile, first row, end row, stages)
  struct Tile {
    int e, nt, kt, m0, m1, nks;
  };
  auto tile_of = [&](int r) {
    Tile t;
    const int id = r < nfull ? r * G + slot : R * G + pc_t;
    t.e = id / per_e;
    const int rem = id - t.e * per_e;
    // Within an expert, strips of kStripN n tiles, k tile major inside a
    // strip: an XCD's 32 consecutive slots then cover 4 n x 8 k tiles, so
    // each dY slice is shared by 8 of its workgroups and each X slice by 4
    // in its L2 (row-major: one n tile x 32 k tiles, every X slice read by
    // one workgroup of the XCD).
    const int strip = rem / (kStripN * a.k_tiles);
    const int in_strip = rem - strip * kStripN * a.k_tiles;
    const int gn = min(kStripN, a.n_tiles - strip * kStripN);
    t.kt = in_strip / gn;
    t.nt = strip * kStripN + (in_strip - t.kt * gn);
    t.m0 = t.e == 0 ? 0 : sload_int(a.offs + t.e - 1);
    t.m1 = sload_int(a.offs + t.e);
    t.m0 = min(max(t.m0, 0), a.M);
    t.m1 = min(max(t.m1, t.m0), a.M);
    t.nks = max(1, (t.m1 - t.m0 + TK - 1) / TK);
    if (r >= nfull) {
      // piece pc_j: stages [k0, k1) of the tile's rows (an empty share runs
      // one fully masked stage and contributes zeros)
      const int k0 = pc_j * t.nks / np, k1 = (pc_j + 1) * t.nks / np;
      const int m_end = t.m1;
      t.m1 = min(t.m0 + TK * k1, m_end);
      t.m0 = min(t.m0 + TK * k0, m_end);
      t.nks = max(1, k1 - k0);
    }
    return t;
  };

  // ---- DMA stream: a cursor over (tile round, stage) --------------------------
  // instruction i of wave w moves rows 2 (WAVES i + w) and + 1 of an operand;
  // lane l: row + (l >> 5), physical chunk l & 31.
  int c_r = 0, c_ks = 0;
  Tile c_t = tile_of(0);
  auto issue = [&](int s) {
    const int m_stage = c_t.m0 + TK * c_ks;
    const int nvalid = c_t.m1 - m_stage;  // may be <= 0 for an expert without rows
    const uint64_t xb = (uint64_t)(a.x + (int64_t)c_t.kt * TP);
    const uint64_t yb = (uint64_t)(a.dy + (int64_t)c_t.nt * TQ);
    const uint32_t st = lds0 + (uint32_t)((s & 1) * STAGE_BYTES) + w * 1024;
    if (a.M > 0) {  // no rows at all: every stage is masked, nothing to load
#pragma unroll
    for (int i = 0; i < DMA_OP; ++i) {
      const int row = 2 * (WAVES * i + w) + (l >> 5);
      const int lc = (l & 31) ^ ptswz(row);
      const int m = min(max(m_stage + min(row, nvalid - 1), 0), a.M - 1);
      const int xcol = min(c_t.kt * TP + 8 * lc, a.K - 8) - c_t.kt * TP;
      dma16((uint32_t)(m * a.ldx * 2 + xcol * 2), xb, st + i * (WAVES * 1024));
    }
#pragma unroll
    for (int i = 0; i < DMA_OP; ++i) {
      const int row = 2 * (WAVES * i + w) + (l >> 5);
      const int lc = (l & 31) ^ ptswz(row);
      const int m = min(max(m_stage + min(row, nvalid - 1), 0), a.M - 1);
      const int ycol = min(c_t.nt * TQ + 8 * lc, a.N - 8) - c_t.nt * TQ;
      dma16((uint32_t)(m * a.lddy * 2 + ycol * 2), yb, st + OP_BYTES + i * (WAVES * 1024));
    }
    }
    // advance; past the last stage keep re-loading it
    if (c_ks + 1 < c_t.nks) {
      ++c_ks;
    } else if (c_r + 1 < nmy) {
      ++c_r;
      c_ks = 0;
      c_t = tile_of(c_r);
    }
  };

  // ---- fragments: transposed reads (see gemm_fwd.hip, PT) ---------------------
  const int tr_row = 8 * ((l >> 5) & 1) + ((l & 15) >> 2);
  const int tr_col = 16 * ((l >> 4) & 1) + 4 * (l & 3);
  const int bsw = ((l >> 2) & 3) ^ ((l >> 5) & 1);
  int arow[NPB], brow[NJ];
#pragma unroll
  for (int pb = 0; pb < NPB; ++pb) arow[pb] = (TP / WPN) * wp + 32 * pb;
#pragma unroll
  for (int j = 0; j < NJ; ++j) brow[j] = (TQ / 2) * wq + 32 * j;
  // Offset of the lane's 8-byte piece for a 32-column block at col0 (uniform)
  // and reduction rows 16 kk + 4 t + tr_row: the chunk XOR depends on the
  // lane and on kk & 1 only (see gemm_fwd.hip, PT).
  const int tr_base = tr_row * ROW_BYTES + ((tr_col & 4) << 1);
  const int tc8 = tr_col >> 3;
  const int swz0 = 4 * bsw, swz1 = 4 * (bsw ^ 2);
  auto tr8 = [&](const char* st, int col0, int kk) {
    const int off = tr_base + ((((col0 >> 3) + tc8) ^ ((kk & 1) ? swz1 : swz0)) << 4) + (16 * kk) * ROW_BYTES;
    short4_t v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_t*)(st + off));
    short4_t v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_t*)(st + off + 4 * ROW_BYTES));
    return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7));
  };
  auto read_frag = [&](Frag& f, int s, int kk) {
    const char* st = smem + (s & 1) * STAGE_BYTES;
#pragma unroll
    for (int pb = 0; pb < NPB; ++pb) f.a[pb] = tr8(st, arow[pb], kk);
#pragma unroll
    for (int j = 0; j < NJ; ++j) f.b[j] = tr8(st + OP_BYTES, brow[j], kk);
  };
  // Rows >= nvalid of a stage contribute nothing: zero them in both the x
  // and the dy fragments (the clamped rows loaded there belong to the same
  // or, for an expert without rows, the previous expert; zeroing only one
  // operand would turn an Inf or NaN there into NaN instead of the exact
  // zeros the gradient of an empty expert is).  Lane l holds rows
  // 16 kk + 8 (l >> 5) + {0..3} and + 4 + {0..3}.
  auto mask_frag = [&](Frag& f, int kk, int nvalid) {
    // element i of the lane's 8 is row 16 kk + 8 (l >> 5) + i: kept if i < rem
    const int rem = nvalid - 16 * kk - 8 * ((l >> 5) & 1);
    uint32_t keep[4];
#pragma unroll
    for (int d = 0; d < 4; ++d)
      keep[d] = (2 * d < rem ? 0x0000ffffu : 0u) | (2 * d + 1 < rem ? 0xffff0000u : 0u);
#pragma unroll
    for (int pb = 0; pb < NPB; ++pb) {
      u32x4_t v = __builtin_bit_cast(u32x4_t, f.a[pb]);
#pragma unroll
      for (int d = 0; d < 4; ++d) v[d] &= keep[d];
      f.a[pb] = __builtin_bit_cast(bf16x8_t, v);
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      u32x4_t v = __builtin_bit_cast(u32x4_t, f.b[j]);
#pragma unroll
      for (int d = 0; d < 4; ++d) v[d] &= keep[d];
      f.b[j] = __builtin_bit_cast(bf16x8_t, v);
    }
  };

  // ---- prologue --------------------------------------------------------------
  issue(0);
  issue(1);
  wait_vm_barrier<DMA_PER_STAGE>();
  Frag f0, f1;
  read_frag(f0, 0, 0);

  int s = 0;
  for (int r = 0; r < nmy; ++r) {
    const Tile t = tile_of(r);
    floatx16_t acc[NPB][NJ];
#pragma unroll
    for (int i = 0; i < NPB; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
    auto mfma = [&](const Frag& f) {
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int pb = 0; pb < NPB; ++pb)
          acc[pb][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[pb], f.b[j], acc[pb][j], 0, 0, 0);
    };
    for (int ks = 0; ks < t.nks; ++ks, ++s) {
      const int nvalid = t.m1 - (t.m0 + TK * ks);
      const bool partial = nvalid < TK;  // wave-uniform
      if (partial) mask_frag(f0, 0, nvalid);
      read_frag(f1, s, 1);
      if (partial) mask_frag(f1, 1, nvalid);
      mfma(f0);
      read_frag(f0, s, 2);
      if (partial) mask_frag(f0, 2, nvalid);
      mfma(f1);
      read_frag(f1, s, 3);
      if (partial) mask_frag(f1, 3, nvalid);
      mfma(f0);
      wait_vm_barrier<0>();  // stage s + 1 landed, every wave done with stage s
      issue(s + 2);
      read_frag(f0, s + 1, 0);
      mfma(f1);
    }

    // ---- split leftover tile: publish this piece's sums; the last piece to
    //      arrive adds all of them in piece order and runs the epilogue.
    //      The partials are written back from this XCD's L2 (release) before
    //      the arrival is counted, and the last piece invalidates its caches
    //      (acquire) before it reads the others'; it resets the counter.
    if (np > 1 && r >= nfull) {
      constexpr int NV4 = NPB * NJ * 4;                   // float4 per lane
      constexpr uint32_t WAVE_BYTES = NV4 * 64 * 16;      // 32 KB
      constexpr uint64_t PIECE_BYTES = (uint64_t)WAVES * WAVE_BYTES;  // 256 KB
      static_assert(PIECE_BYTES <= kSplitPartBytes, "partial of a piece");
      // The bases are made opaque here so that no address is computed (and
      // kept live) in the k loop.
      uint64_t pw = (uint64_t)a.part + (uint64_t)w * WAVE_BYTES;
      asm volatile("" : "+s"(pw));
      uint32_t loff = (uint32_t)l * 16u;
      asm volatile("" : "+v"(loff));
      auto piece = [&](int j) { return pw + (uint64_t)(pc_t * np + j) * PIECE_BYTES; };
      const uint64_t mine = piece(pc_j);
#pragma unroll
      for (int pb = 0; pb < NPB; ++pb)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
          for (int g = 0; g < 4; ++g)
            *(gfloatx4_t*)(mine + (uint32_t)(((pb * NJ + j) * 4 + g) * 1024) + loff) =
                floatx4_t{acc[pb][j][4 * g], acc[pb][j][4 * g + 1], acc[pb][j][4 * g + 2], acc[pb][j][4 * g + 3]};
      wait_vm<0>();  // this wave's partial has reached L2; every DMA has landed
      __syncthreads();
      // (the stage buffers are idle: no DMA is issued after the last unit)
      int* flag = (int*)smem;
      if (w == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        gint_t* cnt = (gint_t*)(a.split_cnt + pc_t);
        int old = 0;
        if (l == 0) old = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        old = __builtin_amdgcn_readfirstlane(old);
        if (old == np - 1) {
          if (l == 0) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
          // the cache invalidation has completed before the barrier below
          // lets the other waves load the partials
          wait_vm<0>();
        }
        if (l == 0) *flag = (old == np - 1);
      }
      __syncthreads();
      if (__builtin_amdgcn_readfirstlane(*flag) == 0) return;
#pragma unroll
      for (int pb = 0; pb < NPB; ++pb)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
          for (int v = 0; v < 16; ++v) acc[pb][j][v] = 0.f;
      // the sum in piece order, one 16-float block (four loads) at a time
      for (int jp = 0; jp < np; ++jp) {
        const uint64_t src = piece(jp);
#pragma unroll
        for (int pb = 0; pb < NPB; ++pb)
#pragma unroll
          for (int j = 0; j < NJ; ++j) {
            floatx4_t v[4];
#pragma unroll
            for (int g = 0; g < 4; ++g)
              v[g] = *(const gfloatx4_t*)(src + (uint32_t)(((pb * NJ + j) * 4 + g) * 1024) + loff);
#pragma unroll
            for (int g = 0; g < 4; ++g)
#pragma unroll
              for (int i = 0; i < 4; ++i) acc[pb][j][4 * g + i] += v[g][i];
            __builtin_amdgcn_sched_barrier(0);
          }
      }
    }

    // ---- epilogue: acc[pb][j][4g + i] = dw[e][n][k], n = nt*TQ + brow[j] +
    //      lane % 32, k = kt*TP + arow[pb] + 8g + 4 (lane / 32) + i.
    int er32 = l & 31;
    asm volatile("" : "+v"(er32));
    const int half = l >> 5;
    // Both forms go through the wave's private 4 KB LDS slab (row r: 128
    // bytes, 16-byte chunk c at c ^ (r & 7)) and leave as streaming stores
    // of 8 whole 128-byte rows per instruction: the gradient is written once
    // and not read here again, and cached it would evict the operand lines
    // the other workgroups of the XCD are about to read (routed C3 dW2 934
    // -> 724 us in bf16).
    char* slab = smem + LDS_BYTES + w * SLAB_BYTES;
    if (a.dw_fp32) {
      // fp32: one 32-row x 32-column block (128 bytes per row) at a time
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
#pragma unroll
        for (int pb = 0; pb < NPB; ++pb) {
          if (t.kt * TP + arow[pb] < a.K) {  // wave-uniform: the block's 32 columns are valid together
            const floatx16_t& v = acc[pb][j];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              const int chunk = (2 * g + half) ^ (er32 & 7);  // columns 8g + 4 half .. + 3
              *(float4*)(slab + er32 * 128 + chunk * 16) = make_float4(v[4 * g], v[4 * g + 1], v[4 * g + 2], v[4 * g + 3]);
            }
            lds_wait();  // the slab writes have landed
            uint4 o4[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int r = 8 * i + (l >> 3);
              o4[i] = *(const uint4*)(slab + r * 128 + (((l & 7) ^ (r & 7)) << 4));
            }
            lds_wait();  // read before the next block overwrites the slab
            const int col = t.kt * TP + arow[pb] + 4 * (l & 7);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int n = t.nt * TQ + brow[j] + 8 * i + (l >> 3);
              if (n < a.N) store_stream((uint4*)((float*)a.dw + ((int64_t)t.e * a.N + n) * a.K + col), o4[i]);
            }
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    } else if (t.kt * TP + arow[0] < a.K) {  // the wave's 64 columns are valid together
      // bf16: one 32-row block (the wave's 64 columns, 128 bytes per row)
      // at a time
      const int col = t.kt * TP + arow[0] + 8 * (l & 7);
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
#pragma unroll
        for (int pb = 0; pb < NPB; ++pb)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const floatx16_t& v = acc[pb][j];
            const int chunk = (4 * pb + g) ^ (er32 & 7);
            *(uint2*)(slab + er32 * 128 + chunk * 16 + half * 8) =
                make_uint2(pack_bf16x2(v[4 * g], v[4 * g + 1]), pack_bf16x2(v[4 * g + 2], v[4 * g + 3]));
          }
        lds_wait();  // the slab writes have landed
        uint4 o4[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 8 * i + (l >> 3);
          o4[i] = *(const uint4*)(slab + r * 128 + (((l & 7) ^ (r & 7)) << 4));
        }
        lds_wait();  // read before the next block overwrites the slab
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 8 * i + (l >> 3);
          const uint4 o = o4[i];
          const int n = t.nt * TQ + brow[j] + r;
          if (n < a.N) store_stream((uint4*)((bf16_t*)a.dw + ((int64_t)t.e * a.N + n) * a.K + col), o);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  wait_vm<0>();
}

// Arrival counters of the split tail tiles to zero (a kernel, not a memset,
// so that the sequence can be captured in a HIP graph).
__global__ __launch_bounds__(256) void split_cnt_zero_kernel(int* __restrict__ cnt, int n) {
  for (int i = threadIdx.x; i < n; i += 256) cnt[i] = 0;
}

}  // namespace

hipError_t launch_split_cnt_zero(int* split_cnt, int n, hipStream_t stream) {
  return launch_k(false, split_cnt_zero_kernel, dim3(1), dim3(256), 0, stream, split_cnt, n);
}

hipError_t launch_wgrad_dma(const WgradDmaArgs& a, hipStream_t stream) {
  // set once per process (thread-safe static initialisation)
  static const hipError_t attr_err =
      hipFuncSetAttribute((const void*)gg_wgrad_dma_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, LDS_TOTAL);
  if (attr_err != hipSuccess) return attr_err;
  const int grid = (num_cus() + 7) & ~7;
  return launch_k(false, gg_wgrad_dma_kernel, dim3(grid), dim3(THREADS), LDS_TOTAL, stream, a);
}

}  // namespace ttamd
