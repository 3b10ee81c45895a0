// Persistent fp8 (e4m3) grouped GEMM with 128 x 128 block scales for the
// expert FFN forward on MI355X (gfx950).
//
//   out[q, p] = sum_kb  sx[kb, q] * sw[e(q), p / 128, kb] *
//                       sum_{k in block kb} xq[q, k] * wq[e(q), p, k]
//
// xq: routed activations, e4m3 [M, K], with per-row scales for every 128
// channels stored k-block major, sx [K/128, M] (one contiguous run of rows per
// k-block, so a tile's scales for one k-block are one 1 KB line run).
// wq: weights e4m3 [E, N, K] with one fp32 scale per 128 x 128 block,
// sw [E, N/128, K/128].  The scales are the absmax / 448 recipe; the
// reference semantics are "dequantise both operands, fp32 GEMM".
//
// Tile: up to 256 token rows (Q) x 256 weight rows (P; SWIGLU: 128 gate rows
// and the 128 matching up rows); k in stages of 128 (one scale block, one
// 128-byte line per row).
//   * 8 waves, two per SIMD, 2 x 4: wave (wq, wp) owns token rows 128wq..
//     and 64 weight rows (SWIGLU: 32 gate rows and the 32 matching up rows),
//     i.e. 4 x 8 blocks of v_mfma_f32_16x16x128_f8f6f4 (no hardware
//     scales): one MFMA covers a block's whole k = 128 scale block, and its
//     partial sum goes straight into the fp32 accumulator times sx * sw, so
//     the fp32 block scales are applied once per block as in the dequantised
//     form, with no partial sums kept across MFMAs.  The scale FMAs of token
//     block jb - 1 run under block jb's MFMAs, and with two waves per SIMD
//     under the other wave's as well.
//   * The 256 x 128 tile was bound by the L2 -> LDS stream (each CU keeps
//     about 64 line requests in flight), so the tile is as large as the
//     registers allow: 256 x 256 moves 66 KB per 16.8 MFLOP stage where
//     256 x 128 moved 48 KB per 8.4.  With it a stage's DMA has landed
//     before the barrier that needs it (~1 % of the stage waiting), and the
//     stage is the MFMAs, the block-scale FMAs and the fragment reads of the
//     two waves of each SIMD.  The 128 accumulators leave room for the 4
//     weight fragments of the stage and only 2 token fragments, read just
//     before use.
//   * Two LDS stages of 66 KB: 32 KB weight rows + 32 KB token rows (DMA,
//     global_load_lds_dwordx4, 8 rows per instruction, XOR-swizzled 16-byte
//     chunks as in the bf16 kernel), 1 KB of token-row scales (waves 0-3)
//     and the stage's weight-block scales (waves 4-7 each load a copy, so
//     every wave issues the same DMA count; all read wave 4's).  At the top
//     of stage s every wave waits for stage s (the only one in flight) and
//     passes the barrier, which also means stage s - 1 has been read, and
//     stage s + 1's weight rows are issued into its buffer (its token rows
//     and scales after the first token block's MFMAs): one stage ahead
//     keeps the bounding DMA stream busy.
//   * A wave computes only the 16-row token blocks of its half that hold
//     tile rows (0, 2, 4, 6 or 8, rounded up to even): the k loop is
//     instantiated per count and picked per tile.  The skipped blocks hold
//     clamped copies of the tile's last row, whose products are never
//     stored (short tiles of skewed expert loads).
//   * Persistent workgroups, XCD-aware slots, flattened (tile, stage) DMA
//     stream and the EPI_SCATTER metadata in LDS follow gemm_fwd.hip.
#include <type_traits>

#include "common.h"
#include "dma_asm.h"
#include "gemm_common.h"
#include "kernels.h"

namespace ttamd {
namespace {

using namespace dma;

constexpr int TQ = 256;   // token rows
constexpr int TP = 256;   // weight rows (SWIGLU: 128 gate + the 128 matching up rows)
constexpr int TKB = 128;  // k per stage (bytes per row)
constexpr int NSTAGE = 2;
constexpr int WAVES = 8;
constexpr int FTHREADS = 64 * WAVES;
constexpr int P_BYTES = TP * TKB;  // 32 KB
constexpr int Q_BYTES = TQ * TKB;  // 32 KB
constexpr int SX_OFF = P_BYTES + Q_BYTES;
constexpr int SW_OFF = SX_OFF + TQ * 4;
constexpr int STAGE_BYTES = SW_OFF + 4 * 256;     // 66 KB
constexpr int LDS_BYTES = NSTAGE * STAGE_BYTES;   // 132 KB
constexpr int DMA_P = TP / 8 / WAVES;             // 4
constexpr int DMA_Q = TQ / 8 / WAVES;             // 4
static_assert(TQ == 2 * 128 && TP == 4 * 64 && WAVES == 8, "wave layout: 2 token halves x 4 weight quarters");
// EPI_SCATTER metadata slots (tile round % 3): tile r's slot is written
// when its first stage is issued, at the top of tile r - 1's last stage,
// after every wave has passed tile r - 2's epilogue.
constexpr int META_BYTES = TQ * 8;
constexpr int META_SLOTS = 3;
constexpr int LDS_TOTAL = LDS_BYTES + META_SLOTS * META_BYTES;  // 138 KB
static_assert(LDS_TOTAL <= 160 * 1024, "LDS");

typedef int i32x8_t __attribute__((ext_vector_type(8)));

// Chunk permutation of 128-byte LDS rows (as in gemm_fwd.hip).
__device__ __forceinline__ int cswz(int r) { return (r ^ (r >> 3)) & 7; }

// A wave's blocks of 16 rows: NPB16 weight blocks (held for the stage) and
// NJ16 token blocks (read just before use, NBS in registers at a time);
// lane l holds bytes 32 (l / 16) .. + 31 of row l % 16.
constexpr int NPB16 = 4;
constexpr int NJ16 = 8;
constexpr int NBS = 2;

template <int EPI>
__global__ __launch_bounds__(FTHREADS, 1) void gg_fp8_kernel(const Fp8Args a) {
  extern __shared__ __attribute__((aligned(1024))) char smem[];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wq = w >> 2;  // token half: rows 128 wq ..
  const int wp = w & 3;   // weight quarter; waves w and w + 4 share a SIMD
  const int l = threadIdx.x & 63;
  const int G = gridDim.x;
  const int b = blockIdx.x;
  const int slot = (b & 7) * (G >> 3) + (b >> 3);
  const int ntiles = sload_int(a.n_qtiles) * a.np_tiles;
  const int nmy = slot < ntiles ? (ntiles - slot + G - 1) / G : 0;
  const int ksteps = a.kred / TKB;
  const int total = nmy * ksteps;
  if (total == 0) return;

  const uint32_t lds0 = lds_addr(smem);
  const int drow = l >> 3;

  // ---- DMA stream -----------------------------------------------------------
  int d_r = -1;
  uint64_t d_pbase = 0, d_qbase = 0, d_scbase = 0, d_scstep = 0;
  int d_qmax = 0, d_pmax = 0, d_hmax = 0;
  uint32_t d_scoff = 0;
  // DMA instruction i of wave w moves tile rows rr0 + 64 i (row block
  // 8 i + w); its chunk permutation (drow ^ w) & 7 is the same for every i,
  // so the per-lane offsets are recomputed at issue from rr0 and lch16
  // instead of being held through the k loop.
  static_assert(WAVES == 8, "row block 8 i + w has chunk permutation term w");
  const int rr0 = 8 * w + drow;
  const uint32_t lch16 = (uint32_t)(((l & 7) ^ ((drow ^ w) & 7)) * 16);
  const uint32_t d_sclds = (w < 4) ? (uint32_t)(SX_OFF + w * 256) : (uint32_t)(SW_OFF + (w - 4) * 256);
  auto dma_tile = [&](int r) {
    const int tile = r * G + slot;
    const int qt = tile / a.np_tiles;
    const int pt = tile - qt * a.np_tiles;
    const int4 ti = sload_int4(a.table + qt);
    const int qmax = ti.z - ti.y - 1;
    d_qmax = qmax;
    d_pmax = a.n_p - 1 - pt * TP;  // last weight row of a partial tile (STORE, SCATTER)
    d_hmax = (int)a.hidden - 1 - pt * 128;  // SWIGLU: last gate (and up) row of the tile
    const int64_t prow0 = (EPI == EPI_SWIGLU) ? (int64_t)pt * 128 : (int64_t)pt * TP;
    d_pbase = (uint64_t)(a.p + (int64_t)ti.x * a.p_estride + prow0 * a.ldp);
    d_qbase = (uint64_t)(a.q + (int64_t)ti.y * a.ldq);
    if (w < 4) {
      // token-row scales: wave w loads rows 64w + lane (clamped) of each k-block
      d_scbase = (uint64_t)(a.sx + ti.y);
      d_scoff = (uint32_t)(min(64 * w + l, qmax) * 4);
      d_scstep = (uint64_t)a.ldsx * 4;
    } else {
      // weight-block scales; every wave 4..7 loads a copy.  STORE, SCATTER:
      // lane parity selects the tile's first or second 128-row block.
      // SWIGLU: lane 0 the gate block (the tile's 128 gate rows start on a
      // block), lane 1 + q the up block of weight quarter q (with H % 128 ==
      // 64 the tile's up rows straddle two blocks; a quarter's 32 do not).
      const int64_t kb_n = a.kred / TKB;
      // (32-bit: H < 2^20, so hidden + 128 pt + 96 fits; a 64-bit lane value
      // here was kept live through the k loop and spilled)
      int blk;
      if constexpr (EPI == EPI_SWIGLU)
        blk = (l == 0) ? pt : ((int)a.hidden + pt * 128 + 32 * min(l - 1, 3)) >> 7;
      else
        blk = 2 * pt + (l & 1);
      blk = min(blk, a.n_p / 128 - 1);
      d_scbase = (uint64_t)(a.sw + (int64_t)ti.x * a.sw_estride);
      d_scoff = (uint32_t)(blk * kb_n * 4);
      d_scstep = 4;
    }
    if (EPI == EPI_SCATTER && w < 4) {
      const uint32_t q = (uint32_t)min(64 * w + l, qmax);
      const uint32_t m = lds0 + LDS_BYTES + (uint32_t)((r % META_SLOTS) * META_BYTES) + w * 256;
      if (a.dest) dma4(q * 4, (uint64_t)(a.dest + ti.y), m);
      if (a.row_scale) dma4(q * 4, (uint64_t)(a.row_scale + ti.y), m + TQ * 4);
    }
    d_r = r;
  };
  // A stage's weight rows are issued at the barrier that frees their buffer,
  // its token rows and scales after the first token block's MFMAs (see the
  // k loop); issue_p sets the stage's bases, which issue_q reads.
  uint64_t d_sqb = 0;
  uint32_t d_sst = 0;
  int d_sks = 0;
  auto issue_p = [&](int s) {
    const int r = s / ksteps;
    const int ks = s - r * ksteps;
    if (r != d_r) dma_tile(r);
    const uint64_t pb = d_pbase + (uint64_t)ks * TKB;
    d_sqb = d_qbase + (uint64_t)ks * TKB;
    d_sst = lds0 + (uint32_t)((s % NSTAGE) * STAGE_BYTES);
    d_sks = ks;
#pragma unroll
    for (int i = 0; i < DMA_P; ++i) {
      int prow;  // weight row relative to d_pbase
      if constexpr (EPI == EPI_SWIGLU)
        prow = (i < 2) ? min(rr0 + 64 * i, d_hmax) : (int)a.hidden + min(rr0 + 64 * (i - 2), d_hmax);
      else
        prow = min(rr0 + 64 * i, d_pmax);
      dma16((uint32_t)(prow * a.ldp) + lch16, pb, d_sst + w * 1024 + i * (WAVES * 1024));
    }
  };
  auto issue_q = [&]() {
#pragma unroll
    for (int i = 0; i < DMA_Q; ++i)
      dma16((uint32_t)(min(rr0 + 64 * i, d_qmax) * a.ldq) + lch16, d_sqb, d_sst + P_BYTES + w * 1024 + i * (WAVES * 1024));
    dma4(d_scoff, d_scbase + (uint64_t)d_sks * d_scstep, d_sst + d_sclds);
  };

  // ---- fragment geometry -------------------------------------------------------
  const int r16 = l & 15;
  const int g4 = l >> 4;
  const int f16 = cswz(r16);
  int arow[NPB16];  // weight block starts (tile rows)
#pragma unroll
  for (int pb = 0; pb < NPB16; ++pb)
    arow[pb] = (EPI == EPI_SWIGLU) ? (pb < 2 ? 32 * wp + 16 * pb : 128 + 32 * wp + 16 * (pb - 2))
                                   : 64 * wp + 16 * pb;
  // Row 16m + r16 of a 128-byte-row operand: cswz = f16 ^ ((2m) & 6) (16m >> 3
  // = 2m is even, so adding r16 >> 3 does not carry).
  auto frag16 = [&](const char* base, int row0) {
    const int x = f16 ^ ((row0 >> 3) & 6);
    const char* row = base + (row0 + r16) * TKB;
    const i32x4_t lo = *(const i32x4_t*)(row + (((2 * g4) ^ x) * 16));
    const i32x4_t hi = *(const i32x4_t*)(row + (((2 * g4 + 1) ^ x) * 16));
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  };
  // weight-block scale of block pb (the copy wave 4 loaded)
  auto sw_lane = [&](int pb) { return (EPI == EPI_SWIGLU) ? (pb < 2 ? 0 : 1 + wp) : (wp >> 1); };

  // ---- prologue: stage 0 in flight ----------------------------------------------
  issue_p(0);
  issue_q();

  int s = 0;
  for (int r = 0; r < nmy; ++r) {
    const int tile = r * G + slot;
    const int qt = tile / a.np_tiles;
    const int pt = tile - qt * a.np_tiles;
    const int4 ti = sload_int4(a.table + qt);
    const int row0 = ti.y, row1 = ti.z;

    floatx4_t acc[NPB16][NJ16];
#pragma unroll
    for (int i = 0; i < NPB16; ++i)
#pragma unroll
      for (int j = 0; j < NJ16; ++j)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[i][j][v] = 0.f;

    // Token blocks of this wave's half that hold tile rows (rounded up to
    // an even count): the blocks past them only hold clamped copies of the
    // last row, whose products are never stored, so they are skipped.
    const int hq = min(max(row1 - row0 - 128 * wq, 0), 128);
    const int nbw = (((hq + 15) >> 4) + 1) & ~1;
    auto kloop = [&](auto nbc) {
      constexpr int NB = decltype(nbc)::value;
      for (int ks = 0; ks < ksteps; ++ks, ++s) {
        // Stage s has landed (the only stage in flight) and every wave is
        // done with stage s - 1: its buffer takes stage s + 1.  The DMA
        // stream is the bound, so one stage ahead keeps it busy.
        wait_vm_barrier<0>();
        const bool more = s + 1 < total;
        if (more) issue_p(s + 1);
        if constexpr (NB == 0) {
          if (more) issue_q();
        } else {
          const char* st = smem + (s % NSTAGE) * STAGE_BYTES;
          i32x8_t fa[NPB16];
          // A block's weight scale is one value for the whole wave (every lane
          // reads the same LDS word): kept in SGPRs, it frees VGPRs for the
          // accumulators and fragments.
          float swv[NPB16];
#pragma unroll
          for (int pb = 0; pb < NPB16; ++pb) {
            fa[pb] = frag16(st, arow[pb]);
            swv[pb] = __int_as_float(__builtin_amdgcn_readfirstlane(*(const int*)(st + SW_OFF + sw_lane(pb) * 4)));
          }
          i32x8_t fb[NBS];
          float sxv[NBS];
          auto read_b = [&](int jb) {
            const int row = 128 * wq + 16 * jb;
            fb[jb % NBS] = frag16(st + P_BYTES, row);
            sxv[jb % NBS] = *(const float*)(st + SX_OFF + (row + r16) * 4);
          };
          read_b(0);
          read_b(1);
          float sx_prev = 0.f;
          floatx4_t part[2][NPB16];
          auto scale_add = [&](int jb, float sxj) {
#pragma unroll
            for (int pb = 0; pb < NPB16; ++pb) {
              const float sc = swv[pb] * sxj;
#pragma unroll
              for (int v = 0; v < 4; ++v) acc[pb][jb][v] += part[jb & 1][pb][v] * sc;
            }
          };
#pragma unroll
          for (int jb = 0; jb < NB; ++jb) {
#pragma unroll
            for (int pb = 0; pb < NPB16; ++pb) {
              floatx4_t z = {};
              // Zero scale operands make the compiler emit the unscaled
              // v_mfma_f32_16x16x128_f8f6f4; the scaled form with unit E8M0
              // scales (127) gives bit-identical sums and runs 2-3 % slower here.
              part[jb & 1][pb] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(fa[pb], fb[jb % NBS], z, 0, 0, 0, 0, 0, 0);
            }
            // block jb - 1's scale FMAs run under block jb's MFMAs; block jb's
            // slot then takes block jb + 2, so its row scale is kept aside first
            if (jb > 0) scale_add(jb - 1, sx_prev);
            sx_prev = sxv[jb % NBS];
            if (jb + 2 < NB) read_b(jb + 2);
            if (jb == 0 && more) issue_q();  // (later placements spill)
          }
          scale_add(NB - 1, sx_prev);
        }
      }
    };
    switch (nbw) {
      case 8: kloop(std::integral_constant<int, 8>{}); break;
      case 6: kloop(std::integral_constant<int, 6>{}); break;
      case 4: kloop(std::integral_constant<int, 4>{}); break;
      case 2: kloop(std::integral_constant<int, 2>{}); break;
      default: kloop(std::integral_constant<int, 0>{}); break;
    }

    // ---- epilogue: acc[pb][jb][i] is (token row 128wq + 16jb + lane % 16,
    //      weight row arow[pb] + 4 (lane / 16) + i).  The lane's row and
    //      column group are re-derived here from an opaque copy of the lane
    //      id, so that nothing epilogue-only stays live through the k loop.
    int el = l;
    asm volatile("" : "+v"(el));
    const int er16 = el & 15;
    const int eg4 = el >> 4;
#pragma unroll
    for (int jb = 0; jb < NJ16; ++jb) {
      const int gq = row0 + 128 * wq + 16 * jb + er16;
      const bool row_ok = gq < row1;
      if constexpr (EPI == EPI_SWIGLU) {
        const float L = a.limit;
        // wave-uniform: this quarter's 32 gate columns lie past H (H % 128 == 64)
        if (pt * 128 + 32 * wp >= a.hidden) continue;
        // The clamp (swiglu_limit) is wave-uniform too: one code path each,
        // so that the unclamped SwiGLU carries no min / max per value.
        auto swiglu_rows = [&](auto clampc) {
          constexpr bool CLAMP = decltype(clampc)::value;
#pragma unroll
          for (int pb = 0; pb < 2; ++pb) {
            const int col = pt * 128 + arow[pb] + 4 * eg4;
            float av[4], gv[4], uv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              gv[i] = round_bf16(acc[pb][jb][i]);
              uv[i] = round_bf16(acc[pb + 2][jb][i]);
              float gc = gv[i], uc = uv[i];
              if constexpr (CLAMP) {
                gc = clamp_max_nan(gc, L);
                uc = clamp_nan(uc, L);
              }
              av[i] = silu_f(gc) * uc;
            }
            if (row_ok) {
              bf16_t* orow = a.out + (int64_t)gq * a.ldo + col;
              *(uint2*)orow = make_uint2(pack_bf16x2(av[0], av[1]), pack_bf16x2(av[2], av[3]));
              if (a.h_out) {
                bf16_t* hrow = a.h_out + (int64_t)gq * a.ldh + col;
                *(uint2*)hrow = make_uint2(pack_bf16x2(gv[0], gv[1]), pack_bf16x2(gv[2], gv[3]));
                *(uint2*)(hrow + a.hidden) = make_uint2(pack_bf16x2(uv[0], uv[1]), pack_bf16x2(uv[2], uv[3]));
              }
            }
          }
        };
        if (a.limit == a.limit)
          swiglu_rows(std::true_type{});
        else
          swiglu_rows(std::false_type{});
      } else if (pt * TP + 64 * wp < a.n_p) {  // wave-uniform: this quarter holds rows of N
        float scl = 1.f;
        int orow_idx = gq;
        if constexpr (EPI == EPI_SCATTER) {
          const int* meta = (const int*)(smem + LDS_BYTES + (r % META_SLOTS) * META_BYTES);
          const int qrow = 128 * wq + 16 * jb + er16;
          if (a.dest) orow_idx = min(max(meta[qrow], 0), a.n_dest - 1);
          if (a.row_scale) scl = __int_as_float(meta[TQ + qrow]);
        }
        bf16_t* orow = a.out + (int64_t)orow_idx * a.ldo;
#pragma unroll
        for (int pb = 0; pb < NPB16; ++pb) {
          const int col = pt * TP + arow[pb] + 4 * eg4;
          const floatx4_t& v = acc[pb][jb];
          const uint2 val = make_uint2(pack_bf16x2(v[0] * scl, v[1] * scl), pack_bf16x2(v[2] * scl, v[3] * scl));
          if (row_ok) *(uint2*)(orow + col) = val;
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  wait_vm<0>();  // DMAs have landed before the workgroup exits
}

template <int EPI>
hipError_t launch_fp8(const Fp8Args& a, hipStream_t stream) {
  // set once per process (thread-safe static initialisation)
  static const hipError_t attr_err =
      hipFuncSetAttribute((const void*)gg_fp8_kernel<EPI>, hipFuncAttributeMaxDynamicSharedMemorySize, LDS_TOTAL);
  if (attr_err != hipSuccess) return attr_err;
  const int grid = (num_cus() + 7) & ~7;
  return launch_k(true, gg_fp8_kernel<EPI>, dim3(grid), dim3(FTHREADS), LDS_TOTAL, stream, a);
}

}  // namespace

hipError_t launch_fp8_gemm(int epi, const Fp8Args& a, hipStream_t stream) {
  if (epi == EPI_SWIGLU) return launch_fp8<EPI_SWIGLU>(a, stream);
  if (epi == EPI_SCATTER) return launch_fp8<EPI_SCATTER>(a, stream);
  return launch_fp8<EPI_STORE>(a, stream);
}

}  // namespace ttamd
