// Pieces shared by the grouped GEMM kernels (internal to libttamd_moe.so).
#pragma once

#include "common.h"

namespace ttamd {

// Epilogue variants of the token-row GEMMs.
enum Epi {
  EPI_STORE = 0,       // out[q][p] = acc
  EPI_SWIGLU = 1,      // gate/up pairs -> silu(clamp(gate)) * clamp(up)
  EPI_SCATTER = 2,     // out[dest[q]][p] = scale[q] * acc
  EPI_SWIGLU_BWD = 3,  // dh from dA = acc and the saved pre-activation h
};

// 1 / (1 + exp(-x)) with the hardware reciprocal (1 ulp) in place of an
// IEEE division (about ten instructions): the GEMM epilogues that use it are
// VALU-bound and round their results to bf16.
__device__ __forceinline__ float sigmoid_f(float x) { return __builtin_amdgcn_rcpf(1.f + __expf(-x)); }
__device__ __forceinline__ float silu_f(float x) { return x * sigmoid_f(x); }

// torch.clamp(x, max=L) and torch.clamp(x, -L, L): NaN stays NaN (the IEEE
// 754-2019 minimum / maximum, v_minimum3_f32 / v_maximum3_f32 on gfx950),
// where fminf / fmaxf would return the limit.
__device__ __forceinline__ float clamp_max_nan(float x, float L) { return __builtin_elementwise_minimum(x, L); }
__device__ __forceinline__ float clamp_nan(float x, float L) {
  return __builtin_elementwise_maximum(__builtin_elementwise_minimum(x, L), -L);
}

// Token-row tiles: table[i] = {expert, first row, end row, 0}, at most
// kFwdTileRows rows (bf16 forward and dgrad) or kFp8TileRows (fp8).  The
// workspace is sized for tiles of kTileRows rows, fewer rows than either,
// so it always holds the table.
constexpr int kTileRows = 128;
constexpr int kFwdTileRows = 320;

// Tile plan of a token-row GEMM: int4 header {number of tiles, ...}, the
// arrival counters of the split tail tiles (kSplitTiles ints, zeroed
// whenever a table is built and left at zero by every GEMM that uses them),
// then the tile table.
constexpr int kSplitTiles = 512;
struct TileTable {
  int* count;
  int* split_cnt;
  int4* table;
};

inline int max_row_tiles(int M, int E) { return M / kTileRows + E + 1; }

inline TileTable tile_table_in(void* ws) {
  TileTable t;
  t.count = (int*)ws;
  t.split_cnt = (int*)ws + 4;
  t.table = (int4*)(t.split_cnt + kSplitTiles);
  return t;
}

// Tail split of the forward / dgrad GEMM: the tiles left over after the
// last full round of the persistent walk are cut along k into pieces that
// run on the otherwise idle CUs; each piece writes its fp32 accumulators
// (kSplitPartBytes, register order) to the partial-sum area of the GEMM's
// workspace, and the last piece of a tile to arrive adds them in piece
// order and runs the epilogue.  At most kSplitMaxPieces pieces per tile,
// each of at least kSplitMinStages k stages, and only for walks of at most
// kSplitMaxRounds full rounds: with more, the ragged tile heights of skewed
// routing decide the finish time more than the leftover tiles do (C4's
// Zipf w13, 7 rounds + 32 tiles: no gain; C3's shared w13, 6 rounds + 128
// tiles of equal height: -40 us).
constexpr size_t kSplitPartBytes = 327680;  // 8 waves x 160 fp32 x 64 lanes
constexpr int kSplitMaxPieces = 8;
constexpr int kSplitMinStages = 8;
constexpr int kSplitMaxRounds = 6;

// Builds the tile table with one workgroup of NT threads (every thread
// calls it; it synchronises the workgroup).  `range(e, r0, r1)` gives the
// rows [r0, r1) of expert e.  An expert's rows are split into the fewest
// tiles of at most max_rows rows, of equal height rounded up to 32 rows
// (540 rows at max_rows = 320 give 2 tiles of 288 rather than 320 + 220);
// tiles are numbered in expert order.  Entries past the last tile, up to
// max_tiles, are {-1, 0, 0, 0}.  The split-tile arrival counters are
// zeroed.  sh: NT / 64 + 1 ints of LDS.
template <int NT, typename Range>
__device__ void block_tile_table(Range range, int E, int max_tiles, int max_rows, int4* __restrict__ table,
                                 int* __restrict__ count, int* __restrict__ split_cnt, int* sh) {
  constexpr int NW = NT / kWave;
  const int tid = threadIdx.x;
  for (int i = tid; i < kSplitTiles; i += NT) split_cnt[i] = 0;
  const int w = tid / kWave, l = lane_id();
  int carry = 0;
  for (int e0 = 0; e0 < E; e0 += NT) {
    const int e = e0 + tid;
    int r0 = 0, r1 = 0, nt = 0, h = max_rows;
    if (e < E) {
      range(e, r0, r1);
      const int c = r1 - r0;
      if (c > 0) {
        const int n0 = (c + max_rows - 1) / max_rows;
        h = (((c + n0 - 1) / n0) + 31) & ~31;
        nt = (c + h - 1) / h;
      }
    }
    const int incl = wave_inclusive_scan(nt);
    if (l == kWave - 1) sh[w] = incl;
    __syncthreads();
    if (w == 0) {
      const int v = (l < NW) ? sh[l] : 0;
      const int vi = wave_inclusive_scan(v);
      if (l < NW) sh[l] = vi;  // inclusive over waves
    }
    __syncthreads();
    const int start = carry + ((w > 0) ? sh[w - 1] : 0) + incl - nt;
    for (int t = 0; t < nt; ++t) {
      const int i = start + t;
      if (i < max_tiles) table[i] = make_int4(e, r0 + t * h, min(r0 + (t + 1) * h, r1), 0);
    }
    carry += sh[NW - 1];
    __syncthreads();  // sh is rewritten by the next round
  }
  for (int i = carry + tid; i < max_tiles; i += NT) table[i] = make_int4(-1, 0, 0, 0);
  if (tid == 0) *count = min(carry, max_tiles);
}

// Forward GEMM description (gemm_fwd.hip).
//   act [M][kred] bf16, w [E][N or 2N][kred] bf16.
//   EPI_SWIGLU: n = H (w holds 2H rows: gate then up), out [M][H], h_out [M][2H].
//   EPI_STORE / EPI_SCATTER: n = N, out [M or n_dest][N].
struct FwdGemm {
  const void* act;
  const int* act_index;  // nullable: gathered activation rows (act row = act_index[j] / act_div)
  int act_div;
  int n_act;
  const void* w;
  int kred;
  int n;
  const int4* table;
  const int* n_qtiles;
  int* split_cnt;  // the plan's arrival counters
  float* part;     // nullable: partial sums of split tail tiles (no split when null)
  void* out;
  float limit;
  void* h_out;
  const float* row_scale;
  const int* dest;
  int n_dest;
  int accumulate;     // EPI_SCATTER: out[dest] = bf16(out[dest] + v) instead of bf16(v)
  int scale_sigmoid;  // EPI_SCATTER: the row scale is sigmoid(row_scale[j])
};

// Kernel arguments of the forward and dgrad GEMMs (gemm_fwd.hip).
struct FwdArgs {
  const bf16_t* q;  // activations [M][kred], or [n_q_in][kred] gathered through q_index
  int64_t ldq;
  const int* q_index;  // nullable: token row j reads q row q_index[j] / q_div
  int q_div;
  int n_q_in;
  const bf16_t* p;  // weights, expert e at p + e * p_estride, rows of ldp
  int64_t p_estride;
  int64_t ldp;
  int kred;
  int n_p;       // valid weight rows (SWIGLU: H, the gate half)
  int np_tiles;  // weight-row tiles per token tile
  const int4* table;
  const int* n_qtiles;
  // tail split (null part: none); part and split_cnt adjacent (the kernel
  // reads both with one scalar load)
  float* part;
  int* split_cnt;
  int split_max;
  bf16_t* out;
  int64_t ldo;
  // EPI_SWIGLU
  int64_t hidden;
  float limit;  // NaN = no clamp
  bf16_t* h_out;
  int64_t ldh;
  // EPI_SWIGLU_BWD
  const bf16_t* h_in;  // saved pre-activation [M][2H]
  bf16_t* a_out;       // recomputed activation [M][H] (nullable)
  // EPI_SCATTER
  const float* row_scale;
  const int* dest;
  int n_dest;
  int accumulate;
  int scale_sigmoid;
};
// The split path of the forward kernel reads part and split_cnt with one
// 16-byte scalar load at offsetof(FwdArgs, part).
static_assert(offsetof(FwdArgs, split_cnt) == offsetof(FwdArgs, part) + sizeof(float*) &&
                  offsetof(FwdArgs, part) % 8 == 0,
              "FwdArgs: split_cnt must directly follow part");

// Grouped dgrad through the forward kernel's reduction-major weight mode:
// out[m, k] = sum_n dy[m, n] w[e(m), n, k], w [E, n_red, n_out].
struct DgradGemm {
  const void* dy;  // [M][n_red]
  const void* w;
  int n_red;
  int n_out;
  const int4* table;
  const int* n_qtiles;
  int* split_cnt;
  float* part;  // nullable
  void* out;  // EPI_STORE: [M][n_out]; EPI_SWIGLU_BWD: dh [M][2 n_out]
  // EPI_SWIGLU_BWD
  const void* h;  // [M][2 n_out]
  float limit;
  void* a_out;
};

// Grouped weight gradient (gemm_wgrad.hip): dw[e][n][k] = sum over the
// expert's rows m of dy[m][n] * x[m][k].
struct WgradDmaArgs {
  const bf16_t* dy;  // [M][N]
  int64_t lddy;
  const bf16_t* x;  // [M][K]
  int64_t ldx;
  const int* offs;  // inclusive, [E]
  int E, M, N, K;
  int n_tiles, k_tiles;  // per expert, 256-wide
  void* dw;              // [E][N][K]
  int dw_fp32;
  // Tail split (split_np > 1): the tiles left over after the last full
  // round are cut along the reduction rows into split_np pieces; each
  // piece writes its fp32 sums (kSplitPartBytes at most) to `part` and
  // counts its arrival in split_cnt[leftover tile] (zero on entry, left at
  // zero).  split_np <= 1: no split.
  float* part;
  int* split_cnt;
  int split_np;
};
hipError_t launch_wgrad_dma(const WgradDmaArgs& a, hipStream_t stream);
hipError_t launch_split_cnt_zero(int* split_cnt, int n, hipStream_t stream);

// Kernel arguments of the fp8 forward GEMM (gemm_fp8.hip).  Activations and
// weights are e4m3 bytes; strides are in bytes for them, in elements for
// the scale and output arrays.
struct Fp8Args {
  const uint8_t* q;  // activations [M][kred] e4m3
  int64_t ldq;
  const uint8_t* p;  // weights, expert e at p + e * p_estride, rows of ldp bytes
  int64_t p_estride;
  int64_t ldp;
  int kred;
  int np_tiles;  // weight-row tiles per token tile
  int n_p;       // weight rows N (STORE, SCATTER: the last tile may hold only 128)
  const int4* table;
  const int* n_qtiles;
  const float* sx;  // activation scales [kred/128][ldsx] (k-block major)
  int64_t ldsx;
  const float* sw;  // weight block scales, expert e at sw + e * sw_estride: [N/128][kred/128]
  int64_t sw_estride;
  bf16_t* out;
  int64_t ldo;
  // EPI_SWIGLU
  int64_t hidden;
  float limit;  // NaN = no clamp
  bf16_t* h_out;
  int64_t ldh;
  // EPI_SCATTER
  const float* row_scale;
  const int* dest;
  int n_dest;
};

// Token tiles of the fp8 GEMM have at most this many rows.
constexpr int kFp8TileRows = 256;

int num_cus();

hipError_t launch_tile_map(const int* offs, int E, int M, int max_rows, void* ws,
                           hipStream_t stream);
// Forward GEMM over a tile table of at most kFwdTileRows rows per tile.
hipError_t launch_fwd_gemm(int epi, const FwdGemm& g, hipStream_t stream);
// dgrad GEMM (EPI_STORE or EPI_SWIGLU_BWD) over the same tile table.
hipError_t launch_dgrad_gemm(int epi, const DgradGemm& g, hipStream_t stream);
// fp8 forward GEMM over a tile table of at most kFp8TileRows rows per tile.
hipError_t launch_fp8_gemm(int epi, const Fp8Args& a, hipStream_t stream);

}  // namespace ttamd
