// Host-side launchers of the grouped GEMMs and the device tile scheduler.
//
// The GEMM kernels live in gemm_fwd.hip (forward, dgrad), gemm_wgrad.hip
// (weight gradient) and gemm_fp8.hip (fp8 forward); this file builds the
// token-row tile table on the device (no count reaches the host) and maps
// each C-ABI operation onto a kernel configuration.
//
// Reference semantics (torchtitanturbo/models/common/npu_gmm.py):
//   :17-18, :31, :38  torch._grouped_mm(x, w.transpose(-2, -1), offs)
//   :32-36            optional clamp with swiglu_limit
//   :37               npu_swiglu: silu(gate) * up, gate = first H columns
#include <algorithm>

#include "common.h"
#include "gemm_common.h"
#include "kernels.h"

namespace ttamd {

// ---------------------------------------------------------------------------
// Tile table: token tile i -> {expert, first row, end row}.  Built on the
// device from the inclusive group offsets, so no count reaches the host
// (block_tile_table: equal-height tiles of at most max_rows rows per
// expert).  A null offs means one expert (E == 1) with all M rows.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void tile_map_kernel(const int* __restrict__ offs, int E,
                                                        int M, int max_tiles, int max_rows,
                                                        int4* __restrict__ table,
                                                        int* __restrict__ count,
                                                        int* __restrict__ split_cnt) {
  __shared__ int sh[1024 / kWave + 1];
  auto range = [&](int e, int& r0, int& r1) {
    // offs == nullptr: one expert owning all M rows
    const int a = (e == 0 || !offs) ? 0 : offs[e - 1];
    const int b = offs ? offs[e] : M;
    r0 = min(max(a, 0), M);
    r1 = min(max(b, r0), M);
  };
  block_tile_table<1024>(range, E, max_tiles, max_rows, table, count, split_cnt, sh);
}

hipError_t launch_tile_map(const int* offs, int E, int M, int max_rows, void* ws, hipStream_t stream) {
  TileTable tt = tile_table_in(ws);
  return launch_k(false, tile_map_kernel, dim3(1), dim3(1024), 0, stream, offs, E, M, max_row_tiles(M, E),
                  max_rows, tt.table, tt.count, tt.split_cnt);
}

// ---------------------------------------------------------------------------
// Launchers.
// ---------------------------------------------------------------------------
int gemm_max_qtiles(int M, int E) { return max_row_tiles(M, E); }

int gemm_fwd_tile_rows() { return kFwdTileRows; }

static size_t al256(size_t b) { return (b + 255) & ~(size_t)255; }

// The tile plan: header, split-tile counters, tile table.
size_t gemm_plan_bytes(int64_t M, int E) {
  return sizeof(int4) + kSplitTiles * sizeof(int) + (size_t)max_row_tiles((int)M, E) * sizeof(int4) + 256;
}

// Partial sums of the split leftover tiles: one piece per workgroup at most.
static size_t gemm_split_bytes() { return (size_t)((num_cus() + 7) & ~7) * kSplitPartBytes; }

// GEMM workspace: the tile plan, then the partial-sum area.
size_t gemm_workspace_bytes(int64_t M, int E) { return al256(gemm_plan_bytes(M, E)) + gemm_split_bytes(); }

static float* split_part_in(void* ws, int M, int E) { return (float*)((char*)ws + al256(gemm_plan_bytes(M, E))); }

// One probe per host thread: a thread's arming stamps only the launches
// that thread makes (other threads' launches never see it).
Probe& probe() {
  thread_local Probe p;
  return p;
}

void gemm_probe_arm(hipEvent_t start, hipEvent_t end) {
  probe().gemm_start = start;
  probe().gemm_end = end;
}

void probe_chain_arm(const hipEvent_t* events, int n_launches) {
  Probe& p = probe();
  p.chain_n = p.chain_i = 0;
  for (int i = 0; i < 2 * n_launches; ++i) p.chain[i] = events[i];
  p.chain_n = n_launches > 0 ? n_launches : 0;
}

// plan: the tile plan; part: the partial-sum area of split leftover tiles
// (nullable: no split).  table_ready: `plan` already holds the tile table
// of these rows (built for kFwdTileRows-row tiles), so no tile-map launch.
static hipError_t fwd(int epi, FwdGemm g, const int* offs, int E, int M, void* plan, float* part,
                      hipStream_t stream, bool table_ready = false) {
  if (!table_ready) {
    hipError_t err = launch_tile_map(offs, E, M, kFwdTileRows, plan, stream);
    if (err != hipSuccess) return err;
  }
  const TileTable tt = tile_table_in(plan);
  g.table = tt.table;
  g.n_qtiles = tt.count;
  g.split_cnt = tt.split_cnt;
  g.part = part;
  return launch_fwd_gemm(epi, g, stream);
}
static hipError_t fwd(int epi, FwdGemm g, const int* offs, int E, int M, void* ws, hipStream_t stream) {
  return fwd(epi, g, offs, E, M, ws, split_part_in(ws, M, E), stream);
}

hipError_t launch_grouped_mm(const void* x, const void* w, const int* offs, int M, int E,
                             int N, int K, void* out, void* ws, hipStream_t stream) {
  FwdGemm g = {};
  g.act = x; g.w = w; g.kred = K; g.n = N; g.out = out;
  return fwd(EPI_STORE, g, offs, E, M, ws, stream);
}

hipError_t launch_grouped_mm_swiglu(const void* x, const void* w13, const int* offs, int M,
                                    int E, int H, int D, float limit, void* a_out, void* h_out,
                                    void* ws, hipStream_t stream) {
  FwdGemm g = {};
  g.act = x; g.w = w13; g.kred = D; g.n = H; g.out = a_out; g.limit = limit; g.h_out = h_out;
  return fwd(EPI_SWIGLU, g, offs, E, M, ws, stream);
}

hipError_t launch_grouped_mm_swiglu_gather(const void* tokens, int n_tokens, const int* src_index,
                                           int src_div, const void* w13, const int* offs, int M, int E,
                                           int H, int D, float limit, void* a_out, void* h_out, void* ws,
                                           hipStream_t stream) {
  FwdGemm g = {};
  g.act = tokens; g.act_index = src_index; g.act_div = src_div; g.n_act = n_tokens;
  g.w = w13; g.kred = D; g.n = H; g.out = a_out; g.limit = limit; g.h_out = h_out;
  return fwd(EPI_SWIGLU, g, offs, E, M, ws, stream);
}

hipError_t launch_grouped_mm_unpermute(const void* act, const void* w2, const int* offs, int M,
                                       int E, int D, int H, const float* row_scale,
                                       const int* dest, int n_dest, void* out, void* ws,
                                       hipStream_t stream) {
  FwdGemm g = {};
  g.act = act; g.w = w2; g.kred = H; g.n = D; g.out = out;
  g.row_scale = row_scale; g.dest = dest; g.n_dest = n_dest;
  return fwd(EPI_SCATTER, g, offs, E, M, ws, stream);
}

// ---- the expert stage of the MoE layer forward in one call ---------------------
size_t moe_experts_forward_workspace_bytes(int64_t T, int64_t D, int64_t H, int E, int K, bool permute_first) {
  const int64_t M = T * K;
  auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
  size_t n = al(gemm_workspace_bytes(M, E));                 // tile plan
  n += al((size_t)M * H * 2);                                // a = swiglu(x w13^T)
  if (permute_first) n += al((size_t)M * D * 2);             // routed rows
  if (K > 1) n += al((size_t)M * D * 2);                     // y in flat-slot order
  return n;
}

hipError_t launch_moe_experts_forward(const void* tokens, int T, int D, int H, int E, int K,
                                      const int* sorted_idx, const int* offs, const float* sorted_scores,
                                      bool score_before, float limit, const void* w13, const void* w2,
                                      void* out, void* plan, void* ws, hipStream_t stream) {
  const int M = T * K;
  const bool permute_first = score_before || D < 128;
  auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
  char* p = (char*)ws;
  void* own_plan = p;
  p += al(gemm_workspace_bytes(M, E));
  void* a = p;
  p += al((size_t)M * H * 2);
  void* routed = nullptr;
  if (permute_first) {
    routed = p;
    p += al((size_t)M * D * 2);
  }
  void* y = (K > 1) ? (void*)p : out;
  hipError_t err;
  // one tile table for both GEMMs
  void* tp = plan;
  float* part = split_part_in(own_plan, M, E);
  if (tp == nullptr) {
    tp = own_plan;
    if ((err = launch_tile_map(offs, E, M, kFwdTileRows, tp, stream)) != hipSuccess) return err;
  }
  if (permute_first) {
    err = launch_gather_rows(tokens, sorted_idx, score_before ? sorted_scores : nullptr, false, T, M, M, D, K,
                             routed, stream);
    if (err != hipSuccess) return err;
    FwdGemm g = {};
    g.act = routed; g.w = w13; g.kred = D; g.n = H; g.out = a; g.limit = limit;
    err = fwd(EPI_SWIGLU, g, offs, E, M, tp, part, stream, true);
  } else {
    FwdGemm g = {};
    g.act = tokens; g.act_index = sorted_idx; g.act_div = K; g.n_act = T;
    g.w = w13; g.kred = D; g.n = H; g.out = a; g.limit = limit;
    err = fwd(EPI_SWIGLU, g, offs, E, M, tp, part, stream, true);
  }
  if (err != hipSuccess) return err;
  FwdGemm g2 = {};
  g2.act = a; g2.w = w2; g2.kred = H; g2.n = D; g2.out = y;
  g2.row_scale = score_before ? nullptr : sorted_scores;
  g2.dest = sorted_idx;
  g2.n_dest = (K > 1) ? M : T;
  if ((err = fwd(EPI_SCATTER, g2, offs, E, M, tp, part, stream, true)) != hipSuccess) return err;
  if (K > 1) return launch_combine(y, nullptr, nullptr, T, K, D, out, stream);
  return hipSuccess;
}

// ---- fp8 forward (gemm_fp8.hip) ----------------------------------------------
static hipError_t fp8(int epi, Fp8Args a, const int* offs, int E, int M, void* ws,
                      hipStream_t stream) {
  hipError_t err = launch_tile_map(offs, E, M, kFp8TileRows, ws, stream);
  if (err != hipSuccess) return err;
  const TileTable tt = tile_table_in(ws);
  a.table = tt.table;
  a.n_qtiles = tt.count;
  return launch_fp8_gemm(epi, a, stream);
}

static Fp8Args fp8_args(const void* xq, const float* sx, const void* wq, const float* sw, int M,
                        int N_rows, int K) {
  Fp8Args a = {};
  a.q = (const uint8_t*)xq;
  a.ldq = K;
  a.p = (const uint8_t*)wq;
  a.p_estride = (int64_t)N_rows * K;
  a.ldp = K;
  a.kred = K;
  a.sx = sx;
  a.ldsx = M;
  a.sw = sw;
  a.sw_estride = (int64_t)(N_rows / 128) * (K / 128);
  return a;
}

hipError_t launch_grouped_mm_fp8(const void* xq, const float* sx, const void* wq, const float* sw,
                                 const int* offs, int M, int E, int N, int K, void* out, void* ws,
                                 hipStream_t stream) {
  Fp8Args a = fp8_args(xq, sx, wq, sw, M, N, K);
  a.np_tiles = (N + 255) / 256;
  a.n_p = N;
  a.out = (bf16_t*)out;
  a.ldo = N;
  return fp8(EPI_STORE, a, offs, E, M, ws, stream);
}

hipError_t launch_grouped_mm_fp8_swiglu(const void* xq, const float* sx, const void* w13q,
                                        const float* s13, const int* offs, int M, int E, int H, int D,
                                        float limit, void* a_out, void* h_out, void* ws,
                                        hipStream_t stream) {
  Fp8Args a = fp8_args(xq, sx, w13q, s13, M, 2 * H, D);
  a.np_tiles = (H + 127) / 128;  // 128 gate + 128 up rows per tile (H % 64 == 0)
  a.n_p = 2 * H;
  a.out = (bf16_t*)a_out;
  a.ldo = H;
  a.hidden = H;
  a.limit = limit;
  a.h_out = (bf16_t*)h_out;
  a.ldh = 2 * (int64_t)H;
  return fp8(EPI_SWIGLU, a, offs, E, M, ws, stream);
}

hipError_t launch_grouped_mm_fp8_unpermute(const void* aq, const float* sa, const void* w2q,
                                           const float* s2, const int* offs, int M, int E, int D, int H,
                                           const float* row_scale, const int* dest, int n_dest,
                                           void* out, void* ws, hipStream_t stream) {
  Fp8Args a = fp8_args(aq, sa, w2q, s2, M, D, H);
  a.np_tiles = (D + 255) / 256;
  a.n_p = D;
  a.out = (bf16_t*)out;
  a.ldo = D;
  a.row_scale = row_scale;
  a.dest = dest;
  a.n_dest = n_dest;
  return fp8(EPI_SCATTER, a, offs, E, M, ws, stream);
}

static hipError_t dgrad(int epi, DgradGemm g, const int* offs, int E, int M, void* plan, float* part,
                        hipStream_t stream) {
  hipError_t err = launch_tile_map(offs, E, M, kFwdTileRows, plan, stream);
  if (err != hipSuccess) return err;
  const TileTable tt = tile_table_in(plan);
  g.table = tt.table;
  g.n_qtiles = tt.count;
  g.split_cnt = tt.split_cnt;
  g.part = part;
  return launch_dgrad_gemm(epi, g, stream);
}

hipError_t launch_shared_expert_add(const void* x, int T, int D, int H, const void* w13s, const void* w2s,
                                   const float* gate_logits, float limit, void* a_scratch, void* out,
                                   void* ws, hipStream_t stream) {
  // one expert with all T rows: a = swiglu(x w13s^T), then out += g(t) * (a w2s^T)
  FwdGemm g1 = {};
  g1.act = x; g1.w = w13s; g1.kred = D; g1.n = H; g1.out = a_scratch; g1.limit = limit;
  hipError_t err = fwd(EPI_SWIGLU, g1, nullptr, 1, T, ws, stream);
  if (err != hipSuccess) return err;
  FwdGemm g2 = {};
  g2.act = a_scratch; g2.w = w2s; g2.kred = H; g2.n = D; g2.out = out; g2.n_dest = T;
  g2.row_scale = gate_logits; g2.scale_sigmoid = 1; g2.accumulate = 1;
  return fwd(EPI_SCATTER, g2, nullptr, 1, T, ws, stream);
}

hipError_t launch_grouped_mm_dgrad(const void* dy, const void* w, const int* offs, int M, int E,
                                   int N, int K, void* dx, void* ws, hipStream_t stream) {
  // dx[m][k] = sum_n dy[m][n] w[e][n][k]
  DgradGemm g = {};
  g.dy = dy; g.w = w; g.n_red = N; g.n_out = K; g.out = dx;
  return dgrad(EPI_STORE, g, offs, E, M, ws, split_part_in(ws, M, E), stream);
}

hipError_t launch_grouped_mm_dgrad_unsplit(const void* dy, const void* w, const int* offs, int M, int E, int N,
                                           int K, void* dx, void* plan, hipStream_t stream) {
  DgradGemm g = {};
  g.dy = dy; g.w = w; g.n_red = N; g.n_out = K; g.out = dx;
  return dgrad(EPI_STORE, g, offs, E, M, plan, nullptr, stream);
}

hipError_t launch_grouped_mm_dgrad_swiglu(const void* dy, const void* w2, const void* h,
                                          const int* offs, int M, int E, int D, int H,
                                          float limit, void* dh, void* a_out, void* ws,
                                          hipStream_t stream) {
  // g[m][p] = sum_d dy[m][d] w2[e][d][p], then the SwiGLU backward with h
  DgradGemm g = {};
  g.dy = dy; g.w = w2; g.n_red = D; g.n_out = H; g.out = dh; g.h = h; g.limit = limit; g.a_out = a_out;
  return dgrad(EPI_SWIGLU_BWD, g, offs, E, M, ws, split_part_in(ws, M, E), stream);
}

hipError_t launch_grouped_mm_wgrad(const void* dy, const void* x, const int* offs, int M, int E,
                                   int N, int K, void* dw, bool fp32, void* ws, hipStream_t stream) {
  WgradDmaArgs a = {};
  a.dy = (const bf16_t*)dy; a.lddy = N;
  a.x = (const bf16_t*)x; a.ldx = K;
  a.offs = offs; a.E = E; a.M = M; a.N = N; a.K = K;
  a.n_tiles = (N + 255) / 256; a.k_tiles = (K + 255) / 256;
  a.dw = dw; a.dw_fp32 = fp32 ? 1 : 0;
  a.split_np = 1;
  if (ws != nullptr) {
    // Tail split for a walk of at most kSplitMaxRounds full rounds with
    // tiles left over: up to kSplitMaxPieces pieces per leftover tile, so
    // that the pieces fill the otherwise idle workgroups, each piece of at
    // least kSplitMinStages stages of the average expert's rows.
    const int G = (num_cus() + 7) & ~7;
    const int ntiles = E * a.n_tiles * a.k_tiles;
    const int R = ntiles / G, rt = ntiles - R * G;
    if (rt > 0 && rt <= kSplitTiles && R <= kSplitMaxRounds) {
      int np = std::min(kSplitMaxPieces, G / rt);
      const int avg_stages = (M / E + 63) / 64;
      while (np > 1 && avg_stages < np * kSplitMinStages) --np;
      if (np > 1) {
        TileTable tt = tile_table_in(ws);
        hipError_t err = launch_split_cnt_zero(tt.split_cnt, rt, stream);
        if (err != hipSuccess) return err;
        a.part = split_part_in(ws, M, E);
        a.split_cnt = tt.split_cnt;
        a.split_np = np;
      }
    }
  }
  return launch_wgrad_dma(a, stream);
}

}  // namespace ttamd
