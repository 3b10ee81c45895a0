// Grouped GEMMs over ragged expert segments on MI355X (gfx950) MFMA.
//
// One kernel family computes C^T tiles with v_mfma_f32_32x32x16_bf16: the
// MFMA "A" operand is the matrix whose index is the output's contiguous
// dimension (P), the "B" operand the one indexing output rows (Q), so each
// lane ends up holding 4 consecutive output columns per register group and
// the epilogue stores 8-byte (bf16) / 16-byte (fp32) pieces.
//
//   rows kernel  (forward, dgrad): output rows q are routed token rows,
//                grouped by expert through a device tile table (no host
//                sync); the reduction length is fixed (D or H);
//   wgrad kernel: output is one [N, K] weight gradient per expert, the
//                reduction runs over the expert's ragged row range.
//
// Tiles are 128 (P) x 128 (Q) x 64 (k), 256 threads = 4 waves in a 2 x 2
// arrangement, each wave 64 x 64 = 2 x 2 MFMA blocks.  Both operands are
// staged through LDS in a k-contiguous layout with a 16-byte-chunk XOR
// swizzle (conflict-free MFMA fragment reads), double-buffered so the global
// loads of step k+1 are in flight while step k runs on the matrix cores.
// Operands whose memory layout has the reduction index strided (the weight
// in dgrad, both operands in wgrad) are transposed in registers (8 x 4 bf16
// blocks) on their way into LDS.
//
// Reference semantics (torchtitanturbo/models/common/npu_gmm.py):
//   :17-18, :31, :38  torch._grouped_mm(x, w.transpose(-2, -1), offs)
//   :32-36            optional clamp with swiglu_limit
//   :37               npu_swiglu: silu(gate) * up, gate = first H columns
#include "common.h"
#include "gemm_common.h"
#include "kernels.h"

namespace ttamd {

constexpr int BP = 128;  // tile extent along P (output contiguous dim)
constexpr int BQ = 128;  // tile extent along Q (output rows)
constexpr int BK = 64;   // reduction step
constexpr int kGemmThreads = 256;
constexpr int kTileElems = 128 * BK;  // one operand tile in LDS (bf16)

// Physical 16-byte chunk of logical chunk c in LDS row r.
__device__ __forceinline__ int swz(int r, int c) { return c ^ ((r ^ (r >> 2)) & 7); }

__device__ __forceinline__ int lds_off(int r, int c) { return r * BK + swz(r, c) * 8; }

// ---------------------------------------------------------------------------
// Tile table: token tile i -> {expert, first row, end row}.  Built on the
// device from the inclusive group offsets, so no count reaches the host.
// An expert's rows are split into the fewest tiles of at most max_rows rows,
// of equal height rounded up to 32 rows (540 rows at max_rows = 256 give
// 3 tiles of 192 rather than 256 + 256 + 28).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void tile_map_kernel(const int* __restrict__ offs, int E,
                                                        int M, int max_tiles, int max_rows,
                                                        int4* __restrict__ table,
                                                        int* __restrict__ count) {
  __shared__ int wave_sums[16];
  const int tid = threadIdx.x;
  int r0 = 0, r1 = 0, nt = 0, h = max_rows;
  if (tid < E) {
    const int a = (tid == 0) ? 0 : offs[tid - 1];
    const int b = offs[tid];
    r0 = min(max(a, 0), M);
    r1 = min(max(b, r0), M);
    const int c = r1 - r0;
    if (c > 0) {
      const int n0 = (c + max_rows - 1) / max_rows;
      h = (((c + n0 - 1) / n0) + 31) & ~31;
      nt = (c + h - 1) / h;
    }
  }
  const int incl = wave_inclusive_scan(nt);
  const int w = tid / kWave, l = lane_id();
  if (l == kWave - 1) wave_sums[w] = incl;
  __syncthreads();
  if (w == 0) {
    const int v = (l < 16) ? wave_sums[l] : 0;
    const int vi = wave_inclusive_scan(v);
    if (l < 16) wave_sums[l] = vi;  // inclusive
  }
  __syncthreads();
  const int start = ((w > 0) ? wave_sums[w - 1] : 0) + incl - nt;
  const int total = wave_sums[15];
  for (int t = 0; t < nt; ++t) {
    const int i = start + t;
    if (i < max_tiles) table[i] = make_int4(tid, r0 + t * h, min(r0 + (t + 1) * h, r1), 0);
  }
  for (int i = total + tid; i < max_tiles; i += 1024) table[i] = make_int4(-1, 0, 0, 0);
  if (tid == 0) *count = min(total, max_tiles);
}

hipError_t launch_tile_map(const int* offs, int E, int M, int max_rows, void* ws, hipStream_t stream) {
  TileTable tt = tile_table_in(ws);
  hipLaunchKernelGGL(tile_map_kernel, dim3(1), dim3(1024), 0, stream, offs, E, M,
                     max_row_tiles(M, E), max_rows, tt.table, tt.count);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Operand loaders.  A thread moves 4 x 16 bytes of a 128 x 64 tile per step.
// ---------------------------------------------------------------------------

// k-contiguous source: row r of the tile is at src_row(r) * ld + k0.
struct DirectLoad {
  u32x4_t v[4];
};

// Source with the row index contiguous: element (r, k) at (k0 + k) * ld + r0 + r.
// A thread loads an 8 (k) x 4 (r) block as 8 x 8 bytes.
struct TransLoad {
  u32x2_t v[8];
};

__device__ __forceinline__ void store_direct(bf16_t* lds, const DirectLoad& d) {
  const int t = threadIdx.x;
  const int c = t & 7;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = (t >> 3) + 32 * i;
    *(u32x4_t*)(lds + lds_off(r, c)) = d.v[i];
  }
}

__device__ __forceinline__ void store_trans(bf16_t* lds, const TransLoad& d) {
  const int t = threadIdx.x;
  const int pc = t & 31;  // 4-row group
  const int kb = t >> 5;  // 8-k chunk
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = pc * 4 + j;
    u32x4_t o;
    // element j of each k row: dword (j >> 1), half (j & 1)
    uint32_t e[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t dw = (j < 2) ? d.v[i].x : d.v[i].y;
      e[i] = (j & 1) ? (dw >> 16) : (dw & 0xffffu);
    }
    o.x = e[0] | (e[1] << 16);
    o.y = e[2] | (e[3] << 16);
    o.z = e[4] | (e[5] << 16);
    o.w = e[6] | (e[7] << 16);
    *(u32x4_t*)(lds + lds_off(r, kb)) = o;
  }
}

// ---------------------------------------------------------------------------
// MFMA block: the wave's 2 x 2 blocks of 32 x 32 over one BK step.
// prow[pb], qrow[qb]: first LDS row of each 32-row block.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void mfma_step(const bf16_t* ldsP, const bf16_t* ldsQ,
                                          const int prow[2], const int qrow[2],
                                          floatx16_t acc[2][2]) {
  const int l = lane_id();
  const int r32 = l & 31;
  const int half = l >> 5;
#pragma unroll
  for (int kk = 0; kk < BK / 16; ++kk) {
    const int c = kk * 2 + half;
    bf16x8_t pf[2], qf[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int rp = prow[b] + r32;
      const int rq = qrow[b] + r32;
      pf[b] = *(const bf16x8_t*)(ldsP + lds_off(rp, c));
      qf[b] = *(const bf16x8_t*)(ldsQ + lds_off(rq, c));
    }
#pragma unroll
    for (int pb = 0; pb < 2; ++pb)
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
        acc[pb][qb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pf[pb], qf[qb], acc[pb][qb], 0, 0, 0);
  }
}

// ---------------------------------------------------------------------------
// Rows kernel (forward and dgrad).
// ---------------------------------------------------------------------------
struct RowsArgs {
  const bf16_t* q;  // activations [M][Kred], k contiguous
  int64_t ldq;
  const bf16_t* p;  // weights, per expert at p + e * p_estride
  int64_t p_estride;
  int64_t ldp;  // !P_TRANS: row stride of [N][Kred]; P_TRANS: row stride of [Kred][N]
  int kred;
  int np_tiles;
  int max_qtiles;
  int grid_per_xcd;
  const int4* table;
  bf16_t* out;
  int64_t ldo;
  // EPI_SWIGLU / EPI_SWIGLU_BWD
  int64_t hidden;  // H: up rows start at H in w13, up cols at H in h / dh
  float limit;     // NaN = no clamp
  bf16_t* h_out;   // SWIGLU: pre-activation out (nullable)
  const bf16_t* h_in;  // SWIGLU_BWD: saved pre-activation
  bf16_t* a_out;       // SWIGLU_BWD: recomputed activation (nullable)
  int64_t ldh;
  // EPI_SCATTER
  const float* row_scale;
  const int* dest;
  int n_dest;
};

template <int EPI, bool P_TRANS>
__global__ __launch_bounds__(kGemmThreads) void gg_rows_kernel(const RowsArgs args) {
  // XCD-aware remap: consecutive hardware block ids go round-robin over the
  // 8 XCDs; give each XCD a contiguous range of logical tiles so blocks that
  // share an expert's weights and a q-tile's rows meet in the same L2.
  const int bid = blockIdx.x;
  const int logical = (bid & 7) * args.grid_per_xcd + (bid >> 3);
  const int qt = logical / args.np_tiles;
  const int pt = logical - qt * args.np_tiles;
  if (qt >= args.max_qtiles) return;
  const int4 tile = args.table[qt];
  const int e = tile.x;
  if (e < 0) return;
  const int row0 = tile.y, row1 = tile.z;

  __shared__ __attribute__((aligned(16))) bf16_t lds[2][2][kTileElems];  // [buf][P/Q]

  const int t = threadIdx.x;
  const int wave = t / kWave;
  const int wp = wave & 1, wq = wave >> 1;
  const int l = lane_id();

  // ---- source addresses -------------------------------------------------
  // Row offsets are recomputed per load from loop invariants (the compiler
  // hoists them); keeping them in arrays would push them to scratch.
  const bf16_t* pbase = args.p + (int64_t)e * args.p_estride;
  const bf16_t* qbase = args.q + (t & 7) * 8;
  const int rq0 = row0 + (t >> 3);
  const int rqmax = row1 - 1;
  const bf16_t* pdbase = pbase + (t & 7) * 8;
  const bf16_t* ptsrc = pbase + (int64_t)((t >> 5) * 8) * args.ldp + pt * BP + (t & 31) * 4;

#define TTAMD_LOAD_Q(k0, d)                                                       \
  _Pragma("unroll") for (int i = 0; i < 4; ++i) {                                 \
    const int gr = min(rq0 + 32 * i, rqmax);                                      \
    (d).v[i] = *(const u32x4_t*)(qbase + (int64_t)gr * args.ldq + (k0));            \
  }
#define TTAMD_LOAD_P(k0, d)                                                       \
  _Pragma("unroll") for (int i = 0; i < 4; ++i) {                                 \
    const int r = (t >> 3) + 32 * i;                                              \
    int prow;                                                                     \
    if constexpr (EPI == EPI_SWIGLU)                                              \
      prow = (r < 64) ? pt * 64 + r : (int)args.hidden + pt * 64 + (r - 64);      \
    else                                                                          \
      prow = pt * BP + r;                                                         \
    (d).v[i] = *(const u32x4_t*)(pdbase + (int64_t)prow * args.ldp + (k0));         \
  }
#define TTAMD_LOAD_PT(k0, d)                                                      \
  _Pragma("unroll") for (int i = 0; i < 8; ++i)                                   \
    (d).v[i] = *(const u32x2_t*)(ptsrc + (int64_t)((k0) + i) * args.ldp);

  floatx16_t acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[a][b][i] = 0.f;

  int prow_l[2], qrow_l[2];
  if constexpr (EPI == EPI_SWIGLU) {
    prow_l[0] = wp * 32;       // gate block
    prow_l[1] = 64 + wp * 32;  // matching up block
  } else {
    prow_l[0] = wp * 64;
    prow_l[1] = wp * 64 + 32;
  }
  qrow_l[0] = wq * 64;
  qrow_l[1] = wq * 64 + 32;

  const int ksteps = args.kred / BK;
  DirectLoad dq, dp;
  TransLoad dpt;
  TTAMD_LOAD_Q(0, dq);
  if constexpr (P_TRANS) { TTAMD_LOAD_PT(0, dpt); } else { TTAMD_LOAD_P(0, dp); }
  store_direct(lds[0][1], dq);
  if constexpr (P_TRANS) store_trans(lds[0][0], dpt); else store_direct(lds[0][0], dp);
  __syncthreads();

  for (int ks = 0; ks < ksteps; ++ks) {
    const int cur = ks & 1;
    const bool more = ks + 1 < ksteps;
    if (more) {
      const int k0 = (ks + 1) * BK;
      TTAMD_LOAD_Q(k0, dq);
      if constexpr (P_TRANS) { TTAMD_LOAD_PT(k0, dpt); } else { TTAMD_LOAD_P(k0, dp); }
    }
    mfma_step(lds[cur][0], lds[cur][1], prow_l, qrow_l, acc);
    if (more) {
      store_direct(lds[cur ^ 1][1], dq);
      if constexpr (P_TRANS) store_trans(lds[cur ^ 1][0], dpt); else store_direct(lds[cur ^ 1][0], dp);
    }
    __syncthreads();
  }

#undef TTAMD_LOAD_Q
#undef TTAMD_LOAD_P
#undef TTAMD_LOAD_PT

  // ---- epilogue ----------------------------------------------------------
  // acc[pb][qb][4g + i]: Q row = qrow_l[qb] + (l & 31),
  //                      P col = prow_l[pb] + 8g + 4 * (l >> 5) + i.
  const int half = l >> 5;
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int gq = row0 + qrow_l[qb] + (l & 31);
    if (gq >= row1) continue;
    if constexpr (EPI == EPI_SWIGLU) {
      const bool clamp = (args.limit == args.limit);
      const float L = args.limit;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int col = pt * 64 + wp * 32 + 8 * g + 4 * half;
        float av[4], gv[4], uv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          // h is bf16 in the reference (grouped_mm output); SwiGLU reads it.
          gv[i] = round_bf16(acc[0][qb][4 * g + i]);
          uv[i] = round_bf16(acc[1][qb][4 * g + i]);
          float gc = gv[i], uc = uv[i];
          if (clamp) {
            gc = fminf(gc, L);
            uc = fminf(fmaxf(uc, -L), L);
          }
          av[i] = silu_f(gc) * uc;
        }
        bf16_t* orow = args.out + (int64_t)gq * args.ldo + col;
        *(uint2*)orow = make_uint2(pack_bf16x2(av[0], av[1]), pack_bf16x2(av[2], av[3]));
        if (args.h_out) {
          bf16_t* hrow = args.h_out + (int64_t)gq * args.ldh + col;
          *(uint2*)hrow = make_uint2(pack_bf16x2(gv[0], gv[1]), pack_bf16x2(gv[2], gv[3]));
          *(uint2*)(hrow + args.hidden) =
              make_uint2(pack_bf16x2(uv[0], uv[1]), pack_bf16x2(uv[2], uv[3]));
        }
      }
    } else if constexpr (EPI == EPI_SWIGLU_BWD) {
      const bool clamp = (args.limit == args.limit);
      const float L = args.limit;
#pragma unroll
      for (int pb = 0; pb < 2; ++pb) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int col = pt * BP + prow_l[pb] + 8 * g + 4 * half;
          const bf16_t* hrow = args.h_in + (int64_t)gq * args.ldh + col;
          const uint2 hg = *(const uint2*)hrow;
          const uint2 hu = *(const uint2*)(hrow + args.hidden);
          const float gate[4] = {bf16_to_f32(hg.x & 0xffff), bf16_to_f32(hg.x >> 16),
                                 bf16_to_f32(hg.y & 0xffff), bf16_to_f32(hg.y >> 16)};
          const float up[4] = {bf16_to_f32(hu.x & 0xffff), bf16_to_f32(hu.x >> 16),
                               bf16_to_f32(hu.y & 0xffff), bf16_to_f32(hu.y >> 16)};
          float dg[4], du[4], av[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float gd = acc[pb][qb][4 * g + i];
            float gc = gate[i], uc = up[i];
            float mg = 1.f, mu = 1.f;
            if (clamp) {
              if (gc > L) { gc = L; mg = 0.f; }
              if (uc > L) { uc = L; mu = 0.f; }
              if (uc < -L) { uc = -L; mu = 0.f; }
            }
            const float sig = 1.f / (1.f + __expf(-gc));
            const float s = gc * sig;
            const float ds = sig * (1.f + gc * (1.f - sig));
            dg[i] = gd * uc * ds * mg;
            du[i] = gd * s * mu;
            av[i] = s * uc;
          }
          bf16_t* drow = args.out + (int64_t)gq * args.ldo + col;
          *(uint2*)drow = make_uint2(pack_bf16x2(dg[0], dg[1]), pack_bf16x2(dg[2], dg[3]));
          *(uint2*)(drow + args.hidden) =
              make_uint2(pack_bf16x2(du[0], du[1]), pack_bf16x2(du[2], du[3]));
          if (args.a_out) {
            bf16_t* arow = args.a_out + (int64_t)gq * args.hidden + col;
            *(uint2*)arow = make_uint2(pack_bf16x2(av[0], av[1]), pack_bf16x2(av[2], av[3]));
          }
        }
      }
    } else {
      int64_t orow_idx = gq;
      float sc = 1.f;
      if constexpr (EPI == EPI_SCATTER) {
        if (args.dest) orow_idx = min(max(args.dest[gq], 0), args.n_dest - 1);
        if (args.row_scale) sc = args.row_scale[gq];
      }
      bf16_t* orow = args.out + orow_idx * args.ldo + pt * BP;
#pragma unroll
      for (int pb = 0; pb < 2; ++pb) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int col = prow_l[pb] + 8 * g + 4 * half;
          const float v[4] = {acc[pb][qb][4 * g], acc[pb][qb][4 * g + 1], acc[pb][qb][4 * g + 2],
                              acc[pb][qb][4 * g + 3]};
          *(uint2*)(orow + col) =
              make_uint2(pack_bf16x2(v[0] * sc, v[1] * sc), pack_bf16x2(v[2] * sc, v[3] * sc));
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Wgrad kernel: dw[e][n][k] = sum_{m in group e} dy[m][n] * x[m][k].
// MFMA A operand indexes k (the output's contiguous dim), B indexes n; both
// come from row-major [M][.] activations, i.e. reduction-strided, and are
// transposed in registers.  Rows outside the group load as zeros.
// ---------------------------------------------------------------------------
struct WgradArgs {
  const bf16_t* dy;  // [M][N]
  int64_t lddy;
  const bf16_t* x;  // [M][K]
  int64_t ldx;
  const int* offs;  // inclusive, [E]
  int E, M;
  int n_tiles, k_tiles;  // per expert: N / 128, K / 128
  int grid_per_xcd;
  void* dw;  // [E][N][K]
  int dw_fp32;
  int64_t N, K;
};

__global__ __launch_bounds__(kGemmThreads) void gg_wgrad_kernel(const WgradArgs args) {
  const int bid = blockIdx.x;
  const int logical = (bid & 7) * args.grid_per_xcd + (bid >> 3);
  const int per_e = args.n_tiles * args.k_tiles;
  const int e = logical / per_e;
  if (e >= args.E) return;
  const int rem = logical - e * per_e;
  const int nt = rem / args.k_tiles;
  const int kt = rem - nt * args.k_tiles;
  int m0 = (e == 0) ? 0 : args.offs[e - 1];
  int m1 = args.offs[e];
  m0 = min(max(m0, 0), args.M);
  m1 = min(max(m1, m0), args.M);

  __shared__ __attribute__((aligned(16))) bf16_t lds[2][2][kTileElems];  // [buf][P=x / Q=dy]

  const int t = threadIdx.x;
  const int wave = t / kWave;
  const int wp = wave & 1, wq = wave >> 1;
  const int l = lane_id();

  // transposed loads: element (r, m) at base + m * ld + col0 + r
  const int kb = t >> 5;
  const int rc = (t & 31) * 4;
  const bf16_t* xs = args.x + kt * 128 + rc;
  const bf16_t* ys = args.dy + nt * 128 + rc;

  auto load = [&](const bf16_t* base, int64_t ld, int mstart, TransLoad& d) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int m = mstart + kb * 8 + i;
      d.v[i] = (m < m1) ? *(const u32x2_t*)(base + (int64_t)m * ld) : u32x2_t{0u, 0u};
    }
  };

  floatx16_t acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[a][b][i] = 0.f;
  int prow_l[2] = {wp * 64, wp * 64 + 32};
  int qrow_l[2] = {wq * 64, wq * 64 + 32};

  const int ksteps = (m1 - m0 + BK - 1) / BK;
  if (ksteps > 0) {
    TransLoad dx, dd;
    load(xs, args.ldx, m0, dx);
    load(ys, args.lddy, m0, dd);
    store_trans(lds[0][0], dx);
    store_trans(lds[0][1], dd);
    __syncthreads();
    for (int ks = 0; ks < ksteps; ++ks) {
      const int cur = ks & 1;
      const bool more = ks + 1 < ksteps;
      if (more) {
        const int ms = m0 + (ks + 1) * BK;
        load(xs, args.ldx, ms, dx);
        load(ys, args.lddy, ms, dd);
      }
      mfma_step(lds[cur][0], lds[cur][1], prow_l, qrow_l, acc);
      if (more) {
        store_trans(lds[cur ^ 1][0], dx);
        store_trans(lds[cur ^ 1][1], dd);
      }
      __syncthreads();
    }
  }

  const int half = l >> 5;
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int64_t n = (int64_t)nt * 128 + qrow_l[qb] + (l & 31);
    const int64_t rowoff = ((int64_t)e * args.N + n) * args.K + (int64_t)kt * 128;
#pragma unroll
    for (int pb = 0; pb < 2; ++pb) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int col = prow_l[pb] + 8 * g + 4 * half;
        const float v[4] = {acc[pb][qb][4 * g], acc[pb][qb][4 * g + 1], acc[pb][qb][4 * g + 2],
                            acc[pb][qb][4 * g + 3]};
        if (args.dw_fp32) {
          *(float4*)((float*)args.dw + rowoff + col) = make_float4(v[0], v[1], v[2], v[3]);
        } else {
          *(uint2*)((bf16_t*)args.dw + rowoff + col) =
              make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Host-side launchers.
// ---------------------------------------------------------------------------
int gemm_max_qtiles(int M, int E) { return max_row_tiles(M, E); }

size_t gemm_workspace_bytes(int64_t M, int E) {
  return (size_t)(max_row_tiles((int)M, E) + 1) * sizeof(int4) + 256;
}

static int round_up8(int x) { return (x + 7) & ~7; }

static hipError_t launch_rows(int epi, bool ptrans, RowsArgs a, const int* offs, int E, int M,
                              void* ws, hipStream_t stream) {
  const int max_q = gemm_max_qtiles(M, E);
  hipError_t err = launch_tile_map(offs, E, M, BQ, ws, stream);
  if (err != hipSuccess) return err;
  a.table = tile_table_in(ws).table;
  a.max_qtiles = max_q;
  const int grid = round_up8(max_q * a.np_tiles);
  a.grid_per_xcd = grid / 8;
  // Only the dgrad orientation (weight reduction index strided) runs here.
  if (!ptrans) return hipErrorInvalidValue;
  if (epi == EPI_STORE)
    hipLaunchKernelGGL((gg_rows_kernel<EPI_STORE, true>), dim3(grid), dim3(kGemmThreads), 0, stream, a);
  else
    hipLaunchKernelGGL((gg_rows_kernel<EPI_SWIGLU_BWD, true>), dim3(grid), dim3(kGemmThreads), 0, stream, a);
  return hipGetLastError();
}

static hipError_t fwd(int epi, FwdGemm g, const int* offs, int E, int M, void* ws,
                      hipStream_t stream) {
  hipError_t err = launch_tile_map(offs, E, M, kFwdTileRows, ws, stream);
  if (err != hipSuccess) return err;
  const TileTable tt = tile_table_in(ws);
  g.table = tt.table;
  g.n_qtiles = tt.count;
  return launch_fwd_gemm(epi, g, stream);
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
  a.np_tiles = N / 128;
  a.out = (bf16_t*)out;
  a.ldo = N;
  return fp8(EPI_STORE, a, offs, E, M, ws, stream);
}

hipError_t launch_grouped_mm_fp8_swiglu(const void* xq, const float* sx, const void* w13q,
                                        const float* s13, const int* offs, int M, int E, int H, int D,
                                        float limit, void* a_out, void* h_out, void* ws,
                                        hipStream_t stream) {
  Fp8Args a = fp8_args(xq, sx, w13q, s13, M, 2 * H, D);
  a.np_tiles = H / 64;
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
  a.np_tiles = D / 128;
  a.out = (bf16_t*)out;
  a.ldo = D;
  a.row_scale = row_scale;
  a.dest = dest;
  a.n_dest = n_dest;
  return fp8(EPI_SCATTER, a, offs, E, M, ws, stream);
}

static hipError_t dgrad(int epi, DgradGemm g, const int* offs, int E, int M, void* ws,
                        hipStream_t stream) {
  hipError_t err = launch_tile_map(offs, E, M, kFwdTileRows, ws, stream);
  if (err != hipSuccess) return err;
  const TileTable tt = tile_table_in(ws);
  g.table = tt.table;
  g.n_qtiles = tt.count;
  return launch_dgrad_gemm(epi, g, stream);
}

hipError_t launch_grouped_mm_dgrad(const void* dy, const void* w, const int* offs, int M, int E,
                                   int N, int K, void* dx, void* ws, hipStream_t stream) {
  // dx[m][k] = sum_n dy[m][n] w[e][n][k]
  DgradGemm g = {};
  g.dy = dy; g.w = w; g.n_red = N; g.n_out = K; g.out = dx;
  return dgrad(EPI_STORE, g, offs, E, M, ws, stream);
}

hipError_t launch_grouped_mm_dgrad_swiglu(const void* dy, const void* w2, const void* h,
                                          const int* offs, int M, int E, int D, int H,
                                          float limit, void* dh, void* a_out, void* ws,
                                          hipStream_t stream) {
  // g[m][p] = sum_d dy[m][d] w2[e][d][p], then the SwiGLU backward with h
  DgradGemm g = {};
  g.dy = dy; g.w = w2; g.n_red = D; g.n_out = H; g.out = dh; g.h = h; g.limit = limit; g.a_out = a_out;
  return dgrad(EPI_SWIGLU_BWD, g, offs, E, M, ws, stream);
}

hipError_t launch_grouped_mm_wgrad(const void* dy, const void* x, const int* offs, int M, int E,
                                   int N, int K, void* dw, bool fp32, hipStream_t stream) {
  WgradDmaArgs a = {};
  a.dy = (const bf16_t*)dy; a.lddy = N;
  a.x = (const bf16_t*)x; a.ldx = K;
  a.offs = offs; a.E = E; a.M = M; a.N = N; a.K = K;
  a.n_tiles = (N + 255) / 256; a.k_tiles = (K + 255) / 256;
  a.dw = dw; a.dw_fp32 = fp32 ? 1 : 0;
  return launch_wgrad_dma(a, stream);
}

}  // namespace ttamd
