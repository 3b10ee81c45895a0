// Persistent grouped GEMM for the expert FFN forward on MI355X (gfx950).
//
//   out[q, p] = sum_k act[q, k] * w[e(q), p, k]        (k contiguous in both)
//
// q runs over routed token rows grouped by expert (ragged segments), p over
// weight rows.  Used for the w13 up-projection with SwiGLU fused into the
// epilogue, for the w2 down-projection with the routing-weight scale and the
// un-permute scatter fused into the epilogue, and for the plain grouped GEMM.
//
// Tile: 128 token rows (Q) x 256 weight rows (P), k in stages of 64.
//   * 4 waves, one per SIMD; wave w owns all 128 Q rows and 64 P rows, i.e.
//     2 x 4 accumulators of v_mfma_f32_32x32x16_bf16 (128 fp32 AGPRs/lane).
//     The MFMA A operand is the weight tile (P), B the token tile (Q), so a
//     lane holds 4 consecutive output columns per register group.
//   * Three LDS stage buffers of 48 KB (32 KB weights + 16 KB tokens) filled
//     by global_load_lds_dwordx4 (HBM/L2 -> LDS, no VGPR staging).  LDS rows
//     are 128 B; the 16-byte chunk c of row r sits at c ^ ((r >> 1) & 7).  A
//     wave's DMA writes 1 KB of LDS contiguously, so the permutation is
//     applied to the global addresses instead.
//   * Register-level pipeline: while the 32 MFMAs of stage i run, the wave
//     reads all 24 MFMA fragments of stage i + 1 from LDS into a second
//     register set.  The LDS buffer of the stage being computed is therefore
//     free, and three stages (i + 1 .. i + 3) are in flight or landed.
//   * DMA addresses: per tile, a wave-uniform byte base (SGPRs) plus one
//     32-bit per-lane offset per DMA instruction; per stage only the uniform
//     k offset changes, so each DMA is a single instruction.
//   * Persistent: one workgroup per CU walks the tile list with stride
//     gridDim.x; the pipeline runs over the flattened (tile, k-stage)
//     sequence, so the next tile's first stages load during the current
//     tile's last ones.  Within a round the 32 workgroups of one XCD take 32
//     consecutive tiles (same expert), so the weights are shared in its L2.
//   * The last Q tile of an expert is usually partial: the MFMAs of 32-row
//     blocks past the expert's end are skipped (per-tile specialisation).
//
// Reference semantics (torchtitanturbo/models/common/npu_gmm.py):
//   :17-18, :31, :38  torch._grouped_mm(x, w.transpose(-2, -1), offs)
//   :32-36            optional clamp with swiglu_limit
//   :37               npu_swiglu: silu(gate) * up, gate = first H columns
#include <type_traits>

#include "common.h"
#include "gemm_common.h"
#include "kernels.h"

namespace ttamd {
namespace {

constexpr int FQ = 128;
constexpr int FP = 256;
constexpr int FK = 64;
constexpr int FSTAGES = 3;
constexpr int FTHREADS = 256;
constexpr int F_P_BYTES = FP * FK * 2;                    // 32 KB
constexpr int F_Q_BYTES = FQ * FK * 2;                    // 16 KB
constexpr int F_STAGE_BYTES = F_P_BYTES + F_Q_BYTES;      // 48 KB
constexpr int F_LDS_BYTES = FSTAGES * F_STAGE_BYTES;      // 144 KB
constexpr int F_LOADS = (F_STAGE_BYTES / 16) / FTHREADS;  // 12 DMA / lane / stage

typedef __attribute__((address_space(3))) char* lds_ptr_t;
typedef int i32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t lds_addr(const char* p) {
  return (uint32_t)(uintptr_t)(lds_ptr_t)p;
}

// ---------------------------------------------------------------------------
// Memory operations the compiler must not track or move.
//
// The LDS DMA loads, the stage barrier and the tile-table loads are inline
// asm: the compiler neither tracks the DMA (it would wait for every DMA in
// flight before each LDS read) nor moves memory operations across them
// ("memory" clobber).  The kernel counts its own vector-memory operations
// and waits with explicit vmcnt values.  Vector memory operations of a wave
// complete in issue order, so "at most N in flight" means "all but the N
// most recent have completed".
// ---------------------------------------------------------------------------

// A wave-uniform 64-bit value in SGPRs.
__device__ __forceinline__ uint64_t uniform64(uint64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}

// Hazards the compiler cannot see through inline asm (GFX9 family manual
// wait states): a VMEM instruction that reads an SGPR written by a VALU
// instruction (v_readfirstlane) needs 5 wait states, and an LDS DMA that
// reads M0 written by a SALU instruction needs 1.  The compiler computes the
// SGPR base and M0 right before each asm statement, so every asm statement
// that reads SGPR operands starts with s_nop 4 (5 wait states).

// 16 bytes per lane from sbase + voff to LDS [lds + 16 * lane].
__device__ __forceinline__ void dma16(uint32_t voff, uint64_t sbase, uint32_t lds) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(uniform64(sbase)),
               "{m0}"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}

// At most N vector-memory operations of this wave in flight, its LDS reads
// complete, then a workgroup barrier.
template <int N>
__device__ __forceinline__ void wait_vm_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// Wave-uniform loads through the scalar cache (read only).
__device__ __forceinline__ int4 sload_int4(const int4* p) {
  i32x4_t v;
  asm volatile("s_nop 4\n\ts_load_dwordx4 %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)"
               : "=s"(v)
               : "s"(uniform64((uint64_t)p))
               : "memory");
  return make_int4(__builtin_amdgcn_readfirstlane(v[0]), __builtin_amdgcn_readfirstlane(v[1]),
                   __builtin_amdgcn_readfirstlane(v[2]), __builtin_amdgcn_readfirstlane(v[3]));
}

__device__ __forceinline__ int sload_int(const int* p) {
  int v;
  asm volatile("s_nop 4\n\ts_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)"
               : "=s"(v)
               : "s"(uniform64((uint64_t)p))
               : "memory");
  return __builtin_amdgcn_readfirstlane(v);
}

struct FwdArgs {
  const bf16_t* q;  // activations [M][kred]
  int64_t ldq;
  const bf16_t* p;  // weights, expert e at p + e * p_estride, rows of ldp
  int64_t p_estride;
  int64_t ldp;
  int kred;
  int n_p;       // valid weight rows (SWIGLU: H, the gate half)
  int np_tiles;  // weight-row tiles per Q tile
  const int4* table;
  const int* n_qtiles;
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

// MFMA fragments of one 64-deep stage: per k16 step, 2 weight fragments and
// 4 token fragments (8 bf16 each).
struct Frags {
  bf16x8_t p[4][2];
  bf16x8_t q[4][4];
};

__device__ __forceinline__ void read_frags(Frags& f, const bf16_t* p0, const bf16_t* p1,
                                           const bf16_t* q, int half, int fs) {
#pragma unroll
  for (int kk = 0; kk < FK / 16; ++kk) {
    const int pc = ((kk * 2 + half) ^ fs) * 8;
    f.p[kk][0] = *(const bf16x8_t*)(p0 + pc);
    f.p[kk][1] = *(const bf16x8_t*)(p1 + pc);
#pragma unroll
    for (int j = 0; j < 4; ++j) f.q[kk][j] = *(const bf16x8_t*)(q + j * 32 * FK + pc);
  }
}

// MFMAs of one stage from `cur`, interleaved with the LDS reads of the next
// stage into `nxt`.
template <int NQB>
__device__ __forceinline__ void mfma_stage(const Frags& cur, Frags& nxt, const bf16_t* p0,
                                           const bf16_t* p1, const bf16_t* q, int half, int fs,
                                           floatx16_t (&acc)[2][NQB]) {
#pragma unroll
  for (int kk = 0; kk < FK / 16; ++kk) {
    const int pc = ((kk * 2 + half) ^ fs) * 8;
#pragma unroll
    for (int j = 0; j < NQB; ++j) {
      acc[0][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cur.p[kk][0], cur.q[kk][j], acc[0][j], 0, 0, 0);
      acc[1][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cur.p[kk][1], cur.q[kk][j], acc[1][j], 0, 0, 0);
    }
    nxt.p[kk][0] = *(const bf16x8_t*)(p0 + pc);
    nxt.p[kk][1] = *(const bf16x8_t*)(p1 + pc);
#pragma unroll
    for (int j = 0; j < 4; ++j) nxt.q[kk][j] = *(const bf16x8_t*)(q + j * 32 * FK + pc);
    // Alternate MFMA and LDS read so the reads hide under the matrix pipe.
#pragma unroll
    for (int t = 0; t < 6; ++t) {
      if (t < 2 * NQB) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    if (2 * NQB > 6) __builtin_amdgcn_sched_group_barrier(0x008, 2 * NQB - 6, 0);
  }
}

template <int EPI>
__global__ __launch_bounds__(FTHREADS, 1) void gg_fwd_kernel(const FwdArgs a) {
  extern __shared__ __attribute__((aligned(1024))) char smem[];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = threadIdx.x & 63;
  const int G = gridDim.x;
  const int b = blockIdx.x;
  // XCD-aware slot: hardware block ids go round-robin over the 8 XCDs; give
  // XCD x the slots [x*G/8, (x+1)*G/8) so that it takes consecutive tiles.
  const int slot = (b & 7) * (G >> 3) + (b >> 3);
  const int ntiles = sload_int(a.n_qtiles) * a.np_tiles;
  const int nmy = slot < ntiles ? (ntiles - slot + G - 1) / G : 0;
  const int ksteps = a.kred / FK;
  const int total = nmy * ksteps;
  if (total == 0) return;

  const uint32_t lds0 = lds_addr(smem);
  const int lrow = l >> 3;
  // chunk permutation of the rows this lane's DMAs write: row (4i + w) * 8 +
  // lrow has (row >> 1) & 7 = (4w + lrow / 2) & 7 for every i.
  const int dchunk = (l & 7) ^ ((4 * w + (lrow >> 1)) & 7);

  // ---- DMA stream -----------------------------------------------------------
  int d_r = -1;  // tile round whose addresses are loaded
  uint64_t d_pbase = 0, d_qbase = 0;
  uint32_t d_voff[F_LOADS];
  auto dma_tile = [&](int r) {
    const int tile = r * G + slot;
    const int qt = tile / a.np_tiles;
    const int pt = tile - qt * a.np_tiles;
    const int4 ti = sload_int4(a.table + qt);
    const int64_t ldp2 = a.ldp * 2;
    if constexpr (EPI == EPI_SWIGLU) {
      d_pbase = uniform64((uint64_t)(a.p + (int64_t)ti.x * a.p_estride + (int64_t)pt * 128 * a.ldp));
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int rr = (i * 4 + w) * 8 + lrow;  // 0..255: gate rows then up rows
        const int col = min(pt * 128 + (rr & 127), a.n_p - 1) - pt * 128;
        const int prow = (rr < 128) ? col : (int)a.hidden + col;
        d_voff[i] = (uint32_t)(prow * ldp2 + dchunk * 16);
      }
    } else {
      d_pbase = uniform64((uint64_t)(a.p + (int64_t)ti.x * a.p_estride + (int64_t)pt * FP * a.ldp));
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int rr = (i * 4 + w) * 8 + lrow;
        const int prow = min(pt * FP + rr, a.n_p - 1) - pt * FP;
        d_voff[i] = (uint32_t)(prow * ldp2 + dchunk * 16);
      }
    }
    d_qbase = uniform64((uint64_t)(a.q + (int64_t)ti.y * a.ldq));
    const int qmax = ti.z - ti.y - 1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int rr = (i * 4 + w) * 8 + lrow;  // 0..127
      d_voff[8 + i] = (uint32_t)(min(rr, qmax) * a.ldq * 2 + dchunk * 16);
    }
    d_r = r;
  };
  auto issue = [&](int s) {
    const int r = s / ksteps;
    const int ks = s - r * ksteps;
    if (r != d_r) dma_tile(r);
    const uint64_t pb = d_pbase + (uint64_t)ks * (FK * 2);
    const uint64_t qb = d_qbase + (uint64_t)ks * (FK * 2);
    const uint32_t st = lds0 + (uint32_t)((s % FSTAGES) * F_STAGE_BYTES) + w * 1024;
#pragma unroll
    for (int i = 0; i < 8; ++i) dma16(d_voff[i], pb, st + i * 4096);
#pragma unroll
    for (int i = 0; i < 4; ++i) dma16(d_voff[8 + i], qb, st + F_P_BYTES + i * 4096);
  };

  // ---- fragment geometry -----------------------------------------------------
  // P blocks of this wave: SWIGLU pairs the gate block (rows 32w..) with the
  // up block (rows 128 + 32w..); otherwise rows 64w.. and 64w + 32...
  const int prow0 = (EPI == EPI_SWIGLU) ? 32 * w : 64 * w;
  const int prow1 = (EPI == EPI_SWIGLU) ? 128 + 32 * w : 64 * w + 32;
  const int r32 = l & 31;
  const int half = l >> 5;
  const int fs = (r32 >> 1) & 7;  // chunk permutation of rows 32j + r32
  const int pa0 = (prow0 + r32) * FK;
  const int pa1 = (prow1 + r32) * FK;
  const int qa = F_P_BYTES / 2 + r32 * FK;  // in bf16 elements from the stage base
  auto stage_ptr = [&](int s) { return (const bf16_t*)(smem + (s % FSTAGES) * F_STAGE_BYTES); };

  // ---- prologue: stages 0..2 in flight, fragments of stage 0 in registers ----
#pragma unroll
  for (int s0 = 0; s0 < FSTAGES; ++s0)
    if (s0 < total) issue(s0);
  if (total >= 3)
    wait_vm_barrier<2 * F_LOADS>();
  else if (total == 2)
    wait_vm_barrier<F_LOADS>();
  else
    wait_vm_barrier<0>();
  Frags fr[2];
  {
    const bf16_t* st = stage_ptr(0);
    read_frags(fr[0], st + pa0, st + pa1, st + qa, half, fs);
  }

  int s = 0;
  // One tile: ksteps stages, then the epilogue.  NQB = 32-row token blocks
  // holding rows of the expert; the accumulators live only inside this
  // specialisation, so they stay in AGPRs without copies.
  auto run_tile = [&](auto nqb_tag, int row0, int row1, int pt) {
    constexpr int NQB = decltype(nqb_tag)::value;
    floatx16_t acc[2][NQB];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < NQB; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

    // One stage: compute from `cur`, read the next stage into `nxt`.
    auto stage = [&](const Frags& cur, Frags& nxt) {
      // Stage s + 1 has landed once only the DMAs of stage s + 2 may still be
      // in flight; all LDS reads of stage s are complete (lgkmcnt), so its
      // buffer takes the DMAs of stage s + 3.
      if (s + 2 < total)
        wait_vm_barrier<F_LOADS>();
      else
        wait_vm_barrier<0>();
      if (s + FSTAGES < total) issue(s + FSTAGES);
      // Next stage's fragments (a valid stage buffer even past the end).
      const bf16_t* nst = stage_ptr(s + 1);
      mfma_stage<NQB>(cur, nxt, nst + pa0, nst + pa1, nst + qa, half, fs, acc);
      ++s;
    };
    // Stages alternate between the two fragment sets; a tile always starts
    // with its fragments in fr[0].
    int ks = 0;
    for (; ks + 1 < ksteps; ks += 2) {
      stage(fr[0], fr[1]);
      stage(fr[1], fr[0]);
    }
    if (ks < ksteps) {
      stage(fr[0], fr[1]);
      fr[0] = fr[1];
    }

    // ---- epilogue: acc[pb][j][4g + i] is (Q row 32j + r32,
    //      P row prow_pb + 8g + 4 * half + i) ---------------------------------
#pragma unroll
    for (int j = 0; j < NQB; ++j) {
      const int gq = row0 + 32 * j + r32;
      if (gq >= row1) continue;
      if constexpr (EPI == EPI_SWIGLU) {
        const bool clamp = (a.limit == a.limit);
        const float L = a.limit;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int col = pt * 128 + 32 * w + 8 * g + 4 * half;
          if (col >= a.n_p) continue;
          float av[4], gv[4], uv[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            // h is materialised in bf16 by the reference; SwiGLU reads it.
            gv[i] = round_bf16(acc[0][j][4 * g + i]);
            uv[i] = round_bf16(acc[1][j][4 * g + i]);
            float gc = gv[i], uc = uv[i];
            if (clamp) {
              gc = fminf(gc, L);
              uc = fminf(fmaxf(uc, -L), L);
            }
            av[i] = silu_f(gc) * uc;
          }
          bf16_t* orow = a.out + (int64_t)gq * a.ldo + col;
          *(uint2*)orow = make_uint2(pack_bf16x2(av[0], av[1]), pack_bf16x2(av[2], av[3]));
          if (a.h_out) {
            bf16_t* hrow = a.h_out + (int64_t)gq * a.ldh + col;
            *(uint2*)hrow = make_uint2(pack_bf16x2(gv[0], gv[1]), pack_bf16x2(gv[2], gv[3]));
            *(uint2*)(hrow + a.hidden) =
                make_uint2(pack_bf16x2(uv[0], uv[1]), pack_bf16x2(uv[2], uv[3]));
          }
        }
      } else {
        int64_t orow_idx = gq;
        float sc = 1.f;
        if constexpr (EPI == EPI_SCATTER) {
          if (a.dest) orow_idx = min(max(a.dest[gq], 0), a.n_dest - 1);
          if (a.row_scale) sc = a.row_scale[gq];
        }
        bf16_t* orow = a.out + orow_idx * a.ldo;
#pragma unroll
        for (int pb = 0; pb < 2; ++pb) {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int col = pt * FP + (pb ? prow1 : prow0) + 8 * g + 4 * half;
            if (col >= a.n_p) continue;
            const floatx16_t& v = acc[pb][j];
            *(uint2*)(orow + col) = make_uint2(pack_bf16x2(v[4 * g] * sc, v[4 * g + 1] * sc),
                                               pack_bf16x2(v[4 * g + 2] * sc, v[4 * g + 3] * sc));
          }
        }
      }
    }
  };

  for (int r = 0; r < nmy; ++r) {
    const int tile = r * G + slot;
    const int qt = tile / a.np_tiles;
    const int pt = tile - qt * a.np_tiles;
    const int4 ti = sload_int4(a.table + qt);
    const int nqb = (ti.z - ti.y + 31) >> 5;
    if (nqb >= 4)
      run_tile(std::integral_constant<int, 4>{}, ti.y, ti.z, pt);
    else if (nqb == 3)
      run_tile(std::integral_constant<int, 3>{}, ti.y, ti.z, pt);
    else if (nqb == 2)
      run_tile(std::integral_constant<int, 2>{}, ti.y, ti.z, pt);
    else
      run_tile(std::integral_constant<int, 1>{}, ti.y, ti.z, pt);
  }
}

int g_num_cus = 0;

int num_cus() {
  if (g_num_cus == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    g_num_cus = n;
  }
  return g_num_cus;
}

template <int EPI>
hipError_t launch_fwd(FwdArgs a, hipStream_t stream) {
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t err = hipFuncSetAttribute((const void*)gg_fwd_kernel<EPI>,
                                         hipFuncAttributeMaxDynamicSharedMemorySize, F_LDS_BYTES);
    if (err != hipSuccess) return err;
    attr_set = true;
  }
  const int grid = (num_cus() + 7) & ~7;
  hipLaunchKernelGGL(gg_fwd_kernel<EPI>, dim3(grid), dim3(FTHREADS), F_LDS_BYTES, stream, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_fwd_gemm(int epi, const FwdGemm& g, hipStream_t stream) {
  FwdArgs a = {};
  a.q = (const bf16_t*)g.act;
  a.ldq = g.kred;
  a.p = (const bf16_t*)g.w;
  a.kred = g.kred;
  a.ldp = g.kred;
  a.table = g.table;
  a.n_qtiles = g.n_qtiles;
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
    return launch_fwd<EPI_SWIGLU>(a, stream);
  }
  a.p_estride = (int64_t)g.n * g.kred;
  a.n_p = g.n;
  a.np_tiles = (g.n + FP - 1) / FP;
  a.ldo = g.n;
  a.row_scale = g.row_scale;
  a.dest = g.dest;
  a.n_dest = g.n_dest;
  if (epi == EPI_SCATTER) return launch_fwd<EPI_SCATTER>(a, stream);
  return launch_fwd<EPI_STORE>(a, stream);
}

}  // namespace ttamd
