// Fused MoE router on MI355X (gfx950): gate GEMM + score + top-k + renorm in
// one kernel, so the router logits never round-trip through HBM.
//
//   logits[t, e] = bf16(sum_d x[t, d] * w[e, d])      F.linear in bf16
//   s[t, e]      = softmax_e(logits[t]) in fp32       or sigmoid(logits)
//   pick the top_k of s (+ expert_bias, for the selection only), descending,
//   ties to the lower expert id; optional renormalisation by the picked sum
//   (+ eps); times route_scale.
//
// Reference: UPSTREAM TorchTitan TokenChoiceTopKRouter (gate nn.Linear, fp32
// score, topk, renorm); in-reference closed form
// torchtitanturbo/models/qwen3_5/model.py:752-766 (F.linear :757, softmax in
// fp32 :758, topk :759-761, renorm :762-764).
//
// Layout: one workgroup (4 waves) per 32 tokens.  k runs in stages of 64:
// each stage holds the 32 token rows and the (32 * EB) expert rows as whole
// 128-byte lines in LDS, filled by global_load_lds_dwordx4 (NST buffers,
// NST - 1 stages in flight: the stream is latency-bound, so the pipeline
// fills the LDS).  Wave w owns expert blocks w, w + 4, ... and runs
// v_mfma_f32_32x32x16_bf16 with the expert block as A and the tokens as B,
// so lane l ends with 16 logits of token l % 32.  The logits go through LDS
// to the top-k, where 16 lanes own one token (4 tokens per wave at a time).
#include "common.h"
#include "dma_asm.h"
#include "kernels.h"

namespace ttamd {
namespace {

using namespace dma;

constexpr int RT = 32;      // tokens per workgroup
constexpr int RWAVES = 4;
constexpr int RTHREADS = 64 * RWAVES;
constexpr int RTK = 64;     // k per stage: 128-byte rows

// Stage buffers: as many as fit next to the logits block (at most 8), so
// that up to 7 stages stream in at once.
template <int EB>
constexpr int router_nst() {
  constexpr int stage = (RT + 32 * EB) * 128;
  constexpr int lg = RT * (32 * EB + 1) * 4;
  constexpr int n = (160 * 1024 - lg) / stage;
  return n > 8 ? 8 : n;
}

struct RouterArgs {
  const bf16_t* x;     // [T, D]
  const bf16_t* w;     // [E, D]
  const float* bias;   // [E] or null
  int T, E, D, K;
  int score_func;      // 0 softmax, 1 sigmoid
  int renorm;
  float eps, route_scale;
  float* scores;       // [T, K]
  int64_t* idx;        // [T, K]
  bf16_t* logits;      // [T, E] or null
};

template <int EB>
__global__ __launch_bounds__(RTHREADS) void router_fused_kernel(const RouterArgs a) {
  constexpr int EP = 32 * EB;       // experts padded to whole MFMA blocks
  constexpr int ROWS = RT + EP;     // stage rows: tokens, then experts
  constexpr int STAGE = ROWS * 128;
  constexpr int DPW = ROWS / 8 / RWAVES;  // DMA instructions per wave per stage (= 1 + EB)
  constexpr int PL = EP / 16;       // top-k values per lane
  constexpr int LGS = EP + 1;       // logits row stride in LDS (floats)
  constexpr int NST = router_nst<EB>();
  static_assert(ROWS % (8 * RWAVES) == 0, "stage rows");
  static_assert(NST >= 3 && (NST - 2) * DPW < 64, "pipeline depth");
  extern __shared__ __attribute__((aligned(1024))) char smem[];
  float* lg = (float*)(smem + NST * STAGE);

  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = threadIdx.x & 63;
  const int t0 = blockIdx.x * RT;
  const int nst = a.D / RTK;
  const uint32_t lds0 = lds_addr(smem);
  const int64_t ld2 = (int64_t)a.D * 2;

  // DMA geometry: instruction i of wave w moves row block rb = 4 i + w (rows
  // 8 rb .. 8 rb + 7); instruction 0 carries token rows, the rest expert rows.
  // LDS row r holds its logical 16-byte chunk c at physical chunk c ^ cswz(r).
  uint32_t voff[DPW];
#pragma unroll
  for (int i = 0; i < DPW; ++i) {
    const int rb = RWAVES * i + w;
    const int row = 8 * rb + (l >> 3);
    const int lchunk = (l & 7) ^ cswz(row);
    const int src = (i == 0) ? min(row, a.T - 1 - t0) : min(row - RT, a.E - 1);
    voff[i] = (uint32_t)(src * ld2 + lchunk * 16);
  }
  const uint64_t xbase = (uint64_t)(a.x + (int64_t)t0 * a.D);
  const uint64_t wbase = (uint64_t)a.w;
  auto issue = [&](int s) {
    const int sc = min(s, nst - 1);  // past the end: re-load the last stage
    const uint32_t st = lds0 + (uint32_t)((s % NST) * STAGE) + w * 1024;
    dma16(voff[0], xbase + (uint64_t)sc * 128, st);
#pragma unroll
    for (int i = 1; i < DPW; ++i) dma16(voff[i], wbase + (uint64_t)sc * 128, st + i * (RWAVES * 1024));
  };

  constexpr int NEB = (EB + RWAVES - 1) / RWAVES;  // expert blocks per wave
  floatx16_t acc[NEB];
#pragma unroll
  for (int b = 0; b < NEB; ++b)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[b][v] = 0.f;

  const int r32 = l & 31;
  const int half = l >> 5;
#pragma unroll
  for (int s = 0; s < NST - 1; ++s) issue(s);
  for (int s = 0; s < nst; ++s) {
    wait_vm_barrier<(NST - 2) * DPW>();  // stage s landed; every wave is done with stage s - 1
    issue(s + NST - 1);                  // into the buffer stage s - 1 used
    const char* st = smem + (s % NST) * STAGE;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int c = 2 * kk + half;
      const bf16x8_t bx = *(const bf16x8_t*)(st + r32 * 128 + ((c ^ cswz(r32)) << 4));
#pragma unroll
      for (int b = 0; b < NEB; ++b) {
        const int eb = w + RWAVES * b;
        if (eb < EB) {
          const int row = RT + 32 * eb + r32;
          const bf16x8_t aw = *(const bf16x8_t*)(st + row * 128 + ((c ^ cswz(row)) << 4));
          acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(aw, bx, acc[b], 0, 0, 0);
        }
      }
    }
  }
  wait_vm<0>();

  // ---- logits: lane l holds token r32, experts 32 eb + 8 g + 4 half + v ------
  const int tok = t0 + r32;
#pragma unroll
  for (int b = 0; b < NEB; ++b) {
    const int eb = w + RWAVES * b;
    if (eb < EB) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int e0 = 32 * eb + 8 * g + 4 * half;
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          v[i] = round_bf16(acc[b][4 * g + i]);
          lg[r32 * LGS + e0 + i] = v[i];
        }
        if (a.logits && tok < a.T && e0 < a.E) {
          // E % 4 == 0: the 4 experts are valid together
          *(uint2*)(a.logits + (int64_t)tok * a.E + e0) =
              make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
        }
      }
    }
  }
  __syncthreads();

  // ---- top-k: 16 lanes per token, lane i holds experts i + 16 m -------------
  const int gi = l & 15;
#pragma unroll 1
  for (int pass = 0; pass < RT / (RWAVES * 4); ++pass) {
    const int j = pass * (RWAVES * 4) + w * 4 + (l >> 4);  // token of this lane group
    const int t = t0 + j;
    float sc[PL], sel[PL];
    float mx = -INFINITY;
#pragma unroll
    for (int m = 0; m < PL; ++m) {
      const int e = gi + 16 * m;
      sc[m] = (e < a.E) ? lg[j * LGS + e] : -INFINITY;
      mx = fmaxf(mx, sc[m]);
    }
    if (a.score_func == 0) {
#pragma unroll
      for (int off = 8; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 16));
      float sum = 0.f;
#pragma unroll
      for (int m = 0; m < PL; ++m) {
        const int e = gi + 16 * m;
        sc[m] = (e < a.E) ? expf(sc[m] - mx) : 0.f;
        sum += sc[m];
      }
#pragma unroll
      for (int off = 8; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 16);
#pragma unroll
      for (int m = 0; m < PL; ++m) sc[m] = sc[m] / sum;
    } else {
#pragma unroll
      for (int m = 0; m < PL; ++m) sc[m] = 1.f / (1.f + expf(-sc[m]));
    }
#pragma unroll
    for (int m = 0; m < PL; ++m) {
      const int e = gi + 16 * m;
      sel[m] = (e < a.E) ? (a.bias ? sc[m] + a.bias[e] : sc[m]) : -INFINITY;
    }
    float picked = 0.f, my_v = 0.f;
    int my_i = 0;
    for (int k = 0; k < a.K; ++k) {
      float bv = -INFINITY;
      int bi = 0x7fffffff;
#pragma unroll
      for (int m = 0; m < PL; ++m) {
        const int e = gi + 16 * m;
        if (e < a.E && (sel[m] > bv || (sel[m] == bv && e < bi))) {
          bv = sel[m];
          bi = e;
        }
      }
#pragma unroll
      for (int off = 8; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off, 16);
        const int oi = __shfl_xor(bi, off, 16);
        if (ov > bv || (ov == bv && oi < bi)) {
          bv = ov;
          bi = oi;
        }
      }
      bi = min(max(bi, 0), a.E - 1);  // K <= E keeps a valid pick; stay in range regardless
      const int owner = bi & 15;
      const int slot = bi >> 4;
      float v = 0.f;
#pragma unroll
      for (int m = 0; m < PL; ++m)
        if (m == slot) v = sc[m];
      v = __shfl(v, owner, 16);
#pragma unroll
      for (int m = 0; m < PL; ++m)
        if (m == slot && gi == owner) sel[m] = -INFINITY;
      picked += v;
      if (gi == k) {
        my_v = v;
        my_i = bi;
      }
    }
    if (gi < a.K && t < a.T) {
      float v = my_v;
      if (a.renorm) v = v / (picked + a.eps);
      a.scores[(int64_t)t * a.K + gi] = v * a.route_scale;
      a.idx[(int64_t)t * a.K + gi] = my_i;
    }
  }
}

template <int EB>
hipError_t launch_eb(const RouterArgs& a, hipStream_t stream) {
  constexpr int EP = 32 * EB;
  constexpr int lds = router_nst<EB>() * (RT + EP) * 128 + RT * (EP + 1) * 4;
  static_assert(lds <= 160 * 1024, "router LDS");
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t err = hipFuncSetAttribute((const void*)router_fused_kernel<EB>,
                                         hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (err != hipSuccess) return err;
    attr_set = true;
  }
  const int grid = (a.T + RT - 1) / RT;
  hipLaunchKernelGGL(router_fused_kernel<EB>, dim3(grid), dim3(RTHREADS), lds, stream, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_router_fused(const void* x, const void* w, const float* bias, int T, int E, int D, int K,
                               int score_func, int renorm, float renorm_eps, float route_scale,
                               float* top_scores, int64_t* top_idx, void* logits, hipStream_t stream) {
  if (T == 0) return hipSuccess;
  RouterArgs a;
  a.x = (const bf16_t*)x;
  a.w = (const bf16_t*)w;
  a.bias = bias;
  a.T = T;
  a.E = E;
  a.D = D;
  a.K = K;
  a.score_func = score_func;
  a.renorm = renorm;
  a.eps = renorm_eps;
  a.route_scale = route_scale;
  a.scores = top_scores;
  a.idx = top_idx;
  a.logits = (bf16_t*)logits;
  if (E <= 32) return launch_eb<1>(a, stream);
  if (E <= 64) return launch_eb<2>(a, stream);
  if (E <= 128) return launch_eb<4>(a, stream);
  return launch_eb<8>(a, stream);
}

}  // namespace ttamd
