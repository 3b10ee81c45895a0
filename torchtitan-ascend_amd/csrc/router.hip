// MoE router on MI355X (gfx950): gate GEMM + score + top-k + renorm.
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
// Two kernels.  The gate GEMM is memory-bound and every CU can only pull its
// operands at the rate its in-flight line requests allow, so what matters
// is the bytes each CU moves.  Giving each workgroup all experts for a few
// tokens would make every CU stream the whole router weight; instead
//   * router_gemm_kernel<EB>: a workgroup (4 waves) takes 128 tokens and one
//     slice of D, streams those token rows and the slice of every expert
//     row through LDS (whole 128-byte lines, global_load_lds_dwordx4, NST
//     stage buffers) into v_mfma_f32_32x32x16_bf16 (wave w: token block w,
//     all expert blocks), and writes fp32 partial logits [S][T][E];
//   * router_topk_partials_kernel: sums the S partial logits of a token in a
//     fixed order, rounds to bf16 (the Linear's output dtype) and runs the
//     score + top-k with 16 lanes per token (4 tokens per wave).
// The split count S is chosen so that the first kernel has about one
// workgroup per CU.
#include <type_traits>

#include "common.h"
#include "dma_asm.h"
#include "gemm_common.h"
#include "kernels.h"

namespace ttamd {
namespace {

using namespace dma;

constexpr int RT = 128;     // tokens per workgroup of the gate GEMM
constexpr int RWAVES = 4;   // one 32-token block per wave
constexpr int RTHREADS = 64 * RWAVES;
constexpr int RTK = 64;     // k per stage: 128-byte rows
constexpr int kRouterMaxE = 256;
constexpr int kRouterMaxSplits = 4;  // slices of D (partial logits per token and expert)

// Stage buffers of the gate GEMM: as many as fit (at most 6).
template <int EB>
constexpr int router_nst() {
  constexpr int stage = (RT + 32 * EB) * 128;
  constexpr int n = (160 * 1024) / stage;
  return n > 6 ? 6 : n;
}

struct RouterGemmArgs {
  const bf16_t* x;  // [T, D]
  const bf16_t* w;  // [E, D]
  int T, E, D;
  int kstages;      // 64-wide k stages per split
  float* part;      // [S][T][E] fp32
  int* zero;        // nullable: ints cleared for the top-k kernel's histogram
  int nzero;
};

template <int EB>
__global__ __launch_bounds__(RTHREADS) void router_gemm_kernel(const RouterGemmArgs a) {
  constexpr int EP = 32 * EB;
  constexpr int ROWS = RT + EP;            // stage rows: tokens, then experts
  constexpr int STAGE = ROWS * 128;
  constexpr int DPW = ROWS / 8 / RWAVES;   // DMA instructions per wave per stage
  constexpr int TPW = RT / 8 / RWAVES;     // of which token rows (= 4)
  constexpr int NST = router_nst<EB>();
  static_assert(ROWS % (8 * RWAVES) == 0 && NST >= 3 && (NST - 2) * DPW < 64, "router geometry");
  extern __shared__ __attribute__((aligned(1024))) char smem[];

  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = threadIdx.x & 63;
  const int t0 = blockIdx.x * RT;
  const int split = blockIdx.y;
  const int k0 = split * a.kstages;                    // first stage of this slice
  const int nst = min(a.kstages, a.D / RTK - k0);      // stages of this slice
  const uint32_t lds0 = lds_addr(smem);
  const int64_t ld2 = (int64_t)a.D * 2;
  if (a.zero) {  // the route histogram the top-k kernel accumulates into
    const int nb = gridDim.x * gridDim.y;
    for (int i = (blockIdx.y * gridDim.x + blockIdx.x) * RTHREADS + threadIdx.x; i < a.nzero; i += nb * RTHREADS)
      a.zero[i] = 0;
  }

  // Instruction i of wave w moves row block rb = 4 i + w (rows 8 rb ..
  // 8 rb + 7): instructions 0..TPW-1 carry token rows, the rest expert rows.
  // LDS row r holds its logical 16-byte chunk c at physical chunk c ^ cswz(r).
  uint32_t voff[DPW];
#pragma unroll
  for (int i = 0; i < DPW; ++i) {
    const int rb = RWAVES * i + w;
    const int row = 8 * rb + (l >> 3);
    const int lchunk = (l & 7) ^ cswz(row);
    const int src = (i < TPW) ? min(row, a.T - 1 - t0) : min(row - RT, a.E - 1);
    voff[i] = (uint32_t)(src * ld2 + lchunk * 16);
  }
  const uint64_t xbase = (uint64_t)(a.x + (int64_t)t0 * a.D + (int64_t)k0 * RTK);
  const uint64_t wbase = (uint64_t)(a.w + (int64_t)k0 * RTK);
  auto issue = [&](int s) {
    const int sc = min(s, nst - 1);  // past the end: re-load the last stage
    const uint32_t st = lds0 + (uint32_t)((s % NST) * STAGE) + w * 1024;
#pragma unroll
    for (int i = 0; i < DPW; ++i)
      dma16(voff[i], (i < TPW ? xbase : wbase) + (uint64_t)sc * 128, st + i * (RWAVES * 1024));
  };

  floatx16_t acc[EB];
#pragma unroll
  for (int b = 0; b < EB; ++b)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[b][v] = 0.f;

  const int r32 = l & 31;
  const int half = l >> 5;
  const int trow = 32 * w + r32;  // this lane's token row in the stage
#pragma unroll
  for (int s = 0; s < NST - 1; ++s) issue(s);
  for (int s = 0; s < nst; ++s) {
    wait_vm_barrier<(NST - 2) * DPW>();  // stage s landed; every wave is done with stage s - 1
    issue(s + NST - 1);                  // into the buffer stage s - 1 used
    const char* st = smem + (s % NST) * STAGE;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int c = 2 * kk + half;
      const bf16x8_t bx = *(const bf16x8_t*)(st + trow * 128 + ((c ^ cswz(trow)) << 4));
#pragma unroll
      for (int b = 0; b < EB; ++b) {
        const int row = RT + 32 * b + r32;
        const bf16x8_t aw = *(const bf16x8_t*)(st + row * 128 + ((c ^ cswz(row)) << 4));
        acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(aw, bx, acc[b], 0, 0, 0);
      }
    }
  }
  wait_vm<0>();

  // lane l holds token t0 + trow, experts 32 b + 8 g + 4 half + v
  const int tok = t0 + trow;
  if (tok < a.T) {
    float* prow = a.part + ((int64_t)split * a.T + tok) * a.E;
#pragma unroll
    for (int b = 0; b < EB; ++b)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int e0 = 32 * b + 8 * g + 4 * half;
        if ((a.E & 3) == 0 && e0 + 3 < a.E) {
          *(floatx4_t*)(prow + e0) = floatx4_t{acc[b][4 * g], acc[b][4 * g + 1], acc[b][4 * g + 2], acc[b][4 * g + 3]};
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (e0 + i < a.E) prow[e0 + i] = acc[b][4 * g + i];
        }
      }
  }
}

struct RouterTopkArgs {
  const float* part;  // [S][T][E]
  int S, T, E, K;
  const float* bias;  // [E] or null
  int score_func;     // 0 softmax, 1 sigmoid
  int renorm;
  float eps, route_scale;
  float* scores;      // [T, K]
  int64_t* idx;       // [T, K]
  bf16_t* logits;     // [T, E] or null
  // nullable: per-chunk expert histogram of the picks (route layout,
  // hist[e * nchunks + (t * K + k) / chunk]), accumulated with atomics
  int* hist;
  int nchunks, chunk;
};

// sel_key (common.h) orders the selection values; a picked slot gets key 0.

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
  return (uint32_t)dpp_i<CTRL>((int)v);
}

// Unsigned max / min over the 16 lanes of a DPP row (every lane gets it).
__device__ __forceinline__ uint32_t row16_umax(uint32_t v) {
  v = max(v, dpp_u<kDppXor1>(v));
  v = max(v, dpp_u<kDppXor2>(v));
  v = max(v, dpp_u<kDppHalfMirror>(v));
  return max(v, dpp_u<kDppMirror>(v));
}
__device__ __forceinline__ uint32_t row16_umin(uint32_t v) {
  v = min(v, dpp_u<kDppXor1>(v));
  v = min(v, dpp_u<kDppXor2>(v));
  v = min(v, dpp_u<kDppHalfMirror>(v));
  return min(v, dpp_u<kDppMirror>(v));
}

// 16 lanes per token, 4 tokens per wave, 16 tokens per workgroup.  Lane i
// holds experts in runs of G = min(PL, 4) consecutive ids,
// e(m) = G i + m % G + 16 G (m / G), so each run of partials is one 4G-byte
// load (the 16 lanes of a token read 64 G contiguous bytes per run).  FULL:
// E == 16 PL, every slot holds an expert.
//
// Selection: each of the K rounds takes the largest key of the row (DPP
// max), then the lowest expert id holding it (DPP min) -- the (value desc,
// id asc) order of a stable top-k, -inf after every finite value and NaN
// last -- and clears that slot.  The picked
// scores reach their output lanes through LDS and are summed in pick order
// for the renormalisation.
template <int PL, bool FULL>
__global__ __launch_bounds__(256) void router_topk_partials_kernel(const RouterTopkArgs a) {
  constexpr int G = PL < 4 ? PL : 4;
  __shared__ __attribute__((aligned(16))) float lsc[16][16 * PL];  // scores by expert id
  __shared__ float lpick[16][16];                                  // picked scores, pick order
  const int l = threadIdx.x & 63;
  const int gi = l & 15;
  const int tl = threadIdx.x >> 4;
  const int t = blockIdx.x * 16 + tl;
  const bool valid = t < a.T;
  const int tt = valid ? t : a.T - 1;
  const int E = FULL ? 16 * PL : a.E;
  auto eid = [&](int m) { return G * gi + m % G + 16 * G * (m / G); };
  auto live = [&](int m) { return FULL || eid(m) < E; };
  // every partial first (one batch of independent loads), then the sums in
  // split order
  float pv[kRouterMaxSplits][PL];
  const bool vec = FULL || (E % G) == 0;  // runs never straddle E and stay aligned
#pragma unroll
  for (int s = 0; s < kRouterMaxSplits; ++s)
#pragma unroll
    for (int m0 = 0; m0 < PL; m0 += G) {
      const int e0 = eid(m0);
      const float* src = a.part + ((int64_t)s * a.T + tt) * E + e0;
      if (s < a.S && vec && (FULL || e0 < E)) {
        if constexpr (G == 4) {
          const float4 v = *(const float4*)src;
          pv[s][m0] = v.x; pv[s][m0 + 1] = v.y; pv[s][m0 + 2] = v.z; pv[s][m0 + 3] = v.w;
        } else if constexpr (G == 2) {
          const float2 v = *(const float2*)src;
          pv[s][m0] = v.x; pv[s][m0 + 1] = v.y;
        } else {
          pv[s][m0] = src[0];
        }
      } else {
#pragma unroll
        for (int i = 0; i < G; ++i) pv[s][m0 + i] = (s < a.S && e0 + i < E) ? src[i] : 0.f;
      }
    }
  float sc[PL];
  float mx = -INFINITY;
#pragma unroll
  for (int m = 0; m < PL; ++m) {
    float z = -INFINITY;
    if (live(m)) {
      z = pv[0][m];
#pragma unroll
      for (int s = 1; s < kRouterMaxSplits; ++s)
        if (s < a.S) z += pv[s][m];
      z = round_bf16(z);
    }
    sc[m] = z;
    mx = fmaxf(mx, z);
  }
  if (a.logits && valid) {
    bf16_t* lrow = a.logits + (int64_t)t * E;
#pragma unroll
    for (int m0 = 0; m0 < PL; m0 += G) {
      const int e0 = eid(m0);
      if constexpr (FULL && G == 4) {
        *(u32x2_t*)(lrow + e0) = u32x2_t{pack_bf16x2(sc[m0], sc[m0 + 1]), pack_bf16x2(sc[m0 + 2], sc[m0 + 3])};
      } else if constexpr (FULL && G == 2) {
        *(uint32_t*)(lrow + e0) = pack_bf16x2(sc[m0], sc[m0 + 1]);
      } else {
#pragma unroll
        for (int i = 0; i < G; ++i)
          if (e0 + i < E) lrow[e0 + i] = (bf16_t)f32_to_bf16(sc[m0 + i]);
      }
    }
  }
  if (a.score_func == 0) {
    mx = row16_max(mx);
    float sum = 0.f;
#pragma unroll
    for (int m = 0; m < PL; ++m) {
      sc[m] = live(m) ? expf(sc[m] - mx) : 0.f;
      sum += sc[m];
    }
    sum = row16_sum(sum);
#pragma unroll
    for (int m = 0; m < PL; ++m) sc[m] = sc[m] / sum;
  } else {
#pragma unroll
    for (int m = 0; m < PL; ++m) sc[m] = 1.f / (1.f + expf(-sc[m]));
  }
  uint32_t key[PL];
#pragma unroll
  for (int m = 0; m < PL; ++m) key[m] = live(m) ? sel_key(a.bias ? sc[m] + a.bias[eid(m)] : sc[m]) : 0u;
  int my_i = 0;
  for (int k = 0; k < a.K; ++k) {
    uint32_t km = key[0];
#pragma unroll
    for (int m = 1; m < PL; ++m) km = max(km, key[m]);
    km = row16_umax(km);
    uint32_t cand = 0xffffffffu;
#pragma unroll
    for (int m = PL - 1; m >= 0; --m) cand = (key[m] == km) ? (uint32_t)eid(m) : cand;
    cand = row16_umin(cand);
    // every expert keeps a key >= 1 until picked and K <= E, so some slot
    // holds km; the clamp only keeps the index in range regardless
    const int win = (int)min(cand, (uint32_t)(E - 1));
#pragma unroll
    for (int m = 0; m < PL; ++m) key[m] = (eid(m) == win) ? 0u : key[m];
    if (gi == k) my_i = win;
  }
  const bool out = gi < a.K;
  if (a.hist) {
    // The workgroup's 16 K flat slots (K <= 16) span at most two chunks:
    // count them in LDS, then one atomic per nonzero (expert, chunk),
    // issued before the score exchange so that their round trips overlap it.
    __shared__ int lh[2 * kRouterMaxE];
    const int c0 = (int)(((int64_t)blockIdx.x * 16 * a.K) / a.chunk);
    for (int i = threadIdx.x; i < 2 * E; i += 256) lh[i] = 0;
    __syncthreads();
    if (out && valid) {
      const int c = (int)(((int64_t)t * a.K + gi) / a.chunk) - c0;  // 0 or 1
      atomicAdd(&lh[min(max(c, 0), 1) * E + my_i], 1);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < 2 * E; i += 256) {
      const int n = lh[i];
      const int c = c0 + i / E;
      if (n > 0 && c < a.nchunks) atomicAdd(&a.hist[(int64_t)(i % E) * a.nchunks + c], n);
    }
  }
  // scores of the picks: the owner lanes publish, the output lanes read
  float* srow = lsc[tl];
#pragma unroll
  for (int m0 = 0; m0 < PL; m0 += G) {
    const int e0 = eid(m0);
    if constexpr (FULL && G == 4) {
      *(float4*)(srow + e0) = make_float4(sc[m0], sc[m0 + 1], sc[m0 + 2], sc[m0 + 3]);
    } else {
#pragma unroll
      for (int i = 0; i < G; ++i)
        if (e0 + i < 16 * PL) srow[e0 + i] = sc[m0 + i];
    }
  }
  lds_wait();
  const float my_v = out ? srow[my_i] : 0.f;
  lpick[tl][gi] = my_v;
  lds_wait();
  float picked = 0.f;
  for (int k = 0; k < a.K; ++k) picked += lpick[tl][k];
  if (out && valid) {
    float v = my_v;
    if (a.renorm) v = v / (picked + a.eps);
    a.scores[(int64_t)t * a.K + gi] = v * a.route_scale;
    a.idx[(int64_t)t * a.K + gi] = my_i;
  }
}

// ---------------------------------------------------------------------------
// Router backward, elementwise part: d(top_scores) [T, K] -> d(logits) bf16.
// Autograd of the upstream router's op sequence (closed form
// models/qwen3_5/model.py:757-765): top_scores = route_scale * (s[idx] /
// (sum_k s[idx_k] + eps) if renorm else s[idx]), s = softmax / sigmoid of
// the bf16 logits in fp32; the gradient reaches the logits cast back to
// bf16 (the Linear's dtype).  Each step in the order torch's backward
// formulas take it:
//   g_k   = route_scale * grad_top[k]
//   renorm: gd = sum_k (-g_k * s_k / (S * S)); ds_k = g_k / S + gd
//   softmax: dz = (ds - sum_e ds_e s_e) * s;  sigmoid: dz = ds * (1 - s) * s
// s is recomputed from the logits with the forward kernel's arithmetic.
// 16 lanes per token (the forward's lane -> expert map); columns E..ldd-1
// of the output (padding for the GEMMs that follow) are zero.
struct RouterBwdArgs {
  const bf16_t* logits;  // [T, E]
  const int64_t* idx;    // [T, K]
  const float* grad;     // [T, K]
  int T, E, K;
  int score_func, renorm;
  float eps, route_scale;
  bf16_t* dlogits;  // [T, ldd]
  int ldd;
};

template <int PL>
__global__ __launch_bounds__(256) void router_backward_kernel(const RouterBwdArgs a) {
  constexpr int G = PL < 4 ? PL : 4;
  const int gi = threadIdx.x & 15;
  const int t = blockIdx.x * 16 + (threadIdx.x >> 4);
  const bool valid = t < a.T;
  const int tt = valid ? t : a.T - 1;
  auto eid = [&](int m) { return G * gi + m % G + 16 * G * (m / G); };
  float sc[PL];
  float mx = -INFINITY;
#pragma unroll
  for (int m = 0; m < PL; ++m) {
    const int e = eid(m);
    const float z = (e < a.E) ? bf16_to_f32(a.logits[(int64_t)tt * a.E + e]) : -INFINITY;
    sc[m] = z;
    mx = fmaxf(mx, z);
  }
  if (a.score_func == 0) {
    mx = row16_max(mx);
    float sum = 0.f;
#pragma unroll
    for (int m = 0; m < PL; ++m) {
      const int e = eid(m);
      sc[m] = (e < a.E) ? expf(sc[m] - mx) : 0.f;
      sum += sc[m];
    }
    sum = row16_sum(sum);
#pragma unroll
    for (int m = 0; m < PL; ++m) sc[m] = sc[m] / sum;
  } else {
#pragma unroll
    for (int m = 0; m < PL; ++m) sc[m] = 1.f / (1.f + expf(-sc[m]));
  }
  // picked experts, their scores (broadcast over the 16 lanes) and grads
  float ds[PL];
#pragma unroll
  for (int m = 0; m < PL; ++m) ds[m] = 0.f;
  float S = 0.f, gd = 0.f;
  if (a.renorm) {
    for (int k = 0; k < a.K; ++k) {
      const int ek = (int)a.idx[(int64_t)tt * a.K + k];
      float v = 0.f;
#pragma unroll
      for (int m = 0; m < PL; ++m)
        if (eid(m) == ek) v = sc[m];
      S += row16_sum(v);  // one lane holds s[ek]; picked in k order, as the forward sums them
    }
    S += a.eps;
    for (int k = 0; k < a.K; ++k) {
      const int ek = (int)a.idx[(int64_t)tt * a.K + k];
      const float g = a.grad[(int64_t)tt * a.K + k] * a.route_scale;
      float v = 0.f;
#pragma unroll
      for (int m = 0; m < PL; ++m)
        if (eid(m) == ek) v = sc[m];
      gd += -g * row16_sum(v) / (S * S);
    }
  }
  for (int k = 0; k < a.K; ++k) {
    const int ek = (int)a.idx[(int64_t)tt * a.K + k];
    const float g = a.grad[(int64_t)tt * a.K + k] * a.route_scale;
    const float d = a.renorm ? g / S + gd : g;
#pragma unroll
    for (int m = 0; m < PL; ++m)
      if (eid(m) == ek) ds[m] += d;
  }
  if (a.score_func == 0) {
    float dot = 0.f;
#pragma unroll
    for (int m = 0; m < PL; ++m) dot += ds[m] * sc[m];
    dot = row16_sum(dot);
#pragma unroll
    for (int m = 0; m < PL; ++m) ds[m] = (ds[m] - dot) * sc[m];
  } else {
#pragma unroll
    for (int m = 0; m < PL; ++m) ds[m] = ds[m] * (1.f - sc[m]) * sc[m];
  }
  if (!valid) return;
  bf16_t* row = a.dlogits + (int64_t)t * a.ldd;
#pragma unroll
  for (int m = 0; m < PL; ++m) {
    const int e = eid(m);
    if (e < a.E) row[e] = (bf16_t)f32_to_bf16(ds[m]);
  }
  for (int e = a.E + gi; e < a.ldd; e += 16) row[e] = 0;
}

// w_pad [ldd rows][D] = w_router rows, then zero rows; offs1[0] = T (one
// expert owning every token row, for the padded dgrad); offsg[g] = the end of
// token group g of G near-equal groups (the weight gradient's partial sums).
__global__ __launch_bounds__(256) void router_pad_kernel(const uint4* __restrict__ w, int E, int ldd, int cpr,
                                                         uint4* __restrict__ w_pad, int* offs1, int T, int* offsg,
                                                         int G) {
  const int total = ldd * cpr;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < total; i += gridDim.x * 256)
    w_pad[i] = (i / cpr < E) ? w[i] : make_uint4(0, 0, 0, 0);
  if (blockIdx.x == 0) {
    if (threadIdx.x == 0) offs1[0] = T;
    for (int g = threadIdx.x; g < G; g += 256) offsg[g] = (int)((int64_t)T * (g + 1) / G);
  }
}

// dw[e][d] (fp32 or bf16) = sum over the G token groups of part[g][e][d], in
// group order (deterministic).  part rows are n_part >= E wide.
__global__ __launch_bounds__(256) void router_dw_reduce_kernel(const float4* __restrict__ part, int G, int n_part,
                                                               int E, int D4, void* dst, int fp32) {
  const int n = E * D4;
  const int64_t gstride = (int64_t)n_part * D4;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) {
    float4 acc = part[i];
    for (int g = 1; g < G; ++g) {
      const float4 v = part[g * gstride + i];
      acc.x += v.x;
      acc.y += v.y;
      acc.z += v.z;
      acc.w += v.w;
    }
    if (fp32)
      ((float4*)dst)[i] = acc;
    else
      ((uint2*)dst)[i] = make_uint2(pack_bf16x2(acc.x, acc.y), pack_bf16x2(acc.z, acc.w));
  }
}

template <int EB>
hipError_t launch_gemm_eb(const RouterGemmArgs& a, int S, hipStream_t stream) {
  constexpr int lds = router_nst<EB>() * (RT + 32 * EB) * 128;
  static_assert(lds <= 160 * 1024, "router LDS");
  // set once per process (thread-safe static initialisation)
  static const hipError_t attr_err =
      hipFuncSetAttribute((const void*)router_gemm_kernel<EB>, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (attr_err != hipSuccess) return attr_err;
  return launch_k(false, router_gemm_kernel<EB>, dim3((a.T + RT - 1) / RT, S), dim3(RTHREADS), lds, stream, a);
}

// Slices of D: enough gate-GEMM workgroups to give every CU one (each CU
// then moves T*D*2/CUs bytes of x plus E*D*2/S of the weight), at most
// kRouterMaxSplits (the partial logits cost 8*S*T*E bytes of traffic), each
// slice at least 4 stages (256 columns) long.
int router_splits(int T, int D) {
  const int tiles = (T + RT - 1) / RT;
  const int stages = D / RTK;
  int S = (num_cus() + tiles - 1) / tiles;
  S = max(1, min(min(S, kRouterMaxSplits), stages / 4));
  const int per = (stages + S - 1) / S;
  return (stages + per - 1) / per;  // no empty slice
}

}  // namespace

size_t router_workspace_bytes(int64_t T, int E, int64_t D) {
  if (T <= 0) return 0;
  return (size_t)router_splits((int)T, (int)D) * (size_t)T * (size_t)E * sizeof(float) + 256;
}

hipError_t launch_router_fused(const void* x, const void* w, const float* bias, int T, int E, int D, int K,
                               int score_func, int renorm, float renorm_eps, float route_scale,
                               float* top_scores, int64_t* top_idx, void* logits, void* ws,
                               hipStream_t stream) {
  return launch_router_hist(x, w, bias, T, E, D, K, score_func, renorm, renorm_eps, route_scale, top_scores,
                            top_idx, logits, ws, nullptr, stream);
}

hipError_t launch_router_hist(const void* x, const void* w, const float* bias, int T, int E, int D, int K,
                              int score_func, int renorm, float renorm_eps, float route_scale,
                              float* top_scores, int64_t* top_idx, void* logits, void* ws, int* hist,
                              hipStream_t stream) {
  if (T == 0) return hipSuccess;
  const int S = router_splits(T, D);
  RouterGemmArgs g;
  g.x = (const bf16_t*)x;
  g.w = (const bf16_t*)w;
  g.T = T;
  g.E = E;
  g.D = D;
  const int stages = D / RTK;
  g.kstages = (stages + S - 1) / S;
  g.part = (float*)ws;
  const int nchunks = route_num_chunks((int64_t)T * K);
  g.zero = hist;
  g.nzero = hist ? (E + 1) * nchunks : 0;
  hipError_t err;
  if (E <= 32) err = launch_gemm_eb<1>(g, S, stream);
  else if (E <= 64) err = launch_gemm_eb<2>(g, S, stream);
  else if (E <= 128) err = launch_gemm_eb<4>(g, S, stream);
  else err = launch_gemm_eb<8>(g, S, stream);
  if (err != hipSuccess) return err;

  RouterTopkArgs k;
  k.part = g.part;
  k.S = S;
  k.T = T;
  k.E = E;
  k.K = K;
  k.bias = bias;
  k.score_func = score_func;
  k.renorm = renorm;
  k.eps = renorm_eps;
  k.route_scale = route_scale;
  k.scores = top_scores;
  k.idx = top_idx;
  k.logits = (bf16_t*)logits;
  k.hist = hist;
  k.nchunks = nchunks;
  k.chunk = route_chunk_labels();
  const dim3 grid((T + 15) / 16);
  auto go = [&](auto pl) {
    constexpr int PL = decltype(pl)::value;
    if (E == 16 * PL) return launch_k(false, router_topk_partials_kernel<PL, true>, grid, dim3(256), 0, stream, k);
    return launch_k(false, router_topk_partials_kernel<PL, false>, grid, dim3(256), 0, stream, k);
  };
  if (E <= 32) return go(std::integral_constant<int, 2>{});
  if (E <= 64) return go(std::integral_constant<int, 4>{});
  if (E <= 128) return go(std::integral_constant<int, 8>{});
  return go(std::integral_constant<int, 16>{});
}

static_assert(kRouterMaxE == 256, "EB = 8 covers 256 experts");

// ---------------------------------------------------------------------------
// Router backward: d(logits) (kernel above), then dx = dlogits . W_r and
// dx = dlogits . w_router on the grouped dgrad kernel as one expert, with the
// expert count padded to a multiple of 128 (zero logit-gradient columns and
// zero weight rows contribute nothing).  dW_r = dlogits^T . x on the wgrad
// kernel with the T tokens split into G groups as its "experts": G partial
// [E][D] sums, then one pass adds them in group order.  One group would leave
// the launch with D / 256 tiles (20 of 256 CUs at D = 5120).
// ---------------------------------------------------------------------------
static int router_pad_e(int E) { return (E + 127) & ~127; }
static int router_dw_rows(int E) { return E < 8 ? 8 : (E + 7) & ~7; }  // the wgrad's dy columns read (>= 8)
static int router_dw_groups(int64_t T, int E, int64_t D) {
  const int tiles = ((router_dw_rows(E) + 255) / 256) * (int)((D + 255) / 256);
  int g = 256 / tiles;  // about one tile per CU of an MI355X
  g = g < 1 ? 1 : (g > 32 ? 32 : g);
  const int64_t by_rows = T / 256;  // at least 256 rows (4 stages) per group
  return (int)(by_rows < 1 ? 1 : (g < by_rows ? g : by_rows));
}
static size_t al256(size_t b) { return (b + 255) & ~(size_t)255; }

size_t router_backward_workspace_bytes(int64_t T, int E, int64_t D) {
  const int64_t P = router_pad_e(E);
  const int64_t G = router_dw_groups(T, E, D);
  return al256((size_t)T * P * 2) + al256((size_t)P * D * 2) + al256((size_t)G * router_dw_rows(E) * D * 4) +
         al256(16) + al256((size_t)G * 4) + al256(gemm_plan_bytes(T, 1));
}

hipError_t launch_router_backward(const float* grad, const int64_t* idx, const void* logits, const void* x,
                                  const void* w, int T, int E, int D, int K, int score_func, int renorm,
                                  float renorm_eps, float route_scale, void* dx, void* dw, bool dw_fp32,
                                  void* ws, hipStream_t stream) {
  if (T == 0) return hipSuccess;
  const int P = router_pad_e(E);
  const int G = router_dw_groups(T, E, D);
  const int NR = router_dw_rows(E);
  char* p = (char*)ws;
  bf16_t* dlog = (bf16_t*)p;
  p += al256((size_t)T * P * 2);
  bf16_t* w_pad = (bf16_t*)p;
  p += al256((size_t)P * D * 2);
  float* dw_part = (float*)p;
  p += al256((size_t)G * NR * D * 4);
  int* offs1 = (int*)p;
  p += al256(16);
  int* offsg = (int*)p;
  p += al256((size_t)G * 4);
  void* gws = p;

  RouterBwdArgs b;
  b.logits = (const bf16_t*)logits;
  b.idx = idx;
  b.grad = grad;
  b.T = T;
  b.E = E;
  b.K = K;
  b.score_func = score_func;
  b.renorm = renorm;
  b.eps = renorm_eps;
  b.route_scale = route_scale;
  b.dlogits = dlog;
  b.ldd = P;
  const dim3 grid((T + 15) / 16);
  hipError_t err;
  if (E <= 32) err = launch_k(false, router_backward_kernel<2>, grid, dim3(256), 0, stream, b);
  else if (E <= 64) err = launch_k(false, router_backward_kernel<4>, grid, dim3(256), 0, stream, b);
  else if (E <= 128) err = launch_k(false, router_backward_kernel<8>, grid, dim3(256), 0, stream, b);
  else err = launch_k(false, router_backward_kernel<16>, grid, dim3(256), 0, stream, b);
  if (err != hipSuccess) return err;
  const int cpr = D / 8;
  const int pg = min(2048, (P * cpr + 255) / 256);
  if ((err = launch_k(false, router_pad_kernel, dim3(pg), dim3(256), 0, stream, (const uint4*)w, E, P, cpr,
                      (uint4*)w_pad, offs1, T, offsg, G)) != hipSuccess)
    return err;
  if (dx) {
    // dx[t][d] = sum_e dlogits[t][e] w[e][d]: dgrad with the weight [1][P][D]
    // (a reduction of P <= 1024 is at most 16 k stages: not worth splitting)
    if ((err = launch_grouped_mm_dgrad_unsplit(dlog, w_pad, offs1, T, 1, P, D, dx, gws, stream)) != hipSuccess)
      return err;
  }
  if (dw) {
    // dw_part[g][e][d] = sum over the tokens t of group g of dlogits[t][e] x[t][d]
    // (columns E..NR-1 of dlogits are the zero padding)
    WgradDmaArgs wa = {};
    wa.dy = dlog;
    wa.lddy = P;
    wa.x = (const bf16_t*)x;
    wa.ldx = D;
    wa.offs = offsg;
    wa.E = G;
    wa.M = T;
    wa.N = NR;
    wa.K = D;
    wa.n_tiles = (NR + 255) / 256;
    wa.k_tiles = (D + 255) / 256;
    wa.dw = dw_part;
    wa.dw_fp32 = 1;
    if ((err = launch_wgrad_dma(wa, stream)) != hipSuccess) return err;
    const int n4 = E * (D / 4);
    err = launch_k(false, router_dw_reduce_kernel, dim3(min(2048, (n4 + 255) / 256)), dim3(256), 0, stream,
                   (const float4*)dw_part, G, NR, E, D / 4, dw, dw_fp32 ? 1 : 0);
  }
  return err;
}

}  // namespace ttamd
