/*
 * ttamd_moe.h -- C ABI of the MI355X (gfx950) MoE expert path.
 *
 * Plain pointers and sizes only; no torch types.  Every pointer named
 * "device" is HBM memory of the current HIP device; `stream` is a
 * hipStream_t passed as void* (NULL = the legacy default stream).  All calls
 * are asynchronous on `stream` and never synchronise the host.
 *
 * Return value: 0 on success, otherwise a TTAMD_E* code; the message of the
 * last failure on the calling thread is returned by ttamd_last_error().
 * Argument checks (null pointers, sizes, alignment, 32-bit index range) are
 * done on the host before anything is launched, so a rejected call launches
 * nothing.
 *
 * bf16 tensors are raw 16-bit brain-float bits, row-major.  Routed rows are
 * numbered j = 0..M-1 with M = num_tokens * topk; "flat" slot s = t*topk + k
 * is the k-th expert choice of token t (the order of
 * selected_experts_indices.view(-1) in the reference).
 *
 * Group offsets follow torch._grouped_mm as the reference calls it
 * (torchtitanturbo/models/common/npu_gmm.py:29): `offs` is the INCLUSIVE
 * cumulative sum of per-expert row counts, int32[E]; expert e owns rows
 * [offs[e-1], offs[e]) with offs[-1] = 0.  Rows at or past offs[E-1] are not
 * read and not written.
 */
#ifndef TTAMD_MOE_H
#define TTAMD_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TTAMD_ABI_VERSION 1

enum {
  TTAMD_OK = 0,
  TTAMD_EINVAL = 1,  /* bad argument: null pointer, size, alignment, range */
  TTAMD_ERUNTIME = 2 /* a HIP runtime call failed (launch, attribute query) */
};

/* Score function applied by the router top-k (upstream TokenChoiceTopKRouter). */
enum { TTAMD_SCORE_SOFTMAX = 0, TTAMD_SCORE_SIGMOID = 1 };

int ttamd_abi_version(void);
const char* ttamd_last_error(void);

/* ------------------------------------------------------------------------ *
 * Routing: router top-k, histogram, stable counting sort, row permute.      *
 * ------------------------------------------------------------------------ */

/*
 * Router top-k over per-token expert logits (fp32 [T,E]).
 * Replaces the selection stage of upstream TokenChoiceTopKRouter; the
 * in-reference closed form is torchtitanturbo/models/qwen3_5/model.py:757-765
 * (softmax in fp32, topk, renormalise by the sum of the k values).
 *   score = softmax(logits) or sigmoid(logits), fp32;
 *   pick k experts with the largest score (ties: lower expert id first),
 *   in descending score order;
 *   if renorm: top_scores /= (sum of the k picked scores + renorm_eps);
 *   top_scores *= route_scale.
 * expert_bias (nullable, fp32[E]) is added to the score for SELECTION only
 * (the returned score is the unbiased one), as upstream's load-balancing
 * bias does.  Outputs: top_scores fp32[T,K], top_indices int64[T,K].
 * Requires 1 <= K <= E <= 1024, K <= 16.
 */
int ttamd_router_topk(const float* logits, const float* expert_bias,
                      int64_t num_tokens, int num_experts, int topk,
                      int score_func, int renorm, float renorm_eps,
                      float route_scale, float* top_scores,
                      int64_t* top_indices, void* stream);

/*
 * Router forward: gate GEMM + score + top-k (+ renorm).
 * Replaces upstream TokenChoiceTopKRouter.forward (gate nn.Linear in bf16,
 * fp32 score, topk, renorm); in-reference closed form
 * torchtitanturbo/models/qwen3_5/model.py:752-766 (F.linear :757, softmax
 * fp32 :758, topk :759-761, renorm :762-764).
 *   logits[t, e] = bf16(sum_d x[t, d] * w_router[e, d])  (fp32 accumulate)
 *   then exactly as ttamd_router_topk on those logits.
 * x bf16 [T, D], w_router bf16 [E, D]; D % 64 == 0; 1 <= K <= min(16, E);
 * E <= 256.  logits_out (nullable) receives the bf16 logits [T, E].
 * Outputs as ttamd_router_topk.  workspace: ttamd_router_workspace_bytes
 * (fp32 partial logits of the split gate GEMM).
 */
size_t ttamd_router_workspace_bytes(int64_t num_tokens, int num_experts,
                                    int64_t dim);
int ttamd_router_fused(const void* x, const void* w_router,
                       const float* expert_bias, int64_t num_tokens,
                       int num_experts, int64_t dim, int topk, int score_func,
                       int renorm, float renorm_eps, float route_scale,
                       float* top_scores, int64_t* top_indices,
                       void* logits_out, void* workspace,
                       size_t workspace_bytes, void* stream);

/*
 * Router backward: the autograd of the router forward above.
 * Replaces the backward torch autograd runs through upstream
 * TokenChoiceTopKRouter.forward (closed form
 * torchtitanturbo/models/qwen3_5/model.py:752-766: gate nn.Linear in bf16,
 * softmax / sigmoid in fp32, topk / gather, renorm, route_scale).
 *   g_k    = route_scale * grad_top_scores[t, k]
 *   renorm: S = sum_k s[idx_k] + eps; ds[idx_k] = g_k / S
 *           + sum_j (-g_j s[idx_j] / S^2); else ds[idx_k] = g_k (0 elsewhere)
 *   softmax: dz = (ds - <ds, s>) * s;  sigmoid: dz = ds * (1 - s) * s
 *   dlogits = bf16(dz)  (the gradient of the bf16 logits)
 *   grad_x [T, D] bf16 = dlogits . w_router          (nullable)
 *   grad_w_router [E, D] = dlogits^T . x              (nullable; fp32 when
 *                                                      grad_w_is_fp32, else bf16)
 * s is recomputed from logits (bf16 [T, E], the forward's logits_out).
 * expert_bias only steers the selection and has no gradient here.
 * D % 128 == 0; other limits as ttamd_router_fused.  workspace:
 * ttamd_router_backward_workspace_bytes.
 */
size_t ttamd_router_backward_workspace_bytes(int64_t num_tokens,
                                             int num_experts, int64_t dim);
int ttamd_router_backward(const float* grad_top_scores,
                          const int64_t* top_indices, const void* logits,
                          const void* x, const void* w_router,
                          int64_t num_tokens, int num_experts, int64_t dim,
                          int topk, int score_func, int renorm,
                          float renorm_eps, float route_scale, void* grad_x,
                          void* grad_w_router, int grad_w_is_fp32,
                          void* workspace, size_t workspace_bytes,
                          void* stream);

/*
 * Router + dispatch order in one call: the router of ttamd_router_fused,
 * then the histogram and stable order of ttamd_moe_route over its picks
 * (selected_experts_indices.view(-1)), with no round trip between them.
 * Replaces upstream TokenChoiceTopKRouter.forward (closed form
 * torchtitanturbo/models/qwen3_5/model.py:752-766) followed by dispatch's
 * histc + stable argsort (reached from npu_gmm.py:106-108).
 *   Outputs: top_scores / top_indices as ttamd_router_fused; counts,
 *   offsets, sorted_indices, inverse, sorted_scores as ttamd_moe_route
 *   (counts, offsets, inverse, sorted_scores nullable; sorted_scores[j] =
 *   top_scores.view(-1)[sorted_indices[j]]).
 *   tokens_per_expert (nullable, fp32 [E]) += counts: upstream's
 *   load-balancing accumulator (router.tokens_per_expert.add_(histc)).
 *   gemm_plan (nullable, ttamd_gemm_plan_bytes(T*topk, E) bytes)
 *   receives the token-tile table of the expert-sorted rows that
 *   ttamd_moe_experts_forward can use for both grouped GEMMs.
 *   counts and offsets may be NULL only when gemm_plan and
 *   tokens_per_expert are both NULL (TTAMD_EINVAL otherwise): the tile
 *   table is built from the offsets and the accumulator from the counts.
 * Same argument limits as ttamd_router_fused; workspace:
 * ttamd_router_route_workspace_bytes.  Launches: gate GEMM, score + top-k
 * + histogram, rank (the histogram scan folded in for (E + 1) *
 * ceil(T*topk / 1024) <= 32768).
 */
size_t ttamd_router_route_workspace_bytes(int64_t num_tokens, int num_experts,
                                          int64_t dim, int topk);
int ttamd_router_route(const void* x, const void* w_router,
                       const float* expert_bias, int64_t num_tokens,
                       int num_experts, int64_t dim, int topk, int score_func,
                       int renorm, float renorm_eps, float route_scale,
                       float* top_scores, int64_t* top_indices,
                       int32_t* counts, int32_t* offsets,
                       int32_t* sorted_indices, int32_t* inverse,
                       float* sorted_scores, float* tokens_per_expert,
                       void* gemm_plan, size_t gemm_plan_bytes,
                       void* workspace, size_t workspace_bytes, void* stream);

/* Bytes of device workspace ttamd_moe_route / ttamd_moe_token_permute need. */
size_t ttamd_route_workspace_bytes(int64_t num_flat, int num_experts);

/*
 * Per-expert histogram + stable counting sort of flat expert labels.
 * Replaces upstream dispatch's `torch.histc(idx.view(-1), bins=E)` +
 * `torch.argsort(idx.view(-1), stable=True)` (reached from
 * torchtitanturbo/models/common/npu_gmm.py:106-108) and the index half of
 * torch_npu.npu_moe_token_permute (npu_permute.py:74-76).
 *   labels: device int64 (labels_are_int64=1) or int32 [num_flat]
 *   counts[e]   = #{s : labels[s] == e}                       int32[E]
 *   offsets[e]  = sum_{e'<e} counts[e'], offsets[E] = #valid   int32[E+1]
 *   sorted_indices[j] = the j-th flat slot in stable label order int32[M]
 *   inverse[s]  = position j of slot s (nullable)               int32[M]
 *   sorted_scores[j] = scores[sorted_indices[j]] (both nullable) fp32[M]
 * Labels outside [0,E) are sorted after every valid label (positions
 * [offsets[E], M)), so sorted_indices is always a permutation of [0,M).
 * Bit-exact: identical to a stable argsort for every valid input.
 */
int ttamd_moe_route(const void* labels, int labels_are_int64, int64_t num_flat,
                    int num_experts, const float* scores, int32_t* counts,
                    int32_t* offsets, int32_t* sorted_indices,
                    int32_t* inverse, float* sorted_scores, void* workspace,
                    size_t workspace_bytes, void* stream);

/*
 * ttamd_moe_route without a workspace argument: it allocates nothing.
 * No counterpart in the reference.  It is for callers that cannot allocate
 * device memory: code under HIP graph capture, tight serving loops and
 * harnesses that forbid hipMalloc.
 *   Same arguments (minus the workspace), outputs and bit-exact results as
 *   ttamd_moe_route.  The per-chunk histogram lives in a device array the
 *   library holds on each device it runs on, TTAMD_ROUTE_NOALLOC_WORKSPACE_BYTES
 *   long, from the first call on that device until the process ends.
 *   Limit: the histogram, (E + 1) * ceil(num_flat / 1024) int32, must fit
 *   that array (at most 2^20 ints: e.g. up to 2^20 labels with E <= 1023);
 *   larger calls are rejected with TTAMD_EINVAL and launch nothing.
 *   Every call on one device shares that device's array: calls that overlap
 *   on one device (other streams, other host threads) race and give wrong
 *   results, so serialise them.  The array keeps the last call's contents;
 *   nothing in it has to start at zero.  The device is the one `stream`
 *   belongs to (the current device for a NULL stream).
 */
#define TTAMD_ROUTE_NOALLOC_WORKSPACE_BYTES ((size_t)4 << 20)
int ttamd_moe_route_noalloc(const void* labels, int labels_are_int64,
                            int64_t num_flat, int num_experts,
                            const float* scores, int32_t* counts,
                            int32_t* offsets, int32_t* sorted_indices,
                            int32_t* inverse, float* sorted_scores,
                            void* stream);

/*
 * Row gather of the permute: out[j] = in[src_index[j] / topk], optionally
 * multiplied by row_scale[j] in fp32 and rounded to bf16 once (upstream
 * dispatch with score_before_experts).  bf16 [num_in_rows, hidden] ->
 * bf16 [num_out_rows, hidden].  hidden % 8 == 0, 16-byte aligned rows.
 */
int ttamd_moe_gather_rows(const void* in, const int32_t* src_index,
                          const float* row_scale, int64_t num_in_rows,
                          int64_t num_out_rows, int64_t hidden, int topk,
                          void* out, void* stream);

/*
 * The permute rows of ttamd_moe_gather_rows in scatter form, from the
 * inverse map of ttamd_moe_route: out[inverse[t*topk + k]] = tokens[t],
 * optionally times scores[t*topk + k] in fp32 and rounded to bf16 once
 * (score before experts).  Identical output to ttamd_moe_gather_rows with
 * src_index = sorted_indices and row_scale = sorted_scores, but each token
 * row is read from HBM once.  tokens bf16 [T, D] -> out bf16 [T*topk, D];
 * topk <= 64.
 */
int ttamd_moe_dispatch_rows(const void* tokens, const int32_t* inverse,
                            const float* scores, int64_t num_tokens,
                            int64_t hidden, int topk, void* out, void* stream);

/*
 * Drop-in for torch_npu.npu_moe_token_permute(tokens, indices)
 * (torchtitanturbo/models/common/npu_permute.py:74-76): stable sort of the
 * flat labels and gather of token rows.  tokens bf16 [T,D]; labels
 * [T*topk] (int64 or int32); permuted bf16 [T*topk, D];
 * sorted_indices int32 [T*topk] = stable argsort of the labels (the map
 * ttamd_moe_token_unpermute takes back).  num_experts bounds the label
 * range (labels outside [0,num_experts) sort last).  counts (nullable)
 * int32[num_experts] receives the histogram.
 */
int ttamd_moe_token_permute(const void* tokens, const void* labels,
                            int labels_are_int64, int64_t num_tokens,
                            int64_t hidden, int topk, int num_experts,
                            void* permuted, int32_t* sorted_indices,
                            int32_t* counts, void* workspace,
                            size_t workspace_bytes, void* stream);

/* Bytes of device workspace ttamd_moe_token_unpermute needs. */
size_t ttamd_unpermute_workspace_bytes(int64_t num_tokens, int topk);

/*
 * Drop-in for torch_npu._npu_moe_token_unpermute_with_routing_map
 * (npu_permute.py:23-30) and for upstream combine's unsort + K-way sum:
 *   out[t] = sum_k w(t,k) * permuted[j(t,k)],  j(t,k) = position of flat
 *   slot t*topk+k in sorted_indices, w = probs[t,k] (fp32, nullable -> 1).
 * Accumulates in fp32, rounds to bf16 once.  permuted bf16 [T*topk, D],
 * out bf16 [T, D].  Deterministic (fixed k order, no atomics).
 */
int ttamd_moe_token_unpermute(const void* permuted,
                              const int32_t* sorted_indices,
                              const float* probs, int64_t num_tokens,
                              int64_t hidden, int topk, void* out,
                              void* workspace, size_t workspace_bytes,
                              void* stream);

/*
 * Same sum, given the inverse map (inverse[s] = position of flat slot s)
 * that ttamd_moe_route returns; needs no workspace.
 */
int ttamd_moe_combine(const void* permuted, const int32_t* inverse,
                      const float* probs, int64_t num_tokens, int64_t hidden,
                      int topk, void* out, void* stream);

/*
 * Drop-in for torch_npu.npu_moe_token_unpermute_with_routing_map_grad
 * (npu_permute.py:41-50):
 *   grad_permuted[j] = w(s) * grad_out[s / topk],  s = sorted_indices[j],
 *   w(s) = probs[s] (nullable -> 1), rounded to bf16 once.
 * If grad_probs is non-null (and probs, permuted are given):
 *   grad_probs[s] = <grad_out[s/topk], permuted[j]> accumulated in fp32.
 */
int ttamd_moe_token_unpermute_grad(const void* grad_out,
                                   const int32_t* sorted_indices,
                                   const float* probs, const void* permuted,
                                   int64_t num_tokens, int64_t hidden,
                                   int topk, void* grad_permuted,
                                   float* grad_probs, void* stream);

/*
 * Row dot products: out[o(j)] = <a[j], b[b_index[j] / b_div]> in fp32,
 * o(j) = out_by_index ? b_index[j] : j (b_index nullable -> j).
 * Used for routing-score gradients.
 */
int ttamd_moe_rowdot(const void* a, const void* b, const int32_t* b_index,
                     int b_div, int out_by_index, int64_t num_rows,
                     int64_t num_b_rows, int64_t hidden, float* out,
                     void* stream);

/*
 * Expert labels of rows laid out as num_groups consecutive groups
 * (source rank r, local expert e), g = r * num_local_experts + e:
 *   labels[j] = g(j) % num_local_experts, g(j) the group holding row j;
 *   rows past sum(counts_group) get label num_local_experts.
 * Replaces the label construction of NpuTokenDispatcher._permute
 * (torchtitanturbo/models/common/npu_permute.py:68-72:
 * arange(E_loc).repeat(ep).repeat_interleave(counts)), with no host sync.
 * counts_group int32 [num_groups], num_groups <= 8192; labels int32 [rows].
 */
int ttamd_moe_group_labels(const int32_t* counts_group, int num_groups,
                           int num_local_experts, int64_t num_rows,
                           int32_t* labels, void* stream);

/* ------------------------------------------------------------------------ *
 * Grouped GEMMs over ragged expert segments (bf16 in, fp32 accumulate).     *
 * ------------------------------------------------------------------------ */

/* Bytes of device workspace every ttamd_grouped_mm* call needs: the
 * tile plan (ttamd_gemm_plan_bytes) followed by the partial sums of the
 * GEMMs' split leftover tiles (tiles left after the last full round of the
 * persistent walk are cut along k over the idle CUs; the last piece of a
 * tile adds the pieces in a fixed order, so results do not depend on which
 * piece finishes last). */
size_t ttamd_gemm_workspace_bytes(int64_t num_rows, int num_experts);

/* Bytes of a tile plan (gemm_plan of ttamd_router_route and
 * ttamd_moe_experts_forward): the token-tile table of num_rows
 * expert-sorted rows and the split-tile arrival counters.  No counterpart
 * in the reference, whose grouped GEMM plans inside the operator. */
size_t ttamd_gemm_plan_bytes(int64_t num_rows, int num_experts);

/*
 * out[m, n] = sum_k x[m, k] * w[e(m), n, k]  (bf16 out).
 * Replaces torch._grouped_mm(x, w.transpose(-2,-1), offs)
 * (torchtitanturbo/models/common/npu_gmm.py:17-18, :38).
 * x [M, K], w [E, N, K], out [M, N]; N % 128 == 0, K % 64 == 0.
 */
int ttamd_grouped_mm(const void* x, const void* w, const int32_t* offs,
                     int64_t num_rows, int num_experts, int64_t n, int64_t k,
                     void* out, void* workspace, size_t workspace_bytes,
                     void* stream);

/*
 * Fused expert up-projection: h = x @ w13[e]^T (w13 [E, 2H, D], rows 0..H-1
 * gate, H..2H-1 up), optional clamp (gate <= L, -L <= up <= L with
 * L = swiglu_limit, applied for every L >= 0, including 0; as torch.clamp, a
 * NaN stays NaN), a = silu(gate) * up.
 * Replaces npu_gmm.py:29-37 (cumsum, grouped_mm w13, clamp, npu_swiglu).
 * x [M, D] -> a [M, H] bf16; h_out (nullable) receives the unclamped
 * pre-activation bf16 [M, 2H] for the backward.  H % 64 == 0, D % 64 == 0.
 * swiglu_limit: NaN = no clamp (the reference's swiglu_limit=None);
 * negative values are refused.
 */
int ttamd_grouped_mm_swiglu(const void* x, const void* w13,
                            const int32_t* offs, int64_t num_rows,
                            int num_experts, int64_t hidden, int64_t dim,
                            float swiglu_limit, void* a_out, void* h_out,
                            void* workspace, size_t workspace_bytes,
                            void* stream);

/*
 * ttamd_grouped_mm_swiglu with the permute gather fused into its loads:
 * routed row j is tokens[src_index[j] / src_div] (src_index =
 * sorted_indices of ttamd_moe_route, src_div = topk), so the routed
 * [M, D] copy is never written.  Replaces the gather of
 * npu_moe_token_permute (npu_permute.py:74-76; upstream dispatch's
 * index_select, reached from npu_gmm.py:106-108) plus npu_gmm.py:29-37 on
 * the inference path (score applied after the experts).  tokens bf16
 * [num_tokens, D] (< 4 GiB); H % 64 == 0, D % 64 == 0, D >= 128.
 */
int ttamd_grouped_mm_swiglu_gather(const void* tokens, int64_t num_tokens,
                                   const int32_t* src_index, int src_div,
                                   const void* w13, const int32_t* offs,
                                   int64_t num_rows, int num_experts,
                                   int64_t hidden, int64_t dim,
                                   float swiglu_limit, void* a_out,
                                   void* h_out, void* workspace,
                                   size_t workspace_bytes, void* stream);

/*
 * Fused expert down-projection + routing-weight scale + un-permute:
 *   y[j] = a[j] @ w2[e(j)]^T  (w2 [E, D, H]),  fp32
 *   v    = row_scale ? row_scale[j] * y[j] : y[j]
 *   out[dest[j]] = bf16(v)   (dest nullable -> j)
 * With dest = sorted_indices and topk = 1 this writes the combined layer
 * output [T, D] directly; with topk > 1 it writes the flat-slot-ordered
 * buffer that ttamd_moe_sum_topk reduces.  Replaces npu_gmm.py:38 plus the
 * unsort/score multiply of upstream combine.  D % 128 == 0, H % 64 == 0.
 */
int ttamd_grouped_mm_unpermute(const void* a, const void* w2,
                               const int32_t* offs, int64_t num_rows,
                               int num_experts, int64_t dim, int64_t hidden,
                               const float* row_scale, const int32_t* dest,
                               int64_t num_dest_rows, void* out,
                               void* workspace, size_t workspace_bytes,
                               void* stream);

/*
 * The expert stage of the MoE layer forward (inference) in one call:
 * NpuGroupedExperts.forward's dispatch -> _run_experts_grouped_mm ->
 * combine (torchtitanturbo/models/common/npu_gmm.py:100-110 with :21-40),
 * given the routing of ttamd_moe_route / ttamd_router_route:
 *   routed[j] = tokens[sorted_indices[j] / topk] (* sorted_scores[j] when
 *               score_before_experts, rounded to bf16 once);
 *   a = silu(gate) * up of routed @ w13[e]^T (clamp as
 *       ttamd_grouped_mm_swiglu);
 *   y[j] = a[j] @ w2[e]^T (* sorted_scores[j] when the score comes after);
 *   out[t] = sum_k y[j(t, k)]  (fp32 sum, bf16 out; topk = 1: a scatter).
 * tokens bf16 [T, D]; offs inclusive int32 [E] (ttamd_moe_route's offsets
 * + 1); w13 [E, 2H, D], w2 [E, D, H]; out bf16 [T, D].  Every label must be
 * in [0, E) (offs[E-1] = T * topk).  D % 128 == 0, H % 64 == 0.
 * Without score_before_experts the gather is fused into the w13 GEMM's
 * loads (the routed copy is never written).  gemm_plan (nullable): the tile
 * plan from ttamd_router_route for these offs; both GEMMs use it (null:
 * one is built in the workspace).  Its split-tile counters are counted up
 * and back to zero by each GEMM, so one plan serves one call at a time.
 * workspace:
 * ttamd_moe_experts_forward_workspace_bytes (tile table, a, and for
 * score-before the routed rows, for topk > 1 y).
 */
size_t ttamd_moe_experts_forward_workspace_bytes(int64_t num_tokens,
                                                 int64_t dim, int64_t hidden,
                                                 int num_experts, int topk,
                                                 int score_before_experts);
int ttamd_moe_experts_forward(const void* tokens, int64_t num_tokens,
                              int64_t dim, int64_t hidden, int num_experts,
                              int topk, const int32_t* sorted_indices,
                              const int32_t* offs, const float* sorted_scores,
                              int score_before_experts, float swiglu_limit,
                              const void* w13, const void* w2, void* out,
                              void* gemm_plan, size_t gemm_plan_bytes,
                              void* workspace, size_t workspace_bytes,
                              void* stream);

/* out[t] = sum_{k<topk} in[t*topk + k] (fp32 accumulate, bf16 out). */
int ttamd_moe_sum_topk(const void* in, int64_t num_tokens, int64_t hidden,
                       int topk, void* out, void* stream);

/*
 * Shared expert fused into the combine: out[t] += g(t) * FFN(x[t]), where
 *   FFN(x) = (silu(gate) * up) @ w2_shared^T with [gate | up] = x @ w13_shared^T
 *            (gate rows 0..H-1, up rows H..2H-1; optional clamp as
 *            ttamd_grouped_mm_swiglu), one bf16 FeedForward;
 *   g(t)   = sigmoid(gate_logits[t]) when gate_logits (fp32 [T]) is given,
 *            else 1.
 * Replaces the shared-expert tail of the reference MoE block,
 * torchtitanturbo/models/qwen3_5/model.py:796-809 (shared_expert FeedForward,
 * sigmoid(shared_expert_gate(x)) * shared, expert_output + shared), and
 * UPSTREAM Llama4's ungated `out + shared_experts(x)`.  out bf16 [T, D]
 * holds the combined routed output on entry and the sum on return;
 * a_scratch bf16 [T, H] is caller-owned scratch (the SwiGLU output).
 * x bf16 [T, D]; w13_shared [2H, D]; w2_shared [D, H]; D % 128 == 0,
 * H % 64 == 0; workspace: ttamd_gemm_workspace_bytes(T, 1).
 * swiglu_limit: NaN = no clamp (the reference's swiglu_limit=None), else
 * >= 0 (0 clamps to zero, as ttamd_grouped_mm_swiglu does).
 */
int ttamd_shared_expert_add(const void* x, int64_t num_tokens, int64_t dim,
                            int64_t hidden, const void* w13_shared,
                            const void* w2_shared, const float* gate_logits,
                            float swiglu_limit, void* a_scratch, void* out,
                            void* workspace, size_t workspace_bytes,
                            void* stream);

/*
 * Grouped dgrad: dx[m, k] = sum_n dy[m, n] * w[e(m), n, k]  (bf16 out).
 * Backward of ttamd_grouped_mm w.r.t. x; w [E, N, K] with K contiguous.
 * N % 64 == 0, K % 128 == 0.
 */
int ttamd_grouped_mm_dgrad(const void* dy, const void* w, const int32_t* offs,
                           int64_t num_rows, int num_experts, int64_t n,
                           int64_t k, void* dx, void* workspace,
                           size_t workspace_bytes, void* stream);

/*
 * Grouped dgrad of the down projection fused with the SwiGLU backward:
 *   g[m, p]  = sum_d dy[m, d] * w2[e(m), d, p]          (dA, fp32)
 *   with h = [gate | up] from ttamd_grouped_mm_swiglu (h_out), L = limit:
 *   gc = min(gate, L), uc = clamp(up, -L, L)   (NaN stays NaN)
 *   dgate = [gate <= L]      ? g * uc * silu'(gc) : 0
 *   dup   = [-L <= up <= L]  ? g * silu(gc)       : 0
 *   (torch.clamp's backward: exactly 0 where it clamps or meets a NaN;
 *   without a clamp every mask is true)
 *   dh[m] = [dgate | dup]  bf16 [M, 2H]
 * a_out (nullable) receives silu(gc)*uc recomputed in bf16 [M, H].
 * D % 64 == 0, H % 128 == 0; swiglu_limit NaN = no clamp.
 */
int ttamd_grouped_mm_dgrad_swiglu(const void* dy, const void* w2,
                                  const void* h, const int32_t* offs,
                                  int64_t num_rows, int num_experts,
                                  int64_t dim, int64_t hidden,
                                  float swiglu_limit, void* dh, void* a_out,
                                  void* workspace, size_t workspace_bytes,
                                  void* stream);

/*
 * Grouped wgrad: dw[e, n, k] = sum_{m in group e} dy[m, n] * x[m, k].
 * dy [M, N], x [M, K] bf16; dw [E, N, K] fp32 (dw_is_fp32=1) or bf16.
 * Experts with no rows get zeros.  N % 128 == 0, K % 128 == 0.
 * workspace: NULL, or ttamd_gemm_workspace_bytes(num_rows, num_experts)
 * bytes (contents need no initialisation): with it, the output tiles left
 * over after the last full round of the persistent walk are cut along the
 * rows into pieces that run on the otherwise idle CUs.  Deterministic
 * either way: the pieces' fp32 sums are added in piece order, whichever
 * finishes last (one arrival counter per leftover tile).
 */
int ttamd_grouped_mm_wgrad(const void* dy, const void* x, const int32_t* offs,
                           int64_t num_rows, int num_experts, int64_t n,
                           int64_t k, void* dw, int dw_is_fp32,
                           void* workspace, size_t workspace_bytes,
                           void* stream);

/* ------------------------------------------------------------------------ *
 * fp8 e4m3 experts with fp32 block scales.               *
 * The reference has no fp8 path; these follow the published recipe the      *
 * north star names: scale = absmax / 448 per block, code = e4m3fn(v /       *
 * scale) rounded to nearest even, value = code * scale, GEMM in fp32.      *
 * e4m3 is the OCP "fn" format (bias 7, max 448, 0x7f = NaN).  An all-zero   *
 * block has scale 0 and codes 0.  Inputs are finite.                        *
 * ------------------------------------------------------------------------ */

/*
 * Activations: one scale per row and 128 channels.
 *   row j of the output is input row src_index[j] / src_div (src_index
 *   nullable -> j), optionally multiplied by row_scale[j] in fp32 and
 *   rounded to bf16 first (score-before-experts dispatch);
 *   q_out uint8 [num_rows, k]; scale_t fp32 [k / 128, num_rows] (k-block
 *   major, the layout the fp8 GEMMs read).
 * Fuses the permute gather of ttamd_moe_gather_rows with the quantisation.
 * k % 128 == 0, k <= 8192.
 */
int ttamd_quantize_fp8_rows(const void* in, const int32_t* src_index, int src_div,
                            const float* row_scale, int64_t num_in_rows,
                            int64_t num_rows, int64_t k, void* q_out,
                            float* scale_t, void* stream);

/*
 * Weights: one scale per 128 x 128 block of each expert matrix.
 * w bf16 [E, n, k] -> q_out uint8 [E, n, k], scale fp32 [E, n/128, k/128].
 * n % 128 == 0, k % 128 == 0, k <= 8192.
 */
int ttamd_quantize_fp8_blocks(const void* w, int num_experts, int64_t n,
                              int64_t k, void* q_out, float* scale,
                              void* stream);

/*
 * fp8 grouped GEMM: out[m, n] = sum_k (xq[m,k] * sx) * (wq[e(m),n,k] * sw)
 * with fp32 accumulation, bf16 out.  xq uint8 [M, k], sx_t fp32 [k/128, M]
 * (from ttamd_quantize_fp8_rows), wq uint8 [E, n, k], sw fp32
 * [E, n/128, k/128].  Replaces npu_gmm.py:31/:38's torch._grouped_mm on
 * dequantised operands.  n % 128 == 0, k % 128 == 0.
 */
int ttamd_grouped_mm_fp8(const void* xq, const float* sx_t, const void* wq,
                         const float* sw, const int32_t* offs, int64_t num_rows,
                         int num_experts, int64_t n, int64_t k, void* out,
                         void* workspace, size_t workspace_bytes, void* stream);

/*
 * fp8 version of ttamd_grouped_mm_swiglu: w13q [E, 2H, D] with scales
 * [E, 2H/128, D/128]; same clamp, SwiGLU and bf16 outputs (a [M, H],
 * optional h [M, 2H]).  H % 64 == 0, D % 128 == 0.
 */
int ttamd_grouped_mm_fp8_swiglu(const void* xq, const float* sx_t,
                                const void* w13q, const float* s13,
                                const int32_t* offs, int64_t num_rows,
                                int num_experts, int64_t hidden, int64_t dim,
                                float swiglu_limit, void* a_out, void* h_out,
                                void* workspace, size_t workspace_bytes,
                                void* stream);

/*
 * fp8 version of ttamd_grouped_mm_unpermute: aq uint8 [M, H] with sa_t
 * [H/128, M], w2q [E, D, H] with scales [E, D/128, H/128]; same routing
 * scale and scatter.  D % 128 == 0, H % 128 == 0.
 */
int ttamd_grouped_mm_fp8_unpermute(const void* aq, const float* sa_t,
                                   const void* w2q, const float* s2,
                                   const int32_t* offs, int64_t num_rows,
                                   int num_experts, int64_t dim, int64_t hidden,
                                   const float* row_scale, const int32_t* dest,
                                   int64_t num_dest_rows, void* out,
                                   void* workspace, size_t workspace_bytes,
                                   void* stream);

/* ------------------------------------------------------------------------
 * Kernel timing probe.  No counterpart in the reference: a measurement aid
 * for benchmarks that need one kernel's duration from inside a larger op.
 * ------------------------------------------------------------------------ */

/*
 * Arm the probe: the next grouped-GEMM main kernel this host thread
 * launches (any
 * ttamd_grouped_mm* entry point, forward or dgrad, bf16 or fp8; not the
 * tile-table kernel before it) takes start_event and end_event as its own
 * start and end stamps (hipExtLaunchKernelGGL: nothing is enqueued between
 * kernels), then the probe disarms.  The events are caller-owned
 * hipEvent_t created with timing enabled (torch.cuda.Event(enable_timing=
 * True) after one record()).  NULL for both disarms.  While a launch chain
 * (ttamd_probe_launches) is armed it takes the launches first.  The
 * probe is per host thread: launches from other threads (for example
 * torch's autograd worker running a backward) are not stamped.
 */
int ttamd_probe_next_gemm(void* start_event, void* end_event);

/*
 * Arm a chain over the next num_launches kernel launches of this host
 * thread's library calls (router, route, permute / quantise, grouped GEMMs, K-way
 * sum: every kernel the entry points launch), whatever they are: launch i
 * takes events[2 i] and events[2 i + 1] as its start and end stamps
 * (caller-owned hipEvent_t with timing enabled; the stamps come from the
 * kernel's own dispatch), or runs unstamped when both are NULL, so a
 * caller can time one chosen kernel of a sequence.  A stamped dispatch
 * costs a few microseconds of GPU time.  0 <= num_launches <= 16; 0
 * disarms.  Per host thread, as ttamd_probe_next_gemm.
 */
int ttamd_probe_launches(void* const* events, int num_launches);

#ifdef __cplusplus
}
#endif

#endif /* TTAMD_MOE_H */
