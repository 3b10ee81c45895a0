// extern "C" entry points of libttamd_moe.so (declared in include/ttamd_moe.h).
//
// This layer owns argument validation: every size, alignment and range the
// kernels rely on is checked here, on the host, before anything is launched.
// A rejected call returns TTAMD_EINVAL and launches nothing.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/ttamd_moe.h"
#include "kernels.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int check_hip(hipError_t err, const char* what) {
  if (err != hipSuccess) return fail(TTAMD_ERUNTIME, "%s: %s", what, hipGetErrorString(err));
  return TTAMD_OK;
}

constexpr int64_t kI32Max = 2147483647;

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

#define REQUIRE(cond, ...)                        \
  do {                                            \
    if (!(cond)) return fail(TTAMD_EINVAL, __VA_ARGS__); \
  } while (0)

// Rows of `hidden` bf16 moved as 16-byte chunks.
int check_rows(const char* fn, const char* name, const void* p, int64_t rows, int64_t hidden) {
  if (rows > 0 && p == nullptr) return fail(TTAMD_EINVAL, "%s: %s is null", fn, name);
  if (rows > 0 && !aligned16(p))
    return fail(TTAMD_EINVAL, "%s: %s must be 16-byte aligned", fn, name);
  // 16-byte chunk indices stay below 2^30 so grid-stride arithmetic never
  // approaches the int32 range.
  if (rows * (hidden / 8) > (int64_t(1) << 30))
    return fail(TTAMD_EINVAL, "%s: %s has too many elements (%lld x %lld)", fn, name,
                (long long)rows, (long long)hidden);
  return TTAMD_OK;
}

int check_hidden(const char* fn, int64_t hidden) {
  if (hidden <= 0 || hidden % 8 != 0)
    return fail(TTAMD_EINVAL, "%s: hidden must be a positive multiple of 8 (got %lld)", fn,
                (long long)hidden);
  return TTAMD_OK;
}

int check_gemm_common(const char* fn, const int32_t* offs, int64_t M, int E) {
  REQUIRE(offs != nullptr, "%s: offs is null", fn);
  REQUIRE(E >= 1 && E <= 1024, "%s: num_experts must be in [1, 1024] (got %d)", fn, E);
  REQUIRE(M >= 0 && M <= (1 << 28), "%s: num_rows out of range (%lld)", fn, (long long)M);
  return TTAMD_OK;
}

int check_dim(const char* fn, const char* name, int64_t v, int mult) {
  if (v <= 0 || v % mult != 0 || v > (1 << 20))
    return fail(TTAMD_EINVAL, "%s: %s must be a positive multiple of %d (got %lld)", fn, name,
                mult, (long long)v);
  return TTAMD_OK;
}

int check_ws(const char* fn, const void* ws, size_t have, size_t need) {
  if (need > 0 && (ws == nullptr || have < need))
    return fail(TTAMD_EINVAL, "%s: workspace too small (%zu bytes, need %zu)", fn, have, need);
  if (ws != nullptr && !aligned16(ws)) return fail(TTAMD_EINVAL, "%s: workspace must be 16-byte aligned", fn);
  return TTAMD_OK;
}

#define TRY(expr)            \
  do {                       \
    int _rc = (expr);        \
    if (_rc != TTAMD_OK) return _rc; \
  } while (0)

}  // namespace

extern "C" {

int ttamd_abi_version(void) { return TTAMD_ABI_VERSION; }

const char* ttamd_last_error(void) { return g_last_error.c_str(); }

int ttamd_router_topk(const float* logits, const float* expert_bias, int64_t num_tokens,
                      int num_experts, int topk, int score_func, int renorm, float renorm_eps,
                      float route_scale, float* top_scores, int64_t* top_indices, void* stream) {
  const char* fn = "ttamd_router_topk";
  REQUIRE(num_tokens >= 0 && num_tokens * (int64_t)num_experts <= kI32Max * 4LL,
          "%s: num_tokens out of range", fn);
  REQUIRE(num_experts >= 1 && num_experts <= 1024, "%s: num_experts must be in [1, 1024]", fn);
  REQUIRE(topk >= 1 && topk <= 16 && topk <= num_experts, "%s: topk must be in [1, min(16, E)]",
          fn);
  REQUIRE(score_func == TTAMD_SCORE_SOFTMAX || score_func == TTAMD_SCORE_SIGMOID,
          "%s: unknown score_func %d", fn, score_func);
  REQUIRE(num_tokens <= kI32Max, "%s: num_tokens too large", fn);
  if (num_tokens > 0)
    REQUIRE(logits && top_scores && top_indices, "%s: null pointer argument", fn);
  return check_hip(ttamd::launch_router_topk(logits, expert_bias, (int)num_tokens, num_experts,
                                             topk, score_func, renorm, renorm_eps, route_scale,
                                             top_scores, top_indices, (hipStream_t)stream),
                   fn);
}

size_t ttamd_router_workspace_bytes(int64_t num_tokens, int num_experts, int64_t dim) {
  if (num_tokens <= 0 || num_experts < 1 || dim < 64) return 0;
  return ttamd::router_workspace_bytes(num_tokens, num_experts, dim);
}

int ttamd_router_fused(const void* x, const void* w_router, const float* expert_bias,
                       int64_t num_tokens, int num_experts, int64_t dim, int topk, int score_func,
                       int renorm, float renorm_eps, float route_scale, float* top_scores,
                       int64_t* top_indices, void* logits_out, void* workspace, size_t workspace_bytes,
                       void* stream) {
  const char* fn = "ttamd_router_fused";
  REQUIRE(num_tokens >= 0 && num_tokens <= (1 << 24), "%s: num_tokens out of range", fn);
  REQUIRE(num_experts >= 1 && num_experts <= 256, "%s: num_experts must be in [1, 256]", fn);
  REQUIRE(topk >= 1 && topk <= 16 && topk <= num_experts, "%s: topk must be in [1, min(16, E)]",
          fn);
  REQUIRE(score_func == TTAMD_SCORE_SOFTMAX || score_func == TTAMD_SCORE_SIGMOID,
          "%s: unknown score_func %d", fn, score_func);
  REQUIRE(dim >= 64 && dim % 64 == 0 && dim <= (1 << 20), "%s: dim must be a positive multiple of 64",
          fn);
  REQUIRE((int64_t)num_experts * dim * 2 < kI32Max && 128 * dim * 2 < kI32Max,
          "%s: router weight too large", fn);
  if (num_tokens == 0) return TTAMD_OK;
  REQUIRE(x && w_router && top_scores && top_indices, "%s: null pointer argument", fn);
  REQUIRE(aligned16(x) && aligned16(w_router), "%s: x and w_router must be 16-byte aligned", fn);
  TRY(check_ws(fn, workspace, workspace_bytes, ttamd::router_workspace_bytes(num_tokens, num_experts, dim)));
  return check_hip(ttamd::launch_router_fused(x, w_router, expert_bias, (int)num_tokens, num_experts,
                                              (int)dim, topk, score_func, renorm, renorm_eps,
                                              route_scale, top_scores, top_indices, logits_out, workspace,
                                              (hipStream_t)stream),
                   fn);
}

size_t ttamd_route_workspace_bytes(int64_t num_flat, int num_experts) {
  if (num_flat < 0 || num_experts < 1) return 0;
  return ttamd::route_workspace_bytes(num_flat, num_experts);
}

static int route_arg_checks(const char* fn, const void* labels, int64_t M, int E, const float* scores,
                            const int32_t* sorted, const float* sorted_scores) {
  REQUIRE(M >= 0 && M <= (1 << 28), "%s: number of labels out of range (%lld)", fn,
          (long long)M);
  REQUIRE(E >= 1 && E <= 1024, "%s: num_experts must be in [1, 1024] (got %d)", fn, E);
  if (M > 0) REQUIRE(labels && sorted, "%s: null pointer argument", fn);
  REQUIRE((scores == nullptr) == (sorted_scores == nullptr),
          "%s: scores and sorted_scores must be given together", fn);
  return TTAMD_OK;
}

static int route_checks(const char* fn, const void* labels, int64_t M, int E, const float* scores,
                        const int32_t* sorted, const float* sorted_scores, const void* ws,
                        size_t ws_bytes) {
  TRY(route_arg_checks(fn, labels, M, E, scores, sorted, sorted_scores));
  TRY(check_ws(fn, ws, ws_bytes, ttamd::route_workspace_bytes(M, E)));
  return TTAMD_OK;
}

int ttamd_moe_route(const void* labels, int labels_are_int64, int64_t num_flat, int num_experts,
                    const float* scores, int32_t* counts, int32_t* offsets,
                    int32_t* sorted_indices, int32_t* inverse, float* sorted_scores,
                    void* workspace, size_t workspace_bytes, void* stream) {
  const char* fn = "ttamd_moe_route";
  TRY(route_checks(fn, labels, num_flat, num_experts, scores, sorted_indices, sorted_scores,
                   workspace, workspace_bytes));
  return check_hip(ttamd::launch_route(labels, labels_are_int64 != 0, (int)num_flat, num_experts,
                                       scores, counts, offsets, sorted_indices, inverse,
                                       sorted_scores, workspace, (hipStream_t)stream),
                   fn);
}

int ttamd_moe_route_noalloc(const void* labels, int labels_are_int64, int64_t num_flat,
                            int num_experts, const float* scores, int32_t* counts, int32_t* offsets,
                            int32_t* sorted_indices, int32_t* inverse, float* sorted_scores,
                            void* stream) {
  const char* fn = "ttamd_moe_route_noalloc";
  TRY(route_arg_checks(fn, labels, num_flat, num_experts, scores, sorted_indices, sorted_scores));
  const size_t need = ttamd::route_hist_bytes(num_flat, num_experts);
  REQUIRE(need <= ttamd::route_scratch_bytes(),
          "%s: %lld labels over %d experts need %zu bytes of route workspace, more than the %zu bytes "
          "the library holds per device; use ttamd_moe_route with a caller workspace",
          fn, (long long)num_flat, num_experts, need, ttamd::route_scratch_bytes());
  void* ws = nullptr;
  TRY(check_hip(ttamd::route_scratch((hipStream_t)stream, &ws), fn));
  return check_hip(ttamd::launch_route(labels, labels_are_int64 != 0, (int)num_flat, num_experts,
                                       scores, counts, offsets, sorted_indices, inverse,
                                       sorted_scores, ws, (hipStream_t)stream),
                   fn);
}

size_t ttamd_router_backward_workspace_bytes(int64_t num_tokens, int num_experts, int64_t dim) {
  if (num_tokens < 0 || num_experts < 1 || dim < 1) return 0;
  return ttamd::router_backward_workspace_bytes(num_tokens, num_experts, dim);
}

int ttamd_router_backward(const float* grad_top_scores, const int64_t* top_indices, const void* logits,
                          const void* x, const void* w_router, int64_t num_tokens, int num_experts, int64_t dim,
                          int topk, int score_func, int renorm, float renorm_eps, float route_scale, void* grad_x,
                          void* grad_w_router, int grad_w_is_fp32, void* workspace, size_t workspace_bytes,
                          void* stream) {
  const char* fn = "ttamd_router_backward";
  REQUIRE(num_tokens >= 0 && num_tokens <= (1 << 24), "%s: num_tokens out of range", fn);
  REQUIRE(num_experts >= 1 && num_experts <= 256, "%s: num_experts must be in [1, 256]", fn);
  REQUIRE(topk >= 1 && topk <= 16 && topk <= num_experts, "%s: topk must be in [1, min(16, E)]", fn);
  REQUIRE(score_func == TTAMD_SCORE_SOFTMAX || score_func == TTAMD_SCORE_SIGMOID,
          "%s: unknown score_func %d", fn, score_func);
  REQUIRE(dim >= 128 && dim % 128 == 0 && dim <= (1 << 20), "%s: dim must be a positive multiple of 128", fn);
  if (num_tokens == 0) return TTAMD_OK;
  REQUIRE(grad_top_scores && top_indices && logits && w_router, "%s: null pointer argument", fn);
  REQUIRE(grad_w_router == nullptr || x != nullptr, "%s: the weight gradient needs x", fn);
  REQUIRE(aligned16(w_router), "%s: w_router must be 16-byte aligned", fn);
  if (x) TRY(check_rows(fn, "x", x, num_tokens, dim));
  if (grad_x) TRY(check_rows(fn, "grad_x", grad_x, num_tokens, dim));
  if (grad_w_router) REQUIRE(aligned16(grad_w_router), "%s: grad_w_router must be 16-byte aligned", fn);
  REQUIRE(num_tokens * dim * 2 <= (int64_t)0xffffffffLL, "%s: x must stay below 4 GiB", fn);
  TRY(check_ws(fn, workspace, workspace_bytes, ttamd::router_backward_workspace_bytes(num_tokens, num_experts, dim)));
  return check_hip(ttamd::launch_router_backward(grad_top_scores, top_indices, logits, x, w_router, (int)num_tokens,
                                                 num_experts, (int)dim, topk, score_func, renorm, renorm_eps,
                                                 route_scale, grad_x, grad_w_router, grad_w_is_fp32 != 0, workspace,
                                                 (hipStream_t)stream),
                   fn);
}

static size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

size_t ttamd_router_route_workspace_bytes(int64_t num_tokens, int num_experts, int64_t dim, int topk) {
  if (num_tokens < 0 || num_experts < 1 || dim < 64 || topk < 1) return 0;
  return align256(ttamd::router_workspace_bytes(num_tokens, num_experts, dim)) +
         ttamd::route_workspace_bytes(num_tokens * topk, num_experts);
}

int ttamd_router_route(const void* x, const void* w_router, const float* expert_bias, int64_t num_tokens,
                       int num_experts, int64_t dim, int topk, int score_func, int renorm, float renorm_eps,
                       float route_scale, float* top_scores, int64_t* top_indices, int32_t* counts,
                       int32_t* offsets, int32_t* sorted_indices, int32_t* inverse, float* sorted_scores,
                       float* tokens_per_expert, void* gemm_plan, size_t gemm_plan_bytes, void* workspace,
                       size_t workspace_bytes, void* stream) {
  const char* fn = "ttamd_router_route";
  REQUIRE(num_tokens >= 0 && num_tokens <= (1 << 24), "%s: num_tokens out of range", fn);
  REQUIRE(num_experts >= 1 && num_experts <= 256, "%s: num_experts must be in [1, 256]", fn);
  REQUIRE(topk >= 1 && topk <= 16 && topk <= num_experts, "%s: topk must be in [1, min(16, E)]", fn);
  REQUIRE(score_func == TTAMD_SCORE_SOFTMAX || score_func == TTAMD_SCORE_SIGMOID,
          "%s: unknown score_func %d", fn, score_func);
  REQUIRE(dim >= 64 && dim % 64 == 0 && dim <= (1 << 20), "%s: dim must be a positive multiple of 64", fn);
  REQUIRE((int64_t)num_experts * dim * 2 < kI32Max && 128 * dim * 2 < kI32Max, "%s: router weight too large",
          fn);
  const int64_t M = num_tokens * topk;
  REQUIRE(M <= (1 << 28), "%s: too many routed rows", fn);
  REQUIRE(num_tokens == 0 || (x && w_router && top_scores && top_indices && sorted_indices),
          "%s: null pointer argument", fn);
  REQUIRE(w_router != nullptr, "%s: w_router is null", fn);
  REQUIRE(aligned16(x) && aligned16(w_router), "%s: x and w_router must be 16-byte aligned", fn);
  // the tile table is built from the offsets, the accumulator from the
  // counts (on every scan path), so both buffers must be given with them
  REQUIRE((gemm_plan == nullptr && tokens_per_expert == nullptr) || (counts && offsets),
          "%s: gemm_plan and tokens_per_expert need the counts and offsets buffers", fn);
  const size_t rbytes = align256(ttamd::router_workspace_bytes(num_tokens, num_experts, dim));
  TRY(check_ws(fn, workspace, workspace_bytes, ttamd_router_route_workspace_bytes(num_tokens, num_experts, dim, topk)));
  if (gemm_plan) {
    REQUIRE(aligned16(gemm_plan), "%s: gemm_plan must be 16-byte aligned", fn);
    REQUIRE(gemm_plan_bytes >= ttamd::gemm_plan_bytes(M, num_experts),
            "%s: gemm_plan too small (%zu bytes, need %zu)", fn, gemm_plan_bytes,
            ttamd::gemm_plan_bytes(M, num_experts));
  }
  hipStream_t s = (hipStream_t)stream;
  int* hist = (int*)((char*)workspace + rbytes);
  TRY(check_hip(ttamd::launch_router_hist(x, w_router, expert_bias, (int)num_tokens, num_experts, (int)dim, topk,
                                          score_func, renorm, renorm_eps, route_scale, top_scores, top_indices,
                                          nullptr, workspace, hist, s),
                fn));
  return check_hip(ttamd::launch_route_from_hist(top_indices, true, (int)M, num_experts, top_scores, counts, offsets,
                                                 sorted_indices, inverse, sorted_scores, hist, tokens_per_expert,
                                                 gemm_plan, ttamd::gemm_fwd_tile_rows(), s),
                   fn);
}

size_t ttamd_moe_experts_forward_workspace_bytes(int64_t num_tokens, int64_t dim, int64_t hidden,
                                                 int num_experts, int topk, int score_before_experts) {
  if (num_tokens < 0 || dim < 1 || hidden < 1 || num_experts < 1 || topk < 1) return 0;
  return ttamd::moe_experts_forward_workspace_bytes(num_tokens, dim, hidden, num_experts, topk,
                                                    score_before_experts != 0 || dim < 128);
}

int ttamd_moe_experts_forward(const void* tokens, int64_t num_tokens, int64_t dim, int64_t hidden,
                              int num_experts, int topk, const int32_t* sorted_indices, const int32_t* offs,
                              const float* sorted_scores, int score_before_experts, float swiglu_limit,
                              const void* w13, const void* w2, void* out, void* gemm_plan,
                              size_t gemm_plan_bytes, void* workspace, size_t workspace_bytes, void* stream) {
  const char* fn = "ttamd_moe_experts_forward";
  REQUIRE(topk >= 1 && topk <= 64, "%s: topk must be in [1, 64]", fn);
  REQUIRE(num_tokens >= 0 && num_tokens * topk <= (1 << 28), "%s: num_tokens out of range", fn);
  const int64_t M = num_tokens * topk;
  TRY(check_gemm_common(fn, offs, M, num_experts));
  TRY(check_dim(fn, "dim", dim, 128));
  TRY(check_dim(fn, "hidden", hidden, 64));
  REQUIRE(std::isnan(swiglu_limit) || swiglu_limit >= 0.f, "%s: swiglu_limit must be NaN (no clamp) or >= 0",
          fn);
  REQUIRE(w13 && aligned16(w13) && w2 && aligned16(w2), "%s: w13 and w2 must be non-null and 16-byte aligned",
          fn);
  REQUIRE(num_tokens * dim * 2 <= (int64_t)0xffffffffLL, "%s: tokens must stay below 4 GiB", fn);
  TRY(check_rows(fn, "tokens", tokens, num_tokens, dim));
  TRY(check_rows(fn, "out", out, num_tokens, dim));
  REQUIRE(M * (dim / 8) <= (int64_t(1) << 30) && M * (hidden / 8) <= (int64_t(1) << 30),
          "%s: too many routed elements (%lld rows)", fn, (long long)M);
  if (M > 0) REQUIRE(sorted_indices != nullptr, "%s: sorted_indices is null", fn);
  REQUIRE(score_before_experts == 0 || sorted_scores != nullptr || M == 0,
          "%s: score_before_experts needs sorted_scores", fn);
  if (gemm_plan) {
    REQUIRE(aligned16(gemm_plan), "%s: gemm_plan must be 16-byte aligned", fn);
    REQUIRE(gemm_plan_bytes >= ttamd::gemm_plan_bytes(M, num_experts),
            "%s: gemm_plan too small (%zu bytes, need %zu)", fn, gemm_plan_bytes,
            ttamd::gemm_plan_bytes(M, num_experts));
  }
  TRY(check_ws(fn, workspace, workspace_bytes,
               ttamd_moe_experts_forward_workspace_bytes(num_tokens, dim, hidden, num_experts, topk,
                                                         score_before_experts)));
  if (M == 0) return TTAMD_OK;
  return check_hip(ttamd::launch_moe_experts_forward(tokens, (int)num_tokens, (int)dim, (int)hidden, num_experts,
                                                     topk, sorted_indices, offs, sorted_scores,
                                                     score_before_experts != 0, swiglu_limit, w13, w2, out,
                                                     gemm_plan, workspace, (hipStream_t)stream),
                   fn);
}

int ttamd_moe_gather_rows(const void* in, const int32_t* src_index, const float* row_scale,
                          int64_t num_in_rows, int64_t num_out_rows, int64_t hidden, int topk,
                          void* out, void* stream) {
  const char* fn = "ttamd_moe_gather_rows";
  TRY(check_hidden(fn, hidden));
  REQUIRE(topk >= 1, "%s: topk must be >= 1", fn);
  REQUIRE(num_in_rows >= 0 && num_out_rows >= 0, "%s: negative row count", fn);
  REQUIRE(num_out_rows == 0 || num_in_rows > 0, "%s: no input rows to gather from", fn);
  REQUIRE(num_in_rows * topk <= kI32Max, "%s: too many rows", fn);
  TRY(check_rows(fn, "in", in, num_in_rows, hidden));
  TRY(check_rows(fn, "out", out, num_out_rows, hidden));
  if (num_out_rows > 0) REQUIRE(src_index != nullptr, "%s: src_index is null", fn);
  return check_hip(ttamd::launch_gather_rows(in, src_index, row_scale, false, (int)num_in_rows,
                                             (int)(num_in_rows * topk), (int)num_out_rows,
                                             (int)hidden, topk, out, (hipStream_t)stream),
                   fn);
}

int ttamd_moe_token_permute(const void* tokens, const void* labels, int labels_are_int64,
                            int64_t num_tokens, int64_t hidden, int topk, int num_experts,
                            void* permuted, int32_t* sorted_indices, int32_t* counts,
                            void* workspace, size_t workspace_bytes, void* stream) {
  const char* fn = "ttamd_moe_token_permute";
  TRY(check_hidden(fn, hidden));
  REQUIRE(topk >= 1, "%s: topk must be >= 1", fn);
  REQUIRE(num_tokens >= 0, "%s: negative num_tokens", fn);
  const int64_t M = num_tokens * topk;
  TRY(route_checks(fn, labels, M, num_experts, nullptr, sorted_indices, nullptr, workspace,
                   workspace_bytes));
  TRY(check_rows(fn, "tokens", tokens, num_tokens, hidden));
  TRY(check_rows(fn, "permuted", permuted, M, hidden));
  hipStream_t s = (hipStream_t)stream;
  TRY(check_hip(ttamd::launch_route(labels, labels_are_int64 != 0, (int)M, num_experts, nullptr,
                                    counts, nullptr, sorted_indices, nullptr, nullptr, workspace,
                                    s),
                fn));
  return check_hip(ttamd::launch_gather_rows(tokens, sorted_indices, nullptr, false,
                                             (int)num_tokens, (int)M, (int)M, (int)hidden, topk,
                                             permuted, s),
                   fn);
}

size_t ttamd_unpermute_workspace_bytes(int64_t num_tokens, int topk) {
  if (num_tokens < 0 || topk < 1) return 0;
  return (size_t)(num_tokens * topk) * sizeof(int32_t) + 256;
}

int ttamd_moe_token_unpermute(const void* permuted, const int32_t* sorted_indices,
                              const float* probs, int64_t num_tokens, int64_t hidden, int topk,
                              void* out, void* workspace, size_t workspace_bytes, void* stream) {
  const char* fn = "ttamd_moe_token_unpermute";
  TRY(check_hidden(fn, hidden));
  REQUIRE(topk >= 1, "%s: topk must be >= 1", fn);
  REQUIRE(num_tokens >= 0, "%s: negative num_tokens", fn);
  const int64_t M = num_tokens * topk;
  TRY(check_rows(fn, "permuted", permuted, M, hidden));
  TRY(check_rows(fn, "out", out, num_tokens, hidden));
  if (M > 0) REQUIRE(sorted_indices != nullptr, "%s: sorted_indices is null", fn);
  TRY(check_ws(fn, workspace, workspace_bytes, ttamd_unpermute_workspace_bytes(num_tokens, topk)));
  hipStream_t s = (hipStream_t)stream;
  int32_t* inv = (int32_t*)workspace;
  TRY(check_hip(ttamd::launch_invert_perm(sorted_indices, (int)M, inv, s), fn));
  return check_hip(ttamd::launch_combine(permuted, inv, probs, (int)num_tokens, topk, (int)hidden,
                                         out, s),
                   fn);
}

int ttamd_moe_combine(const void* permuted, const int32_t* inverse, const float* probs,
                      int64_t num_tokens, int64_t hidden, int topk, void* out, void* stream) {
  const char* fn = "ttamd_moe_combine";
  TRY(check_hidden(fn, hidden));
  REQUIRE(topk >= 1, "%s: topk must be >= 1", fn);
  REQUIRE(num_tokens >= 0, "%s: negative num_tokens", fn);
  const int64_t M = num_tokens * topk;
  TRY(check_rows(fn, "permuted", permuted, M, hidden));
  TRY(check_rows(fn, "out", out, num_tokens, hidden));
  if (M > 0) REQUIRE(inverse != nullptr, "%s: inverse is null", fn);
  return check_hip(ttamd::launch_combine(permuted, inverse, probs, (int)num_tokens, topk,
                                         (int)hidden, out, (hipStream_t)stream),
                   fn);
}

int ttamd_moe_dispatch_rows(const void* tokens, const int32_t* inverse, const float* scores,
                            int64_t num_tokens, int64_t hidden, int topk, void* out, void* stream) {
  const char* fn = "ttamd_moe_dispatch_rows";
  TRY(check_hidden(fn, hidden));
  REQUIRE(topk >= 1 && topk <= 64, "%s: topk must be in [1, 64]", fn);
  REQUIRE(num_tokens >= 0 && num_tokens * topk <= kI32Max, "%s: num_tokens out of range", fn);
  TRY(check_rows(fn, "tokens", tokens, num_tokens, hidden));
  TRY(check_rows(fn, "out", out, num_tokens * topk, hidden));
  if (num_tokens > 0) REQUIRE(inverse != nullptr, "%s: inverse is null", fn);
  return check_hip(ttamd::launch_dispatch_rows(tokens, inverse, scores, (int)num_tokens, topk, (int)hidden,
                                               out, (hipStream_t)stream),
                   fn);
}

int ttamd_moe_sum_topk(const void* in, int64_t num_tokens, int64_t hidden, int topk, void* out,
                       void* stream) {
  const char* fn = "ttamd_moe_sum_topk";
  TRY(check_hidden(fn, hidden));
  REQUIRE(topk >= 1, "%s: topk must be >= 1", fn);
  REQUIRE(num_tokens >= 0, "%s: negative num_tokens", fn);
  TRY(check_rows(fn, "in", in, num_tokens * topk, hidden));
  TRY(check_rows(fn, "out", out, num_tokens, hidden));
  return check_hip(ttamd::launch_combine(in, nullptr, nullptr, (int)num_tokens, topk, (int)hidden,
                                         out, (hipStream_t)stream),
                   fn);
}

int ttamd_moe_token_unpermute_grad(const void* grad_out, const int32_t* sorted_indices,
                                   const float* probs, const void* permuted, int64_t num_tokens,
                                   int64_t hidden, int topk, void* grad_permuted,
                                   float* grad_probs, void* stream) {
  const char* fn = "ttamd_moe_token_unpermute_grad";
  TRY(check_hidden(fn, hidden));
  REQUIRE(topk >= 1, "%s: topk must be >= 1", fn);
  REQUIRE(num_tokens >= 0, "%s: negative num_tokens", fn);
  const int64_t M = num_tokens * topk;
  TRY(check_rows(fn, "grad_out", grad_out, num_tokens, hidden));
  TRY(check_rows(fn, "grad_permuted", grad_permuted, M, hidden));
  if (M > 0) REQUIRE(sorted_indices != nullptr, "%s: sorted_indices is null", fn);
  if (grad_probs) {
    REQUIRE(probs != nullptr && permuted != nullptr,
            "%s: grad_probs needs probs and permuted", fn);
    TRY(check_rows(fn, "permuted", permuted, M, hidden));
  }
  hipStream_t s = (hipStream_t)stream;
  if (M == 0) return TTAMD_OK;
  TRY(check_hip(ttamd::launch_gather_rows(grad_out, sorted_indices, probs, true, (int)num_tokens,
                                          (int)M, (int)M, (int)hidden, topk, grad_permuted, s),
                fn));
  if (grad_probs)
    TRY(check_hip(ttamd::launch_rowdot(permuted, grad_out, sorted_indices, topk, true, (int)M,
                                       (int)num_tokens, (int)M, (int)hidden, grad_probs, s),
                  fn));
  return TTAMD_OK;
}

int ttamd_moe_rowdot(const void* a, const void* b, const int32_t* b_index, int b_div,
                     int out_by_index, int64_t num_rows, int64_t num_b_rows, int64_t hidden,
                     float* out, void* stream) {
  const char* fn = "ttamd_moe_rowdot";
  TRY(check_hidden(fn, hidden));
  REQUIRE(b_div >= 1, "%s: b_div must be >= 1", fn);
  REQUIRE(num_rows >= 0 && num_b_rows >= 0, "%s: negative row count", fn);
  REQUIRE(num_rows == 0 || num_b_rows > 0, "%s: b has no rows", fn);
  TRY(check_rows(fn, "a", a, num_rows, hidden));
  TRY(check_rows(fn, "b", b, num_b_rows, hidden));
  if (num_rows > 0) REQUIRE(out != nullptr, "%s: out is null", fn);
  REQUIRE(!out_by_index || b_index != nullptr, "%s: out_by_index needs b_index", fn);
  REQUIRE(num_b_rows * (int64_t)b_div <= kI32Max, "%s: too many rows", fn);
  return check_hip(ttamd::launch_rowdot(a, b, b_index, b_div, out_by_index != 0, (int)num_rows,
                                        (int)num_b_rows, (int)num_rows, (int)hidden, out,
                                        (hipStream_t)stream),
                   fn);
}

int ttamd_moe_group_labels(const int32_t* counts_group, int num_groups, int num_local_experts,
                           int64_t num_rows, int32_t* labels, void* stream) {
  const char* fn = "ttamd_moe_group_labels";
  REQUIRE(num_groups >= 1 && num_groups <= 8192, "%s: num_groups must be in [1, 8192]", fn);
  REQUIRE(num_local_experts >= 1 && num_groups % num_local_experts == 0,
          "%s: num_groups must be a multiple of num_local_experts", fn);
  REQUIRE(num_rows >= 0 && num_rows <= kI32Max, "%s: num_rows out of range", fn);
  REQUIRE(counts_group != nullptr, "%s: counts_group is null", fn);
  if (num_rows > 0) REQUIRE(labels != nullptr, "%s: labels is null", fn);
  return check_hip(ttamd::launch_group_labels(counts_group, num_groups, num_local_experts,
                                              (int)num_rows, labels, (hipStream_t)stream),
                   fn);
}

int ttamd_probe_next_gemm(void* start_event, void* end_event) {
  REQUIRE((start_event == nullptr) == (end_event == nullptr),
          "ttamd_probe_next_gemm: give both events or neither");
  ttamd::gemm_probe_arm((hipEvent_t)start_event, (hipEvent_t)end_event);
  return 0;
}

int ttamd_probe_launches(void* const* events, int num_launches) {
  const char* fn = "ttamd_probe_launches";
  REQUIRE(num_launches >= 0 && num_launches <= ttamd::kProbeMaxChain, "%s: num_launches must be in [0, %d]", fn,
          ttamd::kProbeMaxChain);
  REQUIRE(num_launches == 0 || events != nullptr, "%s: events is null", fn);
  for (int i = 0; i < num_launches; ++i)
    REQUIRE((events[2 * i] == nullptr) == (events[2 * i + 1] == nullptr),
            "%s: events[%d] and events[%d] must both be given or both be NULL", fn, 2 * i, 2 * i + 1);
  ttamd::probe_chain_arm((const hipEvent_t*)events, num_launches);
  return 0;
}

size_t ttamd_gemm_workspace_bytes(int64_t num_rows, int num_experts) {
  if (num_rows < 0 || num_experts < 1) return 0;
  return ttamd::gemm_workspace_bytes(num_rows, num_experts);
}

size_t ttamd_gemm_plan_bytes(int64_t num_rows, int num_experts) {
  if (num_rows < 0 || num_experts < 1) return 0;
  return ttamd::gemm_plan_bytes(num_rows, num_experts);
}

int ttamd_grouped_mm(const void* x, const void* w, const int32_t* offs, int64_t num_rows,
                     int num_experts, int64_t n, int64_t k, void* out, void* workspace,
                     size_t workspace_bytes, void* stream) {
  const char* fn = "ttamd_grouped_mm";
  TRY(check_gemm_common(fn, offs, num_rows, num_experts));
  TRY(check_dim(fn, "n", n, 128));
  TRY(check_dim(fn, "k", k, 64));
  REQUIRE(w && aligned16(w), "%s: w must be non-null and 16-byte aligned", fn);
  TRY(check_rows(fn, "x", x, num_rows, k));
  TRY(check_rows(fn, "out", out, num_rows, n));
  TRY(check_ws(fn, workspace, workspace_bytes, ttamd::gemm_workspace_bytes(num_rows, num_experts)));
  if (num_rows == 0) return TTAMD_OK;
  return check_hip(ttamd::launch_grouped_mm(x, w, offs, (int)num_rows, num_experts, (int)n, (int)k,
                                            out, workspace, (hipStream_t)stream),
                   fn);
}

int ttamd_grouped_mm_swiglu(const void* x, const void* w13, const int32_t* offs,
                            int64_t num_rows, int num_experts, int64_t hidden, int64_t dim,
                            float swiglu_limit, void* a_out, void* h_out, void* workspace,
                            size_t workspace_bytes, void* stream) {
  const char* fn = "ttamd_grouped_mm_swiglu";
  TRY(check_gemm_common(fn, offs, num_rows, num_experts));
  TRY(check_dim(fn, "hidden", hidden, 64));
  TRY(check_dim(fn, "dim", dim, 64));
  REQUIRE(std::isnan(swiglu_limit) || swiglu_limit >= 0.f,
          "%s: swiglu_limit must be NaN (no clamp) or >= 0", fn);
  REQUIRE(w13 && aligned16(w13), "%s: w13 must be non-null and 16-byte aligned", fn);
  TRY(check_rows(fn, "x", x, num_rows, dim));
  TRY(check_rows(fn, "a_out", a_out, num_rows, hidden));
  if (h_out) TRY(check_rows(fn, "h_out", h_out, num_rows, 2 * hidden));
  TRY(check_ws(fn, workspace, workspace_bytes, ttamd::gemm_workspace_bytes(num_rows, num_experts)));
  if (num_rows == 0) return TTAMD_OK;
  return check_hip(ttamd::launch_grouped_mm_swiglu(x, w13, offs, (int)num_rows, num_experts,
                                                   (int)hidden, (int)dim, swiglu_limit, a_out,
                                                   h_out, workspace, (hipStream_t)stream),
                   fn);
}

int ttamd_grouped_mm_swiglu_gather(const void* tokens, int64_t num_tokens, const int32_t* src_index,
                                   int src_div, const void* w13, const int32_t* offs, int64_t num_rows,
                                   int num_experts, int64_t hidden, int64_t dim, float swiglu_limit,
                                   void* a_out, void* h_out, void* workspace, size_t workspace_bytes,
                                   void* stream) {
  const char* fn = "ttamd_grouped_mm_swiglu_gather";
  TRY(check_gemm_common(fn, offs, num_rows, num_experts));
  TRY(check_dim(fn, "hidden", hidden, 64));
  TRY(check_dim(fn, "dim", dim, 64));
  REQUIRE(dim >= 128, "%s: dim must be >= 128 (got %lld)", fn, (long long)dim);
  REQUIRE(w13 && aligned16(w13), "%s: w13 must be non-null and 16-byte aligned", fn);
  REQUIRE(src_div >= 1, "%s: src_div must be >= 1", fn);
  REQUIRE(num_tokens >= 1 || num_rows == 0, "%s: no token rows", fn);
  REQUIRE(num_tokens * dim * 2 <= (int64_t)0xffffffffLL, "%s: tokens must stay below 4 GiB", fn);
  TRY(check_rows(fn, "tokens", tokens, num_tokens, dim));
  if (num_rows > 0) REQUIRE(src_index != nullptr, "%s: src_index is null", fn);
  TRY(check_rows(fn, "a_out", a_out, num_rows, hidden));
  if (h_out) TRY(check_rows(fn, "h_out", h_out, num_rows, 2 * hidden));
  TRY(check_ws(fn, workspace, workspace_bytes, ttamd::gemm_workspace_bytes(num_rows, num_experts)));
  if (num_rows == 0) return TTAMD_OK;
  return check_hip(ttamd::launch_grouped_mm_swiglu_gather(tokens, (int)num_tokens, src_index, src_div, w13,
                                                          offs, (int)num_rows, num_experts, (int)hidden,
                                                          (int)dim, swiglu_limit, a_out, h_out, workspace,
                                                          (hipStream_t)stream),
                   fn);
}

int ttamd_grouped_mm_unpermute(const void* a, const void* w2, const int32_t* offs,
                               int64_t num_rows, int num_experts, int64_t dim, int64_t hidden,
                               const float* row_scale, const int32_t* dest, int64_t num_dest_rows,
                               void* out, void* workspace, size_t workspace_bytes, void* stream) {
  const char* fn = "ttamd_grouped_mm_unpermute";
  TRY(check_gemm_common(fn, offs, num_rows, num_experts));
  TRY(check_dim(fn, "dim", dim, 128));
  TRY(check_dim(fn, "hidden", hidden, 64));
  REQUIRE(w2 && aligned16(w2), "%s: w2 must be non-null and 16-byte aligned", fn);
  TRY(check_rows(fn, "a", a, num_rows, hidden));
  if (dest == nullptr)
    REQUIRE(num_dest_rows >= num_rows, "%s: out needs num_rows rows when dest is null", fn);
  REQUIRE(num_dest_rows >= 0, "%s: negative num_dest_rows", fn);
  REQUIRE(num_rows == 0 || num_dest_rows > 0, "%s: out has no rows", fn);
  TRY(check_rows(fn, "out", out, num_dest_rows, dim));
  TRY(check_ws(fn, workspace, workspace_bytes, ttamd::gemm_workspace_bytes(num_rows, num_experts)));
  if (num_rows == 0) return TTAMD_OK;
  return check_hip(ttamd::launch_grouped_mm_unpermute(a, w2, offs, (int)num_rows, num_experts,
                                                      (int)dim, (int)hidden, row_scale, dest,
                                                      (int)num_dest_rows, out, workspace,
                                                      (hipStream_t)stream),
                   fn);
}

int ttamd_shared_expert_add(const void* x, int64_t num_tokens, int64_t dim, int64_t hidden,
                            const void* w13_shared, const void* w2_shared, const float* gate_logits,
                            float swiglu_limit, void* a_scratch, void* out, void* workspace,
                            size_t workspace_bytes, void* stream) {
  const char* fn = "ttamd_shared_expert_add";
  REQUIRE(num_tokens >= 0 && num_tokens <= (1 << 28), "%s: num_tokens out of range", fn);
  TRY(check_dim(fn, "dim", dim, 128));
  TRY(check_dim(fn, "hidden", hidden, 64));
  REQUIRE(w13_shared && aligned16(w13_shared) && w2_shared && aligned16(w2_shared),
          "%s: shared weights must be non-null and 16-byte aligned", fn);
  TRY(check_rows(fn, "x", x, num_tokens, dim));
  TRY(check_rows(fn, "a_scratch", a_scratch, num_tokens, hidden));
  TRY(check_rows(fn, "out", out, num_tokens, dim));
  if (num_tokens > 0)
    REQUIRE(a_scratch != out && a_scratch != x, "%s: a_scratch must not alias x or out", fn);
  REQUIRE(std::isnan(swiglu_limit) || swiglu_limit >= 0.f,
          "%s: swiglu_limit must be NaN (no clamp) or >= 0", fn);
  TRY(check_ws(fn, workspace, workspace_bytes, ttamd::gemm_workspace_bytes(num_tokens, 1)));
  if (num_tokens == 0) return TTAMD_OK;
  return check_hip(ttamd::launch_shared_expert_add(x, (int)num_tokens, (int)dim, (int)hidden, w13_shared,
                                                   w2_shared, gate_logits, swiglu_limit, a_scratch, out, workspace,
                                                   (hipStream_t)stream),
                   fn);
}

int ttamd_grouped_mm_dgrad(const void* dy, const void* w, const int32_t* offs, int64_t num_rows,
                           int num_experts, int64_t n, int64_t k, void* dx, void* workspace,
                           size_t workspace_bytes, void* stream) {
  const char* fn = "ttamd_grouped_mm_dgrad";
  TRY(check_gemm_common(fn, offs, num_rows, num_experts));
  TRY(check_dim(fn, "n", n, 64));
  TRY(check_dim(fn, "k", k, 128));
  REQUIRE(w && aligned16(w), "%s: w must be non-null and 16-byte aligned", fn);
  TRY(check_rows(fn, "dy", dy, num_rows, n));
  TRY(check_rows(fn, "dx", dx, num_rows, k));
  TRY(check_ws(fn, workspace, workspace_bytes, ttamd::gemm_workspace_bytes(num_rows, num_experts)));
  if (num_rows == 0) return TTAMD_OK;
  return check_hip(ttamd::launch_grouped_mm_dgrad(dy, w, offs, (int)num_rows, num_experts, (int)n,
                                                  (int)k, dx, workspace, (hipStream_t)stream),
                   fn);
}

int ttamd_grouped_mm_dgrad_swiglu(const void* dy, const void* w2, const void* h,
                                  const int32_t* offs, int64_t num_rows, int num_experts,
                                  int64_t dim, int64_t hidden, float swiglu_limit, void* dh,
                                  void* a_out, void* workspace, size_t workspace_bytes,
                                  void* stream) {
  const char* fn = "ttamd_grouped_mm_dgrad_swiglu";
  TRY(check_gemm_common(fn, offs, num_rows, num_experts));
  TRY(check_dim(fn, "dim", dim, 64));
  TRY(check_dim(fn, "hidden", hidden, 128));
  REQUIRE(std::isnan(swiglu_limit) || swiglu_limit >= 0.f,
          "%s: swiglu_limit must be NaN (no clamp) or >= 0", fn);
  REQUIRE(w2 && aligned16(w2), "%s: w2 must be non-null and 16-byte aligned", fn);
  TRY(check_rows(fn, "dy", dy, num_rows, dim));
  TRY(check_rows(fn, "h", h, num_rows, 2 * hidden));
  TRY(check_rows(fn, "dh", dh, num_rows, 2 * hidden));
  if (a_out) TRY(check_rows(fn, "a_out", a_out, num_rows, hidden));
  TRY(check_ws(fn, workspace, workspace_bytes, ttamd::gemm_workspace_bytes(num_rows, num_experts)));
  if (num_rows == 0) return TTAMD_OK;
  return check_hip(ttamd::launch_grouped_mm_dgrad_swiglu(dy, w2, h, offs, (int)num_rows,
                                                         num_experts, (int)dim, (int)hidden,
                                                         swiglu_limit, dh, a_out, workspace,
                                                         (hipStream_t)stream),
                   fn);
}

int ttamd_grouped_mm_wgrad(const void* dy, const void* x, const int32_t* offs, int64_t num_rows,
                           int num_experts, int64_t n, int64_t k, void* dw, int dw_is_fp32,
                           void* workspace, size_t workspace_bytes, void* stream) {
  const char* fn = "ttamd_grouped_mm_wgrad";
  TRY(check_gemm_common(fn, offs, num_rows, num_experts));
  if (workspace != nullptr)
    TRY(check_ws(fn, workspace, workspace_bytes, ttamd::gemm_workspace_bytes(num_rows, num_experts)));
  TRY(check_dim(fn, "n", n, 128));
  TRY(check_dim(fn, "k", k, 128));
  TRY(check_rows(fn, "dy", dy, num_rows, n));
  TRY(check_rows(fn, "x", x, num_rows, k));
  REQUIRE(dw && aligned16(dw), "%s: dw must be non-null and 16-byte aligned", fn);
  REQUIRE((int64_t)num_experts * n * k <= (int64_t)1 << 40, "%s: dw too large", fn);
  REQUIRE((int64_t)num_experts * (n / 128) * (k / 128) <= kI32Max, "%s: too many tiles", fn);
  REQUIRE(num_rows * n * 2 <= (int64_t)0xffffffffLL && num_rows * k * 2 <= (int64_t)0xffffffffLL,
          "%s: dy and x must each stay below 4 GiB", fn);
  return check_hip(ttamd::launch_grouped_mm_wgrad(dy, x, offs, (int)num_rows, num_experts, (int)n,
                                                  (int)k, dw, dw_is_fp32 != 0, workspace,
                                                  (hipStream_t)stream),
                   fn);
}

// ---------------------------------------------------------------------------
// fp8 e4m3 path
// ---------------------------------------------------------------------------
namespace {

int check_fp8_k(const char* fn, const char* name, int64_t k) {
  if (k <= 0 || k % 128 != 0 || k > 8192)
    return fail(TTAMD_EINVAL, "%s: %s must be a positive multiple of 128 up to 8192 (got %lld)", fn, name,
                (long long)k);
  return TTAMD_OK;
}

int check_bytes(const char* fn, const char* name, const void* p, int64_t n) {
  if (n > 0 && p == nullptr) return fail(TTAMD_EINVAL, "%s: %s is null", fn, name);
  if (n > 0 && !aligned16(p)) return fail(TTAMD_EINVAL, "%s: %s must be 16-byte aligned", fn, name);
  if (n > (int64_t(1) << 34)) return fail(TTAMD_EINVAL, "%s: %s too large", fn, name);
  return TTAMD_OK;
}

int check_fp8_gemm(const char* fn, const void* xq, const float* sx, const void* wq, const float* sw,
                   int64_t M, int E, int64_t n_rows, int64_t k) {
  TRY(check_fp8_k(fn, "k", k));
  TRY(check_bytes(fn, "xq", xq, M * k));
  TRY(check_bytes(fn, "wq", wq, (int64_t)E * n_rows * k));
  REQUIRE(M * k <= kI32Max, "%s: activation rows x k must stay below 2^31 bytes", fn);
  REQUIRE(n_rows * k <= kI32Max, "%s: one expert's weights must stay below 2^31 bytes", fn);
  if (M > 0) REQUIRE(sx != nullptr && sw != nullptr, "%s: null scale pointer", fn);
  return TTAMD_OK;
}

}  // namespace

int ttamd_quantize_fp8_rows(const void* in, const int32_t* src_index, int src_div, const float* row_scale,
                            int64_t num_in_rows, int64_t num_rows, int64_t k, void* q_out, float* scale_t,
                            void* stream) {
  const char* fn = "ttamd_quantize_fp8_rows";
  TRY(check_fp8_k(fn, "k", k));
  REQUIRE(num_rows >= 0 && num_rows <= (1 << 28), "%s: num_rows out of range", fn);
  REQUIRE(num_in_rows >= 0 && num_in_rows <= kI32Max, "%s: num_in_rows out of range", fn);
  if (src_index == nullptr)
    REQUIRE(num_in_rows >= num_rows, "%s: without src_index the input needs num_rows rows", fn);
  else
    REQUIRE(src_div >= 1 && num_in_rows >= 1, "%s: src_div must be >= 1 and the input non-empty", fn);
  TRY(check_rows(fn, "in", in, num_in_rows, k));
  TRY(check_bytes(fn, "q_out", q_out, num_rows * k));
  if (num_rows > 0) REQUIRE(scale_t != nullptr, "%s: scale_t is null", fn);
  if (num_rows == 0) return TTAMD_OK;
  return check_hip(ttamd::launch_quantize_rows(in, src_index, src_div, row_scale, (int)num_in_rows,
                                               (int)num_rows, (int)k, q_out, scale_t, (hipStream_t)stream),
                   fn);
}

int ttamd_quantize_fp8_blocks(const void* w, int num_experts, int64_t n, int64_t k, void* q_out, float* scale,
                              void* stream) {
  const char* fn = "ttamd_quantize_fp8_blocks";
  REQUIRE(num_experts >= 0 && num_experts <= 1024, "%s: num_experts out of range", fn);
  TRY(check_dim(fn, "n", n, 128));
  TRY(check_fp8_k(fn, "k", k));
  const int64_t rows = (int64_t)num_experts * n;
  TRY(check_rows(fn, "w", w, rows, k));
  TRY(check_bytes(fn, "q_out", q_out, rows * k));
  REQUIRE((int64_t)num_experts * (n / 128) * (k / 128) <= kI32Max, "%s: too many blocks", fn);
  if (rows > 0) REQUIRE(scale != nullptr, "%s: scale is null", fn);
  if (rows == 0) return TTAMD_OK;
  return check_hip(ttamd::launch_quantize_blocks(w, num_experts, (int)n, (int)k, q_out, scale,
                                                 (hipStream_t)stream),
                   fn);
}

int ttamd_grouped_mm_fp8(const void* xq, const float* sx_t, const void* wq, const float* sw,
                         const int32_t* offs, int64_t num_rows, int num_experts, int64_t n, int64_t k,
                         void* out, void* workspace, size_t workspace_bytes, void* stream) {
  const char* fn = "ttamd_grouped_mm_fp8";
  TRY(check_gemm_common(fn, offs, num_rows, num_experts));
  TRY(check_dim(fn, "n", n, 128));
  TRY(check_fp8_gemm(fn, xq, sx_t, wq, sw, num_rows, num_experts, n, k));
  TRY(check_rows(fn, "out", out, num_rows, n));
  TRY(check_ws(fn, workspace, workspace_bytes, ttamd::gemm_workspace_bytes(num_rows, num_experts)));
  if (num_rows == 0) return TTAMD_OK;
  return check_hip(ttamd::launch_grouped_mm_fp8(xq, sx_t, wq, sw, offs, (int)num_rows, num_experts, (int)n,
                                                (int)k, out, workspace, (hipStream_t)stream),
                   fn);
}

int ttamd_grouped_mm_fp8_swiglu(const void* xq, const float* sx_t, const void* w13q, const float* s13,
                                const int32_t* offs, int64_t num_rows, int num_experts, int64_t hidden,
                                int64_t dim, float swiglu_limit, void* a_out, void* h_out, void* workspace,
                                size_t workspace_bytes, void* stream) {
  const char* fn = "ttamd_grouped_mm_fp8_swiglu";
  TRY(check_gemm_common(fn, offs, num_rows, num_experts));
  TRY(check_dim(fn, "hidden", hidden, 64));
  TRY(check_fp8_gemm(fn, xq, sx_t, w13q, s13, num_rows, num_experts, 2 * hidden, dim));
  TRY(check_rows(fn, "a_out", a_out, num_rows, hidden));
  if (h_out) TRY(check_rows(fn, "h_out", h_out, num_rows, 2 * hidden));
  TRY(check_ws(fn, workspace, workspace_bytes, ttamd::gemm_workspace_bytes(num_rows, num_experts)));
  if (num_rows == 0) return TTAMD_OK;
  return check_hip(ttamd::launch_grouped_mm_fp8_swiglu(xq, sx_t, w13q, s13, offs, (int)num_rows, num_experts,
                                                       (int)hidden, (int)dim, swiglu_limit, a_out, h_out,
                                                       workspace, (hipStream_t)stream),
                   fn);
}

int ttamd_grouped_mm_fp8_unpermute(const void* aq, const float* sa_t, const void* w2q, const float* s2,
                                   const int32_t* offs, int64_t num_rows, int num_experts, int64_t dim,
                                   int64_t hidden, const float* row_scale, const int32_t* dest,
                                   int64_t num_dest_rows, void* out, void* workspace, size_t workspace_bytes,
                                   void* stream) {
  const char* fn = "ttamd_grouped_mm_fp8_unpermute";
  TRY(check_gemm_common(fn, offs, num_rows, num_experts));
  TRY(check_dim(fn, "dim", dim, 128));
  TRY(check_fp8_gemm(fn, aq, sa_t, w2q, s2, num_rows, num_experts, dim, hidden));
  if (dest == nullptr)
    REQUIRE(num_dest_rows >= num_rows, "%s: out needs num_rows rows when dest is null", fn);
  REQUIRE(num_dest_rows >= 0, "%s: negative num_dest_rows", fn);
  REQUIRE(num_rows == 0 || num_dest_rows > 0, "%s: out has no rows", fn);
  TRY(check_rows(fn, "out", out, num_dest_rows, dim));
  TRY(check_ws(fn, workspace, workspace_bytes, ttamd::gemm_workspace_bytes(num_rows, num_experts)));
  if (num_rows == 0) return TTAMD_OK;
  return check_hip(ttamd::launch_grouped_mm_fp8_unpermute(aq, sa_t, w2q, s2, offs, (int)num_rows, num_experts,
                                                          (int)dim, (int)hidden, row_scale, dest,
                                                          (int)num_dest_rows, out, workspace,
                                                          (hipStream_t)stream),
                   fn);
}

}  // extern "C"
