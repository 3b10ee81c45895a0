// Host-side launchers of the device kernels (internal to libttamd_moe.so).
// All sizes have been validated by the C ABI layer before these are called.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "probe.h"

namespace ttamd {

// routing.hip
size_t route_workspace_bytes(int64_t M, int E);
// Bytes of the per-chunk histogram the route kernels read and write.
size_t route_hist_bytes(int64_t M, int E);
// Histogram geometry: chunks of route_chunk_labels() flat labels, the
// histogram stored bucket-major, hist[b * num_chunks + chunk].
int route_num_chunks(int64_t M);
int route_chunk_labels();
// The rank pass folds the histogram scan in (one launch) for histograms of
// at most 32768 entries.
bool route_fused_scan(int64_t M, int E);
// Scan + rank from an accumulated histogram: counts, offsets, the stable
// order; optionally adds the counts to tokens_per_expert and builds the
// forward GEMMs' tile table (tiles of at most plan_max_rows rows) in `plan`
// (gemm workspace layout).
hipError_t launch_route_from_hist(const void* labels, bool is64, int M, int E, const float* scores,
                                  int* counts, int* offsets, int* sorted_idx, int* inverse,
                                  float* sorted_scores, int* hist, float* tokens_per_expert,
                                  void* plan, int plan_max_rows, hipStream_t stream);
hipError_t launch_route(const void* labels, bool is64, int M, int E, const float* scores,
                        int* counts, int* offsets, int* sorted_idx, int* inverse,
                        float* sorted_scores, void* ws, hipStream_t stream);
// The library-owned route workspace of the device that runs `stream` (the
// current device for a null stream): its size, and its device address
// (looked up once per device, then cached).
size_t route_scratch_bytes();
hipError_t route_scratch(hipStream_t stream, void** ptr);
hipError_t launch_gather_rows(const void* in, const int* src, const float* scale,
                              bool scale_by_src, int n_in, int n_src_max, int rows, int hidden,
                              int div, void* out, hipStream_t stream);
hipError_t launch_invert_perm(const int* sorted, int M, int* inv, hipStream_t stream);
hipError_t launch_dispatch_rows(const void* in, const int* inverse, const float* scores, int T, int K,
                                int hidden, void* out, hipStream_t stream);
hipError_t launch_combine(const void* in, const int* inverse, const float* probs, int T,
                          int topk, int hidden, void* out, hipStream_t stream);
hipError_t launch_rowdot(const void* a, const void* b, const int* bidx, int bdiv,
                         bool out_by_bidx, int rows, int n_b, int n_out, int hidden, float* out,
                         hipStream_t stream);
hipError_t launch_group_labels(const int* counts_group, int G, int E_loc, int rows, int* labels,
                               hipStream_t stream);
hipError_t launch_router_topk(const float* logits, const float* bias, int T, int E, int K,
                              int score_func, int renorm, float renorm_eps, float route_scale,
                              float* top_scores, int64_t* top_idx, hipStream_t stream);

// router.hip
size_t router_workspace_bytes(int64_t T, int E, int64_t D);
hipError_t launch_router_fused(const void* x, const void* w, const float* bias, int T, int E, int D, int K,
                               int score_func, int renorm, float renorm_eps, float route_scale,
                               float* top_scores, int64_t* top_idx, void* logits, void* ws,
                               hipStream_t stream);
// The same router, also accumulating the route histogram of the picks into
// `hist` ((E + 1) * route_num_chunks(T * K) ints, cleared by the gate GEMM
// kernel first), ready for launch_route_from_hist.
hipError_t launch_router_hist(const void* x, const void* w, const float* bias, int T, int E, int D, int K,
                              int score_func, int renorm, float renorm_eps, float route_scale,
                              float* top_scores, int64_t* top_idx, void* logits, void* ws, int* hist,
                              hipStream_t stream);

// Router backward: d(top_scores) -> d(logits) -> dx (bf16 [T, D], nullable)
// and dW_r ([E, D], fp32 or bf16, nullable).
size_t router_backward_workspace_bytes(int64_t T, int E, int64_t D);
hipError_t launch_router_backward(const float* grad, const int64_t* idx, const void* logits, const void* x,
                                  const void* w, int T, int E, int D, int K, int score_func, int renorm,
                                  float renorm_eps, float route_scale, void* dx, void* dw, bool dw_fp32,
                                  void* ws, hipStream_t stream);

// gemm.hip
int gemm_max_qtiles(int M, int E);
size_t gemm_workspace_bytes(int64_t M, int E);
size_t gemm_plan_bytes(int64_t M, int E);
// Largest token tile of the bf16 forward / dgrad GEMMs (tile plans are built for it).
int gemm_fwd_tile_rows();
// The next forward grouped-GEMM launch records these events around its main
// kernel on its stream, then the probe disarms (nullptr, nullptr: disarm).
void gemm_probe_arm(hipEvent_t start, hipEvent_t end);
// The next n_launches kernel launches of the library take the event pairs
// (events[2 i], events[2 i + 1]) as their start and end stamps (n_launches
// <= kProbeMaxChain; 0 disarms).
void probe_chain_arm(const hipEvent_t* events, int n_launches);
hipError_t launch_grouped_mm(const void* x, const void* w, const int* offs, int M, int E, int N,
                             int K, void* out, void* ws, hipStream_t stream);
hipError_t launch_grouped_mm_swiglu(const void* x, const void* w13, const int* offs, int M,
                                    int E, int H, int D, float limit, void* a_out, void* h_out,
                                    void* ws, hipStream_t stream);
hipError_t launch_grouped_mm_swiglu_gather(const void* tokens, int n_tokens, const int* src_index,
                                           int src_div, const void* w13, const int* offs, int M, int E,
                                           int H, int D, float limit, void* a_out, void* h_out, void* ws,
                                           hipStream_t stream);
hipError_t launch_grouped_mm_unpermute(const void* act, const void* w2, const int* offs, int M,
                                       int E, int D, int H, const float* row_scale,
                                       const int* dest, int n_dest, void* out, void* ws,
                                       hipStream_t stream);
hipError_t launch_shared_expert_add(const void* x, int T, int D, int H, const void* w13s, const void* w2s,
                                   const float* gate_logits, float limit, void* a_scratch, void* out,
                                   void* ws, hipStream_t stream);
// The expert stage of the inference forward: (gather [+ score] ->) w13 +
// SwiGLU -> w2 + score + scatter (-> K-way sum), both GEMMs on one tile
// table (`plan`, or one built into the workspace when plan is null).
size_t moe_experts_forward_workspace_bytes(int64_t T, int64_t D, int64_t H, int E, int K, bool permute_first);
hipError_t launch_moe_experts_forward(const void* tokens, int T, int D, int H, int E, int K,
                                      const int* sorted_idx, const int* offs, const float* sorted_scores,
                                      bool score_before, float limit, const void* w13, const void* w2,
                                      void* out, void* plan, void* ws, hipStream_t stream);
hipError_t launch_grouped_mm_dgrad(const void* dy, const void* w, const int* offs, int M, int E,
                                   int N, int K, void* dx, void* ws, hipStream_t stream);
// The same without the tail split: plan is gemm_plan_bytes(M, E) bytes.
hipError_t launch_grouped_mm_dgrad_unsplit(const void* dy, const void* w, const int* offs, int M, int E, int N,
                                           int K, void* dx, void* plan, hipStream_t stream);
hipError_t launch_grouped_mm_dgrad_swiglu(const void* dy, const void* w2, const void* h,
                                          const int* offs, int M, int E, int D, int H,
                                          float limit, void* dh, void* a_out, void* ws,
                                          hipStream_t stream);
// ws: NULL (no tail split) or gemm_workspace_bytes(M, E) bytes (the
// leftover tiles' partial sums and arrival counters).
hipError_t launch_grouped_mm_wgrad(const void* dy, const void* x, const int* offs, int M, int E,
                                   int N, int K, void* dw, bool fp32, void* ws, hipStream_t stream);

// fp8 e4m3 path (quant.hip, gemm_fp8.hip via gemm.hip)
hipError_t launch_quantize_rows(const void* in, const int* src_index, int src_div, const float* row_mul,
                                int n_in, int R, int K, void* q_out, float* scale_t, hipStream_t stream);
hipError_t launch_quantize_blocks(const void* w, int E, int N, int K, void* q_out, float* scale,
                                  hipStream_t stream);
hipError_t launch_grouped_mm_fp8(const void* xq, const float* sx, const void* wq, const float* sw,
                                 const int* offs, int M, int E, int N, int K, void* out, void* ws,
                                 hipStream_t stream);
hipError_t launch_grouped_mm_fp8_swiglu(const void* xq, const float* sx, const void* w13q,
                                        const float* s13, const int* offs, int M, int E, int H, int D,
                                        float limit, void* a_out, void* h_out, void* ws,
                                        hipStream_t stream);
hipError_t launch_grouped_mm_fp8_unpermute(const void* aq, const float* sa, const void* w2q,
                                           const float* s2, const int* offs, int M, int E, int D, int H,
                                           const float* row_scale, const int* dest, int n_dest,
                                           void* out, void* ws, hipStream_t stream);

}  // namespace ttamd
