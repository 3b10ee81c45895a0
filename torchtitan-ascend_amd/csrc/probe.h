// Kernel timing probe (internal to libttamd_moe.so; a measurement aid with
// no counterpart in the reference).
//
// Two ways to arm it, both from one host thread:
//   * the next forward grouped-GEMM launch records an event pair immediately
//     around its main kernel (gemm_start / gemm_end), then disarms;
//   * a chain over the next n kernel launches of the library, whatever they
//     are: chain[0] is recorded before the first and chain[i + 1] after the
//     i-th, so launch i runs between chain[i] and chain[i + 1] and n launches
//     cost n + 1 event records (adjacent launches share their boundary).
// Every launch site of the library that the probe may time goes through
// probed(); it is one kernel launch.
#pragma once

#include <hip/hip_runtime.h>

namespace ttamd {

constexpr int kProbeMaxChain = 16;

struct Probe {
  hipEvent_t gemm_start = nullptr, gemm_end = nullptr;
  hipEvent_t chain[kProbeMaxChain + 1] = {};
  int chain_n = 0;  // launches the chain covers (0: disarmed)
  int chain_i = 0;  // launches already recorded
};

Probe& probe();

// Launch `main` (one kernel) on `stream`, recording the armed events around
// it; gemm: the launch is a forward grouped-GEMM main kernel.
template <typename F>
hipError_t probed(hipStream_t stream, bool gemm, F&& main) {
  Probe& p = probe();
  hipEvent_t g0 = nullptr, g1 = nullptr, c0 = nullptr, c1 = nullptr;
  if (gemm && p.gemm_start && p.gemm_end) {
    g0 = p.gemm_start;
    g1 = p.gemm_end;
    p.gemm_start = p.gemm_end = nullptr;
  }
  if (p.chain_i < p.chain_n) {
    c0 = p.chain_i == 0 ? p.chain[0] : nullptr;
    c1 = p.chain[p.chain_i + 1];
    if (++p.chain_i == p.chain_n) p.chain_n = p.chain_i = 0;
  }
  hipError_t err = hipSuccess;
  if (c0 && (err = hipEventRecord(c0, stream)) != hipSuccess) return err;
  if (g0 && (err = hipEventRecord(g0, stream)) != hipSuccess) return err;
  if ((err = main()) != hipSuccess) return err;
  if (g1 && (err = hipEventRecord(g1, stream)) != hipSuccess) return err;
  if (c1 && (err = hipEventRecord(c1, stream)) != hipSuccess) return err;
  return hipSuccess;
}

}  // namespace ttamd
