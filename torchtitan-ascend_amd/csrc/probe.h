// Kernel timing probe and the launch helper every kernel of the library
// goes through (internal to libttamd_moe.so; the probe is a measurement aid
// with no counterpart in the reference).
//
// A probed launch passes its event pair to hipExtLaunchKernelGGL, which
// stamps the kernel's own start and end from its dispatch: nothing is
// enqueued between kernels, so the timed kernels run back to back exactly
// as unprobed ones do.  The probe is per host thread (the launches of the
// thread that armed it).  Two ways to arm it:
//   * the next grouped-GEMM main kernel (forward, dgrad, fp8) takes the
//     pair (gemm_start, gemm_end), then the probe disarms;
//   * a chain over the next n kernel launches of the library, whatever they
//     are: launch i takes (chain[2 i], chain[2 i + 1]).
// While a chain is armed it takes every launch (the GEMM pair waits).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstdint>

namespace ttamd {

constexpr int kProbeMaxChain = 16;

struct Probe {
  hipEvent_t gemm_start = nullptr, gemm_end = nullptr;
  hipEvent_t chain[2 * kProbeMaxChain] = {};
  int chain_n = 0;  // launches the chain covers (0: disarmed)
  int chain_i = 0;  // launches already taken
};

Probe& probe();

// Launch `kernel` on `stream`; gemm: it is a grouped-GEMM main kernel.
template <typename F, typename... Args>
hipError_t launch_k(bool gemm, F kernel, dim3 grid, dim3 block, uint32_t shmem, hipStream_t stream,
                    Args... args) {
  Probe& p = probe();
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (p.chain_i < p.chain_n) {
    e0 = p.chain[2 * p.chain_i];
    e1 = p.chain[2 * p.chain_i + 1];
    if (++p.chain_i == p.chain_n) p.chain_n = p.chain_i = 0;
  } else if (gemm && p.gemm_start && p.gemm_end) {
    e0 = p.gemm_start;
    e1 = p.gemm_end;
    p.gemm_start = p.gemm_end = nullptr;
  }
  hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream, e0, e1, 0, args...);
  return hipGetLastError();
}

}  // namespace ttamd
