// MFMA ceiling probe (measurement aid; no counterpart in the reference).
//
// The forward grouped GEMM's k loop with everything else taken out: 8 waves
// per CU, two 72 KB LDS stage buffers holding pseudo-random bf16 values,
// per k16 step the fragment reads of the next step (the kernel's swizzled
// addresses, 2 weight + 5 token blocks per wave) while 10
// v_mfma_f32_32x32x16_bf16 run on the current ones, one workgroup barrier per
// 64-wide stage, tiles of 32 stages.  No global memory traffic, no epilogue.
//
// With constant operands this loop runs at ~85 % of the 2.5 PFLOP/s dense
// bf16 peak; with random operands the chip's power management lowers the
// clock and it runs at ~62 %.  That second figure is the ceiling a bf16 GEMM
// on realistic data can approach on the GPU it is measured on.
#include "common.h"
#include "gemm_common.h"
#include "kernels.h"

namespace ttamd {
namespace {

constexpr int PNPB = 2, PNJ = 5, PWAVES = 8;
constexpr int PROW = 128;
constexpr int PP_BYTES = 256 * PROW;
constexpr int PSTAGE = 576 * PROW;  // 72 KB, as gg_fwd_kernel
constexpr int PLDS = 2 * PSTAGE;
constexpr int PTILE_STAGES = 32;

__global__ __launch_bounds__(64 * PWAVES, 1) void mfma_loop_kernel(int64_t stages, float* sink) {
  extern __shared__ __attribute__((aligned(1024))) char smem[];
  const int l = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r32 = l & 31, half = l >> 5, fa = (r32 ^ (r32 >> 3)) & 7;
  const int wq = w / 4, wp = w % 4;
  // random bf16 pairs, magnitudes 2^-7 .. 2^-5, both signs
  for (int i = threadIdx.x; i < PLDS / 4; i += blockDim.x) {
    uint32_t h = (uint32_t)(i + 977 * blockIdx.x) * 2654435761u + 12345u;
    h ^= h >> 13;
    h *= 0x5bd1e995u;
    h ^= h >> 15;
    const uint32_t lo = 0x3c00u + (h & 0x3ffu) + ((h >> 10) & 1u) * 0x8000u;
    const uint32_t hi = 0x3c00u + ((h >> 11) & 0x3ffu) + ((h >> 21) & 1u) * 0x8000u;
    ((uint32_t*)smem)[i] = lo | (hi << 16);
  }
  __syncthreads();
  struct Frag {
    bf16x8_t a[PNPB];
    bf16x8_t b[PNJ];
  };
  auto read_frag = [&](Frag& f, int64_t s, int kk) {
    const char* st = smem + (s & 1) * PSTAGE;
#pragma unroll
    for (int pb = 0; pb < PNPB; ++pb) {
      const int pc = (2 * kk + half) ^ fa ^ (4 * (pb & 1));
      f.a[pb] = *(const bf16x8_t*)(st + (64 * wp + 32 * pb + r32) * PROW + pc * 16);
    }
#pragma unroll
    for (int j = 0; j < PNJ; ++j) {
      const int pc = (2 * kk + half) ^ fa ^ (4 * wq);
      f.b[j] = *(const bf16x8_t*)(st + PP_BYTES + (64 * j + 32 * wq + r32) * PROW + pc * 16);
    }
  };
  float sum = 0.f;
  int64_t s = 0;
  Frag f0, f1;
  for (int64_t t0 = 0; t0 < stages; t0 += PTILE_STAGES) {
    const int64_t ns = min((int64_t)PTILE_STAGES, stages - t0);
    floatx16_t acc[PNPB][PNJ];
#pragma unroll
    for (int i = 0; i < PNPB; ++i)
#pragma unroll
      for (int j = 0; j < PNJ; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
    auto mfma = [&](const Frag& f) {
#pragma unroll
      for (int j = 0; j < PNJ; ++j)
#pragma unroll
        for (int pb = 0; pb < PNPB; ++pb)
          acc[pb][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[pb], f.b[j], acc[pb][j], 0, 0, 0);
    };
    read_frag(f0, s, 0);
    for (int64_t ks = 0; ks < ns; ++ks, ++s) {
      read_frag(f1, s, 1);
      mfma(f0);
      read_frag(f0, s, 2);
      mfma(f1);
      read_frag(f1, s, 3);
      mfma(f0);
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      if (ks + 1 < ns) read_frag(f0, s + 1, 0);
      mfma(f1);
    }
#pragma unroll
    for (int i = 0; i < PNPB; ++i)
#pragma unroll
      for (int j = 0; j < PNJ; ++j) sum += acc[i][j][0] + acc[i][j][15];
  }
  // keep the accumulators live; the condition never holds for these inputs
  if (sum == 1.2345e30f) sink[0] = sum;
}

}  // namespace

double probe_mfma_loop_flops(int64_t stages) {
  return (double)num_cus() * PWAVES * (double)stages * 4.0 * PNPB * PNJ * 32.0 * 32.0 * 16.0 * 2.0;
}

hipError_t launch_probe_mfma_loop(int64_t stages, float* sink, hipStream_t stream) {
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t err = hipFuncSetAttribute((const void*)mfma_loop_kernel,
                                         hipFuncAttributeMaxDynamicSharedMemorySize, PLDS);
    if (err != hipSuccess) return err;
    attr_set = true;
  }
  hipLaunchKernelGGL(mfma_loop_kernel, dim3(num_cus()), dim3(64 * PWAVES), PLDS, stream, stages, sink);
  return hipGetLastError();
}

}  // namespace ttamd
