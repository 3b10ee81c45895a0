// fp8 e4m3 quantisation with fp32 block scales (absmax / 448) on MI355X.
//
//   rows:   activations [R, K], one scale per row and 128 channels, written
//           k-block major (scale_t[K/128][R]) for the fp8 GEMM's DMA; the
//           rows can be gathered on the way (routed row j reads input row
//           src_index[j] / src_div), which fuses the MoE permute.
//   blocks: weights [E, N, K], one scale per 128 x 128 block ([E][N/128][K/128]).
//
// e4m3 here is the OCP "fn" variant (bias 7, largest finite 448, no
// infinities, code 0x7f = NaN), the format the gfx950 fp8 MFMA reads with
// cbsz/blgp = 0.  The conversion rounds to nearest even and is done with
// integer operations on the float32 bits, so it does not depend on the
// hardware conversion instructions' saturation mode.  |v| above 464 (half
// way to 480) gives NaN, which the absmax / 448 recipe never produces.
#include "common.h"
#include "kernels.h"

namespace ttamd {

__device__ __forceinline__ uint32_t f32_to_e4m3(float v) {
  uint32_t u = __float_as_uint(v);
  const uint32_t sign = (u >> 24) & 0x80u;
  u &= 0x7fffffffu;
  if (u > 0x43e80000u) return sign | 0x7fu;  // > 464, inf, NaN
  if (u < 0x3c800000u) {                     // below 2^-6: multiples of 2^-9
    const float t = __uint_as_float(u) * 512.0f;  // exact
    return sign | (uint32_t)__builtin_rintf(t);   // 0..8 (8 = smallest normal 0x08)
  }
  // keep 3 mantissa bits, round to nearest even (a carry bumps the exponent)
  const uint32_t r = u + 0x7ffffu + ((u >> 20) & 1u);
  const uint32_t e = (r >> 23) - 127u + 7u;
  return sign | (e << 3) | ((r >> 20) & 7u);
}

// Can the e4m3 rounding of q depend on bits an approximate quotient gets
// wrong?  In the normal e4m3 range the cast keeps 3 mantissa bits, so only a
// quotient within a few fp32 ulps of the halfway pattern (low 20 bits =
// 0x80000) can round differently; 16 ulps each side is a wide margin for
// f * rcp(s) (two roundings plus rcp's 1 ulp).  Below 2^-6 (e4m3 subnormals,
// zero) the quotient is always taken exactly.
__device__ __forceinline__ bool e4m3_tie_risk(float q) {
  const uint32_t u = __float_as_uint(q) & 0x7fffffffu;
  return u < 0x3c800000u || ((u & 0xfffffu) - 0x7fff0u) <= 0x20u;
}

// ---------------------------------------------------------------------------
// Rows: a workgroup of 4 waves quantises 16 rows (4 per wave).  Lane l holds
// 8 consecutive channels of every 512-channel step (16 lanes form one
// 128-channel block).  All of a row's loads are issued before any of its
// arithmetic (up to kMaxSteps x 16 bytes per lane), so a wave keeps its whole
// row in flight instead of one 1 KB step at a time.  Scales go through LDS
// so that each k-block's 16 row scales leave as one 64-byte store.
// The quotient v / s is f * rcp(s), replaced by the exact division wherever
// e4m3_tie_risk says the last bits could matter (a wave-uniform branch,
// taken for a few percent of steps), and v_cvt_pk_fp8_f32 (round to nearest
// even, OCP e4m3) packs the bytes: the result is the IEEE quotient's cast,
// bit for bit, at a fraction of the VALU work of a division per element.
// ---------------------------------------------------------------------------
constexpr int kQRows = 16;
constexpr int kMaxKBlocks = 64;  // K <= 8192
constexpr int kMaxSteps = kMaxKBlocks / 4;  // 512-channel steps per row

__global__ __launch_bounds__(256) void quantize_rows_kernel(const uint4* __restrict__ in,
                                                            const int* __restrict__ src_index,
                                                            int src_div, const float* __restrict__ row_mul,
                                                            int n_in, int R, int K,
                                                            uint2* __restrict__ q_out,
                                                            float* __restrict__ scale_t) {
  __shared__ float sc[kMaxKBlocks][kQRows];
  const int w = threadIdx.x >> 6;
  const int l = threadIdx.x & 63;
  const int row_base = blockIdx.x * kQRows;
  const int kv = K / 8;  // 16-byte vectors per row
  const int nkb = K / 128;
  for (int rr = w; rr < kQRows; rr += 4) {
    const int row = row_base + rr;
    if (row >= R) break;
    int src = row;
    if (src_index) src = min(max(src_index[row] / src_div, 0), n_in - 1);
    const float mul = row_mul ? row_mul[row] : 1.f;
    const uint4* irow = in + (int64_t)src * kv;
    uint2* orow = q_out + (int64_t)row * kv;
    uint4 v[kMaxSteps];
#pragma unroll
    for (int it = 0; it < kMaxSteps; ++it) {
      const int c = l + 64 * it;
      // the row is read once: streaming load (C5 gather + quantise 161 -> 153 us)
      v[it] = (c < kv) ? load_stream(&irow[c]) : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int it = 0; it < kMaxSteps; ++it) {
      if (64 * it >= kv) break;  // wave-uniform
      const int c = l + 64 * it;
      const bool ok = c < kv;
      float f[8];
      unpack8(v[it], f);  // zero past the row end
      if (row_mul) {
        // the dispatched row is materialised in bf16 after the score multiply
#pragma unroll
        for (int i = 0; i < 8; ++i) f[i] = bf16_to_f32(f32_to_bf16(f[i] * mul));
      }
      float m = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(f[i]));
      m = row16_max(m);  // the block's 16 lanes are one DPP row
      const float s = m / 448.0f;
      const float rs = (s > 0.f) ? __builtin_amdgcn_rcpf(s) : 0.f;
      float q[8];
      bool risk = false;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        q[i] = f[i] * rs;
        risk |= e4m3_tie_risk(q[i]);
      }
      if (__builtin_amdgcn_ballot_w64(risk && s > 0.f)) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (s > 0.f && e4m3_tie_risk(q[i])) q[i] = f[i] / s;
      }
      int lo = __builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false);
      lo = __builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], lo, true);
      int hi = __builtin_amdgcn_cvt_pk_fp8_f32(q[4], q[5], 0, false);
      hi = __builtin_amdgcn_cvt_pk_fp8_f32(q[6], q[7], hi, true);
      if (ok) {
        orow[c] = make_uint2((uint32_t)lo, (uint32_t)hi);
        if ((l & 15) == 0) sc[c >> 4][rr] = s;
      }
    }
  }
  __syncthreads();
  // scale_t[kb][row_base .. row_base + 15]
  for (int i = threadIdx.x; i < nkb * kQRows; i += 256) {
    const int kb = i / kQRows, rr = i % kQRows;
    if (row_base + rr < R) scale_t[(int64_t)kb * R + row_base + rr] = sc[kb][rr];
  }
}

// ---------------------------------------------------------------------------
// Blocks: one workgroup per 128 x 128 block; thread t covers row t / 2,
// channels 64 (t & 1) .. + 63.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void quantize_blocks_kernel(const uint4* __restrict__ w, int N, int K,
                                                              uint2* __restrict__ q_out,
                                                              float* __restrict__ scale) {
  __shared__ float red[4];
  const int nb = N / 128, kb = K / 128;
  const int blk = blockIdx.x;
  const int e = blk / (nb * kb);
  const int rem = blk - e * nb * kb;
  const int bn = rem / kb, bk = rem - bn * kb;
  const int t = threadIdx.x;
  const int64_t row = (int64_t)e * N + bn * 128 + (t >> 1);
  const int64_t v0 = row * (K / 8) + bk * 16 + (t & 1) * 8;  // first 16-byte vector
  float f[64];
#pragma unroll
  for (int i = 0; i < 8; ++i) unpack8(w[v0 + i], f + 8 * i);
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < 64; ++i) m = fmaxf(m, fabsf(f[i]));
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  if ((t & 63) == 0) red[t >> 6] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float s = m / 448.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    uint32_t b[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) b[j] = (s > 0.f) ? f32_to_e4m3(f[8 * i + j] / s) : 0u;
    q_out[v0 + i] = make_uint2(b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24),
                               b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24));
  }
  if (t == 0) scale[blk] = s;
}

hipError_t launch_quantize_rows(const void* in, const int* src_index, int src_div, const float* row_mul,
                                int n_in, int R, int K, void* q_out, float* scale_t, hipStream_t stream) {
  if (R == 0) return hipSuccess;
  const int grid = (R + kQRows - 1) / kQRows;
  return launch_k(false, quantize_rows_kernel, dim3(grid), dim3(256), 0, stream, (const uint4*)in, src_index,
                  src_div, row_mul, n_in, R, K, (uint2*)q_out, scale_t);
}

hipError_t launch_quantize_blocks(const void* w, int E, int N, int K, void* q_out, float* scale,
                                  hipStream_t stream) {
  const int64_t nblk = (int64_t)E * (N / 128) * (K / 128);
  if (nblk == 0) return hipSuccess;
  return launch_k(false, quantize_blocks_kernel, dim3((unsigned)nblk), dim3(256), 0, stream, (const uint4*)w, N,
                  K, (uint2*)q_out, scale);
}

}  // namespace ttamd
