// Shared device helpers for the MI355X (gfx950) MoE expert path.
//
// Everything here is written for CDNA4 only: 64-lane wavefronts, MFMA bf16
// matrix cores, 160 KB LDS per CU.  bf16 values travel as raw uint16_t bits;
// conversion to bf16 uses the hardware round-to-nearest-even instruction
// (v_cvt_pk_bf16_f32) through clang's __bf16 cast.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace ttamd {

typedef uint16_t bf16_t;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));
typedef float floatx16_t __attribute__((ext_vector_type(16)));
// Native 8- and 16-byte vectors for register staging (HIP's uint2/uint4 are
// union-based structs that the optimiser cannot always keep in registers).
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  __bf16 b = (__bf16)f;
  return (uint32_t)__builtin_bit_cast(uint16_t, b);
}

// fp32 -> bf16 (round to nearest even) -> fp32.
__device__ __forceinline__ float round_bf16(float x) { return bf16_to_f32(f32_to_bf16(x)); }

// Pack two floats into one dword of two bf16 (lo in bits 0..15).  The
// two-wide conversion is one v_cvt_pk_bf16_f32 with both sources; two
// scalar casts cost two conversions, a shift and an or.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
}

// Unpack 8 bf16 held in a uint4 into 8 floats.
__device__ __forceinline__ void unpack8(const uint4& v, float* f) {
  f[0] = __uint_as_float(v.x << 16);
  f[1] = __uint_as_float(v.x & 0xffff0000u);
  f[2] = __uint_as_float(v.y << 16);
  f[3] = __uint_as_float(v.y & 0xffff0000u);
  f[4] = __uint_as_float(v.z << 16);
  f[5] = __uint_as_float(v.z & 0xffff0000u);
  f[6] = __uint_as_float(v.w << 16);
  f[7] = __uint_as_float(v.w & 0xffff0000u);
}

__device__ __forceinline__ uint4 pack8(const float* f) {
  uint4 v;
  v.x = pack_bf16x2(f[0], f[1]);
  v.y = pack_bf16x2(f[2], f[3]);
  v.z = pack_bf16x2(f[4], f[5]);
  v.w = pack_bf16x2(f[6], f[7]);
  return v;
}

// Streaming (non-temporal) 16-byte load and store, for data a kernel reads
// or writes exactly once.
__device__ __forceinline__ uint4 load_stream(const uint4* p) {
  const u32x4_t q = __builtin_nontemporal_load((const u32x4_t*)p);
  return make_uint4(q[0], q[1], q[2], q[3]);
}
__device__ __forceinline__ void store_stream(uint4* p, const uint4& v) {
  __builtin_nontemporal_store(u32x4_t{v.x, v.y, v.z, v.w}, (u32x4_t*)p);
}

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & (kWave - 1)); }

// The wave's LDS writes (and reads) issued so far have completed.  A wave
// that reads back LDS it has just written itself waits here first:
// measured on gfx950, a ds_read following a masked run of ds_writes to the
// same bytes could return the old contents.  Also a compiler barrier for
// memory operations.
__device__ __forceinline__ void lds_wait() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// All-reduce over the 16 lanes of a DPP row in four pairwise steps: xor 1,
// xor 2 (quad permutes), then the half-row and row mirrors.  Each step
// combines a lane with one partner and the pairs are symmetric, so with a
// commutative combine every lane ends with bit-identical results.
constexpr int kDppXor1 = 0xb1;        // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4e;        // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141;  // lane i <-> 7 - i within each 8
constexpr int kDppMirror = 0x140;      // lane i <-> 15 - i within the row

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_mov_dpp(v, CTRL, 0xf, 0xf, false);
}

__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f<kDppXor1>(v));
  v = fmaxf(v, dpp_f<kDppXor2>(v));
  v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
  return fmaxf(v, dpp_f<kDppMirror>(v));
}

__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f<kDppXor1>(v);
  v += dpp_f<kDppXor2>(v);
  v += dpp_f<kDppHalfMirror>(v);
  return v + dpp_f<kDppMirror>(v);
}

// Order-preserving unsigned key of a router selection value: a larger value
// has a larger key, -inf the smallest of any number, NaN above +inf (the
// largest key, whatever its sign and payload: torch.topk ranks NaN as the
// largest value), and 0 is left for a slot already picked.  -0 becomes +0
// first (the two compare equal).  Picking the largest key, ties to the lower
// expert id, is the order of torch.sort(values, descending=True,
// stable=True): NaN first, then the numbers in descending order.
__device__ __forceinline__ uint32_t sel_key(float v) {
  const uint32_t b = __float_as_uint(v + 0.f);
  const uint32_t k = b ^ ((uint32_t)((int32_t)b >> 31) | 0x80000000u);
  return v == v ? k : 0xffffffffu;
}

__device__ __forceinline__ uint64_t lanemask_lt() {
  const int l = lane_id();
  return (l == 0) ? 0ull : (~0ull >> (64 - l));
}

// Wave-wide ballot as a 64-bit mask.
__device__ __forceinline__ uint64_t ballot64(bool p) {
  return (uint64_t)__builtin_amdgcn_ballot_w64(p);
}

// Inclusive wave prefix sum of a 32-bit int (64 lanes), via LDS-free shuffles.
__device__ __forceinline__ int wave_inclusive_scan(int v) {
  const int l = lane_id();
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    int t = __shfl_up(v, off, kWave);
    if (l >= off) v += t;
  }
  return v;
}

__device__ __forceinline__ int wave_reduce_sum(int v) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ float wave_reduce_sumf(float v) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

}  // namespace ttamd
