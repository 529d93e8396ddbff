// Shared device helpers for the acorninfer_amd HIP kernels (gfx950 / CDNA4).
//
// Conventions used by every kernel in this library:
//  * activations are one of fp32 / fp16 / bf16, selected by an integer dtype
//    code (ACORN_F32=0, ACORN_F16=1, ACORN_BF16=2) at the C-ABI;
//  * every entry point launches only on the stream it is given, never
//    allocates, never synchronises, and returns 0 or a negative error code;
//  * a wavefront is 64 lanes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/acorn_hip.h"

namespace acorn {

constexpr int kWave = 64;

// ---- scalar conversions -------------------------------------------------
// __bf16 <-> float conversions lower to v_cvt_pk_bf16_f32 (RNE) on gfx950;
// _Float16 conversions are IEEE RNE as well.
template <typename T> __device__ __forceinline__ float to_f32(T v) { return (float)v; }
template <typename T> __device__ __forceinline__ T from_f32(float v) { return (T)v; }

// Round a float to the grid of T and widen it back (identity for float).
template <typename T> __device__ __forceinline__ float round_to(float v) {
  return (float)(T)v;
}
template <> __device__ __forceinline__ float round_to<float>(float v) { return v; }

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}
__device__ __forceinline__ float bf16_lo(uint32_t pair) { return __uint_as_float(pair << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t pair) { return __uint_as_float(pair & 0xffff0000u); }

// Two floats -> a bf16 pair (round to nearest even), lo in the low half; the
// vector conversion selects one v_cvt_pk_bf16_f32.
typedef __bf16 acorn_bf16x2 __attribute__((ext_vector_type(2)));
typedef float acorn_f32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const acorn_f32x2 f = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, acorn_bf16x2));
}

// ---- streamed loads --------------------------------------------------------
// Weights that a decode step reads exactly once may be loaded with the
// non-temporal cache policy (global_load ... nt) where every load
// instruction consumes whole 128-byte lines: on gfx950 such streams reach a
// higher HBM read rate (about 6.7 vs 5.9 TB/s for a 2 GiB linear read). Where
// an instruction reads half lines (16 rows x 64 bytes, the MFMA A layout) the
// policy is slower (the other half is fetched again), so those loads keep the
// default policy.
template <typename V>
__device__ __forceinline__ V load_nt(const V* p) {
  return __builtin_nontemporal_load(p);
}

// ---- split-K partial sums -------------------------------------------------
// sum_s p[s * plane] for s < nsplit, added in split order (so results do not
// depend on the launch). The loads of a batch of splits are issued before the
// first add: indices past the split count are clamped (in bounds, no branch)
// and their values discarded by a uniform test, which keeps the wait counts
// static.
constexpr int kSplitBatch = 8;
__device__ __forceinline__ float sum_splits(const float* p, size_t plane, int nsplit) {
  float a = 0.f;
  for (int s0 = 0; s0 < nsplit; s0 += kSplitBatch) {
    float v[kSplitBatch];
#pragma unroll
    for (int u = 0; u < kSplitBatch; ++u) v[u] = p[(size_t)min(s0 + u, nsplit - 1) * plane];
#pragma unroll
    for (int u = 0; u < kSplitBatch; ++u)
      if (s0 + u < nsplit) a = s0 + u == 0 ? v[u] : a + v[u];
  }
  return a;
}
// The same over 8 consecutive floats (16-byte aligned), 4 splits per batch.
__device__ __forceinline__ void sum_splits8(const float* p, size_t plane, int nsplit,
                                            float (&a)[8]) {
  typedef float f8 __attribute__((ext_vector_type(8)));
  for (int s0 = 0; s0 < nsplit; s0 += 4) {
    f8 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = *(const f8*)(p + (size_t)min(s0 + u, nsplit - 1) * plane);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (s0 + u < nsplit) {
#pragma unroll
        for (int i = 0; i < 8; ++i) a[i] = s0 + u == 0 ? v[u][i] : a[i] + v[u][i];
      }
    }
  }
}

// ---- wavefront reductions -----------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

// Block-wide sum for blockDim.x == NT (multiple of 64); every thread gets the
// total. `red` must hold NT/64 floats of LDS.
template <int NT>
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  if (NT == kWave) return v;
  if (lane == 0) red[wid] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < NT / kWave; ++i) t += red[i];
  __syncthreads();
  return t;
}

}  // namespace acorn

// Launch-error mapping shared by every entry point.
#define ACORN_LAUNCH_CHECK()                                    \
  do {                                                          \
    hipError_t _e = hipGetLastError();                          \
    if (_e != hipSuccess) return ACORN_ERR_HIP - (int)_e;       \
  } while (0)
