// Per-head RMSNorm and RoPE of one row of head_dim values, in the rounding
// chain of the reference torch path (acorninfer/ops/rope.py:1-13, 116-125;
// models/qwen3.py:50-60), shared by the qkv epilogue (rope.hip) and the
// attention kernel that runs the epilogue itself (paged_attention.hip), so
// that both produce the same bits.
//   norm:  r((x * rsqrt(mean(x^2) + eps)) * w), rsqrt as a correctly rounded 1/sqrt
//   rope:  cos/sin in fp32 rounded to T; y1 = r(r(x1*c) - r(x2*s)), y2 = r(r(x2*c) + r(x1*s))
// FMA contraction is disabled so every product is rounded as torch does.
#pragma once
#include "common.h"

namespace acorn {

// cos and sin of the pair's angle, rounded to T
template <typename T>
__device__ __forceinline__ void rope_cs(float pos, float inv_freq, float& c, float& s) {
#pragma clang fp contract(off)
  const float f = pos * inv_freq;
  c = round_to<T>(cosf(f));
  s = round_to<T>(sinf(f));
}

template <typename T>
__device__ __forceinline__ void rope_pair_cs(float& x1, float& x2, float c, float s) {
#pragma clang fp contract(off)
  const float t1 = round_to<T>(x1 * c), t2 = round_to<T>(x2 * s);
  const float t3 = round_to<T>(x2 * c), t4 = round_to<T>(x1 * s);
  x1 = round_to<T>(t1 - t2);
  x2 = round_to<T>(t3 + t4);
}

template <typename T>
__device__ __forceinline__ void rope_pair(float& x1, float& x2, float pos, float inv_freq) {
  float c, s;
  rope_cs<T>(pos, inv_freq, c, s);
  rope_pair_cs<T>(x1, x2, c, s);
}

// Per-head RMSNorm over the lane's NP pairs (x1[j], x2[j]) followed by RoPE,
// with the norm weights (w1 = w[i], w2 = w[i + half]) and the rotation's
// rounded cos and sin (rope_cs) already in registers.
template <typename T, int NP>
__device__ __forceinline__ void norm_rope_cs(float (&x1)[NP], float (&x2)[NP], int half,
                                             const float (&w1)[NP], const float (&w2)[NP],
                                             float eps, const float (&cs)[NP],
                                             const float (&sn)[NP]) {
#pragma clang fp contract(off)
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NP; ++j) {
    const int i = (threadIdx.x & (kWave - 1)) + j * kWave;
    if (i < half) ss += x1[j] * x1[j] + x2[j] * x2[j];
  }
  ss = wave_sum(ss);
  const float inv = 1.0f / sqrtf(ss / (float)(2 * half) + eps);
#pragma unroll
  for (int j = 0; j < NP; ++j) {
    const int i = (threadIdx.x & (kWave - 1)) + j * kWave;
    if (i < half) {
      x1[j] = round_to<T>((x1[j] * inv) * w1[j]);
      x2[j] = round_to<T>((x2[j] * inv) * w2[j]);
      rope_pair_cs<T>(x1[j], x2[j], cs[j], sn[j]);
    }
  }
}

// The same with the frequencies instead of cos and sin.
template <typename T, int NP>
__device__ __forceinline__ void norm_rope_pre(float (&x1)[NP], float (&x2)[NP], int half,
                                              const float (&w1)[NP], const float (&w2)[NP],
                                              float eps, float pos, const float (&fr)[NP]) {
  float cs[NP], sn[NP];
#pragma unroll
  for (int j = 0; j < NP; ++j) rope_cs<T>(pos, fr[j], cs[j], sn[j]);
  norm_rope_cs<T, NP>(x1, x2, half, w1, w2, eps, cs, sn);
}

}  // namespace acorn
