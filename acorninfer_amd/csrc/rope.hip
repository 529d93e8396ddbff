// K2: half-rotate RoPE, optionally preceded by the per-head q/k RMSNorm and
// followed by the paged-KV scatter of the decode step.
//
// Rounding mirrors the reference torch path (acorninfer/ops/rope.py:1-13,
// 116-125): cos/sin are computed in fp32 and rounded to the activation dtype;
// each product is rounded; the sum/difference is rounded again:
//   y1 = r(r(x1*c) - r(x2*s)),  y2 = r(r(x2*c) + r(x1*s))
// The per-head norm is models/qwen3.py:50-60: r((x * rsqrt(mean(x^2)+eps)) * w).
// FMA contraction is disabled so every product is rounded as torch does.
#include "common.h"
#include "qkv_math.h"

using namespace acorn;

namespace {

constexpr int kMaxPairs = 2;  // head_dim <= 256 -> half <= 128 -> 2 pairs per lane

// One wavefront per row of head_dim values.
template <typename T, bool POS64>
__global__ __launch_bounds__(kWave) void rope_kernel(T* __restrict__ x, int heads, int D,
                                                     const void* __restrict__ pos,
                                                     const float* __restrict__ inv_freq) {
  const int row = blockIdx.x;
  const int b = row / heads;
  const float p = POS64 ? (float)((const int64_t*)pos)[b] : (float)((const int32_t*)pos)[b];
  T* base = x + (size_t)row * D;
  const int half = D / 2;
  for (int i = threadIdx.x; i < half; i += kWave) {
    float x1 = to_f32(base[i]), x2 = to_f32(base[i + half]);
    rope_pair<T>(x1, x2, p, inv_freq[i]);
    base[i] = from_f32<T>(x1);
    base[i + half] = from_f32<T>(x2);
  }
}

// The same, loading the weights and frequencies of the lane's pairs.
template <typename T, typename TW>
__device__ __forceinline__ void norm_rope_row(float (&x1)[kMaxPairs], float (&x2)[kMaxPairs],
                                              int half, const TW* __restrict__ w, float eps,
                                              float pos, const float* __restrict__ inv_freq) {
  float w1[kMaxPairs], w2[kMaxPairs], fr[kMaxPairs];
#pragma unroll
  for (int j = 0; j < kMaxPairs; ++j) {
    const int i = min(threadIdx.x + j * kWave, half - 1);
    w1[j] = to_f32(w[i]);
    w2[j] = to_f32(w[i + half]);
    fr[j] = inv_freq[i];
  }
  norm_rope_pre<T, kMaxPairs>(x1, x2, half, w1, w2, eps, pos, fr);
}

template <typename T, typename TW, bool POS64>
__global__ __launch_bounds__(kWave) void qknorm_rope_kernel(
    T* __restrict__ q, T* __restrict__ k, int q_heads, int kv_heads, int D,
    const TW* __restrict__ q_w, const TW* __restrict__ k_w, float eps,
    const void* __restrict__ pos, const float* __restrict__ inv_freq) {
  const int rows_per_b = q_heads + kv_heads;
  const int b = blockIdx.x / rows_per_b;
  const int h = blockIdx.x % rows_per_b;
  const bool is_q = h < q_heads;
  T* base = is_q ? q + ((size_t)b * q_heads + h) * D
                 : k + ((size_t)b * kv_heads + (h - q_heads)) * D;
  const TW* w = is_q ? q_w : k_w;
  const float p = POS64 ? (float)((const int64_t*)pos)[b] : (float)((const int32_t*)pos)[b];
  const int half = D / 2;
  float x1[kMaxPairs], x2[kMaxPairs];
#pragma unroll
  for (int j = 0; j < kMaxPairs; ++j) {
    const int i = threadIdx.x + j * kWave;
    x1[j] = i < half ? to_f32(base[i]) : 0.f;
    x2[j] = i < half ? to_f32(base[i + half]) : 0.f;
  }
  norm_rope_row<T, TW>(x1, x2, half, w, eps, p, inv_freq);
#pragma unroll
  for (int j = 0; j < kMaxPairs; ++j) {
    const int i = threadIdx.x + j * kWave;
    if (i < half) {
      base[i] = from_f32<T>(x1[j]);
      base[i + half] = from_f32<T>(x2[j]);
    }
  }
}

// Decode-step epilogue of the fused qkv projection. Rows per batch entry:
// [0, H) q heads, [H, H+KV) k heads, [H+KV, H+2KV) v heads. One wavefront per
// row, kEpiWaves rows per workgroup; lane pairs (i, i + half), NP per lane.
// Everything the row needs (the first kSplitBatch split partials of each
// element, the norm weights, the frequencies, the position and the page slot)
// is requested before any of it is used: one memory round trip (ONE: the
// partials are one plane, requested once). Indices past the row re-read its
// last pair (unconditional loads keep the wait counts static); those lanes
// store nothing. Partials are added in split order, as acorn::sum_splits does.
constexpr int kEpiWaves = 4;

template <typename T, typename TW, int NP, bool ONE>
__global__ __launch_bounds__(kEpiWaves * kWave) void qkv_epilogue_kernel(
    const float* __restrict__ part, int nsplit, T* __restrict__ q_out,
    T* __restrict__ k_pages, T* __restrict__ v_pages, const int64_t* __restrict__ pages,
    const int64_t* __restrict__ slots, int batch, int H, int KV, int D, int P,
    int64_t num_blocks, const TW* __restrict__ q_w, const TW* __restrict__ k_w, float eps,
    const int64_t* __restrict__ pos, const float* __restrict__ inv_freq) {
#pragma clang fp contract(off)
  const int rows_per_b = H + 2 * KV;
  const int lane = threadIdx.x & (kWave - 1);
  const int row = blockIdx.x * kEpiWaves + (int)(threadIdx.x / kWave);
  if (row >= batch * rows_per_b) return;      // whole waves
  const int b = row / rows_per_b;
  const int h = row % rows_per_b;
  const int half = D / 2;
  const size_t width = (size_t)rows_per_b * D;
  const size_t plane = (size_t)batch * width;
  const float* src = part + (size_t)b * width + (size_t)h * D;
  const TW* w = h < H ? q_w : k_w;  // v rows load them too, unused
  // ---- requests ----
  constexpr int NB = ONE ? 1 : kSplitBatch;
  float pa[NP][NB], pc[NP][NB], w1[NP], w2[NP], fr[NP];
#pragma unroll
  for (int j = 0; j < NP; ++j) {
    const int ic = min(lane + j * kWave, half - 1);
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const float* p = src + (size_t)min(u, nsplit - 1) * plane + ic;
      pa[j][u] = p[0];
      pc[j][u] = p[half];
    }
    w1[j] = to_f32(w[ic]);
    w2[j] = to_f32(w[ic + half]);
    fr[j] = inv_freq[ic];
  }
  const float p = (float)pos[b];
  const uint64_t page = (uint64_t)pages[b], slot = (uint64_t)slots[b];
  // ---- use ----
  float x1[NP], x2[NP];
#pragma unroll
  for (int j = 0; j < NP; ++j) {
    float a = pa[j][0], c = pc[j][0];
#pragma unroll
    for (int u = 1; u < NB; ++u) {
      if (u < nsplit) {
        a = a + pa[j][u];
        c = c + pc[j][u];
      }
    }
    const int ic = min(lane + j * kWave, half - 1);
    for (int sp = NB; sp < nsplit; ++sp) {
      const float* q = src + (size_t)sp * plane + ic;
      a = a + q[0];
      c = c + q[half];
    }
    x1[j] = round_to<T>(a);  // the projection's bf16 output
    x2[j] = round_to<T>(c);
  }
  T* dst = nullptr;
  if (h < H) {
    norm_rope_pre<T, NP>(x1, x2, half, w1, w2, eps, p, fr);
    dst = q_out + ((size_t)b * H + h) * D;
  } else {
    const int kvh = h < H + KV ? h - H : h - H - KV;
    // A (page, slot) outside the pool is dropped rather than written.
    const bool in_pool = page < (uint64_t)num_blocks && slot < (uint64_t)P;
    const size_t off = in_pool ? ((page * P + slot) * KV + kvh) * D : 0;
    if (h < H + KV) {
      norm_rope_pre<T, NP>(x1, x2, half, w1, w2, eps, p, fr);
      if (in_pool) dst = k_pages + off;
    } else {
      if (in_pool) dst = v_pages + off;
    }
  }
#pragma unroll
  for (int j = 0; j < NP; ++j) {
    const int i = lane + j * kWave;
    if (dst && i < half) {
      dst[i] = from_f32<T>(x1[j]);
      dst[i + half] = from_f32<T>(x2[j]);
    }
  }
}

// Prefill sizes (one split, head_dim 128): one wavefront per token row, lane
// i owning pair (i, i + 64) of every head, so the row's cos/sin (the same for
// all of its q and k heads) are computed once per row instead of once per
// head; the heads' partials are requested 8 heads at a time. The same
// arithmetic as qkv_epilogue_kernel, so the same bits.
constexpr int kRowHeads = 8;
constexpr int64_t kEpiRowsMin = 256;   // token rows from which the row form is used

template <typename T, typename TW, typename PT>
__global__ __launch_bounds__(kEpiWaves * kWave) void qkv_epilogue_rows_kernel(
    const PT* __restrict__ part, T* __restrict__ q_out, T* __restrict__ k_pages,
    T* __restrict__ v_pages, const int64_t* __restrict__ pages,
    const int64_t* __restrict__ slots, int batch, int H, int KV, int P, int64_t num_blocks,
    const TW* __restrict__ q_w, const TW* __restrict__ k_w, float eps,
    const int64_t* __restrict__ pos, const float* __restrict__ inv_freq) {
#pragma clang fp contract(off)
  constexpr int D = 128, HALF = 64;
  const int lane = threadIdx.x & (kWave - 1);
  const int b = blockIdx.x * kEpiWaves + (int)(threadIdx.x / kWave);
  if (b >= batch) return;                     // whole waves
  const int NH = H + 2 * KV;
  const PT* src = part + (size_t)b * NH * D + lane;
  float cs[1], sn[1];
  rope_cs<T>((float)pos[b], inv_freq[lane], cs[0], sn[0]);
  const float qw1[1] = {to_f32(q_w[lane])}, qw2[1] = {to_f32(q_w[lane + HALF])};
  const float kw1[1] = {to_f32(k_w[lane])}, kw2[1] = {to_f32(k_w[lane + HALF])};
  const uint64_t page = (uint64_t)pages[b], slot = (uint64_t)slots[b];
  // a (page, slot) outside the pool is dropped rather than written
  const bool in_pool = page < (uint64_t)num_blocks && slot < (uint64_t)P;
  const size_t kv_off = in_pool ? (page * P + slot) * KV * D : 0;
  for (int h0 = 0; h0 < NH; h0 += kRowHeads) {
    float a[kRowHeads], c[kRowHeads];
#pragma unroll
    for (int u = 0; u < kRowHeads; ++u) {
      const PT* p = src + (size_t)min(h0 + u, NH - 1) * D;
      a[u] = to_f32(p[0]);
      c[u] = to_f32(p[HALF]);
    }
#pragma unroll
    for (int u = 0; u < kRowHeads; ++u) {
      const int h = h0 + u;
      if (h >= NH) break;                       // uniform
      float x1[1] = {round_to<T>(a[u])}, x2[1] = {round_to<T>(c[u])};
      T* dst;
      if (h < H) {
        norm_rope_cs<T, 1>(x1, x2, HALF, qw1, qw2, eps, cs, sn);
        dst = q_out + ((size_t)b * H + h) * D;
      } else if (h < H + KV) {
        norm_rope_cs<T, 1>(x1, x2, HALF, kw1, kw2, eps, cs, sn);
        dst = in_pool ? k_pages + kv_off + (size_t)(h - H) * D : nullptr;
      } else {
        dst = in_pool ? v_pages + kv_off + (size_t)(h - H - KV) * D : nullptr;
      }
      if (dst) {
        dst[lane] = from_f32<T>(x1[0]);
        dst[lane + HALF] = from_f32<T>(x2[0]);
      }
    }
  }
}

bool head_dim_ok(int64_t D) { return D >= 2 && D <= 2 * kMaxPairs * kWave && (D & (D - 1)) == 0; }

template <typename T>
int launch_rope(void* x, int64_t batch, int64_t heads, int64_t D, const void* pos, int pos64,
                const float* inv_freq, hipStream_t st) {
  dim3 grid((unsigned)(batch * heads)), block(kWave);
  if (pos64)
    rope_kernel<T, true><<<grid, block, 0, st>>>((T*)x, (int)heads, (int)D, pos, inv_freq);
  else
    rope_kernel<T, false><<<grid, block, 0, st>>>((T*)x, (int)heads, (int)D, pos, inv_freq);
  ACORN_LAUNCH_CHECK();
  return ACORN_OK;
}

template <typename T, typename TW>
int launch_qknorm(void* q, void* k, int64_t batch, int64_t H, int64_t KV, int64_t D,
                  const void* qw, const void* kw, float eps, const void* pos, int pos64,
                  const float* inv_freq, hipStream_t st) {
  dim3 grid((unsigned)(batch * (H + KV))), block(kWave);
  if (pos64)
    qknorm_rope_kernel<T, TW, true><<<grid, block, 0, st>>>(
        (T*)q, (T*)k, (int)H, (int)KV, (int)D, (const TW*)qw, (const TW*)kw, eps, pos, inv_freq);
  else
    qknorm_rope_kernel<T, TW, false><<<grid, block, 0, st>>>(
        (T*)q, (T*)k, (int)H, (int)KV, (int)D, (const TW*)qw, (const TW*)kw, eps, pos, inv_freq);
  ACORN_LAUNCH_CHECK();
  return ACORN_OK;
}

template <typename T, typename TW>
int launch_qkv(const float* part, int64_t nsplit, void* q_out, void* kp, void* vp,
               const int64_t* pages, const int64_t* slots, int64_t batch, int64_t H, int64_t KV,
               int64_t D, int64_t P, int64_t NB, const void* qw, const void* kw, float eps,
               const int64_t* pos, const float* inv_freq, hipStream_t st) {
  // nsplit == 0: part holds the projection's output in T (one rounded plane)
  if (nsplit == 0 && (D != 128 || batch < kEpiRowsMin)) return ACORN_ERR_UNSUPPORTED;
  if (nsplit <= 1 && D == 128 && batch >= kEpiRowsMin) {
    const dim3 grid((unsigned)((batch + kEpiWaves - 1) / kEpiWaves)), block(kEpiWaves * kWave);
    if (nsplit == 0)
      qkv_epilogue_rows_kernel<T, TW, T><<<grid, block, 0, st>>>(
          (const T*)part, (T*)q_out, (T*)kp, (T*)vp, pages, slots, (int)batch, (int)H, (int)KV,
          (int)P, NB, (const TW*)qw, (const TW*)kw, eps, pos, inv_freq);
    else
      qkv_epilogue_rows_kernel<T, TW, float><<<grid, block, 0, st>>>(
          part, (T*)q_out, (T*)kp, (T*)vp, pages, slots, (int)batch, (int)H, (int)KV, (int)P,
          NB, (const TW*)qw, (const TW*)kw, eps, pos, inv_freq);
    ACORN_LAUNCH_CHECK();
    return ACORN_OK;
  }
  const int64_t rows = batch * (H + 2 * KV);
  dim3 grid((unsigned)((rows + kEpiWaves - 1) / kEpiWaves)), block(kEpiWaves * kWave);
  auto kfn = D <= 2 * kWave ? (nsplit == 1 ? qkv_epilogue_kernel<T, TW, 1, true>
                                           : qkv_epilogue_kernel<T, TW, 1, false>)
                            : (nsplit == 1 ? qkv_epilogue_kernel<T, TW, kMaxPairs, true>
                                           : qkv_epilogue_kernel<T, TW, kMaxPairs, false>);
  kfn<<<grid, block, 0, st>>>(
      part, (int)nsplit, (T*)q_out, (T*)kp, (T*)vp, pages, slots, (int)batch, (int)H, (int)KV,
      (int)D, (int)P, NB, (const TW*)qw, (const TW*)kw, eps, pos, inv_freq);
  ACORN_LAUNCH_CHECK();
  return ACORN_OK;
}

#define ACORN_DISPATCH_T(dtype, FN, ...)                 \
  switch (dtype) {                                       \
    case ACORN_F32: return FN<float>(__VA_ARGS__);       \
    case ACORN_F16: return FN<_Float16>(__VA_ARGS__);    \
    case ACORN_BF16: return FN<__bf16>(__VA_ARGS__);     \
  }                                                      \
  return ACORN_ERR_DTYPE;

#define ACORN_DISPATCH_TW(dtype, wdtype, FN, ...)                                   \
  switch (dtype * 3 + wdtype) {                                                     \
    case ACORN_F32 * 3 + ACORN_F32: return FN<float, float>(__VA_ARGS__);           \
    case ACORN_F32 * 3 + ACORN_F16: return FN<float, _Float16>(__VA_ARGS__);        \
    case ACORN_F32 * 3 + ACORN_BF16: return FN<float, __bf16>(__VA_ARGS__);         \
    case ACORN_F16 * 3 + ACORN_F32: return FN<_Float16, float>(__VA_ARGS__);        \
    case ACORN_F16 * 3 + ACORN_F16: return FN<_Float16, _Float16>(__VA_ARGS__);     \
    case ACORN_F16 * 3 + ACORN_BF16: return FN<_Float16, __bf16>(__VA_ARGS__);      \
    case ACORN_BF16 * 3 + ACORN_F32: return FN<__bf16, float>(__VA_ARGS__);         \
    case ACORN_BF16 * 3 + ACORN_F16: return FN<__bf16, _Float16>(__VA_ARGS__);      \
    case ACORN_BF16 * 3 + ACORN_BF16: return FN<__bf16, __bf16>(__VA_ARGS__);       \
  }                                                                                 \
  return ACORN_ERR_DTYPE;

}  // namespace

extern "C" int acorn_rope_inplace(void* x, int64_t batch, int64_t heads, int64_t head_dim,
                                  const void* positions, int pos_is_i64, const float* inv_freq,
                                  int dtype, void* stream) {
  if (batch < 0 || heads < 0 || !head_dim_ok(head_dim)) return ACORN_ERR_SHAPE;
  if (batch * heads == 0) return ACORN_OK;
  if (!x || !positions || !inv_freq) return ACORN_ERR_VALUE;
  ACORN_DISPATCH_T(dtype, launch_rope, x, batch, heads, head_dim, positions, pos_is_i64,
                   inv_freq, (hipStream_t)stream)
}

extern "C" int acorn_qknorm_rope_inplace(void* q, void* k, int64_t batch, int64_t q_heads,
                                         int64_t kv_heads, int64_t head_dim, const void* q_w,
                                         const void* k_w, float eps, const void* positions,
                                         int pos_is_i64, const float* inv_freq, int dtype,
                                         int wdtype, void* stream) {
  if (batch < 0 || q_heads < 0 || kv_heads < 0 || !head_dim_ok(head_dim)) return ACORN_ERR_SHAPE;
  if (batch * (q_heads + kv_heads) == 0) return ACORN_OK;
  if (!q || !k || !q_w || !k_w || !positions || !inv_freq) return ACORN_ERR_VALUE;
  ACORN_DISPATCH_TW(dtype, wdtype, launch_qknorm, q, k, batch, q_heads, kv_heads, head_dim, q_w,
                    k_w, eps, positions, pos_is_i64, inv_freq, (hipStream_t)stream)
}

extern "C" int acorn_qkv_epilogue(const float* part, int64_t nsplit, void* q_out, void* k_pages,
                                  void* v_pages, const int64_t* pages, const int64_t* slots,
                                  int64_t batch, int64_t q_heads, int64_t kv_heads,
                                  int64_t head_dim, int64_t page_size, int64_t num_blocks,
                                  const void* q_w,
                                  const void* k_w, float eps, const int64_t* positions,
                                  const float* inv_freq, int dtype, int wdtype, void* stream) {
  if (batch < 0 || q_heads <= 0 || kv_heads <= 0 || page_size <= 0 || num_blocks <= 0 ||
      nsplit < 0 || !head_dim_ok(head_dim))
    return ACORN_ERR_SHAPE;
  if (batch == 0) return ACORN_OK;
  if (!part || !q_out || !k_pages || !v_pages || !pages || !slots || !q_w || !k_w ||
      !positions || !inv_freq)
    return ACORN_ERR_VALUE;
  ACORN_DISPATCH_TW(dtype, wdtype, launch_qkv, part, nsplit, q_out, k_pages, v_pages, pages,
                    slots, batch, q_heads, kv_heads, head_dim, page_size, num_blocks, q_w, k_w, eps,
                    positions, inv_freq, (hipStream_t)stream)
}
