// K1: fused residual add + RMSNorm, one workgroup per row.
//
// Numerics follow acorninfer/ops/rmsnorm.py:74-82 (the reference oracle):
//   r      = round_T(residual + x)            (fp32 add, one rounding)
//   normed = round_T((r * rsqrt(mean(r*r) + eps)) * w)   (fp32 throughout)
// with rsqrt computed as a correctly rounded 1/sqrt, and no FMA contraction so
// each product is rounded as torch rounds it.
#include "common.h"

using namespace acorn;

namespace {

constexpr int kNT = 256;     // threads per row
constexpr int kCache = 16;   // elements per thread kept in registers (4096 cols)

template <typename T, typename TW, bool HAS_RES, bool FROM_PART>
__global__ __launch_bounds__(kNT) void fused_add_rmsnorm_kernel(
    const T* __restrict__ x, const float* __restrict__ part, int nsplit,
    const T* __restrict__ res, T* __restrict__ res_out, const TW* __restrict__ w,
    T* __restrict__ normed, T* __restrict__ x_out, int rows, int cols, float eps) {
#pragma clang fp contract(off)
  __shared__ float red[kNT / kWave];
  const int row = blockIdx.x;
  const size_t base = (size_t)row * cols;
  const size_t plane = (size_t)rows * cols;

  auto load_x = [&](int i) -> float {
    if constexpr (FROM_PART) {
      float xr = round_to<T>(sum_splits(part + base + i, plane, nsplit));
      if (x_out) x_out[base + i] = from_f32<T>(xr);
      return xr;
    } else {
      return to_f32(x[base + i]);
    }
  };

  float v[kCache];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < kCache; ++j) {
    const int i = threadIdx.x + j * kNT;
    v[j] = 0.f;
    if (i < cols) {
      float a = load_x(i);
      if constexpr (HAS_RES) a = to_f32(res[base + i]) + a;
      const float r = round_to<T>(a);
      res_out[base + i] = from_f32<T>(r);
      v[j] = r;
      ss += r * r;
    }
  }
  for (int i = threadIdx.x + kCache * kNT; i < cols; i += kNT) {
    float a = load_x(i);
    if constexpr (HAS_RES) a = to_f32(res[base + i]) + a;
    const float r = round_to<T>(a);
    res_out[base + i] = from_f32<T>(r);
    ss += r * r;
  }
  ss = block_sum<kNT>(ss, red);
  const float inv = 1.0f / sqrtf(ss / (float)cols + eps);
#pragma unroll
  for (int j = 0; j < kCache; ++j) {
    const int i = threadIdx.x + j * kNT;
    if (i < cols) normed[base + i] = from_f32<T>((v[j] * inv) * to_f32(w[i]));
  }
  for (int i = threadIdx.x + kCache * kNT; i < cols; i += kNT) {
    // Re-read this thread's own store: program order makes it visible.
    const float r = to_f32(res_out[base + i]);
    normed[base + i] = from_f32<T>((r * inv) * to_f32(w[i]));
  }
}

// Vectorised form for cols % 8 == 0 and cols <= 8 * kVecNT * kVMax: each
// thread owns up to VM 8-element vectors of the row and requests every
// load it needs (weights, residual, and the first kPartBatch split partials,
// or x) before using any, so the row costs one memory round trip before the
// reduction. Vector indices past the row re-read its last vector (loads stay
// unconditional, which keeps the wait counts static); their results are not
// stored. Split partials are added in split order, as acorn::sum_splits does.
constexpr int kVecNT = 512;    // threads per row
constexpr int kVMax = 2;       // largest VM: cols <= 8192
constexpr int kPartBatch = 8;  // split partials requested per vector up front

template <typename T>
__device__ __forceinline__ void load8(const T* p, float (&v)[8]) {
  T t[8];
  __builtin_memcpy(t, p, sizeof(t));
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = to_f32(t[i]);
}
template <typename T>
__device__ __forceinline__ void store8(T* p, const float (&v)[8]) {
  T t[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) t[i] = from_f32<T>(v[i]);
  __builtin_memcpy(p, t, sizeof(t));
}

template <typename T, typename TW, bool HAS_RES, bool FROM_PART, int VM>
__global__ __launch_bounds__(kVecNT) void fused_add_rmsnorm_vec_kernel(
    const T* __restrict__ x, const float* __restrict__ part, int nsplit,
    const T* __restrict__ res, T* __restrict__ res_out, const TW* __restrict__ w,
    T* __restrict__ normed, T* __restrict__ x_out, int rows, int cols, float eps) {
#pragma clang fp contract(off)
  typedef float f8 __attribute__((ext_vector_type(8)));
  __shared__ float red[kVecNT / kWave];
  const size_t base = (size_t)blockIdx.x * cols;
  const size_t plane = (size_t)rows * cols;
  const int nvec = cols / 8;
  int vi[VM];
  size_t col[VM];
#pragma unroll
  for (int j = 0; j < VM; ++j) {
    vi[j] = threadIdx.x + j * kVecNT;
    col[j] = (size_t)min(vi[j], nvec - 1) * 8;
  }
  // ---- requests ----
  float wv[VM][8], rv[VM][8], a[VM][8];
  f8 pv[VM][kPartBatch];
#pragma unroll
  for (int j = 0; j < VM; ++j) {
    load8<TW>(w + col[j], wv[j]);
    if constexpr (HAS_RES) load8<T>(res + base + col[j], rv[j]);
    if constexpr (FROM_PART) {
#pragma unroll
      for (int u = 0; u < kPartBatch; ++u)
        pv[j][u] = *(const f8*)(part + (size_t)min(u, nsplit - 1) * plane + base + col[j]);
    } else {
      load8<T>(x + base + col[j], a[j]);
    }
  }
  // ---- use ----
  float v[VM][8];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < VM; ++j) {
    const bool own = vi[j] < nvec;
    if constexpr (FROM_PART) {
#pragma unroll
      for (int i = 0; i < 8; ++i) a[j][i] = pv[j][0][i];
#pragma unroll
      for (int u = 1; u < kPartBatch; ++u) {
        if (u < nsplit) {
#pragma unroll
          for (int i = 0; i < 8; ++i) a[j][i] = a[j][i] + pv[j][u][i];
        }
      }
      for (int sp = kPartBatch; sp < nsplit; ++sp) {
        const f8 q = *(const f8*)(part + (size_t)sp * plane + base + col[j]);
#pragma unroll
        for (int i = 0; i < 8; ++i) a[j][i] = a[j][i] + q[i];
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) a[j][i] = round_to<T>(a[j][i]);
      if (x_out && own) store8<T>(x_out + base + col[j], a[j]);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float t = a[j][i];
      if constexpr (HAS_RES) t = rv[j][i] + t;
      v[j][i] = round_to<T>(t);
      if (own) ss += v[j][i] * v[j][i];
    }
    if (own) store8<T>(res_out + base + col[j], v[j]);
  }
  ss = block_sum<kVecNT>(ss, red);
  const float inv = 1.0f / sqrtf(ss / (float)cols + eps);
#pragma unroll
  for (int j = 0; j < VM; ++j) {
    if (vi[j] < nvec) {
      float o[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = (v[j][i] * inv) * wv[j][i];
      store8<T>(normed + base + col[j], o);
    }
  }
}

template <typename T, typename TW>
int launch_k1(const void* x, const float* part, int nsplit, const void* res, void* res_out,
              const void* w, void* normed, void* x_out, int64_t rows, int64_t cols, float eps,
              hipStream_t st) {
  dim3 grid((unsigned)rows);
  const T* xp = (const T*)x;
  const T* rp = (const T*)res;
  T* rop = (T*)res_out;
  const TW* wp = (const TW*)w;
  T* np = (T*)normed;
  T* xo = (T*)x_out;
#define ACORN_K1(NT, ...)                                                                \
  __VA_ARGS__<<<grid, dim3(NT), 0, st>>>(xp, part, nsplit, rp, rop, wp, np, xo, (int)rows, \
                                        (int)cols, eps)
#define ACORN_K1_RP(NT, KERNEL, ...)                                  \
  do {                                                                \
    if (part) {                                                       \
      if (res) ACORN_K1(NT, KERNEL<T, TW, true, true __VA_ARGS__>);   \
      else ACORN_K1(NT, KERNEL<T, TW, false, true __VA_ARGS__>);      \
    } else {                                                          \
      if (res) ACORN_K1(NT, KERNEL<T, TW, true, false __VA_ARGS__>);  \
      else ACORN_K1(NT, KERNEL<T, TW, false, false __VA_ARGS__>);     \
    }                                                                 \
  } while (0)
  if (cols % 8 == 0 && cols <= 8 * kVecNT) {
    ACORN_K1_RP(kVecNT, fused_add_rmsnorm_vec_kernel, , 1);
  } else if (cols % 8 == 0 && cols <= 8 * kVecNT * kVMax) {
    ACORN_K1_RP(kVecNT, fused_add_rmsnorm_vec_kernel, , kVMax);
  } else {
    ACORN_K1_RP(kNT, fused_add_rmsnorm_kernel);
  }
#undef ACORN_K1_RP
#undef ACORN_K1
  ACORN_LAUNCH_CHECK();
  return ACORN_OK;
}

template <typename T>
int dispatch_w(int wdtype, const void* x, const float* part, int nsplit, const void* res,
               void* res_out, const void* w, void* normed, void* x_out, int64_t rows,
               int64_t cols, float eps, hipStream_t st) {
  switch (wdtype) {
    case ACORN_F32:
      return launch_k1<T, float>(x, part, nsplit, res, res_out, w, normed, x_out, rows, cols, eps, st);
    case ACORN_F16:
      return launch_k1<T, _Float16>(x, part, nsplit, res, res_out, w, normed, x_out, rows, cols, eps, st);
    case ACORN_BF16:
      return launch_k1<T, __bf16>(x, part, nsplit, res, res_out, w, normed, x_out, rows, cols, eps, st);
  }
  return ACORN_ERR_DTYPE;
}

int k1_entry(const void* x, const float* part, int64_t nsplit, const void* res, void* res_out,
             const void* w, void* normed, void* x_out, int64_t rows, int64_t cols, float eps,
             int dtype, int wdtype, void* stream) {
  if (rows < 0 || cols <= 0 || nsplit < 0) return ACORN_ERR_SHAPE;
  if (rows == 0) return ACORN_OK;
  if (rows > 0x7fffffff || cols > 0x7fffffff || rows * cols > ((int64_t)1 << 40))
    return ACORN_ERR_SHAPE;
  if (!res_out || !w || !normed || (!x && !part)) return ACORN_ERR_VALUE;
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case ACORN_F32:
      return dispatch_w<float>(wdtype, x, part, (int)nsplit, res, res_out, w, normed, x_out, rows, cols, eps, st);
    case ACORN_F16:
      return dispatch_w<_Float16>(wdtype, x, part, (int)nsplit, res, res_out, w, normed, x_out, rows, cols, eps, st);
    case ACORN_BF16:
      return dispatch_w<__bf16>(wdtype, x, part, (int)nsplit, res, res_out, w, normed, x_out, rows, cols, eps, st);
  }
  return ACORN_ERR_DTYPE;
}

}  // namespace

extern "C" int acorn_fused_add_rmsnorm(const void* x, const void* residual, void* residual_out,
                                       const void* weight, void* normed, int64_t rows,
                                       int64_t cols, float eps, int dtype, int wdtype,
                                       void* stream) {
  if (!x) return ACORN_ERR_VALUE;
  return k1_entry(x, nullptr, 0, residual, residual_out, weight, normed, nullptr, rows, cols,
                  eps, dtype, wdtype, stream);
}

extern "C" int acorn_fused_add_rmsnorm_partials(const float* part, int64_t nsplit,
                                                const void* residual, void* residual_out,
                                                const void* weight, void* normed, void* x_out,
                                                int64_t rows, int64_t cols, float eps, int dtype,
                                                int wdtype, void* stream) {
  if (!part || nsplit < 1) return ACORN_ERR_VALUE;
  return k1_entry(nullptr, part, nsplit, residual, residual_out, weight, normed, x_out, rows,
                  cols, eps, dtype, wdtype, stream);
}

extern "C" int acorn_version(void) { return 1; }
