// Small kernels of the decode step: embedding gather, SwiGLU activation and
// greedy argmax.
//
//  * embedding: out[b, :] = table[ids[b], :]   (models/qwen3.py:585, nn.Embedding)
//  * silu_mul : act = r(r(silu(r(g))) * r(u)) where g/u are the gate/up halves
//               of the fused gate|up projection, summed over its split-K
//               partials in split order (models/qwen3.py:392-396:
//               F.silu(gate(x)) * up(x), every bf16 op rounded).
//  * argmax   : first index of the maximum of each row (torch.argmax,
//               engine/graph_runner.py:177); NaN compares greater than every
//               number, as in torch.
#include <algorithm>

#include "common.h"

using namespace acorn;

namespace {

// ---- embedding ------------------------------------------------------------
// One workgroup per row; 16-byte vector copies.
template <typename T>
__global__ __launch_bounds__(256) void embedding_kernel(const T* __restrict__ table,
                                                        const int64_t* __restrict__ ids,
                                                        T* __restrict__ out, int64_t vocab,
                                                        int cols) {
  const int b = blockIdx.x;
  int64_t id = ids[b];
  if (id < 0 || id >= vocab) id = 0;  // out-of-range ids read row 0, never past the table
  const T* src = table + id * cols;
  T* dst = out + (size_t)b * cols;
  constexpr int V = 16 / sizeof(T);
  if (cols % V == 0) {
    for (int i = threadIdx.x * V; i < cols; i += blockDim.x * V)
      *(uint4*)(dst + i) = *(const uint4*)(src + i);
  } else {
    for (int i = threadIdx.x; i < cols; i += blockDim.x) dst[i] = src[i];
  }
}

// ---- SwiGLU ----------------------------------------------------------------
template <typename T>
__device__ __forceinline__ float silu_r(float g) {
#pragma clang fp contract(off)
  // torch evaluates silu(x) as x / (1 + exp(-x)) in fp32 and rounds once.
  return round_to<T>(g / (1.0f + expf(-g)));
}

// part: [nsplit, rows, 2*inter] fp32 or NULL; gu: [rows, 2*inter] T when
// part is NULL. Columns are gate-first ([gate | up]) or, with il16, in
// 16-column blocks alternating gate and up. act: [rows, inter].
template <typename T>
__global__ __launch_bounds__(256) void silu_mul_kernel(const float* __restrict__ part,
                                                       int nsplit, const T* __restrict__ gu,
                                                       T* __restrict__ act, int rows,
                                                       int inter, int il16) {
#pragma clang fp contract(off)
  const size_t n = (size_t)rows * inter;
  const size_t plane = (size_t)rows * 2 * inter;
  for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < n;
       e += (size_t)gridDim.x * blockDim.x) {
    const size_t r = e / inter, i = e % inter;
    const size_t gi = r * 2 * inter + (il16 ? (i / 16) * 32 + i % 16 : i);
    const size_t ui = gi + (il16 ? 16 : inter);
    float g, u;
    if (part) {
      g = sum_splits(part + gi, plane, nsplit);
      u = sum_splits(part + ui, plane, nsplit);
      g = round_to<T>(g);
      u = round_to<T>(u);
    } else {
      g = to_f32(gu[gi]);
      u = to_f32(gu[ui]);
    }
    act[e] = from_f32<T>(silu_r<T>(g) * u);
  }
}

// ---- argmax ----------------------------------------------------------------
// (value, index) ordering: larger value wins, NaN beats numbers, ties go to
// the smaller index.
__device__ __forceinline__ bool better(float v, int64_t i, float bv, int64_t bi) {
  const bool vn = v != v, bn = bv != bv;
  if (vn != bn) return vn;
  if (!vn && v != bv) return v > bv;
  return i < bi;
}

constexpr int kArgNT = 1024;

template <typename T>
__global__ __launch_bounds__(kArgNT) void argmax_kernel(const T* __restrict__ x,
                                                        int64_t cols,
                                                        int64_t* __restrict__ out) {
  __shared__ float sv[kArgNT / kWave];
  __shared__ int64_t si[kArgNT / kWave];
  const T* row = x + (size_t)blockIdx.x * cols;
  float bv = -INFINITY;
  int64_t bi = INT64_MAX;
  for (int64_t i = threadIdx.x; i < cols; i += kArgNT) {
    const float v = to_f32(row[i]);
    if (better(v, i, bv, bi)) {
      bv = v;
      bi = i;
    }
  }
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int64_t oi = __shfl_xor(bi, o);
    if (better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  const int lane = threadIdx.x % kWave, wid = threadIdx.x / kWave;
  if (lane == 0) {
    sv[wid] = bv;
    si[wid] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kArgNT / kWave; ++w)
      if (better(sv[w], si[w], bv, bi)) {
        bv = sv[w];
        bi = si[w];
      }
    out[blockIdx.x] = bi == INT64_MAX ? 0 : bi;
  }
}


// ---- KV scatter ------------------------------------------------------------
// k/v: [B, KV, D]; pages: [NB, P, KV, D]. One workgroup per (b, kv head).
template <typename T>
__global__ __launch_bounds__(64) void kv_scatter_kernel(
    const T* __restrict__ k, const T* __restrict__ v, T* __restrict__ k_pages,
    T* __restrict__ v_pages, const int64_t* __restrict__ pages,
    const int64_t* __restrict__ slots, int KV, int D, int P, int64_t num_blocks) {
  const int b = blockIdx.x / KV, h = blockIdx.x % KV;
  const uint64_t page = (uint64_t)pages[b], slot = (uint64_t)slots[b];
  if (page >= (uint64_t)num_blocks || slot >= (uint64_t)P) return;  // outside the pool
  const size_t src = ((size_t)b * KV + h) * D;
  const size_t dst = ((page * P + slot) * KV + h) * D;
  for (int i = threadIdx.x; i < D; i += blockDim.x) {
    k_pages[dst + i] = k[src + i];
    v_pages[dst + i] = v[src + i];
  }
}

}  // namespace

extern "C" int acorn_embedding(const void* table, const int64_t* ids, void* out, int64_t rows,
                               int64_t vocab, int64_t cols, int dtype, void* stream) {
  if (rows < 0 || vocab <= 0 || cols <= 0 || rows > 0x7fffffff || cols > 0x7fffffff)
    return ACORN_ERR_SHAPE;
  if (rows == 0) return ACORN_OK;
  if (!table || !ids || !out) return ACORN_ERR_VALUE;
  hipStream_t st = (hipStream_t)stream;
  dim3 grid((unsigned)rows), block(256);
  switch (dtype) {
    case ACORN_F32:
      embedding_kernel<float><<<grid, block, 0, st>>>((const float*)table, ids, (float*)out, vocab, (int)cols);
      break;
    case ACORN_F16:
      embedding_kernel<_Float16><<<grid, block, 0, st>>>((const _Float16*)table, ids, (_Float16*)out, vocab, (int)cols);
      break;
    case ACORN_BF16:
      embedding_kernel<__bf16><<<grid, block, 0, st>>>((const __bf16*)table, ids, (__bf16*)out, vocab, (int)cols);
      break;
    default:
      return ACORN_ERR_DTYPE;
  }
  ACORN_LAUNCH_CHECK();
  return ACORN_OK;
}

extern "C" int acorn_silu_mul(const float* part, int64_t nsplit, const void* gate_up, void* act,
                              int64_t rows, int64_t inter, int interleaved16, int dtype,
                              void* stream) {
  if (rows < 0 || inter <= 0 || (part && nsplit < 1)) return ACORN_ERR_SHAPE;
  if (interleaved16 && inter % 16) return ACORN_ERR_SHAPE;
  if (rows * inter > ((int64_t)1 << 40)) return ACORN_ERR_SHAPE;
  if (rows == 0) return ACORN_OK;
  if (!act || (!part && !gate_up)) return ACORN_ERR_VALUE;
  hipStream_t st = (hipStream_t)stream;
  const int64_t n = rows * inter;
  const unsigned blocks = (unsigned)std::min<int64_t>((n + 255) / 256, 4096);
  switch (dtype) {
    case ACORN_F32:
      silu_mul_kernel<float><<<blocks, 256, 0, st>>>(part, (int)nsplit, (const float*)gate_up, (float*)act, (int)rows, (int)inter, interleaved16);
      break;
    case ACORN_F16:
      silu_mul_kernel<_Float16><<<blocks, 256, 0, st>>>(part, (int)nsplit, (const _Float16*)gate_up, (_Float16*)act, (int)rows, (int)inter, interleaved16);
      break;
    case ACORN_BF16:
      silu_mul_kernel<__bf16><<<blocks, 256, 0, st>>>(part, (int)nsplit, (const __bf16*)gate_up, (__bf16*)act, (int)rows, (int)inter, interleaved16);
      break;
    default:
      return ACORN_ERR_DTYPE;
  }
  ACORN_LAUNCH_CHECK();
  return ACORN_OK;
}

extern "C" int acorn_argmax(const void* x, int64_t rows, int64_t cols, int64_t* out, int dtype,
                            void* stream) {
  if (rows < 0 || cols <= 0 || rows > 0x7fffffff) return ACORN_ERR_SHAPE;
  if (rows == 0) return ACORN_OK;
  if (!x || !out) return ACORN_ERR_VALUE;
  hipStream_t st = (hipStream_t)stream;
  dim3 grid((unsigned)rows), block(kArgNT);
  switch (dtype) {
    case ACORN_F32: argmax_kernel<float><<<grid, block, 0, st>>>((const float*)x, cols, out); break;
    case ACORN_F16: argmax_kernel<_Float16><<<grid, block, 0, st>>>((const _Float16*)x, cols, out); break;
    case ACORN_BF16: argmax_kernel<__bf16><<<grid, block, 0, st>>>((const __bf16*)x, cols, out); break;
    default: return ACORN_ERR_DTYPE;
  }
  ACORN_LAUNCH_CHECK();
  return ACORN_OK;
}

extern "C" int acorn_kv_scatter(const void* k, const void* v, void* k_pages, void* v_pages,
                                const int64_t* pages, const int64_t* slots, int64_t batch,
                                int64_t kv_heads, int64_t head_dim, int64_t page_size,
                                int64_t num_blocks, int dtype, void* stream) {
  if (batch < 0 || kv_heads <= 0 || head_dim <= 0 || page_size <= 0 || num_blocks <= 0 ||
      batch * kv_heads > 0x7fffffff)
    return ACORN_ERR_SHAPE;
  if (batch == 0) return ACORN_OK;
  if (!k || !v || !k_pages || !v_pages || !pages || !slots) return ACORN_ERR_VALUE;
  hipStream_t st = (hipStream_t)stream;
  dim3 grid((unsigned)(batch * kv_heads)), block(64);
  const int KV = (int)kv_heads, D = (int)head_dim, P = (int)page_size;
  switch (dtype) {
    case ACORN_F32:
      kv_scatter_kernel<float><<<grid, block, 0, st>>>((const float*)k, (const float*)v, (float*)k_pages, (float*)v_pages, pages, slots, KV, D, P, num_blocks);
      break;
    case ACORN_F16:
      kv_scatter_kernel<_Float16><<<grid, block, 0, st>>>((const _Float16*)k, (const _Float16*)v, (_Float16*)k_pages, (_Float16*)v_pages, pages, slots, KV, D, P, num_blocks);
      break;
    case ACORN_BF16:
      kv_scatter_kernel<__bf16><<<grid, block, 0, st>>>((const __bf16*)k, (const __bf16*)v, (__bf16*)k_pages, (__bf16*)v_pages, pages, slots, KV, D, P, num_blocks);
      break;
    default:
      return ACORN_ERR_DTYPE;
  }
  ACORN_LAUNCH_CHECK();
  return ACORN_OK;
}
