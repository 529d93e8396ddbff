// K3: flash-decoding over the paged KV cache.
//
// Semantics follow acorninfer/ops/paged_attention.py:125-152 (kernel
// :33-122, oracle :192-216): for each (b, h) out = softmax(q . K^T * scale) V
// over tokens 0..L_b-1, token t stored at (tables[b, t/P], t%P), kv head
// h / (H/KV). Splits are page aligned: split sp covers pages
// [sp*pps, (sp+1)*pps) with pps = ceil(ceil(L/P)/S); an empty split writes
// (m=-inf, l=0, acc=0) and contributes nothing to the merge.
//
// MI355X design (not the reference's per-q-head grid):
//  * one wavefront per (split, kv head, sequence) serves all REP = H/KV query
//    heads, so every K/V byte is read from HBM once (GQA reuse);
//  * tokens are processed in chunks of 16: for q.k each token gets 4 lanes
//    (D/4 dims each, 16-byte loads, quad shuffle to finish the dot); for p.V
//    each lane owns D/64 output dims of every head and streams the chunk's 16
//    V rows with coalesced 4-byte loads, so no end-of-split lane reduction is
//    needed;
//  * the next chunk's K/V are loaded before the current chunk is consumed;
//  * scores live in the log2 domain (exp2), the workspace m is log2-domain.
#include "common.h"

using namespace acorn;

namespace {

constexpr int kChunk = 16;  // tokens per step
constexpr int kLPT = 4;     // lanes per token in the q.k phase
constexpr float kLog2e = 1.4426950408889634f;

template <typename T, int N>
struct Vec {
  T v[N];
};

template <typename T, int N>
__device__ __forceinline__ Vec<T, N> load_vec(const T* p) {
  Vec<T, N> r;
  __builtin_memcpy(&r, p, sizeof(r));
  return r;
}

template <typename T, int D, int REP>
__global__ __launch_bounds__(kWave) void paged_attn_split_kernel(
    const T* __restrict__ q, const T* __restrict__ k_pages, const T* __restrict__ v_pages,
    const int32_t* __restrict__ tables, const int32_t* __restrict__ lens, T* __restrict__ out,
    float* __restrict__ ws_acc, float* __restrict__ ws_m, float* __restrict__ ws_l, int H,
    int KV, int P, int num_blocks, int table_stride, int S, float scale_log2) {
  constexpr int DQ = D / kLPT;                 // q.k dims per lane
  constexpr int DPO = D >= kWave ? D / kWave : 1;  // p.V dims per lane
  constexpr bool kPVAll = D >= kWave;
  __shared__ float p_lds[kChunk][REP];

  const int sp = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int lane = threadIdx.x;
  const int tc = lane / kLPT, c = lane % kLPT;
  const bool pv_active = kPVAll || lane < D;
  const int d0 = kPVAll ? lane * DPO : lane;

  // Bounds guards: a length beyond the table row or a block id outside the
  // pool is clamped so that a malformed table can never read outside the
  // caller's buffers (valid inputs are unaffected).
  const int L = min(max(lens[b], 0), table_stride * P);
  const int npages = (L + P - 1) / P;
  const int pps = (npages + S - 1) / S;
  const int start = sp * pps * P;
  const int end = min(start + pps * P, L);
  const int32_t* trow = tables + (size_t)b * table_stride;
  const size_t tok_stride = (size_t)KV * D;  // elements between slots of a page

  // q for the REP heads of this kv head, this lane's D/4 dims, as fp32.
  float qf[REP][DQ];
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    const T* qp = q + ((size_t)b * H + kvh * REP + h) * D + c * DQ;
    Vec<T, DQ> qv = load_vec<T, DQ>(qp);
#pragma unroll
    for (int i = 0; i < DQ; ++i) qf[h][i] = to_f32(qv.v[i]) * scale_log2;
  }

  float m_run[REP], l_run[REP], acc[REP][DPO];
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    m_run[h] = -INFINITY;
    l_run[h] = 0.f;
#pragma unroll
    for (int i = 0; i < DPO; ++i) acc[h][i] = 0.f;
  }

  auto block_of = [&](int t) -> size_t {
    const unsigned page = (unsigned)trow[t / P];
    return page < (unsigned)num_blocks ? page : 0u;
  };
  auto k_addr = [&](int t) -> const T* {
    const size_t page = block_of(t);
    return k_pages + ((size_t)page * P + (t % P)) * tok_stride + (size_t)kvh * D + c * DQ;
  };
  auto v_addr = [&](int t) -> const T* {
    const size_t page = block_of(t);
    return v_pages + ((size_t)page * P + (t % P)) * tok_stride + (size_t)kvh * D + d0;
  };

  Vec<T, DQ> kcur, knxt;
  Vec<T, DPO> vcur[kChunk], vnxt[kChunk];
  auto load_chunk = [&](int t0, Vec<T, DQ>& kv, Vec<T, DPO>(&vv)[kChunk]) {
    const int t = t0 + tc;
    if (t < end) kv = load_vec<T, DQ>(k_addr(t));
#pragma unroll
    for (int j = 0; j < kChunk; ++j) {
      if (pv_active && t0 + j < end) vv[j] = load_vec<T, DPO>(v_addr(t0 + j));
    }
  };

  if (start < end) load_chunk(start, kcur, vcur);
  for (int t0 = start; t0 < end; t0 += kChunk) {
    const bool has_next = t0 + kChunk < end;
    if (has_next) load_chunk(t0 + kChunk, knxt, vnxt);

    // ---- scores for this lane's token, all REP heads --------------------
    const int t = t0 + tc;
    const bool valid = t < end;
    float s[REP];
#pragma unroll
    for (int h = 0; h < REP; ++h) {
      float a = 0.f;
#pragma unroll
      for (int i = 0; i < DQ; ++i) a += qf[h][i] * to_f32(kcur.v[i]);
      a += __shfl_xor(a, 1);
      a += __shfl_xor(a, 2);
      s[h] = valid ? a : -INFINITY;
    }
    // ---- online softmax (log2 domain) ----------------------------------
    float alpha[REP];
#pragma unroll
    for (int h = 0; h < REP; ++h) {
      float mx = s[h];
#pragma unroll
      for (int o = kLPT; o < kWave; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
      const float m_new = fmaxf(m_run[h], mx);  // finite: chunk holds >= 1 token
      alpha[h] = exp2f(m_run[h] - m_new);        // 0 on the first chunk
      m_run[h] = m_new;
      const float p = exp2f(s[h] - m_new);       // 0 for masked tokens
      l_run[h] = l_run[h] * alpha[h] + (c == 0 ? p : 0.f);
      if (c == 0) p_lds[tc][h] = p;
    }
    __syncthreads();
    // ---- acc = acc*alpha + p . V ----------------------------------------
#pragma unroll
    for (int h = 0; h < REP; ++h)
#pragma unroll
      for (int i = 0; i < DPO; ++i) acc[h][i] *= alpha[h];
    if (pv_active) {
#pragma unroll
      for (int j = 0; j < kChunk; ++j) {
        if (t0 + j < end) {
#pragma unroll
          for (int h = 0; h < REP; ++h) {
            const float p = p_lds[j][h];
#pragma unroll
            for (int i = 0; i < DPO; ++i) acc[h][i] += p * to_f32(vcur[j].v[i]);
          }
        }
      }
    }
    __syncthreads();
    if (has_next) {
      kcur = knxt;
#pragma unroll
      for (int j = 0; j < kChunk; ++j) vcur[j] = vnxt[j];
    }
  }

  // ---- write this split's partial (or the final output when S == 1) ------
#pragma unroll
  for (int h = 0; h < REP; ++h) l_run[h] = wave_sum(l_run[h]);
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    const int hq = kvh * REP + h;
    const size_t row = (size_t)b * H + hq;
    if (S == 1) {
      // start < end always holds for S == 1 (L >= 1).
      const float inv = 1.0f / l_run[h];
      if (pv_active) {
#pragma unroll
        for (int i = 0; i < DPO; ++i) out[row * D + d0 + i] = from_f32<T>(acc[h][i] * inv);
      }
    } else {
      const size_t slot = row * S + sp;
      if (pv_active) {
#pragma unroll
        for (int i = 0; i < DPO; ++i) ws_acc[slot * D + d0 + i] = acc[h][i];
      }
      if (lane == 0) {
        ws_m[slot] = m_run[h];
        ws_l[slot] = l_run[h];
      }
    }
  }
}

// Phase 2: merge S partials of one (b, h) with the common max.
template <typename T, int D>
__global__ __launch_bounds__(kWave) void paged_attn_combine_kernel(
    const float* __restrict__ ws_acc, const float* __restrict__ ws_m,
    const float* __restrict__ ws_l, T* __restrict__ out, int S) {
  const size_t row = blockIdx.x;
  const int lane = threadIdx.x;
  float mx = -INFINITY;
  for (int s = lane; s < S; s += kWave) mx = fmaxf(mx, ws_m[row * S + s]);
  mx = wave_max(mx);  // finite: split 0 is never empty (L >= 1)
  float lsum = 0.f;
  for (int s = lane; s < S; s += kWave) lsum += exp2f(ws_m[row * S + s] - mx) * ws_l[row * S + s];
  lsum = wave_sum(lsum);
  const float inv = 1.0f / lsum;
  for (int d = lane; d < D; d += kWave) {
    float a = 0.f;
    for (int s = 0; s < S; ++s) a += exp2f(ws_m[row * S + s] - mx) * ws_acc[(row * S + s) * D + d];
    out[row * D + d] = from_f32<T>(a * inv);
  }
}

template <typename T, int D, int REP>
int launch_attn(const void* q, const void* kp, const void* vp, const int32_t* tables,
                const int32_t* lens, void* out, float* ws_acc, float* ws_ml, int64_t B,
                int64_t H, int64_t KV, int64_t P, int64_t num_blocks, int64_t table_stride, int64_t S, float scale,
                hipStream_t st) {
  dim3 grid((unsigned)S, (unsigned)KV, (unsigned)B), block(kWave);
  float* ws_m = ws_ml;
  float* ws_l = ws_ml ? ws_ml + B * H * S : nullptr;
  paged_attn_split_kernel<T, D, REP><<<grid, block, 0, st>>>(
      (const T*)q, (const T*)kp, (const T*)vp, tables, lens, (T*)out, ws_acc, ws_m, ws_l,
      (int)H, (int)KV, (int)P, (int)num_blocks, (int)table_stride, (int)S, scale * kLog2e);
  ACORN_LAUNCH_CHECK();
  if (S > 1) {
    paged_attn_combine_kernel<T, D><<<dim3((unsigned)(B * H)), dim3(kWave), 0, st>>>(
        ws_acc, ws_m, ws_l, (T*)out, (int)S);
    ACORN_LAUNCH_CHECK();
  }
  return ACORN_OK;
}

template <typename T, int D>
int dispatch_rep(int64_t rep, const void* q, const void* kp, const void* vp,
                 const int32_t* tables, const int32_t* lens, void* out, float* ws_acc,
                 float* ws_ml, int64_t B, int64_t H, int64_t KV, int64_t P, int64_t num_blocks, int64_t ts,
                 int64_t S, float scale, hipStream_t st) {
  switch (rep) {
    case 1: return launch_attn<T, D, 1>(q, kp, vp, tables, lens, out, ws_acc, ws_ml, B, H, KV, P, num_blocks, ts, S, scale, st);
    case 2: return launch_attn<T, D, 2>(q, kp, vp, tables, lens, out, ws_acc, ws_ml, B, H, KV, P, num_blocks, ts, S, scale, st);
    case 4: return launch_attn<T, D, 4>(q, kp, vp, tables, lens, out, ws_acc, ws_ml, B, H, KV, P, num_blocks, ts, S, scale, st);
    case 8: return launch_attn<T, D, 8>(q, kp, vp, tables, lens, out, ws_acc, ws_ml, B, H, KV, P, num_blocks, ts, S, scale, st);
  }
  return ACORN_ERR_UNSUPPORTED;
}

template <typename T>
int dispatch_d(int64_t D, int64_t rep, const void* q, const void* kp, const void* vp,
               const int32_t* tables, const int32_t* lens, void* out, float* ws_acc,
               float* ws_ml, int64_t B, int64_t H, int64_t KV, int64_t P, int64_t num_blocks, int64_t ts,
               int64_t S, float scale, hipStream_t st) {
  switch (D) {
    case 16: return dispatch_rep<T, 16>(rep, q, kp, vp, tables, lens, out, ws_acc, ws_ml, B, H, KV, P, num_blocks, ts, S, scale, st);
    case 32: return dispatch_rep<T, 32>(rep, q, kp, vp, tables, lens, out, ws_acc, ws_ml, B, H, KV, P, num_blocks, ts, S, scale, st);
    case 64: return dispatch_rep<T, 64>(rep, q, kp, vp, tables, lens, out, ws_acc, ws_ml, B, H, KV, P, num_blocks, ts, S, scale, st);
    case 128: return dispatch_rep<T, 128>(rep, q, kp, vp, tables, lens, out, ws_acc, ws_ml, B, H, KV, P, num_blocks, ts, S, scale, st);
  }
  return ACORN_ERR_UNSUPPORTED;
}

}  // namespace

extern "C" int acorn_paged_attention(const void* q, const void* k_pages, const void* v_pages,
                                     const int32_t* tables, const int32_t* seq_lens, void* out,
                                     float* ws_acc, float* ws_ml, int64_t B, int64_t H,
                                     int64_t KV, int64_t D, int64_t P, int64_t num_blocks,
                                     int64_t table_stride, int64_t num_splits, float scale,
                                     int dtype, void* stream) {
  if (B < 0 || H <= 0 || KV <= 0 || D <= 0 || P <= 0 || num_blocks <= 0 || num_splits < 1 ||
      table_stride < 1)
    return ACORN_ERR_SHAPE;
  if ((D & (D - 1)) != 0 || (P & (P - 1)) != 0 || H % KV != 0) return ACORN_ERR_SHAPE;
  if (num_splits > 65535 || KV > 65535 || B > 65535) return ACORN_ERR_SHAPE;
  if (B == 0) return ACORN_OK;
  if (!q || !k_pages || !v_pages || !tables || !seq_lens || !out) return ACORN_ERR_VALUE;
  if (num_splits > 1 && (!ws_acc || !ws_ml)) return ACORN_ERR_VALUE;
  const int64_t rep = H / KV;
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case ACORN_F32: return dispatch_d<float>(D, rep, q, k_pages, v_pages, tables, seq_lens, out, ws_acc, ws_ml, B, H, KV, P, num_blocks, table_stride, num_splits, scale, st);
    case ACORN_F16: return dispatch_d<_Float16>(D, rep, q, k_pages, v_pages, tables, seq_lens, out, ws_acc, ws_ml, B, H, KV, P, num_blocks, table_stride, num_splits, scale, st);
    case ACORN_BF16: return dispatch_d<__bf16>(D, rep, q, k_pages, v_pages, tables, seq_lens, out, ws_acc, ws_ml, B, H, KV, P, num_blocks, table_stride, num_splits, scale, st);
  }
  return ACORN_ERR_DTYPE;
}
