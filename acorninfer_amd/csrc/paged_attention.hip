// K3: flash-decoding over the paged KV cache.
//
// Semantics follow acorninfer/ops/paged_attention.py:125-152 (kernel
// :33-122, oracle :192-216): for each (b, h) out = softmax(q . K^T * scale) V
// over tokens 0..L_b-1, token t stored at (tables[b, t/P], t%P), kv head
// h / (H/KV). Splits are page aligned and of one size per launch: split sp
// covers pages [sp*pps, (sp+1)*pps) with pps = ceil(table_stride / S), so a
// sequence uses nsb = ceil(ceil(L/P) / pps) splits and every workgroup has at
// most the same pps pages of work. Splits past nsb exit at once; a sequence
// with nsb = 1 gets its output written directly, the others' partials
// (log2-domain max m, sum l, unnormalised acc) are merged by the combine
// kernel.
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
#include <mutex>
#include <type_traits>

#include "common.h"
#include "qkv_math.h"

using namespace acorn;

namespace {

constexpr int kChunk = 16;  // tokens per step
constexpr int kLPT = 4;     // lanes per token in the q.k phase
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kAttnWaves = 8;  // waves per workgroup of the single-kernel form
constexpr int64_t kCUs = 256;   // MI355X compute units (the head-group rule)
constexpr int kOneWavePages = 16;  // MFMA form: splits of at most this many pages use one wave
#ifndef ACORN_K3_ONE_WAVE_DEPTH
#define ACORN_K3_ONE_WAVE_DEPTH 3
#endif
constexpr int kOneWaveDepth = ACORN_K3_ONE_WAVE_DEPTH;  // chunks in flight per one-wave split

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
  const int pps = (table_stride + S - 1) / S;            // pages per split
  const int nsb = max(1, (npages + pps - 1) / pps);      // splits this sequence uses
  if (sp >= nsb) return;
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

  // ---- write this split's partial (or the final output for one split) ----
#pragma unroll
  for (int h = 0; h < REP; ++h) l_run[h] = wave_sum(l_run[h]);
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    const int hq = kvh * REP + h;
    const size_t row = (size_t)b * H + hq;
    if (nsb == 1) {
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

// ---------------------------------------------------------------------------
// Single-kernel form for D in {64, 128} (the Qwen3 head size): one
// workgroup of NWV waves per (split, kv head, sequence). The waves divide the
// workgroup's pages; inside a wave a token's D values are spread over D/8
// lanes (8 values, one 16-byte load for bf16, per lane), so a 16-token chunk
// costs each lane D/32 loads of K and of V. The next chunk's K/V are loaded
// into the second register set while the current chunk is processed. The
// workgroup's block-table entries are staged in LDS first. At the end the
// waves' (m, l, acc) are merged in LDS and the output (or, with S > 1
// workgroup splits, this split's partial for the combine kernel) is written.
template <typename T>
struct V8 {
  T v[8];
};

// DPP lane permutations within a row of 16 lanes (gfx9 encodings).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
// Sum over groups of N lanes (N in {2, 4, 8, 16}, aligned within a row of
// 16); every lane of the group receives the sum.
template <int N>
__device__ __forceinline__ float group_sum(float v) {
  v += dpp<0xB1>(v);                      // quad_perm [1,0,3,2]: lane ^ 1
  if constexpr (N >= 4) v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]: lane ^ 2
  if constexpr (N >= 8) v += dpp<0x141>(v);  // row_half_mirror: lane i <- 7-i
  if constexpr (N >= 16) v += dpp<0x140>(v); // row_mirror: lane i <- 15-i
  return v;
}

template <typename T>
__device__ __forceinline__ void load8f(const T* p, float (&f)[8]) {
  V8<T> r;
  __builtin_memcpy(&r, p, sizeof(r));
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = to_f32(r.v[i]);
}

template <typename T, int D, int REP, int NWV>
__global__ __launch_bounds__(NWV * kWave) void paged_attn_wg_kernel(
    const T* __restrict__ q, const T* __restrict__ k_pages, const T* __restrict__ v_pages,
    const int32_t* __restrict__ tables, const int32_t* __restrict__ lens, T* __restrict__ out,
    float* __restrict__ ws_acc, float* __restrict__ ws_m, float* __restrict__ ws_l, int H,
    int KV, int P, int num_blocks, int table_stride, int S, float scale_log2) {
  constexpr int LPT = D / 8;                   // lanes per token
  constexpr int TR = kWave / LPT;              // tokens per wave-wide load
  constexpr int CH = 16;                       // tokens per chunk
  constexpr int NL = CH / TR;                  // loads per lane per chunk
  static_assert(NL >= 1, "D too small for this kernel");
  extern __shared__ __align__(16) unsigned char smem[];
  float* sacc = (float*)smem;                  // [NWV][REP][D]
  float* sm = sacc + NWV * REP * D;            // [NWV][REP]
  float* sl = sm + NWV * REP;                  // [NWV][REP]
  int* tbl = (int*)(sl + NWV * REP);           // this workgroup's block ids

  const int sp = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int wid = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int g = lane / LPT, c = lane % LPT;

  const int L = min(max(lens[b], 0), table_stride * P);
  const int npages = (L + P - 1) / P;
  const int pps = (table_stride + S - 1) / S;            // pages per split
  const int nsb = max(1, (npages + pps - 1) / pps);      // splits this sequence uses
  if (sp >= nsb) return;                                 // uniform over the workgroup
  const int wp0 = sp * pps, wp1 = min(wp0 + pps, npages);
  const int32_t* trow = tables + (size_t)b * table_stride;
  for (int i = threadIdx.x; i < wp1 - wp0; i += NWV * kWave) {
    const unsigned pg = (unsigned)trow[wp0 + i];
    tbl[i] = pg < (unsigned)num_blocks ? (int)pg : 0;
  }
  // this wave's pages and tokens
  const int ppv = (wp1 - wp0 + NWV - 1) / NWV;
  const int vp0 = min(wp0 + wid * ppv, wp1), vp1 = min(vp0 + ppv, wp1);
  const int tstart = vp0 * P, tend = min(vp1 * P, L);

  float qf[REP][8];
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    load8f<T>(q + ((size_t)b * H + kvh * REP + h) * D + c * 8, qf[h]);
#pragma unroll
    for (int i = 0; i < 8; ++i) qf[h][i] *= scale_log2;
  }
  float m[REP], l[REP], acc[REP][8];
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[h][i] = 0.f;
  }
  __syncthreads();  // tbl ready

  const size_t tok_stride = (size_t)KV * D;
  // Raw (unconverted) chunk registers; tokens past the end are zero so that
  // p = 0 multiplies a finite value.
  auto load_chunk = [&](int t0, V8<T> (&kr)[NL], V8<T> (&vr)[NL]) {
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int t = t0 + g + TR * i;
      if (t < tend) {
        const size_t off =
            ((size_t)tbl[t / P - wp0] * P + (t % P)) * tok_stride + (size_t)kvh * D + c * 8;
        __builtin_memcpy(&kr[i], k_pages + off, sizeof(V8<T>));
        __builtin_memcpy(&vr[i], v_pages + off, sizeof(V8<T>));
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          kr[i].v[j] = from_f32<T>(0.f);
          vr[i].v[j] = from_f32<T>(0.f);
        }
      }
    }
  };
  // Each group of LPT lanes keeps its own online-softmax state over its
  // tokens (t0 + g + TR*i); the groups are merged once, after the loop.
  auto consume = [&](int t0, const V8<T> (&kr)[NL], const V8<T> (&vr)[NL]) {
#pragma unroll
    for (int h = 0; h < REP; ++h) {
      float sc[NL];
      float mx = -INFINITY;
#pragma unroll
      for (int i = 0; i < NL; ++i) {
        float d = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) d += qf[h][j] * to_f32(kr[i].v[j]);
        d = group_sum<LPT>(d);
        sc[i] = (t0 + g + TR * i < tend) ? d : -INFINITY;
        mx = fmaxf(mx, sc[i]);
      }
      if (mx == -INFINITY) continue;       // no token of this group in the chunk
      const float mn = fmaxf(m[h], mx);
      const float alpha = exp2f(m[h] - mn);
      m[h] = mn;
      float ps = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[h][j] *= alpha;
#pragma unroll
      for (int i = 0; i < NL; ++i) {
        const float p = exp2f(sc[i] - mn);
        ps += p;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[h][j] += p * to_f32(vr[i].v[j]);
      }
      l[h] = l[h] * alpha + ps;
    }
  };

  {
    // three chunks in flight per wave: consume chunk c while c+1, c+2 load
    V8<T> ka[NL], va[NL], kb[NL], vb[NL], kc[NL], vc[NL];
    if (tstart < tend) load_chunk(tstart, ka, va);
    if (tstart + CH < tend) load_chunk(tstart + CH, kb, vb);
    if (tstart + 2 * CH < tend) load_chunk(tstart + 2 * CH, kc, vc);
    for (int t0 = tstart; t0 < tend; t0 += 3 * CH) {
      consume(t0, ka, va);
      if (t0 + 3 * CH < tend) load_chunk(t0 + 3 * CH, ka, va);
      if (t0 + CH >= tend) break;
      consume(t0 + CH, kb, vb);
      if (t0 + 4 * CH < tend) load_chunk(t0 + 4 * CH, kb, vb);
      if (t0 + 2 * CH >= tend) break;
      consume(t0 + 2 * CH, kc, vc);
      if (t0 + 5 * CH < tend) load_chunk(t0 + 5 * CH, kc, vc);
    }
  }
  // merge the wave's token groups (a group's lanes hold equal m and l)
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    float M = m[h];
#pragma unroll
    for (int o = LPT; o < kWave; o <<= 1) M = fmaxf(M, __shfl_xor(M, o));
    const float f = M == -INFINITY ? 0.f : exp2f(m[h] - M);
    m[h] = M;
    l[h] *= f;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[h][j] *= f;
#pragma unroll
    for (int o = LPT; o < kWave; o <<= 1) {
      l[h] += __shfl_xor(l[h], o);
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[h][j] += __shfl_xor(acc[h][j], o);
    }
  }
  if (g == 0) {
#pragma unroll
    for (int h = 0; h < REP; ++h)
#pragma unroll
      for (int j = 0; j < 8; ++j) sacc[(wid * REP + h) * D + c * 8 + j] = acc[h][j];
  }
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < REP; ++h) {
      sm[wid * REP + h] = m[h];
      sl[wid * REP + h] = l[h];
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < REP * D; e += NWV * kWave) {
    const int h = e / D, d = e % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NWV; ++w) M = fmaxf(M, sm[w * REP + h]);
    float num = 0.f, den = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < NWV; ++w) {
        const float f = exp2f(sm[w * REP + h] - M);
        num += f * sacc[(w * REP + h) * D + d];
        den += f * sl[w * REP + h];
      }
    }
    const size_t row = (size_t)b * H + kvh * REP + h;
    if (nsb == 1) {
      out[row * D + d] = from_f32<T>(num / den);
    } else {
      const size_t slot = row * S + sp;
      ws_acc[slot * D + d] = num;
      if (d == 0) {
        ws_m[slot] = M;
        ws_l[slot] = den;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// MFMA form (bf16 / fp16, D in {64, 128}): the main decode kernel.
//
// A workgroup of NWV waves serves one (split, kv head, sequence); the waves
// divide the split's pages. Per 16-token chunk of a wave, with lane = 16 r + c:
//  * S^T = K q^T on v_mfma_f32_16x16x32: A = K straight from the page (row =
//    token c, 8 dims per k-block), B = q^T (column = head c; the REP heads are
//    padded to 16 with zero rows of q), D/32 MFMAs. Register i of lane (r, c)
//    then holds the score of head c for token 4 r + i.
//  * online softmax in that layout. A head's running max m moves only when a
//    score exceeds it by more than kMaxSlack (log2 units): most chunks then
//    need no cross-lane max and no rescale, and p = 2^(s - m) stays below
//    2^kMaxSlack. p is rounded to T and l sums the rounded values, so the
//    output is the p-weighted mean of V up to fp32 accumulation.
//  * O^T += V^T P^T on v_mfma_f32_16x16x16: B = the p of lane (r, c) as it
//    stands (head c, tokens 4 r .. 4 r + 3); A = V^T, for which lane (r, c)
//    loads dims [c D/16, (c + 1) D/16) of tokens 4 r .. 4 r + 3 and
//    transposes them in registers with v_perm (output row c of MFMA b is dim
//    c D/16 + b). Register i of accumulator b of lane (r, c) holds dim
//    D/16 (4 r + i) + b of head c.
//  * chunks are page aligned when P % 16 == 0: one block-table lookup per
//    chunk (wave-uniform), and a chunk's loads stay inside its page, so only a
//    sequence's last chunk can be partial; there the rows past the end are
//    masked (scores to -inf, V rows to zero, so stale cache contents cannot
//    reach the sum). Three chunks are in flight per wave.
// At the end the waves' (m, l, acc) are merged in LDS and the output (or this
// split's partial for the combine kernel) is written.
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr float kMaxSlack = 8.0f;

template <typename T>
__device__ __forceinline__ f32x4_t mfma16x16x32(u32x4_t a, u32x4_t b, f32x4_t c) {
  if constexpr (std::is_same<T, __bf16>::value)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                    __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                   __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

template <typename T>
__device__ __forceinline__ f32x4_t mfma16x16x16(u32x2_t a, u32x2_t b, f32x4_t c) {
  if constexpr (std::is_same<T, __bf16>::value)
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4_t, a),
                                                      __builtin_bit_cast(s16x4_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4_t, a),
                                                  __builtin_bit_cast(f16x4_t, b), c, 0, 0, 0);
}

// Two values already on T's grid, packed lo | hi << 16.
template <typename T>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  const T a = (T)lo, b = (T)hi;
  return (uint32_t)__builtin_bit_cast(uint16_t, a) |
         ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

// Two floats rounded to T's grid, packed lo | hi << 16; sum gains the two
// rounded values (lo first).
template <typename T>
__device__ __forceinline__ uint32_t pack_sum(float lo, float hi, float& sum) {
  if constexpr (std::is_same<T, __bf16>::value) {
    const uint32_t u = pack_bf16x2(lo, hi);
    sum += bf16_lo(u);
    sum += bf16_hi(u);
    return u;
  } else {
    const float a = round_to<T>(lo), b = round_to<T>(hi);
    sum += a;
    sum += b;
    return pack2<T>(a, b);
  }
}

// Byte offset of the per-wave K slabs in the MFMA kernel's dynamic LDS:
// after the wave partials [NWV][REP][D], their (m, l) and the split's pps
// block ids, rounded up to 16 bytes.
__host__ __device__ constexpr size_t k3_slab_offset(int nwv, int rep, int d, int pps) {
  return ((size_t)(nwv * rep * d + 2 * nwv * rep) * 4 + (size_t)pps * 4 + 15) / 16 * 16;
}
__host__ __device__ constexpr size_t k3_slab_bytes(int nwv, int d) {
  return (size_t)nwv * kChunk * (2 * d + 16);
}

// The qkv epilogue run by the attention kernel itself (EPI): instead of q,
// the kernel reads the qkv projection's split-K partials and the epilogue's
// inputs, exactly as qkv_epilogue_kernel (rope.hip) does.
struct EpiArgs {
  const float* part;      // [nsplit][batch][(H + 2 KV) * D] fp32 partials
  int nsplit, batch;
  const void* q_w;        // [D] q/k RMSNorm weights, activation dtype
  const void* k_w;
  float eps;
  const int64_t* pos;     // [batch] positions of the new tokens
  const float* inv_freq;  // [D / 2]
  const int64_t* pages;   // [batch] (page, slot) the new k/v go to
  const int64_t* slots;
  void* k_dst;            // the pools again, written through these
  void* v_dst;
};
constexpr int kQB = 4;    // EPI: split partials requested per element up front

// EPI LDS after the slabs, per wave: q of the REP heads [REP][D], then the
// new k and v rows.
__host__ __device__ constexpr size_t k3_epi_bytes(int rep, int d) {
  return (size_t)(rep + 2) * d * 2;
}

template <typename T, int D, int REP, int NWV, bool PAGE16, int DEPTH = 3, bool EPI = false>
__global__ __launch_bounds__(NWV * kWave, NWV == 1 ? (DEPTH <= 2 ? 4 : 3) : 2) void paged_attn_mfma_kernel(
    const T* __restrict__ q, const T* __restrict__ k_pages, const T* __restrict__ v_pages,
    const int32_t* __restrict__ tables, const int32_t* __restrict__ lens, T* __restrict__ out,
    float* __restrict__ ws_acc, float* __restrict__ ws_m, float* __restrict__ ws_l, int H,
    int KV, int P, int num_blocks, int table_stride, int S, float scale_log2, EpiArgs e) {
  static_assert(!EPI || PAGE16, "EPI is built for 16-token pages");
  constexpr int KB = D / 32;                   // q.k MFMA k-blocks
  constexpr int DPL = D / 16;                  // P V: dims per lane per token = MFMAs per chunk
  constexpr int VW = DPL / 2;                  // ... in 32-bit words
  constexpr int CH = 16;                       // tokens per chunk
  static_assert(REP <= 16 && (D == 64 || D == 128), "unsupported shape");
  extern __shared__ __align__(16) unsigned char smem[];
  float* sacc = (float*)smem;                  // [NWV][REP][D]
  float* sm = sacc + NWV * REP * D;            // [NWV][REP]
  float* sl = sm + NWV * REP;                  // [NWV][REP]
  int* tbl = (int*)(sl + NWV * REP);

  // kv head fastest in the grid: the KV workgroups of one split read the same
  // pages (the heads of a token are adjacent in a page) at about the same time.
  // Head groups: gridDim.x = KV * G, G = (H / KV) / REP workgroups per kv
  // head, group g = blockIdx.x / KV serving q heads qh0 .. qh0 + REP - 1 (G > 1
  // gives a small batch's one split more workgroups than its (sequence, kv
  // head) pairs, without a combine). Workgroups are dealt to the 8 XCDs round
  // robin, so with KV a multiple of 8 a kv head's groups share one XCD and
  // its pages are fetched once into that XCD's L2.
  const int kvh = blockIdx.x % KV, sp = blockIdx.y, b = blockIdx.z;
  const int qh0 = kvh * (H / KV) + (int)(blockIdx.x / KV) * REP;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int lane = threadIdx.x % kWave;
  const int r = lane >> 4, c = lane & 15;
  const int pshift = __builtin_ctz(P);

  // The partition is fixed per launch (pps pages per split, ppv per wave),
  // so a wave's block ids are requested together with the length.
  const int pps = (table_stride + S - 1) / S;
  const int ppv = (pps + NWV - 1) / NWV;
  const int wp0 = sp * pps;
  const int vn0 = wp0 + wid * ppv;                   // the wave's first page, if any
  const bool reg_pages = ppv <= kWave;               // one block id per lane
  const int32_t* trow = tables + (size_t)b * table_stride;
  int pgr = 0;
  if (reg_pages && lane < ppv && vn0 + lane < min(wp0 + pps, table_stride))
    pgr = trow[vn0 + lane];
  const int L = min(max(lens[b], 0), table_stride * P);
  // q^T as the B operand (raw; the softmax scale is applied to S), requested
  // together with the block ids and the length: one round trip before K/V.
  // Columns c >= REP repeat head REP-1 (unconditional loads keep the wait
  // counts static); MFMA columns are independent and those are never stored.
  // (The empty asm pins the loads here; otherwise they sink below the early
  // exit and cost a second round trip.)
  // EPI: instead of q, the first kQB split partials of the REP q heads' lane
  // pairs (i, i + D/2), their norm weights and frequency, and the position.
  constexpr int HALF = D / 2;
  const int ic = min(lane, HALF - 1);                // this lane's pair
  const size_t width = (size_t)(H + 2 * KV) * D;
  const size_t qplane = (size_t)e.batch * width;
  const float* qsrc = EPI ? e.part + (size_t)b * width + (size_t)qh0 * D + ic : nullptr;
  float qpa[EPI ? REP : 1][kQB], qpc[EPI ? REP : 1][kQB], qw1 = 0.f, qw2 = 0.f, qfr = 0.f;
  float epos = 0.f;
  // ... and this kv head's k and v partials and k norm weights, for the wave
  // that turns out to hold the new token (known only with the length)
  float kpa[kQB], kpc[kQB], vpa[kQB], vpc[kQB], kw1 = 0.f, kw2 = 0.f;
  int64_t epage = 0, eslot = 0;
  const float* ksrc = EPI ? e.part + (size_t)b * width + (size_t)(H + kvh) * D + ic : nullptr;
  const float* vsrc = EPI ? e.part + (size_t)b * width + (size_t)(H + KV + kvh) * D + ic : nullptr;
  u32x4_t qb[KB];
  if constexpr (EPI) {
#pragma unroll
    for (int h = 0; h < REP; ++h) {
#pragma unroll
      for (int u = 0; u < kQB; ++u) {
        const float* pp = qsrc + (size_t)min(u, e.nsplit - 1) * qplane + h * D;
        qpa[h][u] = pp[0];
        qpc[h][u] = pp[HALF];
      }
    }
    qw1 = to_f32(((const T*)e.q_w)[ic]);
    qw2 = to_f32(((const T*)e.q_w)[ic + HALF]);
    qfr = e.inv_freq[ic];
    epos = (float)e.pos[b];
#pragma unroll
    for (int u = 0; u < kQB; ++u) {
      const size_t o = (size_t)min(u, e.nsplit - 1) * qplane;
      kpa[u] = ksrc[o];
      kpc[u] = ksrc[o + HALF];
      vpa[u] = vsrc[o];
      vpc[u] = vsrc[o + HALF];
    }
    kw1 = to_f32(((const T*)e.k_w)[ic]);
    kw2 = to_f32(((const T*)e.k_w)[ic + HALF]);
    epage = e.pages[b];
    eslot = e.slots[b];
#pragma unroll
    for (int h = 0; h < REP; ++h)
#pragma unroll
      for (int u = 0; u < kQB; ++u) asm volatile("" ::"v"(qpa[h][u]), "v"(qpc[h][u]));
    asm volatile("" ::"v"(qw1), "v"(qw2), "v"(qfr), "v"(epos), "v"(kw1), "v"(kw2));
#pragma unroll
    for (int u = 0; u < kQB; ++u)
      asm volatile("" ::"v"(kpa[u]), "v"(kpc[u]), "v"(vpa[u]), "v"(vpc[u]));
  } else {
#pragma unroll
    for (int j = 0; j < KB; ++j)
      qb[j] = *(const u32x4_t*)(q + ((size_t)b * H + qh0 + min(c, REP - 1)) * D + 32 * j + 8 * r);
#pragma unroll
    for (int j = 0; j < KB; ++j) asm volatile("" ::"v"(qb[j]));
  }
  const int npages = (L + P - 1) >> pshift;
  const int nsb = max(1, (npages + pps - 1) / pps);  // splits this sequence uses
  if (sp >= nsb) return;                             // uniform over the workgroup
  const int wp1 = min(wp0 + pps, npages);
  pgr = (unsigned)pgr < (unsigned)num_blocks ? pgr : 0;
  if (!reg_pages) {
    for (int i = threadIdx.x; i < wp1 - wp0; i += NWV * kWave) {
      const unsigned pg = (unsigned)trow[wp0 + i];
      tbl[i] = pg < (unsigned)num_blocks ? (int)pg : 0;
    }
  }
  const int vp0 = min(vn0, wp1), vp1 = min(vp0 + ppv, wp1);
  const int tstart = vp0 << pshift, tend = min(vp1 << pshift, L);
  // PAGE16: K rows are loaded like V rows (each load instruction reads four
  // tokens' whole 2D-byte rows, so every cache line is fetched by one
  // instruction) and turned into the MFMA A layout through this wave's slab.
  // Loading the A layout directly would read 16 tokens' 64-byte pieces per
  // instruction, each line split over two instructions.
  constexpr int KPITCH = 2 * D + 16;           // bytes per slab row
  uint8_t* kslab = (uint8_t*)smem + k3_slab_offset(NWV, REP, D, pps) + (size_t)wid * CH * KPITCH;
  // EPI: q of the REP heads, then the new token's k and v rows (activation
  // dtype), one such region per wave
  T* qs = (T*)((uint8_t*)smem + k3_slab_offset(NWV, REP, D, pps) + k3_slab_bytes(NWV, D) +
               (size_t)wid * k3_epi_bytes(REP, D));
  T* kn = qs + REP * D;
  T* vn = kn + D;
  // the wave that holds the new token (the last page; page 0 of a sequence
  // without tokens) writes its k and v: in the sequence's last split, the
  // wave whose pages contain it
  const int own_wid = NWV == 1 ? 0 : min(max(max(npages, 1) - 1 - wp0, 0) / ppv, NWV - 1);
  const bool owner = EPI && sp == nsb - 1 && wid == own_wid;
  float m = -INFINITY, l = 0.f;
  f32x4_t acc[DPL];
#pragma unroll
  for (int j = 0; j < DPL; ++j) acc[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  if (!reg_pages) __syncthreads();  // tbl ready
  // Prefetches past the wave's last chunk are still issued (an unconditional
  // load count keeps the wait counts static): they read one line of the last
  // chunk with every lane.
  const int tlast = tstart + max(tend - tstart - 1, 0) / CH * CH;

  const int tok_stride = KV * D;
  const int v_off = 4 * r * tok_stride + DPL * c;    // this lane's V rows / dims
  struct Chunk {
    u32x4_t k[PAGE16 ? 1 : KB];                // A layout (pages of < 16 tokens)
    uint32_t kr[PAGE16 ? 4 : 1][VW];           // V layout (PAGE16)
    uint32_t v[4][VW];
  };
  auto page_base = [&](int t) -> size_t {            // element offset of token t's row
    // every lane calls this (the shuffle reads other lanes' registers)
    const int pg = reg_pages ? __shfl(pgr, (t >> pshift) - vp0) : tbl[(t >> pshift) - wp0];
    return ((size_t)pg * P + (t & (P - 1))) * tok_stride + (size_t)kvh * D;
  };
  auto load_chunk = [&](int t0, Chunk& ch) {
    const bool spare = t0 > tlast;
    t0 = min(t0, tlast);
    if constexpr (PAGE16) {
      // the whole chunk lies in one page: a uniform base, per-lane offsets
      const int pi = (t0 >> pshift) - vp0;
      // (a wave without pages, possible with NWV > 1, still issues the EPI
      // form's first load: from the table slot after the split's last,
      // clamped into the pool like every block id)
      const int pgt = reg_pages ? __builtin_amdgcn_readlane(pgr, pi)
                                : __builtin_amdgcn_readfirstlane(tbl[pi + vp0 - wp0]);
      const int pg = (unsigned)pgt < (unsigned)num_blocks ? pgt : 0;
      const size_t base = ((size_t)pg * P + (t0 & (P - 1))) * tok_stride + (size_t)kvh * D;
      const T* kb = k_pages + base + (spare ? 0 : v_off);
      const T* vb = v_pages + base + (spare ? 0 : v_off);
      const int vstep = spare ? 0 : tok_stride;
      if constexpr (VW == 4) {
        // D = 128: each instruction reads four tokens' whole 256-byte rows,
        // read once per step, so with the non-temporal policy
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const u32x4_t kv4 = load_nt((const u32x4_t*)(kb + j * vstep));
          const u32x4_t vv4 = load_nt((const u32x4_t*)(vb + j * vstep));
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            ch.kr[j][w] = kv4[w];
            ch.v[j][w] = vv4[w];
          }
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) __builtin_memcpy(ch.kr[j], kb + j * vstep, sizeof(ch.kr[j]));
#pragma unroll
        for (int j = 0; j < 4; ++j) __builtin_memcpy(ch.v[j], vb + j * vstep, sizeof(ch.v[j]));
      }
    } else {
      // pages smaller than a chunk: one lookup per token, rows past the end
      // read as zero
      const int tk = t0 + c;
      const size_t kbase = page_base(min(tk, tend - 1));
#pragma unroll
      for (int j = 0; j < KB; ++j) ch.k[j] = u32x4_t{0u, 0u, 0u, 0u};
      if (tk < tend) {
        const T* kb = k_pages + kbase + 8 * r;
#pragma unroll
        for (int j = 0; j < KB; ++j) ch.k[j] = *(const u32x4_t*)(kb + 32 * j);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int tv = t0 + 4 * r + j;
        const size_t vbase = page_base(min(tv, tend - 1));
#pragma unroll
        for (int w = 0; w < VW; ++w) ch.v[j][w] = 0u;
        if (tv < tend)
          __builtin_memcpy(ch.v[j], v_pages + vbase + DPL * c, sizeof(ch.v[j]));
      }
    }
  };
  auto consume = [&](int t0, Chunk& ch) {
    f32x4_t sc = {0.f, 0.f, 0.f, 0.f};
    if constexpr (PAGE16) {
      // slab row = token, lane (r, c) wrote tokens 4 r + j, dims DPL c ...;
      // it reads token c, dims 32 j + 8 r ... (the A operand of k-block j)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint8_t* dst = kslab + (4 * r + j) * KPITCH + 2 * DPL * c;
        if constexpr (VW == 4)
          *(u32x4_t*)dst = u32x4_t{ch.kr[j][0], ch.kr[j][1], ch.kr[j][2], ch.kr[j][3]};
        else
#pragma unroll
          for (int w = 0; w < VW; ++w) ((uint32_t*)dst)[w] = ch.kr[j][w];
      }
      if constexpr (EPI) {
        const int rho = L - 1 - t0;                // the new token's row, if in this chunk
        if (owner && rho >= 0 && rho < CH) {
          uint32_t w[VW];
          __builtin_memcpy(w, kn + DPL * c, sizeof(w));
          if (r == 0) {
#pragma unroll
            for (int i = 0; i < VW; ++i) ((uint32_t*)(kslab + rho * KPITCH + 2 * DPL * c))[i] = w[i];
          }
          __builtin_memcpy(w, vn + DPL * c, sizeof(w));
          // lane (r, c) holds V rows 4 r + jj: a select per row (a branch or
          // an indexed store would put the chunk in scratch)
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const bool hit = 4 * r + jj == rho;
#pragma unroll
            for (int i = 0; i < VW; ++i) ch.v[jj][i] = hit ? w[i] : ch.v[jj][i];
          }
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int j = 0; j < KB; ++j)
        sc = mfma16x16x32<T>(*(const u32x4_t*)(kslab + c * KPITCH + 2 * (32 * j + 8 * r)), qb[j], sc);
    } else {
#pragma unroll
      for (int j = 0; j < KB; ++j) sc = mfma16x16x32<T>(ch.k[j], qb[j], sc);
    }
    float s[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) s[i] = sc[i] * scale_log2;
    if (t0 + CH > tend) {                      // the sequence's last chunk
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (t0 + 4 * r + i >= tend) {
          s[i] = -INFINITY;
#pragma unroll
          for (int w = 0; w < VW; ++w) ch.v[i][w] = 0u;
        }
      }
    }
    float mx = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    // row 0 holds token t0 < tend, so the head max below is finite
    if (__builtin_amdgcn_ballot_w64(mx > m + kMaxSlack) != 0) {
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float mn = fmaxf(m, mx);
      const float alpha = __builtin_amdgcn_exp2f(m - mn);
      m = mn;
      l *= alpha;
#pragma unroll
      for (int j = 0; j < DPL; ++j) acc[j] *= alpha;
    }
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[i] = round_to<T>(__builtin_amdgcn_exp2f(s[i] - m));
      l += p[i];
    }
    const u32x2_t pb = {pack2<T>(p[0], p[1]), pack2<T>(p[2], p[3])};
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      // element j of each of the lane's four V rows: word j/2, half j%2
      const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
      const u32x2_t va = {__builtin_amdgcn_perm(ch.v[1][j / 2], ch.v[0][j / 2], sel),
                          __builtin_amdgcn_perm(ch.v[3][j / 2], ch.v[2][j / 2], sel)};
      acc[j] = mfma16x16x16<T>(va, pb, acc[j]);
    }
  };

  // EPI: the epilogue's arithmetic (split partials added in split order,
  // rounded, per-head RMSNorm, RoPE; one pair per lane) for the REP q heads
  // into LDS, then the B operand from there. The wave whose split holds the
  // new token (the sequence's last split) also computes this kv head's k and
  // v, stores them at (page, slot) as the epilogue does, and keeps them in
  // LDS: the chunk loaded from the pool holds that row's old contents, so
  // consume() patches it from there. The split's first chunk is requested
  // before this work, so that its round trip overlaps it (one-page splits
  // have no other); the load is unconditional and in bounds (a split that
  // exists has a page, the block ids are clamped, a zero length reads the
  // first row of a valid page).
  Chunk cs[DEPTH];
  if constexpr (EPI) {
    load_chunk(tstart, cs[0]);
    float ecs[1], esn[1];
    rope_cs<T>(epos, qfr, ecs[0], esn[0]);         // shared by the q heads and k
    const float qw1a[1] = {qw1}, qw2a[1] = {qw2};
#pragma unroll
    for (int h = 0; h < REP; ++h) {
      float a = qpa[h][0], cc = qpc[h][0];
#pragma unroll
      for (int u = 1; u < kQB; ++u) {
        if (u < e.nsplit) {
          a = a + qpa[h][u];
          cc = cc + qpc[h][u];
        }
      }
      for (int s2 = kQB; s2 < e.nsplit; ++s2) {
        const float* pp = qsrc + (size_t)s2 * qplane + h * D;
        a = a + pp[0];
        cc = cc + pp[HALF];
      }
      float x1[1] = {round_to<T>(a)}, x2[1] = {round_to<T>(cc)};
      norm_rope_cs<T, 1>(x1, x2, HALF, qw1a, qw2a, e.eps, ecs, esn);
      if (lane < HALF) {
        qs[h * D + lane] = from_f32<T>(x1[0]);
        qs[h * D + lane + HALF] = from_f32<T>(x2[0]);
      }
    }
    if (owner) {
      float ka = kpa[0], kc = kpc[0], va = vpa[0], vc = vpc[0];
#pragma unroll
      for (int u = 1; u < kQB; ++u) {
        if (u < e.nsplit) {
          ka = ka + kpa[u];
          kc = kc + kpc[u];
          va = va + vpa[u];
          vc = vc + vpc[u];
        }
      }
      for (int s2 = kQB; s2 < e.nsplit; ++s2) {
        const size_t o = (size_t)s2 * qplane;
        ka = ka + ksrc[o];
        kc = kc + ksrc[o + HALF];
        va = va + vsrc[o];
        vc = vc + vsrc[o + HALF];
      }
      float k1[1] = {round_to<T>(ka)}, k2[1] = {round_to<T>(kc)};
      const float kw1a[1] = {kw1}, kw2a[1] = {kw2};
      norm_rope_cs<T, 1>(k1, k2, HALF, kw1a, kw2a, e.eps, ecs, esn);
      const float v1 = round_to<T>(va), v2 = round_to<T>(vc);
      // a (page, slot) outside the pool is dropped rather than written
      const uint64_t page = (uint64_t)epage, slot = (uint64_t)eslot;
      const bool in_pool = page < (uint64_t)num_blocks && slot < (uint64_t)P;
      if (lane < HALF) {
        kn[lane] = from_f32<T>(k1[0]);
        kn[lane + HALF] = from_f32<T>(k2[0]);
        vn[lane] = from_f32<T>(v1);
        vn[lane + HALF] = from_f32<T>(v2);
        if (in_pool) {
          const size_t off = ((page * P + slot) * KV + kvh) * D;
          T* kd = (T*)e.k_dst + off;
          T* vd = (T*)e.v_dst + off;
          kd[lane] = from_f32<T>(k1[0]);
          kd[lane + HALF] = from_f32<T>(k2[0]);
          vd[lane] = from_f32<T>(v1);
          vd[lane + HALF] = from_f32<T>(v2);
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // the B operand: head min(c, REP-1), dims 32 j + 8 r ...
#pragma unroll
    for (int j = 0; j < KB; ++j)
      qb[j] = *(const u32x4_t*)(qs + min(c, REP - 1) * D + 32 * j + 8 * r);
  }

  if (tstart < tend) {
    // DEPTH chunks in flight: chunk slot i is refilled right after use
#pragma unroll
    for (int i = EPI ? 1 : 0; i < DEPTH; ++i) load_chunk(tstart + i * CH, cs[i]);
    bool more = true;
    for (int t0 = tstart; more; t0 += DEPTH * CH) {
#pragma unroll
      for (int i = 0; i < DEPTH; ++i) {
        if (more) {
          consume(t0 + i * CH, cs[i]);
          load_chunk(t0 + (i + DEPTH) * CH, cs[i]);
          more = t0 + (i + 1) * CH < tend;
        }
      }
    }
  }
  // l: each lane summed its own tokens; add the four lane rows of a head
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);
  if constexpr (NWV == 1) {
    // a one-wave split writes its result straight from the accumulators:
    // lane (r, c < REP) holds dims DPL (4 r + i) + j of head c
    if (c < REP) {
      const size_t orow = (size_t)b * H + qh0 + c;
      if (nsb == 1) {
        const float inv = 1.0f / l;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          uint32_t w[VW];
#pragma unroll
          for (int j = 0; j < VW; ++j)
            w[j] = pack2<T>(acc[2 * j][i] * inv, acc[2 * j + 1][i] * inv);
          __builtin_memcpy(out + orow * D + DPL * (4 * r + i), w, sizeof(w));
        }
      } else {
        // the split's normalised output acc / l in fp16 (|acc / l| <= max |v|),
        // half the bytes of fp32 partials to write here and read in the combine
        const size_t slot = orow * S + sp;
        const float inv = 1.0f / l;
        _Float16* wp = (_Float16*)ws_acc + slot * D;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          _Float16 f[DPL];
#pragma unroll
          for (int j = 0; j < DPL; ++j) f[j] = (_Float16)(acc[j][i] * inv);
          __builtin_memcpy(wp + DPL * (4 * r + i), f, sizeof(f));
        }
        if (r == 0) {
          ws_m[slot] = m;
          ws_l[slot] = l;
        }
      }
    }
    return;
  }
  if (c < REP) {
    float* dst = sacc + (wid * REP + c) * D;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < DPL; ++j) dst[DPL * (4 * r + i) + j] = acc[j][i];
    if (r == 0) {
      sm[wid * REP + c] = m;
      sl[wid * REP + c] = l;
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < REP * D; e += NWV * kWave) {
    const int h = e / D, d = e % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NWV; ++w) M = fmaxf(M, sm[w * REP + h]);
    float num = 0.f, den = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < NWV; ++w) {
        const float f = exp2f(sm[w * REP + h] - M);
        num += f * sacc[(w * REP + h) * D + d];
        den += f * sl[w * REP + h];
      }
    }
    const size_t orow = (size_t)b * H + qh0 + h;
    if (nsb == 1) {
      out[orow * D + d] = from_f32<T>(num / den);
    } else {
      const size_t slot = orow * S + sp;
      ((_Float16*)ws_acc)[slot * D + d] = (_Float16)(num / den);  // normalised, as above
      if (d == 0) {
        ws_m[slot] = M;
        ws_l[slot] = den;
      }
    }
  }
}

// Phase 2: merge the partials of one (b, h) with the common max.
// Only sequences that used more than one split have partials; the kernels
// above wrote the others' output directly.
//
// One workgroup of kCombineWaves waves per (b, h), built so that one round
// trip to memory suffices for up to kWave splits: the length, every split's
// (m, l) (lane s) and each wave's share of the partial rows (s = wave,
// wave + kCombineWaves, ...) are all requested before any of them is used;
// slots past the sequence's split count are masked by selection, so stale
// workspace contents never reach the sums. The waves' sums are added in LDS
// in a fixed order.
constexpr int kCombineWaves = 4;

// NORM: the MFMA kernel's partials, each split's normalised output acc / l in
// fp16 (weight w_s l_s); else fp32 unnormalised acc (weight w_s).
template <typename T, int D, bool NORM>
__global__ __launch_bounds__(kCombineWaves * kWave) void paged_attn_combine_kernel(
    const float* __restrict__ ws_acc, const float* __restrict__ ws_m,
    const float* __restrict__ ws_l, T* __restrict__ out, const int32_t* __restrict__ lens,
    int H, int P, int table_stride, int S) {
  constexpr int DL = (D + kWave - 1) / kWave;        // dims per lane
  constexpr int SPW = kWave / kCombineWaves;         // slots per wave per round
  __shared__ float part[kCombineWaves][D];
  const size_t row = blockIdx.x;
  const int wid = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int d0 = lane * DL;
  const float* m = ws_m + row * S;
  const float* l = ws_l + row * S;
  const float* src = ws_acc + row * S * D;
  const _Float16* srch = (const _Float16*)ws_acc + row * S * D;
  const int pps = (table_stride + S - 1) / S;
  float a[DL];
#pragma unroll
  for (int i = 0; i < DL; ++i) a[i] = 0.f;
  float M = -INFINITY, lsum = 0.f;
  // the length as a vector load (a VGPR index), so that it is in flight with
  // the partial rows instead of a scalar round trip ahead of them
  int bi = (int)(row / H);
  asm volatile("" : "+v"(bi));
  const int lraw = lens[bi];
  int nsb = 0;
  for (int s0 = 0; s0 < S; s0 += kWave) {
    // ---- requests: (m, l) of slots s0 + lane, this wave's rows ----
    // Slots past S re-read slot S-1 and dims past D re-read dim D-1
    // (unconditional loads keep the wait counts static); every use below is
    // masked by s < nsb <= S.
    const float ml = m[min(s0 + lane, S - 1)];
    const float ll = l[min(s0 + lane, S - 1)];
    float x[SPW][DL];
#pragma unroll
    for (int k = 0; k < SPW; ++k) {
      const int s = min(s0 + wid + kCombineWaves * k, S - 1);
#pragma unroll
      for (int i = 0; i < DL; ++i) {
        const size_t e = (size_t)s * D + min(d0 + i, D - 1);
        x[k][i] = NORM ? (float)srch[e] : src[e];
      }
    }
    // The empty asm pins the requests (with the length above) ahead of the
    // early exit; otherwise they sink below it and cost a second round trip.
    asm volatile("" ::"v"(ml), "v"(ll), "v"(lraw));
#pragma unroll
    for (int k = 0; k < SPW; ++k)
#pragma unroll
      for (int i = 0; i < DL; ++i) asm volatile("" ::"v"(x[k][i]));
    // ---- use ----
    const int L = min(max(__builtin_amdgcn_readfirstlane(lraw), 0), table_stride * P);
    nsb = ((L + P - 1) / P + pps - 1) / pps;         // <= S
    if (nsb <= 1) return;                            // uniform over the workgroup
    const bool used = s0 + lane < nsb;
    const float mv = used ? ml : -INFINITY;
    const float Mr = wave_max(mv);                   // finite when s0 < nsb
    if (s0 >= nsb) break;
    const float Mn = fmaxf(M, Mr);
    const float scale_old = exp2f(M - Mn);           // 0 on the first round
    const float wl = used ? exp2f(ml - Mn) : 0.f;
    lsum = lsum * scale_old + wave_sum(used ? wl * ll : 0.f);
#pragma unroll
    for (int i = 0; i < DL; ++i) a[i] *= scale_old;
    M = Mn;
#pragma unroll
    for (int k = 0; k < SPW; ++k) {
      const int s = s0 + wid + kCombineWaves * k;
      const float w = __shfl(NORM ? wl * ll : wl, wid + kCombineWaves * k);
      if (s < nsb) {
#pragma unroll
        for (int i = 0; i < DL; ++i) a[i] += w * x[k][i];
      }
    }
  }
#pragma unroll
  for (int i = 0; i < DL; ++i)
    if (d0 + i < D) part[wid][d0 + i] = a[i];
  __syncthreads();
  const float inv = 1.0f / lsum;
  for (int d = threadIdx.x; d < D; d += kCombineWaves * kWave) {
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < kCombineWaves; ++w) t += part[w][d];
    out[row * D + d] = from_f32<T>(t * inv);
  }
}

// Head groups per kv head for the MFMA kernel: a single split over at most
// kHeadGroupPages pages and fewer (sequence, kv head) pairs than half the CUs
// gives each pair's q heads up to rep workgroups (halving the heads per
// workgroup while the grid stays within the CU count), so a small batch fills
// the chip without split partials and a combine launch.
constexpr int64_t kHeadGroupPages = 64;
int64_t k3_head_groups(int64_t B, int64_t KV, int64_t rep, int64_t S, int64_t ts) {
  if (S != 1 || ts > kHeadGroupPages) return 1;
  int64_t g = 1;
  while (g < rep && B * KV * g * 2 <= kCUs) g *= 2;
  return g;
}

template <typename T, int D, int REP>
int launch_attn(const void* q, const void* kp, const void* vp, const int32_t* tables,
                const int32_t* lens, void* out, float* ws_acc, float* ws_ml, int64_t B,
                int64_t H, int64_t KV, int64_t P, int64_t num_blocks, int64_t table_stride, int64_t S, float scale,
                hipStream_t st, const EpiArgs* epi, int64_t G) {
  // G head groups per kv head (REP = H / KV / G q heads each): the MFMA kernel only
  if (G != 1 && (D < 64 || std::is_same<T, float>::value)) return ACORN_ERR_UNSUPPORTED;
  dim3 grid((unsigned)S, (unsigned)KV, (unsigned)B);
  float* ws_m = ws_ml;
  float* ws_l = ws_ml ? ws_ml + B * H * S : nullptr;
  if constexpr (D >= 64 && !std::is_same<T, float>::value) {
    // small splits run as one-wave workgroups (many independent work units
    // that the dispatcher spreads over the CUs); large ones as NWV waves
    // merged in LDS
    const int64_t pps = (table_stride + S - 1) / S;
    const bool page16 = P % 16 == 0;
    const bool one = pps <= kOneWavePages;
    if (epi && !page16) return ACORN_ERR_UNSUPPORTED;
    const int nwv = one ? 1 : kAttnWaves;
    const size_t lds = k3_slab_offset(nwv, REP, D, (int)pps) +
                       (page16 ? k3_slab_bytes(nwv, D) : 0) +
                       (epi ? (size_t)nwv * k3_epi_bytes(REP, D) : 0);
    if (lds > 160 * 1024) return ACORN_ERR_UNSUPPORTED;
    const int which = epi ? (one ? 4 : 5) : (one ? 2 : 0) + (page16 ? 1 : 0);
    using KFn = void (*)(const T*, const T*, const T*, const int32_t*, const int32_t*, T*, float*,
                         float*, float*, int, int, int, int, int, int, float, EpiArgs);
    const KFn fns[6] = {paged_attn_mfma_kernel<T, D, REP, kAttnWaves, false>,
                        paged_attn_mfma_kernel<T, D, REP, kAttnWaves, true>,
                        paged_attn_mfma_kernel<T, D, REP, 1, false, kOneWaveDepth>,
                        paged_attn_mfma_kernel<T, D, REP, 1, true, kOneWaveDepth>,
                        paged_attn_mfma_kernel<T, D, REP, 1, true, kOneWaveDepth, true>,
                        paged_attn_mfma_kernel<T, D, REP, kAttnWaves, true, 3, true>};
    const KFn kfn = fns[which];
    static bool lds_raised[6] = {false, false, false, false, false, false};
    if (!lds_raised[which] && lds > 64 * 1024) {
      (void)hipFuncSetAttribute((const void*)kfn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                160 * 1024);
      lds_raised[which] = true;
    }
    kfn<<<dim3((unsigned)(KV * G), (unsigned)S, (unsigned)B), dim3(nwv * kWave), lds, st>>>(
        (const T*)q, (const T*)kp, (const T*)vp, tables, lens, (T*)out, ws_acc, ws_m, ws_l,
        (int)H, (int)KV, (int)P, (int)num_blocks, (int)table_stride, (int)S, scale * kLog2e,
        epi ? *epi : EpiArgs{});
  } else if constexpr (D >= 64) {
    if (epi) return ACORN_ERR_UNSUPPORTED;
    constexpr int NWV = kAttnWaves;
    const int64_t ppw = (table_stride + S - 1) / S;  // most pages one workgroup can get
    const size_t lds = (size_t)(NWV * REP * D + 2 * NWV * REP) * 4 + (size_t)ppw * 4;
    if (lds > 160 * 1024) return ACORN_ERR_UNSUPPORTED;
    auto kfn = paged_attn_wg_kernel<T, D, REP, NWV>;
    static bool lds_raised = false;
    if (!lds_raised && lds > 64 * 1024) {
      (void)hipFuncSetAttribute((const void*)kfn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                160 * 1024);
      lds_raised = true;
    }
    kfn<<<grid, dim3(NWV * kWave), lds, st>>>(
        (const T*)q, (const T*)kp, (const T*)vp, tables, lens, (T*)out, ws_acc, ws_m, ws_l,
        (int)H, (int)KV, (int)P, (int)num_blocks, (int)table_stride, (int)S, scale * kLog2e);
  } else {
    if (epi) return ACORN_ERR_UNSUPPORTED;
    paged_attn_split_kernel<T, D, REP><<<grid, dim3(kWave), 0, st>>>(
        (const T*)q, (const T*)kp, (const T*)vp, tables, lens, (T*)out, ws_acc, ws_m, ws_l,
        (int)H, (int)KV, (int)P, (int)num_blocks, (int)table_stride, (int)S, scale * kLog2e);
  }
  ACORN_LAUNCH_CHECK();
  if (S > 1) {
    // the MFMA kernel (bf16 / fp16, D >= 64) writes normalised fp16 partials
    constexpr bool kNorm = D >= 64 && !std::is_same<T, float>::value;
    paged_attn_combine_kernel<T, D, kNorm><<<dim3((unsigned)(B * H)), dim3(kCombineWaves * kWave), 0, st>>>(
        ws_acc, ws_m, ws_l, (T*)out, lens, (int)H, (int)P, (int)table_stride, (int)S);
    ACORN_LAUNCH_CHECK();
  }
  return ACORN_OK;
}

template <typename T, int D>
int dispatch_rep(int64_t rep, const void* q, const void* kp, const void* vp,
                 const int32_t* tables, const int32_t* lens, void* out, float* ws_acc,
                 float* ws_ml, int64_t B, int64_t H, int64_t KV, int64_t P, int64_t num_blocks, int64_t ts,
                 int64_t S, float scale, hipStream_t st, const EpiArgs* epi, int64_t G) {
  switch (rep) {   // q heads per workgroup
    case 1: return launch_attn<T, D, 1>(q, kp, vp, tables, lens, out, ws_acc, ws_ml, B, H, KV, P, num_blocks, ts, S, scale, st, epi, G);
    case 2: return launch_attn<T, D, 2>(q, kp, vp, tables, lens, out, ws_acc, ws_ml, B, H, KV, P, num_blocks, ts, S, scale, st, epi, G);
    case 4: return launch_attn<T, D, 4>(q, kp, vp, tables, lens, out, ws_acc, ws_ml, B, H, KV, P, num_blocks, ts, S, scale, st, epi, G);
    case 8: return launch_attn<T, D, 8>(q, kp, vp, tables, lens, out, ws_acc, ws_ml, B, H, KV, P, num_blocks, ts, S, scale, st, epi, G);
  }
  return ACORN_ERR_UNSUPPORTED;
}

template <typename T>
int dispatch_d(int64_t D, int64_t rep, const void* q, const void* kp, const void* vp,
               const int32_t* tables, const int32_t* lens, void* out, float* ws_acc,
               float* ws_ml, int64_t B, int64_t H, int64_t KV, int64_t P, int64_t num_blocks, int64_t ts,
               int64_t S, float scale, hipStream_t st, const EpiArgs* epi = nullptr) {
  const int64_t G = D >= 64 && !std::is_same<T, float>::value ? k3_head_groups(B, KV, rep, S, ts) : 1;
  const int64_t r = rep / G;
  switch (D) {
    case 16: return dispatch_rep<T, 16>(r, q, kp, vp, tables, lens, out, ws_acc, ws_ml, B, H, KV, P, num_blocks, ts, S, scale, st, epi, G);
    case 32: return dispatch_rep<T, 32>(r, q, kp, vp, tables, lens, out, ws_acc, ws_ml, B, H, KV, P, num_blocks, ts, S, scale, st, epi, G);
    case 64: return dispatch_rep<T, 64>(r, q, kp, vp, tables, lens, out, ws_acc, ws_ml, B, H, KV, P, num_blocks, ts, S, scale, st, epi, G);
    case 128: return dispatch_rep<T, 128>(r, q, kp, vp, tables, lens, out, ws_acc, ws_ml, B, H, KV, P, num_blocks, ts, S, scale, st, epi, G);
  }
  return ACORN_ERR_UNSUPPORTED;
}

// ---------------------------------------------------------------------------
// Prefill attention: query-tiled flash attention over the paged cache with a
// causal mask, for a chunked prefill whose new rows' K/V are already in the
// pool. Row j of sequence n (q row seq_row0[n] + j) sits at position
// seq_pos0[n] + j and attends to that sequence's tokens 0 .. its position.
// It uses the decode K3's MFMA layout with the 16 columns of S^T = K Q^T being
// 16 consecutive query tokens of one head instead of the heads of one token:
//  * a workgroup serves the REP q heads of one kv head for QG x 32 query
//    tokens: wave (head, group) owns two 16-token query blocks (QW = 2), so
//    every K / V operand it reads feeds two MFMAs;
//  * the kv head's keys are walked in chunks of 64 tokens that the whole
//    workgroup stages in LDS once (K and V rows, coalesced 16-byte loads, two
//    buffers, one barrier per chunk); the next chunk's loads are in flight
//    while the current one is consumed, and its page ids one chunk earlier.
//    Rows are padded to 2 D + 32 bytes: the score operand reads (16 rows x
//    64 bytes) and the transposing V reads (16 rows x 32 bytes) then run
//    without LDS bank conflicts on gfx950 (a probe: 2 D + 16 adds conflict
//    cycles to the former and 2 D to both);
//  * per 32 keys and query block: 2 D/32 v_mfma_f32_16x16x32 for the scores,
//    the online softmax per query column (lazy max; the scale is applied
//    inside the exp2 argument by one fma), D/16 v_mfma_f32_16x16x32 for P V
//    (the scores of the two 16-key halves are its B operand as they lie;
//    16x16x16 runs at half the rate on gfx950; the V^T operand comes from
//    LDS through ds_read_b64_tr_b16, no register transposes); blocks whose
//    queries all precede the keys skip the scores and add P = 0; keys past a
//    query's position are masked where a chunk crosses the diagonal, and the
//    first chunk holds key 0, so every column's max is finite from the
//    start; rows past the last key re-read it (finite, masked);
//  * the longest query tiles (the last ones) are dispatched first.
// A workgroup reads its keys once for REP x QG x 32 query rows: O(L^2 / 32)
// K / V bytes per prompt of L tokens and kv head, against O(L^2) for one
// decode row per token.
template <typename T, int D, int REP, int QG, int KC>
__global__ __launch_bounds__(REP * QG * kWave, 2) void paged_prefill_kernel(
    const T* __restrict__ q, const T* __restrict__ k_pages, const T* __restrict__ v_pages,
    const int32_t* __restrict__ tables, const int32_t* __restrict__ seq_row0,
    const int32_t* __restrict__ seq_pos0, const int32_t* __restrict__ seq_nq, T* __restrict__ out,
    int R, int H, int KV, int P, int num_blocks, int table_stride, float scale_log2) {
  constexpr int QW = 2;                          // 16-query blocks per wave
  constexpr int NT = REP * QG * kWave;           // threads
  constexpr int KB = D / 32, DPL = D / 16;
  constexpr int KPITCH = 2 * D + 32;             // bytes per staged K row (padded)
  constexpr int VPITCH = KPITCH;                 // bytes per staged V row
  constexpr int RP = 2 * D / 16;                 // 16-byte pieces per K / V row
  constexpr int PPT = 2 * KC * RP / NT;          // pieces per thread per chunk
  constexpr int WQ = QG * QW * 16;               // query rows per workgroup
  static_assert(2 * KC * RP % NT == 0 && PPT >= 1, "whole pieces per thread");
  static_assert(KC % 32 == 0, "a chunk is whole 32-key P V MFMAs");
  __shared__ __align__(16) uint8_t kvs[2][KC * (KPITCH + VPITCH)];   // [buffer][K rows | V rows]
  const int kvh = blockIdx.y, n = blockIdx.z;
  const int tid = threadIdx.x;
  const int wid = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int lane = tid % kWave;
  const int r = lane >> 4, c = lane & 15;
  const int hq = wid % REP, sub = wid / REP;
  const int h = kvh * REP + hq;
  const int pos0 = seq_pos0[n];
  const int row0 = seq_row0[n];
  // rows past q's R rows are not served (so bad metadata cannot reach past q / out)
  const int nq = row0 < 0 || pos0 < 0 ? 0 : min(seq_nq[n], R - row0);
  const int wg_j0 = (gridDim.x - 1 - blockIdx.x) * WQ;          // longest tiles first
  if (wg_j0 >= nq) return;                                       // uniform over the workgroup
  const int j0 = wg_j0 + sub * QW * 16;                          // this wave's first query row
  const int nvalid = max(0, min(QW * 16, nq - j0));              // 0: the wave only stages
  const int L = pos0 + min(wg_j0 + WQ, nq);                      // keys of the workgroup's last query
  const int nchunks = (L + KC - 1) / KC;
  const int32_t* trow = tables + (size_t)n * table_stride;
  const int pshift = __builtin_ctz(P);
  const int tok_stride = KV * D;

  // the queries: block qw's column c is query row j0 + 16 qw + c (clamped)
  u32x4_t qb[QW][KB];
  int pc[QW];
#pragma unroll
  for (int qw = 0; qw < QW; ++qw) {
    const int jc = min(16 * qw + c, max(nvalid - 1, 0));
    pc[qw] = pos0 + j0 + jc;
    const size_t qrow = (size_t)(row0 + min(j0 + jc, nq - 1));
#pragma unroll
    for (int jb = 0; jb < KB; ++jb)
      qb[qw][jb] = *(const u32x4_t*)(q + (qrow * H + h) * D + 32 * jb + 8 * r);
  }

  // staging: this thread moves the 16-byte column pcol of rows prow0 + i NT / RP
  // (i < PH) of K and of V; a row's K and V pieces share its page id
  static_assert(NT % RP == 0 && PPT % 2 == 0, "whole rows per wave");
  constexpr int PH = PPT / 2, RSTEP = NT / RP;
  const int pcol = tid % RP, prow0 = tid / RP;
  const uint32_t poff0 = (uint32_t)(prow0 * KPITCH + pcol * 16);
  const T* kbase = k_pages + (size_t)kvh * D + pcol * 8;
  const T* vbase = v_pages + (size_t)kvh * D + pcol * 8;
  auto page_of = [&](int chunk, int i) {
    const int t = min(chunk * KC + prow0 + i * RSTEP, L - 1);
    const unsigned pg = (unsigned)trow[min(t >> pshift, table_stride - 1)];
    return pg < (unsigned)num_blocks ? (int)pg : 0;
  };
  int pg[PH], pg_next[PH];
  u32x4_t stage[PPT];
  auto load_chunk = [&](int chunk, const int (&pgs)[PH]) {
#pragma unroll
    for (int i = 0; i < PH; ++i) {
      const int t = min(chunk * KC + prow0 + i * RSTEP, L - 1);
      const size_t off = ((size_t)pgs[i] * P + (t & (P - 1))) * tok_stride;
      stage[i] = *(const u32x4_t*)(kbase + off);
      stage[PH + i] = *(const u32x4_t*)(vbase + off);
    }
  };
  auto store_chunk = [&](int b) {
#pragma unroll
    for (int i = 0; i < PH; ++i) {
      *(u32x4_t*)(kvs[b] + poff0 + i * RSTEP * KPITCH) = stage[i];
      *(u32x4_t*)(kvs[b] + KC * KPITCH + poff0 + i * RSTEP * VPITCH) = stage[PH + i];
    }
  };

  float m[QW], l[QW];
  f32x4_t acc[QW][DPL];
#pragma unroll
  for (int qw = 0; qw < QW; ++qw) {
    m[qw] = -INFINITY;
    l[qw] = 0.f;
#pragma unroll
    for (int jj = 0; jj < DPL; ++jj) acc[qw][jj] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  // one 32-key chunk of buffer b, keys from t0: the scores of its two 16-key
  // halves (S^T = K Q^T, lane (r, c) holds keys 4 r .. 4 r + 3 of each half
  // for query c) are exactly the B operand of one v_mfma_f32_16x16x32 for
  // P V when the MFMA's k slot s of lane group r stands for key 4 r + s
  // (s < 4) or 16 + 4 r + s - 4 (half 1); the V^T operand follows the same
  // key order, so P never moves between lanes. That operand comes from LDS
  // transposed by ds_read_b64_tr_b16: within each 16-lane group, lane j
  // receives element j % 4 of the 8 bytes lane 4 e + j / 4 addressed, for
  // e = 0..3. Lane 4 e + q of group r addresses key 4 r + e (+ 16 for the
  // second half), dims 16 jj + 4 q .. + 3, so lane (r, c) receives dim
  // 16 jj + c of keys 4 r .. 4 r + 3: row c of block jj's A operand.
  const uint32_t vlane = (uint32_t)((4 * r + (c >> 2)) * VPITCH + 8 * (c & 3));
  // One 32-key step, software-pipelined by one step: this step's score
  // MFMAs are issued first, then the previous step's P V MFMAs (va / pb,
  // held in registers across the chunk barrier), and this step's softmax
  // runs while those execute; its P and V operands are left in va / pb.
  u32x4_t va[DPL], pb[QW];
  bool pend = false;                             // va / pb hold a step whose P V is due
  auto pv = [&]() {
#pragma unroll
    for (int jj = 0; jj < DPL; ++jj)
#pragma unroll
      for (int qw = 0; qw < QW; ++qw) acc[qw][jj] = mfma16x16x32<T>(va[jj], pb[qw], acc[qw][jj]);
  };
  auto step = [&](int b, int sub, int t0) {
    const uint8_t* kbuf = kvs[b] + 32 * sub * KPITCH;
    const uint8_t* vbuf = kvs[b] + KC * KPITCH + 32 * sub * VPITCH;
    u32x4_t kf[2][KB];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int jb = 0; jb < KB; ++jb)
        kf[hh][jb] = *(const u32x4_t*)(kbuf + (16 * hh + c) * KPITCH + 2 * (32 * jb + 8 * r));
    f32x4_t S[QW][2];
    bool live[QW];
#pragma unroll
    for (int qw = 0; qw < QW; ++qw) {
      // the block's queries all precede these keys, or it has none: nothing to add
      live[qw] = 16 * qw < nvalid && t0 <= pos0 + j0 + min(16 * qw + 15, nvalid - 1);
      if (!live[qw]) continue;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        S[qw][hh] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int jb = 0; jb < KB; ++jb)
          S[qw][hh] = mfma16x16x32<T>(kf[hh][jb], qb[qw][jb], S[qw][hh]);
      }
    }
    if (pend) pv();
    pend = live[0] || live[QW - 1];
    if (!pend) return;
#pragma unroll
    for (int qw = 0; qw < QW; ++qw) {
      // a block without live queries adds P = 0 (V rows are finite), so the
      // P V MFMAs run unconditionally
      if (!live[qw]) {
        pb[qw] = u32x4_t{0u, 0u, 0u, 0u};
        continue;
      }
      float sv[8];                               // raw scores; scaled inside the exp2
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int i = 0; i < 4; ++i) sv[4 * hh + i] = S[qw][hh][i];
      if (t0 + 31 > pos0 + j0 + 16 * qw) {       // the keys cross some column's diagonal
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (t0 + 16 * hh + 4 * r + i > pc[qw]) sv[4 * hh + i] = -INFINITY;
      }
      float mx = sv[0];
#pragma unroll
      for (int i = 1; i < 8; ++i) mx = fmaxf(mx, sv[i]);
      mx *= scale_log2;                          // scale_log2 > 0: the max of the scaled scores
      if (__builtin_amdgcn_ballot_w64(mx > m[qw] + kMaxSlack) != 0) {
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float mn = fmaxf(m[qw], mx);
        const float alpha = __builtin_amdgcn_exp2f(m[qw] - mn);
        m[qw] = mn;
        l[qw] *= alpha;
#pragma unroll
        for (int jj = 0; jj < DPL; ++jj) acc[qw][jj] *= alpha;
      }
      const float nm = -m[qw];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        pb[qw][i] = pack_sum<T>(__builtin_amdgcn_exp2f(__builtin_fmaf(sv[2 * i], scale_log2, nm)),
                                __builtin_amdgcn_exp2f(__builtin_fmaf(sv[2 * i + 1], scale_log2, nm)),
                                l[qw]);
    }
    typedef __attribute__((address_space(3))) s16x4_t lds_s16x4;
    const __attribute__((address_space(3))) uint8_t* vl =
        (const __attribute__((address_space(3))) uint8_t*)vbuf + vlane;
#pragma unroll
    for (int jj = 0; jj < DPL; ++jj) {
      const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vl + 32 * jj));
      const s16x4_t hi =
          __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vl + 16 * VPITCH + 32 * jj));
      const u32x2_t l2 = __builtin_bit_cast(u32x2_t, lo), h2 = __builtin_bit_cast(u32x2_t, hi);
      va[jj] = u32x4_t{l2[0], l2[1], h2[0], h2[1]};
    }
  };

  // prologue: chunk 0 staged, chunk 1's loads and page ids in flight
#pragma unroll
  for (int i = 0; i < PH; ++i) pg[i] = page_of(0, i);
  load_chunk(0, pg);
#pragma unroll
  for (int i = 0; i < PH; ++i) pg_next[i] = page_of(min(1, nchunks - 1), i);
  store_chunk(0);
  load_chunk(min(1, nchunks - 1), pg_next);
  __syncthreads();
  for (int ci = 0; ci < nchunks; ++ci) {
    const int b = ci & 1;
    // page ids two chunks ahead
#pragma unroll
    for (int i = 0; i < PH; ++i) pg[i] = page_of(min(ci + 2, nchunks - 1), i);
    __builtin_amdgcn_sched_barrier(0);
    if (nvalid > 0) {
#pragma unroll
      for (int sub = 0; sub < KC / 32; ++sub) step(b, sub, ci * KC + 32 * sub);
    }
    __builtin_amdgcn_sched_barrier(0);
    store_chunk(b ^ 1);                         // chunk ci + 1 (its buffer was last read in ci - 1)
    __builtin_amdgcn_sched_barrier(0);
    load_chunk(min(ci + 2, nchunks - 1), pg);
    __syncthreads();
  }
  if (nvalid == 0) return;
  if (pend) pv();
  // lane (r, c) of block qw holds dims 16 jj + 4 r + i of query column 16 qw + c
#pragma unroll
  for (int qw = 0; qw < QW; ++qw) {
    float lt = l[qw];
    lt += __shfl_xor(lt, 16);
    lt += __shfl_xor(lt, 32);
    if (16 * qw + c < nvalid) {
      const size_t orow = (size_t)(row0 + j0 + 16 * qw + c) * H + h;
      const float inv = 1.0f / lt;
#pragma unroll
      for (int jj = 0; jj < DPL; ++jj) {
        const u32x2_t w = {pack2<T>(acc[qw][jj][0] * inv, acc[qw][jj][1] * inv),
                           pack2<T>(acc[qw][jj][2] * inv, acc[qw][jj][3] * inv)};
        *(u32x2_t*)(out + orow * D + 16 * jj + 4 * r) = w;
      }
    }
  }
}

constexpr int kPrefillChunk = 64;   // keys staged per barrier (32: 3% slower at 8192 tokens)

template <typename T, int D, int REP>
int launch_prefill(const void* q, const void* kp, const void* vp, const int32_t* tables,
                   const int32_t* row0, const int32_t* pos0, const int32_t* nq, void* out,
                   int64_t N, int64_t R, int64_t max_nq, int64_t H, int64_t KV, int64_t P,
                   int64_t num_blocks, int64_t table_stride, float scale, hipStream_t st) {
  // four waves per workgroup (eight for 8 q heads per kv head), 32 query rows each
  constexpr int QG = REP >= 4 ? 1 : 4 / REP;
  const int64_t tiles = (max_nq + 32 * QG - 1) / (32 * QG);
  paged_prefill_kernel<T, D, REP, QG, kPrefillChunk>
      <<<dim3((unsigned)tiles, (unsigned)KV, (unsigned)N), dim3(REP * QG * kWave), 0, st>>>(
          (const T*)q, (const T*)kp, (const T*)vp, tables, row0, pos0, nq, (T*)out, (int)R,
          (int)H, (int)KV, (int)P, (int)num_blocks, (int)table_stride, scale * kLog2e);
  ACORN_LAUNCH_CHECK();
  return ACORN_OK;
}

template <typename T, int D>
int prefill_rep(int64_t rep, const void* q, const void* kp, const void* vp,
                const int32_t* tables, const int32_t* row0, const int32_t* pos0,
                const int32_t* nq, void* out, int64_t N, int64_t R, int64_t max_nq, int64_t H,
                int64_t KV, int64_t P, int64_t num_blocks, int64_t ts, float scale,
                hipStream_t st) {
  switch (rep) {
    case 1: return launch_prefill<T, D, 1>(q, kp, vp, tables, row0, pos0, nq, out, N, R, max_nq, H, KV, P, num_blocks, ts, scale, st);
    case 2: return launch_prefill<T, D, 2>(q, kp, vp, tables, row0, pos0, nq, out, N, R, max_nq, H, KV, P, num_blocks, ts, scale, st);
    case 4: return launch_prefill<T, D, 4>(q, kp, vp, tables, row0, pos0, nq, out, N, R, max_nq, H, KV, P, num_blocks, ts, scale, st);
    case 8: return launch_prefill<T, D, 8>(q, kp, vp, tables, row0, pos0, nq, out, N, R, max_nq, H, KV, P, num_blocks, ts, scale, st);
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

extern "C" int acorn_paged_prefill_attention(const void* q, const void* k_pages,
                                             const void* v_pages, const int32_t* tables,
                                             const int32_t* seq_row0, const int32_t* seq_pos0,
                                             const int32_t* seq_nq, void* out, int64_t N,
                                             int64_t R, int64_t max_nq, int64_t H, int64_t KV,
                                             int64_t D, int64_t P, int64_t num_blocks,
                                             int64_t table_stride, float scale, int dtype,
                                             void* stream) {
  if (N < 0 || R < 0 || max_nq < 0 || H <= 0 || KV <= 0 || D <= 0 || P <= 0 ||
      num_blocks <= 0 || table_stride < 1)
    return ACORN_ERR_SHAPE;
  if ((P & (P - 1)) != 0 || P % 16 != 0 || H % KV != 0) return ACORN_ERR_SHAPE;
  if (KV > 65535 || N > 65535 || R > 0x7fffffff || max_nq > 0x7fffffff) return ACORN_ERR_SHAPE;
  if (N == 0 || R == 0 || max_nq == 0) return ACORN_OK;
  if (!q || !k_pages || !v_pages || !tables || !seq_row0 || !seq_pos0 || !seq_nq || !out)
    return ACORN_ERR_VALUE;
  const int64_t rep = H / KV;
  hipStream_t st = (hipStream_t)stream;
  if (D != 64 && D != 128) return ACORN_ERR_UNSUPPORTED;
  switch (dtype) {
    case ACORN_F16:
      return D == 64 ? prefill_rep<_Float16, 64>(rep, q, k_pages, v_pages, tables, seq_row0, seq_pos0, seq_nq, out, N, R, max_nq, H, KV, P, num_blocks, table_stride, scale, st)
                     : prefill_rep<_Float16, 128>(rep, q, k_pages, v_pages, tables, seq_row0, seq_pos0, seq_nq, out, N, R, max_nq, H, KV, P, num_blocks, table_stride, scale, st);
    case ACORN_BF16:
      return D == 64 ? prefill_rep<__bf16, 64>(rep, q, k_pages, v_pages, tables, seq_row0, seq_pos0, seq_nq, out, N, R, max_nq, H, KV, P, num_blocks, table_stride, scale, st)
                     : prefill_rep<__bf16, 128>(rep, q, k_pages, v_pages, tables, seq_row0, seq_pos0, seq_nq, out, N, R, max_nq, H, KV, P, num_blocks, table_stride, scale, st);
  }
  return ACORN_ERR_UNSUPPORTED;
}

// ---------------------------------------------------------------------------
// Allocation-free K3: the split partials live in this file-scope array, one
// copy per GPU, held until the process ends. Host code never passes the
// array's name to a kernel (on the host it is only a stand-in for the symbol);
// it passes the device address hipGetSymbolAddress returns, looked up once per
// device with that device current and kept in g_scratch.
constexpr size_t kScratchBytes = (size_t)ACORN_K3_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices];

// This device's copy of `scratch`, for a launch on `st`, which must belong
// to the current device.
int scratch_for(hipStream_t st, unsigned char** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return ACORN_ERR_HIP - (int)e;
  if (st != nullptr) {
    int sdev = -1;
    e = hipStreamGetDevice(st, &sdev);
    if (e != hipSuccess) return ACORN_ERR_HIP - (int)e;
    if (sdev != dev) return ACORN_ERR_VALUE;
  }
  if (dev < 0 || dev >= kMaxDevices) return ACORN_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return ACORN_ERR_HIP - (int)e;
    g_scratch[dev] = p;
  }
  *out = (unsigned char*)g_scratch[dev];
  return ACORN_OK;
}

}  // namespace

extern "C" int acorn_paged_attention_noalloc(const void* q, const void* k_pages,
                                             const void* v_pages, const int32_t* tables,
                                             const int32_t* seq_lens, void* out, int64_t B,
                                             int64_t H, int64_t KV, int64_t D, int64_t P,
                                             int64_t num_blocks, int64_t table_stride,
                                             int64_t num_splits, float scale, int dtype,
                                             void* stream) {
  // the shape contract of acorn_paged_attention, checked before the size
  if (B < 0 || H <= 0 || KV <= 0 || D <= 0 || P <= 0 || num_blocks <= 0 || num_splits < 1 ||
      table_stride < 1)
    return ACORN_ERR_SHAPE;
  if (num_splits > 65535 || KV > 65535 || B > 65535 || H > 65535 || D > 65535)
    return ACORN_ERR_SHAPE;
  if (B == 0) return ACORN_OK;
  float* ws_acc = nullptr;
  float* ws_ml = nullptr;
  if (num_splits > 1) {
    // partials [B*H*S*D] fp32, then m|l [2*B*H*S] fp32 (each B, H, S, D
    // < 2^16, so the products fit in 64 bits)
    const size_t rows = (size_t)B * (size_t)H * (size_t)num_splits;
    const size_t acc_bytes = (rows * (size_t)D * 4 + 255) / 256 * 256;
    if (acc_bytes + rows * 8 > kScratchBytes) return ACORN_ERR_SCRATCH;
    unsigned char* base = nullptr;
    const int rc = scratch_for((hipStream_t)stream, &base);
    if (rc != ACORN_OK) return rc;
    ws_acc = (float*)base;
    ws_ml = (float*)(base + acc_bytes);
  }
  return acorn_paged_attention(q, k_pages, v_pages, tables, seq_lens, out, ws_acc, ws_ml, B, H,
                               KV, D, P, num_blocks, table_stride, num_splits, scale, dtype,
                               stream);
}

extern "C" int acorn_paged_attention_qkv_supported(int64_t H, int64_t KV, int64_t D, int64_t P,
                                                   int64_t table_stride, int64_t num_splits,
                                                   int dtype, int wdtype) {
  if (H <= 0 || KV <= 0 || H % KV != 0 || num_splits < 1 || table_stride < 1 || P <= 0) return 0;
  const int64_t rep = H / KV;
  if (!(dtype == ACORN_BF16 || dtype == ACORN_F16) || wdtype != dtype) return 0;
  if (!(D == 64 || D == 128) || P % 16 != 0 || (P & (P - 1)) != 0) return 0;
  if (!(rep == 1 || rep == 2 || rep == 4 || rep == 8)) return 0;
  // one-wave splits, or workgroups of kAttnWaves waves whose LDS (block ids,
  // wave partials, K slabs and the epilogue's rows) fits
  const int64_t pps = (table_stride + num_splits - 1) / num_splits;
  if (pps <= kOneWavePages) return 1;
  if (pps > (int64_t)1 << 20) return 0;
  const size_t lds = k3_slab_offset(kAttnWaves, (int)rep, (int)D, (int)pps) +
                     k3_slab_bytes(kAttnWaves, (int)D) + (size_t)kAttnWaves * k3_epi_bytes((int)rep, (int)D);
  return lds <= 160 * 1024 ? 1 : 0;
}

extern "C" int acorn_paged_attention_qkv(const float* part, int64_t nsplit, void* k_pages,
                                         void* v_pages, const int64_t* pages, const int64_t* slots,
                                         const int32_t* tables, const int32_t* seq_lens, void* out,
                                         float* ws_acc, float* ws_ml, int64_t B, int64_t H,
                                         int64_t KV, int64_t D, int64_t P, int64_t num_blocks,
                                         int64_t table_stride, int64_t num_splits, float scale,
                                         const void* q_w, const void* k_w, float eps,
                                         const int64_t* positions, const float* inv_freq,
                                         int dtype, int wdtype, void* stream) {
  if (B < 0 || H <= 0 || KV <= 0 || D <= 0 || P <= 0 || num_blocks <= 0 || num_splits < 1 ||
      table_stride < 1 || nsplit < 1)
    return ACORN_ERR_SHAPE;
  if ((D & (D - 1)) != 0 || (P & (P - 1)) != 0 || H % KV != 0) return ACORN_ERR_SHAPE;
  if (num_splits > 65535 || KV > 65535 || B > 65535 || nsplit > 0x7fffffff ||
      num_blocks > 0x7fffffff)
    return ACORN_ERR_SHAPE;
  if (!acorn_paged_attention_qkv_supported(H, KV, D, P, table_stride, num_splits, dtype, wdtype))
    return ACORN_ERR_UNSUPPORTED;
  if (B == 0) return ACORN_OK;
  if (!part || !k_pages || !v_pages || !pages || !slots || !tables || !seq_lens || !out || !q_w ||
      !k_w || !positions || !inv_freq)
    return ACORN_ERR_VALUE;
  if (num_splits > 1 && (!ws_acc || !ws_ml)) return ACORN_ERR_VALUE;
  const EpiArgs e{part, (int)nsplit, (int)B, q_w, k_w, eps, positions, inv_freq,
                  pages, slots, k_pages, v_pages};
  hipStream_t st = (hipStream_t)stream;
  const int64_t rep = H / KV;
  if (dtype == ACORN_BF16)
    return dispatch_d<__bf16>(D, rep, nullptr, k_pages, v_pages, tables, seq_lens, out, ws_acc,
                              ws_ml, B, H, KV, P, num_blocks, table_stride, num_splits, scale, st,
                              &e);
  return dispatch_d<_Float16>(D, rep, nullptr, k_pages, v_pages, tables, seq_lens, out, ws_acc,
                              ws_ml, B, H, KV, P, num_blocks, table_stride, num_splits, scale, st,
                              &e);
}
