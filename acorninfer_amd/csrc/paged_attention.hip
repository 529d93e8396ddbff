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
#include <type_traits>

#include "common.h"

using namespace acorn;

namespace {

constexpr int kChunk = 16;  // tokens per step
constexpr int kLPT = 4;     // lanes per token in the q.k phase
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kAttnWaves = 8;  // waves per workgroup of the single-kernel form

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
  const int ppw = (npages + S - 1) / S;        // pages per workgroup split
  const int wp0 = min(sp * ppw, npages), wp1 = min(wp0 + ppw, npages);
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
    if (S == 1) {
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
// Per 16-token chunk of a wave:
//  * S = q K^T on v_mfma_f32_16x16x32: A = q (the REP heads padded to 16
//    rows; lane row = lane % 16, k = 8 * (lane / 16)), B = K^T loaded straight
//    from the page (lane column = token lane % 16, 8 dims per k-block), D/32
//    MFMAs. The result puts head 4*(lane/16)+i of token lane%16 in register i.
//  * online softmax on that layout: row max / row sum over the 16 tokens with
//    DPP; each lane row tracks (m, l) of its four heads.
//  * P V on VALU in the row layout (lane = 8 dims of one token, 16-byte V
//    loads); p and the rescale factors reach those lanes through a per-wave
//    LDS slot (same-wave LDS traffic needs no barrier).
//  * chunks are page aligned when P % 16 == 0, so a chunk costs one block-table
//    lookup; three chunks are in flight per wave.
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

template <typename T>
__device__ __forceinline__ f32x4_t mfma16x16x32(u32x4_t a, u32x4_t b, f32x4_t c) {
  if constexpr (std::is_same<T, __bf16>::value)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                    __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                   __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp<0xB1>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  v = fmaxf(v, dpp<0x141>(v));
  v = fmaxf(v, dpp<0x140>(v));
  return v;
}

template <typename T, int D, int REP, int NWV, bool PAGE16>
__global__ __launch_bounds__(NWV * kWave) void paged_attn_mfma_kernel(
    const T* __restrict__ q, const T* __restrict__ k_pages, const T* __restrict__ v_pages,
    const int32_t* __restrict__ tables, const int32_t* __restrict__ lens, T* __restrict__ out,
    float* __restrict__ ws_acc, float* __restrict__ ws_m, float* __restrict__ ws_l, int H,
    int KV, int P, int num_blocks, int table_stride, int S, float scale_log2) {
  constexpr int KB = D / 32;                   // MFMA k-blocks
  constexpr int LPT = D / 8;                   // P V layout: lanes per token
  constexpr int TR = kWave / LPT;              // tokens per wave-wide V load
  constexpr int CH = 16;                       // tokens per chunk
  constexpr int NL = CH / TR;                  // V loads per lane per chunk
  constexpr int HG = (REP + 3) / 4;            // lane rows that hold scores
  static_assert(REP <= 16 && NL >= 1, "unsupported shape");
  extern __shared__ __align__(16) unsigned char smem[];
  float* sacc = (float*)smem;                  // [NWV][REP][D]
  float* sm = sacc + NWV * REP * D;            // [NWV][REP]
  float* sl = sm + NWV * REP;                  // [NWV][REP]
  float* pl = sl + NWV * REP;                  // [NWV][CH][4*HG]  p per token and head
  float* al = pl + NWV * CH * 4 * HG;          // [NWV][4*HG]      rescale per head
  int* tbl = (int*)(al + NWV * 4 * HG);

  const int sp = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int wid = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int row = lane >> 4, col = lane & 15;  // MFMA layout
  const int g = lane / LPT, c = lane % LPT;    // P V layout
  float* mypl = pl + wid * CH * 4 * HG;
  float* myal = al + wid * 4 * HG;

  const int L = min(max(lens[b], 0), table_stride * P);
  const int npages = (L + P - 1) / P;
  const int ppw = (npages + S - 1) / S;
  const int wp0 = min(sp * ppw, npages), wp1 = min(wp0 + ppw, npages);
  const int32_t* trow = tables + (size_t)b * table_stride;
  for (int i = threadIdx.x; i < wp1 - wp0; i += NWV * kWave) {
    const unsigned pg = (unsigned)trow[wp0 + i];
    tbl[i] = pg < (unsigned)num_blocks ? (int)pg : 0;
  }
  const int ppv = (wp1 - wp0 + NWV - 1) / NWV;
  const int vp0 = min(wp0 + wid * ppv, wp1), vp1 = min(vp0 + ppv, wp1);
  const int tstart = vp0 * P, tend = min(vp1 * P, L);

  // q as the MFMA A operand (raw; the softmax scale is applied to S)
  u32x4_t qa[KB];
#pragma unroll
  for (int j = 0; j < KB; ++j) {
    qa[j] = u32x4_t{0u, 0u, 0u, 0u};
    if (col < REP)
      qa[j] = *(const u32x4_t*)(q + ((size_t)b * H + kvh * REP + col) * D + 32 * j + 8 * row);
  }
  float m4[4], l4[4], acc[REP][8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m4[i] = -INFINITY;
    l4[i] = 0.f;
  }
#pragma unroll
  for (int h = 0; h < REP; ++h)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[h][j] = 0.f;
  __syncthreads();  // tbl ready

  const size_t tok_stride = (size_t)KV * D;
  struct Chunk {
    u32x4_t k[KB];
    u32x4_t v[NL];
  };
  auto token_base = [&](int t) -> size_t {
    return ((size_t)tbl[t / P - wp0] * P + (t % P)) * tok_stride + (size_t)kvh * D;
  };
  auto load_chunk = [&](int t0, Chunk& ch) {
    // K in B layout: token t0 + col, dims 32j + 8*row
    {
      const int t = t0 + col;
      size_t base;
      if constexpr (PAGE16)
        base = ((size_t)tbl[t0 / P - wp0] * P + (t0 % P) + col) * tok_stride + (size_t)kvh * D;
      else
        base = t < tend ? token_base(t) : 0;
#pragma unroll
      for (int j = 0; j < KB; ++j) {
        ch.k[j] = u32x4_t{0u, 0u, 0u, 0u};
        if (t < tend) ch.k[j] = *(const u32x4_t*)(k_pages + base + 32 * j + 8 * row);
      }
    }
    // V in row layout: tokens t0 + g + TR*i, dims 8c..8c+7
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int t = t0 + g + TR * i;
      ch.v[i] = u32x4_t{0u, 0u, 0u, 0u};
      if (t < tend) {
        size_t base;
        if constexpr (PAGE16)
          base = ((size_t)tbl[t0 / P - wp0] * P + (t0 % P) + g + TR * i) * tok_stride +
                 (size_t)kvh * D;
        else
          base = token_base(t);
        ch.v[i] = *(const u32x4_t*)(v_pages + base + 8 * c);
      }
    }
  };
  auto consume = [&](int t0, const Chunk& ch) {
    f32x4_t sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < KB; ++j) sc = mfma16x16x32<T>(qa[j], ch.k[j], sc);
    const bool valid = t0 + col < tend;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (4 * row + i >= 4 * HG) continue;
      const float s = valid ? sc[i] * scale_log2 : -INFINITY;
      const float mx = row16_max(s);           // finite: the chunk holds >= 1 token
      const float mn = fmaxf(m4[i], mx);
      const float alpha = exp2f(m4[i] - mn);
      const float p = exp2f(s - mn);
      l4[i] = l4[i] * alpha + group_sum<16>(p);
      m4[i] = mn;
      if (row < HG) {
        mypl[col * 4 * HG + 4 * row + i] = p;
        if (col == 0) myal[4 * row + i] = alpha;
      }
    }
    // P V on the row layout
    float pv[NL][REP], alph[REP];
#pragma unroll
    for (int h = 0; h < REP; ++h) alph[h] = myal[h];
#pragma unroll
    for (int i = 0; i < NL; ++i)
#pragma unroll
      for (int h = 0; h < REP; ++h) pv[i][h] = mypl[(g + TR * i) * 4 * HG + h];
#pragma unroll
    for (int h = 0; h < REP; ++h) {
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[h][j] *= alph[h];
#pragma unroll
      for (int i = 0; i < NL; ++i) {
        const V8<T> vv = __builtin_bit_cast(V8<T>, ch.v[i]);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[h][j] += pv[i][h] * to_f32(vv.v[j]);
      }
    }
  };

  {
    Chunk ca, cb, cc;
    if (tstart < tend) load_chunk(tstart, ca);
    if (tstart + CH < tend) load_chunk(tstart + CH, cb);
    if (tstart + 2 * CH < tend) load_chunk(tstart + 2 * CH, cc);
    for (int t0 = tstart; t0 < tend; t0 += 3 * CH) {
      consume(t0, ca);
      if (t0 + 3 * CH < tend) load_chunk(t0 + 3 * CH, ca);
      if (t0 + CH >= tend) break;
      consume(t0 + CH, cb);
      if (t0 + 4 * CH < tend) load_chunk(t0 + 4 * CH, cb);
      if (t0 + 2 * CH >= tend) break;
      consume(t0 + 2 * CH, cc);
      if (t0 + 5 * CH < tend) load_chunk(t0 + 5 * CH, cc);
    }
  }
  // sum the token groups' P V (all groups used the same running max)
#pragma unroll
  for (int h = 0; h < REP; ++h)
#pragma unroll
    for (int o = LPT; o < kWave; o <<= 1)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[h][j] += __shfl_xor(acc[h][j], o);
  if (g == 0) {
#pragma unroll
    for (int h = 0; h < REP; ++h)
#pragma unroll
      for (int j = 0; j < 8; ++j) sacc[(wid * REP + h) * D + c * 8 + j] = acc[h][j];
  }
  if (col == 0 && row < HG) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 4 * row + i;
      if (h < REP) {
        sm[wid * REP + h] = m4[i];
        sl[wid * REP + h] = l4[i];
      }
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
    const size_t orow = (size_t)b * H + kvh * REP + h;
    if (S == 1) {
      out[orow * D + d] = from_f32<T>(num / den);
    } else {
      const size_t slot = orow * S + sp;
      ws_acc[slot * D + d] = num;
      if (d == 0) {
        ws_m[slot] = M;
        ws_l[slot] = den;
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
  dim3 grid((unsigned)S, (unsigned)KV, (unsigned)B);
  float* ws_m = ws_ml;
  float* ws_l = ws_ml ? ws_ml + B * H * S : nullptr;
  if constexpr (D >= 64 && !std::is_same<T, float>::value) {
    constexpr int NWV = kAttnWaves;
    constexpr int HG = (REP + 3) / 4;
    const int64_t ppw = (table_stride + S - 1) / S;
    const size_t lds = (size_t)(NWV * REP * D + 2 * NWV * REP + NWV * 16 * 4 * HG +
                                NWV * 4 * HG) * 4 + (size_t)ppw * 4;
    if (lds > 160 * 1024) return ACORN_ERR_UNSUPPORTED;
    const bool page16 = P % 16 == 0;
    auto kfn = page16 ? paged_attn_mfma_kernel<T, D, REP, NWV, true>
                      : paged_attn_mfma_kernel<T, D, REP, NWV, false>;
    static bool lds_raised[2] = {false, false};
    if (!lds_raised[page16] && lds > 64 * 1024) {
      (void)hipFuncSetAttribute((const void*)kfn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                160 * 1024);
      lds_raised[page16] = true;
    }
    kfn<<<grid, dim3(NWV * kWave), lds, st>>>(
        (const T*)q, (const T*)kp, (const T*)vp, tables, lens, (T*)out, ws_acc, ws_m, ws_l,
        (int)H, (int)KV, (int)P, (int)num_blocks, (int)table_stride, (int)S, scale * kLog2e);
  } else if constexpr (D >= 64) {
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
    paged_attn_split_kernel<T, D, REP><<<grid, dim3(kWave), 0, st>>>(
        (const T*)q, (const T*)kp, (const T*)vp, tables, lens, (T*)out, ws_acc, ws_m, ws_l,
        (int)H, (int)KV, (int)P, (int)num_blocks, (int)table_stride, (int)S, scale * kLog2e);
  }
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
