// Token sampler: temperature -> top-k -> top-p -> draw, one workgroup per row.
//
// Semantics follow acorninfer/sampler.py:38-68 (HF warper order):
//   x = logits / T                                   (fp32)
//   top-k: remove x < kth-largest(x)                 (ties with the kth are kept)
//   top-p: over the kept x sorted ascending (stable), cum = cumsum(softmax);
//          remove where cum <= 1 - p, always keep the largest
//   draw : token with probability softmax(x)[kept] (inverse CDF of a given
//          uniform u over the kept tokens in vocabulary order); logprob is the
//          log-softmax of the processed logits at the token.
// temperature == 0 means greedy (argmax, logprob 0), as Executor._sample
// routes it (engine/executor.py:128-138).
//
// Design: the row is never sorted. Keys are the order-preserving uint32 image
// of fp32. top-k is a 4-pass radix select (8-bit digits, MSB first) with
// count histograms; top-p is the same descent over the softmax mass, with
// masses accumulated as 2^-40 fixed-point integers so that the LDS atomics
// are order independent (deterministic). The tie group at the top-p boundary
// is resolved in the stable ascending order HF sorts in: among equal values
// the higher vocabulary index is nearer the top.
#include <algorithm>

#include "common.h"

using namespace acorn;

namespace {

constexpr int kNT = 1024;
constexpr double kFix = 1099511627776.0;  // 2^40

typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
typedef uint16_t u16x2v __attribute__((ext_vector_type(2)));

// Element e of a 16-byte vector of T as float.
template <typename T> __device__ __forceinline__ float word_elem(const u32x4v& w, int e);
template <> __device__ __forceinline__ float word_elem<__bf16>(const u32x4v& w, int e) {
  return (e & 1) ? bf16_hi(w[e / 2]) : bf16_lo(w[e / 2]);
}
template <> __device__ __forceinline__ float word_elem<_Float16>(const u32x4v& w, int e) {
  const uint32_t v = w[e / 2];
  return (float)__builtin_bit_cast(_Float16, (uint16_t)((e & 1) ? v >> 16 : v & 0xffffu));
}
template <> __device__ __forceinline__ float word_elem<float>(const u32x4v& w, int e) {
  return __uint_as_float(w[e]);
}

// Exponent fields of a 16-byte vector folded into a running unsigned max
// (per 16-bit half for the half types): a field of all ones, i.e. an inf or
// NaN somewhere, survives as the maximum.
template <typename T> struct ExpBits;
template <> struct ExpBits<__bf16> { static constexpr uint32_t kMask = 0x7F807F80u; };
template <> struct ExpBits<_Float16> { static constexpr uint32_t kMask = 0x7C007C00u; };
template <> struct ExpBits<float> { static constexpr uint32_t kMask = 0x7F800000u; };
template <typename T> __device__ __forceinline__ uint32_t fold_exp(uint32_t acc, const u32x4v& w) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t x = w[i] & ExpBits<T>::kMask;
    if constexpr (sizeof(T) == 2)
      acc = __builtin_bit_cast(uint32_t, __builtin_elementwise_max(
                                             __builtin_bit_cast(u16x2v, acc),
                                             __builtin_bit_cast(u16x2v, x)));
    else
      acc = max(acc, x);
  }
  return acc;
}
template <typename T> __device__ __forceinline__ bool exp_all_ones(uint32_t acc) {
  constexpr uint32_t m = ExpBits<T>::kMask;
  if constexpr (sizeof(T) == 2)
    return (acc & 0xffffu) == (m & 0xffffu) || (acc >> 16) == (m >> 16);
  else
    return acc == m;
}

__device__ __forceinline__ uint32_t okey(float x) {
  const uint32_t u = __float_as_uint(x);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Block-wide exclusive scan of one float per thread (fixed order).
__device__ float block_exclusive_scan(float v, float* buf, float* total) {
  buf[threadIdx.x] = v;
  __syncthreads();
  for (int off = 1; off < kNT; off <<= 1) {
    const float add = threadIdx.x >= off ? buf[threadIdx.x - off] : 0.f;
    __syncthreads();
    buf[threadIdx.x] += add;
    __syncthreads();
  }
  const float incl = buf[threadIdx.x];
  *total = buf[kNT - 1];
  __syncthreads();
  return incl - v;
}

__device__ uint32_t block_exclusive_scan_u32(uint32_t v, uint32_t* buf, uint32_t* total) {
  buf[threadIdx.x] = v;
  __syncthreads();
  for (int off = 1; off < kNT; off <<= 1) {
    const uint32_t add = threadIdx.x >= off ? buf[threadIdx.x - off] : 0u;
    __syncthreads();
    buf[threadIdx.x] += add;
    __syncthreads();
  }
  const uint32_t incl = buf[threadIdx.x];
  *total = buf[kNT - 1];
  __syncthreads();
  return incl - v;
}

template <typename T>
__global__ __launch_bounds__(kNT) void sample_kernel(
    const T* __restrict__ logits, int64_t V, const float* __restrict__ temperature,
    const int32_t* __restrict__ top_k, const float* __restrict__ top_p,
    const float* __restrict__ uniform, int64_t* __restrict__ token, float* __restrict__ logprob,
    float* __restrict__ processed, int32_t* __restrict__ status) {
  __shared__ uint32_t hcnt[256];
  __shared__ unsigned long long hmass[256];
  __shared__ float sbuf[kNT];
  __shared__ uint32_t ubuf[kNT];
  __shared__ float red_f[kNT / kWave];
  __shared__ int64_t red_i[kNT / kWave];
  __shared__ uint32_t sh_u32[8];
  __shared__ unsigned long long sh_u64[4];
  __shared__ float sh_f[4];
  __shared__ int sh_bad;

  const int64_t r = blockIdx.x;
  const T* row = logits + r * V;
  const float Tm = temperature[r];
  const int tid = threadIdx.x, lane = tid % kWave, wid = tid / kWave;
  if (tid == 0) sh_bad = 0;
  __syncthreads();

  // ---- pass 1: max (first index on ties), finiteness --------------------
  // 16-byte vectors, kUnroll of them in flight per thread (a 151936-entry
  // bf16 row is two rounds of requests); a scalar tail. Vector indices past
  // the row re-read its last vector (unconditional loads keep the wait
  // counts static) and are not visited.
  // A single workgroup reads the whole row, so the per-element work is what
  // bounds it: per vector only its maximum is compared with the running one
  // (the vector index of the first strict improvement is kept) and the
  // exponent fields are folded into an integer max for the finiteness test.
  // After the loop the kept vector is read again and its first element equal
  // to the maximum taken: the thread's first maximum in index order, as an
  // element-by-element scan would find.
  float bv = -INFINITY;
  int64_t bi = INT64_MAX;
  bool bad = false;
  auto visit = [&](float l, int64_t i) {
    if (!(l == l) || l == INFINITY || l == -INFINITY) bad = true;
    if (l > bv || (l == bv && i < bi)) {
      bv = l;
      bi = i;
    }
  };
  {
    constexpr int E = 16 / sizeof(T);                 // elements per vector
    constexpr int kUnroll = 10;
    const bool aligned = ((uintptr_t)row % 16) == 0;
    const int64_t nvec = aligned ? V / E : 0;
    const u32x4v* rv = (const u32x4v*)row;
    float vbest = -INFINITY;
    int64_t jbest = -1;
    uint32_t emax = 0;
    for (int64_t j0 = tid; j0 < nvec; j0 += (int64_t)kNT * kUnroll) {
      u32x4v buf[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) buf[u] = rv[min(j0 + (int64_t)u * kNT, nvec - 1)];
      // (the empty asm keeps every load ahead of the guarded uses below;
      // a load sunk into a guarded block is waited for on its own)
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) asm volatile("" ::"v"(buf[u]));
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int64_t j = j0 + (int64_t)u * kNT;
        if (j < nvec) {
          float vm = word_elem<T>(buf[u], 0);
#pragma unroll
          for (int e = 1; e < E; ++e) vm = fmaxf(vm, word_elem<T>(buf[u], e));
          emax = fold_exp<T>(emax, buf[u]);
          if (vm > vbest) {
            vbest = vm;
            jbest = j;
          }
        }
      }
    }
    if (exp_all_ones<T>(emax)) bad = true;
    if (jbest >= 0) {
      const u32x4v w = rv[jbest];
      int ebest = E - 1;
#pragma unroll
      for (int e = E - 2; e >= 0; --e) ebest = word_elem<T>(w, e) == vbest ? e : ebest;
      bv = vbest;
      bi = jbest * E + ebest;
    }
    for (int64_t i = nvec * E + tid; i < V; i += kNT) visit(to_f32(row[i]), i);
  }
  if (bad) sh_bad = 1;  // benign race: every writer stores 1
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int64_t oi = __shfl_xor(bi, o);
    if (ov > bv || (ov == bv && oi < bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if (lane == 0) {
    red_f[wid] = bv;
    red_i[wid] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kNT / kWave; ++w)
      if (red_f[w] > bv || (red_f[w] == bv && red_i[w] < bi)) {
        bv = red_f[w];
        bi = red_i[w];
      }
    red_f[0] = bv;
    red_i[0] = bi;
  }
  __syncthreads();
  const float lmax = red_f[0];
  const int64_t imax = red_i[0];
  if (sh_bad) {
    if (tid == 0) {
      status[r] = 1;
      token[r] = imax == INT64_MAX ? 0 : imax;
      logprob[r] = NAN;
    }
    return;
  }
  if (!(Tm > 0.f)) {  // greedy
    if (tid == 0) {
      status[r] = 0;
      token[r] = imax;
      logprob[r] = 0.f;
    }
    if (processed)
      for (int64_t i = tid; i < V; i += kNT) processed[r * V + i] = to_f32(row[i]);
    return;
  }
  const float M = lmax / Tm;  // max of x (division is monotone for T > 0)

  // ---- top-k: kth largest key by radix select on counts -------------------
  const int64_t kk = top_k[r];
  uint32_t kkey = 0;  // keep key >= kkey
  if (kk > 0 && kk < V) {
    uint32_t prefix = 0, pmask = 0;
    uint32_t remaining = (uint32_t)kk;
    for (int shift = 24; shift >= 0; shift -= 8) {
      for (int b = tid; b < 256; b += kNT) hcnt[b] = 0;
      __syncthreads();
      for (int64_t i = tid; i < V; i += kNT) {
        const uint32_t key = okey(to_f32(row[i]) / Tm);
        if ((key & pmask) == prefix) atomicAdd(&hcnt[(key >> shift) & 255u], 1u);
      }
      __syncthreads();
      if (tid == 0) {
        uint32_t acc = 0;
        int d = 255;
        for (; d > 0; --d) {
          if (acc + hcnt[d] >= remaining) break;
          acc += hcnt[d];
        }
        sh_u32[0] = (uint32_t)d;
        sh_u32[1] = remaining - acc;
      }
      __syncthreads();
      prefix |= sh_u32[0] << shift;
      pmask |= 255u << shift;
      remaining = sh_u32[1];
      __syncthreads();
    }
    kkey = prefix;
  }

  // ---- mass of the top-k set: Z = sum exp(x - M) over key >= kkey ---------
  // (fixed-point, order independent)
  auto wfix = [&](float x) -> unsigned long long {
    return (unsigned long long)((double)exp2f((x - M) * 1.4426950408889634f) * kFix);
  };
  unsigned long long zl = 0;
  for (int64_t i = tid; i < V; i += kNT) {
    const float x = to_f32(row[i]) / Tm;
    if (okey(x) >= kkey) zl += wfix(x);
  }
  if (tid == 0) sh_u64[0] = 0;
  __syncthreads();
  atomicAdd(&sh_u64[0], zl);
  __syncthreads();
  const unsigned long long Zk = sh_u64[0];

  // ---- top-p: descend on mass to the boundary key --------------------------
  const float pp = top_p[r];
  uint32_t pkey = kkey;           // keep key > pkey, plus n_keep of the ties at pkey
  uint32_t tie_keep = 0xffffffffu;  // all ties kept unless reduced below
  bool ptie = false;
  if (pp < 1.0f) {
    const unsigned long long target = (unsigned long long)((double)pp * (double)Zk);
    uint32_t prefix = 0, pmask = 0;
    unsigned long long above = 0;
    uint32_t tie_cnt = 0;
    unsigned long long tie_mass = 0;
    for (int shift = 24; shift >= 0; shift -= 8) {
      for (int b = tid; b < 256; b += kNT) {
        hmass[b] = 0;
        hcnt[b] = 0;
      }
      __syncthreads();
      for (int64_t i = tid; i < V; i += kNT) {
        const float x = to_f32(row[i]) / Tm;
        const uint32_t key = okey(x);
        if (key >= kkey && (key & pmask) == prefix) {
          atomicAdd(&hmass[(key >> shift) & 255u], wfix(x));
          atomicAdd(&hcnt[(key >> shift) & 255u], 1u);
        }
      }
      __syncthreads();
      if (tid == 0) {
        unsigned long long acc = above;
        int d = 255;
        for (; d > 0; --d) {
          if (hcnt[d] && acc + hmass[d] >= target) break;
          acc += hmass[d];
        }
        // d == 0 is the last candidate bin
        sh_u32[0] = (uint32_t)d;
        sh_u64[1] = acc;
        sh_u32[2] = hcnt[d];
        sh_u64[2] = hmass[d];
      }
      __syncthreads();
      prefix |= sh_u32[0] << shift;
      pmask |= 255u << shift;
      above = sh_u64[1];
      tie_cnt = sh_u32[2];
      tie_mass = sh_u64[2];
      __syncthreads();
    }
    // tokens strictly above `prefix` hold mass `above` < target; the tie
    // group at `prefix` (tie_cnt tokens, equal mass q each) is kept while
    // above + r*q < target, r counted from the highest index down.
    pkey = prefix;
    if (tie_cnt > 0) {
      const double q = (double)tie_mass / (double)tie_cnt;
      uint32_t nk = 1;
      if (q > 0.0) {
        const double t = ((double)target - (double)above) / q;
        nk = (uint32_t)std::min<double>((double)tie_cnt, std::max(1.0, ceil(t)));
      } else {
        nk = tie_cnt;
      }
      if (nk < tie_cnt) {
        tie_keep = nk;
        ptie = true;
      }
    }
  }

  // ---- final keep rule, per contiguous segment (vocabulary order) -------
  const int64_t seg = (V + kNT - 1) / kNT;
  const int64_t s0 = std::min<int64_t>((int64_t)tid * seg, V);
  const int64_t s1 = std::min<int64_t>(s0 + seg, V);
  // ties at pkey: rank from the highest index (only needed when partially kept)
  uint32_t ties_after = 0;
  if (ptie) {
    uint32_t mine = 0;
    for (int64_t i = s0; i < s1; ++i)
      if (okey(to_f32(row[i]) / Tm) == pkey) ++mine;
    // exclusive scan from the end: ties in segments after mine
    uint32_t tot;
    const uint32_t before = block_exclusive_scan_u32(mine, ubuf, &tot);
    ties_after = tot - before - mine;
  }
  const bool use_p = pp < 1.0f;
  auto kept_at = [&](float x, uint32_t& tie_rank_from_end) -> bool {
    const uint32_t key = okey(x);
    if (key < kkey) return false;
    if (!use_p) return true;
    if (key > pkey) return true;
    if (key < pkey) return false;
    if (!ptie) return true;
    return tie_rank_from_end < tie_keep;
  };

  // segment mass (fp32, vocabulary order) for the inverse CDF
  float segm = 0.f;
  {
    uint32_t rank = ties_after;
    // walk backward to know each tie's rank from the end
    for (int64_t i = s1 - 1; i >= s0; --i) {
      const float x = to_f32(row[i]) / Tm;
      uint32_t rk = rank;
      const bool tie = okey(x) == pkey;
      if (kept_at(x, rk)) segm += exp2f((x - M) * 1.4426950408889634f);
      if (tie) ++rank;
    }
  }
  float Zf;
  const float before = block_exclusive_scan(segm, sbuf, &Zf);
  const float target = uniform[r] * Zf;
  // the segment where the running mass first exceeds the target
  if (tid == 0) {
    sh_u32[3] = 0xffffffffu;
    sh_f[0] = 0.f;
  }
  __syncthreads();
  if (segm > 0.f && before <= target && target < before + segm) atomicMin(&sh_u32[3], (uint32_t)tid);
  __syncthreads();
  uint32_t owner = sh_u32[3];
  if (owner == 0xffffffffu) {
    // rounding put the target at the very end: the last segment with mass
    if (tid == 0) sh_u32[4] = 0;
    __syncthreads();
    if (segm > 0.f) atomicMax(&sh_u32[4], (uint32_t)tid);
    __syncthreads();
    owner = sh_u32[4];
  }
  if ((uint32_t)tid == owner) {
    // forward walk; tie ranks from the end need the segment's tie total
    uint32_t seg_ties = 0;
    if (ptie)
      for (int64_t i = s0; i < s1; ++i)
        if (okey(to_f32(row[i]) / Tm) == pkey) ++seg_ties;
    uint32_t ties_seen = 0;
    float run = before;
    int64_t pick = -1, last_kept = -1;
    for (int64_t i = s0; i < s1; ++i) {
      const float x = to_f32(row[i]) / Tm;
      const bool tie = okey(x) == pkey;
      uint32_t rk = ties_after + (seg_ties - ties_seen - (tie ? 1u : 0u));
      if (kept_at(x, rk)) {
        run += exp2f((x - M) * 1.4426950408889634f);
        last_kept = i;
        if (run > target) {
          pick = i;
          break;
        }
      }
      if (tie) ++ties_seen;
    }
    if (pick < 0) pick = last_kept;
    const float xt = to_f32(row[pick]) / Tm;
    token[r] = pick;
    logprob[r] = (xt - M) - logf(Zf);
    status[r] = 0;
  }
  if (processed) {
    uint32_t rank = ties_after;
    for (int64_t i = s1 - 1; i >= s0; --i) {
      const float x = to_f32(row[i]) / Tm;
      uint32_t rk = rank;
      const bool tie = okey(x) == pkey;
      processed[r * V + i] = kept_at(x, rk) ? x : -INFINITY;
      if (tie) ++rank;
    }
  }
}

}  // namespace

extern "C" int acorn_sample(const void* logits, int64_t rows, int64_t vocab, int dtype,
                            const float* temperature, const int32_t* top_k, const float* top_p,
                            const float* uniform, int64_t* token, float* logprob,
                            float* processed, int32_t* status, void* stream) {
  if (rows < 0 || vocab <= 0 || rows > 0x7fffffff || vocab > ((int64_t)1 << 31))
    return ACORN_ERR_SHAPE;
  if (rows == 0) return ACORN_OK;
  if (!logits || !temperature || !top_k || !top_p || !uniform || !token || !logprob || !status)
    return ACORN_ERR_VALUE;
  hipStream_t st = (hipStream_t)stream;
  dim3 grid((unsigned)rows), block(kNT);
  switch (dtype) {
    case ACORN_F32:
      sample_kernel<float><<<grid, block, 0, st>>>((const float*)logits, vocab, temperature, top_k, top_p, uniform, token, logprob, processed, status);
      break;
    case ACORN_F16:
      sample_kernel<_Float16><<<grid, block, 0, st>>>((const _Float16*)logits, vocab, temperature, top_k, top_p, uniform, token, logprob, processed, status);
      break;
    case ACORN_BF16:
      sample_kernel<__bf16><<<grid, block, 0, st>>>((const __bf16*)logits, vocab, temperature, top_k, top_p, uniform, token, logprob, processed, status);
      break;
    default:
      return ACORN_ERR_DTYPE;
  }
  ACORN_LAUNCH_CHECK();
  return ACORN_OK;
}
