// Weight-only GEMM y[M,N] = x[M,K] @ dequant(W)[N,K]^T on gfx950 MFMA.
//
// Formats (acorn_hip.h): dense bf16, int8 per-channel (fp16 scale [N], the
// reference's W8A16, acorninfer/quant/quantize.py:89-99) and packed uint4
// group-128 (fp16 scale [N,K/128], optional fp16 zero [N,K/128]; byte =
// u_even | u_odd << 4 as in quantize.py:122-131; symmetric int4 v in [-8,7]
// is stored as u = v + 8 with zero = -8*scale, which dequantises exactly).
//
// Design (decode is HBM-bound on the weight stream, so the goal is to keep
// the VALU cost of dequantisation below the HBM rate and to have every weight
// byte in flight early):
//  * v_mfma_f32_16x16x32_bf16 with the WEIGHTS as the 16-row A operand and x
//    (M <= 16 rows, zero/duplicate padded) as the B operand. A 16-byte load
//    per lane feeds 1 (bf16), 2 (int8) or 4 (int4) MFMAs.
//  * int4 -> bf16 in two VALU ops per dword: (w >> 4p) & 0x000F000F | 0x43004300
//    gives the bf16 pair (128+u_p, 128+u_{p+4}); the (p, p+4) pairing is a
//    k permutation that is applied once to x when it is staged into LDS.
//  * int8 -> bf16 via (q ^ 0x80) -> v_cvt_f32_ubyteN -> v_cvt_pk_bf16_f32,
//    i.e. 128+q, exact.
//  * The +128 offset is removed with sum_k x = ones-MFMA on the same B
//    operand: y = s * (C - 128 X) (+ zero X for int4), applied per 128-group
//    (int4) or once at the end (int8).
//  * x for the workgroup's K chunk is staged in LDS in MFMA-B order
//    ([k/8][row][8]), so every B fetch is one conflict-free ds_read_b128.
//  * A workgroup = NW waves splitting the chunk's K; waves are reduced through
//    LDS in fixed order; split-K across workgroups writes fp32 partials that
//    the consumer (or acorn_splitk_reduce) sums in fixed order: results are
//    bitwise deterministic and graph-replay stable.
#include <algorithm>

#include "common.h"

using namespace acorn;

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <int WFMT> struct Fmt;
template <> struct Fmt<ACORN_WFMT_BF16> {
  static constexpr int KU = 32;     // k covered by one 16-byte lane load across the wave
  static constexpr int MPU = 1;     // MFMAs per unit
  static constexpr int BPK_NUM = 2, BPK_DEN = 1;  // bytes per k = NUM/DEN
};
template <> struct Fmt<ACORN_WFMT_W8> {
  static constexpr int KU = 64, MPU = 2, BPK_NUM = 1, BPK_DEN = 1;
};
template <> struct Fmt<ACORN_WFMT_W4> {
  static constexpr int KU = 128, MPU = 4, BPK_NUM = 1, BPK_DEN = 2;
};

__device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                  __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// int4: 8 nibbles (columns c..c+7) -> bf16 (128+u) in MFMA item order
// (p, p+4) per dword.
__device__ __forceinline__ u32x4 unpack_w4(uint32_t w) {
  u32x4 r;
  r[0] = (w & 0x000F000Fu) | 0x43004300u;
  r[1] = ((w >> 4) & 0x000F000Fu) | 0x43004300u;
  r[2] = ((w >> 8) & 0x000F000Fu) | 0x43004300u;
  r[3] = ((w >> 12) & 0x000F000Fu) | 0x43004300u;
  return r;
}

// Byte I of v as float (selects v_cvt_f32_ubyteI).
template <int I> __device__ __forceinline__ float ubyte_f32(uint32_t v) {
  return (float)((v >> (8 * I)) & 0xffu);
}

// int8: 8 signed bytes -> bf16 (128+q) in natural order.
__device__ __forceinline__ u32x4 unpack_w8(uint32_t lo, uint32_t hi) {
  lo ^= 0x80808080u;
  hi ^= 0x80808080u;
  u32x4 r;
  r[0] = pack_bf16x2(ubyte_f32<0>(lo), ubyte_f32<1>(lo));
  r[1] = pack_bf16x2(ubyte_f32<2>(lo), ubyte_f32<3>(lo));
  r[2] = pack_bf16x2(ubyte_f32<0>(hi), ubyte_f32<1>(hi));
  r[3] = pack_bf16x2(ubyte_f32<2>(hi), ubyte_f32<3>(hi));
  return r;
}

__device__ __forceinline__ float h2f(const _Float16* p, size_t i) { return (float)p[i]; }

// Grid: x = N / (16*RT) row blocks, y = ksplit, z = ceil(M / (16*MT)) m blocks.
// Each workgroup covers K range [y*Kwg, (y+1)*Kwg), Kwg = nchunk * NW*UPW*KU.
template <int WFMT, int RT, int MT, int UPW>
__global__ __launch_bounds__(256) void wgemm_kernel(
    const __bf16* __restrict__ x, const uint8_t* __restrict__ w,
    const _Float16* __restrict__ scale, const _Float16* __restrict__ zero,
    __bf16* __restrict__ out, float* __restrict__ part, int M, int N, int K, int nchunk,
    int log2R) {
  using F = Fmt<WFMT>;
  constexpr int KU = F::KU, MPU = F::MPU;
  constexpr int ROWS = 16 * RT;
  extern __shared__ __align__(16) unsigned char smem[];

  const int NW = blockDim.x / kWave;
  const int wid = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int lg = lane / 16, lr = lane % 16;
  const int R = 1 << log2R;                 // LDS rows per m tile
  const int n0 = blockIdx.x * ROWS;
  const int mblk = blockIdx.z * 16 * MT;
  const int kc = NW * UPW * KU;             // k per chunk
  const int k_wg0 = blockIdx.y * nchunk * kc;
  const int groups_c = kc / 128;            // int4 groups per chunk
  const size_t wrow_bytes = (size_t)K * F::BPK_NUM / F::BPK_DEN;

  // LDS carve-up: x chunk [MT][kc/8][R][16B] | int4 scale [groups_c][ROWS] | zero
  u32x4* xs = (u32x4*)smem;
  const int xs_vecs = MT * (kc / 8) * R;
  _Float16* s_lds = (_Float16*)(smem + (size_t)xs_vecs * 16);
  _Float16* z_lds = s_lds + groups_c * ROWS;

  f32x4 acc[RT][MT];
  f32x4 xtot[MT];  // int8: running sum_k x per column
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[rt][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) xtot[mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  const u32x4 ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};

  for (int ch = 0; ch < nchunk; ++ch) {
    const int kchunk0 = k_wg0 + ch * kc;
    const int kw0 = kchunk0 + wid * UPW * KU;  // this wave's first k
    // ---- issue this wave's weight loads (16 B per lane per unit) ---------
    u32x4 wreg[RT][UPW];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const uint8_t* rowp = w + (size_t)(n0 + rt * 16 + lr) * wrow_bytes;
#pragma unroll
      for (int u = 0; u < UPW; ++u) {
        const int k = kw0 + u * KU + (KU / 4) * lg;
        wreg[rt][u] = *(const u32x4*)(rowp + (size_t)k * F::BPK_NUM / F::BPK_DEN);
      }
    }
    // ---- stage x chunk into LDS (MFMA-B order; int4 k-permutation) -------
    const int cpr = kc / 8;  // 16-byte pieces per row
    for (int p = threadIdx.x; p < MT * R * cpr; p += blockDim.x) {
      const int c = p % cpr, rr = p / cpr;  // rr = mt * R + row
      const int mt = rr / R, row = rr % R;
      const int m = mblk + mt * 16 + row;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (m < M) {
        v = *(const u32x4*)(x + (size_t)m * K + kchunk0 + c * 8);
        if constexpr (WFMT == ACORN_WFMT_W4) {
          // items [x0,x4,x1,x5,x2,x6,x3,x7] to match unpack_w4's pairing
          u32x4 t;
          t[0] = __builtin_amdgcn_perm(v[2], v[0], 0x05040100u);
          t[1] = __builtin_amdgcn_perm(v[2], v[0], 0x07060302u);
          t[2] = __builtin_amdgcn_perm(v[3], v[1], 0x05040100u);
          t[3] = __builtin_amdgcn_perm(v[3], v[1], 0x07060302u);
          v = t;
        }
      }
      xs[((size_t)mt * cpr + c) * R + row] = v;
    }
    if constexpr (WFMT == ACORN_WFMT_W4) {
      const int G = K / 128, g0 = kchunk0 / 128;
      for (int p = threadIdx.x; p < ROWS * groups_c; p += blockDim.x) {
        const int g = p % groups_c, row = p / groups_c;
        const size_t gi = (size_t)(n0 + row) * G + g0 + g;
        s_lds[g * ROWS + row] = scale[gi];
        if (zero) z_lds[g * ROWS + row] = zero[gi];
      }
    }
    __syncthreads();

    // ---- MFMA over this wave's units --------------------------------------
#pragma unroll
    for (int u = 0; u < UPW; ++u) {
      const int c0 = (wid * UPW * KU + u * KU) / 8 + (KU / 32) * lg;  // chunk-local
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        u32x4 bop[MPU];
#pragma unroll
        for (int j = 0; j < MPU; ++j)
          bop[j] = xs[((size_t)mt * cpr + c0 + j) * R + (lr & (R - 1))];
        if constexpr (WFMT == ACORN_WFMT_BF16) {
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) acc[rt][mt] = mfma(wreg[rt][u], bop[0], acc[rt][mt]);
        } else if constexpr (WFMT == ACORN_WFMT_W8) {
#pragma unroll
          for (int j = 0; j < MPU; ++j) xtot[mt] = mfma(ones, bop[j], xtot[mt]);
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) {
            const u32x4 q = wreg[rt][u];
            acc[rt][mt] = mfma(unpack_w8(q[0], q[1]), bop[0], acc[rt][mt]);
            acc[rt][mt] = mfma(unpack_w8(q[2], q[3]), bop[1], acc[rt][mt]);
          }
        } else {  // int4: one 128-group per unit
          f32x4 xg = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int j = 0; j < MPU; ++j) xg = mfma(ones, bop[j], xg);
          const int g = (wid * UPW * KU + u * KU) / 128;  // chunk-local group
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) {
            const u32x4 q = wreg[rt][u];
            f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < MPU; ++j) c = mfma(unpack_w4(q[j]), bop[j], c);
            const int rbase = g * ROWS + rt * 16 + 4 * lg;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float s = (float)s_lds[rbase + i];
              const float zc = zero ? (float)z_lds[rbase + i] - 128.f * s : -136.f * s;
              acc[rt][mt][i] += s * c[i] + zc * xg[i];
            }
          }
        }
      }
    }
    __syncthreads();
  }

  // ---- int8 per-channel epilogue: y = s * (C - 128 X) ---------------------
  if constexpr (WFMT == ACORN_WFMT_W8) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float s = h2f(scale, (size_t)n0 + rt * 16 + 4 * lg + i);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          acc[rt][mt][i] = s * (acc[rt][mt][i] - 128.f * xtot[mt][i]);
      }
    }
  }

  // ---- reduce the NW waves (fixed order) and store ------------------------
  const size_t plane = (size_t)M * N;
  auto store = [&](int rt, int mt, int i, int ln, float v) {
    const int n = n0 + rt * 16 + 4 * (ln / 16) + i;
    const int m = mblk + mt * 16 + (ln % 16);
    if (m >= M) return;
    if (part)
      part[(size_t)blockIdx.y * plane + (size_t)m * N + n] = v;
    else
      out[(size_t)m * N + n] = (__bf16)v;
  };
  if (NW == 1) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) store(rt, mt, i, lane, acc[rt][mt][i]);
    return;
  }
  float* red = (float*)smem;  // [NW][RT][MT][4][64]
  constexpr int TILE = RT * MT * 4 * kWave;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        red[(size_t)wid * TILE + ((rt * MT + mt) * 4 + i) * kWave + lane] = acc[rt][mt][i];
  __syncthreads();
  for (int e = threadIdx.x; e < TILE; e += blockDim.x) {
    float v = red[e];
    for (int ww = 1; ww < NW; ++ww) v += red[(size_t)ww * TILE + e];
    const int ln = e % kWave, i = (e / kWave) % 4, rm = e / (4 * kWave);
    store(rm / MT, rm % MT, i, ln, v);
  }
}

// fp32 weights and activations (the fp32 parity path; not a performance
// path). One wavefront per weight row; lanes stride K by 4-float vectors and
// the M dot products are finished with a wavefront reduction. Writes fp32
// y[m, n] into part[blockIdx.y, m, n] for the K range of split blockIdx.y.
__global__ __launch_bounds__(256) void f32_gemv_kernel(const float* __restrict__ x,
                                                       const float* __restrict__ w,
                                                       float* __restrict__ part, int M, int N,
                                                       int K, int kper) {
  const int wid = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int n = blockIdx.x * (blockDim.x / kWave) + wid;
  if (n >= N) return;
  const int k0 = blockIdx.y * kper, k1 = min(K, k0 + kper);
  const float* wr = w + (size_t)n * K;
  for (int m = 0; m < M; ++m) {
    const float* xr = x + (size_t)m * K;
    float a = 0.f;
    for (int k = k0 + lane; k < k1; k += kWave) a += xr[k] * wr[k];
    a = wave_sum(a);
    if (lane == 0) part[(size_t)blockIdx.y * M * N + (size_t)m * N + n] = a;
  }
}

// Split-K reduction (fixed order) with the output cast.
template <typename T>
__global__ void splitk_reduce_kernel(const float* __restrict__ part, int nsplit, size_t count,
                                     T* __restrict__ out) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= count) return;
  float a = part[i];
  for (int s = 1; s < nsplit; ++s) a += part[(size_t)s * count + i];
  out[i] = (T)a;
}

struct Cfg {
  int rt, mt, upw;
};

template <int WFMT, int RT, int MT, int UPW>
void launch_one(dim3 grid, dim3 block, size_t lds, hipStream_t st, const void* x, const void* w,
                const void* s, const void* z, void* out, float* part, int M, int N, int K,
                int nchunk, int log2R) {
  auto kfn = wgemm_kernel<WFMT, RT, MT, UPW>;
  kfn<<<grid, block, lds, st>>>((const __bf16*)x, (const uint8_t*)w, (const _Float16*)s,
                                (const _Float16*)z, (__bf16*)out, part, M, N, K, nchunk, log2R);
}

template <int WFMT, int RT, int MT>
int dispatch_upw(int upw, dim3 grid, dim3 block, size_t lds, hipStream_t st, const void* x,
                 const void* w, const void* s, const void* z, void* out, float* part, int M,
                 int N, int K, int nchunk, int log2R) {
  switch (upw) {
    case 2: launch_one<WFMT, RT, MT, 2>(grid, block, lds, st, x, w, s, z, out, part, M, N, K, nchunk, log2R); return 0;
    case 4: launch_one<WFMT, RT, MT, 4>(grid, block, lds, st, x, w, s, z, out, part, M, N, K, nchunk, log2R); return 0;
    case 8: launch_one<WFMT, RT, MT, 8>(grid, block, lds, st, x, w, s, z, out, part, M, N, K, nchunk, log2R); return 0;
  }
  return ACORN_ERR_UNSUPPORTED;
}

template <int WFMT>
int dispatch_cfg(const Cfg& c, dim3 grid, dim3 block, size_t lds, hipStream_t st, const void* x,
                 const void* w, const void* s, const void* z, void* out, float* part, int M,
                 int N, int K, int nchunk, int log2R) {
#define ACORN_CASE(RT_, MT_)                                                                 \
  if (c.rt == RT_ && c.mt == MT_)                                                            \
    return dispatch_upw<WFMT, RT_, MT_>(c.upw, grid, block, lds, st, x, w, s, z, out, part, M, \
                                        N, K, nchunk, log2R);
  ACORN_CASE(1, 1)
  ACORN_CASE(2, 1)
  ACORN_CASE(1, 2)
  ACORN_CASE(1, 4)
#undef ACORN_CASE
  return ACORN_ERR_UNSUPPORTED;
}

int ilog2_ceil(int v) {
  int r = 0;
  while ((1 << r) < v) ++r;
  return r;
}

int ku_of(int wfmt) {
  if (wfmt == ACORN_WFMT_F32) return 4;
  return wfmt == ACORN_WFMT_BF16 ? 32 : wfmt == ACORN_WFMT_W8 ? 64 : 128;
}

// Plan: M-tiles, units per wave, waves, k-split. Keeps the LDS x chunk
// <= 64 KiB and every weight byte in a register load issued up front.
int plan(int64_t M, int64_t N, int64_t K, int wfmt, int want_partials, Cfg* cfg, int* nw,
         int* ksplit, int* nchunk) {
  const int ku = ku_of(wfmt);
  if (M <= 0 || N <= 0 || K <= 0) return ACORN_ERR_SHAPE;
  if (wfmt == ACORN_WFMT_F32) {
    cfg->rt = 1;
    cfg->mt = 1;
    cfg->upw = 1;
    *nw = 4;
    *ksplit = 1;
    *nchunk = 1;
    return ACORN_OK;
  }
  cfg->mt = M <= 16 ? 1 : M <= 32 ? 2 : 4;
  cfg->rt = 1;
  const int R = cfg->mt == 1 ? (1 << ilog2_ceil((int)M)) : 16;
  if (N % 16) return ACORN_ERR_SHAPE;
  if (K % ku) return ACORN_ERR_SHAPE;
  // units per wave (8 -> every lane holds 128 B of weights per row tile)
  int upw = 8;
  while (upw > 2 && K % (ku * upw)) upw /= 2;
  if (K % (ku * upw)) return ACORN_ERR_SHAPE;
  // waves per workgroup along K: as many as divide K, <= 4
  int w = 4;
  while (w > 1 && (K % ((int64_t)ku * upw * w))) --w;
  // LDS budget for the x chunk
  while (w > 1 && (int64_t)cfg->mt * R * ku * upw * w * 2 > 64 * 1024) --w;
  while (K % ((int64_t)ku * upw * w)) --w;
  const int64_t kc = (int64_t)ku * upw * w;
  const int64_t chunks = K / kc;
  cfg->upw = upw;
  *nw = w;
  if (want_partials) {
    *ksplit = (int)chunks;
    *nchunk = 1;
  } else {
    *ksplit = 1;
    *nchunk = (int)chunks;
  }
  return ACORN_OK;
}

}  // namespace

extern "C" int acorn_gemm_plan(int64_t M, int64_t N, int64_t K, int wfmt, int want_partials,
                               int* rt, int* nw, int* ksplit) {
  Cfg c;
  int w, ks, nch;
  int rc = plan(M, N, K, wfmt, want_partials, &c, &w, &ks, &nch);
  if (rc) return rc;
  if (rt) *rt = c.rt;
  if (nw) *nw = w;
  if (ksplit) *ksplit = ks;
  return ACORN_OK;
}

extern "C" int acorn_quant_gemm(const void* x, const void* w, const void* scale,
                                const void* zero, void* out_bf16, float* out_part, int64_t M,
                                int64_t N, int64_t K, int wfmt, int rt, int nw, int ksplit,
                                void* stream) {
  if (wfmt != ACORN_WFMT_BF16 && wfmt != ACORN_WFMT_W8 && wfmt != ACORN_WFMT_W4 &&
      wfmt != ACORN_WFMT_F32)
    return ACORN_ERR_DTYPE;
  if (M < 0 || N <= 0 || K <= 0) return ACORN_ERR_SHAPE;
  if (M == 0) return ACORN_OK;
  if (wfmt == ACORN_WFMT_F32) {
    // fp32 output always goes through out_part ([ksplit, M, N]).
    if (!x || !w || !out_part) return ACORN_ERR_VALUE;
    if (M > 65535 || N > ((int64_t)1 << 30) || K > ((int64_t)1 << 30)) return ACORN_ERR_SHAPE;
    const int ks = ksplit > 0 ? ksplit : 1;
    const int64_t kper = (K + ks - 1) / ks;
    dim3 grid((unsigned)((N + 3) / 4), (unsigned)ks), block(256);
    f32_gemv_kernel<<<grid, block, 0, (hipStream_t)stream>>>(
        (const float*)x, (const float*)w, out_part, (int)M, (int)N, (int)K, (int)kper);
    ACORN_LAUNCH_CHECK();
    return ACORN_OK;
  }
  if (!x || !w || (wfmt != ACORN_WFMT_BF16 && !scale)) return ACORN_ERR_VALUE;
  if (!out_bf16 && !out_part) return ACORN_ERR_VALUE;
  if (M > 65535 * 64 || N > ((int64_t)1 << 30) || K > ((int64_t)1 << 30)) return ACORN_ERR_SHAPE;
  Cfg c;
  int pw, pks, pnch;
  int rc = plan(M, N, K, wfmt, out_part != nullptr, &c, &pw, &pks, &pnch);
  if (rc) return rc;
  if (rt > 0) c.rt = rt;
  if (nw > 0) pw = nw;
  if (ksplit > 0) pks = ksplit;
  if (!out_part && pks != 1) return ACORN_ERR_VALUE;
  const int ku = ku_of(wfmt);
  const int64_t rows = 16 * (int64_t)c.rt;
  if (N % rows) return ACORN_ERR_SHAPE;
  if (pw < 1 || pw > 4 || pks < 1) return ACORN_ERR_SHAPE;
  // Fit (waves, units per wave) so that ksplit workgroups tile K exactly.
  if (K % ((int64_t)ku * c.upw * pw * pks)) {
    bool found = false;
    for (int ww = pw; ww >= 1 && !found; --ww)
      for (int u = c.upw; u >= 2 && !found; u /= 2)
        if (K % ((int64_t)ku * u * ww * pks) == 0) {
          pw = ww;
          c.upw = u;
          found = true;
        }
    if (!found) return ACORN_ERR_SHAPE;
  }
  const int64_t kc = (int64_t)ku * c.upw * pw;
  const int64_t nchunk = K / (kc * pks);
  const int R = c.mt == 1 ? (1 << ilog2_ceil((int)std::min<int64_t>(M, 16))) : 16;
  const int log2R = ilog2_ceil(R);
  const int groups_c = (int)(kc / 128);
  size_t lds = (size_t)c.mt * (kc / 8) * R * 16;
  if (wfmt == ACORN_WFMT_W4) lds += (size_t)groups_c * rows * 2 * 2;
  const size_t red = (size_t)pw * c.rt * c.mt * 4 * kWave * 4;
  lds = std::max(lds, red);
  if (lds > 160 * 1024) return ACORN_ERR_UNSUPPORTED;
  const int64_t mblocks = (M + 16 * c.mt - 1) / (16 * c.mt);
  dim3 grid((unsigned)(N / rows), (unsigned)pks, (unsigned)mblocks), block(kWave * pw);
  hipStream_t st = (hipStream_t)stream;
  switch (wfmt) {
    case ACORN_WFMT_BF16: rc = dispatch_cfg<ACORN_WFMT_BF16>(c, grid, block, lds, st, x, w, scale, zero, out_bf16, out_part, (int)M, (int)N, (int)K, (int)nchunk, log2R); break;
    case ACORN_WFMT_W8: rc = dispatch_cfg<ACORN_WFMT_W8>(c, grid, block, lds, st, x, w, scale, zero, out_bf16, out_part, (int)M, (int)N, (int)K, (int)nchunk, log2R); break;
    case ACORN_WFMT_W4: rc = dispatch_cfg<ACORN_WFMT_W4>(c, grid, block, lds, st, x, w, scale, zero, out_bf16, out_part, (int)M, (int)N, (int)K, (int)nchunk, log2R); break;
  }
  if (rc) return rc;
  ACORN_LAUNCH_CHECK();
  return ACORN_OK;
}

extern "C" int acorn_splitk_reduce(const float* part, int64_t nsplit, int64_t count, void* out,
                                   int dtype, void* stream) {
  if (nsplit < 1 || count < 0) return ACORN_ERR_SHAPE;
  if (count == 0) return ACORN_OK;
  if (!part || !out) return ACORN_ERR_VALUE;
  dim3 grid((unsigned)((count + 255) / 256)), block(256);
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case ACORN_F32: splitk_reduce_kernel<float><<<grid, block, 0, st>>>(part, (int)nsplit, (size_t)count, (float*)out); break;
    case ACORN_F16: splitk_reduce_kernel<_Float16><<<grid, block, 0, st>>>(part, (int)nsplit, (size_t)count, (_Float16*)out); break;
    case ACORN_BF16: splitk_reduce_kernel<__bf16><<<grid, block, 0, st>>>(part, (int)nsplit, (size_t)count, (__bf16*)out); break;
    default: return ACORN_ERR_DTYPE;
  }
  ACORN_LAUNCH_CHECK();
  return ACORN_OK;
}
