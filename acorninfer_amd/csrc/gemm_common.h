// Device helpers shared by the weight-only GEMM kernels (quant_gemm.hip,
// w4_decode.hip, w8_decode.hip, bf16_decode.hip, dense_gemm.hip), the block
// layouts' index maps, and the interfaces of the kernels that quant_gemm.hip's
// planner dispatches to.
#pragma once

#include "common.h"

namespace acorn {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 h16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                  __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// int4: the 8 nibbles of a W4B word -> bf16 (128+u) pairs (nibble q, nibble
// q+4), q = 0..3: in the W4B nibble order (k offsets 0,2,4,6,1,3,5,7) that is
// k offsets (2q, 2q+1), the natural order of x.
// The mask and the bias are made opaque register values (an SGPR and a VGPR):
// with literal operands the compiler emits v_and_b32 + v_or_b32 (gfx950's
// VOP3 forms take no literal), with registers it can use one v_and_or_b32.
__device__ __forceinline__ u32x4 unpack_w4(uint32_t w) {
  uint32_t m = 0x000F000Fu, c = 0x43004300u;
  asm("" : "+s"(m));
  asm("" : "+v"(c));
  u32x4 r;
  r[0] = (w & m) | c;
  r[1] = ((w >> 4) & m) | c;
  r[2] = ((w >> 8) & m) | c;
  r[3] = ((w >> 12) & m) | c;
  return r;
}

// Byte I of v as float (selects v_cvt_f32_ubyteI).
template <int I> __device__ __forceinline__ float ubyte_f32(uint32_t v) {
  return (float)((v >> (8 * I)) & 0xffu);
}

// NDW consecutive dwords from a 4*NDW-byte aligned address (one vector load
// per 16 bytes).
template <int NDW>
__device__ __forceinline__ void load_dwords(const void* p, uint32_t (&d)[NDW]) {
  if constexpr (NDW == 1) {
    d[0] = *(const uint32_t*)p;
  } else if constexpr (NDW == 2) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 t = *(const u32x2*)p;
    d[0] = t[0];
    d[1] = t[1];
  } else {
    static_assert(NDW % 4 == 0, "whole 16-byte pieces");
#pragma unroll
    for (int c = 0; c < NDW / 4; ++c) {
      const u32x4 t = *(const u32x4*)((const uint32_t*)p + 4 * c);
#pragma unroll
      for (int j = 0; j < 4; ++j) d[4 * c + j] = t[j];
    }
  }
}

// Lane l gets lane (l + 8) mod 16 of its 16-lane row (DPP row rotate by 8):
// the paired-x form of the direct kernels (M <= 8) loads two k blocks of x
// with one instruction, lanes 0..7 the first block's rows and 8..15 the
// second's, and rotates the second into lanes 0..7 for its MFMAs (columns
// 8..15 of an MFMA then hold the other block's x: outputs never stored).
__device__ __forceinline__ u32x4 rot8(const u32x4& v) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    r[i] = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v[i], 0x128, 0xF, 0xF, false);
  return r;
}

// s_h * v + acc in fp32, s_h the fp16 number h of a run of packed halves
// (exactly converted, one rounding): the compiler makes it one v_fma_mix_f32
// that selects the half of the packed dword itself (op_sel), so no shift
// touches a loaded scale before its use. h must fold to a constant. Plain
// code rather than asm: the compiler then puts in the wait states an MFMA
// result needs before a VALU reads it, wherever the accumulators live (VGPRs
// under a 512-thread launch bound, AGPRs otherwise).
template <int NDW>
__device__ __forceinline__ float fma_half(const uint32_t (&d)[NDW], int h, float v, float acc) {
  const uint32_t w = d[h / 2];
  const _Float16 s = __builtin_bit_cast(_Float16, (uint16_t)((h & 1) ? (w >> 16) : (w & 0xffffu)));
  return __builtin_fmaf((float)s, v, acc);
}

// SwiGLU epilogue of the fused gate|up projection: g, u rounded to bf16,
// act = round(round(silu(g)) * u), silu(g) = g / (1 + exp(-g)) in fp32
// (models/qwen3.py:392-396, each torch bf16 op rounded).
__device__ __forceinline__ float swiglu_bf16(float g, float u) {
#pragma clang fp contract(off)
  g = (float)(__bf16)g;
  u = (float)(__bf16)u;
  const float sg = (float)(__bf16)(g / (1.0f + expf(-g)));
  return sg * u;
}

// ---- the RMSNorm folded into the decode GEMMs (direct kernels) ------------
// RMSNorm(v) @ W^T = inv * (bf16(v * w) @ W^T) per row (inv = 1 / rms(v), w
// the norm weight), so the norm splits between the two projections around
// it. A producer projection (o, down) that finishes its columns in one
// launch (one split) writes the new residual v = bf16(res + bf16(y)), the
// weighted rows xw = bf16(v * w) of the next norm and, per 16 columns of v,
// the fp32 sum of v^2 (ss [M][N / 16]). The consumer projection (gate|up, the
// next layer's qkv) is the plain GEMM of xw whose rows are multiplied by inv
// = 1 / sqrt(sum ss / cols + eps) before its epilogue (K1's inv, rmsnorm.hip,
// with the sum of squares added in another order; the bf16 rounding falls on
// v * w instead of (v * inv) * w).
struct NormIn {
  const float* ss;       // [M][nss] per-16-column sums of squares of the residual
  int nss;               // K / 16
  float eps;
};
struct ResidOut {
  const __bf16* res;     // [M, N] residual in
  __bf16* res_out;       // [M, N] residual out (may alias res: each element is read and
                         // written by the same lane)
  float* ss;             // [M][N / 16]
  const __bf16* nw;      // [N] the next norm's weight
  __bf16* xw;            // [M, N] bf16(res_out * nw)
};

// Row m's 1 / rms from its nss partial sums, the same value in every lane
// that serves row m. With mp the power of two >= M (at most 16), lane l
// serves row l % mp (rows past M re-read row M - 1) and adds part l / mp of
// its sums, in order: 64 / mp parts of per = ceil(nss mp / 64) sums; the
// parts are then added by an xor butterfly over lane strides mp, 2 mp .. 32.
// Every lane loads, so a small batch reads each sum once instead of once per
// lane group. In two halves, so that the sums are requested before a
// kernel's first weights and added after them (loads complete in order:
// waiting for the sums does not wait for the weights): parts of 4, 8, 16, 32
// or 64 sums go through registers, others are read at the finish.
constexpr int kNormRegs = 64;
struct NormRegs {
  f32x4 v[kNormRegs / 4];
};
// v of lane l ^ O (O < 32: a bitmask-mode ds_swizzle, no address register)
template <int O>
__device__ __forceinline__ float swizzle_xor(float v) {
  static_assert(O > 0 && O < 32 && (O & (O - 1)) == 0, "a lane stride inside 32 lanes");
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1F | (O << 10)));
}
__device__ __forceinline__ int norm_rows(int M) {
  return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : M <= 8 ? 8 : 16;
}
// vectors per lane in registers: parts of 4, 8, 16, 32 or 64 sums; 0 = read
// at the finish
__device__ __forceinline__ int norm_vectors(int nss, int parts) {
  const int per = nss / parts;
  if (nss % parts || per % 4) return 0;
  const int nv = per / 4;
  return (nv & (nv - 1)) == 0 && nv <= kNormRegs / 4 ? nv : 0;
}
template <int NV>
__device__ __forceinline__ void norm_load(const float* p, NormRegs& r) {
#pragma unroll
  for (int t = 0; t < NV; ++t) r.v[t] = *(const f32x4*)(p + 4 * t);
}
template <int NV>
__device__ __forceinline__ float norm_add(const NormRegs& r) {
#pragma clang fp contract(off)
  float s = 0.f;
#pragma unroll
  for (int t = 0; t < NV; ++t) {
    s = s + r.v[t][0];
    s = s + r.v[t][1];
    s = s + r.v[t][2];
    s = s + r.v[t][3];
  }
  return s;
}
__device__ __forceinline__ void norm_issue(const NormIn& n, int M, int lane, NormRegs& r) {
  const int mp = norm_rows(M), parts = kWave / mp;
  const int nv = norm_vectors(n.nss, parts);
  const float* p = n.ss + (size_t)min(lane % mp, M - 1) * n.nss + (lane / mp) * 4 * nv;
  switch (nv) {                                            // uniform
    case 1: norm_load<1>(p, r); break;
    case 2: norm_load<2>(p, r); break;
    case 4: norm_load<4>(p, r); break;
    case 8: norm_load<8>(p, r); break;
    case 16: norm_load<16>(p, r); break;
    default: break;
  }
}
__device__ __forceinline__ float norm_finish(const NormIn& n, int M, int lane, int cols,
                                             const NormRegs& r) {
#pragma clang fp contract(off)
  const int mp = norm_rows(M), parts = kWave / mp;
  float s = 0.f;
  switch (norm_vectors(n.nss, parts)) {
    case 1: s = norm_add<1>(r); break;
    case 2: s = norm_add<2>(r); break;
    case 4: s = norm_add<4>(r); break;
    case 8: s = norm_add<8>(r); break;
    case 16: s = norm_add<16>(r); break;
    default: {
      const int per = (n.nss + parts - 1) / parts;
      const int t0 = (lane / mp) * per, t1 = min(t0 + per, n.nss);
      const float* p = n.ss + (size_t)min(lane % mp, M - 1) * n.nss;
      for (int t = t0; t < t1; ++t) s = s + p[t];
    }
  }
  // strides below 32 by a swizzle (lane ^ O within 32 lanes), 32 by a permute
  if (mp <= 1) s = s + swizzle_xor<1>(s);
  if (mp <= 2) s = s + swizzle_xor<2>(s);
  if (mp <= 4) s = s + swizzle_xor<4>(s);
  if (mp <= 8) s = s + swizzle_xor<8>(s);
  s = s + swizzle_xor<16>(s);
  s = s + __shfl_xor(s, 32);
  return 1.0f / sqrtf(s / (float)cols + n.eps);
}

// The producer's epilogue for the 4 columns n .. n + 3 of row m held by one
// lane (y fp32, off = m N + n): v = bf16(res + bf16(y)) stored to res_out and
// bf16(v * w) to xw; returns their sum of squares in column order.
__device__ __forceinline__ float resid_store4(const ResidOut& r, size_t off, int n,
                                              const float (&y)[4]) {
#pragma clang fp contract(off)
  uint32_t rin[2], win[2];
  __builtin_memcpy(rin, r.res + off, sizeof(rin));
  __builtin_memcpy(win, r.nw + n, sizeof(win));
  float v[4], vw[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float rv = __uint_as_float(i & 1 ? rin[i / 2] & 0xffff0000u : rin[i / 2] << 16);
    const float wv = __uint_as_float(i & 1 ? win[i / 2] & 0xffff0000u : win[i / 2] << 16);
    const float yb = (float)(__bf16)y[i];
    v[i] = (float)(__bf16)(rv + yb);
    vw[i] = v[i] * wv;
  }
  const uint32_t o[2] = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
  __builtin_memcpy(r.res_out + off, o, sizeof(o));
  const uint32_t ow[2] = {pack_bf16x2(vw[0], vw[1]), pack_bf16x2(vw[2], vw[3])};
  __builtin_memcpy(r.xw + off, ow, sizeof(ow));
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) s = s + v[i] * v[i];
  return s;
}

// ---- W4B: int4 weights in 1 KB blocks (ACORN_WFMT_W4B) -------------------
// Block (n/16, g) holds rows 16*(n/16) .. +15 x the 128 k of group g as one
// wave's MFMA A operand: lane (c%4)*16 + n%16 has the 16 bytes of row n,
// k in [32c, 32c+32) (c = k/32 within the tensor); word j of those bytes
// holds k 32c + 8j .. + 7 with nibble p (bits 4p..4p+3) at k offset
// 0,2,4,6,1,3,5,7 for p = 0..7.
__host__ __device__ inline size_t w4b_chunk_offset(int64_t n, int64_t c, int64_t K) {
  return ((size_t)(n / 16) * (size_t)(K / 128) + (size_t)(c / 4)) * 1024 +
         (size_t)((c % 4) * 16 + n % 16) * 16;
}
// W8B: int8 weights (stored as q + 128) in 1 KB blocks of 16 rows x 64 k;
// the 16 bytes of row n, k in [16c, 16c+16) (c = k/16 within the tensor).
__host__ __device__ inline size_t w8b_chunk_offset(int64_t n, int64_t c, int64_t K) {
  return ((size_t)(n / 16) * (size_t)(K / 64) + (size_t)(c / 4)) * 1024 +
         (size_t)((c % 4) * 16 + n % 16) * 16;
}
// BF16B: bf16 weights in 1 KB blocks of 16 rows x 32 k; the 8 bf16 (16
// bytes) of row n, k in [8c, 8c+8) (c = k/8 within the tensor), as a byte
// offset.
__host__ __device__ inline size_t bf16b_piece_offset(int64_t n, int64_t c, int64_t K) {
  return ((size_t)(n / 16) * (size_t)(K / 32) + (size_t)(c / 4)) * 1024 +
         (size_t)((c % 4) * 16 + n % 16) * 16;
}
// Scale (zero) of row n, group g: records of 4 rows x 4 groups per lane
// group, so a lane's scales of consecutive groups are contiguous.
__host__ __device__ inline size_t w4b_half_index(int64_t n, int64_t g, int64_t K) {
  return ((size_t)(n / 16) * (size_t)(K / 512) + (size_t)(g / 4)) * 64 +
         (size_t)((n % 16) / 4) * 16 + (size_t)(g % 4) * 4 + (size_t)(n % 4);
}

// ---- the W4B decode kernels (w4_decode.hip), M <= 64 ------------------------
// cfg knobs: rt (row tiles of 16 per wave), upw (groups per pipeline stage),
// nw (waves per workgroup; above 16 rows 10*nw + kw when kw waves share rows
// and split K), ksplit, depth (stages in flight per wave); 0 = choose.
// M <= 16 runs the direct kernel (x read into MFMA registers by every wave),
// 16 < M <= 64 the kernel that stages x in LDS.
struct W4bPlan {
  bool direct;     // the M <= 16 kernel
  int rt, upw, nw, ksplit, depth;
  int kw;          // K slices per row group (waves sharing rows)
  int nw_field;    // the cfg value of nw (nw, or 10*nw + kw)
  int R;           // x rows staged in LDS (16 mb; M for the direct kernel)
  int mb;          // 16-column blocks of x per wave (M <= 16 mb)
  int groups;      // workgroups along N
  size_t lds;      // dynamic LDS bytes
  bool swiglu;
  int mode;        // the direct kernel: 0 plain, 1 NormIn, 2 ResidOut (as DirectPlan)
  bool hx;         // the direct kernel's paired-x form (M <= 8, upw 2)
};
int w4b_make_plan(int64_t M, int64_t N, int64_t K, const int* cfg, bool swiglu, W4bPlan* p);
// out (bf16 [M,N], or act [M,N/2] for swiglu) when given and ksplit == 1;
// otherwise fp32 partials part[ksplit, M, N].
int w4b_launch(const W4bPlan& p, const void* x, const void* w, const void* scale,
               const void* zero, void* out, float* part, int64_t M, int64_t N, int64_t K,
               const NormIn* ni, const ResidOut* ro, hipStream_t st);

// ---- the int4 GEMM for 17..256 rows (w4_decode.hip) ----------------------------
// cfg knobs (rt = kMidRT marks the request): upw = row tiles per wave (1, 2),
// nw = waves (4, 8), ksplit, tpw = groups in flight (2, 4); 64 x rows per
// workgroup, x streamed through LDS one 128-k group at a time.
struct W4mPlan {
  int rt, nw, ksplit, depth;
  int groups;      // row blocks of nw * rt * 16 rows
  int mblocks;     // blocks of 64 x rows
  size_t lds;
};
int w4m_make_plan(int64_t M, int64_t N, int64_t K, const int* cfg, W4mPlan* p);
int w4m_launch(const W4mPlan& p, const void* x, const void* w, const void* scale, void* out,
               float* part, int64_t M, int64_t N, int64_t K, hipStream_t st);
// ---- the int8 GEMM for 17..256 rows (w8_decode.hip) ----------------------------
// The same knobs and request (rt = kMidRT) on W8B weights: upw = row tiles per
// wave (1, 2), nw = waves (4, 8), ksplit, tpw = 128-k steps in flight (2, 4).
struct W8mPlan {
  int rt, nw, ksplit, depth;
  int groups;      // row blocks of nw * rt * 16 rows
  int mblocks;     // blocks of 64 x rows
  size_t lds;
};
int w8m_make_plan(int64_t M, int64_t N, int64_t K, const int* cfg, W8mPlan* p);
int w8m_launch(const W8mPlan& p, const void* x, const void* w, const void* scale, void* out,
               float* part, int64_t M, int64_t N, int64_t K, hipStream_t st);
// W4B weights -> bf16 [N, K] in row order (N % 16 == 0, K % 512 == 0).
int w4b_dequant(const void* w, const void* scale, void* out, int64_t N, int64_t K,
                hipStream_t st);

// ---- the W8B and BF16B decode kernels (w8_decode.hip, bf16_decode.hip) ------
// M <= 16, weights in 1 KB blocks, x read straight into MFMA registers.
// cfg knobs: rt (row tiles of 16 per wave), upw (blocks per pipeline stage),
// nw (the wave layout: 1 or 4 waves on their own rows, 22 / 44 = 2 / 4 waves
// splitting K over shared rows), ksplit, depth (stages in flight).
struct DirectPlan {
  int rt, upw, nw_field, rg, kw, ksplit, depth;
  int groups;      // workgroups along N
  bool swiglu;
  int mode;        // 0 plain, 1 rows scaled by 1 / rms (NormIn), 2 residual epilogue (ResidOut)
  bool hx;         // the paired-x form (M <= 8, upw 2; see rot8)
};
int w8b_make_plan(int64_t M, int64_t N, int64_t K, const int* cfg, bool swiglu, DirectPlan* p);
// out (bf16 [M,N], or act [M,N/2] for swiglu) when given and ksplit == 1;
// otherwise fp32 partials part[ksplit, M, N] (each already scaled).
int w8b_launch(const DirectPlan& p, const void* x, const void* w, const void* scale, void* out,
               float* part, int64_t M, int64_t N, int64_t K, const NormIn* ni,
               const ResidOut* ro, hipStream_t st);
int bf16b_make_plan(int64_t M, int64_t N, int64_t K, const int* cfg, bool swiglu,
                    DirectPlan* p);
int bf16b_launch(const DirectPlan& p, const void* x, const void* w, void* out, float* part,
                 int64_t M, int64_t N, int64_t K, const NormIn* ni, const ResidOut* ro,
                 hipStream_t st);

// ---- the large-M bf16 GEMM (dense_gemm.hip) ---------------------------------
// out[M,N] = x[M,K] . w[N,K]^T, bf16 operands: (4 wn) x bm output tiles (wn
// weight rows per wave: 64 or 128; bm 64 or 128), weights prefetched `depth`
// K steps of 64 ahead (2 or 4), the K range cut into ks splits. fp32 output
// when out_f32 is given (split s into out_f32 + s*M*N), else bf16 into
// out_bf16 (ks == 1 only). blocked: w in the BF16B layout (every form but
// the register-staged 256 x 256 one).
bool dense_gemm_supported(int64_t N, int64_t K, int wn, int bm, int depth, int ks, bool blocked);
// gate|up (16-row interleave) with the SwiGLU epilogue: act [M, N / 2] bf16,
// one split, the direct-to-LDS form (bm 256, wn 128) and N % 32 == 0
bool dense_gemm_swiglu_supported(int64_t N, int64_t K, int wn, int bm, int depth, bool blocked);
int dense_gemm_swiglu_launch(const void* x, const void* w, void* act, int64_t M, int64_t N,
                             int64_t K, int wn, int bm, int depth, bool blocked, hipStream_t st);
int dense_gemm_launch(const void* x, const void* w, void* out_bf16, float* out_f32, int64_t M,
                      int64_t N, int64_t K, int wn, int bm, int depth, int ks, bool blocked,
                      hipStream_t st);

}  // namespace acorn
