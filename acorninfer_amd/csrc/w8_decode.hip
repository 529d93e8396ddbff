// Weight-only int8 GEMM at decode sizes (M <= 16) over the W8B block layout.
//
// y[M,N] = s[n] * (x[M,K] @ q[N,K]^T): q int8 per output channel with an fp16
// scale (the reference's production quant path, acorninfer/ops/quant_gemm.py:
// 125-154, _w8_gemm_kernel), bf16 x, fp32 accumulation.
//
// Built like the int4 direct kernel (w4_decode.hip):
//  * The weights of 16 rows x 64 k are one contiguous 1 KB block (ACORN_WFMT_W8B):
//    lane lg * 16 + r holds row r's 16 consecutive k 16 lg .. 16 lg + 15, so a
//    wave reads a block with one 16-byte load per lane (whole cache lines,
//    non-temporal policy) and feeds two v_mfma_f32_16x16x32_bf16 from it: MFMA
//    j takes the lane's bytes 8 j .. 8 j + 7, i.e. its k slots 8 lg .. 8 lg + 7
//    stand for k 16 lg + 8 j + i, and x is read in the same order.
//  * Each byte is stored as u = q + 128, so v_cvt_f32_ubyteN gives it as a
//    float and v_cvt_pk_bf16_f32 packs two (exact: u < 256 has 8 significant
//    bits): 1.5 VALU per weight. The bias is removed once per wave: an MFMA
//    chain of a constant -128 operand against x gives -128 X, added to every
//    tile at the end. The per-channel scale is applied in the epilogue.
//  * Every wave reads its x operands from memory straight into MFMA B
//    registers with its weights (no LDS staging, no barrier before the first
//    MFMA); KW > 1 waves of a workgroup split K over the same rows and add
//    their results through LDS in fixed order at the end.
//  * Split-K (ksplit > 1) writes scaled fp32 partials [ksplit, M, N], summed
//    in split order by the consumer (bitwise deterministic).
//  * MODE 1 / 2: the RMSNorm folded in as in bf16_decode.hip (results scaled
//    by the rows' 1 / rms, after the per-channel scale; the residual epilogue
//    with the weighted rows and the sums of squares).
#include "gemm_common.h"

using namespace acorn;

namespace {

struct W8dArgs {
  const __bf16* x;
  const uint8_t* w;
  const _Float16* scale;
  __bf16* out;    // bf16 [M, N] (act [M, N/2] with SWIGLU) when ksplit == 1
  float* part;    // fp32 [ksplit, M, N] otherwise
  int M, N, K;
  int kr;         // K range of a split (a multiple of 64 * KW * UPW * DEPTH)
  NormIn ni;      // MODE 1
  ResidOut ro;    // MODE 2
};

template <int RT, int UPW, bool HX>
struct W8Stage {
  u32x4 w[RT][UPW];          // block (tile rt, block u): this lane's 16 bytes
  // B operand of MFMA j of block u: x row lr, k 16 lg + 8 j .. (HX: of block
  // pair u / 2, lanes lr < 8 the even block's rows, lr >= 8 the odd one's)
  u32x4 x[HX ? UPW / 2 : UPW][2];
};

// bf16 -128 in every slot: an MFMA of it against x gives -128 X per column
constexpr uint32_t kNeg128x2 = 0xC300C300u;

// 8 biased bytes (k slots of one MFMA) -> bf16 (q + 128) in slot order
__device__ __forceinline__ u32x4 unpack_w8(uint32_t a, uint32_t b) {
  u32x4 r;
  r[0] = pack_bf16x2(ubyte_f32<0>(a), ubyte_f32<1>(a));
  r[1] = pack_bf16x2(ubyte_f32<2>(a), ubyte_f32<3>(a));
  r[2] = pack_bf16x2(ubyte_f32<0>(b), ubyte_f32<1>(b));
  r[3] = pack_bf16x2(ubyte_f32<2>(b), ubyte_f32<3>(b));
  return r;
}

// Grid: x = tile groups of RG * RT 16-row tiles, y = ksplit; block RG * KW
// waves. Row group r of workgroup b owns tiles (b RG + r) RT .. + RT - 1; its
// KW waves split the split's K range. Lane (lr, lg) holds x row min(lr, M - 1)
// (rows past M feed only columns that are never stored).
// HX (M <= 8, UPW even): the paired-x form (gemm_common.h, rot8).
template <int RT, int UPW, int DEPTH, int RG, int KW, bool SWIGLU, int MODE, bool HX = false>
__global__ __launch_bounds__(RG * KW * kWave) void w8b_direct_kernel(W8dArgs a) {
  static_assert(!HX || UPW % 2 == 0, "x in block pairs");
  constexpr int NW = RG * KW;
  constexpr bool NORM = MODE == 1;
  static_assert(MODE != 2 || !SWIGLU, "the residual epilogue replaces a plain output");
  const int wid = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int lg = lane >> 4, lr = lane & 15;
  const int rg = wid / KW, kq = wid % KW;
  const int KB = a.K / 64;                        // blocks per row
  const int t0 = (blockIdx.x * RG + rg) * RT;
  const bool active = t0 < a.N / 16;              // (N / 16) % RT == 0 by the plan
  const int tt = active ? t0 : 0;                 // idle waves read tile 0, store nothing
  const int BW = a.kr / (64 * KW);                // blocks of this wave
  const int kw0 = blockIdx.y * a.kr + kq * BW * 64;
  const int ns = BW / UPW;                        // stages, a multiple of DEPTH
  const uint8_t* wb = a.w + ((size_t)tt * KB + kw0 / 64) * 1024 + lane * 16;
  const __bf16* xb = HX ? a.x + (size_t)min(lr & 7, a.M - 1) * a.K + kw0 + 16 * lg + 64 * (lr >> 3)
                        : a.x + (size_t)min(lr, a.M - 1) * a.K + kw0 + 16 * lg;
  auto load = [&](int s, W8Stage<RT, UPW, HX>& r) {
#pragma unroll
    for (int u = 0; u < (HX ? UPW / 2 : UPW); ++u)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        r.x[u][j] = *(const u32x4*)(xb + (s * UPW + (HX ? 2 * u : u)) * 64 + 8 * j);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int u = 0; u < UPW; ++u)
        r.w[rt][u] = load_nt((const u32x4*)(wb + ((size_t)rt * KB + s * UPW + u) * 1024));
  };

  NormRegs nr;
  if constexpr (NORM) norm_issue(a.ni, a.M, lane, nr);
  W8Stage<RT, UPW, HX> ring[DEPTH];
  // in stage order, as the loop reissues them (the loop's static waits assume
  // that order; left free, the scheduler reorders the first stages' loads)
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) {
    load(d, ring[d]);
    __builtin_amdgcn_sched_barrier(0);
  }
  float inv = 1.f;
  if constexpr (NORM) inv = norm_finish(a.ni, a.M, lane, a.K, nr);
  f32x4 acc[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) acc[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
  f32x4 xacc = {0.f, 0.f, 0.f, 0.f};             // -128 X over the wave's K range
  const u32x4 neg128 = {kNeg128x2, kNeg128x2, kNeg128x2, kNeg128x2};
  auto compute = [&](const W8Stage<RT, UPW, HX>& r) {
#pragma unroll
    for (int u = 0; u < UPW; ++u) {
      u32x4 xu[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) xu[j] = HX && (u & 1) ? rot8(r.x[u / 2][j]) : r.x[HX ? u / 2 : u][j];
#pragma unroll
      for (int j = 0; j < 2; ++j) xacc = mfma(neg128, xu[j], xacc);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[rt] = mfma(unpack_w8(r.w[rt][u][2 * j], r.w[rt][u][2 * j + 1]), xu[j], acc[rt]);
      // one block at a time: keeps the unpacked operands of later blocks from
      // being hoisted past the register ring's budget
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  int s0 = 0;
  for (; s0 + DEPTH < ns; s0 += DEPTH) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      compute(ring[d]);
      load(s0 + DEPTH + d, ring[d]);
    }
  }
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) compute(ring[d]);
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[rt][i] += xacc[i];
  if constexpr (KW > 1) {
    // the K slices of a row group, added in slice order by slice 0
    __shared__ f32x4 red[NW][RT][kWave];
    if (kq != 0) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) red[wid][rt][lane] = acc[rt];
    }
    __syncthreads();
    if (kq != 0) return;
#pragma unroll
    for (int q = 1; q < KW; ++q)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const f32x4 v = red[wid + q][rt][lane];
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[rt][i] += v[i];
      }
  }
  if (!active || lr >= a.M) return;

  // lane (lr, lg) holds rows 4 lg .. 4 lg + 3 of each tile, column (x row) lr;
  // the per-channel scale of those rows
  float y[RT][4];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    uint32_t sd[2];
    load_dwords(a.scale + (t0 + rt) * 16 + 4 * lg, sd);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      y[rt][i] = (float)__builtin_bit_cast(h16x2, sd[i / 2])[i & 1] * acc[rt][i];
  }
  if constexpr (NORM) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int i = 0; i < 4; ++i) y[rt][i] = y[rt][i] * inv;
  }
  if constexpr (SWIGLU) {
    // tiles 2p (gate) and 2p + 1 (up) hold the 16 outputs of block t0 / 2 + p
    const int NA = a.N / 2;
#pragma unroll
    for (int p = 0; p < RT / 2; ++p) {
      const int n = (t0 / 2 + p) * 16 + 4 * lg;
      uint32_t v[2];
      v[0] = pack_bf16x2(swiglu_bf16(y[2 * p][0], y[2 * p + 1][0]),
                         swiglu_bf16(y[2 * p][1], y[2 * p + 1][1]));
      v[1] = pack_bf16x2(swiglu_bf16(y[2 * p][2], y[2 * p + 1][2]),
                         swiglu_bf16(y[2 * p][3], y[2 * p + 1][3]));
      __builtin_memcpy(a.out + (size_t)lr * NA + n, v, sizeof(v));
    }
  } else if constexpr (MODE == 2) {
    // the new residual, and per tile the sum of its squares over the 16 rows
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int n = (t0 + rt) * 16 + 4 * lg;
      float sq = resid_store4(a.ro, (size_t)lr * a.N + n, n, y[rt]);
      sq = sq + __shfl_xor(sq, 16);
      sq = sq + __shfl_xor(sq, 32);
      if (lg == 0) a.ro.ss[(size_t)lr * (a.N / 16) + t0 + rt] = sq;
    }
  } else if (a.out) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int n = (t0 + rt) * 16 + 4 * lg;
      uint32_t v[2] = {pack_bf16x2(y[rt][0], y[rt][1]), pack_bf16x2(y[rt][2], y[rt][3])};
      __builtin_memcpy(a.out + (size_t)lr * a.N + n, v, sizeof(v));
    }
  } else {
    float* dst = a.part + ((size_t)blockIdx.y * a.M + lr) * a.N;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
      *(f32x4*)(dst + (t0 + rt) * 16 + 4 * lg) = f32x4{y[rt][0], y[rt][1], y[rt][2], y[rt][3]};
  }
}

// registers of one stage (dwords per lane): weights and x operands (HX: half)
constexpr int stage_dwords(int rt, int upw, bool hx = false) {
  return 4 * rt * upw + 8 * (hx ? upw / 2 : upw);
}
constexpr int kRingDwords = 192;   // the ring's budget (depth x stage)

template <int RT, int UPW, int DEPTH, int RG, int KW, bool HX>
int launch_x(const DirectPlan& p, const W8dArgs& a, hipStream_t st) {
  const dim3 grid((unsigned)p.groups, (unsigned)p.ksplit), block(RG * KW * kWave);
  if constexpr (RT >= 2) {
    if (p.swiglu) {
      if (p.mode == 1)
        w8b_direct_kernel<RT, UPW, DEPTH, RG, KW, true, 1, HX><<<grid, block, 0, st>>>(a);
      else
        w8b_direct_kernel<RT, UPW, DEPTH, RG, KW, true, 0, HX><<<grid, block, 0, st>>>(a);
      return ACORN_OK;
    }
  }
  if (p.swiglu) return ACORN_ERR_UNSUPPORTED;
  switch (p.mode) {
    case 0: w8b_direct_kernel<RT, UPW, DEPTH, RG, KW, false, 0, HX><<<grid, block, 0, st>>>(a); break;
    case 1: w8b_direct_kernel<RT, UPW, DEPTH, RG, KW, false, 1, HX><<<grid, block, 0, st>>>(a); break;
    case 2: w8b_direct_kernel<RT, UPW, DEPTH, RG, KW, false, 2, HX><<<grid, block, 0, st>>>(a); break;
    default: return ACORN_ERR_UNSUPPORTED;
  }
  return ACORN_OK;
}

// the paired-x form where the plan asks for it, each form only within the
// ring's budget
template <int RT, int UPW, int DEPTH, int RG, int KW>
int launch(const DirectPlan& p, const W8dArgs& a, hipStream_t st) {
  if constexpr (UPW % 2 == 0 && DEPTH * stage_dwords(RT, UPW, true) <= kRingDwords) {
    if (p.hx) return launch_x<RT, UPW, DEPTH, RG, KW, true>(p, a, st);
  }
  if constexpr (DEPTH * stage_dwords(RT, UPW) <= kRingDwords) {
    if (!p.hx) return launch_x<RT, UPW, DEPTH, RG, KW, false>(p, a, st);
  }
  return ACORN_ERR_UNSUPPORTED;
}

template <int RT, int UPW, int DEPTH>
int by_layout(const DirectPlan& p, const W8dArgs& a, hipStream_t st) {
  switch (p.nw_field) {
    case 1: return launch<RT, UPW, DEPTH, 1, 1>(p, a, st);
    case 4: return launch<RT, UPW, DEPTH, 4, 1>(p, a, st);
    case 22: return launch<RT, UPW, DEPTH, 1, 2>(p, a, st);
    case 44: return launch<RT, UPW, DEPTH, 1, 4>(p, a, st);
  }
  return ACORN_ERR_UNSUPPORTED;
}

template <int RT, int UPW>
int by_depth(const DirectPlan& p, const W8dArgs& a, hipStream_t st) {
  constexpr bool kPair = UPW % 2 == 0;
  switch (p.depth) {
    case 1: return by_layout<RT, UPW, 1>(p, a, st);
    case 2: return by_layout<RT, UPW, 2>(p, a, st);
    case 4:
      if constexpr (4 * stage_dwords(RT, UPW, kPair) <= kRingDwords)
        return by_layout<RT, UPW, 4>(p, a, st);
      break;
    case 8:
      if constexpr (8 * stage_dwords(RT, UPW, kPair) <= kRingDwords)
        return by_layout<RT, UPW, 8>(p, a, st);
      break;
  }
  return ACORN_ERR_UNSUPPORTED;
}

template <int RT>
int by_upw(const DirectPlan& p, const W8dArgs& a, hipStream_t st) {
  switch (p.upw) {
    case 1: return by_depth<RT, 1>(p, a, st);
    case 2: return by_depth<RT, 2>(p, a, st);
  }
  return ACORN_ERR_UNSUPPORTED;
}

int divisor_at_least(int64_t n, int64_t v) {
  while (v <= n && n % v) ++v;
  return v <= n ? (int)v : 0;
}


// ---------------------------------------------------------------------------
// int8 GEMM for batches of 17..256 rows (decode buckets 32 / 64, configuration
// 3's M = 64 / 256), on the same W8B blocks, built as the int4 mid-M kernel
// (w4_decode.hip): a workgroup of NW waves owns NW * RT 16-row tiles x 64
// columns of x over a K range, and x moves through LDS 128 k (two blocks) at
// a time:
//  * every thread loads its share of the step's x (2 or 4 pieces of 16 bytes)
//    and each wave its RT x 2 weight blocks, DEPTH steps ahead in a register
//    ring (a step's loads are issued together, in step order);
//  * per step: one barrier, then four waves form the step's column sums of x
//    (MFMAs against ones) for the -128 X correction, each wave unpacks each
//    weight block once (q + 128 -> bf16, exact) and runs RT x 2 x 2 x 4 MFMAs
//    (every unpacked operand feeds the four column blocks, every x operand
//    the RT tiles), and the next step's x pieces go to the other LDS buffer;
//    the column sums are added to the running ones a step later, after the
//    next barrier;
//  * y = s[n] (C - 128 X) at the end, C the MFMA sum over the biased weights
//    and X each column's sum of x over the K range, added up per step in
//    fp32; split-K partials as everywhere else: fp32 [ksplit, M, N] of the
//    scaled values, summed in split order by the consumer.
struct W8mArgs {
  const __bf16* x;
  const uint8_t* w;
  const _Float16* scale;
  __bf16* out;    // bf16 [M, N] when ksplit == 1
  float* part;    // fp32 [ksplit, M, N] otherwise
  int M, N, K;
  int kr;         // K range of a split (a multiple of 128 * DEPTH)
};

constexpr int kW8MidBM = 64;                    // columns (x rows) per workgroup
constexpr int kW8MidMB = kW8MidBM / 16;
constexpr int kW8MidXP = kW8MidBM + 1;          // LDS pitch of one k piece (16-byte slots)

template <int RT, int NW, int DEPTH>
__global__ __launch_bounds__(NW * kWave, 1) void w8b_mid_kernel(W8mArgs a) {
  constexpr int NT = NW * kWave;
  constexpr int XPT = kW8MidBM * 16 / NT;        // x pieces per thread per step
  static_assert(XPT >= 1 && kW8MidBM * 16 % NT == 0, "whole x pieces per thread");
  extern __shared__ __align__(16) unsigned char smem[];
  u32x4* xs = (u32x4*)smem;                      // [2][16 pieces][kW8MidXP rows]
  float* xsum = (float*)(smem + 2 * 16 * kW8MidXP * 16);   // [2][64]
  const int wid = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int lg = lane >> 4, lr = lane & 15;
  int tile, split, mblk;
  {
    // the M blocks of one (row block, split) on one XCD (workgroups are dealt
    // to the 8 XCDs round robin), so their weight re-reads come from its L2
    const int ntl = gridDim.x, nks = gridDim.y, nmb = gridDim.z;
    const int lin = blockIdx.x + ntl * (blockIdx.y + nks * blockIdx.z);
    const int units = ntl * nks;
    int unit;
    if (nmb > 1 && units % 8 == 0) {
      const int xcd = lin % 8, j = lin / 8;
      unit = xcd * (units / 8) + j / nmb;
      mblk = j % nmb;
    } else {
      unit = lin % units;
      mblk = lin / units;
    }
    tile = unit % ntl;
    split = unit / ntl;
  }
  const int KB = a.K / 64;                       // blocks per row
  const int t0 = (tile * NW + wid) * RT;         // this wave's first 16-row tile
  const int sbase = split * (a.kr / 128);        // first 128-k step of the split
  const int nch = a.kr / 128;
  const int m0 = mblk * kW8MidBM;

  struct Slot {
    u32x4 x[XPT];
    u32x4 w[RT][2];
  };
  // piece p of a step: x row p / 16, k piece p % 16 (8 k), so that a wave's
  // load covers 4 rows x 256 contiguous bytes (rows past M re-read row M - 1;
  // their columns are never stored); it goes to LDS slot piece * kW8MidXP +
  // row, whose pad keeps the stores and the operand reads free of bank
  // conflicts
  auto load = [&](int c, Slot& sl) {
    const int st = sbase + min(c, nch - 1);
#pragma unroll
    for (int u = 0; u < XPT; ++u) {
      const int p = (int)threadIdx.x + NT * u;
      const int m = min(m0 + p / 16, a.M - 1);
      sl.x[u] = *(const u32x4*)(a.x + (size_t)m * a.K + st * 128 + (p % 16) * 8);
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int u = 0; u < 2; ++u)
        sl.w[rt][u] = load_nt((const u32x4*)(a.w + ((size_t)(t0 + rt) * KB + 2 * st + u) * 1024 +
                                             lane * 16));
  };

  f32x4 acc[RT][kW8MidMB];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int mb = 0; mb < kW8MidMB; ++mb) acc[rt][mb] = f32x4{0.f, 0.f, 0.f, 0.f};
  float xt[kW8MidMB];                            // column lr's sum of x so far, per block
#pragma unroll
  for (int mb = 0; mb < kW8MidMB; ++mb) xt[mb] = 0.f;
  const u32x4 ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};

  auto store_x = [&](int c, const Slot& sl) {
    u32x4* xb = xs + (c & 1) * 16 * kW8MidXP;
#pragma unroll
    for (int u = 0; u < XPT; ++u) {
      const int p = (int)threadIdx.x + NT * u;
      xb[(p % 16) * kW8MidXP + p / 16] = sl.x[u];
    }
  };
  // One barrier per step: x of step c was stored at the end of step c - 1
  // (into the other buffer than the one step c - 1 read), and the column sums
  // of step c are formed during step c and added during step c + 1.
  auto step = [&](int c, const Slot& sl, const Slot& next) {
    const int b = c & 1;
    const u32x4* xb = xs + b * 16 * kW8MidXP;
    __syncthreads();
    if (c > 0) {
#pragma unroll
      for (int mb = 0; mb < kW8MidMB; ++mb) xt[mb] += xsum[(b ^ 1) * kW8MidBM + mb * 16 + lr];
    }
    if (wid < kW8MidMB) {
      f32x4 xg = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j) xg = mfma(ones, xb[(4 * lg + j) * kW8MidXP + wid * 16 + lr], xg);
      if (lg == 0) xsum[b * kW8MidBM + wid * 16 + lr] = xg[0];
    }
    // block u, MFMA j: the lane's k slots stand for k 64 u + 16 lg + 8 j ..,
    // i.e. x piece 8 u + 2 lg + j of the step
    u32x4 aw[RT][2][2];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          aw[rt][u][j] = unpack_w8(sl.w[rt][u][2 * j], sl.w[rt][u][2 * j + 1]);
#pragma unroll
    for (int mb = 0; mb < kW8MidMB; ++mb) {
      u32x4 bx[2][2];
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          bx[u][j] = xb[(8 * u + 2 * lg + j) * kW8MidXP + mb * 16 + lr];
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int j = 0; j < 2; ++j) acc[rt][mb] = mfma(aw[rt][u][j], bx[u][j], acc[rt][mb]);
    }
    if (c + 1 < nch) store_x(c + 1, next);
  };

  Slot ring[DEPTH];
  // in slot order, as the loop reissues them (the loop's static waits assume it)
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) {
    load(d, ring[d]);
    __builtin_amdgcn_sched_barrier(0);
  }
  store_x(0, ring[0]);
  for (int c0 = 0; c0 < nch; c0 += DEPTH) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      step(c0 + d, ring[d], ring[(d + 1) % DEPTH]);
      load(c0 + d + DEPTH, ring[d]);   // past the end: re-reads the last step
    }
  }
  __syncthreads();                     // the last step's column sums
#pragma unroll
  for (int mb = 0; mb < kW8MidMB; ++mb) xt[mb] += xsum[((nch - 1) & 1) * kW8MidBM + mb * 16 + lr];

  // lane (lr, lg) holds rows 4 lg .. 4 lg + 3 of tile t0 + rt, column 16 mb + lr
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    uint32_t sd[2];
    load_dwords(a.scale + (t0 + rt) * 16 + 4 * lg, sd);
#pragma unroll
    for (int mb = 0; mb < kW8MidMB; ++mb) {
      const int m = m0 + mb * 16 + lr;
      if (m >= a.M) break;
      const int n = (t0 + rt) * 16 + 4 * lg;
      float y[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        y[i] = (float)__builtin_bit_cast(h16x2, sd[i / 2])[i & 1] *
               __builtin_fmaf(xt[mb], -128.f, acc[rt][mb][i]);
      if (a.out) {
        uint32_t v[2] = {pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])};
        __builtin_memcpy(a.out + (size_t)m * a.N + n, v, sizeof(v));
      } else {
        *(f32x4*)(a.part + ((size_t)split * a.M + m) * a.N + n) = f32x4{y[0], y[1], y[2], y[3]};
      }
    }
  }
}

template <int RT, int NW, int DEPTH>
int launch_mid(const W8mPlan& p, const W8mArgs& a, hipStream_t st) {
  w8b_mid_kernel<RT, NW, DEPTH><<<dim3((unsigned)p.groups, (unsigned)p.ksplit,
                                       (unsigned)p.mblocks),
                                  dim3(NW * kWave), p.lds, st>>>(a);
  return ACORN_OK;
}

}  // namespace

namespace acorn {

// rt 1/2/4 (swiglu 2/4; N/16 divisible by rt), upw 1/2 blocks of 64 k per
// stage, the wave layout in the nw field (1 or 4 waves on their own rows; 22,
// 44 = 2 or 4 waves splitting K over one row group), depth 1/2/4 within the
// ring's register budget, and split counts that give every wave a whole
// number of depth rounds. With 0 the plan takes rt 2, upw 2, one wave per
// workgroup, depth 4 (16 KB of weights in flight per wave), and the fewest
// splits that launch at least three waves per CU.
int w8b_make_plan(int64_t M, int64_t N, int64_t K, const int* cfg, bool swiglu, DirectPlan* p) {
  if (M < 1 || M > 16) return ACORN_ERR_UNSUPPORTED;
  if (N % 16 || K % 64) return ACORN_ERR_SHAPE;
  if (swiglu && N % 32) return ACORN_ERR_SHAPE;
  const int64_t ntiles = N / 16, KB = K / 64;
  int rt = cfg && cfg[0] > 0 ? cfg[0] : 2;
  const int upw = cfg && cfg[1] > 0 ? cfg[1] : 2;
  const int nwf = cfg && cfg[2] > 0 ? cfg[2] : 1;
  const int req_ks = cfg ? cfg[3] : 0;
  int depth = cfg && cfg[4] > 0 ? cfg[4] : 4;
  if (rt != 1 && rt != 2 && rt != 4) return ACORN_ERR_UNSUPPORTED;
  if (swiglu && rt < 2) rt = 2;
  while (rt > (swiglu ? 2 : 1) && ntiles % rt) rt /= 2;
  if (ntiles % rt) return ACORN_ERR_UNSUPPORTED;
  if (upw != 1 && upw != 2) return ACORN_ERR_UNSUPPORTED;
  if (nwf != 1 && nwf != 4 && nwf != 22 && nwf != 44) return ACORN_ERR_UNSUPPORTED;
  const int nw = nwf < 10 ? nwf : nwf / 10, kw = nwf < 10 ? 1 : nwf % 10;
  if (depth != 1 && depth != 2 && depth != 4 && depth != 8) return ACORN_ERR_UNSUPPORTED;
  // M <= 8 with two blocks per stage: the paired-x form (half the x registers)
  const bool hx = M <= 8 && upw == 2;
  while (depth > 1 && (depth * stage_dwords(rt, upw, hx) > kRingDwords || KB % (kw * upw * depth)))
    depth /= 2;
  if (KB % (kw * upw * depth)) return ACORN_ERR_SHAPE;
  const int64_t q = KB / (kw * upw * depth);    // ks must divide this
  const int64_t waves = ntiles / rt * kw;
  int ks;
  if (swiglu) {
    ks = 1;
  } else if (req_ks > 0) {
    ks = divisor_at_least(q, req_ks);
    if (!ks) return ACORN_ERR_UNSUPPORTED;
  } else {
    ks = 1;
    while (waves * ks < 3 * 256) {
      const int nx = divisor_at_least(q, ks + 1);
      if (!nx) break;
      ks = nx;
    }
  }
  const int64_t rgs = nw / kw;
  const int64_t groups = (ntiles / rt + rgs - 1) / rgs;
  if (groups > 0x7fffffff || ks > 65535) return ACORN_ERR_SHAPE;
  p->rt = rt;
  p->upw = upw;
  p->nw_field = nwf;
  p->rg = (int)rgs;
  p->kw = kw;
  p->ksplit = ks;
  p->depth = depth;
  p->groups = (int)groups;
  p->swiglu = swiglu;
  p->mode = 0;
  p->hx = hx;
  return ACORN_OK;
}

int w8b_launch(const DirectPlan& p, const void* x, const void* w, const void* scale, void* out,
               float* part, int64_t M, int64_t N, int64_t K, const NormIn* ni,
               const ResidOut* ro, hipStream_t st) {
  if (!x || !w || !scale) return ACORN_ERR_VALUE;
  if (M < 1 || M > 16) return ACORN_ERR_UNSUPPORTED;
  if (p.ksplit > 1) out = nullptr;
  if (p.mode == 2) {
    if (!ro || !ro->res || !ro->res_out || !ro->ss || !ro->nw || !ro->xw) return ACORN_ERR_VALUE;
    if (p.ksplit != 1 || p.swiglu) return ACORN_ERR_UNSUPPORTED;
  } else if (!out && (!part || p.swiglu)) {
    return ACORN_ERR_VALUE;
  }
  if (p.mode == 1 && (!ni || !ni->ss || ni->nss * 16 != K)) return ACORN_ERR_VALUE;
  W8dArgs a{(const __bf16*)x, (const uint8_t*)w, (const _Float16*)scale, (__bf16*)out,
            part, (int)M, (int)N, (int)K, (int)(K / p.ksplit), NormIn{}, ResidOut{}};
  if (ni) a.ni = *ni;
  if (ro) a.ro = *ro;
  int rc = ACORN_ERR_UNSUPPORTED;
  switch (p.rt) {
    case 1: rc = by_upw<1>(p, a, st); break;
    case 2: rc = by_upw<2>(p, a, st); break;
    case 4: rc = by_upw<4>(p, a, st); break;
  }
  if (rc) return rc;
  ACORN_LAUNCH_CHECK();
  return ACORN_OK;
}

// Knobs as the int4 mid-M kernel's: rt (16-row tiles per wave) 1 or 2, nw
// (waves) 4 or 8, ksplit, depth (128-k steps in flight) 2 or 4; N a whole
// number of NW * RT * 16 row blocks, K of 128-k steps, and each split's step
// count of depth rounds. With ksplit 0 the split grows from 1 while the launch
// has fewer workgroups than 256 and each split keeps 4 depth rounds.
int w8m_make_plan(int64_t M, int64_t N, int64_t K, const int* cfg, W8mPlan* p) {
  if (M < 1 || M > 65535 * (int64_t)kW8MidBM) return ACORN_ERR_SHAPE;
  if (K % 128) return ACORN_ERR_SHAPE;
  const int rt = cfg && cfg[1] > 0 ? cfg[1] : 2;
  const int nw = cfg && cfg[2] > 0 ? cfg[2] : 8;
  const int req_ks = cfg ? cfg[3] : 0;
  const int depth = cfg && cfg[4] > 0 ? cfg[4] : 2;
  if ((rt != 1 && rt != 2) || (nw != 4 && nw != 8) || (depth != 2 && depth != 4))
    return ACORN_ERR_UNSUPPORTED;
  const int64_t rows = (int64_t)nw * rt * 16;
  if (N % rows) return ACORN_ERR_UNSUPPORTED;
  const int64_t G = K / 128, groups = N / rows, mblocks = (M + kW8MidBM - 1) / kW8MidBM;
  auto fits = [&](int64_t ks) { return ks >= 1 && G % ks == 0 && (G / ks) % depth == 0; };
  int64_t ks;
  if (req_ks > 0) {
    ks = req_ks;
    while (ks <= G && !fits(ks)) ++ks;
    if (ks > G) return ACORN_ERR_UNSUPPORTED;
  } else {
    ks = 1;
    if (!fits(1)) return ACORN_ERR_UNSUPPORTED;
    while (groups * mblocks * ks < 256) {
      int64_t nx = ks + 1;
      while (nx <= G && !fits(nx)) ++nx;
      if (nx > G || G / nx < 4 * depth) break;
      ks = nx;
    }
  }
  if (groups > 0x7fffffff || ks > 65535 || mblocks > 65535) return ACORN_ERR_SHAPE;
  p->rt = rt;
  p->nw = nw;
  p->ksplit = (int)ks;
  p->depth = depth;
  p->groups = (int)groups;
  p->mblocks = (int)mblocks;
  p->lds = (size_t)2 * 16 * kW8MidXP * 16 + (size_t)2 * kW8MidBM * 4;
  return ACORN_OK;
}

int w8m_launch(const W8mPlan& p, const void* x, const void* w, const void* scale, void* out,
               float* part, int64_t M, int64_t N, int64_t K, hipStream_t st) {
  if (!x || !w || !scale) return ACORN_ERR_VALUE;
  if (p.ksplit > 1) out = nullptr;
  if (!out && !part) return ACORN_ERR_VALUE;
  const W8mArgs a{(const __bf16*)x, (const uint8_t*)w, (const _Float16*)scale, (__bf16*)out,
                  part, (int)M, (int)N, (int)K, (int)(K / p.ksplit)};
  int rc = ACORN_ERR_UNSUPPORTED;
  switch (p.rt * 100 + p.nw * 10 + p.depth) {
    case 142: rc = launch_mid<1, 4, 2>(p, a, st); break;
    case 144: rc = launch_mid<1, 4, 4>(p, a, st); break;
    case 182: rc = launch_mid<1, 8, 2>(p, a, st); break;
    case 184: rc = launch_mid<1, 8, 4>(p, a, st); break;
    case 242: rc = launch_mid<2, 4, 2>(p, a, st); break;
    case 244: rc = launch_mid<2, 4, 4>(p, a, st); break;
    case 282: rc = launch_mid<2, 8, 2>(p, a, st); break;
    case 284: rc = launch_mid<2, 8, 4>(p, a, st); break;
  }
  if (rc) return rc;
  ACORN_LAUNCH_CHECK();
  return ACORN_OK;
}

}  // namespace acorn
