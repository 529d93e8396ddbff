// bf16 GEMM at decode sizes (M <= 16) over the BF16B block layout.
//
// y[M,N] = x[M,K] @ W[N,K]^T, bf16 x and W, fp32 accumulation: the bf16
// projections of a decode step (the reference's decode GEMM,
// acorninfer/ops/decode_gemm.py:236-257, and its lm_head) at M = batch rows.
//
// Built like the int8 and int4 direct kernels (w8_decode.hip, w4_decode.hip),
// with nothing to unpack:
//  * The weights of 16 rows x 32 k are one contiguous 1 KB block
//    (ACORN_WFMT_BF16B): lane lg * 16 + r holds row r's 8 consecutive k
//    8 lg .. 8 lg + 7, exactly the A operand of one v_mfma_f32_16x16x32_bf16,
//    so a wave reads a block with one 16-byte load per lane (whole cache
//    lines, non-temporal policy) and feeds it to the MFMA as loaded. Read in
//    the natural [N, K] layout the same operand is 16 rows x 64 bytes, half
//    lines; that streamed 15-25% slower on the 8B shapes.
//  * Every wave reads its x operands from memory straight into MFMA B
//    registers with its weights (no LDS staging, no barrier before the first
//    MFMA); a B operand serves the RT row tiles of the wave.
//  * KW > 1 waves of a workgroup split K over the same rows and add their
//    results through LDS in fixed order at the end.
//  * Split-K (ksplit > 1) writes fp32 partials [ksplit, M, N], summed in split
//    order by the consumer (bitwise deterministic).
//  * MODE 1 (NormIn): x is the residual times the norm weight; each lane
//    computes its row's 1 / rms from the producer's per-16-column sums of
//    squares (requested before the weights) and multiplies its results by it
//    before the epilogue. MODE 2 (ResidOut, one split, no SwiGLU): instead of
//    y the epilogue stores the new residual bf16(res + bf16(y)), its rows
//    times the next norm's weight, and each 16-row tile's sum of squares per
//    x row (the RMSNorm folded into the GEMMs, gemm_common.h).
#include "gemm_common.h"

using namespace acorn;

namespace {

struct BfdArgs {
  const __bf16* x;
  const uint8_t* w;
  __bf16* out;    // bf16 [M, N] (act [M, N/2] with SWIGLU) when ksplit == 1
  float* part;    // fp32 [ksplit, M, N] otherwise
  int M, N, K;
  int kr;         // K range of a split (a multiple of 32 * KW * UPW * DEPTH)
  NormIn ni;      // MODE 1
  ResidOut ro;    // MODE 2
};

template <int RT, int UPW, bool HX>
struct BfdStage {
  u32x4 w[RT][UPW];          // block (tile rt, block u): this lane's 16 bytes
  // B operand of block u: x row lr, k 8 lg .. 8 lg + 7 (HX: of block pair
  // u / 2, lanes lr < 8 the even block's rows, lr >= 8 the odd one's)
  u32x4 x[HX ? UPW / 2 : UPW];
};

// Grid: x = tile groups of RG * RT 16-row tiles, y = ksplit; block RG * KW
// waves. Row group r of workgroup b owns tiles (b RG + r) RT .. + RT - 1; its
// KW waves split the split's K range. Lane (lr, lg) holds x row min(lr, M - 1)
// (rows past M feed only columns that are never stored).
// HX (M <= 8, UPW even): the paired-x form (gemm_common.h, rot8).
template <int RT, int UPW, int DEPTH, int RG, int KW, bool SWIGLU, int MODE, bool HX = false>
__global__ __launch_bounds__(RG * KW * kWave) void bf16b_direct_kernel(BfdArgs a) {
  static_assert(!HX || UPW % 2 == 0, "x in block pairs");
  constexpr int NW = RG * KW;
  constexpr bool NORM = MODE == 1;
  static_assert(MODE != 2 || !SWIGLU, "the residual epilogue replaces a plain output");
  const int wid = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int lg = lane >> 4, lr = lane & 15;
  const int rg = wid / KW, kq = wid % KW;
  const int KB = a.K / 32;                        // blocks per row tile
  const int t0 = (blockIdx.x * RG + rg) * RT;
  const bool active = t0 < a.N / 16;              // (N / 16) % RT == 0 by the plan
  const int tt = active ? t0 : 0;                 // idle waves read tile 0, store nothing
  const int BW = a.kr / (32 * KW);                // blocks of this wave
  const int kw0 = blockIdx.y * a.kr + kq * BW * 32;
  const int ns = BW / UPW;                        // stages, a multiple of DEPTH
  const uint8_t* wb = a.w + ((size_t)tt * KB + kw0 / 32) * 1024 + lane * 16;
  const __bf16* xb = HX ? a.x + (size_t)min(lr & 7, a.M - 1) * a.K + kw0 + 8 * lg + 32 * (lr >> 3)
                        : a.x + (size_t)min(lr, a.M - 1) * a.K + kw0 + 8 * lg;
  auto load = [&](int s, BfdStage<RT, UPW, HX>& r) {
#pragma unroll
    for (int u = 0; u < (HX ? UPW / 2 : UPW); ++u)
      r.x[u] = *(const u32x4*)(xb + (s * UPW + (HX ? 2 * u : u)) * 32);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int u = 0; u < UPW; ++u)
        r.w[rt][u] = load_nt((const u32x4*)(wb + ((size_t)rt * KB + s * UPW + u) * 1024));
  };

  // MODE 1: this row's 1 / rms, its sums requested ahead of the weights
  NormRegs nr;
  if constexpr (NORM) norm_issue(a.ni, a.M, lane, nr);
  BfdStage<RT, UPW, HX> ring[DEPTH];
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
  auto compute = [&](const BfdStage<RT, UPW, HX>& r) {
#pragma unroll
    for (int u = 0; u < UPW; ++u) {
      const u32x4 xu = HX && (u & 1) ? rot8(r.x[u / 2]) : r.x[HX ? u / 2 : u];
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) acc[rt] = mfma(r.w[rt][u], xu, acc[rt]);
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

  // lane (lr, lg) holds rows 4 lg .. 4 lg + 3 of each tile, column (x row) lr
  if constexpr (NORM) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[rt][i] = acc[rt][i] * inv;
  }
  if constexpr (SWIGLU) {
    // tiles 2p (gate) and 2p + 1 (up) hold the 16 outputs of block t0 / 2 + p
    const int NA = a.N / 2;
#pragma unroll
    for (int p = 0; p < RT / 2; ++p) {
      const int n = (t0 / 2 + p) * 16 + 4 * lg;
      uint32_t v[2];
      v[0] = pack_bf16x2(swiglu_bf16(acc[2 * p][0], acc[2 * p + 1][0]),
                         swiglu_bf16(acc[2 * p][1], acc[2 * p + 1][1]));
      v[1] = pack_bf16x2(swiglu_bf16(acc[2 * p][2], acc[2 * p + 1][2]),
                         swiglu_bf16(acc[2 * p][3], acc[2 * p + 1][3]));
      __builtin_memcpy(a.out + (size_t)lr * NA + n, v, sizeof(v));
    }
  } else if constexpr (MODE == 2) {
    // the new residual, and per tile the sum of its squares over the 16 rows
    // (lane groups 0..3 hold rows 4 lg .. 4 lg + 3: added pairwise, in order)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int n = (t0 + rt) * 16 + 4 * lg;
      const float y[4] = {acc[rt][0], acc[rt][1], acc[rt][2], acc[rt][3]};
      float sq = resid_store4(a.ro, (size_t)lr * a.N + n, n, y);
      sq = sq + __shfl_xor(sq, 16);
      sq = sq + __shfl_xor(sq, 32);
      if (lg == 0) a.ro.ss[(size_t)lr * (a.N / 16) + t0 + rt] = sq;
    }
  } else if (a.out) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int n = (t0 + rt) * 16 + 4 * lg;
      uint32_t v[2] = {pack_bf16x2(acc[rt][0], acc[rt][1]), pack_bf16x2(acc[rt][2], acc[rt][3])};
      __builtin_memcpy(a.out + (size_t)lr * a.N + n, v, sizeof(v));
    }
  } else {
    float* dst = a.part + ((size_t)blockIdx.y * a.M + lr) * a.N;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) *(f32x4*)(dst + (t0 + rt) * 16 + 4 * lg) = acc[rt];
  }
}

// registers of one stage (dwords per lane): weights and x operands (HX: half)
constexpr int stage_dwords(int rt, int upw, bool hx = false) {
  return 4 * rt * upw + 4 * (hx ? upw / 2 : upw);
}
constexpr int kRingDwords = 192;   // the ring's budget (depth x stage)

template <int RT, int UPW, int DEPTH, int RG, int KW, bool HX>
int launch_x(const DirectPlan& p, const BfdArgs& a, hipStream_t st) {
  const dim3 grid((unsigned)p.groups, (unsigned)p.ksplit), block(RG * KW * kWave);
  if constexpr (RT >= 2) {
    if (p.swiglu) {
      if (p.mode == 1)
        bf16b_direct_kernel<RT, UPW, DEPTH, RG, KW, true, 1, HX><<<grid, block, 0, st>>>(a);
      else
        bf16b_direct_kernel<RT, UPW, DEPTH, RG, KW, true, 0, HX><<<grid, block, 0, st>>>(a);
      return ACORN_OK;
    }
  }
  if (p.swiglu) return ACORN_ERR_UNSUPPORTED;
  switch (p.mode) {
    case 0: bf16b_direct_kernel<RT, UPW, DEPTH, RG, KW, false, 0, HX><<<grid, block, 0, st>>>(a); break;
    case 1: bf16b_direct_kernel<RT, UPW, DEPTH, RG, KW, false, 1, HX><<<grid, block, 0, st>>>(a); break;
    case 2: bf16b_direct_kernel<RT, UPW, DEPTH, RG, KW, false, 2, HX><<<grid, block, 0, st>>>(a); break;
    default: return ACORN_ERR_UNSUPPORTED;
  }
  return ACORN_OK;
}

// the paired-x form where the plan asks for it, each form only within the
// ring's budget
template <int RT, int UPW, int DEPTH, int RG, int KW>
int launch(const DirectPlan& p, const BfdArgs& a, hipStream_t st) {
  if constexpr (UPW % 2 == 0 && DEPTH * stage_dwords(RT, UPW, true) <= kRingDwords) {
    if (p.hx) return launch_x<RT, UPW, DEPTH, RG, KW, true>(p, a, st);
  }
  if constexpr (DEPTH * stage_dwords(RT, UPW) <= kRingDwords) {
    if (!p.hx) return launch_x<RT, UPW, DEPTH, RG, KW, false>(p, a, st);
  }
  return ACORN_ERR_UNSUPPORTED;
}

template <int RT, int UPW, int DEPTH>
int by_layout(const DirectPlan& p, const BfdArgs& a, hipStream_t st) {
  switch (p.nw_field) {
    case 1: return launch<RT, UPW, DEPTH, 1, 1>(p, a, st);
    case 4: return launch<RT, UPW, DEPTH, 4, 1>(p, a, st);
    case 22: return launch<RT, UPW, DEPTH, 1, 2>(p, a, st);
    case 44: return launch<RT, UPW, DEPTH, 1, 4>(p, a, st);
  }
  return ACORN_ERR_UNSUPPORTED;
}


template <int RT, int UPW>
int by_depth(const DirectPlan& p, const BfdArgs& a, hipStream_t st) {
  switch (p.depth) {
    case 2: return by_layout<RT, UPW, 2>(p, a, st);
    case 4:
      if constexpr (4 * stage_dwords(RT, UPW, UPW % 2 == 0) <= kRingDwords)
        return by_layout<RT, UPW, 4>(p, a, st);
      break;
    case 8:
      if constexpr (8 * stage_dwords(RT, UPW, UPW % 2 == 0) <= kRingDwords)
        return by_layout<RT, UPW, 8>(p, a, st);
      break;
  }
  return ACORN_ERR_UNSUPPORTED;
}

template <int RT>
int by_upw(const DirectPlan& p, const BfdArgs& a, hipStream_t st) {
  switch (p.upw) {
    case 1: return by_depth<RT, 1>(p, a, st);
    case 2: return by_depth<RT, 2>(p, a, st);
    case 4: return by_depth<RT, 4>(p, a, st);
  }
  return ACORN_ERR_UNSUPPORTED;
}

int divisor_at_least(int64_t n, int64_t v) {
  while (v <= n && n % v) ++v;
  return v <= n ? (int)v : 0;
}

}  // namespace

namespace acorn {

// rt 1/2/4 (swiglu 2/4; N/16 divisible by rt), upw 1/2/4 blocks of 32 k per
// stage, the wave layout in the nw field (1 or 4 waves on their own rows; 22,
// 44 = 2 or 4 waves splitting K over one row group), depth 2/4/8 within the
// ring's register budget (then upw lowered where the rows are too short for
// it), and split counts that give every wave a whole number of depth rounds. With 0 the plan takes rt 1 (2 with swiglu), upw 2,
// one wave per workgroup, depth 4 (8 KB of weights in flight per wave), and
// the fewest splits that launch at least three waves per CU.
int bf16b_make_plan(int64_t M, int64_t N, int64_t K, const int* cfg, bool swiglu,
                    DirectPlan* p) {
  if (M < 1 || M > 16) return ACORN_ERR_UNSUPPORTED;
  if (N % 16 || K % 64) return ACORN_ERR_SHAPE;
  if (swiglu && N % 32) return ACORN_ERR_SHAPE;
  const int64_t ntiles = N / 16, KB = K / 32;
  int rt = cfg && cfg[0] > 0 ? cfg[0] : swiglu ? 2 : 1;
  int upw = cfg && cfg[1] > 0 ? cfg[1] : 2;
  const int nwf = cfg && cfg[2] > 0 ? cfg[2] : 1;
  const int req_ks = cfg ? cfg[3] : 0;
  int depth = cfg && cfg[4] > 0 ? cfg[4] : 4;
  if (rt != 1 && rt != 2 && rt != 4) return ACORN_ERR_UNSUPPORTED;
  if (swiglu && rt < 2) rt = 2;
  while (rt > (swiglu ? 2 : 1) && ntiles % rt) rt /= 2;
  if (ntiles % rt) return ACORN_ERR_UNSUPPORTED;
  if (upw != 1 && upw != 2 && upw != 4) return ACORN_ERR_UNSUPPORTED;
  if (nwf != 1 && nwf != 4 && nwf != 22 && nwf != 44) return ACORN_ERR_UNSUPPORTED;
  const int nw = nwf < 10 ? nwf : nwf / 10, kw = nwf < 10 ? 1 : nwf % 10;
  if (depth != 2 && depth != 4 && depth != 8) return ACORN_ERR_UNSUPPORTED;
  // M <= 8 with an even number of blocks per stage: the paired-x form
  const bool hx = M <= 8 && upw % 2 == 0;
  while (depth > 2 && (depth * stage_dwords(rt, upw, hx) > kRingDwords || KB % (kw * upw * depth)))
    depth /= 2;
  while (upw > 1 && KB % (kw * upw * depth)) upw /= 2;   // short rows (K of 64 or 128)
  if (depth * stage_dwords(rt, upw, hx && upw % 2 == 0) > kRingDwords) return ACORN_ERR_UNSUPPORTED;
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
  p->hx = hx && upw % 2 == 0;
  return ACORN_OK;
}

int bf16b_launch(const DirectPlan& p, const void* x, const void* w, void* out, float* part,
                 int64_t M, int64_t N, int64_t K, const NormIn* ni, const ResidOut* ro,
                 hipStream_t st) {
  if (!x || !w) return ACORN_ERR_VALUE;
  if (M < 1 || M > 16) return ACORN_ERR_UNSUPPORTED;
  if (p.ksplit > 1) out = nullptr;
  if (p.mode == 2) {
    // the residual epilogue: one split, no SwiGLU, complete 16-row tiles
    if (!ro || !ro->res || !ro->res_out || !ro->ss || !ro->nw || !ro->xw) return ACORN_ERR_VALUE;
    if (p.ksplit != 1 || p.swiglu) return ACORN_ERR_UNSUPPORTED;
  } else if (!out && (!part || p.swiglu)) {
    return ACORN_ERR_VALUE;
  }
  if (p.mode == 1 && (!ni || !ni->ss || ni->nss * 16 != K)) return ACORN_ERR_VALUE;
  BfdArgs a{(const __bf16*)x, (const uint8_t*)w, (__bf16*)out, part, (int)M, (int)N,
            (int)K, (int)(K / p.ksplit), NormIn{}, ResidOut{}};
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

}  // namespace acorn
