// Weight-only int4 GEMM at decode sizes (M <= 64) over the W4B block layout.
//
// y[M,N] = x[M,K] @ ((u - 8) * s)^T: u the stored nibble (symmetric int4
// v = u - 8, the reference's m7 spike format with zero = -8 s,
// scripts/m7_spike.py:152-231), s fp16 per (row, 128-k group), bf16 x,
// fp32 accumulation.
//
// Built for the gfx950 memory path:
//  * The weights of 16 rows x 128 k (one group) are one contiguous 1 KB block
//    in MFMA A-operand order (ACORN_WFMT_W4B). A wave reads a block with one
//    16-byte load per lane (whole cache lines, non-temporal policy) and feeds
//    four v_mfma_f32_16x16x32_bf16 from it; no data moves between lanes.
//  * int4 -> bf16 (128 + u): one v_and_or_b32 per bf16 pair, plus a shift for
//    three of the four pairs of a dword. The layout stores each dword's
//    nibbles in the order that pairing needs (k offsets 0,2,4,6 | 1,3,5,7), so
//    the unpacked operand is in natural k order and x is used as it is.
//  * Per group: y += s * (C - 136 X), C the group's MFMA sum over the biased
//    weights and X the sum of x over the group; the fp16 scale is read from
//    its packed pair by v_fma_mix_f32.
//  * Split-K (ksplit > 1) writes fp32 partials [ksplit, M, N], summed in split
//    order by the consumer (bitwise deterministic).
//
// Two kernels:
//  * M <= 16 (decode buckets up to 16): w4b_direct_kernel. Every wave is
//    independent: its x operands come from memory (L2) straight into MFMA B
//    registers with its weights, so no wave waits for a workgroup to stage x
//    or for a barrier before its first MFMA. X and the bias come from one more
//    MFMA chain per group (a constant -136 operand against x) that seeds the
//    tiles' accumulators.
//  * 16 < M <= 64 (decode buckets of 32 and 64, configuration 3's M = 64):
//    w4b_decode_kernel, MB = 2 or 4 16-column blocks of x per wave with x
//    staged in LDS by the workgroup (every unpacked weight operand feeds MB
//    MFMAs and every x operand RT, so the same loads carry MB times the
//    arithmetic).
#include "gemm_common.h"

using namespace acorn;

namespace {

// ---- M <= 16 ----------------------------------------------------------------
struct W4dArgs {
  const __bf16* x;
  const uint8_t* w;
  const _Float16* scale;
  __bf16* out;    // bf16 [M, N] (act [M, N/2] with SWIGLU) when ksplit == 1
  float* part;    // fp32 [ksplit, M, N] otherwise
  int M, N, K;
  int kr;         // K range of a split (a multiple of 128 * UPW * DEPTH)
  NormIn ni;      // MODE 1: results scaled by the rows' 1 / rms (gemm_common.h)
  ResidOut ro;    // MODE 2: the residual epilogue (gemm_common.h)
};

template <int RT, int UPW, bool HX>
struct DStage {
  u32x4 w[RT][UPW];          // unit (rt, u): this lane's 16 bytes of block (tile, group)
  // B operand of MFMA j of group u: x row lr, k 32 lg + 8 j .. (HX: of group
  // pair u / 2, lanes lr < 8 holding the even group and lr >= 8 the odd one)
  u32x4 x[HX ? UPW / 2 : UPW][4];
  uint32_t s[RT][2 * UPW];   // fp16 scales: half 4u + i is row 4 lg + i of group u
};

// bf16 -136 in every slot: an MFMA of it against x gives -136 X per column
constexpr uint32_t kNeg136x2 = 0xC308C308u;

// Grid: x = tile groups of RG * RT 16-row tiles, y = ksplit; block RG * KW
// waves. Row group r of workgroup b owns tiles (b RG + r) RT .. + RT - 1; its
// KW waves split the split's K range (KW > 1 gives a projection more waves
// without split-K partials: they add their results through LDS in fixed
// order at the end). Each wave keeps DEPTH stages of UPW groups in flight.
// Lane (lr, lg) holds x row min(lr, M - 1) (rows past M feed only columns
// that are never stored). HX (M <= 8, UPW even): a wave's x loads carry two
// groups at once, lanes lr < 8 the even group's rows and lr >= 8 the odd
// one's; the odd group's operand is the same registers rotated by 8 lanes
// (its columns 8..15 then hold the even group's x: never stored). Half the x
// loads and x registers, four DPP moves per operand.
template <int RT, int UPW, int DEPTH, int RG, int KW, bool SWIGLU, int MODE, bool HX = false>
__global__ __launch_bounds__(RG * KW * kWave) void w4b_direct_kernel(W4dArgs a) {
  constexpr int NW = RG * KW;
  constexpr bool NORM = MODE == 1;
  static_assert(MODE != 2 || !SWIGLU, "the residual epilogue replaces a plain output");
  static_assert(!HX || UPW % 2 == 0, "x in group pairs");
  const int wid = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int lg = lane >> 4, lr = lane & 15;
  const int rg = wid / KW, kq = wid % KW;
  const int G = a.K / 128, G4 = a.K / 512;
  const int t0 = (blockIdx.x * RG + rg) * RT;
  const bool active = t0 < a.N / 16;              // (N / 16) % RT == 0 by the plan
  const int tt = active ? t0 : 0;                 // idle waves read tile 0, store nothing
  const int GW = a.kr / (128 * KW);               // groups of this wave
  const int kw0 = blockIdx.y * a.kr + kq * GW * 128;
  const unsigned g0 = (unsigned)(kw0 / 128);
  const int ns = GW / UPW;                        // stages, a multiple of DEPTH
  const uint8_t* wb = a.w + ((size_t)tt * G + g0) * 1024 + lane * 16;
  const __bf16* xb = HX ? a.x + (size_t)min(lr & 7, a.M - 1) * a.K + kw0 + 32 * lg + 128 * (lr >> 3)
                        : a.x + (size_t)min(lr, a.M - 1) * a.K + kw0 + 32 * lg;
  const _Float16* sb = a.scale + (size_t)tt * G4 * 64 + lg * 16;
  auto load = [&](int s, DStage<RT, UPW, HX>& r) {
#pragma unroll
    for (int u = 0; u < (HX ? UPW / 2 : UPW); ++u)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        r.x[u][j] = *(const u32x4*)(xb + (s * UPW + (HX ? 2 * u : u)) * 128 + 8 * j);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int u = 0; u < UPW; ++u)
        r.w[rt][u] = load_nt((const u32x4*)(wb + ((size_t)rt * G + s * UPW + u) * 1024));
    const unsigned g = g0 + (unsigned)(s * UPW);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
      load_dwords(sb + (size_t)rt * G4 * 64 + (g / 4) * 64 + (g % 4) * 4, r.s[rt]);
  };

  NormRegs nr;
  if constexpr (NORM) norm_issue(a.ni, a.M, lane, nr);
  DStage<RT, UPW, HX> ring[DEPTH];
  // The first stages are issued in stage order, as the loop reissues them.
  // Left free, the scheduler moves every stage's scale load after the last
  // stage's weights; loads complete in order, so the loop's (static) wait
  // for stage 0's scales would then wait for the whole ring, every round.
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
  const u32x4 neg136 = {kNeg136x2, kNeg136x2, kNeg136x2, kNeg136x2};
  auto compute = [&](const DStage<RT, UPW, HX>& r) {
#pragma unroll
    for (int u = 0; u < UPW; ++u) {
      u32x4 xu[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) xu[j] = HX && (u & 1) ? rot8(r.x[u / 2][j]) : r.x[HX ? u / 2 : u][j];
      f32x4 xb136 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j) xb136 = mfma(neg136, xu[j], xb136);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        f32x4 cc = xb136;                          // C - 136 X
#pragma unroll
        for (int j = 0; j < 4; ++j) cc = mfma(unpack_w4(r.w[rt][u][j]), xu[j], cc);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[rt][i] = fma_half(r.s[rt], 4 * u + i, cc[i], acc[rt][i]);
      }
      // one group at a time: without this fence the scheduler hoists the
      // unpacking of later groups and the register ring no longer fits
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

// ---- 16 < M <= 64 -----------------------------------------------------------
//  * The waves of a workgroup share the staged x. They form NW/KW row groups
//    of RT row tiles; the KW waves of a row group split the workgroup's K
//    range and add their results through LDS in fixed order at the end
//    (KW = 1: each wave owns its rows over the whole range and stores them
//    itself). K slices inside a workgroup give small projections many waves
//    without split-K partials or a second pass.
//  * Each wave keeps DEPTH stages (UPW groups x RT row tiles) of loads in
//    flight. Every load is unconditional and the stage count is a multiple
//    of DEPTH, so the compiler's wait counts are static.
//  * X per (group, column) is an MFMA of ones against the staged x, once per
//    workgroup.
struct W4bArgs {
  const __bf16* x;
  const uint8_t* w;
  const _Float16* scale;
  __bf16* out;    // bf16 [M, N] when ksplit == 1
  float* part;    // fp32 [ksplit, M, N] otherwise
  int M, N, K;
  int kr;         // K range of a workgroup (a multiple of 128 * KW * UPW * DEPTH)
};

template <int RT, int UPW>
struct Stage {
  u32x4 w[RT][UPW];          // unit (rt, u): this lane's 16 bytes of block (tile, group)
  uint32_t s[RT][2 * UPW];   // fp16 scales: half 4u + i is row 4*lg + i of group u
};

// Grid: x = groups of (NW/KW)*RT row tiles, y = ksplit. Block: NW waves.
// MB: 16-column blocks of x (2 or 4; R = 16 MB rows staged).
template <int RT, int UPW, int DEPTH, int NW, int KW, int MB>
__global__ __launch_bounds__(NW * kWave, 2) void w4b_decode_kernel(W4bArgs a) {
  static_assert(NW % KW == 0, "K slices divide the waves");
  static_assert(MB == 2 || MB == 4, "M <= 16 is the direct kernel's");
  constexpr int R = 16 * MB;                      // x rows staged
  constexpr int NT = NW * kWave;
  extern __shared__ __align__(16) unsigned char smem[];
  const int wid = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int lg = lane >> 4, lr = lane & 15;
  const int KR = a.kr, kr0 = blockIdx.y * KR;
  const int GR = KR / 128, CPR = KR / 8;
  const int G = a.K / 128, G4 = a.K / 512;
  const int rg = wid / KW, kq = wid % KW;        // row group, K slice
  const int t0 = (blockIdx.x * (NW / KW) + rg) * RT;   // the row group's first tile
  const bool active = t0 < a.N / 16;              // (N / 16) % RT == 0 by the plan
  const int tt = active ? t0 : 0;                 // idle waves read tile 0, store nothing
  // LDS: x pieces [CPR][R] (16 bytes each) | group sums [GR][R]
  //      | K-slice results [NW][RT][MB][4][64] (KW > 1)
  u32x4* xs = (u32x4*)smem;
  float* xgs = (float*)(smem + (size_t)CPR * R * 16);

  const int GW = GR / KW, gw0 = kq * GW;          // this wave's groups of the range
  const int ns = GW / UPW;                        // stages of this wave
  const uint8_t* wb = a.w + ((size_t)tt * G + kr0 / 128 + gw0) * 1024 + lane * 16;
  auto load = [&](int s, Stage<RT, UPW>& r) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int u = 0; u < UPW; ++u)
        r.w[rt][u] = load_nt((const u32x4*)(wb + ((size_t)rt * G + s * UPW + u) * 1024));
    const unsigned g = (unsigned)(kr0 / 128 + gw0 + s * UPW);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
      load_dwords(a.scale + ((((size_t)(tt + rt) * G4 + g / 4) * 4 + lg) * 16 + (g % 4) * 4),
                  r.s[rt]);
  };

  // ---- x's first pieces, then the first DEPTH stages, then the rest of x ------
  // x [M, kr0 .. kr0+KR) goes to LDS as piece p = c * R + row (consecutive
  // threads write consecutive 16 bytes); rows past M re-read row M-1 (their
  // slots feed only output columns that are never stored). The first XB
  // pieces per thread are requested before the weights, so waiting for them
  // (an L2 round trip) does not wait for the weights: loads complete in order.
  constexpr int XB = 8;
  const int xtotal = R * CPR;
  auto x_load = [&](int p) -> u32x4 {
    p = min(p, xtotal - 1);
    const int m = min(p % R, a.M - 1), c = p / R;
    return *(const u32x4*)(a.x + (size_t)m * a.K + kr0 + c * 8);
  };
  u32x4 xv[XB];
#pragma unroll
  for (int u = 0; u < XB; ++u) xv[u] = x_load((int)threadIdx.x + u * NT);
  Stage<RT, UPW> ring[DEPTH];
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) {   // in stage order (see w4b_direct_kernel)
    load(d, ring[d]);
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int u = 0; u < XB; ++u)
    if ((int)threadIdx.x + u * NT < xtotal) xs[threadIdx.x + u * NT] = xv[u];
  for (int p0 = threadIdx.x + NT * XB; p0 < xtotal; p0 += NT * XB) {
#pragma unroll
    for (int u = 0; u < XB; ++u) xv[u] = x_load(p0 + u * NT);
#pragma unroll
    for (int u = 0; u < XB; ++u)
      if (p0 + u * NT < xtotal) xs[p0 + u * NT] = xv[u];
  }
  __syncthreads();
  // X per (group, column): an MFMA of ones against the group's x
  const u32x4 ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
  for (int q = wid; q < GR * MB; q += NW) {
    const int g = q / MB, mb = q % MB;
    f32x4 xg = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) xg = mfma(ones, xs[(g * 16 + 4 * lg + j) * R + mb * 16 + lr], xg);
    if (lg == 0) xgs[g * R + mb * 16 + lr] = xg[0];
  }
  __syncthreads();

  // ---- stream ------------------------------------------------------------------
  f32x4 acc[RT][MB];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[rt][mb] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](const Stage<RT, UPW>& r, int s) {
#pragma unroll
    for (int u = 0; u < UPW; ++u) {
      const int gl = gw0 + s * UPW + u;
      // the RT tiles' unpacked operands, then one column block at a time
      u32x4 aw[RT][4];
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int j = 0; j < 4; ++j) aw[rt][j] = unpack_w4(r.w[rt][u][j]);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const u32x4* xp = xs + (gl * 16 + 4 * lg) * R + mb * 16 + lr;
        u32x4 b[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) b[j] = xp[j * R];
        const float xg = xgs[gl * R + mb * 16 + lr];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          f32x4 cc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int j = 0; j < 4; ++j) cc = mfma(aw[rt][j], b[j], cc);
#pragma unroll
          for (int i = 0; i < 4; ++i)
            acc[rt][mb][i] = fma_half(r.s[rt], 4 * u + i, __builtin_fmaf(xg, -136.f, cc[i]),
                                      acc[rt][mb][i]);
        }
      }
      // one group at a time: without this fence the scheduler hoists the
      // unpacking of later groups and the register ring no longer fits
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  if (active) {
    int s0 = 0;
    for (; s0 + DEPTH < ns; s0 += DEPTH) {
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) {
        compute(ring[d], s0 + d);
        load(s0 + DEPTH + d, ring[d]);
      }
    }
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) compute(ring[d], s0 + d);
  }
  if constexpr (KW > 1) {
    // the K slices of a row group, added in slice order by slice 0
    float* red = xgs + GR * R;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          red[(((wid * RT + rt) * MB + mb) * 4 + i) * kWave + lane] = acc[rt][mb][i];
    __syncthreads();
    if (kq != 0) return;
#pragma unroll
    for (int q = 1; q < KW; ++q)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            acc[rt][mb][i] += red[((((wid + q) * RT + rt) * MB + mb) * 4 + i) * kWave + lane];
  }
  if (!active) return;

  // ---- store: lane (lr, lg) holds rows 4*lg .. 4*lg+3 of column 16 mb + lr ---
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int m = mb * 16 + lr;
    if (m >= a.M) break;
    if (a.out) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const int n = (t0 + rt) * 16 + 4 * lg;
        uint32_t v[2] = {pack_bf16x2(acc[rt][mb][0], acc[rt][mb][1]),
                         pack_bf16x2(acc[rt][mb][2], acc[rt][mb][3])};
        __builtin_memcpy(a.out + (size_t)m * a.N + n, v, sizeof(v));
      }
    } else {
      float* dst = a.part + ((size_t)blockIdx.y * a.M + m) * a.N;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) *(f32x4*)(dst + (t0 + rt) * 16 + 4 * lg) = acc[rt][mb];
    }
  }
}

// ---------------------------------------------------------------------------
// int4 GEMM for batches of 17..256 rows (a decode bucket of 64, configuration
// 3's M = 64 / 256), on the same W4B blocks. At these M the cost is moving x:
// every workgroup needs x for its K range, so the rows per workgroup set the x
// traffic (N / rows re-reads of it) and the split count the partial traffic.
// Here a workgroup of NW waves owns NW * RT 16-row tiles (256 rows at NW = 8,
// RT = 2) x 64 columns of x over a K range, and x moves through LDS one
// 128-k group at a time:
//  * every thread loads its share of the group's x (2 or 4 pieces of 16 bytes)
//    and each wave its RT weight blocks and their scales, DEPTH groups ahead in
//    a register ring (the loads of a group are issued together, so waiting for
//    the oldest group never waits for a later one);
//  * per group: the x pieces go to LDS (two buffers), one barrier, four waves
//    form X (the sum of x over the group, per column) with MFMAs against ones,
//    a second barrier, then each wave runs RT x 4 x 4 MFMAs: the unpacked
//    weight operands of a tile feed the four column blocks, each x operand the
//    RT tiles, and y += s (C - 136 X) as in the decode kernel;
//  * the M blocks of one (row block, split) are dealt to one XCD, so their
//    weight re-reads come from its L2;
//  * split-K partials as everywhere else: fp32 [ksplit, M, N], summed in split
//    order by the consumer.
struct W4mArgs {
  const __bf16* x;
  const uint8_t* w;
  const _Float16* scale;
  __bf16* out;    // bf16 [M, N] when ksplit == 1
  float* part;    // fp32 [ksplit, M, N] otherwise
  int M, N, K;
  int kr;         // K range of a split (a multiple of 128 * DEPTH)
};

constexpr int kMidBM = 64;                      // columns (x rows) per workgroup
constexpr int kMidMB = kMidBM / 16;
constexpr int kMidXP = kMidBM + 1;              // LDS pitch of one k piece (16-byte slots)

template <int RT, int NW, int DEPTH>
__global__ __launch_bounds__(NW * kWave, 1) void w4b_mid_kernel(W4mArgs a) {
  constexpr int NT = NW * kWave;
  constexpr int XPT = kMidBM * 16 / NT;          // x pieces per thread per group
  static_assert(XPT >= 1 && kMidBM * 16 % NT == 0, "whole x pieces per thread");
  extern __shared__ __align__(16) unsigned char smem[];
  u32x4* xs = (u32x4*)smem;                      // [2][16 pieces][kMidXP rows]
  float* xsum = (float*)(smem + 2 * 16 * kMidXP * 16);   // [2][64]
  const int wid = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int lg = lane >> 4, lr = lane & 15;
  int tile, split, mblk;
  {
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
  const int G = a.K / 128, G4 = a.K / 512;
  const int t0 = (tile * NW + wid) * RT;         // this wave's first 16-row tile
  const int gbase = split * (a.kr / 128);
  const int nch = a.kr / 128;
  const int m0 = mblk * kMidBM;

  struct Slot {
    u32x4 x[XPT];
    u32x4 w[RT];
    uint32_t s[RT][2];
  };
  // piece p of a group: x row p / 16, k piece p % 16 (8 k), so that a
  // wave's load covers 4 rows x 256 contiguous bytes (rows past M re-read row
  // M - 1; their columns are never stored); it goes to LDS slot
  // piece * kMidXP + row, whose pad makes the stores and the MFMA operand
  // reads (16 lanes: 16 consecutive rows of one piece) free of bank conflicts
  auto load = [&](int c, Slot& sl) {
    const int g = gbase + min(c, nch - 1);
#pragma unroll
    for (int u = 0; u < XPT; ++u) {
      const int p = (int)threadIdx.x + NT * u;
      const int m = min(m0 + p / 16, a.M - 1);
      sl.x[u] = *(const u32x4*)(a.x + (size_t)m * a.K + g * 128 + (p % 16) * 8);
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const size_t t = (size_t)(t0 + rt);
      sl.w[rt] = load_nt((const u32x4*)(a.w + (t * G + g) * 1024 + lane * 16));
      load_dwords(a.scale + (((t * G4 + g / 4) * 4 + lg) * 16 + (g % 4) * 4), sl.s[rt]);
    }
  };

  f32x4 acc[RT][kMidMB];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int mb = 0; mb < kMidMB; ++mb) acc[rt][mb] = f32x4{0.f, 0.f, 0.f, 0.f};
  const u32x4 ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};

  auto group = [&](int c, const Slot& sl) {
    const int b = c & 1;
    u32x4* xb = xs + b * 16 * kMidXP;
#pragma unroll
    for (int u = 0; u < XPT; ++u) {
      const int p = (int)threadIdx.x + NT * u;
      xb[(p % 16) * kMidXP + p / 16] = sl.x[u];
    }
    __syncthreads();
    if (wid < kMidMB) {
      f32x4 xg = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j) xg = mfma(ones, xb[(4 * lg + j) * kMidXP + wid * 16 + lr], xg);
      if (lg == 0) xsum[b * kMidBM + wid * 16 + lr] = xg[0];
    }
    __syncthreads();
    u32x4 aw[RT][4];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int j = 0; j < 4; ++j) aw[rt][j] = unpack_w4(sl.w[rt][j]);
#pragma unroll
    for (int mb = 0; mb < kMidMB; ++mb) {
      u32x4 bx[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) bx[j] = xb[(4 * lg + j) * kMidXP + mb * 16 + lr];
      const float xg = xsum[b * kMidBM + mb * 16 + lr];
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        f32x4 cc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) cc = mfma(aw[rt][j], bx[j], cc);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          acc[rt][mb][i] = fma_half(sl.s[rt], i, __builtin_fmaf(xg, -136.f, cc[i]),
                                    acc[rt][mb][i]);
      }
    }
  };

  Slot ring[DEPTH];
  // in slot order, as the loop reissues them: left free, the scheduler issued
  // slot 0's x last, and the loop's static wait for it drained the whole ring
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) {
    load(d, ring[d]);
    __builtin_amdgcn_sched_barrier(0);
  }
  for (int c0 = 0; c0 < nch; c0 += DEPTH) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      group(c0 + d, ring[d]);
      load(c0 + d + DEPTH, ring[d]);   // past the end: re-reads the last group
    }
  }

  // lane (lr, lg) holds rows 4 lg .. 4 lg + 3 of tile t0 + rt, column 16 mb + lr
#pragma unroll
  for (int mb = 0; mb < kMidMB; ++mb) {
    const int m = m0 + mb * 16 + lr;
    if (m >= a.M) break;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int n = (t0 + rt) * 16 + 4 * lg;
      if (a.out) {
        uint32_t v[2] = {pack_bf16x2(acc[rt][mb][0], acc[rt][mb][1]),
                         pack_bf16x2(acc[rt][mb][2], acc[rt][mb][3])};
        __builtin_memcpy(a.out + (size_t)m * a.N + n, v, sizeof(v));
      } else {
        *(f32x4*)(a.part + ((size_t)split * a.M + m) * a.N + n) = acc[rt][mb];
      }
    }
  }
}

template <int RT, int NW, int DEPTH>
int launch_mid(const W4mPlan& p, const W4mArgs& a, hipStream_t st) {
  w4b_mid_kernel<RT, NW, DEPTH><<<dim3((unsigned)p.groups, (unsigned)p.ksplit,
                                       (unsigned)p.mblocks),
                                  dim3(NW * kWave), p.lds, st>>>(a);
  return ACORN_OK;
}

size_t w4b_lds(int R, int64_t kr, int nw, int kw, int rt, int mb) {
  return (size_t)kr * R * 2 + (size_t)(kr / 128) * R * 4 +
         (kw > 1 ? (size_t)nw * rt * mb * 4 * kWave * 4 : 0);
}

// ---- launchers: the direct kernel (M <= 16) ---------------------------------
// registers of one stage (dwords per lane): weights, x operands (HX: half),
// scales
constexpr int direct_stage_dwords(int rt, int upw, bool hx = false) {
  return 4 * rt * upw + 16 * (hx ? upw / 2 : upw) + 2 * rt * upw;
}
constexpr int kDirectRingDwords = 160;   // the ring's budget (depth x stage)

template <int RT, int UPW, int DEPTH, int RG, int KW, bool HX>
int launch_direct_x(const W4bPlan& p, const W4dArgs& a, hipStream_t st) {
  const dim3 grid((unsigned)p.groups, (unsigned)p.ksplit), block(RG * KW * kWave);
  if constexpr (RT >= 2) {
    if (p.swiglu) {
      if (p.mode == 1)
        w4b_direct_kernel<RT, UPW, DEPTH, RG, KW, true, 1, HX><<<grid, block, 0, st>>>(a);
      else
        w4b_direct_kernel<RT, UPW, DEPTH, RG, KW, true, 0, HX><<<grid, block, 0, st>>>(a);
      return ACORN_OK;
    }
  }
  if (p.swiglu) return ACORN_ERR_UNSUPPORTED;
  switch (p.mode) {
    case 0: w4b_direct_kernel<RT, UPW, DEPTH, RG, KW, false, 0, HX><<<grid, block, 0, st>>>(a); break;
    case 1: w4b_direct_kernel<RT, UPW, DEPTH, RG, KW, false, 1, HX><<<grid, block, 0, st>>>(a); break;
    case 2: w4b_direct_kernel<RT, UPW, DEPTH, RG, KW, false, 2, HX><<<grid, block, 0, st>>>(a); break;
    default: return ACORN_ERR_UNSUPPORTED;
  }
  return ACORN_OK;
}

// the paired-x form where the plan asks for it (M <= 8, two groups per stage),
// each form only within the ring's budget
template <int RT, int UPW, int DEPTH, int RG, int KW>
int launch_direct(const W4bPlan& p, const W4dArgs& a, hipStream_t st) {
  if constexpr (UPW % 2 == 0 && DEPTH * direct_stage_dwords(RT, UPW, true) <= kDirectRingDwords) {
    if (p.hx) return launch_direct_x<RT, UPW, DEPTH, RG, KW, true>(p, a, st);
  }
  if constexpr (DEPTH * direct_stage_dwords(RT, UPW) <= kDirectRingDwords) {
    if (!p.hx) return launch_direct_x<RT, UPW, DEPTH, RG, KW, false>(p, a, st);
  }
  return ACORN_ERR_UNSUPPORTED;
}

// wave layouts (the nw field): 1 or 4 waves on their own rows, or 10 nw + kw
// with kw waves splitting K over nw / kw row groups (22, 44, 84, 88). The
// eight-wave layouts give a projection that runs in one split (the residual
// epilogue) twice the waves of 44.
template <int RT, int UPW, int DEPTH>
int direct_nw(const W4bPlan& p, const W4dArgs& a, hipStream_t st) {
  switch (p.nw_field) {
    case 1: return launch_direct<RT, UPW, DEPTH, 1, 1>(p, a, st);
    case 4: return launch_direct<RT, UPW, DEPTH, 4, 1>(p, a, st);
    case 22: return launch_direct<RT, UPW, DEPTH, 1, 2>(p, a, st);
    case 44: return launch_direct<RT, UPW, DEPTH, 1, 4>(p, a, st);
    case 84: return launch_direct<RT, UPW, DEPTH, 2, 4>(p, a, st);
    case 88: return launch_direct<RT, UPW, DEPTH, 1, 8>(p, a, st);
  }
  return ACORN_ERR_UNSUPPORTED;
}

template <int RT, int UPW>
int direct_depth(const W4bPlan& p, const W4dArgs& a, hipStream_t st) {
  switch (p.depth) {
    case 1: return direct_nw<RT, UPW, 1>(p, a, st);
    case 2: return direct_nw<RT, UPW, 2>(p, a, st);
    case 4:
      if constexpr (4 * direct_stage_dwords(RT, UPW, UPW % 2 == 0) <= kDirectRingDwords)
        return direct_nw<RT, UPW, 4>(p, a, st);
      break;
  }
  return ACORN_ERR_UNSUPPORTED;
}

template <int RT>
int direct_upw(const W4bPlan& p, const W4dArgs& a, hipStream_t st) {
  switch (p.upw) {
    case 1: return direct_depth<RT, 1>(p, a, st);
    case 2: return direct_depth<RT, 2>(p, a, st);
  }
  return ACORN_ERR_UNSUPPORTED;
}

// ---- launchers: the LDS kernel (16 < M <= 64) -------------------------------
template <int RT, int UPW, int DEPTH, int NW, int KW, int MB>
int launch5(const W4bPlan& p, const W4bArgs& a, hipStream_t st) {
  auto kfn = w4b_decode_kernel<RT, UPW, DEPTH, NW, KW, MB>;
  static bool raised = false;  // once per kernel, before any graph capture
  if (!raised && p.lds > 64 * 1024) {
    (void)hipFuncSetAttribute((const void*)kfn, hipFuncAttributeMaxDynamicSharedMemorySize,
                              160 * 1024);
    raised = true;
  }
  dim3 grid((unsigned)p.groups, (unsigned)p.ksplit), block(NW * kWave);
  kfn<<<grid, block, p.lds, st>>>(a);
  return ACORN_OK;
}

// (waves, K slices) per workgroup
template <int RT, int UPW, int DEPTH, int MB>
int launch3(const W4bPlan& p, const W4bArgs& a, hipStream_t st) {
  switch (p.nw * 16 + p.kw) {
    case 2 * 16 + 1: return launch5<RT, UPW, DEPTH, 2, 1, MB>(p, a, st);
    case 4 * 16 + 1: return launch5<RT, UPW, DEPTH, 4, 1, MB>(p, a, st);
    case 4 * 16 + 2: return launch5<RT, UPW, DEPTH, 4, 2, MB>(p, a, st);
    case 4 * 16 + 4: return launch5<RT, UPW, DEPTH, 4, 4, MB>(p, a, st);
    case 8 * 16 + 2: return launch5<RT, UPW, DEPTH, 8, 2, MB>(p, a, st);
    case 8 * 16 + 4: return launch5<RT, UPW, DEPTH, 8, 4, MB>(p, a, st);
  }
  return ACORN_ERR_UNSUPPORTED;
}

// one or two stages in flight of one or two groups
template <int RT, int UPW, int MB>
int launch2(const W4bPlan& p, const W4bArgs& a, hipStream_t st) {
  switch (p.depth) {
    case 1: return launch3<RT, UPW, 1, MB>(p, a, st);
    case 2: return launch3<RT, UPW, 2, MB>(p, a, st);
  }
  return ACORN_ERR_UNSUPPORTED;
}

template <int RT, int MB>
int launch1(const W4bPlan& p, const W4bArgs& a, hipStream_t st) {
  switch (p.upw) {
    case 1: return launch2<RT, 1, MB>(p, a, st);
    case 2: return launch2<RT, 2, MB>(p, a, st);
  }
  return ACORN_ERR_UNSUPPORTED;
}

template <int MB>
int launch_rt(const W4bPlan& p, const W4bArgs& a, hipStream_t st) {
  switch (p.rt) {
    case 1: return launch1<1, MB>(p, a, st);
    case 2: return launch1<2, MB>(p, a, st);
    case 4:
      if constexpr (MB <= 2) return launch1<4, MB>(p, a, st);
      break;
  }
  return ACORN_ERR_UNSUPPORTED;
}

int divisor_at_least(int64_t n, int64_t v) {
  while (v <= n && n % v) ++v;
  return v <= n ? (int)v : 0;
}

// M <= 16: rt 1/2/4 (swiglu 2/4; N/16 divisible by rt), upw 1/2, the wave
// layout in the nw field (1 or 4 waves on their own rows; 22, 44, 84, 88 = nw
// waves in nw / kw row groups of kw K slices; at M <= 8 upw 2 takes the
// paired-x form, whose smaller stages fit deeper rings), depth 1/2/4 within the ring's
// register budget, and split counts that give every wave a whole number of
// depth rounds. With 0 the plan takes rt 2, upw 1, one wave per workgroup,
// depth 4, and the fewest splits that launch at least three waves per CU.
int direct_plan(int64_t M, int64_t N, int64_t K, const int* cfg, bool swiglu, W4bPlan* p) {
  const int64_t ntiles = N / 16, G = K / 128;
  int rt = cfg && cfg[0] > 0 ? cfg[0] : 2;
  const int upw = cfg && cfg[1] > 0 ? cfg[1] : 1;
  const int nwf = cfg && cfg[2] > 0 ? cfg[2] : 1;
  const int req_ks = cfg ? cfg[3] : 0;
  int depth = cfg && cfg[4] > 0 ? cfg[4] : 4;
  if (rt != 1 && rt != 2 && rt != 4) return ACORN_ERR_UNSUPPORTED;
  if (swiglu && rt < 2) rt = 2;
  while (rt > (swiglu ? 2 : 1) && ntiles % rt) rt /= 2;
  if (ntiles % rt) return ACORN_ERR_UNSUPPORTED;
  if (upw != 1 && upw != 2) return ACORN_ERR_UNSUPPORTED;
  if (nwf != 1 && nwf != 4 && nwf != 22 && nwf != 44 && nwf != 84 && nwf != 88)
    return ACORN_ERR_UNSUPPORTED;
  const int nw = nwf < 10 ? nwf : nwf / 10, kw = nwf < 10 ? 1 : nwf % 10;
  if (depth != 1 && depth != 2 && depth != 4) return ACORN_ERR_UNSUPPORTED;
  // M <= 8 with two groups per stage: the paired-x form (half the x registers)
  const bool hx = M <= 8 && upw == 2;
  while (depth > 1 && (depth * direct_stage_dwords(rt, upw, hx) > kDirectRingDwords ||
                       G % (kw * upw * depth)))
    depth /= 2;
  // K % 512 == 0 makes the default (kw = upw = depth = 1) always fit: what
  // does not is a request the shape cannot honour
  if (G % (kw * upw * depth)) return ACORN_ERR_UNSUPPORTED;
  const int64_t q = G / (kw * upw * depth);     // ks must divide this
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
  const int64_t rgs = nw / kw;                 // row groups per workgroup
  const int64_t groups = (ntiles / rt + rgs - 1) / rgs;
  if (groups > 0x7fffffff || ks > 65535) return ACORN_ERR_SHAPE;
  p->direct = true;
  p->rt = rt;
  p->upw = upw;
  p->nw = nw;
  p->kw = kw;
  p->nw_field = nwf;
  p->ksplit = ks;
  p->depth = depth;
  p->R = (int)M;
  p->mb = 1;
  p->groups = (int)groups;
  p->lds = 0;
  p->swiglu = swiglu;
  p->mode = 0;
  p->hx = hx;
  return ACORN_OK;
}

}  // namespace

namespace acorn {

// M <= 16: the direct kernel (direct_plan). 16 < M <= 64: the LDS kernel with
// mb = ceil(M / 16) column blocks (32 or 64 x rows staged): rt 1/2/4 with
// rt * mb <= 8, upw and depth 1 or 2, and the wave layout in the nw field:
// 2 or 4 = that many waves with one K slice, 10*nw + kw = nw waves in nw/kw
// row groups of kw K slices (42, 44, 82, 84). ksplit and kw divide the
// per-row stage count G/upw so that every wave's K range holds a whole
// number of depth-stage rounds. With 0 the split grows from 1 until about two
// workgroups per CU are launched, while one workgroup's x fits its LDS budget
// and each K range keeps at least 512 k. No fused SwiGLU above 16 rows.
int w4b_make_plan(int64_t M, int64_t N, int64_t K, const int* cfg, bool swiglu, W4bPlan* p) {
  if (M < 1 || M > 64) return ACORN_ERR_UNSUPPORTED;
  if (N % 16 || K % 512) return ACORN_ERR_SHAPE;
  if (swiglu && N % 32) return ACORN_ERR_SHAPE;
  if (M <= 16) return direct_plan(M, N, K, cfg, swiglu, p);
  if (swiglu) return ACORN_ERR_UNSUPPORTED;
  const int mb = M <= 32 ? 2 : 4;
  const int64_t ntiles = N / 16, G = K / 128;
  int rt = cfg && cfg[0] > 0 ? cfg[0] : 2;
  int upw = cfg && cfg[1] > 0 ? cfg[1] : 2;
  const int nwf = cfg && cfg[2] > 0 ? cfg[2] : 4;
  const int req_ks = cfg ? cfg[3] : 0, req_depth = cfg ? cfg[4] : 0;
  const int nw = nwf < 10 ? nwf : nwf / 10, kw = nwf < 10 ? 1 : nwf % 10;
  const bool layout_ok = (kw == 1 && (nw == 2 || nw == 4)) ||
                         (nw == 4 && (kw == 2 || kw == 4)) || (nw == 8 && (kw == 2 || kw == 4));
  if (!layout_ok) return ACORN_ERR_UNSUPPORTED;
  if (rt != 1 && rt != 2 && rt != 4) return ACORN_ERR_UNSUPPORTED;
  while (rt > 1 && ntiles % rt) rt /= 2;
  if (upw != 1 && upw != 2) return ACORN_ERR_UNSUPPORTED;
  if (rt * mb > 8) return ACORN_ERR_UNSUPPORTED;
  const int R = 16 * mb;
  if (G % upw) return ACORN_ERR_SHAPE;
  const int64_t stages = G / upw;            // per row over the whole K
  if (stages % kw) return ACORN_ERR_UNSUPPORTED;
  const int64_t slices = stages / kw;        // per K slice with one split
  const size_t lds_cap = 160 * 1024, lds_default = 80 * 1024;
  const int64_t groups = (ntiles / rt + nw / kw - 1) / (nw / kw);
  auto lds = [&](int ks) { return w4b_lds(R, K / ks, nw, kw, rt, mb); };
  int ks;
  if (req_ks > 0) {
    ks = divisor_at_least(slices, req_ks);
    while (ks && lds(ks) > lds_cap) ks = divisor_at_least(slices, ks + 1);
    if (!ks) return ACORN_ERR_UNSUPPORTED;
  } else {
    ks = 1;
    while (lds(ks) > lds_default) {
      const int nx = divisor_at_least(slices, ks + 1);
      if (!nx) break;
      ks = nx;
    }
    while (groups * ks < 2 * 256) {
      const int nx = divisor_at_least(slices, ks + 1);
      if (!nx || K / nx / kw < 512) break;
      ks = nx;
    }
  }
  if (lds(ks) > lds_cap) return ACORN_ERR_UNSUPPORTED;
  const int64_t ns = slices / ks;            // stages of one wave
  int depth = req_depth > 0 ? req_depth : 2;
  if (depth != 1 && depth != 2 && depth != 4 && depth != 8) return ACORN_ERR_UNSUPPORTED;
  while (depth > 1 && (ns % depth || depth > 2)) depth /= 2;
  p->direct = false;
  p->rt = rt;
  p->upw = upw;
  p->nw = nw;
  p->kw = kw;
  p->nw_field = nwf < 10 ? nw : nwf;
  p->ksplit = ks;
  p->depth = depth;
  p->R = R;
  p->mb = mb;
  p->groups = (int)groups;
  p->lds = lds(ks);
  p->swiglu = false;
  p->mode = 0;
  p->hx = false;
  if (groups > 0x7fffffff || ks > 65535) return ACORN_ERR_SHAPE;
  return ACORN_OK;
}

int w4b_launch(const W4bPlan& p, const void* x, const void* w, const void* scale,
               const void* zero, void* out, float* part, int64_t M, int64_t N, int64_t K,
               const NormIn* ni, const ResidOut* ro, hipStream_t st) {
  if (zero) return ACORN_ERR_UNSUPPORTED;  // the block layout is the symmetric format
  if (!x || !w || !scale) return ACORN_ERR_VALUE;
  // bf16 (or SwiGLU act) output only with one split; else fp32 partials
  if (p.ksplit > 1) out = nullptr;
  if (p.mode != 0 && !p.direct) return ACORN_ERR_UNSUPPORTED;
  if (p.mode == 2) {
    if (!ro || !ro->res || !ro->res_out || !ro->ss || !ro->nw || !ro->xw) return ACORN_ERR_VALUE;
    if (p.ksplit != 1 || p.swiglu) return ACORN_ERR_UNSUPPORTED;
  } else if (!out && (!part || p.swiglu)) {
    return ACORN_ERR_VALUE;
  }
  if (p.mode == 1 && (!ni || !ni->ss || ni->nss * 16 != K)) return ACORN_ERR_VALUE;
  int rc = ACORN_ERR_UNSUPPORTED;
  if (p.direct) {
    if (M > 16) return ACORN_ERR_UNSUPPORTED;
    W4dArgs a{(const __bf16*)x, (const uint8_t*)w, (const _Float16*)scale, (__bf16*)out,
              part, (int)M, (int)N, (int)K, (int)(K / p.ksplit), NormIn{}, ResidOut{}};
    if (ni) a.ni = *ni;
    if (ro) a.ro = *ro;
    switch (p.rt) {
      case 1: rc = direct_upw<1>(p, a, st); break;
      case 2: rc = direct_upw<2>(p, a, st); break;
      case 4: rc = direct_upw<4>(p, a, st); break;
    }
  } else {
    if (M <= 16 || M > 16 * p.mb) return ACORN_ERR_UNSUPPORTED;
    const W4bArgs a{(const __bf16*)x, (const uint8_t*)w, (const _Float16*)scale, (__bf16*)out,
                    part, (int)M, (int)N, (int)K, (int)(K / p.ksplit)};
    switch (p.mb) {
      case 2: rc = launch_rt<2>(p, a, st); break;
      case 4: rc = launch_rt<4>(p, a, st); break;
    }
  }
  if (rc) return rc;
  ACORN_LAUNCH_CHECK();
  return ACORN_OK;
}

// Knobs: rt (16-row tiles per wave) 1 or 2, nw (waves) 4 or 8, ksplit, depth
// (groups in flight) 2 or 4, and 8 for rt 1 with 8 waves (rt 2 with 8 waves
// and depth 8 spills its registers); N must be a whole number of NW * RT * 16 row
// blocks, K of 128-k groups, and each split's group count of depth rounds. With
// ksplit 0 the split grows from 1 while the launch has fewer workgroups than
// 256 (two rounds of CUs at most) and each split keeps 4 depth rounds.
int w4m_make_plan(int64_t M, int64_t N, int64_t K, const int* cfg, W4mPlan* p) {
  if (M < 1 || M > 65535 * (int64_t)kMidBM) return ACORN_ERR_SHAPE;
  if (K % 512) return ACORN_ERR_SHAPE;
  const int rt = cfg && cfg[1] > 0 ? cfg[1] : 2;
  const int nw = cfg && cfg[2] > 0 ? cfg[2] : 8;
  const int req_ks = cfg ? cfg[3] : 0;
  const int depth = cfg && cfg[4] > 0 ? cfg[4] : 2;
  if ((rt != 1 && rt != 2) || (nw != 4 && nw != 8) ||
      (depth != 2 && depth != 4 && !(depth == 8 && rt == 1 && nw == 8)))
    return ACORN_ERR_UNSUPPORTED;
  const int64_t rows = (int64_t)nw * rt * 16;
  if (N % rows) return ACORN_ERR_UNSUPPORTED;
  const int64_t G = K / 128, groups = N / rows, mblocks = (M + kMidBM - 1) / kMidBM;
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
  p->lds = (size_t)2 * 16 * kMidXP * 16 + (size_t)2 * kMidBM * 4;
  return ACORN_OK;
}

int w4m_launch(const W4mPlan& p, const void* x, const void* w, const void* scale, void* out,
               float* part, int64_t M, int64_t N, int64_t K, hipStream_t st) {
  if (!x || !w || !scale) return ACORN_ERR_VALUE;
  if (p.ksplit > 1) out = nullptr;
  if (!out && !part) return ACORN_ERR_VALUE;
  W4mArgs a;
  a.x = (const __bf16*)x;
  a.w = (const uint8_t*)w;
  a.scale = (const _Float16*)scale;
  a.out = (__bf16*)out;
  a.part = part;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.kr = (int)(K / p.ksplit);
  int rc = ACORN_ERR_UNSUPPORTED;
  switch (p.rt * 100 + p.nw * 10 + p.depth) {
    case 142: rc = launch_mid<1, 4, 2>(p, a, st); break;
    case 144: rc = launch_mid<1, 4, 4>(p, a, st); break;
    case 182: rc = launch_mid<1, 8, 2>(p, a, st); break;
    case 184: rc = launch_mid<1, 8, 4>(p, a, st); break;
    case 242: rc = launch_mid<2, 4, 2>(p, a, st); break;
    case 244: rc = launch_mid<2, 4, 4>(p, a, st); break;
    case 188: rc = launch_mid<1, 8, 8>(p, a, st); break;
    case 282: rc = launch_mid<2, 8, 2>(p, a, st); break;
    case 284: rc = launch_mid<2, 8, 4>(p, a, st); break;
  }
  if (rc) return rc;
  ACORN_LAUNCH_CHECK();
  return ACORN_OK;
}

}  // namespace acorn

// ---- W4B -> bf16 [N, K] (prefill-sized projections) ------------------------
// out[n, k] = bf16_rne((u - 8) * s(n, k / 128)). (u - 8) * s is exact in fp32
// (a 4-bit integer times an 11-bit significand), so the result is the
// weight rounded once to bf16. One wave per 1 KB block (16 rows x 128 k;
// 4 KB of output). The output is four fifths of the traffic, so every store
// instruction writes whole 128-byte lines: 8 lanes per line (16 bytes = 8 k
// each), 8 rows per instruction, 4 instructions per block. A lane's loads
// follow its stores: 4 bytes (8 nibbles) per line it writes, from the block's
// 16-byte piece (chunk c, row r); each load instruction reads two whole
// lines of the block.
namespace {

__global__ __launch_bounds__(256) void w4b_dequant_kernel(const uint32_t* __restrict__ w,
                                                          const _Float16* __restrict__ scale,
                                                          __bf16* __restrict__ out, int64_t K,
                                                          int64_t blocks) {
  const int64_t b = (int64_t)blockIdx.x * 4 + threadIdx.x / kWave;
  if (b >= blocks) return;
  const int lane = threadIdx.x % kWave;
  const int j = lane & 7, rr = lane >> 3;
  const int64_t G = K / 128;
  const int64_t t = b / G, g = b % G;
  const uint32_t* blk = w + b * 256;
  uint32_t d[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int h = i >> 1, r = (i & 1) * 8 + rr, c = 2 * h + (j >> 2);
    d[i] = __builtin_nontemporal_load(blk + (c * 16 + r) * 4 + (j & 3));
  }
  float s[2];
#pragma unroll
  for (int e = 0; e < 2; ++e) s[e] = (float)scale[w4b_half_index(t * 16 + e * 8 + rr, g, K)];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int h = i >> 1, r = (i & 1) * 8 + rr;
    const float sc = s[i & 1];
    u32x4 o;
    // k offsets 2q and 2q + 1 of the word are its nibbles q and q + 4
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int lo = (int)((d[i] >> (4 * q)) & 15u), hi = (int)((d[i] >> (4 * q + 16)) & 15u);
      o[q] = pack_bf16x2((float)(lo - 8) * sc, (float)(hi - 8) * sc);
    }
    *(u32x4*)(out + (t * 16 + r) * K + g * 128 + 64 * h + 8 * j) = o;
  }
}

}  // namespace

namespace acorn {

int w4b_dequant(const void* w, const void* scale, void* out, int64_t N, int64_t K,
                hipStream_t st) {
  if (N <= 0 || K <= 0 || N % 16 || K % 512) return ACORN_ERR_SHAPE;
  if (!w || !scale || !out) return ACORN_ERR_VALUE;
  const int64_t blocks = (N / 16) * (K / 128);
  const int64_t wgs = (blocks + 3) / 4;
  if (wgs > 0x7fffffff) return ACORN_ERR_SHAPE;
  w4b_dequant_kernel<<<(unsigned)wgs, 256, 0, st>>>((const uint32_t*)w, (const _Float16*)scale,
                                                    (__bf16*)out, K, blocks);
  ACORN_LAUNCH_CHECK();
  return ACORN_OK;
}

}  // namespace acorn
