// Weight-only GEMM y[M,N] = x[M,K] @ dequant(W)[N,K]^T on gfx950 MFMA.
//
// Formats (acorn_hip.h): dense bf16, int8 per-channel (fp16 scale [N], the
// reference's W8A16, acorninfer/quant/quantize.py:89-99) and packed uint4
// group-128 (fp16 scale [N,K/128], optional fp16 zero [N,K/128]; byte =
// u_even | u_odd << 4 as in quantize.py:122-131; symmetric int4 v in [-8,7]
// is stored as u = v + 8 with zero = -8*scale, which dequantises exactly).
// A fourth format, dense fp32 with fp32 activations, is a plain VALU kernel
// for the fp32 parity path.
//
// Decode (M <= 16) is a weight stream, so the kernel is built to keep HBM
// busy:
//  * v_mfma_f32_16x16x32_bf16 with the WEIGHTS as the 16-row A operand and x
//    (M rows, padded) as the B operand. One 16-byte load per lane feeds 1
//    (bf16), 2 (int8) or 4 (int4) MFMAs. Weights are loaded in whole cache
//    lines with the non-temporal policy and moved into the A layout through
//    a per-wave LDS slab.
//  * int4 -> bf16 in two VALU ops per dword: (w >> 4p) & 0x000F000F | 0x43004300
//    is the bf16 pair (128+u_p, 128+u_{p+4}); the (p, p+4) pairing is a k
//    permutation applied once to x when it is staged into LDS.
//    int8 -> bf16 via (q ^ 0x80) -> v_cvt_f32_ubyteN -> v_cvt_pk_bf16_f32
//    (= 128+q, exact). The +128 offset is removed with X = sum_k x (an MFMA
//    against ones, computed once per workgroup because x does not change
//    from tile to tile): y = s*(C - 128 X) (+ zero*X for int4), per 128-group
//    for int4, once per row for int8.
//  * A workgroup owns a run of 16*RT-row tiles and one K range (split
//    blockIdx.y). x for the whole K range is staged in LDS once, in MFMA-B
//    order ([k/8][row][8], one conflict-free ds_read_b128 per B fetch).
//    The NW waves split the K range and walk (tile, k-chunk) steps through
//    a ring of D register sets (D = 8, 4, 2 or 1 by the step's size). The
//    first x loads, then the first D steps' weights and scales, are issued
//    before anything waits, so a decode-sized workgroup (nsteps <= D) has
//    all of its HBM reads in flight at once. Every load is unconditional
//    (clamped indices): a load under a branch makes the compiler wait for
//    all outstanding loads before the next use.
//  * At the end of a tile the waves' partials are summed through
//    double-buffered LDS in fixed wave order (one barrier per tile).
//  * Split-K (ksplit > 1): each split writes fp32 partials, which the
//    consumer (the decode step's K1 / SwiGLU / qkv epilogue, or
//    splitk_reduce_kernel for a bf16 output) sums in split order, so results
//    are bitwise deterministic. There is no cross-workgroup reduction inside
//    the kernel: on CDNA an agent-scope fence writes back and invalidates the
//    XCD's whole L2.
#include <algorithm>

#include "gemm_common.h"

using namespace acorn;

namespace {

template <int WFMT> struct Fmt;
template <> struct Fmt<ACORN_WFMT_BF16> {
  static constexpr int KU = 32;                   // k of one 16-byte lane load across the wave
  static constexpr int MPU = 1;                   // MFMAs per unit
  static constexpr int BPK_NUM = 2, BPK_DEN = 1;  // bytes per k
};
template <> struct Fmt<ACORN_WFMT_W8> {
  static constexpr int KU = 64, MPU = 2, BPK_NUM = 1, BPK_DEN = 1;
};
template <> struct Fmt<ACORN_WFMT_W4> {
  static constexpr int KU = 128, MPU = 4, BPK_NUM = 1, BPK_DEN = 2;
};

// int4 in either layout (natural rows, or the 1 KB blocks of W4B)
template <int WFMT> constexpr bool kIsW4 = WFMT == ACORN_WFMT_W4 || WFMT == ACORN_WFMT_W4B;
// int8 in either layout (natural rows, or the biased 1 KB blocks of W8B)
template <int WFMT> constexpr bool kIsW8 = WFMT == ACORN_WFMT_W8 || WFMT == ACORN_WFMT_W8B;

// x staged for the streaming kernel over natural-layout int4 (low nibble =
// even k): the 8 bf16 of a 16-byte piece reordered to [x0,x4,x1,x5,x2,x6,x3,
// x7], unpack_w4's pairing (nibble q, nibble q+4) of a natural word.
__device__ __forceinline__ u32x4 w4_order_x(u32x4 w) {
  u32x4 t;
  t[0] = __builtin_amdgcn_perm(w[2], w[0], 0x05040100u);
  t[1] = __builtin_amdgcn_perm(w[2], w[0], 0x07060302u);
  t[2] = __builtin_amdgcn_perm(w[3], w[1], 0x05040100u);
  t[3] = __builtin_amdgcn_perm(w[3], w[1], 0x07060302u);
  return t;
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

// fp16 number u of a run of packed halves (even u in the low half).
template <int NDW>
__device__ __forceinline__ float half_at(const uint32_t (&d)[NDW], int u) {
  const uint32_t v = d[u / 2];
  return (float)__builtin_bit_cast(_Float16, (uint16_t)((u & 1) ? v >> 16 : v & 0xffffu));
}

// Registers of one pipeline step: this lane's weight units plus the scales
// of the output rows it holds (rows 4*(lane/16)+i of each 16-row group), as
// packed fp16 pairs. int4 keeps UPW group scales (and, with ZERO, zero
// points) per row; int8 keeps the 4 channel scales.
template <int WFMT, int RT, int UPW, bool ZERO>
struct StepRegs {
  static constexpr bool W4 = WFMT == ACORN_WFMT_W4;
  static constexpr int NR = W4 ? 4 : 1;
  static constexpr int NDW = W4 ? (UPW + 1) / 2 : 2;
  u32x4 w[RT][UPW];
  uint32_t s[RT][NR][NDW];
  uint32_t z[RT][ZERO ? 4 : 1][ZERO ? NDW : 1];
};

struct KArgs {
  const __bf16* x;
  const uint8_t* w;
  const _Float16* scale;
  const _Float16* zero;
  __bf16* out;
  float* part;
  int M, N, K;
  int nk;          // k-chunks per tile (K range = nk * KC)
  int tpw;         // tiles per workgroup
  int ksplit;
  int log2R;       // LDS rows per m tile = 1 << log2R
};

// Grid: x = tile groups, y = ksplit, z = m blocks of 16*MT rows.
// SWIGLU: RT == 2, the tile's first 16 weight rows are gate rows and the next
// 16 the up rows of the same 16 outputs; out is act [M, N/2] (ksplit == 1).
// ZERO: int4 with zero points (a.zero != nullptr).
template <int WFMT, int RT, int MT, int UPW, int NW, bool SWIGLU, bool ZERO>
__global__ __launch_bounds__(NW * kWave, NW == 8 ? 2 : 3) void wgemm_kernel(KArgs a) {
  using F = Fmt<WFMT>;
  constexpr int KU = F::KU, MPU = F::MPU, ROWS = 16 * RT;
  constexpr int KC = NW * UPW * KU;               // k per chunk (all waves)
  constexpr int TILE = RT * MT * 4 * kWave;       // floats of one wave's tile partial
  constexpr int NT = NW * kWave;
  extern __shared__ __align__(16) unsigned char smem[];

  const int wid = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int lg = lane >> 4, lr = lane & 15;
  const int R = 1 << a.log2R;
  const int nk = a.nk;
  const int KR = nk * KC;                         // K range of this workgroup
  const int kr0 = blockIdx.y * KR;
  const int CPR = KR / 8;                         // 16-byte x pieces per row
  const int GR = KR / 128;                        // int4 groups in the K range
  const int ntiles = a.N / ROWS;
  const int t_begin = blockIdx.x * a.tpw;
  const int t_end = min(t_begin + a.tpw, ntiles);
  if (t_begin >= t_end) return;                   // uniform for the workgroup
  const int mblk = blockIdx.z * 16 * MT;
  const size_t wrow = (size_t)a.K * F::BPK_NUM / F::BPK_DEN;
  const int G = a.K / 128;

  // LDS: x [MT][CPR][R] u32x4 | int4 group sums [MT][GR][16] f32 | red [2][NW][TILE]
  //      | per-wave slabs [NW][ROWS][SBW + 16] bytes
  u32x4* xs = (u32x4*)smem;
  float* xgs = (float*)(smem + (size_t)MT * CPR * R * 16);
  float* red = xgs + (WFMT == ACORN_WFMT_W4 ? MT * GR * 16 : 0);
  // Weights are read in whole cache lines: a wave's step covers ROWS rows x
  // SBW contiguous bytes per row, and load instruction q reads rows
  // RPI*q .. RPI*q+RPI-1 (LPR lanes per row, 16 bytes each) with the
  // non-temporal policy. The MFMA A layout (16 rows x 64 bytes per
  // instruction) would read half lines, which streams slower. The wave turns
  // a step into the A layout through its own LDS slab (one write and one
  // read per 16 bytes; no barrier, LDS operations of a wave run in order).
  constexpr int SBW = UPW * 64, LPR = SBW / 16, RPI = kWave / LPR, SPITCH = SBW + 16;
  uint8_t* slab = (uint8_t*)(red + 2 * NW * TILE) + (size_t)wid * ROWS * SPITCH;
  const int fl_row = lane / LPR, fl_byte = 16 * (lane % LPR);

  auto load_step = [&](int s, StepRegs<WFMT, RT, UPW, ZERO>& r) {
    const int t = t_begin + s / nk, c = s % nk;
    const int kw = kr0 + c * KC + wid * UPW * KU;  // this wave's first k of the step
    const uint8_t* stp = a.w + (size_t)t * ROWS * wrow + (size_t)kw * F::BPK_NUM / F::BPK_DEN + fl_byte;
#pragma unroll
    for (int q = 0; q < RT * UPW; ++q)
      r.w[q / UPW][q % UPW] = load_nt((const u32x4*)(stp + (size_t)(RPI * q + fl_row) * wrow));
    if constexpr (WFMT == ACORN_WFMT_W4) {
      const int g0 = kw / 128;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const size_t row = (size_t)t * ROWS + rt * 16 + 4 * lg + i;
          load_dwords(a.scale + row * G + g0, r.s[rt][i]);
          if constexpr (ZERO) load_dwords(a.zero + row * G + g0, r.z[rt][i]);
        }
    } else if constexpr (WFMT == ACORN_WFMT_W8) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
        load_dwords(a.scale + (size_t)t * ROWS + rt * 16 + 4 * lg, r.s[rt][0]);
    }
  };

  const u32x4 ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
  f32x4 x8[MT];  // int8: sum of x over this wave's k (all chunks), per column

  auto compute = [&](const StepRegs<WFMT, RT, UPW, ZERO>& r0, int c, f32x4 (&acc)[RT][MT]) {
    // line layout -> A layout: unit u of row tile rt is 16 rows x 64 bytes
    StepRegs<WFMT, RT, UPW, ZERO> r = r0;
#pragma unroll
    for (int q = 0; q < RT * UPW; ++q)
      *(u32x4*)(slab + (RPI * q + fl_row) * SPITCH + fl_byte) = r0.w[q / UPW][q % UPW];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int u = 0; u < UPW; ++u)
        r.w[rt][u] = *(const u32x4*)(slab + (rt * 16 + lr) * SPITCH + 64 * u + 16 * lg);
#pragma unroll
    for (int u = 0; u < UPW; ++u) {
      const int kl = c * KC + wid * UPW * KU + u * KU;  // workgroup-local k of unit u
      const int c0 = kl / 8 + (KU / 32) * lg;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        u32x4 bop[MPU];
#pragma unroll
        for (int j = 0; j < MPU; ++j) bop[j] = xs[((size_t)mt * CPR + c0 + j) * R + (lr & (R - 1))];
        if constexpr (WFMT == ACORN_WFMT_BF16) {
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) acc[rt][mt] = mfma(r.w[rt][u], bop[0], acc[rt][mt]);
        } else if constexpr (WFMT == ACORN_WFMT_W8) {
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) {
            const u32x4 q = r.w[rt][u];
            acc[rt][mt] = mfma(unpack_w8(q[0], q[1]), bop[0], acc[rt][mt]);
            acc[rt][mt] = mfma(unpack_w8(q[2], q[3]), bop[1], acc[rt][mt]);
          }
        } else {
          const float xg = xgs[((size_t)mt * GR + kl / 128) * 16 + lr];
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) {
            const u32x4 q = r.w[rt][u];
            f32x4 cc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < MPU; ++j) cc = mfma(unpack_w4(q[j]), bop[j], cc);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float s = half_at(r.s[rt][i], u);
              float zc;
              if constexpr (ZERO) zc = half_at(r.z[rt][i], u) - 128.f * s;
              else zc = -136.f * s;
              acc[rt][mt][i] += s * cc[i] + zc * xg;
            }
          }
        }
      }
    }
  };

  const size_t plane = (size_t)a.M * a.N;
  auto out_index = [&](int t, int e, int& m, int& n) {
    const int ln = e % kWave, i = (e / kWave) % 4, rm = e / (4 * kWave);
    const int rt = rm / MT, mt = rm % MT;
    n = t * ROWS + rt * 16 + 4 * (ln / 16) + i;
    m = mblk + mt * 16 + (ln % 16);
  };

  int rbuf = 0;
  auto finish_tile = [&](int t, const StepRegs<WFMT, RT, UPW, ZERO>& r, f32x4 (&acc)[RT][MT]) {
    if constexpr (WFMT == ACORN_WFMT_W8) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float s = half_at(r.s[rt][0], i);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) acc[rt][mt][i] = s * (acc[rt][mt][i] - 128.f * x8[mt][i]);
        }
    }
    float* rb = red + (size_t)rbuf * NW * TILE;
    rbuf ^= 1;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          rb[(size_t)wid * TILE + ((rt * MT + mt) * 4 + i) * kWave + lane] = acc[rt][mt][i];
          acc[rt][mt][i] = 0.f;
        }
    __syncthreads();
    if constexpr (SWIGLU) {
      constexpr int HALF = TILE / 2;  // rt = 0 (gate) entries; rt = 1 (up) follow
      const int NA = a.N / 2;
      for (int e = threadIdx.x; e < HALF; e += NT) {
        float gv = rb[e], uv = rb[e + HALF];
#pragma unroll
        for (int ww = 1; ww < NW; ++ww) {
          gv += rb[(size_t)ww * TILE + e];
          uv += rb[(size_t)ww * TILE + e + HALF];
        }
        const int ln = e % kWave, i = (e / kWave) % 4, mt = e / (4 * kWave);
        const int m = mblk + mt * 16 + (ln % 16);
        const int n = t * 16 + 4 * (ln / 16) + i;
        if (m < a.M) a.out[(size_t)m * NA + n] = (__bf16)swiglu_bf16(gv, uv);
      }
      return;
    }
    const bool direct = a.ksplit == 1 && a.out != nullptr;
    for (int e = threadIdx.x; e < TILE; e += NT) {
      float v = rb[e];
#pragma unroll
      for (int ww = 1; ww < NW; ++ww) v += rb[(size_t)ww * TILE + e];
      int m, n;
      out_index(t, e, m, n);
      if (m >= a.M) continue;
      if (direct)
        a.out[(size_t)m * a.N + n] = (__bf16)v;
      else
        a.part[(size_t)blockIdx.y * plane + (size_t)m * a.N + n] = v;
    }
  };

  const int nsteps = (t_end - t_begin) * nk;

  // ---- loads: the first x batch, then the first D steps' weights ----------
  // x for the whole K range is staged into LDS in MFMA-B order (int4: the
  // unpack_w4 k-permutation). The first XB pieces per thread are loaded
  // before any weight so that waiting for them leaves the weights in flight;
  // indices past the end are clamped (loads stay unconditional, the stores
  // are skipped). Rows past M (padding up to R or the m tile) re-read row
  // M-1: their outputs are never written.
  constexpr int XB = 4;
  const int xtotal = MT * R * CPR;
  auto x_load = [&](int p) -> u32x4 {
    const int c = p % CPR, rr = p / CPR;  // rr = mt * R + row
    const int m = min(mblk + (rr / R) * 16 + rr % R, a.M - 1);
    return *(const u32x4*)(a.x + (size_t)m * a.K + kr0 + c * 8);
  };
  auto x_store = [&](int p, u32x4 w) {
    const int c = p % CPR, rr = p / CPR;
    const int mt = rr / R, row = rr % R;
    if constexpr (WFMT == ACORN_WFMT_W4) w = w4_order_x(w);
    xs[((size_t)mt * CPR + c) * R + row] = w;
  };
  u32x4 xv[XB];
#pragma unroll
  for (int u = 0; u < XB; ++u) xv[u] = x_load(min((int)threadIdx.x + u * NT, xtotal - 1));

  // D steps in flight per wave, as many as the registers allow without
  // spilling: bf16 steps are weights only (4 VGPRs per unit), so about 64
  // VGPRs of ring; int4/int8 steps also carry scales and the dequantised
  // operands, so they keep a shallower ring. A workgroup with nsteps <= D
  // has every weight of its work requested here, before x is stored.
  constexpr int kUnits = RT * UPW * MT;
  constexpr int D = WFMT == ACORN_WFMT_BF16
                        ? (kUnits <= 2 ? 8 : kUnits <= 4 ? 4 : kUnits <= 8 ? 2 : 1)
                        : (RT * UPW <= 2 ? 4 : RT * UPW <= 8 ? 2 : 1);
  StepRegs<WFMT, RT, UPW, ZERO> ring[D];
  load_step(0, ring[0]);
#pragma unroll
  for (int d = 1; d < D; ++d)
    if (d < nsteps) load_step(d, ring[d]);

#pragma unroll
  for (int u = 0; u < XB; ++u) {
    const int p = (int)threadIdx.x + u * NT;
    if (p < xtotal) x_store(p, xv[u]);
  }
  for (int p0 = (int)threadIdx.x + NT * XB; p0 < xtotal; p0 += NT * XB) {
#pragma unroll
    for (int u = 0; u < XB; ++u) xv[u] = x_load(min(p0 + u * NT, xtotal - 1));
#pragma unroll
    for (int u = 0; u < XB; ++u)
      if (p0 + u * NT < xtotal) x_store(p0 + u * NT, xv[u]);
  }
  __syncthreads();
  // ---- per-workgroup x sums (tile independent) -----------------------------
  if constexpr (WFMT == ACORN_WFMT_W4) {
    for (int g = wid; g < GR; g += NW) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        f32x4 xg = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < MPU; ++j)
          xg = mfma(ones, xs[((size_t)mt * CPR + g * 16 + 4 * lg + j) * R + (lr & (R - 1))], xg);
        if (lg == 0) xgs[((size_t)mt * GR + g) * 16 + lr] = xg[0];
      }
    }
    __syncthreads();
  } else if constexpr (WFMT == ACORN_WFMT_W8) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) x8[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int c = 0; c < nk; ++c)
#pragma unroll
      for (int u = 0; u < UPW; ++u) {
        const int c0 = (c * KC + wid * UPW * KU + u * KU) / 8 + 2 * lg;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            x8[mt] = mfma(ones, xs[((size_t)mt * CPR + c0 + j) * R + (lr & (R - 1))], x8[mt]);
      }
  }

  // ---- main pipeline --------------------------------------------------------
  f32x4 acc[RT][MT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[rt][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto step = [&](int s, const StepRegs<WFMT, RT, UPW, ZERO>& r) {
    compute(r, s % nk, acc);
    if (s % nk == nk - 1) finish_tile(t_begin + s / nk, r, acc);
  };
  if (nsteps <= D) {
#pragma unroll
    for (int d = 0; d < D; ++d)
      if (d < nsteps) step(d, ring[d]);
  } else {
    // ring refill: step s + D goes into the slot step s leaves; refills past
    // the end re-request the last step (unconditional loads keep the wait
    // counts static)
    for (int s0 = 0; s0 < nsteps; s0 += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        if (s0 + d < nsteps) step(s0 + d, ring[d]);
        load_step(min(s0 + d + D, nsteps - 1), ring[d]);
      }
    }
  }
}

// fp32 weights and activations (the fp32 parity path; not a performance
// path). One wavefront per weight row; lanes stride K and the M dot products
// are finished with a wavefront reduction. Writes fp32 y[m, n] into
// part[blockIdx.y, m, n] for the K range of split blockIdx.y.
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
    float acc = 0.f;
    for (int k = k0 + lane; k < k1; k += kWave) acc += xr[k] * wr[k];
    acc = wave_sum(acc);
    if (lane == 0) part[(size_t)blockIdx.y * M * N + (size_t)m * N + n] = acc;
  }
}

// ---------------------------------------------------------------------------
// Tiled form for M > 16, where the product is a dense contraction rather
// than a weight stream:
//  * a workgroup of 4 waves owns a BN (N) x BM (M) output tile and one K
//    range (a split; the block id is remapped so that the M blocks of one
//    weight tile run on one XCD); each wave a BN/2 x BM/2 quarter (2 x 2
//    waves). A K step is BK = 8192 / BN wide (BN 128: 64, BN 64: 128), so a
//    thread always loads 32 consecutive k of one weight row per step;
//  * per K step the weights are dequantised once into LDS as bf16
//    and x is staged beside them, both double-buffered with one barrier per
//    step; the global loads of the next DP steps are in flight (a ring of DP
//    register stages) while the MFMAs run. DP divides the step count, so
//    the loop has no data-dependent branch and the wait counts are static;
//    prefetches past the last step re-read it.
//    LDS rows are padded by 8 bf16 so the 16 rows of an MFMA operand fetch
//    spread over the banks;
//  * dequantisation: int8 -> bf16(q) exactly, the channel scale applied to
//    the fp32 result; int4 -> bf16(u * s + z) per 128-group (z = -8 s for
//    the symmetric form), one rounding per weight, as a dequantise-then-dot
//    kernel does; bf16 as is;
//  * v_mfma_f32_16x16x32_bf16 with W as A (rows n) and x as B (columns m);
//  * output as in the streaming form: bf16 when ksplit == 1, else fp32
//    partials [ksplit, M, N].
constexpr int kTileKN = 8192;                          // BN * BK

// Occupancy: the LDS tiles allow two or three workgroups per CU, so the
// register budget is that of two waves per SIMD (without the bound the
// compiler assumes more and spills the accumulators' neighbours into AGPRs).
template <int WFMT, int BM, int BN, int DP>
__global__ __launch_bounds__(256, 2) void wgemm_tile_kernel(KArgs a) {
  constexpr int BK = kTileKN / BN, KP = BK + 8;       // K step, LDS row pitch (bf16)
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int MB = WM / 16, NB = WN / 16;          // 16x16 blocks per wave
  constexpr int CPR = BK / 8;                         // 16-byte x chunks per row per step
  constexpr int XR = BM * CPR / 256;                  // 16-byte x loads per thread per step
  constexpr int TPR = 256 / BN;                       // threads per weight row
  constexpr int WR = kIsW4<WFMT> ? 1 : kIsW8<WFMT> ? 2 : 4;
  static_assert(XR >= 1 && MB >= 1 && NB >= 1 && BK / TPR == 32, "unsupported tile");
  extern __shared__ __align__(16) unsigned char smem[];
  __bf16* xs = (__bf16*)smem;                         // [2][BM][KP]
  __bf16* wsm = xs + 2 * BM * KP;                     // [2][BN][KP]
  _Float16* gsl = (_Float16*)(wsm + 2 * BN * KP);     // int4: [BN][G] scales, then zeros

  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63;
  const int r = lane >> 4, c = lane & 15;
  // XCD-aware order: workgroups are dealt to the 8 XCDs round-robin by
  // linear id, and each XCD has its own L2. The M blocks of one (N tile,
  // split) read the same weights, so they go to the same XCD at about the
  // same time: the first read comes from HBM, the others from that L2.
  int tile_n, split, mblk;
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
    tile_n = unit % ntl;
    split = unit / ntl;
  }
  const int n0 = tile_n * BN, m0 = mblk * BM;
  const int K = a.K;
  const int kper = K / a.ksplit, kb = split * kper, nsteps = kper / BK;
  const int wn = (wid & 1) * WN, wm = (wid >> 1) * WM;
  const int wrow = tid / TPR, wpart = tid % TPR;      // this thread's weight row / 32-k part
  constexpr int PPR = BK / 8, BROWS = 256 / PPR;      // bf16: 16-byte pieces per row, rows per load
  const int brow = tid / PPR, bpiece = tid % PPR;

  struct Stage {
    u32x4 x[XR], w[WR];
  };
  // int4: the tile's group scales (and zeros) for this K range, loaded once
  const int G = kper / 128;
  if constexpr (kIsW4<WFMT>) {
    // eight independent loads in flight per thread per round
    for (int i0 = 0; i0 < BN * G; i0 += 256 * 8) {
      _Float16 sv[8], zv[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int i = min(i0 + tid + 256 * u, BN * G - 1);
        const int n = n0 + i / G, g = kb / 128 + i % G;
        const size_t gi = WFMT == ACORN_WFMT_W4B ? w4b_half_index(n, g, K)
                                                 : (size_t)n * (K / 128) + g;
        sv[u] = a.scale[gi];
        zv[u] = a.zero ? a.zero[gi] : (_Float16)0.f;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int i = i0 + tid + 256 * u;
        if (i < BN * G) {
          gsl[i] = sv[u];
          gsl[BN * G + i] = zv[u];
        }
      }
    }
    __syncthreads();
  }
  auto gload = [&](int s, Stage& st) {
    const int k0 = kb + min(s, nsteps - 1) * BK;
    u32x4 (&xr)[XR] = st.x;
    u32x4 (&wr)[WR] = st.w;
#pragma unroll
    for (int j = 0; j < XR; ++j) {
      // rows past M re-read row M-1 (no branch, so the wait counts stay
      // static); their outputs are never stored
      const int q = tid + 256 * j, row = q / CPR, ch = q % CPR, m = min(m0 + row, a.M - 1);
      xr[j] = *(const u32x4*)(a.x + (size_t)m * K + k0 + 8 * ch);
    }
    const size_t wk = (size_t)(n0 + wrow) * K + k0 + 32 * wpart;   // weight element index
    if constexpr (WFMT == ACORN_WFMT_W4B) {
      // the same 16 bytes (row n, 32-k chunk c) in the 1 KB block layout
      wr[0] = *(const u32x4*)(a.w + w4b_chunk_offset(n0 + wrow, (k0 + 32 * wpart) / 32, K));
    } else if constexpr (WFMT == ACORN_WFMT_W4) {
      wr[0] = *(const u32x4*)(a.w + wk / 2);
    } else if constexpr (WFMT == ACORN_WFMT_W8B) {
      // the same 16-byte pieces (row n, 16-k chunk c) in the 1 KB block layout
#pragma unroll
      for (int j = 0; j < WR; ++j)
        wr[j] = *(const u32x4*)(a.w + w8b_chunk_offset(n0 + wrow, (k0 + 32 * wpart) / 16 + j, K));
    } else if constexpr (WFMT == ACORN_WFMT_W8) {
#pragma unroll
      for (int j = 0; j < WR; ++j) wr[j] = *(const u32x4*)(a.w + wk + 16 * j);
    } else if constexpr (WFMT == ACORN_WFMT_BF16B) {
      // the same pieces in the 1 KB block layout: an instruction covers
      // BROWS rows x BK k, whole blocks, so again whole cache lines
#pragma unroll
      for (int j = 0; j < WR; ++j)
        wr[j] = load_nt((const u32x4*)(a.w + bf16b_piece_offset(n0 + brow + BROWS * j, k0 / 8 + bpiece, K)));
    } else {
      // bf16: instruction j reads whole 16-byte pieces of rows BROWS*j + t/PPR,
      // consecutive threads consecutive pieces, so each instruction consumes
      // whole cache lines and can use the non-temporal policy
#pragma unroll
      for (int j = 0; j < WR; ++j)
        wr[j] = load_nt((const u32x4*)(a.w + 2 * ((size_t)(n0 + brow + BROWS * j) * K + k0 + 8 * bpiece)));
    }
  };
  auto lstore = [&](int s, const Stage& st) {
    const u32x4 (&xr)[XR] = st.x;
    const u32x4 (&wr)[WR] = st.w;
    __bf16* xd = xs + (s & 1) * BM * KP;
#pragma unroll
    for (int j = 0; j < XR; ++j) {
      const int q = tid + 256 * j, row = q / CPR, ch = q % CPR;
      *(u32x4*)(xd + row * KP + 8 * ch) = xr[j];
    }
    __bf16* wd = wsm + (s & 1) * BN * KP + wrow * KP + 32 * wpart;
    if constexpr (kIsW4<WFMT>) {
      const int g = (min(s, nsteps - 1) * BK + 32 * wpart) / 128;
      const float gs = (float)gsl[wrow * G + g];
      const float gz = a.zero ? (float)gsl[BN * G + wrow * G + g] : -8.f * gs;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        // nibbles k = 8d .. 8d+7 (low nibble = even k) -> bf16(u * s + z)
        const uint32_t w = wr[0][d];
        uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
        // opaque to the optimiser: otherwise it folds the masks into a
        // bit-field extract per nibble ahead of each v_cvt_f32_ubyteN
        asm volatile("" : "+v"(lo), "+v"(hi));
        u32x4 o;
        if constexpr (WFMT == ACORN_WFMT_W4B) {
          // W4B nibble order: lo's bytes are k offsets 0, 4, 1, 5 and hi's 2, 6, 3, 7
          o[0] = pack_bf16x2(ubyte_f32<0>(lo) * gs + gz, ubyte_f32<2>(lo) * gs + gz);
          o[1] = pack_bf16x2(ubyte_f32<0>(hi) * gs + gz, ubyte_f32<2>(hi) * gs + gz);
          o[2] = pack_bf16x2(ubyte_f32<1>(lo) * gs + gz, ubyte_f32<3>(lo) * gs + gz);
          o[3] = pack_bf16x2(ubyte_f32<1>(hi) * gs + gz, ubyte_f32<3>(hi) * gs + gz);
        } else {
          o[0] = pack_bf16x2(ubyte_f32<0>(lo) * gs + gz, ubyte_f32<0>(hi) * gs + gz);
          o[1] = pack_bf16x2(ubyte_f32<1>(lo) * gs + gz, ubyte_f32<1>(hi) * gs + gz);
          o[2] = pack_bf16x2(ubyte_f32<2>(lo) * gs + gz, ubyte_f32<2>(hi) * gs + gz);
          o[3] = pack_bf16x2(ubyte_f32<3>(lo) * gs + gz, ubyte_f32<3>(hi) * gs + gz);
        }
        *(u32x4*)(wd + 8 * d) = o;
      }
    } else if constexpr (kIsW8<WFMT>) {
#pragma unroll
      for (int j = 0; j < WR; ++j) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          // 8 signed bytes -> bf16(q), exact; ^0x80 (W8B stores q + 128
          // already) then -128 keeps the conversion on v_cvt_f32_ubyteN
          constexpr uint32_t kFlip = WFMT == ACORN_WFMT_W8B ? 0u : 0x80808080u;
          const uint32_t lo = wr[j][2 * h] ^ kFlip, hi = wr[j][2 * h + 1] ^ kFlip;
          u32x4 o;
          o[0] = pack_bf16x2(ubyte_f32<0>(lo) - 128.f, ubyte_f32<1>(lo) - 128.f);
          o[1] = pack_bf16x2(ubyte_f32<2>(lo) - 128.f, ubyte_f32<3>(lo) - 128.f);
          o[2] = pack_bf16x2(ubyte_f32<0>(hi) - 128.f, ubyte_f32<1>(hi) - 128.f);
          o[3] = pack_bf16x2(ubyte_f32<2>(hi) - 128.f, ubyte_f32<3>(hi) - 128.f);
          *(u32x4*)(wd + 16 * j + 8 * h) = o;
        }
      }
    } else {
      __bf16* wb = wsm + (s & 1) * BN * KP + brow * KP + 8 * bpiece;
#pragma unroll
      for (int j = 0; j < WR; ++j) *(u32x4*)(wb + BROWS * j * KP) = wr[j];
    }
  };

  f32x4 acc[NB][MB];
#pragma unroll
  for (int i = 0; i < NB; ++i)
#pragma unroll
    for (int j = 0; j < MB; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int s) {
    const __bf16* xd = xs + (s & 1) * BM * KP;
    const __bf16* wd = wsm + (s & 1) * BN * KP;
#pragma unroll
    for (int kk = 0; kk < BK; kk += 32) {
      u32x4 af[NB], bfr[MB];
#pragma unroll
      for (int i = 0; i < NB; ++i) af[i] = *(const u32x4*)(wd + (wn + 16 * i + c) * KP + kk + 8 * r);
#pragma unroll
      for (int j = 0; j < MB; ++j) bfr[j] = *(const u32x4*)(xd + (wm + 16 * j + c) * KP + kk + 8 * r);
#pragma unroll
      for (int i = 0; i < NB; ++i)
#pragma unroll
        for (int j = 0; j < MB; ++j) acc[i][j] = mfma(af[i], bfr[j], acc[i][j]);
    }
  };

  // step t's registers live in ring[t % DP]
  Stage ring[DP];
#pragma unroll
  for (int d = 0; d < DP; ++d) gload(d, ring[d]);
  lstore(0, ring[0]);
  __syncthreads();
  for (int s0 = 0; s0 < nsteps; s0 += DP) {
#pragma unroll
    for (int d = 0; d < DP; ++d) {
      const int s = s0 + d;
      if constexpr (DP > 1) gload(s + DP, ring[d]);   // ring[d] went to LDS last step
      compute(s);
      if constexpr (DP == 1) gload(s + 1, ring[0]);
      lstore(s + 1, ring[(d + 1) % DP]);              // harmless past the end
      __syncthreads();
    }
  }

  // ---- epilogue ----
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int n = n0 + wn + 16 * i + 4 * r;
    float sc[4] = {1.f, 1.f, 1.f, 1.f};
    if constexpr (kIsW8<WFMT>) {
#pragma unroll
      for (int e = 0; e < 4; ++e) sc[e] = (float)a.scale[n + e];
    }
#pragma unroll
    for (int j = 0; j < MB; ++j) {
      const int m = m0 + wm + 16 * j + c;
      if (m >= a.M) continue;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = sc[e] * acc[i][j][e];
      if (a.out) {
        uint32_t p[2] = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
        __builtin_memcpy(a.out + (size_t)m * a.N + n, p, sizeof(p));
      } else {
        float* dst = a.part + ((size_t)split * a.M + m) * a.N + n;
        *(f32x4*)dst = f32x4{v[0], v[1], v[2], v[3]};
      }
    }
  }
}

size_t tile_lds_bytes(int wfmt, int bm, int bn, int64_t kper) {
  const int kp = kTileKN / bn + 8;
  size_t b = (size_t)2 * (bm + bn) * kp * 2;
  if (wfmt == ACORN_WFMT_W4 || wfmt == ACORN_WFMT_W4B)
    b += (size_t)2 * bn * (kper / 128) * 2;  // scales + zeros
  return b;
}

// Split-K reduction (fixed order) with the output cast.
template <typename T>
__global__ void splitk_reduce_kernel(const float* __restrict__ part, int nsplit, size_t count,
                                     T* __restrict__ out) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= count) return;
  float acc = part[i];
  for (int s = 1; s < nsplit; ++s) acc += part[(size_t)s * count + i];
  out[i] = (T)acc;
}

// ----------------------------------------------------------------- planning --

struct Tiling {
  int rt, upw, nw, ksplit, tpw;  // the tunable knobs (acorn_gemm_plan's cfg[0..4])
  int mt, R, nk, ntiles, mblocks, groups;
  size_t lds;
  int swiglu;                    // fused SwiGLU epilogue (rt == 2, ksplit == 1)
  int kind;                      // 0 = streaming kernel, 1 = tiled kernel (rt == 0, upw = BM),
                                 // 2 = W4B decode kernel (tpw = its pipeline depth),
                                 // 3 = large-M bf16 kernel (rt == kDenseRT, upw = BM,
                                 //     nw = weight rows per wave, tpw = prefetch depth),
                                 // 4 = W4B mid-M kernel (rt == kMidRT, upw = row tiles
                                 //     per wave, nw = waves, tpw = groups in flight),
                                 // 5 = W8B decode kernel (tpw = its pipeline depth),
                                 // 6 = BF16B decode kernel (tpw = its pipeline depth),
                                 // 7 = W8B mid-M kernel (as 4, tpw = steps in flight)
  W4bPlan w4b;
  DirectPlan w8b;
  DirectPlan bf16b;
  W4mPlan w4m;
  W8mPlan w8m;
};

int ilog2_ceil(int v) {
  int r = 0;
  while ((1 << r) < v) ++r;
  return r;
}

int ku_of(int wfmt) {
  return wfmt == ACORN_WFMT_BF16 ? 32 : wfmt == ACORN_WFMT_W8 ? 64 : 128;
}

bool supported(int rt, int mt, int upw, int nw) {
  const bool shape = (mt == 1 && (rt == 1 || rt == 2 || rt == 4)) || (rt == 1 && (mt == 2 || mt == 4));
  const bool u = upw == 2 || upw == 4 || upw == 8 || upw == 16;
  const bool w = nw == 1 || nw == 2 || nw == 4 || nw == 8;
  return shape && u && w && rt * upw <= 16 && (mt == 1 || upw <= 8) && (mt == 1 || nw <= 4);
}

constexpr int kCUs = 256;
constexpr int64_t kTargetWG = 4 * kCUs;  // default workgroups per launch

size_t lds_bytes(int wfmt, int mt, int R, int rt, int nw, int KR, int upw) {
  size_t b = (size_t)mt * R * KR * 2;
  if (wfmt == ACORN_WFMT_W4) b += (size_t)mt * (KR / 128) * 16 * 4;
  b += (size_t)2 * nw * rt * mt * 4 * kWave * 4;
  b += (size_t)nw * 16 * rt * (upw * 64 + 16);  // per-wave line-to-A-layout slabs
  return b;
}

// Tiled kernel plan (M > 16). Request: BM in upw (32 / 64 / 128), BN in nw
// (64 / 128), 0 = choose (BN 64 for M <= 64, else 128; BM from M). The K
// split keeps every split on whole K steps (int4: whole 128-k groups). By
// default it grows until about two workgroups per CU are launched, while each
// split keeps at least 256 k and, for M <= 64 (weight-bound), the fp32
// partials (written and read again, 8*ksplit*M*N bytes) stay below half the
// weight bytes.
int make_tile_plan(int64_t M, int64_t N, int64_t K, int wfmt, int req_bm, int req_bn,
                   int req_ks, Tiling* t) {
  const int bn = (req_bn == 64 || req_bn == 128) ? req_bn : M <= 64 ? 64 : 128;
  if (N % bn) return ACORN_ERR_UNSUPPORTED;
  const int bk = kTileKN / bn;
  const int align = (wfmt == ACORN_WFMT_W4 || wfmt == ACORN_WFMT_W4B) ? std::max(128, bk) : bk;
  if (wfmt == ACORN_WFMT_W4B && (K % 512 || N % 16)) return ACORN_ERR_SHAPE;
  if ((wfmt == ACORN_WFMT_W8B || wfmt == ACORN_WFMT_BF16B) && (K % 64 || N % 16))
    return ACORN_ERR_SHAPE;
  if (K % align) return ACORN_ERR_SHAPE;
  const int bm = (req_bm == 32 || req_bm == 64 || req_bm == 128) ? req_bm
                 : M <= 32 ? 32 : M <= 64 ? 64 : 128;
  const int64_t units = K / align;
  t->kind = 1;
  t->rt = 0;
  t->upw = bm;
  t->nw = bn;
  t->tpw = 1;
  t->mt = 0;
  t->R = 0;
  t->swiglu = 0;
  t->ntiles = (int)(N / bn);
  t->mblocks = (int)((M + bm - 1) / bm);
  t->groups = t->ntiles;
  int64_t ks;
  if (req_ks > 0) {
    ks = req_ks;
    while (ks <= units && units % ks) ++ks;
    if (ks > units) return ACORN_ERR_UNSUPPORTED;
  } else {
    ks = 1;
    const int64_t tiles = (int64_t)t->ntiles * t->mblocks;
    const double wbytes = (double)N * K * ((wfmt == ACORN_WFMT_W4 || wfmt == ACORN_WFMT_W4B) ? 0.5
                                           : (wfmt == ACORN_WFMT_W8 || wfmt == ACORN_WFMT_W8B) ? 1
                                                                                            : 2);
    while (tiles * ks < 2 * kCUs) {
      int64_t nx = ks + 1;
      while (nx <= units && units % nx) ++nx;
      if (nx > units || K / nx < 256) break;
      // weight-bound sizes: the fp32 partials (written, then read by the
      // reduction) stay below half the weight bytes (beyond that they cost
      // more than the extra workgroups gain); MFMA-bound sizes need the
      // workgroups more than they mind the partials
      if (M <= 64 && 8.0 * nx * M * N > 0.5 * wbytes) break;
      ks = nx;
    }
  }
  t->ksplit = (int)ks;
  t->nk = (int)(K / ks / bk);
  t->lds = tile_lds_bytes(wfmt, bm, bn, K / ks);
  if (t->lds > 160 * 1024) return ACORN_ERR_UNSUPPORTED;
  if (t->ksplit > 65535 || t->mblocks > 65535 || t->ntiles > 0x7fffffff) return ACORN_ERR_SHAPE;
  return ACORN_OK;
}

// cfg: {rt, upw, nw, ksplit, tpw}; 0 = choose. swiglu: fused SwiGLU epilogue,
// which fixes rt = 2 and ksplit = 1. For M > 16 an rt of 0 selects the tiled
// kernel (upw = its BM), rt >= 1 the streaming kernel.
// bf16 at prefill sizes: the large-M kernel (dense_gemm.hip, its 256 x 256
// direct-to-LDS form) by default from kDenseMinM rows on, or on request
// (rt == kDenseRT); with the SwiGLU epilogue from kDenseLdsM rows. At 256 /
// 384 rows on the 8B shapes the 256 x 256 form took qkv 26.9 / 36.5 us,
// gate|up 62.4 / 110.2, down 37.3 / 48.6 against 35.4 / 45.8, 86.1 / 142.3,
// 44.6 / 77.5 on the tiled kernel; the fused SwiGLU (one split) does not pay
// below 512 rows.
constexpr int kDenseRT = -2;
constexpr int64_t kDenseMinM = 256;
constexpr int64_t kDenseLdsM = 512;
// W4B above 16 rows on request (rt == kMidRT): the mid-M int4 kernel
constexpr int kMidRT = -3;

int make_plan(int64_t M, int64_t N, int64_t K, int wfmt, const int* cfg, Tiling* t,
              bool swiglu = false) {
  if (M <= 0 || N <= 0 || K <= 0) return ACORN_ERR_SHAPE;
  // the block layouts exist only for whole blocks
  if ((wfmt == ACORN_WFMT_W8B || wfmt == ACORN_WFMT_BF16B) && (N % 16 || K % 64))
    return ACORN_ERR_SHAPE;
  if (wfmt == ACORN_WFMT_W4B && (N % 16 || K % 512)) return ACORN_ERR_SHAPE;
  t->swiglu = swiglu;
  t->kind = 0;
  const bool no_request = !cfg || (cfg[0] == 0 && cfg[1] == 0 && cfg[2] == 0 && cfg[3] <= 1 &&
                                   cfg[4] == 0);
  // the SwiGLU epilogue is built into the direct-to-LDS form only (from
  // kDenseLdsM rows, or on request)
  const bool blocked = wfmt == ACORN_WFMT_BF16B;
  if ((wfmt == ACORN_WFMT_BF16 || blocked) &&
      ((cfg && cfg[0] == kDenseRT) || (no_request && M >= (swiglu ? kDenseLdsM : kDenseMinM)))) {
    const bool req = cfg && cfg[0] == kDenseRT;
    // from kDenseMinM rows the 256 x 256 tiles with both operands in LDS
    const int bm = req && cfg[1] > 0 ? cfg[1] : M >= kDenseMinM ? 256 : 128;
    const int wn = req && cfg[2] > 0              ? cfg[2]
                   : bm == 256 && !(req && cfg[4] == 2) ? 128    // depth 2: the staged form
                                                        : 64;
    // (bm 256: wn 64 is the register-staged form, depth 2, natural weights
    // only; wn 128 the direct-to-LDS form, a 4-stage ring)
    const int depth = req && cfg[4] > 0 ? cfg[4] : bm == 256 ? (wn == 128 ? 4 : 2) : 4;
    const int ntile = bm == 256 ? 256 : 4 * wn;    // weight rows per workgroup
    int ks = req && cfg[3] > 0 ? cfg[3] : 1;
    if (!(req && cfg[3] > 0) && !swiglu) {
      // split K while the launch has fewer workgroups than CUs; the 256 x 256
      // form (one workgroup per CU) stops before a second round of workgroups:
      // at M = 512 / 2048 one round with fewer splits measured faster (qkv
      // 37 vs 49 us with 4 / 8 splits at 512 rows, 106 vs 115 us with 1 / 2 at
      // 2048) since every split adds an fp32 plane of traffic
      const int64_t tiles = ((N + ntile - 1) / ntile) * ((M + bm - 1) / bm);
      if (bm == 256) {
        while (tiles * 2 * ks <= kCUs && ks < 16 &&
               dense_gemm_supported(N, K, wn, bm, depth, 2 * ks, blocked))
          ks *= 2;
      } else {
        while (tiles * ks < kCUs && ks < 8 && dense_gemm_supported(N, K, wn, bm, depth, 2 * ks, blocked))
          ks *= 2;
      }
    }
    if (swiglu ? ks == 1 && dense_gemm_swiglu_supported(N, K, wn, bm, depth, blocked)
               : dense_gemm_supported(N, K, wn, bm, depth, ks, blocked)) {
      t->kind = 3;
      t->rt = kDenseRT;
      t->upw = bm;
      t->nw = wn;
      t->ksplit = ks;
      t->tpw = depth;
      t->mt = 1;
      t->R = bm;
      t->nk = (int)(K / 64);
      t->ntiles = (int)((N + ntile - 1) / ntile);
      t->mblocks = (int)((M + bm - 1) / bm);
      t->groups = 1;
      t->lds = 0;
      return ACORN_OK;
    }
    if (req) return ACORN_ERR_UNSUPPORTED;
  }
  if (cfg && cfg[0] == kDenseRT) return ACORN_ERR_UNSUPPORTED;
  if (cfg && cfg[0] == kMidRT) {
    if ((wfmt != ACORN_WFMT_W4B && wfmt != ACORN_WFMT_W8B) || swiglu || M <= 16)
      return ACORN_ERR_UNSUPPORTED;
    const bool w4 = wfmt == ACORN_WFMT_W4B;
    const int rc = w4 ? w4m_make_plan(M, N, K, cfg, &t->w4m) : w8m_make_plan(M, N, K, cfg, &t->w8m);
    if (rc) return rc;
    t->kind = w4 ? 4 : 7;
    t->rt = kMidRT;
    t->upw = w4 ? t->w4m.rt : t->w8m.rt;
    t->nw = w4 ? t->w4m.nw : t->w8m.nw;
    t->ksplit = w4 ? t->w4m.ksplit : t->w8m.ksplit;
    t->tpw = w4 ? t->w4m.depth : t->w8m.depth;
    t->mt = 1;
    t->R = 1;
    t->nk = 0;
    t->ntiles = w4 ? t->w4m.groups : t->w8m.groups;
    t->mblocks = w4 ? t->w4m.mblocks : t->w8m.mblocks;
    t->groups = t->ntiles;
    t->lds = w4 ? t->w4m.lds : t->w8m.lds;
    return ACORN_OK;
  }
  if (wfmt == ACORN_WFMT_W4B && ((M <= 16 && !(cfg && cfg[0] == 0 && cfg[1] >= 32)) ||
                                  (M <= 64 && cfg && cfg[0] > 0))) {
    // decode sizes in the block layout: the W4B decode kernel (up to 64 rows
    // of x on request)
    const int rc = w4b_make_plan(M, N, K, cfg, swiglu, &t->w4b);
    if (rc) return rc;
    t->kind = 2;
    t->rt = t->w4b.rt;
    t->upw = t->w4b.upw;
    t->nw = t->w4b.nw_field;
    t->ksplit = t->w4b.ksplit;
    t->tpw = t->w4b.depth;
    t->mt = 1;
    t->R = t->w4b.R;
    t->ntiles = (int)(N / 16);
    t->mblocks = 1;
    t->groups = t->w4b.groups;
    t->lds = t->w4b.lds;
    return ACORN_OK;
  }
  if (wfmt == ACORN_WFMT_W4B && (swiglu || (cfg && cfg[0] > 0)))
    return ACORN_ERR_UNSUPPORTED;  // M > 64 in the block layout: the tiled kernel only
  if (wfmt == ACORN_WFMT_W8B && M <= 16 && !(cfg && cfg[0] == 0 && cfg[1] >= 32)) {
    // decode sizes in the int8 block layout: the W8B decode kernel
    const int rc = w8b_make_plan(M, N, K, cfg, swiglu, &t->w8b);
    if (rc) return rc;
    t->kind = 5;
    t->rt = t->w8b.rt;
    t->upw = t->w8b.upw;
    t->nw = t->w8b.nw_field;
    t->ksplit = t->w8b.ksplit;
    t->tpw = t->w8b.depth;
    t->mt = 1;
    t->R = (int)M;
    t->ntiles = (int)(N / 16);
    t->mblocks = 1;
    t->groups = t->w8b.groups;
    t->lds = 0;
    return ACORN_OK;
  }
  if (wfmt == ACORN_WFMT_W8B && (swiglu || (cfg && cfg[0] > 0)))
    return ACORN_ERR_UNSUPPORTED;  // M > 16 in the block layout: the tiled kernel only
  if (blocked && M <= 16 && !(cfg && cfg[0] == 0 && cfg[1] >= 32)) {
    // decode sizes in the bf16 block layout: the BF16B decode kernel
    const int rc = bf16b_make_plan(M, N, K, cfg, swiglu, &t->bf16b);
    if (rc) return rc;
    t->kind = 6;
    t->rt = t->bf16b.rt;
    t->upw = t->bf16b.upw;
    t->nw = t->bf16b.nw_field;
    t->ksplit = t->bf16b.ksplit;
    t->tpw = t->bf16b.depth;
    t->mt = 1;
    t->R = (int)M;
    t->ntiles = (int)(N / 16);
    t->mblocks = 1;
    t->groups = t->bf16b.groups;
    t->lds = 0;
    return ACORN_OK;
  }
  if (blocked && (swiglu || (cfg && cfg[0] > 0)))
    return ACORN_ERR_UNSUPPORTED;  // bf16 blocks above 16 rows: the tiled or large-M kernel
  // the tiled kernel: the default for M > 16; for M <= 16 on request (rt 0
  // with an M tile of 32 or more in upw)
  if (!swiglu && ((M > 16 && (!cfg || cfg[0] <= 0)) || (cfg && cfg[0] == 0 && cfg[1] >= 32)))
    return make_tile_plan(M, N, K, wfmt, cfg ? cfg[1] : 0, cfg ? cfg[2] : 0, cfg ? cfg[3] : 0, t);
  if (swiglu && (M > 16 || N % 32)) return ACORN_ERR_UNSUPPORTED;
  const int ku = ku_of(wfmt);
  if (N % 16 || K % ku) return ACORN_ERR_SHAPE;
  if (wfmt == ACORN_WFMT_W4 && K % 128) return ACORN_ERR_SHAPE;
  const int req_rt = cfg ? cfg[0] : 0, req_upw = cfg ? cfg[1] : 0, req_nw = cfg ? cfg[2] : 0;
  const int req_ks = cfg ? cfg[3] : 0, req_tpw = cfg ? cfg[4] : 0;
  t->mt = M <= 16 ? 1 : M <= 32 ? 2 : 4;
  t->R = t->mt == 1 ? (1 << ilog2_ceil((int)M)) : 16;
  t->rt = swiglu ? 2 : req_rt > 0 ? req_rt : 1;
  if (t->mt > 1) t->rt = 1;
  while (t->rt > 1 && N % (16 * t->rt)) t->rt /= 2;
  t->upw = req_upw > 0 ? req_upw : (wfmt == ACORN_WFMT_W4 ? 4 : 8);
  t->nw = req_nw > 0 ? req_nw : 4;
  if (t->mt > 1) {
    t->upw = std::min(t->upw, 8);
    t->nw = std::min(t->nw, 4);
  }
  while (t->rt * t->upw > 16) t->upw /= 2;
  const int64_t G = K / 128;
  auto kc = [&]() { return (int64_t)t->nw * t->upw * ku; };
  auto fits = [&]() {
    return K % kc() == 0 && (wfmt != ACORN_WFMT_W4 || G % t->upw == 0);
  };
  while (!fits() && t->upw > 2) t->upw /= 2;
  while (!fits() && t->nw > 1) t->nw /= 2;
  if (!fits()) return ACORN_ERR_SHAPE;
  if (!supported(t->rt, t->mt, t->upw, t->nw)) return ACORN_ERR_UNSUPPORTED;
  // LDS budget per workgroup: two workgroups per CU for decode sizes, one
  // for larger M (which is MFMA-bound anyway).
  const size_t limit = t->mt == 1 ? 80 * 1024 : 160 * 1024;
  auto lds_for = [&](int64_t kr) { return lds_bytes(wfmt, t->mt, t->R, t->rt, t->nw, (int)kr, t->upw); };
  while (lds_for(kc()) > limit && t->nw > 1) t->nw /= 2;
  while (lds_for(kc()) > limit && t->upw > 2) t->upw /= 2;
  if (!fits() || lds_for(kc()) > 160 * 1024) return ACORN_ERR_UNSUPPORTED;
  int64_t chunks = K / kc();
  if (swiglu) {
    // the whole K range is staged: narrow the workgroup (fewer waves, then
    // shorter steps) until x, the reduction buffers and the slabs fit
    t->ksplit = 1;
    while (lds_for(K) > 160 * 1024 && t->nw > 1) t->nw /= 2;
    while (lds_for(K) > 160 * 1024 && t->upw > 2) t->upw /= 2;
    if (lds_for(K) > 160 * 1024 || !supported(t->rt, t->mt, t->upw, t->nw))
      return ACORN_ERR_UNSUPPORTED;
    chunks = K / kc();
  } else if (req_ks > 0) {
    // a requested split is raised to the next divisor of the chunk count
    // whose K range fits the LDS of one workgroup
    t->ksplit = req_ks;
    while (t->ksplit <= chunks && (chunks % t->ksplit || lds_for(K / t->ksplit) > 160 * 1024))
      ++t->ksplit;
    if (t->ksplit > chunks) return ACORN_ERR_UNSUPPORTED;
  } else {
    // default: about kTargetWG workgroups of one tile each, splitting K as
    // far as needed to reach that count (and to fit the LDS budget)
    t->ksplit = 1;
    while (chunks % t->ksplit || lds_for(K / t->ksplit) > limit) ++t->ksplit;
    const int64_t ntl = N / (16 * t->rt);
    while (ntl * t->ksplit < kTargetWG) {
      int64_t nx = t->ksplit + 1;
      while (nx <= chunks && chunks % nx) ++nx;
      if (nx > chunks) break;
      t->ksplit = (int)nx;
    }
  }
  t->nk = (int)(chunks / t->ksplit);
  t->ntiles = (int)(N / (16 * t->rt));
  t->mblocks = (int)((M + 16 * t->mt - 1) / (16 * t->mt));
  if (req_tpw > 0) {
    t->tpw = req_tpw;
  } else {
    const int64_t groups = std::max<int64_t>(1, kTargetWG / ((int64_t)t->ksplit * t->mblocks));
    t->tpw = (int)std::max<int64_t>(1, (t->ntiles + groups - 1) / groups);
  }
  t->groups = (t->ntiles + t->tpw - 1) / t->tpw;
  t->lds = lds_bytes(wfmt, t->mt, t->R, t->rt, t->nw, (int)(K / t->ksplit), t->upw);
  if (t->lds > 160 * 1024) return ACORN_ERR_UNSUPPORTED;
  if (t->groups > 0x7fffffff || t->ksplit > 65535 || t->mblocks > 65535) return ACORN_ERR_SHAPE;
  return ACORN_OK;
}

template <int WFMT, int RT, int MT, int UPW, int NW>
void launch_one(const Tiling& t, const KArgs& a, hipStream_t st) {
  auto kfn = wgemm_kernel<WFMT, RT, MT, UPW, NW, false, false>;
  int variant = 0;
  if constexpr (RT == 2) {
    if (t.swiglu) {
      kfn = wgemm_kernel<WFMT, RT, MT, UPW, NW, true, false>;
      variant = 1;
    }
  }
  if constexpr (WFMT == ACORN_WFMT_W4) {
    if (a.zero) {
      kfn = wgemm_kernel<WFMT, RT, MT, UPW, NW, false, true>;
      variant = 2;
      if constexpr (RT == 2) {
        if (t.swiglu) {
          kfn = wgemm_kernel<WFMT, RT, MT, UPW, NW, true, true>;
          variant = 3;
        }
      }
    }
  }
  static bool lds_raised[4] = {false, false, false, false};  // once per kernel, before any capture
  if (!lds_raised[variant] && t.lds > 64 * 1024) {
    (void)hipFuncSetAttribute((const void*)kfn, hipFuncAttributeMaxDynamicSharedMemorySize,
                              160 * 1024);
    lds_raised[variant] = true;
  }
  dim3 grid((unsigned)t.groups, (unsigned)t.ksplit, (unsigned)t.mblocks), block(NW * kWave);
  kfn<<<grid, block, t.lds, st>>>(a);
}

template <int WFMT, int RT, int MT, int UPW>
int dispatch_nw(const Tiling& t, const KArgs& a, hipStream_t st) {
  switch (t.nw) {
    case 1: launch_one<WFMT, RT, MT, UPW, 1>(t, a, st); return ACORN_OK;
    case 2: launch_one<WFMT, RT, MT, UPW, 2>(t, a, st); return ACORN_OK;
    case 4: launch_one<WFMT, RT, MT, UPW, 4>(t, a, st); return ACORN_OK;
    case 8:
      if constexpr (MT == 1) {
        launch_one<WFMT, RT, MT, UPW, 8>(t, a, st);
        return ACORN_OK;
      }
  }
  return ACORN_ERR_UNSUPPORTED;
}

template <int WFMT, int RT, int MT>
int dispatch_upw(const Tiling& t, const KArgs& a, hipStream_t st) {
  switch (t.upw) {
    case 2: return dispatch_nw<WFMT, RT, MT, 2>(t, a, st);
    case 4: return dispatch_nw<WFMT, RT, MT, 4>(t, a, st);
    case 8:
      if constexpr (RT <= 2) return dispatch_nw<WFMT, RT, MT, 8>(t, a, st);
      break;
    case 16:
      if constexpr (RT == 1 && MT == 1) return dispatch_nw<WFMT, RT, MT, 16>(t, a, st);
      break;
  }
  return ACORN_ERR_UNSUPPORTED;
}

template <int WFMT>
int dispatch_tile(const Tiling& t, const KArgs& a, hipStream_t st) {
  if (t.mt == 1) {
    switch (t.rt) {
      case 1: return dispatch_upw<WFMT, 1, 1>(t, a, st);
      case 2: return dispatch_upw<WFMT, 2, 1>(t, a, st);
      case 4: return dispatch_upw<WFMT, 4, 1>(t, a, st);
    }
  } else if (t.rt == 1) {
    if (t.mt == 2) return dispatch_upw<WFMT, 1, 2>(t, a, st);
    if (t.mt == 4) return dispatch_upw<WFMT, 1, 4>(t, a, st);
  }
  return ACORN_ERR_UNSUPPORTED;
}

template <int WFMT, int BM, int BN, int DP>
void launch_tiled(const Tiling& t, const KArgs& a, hipStream_t st) {
  auto kfn = wgemm_tile_kernel<WFMT, BM, BN, DP>;
  static bool lds_raised = false;  // once per instantiation, before any capture
  if (!lds_raised && t.lds > 64 * 1024) {
    (void)hipFuncSetAttribute((const void*)kfn, hipFuncAttributeMaxDynamicSharedMemorySize,
                              160 * 1024);
    lds_raised = true;
  }
  dim3 grid((unsigned)t.ntiles, (unsigned)t.ksplit, (unsigned)t.mblocks), block(256);
  kfn<<<grid, block, t.lds, st>>>(a);
}

// Prefetch depth: as deep as the registers allow for the tile (4 steps for
// BM <= 64, 2 for BM = 128), reduced until it divides the step count.
template <int WFMT, int BM, int BN>
void launch_tiled_dp(const Tiling& t, const KArgs& a, hipStream_t st) {
  const int steps = t.nk;
  if (BM <= 64 && steps % 4 == 0) launch_tiled<WFMT, BM, BN, 4>(t, a, st);
  else if (steps % 2 == 0) launch_tiled<WFMT, BM, BN, 2>(t, a, st);
  else launch_tiled<WFMT, BM, BN, 1>(t, a, st);
}

template <int WFMT, int BN>
int dispatch_tiled_bm(const Tiling& t, const KArgs& a, hipStream_t st) {
  switch (t.upw) {
    case 32: launch_tiled_dp<WFMT, 32, BN>(t, a, st); return ACORN_OK;
    case 64: launch_tiled_dp<WFMT, 64, BN>(t, a, st); return ACORN_OK;
    case 128: launch_tiled_dp<WFMT, 128, BN>(t, a, st); return ACORN_OK;
  }
  return ACORN_ERR_UNSUPPORTED;
}

template <int WFMT>
int dispatch_tiled(const Tiling& t, const KArgs& a, hipStream_t st) {
  switch (t.nw) {
    case 64: return dispatch_tiled_bm<WFMT, 64>(t, a, st);
    case 128: return dispatch_tiled_bm<WFMT, 128>(t, a, st);
  }
  return ACORN_ERR_UNSUPPORTED;
}

int plan_entry(int64_t M, int64_t N, int64_t K, int wfmt, int* cfg, bool swiglu) {
  if (!cfg) return ACORN_ERR_VALUE;
  if (wfmt != ACORN_WFMT_BF16 && wfmt != ACORN_WFMT_W8 && wfmt != ACORN_WFMT_W4 &&
      wfmt != ACORN_WFMT_W4B && wfmt != ACORN_WFMT_W8B && wfmt != ACORN_WFMT_BF16B)
    return ACORN_ERR_DTYPE;
  Tiling t;
  const int rc = make_plan(M, N, K, wfmt, cfg, &t, swiglu);
  if (rc) return rc;
  cfg[0] = t.rt;
  cfg[1] = t.upw;
  cfg[2] = t.nw;
  cfg[3] = t.ksplit;
  cfg[4] = t.tpw;
  cfg[5] = t.ntiles * t.mblocks;  // output tiles of the launch
  return ACORN_OK;
}

int gemm_entry(const void* x, const void* w, const void* scale, const void* zero,
               void* out_bf16, float* part, int64_t M, int64_t N, int64_t K, int wfmt,
               const int* cfg, bool swiglu, hipStream_t st, const NormIn* ni = nullptr,
               const ResidOut* ro = nullptr) {
  if (!x || !w || (wfmt != ACORN_WFMT_BF16 && wfmt != ACORN_WFMT_BF16B && !scale))
    return ACORN_ERR_VALUE;
  if (!out_bf16 && !part && !ro) return ACORN_ERR_VALUE;
  if (M > 65535 * 64 || N > ((int64_t)1 << 30) || K > ((int64_t)1 << 30)) return ACORN_ERR_SHAPE;
  Tiling t;
  int rc = make_plan(M, N, K, wfmt, cfg, &t, swiglu);
  if (rc) return rc;
  // the folded RMSNorm is built into the direct decode kernels only
  const int mode = ni ? 1 : ro ? 2 : 0;
  if (mode) {
    if (!(t.kind == 6 || t.kind == 5 || (t.kind == 2 && t.w4b.direct)))
      return ACORN_ERR_UNSUPPORTED;
    t.bf16b.mode = t.w8b.mode = t.w4b.mode = mode;
  }
  // ksplit > 1 with a bf16 output needs the partials workspace
  if (out_bf16 && t.ksplit > 1 && !part) return ACORN_ERR_VALUE;
  KArgs a;
  a.x = (const __bf16*)x;
  a.w = (const uint8_t*)w;
  a.scale = (const _Float16*)scale;
  a.zero = (const _Float16*)zero;
  a.out = t.ksplit == 1 ? (__bf16*)out_bf16 : nullptr;
  a.part = part;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.nk = t.nk;
  a.tpw = t.tpw;
  a.ksplit = t.ksplit;
  a.log2R = ilog2_ceil(t.R);
  if (t.kind == 3) {
    // bf16 straight into out (one split), else fp32 split planes into part
    const bool direct = out_bf16 && t.ksplit == 1;
    const bool blk = wfmt == ACORN_WFMT_BF16B;
    rc = t.swiglu ? dense_gemm_swiglu_launch(x, w, out_bf16, M, N, K, t.nw, t.upw, t.tpw, blk, st)
                  : dense_gemm_launch(x, w, direct ? out_bf16 : nullptr, direct ? nullptr : part,
                                      M, N, K, t.nw, t.upw, t.tpw, t.ksplit, blk, st);
  } else if (t.kind == 2) {
    rc = w4b_launch(t.w4b, x, w, scale, zero, t.ksplit == 1 ? out_bf16 : nullptr, part, M, N, K,
                    ni, ro, st);
  } else if (t.kind == 4) {
    if (zero) return ACORN_ERR_UNSUPPORTED;  // the block layout is the symmetric format
    rc = w4m_launch(t.w4m, x, w, scale, t.ksplit == 1 ? out_bf16 : nullptr, part, M, N, K, st);
  } else if (t.kind == 7) {
    rc = w8m_launch(t.w8m, x, w, scale, t.ksplit == 1 ? out_bf16 : nullptr, part, M, N, K, st);
  } else if (t.kind == 5) {
    rc = w8b_launch(t.w8b, x, w, scale, t.ksplit == 1 ? out_bf16 : nullptr, part, M, N, K, ni,
                    ro, st);
  } else if (t.kind == 6) {
    rc = bf16b_launch(t.bf16b, x, w, t.ksplit == 1 ? out_bf16 : nullptr, part, M, N, K, ni, ro,
                      st);
  } else if (t.kind == 1) {
    switch (wfmt) {
      case ACORN_WFMT_BF16: rc = dispatch_tiled<ACORN_WFMT_BF16>(t, a, st); break;
      case ACORN_WFMT_W8: rc = dispatch_tiled<ACORN_WFMT_W8>(t, a, st); break;
      case ACORN_WFMT_W4: rc = dispatch_tiled<ACORN_WFMT_W4>(t, a, st); break;
      case ACORN_WFMT_W4B: rc = dispatch_tiled<ACORN_WFMT_W4B>(t, a, st); break;
      case ACORN_WFMT_W8B: rc = dispatch_tiled<ACORN_WFMT_W8B>(t, a, st); break;
      case ACORN_WFMT_BF16B: rc = dispatch_tiled<ACORN_WFMT_BF16B>(t, a, st); break;
    }
  } else {
    switch (wfmt) {
      case ACORN_WFMT_BF16: rc = dispatch_tile<ACORN_WFMT_BF16>(t, a, st); break;
      case ACORN_WFMT_W8: rc = dispatch_tile<ACORN_WFMT_W8>(t, a, st); break;
      case ACORN_WFMT_W4: rc = dispatch_tile<ACORN_WFMT_W4>(t, a, st); break;
    }
  }
  if (rc) return rc;
  ACORN_LAUNCH_CHECK();
  if (out_bf16 && t.ksplit > 1) {
    const int64_t count = M * N;
    splitk_reduce_kernel<__bf16><<<(unsigned)((count + 255) / 256), 256, 0, st>>>(
        part, t.ksplit, (size_t)count, (__bf16*)out_bf16);
    ACORN_LAUNCH_CHECK();
  }
  return ACORN_OK;
}

}  // namespace

extern "C" int acorn_gemm_plan(int64_t M, int64_t N, int64_t K, int wfmt, int* cfg) {
  if (!cfg) return ACORN_ERR_VALUE;
  if (wfmt == ACORN_WFMT_F32) {
    cfg[0] = 1; cfg[1] = 1; cfg[2] = 4; cfg[3] = cfg[3] > 0 ? cfg[3] : 1; cfg[4] = 1; cfg[5] = 0;
    return ACORN_OK;
  }
  return plan_entry(M, N, K, wfmt, cfg, false);
}

extern "C" int acorn_gemm_swiglu_plan(int64_t M, int64_t N, int64_t K, int wfmt, int* cfg) {
  return plan_entry(M, N, K, wfmt, cfg, true);
}

extern "C" int acorn_quant_gemm(const void* x, const void* w, const void* scale,
                                const void* zero, void* out_bf16, float* part, int64_t M,
                                int64_t N, int64_t K, int wfmt, const int* cfg, void* stream) {
  if (wfmt != ACORN_WFMT_BF16 && wfmt != ACORN_WFMT_W8 && wfmt != ACORN_WFMT_W4 &&
      wfmt != ACORN_WFMT_W4B && wfmt != ACORN_WFMT_W8B && wfmt != ACORN_WFMT_BF16B &&
      wfmt != ACORN_WFMT_F32)
    return ACORN_ERR_DTYPE;
  if (M < 0 || N <= 0 || K <= 0) return ACORN_ERR_SHAPE;
  if (M == 0) return ACORN_OK;
  hipStream_t st = (hipStream_t)stream;
  if (wfmt == ACORN_WFMT_F32) {
    // fp32 output always goes through part ([ksplit, M, N]).
    if (!x || !w || !part) return ACORN_ERR_VALUE;
    if (M > 65535 || N > ((int64_t)1 << 30) || K > ((int64_t)1 << 30)) return ACORN_ERR_SHAPE;
    const int ks = cfg && cfg[3] > 0 ? cfg[3] : 1;
    const int64_t kper = (K + ks - 1) / ks;
    dim3 grid((unsigned)((N + 3) / 4), (unsigned)ks), block(256);
    f32_gemv_kernel<<<grid, block, 0, st>>>((const float*)x, (const float*)w, part, (int)M,
                                            (int)N, (int)K, (int)kper);
    ACORN_LAUNCH_CHECK();
    return ACORN_OK;
  }
  return gemm_entry(x, w, scale, zero, out_bf16, part, M, N, K, wfmt, cfg, false, st);
}

extern "C" int acorn_quant_gemm_swiglu(const void* x, const void* w, const void* scale,
                                       const void* zero, void* act, int64_t M, int64_t N,
                                       int64_t K, int wfmt, const int* cfg, void* stream) {
  if (wfmt != ACORN_WFMT_BF16 && wfmt != ACORN_WFMT_W8 && wfmt != ACORN_WFMT_W4 &&
      wfmt != ACORN_WFMT_W4B && wfmt != ACORN_WFMT_W8B && wfmt != ACORN_WFMT_BF16B)
    return ACORN_ERR_DTYPE;
  if (M < 0 || N <= 0 || K <= 0) return ACORN_ERR_SHAPE;
  if (M == 0) return ACORN_OK;
  if (!act) return ACORN_ERR_VALUE;
  return gemm_entry(x, w, scale, zero, act, nullptr, M, N, K, wfmt, cfg, true,
                    (hipStream_t)stream);
}

extern "C" int acorn_quant_gemm_norm(const void* x, const void* w, const void* scale,
                                     void* out_bf16, float* part, int64_t M, int64_t N,
                                     int64_t K, int wfmt, const int* cfg, int swiglu,
                                     const float* ss_in, float eps, const void* res,
                                     void* res_out, float* ss_out, const void* norm_w,
                                     void* xw_out, void* stream) {
  if (wfmt != ACORN_WFMT_BF16B && wfmt != ACORN_WFMT_W8B && wfmt != ACORN_WFMT_W4B)
    return ACORN_ERR_DTYPE;
  if (M < 0 || N <= 0 || K <= 0 || N % 16 || K % 16) return ACORN_ERR_SHAPE;
  if (M == 0) return ACORN_OK;
  const bool norm = ss_in != nullptr, resid = res != nullptr;
  if (norm == resid) return ACORN_ERR_VALUE;                 // exactly one of the two
  if (resid && swiglu) return ACORN_ERR_UNSUPPORTED;
  if (resid && (!res_out || !ss_out || !norm_w || !xw_out)) return ACORN_ERR_VALUE;
  if (swiglu && !out_bf16) return ACORN_ERR_VALUE;
  const NormIn ni{ss_in, (int)(K / 16), eps};
  const ResidOut ro{(const __bf16*)res, (__bf16*)res_out, ss_out, (const __bf16*)norm_w,
                    (__bf16*)xw_out};
  return gemm_entry(x, w, scale, nullptr, out_bf16, part, M, N, K, wfmt, cfg, swiglu != 0,
                    (hipStream_t)stream, norm ? &ni : nullptr, resid ? &ro : nullptr);
}

extern "C" int acorn_dequant_w4b(const void* w, const void* scale, void* out_bf16, int64_t N,
                                 int64_t K, void* stream) {
  return w4b_dequant(w, scale, out_bf16, N, K, (hipStream_t)stream);
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
