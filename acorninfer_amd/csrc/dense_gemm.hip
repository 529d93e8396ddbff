// Large-M bf16 projection GEMM (prefill sizes): out[M, N] = x[M, K] . w[N, K]^T
// with x and w both K-contiguous, fp32 accumulation, bf16 or fp32 output.
//
// Shape of the work, for gfx950's v_mfma_f32_16x16x32_bf16:
//  * a workgroup of 4 waves owns a (4 WN) (n) x BM (m) output tile; wave w
//    owns the WN weight rows [WN w, WN w + WN) of it and all BM columns, so a
//    wave holds WN/16 x BM/16 accumulator blocks;
//  * weights go from global memory straight into registers in the MFMA A
//    operand layout (lane (r, c) of a 16-row block holds 8 consecutive k of
//    row c at k = 8 r): each weight byte is read by exactly one wave, no LDS;
//  * x goes through LDS: the workgroup stages the BM x 64 slice of a K step
//    once and all 4 waves read their B operands from it (double-buffered,
//    one barrier per K step);
//  * weights are prefetched DEPTH K steps ahead in a register ring, x one
//    step ahead (scheduling fences keep the x loads at the top of the step
//    and its LDS store after the MFMAs); DEPTH divides the step count, so the
//    loop has no data-dependent branch and the wait counts are static; loads
//    past the last step re-read it;
//  * launches with fewer tiles than CUs split K (blockIdx.y): split s sums
//    its K range into its own fp32 plane, which the consumer adds in order;
//  * workgroup ids are remapped so that consecutive tiles run on one XCD
//    (the dispatcher deals ids round-robin over the 8 XCDs), and the tiles of
//    an XCD cover 4 weight tiles x 8 x tiles, which share its L2.
// Per 32 k a wave reads BM/16 B operands (1 KB each) from LDS for
// WN/16 x BM/16 MFMAs. With one wave per SIMD this form stays near 0.8-0.9
// PFLOP/s at M >= 2048 (reading the weights in whole lines through an LDS slab
// instead was slower: the loads are not its bound). Two 256 x 256 forms
// follow, both operands in LDS and two waves per SIMD: one stages through
// registers (1.0-1.06 PFLOP/s at M = 2048-8192), the other loads straight
// into LDS (global_load_lds) in whole 128-byte rows through two pair-of-stage
// buffers, the planner's default from 512 rows (1.11-1.33 PFLOP/s at
// M = 8192; hipBLASLt: 1.3-1.5).
#include <hip/hip_runtime.h>

#include "acorn_hip.h"
#include "gemm_common.h"

namespace acorn {
namespace {

constexpr int kDenseBK = 64;               // k per step
constexpr int kXPitch = kDenseBK * 2 + 16; // bytes per staged x row (padded by 8 bf16)

// BLK: w in the BF16B layout (1 KB blocks of 16 rows x 32 k in the A operand
// lane order), read at the same lanes' addresses.
template <typename OUT, int WN, int BM, int DEPTH, bool BLK>
__global__ __launch_bounds__(256, 1) void dense_gemm_kernel(const __bf16* __restrict__ x,
                                                            const __bf16* __restrict__ w,
                                                            OUT* __restrict__ out, int M, int N,
                                                            int K, int tiles_n, int tiles_m,
                                                            int steps) {
  constexpr int NB = WN / 16;                       // accumulator blocks along n (per wave)
  constexpr int MB = BM / 16;                       // accumulator blocks along m
  constexpr int XP = BM * kDenseBK / 8 / 256;       // 16-byte x pieces per thread per step
  __shared__ __align__(16) uint8_t xs[2][BM * kXPitch];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wid = tid >> 6;
  const int r = lane >> 4, c = lane & 15;
  // tile of this workgroup: XCD-contiguous ids, then groups of 4 weight tiles
  const int G = tiles_n * tiles_m;
  int t = blockIdx.x;
  if (G % 8 == 0) t = (t % 8) * (G / 8) + t / 8;
  constexpr int GN = 4;
  const int group = t / (GN * tiles_m);
  const int first_n = group * GN;
  const int gsize = min(tiles_n - first_n, GN);
  const int in_group = t - group * GN * tiles_m;
  const int tn = first_n + in_group % gsize;
  const int tm = in_group / gsize;
  const int n0 = tn * 4 * WN + wid * WN;
  const int m0 = tm * BM;
  // split blockIdx.y of the K range: `steps` K steps from k = blockIdx.y * steps * 64,
  // written to its own fp32 plane of out
  const int kbase = blockIdx.y * steps * kDenseBK;
  out += (size_t)blockIdx.y * M * N;

  // weight rows of the wave's NB blocks (rows past N re-read row N - 1; in
  // blocks, tiles past N re-read the last tile), and the element step per k
  constexpr int KSTR = BLK ? 16 : 1;
  const __bf16* wrow[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    if constexpr (BLK)
      wrow[nb] = w + ((size_t)min((n0 + 16 * nb) / 16, N / 16 - 1) * (K / 32) + kbase / 32) * 512 +
                 8 * lane;
    else
      wrow[nb] = w + (size_t)min(n0 + 16 * nb + c, N - 1) * K + kbase + 8 * r;
  }
  // the x pieces this thread stages: row p / 8, k (p % 8) * 8 of the step
  const __bf16* xrow[XP];
  uint32_t xoff[XP];
#pragma unroll
  for (int i = 0; i < XP; ++i) {
    const int p = tid + 256 * i;
    xrow[i] = x + (size_t)min(m0 + p / 8, M - 1) * K + kbase + (p % 8) * 8;
    xoff[i] = (uint32_t)((p / 8) * kXPitch + (p % 8) * 16);
  }
  u32x4 wr[DEPTH][NB][2];
  u32x4 xr[XP];
  auto load_w = [&](int s, u32x4 (&dst)[NB][2]) {
    const int k0 = s * kDenseBK;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) dst[nb][kk] = *(const u32x4*)(wrow[nb] + KSTR * (k0 + 32 * kk));
  };
  auto load_x = [&](int s) {
    const int k0 = s * kDenseBK;
#pragma unroll
    for (int i = 0; i < XP; ++i) xr[i] = *(const u32x4*)(xrow[i] + k0);
  };
  auto store_x = [&](int b) {
#pragma unroll
    for (int i = 0; i < XP; ++i) *(u32x4*)(xs[b] + xoff[i]) = xr[i];
  };
  f32x4 acc[NB][MB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int d = 0; d < DEPTH; ++d) load_w(min(d, steps - 1), wr[d]);
  load_x(0);
  store_x(0);
  __syncthreads();
  for (int s0 = 0; s0 < steps; s0 += DEPTH) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      const int s = s0 + d;
      const int b = s & 1;
      load_x(min(s + 1, steps - 1));
      // keep the x loads here, a whole step ahead of their LDS store (the
      // scheduler would sink them next to it and expose their latency)
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        u32x4 xb[MB];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
          xb[mb] = *(const u32x4*)(xs[b] + (16 * mb + c) * kXPitch + 64 * kk + 16 * r);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = mfma(wr[d][nb][kk], xb[mb], acc[nb][mb]);
      }
      // and the LDS store of the next step's x after this step's MFMAs
      __builtin_amdgcn_sched_barrier(0);
      load_w(min(s + DEPTH, steps - 1), wr[d]);
      store_x(b ^ 1);
      __syncthreads();
    }
  }
  // lane (r, c) of block (nb, mb) holds out[m0 + 16 mb + c][n0 + 16 nb + 4 r + i]
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int m = m0 + 16 * mb + c;
    if (m >= M) continue;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int n = n0 + 16 * nb + 4 * r;
      if (n >= N) continue;
      OUT* o = out + (size_t)m * N + n;
      if constexpr (sizeof(OUT) == 4) {
        *(f32x4*)o = acc[nb][mb];
      } else {
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        u32x2 v;
        v[0] = pack_bf16x2(acc[nb][mb][0], acc[nb][mb][1]);
        v[1] = pack_bf16x2(acc[nb][mb][2], acc[nb][mb][3]);
        *(u32x2*)o = v;
      }
    }
  }
}

// Both operands through LDS (bm == kLdsTile): a workgroup of 8 waves (two per
// SIMD, so one wave's LDS and memory waits overlap the other's MFMAs) owns a
// 256 (n) x 256 (m) output tile; wave (wn, wm) of its 2 x 4 grid owns 128 x 64
// of it (8 x 4 accumulator blocks). Per K step of 64 the workgroup stages the
// step's 256 weight rows and 256 x rows from registers into padded LDS rows
// (whole 128-byte lines: 8 consecutive threads per row; two buffers, one
// barrier per step), with the next step's global loads in flight in
// registers; each wave then reads 8 A and 4 B operands per 32 k for 32 MFMAs
// (5.3 FLOPs per LDS byte against 2 for the 64 x 128 wave tile above).
constexpr int kLdsTile = 256;

template <typename OUT, int DEPTH>
__global__ __launch_bounds__(512, 1) void dense_lds_kernel(const __bf16* __restrict__ x,
                                                           const __bf16* __restrict__ w,
                                                           OUT* __restrict__ out, int M, int N,
                                                           int K, int tiles_n, int tiles_m,
                                                           int steps) {
  constexpr int T = kLdsTile, NT = 512;
  constexpr int PPT = T * 8 / NT;                   // 16-byte pieces per thread per operand
  constexpr int NB = 8, MB = 4;                     // accumulator blocks per wave
  __shared__ __align__(16) uint8_t sw[2][T * kXPitch];
  __shared__ __align__(16) uint8_t sx[2][T * kXPitch];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wid = tid >> 6;
  const int r = lane >> 4, c = lane & 15;
  const int G = tiles_n * tiles_m;
  int t = blockIdx.x;
  if (G % 8 == 0) t = (t % 8) * (G / 8) + t / 8;
  constexpr int GN = 4;
  const int group = t / (GN * tiles_m);
  const int first_n = group * GN;
  const int gsize = min(tiles_n - first_n, GN);
  const int in_group = t - group * GN * tiles_m;
  const int tn = first_n + in_group % gsize;
  const int tm = in_group / gsize;
  const int n0 = tn * T, m0 = tm * T;
  const int wn = (wid & 1) * 128, wm = (wid >> 1) * 64;
  const int kbase = blockIdx.y * steps * kDenseBK;
  out += (size_t)blockIdx.y * M * N;

  // piece q = tid + 512 u of an operand: row q / 8, 16-byte piece q % 8;
  // row offsets are recomputed per load (registers go to the accumulators)
  const __bf16* wb = w + kbase + (tid % 8) * 8;
  const __bf16* xb = x + kbase + (tid % 8) * 8;
  const int wr0 = n0 + tid / 8, xr0 = m0 + tid / 8;
  const uint32_t soff = (uint32_t)((tid / 8) * kXPitch + (tid % 8) * 16);
  struct Stage {
    u32x4 w[PPT], x[PPT];
  };
  auto gload = [&](int s, Stage& st) {
    const int k0 = min(s, steps - 1) * kDenseBK;
#pragma unroll
    for (int u = 0; u < PPT; ++u)
      st.w[u] = load_nt((const u32x4*)(wb + (size_t)min(wr0 + 64 * u, N - 1) * K + k0));
#pragma unroll
    for (int u = 0; u < PPT; ++u)
      st.x[u] = *(const u32x4*)(xb + (size_t)min(xr0 + 64 * u, M - 1) * K + k0);
  };
  auto lstore = [&](int b, const Stage& st) {
#pragma unroll
    for (int u = 0; u < PPT; ++u) *(u32x4*)(sw[b] + soff + u * 64 * kXPitch) = st.w[u];
#pragma unroll
    for (int u = 0; u < PPT; ++u) *(u32x4*)(sx[b] + soff + u * 64 * kXPitch) = st.x[u];
  };
  f32x4 acc[NB][MB];
#pragma unroll
  for (int i = 0; i < NB; ++i)
#pragma unroll
    for (int j = 0; j < MB; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](int b) {
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      u32x4 a[NB], bx[MB];
#pragma unroll
      for (int j = 0; j < MB; ++j)
        bx[j] = *(const u32x4*)(sx[b] + (wm + 16 * j + c) * kXPitch + 64 * kk + 16 * r);
#pragma unroll
      for (int i = 0; i < NB; ++i)
        a[i] = *(const u32x4*)(sw[b] + (wn + 16 * i + c) * kXPitch + 64 * kk + 16 * r);
#pragma unroll
      for (int i = 0; i < NB; ++i)
#pragma unroll
        for (int j = 0; j < MB; ++j) acc[i][j] = mfma(a[i], bx[j], acc[i][j]);
    }
  };

  Stage st;
  gload(0, st);
  lstore(0, st);
  gload(1, st);
  __syncthreads();
  for (int s = 0; s < steps; ++s) {
    compute(s & 1);
    lstore((s + 1) & 1, st);                         // harmless past the end
    gload(s + 2, st);
    __syncthreads();
  }
  // lane (r, c) of block (i, j) holds out[m0 + wm + 16 j + c][n0 + wn + 16 i + 4 r + e]
#pragma unroll
  for (int j = 0; j < MB; ++j) {
    const int m = m0 + wm + 16 * j + c;
    if (m >= M) continue;
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int n = n0 + wn + 16 * i + 4 * r;
      if (n >= N) continue;
      OUT* o = out + (size_t)m * N + n;
      if constexpr (sizeof(OUT) == 4) {
        *(f32x4*)o = acc[i][j];
      } else {
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        u32x2 v;
        v[0] = pack_bf16x2(acc[i][j][0], acc[i][j][1]);
        v[1] = pack_bf16x2(acc[i][j][2], acc[i][j][3]);
        *(u32x2*)o = v;
      }
    }
  }
}

// Direct-to-LDS form (bm == kLdsTile, wn == 128): a workgroup of NW = 8 waves,
// two per SIMD, owns a 256 x 256 output tile; wave (wn, wm) of its 2 x 4 grid
// owns 128 x 64 of it (8 x 4 accumulator blocks), so every weight operand it
// reads from LDS feeds 4 MFMAs and every x operand 8. Both operands go from
// memory into LDS with global_load_lds_dwordx4 (no staging registers, no LDS
// store instructions). A stage is 32 k (one v_mfma_f32_16x16x32 deep); the
// loads move a pair of stages at once, in whole 128-byte rows (64 k), into a
// ring of two pair buffers (128 KB): while pair d is multiplied, pair d + 1
// is in flight, and each stage reads the next stage's operands into the
// second register set. The loads of pair d + 2 are issued one per
// accumulator row through stage 2 d + 1 (8-10% faster on qkv at M = 8192
// than all of them right after the barrier). 16-byte piece p of row R sits
// at slot p ^ ((R >> 1) & 7) of its 128-byte LDS row; an MFMA operand read (lane (r, c): row c of a
// 16-row block, piece 4 h + r of stage half h) then touches every bank group
// once per 16 lanes. One barrier per pair of stages; the memory waits are
// explicit (vmcnt counts this wave's loads). Measured alternatives at M = 8192
// on the 8B shapes: half-line loads (64-byte rows, one stage per load, a ring
// of four stages, one barrier per stage) 3-6% slower; a fifth such stage (all
// 160 KB of LDS) slower again; four waves of 128 x 128 5-7% slower; two
// workgroups of 4 waves per CU (3 stages each) 15% slower. An ablation copy
// without the memory-to-LDS loads runs at 1.9-2.25 PFLOP/s, one without the
// LDS operand reads at 1.26-1.41: the loads bound the kernel.
constexpr int kDlBK = 32;                 // k per stage
constexpr int kDlStages = 4;              // LDS stages: two pair buffers
constexpr int kDlOpBytes = kLdsTile * kDlBK * 2;   // one operand of one stage: 16 KB

// BLK: w in the BF16B layout. Its loads move whole 1 KB blocks (16 rows x 32
// k) instead of 128-byte rows; block (row tile t, stage half h) of a pair
// sits at LDS block 2 t + h, and a lane's A operand is its own 16 bytes of a
// block (no swizzle needed: 64 lanes read 1 KB contiguously).
template <typename OUT, int NW, bool SWIGLU, bool BLK>
__global__ __launch_bounds__(NW * 64, 1) void dense_dl_kernel(const __bf16* __restrict__ x,
                                                              const __bf16* __restrict__ w,
                                                              OUT* __restrict__ out, int M,
                                                              int N, int K, int tiles_n,
                                                              int tiles_m, int steps) {
  constexpr int T = kLdsTile;
  constexpr int NB = 8, MB = 32 / NW;          // wave tile 128 x 16 MB
  constexpr int LPW = 32 / NW;                 // 1 KB loads per wave per operand per pair of stages
  constexpr int PAIR = 2 * kDlOpBytes;         // one operand of a pair of stages: 256 rows x 128 B
  __shared__ __align__(1024) uint8_t lds[2][2][PAIR];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane >> 4, c = lane & 15;
  const int G = tiles_n * tiles_m;
  int t = blockIdx.x;
  if (G % 8 == 0) t = (t % 8) * (G / 8) + t / 8;
  constexpr int GN = 4;
  const int group = t / (GN * tiles_m);
  const int first_n = group * GN;
  const int gsize = min(tiles_n - first_n, GN);
  const int in_group = t - group * GN * tiles_m;
  const int tn = first_n + in_group % gsize;
  const int tm = in_group / gsize;
  const int n0 = tn * T, m0 = tm * T;
  const int wn = (wid & 1) * 128, wm = (wid >> 1) * 16 * MB;
  const int kbase = blockIdx.y * steps * kDlBK;
  out += (size_t)blockIdx.y * M * N;

  // a pair of stages (64 k) is loaded at once, in whole 128-byte rows: load j
  // of this wave fills rows 8 (LPW wid + j) .. + 7 of an operand, lane L
  // writing row 8 (LPW wid + j) + L / 8, slot L % 8, with global piece
  // (L % 8) ^ ((row >> 1) & 7)
  constexpr int KSTR = BLK ? 16 : 1;             // weight elements per k
  const __bf16* wsrc[LPW];
  const __bf16* xsrc[LPW];
#pragma unroll
  for (int j = 0; j < LPW; ++j) {
    const int row = 8 * (LPW * wid + j) + (lane >> 3);
    const int piece = (lane & 7) ^ ((row >> 1) & 7);
    if constexpr (BLK) {
      const int b = LPW * wid + j;                // block (tile b / 2, half b % 2)
      wsrc[j] = w + ((size_t)min(n0 / 16 + b / 2, N / 16 - 1) * (K / 32) + kbase / 32 + b % 2) * 512 +
                8 * lane;
    } else {
      wsrc[j] = w + (size_t)min(n0 + row, N - 1) * K + kbase + 8 * piece;
    }
    xsrc[j] = x + (size_t)min(m0 + row, M - 1) * K + kbase + 8 * piece;
  }
  // operand reads of stage half h: block i's row wn + 16 i + c, piece 4 h + r
  // at slot (4 h + r) ^ (c >> 1); block i sits 2048 bytes after block 0 (in
  // blocks: LDS block 2 (wn / 16 + i) + h, the lane's own 16 bytes)
  const uint32_t aoff0 = BLK ? (uint32_t)(wn * 128 + 16 * lane)
                             : (uint32_t)((wn + c) * 128 + 16 * (r ^ (c >> 1)));
  const uint32_t aoff1 = BLK ? aoff0 + 1024u
                             : (uint32_t)((wn + c) * 128 + 16 * ((4 + r) ^ (c >> 1)));
  const uint32_t boff0 = (uint32_t)((wm + c) * 128 + 16 * (r ^ (c >> 1)));
  const uint32_t boff1 = (uint32_t)((wm + c) * 128 + 16 * ((4 + r) ^ (c >> 1)));

  // the LDS DMA is issued from inline assembly, so the compiler neither
  // orders LDS reads behind it nor waits for it: the explicit vmcnt waits
  // below do (this wave's loads; the barrier makes every wave's visible)
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)(&lds[0][0][0]);
  auto dma = [&](const __bf16* src, uint32_t dst) {
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :: "v"(src), "s"(dst) : "memory", "m0");
#pragma clang diagnostic pop
  };
  const int pairs = steps / 2;
  auto issue = [&](int d) {                    // stages 2 d, 2 d + 1 into buffer d & 1
    const int k0 = min(d, pairs - 1) * 2 * kDlBK;
    const uint32_t base = lds0 + (uint32_t)((d & 1) * 2 * PAIR + LPW * wid * 1024);
#pragma unroll
    for (int j = 0; j < LPW; ++j) dma(wsrc[j] + KSTR * k0, base + j * 1024);
#pragma unroll
    for (int j = 0; j < LPW; ++j) dma(xsrc[j] + k0, base + PAIR + j * 1024);
  };
  auto opA = [&](int s, int i) {
    return *(const u32x4*)(&lds[(s >> 1) & 1][0][((s & 1) ? aoff1 : aoff0) + 2048 * i]);
  };
  auto opB = [&](int s, int j) {
    return *(const u32x4*)(&lds[(s >> 1) & 1][1][((s & 1) ? boff1 : boff0) + 2048 * j]);
  };

  f32x4 acc[NB][MB];
#pragma unroll
  for (int i = 0; i < NB; ++i)
#pragma unroll
    for (int j = 0; j < MB; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  // one stage: row i's 8 MFMAs, then a[i] is refilled with stage s + 1's
  // block i (its last use in this stage is done); bn receives stage s + 1's
  // x operands up front, into the set this stage does not read
  u32x4 a[NB], b0[MB], b1[MB];
  auto issue_one = [&](int d, int i) {
    const int k0 = min(d, pairs - 1) * 2 * kDlBK;
    const uint32_t base = lds0 + (uint32_t)((d & 1) * 2 * PAIR + LPW * wid * 1024);
    if (i < LPW) dma(wsrc[i] + KSTR * k0, base + i * 1024);
    else dma(xsrc[i - LPW] + k0, base + PAIR + (i - LPW) * 1024);
  };
  auto stage = [&](int s, const u32x4 (&bc)[MB], u32x4 (&bn)[MB], int dq) {
#pragma unroll
    for (int j = 0; j < MB; ++j) bn[j] = opB(s + 1, j);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NB; ++i) {
#pragma unroll
      for (int j = 0; j < MB; ++j) acc[i][j] = mfma(a[i], bc[j], acc[i][j]);
      a[i] = opA(s + 1, i);
      if (dq >= 0 && i < 2 * LPW) issue_one(dq, i);
      // keep the refill here, a stage ahead of its use
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // vmcnt(n) with the other counters left open (gfx9 encoding)
#define ACORN_DL_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))

  constexpr int LPS = 2 * LPW;        // this wave's loads per pair of stages
  issue(0);
  issue(1);
  ACORN_DL_VMCNT(LPS);                // this wave's pair-0 loads have landed
  __syncthreads();
#pragma unroll
  for (int i = 0; i < NB; ++i) a[i] = opA(0, i);
#pragma unroll
  for (int j = 0; j < MB; ++j) b0[j] = opB(0, j);
  // pair d: stage 2 d reads stage 2 d + 1's operands (same buffer); then
  // pair d + 1 has landed everywhere (barrier) and every wave has read its
  // last operands from buffer d & 1, which receives pair d + 2; stage 2 d + 1
  // reads pair d + 1's first operands
  for (int d = 0; d < pairs; ++d) {
    stage(2 * d, b0, b1, -1);
    ACORN_DL_VMCNT(0);
    __syncthreads();
    stage(2 * d + 1, b1, b0, d + 2);
  }
#undef ACORN_DL_VMCNT
  __builtin_amdgcn_s_waitcnt(0);      // no LDS write of this wave outlives it

  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  if constexpr (SWIGLU) {
    // gate|up rows interleaved in 16-row blocks: the wave's blocks 2q (gate)
    // and 2q + 1 (up) hold the same 16 outputs, pair (n0 + wn) / 32 + q;
    // out is act [M, N / 2]
#pragma unroll
    for (int j = 0; j < MB; ++j) {
      const int m = m0 + wm + 16 * j + c;
      if (m >= M) continue;
#pragma unroll
      for (int q = 0; q < NB / 2; ++q) {
        const int nb = n0 + wn + 32 * q;
        if (nb >= N) continue;
        const f32x4 g = acc[2 * q][j], u = acc[2 * q + 1][j];
        u32x2 v;
        v[0] = pack_bf16x2(swiglu_bf16(g[0], u[0]), swiglu_bf16(g[1], u[1]));
        v[1] = pack_bf16x2(swiglu_bf16(g[2], u[2]), swiglu_bf16(g[3], u[3]));
        *(u32x2*)(out + (size_t)m * (N / 2) + nb / 2 + 4 * r) = v;
      }
    }
    return;
  }
  // lane (r, c) of block (i, j) holds out[m0 + wm + 16 j + c][n0 + wn + 16 i + 4 r + e]
#pragma unroll
  for (int j = 0; j < MB; ++j) {
    const int m = m0 + wm + 16 * j + c;
    if (m >= M) continue;
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int n = n0 + wn + 16 * i + 4 * r;
      if (n >= N) continue;
      OUT* o = out + (size_t)m * N + n;
      if constexpr (sizeof(OUT) == 4) {
        *(f32x4*)o = acc[i][j];
      } else {
        u32x2 v;
        v[0] = pack_bf16x2(acc[i][j][0], acc[i][j][1]);
        v[1] = pack_bf16x2(acc[i][j][2], acc[i][j][3]);
        *(u32x2*)o = v;
      }
    }
  }
}

template <typename OUT, int NW, bool SWIGLU, bool BLK>
int launch_dl(const void* x, const void* w, void* out, int64_t M, int64_t N, int64_t K, int ks,
              hipStream_t st) {
  const int64_t tiles_n = (N + kLdsTile - 1) / kLdsTile, tiles_m = (M + kLdsTile - 1) / kLdsTile;
  if (tiles_n * tiles_m > 0x7fffffff) return ACORN_ERR_SHAPE;
  dense_dl_kernel<OUT, NW, SWIGLU, BLK>
      <<<dim3((unsigned)(tiles_n * tiles_m), (unsigned)ks), dim3(NW * 64), 0, st>>>(
      (const __bf16*)x, (const __bf16*)w, (OUT*)out, (int)M, (int)N, (int)K, (int)tiles_n,
      (int)tiles_m, (int)(K / kDlBK / ks));
  return ACORN_OK;
}

template <typename OUT, int DEPTH>
int launch_lds(const void* x, const void* w, void* out, int64_t M, int64_t N, int64_t K, int ks,
               hipStream_t st) {
  const int64_t tiles_n = (N + kLdsTile - 1) / kLdsTile, tiles_m = (M + kLdsTile - 1) / kLdsTile;
  if (tiles_n * tiles_m > 0x7fffffff) return ACORN_ERR_SHAPE;
  dense_lds_kernel<OUT, DEPTH>
      <<<dim3((unsigned)(tiles_n * tiles_m), (unsigned)ks), dim3(512), 0, st>>>(
          (const __bf16*)x, (const __bf16*)w, (OUT*)out, (int)M, (int)N, (int)K, (int)tiles_n,
          (int)tiles_m, (int)(K / kDenseBK / ks));
  return ACORN_OK;
}

template <typename OUT, int WN, int BM, int DEPTH, bool BLK>
int launch(const void* x, const void* w, void* out, int64_t M, int64_t N, int64_t K, int ks,
           hipStream_t st) {
  const int64_t tiles_n = (N + 4 * WN - 1) / (4 * WN), tiles_m = (M + BM - 1) / BM;
  if (tiles_n * tiles_m > 0x7fffffff) return ACORN_ERR_SHAPE;
  dense_gemm_kernel<OUT, WN, BM, DEPTH, BLK>
      <<<dim3((unsigned)(tiles_n * tiles_m), (unsigned)ks), dim3(256), 0, st>>>(
          (const __bf16*)x, (const __bf16*)w, (OUT*)out, (int)M, (int)N, (int)K, (int)tiles_n,
          (int)tiles_m, (int)(K / kDenseBK / ks));
  return ACORN_OK;
}

template <typename OUT, bool BLK>
int dispatch(int wn, int bm, int depth, const void* x, const void* w, void* out, int64_t M,
             int64_t N, int64_t K, int ks, hipStream_t st) {
  if (bm == kLdsTile) {
    if constexpr (!BLK) {
      if (wn == 64 && depth == 2) return launch_lds<OUT, 2>(x, w, out, M, N, K, ks, st);
    }
    if (wn == 128 && depth == kDlStages)
      return launch_dl<OUT, 8, false, BLK>(x, w, out, M, N, K, ks, st);
  } else if (wn == 64) {
    if (bm == 128 && depth == 2) return launch<OUT, 64, 128, 2, BLK>(x, w, out, M, N, K, ks, st);
    if (bm == 128 && depth == 4) return launch<OUT, 64, 128, 4, BLK>(x, w, out, M, N, K, ks, st);
    if (bm == 64 && depth == 2) return launch<OUT, 64, 64, 2, BLK>(x, w, out, M, N, K, ks, st);
    if (bm == 64 && depth == 4) return launch<OUT, 64, 64, 4, BLK>(x, w, out, M, N, K, ks, st);
  } else if (wn == 128) {
    if (bm == 64 && depth == 2) return launch<OUT, 128, 64, 2, BLK>(x, w, out, M, N, K, ks, st);
  }
  return ACORN_ERR_UNSUPPORTED;
}

}  // namespace

bool dense_gemm_supported(int64_t N, int64_t K, int wn, int bm, int depth, int ks, bool blocked) {
  // the block layout: whole 16-row tiles and 64-k steps; not the
  // register-staged 256 x 256 form
  if (blocked && (N % 16 || K % 64 || (bm == kLdsTile && wn != 128))) return false;
  if (bm == kLdsTile && wn == 128)   // direct-to-LDS form: 32 k per stage
    return depth == kDlStages && ks >= 1 && ks <= 64 && N % 4 == 0 && K % kDlBK == 0 &&
           (K / kDlBK) % (2 * ks) == 0;
  const bool built = bm == kLdsTile ? wn == 64 && depth == 2
                   : wn == 64 ? (bm == 64 || bm == 128) && (depth == 2 || depth == 4)
                   : wn == 128 ? bm == 64 && depth == 2
                               : false;
  return built && ks >= 1 && ks <= 64 && N % 4 == 0 && K % kDenseBK == 0 &&
         (K / kDenseBK) % ((int64_t)depth * ks) == 0;
}

int dense_gemm_launch(const void* x, const void* w, void* out_bf16, float* out_f32, int64_t M,
                      int64_t N, int64_t K, int wn, int bm, int depth, int ks, bool blocked,
                      hipStream_t st) {
  if (!dense_gemm_supported(N, K, wn, bm, depth, ks, blocked)) return ACORN_ERR_UNSUPPORTED;
  if (out_f32)
    return blocked ? dispatch<float, true>(wn, bm, depth, x, w, out_f32, M, N, K, ks, st)
                   : dispatch<float, false>(wn, bm, depth, x, w, out_f32, M, N, K, ks, st);
  if (ks != 1) return ACORN_ERR_VALUE;
  return blocked ? dispatch<__bf16, true>(wn, bm, depth, x, w, out_bf16, M, N, K, 1, st)
                 : dispatch<__bf16, false>(wn, bm, depth, x, w, out_bf16, M, N, K, 1, st);
}

bool dense_gemm_swiglu_supported(int64_t N, int64_t K, int wn, int bm, int depth, bool blocked) {
  return bm == kLdsTile && wn == 128 && N % 32 == 0 &&
         dense_gemm_supported(N, K, wn, bm, depth, 1, blocked);
}

int dense_gemm_swiglu_launch(const void* x, const void* w, void* act, int64_t M, int64_t N,
                             int64_t K, int wn, int bm, int depth, bool blocked, hipStream_t st) {
  if (!dense_gemm_swiglu_supported(N, K, wn, bm, depth, blocked)) return ACORN_ERR_UNSUPPORTED;
  return blocked ? launch_dl<__bf16, 8, true, true>(x, w, act, M, N, K, 1, st)
                 : launch_dl<__bf16, 8, true, false>(x, w, act, M, N, K, 1, st);
}

}  // namespace acorn
