/*
 * acorn_hip.h — C-ABI of libacorn_hip.so, the MI355X (gfx950) kernels behind
 * the acorninfer_amd Python operators.
 *
 * Every entry point:
 *   - takes plain device pointers, int64 sizes and a hipStream_t (passed as
 *     void* so this header needs no HIP include);
 *   - launches only on that stream, never allocates, never synchronises, so
 *     it can be recorded into a hipGraph;
 *   - returns ACORN_OK (0) or a negative error code (below). Launch failures
 *     come back as ACORN_ERR_HIP - hipError_t.
 *
 * The Python layer (acorninfer_amd/_lib.py) maps the codes onto the
 * exceptions the reference raises at the same boundary.
 */
#ifndef ACORN_HIP_H_
#define ACORN_HIP_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* activation / weight dtype codes */
#define ACORN_F32 0
#define ACORN_F16 1
#define ACORN_BF16 2

/* weight formats of the quantised GEMM */
#define ACORN_WFMT_BF16 0 /* dense bf16 [N,K] (nn.Linear layout) */
#define ACORN_WFMT_W8 1   /* int8 [N,K], fp16 per-channel scale [N] */
#define ACORN_WFMT_W4 2   /* packed uint4 [N,K/2] (low nibble = even k),
                             fp16 scale [N,K/128], optional fp16 zero [N,K/128];
                             no zero pointer = symmetric (w = (u-8)*s) */
#define ACORN_WFMT_F32 3  /* dense fp32 [N,K] with fp32 activations; output
                             only through out_part (the fp32 parity path) */
#define ACORN_WFMT_W4B 4  /* ACORN_WFMT_W4's values in 1 KB blocks (N % 16 == 0,
                             K % 512 == 0): the 16 bytes of row n, k in
                             [32c, 32c+32) sit at byte
                             ((n/16)*(K/128) + c/4)*1024 + ((c%4)*16 + n%16)*16,
                             32-bit word j of them holding k 32c+8j .. +7 with
                             nibble p (bits 4p..4p+3) at k offset 0,2,4,6,1,3,5,7
                             for p = 0..7; scale of (n, group g) at half index
                             ((n/16)*(K/512) + g/4)*64 + ((n%16)/4)*16 + (g%4)*4 + n%4.
                             Symmetric only; a block is one wave's MFMA A
                             operand for 16 rows x 128 k. */
#define ACORN_WFMT_W8B 5  /* ACORN_WFMT_W8's values in 1 KB blocks (N % 16 == 0,
                             K % 64 == 0), each stored as the byte q + 128:
                             the 16 bytes of row n, k in [16c, 16c+16) sit at
                             byte ((n/16)*(K/64) + c/4)*1024 + ((c%4)*16 + n%16)*16;
                             fp16 per-channel scale [N] as in W8. A block is
                             one wave's MFMA A operands for 16 rows x 64 k. */
#define ACORN_WFMT_BF16B 6 /* ACORN_WFMT_BF16's values in 1 KB blocks (N % 16 == 0,
                             K % 64 == 0): the 8 bf16 of row n, k in [8c, 8c+8)
                             sit at element ((n/16)*(K/32) + c/4)*512 +
                             ((c%4)*16 + n%16)*8. A block is one wave's MFMA A
                             operand for 16 rows x 32 k. */

/* error codes */
#define ACORN_OK 0
#define ACORN_ERR_SHAPE (-1)       /* shape/contiguity contract (reference: AssertionError) */
#define ACORN_ERR_DTYPE (-2)       /* unsupported dtype combination */
#define ACORN_ERR_VALUE (-3)       /* bad argument value (reference: ValueError) */
#define ACORN_ERR_UNSUPPORTED (-4) /* configuration not built (reference: NotImplementedError) */
#define ACORN_ERR_SCRATCH (-5)     /* request exceeds the fixed scratch of an allocation-free
                                      entry point */
#define ACORN_ERR_HIP (-1000)      /* ACORN_ERR_HIP - hipError_t */

/* Size of the fixed device scratch of acorn_paged_attention_noalloc (bytes). */
#define ACORN_K3_SCRATCH_BYTES (32 << 20)

/* Library version, bumped when an entry point changes meaning. */
int acorn_version(void);

/*
 * K1 fused residual add + RMSNorm.
 * Replaces acorninfer/ops/rmsnorm.py:39-71 (fused_add_rmsnorm).
 *   residual == NULL : residual_out = x,                   normed = rmsnorm(x)
 *   otherwise        : residual_out = round_T(residual+x), normed = rmsnorm(residual_out)
 * rmsnorm(r) = round_T(r * rsqrt(mean(r^2) + eps) * w) computed in fp32.
 * x, residual, residual_out, normed: [rows, cols] contiguous, dtype `dtype`;
 * weight: [cols], dtype `wdtype`. x and residual are never written.
 */
int acorn_fused_add_rmsnorm(const void* x, const void* residual, void* residual_out,
                            const void* weight, void* normed, int64_t rows, int64_t cols,
                            float eps, int dtype, int wdtype, void* stream);

/*
 * K1 variant that first reduces `nsplit` fp32 split-K partials of the
 * previous projection: x = round_T(sum_s part[s, rows, cols]) (summed in
 * order s = 0..nsplit-1), then behaves as acorn_fused_add_rmsnorm. x_out (may
 * be NULL) receives the rounded x. No counterpart in the reference: it fuses
 * the projection's output cast (qwen3.py:232-233, 392-396) into K1.
 */
int acorn_fused_add_rmsnorm_partials(const float* part, int64_t nsplit, const void* residual,
                                     void* residual_out, const void* weight, void* normed,
                                     void* x_out, int64_t rows, int64_t cols, float eps,
                                     int dtype, int wdtype, void* stream);

/*
 * K2 in-place half-rotate RoPE on rows of `head_dim` values.
 * Replaces acorninfer/ops/rope.py:91-113 (fused_rope_inplace), one call per
 * tensor. x: [batch, heads, head_dim] contiguous; positions: [batch] int32 or
 * int64 (pos_is_i64); inv_freq: [head_dim/2] fp32. Rounding mirrors the
 * reference's three-step torch path (rope.py:1-13).
 */
int acorn_rope_inplace(void* x, int64_t batch, int64_t heads, int64_t head_dim,
                       const void* positions, int pos_is_i64, const float* inv_freq,
                       int dtype, void* stream);

/*
 * K2 fused per-head q/k RMSNorm + RoPE, in place on q [batch, q_heads, D] and
 * k [batch, kv_heads, D]. The norm is models/qwen3.py:50-60 (RMSNorm over D)
 * applied as q_norm/k_norm (qwen3.py:184-185), followed by rope.py's rotation.
 * q_w, k_w: [D] dtype `wdtype`.
 */
int acorn_qknorm_rope_inplace(void* q, void* k, int64_t batch, int64_t q_heads,
                              int64_t kv_heads, int64_t head_dim, const void* q_w,
                              const void* k_w, float eps, const void* positions,
                              int pos_is_i64, const float* inv_freq, int dtype, int wdtype,
                              void* stream);

/*
 * Decode-step fusion of the qkv projection's epilogue with K2 and the KV
 * scatter: reduces `nsplit` fp32 partials of the fused qkv projection
 * part[s, batch, (H + 2*KV)*D], rounds to T, applies q/k RMSNorm + RoPE,
 * writes q_out [batch, H, D] and scatters k, v into
 * k_pages/v_pages [num_blocks, page, KV, D] at (pages[b], slots[b]) (int64);
 * a (page, slot) outside [0, num_blocks) x [0, page_size) is not written.
 * Semantics = qwen3.py:180-192 followed by cache/pager.py:87-113
 * (scatter_decode). No single reference function. nsplit == 0: `part` holds
 * the projection's output already rounded to T, [batch, (H + 2*KV)*D] (a
 * one-split GEMM that wrote T), the same bits as one fp32 plane of it; built
 * for D == 128 from 256 rows (ACORN_ERR_UNSUPPORTED otherwise).
 */
int acorn_qkv_epilogue(const float* part, int64_t nsplit, void* q_out, void* k_pages,
                       void* v_pages, const int64_t* pages, const int64_t* slots,
                       int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                       int64_t page_size, int64_t num_blocks, const void* q_w,
                       const void* k_w, float eps,
                       const int64_t* positions, const float* inv_freq, int dtype,
                       int wdtype, void* stream);

/*
 * K3 flash-decoding paged attention (phase 1 + phase 2).
 * Replaces acorninfer/ops/paged_attention.py:125-152 (paged_decode_attention).
 * q: [B, H, D]; k_pages, v_pages: [NB, P, KV, D]; tables: [B, table_stride]
 * int32; seq_lens: [B] int32 (>= 1, includes the current token);
 * out: [B, H, D]. Token t of sequence b lives at (tables[b, t/P], t%P);
 * q head h reads kv head h / (H/KV). One workgroup serves all H/KV q heads of
 * a kv head (GQA reuse); with bf16/fp16 activations, D >= 64, num_splits == 1
 * over at most 64 pages and fewer (sequence, kv head) pairs than half the 256
 * CUs, the launch gives the q heads of a kv head up to H/KV workgroups of their
 * own instead (no partials, no combine). Workspace: ws_acc [B*H*num_splits*D] fp32 and
 * ws_ml [2*B*H*num_splits] fp32, caller-owned (bf16/fp16 activations with
 * D >= 64 keep each split's normalised output there in fp16, using half of it).
 */
int acorn_paged_attention(const void* q, const void* k_pages, const void* v_pages,
                          const int32_t* tables, const int32_t* seq_lens, void* out,
                          float* ws_acc, float* ws_ml, int64_t B, int64_t H, int64_t KV,
                          int64_t D, int64_t P, int64_t num_blocks, int64_t table_stride,
                          int64_t num_splits, float scale, int dtype, void* stream);

/*
 * acorn_paged_attention with no workspace arguments, for callers that cannot
 * allocate device memory (code under hipGraph capture, serving loops and
 * harnesses that forbid hipMalloc). No counterpart in the reference.
 * Arguments and results are those of acorn_paged_attention (the same kernels,
 * the same bits). The split partials (B*H*num_splits*(D+2) fp32 values, the
 * first part rounded up to 256 bytes) live in a static device array of
 * ACORN_K3_SCRATCH_BYTES per GPU, held until the process ends; a larger
 * request returns ACORN_ERR_SCRATCH and launches nothing (num_splits == 1
 * needs none). Nothing in the scratch has to start at zero: every partial the
 * combine reads is written by the same call. The array is looked up once per
 * device, on the first call with that device current (make that call outside
 * graph capture); `stream` must belong to the current device
 * (ACORN_ERR_VALUE otherwise). Calls that overlap on one GPU (concurrent
 * streams, or graphs replayed concurrently) share the array and race.
 * It calls no hipMalloc, hipFree or other allocating routine.
 */
int acorn_paged_attention_noalloc(const void* q, const void* k_pages, const void* v_pages,
                                  const int32_t* tables, const int32_t* seq_lens, void* out,
                                  int64_t B, int64_t H, int64_t KV, int64_t D, int64_t P,
                                  int64_t num_blocks, int64_t table_stride, int64_t num_splits,
                                  float scale, int dtype, void* stream);

/*
 * Decode-step fusion of acorn_qkv_epilogue with K3: the attention kernel
 * reduces the qkv projection's partials for its own q heads (q is never
 * written), and the workgroup holding each sequence's last split also
 * computes that kv head's new k, v, stores them at (pages[b], slots[b]) as
 * acorn_qkv_epilogue does, and attends to them. Arguments are those of the
 * two entry points (tables/seq_lens/out/ws as in acorn_paged_attention,
 * part..inv_freq as in acorn_qkv_epilogue, positions int64); the results are
 * the same bits (one split over a small batch: every q head group's
 * workgroup stores the same new k, v). No single reference function: qwen3.py:180-192, then
 * cache/pager.py:87-113 (scatter_decode), then paged_attention.py:125-152.
 * Returns ACORN_ERR_UNSUPPORTED, launching nothing, unless
 * acorn_paged_attention_qkv_supported() holds for the shape.
 */
int acorn_paged_attention_qkv(const float* part, int64_t nsplit, void* k_pages, void* v_pages,
                              const int64_t* pages, const int64_t* slots, const int32_t* tables,
                              const int32_t* seq_lens, void* out, float* ws_acc, float* ws_ml,
                              int64_t B, int64_t H, int64_t KV, int64_t D, int64_t P,
                              int64_t num_blocks, int64_t table_stride, int64_t num_splits,
                              float scale, const void* q_w, const void* k_w, float eps,
                              const int64_t* positions, const float* inv_freq, int dtype,
                              int wdtype, void* stream);

/*
 * Prefill attention over the paged cache: causal softmax(q . K^T * scale) V for
 * the rows of a (chunked) prefill whose new K/V are already in the pool.
 * Replaces the per-row SDPA of acorninfer/models/qwen3.py:291-382 (the
 * prefill attention of forward_prefill_batch / forward_extend, :597-686).
 *   q, out [R, H, D] (rows of all N sequences); sequence n's rows are
 *   q[seq_row0[n] .. seq_row0[n] + seq_nq[n]), at positions seq_pos0[n] + j;
 *   row j attends to the sequence's tokens 0 .. seq_pos0[n] + j, stored at
 *   (tables[n, t / P], t % P) of k/v_pages [num_blocks, P, KV, D].
 *   max_nq >= every seq_nq[n] (rows past max_nq, or past row R - 1, are not
 *   written); seq_* int32 [N]; tables int32 [N, table_stride].
 * bf16 / fp16, D in {64, 128}, P a multiple of 16, H/KV in {1, 2, 4, 8}; no
 * workspace (one pass per 16-token query tile, no split).
 */
int acorn_paged_prefill_attention(const void* q, const void* k_pages, const void* v_pages,
                                  const int32_t* tables, const int32_t* seq_row0,
                                  const int32_t* seq_pos0, const int32_t* seq_nq, void* out,
                                  int64_t N, int64_t R, int64_t max_nq, int64_t H, int64_t KV,
                                  int64_t D, int64_t P, int64_t num_blocks, int64_t table_stride,
                                  float scale, int dtype, void* stream);

/*
 * 1 when acorn_paged_attention_qkv supports the shape: bf16 or fp16
 * activations with norm weights of the same dtype, D in {64, 128}, H/KV in
 * {1, 2, 4, 8}, pages of a power-of-two multiple of 16 tokens, and splits
 * (ceil(table_stride / num_splits) pages) of at most 16 pages or of a size
 * whose eight-wave workgroup fits the 160 KB of LDS (block ids, which grow
 * with the split, wave partials, K slabs, the epilogue's rows); else 0. No
 * reference counterpart.
 */
int acorn_paged_attention_qkv_supported(int64_t H, int64_t KV, int64_t D, int64_t P,
                                        int64_t table_stride, int64_t num_splits, int dtype,
                                        int wdtype);

/*
 * Weight-only quantised GEMM y[M,N] = x[M,K] @ dequant(W)[N,K]^T, bf16 in,
 * fp32 accumulate.
 * Replaces acorninfer/ops/quant_gemm.py:257-294 (quant_gemm, W8) and the W4
 * spike scripts/m7_spike.py:152-231, plus the bf16 decode GEMM
 * acorninfer/ops/decode_gemm.py:236-257.
 *   wfmt ACORN_WFMT_BF16: w bf16 [N,K]
 *   wfmt ACORN_WFMT_W8  : w int8 [N,K], scale fp16 [N]
 *   wfmt ACORN_WFMT_W4  : w uint8 [N,K/2], scale fp16 [N,K/128], zero fp16
 *                         [N,K/128] or NULL (symmetric, zero = -8*scale)
 *   wfmt ACORN_WFMT_W4B : as W4, in the blocked layout above (the decode
 *                         model's int4 weights)
 *   wfmt ACORN_WFMT_W8B : as W8, in the blocked layout above (the decode
 *                         model's int8 weights)
 *   wfmt ACORN_WFMT_BF16B: as BF16, in the blocked layout above (the decode
 *                         model's bf16 weights)
 *   wfmt ACORN_WFMT_F32 : w fp32 [N,K], x fp32 [M,K]; fp32 result in part
 * cfg: NULL or int[6] {rt, upw, nw, ksplit, tpw, -}; 0 entries are chosen by
 * the planner (acorn_gemm_plan). With the chosen ksplit:
 *   out_bf16 != NULL, ksplit == 1: writes bf16 [M,N];
 *   out_bf16 != NULL, ksplit > 1 : part is an fp32 workspace [ksplit,M,N]; a
 *       second launch sums the partials in split order into out_bf16
 *       (bitwise deterministic);
 *   out_bf16 == NULL             : writes fp32 partials part[ksplit,M,N].
 */
int acorn_quant_gemm(const void* x, const void* w, const void* scale, const void* zero,
                     void* out_bf16, float* part, int64_t M, int64_t N, int64_t K, int wfmt,
                     const int* cfg, void* stream);

/*
 * gate|up projection with the SwiGLU activation fused into its epilogue:
 *   act[m, j] = round(round(silu(g)) * u),  g = round(x[m] . Wg[j]), u = round(x[m] . Wu[j])
 * (acorninfer/models/qwen3.py:392-396: F.silu(gate_proj(x)) * up_proj(x), each
 * bf16 op rounded; silu(g) = g / (1 + exp(-g)) in fp32). No single reference
 * function: it fuses gate_proj, up_proj and the activation of Qwen3MLP.
 * w holds the gate and up weights interleaved in 16-row blocks: rows
 * [32i, 32i+16) are gate rows 16i..16i+15 and rows [32i+16, 32i+32) the up
 * rows of the same outputs (scales / zeros interleaved the same way); N is
 * the interleaved row count (2 * intermediate), act is [M, N/2] bf16.
 * Decode sizes (M <= 16; cfg as for acorn_quant_gemm, rt is 2 and ksplit 1
 * by construction), and bf16 weights at prefill sizes (from 512 rows, or
 * cfg[0] == -2: the large-M kernel's 256 x 256 direct-to-LDS form, ksplit 1,
 * N % 32 == 0), where the act is bitwise what acorn_silu_mul gives on the
 * one-split fp32 output.
 */
int acorn_quant_gemm_swiglu(const void* x, const void* w, const void* scale, const void* zero,
                            void* act, int64_t M, int64_t N, int64_t K, int wfmt,
                            const int* cfg, void* stream);

/*
 * Decode GEMM (M <= 16, block formats BF16B / W8B / W4B) with the RMSNorm that
 * sits between two projections folded in, so that the step needs no K1
 * launch there. Replaces the pair acorn_quant_gemm + acorn_fused_add_rmsnorm
 * (acorninfer/ops/rmsnorm.py:39-82 after a projection, models/qwen3.py:
 * 412-439) split across the producer and the consumer projection, from
 * RMSNorm(v) @ W^T = inv * (bf16(v * norm_w) @ W^T) per row:
 *   producer (res != NULL; ksplit 1, swiglu 0): instead of y the launch
 *       stores the new residual res_out[m, n] = bf16(res[m, n] + bf16(y[m, n]))
 *       (res_out may be res), the weighted rows xw_out[m, n] =
 *       bf16(res_out[m, n] * norm_w[n]) (norm_w [N]: the next RMSNorm's
 *       weight) and ss_out[m][n / 16] = the fp32 sum of
 *       res_out[m, 16t .. 16t + 15]^2 per 16 columns t; out_bf16 and part are
 *       unused;
 *   consumer (ss_in != NULL): x is the producer's xw_out [M, K]; every result
 *       of row m (each split's partial, or the values the SwiGLU act is made
 *       of) is multiplied by inv = 1 / sqrt(sum_t ss_in[m][t] / K + eps) before
 *       it is stored, ss_in [M][K / 16] the producer's sums: K1's inv with its
 *       sum of squares added in another order, and the bf16 rounding of the
 *       normalised row on v * norm_w instead of (v * inv) * norm_w (so within
 *       rounding of the K1 pair, not bitwise). The output is as
 *       acorn_quant_gemm's (or the SwiGLU act with swiglu != 0).
 * Exactly one of ss_in, res is given. cfg as for acorn_quant_gemm (the
 * direct kernels' tilings); other tilings return ACORN_ERR_UNSUPPORTED.
 */
int acorn_quant_gemm_norm(const void* x, const void* w, const void* scale, void* out_bf16,
                          float* part, int64_t M, int64_t N, int64_t K, int wfmt,
                          const int* cfg, int swiglu, const float* ss_in, float eps,
                          const void* res, void* res_out, float* ss_out, const void* norm_w,
                          void* xw_out, void* stream);

/* Tiling of acorn_quant_gemm_swiglu, as acorn_gemm_plan. */
int acorn_gemm_swiglu_plan(int64_t M, int64_t N, int64_t K, int wfmt, int* cfg);

/*
 * ACORN_WFMT_W4B weights (symmetric int4, scale fp16 per 128-k group) -> bf16
 * [N, K] in the weight's row order: out[n, k] = bf16_rne((u - 8) * s), the
 * dequantisation the reference's large-M quantised GEMM applies in-kernel
 * before its bf16 dot (acorninfer/ops/quant_gemm.py:175-183: int -> fp32 x
 * scale -> bf16). With acorn_quant_gemm on ACORN_WFMT_BF16 it forms the
 * int4 GEMM at prefill sizes (from about 512 rows), where the bf16 MFMA kernel
 * outruns any in-kernel unpacking. N % 16 == 0, K % 512 == 0; out holds
 * N * K bf16 (the caller's workspace).
 */
int acorn_dequant_w4b(const void* w, const void* scale, void* out_bf16, int64_t N, int64_t K,
                      void* stream);

/* Deterministic split-K reduction: out[M*N] = round_T(sum_s part[s, M*N]). */
int acorn_splitk_reduce(const float* part, int64_t nsplit, int64_t count, void* out,
                        int dtype, void* stream);

/*
 * Tiling for acorn_quant_gemm: cfg[0..4] hold requests (0 = choose) and are
 * overwritten with the full choice {rt: 16-row tiles per wavefront row block,
 * upw: 16-byte weight loads per lane per step, nw: wavefronts per workgroup,
 * ksplit: K splits, tpw: tiles per workgroup}; cfg[5] receives the number of
 * output tiles. No GPU access.
 */
int acorn_gemm_plan(int64_t M, int64_t N, int64_t K, int wfmt, int* cfg);

/*
 * Embedding row gather: out[b, :] = table[ids[b], :].
 * Replaces nn.Embedding in acorninfer/models/qwen3.py:585 (embed_tokens).
 * table: [vocab, cols]; ids: [rows] int64 (an id outside [0, vocab) reads
 * row 0); out: [rows, cols].
 */
int acorn_embedding(const void* table, const int64_t* ids, void* out, int64_t rows,
                    int64_t vocab, int64_t cols, int dtype, void* stream);

/*
 * SwiGLU activation of the fused gate|up projection:
 *   act[r, i] = round(round(silu(g)) * u),  g = gate_up[r, i], u = gate_up[r, inter + i]
 * Replaces F.silu(gate_proj(x)) * up_proj(x) in acorninfer/models/qwen3.py:392-396.
 * part != NULL: g, u = round(sum_s part[s, r, .]) over `nsplit` fp32 split-K
 * partials [nsplit, rows, 2*inter] (summed in split order); otherwise
 * gate_up [rows, 2*inter] of dtype `dtype` is read. Columns are [gate | up],
 * or with interleaved16 the 16-column blocks of acorn_quant_gemm_swiglu's
 * weight layout (gate block i at 32i, up block i at 32i+16). act: [rows, inter].
 */
int acorn_silu_mul(const float* part, int64_t nsplit, const void* gate_up, void* act,
                   int64_t rows, int64_t inter, int interleaved16, int dtype, void* stream);

/*
 * Greedy token choice: out[r] = first index of the row maximum of x[rows, cols]
 * (NaN ranks above every number). Replaces logits.argmax(dim=1) in
 * acorninfer/engine/graph_runner.py:177 and engine/executor.py:105-107.
 */
int acorn_argmax(const void* x, int64_t rows, int64_t cols, int64_t* out, int dtype,
                 void* stream);

/*
 * Decode-step KV write: k_pages[pages[b], slots[b], h, :] = k[b, h, :] (same
 * for v). Replaces PagedKVCache.scatter_decode in
 * acorninfer/cache/pager.py:87-113 (torch index_put). k, v: [batch, kv_heads,
 * head_dim]; k_pages, v_pages: [num_blocks, page_size, kv_heads, head_dim];
 * pages, slots: [batch] int64. A (page, slot) outside the pool is skipped.
 */
int acorn_kv_scatter(const void* k, const void* v, void* k_pages, void* v_pages,
                     const int64_t* pages, const int64_t* slots, int64_t batch,
                     int64_t kv_heads, int64_t head_dim, int64_t page_size,
                     int64_t num_blocks, int dtype, void* stream);

/*
 * Token sampling, one row per sequence: temperature -> top-k -> top-p -> draw.
 * Replaces acorninfer/sampler.py:38-68 (Sampler.process / Sampler.sample) and
 * the greedy branch of engine/executor.py:128-138.
 * logits [rows, vocab] (dtype); per row: temperature (0 = greedy argmax, logprob
 * 0), top_k (0 = off), top_p (1 = off), uniform u in [0, 1). The token is the
 * inverse-CDF draw of u over the kept tokens in vocabulary order; logprob is
 * log_softmax(processed)[token]. processed (NULL or fp32 [rows, vocab]) receives
 * x = logits / T where kept and -inf elsewhere. status[r] = 1 when the row holds
 * NaN or +-inf (the reference raises ValueError), else 0. Deterministic.
 */
int acorn_sample(const void* logits, int64_t rows, int64_t vocab, int dtype,
                 const float* temperature, const int32_t* top_k, const float* top_p,
                 const float* uniform, int64_t* token, float* logprob, float* processed,
                 int32_t* status, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ACORN_HIP_H_ */
