/*
 * laprune_hip.h — C ABI of the MI355X (gfx950) decode-time retrieval path.
 *
 * Every entry point takes caller-owned device pointers for inputs AND outputs,
 * explicit sizes/strides and a hipStream_t, launches asynchronously on that
 * stream and returns an int status (LAP_OK on success).  Nothing here
 * allocates device memory: kernels that need scratch take a workspace pointer
 * whose size is reported by the matching *_workspace_size() query.  On error
 * the status is non-zero and lap_last_error() returns a thread-local message.
 *
 * Element types are passed as LAP_DTYPE_* codes.  Strides are in elements.
 * fp16/bf16 values are raw 16-bit patterns (uint16_t in memory).
 *
 * Reference interfaces replaced (paths relative to the LAPrune source tree):
 *   aq_kernels/aq_lut_gqa.cu, aq_kernels/aq_lut.cu,
 *   aq_kernels/fused_linear_encode.cu, laprune/llm/aq_kv.py,
 *   laprune/llm/modifiers/aq_evaluation.py.
 */
#ifndef LAPRUNE_HIP_H
#define LAPRUNE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* hipStream_t is an opaque pointer; declared here as void* so the header does
 * not depend on the HIP headers (0 = the null stream). */
typedef void* lap_stream_t;

/* ---- status codes ------------------------------------------------------ */
#define LAP_OK              0
#define LAP_ERR_INVALID     1   /* bad shape / stride / dtype / range      */
#define LAP_ERR_UNSUPPORTED 2   /* valid request this build does not serve  */
#define LAP_ERR_HIP         3   /* HIP runtime or launch failure            */
#define LAP_ERR_WORKSPACE   4   /* workspace missing or too small           */

/* ---- element type codes ------------------------------------------------ */
#define LAP_DTYPE_F32   0
#define LAP_DTYPE_F16   1
#define LAP_DTYPE_BF16  2
#define LAP_DTYPE_U8    3
#define LAP_DTYPE_I8    4
#define LAP_DTYPE_I32   5
#define LAP_DTYPE_I64   6

/* ---- LUT layouts ------------------------------------------------------- */
#define LAP_LUT_HMK   0   /* [Hq][M][K]       (reference layout)          */
#define LAP_LUT_GMKG  1   /* [Hq/G][M][K][G]  (interleaved, scorer LDS)   */

/* ---- top-k key modes ---------------------------------------------------- */
#define LAP_KEY_F16   0   /* rank the fp16 score itself                     */
#define LAP_KEY_BF16  1   /* rank bf16(fp16 score): the model-dtype cast    */
/* OR-ed into the key_mode of lap_retrieve_score / _topk / _topk_ragged: one
 * top-k per query head (the reference's selection, aq_evaluation.py:198-201)
 * instead of one per KV group on the group max.  Selection rows are then
 * B*Hkv*4, row b*Hq + h; size the workspace with
 * lap_retrieve_workspace_size(B*Hkv*4, T). */
#define LAP_SELECT_PER_HEAD 0x10

/* ---- per-sequence plan of one decode step (ragged batches) ---------------
 * The reference decodes a batch with one shared length
 * (laprune/llm/modifiers/aq_evaluation.py:150-155: seq_len, total_seq_len).
 * The *_ragged entry points take a device array plans[B] instead, one per
 * sequence b; each field has the meaning of the scalar argument it replaces
 * in the uniform entry point (the arithmetic of aq_evaluation.py:185-218):
 *   t_codes     encoded tokens: columns [0, t_codes) are scored
 *   t_total     cached tokens: keep-set rows must lie in [0, t_total)
 *   cand_start, cand_end   candidate window (within [0, t_codes))
 *   k           tokens to select (min'd with the window size and k_cols)
 *   sink, tail_start, tail_count   keep set [0, sink) ++ [tail_start, +tail_count)
 * Plans live in device memory so that a captured graph can be replayed after
 * the host rewrites them. */
typedef struct lap_row_plan {
  int32_t t_codes, t_total;
  int32_t cand_start, cand_end;
  int32_t k;
  int32_t sink, tail_start, tail_count;
} lap_row_plan;

/* Message of the last failed call on this thread ("" if none). */
const char* lap_last_error(void);
/* ABI version: bumped when any signature below changes. */
int lap_abi_version(void);
/* Device facts used for launch shaping (current device). */
int lap_device_info(int* cu_count, int* lds_bytes_per_block, int* wave_size);

/* ======================================================================= *
 * A1  LUT builder                                                          *
 * Replaces: laprune/llm/aq_kv.py:681-682 (torch.matmul(q, C.reshape(MK,d).t())
 *   .reshape(Hq,M,K)), fp32 form aq_kv.py:620 (einsum "mkd,qd->qmk").
 * lut[h,m,k] = fp16_rne( fmaf-chain over d = 0..D-1 of q[h,d]*C[m,k,d] ),
 * accumulated sequentially in fp32 from 0.
 *   q          [Hq][D], row stride q_row_stride, dtype f32/f16/bf16
 *   codebooks  [M][K][D] contiguous, dtype f32/f16
 *   lut_out    fp16, layout LAP_LUT_HMK or LAP_LUT_GMKG (needs Hq % G == 0)
 * ======================================================================= */
int lap_lut_build(const void* q, int q_dtype, int64_t q_row_stride,
                  const void* codebooks, int cb_dtype,
                  int Hq, int D, int M, int K, int G, int layout,
                  void* lut_out, lap_stream_t stream);

/* ======================================================================= *
 * A2  GQA LUT scorers                                                      *
 * Score accumulation contract (all scorers): acc = 0.0f; for m ascending:
 * acc += (float)lut_fp16[h, m, code]; out = fp16_rne(acc).
 * ======================================================================= */

/* Replaces: aq_lut_gather_grouped, aq_kernels/aq_lut_gqa.cu:460-534
 * (kernels :111-149 and :157-212).
 *   lut    fp16, layout LAP_LUT_HMK ([Hkv*G][M][K]) or LAP_LUT_GMKG
 *   codes  u8 [Hkv][T][M] with strides (codes_stride_h, codes_stride_t, 1)
 *   out    fp16 [Hkv*G][T] contiguous
 * G in 1..4. */
int lap_lut_score_grouped(const void* lut, int lut_layout,
                          const uint8_t* codes, int64_t codes_stride_h,
                          int64_t codes_stride_t,
                          int Hkv, int G, int T, int M, int K,
                          void* out, lap_stream_t stream);

/* Replaces: aq_lut_gather (bound as aq_lut_gather_gqa),
 * aq_kernels/aq_lut_gqa.cu:350-422 (kernel :20-76).
 *   lut      fp16 [H][M_stride][K] contiguous, H = Hkv*G (any G >= 1)
 *   codes    u8 [Hkv][T][M_stride], strides (cs_h, cs_t, 1)
 *   indices  int64 [H][N] or NULL (dense: N = T); an index outside [0,T)
 *            scores 0
 *   out      fp16 [H][N]
 * Only m in [M_start, M_end) is summed. */
int lap_lut_score_gqa(const void* lut, const uint8_t* codes,
                      int64_t codes_stride_h, int64_t codes_stride_t,
                      int Hkv, int G, int T, int M_stride, int K,
                      int M_start, int M_end,
                      const int64_t* indices, int N,
                      void* out, lap_stream_t stream);

/* Replaces: aq_lut_gather_forward, aq_kernels/aq_lut.cu:641-738
 * (kernels :581-639).
 *   lut    [Q][M*K], dtype f16 or f32 (f32 sums in f32, no rounding to f16)
 *   codes  [Q][N][M] contiguous, dtype u8/i8/i64; the low 8 bits are read as
 *          an unsigned code and clamped to [0, K-1]
 *   out    [Q][N], same dtype as lut */
int lap_lut_score_mha(const void* lut, int lut_dtype,
                      const void* codes, int codes_dtype,
                      int Q, int N, int M, int K,
                      void* out, lap_stream_t stream);

/* Replaces: aq_lut_forward, aq_kernels/aq_lut.cu:445-574 (kernels :37-149).
 * Direct scoring without a LUT: score[q,n] = sum over m (code valid) of
 * dot(q, C[m,code]) in one fp32 accumulator.
 *   f32: acc = fmaf(q[i], c[i], acc) for m, then i ascending
 *   f16: per pair (i, i+1): p = fp16_rne(q*c) lanewise; acc += (p0 + p1)
 *   q [Q][D], codebooks [M][K][D], codes [Q][N][M] (u8/i8/i64; low 8 bits),
 *   out [Q][N] same dtype as q (f32 or f16).  Codes >= K are skipped. */
int lap_aq_lut_direct(const void* q, const void* codebooks, int dtype,
                      const void* codes, int codes_dtype,
                      int Q, int N, int M, int K, int D,
                      void* out, lap_stream_t stream);

/* Replaces: AQLayerCodebookManager.reconstruct, laprune/llm/aq_kv.py:431-457.
 * out[n] = sum over m ascending of codebooks[m][code(n, m)], elementwise fp32
 * from 0 (the reference's recon += C_m[codes[:, m]] loop).
 *   codebooks  [M][K][D] fp32 contiguous, 16-byte aligned, D % 4 == 0
 *   codes      [N][M] rows codes_row_stride elements apart, dtype u8/i8/i64;
 *              the low 8 bits are read as an unsigned code, clamped to K-1
 *   out        [N][D] fp32 contiguous, 16-byte aligned */
int lap_aq_reconstruct(const float* codebooks, int M, int K, int D, const void* codes,
                       int codes_dtype, int64_t codes_row_stride, int N, float* out,
                       lap_stream_t stream);

/* ======================================================================= *
 * A3  Top-k selection                                                      *
 * Replaces: torch.topk(scores[..., cand_start:cand_end], k, sorted=False)
 *   at laprune/llm/modifiers/aq_evaluation.py:198-201.
 * Rows r = 0..R-1 select over columns [cand_start, cand_end) of
 *   key(r, t) = max over g < group of score[(r*group + g), t]   (fp16)
 * mapped through key_mode.  The k largest keys are kept; among equal keys
 * the lowest column wins.  Output: column indices (t, absolute, i.e.
 * including cand_start) in ascending order, out[r][0..k_eff), with
 * k_eff = min(k, cand_end - cand_start); entries past k_eff are not written.
 *   scores   fp16 [R*group][T] with row stride score_row_stride
 *   out_idx  [R][k] int32 or int64 (out_dtype)
 * ======================================================================= */
int lap_topk_workspace_size(int R, int cand_len, size_t* bytes);
int lap_topk_select(const void* scores, int64_t score_row_stride,
                    int R, int group, int T, int cand_start, int cand_end,
                    int k, int key_mode, void* out_idx, int out_dtype,
                    void* workspace, size_t workspace_bytes,
                    lap_stream_t stream);

/* Fused score + select for one decode step (A1 output -> A2 -> A3).
 * lut is LAP_LUT_GMKG fp16 for G = 4, M = 32, K = 256.  Per KV row r the
 * group key is max_g fp16(score); selection as lap_topk_select.  Optional
 * per-head fp16 scores are written when scores_out != NULL ([Hkv*4][T]).
 * R = B*Hkv rows; codes row r = (b, hkv) at codes + b*cs_b + hkv*cs_h. */
int lap_retrieve_workspace_size(int R, int T, size_t* bytes);
/* The two halves of lap_retrieve_topk, for callers that time or overlap them:
 * lap_retrieve_score runs the scorer and leaves group keys and level-1
 * histograms in the workspace; lap_retrieve_select (same workspace, same
 * B/Hkv/T/window, on the same stream afterwards) emits the indices. */
int lap_retrieve_score(const void* lut_gmkg, const uint8_t* codes,
                       int64_t codes_stride_b, int64_t codes_stride_h,
                       int64_t codes_stride_t, int B, int Hkv, int T,
                       int cand_start, int cand_end, int key_mode,
                       void* scores_out, void* workspace, size_t workspace_bytes,
                       lap_stream_t stream);
int lap_retrieve_select(int B, int Hkv, int T, int cand_start, int cand_end, int k,
                        void* out_idx, int out_dtype, void* workspace,
                        size_t workspace_bytes, lap_stream_t stream);
/* lap_retrieve_select after a lap_retrieve_score with LAP_SELECT_PER_HEAD:
 * one top-k per query head, out_idx [B][Hkv*4][k] (replaces the per-head
 * torch.topk, aq_evaluation.py:198-201). */
int lap_retrieve_select_heads(int B, int Hkv, int T, int cand_start, int cand_end, int k,
                              void* out_idx, int out_dtype, void* workspace,
                              size_t workspace_bytes, lap_stream_t stream);
int lap_retrieve_topk(const void* lut_gmkg, const uint8_t* codes,
                      int64_t codes_stride_b, int64_t codes_stride_h,
                      int64_t codes_stride_t, int B, int Hkv, int T,
                      int cand_start, int cand_end, int k, int key_mode,
                      void* scores_out, void* out_idx, int out_dtype,
                      void* workspace, size_t workspace_bytes,
                      lap_stream_t stream);

/* Ragged forms of lap_retrieve_topk and lap_topk_select (no counterpart in
 * the reference, which has one length per batch; they replace the same
 * torch.topk call, aq_evaluation.py:198-201, once per sequence).
 * Row r belongs to sequence r / rows_per_plan (lap_retrieve_topk_ragged:
 * rows_per_plan = Hkv).  T bounds the columns scored and read: every plan is
 * clamped to [0, T).  Row r writes out[r][0..k_r) as the uniform call would
 * for its own window and budget, k_r = min(plan.k, window size, k_cols), and
 * sets out[r][k_r..k_cols) to -1.  Scores past a row's t_codes are not
 * written.  Workspaces: lap_retrieve_workspace_size(B*Hkv, T) and
 * lap_topk_workspace_size(R, T). */
int lap_retrieve_topk_ragged(const void* lut_gmkg, const uint8_t* codes,
                             int64_t codes_stride_b, int64_t codes_stride_h,
                             int64_t codes_stride_t, int B, int Hkv, int T,
                             const lap_row_plan* plans, int k_cols, int key_mode,
                             void* scores_out, void* out_idx, int out_dtype,
                             void* workspace, size_t workspace_bytes,
                             lap_stream_t stream);
int lap_topk_select_ragged(const void* scores, int64_t score_row_stride,
                           int R, int group, int rows_per_plan, int T,
                           const lap_row_plan* plans, int k_cols, int key_mode,
                           void* out_idx, int out_dtype,
                           void* workspace, size_t workspace_bytes,
                           lap_stream_t stream);

/* ======================================================================= *
 * A4  Native-GQA K/V gather                                                *
 * Replaces: gqa_gather_kv and gqa_gather_kv_with_tail,
 *   aq_kernels/aq_lut_gqa.cu:536-604 and :606-664 (kernels :222-323).
 *   keys, vals  [B][Hkv][T][D] with strides (sb, sh, st, 1), f16 or bf16
 *   indices     int64 [B][Hq][explicit_N] contiguous
 *   out_k/out_v [B][Hq][N][D] contiguous, N = explicit_N + tail_count;
 *   row n < explicit_N copies token indices[b,hq,n]; row explicit_N + j
 *   copies token tail_start + j.  Rows whose token is outside [0,T) are
 *   left unwritten.  tail_start < 0 means no tail (tail_count must be 0).
 * ======================================================================= */
int lap_gqa_gather_kv(const void* keys, const void* vals, int dtype,
                      int B, int Hkv, int T, int D,
                      int64_t k_sb, int64_t k_sh, int64_t k_st,
                      int64_t v_sb, int64_t v_sh, int64_t v_st,
                      const int64_t* indices, int Hq, int explicit_N,
                      int tail_start, int tail_count,
                      void* out_k, void* out_v, lap_stream_t stream);

/* ======================================================================= *
 * A5  Sparse-attention decode with the gather fused in                    *
 * Replaces: the gather at aq_evaluation.py:243-247 plus
 *   F.scaled_dot_product_attention(Q_rope, K_sel, V_sel) at :251; native
 *   model aq_kernels/aq_lut.cu:195-324 (sparse_attn_q1_kernel).
 * For each batch b and query head h, over the keep list
 *   L(b,h) = indices[b, row(h), 0..n_idx) ++ [0, sink_count)
 *            ++ [tail_start, tail_start + tail_count)
 * with row(h) = h / (Hq / H_idx) (H_idx = Hq: per-head lists, H_idx = Hkv:
 * one list per KV group):
 *   o[b,h] = sum_j softmax_j(scale * q[b,h].K[b,h/G,L_j]) V[b,h/G,L_j]
 * in fp32, written in the q dtype.  Indices outside [0,T) are skipped.
 *   q     [B][Hq][D] with row strides (q_sb, q_sh), f16/bf16
 *   K/V   [B][Hkv][T][D] strides (sb, sh, st, 1), same dtype as q
 *   indices int32 or int64 [B][H_idx][n_idx] contiguous (may be NULL if
 *           n_idx == 0)
 *   out   [B][Hq][D] contiguous, q dtype
 * ======================================================================= */
/* Workspace of the two decode entry points: the fp32 split partials
 * (m, l, o) the combine kernel merges.  Calls that share a workspace must be
 * ordered (same stream). */
int lap_attn_decode_workspace_size(int B, int Hq, int D, int max_keys, size_t* bytes);
int lap_sparse_attn_decode(const void* q, int64_t q_sb, int64_t q_sh,
                           const void* keys, const void* vals, int dtype,
                           int B, int Hq, int Hkv, int T, int D,
                           int64_t k_sb, int64_t k_sh, int64_t k_st,
                           int64_t v_sb, int64_t v_sh, int64_t v_st,
                           const void* indices, int idx_dtype, int H_idx,
                           int n_idx, int sink_count,
                           int tail_start, int tail_count, float scale,
                           void* out, void* workspace, size_t workspace_bytes,
                           lap_stream_t stream);

/* Dense single-query decode over all T tokens (flash-decode, split-K).
 * Replaces: laprune/attention.py:62-65 (SDPA with num_queries == 1, native
 * GQA).  Same argument meaning as lap_sparse_attn_decode with the keep list
 * [0, T). */
int lap_dense_attn_decode(const void* q, int64_t q_sb, int64_t q_sh,
                          const void* keys, const void* vals, int dtype,
                          int B, int Hq, int Hkv, int T, int D,
                          int64_t k_sb, int64_t k_sh, int64_t k_st,
                          int64_t v_sb, int64_t v_sh, int64_t v_st,
                          float scale, void* out,
                          void* workspace, size_t workspace_bytes,
                          lap_stream_t stream);

/* Ragged form of lap_sparse_attn_decode (no counterpart in the reference,
 * which has one length per batch; it replaces the same gather + SDPA,
 * aq_evaluation.py:243-251, once per sequence).  Sequence b attends over
 *   indices[b, row(h), 0..k_cols) ++ [0, plans[b].sink)
 *   ++ [plans[b].tail_start, + plans[b].tail_count)
 * skipping index entries < 0 (the padding of the ragged top-k) and rows
 * outside [0, min(plans[b].t_total, T)).  max_sink and max_tail bound every
 * plan's sink and tail_count (they size the split-K grid; a plan above them
 * is clamped).  With k_cols = 0, sink = 0 and tail [0, t_total) this is the
 * dense decode of each sequence.  Workspace:
 * lap_attn_decode_workspace_size(B, Hq, D, k_cols + max_sink + max_tail). */
int lap_sparse_attn_decode_ragged(const void* q, int64_t q_sb, int64_t q_sh,
                                  const void* keys, const void* vals, int dtype,
                                  int B, int Hq, int Hkv, int T, int D,
                                  int64_t k_sb, int64_t k_sh, int64_t k_st,
                                  int64_t v_sb, int64_t v_sh, int64_t v_st,
                                  const void* indices, int idx_dtype, int H_idx,
                                  int k_cols, const lap_row_plan* plans,
                                  int max_sink, int max_tail, float scale,
                                  void* out, void* workspace, size_t workspace_bytes,
                                  lap_stream_t stream);

/* ======================================================================= *
 * A2 + A3 + A4 + A5  One decode step after the LUT                         *
 * Replaces the chain of _decode_attention for one layer and one token,     *
 *   laprune/llm/modifiers/aq_evaluation.py:146-253: grouped LUT scoring    *
 *   (aq_kv.py:684 -> aq_kernels/aq_lut_gqa.cu:460-534), the candidate      *
 *   window and torch.topk (aq_evaluation.py:185-205), the keep set         *
 *   (:210-237), the K/V gather (aq_lut_gqa.cu:606-664) and SDPA (:251).    *
 * ======================================================================= *
 * Same results as lap_retrieve_topk (lap_retrieve_topk_ragged when plans is
 * non-NULL) followed by lap_sparse_attn_decode (_ragged) with H_idx = Hkv
 * (or Hq with LAP_SELECT_PER_HEAD): the selected indices in out_idx
 * [B][rows][k] (ragged: [B][rows][k_cols], padded with -1) and the attention
 * output in out [B][Hq][D].  Uniform calls pass the window, budget, sink and
 * tail as scalars (k is clamped to the window; k_cols, max_sink and max_tail
 * are ignored); ragged calls read them per sequence from plans.
 *   codes  u8 [B][Hkv][>=T][32] strides (b, h, t, 1), 16-byte aligned (may
 *          be NULL when the call selects nothing: k = 0, or k_cols = 0)
 *   T      code columns scored (the grid; plans clamp to it), T_kv K/V rows
 *   q, K, V as lap_sparse_attn_decode; G = Hq / Hkv from 1 to 8
 *   lut_gmkg  fp16 LUT of the B * Hq query heads: G = 4, LAP_LUT_GMKG
 *          [B * Hkv][32][256][4]; other G, LAP_LUT_HMK [B * Hq][32][256]
 * With G = 4 and D = 128, group and per-head selection run as one launch
 * (per KV row, the workgroups of one XCD score, select and attend, and the
 * last merges); other shapes run the kernel chain (G = 4: lap_retrieve_topk;
 * other G: lap_lut_score_gqa of every head, then lap_topk_select (_ragged)
 * over the group max or each head's row; then the sparse attention).
 * Workspace: lap_decode_step_workspace_size
 * with keep_max = k + sink + tail (ragged: k_cols + max_sink + max_tail).  It
 * must be zero-filled once before its first use; every call leaves its
 * barrier words and histograms at zero again.  Their layout does not depend
 * on the call (it is laid out for 256 KV rows), so a workspace sized for
 * the largest batch serves every smaller one.  Calls that share a workspace
 * must be ordered (same stream). */
int lap_decode_step_workspace_size(int B, int Hq, int Hkv, int T, int D, int keep_max,
                                   int key_mode, size_t* bytes);
int lap_decode_step(const void* lut_gmkg, const uint8_t* codes,
                    int64_t codes_stride_b, int64_t codes_stride_h, int64_t codes_stride_t,
                    int T, int cand_start, int cand_end, int k,
                    int sink_count, int tail_start, int tail_count,
                    const lap_row_plan* plans, int k_cols, int max_sink, int max_tail,
                    int key_mode,
                    const void* q, int64_t q_sb, int64_t q_sh,
                    const void* keys, const void* vals, int dtype,
                    int B, int Hq, int Hkv, int T_kv, int D,
                    int64_t k_sb, int64_t k_sh, int64_t k_st,
                    int64_t v_sb, int64_t v_sh, int64_t v_st, float scale,
                    void* out_idx, int idx_dtype, void* out,
                    void* workspace, size_t workspace_bytes, lap_stream_t stream);
/* Health counters of the one-launch step in a lap_decode_step workspace
 * (copied to the host, synchronising): rows whose workgroups did not all run
 * on one XCD (their exchange through that XCD's L2 then has no guarantee),
 * and barrier spins that gave up.  Both stay zero on a healthy device; a
 * non-zero count means the calls since the workspace was zeroed are not to
 * be trusted. */
int lap_decode_step_status(const void* workspace, size_t workspace_bytes,
                           uint32_t* split_rows, uint32_t* timeouts);
/* lap_decode_step without a workspace: no counterpart in the reference.  For
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments,
 * results and errors as lap_decode_step, minus the workspace; the step's
 * scratch is a static device array of 64 MiB per GPU (held by every GPU the
 * library runs on until the process ends), its row barriers and histograms
 * laid out for B * Hkv <= 256 KV rows.  Shapes that need more scratch than
 * that (or more rows) fail with LAP_ERR_WORKSPACE; nothing is allocated.
 * Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (different streams, or other threads) race and must not be issued. */
int lap_decode_step_noalloc(const void* lut_gmkg, const uint8_t* codes,
                            int64_t codes_stride_b, int64_t codes_stride_h,
                            int64_t codes_stride_t,
                            int T, int cand_start, int cand_end, int k,
                            int sink_count, int tail_start, int tail_count,
                            const lap_row_plan* plans, int k_cols, int max_sink, int max_tail,
                            int key_mode,
                            const void* q, int64_t q_sb, int64_t q_sh,
                            const void* keys, const void* vals, int dtype,
                            int B, int Hq, int Hkv, int T_kv, int D,
                            int64_t k_sb, int64_t k_sh, int64_t k_st,
                            int64_t v_sb, int64_t v_sh, int64_t v_st, float scale,
                            void* out_idx, int idx_dtype, void* out, lap_stream_t stream);
/* Health counters of lap_decode_step_noalloc's static scratch on the current
 * device (the two words lap_decode_step_status reads from a workspace), read
 * after a device synchronisation; zeros before the first call on the
 * device.  No counterpart in the reference. */
int lap_decode_step_noalloc_status(uint32_t* split_rows, uint32_t* timeouts);
/* Zero the static scratch's counters, row barriers and row histograms on
 * the current device (a fill kernel on `stream`, nothing allocated): the
 * reset after a call whose counters came back non-zero.  No counterpart in
 * the reference. */
int lap_decode_step_noalloc_reset(lap_stream_t stream);

/* ======================================================================= *
 * A6  Greedy AQ encode                                                     *
 * Replaces: fused_linear_encode_forward, aq_kernels/fused_linear_encode.cu:
 *   168-234 (kernel :34-102), called from laprune/llm/aq_kv.py:44-75; the
 *   contract followed is the fp32 greedy path of laprune/quantizer.py:
 *   346-355 (_batch_icm_lut, iters = 0):
 *     r = x; for m: dist_k = (rn + cn[m,k]) - 2*dot(r, C[m,k]);
 *     code_m = lowest k with minimal dist; r = r - C[m,code_m]
 *   with dot/rn/cn all computed by dot16: 16 fmaf chains over consecutive
 *   blocks (chain j sums d = j*L .. j*L+L-1 in order, L = D/16, from 0),
 *   folded pairwise s[j] += s[j+w] for w = 8, 4, 2, 1.  Requires
 *   D % 16 == 0, K <= 256.
 * lap_encode_prepare fills prep (size lap_encode_prep_size) from the
 * codebooks once; lap_encode_greedy then encodes N rows.
 *   x          [N][D] fp32 with row stride x_row_stride
 *   codebooks  [M][K][D] fp32 contiguous
 *   codes_out  u8 [N][M] with row stride codes_row_stride
 *   resid_norm fp32 [N] (sqrtf(rn_final)), may be NULL
 * ======================================================================= */
int lap_encode_prep_size(int M, int K, int D, size_t* bytes);
int lap_encode_prepare(const float* codebooks, int M, int K, int D,
                       void* prep, size_t prep_bytes, lap_stream_t stream);
int lap_encode_greedy(const float* x, int64_t x_row_stride, int N, int D,
                      const float* codebooks, int M, int K,
                      const void* prep, size_t prep_bytes,
                      uint8_t* codes_out, int64_t codes_row_stride,
                      float* resid_norm, lap_stream_t stream);

/* Replaces: the encode of the not-yet-encoded key tail in _prepare_aq_cache,
 *   laprune/llm/modifiers/aq_evaluation.py:367-405 (codes[:, :, encoded_len:
 *   seq_len] = encode_keys_batch(keys[:, :, encoded_len:seq_len]), through
 *   laprune/llm/aq_kv.py:390-428), and its prefill form (:430-447).
 * Same contract as lap_encode_greedy, with the rows taken straight from a
 * strided key cache and the codes written straight into a strided code cache:
 * for every (b, h) and t in [t0, t1), keys[b, h, t, :] -> codes[b, h, t, :].
 *   keys       f32/f16/bf16 [B][Hkv][T][D], strides (k_sb, k_sh, k_st, 1)
 *   codes      u8 [B][Hkv][Tcap][M], strides (c_sb, c_sh, c_st, 1)
 *   resid_norm fp32 [B*Hkv*(t1-t0)] in (b, h, t) order, may be NULL */
int lap_encode_keys(const void* keys, int key_dtype,
                    int64_t k_sb, int64_t k_sh, int64_t k_st,
                    int B, int Hkv, int t0, int t1, int D,
                    const float* codebooks, int M, int K,
                    const void* prep, size_t prep_bytes,
                    uint8_t* codes, int64_t c_sb, int64_t c_sh, int64_t c_st,
                    float* resid_norm, lap_stream_t stream);

/* Per-sequence form of lap_encode_keys for decode steps that replay one
 * captured graph: the token range of sequence b is read from device memory,
 * ranges[2b] .. ranges[2b+1] (empty when the sequence has no full encode
 * buffer this step), at most max_len tokens (the decode group size).  Replaces
 * the same tail encode, aq_evaluation.py:367-405, done per sequence.  t_cap is
 * the token capacity of both buffers: a range is clipped to [0, t_cap), so no
 * range read from memory can address outside them.  Rows past a range are not
 * touched; workgroups with no row in range exit at once.  No residual norms. */
int lap_encode_keys_ranges(const void* keys, int key_dtype,
                           int64_t k_sb, int64_t k_sh, int64_t k_st,
                           int B, int Hkv, const int32_t* ranges, int max_len, int t_cap, int D,
                           const float* codebooks, int M, int K,
                           const void* prep, size_t prep_bytes,
                           uint8_t* codes, int64_t c_sb, int64_t c_sh, int64_t c_st,
                           lap_stream_t stream);

/* Decode-step rotary embedding and cache append, one token per sequence:
 * HF apply_rotary_pos_emb (rotate_half convention) as aq_evaluation.py:296-305
 * applies it to the step's q and k, and the cache write of _kv_cache_append
 * (aq_evaluation.py:65-112), in one launch.  Arithmetic as torch's in the
 * model dtype: rnd(rnd(x * cos) + rnd(rotate_half(x) * sin)), bit-identical.
 *   q   [B][Hq][D]  strides (q_sb, q_sh, 1);  k, v [B][Hkv][D] likewise
 *   cos, sin [B][D] stride cs_sb, same dtype (fp16/bf16)
 *   pos int64 [B] device positions; cache rows at pos >= t_cap (or < 0) are
 *       not written
 * Writes rope(q) to q_out [B][Hq][D] (contiguous), rope(k) to
 * cache_k[b][h][pos[b]] and v to cache_v[b][h][pos[b]]. */
int lap_rope_append(const void* q, int64_t q_sb, int64_t q_sh,
                    const void* k, int64_t k_sb, int64_t k_sh,
                    const void* v, int64_t v_sb, int64_t v_sh,
                    const void* cos, const void* sin, int64_t cs_sb, int dtype,
                    int B, int Hq, int Hkv, int D, const int64_t* pos,
                    void* cache_k, int64_t ck_sb, int64_t ck_sh, int64_t ck_st,
                    void* cache_v, int64_t cv_sb, int64_t cv_sh, int64_t cv_st,
                    int t_cap, void* q_out, lap_stream_t stream);

/* ======================================================================= *
 * Diagnostics: measurement kernels (no counterpart in the reference; not  *
 * on the path and never called by it).                                    *
 * They time what the fused G = 4 scorer's launch shape costs before any   *
 * scoring: bench.py reports them beside the scorer.  Both take the        *
 * scorer's grid for R KV rows of T tokens (R * ceil(T / 4096) workgroups   *
 * of 1024 threads).                                                        *
 * lap_floor_empty: no work, the scorer's 68 KiB of LDS per workgroup.      *
 * lap_floor_stream: the scorer's reads without its lookups and adds: each  *
 *   workgroup copies row r's 64 KiB GMKG table (lut + r * 32768 fp16) into *
 *   LDS and reads the 32-byte code rows codes + r * cs_r + t * cs_t of its  *
 *   4096 tokens (t clamped to T - 1), `ahead` (1 or 4) of its four         *
 *   1024-token stages in flight.  out[i] (u32, one per workgroup) is the    *
 *   XOR of every 32-bit word the workgroup read.                           *
 * ======================================================================= */
int lap_floor_empty(int R, int T, lap_stream_t stream);
int lap_floor_stream(const void* lut, const void* codes, int64_t cs_r, int64_t cs_t,
                     int R, int T, int ahead, uint32_t* out, lap_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* LAPRUNE_HIP_H */
