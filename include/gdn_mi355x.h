/*
 * gdn_mi355x.h -- C ABI of the MI355X (gfx950) Gated DeltaNet hot-path library
 * (libgdn_mi355x.so).
 *
 * Every entry point takes plain device pointers, sizes and element strides, launches HIP kernels
 * on the given stream (a hipStream_t passed as void*; NULL = the legacy default stream), never
 * allocates, never synchronises the host, and is therefore safe inside hipGraph stream capture.
 * Tensors are dense row-major unless a stride argument says otherwise; strides are in elements.
 *
 * Dtype codes: GDN_F32 = 0, GDN_BF16 = 1, GDN_F16 = 2 (IEEE half; taken by gdn_chunk_prefill_generic
 * only).  bf16 is stored as the upper 16 bits of an IEEE fp32.
 * Return value: 0 on success, otherwise a GDN_E* code; gdn_last_error() then returns a message
 * (thread-local, valid until the next call on the same thread).
 *
 * Each declaration names the reference function it replaces (file:line in the reference
 * repository; "HF:" = transformers models/qwen3_5/modeling_qwen3_5.py, the third-party module the
 * reference patches).
 */
#ifndef GDN_MI355X_H
#define GDN_MI355X_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { GDN_F32 = 0, GDN_BF16 = 1, GDN_F16 = 2 };
enum {
  GDN_OK = 0,
  GDN_EINVAL = 1,   /* bad shape, dtype, stride, alignment or null pointer */
  GDN_EUNSUP = 2,   /* valid but not supported by this build (e.g. head_dim != 128) */
  GDN_ELAUNCH = 3   /* the HIP launch failed; the message carries hipGetErrorString */
};

/* Library version (major*10000 + minor*100 + patch). */
int gdn_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char* gdn_last_error(void);

/* Limits of this build: writes head_dim (128), max value heads per key head, max conv kernel. */
int gdn_limits(int* head_dim, int* max_group_ratio, int* max_conv_kernel);


/*
 * Single-token recurrent gated delta rule (decode), fp32 state.
 * Replaces recurrent_single_step (src/recurrent_single_step.py:8-32) for T == 1.
 *   q, k      [N, Hqk, D]  (dtype in_dtype), row (token) stride q_stride / k_stride; value head h
 *                          reads key head h / (Hv / Hqk) (Hqk == Hv for repeat_interleave'd input)
 *   v         [N, Hv, D]   (in_dtype), row stride v_stride
 *   g         [N, Hv] fp32 (log decay), beta [N, Hv] (beta_dtype)
 *   state_in  [N, Hv, D, D] fp32 (dk rows, dv columns), NULL = zero state
 *   state_out [N, Hv, D, D] fp32, may equal state_in (in-place update), NULL = do not write
 *   out       [N, Hv, D] (in_dtype)
 *   use_qk_l2norm: apply l2norm(x)=x*rsqrt(sum x^2 + 1e-6) to q, k in in_dtype first.
 */
int gdn_recurrent_step(const void* q, int64_t q_stride, const void* k, int64_t k_stride,
                       const void* v, int64_t v_stride, const float* g, const void* beta,
                       int beta_dtype, const float* state_in, float* state_out, void* out,
                       int N, int Hqk, int Hv, int D, int in_dtype, int use_qk_l2norm,
                       void* stream);

/*
 * Decode depthwise causal conv update with SiLU, conv state shifted in place.
 * Replaces elem_conv_update (src/cb_engine.py:43-51); same contract as HF causal_conv1d_update
 * with activation "silu" (HF:200-217).
 *   x      [N, C] bf16, row stride x_stride;  state [N, C, K] bf16 (in place)
 *   weight [C, K] bf16;  bias [C] bf16 or NULL;  out [N, C] bf16, row stride out_stride
 */
int gdn_conv_update(const void* x, int64_t x_stride, void* state, const void* weight,
                    const void* bias, void* out, int64_t out_stride, int N, int C, int K,
                    void* stream);

/*
 * Gated RMSNorm: out = silu(gate) * (weight * bf16(x * rsqrt(mean(x^2) + eps))), HF order.
 * Replaces Qwen3_5RMSNormGated.forward (HF:175-184) / fused_gated_rmsnorm (src/cb_engine.py:65-67).
 *   x, gate, out [rows, D] bf16 (row strides x_stride, gate_stride; out dense);
 *   weight [D] (w_dtype: GDN_BF16 or GDN_F32).
 */
int gdn_gated_rmsnorm(const void* x, int64_t x_stride, const void* gate, int64_t gate_stride,
                      const void* weight, int w_dtype, void* out, int64_t rows, int D, float eps,
                      void* stream);

/*
 * Fused GDN decode layer core for N slots x 1 token (everything between the input projections
 * and out_proj of CBEngine._gdn, src/cb_engine.py:318-351, with --elem-conv):
 *   conv update + SiLU (conv_state shifted in place) -> split q|k|v -> beta = sigmoid(b),
 *   g = -exp(A_log) * softplus(a + dt_bias) -> l2norm(q), l2norm(k) -> recurrent step with value
 *   head h reading key head h / (Hv/Hk) -> rec_state updated in place -> gated RMSNorm with z.
 *   mixed   [N, C] bf16 (pre-conv in_proj_qkv output, channels q(Hk*D) | k(Hk*D) | v(Hv*D)),
 *           row stride mixed_stride;  C = (2*Hk + Hv) * D
 *   z       [N, Hv*D] bf16 row stride z_stride (8-byte aligned, z_stride % 4 == 0);
 *           a, b [N, Hv] bf16 row strides ab_stride
 *   conv_state [N, C, K] bf16 (in place);  conv_w [C, K] bf16;  conv_b [C] bf16 or NULL
 *   A_log, dt_bias [Hv] fp32;  norm_w [D] (norm_w_dtype; 8-byte aligned bf16 / 16-byte fp32)
 *   rec_state [N, Hv, D, D] fp32 (in place, 16-byte aligned);  out [N, Hv*D] bf16 (the normed
 *           core, 8-byte aligned)
 */
int gdn_decode_fused(const void* mixed, int64_t mixed_stride, const void* z, int64_t z_stride,
                     const void* a, const void* b, int64_t ab_stride, void* conv_state,
                     const void* conv_w, const void* conv_b, const float* A_log,
                     const float* dt_bias, const void* norm_w, int norm_w_dtype, float eps,
                     float* rec_state, void* out, int N, int Hk, int Hv, int D, int K,
                     void* stream);

/*
 * (I - X)^{-1} for a batch of strictly lower-triangular 64x64 fp32 matrices (only the strictly
 * lower part of X is read), by the routine the chunked prefill's inverse kernel runs (reg_inv64:
 * the four 16x16 diagonal blocks by forward substitution, the blocks below them on the fp32 MFMA,
 * in registers, one wave per matrix).
 * Replaces _unit_lower_inv / _small_unit_lower_inv (src/gdn_chunk_fast.py:21-62).
 *   X, T [batch, 64, 64] fp32, 16-byte aligned;  n must be 64.
 */
int gdn_unit_lower_inv(const float* X, float* T, int64_t batch, int n, void* stream);

/*
 * The chunked prefill's first kernel alone (gdn_chunk_prefill's arguments for k, g, beta and the
 * sequence table; bf16 keys, D = 128): for every (chunk, value head) the T diag(beta) it hands to
 * the output pass, expanded to dense fp32 (t_out [total_chunks, Hv, 64, 64]: row i, column j =
 * T[i][j] beta_j of the chunk's X = -(beta_i k_i.k_j e^{G_i - G_j})_{i>j}, T = (I - X)^{-1}, as the
 * bf16 value stored), and with use_qk_l2norm the K rows' l2norm factors bf16(rsqrt(...))
 * (factor_out [total_chunks, Hv, 64] or NULL).  Chunks are numbered as seq_chunk0 numbers them.
 * The state-independent part of src/gdn_chunk_fast2.py:31-43 (attn = _unit_lower_inv(X), times
 * diag(beta) as v_beta and k_beta carry it); it exposes what the hot path computes so that it can
 * be checked on its own.  workspace: gdn_chunk_prefill_workspace_bytes(total_chunks, nseq, Hv).
 */
int gdn_chunk_prefill_inverse(const void* k, int64_t k_stride, const float* g, const void* beta,
                              int beta_dtype, int64_t total_tokens, const int32_t* cu_seqlens,
                              const int32_t* seq_chunk0, int64_t total_chunks, int nseq, int seq_len,
                              int Hqk, int Hv, int D, int in_dtype, int use_qk_l2norm, float* t_out,
                              float* factor_out, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Chunked gated delta rule for any head dims and input dtype, in fp32 throughout (fp32 MFMA):
 * fast_chunk_gated_delta_rule_v2 (src/gdn_chunk_fast2.py:11-62) takes any float dtype, d_k and
 * d_v; this is that general form (gdn_chunk_prefill takes it for everything but bf16 q/k/v with
 * D = 128, which has the segment-parallel kernels).  It walks each sequence's 64-token chunks in
 * order, one workgroup per (sequence, value head, 64 value columns); no workspace.
 *   q, k [total_tokens, Hqk, Dk], v [total_tokens, Hv, Dv] in in_dtype (GDN_F32, GDN_BF16 or
 *   GDN_F16), token strides q_stride / k_stride / v_stride;  Dk, Dv in {16, 32, 64, 128};
 *   g [total_tokens, Hv] fp32;  beta [total_tokens, Hv] (beta_dtype: GDN_F32, GDN_BF16, GDN_F16);
 *   initial_state / final_state [n_rows, Hv, Dk, Dv] fp32 or NULL, rows as gdn_chunk_prefill_rows
 *   (state_rows NULL: row s, n_rows = nseq);  out [total_tokens, Hv, Dv] in in_dtype (dense);
 *   cu_seqlens device int32 [nseq+1] or NULL (nseq sequences of seq_len tokens).
 *   use_qk_l2norm: q, k l2-normalised in in_dtype first (each op rounded to in_dtype, as torch).
 */
int gdn_chunk_prefill_generic(const void* q, int64_t q_stride, const void* k, int64_t k_stride,
                              const void* v, int64_t v_stride, const float* g, const void* beta,
                              int beta_dtype, const float* initial_state, float* final_state,
                              const int32_t* state_rows, int n_rows, void* out, int64_t total_tokens,
                              const int32_t* cu_seqlens, int nseq, int seq_len, int Hqk, int Hv, int Dk,
                              int Dv, int in_dtype, int use_qk_l2norm, void* stream);

/*
 * Bytes of device workspace gdn_chunk_prefill needs for `total_chunks` 64-token chunks of `nseq`
 * sequences and Hv value heads (-1 for bad sizes): the segment table and flags (a few bytes per
 * sequence and per segment), the fp32 transition maps of the segments that have a successor (at
 * most 32 MiB: sequences are cut into segments so that at most about 256 (segment, value head)
 * items exist) and the intra-chunk inverse's output (10.5 KiB per (chunk, value head): T diag(beta) as
 * bf16 hi + lo, the K row factors, g and a flag).
 */
int64_t gdn_chunk_prefill_workspace_bytes(int64_t total_chunks, int nseq, int Hv);

/*
 * Chunked gated delta rule prefill (chunk 64, fp32 state), optionally over packed sequences.
 * Replaces fast_chunk_gated_delta_rule_v2 (src/gdn_chunk_fast2.py:11-62) and
 * fast_chunk_gated_delta_rule (src/gdn_chunk_fast.py:65-142), both with HF's signature
 * torch_chunk_gated_delta_rule (HF:249-260).
 *   q, k [total_tokens, Hqk, D] bf16, token stride q_stride / k_stride (value head h reads key
 *        head h / (Hv / Hqk));  v [total_tokens, Hv, D] bf16, token stride v_stride
 *        (other dtypes and D in {16, 32, 64}: the call runs gdn_chunk_prefill_generic, and the
 *        chunk table and workspace arguments are not used)
 *   g [total_tokens, Hv] fp32 (log decay);  beta [total_tokens, Hv] (beta_dtype)
 *   initial_state / final_state [nseq, Hv, D, D] fp32, 16-byte aligned, either may be NULL
 *     (zero / not written)
 *   out [total_tokens, Hv, D] bf16 (dense)
 *   cu_seqlens: device int32 [nseq+1] (packed varlen) with seq_chunk0: device int32 [nseq+1],
 *     seq_chunk0[s] = sum over earlier sequences of ceil(len/64); or both NULL for nseq
 *     sequences of seq_len tokens.  total_chunks = sum of ceil(len/64) over sequences.  With
 *     cu_seqlens, seq_len is 0 or an upper bound of every sequence's length: when no sequence can
 *     span more than one segment the call skips the segment summaries (one launch).  A bound
 *     below a sequence's true length gives wrong results for that sequence.
 *   workspace: device memory of gdn_chunk_prefill_workspace_bytes(total_chunks, nseq, Hv) bytes,
 *     256-byte aligned (caller-owned; contents are scratch).
 */
int gdn_chunk_prefill(const void* q, int64_t q_stride, const void* k, int64_t k_stride,
                      const void* v, int64_t v_stride, const float* g, const void* beta,
                      int beta_dtype, const float* initial_state, float* final_state, void* out,
                      int64_t total_tokens, const int32_t* cu_seqlens, const int32_t* seq_chunk0,
                      int64_t total_chunks, int nseq, int seq_len, int Hqk, int Hv, int D,
                      int in_dtype, int use_qk_l2norm, void* workspace, int64_t workspace_bytes,
                      void* stream);

/*
 * Depthwise causal conv prefill + SiLU over packed prompts, and the decode conv state they leave
 * (the last K inputs, left zero-padded).  Replaces the conv of TPEngine.prefill /
 * TPEngine.prefill_chunk (src/cb_tp.py:158-164, :236-244, :260) and HF causal_conv1d_fn with the
 * cache conv-state capture (HF:220-239).
 *   x [total_tokens, C] bf16 (token-major, row stride x_stride); weight [C, K] bf16; bias [C] or NULL
 *   history [nseq, C, K] bf16 (the previous K inputs of each sequence) or NULL (zero history)
 *   out [total_tokens, C] bf16 (dense);  state_out [nseq, C, K] bf16 or NULL
 *   cu_seqlens device int32 [nseq+1] or NULL (nseq sequences of seq_len tokens)
 */
int gdn_conv_prefill(const void* x, int64_t x_stride, const void* weight, const void* bias,
                     const void* history, void* out, void* state_out, int64_t total_tokens,
                     const int32_t* cu_seqlens, int nseq, int seq_len, int C, int K, void* stream);

/*
 * GDN gating: beta = sigmoid(b) (bf16), g = -exp(A_log) * softplus(a + dt_bias) (fp32).
 * Replaces src/cb_engine.py:337-338 (HF:497-498).
 *   a, b [rows, Hv] bf16 (row stride ab_stride); A_log, dt_bias [Hv] fp32;
 *   beta_out [rows, Hv] bf16; g_out [rows, Hv] fp32 (dense).
 */
int gdn_gating(const void* a, const void* b, int64_t ab_stride, const float* A_log,
               const float* dt_bias, void* beta_out, float* g_out, int64_t rows, int Hv,
               void* stream);

/*
 * Slot-row variants for a continuous-batching engine's state buffers.  The engine keeps one row per
 * slot: conv state [n_rows, C, K] bf16, recurrent state [n_rows, Hv, D, D] fp32
 * (src/cb_engine.py:108-112).
 */

/*
 * gdn_decode_fused for a dense step over all N slots where only some advance.  active [N] uint8
 * (device): nonzero = advance the slot; a zero slot's conv and recurrent state are left untouched
 * and its output rows are zero.  NULL = every slot advances (that is gdn_decode_fused).  Replaces
 * the save / restore of held slots around the dense decode step (src/cb_tp.py:274-285).
 */
int gdn_decode_fused_masked(const void* mixed, int64_t mixed_stride, const void* z, int64_t z_stride,
                            const void* a, const void* b, int64_t ab_stride, void* conv_state,
                            const void* conv_w, const void* conv_b, const float* A_log,
                            const float* dt_bias, const void* norm_w, int norm_w_dtype, float eps,
                            float* rec_state, void* out, const uint8_t* active, int N, int Hk, int Hv,
                            int D, int K, void* stream);

/*
 * gdn_chunk_prefill with the sequences' states in slot rows.  initial_state / final_state are
 * [n_rows, Hv, D, D] fp32 and sequence s reads and writes row state_rows[s] (device int32 [nseq]);
 * a row outside [0, n_rows) is neither read nor written (zero initial state, no final state).
 * initial_state and final_state may be the same buffer (a continuation chunk updates its slot in
 * place).  state_rows NULL: row s, and n_rows must equal nseq (that is gdn_chunk_prefill).
 * Replaces the slot copies after prefill, self.rec[i][slot] = last (src/cb_tp.py:179, :262;
 * src/cb_engine.py:198-205), and the continuation's initial_state = self.rec[i][slot]
 * (src/cb_tp.py:256).
 */
int gdn_chunk_prefill_rows(const void* q, int64_t q_stride, const void* k, int64_t k_stride,
                           const void* v, int64_t v_stride, const float* g, const void* beta,
                           int beta_dtype, const float* initial_state, float* final_state,
                           const int32_t* state_rows, int n_rows, void* out, int64_t total_tokens,
                           const int32_t* cu_seqlens, const int32_t* seq_chunk0, int64_t total_chunks,
                           int nseq, int seq_len, int Hqk, int Hv, int D, int in_dtype,
                           int use_qk_l2norm, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * gdn_chunk_prefill_rows whose output rows pass through the layer's gated RMSNorm before they are
 * stored: out[t, h] = gdn_gated_rmsnorm(o[t, h], z[t, h], norm_weight, eps), with o the rule's
 * output rounded to bf16 first -- bit for bit what the two calls in a row give.  Replaces the
 * rule's output write and the Qwen3_5RMSNormGated call that follows it in the GDN prefill layer
 * (src/cb_tp.py:171-176; HF:175-184), saving the output's round trip through HBM.
 *   z: gate rows [total_tokens, >= Hv * D] bf16, row stride z_stride elements (a multiple of 8),
 *      16-byte aligned; head h of token t at z + t * z_stride + h * D;
 *   norm_weight [D] (norm_w_dtype: GDN_BF16 or GDN_F32);  in_dtype must be GDN_BF16, D = 128.
 */
int gdn_chunk_prefill_rows_gated(const void* q, int64_t q_stride, const void* k, int64_t k_stride,
                                 const void* v, int64_t v_stride, const float* g, const void* beta,
                                 int beta_dtype, const float* initial_state, float* final_state,
                                 const int32_t* state_rows, int n_rows, void* out, int64_t total_tokens,
                                 const int32_t* cu_seqlens, const int32_t* seq_chunk0, int64_t total_chunks,
                                 int nseq, int seq_len, int Hqk, int Hv, int D, int in_dtype,
                                 int use_qk_l2norm, const void* z, int64_t z_stride, const void* norm_weight,
                                 int norm_w_dtype, float eps, void* workspace, int64_t workspace_bytes,
                                 void* stream);

/*
 * gdn_chunk_prefill_rows without a workspace argument and without any allocation: the kernels'
 * workspace is a static device array of GDN_NOALLOC_SCRATCH_BYTES (256 MiB) that the library holds on
 * every GPU it runs on until the process ends.  A call whose
 * gdn_chunk_prefill_workspace_bytes(total_chunks, nseq, Hv) exceeds it is rejected with GDN_EINVAL
 * before any launch (the workspace is at most about 32 MiB plus 10.5 KiB per (chunk, value head): 256 MiB
 * holds e.g. 44,416 tokens at Hv = 32).  Every
 * call on one GPU shares that GPU's array: calls that overlap on one GPU (other streams, other host
 * threads) race and give wrong results -- order them on one stream.  The array needs no clearing
 * (every record a call uses, the same call writes first).
 * No counterpart in the reference: for callers that cannot allocate (code under HIP graph capture,
 * serving loops, harnesses that forbid hipMalloc).
 */
#define GDN_NOALLOC_SCRATCH_BYTES (256ll << 20)
int gdn_chunk_prefill_noalloc(const void* q, int64_t q_stride, const void* k, int64_t k_stride,
                              const void* v, int64_t v_stride, const float* g, const void* beta,
                              int beta_dtype, const float* initial_state, float* final_state,
                              const int32_t* state_rows, int n_rows, void* out, int64_t total_tokens,
                              const int32_t* cu_seqlens, const int32_t* seq_chunk0, int64_t total_chunks,
                              int nseq, int seq_len, int Hqk, int Hv, int D, int in_dtype,
                              int use_qk_l2norm, void* stream);

/*
 * gdn_conv_prefill with history and decode conv state in slot rows [n_rows, C, K] bf16: sequence
 * s reads its history from row state_rows[s] and writes its new state there (rows outside
 * [0, n_rows): zero history, no state).  history and state_out may be the same buffer.
 * Replaces self.conv[i][slot] = conv_state / full_in[..., -K:] and the continuation's
 * prev = self.conv[i][slot] (src/cb_tp.py:178, :240, :260).
 */
int gdn_conv_prefill_rows(const void* x, int64_t x_stride, const void* weight, const void* bias,
                          const void* history, void* out, void* state_out, const int32_t* state_rows,
                          int n_rows, int64_t total_tokens, const int32_t* cu_seqlens, int nseq,
                          int seq_len, int C, int K, void* stream);

/*
 * The whole GDN prefill layer between the input projections and out_proj, for one or more packed
 * prompts (src/cb_tp.py:153-181 fresh, :230-263 continued): conv prefill + SiLU and the decode conv
 * state (gdn_conv_prefill_rows), split q | k | v, gating (gdn_gating), the chunked rule with l2norm,
 * value head h reading key head h / (Hv / Hk), and the gated RMSNorm
 * (gdn_chunk_prefill_rows_gated) -- the same results as those calls in a row, bit for bit, in
 * fewer launches: the conv, the state capture, the gating and the segment table share one launch.
 *   mixed [total_tokens, (2 Hk + Hv) D] bf16 (pre-conv in_proj_qkv rows), row stride mixed_stride
 *     (a multiple of 8, 16-byte aligned);  z [total_tokens, >= Hv D] bf16, row stride z_stride (a
 *     multiple of 8, 16-byte aligned);  a, b [total_tokens, Hv] bf16, row stride ab_stride;
 *   conv_w [(2 Hk + Hv) D, K] bf16 (16-byte aligned), conv_b [(2 Hk + Hv) D] bf16 or NULL;
 *   A_log, dt_bias [Hv] fp32;  norm_w [D] (norm_w_dtype GDN_BF16 or GDN_F32), eps;
 *   conv_history / conv_state: [n_rows, C, K] bf16 with state_rows (slot rows, as
 *     gdn_conv_prefill_rows; may be the same buffer), else [nseq, C, K]; conv_history NULL = zero;
 *   initial_state / final_state: [n_rows or nseq, Hv, D, D] fp32 as gdn_chunk_prefill_rows;
 *   out [total_tokens, Hv D] bf16 (the normed core);  cu_seqlens, seq_chunk0, total_chunks, nseq,
 *     seq_len as gdn_chunk_prefill;  D = 128, K <= 8;
 *   workspace: gdn_prefill_layer_workspace_bytes(total_tokens, total_chunks, nseq, Hk, Hv, D) bytes,
 *     256-byte aligned (the conv output, beta and g, then the chunked rule's workspace).
 */
int64_t gdn_prefill_layer_workspace_bytes(int64_t total_tokens, int64_t total_chunks, int nseq, int Hk,
                                          int Hv, int D);
int gdn_prefill_layer_rows(const void* mixed, int64_t mixed_stride, const void* z, int64_t z_stride,
                           const void* a, const void* b, int64_t ab_stride, const void* conv_w,
                           const void* conv_b, const float* A_log, const float* dt_bias,
                           const void* norm_w, int norm_w_dtype, float eps, const void* conv_history,
                           void* conv_state, const float* initial_state, float* final_state,
                           const int32_t* state_rows, int n_rows, void* out, int64_t total_tokens,
                           const int32_t* cu_seqlens, const int32_t* seq_chunk0, int64_t total_chunks,
                           int nseq, int seq_len, int Hk, int Hv, int D, int K, void* workspace,
                           int64_t workspace_bytes, void* stream);

/*
 * Decode-step projections: out[M, N] = x[M, K] W[N, K]^T, M <= 16 rows (one token per slot), bf16 x,
 * W (nn.Linear weight layout [out_features, in_features]) and out, fp32 accumulation.  Replaces the
 * GDN layer's in_proj_qkv / in_proj_z / in_proj_b / in_proj_a and out_proj calls of the decode step
 * (src/cb_engine.py:320-323, :352; torch nn.Linear on the reference's device); the rest of a decode
 * step's linears (attention, MLP, LM head) take it too.  K must be a multiple of 128; x and W rows
 * 16-byte aligned.  workspace: fp32, gdn_decode_linear_workspace_bytes(M, N, K) bytes (0: none is
 * needed -- K is split over workgroups, through the workspace, only when N is small).
 */
int64_t gdn_decode_linear_workspace_bytes(int M, int64_t N, int64_t K);
int gdn_decode_linear(const void* x, int64_t x_stride, const void* W, int64_t w_stride, void* out,
                      int64_t out_stride, int M, int64_t N, int64_t K, float* workspace,
                      int64_t workspace_bytes, void* stream);

/*
 * The same product on a weight packed once (at load time) by gdn_decode_linear_pack into the
 * kernel's fragment-major layout (gdn_decode_linear_packed_elems(N, K) bf16 values, rows padded to
 * a multiple of 16 with zeros), so that every weight load reads 1 KB contiguous.
 */
int64_t gdn_decode_linear_packed_elems(int64_t N, int64_t K);
int gdn_decode_linear_pack(const void* W, int64_t w_stride, void* packed, int64_t N, int64_t K, void* stream);
int gdn_decode_linear_packed(const void* x, int64_t x_stride, const void* packed, void* out, int64_t out_stride,
                             int M, int64_t N, int64_t K, float* workspace, int64_t workspace_bytes,
                             void* stream);

/*
 * Residual add + RMSNorm between the layers of a decode step (HF Qwen3_5RMSNorm: fp32
 * x * rsqrt(mean(x^2) + eps) * (1 + w), cast to bf16; the residual h + delta rounded to bf16 as
 * torch does).  h, delta, h_out, x_out [M, H] bf16 rows, w [H] bf16.  delta NULL: x_out = norm(h)
 * and h_out is not written; otherwise h_out = h + delta (h_out may be h) and x_out = norm(h_out).
 * Replaces the residual adds and the input / post-attention layernorms around each layer
 * (HF modeling_qwen3_5.py Qwen3_5DecoderLayer.forward) in the graph-captured decode step
 * (src/cb_engine.py:153-172).
 */
int gdn_add_rmsnorm(const void* h, const void* delta, const void* w, void* h_out, void* x_out, int M, int H,
                    float eps, void* stream);

/*
 * Split-K partial sums of a decode projection, for a consumer that reduces them itself (no reduction
 * launch, no bf16 round trip of the projection's output).  The reference's nn.Linear outputs
 * (o_proj / out_proj / mlp.down_proj feeding the residual add, mlp.gate_up feeding SwiGLU) are
 * exactly bf16(sum over splits, in split order) of these partials.
 *   gdn_decode_linear_splits: the number of K splits gdn_decode_linear(_packed) uses for (M, N, K).
 *   gdn_decode_linear_packed_partial: part [splits][M][N] fp32 (16-byte aligned, part_bytes >=
 *     splits * M * N * 4), written even with one split; otherwise as gdn_decode_linear_packed.
 *   gdn_add_rmsnorm_partial: gdn_add_rmsnorm with delta = bf16(sum of part [splits][M][H]);
 *     H % 8 == 0, H <= 8192, 16-byte aligned rows; h_out may alias h.
 *   gdn_swiglu_partial: out[M, m] = bf16(bf16(silu(g)) * u) with g, u = bf16(sum of part
 *     [splits][M][2m]) columns j and m + j (HF Qwen3_5MLP: act_fn(gate_proj(x)) * up_proj(x) with
 *     gate|up as one projection); m % 8 == 0, part and out 16-byte aligned.
 */
int gdn_decode_linear_splits(int M, int64_t N, int64_t K);
int gdn_decode_linear_packed_partial(const void* x, int64_t x_stride, const void* packed, float* part, int M,
                                     int64_t N, int64_t K, int64_t part_bytes, void* stream);
int gdn_add_rmsnorm_partial(const void* h, const float* part, int splits, const void* w, void* h_out, void* x_out,
                            int M, int H, float eps, void* stream);
int gdn_swiglu_partial(const float* part, int splits, void* out, int M, int64_t m, void* stream);

/*
 * GQA decode attention of the hybrid stack's full-attention layers, one new token for each of N
 * slots.  It has no counterpart inside the reference's GDN path: it is the attention layer the
 * reference's engine runs between its GDN layers, HF Qwen3_5Attention.forward
 * (transformers modeling_qwen3_5.py:629-700: gated q, q/k Qwen3_5RMSNorm, partial rotary,
 * softmax(q k^T / sqrt(hd)) v, times sigmoid(gate)), here in three launches on a per-slot cache.
 *   proj [N, proj_stride] bf16: per query head h its q (hd) then its gate (hd) at h * 2hd, then the
 *     kv key rows (hd each) at 2 nh hd, then the kv value rows at (2 nh + kv) hd.
 *   pos [N] int64 (device): the position of the new token; it is written to the caches there and
 *     attends to positions 0..pos.  The caller keeps 0 <= pos < T: a position >= T is not written and
 *     the attended range is clamped to T; a negative position writes nothing and gives a zero output.
 *   q_norm_w, k_norm_w [hd] bf16 (the norm multiplies by 1 + w); inv_freq [rd / 2] fp32 (the rotary
 *     angle of pair i is float(pos) * inv_freq[i], applied to the first rd dims).
 *   k_cache_t [N, kv, hd, T] bf16 (K transposed), v_cache [N, kv, T, hd] bf16; T % 4 == 0.
 *   out [N, out_stride] bf16: the gated attention output, nh * hd columns (o_proj's input).
 *   work: gdn_attn_decode_workspace_bytes(N, nh, hd, T) bytes, 256-byte aligned.
 * hd in {64, 128, 256}; nh / kv in {1, 2, 4, 6, 8}.  Scores and the softmax run in fp32; P V
 * multiplies bf16-rounded probabilities with bf16 V and accumulates in fp32.
 */
int64_t gdn_attn_decode_workspace_bytes(int N, int nh, int hd, int T);
int gdn_attn_decode(const void* proj, int64_t proj_stride, const int64_t* pos, const void* q_norm_w,
                    const void* k_norm_w, const float* inv_freq, void* k_cache_t, void* v_cache, void* out,
                    int64_t out_stride, float* work, int64_t work_bytes, int N, int nh, int kv, int hd, int rd, int T,
                    float eps, void* stream);
/* The same with the projection given as its split-K partial sums (gdn_decode_linear_packed_partial):
 * part [splits][N][(2 nh + 2 kv) hd] fp32; every value is bf16(sum over splits, in split order), as in
 * the reduced projection, so the result is identical and the reduction launch disappears. */
int gdn_attn_decode_partial(const float* part, int splits, const int64_t* pos, const void* q_norm_w,
                            const void* k_norm_w, const float* inv_freq, void* k_cache_t, void* v_cache, void* out,
                            int64_t out_stride, float* work, int64_t work_bytes, int N, int nh, int kv, int hd, int rd,
                            int T, float eps, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GDN_MI355X_H */
