/*
 * trida_hip.h — C ABI of the MI355X (gfx950) self-speculative decode step.
 *
 * Every entry point takes raw device pointers, int64 sizes and a hipStream_t passed as `void*`, and
 * enqueues its kernels on that stream. Conventions shared by all of them:
 *   - Ownership: the caller allocates every input, output and workspace buffer. No entry point
 *     allocates device memory, frees it, or synchronises the host.
 *   - Scratch: device memory of at least the size the matching `*_scratch_bytes` call returns.
 *     Scratch marked "zeroed" must be all-zero before its first use; the kernels leave it all-zero
 *     again when they finish, so one zeroing at allocation time suffices.
 *   - bf16 tensors are passed as `uint16_t*` holding the bf16 bit patterns.
 *   - Return value: 0 on success; TRIDA_ERR_* (< 0) on a rejected argument or a failed launch.
 *     trida_last_error() returns a message for the calling thread's last failure.
 *   - Stream-ordered and reentrant; calls that share a workspace must not overlap in time.
 * Layouts are row-major and contiguous unless a stride argument says otherwise.
 */
#ifndef TRIDA_HIP_H
#define TRIDA_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TRIDA_OK 0
#define TRIDA_ERR_ARG (-1)       /* bad shape / size / mode argument */
#define TRIDA_ERR_NULL (-2)      /* required pointer is NULL */
#define TRIDA_ERR_ALIGN (-3)     /* pointer or stride alignment the kernel needs is not met */
#define TRIDA_ERR_WORKSPACE (-4) /* workspace too small */
#define TRIDA_ERR_LAUNCH (-5)    /* HIP launch error */

/* Library version (major*10000 + minor*100 + patch) and the calling thread's last error message. */
int trida_version(void);
const char* trida_last_error(void);

/* ------------------------------------------------------------------------------------------------
 * Greedy self-spec acceptance.
 * Replaces the greedy branch of TridaDiffusionSampler._selfspec_step
 *   (inference/zoro-1/vllm/vllm_native_diffusion/qwen3_5_diffusion.py:906-914)
 * and the greedy verify of selfspec_generate (inference/zoro-1/mlx/trida_mlx/decode.py:323-332).
 *
 * logits   [B, R, V], dtype 0 = fp32 or 1 = bf16, element (b, r, x) at
 *          logits + b*batch_stride + r*row_stride + x (strides in elements). Row j (j < K) verifies
 *          draft j; row n_acc gives the bonus token (shift readout).
 * drafts   [B, K] int64 (row stride draft_stride); n_live [B] int32 or NULL (= K): draft j only counts
 *          when j < n_live[b]. ctx_len [B] int64 or NULL (= 0).
 * Outputs: argmax_out [B, R] int64 (or NULL), n_acc [B] int32, bonus [B] int64,
 *          crop [B] int64 = ctx_len + 1 + n_acc (KV entries kept: prefix + pending + accepted).
 * argmax is exact with the first index winning ties and NaN ranking above every number (bf16 values
 * compare as their exact fp32 widening). Requires R >= K + 1, V < 2^31, R <= 1024.
 * Two launches: a split-V argmax (each split of each row to scratch), then one block per sequence
 * reduces the splits and runs a wave ballot prefix scan. splits = 0 picks the split count.
 * scratch: trida_greedy_accept_scratch_bytes(B, R, V, dtype, splits) bytes, no initialisation needed.
 */
int64_t trida_greedy_accept_scratch_bytes(int64_t B, int64_t R, int64_t V, int dtype, int64_t splits);
int trida_greedy_accept(const void* logits, int dtype, int64_t B, int64_t R, int64_t V, int64_t batch_stride,
                        int64_t row_stride, const int64_t* drafts, int64_t K, int64_t draft_stride,
                        const int32_t* n_live, const int64_t* ctx_len, int64_t* argmax_out,
                        int32_t* n_acc, int64_t* bonus, int64_t* crop, void* scratch,
                        int64_t scratch_bytes, int64_t splits, void* stream);

/* Allocation-free greedy acceptance. No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Same arguments, kernels and results as trida_greedy_accept without the scratch
 * arguments: the split results go to a fixed device array of TRIDA_GREEDY_ACCEPT_NOALLOC_SCRATCH_BYTES
 * bytes that the library holds on every GPU it runs on until the process ends (its address is looked
 * up once per device, on the first call there). Shapes whose scratch
 * (trida_greedy_accept_scratch_bytes) exceeds that size are rejected with TRIDA_ERR_WORKSPACE; 1 MiB
 * covers e.g. B = 64 sequences of 33 rows over V = 248320 bf16 or fp32 at the default split count.
 * Calls that overlap in time on one GPU share the array and race; serialise them (one stream, or
 * events). The entry point calls no allocating routine. */
#define TRIDA_GREEDY_ACCEPT_NOALLOC_SCRATCH_BYTES (1 << 20)
int trida_greedy_accept_noalloc(const void* logits, int dtype, int64_t B, int64_t R, int64_t V, int64_t batch_stride,
                                int64_t row_stride, const int64_t* drafts, int64_t K, int64_t draft_stride,
                                const int32_t* n_live, const int64_t* ctx_len, int64_t* argmax_out, int32_t* n_acc,
                                int64_t* bonus, int64_t* crop, int64_t splits, void* stream);

/* Row argmax (first index on ties) and, when conf is not NULL, the softmax probability of the argmax
 * (the confidence the denoising passes rank MASK slots by). Replaces the argmax / max-softmax readout
 * of the block-diffusion denoise step (_shifted_conf_pred, qwen3_5_diffusion.py:446-467).
 * logits [rows, V] (dtype 0 fp32 / 1 bf16, row stride in elements); argmax [rows] int64; conf [rows]
 * fp32. scratch: trida_row_argmax_scratch_bytes(rows, V, dtype, splits). */
int64_t trida_row_argmax_scratch_bytes(int64_t rows, int64_t V, int dtype, int64_t splits);

/* The unmasking of one denoise pass over a draft canvas: per sequence b, the `count` slots j < block
 * with masked[b, j] != 0 and the highest conf[b, j] (ties: the lower slot first; unmasked slots rank
 * last) set canvas[b, j + 1] = argmax[b, j] (the shift readout: row j predicts slot j + 1) and clear
 * masked[b, j]. Replaces the commit of the most confident MASK positions of _denoise_shift_step
 * (qwen3_5_diffusion.py:476-635), with a fixed number of slots per pass instead of a confidence
 * threshold. argmax, conf: [B, >= block] (row stride row_stride), as trida_row_argmax writes them;
 * masked [B, block] bytes; canvas [B, >= block + 1] int64 (row stride canvas_stride); block <= 1024. */
int trida_unmask_top(const int64_t* argmax, const float* conf, int64_t row_stride, uint8_t* masked,
                     int64_t* canvas, int64_t canvas_stride, int64_t B, int64_t block, int64_t count, void* stream);
int trida_row_argmax(const void* logits, int dtype, int64_t rows, int64_t V, int64_t row_stride, int64_t* argmax,
                     float* conf, void* scratch, int64_t scratch_bytes, int64_t splits, void* stream);

/* One step of the bd_bidir_shift self-spec canvas decided on the device (the host logic of
 * selfspec_generate, inference/zoro-1/mlx/trida_mlx/decode.py:318-384; the vLLM plugin's next-canvas
 * build, qwen3_5_diffusion.py:924-951), so that canvas forward, acceptance, this and the rollback replay
 * from one graph. Per sequence b (canvas [B, 2N-1] int64 with row stride canvas_stride; argmax [B, >= 2N-1]
 * of the canvas logits, row j predicting slot j + 1; n_acc [B] = leading specs accepted, as
 * trida_greedy_accept returns with n_live = N - 1 for a verify canvas and 0 for a cold one):
 *   verify[b] == 0 (cold canvas [t0, MASK x (2N-2)]): emit argmax[0]; next canvas [argmax[0],
 *     argmax[1..N-1], MASK x (N-1)], verify; keep 1 row.
 *   verify[b] != 0 ([pending, spec_1..spec_{N-1}, MASK x (N-1)]), a = n_acc[b]: a < N-1: emit
 *     spec_1..spec_a, argmax[a]; next canvas [argmax[a], MASK x (2N-2)], cold; keep 1 + a rows. a = N-1:
 *     emit the specs and argmax[N-1]; next canvas [argmax[N-1], argmax[N..2N-2], MASK x (N-1)], verify;
 *     keep N rows.
 * Outputs: canvas and verify updated in place, n_keep [B] int32 (rows to commit), emit [B, N] int64 and
 * n_emit [B] int32 (tokens emitted this step), committed [B, N] int64 (the first n_keep canvas tokens this
 * step commits), kind [B] int32 (1 if the step was a verify round). 2 <= N <= 512. */
int trida_canvas_advance(const int64_t* argmax, int64_t argmax_stride, const int32_t* n_acc, int64_t* canvas,
                         int64_t canvas_stride, uint8_t* verify, int32_t* n_keep, int64_t* emit, int32_t* n_emit,
                         int64_t* committed, int32_t* kind, int64_t B, int64_t N, int64_t mask_id, void* stream);

/* ------------------------------------------------------------------------------------------------
 * Banned and gated tokens, in place on logit rows before an argmax or a sampling entry point reads
 * them. Replaces apply_ban (inference/zoro-1/mlx/trida_mlx/decode.py:76-99), which the reference applies
 * to greedy and sampled rows, drafts and verify alike.
 * logits [rows, V] (dtype 0 fp32 / 1 bf16, row stride in elements).
 * trida_ban_tokens: x[r, ids[j]] = -inf for j < n_ids (ids outside [0, V) are skipped); rows <= 65535.
 * trida_gate_tokens: per row, lse = logsumexp of the row; for gate g, p = exp(x[r, ids[g]] - lse)
 *   (written to raw_p [rows, n_gate] fp32 when not NULL; 0 for an id outside [0, V) or a row with no
 *   finite value), and x[r, ids[g]] = -inf where thr[g] > 0 and p < thr[g]. Every p of a row is taken
 *   before any gate writes. Apply the ban first (the reference's order). n_gate <= 512. thr NULL (raw_p
 *   given): a note-only pass that writes raw_p and leaves the row unchanged -- the raw probabilities
 *   _gate_note records (decode.py:63-73) come from the rows before the ban, so a caller that logs them
 *   runs it before trida_ban_tokens. */
int trida_ban_tokens(void* logits, int dtype, int64_t rows, int64_t V, int64_t row_stride, const int64_t* ids,
                     int64_t n_ids, void* stream);
int trida_gate_tokens(void* logits, int dtype, int64_t rows, int64_t V, int64_t row_stride, const int64_t* ids,
                      const float* thr, int64_t n_gate, float* raw_p, void* stream);

/* ------------------------------------------------------------------------------------------------
 * Sampled self-spec acceptance (speculative rejection sampling).
 * Replaces the sampled verify of selfspec_generate (inference/zoro-1/mlx/trida_mlx/decode.py:333-354)
 * with truncated_probs (decode.py:102-130), the role of _ss_sample_verify
 *   (inference/zoro-1/vllm/vllm_native_diffusion/qwen3_5_diffusion.py:787-880).
 *
 * P_i = truncated distribution of verify row i: y = logit / T (fp32 division) with ban_id at -inf;
 * top-k keeps y >= the k-th largest (0 < top_k < V, top_k <= 4096); the nucleus (top_p < 1) is taken
 * over those k largest values (or the whole row) in descending order and keeps every value whose
 * preceding mass is < top_p; the kept set is every y >= the last kept value (ties kept).
 * Draft i (i < min(K, n_live)) is accepted iff ratio >= 1 or u_accept[i] < ratio, ratio = P_i(d_i) /
 * q_i(d_i) (0 where q = 0); n_acc = leading accepted drafts. token = the correction drawn from
 * max(0, P_a - q_a) normalised (P_a if that mass is 0), a = n_acc < K, or the bonus from P_K when
 * every draft is accepted; the draw is the inverse CDF in vocabulary order at u_sample[b]
 * (token = min{x : cdf(x) > u * total}). crop = ctx_len + 1 + n_acc.
 * p_logits [B, R, V] fp32 (R >= K + 1), q_probs [B, K, V] fp32 probabilities the drafts were drawn
 * from, drafts [B, K] int64, n_live [B] int32 or NULL, u_accept [B, K] fp32 (row stride u_stride),
 * u_sample [B] fp32, ctx_len [B] int64 or NULL. Outputs n_acc [B] int32, token [B] int64, crop [B]
 * int64, ratio [B, K] fp64 or NULL (rows up to the first rejection; 0 after it), status [B] int32
 * (nonzero: a NaN / +inf logit or a row with no finite logit among the rows evaluated; the outputs of
 * that sequence are then undefined). K <= 64. Rows past a sequence's first rejection are never read:
 * the rows are evaluated in groups, each followed by a per-sequence accept scan.
 * scratch: trida_sample_accept_scratch_bytes(B, R, V, K) bytes, 256-byte aligned, no initialisation.
 */
int64_t trida_sample_accept_scratch_bytes(int64_t B, int64_t R, int64_t V, int64_t K);
int trida_sample_accept(const float* p_logits, int64_t B, int64_t R, int64_t V, int64_t p_batch_stride,
                        int64_t p_row_stride, const float* q_probs, int64_t q_batch_stride, int64_t q_row_stride,
                        const int64_t* drafts, int64_t K, int64_t draft_stride, const int32_t* n_live,
                        const float* u_accept, int64_t u_stride, const float* u_sample, const int64_t* ctx_len,
                        float temperature, int64_t top_k, float top_p, int64_t ban_id, int32_t* n_acc,
                        int64_t* token, int64_t* crop, double* ratio, int32_t* status, void* scratch,
                        int64_t scratch_bytes, void* stream);

/* Truncation statistics of rows [B, R, V] fp32 (the statistics of truncated_probs, decode.py:102-130):
 * m = max y, thr = smallest kept y (-inf: nothing truncated), zk = sum over kept y of exp(y - m), so
 * P(x) = [y_x >= thr] exp(y_x - m) / zk. status 1 = NaN / +inf logit, 2 = no finite logit. flags bit 0
 * skips the one-pass window path (exact radix select only); passes [B*R] (or NULL) reports how many
 * streaming passes each row took. Outputs are [B*R], row-major. */
int trida_truncate_stats(const float* logits, int64_t B, int64_t R, int64_t V, int64_t batch_stride,
                         int64_t row_stride, float temperature, int64_t top_k, float top_p, int64_t ban_id, int flags,
                         float* m, float* thr, double* zk, int32_t* status, int32_t* passes, void* stream);

/* Writes the truncated distributions P [B, R, V] fp32 from the statistics above (the probability rows
 * selfspec_generate keeps as the next step's draft distributions, decode.py:354, 378). */
int trida_truncated_probs(const float* logits, int64_t B, int64_t R, int64_t V, int64_t batch_stride,
                          int64_t row_stride, float temperature, int64_t ban_id, const float* m, const float* thr,
                          const double* zk, float* probs, int64_t out_batch_stride, int64_t out_row_stride,
                          void* stream);

/* Row-mapped truncated distributions: for sequence b and j < K, row out_rows[b*K + j] of probs[b] (Ro
 * rows) = P of logits row in_rows[b*K + j] (R rows; its statistics at [b, in_rows[b*K + j]]). It writes
 * the q rows of the slots a draft pass unmasks straight from the pass's rows (the q-row write of the draft
 * proposal, qwen3_5_diffusion.py:250-285; decode.py:376-378 keeps the P rows as q) in one launch. An index
 * outside its range skips that row (the maps are device data). */
int trida_truncated_probs_rows(const float* logits, int64_t B, int64_t R, int64_t V, int64_t batch_stride,
                               int64_t row_stride, float temperature, int64_t ban_id, const float* m,
                               const float* thr, const double* zk, const int64_t* in_rows, const int64_t* out_rows,
                               int64_t K, float* probs, int64_t Ro, int64_t out_batch_stride,
                               int64_t out_row_stride, void* stream);

/* dst[b, k, :] = fp32(src[b, rows[b*K + k], :]) for bf16 (dtype 1) or fp32 (dtype 0) logits [B, R, V]:
 * the still-masked rows of a draft pass's logits (the rows the draft proposal reads,
 * qwen3_5_diffusion.py:250-285) gathered and widened in one pass. A row index outside [0, R) skips that
 * row. */
int trida_gather_rows(const void* src, int dtype, int64_t B, int64_t R, int64_t V, int64_t batch_stride,
                      int64_t row_stride, const int64_t* rows, int64_t K, float* dst, int64_t out_batch_stride,
                      int64_t out_row_stride, void* stream);

/* Draws one token per row from the truncated distribution of statistics (m, thr, zk) given by
 * trida_truncate_stats: the inverse CDF in vocabulary order of P(x) = [y_x >= thr] exp(y_x - m) / zk at
 * u[r] (token = min{x : cdf(x) > u * total}), the draw the sampled acceptance makes for its bonus token.
 * It is the proposal draw of the draft pass (sample_from_probs(truncated_probs(...)),
 * inference/zoro-1/mlx/trida_mlx/decode.py:133-134, 374-378; _ss_draft_gumbel_kernel,
 * inference/zoro-1/vllm/vllm_native_diffusion/qwen3_5_diffusion.py:250-285), with the row statistics
 * computed once and shared with the q rows. logits [rows, V] fp32 (row stride in elements), m, thr,
 * zk, u [rows]; token [rows] int64. rows <= 65535. scratch: trida_sample_rows_scratch_bytes(rows, V)
 * bytes, 256-byte aligned, no initialisation. */
int64_t trida_sample_rows_scratch_bytes(int64_t rows, int64_t V);
int trida_sample_rows(const float* logits, int64_t rows, int64_t V, int64_t row_stride, float temperature,
                      int64_t ban_id, const float* m, const float* thr, const double* zk, const float* u,
                      int64_t* token, void* scratch, int64_t scratch_bytes, void* stream);

/* ------------------------------------------------------------------------------------------------
 * GDN layer front half: depthwise causal conv (width Kc in 2..4) over [window ++ x] + SiLU, split into
 * q / k / v, per-head l2norm of q and k (eps 1e-6), gates g = -exp(A_log) * softplus(a + dt_bias) and
 * beta = sigmoid(b). Replaces the conv / split / normalise / gate steps of TridaRuntime._gdn
 *   (inference/zoro-1/mlx/trida_mlx/model.py:285-303) and the fused prep inside
 *   fused_selfspec_gdn_layer (inference/zoro-1/vllm/vllm_native_diffusion/qwen3_5_diffusion.py:2211-2220).
 * x [B, T, C] bf16 pre-conv rows (batch stride x_sb, row stride x_st, elements), C = 2*Hk*Dk + Hv*Dv;
 * window [B, Kc-1, C] bf16; conv_w [C, Kc] bf16; a, b [B, T, Hv] bf16 (strides ab_sb, ab_st);
 * A_log, dt_bias [Hv] fp32. Outputs (contiguous): q, k [B, T, Hk, Dk] bf16 unit-norm, v [B, T, Hv, Dv]
 * bf16, g, beta [B, T, Hv] fp32, and window_out [B, Kc-1, C] (last Kc-1 rows of [window ++ x]) when
 * not NULL; window_out must not alias window. pre_out [B, T, C] (contiguous, 16-byte aligned, not x)
 * receives a copy of the pre-conv rows x when not NULL: the rows a rollback rebuilds the conv window
 * from (the raw mixed_qkv rows that fused_selfspec_gdn_layer keeps, qwen3_5_diffusion.py:2219).
 * Dk in {32, 64, 128}, Dv % 8 == 0.
 * State-pool and packed forms (each NULL = the contiguous form above), the arguments of the vLLM
 * calls this replaces (causal_conv1d_fn(x, weight, bias, conv_states, cache_indices, query_start_loc),
 * qwen3_5_diffusion.py:2227-2231; fused_selfspec_gdn_layer's conv_bias / win / win_idx / pre_out /
 * slot_idx, :2211-2220):
 *   conv_bias [C] bf16, added to the conv before the SiLU (16-byte aligned);
 *   win_idx [B] int32: sequence b reads window row win_idx[b] of a [rows, Kc-1, C] pool (vLLM's
 *     ss_slots1_i32 into ss_win_clean / ss_win_kern) and writes window_out row win_idx[b];
 *   pre_idx [B] int32: sequence b writes pre_out slot pre_idx[b] of a [slots, T, C] pool (slot_idx into
 *     ss_preconv);
 *   cu_seqlens [B + 1] int32 (packed ragged batch, query_start_loc): sequence b is rows
 *     cu_seqlens[b] .. cu_seqlens[b + 1] - 1 of x ([total, C], row stride x_st), a / b (row stride
 *     ab_st) and the outputs q, k, v, g, beta ([total, ...]); T is then an upper bound of every
 *     sequence's rows (the launch covers B x T rows; rows past T are not processed).
 */
int trida_gdn_prep(const uint16_t* x, const uint16_t* window, const uint16_t* conv_w, const uint16_t* a,
                   const uint16_t* b, const float* A_log, const float* dt_bias, uint16_t* q, uint16_t* k,
                   uint16_t* v, float* g, float* beta, uint16_t* window_out, uint16_t* pre_out, int64_t B, int64_t T,
                   int64_t Kc, int64_t Hk, int64_t Hv, int64_t Dk, int64_t Dv, int64_t x_sb, int64_t x_st,
                   int64_t ab_sb, int64_t ab_st, const uint16_t* conv_bias, const int32_t* win_idx,
                   const int32_t* pre_idx, const int32_t* cu_seqlens, void* stream);

/* ------------------------------------------------------------------------------------------------
 * Gated delta rule, recurrent form, with the block-causal canvas readout.
 * Replaces canvas_gdn_fused (inference/zoro-1/mlx/trida_mlx/kernels.py:118-131) and
 *   fused_recurrent_block_causal_gated_delta_rule(..., causal_mode, num_clean, initial_state,
 *   output_final_state) (qwen3_5_diffusion.py:2408-2415).
 * Per value head h (key head h / (Hv/Hk)) and row t, with g the log decay and q scaled by `scale`:
 *   S = e^g S; delta = beta (v - S k); S += delta k^T; o_t = S q_t.
 * causal_mode 1: every row reads its own state. causal_mode 2: rows t < num_clean read their own
 * state, rows t >= num_clean read the block-end state.
 * q, k [B, T, Hk, Dk] bf16, v [B, T, Hv, Dv] bf16, g, beta [B, T, Hv] fp32 (all contiguous);
 * state_in [B, Hv, Dv, Dk] fp32 (row v of head h holds S[:, v]); out [B, T, Hv, Dv] bf16.
 * state_out (NULL or, may alias state_in): state after all T rows. state_clean (NULL or a separate
 * buffer): state after min(num_clean, T) rows. Dk in {32, 64, 128, 256}, Dv % 4 == 0.
 * State-pool, ring and packed forms (each NULL = the contiguous form), the arguments of
 *   fused_recurrent_block_causal_gated_delta_rule_packed(..., ssm_states, cache_indices, block_size,
 *   causal_mode, num_clean, intermediate_states_buffer, intermediate_state_indices, cache_steps)
 *   (qwen3_5_diffusion.py:2234-2240, 2384-2393) and of the legacy call's cu_seqlens (:2408-2415):
 *   state_idx [B] int32 (cache_indices / ssm_idx): sequence b reads state_in row state_idx[b] of a
 *     [rows, Hv, Dv, Dk] pool and writes state_out row state_idx[b] (rows must be distinct when
 *     state_out aliases state_in); state_clean stays [B, Hv, Dv, Dk];
 *   inter [rows, cache_steps, Hv, Dv, Dk] fp32 (intermediate_states_buffer), inter_idx [B] int32
 *     (intermediate_state_indices; NULL = row b): entry (inter_idx[b], j) receives the state after
 *     rows 0..j of sequence b for j < min(cache_steps, rows of b) -- the self-spec ring, from which a
 *     step with n_acc accepted drafts continues at j = n_acc (:1821-1837, 228-248);
 *   cu_seqlens [B + 1] int32 (packed ragged batch): sequence b is rows cu_seqlens[b] ..
 *     cu_seqlens[b + 1] - 1 of q, k, v, g, beta and out ([total, ...]); num_clean counts from each
 *     sequence's first row; T is an upper bound of every sequence's rows (rows past T are not
 *     processed).
 * The index vectors and cu_seqlens (here and in trida_gdn_prep / trida_gdn_fused_layer) are read on the
 * device as given, as the reference's kernels read theirs: an entry outside [0, rows) of its pool, or a
 * cu_seqlens past the packed tensors, addresses memory outside them. The Python wrappers check them on
 * the host before the launch whenever the stream is not being captured.
 */
int trida_gdr_recurrent(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g,
                        const float* beta, const float* state_in, uint16_t* out, float* state_out,
                        float* state_clean, int64_t B, int64_t T, int64_t Hk, int64_t Hv, int64_t Dk,
                        int64_t Dv, int causal_mode, int64_t num_clean, float scale, const int32_t* cu_seqlens,
                        const int32_t* state_idx, float* inter, const int32_t* inter_idx, int64_t cache_steps,
                        void* stream);

/* Fused self-spec GDN layer, one launch for a block of T <= 64 rows: depthwise causal conv over
 * [window ++ x] + SiLU, split, l2norm(q, k), gates, then the recurrence and readout of
 * trida_gdr_recurrent. Replaces fused_selfspec_gdn_layer(mixed_qkv, a, b, A_log, dt_bias, conv_weight,
 *   conv_bias, win, win_idx, ssm_states, ssm_idx, inter, inter_idx, block_size, num_clean, cache_steps,
 *   out, pre_out, slot_idx) (inference/zoro-1/vllm/vllm_native_diffusion/
 *   qwen3_5_diffusion.py:2207-2221) and the Metal canvas_gdn_fused front half
 *   (inference/zoro-1/mlx/trida_mlx/kernels.py:118-131, model.py:289-303).
 * Inputs as trida_gdn_prep (x, window, conv_w, a, b, A_log, dt_bias, strides) plus state_in; outputs as
 * trida_gdr_recurrent (out, state_out, state_clean) and, each optional (NULL = not written), the rows a
 * rollback needs: k_out [B, T, Hk, Dk] bf16, v_out [B, T, Hv, Dv] bf16, g_out, beta_out [B, T, Hv] fp32
 * (given together), pre_out [B, T, C] bf16 raw pre-conv rows, window_out [B, Kc-1, C] (must not alias
 * window). Results are bit-identical to trida_gdn_prep followed by trida_gdr_recurrent.
 * Dk in {32, 64, 128}, Dv % 8 == 0, 2 <= Kc <= 4.
 * The vLLM call's pool / ring arguments (each NULL = contiguous): conv_bias (conv_bias), win_idx (win_idx,
 * the window row read and the window_out row written), state_idx (ssm_idx, into ssm_states =
 * ring[prev] viewed as [(2R+1) N, Hv, Dv, Dk]), inter / inter_idx / cache_steps (inter = ring[cur] as
 * [2R+1, N, Hv, Dv, Dk], inter_idx, cache_steps = N: the state after rows 0..j, j < cache_steps),
 * pre_idx (slot_idx, the pre_out slot of a [slots, T, C] pool), with the meanings of trida_gdn_prep and
 * trida_gdr_recurrent. The batch is B uniform blocks of T rows (block_size = T). */
int trida_gdn_fused_layer(const uint16_t* x, const uint16_t* window, const uint16_t* conv_w, const uint16_t* a,
                          const uint16_t* b, const float* A_log, const float* dt_bias, const float* state_in,
                          uint16_t* out, float* state_out, float* state_clean, uint16_t* k_out, uint16_t* v_out,
                          float* g_out, float* beta_out, uint16_t* pre_out, uint16_t* window_out, int64_t B,
                          int64_t T, int64_t Kc, int64_t Hk, int64_t Hv, int64_t Dk, int64_t Dv, int64_t x_sb,
                          int64_t x_st, int64_t ab_sb, int64_t ab_st, int causal_mode, int64_t num_clean,
                          float scale, const uint16_t* conv_bias, const int32_t* win_idx, const int32_t* state_idx,
                          float* inter, const int32_t* inter_idx, int64_t cache_steps, const int32_t* pre_idx,
                          void* stream);

/* Block-bidirectional gated delta rule: the training research path _block_bidirectional_gdr
 *   (train/models/hybrid.py:461-536) for blocks of block_size consecutive rows (the last block may be
 *   shorter). Per block with causal entry state E: out_f = the causal readout (forward sub-scan from E),
 *   out_b = the readout of a sub-scan over the block's rows in reverse order from E, out =
 *   (out_f + out_b) / 2. state_out (NULL or may alias state_in) = the causal state after all T rows.
 *   Layouts and Dk / Dv limits as trida_gdr_recurrent; 1 <= block_size <= 64. */
int trida_gdr_block_bidir(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g, const float* beta,
                          const float* state_in, uint16_t* out, float* state_out, int64_t B, int64_t T, int64_t Hk,
                          int64_t Hv, int64_t Dk, int64_t Dv, int64_t block_size, float scale, void* stream);

/* ------------------------------------------------------------------------------------------------
 * Gated delta rule, chunked WY / UT form on MFMA (v_mfma_f32_16x16x32_bf16), same recurrence and
 * readout as trida_gdr_recurrent. Replaces chunk_gated_delta_rule(q, k, v, g, beta, chunk_size=64,
 *   initial_state, output_final_state) (transformers modeling_qwen3_5.py torch_chunk_gated_delta_rule,
 *   the reference's declared CPU path, train/models/hybrid.py:31-35; FLA / HybridDiffusion
 *   chunk_block_causal_gated_delta_rule, train/models/hybrid.py:271-281) and, for blocks of T <= 64 rows,
 *   fused_recurrent_block_causal_gated_delta_rule(..., causal_mode, num_clean)
 *   (inference/zoro-1/vllm/vllm_native_diffusion/qwen3_5_diffusion.py:2408-2415).
 * Per chunk of 64 rows: T = (I + strict_lower(beta K K^T e^{G_t - G_s}))^{-1},
 *   v_new = T diag(beta) (V - e^G K S^T), o = scale (e^G Q S^T + (Q K^T e^{G_t - G_s})_{s<=t} v_new),
 *   S^T' = e^{G_last} S^T + K^T diag(e^{G_last - G}) v_new, with G the in-chunk cumulative log decay.
 * Layouts as trida_gdr_recurrent: q, k [B, T, Hk, Dk] bf16, v [B, T, Hv, Dv] bf16, g, beta [B, T, Hv]
 * fp32, state_in [B, Hv, Dv, Dk] fp32 (row v = column v of S^T), out [B, T, Hv, Dv] bf16.
 * out may be NULL (no readout; q may then be NULL). state_out (NULL, or may alias state_in): the state
 * after the first n rows, n = T, or n = n_keep[b % seq_mod] clamped to [0, T] when n_keep is not NULL
 * (the rollback of TridaRuntime.commit, inference/zoro-1/mlx/trida_mlx/model.py:486-507).
 * causal_mode 2 (rows >= num_clean read the block-end state) needs T <= 64 and no n_keep.
 * Dk in {32, 64, 128}, Dv % 16 == 0. T <= 64: one launch (prep and scan fused per workgroup); T > 64:
 * a chunk-parallel prep launch then a sequential scan launch, with a workspace of
 * trida_gdr_chunk_workspace_bytes(B, T, Hv) bytes (0 for T <= 64), 16-byte aligned, no initialisation.
 * Packed and state-pool forms (NULL = contiguous), the prefill call's
 *   chunk_gated_delta_rule(..., initial_state=ssm_state[indices], cu_seqlens=query_start_loc)
 *   (FLA's varlen interface as the vLLM Qwen3.5 prefill calls it; the indices as
 *   qwen3_5_diffusion.py:2384-2393 pass them): cu_seqlens [B + 1] int32: sequence b is rows
 *   cu_seqlens[b] .. cu_seqlens[b + 1] - 1 of q, k, v, g, beta, out ([total, ...]), at most T of them
 *   (T: an upper bound of every sequence's rows, which sizes the launch and the workspace);
 *   state_idx [B] int32: sequence b reads state_in row state_idx[b] and writes state_out row
 *   state_idx[b] of [rows, Hv, Dv, Dk] pools (distinct rows when they alias). These forms run the
 *   general chunk kernels (prep + scan, or the fused single chunk for T <= 64).
 */
int64_t trida_gdr_chunk_workspace_bytes(int64_t B, int64_t T, int64_t Hv);
int trida_gdr_chunk(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g, const float* beta,
                    const float* state_in, uint16_t* out, float* state_out, const int32_t* n_keep, int64_t seq_mod,
                    int64_t B, int64_t T, int64_t Hk, int64_t Hv, int64_t Dk, int64_t Dv, int causal_mode,
                    int64_t num_clean, float scale, void* workspace, int64_t workspace_bytes,
                    const int32_t* cu_seqlens, const int32_t* state_idx, void* stream);

/* ------------------------------------------------------------------------------------------------
 * GDN state snapshot: one coalesced copy of state_elems fp32 recurrent-state values and window_elems
 * bf16 conv-window values (any number of layers and sequences laid out contiguously).
 * Replaces the GDN backup before a draft/verify block (SGLang patch
 *   inference/zoro-1/sglang/two_stream_diffusion.patch:521-549, 557-569) and
 *   SeqCache.snapshot (inference/zoro-1/mlx/trida_mlx/model.py:184-190).
 * state_elems % 4 == 0, window_elems % 8 == 0, all buffers 16-byte aligned.
 */
int trida_gdn_snapshot(const float* state, float* snap_state, int64_t state_elems, const uint16_t* window,
                       uint16_t* snap_window, int64_t window_elems, void* stream);

/* ------------------------------------------------------------------------------------------------
 * GDN rollback to an accepted prefix of the block. Replaces TridaRuntime.commit
 *   (inference/zoro-1/mlx/trida_mlx/model.py:486-507) and the conv-window rebuild of _selfspec_step
 *   (qwen3_5_diffusion.py:963-975).
 * For each of NB (layer, sequence) slots b, with n = n_keep[b % seq_mod] clamped to [0, T]:
 *   state[b]  = snap_state[b] advanced by block rows 0..n-1 (k, v, g, beta as trida_gdn_prep writes
 *               them, [NB, T, ...]); may alias snap_state.
 *   window[b] = last Kc-1 rows of (snap_window[b] ++ preconv[b, :n]); may alias snap_window.
 * preconv [NB, T, C] bf16 with strides x_sb, x_st. Either part is skipped when its pointers are NULL.
 * skip_full != 0 leaves slots with n == T untouched (their state already covers the whole block).
 * Pool form of the window part (NULL = row / slot b): win_idx [NB] int32 picks slot b's row of
 * snap_window and window ([rows, Kc-1, C] pools; distinct rows when they alias), pre_idx [NB] int32 its
 * preconv slot (x_sb apart). This is the self-spec sampler's window rebuild over every layer at once,
 * wc[:, slot + 1] = last Kc-1 rows of (wc[:, slot + 1] ++ preconv[:, slot, :n_acc + 1])
 * (qwen3_5_diffusion.py:963-975), with win_idx = l (R + 2) + slot + 1 and pre_idx = l (R + 1) + slot.
 */
int trida_gdn_restore(const float* snap_state, float* state, const uint16_t* k, const uint16_t* v,
                      const float* g, const float* beta, const uint16_t* snap_window, uint16_t* window,
                      const uint16_t* preconv, const int32_t* n_keep, int64_t NB, int64_t seq_mod, int64_t T,
                      int64_t Hk, int64_t Hv, int64_t Dk, int64_t Dv, int64_t C, int64_t Kc, int64_t x_sb,
                      int64_t x_st, int skip_full, const int32_t* win_idx, const int32_t* pre_idx, void* stream);

/* ------------------------------------------------------------------------------------------------
 * Canvas attention over a bf16 KV cache, with the draft / verify / mixed masks and GQA.
 * Replaces TridaRuntime._attention + _canvas_mask (inference/zoro-1/mlx/trida_mlx/model.py:262-280,
 *   461-470) and the FA3 canvas call with the E3 bidirectional MASK rows
 *   (qwen3_5_diffusion.py:2516-2578).
 * q [B, T, Hq, D] bf16 (normalised, rotated); k_cache, v_cache [B, Hkv, Lmax, D] bf16 holding the
 * block's own keys at [prefix_len[b], prefix_len[b] + T); prefix_len [B] int32 on the device.
 * Row t (query head hq = hk * (Hq/Hkv) + g) sees every prefix key and, inside the block, column j when
 *   mask_mode 0 (verify): j <= t;  1 (draft): always;  2 (canvas): j <= t for t < n_clean, else always.
 * out [B, T, Hq, D] bf16 = softmax(scale q k^T) v, times sigmoid(gate) when gate is not NULL (gate
 * element (b, t, h, d) at gate + (b*T + t)*gate_row_stride + h*gate_head_stride + d).
 * KV crop after acceptance is a change of prefix_len only (a prefix_len above Lmax - T is read as
 * Lmax - T, so keys stay inside the cache). D in {64, 128, 256}.
 * max_keys: an upper bound of prefix_len + T used to plan splits (0 = Lmax); splits 0 = auto.
 * scratch: trida_attn_canvas_scratch_bytes(B, T, Hq, Hkv, D, max_keys, splits) bytes.
 */
int64_t trida_attn_canvas_scratch_bytes(int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int64_t D,
                                        int64_t max_keys, int64_t splits);
/* Diagnostic switch (no reference counterpart; for checking one combine against the other): with on != 0
 * the key splits of trida_attn_canvas are always merged by the general combine, also for two splits, which
 * otherwise take a one-round-trip kernel of the same arithmetic (bitwise the same results). Process-wide;
 * not for use while another thread launches attention. */
int trida_attn_set_combine_general(int on);
int trida_attn_canvas(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                      const int32_t* prefix_len, const uint16_t* gate, int64_t gate_row_stride,
                      int64_t gate_head_stride, uint16_t* out, int64_t B, int64_t T, int64_t Hq, int64_t Hkv,
                      int64_t D, int64_t Lmax, int mask_mode, int64_t n_clean, float scale, int64_t max_keys,
                      int64_t splits, void* scratch, int64_t scratch_bytes, void* stream);
/* trida_attn_canvas with the output rows [B * T, Hq * D] (B * T <= 48) written in the fragment order of a
 * weight-streaming GEMM's X (trida_ws_frag below) to out_frag (trida_ws_frag_elems(Hq * D) bf16,
 * 16-byte aligned), the output projection's input. No counterpart in the reference (an internal layout
 * between two kernels of the decoder forward). */
int trida_attn_canvas_frag(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                           const int32_t* prefix_len, const uint16_t* gate, int64_t gate_row_stride,
                           int64_t gate_head_stride, uint16_t* out_frag, int64_t B, int64_t T, int64_t Hq,
                           int64_t Hkv, int64_t D, int64_t Lmax, int mask_mode, int64_t n_clean, float scale,
                           int64_t max_keys, int64_t splits, void* scratch, int64_t scratch_bytes, void* stream);

/* ------------------------------------------------------------------------------------------------
 * Row-wise decoder kernels around the GEMMs (bf16 storage, fp32 arithmetic). They replace the torch
 * elementwise ops of the Qwen3.5 decoder layer the reference runtime calls through mlx-lm / vLLM
 * (TridaRuntime._forward, inference/zoro-1/mlx/trida_mlx/model.py:337-364).
 * add_rmsnorm: x = x + r (in place, r may be NULL), out = x * rsqrt(mean(x^2) + eps) * (1 + w)
 *   (zero_centred = 1, Qwen3.5 RMSNorm) or * w (zero_centred = 0). Row strides in elements.
 * silu_mul: out = silu(gu[:, :inter]) * gu[:, inter:2*inter] (SwiGLU).
 * gated_rmsnorm: per value head, out = bf16(o * rsqrt(mean(o^2) + eps)) * w * silu(z)
 *   (Qwen3.5 RMSNormGated); o, out [rows, H, Dv] contiguous, z row stride z_st.
 * attn_prep: one canvas block of full-attention rows. qkv rows hold [Hq x (q | gate)] [Hkv x k] [Hkv x v]
 *   (each D wide); q and k get a per-head zero-centred RMSNorm and rotate-half RoPE on the first
 *   rot_dim dims at position pos0[b] + t (inv_freq_i = theta^(-2i/rot_dim)); q goes to q_out
 *   [B, T, Hq, D], k and v to the caches [B, Hkv, Lmax, D] at slot slot0[b] + t (rows whose slot is
 *   outside [0, Lmax) write no K / V).
 */
/* Weight-streaming bf16 GEMM for canvas-sized activations: out = X[M, K] W[N, K]^T (torch Linear weight
 * layout), fp32 accumulation, 1 <= M <= 48, N % 16 == 0, K % 32 == 0. It replaces the projection and MLP
 * matmuls of the decoder forward at decode-step sizes (TridaRuntime._forward,
 * inference/zoro-1/mlx/trida_mlx/model.py:337-364), which are bound by the weight stream.
 * trida_wsgemm_shuffle writes the weights once into the kernel's layout Wp (N * K bf16, 16-byte aligned):
 *   tile t (16 rows) x k-step s (32 columns) x lane l = 16 g + r -> 8 bf16 of W[row][32 s + 8 g ..];
 *   row = 16 t + r, or with pair_halves = 1 (W = [gate; up], N / 2 rows each) row = 8 t + r for r < 8
 *   and N / 2 + 8 t + r - 8 otherwise, which the SwiGLU epilogue needs. With col_scale (K bf16, may be
 *   NULL) every column k is scaled first: bf16(W[row][k] * (1 + col_scale[k])) (zero_centred = 1) or
 *   bf16(W[row][k] * col_scale[k]): an RMSNorm weight folded in for trida_wsgemm_norm.
 * trida_wsgemm epilogues: 0 = bf16 out [M, N] (row stride out_row_stride); 1 = fp32 partial planes
 *   out[kg][M][N] (dense; kg from trida_wsgemm_plan), summed by trida_add_rmsnorm_parts or
 *   trida_residual_parts; 2 = SwiGLU: bf16 out[M, N / 2] = silu(gate) * up over pair_halves weights
 *   (gate and up rounded to bf16 first, as a bf16 GEMM output would be).
 * Epilogues 0 and 2 need K <= 2560 (one workgroup holds the whole K). The plan depends on (N, K, epilogue)
 * only, so a row of the result is bitwise independent of M.
 * trida_wsgemm_plan returns in *kgroups the number of partial planes epilogue 1 writes (1 otherwise). */
int trida_wsgemm_shuffle(const uint16_t* W, int64_t N, int64_t K, int64_t w_row_stride, int pair_halves,
                         const uint16_t* col_scale, int zero_centred, uint16_t* Wp, void* stream);
int trida_wsgemm_plan(int64_t N, int64_t K, int epilogue, int32_t* kgroups);
int trida_wsgemm(const uint16_t* X, int64_t x_row_stride, const uint16_t* Wp, int64_t M, int64_t N, int64_t K,
                 int epilogue, void* out, int64_t out_row_stride, void* stream);
/* trida_wsgemm with the decoder layer's RMSNorm fused in (epilogue 0 or 2): X is the raw residual stream h
 * [M, K] and Wp was shuffled with the norm weight as col_scale; row m of the result (before the SwiGLU) is
 * inv_m * (h W'^T)[m], inv_m = rsqrt(sum_c ss[m][c] / K + eps) over the trida_residual_ss_chunks(K)
 * per-chunk sums of squares trida_residual_parts wrote for row m. It stands for the reference's
 * RMSNorm + projection (inference/zoro-1/mlx/trida_mlx/model.py:337-364) with the norm weight applied to
 * the weights instead of the activations (a different bf16 rounding point, same operator). */
int trida_wsgemm_norm(const uint16_t* X, int64_t x_row_stride, const float* ss, float eps, const uint16_t* Wp, int64_t M,
                      int64_t N, int64_t K, int epilogue, void* out, int64_t out_row_stride, void* stream);
/* The residual add of a projection's partial planes, spread over rows x trida_residual_ss_chunks(dim)
 * one-wave workgroups: h = bf16(h + bf16(sum of the n_parts fp32 planes [rows, dim], plane_stride elements
 * apart, summed in plane order)) in place (n_parts = 0: h unchanged), and ss[row][c] = sum of h^2 over
 * elements [256 c, 256 c + 256) of the row (fp32 [rows, trida_residual_ss_chunks(dim)]). */
int64_t trida_residual_ss_chunks(int64_t dim);
int trida_residual_parts(uint16_t* h, int64_t h_row_stride, const float* parts, int64_t n_parts, int64_t plane_stride,
                         int64_t rows, int64_t dim, float* ss, void* stream);
/* Fragment order of a weight-streaming GEMM's activations X [M, K] (M <= 48, K % 32 == 0): the operand
 * layout of the kernel's matrix-core step, so that each of its X loads reads 1 KB of consecutive bytes
 * (row-major X gives each load 16 rows x 64 bytes, half a cache line per row, and the workgroup's X slice
 * takes twice as long to arrive). Xf holds trida_ws_frag_elems(K) bf16 (16-byte aligned); X[m][k] sits at
 * element ((k / 32 * 3 + m / 16) * 64 + (k % 32) / 8 * 16 + m % 16) * 8 + k % 8, whatever M is; entries
 * of rows >= M are neither written nor read. No counterpart in the reference (an internal layout between
 * the kernels of one decoder forward, inference/zoro-1/mlx/trida_mlx/model.py:337-364).
 * trida_ws_frag converts row-major X; trida_residual_parts_frag is trida_residual_parts that also writes
 * the updated h in fragment order to h_frag (rows <= 48, dim % 32 == 0); trida_gated_rmsnorm_frag writes
 * trida_gated_rmsnorm's output in fragment order (K = H * Dv). trida_wsgemm_ex is trida_wsgemm (ss NULL)
 * or trida_wsgemm_norm (ss given) with flags: TRIDA_WS_X_FRAG = X in fragment order (x_row_stride
 * unused), TRIDA_WS_OUT_FRAG = the bf16 output of epilogue 0 or 2 in fragment order for the next GEMM
 * (out_row_stride unused). The results are bitwise those of the row-major forms. */
#define TRIDA_WS_X_FRAG 1
#define TRIDA_WS_OUT_FRAG 2
/* Greedy verify fused into the LM head: the LM-head GEMM of a greedy verify block (M = B * R <= 48 rows of
 * normed hidden states, W the [V, K] embedding / head shuffled by trida_wsgemm_shuffle) with an argmax
 * epilogue. Replaces lm_head + argmax of the greedy branch of _selfspec_step
 * (inference/zoro-1/vllm/vllm_native_diffusion/qwen3_5_diffusion.py:906-914) and of selfspec_generate's
 * verify (inference/zoro-1/mlx/trida_mlx/decode.py:323-332): each workgroup reduces every row of the bf16
 * logits of its columns to (max, first index; NaN above every number) while the weights stream, and
 * writes pval / pidx [M][S] (fp32 / int32, S = trida_wsgemm_argmax_splits(V, K) column splits in column
 * order); the logits are not written unless `logits` is given (bf16 [M, V], row stride out_row_stride,
 * bitwise the store epilogue's). trida_greedy_accept_splits then runs the acceptance of
 * trida_greedy_accept (argmax_out, n_acc, bonus, crop; same arguments and results) from those pairs
 * (pval / pidx laid out [B, R, S]), so the verify step never reads the logits back: a 33 x 248320 head
 * leaves 33 x 255 pairs (67 KB) instead of 16.4 MB of logits. flags: TRIDA_WS_X_FRAG. 1 <= S <= 2048. */
int64_t trida_wsgemm_argmax_splits(int64_t N, int64_t K);
int trida_wsgemm_argmax(const uint16_t* X, int64_t x_row_stride, const uint16_t* Wp, int64_t M, int64_t N, int64_t K,
                        int flags, uint16_t* logits, int64_t out_row_stride, float* pval, int32_t* pidx, void* stream);
int trida_greedy_accept_splits(const float* pval, const int32_t* pidx, int64_t B, int64_t R, int64_t S,
                               const int64_t* drafts, int64_t K, int64_t draft_stride, const int32_t* n_live,
                               const int64_t* ctx_len, int64_t* argmax_out, int32_t* n_acc, int64_t* bonus,
                               int64_t* crop, void* stream);
/* A denoise pass's readout fused into the LM head: lm_head + the argmax and its softmax probability per row
 * (the confidence of _denoise_shift_step, inference/zoro-1/vllm/vllm_native_diffusion/qwen3_5_diffusion.py:446-467,
 * that trida_row_argmax computes from logits). trida_wsgemm_argmax_conf is trida_wsgemm_argmax with psum [M][S]
 * too: sum exp(x - pval) over the workgroup's bf16 logits. trida_argmax_conf_splits reduces the triples of rows
 * [B, R] (laid out [B, R, S], S <= 256) to argmax (int64) and conf (fp32) at b * out_row_stride + r: the
 * argmax is trida_row_argmax's (first index, NaN first), conf = 1 / sum_s psum_s e^{pval_s - max} (the same
 * value up to the fp32 summation order). */
int trida_wsgemm_argmax_conf(const uint16_t* X, int64_t x_row_stride, const uint16_t* Wp, int64_t M, int64_t N,
                             int64_t K, int flags, uint16_t* logits, int64_t out_row_stride, float* pval,
                             int32_t* pidx, float* psum, void* stream);
int trida_argmax_conf_splits(const float* pval, const int32_t* pidx, const float* psum, int64_t B, int64_t R,
                             int64_t S, int64_t* argmax, float* conf, int64_t out_row_stride, void* stream);
int64_t trida_ws_frag_elems(int64_t K);
int trida_ws_frag(const uint16_t* X, int64_t x_row_stride, int64_t M, int64_t K, uint16_t* Xf, void* stream);
int trida_wsgemm_ex(const uint16_t* X, int64_t x_row_stride, const float* ss, float eps, const uint16_t* Wp, int64_t M,
                    int64_t N, int64_t K, int epilogue, void* out, int64_t out_row_stride, int flags, void* stream);
int trida_residual_parts_frag(uint16_t* h, int64_t h_row_stride, const float* parts, int64_t n_parts,
                              int64_t plane_stride, int64_t rows, int64_t dim, float* ss, uint16_t* h_frag,
                              void* stream);
/* A GDN layer's gated RMSNorm folded into its recurrence and out projection (no reference counterpart as a
 * call: the decode step's gdr -> RMSNormGated(o, z) -> out_proj, inference/zoro-1/vllm/vllm_native_diffusion/
 * qwen3_5_diffusion.py:2207-2221 and the mlx model's GDN mixer, with no kernel between the recurrence and the
 * projection). trida_gdr_recurrent_gnorm is trida_gdr_recurrent (contiguous form, B * T <= 48, T <= 40) that
 * also writes u = bf16(bf16(o) * gnorm_w * silu(z)) in the weight-streaming GEMM's fragment order (u_frag,
 * trida_ws_frag_elems(Hv * Dv) elements) and ss_parts [B * T][Hv][Dv / 8], the sums of bf16(o)^2 over each 8
 * columns; z rows of Hv * Dv at z_row_stride. trida_wsgemm_headnorm is the partial-plane projection of those u
 * rows (K = heads * head width, a multiple of 32 columns per head) with each head's partial sums of a row
 * scaled by rsqrt(sum of its ss_parts / head width + eps): planes = trida_wsgemm_headnorm_planes(N, K, heads).
 * The result equals trida_gated_rmsnorm_frag then trida_wsgemm_ex epilogue 1 up to where the bf16 roundings
 * fall (bf16(o * inv) is not formed). */
int trida_gdr_recurrent_gnorm(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g,
                              const float* beta, const float* state_in, uint16_t* out, float* state_out,
                              float* state_clean, int64_t B, int64_t T, int64_t Hk, int64_t Hv, int64_t Dk, int64_t Dv,
                              int causal_mode, int64_t num_clean, float scale, const uint16_t* z,
                              int64_t z_row_stride, const uint16_t* gnorm_w, uint16_t* u_frag, float* ss_parts,
                              void* stream);
int trida_wsgemm_headnorm_planes(int64_t N, int64_t K, int64_t heads, int32_t* kgroups);
int trida_wsgemm_headnorm(const uint16_t* Xf, const uint16_t* Wp, int64_t M, int64_t N, int64_t K,
                          const float* ss_parts, int64_t heads, float eps, float* parts, void* stream);

int trida_add_rmsnorm(uint16_t* x, const uint16_t* r, const uint16_t* w, uint16_t* out, int64_t rows, int64_t dim,
                      int64_t x_st, int64_t r_st, int64_t o_st, float eps, int zero_centred, void* stream);
/* add_rmsnorm whose residual is the sum of n_parts fp32 planes (plane_stride elements apart, rows of dim
 * floats): the partial planes of trida_wsgemm epilogue 1, summed in plane order and rounded to bf16. */
int trida_add_rmsnorm_parts(uint16_t* x, const float* parts, int64_t n_parts, int64_t plane_stride, const uint16_t* w,
                            uint16_t* out, int64_t rows, int64_t dim, int64_t x_st, int64_t o_st, float eps,
                            int zero_centred, void* stream);
int trida_silu_mul(const uint16_t* gu, uint16_t* out, int64_t rows, int64_t inter, int64_t g_st, int64_t o_st,
                   void* stream);
int trida_gated_rmsnorm(const uint16_t* o, const uint16_t* z, const uint16_t* w, uint16_t* out, int64_t rows,
                        int64_t H, int64_t Dv, int64_t z_st, float eps, void* stream);
int trida_gated_rmsnorm_frag(const uint16_t* o, const uint16_t* z, const uint16_t* w, uint16_t* out_frag, int64_t rows,
                             int64_t H, int64_t Dv, int64_t z_st, float eps, void* stream);
int trida_attn_prep(const uint16_t* qkv, int64_t qkv_row_stride, const uint16_t* q_norm_w, const uint16_t* k_norm_w,
                    const int32_t* pos0, const int32_t* slot0, uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache,
                    int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int64_t D, int64_t Lmax, int64_t rot_dim,
                    float rope_theta, float eps, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TRIDA_HIP_H */
