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
 * logits   [B, R, V] fp32, row r of sequence b at logits + b*batch_stride + r*row_stride.
 *          Row j (j < K) verifies draft j; row n_acc gives the bonus token (shift readout).
 * drafts   [B, K] int64 (row stride draft_stride); n_live [B] int32 or NULL (= K): draft j only counts
 *          when j < n_live[b]. ctx_len [B] int64 or NULL (= 0).
 * Outputs: argmax_out [B, R] int64 (or NULL), n_acc [B] int32, bonus [B] int64,
 *          crop [B] int64 = ctx_len + 1 + n_acc (KV entries kept: prefix + pending + accepted).
 * argmax is exact on fp32 with the first index winning ties and NaN ranking above every number.
 * Requires R >= K + 1, V < 2^31, R <= 1024. Two launches: a split-V argmax (each split of each row
 * to scratch), then one block per sequence reduces the splits and runs a wave ballot prefix scan.
 * splits = 0 picks the split count. scratch: trida_greedy_accept_scratch_bytes(B, R, V, splits) bytes,
 * no initialisation needed.
 */
int64_t trida_greedy_accept_scratch_bytes(int64_t B, int64_t R, int64_t V, int64_t splits);
int trida_greedy_accept(const float* logits, int64_t B, int64_t R, int64_t V, int64_t batch_stride,
                        int64_t row_stride, const int64_t* drafts, int64_t K, int64_t draft_stride,
                        const int32_t* n_live, const int64_t* ctx_len, int64_t* argmax_out,
                        int32_t* n_acc, int64_t* bonus, int64_t* crop, void* scratch,
                        int64_t scratch_bytes, int64_t splits, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TRIDA_HIP_H */
