/*
 * loopspec_hip.h -- C-ABI of the MI355X (gfx950) LoopSpec verify-and-sample library
 * (libloopspec_hip.so).
 *
 * Conventions for every entry point:
 *   - Return an int status: LS_OK (0) on success, otherwise an LS_ERR_* code; the
 *     message is available from ls_last_error() on the calling thread.
 *   - All tensor arguments are raw device pointers. Strides are in ELEMENTS and the
 *     vocabulary axis is always contiguous (unit stride).
 *   - `stream` is a hipStream_t passed as an opaque pointer (NULL = default stream).
 *     Work is only enqueued; no entry point synchronises the device or allocates
 *     device memory. Scratch memory comes from the caller's `workspace`, which must
 *     be zero-filled once when it is allocated; kernels leave it zeroed again, so
 *     a workspace can be reused by later calls on the same stream (and inside a
 *     captured graph). Calls that share a workspace must be stream-ordered.
 *   - Token ids, row ids and slot ids are int64 unless stated; KV mapping tables
 *     are int32, matching the reference's layout contracts
 *     (sglang_recurrent/loopspec/sampling/sampler.py:3-12,
 *      sglang_recurrent/loopspec/graph_ops.py:221-233).
 */
#ifndef LOOPSPEC_HIP_H_
#define LOOPSPEC_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* ls_stream_t; /* hipStream_t */

enum {
  LS_OK = 0,
  LS_ERR_VALUE = 1,   /* bad shape / argument: Python raises ValueError   */
  LS_ERR_RUNTIME = 2, /* unsupported layout / device: RuntimeError        */
  LS_ERR_HIP = 3      /* HIP runtime error (launch, attribute query, ...) */
};

enum { LS_DTYPE_F32 = 0, LS_DTYPE_BF16 = 1, LS_DTYPE_F16 = 2 };

/* Library ABI version (bumped on any signature change). */
int ls_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* ls_last_error(void);

/* Set a tuning option by name (e.g. "greedy_splits"); 0 restores the heuristic.
 * Unknown names return LS_ERR_VALUE. */
int ls_set_option(const char* name, int64_t value);

/* ------------------------------------------------------------------------------
 * (b) Greedy verification
 * ------------------------------------------------------------------------------ */

/* Row-wise argmax with torch.argmax semantics: first index of the maximum, NaN
 * counts as the maximum (first NaN wins), -0 == +0.
 * Replaces: GreedyDecisionPolicy.queue's torch.argmax over every endpoint row
 *   (sglang_recurrent/loopspec/decisions.py:116).
 * logits: [rows, vocab] of `dtype`, row stride `row_stride` elements.
 * out:    int64 [rows] (contiguous). */
int ls_argmax_rows(const void* logits, int dtype, int64_t rows, int64_t vocab,
                   int64_t row_stride, int64_t* out, void* workspace,
                   uint64_t workspace_bytes, ls_stream_t stream);
uint64_t ls_argmax_rows_workspace(int64_t rows, int64_t vocab);

/* Fused greedy verify over a chain of k draft positions, one launch:
 * argmax of every target row [B, k+1, V] and draft row [B, k, V], then the
 * accept-prefix scan. Row (b, i) of the target lives at
 * target_logits + b*target_batch_stride + i*target_pos_stride (elements);
 * same for the draft. If draft_logits is NULL, draft_tokens [B, k] (int64,
 * contiguous) supplies the draft ids instead.
 *   accept_len[b] = number of leading positions with draft id == target argmax;
 *   tokens[b, j]  = target argmax at j for j <= accept_len[b] (the accepted
 *                   prefix followed by the correction or bonus token), -1 after.
 * row_argmax (optional, may be NULL): int64 [B, 2k+1] = target argmax at
 *   positions 0..k followed by the draft argmax at 0..k-1.
 * Replaces the greedy final-endpoint rule of GreedyDecisionPolicy.resolve
 *   (sglang_recurrent/loopspec/decisions.py:157-170) applied along the
 *   pipeline's accept prefix (sglang_recurrent/loopspec/pipeline.py:365-412). */
int ls_greedy_verify(const void* target_logits, int64_t target_batch_stride,
                     int64_t target_pos_stride, const void* draft_logits,
                     int64_t draft_batch_stride, int64_t draft_pos_stride,
                     const int64_t* draft_tokens, int dtype, int64_t batch, int64_t k,
                     int64_t vocab, int32_t* accept_len, int64_t* tokens,
                     int64_t* row_argmax, void* workspace, uint64_t workspace_bytes,
                     ls_stream_t stream);
uint64_t ls_greedy_verify_workspace(int64_t batch, int64_t k, int64_t vocab);

#ifdef __cplusplus
}
#endif

#endif /* LOOPSPEC_HIP_H_ */
