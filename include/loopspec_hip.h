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
 *     be zero-filled once when it is allocated. Every kernel leaves the words that
 *     must start at zero (arrival counters, combine slots) zeroed again, so a
 *     workspace can be reused by later calls of the SAME entry point on the same
 *     stream (and inside a captured graph), whatever their shapes. Do not share one
 *     workspace between different entry points. Calls that share a workspace must
 *     be stream-ordered; concurrent calls on one workspace race.
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

/* ------------------------------------------------------------------------------
 * (a) logit processing + (c) lossless speculative sampling
 *
 * Shared processing of a logits row (any of f32/bf16/f16, contiguous vocab,
 * 16-byte aligned rows, vocab*elem_bytes a multiple of 16):
 *   x = logits; for ids in the row's history (if penalty != 1):
 *       x <- x < 0 ? x*penalty : x*RN(1/penalty);  then x <- x*RN(1/T) (T != 1);
 *   p = softmax(x) in the library's declared arithmetic (see DESIGN.md of the
 *   repository: ls_exp, 2^-46 fixed-point masses);
 *   top_p < 1: keep p >= c with c = max{v : sum_{p>=v} fx46(p) >= fx46(top_p)}
 *   (ties kept; the whole row if no v qualifies), renormalise by the retained
 *   mass -- the value semantics of sort + cumsum + searchsorted(right=False)
 *   + gather + where + sum of filtered_probabilities
 *   (sglang_recurrent/loopspec/sampling/distributions.py:14-86).
 *   top_k must be 0 or >= vocab (top-k filtering is not offered here).
 * ------------------------------------------------------------------------------ */

/* Fused chain verify, one launch for B batch elements of k draft positions:
 * filters every target row [B, k+1, V] (P_i) and draft row [B, k, V] (Q_i);
 * position i accepts draft_tokens[b, i] iff u[b,i] < min(1, P_i[x]/Q_i[x])
 * (sglang_recurrent/loopspec/sampling/sampler.py:428-460); the first rejection
 * at i emits a draw from normalize(max(P_i - Q_i, 0)) (falling back to P_i at
 * zero mass, sglang_recurrent/loopspec/sampling/rejection.py:60-69) with
 * u[b, k+i]; if all k accept, a bonus draw from P_k with u[b, 2k]
 * (direct final sample, sglang_recurrent/loopspec/sampling/policy.py:156-165).
 * Draws are inverse-CDF over token index (sampler.py:22-102).
 *   uniforms: float32 [B, 2k+1] contiguous; draft_tokens: int64 [B, k].
 *   history: int32 rows of token ids (row stride history_stride), lengths
 *            history_len[B]; used only when penalty != 1.
 *   accept_len: int32 [B]; tokens: int64 [B, k+1] (emitted tokens, -1 padded).
 * Replaces SamplingDecisionPolicy.queue/read for q1 verification
 * (sglang_recurrent/loopspec/sampling/policy.py:220-283) along the pipeline's
 * accept prefix (sglang_recurrent/loopspec/pipeline.py:365-412). */
int ls_spec_verify(const void* target_logits, int64_t target_batch_stride,
                   int64_t target_pos_stride, const void* draft_logits,
                   int64_t draft_batch_stride, int64_t draft_pos_stride,
                   const int64_t* draft_tokens, const float* uniforms, int dtype,
                   int64_t batch, int64_t k, int64_t vocab, float temperature, float top_p,
                   int64_t top_k, float penalty, const int32_t* history,
                   int64_t history_stride, const int32_t* history_len,
                   int32_t* accept_len, int64_t* tokens, void* workspace,
                   uint64_t workspace_bytes, ls_stream_t stream);
uint64_t ls_spec_verify_workspace(int64_t batch, int64_t k, int64_t vocab);

/* Filter each logits row and draw one token per row with uniforms[row]
 * (float32 [rows]) into out_tokens (int64 [rows]); history rows as above,
 * one per logits row. Replaces prepare_sampling_probabilities followed by
 * sample_probabilities / CategoricalSampler.sample
 * (sglang_recurrent/loopspec/sampling/distributions.py:89-171). */
int ls_sample_logits(const void* logits, int64_t row_stride, int dtype, int64_t rows,
                     int64_t vocab, float temperature, float top_p, int64_t top_k,
                     float penalty, const int32_t* history, int64_t history_stride,
                     const int32_t* history_len, const float* uniforms, int64_t* out_tokens,
                     ls_stream_t stream);

/* Dense filtering: probs_out (optional, [rows, V] float32, row stride
 * probs_stride) receives p; filtered_out (optional) the filtered, renormalised
 * distribution (p itself when top_p == 1); cutoff_out / mass_out (optional,
 * float32 [rows]) the cutoff value and binary32 retained mass. top_p_rows
 * (optional, float32 [rows]) overrides top_p per row when top_p < 1.
 * Replaces filtered_probabilities and the probability/cutoff part of
 * prepare_sampling_probabilities (distributions.py:14-149). */
int ls_filter_logits(const void* logits, int64_t row_stride, int dtype, int64_t rows,
                     int64_t vocab, float temperature, float top_p, const float* top_p_rows,
                     int64_t top_k, float* probs_out, int64_t probs_stride,
                     float* filtered_out, int64_t filtered_stride, float* cutoff_out,
                     float* mass_out, ls_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* LOOPSPEC_HIP_H_ */
