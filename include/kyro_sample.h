/*
 * kyro_sample.h — plain-decode sampling with the worker's logit processors.
 *
 *   kyro_sample_tokens  replaces, for a batch of rows, the per-request tail of Worker::run_loop
 *                       (src/worker.rs:141-197: logit bias, frequency / presence penalties,
 *                       grammar mask) and sample_token (src/worker.rs:267-362), with the uniform
 *                       passed in instead of drawn from an unseeded rand::rng().
 *   kyro_penalty_adds   the reference's penalty vector for one request (worker.rs:154-181), on
 *                       the host, as the sparse list kyro_sample_tokens takes.
 */
#ifndef KYRO_SAMPLE_H
#define KYRO_SAMPLE_H

#include <stddef.h>
#include <stdint.h>

#include "kyro_verify.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct kyro_sample_params {
    int32_t batch_size;    /* B */
    int32_t vocab_size;    /* V */
    int32_t logits_dtype;  /* KYRO_F32 */
    int32_t num_masks;     /* rows of allowed_mask (0 when it is NULL) */
} kyro_sample_params;

/*
 * One token per row b of logits [B, V] (f32, device). Processing (worker.rs:141-190), in the
 * reference's order: y = ((logits + bias) + penalty) + mask, where
 *   bias     entries bias_tokens / bias_values [bias_offsets[b], bias_offsets[b+1]) (distinct
 *            tokens per row; NULL bias_offsets: none),
 *   penalty  entries penalty_tokens / penalty_values likewise (e.g. from kyro_penalty_adds),
 *   mask     -inf where bit v of allowed_mask[mask_row[b]] (ceil(V/32) uint32 words per mask,
 *            bit v % 32 of word v / 32) is clear; mask_row[b] = -1 or NULL mask_row: no mask.
 * Sampling (sample_token, worker.rs:267-362):
 *   temperature[b] <= 0: argmax(y), the first index among equal maxima.
 *   otherwise z = y * f32(1 / T); top_k[b] in (0, V) keeps the k largest z (ties: lower index);
 *   p = exp(z - max) / sum over the kept tokens;
 *   top_p[b] < 1: the kept tokens sorted by p descending (ties: lower index) are cut after the
 *     first whose running sum exceeds top_p, and r = u[b] * (mass of the cut);
 *   otherwise r = u[b], walking in index order, or, after top-k alone, in the same descending
 *     order (the reference leaves that order to select_nth_unstable).
 *   The token is the first whose running sum reaches r. If rounding leaves none, it is the most
 *   probable kept token after top-p, the least probable kept token after top-k alone, and the
 *   last index otherwise (worker.rs:340-360). A row whose tokens are all masked gets V - 1.
 * top_p / top_k may be NULL (1.0 / off). u[b] in [0, 1). out_tokens [B] uint32.
 * A bias / penalty token >= V or a mask_row >= num_masks latches KYRO_EINVAL for kyro_sync.
 */
int kyro_sample_tokens(kyro_ctx ctx, const kyro_sample_params* params, const float* logits,
                       const float* temperature, const float* top_p, const int32_t* top_k,
                       const float* u, const int32_t* bias_offsets, const uint32_t* bias_tokens,
                       const float* bias_values, const int32_t* penalty_offsets,
                       const uint32_t* penalty_tokens, const float* penalty_values,
                       const uint32_t* allowed_mask, const int32_t* mask_row, uint32_t* out_tokens);

/*
 * The additive penalty of one request from its generated tokens (HOST arrays), as worker.rs:154-181
 * computes it in f32: every occurrence of token t adds frequency_penalty to entry t, then every
 * occurrence replaces entry t by min(entry, 0) + presence_penalty. Tokens >= vocab_size are
 * skipped. Writes the touched tokens in increasing order with their values (up to cap);
 * *out_n receives the count. Both penalties 0: no entries (the reference skips the step).
 */
int kyro_penalty_adds(const uint32_t* generated, int64_t n, float frequency_penalty,
                      float presence_penalty, int32_t vocab_size, uint32_t* out_tokens,
                      float* out_values, int64_t cap, int64_t* out_n);

#ifdef __cplusplus
}
#endif

#endif /* KYRO_SAMPLE_H */
