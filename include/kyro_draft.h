/*
 * kyro_draft.h — n-gram drafting for the verify step.
 *
 *   kyro_ngram_build   replaces  SpeculativeDecoder::build_ngram_table (src/speculative.rs:196-208):
 *                                every window of a corpus sequence maps its first order-1 tokens
 *                                to the next one; a later window overwrites an earlier one
 *                                (HashMap::insert), in corpus order.
 *   kyro_ngram_draft   replaces  generate_drafts' DraftStrategy::Ngram arm (:239-256) for a batch:
 *                                up to max_draft times, stop if the context (plus drafts so far)
 *                                is shorter than `order`, else look up its last order-1 tokens and
 *                                append the stored token, stopping at the first miss.
 * The table is built on the host (exact keys, open addressing) and uploaded once; drafting runs
 * on the device and writes draft_tokens / num_draft in the layout kyro_spec_verify reads, so a
 * draft -> verify loop needs no host round trip.
 */
#ifndef KYRO_DRAFT_H
#define KYRO_DRAFT_H

#include <stddef.h>
#include <stdint.h>

#include "kyro_verify.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct kyro_ngram_s* kyro_ngram;

/* Builds the table from num_seqs HOST sequences: sequence s is tokens[offsets[s], offsets[s+1]).
 * order >= 2 (the reference's windows need a prefix). */
int kyro_ngram_build(const uint32_t* tokens, const int64_t* offsets, int64_t num_seqs, int32_t order,
                     kyro_ngram* out);
int kyro_ngram_destroy(kyro_ngram t);
/* Host lookup of one prefix of order-1 tokens: 1 and *next when present, 0 when absent. */
int kyro_ngram_lookup(kyro_ngram t, const uint32_t* prefix, uint32_t* next);
int64_t kyro_ngram_size(kyro_ngram t);  /* distinct prefixes; -1 for a null handle */
/* Copies the table to ctx's device (once; later calls reuse it). */
int kyro_ngram_upload(kyro_ngram t, kyro_ctx ctx);
/* Drafts for B sequences on ctx's stream. Device arrays:
 *   context_tail [B, order-1] uint32: each sequence's last order-1 context tokens (entries before
 *                the start of a shorter context are ignored)
 *   context_len  [B] int64: context length
 *   draft_tokens [B, max_draft] uint32 out (unused entries 0xFFFFFFFF), num_draft [B] int32 out.
 * The table must have been uploaded to ctx's device. */
int kyro_ngram_draft(kyro_ngram t, kyro_ctx ctx, int32_t batch_size, int32_t max_draft,
                     const uint32_t* context_tail, const int64_t* context_len, uint32_t* draft_tokens,
                     int32_t* num_draft);

#ifdef __cplusplus
}
#endif

#endif /* KYRO_DRAFT_H */
