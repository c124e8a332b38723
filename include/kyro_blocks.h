/*
 * kyro_blocks.h — KV block allocation with prefix sharing, and the device block tables the
 * verify step reads.
 *
 *   kyro_bm_*      replaces  BlockManager (src/scheduler/block_manager.rs:15-153):
 *                            allocate_with_prefix :53-102, allocate :107-124, free :128-153
 *   kyro_radix_*   replaces  RadixCache (src/scheduler/radix_cache.rs:29-155):
 *                            match_prefix :49-86, insert :89-120, evict_lru :122-135
 *   kyro_bm_write_tables     the device side: the [B, max_blocks] int64 block table and [B] int64
 *                            context lengths that kyro_paged_attention_mq / kyro_paged_kv_append
 *                            read (attention_kernel.rs:56 layout), written on the context's stream
 *   kyro_copy_blocks         the copy-on-write of a partially matched prefix block
 *
 * Differences from the reference, each so that the tables stay correct for attention:
 *  - The prefix cache is keyed by block contents: a node is one block. A match returns the
 *    blocks holding the longest cached prefix; when it ends inside a block, that block is
 *    partially matched. kyro_bm_allocate_with_prefix shares the whole blocks and gives the
 *    request a fresh block plus a pending copy of the partially matched one (the request writes
 *    its own tokens into the rest of that block, so it cannot be shared). The matched token
 *    count is the reference's cached_token_count (partial matches included).
 *  - Eviction takes the least recently used leaf of the whole tree (logical clock); the
 *    reference picks among one tree level in HashMap order with wall-clock stamps.
 *  - Every reference (the cache's, each request's, a pending copy's) is dropped exactly once, and
 *    blocks evicted after an insert are returned to the free pool.
 *  - A request's block list grows and shrinks with its token count (kyro_bm_append_slots for
 *    decode and verify rows, kyro_bm_truncate for rejected drafts); the reference only
 *    allocates for the prompt.
 * A kyro_bm / kyro_radix is not thread-safe (the reference's scheduler holds it under a lock).
 */
#ifndef KYRO_BLOCKS_H
#define KYRO_BLOCKS_H

#include <stddef.h>
#include <stdint.h>

#include "kyro_verify.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct kyro_bm_s* kyro_bm;
typedef struct kyro_radix_s* kyro_radix;

/* ---------------------------------------------------------------- prefix cache */

/* RadixCache::new(max_capacity) (radix_cache.rs:38-44), for blocks of block_size tokens. */
int kyro_radix_create(int32_t block_size, int64_t max_capacity, kyro_radix* out);
int kyro_radix_destroy(kyro_radix r);
/* Longest cached prefix of tokens[0..n): up to `cap` block ids into out_blocks, their number in
 * out_num_blocks and the matched token count in out_matched (the last block may hold only part
 * of the match). Marks the matched blocks as used. */
int kyro_radix_match_prefix(kyro_radix r, const uint32_t* tokens, int64_t n, int64_t* out_blocks,
                            int64_t cap, int64_t* out_num_blocks, int64_t* out_matched);
/* Caches tokens[0..n) held by blocks[0..ceil(n / block_size)); then evicts down to capacity.
 * out_taken (optional, one per block): 1 where the cache took the block, 0 where those tokens
 * were already cached. */
int kyro_radix_insert(kyro_radix r, const uint32_t* tokens, int64_t n, const int64_t* blocks,
                      uint8_t* out_taken);
/* Evicts least-recently-used leaves down to capacity; up to `cap` evicted ids into out. */
int kyro_radix_evict_lru(kyro_radix r, int64_t* out, int64_t cap, int64_t* out_n);
int64_t kyro_radix_num_cached_blocks(kyro_radix r);

/* ---------------------------------------------------------------- block manager */

/* BlockManager::new(block_size, num_gpu_blocks, num_cpu_blocks) (block_manager.rs:32-50): all
 * GPU blocks free, a prefix cache of num_gpu_blocks / 3 blocks. */
int kyro_bm_create(int32_t block_size, int64_t num_gpu_blocks, int64_t num_cpu_blocks, kyro_bm* out);
int kyro_bm_destroy(kyro_bm bm);
/* Blocks for a new request's prompt, reusing the longest cached prefix. KYRO_ENOSPACE when the
 * free pool (after evicting cache leaves) cannot hold the rest; nothing changes then.
 * out_cached_tokens: prompt tokens whose K/V is already cached (the request computes the rest).
 * A partially matched block leaves a pending copy (kyro_bm_take_copies). */
int kyro_bm_allocate_with_prefix(kyro_bm bm, uint64_t request_id, const uint32_t* tokens, int64_t n,
                                 int64_t* out_cached_tokens);
/* Blocks for num_tokens without prefix caching (block_manager.rs:107-124). */
int kyro_bm_allocate(kyro_bm bm, uint64_t request_id, int64_t num_tokens);
/* Room for n more tokens of a request (a decode token, the k + 1 rows of a verify step). */
int kyro_bm_append_slots(kyro_bm bm, uint64_t request_id, int64_t n);
/* Shrinks a request to num_tokens (>= its prompt length), releasing blocks no longer needed. */
int kyro_bm_truncate(kyro_bm bm, uint64_t request_id, int64_t num_tokens);
/* Ends a request. cache_prompt != 0 hands its prompt blocks to the prefix cache (their K/V must
 * have been written); 0 releases them. */
int kyro_bm_free(kyro_bm bm, uint64_t request_id, int32_t cache_prompt);
/* A request's block ids (up to cap) and token count; out_n receives the full count. */
int kyro_bm_request_blocks(kyro_bm bm, uint64_t request_id, int64_t* out, int64_t cap,
                           int64_t* out_n, int64_t* out_num_tokens);
/* Pending copy-on-write copies (source block -> destination block), handed out once. Queue
 * them (kyro_copy_blocks, for every layer's cache) before any other write into the caches. With
 * cap too small nothing is taken and out_n receives the count. */
int kyro_bm_take_copies(kyro_bm bm, int64_t* src, int64_t* dst, int64_t cap, int64_t* out_n);
int64_t kyro_bm_num_free_blocks(kyro_bm bm);    /* -1 for a null handle */
/* Consistency check for tests and debugging: every block's reference count equals its holders
 * (requests, cache entries, pending copies) and the free pool is exactly the unheld blocks.
 * KYRO_EINVAL with the first disagreement otherwise. */
int kyro_bm_check(kyro_bm bm);
int64_t kyro_bm_num_cached_blocks(kyro_bm bm);  /* -1 for a null handle */
/* The prefix cache's match, as kyro_radix_match_prefix (marks the blocks as used). */
int kyro_bm_match_prefix(kyro_bm bm, const uint32_t* tokens, int64_t n, int64_t* out_blocks,
                         int64_t cap, int64_t* out_num_blocks, int64_t* out_matched);
/* Writes, on ctx's stream, block_table[b][i] = i-th block of request_ids[b] (0 past its blocks)
 * for b < B, i < max_blocks, and context_lens[b] = its token count (context_lens may be NULL).
 * Device pointers: block_table [B, max_blocks] int64, context_lens [B] int64. A request with
 * more than max_blocks blocks, or an unknown id, is KYRO_EINVAL. out_shared (host, may be NULL)
 * receives 1 when some block appears in the tables of two of the requests, else 0: the
 * kv_reuse hint of the attention launch over these tables (KYRO_KV_REUSE_SHARED when 1). */
int kyro_bm_write_tables(kyro_bm bm, kyro_ctx ctx, const uint64_t* request_ids, int32_t B,
                         int32_t max_blocks, int64_t* block_table, int64_t* context_lens,
                         int32_t* out_shared);

/* ---------------------------------------------------------------- block copies */

typedef struct kyro_copy_blocks_params {
    int32_t block_size;
    int32_t num_kv_heads;
    int32_t head_dim;
    int32_t num_blocks;  /* leading dim of the caches */
    int32_t dtype;       /* kyro_dtype of the caches */
} kyro_copy_blocks_params;

/* key_cache[dst[i]] = key_cache[src[i]] and the same for value_cache, i < n, on ctx's stream;
 * src / dst are HOST arrays of block ids. Pairs must not chain (no dst is another pair's src). */
int kyro_copy_blocks(kyro_ctx ctx, const kyro_copy_blocks_params* params, void* key_cache,
                     void* value_cache, const int64_t* src, const int64_t* dst, int64_t n);

#ifdef __cplusplus
}
#endif

#endif /* KYRO_BLOCKS_H */
