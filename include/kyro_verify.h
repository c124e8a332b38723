/*
 * kyro_verify.h — C ABI of the MI355X (gfx950) speculative-decoding verify step.
 *
 * Two device operations replace the two hot functions of Kyro's verify path:
 *
 *   kyro_paged_attention_mq  replaces  PagedAttention::forward
 *                                       (src/model/attention_kernel.rs:22-31, body :59-136)
 *   kyro_spec_verify         replaces  SpeculativeDecoder::verify_drafts
 *                                       (src/speculative.rs:286-339), extended from greedy
 *                                       argmax-match to p/q rejection sampling with the
 *                                       sampling conventions of sample_token
 *                                       (src/worker.rs:267-362)
 *
 * and one writes the cache the attention reads:
 *
 *   kyro_paged_kv_append     replaces  KVCacheManager::append_kv (src/model/kv_cache.rs:49-75)
 *                                       as called before attention (src/model/llama.rs:80-84),
 *                                       for a block-table cache instead of per-request tensors
 *
 * Everything else here is plumbing a Rust `extern "C"` block (or ctypes, or C++) binds to:
 * a per-device context that owns a HIP stream and a scratch arena, opaque device buffers,
 * and status codes with a thread-local message.
 *
 * Conventions
 *  - Every data pointer passed to a compute entry point is a DEVICE pointer on the context's
 *    device (from kyro_buf_ptr, hipMalloc, or a torch tensor's data_ptr()).
 *  - Compute calls are asynchronous on the context's stream. Errors that only the device can
 *    see (an out-of-range block id, a context length beyond the block table) are latched in a
 *    device word; the offending blocks are skipped, never dereferenced, and the next
 *    kyro_sync()/kyro_check() on the context returns KYRO_EINVAL with a message.
 *  - No C++ exception crosses this boundary. Every function returns a kyro_status; the text of
 *    the last failure on the calling thread is kyro_last_error().
 *  - A kyro_ctx may be moved between threads but must not be used by two threads at once
 *    (the reference model object is Send but not Sync: src/worker.rs:14, src/model/loader.rs:13).
 */
#ifndef KYRO_VERIFY_H
#define KYRO_VERIFY_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KYRO_ABI_VERSION 9

typedef enum kyro_status {
    KYRO_OK = 0,
    KYRO_EINVAL = 1,       /* bad argument, shape, or (latched) bad block id / context length */
    KYRO_EOOM = 2,         /* device allocation failed */
    KYRO_EHIP = 3,         /* a HIP runtime call failed */
    KYRO_EUNSUPPORTED = 4, /* valid request this build has no kernel for (e.g. head_dim 100) */
    KYRO_ENOSPACE = 5      /* not enough free KV blocks, even after evicting the prefix cache */
} kyro_status;

typedef enum kyro_dtype {
    KYRO_F32 = 0,
    KYRO_BF16 = 1
} kyro_dtype;

typedef struct kyro_ctx_s* kyro_ctx;
typedef struct kyro_buf_s* kyro_buf;

/* ---------------------------------------------------------------- context and errors */

/* Text of the last error raised on the calling thread ("" if none). Never NULL. */
const char* kyro_last_error(void);

/* ABI version of the loaded library (KYRO_ABI_VERSION at build time). */
int kyro_abi_version(void);

/* Creates a context on HIP device `device` with its own non-blocking stream. */
int kyro_ctx_create(int device, kyro_ctx* out);
int kyro_ctx_destroy(kyro_ctx ctx);

/* Makes subsequent calls on `ctx` run on `hip_stream` (a hipStream_t; NULL = HIP's null stream,
 * which is what torch's default stream handle 0 denotes). A new context uses a stream of its own
 * until this is called. The caller keeps ownership of the stream. */
int kyro_ctx_set_stream(kyro_ctx ctx, void* hip_stream);

/* Grows the context's scratch arena to at least `bytes` now, so later calls do not allocate.
 * A call that needs more arena than the context holds synchronises the stream, frees the arena
 * and allocates a larger one; kernels captured into a HIP graph before that point would then
 * address freed memory. A caller that captures calls into a graph should reserve the largest
 * arena those calls need first (or re-capture after a growth). The balanced attention schedule
 * and the one-launch decode sampler (kyro_sample_tokens without processors, top-k or top-p) also
 * keep small counters in the context that every launch returns to zero, so their launches replay
 * from a graph as they run eagerly. */
int kyro_ctx_reserve(kyro_ctx ctx, size_t bytes);

/* Waits for all work queued on the context's stream, then reports latched device errors. */
int kyro_sync(kyro_ctx ctx);

/* Reports (and clears) latched device errors after waiting for the stream. Same as kyro_sync. */
int kyro_check(kyro_ctx ctx);

/* ---------------------------------------------------------------- device buffers */

int kyro_buf_alloc(kyro_ctx ctx, size_t bytes, kyro_buf* out);
int kyro_buf_free(kyro_buf buf);
void* kyro_buf_ptr(kyro_buf buf);
size_t kyro_buf_size(kyro_buf buf);
/* Synchronous host->device / device->host copies on the context's stream. */
int kyro_buf_upload(kyro_ctx ctx, kyro_buf dst, size_t dst_offset, const void* src, size_t bytes);
int kyro_buf_download(kyro_ctx ctx, void* dst, kyro_buf src, size_t src_offset, size_t bytes);

/* ---------------------------------------------------------------- paged attention */

/* Attention-kernel choice. AUTO picks the MFMA kernel whenever it applies (a block_size that is a
 * multiple of 16, and head_dim 128 with bf16 or f32 caches, or with bf16 caches head_dim 80, 112
 * or any multiple of 32 from 64 to 256), whatever the number of query rows, and the vector kernel
 * otherwise (every other head_dim that is a multiple of 8 up to 256, block sizes that are not
 * multiples of 16). */
typedef enum kyro_attn_path {
    KYRO_ATTN_AUTO = 0,
    KYRO_ATTN_VECTOR = 1,
    KYRO_ATTN_MFMA = 2
} kyro_attn_path;

/* How often one launch reads each cached (block, kv head) slab; a cache-policy hint for the MFMA
 * kernel's K/V loads that never changes results. Streaming loads (the nontemporal hint) read
 * data used once ~14% faster, but a slab read again soon after (by another row group of the
 * same kv head, or by another sequence whose table holds the same block) then comes from HBM
 * again instead of L2.
 *   AUTO:   streaming when each slab is read by one workgroup, i.e. a kv head's query rows
 *           (GQA group x max_q_len) fit one row group (16, 32, 64 or 80 rows for bf16
 *           caches); cached otherwise. With 64- and 80-row groups the choice is made per
 *           sequence: those whose rows fit one group stream. Right when no two sequences of the
 *           batch share a block.
 *   SHARED: cached loads; for tables that share blocks between sequences (prefix caching;
 *           kyro_bm_write_tables reports it).
 *   STREAM: streaming loads regardless. */
typedef enum kyro_kv_reuse {
    KYRO_KV_REUSE_AUTO = 0,
    KYRO_KV_REUSE_SHARED = 1,
    KYRO_KV_REUSE_STREAM = 2
} kyro_kv_reuse;

/* How the MFMA kernel spreads work over the chip. Results do not depend on it beyond float
 * rounding of split merges.
 *   AUTO:     BALANCED when num_splits is 0, the batch has at most 1024 sequences and either
 *             max_blocks_per_seq > 256 or GRID would split contexts; GRID otherwise.
 *   GRID:     one workgroup per (sequence, kv head pair, context split, row group), with
 *             num_splits splits of max_blocks_per_seq (0: chosen from the shapes alone).
 *   BALANCED: a persistent grid of one workgroup per CU reads the context lengths on the
 *             device, splits only sequences longer than the per-CU share of the work, and starts
 *             the longest work items first (at most 1024 sequences, num_splits must be 0; an
 *             extra combine launch always follows). For batches whose context lengths differ
 *             widely. */
typedef enum kyro_attn_schedule {
    KYRO_ATTN_SCHEDULE_AUTO = 0,
    KYRO_ATTN_SCHEDULE_GRID = 1,
    KYRO_ATTN_SCHEDULE_BALANCED = 2
} kyro_attn_schedule;

/* Mirrors PagedAttention { block_size, num_heads, head_dim, num_kv_heads }
 * (src/model/attention_kernel.rs:4-9) plus the shapes the Rust side reads off its tensors. */
typedef struct kyro_paged_attention_params {
    int32_t block_size;          /* tokens per KV block (Kyro uses 16: src/model/llama.rs:46) */
    int32_t num_heads;           /* query heads H */
    int32_t head_dim;            /* D: a multiple of 8, at most 256 */
    int32_t num_kv_heads;        /* Hkv; H % Hkv == 0; query head h reads kv head h / (H/Hkv) */
    int32_t batch_size;          /* B */
    int32_t total_q;             /* rows of `query`: B when q_start_loc is NULL */
    int32_t max_blocks_per_seq;  /* width of block_table */
    int32_t num_blocks;          /* leading dim of the caches; ids outside [0,num_blocks) latch EINVAL */
    int32_t dtype;               /* kyro_dtype of query and caches */
    int32_t out_dtype;           /* kyro_dtype of out (the reference returns F32) */
    int32_t causal;              /* 1: query j of a sequence with q_len rows sees keys
                                    [0, ctx - q_len + j]; 0: every query sees [0, ctx) */
    float scale;                 /* 0 => 1/sqrt(head_dim) (attention_kernel.rs:69) */
    int32_t path;                /* kyro_attn_path */
    int32_t num_splits;          /* context splits per (sequence, kv head); 0 => automatic */
    int32_t max_q_len;           /* upper bound on query rows per sequence; 0 => 1 without
                                    q_start_loc, total_q with it (sizes the split workspace;
                                    a sequence above it latches KYRO_EINVAL) */
    int32_t kv_reuse;            /* kyro_kv_reuse (0 => AUTO) */
    int32_t schedule;            /* kyro_attn_schedule (0 => AUTO); MFMA kernel only */
} kyro_paged_attention_params;

/*
 * Multi-query paged attention over a block-table KV cache.
 *   query        [total_q, H, D]                    dtype
 *   q_start_loc  [B+1] int32, rows of sequence b are [q_start_loc[b], q_start_loc[b+1]);
 *                NULL => one row per sequence (the reference's [B, H, D] query)
 *   key_cache    [num_blocks, Hkv, block_size, D]   dtype   (attention_kernel.rs:54)
 *   value_cache  [num_blocks, Hkv, block_size, D]   dtype   (attention_kernel.rs:55)
 *   block_table  [B, max_blocks_per_seq] int64               (attention_kernel.rs:56)
 *   context_lens [B] int64; includes the sequence's own query positions (llama.rs:83-84)
 *   out          [total_q, H, D]                    out_dtype
 * A sequence with context length 0 gets zeros (attention_kernel.rs:77-84); a partial last
 * block is truncated (:91-93); block ids may repeat (aliasing, the test at :214).
 */
int kyro_paged_attention_mq(kyro_ctx ctx, const kyro_paged_attention_params* params,
                            const void* query, const int32_t* q_start_loc,
                            const void* key_cache, const void* value_cache,
                            const int64_t* block_table, const int64_t* context_lens,
                            void* out);

/* Scratch bytes a kyro_paged_attention_mq call with these params takes from the context's arena
 * (has_q_start_loc: whether the call passes q_start_loc). Host only, no device work; ctx may be
 * NULL, which sizes for a 256-CU device. A caller that captures calls into a HIP graph passes the
 * largest of these to kyro_ctx_reserve first. No counterpart in the reference (candle allocates
 * per op). */
int kyro_paged_attention_workspace(kyro_ctx ctx, const kyro_paged_attention_params* params,
                                   int has_q_start_loc, size_t* bytes);

/* What a kyro_paged_attention_mq call with these params launches (kernel instance, schedule,
 * splits, workgroups), as text for logs and benchmarks. Host only, like the workspace query; ctx
 * may be NULL (a 256-CU device). buf gets at most len bytes (terminated), *needed (may be NULL)
 * the full length with its terminator. No counterpart in the reference. */
int kyro_paged_attention_describe(kyro_ctx ctx, const kyro_paged_attention_params* params, int has_q_start_loc,
                                  char* buf, size_t len, size_t* needed);

/* The balanced schedule's plan for one batch, computed on the host with the chunk and split
 * arithmetic the device plan runs, from host copies of the context lengths and the per-sequence
 * query rows (q_lens NULL: one row each). For analysis and tests; no counterpart in the
 * reference. num_cus 0 means 256; chunk_quarters 0 means the library's chunk length (a sequence
 * longer than the per-workgroup share L of the work splits into chunks of about
 * L x chunk_quarters / 4 blocks, 5L/4 by default; other values model other chunk lengths, the
 * slot bound included). Fails with KYRO_EINVAL when the params
 * would run on the grid schedule. out_splits [B] (may be NULL): splits per sequence (0 for a
 * sequence without rows). */
typedef struct kyro_attention_plan {
    int32_t grid;          /* persistent workgroups */
    int32_t chunk_blocks;  /* 16-token slots per split of a sequence that splits (the MFMA
                              kernels walk a block of 16 m tokens as m slots) */
    int64_t items;         /* work items: sequence x kv head group x split x row group, one
                              partial-state slot each */
    int64_t slot_bound;    /* partial-state slots a launch with these params sizes; the device
                              latches KYRO_EINVAL instead of running a plan with more items */
} kyro_attention_plan;

int kyro_paged_attention_plan(const kyro_paged_attention_params* params, int num_cus, int chunk_quarters,
                              const int64_t* context_lens, const int32_t* q_lens, int32_t* out_splits,
                              kyro_attention_plan* out);

/* ---------------------------------------------------------------- speculative verify */

typedef struct kyro_spec_verify_params {
    int32_t batch_size;   /* B */
    int32_t max_draft;    /* kmax: target_logits has kmax+1 rows per sequence, draft kmax */
    int32_t vocab_size;   /* V */
    int32_t logits_dtype; /* kyro_dtype of both logits tensors (KYRO_F32) */
    int32_t window;       /* draft positions whose logit rows are read before the first
                             acceptance scan; rows after it are read only for sequences that
                             accept all of them. 0 = default: 3, or every row in one pass when
                             all rows of the batch total at most 64 MB; >= max_draft + 1 reads
                             every row in one pass. Outputs do not depend on it, only the time
                             does: a caller that tracks its acceptance can tune it (measured best:
                             3 for Llama-3-8B with 1.4 of 7 drafts accepted on average, 1 for a
                             mixed batch with 0.7 of up to 8). */
} kyro_spec_verify_params;

/*
 * Fused acceptance for one verify step, per sequence b with k = num_draft[b] <= kmax and
 * T = temperature[b]:
 *   T > 0:  p_i = softmax(target_logits[b,i,:] / T) for i <= k, q_i = softmax(draft_logits[b,i,:] / T)
 *           for i < k. Draft x_i = draft_tokens[b,i] is accepted while u_accept[b,i] < min(1, p_i(x_i)
 *           / q_i(x_i)) (q_i(x_i) == 0 accepts). At the first rejection j one token is drawn from
 *           max(p_j - q_j, 0) / sum with u_resample[b]; after k acceptances the bonus token is drawn
 *           from p_k. Draws are the inverse-CDF walk in index order of sample_token
 *           (src/worker.rs:352-360): the first v with cumsum(v) >= u * total; if rounding leaves
 *           none, the last index with positive mass. A residual that sums to zero falls back to p_j.
 *   T <= 0: greedy, as verify_drafts (src/speculative.rs:315-323): accept while argmax(target row i)
 *           == x_i (ties -> lowest index), emit argmax(target row j) at the first mismatch, and
 *           argmax(target row k) as the bonus after k acceptances.
 * Outputs: out_accepted[b] = accepted drafts in [0, k]; out_tokens[b, 0..out_accepted[b]] = the
 * accepted drafts, out_tokens[b, out_accepted[b]] = the correction or bonus token, the rest
 * 0xFFFFFFFF. Optional (NULL to skip): out_p_draft[b,i] = p_i(x_i), out_q_draft[b,i] = q_i(x_i)
 * for the drafts the scan evaluates, i <= out_accepted[b] and i < k, of sampled sequences; NaN
 * elsewhere (the scan stops at the first rejection, as the loop of speculative.rs:315-323) and
 * for greedy sequences.
 * Shapes: target_logits [B, kmax+1, V], draft_logits [B, kmax, V] (may be NULL when every
 * sequence is greedy or kmax == 0), draft_tokens [B, kmax] uint32, num_draft [B] int32,
 * temperature [B] f32, u_accept [B, kmax] f32, u_resample [B] f32; uniforms in (0, 1).
 */
int kyro_spec_verify(kyro_ctx ctx, const kyro_spec_verify_params* params,
                     const void* target_logits, const void* draft_logits,
                     const uint32_t* draft_tokens, const int32_t* num_draft,
                     const float* temperature, const float* u_accept, const float* u_resample,
                     int32_t* out_accepted, uint32_t* out_tokens,
                     float* out_p_draft, float* out_q_draft);

/* Scratch bytes a kyro_spec_verify call with these params takes from the context's arena. Host
 * only, no device work. */
int kyro_spec_verify_workspace(const kyro_spec_verify_params* params, size_t* bytes);

/* What a kyro_spec_verify call with these params launches (window, chunking, kernels), as text
 * for logs and benchmarks. Host only; buf gets at most len bytes (terminated), *needed (may be
 * NULL) the full length with its terminator. No counterpart in the reference. */
int kyro_spec_verify_describe(const kyro_spec_verify_params* params, char* buf, size_t len, size_t* needed);

/* Maximum scratch of kyro_spec_verify_noalloc, in bytes (16 MiB). */
#define KYRO_SPEC_VERIFY_NOALLOC_SCRATCH_BYTES (16u << 20)

/*
 * kyro_spec_verify with no allocation: the same kernels, arguments and results, with the scratch
 * (chunk statistics, per-sequence plans, chunk sums) in a fixed array of this library on each
 * device instead of the context's arena. It calls no hipMalloc / hipFree and no allocating
 * routine, so it can run where allocation is not allowed: code under HIP graph capture, tight
 * serving loops, harnesses that forbid it. No counterpart in the reference; this is for callers
 * that cannot allocate.
 * Limit: a call whose scratch (kyro_spec_verify_workspace) exceeds
 * KYRO_SPEC_VERIFY_NOALLOC_SCRATCH_BYTES fails with KYRO_EINVAL (about B x (2 kmax + 1) x
 * ceil(V / 4096) x 8 bytes: B 64, kmax 7, V 128256 needs 270 KB; B 1024, kmax 8, V 256000 needs
 * 9 MB). The array is set up at kyro_ctx_create and held until the process ends. Every call on a
 * device shares that device's array: calls that overlap on one device (two contexts, or two
 * streams) race and must be ordered by the caller. The kernels write every scratch entry they
 * read within a call, so the last call's contents never reach the next one.
 */
int kyro_spec_verify_noalloc(kyro_ctx ctx, const kyro_spec_verify_params* params,
                             const void* target_logits, const void* draft_logits,
                             const uint32_t* draft_tokens, const int32_t* num_draft,
                             const float* temperature, const float* u_accept, const float* u_resample,
                             int32_t* out_accepted, uint32_t* out_tokens,
                             float* out_p_draft, float* out_q_draft);

/* ---------------------------------------------------------------- paged KV write */

typedef struct kyro_kv_append_params {
    int32_t block_size;          /* tokens per KV block */
    int32_t num_kv_heads;        /* Hkv */
    int32_t head_dim;            /* D, a multiple of 8 */
    int32_t batch_size;          /* B */
    int32_t total_q;             /* rows of key / value: B when q_start_loc is NULL */
    int32_t max_blocks_per_seq;  /* width of block_table */
    int32_t num_blocks;          /* leading dim of the caches; ids outside [0,num_blocks) latch EINVAL */
    int32_t src_dtype;           /* kyro_dtype of key / value */
    int32_t cache_dtype;         /* kyro_dtype of the caches; F32 -> BF16 rounds to nearest even */
    int32_t max_q_len;           /* upper bound on new rows per sequence; 0 => 1 without
                                    q_start_loc, total_q with it */
} kyro_kv_append_params;

/*
 * Writes each sequence's new K/V rows into the block-table cache, where attention reads them.
 * KVCacheManager::append_kv (src/model/kv_cache.rs:49-75) concatenates a request's new
 * [1, seq_len, Hkv, D] rows onto its cache and grows num_cached_tokens by seq_len; llama.rs:80-84
 * appends before attention, so the context length attention sees includes the new rows. Here the
 * caller passes that context length: new row j of sequence b (q_len rows) goes to token position
 * p = context_lens[b] - q_len + j, i.e. slot p % block_size of block block_table[b][p / block_size].
 *   key, value   [total_q, Hkv, D]                  src_dtype
 *   q_start_loc  [B+1] int32 as for kyro_paged_attention_mq; NULL => one row per sequence
 *   block_table  [B, max_blocks_per_seq] int64
 *   context_lens [B] int64, after the append (>= q_len, <= max_blocks_per_seq * block_size)
 *   key_cache, value_cache [num_blocks, Hkv, block_size, D]  cache_dtype (written in place; a bf16 row widens exactly into an f32 cache)
 * Only the new rows' slots are written. Two sequences must not map a new row to the same slot
 * (shared prefix blocks hold only old tokens). A bad block id, context length or q_start_loc
 * latches KYRO_EINVAL for the next kyro_sync and the offending rows are not written.
 */
int kyro_paged_kv_append(kyro_ctx ctx, const kyro_kv_append_params* params,
                         const void* key, const void* value, const int32_t* q_start_loc,
                         const int64_t* block_table, const int64_t* context_lens,
                         void* key_cache, void* value_cache);

#ifdef __cplusplus
}
#endif

#endif /* KYRO_VERIFY_H */
