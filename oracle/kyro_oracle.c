/*
 * kyro_oracle.c — CPU oracle for the speculative-decoding verify step.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker the GPU path is compared against; only the
 * tests, the smoke check and the CPU-baseline leg of the benchmark load it. The product path
 * (libkyro_verify.so) never links, loads or falls back to it.
 *
 * Built twice from this one source:
 *   libkyro_oracle.so      ACC = double  — the parity oracle
 *   libkyro_oracle_f32.so  ACC = float   — the CPU baseline: the same algorithm in the reference's
 *                                          f32 arithmetic (candle CPU tensors are f32)
 *
 * What each function restates (paths relative to the Kyro source tree):
 *   oracle_paged_attention_mq  src/model/attention_kernel.rs:59-136 — per sequence, gather the
 *       context through the block table 16 tokens at a time (:86-108), softmax over the
 *       scaled scores (:69,:102,:112), weighted sum of V (:116-130); ctx = 0 gives zeros
 *       (:77-84); the partial last block is truncated (:91-93); GQA maps query head h to
 *       kv head h / (H/Hkv) (:34-48). It is textbook attention in the reference's layouts; it
 *       does NOT reproduce the reference's score-layout permutation at :104-111, which mixes
 *       heads whenever num_heads > 1 and ctx > 1. Extended to q_len query rows per sequence
 *       with the causal rule of src/model/llama.rs:83-84,109 (the new rows' K/V are appended
 *       before attention, so ctx includes them and row j sees keys [0, ctx - q_len + j]).
 *   oracle_spec_verify  src/speculative.rs:286-339 (greedy accept-until-mismatch, emitting the
 *       target argmax at the first mismatch) extended to p/q rejection sampling (Leviathan et al.
 *       2023, Algorithm 1; Chen et al. 2023) with the sampling conventions of
 *       src/worker.rs:290-360: T <= 0 is argmax, logits are divided by T, softmax subtracts the
 *       max, and a draw is the inverse-CDF walk in index order `r -= p; if r <= 0 -> id`.
 *   oracle_sample_token  src/worker.rs:267-362 with the uniform passed in (the reference draws it
 *       from an unseeded rand::rng()).
 *   oracle_sample_decode  src/worker.rs:141-197 (logit bias, frequency / presence penalty as a
 *       sparse additive list, grammar mask as bits) followed by sample_token, for a batch.
 *   oracle_kv_append  src/model/kv_cache.rs:49-75 (append_kv: a request's new [seq_len, Hkv, D]
 *       rows go after its cached ones and num_cached_tokens grows by seq_len) for a block-table
 *       cache, as called before attention at src/model/llama.rs:80-84: new row j of a sequence
 *       with q_len new rows and context length ctx (after the append) is token ctx - q_len + j,
 *       slot (p % bs) of block table[b][p / bs]. f32 rows stored into a bf16 cache round to
 *       nearest even; NaN becomes 0x7FC0.
 *
 * Pinning (tests/test_oracle.py, tests/test_kv_append_oracle.py): attention against torch-CPU scaled_dot_product_attention on
 * the gathered contiguous KV, and the closed forms all-ones -> 1, ctx 0 -> 0, single key -> V,
 * equal keys -> mean(V), block-permutation invariance, GQA == MHA with repeated KV, causal row j
 * == non-causal over ctx - q_len + j + 1 keys. Sampler against the argmax/sampling known-answer
 * tests of src/worker.rs:395-449, numpy searchsorted for the inverse-CDF walk, q == p accepting
 * everything, and a chi-square test that the first emitted token follows p_0 whatever q is
 * (Leviathan et al. 2023, Theorem 1) — a residual with a wrong sign or a dropped max(.,0) fails it.
 * KV append against the reference's append_kv tests (context 2 then 5; ones in, ones cached),
 * torch's float32 -> bfloat16 conversion, a gather of the written positions through the block
 * table that returns the new rows with every other slot unchanged, and attention after the
 * append equal to attention over the contiguous old + new K/V.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef ORACLE_F32
typedef float acc_t;
#define ACC_EXP expf
#define ACC_SQRT sqrtf
#else
typedef double acc_t;
#define ACC_EXP exp
#define ACC_SQRT sqrt
#endif

#define ORACLE_OK 0
#define ORACLE_EINVAL 1

static inline float bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* ------------------------------------------------------------------ attention */

typedef struct oracle_attn_args {
    int32_t block_size, num_heads, head_dim, num_kv_heads;
    int32_t batch_size, total_q, max_blocks_per_seq, num_blocks;
    int32_t dtype;  /* 0 = f32, 1 = bf16 (uint16 storage) */
    int32_t causal;
    double scale;   /* <= 0 => 1/sqrt(head_dim) */
    const void* query;          /* [total_q, H, D] */
    const int32_t* q_start_loc; /* [B+1] or NULL (one row per sequence) */
    const void* key_cache;      /* [num_blocks, Hkv, bs, D] */
    const void* value_cache;
    const int64_t* block_table; /* [B, max_blocks_per_seq] */
    const int64_t* context_lens;/* [B] */
    double* out;                /* [total_q, H, D] */
} oracle_attn_args;

static inline acc_t load_elem(const void* base, int dtype, size_t idx) {
    if (dtype == 1) return (acc_t)bf16_to_f32(((const uint16_t*)base)[idx]);
    return (acc_t)((const float*)base)[idx];
}

typedef struct attn_job {
    const oracle_attn_args* a;
    int64_t next;       /* shared work counter over (b, h) */
    pthread_mutex_t mu;
    int status;
} attn_job;

/* One (sequence, query head) pair: every query row of the sequence for that head. */
static int attn_one(const oracle_attn_args* a, int b, int h, acc_t* scores, acc_t* acc) {
    const int D = a->head_dim, H = a->num_heads, Hkv = a->num_kv_heads, bs = a->block_size;
    const int group = H / Hkv;
    const int kvh = h / group;
    const int64_t ctx = a->context_lens[b];
    const int q0 = a->q_start_loc ? a->q_start_loc[b] : b;
    const int q1 = a->q_start_loc ? a->q_start_loc[b + 1] : b + 1;
    const int q_len = q1 - q0;
    const acc_t scale = a->scale > 0 ? (acc_t)a->scale : (acc_t)1 / ACC_SQRT((acc_t)D);
    if (ctx < 0 || ctx > (int64_t)a->max_blocks_per_seq * bs) return ORACLE_EINVAL;
    for (int j = 0; j < q_len; ++j) {
        const size_t qrow = ((size_t)(q0 + j) * H + h) * D;
        double* o = a->out + qrow;
        int64_t visible = a->causal ? ctx - q_len + j + 1 : ctx;
        if (visible > ctx) visible = ctx;
        if (visible <= 0) {
            for (int d = 0; d < D; ++d) o[d] = 0.0;
            continue;
        }
        acc_t m = -INFINITY;
        for (int64_t t = 0; t < visible; ++t) {
            const int64_t blk = a->block_table[(size_t)b * a->max_blocks_per_seq + t / bs];
            if (blk < 0 || blk >= a->num_blocks) return ORACLE_EINVAL;
            const size_t kbase = (((size_t)blk * Hkv + kvh) * bs + (size_t)(t % bs)) * D;
            acc_t s = 0;
            for (int d = 0; d < D; ++d)
                s += load_elem(a->query, a->dtype, qrow + d) * load_elem(a->key_cache, a->dtype, kbase + d);
            s *= scale;
            scores[t] = s;
            if (s > m) m = s;
        }
        acc_t z = 0;
        for (int64_t t = 0; t < visible; ++t) {
            scores[t] = ACC_EXP(scores[t] - m);
            z += scores[t];
        }
        for (int d = 0; d < D; ++d) acc[d] = 0;
        for (int64_t t = 0; t < visible; ++t) {
            const int64_t blk = a->block_table[(size_t)b * a->max_blocks_per_seq + t / bs];
            const size_t vbase = (((size_t)blk * Hkv + kvh) * bs + (size_t)(t % bs)) * D;
            const acc_t w = scores[t];
            for (int d = 0; d < D; ++d) acc[d] += w * load_elem(a->value_cache, a->dtype, vbase + d);
        }
        for (int d = 0; d < D; ++d) o[d] = (double)(acc[d] / z);
    }
    return ORACLE_OK;
}

static void* attn_worker(void* arg) {
    attn_job* job = (attn_job*)arg;
    const oracle_attn_args* a = job->a;
    const int64_t total = (int64_t)a->batch_size * a->num_heads;
    int64_t max_ctx = 1;
    for (int b = 0; b < a->batch_size; ++b)
        if (a->context_lens[b] > max_ctx) max_ctx = a->context_lens[b];
    acc_t* scores = (acc_t*)malloc(sizeof(acc_t) * (size_t)max_ctx);
    acc_t* acc = (acc_t*)malloc(sizeof(acc_t) * (size_t)a->head_dim);
    for (;;) {
        pthread_mutex_lock(&job->mu);
        int64_t w = job->next++;
        pthread_mutex_unlock(&job->mu);
        if (w >= total) break;
        int rc = attn_one(a, (int)(w / a->num_heads), (int)(w % a->num_heads), scores, acc);
        if (rc != ORACLE_OK) {
            pthread_mutex_lock(&job->mu);
            job->status = rc;
            pthread_mutex_unlock(&job->mu);
        }
    }
    free(scores);
    free(acc);
    return NULL;
}

int oracle_paged_attention_mq(const oracle_attn_args* a, int threads) {
    if (!a || a->block_size <= 0 || a->num_heads <= 0 || a->head_dim <= 0 || a->num_kv_heads <= 0 ||
        a->num_heads % a->num_kv_heads != 0 || a->batch_size < 0)
        return ORACLE_EINVAL;
    attn_job job;
    job.a = a;
    job.next = 0;
    job.status = ORACLE_OK;
    pthread_mutex_init(&job.mu, NULL);
    if (threads < 1) threads = 1;
    if (threads == 1) {
        attn_worker(&job);
    } else {
        pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)threads);
        for (int i = 0; i < threads; ++i) pthread_create(&th[i], NULL, attn_worker, &job);
        for (int i = 0; i < threads; ++i) pthread_join(th[i], NULL);
        free(th);
    }
    pthread_mutex_destroy(&job.mu);
    return job.status;
}

/* ------------------------------------------------------------------ sampling */

/* argmax with the lowest index winning ties. */
static int argmax_f32(const float* x, int n) {
    int best = 0;
    for (int v = 1; v < n; ++v)
        if (x[v] > x[best]) best = v;
    return best;
}

/* p = softmax(x / T) with the max subtracted (src/worker.rs:298,314-323). */
static void softmax_t(const float* x, int n, double T, acc_t* p) {
    acc_t m = -INFINITY;
    for (int v = 0; v < n; ++v) {
        acc_t y = (acc_t)x[v] / (acc_t)T;
        p[v] = y;
        if (y > m) m = y;
    }
    acc_t z = 0;
    for (int v = 0; v < n; ++v) {
        p[v] = ACC_EXP(p[v] - m);
        z += p[v];
    }
    for (int v = 0; v < n; ++v) p[v] /= z;
}

/* Inverse-CDF draw in index order over unnormalised masses w (src/worker.rs:352-360): the first v
 * whose running sum reaches u * total. If rounding leaves no crossing, the last index with
 * positive mass. *margin = distance of u from the nearest CDF boundary of the chosen token, in
 * normalised units (a draw with margin < 1e-5 may legitimately differ under f32 rounding). */
static int inverse_cdf(const acc_t* w, int n, double u, double* margin) {
    acc_t total = 0;
    for (int v = 0; v < n; ++v) total += w[v];
    const acc_t target = (acc_t)u * total;
    acc_t cum = 0, prev = 0;
    int last_pos = n - 1;
    for (int v = 0; v < n; ++v) {
        if (w[v] > 0) last_pos = v;
        prev = cum;
        cum += w[v];
        if (w[v] > 0 && cum >= target) {
            if (margin) {
                double lo = (double)(target - prev) / (double)total;
                double hi = (double)(cum - target) / (double)total;
                *margin = lo < hi ? lo : hi;
            }
            return v;
        }
    }
    if (margin) *margin = 0.0;
    return last_pos;
}

/*
 * Verify step for B sequences. Greedy sequences (T <= 0) follow src/speculative.rs:315-323 and add
 * the argmax of target row k as the bonus token after full acceptance. Outputs as in
 * include/kyro_verify.h (kyro_spec_verify) plus two margin arrays:
 *   accept_margin [B, kmax]: |u_i - min(1, p_i(x_i)/q_i(x_i))| for every evaluated position (NaN
 *                            for positions after the first rejection and for greedy sequences)
 *   resample_margin [B]:     margin of the final inverse-CDF draw (+inf for greedy sequences)
 */
int oracle_spec_verify(int32_t B, int32_t kmax, int32_t V, const float* target, const float* draft,
                       const uint32_t* draft_tokens, const int32_t* num_draft,
                       const float* temperature, const float* u_accept, const float* u_resample,
                       int32_t* out_accepted, uint32_t* out_tokens, double* out_p, double* out_q,
                       double* accept_margin, double* resample_margin) {
    if (B < 0 || kmax < 0 || V <= 0) return ORACLE_EINVAL;
    acc_t* p = (acc_t*)malloc(sizeof(acc_t) * (size_t)V);
    acc_t* q = (acc_t*)malloc(sizeof(acc_t) * (size_t)V);
    for (int b = 0; b < B; ++b) {
        const int k = num_draft[b];
        if (k < 0 || k > kmax) {
            free(p);
            free(q);
            return ORACLE_EINVAL;
        }
        const double T = temperature[b];
        for (int i = 0; i <= kmax; ++i) out_tokens[(size_t)b * (kmax + 1) + i] = 0xFFFFFFFFu;
        for (int i = 0; i < kmax; ++i) {
            if (out_p) out_p[(size_t)b * kmax + i] = NAN;
            if (out_q) out_q[(size_t)b * kmax + i] = NAN;
            if (accept_margin) accept_margin[(size_t)b * kmax + i] = NAN;
        }
        const float* trow = target + (size_t)b * (kmax + 1) * V;
        const float* drow = draft ? draft + (size_t)b * kmax * V : NULL;
        const uint32_t* x = draft_tokens + (size_t)b * kmax;
        int j = 0;
        uint32_t emit;
        if (T <= 0) {
            while (j < k) {
                int top = argmax_f32(trow + (size_t)j * V, V);
                if ((uint32_t)top != x[j]) break;
                ++j;
            }
            emit = (uint32_t)argmax_f32(trow + (size_t)j * V, V);
            if (resample_margin) resample_margin[b] = INFINITY;
        } else {
            int rejected = 0;
            while (j < k) {
                softmax_t(trow + (size_t)j * V, V, T, p);
                softmax_t(drow + (size_t)j * V, V, T, q);
                const uint32_t xi = x[j];
                if (xi >= (uint32_t)V) {
                    free(p);
                    free(q);
                    return ORACLE_EINVAL;
                }
                const double pv = (double)p[xi], qv = (double)q[xi];
                if (out_p) out_p[(size_t)b * kmax + j] = pv;
                if (out_q) out_q[(size_t)b * kmax + j] = qv;
                const double ratio = qv > 0 ? (pv / qv < 1.0 ? pv / qv : 1.0) : 1.0;
                const double u = (double)u_accept[(size_t)b * kmax + j];
                if (accept_margin) accept_margin[(size_t)b * kmax + j] = fabs(u - ratio);
                const int accept = qv > 0 ? (u < ratio) : 1;
                if (!accept) {
                    rejected = 1;
                    break;
                }
                ++j;
            }
            if (rejected) {
                /* residual max(p - q, 0); p and q still hold row j */
                acc_t total = 0;
                for (int v = 0; v < V; ++v) {
                    acc_t r = p[v] - q[v];
                    q[v] = r > 0 ? r : 0;
                    total += q[v];
                }
                const acc_t* w = total > 0 ? q : p;
                emit = (uint32_t)inverse_cdf(w, V, (double)u_resample[b],
                                             resample_margin ? &resample_margin[b] : NULL);
            } else {
                softmax_t(trow + (size_t)k * V, V, T, p);
                emit = (uint32_t)inverse_cdf(p, V, (double)u_resample[b],
                                             resample_margin ? &resample_margin[b] : NULL);
            }
        }
        out_accepted[b] = j;
        for (int i = 0; i < j; ++i) out_tokens[(size_t)b * (kmax + 1) + i] = x[i];
        out_tokens[(size_t)b * (kmax + 1) + j] = emit;
    }
    free(p);
    free(q);
    return ORACLE_OK;
}

/*
 * sample_token (src/worker.rs:267-362) on scaled logits z, with the uniform `u` passed in:
 * optional top-k keeping the k largest z (:306-311; ties go to the lower index), softmax with the
 * max subtracted (:314-323), optional top-p over the probabilities sorted descending (ties: lower
 * index), cut after the first entry whose running sum exceeds top_p (:325-338), then the walk
 * `r -= p; if r <= 0` (:340-360) with r = u * (mass of the cut) after top-p and r = u otherwise.
 * The walk runs in index order without filters and in the descending order after top-k alone
 * (the reference leaves that order to select_nth_unstable). Fallbacks: the most probable kept
 * token after top-p, the last one walked otherwise. *margin (if given) receives the distance of
 * r (and of top_p) from the nearest running sum that would change the decision.
 */
static const acc_t* g_sort_keys;
static int cmp_desc(const void* a, const void* b) {
    const acc_t x = g_sort_keys[*(const int*)a], y = g_sort_keys[*(const int*)b];
    if (x > y) return -1;
    if (x < y) return 1;
    return (*(const int*)a) - (*(const int*)b);
}

static int sample_core(const float* z, int32_t V, float top_p, int32_t top_k, double u, double* margin) {
    acc_t* zz = (acc_t*)malloc(sizeof(acc_t) * (size_t)V);
    int* ids = (int*)malloc(sizeof(int) * (size_t)V);
    acc_t* pr = (acc_t*)malloc(sizeof(acc_t) * (size_t)V);
    for (int v = 0; v < V; ++v) {
        zz[v] = (acc_t)z[v];
        ids[v] = v;
    }
    int n = V;
    const int filtered = (top_k > 0 && top_k < V) || top_p < 1.0f;
    if (filtered) {  /* descending z, ties by index (a strictly monotone exp keeps the order of p) */
        g_sort_keys = zz;
        qsort(ids, (size_t)V, sizeof(int), cmp_desc);
        if (top_k > 0 && top_k < V) n = top_k;
    }
    acc_t m = -INFINITY;
    for (int i = 0; i < n; ++i)
        if (zz[ids[i]] > m) m = zz[ids[i]];
    acc_t zsum = 0;
    for (int i = 0; i < n; ++i) {
        pr[i] = ACC_EXP(zz[ids[i]] - m);
        zsum += pr[i];
    }
    for (int i = 0; i < n; ++i) pr[i] /= zsum;
    double mg = INFINITY;
    int cut = n;
    acc_t r = (acc_t)u;
    if (top_p < 1.0f) {
        acc_t cum = 0, prev = 0;
        for (int i = 0; i < n; ++i) {
            prev = cum;
            cum += pr[i];
            if (cum > (acc_t)top_p) {
                cut = i + 1;
                break;
            }
        }
        if (cut < n || cum > (acc_t)top_p) {
            const double a = (double)cum - (double)top_p, b = (double)top_p - (double)prev;
            mg = a < b ? a : b;
        }
        acc_t kept = 0;
        for (int i = 0; i < cut; ++i) kept += pr[i];
        r = (acc_t)u * kept;
    }
    int result = -1;
    acc_t cum = 0;
    for (int i = 0; i < cut; ++i) {
        const acc_t before = cum;
        cum += pr[i];
        if (r - cum <= 0) {
            result = ids[i];
            const double a = (double)cum - (double)r, b = (double)r - (double)before;
            const double d = a < b ? a : b;
            if (d < mg) mg = d;
            break;
        }
    }
    if (result < 0) {
        result = top_p < 1.0f ? ids[0] : ids[cut - 1];
        const double d = (double)r - (double)cum;
        if (d < mg) mg = d;
    }
    if (margin) *margin = mg;
    free(zz);
    free(ids);
    free(pr);
    return result;
}

/* candle's `logits / T` on f32 data: x * (float)(1 / T) + 0 (worker.rs:298). */
static void scale_row(const float* x, int32_t V, float temperature, float* z) {
    const float s = (float)(1.0 / (double)temperature);
    for (int v = 0; v < V; ++v) z[v] = x[v] * s + 0.0f;
}

int oracle_sample_token(const float* logits, int32_t V, float temperature, float top_p, int32_t top_k,
                        double u) {
    if (V <= 0) return -1;
    if (temperature <= 0) return argmax_f32(logits, V);
    float* z = (float*)malloc(sizeof(float) * (size_t)V);
    scale_row(logits, V, temperature, z);
    const int t = sample_core(z, V, top_p, top_k, u, NULL);
    free(z);
    return t;
}

/*
 * The worker's decode step for a batch of rows (src/worker.rs:141-197 then sample_token):
 * y = ((logits + bias) + penalty) + mask in f32, the bias and penalty entries given per row as
 * sparse lists (CSR offsets, tokens, values; NULL offsets: none) and the mask as bit rows
 * (-inf where bit v of masks[mask_row[b]] is clear; mask_row NULL or -1: none). A row whose
 * tokens are all masked gets V - 1. margins (optional) as for sample_core; +inf for argmax rows.
 */
int oracle_sample_decode(int32_t B, int32_t V, const float* logits, const float* temperature,
                         const float* top_p, const int32_t* top_k, const float* u,
                         const int32_t* bias_off, const uint32_t* bias_tok, const float* bias_val,
                         const int32_t* pen_off, const uint32_t* pen_tok, const float* pen_val,
                         const uint32_t* masks, const int32_t* mask_row, uint32_t* out,
                         double* margins) {
    float* y = (float*)malloc(sizeof(float) * (size_t)V);
    float* z = (float*)malloc(sizeof(float) * (size_t)V);
    const int words = (V + 31) / 32;
    int rc = ORACLE_OK;
    for (int b = 0; b < B; ++b) {
        memcpy(y, logits + (size_t)b * V, sizeof(float) * (size_t)V);
        if (bias_off)
            for (int i = bias_off[b]; i < bias_off[b + 1]; ++i) {
                if (bias_tok[i] < (uint32_t)V) y[bias_tok[i]] = y[bias_tok[i]] + bias_val[i];
                else rc = ORACLE_EINVAL;
            }
        if (pen_off)
            for (int i = pen_off[b]; i < pen_off[b + 1]; ++i) {
                if (pen_tok[i] < (uint32_t)V) y[pen_tok[i]] = y[pen_tok[i]] + pen_val[i];
                else rc = ORACLE_EINVAL;
            }
        if (mask_row && mask_row[b] >= 0) {
            const uint32_t* mk = masks + (size_t)mask_row[b] * words;
            for (int v = 0; v < V; ++v) y[v] = y[v] + (((mk[v >> 5] >> (v & 31)) & 1u) ? 0.0f : -INFINITY);
        }
        double mg = INFINITY;
        const float T = temperature[b];
        int tok;
        if (!(T > 0)) {
            tok = argmax_f32(y, V);
        } else {
            int any = 0;
            for (int v = 0; v < V && !any; ++v) any = y[v] != -INFINITY;
            if (!any) {
                tok = V - 1;
            } else {
                scale_row(y, V, T, z);
                tok = sample_core(z, V, top_p ? top_p[b] : 1.0f, top_k ? top_k[b] : 0, (double)u[b], &mg);
            }
        }
        out[b] = (uint32_t)tok;
        if (margins) margins[b] = mg;
    }
    free(y);
    free(z);
    return rc;
}

/* ------------------------------------------------------------------------- paged KV append */

static uint16_t f32_to_bf16_rne(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

/* Returns ORACLE_EINVAL (and writes nothing for that sequence) for a bad q_start_loc, context
 * length or block id, like the device's latched errors. Other sequences are still written. */
int oracle_kv_append(int32_t B, int32_t Hkv, int32_t D, int32_t bs, int32_t max_blocks,
                     int32_t num_blocks, int32_t total_q, int32_t src_bf16, int32_t cache_bf16,
                     const void* key, const void* value, const int32_t* q_start,
                     const int64_t* table, const int64_t* ctx_lens, void* kc, void* vc) {
    int rc = ORACLE_OK;
    for (int b = 0; b < B; ++b) {
        const int r0 = q_start ? q_start[b] : b, r1 = q_start ? q_start[b + 1] : b + 1;
        const int64_t ctx = ctx_lens[b];
        const int q_len = r1 - r0;
        if (r0 < 0 || r1 < r0 || r1 > total_q || ctx < q_len || ctx > (int64_t)max_blocks * bs) {
            rc = ORACLE_EINVAL;
            continue;
        }
        for (int j = 0; j < q_len; ++j) {
            const int64_t pos = ctx - q_len + j;
            const int64_t blk = table[(size_t)b * max_blocks + (size_t)(pos / bs)];
            if (blk < 0 || blk >= num_blocks) {
                rc = ORACLE_EINVAL;
                continue;
            }
            const int slot = (int)(pos % bs);
            for (int h = 0; h < Hkv; ++h) {
                const size_t src = ((size_t)(r0 + j) * Hkv + h) * D;
                const size_t dst = (((size_t)blk * Hkv + h) * bs + slot) * D;
                for (int d = 0; d < D; ++d) {
                    for (int which = 0; which < 2; ++which) {
                        const void* in = which ? value : key;
                        void* out = which ? vc : kc;
                        if (src_bf16 && cache_bf16) {
                            ((uint16_t*)out)[dst + d] = ((const uint16_t*)in)[src + d];
                        } else {
                            const float x = src_bf16 ? bf16_to_f32(((const uint16_t*)in)[src + d])
                                                     : ((const float*)in)[src + d];
                            if (cache_bf16) ((uint16_t*)out)[dst + d] = f32_to_bf16_rne(x);
                            else ((float*)out)[dst + d] = x;
                        }
                    }
                }
            }
        }
    }
    return rc;
}
