/*
 * A C99 consumer of libkyro_verify.so, using only the C ABI (no HIP or torch headers): the calls
 * a Rust `extern "C"` shim would make for one verify step. Device memory comes from kyro_buf_*.
 *
 *   1. paged attention on the reference's all-ones case (attention_kernel.rs:198-227: every
 *      output is 1.0), with two query rows per sequence and an aliased block table;
 *   2. greedy verification with known answers (speculative.rs:315-323 plus the bonus token);
 *   3. n-gram drafts from a corpus fed straight into the verify call;
 *   4. the device-side error path: a bad block id is reported by kyro_sync, then the context
 *      works again.
 * Prints "ok" and exits 0 on success; prints the failing check and exits 1 otherwise.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "kyro_draft.h"
#include "kyro_verify.h"

#define CHECK(cond, ...)                             \
    do {                                             \
        if (!(cond)) {                               \
            fprintf(stderr, "check failed: " __VA_ARGS__); \
            fprintf(stderr, " (%s)\n", kyro_last_error()); \
            exit(1);                                 \
        }                                            \
    } while (0)

/* A device buffer of `bytes`, filled from src (NULL: left as allocated, for outputs). */
static kyro_buf upload(kyro_ctx ctx, const void* src, size_t bytes) {
    kyro_buf b = NULL;
    CHECK(kyro_buf_alloc(ctx, bytes ? bytes : 4, &b) == KYRO_OK, "alloc %zu", bytes);
    if (src && bytes) CHECK(kyro_buf_upload(ctx, b, 0, src, bytes) == KYRO_OK, "upload");
    return b;
}

int main(void) {
    CHECK(kyro_abi_version() == KYRO_ABI_VERSION, "abi version %d", kyro_abi_version());
    kyro_ctx ctx = NULL;
    CHECK(kyro_ctx_create(0, &ctx) == KYRO_OK, "ctx_create");

    /* 1. attention: B 2, H 8, Hkv 2, D 64, block 16, ctx {24, 9}, 2 query rows each */
    enum { B = 2, H = 8, HKV = 2, D = 64, BS = 16, NB = 4, MB = 2, TQ = 4 };
    static float q[TQ * H * D], kc[NB * HKV * BS * D], vc[NB * HKV * BS * D], out[TQ * H * D];
    for (size_t i = 0; i < sizeof(q) / 4; ++i) q[i] = 1.0f;
    for (size_t i = 0; i < sizeof(kc) / 4; ++i) kc[i] = vc[i] = 1.0f;
    const int64_t table[B * MB] = {0, 1, 0, 0}; /* sequence 1 aliases block 0 */
    const int64_t lens[B] = {24, 9};
    const int32_t qs[B + 1] = {0, 2, 4};
    kyro_buf bq = upload(ctx, q, sizeof(q)), bk = upload(ctx, kc, sizeof(kc)), bv = upload(ctx, vc, sizeof(vc));
    kyro_buf bt = upload(ctx, table, sizeof(table)), bl = upload(ctx, lens, sizeof(lens)), bqs = upload(ctx, qs, sizeof(qs));
    kyro_buf bo = upload(ctx, NULL, sizeof(out));
    kyro_paged_attention_params ap = {BS, H, D, HKV, B, TQ, MB, NB, KYRO_F32, KYRO_F32, 1, 0.f, KYRO_ATTN_AUTO, 0, 2,
                                      KYRO_KV_REUSE_AUTO};
    CHECK(kyro_paged_attention_mq(ctx, &ap, kyro_buf_ptr(bq), kyro_buf_ptr(bqs), kyro_buf_ptr(bk), kyro_buf_ptr(bv),
                                  kyro_buf_ptr(bt), kyro_buf_ptr(bl), kyro_buf_ptr(bo)) == KYRO_OK, "attention");
    CHECK(kyro_buf_download(ctx, out, bo, 0, sizeof(out)) == KYRO_OK, "download");
    for (size_t i = 0; i < sizeof(out) / 4; ++i) CHECK(fabsf(out[i] - 1.0f) < 1e-5f, "attention out[%zu] = %g", i, out[i]);

    /* 2. greedy verify: V 10, k 4 */
    enum { VB = 3, K = 4, V = 10 };
    static float tl[VB * (K + 1) * V];
    const int top[VB][K + 1] = {{3, 1, 4, 1, 5}, {2, 7, 1, 8, 2}, {0, 0, 0, 0, 9}};
    for (int b = 0; b < VB; ++b)
        for (int i = 0; i <= K; ++i) tl[(b * (K + 1) + i) * V + top[b][i]] = 5.0f;
    const uint32_t dt[VB * K] = {3, 1, 4, 1, 2, 7, 3, 8, 0, 0, 9, 0};
    const int32_t nd[VB] = {4, 4, 4};
    const float temp[VB] = {0, 0, 0}, ua[VB * K] = {.5f, .5f, .5f, .5f, .5f, .5f, .5f, .5f, .5f, .5f, .5f, .5f},
                ur[VB] = {.5f, .5f, .5f};
    kyro_buf btl = upload(ctx, tl, sizeof(tl)), bdt = upload(ctx, dt, sizeof(dt)), bnd = upload(ctx, nd, sizeof(nd));
    kyro_buf btm = upload(ctx, temp, sizeof(temp)), bua = upload(ctx, ua, sizeof(ua)), bur = upload(ctx, ur, sizeof(ur));
    kyro_buf bacc = upload(ctx, NULL, VB * 4), btok = upload(ctx, NULL, VB * (K + 1) * 4);
    kyro_spec_verify_params vp = {VB, K, V, KYRO_F32, 0};
    CHECK(kyro_spec_verify(ctx, &vp, kyro_buf_ptr(btl), NULL, kyro_buf_ptr(bdt), kyro_buf_ptr(bnd), kyro_buf_ptr(btm),
                           kyro_buf_ptr(bua), kyro_buf_ptr(bur), kyro_buf_ptr(bacc), kyro_buf_ptr(btok), NULL, NULL) == KYRO_OK,
          "spec_verify");
    int32_t acc[VB];
    uint32_t tok[VB * (K + 1)];
    CHECK(kyro_buf_download(ctx, acc, bacc, 0, sizeof(acc)) == KYRO_OK, "download acc");
    CHECK(kyro_buf_download(ctx, tok, btok, 0, sizeof(tok)) == KYRO_OK, "download tokens");
    const int exp_acc[VB] = {4, 2, 2};
    const uint32_t exp_last[VB] = {5, 1, 0};
    for (int b = 0; b < VB; ++b) {
        CHECK(acc[b] == exp_acc[b], "accepted[%d] = %d", b, acc[b]);
        CHECK(tok[b * (K + 1) + acc[b]] == exp_last[b], "emitted[%d] = %u", b, tok[b * (K + 1) + acc[b]]);
    }

    /* 3. n-gram drafts (order 2) into the verify call */
    const uint32_t corpus[] = {3, 1, 4, 1, 5, 9, 2, 6};
    const int64_t offs[2] = {0, 8};
    kyro_ngram ng = NULL;
    CHECK(kyro_ngram_build(corpus, offs, 1, 2, &ng) == KYRO_OK, "ngram_build");
    CHECK(kyro_ngram_upload(ng, ctx) == KYRO_OK, "ngram_upload");
    const uint32_t tails[VB] = {3, 9, 7}; /* last token of each context */
    const int64_t clen[VB] = {5, 5, 5};
    kyro_buf btail = upload(ctx, tails, sizeof(tails)), bclen = upload(ctx, clen, sizeof(clen));
    CHECK(kyro_ngram_draft(ng, ctx, VB, K, kyro_buf_ptr(btail), kyro_buf_ptr(bclen), kyro_buf_ptr(bdt), kyro_buf_ptr(bnd)) == KYRO_OK,
          "ngram_draft");
    int32_t nd2[VB];
    uint32_t dt2[VB * K];
    CHECK(kyro_buf_download(ctx, nd2, bnd, 0, sizeof(nd2)) == KYRO_OK, "download num_draft");
    CHECK(kyro_buf_download(ctx, dt2, bdt, 0, sizeof(dt2)) == KYRO_OK, "download drafts");
    /* 3 -> 1 -> 5 (1 maps to its last successor, 5) -> 9 -> 2; 9 -> 2 -> 6 then a miss; 7: none */
    const uint32_t e0[4] = {1, 5, 9, 2}, e1[2] = {2, 6};
    CHECK(nd2[0] == 4 && nd2[1] == 2 && nd2[2] == 0, "num_draft %d %d %d", nd2[0], nd2[1], nd2[2]);
    for (int i = 0; i < 4; ++i) CHECK(dt2[i] == e0[i], "draft[0][%d] = %u", i, dt2[i]);
    for (int i = 0; i < 2; ++i) CHECK(dt2[K + i] == e1[i], "draft[1][%d] = %u", i, dt2[K + i]);
    CHECK(kyro_spec_verify(ctx, &vp, kyro_buf_ptr(btl), NULL, kyro_buf_ptr(bdt), kyro_buf_ptr(bnd), kyro_buf_ptr(btm),
                           kyro_buf_ptr(bua), kyro_buf_ptr(bur), kyro_buf_ptr(bacc), kyro_buf_ptr(btok), NULL, NULL) == KYRO_OK,
          "spec_verify on drafts");
    CHECK(kyro_sync(ctx) == KYRO_OK, "sync after drafts");
    CHECK(kyro_buf_download(ctx, acc, bacc, 0, sizeof(acc)) == KYRO_OK, "download acc 2");
    /* sequence 0 drafts 1 where row 0's argmax is 3; sequence 1 drafts 2 (= row 0's argmax) then
     * 6 where row 1's argmax is 7; sequence 2 has no drafts */
    CHECK(acc[0] == 0 && acc[1] == 1 && acc[2] == 0, "accepted %d %d %d", acc[0], acc[1], acc[2]);

    /* 4. a bad block id is reported by the next sync, and the context recovers */
    const int64_t bad[B * MB] = {0, 99, 0, 0};
    CHECK(kyro_buf_upload(ctx, bt, 0, bad, sizeof(bad)) == KYRO_OK, "upload bad table");
    CHECK(kyro_paged_attention_mq(ctx, &ap, kyro_buf_ptr(bq), kyro_buf_ptr(bqs), kyro_buf_ptr(bk), kyro_buf_ptr(bv),
                                  kyro_buf_ptr(bt), kyro_buf_ptr(bl), kyro_buf_ptr(bo)) == KYRO_OK, "attention (bad ids queued)");
    CHECK(kyro_sync(ctx) == KYRO_EINVAL, "bad block id not reported");
    CHECK(strstr(kyro_last_error(), "block_table") != NULL, "message");
    CHECK(kyro_buf_upload(ctx, bt, 0, table, sizeof(table)) == KYRO_OK, "restore table");
    CHECK(kyro_paged_attention_mq(ctx, &ap, kyro_buf_ptr(bq), kyro_buf_ptr(bqs), kyro_buf_ptr(bk), kyro_buf_ptr(bv),
                                  kyro_buf_ptr(bt), kyro_buf_ptr(bl), kyro_buf_ptr(bo)) == KYRO_OK, "attention again");
    CHECK(kyro_sync(ctx) == KYRO_OK, "sync after recovery");

    kyro_buf all[] = {bq, bk, bv, bt, bl, bqs, bo, btl, bdt, bnd, btm, bua, bur, bacc, btok, btail, bclen};
    for (size_t i = 0; i < sizeof(all) / sizeof(all[0]); ++i) kyro_buf_free(all[i]);
    kyro_ngram_destroy(ng);
    CHECK(kyro_ctx_destroy(ctx) == KYRO_OK, "ctx_destroy");
    printf("ok\n");
    return 0;
}
