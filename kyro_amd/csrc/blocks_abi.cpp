// C ABI of the block manager, the prefix cache, the device block-table writer and block copies
// (include/kyro_blocks.h). Host logic lives in block_manager.cpp; this file validates arguments,
// converts statuses and queues the device work on the context's stream.
#include <algorithm>
#include <vector>

#include "block_manager.hpp"
#include "context.hpp"
#include "kernels.hpp"
#include "kyro_blocks.h"

using namespace kyro::rt;

struct kyro_bm_s {
    kyro::bm::BlockManager m;
    // Per block: (call number << 32) | (1 + the request that listed it last), for telling
    // kyro_bm_write_tables' callers whether two requests share a block.
    std::vector<uint64_t> seen;
    uint32_t calls = 0;
    kyro_bm_s(int bs, int64_t gpu, int64_t cpu) : m(bs, gpu, cpu), seen((size_t)gpu, 0) {}
};

struct kyro_radix_s {
    kyro::bm::RadixCache c;
    kyro_radix_s(int bs, int64_t cap) : c(bs, cap) {}
};

namespace {

int bm_status(int s, const char* what, uint64_t rid) {
    if (s == kyro::bm::OK) return KYRO_OK;
    if (s == kyro::bm::ENOSPACE)
        return fail(KYRO_ENOSPACE, "%s: not enough free KV blocks for request %llu", what, (unsigned long long)rid);
    return fail(KYRO_EINVAL, "%s: bad request %llu or size (unknown id, id in use, or out of range)", what,
                (unsigned long long)rid);
}

int copy_match(const std::pair<std::vector<int64_t>, int64_t>& m, int64_t* out, int64_t cap,
               int64_t* out_n, int64_t* out_matched) {
    const int64_t nb = (int64_t)m.first.size();
    if (out_n) *out_n = nb;
    if (out_matched) *out_matched = m.second;
    if (out) std::copy(m.first.begin(), m.first.begin() + std::min(nb, std::max<int64_t>(cap, 0)), out);
    return KYRO_OK;
}

}  // namespace

extern "C" {

// ------------------------------------------------------------------------- prefix cache

int kyro_radix_create(int32_t block_size, int64_t max_capacity, kyro_radix* out) {
    return guarded([&]() -> int {
        if (!out) return fail(KYRO_EINVAL, "radix_create: out is null");
        *out = nullptr;
        if (block_size <= 0 || max_capacity < 0)
            return fail(KYRO_EINVAL, "radix_create: block_size must be > 0 and max_capacity >= 0");
        *out = new kyro_radix_s(block_size, max_capacity);
        return KYRO_OK;
    });
}

int kyro_radix_destroy(kyro_radix r) {
    return guarded([&]() -> int {
        delete r;
        return KYRO_OK;
    });
}

int kyro_radix_match_prefix(kyro_radix r, const uint32_t* tokens, int64_t n, int64_t* out_blocks,
                            int64_t cap, int64_t* out_num_blocks, int64_t* out_matched) {
    return guarded([&]() -> int {
        if (!r || n < 0 || (n > 0 && !tokens)) return fail(KYRO_EINVAL, "radix_match_prefix: bad arguments");
        return copy_match(r->c.match_prefix(tokens, n), out_blocks, cap, out_num_blocks, out_matched);
    });
}

int kyro_radix_insert(kyro_radix r, const uint32_t* tokens, int64_t n, const int64_t* blocks,
                      uint8_t* out_taken) {
    return guarded([&]() -> int {
        if (!r || n < 0 || (n > 0 && (!tokens || !blocks))) return fail(KYRO_EINVAL, "radix_insert: bad arguments");
        const std::vector<bool> taken = r->c.insert(tokens, n, blocks, nullptr);
        if (out_taken)
            for (size_t i = 0; i < taken.size(); ++i) out_taken[i] = taken[i] ? 1 : 0;
        return KYRO_OK;
    });
}

int kyro_radix_evict_lru(kyro_radix r, int64_t* out, int64_t cap, int64_t* out_n) {
    return guarded([&]() -> int {
        if (!r) return fail(KYRO_EINVAL, "radix_evict_lru: null handle");
        const std::vector<int64_t> ev = r->c.evict_lru();
        if (out_n) *out_n = (int64_t)ev.size();
        if (out) std::copy(ev.begin(), ev.begin() + std::min<int64_t>((int64_t)ev.size(), std::max<int64_t>(cap, 0)), out);
        return KYRO_OK;
    });
}

int64_t kyro_radix_num_cached_blocks(kyro_radix r) { return r ? r->c.num_cached_blocks() : -1; }

// ------------------------------------------------------------------------ block manager

int kyro_bm_create(int32_t block_size, int64_t num_gpu_blocks, int64_t num_cpu_blocks, kyro_bm* out) {
    return guarded([&]() -> int {
        if (!out) return fail(KYRO_EINVAL, "bm_create: out is null");
        *out = nullptr;
        if (block_size <= 0 || num_gpu_blocks < 0 || num_cpu_blocks < 0)
            return fail(KYRO_EINVAL, "bm_create: block_size must be > 0 and block counts >= 0");
        *out = new kyro_bm_s(block_size, num_gpu_blocks, num_cpu_blocks);
        return KYRO_OK;
    });
}

int kyro_bm_destroy(kyro_bm bm) {
    return guarded([&]() -> int {
        delete bm;
        return KYRO_OK;
    });
}

int kyro_bm_allocate_with_prefix(kyro_bm bm, uint64_t request_id, const uint32_t* tokens, int64_t n,
                                 int64_t* out_cached_tokens) {
    return guarded([&]() -> int {
        if (!bm || n < 0 || (n > 0 && !tokens) || !out_cached_tokens)
            return fail(KYRO_EINVAL, "bm_allocate_with_prefix: bad arguments");
        return bm_status(bm->m.allocate_with_prefix(request_id, tokens, n, out_cached_tokens),
                         "bm_allocate_with_prefix", request_id);
    });
}

int kyro_bm_allocate(kyro_bm bm, uint64_t request_id, int64_t num_tokens) {
    return guarded([&]() -> int {
        if (!bm) return fail(KYRO_EINVAL, "bm_allocate: null handle");
        return bm_status(bm->m.allocate(request_id, num_tokens), "bm_allocate", request_id);
    });
}

int kyro_bm_append_slots(kyro_bm bm, uint64_t request_id, int64_t n) {
    return guarded([&]() -> int {
        if (!bm) return fail(KYRO_EINVAL, "bm_append_slots: null handle");
        return bm_status(bm->m.append_slots(request_id, n), "bm_append_slots", request_id);
    });
}

int kyro_bm_truncate(kyro_bm bm, uint64_t request_id, int64_t num_tokens) {
    return guarded([&]() -> int {
        if (!bm) return fail(KYRO_EINVAL, "bm_truncate: null handle");
        return bm_status(bm->m.truncate(request_id, num_tokens), "bm_truncate", request_id);
    });
}

int kyro_bm_free(kyro_bm bm, uint64_t request_id, int32_t cache_prompt) {
    return guarded([&]() -> int {
        if (!bm) return fail(KYRO_EINVAL, "bm_free: null handle");
        return bm_status(bm->m.free(request_id, cache_prompt != 0), "bm_free", request_id);
    });
}

int kyro_bm_request_blocks(kyro_bm bm, uint64_t request_id, int64_t* out, int64_t cap, int64_t* out_n,
                           int64_t* out_num_tokens) {
    return guarded([&]() -> int {
        if (!bm) return fail(KYRO_EINVAL, "bm_request_blocks: null handle");
        const kyro::bm::Request* r = bm->m.find(request_id);
        if (!r) return fail(KYRO_EINVAL, "bm_request_blocks: unknown request %llu", (unsigned long long)request_id);
        const int64_t nb = (int64_t)r->blocks.size();
        if (out_n) *out_n = nb;
        if (out_num_tokens) *out_num_tokens = r->num_tokens;
        if (out) std::copy(r->blocks.begin(), r->blocks.begin() + std::min(nb, std::max<int64_t>(cap, 0)), out);
        return KYRO_OK;
    });
}

int kyro_bm_take_copies(kyro_bm bm, int64_t* src, int64_t* dst, int64_t cap, int64_t* out_n) {
    return guarded([&]() -> int {
        if (!bm || !out_n) return fail(KYRO_EINVAL, "bm_take_copies: bad arguments");
        // Peek first: nothing is taken unless it all fits.
        std::vector<std::pair<int64_t, int64_t>> c = bm->m.take_copies_peek();
        *out_n = (int64_t)c.size();
        if ((int64_t)c.size() > cap || (!c.empty() && (!src || !dst))) return KYRO_OK;
        c = bm->m.take_copies();
        for (size_t i = 0; i < c.size(); ++i) {
            src[i] = c[i].first;
            dst[i] = c[i].second;
        }
        return KYRO_OK;
    });
}

int64_t kyro_bm_num_free_blocks(kyro_bm bm) { return bm ? bm->m.num_free_blocks() : -1; }

int kyro_bm_check(kyro_bm bm) {
    return guarded([&]() -> int {
        if (!bm) return fail(KYRO_EINVAL, "bm_check: null handle");
        const std::string e = bm->m.check();
        if (!e.empty()) return fail(KYRO_EINVAL, "bm_check: %s", e.c_str());
        return KYRO_OK;
    });
}

int64_t kyro_bm_num_cached_blocks(kyro_bm bm) { return bm ? bm->m.cache().num_cached_blocks() : -1; }

int kyro_bm_match_prefix(kyro_bm bm, const uint32_t* tokens, int64_t n, int64_t* out_blocks, int64_t cap,
                         int64_t* out_num_blocks, int64_t* out_matched) {
    return guarded([&]() -> int {
        if (!bm || n < 0 || (n > 0 && !tokens)) return fail(KYRO_EINVAL, "bm_match_prefix: bad arguments");
        return copy_match(bm->m.cache().match_prefix(tokens, n), out_blocks, cap, out_num_blocks, out_matched);
    });
}

int kyro_bm_write_tables(kyro_bm bm, kyro_ctx ctx, const uint64_t* request_ids, int32_t B, int32_t max_blocks,
                         int64_t* block_table, int64_t* context_lens, int32_t* out_shared) {
    return guarded([&]() -> int {
        if (int rc = check_ctx(ctx)) return rc;
        if (!bm || B < 0 || max_blocks <= 0 || (B > 0 && (!request_ids || !block_table)))
            return fail(KYRO_EINVAL, "bm_write_tables: bad arguments");
        if (out_shared) *out_shared = 0;
        if (B == 0) return KYRO_OK;
        if (++bm->calls == 0) {  // the call counter wrapped: forget every older mark
            std::fill(bm->seen.begin(), bm->seen.end(), 0);
            bm->calls = 1;
        }
        const uint64_t call = (uint64_t)bm->calls << 32;
        int32_t shared = 0;
        std::vector<int64_t> table((size_t)B * max_blocks, 0), lens((size_t)B, 0);
        for (int32_t b = 0; b < B; ++b) {
            const kyro::bm::Request* r = bm->m.find(request_ids[b]);
            if (!r)
                return fail(KYRO_EINVAL, "bm_write_tables: unknown request %llu", (unsigned long long)request_ids[b]);
            if ((int64_t)r->blocks.size() > max_blocks)
                return fail(KYRO_EINVAL, "bm_write_tables: request %llu holds %zu blocks > max_blocks %d",
                            (unsigned long long)request_ids[b], r->blocks.size(), max_blocks);
            std::copy(r->blocks.begin(), r->blocks.end(), table.begin() + (size_t)b * max_blocks);
            lens[(size_t)b] = r->num_tokens;
            for (const int64_t blk : r->blocks) {
                if (blk < 0 || (size_t)blk >= bm->seen.size()) continue;
                uint64_t& s = bm->seen[(size_t)blk];
                const uint64_t mine = call | (uint64_t)(b + 1);
                if ((s & ~0xffffffffull) == call && s != mine) shared = 1;
                s = mine;
            }
        }
        if (out_shared) *out_shared = shared;
        DeviceGuard dg(ctx->device);
        KYRO_HIP(dg.status);
        Upload ups[2] = {{block_table, table.data(), table.size() * sizeof(int64_t)},
                         {context_lens, lens.data(), context_lens ? lens.size() * sizeof(int64_t) : 0}};
        return stage_uploads(ctx, ups, context_lens ? 2 : 1);
    });
}

// ------------------------------------------------------------------------------- copies

int kyro_copy_blocks(kyro_ctx ctx, const kyro_copy_blocks_params* p, void* key_cache, void* value_cache,
                     const int64_t* src, const int64_t* dst, int64_t n) {
    return guarded([&]() -> int {
        if (int rc = check_ctx(ctx)) return rc;
        if (!p || n < 0) return fail(KYRO_EINVAL, "copy_blocks: bad arguments");
        if (n == 0) return KYRO_OK;
        if (!src || !dst || !key_cache || !value_cache) return fail(KYRO_EINVAL, "copy_blocks: null pointer");
        if (p->block_size <= 0 || p->num_kv_heads <= 0 || p->head_dim <= 0 || p->num_blocks <= 0 ||
            (p->dtype != KYRO_F32 && p->dtype != KYRO_BF16))
            return fail(KYRO_EINVAL, "copy_blocks: bad params");
        const size_t elem = p->dtype == KYRO_F32 ? 4 : 2;
        const size_t slab = (size_t)p->num_kv_heads * p->block_size * p->head_dim * elem;
        if (slab % 16 != 0) return fail(KYRO_EUNSUPPORTED, "copy_blocks: a block is not a multiple of 16 bytes");
        if ((reinterpret_cast<uintptr_t>(key_cache) | reinterpret_cast<uintptr_t>(value_cache)) % 16 != 0)
            return fail(KYRO_EINVAL, "copy_blocks: caches must be 16-byte aligned");
        std::vector<int64_t> pairs((size_t)(2 * n));
        std::vector<char> is_src((size_t)p->num_blocks, 0);
        for (int64_t i = 0; i < n; ++i) {
            if (src[i] < 0 || src[i] >= p->num_blocks || dst[i] < 0 || dst[i] >= p->num_blocks)
                return fail(KYRO_EINVAL, "copy_blocks: block id outside [0, %d)", p->num_blocks);
            pairs[(size_t)i] = src[i];
            pairs[(size_t)(n + i)] = dst[i];
            is_src[(size_t)src[i]] = 1;
        }
        for (int64_t i = 0; i < n; ++i)
            if (is_src[(size_t)dst[i]]) return fail(KYRO_EINVAL, "copy_blocks: block %lld is both a source and a destination",
                                                    (long long)dst[i]);
        DeviceGuard dg(ctx->device);
        KYRO_HIP(dg.status);
        kyro::CopyBlocksArgs a{};
        if (n <= kyro::kCopyInline) {  // the pairs travel in the kernel arguments: no upload
            a.pairs = nullptr;
            for (int64_t i = 0; i < n; ++i) {
                a.inl[0][i] = (int32_t)src[i];
                a.inl[1][i] = (int32_t)dst[i];
            }
        } else {
            const size_t pair_bytes = pairs.size() * sizeof(int64_t);
            if (int rc = ensure_arena(ctx, pair_bytes)) return rc;
            Upload up = {ctx->arena, pairs.data(), pair_bytes};
            if (int rc = stage_uploads(ctx, &up, 1)) return rc;
            a.pairs = static_cast<const int64_t*>(ctx->arena);
        }
        a.n = n;
        a.slab_vecs = (int64_t)(slab / 16);
        a.kc = static_cast<uint4*>(key_cache);
        a.vc = static_cast<uint4*>(value_cache);
        KYRO_HIP(kyro::launch_copy_blocks(a, ctx->stream));
        return KYRO_OK;
    });
}

}  // extern "C"
