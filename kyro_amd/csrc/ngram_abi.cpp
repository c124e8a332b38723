// C ABI of n-gram drafting (include/kyro_draft.h): the table is built on the host with the
// reference's semantics, laid out for open addressing, and copied to each device that drafts.
#include <map>
#include <unordered_map>
#include <vector>

#include "context.hpp"
#include "kernels.hpp"
#include "kyro_draft.h"

using namespace kyro::rt;

struct kyro_ngram_s {
    int order = 0;
    std::vector<uint32_t> slots;  // [capacity, order]: key tokens, then the next token
    std::vector<uint8_t> used;
    uint64_t mask = 0;
    int64_t size = 0;
    std::map<int, std::pair<void*, void*>> dev;  // device -> (slots, used)
};

namespace {

constexpr int kMaxOrder = 16;

struct KeyHash {
    size_t operator()(const std::vector<uint32_t>& k) const {
        return (size_t)kyro::ngram_hash(k.data(), (int)k.size());
    }
};

// Slot of `key` (n tokens) in the table: the matching slot, or the first free one on its probe path.
uint64_t find_slot(const kyro_ngram_s* t, const uint32_t* key, int n) {
    uint64_t s = kyro::ngram_hash(key, n) & t->mask;
    while (t->used[s]) {
        const uint32_t* e = &t->slots[s * (uint64_t)t->order];
        bool eq = true;
        for (int i = 0; i < n && eq; ++i) eq = e[i] == key[i];
        if (eq) break;
        s = (s + 1) & t->mask;
    }
    return s;
}

}  // namespace

extern "C" {

// speculative.rs:196-208: windows of `order` tokens, the first order-1 mapping to the last; a
// later window replaces an earlier one with the same prefix.
int kyro_ngram_build(const uint32_t* tokens, const int64_t* offsets, int64_t num_seqs, int32_t order, kyro_ngram* out) {
    return guarded([&]() -> int {
        if (!out) return fail(KYRO_EINVAL, "ngram_build: out is null");
        *out = nullptr;
        if (order < 2 || order > kMaxOrder)
            return fail(KYRO_EUNSUPPORTED, "ngram_build: order must be in [2, %d]", kMaxOrder);
        if (num_seqs < 0 || (num_seqs > 0 && !offsets)) return fail(KYRO_EINVAL, "ngram_build: bad corpus");
        const int n = order - 1;
        std::unordered_map<std::vector<uint32_t>, uint32_t, KeyHash> table;
        for (int64_t s = 0; s < num_seqs; ++s) {
            const int64_t a = offsets[s], b = offsets[s + 1];
            if (b < a || a < 0) return fail(KYRO_EINVAL, "ngram_build: offsets not monotone");
            if (b - a < order) continue;
            if (!tokens) return fail(KYRO_EINVAL, "ngram_build: tokens is null");
            for (int64_t i = a; i + order <= b; ++i)
                table[std::vector<uint32_t>(tokens + i, tokens + i + n)] = tokens[i + n];
        }
        auto* t = new kyro_ngram_s();
        t->order = order;
        t->size = (int64_t)table.size();
        uint64_t cap = 16;
        while (cap < 2 * (uint64_t)table.size()) cap <<= 1;
        t->mask = cap - 1;
        t->slots.assign(cap * (uint64_t)order, 0);
        t->used.assign(cap, 0);
        for (const auto& kv : table) {
            const uint64_t s = find_slot(t, kv.first.data(), n);
            std::copy(kv.first.begin(), kv.first.end(), t->slots.begin() + s * order);
            t->slots[s * order + n] = kv.second;
            t->used[s] = 1;
        }
        *out = t;
        return KYRO_OK;
    });
}

int kyro_ngram_destroy(kyro_ngram t) {
    return guarded([&]() -> int {
        if (!t) return KYRO_OK;
        for (auto& d : t->dev) {
            DeviceGuard dg(d.first);
            (void)hipFree(d.second.first);
            (void)hipFree(d.second.second);
        }
        delete t;
        return KYRO_OK;
    });
}

int kyro_ngram_lookup(kyro_ngram t, const uint32_t* prefix, uint32_t* next) {
    if (!t || !prefix) return 0;
    const uint64_t s = find_slot(t, prefix, t->order - 1);
    if (!t->used[s]) return 0;
    if (next) *next = t->slots[s * t->order + t->order - 1];
    return 1;
}

int64_t kyro_ngram_size(kyro_ngram t) { return t ? t->size : -1; }

int kyro_ngram_upload(kyro_ngram t, kyro_ctx ctx) {
    return guarded([&]() -> int {
        if (int rc = check_ctx(ctx)) return rc;
        if (!t) return fail(KYRO_EINVAL, "ngram_upload: null table");
        if (t->dev.count(ctx->device)) return KYRO_OK;
        DeviceGuard dg(ctx->device);
        KYRO_HIP(dg.status);
        void *s = nullptr, *u = nullptr;
        KYRO_HIP(hipMalloc(&s, t->slots.size() * sizeof(uint32_t)));
        hipError_t e = hipMalloc(&u, t->used.size());
        if (e == hipSuccess) e = hipMemcpy(s, t->slots.data(), t->slots.size() * sizeof(uint32_t), hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(u, t->used.data(), t->used.size(), hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            (void)hipFree(s);
            if (u) (void)hipFree(u);
            return fail(e == hipErrorOutOfMemory ? KYRO_EOOM : KYRO_EHIP, "ngram_upload: %s", hipGetErrorString(e));
        }
        t->dev[ctx->device] = {s, u};
        return KYRO_OK;
    });
}

int kyro_ngram_draft(kyro_ngram t, kyro_ctx ctx, int32_t batch_size, int32_t max_draft, const uint32_t* context_tail,
                     const int64_t* context_len, uint32_t* draft_tokens, int32_t* num_draft) {
    return guarded([&]() -> int {
        if (int rc = check_ctx(ctx)) return rc;
        if (!t) return fail(KYRO_EINVAL, "ngram_draft: null table");
        if (batch_size < 0 || max_draft < 0) return fail(KYRO_EINVAL, "ngram_draft: negative size");
        if (batch_size == 0) return KYRO_OK;
        if (!context_tail || !context_len || !num_draft || (max_draft > 0 && !draft_tokens))
            return fail(KYRO_EINVAL, "ngram_draft: null device pointer");
        auto it = t->dev.find(ctx->device);
        if (it == t->dev.end()) return fail(KYRO_EINVAL, "ngram_draft: table not uploaded to device %d", ctx->device);
        kyro::NgramArgs a{};
        a.slots = static_cast<const uint32_t*>(it->second.first);
        a.used = static_cast<const uint8_t*>(it->second.second);
        a.mask = t->mask;
        a.order = t->order;
        a.ctx_tail = context_tail;
        a.ctx_len = context_len;
        a.draft = draft_tokens;
        a.num_draft = num_draft;
        a.B = batch_size;
        a.kmax = max_draft;
        DeviceGuard dg(ctx->device);
        KYRO_HIP(dg.status);
        KYRO_HIP(kyro::launch_ngram_draft(a, ctx->stream));
        return KYRO_OK;
    });
}

}  // extern "C"
