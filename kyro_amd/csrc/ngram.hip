// N-gram drafting on the device: one wave per sequence walks up to kmax lookups in the uploaded
// open-addressing table (linear probing, exact keys), as generate_drafts' Ngram arm
// (src/speculative.rs:239-256) does per request. Each lookup is one round of loads: lane l reads
// the used flag, key tokens and next token of slot h + l (64 consecutive slots of the probe
// sequence at once), and a ballot finds the first slot that either holds the key or is unused
// (the end of the probe sequence). A lookup is then one memory round trip however many slots
// collide, instead of two per probed slot.
#include "common.hpp"
#include "kernels.hpp"

namespace kyro {
namespace {

constexpr int kMaxOrder = 16;  // order - 1 <= 15 key tokens held in registers

__global__ __launch_bounds__(256) void ngram_draft_kernel(NgramArgs a) {
    const int b = blockIdx.x * 4 + (int)(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (b >= a.B) return;  // uniform per wave
    const int n = a.order - 1;
    uint32_t win[kMaxOrder];  // the last n tokens of context + drafts (the same in every lane)
    const int64_t len = a.ctx_len[b];
    for (int i = 0; i < n; ++i) win[i] = a.ctx_tail[(size_t)b * n + i];
    uint32_t* out = a.draft + (size_t)b * a.kmax;
    int k = 0;
    for (; k < a.kmax; ++k) {
        if (len + k < a.order) break;  // speculative.rs:245: ctx.len() < order stops drafting
        const uint64_t h = ngram_hash(win, n) & a.mask;
        uint32_t next = 0;
        bool hit = false;
        // The table is never full, so an unused slot ends every probe sequence.
        for (uint64_t base = 0; base <= a.mask; base += 64) {
            const uint64_t slot = (h + base + (uint64_t)lane) & a.mask;
            const bool used = a.used[slot] != 0;
            const uint32_t* e = a.slots + slot * (uint64_t)a.order;
            bool eq = used;
            for (int i = 0; i < n; ++i) eq = eq && e[i] == win[i];
            const uint32_t nx = e[n];
            const unsigned long long found = __ballot(eq || !used);
            if (found) {
                const int first = __ffsll((long long)found) - 1;
                hit = __builtin_amdgcn_readlane((int)eq, first) != 0;
                next = (uint32_t)__builtin_amdgcn_readlane((int)nx, first);
                break;
            }
        }
        if (!hit) break;
        if (lane == 0) out[k] = next;
        for (int i = 0; i + 1 < n; ++i) win[i] = win[i + 1];
        if (n > 0) win[n - 1] = next;
    }
    if (lane == 0) a.num_draft[b] = k;
    for (int i = k + lane; i < a.kmax; i += 64) out[i] = 0xFFFFFFFFu;
}

}  // namespace

hipError_t launch_ngram_draft(const NgramArgs& a, hipStream_t stream) {
    if (a.B == 0) return hipSuccess;
    ngram_draft_kernel<<<dim3((unsigned)((a.B + 3) / 4)), 256, 0, stream>>>(a);
    return hipGetLastError();
}

}  // namespace kyro
