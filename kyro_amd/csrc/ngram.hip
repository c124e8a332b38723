// N-gram drafting on the device: one lane per sequence walks up to kmax lookups in the uploaded
// open-addressing table (linear probing, exact keys), as generate_drafts' Ngram arm
// (src/speculative.rs:239-256) does per request.
#include "common.hpp"
#include "kernels.hpp"

namespace kyro {
namespace {

constexpr int kMaxOrder = 16;  // order - 1 <= 15 key tokens held in registers

__global__ __launch_bounds__(256) void ngram_draft_kernel(NgramArgs a) {
    const int b = blockIdx.x * 256 + threadIdx.x;
    if (b >= a.B) return;
    const int n = a.order - 1;
    uint32_t win[kMaxOrder];  // the last n tokens of context + drafts
    const int64_t len = a.ctx_len[b];
    for (int i = 0; i < n; ++i) win[i] = a.ctx_tail[(size_t)b * n + i];
    uint32_t* out = a.draft + (size_t)b * a.kmax;
    int k = 0;
    for (; k < a.kmax; ++k) {
        if (len + k < a.order) break;  // speculative.rs:245: ctx.len() < order stops drafting
        uint64_t slot = ngram_hash(win, n) & a.mask;
        uint32_t next = 0;
        bool hit = false;
        for (uint64_t probe = 0; probe <= a.mask; ++probe) {  // the table is never full
            if (!a.used[slot]) break;
            const uint32_t* e = a.slots + slot * (uint64_t)a.order;
            bool eq = true;
            for (int i = 0; i < n; ++i) eq = eq && e[i] == win[i];
            if (eq) {
                next = e[n];
                hit = true;
                break;
            }
            slot = (slot + 1) & a.mask;
        }
        if (!hit) break;
        out[k] = next;
        for (int i = 0; i + 1 < n; ++i) win[i] = win[i + 1];
        if (n > 0) win[n - 1] = next;
    }
    a.num_draft[b] = k;
    for (int i = k; i < a.kmax; ++i) out[i] = 0xFFFFFFFFu;
}

}  // namespace

hipError_t launch_ngram_draft(const NgramArgs& a, hipStream_t stream) {
    if (a.B == 0) return hipSuccess;
    ngram_draft_kernel<<<dim3((unsigned)((a.B + 255) / 256)), 256, 0, stream>>>(a);
    return hipGetLastError();
}

}  // namespace kyro
