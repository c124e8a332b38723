// C ABI of the plain-decode sampler (include/kyro_sample.h): argument checks, the workspace for
// processed rows, and the host-side penalty vector.
#include <algorithm>
#include <cmath>
#include <map>

#include "context.hpp"
#include "kernels.hpp"
#include "kyro_sample.h"

using namespace kyro::rt;

extern "C" {

int kyro_sample_tokens(kyro_ctx ctx, const kyro_sample_params* p, const float* logits, const float* temperature,
                       const float* top_p, const int32_t* top_k, const float* u, const int32_t* bias_offsets,
                       const uint32_t* bias_tokens, const float* bias_values, const int32_t* penalty_offsets,
                       const uint32_t* penalty_tokens, const float* penalty_values, const uint32_t* allowed_mask,
                       const int32_t* mask_row, uint32_t* out_tokens) {
    return guarded([&]() -> int {
        if (int rc = check_ctx(ctx)) return rc;
        if (!p) return fail(KYRO_EINVAL, "sample_tokens: params is null");
        if (p->batch_size < 0 || p->vocab_size <= 0 || p->num_masks < 0)
            return fail(KYRO_EINVAL, "sample_tokens: need batch_size >= 0, vocab_size > 0, num_masks >= 0");
        if (p->logits_dtype != KYRO_F32) return fail(KYRO_EUNSUPPORTED, "sample_tokens: logits_dtype must be KYRO_F32");
        if (p->batch_size == 0) return KYRO_OK;
        if (!logits || !temperature || !u || !out_tokens) return fail(KYRO_EINVAL, "sample_tokens: null device pointer");
        if (bias_offsets && (!bias_tokens || !bias_values))
            return fail(KYRO_EINVAL, "sample_tokens: bias_offsets without bias_tokens / bias_values");
        if (penalty_offsets && (!penalty_tokens || !penalty_values))
            return fail(KYRO_EINVAL, "sample_tokens: penalty_offsets without penalty_tokens / penalty_values");
        if (mask_row && (!allowed_mask || p->num_masks == 0))
            return fail(KYRO_EINVAL, "sample_tokens: mask_row without allowed_mask / num_masks");
        kyro::SampleArgs a{};
        a.logits = logits;
        a.temperature = temperature;
        a.top_p = top_p;
        a.top_k = top_k;
        a.u = u;
        a.bias_off = bias_offsets;
        a.bias_tok = bias_tokens;
        a.bias_val = bias_values;
        a.pen_off = penalty_offsets;
        a.pen_tok = penalty_tokens;
        a.pen_val = penalty_values;
        a.mask = allowed_mask;
        a.mask_row = mask_row;
        a.out = out_tokens;
        a.B = p->batch_size;
        a.V = p->vocab_size;
        a.num_masks = p->num_masks;
        a.mask_words = (p->vocab_size + 31) / 32;
        a.vec4 = (p->vocab_size % 4 == 0) && (reinterpret_cast<uintptr_t>(logits) % 16 == 0);
        a.C = (a.V + kyro::kSampleChunk - 1) / kyro::kSampleChunk;
        if (a.C > kyro::kSampleMaxChunks)
            return fail(KYRO_EUNSUPPORTED, "sample_tokens: vocab_size %d > %d", p->vocab_size,
                        kyro::kSampleMaxChunks * kyro::kSampleChunk);
        // Arena: processed rows (when a processor is given), chunk statistics, and for top-k /
        // top-p the chunks' thresholds, counts and candidate lists.
        const bool filtered = top_p || top_k;
        const bool processed = bias_offsets || penalty_offsets || mask_row;
        // Rows without processors, top-k or top-p take the one-launch pass: segments of
        // kSampleSeg entries, kSampleSegsPerWg per workgroup (one a wave) while the row allows,
        // at most kSampleRowWgsMax workgroups a row.
        const int nseg = (a.V + kyro::kSampleSeg - 1) / kyro::kSampleSeg;
        if (!filtered && !processed && a.vec4 && a.B <= kyro::kSampleRowCounters && nseg <= 1024)
            a.row_wgs = std::min(kyro::kSampleRowWgsMax,
                                 std::max(1, (nseg + kyro::kSampleSegsPerWg - 1) / kyro::kSampleSegsPerWg));
        const size_t seg_b = a.row_wgs ? align_up((size_t)a.B * nseg * sizeof(float2), 256) : 0;
        const size_t ws_b = processed ? align_up((size_t)a.B * a.V * sizeof(float), 256) : 0;
        const size_t cstat_b = align_up((size_t)a.B * a.C * sizeof(float2), 256);
        const size_t thr_b = filtered ? align_up((size_t)a.B * a.C * sizeof(float), 256) : 0;
        const size_t cnt_b = filtered ? align_up((size_t)a.B * a.C * sizeof(int), 256) : 0;
        const size_t cand_b = filtered ? align_up((size_t)a.B * kyro::kSampleCand * sizeof(unsigned long long), 256) : 0;
        a.ccap = std::min(kyro::kSampleChunkCand, kyro::kSampleCand / a.C);
        // The select pass copies a chunk's list with 1024 / C threads, at most 16 entries each
        // (true for every C up to kSampleMaxChunks).
        if ((a.ccap + 1024 / a.C - 1) / (1024 / a.C) > 16)
            return fail(KYRO_EUNSUPPORTED, "sample_tokens: %d chunks leave too few copy threads", a.C);
        DeviceGuard dg(ctx->device);
        KYRO_HIP(dg.status);
        if (int rc = ensure_arena(ctx, ws_b + cstat_b + thr_b + cnt_b + cand_b + seg_b)) return rc;
        char* base = static_cast<char*>(ctx->arena);
        a.ws = ws_b ? reinterpret_cast<float*>(base) : nullptr;
        base += ws_b;
        a.cstat = reinterpret_cast<float2*>(base);
        base += cstat_b;
        a.cthr = thr_b ? reinterpret_cast<float*>(base) : nullptr;
        base += thr_b;
        a.ccount = cnt_b ? reinterpret_cast<int*>(base) : nullptr;
        base += cnt_b;
        a.cand = cand_b ? reinterpret_cast<unsigned long long*>(base) : nullptr;
        base += cand_b;
        a.segs = seg_b ? reinterpret_cast<float2*>(base) : nullptr;
        a.row_cnt = ctx->row_cnt;
        a.err = ctx->err;
        KYRO_HIP(kyro::launch_sample(a, ctx->stream));
        return KYRO_OK;
    });
}

// worker.rs:154-181, per token: the first loop adds frequency_penalty once per occurrence, the
// second replaces the entry by min(entry, 0) + presence_penalty once per occurrence. Other
// tokens do not affect an entry, so each token's value follows from its count, in the same f32
// operations and order.
int kyro_penalty_adds(const uint32_t* generated, int64_t n, float frequency_penalty, float presence_penalty,
                      int32_t vocab_size, uint32_t* out_tokens, float* out_values, int64_t cap, int64_t* out_n) {
    return guarded([&]() -> int {
        if (n < 0 || (n > 0 && !generated) || !out_n || vocab_size <= 0)
            return fail(KYRO_EINVAL, "penalty_adds: bad arguments");
        *out_n = 0;
        if (frequency_penalty == 0.0f && presence_penalty == 0.0f) return KYRO_OK;
        std::map<uint32_t, int64_t> count;
        for (int64_t i = 0; i < n; ++i)
            if (generated[i] < (uint32_t)vocab_size) ++count[generated[i]];
        *out_n = (int64_t)count.size();
        int64_t i = 0;
        for (const auto& kv : count) {
            if (i >= cap) break;
            float m = 0.0f;
            for (int64_t c = 0; c < kv.second; ++c) m += frequency_penalty;
            for (int64_t c = 0; c < kv.second; ++c) m = std::fmin(m, 0.0f) + presence_penalty;  // f32::min
            if (out_tokens) out_tokens[i] = kv.first;
            if (out_values) out_values[i] = m;
            ++i;
        }
        return KYRO_OK;
    });
}

}  // extern "C"
