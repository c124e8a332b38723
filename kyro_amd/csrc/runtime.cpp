// Host runtime behind include/kyro_verify.h: contexts, device buffers, scratch arena, argument
// validation, kernel selection and error reporting. No C++ exception leaves this file: each
// entry point catches everything and returns a kyro_status (the Rust caller is built with
// panic = "abort", Cargo.toml:41, so an unwinding exception would take the process down).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "context.hpp"
#include "kernels.hpp"
#include "kyro_testing.h"
#include "kyro_verify.h"

namespace {
thread_local std::string g_last_error;
// Partial-state slots a balanced-schedule launch sizes at most (0: the bound); set only through
// kyro_testing_set_plan_slot_cap.
std::atomic<int64_t> g_test_plan_slot_cap{0};
}  // namespace

struct kyro_buf_s {
    int device = 0;
    void* ptr = nullptr;
    size_t bytes = 0;
};

namespace kyro {
namespace rt {

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int check_ctx(kyro_ctx ctx) {
    if (!ctx) return fail(KYRO_EINVAL, "null kyro_ctx");
    return KYRO_OK;
}

int ensure_arena(kyro_ctx ctx, size_t bytes) {
    if (bytes <= ctx->arena_bytes) return KYRO_OK;
    // Growing frees the arena that kernels already captured into a graph would address, and a
    // synchronisation inside a capture invalidates it: refuse, and name what to reserve.
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    KYRO_HIP(hipStreamIsCapturing(ctx->stream, &cap));
    if (cap != hipStreamCaptureStatusNone)
        return fail(KYRO_EINVAL, "the call needs %zu bytes of scratch arena and the context holds %zu; the stream "
                    "is capturing a graph, so the arena cannot grow now: call kyro_ctx_reserve(ctx, %zu) "
                    "(or the size queries kyro_paged_attention_workspace / kyro_spec_verify_workspace) "
                    "before capturing", bytes, ctx->arena_bytes, bytes);
    const size_t want = align_up(std::max(bytes, ctx->arena_bytes * 3 / 2), size_t(1) << 20);
    KYRO_HIP(hipStreamSynchronize(ctx->stream));
    if (ctx->arena) KYRO_HIP(hipFree(ctx->arena));
    ctx->arena = nullptr;
    ctx->arena_bytes = 0;
    KYRO_HIP(hipMalloc(&ctx->arena, want));
    ctx->arena_bytes = want;
    return KYRO_OK;
}

int stage_uploads(kyro_ctx ctx, const Upload* ups, int n) {
    size_t total = 0;
    for (int i = 0; i < n; ++i) total += align_up(ups[i].bytes, 256);
    if (total == 0) return KYRO_OK;
    if (total > ctx->pinned_slot_bytes) {  // grow: every slot's copies must have left staging
        for (int s = 0; s < kStageSlots; ++s)
            if (ctx->pinned_done[s]) KYRO_HIP(hipEventSynchronize(ctx->pinned_done[s]));
        const size_t want = align_up(std::max(total, ctx->pinned_slot_bytes * 3 / 2), size_t(1) << 16);
        if (ctx->pinned) KYRO_HIP(hipHostFree(ctx->pinned));
        ctx->pinned = nullptr;
        ctx->pinned_slot_bytes = 0;
        // Coherent and mapped: small uploads are read by a kernel straight from staging.
        KYRO_HIP(hipHostMalloc(&ctx->pinned, want * kStageSlots, hipHostMallocMapped | hipHostMallocCoherent));
        KYRO_HIP(hipHostGetDevicePointer(&ctx->pinned_dev, ctx->pinned, 0));
        ctx->pinned_slot_bytes = want;
    }
    const int slot = ctx->pinned_next;
    ctx->pinned_next = (slot + 1) % kStageSlots;
    if (!ctx->pinned_done[slot]) KYRO_HIP(hipEventCreateWithFlags(&ctx->pinned_done[slot], hipEventDisableTiming));
    else KYRO_HIP(hipEventSynchronize(ctx->pinned_done[slot]));  // the slot's last upload has left it
    char* p = static_cast<char*>(ctx->pinned) + (size_t)slot * ctx->pinned_slot_bytes;
    // Small uploads of whole 8-byte words go out in one scatter kernel that reads staging
    // directly; the others as one host-to-device copy each.
    bool scatter = n <= kyro::kMaxUploads && total <= (size_t(1) << 22);
    for (int i = 0; i < n; ++i)
        if (ups[i].bytes % 8 != 0 || reinterpret_cast<uintptr_t>(ups[i].dst) % 8 != 0) scatter = false;
    kyro::UploadArgs sa{};
    sa.src = static_cast<const char*>(ctx->pinned_dev) + (size_t)slot * ctx->pinned_slot_bytes;
    size_t off = 0;
    for (int i = 0; i < n; ++i) {
        if (ups[i].bytes == 0) continue;
        std::memcpy(p + off, ups[i].src, ups[i].bytes);
        if (scatter) {
            sa.off[sa.n] = (int64_t)off;
            sa.dst[sa.n] = static_cast<uint64_t*>(ups[i].dst);
            sa.words[sa.n] = (int64_t)(ups[i].bytes / 8);
            ++sa.n;
        } else {
            KYRO_HIP(hipMemcpyAsync(ups[i].dst, p + off, ups[i].bytes, hipMemcpyHostToDevice, ctx->stream));
        }
        off += align_up(ups[i].bytes, 256);
    }
    if (scatter) KYRO_HIP(kyro::launch_upload_scatter(sa, ctx->stream));
    KYRO_HIP(hipEventRecord(ctx->pinned_done[slot], ctx->stream));
    return KYRO_OK;
}

}  // namespace rt
}  // namespace kyro

using namespace kyro::rt;

namespace {

int sync_and_report(kyro_ctx ctx) {
    KYRO_HIP(hipStreamSynchronize(ctx->stream));
    int err = 0;
    KYRO_HIP(hipMemcpy(&err, ctx->err, sizeof(int), hipMemcpyDeviceToHost));
    if (err == 0) return KYRO_OK;
    KYRO_HIP(hipMemset(ctx->err, 0, sizeof(int)));
    std::string msg = "device-side validation failed:";
    if (err & kyro::ERR_BLOCK_ID) msg += " block_table entry outside [0, num_blocks);";
    if (err & kyro::ERR_CTX_LEN)
        msg += " context length < 0 or > max_blocks_per_seq * block_size (or, for kv_append, below the new rows);";
    if (err & kyro::ERR_Q_LAYOUT) msg += " q_start_loc not monotone / out of range, or q_len > max_q_len;";
    if (err & kyro::ERR_TOKEN) msg += " a draft, bias or penalty token id >= vocab_size, or a mask_row >= num_masks;";
    if (err & kyro::ERR_NUM_DRAFT) msg += " num_draft outside [0, max_draft];";
    if (err & kyro::ERR_NO_DRAFT) msg += " draft_logits is NULL but a sampled sequence has drafts;";
    if (err & kyro::ERR_PLAN)
        msg += " balanced attention schedule: the plan needs more partial-state slots than were sized "
               "(internal error; no item ran);";
    return fail(KYRO_EINVAL, "%s", msg.c_str());
}

}  // namespace

namespace {

constexpr int kDefaultCUs = 256;  // MI355X; used when no context (device) is given

// Everything a paged-attention launch decides from its params alone: validation, kernel, work
// decomposition, schedule and workspace size. No device call.
struct AttnSetup {
    kyro::AttnArgs a{};
    int kernel = 0;
    bool empty = false;      // nothing to launch (B or total_q is 0)
    size_t plan_slots = 0;   // balanced schedule: partial-state slots sized
    size_t ws_bytes = 0;     // arena bytes the launch takes
};

int attention_setup(const kyro_paged_attention_params* p, bool have_q_start, int num_cus, AttnSetup& s,
                    int chunk_quarters = kyro::kPlanChunkQuarters) {
    if (!p) return fail(KYRO_EINVAL, "paged_attention: params is null");
    if (p->block_size <= 0 || p->num_heads <= 0 || p->head_dim <= 0 || p->num_kv_heads <= 0)
        return fail(KYRO_EINVAL, "paged_attention: block_size/num_heads/head_dim/num_kv_heads must be > 0");
    if (p->num_heads % p->num_kv_heads != 0)
        return fail(KYRO_EINVAL, "paged_attention: num_heads %d not a multiple of num_kv_heads %d",
                    p->num_heads, p->num_kv_heads);
    if (p->batch_size < 0 || p->total_q < 0 || p->max_blocks_per_seq < 0 || p->num_blocks < 0)
        return fail(KYRO_EINVAL, "paged_attention: negative shape");
    if (p->dtype != KYRO_F32 && p->dtype != KYRO_BF16)
        return fail(KYRO_EINVAL, "paged_attention: dtype %d unknown", p->dtype);
    if (p->out_dtype != KYRO_F32 && p->out_dtype != KYRO_BF16)
        return fail(KYRO_EINVAL, "paged_attention: out_dtype %d unknown", p->out_dtype);
    if (!have_q_start && p->total_q != p->batch_size)
        return fail(KYRO_EINVAL, "paged_attention: total_q %d != batch_size %d without q_start_loc",
                    p->total_q, p->batch_size);
    if (p->head_dim % 8 != 0 || p->head_dim > kyro::kMaxHeadDim)
        return fail(KYRO_EUNSUPPORTED, "paged_attention: head_dim %d (supported: multiples of 8 up to %d)",
                    p->head_dim, kyro::kMaxHeadDim);
    if (p->path < KYRO_ATTN_AUTO || p->path > KYRO_ATTN_MFMA)
        return fail(KYRO_EINVAL, "paged_attention: path %d unknown", p->path);
    if (p->kv_reuse < KYRO_KV_REUSE_AUTO || p->kv_reuse > KYRO_KV_REUSE_STREAM)
        return fail(KYRO_EINVAL, "paged_attention: kv_reuse %d unknown", p->kv_reuse);
    if (p->schedule < KYRO_ATTN_SCHEDULE_AUTO || p->schedule > KYRO_ATTN_SCHEDULE_BALANCED)
        return fail(KYRO_EINVAL, "paged_attention: schedule %d unknown", p->schedule);
    if (p->schedule == KYRO_ATTN_SCHEDULE_BALANCED && p->num_splits != 0)
        return fail(KYRO_EINVAL, "paged_attention: the balanced schedule chooses its own splits (num_splits must be 0)");
    if (p->schedule == KYRO_ATTN_SCHEDULE_BALANCED && p->batch_size > kyro::kPlanMaxSeqs)
        return fail(KYRO_EUNSUPPORTED, "paged_attention: the balanced schedule plans at most %d sequences",
                    kyro::kPlanMaxSeqs);
    if (p->batch_size == 0 || p->total_q == 0) {
        s.empty = true;
        return KYRO_OK;
    }
    const int group = p->num_heads / p->num_kv_heads;
    int max_q_len = p->max_q_len;
    if (max_q_len <= 0) max_q_len = have_q_start ? p->total_q : 1;
    if (!have_q_start) max_q_len = 1;

    // The MFMA kernels walk 16-token slots: any block size that is a multiple of 16, with every
    // slot's index (block x kv heads x slots per block) in 31 bits.
    const bool mfma_blocks = p->block_size % 16 == 0 &&
                             (long long)p->num_blocks * p->num_kv_heads * (p->block_size / 16) < (1ll << 31);
    const bool mfma_ok = mfma_blocks && kyro::mfma_head_dim(p->head_dim, p->dtype == KYRO_BF16);
    int kernel;
    if (p->path == KYRO_ATTN_MFMA) {
        if (!mfma_ok)
            return fail(KYRO_EUNSUPPORTED, "paged_attention: the MFMA kernel needs a block_size that is a multiple of "
                        "16 and head_dim 128 (bf16 caches: 80, 112 or a multiple of 32 from 64 to 256); got block_size %d, "
                        "head_dim %d",
                        p->block_size, p->head_dim);
        kernel = kyro::ATTN_KERNEL_MFMA;
    } else if (p->path == KYRO_ATTN_VECTOR) {
        kernel = kyro::ATTN_KERNEL_VECTOR;
    } else {
        // MFMA wherever it applies, one query row per kv head included: the kernel is
        // memory-bound, so padding rows to a 16-row tile costs nothing measurable (MHA decode,
        // 1 row per kv head: 67 us against the vector kernel's 207 us).
        kernel = mfma_ok ? kyro::ATTN_KERNEL_MFMA : kyro::ATTN_KERNEL_VECTOR;
    }
    if (p->schedule == KYRO_ATTN_SCHEDULE_BALANCED && kernel != kyro::ATTN_KERNEL_MFMA)
        return fail(KYRO_EUNSUPPORTED, "paged_attention: the balanced schedule runs on the MFMA kernel "
                    "(block_size a multiple of 16; head_dim 128, or 80, 112 or a multiple of 32 from 64 to 256 with "
                    "bf16 caches)");

    kyro::AttnArgs& a = s.a;
    a.B = p->batch_size;
    a.H = p->num_heads;
    a.Hkv = p->num_kv_heads;
    a.group = group;
    a.D = p->head_dim;
    a.bs = p->block_size;
    a.ubs = kernel == kyro::ATTN_KERNEL_MFMA ? 16 : p->block_size;
    a.sub = a.bs / a.ubs;
    a.max_blocks = p->max_blocks_per_seq;
    a.num_blocks = p->num_blocks;
    a.total_q = p->total_q;
    a.max_q_len = max_q_len;
    a.rows_cap = group * max_q_len;
    a.causal = p->causal ? 1 : 0;
    a.out_bf16 = p->out_dtype == KYRO_BF16;
    a.dtype_bf16 = p->dtype == KYRO_BF16;
    const double scale = p->scale > 0 ? (double)p->scale : 1.0 / std::sqrt((double)p->head_dim);
    a.scale_log2 = (float)(scale * 1.4426950408889634);
    a.units = p->batch_size * p->num_kv_heads;
    // Row groups: a unit's group * max_q_len query rows are spread over workgroups of 8
    // (vector) or 16 / 32 / 64 / 80 (MFMA) rows that stream the same K/V. The five-tile choice
    // reads the average rows per kv head from total_q (an upper bound when q has padding rows).
    const int rows_per_group = kernel == kyro::ATTN_KERNEL_MFMA
                                   ? kyro::mfma_rows_per_group(a.rows_cap, p->dtype == KYRO_BF16, p->head_dim,
                                                               (long long)p->total_q * group, p->batch_size)
                                   : kyro::kVectorRowsPerGroup;
    // The MFMA kernel gives one workgroup two adjacent kv heads of a sequence when it can (two
    // waves per head): the workgroup then reads both heads' slabs of each block together, and
    // the Llama-3-8B step fits the chip in one round of workgroups. The 64-row kernel takes one
    // kv head per workgroup (its four waves and its LDS are that head's), and so does the
    // one-tile kernel under MHA (one query head per kv head): twice the workgroups, two a CU,
    // each streaming half the bytes, which evens out ragged context lengths (MHA Llama-2-7B
    // batch, ctx 512-2048: bf16 61.7 -> 57.3 us, f32 131.5 -> 121.7 us; uniform MHA shapes
    // 0.5-1.5% faster in bf16, 2-2.5% slower in f32). GQA batches keep head pairs (ragged GQA
    // 32/8 decode measured 107 -> 111 us with one head).
    const bool one_head = rows_per_group <= 16 && group == 1;
    a.hpw = (kernel == kyro::ATTN_KERNEL_MFMA && p->num_kv_heads % 2 == 0 && rows_per_group <= 32 && !one_head)
                ? 2 : 1;
    a.ugroups = a.units / a.hpw;
    a.ugroups_padded = (a.ugroups + 7) / 8 * 8;
    a.row_groups = std::max(1, (a.rows_cap + rows_per_group - 1) / rows_per_group);
    a.rows_per_group = rows_per_group;
    // Streaming K/V loads unless another workgroup reads the same slabs: the other row groups
    // of a kv head, or (as the caller says) other sequences holding the same blocks. The
    // four- and five-tile kernels decide per unit under AUTO: on a ragged batch only the units
    // with more rows than a group holds have a second row group.
    a.stream_kv = p->kv_reuse == KYRO_KV_REUSE_STREAM || (p->kv_reuse == KYRO_KV_REUSE_AUTO && a.row_groups == 1);
    if (p->kv_reuse == KYRO_KV_REUSE_AUTO && a.row_groups > 1 && rows_per_group >= kyro::kMfmaManyRows)
        a.stream_kv = kyro::kKvPerUnit;

    // Context splits: enough workgroups to cover the chip, chunks of whole slot pairs (a slot is
    // a block of the vector kernel, 16 tokens of the MFMA kernels).
    const long long mb_slots = (long long)std::max(1, p->max_blocks_per_seq) * a.sub;
    if (mb_slots > (1ll << 30))
        return fail(KYRO_EUNSUPPORTED, "paged_attention: max_blocks_per_seq %d x block_size %d tokens is too long",
                    p->max_blocks_per_seq, p->block_size);
    const int mb = (int)mb_slots;
    int splits = p->num_splits;
    if (splits <= 0) {
        // At most ~256 blocks (4096 tokens) per workgroup so a long context does not leave
        // one CU streaming it alone; more splits only when the workgroups cannot cover the
        // chip's CUs (the MFMA kernel holds one workgroup per CU), down to 16-block chunks.
        // With four or more workgroups per CU already, splitting only adds per-workgroup
        // set-up and a combine pass (one workgroup fills a CU, so nothing hides them).
        constexpr int kTargetChunk = 256, kMinChunk = 16;
        const int kCUs = num_cus;
        const int per_split = a.ugroups * a.row_groups;
        splits = per_split >= 4 * kCUs ? 1 : (mb + kTargetChunk - 1) / kTargetChunk;
        if (per_split * splits < kCUs)
            splits = std::min((kCUs + per_split - 1) / per_split, std::max(1, mb / kMinChunk));
    }
    // Longest split: the LDS block-id staging, and for the MFMA kernel the block pairs a wave
    // holds ids for (its waves per head x two 64-lane slots).
    const int max_chunk = kernel == kyro::ATTN_KERNEL_MFMA
                              ? std::min(kyro::kMaxChunkBlocks, 2 * kyro::kMfmaMaxPairsPerWave * (4 / a.hpw))
                              : kyro::kMaxChunkBlocks;
    splits = std::min(splits, mb);
    splits = std::max(splits, (mb + max_chunk - 1) / max_chunk);
    int chunk = (mb + splits - 1) / splits;
    chunk = std::min((chunk + 1) / 2 * 2, max_chunk);
    splits = (mb + chunk - 1) / chunk;
    a.splits = splits;
    a.chunk_blocks = chunk;
    // The balanced schedule: asked for, or where the grid's splits (from the table width
    // alone) would have to guess at the context lengths: a split grid, or a table wider than
    // 256 blocks (4096 tokens), where a few long sequences can leave one workgroup streaming
    // long after the rest of the chip is idle.
    a.plan = kernel == kyro::ATTN_KERNEL_MFMA && p->num_splits == 0 && p->batch_size <= kyro::kPlanMaxSeqs &&
             (p->schedule == KYRO_ATTN_SCHEDULE_BALANCED ||
              (p->schedule == KYRO_ATTN_SCHEDULE_AUTO && (splits > 1 || mb > 256)));
    if (a.plan) {
        // One persistent workgroup per CU, in whole rounds of the 8 XCD lanes the plan deals
        // to (a partitioned device with fewer CUs still gets every lane covered).
        a.plan_grid = std::max(8, num_cus / 8 * 8);
        a.plan_rw = rows_per_group;
        a.plan_max_chunk = max_chunk / 2 * 2;
        a.splits = 1;
        s.plan_slots = (size_t)kyro::plan_slot_bound(a.B, a.ugroups / a.B, a.row_groups, mb, a.plan_max_chunk,
                                                     a.plan_grid, chunk_quarters);
        // kyro_testing_set_plan_slot_cap lowers the slots sized, so that a test can drive the
        // device plan's overflow check (ERR_PLAN, no item runs) without a plan/bound mismatch.
        // Zero (the state a process starts in) sizes the bound.
        const int64_t cap = g_test_plan_slot_cap.load(std::memory_order_relaxed);
        if (cap > 0 && (size_t)cap < s.plan_slots) s.plan_slots = (size_t)cap;
        a.plan_slots = (long long)s.plan_slots;
    }
    // One launch carries at most 2^32 - 1 work items along x.
    if (!a.plan && (uint64_t)a.ugroups_padded * splits * a.row_groups * 256 > 0xffffffffull)
        return fail(KYRO_EUNSUPPORTED, "paged_attention: %d units x %d splits x %d row groups is too large for one launch",
                    a.units, splits, a.row_groups);
    s.kernel = kernel;
    if (a.plan) {
        const size_t rows = s.plan_slots * a.hpw * a.plan_rw;
        s.ws_bytes = 2 * align_up(rows * sizeof(float), 256) + align_up(rows * a.D * sizeof(float), 256) +
                     align_up((size_t)a.B * sizeof(int4), 256) + align_up((size_t)(a.B + 1) * sizeof(int), 256);
    } else if (a.splits > 1) {
        const size_t rows = (size_t)a.units * a.splits * a.rows_cap;
        s.ws_bytes = 2 * align_up(rows * sizeof(float), 256) + align_up(rows * a.D * sizeof(float), 256);
    }
    return KYRO_OK;
}

// Points the launch's partial-state arrays (and the plan's per-sequence tables) into `base`,
// s.ws_bytes of device memory.
void attention_workspace(AttnSetup& s, char* base) {
    kyro::AttnArgs& a = s.a;
    const size_t rows = a.plan ? s.plan_slots * a.hpw * a.plan_rw : (size_t)a.units * a.splits * a.rows_cap;
    const size_t mb_bytes = align_up(rows * sizeof(float), 256);
    a.ws_m = reinterpret_cast<float*>(base);
    a.ws_l = reinterpret_cast<float*>(base + mb_bytes);
    a.ws_acc = reinterpret_cast<float*>(base + 2 * mb_bytes);
    if (a.plan) {
        char* p = base + 2 * mb_bytes + align_up(rows * a.D * sizeof(float), 256);
        a.plan_seq = reinterpret_cast<int4*>(p);
        a.plan_cw = reinterpret_cast<int*>(p + align_up((size_t)a.B * sizeof(int4), 256));
    }
}

// Everything a verify launch decides from its params alone: validation, chunking, window,
// tail grid and workspace size. No device call.
struct SpecSetup {
    kyro::SpecArgs a{};
    bool empty = false;  // batch_size 0
    size_t stats_b = 0, plan_b = 0, csum_b = 0, gath_b = 0, tail_b = 0;
    size_t ws_bytes = 0;
};

int spec_setup(const kyro_spec_verify_params* p, SpecSetup& s) {
    if (!p) return fail(KYRO_EINVAL, "spec_verify: params is null");
    if (p->batch_size < 0 || p->max_draft < 0 || p->vocab_size <= 0)
        return fail(KYRO_EINVAL, "spec_verify: need batch_size >= 0, max_draft >= 0, vocab_size > 0");
    if (p->max_draft > kyro::kMaxDraft)
        return fail(KYRO_EUNSUPPORTED, "spec_verify: max_draft %d > %d", p->max_draft, kyro::kMaxDraft);
    if (p->logits_dtype != KYRO_F32)
        return fail(KYRO_EUNSUPPORTED, "spec_verify: logits_dtype must be KYRO_F32");
    if (p->window < 0) return fail(KYRO_EINVAL, "spec_verify: window must be >= 0");
    if (p->batch_size == 0) {
        s.empty = true;
        return KYRO_OK;
    }
    kyro::SpecArgs& a = s.a;
    a.B = p->batch_size;
    a.kmax = p->max_draft;
    a.V = p->vocab_size;
    a.chunk = kyro::kSpecChunk;
    a.C = (a.V + a.chunk - 1) / a.chunk;
    // Rows of the first win draft positions are read for every sequence; the rest only for
    // sequences still undecided after them, spread over up to kSpecTailWgs workgroups. Batches
    // beyond kMaxLazyBatch read every row in the first pass, and so do batches whose rows
    // all together are few enough that reading them costs less than the tail pass's launch
    // (rejection-only B 8, k 4, V 32000: 9.2 MB, 20.7 us instead of 27.1 us at W = 3).
    a.win = p->window > 0 ? std::min(p->window, a.kmax + 1) : std::max(1, kyro::kSpecWindow);
    const long long all_rows_bytes = (long long)a.B * (2 * a.kmax + 1) * a.V * (long long)sizeof(float);
    if (p->window == 0 && all_rows_bytes <= kyro::kSpecEagerBytes) a.win = a.kmax + 1;
    if (a.B > kyro::kMaxLazyBatch) a.win = a.kmax + 1;
    const long long tail_items = a.kmax >= a.win ? (long long)a.B * (2 * (a.kmax - a.win) + 1) * a.C : 1;
    // Up to kSpecTailWgs workgroups, more when that would give one workgroup more than 64
    // items (the tail pass keeps one item's location per lane of a wave).
    a.tail_wgs = (int)std::min<long long>(
        INT32_MAX, std::max({1LL, std::min((long long)kyro::kSpecTailWgs, tail_items), (tail_items + 63) / 64}));
    s.stats_b = align_up((size_t)a.B * (2 * a.kmax + 1) * a.C * sizeof(float2), 256);
    s.plan_b = 2 * align_up((size_t)a.B * sizeof(kyro::SpecPlan), 256);
    s.csum_b = align_up((size_t)a.B * a.C * sizeof(float2), 256);
    s.gath_b = align_up((size_t)a.B * (2 * a.kmax + 1) * sizeof(float), 256);
    s.tail_b = align_up((size_t)a.B * sizeof(int2), 256);
    s.ws_bytes = s.stats_b + s.plan_b + s.csum_b + s.gath_b + s.tail_b;
    return KYRO_OK;
}

// Checks and binds the caller's device pointers.
int spec_bind(SpecSetup& s, const void* target_logits, const void* draft_logits, const uint32_t* draft_tokens,
              const int32_t* num_draft, const float* temperature, const float* u_accept, const float* u_resample,
              int32_t* out_accepted, uint32_t* out_tokens, float* out_p_draft, float* out_q_draft) {
    kyro::SpecArgs& a = s.a;
    if (!target_logits || !num_draft || !temperature || !u_resample || !out_accepted || !out_tokens)
        return fail(KYRO_EINVAL, "spec_verify: null device pointer");
    if (a.kmax > 0 && (!draft_tokens || !u_accept))
        return fail(KYRO_EINVAL, "spec_verify: draft_tokens and u_accept are required when max_draft > 0");
    a.target = static_cast<const float*>(target_logits);
    a.draft = static_cast<const float*>(draft_logits);
    a.draft_tokens = draft_tokens;
    a.num_draft = num_draft;
    a.temperature = temperature;
    a.u_accept = u_accept;
    a.u_res = u_resample;
    a.out_accepted = out_accepted;
    a.out_tokens = out_tokens;
    a.out_p = out_p_draft;
    a.out_q = out_q_draft;
    const bool aligned = (reinterpret_cast<uintptr_t>(target_logits) % 16 == 0) &&
                         (reinterpret_cast<uintptr_t>(draft_logits) % 16 == 0);
    a.vec4 = (a.V % 4 == 0) && aligned;
    return KYRO_OK;
}

// Points the launch's statistics, plans and chunk sums into `base`, s.ws_bytes of device memory.
void spec_workspace(SpecSetup& s, char* base) {
    kyro::SpecArgs& a = s.a;
    a.stats = reinterpret_cast<float2*>(base);
    a.plan = reinterpret_cast<kyro::SpecPlan*>(base + s.stats_b);
    a.plan_tail = reinterpret_cast<kyro::SpecPlan*>(base + s.stats_b + s.plan_b / 2);
    a.csum = reinterpret_cast<float2*>(base + s.stats_b + s.plan_b);
    a.gath = reinterpret_cast<float*>(base + s.stats_b + s.plan_b + s.csum_b);
    a.tail = reinterpret_cast<int2*>(base + s.stats_b + s.plan_b + s.csum_b + s.gath_b);
}

}  // namespace

extern "C" {

const char* kyro_last_error(void) { return g_last_error.c_str(); }

int kyro_abi_version(void) { return KYRO_ABI_VERSION; }

int64_t kyro_testing_set_plan_slot_cap(int64_t cap) {
    return g_test_plan_slot_cap.exchange(cap < 0 ? 0 : cap, std::memory_order_relaxed);
}

int kyro_ctx_create(int device, kyro_ctx* out) {
    return guarded([&]() -> int {
        if (!out) return fail(KYRO_EINVAL, "kyro_ctx_create: out is null");
        *out = nullptr;
        int n = 0;
        KYRO_HIP(hipGetDeviceCount(&n));
        if (device < 0 || device >= n)
            return fail(KYRO_EINVAL, "kyro_ctx_create: device %d not in [0, %d)", device, n);
        DeviceGuard dg(device);
        KYRO_HIP(dg.status);
        kyro_ctx ctx = new kyro_ctx_s();
        ctx->device = device;
        hipError_t e = hipStreamCreateWithFlags(&ctx->own_stream, hipStreamNonBlocking);
        if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&ctx->err), sizeof(int));
        if (e == hipSuccess) e = hipMemset(ctx->err, 0, sizeof(int));
        if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&ctx->sched), kyro::kSchedWords * sizeof(int));
        if (e == hipSuccess) e = hipMemset(ctx->sched, 0, kyro::kSchedWords * sizeof(int));
        if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&ctx->row_cnt), kyro::kSampleRowCounters * sizeof(int));
        if (e == hipSuccess) e = hipMemset(ctx->row_cnt, 0, kyro::kSampleRowCounters * sizeof(int));
        if (e == hipSuccess) e = hipDeviceGetAttribute(&ctx->num_cus, hipDeviceAttributeMultiprocessorCount, device);
        if (e == hipSuccess && ctx->num_cus <= 0) e = hipErrorInvalidDevice;
        // Set-up of kyro_spec_verify_noalloc: the static scratch array's address on this device.
        // That entry point is optional: when the lookup fails the context is still created,
        // noalloc_scratch stays null and only kyro_spec_verify_noalloc reports KYRO_EHIP.
        if (e == hipSuccess && kyro::noalloc_scratch(device, &ctx->noalloc_scratch) != hipSuccess) {
            ctx->noalloc_scratch = nullptr;
            (void)hipGetLastError();  // the failed lookup must not surface from a later call
        }
        if (e == hipSuccess) e = hipStreamSynchronize(0);  // the memsets are done before any launch
        if (e != hipSuccess) {
            if (ctx->err) (void)hipFree(ctx->err);
            if (ctx->sched) (void)hipFree(ctx->sched);
            if (ctx->row_cnt) (void)hipFree(ctx->row_cnt);
            if (ctx->own_stream) (void)hipStreamDestroy(ctx->own_stream);
            delete ctx;
            return fail(KYRO_EHIP, "kyro_ctx_create: %s", hipGetErrorString(e));
        }
        ctx->stream = ctx->own_stream;
        *out = ctx;
        return KYRO_OK;
    });
}

int kyro_ctx_destroy(kyro_ctx ctx) {
    return guarded([&]() -> int {
        if (!ctx) return KYRO_OK;
        DeviceGuard dg(ctx->device);
        (void)hipStreamSynchronize(ctx->stream);
        if (ctx->stream != ctx->own_stream) (void)hipStreamSynchronize(ctx->own_stream);
        if (ctx->arena) (void)hipFree(ctx->arena);
        if (ctx->err) (void)hipFree(ctx->err);
        if (ctx->sched) (void)hipFree(ctx->sched);
        if (ctx->row_cnt) (void)hipFree(ctx->row_cnt);
        for (hipEvent_t& e : ctx->pinned_done)
            if (e) (void)hipEventSynchronize(e);
        if (ctx->pinned) (void)hipHostFree(ctx->pinned);
        for (hipEvent_t& e : ctx->pinned_done)
            if (e) (void)hipEventDestroy(e);
        if (ctx->own_stream) (void)hipStreamDestroy(ctx->own_stream);
        delete ctx;
        return KYRO_OK;
    });
}

int kyro_ctx_set_stream(kyro_ctx ctx, void* hip_stream) {
    return guarded([&]() -> int {
        if (int rc = check_ctx(ctx)) return rc;
        hipStream_t next = static_cast<hipStream_t>(hip_stream);
        if (next == ctx->stream) return KYRO_OK;
        DeviceGuard dg(ctx->device);
        KYRO_HIP(dg.status);
        // The arena is ordered on one stream at a time: drain the old one before switching.
        KYRO_HIP(hipStreamSynchronize(ctx->stream));
        ctx->stream = next;
        return KYRO_OK;
    });
}

int kyro_ctx_reserve(kyro_ctx ctx, size_t bytes) {
    return guarded([&]() -> int {
        if (int rc = check_ctx(ctx)) return rc;
        DeviceGuard dg(ctx->device);
        KYRO_HIP(dg.status);
        return ensure_arena(ctx, bytes);
    });
}

int kyro_sync(kyro_ctx ctx) {
    return guarded([&]() -> int {
        if (int rc = check_ctx(ctx)) return rc;
        DeviceGuard dg(ctx->device);
        KYRO_HIP(dg.status);
        return sync_and_report(ctx);
    });
}

int kyro_check(kyro_ctx ctx) { return kyro_sync(ctx); }

int kyro_buf_alloc(kyro_ctx ctx, size_t bytes, kyro_buf* out) {
    return guarded([&]() -> int {
        if (int rc = check_ctx(ctx)) return rc;
        if (!out) return fail(KYRO_EINVAL, "kyro_buf_alloc: out is null");
        *out = nullptr;
        DeviceGuard dg(ctx->device);
        KYRO_HIP(dg.status);
        void* p = nullptr;
        KYRO_HIP(hipMalloc(&p, bytes ? bytes : 1));
        kyro_buf b = new kyro_buf_s();
        b->device = ctx->device;
        b->ptr = p;
        b->bytes = bytes;
        *out = b;
        return KYRO_OK;
    });
}

int kyro_buf_free(kyro_buf buf) {
    return guarded([&]() -> int {
        if (!buf) return KYRO_OK;
        DeviceGuard dg(buf->device);
        if (buf->ptr) KYRO_HIP(hipFree(buf->ptr));
        delete buf;
        return KYRO_OK;
    });
}

void* kyro_buf_ptr(kyro_buf buf) { return buf ? buf->ptr : nullptr; }

size_t kyro_buf_size(kyro_buf buf) { return buf ? buf->bytes : 0; }

int kyro_buf_upload(kyro_ctx ctx, kyro_buf dst, size_t dst_offset, const void* src, size_t bytes) {
    return guarded([&]() -> int {
        if (int rc = check_ctx(ctx)) return rc;
        if (!dst || (!src && bytes)) return fail(KYRO_EINVAL, "kyro_buf_upload: null buffer");
        if (dst_offset > dst->bytes || bytes > dst->bytes - dst_offset)
            return fail(KYRO_EINVAL, "kyro_buf_upload: %zu bytes at offset %zu exceed buffer of %zu",
                        bytes, dst_offset, dst->bytes);
        DeviceGuard dg(ctx->device);
        KYRO_HIP(dg.status);
        KYRO_HIP(hipMemcpyAsync(static_cast<char*>(dst->ptr) + dst_offset, src, bytes,
                                hipMemcpyHostToDevice, ctx->stream));
        KYRO_HIP(hipStreamSynchronize(ctx->stream));
        return KYRO_OK;
    });
}

int kyro_buf_download(kyro_ctx ctx, void* dst, kyro_buf src, size_t src_offset, size_t bytes) {
    return guarded([&]() -> int {
        if (int rc = check_ctx(ctx)) return rc;
        if (!src || (!dst && bytes)) return fail(KYRO_EINVAL, "kyro_buf_download: null buffer");
        if (src_offset > src->bytes || bytes > src->bytes - src_offset)
            return fail(KYRO_EINVAL, "kyro_buf_download: %zu bytes at offset %zu exceed buffer of %zu",
                        bytes, src_offset, src->bytes);
        DeviceGuard dg(ctx->device);
        KYRO_HIP(dg.status);
        KYRO_HIP(hipMemcpyAsync(dst, static_cast<const char*>(src->ptr) + src_offset, bytes,
                                hipMemcpyDeviceToHost, ctx->stream));
        KYRO_HIP(hipStreamSynchronize(ctx->stream));
        return KYRO_OK;
    });
}

int kyro_paged_attention_mq(kyro_ctx ctx, const kyro_paged_attention_params* p, const void* query,
                            const int32_t* q_start_loc, const void* key_cache,
                            const void* value_cache, const int64_t* block_table,
                            const int64_t* context_lens, void* out) {
    return guarded([&]() -> int {
        if (int rc = check_ctx(ctx)) return rc;
        AttnSetup s;
        if (int rc = attention_setup(p, q_start_loc != nullptr, ctx->num_cus, s)) return rc;
        if (s.empty) return KYRO_OK;
        if (!query || !key_cache || !value_cache || !block_table || !context_lens || !out)
            return fail(KYRO_EINVAL, "paged_attention: null device pointer");
        kyro::AttnArgs& a = s.a;
        a.q = query;
        a.q_start = q_start_loc;
        a.k = key_cache;
        a.v = value_cache;
        a.table = block_table;
        a.ctx_lens = context_lens;
        a.out = out;
        DeviceGuard dg(ctx->device);
        KYRO_HIP(dg.status);
        if (s.ws_bytes) {
            if (int rc = ensure_arena(ctx, s.ws_bytes)) return rc;
            attention_workspace(s, static_cast<char*>(ctx->arena));
        }
        if (a.plan) a.sched = ctx->sched;
        a.err = ctx->err;
        KYRO_HIP(kyro::launch_paged_attention(a, s.kernel, ctx->stream));
        return KYRO_OK;
    });
}

int kyro_paged_attention_workspace(kyro_ctx ctx, const kyro_paged_attention_params* p, int has_q_start_loc,
                                   size_t* bytes) {
    return guarded([&]() -> int {
        if (!bytes) return fail(KYRO_EINVAL, "paged_attention_workspace: bytes is null");
        *bytes = 0;
        // A null context sizes for kDefaultCUs (256) compute units; a device with more needs its
        // context here, since the balanced schedule's persistent grid follows the CU count.
        AttnSetup s;
        if (int rc = attention_setup(p, has_q_start_loc != 0, ctx ? ctx->num_cus : kDefaultCUs, s)) return rc;
        *bytes = s.ws_bytes;
        return KYRO_OK;
    });
}

namespace {
// Writes `text` to buf (at most len bytes with its terminator) and the full length to *needed.
int put_text(const std::string& text, char* buf, size_t len, size_t* needed) {
    if (needed) *needed = text.size() + 1;
    if (buf && len > 0) {
        const size_t n = std::min(len - 1, text.size());
        std::memcpy(buf, text.data(), n);
        buf[n] = '\0';
    }
    return KYRO_OK;
}
}  // namespace

int kyro_paged_attention_describe(kyro_ctx ctx, const kyro_paged_attention_params* p, int has_q_start_loc,
                                  char* buf, size_t len, size_t* needed) {
    return guarded([&]() -> int {
        AttnSetup s;
        if (int rc = attention_setup(p, has_q_start_loc != 0, ctx ? ctx->num_cus : kDefaultCUs, s)) return rc;
        if (s.empty) return put_text("nothing to launch (no sequences or no query rows)", buf, len, needed);
        const kyro::AttnArgs& a = s.a;
        char t[512];
        if (s.kernel == kyro::ATTN_KERNEL_MFMA) {
            const int rpg = a.rows_per_group;
            const char* pol = a.stream_kv == kyro::kKvPerUnit ? "per-unit" : a.stream_kv ? "stream" : "cached";
            std::snprintf(t, sizeof t,
                          "%s<row tiles %d, kv heads per workgroup %d, K/V loads %s> schedule %s, "
                          "row groups %d, %s %d, workgroups %d%s",
                          a.dtype_bf16 ? "attn_mfma_kernel" : "attn_mfma_f32_kernel", rpg / 16, a.hpw, pol,
                          a.plan ? "balanced" : "grid", a.row_groups, a.plan ? "max chunk blocks" : "splits",
                          a.plan ? a.plan_max_chunk : a.splits,
                          a.plan ? a.plan_grid : a.ugroups_padded * a.splits * a.row_groups,
                          a.plan ? " + attn_combine_plan_kernel" : a.splits > 1 ? " + attn_combine_kernel" : "");
        } else {
            std::snprintf(t, sizeof t,
                          "attn_vector_kernel<%s, head_dim %d> schedule grid, row groups %d, splits %d, "
                          "workgroups %d%s",
                          a.dtype_bf16 ? "bf16" : "f32", a.D, a.row_groups, a.splits,
                          a.ugroups_padded * a.splits * a.row_groups, a.splits > 1 ? " + attn_combine_kernel" : "");
        }
        return put_text(t, buf, len, needed);
    });
}

int kyro_spec_verify_describe(const kyro_spec_verify_params* p, char* buf, size_t len, size_t* needed) {
    return guarded([&]() -> int {
        SpecSetup s;
        if (int rc = spec_setup(p, s)) return rc;
        if (s.empty) return put_text("nothing to launch (no sequences)", buf, len, needed);
        const kyro::SpecArgs& a = s.a;
        char t[512];
        const bool tail = a.kmax >= a.win;
        const std::string first = tail ? "window of " + std::to_string(a.win) + " of " + std::to_string(a.kmax) +
                                             " draft positions"
                                       : "every row in the first pass";
        const std::string mid = tail ? "spec_decide_kernel, spec_stats_tail_kernel on " + std::to_string(a.tail_wgs) +
                                           " workgroups, spec_resample_kernel"
                                     : "spec_resample_kernel with the acceptance scan";
        std::snprintf(t, sizeof t, "%s; chunks of %d entries, %d per row; spec_stats_kernel, %s, spec_pick_kernel",
                      first.c_str(), a.chunk, a.C, mid.c_str());
        return put_text(t, buf, len, needed);
    });
}

int kyro_paged_attention_plan(const kyro_paged_attention_params* p, int num_cus, int chunk_quarters,
                              const int64_t* context_lens, const int32_t* q_lens, int32_t* out_splits,
                              kyro_attention_plan* out) {
    return guarded([&]() -> int {
        if (!out) return fail(KYRO_EINVAL, "paged_attention_plan: out is null");
        *out = kyro_attention_plan{};
        if (num_cus <= 0) num_cus = kDefaultCUs;
        if (chunk_quarters <= 0) chunk_quarters = kyro::kPlanChunkQuarters;
        AttnSetup s;
        if (int rc = attention_setup(p, q_lens != nullptr, num_cus, s, chunk_quarters)) return rc;
        const kyro::AttnArgs& a = s.a;
        if (s.empty) return KYRO_OK;
        if (!context_lens) return fail(KYRO_EINVAL, "paged_attention_plan: context_lens is null");
        if (!a.plan) return fail(KYRO_EINVAL, "paged_attention_plan: these params run on the grid schedule");
        // The per-sequence quantities of the device plan (plan_build in paged_attention.hip):
        // row groups r, blocks nb, work U r nb; the chunk and the splits come from the functions
        // the device uses.
        const int U = a.Hkv / a.hpw;
        std::vector<int> r(a.B), nb(a.B);
        long long T = 0;
        int maxnb = 0;
        for (int b = 0; b < a.B; ++b) {
            const long long c = context_lens[b];
            const int ql = q_lens ? q_lens[b] : 1;
            if (c < 0 || c > (long long)a.max_blocks * a.bs || ql < 0 || ql > a.max_q_len)
                return fail(KYRO_EINVAL, "paged_attention_plan: sequence %d: context length %lld or rows %d out of range",
                            b, c, ql);
            r[b] = (ql * a.group + a.plan_rw - 1) / a.plan_rw;
            nb[b] = (int)((c + a.ubs - 1) / a.ubs);
            T += (long long)U * r[b] * nb[b];
            if (r[b] > 0) maxnb = std::max(maxnb, nb[b]);
        }
        const int C = kyro::plan_chunk_blocks(T, maxnb, a.plan_grid, a.plan_max_chunk, chunk_quarters);
        long long items = 0;
        for (int b = 0; b < a.B; ++b) {
            int ns, ch;
            kyro::plan_split(nb[b], C, ns, ch);
            if (out_splits) out_splits[b] = r[b] > 0 ? ns : 0;
            if (r[b] > 0) items += (long long)U * ns * r[b];
        }
        out->grid = a.plan_grid;
        out->chunk_blocks = C;
        out->items = items;
        out->slot_bound = s.plan_slots;
        return KYRO_OK;
    });
}

int kyro_spec_verify(kyro_ctx ctx, const kyro_spec_verify_params* p, const void* target_logits,
                     const void* draft_logits, const uint32_t* draft_tokens,
                     const int32_t* num_draft, const float* temperature, const float* u_accept,
                     const float* u_resample, int32_t* out_accepted, uint32_t* out_tokens,
                     float* out_p_draft, float* out_q_draft) {
    return guarded([&]() -> int {
        if (int rc = check_ctx(ctx)) return rc;
        SpecSetup s;
        if (int rc = spec_setup(p, s)) return rc;
        if (s.empty) return KYRO_OK;
        if (int rc = spec_bind(s, target_logits, draft_logits, draft_tokens, num_draft, temperature, u_accept,
                               u_resample, out_accepted, out_tokens, out_p_draft, out_q_draft))
            return rc;
        DeviceGuard dg(ctx->device);
        KYRO_HIP(dg.status);
        if (int rc = ensure_arena(ctx, s.ws_bytes)) return rc;
        spec_workspace(s, static_cast<char*>(ctx->arena));
        s.a.err = ctx->err;
        KYRO_HIP(kyro::launch_spec_verify(s.a, ctx->stream));
        return KYRO_OK;
    });
}

int kyro_spec_verify_noalloc(kyro_ctx ctx, const kyro_spec_verify_params* p, const void* target_logits,
                             const void* draft_logits, const uint32_t* draft_tokens,
                             const int32_t* num_draft, const float* temperature, const float* u_accept,
                             const float* u_resample, int32_t* out_accepted, uint32_t* out_tokens,
                             float* out_p_draft, float* out_q_draft) {
    return guarded([&]() -> int {
        if (int rc = check_ctx(ctx)) return rc;
        SpecSetup s;
        if (int rc = spec_setup(p, s)) return rc;
        if (s.empty) return KYRO_OK;
        if (s.ws_bytes > kyro::kNoAllocScratchBytes)
            return fail(KYRO_EINVAL, "spec_verify_noalloc: the call needs %zu bytes of scratch; the allocation-free "
                        "variant holds %zu (use kyro_spec_verify)", s.ws_bytes, kyro::kNoAllocScratchBytes);
        if (!ctx->noalloc_scratch) return fail(KYRO_EHIP, "spec_verify_noalloc: scratch array not set up");
        if (int rc = spec_bind(s, target_logits, draft_logits, draft_tokens, num_draft, temperature, u_accept,
                               u_resample, out_accepted, out_tokens, out_p_draft, out_q_draft))
            return rc;
        DeviceGuard dg(ctx->device);
        KYRO_HIP(dg.status);
        // The same kernels as kyro_spec_verify, with the scratch in the static array: they write
        // every scratch entry they read within the call, so nothing needs clearing.
        spec_workspace(s, static_cast<char*>(ctx->noalloc_scratch));
        s.a.err = ctx->err;
        KYRO_HIP(kyro::launch_spec_verify(s.a, ctx->stream));
        return KYRO_OK;
    });
}

int kyro_spec_verify_workspace(const kyro_spec_verify_params* p, size_t* bytes) {
    return guarded([&]() -> int {
        if (!bytes) return fail(KYRO_EINVAL, "spec_verify_workspace: bytes is null");
        *bytes = 0;
        SpecSetup s;
        if (int rc = spec_setup(p, s)) return rc;
        *bytes = s.ws_bytes;
        return KYRO_OK;
    });
}

int kyro_paged_kv_append(kyro_ctx ctx, const kyro_kv_append_params* p, const void* key,
                         const void* value, const int32_t* q_start_loc, const int64_t* block_table,
                         const int64_t* context_lens, void* key_cache, void* value_cache) {
    return guarded([&]() -> int {
        if (int rc = check_ctx(ctx)) return rc;
        if (!p) return fail(KYRO_EINVAL, "kv_append: params is null");
        if (p->block_size <= 0 || p->num_kv_heads <= 0 || p->head_dim <= 0 || p->batch_size < 0 ||
            p->total_q < 0 || p->max_blocks_per_seq <= 0 || p->num_blocks <= 0 || p->max_q_len < 0)
            return fail(KYRO_EINVAL, "kv_append: sizes must be positive (batch_size, total_q, max_q_len >= 0)");
        if (p->head_dim % 8 != 0)
            return fail(KYRO_EUNSUPPORTED, "kv_append: head_dim %d is not a multiple of 8", p->head_dim);
        if ((p->src_dtype != KYRO_F32 && p->src_dtype != KYRO_BF16) ||
            (p->cache_dtype != KYRO_F32 && p->cache_dtype != KYRO_BF16))
            return fail(KYRO_EINVAL, "kv_append: unknown dtype");
        if (!q_start_loc && p->total_q != p->batch_size)
            return fail(KYRO_EINVAL, "kv_append: without q_start_loc total_q must equal batch_size");
        if (p->batch_size == 0 || p->total_q == 0) return KYRO_OK;
        if (!key || !value || !block_table || !context_lens || !key_cache || !value_cache)
            return fail(KYRO_EINVAL, "kv_append: null device pointer");
        const size_t row_vecs = (size_t)p->num_kv_heads * p->head_dim / 8;
        if (row_vecs > (size_t)INT32_MAX / 2)
            return fail(KYRO_EUNSUPPORTED, "kv_append: num_kv_heads * head_dim too large");
        kyro::KvAppendArgs a{};
        a.key = key;
        a.value = value;
        a.q_start = q_start_loc;
        a.table = block_table;
        a.ctx_lens = context_lens;
        a.kc = key_cache;
        a.vc = value_cache;
        a.B = p->batch_size;
        a.Hkv = p->num_kv_heads;
        a.D = p->head_dim;
        a.bs = p->block_size;
        a.max_blocks = p->max_blocks_per_seq;
        a.num_blocks = p->num_blocks;
        a.total_q = p->total_q;
        a.max_q_len = p->max_q_len > 0 ? p->max_q_len : (q_start_loc ? p->total_q : 1);
        if (!q_start_loc) a.max_q_len = 1;
        a.src_bf16 = p->src_dtype == KYRO_BF16;
        a.cache_bf16 = p->cache_dtype == KYRO_BF16;
        a.vecs_per_row = (int)row_vecs;
        if ((long long)a.max_q_len * a.vecs_per_row > (long long)INT32_MAX - 256)
            return fail(KYRO_EUNSUPPORTED, "kv_append: max_q_len * num_kv_heads * head_dim too large");
        const uintptr_t align = reinterpret_cast<uintptr_t>(key) | reinterpret_cast<uintptr_t>(value) |
                                reinterpret_cast<uintptr_t>(key_cache) | reinterpret_cast<uintptr_t>(value_cache);
        if (align % 16 != 0) return fail(KYRO_EINVAL, "kv_append: tensors must be 16-byte aligned");
        DeviceGuard dg(ctx->device);
        KYRO_HIP(dg.status);
        a.err = ctx->err;
        KYRO_HIP(kyro::launch_kv_append(a, ctx->stream));
        return KYRO_OK;
    });
}

}  // extern "C"
