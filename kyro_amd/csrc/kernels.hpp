// Kernel argument blocks and launchers shared by the host runtime and the .hip kernel files.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kyro {

// Bits latched into the context's device error word. The host turns them into KYRO_EINVAL.
enum ErrorBits : int {
    ERR_BLOCK_ID = 1,   // block_table entry outside [0, num_blocks)
    ERR_CTX_LEN = 2,    // context length < 0 or > max_blocks_per_seq * block_size (kv append: < q_len)
    ERR_Q_LAYOUT = 4,   // q_start_loc not monotone, out of [0, total_q], or a q_len > max_q_len
    ERR_TOKEN = 8,      // draft token id >= vocab_size
    ERR_NUM_DRAFT = 16, // num_draft outside [0, max_draft]
    ERR_NO_DRAFT = 32,  // a sampled sequence with drafts but no draft_logits
    ERR_PLAN = 64       // balanced attention schedule: more partial-state slots than the host sized
};


enum AttnKernel : int { ATTN_KERNEL_VECTOR = 1, ATTN_KERNEL_MFMA = 2 };

// Cache-policy operands of buffer loads on gfx950: default, or the nontemporal hint (bit 1) for
// data a launch reads once. Streaming 1 GiB with 16-byte loads measured 6.0 TB/s with the default
// policy and 6.8-7.0 TB/s with the hint; data read again by another workgroup then misses L2.
constexpr int kLoadCached = 0;
constexpr int kLoadStream = 2;
// Not a hardware policy: the kernel picks kLoadStream or kLoadCached per unit.
constexpr int kLoadPerUnit = -1;
// AttnArgs::stream_kv value that selects kLoadPerUnit (four- and five-tile kernels only).
constexpr int kKvPerUnit = 2;

// Upper bound on the blocks one attention workgroup streams (its split); the block ids of a
// split are staged in LDS.
constexpr int kMaxChunkBlocks = 1024;

struct AttnArgs {
    const void* q;
    const int32_t* q_start;  // [B+1] or nullptr (row b belongs to sequence b)
    const void* k;
    const void* v;
    const int64_t* table;
    const int64_t* ctx_lens;
    void* out;
    float* ws_m;     // [units, splits, rows_cap]
    float* ws_l;     // [units, splits, rows_cap]
    float* ws_acc;   // [units, splits, rows_cap, D]
    int* err;        // device error word
    int B, H, Hkv, group, D, bs;
    // Tokens per block slot the kernel walks (ubs) and slots per cache block (sub = bs / ubs):
    // the vector kernel walks whole blocks (ubs = bs, sub = 1); the MFMA kernels walk 16-token
    // slots, so a block of 16 m tokens is m slots. Slot s of block p, kv head h is the 16 x D
    // slab at element ((p Hkv + h) bs + 16 s) D of a cache.
    int ubs, sub;
    int max_blocks, num_blocks, total_q, max_q_len, rows_cap;
    int causal, out_bf16, dtype_bf16;
    float scale_log2;  // softmax scale * log2(e)
    int splits, chunk_blocks, units;
    int hpw;           // kv heads (units) per workgroup: 2 in the MFMA kernel when Hkv is even
    int ugroups;       // units / hpw
    int ugroups_padded;  // ugroups rounded up to a multiple of 8 (the XCD count)
    int row_groups;    // workgroups per (unit group, split), each covering rows_per_group rows
    int rows_per_group;  // query rows of a row group (MFMA: 16, 32, 64 or 80; vector: 8)
    int stream_kv;     // MFMA kernel: K/V loads with kLoadStream (1), kLoadCached (0) or per unit (kKvPerUnit)
    // Balanced schedule (MFMA kernel, automatic splits): a persistent grid of plan_grid
    // workgroups computes per-sequence splits from the context lengths and walks the work items
    // largest first. Partial states live in per-item slots of plan_rw rows per kv head;
    // plan_seq[b] = {splits, row groups, first slot, 0} tells the combine pass where.
    int plan;
    int plan_grid;
    int plan_rw;
    int plan_max_chunk;
    long long plan_slots;  // partial-state slots in the workspace (plan_slot_bound)
    int4* plan_seq;
    // [B + 1]: the combine pass's work units ((kv head, 8-row chunk) of a split sequence) before
    // sequence b; [B] is their total.
    int* plan_cw;
    // kSchedWords counters, zero at launch: the items claimed on each of the 8 XCD lanes beyond
    // the grid's first items, then the workgroups done; the last workgroup resets them to zero.
    int* sched;
};

constexpr int kSchedWords = 9;

// Sequences one balanced-schedule launch can plan (four per thread of a workgroup).
constexpr int kPlanMaxSeqs = 1024;
// Shortest split the balanced schedule makes, in blocks.
constexpr int kPlanMinChunk = 16;
// A sequence longer than the per-workgroup share L of the work splits into chunks of about
// L x kPlanChunkQuarters / 4 blocks (5L/4: on a batch of log-uniform lengths with a 64-block
// shared prefix, 143.0 us against 145.7 us at 3L/2 and 154.8 us at L, with the claim-free
// assignment the schedule then uses; L/2, 3L/4 and 2L all leave a longer tail).
// plan_slot_bound takes the same count.
#ifndef KYRO_PLAN_CHUNK_QUARTERS
#define KYRO_PLAN_CHUNK_QUARTERS 5
#endif
constexpr int kPlanChunkQuarters = KYRO_PLAN_CHUNK_QUARTERS;

// Balanced-schedule chunk length in blocks, from the total work T (kv head groups x row groups x
// blocks, summed over sequences), the longest sequence maxnb (blocks) and the persistent grid:
// L = ceil(T / grid); C = L when no sequence is longer than L, else ceil(L x quarters / 4); then
// at least kPlanMinChunk, rounded up to even, at most max_chunk (even). The device plan and the
// host checks share this function.
__host__ __device__ inline int plan_chunk_blocks(long long T, int maxnb, int grid, int max_chunk,
                                                 int quarters = kPlanChunkQuarters) {
    const long long L = (T + grid - 1) / grid;
    long long CL = maxnb <= L ? L : (L * quarters + 3) / 4;
    CL = CL < kPlanMinChunk ? kPlanMinChunk : CL;
    CL = (CL + 1) & ~1ll;
    return (int)(CL > max_chunk ? max_chunk : CL);
}

// Splits of a sequence of nb blocks under chunk length C: one split when nb <= C (ch = nb), else
// ns = ceil(nb / C) chunks of ch = C blocks from the start, the last one shorter.
__host__ __device__ inline void plan_split(int nb, int C, int& ns, int& ch) {
    ns = 1;
    ch = nb;
    if (nb > C) {
        ns = (nb + C - 1) / C;
        ch = C;
    }
}

// Upper bound on the partial-state slots of a balanced-schedule launch (one slot per item:
// sequence x kv head group x split x row group). Every split but one per item group is at least
// C >= min(L x quarters / 4, max_chunk) blocks long and the work is at most L x grid blocks, so
// the extra splits number at most ceil(4 x grid / quarters) (or work / max_chunk), plus one per
// (kv head group, row group) of every sequence. The device plan compares its slot total with
// this bound and latches ERR_PLAN instead of writing past it.
__host__ __device__ inline long long plan_slot_bound(long long B, long long ugroups_per_seq, long long row_groups,
                                                     long long max_blocks, long long max_chunk, long long grid,
                                                     int quarters = kPlanChunkQuarters) {
    const long long s = B * ugroups_per_seq * row_groups;
    const long long by_chunk = (s * max_blocks + max_chunk - 1) / max_chunk;
    const long long by_share = (4 * grid + quarters - 1) / quarters;
    return s + (by_chunk > by_share ? by_chunk : by_share);
}

// Block pairs one MFMA wave can hold the ids of (two 64-lane slots). A split has at most
// 2 * kMfmaMaxPairsPerWave * (kernel waves per head) blocks.
constexpr int kMfmaMaxPairsPerWave = 128;

// Head dims the attention kernels take: the vector kernel every multiple of 8 up to
// kMaxHeadDim (X(d) is applied to each), the bf16 MFMA kernel the ones listed below.
constexpr int kMaxHeadDim = 256;
#define KYRO_HEAD_DIMS(X)                                                                           \
    X(8) X(16) X(24) X(32) X(40) X(48) X(56) X(64) X(72) X(80) X(88) X(96) X(104) X(112) X(120)     \
    X(128) X(136) X(144) X(152) X(160) X(168) X(176) X(184) X(192) X(200) X(208) X(216) X(224)      \
    X(232) X(240) X(248) X(256)

// Query rows one attention workgroup covers.
constexpr int kVectorRowsPerGroup = 8;
// MFMA kernels: one 16-row tile, two (32 rows), or for bf16 units of more than 32 rows four
// (kMfmaManyRows: one kv head per workgroup, Q read from LDS, only the unit's tiles computed),
// so that a unit of up to 64 rows streams its K/V once instead of once per 32-row group.
// Five tiles (kMfmaWideRows) where they take fewer row groups than four and the batch's
// average unit (total_rows / seqs rows per kv head) fills more than half of what the last
// 64-row group would hold: GQA 64/8 with 8 drafts on every sequence (72 rows a unit) then
// streams each unit's K/V once instead of twice (B 64, ctx 4096: 331 -> 235 us). The five-tile
// kernel copies about 1.7x as many values through AGPRs per block pair as the four-tile one (both
// hold more than the 256 VGPRs a wave can address), so a batch with few such units keeps four
// (mixed GQA 64/8, 0-8 drafts: 385 us with four, 396 with five).
// Head dims other than 128 take at most two tiles (one at 256: its K/V pairs and accumulators
// fill the register file).
constexpr int kMfmaManyRows = 64;
constexpr int kMfmaWideRows = 80;
inline int mfma_rows_per_group(int rows, bool bf16, int D, long long total_rows, int seqs) {
    if (D > 128) return 16;
    if (rows <= 16) return 16;
    if (rows <= 32 || !bf16 || D != 128) return 32;
    const int groups4 = (rows + kMfmaManyRows - 1) / kMfmaManyRows;
    const int groups5 = (rows + kMfmaWideRows - 1) / kMfmaWideRows;
    const long long lo = (long long)kMfmaManyRows * (groups4 - 1);  // rows before the last 64-row group
    const bool wide = groups5 < groups4 && 2 * total_rows > (long long)seqs * (rows + lo);
    return wide ? kMfmaWideRows : kMfmaManyRows;
}

// Head dims the bf16 MFMA kernel is built for: every multiple of 32 from 64 to 256, and 80 and 112
// in the operand layouts of 96 and 128; f32 caches take it at 128 only.
__host__ __device__ inline bool mfma_head_dim(int D, bool bf16) {
    return D == 128 || (bf16 && ((D % 32 == 0 && D >= 64 && D <= 256) || D == 80 || D == 112));
}

hipError_t launch_paged_attention(const AttnArgs& a, int kernel, hipStream_t stream);
// The bf16 MFMA kernel at head dims 64, 80, 96 and 256, and at 112, 160, 192 and 224 (a
// translation unit each).
hipError_t launch_paged_attention_mfma_hd(const AttnArgs& a, hipStream_t stream);
hipError_t launch_paged_attention_mfma_hd_wide(const AttnArgs& a, hipStream_t stream);

// Per-sequence decision taken after the acceptance scan.
struct SpecPlan {
    int mode;   // SPEC_DONE, SPEC_RESIDUAL (row j of target and draft), SPEC_PLAIN (row j of target)
    int row;    // j
    float mt, inv_zt;  // target row max logit, 1 / sum exp
    float md, inv_zd;  // draft row max logit, 1 / sum exp
    float c2;          // log2(e) / T
    float u;           // u_resample
};

// SPEC_PENDING: no decision within the statistics computed so far (the rows of the first draft
// positions only); the remaining rows are needed.
enum SpecMode : int { SPEC_DONE = 0, SPEC_RESIDUAL = 1, SPEC_PLAIN = 2, SPEC_PENDING = 3 };

struct SpecArgs {
    const float* target;  // [B, kmax+1, V]
    const float* draft;   // [B, kmax, V] or nullptr
    const uint32_t* draft_tokens;
    const int32_t* num_draft;
    const float* temperature;
    const float* u_accept;
    const float* u_res;
    int32_t* out_accepted;
    uint32_t* out_tokens;
    float* out_p;
    float* out_q;
    float2* stats;   // [B, 2 kmax + 1, C]: {max, sum exp} (sampled) or {max, index bits} (greedy)
    SpecPlan* plan;       // [B]: from the window's scan (SPEC_PENDING: see plan_tail)
    SpecPlan* plan_tail;  // [B]: plan of a sequence that was pending, from the full scan
    float2* csum;    // [B, C]: {residual mass, p mass} of the resampled row, per chunk
    float* gath;     // [B, 2 kmax + 1]: logit of the row's draft token (sampled rows < k)
    int2* tail;      // [B]: {items (row x chunk) left after the window, target rows left | greedy << 16}
    int* err;
    int B, kmax, V, C, chunk, vec4;
    int win;          // draft positions whose rows the first statistics pass reads
    int tail_wgs;     // workgroups of the pass over the remaining rows
};

hipError_t launch_spec_verify(const SpecArgs& a, hipStream_t stream);

// Scratch of the allocation-free verify entry point: a static device array per device.
constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;
// The array's device address on `device`, which must be current; resolved once per device.
hipError_t noalloc_scratch(int device, void** out);

struct KvAppendArgs {
    const void* key;         // [total_q, Hkv, D] src dtype
    const void* value;
    const int32_t* q_start;  // [B+1] or nullptr
    const int64_t* table;
    const int64_t* ctx_lens;
    void* kc;                // [num_blocks, Hkv, bs, D] cache dtype
    void* vc;
    int* err;
    int B, Hkv, D, bs, max_blocks, num_blocks, total_q, max_q_len;
    int src_bf16, cache_bf16;
    int vecs_per_row;        // Hkv * D / 8: one thread moves 8 elements of K and of V
};

hipError_t launch_kv_append(const KvAppendArgs& a, hipStream_t stream);

// Whole-block copies within a cache pair (copy-on-write of a prefix block).
constexpr int kCopyInline = 240;  // block pairs passed in the kernel arguments (2 x 240 x 4 B)
struct CopyBlocksArgs {
    const int64_t* pairs;  // [2, n]: sources then destinations; nullptr: in `inl` (n <= kCopyInline)
    int64_t n;
    int64_t slab_vecs;     // 16-byte vectors in one block of one cache
    uint4* kc;
    uint4* vc;
    int32_t inl[2][kCopyInline];
};

hipError_t launch_copy_blocks(const CopyBlocksArgs& a, hipStream_t stream);

// Scatter of up to kMaxUploads staged uploads (8-byte words) from device-mapped host staging.
constexpr int kMaxUploads = 4;
struct UploadArgs {
    const char* src;                 // the staging slot, as the device addresses it
    int n;
    int64_t off[kMaxUploads];        // byte offset of upload u in the slot (8-byte aligned)
    uint64_t* dst[kMaxUploads];
    int64_t words[kMaxUploads];
};

hipError_t launch_upload_scatter(const UploadArgs& a, hipStream_t stream);

// Plain-decode sampling with logit processors.
constexpr int kSampleChunk = 4096;      // vocabulary entries per workgroup of the chunked passes
constexpr int kSampleCand = 8192;       // candidates a row holds in LDS (the chunks' lists together)
constexpr int kSampleChunkCand = 256;   // most candidates one chunk lists
constexpr int kSampleMaxChunks = 1024;  // chunks per row (one per thread of the select pass)

struct SampleArgs {
    const float* logits;        // [B, V]
    float* ws;                  // [B, V] processed rows (rows that have a processor)
    float2* cstat;              // [B, C]: per chunk {max z, sum exp(z - max)} or {max y, index}
    // Top-k / top-p rows: chunk c of row b lists every entry with z >= cthr[b, C + c] (-inf: every
    // finite entry), ccount[b, C + c] of them (-1: no threshold kept the list within ccap), at
    // cand[b, c ccap ...] as (key << 32) | ~index.
    float* cthr;                // [B, C]
    int* ccount;                // [B, C]
    unsigned long long* cand;   // [B, kSampleCand]
    int ccap;                   // list slots per chunk: min(kSampleChunkCand, kSampleCand / C)
    int C;                      // chunks per row
    const float* temperature;   // [B]
    const float* top_p;         // [B] or nullptr (1.0)
    const int32_t* top_k;       // [B] or nullptr (off)
    const float* u;             // [B]
    const int32_t* bias_off;    // [B+1] or nullptr
    const uint32_t* bias_tok;
    const float* bias_val;
    const int32_t* pen_off;     // [B+1] or nullptr
    const uint32_t* pen_tok;
    const float* pen_val;
    const uint32_t* mask;       // [num_masks, mask_words]
    const int32_t* mask_row;    // [B] (-1: no mask) or nullptr
    uint32_t* out;              // [B]
    int* err;
    int B, V, num_masks, mask_words;
    int vec4;                   // rows (logits and workspace) are 16-byte aligned
    // Rows without processors, top-k or top-p: workgroups per row of the one-launch pass (0: the
    // chunked passes), its per-segment statistics [B, ceil(V / 2048)] and the per-row counters
    // (zero between launches).
    int row_wgs;
    float2* segs;
    int* row_cnt;
};

// Rows per launch the one-launch decode pass counts with the context's counters.
constexpr int kSampleRowCounters = 16384;
// The one-launch decode pass: entries per segment (one wave reduces a segment), segments per
// workgroup (one per wave of its 1024 threads) and workgroups per row at most.
#ifndef KYRO_SAMPLE_SEG
#define KYRO_SAMPLE_SEG 2048
#endif
#ifndef KYRO_SAMPLE_ROW_WGS
#define KYRO_SAMPLE_ROW_WGS 8
#endif
constexpr int kSampleSeg = KYRO_SAMPLE_SEG;
constexpr int kSampleSegsPerWg = 16;
constexpr int kSampleRowWgsMax = KYRO_SAMPLE_ROW_WGS;

hipError_t launch_sample(const SampleArgs& a, hipStream_t stream);

// N-gram drafting against an open-addressing table of (order-1)-token keys.
struct NgramArgs {
    const uint32_t* slots;  // [capacity, order]: key tokens then the next token
    const uint8_t* used;    // [capacity]
    uint64_t mask;          // capacity - 1 (a power of two)
    int order;
    const uint32_t* ctx_tail;  // [B, order-1]
    const int64_t* ctx_len;    // [B]
    uint32_t* draft;           // [B, kmax]
    int32_t* num_draft;        // [B]
    int B, kmax;
};

// FNV-1a over the key tokens: the host table and the device lookups must agree.
__host__ __device__ inline uint64_t ngram_hash(const uint32_t* key, int n) {
    uint64_t h = 1469598103934665603ull;
    for (int i = 0; i < n; ++i) {
        h ^= key[i];
        h *= 1099511628211ull;
    }
    return h;
}

hipError_t launch_ngram_draft(const NgramArgs& a, hipStream_t stream);

#ifndef KYRO_SPEC_CHUNK
#define KYRO_SPEC_CHUNK 4096
#endif
constexpr int kSpecChunk = KYRO_SPEC_CHUNK;  // vocabulary entries per workgroup in the streaming passes
constexpr int kMaxDraft = 63;                // one wave holds the acceptance decisions of a sequence
// Draft positions read before the first acceptance scan. With per-position acceptance rate a
// and k drafts, a sequence's rows read are about 2W + a^W (2 (k - W) + 1) (window rows, plus the
// rest when the window is all accepted); W = 3 is the smallest for a between 0.5 and 0.8 at k = 7.
#ifndef KYRO_SPEC_WINDOW
#define KYRO_SPEC_WINDOW 3
#endif
constexpr int kSpecWindow = KYRO_SPEC_WINDOW;
constexpr int kMaxLazyBatch = 2048;  // larger batches read every row in the first pass
// Default window: batches whose logit rows total at most this many bytes read them all in the
// first pass (at ~6 TB/s, 64 MB take about as long as the tail pass's fixed cost).
constexpr long long kSpecEagerBytes = 64ll << 20;
// Workgroups of the pass over the remaining rows (more when one would hold more than 64 items).
// On the Llama-3-8B step (~2,900 pending items) 512 measured 246.1-246.5 us cold against
// 247.3 with 2048, 1024 in between; 384 and 256 were slower (246.6-246.9, 249.5).
#ifndef KYRO_SPEC_TAIL_WGS
#define KYRO_SPEC_TAIL_WGS 512
#endif
constexpr int kSpecTailWgs = KYRO_SPEC_TAIL_WGS;


}  // namespace kyro
