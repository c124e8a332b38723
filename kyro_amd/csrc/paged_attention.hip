// Multi-query paged attention for the verify step on gfx950.
//
// Replaces PagedAttention::forward / paged_attention_kernel (src/model/attention_kernel.rs:22-136)
// for q_len >= 1 query rows per sequence, in the reference's layouts:
//   query [total_q, H, D], caches [num_blocks, Hkv, block_size, D], block_table [B, max_blocks]
//   int64, context_lens [B] int64, out [total_q, H, D].
//
// Work decomposition. One workgroup (4 waves) owns one (sequence, kv head, context split).
// Every query row that reads that kv head — the GQA group x the sequence's q_len rows — is
// processed together, so each K/V byte is read from HBM exactly once. The 4 waves stream disjoint
// blocks of the split with private online-softmax state and merge through LDS at the end; splits
// of one (sequence, kv head) park their partial state in a workspace that attn_combine_kernel
// merges (a kernel boundary orders the two passes; an agent-scope fence per workgroup, which
// writes back the XCD's L2, cost more than the whole second launch).
// Workgroups are numbered so that all splits of one (sequence, kv head) land on one XCD (the
// dispatcher deals workgroups round-robin over the 8 XCDs), keeping that merge in one L2.
//
// Three kernels share that frame:
//  * attn_mfma_kernel (bf16, D = 128, block_size 16): scores S^T = K Q^T and O^T = V^T P^T on
//    v_mfma_f32_16x16x32_bf16. V is loaded with 128-bit loads of 4 full 256-byte token rows per
//    instruction and transposed in registers with v_perm_b32. K is loaded either straight into
//    the MFMA operand layout (16 token rows x 64 contiguous bytes per instruction: the two-tile
//    grid kernel of uniform batches) or by whole token rows straight into a per-wave LDS tile
//    (buffer_load ... lds) and read from there in operand layout (the other instances). A wave
//    holds one or two 16-row tiles with Q in registers; bf16 units of 33 to 64 rows take a
//    four-tile instance instead (one kv head per workgroup, Q staged in LDS, only the tiles
//    that hold the unit's rows computed), so that such a unit streams its K/V once. The softmax'd S^T fragment is already the P^T operand of the PV
//    product, and the output column of O^T is the query row, so the per-row rescale stays in the
//    lane that owns the row's softmax state.
//  * attn_mfma_f32_kernel (f32, D = 128, block_size 16): the same products on
//    v_mfma_f32_16x16x4_f32, one 16-token block per step;
//  * attn_vector_kernel (f32 or bf16, D = 64 or 128, any block size): 16 lanes per token row,
//    4 token rows per wave per step, dot products reduced with DPP inside each 16-lane row.
// Both MFMA kernels run under either schedule: a grid of one workgroup per work item, or the
// balanced schedule, a persistent grid that plans splits from the context lengths on the device.
#include "common.hpp"
#include "kernels.hpp"

namespace kyro {

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;

struct SeqInfo {
    int b, kvh, q0, q_len, rows, nblk;
    int ctx;
    bool ok;
};

// Workgroup -> (unit group, split, row group). A unit is sequence * Hkv + kv head; a group is
// a.hpw consecutive units (kv heads of one sequence). Consecutive workgroups go to different
// XCDs; the splits and row groups of one group share (blockIdx % 8) and therefore one XCD, and a
// group's row groups are dispatched back to back, so the K/V they all read is fetched from HBM
// once and served to the others from that XCD's L2.
__device__ __forceinline__ bool map_workgroup(const AttnArgs& a, int& ugroup, int& split, int& rg) {
    const int wg = blockIdx.x;
    const int xcd = wg & 7;
    const int local = wg >> 3;
    rg = local % a.row_groups;
    const int rest = local / a.row_groups;
    split = rest % a.splits;
    ugroup = (rest / a.splits) * 8 + xcd;
    return ugroup < a.ugroups;
}

__device__ SeqInfo seq_info(const AttnArgs& a, int unit) {
    SeqInfo s;
    s.b = unit / a.Hkv;
    s.kvh = unit % a.Hkv;
    const int64_t ctx = a.ctx_lens[s.b];
    s.ok = true;
    if (ctx < 0 || ctx > (int64_t)a.max_blocks * a.bs) {
        if (threadIdx.x == 0) latch_error(a.err, ERR_CTX_LEN);
        s.ok = false;
    }
    int q0 = s.b, q1 = s.b + 1;
    if (a.q_start) {
        q0 = a.q_start[s.b];
        q1 = a.q_start[s.b + 1];
    }
    if (q0 < 0 || q1 < q0 || q1 > a.total_q || q1 - q0 > a.max_q_len) {
        if (threadIdx.x == 0) latch_error(a.err, ERR_Q_LAYOUT);
        s.ok = false;
    }
    s.ctx = s.ok ? (int)ctx : 0;
    s.q0 = q0;
    s.q_len = s.ok ? q1 - q0 : 0;
    s.rows = s.q_len * a.group;
    s.nblk = (s.ctx + a.ubs - 1) / a.ubs;
    return s;
}

__device__ __forceinline__ int num_splits_for(const AttnArgs& a, int nblk) {
    const int n = (nblk + a.chunk_blocks - 1) / a.chunk_blocks;
    return n < 1 ? 1 : n;
}

// Output row of local row n (n = j * group + head-in-group) of a sequence.
__device__ __forceinline__ size_t out_row(const AttnArgs& a, const SeqInfo& si, int n) {
    const int j = n / a.group;
    const int hg = n - j * a.group;
    return (size_t)(si.q0 + j) * a.H + (size_t)si.kvh * a.group + hg;
}

__device__ __forceinline__ int64_t checked_block(const AttnArgs& a, int b, int i) {
    const int64_t blk = a.table[(size_t)b * a.max_blocks + i];
    if (blk < 0 || blk >= a.num_blocks) {
        latch_error(a.err, ERR_BLOCK_ID);
        return -1;
    }
    return blk;
}

template <int D>
__device__ __forceinline__ void store_row4(const AttnArgs& a, size_t row, int d, float x0, float x1,
                                           float x2, float x3) {
    if (a.out_bf16) {
        uint2 w;
        w.x = pack_bf16x2(x0, x1);
        w.y = pack_bf16x2(x2, x3);
        *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(a.out) + row * D + d) = w;
    } else {
        *reinterpret_cast<float4*>(reinterpret_cast<float*>(a.out) + row * D + d) =
            make_float4(x0, x1, x2, x3);
    }
}

// Shared LDS frame of one workgroup: the merged (unnormalised) accumulator of up to R rows,
// each wave's running max, each wave's rescaled row sums.
template <int R, int D>
struct Frame {
    static constexpr int kStride = D + 4;  // pad rows to spread LDS banks
    float acc[R * kStride];
    float m[kWaves][R];
    float l[kWaves][R];
    float mx[R];
};

// After every wave has added its rescaled accumulator: either normalise and store the rows
// (single split) or park the split's partial state in the workspace, local row n at workspace
// row pbase + n. The frame holds D columns; rows in memory (out, workspace) hold the first DR.
template <int R, int D, int DR = D>
__device__ void frame_flush(const AttnArgs& a, const SeqInfo& si, int nsplit, int row0, int nrows,
                            Frame<R, D>& f, int nslots, size_t pbase) {
    constexpr int Q = DR / 4;
    if (nsplit == 1) {
        for (int idx = threadIdx.x; idx < nrows * Q; idx += kThreads) {
            const int n = idx / Q, d = (idx - n * Q) * 4;
            float L = 0.f;
            for (int w = 0; w < nslots; ++w) L += f.l[w][n];
            const float inv = L > 0.f ? 1.f / L : 0.f;
            const float* src = &f.acc[n * Frame<R, D>::kStride + d];
            store_row4<DR>(a, out_row(a, si, row0 + n), d, src[0] * inv, src[1] * inv, src[2] * inv,
                           src[3] * inv);
        }
        return;
    }
    for (int n = threadIdx.x; n < nrows; n += kThreads) {
        float L = 0.f;
        for (int w = 0; w < nslots; ++w) L += f.l[w][n];
        a.ws_m[pbase + n] = f.mx[n];
        a.ws_l[pbase + n] = L;
    }
    for (int idx = threadIdx.x; idx < nrows * Q; idx += kThreads) {
        const int n = idx / Q, d = (idx - n * Q) * 4;
        const float* src = &f.acc[n * Frame<R, D>::kStride + d];
        *reinterpret_cast<float4*>(a.ws_acc + (pbase + n) * DR + d) = make_float4(src[0], src[1], src[2], src[3]);
    }
}

// Second pass for multi-split units: merges the parked partial states of every split of one
// (sequence, kv head) and writes the normalised rows. The grid is (unit, block of rows): a
// workgroup takes kThreads / (D / 4) rows of one unit, a thread one 4-float column of one row;
// units whose sequence needed a single split were stored directly by the first pass and exit
// here. The split loops are unrolled so that their loads are issued together.
//
// Under the balanced schedule the split count and the slots come from plan_seq (written by the
// first pass): split s of row n (row group n / plan_rw) of kv head h sits in slot
// first + (s * ugroups_per_seq + h / hpw) * row_groups + n / plan_rw, head h % hpw.
// Merges the nsplit partial states of one output row (workspace rows r0 + s * stride) into this
// thread's four columns d .. d + 3 and stores them. The loads of kMergeBatch splits are issued
// together (a split index past the last reads the last split again and is dropped), so a row with
// up to kMergeBatch splits costs one memory round trip; longer rows merge batch after batch with
// the usual running-max rescale (for one batch this is the plain two-pass formula).
constexpr int kMergeBatch = 16;
template <int D>
__device__ __forceinline__ void merge_row(const AttnArgs& a, const SeqInfo& si, int n, int d, size_t r0,
                                          size_t stride, int nsplit) {
    float M = kNegInf, L = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s0 = 0; s0 < nsplit; s0 += kMergeBatch) {
        float m[kMergeBatch], l[kMergeBatch];
        float4 v[kMergeBatch];
#pragma unroll
        for (int i = 0; i < kMergeBatch; ++i) {
            const size_t r = r0 + (size_t)min(s0 + i, nsplit - 1) * stride;
            m[i] = a.ws_m[r];
            l[i] = a.ws_l[r];
            v[i] = *reinterpret_cast<const float4*>(a.ws_acc + r * D + d);
        }
        float mb = M;
#pragma unroll
        for (int i = 0; i < kMergeBatch; ++i) mb = s0 + i < nsplit ? fmaxf(mb, m[i]) : mb;
        if (mb == kNegInf) continue;  // nothing visible so far
        if (M != kNegInf) {
            const float f = fast_exp2(M - mb);
            L *= f;
            acc.x *= f;
            acc.y *= f;
            acc.z *= f;
            acc.w *= f;
        }
        M = mb;
#pragma unroll
        for (int i = 0; i < kMergeBatch; ++i) {
            const float w = s0 + i < nsplit ? fast_exp2(m[i] - M) : 0.f;
            L += w * l[i];
            acc.x += w * v[i].x;
            acc.y += w * v[i].y;
            acc.z += w * v[i].z;
            acc.w += w * v[i].w;
        }
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    store_row4<D>(a, out_row(a, si, n), d, acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
}

// Grid schedule: one workgroup per (unit, RPW rows); every unit has the same split count rule.
template <int D>
__global__ __launch_bounds__(kThreads) void attn_combine_kernel(AttnArgs a) {
    constexpr int Q = D / 4;
    constexpr int RPW = kThreads / Q;  // rows per workgroup
    const int unit = blockIdx.x;
    if (unit >= a.units) return;
    const SeqInfo si = seq_info(a, unit);
    if (!si.ok) return;
    if ((int)threadIdx.x >= RPW * Q) return;  // head dims that do not divide the workgroup
    const int n = blockIdx.y * RPW + (int)threadIdx.x / Q;
    if (n >= si.rows) return;
    const int nsplit = num_splits_for(a, si.nblk);
    if (nsplit <= 1) return;
    merge_row<D>(a, si, n, ((int)threadIdx.x % Q) * 4, (size_t)unit * a.splits * a.rows_cap + n, a.rows_cap,
                 nsplit);
}

// Balanced schedule: the plan lists the combine work, one unit per (kv head, kCombineRows rows)
// of each split sequence, with per-sequence prefix counts in plan_cw. A grid of any size walks
// the list; with nothing split every workgroup reads one word and returns. A row takes 32
// threads, each merging the 4-column groups c, c + 32, .. of the row's D / 4.
constexpr int kCombineRows = kThreads / 32;
template <int D>
__global__ __launch_bounds__(kThreads) void attn_combine_plan_kernel(AttnArgs a) {
    constexpr int Q = D / 4;
    __shared__ int cw[kPlanMaxSeqs + 1];
    const int total = a.plan_cw[a.B];
    if ((int)blockIdx.x >= total) return;
    for (int i = threadIdx.x; i <= a.B; i += kThreads) cw[i] = a.plan_cw[i];
    __syncthreads();
    const int col = (int)threadIdx.x % 32;
    const int upseq = a.ugroups / a.B;
    for (int w = blockIdx.x; w < total; w += gridDim.x) {
        // The last sequence whose work starts at or before w (it has work: see plan_build).
        int lo = 0, hi = a.B - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (cw[mid] <= w) lo = mid;
            else hi = mid - 1;
        }
        SeqInfo si;
        si.b = lo;
        si.q0 = a.q_start ? a.q_start[lo] : lo;
        const int q1 = a.q_start ? a.q_start[lo + 1] : lo + 1;
        const int4 ps = a.plan_seq[lo];
        si.rows = (q1 - si.q0) * a.group;
        const int chunks = (si.rows + kCombineRows - 1) / kCombineRows;
        const int local = w - cw[lo];
        si.kvh = local / chunks;
        const int n = (local - si.kvh * chunks) * kCombineRows + (int)threadIdx.x / 32;
        if (n >= si.rows) continue;
        const int nrg = ps.y, first = ps.z;
        const int rg = n / a.plan_rw;
        const size_t slot = (size_t)first + (size_t)(si.kvh / a.hpw) * nrg + rg;
        for (int c = col; c < Q; c += 32)
            merge_row<D>(a, si, n, 4 * c, (slot * a.hpw + si.kvh % a.hpw) * a.plan_rw + (n - rg * a.plan_rw),
                         (size_t)upseq * nrg * a.hpw * a.plan_rw, ps.x);
    }
}

// ------------------------------------------------------------------------------ MFMA kernel

constexpr int kMfmaD = 128;  // the head dim of the f32 MFMA kernel and of the LDS-staged K forms
constexpr int kMfmaBS = 16;
// One (block, kv head) slab of zeros, read in place of a missing block (static device memory is
// zero-initialised when the code object loads, and nothing writes it).
__device__ uint16_t kZeroSlab[kMfmaBS * kMaxHeadDim];

// K and V of one pair of 16-token blocks, in MFMA operand layout (K: loaded so under kKDirect,
// read from the wave's LDS tile just before the products under kKDma) or ready for the
// in-register transpose (V). With T = D / 16 head dims per lane for V: D / 2 VGPRs (64 at
// D = 128; 32 live across a prefetch under kKDma).
template <int D>
struct KVPair {
    static constexpr int kSteps = D / 32;  // head-dim steps of the S^T product
    static constexpr int kVW = D / 32;     // V words per lane and token (T bf16)
    bf16x8 k[2][kSteps];    // [block][head-dim step]: token r, head dims 32 s + 8 g .. + 7
    uint32_t v[2][4][kVW];  // [block][e]: token 4 g + e, head dims T r .. T r + T - 1
};

// How K reaches the MFMA A-operand layout:
//  * kKDirect: loaded straight into that layout, 16 token rows x 64 bytes per instruction (half
//    lines), which holds one workgroup to ~28 GB/s against ~66 GB/s for whole lines;
//  * kKDma: whole 256-byte token rows per 16 lanes, loaded straight into a per-wave LDS tile
//    (buffer_load ... lds: lane l's 16 bytes land at tile + 16 l) with the source chunk of each
//    lane XOR-swizzled so that the MFMA-layout reads hit distinct banks; one tile per register
//    buffer, so the next pair's K lands while this pair's is read.
// Row loads pay where a workgroup's own rate sets the pace: one 16-row tile (MHA and decode
// shapes) and the balanced schedule's uneven batches. On a uniform batch with two tiles (the
// Llama-3-8B step on the grid) every CU streams at its share of HBM anyway, and the LDS pass
// cost 167.0 -> 169.8 us there, so that kernel loads K directly. KYRO_ATTN_K_GRID2 is the mode
// of the two-tile grid kernel, KYRO_ATTN_K_OTHER that of the others.
enum { kKDirect = 0, kKDma = 1 };
#ifndef KYRO_ATTN_K_GRID2
#define KYRO_ATTN_K_GRID2 0
#endif
#ifndef KYRO_ATTN_K_OTHER
#define KYRO_ATTN_K_OTHER 1
#endif
template <int NTW, bool PLAN>
constexpr int kKModeFor = NTW > 2 ? kKDma : (NTW == 1 || PLAN) ? KYRO_ATTN_K_OTHER : KYRO_ATTN_K_GRID2;

// Issues the 16 loads of one block pair. A negative block id reads as zeros (never dereferenced).
// Word 3 of a raw buffer resource on gfx9-family parts (32-bit data format, no swizzle).
constexpr int kRawBufferWord3 = 0x00020000;

// Loads the K and V operands of a pair of blocks (block ids uniform across the wave; -1 for a
// missing block: past the split, or a bad id). Each (block, kv head) slab is read through a
// buffer resource with fixed per-lane offsets, and a missing block reads the zero slab: the
// addresses are scalar and the loads are issued without a branch, so the loop's waits can leave
// a prefetched pair in flight. POL is the loads' cache policy (kLoadCached or kLoadStream).
//
// D is the operand layout (a multiple of 32) and DR the head dim of the cache rows (DR <= D, a
// multiple of 8): with DR < D the layout's last head-dim slots are padding. K slots past DR read
// as zeros (an offset beyond the slab, which the range check answers with zeros), so padded dims
// add nothing to S = K Q^T whatever the slab holds; V loads there read the next token's row or
// zeros, which only reach the padded output dims, never stored.
template <int POL, int KM, int D, int DR = D>
__device__ __forceinline__ void load_pair(KVPair<D>& p, uint4* __restrict__ kt, const uint16_t* __restrict__ kp,
                                          const uint16_t* __restrict__ vp, int blk0, int blk1,
                                          size_t slot_stride, size_t kv_off, int r, int g) {
    static_assert(KM != kKDma || (D == kMfmaD && DR == D), "the LDS-staged K tiles hold 256-byte token rows");
    constexpr int kSlabBytes = kMfmaBS * DR * 2;
    constexpr int T = D / 16;
    const int koff = (r * DR + 8 * g) * 2;       // bytes; + 64 s for head-dim slot s
    const int voff = (4 * g * DR + T * r) * 2;   // bytes; + 2 DR e for token 4 g + e
    constexpr int kPastSlab = 1 << 28;           // any offset at or past kSlabBytes reads zeros
    __amdgpu_buffer_rsrc_t kr[2], vr[2];
#pragma unroll
    for (int bi = 0; bi < 2; ++bi) {
        const int blk = bi ? blk1 : blk0;
        const size_t base = (size_t)(blk >= 0 ? blk : 0) * slot_stride + kv_off;
        const uint16_t* kslab = blk >= 0 ? kp + base : kZeroSlab;
        const uint16_t* vslab = blk >= 0 ? vp + base : kZeroSlab;
        kr[bi] = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(kslab), (short)0, kSlabBytes, kRawBufferWord3);
        vr[bi] = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(vslab), (short)0, kSlabBytes, kRawBufferWord3);
    }
    // K of both blocks first: the computation of this pair starts with K (S = K Q^T) while the
    // V loads may still be in flight.
#pragma unroll
    for (int bi = 0; bi < 2; ++bi) {
        if constexpr (KM == kKDma) {
            // Instruction e: tokens 4 e .. 4 e + 3, lane (r, g) -> LDS slot r of token t = 4 e + g,
            // which holds the token's 16-byte chunk r ^ t.
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int t = 4 * e + g;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    kr[bi], (__attribute__((address_space(3))) void*)(kt + bi * 256 + e * 64), 16,
                    t * 256 + 16 * (r ^ t), 0, 0, POL);
            }
        } else {
#pragma unroll
            for (int s = 0; s < KVPair<D>::kSteps; ++s) {
                const int off = (DR < D && 32 * s + 8 * g >= DR) ? kPastSlab : koff;
                p.k[bi][s] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(kr[bi], off, 64 * s, POL));
            }
        }
    }
    // V: T consecutive bf16 of one token row per lane (16 bytes at D = 128, 8 at 64, 12 at 96,
    // 32 at 256; 20, 24 and 28 at 160, 192 and 224), in 16-byte loads and one narrower load for
    // the rest (the offsets are 4-byte aligned, which buffer loads of several dwords accept).
    constexpr int kVW = KVPair<D>::kVW;
    constexpr int kV4 = kVW / 4 * 4;  // words loaded 16 bytes at a time
#pragma unroll
    for (int bi = 0; bi < 2; ++bi)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            uint32_t* w = p.v[bi][e];
#pragma unroll
            for (int q = 0; q < kV4; q += 4) {
                const auto x = __builtin_amdgcn_raw_buffer_load_b128(vr[bi], voff, 2 * DR * e + 4 * q, POL);
                w[q] = x[0];
                w[q + 1] = x[1];
                w[q + 2] = x[2];
                w[q + 3] = x[3];
            }
            if constexpr (kVW - kV4 == 3) {
                const auto x = __builtin_amdgcn_raw_buffer_load_b96(vr[bi], voff, 2 * DR * e + 4 * kV4, POL);
                w[kV4] = x[0];
                w[kV4 + 1] = x[1];
                w[kV4 + 2] = x[2];
            } else if constexpr (kVW - kV4 == 2) {
                const auto x = __builtin_amdgcn_raw_buffer_load_b64(vr[bi], voff, 2 * DR * e + 4 * kV4, POL);
                w[kV4] = x[0];
                w[kV4 + 1] = x[1];
            } else if constexpr (kVW - kV4 == 1) {
                w[kV4] = __builtin_amdgcn_raw_buffer_load_b32(vr[bi], voff, 2 * DR * e + 4 * kV4, POL);
            }
        }
}

// One wave's LDS tile for the K of one block pair: [block][token][16-byte chunk], the chunk
// index XOR-ed with the token so that the MFMA-layout reads (16 tokens, one chunk each) fall in
// distinct banks.
constexpr int kKStageChunks = 2 * kMfmaBS * (kMfmaD / 8);  // uint4 per wave (8 KiB)
// Staged Q rows of the many-tile kernels: 16 uint4 per row plus one of padding, so that the 16
// rows one MFMA operand read touches start 4 banks apart.
constexpr int kQStride = kMfmaD / 8 + 1;

// K of a pair in MFMA A-operand layout (register s: token r, chunk 4 s + g) from a swizzled tile
// (token t's chunk c at slot c ^ t). The tile belongs to the calling wave alone.
__device__ __forceinline__ void read_k_tile(KVPair<kMfmaD>& p, const uint4* __restrict__ tile, int r, int g) {
#pragma unroll
    for (int bi = 0; bi < 2; ++bi)
#pragma unroll
        for (int s = 0; s < 4; ++s) p.k[bi][s] = __builtin_bit_cast(bf16x8, tile[bi * 256 + r * 16 + ((4 * s + g) ^ r)]);
}

// Stages the 16-token slots [blk_begin, blk_end) of the workgroup's split in LDS, validated once,
// so the streaming loop never waits on a table load before issuing K/V loads. Slot i is slot
// i % sub of block table[i / sub]; it is staged as p Hkv sub + i % sub (-1 for a bad id), the
// index of its kv-head-0 slab in units of one 16 x D slab, so that the slab of kv head h starts
// at element (id x 16 D + h bs D) of a cache.
__device__ __forceinline__ void stage_block_ids(const AttnArgs& a, const SeqInfo& si, int blk_begin,
                                                int blk_end, int* s_blk) {
    for (int i = blk_begin + (int)threadIdx.x; i < blk_end; i += kThreads) {
        const int q = i / a.sub;
        const int64_t blk = checked_block(a, si.b, q);
        s_blk[i - blk_begin] = blk < 0 ? -1 : (int)blk * a.Hkv * a.sub + (i - q * a.sub);
    }
    __syncthreads();
}

// ------------------------------------------------------------------------ balanced schedule
//
// Under automatic splits every workgroup of the MFMA launch reads all context lengths and derives
// the same plan in LDS (no extra launch and no host round trip):
//  * work of sequence b: W_b = kv head groups x row groups x blocks; per-workgroup share
//    L = ceil(sum W / grid);
//  * chunk C = L when no sequence is longer than L (nothing splits, so a uniform batch keeps one
//    item per (sequence, kv head group)), else ceil(L x kPlanChunkQuarters / 4) (5L / 4), within
//    [kPlanMinChunk, max chunk];
//  * a longer sequence splits into chunks of C blocks from its start, the last one shorter;
//  * item groups (sequence, chunk, kv head group) come in two phases: first every chunk but the
//    last of each split sequence (all C blocks long), then the last chunk of every sequence (for
//    an unsplit sequence its only chunk), ordered by length, longest first. Greedy claiming then
//    runs largest-first over single items rather than whole sequences: the short last chunks and
//    short sequences fill in at the end, which measured shorter tails than splitting each
//    sequence into equal chunks ordered by sequence;
//  * item groups are dealt to 8 lanes, one per XCD, in a snake (lanes 0..7, then 7..0), which
//    keeps the lanes' totals even; the row groups of an item group take consecutive positions of
//    one lane, so they run together on one XCD and share its L2;
//  * a workgroup takes one item of its XCD's lane at a time: first item w / 8; then, when the
//    lane has at most two items per workgroup, item 2 nw - 1 - w / 8 (nw workgroups a lane: the
//    largest of the rest go to the smallest first items, no claims); otherwise the next
//    unclaimed one (a counter per lane), so the workgroups of an XCD share its lane's items
//    greedily, largest first. Each workgroup keeps only its own lane's item counts.
struct PlanLds {
    alignas(16) uint32_t key[kPlanMaxSeqs];  // by sequence: (last chunk << 16) | (0xffff - b); larger first
    // By sequence:
    int ns[kPlanMaxSeqs];      // splits (0: no rows)
    int r[kPlanMaxSeqs];       // row groups
    int ctx[kPlanMaxSeqs];
    int q0[kPlanMaxSeqs];
    int qlen[kPlanMaxSeqs];
    int gA[kPlanMaxSeqs];      // first phase-A item group
    int slot0[kPlanMaxSeqs];   // first partial-state slot
    int lane0A[kPlanMaxSeqs];  // this lane's phase-A items of earlier sequences
    // By phase-B position (last chunks, longest first):
    int bB[kPlanMaxSeqs];      // sequence
    int lane0B[kPlanMaxSeqs];  // this lane's items before the position (phase A included)
    int lenA, len;             // this lane's phase-A items, all its items
    int GA;                    // phase-A item groups (all lanes)
    int C;                     // chunk length, blocks
    int red[kWaves][9];
    long long red64[kWaves];
};
static_assert(kPlanMaxSeqs % kThreads == 0, "plan_build reads kPlanMaxSeqs / kThreads sequences per thread");

// Item group g goes to lane snake_lane(g): lanes 0..7 in even rounds of 8 groups and 7..0 in odd
// ones, so that with groups sorted largest first no lane always gets the larger of each round.
__device__ __forceinline__ int snake_pos(int r, int x) { return (r & 1) ? 7 - x : x; }

// Number of groups g in [A, A + n) on lane x.
__device__ __forceinline__ int snake_count(int A, int n, int x) {
    if (n <= 0) return 0;
    const int r0 = A >> 3, r1 = (A + n - 1) >> 3;
    int c = max(0, r1 - r0 - 1);
    const int first = 8 * r0 + snake_pos(r0, x);
    c += (first >= A && first < A + n) ? 1 : 0;
    if (r1 > r0) c += (8 * r1 + snake_pos(r1, x) < A + n) ? 1 : 0;
    return c;
}

// The i-th group (from 0) of [A, A + n) on lane x.
__device__ __forceinline__ int snake_nth(int A, int x, int i) {
    const int r0 = A >> 3;
    const int r = (8 * r0 + snake_pos(r0, x) >= A ? r0 : r0 + 1) + i;
    return 8 * r + snake_pos(r, x);
}

// Inclusive prefix sum over a wave's 64 lanes: row_shr 1, 2, 4, 8 within each row of 16 lanes,
// then row_bcast 15 (row 0's total into row 1, row 2's into row 3) and row_bcast 31 (the first
// two rows' total into rows 2 and 3). Lanes a DPP source does not reach add 0.
__device__ __forceinline__ int wave_incl_sum(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15, rows 1 and 3
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31, rows 2 and 3
    return x;
}

// Exclusive prefix sums of V values per thread over the workgroup's threads; total[] gets the
// sums. `red` is LDS scratch.
template <int V>
__device__ __forceinline__ void block_scan_excl(int (&v)[V], int (&total)[V], int (*red)[9]) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int incl[V];
#pragma unroll
    for (int j = 0; j < V; ++j) incl[j] = wave_incl_sum(v[j]);
    if (lane == 63) {
#pragma unroll
        for (int j = 0; j < V; ++j) red[wave][j] = incl[j];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < V; ++j) {
        int before = 0, tot = 0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            before += w < wave ? red[w][j] : 0;
            tot += red[w][j];
        }
        v[j] = incl[j] - v[j] + before;
        total[j] = tot;
    }
    __syncthreads();
}

// Local exclusive prefix of V values over a thread's S consecutive entries, then the block scan
// of the thread totals: v[j][k] becomes the exclusive prefix of entry j in the workgroup's order,
// total[k] the sum of all.
template <int S, int V>
__device__ __forceinline__ void scan_owned(int (&v)[S][V], int (&total)[V], int (*red)[9]) {
    int run[V];
#pragma unroll
    for (int k = 0; k < V; ++k) run[k] = 0;
#pragma unroll
    for (int j = 0; j < S; ++j)
#pragma unroll
        for (int k = 0; k < V; ++k) {
            const int x = v[j][k];
            v[j][k] = run[k];
            run[k] += x;
        }
    block_scan_excl<V>(run, total, red);
#pragma unroll
    for (int j = 0; j < S; ++j)
#pragma unroll
        for (int k = 0; k < V; ++k) v[j][k] += run[k];
}

// Builds the plan (every thread of the workgroup takes part; thread t owns sequences and
// phase-B positions S t .. S t + S - 1, S = kPlanMaxSeqs / kThreads). Workgroup 0 latches input
// errors and publishes {splits, row groups, first slot} per sequence and the combine pass's work
// list.
template <int RW, int HP>
__device__ void plan_build(const AttnArgs& a, PlanLds& P) {
    constexpr int S = kPlanMaxSeqs / kThreads;
    const int t = threadIdx.x;
    const int wave = t >> 6;
    const int x = (int)blockIdx.x & 7;  // this workgroup's lane
    const int U = a.Hkv / HP;
    // Context lengths and rows, read coalesced (thread t: sequences t, t + kThreads, ..) into LDS.
    long long w = 0;
    int mx = 0;
#pragma unroll
    for (int j = 0; j < S; ++j) {
        const int sq = t + j * kThreads;
        if (sq < a.B) {
            const int64_t c = a.ctx_lens[sq];
            int s0 = sq, s1 = sq + 1;
            if (a.q_start) {
                s0 = a.q_start[sq];
                s1 = a.q_start[sq + 1];
            }
            bool ok = true;
            if (c < 0 || c > (int64_t)a.max_blocks * a.bs) {
                ok = false;
                if (blockIdx.x == 0) latch_error(a.err, ERR_CTX_LEN);
            }
            if (s0 < 0 || s1 < s0 || s1 > a.total_q || s1 - s0 > a.max_q_len) {
                ok = false;
                if (blockIdx.x == 0) latch_error(a.err, ERR_Q_LAYOUT);
            }
            const int ctx = ok ? (int)c : 0;
            const int ql = ok ? s1 - s0 : 0;
            const int r = (ql * a.group + RW - 1) / RW;
            const int nb = (ctx + a.ubs - 1) / a.ubs;
            P.ctx[sq] = ctx;
            P.q0[sq] = ok ? s0 : 0;
            P.qlen[sq] = ql;
            P.r[sq] = r;
            w += (long long)U * r * nb;  // total work and the longest sequence that has rows
            mx = max(mx, r > 0 ? nb : 0);
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        w += __shfl_xor(w, o, 64);
        mx = max(mx, __shfl_xor(mx, o, 64));
    }
    if ((t & 63) == 0) {
        P.red64[wave] = w;
        P.red[wave][0] = mx;
    }
    __syncthreads();
    long long T = 0;
    int maxnb = 0;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) {
        T += P.red64[i];
        maxnb = max(maxnb, P.red[i][0]);
    }
    const int C = plan_chunk_blocks(T, maxnb, a.plan_grid, a.plan_max_chunk);
    // Thread t owns sequences S t .. S t + S - 1 from here on. Per sequence: splits, phase-A item
    // groups, partial-state slots and the combine pass's work units (kCombineRows-row chunks of
    // every kv head of a split sequence), prefix-summed in sequence order.
    int r[S], ns[S], v3[S][3], t3[3];
#pragma unroll
    for (int j = 0; j < S; ++j) {
        const int sq = S * t + j;
        r[j] = sq < a.B ? P.r[sq] : 0;
        const int nb = sq < a.B ? (P.ctx[sq] + a.ubs - 1) / a.ubs : 0;
        const int ql = sq < a.B ? P.qlen[sq] : 0;
        int n, ch;
        plan_split(nb, C, n, ch);
        ns[j] = r[j] > 0 ? n : 0;
        const int last = nb - (n - 1) * C;  // blocks of the last chunk
        // Unique per sequence (a sequence without rows sorts last); padding ranks below all.
        P.key[sq] = sq < a.B ? ((uint32_t)(r[j] > 0 ? last : 0) << 16) | (uint32_t)(0xffff - sq) : 0u;
        v3[j][0] = r[j] > 0 ? (n - 1) * U : 0;
        v3[j][1] = ns[j] * U * r[j];
        v3[j][2] = ns[j] > 1 ? a.Hkv * ((ql * a.group + kCombineRows - 1) / kCombineRows) : 0;
    }
    scan_owned<S, 3>(v3, t3, P.red);  // its barriers also publish P.key
    if (t3[1] > a.plan_slots) {
        // More partial-state slots than the workspace holds: a plan/bound mismatch. Latch it and
        // run no item (every workgroup derives the same totals, so all of them skip the walk and
        // still count themselves done); the combine pass sees no work.
        if (t == 0) P.len = P.lenA = 0;
        for (int sq = t; sq < a.B; sq += kThreads)
            if (blockIdx.x == 0) a.plan_seq[sq] = make_int4(0, 0, 0, 0);
        if (blockIdx.x == 0 && t == 0) {
            a.plan_cw[a.B] = 0;
            latch_error(a.err, ERR_PLAN);
        }
        __syncthreads();
        return;
    }
    const int GA = t3[0];
#pragma unroll
    for (int j = 0; j < S; ++j) {
        const int sq = S * t + j;
        if (sq < a.B) {
            P.ns[sq] = ns[j];
            P.gA[sq] = v3[j][0];
            P.slot0[sq] = v3[j][1];
            if (blockIdx.x == 0) {
                a.plan_seq[sq] = make_int4(ns[j], r[j], v3[j][1], 0);
                a.plan_cw[sq] = v3[j][2];
            }
        }
    }
    if (blockIdx.x == 0 && t == 0) a.plan_cw[a.B] = t3[2];
    // Phase-B order: up to kThreads sequences by last chunk, longest first (rank = count of
    // larger keys, four keys per LDS read); larger batches keep their order.
    for (int sq = t; sq < a.B; sq += kThreads) {
        int rank = sq;
        if (a.B <= kThreads) {
            const uint32_t key = P.key[sq];
            rank = 0;
            const uint4* k4 = reinterpret_cast<const uint4*>(P.key);
#pragma unroll 4
            for (int i = 0; i < (a.B + 3) / 4; ++i) {
                const uint4 k = k4[i];
                rank += (k.x > key ? 1 : 0) + (k.y > key ? 1 : 0) + (k.z > key ? 1 : 0) + (k.w > key ? 1 : 0);
            }
        }
        P.bB[rank] = sq;
    }
    __syncthreads();
    // This lane's items: phase A per sequence (its groups from gA on), phase B per position (U
    // groups each, from GA + U p on); the row groups of a group are consecutive.
    int c2[S][2], t2[2];
#pragma unroll
    for (int j = 0; j < S; ++j) {
        const int i = S * t + j;
        c2[j][0] = snake_count(v3[j][0], r[j] > 0 ? (ns[j] - 1) * U : 0, x) * r[j];
        c2[j][1] = i < a.B ? snake_count(GA + U * i, U, x) * P.r[P.bB[i]] : 0;
    }
    scan_owned<S, 2>(c2, t2, P.red);
#pragma unroll
    for (int j = 0; j < S; ++j) {
        const int i = S * t + j;
        if (i < a.B) {
            P.lane0A[i] = c2[j][0];
            P.lane0B[i] = t2[0] + c2[j][1];
        }
    }
    if (t == 0) {
        P.lenA = t2[0];
        P.len = t2[0] + t2[1];
        P.GA = GA;
        P.C = C;
    }
    __syncthreads();
}

struct PlanItem {
    int b;      // sequence
    int hp;     // kv head group within the sequence
    int rg;     // row group
    int chunk;  // split
    int slot;   // partial-state slot
};

// The k-th item of this workgroup's lane, or false past the lane's last item.
template <int HP>
__device__ __forceinline__ bool plan_item(const AttnArgs& a, const PlanLds& P, int k, PlanItem& it) {
    if (k >= P.len) return false;
    const int x = (int)blockIdx.x & 7;
    const int U = a.Hkv / HP;
    int b, g0, idx, c0;
    // The last entry whose items start at or before k (it has items: an entry without any shares
    // its start with the next one).
    int lo = 0, hi = a.B - 1;
    if (k < P.lenA) {
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (P.lane0A[mid] <= k) lo = mid;
            else hi = mid - 1;
        }
        b = lo;
        g0 = P.gA[b];
        idx = k - P.lane0A[b];
        c0 = 0;
    } else {
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (P.lane0B[mid] <= k) lo = mid;
            else hi = mid - 1;
        }
        b = P.bB[lo];
        g0 = P.GA + U * lo;
        idx = k - P.lane0B[lo];
        c0 = P.ns[b] - 1;
    }
    const int rr = P.r[b];
    const int igl = idx / rr;
    const int q = snake_nth(g0, x, igl) - g0;  // item group within the entry
    it.b = b;
    it.rg = idx - igl * rr;
    it.chunk = c0 + q / U;
    it.hp = q - (q / U) * U;
    it.slot = P.slot0[b] + (it.chunk * U + it.hp) * rr + it.rg;
    return true;
}

// A workgroup covers NTW 16-row tiles of its unit's rows (NTW 1 or 2: the accumulators of two
// tiles plus two K/V pair buffers fill the register file without spills); units with more rows
// (a large GQA group times many draft positions) get one workgroup per 32-row group.
//
// With HP = 2 a workgroup takes two adjacent kv heads of the sequence, two waves each: the
// workgroup then reads both heads' slabs of each block together (8 KiB contiguous of K and of
// V), and a batch with 2 x 256 units runs as one round of workgroups on 256 CUs instead of two.
// POL is the cache policy of the K/V loads: kLoadStream when no other workgroup reads the same
// slabs (the host decides), kLoadCached otherwise, or kLoadPerUnit: streaming for units whose
// rows fit one row group, cached for the others (their row groups share the slabs in L2).
//
// mfma_item runs one work item: kv head group ug of sequence si.b (si describes this wave's kv
// head), row group rg, blocks [blk_begin, blk_end) of nsplit; partial states (nsplit > 1) go to
// workspace rows pb0 + h * pbstep + n for head h of the group. D is the operand layout and DR
// the head dim of query, cache and output rows (load_pair).
template <int NTW, int HP, int POL, int KM, int D, int DR = D>
__device__ __forceinline__ void mfma_item(const AttnArgs& a, Frame<NTW * 16, D> (&frame)[HP], int* s_blk,
                                          uint4* kstA, uint4* kstB, uint4* sq, const SeqInfo& si, int ug, int rg,
                                          int blk_begin, int blk_end, int nsplit, size_t pb0, size_t pbstep) {
    static_assert(D % 32 == 0 && D <= kMaxHeadDim, "the bf16 MFMA kernel's operand layout is a multiple of 32");
    static_assert(DR % 8 == 0 && DR <= D && DR > D - 32, "cache rows fill the layout's last 32-dim step in part");
    constexpr int RW = NTW * 16;      // rows of one wave (one tile group)
    constexpr int KS = D / 32;        // head-dim steps of S^T = K Q^T
    constexpr int T = D / 16;         // d-tiles of O^T (lane row r <-> head dims T r + dt)
    constexpr int WPH = kWaves / HP;  // waves per kv head
    // More than two tiles: Q is read from LDS per tile (sq, staged once per item) and only the
    // tiles that hold rows of this unit are computed.
    constexpr bool QL = NTW > 2;
    static_assert(!QL || (HP == 1 && KM == kKDma && D == kMfmaD && DR == D),
                  "the many-tile form needs one kv head and K in LDS");
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform by construction
    const int hw = wave / WPH;  // this wave's kv head within the group
    const int wp = wave % WPH;  // and its place among that head's waves
    const int row0 = rg * RW;

    const int lane = threadIdx.x & 63;
    const int r = lane & 15;  // MFMA row/column within a 16-tile
    const int g = lane >> 4;  // 16-lane group
    const uint16_t* __restrict__ qp = reinterpret_cast<const uint16_t*>(a.q);
    const uint16_t* __restrict__ kp = reinterpret_cast<const uint16_t*>(a.k);
    const uint16_t* __restrict__ vp = reinterpret_cast<const uint16_t*>(a.v);
    const size_t slot_stride = (size_t)kMfmaBS * DR;          // one (slot, kv head) slab
    const size_t kv_off = (size_t)si.kvh * a.bs * DR;          // kv head si.kvh within a block
    const float c = a.scale_log2;
    // Tokens below full_vis are visible to every query row of the sequence.
    const int full_vis = a.causal ? si.ctx - si.q_len + 1 : si.ctx;
    // Row tiles of this row group that hold rows of the unit (uniform).
    const int ntile = QL ? min(NTW, (min(RW, si.rows - row0) + 15) / 16) : NTW;

    if constexpr (QL) {
        // The row group's Q rows, one padded 272-byte row each (rows past the unit are zero).
        // The previous item's readers are past the frame merge's barriers.
        for (int idx = threadIdx.x; idx < RW * 16; idx += kThreads) {
            const int n = idx >> 4, ch = idx & 15;
            uint4 v = make_uint4(0, 0, 0, 0);
            if (row0 + n < si.rows) v = load16(qp + out_row(a, si, row0 + n) * D + 8 * ch);
            sq[n * kQStride + ch] = v;
        }
    }
    stage_block_ids(a, si, blk_begin, blk_end, s_blk);  // its barrier also publishes sq

    {
        // Q^T operands: lane holds row n = row0 + 16 nt + r, head-dim slots 32 s + 8 g .. + 7.
        // Padding rows (n >= rows) get Q = 0 and full visibility; they are never stored.
        bf16x8 qB[QL ? 1 : NTW][KS];
        int vis[NTW];
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt) {
            const int n = row0 + nt * 16 + r;
            if (n < si.rows) {
                const int j = n / a.group;
                if constexpr (!QL) {
                    const size_t qrow = out_row(a, si, n);
#pragma unroll
                    for (int s = 0; s < KS; ++s)
                        qB[nt][s] = __builtin_bit_cast(bf16x8, (DR < D && 32 * s + 8 * g >= DR)
                                                                   ? make_uint4(0, 0, 0, 0)
                                                                   : load16(qp + qrow * DR + 32 * s + 8 * g));
                }
                vis[nt] = a.causal ? si.ctx - si.q_len + j + 1 : si.ctx;
            } else {
                if constexpr (!QL) {
#pragma unroll
                    for (int s = 0; s < KS; ++s) qB[nt][s] = __builtin_bit_cast(bf16x8, make_uint4(0, 0, 0, 0));
                }
                vis[nt] = si.ctx;
            }
        }

        float m[NTW], lsum[NTW];  // running max (log2 units, scaled) and this lane's partial sum
        f32x4 O[T][NTW];
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt) {
            m[nt] = kNegInf;
            lsum[nt] = 0.f;
#pragma unroll
            for (int dt = 0; dt < T; ++dt) O[dt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
        }

        // Online softmax of row tile nt over one pair (S^T fragments s0, s1 of its two blocks):
        // updates the tile's running max and sum, rescales its accumulator when the max rose, and
        // returns P^T as the B operand of the PV product.
        auto softmax_tile = [&](int nt, const f32x4& s0, const f32x4& s1, bool full, int pb, int blk0,
                                int blk1) -> bf16x8 {
            float sv[8];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                sv[e] = s0[e];
                sv[4 + e] = s1[e];
            }
            if (!full) {
#pragma unroll
                for (int bi = 0; bi < 2; ++bi)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int t = (pb + bi) * kMfmaBS + 4 * g + e;
                        const bool ok = (bi ? blk1 : blk0) >= 0 && t < vis[nt];
                        if (!ok) sv[bi * 4 + e] = kNegInf;
                    }
            }
            float mx = sv[0];
#pragma unroll
            for (int i = 1; i < 8; ++i) mx = fmaxf(mx, sv[i]);
            mx = max_over_rows(mx);
            const float m_new = fmaxf(m[nt], mx * c);
            const float mref = (m_new == kNegInf) ? 0.f : m_new;
            const float alpha = fast_exp2(m[nt] - mref);
            float ps = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                sv[i] = fast_exp2(__builtin_fmaf(sv[i], c, -mref));
                ps += sv[i];
            }
            lsum[nt] = lsum[nt] * alpha + ps;
            if (__any(m_new > m[nt] && m[nt] != kNegInf)) {
#pragma unroll
                for (int dt = 0; dt < T; ++dt) O[dt][nt] *= alpha;
            }
            m[nt] = m_new;
            uint4 pw;
            pw.x = pack_bf16x2(sv[0], sv[1]);
            pw.y = pack_bf16x2(sv[2], sv[3]);
            pw.z = pack_bf16x2(sv[4], sv[5]);
            pw.w = pack_bf16x2(sv[6], sv[7]);
            return __builtin_bit_cast(bf16x8, pw);
        };
        // V^T operand of d-tile dt: lane row r <-> head dim T r + dt, k-slots 8 g .. 8 g + 7 <->
        // tokens 4 g .. 4 g + 3 of block 0 then of block 1.
        auto v_operand = [&](const KVPair<D>& kv, int dt) -> bf16x8 {
            const uint32_t sel = (dt & 1) ? 0x07060302u : 0x05040100u;
            const int w = dt >> 1;
            uint4 av;
            av.x = __builtin_amdgcn_perm(kv.v[0][1][w], kv.v[0][0][w], sel);
            av.y = __builtin_amdgcn_perm(kv.v[0][3][w], kv.v[0][2][w], sel);
            av.z = __builtin_amdgcn_perm(kv.v[1][1][w], kv.v[1][0][w], sel);
            av.w = __builtin_amdgcn_perm(kv.v[1][3][w], kv.v[1][2][w], sel);
            return __builtin_bit_cast(bf16x8, av);
        };

        // One pair of blocks = 32 tokens = one K-step of the PV MFMA.
        // The wave's K tiles under kKDma, one per register buffer.
        uint4* const ktA = KM == kKDma ? kstA + wave * kKStageChunks : kstA;
        uint4* const ktB = KM == kKDma ? kstB + wave * kKStageChunks : kstB;
        auto compute = [&](KVPair<D>& kv, const uint4* kt, int pb, int blk0, int blk1) {
            if constexpr (KM == kKDma) {
                // Keep the next pair's loads (issued just before) ahead of this pair's tile
                // reads, which then wait for this pair's K only; without the barrier the
                // compiler hoists the reads above the loads and the prefetch is lost.
                __builtin_amdgcn_sched_barrier(0);
                read_k_tile(kv, kt, r, g);
            }
            const bool full = blk0 >= 0 && blk1 >= 0 && (pb + 2) * kMfmaBS <= full_vis;
            if constexpr (QL) {
                if (!full) {  // as below: V of tokens past the context is zeroed
#pragma unroll
                    for (int bi = 0; bi < 2; ++bi)
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if ((pb + bi) * kMfmaBS + 4 * g + e >= si.ctx)
#pragma unroll
                                for (int q = 0; q < KVPair<D>::kVW; ++q) kv.v[bi][e][q] = 0u;
                }
#pragma unroll
                for (int nt = 0; nt < NTW; ++nt) {
                    if (nt < ntile) {  // uniform: tiles past the unit's rows are skipped
                        bf16x8 q[4];
#pragma unroll
                        for (int s = 0; s < 4; ++s)
                            q[s] = __builtin_bit_cast(bf16x8, sq[(nt * 16 + r) * kQStride + 4 * s + g]);
                        f32x4 S2[2];
#pragma unroll
                        for (int bi = 0; bi < 2; ++bi) {
                            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                            for (int s = 0; s < KS; ++s)
                                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kv.k[bi][s], q[s], acc, 0, 0, 0);
                            S2[bi] = acc;
                        }
                        const bf16x8 pB = softmax_tile(nt, S2[0], S2[1], full, pb, blk0, blk1);
                        // The V^T operands are written per tile; the compiler builds the eight once
                        // per block pair and keeps them for the other tiles (32 registers).
#pragma unroll
                        for (int dt = 0; dt < T; ++dt)
                            O[dt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v_operand(kv, dt), pB, O[dt][nt], 0, 0, 0);
                    }
                }
                return;
            }
            // S^T tiles: rows = 16 tokens of block bi, columns = 16 query rows of tile nt.
            f32x4 S[2][NTW];
#pragma unroll
            for (int bi = 0; bi < 2; ++bi)
#pragma unroll
                for (int nt = 0; nt < NTW; ++nt) {
                    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int s = 0; s < KS; ++s)
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kv.k[bi][s], qB[nt][s], acc, 0, 0, 0);
                    S[bi][nt] = acc;
                }
            if (!full) {
                // Tokens past the context (the unused tail of the last block) get V = 0, so that
                // whatever those cache slots hold cannot reach O through a zero probability.
#pragma unroll
                for (int bi = 0; bi < 2; ++bi)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if ((pb + bi) * kMfmaBS + 4 * g + e >= si.ctx)
#pragma unroll
                            for (int q = 0; q < KVPair<D>::kVW; ++q) kv.v[bi][e][q] = 0u;
            }
            bf16x8 pB[NTW];
#pragma unroll
            for (int nt = 0; nt < NTW; ++nt) pB[nt] = softmax_tile(nt, S[0][nt], S[1][nt], full, pb, blk0, blk1);

            // O^T += V^T P^T.
#pragma unroll
            for (int dt = 0; dt < T; ++dt) {
                const bf16x8 A = v_operand(kv, dt);
#pragma unroll
                for (int nt = 0; nt < NTW; ++nt)
                    O[dt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, pB[nt], O[dt][nt], 0, 0, 0);
            }
        };

        // Each wave streams the pairs wp, wp + WPH, wp + 2 WPH, ... of the split for its kv head.
        // The loads of the next pair are issued before the current pair is computed (two
        // register buffers, unrolled).
        constexpr int step = 2 * WPH;
        {
            // Pair j of this wave covers blocks pb0 + j step and pb0 + j step + 1. Lane j % 64 holds
            // the ids of pair j in slot j / 64 (the host keeps a split within
            // kMfmaMaxPairsPerWave pairs per wave); the loop reads them with readlane into scalar
            // registers and needs no vector temporaries for addressing.
            constexpr int kPairSlots = kMfmaMaxPairsPerWave / 64;
            const int pb0 = blk_begin + 2 * wp;
            int pid0[kPairSlots], pid1[kPairSlots];
#pragma unroll
            for (int t = 0; t < kPairSlots; ++t) {
                const int pbj = pb0 + (t * 64 + lane) * step;
                pid0[t] = pbj < blk_end ? s_blk[pbj - blk_begin] : -1;
                pid1[t] = pbj + 1 < blk_end ? s_blk[pbj + 1 - blk_begin] : -1;
            }
            auto pair_ids = [&](int j, int& b0, int& b1) {
                b0 = __builtin_amdgcn_readlane(pid0[0], j & 63);
                b1 = __builtin_amdgcn_readlane(pid1[0], j & 63);
#pragma unroll
                for (int t = 1; t < kPairSlots; ++t) {
                    const int x0 = __builtin_amdgcn_readlane(pid0[t], j & 63);
                    const int x1 = __builtin_amdgcn_readlane(pid1[t], j & 63);
                    b0 = (j >> 6) == t ? x0 : b0;
                    b1 = (j >> 6) == t ? x1 : b1;
                }
            };
            const int npairs = pb0 < blk_end ? (blk_end - 1 - pb0) / step + 1 : 0;
            // The ids of the pair after j, or -1 (the zero slab, cache-hot) past the last pair.
            auto next_ids = [&](int j, int& b0, int& b1) {
                pair_ids(min(j + 1, kPairSlots * 64 - 1), b0, b1);
                b0 = j + 1 < npairs ? b0 : -1;
                b1 = j + 1 < npairs ? b1 : -1;
            };
            KVPair<D> bufA, bufB;
            // The next pair's loads are issued unconditionally: past the last pair they read
            // the zero slab (and are dropped), so no branch separates a prefetch from the wait
            // that precedes the computation of the pair before it. P is the loads' cache policy.
            auto stream = [&](auto pol) {
                constexpr int P = decltype(pol)::value;
                int j = 0, a0, a1, b0, b1;
                pair_ids(0, a0, a1);
                load_pair<P, KM, D, DR>(bufA, ktA, kp, vp, a0, a1, slot_stride, kv_off, r, g);
                while (true) {
                    next_ids(j, b0, b1);
                    load_pair<P, KM, D, DR>(bufB, ktB, kp, vp, b0, b1, slot_stride, kv_off, r, g);
                    compute(bufA, ktA, pb0 + j * step, a0, a1);
                    if (++j >= npairs) break;
                    next_ids(j, a0, a1);
                    load_pair<P, KM, D, DR>(bufA, ktA, kp, vp, a0, a1, slot_stride, kv_off, r, g);
                    compute(bufB, ktB, pb0 + j * step, b0, b1);
                    if (++j >= npairs) break;
                }
            };
            if (npairs > 0) {
                if constexpr (POL == kLoadPerUnit) {
                    // A unit whose rows fit this row group is read by no other workgroup.
                    if (si.rows <= RW) stream(std::integral_constant<int, kLoadStream>{});
                    else stream(std::integral_constant<int, kLoadCached>{});
                } else {
                    stream(std::integral_constant<int, POL>{});
                }
            }
        }

        if constexpr (QL) {
            // The frame shares LDS with the K tiles: every wave's last (dropped) prefetch must
            // have landed, and every wave must be done reading its tiles, before it is written.
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
        }

        // Row sums: each lane summed its own 8 tokens per pair; fold the four 16-lane groups.
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt) {
            lsum[nt] += shfl_xor_f(lsum[nt], 16);
            lsum[nt] += shfl_xor_f(lsum[nt], 32);
        }

        // Merge each kv head's waves in its frame: common max, then the rescaled accumulators
        // are added into LDS in a fixed order (the head's first wave stores), so the result is
        // bitwise reproducible. Lane (r, g) owns head dims T (4 g + e) + dt of row 16 nt + r.
        Frame<RW, D>& fr = frame[hw];
        if (g == 0) {
#pragma unroll
            for (int nt = 0; nt < NTW; ++nt) fr.m[wp][nt * 16 + r] = m[nt];
        }
        __syncthreads();
        float f[NTW];
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt) {
            const int n = nt * 16 + r;
            float M = fr.m[0][n];
#pragma unroll
            for (int w = 1; w < WPH; ++w) M = fmaxf(M, fr.m[w][n]);
            f[nt] = (m[nt] == kNegInf) ? 0.f : fast_exp2(m[nt] - M);
            if (g == 0) {
                fr.l[wp][n] = lsum[nt] * f[nt];
                if (wp == 0) fr.mx[n] = M;
            }
        }
        for (int w = 0; w < WPH; ++w) {  // every wave of the workgroup takes part in each barrier
            if (wp == w) {
#pragma unroll
                for (int nt = 0; nt < NTW; ++nt) {
                    if (QL && nt >= ntile) continue;  // rows past the unit: never stored
                    float* dst = &fr.acc[(nt * 16 + r) * Frame<RW, D>::kStride + 4 * T * g];
#pragma unroll
                    for (int e = 0; e < 4; ++e)
#pragma unroll
                        for (int dt = 0; dt < T; ++dt) {
                            const float v = O[dt][nt][e] * f[nt];
                            dst[T * e + dt] = (w == 0) ? v : dst[T * e + dt] + v;
                        }
                }
            }
            __syncthreads();
        }
        const int nrows = min(RW, si.rows - row0);
#pragma unroll
        for (int h = 0; h < HP; ++h) {  // the whole workgroup stores each head's rows
            SeqInfo sh = si;
            sh.kvh = (ug * HP + h) % a.Hkv;
            frame_flush<RW, D, DR>(a, sh, nsplit, row0, nrows > 0 ? nrows : 0, frame[h], WPH, pb0 + h * pbstep);
        }
    }
}

// ------------------------------------------------------------------ MFMA kernel, f32 caches
//
// The reference's own dtype. v_mfma_f32_16x16x4_f32 takes one f32 per lane for each operand:
// A lane l = A[l % 16][l / 16], B lane l = B[l / 16][l % 16], and D lane l, element e =
// D[4 (l / 16) + e][l % 16]. The kernel streams one 16-token block at a time (an f32 block is
// as many registers as a bf16 pair), with the same frame, schedule and merge as the bf16 kernel.
//  * S^T = K Q^T: lane (r, g) loads K[token r][16 s + 4 g .. + 3] (s = 0..7; 16 rows x 64
//    contiguous bytes per instruction), and MFMA (s, e) contracts dims 16 s + 4 g + e; Q is loaded
//    the same way for its rows.
//  * O^T += V^T P^T over tokens 4 g + q at step q (q = 0..3): the softmax'd S^T fragment of lane
//    (row r, g) holds tokens 4 g + e, so element q is already the B operand of step q (no
//    shuffle). Lane (r, g) loads V[token 4 g + q][64 h + 4 r .. + 3] (h = 0, 1): component e_t
//    is the A operand of the d-tile holding dims 64 h + 4 i + e_t, and the accumulator of that
//    tile gives lane (r, g) dims 64 h + 16 g + 4 e' + e_t of row r.
// 32 + 32 MFMAs per block and 16-row tile: at 32 cycles each, about 60% of a block's streaming
// time for two tiles (GQA 32/8 with 8 draft rows), so the loads still set the pace.

__device__ float kZeroSlabF32[kMfmaBS * kMfmaD];

struct KVBlockF32 {
    float4 k[8];  // [s]: token r, dims 16 s + 4 g .. + 3
    float4 v[8];  // [2 q + h]: token 4 g + q, dims 64 h + 4 r .. + 3
};

template <int POL>
__device__ __forceinline__ void load_block_f32(KVBlockF32& kv, const float* __restrict__ kp,
                                               const float* __restrict__ vp, int blk, size_t slot_stride,
                                               size_t kv_off, int r, int g) {
    constexpr int kSlabBytes = kMfmaBS * kMfmaD * 4;
    const size_t base = (size_t)(blk >= 0 ? blk : 0) * slot_stride + kv_off;
    const float* kslab = blk >= 0 ? kp + base : kZeroSlabF32;
    const float* vslab = blk >= 0 ? vp + base : kZeroSlabF32;
    const __amdgpu_buffer_rsrc_t kr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(kslab), (short)0, kSlabBytes, kRawBufferWord3);
    const __amdgpu_buffer_rsrc_t vr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(vslab), (short)0, kSlabBytes, kRawBufferWord3);
    const int koff = (r * kMfmaD + 4 * g) * 4;       // + 64 s
    const int voff = (4 * g * kMfmaD + 4 * r) * 4;   // + (q * 128 + 64 h) * 4
#pragma unroll
    for (int s = 0; s < 8; ++s)
        kv.k[s] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(kr, koff, 64 * s, POL));
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int h = 0; h < 2; ++h)
            kv.v[2 * q + h] =
                __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(vr, voff, (q * kMfmaD + 64 * h) * 4, POL));
}

__device__ __forceinline__ float f4_get(const float4& v, int i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// One work item of the f32 kernel; the arguments are those of mfma_item.
template <int NTW, int HP, int POL>
__device__ __forceinline__ void mfma_item_f32(const AttnArgs& a, Frame<NTW * 16, kMfmaD> (&frame)[HP], int* s_blk,
                                              const SeqInfo& si, int ug, int rg, int blk_begin, int blk_end,
                                              int nsplit, size_t pb0, size_t pbstep) {
    constexpr int D = kMfmaD;
    constexpr int RW = NTW * 16;
    constexpr int WPH = kWaves / HP;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int hw = wave / WPH;
    const int wp = wave % WPH;
    const int row0 = rg * RW;

    const int lane = threadIdx.x & 63;
    const int r = lane & 15;
    const int g = lane >> 4;
    const float* __restrict__ qp = reinterpret_cast<const float*>(a.q);
    const float* __restrict__ kp = reinterpret_cast<const float*>(a.k);
    const float* __restrict__ vp = reinterpret_cast<const float*>(a.v);
    const size_t slot_stride = (size_t)kMfmaBS * D;
    const size_t kv_off = (size_t)si.kvh * a.bs * D;
    const float c = a.scale_log2;
    const int full_vis = a.causal ? si.ctx - si.q_len + 1 : si.ctx;

    stage_block_ids(a, si, blk_begin, blk_end, s_blk);

    {
        // Q^T operands: lane (r, g) holds row row0 + 16 nt + r, dims 16 s + 4 g .. + 3.
        float4 qB[NTW][8];
        int vis[NTW];
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt) {
            const int n = row0 + nt * 16 + r;
            if (n < si.rows) {
                const int j = n / a.group;
                const size_t qrow = out_row(a, si, n);
#pragma unroll
                for (int s = 0; s < 8; ++s) qB[nt][s] = *reinterpret_cast<const float4*>(qp + qrow * D + 16 * s + 4 * g);
                vis[nt] = a.causal ? si.ctx - si.q_len + j + 1 : si.ctx;
            } else {
#pragma unroll
                for (int s = 0; s < 8; ++s) qB[nt][s] = make_float4(0.f, 0.f, 0.f, 0.f);
                vis[nt] = si.ctx;
            }
        }

        float m[NTW], lsum[NTW];
        f32x4 O[8][NTW];  // [2 h + ... ] d-tile dt = 4 h + e_t
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt) {
            m[nt] = kNegInf;
            lsum[nt] = 0.f;
#pragma unroll
            for (int dt = 0; dt < 8; ++dt) O[dt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
        }

        auto compute = [&](KVBlockF32& kv, int pb, int blk) {
            f32x4 S[NTW];
#pragma unroll
            for (int nt = 0; nt < NTW; ++nt) {
                f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int s = 0; s < 8; ++s)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(f4_get(kv.k[s], e), f4_get(qB[nt][s], e), acc, 0, 0, 0);
                S[nt] = acc;
            }
            const bool full = blk >= 0 && (pb + 1) * kMfmaBS <= full_vis;
            if (!full) {
                // V rows of tokens past the context are zeroed, as in the bf16 kernel.
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    if (pb * kMfmaBS + 4 * g + q >= si.ctx) {
                        kv.v[2 * q] = make_float4(0.f, 0.f, 0.f, 0.f);
                        kv.v[2 * q + 1] = make_float4(0.f, 0.f, 0.f, 0.f);
                    }
            }
            float pv[NTW][4];
#pragma unroll
            for (int nt = 0; nt < NTW; ++nt) {
                float sv[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) sv[e] = S[nt][e];
                if (!full) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int t = pb * kMfmaBS + 4 * g + e;
                        if (!(blk >= 0 && t < vis[nt])) sv[e] = kNegInf;
                    }
                }
                float mx = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
                mx = max_over_rows(mx);
                const float m_new = fmaxf(m[nt], mx * c);
                const float mref = (m_new == kNegInf) ? 0.f : m_new;
                const float alpha = fast_exp2(m[nt] - mref);
                float ps = 0.f;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    pv[nt][e] = fast_exp2(__builtin_fmaf(sv[e], c, -mref));
                    ps += pv[nt][e];
                }
                lsum[nt] = lsum[nt] * alpha + ps;
                if (__any(m_new > m[nt] && m[nt] != kNegInf)) {
#pragma unroll
                    for (int dt = 0; dt < 8; ++dt) O[dt][nt] *= alpha;
                }
                m[nt] = m_new;
            }
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int dt = 0; dt < 8; ++dt) {
                    const float av = f4_get(kv.v[2 * q + (dt >> 2)], dt & 3);
#pragma unroll
                    for (int nt = 0; nt < NTW; ++nt)
                        O[dt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, pv[nt][q], O[dt][nt], 0, 0, 0);
                }
        };

        // Each wave streams blocks wp, wp + WPH, ... of the split; the next block's loads are issued
        // before the current block is computed. Lane j % 64 holds the id of the wave's block j in
        // slot j / 64.
        {
            constexpr int kSlots = 2 * kMfmaMaxPairsPerWave / 64;
            const int b0 = blk_begin + wp;
            int bid[kSlots];
#pragma unroll
            for (int t = 0; t < kSlots; ++t) {
                const int bj = b0 + (t * 64 + lane) * WPH;
                bid[t] = bj < blk_end ? s_blk[bj - blk_begin] : -1;
            }
            auto block_id = [&](int j) {
                int x = __builtin_amdgcn_readlane(bid[0], j & 63);
#pragma unroll
                for (int t = 1; t < kSlots; ++t) {
                    const int y = __builtin_amdgcn_readlane(bid[t], j & 63);
                    x = (j >> 6) == t ? y : x;
                }
                return x;
            };
            const int nblk = b0 < blk_end ? (blk_end - 1 - b0) / WPH + 1 : 0;
            auto next_id = [&](int j) {
                const int x = block_id(min(j + 1, kSlots * 64 - 1));
                return j + 1 < nblk ? x : -1;
            };
            KVBlockF32 bufA, bufB;
            if (nblk > 0) {
                int j = 0;
                int ia = block_id(0), ib;
                load_block_f32<POL>(bufA, kp, vp, ia, slot_stride, kv_off, r, g);
                while (true) {
                    ib = next_id(j);
                    load_block_f32<POL>(bufB, kp, vp, ib, slot_stride, kv_off, r, g);
                    compute(bufA, b0 + j * WPH, ia);
                    if (++j >= nblk) break;
                    ia = next_id(j);
                    load_block_f32<POL>(bufA, kp, vp, ia, slot_stride, kv_off, r, g);
                    compute(bufB, b0 + j * WPH, ib);
                    if (++j >= nblk) break;
                }
            }
        }

#pragma unroll
        for (int nt = 0; nt < NTW; ++nt) {
            lsum[nt] += shfl_xor_f(lsum[nt], 16);
            lsum[nt] += shfl_xor_f(lsum[nt], 32);
        }

        Frame<RW, D>& fr = frame[hw];
        if (g == 0) {
#pragma unroll
            for (int nt = 0; nt < NTW; ++nt) fr.m[wp][nt * 16 + r] = m[nt];
        }
        __syncthreads();
        float f[NTW];
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt) {
            const int n = nt * 16 + r;
            float M = fr.m[0][n];
#pragma unroll
            for (int w = 1; w < WPH; ++w) M = fmaxf(M, fr.m[w][n]);
            f[nt] = (m[nt] == kNegInf) ? 0.f : fast_exp2(m[nt] - M);
            if (g == 0) {
                fr.l[wp][n] = lsum[nt] * f[nt];
                if (wp == 0) fr.mx[n] = M;
            }
        }
        // Lane (r, g) holds dims 64 h + 16 g + 4 e' + e_t of row 16 nt + r in O[4 h + e_t][nt][e'].
        for (int w = 0; w < WPH; ++w) {
            if (wp == w) {
#pragma unroll
                for (int nt = 0; nt < NTW; ++nt) {
                    float* dst = &fr.acc[(nt * 16 + r) * Frame<RW, D>::kStride + 16 * g];
#pragma unroll
                    for (int h = 0; h < 2; ++h)
#pragma unroll
                        for (int e2 = 0; e2 < 4; ++e2)
#pragma unroll
                            for (int et = 0; et < 4; ++et) {
                                const float v = O[4 * h + et][nt][e2] * f[nt];
                                float* p = dst + 64 * h + 4 * e2 + et;
                                *p = (w == 0) ? v : *p + v;
                            }
                }
            }
            __syncthreads();
        }
        const int nrows = min(RW, si.rows - row0);
#pragma unroll
        for (int h = 0; h < HP; ++h) {
            SeqInfo sh = si;
            sh.kvh = (ug * HP + h) % a.Hkv;
            frame_flush<RW, D>(a, sh, nsplit, row0, nrows > 0 ? nrows : 0, frame[h], WPH, pb0 + h * pbstep);
        }
    }
}

// PLAN: the balanced schedule (a persistent grid walking the plan's items) or one workgroup per
// (kv head group, split, row group) of the grid schedule. `item` runs one work item: (this
// wave's SeqInfo, kv head group, row group, first block, end block, splits, workspace row of
// head 0, workspace rows between heads).
template <int NTW, int HP, bool PLAN, typename Item>
__device__ __forceinline__ void mfma_schedule(const AttnArgs& a, Item&& item) {
    constexpr int RW = NTW * 16;
    constexpr int WPH = kWaves / HP;
    const int hw = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) / WPH;

    if constexpr (PLAN) {
        __shared__ PlanLds plan;
        plan_build<RW, HP>(a, plan);
        const int G = a.plan_grid;  // a multiple of 8
        const int U = a.Hkv / HP;
        // Workgroup w works on lane x = w % 8, the items dealt to its XCD: first the lane's item
        // k = w / 8, then (below) one assigned item or whichever item of the lane is next
        // unclaimed when it becomes free. The G / 8 workgroups of an XCD thus take the lane's
        // items largest first, and the row groups of one item group (consecutive on the lane)
        // run together and share its L2.
        __shared__ int s_claim;
        const int x = (int)blockIdx.x & 7;
        const int len = plan.len;
        const int C = plan.C;
        const int nw = G / 8, pw = (int)blockIdx.x >> 3;  // workgroups of the lane, this one's place
        for (int k = pw; k < len;) {
            PlanItem it = {0, 0, 0, 0, 0};
            const bool has = plan_item<HP>(a, plan, k, it);
            // Plan values come from LDS: make them scalar for the addressing that follows.
            const int b = __builtin_amdgcn_readfirstlane(it.b);
            const int hp = __builtin_amdgcn_readfirstlane(it.hp);
            const int rg = __builtin_amdgcn_readfirstlane(it.rg);
            const int chunk = __builtin_amdgcn_readfirstlane(it.chunk);
            const int slot = __builtin_amdgcn_readfirstlane(it.slot);
            SeqInfo si;
            si.b = b;
            si.kvh = hp * HP + hw;
            si.ctx = __builtin_amdgcn_readfirstlane(plan.ctx[b]);
            si.q0 = __builtin_amdgcn_readfirstlane(plan.q0[b]);
            si.q_len = __builtin_amdgcn_readfirstlane(plan.qlen[b]);
            si.rows = si.q_len * a.group;
            si.nblk = (si.ctx + a.ubs - 1) / a.ubs;
            si.ok = true;
            const int nsplit = __builtin_amdgcn_readfirstlane(plan.ns[b]);
            const int blk_begin = chunk * C;
            const int blk_end = min(si.nblk, blk_begin + C);
            if (__builtin_amdgcn_readfirstlane(has ? 1 : 0))
                item(si, si.b * U + hp, rg, blk_begin, blk_end, nsplit, (size_t)slot * HP * RW, (size_t)RW);
            if (len <= 2 * nw) {
                // At most one item per workgroup beyond its first: no claims. Item nw + i goes
                // to workgroup nw - 1 - i, so the largest of the rest join the smallest first
                // items (skewed prefix, chunks of 5L/4: 146.2 -> 143.0 us). With more items per
                // workgroup the claims adapt to the rates each one sees and measured better
                // (mixed GQA 64/8: 391 against 406 us for the same rule continued as a snake).
                k = k < nw ? 2 * nw - 1 - pw : len;
            } else {
                // Claimed after the item: an atomic issued before it would sit at the head of
                // the in-order load counter and hold up the item's first waits (measured: 437
                // -> 474 us on the mixed GQA 64/8 batch).
                if (threadIdx.x == 0) s_claim = nw + atomicAdd(&a.sched[x], 1);
                __syncthreads();
                k = s_claim;
                __syncthreads();  // s_claim is written again after the next item
            }
        }
        // The last workgroup out resets the counters for the next launch: every other workgroup
        // has had its last claim answered before it counts itself done.
        if (threadIdx.x == 0 && atomicAdd(&a.sched[8], 1) == G - 1) {
#pragma unroll
            for (int j = 0; j < kSchedWords; ++j) a.sched[j] = 0;
        }
    } else {
        int ug, split, rg;
        if (!map_workgroup(a, ug, split, rg)) return;
        // The group's units belong to one sequence, so everything but the kv head is the same for
        // every wave, and the early returns below are taken by the whole workgroup or by none of it.
        const SeqInfo si = seq_info(a, ug * HP + hw);
        if (!si.ok) return;
        const int nsplit = num_splits_for(a, si.nblk);
        if (split >= nsplit) return;
        if (rg > 0 && rg * RW >= si.rows) return;  // this row group is past the sequence's rows
        const int blk_begin = split * a.chunk_blocks;
        const int blk_end = min(si.nblk, blk_begin + a.chunk_blocks);
        item(si, ug, rg, blk_begin, blk_end, nsplit, ((size_t)ug * HP * a.splits + split) * a.rows_cap + rg * RW,
             (size_t)a.splits * a.rows_cap);
    }
}

// The LDS merge frames of a workgroup's heads; the many-tile kernel keeps its one frame in its
// first K-tile array instead.
template <int NTW, int HP, bool QL, int D>
struct FrameLds {
    Frame<NTW * 16, D> f[HP];
};
template <int NTW, int HP, int D>
struct FrameLds<NTW, HP, true, D> {};

// bf16 caches. Head dims other than 128 load K straight into operand layout and take at most
// two row tiles per wave (the LDS-staged K tiles and the many-tile form are built for 256-byte
// token rows).
template <int NTW, int HP, int POL, bool PLAN, int D = kMfmaD, int DR = D>
__global__ __launch_bounds__(kThreads) void attn_mfma_kernel(AttnArgs a) {
    using Fr = Frame<NTW * 16, D>;
    constexpr bool QL = NTW > 2;
    __shared__ FrameLds<NTW, HP, QL, D> s_fr;
    __shared__ int s_blk[kMaxChunkBlocks];
    constexpr int KM = (D == kMfmaD && DR == D) ? kKModeFor<NTW, PLAN> : kKDirect;
    // Two separate arrays, so that the compiler's wait for one tile's loads does not also wait
    // for the other's (it tells LDS DMA destinations apart by the object written). The
    // many-tile kernel keeps its merge frame in the first (the frame is used only after the
    // streaming, behind a wait for every tile load and a barrier).
    constexpr int kTileU4 = KM == kKDma ? kWaves * kKStageChunks : 1;
    constexpr int kFrameU4 = (int)((sizeof(Fr) * HP + 15) / 16);
    __shared__ uint4 s_kstA[QL && kFrameU4 > kTileU4 ? kFrameU4 : kTileU4];
    __shared__ uint4 s_kstB[kTileU4];
    __shared__ uint4 s_q[QL ? NTW * 16 * kQStride : 1];
    Fr* fp;
    if constexpr (QL) fp = reinterpret_cast<Fr*>(s_kstA);
    else fp = s_fr.f;
    Fr (&frame)[HP] = *reinterpret_cast<Fr(*)[HP]>(fp);
    mfma_schedule<NTW, HP, PLAN>(a, [&](const SeqInfo& si, int ug, int rg, int bb, int be, int ns, size_t pb0,
                                        size_t pbs) {
        mfma_item<NTW, HP, POL, KM, D, DR>(a, frame, s_blk, s_kstA, s_kstB, s_q, si, ug, rg, bb, be, ns, pb0, pbs);
    });
}

// f32 caches.
template <int NTW, int HP, int POL, bool PLAN>
__global__ __launch_bounds__(kThreads) void attn_mfma_f32_kernel(AttnArgs a) {
    __shared__ Frame<NTW * 16, kMfmaD> frame[HP];
    __shared__ int s_blk[kMaxChunkBlocks];
    mfma_schedule<NTW, HP, PLAN>(a, [&](const SeqInfo& si, int ug, int rg, int bb, int be, int ns, size_t pb0,
                                        size_t pbs) {
        mfma_item_f32<NTW, HP, POL>(a, frame, s_blk, si, ug, rg, bb, be, ns, pb0, pbs);
    });
}


// ---------------------------------------------------------------------------- vector kernel

template <typename T>
struct Elem;
// N consecutive elements at p, in the widest loads their alignment allows: a lane's slice starts
// at a multiple of N elements of a row that starts 16-byte aligned (the head dim is a multiple
// of 8), so N divisible by 4 (f32) or 8 (bf16) gives 16-byte loads, and smaller powers of two
// narrower ones.
template <>
struct Elem<float> {
    template <int N>
    __device__ static __forceinline__ void load(const float* p, float (&x)[N]) {
        if constexpr (N % 4 == 0) {
#pragma unroll
            for (int i = 0; i < N; i += 4) {
                const float4 v = *reinterpret_cast<const float4*>(p + i);
                x[i] = v.x;
                x[i + 1] = v.y;
                x[i + 2] = v.z;
                x[i + 3] = v.w;
            }
        } else if constexpr (N % 2 == 0) {
#pragma unroll
            for (int i = 0; i < N; i += 2) {
                const float2 v = *reinterpret_cast<const float2*>(p + i);
                x[i] = v.x;
                x[i + 1] = v.y;
            }
        } else {
#pragma unroll
            for (int i = 0; i < N; ++i) x[i] = p[i];
        }
    }
};
template <>
struct Elem<uint16_t> {
    template <int N>
    __device__ static __forceinline__ void load(const uint16_t* p, float (&x)[N]) {
        if constexpr (N % 8 == 0) {
#pragma unroll
            for (int i = 0; i < N; i += 8) {
                const uint4 v = load16(p + i);
                const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    x[i + 2 * k] = bf16_lo(w[k]);
                    x[i + 2 * k + 1] = bf16_hi(w[k]);
                }
            }
        } else if constexpr (N % 4 == 0) {
#pragma unroll
            for (int i = 0; i < N; i += 4) {
                const uint2 v = *reinterpret_cast<const uint2*>(p + i);
                x[i] = bf16_lo(v.x);
                x[i + 1] = bf16_hi(v.x);
                x[i + 2] = bf16_lo(v.y);
                x[i + 3] = bf16_hi(v.y);
            }
        } else if constexpr (N % 2 == 0) {
#pragma unroll
            for (int i = 0; i < N; i += 2) {
                const uint32_t v = *reinterpret_cast<const uint32_t*>(p + i);
                x[i] = bf16_lo(v);
                x[i + 1] = bf16_hi(v);
            }
        } else {
#pragma unroll
            for (int i = 0; i < N; ++i) x[i] = __uint_as_float((uint32_t)p[i] << 16);
        }
    }
};

constexpr int kVecRows = kVectorRowsPerGroup;

// Lanes that share one token row of the vector kernel: 16 when the head dim is a multiple of
// 16, else 8 (head dims 8, 24, 40, ...).
template <int D>
constexpr int kVecLanesPerRow = D % 16 == 0 ? 16 : 8;

// Sum over the lanes of one token row.
template <int LPR>
__device__ __forceinline__ float token_row_sum(float v) {
    if constexpr (LPR == 16) return row16_sum(v);
    else return row8_sum(v);
}

template <typename T, int D>
__global__ __launch_bounds__(kThreads) void attn_vector_kernel(AttnArgs a) {
    static_assert(D % 8 == 0 && D <= kMaxHeadDim, "head dim: a multiple of 8, at most kMaxHeadDim");
    constexpr int R = kVecRows;
    constexpr int LPR = kVecLanesPerRow<D>;
    constexpr int DPL = D / LPR;   // head-dim elements per lane
    constexpr int TPW = 64 / LPR;  // token rows a wave takes per step
    __shared__ Frame<R, D> frame;

    int unit, split, rg;
    if (!map_workgroup(a, unit, split, rg)) return;
    const SeqInfo si = seq_info(a, unit);
    if (!si.ok) return;
    const int nsplit = num_splits_for(a, si.nblk);
    if (split >= nsplit) return;
    const int row0 = rg * R;
    if (row0 > 0 && row0 >= si.rows) return;  // this row group is past the sequence's rows

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int r = lane % LPR;  // head-dim slice [r * DPL, r * DPL + DPL)
    const int g = lane / LPR;  // token row within the wave's TPW
    const T* __restrict__ qp = reinterpret_cast<const T*>(a.q);
    const T* __restrict__ kp = reinterpret_cast<const T*>(a.k);
    const T* __restrict__ vp = reinterpret_cast<const T*>(a.v);
    const int t_begin = split * a.chunk_blocks * a.bs;
    const int t_end = min(si.ctx, (split + 1) * a.chunk_blocks * a.bs);

    {
        const int nrows = min(R, si.rows - row0);
        float q[R][DPL];
        int vis[R];
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const int n = row0 + i;
            if (n < si.rows) {
                Elem<T>::load(qp + out_row(a, si, n) * D + r * DPL, q[i]);
                vis[i] = a.causal ? si.ctx - si.q_len + n / a.group + 1 : si.ctx;
            } else {
#pragma unroll
                for (int d = 0; d < DPL; ++d) q[i][d] = 0.f;
                vis[i] = 0;
            }
        }
        float m[R], l[R], acc[R][DPL];
#pragma unroll
        for (int i = 0; i < R; ++i) {
            m[i] = kNegInf;
            l[i] = 0.f;
#pragma unroll
            for (int d = 0; d < DPL; ++d) acc[i][d] = 0.f;
        }

        for (int t0 = t_begin + TPW * wave; t0 < t_end; t0 += TPW * kWaves) {
            const int t = t0 + g;
            const bool tok_ok = t < t_end;
            int64_t blk = -1;
            if (tok_ok) blk = checked_block(a, si.b, t / a.bs);
            float kx[DPL], vx[DPL];
            if (blk >= 0) {
                const size_t off = (((size_t)blk * a.Hkv + si.kvh) * a.bs + (t % a.bs)) * D + r * DPL;
                Elem<T>::load(kp + off, kx);
                Elem<T>::load(vp + off, vx);
            } else {
#pragma unroll
                for (int d = 0; d < DPL; ++d) kx[d] = vx[d] = 0.f;
            }
#pragma unroll
            for (int i = 0; i < R; ++i) {
                float s = 0.f;
#pragma unroll
                for (int d = 0; d < DPL; ++d) s += q[i][d] * kx[d];
                s = token_row_sum<LPR>(s);
                s = (blk >= 0 && t < vis[i]) ? s * a.scale_log2 : kNegInf;
                const float m_new = fmaxf(m[i], s);
                const float mref = (m_new == kNegInf) ? 0.f : m_new;
                const float alpha = fast_exp2(m[i] - mref);
                const float p = fast_exp2(s - mref);
                l[i] = l[i] * alpha + p;
#pragma unroll
                for (int d = 0; d < DPL; ++d) acc[i][d] = acc[i][d] * alpha + p * vx[d];
                m[i] = m_new;
            }
        }

        // Fold the wave's TPW token rows (LPR-lane groups), then merge waves in LDS.
#pragma unroll
        for (int i = 0; i < R; ++i) {
            float M = m[i];
#pragma unroll
            for (int x = LPR; x < 64; x *= 2) M = fmaxf(M, shfl_xor_f(M, x));
            const float f = (m[i] == kNegInf) ? 0.f : fast_exp2(m[i] - M);
            l[i] *= f;
#pragma unroll
            for (int x = LPR; x < 64; x *= 2) l[i] += shfl_xor_f(l[i], x);
#pragma unroll
            for (int d = 0; d < DPL; ++d) {
                float v = acc[i][d] * f;
#pragma unroll
                for (int x = LPR; x < 64; x *= 2) v += shfl_xor_f(v, x);
                acc[i][d] = v;
            }
            m[i] = M;
        }
        if (lane == 0) {
#pragma unroll
            for (int i = 0; i < R; ++i) frame.m[wave][i] = m[i];
        }
        __syncthreads();
        float f[R];
#pragma unroll
        for (int i = 0; i < R; ++i) {
            float M = frame.m[0][i];
#pragma unroll
            for (int w = 1; w < kWaves; ++w) M = fmaxf(M, frame.m[w][i]);
            f[i] = (m[i] == kNegInf) ? 0.f : fast_exp2(m[i] - M);
            if (lane == 0) {
                frame.l[wave][i] = l[i] * f[i];
                if (wave == 0) frame.mx[i] = M;
            }
        }
        // Fixed-order merge (wave 0 stores, the others add in turn): bitwise reproducible.
        for (int w = 0; w < kWaves; ++w) {
            if (wave == w && g == 0) {
#pragma unroll
                for (int i = 0; i < R; ++i)
#pragma unroll
                    for (int d = 0; d < DPL; ++d) {
                        float* p = &frame.acc[i * Frame<R, D>::kStride + r * DPL + d];
                        const float v = acc[i][d] * f[i];
                        *p = (w == 0) ? v : *p + v;
                    }
            }
            __syncthreads();
        }
        frame_flush<R, D>(a, si, nsplit, row0, nrows > 0 ? nrows : 0, frame, kWaves,
                          ((size_t)unit * a.splits + split) * a.rows_cap + row0);
    }
}

// ------------------------------------------------------------------------------ launcher

#ifdef KYRO_ATTN_HD_UNIT
// The bf16 MFMA kernel at head dims other than 128 (64, 80, 96 and 256 in one translation unit,
// 112, 160, 192 and 224 in another, so that their instances compile in parallel with the rest):
// at most two row tiles per wave (one above 128, where the K/V pairs and accumulators fill the
// register file), one or two kv heads per workgroup, streaming or cached K/V loads, grid or
// balanced schedule. D is the operand layout, DR the head dim (80 runs in the layout of 96, 112
// in that of 128).
template <int D, int DR = D>
hipError_t launch_mfma_hd(const AttnArgs& a, const dim3 grid, hipStream_t stream) {
    const dim3 block(kThreads);
    const int rpg = a.rows_per_group;
#define KYRO_HD_LAUNCH(NT, POL, PLAN)                                                           \
    {                                                                                           \
        if (a.hpw == 2) attn_mfma_kernel<NT, 2, POL, PLAN, D, DR><<<grid, block, 0, stream>>>(a); \
        else attn_mfma_kernel<NT, 1, POL, PLAN, D, DR><<<grid, block, 0, stream>>>(a);          \
    }
#define KYRO_HD_POL(NT, PLAN)                                                               \
    {                                                                                       \
        if (a.stream_kv) KYRO_HD_LAUNCH(NT, kLoadStream, PLAN)                              \
        else KYRO_HD_LAUNCH(NT, kLoadCached, PLAN)                                          \
    }
    if constexpr (D > kMfmaD) {  // one row tile
        if (a.plan) KYRO_HD_POL(1, true)
        else KYRO_HD_POL(1, false)
    } else {
        if (rpg == 16) {
            if (a.plan) KYRO_HD_POL(1, true)
            else KYRO_HD_POL(1, false)
        } else {
            if (a.plan) KYRO_HD_POL(2, true)
            else KYRO_HD_POL(2, false)
        }
    }
#undef KYRO_HD_POL
#undef KYRO_HD_LAUNCH
    if (a.plan) {
        constexpr long long kCombineMaxGrid = 2048;
        const long long units = (long long)a.units * ((a.rows_cap + kCombineRows - 1) / kCombineRows);
        attn_combine_plan_kernel<DR><<<dim3((unsigned)(units < kCombineMaxGrid ? units : kCombineMaxGrid)), block, 0,
                                        stream>>>(a);
    } else if (a.splits > 1) {
        const int rpw = kThreads / (DR / 4);
        const dim3 cgrid((unsigned)a.units, (unsigned)((a.rows_cap + rpw - 1) / rpw));
        attn_combine_kernel<DR><<<cgrid, block, 0, stream>>>(a);
    }
    return hipGetLastError();
}

}  // namespace

#if KYRO_ATTN_HD_UNIT == 1
hipError_t launch_paged_attention_mfma_hd(const AttnArgs& a, hipStream_t stream) {
    const dim3 grid((unsigned)(a.plan ? a.plan_grid : a.ugroups_padded * a.splits * a.row_groups));
    if (grid.x == 0) return hipSuccess;
    switch (a.D) {
        case 64: return launch_mfma_hd<64>(a, grid, stream);
        case 80: return launch_mfma_hd<96, 80>(a, grid, stream);
        case 96: return launch_mfma_hd<96>(a, grid, stream);
        case 256: return launch_mfma_hd<256>(a, grid, stream);
        default: return hipErrorInvalidValue;
    }
}
#else
hipError_t launch_paged_attention_mfma_hd_wide(const AttnArgs& a, hipStream_t stream) {
    const dim3 grid((unsigned)(a.plan ? a.plan_grid : a.ugroups_padded * a.splits * a.row_groups));
    if (grid.x == 0) return hipSuccess;
    switch (a.D) {
        case 112: return launch_mfma_hd<128, 112>(a, grid, stream);
        case 160: return launch_mfma_hd<160>(a, grid, stream);
        case 192: return launch_mfma_hd<192>(a, grid, stream);
        case 224: return launch_mfma_hd<224>(a, grid, stream);
        default: return hipErrorInvalidValue;
    }
}
#endif

#else  // KYRO_ATTN_HD_UNIT

}  // namespace

hipError_t launch_paged_attention(const AttnArgs& a, int path, hipStream_t stream) {
    const dim3 block(kThreads);
    const dim3 grid((unsigned)(a.plan ? a.plan_grid : a.ugroups_padded * a.splits * a.row_groups));
    if (grid.x == 0) return hipSuccess;
    if (path == ATTN_KERNEL_MFMA && a.D != kMfmaD)
        return (a.D == 112 || a.D == 160 || a.D == 192 || a.D == 224) ? launch_paged_attention_mfma_hd_wide(a, stream)
                                                                       : launch_paged_attention_mfma_hd(a, stream);
    if (path == ATTN_KERNEL_MFMA) {
        const int rpg = a.rows_per_group;
        const bool rows16 = rpg == 16;
#define KYRO_MFMA_LAUNCH2(K, POL, PLAN)                                                     \
        if (a.hpw == 2) {                                                                   \
            if (rows16) K<1, 2, POL, PLAN><<<grid, block, 0, stream>>>(a);                  \
            else K<2, 2, POL, PLAN><<<grid, block, 0, stream>>>(a);                         \
        } else {                                                                            \
            if (rows16) K<1, 1, POL, PLAN><<<grid, block, 0, stream>>>(a);                  \
            else K<2, 1, POL, PLAN><<<grid, block, 0, stream>>>(a);                         \
        }
#define KYRO_MFMA_LAUNCH(POL, PLAN)                                                         \
        if (a.dtype_bf16) {                                                                 \
            if (rpg == kMfmaWideRows) attn_mfma_kernel<kMfmaWideRows / 16, 1, POL, PLAN><<<grid, block, 0, stream>>>(a); \
            else if (rpg == kMfmaManyRows) attn_mfma_kernel<kMfmaManyRows / 16, 1, POL, PLAN><<<grid, block, 0, stream>>>(a); \
            else { KYRO_MFMA_LAUNCH2(attn_mfma_kernel, POL, PLAN) }                         \
        } else {                                                                            \
            KYRO_MFMA_LAUNCH2(attn_mfma_f32_kernel, POL, PLAN)                              \
        }
        if (a.stream_kv == kKvPerUnit) {  // four- and five-tile kernels only (the host decides)
            if (rpg == kMfmaWideRows) {
                if (a.plan) attn_mfma_kernel<kMfmaWideRows / 16, 1, kLoadPerUnit, true><<<grid, block, 0, stream>>>(a);
                else attn_mfma_kernel<kMfmaWideRows / 16, 1, kLoadPerUnit, false><<<grid, block, 0, stream>>>(a);
            } else if (a.plan) {
                attn_mfma_kernel<kMfmaManyRows / 16, 1, kLoadPerUnit, true><<<grid, block, 0, stream>>>(a);
            } else {
                attn_mfma_kernel<kMfmaManyRows / 16, 1, kLoadPerUnit, false><<<grid, block, 0, stream>>>(a);
            }
        } else if (a.plan) {
            if (a.stream_kv) {
                KYRO_MFMA_LAUNCH(kLoadStream, true)
            } else {
                KYRO_MFMA_LAUNCH(kLoadCached, true)
            }
        } else {
            if (a.stream_kv) {
                KYRO_MFMA_LAUNCH(kLoadStream, false)
            } else {
                KYRO_MFMA_LAUNCH(kLoadCached, false)
            }
        }
#undef KYRO_MFMA_LAUNCH
#undef KYRO_MFMA_LAUNCH2
    } else {
        const bool bf16 = a.dtype_bf16;
        switch (a.D) {  // the host admits multiples of 8 up to kMaxHeadDim
#define KYRO_VEC_CASE(DD)                                                                  \
            case DD:                                                                       \
                if (bf16) attn_vector_kernel<uint16_t, DD><<<grid, block, 0, stream>>>(a); \
                else attn_vector_kernel<float, DD><<<grid, block, 0, stream>>>(a);         \
                break;
            KYRO_HEAD_DIMS(KYRO_VEC_CASE)
#undef KYRO_VEC_CASE
            default:
                return hipErrorInvalidValue;
        }
    }
    if (a.plan) {
        // At most one workgroup per possible work unit, and at most kCombineMaxGrid of them
        // (each then walks several units).
        constexpr long long kCombineMaxGrid = 2048;
        const long long units = (long long)a.units * ((a.rows_cap + kCombineRows - 1) / kCombineRows);
        attn_combine_plan_kernel<kMfmaD><<<dim3((unsigned)(units < kCombineMaxGrid ? units : kCombineMaxGrid)), block, 0, stream>>>(a);
    } else if (a.splits > 1) {
        const int rpw = kThreads / (a.D / 4);
        const dim3 cgrid((unsigned)a.units, (unsigned)((a.rows_cap + rpw - 1) / rpw));
        switch (a.D) {
#define KYRO_COMBINE_CASE(DD)                                                   \
            case DD:                                                            \
                attn_combine_kernel<DD><<<cgrid, block, 0, stream>>>(a);        \
                break;
            KYRO_HEAD_DIMS(KYRO_COMBINE_CASE)
#undef KYRO_COMBINE_CASE
            default:
                return hipErrorInvalidValue;
        }
    }
    return hipGetLastError();
}

#endif  // KYRO_ATTN_HD_UNIT

}  // namespace kyro
