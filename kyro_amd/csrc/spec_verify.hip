// Fused acceptance sampling for the speculative verify step on gfx950.
//
// Replaces SpeculativeDecoder::verify_drafts (src/speculative.rs:286-339) for a whole batch, with
// the standard rejection rule (accept while u < min(1, p/q); resample from max(p - q, 0) at the
// first rejection, from p after full acceptance) and the greedy argmax-match rule of the reference
// when T <= 0. Draws are sample_token's inverse-CDF walk in index order (src/worker.rs:352-360).
//
// Five stream-ordered kernels, sized so the streaming passes spread over the whole chip:
//   1. spec_stats_kernel       grid (sequence x vocab chunk, window row): one streaming pass over
//                               the rows of the first `win` draft positions; per chunk
//                               {max, sum exp2((x - max) log2e / T)}, or {max, first argmax} for
//                               greedy rows, and the logit at the row's draft token as it streams
//                               past. Draft rows of greedy sequences and rows past k are never read.
//   2. spec_decide_kernel      one wave per sequence: the acceptance scan over the window (lane i
//                               tests u_i q_i(x_i) < p_i(x_i), a ballot finds the first rejection);
//                               a sequence that accepted every window draft is left pending, with
//                               the (row, chunk) items of its remaining rows.
//   3. spec_stats_tail_kernel  the pending sequences' remaining rows, as in 1, over a fixed grid.
//   4. spec_resample_kernel    grid (sequence x vocab chunk): a pending sequence's scan is finished
//                               here (every workgroup; the chunk-0 one stores the outputs), then
//                               each workgroup sums the residual (and p) mass of its chunk of the
//                               row to resample.
//   5. spec_pick_kernel        one workgroup per sequence: locates the chunk holding u * total with
//                               a block scan of the chunk sums, then walks that chunk in index order.
// The draw stays a launch of its own: handing the chunk sums to the last resample workgroup of a
// sequence instead needs a device-scope release per workgroup, which on gfx950 writes back the
// XCD's L2 (buffer_wbl2), and that took the sampler from 73 to 166 µs.
// Right after the streaming pass every dependent global round trip costs microseconds (cold
// caches and translations), so each kernel issues all loads that do not depend on another load
// at entry, and acceptance is recomputed per workgroup rather than handed over by a launch.
#include "common.hpp"
#include "kernels.hpp"

namespace kyro {
namespace {

constexpr int kT = 256;
constexpr int kPer = kSpecChunk / kT;  // logits per thread in a chunk
// Cache policy of the window and tail passes' logit loads (kLoadCached or kLoadStream). The
// window pass streams (bench step with caches evicted before it: 249.0 -> 246.1 us, back to back
// 233.4 -> 232.6 us); the tail pass keeps the default (streaming it too: 247.6 / 234.8 us).
#ifndef KYRO_SPEC_WINDOW_POLICY
#define KYRO_SPEC_WINDOW_POLICY 2
#endif
#ifndef KYRO_SPEC_TAIL_POLICY
#define KYRO_SPEC_TAIL_POLICY 0
#endif
constexpr int kSpecWindowPolicy = KYRO_SPEC_WINDOW_POLICY;
constexpr int kSpecTailPolicy = KYRO_SPEC_TAIL_POLICY;
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float block_max(float v, float* sh) {
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    const float r = fmaxf(fmaxf(sh[0], sh[1]), fmaxf(sh[2], sh[3]));
    __syncthreads();
    return r;
}

__device__ __forceinline__ float block_sum(float v, float* sh) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    const float r = (sh[0] + sh[1]) + (sh[2] + sh[3]);
    __syncthreads();
    return r;
}

struct ArgMax {
    float v;
    int i;
};

// Larger value wins; equal values resolve to the lower index (first maximum).
__device__ __forceinline__ ArgMax argmax_pick(ArgMax a, ArgMax b) {
    return (b.v > a.v || (b.v == a.v && b.i < a.i)) ? b : a;
}

__device__ __forceinline__ ArgMax wave_argmax(ArgMax x) {
    for (int m = 32; m >= 1; m >>= 1) {
        ArgMax o;
        o.v = __shfl_xor(x.v, m, 64);
        o.i = __shfl_xor(x.i, m, 64);
        x = argmax_pick(x, o);
    }
    return x;
}

__device__ ArgMax block_argmax(ArgMax x, float* shv, int* shi) {
    x = wave_argmax(x);
    if ((threadIdx.x & 63) == 0) {
        shv[threadIdx.x >> 6] = x.v;
        shi[threadIdx.x >> 6] = x.i;
    }
    __syncthreads();
    ArgMax r = {shv[0], shi[0]};
    for (int w = 1; w < 4; ++w) r = argmax_pick(r, ArgMax{shv[w], shi[w]});
    __syncthreads();
    return r;
}

// A chunk [v0, v1) of a row is shared by the workgroup in the strided layout: consecutive
// threads take consecutive 16-byte vectors (or floats), so every load instruction is coalesced
// (a layout where each thread owns a contiguous run issues four times the memory requests and
// measured slower in the draw). Positions past v1 load as -inf, which every consumer maps to zero
// mass; element indices are recomputed from the position, not stored.
template <bool VEC>
__device__ __forceinline__ int strided_index(int v0, int i) {
    if constexpr (VEC) return v0 + ((i >> 2) * kT + (int)threadIdx.x) * 4 + (i & 3);
    else return v0 + i * kT + (int)threadIdx.x;
}


// Every load is issued unconditionally: a position past v1 reads the chunk's last vector (or
// float) instead and is replaced by -inf afterwards (v0 < v1, and v1 is a multiple of 4 on the
// vector path). Without branches around the loads the compiler can count the loads still in
// flight exactly, so a prefetch issued before a reduction is not waited for by it.
template <bool VEC>
__device__ __forceinline__ void load_strided(const float* row, int v0, int v1, float (&x)[kPer]) {
    if constexpr (VEC) {
#pragma unroll
        for (int it = 0; it < kPer / 4; ++it) {
            const int v = v0 + (it * kT + (int)threadIdx.x) * 4;
            const float4 f = *reinterpret_cast<const float4*>(row + min(v, v1 - 4));
            const bool in = v < v1;
            x[it * 4 + 0] = in ? f.x : kNegInf;
            x[it * 4 + 1] = in ? f.y : kNegInf;
            x[it * 4 + 2] = in ? f.z : kNegInf;
            x[it * 4 + 3] = in ? f.w : kNegInf;
        }
    } else {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int v = strided_index<false>(v0, i);
            const float f = row[min(v, v1 - 1)];
            x[i] = v < v1 ? f : kNegInf;
        }
    }
}

// Word 3 of a raw buffer resource on gfx9-family parts: 32-bit data format, no swizzle, no
// thread-id addressing. With stride 0 the hardware checks each access against num_records
// (bytes) and returns zeros past it instead of faulting.
constexpr int kRawBufferWord3 = 0x00020000;

// The strided-layout load of a chunk through a buffer resource over its `bytes` bytes at
// `chunk`: the per-thread offsets do not depend on the chunk, so a loop can issue one chunk
// after another without vector address arithmetic, and positions past the chunk's end read as
// zeros (the consumer masks them, strided_index >= v1).
template <bool VEC, int POL = kLoadCached>
__device__ __forceinline__ void load_buffer(const float* chunk, int bytes, float (&x)[kPer]) {
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(chunk), (short)0, bytes, kRawBufferWord3);
    if constexpr (VEC) {
#pragma unroll
        for (int it = 0; it < kPer / 4; ++it) {
            const auto f = __builtin_amdgcn_raw_buffer_load_b128(r, (int)threadIdx.x * 16, it * kT * 16, POL);
            x[it * 4 + 0] = __uint_as_float(f[0]);
            x[it * 4 + 1] = __uint_as_float(f[1]);
            x[it * 4 + 2] = __uint_as_float(f[2]);
            x[it * 4 + 3] = __uint_as_float(f[3]);
        }
    } else {
#pragma unroll
        for (int i = 0; i < kPer; ++i)
            x[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, (int)threadIdx.x * 4, i * kT * 4, POL));
    }
}

__device__ __forceinline__ const float* target_row(const SpecArgs& a, int b, int i) {
    return a.target + ((size_t)b * (a.kmax + 1) + i) * a.V;
}
__device__ __forceinline__ const float* draft_row(const SpecArgs& a, int b, int i) {
    return a.draft + ((size_t)b * a.kmax + i) * a.V;
}

// Probability mass used by the resampling draw at one vocabulary entry.
__device__ __forceinline__ float draw_mass(const SpecPlan& pl, float t, float d, bool residual) {
    const float p = fast_exp2((t - pl.mt) * pl.c2) * pl.inv_zt;
    if (!residual) return p;
    const float q = fast_exp2((d - pl.md) * pl.c2) * pl.inv_zd;
    return fmaxf(p - q, 0.f);
}

// ------------------------------------------------------------------------- pass 1: statistics

// Statistics row `row` of sequence b (target row i is row i, draft row i is row kmax + 1 + i).
__device__ __forceinline__ const float* stats_row_base(const SpecArgs& a, int b, int row) {
    return row <= a.kmax ? target_row(a, b, row) : draft_row(a, b, row - a.kmax - 1);
}

// The draft token whose logit a statistics row captures: sampled rows below k only.
__device__ __forceinline__ uint32_t row_token(const SpecArgs& a, int b, int row, int k, float T) {
    const int pos = row <= a.kmax ? row : row - a.kmax - 1;
    return (T > 0.f && pos < k) ? a.draft_tokens[(size_t)b * a.kmax + pos] : 0xFFFFFFFFu;
}

// Reduces one chunk [v0, v1) of a statistics row (loaded into x in the strided layout) to
// {max, sum exp2((x - max) log2e / T)}, or {max, first argmax as int bits} for a greedy row
// (T <= 0). Every thread returns the result; nothing is stored.
template <bool VEC>
__device__ __forceinline__ float2 chunk_reduce(int v0, int v1, float T, const float (&x)[kPer], float* shv,
                                               int* shi) {
    if (!(T > 0.f)) {
        ArgMax best = {kNegInf, 0x7fffffff};
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int v = strided_index<VEC>(v0, i);
            if (v < v1) best = argmax_pick(best, ArgMax{x[i], v});
        }
        best = block_argmax(best, shv, shi);
        return make_float2(best.v, __int_as_float(best.i));
    }
    float m = kNegInf;
#pragma unroll
    for (int i = 0; i < kPer; ++i) m = fmaxf(m, x[i]);
    m = block_max(m, shv);
    const float c2 = kLog2e / T;
    float s = 0.f;
    if (m != kNegInf) {
#pragma unroll
        for (int i = 0; i < kPer; ++i) s += fast_exp2((x[i] - m) * c2);
    }
    s = block_sum(s, shv);
    return make_float2(m, s);
}

// Whether the draft token `tok` lies in the chunk [v0, v1) (the same answer on every thread);
// the thread holding its logit writes the logit to *dst.
template <bool VEC>
__device__ __forceinline__ bool token_logit(int v0, int v1, uint32_t tok, const float (&x)[kPer], float* dst) {
    if (!(tok >= (uint32_t)v0 && tok < (uint32_t)v1)) return false;
#pragma unroll
    for (int i = 0; i < kPer; ++i)
        if (strided_index<VEC>(v0, i) == (int)tok) *dst = x[i];
    return true;
}

// Statistics of chunk c of statistics row `row` of sequence b, stored in place, and the logit at
// the row's draft token `tok` (row_token, loaded by the caller with x) for the acceptance scan.
template <bool VEC>
__device__ __forceinline__ void chunk_stats(const SpecArgs& a, int b, int row, int c, uint32_t tok, float T,
                                            const float (&x)[kPer], float* shv, int* shi) {
    const int v0 = c * a.chunk;
    const int v1 = min(a.V, v0 + a.chunk);
    token_logit<VEC>(v0, v1, tok, x, a.gath + (size_t)b * (2 * a.kmax + 1) + row);
    const float2 st = chunk_reduce<VEC>(v0, v1, T, x, shv, shi);
    if (threadIdx.x == 0) a.stats[((size_t)b * (2 * a.kmax + 1) + row) * a.C + c] = st;
}

// Pass 1a: the rows of the first `win` draft positions (target rows 0 .. win - 1, draft rows
// 0 .. win - 1), grid (sequence x vocab chunk, row). The chunk is loaded together with the
// sequence's k and temperature and the row's draft token, so a workgroup makes one round trip;
// rows past a sequence's k, and draft rows of greedy sequences, are then dropped unreduced (at
// most 2 win rows of a sequence with k < win are read for nothing).
template <bool VEC>
__global__ __launch_bounds__(kT) void spec_stats_kernel(SpecArgs a) {
    __shared__ float shv[4];
    __shared__ int shi[4];
    const int c = blockIdx.x % a.C, b = blockIdx.x / a.C;
    const int wt = min(a.win, a.kmax + 1);  // target rows in the window
    const int y = blockIdx.y;
    const bool target = y < wt;
    if (!target && a.draft == nullptr) return;
    const int pos = target ? y : y - wt;  // draft position of the row
    const int row = target ? y : a.kmax + 1 + pos;
    const int v0 = c * a.chunk;
    const int v1 = min(a.V, v0 + a.chunk);
    float x[kPer];
    load_buffer<VEC, kSpecWindowPolicy>(stats_row_base(a, b, row) + v0, (v1 - v0) * 4, x);
    const int k = a.num_draft[b];
    const float T = a.temperature[b];
    const uint32_t tk = a.kmax > 0 ? a.draft_tokens[(size_t)b * a.kmax + min(pos, a.kmax - 1)] : 0u;
    if (k < 0 || k > a.kmax) return;  // reported by the acceptance pass
    if (target ? pos > k : (!(T > 0.f) || pos >= k)) return;
    const uint32_t tok = (T > 0.f && pos < k) ? tk : 0xFFFFFFFFu;
    if (v1 - v0 < a.chunk) {  // the row's last chunk, partial: its tail read as zeros
#pragma unroll
        for (int i = 0; i < kPer; ++i)
            if (strided_index<VEC>(v0, i) >= v1) x[i] = kNegInf;
    }
    chunk_stats<VEC>(a, b, row, c, tok, T, x, shv, shi);
}

// ------------------------------------------------------------------------- pass 2: acceptance

// Folds chunk statistic y into the running (max, sum) x of one lane.
__device__ __forceinline__ float2 fold_stats(float2 x, float2 y, float c2) {
    const float m = fmaxf(x.x, y.x);
    if (m == kNegInf) return x;
    return make_float2(m, x.y * fast_exp2((x.x - m) * c2) + y.y * fast_exp2((y.x - m) * c2));
}

struct AcceptShared {
    SpecPlan plan;
};

constexpr int kChunkGroup = 32;  // chunk statistics a lane folds per batch of loads

// Acceptance of sequence b, run by the first wave of a workgroup, in one round of loads (the
// draft tokens' logits were captured by the statistics pass). Lane r owns statistics row r
// (and row r + 64 when there are more than 64) and folds that row's chunk statistics itself;
// lane i then decides draft i, reading the rows it needs from their owners with shuffles, and a
// ballot finds the first rejection. Only the statistics of the first `avail` draft positions
// (target and draft rows 0 .. avail - 1) are read: when neither a rejection nor the end of the
// drafts falls inside them the plan is SPEC_PENDING. When `writer` is set (which needs a
// decision) the sequence's outputs are stored, and the plan in plan_out[b]. The plan for the
// draw also lands in sh.plan.
__device__ void accept_sequence(const SpecArgs& a, int b, int avail, bool writer, SpecPlan* plan_out,
                                AcceptShared& sh) {
    const int lane = threadIdx.x;
    const int R = 2 * a.kmax + 1;
    const int C = a.C;
    const float2* st = a.stats + (size_t)b * R * C;
    const int r0 = lane, r1 = lane + 64;
    auto row_ok = [&](int r) { return r < R && (r <= a.kmax ? r < avail : r - a.kmax - 1 < avail); };
    // Round 1: every load that does not depend on another load.
    const int k = a.num_draft[b];
    const float T = a.temperature[b];
    const float ures = a.u_res[b];
    uint32_t x = 0;
    float u = 0.f, tx = 0.f, dx = 0.f;
    if (lane < a.kmax) {
        x = a.draft_tokens[(size_t)b * a.kmax + lane];
        u = a.u_accept[(size_t)b * a.kmax + lane];
        tx = a.gath[(size_t)b * R + lane];               // target logit at x (sampled, lane < k)
        dx = a.gath[(size_t)b * R + a.kmax + 1 + lane];  // draft logit at x
    }
    float2 y[kChunkGroup];  // first batch of this lane's row statistics
#pragma unroll
    for (int i = 0; i < kChunkGroup; ++i)
        y[i] = (row_ok(r0) && i < C) ? st[(size_t)r0 * C + i] : make_float2(kNegInf, 0.f);

    uint32_t* toks = a.out_tokens + (size_t)b * (a.kmax + 1);
    const bool greedy = !(T > 0.f);
    int err = 0;
    if (k < 0 || k > a.kmax) err = ERR_NUM_DRAFT;
    else if (!greedy && k > 0 && a.draft == nullptr) err = ERR_NO_DRAFT;
    else if (__any(lane < k && x >= (uint32_t)a.V)) err = ERR_TOKEN;
    if (err) {
        if (writer) {
            if (lane < a.kmax) {
                if (a.out_p) a.out_p[(size_t)b * a.kmax + lane] = __builtin_nanf("");
                if (a.out_q) a.out_q[(size_t)b * a.kmax + lane] = __builtin_nanf("");
            }
            if (lane == 0) {
                latch_error(a.err, err);
                a.out_accepted[b] = 0;
                plan_out[b].mode = SPEC_DONE;
            }
            if (lane <= a.kmax) toks[lane] = 0xFFFFFFFFu;
        }
        if (lane == 0) sh.plan.mode = SPEC_DONE;
        return;
    }
    const float c2 = greedy ? 0.f : kLog2e / T;
    // Fold the owned rows. Rows that were not computed hold stale values and are never read.
    // The first batch of row r0 is already in y; later batches (more than kChunkGroup chunks, or
    // the second row of sequences with more than 64 statistics rows) are loaded here.
    auto fold_row = [&](int r, bool preloaded, float& m, float& z, ArgMax& g) {
        for (int cb = 0; cb < C; cb += kChunkGroup) {
            if (cb > 0 || !preloaded) {
#pragma unroll
                for (int i = 0; i < kChunkGroup; ++i) {
                    const int c = cb + i;
                    y[i] = (row_ok(r) && c < C) ? st[(size_t)r * C + c] : make_float2(kNegInf, 0.f);
                }
            }
            if (greedy) {
#pragma unroll
                for (int i = 0; i < kChunkGroup; ++i)
                    if (cb + i < C) g = argmax_pick(g, ArgMax{y[i].x, __float_as_int(y[i].y)});
            } else {
                float bm = kNegInf;
#pragma unroll
                for (int i = 0; i < kChunkGroup; ++i) bm = fmaxf(bm, y[i].x);
                float bs = 0.f;
#pragma unroll
                for (int i = 0; i < kChunkGroup; ++i)
                    if (y[i].x != kNegInf) bs = __builtin_fmaf(y[i].y, fast_exp2((y[i].x - bm) * c2), bs);
                const float2 f = fold_stats(make_float2(m, z), make_float2(bm, bs), c2);
                m = f.x;
                z = f.y;
            }
        }
    };
    float m0 = kNegInf, m1 = kNegInf, z0 = 0.f, z1 = 0.f;  // sampled: running max and sum
    ArgMax g0 = {kNegInf, 0x7fffffff}, g1 = g0;             // greedy: running first argmax
    fold_row(r0, true, m0, z0, g0);
    if (R > 64) fold_row(r1, false, m1, z1, g1);
    const float iz0 = z0 > 0.f ? 1.f / z0 : 0.f;
    const float iz1 = z1 > 0.f ? 1.f / z1 : 0.f;
    // Value of statistics row rho from its owner lane (every lane takes part in both shuffles).
    auto row_val = [&](float v0, float v1, int rho) {
        const float w0 = __shfl(v0, rho & 63, 64);
        const float w1 = __shfl(v1, rho & 63, 64);
        return rho < 64 ? w0 : w1;
    };
    bool accept = true;
    const int lim = min(k, avail);     // drafts whose rows were read
    const int dr = a.kmax + 1 + lane;  // this lane's draft row
    float p = __builtin_nanf(""), q = __builtin_nanf("");
    if (greedy) {
        const int top = g0.i;  // this lane's own row (lane < 64)
        accept = lane >= lim || top == (int)x;
    } else {
        const float mt = m0, izt = iz0;  // this lane's own row (lane < 64)
        const float md = row_val(m0, m1, dr), izd = row_val(iz0, iz1, dr);
        if (lane < lim) {
            p = fast_exp2((tx - mt) * c2) * izt;
            q = fast_exp2((dx - md) * c2) * izd;
            accept = !(q > 0.f) || (u * q < p);
        }
    }
    const unsigned long long rejected = __ballot(lane < lim && !accept);
    if (!rejected && k >= avail) {  // undecided: the bonus row or a later draft is outside the window
        if (lane == 0) sh.plan.mode = SPEC_PENDING;
        return;
    }
    const int j = rejected ? __ffsll((long long)rejected) - 1 : k;
    if (writer && lane <= a.kmax) toks[lane] = (lane < j) ? x : 0xFFFFFFFFu;
    if (writer && lane < a.kmax) {  // the scan stops at j: later positions are never evaluated
        if (a.out_p) a.out_p[(size_t)b * a.kmax + lane] = lane <= j ? p : __builtin_nanf("");
        if (a.out_q) a.out_q[(size_t)b * a.kmax + lane] = lane <= j ? q : __builtin_nanf("");
    }
    // Row j's statistics: the source lanes are uniform, so they are read as scalars.
    auto lane_val = [&](float v0, float v1, int rho) {
        return rho < 64 ? readlane_f(v0, rho & 63) : readlane_f(v1, rho & 63);
    };
    const int jt = greedy ? (j < 64 ? __builtin_amdgcn_readlane(g0.i, j & 63) : __builtin_amdgcn_readlane(g1.i, j & 63)) : 0;
    const float mj = lane_val(m0, m1, j), izj = lane_val(iz0, iz1, j);
    const float mdj = lane_val(m0, m1, a.kmax + 1 + j), izdj = lane_val(iz0, iz1, a.kmax + 1 + j);
    if (lane != 0) return;
    SpecPlan pl;
    pl.row = j;
    if (greedy) {
        pl.mode = SPEC_DONE;
        if (writer) toks[j] = (uint32_t)jt;
    } else {
        pl.mode = j < k ? SPEC_RESIDUAL : SPEC_PLAIN;
        pl.c2 = c2;
        pl.u = ures;
        pl.mt = mj;
        pl.inv_zt = izj;
        pl.md = j < k ? mdj : 0.f;
        pl.inv_zd = j < k ? izdj : 0.f;
    }
    if (writer) {
        a.out_accepted[b] = j;
        plan_out[b] = pl;
    }
    sh.plan = pl;
}

struct DrawShared {
    int chunk, last_chunk, pick, last;
    float rem;
    float wsum[4];
    float red[8];
    float steps[4][kPer];  // per wave, per step of the located chunk: mass
};

// Largest run of chunk sums a thread of the draw keeps in registers (vocabularies up to
// kT x kRunMax x kSpecChunk entries); longer runs are read from memory again in the walk.
constexpr int kRunMax = 4;

__device__ __forceinline__ int wave_max_int(int v) {
    for (int m = 32; m >= 1; m >>= 1) v = max(v, __shfl_xor(v, m, 64));
    return v;
}

// Inverse-CDF draw for sequence b from its chunk sums (a.csum; rv holds this thread's run of
// them when it has at most kRunMax, and my_r / my_p are the run's totals, loaded by the caller),
// run by a whole workgroup.
// Locates the chunk holding u * total with a block scan of the chunk masses (thread t owns the
// contiguous run [t * per, t * per + per), so the scan keeps index order), then walks that
// chunk in index order and stores the token at out_tokens[b][pl.row]. Every cross-thread choice
// (the first crossing, the last entry with mass) is settled within each wave by ballots and lane
// reads before one thread per wave touches the shared word: 256 contending LDS atomics on one
// address cost ~3.7 us here.
template <bool VEC>
__device__ void draw_token(const SpecArgs& a, int b, const SpecPlan& pl, DrawShared& ds, const float2 (&rv)[kRunMax],
                           float my_r, float my_p) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const float2* cs = a.csum + (size_t)b * a.C;
    const int per = (a.C + kT - 1) / kT;
    const int c0 = threadIdx.x * per;
    const int nrun = max(0, min(a.C, c0 + per) - c0);
    if (threadIdx.x == 0) {
        ds.chunk = 0x7fffffff;
        ds.last_chunk = -1;
        ds.pick = 0x7fffffff;
        ds.last = -1;
    }
    float R = wave_sum(my_r), P = wave_sum(my_p);
    if (lane == 0) {
        ds.red[wave] = R;
        ds.red[4 + wave] = P;
    }
    __syncthreads();
    R = (ds.red[0] + ds.red[1]) + (ds.red[2] + ds.red[3]);
    P = (ds.red[4] + ds.red[5]) + (ds.red[6] + ds.red[7]);
    // A residual that vanished (p == q up to rounding) falls back to drawing from p.
    const bool use_res = (pl.mode == SPEC_RESIDUAL) && R > 0.f;
    const float target = pl.u * (use_res ? R : P);
    const float mine = use_res ? my_r : my_p;
    const float inc = wave_incl_scan_f(mine);
    if (lane == 63) ds.wsum[wave] = inc;
    __syncthreads();
    float ex = inc - mine;
    for (int w2 = 0; w2 < wave; ++w2) ex += ds.wsum[w2];
    // Walk this thread's run in order: its first chunk where the running sum reaches the target
    // (when the run's total does), and its last chunk with mass.
    int my_chunk = 0x7fffffff, my_lastc = -1;
    float my_rem = 0.f;
    if (mine > 0.f) {
        const bool reach = ex + mine >= target;
        float cum = ex;
        auto step = [&](int c, float w) {
            if (w > 0.f) {
                my_lastc = c;
                if (reach && my_chunk == 0x7fffffff && cum + w >= target) {
                    my_chunk = c;
                    my_rem = target - cum;
                }
            }
            cum += w;
        };
        if (per <= kRunMax) {
#pragma unroll
            for (int i = 0; i < kRunMax; ++i)
                if (i < nrun) step(c0 + i, use_res ? rv[i].x : rv[i].y);
        } else {
            for (int i = 0; i < nrun; ++i) step(c0 + i, use_res ? cs[c0 + i].x : cs[c0 + i].y);
        }
    }
    // Runs ascend with the thread index: the wave's lowest crossing lane holds its first crossing.
    const unsigned long long hit = __ballot(my_chunk != 0x7fffffff);
    const int lastc = wave_max_int(my_lastc);
    if (lane == 0) {
        if (hit) atomicMin(&ds.chunk, __builtin_amdgcn_readlane(my_chunk, __ffsll((long long)hit) - 1));
        if (lastc >= 0) atomicMax(&ds.last_chunk, lastc);
    }
    __syncthreads();
    // The thread whose run holds the winning chunk publishes the remainder it computed.
    const int won = ds.chunk;
    if (won != 0x7fffffff) {
        if (my_chunk == won) ds.rem = my_rem;
    } else if (threadIdx.x == 0) {  // rounding left u * total past the end
        ds.chunk = ds.last_chunk < 0 ? a.C - 1 : ds.last_chunk;
        ds.rem = __builtin_huge_valf();
    }
    __syncthreads();
    const int chunk = ds.chunk;
    const float rem = ds.rem;
    const int v0 = chunk * a.chunk;
    const int v1 = min(a.V, v0 + a.chunk);
    // The chunk in the streaming passes' strided layout (every load coalesced): step q of thread
    // t covers entries EPS t .. EPS t + EPS - 1 of the step's EPS x kT consecutive entries, so the
    // index order is (step, thread, entry). The walk locates the step from the step totals, then
    // the thread from a block scan of that step, then the entry.
    constexpr int EPS = VEC ? 4 : 1;
    constexpr int NSTEP = kPer / EPS;
    float t[kPer], d[kPer], w[kPer];
    load_strided<VEC>(target_row(a, b, pl.row), v0, v1, t);
    if (use_res) load_strided<VEC>(draft_row(a, b, pl.row), v0, v1, d);
    float st[NSTEP];
    int my_last = -1;
#pragma unroll
    for (int q = 0; q < NSTEP; ++q) {
        st[q] = 0.f;
#pragma unroll
        for (int e = 0; e < EPS; ++e) {
            const int i = q * EPS + e;
            w[i] = draw_mass(pl, t[i], use_res ? d[i] : kNegInf, use_res);  // -inf past v1 -> 0
            st[q] += w[i];
            if (w[i] > 0.f) my_last = strided_index<VEC>(v0, i);  // steps ascend: the last one wins
        }
    }
#pragma unroll
    for (int q = 0; q < NSTEP; ++q) {
        const float x = wave_sum(st[q]);
        if (lane == 0) ds.steps[wave][q] = x;
    }
    {
        const int wl = wave_max_int(my_last);
        if (lane == 0 && wl >= 0) atomicMax(&ds.last, wl);
    }
    __syncthreads();
    // The step holding rem (uniform: every thread folds the same totals in the same order).
    int sel = -1;
    float rem2 = 0.f, cum = 0.f;
#pragma unroll
    for (int q = 0; q < NSTEP; ++q) {
        const float x = (ds.steps[0][q] + ds.steps[1][q]) + (ds.steps[2][q] + ds.steps[3][q]);
        if (sel < 0 && x > 0.f && cum + x >= rem) {
            sel = q;
            rem2 = rem - cum;
        }
        cum += x;
    }
    if (sel >= 0) {  // uniform
        float mine = 0.f;
#pragma unroll
        for (int q = 0; q < NSTEP; ++q) mine = q == sel ? st[q] : mine;
        const float inc2 = wave_incl_scan_f(mine);
        if (lane == 63) ds.wsum[wave] = inc2;
        __syncthreads();
        float ex2 = inc2 - mine;
        for (int w2 = 0; w2 < wave; ++w2) ex2 += ds.wsum[w2];
        const bool cand = ex2 < rem2 && ex2 + mine >= rem2;
        int pick = -1, last = -1;
        if (cand) {
            float c = ex2;
#pragma unroll
            for (int q = 0; q < NSTEP; ++q) {
                if (q != sel) continue;
#pragma unroll
                for (int e = 0; e < EPS; ++e) {
                    const int i = q * EPS + e;
                    if (w[i] > 0.f) {
                        last = strided_index<VEC>(v0, i);
                        c += w[i];
                        if (pick < 0 && c >= rem2) pick = last;
                    }
                }
            }
        }
        // Within step sel the entries ascend with the thread index: the wave's lowest candidate.
        const unsigned long long cl = __ballot(cand);
        if (cl) {
            const int l = __ffsll((long long)cl) - 1;
            const int v = __builtin_amdgcn_readlane(pick >= 0 ? pick : last, l);
            if (lane == 0) atomicMin(&ds.pick, v);
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int v = ds.pick != 0x7fffffff ? ds.pick : ds.last;
        if (v < 0) v = v1 - 1;
        a.out_tokens[(size_t)b * (a.kmax + 1) + pl.row] = (uint32_t)v;
    }
}

// Pass 2: acceptance over the window, one wave per sequence. A decided sequence gets its outputs
// and its draw plan here. An undecided one (every draft in the window accepted, more drafts or
// the bonus row beyond it) is marked SPEC_PENDING, with the (row, chunk) items of its remaining
// rows for the next pass: the scan of speculative.rs:315-323 stops at the first rejection, so
// rows after it are never needed.
__global__ __launch_bounds__(64) void spec_decide_kernel(SpecArgs a) {
    __shared__ AcceptShared acc;
    const int b = blockIdx.x;
    accept_sequence(a, b, a.win, true, a.plan, acc);
    if (threadIdx.x != 0) return;
    if (acc.plan.mode != SPEC_PENDING) {
        a.tail[b] = make_int2(0, 0);
        return;
    }
    const int k = a.num_draft[b];  // in [win, kmax]: the scan checked it
    const bool greedy = !(a.temperature[b] > 0.f);
    const int nt = k - a.win + 1;             // target rows win .. k
    const int nd = greedy ? 0 : k - a.win;    // draft rows win .. k - 1
    a.tail[b] = make_int2((nt + nd) * a.C, nt | (greedy ? 1 << 16 : 0));
    a.plan[b].mode = SPEC_PENDING;
}

// Pass 3: the remaining rows of the pending sequences, spread evenly over a fixed grid. Every
// workgroup scans the per-sequence item counts into LDS, then takes items blockIdx.x,
// blockIdx.x + gridDim.x, ... (item -> sequence by the scan, -> row and chunk by division),
// loading the next item before reducing the current one.
template <bool VEC>
__global__ __launch_bounds__(kT) void spec_stats_tail_kernel(SpecArgs a) {
    __shared__ int s_pre[kMaxLazyBatch + 1];  // exclusive prefix of the item counts
    __shared__ int s_info[kMaxLazyBatch];     // target rows left | greedy << 16
    __shared__ int s_wsum[4];
    __shared__ float shv[4];
    __shared__ int shi[4];
    __shared__ float s_tok[2];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    constexpr int kTiles = kMaxLazyBatch / kT;
    int2 ti[kTiles];
#pragma unroll
    for (int t = 0; t < kTiles; ++t) {  // every load first, then the scan
        const int i = t * kT + (int)threadIdx.x;
        ti[t] = i < a.B ? a.tail[i] : make_int2(0, 0);
    }
    int carry = 0;
#pragma unroll
    for (int t = 0; t < kTiles; ++t) {
        if (t * kT >= a.B) break;
        const int i = t * kT + (int)threadIdx.x;
        const int inc = wave_incl_scan_i(ti[t].x);
        if (lane == 63) s_wsum[wave] = inc;
        __syncthreads();
        int before = carry;
        for (int w = 0; w < wave; ++w) before += s_wsum[w];
        if (i < a.B) {
            s_pre[i + 1] = before + inc;
            s_info[i] = ti[t].y;
        }
        carry += (s_wsum[0] + s_wsum[1]) + (s_wsum[2] + s_wsum[3]);
        __syncthreads();
    }
    if (threadIdx.x == 0) s_pre[0] = 0;
    __syncthreads();
    const int total = s_pre[a.B];
    const int step = gridDim.x;
    if ((int)blockIdx.x >= total) return;
    // This workgroup's items are blockIdx.x + j * step, j < n_items <= 64 (the host sizes the
    // grid for that). Lane j of every wave locates item j here: the sequence is the last one
    // whose prefix is <= the item (binary search), then the row and chunk within it. The loop
    // reads an item's location from lane j with readlane into scalar registers, so it needs no
    // vector temporaries that could alias a load still in flight.
    const int n_items = (total - 1 - (int)blockIdx.x) / step + 1;
    uint32_t lptr_lo, lptr_hi;  // address of the item's chunk
    int lrow, lc, lflags, ltok;
    float lT;
    {
        const int item = (int)blockIdx.x + min(lane, n_items - 1) * step;
        int lo = 0, hi = a.B - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (s_pre[mid] <= item) lo = mid;
            else hi = mid - 1;
        }
        const int local = item - s_pre[lo];
        const int info = s_info[lo];
        const int nt = info & 0xffff;  // target rows left
        const bool greedy = (info >> 16) != 0;
        const int k = nt + a.win - 1;
        const int ri = local / a.C;
        const int row = ri < nt ? a.win + ri : a.kmax + 1 + a.win + (ri - nt);
        const int pos = row <= a.kmax ? row : row - a.kmax - 1;
        const int c = local - ri * a.C;
        const int v0 = c * a.chunk;
        const uint64_t ptr = reinterpret_cast<uint64_t>(stats_row_base(a, lo, row) + v0);
        lptr_lo = (uint32_t)ptr;
        lptr_hi = (uint32_t)(ptr >> 32);
        lrow = lo * (2 * a.kmax + 1) + row;
        lc = c;
        // The row's temperature and draft token, raw: they are selected on (greedy rows take
        // T = 0, and only sampled rows below k capture a token) when the item is reduced, so the
        // first chunk loads do not wait for these two.
        lT = a.temperature[lo];
        ltok = (int)a.draft_tokens[(size_t)lo * a.kmax + min(pos, a.kmax - 1)];
        lflags = (int)!greedy | ((int)(pos < k) << 1);
    }
    struct Item {
        int j;     // index of the item within this workgroup's items (its lane)
        int r, c;  // statistics row (sequence * (2 kmax + 1) + row) and chunk
    };
    // The loop issues nothing but an item's chunk loads, unconditionally (the prefetch past the
    // last item re-loads the last one, and is dropped), from scalar addresses and fixed
    // per-thread offsets, into registers that stay raw until the item is reduced: with no branch
    // around a load, no vector address arithmetic and no select on loaded values, the wait
    // before an item's reduction leaves the next item's loads in flight.
    auto load_item = [&](int j, Item& m, float (&x)[kPer]) {
        j = min(j, n_items - 1);
        const uint64_t ptr = (uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)lptr_lo, j) |
                             ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)lptr_hi, j) << 32);
        m.j = j;
        m.r = __builtin_amdgcn_readlane(lrow, j);
        m.c = __builtin_amdgcn_readlane(lc, j);
        const int v0 = m.c * a.chunk;
        load_buffer<VEC, kSpecTailPolicy>(reinterpret_cast<const float*>(ptr), (min(a.V, v0 + a.chunk) - v0) * 4, x);
    };
    // Results are not stored inside the loop: a store there is counted with the loads, and a wait
    // for it (before its data registers are reused) would also wait for the prefetch issued
    // before it. Thread `held` (= the item's j < 64) keeps the item's statistics (and draft-token
    // logit) in registers instead; they are stored after the loop.
    float2 res = make_float2(0.f, 0.f);
    size_t res_at = 0;
    int g_at = -1;
    float gval = 0.f;
    int held = 0, parity = 0;
    auto flush = [&]() {
        if ((int)threadIdx.x < held) {
            a.stats[res_at] = res;
            if (g_at >= 0) a.gath[g_at] = gval;
        }
        held = 0;
    };
    auto reduce_item = [&](const Item& m, float (&x)[kPer]) {
        const int v0 = m.c * a.chunk;
        const int v1 = min(a.V, v0 + a.chunk);
        if (v1 - v0 < a.chunk) {  // the row's last chunk, partial: its tail read as zeros
#pragma unroll
            for (int i = 0; i < kPer; ++i)
                if (strided_index<VEC>(v0, i) >= v1) x[i] = kNegInf;
        }
        const int fl = __builtin_amdgcn_readlane(lflags, m.j);
        const float T = (fl & 1) ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lT), m.j)) : 0.f;
        const uint32_t tok = fl == 3 ? (uint32_t)__builtin_amdgcn_readlane(ltok, m.j) : 0xFFFFFFFFu;
        // s_tok alternates between two slots: the barriers inside the next item's reduction
        // separate this item's read from the write two items later.
        const bool has_tok = token_logit<VEC>(v0, v1, tok, x, &s_tok[parity]);
        const float2 st = chunk_reduce<VEC>(v0, v1, T, x, shv, shi);  // its barriers publish s_tok
        if ((int)threadIdx.x == held) {
            res = st;
            res_at = (size_t)m.r * a.C + m.c;
            g_at = has_tok ? m.r : -1;
            gval = has_tok ? s_tok[parity] : 0.f;
        }
        parity ^= 1;
        ++held;
    };
    float xa[kPer], xb[kPer];
    Item ma, mb;
    int j = 0;
    load_item(0, ma, xa);
    while (true) {
        load_item(j + 1, mb, xb);
        reduce_item(ma, xa);
        if (++j >= n_items) break;
        load_item(j + 1, ma, xa);
        reduce_item(mb, xb);
        if (++j >= n_items) break;
    }
    flush();
}

// Residual (and p) mass of one chunk of the row to resample. The plan comes from the window's
// scan; a sequence that was pending repeats the scan over all its rows here (wave 0, in every
// chunk workgroup; the chunk-0 workgroup stores the outputs).
// EAGER: every row was read by the statistics pass and no decide pass ran; every workgroup runs
// the whole acceptance scan itself (one round of loads, as the decide pass would), the chunk-0
// one stores the outputs and the plan in plan[b], which no other workgroup of this launch reads.
template <bool VEC, bool EAGER>
__global__ __launch_bounds__(kT) void spec_resample_kernel(SpecArgs a) {
    __shared__ AcceptShared acc;
    __shared__ float sh[4];
    const int c = blockIdx.x % a.C, b = blockIdx.x / a.C;
    if (threadIdx.x < 64) {
        if constexpr (EAGER) {
            accept_sequence(a, b, a.kmax + 1, c == 0, a.plan, acc);
        } else {
            const SpecPlan pl = a.plan[b];
            // plan[b] is only read here; the full scan's plan goes to plan_tail.
            if (pl.mode == SPEC_PENDING) accept_sequence(a, b, a.kmax + 1, c == 0, a.plan_tail, acc);
            else if (threadIdx.x == 0) acc.plan = pl;
        }
    }
    __syncthreads();
    const SpecPlan pl = acc.plan;
    if (pl.mode == SPEC_DONE) return;
    const bool residual = pl.mode == SPEC_RESIDUAL;
    const int v0 = c * a.chunk;
    const int v1 = min(a.V, v0 + a.chunk);
    float t[kPer], d[kPer];
    load_strided<VEC>(target_row(a, b, pl.row), v0, v1, t);
    if (residual) load_strided<VEC>(draft_row(a, b, pl.row), v0, v1, d);
    float sr = 0.f, sp = 0.f;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {  // positions past v1 hold -inf: zero mass
        const float p = fast_exp2((t[i] - pl.mt) * pl.c2) * pl.inv_zt;
        sp += p;
        if (residual) sr += fmaxf(p - fast_exp2((d[i] - pl.md) * pl.c2) * pl.inv_zd, 0.f);
    }
    sr = block_sum(sr, sh);
    sp = block_sum(sp, sh);
    if (threadIdx.x == 0) a.csum[(size_t)b * a.C + c] = make_float2(sr, sp);
}

// ------------------------------------------------------------------------------- pass 3: draw

template <bool VEC>
__global__ __launch_bounds__(kT) void spec_pick_kernel(SpecArgs a) {
    __shared__ DrawShared ds;
    const int b = blockIdx.x;
    // The chunk sums and the plan are independent loads: issue both before using either.
    const float2* cs = a.csum + (size_t)b * a.C;
    const int per = (a.C + kT - 1) / kT;
    const int c0 = threadIdx.x * per;
    const int nrun = max(0, min(a.C, c0 + per) - c0);
    float2 rv[kRunMax];
    float my_r = 0.f, my_p = 0.f;
    if (per <= kRunMax) {
#pragma unroll
        for (int i = 0; i < kRunMax; ++i) rv[i] = i < nrun ? cs[c0 + i] : make_float2(0.f, 0.f);
    }
    const SpecPlan p0 = a.plan[b], p1 = a.plan_tail[b];
    if (per <= kRunMax) {
#pragma unroll
        for (int i = 0; i < kRunMax; ++i) {
            my_r += rv[i].x;
            my_p += rv[i].y;
        }
    } else {
        for (int i = 0; i < nrun; ++i) {
            const float2 w = cs[c0 + i];
            my_r += w.x;
            my_p += w.y;
        }
    }
    const SpecPlan pl = p0.mode == SPEC_PENDING ? p1 : p0;
    if (pl.mode == SPEC_DONE) return;
    draw_token<VEC>(a, b, pl, ds, rv, my_r, my_p);
}

}  // namespace

hipError_t launch_spec_verify(const SpecArgs& a, hipStream_t stream) {
    if (a.B == 0) return hipSuccess;
    // Window rows: target rows 0 .. min(win, kmax + 1) - 1, draft rows 0 .. min(win, kmax) - 1.
    const dim3 wgrid(a.C * a.B, min(a.win, a.kmax + 1) + min(a.win, a.kmax));
    // Every row in the first pass (the window covers the drafts and the bonus row): no decide
    // pass; the resample pass runs the acceptance scan in each workgroup (four launches to three).
    const bool eager = a.win > a.kmax;
    auto run = [&](auto vec) {
        constexpr bool V4 = decltype(vec)::value;
        spec_stats_kernel<V4><<<wgrid, kT, 0, stream>>>(a);
        if (eager) {
            spec_resample_kernel<V4, true><<<dim3(a.C * a.B), kT, 0, stream>>>(a);
        } else {
            spec_decide_kernel<<<dim3(a.B), 64, 0, stream>>>(a);
            spec_stats_tail_kernel<V4><<<dim3(a.tail_wgs), kT, 0, stream>>>(a);
            spec_resample_kernel<V4, false><<<dim3(a.C * a.B), kT, 0, stream>>>(a);
        }
        spec_pick_kernel<V4><<<dim3(a.B), kT, 0, stream>>>(a);
    };
    if (a.vec4) run(std::true_type{});
    else run(std::false_type{});
    return hipGetLastError();
}

}  // namespace kyro
