// Fused acceptance sampling for the speculative verify step on gfx950.
//
// Replaces SpeculativeDecoder::verify_drafts (src/speculative.rs:286-339) for a whole batch, with
// the north-star rejection rule (accept while u < min(1, p/q); resample from max(p - q, 0) at the
// first rejection, from p after full acceptance) and the greedy argmax-match rule of the reference
// when T <= 0. Draws are sample_token's inverse-CDF walk in index order (src/worker.rs:352-360).
//
// Four stream-ordered kernels, sized so the dominant pass spreads over the whole chip:
//   1. spec_stats_kernel      grid (sequence x vocab chunk, row): one streaming pass over every
//                              needed logit row; per chunk {max, sum exp2((x - max) log2e / T)},
//                              or {max, first argmax} for greedy rows. Draft rows of greedy
//                              sequences and rows past a sequence's k are never read.
//   2. spec_accept_kernel     one wave per sequence: merges the chunk statistics, evaluates
//                              u_i q_i(x_i) < p_i(x_i) in lane i and finds the first rejection
//                              with a ballot; greedy sequences finish here.
//   3. spec_resample_kernel   grid (sequence x vocab chunk): residual (and p) mass per chunk of the
//                              one row that is resampled.
//   4. spec_pick_kernel       one workgroup per sequence: locates the chunk holding u * total,
//                              then walks that chunk in index order with a block scan.
#include "common.hpp"
#include "kernels.hpp"

namespace kyro {
namespace {

constexpr int kT = 256;
constexpr int kPer = kSpecChunk / kT;  // logits per thread in a chunk
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

__device__ ArgMax block_argmax(ArgMax x, float* shv, int* shi) {
    for (int m = 32; m >= 1; m >>= 1) {
        ArgMax o;
        o.v = __shfl_xor(x.v, m, 64);
        o.i = __shfl_xor(x.i, m, 64);
        x = argmax_pick(x, o);
    }
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

// Loads this thread's share of chunk [v0, v1) of a row: strided (coalesced) layout.
__device__ __forceinline__ void load_chunk_strided(const float* row, int v0, int v1, int vec4,
                                                   float (&x)[kPer], int (&idx)[kPer]) {
    if (vec4) {
#pragma unroll
        for (int it = 0; it < kPer / 4; ++it) {
            const int v = v0 + (it * kT + (int)threadIdx.x) * 4;
            float4 f = make_float4(kNegInf, kNegInf, kNegInf, kNegInf);
            if (v < v1) f = *reinterpret_cast<const float4*>(row + v);
            x[it * 4 + 0] = f.x;
            x[it * 4 + 1] = f.y;
            x[it * 4 + 2] = f.z;
            x[it * 4 + 3] = f.w;
#pragma unroll
            for (int e = 0; e < 4; ++e) idx[it * 4 + e] = (v < v1) ? v + e : -1;
        }
    } else {
#pragma unroll
        for (int it = 0; it < kPer; ++it) {
            const int v = v0 + it * kT + (int)threadIdx.x;
            x[it] = (v < v1) ? row[v] : kNegInf;
            idx[it] = (v < v1) ? v : -1;
        }
    }
}

// Loads a contiguous run of kPer logits per thread (index order preserved within the thread).
__device__ __forceinline__ void load_chunk_contig(const float* row, int v0, int v1, int vec4,
                                                  float (&x)[kPer], int (&idx)[kPer]) {
    const int t0 = v0 + (int)threadIdx.x * kPer;
    if (vec4) {
#pragma unroll
        for (int it = 0; it < kPer / 4; ++it) {
            const int v = t0 + it * 4;
            float4 f = make_float4(kNegInf, kNegInf, kNegInf, kNegInf);
            if (v < v1) f = *reinterpret_cast<const float4*>(row + v);
            x[it * 4 + 0] = f.x;
            x[it * 4 + 1] = f.y;
            x[it * 4 + 2] = f.z;
            x[it * 4 + 3] = f.w;
#pragma unroll
            for (int e = 0; e < 4; ++e) idx[it * 4 + e] = (v < v1) ? v + e : -1;
        }
    } else {
#pragma unroll
        for (int it = 0; it < kPer; ++it) {
            const int v = t0 + it;
            x[it] = (v < v1) ? row[v] : kNegInf;
            idx[it] = (v < v1) ? v : -1;
        }
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

__global__ __launch_bounds__(kT) void spec_stats_kernel(SpecArgs a) {
    __shared__ float shv[4];
    __shared__ int shi[4];
    const int c = blockIdx.x % a.C, b = blockIdx.x / a.C, row = blockIdx.y;
    const int k = a.num_draft[b];
    if (k < 0 || k > a.kmax) return;  // reported by spec_accept_kernel
    const float T = a.temperature[b];
    const bool greedy = !(T > 0.f);
    const float* base;
    if (row <= a.kmax) {
        if (row > k) return;
        base = target_row(a, b, row);
    } else {
        const int i = row - a.kmax - 1;
        if (greedy || i >= k || a.draft == nullptr) return;
        base = draft_row(a, b, i);
    }
    const int v0 = c * a.chunk;
    const int v1 = min(a.V, v0 + a.chunk);
    float x[kPer];
    int idx[kPer];
    load_chunk_strided(base, v0, v1, a.vec4, x, idx);
    float2* out = a.stats + ((size_t)b * (2 * a.kmax + 1) + row) * a.C + c;
    if (greedy) {
        ArgMax best = {kNegInf, 0x7fffffff};
#pragma unroll
        for (int i = 0; i < kPer; ++i)
            if (idx[i] >= 0) best = argmax_pick(best, ArgMax{x[i], idx[i]});
        best = block_argmax(best, shv, shi);
        if (threadIdx.x == 0) *out = make_float2(best.v, __int_as_float(best.i));
        return;
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
    if (threadIdx.x == 0) *out = make_float2(m, s);
}

// Merges the per-chunk {max, sum} of one row into {max, 1 / sum}.
__device__ __forceinline__ void merge_row(const float2* st, int C, float c2, float& m, float& inv_z) {
    m = kNegInf;
    for (int c = 0; c < C; ++c) m = fmaxf(m, st[c].x);
    float z = 0.f;
    if (m != kNegInf)
        for (int c = 0; c < C; ++c) z += st[c].y * fast_exp2((st[c].x - m) * c2);
    inv_z = z > 0.f ? 1.f / z : 0.f;
}

__device__ __forceinline__ int merge_argmax(const float2* st, int C) {
    ArgMax best = {st[0].x, __float_as_int(st[0].y)};
    for (int c = 1; c < C; ++c) best = argmax_pick(best, ArgMax{st[c].x, __float_as_int(st[c].y)});
    return best.i;
}

__global__ __launch_bounds__(64) void spec_accept_kernel(SpecArgs a) {
    const int b = blockIdx.x;
    const int lane = threadIdx.x;
    const int k = a.num_draft[b];
    uint32_t* toks = a.out_tokens + (size_t)b * (a.kmax + 1);
    SpecPlan* plan = a.plan + b;
    if (lane < a.kmax) {
        if (a.out_p) a.out_p[(size_t)b * a.kmax + lane] = __builtin_nanf("");
        if (a.out_q) a.out_q[(size_t)b * a.kmax + lane] = __builtin_nanf("");
    }
    if (k < 0 || k > a.kmax) {
        if (lane == 0) {
            latch_error(a.err, ERR_NUM_DRAFT);
            a.out_accepted[b] = 0;
            plan->mode = SPEC_DONE;
        }
        if (lane <= a.kmax) toks[lane] = 0xFFFFFFFFu;
        return;
    }
    const float T = a.temperature[b];
    const bool greedy = !(T > 0.f);
    if (!greedy && k > 0 && a.draft == nullptr) {  // sampled drafts need draft logits
        if (lane == 0) {
            latch_error(a.err, ERR_NO_DRAFT);
            a.out_accepted[b] = 0;
            plan->mode = SPEC_DONE;
        }
        if (lane <= a.kmax) toks[lane] = 0xFFFFFFFFu;
        return;
    }
    const float c2 = greedy ? 0.f : kLog2e / T;
    const float2* st = a.stats + (size_t)b * (2 * a.kmax + 1) * a.C;
    bool accept = true, bad = false;
    uint32_t x = 0;
    if (lane < k) {
        x = a.draft_tokens[(size_t)b * a.kmax + lane];
        if (x >= (uint32_t)a.V) {
            bad = true;
        } else if (greedy) {
            accept = merge_argmax(st + (size_t)lane * a.C, a.C) == (int)x;
        } else {
            float mt, izt, md, izd;
            merge_row(st + (size_t)lane * a.C, a.C, c2, mt, izt);
            merge_row(st + (size_t)(a.kmax + 1 + lane) * a.C, a.C, c2, md, izd);
            const float p = fast_exp2((target_row(a, b, lane)[x] - mt) * c2) * izt;
            const float q = fast_exp2((draft_row(a, b, lane)[x] - md) * c2) * izd;
            const float u = a.u_accept[(size_t)b * a.kmax + lane];
            accept = !(q > 0.f) || (u * q < p);
            if (a.out_p) a.out_p[(size_t)b * a.kmax + lane] = p;
            if (a.out_q) a.out_q[(size_t)b * a.kmax + lane] = q;
        }
    }
    if (__any(bad)) {
        if (lane == 0) {
            latch_error(a.err, ERR_TOKEN);
            a.out_accepted[b] = 0;
            plan->mode = SPEC_DONE;
        }
        if (lane <= a.kmax) toks[lane] = 0xFFFFFFFFu;
        return;
    }
    const unsigned long long rejected = __ballot(lane < k && !accept);
    const int j = rejected ? __ffsll((long long)rejected) - 1 : k;
    if (lane <= a.kmax) toks[lane] = (lane < j) ? x : 0xFFFFFFFFu;
    if (lane != 0) return;
    a.out_accepted[b] = j;
    if (greedy) {
        toks[j] = (uint32_t)merge_argmax(st + (size_t)j * a.C, a.C);
        plan->mode = SPEC_DONE;
        return;
    }
    SpecPlan pl;
    pl.mode = j < k ? SPEC_RESIDUAL : SPEC_PLAIN;
    pl.row = j;
    pl.c2 = c2;
    pl.u = a.u_res[b];
    merge_row(st + (size_t)j * a.C, a.C, c2, pl.mt, pl.inv_zt);
    pl.md = 0.f;
    pl.inv_zd = 0.f;
    if (j < k) merge_row(st + (size_t)(a.kmax + 1 + j) * a.C, a.C, c2, pl.md, pl.inv_zd);
    *plan = pl;
}

__global__ __launch_bounds__(kT) void spec_resample_kernel(SpecArgs a) {
    __shared__ float sh[4];
    const int c = blockIdx.x % a.C, b = blockIdx.x / a.C;
    const SpecPlan pl = a.plan[b];
    if (pl.mode == SPEC_DONE) return;
    const bool residual = pl.mode == SPEC_RESIDUAL;
    const int v0 = c * a.chunk;
    const int v1 = min(a.V, v0 + a.chunk);
    float t[kPer], d[kPer];
    int idx[kPer];
    load_chunk_strided(target_row(a, b, pl.row), v0, v1, a.vec4, t, idx);
    if (residual) load_chunk_strided(draft_row(a, b, pl.row), v0, v1, a.vec4, d, idx);
    float sr = 0.f, sp = 0.f;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        if (idx[i] < 0) continue;
        const float p = fast_exp2((t[i] - pl.mt) * pl.c2) * pl.inv_zt;
        sp += p;
        if (residual) sr += fmaxf(p - fast_exp2((d[i] - pl.md) * pl.c2) * pl.inv_zd, 0.f);
    }
    sr = block_sum(sr, sh);
    sp = block_sum(sp, sh);
    if (threadIdx.x == 0) a.csum[(size_t)b * a.C + c] = make_float2(sr, sp);
}

__global__ __launch_bounds__(kT) void spec_pick_kernel(SpecArgs a) {
    __shared__ int s_chunk;
    __shared__ float s_rem;
    __shared__ int s_use_res;
    __shared__ float s_wsum[4];
    __shared__ int s_pick;
    __shared__ int s_last;
    const int b = blockIdx.x;
    const SpecPlan pl = a.plan[b];
    if (pl.mode == SPEC_DONE) return;
    const float2* cs = a.csum + (size_t)b * a.C;
    if (threadIdx.x == 0) {
        float R = 0.f, P = 0.f;
        for (int c = 0; c < a.C; ++c) {
            R += cs[c].x;
            P += cs[c].y;
        }
        const int use_res = (pl.mode == SPEC_RESIDUAL) && R > 0.f;
        const float target = pl.u * (use_res ? R : P);
        float cum = 0.f;
        int chunk = -1, last_pos = -1;
        float rem = 0.f;
        for (int c = 0; c < a.C; ++c) {
            const float w = use_res ? cs[c].x : cs[c].y;
            if (w > 0.f) {
                last_pos = c;
                if (cum + w >= target) {
                    chunk = c;
                    rem = target - cum;
                    break;
                }
            }
            cum += w;
        }
        if (chunk < 0) {  // rounding left u * total beyond the last boundary
            chunk = last_pos < 0 ? a.C - 1 : last_pos;
            rem = __builtin_huge_valf();
        }
        s_chunk = chunk;
        s_rem = rem;
        s_use_res = use_res;
        s_pick = 0x7fffffff;
        s_last = -1;
    }
    __syncthreads();
    const int chunk = s_chunk;
    const float rem = s_rem;
    const bool residual = s_use_res != 0;
    const int v0 = chunk * a.chunk;
    const int v1 = min(a.V, v0 + a.chunk);
    float t[kPer], d[kPer], w[kPer];
    int idx[kPer];
    load_chunk_contig(target_row(a, b, pl.row), v0, v1, a.vec4, t, idx);
    if (residual) load_chunk_contig(draft_row(a, b, pl.row), v0, v1, a.vec4, d, idx);
    float ts = 0.f;
    int my_last = -1;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        w[i] = idx[i] >= 0 ? draw_mass(pl, t[i], residual ? d[i] : 0.f, residual) : 0.f;
        ts += w[i];
        if (w[i] > 0.f) my_last = idx[i];
    }
    // Exclusive scan of the per-thread sums in thread (= index) order.
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float inc = ts;
    for (int o = 1; o < 64; o <<= 1) {
        const float y = __shfl_up(inc, o, 64);
        if (lane >= o) inc += y;
    }
    if (lane == 63) s_wsum[wave] = inc;
    __syncthreads();
    float ex = inc - ts;
    for (int w2 = 0; w2 < wave; ++w2) ex += s_wsum[w2];
    if (ex < rem && ex + ts >= rem) {
        float cum = ex;
        int pick = my_last;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            if (w[i] > 0.f) {
                cum += w[i];
                if (cum >= rem) {
                    pick = idx[i];
                    break;
                }
            }
        }
        atomicMin(&s_pick, pick);
    }
    atomicMax(&s_last, my_last);
    __syncthreads();
    if (threadIdx.x == 0) {
        int v = s_pick != 0x7fffffff ? s_pick : s_last;
        if (v < 0) v = v1 - 1;
        a.out_tokens[(size_t)b * (a.kmax + 1) + pl.row] = (uint32_t)v;
    }
}

}  // namespace

hipError_t launch_spec_verify(const SpecArgs& a, hipStream_t stream) {
    if (a.B == 0) return hipSuccess;
    spec_stats_kernel<<<dim3(a.C * a.B, 2 * a.kmax + 1), kT, 0, stream>>>(a);
    spec_accept_kernel<<<dim3(a.B), 64, 0, stream>>>(a);
    spec_resample_kernel<<<dim3(a.C * a.B), kT, 0, stream>>>(a);
    spec_pick_kernel<<<dim3(a.B), kT, 0, stream>>>(a);
    return hipGetLastError();
}

}  // namespace kyro
