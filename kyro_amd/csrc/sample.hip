// Fused plain-decode sampling with the worker's logit processors, on gfx950.
//
// Replaces the per-request path of Worker::run_loop (src/worker.rs:141-197: logit bias, frequency
// and presence penalties, grammar mask) followed by sample_token (src/worker.rs:267-362), for a
// batch of rows at once. Per row b, with x the row's logits:
//   processed   y = ((x + bias) + penalty) + mask, the mask adding -inf to disallowed tokens
//               (grammar.rs:38-47); bias and penalty arrive as sparse per-row lists
//   T <= 0      argmax(y), first index among equal maxima (worker.rs:290-296)
//   T > 0       z = y * f32(1/T) (candle's affine for `logits / T`, worker.rs:298); top-k keeps
//               the k largest z (ties: lower index); p = exp(z - max) / sum over the kept set;
//               top-p < 1 sorts the kept set by p descending (ties: lower index), cuts after the
//               first entry whose running sum exceeds top_p, and walks the cut with r = u * its
//               mass; otherwise the walk runs in index order with r = u, or, after top-k alone,
//               in the same descending order (the reference leaves that order to
//               select_nth_unstable). The token is the first whose running sum reaches r
//               (`r -= p; if r <= 0`); when rounding leaves none: the most probable kept token
//               after top-p, the least probable kept token after top-k alone, the last index
//               otherwise (worker.rs:340-360).
//
// A batch with no processor, top-k or top-p takes one launch, sample_plain_kernel (below: a few
// workgroups a row, the last to finish combining the row's segment statistics and walking it).
// Otherwise the row is split into 4096-entry chunks so that a batch of a few rows still fills
// the chip:
//   sample_prepare_kernel  (rows with a processor; grid chunk x row) copies the row into the
//                          workspace with the mask, then the bias, then the penalty applied.
//   sample_stats_kernel    (grid chunk x row) per chunk: {max z, sum exp(z - max z)}, or the first
//                          maximum at T <= 0. Top-k / top-p rows also list the chunk's
//                          candidates: every entry at or above a threshold t chosen by block-wide
//                          counts (wave ballots, no atomics) on a grid of 1/64 nat below the
//                          chunk's max: for top-k the highest t with k entries above it, for top-p
//                          alone the lowest t whose list fits (ccap entries), or the bound below
//                          which top-p never keeps a token.
//   sample_select_kernel   (one workgroup per row) settles greedy and plain rows: the first
//                          maximum, or Z, the chunk where the running mass reaches u Z and the
//                          walk inside it. Top-k / top-p rows gather the chunks' lists into LDS.
//                          For top-k they hold the row's k largest; for top-p alone every token
//                          at or above the largest threshold. The row is then cut and walked in
//                          descending order (key descending, index ascending): up to kSortMax
//                          candidates sorted with running sums; more searched with mass
//                          histograms over the key's digits. Rows whose lists do not cover the
//                          kept set (or the top-p cut) gather candidates from the row in the same
//                          workgroup (a binned pass, then a gathering pass); what that leaves
//                          runs exact radix selects over the whole row: three passes (11 + 11 +
//                          10 bits) of mass histograms in LDS (64-bit fixed point, 2^-52
//                          resolution, so the sums do not depend on thread order), then a pass in
//                          index order for ties between equal keys.
#include <cfloat>

#include "common.hpp"
#include "kernels.hpp"

namespace kyro {
namespace {

constexpr int kRT = 1024;  // threads of the row kernel
constexpr int kRW = kRT / 64;
// Top-p alone: the most lanes a chunk's list threshold leaves above it when the skip bound lists
// too many (fewer candidates search faster; lists too short to reach the cut send the row to the
// row gather below). 96 lost the cut on the 64-row N(0, 3.5) batch; 128 kept it at 0.4 us more a
// call, 160 and 256 at 1.5 and 2.8 us more.
#ifndef KYRO_SAMPLE_P_TARGET
#define KYRO_SAMPLE_P_TARGET 112
#endif
constexpr int kBins = 2048;
static_assert(kBins >= 2 * kSampleMaxChunks, "the select pass keeps list lengths and offsets in RowShared::cnt");
constexpr int kCap = kSampleCand;            // candidates held in LDS
// Up to this many candidates are sorted (bitonic, in LDS); more are searched by mass histograms,
// whose per-level cost does not grow with the count.
constexpr int kSortMax = 512;
constexpr double kFix = 4503599627370496.0;  // 2^52: fixed-point unit of probability mass
constexpr float kLog2e = 1.4426950408889634f;
using u64 = unsigned long long;

// Unsigned key with the order of the float (larger float, larger key).
__device__ __forceinline__ uint32_t order_key(float z) {
    const uint32_t u = __float_as_uint(z);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Inclusive u64 wave scan with the DPP steps of wave_incl_scan_f (both halves move together).
__device__ __forceinline__ u64 wave_incl_scan_u64(u64 x) {
#define KYRO_STEP_U64(ctrl, rmask)                                                   \
    {                                                                                \
        const uint32_t lo = (uint32_t)KYRO_DPP((int)(uint32_t)x, ctrl, rmask);       \
        const uint32_t hi = (uint32_t)KYRO_DPP((int)(uint32_t)(x >> 32), ctrl, rmask); \
        x += ((u64)hi << 32) | lo;                                                   \
    }
    KYRO_DPP_SCAN(KYRO_STEP_U64);
#undef KYRO_STEP_U64
    return x;
}

// Wave sum: the 16-lane rows with DPP, then the four row totals read as scalars.
__device__ __forceinline__ u64 wave_sum_u64(u64 x) {
#define KYRO_RSTEP_U64(ctrl)                                                         \
    {                                                                                \
        const uint32_t lo = (uint32_t)KYRO_DPP((int)(uint32_t)x, ctrl, 0xf);         \
        const uint32_t hi = (uint32_t)KYRO_DPP((int)(uint32_t)(x >> 32), ctrl, 0xf); \
        x += ((u64)hi << 32) | lo;                                                   \
    }
    KYRO_RSTEP_U64(0xB1);   // quad_perm [1,0,3,2]
    KYRO_RSTEP_U64(0x4E);   // quad_perm [2,3,0,1]
    KYRO_RSTEP_U64(0x141);  // row_half_mirror
    KYRO_RSTEP_U64(0x140);  // row_mirror
#undef KYRO_RSTEP_U64
    auto lane_u64 = [&](int l) {
        return ((u64)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(x >> 32), l) << 32) |
               (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)x, l);
    };
    return (lane_u64(0) + lane_u64(16)) + (lane_u64(32) + lane_u64(48));
}

// Wave reductions of 32-bit values with op: the 16-lane rows with DPP, then the four row
// results read as scalars (every lane gets the same value).
template <class Op>
__device__ __forceinline__ int wave_reduce_i(int x, Op op) {
    x = op(x, KYRO_DPP(x, 0xB1, 0xf));   // quad_perm [1,0,3,2]
    x = op(x, KYRO_DPP(x, 0x4E, 0xf));   // quad_perm [2,3,0,1]
    x = op(x, KYRO_DPP(x, 0x141, 0xf));  // row_half_mirror
    x = op(x, KYRO_DPP(x, 0x140, 0xf));  // row_mirror
    return op(op(__builtin_amdgcn_readlane(x, 0), __builtin_amdgcn_readlane(x, 16)),
              op(__builtin_amdgcn_readlane(x, 32), __builtin_amdgcn_readlane(x, 48)));
}

// Wave argmax over (v, i) pairs: larger v, then lower i; every lane gets the result.
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
    auto take = [&](float ov, int oi) {
        if (ov > v || (ov == v && oi < i)) {
            v = ov;
            i = oi;
        }
    };
#define KYRO_ASTEP(ctrl) take(__int_as_float(KYRO_DPP(__float_as_int(v), ctrl, 0xf)), KYRO_DPP(i, ctrl, 0xf))
    KYRO_ASTEP(0xB1);
    KYRO_ASTEP(0x4E);
    KYRO_ASTEP(0x141);
    KYRO_ASTEP(0x140);
#undef KYRO_ASTEP
    const float v0 = readlane_f(v, 0);
    const int i0 = __builtin_amdgcn_readlane(i, 0);
    const float v16 = readlane_f(v, 16), v32 = readlane_f(v, 32), v48 = readlane_f(v, 48);
    const int i16 = __builtin_amdgcn_readlane(i, 16), i32 = __builtin_amdgcn_readlane(i, 32),
              i48 = __builtin_amdgcn_readlane(i, 48);
    v = v0;
    i = i0;
    take(v16, i16);
    take(v32, i32);
    take(v48, i48);
}

struct RowShared {
    u64 hist[kBins];
    uint32_t cnt[kBins];
    u64 cand[kCap];  // (key << 32) | ~index: descending order = key descending, index ascending
    float cum[kCap];
    u64 wsum[kRW];
    float fred[kRW];
    int ired[kRW];
    int found;       // search result: bin / element index, or -1
    u64 before;      // mass before the found bin / element
    u64 mass;        // its mass
    int count;
    int nsmall;           // members of a search's last bin, gathered for one wave to sort
    int sidx[64];
};

// Calls f(v, y[v]) for the elements this thread owns (strided over the block), with four 16-byte
// loads in flight per iteration when the row is 16-byte aligned.
template <class F>
__device__ __forceinline__ void row_for_each(const float* y, int V, bool vec4, F f) {
    const int tid = threadIdx.x;
    if (vec4) {
        const float4* p = reinterpret_cast<const float4*>(y);
        const int n4 = V >> 2;
        int i = tid;
        for (; i + 3 * kRT < n4; i += 4 * kRT) {
            const float4 q0 = p[i], q1 = p[i + kRT], q2 = p[i + 2 * kRT], q3 = p[i + 3 * kRT];
            auto four = [&](int v, const float4& q) {
                f(v, q.x);
                f(v + 1, q.y);
                f(v + 2, q.z);
                f(v + 3, q.w);
            };
            four(4 * i, q0);
            four(4 * (i + kRT), q1);
            four(4 * (i + 2 * kRT), q2);
            four(4 * (i + 3 * kRT), q3);
        }
        for (; i < n4; i += kRT) {
            const float4 q = p[i];
            f(4 * i, q.x);
            f(4 * i + 1, q.y);
            f(4 * i + 2, q.z);
            f(4 * i + 3, q.w);
        }
        for (int v = 4 * n4 + tid; v < V; v += kRT) f(v, y[v]);
    } else {
#pragma unroll 4
        for (int v = tid; v < V; v += kRT) f(v, y[v]);
    }
}

__device__ __forceinline__ float block_max_f(float v, RowShared& sh) {
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0) sh.fred[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = sh.fred[0];
    for (int w = 1; w < kRW; ++w) r = fmaxf(r, sh.fred[w]);
    __syncthreads();
    return r;
}

__device__ __forceinline__ float block_sum_f(float v, RowShared& sh) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) sh.fred[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = 0.f;
    for (int w = 0; w < kRW; ++w) r += sh.fred[w];
    __syncthreads();
    return r;
}

__device__ __forceinline__ int block_sum_i(int v, RowShared& sh) {
    v = wave_reduce_i(v, [](int x, int y) { return x + y; });
    if ((threadIdx.x & 63) == 0) sh.ired[threadIdx.x >> 6] = v;
    __syncthreads();
    int r = 0;
    for (int w = 0; w < kRW; ++w) r += sh.ired[w];
    __syncthreads();
    return r;
}

// Bits every key in [lo, hi] (each thread's range, merged over the block) shares, counted from
// the top (32 when all keys are equal), and their value: the first digit of a search over the
// candidates can start below them.
__device__ __forceinline__ void key_range_prefix(uint32_t lo, uint32_t hi, RowShared& sh, int* bits, uint64_t* prefix,
                                                 uint32_t* lo_out = nullptr) {
    lo = (uint32_t)wave_reduce_i((int)lo, [](int x, int y) { return (int)min((uint32_t)x, (uint32_t)y); });
    hi = (uint32_t)wave_reduce_i((int)hi, [](int x, int y) { return (int)max((uint32_t)x, (uint32_t)y); });
    if ((threadIdx.x & 63) == 0) {
        sh.ired[threadIdx.x >> 6] = (int)lo;
        sh.wsum[threadIdx.x >> 6] = hi;
    }
    __syncthreads();
    for (int w = 0; w < kRW; ++w) {
        lo = min(lo, (uint32_t)sh.ired[w]);
        hi = max(hi, (uint32_t)sh.wsum[w]);
    }
    __syncthreads();
    const int b = (lo >= hi) ? 32 : __clz((int)(lo ^ hi));
    *bits = b;
    *prefix = b == 0 ? 0 : (uint64_t)(lo >> (32 - b));
    if (lo_out) *lo_out = lo;
}

// First index holding the maximum of v over the block (v = -inf for no candidate).
__device__ __forceinline__ int block_argmax(float v, int i, RowShared& sh) {
    wave_argmax(v, i);
    if ((threadIdx.x & 63) == 0) {
        sh.fred[threadIdx.x >> 6] = v;
        sh.ired[threadIdx.x >> 6] = i;
    }
    __syncthreads();
    float bv = sh.fred[0];
    int bi = sh.ired[0];
    for (int w = 1; w < kRW; ++w)
        if (sh.fred[w] > bv || (sh.fred[w] == bv && sh.ired[w] < bi)) {
            bv = sh.fred[w];
            bi = sh.ired[w];
        }
    __syncthreads();
    return bi;
}

// One sampled row: the processed logits, the temperature scale and the kept-set bounds.
struct Row {
    const float* y;
    int V;
    bool vec4;
    float s;        // f32(1 / T)
    float m;        // max of z
    float z_sum;    // sum of exp(z - m) over the kept set
    // kept set (top-k): key > kk, or key == kk and index <= ki; kk = 0 keeps everything
    uint32_t kk;
    int ki;
    // nucleus (top-p cut): key > ck, or key == ck and index <= ci; ck = 0 keeps the kept set
    uint32_t ck;
    int ci;

    __device__ float z(int v) const { return y[v] * s + 0.0f; }
    __device__ bool kept(uint32_t key, int v) const { return key > kk || (key == kk && v <= ki); }
    __device__ bool in_cut(uint32_t key, int v) const { return key > ck || (key == ck && v <= ci); }
    __device__ float e(float zv) const { return fast_exp2((zv - m) * kLog2e); }
    __device__ float prob(float zv) const { return e(zv) / z_sum; }
};

__device__ __forceinline__ u64 fix_mass(float p) { return (u64)llrint((double)p * kFix); }

// Searches the elements selected by `member` in descending key order (ties: ascending index)
// for the first one whose running mass (`mass_of`) reaches theta (exceeds it when strict).
// Returns its index, or -1 when the whole set's mass falls short; *before gets the mass ahead
// of it and *mass its own.
template <class Member, class MassOf>
__device__ __forceinline__ int desc_search(const Row& r, Member member, MassOf mass_of, u64 theta, bool strict, RowShared& sh,
                           u64* before_out, u64* mass_out) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint32_t prefix = 0;
    int pbits = 0;
    u64 before = 0;
    for (int lvl = 0; lvl < 3; ++lvl) {
        const int bits = lvl < 2 ? 11 : 10;
        const int nb = 1 << bits;
        for (int i = tid; i < nb; i += kRT) sh.hist[i] = 0;
        __syncthreads();
        row_for_each(r.y, r.V, r.vec4, [&](int v, float yv) {
            const float zv = yv * r.s + 0.0f;
            const uint32_t key = order_key(zv);
            if (!member(key, v)) return;
            if (pbits > 0 && (key >> (32 - pbits)) != prefix) return;
            const uint32_t d = (key >> (32 - pbits - bits)) & (uint32_t)(nb - 1);
            const u64 m = mass_of(zv);
            if (m) atomicAdd(&sh.hist[d], m);
        });
        __syncthreads();
        // Running mass over the bins from the top: thread t owns descending positions 2t, 2t+1.
        const int j0 = 2 * tid, j1 = 2 * tid + 1;
        const u64 m0 = j0 < nb ? sh.hist[nb - 1 - j0] : 0;
        const u64 m1 = j1 < nb ? sh.hist[nb - 1 - j1] : 0;
        const u64 incl = wave_incl_scan_u64(m0 + m1);
        if (lane == 63) sh.wsum[wave] = incl;
        if (tid == 0) sh.found = -1;
        __syncthreads();
        u64 base = before;
        for (int w = 0; w < wave; ++w) base += sh.wsum[w];
        const u64 ex0 = base + incl - (m0 + m1), in0 = ex0 + m0, in1 = in0 + m1;
        auto crosses = [&](u64 ex, u64 in) { return strict ? (ex <= theta && in > theta) : (ex < theta && in >= theta); };
        if (j0 < nb && m0 && crosses(ex0, in0)) {
            sh.found = nb - 1 - j0;
            sh.before = ex0;
        } else if (j1 < nb && m1 && crosses(in0, in1)) {
            sh.found = nb - 1 - j1;
            sh.before = in0;
        }
        __syncthreads();
        const int d = sh.found;
        if (d < 0) return -1;
        before = sh.before;
        prefix = (prefix << bits) | (uint32_t)d;
        pbits += bits;
        __syncthreads();
    }
    // Equal keys: index order. Wave w scans the contiguous chunk [w L, w L + L).
    const uint32_t key_star = prefix;
    const int L = (r.V + kRW - 1) / kRW;
    const int c0 = wave * L, c1 = min(r.V, c0 + L);
    u64 part = 0;
    for (int v = c0 + lane; v < c1; v += 64) {
        const float zv = r.z(v);
        const uint32_t key = order_key(zv);
        if (key == key_star && member(key, v)) part += mass_of(zv);
    }
    part = wave_sum_u64(part);
    if (lane == 0) sh.wsum[wave] = part;
    if (tid == 0) sh.found = -1;
    __syncthreads();
    u64 wb = before;
    for (int w = 0; w < wave; ++w) wb += sh.wsum[w];
    const bool my_wave = strict ? (wb <= theta && wb + sh.wsum[wave] > theta)
                                : (wb < theta && wb + sh.wsum[wave] >= theta);
    if (my_wave) {  // exactly one wave holds the crossing
        for (int t0 = c0; t0 < c1; t0 += 64) {
            const int v = t0 + lane;
            u64 m = 0;
            if (v < c1) {
                const float zv = r.z(v);
                const uint32_t key = order_key(zv);
                if (key == key_star && member(key, v)) m = mass_of(zv);
            }
            const u64 in = wb + wave_incl_scan_u64(m);
            const u64 ex = in - m;
            const bool hit = m && (strict ? (ex <= theta && in > theta) : (ex < theta && in >= theta));
            const unsigned long long bal = __ballot(hit);
            if (bal) {
                if (lane == __ffsll((long long)bal) - 1) {
                    sh.found = v;
                    sh.before = ex;
                    sh.mass = m;
                }
                break;
            }
            wb = __shfl(in, 63, 64);
        }
    }
    __syncthreads();
    const int found = sh.found;
    *before_out = sh.before;
    *mass_out = sh.mass;
    __syncthreads();
    return found;
}

// Float value of an order_key.
__device__ __forceinline__ float key_value(uint32_t key) {
    return __uint_as_float((key & 0x80000000u) ? (key & 0x7fffffffu) : ~key);
}

// Sorts a[0, n) (n a power of two, at most kCap) into descending order. Whole block. Stages
// whose pairs lie inside one wave's segment of n / kRW entries run without a block barrier (a
// wave's LDS accesses are processed in order; the wavefront fence only keeps the compiler from
// moving them), so only strides of a segment or more pay for __syncthreads.
__device__ __forceinline__ void bitonic_desc(u64* a, int n) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int seg = max(2, n / kRW);  // entries per wave segment (a power of two)
    auto cswap = [&](int lo, int hi, int size) {
        const bool desc = (lo & size) == 0;
        const u64 x = a[lo], y = a[hi];
        if (desc ? x < y : x > y) {
            a[lo] = y;
            a[hi] = x;
        }
    };
    for (int size = 2; size <= n; size <<= 1) {
        for (int sb = __builtin_ctz((unsigned)size) - 1; sb >= 0; --sb) {  // stride = 2^sb
            const int stride = 1 << sb;
            if (2 * stride <= seg) {  // wave w: pairs [w seg / 2, (w + 1) seg / 2) = its segment
                if (wave * seg < n)
                    for (int p = lane; p < seg / 2; p += 64) {
                        const int i = wave * (seg / 2) + p;
                        cswap(((i >> sb) << (sb + 1)) + (i & (stride - 1)), ((i >> sb) << (sb + 1)) + (i & (stride - 1)) + stride, size);
                    }
                __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            } else {
                for (int i = threadIdx.x; i < (n >> 1); i += kRT)
                    cswap(((i >> sb) << (sb + 1)) + (i & (stride - 1)), ((i >> sb) << (sb + 1)) + (i & (stride - 1)) + stride, size);
                __syncthreads();
            }
        }
        if (2 * size > seg) __syncthreads();  // the next size starts with a block-wide stage
    }
}

// In-place inclusive scan of a[0, n), n <= kCap: thread t owns 8 consecutive entries.
__device__ __forceinline__ void block_scan_incl(float* a, int n, RowShared& sh) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int i0 = tid * 8;
    float loc[8];
    float run = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        run += (i0 + j < n) ? a[i0 + j] : 0.f;
        loc[j] = run;
    }
    const float incl = wave_incl_scan_f(run);
    if (lane == 63) sh.fred[wave] = incl;
    __syncthreads();
    float base = incl - run;
    for (int w = 0; w < wave; ++w) base += sh.fred[w];
#pragma unroll
    for (int j = 0; j < 8; ++j)
        if (i0 + j < n) a[i0 + j] = base + loc[j];
    __syncthreads();
}

// First i < n with c[i] >= x (> x when strict) for nondecreasing c; -1 if none. Whole block.
__device__ __forceinline__ int first_at_least(const float* c, int n, float x, bool strict, RowShared& sh) {
    if (threadIdx.x == 0) sh.found = 0x7fffffff;
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += kRT) {
        const bool ok = strict ? c[i] > x : c[i] >= x;
        const bool prev = i > 0 && (strict ? c[i - 1] > x : c[i - 1] >= x);
        if (ok && !prev) atomicMin(&sh.found, i);
    }
    __syncthreads();
    const int f = sh.found;
    __syncthreads();
    return f == 0x7fffffff ? -1 : f;
}

// A search's position after its histogram levels: the found bin's prefix (pbits fixed high bits
// of (key << 32) | ~index), the mass ahead of the bin, and for the first level its bin and
// width, whose histogram sh.hist / sh.cnt still holds when levels == 1.
struct SearchState {
    uint64_t prefix;
    int pbits;
    u64 before;
    int levels;
    int d1, bits1;
    u64 before1;
};

// The bin (of nb in sh.hist, mass before it `before`) where the running mass from the top bin
// down first reaches theta (exceeds it when strict): -1 if none. *before_bin gets the mass ahead
// of it and *count its members (sh.cnt). Whole block.
__device__ __forceinline__ int bin_scan(int nb, u64 before, u64 theta, bool strict, RowShared& sh, u64* before_bin,
                                        int* count) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // Running mass over the bins from the top: thread t owns descending positions 2t, 2t+1.
    const int j0 = 2 * tid, j1 = 2 * tid + 1;
    const u64 m0 = j0 < nb ? sh.hist[nb - 1 - j0] : 0;
    const u64 m1 = j1 < nb ? sh.hist[nb - 1 - j1] : 0;
    const u64 incl = wave_incl_scan_u64(m0 + m1);
    if (lane == 63) sh.wsum[wave] = incl;
    if (tid == 0) sh.found = -1;
    __syncthreads();
    u64 base = before;
    for (int w = 0; w < wave; ++w) base += sh.wsum[w];
    const u64 ex0 = base + incl - (m0 + m1), in0 = ex0 + m0, in1 = in0 + m1;
    auto crosses = [&](u64 ex, u64 in) { return strict ? (ex <= theta && in > theta) : (ex < theta && in >= theta); };
    if (j0 < nb && m0 && crosses(ex0, in0)) {
        sh.found = nb - 1 - j0;
        sh.before = ex0;
        sh.count = (int)sh.cnt[nb - 1 - j0];
    } else if (j1 < nb && m1 && crosses(in0, in1)) {
        sh.found = nb - 1 - j1;
        sh.before = in0;
        sh.count = (int)sh.cnt[nb - 1 - j1];
    }
    __syncthreads();
    const int d = sh.found;
    *before_bin = sh.before;
    *count = sh.count;
    __syncthreads();
    return d;
}

// The members of the bin named by (prefix, pbits) with mass, at most 64, ranked in wave 0 (each
// lane counts the members above its own, broadcast LDS reads) and summed in that order from
// `before`; the first whose running mass reaches theta (exceeds it when strict). Scratch in
// sh.cum, so that sh.hist survives. Returns its index, or -1.
template <class Member, class MassOf>
__device__ __forceinline__ int bin_resolve(int n, Member member, MassOf mass_of, u64 theta, bool strict, RowShared& sh,
                                           uint64_t prefix, int pbits, u64 before, u64* before_out, u64* mass_out,
                                           uint32_t* key_out) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid == 0) sh.nsmall = 0;
    __syncthreads();
    for (int i = tid; i < n; i += kRT) {
        const u64 c = sh.cand[i];
        const uint32_t key = (uint32_t)(c >> 32);
        if ((c >> (64 - pbits)) == prefix && member(key, (int)~(uint32_t)c) && mass_of(key_value(key))) {
            const int slot = atomicAdd(&sh.nsmall, 1);
            if (slot < 64) sh.sidx[slot] = i;
        }
    }
    __syncthreads();
    if (wave == 0) {
        u64* scr = reinterpret_cast<u64*>(sh.cum);
        const int ns = min(sh.nsmall, 64);
        u64 c = 0, m = 0;
        if (lane < ns) {
            c = sh.cand[sh.sidx[lane]];
            m = mass_of(key_value((uint32_t)(c >> 32)));
            scr[lane] = c;
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        __builtin_amdgcn_wave_barrier();
        int rank = 0;
        for (int j = 0; j < ns; ++j) rank += scr[j] > c ? 1 : 0;
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        __builtin_amdgcn_wave_barrier();
        if (lane < ns) {
            scr[64 + rank] = m;
            scr[128 + rank] = c;
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        __builtin_amdgcn_wave_barrier();
        u64 in = before;
        for (int j = 0; j <= lane && j < ns; ++j) in += scr[64 + j];
        m = lane < ns ? scr[64 + lane] : 0;
        c = lane < ns ? scr[128 + lane] : 0;
        const u64 ex = in - m;
        const bool hit = m && (strict ? (ex <= theta && in > theta) : (ex < theta && in >= theta));
        const unsigned long long bal = __ballot(hit);
        if (bal && lane == __ffsll((long long)bal) - 1) {
            sh.found = (int)~(uint32_t)c;
            sh.before = ex;
            sh.mass = m;
            sh.wsum[0] = c >> 32;
        } else if (!bal && lane == 0) {
            sh.found = -1;
        }
    }
    __syncthreads();
    const int found = sh.found;
    *key_out = (uint32_t)sh.wsum[0];
    *mass_out = sh.mass;
    *before_out = sh.before;
    __syncthreads();
    return found;
}

// desc_search over the row's candidate list in LDS instead of the row: entries sh.cand[0, n),
// (key << 32) | ~index. The same order (key descending, then index ascending), the same masses
// and the same crossing rule, found by mass histograms over the key's digits (up to 11 bits each,
// from below the pbits0 top bits every candidate shares, prefix0) and, when several members share
// the found key, over ~index's digits (descending ~index is ascending index). Starting below the
// shared bits spreads the first level's candidates over its bins: a top-p row's candidates fall
// in a handful of 11-bit top bins, and their atomic adds to those few bins serialise. Once the
// found bin holds at most 64 members, bin_resolve settles it. Returns the index, or -1 when the
// members' mass falls short of theta; *key_out gets its key, *st the levels' state.
template <class Member, class MassOf>
__device__ __forceinline__ int cand_search(int n, Member member, MassOf mass_of, u64 theta, bool strict, RowShared& sh,
                                           u64* before_out, u64* mass_out, uint32_t* key_out, int pbits0 = 0,
                                           uint64_t prefix0 = 0, SearchState* st = nullptr) {
    const int tid = threadIdx.x;
    uint64_t prefix = prefix0;
    int pbits = pbits0;
    u64 before = 0;
    bool few = false;
    SearchState s{};
    for (int lvl = 0; lvl < 7 && !few && pbits < 64; ++lvl) {
        // Key digits up to the key's last bit, then ~index digits.
        const int bits = pbits < 32 ? min(11, 32 - pbits) : min(11, 64 - pbits);
        const int nb = 1 << bits;
        for (int i = tid; i < nb; i += kRT) {
            sh.hist[i] = 0;
            sh.cnt[i] = 0;
        }
        __syncthreads();
        for (int i = tid; i < n; i += kRT) {
            const u64 c = sh.cand[i];
            const uint32_t key = (uint32_t)(c >> 32);
            if (!member(key, (int)~(uint32_t)c)) continue;
            if (pbits > 0 && (c >> (64 - pbits)) != prefix) continue;
            const uint32_t d = (uint32_t)(c >> (64 - pbits - bits)) & (uint32_t)(nb - 1);
            const u64 m = mass_of(key_value(key));
            if (m) {
                atomicAdd(&sh.hist[d], m);
                atomicAdd(&sh.cnt[d], 1u);
            }
        }
        __syncthreads();
        u64 bb;
        int cnt;
        const int d = bin_scan(nb, before, theta, strict, sh, &bb, &cnt);
        if (d < 0) return -1;
        if (lvl == 0) {
            s.d1 = d;
            s.bits1 = bits;
            s.before1 = bb;
        }
        s.levels = lvl + 1;
        before = bb;
        few = cnt <= 64;
        prefix = (prefix << bits) | (uint64_t)d;
        pbits += bits;
    }
    s.prefix = prefix;
    s.pbits = pbits;
    s.before = before;
    if (st) *st = s;
    return bin_resolve(n, member, mass_of, theta, strict, sh, prefix, pbits, before, before_out, mass_out, key_out);
}

__device__ __forceinline__ bool row_has_proc(const SampleArgs& a, int b) {
    return (a.bias_off && a.bias_off[b + 1] > a.bias_off[b]) || (a.pen_off && a.pen_off[b + 1] > a.pen_off[b]) ||
           (a.mask_row && a.mask_row[b] >= 0);
}

__device__ __forceinline__ const float* row_ptr(const SampleArgs& a, int b) {
    return (row_has_proc(a, b) ? a.ws : a.logits) + (size_t)b * a.V;
}

// ------------------------------------------------------------------ chunked passes (kCT threads)

constexpr int kChunk = kSampleChunk;  // vocabulary entries per workgroup of a chunked pass
constexpr int kCT = 256;             // threads of a chunked pass
constexpr int kCW = kCT / 64;
constexpr int kCPer = kChunk / kCT;  // entries per thread

// Index of entry i of this thread in chunk [v0, v0 + kChunk), strided layout: consecutive threads
// take consecutive 16-byte vectors (floats when the row is not 16-byte aligned).
__device__ __forceinline__ int chunk_index(int v0, int i, bool vec4) {
    return vec4 ? v0 + ((i >> 2) * kCT + (int)threadIdx.x) * 4 + (i & 3) : v0 + i * kCT + (int)threadIdx.x;
}

// Loads chunk [v0, v1) of row y in the strided layout; positions past v1 get -inf.
__device__ __forceinline__ void load_chunk(const float* y, int v0, int v1, bool vec4, float (&x)[kCPer]) {
    const float ninf = -__builtin_huge_valf();
    if (vec4) {
#pragma unroll
        for (int it = 0; it < kCPer / 4; ++it) {
            const int v = chunk_index(v0, it * 4, true);
            float4 f = make_float4(ninf, ninf, ninf, ninf);
            if (v < v1) f = *reinterpret_cast<const float4*>(y + v);
            x[it * 4 + 0] = f.x;
            x[it * 4 + 1] = f.y;
            x[it * 4 + 2] = f.z;
            x[it * 4 + 3] = f.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < kCPer; ++i) {
            const int v = chunk_index(v0, i, false);
            x[i] = v < v1 ? y[v] : ninf;
        }
    }
}

__device__ __forceinline__ float cblock_max(float v, float* red) {
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = red[0];
    for (int w = 1; w < kCW; ++w) r = fmaxf(r, red[w]);
    __syncthreads();
    return r;
}

__device__ __forceinline__ float cblock_sum(float v, float* red) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = 0.f;
    for (int w = 0; w < kCW; ++w) r += red[w];
    __syncthreads();
    return r;
}

// Copies rows that have a processor into the workspace: the mask (-inf where disallowed), then
// the bias entries, then the penalty entries (worker.rs:142-181; the entries of one list name
// distinct tokens). Grid (chunk, row).
__global__ __launch_bounds__(kCT) void sample_prepare_kernel(SampleArgs a) {
    __shared__ float s_row[kChunk];
    const int c = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
    if (!row_has_proc(a, b)) return;
    const float* x = a.logits + (size_t)b * a.V;
    float* y = a.ws + (size_t)b * a.V;
    const int mr = a.mask_row ? a.mask_row[b] : -1;
    const uint32_t* mask = (mr >= 0 && mr < a.num_masks) ? a.mask + (size_t)mr * a.mask_words : nullptr;
    if (a.mask_row && mr >= a.num_masks && c == 0 && tid == 0) latch_error(a.err, ERR_TOKEN);
    const int v0 = c * kChunk, v1 = min(a.V, v0 + kChunk);
    for (int v = v0 + tid; v < v1; v += kCT) {
        float g = 0.0f;
        if (mask && !((mask[v >> 5] >> (v & 31)) & 1u)) g = -__builtin_huge_valf();
        s_row[v - v0] = x[v] + g;
    }
    __syncthreads();
    auto apply = [&](const int32_t* off, const uint32_t* tok, const float* val) {
        for (int i = off[b] + tid; i < off[b + 1]; i += kCT) {
            const uint32_t t = tok[i];
            if (t >= (uint32_t)v0 && t < (uint32_t)v1) s_row[t - v0] = s_row[t - v0] + val[i];
            else if (t >= (uint32_t)a.V && c == 0) latch_error(a.err, ERR_TOKEN);
        }
        __syncthreads();
    };
    if (a.bias_off) apply(a.bias_off, a.bias_tok, a.bias_val);
    if (a.pen_off) apply(a.pen_off, a.pen_tok, a.pen_val);
    for (int v = v0 + tid; v < v1; v += kCT) y[v] = s_row[v - v0];
}

// Pass 1, grid (chunk, row): per chunk of the processed row, {max z, sum exp(z - max z)} with
// z = y * f32(1 / T) + 0, or {max y, its first index} for T <= 0. Rows with top-k or top-p also
// list the chunk's candidates (threshold, count and (key << 32) | ~index entries) for the select
// pass.
__global__ __launch_bounds__(kCT) void sample_stats_kernel(SampleArgs a) {
    __shared__ float s_red[kCW];
    __shared__ int s_ired[kCW];
    __shared__ uint32_t s_wn[2 * kCW];
    const int c = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float* y = row_ptr(a, b);
    const int v0 = c * kChunk, v1 = min(a.V, v0 + kChunk);
    const bool vec4 = a.vec4;
    float x[kCPer];
    load_chunk(y, v0, v1, vec4, x);
    const float T = a.temperature[b];
    const int k = a.top_k ? a.top_k[b] : 0;  // issued with the chunk's loads
    const float tp = a.top_p ? a.top_p[b] : 1.0f;
    float2* out = a.cstat + (size_t)b * a.C + c;
    if (!(T > 0.f)) {  // first maximum of y (entries of a thread ascend in index)
        float bv = -__builtin_huge_valf();
        int bi = 0x7fffffff;
#pragma unroll
        for (int i = 0; i < kCPer; ++i) {
            const int v = chunk_index(v0, i, vec4);
            if (v < v1 && x[i] > bv) {
                bv = x[i];
                bi = v;
            }
        }
        wave_argmax(bv, bi);
        if (lane == 0) {
            s_red[wave] = bv;
            s_ired[wave] = bi;
        }
        __syncthreads();
        if (tid == 0) {
            for (int w = 1; w < kCW; ++w)
                if (s_red[w] > bv || (s_red[w] == bv && s_ired[w] < bi)) {
                    bv = s_red[w];
                    bi = s_ired[w];
                }
            *out = make_float2(bv, __int_as_float(bi));
        }
        return;
    }
    const float sc = (float)(1.0 / (double)T);
    float m = -__builtin_huge_valf();
#pragma unroll
    for (int i = 0; i < kCPer; ++i) {
        x[i] = x[i] * sc + 0.0f;
        m = fmaxf(m, x[i]);
    }
    const float lmax = m;  // this lane's largest entry
    m = cblock_max(m, s_red);
    float sum = 0.f;
    if (m != -__builtin_huge_valf()) {
#pragma unroll
        for (int i = 0; i < kCPer; ++i) sum += fast_exp2((x[i] - m) * kLog2e);
    }
    sum = cblock_sum(sum, s_red);
    if (tid == 0) *out = make_float2(m, sum);

    const bool use_k = k > 0 && k < a.V, use_p = tp < 1.0f;
    if (!use_k && !use_p) return;
    // The chunk's candidate list: every entry with z >= t, for a t that keeps the list within
    // ccap entries. Counts over the block come from wave ballots (no atomics), two LDS slots per
    // wave alternating so that each count needs one barrier.
    int buf = 0;
    auto count_ge = [&](float t) -> int {
        int n = 0;
#pragma unroll
        for (int i = 0; i < kCPer; ++i) n += (int)__popcll(__ballot(x[i] >= t));
        if (lane == 0) s_wn[buf * kCW + wave] = (uint32_t)n;
        __syncthreads();
        int tot = 0;
#pragma unroll
        for (int w = 0; w < kCW; ++w) tot += (int)s_wn[buf * kCW + w];
        buf ^= 1;
        return __builtin_amdgcn_readfirstlane(tot);  // the same in every lane: keeps the searches scalar
    };
    // The list at t: this thread's hits (bit i: entry i >= t), its offset among the block's hits
    // (a block scan), and the total, which is count_ge(t); shares count_ge's LDS slots.
    uint32_t hits = 0, off = 0;
    auto scan_hits = [&](float t) -> int {
        hits = 0;
#pragma unroll
        for (int i = 0; i < kCPer; ++i)
            if (x[i] >= t) hits |= 1u << i;
        const uint32_t mine = (uint32_t)__popc(hits);
        const uint32_t incl = (uint32_t)wave_incl_scan_i((int)mine);
        if (lane == 63) s_wn[buf * kCW + wave] = incl;
        __syncthreads();
        uint32_t o = incl - mine, tot = 0;
#pragma unroll
        for (int w = 0; w < kCW; ++w) {
            if (w < wave) o += s_wn[buf * kCW + w];
            tot += s_wn[buf * kCW + w];
        }
        buf ^= 1;
        off = o;
        return __builtin_amdgcn_readfirstlane((int)tot);
    };
    const float ninf = -__builtin_huge_valf();
    const int cap = a.ccap;
    // Thresholds on a grid below the chunk's max: t_j = m - j / 8, j < npts (at most 512: 64 nats).
    auto grid_t = [&](int j) { return m - (float)j * 0.125f; };
    // Largest j in [-1, npts) with count_ge(t_j) <= lim (count(t_-1) = 0); *c_lo / *c_hi get the
    // counts at j and j + 1 (-1 when j + 1 = npts was never counted).
    auto bisect = [&](int lim, int npts, int* c_lo, int* c_hi) {
        int lo = -1, hi = npts, clo = 0, chi = -1;
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            const int cm = count_ge(grid_t(mid));
            if (cm <= lim) {
                lo = mid;
                clo = cm;
            } else {
                hi = mid;
                chi = cm;
            }
        }
        *c_lo = clo;
        *c_hi = chi;
        return lo;
    };
    // Lanes whose largest entry is at or above t: one ballot instead of sixteen, and never more
    // than the entries at or above t. Steers the searches; the thresholds kept are counted exactly.
    auto lanes_ge = [&](float t) -> int {
        const int n = (int)__popcll(__ballot(lmax >= t));
        if (lane == 0) s_wn[buf * kCW + wave] = (uint32_t)n;
        __syncthreads();
        int tot = 0;
#pragma unroll
        for (int w = 0; w < kCW; ++w) tot += (int)s_wn[buf * kCW + w];
        buf ^= 1;
        return __builtin_amdgcn_readfirstlane(tot);
    };
    auto bisect_lanes = [&](int lim, int npts) {  // largest j in [-1, npts) with lanes_ge(t_j) <= lim
        int lo = -1, hi = npts;
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (lanes_ge(grid_t(mid)) <= lim) lo = mid;
            else hi = mid;
        }
        return lo;
    };
    float thr = ninf;     // -inf: every finite entry (a complete list)
    int cnt = -1;         // -1: no threshold keeps the list within cap
    bool listed = false;  // hits and off already hold the list at thr
    if (m == ninf) {
        cnt = 0;  // nothing finite in the chunk
    } else if (use_k) {
        // Top-k (with or without top-p): the chunk's own k largest must be listed, so t is the
        // highest grid threshold with at least k entries at or above it; a chunk with fewer
        // than k entries that far up lists every finite entry.
        // The highest grid threshold with k lanes at or above it has at least k entries there;
        // one exact count checks it fits, else the exact search runs.
        const int jl = bisect_lanes(k - 1, 512) + 1;
        const int cl = jl < 512 ? scan_hits(grid_t(jl)) : -1;
        if (cl >= k && cl <= cap) {
            thr = grid_t(jl);
            cnt = cl;
            listed = true;
        } else {
            int clo, chi;
            const int j = bisect(k - 1, 512, &clo, &chi) + 1;
            if (j < 512 && chi <= cap) {
                thr = grid_t(j);
                cnt = chi;
            } else {
                const int fin = count_ge(-FLT_MAX);  // finite entries
                if (fin <= cap) cnt = fin;           // complete
            }
        }
    } else {
        // Top-p alone keeps a token only if p >= (1 - top_p) / V; with log Z >= this chunk's
        // max m, a token with z < m - ln(V / (1 - top_p)) is never kept (one nat of margin for
        // rounding), so the list may start there; else at a grid threshold above it. The select
        // pass checks that the lists reach below the cut.
        const float span = logf((float)a.V / fmaxf(1.f - tp, 1e-30f)) + 1.f;
        const float skip = m - span;
        // The skip bound is counted only when no grid point above it has more than `target` lanes
        // (t_(npts-1) >= skip); otherwise the lowest grid threshold with at most `target` lanes
        // above it, counted exactly, is kept when its entries fit the list's slots (a step up, at
        // most twice, when they do not); else the exact search for at most `target` entries runs.
        const int target = min(cap, KYRO_SAMPLE_P_TARGET);
        const int npts = min(512, (int)ceilf(span * 8.f));
        int j = bisect_lanes(target, npts);
        const int cs = j == npts - 1 ? count_ge(skip) : cap + 1;
        if (cs <= cap) {
            thr = skip;
            cnt = cs;
        } else {
            int cj = j >= 0 ? scan_hits(grid_t(j)) : cap + 1;
            bool at_j = true;
            for (int step = 0; step < 2 && cj > cap && j > 0; ++step) {
                cj = count_ge(grid_t(--j));
                at_j = false;
            }
            if (j >= 0 && cj <= cap) {
                thr = grid_t(j);
                cnt = cj;
                listed = at_j;
            } else {
                int clo, chi;
                const int jx = bisect(target, npts, &clo, &chi);
                if (jx >= 0) {
                    thr = grid_t(jx);
                    cnt = clo;
                }
            }
        }
    }
    // Write the list: a block scan of the per-thread hits places every entry (done above when
    // the threshold's exact count came from it). The list's length is the scan's total; a total
    // above the cap (the counts above disagreeing with the hits) sends the row to the fallback
    // instead of writing past the chunk's slots.
    if (cnt > 0) {
        const int total = listed ? cnt : scan_hits(thr == ninf ? -FLT_MAX : thr);
        cnt = total <= cap ? total : -1;
    }
    if (tid == 0) {
        a.cthr[(size_t)b * a.C + c] = thr;
        a.ccount[(size_t)b * a.C + c] = cnt;
    }
    if (cnt <= 0) return;
    u64* list = a.cand + (size_t)b * kCap + (size_t)c * cap;
#pragma unroll
    for (int i = 0; i < kCPer; ++i)
        if (hits & (1u << i)) {
            list[off] = ((u64)order_key(x[i]) << 32) | (uint32_t)~(uint32_t)chunk_index(v0, i, vec4);
            ++off;
        }
}

// Settles a top-k / top-p row (worker.rs:300-360) from n candidates in sh.cand (n < 0: none):
// the k largest for top-k, or for top-p alone every token with key >= kmin (more below it may be
// present). Candidates sort or are searched in descending order (key descending, index
// ascending). A row whose candidates do not settle the cut gathers candidates from the row itself
// (two passes, below), and what that leaves runs exact radix selects over the whole row: three
// passes (11 + 11 + 10 bits) of mass histograms in LDS (64-bit fixed point, 2^-52 resolution, so
// the sums do not depend on thread order), then a pass in index order for ties between equal
// keys.
__device__ __forceinline__ void finish_row(const SampleArgs& a, int b, RowShared& sh, int n, float M, float Z, uint32_t kmin,
                           float T, int k, float tp, float u, int cp_bits, uint64_t cp) {
    const int tid = threadIdx.x;
    const int V = a.V;
    Row r;
    r.y = row_ptr(a, b);
    r.V = V;
    r.vec4 = a.vec4;
    r.s = (float)(1.0 / (double)T);
    r.m = M;
    r.z_sum = Z;
    r.kk = 0;
    r.ki = V;
    r.ck = 0;
    r.ci = V;
    const bool use_k = k > 0 && k < V;
    const bool use_p = tp < 1.0f;
    // Settles the row from n candidates in sh.cand (see above); false when they do not settle it.
    auto from_candidates = [&](int n, uint32_t kmin, int cp_bits, uint64_t cp) -> bool {
    if (n <= kSortMax) {
        // Few candidates: sorted in LDS, then cut and walked with running sums.
        int np2 = 2;
        while (np2 < n) np2 <<= 1;
        for (int i = n + tid; i < np2; i += kRT) sh.cand[i] = 0;
        __syncthreads();
        bitonic_desc(sh.cand, np2);
        // Top-p alone: the lists are complete only at keys >= kmin (sorted to the front).
        int ncov = n;
        if (kmin) {
            int nb = 0;
            for (int i = tid; i < n; i += kRT) nb += (uint32_t)(sh.cand[i] >> 32) < kmin ? 1 : 0;
            ncov = n - block_sum_i(nb, sh);
        }
        const int ns = use_k ? min(k, n) : ncov;
        auto cz = [&](int i) { return key_value((uint32_t)(sh.cand[i] >> 32)); };
        float zsum = r.z_sum;
        if (use_k) {  // the kept set is the first k candidates
            float zs = 0.f;
            for (int i = tid; i < ns; i += kRT) zs += r.e(cz(i));
            zsum = block_sum_f(zs, sh);
        }
        for (int i = tid; i < ns; i += kRT) sh.cum[i] = r.e(cz(i)) / zsum;
        __syncthreads();
        block_scan_incl(sh.cum, ns, sh);
        int cut = ns;
        float rr = u;
        if (use_p) {
            cut = first_at_least(sh.cum, ns, tp, true, sh);  // first running sum above top_p
            if (cut < 0) cut = ns;
            else cut += 1;
            if (!use_k && cut == ns && ncov < V) cut = -1;  // the cut may lie past the candidates
            if (cut > 0) rr = u * sh.cum[cut - 1];
        }
        if (cut > 0) {
            int pick = first_at_least(sh.cum, cut, rr, false, sh);
            if (pick < 0) pick = use_p ? 0 : ns - 1;
            if (tid == 0) a.out[b] = ~(uint32_t)sh.cand[pick];
            return true;
        }
    }
    if (n > kSortMax) {
        // The same searches as the row path below, over the candidates: they hold the row's k
        // largest (top-k) or, for top-p alone, every token with key >= kmin; cp_bits / cp is the
        // prefix the keys of every candidate at or above kmin share.
        auto every = [](uint32_t, int) { return true; };
        auto unit = [](float) -> u64 { return 1; };
        u64 bf, ms;
        uint32_t key;
        if (use_k) {  // the k-th token in descending order bounds the kept set
            const int kth = cand_search(n, every, unit, (u64)k, false, sh, &bf, &ms, &key, cp_bits, cp);
            if (kth >= 0) {
                r.kk = key;
                r.ki = kth;
            }
            float zs = 0.f;
            for (int i = tid; i < n; i += kRT) {
                const uint32_t kc = (uint32_t)(sh.cand[i] >> 32);
                if (r.kept(kc, (int)~(uint32_t)sh.cand[i])) zs += r.e(key_value(kc));
            }
            r.z_sum = block_sum_f(zs, sh);
        }
        auto kept = [&](uint32_t kc, int v) { return kc >= kmin && r.kept(kc, v); };
        auto pmass = [&](float zv) -> u64 { return fix_mass(r.prob(zv)); };
        u64 total = (u64)llrint(kFix);
        float rr = u;
        bool settled = true;
        SearchState cst{};
        int cut = -1;
        if (use_p) {
            cut = cand_search(n, kept, pmass, (u64)llrint((double)tp * kFix), true, sh, &bf, &ms, &key, cp_bits, cp, &cst);
            if (cut >= 0) {
                r.ck = key;
                r.ci = cut;
                total = bf + ms;
            } else if (!use_k) {
                settled = false;  // the cut may lie past the candidates: the row path finds it
            } else {  // the running sum never exceeds top_p: the whole kept set
                float ts = 0.f;
                for (int i = tid; i < n; i += kRT) {
                    const uint32_t kc = (uint32_t)(sh.cand[i] >> 32);
                    if (r.kept(kc, (int)~(uint32_t)sh.cand[i])) ts += r.prob(key_value(kc));
                }
                total = fix_mass(block_sum_f(ts, sh));
            }
            rr = u * (float)((double)total / kFix);
        }
        if (settled) {
            auto in_cut = [&](uint32_t kc, int v) { return r.kept(kc, v) && r.in_cut(kc, v); };
            const u64 theta = fix_mass(rr);
            int pick;
            if (theta != 0 && cut >= 0 && cst.levels == 1) {
                // The cut search's first-level histogram still holds: its bins above the cut's bin
                // hold only tokens ahead of the cut, so the draw finds its bin there, or in the
                // cut's own bin once theta passes their mass, without another histogram pass.
                int d = cst.d1, cnt = 0;
                u64 bb = cst.before1;
                if (theta <= cst.before1) d = bin_scan(1 << cst.bits1, 0, theta, false, sh, &bb, &cnt);
                if (d >= 0 && cnt <= 64)
                    pick = bin_resolve(n, in_cut, pmass, theta, false, sh, (cp << cst.bits1) | (uint64_t)d,
                                       cp_bits + cst.bits1, bb, &bf, &ms, &key);
                else
                    pick = cand_search(n, in_cut, pmass, theta, false, sh, &bf, &ms, &key, cp_bits, cp);
            } else {
                pick = theta == 0 ? cand_search(n, in_cut, unit, 1, false, sh, &bf, &ms, &key, cp_bits, cp)
                                  : cand_search(n, in_cut, pmass, theta, false, sh, &bf, &ms, &key, cp_bits, cp);
            }
            if (pick < 0) pick = use_p ? cand_search(n, kept, unit, 1, false, sh, &bf, &ms, &key, cp_bits, cp) : r.ki;
            if (tid == 0) a.out[b] = (uint32_t)(pick >= 0 && pick < V ? pick : V - 1);
            return true;
        }
        r.kk = 0;
        r.ki = V;
        r.ck = 0;
        r.ci = V;
        r.z_sum = Z;
    }
    return false;
    };
    if (n >= 0 && from_candidates(n, kmin, cp_bits, cp)) return;
    // Row gather, when the lists did not settle the row: pass A histograms the row in bins of
    // 1/8 nat below M (64 nats) (counts, and for top-p alone masses exp(z - bin top) in 2^-12 units, so
    // that a wave's V / 16 tokens stay below 2^32 for every V; one copy per wave in the candidate
    // array, which is free here), the bins from the top find the
    // bin where the running count reaches k (top-k) or the running mass passes top_p Z (top-p,
    // one bin lower for the masses' rounding), and pass B gathers every token in that bin or
    // above. Both the bin of a token and the gathered set are monotone in z, so every token at
    // or above the least gathered key is present, and the candidate path settles the row exactly
    // or leaves it to the radix selects.
    {
        constexpr int kGB = 512;  // two arrays of kRW x kGB words fill the candidate array
        static_assert(2 * kRW * kGB * 4 <= kCap * 8, "row-gather histograms exceed the candidate array");
        uint32_t* hc = reinterpret_cast<uint32_t*>(sh.cand);
        uint32_t* hm = hc + kRW * kGB;
        const bool by_mass = use_p && !use_k;
        for (int i = tid; i < 2 * kRW * kGB; i += kRT) hc[i] = 0;
        __syncthreads();
        auto bin_of = [&](float zv) { return (M - zv) * 8.f; };  // bin = (int) of it, below kGB
        {
            uint32_t* myc = hc + (tid >> 6) * kGB;
            uint32_t* mym = hm + (tid >> 6) * kGB;
            row_for_each(r.y, V, r.vec4, [&](int, float yv) {
                const float zv = yv * r.s + 0.0f;
                const float d = bin_of(zv);
                if (!(d < (float)kGB)) return;  // below the range, or NaN
                const int bin = (int)fmaxf(d, 0.f);
                atomicAdd(&myc[bin], 1u);
                if (by_mass) {
                    const float e = fast_exp2((zv - (M - 0.125f * (float)bin)) * kLog2e);
                    atomicAdd(&mym[bin], (uint32_t)fminf(e * 4096.f, 4096.f));
                }
            });
        }
        __syncthreads();
        // Thread t < kGB merges bin t; bins in thread order run from the top down.
        int bc = 0;
        float bm = 0.f;
        if (tid < kGB) {
            uint32_t sm = 0;
            for (int w = 0; w < kRW; ++w) {
                bc += (int)hc[w * kGB + tid];
                sm += hm[w * kGB + tid];
            }
            bm = (float)sm * (1.f / 4096.f) * fast_exp2(-0.125f * (float)tid * kLog2e);
        }
        const int cinc = wave_incl_scan_i(bc);
        const float minc = wave_incl_scan_f(bm);
        if ((tid & 63) == 63) {
            sh.ired[tid >> 6] = cinc;
            sh.fred[tid >> 6] = minc;
        }
        if (tid == 0) sh.found = 0x7fffffff;
        __syncthreads();
        int cb = cinc;
        float mb = minc;
        for (int w = 0; w < (tid >> 6); ++w) {
            cb += sh.ired[w];
            mb += sh.fred[w];
        }
        const bool reach = by_mass ? mb > tp * Z : cb >= k;
        if (tid < kGB && reach) atomicMin(&sh.found, tid);
        __syncthreads();
        const int bsel = sh.found == 0x7fffffff ? -1 : min(sh.found + (by_mass ? 1 : 0), kGB - 1);
        if (tid == bsel) sh.count = cb;  // tokens in the bins at or above bsel
        __syncthreads();
        const int ng = bsel >= 0 ? sh.count : kCap + 1;
        __syncthreads();
        if (ng <= kCap) {
            if (tid == 0) sh.nsmall = 0;
            __syncthreads();
            uint32_t lo = 0xffffffffu, hi = 0u;
            row_for_each(r.y, V, r.vec4, [&](int v, float yv) {
                const float zv = yv * r.s + 0.0f;
                const float d = bin_of(zv);
                if (!(d < (float)kGB) || (int)fmaxf(d, 0.f) > bsel) return;
                const uint32_t key = order_key(zv);
                const int slot = atomicAdd(&sh.nsmall, 1);
                if (slot < kCap) sh.cand[slot] = ((u64)key << 32) | (uint32_t)~(uint32_t)v;
                lo = min(lo, key);
                hi = max(hi, key);
            });
            int gbits;
            uint64_t gp;
            uint32_t gmin;
            key_range_prefix(lo, hi, sh, &gbits, &gp, &gmin);  // its barriers order the gather's writes
            const int got = sh.nsmall;
            __syncthreads();
            if (got <= kCap && from_candidates(got, use_k ? 0u : gmin, gbits, gp)) return;
        }
    }
    // Radix selects over the whole row (candidates did not fit in LDS, or did not settle the cut).
    auto all = [](uint32_t, int) { return true; };
    auto one = [](float) -> u64 { return 1; };
    if (use_k) {  // the k-th token in descending order bounds the kept set
        u64 bf, ms;
        const int kth = desc_search(r, all, one, (u64)k, false, sh, &bf, &ms);
        if (kth >= 0) {  // always found: the row has V > k members of mass 1
            r.kk = order_key(r.z(kth));
            r.ki = kth;
        }
    }
    {
        float zs = 0.f;
        row_for_each(r.y, V, r.vec4, [&](int v, float yv) {
            const float zv = yv * r.s + 0.0f;
            if (r.kept(order_key(zv), v)) zs += r.e(zv);
        });
        r.z_sum = block_sum_f(zs, sh);
    }
    // Descending order over the kept set.
    auto kept = [&](uint32_t key, int v) { return r.kept(key, v); };
    auto pmass = [&](float zv) -> u64 { return fix_mass(r.prob(zv)); };
    u64 total = (u64)llrint(kFix);  // the walk's r is u itself when there is no top-p cut
    float rr = u;
    if (use_p) {
        u64 bf, ms;
        const int cut = desc_search(r, kept, pmass, (u64)llrint((double)tp * kFix), true, sh, &bf, &ms);
        if (cut >= 0) {
            r.ck = order_key(r.z(cut));
            r.ci = cut;
            total = bf + ms;
        } else {  // the running sum never exceeds top_p: the whole kept set
            float ts = 0.f;
            for (int v = tid; v < V; v += kRT) {
                const float zv = r.z(v);
                if (r.kept(order_key(zv), v)) ts += r.prob(zv);
            }
            ts = block_sum_f(ts, sh);
            total = fix_mass(ts);
        }
        rr = u * (float)((double)total / kFix);
    }
    auto in_cut = [&](uint32_t key, int v) { return r.kept(key, v) && r.in_cut(key, v); };
    int pick;
    u64 bf, ms;
    const u64 theta = fix_mass(rr);
    if (theta == 0) {  // r <= 0 takes the first token in the order
        pick = desc_search(r, in_cut, one, 1, false, sh, &bf, &ms);
    } else {
        pick = desc_search(r, in_cut, pmass, theta, false, sh, &bf, &ms);
    }
    if (pick < 0) pick = use_p ? desc_search(r, kept, one, 1, false, sh, &bf, &ms) : r.ki;
    if (tid == 0) a.out[b] = (uint32_t)(pick >= 0 && pick < V ? pick : V - 1);
}

// Pass 2, one workgroup per row: merges the chunk statistics. T <= 0: the first maximum. Plain
// sampling: Z, the chunk where the running mass in index order reaches u Z, and the walk inside
// it (worker.rs:352-360). Top-k / top-p: the chunks' candidate lists, gathered into LDS when they
// cover the kept set, then finish_row.
__global__ __launch_bounds__(kRT) void sample_select_kernel(SampleArgs a) {
    __shared__ RowShared sh;
    const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int C = a.C;
    // Every per-row input in one round of loads, issued with the chunk statistics.
    const float T = a.temperature[b];
    const int k = a.top_k ? a.top_k[b] : 0;
    const float tp = a.top_p ? a.top_p[b] : 1.0f;
    const float u = a.u[b];
    const float2 st = tid < C ? a.cstat[(size_t)b * C + tid] : make_float2(-__builtin_huge_valf(), 0.f);
    // List lengths and thresholds, loaded with the statistics (top-k / top-p rows only).
    const int listn = (a.ccount && tid < C) ? a.ccount[(size_t)b * C + tid] : 0;
    const float thr = (a.cthr && tid < C) ? a.cthr[(size_t)b * C + tid] : 0.f;
    if (!(T > 0.f)) {
        const int best = block_argmax(st.x, tid < C ? __float_as_int(st.y) : 0x7fffffff, sh);
        if (tid == 0) {
            a.out[b] = (uint32_t)(best == 0x7fffffff ? 0 : best);
        }
        return;
    }
    const float M = block_max_f(st.x, sh);
    if (M == -__builtin_huge_valf()) {  // every token disallowed
        if (tid == 0) {
            a.out[b] = (uint32_t)(a.V - 1);
        }
        return;
    }
    // Chunk masses exp(z - M) in chunk order: thread t holds chunk t; inclusive scan gives Z.
    const float w = (tid < C && st.x != -__builtin_huge_valf()) ? st.y * fast_exp2((st.x - M) * kLog2e) : 0.f;
    const float winc = wave_incl_scan_f(w);
    if (lane == 63) sh.fred[wave] = winc;
    __syncthreads();
    float cbase = 0.f, Z = 0.f;
    for (int q = 0; q < kRW; ++q) {
        if (q < wave) cbase += sh.fred[q];
        Z += sh.fred[q];
    }
    const float cum = cbase + winc;  // running mass through chunk tid
    __syncthreads();
    const bool use_k = k > 0 && k < a.V, use_p = tp < 1.0f;
    const float sc = (float)(1.0 / (double)T);
    if (!use_k && !use_p) {
        const float rr = u * Z;
        if (tid == 0) sh.found = 0x7fffffff;
        __syncthreads();
        if (tid < C && cum >= rr && (tid == 0 || cum - w < rr)) atomicMin(&sh.found, tid);
        __syncthreads();
        const int cs = sh.found == 0x7fffffff ? C - 1 : sh.found;
        __syncthreads();
        if (tid == cs) sh.fred[0] = cum - w;  // mass before the crossing chunk
        __syncthreads();
        const float rem = rr - sh.fred[0];
        // Walk chunk cs in index order: thread t owns the 4 consecutive entries 4t .. 4t+3.
        const float* y = row_ptr(a, b);
        const int v0 = cs * kChunk, v1 = min(a.V, v0 + kChunk);
        const int v = v0 + 4 * tid;
        float e[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) e[j] = v + j < v1 ? fast_exp2((y[v + j] * sc + 0.0f - M) * kLog2e) : 0.f;
        const float mine = (e[0] + e[1]) + (e[2] + e[3]);
        const float inc = wave_incl_scan_f(mine);
        if (lane == 63) sh.fred[wave] = inc;
        __syncthreads();
        float base = inc - mine;
        for (int q = 0; q < wave; ++q) base += sh.fred[q];
        if (tid == 0) sh.found = 0x7fffffff;
        __syncthreads();
        if (v < v1 && base < rem && base + mine >= rem) {  // this thread's four hold the crossing
            float run = base;
            int pick = -1;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                run += e[j];
                if (pick < 0 && v + j < v1 && run >= rem) pick = v + j;
            }
            atomicMin(&sh.found, pick >= 0 ? pick : min(v + 3, v1 - 1));  // rounding can make two threads claim it
        } else if (tid == 0 && rem <= 0.f) {
            atomicMin(&sh.found, v0);
        }
        __syncthreads();
        if (tid == 0 && sh.found == 0x7fffffff) sh.found = -1;
        __syncthreads();
        if (tid == 0) {
            a.out[b] = (uint32_t)(sh.found >= 0 ? sh.found : a.V - 1);
        }
        return;
    }
    // Top-k / top-p: the chunks' candidate lists (offsets in sh.cnt[kSampleMaxChunks + c]).
    const int cnt = tid < C ? listn : 0;
    const bool ok = tid >= C || (cnt >= 0 && (!use_k || thr == -__builtin_huge_valf() || cnt >= k));
    const bool all_ok = __syncthreads_and(ok) != 0;
    const int cpos = cnt > 0 ? cnt : 0;
    const int cinc = wave_incl_scan_i(cpos);
    if (lane == 63) sh.ired[wave] = cinc;
    __syncthreads();
    int coff = cinc - cpos, n = 0;
    for (int q = 0; q < kRW; ++q) {
        if (q < wave) coff += sh.ired[q];
        n += sh.ired[q];
    }
    if (tid < C) {
        sh.cnt[tid] = (uint32_t)cpos;
        sh.cnt[kSampleMaxChunks + tid] = (uint32_t)coff;
    }
    // Publishes sh.cnt to the copy below, and ends every wave's reads of sh.ired before
    // key_range_prefix rewrites it. Top-k rows take no other barrier on the way.
    __syncthreads();
    // Top-p alone: every list reaches down to its threshold, so all of them hold every token at
    // or above the largest one.
    const float tmax = use_k ? -__builtin_huge_valf() : block_max_f(tid < C ? thr : -__builtin_huge_valf(), sh);
    const bool covered = all_ok && n <= kCap && (!use_k || n >= k);
    const uint32_t kmin = (!use_k && tmax != -__builtin_huge_valf()) ? order_key(tmax) : 0u;
    // Copy the lists into LDS: kRT / C threads per chunk, each with at most 16 entries (C x ccap
    // <= kCap), loaded eight at a time before any is stored. The keys at or above kmin give the
    // searches their shared prefix.
    uint32_t klo = 0xffffffffu, khi = 0u;
    if (covered) {
        const int tpc = kRT / C, c = tid / tpc, sub = tid - c * tpc;
        if (c < C) {
            const int nc = (int)sh.cnt[c], oc = (int)sh.cnt[kSampleMaxChunks + c];
            const u64* src = a.cand + (size_t)b * kCap + (size_t)c * a.ccap;
            for (int q0 = 0; q0 < 16 && sub + q0 * tpc < nc; q0 += 8) {
                u64 e[8];
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const int j = sub + (q0 + q) * tpc;
                    e[q] = j < nc ? src[j] : 0;
                }
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const int j = sub + (q0 + q) * tpc;
                    if (j < nc) {
                        sh.cand[oc + j] = e[q];
                        const uint32_t key = (uint32_t)(e[q] >> 32);
                        if (key >= kmin) {
                            klo = min(klo, key);
                            khi = max(khi, key);
                        }
                    }
                }
            }
        }
    }
    int cp_bits;
    uint64_t cp;
    key_range_prefix(klo, khi, sh, &cp_bits, &cp);  // its barriers also order the copies
    finish_row(a, b, sh, covered ? n : -1, M, Z, kmin, T, k, tp, u, cp_bits, cp);
}

// ------------------------------------------------------- plain and greedy rows in one launch
//
// A batch without processors, top-k or top-p needs only each row's first maximum (T <= 0) or its
// softmax normaliser and one inverse-CDF walk, so one launch settles it. S = a.row_wgs
// workgroups of 1024 threads share a row (one workgroup alone streams at ~54 GB/s when 64 stream
// at once, so a row of 128256 entries takes four to put every CU to work). Wave w of a
// workgroup reduces segments of kSeg entries (eight 16-byte loads a lane, the next segment's
// issued before the current one is reduced) to {max z, sum exp(z - max)} or {max y, first
// index}. The segment statistics are published with device-scope stores and counted on the
// row's counter (a.row_cnt, zero between launches); the workgroup that counts last reads them
// all back with device-scope loads, combines them, finds the segment where the running mass in
// index order reaches u Z, walks it, and resets the counter. No workgroup waits for another:
// the others exit after counting. Masses are grouped by segment instead of by chunk, so a token
// can differ from the chunked passes' only where rounding decides the walk.
constexpr int kSeg = kSampleSeg;          // entries per segment
constexpr int kSegVec = kSeg / (4 * 64);  // 16-byte loads per lane per segment
constexpr int kRawWord3 = 0x00020000;     // raw buffer resource, 32-bit format, no swizzle

struct PlainShared {
    float fred[kRW];
    int ired[kRW];
    int last;
    int found;
    float rem;
};

__device__ __forceinline__ void store_coherent(float2* p, float2 v) {
    __hip_atomic_store(reinterpret_cast<unsigned long long*>(p), __builtin_bit_cast(unsigned long long, v),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float2 load_coherent(const float2* p) {
    return __builtin_bit_cast(float2, __hip_atomic_load(reinterpret_cast<const unsigned long long*>(p), __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT));
}

__global__ __launch_bounds__(kRT) void sample_plain_kernel(SampleArgs a) {
    __shared__ PlainShared sh;
    const int b = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: the segment loop is scalar
    const int S = a.row_wgs;
    const float T = a.temperature[b];
    const float u = a.u[b];
    const float* y = a.logits + (size_t)b * a.V;
    const int n4 = a.V >> 2;  // the row is 16-byte aligned and V a multiple of 4
    const int nseg = (a.V + kSeg - 1) / kSeg;
    const int spw = (nseg + S - 1) / S;  // segments of each workgroup
    const int s0 = (int)blockIdx.x * spw, s1 = min(nseg, s0 + spw);
    const bool greedy = !(T > 0.f);
    const float sc = greedy ? 0.f : (float)(1.0 / (double)T);
    const float ninf = -__builtin_huge_valf();
    float2* segs = a.segs + (size_t)b * nseg;
    // Segment sg's loads for this lane: vectors sg kSeg / 4 + lane + 64 i, through a resource that
    // starts at the segment and ends at the row's end (scalar base and size, fixed lane offsets:
    // no vector address arithmetic between loads); past the row the loads read zeros, which the
    // reduction drops. An index past the workgroup's segments reads nothing.
    auto load_seg = [&](int sg, float4 (&x)[kSegVec]) {
        const int v0 = min(min(sg, s1) * kSeg, a.V);
        const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(y + v0), (short)0, sg < s1 ? (a.V - v0) * 4 : 0, kRawWord3);
#pragma unroll
        for (int i = 0; i < kSegVec; ++i)
            x[i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, lane * 16 + 1024 * i, 0, 0));
    };
    auto reduce_seg = [&](int sg, const float4 (&x)[kSegVec]) {
        const int f0 = sg * (kSeg / 4) + lane;
        float2 st;
        if (greedy) {  // first maximum of y: a lane's entries ascend in index
            float bv = ninf;
            int bi = 0x7fffffff;
#pragma unroll
            for (int i = 0; i < kSegVec; ++i) {
                const int f = f0 + 64 * i;
                const float e[4] = {x[i].x, x[i].y, x[i].z, x[i].w};
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (f < n4 && e[j] > bv) {
                        bv = e[j];
                        bi = 4 * f + j;
                    }
            }
            wave_argmax(bv, bi);
            st = make_float2(bv, __int_as_float(bi));
        } else {
            float m = ninf;
#pragma unroll
            for (int i = 0; i < kSegVec; ++i) {
                if (f0 + 64 * i < n4)
                    m = fmaxf(fmaxf(m, fmaxf(x[i].x * sc + 0.0f, x[i].y * sc + 0.0f)),
                              fmaxf(x[i].z * sc + 0.0f, x[i].w * sc + 0.0f));
            }
            m = wave_max(m);
            float sum = 0.f;
            if (m != ninf) {
#pragma unroll
                for (int i = 0; i < kSegVec; ++i) {
                    if (f0 + 64 * i < n4) {
                        sum += fast_exp2((x[i].x * sc + 0.0f - m) * kLog2e);
                        sum += fast_exp2((x[i].y * sc + 0.0f - m) * kLog2e);
                        sum += fast_exp2((x[i].z * sc + 0.0f - m) * kLog2e);
                        sum += fast_exp2((x[i].w * sc + 0.0f - m) * kLog2e);
                    }
                }
            }
            st = make_float2(m, wave_sum(sum));
        }
        if (lane == 0) store_coherent(segs + sg, st);
    };
    if (s0 + wave < s1) {
        float4 xa[kSegVec], xb[kSegVec];
        int sg = s0 + wave;
        load_seg(sg, xa);
        while (true) {
            load_seg(sg + kRW, xb);
            reduce_seg(sg, xa);
            sg += kRW;
            if (sg >= s1) break;
            load_seg(sg + kRW, xa);
            reduce_seg(sg, xb);
            sg += kRW;
            if (sg >= s1) break;
        }
    }
    if (S > 1) {
        // Every wave's stores have reached the device-coherent level before the workgroup counts
        // itself; the last to count sees every other workgroup's stores.
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0) sh.last = atomicAdd(&a.row_cnt[b], 1) == S - 1;
        __syncthreads();
        if (!sh.last) return;
        if (tid == 0) __hip_atomic_store(&a.row_cnt[b], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
    }
    // The last workgroup: thread t holds segment t (nseg <= kRT).
    const float2 st = tid < nseg ? load_coherent(segs + tid) : make_float2(ninf, __int_as_float(0x7fffffff));
    if (greedy) {
        float bv = st.x;
        int bi = __float_as_int(st.y);
        wave_argmax(bv, bi);
        if (lane == 0) {
            sh.fred[wave] = bv;
            sh.ired[wave] = bi;
        }
        __syncthreads();
        if (tid == 0) {
            bv = sh.fred[0];
            bi = sh.ired[0];
            for (int w = 1; w < kRW; ++w)
                if (sh.fred[w] > bv || (sh.fred[w] == bv && sh.ired[w] < bi)) {
                    bv = sh.fred[w];
                    bi = sh.ired[w];
                }
            a.out[b] = (uint32_t)(bi == 0x7fffffff ? 0 : bi);
        }
        return;
    }
    float M = wave_max(st.x);
    if (lane == 0) sh.fred[wave] = M;
    __syncthreads();
    M = sh.fred[0];
    for (int w = 1; w < kRW; ++w) M = fmaxf(M, sh.fred[w]);
    __syncthreads();
    if (M == ninf) {  // no finite logit
        if (tid == 0) a.out[b] = (uint32_t)(a.V - 1);
        return;
    }
    // Segment masses exp(z - M) in index order; a block scan gives Z and the crossing segment.
    const float w = (tid < nseg && st.x != ninf) ? st.y * fast_exp2((st.x - M) * kLog2e) : 0.f;
    const float winc = wave_incl_scan_f(w);
    if (lane == 63) sh.fred[wave] = winc;
    if (tid == 0) sh.found = 0x7fffffff;
    __syncthreads();
    float cbase = 0.f, Z = 0.f;
    for (int q = 0; q < kRW; ++q) {
        if (q < wave) cbase += sh.fred[q];
        Z += sh.fred[q];
    }
    const float cum = cbase + winc;  // running mass through segment tid
    const float rr = u * Z;
    if (tid < nseg && cum >= rr && (tid == 0 || cum - w < rr)) atomicMin(&sh.found, tid);
    __syncthreads();
    const int cs = sh.found == 0x7fffffff ? nseg - 1 : sh.found;
    if (tid == cs) sh.rem = rr - (cum - w);  // r less the mass before the crossing segment
    __syncthreads();
    const float rem = sh.rem;
    if (tid == 0) sh.found = 0x7fffffff;
    // Walk segment cs in index order: thread t owns the 2 consecutive entries 2t, 2t + 1.
    const int v0 = cs * kSeg, v1 = min(a.V, v0 + kSeg);
    const int v = v0 + 2 * tid;
    const float2 q = v < v1 ? *reinterpret_cast<const float2*>(y + v) : make_float2(0.f, 0.f);
    const float e0 = v < v1 ? fast_exp2((q.x * sc + 0.0f - M) * kLog2e) : 0.f;
    const float e1 = v < v1 ? fast_exp2((q.y * sc + 0.0f - M) * kLog2e) : 0.f;
    const float mine = e0 + e1;
    const float inc = wave_incl_scan_f(mine);
    if (lane == 63) sh.fred[wave] = inc;
    __syncthreads();
    float base = inc - mine;
    for (int q2 = 0; q2 < wave; ++q2) base += sh.fred[q2];
    if (v < v1 && base < rem && base + mine >= rem) {  // this thread's two hold the crossing
        atomicMin(&sh.found, base + e0 >= rem ? v : v + 1);  // rounding can make two threads claim it
    } else if (tid == 0 && rem <= 0.f) {
        atomicMin(&sh.found, v0);
    }
    __syncthreads();
    if (tid == 0) a.out[b] = (uint32_t)(sh.found != 0x7fffffff ? sh.found : a.V - 1);
}

}  // namespace

hipError_t launch_sample(const SampleArgs& a, hipStream_t stream) {
    if (a.B == 0) return hipSuccess;
    if (a.row_wgs > 0) {  // no processor, top-k or top-p: one launch
        sample_plain_kernel<<<dim3((unsigned)a.row_wgs, (unsigned)a.B), kRT, 0, stream>>>(a);
        return hipGetLastError();
    }
    const dim3 grid((unsigned)a.C, (unsigned)a.B);
    if (a.bias_off || a.pen_off || a.mask_row) sample_prepare_kernel<<<grid, kCT, 0, stream>>>(a);
    sample_stats_kernel<<<grid, kCT, 0, stream>>>(a);
    sample_select_kernel<<<dim3((unsigned)a.B), kRT, 0, stream>>>(a);
    return hipGetLastError();
}

}  // namespace kyro
