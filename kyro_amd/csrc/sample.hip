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
// Two kernels:
//   sample_prepare_kernel  (rows with a processor) copies the row into the workspace with the
//                          mask applied; many workgroups per row.
//   sample_row_kernel      one 1024-thread workgroup per row: adds the sparse bias and penalty
//                          entries, then samples with passes over the row (it stays in L2 / the
//                          MALL after the first). Top-k and top-p are exact selects in the
//                          descending order: three radix passes (11 + 11 + 10 bits) over an
//                          order-preserving key of z build mass histograms in LDS (64-bit fixed
//                          point, 2^-52 resolution, so the sums do not depend on thread order),
//                          then a pass in index order settles ties between equal keys.
#include "common.hpp"
#include "kernels.hpp"

namespace kyro {
namespace {

constexpr int kRT = 1024;  // threads of the row kernel
constexpr int kRW = kRT / 64;
constexpr int kBins = 2048;
constexpr int kCap = 8192;                   // candidates sorted in LDS
constexpr double kFix = 4503599627370496.0;  // 2^52: fixed-point unit of probability mass
constexpr double kFixE = 1099511627776.0;    // 2^40: unit of exp(z - max) in the candidate histogram
constexpr float kLog2e = 1.4426950408889634f;
using u64 = unsigned long long;

// Unsigned key with the order of the float (larger float, larger key).
__device__ __forceinline__ uint32_t order_key(float z) {
    const uint32_t u = __float_as_uint(z);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ u64 shfl_up_u64(u64 x, int o) {
    const uint32_t lo = __shfl_up((uint32_t)x, o, 64);
    const uint32_t hi = __shfl_up((uint32_t)(x >> 32), o, 64);
    return ((u64)hi << 32) | lo;
}

__device__ __forceinline__ u64 shfl_xor_u64(u64 x, int o) {
    const uint32_t lo = __shfl_xor((uint32_t)x, o, 64);
    const uint32_t hi = __shfl_xor((uint32_t)(x >> 32), o, 64);
    return ((u64)hi << 32) | lo;
}

__device__ __forceinline__ u64 wave_incl_scan_u64(u64 x) {
    const int lane = threadIdx.x & 63;
    for (int o = 1; o < 64; o <<= 1) {
        const u64 y = shfl_up_u64(x, o);
        if (lane >= o) x += y;
    }
    return x;
}

__device__ __forceinline__ u64 wave_sum_u64(u64 x) {
    for (int o = 32; o >= 1; o >>= 1) x += shfl_xor_u64(x, o);
    return x;
}

__device__ __forceinline__ float wave_incl_scan_f(float x) {
    const int lane = threadIdx.x & 63;
    for (int o = 1; o < 64; o <<= 1) {
        const float y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
    }
    return x;
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

__device__ float block_max_f(float v, RowShared& sh) {
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0) sh.fred[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = sh.fred[0];
    for (int w = 1; w < kRW; ++w) r = fmaxf(r, sh.fred[w]);
    __syncthreads();
    return r;
}

__device__ float block_sum_f(float v, RowShared& sh) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) sh.fred[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = 0.f;
    for (int w = 0; w < kRW; ++w) r += sh.fred[w];
    __syncthreads();
    return r;
}

// First index holding the maximum of v over the block (v = -inf for no candidate).
__device__ int block_argmax(float v, int i, RowShared& sh) {
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(v, o, 64);
        const int oi = __shfl_xor(i, o, 64);
        if (ov > v || (ov == v && oi < i)) {
            v = ov;
            i = oi;
        }
    }
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
__device__ int desc_search(const Row& r, Member member, MassOf mass_of, u64 theta, bool strict, RowShared& sh,
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

// Bin (of kBins) where the running total of h, taken from the top bin down, first reaches theta
// (exceeds it when strict); -1 if it never does. Whole block.
template <class H>
__device__ int desc_bin_search(const H* h, u64 theta, bool strict, RowShared& sh) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int j0 = 2 * tid, j1 = 2 * tid + 1;  // descending positions
    const u64 m0 = (u64)h[kBins - 1 - j0], m1 = (u64)h[kBins - 1 - j1];
    const u64 incl = wave_incl_scan_u64(m0 + m1);
    if (lane == 63) sh.wsum[wave] = incl;
    if (tid == 0) sh.found = -1;
    __syncthreads();
    u64 base = 0;
    for (int w = 0; w < wave; ++w) base += sh.wsum[w];
    const u64 ex0 = base + incl - (m0 + m1), in0 = ex0 + m0, in1 = in0 + m1;
    auto crosses = [&](u64 ex, u64 in) { return strict ? (ex <= theta && in > theta) : (ex < theta && in >= theta); };
    if (m0 && crosses(ex0, in0)) sh.found = kBins - 1 - j0;
    else if (m1 && crosses(in0, in1)) sh.found = kBins - 1 - j1;
    __syncthreads();
    const int d = sh.found;
    __syncthreads();
    return d;
}

// Sorts a[0, n) (n a power of two, at most kCap) into descending order. Whole block.
__device__ void bitonic_desc(u64* a, int n) {
    for (int size = 2; size <= n; size <<= 1) {
        for (int sb = __builtin_ctz((unsigned)size) - 1; sb >= 0; --sb) {  // stride = 2^sb
            const int stride = 1 << sb;
            for (int i = threadIdx.x; i < (n >> 1); i += kRT) {
                const int lo = ((i >> sb) << (sb + 1)) + (i & (stride - 1)), hi = lo + stride;
                const bool desc = (lo & size) == 0;
                const u64 x = a[lo], y = a[hi];
                if (desc ? x < y : x > y) {
                    a[lo] = y;
                    a[hi] = x;
                }
            }
            __syncthreads();
        }
    }
}

// In-place inclusive scan of a[0, n), n <= kCap: thread t owns 8 consecutive entries.
__device__ void block_scan_incl(float* a, int n, RowShared& sh) {
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
__device__ int first_at_least(const float* c, int n, float x, bool strict, RowShared& sh) {
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

__device__ __forceinline__ bool row_has_proc(const SampleArgs& a, int b) {
    return (a.bias_off && a.bias_off[b + 1] > a.bias_off[b]) || (a.pen_off && a.pen_off[b + 1] > a.pen_off[b]) ||
           (a.mask_row && a.mask_row[b] >= 0);
}

// Copies rows that have a processor into the workspace, adding -inf where the mask disallows.
__global__ __launch_bounds__(256) void sample_prepare_kernel(SampleArgs a) {
    const int b = blockIdx.y;
    if (!row_has_proc(a, b)) return;
    const float* x = a.logits + (size_t)b * a.V;
    float* y = a.ws + (size_t)b * a.V;
    const int mr = a.mask_row ? a.mask_row[b] : -1;
    const uint32_t* mask = (mr >= 0 && mr < a.num_masks) ? a.mask + (size_t)mr * a.mask_words : nullptr;
    if (a.mask_row && mr >= a.num_masks) {
        if (blockIdx.x == 0 && threadIdx.x == 0) latch_error(a.err, ERR_TOKEN);
    }
    const int v0 = blockIdx.x * 4096;
    for (int v = v0 + threadIdx.x; v < min(a.V, v0 + 4096); v += 256) {
        float g = 0.0f;
        if (mask && !((mask[v >> 5] >> (v & 31)) & 1u)) g = -__builtin_huge_valf();
        y[v] = x[v] + g;
    }
}

__global__ __launch_bounds__(kRT) void sample_row_kernel(SampleArgs a) {
    __shared__ RowShared sh;
    const int b = blockIdx.x, tid = threadIdx.x;
    const int V = a.V;
    const bool proc = row_has_proc(a, b);
    const float* y = proc ? a.ws + (size_t)b * V : a.logits + (size_t)b * V;
    if (proc) {
        // Bias first, then penalty (worker.rs:142-181). Entries of one list have distinct tokens.
        float* w = a.ws + (size_t)b * V;
        if (a.bias_off) {
            for (int i = a.bias_off[b] + tid; i < a.bias_off[b + 1]; i += kRT) {
                const uint32_t t = a.bias_tok[i];
                if (t < (uint32_t)V) w[t] = w[t] + a.bias_val[i];
                else latch_error(a.err, ERR_TOKEN);
            }
            __syncthreads();
        }
        if (a.pen_off) {
            for (int i = a.pen_off[b] + tid; i < a.pen_off[b + 1]; i += kRT) {
                const uint32_t t = a.pen_tok[i];
                if (t < (uint32_t)V) w[t] = w[t] + a.pen_val[i];
                else latch_error(a.err, ERR_TOKEN);
            }
        }
        __syncthreads();
    }
    const float T = a.temperature[b];
    const bool vec4 = a.vec4;
    if (!(T > 0.f)) {  // argmax of the processed logits
        float bv = -__builtin_huge_valf();
        int bi = 0x7fffffff;
        row_for_each(y, V, vec4, [&](int v, float x) {
            if (x > bv) {
                bv = x;
                bi = v;
            }
        });
        const int best = block_argmax(bv, bi, sh);
        if (tid == 0) a.out[b] = (uint32_t)(best == 0x7fffffff ? 0 : best);
        return;
    }
    Row r;
    r.y = y;
    r.V = V;
    r.vec4 = vec4;
    r.s = (float)(1.0 / (double)T);
    r.kk = 0;
    r.ki = V;
    r.ck = 0;
    r.ci = V;
    const int k = a.top_k ? a.top_k[b] : 0;
    const float tp = a.top_p ? a.top_p[b] : 1.0f;
    const bool use_k = k > 0 && k < V;
    const bool use_p = tp < 1.0f;
    const float u = a.u[b];
    const int lane = tid & 63, wave = tid >> 6;
    if (!use_k && !use_p) {
        float mx = -__builtin_huge_valf();
        row_for_each(y, V, vec4, [&](int, float yv) { mx = fmaxf(mx, yv * r.s + 0.0f); });
        r.m = block_max_f(mx, sh);
        if (r.m == -__builtin_huge_valf()) {  // every token disallowed
            if (tid == 0) a.out[b] = (uint32_t)(V - 1);
            return;
        }
        // Index order: wave w owns the contiguous chunk [w L, w L + L) (L a multiple of 256).
        // The chunk sums of exp(z - max) give the total and the crossing chunk; that wave then
        // walks its chunk 256 entries at a time (4 consecutive per lane).
        const int L = ((V + kRW - 1) / kRW + 255) & ~255;
        const int c0 = min(V, wave * L), c1 = min(V, c0 + L);
        auto ev = [&](int v) { return v < c1 ? r.e(y[v] * r.s + 0.0f) : 0.f; };
        // Four consecutive entries of lane l in tile t0: one 16-byte load when the row allows.
        auto ev4 = [&](int v, float& e0, float& e1, float& e2, float& e3) {
            if (vec4 && v + 3 < c1) {
                const float4 q = *reinterpret_cast<const float4*>(y + v);
                e0 = r.e(q.x * r.s + 0.0f);
                e1 = r.e(q.y * r.s + 0.0f);
                e2 = r.e(q.z * r.s + 0.0f);
                e3 = r.e(q.w * r.s + 0.0f);
            } else {
                e0 = ev(v);
                e1 = ev(v + 1);
                e2 = ev(v + 2);
                e3 = ev(v + 3);
            }
        };
        float part = 0.f;
#pragma unroll 4
        for (int t0 = c0; t0 < c1; t0 += 256) {
            float e0, e1, e2, e3;
            ev4(t0 + 4 * lane, e0, e1, e2, e3);
            part += (e0 + e1) + (e2 + e3);
        }
        part = wave_sum(part);
        if (lane == 0) sh.fred[wave] = part;
        if (tid == 0) sh.found = -1;
        __syncthreads();
        float zsum = 0.f, wb = 0.f;
        for (int w = 0; w < kRW; ++w) {
            if (w == wave) wb = zsum;
            zsum += sh.fred[w];
        }
        const float rr = u * zsum;  // r = u in probability; compare running sums of exp(z - max)
        const bool my_wave = (wave == 0 && rr <= 0.f) ||
                             (wb < rr && (wb + sh.fred[wave] >= rr || wave == kRW - 1));
        if (my_wave) {
            for (int t0 = c0; t0 < c1; t0 += 256) {
                const int v = t0 + 4 * lane;
                float e0, e1, e2, e3;
                ev4(v, e0, e1, e2, e3);
                const float mine = (e0 + e1) + (e2 + e3);
                const float in = wb + wave_incl_scan_f(mine);
                const unsigned long long bal = __ballot(in >= rr);
                if (bal) {
                    const int l = __ffsll((long long)bal) - 1;
                    if (lane == l) {  // the lane's four entries in order
                        const float c0r = in - mine + e0, c1r = c0r + e1, c2r = c1r + e2;
                        int pick = min(v + 3, c1 - 1);
                        if (c2r >= rr) pick = v + 2;
                        if (c1r >= rr) pick = v + 1;
                        if (c0r >= rr) pick = v;
                        sh.found = pick;
                    }
                    break;
                }
                wb = __shfl(in, 63, 64);
            }
        }
        __syncthreads();
        if (tid == 0) a.out[b] = (uint32_t)(sh.found >= 0 ? sh.found : V - 1);
        return;
    }

    // Filtered: max and the histogram of the top 11 key bits.
    for (int i = tid; i < kBins; i += kRT) {
        sh.cnt[i] = 0;
        sh.hist[i] = 0;
    }
    __syncthreads();
    {
        float mx = -__builtin_huge_valf();
        row_for_each(y, V, vec4, [&](int, float yv) {
            const float zv = yv * r.s + 0.0f;
            mx = fmaxf(mx, zv);
            atomicAdd(&sh.cnt[order_key(zv) >> 21], 1u);
        });
        r.m = block_max_f(mx, sh);
    }
    if (r.m == -__builtin_huge_valf()) {
        if (tid == 0) a.out[b] = (uint32_t)(V - 1);
        return;
    }
    // Candidate bins: from the top down to the bin holding the k-th token (top-k), or one bin
    // below the bin where the running mass of exp(z - max) passes top_p (top-p alone).
    int tb;
    if (use_k) {
        tb = desc_bin_search(sh.cnt, (u64)k, false, sh);
    } else {
        float zs = 0.f;
        row_for_each(y, V, vec4, [&](int, float yv) {
            const float zv = yv * r.s + 0.0f;
            const float e = r.e(zv);
            zs += e;
            atomicAdd(&sh.hist[order_key(zv) >> 21], (u64)llrint((double)e * kFixE));
        });
        r.z_sum = block_sum_f(zs, sh);
        u64 tot = 0;
        for (int i = lane; i < kBins; i += 64) tot += sh.hist[i];
        tot = wave_sum_u64(tot);
        tb = desc_bin_search(sh.hist, (u64)llrint((double)tp * (double)tot), true, sh);
        tb = tb > 0 ? tb - 1 : 0;
    }
    uint32_t ncand = 0xffffffffu;  // candidates: tokens in bins tb and above (every wave sums all bins)
    if (tb >= 0) {
        u64 c = 0;
        for (int i = tb + lane; i < kBins; i += 64) c += sh.cnt[i];
        ncand = (uint32_t)wave_sum_u64(c);
    }
    if (tb >= 0 && ncand <= (uint32_t)kCap) {
        if (tid == 0) sh.count = 0;
        __syncthreads();
        row_for_each(y, V, vec4, [&](int v, float yv) {
            const uint32_t key = order_key(yv * r.s + 0.0f);
            if ((int)(key >> 21) >= tb) {
                const int slot = atomicAdd(&sh.count, 1);
                sh.cand[slot] = ((u64)key << 32) | (uint32_t)~(uint32_t)v;
            }
        });
        __syncthreads();
        const int n = sh.count;
        int np2 = 2;
        while (np2 < n) np2 <<= 1;
        for (int i = n + tid; i < np2; i += kRT) sh.cand[i] = 0;
        __syncthreads();
        bitonic_desc(sh.cand, np2);
        const int ns = use_k ? min(k, n) : n;
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
            if (!use_k && cut == ns && n < V) cut = -1;  // the cut lies past the candidates
            if (cut > 0) rr = u * sh.cum[cut - 1];
        }
        if (cut > 0) {
            int pick = first_at_least(sh.cum, cut, rr, false, sh);
            if (pick < 0) pick = use_p ? 0 : ns - 1;
            if (tid == 0) a.out[b] = ~(uint32_t)sh.cand[pick];
            return;
        }
    }
    // Radix selects over the whole row (candidates did not fit in LDS).
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
        row_for_each(y, V, vec4, [&](int v, float yv) {
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

}  // namespace

hipError_t launch_sample(const SampleArgs& a, hipStream_t stream) {
    if (a.B == 0) return hipSuccess;
    if (a.bias_off || a.pen_off || a.mask_row) {
        const dim3 grid((unsigned)((a.V + 4095) / 4096), (unsigned)a.B);
        sample_prepare_kernel<<<grid, 256, 0, stream>>>(a);
    }
    sample_row_kernel<<<dim3((unsigned)a.B), kRT, 0, stream>>>(a);
    return hipGetLastError();
}

}  // namespace kyro
