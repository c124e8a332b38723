// Paged KV write for the new rows of a step (the k + 1 draft positions of a verify step, or a
// prompt's rows at prefill) on gfx950.
//
// Replaces KVCacheManager::append_kv (src/model/kv_cache.rs:49-75) for a block-table cache:
// the reference concatenates a request's new [1, seq_len, Hkv, D] rows onto per-request tensors
// before attention (src/model/llama.rs:80-84); here row j of sequence b lands at token position
// ctx - q_len + j, i.e. slot (p % bs) of block block_table[b][p / bs], in the
// [num_blocks, Hkv, bs, D] layout attention reads.
//
// Pure data movement: each thread moves 8 consecutive elements of one (row, kv head) of K and of
// V (16-byte loads for bf16 rows, two for f32 rows), converting f32 to bf16 with
// round-to-nearest-even when the cache is bf16. grid = (chunks of a sequence's rows, sequence);
// a sequence's bounds, context length and block ids are validated on the device and latched as
// errors (the offending rows are skipped).
#include "common.hpp"
#include "kernels.hpp"

namespace kyro {
namespace {

constexpr int kThreads = 256;

// f32 -> bf16, round to nearest even (overflow rounds to infinity, subnormals round like any
// other value); every NaN becomes the canonical quiet NaN 0x7FC0.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

struct Row8 {
    float f[8];
};

template <bool SRC_BF16>
__device__ __forceinline__ void load_row8(const void* base, size_t off, Row8& r, uint4& raw) {
    if constexpr (SRC_BF16) {
        raw = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(base) + off);
    } else {
        const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(base) + off);
        const float4 x = p[0], y = p[1];
        r.f[0] = x.x; r.f[1] = x.y; r.f[2] = x.z; r.f[3] = x.w;
        r.f[4] = y.x; r.f[5] = y.y; r.f[6] = y.z; r.f[7] = y.w;
    }
}

template <bool SRC_BF16, bool CACHE_BF16>
__device__ __forceinline__ void store_row8(void* base, size_t off, const Row8& r, const uint4& raw) {
    if constexpr (CACHE_BF16) {
        uint4 o;
        if constexpr (SRC_BF16) {
            o = raw;
        } else {
            o.x = f32_to_bf16_bits(r.f[0]) | (f32_to_bf16_bits(r.f[1]) << 16);
            o.y = f32_to_bf16_bits(r.f[2]) | (f32_to_bf16_bits(r.f[3]) << 16);
            o.z = f32_to_bf16_bits(r.f[4]) | (f32_to_bf16_bits(r.f[5]) << 16);
            o.w = f32_to_bf16_bits(r.f[6]) | (f32_to_bf16_bits(r.f[7]) << 16);
        }
        *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(base) + off) = o;
    } else {
        float v[8];
        if constexpr (SRC_BF16) {
            const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[2 * i] = bf16_lo(w[i]);
                v[2 * i + 1] = bf16_hi(w[i]);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = r.f[i];
        }
        float4* p = reinterpret_cast<float4*>(reinterpret_cast<float*>(base) + off);
        p[0] = make_float4(v[0], v[1], v[2], v[3]);
        p[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
}

template <bool SRC_BF16, bool CACHE_BF16>
__global__ __launch_bounds__(kThreads) void kv_append_kernel(KvAppendArgs a) {
    const int b = blockIdx.y;
    int r0 = b, r1 = b + 1;
    if (a.q_start) {
        r0 = a.q_start[b];
        r1 = a.q_start[b + 1];
    }
    const int64_t ctx = a.ctx_lens[b];
    const int q_len = r1 - r0;
    const bool lead = blockIdx.x == 0 && threadIdx.x == 0;  // reports the sequence's errors once
    if (r0 < 0 || r1 < r0 || r1 > a.total_q || q_len > a.max_q_len) {
        if (lead) latch_error(a.err, ERR_Q_LAYOUT);
        return;
    }
    if (ctx < q_len || ctx > (int64_t)a.max_blocks * a.bs) {
        if (lead) latch_error(a.err, ERR_CTX_LEN);
        return;
    }
    const int v = blockIdx.x * kThreads + (int)threadIdx.x;  // 8-element vector within the rows
    const int j = v / a.vecs_per_row;
    if (j >= q_len) return;
    const int within = v - j * a.vecs_per_row;  // = h * (D / 8) + d8
    const int h = within / (a.D / 8);
    const int d = (within - h * (a.D / 8)) * 8;
    // The rows and the block id are independent loads: issue them together.
    const size_t src = ((size_t)(r0 + j) * a.Hkv + h) * a.D + d;
    Row8 rk, rv;
    uint4 raw_k, raw_v;
    load_row8<SRC_BF16>(a.key, src, rk, raw_k);
    load_row8<SRC_BF16>(a.value, src, rv, raw_v);
    const int64_t pos = ctx - q_len + j;
    const int64_t blk = a.table[(size_t)b * a.max_blocks + (size_t)(pos / a.bs)];
    if (blk < 0 || blk >= a.num_blocks) {
        if (d == 0) latch_error(a.err, ERR_BLOCK_ID);
        return;
    }
    const int slot = (int)(pos % a.bs);
    const size_t dst = (((size_t)blk * a.Hkv + h) * a.bs + slot) * a.D + d;
    store_row8<SRC_BF16, CACHE_BF16>(a.kc, dst, rk, raw_k);
    store_row8<SRC_BF16, CACHE_BF16>(a.vc, dst, rv, raw_v);
}

// One workgroup column per pair: consecutive threads copy consecutive 16-byte vectors of the
// block's [Hkv, bs, D] slab in both caches.
__global__ __launch_bounds__(kThreads) void copy_blocks_kernel(CopyBlocksArgs a) {
    const int64_t pair = blockIdx.y;
    const int64_t v = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (v >= a.slab_vecs) return;
    const int64_t src = a.pairs ? a.pairs[pair] : a.inl[0][pair];
    const int64_t dst = a.pairs ? a.pairs[a.n + pair] : a.inl[1][pair];
    a.kc[dst * a.slab_vecs + v] = a.kc[src * a.slab_vecs + v];
    a.vc[dst * a.slab_vecs + v] = a.vc[src * a.slab_vecs + v];
}

}  // namespace

hipError_t launch_copy_blocks(const CopyBlocksArgs& a, hipStream_t stream) {
    if (a.n == 0) return hipSuccess;
    const dim3 grid((unsigned)((a.slab_vecs + kThreads - 1) / kThreads), (unsigned)a.n);
    copy_blocks_kernel<<<grid, kThreads, 0, stream>>>(a);
    return hipGetLastError();
}

hipError_t launch_kv_append(const KvAppendArgs& a, hipStream_t stream) {
    if (a.B == 0 || a.max_q_len == 0) return hipSuccess;
    const long long vecs = (long long)a.max_q_len * a.vecs_per_row;
    const dim3 grid((unsigned)((vecs + kThreads - 1) / kThreads), (unsigned)a.B);
    if (a.src_bf16) {
        if (a.cache_bf16) kv_append_kernel<true, true><<<grid, kThreads, 0, stream>>>(a);
        else kv_append_kernel<true, false><<<grid, kThreads, 0, stream>>>(a);
    } else {
        if (a.cache_bf16) kv_append_kernel<false, true><<<grid, kThreads, 0, stream>>>(a);
        else kv_append_kernel<false, false><<<grid, kThreads, 0, stream>>>(a);
    }
    return hipGetLastError();
}

}  // namespace kyro
