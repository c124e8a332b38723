"""kyro_amd — the speculative-decoding verify step of Kyro on MI355X (gfx950).

HIP kernels behind the C ABI in include/kyro_verify.h (libkyro_verify.so):
multi-query paged attention over a block-table KV cache, fused rejection-sampling
acceptance, and the paged KV write. This package is the Python host mirror of the reference's interface:

    PagedAttention(block_size, num_heads, head_dim, num_kv_heads).forward(...)
        (src/model/attention_kernel.rs:4-31)
    verify_drafts(...)  (src/speculative.rs:286-339, extended to p/q rejection sampling)
    PagedKVCache(block_size, num_kv_heads, head_dim).append_kv(...)
        (src/model/kv_cache.rs:49-75, for the block-table cache the attention reads)
    BlockManager(block_size, num_gpu_blocks, num_cpu_blocks), RadixCache(max_capacity)
        (src/scheduler/block_manager.rs, src/scheduler/radix_cache.rs) and the device tables
    sample_tokens(...)  (src/worker.rs:141-197 logit processors, then sample_token :267-362)
    NgramTable(corpus, order).draft(...)  (src/speculative.rs:196-256, the Ngram draft strategy)
"""
from ._lib import Context, KyroError, context, lib
from .attention import PagedAttention
from .block_manager import BlockManager, RadixCache, copy_blocks
from .drafting import NgramTable, context_tails
from .kv_cache import PagedKVCache
from .sampling import grammar_mask, penalty_adds, sample_token, sample_tokens, sample_tokens_async
from .speculative import VerifyResult, verify_drafts, verify_drafts_async

__all__ = ["BlockManager", "Context", "KyroError", "NgramTable", "PagedAttention", "PagedKVCache", "RadixCache",
           "context_tails",
           "VerifyResult", "context", "copy_blocks", "grammar_mask", "lib", "penalty_adds", "sample_token",
           "sample_tokens", "sample_tokens_async",
           "sync", "verify_drafts", "verify_drafts_async"]


def sync(device: int = 0) -> None:
    """Waits for the device's queued verify-step work and raises on latched device errors."""
    context(device).sync()
