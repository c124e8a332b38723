"""kyro_amd — the speculative-decoding verify step of Kyro on MI355X (gfx950).

Two HIP kernels behind the C ABI in include/kyro_verify.h (libkyro_verify.so):
multi-query paged attention over a block-table KV cache, and fused rejection-sampling
acceptance. This package is the Python host mirror of the reference's interface:

    PagedAttention(block_size, num_heads, head_dim, num_kv_heads).forward(...)
        (src/model/attention_kernel.rs:4-31)
    verify_drafts(...)  (src/speculative.rs:286-339, extended to p/q rejection sampling)
"""
from ._lib import Context, KyroError, context, lib
from .attention import PagedAttention
from .speculative import VerifyResult, verify_drafts, verify_drafts_async

__all__ = ["Context", "KyroError", "PagedAttention", "VerifyResult", "context", "lib",
           "sync", "verify_drafts", "verify_drafts_async"]


def sync(device: int = 0) -> None:
    """Waits for the device's queued verify-step work and raises on latched device errors."""
    context(device).sync()
