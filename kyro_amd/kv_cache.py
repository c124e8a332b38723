"""Paged KV write — host mirror of KVCacheManager::append_kv for a block-table cache.

The reference keeps one growing [1, seq, Hkv, D] tensor per request and appends the new rows
with a concatenation before attention (src/model/kv_cache.rs:49-75, called at
src/model/llama.rs:80-84). Here the cache is the paged [num_blocks, Hkv, block_size, D] layout
that :class:`kyro_amd.PagedAttention` reads, and a batch of sequences appends in one launch:
new row j of a sequence with q_len new rows and context length ctx (counted after the append,
as attention counts it) lands at token position ctx - q_len + j.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

_DTYPES = {torch.float32: _lib.KYRO_F32, torch.bfloat16: _lib.KYRO_BF16}


def _require(t, name, dtypes, ndim, device):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.dtype not in dtypes:
        raise TypeError(f"{name} has dtype {t.dtype}, expected one of {dtypes}")
    if t.dim() != ndim:
        raise ValueError(f"{name} must be {ndim}-D, got shape {tuple(t.shape)}")
    if t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


class PagedKVCache:
    """Writes new K/V rows into block-table caches (kv_cache.rs:21-35 holds num_kv_heads and
    head_dim; the block size is the paged layout's)."""

    def __init__(self, block_size: int, num_kv_heads: int, head_dim: int):
        self.block_size = int(block_size)
        self.num_kv_heads = int(num_kv_heads)
        self.head_dim = int(head_dim)

    def append_kv_async(self, key, value, key_cache, value_cache, block_table, context_lens, *,
                        q_start_loc=None, max_q_len=None):
        """Queues the write on torch's current stream; see :meth:`append_kv`."""
        dev = key.device
        if dev.type != "cuda":
            raise ValueError("append_kv runs on a GPU device; got " + str(dev))
        _require(key, "key", (torch.float32, torch.bfloat16), 3, dev)
        _require(value, "value", (key.dtype,), 3, dev)
        _require(key_cache, "key_cache", (torch.float32, torch.bfloat16), 4, dev)
        _require(value_cache, "value_cache", (key_cache.dtype,), 4, dev)
        _require(block_table, "block_table", (torch.int64,), 2, dev)
        _require(context_lens, "context_lens", (torch.int64,), 1, dev)
        total_q, hkv, d = key.shape
        if tuple(value.shape) != tuple(key.shape):
            raise ValueError("key and value must have the same shape")
        if hkv != self.num_kv_heads or d != self.head_dim:
            raise ValueError(f"key rows are [{hkv}, {d}], expected [{self.num_kv_heads}, {self.head_dim}]")
        nb = key_cache.shape[0]
        want = (nb, self.num_kv_heads, self.block_size, self.head_dim)
        if tuple(key_cache.shape) != want or tuple(value_cache.shape) != want:
            raise ValueError(f"caches must be {want}")
        B = context_lens.shape[0]
        if block_table.shape[0] != B:
            raise ValueError("block_table and context_lens disagree on the batch size")
        if q_start_loc is not None:
            _require(q_start_loc, "q_start_loc", (torch.int32,), 1, dev)
            if q_start_loc.shape[0] != B + 1:
                raise ValueError("q_start_loc must have batch+1 entries")
            if max_q_len is None:
                max_q_len = int((q_start_loc[1:] - q_start_loc[:-1]).max().item()) if B else 0
        else:
            if total_q != B:
                raise ValueError("without q_start_loc key must have one row per sequence")
            max_q_len = 1
        params = _lib.KvAppendParams(self.block_size, self.num_kv_heads, self.head_dim, B, total_q,
                                     block_table.shape[1], nb, _DTYPES[key.dtype],
                                     _DTYPES[key_cache.dtype], int(max_q_len))
        ctx = _lib.context(dev.index or 0)
        ctx.set_stream(torch.cuda.current_stream(dev).cuda_stream)
        ptr = lambda t: t.data_ptr() if t is not None else None  # noqa: E731
        _lib.check(_lib.lib().kyro_paged_kv_append(
            ctx.handle, ctypes.byref(params), ptr(key), ptr(value), ptr(q_start_loc),
            ptr(block_table), ptr(context_lens), ptr(key_cache), ptr(value_cache)))

    def append_kv(self, key, value, key_cache, value_cache, block_table, context_lens, *,
                  q_start_loc=None, max_q_len=None):
        """Appends each sequence's new rows (``key``/``value`` [total_q, Hkv, D], rows of sequence b
        at [q_start_loc[b], q_start_loc[b+1]) or row b without q_start_loc) to the caches in place
        and synchronises, so a bad block id or context length raises KyroError here.
        ``context_lens`` is each sequence's length after the append."""
        self.append_kv_async(key, value, key_cache, value_cache, block_table, context_lens,
                             q_start_loc=q_start_loc, max_q_len=max_q_len)
        _lib.context(key.device.index or 0).sync()
