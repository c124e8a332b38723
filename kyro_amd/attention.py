"""PagedAttention — host mirror of the reference type, running the gfx950 kernels.

Mirrors ``PagedAttention { block_size, num_heads, head_dim, num_kv_heads }`` and its ``forward``
(src/model/attention_kernel.rs:4-31). Tensors are device tensors in the reference's layouts:

    query        [batch, num_heads, head_dim]  or  [total_q, num_heads, head_dim] with q_start_loc
    key_cache    [num_blocks, num_kv_heads, block_size, head_dim]
    value_cache  [num_blocks, num_kv_heads, block_size, head_dim]
    block_table  [batch, max_num_blocks_per_seq]  int64
    context_lens [batch]  int64 (includes the sequence's own query positions)

The result is float32 like the reference (``out_dtype`` may ask for bf16). Unlike the
reference it takes several query rows per sequence (the k+1 verify positions, causal among
themselves) and it does not reproduce the reference's head/token score permutation at
attention_kernel.rs:104-111; it computes softmax(q K^T / sqrt(D)) V per head.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

_DTYPES = {torch.float32: _lib.KYRO_F32, torch.bfloat16: _lib.KYRO_BF16}
_PATHS = {"auto": _lib.KYRO_ATTN_AUTO, "vector": _lib.KYRO_ATTN_VECTOR, "mfma": _lib.KYRO_ATTN_MFMA}
_KV_REUSE = {"auto": _lib.KYRO_KV_REUSE_AUTO, "shared": _lib.KYRO_KV_REUSE_SHARED,
             "stream": _lib.KYRO_KV_REUSE_STREAM}
_SCHEDULES = {"auto": _lib.KYRO_ATTN_SCHEDULE_AUTO, "grid": _lib.KYRO_ATTN_SCHEDULE_GRID,
              "balanced": _lib.KYRO_ATTN_SCHEDULE_BALANCED}


def _require(t: torch.Tensor, name: str, dtype=None, ndim=None, device=None):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if dtype is not None and t.dtype not in (dtype if isinstance(dtype, tuple) else (dtype,)):
        raise TypeError(f"{name} has dtype {t.dtype}, expected {dtype}")
    if ndim is not None and t.dim() != ndim:
        raise ValueError(f"{name} must be {ndim}-D, got shape {tuple(t.shape)}")
    if device is not None and t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


class PagedAttention:
    """Software PagedAttention on MI355X (attention_kernel.rs:4-19)."""

    def __init__(self, block_size: int, num_heads: int, head_dim: int, num_kv_heads: int):
        self.block_size = int(block_size)
        self.num_heads = int(num_heads)
        self.head_dim = int(head_dim)
        self.num_kv_heads = int(num_kv_heads)

    def forward(self, query, key_cache, value_cache, block_table, context_lens, *,
                q_start_loc=None, max_q_len=None, causal=True, out_dtype=torch.float32,
                path="auto", num_splits=0, scale=None, out=None, kv_reuse="auto", schedule="auto"):
        """Attention of every query row against its sequence's paged context.

        ``q_start_loc`` (int32 [batch+1]) gives each sequence's rows of ``query``; ``max_q_len``
        bounds the rows per sequence (computed from q_start_loc when omitted). ``kv_reuse`` is a
        cache-policy hint for the K/V loads that never changes the result: "auto" streams them
        when each cached slab is read once per launch, "shared" keeps them cacheable for tables
        that share blocks between sequences (``BlockManager.write_tables`` reports that),
        "stream" streams them regardless. ``schedule`` ("auto", "grid", "balanced") chooses how
        the MFMA kernel spreads work over the chip: "balanced" reads the context lengths on the
        device and starts the longest work first (for batches of very different lengths). The call
        synchronises, so errors the device detects (bad block ids, context lengths beyond the
        table) raise KyroError here, as the reference returns Err from ``forward``;
        :meth:`forward_async` is the non-blocking variant.
        """
        out = self.forward_async(query, key_cache, value_cache, block_table, context_lens,
                                 q_start_loc=q_start_loc, max_q_len=max_q_len, causal=causal,
                                 out_dtype=out_dtype, path=path, num_splits=num_splits,
                                 scale=scale, out=out, kv_reuse=kv_reuse, schedule=schedule)
        _lib.context(query.device.index or 0).sync()
        return out

    def forward_async(self, query, key_cache, value_cache, block_table, context_lens, *,
                      q_start_loc=None, max_q_len=None, causal=True, out_dtype=torch.float32,
                      path="auto", num_splits=0, scale=None, out=None, kv_reuse="auto", schedule="auto",
                      context=None):
        """Queues the kernel on torch's current stream and returns without synchronising.
        Device-detected errors surface at the next ``kyro_amd.sync(device)``. ``context`` (a
        ``kyro_amd._lib.Context``) runs the call on that context and its arena instead of the
        process-wide one of the device."""
        dev = query.device
        if dev.type != "cuda":
            raise ValueError("PagedAttention.forward runs on a GPU device; got " + str(dev))
        _require(query, "query", dtype=(torch.float32, torch.bfloat16), ndim=3)
        _require(key_cache, "key_cache", dtype=query.dtype, ndim=4, device=dev)
        _require(value_cache, "value_cache", dtype=query.dtype, ndim=4, device=dev)
        _require(block_table, "block_table", dtype=torch.int64, ndim=2, device=dev)
        _require(context_lens, "context_lens", dtype=torch.int64, ndim=1, device=dev)
        if key_cache.shape != value_cache.shape:
            raise ValueError("key_cache and value_cache shapes differ")
        nb, hkv, bs, d = key_cache.shape
        if (hkv, bs, d) != (self.num_kv_heads, self.block_size, self.head_dim):
            raise ValueError(f"cache shape {tuple(key_cache.shape)} does not match "
                             f"(num_blocks, {self.num_kv_heads}, {self.block_size}, {self.head_dim})")
        total_q, h, dq = query.shape
        if (h, dq) != (self.num_heads, self.head_dim):
            raise ValueError(f"query shape {tuple(query.shape)} does not match "
                             f"(*, {self.num_heads}, {self.head_dim})")
        batch = context_lens.shape[0]
        if block_table.shape[0] != batch:
            raise ValueError("block_table and context_lens disagree on the batch size")
        if q_start_loc is not None:
            _require(q_start_loc, "q_start_loc", dtype=torch.int32, ndim=1, device=dev)
            if q_start_loc.shape[0] != batch + 1:
                raise ValueError("q_start_loc must have batch+1 entries")
            if max_q_len is None:
                max_q_len = int((q_start_loc[1:] - q_start_loc[:-1]).max().item()) if batch else 1
        else:
            if total_q != batch:
                raise ValueError("query rows must equal the batch size without q_start_loc")
            max_q_len = 1
        if out_dtype not in _DTYPES:
            raise TypeError(f"out_dtype must be float32 or bfloat16, got {out_dtype}")
        if out is None:
            out = torch.empty((total_q, h, d), dtype=out_dtype, device=dev)
        else:
            _require(out, "out", dtype=out_dtype, ndim=3, device=dev)
            if tuple(out.shape) != (total_q, h, d):
                raise ValueError("out has the wrong shape")
        params = _lib.PagedAttentionParams(
            self.block_size, self.num_heads, self.head_dim, self.num_kv_heads, batch, total_q,
            block_table.shape[1], nb, _DTYPES[query.dtype], _DTYPES[out_dtype], 1 if causal else 0,
            float(scale) if scale else 0.0, _PATHS[path], int(num_splits), int(max_q_len),
            _KV_REUSE[kv_reuse], _SCHEDULES[schedule])
        ctx = context if context is not None else _lib.context(dev.index or 0)
        ctx.set_stream(torch.cuda.current_stream(dev).cuda_stream)
        _lib.check(_lib.lib().kyro_paged_attention_mq(
            ctx.handle, ctypes.byref(params), query.data_ptr(),
            q_start_loc.data_ptr() if q_start_loc is not None else None,
            key_cache.data_ptr(), value_cache.data_ptr(), block_table.data_ptr(),
            context_lens.data_ptr(), out.data_ptr()))
        return out


def describe_attention(attn: PagedAttention, *, batch: int, total_q: int, max_q_len: int, max_blocks_per_seq: int,
                       num_blocks: int, dtype=torch.bfloat16, out_dtype=torch.bfloat16, causal=True, path="auto",
                       num_splits=0, kv_reuse="auto", schedule="auto", device=None) -> str:
    """What ``forward`` with these shapes launches on ``device`` (kernel instance, schedule,
    splits, workgroups), from the library's own choice (``kyro_paged_attention_describe``).
    ``device`` None asks the host-only question for a 256-CU device (no GPU needed)."""
    params = _lib.PagedAttentionParams(
        attn.block_size, attn.num_heads, attn.head_dim, attn.num_kv_heads, int(batch), int(total_q),
        int(max_blocks_per_seq), int(num_blocks), _DTYPES[dtype], _DTYPES[out_dtype], 1 if causal else 0, 0.0,
        _PATHS[path], int(num_splits), int(max_q_len), _KV_REUSE[kv_reuse], _SCHEDULES[schedule])
    handle = _lib.context(device).handle if device is not None else None
    return _lib.describe_text(_lib.lib().kyro_paged_attention_describe, handle, ctypes.byref(params), 1)


def attention_plan(attn: PagedAttention, context_lens, q_lens=None, *, max_blocks_per_seq: int,
                   num_blocks: int = 1, dtype=torch.bfloat16, schedule: str = "balanced",
                   num_cus: int = 0, chunk_quarters: int = 0):
    """The balanced schedule's plan of a batch, computed on the host by the library
    (``kyro_paged_attention_plan``) from host arrays of context lengths and per-sequence query
    rows. No GPU is needed. Returns (kyro_attention_plan fields as a dict, splits per sequence)."""
    import numpy as np

    ctx = np.ascontiguousarray(context_lens, dtype=np.int64)
    batch = int(ctx.shape[0])
    ql = None if q_lens is None else np.ascontiguousarray(q_lens, dtype=np.int32)
    total_q = batch if ql is None else int(ql.sum())
    max_q_len = 1 if ql is None else max(1, int(ql.max()) if batch else 1)
    params = _lib.PagedAttentionParams(
        attn.block_size, attn.num_heads, attn.head_dim, attn.num_kv_heads, batch, total_q,
        int(max_blocks_per_seq), int(num_blocks), _DTYPES[dtype], _lib.KYRO_F32, 1, 0.0, _lib.KYRO_ATTN_MFMA, 0,
        max_q_len, _lib.KYRO_KV_REUSE_AUTO, _SCHEDULES[schedule])
    out = _lib.AttentionPlan()
    splits = np.zeros(batch, np.int32)
    _lib.check(_lib.lib().kyro_paged_attention_plan(
        ctypes.byref(params), int(num_cus), int(chunk_quarters), ctx.ctypes.data,
        ql.ctypes.data if ql is not None else None, splits.ctypes.data, ctypes.byref(out)))
    info = {f: getattr(out, f) for f, _ in _lib.AttentionPlan._fields_}
    return info, splits
