"""KV block allocation with prefix sharing — host mirror of BlockManager and RadixCache.

Mirrors ``BlockManager`` (src/scheduler/block_manager.rs:15-153) and ``RadixCache``
(src/scheduler/radix_cache.rs:29-155) over the C ABI of include/kyro_blocks.h (the logic is
C++ in libkyro_verify.so; nothing here computes). ``BlockManager.write_tables`` produces the
device block table and context lengths the attention and KV-write kernels read, and
:func:`copy_blocks` performs the copy-on-write a partially matched prefix block needs.

Differences from the reference (why: see include/kyro_blocks.h): the prefix tree is keyed by
block contents and shares whole blocks, handing a partially matched block to the request as a
copy; eviction is least-recently-used over the whole tree; references are balanced; a request's
blocks follow its token count (``append_slots`` / ``truncate``).
"""
from __future__ import annotations

import ctypes
from typing import Optional

import numpy as np

from . import _lib


def _u32(tokens) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32).reshape(-1))


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _blocks_out(fn, *args) -> tuple[list[int], int]:
    """Calls a (..., out, cap, out_n, out_extra) entry point twice if the first buffer was short."""
    cap = 64
    while True:
        out = np.zeros(cap, np.int64)
        n, extra = ctypes.c_int64(), ctypes.c_int64()
        _lib.check(fn(*args, _ptr(out), cap, ctypes.byref(n), ctypes.byref(extra)))
        if n.value <= cap:
            return out[: n.value].tolist(), extra.value
        cap = n.value


class RadixCache:
    """RadixCache::new(max_capacity) (radix_cache.rs:38-44) for blocks of ``block_size`` tokens."""

    def __init__(self, max_capacity: int, block_size: int = 16):
        h = ctypes.c_void_p()
        _lib.check(_lib.lib().kyro_radix_create(int(block_size), int(max_capacity), ctypes.byref(h)))
        self._h = h
        self.block_size = int(block_size)
        self.max_capacity = int(max_capacity)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            _lib.lib().kyro_radix_destroy(h)
            self._h = None

    def match_prefix(self, tokens) -> tuple[list[int], int]:
        """(cached block ids, matched token count) — radix_cache.rs:49-86."""
        t = _u32(tokens)
        if t.size == 0:
            return [], 0
        return _blocks_out(lambda o, c, n, m: _lib.lib().kyro_radix_match_prefix(self._h, _ptr(t), t.size, o, c, n, m))

    def insert(self, tokens, block_ids) -> list[bool]:
        """radix_cache.rs:89-120; per block, whether the cache took it."""
        t = _u32(tokens)
        b = np.ascontiguousarray(np.asarray(block_ids, dtype=np.int64).reshape(-1))
        need = -(-t.size // self.block_size)
        if b.size < need:
            raise ValueError(f"{t.size} tokens need {need} blocks, got {b.size}")
        taken = np.zeros(max(need, 1), np.uint8)
        _lib.check(_lib.lib().kyro_radix_insert(self._h, _ptr(t), t.size, _ptr(b), _ptr(taken)))
        return [bool(x) for x in taken[:need]]

    def evict_lru(self) -> list[int]:
        out = np.zeros(max(1, self.num_cached_blocks), np.int64)
        n = ctypes.c_int64()
        _lib.check(_lib.lib().kyro_radix_evict_lru(self._h, _ptr(out), out.size, ctypes.byref(n)))
        return out[: n.value].tolist()

    @property
    def num_cached_blocks(self) -> int:
        return int(_lib.lib().kyro_radix_num_cached_blocks(self._h))


class _BlockTableView:
    """Read-only ``request_id -> [block ids]`` view (the reference's ``block_table`` HashMap)."""

    def __init__(self, bm):
        self._bm = bm

    def __contains__(self, rid) -> bool:
        return self._bm.request(rid) is not None

    def __getitem__(self, rid) -> list[int]:
        r = self._bm.request(rid)
        if r is None:
            raise KeyError(rid)
        return r[0]


class BlockManager:
    """BlockManager::new(block_size, num_gpu_blocks, num_cpu_blocks) (block_manager.rs:32-50)."""

    def __init__(self, block_size: int, num_gpu_blocks: int, num_cpu_blocks: int = 0):
        h = ctypes.c_void_p()
        _lib.check(_lib.lib().kyro_bm_create(int(block_size), int(num_gpu_blocks), int(num_cpu_blocks),
                                             ctypes.byref(h)))
        self._h = h
        self.block_size = int(block_size)
        self.num_gpu_blocks = int(num_gpu_blocks)
        self.num_cpu_blocks = int(num_cpu_blocks)
        self.block_table = _BlockTableView(self)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            _lib.lib().kyro_bm_destroy(h)
            self._h = None

    def allocate_with_prefix(self, request_id: int, prompt_tokens) -> Optional[tuple[list[int], int]]:
        """(blocks, cached token count), or None when the blocks do not fit even after evicting
        the prefix cache (block_manager.rs:53-102)."""
        t = _u32(prompt_tokens)
        cached = ctypes.c_int64()
        rc = _lib.lib().kyro_bm_allocate_with_prefix(self._h, int(request_id), _ptr(t) if t.size else None,
                                                     t.size, ctypes.byref(cached))
        if rc == _lib.KYRO_ENOSPACE:
            return None
        _lib.check(rc)
        return self.block_table[request_id], cached.value

    def allocate(self, request_id: int, num_tokens: int) -> Optional[list[int]]:
        """block_manager.rs:107-124 (no prefix caching)."""
        rc = _lib.lib().kyro_bm_allocate(self._h, int(request_id), int(num_tokens))
        if rc == _lib.KYRO_ENOSPACE:
            return None
        _lib.check(rc)
        return self.block_table[request_id]

    def append_slots(self, request_id: int, n: int) -> bool:
        """Room for n more tokens; False when no blocks are left."""
        rc = _lib.lib().kyro_bm_append_slots(self._h, int(request_id), int(n))
        if rc == _lib.KYRO_ENOSPACE:
            return False
        _lib.check(rc)
        return True

    def truncate(self, request_id: int, num_tokens: int) -> None:
        _lib.check(_lib.lib().kyro_bm_truncate(self._h, int(request_id), int(num_tokens)))

    def free(self, request_id: int, cache_prompt: bool = True) -> None:
        """block_manager.rs:128-153: the prompt's blocks go to the prefix cache."""
        _lib.check(_lib.lib().kyro_bm_free(self._h, int(request_id), 1 if cache_prompt else 0))

    def request(self, request_id: int):
        """(blocks, token count) of a live request, or None."""
        n, nt = ctypes.c_int64(), ctypes.c_int64()
        lib = _lib.lib()
        if lib.kyro_bm_request_blocks(self._h, int(request_id), None, 0, ctypes.byref(n), ctypes.byref(nt)) != 0:
            return None
        out = np.zeros(max(1, n.value), np.int64)
        _lib.check(lib.kyro_bm_request_blocks(self._h, int(request_id), _ptr(out), out.size, ctypes.byref(n),
                                              ctypes.byref(nt)))
        return out[: n.value].tolist(), nt.value

    def take_copies(self) -> list[tuple[int, int]]:
        """Pending (source, destination) block copies from partial prefix matches, handed out once."""
        lib = _lib.lib()
        n = ctypes.c_int64()
        _lib.check(lib.kyro_bm_take_copies(self._h, None, None, 0, ctypes.byref(n)))
        if n.value == 0:
            return []
        src, dst = np.zeros(n.value, np.int64), np.zeros(n.value, np.int64)
        _lib.check(lib.kyro_bm_take_copies(self._h, _ptr(src), _ptr(dst), n.value, ctypes.byref(n)))
        return list(zip(src.tolist(), dst.tolist()))

    def match_prefix(self, tokens) -> tuple[list[int], int]:
        t = _u32(tokens)
        if t.size == 0:
            return [], 0
        return _blocks_out(lambda o, c, n, m: _lib.lib().kyro_bm_match_prefix(self._h, _ptr(t), t.size, o, c, n, m))

    def check(self) -> None:
        """Raises KyroError if reference counts, cache and free pool disagree."""
        _lib.check(_lib.lib().kyro_bm_check(self._h))

    @property
    def num_free_blocks(self) -> int:
        return int(_lib.lib().kyro_bm_num_free_blocks(self._h))

    @property
    def num_cached_blocks(self) -> int:
        return int(_lib.lib().kyro_bm_num_cached_blocks(self._h))

    def write_tables(self, request_ids, block_table, context_lens=None) -> bool:
        """Writes the device block table ([B, max_blocks] int64) and context lengths ([B] int64) of
        the requests, on torch's current stream. Returns True when two of the requests hold a
        common block (then attention over these tables takes ``kv_reuse="shared"``)."""
        import torch

        rid = np.ascontiguousarray(np.asarray(request_ids, dtype=np.uint64).reshape(-1))
        B = rid.size
        if block_table.dtype != torch.int64 or block_table.dim() != 2 or block_table.shape[0] != B \
                or not block_table.is_contiguous():
            raise ValueError("block_table must be a contiguous int64 [B, max_blocks] tensor")
        if context_lens is not None and (context_lens.dtype != torch.int64 or tuple(context_lens.shape) != (B,)):
            raise ValueError("context_lens must be an int64 [B] tensor")
        dev = block_table.device
        ctx = _lib.context(dev.index or 0)
        ctx.set_stream(torch.cuda.current_stream(dev).cuda_stream)
        shared = ctypes.c_int32(0)
        _lib.check(_lib.lib().kyro_bm_write_tables(
            self._h, ctx.handle, _ptr(rid), B, block_table.shape[1], block_table.data_ptr(),
            context_lens.data_ptr() if context_lens is not None else None, ctypes.byref(shared)))
        return bool(shared.value)


def copy_blocks(key_cache, value_cache, pairs) -> None:
    """key_cache[dst] = key_cache[src] (and value_cache) for every (src, dst) pair, on torch's
    current stream; caches are [num_blocks, Hkv, block_size, D] f32 or bf16 device tensors."""
    import torch

    if not pairs:
        return
    dt = {torch.float32: _lib.KYRO_F32, torch.bfloat16: _lib.KYRO_BF16}[key_cache.dtype]
    nb, hkv, bs, d = key_cache.shape
    p = _lib.CopyBlocksParams(bs, hkv, d, nb, dt)
    src = np.ascontiguousarray([s for s, _ in pairs], dtype=np.int64)
    dst = np.ascontiguousarray([t for _, t in pairs], dtype=np.int64)
    dev = key_cache.device
    ctx = _lib.context(dev.index or 0)
    ctx.set_stream(torch.cuda.current_stream(dev).cuda_stream)
    _lib.check(_lib.lib().kyro_copy_blocks(ctx.handle, ctypes.byref(p), key_cache.data_ptr(), value_cache.data_ptr(),
                                           _ptr(src), _ptr(dst), src.size))
