"""N-gram drafting — host mirror of SpeculativeDecoder's Ngram strategy.

``NgramTable(corpus, order)`` is ``build_ngram_table`` (src/speculative.rs:196-208), built by the
library on the host; ``draft`` runs the Ngram arm of ``generate_drafts`` (:239-256) for a batch
on the GPU and returns ``(draft_tokens, num_draft)`` in the layout :func:`kyro_amd.verify_drafts`
takes, so drafting and verification chain on the device.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib


class NgramTable:
    def __init__(self, corpus, order: int):
        seqs = [np.asarray(s, dtype=np.uint32).reshape(-1) for s in corpus]
        offsets = np.zeros(len(seqs) + 1, np.int64)
        for i, s in enumerate(seqs):
            offsets[i + 1] = offsets[i] + s.size
        toks = np.ascontiguousarray(np.concatenate(seqs) if seqs else np.zeros(0, np.uint32))
        h = ctypes.c_void_p()
        _lib.check(_lib.lib().kyro_ngram_build(
            toks.ctypes.data_as(ctypes.c_void_p) if toks.size else None,
            offsets.ctypes.data_as(ctypes.c_void_p), len(seqs), int(order), ctypes.byref(h)))
        self._h = h
        self.order = int(order)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            _lib.lib().kyro_ngram_destroy(h)
            self._h = None

    def __len__(self) -> int:
        return int(_lib.lib().kyro_ngram_size(self._h))

    def get(self, prefix):
        """The stored next token of an (order-1)-token prefix, or None (the reference's HashMap::get)."""
        p = np.ascontiguousarray(np.asarray(prefix, dtype=np.uint32).reshape(-1))
        if p.size != self.order - 1:
            raise ValueError(f"prefix must have {self.order - 1} tokens")
        nxt = ctypes.c_uint32()
        found = _lib.lib().kyro_ngram_lookup(self._h, p.ctypes.data_as(ctypes.c_void_p), ctypes.byref(nxt))
        return int(nxt.value) if found else None

    def draft(self, context_tail, context_len, max_draft: int, *, out=None):
        """Drafts for a batch on torch's current stream. ``context_tail``: int32/uint32 device
        tensor [B, order-1] of each sequence's last order-1 tokens; ``context_len``: int64 [B].
        Returns (draft_tokens int32 [B, max_draft], num_draft int32 [B])."""
        dev = context_len.device
        B = context_len.shape[0]
        if context_tail.dtype not in (torch.int32,) or tuple(context_tail.shape) != (B, self.order - 1) \
                or not context_tail.is_contiguous():
            raise ValueError(f"context_tail must be a contiguous int32 [{B}, {self.order - 1}] tensor")
        if context_len.dtype != torch.int64:
            raise ValueError("context_len must be int64")
        ctx = _lib.context(dev.index or 0)
        ctx.set_stream(torch.cuda.current_stream(dev).cuda_stream)
        _lib.check(_lib.lib().kyro_ngram_upload(self._h, ctx.handle))
        if out is None:
            out = (torch.empty((B, max_draft), dtype=torch.int32, device=dev),
                   torch.empty((B,), dtype=torch.int32, device=dev))
        toks, nd = out
        _lib.check(_lib.lib().kyro_ngram_draft(self._h, ctx.handle, B, int(max_draft), context_tail.data_ptr(),
                                               context_len.data_ptr(), toks.data_ptr(), nd.data_ptr()))
        return toks, nd


def context_tails(contexts, order: int, device):
    """(context_tail int32 [B, order-1], context_len int64 [B]) device tensors from host token
    lists; entries before the start of a short context are 0."""
    n = order - 1
    tail = np.zeros((len(contexts), n), np.uint32)
    lens = np.zeros(len(contexts), np.int64)
    for b, c in enumerate(contexts):
        c = np.asarray(c, dtype=np.uint32).reshape(-1)
        lens[b] = c.size
        take = c[-n:] if n else c[:0]
        if take.size:
            tail[b, n - take.size:] = take
    return torch.from_numpy(tail.view(np.int32)).to(device), torch.from_numpy(lens).to(device)
