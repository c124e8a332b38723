"""Plain-decode sampling with logit processors — host mirror of the worker's decode step.

Mirrors the tail of Worker::run_loop (src/worker.rs:141-197: logit bias, frequency / presence
penalty, grammar mask) and ``sample_token`` (src/worker.rs:267-362) for a batch of rows, over
``kyro_sample_tokens`` (include/kyro_sample.h). Uniforms are inputs (the reference draws them
from an unseeded ``rand::rng()``), so results are reproducible.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib

# GrammarConstraint::Json's valid tokens (src/api/grammar.rs:52-55).
JSON_TOKENS = (0, 10, 32, 34, 91, 93, 123, 125)


def penalty_adds(generated_tokens, frequency_penalty: float, presence_penalty: float,
                 vocab_size: int) -> dict[int, float]:
    """The additive penalty entries of one request (worker.rs:154-181), computed by the library
    in the reference's f32 operations: {token: value} for every generated token below vocab_size
    (empty when both penalties are 0)."""
    g = np.ascontiguousarray(np.asarray(generated_tokens, dtype=np.uint32).reshape(-1))
    n = ctypes.c_int64()
    lib = _lib.lib()
    ptr = g.ctypes.data_as(ctypes.c_void_p) if g.size else None
    _lib.check(lib.kyro_penalty_adds(ptr, g.size, float(frequency_penalty), float(presence_penalty),
                                     int(vocab_size), None, None, 0, ctypes.byref(n)))
    toks = np.zeros(max(1, n.value), np.uint32)
    vals = np.zeros(max(1, n.value), np.float32)
    _lib.check(lib.kyro_penalty_adds(ptr, g.size, float(frequency_penalty), float(presence_penalty),
                                     int(vocab_size), toks.ctypes.data_as(ctypes.c_void_p),
                                     vals.ctypes.data_as(ctypes.c_void_p), n.value, ctypes.byref(n)))
    return {int(t): float(v) for t, v in zip(toks[: n.value], vals[: n.value])}


def grammar_mask(valid_tokens, vocab_size: int) -> np.ndarray:
    """Allowed-token bits for one constraint (GrammarLogitsProcessor::get_valid_tokens,
    grammar.rs:50-59): uint32 [ceil(V/32)], bit v % 32 of word v / 32. ``valid_tokens`` None
    allows everything (GrammarConstraint::None and ::Regex)."""
    words = np.zeros((vocab_size + 31) // 32, np.uint32)
    if valid_tokens is None:
        words[:] = 0xFFFFFFFF
        if vocab_size % 32:
            words[-1] = (1 << (vocab_size % 32)) - 1
        return words
    for t in valid_tokens:
        if 0 <= t < vocab_size:
            words[t >> 5] |= np.uint32(1 << (t & 31))
    return words


def _csr(rows, B, dev):
    if rows is None:
        return None, None, None
    off = np.zeros(B + 1, np.int32)
    toks, vals = [], []
    for b in range(B):
        d = rows[b] or {}
        for t in sorted(d):
            toks.append(int(t))
            vals.append(float(d[t]))
        off[b + 1] = len(toks)
    if not toks:
        return None, None, None
    return (torch.from_numpy(off).to(dev), torch.tensor(np.asarray(toks, np.uint32).view(np.int32), device=dev),
            torch.tensor(vals, dtype=torch.float32, device=dev))


class Processors:
    """Device tensors of the logit processors for a batch (built once, reused across steps)."""

    def __init__(self, B, V, device, *, bias=None, penalty=None, masks=None, mask_row=None):
        self.B, self.V = int(B), int(V)
        self.bias = _csr(bias, self.B, device)
        self.penalty = _csr(penalty, self.B, device)
        self.masks = self.mask_row = None
        self.num_masks = 0
        if masks is not None:
            words = np.ascontiguousarray(np.asarray(masks, np.uint32).reshape(-1, (self.V + 31) // 32))
            self.masks = torch.from_numpy(words.view(np.int32)).to(device)
            self.num_masks = words.shape[0]
            mr = np.zeros(self.B, np.int32) if mask_row is None else np.asarray(mask_row, np.int32).reshape(-1)
            if mr.size != self.B:
                raise ValueError(f"mask_row must have {self.B} entries")
            self.mask_row = torch.from_numpy(np.ascontiguousarray(mr)).to(device)


def sample_tokens_async(logits, temperature, u, *, top_p=None, top_k=None, bias=None, penalty=None,
                        masks=None, mask_row=None, processors=None, out=None):
    """Queues the decode sampler on torch's current stream; see :func:`sample_tokens`.
    ``processors`` (a :class:`Processors`) replaces bias / penalty / masks / mask_row."""
    dev = logits.device
    if dev.type != "cuda":
        raise ValueError("sample_tokens runs on a GPU device; got " + str(dev))
    if logits.dtype != torch.float32 or logits.dim() != 2 or not logits.is_contiguous():
        raise ValueError("logits must be a contiguous float32 [B, V] tensor")
    B, V = logits.shape
    if processors is None:
        processors = Processors(B, V, dev, bias=bias, penalty=penalty, masks=masks, mask_row=mask_row)
    elif (processors.B, processors.V) != (B, V):
        raise ValueError("processors were built for another batch shape")

    def vec(x, name, dtype):
        if x is None:
            return None
        t = x if isinstance(x, torch.Tensor) else torch.as_tensor(np.asarray(x))
        t = t.to(device=dev, dtype=dtype).reshape(-1).contiguous()
        if t.numel() != B:
            raise ValueError(f"{name} must have {B} entries")
        return t

    temperature = vec(temperature, "temperature", torch.float32)
    u = vec(u, "u", torch.float32)
    top_p = vec(top_p, "top_p", torch.float32)
    top_k = vec(top_k, "top_k", torch.int32)
    bo, bt, bv = processors.bias
    po, pt, pv = processors.penalty
    mk, mr, num_masks = processors.masks, processors.mask_row, processors.num_masks
    if out is None:
        out = torch.empty(B, dtype=torch.int32, device=dev)
    params = _lib.SampleParams(B, V, _lib.KYRO_F32, num_masks)
    ctx = _lib.context(dev.index or 0)
    ctx.set_stream(torch.cuda.current_stream(dev).cuda_stream)
    ptr = lambda t: t.data_ptr() if t is not None else None  # noqa: E731
    _lib.check(_lib.lib().kyro_sample_tokens(
        ctx.handle, ctypes.byref(params), ptr(logits), ptr(temperature), ptr(top_p), ptr(top_k), ptr(u),
        ptr(bo), ptr(bt), ptr(bv), ptr(po), ptr(pt), ptr(pv), ptr(mk), ptr(mr), ptr(out)))
    return out


def sample_tokens(logits, temperature, u, *, top_p=None, top_k=None, bias=None, penalty=None,
                  masks=None, mask_row=None):
    """One token per row of ``logits`` [B, V] (float32, device), as the worker's decode step.

    ``temperature``, ``u`` (uniforms in [0, 1)), ``top_p`` (None: 1.0) and ``top_k`` (None or
    <= 0: off) have one entry per row. ``bias`` / ``penalty``: per-row {token: value} dicts (or
    None), e.g. a request's logit_bias and :func:`penalty_adds`. ``masks``: allowed-token bit rows
    (:func:`grammar_mask`) and ``mask_row`` the mask index per row (-1: none). Synchronises, so a
    token id out of range raises KyroError here. Returns int32 [B] token ids."""
    out = sample_tokens_async(logits, temperature, u, top_p=top_p, top_k=top_k, bias=bias, penalty=penalty,
                              masks=masks, mask_row=mask_row)
    _lib.context(logits.device.index or 0).sync()
    return out


def sample_token(logits, temperature: float, top_p: float, top_k, u: float) -> int:
    """sample_token (worker.rs:267-272) for one row on the GPU, with the uniform passed in."""
    row = logits.reshape(1, -1).to(torch.float32).contiguous()
    return int(sample_tokens(row, [temperature], [u], top_p=[top_p], top_k=[top_k or 0])[0].item())
