"""Batched draft verification — host mirror of SpeculativeDecoder::verify_drafts.

The reference verifies one sequence at a time with greedy argmax-match
(src/speculative.rs:286-339). ``verify_drafts`` verifies a whole batch in one pass on the GPU:
sampled sequences (temperature > 0) use rejection sampling against the draft distribution,
greedy sequences (temperature <= 0) use the reference's argmax-match and gain the bonus token
after full acceptance. Uniforms are inputs, so results are reproducible.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib


@dataclass
class VerifyResult:
    accepted: torch.Tensor   # int32 [B]: accepted drafts per sequence
    tokens: torch.Tensor     # int32 [B, kmax+1]: accepted drafts, then the correction/bonus token; -1 pads
    p_draft: torch.Tensor | None = None  # float32 [B, kmax]: p_i(x_i) (NaN where not evaluated)
    q_draft: torch.Tensor | None = None  # float32 [B, kmax]: q_i(x_i)

    def emitted(self):
        """Per-sequence emitted token lists (host), as verify_drafts' Vec<u32>."""
        acc = self.accepted.cpu().tolist()
        tok = self.tokens.cpu().tolist()
        return [row[: a + 1] for a, row in zip(acc, tok)]


def _dev_tensor(t, name, dtype, shape, device):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} has dtype {t.dtype}, expected {dtype}")
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
    if t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def verify_drafts_async(target_logits, draft_logits, draft_tokens, num_draft, temperature,
                        u_accept, u_resample, *, return_probs=False, out=None, window=0,
                        allocation_free=False):
    """Queues the verify kernels on torch's current stream; see :func:`verify_drafts`.
    ``window``: draft positions whose logit rows are read before the first acceptance scan
    (0 = the library default); a tuning knob only, outputs do not depend on it.
    ``allocation_free``: call kyro_spec_verify_noalloc (scratch in the library's fixed per-device
    array, no allocation in the call; pass ``out`` and ``return_probs=False`` for a call that
    allocates nothing on the Python side either)."""
    dev = target_logits.device
    if dev.type != "cuda":
        raise ValueError("verify_drafts runs on a GPU device; got " + str(dev))
    if target_logits.dim() != 3:
        raise ValueError("target_logits must be [B, kmax+1, V]")
    B, k1, V = target_logits.shape
    kmax = k1 - 1
    _dev_tensor(target_logits, "target_logits", torch.float32, (B, k1, V), dev)
    if draft_logits is not None:
        _dev_tensor(draft_logits, "draft_logits", torch.float32, (B, kmax, V), dev)
    _dev_tensor(draft_tokens, "draft_tokens", torch.int32, (B, kmax), dev)
    _dev_tensor(num_draft, "num_draft", torch.int32, (B,), dev)
    _dev_tensor(temperature, "temperature", torch.float32, (B,), dev)
    _dev_tensor(u_accept, "u_accept", torch.float32, (B, kmax), dev)
    _dev_tensor(u_resample, "u_resample", torch.float32, (B,), dev)
    if out is None:
        accepted = torch.empty(B, dtype=torch.int32, device=dev)
        tokens = torch.empty((B, k1), dtype=torch.int32, device=dev)
    else:
        accepted, tokens = out
    p = q = None
    if return_probs:
        p = torch.empty((B, kmax), dtype=torch.float32, device=dev)
        q = torch.empty((B, kmax), dtype=torch.float32, device=dev)
    params = _lib.SpecVerifyParams(B, kmax, V, _lib.KYRO_F32, int(window))
    ctx = _lib.context(dev.index or 0)
    ctx.set_stream(torch.cuda.current_stream(dev).cuda_stream)
    ptr = lambda t: t.data_ptr() if t is not None else None  # noqa: E731
    entry = _lib.lib().kyro_spec_verify_noalloc if allocation_free else _lib.lib().kyro_spec_verify
    _lib.check(entry(
        ctx.handle, ctypes.byref(params), ptr(target_logits), ptr(draft_logits), ptr(draft_tokens),
        ptr(num_draft), ptr(temperature), ptr(u_accept), ptr(u_resample), ptr(accepted),
        ptr(tokens), ptr(p), ptr(q)))
    return VerifyResult(accepted, tokens, p, q)


def verify_drafts(target_logits, draft_logits, draft_tokens, num_draft, temperature, u_accept,
                  u_resample, *, return_probs=False, window=0, allocation_free=False):
    """Verifies a batch of drafts (src/speculative.rs:286-339, rejection rule per Leviathan et
    al. 2023) and synchronises.

    target_logits [B, kmax+1, V] f32, draft_logits [B, kmax, V] f32 (None if every sequence is
    greedy), draft_tokens [B, kmax] int32, num_draft [B] int32 (k_b <= kmax), temperature [B] f32
    (<= 0: greedy), u_accept [B, kmax] f32, u_resample [B] f32, uniforms in (0, 1).
    Returns VerifyResult; ``emitted()`` gives verify_drafts' token lists.
    """
    res = verify_drafts_async(target_logits, draft_logits, draft_tokens, num_draft, temperature,
                              u_accept, u_resample, return_probs=return_probs, window=window,
                              allocation_free=allocation_free)
    _lib.context(target_logits.device.index or 0).sync()
    return res


def describe_verify(batch: int, max_draft: int, vocab: int, window: int = 0) -> str:
    """What a verify call with these shapes launches (window, chunking, kernels), from the
    library's own choice (``kyro_spec_verify_describe``). Host only."""
    params = _lib.SpecVerifyParams(int(batch), int(max_draft), int(vocab), _lib.KYRO_F32, int(window))
    return _lib.describe_text(_lib.lib().kyro_spec_verify_describe, ctypes.byref(params))
