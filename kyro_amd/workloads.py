"""Seeded synthetic inputs for the verify step (host numpy arrays).

Every random draw comes from numpy's Philox4x64-10 bit generator keyed by (seed, stream) — large
normal tensors by (seed, stream * 2^32 + chunk) per 2^22-value chunk — so each tensor has its own
reproducible stream:

    1 query  2 keys  3 values  4 target logits  5 draft noise  6 u_accept  7 u_resample
    8 draft-token draws  9 context lengths  10 block-table shuffle  11 per-sequence k
    12 greedy mask

N(0, s) means standard deviation s. bf16 tensors are produced by rounding float32 to nearest
even and are carried as uint16 bit patterns. Uniforms lie in the open interval (0, 1).

The standard workload builders below give the shapes the verify step is measured and
tested on; every builder takes a ``batch`` override so tests can run a reduced copy.
"""
from __future__ import annotations

import concurrent.futures
import os
from dataclasses import dataclass, field

import numpy as np

S_Q, S_K, S_V, S_TARGET, S_NOISE, S_UACC, S_URES, S_DRAW, S_CTX, S_TABLE, S_KSEQ, S_GREEDY = range(1, 13)


def rng(seed: int, stream: int) -> np.random.Generator:
    return np.random.Generator(np.random.Philox(key=[int(seed), int(stream)]))


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), round to nearest even."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    bias = ((u >> 16) & 1) + np.uint32(0x7FFF)
    return ((u + bias) >> 16).astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def uniforms(g: np.random.Generator, shape) -> np.ndarray:
    """float32 uniforms in (0, 1) on a 2^-24 grid offset by half a step (never 0 or 1)."""
    n = int(np.prod(shape)) if shape else 1
    x = (g.integers(0, 1 << 24, size=n, dtype=np.int64).astype(np.float64) + 0.5) * 2.0 ** -24
    return x.astype(np.float32).reshape(shape)


_CHUNK = 1 << 22
_POOL = None


def _pool():
    global _POOL
    if _POOL is None:
        _POOL = concurrent.futures.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1))
    return _POOL


def normals(seed: int, stream: int, shape, sigma: float = 1.0, bf16: bool = False) -> np.ndarray:
    """N(0, sigma) of `shape`, float32 (or bf16 bits). Chunk c of 2^22 values comes from the
    Philox key (seed, stream * 2^32 + c), so chunks are generated in parallel and the result does
    not depend on the thread count."""
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.uint16 if bf16 else np.float32)

    def fill(c):
        s, e = c * _CHUNK, min(n, (c + 1) * _CHUNK)
        g = np.random.Generator(np.random.Philox(key=[int(seed), (int(stream) << 32) + c]))
        x = g.standard_normal(e - s, dtype=np.float32)
        if sigma != 1.0:
            x *= np.float32(sigma)
        out[s:e] = f32_to_bf16_bits(x) if bf16 else x

    list(_pool().map(fill, range(-(-n // _CHUNK))))
    return out.reshape(shape)


# --------------------------------------------------------------------------------- attention

@dataclass
class AttentionCase:
    num_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    query: np.ndarray          # [total_q, H, D] float32 or uint16 (bf16 bits)
    key_cache: np.ndarray      # [num_blocks, Hkv, bs, D]
    value_cache: np.ndarray
    block_table: np.ndarray    # [B, max_blocks] int64
    context_lens: np.ndarray   # [B] int64
    q_start_loc: np.ndarray    # [B+1] int32
    dtype: str                 # "bf16" or "f32"
    causal: bool = True
    meta: dict = field(default_factory=dict)

    @property
    def batch(self) -> int:
        return int(self.context_lens.shape[0])

    @property
    def max_q_len(self) -> int:
        return int(np.max(np.diff(self.q_start_loc))) if self.batch else 1

    def kv_bytes(self) -> int:
        """Algorithmic K+V bytes: every context token's K and V row for every kv head, once."""
        esz = 2 if self.dtype == "bf16" else 4
        return int(self.context_lens.sum()) * self.num_kv_heads * self.head_dim * esz * 2

    def unique_kv_bytes(self) -> int:
        """K+V bytes of the distinct blocks the tables reference (prefix sharing counted once)."""
        esz = 2 if self.dtype == "bf16" else 4
        ids = set()
        for b in range(self.batch):
            nb = -(-int(self.context_lens[b]) // self.block_size)
            ids.update(self.block_table[b, :nb].tolist())
        return len(ids) * self.num_kv_heads * self.block_size * self.head_dim * esz * 2

    def q_out_bytes(self, out_esz: int = 2) -> int:
        esz = 2 if self.dtype == "bf16" else 4
        rows = int(self.q_start_loc[-1]) * self.num_heads * self.head_dim
        return rows * esz + rows * out_esz


def make_attention_case(*, context_lens, q_lens, num_heads, num_kv_heads, head_dim=128,
                        block_size=16, dtype="bf16", seed=0, num_blocks=None,
                        shared_prefix_blocks=0, causal=True) -> AttentionCase:
    """Q/K/V ~ N(0, 1); each sequence's table is a consecutive slice of one shuffled pool of
    private blocks, after ``shared_prefix_blocks`` blocks (ids 0..P-1) common to all sequences."""
    ctx = np.asarray(context_lens, dtype=np.int64)
    ql = np.asarray(q_lens, dtype=np.int64)
    B = int(ctx.shape[0])
    nblk = -(-ctx // block_size)
    shared = int(shared_prefix_blocks)
    private = nblk - np.minimum(nblk, shared)
    need = shared + int(private.sum())
    nb_total = max(int(num_blocks or 0), need, 1)
    max_blocks = max(int(nblk.max()) if B else 1, 1)
    perm = rng(seed, S_TABLE).permutation(nb_total - shared) + shared
    table = np.zeros((B, max_blocks), dtype=np.int64)
    pos = 0
    for b in range(B):
        s = min(int(nblk[b]), shared)
        table[b, :s] = np.arange(s)
        p = int(private[b])
        table[b, s:s + p] = perm[pos:pos + p]
        pos += p
    q_start = np.zeros(B + 1, dtype=np.int32)
    q_start[1:] = np.cumsum(ql)
    total_q = int(q_start[-1])
    shape_kv = (nb_total, num_kv_heads, block_size, head_dim)
    bf16 = dtype == "bf16"
    q = normals(seed, S_Q, (total_q, num_heads, head_dim), bf16=bf16)
    k = normals(seed, S_K, shape_kv, bf16=bf16)
    v = normals(seed, S_V, shape_kv, bf16=bf16)
    return AttentionCase(num_heads, num_kv_heads, head_dim, block_size, q, k, v, table, ctx,
                         q_start, dtype, causal)


def mha_llama2_7b(batch=16, seed=0) -> AttentionCase:
    """Llama-2-7B layer: 32/32 heads, D 128, bs 16, ctx ~ U[512, 2048], 5 queries, pool 2048."""
    ctx = rng(seed, S_CTX).integers(512, 2049, size=batch)
    return make_attention_case(context_lens=ctx, q_lens=[5] * batch, num_heads=32,
                               num_kv_heads=32, num_blocks=2048 if batch == 16 else None, seed=seed)


def gqa_llama3_8b(batch=64, ctx=4096, seed=0) -> AttentionCase:
    """Llama-3-8B layer: GQA 32/8, D 128, bs 16, every context 4096, k=7 (8 queries), pool 16384."""
    return make_attention_case(context_lens=[ctx] * batch, q_lens=[8] * batch, num_heads=32,
                               num_kv_heads=8, num_blocks=16384 if batch == 64 and ctx == 4096 else None,
                               seed=seed)


def skewed_prefix(batch=32, seed=0) -> AttentionCase:
    """ctx = round(exp(U[ln 128, ln 32768])), 64 shared prefix blocks, GQA 32/8, 5 queries."""
    u = rng(seed, S_CTX).random(batch)
    ctx = np.round(np.exp(np.log(128) + u * (np.log(32768) - np.log(128)))).astype(np.int64)
    return make_attention_case(context_lens=ctx, q_lens=[5] * batch, num_heads=32, num_kv_heads=8,
                               shared_prefix_blocks=64, seed=seed)


def mixed_llama3_70b(batch=128, seed=0):
    """Llama-3-70B layer: GQA 64/8, ctx ~ U[256, 8192], per-sequence k ~ U{0..8} (k+1 queries).
    Returns (case, k) with k the per-sequence draft lengths."""
    ctx = rng(seed, S_CTX).integers(256, 8193, size=batch)
    k = rng(seed, S_KSEQ).integers(0, 9, size=batch)
    case = make_attention_case(context_lens=ctx, q_lens=k + 1, num_heads=64, num_kv_heads=8, seed=seed)
    return case, k


# ---------------------------------------------------------------------------------- sampling

@dataclass
class VerifyCase:
    target: np.ndarray        # [B, kmax+1, V] float32
    draft: np.ndarray         # [B, kmax, V] float32
    draft_tokens: np.ndarray  # [B, kmax] int32
    num_draft: np.ndarray     # [B] int32
    temperature: np.ndarray   # [B] float32
    u_accept: np.ndarray      # [B, kmax] float32
    u_resample: np.ndarray    # [B] float32

    @property
    def batch(self):
        return int(self.target.shape[0])

    def logit_bytes(self, accepted=None) -> int:
        """Algorithmic logit bytes, each row counted once. Without `accepted`: target rows
        0..k_b of every sequence and draft rows 0..k_b-1 of sampled sequences (greedy sequences
        never read draft logits). With the accepted lengths j_b: only the rows the acceptance
        scan evaluates, target rows 0..j_b and draft rows 0..min(j_b, k_b - 1)."""
        V = self.target.shape[2]
        k = self.num_draft.astype(np.int64)
        sampled = self.temperature > 0
        if accepted is None:
            rows = int((k + 1).sum() + (k * sampled).sum())
        else:
            j = np.asarray(accepted).astype(np.int64)
            rows = int((j + 1).sum() + (np.minimum(j + 1, k) * sampled).sum())
        return rows * V * 4


def _softmax64(x: np.ndarray, T: float) -> np.ndarray:
    y = x.astype(np.float64) / T
    y -= y.max(axis=-1, keepdims=True)
    np.exp(y, out=y)
    y /= y.sum(axis=-1, keepdims=True)
    return y


def make_verify_case(*, batch, kmax, vocab, target_sigma, noise_sigma, temperature,
                     num_draft=None, seed=0) -> VerifyCase:
    """target ~ N(0, target_sigma); draft = target[:, :kmax] + N(0, noise_sigma); draft tokens
    x_i ~ q_i = softmax(draft_i / T) by inverse CDF (argmax q_i for greedy sequences)."""
    B, V = int(batch), int(vocab)
    T = np.broadcast_to(np.asarray(temperature, dtype=np.float32), (B,)).copy()
    k = (np.full(B, kmax, dtype=np.int32) if num_draft is None
         else np.asarray(num_draft, dtype=np.int32).copy())
    target = normals(seed, S_TARGET, (B, kmax + 1, V), target_sigma)
    draft = target[:, :kmax] + normals(seed, S_NOISE, (B, kmax, V), noise_sigma)
    draws = uniforms(rng(seed, S_DRAW), (B, kmax))
    tokens = np.zeros((B, kmax), dtype=np.int32)
    for b in range(B):
        for i in range(int(k[b])):
            if T[b] > 0:
                q = _softmax64(draft[b, i], float(T[b]))
                cdf = np.cumsum(q)
                tokens[b, i] = min(int(np.searchsorted(cdf, draws[b, i] * cdf[-1])), V - 1)
            else:
                tokens[b, i] = int(np.argmax(draft[b, i]))
    return VerifyCase(target, draft.astype(np.float32), tokens, k, T,
                      uniforms(rng(seed, S_UACC), (B, kmax)), uniforms(rng(seed, S_URES), (B,)))


def rejection_only_b8(batch=8, seed=0) -> VerifyCase:
    """Rejection sampling only: B 8, k 4, V 32000, target ~ N(0, 2), noise N(0, 0.5), T 1."""
    return make_verify_case(batch=batch, kmax=4, vocab=32000, target_sigma=2.0, noise_sigma=0.5,
                            temperature=1.0, seed=seed)


def verify_llama3_8b(batch=64, vocab=128256, seed=0) -> VerifyCase:
    """Acceptance for the Llama-3-8B verify step: k 7, V 128256, T 0.8, target ~ N(0, 3), noise N(0, 1)."""
    return make_verify_case(batch=batch, kmax=7, vocab=vocab, target_sigma=3.0, noise_sigma=1.0,
                            temperature=0.8, seed=seed)


def verify_skewed(batch=32, vocab=128256, seed=0) -> VerifyCase:
    """Acceptance for the skewed long-context workload: k 4, V 128256, T 1.0 (target N(0, 3),
    noise N(0, 1), the Llama-3-8B logit model)."""
    return make_verify_case(batch=batch, kmax=4, vocab=vocab, target_sigma=3.0, noise_sigma=1.0,
                            temperature=1.0, seed=seed)


def verify_mixed(k, vocab=128256, seed=0) -> VerifyCase:
    """Acceptance for the mixed batch: per-sequence k (kmax 8); even sequences greedy (T 0),
    odd sequences T 0.7 (target N(0, 3), noise N(0, 1))."""
    k = np.asarray(k, dtype=np.int32)
    B = int(k.shape[0])
    T = np.where(np.arange(B) % 2 == 0, 0.0, 0.7).astype(np.float32)
    return make_verify_case(batch=B, kmax=8, vocab=vocab, target_sigma=3.0, noise_sigma=1.0,
                            temperature=T, num_draft=k, seed=seed)
