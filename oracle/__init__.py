"""CPU oracle for the verify step — TEST INFRASTRUCTURE ONLY.

This package is the checker: the tests, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` load it to compute expected results and to time the CPU path. The product library
(``kyro_amd``) never imports it.

The arithmetic lives in ``kyro_oracle.c`` (see its header for the reference lines each function
restates and for how each is pinned). This module only marshals numpy arrays through ctypes.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SRC = os.path.join(_HERE, "kyro_oracle.c")
# KYRO_ORACLE_LIB / KYRO_ORACLE_F32_LIB name other builds of the same source (the tests' sanitizer
# run loads an AddressSanitizer/UBSan build this way).
LIB_F64 = os.environ.get("KYRO_ORACLE_LIB") or os.path.join(_HERE, "libkyro_oracle.so")
LIB_F32 = os.environ.get("KYRO_ORACLE_F32_LIB") or os.path.join(_HERE, "libkyro_oracle_f32.so")


def build(force: bool = True) -> None:
    """Compiles the oracle twice: f64 accumulation (checker) and f32 (CPU baseline)."""
    for out, extra in ((LIB_F64, []), (LIB_F32, ["-DORACLE_F32"])):
        if not force and os.path.exists(out) and os.path.getmtime(out) >= os.path.getmtime(_SRC):
            continue
        cmd = ["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-Wall", "-Wextra", *extra,
               "-o", out + ".tmp", _SRC, "-lm", "-lpthread"]
        subprocess.run(cmd, check=True)
        os.replace(out + ".tmp", out)


class _AttnArgs(ctypes.Structure):
    _fields_ = [
        ("block_size", ctypes.c_int32), ("num_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32), ("num_kv_heads", ctypes.c_int32),
        ("batch_size", ctypes.c_int32), ("total_q", ctypes.c_int32),
        ("max_blocks_per_seq", ctypes.c_int32), ("num_blocks", ctypes.c_int32),
        ("dtype", ctypes.c_int32), ("causal", ctypes.c_int32),
        ("scale", ctypes.c_double),
        ("query", ctypes.c_void_p), ("q_start_loc", ctypes.c_void_p),
        ("key_cache", ctypes.c_void_p), ("value_cache", ctypes.c_void_p),
        ("block_table", ctypes.c_void_p), ("context_lens", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
    ]


_libs: dict = {}


def _lib(precision: str = "f64"):
    path = LIB_F64 if precision == "f64" else LIB_F32
    if path not in _libs:
        if not os.path.exists(path):
            build(force=False)
        lib = ctypes.CDLL(path)
        lib.oracle_paged_attention_mq.argtypes = [ctypes.POINTER(_AttnArgs), ctypes.c_int]
        lib.oracle_paged_attention_mq.restype = ctypes.c_int
        p = ctypes.c_void_p
        lib.oracle_spec_verify.argtypes = [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32] + [p] * 13
        lib.oracle_spec_verify.restype = ctypes.c_int
        lib.oracle_sample_token.argtypes = [p, ctypes.c_int32, ctypes.c_float, ctypes.c_float,
                                            ctypes.c_int32, ctypes.c_double]
        lib.oracle_sample_token.restype = ctypes.c_int
        lib.oracle_sample_decode.argtypes = [ctypes.c_int32, ctypes.c_int32] + [p] * 15
        lib.oracle_sample_decode.restype = ctypes.c_int
        lib.oracle_kv_append.argtypes = [ctypes.c_int32] * 9 + [p] * 7
        lib.oracle_kv_append.restype = ctypes.c_int
        _libs[path] = lib
    return _libs[path]


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def paged_attention_mq(query, key_cache, value_cache, block_table, context_lens, *,
                       num_heads, num_kv_heads, head_dim, block_size, q_start_loc=None,
                       causal=True, scale=0.0, threads=1, precision="f64"):
    """Oracle multi-query paged attention. ``query``/caches are float32 arrays or uint16 arrays
    holding bf16 bits. Returns float64 [total_q, H, D]."""
    is_bf16 = query.dtype == np.uint16
    query = np.ascontiguousarray(query)
    key_cache = np.ascontiguousarray(key_cache)
    value_cache = np.ascontiguousarray(value_cache)
    block_table = np.ascontiguousarray(block_table, dtype=np.int64)
    context_lens = np.ascontiguousarray(context_lens, dtype=np.int64)
    B = int(context_lens.shape[0])
    total_q = int(query.shape[0])
    if q_start_loc is not None:
        q_start_loc = np.ascontiguousarray(q_start_loc, dtype=np.int32)
    out = np.zeros((total_q, num_heads, head_dim), dtype=np.float64)
    args = _AttnArgs(block_size, num_heads, head_dim, num_kv_heads, B, total_q,
                     int(block_table.shape[1]) if block_table.ndim == 2 else 0,
                     int(key_cache.shape[0]), 1 if is_bf16 else 0, 1 if causal else 0, float(scale),
                     _ptr(query), _ptr(q_start_loc), _ptr(key_cache), _ptr(value_cache),
                     _ptr(block_table), _ptr(context_lens), _ptr(out))
    rc = _lib(precision).oracle_paged_attention_mq(ctypes.byref(args), int(threads))
    if rc != 0:
        raise ValueError("oracle_paged_attention_mq: invalid arguments (status %d)" % rc)
    return out


def spec_verify(target_logits, draft_logits, draft_tokens, num_draft, temperature, u_accept,
                u_resample, precision="f64"):
    """Oracle verify step. Returns a dict with accepted [B], tokens [B, kmax+1] (uint32),
    p_draft/q_draft [B, kmax], accept_margin [B, kmax], resample_margin [B]."""
    target_logits = np.ascontiguousarray(target_logits, dtype=np.float32)
    B, k1, V = target_logits.shape
    kmax = k1 - 1
    if draft_logits is not None:
        draft_logits = np.ascontiguousarray(draft_logits, dtype=np.float32)
    draft_tokens = np.ascontiguousarray(draft_tokens, dtype=np.uint32).reshape(B, kmax)
    num_draft = np.ascontiguousarray(num_draft, dtype=np.int32)
    temperature = np.ascontiguousarray(temperature, dtype=np.float32)
    u_accept = np.ascontiguousarray(u_accept, dtype=np.float32).reshape(B, kmax)
    u_resample = np.ascontiguousarray(u_resample, dtype=np.float32)
    accepted = np.zeros(B, dtype=np.int32)
    tokens = np.zeros((B, kmax + 1), dtype=np.uint32)
    p = np.zeros((B, kmax), dtype=np.float64)
    q = np.zeros((B, kmax), dtype=np.float64)
    am = np.zeros((B, kmax), dtype=np.float64)
    rm = np.zeros(B, dtype=np.float64)
    rc = _lib(precision).oracle_spec_verify(
        B, kmax, V, _ptr(target_logits), _ptr(draft_logits), _ptr(draft_tokens), _ptr(num_draft),
        _ptr(temperature), _ptr(u_accept), _ptr(u_resample), _ptr(accepted), _ptr(tokens),
        _ptr(p), _ptr(q), _ptr(am), _ptr(rm))
    if rc != 0:
        raise ValueError("oracle_spec_verify: invalid arguments (status %d)" % rc)
    return {"accepted": accepted, "tokens": tokens, "p_draft": p, "q_draft": q,
            "accept_margin": am, "resample_margin": rm}


def sample_token(logits, temperature, top_p=1.0, top_k=None, u=0.5, precision="f64"):
    """Oracle of sample_token (src/worker.rs:267-362) with the uniform passed in."""
    logits = np.ascontiguousarray(np.asarray(logits, dtype=np.float32).reshape(-1))
    return int(_lib(precision).oracle_sample_token(
        _ptr(logits), int(logits.shape[0]), float(temperature), float(top_p),
        int(top_k) if top_k else 0, float(u)))


def kv_append(key, value, key_cache, value_cache, block_table, context_lens, *, block_size,
              q_start_loc=None):
    """Oracle paged KV append (src/model/kv_cache.rs:49-75 for a block-table cache). ``key`` /
    ``value`` are [total_q, Hkv, D] float32 or uint16 (bf16 bits); the caches (float32 or uint16)
    are updated in place. Returns 0, or 1 if some sequence was rejected (its rows not written)."""
    key = np.ascontiguousarray(key)
    value = np.ascontiguousarray(value)
    assert key_cache.flags.c_contiguous and value_cache.flags.c_contiguous
    block_table = np.ascontiguousarray(block_table, dtype=np.int64)
    context_lens = np.ascontiguousarray(context_lens, dtype=np.int64)
    if q_start_loc is not None:
        q_start_loc = np.ascontiguousarray(q_start_loc, dtype=np.int32)
    B = int(context_lens.shape[0])
    total_q, Hkv, D = key.shape
    return int(_lib().oracle_kv_append(
        B, Hkv, D, block_size, int(block_table.shape[1]), int(key_cache.shape[0]), total_q,
        1 if key.dtype == np.uint16 else 0, 1 if key_cache.dtype == np.uint16 else 0,
        _ptr(key), _ptr(value), _ptr(q_start_loc), _ptr(block_table), _ptr(context_lens),
        _ptr(key_cache), _ptr(value_cache)))


def _csr(rows, B):
    """Per-row {token: value} dicts (or None) -> (offsets int32 [B+1], tokens uint32, values f32)."""
    if rows is None:
        return None, None, None
    off = np.zeros(B + 1, np.int32)
    toks, vals = [], []
    for b in range(B):
        d = rows[b] or {}
        for t in sorted(d):
            toks.append(t)
            vals.append(d[t])
        off[b + 1] = len(toks)
    return (off, np.asarray(toks, np.uint32).reshape(-1), np.asarray(vals, np.float32).reshape(-1))


def sample_decode(logits, temperature, u, *, top_p=None, top_k=None, bias=None, penalty=None,
                  masks=None, mask_row=None, precision="f64"):
    """Oracle of the worker's decode step (src/worker.rs:141-197 then sample_token :267-362) for a
    batch. ``bias`` / ``penalty``: per-row {token: value} dicts (or None); ``masks``: uint32
    [num_masks, ceil(V/32)] allowed-token bits, ``mask_row`` int32 [B] (-1: no mask).
    Returns (tokens uint32 [B], margins float64 [B])."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    B, V = logits.shape
    t = np.ascontiguousarray(temperature, dtype=np.float32).reshape(B)
    uu = np.ascontiguousarray(u, dtype=np.float32).reshape(B)
    tp = None if top_p is None else np.ascontiguousarray(top_p, dtype=np.float32).reshape(B)
    tk = None if top_k is None else np.ascontiguousarray(top_k, dtype=np.int32).reshape(B)
    bo, bt, bv = _csr(bias, B)
    po, pt, pv = _csr(penalty, B)
    mk = None if masks is None else np.ascontiguousarray(masks, dtype=np.uint32)
    mr = None if mask_row is None else np.ascontiguousarray(mask_row, dtype=np.int32).reshape(B)
    out = np.zeros(B, np.uint32)
    mg = np.zeros(B, np.float64)
    rc = _lib(precision).oracle_sample_decode(
        B, V, _ptr(logits), _ptr(t), _ptr(tp), _ptr(tk), _ptr(uu), _ptr(bo), _ptr(bt), _ptr(bv),
        _ptr(po), _ptr(pt), _ptr(pv), _ptr(mk), _ptr(mr), _ptr(out), _ptr(mg))
    if rc != 0:
        raise ValueError("oracle_sample_decode: a bias or penalty token is out of range")
    return out, mg


def ngram_build(corpus, order):
    """build_ngram_table (src/speculative.rs:196-208): {prefix tuple: next}, later windows win."""
    table = {}
    for seq in corpus:
        seq = [int(t) for t in seq]
        if len(seq) < order:
            continue
        for i in range(len(seq) - order + 1):
            table[tuple(seq[i:i + order - 1])] = seq[i + order - 1]
    return table


def ngram_draft(table, context, order, lookahead):
    """generate_drafts' Ngram arm (src/speculative.rs:239-256) for one context."""
    ctx = [int(t) for t in context]
    drafts = []
    for _ in range(lookahead):
        if len(ctx) < order:
            break
        nxt = table.get(tuple(ctx[len(ctx) - (order - 1):]))
        if nxt is None:
            break
        drafts.append(nxt)
        ctx.append(nxt)
    return drafts
