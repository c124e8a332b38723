"""ctypes binding of libkyro_verify.so (the C ABI declared in include/kyro_verify.h).

The library is the only compute path: if it is missing this module raises on first use, and
nothing falls back to a CPU or PyTorch implementation.
"""
from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
# KYRO_VERIFY_LIB names another build of the same library (the tests' host sanitizer run).
LIB_PATH = os.environ.get("KYRO_VERIFY_LIB") or os.path.join(_HERE, "libkyro_verify.so")

KYRO_OK, KYRO_EINVAL, KYRO_EOOM, KYRO_EHIP, KYRO_EUNSUPPORTED, KYRO_ENOSPACE = 0, 1, 2, 3, 4, 5
KYRO_F32, KYRO_BF16 = 0, 1
KYRO_ATTN_AUTO, KYRO_ATTN_VECTOR, KYRO_ATTN_MFMA = 0, 1, 2
KYRO_KV_REUSE_AUTO, KYRO_KV_REUSE_SHARED, KYRO_KV_REUSE_STREAM = 0, 1, 2
KYRO_ATTN_SCHEDULE_AUTO, KYRO_ATTN_SCHEDULE_GRID, KYRO_ATTN_SCHEDULE_BALANCED = 0, 1, 2

SPEC_VERIFY_NOALLOC_SCRATCH_BYTES = 16 << 20  # KYRO_SPEC_VERIFY_NOALLOC_SCRATCH_BYTES

_STATUS_NAMES = {0: "KYRO_OK", 1: "KYRO_EINVAL", 2: "KYRO_EOOM", 3: "KYRO_EHIP", 4: "KYRO_EUNSUPPORTED",
                 5: "KYRO_ENOSPACE"}


class KyroError(RuntimeError):
    """A non-zero kyro_status, with the library's kyro_last_error() text."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{_STATUS_NAMES.get(status, status)}: {message}")
        self.status = status


class PagedAttentionParams(ctypes.Structure):
    _fields_ = [
        ("block_size", ctypes.c_int32), ("num_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32), ("num_kv_heads", ctypes.c_int32),
        ("batch_size", ctypes.c_int32), ("total_q", ctypes.c_int32),
        ("max_blocks_per_seq", ctypes.c_int32), ("num_blocks", ctypes.c_int32),
        ("dtype", ctypes.c_int32), ("out_dtype", ctypes.c_int32),
        ("causal", ctypes.c_int32), ("scale", ctypes.c_float),
        ("path", ctypes.c_int32), ("num_splits", ctypes.c_int32),
        ("max_q_len", ctypes.c_int32), ("kv_reuse", ctypes.c_int32),
        ("schedule", ctypes.c_int32),
    ]


class SpecVerifyParams(ctypes.Structure):
    _fields_ = [
        ("batch_size", ctypes.c_int32), ("max_draft", ctypes.c_int32),
        ("vocab_size", ctypes.c_int32), ("logits_dtype", ctypes.c_int32),
        ("window", ctypes.c_int32),
    ]


class AttentionPlan(ctypes.Structure):
    _fields_ = [("grid", ctypes.c_int32), ("chunk_blocks", ctypes.c_int32), ("items", ctypes.c_int64),
                ("slot_bound", ctypes.c_int64)]


class KvAppendParams(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "block_size", "num_kv_heads", "head_dim", "batch_size", "total_q", "max_blocks_per_seq",
        "num_blocks", "src_dtype", "cache_dtype", "max_q_len")]


class CopyBlocksParams(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("block_size", "num_kv_heads", "head_dim", "num_blocks", "dtype")]


class SampleParams(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("batch_size", "vocab_size", "logits_dtype", "num_masks")]


ABI_VERSION = 9  # KYRO_ABI_VERSION of include/kyro_verify.h

_lib = None
_lib_lock = threading.Lock()

_P = ctypes.c_void_p
_SIGNATURES = {
    "kyro_last_error": ([], ctypes.c_char_p),
    "kyro_abi_version": ([], ctypes.c_int),
    "kyro_ctx_create": ([ctypes.c_int, ctypes.POINTER(_P)], ctypes.c_int),
    "kyro_ctx_destroy": ([_P], ctypes.c_int),
    "kyro_ctx_set_stream": ([_P, _P], ctypes.c_int),
    "kyro_ctx_reserve": ([_P, ctypes.c_size_t], ctypes.c_int),
    "kyro_sync": ([_P], ctypes.c_int),
    "kyro_check": ([_P], ctypes.c_int),
    "kyro_buf_alloc": ([_P, ctypes.c_size_t, ctypes.POINTER(_P)], ctypes.c_int),
    "kyro_buf_free": ([_P], ctypes.c_int),
    "kyro_buf_ptr": ([_P], _P),
    "kyro_buf_size": ([_P], ctypes.c_size_t),
    "kyro_buf_upload": ([_P, _P, ctypes.c_size_t, _P, ctypes.c_size_t], ctypes.c_int),
    "kyro_buf_download": ([_P, _P, _P, ctypes.c_size_t, ctypes.c_size_t], ctypes.c_int),
    "kyro_paged_attention_mq": ([_P, ctypes.POINTER(PagedAttentionParams)] + [_P] * 7, ctypes.c_int),
    "kyro_paged_attention_workspace": ([_P, ctypes.POINTER(PagedAttentionParams), ctypes.c_int,
                                        ctypes.POINTER(ctypes.c_size_t)], ctypes.c_int),
    "kyro_paged_attention_plan": ([ctypes.POINTER(PagedAttentionParams), ctypes.c_int, ctypes.c_int, _P, _P, _P,
                                   ctypes.POINTER(AttentionPlan)], ctypes.c_int),
    "kyro_spec_verify": ([_P, ctypes.POINTER(SpecVerifyParams)] + [_P] * 11, ctypes.c_int),
    "kyro_spec_verify_noalloc": ([_P, ctypes.POINTER(SpecVerifyParams)] + [_P] * 11, ctypes.c_int),
    "kyro_spec_verify_workspace": ([ctypes.POINTER(SpecVerifyParams), ctypes.POINTER(ctypes.c_size_t)], ctypes.c_int),
    "kyro_spec_verify_describe": ([ctypes.POINTER(SpecVerifyParams), ctypes.c_char_p, ctypes.c_size_t,
                                   ctypes.POINTER(ctypes.c_size_t)], ctypes.c_int),
    "kyro_paged_attention_describe": ([_P, ctypes.POINTER(PagedAttentionParams), ctypes.c_int, ctypes.c_char_p,
                                       ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t)], ctypes.c_int),
    "kyro_paged_kv_append": ([_P, ctypes.POINTER(KvAppendParams)] + [_P] * 7, ctypes.c_int),
    # include/kyro_blocks.h
    "kyro_radix_create": ([ctypes.c_int32, ctypes.c_int64, ctypes.POINTER(_P)], ctypes.c_int),
    "kyro_radix_destroy": ([_P], ctypes.c_int),
    "kyro_radix_match_prefix": ([_P, _P, ctypes.c_int64, _P, ctypes.c_int64, _P, _P], ctypes.c_int),
    "kyro_radix_insert": ([_P, _P, ctypes.c_int64, _P, _P], ctypes.c_int),
    "kyro_radix_evict_lru": ([_P, _P, ctypes.c_int64, _P], ctypes.c_int),
    "kyro_radix_num_cached_blocks": ([_P], ctypes.c_int64),
    "kyro_bm_create": ([ctypes.c_int32, ctypes.c_int64, ctypes.c_int64, ctypes.POINTER(_P)], ctypes.c_int),
    "kyro_bm_destroy": ([_P], ctypes.c_int),
    "kyro_bm_allocate_with_prefix": ([_P, ctypes.c_uint64, _P, ctypes.c_int64, _P], ctypes.c_int),
    "kyro_bm_allocate": ([_P, ctypes.c_uint64, ctypes.c_int64], ctypes.c_int),
    "kyro_bm_append_slots": ([_P, ctypes.c_uint64, ctypes.c_int64], ctypes.c_int),
    "kyro_bm_truncate": ([_P, ctypes.c_uint64, ctypes.c_int64], ctypes.c_int),
    "kyro_bm_free": ([_P, ctypes.c_uint64, ctypes.c_int32], ctypes.c_int),
    "kyro_bm_request_blocks": ([_P, ctypes.c_uint64, _P, ctypes.c_int64, _P, _P], ctypes.c_int),
    "kyro_bm_take_copies": ([_P, _P, _P, ctypes.c_int64, _P], ctypes.c_int),
    "kyro_bm_num_free_blocks": ([_P], ctypes.c_int64),
    "kyro_bm_check": ([_P], ctypes.c_int),
    "kyro_bm_num_cached_blocks": ([_P], ctypes.c_int64),
    "kyro_bm_match_prefix": ([_P, _P, ctypes.c_int64, _P, ctypes.c_int64, _P, _P], ctypes.c_int),
    "kyro_bm_write_tables": ([_P, _P, _P, ctypes.c_int32, ctypes.c_int32, _P, _P, _P], ctypes.c_int),
    "kyro_copy_blocks": ([_P, ctypes.POINTER(CopyBlocksParams), _P, _P, _P, _P, ctypes.c_int64], ctypes.c_int),
    # include/kyro_sample.h
    "kyro_sample_tokens": ([_P, ctypes.POINTER(SampleParams)] + [_P] * 14, ctypes.c_int),
    "kyro_penalty_adds": ([_P, ctypes.c_int64, ctypes.c_float, ctypes.c_float, ctypes.c_int32, _P, _P,
                           ctypes.c_int64, _P], ctypes.c_int),
    # include/kyro_draft.h
    "kyro_ngram_build": ([_P, _P, ctypes.c_int64, ctypes.c_int32, ctypes.POINTER(_P)], ctypes.c_int),
    "kyro_ngram_destroy": ([_P], ctypes.c_int),
    "kyro_ngram_lookup": ([_P, _P, _P], ctypes.c_int),
    "kyro_ngram_size": ([_P], ctypes.c_int64),
    "kyro_ngram_upload": ([_P, _P], ctypes.c_int),
    "kyro_ngram_draft": ([_P, _P, ctypes.c_int32, ctypes.c_int32, _P, _P, _P, _P], ctypes.c_int),
    # include/kyro_testing.h
    "kyro_testing_set_plan_slot_cap": ([ctypes.c_int64], ctypes.c_int64),
}


def lib() -> ctypes.CDLL:
    """Loads libkyro_verify.so once. Raises ImportError if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lib_lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise ImportError(
                    f"{LIB_PATH} is missing: build it with `python -m kyro_amd.build` "
                    "(there is no fallback implementation)")
            handle = ctypes.CDLL(LIB_PATH)
            for name, (argtypes, restype) in _SIGNATURES.items():
                fn = getattr(handle, name)
                fn.argtypes = argtypes
                fn.restype = restype
            if handle.kyro_abi_version() != ABI_VERSION:
                raise ImportError(f"{LIB_PATH} has ABI version {handle.kyro_abi_version()}, this "
                                  f"binding needs {ABI_VERSION}: rebuild with `python -m kyro_amd.build`")
            _lib = handle
    return _lib


def last_error() -> str:
    return lib().kyro_last_error().decode("utf-8", "replace")


def check(status: int) -> None:
    if status != KYRO_OK:
        raise KyroError(status, last_error())


class Context:
    """One kyro_ctx: a device, a stream binding and the library's scratch arena."""

    def __init__(self, device: int = 0):
        handle = _P()
        check(lib().kyro_ctx_create(int(device), ctypes.byref(handle)))
        self.handle = handle
        self.device = int(device)
        self._stream = None  # None: the context's own stream

    def set_stream(self, stream_ptr: int) -> None:
        """Binds the context to a hipStream_t handle (0 = HIP's null stream)."""
        if stream_ptr != self._stream:
            check(lib().kyro_ctx_set_stream(self.handle, _P(stream_ptr) if stream_ptr else None))
            self._stream = stream_ptr

    def sync(self) -> None:
        check(lib().kyro_sync(self.handle))

    def reserve(self, nbytes: int) -> None:
        check(lib().kyro_ctx_reserve(self.handle, int(nbytes)))

    def close(self) -> None:
        if getattr(self, "handle", None):
            lib().kyro_ctx_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


_contexts: dict = {}


def context(device: int = 0) -> Context:
    """Process-wide context for a device, created on first use."""
    ctx = _contexts.get(device)
    if ctx is None:
        ctx = _contexts[device] = Context(device)
    return ctx


def describe_text(fn, *args) -> str:
    """Calls a kyro_*_describe query (its trailing buf, len, needed arguments supplied here) and
    returns the text."""
    needed = ctypes.c_size_t()
    check(fn(*args, None, 0, ctypes.byref(needed)))
    buf = ctypes.create_string_buffer(needed.value)
    check(fn(*args, buf, needed.value, None))
    return buf.value.decode()
