"""The C ABI without a GPU: the library loads, exports every function include/kyro_verify.h
declares, and rejects bad arguments with a status code and a message (no crash, no exception)."""
import ctypes
import os
import re

import pytest

from kyro_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", f) for f in sorted(os.listdir(os.path.join(ROOT, "include")))
           if f.endswith(".h")]


def declared_functions():
    names = []
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names += re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\*?\s*(kyro_[a-z0-9_]+)\s*\(",
                            text, flags=re.M)
    return names


def test_header_declares_the_entry_points():
    names = declared_functions()
    for required in ("kyro_paged_attention_mq", "kyro_spec_verify", "kyro_ctx_create",
                     "kyro_last_error", "kyro_buf_alloc"):
        assert required in names


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python binding covers the same set
    assert set(declared_functions()) == set(_lib._SIGNATURES)


def test_abi_version():
    text = open(os.path.join(ROOT, "include", "kyro_verify.h")).read()
    declared = int(re.search(r"#define KYRO_ABI_VERSION (\d+)", text).group(1))
    assert _lib.lib().kyro_abi_version() == declared == _lib.ABI_VERSION


def struct_fields(name):
    """Member names, in order, of `typedef struct name { ... } name;` in the headers."""
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        m = re.search(r"typedef struct " + name + r" \{(.*?)\} " + name + ";", text, flags=re.S)
        if m:
            return re.findall(r"([A-Za-z_][A-Za-z0-9_]*)\s*(?:\[[^]]*\])?\s*;", m.group(1))
    raise AssertionError(f"{name} not declared")


@pytest.mark.parametrize("cname, pyname", [
    ("kyro_paged_attention_params", "PagedAttentionParams"), ("kyro_spec_verify_params", "SpecVerifyParams"),
    ("kyro_kv_append_params", "KvAppendParams"), ("kyro_copy_blocks_params", "CopyBlocksParams"),
    ("kyro_sample_params", "SampleParams"), ("kyro_attention_plan", "AttentionPlan")])
def test_ctypes_structs_mirror_the_headers(cname, pyname):
    assert [f[0] for f in getattr(_lib, pyname)._fields_] == struct_fields(cname)


def test_null_context_is_einval():
    lib = _lib.lib()
    params = _lib.PagedAttentionParams(16, 8, 64, 2, 1, 1, 4, 4, _lib.KYRO_F32, _lib.KYRO_F32, 1, 0.0, 0, 0, 0)
    rc = lib.kyro_paged_attention_mq(None, ctypes.byref(params), None, None, None, None, None, None, None)
    assert rc == _lib.KYRO_EINVAL
    assert "null kyro_ctx" in _lib.last_error()
    sp = _lib.SpecVerifyParams(1, 1, 10, _lib.KYRO_F32)
    rc = lib.kyro_spec_verify(None, ctypes.byref(sp), *([None] * 11))
    assert rc == _lib.KYRO_EINVAL
    assert lib.kyro_sync(None) == _lib.KYRO_EINVAL


def test_buffer_helpers_tolerate_null():
    lib = _lib.lib()
    assert lib.kyro_buf_ptr(None) is None
    assert lib.kyro_buf_size(None) == 0
    assert lib.kyro_buf_free(None) == _lib.KYRO_OK
    assert lib.kyro_ctx_destroy(None) == _lib.KYRO_OK
    out = ctypes.c_void_p()
    assert lib.kyro_buf_alloc(None, 16, ctypes.byref(out)) == _lib.KYRO_EINVAL


def test_bad_device_is_an_error_not_a_crash():
    out = ctypes.c_void_p()
    rc = _lib.lib().kyro_ctx_create(-1, ctypes.byref(out))
    assert rc in (_lib.KYRO_EINVAL, _lib.KYRO_EHIP)
    assert out.value is None
    assert _lib.last_error()


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "absent.so"))
    with pytest.raises(ImportError):
        _lib.lib()


@pytest.mark.parametrize("D, ok", [(8, True), (72, True), (80, True), (96, True), (256, True), (100, False),
                                   (4, False), (264, False)])
def test_head_dim_range(D, ok):
    """The attention entry points take every head dim that is a multiple of 8 up to 256 (the
    reference derives it from the model config, src/model/llama.rs:35) and name the range
    otherwise. Host-only: the workspace query validates the same params as the launch."""
    params = _lib.PagedAttentionParams(16, 8, D, 2, 2, 2, 4, 8, _lib.KYRO_BF16, _lib.KYRO_F32, 1, 0.0, 0, 0, 1)
    nbytes = ctypes.c_size_t()
    rc = _lib.lib().kyro_paged_attention_workspace(None, ctypes.byref(params), 0, ctypes.byref(nbytes))
    if ok:
        assert rc == _lib.KYRO_OK, _lib.last_error()
    else:
        assert rc == _lib.KYRO_EUNSUPPORTED
        assert "multiples of 8 up to 256" in _lib.last_error()
