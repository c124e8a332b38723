"""kyro_spec_verify_noalloc: the allocation-free verify entry point, through the C ABI.

It runs kyro_spec_verify's kernels with their scratch in the library's fixed per-device array.
Its results must equal kyro_spec_verify's bit for bit (and therefore the oracle's, to the verify
bar) on consecutive calls whose sizes differ, whatever the array holds from the last call.
"""
import ctypes

import numpy as np
import pytest
import torch

import kyro_amd
from kyro_amd import _lib
from kyro_amd import workloads as wl
from tests import helpers as h

pytestmark = pytest.mark.gpu


def _bitwise_equal(a, b):
    return torch.equal(a.view(torch.int32), b.view(torch.int32))


def test_noalloc_equals_spec_verify_on_two_calls(gpu):
    """Llama-3-8B verify shape (B 64, k 7, V 128256), then a smaller batch (B 12, k 3, V 5000),
    back to back on the allocation-free entry point; then the same two on kyro_spec_verify."""
    big = wl.verify_llama3_8b()
    small = wl.make_verify_case(batch=12, kmax=3, vocab=5000, target_sigma=2.0, noise_sigma=1.0,
                                temperature=0.9, num_draft=np.arange(12) % 4, seed=9)
    tb, ts = h.verify_tensors(big, gpu), h.verify_tensors(small, gpu)
    got = [kyro_amd.verify_drafts(**tb, return_probs=True, allocation_free=True),
           kyro_amd.verify_drafts(**ts, return_probs=True, allocation_free=True)]
    ref = [kyro_amd.verify_drafts(**tb, return_probs=True), kyro_amd.verify_drafts(**ts, return_probs=True)]
    for case, g, r in zip((big, small), got, ref):
        assert torch.equal(g.accepted, r.accepted) and torch.equal(g.tokens, r.tokens)
        assert _bitwise_equal(g.p_draft, r.p_draft) and _bitwise_equal(g.q_draft, r.q_draft)
        h.assert_verify_parity(g, case, h.oracle_verify(case), max_exempt=1)


def test_noalloc_refuses_a_call_beyond_its_scratch(gpu):
    """B 4096, k 8, V 128256 needs 17.8 MB of scratch, more than the 16 MiB array: the host
    refuses the call before any launch, and the entry point keeps working afterwards."""
    params = _lib.SpecVerifyParams(4096, 8, 128256, _lib.KYRO_F32, 0)
    need = ctypes.c_size_t()
    _lib.check(_lib.lib().kyro_spec_verify_workspace(ctypes.byref(params), ctypes.byref(need)))
    assert need.value > _lib.SPEC_VERIFY_NOALLOC_SCRATCH_BYTES
    dummy = torch.zeros(16, dtype=torch.float32, device=gpu)
    ctx = _lib.context(gpu.index or 0)
    ctx.set_stream(torch.cuda.current_stream(gpu).cuda_stream)
    p = dummy.data_ptr()
    rc = _lib.lib().kyro_spec_verify_noalloc(ctx.handle, ctypes.byref(params), p, p, p, p, p, p, p, p, p, None, None)
    assert rc == _lib.KYRO_EINVAL
    assert "allocation-free" in _lib.last_error() and str(need.value) in _lib.last_error()
    case = wl.make_verify_case(batch=8, kmax=4, vocab=3000, target_sigma=2.0, noise_sigma=1.0, temperature=1.0,
                               seed=2)
    res = kyro_amd.verify_drafts(**h.verify_tensors(case, gpu), return_probs=True, allocation_free=True)
    h.assert_verify_parity(res, case, h.oracle_verify(case))


def test_noalloc_replays_from_a_graph(gpu):
    """Captured into a HIP graph, the call replays to the eager result on every replay, with
    other allocation-free calls of another shape and synchronisations in between."""
    case = wl.make_verify_case(batch=24, kmax=5, vocab=32000, target_sigma=2.5, noise_sigma=0.8,
                               temperature=0.8, num_draft=np.arange(24) % 6, seed=12)
    other = wl.make_verify_case(batch=7, kmax=2, vocab=1000, target_sigma=2.0, noise_sigma=1.0,
                                temperature=1.2, seed=13)
    t, t2 = h.verify_tensors(case, gpu), h.verify_tensors(other, gpu)
    s = torch.cuda.Stream(gpu)
    with torch.cuda.stream(s):
        eager = kyro_amd.verify_drafts_async(**t, allocation_free=True)
        eager2 = kyro_amd.verify_drafts_async(**t2, allocation_free=True)
        out = (torch.empty_like(eager.accepted), torch.empty_like(eager.tokens))
    torch.cuda.synchronize()
    h.assert_verify_parity(eager, case, h.oracle_verify(case), max_exempt=1)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        kyro_amd.verify_drafts_async(**t, out=out, allocation_free=True)
    for _ in range(3):
        out[0].fill_(-1)
        out[1].fill_(-1)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out[0], eager.accepted) and torch.equal(out[1], eager.tokens)
        with torch.cuda.stream(s):
            again = kyro_amd.verify_drafts_async(**t2, allocation_free=True)
        torch.cuda.synchronize()
        assert torch.equal(again.accepted, eager2.accepted) and torch.equal(again.tokens, eager2.tokens)
    kyro_amd.sync(gpu.index or 0)
