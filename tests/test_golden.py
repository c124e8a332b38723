"""The oracle against the committed golden fixtures (tests/golden/, written by make_golden.py) and
the reference's own known-answer tests, on the CPU."""
import hashlib
import json
import os

import numpy as np
import pytest

import oracle
from kyro_amd import workloads as wl

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _digest(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def _load(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


def test_reference_sample_token_kats():
    for kat in _load("reference_kats.json")["sample_token"]:
        for u in (1e-6, 0.37, 1 - 1e-6):
            got = oracle.sample_token(kat["logits"], kat["temperature"], top_p=kat["top_p"],
                                      top_k=kat["top_k"], u=u)
            assert got in kat["expect"], (kat, u, got)


def test_reference_attention_kats():
    for kat in _load("reference_kats.json")["paged_attention"]:
        H, D, Hkv, bs, nb = kat["num_heads"], kat["head_dim"], kat["num_kv_heads"], kat["block_size"], kat["num_blocks"]
        q = np.full((1, H, D), kat["fill"], np.float32)
        kv = np.full((nb, Hkv, bs, D), kat["fill"], np.float32)
        out = oracle.paged_attention_mq(q, kv, kv, np.array(kat["block_table"], np.int64),
                                        np.array(kat["context_lens"], np.int64), num_heads=H,
                                        num_kv_heads=Hkv, head_dim=D, block_size=bs)
        assert list(out.shape) == kat["expect_shape"]
        np.testing.assert_array_equal(out, kat["expect_value"])


@pytest.fixture(scope="module")
def rejection_case():
    return wl.rejection_only_b8()


def test_rejection_b8_inputs_regenerate(rejection_case):
    g = _load("rejection_b8.json")
    c = rejection_case
    assert _digest(c.target) == g["sha256"]["target"]
    assert _digest(c.draft) == g["sha256"]["draft"]
    assert _digest(c.draft_tokens) == g["sha256"]["draft_tokens"]
    assert _digest(c.u_accept) == g["sha256"]["u_accept"]
    assert _digest(c.u_resample) == g["sha256"]["u_resample"]


def test_rejection_b8_oracle_matches_fixture(rejection_case):
    g = _load("rejection_b8.json")
    c = rejection_case
    r = oracle.spec_verify(c.target, c.draft, c.draft_tokens, c.num_draft, c.temperature,
                           c.u_accept, c.u_resample)
    assert r["accepted"].tolist() == g["accepted"]
    assert r["tokens"].astype(np.int64).tolist() == g["tokens"]
    for name in ("p_draft", "q_draft", "accept_margin"):
        want = np.array([[np.nan if v is None else v for v in row] for row in g[name]])
        np.testing.assert_allclose(r[name], want, rtol=1e-12, equal_nan=True)
    # the f32 build (the CPU baseline) reaches the same decisions on this workload
    r32 = oracle.spec_verify(c.target, c.draft, c.draft_tokens, c.num_draft, c.temperature,
                             c.u_accept, c.u_resample, precision="f32")
    assert r32["accepted"].tolist() == g["accepted"]
    assert r32["tokens"].astype(np.int64).tolist() == g["tokens"]


def test_attention_mha_b2_fixture():
    z = np.load(os.path.join(GOLDEN, "attention_mha_b2.npz"))
    case = wl.make_attention_case(context_lens=[17, 40], q_lens=[5, 5], num_heads=32, num_kv_heads=32,
                                  dtype="bf16", seed=0)
    assert _digest(case.query) == str(z["query_sha256"])
    assert _digest(case.key_cache, case.value_cache) == str(z["kv_sha256"])
    np.testing.assert_array_equal(case.block_table, z["block_table"])
    out = oracle.paged_attention_mq(case.query, case.key_cache, case.value_cache, case.block_table,
                                    case.context_lens, num_heads=32, num_kv_heads=32, head_dim=128,
                                    block_size=16, q_start_loc=case.q_start_loc)
    np.testing.assert_allclose(out, z["expected"], rtol=0, atol=1e-6)
