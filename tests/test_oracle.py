"""Pins the CPU oracle before anything is compared against it.

Attention is checked against torch's CPU scaled_dot_product_attention on the gathered,
contiguous KV (an independent implementation) and against closed forms; the sampler against
the reference's own sample_token known-answer tests (src/worker.rs:395-457), numpy's
searchsorted for the inverse-CDF walk, and a chi-square test of Leviathan et al. (2023),
Theorem 1: whatever the draft distribution q, the first emitted token is distributed as p_0.
"""
import numpy as np
import pytest
import scipy.special
import scipy.stats
import torch

import oracle
from kyro_amd import workloads as wl


def _dense_reference(case, causal=True):
    """softmax(q K^T / sqrt(D)) V per head via torch SDPA on the gathered contiguous context."""
    H, Hkv, D, bs = case.num_heads, case.num_kv_heads, case.head_dim, case.block_size
    if case.dtype == "bf16":
        q_all = wl.bf16_bits_to_f32(case.query)
        kc, vc = wl.bf16_bits_to_f32(case.key_cache), wl.bf16_bits_to_f32(case.value_cache)
    else:
        q_all, kc, vc = case.query, case.key_cache, case.value_cache
    out = np.zeros(q_all.shape, dtype=np.float64)
    for b in range(case.batch):
        ctx = int(case.context_lens[b])
        q0, q1 = int(case.q_start_loc[b]), int(case.q_start_loc[b + 1])
        if ctx == 0 or q1 == q0:
            continue
        blocks = case.block_table[b, : -(-ctx // bs)]
        k = kc[blocks].transpose(1, 0, 2, 3).reshape(Hkv, -1, D)[:, :ctx]
        v = vc[blocks].transpose(1, 0, 2, 3).reshape(Hkv, -1, D)[:, :ctx]
        k = torch.from_numpy(np.ascontiguousarray(k)).double().repeat_interleave(H // Hkv, dim=0)
        v = torch.from_numpy(np.ascontiguousarray(v)).double().repeat_interleave(H // Hkv, dim=0)
        q = torch.from_numpy(np.ascontiguousarray(q_all[q0:q1].transpose(1, 0, 2))).double()
        qlen = q1 - q0
        mask = None
        if causal:
            j = torch.arange(qlen)[:, None]
            t = torch.arange(ctx)[None, :]
            mask = t <= (ctx - qlen + j)
            if not bool(mask.any(dim=1).all()):
                raise AssertionError("test case has a query row with no visible key")
        o = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=mask)
        out[q0:q1] = o.transpose(0, 1).numpy()
    return out


def _run_oracle(case, causal=True, **kw):
    return oracle.paged_attention_mq(
        case.query, case.key_cache, case.value_cache, case.block_table, case.context_lens,
        num_heads=case.num_heads, num_kv_heads=case.num_kv_heads, head_dim=case.head_dim,
        block_size=case.block_size, q_start_loc=case.q_start_loc, causal=causal, **kw)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("heads", [(8, 2), (4, 4), (8, 1)])
def test_attention_matches_torch_sdpa(dtype, heads):
    H, Hkv = heads
    case = wl.make_attention_case(context_lens=[17, 40, 5, 33, 16], q_lens=[1, 5, 3, 2, 4],
                                  num_heads=H, num_kv_heads=Hkv, head_dim=64, dtype=dtype, seed=3,
                                  num_blocks=20)
    got = _run_oracle(case)
    ref = _dense_reference(case)
    np.testing.assert_allclose(got, ref, atol=1e-10, rtol=1e-9)


def test_attention_noncausal_matches_torch_sdpa():
    case = wl.make_attention_case(context_lens=[9, 31, 64], q_lens=[2, 2, 3], num_heads=4,
                                  num_kv_heads=2, head_dim=128, dtype="f32", seed=5)
    np.testing.assert_allclose(_run_oracle(case, causal=False), _dense_reference(case, causal=False),
                               atol=1e-10, rtol=1e-9)


def test_attention_f32_build_tracks_f64():
    case = wl.make_attention_case(context_lens=[100, 37], q_lens=[3, 1], num_heads=8,
                                  num_kv_heads=2, head_dim=64, dtype="bf16", seed=7)
    np.testing.assert_allclose(_run_oracle(case, precision="f32"), _run_oracle(case), atol=2e-5)


def test_reference_all_ones_cases():
    """attention_kernel.rs:185-227: all-ones MHA, ctx 8 in one block and ctx 24 over the aliased
    table [0,0,0,0]: softmax of equal scores averages all-ones V -> 1 everywhere."""
    for ctx in (8, 24):
        q = np.ones((1, 8, 64), np.float32)
        kv = np.ones((4, 8, 16, 64), np.float32)
        out = oracle.paged_attention_mq(q, kv, kv, np.zeros((1, 4), np.int64), np.array([ctx]),
                                        num_heads=8, num_kv_heads=8, head_dim=64, block_size=16)
        assert out.shape == (1, 8, 64)
        np.testing.assert_array_equal(out, 1.0)


def test_reference_zero_context():
    """attention_kernel.rs:163-183 (GQA 8/2, D 64, ctx 0): zeros of shape [1, 8, 64]."""
    out = oracle.paged_attention_mq(np.zeros((1, 8, 64), np.float32), np.zeros((4, 2, 16, 64), np.float32),
                                    np.zeros((4, 2, 16, 64), np.float32), np.zeros((1, 4), np.int64),
                                    np.array([0]), num_heads=8, num_kv_heads=2, head_dim=64, block_size=16)
    assert out.shape == (1, 8, 64)
    np.testing.assert_array_equal(out, 0.0)


def test_single_key_returns_its_value_and_equal_keys_average():
    g = np.random.default_rng(0)
    kv = g.standard_normal((3, 2, 16, 64)).astype(np.float32)
    q = g.standard_normal((1, 4, 64)).astype(np.float32)
    table = np.array([[2, 0, 1]], np.int64)
    out = oracle.paged_attention_mq(q, kv, kv.copy(), table, np.array([1]), num_heads=4, num_kv_heads=2,
                                    head_dim=64, block_size=16)
    for h in range(4):
        np.testing.assert_allclose(out[0, h], kv[2, h // 2, 0], rtol=1e-12)
    keys = np.broadcast_to(kv[:1, :, :1], kv.shape).copy()  # one key per kv head, everywhere
    out = oracle.paged_attention_mq(q, keys, kv, table, np.array([40]), num_heads=4, num_kv_heads=2,
                                    head_dim=64, block_size=16)
    vals = np.concatenate([kv[2], kv[0], kv[1]], axis=1)[:, :40]  # [Hkv, 40, D]
    for h in range(4):
        np.testing.assert_allclose(out[0, h], vals[h // 2].astype(np.float64).mean(0), rtol=1e-9, atol=1e-12)


def test_block_permutation_invariance():
    case = wl.make_attention_case(context_lens=[70, 23], q_lens=[4, 2], num_heads=8, num_kv_heads=2,
                                  head_dim=64, dtype="f32", seed=11)
    base = _run_oracle(case)
    nb = case.key_cache.shape[0]
    perm = np.random.default_rng(1).permutation(nb)  # physical block i moves to slot perm[i]
    k2 = np.empty_like(case.key_cache)
    v2 = np.empty_like(case.value_cache)
    k2[perm] = case.key_cache
    v2[perm] = case.value_cache
    case.key_cache, case.value_cache = k2, v2
    case.block_table = perm[case.block_table]
    np.testing.assert_allclose(_run_oracle(case), base, rtol=1e-12, atol=1e-14)


def test_gqa_equals_mha_with_repeated_kv():
    case = wl.make_attention_case(context_lens=[50, 17], q_lens=[3, 1], num_heads=8, num_kv_heads=2,
                                  head_dim=64, dtype="f32", seed=12)
    gqa = _run_oracle(case)
    case.key_cache = np.repeat(case.key_cache, 4, axis=1)
    case.value_cache = np.repeat(case.value_cache, 4, axis=1)
    case.num_kv_heads = 8
    np.testing.assert_allclose(_run_oracle(case), gqa, rtol=1e-12, atol=1e-14)


def test_causal_row_equals_noncausal_prefix():
    case = wl.make_attention_case(context_lens=[45], q_lens=[5], num_heads=4, num_kv_heads=4,
                                  head_dim=64, dtype="f32", seed=13)
    full = _run_oracle(case)
    for j in range(5):
        visible = 45 - 5 + j + 1
        single = oracle.paged_attention_mq(case.query[j:j + 1], case.key_cache, case.value_cache,
                                           case.block_table, np.array([visible]), num_heads=4,
                                           num_kv_heads=4, head_dim=64, block_size=16, causal=False)
        np.testing.assert_allclose(full[j], single[0], rtol=1e-12, atol=1e-14)


def test_invalid_block_id_is_an_error():
    q = np.ones((1, 2, 64), np.float32)
    kv = np.ones((2, 2, 16, 64), np.float32)
    with pytest.raises(ValueError):
        oracle.paged_attention_mq(q, kv, kv, np.array([[0, 7]], np.int64), np.array([20]), num_heads=2,
                                  num_kv_heads=2, head_dim=64, block_size=16)


# ------------------------------------------------------------------------------- sampling


def test_reference_sample_token_kats():
    """src/worker.rs:395-449."""
    assert oracle.sample_token([0.1, 0.2, 0.3, 0.4, 0.5, 10.0, 0.1, 0.2], 0.0) == 5
    assert oracle.sample_token([1.0, 2.0, 3.0, 0.5, 0.1], 0.0) == 2
    assert oracle.sample_token([0.1, 0.2, 5.0, 0.4], 0.0) == 2
    for u in (1e-6, 0.5, 1 - 1e-6):
        assert oracle.sample_token([100.0, 0, 0, 0, 0], 2.0, u=u) == 0
        assert oracle.sample_token([100.0, 0, 0, 0, 0], 1.0, top_p=0.5, u=u) == 0
        assert oracle.sample_token([1.0, 2.0, 10.0, 0.5, 0.1], 1.0, top_k=2, u=u) in (1, 2)
    assert oracle.sample_token([], 1.0) == -1


def test_inverse_cdf_matches_searchsorted():
    g = np.random.default_rng(0)
    logits = g.standard_normal(50).astype(np.float32) * 2
    p = scipy.special.softmax(logits.astype(np.float64) / 0.7)
    cdf = np.cumsum(p)
    for u in g.random(300):
        want = int(np.searchsorted(cdf, u * cdf[-1], side="left"))
        gaps = np.abs(cdf - u * cdf[-1])
        if gaps.min() < 1e-9:
            continue
        assert oracle.sample_token(logits, 0.7, u=u) == want


def _verify(target, draft, tokens, k, T, ua, ur):
    B = target.shape[0]
    return oracle.spec_verify(target, draft, tokens, np.full(B, k, np.int32) if np.isscalar(k) else k,
                              np.full(B, T, np.float32) if np.isscalar(T) else T, ua, ur)


def test_greedy_accept_until_mismatch():
    """speculative.rs:315-323: accept while argmax(t_i) == x_i; emit argmax(t_j) at the mismatch;
    plus the bonus argmax(t_k) after full acceptance. Ties resolve to the lowest index."""
    V, k = 10, 4
    t = np.zeros((3, k + 1, V), np.float32)
    top = [[3, 1, 4, 1, 5], [2, 7, 1, 8, 2], [0, 0, 0, 0, 9]]
    for b in range(3):
        for i in range(k + 1):
            t[b, i, top[b][i]] = 5.0
    t[2, 1, 6] = 5.0  # tie with index 0 in row 1 -> argmax 0
    drafts = np.array([[3, 1, 4, 1], [2, 7, 3, 8], [0, 0, 9, 0]], np.int32)
    r = _verify(t, None, drafts, k, 0.0, np.full((3, k), 0.5, np.float32), np.full(3, 0.5, np.float32))
    assert r["accepted"].tolist() == [4, 2, 2]
    assert r["tokens"][0].tolist() == [3, 1, 4, 1, 5]
    assert r["tokens"][1, :3].tolist() == [2, 7, 1]
    assert r["tokens"][2, :3].tolist() == [0, 0, 0]
    assert (r["tokens"][1, 3:] == 0xFFFFFFFF).all()


def test_identical_draft_accepts_everything_then_samples_p_k():
    g = np.random.default_rng(4)
    B, k, V = 6, 3, 40
    t = (g.standard_normal((B, k + 1, V)) * 2).astype(np.float32)
    d = t[:, :k].copy()
    tokens = g.integers(0, V, (B, k)).astype(np.int32)
    ur = g.random(B).astype(np.float32)
    r = _verify(t, d, tokens, k, 1.3, g.random((B, k)).astype(np.float32), ur)
    assert (r["accepted"] == k).all()
    for b in range(B):
        p = scipy.special.softmax(t[b, k].astype(np.float64) / np.float64(np.float32(1.3)))
        want = int(np.searchsorted(np.cumsum(p), ur[b] * p.sum()))
        assert r["tokens"][b, k] == want
        np.testing.assert_allclose(r["p_draft"][b], r["q_draft"][b], rtol=1e-12)


def test_p_q_at_draft_tokens_match_scipy_softmax():
    case = wl.rejection_only_b8()
    r = _verify(case.target, case.draft, case.draft_tokens, 4, 1.0, case.u_accept, case.u_resample)
    for b in range(case.batch):
        for i in range(int(r["accepted"][b]) + (1 if r["accepted"][b] < 4 else 0)):
            x = case.draft_tokens[b, i]
            p = scipy.special.softmax(case.target[b, i].astype(np.float64))[x]
            q = scipy.special.softmax(case.draft[b, i].astype(np.float64))[x]
            assert abs(r["p_draft"][b, i] - p) < 1e-15 + 1e-12 * p
            assert abs(r["q_draft"][b, i] - q) < 1e-15 + 1e-12 * q
            accept = ua = case.u_accept[b, i] < min(1.0, p / q)
            assert accept == (i < r["accepted"][b]), (b, i, ua)


def test_first_token_law_is_p0_whatever_q():
    """Leviathan et al. 2023, Thm 1: x ~ q, accept with min(1, p/q), else draw from
    norm(max(p - q, 0)): the first emitted token is distributed exactly as p."""
    V, N = 8, 200_000
    g = np.random.default_rng(123)
    t_row = np.array([2.0, 0.5, -1.0, 1.5, 0.0, -0.5, 1.0, -2.0], np.float32)
    d_row = np.array([0.0, 2.0, 1.0, -1.0, 0.5, 1.5, -1.0, 0.0], np.float32)
    T = 1.0
    q = scipy.special.softmax(d_row.astype(np.float64) / T)
    p = scipy.special.softmax(t_row.astype(np.float64) / T)
    x = np.searchsorted(np.cumsum(q), g.random(N) * q.sum()).clip(0, V - 1).astype(np.int32)
    target = np.broadcast_to(np.stack([t_row, t_row])[None], (N, 2, V)).copy()
    draft = np.broadcast_to(d_row[None, None], (N, 1, V)).copy()
    r = _verify(target, draft, x[:, None], 1, T, g.random((N, 1)).astype(np.float32),
                g.random(N).astype(np.float32))
    first = r["tokens"][:, 0].astype(np.int64)
    counts = np.bincount(first, minlength=V)
    chi2, pval = scipy.stats.chisquare(counts, p * N)
    assert pval > 1e-4, (counts, p * N, chi2)
    # the draft law differs enough from p that skipping the correction would be detected
    _, pval_q = scipy.stats.chisquare(np.bincount(x, minlength=V), p * N)
    assert pval_q < 1e-12


def test_bad_inputs_are_errors():
    t = np.zeros((1, 2, 4), np.float32)
    with pytest.raises(ValueError):
        oracle.spec_verify(t, t[:, :1], np.array([[9]], np.int32), np.array([1], np.int32),
                           np.array([1.0], np.float32), np.array([[0.5]], np.float32),
                           np.array([0.5], np.float32))
    with pytest.raises(ValueError):
        oracle.spec_verify(t, t[:, :1], np.array([[0]], np.int32), np.array([2], np.int32),
                           np.array([1.0], np.float32), np.array([[0.5]], np.float32),
                           np.array([0.5], np.float32))
