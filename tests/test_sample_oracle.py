"""The decode-sampler oracle (oracle_sample_decode) and the host penalty helper, without a GPU.

Pins: the reference's sample_token known-answer tests (src/worker.rs:395-457) and grammar tests
(src/api/grammar.rs:66-136); the penalty helper against the reference's two loops run literally,
occurrence by occurrence, over a dense f32 array (worker.rs:161-176); the token law (chi-square:
plain, top-k and top-p draws follow the renormalised distributions, computed with numpy); and
the inverse-CDF mapping against numpy's searchsorted in index order and in the stable
descending order.
"""
import numpy as np
import pytest
import scipy.stats

import kyro_amd
import oracle


def row(x):
    return np.asarray([x], np.float32)


# ----------------------------------------------------------- worker.rs sample_token tests


def test_reference_sample_token_kats():
    one = lambda x, T, **kw: int(oracle.sample_decode(row(x), [T], [0.37], **kw)[0][0])  # noqa: E731
    assert one([0.1, 0.2, 0.3, 0.4, 0.5, 10.0, 0.1, 0.2], 0.0) == 5
    assert one([1.0, 2.0, 3.0, 0.5, 0.1], 0.0) == 2
    assert one([0.1, 0.2, 5.0, 0.4], 0.0) == 2
    assert one([100.0, 0, 0, 0, 0], 2.0) == 0
    assert one([100.0, 0, 0, 0, 0], 1.0, top_p=[0.5]) == 0
    for u in (0.01, 0.5, 0.99):
        t = int(oracle.sample_decode(row([1.0, 2.0, 10.0, 0.5, 0.1]), [1.0], [u], top_k=[2])[0][0])
        assert t in (1, 2)


# ------------------------------------------------------------------ grammar.rs tests


def test_reference_grammar_masks():
    none = kyro_amd.grammar_mask(None, 100)
    assert sum(bin(int(w)).count("1") for w in none) == 100
    js = kyro_amd.grammar_mask(kyro_amd.sampling.JSON_TOKENS, 200)
    allowed = [v for v in range(200) if (int(js[v >> 5]) >> (v & 31)) & 1]
    assert allowed == [0, 10, 32, 34, 91, 93, 123, 125]
    # apply_grammar_mask with no constraint leaves ones unchanged; JSON leaves only its tokens
    ones = np.ones((1, 200), np.float32)
    rng = np.random.default_rng(0)
    for u in rng.random(50):
        t = int(oracle.sample_decode(ones, [1.0], [u], masks=js[None], mask_row=[0])[0][0])
        assert t in allowed
    assert int(oracle.sample_decode(ones[:, :100], [0.0], [0.5], masks=none[None], mask_row=[0])[0][0]) == 0


# -------------------------------------------------------------- penalties (worker.rs:154-181)


def literal_penalty(gen, fp, pp, V):
    """The reference's loops over a dense f32 vector, occurrence by occurrence."""
    mask = np.zeros(V, np.float32)
    fp, pp = np.float32(fp), np.float32(pp)
    for t in gen:
        if t < V:
            mask[t] = np.float32(mask[t] + fp)
    for t in gen:
        if t < V:
            mask[t] = np.float32(min(mask[t], np.float32(0.0)) + pp)
    return mask


@pytest.mark.parametrize("seed", range(6))
def test_penalty_helper_equals_the_reference_loops(seed):
    rng = np.random.default_rng(seed)
    V = 50
    gen = rng.integers(0, V + 5, size=int(rng.integers(0, 200))).tolist()
    fp, pp = (float(x) for x in rng.choice([-1.3, -0.1, 0.0, 0.2, 0.7, 1e-3], size=2))
    got = kyro_amd.penalty_adds(gen, fp, pp, V)
    dense = literal_penalty(gen, fp, pp, V)
    if fp == 0.0 and pp == 0.0:
        assert got == {}
        return
    assert sorted(got) == sorted({t for t in gen if t < V})
    for t, v in got.items():
        assert np.float32(v) == dense[t], (t, v, dense[t])


def test_penalty_closed_forms():
    # non-negative penalties: the second loop replaces any count by exactly presence_penalty
    assert kyro_amd.penalty_adds([7] * 13 + [2], 0.5, 0.25, 10) == {2: 0.25, 7: 0.25}
    # negative frequency penalty survives: count c gives c * fp + pp after one clamp-free pass
    got = kyro_amd.penalty_adds([4, 4, 4], -1.0, 0.5, 10)
    assert got == {4: float(literal_penalty([4, 4, 4], -1.0, 0.5, 10)[4])}


# ------------------------------------------------------------------------- token law


def softmax(z):
    e = np.exp(z - z.max())
    return e / e.sum()


@pytest.mark.parametrize("mode", ["plain", "top_k", "top_p", "top_k_top_p"])
def test_token_law_matches_the_renormalised_distribution(mode):
    rng = np.random.default_rng(3)
    V, N, T = 12, 40000, 0.8
    x = (rng.standard_normal(V) * 0.5).astype(np.float32)
    z = (x * np.float32(1 / T)).astype(np.float64)
    k = 5 if "top_k" in mode else 0
    tp = 0.8 if "top_p" in mode else 1.0
    order = np.argsort(-z, kind="stable")
    keep = order[:k] if k else order
    p = np.zeros(V)
    p[keep] = softmax(z[keep])
    if tp < 1:
        cs = np.cumsum(p[order])
        cut = int(np.argmax(cs > tp)) + 1
        q = np.zeros(V)
        q[order[:cut]] = p[order[:cut]]
        p = q / q.sum()
    u = rng.random(N).astype(np.float32)
    toks, _ = oracle.sample_decode(np.broadcast_to(x, (N, V)).copy(), np.full(N, T), u,
                                   top_k=np.full(N, k), top_p=np.full(N, tp))
    counts = np.bincount(toks.astype(np.int64), minlength=V)
    assert counts[p == 0].sum() == 0
    nz = p > 0
    assert nz.sum() >= 3  # enough categories for the test to have power
    assert scipy.stats.chisquare(counts[nz], p[nz] * N).pvalue > 1e-4


def test_inverse_cdf_maps_like_searchsorted():
    rng = np.random.default_rng(4)
    V = 300
    x = rng.standard_normal(V).astype(np.float32)
    x[::7] = x[3]  # ties
    z = (x * np.float32(1 / 1.3)).astype(np.float64)
    for u in rng.random(200):
        tok, mg = oracle.sample_decode(row(x), [1.3], [u])
        cs = np.cumsum(softmax(z))
        exp_plain = int(np.searchsorted(cs, u, side="left"))
        if mg[0] > 1e-9:
            assert int(tok[0]) == min(exp_plain, V - 1)
        tok, mg = oracle.sample_decode(row(x), [1.3], [u], top_p=[0.7])
        order = np.argsort(-z, kind="stable")
        cs = np.cumsum(softmax(z)[order])
        cut = int(np.argmax(cs > 0.7)) + 1
        r = u * cs[cut - 1]
        exp_p = int(order[min(int(np.searchsorted(cs[:cut], r, side="left")), cut - 1)])
        if mg[0] > 1e-9:
            assert int(tok[0]) == exp_p


def test_bias_penalty_and_mask_are_applied_in_order():
    x = np.zeros((1, 8), np.float32)
    # bias lifts token 3, the penalty lowers it again below token 6's bias
    tok, _ = oracle.sample_decode(x, [0.0], [0.5], bias=[{3: 5.0, 6: 2.0}], penalty=[{3: -4.0}])
    assert int(tok[0]) == 6
    mask = kyro_amd.grammar_mask([1, 3], 8)
    tok, _ = oracle.sample_decode(x, [0.0], [0.5], bias=[{3: 5.0, 6: 9.0}], masks=mask[None], mask_row=[0])
    assert int(tok[0]) == 3
    # everything masked: the last index
    tok, _ = oracle.sample_decode(x, [1.0], [0.5], masks=kyro_amd.grammar_mask([], 8)[None], mask_row=[0])
    assert int(tok[0]) == 7
