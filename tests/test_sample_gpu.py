"""Plain-decode sampling on the GPU against the oracle, through the C ABI (kyro_sample_tokens).

Tokens must match bit for bit, except rows whose decision the oracle places within 1e-5 of a
boundary (|r - running sum| or |top_p - running sum|; f32 sums in another order may land on the
other side). Covers argmax, index-order draws, top-k, top-p, both, ties, the logit processors
(bias, penalties, grammar masks), a fully masked row and bad token ids.
"""
import numpy as np
import pytest
import torch

import kyro_amd
import oracle
from tests import helpers as h

pytestmark = pytest.mark.gpu


def run_both(x, T, u, gpu, max_exempt=1, **kw):
    got = kyro_amd.sample_tokens(torch.from_numpy(x).to(gpu), T, u, **kw).cpu().numpy().astype(np.uint32)
    exp, margin = oracle.sample_decode(x, T, u, **kw)
    bad = np.nonzero(got != exp)[0]
    for b in bad:
        assert margin[b] < h.MARGIN, f"row {b}: gpu {got[b]} vs oracle {exp[b]}, margin {margin[b]:.3g}"
    assert len(bad) <= max_exempt, f"{len(bad)} margin exemptions"
    return got


def test_reference_sample_token_kats(gpu):
    rows = [[0.1, 0.2, 0.3, 0.4, 0.5, 10.0, 0.1, 0.2], [1.0, 2.0, 3.0, 0.5, 0.1, 0, 0, 0],
            [0.1, 0.2, 5.0, 0.4, 0, 0, 0, 0]]
    x = np.array(rows, np.float32)
    assert kyro_amd.sample_tokens(torch.from_numpy(x).to(gpu), [0, 0, 0], [0.5] * 3).tolist() == [5, 2, 2]
    assert kyro_amd.sample_token(torch.tensor([100.0, 0, 0, 0, 0], device=gpu), 2.0, 1.0, None, 0.9) == 0
    assert kyro_amd.sample_token(torch.tensor([100.0, 0, 0, 0, 0], device=gpu), 1.0, 0.5, None, 0.9) == 0
    for u in (0.01, 0.5, 0.99):
        assert kyro_amd.sample_token(torch.tensor([1.0, 2.0, 10.0, 0.5, 0.1], device=gpu), 1.0, 1.0, 2, u) in (1, 2)


@pytest.mark.parametrize("V", [37, 1000, 32000, 128256])
@pytest.mark.parametrize("mode", ["greedy", "plain", "top_k", "top_p", "top_k_top_p"])
def test_matches_oracle(gpu, V, mode):
    rng = np.random.default_rng(V + len(mode))
    B = 24
    x = (rng.standard_normal((B, V)) * 3).astype(np.float32)
    T = np.full(B, 0.0 if mode == "greedy" else 0.8, np.float32)
    T[::5] = 1.7 if mode != "greedy" else 0.0
    u = rng.random(B).astype(np.float32)
    kw = {}
    if "top_k" in mode:
        kw["top_k"] = rng.choice([1, 2, 7, 50, V - 1, 0], size=B).astype(np.int32)
    if "top_p" in mode:
        kw["top_p"] = rng.choice([0.0, 0.3, 0.9, 0.95, 1.0], size=B).astype(np.float32)
    run_both(x, T, u, gpu, **kw)


@pytest.mark.parametrize("V", [8, 2052, 4096, 6148, 128256, 1000004])
def test_plain_and_greedy_rows_mixed(gpu, V):
    """Greedy and sampled rows mixed in one batch without processors, top-k or top-p, from one
    short chunk to 245 chunks, with a short last chunk (2052, 6148), a row of -inf but one entry,
    and a row of -inf (the last index when sampled, index 0 at T 0), u = 0 and u just below 1,
    against the oracle."""
    rng = np.random.default_rng(V + 3)
    B = 20
    x = (rng.standard_normal((B, V)) * 3).astype(np.float32)
    x[4, :] = -np.inf
    x[4, V // 3] = 1.0
    x[5, :] = -np.inf
    x[6, :] = -np.inf
    T = np.where(np.arange(B) % 3 == 0, 0.0, 0.8).astype(np.float32)
    T[5] = 1.0
    T[6] = 0.0
    T[7] = 1.7
    u = rng.random(B).astype(np.float32)
    u[8] = 0.0
    u[9] = np.float32(1.0 - 2 ** -24)
    got = run_both(x, T, u, gpu)
    assert got[4] == V // 3 and got[5] == V - 1 and got[6] == 0


def test_one_launch_rows_repeat_and_change_shape(gpu):
    """Batches without processors, top-k or top-p run in one launch whose workgroups count
    themselves on per-row counters that the last one resets: calls back to back give the same
    tokens, and batches of other sizes and vocabularies (4, 1 and 8 workgroups a row) that
    follow them still match the oracle."""
    rng = np.random.default_rng(23)
    for B, V in ((64, 128256), (64, 128256), (3, 128256), (40, 32000), (17, 300004), (64, 128256)):
        x = (rng.standard_normal((B, V)) * 3).astype(np.float32)
        T = np.where(np.arange(B) % 4 == 0, 0.0, 0.8).astype(np.float32)
        u = rng.random(B).astype(np.float32)
        got = run_both(x, T, u, gpu)
        again = kyro_amd.sample_tokens(torch.from_numpy(x).to(gpu), T, u).cpu().numpy().astype(np.uint32)
        assert np.array_equal(got, again)


def test_one_launch_pass_replays_from_a_graph(gpu):
    """The one-launch pass captured in a HIP graph after an eager call on the same stream (the
    arena already large enough): its per-row counters return to zero in every launch, so each
    replay, with eager calls of another shape and synchronisations in between, gives the eager
    tokens, which match the oracle."""
    rng = np.random.default_rng(41)
    B, V = 64, 128256
    x = (rng.standard_normal((B, V)) * 3).astype(np.float32)
    T = np.where(np.arange(B) % 4 == 0, 0.0, 0.8).astype(np.float32)
    u = rng.random(B).astype(np.float32)
    x2 = (rng.standard_normal((5, 32000)) * 3).astype(np.float32)
    T2, u2 = np.full(5, 0.7, np.float32), rng.random(5).astype(np.float32)
    exp = run_both(x, T, u, gpu)
    dx, dT, du = torch.from_numpy(x).to(gpu), torch.from_numpy(T).to(gpu), torch.from_numpy(u).to(gpu)
    dx2, dT2, du2 = torch.from_numpy(x2).to(gpu), torch.from_numpy(T2).to(gpu), torch.from_numpy(u2).to(gpu)
    procs = kyro_amd.sampling.Processors(B, V, gpu)
    procs2 = kyro_amd.sampling.Processors(5, 32000, gpu)
    s = torch.cuda.Stream(gpu)
    with torch.cuda.stream(s):
        eager = kyro_amd.sample_tokens_async(dx, dT, du, processors=procs).clone()
        eager2 = kyro_amd.sample_tokens_async(dx2, dT2, du2, processors=procs2).clone()
        out = torch.empty(B, dtype=torch.int32, device=gpu)
    torch.cuda.synchronize()
    assert np.array_equal(eager.cpu().numpy().astype(np.uint32), exp)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        kyro_amd.sample_tokens_async(dx, dT, du, processors=procs, out=out)
    for _ in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        with torch.cuda.stream(s):
            again = kyro_amd.sample_tokens_async(dx2, dT2, du2, processors=procs2)
        torch.cuda.synchronize()
        assert torch.equal(again, eager2)


def test_ties_follow_the_index(gpu):
    """Small integer logits: many equal values, so top-k boundaries and the descending order
    depend on the tie rule (lower index first)."""
    rng = np.random.default_rng(7)
    B, V = 40, 500
    x = rng.integers(-3, 4, size=(B, V)).astype(np.float32)
    u = rng.random(B).astype(np.float32)
    T = np.ones(B, np.float32)
    run_both(x, T, u, gpu, top_k=rng.integers(1, 60, size=B).astype(np.int32))
    run_both(x, T, u, gpu, top_p=rng.choice([0.2, 0.5, 0.8], size=B).astype(np.float32))
    run_both(x, np.zeros(B, np.float32), u, gpu)


def test_wide_dynamic_range(gpu):
    """Logits spread over 2^-60 .. 2^60 in magnitude: a 4096-entry chunk then spans more distinct
    key bins than its list holds, so top-k and top-p rows take the exact radix path."""
    rng = np.random.default_rng(17)
    B, V = 12, 32000
    x = (rng.choice([-1.0, 1.0], size=(B, V)) * np.exp2(rng.uniform(-60, 60, size=(B, V)))).astype(np.float32)
    u = rng.random(B).astype(np.float32)
    T = np.full(B, 1.0, np.float32)
    run_both(x, T, u, gpu, top_k=rng.choice([1, 5, 300], size=B).astype(np.int32))
    run_both(x, T, u, gpu, top_p=rng.choice([0.3, 0.9], size=B).astype(np.float32))
    run_both(x, T, u, gpu)


@pytest.mark.parametrize("V,scale,kw", [
    (128256, 3.1, {"top_p": 0.9}),   # nucleus of a few thousand tokens: wider than the chunk lists
    (128256, 3.0, {"top_p": 0.95}),
    (32000, 2.0, {"top_k": 1000}),   # k above a chunk list's slots
    (128256, 3.0, {"top_k": 300, "top_p": 0.9}),
])
def test_rows_the_chunk_lists_do_not_cover(gpu, V, scale, kw):
    """Rows whose kept set the stats pass's per-chunk candidate lists cannot hold: the select pass
    gathers candidates from the row itself (one workgroup, two passes) and settles them exactly."""
    rng = np.random.default_rng(V + int(scale * 10))
    B = 8
    x = (rng.standard_normal((B, V)) * scale).astype(np.float32)
    T = np.ones(B, np.float32)
    u = rng.random(B).astype(np.float32)
    args = {k: np.full(B, v, np.int32 if k == "top_k" else np.float32) for k, v in kw.items()}
    run_both(x, T, u, gpu, **args)


@pytest.mark.parametrize("V", [50001, 200000, 1000003])
def test_list_shapes(gpu, V):
    """Vocabularies whose chunk lists take other shapes: 50001 entries (not a multiple of four:
    scalar loads, a short last chunk) and 200000 (49 chunks, so 167 list slots a chunk instead of
    256), 1000003 (245 chunks: 33 slots, fewer than some k). Top-k, top-p and both, with one row
    masked down to fewer allowed tokens than k."""
    rng = np.random.default_rng(V)
    B = 12
    x = (rng.standard_normal((B, V)) * 3).astype(np.float32)
    T = np.full(B, 0.8, np.float32)
    u = rng.random(B).astype(np.float32)
    masks = np.stack([kyro_amd.grammar_mask(rng.choice(V, size=30, replace=False), V)])
    mask_row = np.full(B, -1, np.int32)
    mask_row[3] = 0
    k = rng.choice([1, 40, 100, 160], size=B).astype(np.int32)
    k[3] = 50  # more than the 30 allowed tokens
    tp = rng.choice([0.5, 0.9, 0.99], size=B).astype(np.float32)
    run_both(x, T, u, gpu, top_k=k, masks=masks, mask_row=mask_row)
    run_both(x, T, u, gpu, top_p=tp, masks=masks, mask_row=mask_row)
    run_both(x, T, u, gpu, top_k=k, top_p=tp, masks=masks, mask_row=mask_row)


def test_processors(gpu):
    rng = np.random.default_rng(8)
    B, V = 16, 5000
    x = rng.standard_normal((B, V)).astype(np.float32)
    bias = [{int(t): float(rng.normal(0, 3)) for t in rng.integers(0, V, size=int(rng.integers(0, 40)))} if b % 3 else None
            for b in range(B)]
    penalty = [kyro_amd.penalty_adds(rng.integers(0, V, size=int(rng.integers(0, 300))), float(rng.choice([0, 0.5, -0.7])),
                                     float(rng.choice([0, 0.3, -0.2])), V) for b in range(B)]
    masks = np.stack([kyro_amd.grammar_mask(None, V), kyro_amd.grammar_mask(kyro_amd.sampling.JSON_TOKENS, V),
                      kyro_amd.grammar_mask(rng.choice(V, size=700, replace=False), V)])
    mask_row = rng.integers(-1, 3, size=B).astype(np.int32)
    T = rng.choice([0.0, 0.6, 1.0], size=B).astype(np.float32)
    u = rng.random(B).astype(np.float32)
    kw = dict(bias=bias, penalty=penalty, masks=masks, mask_row=mask_row)
    got = run_both(x, T, u, gpu, **kw)
    for b in range(B):
        if mask_row[b] == 1:
            assert got[b] in kyro_amd.sampling.JSON_TOKENS
    run_both(x, T, u, gpu, top_k=np.full(B, 20, np.int32), top_p=np.full(B, 0.9, np.float32), **kw)
    # the input logits are untouched (processing happens in the workspace)
    xt = torch.from_numpy(x).to(gpu)
    kyro_amd.sample_tokens(xt, T, u, **kw)
    assert torch.equal(xt.cpu(), torch.from_numpy(x))


def test_fully_masked_row_gets_the_last_index(gpu):
    x = np.zeros((2, 64), np.float32)
    masks = np.stack([kyro_amd.grammar_mask([], 64)])
    got = kyro_amd.sample_tokens(torch.from_numpy(x).to(gpu), [1.0, 0.5], [0.3, 0.6], masks=masks, mask_row=[0, 0])
    assert got.tolist() == [63, 63]


def test_bad_token_ids_raise_and_recover(gpu):
    x = torch.zeros((2, 10), device=gpu)
    with pytest.raises(kyro_amd.KyroError, match="vocab_size"):
        kyro_amd.sample_tokens(x, [1.0, 1.0], [0.5, 0.5], bias=[{10: 1.0}, None])
    assert kyro_amd.sample_tokens(x, [0.0, 0.0], [0.5, 0.5], bias=[{7: 1.0}, {2: 1.0}]).tolist() == [7, 2]


def test_token_law_on_the_gpu(gpu):
    """Chi-square over 60k rows: plain and top-p draws follow the renormalised distributions."""
    rng = np.random.default_rng(9)
    V, N = 10, 60000
    x = (rng.standard_normal(V) * 0.7).astype(np.float32)
    z = (x * np.float32(1 / 0.9)).astype(np.float64)
    u = rng.random(N).astype(np.float32)
    xs = torch.from_numpy(np.broadcast_to(x, (N, V)).copy()).to(gpu)
    import scipy.stats
    for tp in (1.0, 0.75):
        got = kyro_amd.sample_tokens(xs, np.full(N, 0.9, np.float32), u, top_p=np.full(N, tp, np.float32)).cpu().numpy()
        order = np.argsort(-z, kind="stable")
        p = np.exp(z - z.max())
        p /= p.sum()
        if tp < 1:
            cs = np.cumsum(p[order])
            cut = int(np.argmax(cs > tp)) + 1
            q = np.zeros(V)
            q[order[:cut]] = p[order[:cut]]
            p = q / q.sum()
        counts = np.bincount(got, minlength=V)
        nz = p > 0
        assert counts[~nz].sum() == 0
        assert scipy.stats.chisquare(counts[nz], p[nz] * N).pvalue > 1e-4
