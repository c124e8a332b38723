"""Fused acceptance sampling on the GPU against the oracle, through the C ABI (kyro_spec_verify).

Accepted lengths and emitted tokens must match bit for bit, except decisions the oracle places
within 1e-5 of a boundary; probabilities at the draft tokens within 1e-5.
"""
import numpy as np
import pytest
import scipy.special
import scipy.stats
import torch

import kyro_amd
from kyro_amd import workloads as wl
from tests import helpers as h

pytestmark = pytest.mark.gpu


def run(case, gpu, with_draft=True, return_probs=True):
    t = h.verify_tensors(case, gpu, with_draft)
    return kyro_amd.verify_drafts(**t, return_probs=return_probs)


def test_rejection_only_b8_matches_oracle(gpu):
    case = wl.rejection_only_b8()
    res = run(case, gpu)
    h.assert_verify_parity(res, case, h.oracle_verify(case))


def test_greedy_reference_semantics(gpu):
    """speculative.rs:315-323 with the bonus token; ties -> lowest index."""
    V, k = 10, 4
    t = np.zeros((3, k + 1, V), np.float32)
    top = [[3, 1, 4, 1, 5], [2, 7, 1, 8, 2], [0, 0, 0, 0, 9]]
    for b in range(3):
        for i in range(k + 1):
            t[b, i, top[b][i]] = 5.0
    t[2, 1, 6] = 5.0
    case = wl.VerifyCase(t, np.zeros((3, k, V), np.float32),
                         np.array([[3, 1, 4, 1], [2, 7, 3, 8], [0, 0, 9, 0]], np.int32),
                         np.full(3, k, np.int32), np.zeros(3, np.float32),
                         np.full((3, k), 0.5, np.float32), np.full(3, 0.5, np.float32))
    res = run(case, gpu, with_draft=False)
    assert res.emitted() == [[3, 1, 4, 1, 5], [2, 7, 1], [0, 0, 0]]
    h.assert_verify_parity(res, case, h.oracle_verify(case))


def test_reference_sample_token_kats_as_k0(gpu):
    """worker.rs:395-431 as k = 0 verify steps (plain decode): argmax at T = 0, the dominant
    logit at T = 2."""
    rows = [[0.1, 0.2, 0.3, 0.4, 0.5, 10.0, 0.1, 0.2], [1.0, 2.0, 3.0, 0.5, 0.1, 0, 0, 0],
            [100.0, 0, 0, 0, 0, 0, 0, 0]]
    t = np.array(rows, np.float32)[:, None, :]
    rows_T = np.array([0.0, 0.0, 2.0], np.float32)
    case = wl.VerifyCase(t, np.zeros((3, 0, 8), np.float32), np.zeros((3, 0), np.int32),
                         np.zeros(3, np.int32), rows_T, np.zeros((3, 0), np.float32),
                         np.array([0.3, 0.9, 0.999], np.float32))
    res = run(case, gpu, with_draft=False)
    assert res.accepted.cpu().tolist() == [0, 0, 0]
    assert res.tokens[:, 0].cpu().tolist() == [5, 2, 0]


@pytest.mark.parametrize("vocab", [37, 1000, 32000, 50001])
@pytest.mark.parametrize("T", [0.0, 0.7, 1.0, 1.6])
def test_parity_over_vocab_and_temperature(gpu, vocab, T):
    case = wl.make_verify_case(batch=24, kmax=5, vocab=vocab, target_sigma=2.5, noise_sigma=0.8,
                               temperature=T, num_draft=np.arange(24) % 6, seed=vocab)
    res = run(case, gpu)
    h.assert_verify_parity(res, case, h.oracle_verify(case), max_exempt=1)


def test_identical_draft_accepts_all(gpu):
    case = wl.make_verify_case(batch=16, kmax=4, vocab=5000, target_sigma=2.0, noise_sigma=0.0,
                               temperature=1.0, seed=3)
    res = run(case, gpu)
    assert (res.accepted.cpu() == 4).all()
    h.assert_verify_parity(res, case, h.oracle_verify(case))


def test_mixed_batch_reduced(gpu):
    k = wl.rng(0, wl.S_KSEQ).integers(0, 9, size=32)
    case = wl.verify_mixed(k, vocab=20000)
    h.assert_verify_parity(run(case, gpu), case, h.oracle_verify(case), max_exempt=1)


@pytest.mark.parametrize("window", [1, 2, 3, 5, 9, 64])
def test_window_does_not_change_outputs(gpu, window):
    """Rows after the first window are read only for sequences that accept every draft in it;
    every window gives the oracle's outputs, bit for bit the same as reading all rows at once."""
    k = wl.rng(1, wl.S_KSEQ).integers(0, 9, size=40)
    case = wl.verify_mixed(k, vocab=3000)
    t = h.verify_tensors(case, gpu)
    res = kyro_amd.verify_drafts(**t, return_probs=True, window=window)
    h.assert_verify_parity(res, case, h.oracle_verify(case), max_exempt=1)
    ref = kyro_amd.verify_drafts(**t, return_probs=True, window=64)
    assert torch.equal(res.accepted, ref.accepted) and torch.equal(res.tokens, ref.tokens)
    assert torch.equal(torch.nan_to_num(res.p_draft, -1.0), torch.nan_to_num(ref.p_draft, -1.0))


@pytest.mark.parametrize("vocab", [4096, 4097, 5000, 20000, 32768, 50000])
def test_eager_passes_match_the_lazy_passes(gpu, vocab):
    """Every row read at once (window 64: statistics, then resample with the acceptance scan in
    every workgroup, then the draw) against the lazy windows (statistics of the window, decide,
    tail, resample, draw): one chunk, a partial second chunk (4097 also takes the scalar-load
    path), five, eight and thirteen chunks; greedy and sampled sequences with 0 to 8 drafts:
    the outputs are the same bits, and the oracle's."""
    k = wl.rng(vocab, wl.S_KSEQ).integers(0, 9, size=24)
    case = wl.verify_mixed(k, vocab=vocab, seed=vocab)
    t = h.verify_tensors(case, gpu)
    eager = kyro_amd.verify_drafts(**t, return_probs=True, window=64)
    h.assert_verify_parity(eager, case, h.oracle_verify(case), max_exempt=1)
    for window in (1, 3):
        lazy = kyro_amd.verify_drafts(**t, return_probs=True, window=window)
        assert torch.equal(eager.accepted, lazy.accepted) and torch.equal(eager.tokens, lazy.tokens)
        assert torch.equal(torch.nan_to_num(eager.p_draft, -1.0), torch.nan_to_num(lazy.p_draft, -1.0))
        assert torch.equal(torch.nan_to_num(eager.q_draft, -1.0), torch.nan_to_num(lazy.q_draft, -1.0))


def test_tail_pass_with_more_items_than_the_default_grid_holds(gpu):
    """600 sequences that accept every draft (draft logits equal the target's): after a window of
    1 there are 600 x 29 rows x 8 chunks = 139,200 tail items, more than 2048 workgroups x 64 items,
    so the grid grows and every workgroup keeps at most 64. Outputs must equal a single pass over
    all rows bit for bit."""
    g = torch.Generator(device=gpu).manual_seed(3)
    B, kmax, V = 600, 15, 32000
    target = torch.randn((B, kmax + 1, V), generator=g, device=gpu) * 2
    t = dict(target_logits=target, draft_logits=target[:, :kmax].contiguous(),
             draft_tokens=torch.randint(0, V, (B, kmax), generator=g, device=gpu, dtype=torch.int32),
             num_draft=torch.full((B,), kmax, dtype=torch.int32, device=gpu),
             temperature=torch.ones(B, device=gpu),
             u_accept=torch.rand((B, kmax), generator=g, device=gpu),
             u_resample=torch.rand((B,), generator=g, device=gpu))
    res = kyro_amd.verify_drafts(**t, return_probs=True, window=1)
    ref = kyro_amd.verify_drafts(**t, return_probs=True, window=64)
    assert res.accepted.min().item() == kmax
    assert torch.equal(res.accepted, ref.accepted) and torch.equal(res.tokens, ref.tokens)
    assert torch.equal(res.p_draft, ref.p_draft) and torch.equal(res.q_draft, ref.q_draft)


def test_window_all_accepted_reads_bonus_row(gpu):
    """Identical draft and target: every sequence passes the window and its bonus row comes from
    the pass over the remaining rows."""
    case = wl.make_verify_case(batch=12, kmax=6, vocab=4000, target_sigma=2.0, noise_sigma=0.0,
                               temperature=1.0, num_draft=np.arange(12) % 7, seed=5)
    t = h.verify_tensors(case, gpu)
    for window in (1, 2, 6):
        res = kyro_amd.verify_drafts(**t, return_probs=True, window=window)
        assert res.accepted.cpu().tolist() == case.num_draft.tolist()
        h.assert_verify_parity(res, case, h.oracle_verify(case))


def test_full_llama3_8b(gpu):
    case = wl.verify_llama3_8b()
    res = run(case, gpu)
    h.assert_verify_parity(res, case, h.oracle_verify(case), max_exempt=1)
    assert 0 < res.accepted.float().mean().item() < 7


def test_full_skewed(gpu):
    """Acceptance half of the skewed long-context workload (B 32, k 4, V 128256, T 1.0): the
    default window (lazy rows after draft 3) and every row in one pass, both against the oracle."""
    case = wl.verify_skewed()
    orc = h.oracle_verify(case)
    t = h.verify_tensors(case, gpu)
    res = kyro_amd.verify_drafts(**t, return_probs=True)
    h.assert_verify_parity(res, case, orc, max_exempt=1)
    eager = kyro_amd.verify_drafts(**t, return_probs=True, window=64)
    h.assert_verify_parity(eager, case, orc, max_exempt=1)
    assert torch.equal(res.accepted, eager.accepted) and torch.equal(res.tokens, eager.tokens)


def test_full_mixed_llama3_70b(gpu):
    _, k = wl.mixed_llama3_70b()
    case = wl.verify_mixed(k)
    h.assert_verify_parity(run(case, gpu), case, h.oracle_verify(case), max_exempt=1)


def test_first_token_law_is_p0(gpu):
    """Leviathan et al. 2023, Thm 1 on the GPU: with x ~ q the first emitted token follows p."""
    V, N = 8, 120_000
    g = np.random.default_rng(7)
    t_row = np.array([2.0, 0.5, -1.0, 1.5, 0.0, -0.5, 1.0, -2.0], np.float32)
    d_row = np.array([0.0, 2.0, 1.0, -1.0, 0.5, 1.5, -1.0, 0.0], np.float32)
    q = scipy.special.softmax(d_row.astype(np.float64))
    p = scipy.special.softmax(t_row.astype(np.float64))
    x = np.searchsorted(np.cumsum(q), g.random(N)).clip(0, V - 1).astype(np.int32)
    case = wl.VerifyCase(np.broadcast_to(np.stack([t_row, t_row])[None], (N, 2, V)).copy(),
                         np.broadcast_to(d_row[None, None], (N, 1, V)).copy(), x[:, None],
                         np.ones(N, np.int32), np.ones(N, np.float32),
                         g.random((N, 1)).astype(np.float32), g.random(N).astype(np.float32))
    res = run(case, gpu, return_probs=False)
    counts = np.bincount(res.tokens[:, 0].cpu().numpy(), minlength=V)
    assert scipy.stats.chisquare(counts, p * N).pvalue > 1e-4


def test_bad_inputs_raise_and_recover(gpu):
    case = wl.make_verify_case(batch=2, kmax=2, vocab=100, target_sigma=1.0, noise_sigma=1.0,
                               temperature=1.0, seed=1)
    t = h.verify_tensors(case, gpu)
    bad = dict(t)
    bad["num_draft"] = torch.tensor([3, 1], dtype=torch.int32, device=gpu)
    with pytest.raises(kyro_amd.KyroError, match="num_draft"):
        kyro_amd.verify_drafts(**bad)
    bad = dict(t)
    bad["draft_tokens"] = torch.tensor([[5, 100], [1, 2]], dtype=torch.int32, device=gpu)
    with pytest.raises(kyro_amd.KyroError, match="draft, bias or penalty token"):
        kyro_amd.verify_drafts(**bad)
    h.assert_verify_parity(kyro_amd.verify_drafts(**t, return_probs=True), case, h.oracle_verify(case))


def test_rejection_only_b8_matches_golden_fixture(gpu):
    """Committed expected outputs (tests/golden/rejection_b8.json), same exemption rule."""
    import json
    import os

    with open(os.path.join(os.path.dirname(__file__), "golden", "rejection_b8.json")) as f:
        g = json.load(f)
    case = wl.rejection_only_b8()
    res = run(case, gpu)
    fixture = {
        "accepted": np.array(g["accepted"], np.int32),
        "tokens": np.array(g["tokens"], np.uint32),
        "accept_margin": np.array([[np.nan if v is None else v for v in r] for r in g["accept_margin"]]),
        "resample_margin": np.array(g["resample_margin"]),
        "p_draft": np.array([[np.nan if v is None else v for v in r] for r in g["p_draft"]]),
        "q_draft": np.array([[np.nan if v is None else v for v in r] for r in g["q_draft"]]),
    }
    h.assert_verify_parity(res, case, fixture)


def test_verify_step_replays_from_a_graph(gpu):
    """One verify step (attention on the grid schedule, then acceptance with a window of 2 so
    that the decide and tail passes run) captured in a HIP graph after eager calls on the same
    stream: every replay, with an eager step of another shape and synchronisations in between,
    gives the eager outputs bit for bit, and those match the oracle."""
    acase = wl.make_attention_case(context_lens=[1500, 300, 2048, 977, 64, 1024, 1800, 512], q_lens=[8] * 8,
                                   num_heads=32, num_kv_heads=8, dtype="bf16", seed=51)
    vcase = wl.make_verify_case(batch=8, kmax=7, vocab=32000, target_sigma=2.5, noise_sigma=0.4,
                                temperature=0.8, num_draft=np.array([7, 7, 3, 0, 7, 5, 7, 7]), seed=52)
    other_v = wl.make_verify_case(batch=3, kmax=4, vocab=5000, target_sigma=2.0, noise_sigma=0.8,
                                  temperature=1.0, num_draft=np.array([4, 2, 4]), seed=53)
    ta = h.attention_tensors(acase, gpu)
    tv = h.verify_tensors(vcase, gpu)
    to = h.verify_tensors(other_v, gpu)
    attn = kyro_amd.PagedAttention(16, 32, 128, 8)
    aargs = (ta["query"], ta["key_cache"], ta["value_cache"], ta["block_table"], ta["context_lens"])

    def step(att_out, vout):
        attn.forward_async(*aargs, q_start_loc=ta["q_start_loc"], max_q_len=8, out=att_out)
        return kyro_amd.speculative.verify_drafts_async(**tv, window=2, out=vout)

    s = torch.cuda.Stream(gpu)
    with torch.cuda.stream(s):
        att_e = torch.empty(ta["query"].shape, dtype=torch.float32, device=gpu)
        v_e = step(att_e, None)
        other_e = kyro_amd.speculative.verify_drafts_async(**to, window=1)
        att_g = torch.empty_like(att_e)
        v_out = (torch.empty_like(v_e.accepted), torch.empty_like(v_e.tokens))
    torch.cuda.synchronize()
    h.assert_attention_close(att_e, acase, h.oracle_attention(acase), h.ATOL_BF16)
    h.assert_verify_parity(v_e, vcase, h.oracle_verify(vcase), max_exempt=1)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        step(att_g, v_out)
    for _ in range(3):
        att_g.zero_()
        v_out[0].zero_()
        v_out[1].zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(att_g, att_e)
        assert torch.equal(v_out[0], v_e.accepted) and torch.equal(v_out[1], v_e.tokens)
        with torch.cuda.stream(s):
            again = kyro_amd.speculative.verify_drafts_async(**to, window=1)
        torch.cuda.synchronize()
        assert torch.equal(again.accepted, other_e.accepted) and torch.equal(again.tokens, other_e.tokens)
