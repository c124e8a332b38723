"""N-gram drafting on the GPU (kyro_ngram_draft) against the oracle, and chained into the verify
step: the drafts and counts feed kyro_spec_verify directly."""
import numpy as np
import pytest
import torch

import kyro_amd
import oracle
from kyro_amd import workloads as wl
from tests import helpers as h

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("order", [2, 3, 4, 8])
def test_drafts_match_the_oracle(gpu, order):
    rng = np.random.default_rng(order)
    corpus = [[int(t) for t in rng.integers(0, 5, size=int(rng.integers(5, 200)))] for _ in range(40)]
    table = kyro_amd.NgramTable(corpus, order)
    ref = oracle.ngram_build(corpus, order)
    contexts = []
    for b in range(300):
        if b % 3 == 0:  # a stretch of the corpus: long chains of hits
            s = corpus[b % len(corpus)]
            i = int(rng.integers(0, len(s)))
            contexts.append(s[: i + 1])
        else:
            contexts.append([int(t) for t in rng.integers(0, 5, size=int(rng.integers(0, 12)))])
    tail, lens = kyro_amd.context_tails(contexts, order, gpu)
    toks, nd = table.draft(tail, lens, 7)
    toks, nd = toks.cpu().numpy().view(np.uint32), nd.cpu().numpy()
    for b, c in enumerate(contexts):
        exp = oracle.ngram_draft(ref, c, order, 7)
        assert nd[b] == len(exp), (b, c, exp)
        assert toks[b, : len(exp)].tolist() == exp
        assert (toks[b, len(exp):] == 0xFFFFFFFF).all()


def test_drafts_feed_the_verify_step(gpu):
    """Greedy verification of n-gram drafts against target logits that agree with the corpus for
    the first two positions: accepted = min(num_draft, 2) per sequence."""
    corpus = [[(7 * i + 3) % 50 for i in range(400)]]
    table = kyro_amd.NgramTable(corpus, 3)
    contexts = [corpus[0][: 10 + b] for b in range(16)] + [[1], [49, 48, 47]]
    B, k, V = len(contexts), 5, 51
    tail, lens = kyro_amd.context_tails(contexts, 3, gpu)
    toks, nd = table.draft(tail, lens, k)
    ref = oracle.ngram_build(corpus, 3)
    target = np.zeros((B, k + 1, V), np.float32)
    for b, c in enumerate(contexts):
        exp = oracle.ngram_draft(ref, c, 3, k)
        for i, t in enumerate(exp[:2]):
            target[b, i, t] = 10.0
        for i in range(2, k + 1):
            target[b, i, 50] = 10.0  # disagrees: token 50 is never in the corpus
    res = kyro_amd.verify_drafts(torch.from_numpy(target).to(gpu), None, toks, nd,
                                 torch.zeros(B, device=gpu), torch.full((B, k), 0.5, device=gpu),
                                 torch.full((B,), 0.5, device=gpu))
    n = nd.cpu().numpy()
    assert res.accepted.cpu().numpy().tolist() == [min(int(x), 2) for x in n]
