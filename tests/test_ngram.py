"""N-gram table (host C++ through the C ABI) and the drafting oracle, without a GPU.

The reference's test (src/speculative.rs:406-415) plus definitional checks: every window's prefix
is a key, each key maps to the token after its last occurrence (found by a direct scan), the
library's table answers exactly like the oracle's dict, and drafting follows the chain of
lookups and stops at the first miss, at the lookahead, or while the context is shorter than
the order.
"""
import numpy as np
import pytest

import kyro_amd
import oracle


def test_reference_ngram_table_building():
    t = kyro_amd.NgramTable([[1, 2, 3, 4, 5]], 2)
    assert t.get([1]) == 2 and t.get([2]) == 3 and t.get([3]) == 4
    assert t.get([5]) is None
    assert oracle.ngram_build([[1, 2, 3, 4, 5]], 2) == {(1,): 2, (2,): 3, (3,): 4, (4,): 5}


def last_next(corpus, key):
    """Token after the last occurrence of key, scanning the corpus in order."""
    n = len(key)
    found = None
    for seq in corpus:
        for i in range(len(seq) - n):
            if tuple(seq[i:i + n]) == key:
                found = seq[i + n]
    return found


@pytest.mark.parametrize("order", [2, 3, 5])
def test_table_matches_definition_and_oracle(order):
    rng = np.random.default_rng(order)
    corpus = [list(rng.integers(0, 6, size=int(rng.integers(0, 60)))) for _ in range(30)]
    corpus = [[int(t) for t in s] for s in corpus]
    ref = oracle.ngram_build(corpus, order)
    for seq in corpus:
        if len(seq) >= order:
            for i in range(len(seq) - order + 1):
                assert tuple(seq[i:i + order - 1]) in ref
    for key, nxt in ref.items():
        assert last_next([s for s in corpus if len(s) >= order], key) == nxt
    t = kyro_amd.NgramTable(corpus, order)
    assert len(t) == len(ref)
    for key, nxt in ref.items():
        assert t.get(list(key)) == nxt
    for _ in range(200):
        key = tuple(int(x) for x in rng.integers(0, 7, size=order - 1))
        assert t.get(list(key)) == ref.get(key)


def test_drafting_oracle_semantics():
    table = oracle.ngram_build([[1, 2, 3, 1, 2, 4]], 3)  # (1,2)->4 (last), (2,3)->1, (3,1)->2, (2,4) absent
    assert oracle.ngram_draft(table, [9, 1, 2], 3, 5) == [4]            # (2,4) is a miss
    assert oracle.ngram_draft(table, [2, 3], 3, 5) == []                # shorter than the order
    assert oracle.ngram_draft(table, [0, 2, 3], 3, 2) == [1, 2]         # stops at the lookahead
    assert oracle.ngram_draft(table, [0, 2, 3], 3, 9) == [1, 2, 4]


def test_bad_orders_are_rejected():
    with pytest.raises(kyro_amd.KyroError):
        kyro_amd.NgramTable([[1, 2]], 1)
    with pytest.raises(kyro_amd.KyroError):
        kyro_amd.NgramTable([[1, 2]], 17)
