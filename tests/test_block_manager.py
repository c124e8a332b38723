"""Block manager and prefix cache (host C++ through the C ABI), without a GPU.

First the reference's own unit tests (src/scheduler/block_manager.rs:156-230,
src/scheduler/radix_cache.rs:158-236), then model-based checks over random request streams:
an independent simulation of what every block holds (the prompt tokens written into it, block
copies for copy-on-write) must show every live request its own tokens through its block list;
the cached-token count must equal the longest common prefix with any prompt handed to the cache
(while nothing is evicted); and reference counts must always equal the holders (kyro_bm_check).
"""
import numpy as np
import pytest

import kyro_amd
from kyro_amd import BlockManager, RadixCache


# ---------------------------------------------------------- block_manager.rs tests


def make_manager(gpu_blocks):
    return BlockManager(4, gpu_blocks, 2)


def test_allocate_with_prefix_no_cache():
    bm = make_manager(10)
    blocks, cached = bm.allocate_with_prefix(1, [1, 2, 3, 4, 5])
    assert len(blocks) == 2  # 5 tokens, block_size 4
    assert cached == 0
    assert bm.num_free_blocks == 10 - 2


def test_allocate_with_prefix_full_cache_hit():
    bm = make_manager(10)
    tokens = [1, 2, 3, 4]
    bm.allocate_with_prefix(1, tokens)
    bm.free(1)
    blocks, cached = bm.allocate_with_prefix(2, tokens)
    assert blocks
    assert cached == 4


def test_allocate_with_prefix_partial_cache_hit():
    bm = make_manager(10)
    bm.allocate_with_prefix(1, [1, 2])
    bm.free(1)
    _, cached = bm.allocate_with_prefix(2, [1, 2, 3, 4, 5])
    assert cached == 2
    # the partially matched block is copied, not shared
    (src, dst), = bm.take_copies()
    assert src != dst and bm.block_table[2][0] == dst
    bm.check()


def test_oom_returns_none():
    bm = make_manager(1)
    assert bm.allocate_with_prefix(1, [1, 2, 3, 4, 5]) is None
    bm.check()


def test_free_reuses_blocks():
    bm = make_manager(10)
    bm.allocate_with_prefix(1, [1, 2, 3, 4])
    free_before = bm.num_free_blocks
    bm.free(1)
    assert bm.num_free_blocks == free_before  # blocks go to the cache, not the free pool
    assert bm.num_cached_blocks > 0


def test_multiple_requests_unique_block_tables():
    bm = make_manager(20)
    bm.allocate_with_prefix(1, [1, 2, 3, 4])
    bm.allocate_with_prefix(2, [5, 6, 7, 8])
    assert 1 in bm.block_table and 2 in bm.block_table
    assert bm.block_table[1] != bm.block_table[2]


# ------------------------------------------------------------ radix_cache.rs tests


def test_empty_cache_no_match():
    cache = RadixCache(100, block_size=4)
    assert cache.match_prefix([1, 2, 3]) == ([], 0)


def test_insert_and_match_full():
    cache = RadixCache(100, block_size=4)
    cache.insert([1, 2, 3, 4, 5], [10, 11])
    assert cache.num_cached_blocks == 2
    assert cache.match_prefix([1, 2, 3, 4, 5]) == ([10, 11], 5)


def test_insert_and_match_partial():
    cache = RadixCache(100, block_size=4)
    cache.insert([1, 2, 3], [10])
    assert cache.match_prefix([1, 2, 3, 4, 5]) == ([10], 3)


def test_no_match_on_different_prefix():
    cache = RadixCache(100, block_size=4)
    cache.insert([5, 6, 7], [10])
    assert cache.match_prefix([1, 2, 3]) == ([], 0)


def test_insert_multiple_sequences():
    cache = RadixCache(100, block_size=4)
    cache.insert([1, 2, 3], [10])
    cache.insert([4, 5, 6], [11])
    assert cache.num_cached_blocks == 2
    assert cache.match_prefix([1, 2, 3])[0] == [10]
    assert cache.match_prefix([4, 5, 6])[0] == [11]


def test_evict_lru_when_over_capacity():
    cache = RadixCache(1, block_size=4)
    cache.insert([1, 2, 3], [10])
    cache.insert([4, 5, 6], [11])
    assert cache.num_cached_blocks == 1


def test_lru_evicts_oldest():
    cache = RadixCache(1, block_size=4)
    cache.insert([1, 2], [10])
    cache.match_prefix([1, 2])
    cache.insert([3, 4], [11])
    assert cache.num_cached_blocks <= 1
    # least recently used goes first: [3, 4] is newer than the touch of [1, 2]
    assert cache.match_prefix([3, 4]) == ([11], 2)


# ------------------------------------------------------- behaviour beyond the reference


def test_match_returns_each_block_once():
    """The reference stores every block of the sequence in the suffix node, so a match through
    two nodes returns block 10 twice (radix_cache.rs:95); here each block appears once."""
    cache = RadixCache(100, block_size=4)
    cache.insert([1, 2, 3, 4], [10])
    cache.insert([1, 2, 3, 4, 5, 6], [10, 12])
    assert cache.match_prefix([1, 2, 3, 4, 5, 6]) == ([10, 12], 6)


def test_evicted_blocks_return_to_the_pool():
    bm = BlockManager(4, 6, 0)  # cache budget 2 blocks
    for rid in range(4):
        assert bm.allocate_with_prefix(rid, [rid * 10 + i for i in range(8)]) is not None
        bm.free(rid)
        bm.check()
    assert bm.num_cached_blocks <= 2
    assert bm.num_free_blocks + bm.num_cached_blocks == 6


def test_allocation_evicts_until_it_fits():
    bm = BlockManager(4, 9, 0)  # cache budget 3
    bm.allocate_with_prefix(1, list(range(12)))
    bm.free(1)
    assert bm.num_cached_blocks == 3 and bm.num_free_blocks == 6
    assert bm.allocate_with_prefix(2, list(range(100, 136))) is not None  # needs all 9
    assert bm.num_cached_blocks == 0
    bm.check()


def test_append_and_truncate_follow_the_token_count():
    bm = BlockManager(4, 10, 0)
    bm.allocate_with_prefix(1, [1, 2, 3, 4, 5])
    assert len(bm.block_table[1]) == 2
    assert bm.append_slots(1, 8)  # 13 tokens
    assert bm.request(1) == (bm.block_table[1], 13) and len(bm.block_table[1]) == 4
    bm.truncate(1, 6)
    assert len(bm.block_table[1]) == 2 and bm.request(1)[1] == 6
    with pytest.raises(kyro_amd.KyroError):
        bm.truncate(1, 4)  # below the prompt
    assert not bm.append_slots(1, 100)  # does not fit: False, nothing changes
    assert bm.request(1)[1] == 6
    bm.check()


def test_unknown_and_duplicate_requests_are_errors():
    bm = BlockManager(4, 10, 0)
    bm.allocate_with_prefix(1, [1])
    with pytest.raises(kyro_amd.KyroError):
        bm.allocate_with_prefix(1, [2])
    with pytest.raises(kyro_amd.KyroError):
        bm.free(7)
    with pytest.raises(kyro_amd.KyroError):
        bm.append_slots(7, 1)


# ------------------------------------------------------------ model-based checks


class Model:
    """What each block would hold if every request wrote its own tokens, independent of the
    manager's bookkeeping: content[block][slot] = token id."""

    def __init__(self, bm):
        self.bm = bm
        self.content = {}
        self.live = {}        # rid -> token list (prompt + appended)
        self.prompt_len = {}  # rid -> prompt length
        self.cached_prompts = []

    def write(self, rid, start):
        toks = self.live[rid]
        blocks = self.bm.block_table[rid]
        bs = self.bm.block_size
        for p in range(start, len(toks)):
            self.content.setdefault(blocks[p // bs], [None] * bs)[p % bs] = toks[p]

    def apply_copies(self):
        for src, dst in self.bm.take_copies():
            self.content[dst] = list(self.content.get(src, [None] * self.bm.block_size))

    def verify_all(self):
        bs = self.bm.block_size
        for rid, toks in self.live.items():
            blocks, n = self.bm.request(rid)
            assert n == len(toks) and len(blocks) == -(-n // bs)
            seen = [self.content.get(blocks[p // bs], [None] * bs)[p % bs] for p in range(n)]
            assert seen == toks, f"request {rid} reads {seen} for {toks}"


def lcp(a, b):
    n = 0
    for x, y in zip(a, b):
        if x != y:
            break
        n += 1
    return n


@pytest.mark.parametrize("seed", range(8))
def test_random_streams_keep_every_request_consistent(seed):
    rng = np.random.default_rng(seed)
    bs = int(rng.choice([1, 2, 4, 16]))
    roomy = seed % 2 == 0  # a roomy pool never evicts: cached counts are exact longest prefixes
    bm = BlockManager(bs, 60000 if roomy else 48, 0)
    m = Model(bm)
    stems = [[int(x) for x in rng.integers(0, 4, size=int(rng.integers(1, 40)))] for _ in range(6)]
    next_id = 0
    for _ in range(300):
        op = rng.random()
        if op < 0.45 or not m.live:
            stem = stems[int(rng.integers(len(stems)))]
            toks = stem[: int(rng.integers(0, len(stem) + 1))] + [int(x) for x in rng.integers(0, 4, size=int(rng.integers(0, 20)))]
            expect = max([lcp(toks, p) for p in m.cached_prompts], default=0)
            res = bm.allocate_with_prefix(next_id, toks)
            if res is None:
                assert not roomy
                assert next_id not in bm.block_table
            else:
                blocks, cached = res
                assert len(blocks) == -(-len(toks) // bs)
                assert cached == expect if roomy else cached <= expect
                m.live[next_id] = list(toks)
                m.prompt_len[next_id] = len(toks)
                m.apply_copies()
                m.write(next_id, cached)  # the request computes only its uncached tokens
            next_id += 1
        elif op < 0.65:
            rid = int(rng.choice(list(m.live)))
            n = int(rng.integers(1, 2 * bs + 2))
            if bm.append_slots(rid, n):
                old = len(m.live[rid])
                m.live[rid] += [int(x) for x in rng.integers(4, 8, size=n)]
                m.write(rid, old)
        elif op < 0.75:
            rid = int(rng.choice(list(m.live)))
            lo, hi = m.prompt_len[rid], len(m.live[rid])
            if rng.random() < 0.2 and lo > 0:
                with pytest.raises(kyro_amd.KyroError):
                    bm.truncate(rid, lo - 1)
            else:
                keep = int(rng.integers(lo, hi + 1))
                bm.truncate(rid, keep)
                m.live[rid] = m.live[rid][:keep]
        else:
            rid = int(rng.choice(list(m.live)))
            cache = bool(rng.random() < 0.8)
            toks = m.live.pop(rid)
            bm.free(rid, cache_prompt=cache)
            if cache and m.prompt_len[rid]:
                m.cached_prompts.append(toks[: m.prompt_len[rid]])
        bm.check()
        m.verify_all()
    for rid in list(m.live):
        bm.free(rid)
    bm.check()
    assert bm.num_free_blocks + bm.num_cached_blocks == bm.num_gpu_blocks
