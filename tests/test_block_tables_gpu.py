"""Device side of the block manager: kyro_bm_write_tables, kyro_copy_blocks, and a serving
simulation in which requests with shared prefixes get their blocks from the manager, copy
partially matched blocks, write only their uncached tokens' K/V (kyro_paged_kv_append), grow by
verify rows and shrink after rejection, and then read back their own K/V through the device
block tables, both by a gather and through paged attention against the oracle on contiguous K/V.
"""
import numpy as np
import pytest
import torch

import kyro_amd
import oracle
from kyro_amd import BlockManager, copy_blocks

pytestmark = pytest.mark.gpu


def test_write_tables_matches_the_host_lists(gpu):
    rng = np.random.default_rng(0)
    bm = BlockManager(16, 5000, 0)
    rids = []
    for rid in range(40):
        n = int(rng.integers(0, 700))
        assert bm.allocate_with_prefix(rid, rng.integers(0, 3, size=n)) is not None
        if rng.random() < 0.3:
            bm.append_slots(rid, int(rng.integers(1, 40)))
        rids.append(rid)
    for rid in rids[::5]:
        bm.free(rid)
    live = [r for r in rids if r in bm.block_table]
    order = list(rng.permutation(live))
    table = torch.full((len(order), 64), -7, dtype=torch.int64, device=gpu)
    lens = torch.full((len(order),), -7, dtype=torch.int64, device=gpu)
    shared = bm.write_tables(order, table, lens)
    torch.cuda.synchronize()
    blocks_of = [bm.request(rid)[0] for rid in order]
    flat = [x for bl in blocks_of for x in bl]
    assert shared == (len(flat) != len(set(flat)))
    # one request alone never shares a block with another
    assert bm.write_tables(order[:1], table[:1]) is False
    for b, rid in enumerate(order):
        blocks, n = bm.request(rid)
        row = table[b].cpu().numpy()
        assert row[: len(blocks)].tolist() == blocks and not row[len(blocks):].any()
        assert lens[b].item() == n
    with pytest.raises(kyro_amd.KyroError, match="max_blocks"):
        bm.write_tables(order, torch.zeros((len(order), 2), dtype=torch.int64, device=gpu))
    with pytest.raises(kyro_amd.KyroError, match="unknown request"):
        bm.write_tables([10_000], torch.zeros((1, 64), dtype=torch.int64, device=gpu))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_copy_blocks_copies_whole_blocks(gpu, dtype):
    g = torch.Generator(device=gpu).manual_seed(1)
    kc = torch.randn((50, 8, 16, 128), generator=g, device=gpu).to(dtype)
    vc = torch.randn((50, 8, 16, 128), generator=g, device=gpu).to(dtype)
    k0, v0 = kc.clone(), vc.clone()
    pairs = [(3, 7), (40, 0), (5, 49), (12, 13)]
    copy_blocks(kc, vc, pairs)
    ek, ev = k0.clone(), v0.clone()
    for s, d in pairs:
        ek[d], ev[d] = k0[s], v0[s]
    assert torch.equal(kc.view(torch.int16) if dtype == torch.bfloat16 else kc,
                       ek.view(torch.int16) if dtype == torch.bfloat16 else ek)
    assert torch.equal(vc.float(), ev.float())
    with pytest.raises(kyro_amd.KyroError, match="both a source and a destination"):
        copy_blocks(kc, vc, [(1, 2), (2, 3)])
    with pytest.raises(kyro_amd.KyroError, match="outside"):
        copy_blocks(kc, vc, [(1, 50)])


def kv_rows(tokens, start, emb, hkv, d):
    """K and V rows of tokens[start:] at their positions: a token's embedding plus its position."""
    pos = np.arange(start, len(tokens), dtype=np.float32)
    k = emb[np.asarray(tokens[start:], dtype=np.int64)] + pos[:, None, None] * 1e-3
    return k.astype(np.float32), (-k).astype(np.float32)


def test_serving_simulation_reads_back_every_requests_kv(gpu):
    rng = np.random.default_rng(2)
    bs, hkv, d, H = 16, 2, 64, 8
    vocab = 7
    emb = rng.standard_normal((vocab, hkv, d), dtype=np.float32)
    nb = 400
    bm = BlockManager(bs, nb, 0)
    kc = torch.zeros((nb, hkv, bs, d), dtype=torch.float32, device=gpu)
    vc = torch.zeros_like(kc)
    kv = kyro_amd.PagedKVCache(bs, hkv, d)
    attn = kyro_amd.PagedAttention(bs, H, d, hkv)
    stems = [[int(x) for x in rng.integers(0, vocab, size=int(rng.integers(20, 90)))] for _ in range(4)]
    live = {}
    next_id = 0

    def append(rid, toks, start):
        k, v = kv_rows(toks, start, emb, hkv, d)
        n = len(toks) - start
        if n == 0:
            return
        table = torch.zeros((1, 32), dtype=torch.int64, device=gpu)
        lens = torch.zeros((1,), dtype=torch.int64, device=gpu)
        bm.write_tables([rid], table, lens)
        kv.append_kv(torch.from_numpy(k).to(gpu), torch.from_numpy(v).to(gpu), kc, vc, table, lens,
                     q_start_loc=torch.tensor([0, n], dtype=torch.int32, device=gpu), max_q_len=n)

    for step in range(60):
        r = rng.random()
        if r < 0.5 or not live:
            stem = stems[int(rng.integers(len(stems)))]
            toks = stem[: int(rng.integers(1, len(stem) + 1))] + [int(x) for x in rng.integers(0, vocab, size=int(rng.integers(0, 30)))]
            res = bm.allocate_with_prefix(next_id, toks)
            if res is not None:
                copy_blocks(kc, vc, bm.take_copies())
                append(next_id, toks, res[1])
                live[next_id] = list(toks)
            next_id += 1
        elif r < 0.8:
            # a verify step: room for k + 1 rows, write them, keep the accepted ones
            rid = int(rng.choice(list(live)))
            k1 = int(rng.integers(1, 9))
            if bm.append_slots(rid, k1):
                old = len(live[rid])
                live[rid] += [int(x) for x in rng.integers(0, vocab, size=k1)]
                append(rid, live[rid], old)
                keep = old + int(rng.integers(1, k1 + 1))
                bm.truncate(rid, keep)
                live[rid] = live[rid][:keep]
        else:
            rid = int(rng.choice(list(live)))
            del live[rid]
            bm.free(rid)
        bm.check()

    rids = sorted(live)
    B = len(rids)
    table = torch.zeros((B, 32), dtype=torch.int64, device=gpu)
    lens = torch.zeros((B,), dtype=torch.int64, device=gpu)
    shared = bm.write_tables(rids, table, lens)
    torch.cuda.synchronize()
    t_host = table.cpu().numpy()
    flat = [x for rid in rids for x in bm.request(rid)[0]]
    assert shared == (len(flat) != len(set(flat)))
    for b, rid in enumerate(rids):
        toks = live[rid]
        n = len(toks)
        assert lens[b].item() == n
        pos = np.arange(n)
        got_k = kc[torch.from_numpy(t_host[b, pos // bs]).to(gpu), :, torch.from_numpy(pos % bs).to(gpu), :]
        ek, ev = kv_rows(toks, 0, emb, hkv, d)
        np.testing.assert_array_equal(got_k.cpu().numpy(), ek)
        got_v = vc[torch.from_numpy(t_host[b, pos // bs]).to(gpu), :, torch.from_numpy(pos % bs).to(gpu), :]
        np.testing.assert_array_equal(got_v.cpu().numpy(), ev)

    # attention of one query per request through the device tables equals attention over the
    # request's own contiguous K/V
    q = rng.standard_normal((B, H, d), dtype=np.float32)
    out = attn.forward(torch.from_numpy(q).to(gpu), kc, vc, table, lens, kv_reuse="shared" if shared else "auto")
    for b, rid in enumerate(rids):
        toks = live[rid]
        n = len(toks)
        ek, ev = kv_rows(toks, 0, emb, hkv, d)
        nbk = -(-n // bs)
        ck = np.zeros((nbk * bs, hkv, d), np.float32)
        cv = np.zeros_like(ck)
        ck[:n], cv[:n] = ek, ev
        ck = ck.reshape(nbk, bs, hkv, d).transpose(0, 2, 1, 3).copy()
        cv = cv.reshape(nbk, bs, hkv, d).transpose(0, 2, 1, 3).copy()
        ref = oracle.paged_attention_mq(q[b:b + 1], ck, cv, np.arange(nbk)[None], np.array([n]), num_heads=H,
                                        num_kv_heads=hkv, head_dim=d, block_size=bs)
        assert np.max(np.abs(out[b].cpu().numpy() - ref[0])) <= 1e-3
