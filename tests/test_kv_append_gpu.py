"""Paged KV append on the GPU against the oracle, through the C ABI (kyro_paged_kv_append).

Byte work, so the bar is bit-exact: every element of both caches equals the oracle's after the
same append (small cases), and at the Llama-3-8B verify-step size the written slots equal the
oracle's rows and no other element changes.
"""
import numpy as np
import pytest
import torch

import kyro_amd
import oracle
from kyro_amd import workloads as wl
from tests import helpers as h

pytestmark = pytest.mark.gpu


def bits(t: torch.Tensor) -> np.ndarray:
    """Host copy with bf16 tensors as their uint16 bit patterns."""
    t = t.cpu()
    return t.view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.bfloat16 else t.numpy()


def make_case(seed, B, hkv, d, bs, qlen, old, src, cache, extra_blocks=3):
    rng = np.random.default_rng(seed)
    qlen = np.asarray(qlen)
    ctx = np.asarray(old) + qlen
    mb = int(max(1, (ctx.max() + bs - 1) // bs))
    nb = B * mb + extra_blocks
    table = rng.permutation(nb)[: B * mb].reshape(B, mb).astype(np.int64)
    q_start = np.concatenate([[0], np.cumsum(qlen)]).astype(np.int32)
    rows = rng.standard_normal((2, int(qlen.sum()), hkv, d), dtype=np.float32) * 3
    caches = rng.standard_normal((2, nb, hkv, bs, d), dtype=np.float32)
    to_bits = lambda x: torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)  # noqa: E731
    if src == "bf16":
        rows = to_bits(rows)
    if cache == "bf16":
        caches = to_bits(caches)
    return dict(rows=rows, caches=caches, table=table, ctx=ctx.astype(np.int64), q_start=q_start, bs=bs,
                hkv=hkv, d=d)


def run_gpu(c, gpu, ragged=True):
    src_bf16 = c["rows"].dtype == np.uint16
    cache_bf16 = c["caches"].dtype == np.uint16
    k = h.to_device(c["rows"][0], gpu, src_bf16)
    v = h.to_device(c["rows"][1], gpu, src_bf16)
    kc = h.to_device(c["caches"][0], gpu, cache_bf16)
    vc = h.to_device(c["caches"][1], gpu, cache_bf16)
    kv = kyro_amd.PagedKVCache(c["bs"], c["hkv"], c["d"])
    kv.append_kv(k, v, kc, vc, h.to_device(c["table"], gpu), h.to_device(c["ctx"], gpu),
                 q_start_loc=h.to_device(c["q_start"], gpu) if ragged else None)
    return bits(kc), bits(vc)


def run_oracle(c, ragged=True):
    kc, vc = c["caches"][0].copy(), c["caches"][1].copy()
    rc = oracle.kv_append(c["rows"][0], c["rows"][1], kc, vc, c["table"], c["ctx"], block_size=c["bs"],
                          q_start_loc=c["q_start"] if ragged else None)
    assert rc == 0
    return kc, vc


@pytest.mark.parametrize("src,cache", [("f32", "f32"), ("f32", "bf16"), ("bf16", "bf16"), ("bf16", "f32")])
@pytest.mark.parametrize("bs,d", [(16, 128), (16, 64), (8, 128), (32, 64)])
def test_matches_oracle_bitwise(gpu, src, cache, bs, d):
    c = make_case(bs * 7 + d, B=6, hkv=4, d=d, bs=bs, qlen=[8, 1, 0, 5, 33, 2], old=[100, 0, 9, 15, 3, 61],
                  src=src, cache=cache)
    gk, gv = run_gpu(c, gpu)
    ok, ov = run_oracle(c)
    np.testing.assert_array_equal(gk, ok)
    np.testing.assert_array_equal(gv, ov)


def test_one_row_per_sequence_without_q_start(gpu):
    c = make_case(11, B=9, hkv=8, d=128, bs=16, qlen=[1] * 9, old=np.arange(9) * 13, src="bf16", cache="bf16")
    gk, gv = run_gpu(c, gpu, ragged=False)
    ok, ov = run_oracle(c, ragged=False)
    np.testing.assert_array_equal(gk, ok)
    np.testing.assert_array_equal(gv, ov)


def test_f32_specials_round_like_the_oracle(gpu):
    c = make_case(12, B=2, hkv=1, d=64, bs=16, qlen=[3, 2], old=[0, 30], src="f32", cache="bf16")
    flat = c["rows"].reshape(-1)
    specials = np.array([np.nan, -np.nan, np.inf, -np.inf, 0.0, -0.0, 3.4028235e38, 1e-40, 1.00390625,
                         1.01171875, 65504.0, -1e-45], np.float32)
    flat[: specials.size] = specials
    flat.view(np.uint32)[specials.size] = 0x7F800001  # signalling NaN
    gk, gv = run_gpu(c, gpu)
    ok, ov = run_oracle(c)
    np.testing.assert_array_equal(gk, ok)
    np.testing.assert_array_equal(gv, ov)


def test_llama3_8b_verify_step_size(gpu):
    """B 64, 8 new rows each after 4088 cached tokens, Hkv 8, D 128, bf16 rows into a bf16 cache of
    16384 permuted blocks: written slots equal the oracle's rows, nothing else changes."""
    case = wl.gqa_llama3_8b()
    B, hkv, d, bs = case.batch, case.num_kv_heads, case.head_dim, case.block_size
    q_start = case.q_start_loc.astype(np.int32)
    total = int(q_start[-1])
    g = torch.Generator(device=gpu).manual_seed(5)
    k = torch.randn((total, hkv, d), generator=g, device=gpu).to(torch.bfloat16)
    v = torch.randn((total, hkv, d), generator=g, device=gpu).to(torch.bfloat16)
    kc = h.to_device(case.key_cache, gpu, True)
    vc = h.to_device(case.value_cache, gpu, True)
    before_k, before_v = kc.clone(), vc.clone()
    table = h.to_device(case.block_table, gpu)
    ctx = h.to_device(case.context_lens, gpu)
    kyro_amd.PagedKVCache(bs, hkv, d).append_kv(k, v, kc, vc, table, ctx, q_start_loc=h.to_device(q_start, gpu))
    # where each new row must land
    blk = np.empty(total, np.int64)
    slot = np.empty(total, np.int64)
    for b in range(B):
        n = q_start[b + 1] - q_start[b]
        pos = case.context_lens[b] - n + np.arange(n)
        blk[q_start[b]:q_start[b + 1]] = case.block_table[b, pos // bs]
        slot[q_start[b]:q_start[b + 1]] = pos % bs
    # expected rows: the oracle appending every row as its own one-token sequence
    rows_k, rows_v = bits(k), bits(v)
    ek = np.zeros((total, hkv, 1, d), np.uint16)
    ev = np.zeros_like(ek)
    assert oracle.kv_append(rows_k, rows_v, ek, ev, np.arange(total)[:, None], np.ones(total), block_size=1) == 0
    bt, st = torch.from_numpy(blk).to(gpu), torch.from_numpy(slot).to(gpu)
    np.testing.assert_array_equal(bits(kc[bt, :, st, :]), ek[:, :, 0, :])
    np.testing.assert_array_equal(bits(vc[bt, :, st, :]), ev[:, :, 0, :])
    for after, before in ((kc, before_k), (vc, before_v)):
        changed = (after.view(torch.int16) != before.view(torch.int16)).any(dim=3).any(dim=1)  # [nb, bs]
        allowed = torch.zeros_like(changed)
        allowed[bt, st] = True
        assert not (changed & ~allowed).any().item()


def test_append_then_attention_matches_oracle(gpu):
    """The write and the attention that reads it, queued back to back on one stream."""
    rng = np.random.default_rng(21)
    B, H, hkv, d, bs = 4, 32, 8, 128, 16
    old = np.array([500, 17, 0, 1023])
    qlen = np.array([8, 8, 3, 8])
    c = make_case(22, B=B, hkv=hkv, d=d, bs=bs, qlen=qlen, old=old, src="bf16", cache="bf16")
    q = torch.from_numpy(rng.standard_normal((int(qlen.sum()), H, d), dtype=np.float32)).to(torch.bfloat16)
    qg = q.to(gpu)
    kc = h.to_device(c["caches"][0], gpu, True)
    vc = h.to_device(c["caches"][1], gpu, True)
    table, ctx = h.to_device(c["table"], gpu), h.to_device(c["ctx"], gpu)
    qs = h.to_device(c["q_start"], gpu)
    kyro_amd.PagedKVCache(bs, hkv, d).append_kv_async(h.to_device(c["rows"][0], gpu, True),
                                                      h.to_device(c["rows"][1], gpu, True), kc, vc, table, ctx,
                                                      q_start_loc=qs)
    out = kyro_amd.PagedAttention(bs, H, d, hkv).forward(qg, kc, vc, table, ctx, q_start_loc=qs)
    ok, ov = run_oracle(c)
    expect = oracle.paged_attention_mq(q.view(torch.int16).numpy().view(np.uint16), ok, ov, c["table"], c["ctx"],
                                       num_heads=H, num_kv_heads=hkv, head_dim=d, block_size=bs,
                                       q_start_loc=c["q_start"])
    err = float(np.max(np.abs(out.float().cpu().numpy() - expect)))
    assert err <= h.ATOL_BF16, err


def test_bad_inputs_raise_and_recover(gpu):
    c = make_case(31, B=3, hkv=2, d=64, bs=16, qlen=[2, 3, 1], old=[10, 20, 30], src="f32", cache="f32")
    kv = kyro_amd.PagedKVCache(16, 2, 64)
    k, v = h.to_device(c["rows"][0], gpu), h.to_device(c["rows"][1], gpu)
    kc, vc = h.to_device(c["caches"][0], gpu), h.to_device(c["caches"][1], gpu)
    qs = h.to_device(c["q_start"], gpu)
    bad_table = c["table"].copy()
    bad_table[1, 1] = 10_000
    with pytest.raises(kyro_amd.KyroError, match="block_table"):
        kv.append_kv(k, v, kc, vc, h.to_device(bad_table, gpu), h.to_device(c["ctx"], gpu), q_start_loc=qs)
    with pytest.raises(kyro_amd.KyroError, match="context length"):
        kv.append_kv(k, v, kc, vc, h.to_device(c["table"], gpu), h.to_device(np.array([1, 23, 31]), gpu),
                     q_start_loc=qs)
    with pytest.raises(kyro_amd.KyroError, match="q_start_loc"):
        kv.append_kv(k, v, kc, vc, h.to_device(c["table"], gpu), h.to_device(c["ctx"], gpu),
                     q_start_loc=h.to_device(np.array([0, 4, 3, 6], np.int32), gpu), max_q_len=3)
    gk, gv = run_gpu(c, gpu)
    ok, ov = run_oracle(c)
    np.testing.assert_array_equal(gk, ok)
    np.testing.assert_array_equal(gv, ov)
