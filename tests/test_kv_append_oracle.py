"""The paged-KV-append oracle (oracle_kv_append) pinned without the GPU.

Reference behaviour (src/model/kv_cache.rs:49-75, tests :148-176): appending 2 then 3 rows
makes the context 2 then 5 with the rows in order, and appended ones read back as ones. The
oracle is also checked against torch's float32 -> bfloat16 conversion, against a gather of the
written positions through the block table (new rows there, every other slot untouched), and
against attention: appending then attending over the paged cache equals attention over the
contiguous old + new K/V.
"""
import numpy as np
import pytest
import torch

import oracle


def bf16_bits(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def gather(cache, table_row, ctx, bs):
    """Token rows 0..ctx-1 of one sequence: [ctx, Hkv, D]."""
    pos = np.arange(ctx)
    return cache[table_row[pos // bs], :, pos % bs, :]


def test_reference_append_increases_context_in_order():
    """kv_cache.rs:148-162: append 2 rows (ctx 2), then 3 more (ctx 5); the cache holds the
    concatenation, as Tensor::cat along the sequence dim (:57-70)."""
    rng = np.random.default_rng(0)
    bs, hkv, d = 4, 4, 64
    kc = np.zeros((6, hkv, bs, d), np.float32)
    vc = np.zeros_like(kc)
    table = np.array([[3, 1, 5]], np.int64)
    k1, v1 = rng.standard_normal((2, 2, hkv, d), dtype=np.float32)
    k2, v2 = rng.standard_normal((2, 3, hkv, d), dtype=np.float32)
    assert oracle.kv_append(k1, v1, kc, vc, table, [2], block_size=bs, q_start_loc=[0, 2]) == 0
    assert oracle.kv_append(k2, v2, kc, vc, table, [5], block_size=bs, q_start_loc=[0, 3]) == 0
    np.testing.assert_array_equal(gather(kc, table[0], 5, bs), np.concatenate([k1, k2]))
    np.testing.assert_array_equal(gather(vc, table[0], 5, bs), np.concatenate([v1, v2]))
    assert not kc[[0, 2, 4]].any()  # blocks outside the table untouched


def test_reference_ones_are_cached():
    """kv_cache.rs:164-176: appended ones read back as ones (bf16 cache from f32 rows)."""
    kc = np.zeros((2, 4, 16, 64), np.uint16)
    vc = np.zeros_like(kc)
    ones = np.ones((1, 4, 64), np.float32)
    assert oracle.kv_append(ones, ones, kc, vc, np.array([[1]]), [1], block_size=16) == 0
    assert (kc[1, :, 0, :] == 0x3F80).all() and (vc[1, :, 0, :] == 0x3F80).all()
    assert not kc[0].any() and not kc[1, :, 1:].any()


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * 10.0 ** rng.integers(-40, 38, 4000),
        np.array([0.0, -0.0, np.inf, -np.inf, 3.4028235e38, -3.4028235e38, 1e-45, 1e-40,
                  1.00390625, 1.01171875, -1.00390625, 65504.0], np.float32),
        # every tie pattern: low half exactly 0x8000 with even and odd kept bits
        (np.arange(0x3F800000, 0x3F800000 + 64 * 0x10000, 0x10000, dtype=np.uint32) | 0x8000).view(np.float32),
    ]).astype(np.float32)
    x = x[: (x.size // 64) * 64].reshape(-1, 1, 64)
    kc = np.zeros((x.shape[0], 1, 1, 64), np.uint16)
    vc = np.zeros_like(kc)
    table = np.arange(x.shape[0], dtype=np.int64)[:, None]
    assert oracle.kv_append(x, x, kc, vc, table, np.ones(x.shape[0]), block_size=1) == 0
    np.testing.assert_array_equal(kc.reshape(-1), bf16_bits(x.reshape(-1)))


def test_bf16_nan_is_canonical():
    x = np.full((1, 1, 8), np.nan, np.float32)
    x[0, 0, 1] = -np.nan
    x.view(np.uint32)[0, 0, 2] = 0x7F800001
    kc = np.zeros((1, 1, 1, 8), np.uint16)
    vc = np.zeros_like(kc)
    assert oracle.kv_append(x, x, kc, vc, np.array([[0]]), [1], block_size=1) == 0
    assert (kc == 0x7FC0).all()


@pytest.mark.parametrize("src,cache", [("f32", "f32"), ("f32", "bf16"), ("bf16", "bf16"), ("bf16", "f32")])
def test_written_slots_hold_new_rows_and_the_rest_is_untouched(src, cache):
    rng = np.random.default_rng(2)
    B, hkv, d, bs, nb, mb = 5, 2, 64, 8, 40, 6
    qlen = np.array([3, 0, 8, 1, 9])
    ctx = np.array([20, 7, 16, 1, 48])
    q_start = np.concatenate([[0], np.cumsum(qlen)]).astype(np.int32)
    table = rng.permutation(nb)[: B * mb].reshape(B, mb).astype(np.int64)
    rows = rng.standard_normal((2, int(qlen.sum()), hkv, d), dtype=np.float32)
    if src == "bf16":
        rows = bf16_bits(rows)
    init = rng.standard_normal((2, nb, hkv, bs, d), dtype=np.float32)
    caches = bf16_bits(init) if cache == "bf16" else init.copy()
    before = caches.copy()
    kc, vc = caches[0], caches[1]
    assert oracle.kv_append(rows[0], rows[1], kc, vc, table, ctx, block_size=bs, q_start_loc=q_start) == 0
    written = np.zeros((nb, bs), bool)
    for b in range(B):
        for j in range(qlen[b]):
            p = ctx[b] - qlen[b] + j
            blk, slot = table[b, p // bs], p % bs
            written[blk, slot] = True
            for c, r in ((kc, rows[0]), (vc, rows[1])):
                got = c[blk, :, slot, :]
                new = r[q_start[b] + j]
                if src == cache:
                    np.testing.assert_array_equal(got, new)
                elif cache == "bf16":
                    np.testing.assert_array_equal(got, bf16_bits(new))
                else:  # bf16 rows widen exactly
                    np.testing.assert_array_equal(got, (new.astype(np.uint32) << 16).view(np.float32))
    keep = ~written[None, :, None, :, None].repeat(2, 0).repeat(hkv, 2).repeat(d, 4)
    np.testing.assert_array_equal(caches[keep], before[keep])


def test_append_then_attention_equals_contiguous_attention():
    rng = np.random.default_rng(3)
    B, H, hkv, d, bs = 3, 8, 2, 64, 16
    old = np.array([30, 0, 47])
    qlen = np.array([4, 5, 1])
    ctx = old + qlen
    mb = 4
    nb = B * mb
    table = rng.permutation(nb).reshape(B, mb).astype(np.int64)
    kc = rng.standard_normal((nb, hkv, bs, d), dtype=np.float32)
    vc = rng.standard_normal((nb, hkv, bs, d), dtype=np.float32)
    q_start = np.concatenate([[0], np.cumsum(qlen)]).astype(np.int32)
    kn, vn = rng.standard_normal((2, int(qlen.sum()), hkv, d), dtype=np.float32)
    q = rng.standard_normal((int(qlen.sum()), H, d), dtype=np.float32)
    # contiguous reference: old rows gathered from the paged cache, then the new rows
    cont_k = np.zeros((nb, hkv, bs, d), np.float32)
    cont_v = np.zeros_like(cont_k)
    cont_table = np.arange(nb).reshape(B, mb)
    for b in range(B):
        kk = np.concatenate([gather(kc, table[b], old[b], bs), kn[q_start[b]:q_start[b + 1]]])
        vv = np.concatenate([gather(vc, table[b], old[b], bs), vn[q_start[b]:q_start[b + 1]]])
        for t in range(ctx[b]):
            cont_k[cont_table[b, t // bs], :, t % bs] = kk[t]
            cont_v[cont_table[b, t // bs], :, t % bs] = vv[t]
    expect = oracle.paged_attention_mq(q, cont_k, cont_v, cont_table, ctx, num_heads=H, num_kv_heads=hkv,
                                       head_dim=d, block_size=bs, q_start_loc=q_start)
    assert oracle.kv_append(kn, vn, kc, vc, table, ctx, block_size=bs, q_start_loc=q_start) == 0
    got = oracle.paged_attention_mq(q, kc, vc, table, ctx, num_heads=H, num_kv_heads=hkv, head_dim=d,
                                    block_size=bs, q_start_loc=q_start)
    np.testing.assert_allclose(got, expect, rtol=0, atol=1e-12)


def test_bad_inputs_are_rejected_and_skip_only_that_sequence():
    rng = np.random.default_rng(4)
    kc = np.zeros((4, 1, 4, 8), np.float32)
    vc = np.zeros_like(kc)
    rows = rng.standard_normal((2, 3, 1, 8), dtype=np.float32)
    table = np.array([[0, 1], [2, 9]], np.int64)  # 9 is out of range
    # sequence 1 writes position 4 -> block table[1][1] = 9: rejected; sequence 0 still written
    assert oracle.kv_append(rows[0], rows[1], kc, vc, table, [2, 5], block_size=4, q_start_loc=[0, 2, 3]) == 1
    np.testing.assert_array_equal(kc[0, 0, :2], rows[0][:2, 0])
    assert not kc[2:].any()
    # context shorter than the new rows
    kc[:] = 0
    assert oracle.kv_append(rows[0], rows[1], kc, vc, table, [1, 1], block_size=4, q_start_loc=[0, 2, 3]) == 1
    assert not kc[:2].any()
