"""The balanced attention schedule's plan on the host (no GPU): the library's own chunk and split
arithmetic (kyro_paged_attention_plan runs the functions the device plan runs) never needs more
partial-state slots than a launch sizes, over seeded random batches.

A launch sizes its workspace from the params alone (plan_slot_bound), before the context lengths
are known; the device plan then latches KYRO_EINVAL instead of running a plan with more items.
An experimental chunk length once ran against a bound derived for another and wrote past the
workspace: test_a_bound_for_another_chunk_length_is_exceeded shows this check catches that
mismatch.
"""
import numpy as np
import pytest

from kyro_amd import workloads as wl
from kyro_amd.attention import PagedAttention, attention_plan, describe_attention


def _ceil(a, b):
    return -(-a // b)


def _rows_per_group(rows_cap, total_rows, seqs):
    """Rows per MFMA row group for bf16 at head_dim 128: one tile, two, the four-tile kernel's
    64, or the five-tile kernel's 80 where that takes fewer row groups (65-80, 129-160 rows) and
    the average unit (total_rows / seqs) holds more than half of what the last 64-row group
    would."""
    if rows_cap <= 16:
        return 16
    if rows_cap <= 32:
        return 32
    lo = 64 * (_ceil(rows_cap, 64) - 1)
    wide = _ceil(rows_cap, 80) < _ceil(rows_cap, 64) and 2 * total_rows > seqs * (rows_cap + lo)
    return 80 if wide else 64


def _random_batch(g):
    """Context lengths from one of four shapes (uniform short, uniform long, log-uniform over
    128..32768, mostly short with a few very long), ragged row counts 0..9, and a head shape."""
    B = int(g.choice([1, 2, 7, 31, 64, 128, 256, 300, 1024]))
    kind = int(g.integers(0, 4))
    if kind == 0:
        ctx = g.integers(0, 600, size=B)
    elif kind == 1:
        ctx = g.integers(256, 8193, size=B)
    elif kind == 2:
        ctx = np.round(np.exp(np.log(128) + g.random(B) * (np.log(32768) - np.log(128)))).astype(np.int64)
    else:
        ctx = g.integers(1, 400, size=B)
        ctx[g.random(B) < 0.05] = int(g.integers(8000, 32769))
    ql = g.integers(0, 10, size=B) if g.random() < 0.7 else np.full(B, int(g.integers(1, 10)))
    hkv = int(g.choice([1, 2, 4, 8, 16]))
    group = int(g.choice([1, 2, 4, 8]))
    return ctx.astype(np.int64), ql.astype(np.int32), hkv, group


@pytest.mark.parametrize("chunk_quarters", [0, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("num_cus", [256, 80, 32])
def test_slot_bound_holds_over_random_batches(chunk_quarters, num_cus):
    g = np.random.default_rng(1000 * chunk_quarters + num_cus)
    worst = 0.0
    for _ in range(400):
        ctx, ql, hkv, group = _random_batch(g)
        attn = PagedAttention(16, hkv * group, 128, hkv)
        mb = max(1, int(_ceil(ctx.max(), 16)) + int(g.integers(0, 3)))
        info, splits = attention_plan(attn, ctx, ql, max_blocks_per_seq=mb, num_cus=num_cus,
                                      chunk_quarters=chunk_quarters)
        if ql.sum() == 0:  # no query rows: nothing is launched
            assert info["items"] == 0 and info["grid"] == 0
            continue
        assert info["grid"] == max(8, num_cus // 8 * 8)
        assert info["items"] <= info["slot_bound"], (info, ctx.tolist(), ql.tolist(), hkv, group)
        worst = max(worst, info["items"] / info["slot_bound"])
        # Items are sequence x kv head group x split x row group, with the row groups of the
        # launch's row-group size (16, 32, 64 or 80 rows per group for the bf16 MFMA kernels;
        # the 64- and 80-row kernels, and the 16-row one under MHA, take one kv head per
        # workgroup).
        rw = _rows_per_group(group * max(1, int(ql.max())), group * int(ql.sum()), len(ctx))
        hp = 2 if hkv % 2 == 0 and rw <= 32 and not (rw <= 16 and group == 1) else 1
        r = _ceil(ql.astype(np.int64) * group, rw)
        assert info["items"] == int(np.sum((hkv // hp) * splits.astype(np.int64) * r))
        # Splits: one for a sequence within the chunk; otherwise chunks of C blocks from the start,
        # the last one shorter and not empty; none for a sequence without rows.
        nb = _ceil(ctx, 16)
        C = info["chunk_blocks"]
        assert C % 2 == 0 and C >= 16
        for b in range(len(ctx)):
            if r[b] == 0:
                assert splits[b] == 0
            elif nb[b] <= C:
                assert splits[b] == 1
            else:
                assert splits[b] == _ceil(nb[b], C) and (splits[b] - 1) * C < nb[b] <= splits[b] * C
    assert worst > 0.0


@pytest.mark.parametrize("heads,max_q_len,total_q,tiles,row_groups", [
    ((32, 8), 8, 32, 2, 1), ((64, 8), 8, 32, 4, 1), ((64, 8), 9, 36, 5, 1), ((64, 8), 9, 35, 5, 1),
    ((64, 8), 9, 34, 4, 2), ((64, 8), 9, 20, 4, 2), ((16, 2), 12, 48, 4, 2), ((32, 2), 9, 36, 5, 2),
    ((32, 2), 10, 40, 5, 2), ((32, 2), 10, 36, 4, 3), ((32, 2), 11, 44, 4, 3), ((64, 8), 16, 64, 4, 2)])
def test_row_group_size_follows_the_rows_per_kv_head(heads, max_q_len, total_q, tiles, row_groups):
    """bf16, head_dim 128, a batch of 4: 16-row tiles per row group for GQA group x max_q_len
    rows per kv head and total_q query rows. Five tiles where they need fewer row groups than
    four (72, 144 and 160 rows) and the average unit holds more than half of the last 64-row
    group's rows (GQA 64/8, max_q_len 9: 35 of 36 rows in all take five tiles, 34 four); four
    otherwise above 32 rows. As the library reports for a launch."""
    H, Hkv = heads
    text = describe_attention(PagedAttention(16, H, 128, Hkv), batch=4, total_q=total_q,
                              max_q_len=max_q_len, max_blocks_per_seq=64, num_blocks=256)
    assert f"row tiles {tiles}," in text and f"row groups {row_groups}," in text, text
    assert _rows_per_group(H // Hkv * max_q_len, H // Hkv * total_q, 4) == 16 * tiles


def test_a_uniform_batch_keeps_one_item_per_kv_head_group():
    """Llama-3-8B verify shape (64 x 4096 tokens, GQA 32/8, 8 rows): nothing splits."""
    info, splits = attention_plan(PagedAttention(16, 32, 128, 8), [4096] * 64, [8] * 64, max_blocks_per_seq=256)
    assert (splits == 1).all() and info["items"] == 64 * 4


def test_a_bound_for_another_chunk_length_is_exceeded():
    """The Llama-2-7B batch's context lengths (B 16, ctx 512-2048, 5 rows) under GQA 32/8, planned
    with chunks of L/2, need more slots than a bound derived for the library's 5L/4 allows: the
    check above has the power to catch a plan/bound mismatch (one once wrote past the workspace),
    and the shared chunk constant keeps them consistent."""
    ctx = wl.rng(0, wl.S_CTX).integers(512, 2049, size=16)
    attn = PagedAttention(16, 32, 128, 8)
    half, _ = attention_plan(attn, ctx, [5] * 16, max_blocks_per_seq=128, chunk_quarters=2)
    lib, _ = attention_plan(attn, ctx, [5] * 16, max_blocks_per_seq=128)
    assert lib["items"] <= lib["slot_bound"]
    assert half["items"] <= half["slot_bound"]
    assert half["items"] > lib["slot_bound"]


def test_grid_schedule_params_are_refused():
    from kyro_amd._lib import KyroError

    with pytest.raises(KyroError, match="grid schedule"):
        attention_plan(PagedAttention(16, 8, 128, 2), [100, 200], None, max_blocks_per_seq=16, schedule="grid")
