"""Paged attention on the GPU against the oracle, through the C ABI (kyro_paged_attention_mq).

Mirrors the reference's own tests (src/model/attention_kernel.rs:154-227) and then checks values:
small cases and full-size workloads against the oracle on every sequence, and size-independent
properties (block permutation) at full size.
"""
import ctypes

import numpy as np
import pytest
import torch

import kyro_amd
from kyro_amd import workloads as wl
from kyro_amd.attention import describe_attention
from tests import helpers as h

pytestmark = pytest.mark.gpu


def make_attention(block_size, num_heads, head_dim, num_kv_heads):
    return kyro_amd.PagedAttention(block_size, num_heads, head_dim, num_kv_heads)


# ---------------------------------------------------- the reference's tests, on the GPU


def test_paged_attention_creation():
    attn = make_attention(16, 8, 64, 2)
    assert (attn.block_size, attn.num_heads, attn.head_dim, attn.num_kv_heads) == (16, 8, 64, 2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_paged_attention_zero_context(gpu, dtype):
    attn = make_attention(16, 8, 64, 2)
    out = attn.forward(torch.zeros((1, 8, 64), dtype=dtype, device=gpu),
                       torch.zeros((4, 2, 16, 64), dtype=dtype, device=gpu),
                       torch.zeros((4, 2, 16, 64), dtype=dtype, device=gpu),
                       torch.zeros((1, 4), dtype=torch.int64, device=gpu),
                       torch.zeros((1,), dtype=torch.int64, device=gpu))
    assert tuple(out.shape) == (1, 8, 64)
    assert torch.count_nonzero(out) == 0


@pytest.mark.parametrize("ctx", [8, 24])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_paged_attention_mha_all_ones(gpu, ctx, dtype):
    """Single block (ctx 8) and multi-block over the aliased table [0,0,0,0] (ctx 24)."""
    attn = make_attention(16, 8, 64, 8)
    out = attn.forward(torch.ones((1, 8, 64), dtype=dtype, device=gpu),
                       torch.ones((4, 8, 16, 64), dtype=dtype, device=gpu),
                       torch.ones((4, 8, 16, 64), dtype=dtype, device=gpu),
                       torch.zeros((1, 4), dtype=torch.int64, device=gpu),
                       torch.full((1,), ctx, dtype=torch.int64, device=gpu))
    assert tuple(out.shape) == (1, 8, 64)
    torch.testing.assert_close(out, torch.ones_like(out), atol=1e-6, rtol=0)


# ---------------------------------------------------------------- parity with the oracle

SMALL = [
    # (heads, kv heads, D, ctx lens, q lens)
    ((8, 2), 64, [17, 40, 5, 33, 16, 1], [1, 5, 3, 2, 4, 1]),
    ((4, 4), 128, [100, 16, 48, 3], [5, 5, 5, 3]),
    ((32, 8), 128, [129, 300, 40, 257], [8, 8, 8, 8]),
    ((64, 8), 128, [260, 50, 9, 700], [9, 1, 4, 6]),
    ((8, 1), 128, [33, 77], [1, 2]),
    # up to 64 rows per kv head: one four-tile row group (units of 64, 40, 32 and 16 rows)
    ((16, 2), 128, [100, 33, 700, 16], [8, 5, 4, 2]),
    # 80 rows each: one five-tile row group
    ((32, 2), 128, [300, 47], [5, 5]),
    # up to 80 rows, 56 on average: a 64-row group and a 16-row group
    ((32, 2), 128, [300, 47], [5, 2]),
    # 96 rows: a 64-row group and a 32-row group
    ((32, 2), 128, [300, 47], [6, 2]),
]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("shape", SMALL, ids=lambda s: f"{s[0][0]}x{s[0][1]}d{s[1]}")
@pytest.mark.parametrize("path", ["vector", "mfma", "auto"])
@pytest.mark.parametrize("splits", [1, 3])
def test_small_parity(gpu, dtype, shape, path, splits):
    (H, Hkv), D, ctx, ql = shape
    if path == "mfma" and D != 128 and not (dtype == "bf16" and D in MFMA_HEAD_DIMS):
        pytest.skip("the f32 MFMA kernel takes head_dim 128 only")
    case = wl.make_attention_case(context_lens=ctx, q_lens=ql, num_heads=H, num_kv_heads=Hkv,
                                  head_dim=D, dtype=dtype, seed=21, num_blocks=200)
    t = h.attention_tensors(case, gpu)
    attn = make_attention(16, H, D, Hkv)
    out = attn.forward(t["query"], t["key_cache"], t["value_cache"], t["block_table"],
                       t["context_lens"], q_start_loc=t["q_start_loc"], path=path,
                       num_splits=splits)
    h.assert_attention_close(out, case, h.oracle_attention(case),
                             h.ATOL_BF16 if dtype == "bf16" else h.ATOL_F32)


# Head dims of the reference's models (head_dim = hidden_size / num_attention_heads,
# src/model/llama.rs:35, src/model/qwen.rs:31): every multiple of 8 up to 256 runs, including
# ones that are not multiples of 16 (8 lanes per token row instead of 16).
HEAD_DIMS = [8, 64, 72, 80, 96, 112, 128, 160, 192, 224, 248, 256]


# bf16 head dims the MFMA kernel takes besides 128: every multiple of 32 from 64 to 256, and 80
# and 112 (in the operand layouts of 96 and 128, the last 32-dim step half padding)
MFMA_HEAD_DIMS = (64, 80, 96, 112, 160, 192, 224, 256)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("D", HEAD_DIMS)
@pytest.mark.parametrize("heads", [(8, 2), (4, 4), (32, 4)], ids=["gqa8x2", "mha4", "gqa32x4"])
@pytest.mark.parametrize("splits", [1, 3])
def test_head_dims(gpu, dtype, D, heads, splits):
    """Every path that takes the head dim, against the oracle: AUTO (the MFMA kernel where it
    applies), the vector kernel, and for the MFMA head dims the MFMA kernel on the grid and under
    the balanced schedule. 32/4 heads give 64 rows per kv head (several row groups)."""
    H, Hkv = heads
    case = wl.make_attention_case(context_lens=[70, 5, 33, 130], q_lens=[5, 1, 3, 8], num_heads=H,
                                  num_kv_heads=Hkv, head_dim=D, dtype=dtype, seed=40 + D, num_blocks=64)
    t = h.attention_tensors(case, gpu)
    attn = make_attention(16, H, D, Hkv)
    exp = h.oracle_attention(case)
    runs = [dict(num_splits=splits), dict(num_splits=splits, path="vector")]
    if D == 128 or (dtype == "bf16" and D in MFMA_HEAD_DIMS):
        runs.append(dict(num_splits=splits, path="mfma"))
        if splits == 1:
            runs.append(dict(schedule="balanced"))
    for kw in runs:
        for out_dtype in (torch.float32, torch.bfloat16):
            out = attn.forward(t["query"], t["key_cache"], t["value_cache"], t["block_table"],
                               t["context_lens"], q_start_loc=t["q_start_loc"], out_dtype=out_dtype, **kw)
            atol = h.ATOL_BF16 if dtype == "bf16" or out_dtype == torch.bfloat16 else h.ATOL_F32
            h.assert_attention_close(out, case, exp, atol)


@pytest.mark.parametrize("D", MFMA_HEAD_DIMS)
def test_mfma_head_dims_long_and_uneven(gpu, D):
    """MFMA head dims on long, uneven contexts (balanced schedule with splits, partial last
    blocks, causal rows) and on a uniform GQA 32/8 verify shape, against the oracle."""
    for ctx, ql, heads in (([3000, 17, 900, 5000], [8, 8, 1, 5], (32, 8)), ([1024] * 8, [8] * 8, (32, 8)),
                           ([2000, 333], [5, 5], (16, 16))):
        case = wl.make_attention_case(context_lens=ctx, q_lens=ql, num_heads=heads[0], num_kv_heads=heads[1],
                                      head_dim=D, dtype="bf16", seed=D + len(ctx))
        t = h.attention_tensors(case, gpu)
        attn = make_attention(16, heads[0], D, heads[1])
        exp = h.oracle_attention(case)
        for kw in (dict(), dict(schedule="grid"), dict(schedule="balanced")):
            out = attn.forward(t["query"], t["key_cache"], t["value_cache"], t["block_table"], t["context_lens"],
                               q_start_loc=t["q_start_loc"], out_dtype=torch.bfloat16, **kw)
            h.assert_attention_close(out, case, exp, h.ATOL_BF16)


def test_bf16_output_and_noncausal(gpu):
    case = wl.make_attention_case(context_lens=[90, 31], q_lens=[4, 2], num_heads=16, num_kv_heads=4,
                                  dtype="bf16", seed=8)
    t = h.attention_tensors(case, gpu)
    attn = make_attention(16, 16, 128, 4)
    exp = h.oracle_attention(case, causal=False)
    for path in ("vector", "mfma"):
        out = attn.forward(t["query"], t["key_cache"], t["value_cache"], t["block_table"],
                           t["context_lens"], q_start_loc=t["q_start_loc"], causal=False,
                           out_dtype=torch.bfloat16, path=path)
        assert out.dtype == torch.bfloat16
        h.assert_attention_close(out, case, exp, h.ATOL_BF16)


def test_query_rows_without_visible_keys_are_zero(gpu):
    """q_len > ctx under the causal rule: the first rows see no key and come out zero."""
    case = wl.make_attention_case(context_lens=[3], q_lens=[5], num_heads=4, num_kv_heads=4,
                                  dtype="bf16", seed=2)
    t = h.attention_tensors(case, gpu)
    for path in ("vector", "mfma"):
        out = make_attention(16, 4, 128, 4).forward(
            t["query"], t["key_cache"], t["value_cache"], t["block_table"], t["context_lens"],
            q_start_loc=t["q_start_loc"], path=path)
        assert torch.count_nonzero(out[:2]) == 0
        assert torch.count_nonzero(out[2:]) > 0


def test_repeat_calls_are_bitwise_identical(gpu):
    case = wl.gqa_llama3_8b(batch=4, ctx=1000)
    t = h.attention_tensors(case, gpu)
    attn = make_attention(16, 32, 128, 8)
    outs = [attn.forward(t["query"], t["key_cache"], t["value_cache"], t["block_table"],
                         t["context_lens"], q_start_loc=t["q_start_loc"], num_splits=4)
            for _ in range(3)]
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[1], outs[2])


@pytest.mark.parametrize("q_lens, gqa", [([8] * 4, (32, 8)), ([9] * 4, (64, 8)), ([9, 4, 8, 1], (64, 8)),
                                         ([3] * 4, (6, 3))])
def test_kv_reuse_hint_never_changes_the_result(gpu, q_lens, gqa):
    """The hint only picks the K/V loads' cache policy: 32 rows per kv head (one row group,
    streamed under "auto"), 72 rows (a 64-row and an 8-row group, cached under "auto"), ragged
    72/32/64/8 rows (under "auto" the first sequence cached, the others streamed), and an odd kv
    head count (one kv head per workgroup) with 6 rows; every hint gives the same bits."""
    H, Hkv = gqa
    case = wl.make_attention_case(context_lens=[700, 33, 2048, 16], q_lens=q_lens, num_heads=H,
                                  num_kv_heads=Hkv, shared_prefix_blocks=2, seed=5)
    t = h.attention_tensors(case, gpu)
    attn = make_attention(16, H, 128, Hkv)
    args = (t["query"], t["key_cache"], t["value_cache"], t["block_table"], t["context_lens"])
    outs = {r: attn.forward(*args, q_start_loc=t["q_start_loc"], path="mfma", kv_reuse=r)
            for r in ("auto", "shared", "stream")}
    assert torch.equal(outs["auto"], outs["shared"]) and torch.equal(outs["auto"], outs["stream"])
    h.assert_attention_close(outs["auto"], case, h.oracle_attention(case, [0, 2]), h.ATOL_BF16)
    with pytest.raises(KeyError):
        attn.forward(*args, q_start_loc=t["q_start_loc"], kv_reuse="sometimes")


@pytest.mark.parametrize("dtype, D", [("f32", 128), ("bf16", 128), ("bf16", 80), ("bf16", 112), ("f32", 80)])
def test_cache_slots_past_the_context_are_never_used(gpu, dtype, D):
    """The slots after a sequence's last token in its last block, and every block no table
    references, may hold anything (here NaN in K and V): the rows must still equal the oracle's,
    which reads positions below the context length only (attention_kernel.rs:91-93,119-120).
    At head dims 80 and 112 the MFMA kernel's padded K slots would read the next token's row
    (NaN after the context) if they were not zeroed."""
    ctx = [17, 40, 33, 100, 1, 48]
    case = wl.make_attention_case(context_lens=ctx, q_lens=[1, 5, 8, 3, 1, 4], num_heads=8,
                                  num_kv_heads=2, head_dim=D, dtype=dtype, seed=13, num_blocks=64)
    nan = np.uint16(0x7FC0) if dtype == "bf16" else np.float32(np.nan)
    used = set()
    for b, c in enumerate(ctx):
        nb = -(-c // case.block_size)
        used.update(int(x) for x in case.block_table[b, :nb])
        last, tail = int(case.block_table[b, nb - 1]), c - (nb - 1) * case.block_size
        case.key_cache[last, :, tail:, :] = nan
        case.value_cache[last, :, tail:, :] = nan
    unused = [i for i in range(case.key_cache.shape[0]) if i not in used]
    case.key_cache[unused] = nan
    case.value_cache[unused] = nan
    t = h.attention_tensors(case, gpu)
    exp = h.oracle_attention(case)
    attn = make_attention(16, 8, D, 2)
    for path in ("vector", "mfma") if D == 128 or dtype == "bf16" else ("vector",):
        for splits in (1, 2):
            out = attn.forward(t["query"], t["key_cache"], t["value_cache"], t["block_table"],
                               t["context_lens"], q_start_loc=t["q_start_loc"], path=path,
                               num_splits=splits)
            h.assert_attention_close(out, case, exp, h.ATOL_BF16 if dtype == "bf16" else h.ATOL_F32)


# Block sizes besides Kyro's 16 (its --block-size flag, src/config.rs:24-26): the MFMA kernels
# walk a block of 16 m tokens as m 16-token slots; other sizes run on the vector kernel.
BLOCK_SIZES = [8, 32, 48, 64, 256]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("D", [128, 64])
@pytest.mark.parametrize("bs", BLOCK_SIZES)
def test_block_sizes(gpu, dtype, D, bs):
    """Every path at each block size against the oracle: AUTO, the vector kernel, and where the
    MFMA kernel applies (block size a multiple of 16; f32 at head_dim 128 only) the MFMA kernel
    on the grid with 1 and 3 splits and under the balanced schedule. Contexts end inside a
    block's first, middle and last 16-token slot, and cover several blocks."""
    ctx, ql = [70, 5, 33, 130, 600, 16], [5, 1, 3, 8, 2, 4]
    case = wl.make_attention_case(context_lens=ctx, q_lens=ql, num_heads=8, num_kv_heads=2, head_dim=D,
                                  block_size=bs, dtype=dtype, seed=50 + bs + D)
    t = h.attention_tensors(case, gpu)
    attn = make_attention(bs, 8, D, 2)
    exp = h.oracle_attention(case)
    runs = [dict(), dict(path="vector"), dict(path="vector", num_splits=3)]
    mfma = bs % 16 == 0 and (D == 128 or dtype == "bf16")
    if mfma:
        runs += [dict(path="mfma", num_splits=1), dict(path="mfma", num_splits=3), dict(schedule="balanced")]
    else:
        with pytest.raises(kyro_amd.KyroError, match="block_size"):
            attn.forward(t["query"], t["key_cache"], t["value_cache"], t["block_table"], t["context_lens"],
                         q_start_loc=t["q_start_loc"], path="mfma")
    for kw in runs:
        out = attn.forward(t["query"], t["key_cache"], t["value_cache"], t["block_table"], t["context_lens"],
                           q_start_loc=t["q_start_loc"], **kw)
        h.assert_attention_close(out, case, exp, h.ATOL_BF16 if dtype == "bf16" else h.ATOL_F32)


@pytest.mark.parametrize("bs", [32, 64])
def test_block_sizes_nan_past_the_context_and_long(gpu, bs):
    """At 32- and 64-token blocks: NaN in every slot past each context (inside the last block's
    16-token slots too) and in unreferenced blocks, and contexts of 9000 and 20000 tokens under
    both schedules, against the oracle (bf16 KV, GQA 32/8, 8 query rows)."""
    ctx = [17, 40, 33, 100, 1, 48]
    case = wl.make_attention_case(context_lens=ctx, q_lens=[1, 5, 8, 3, 1, 4], num_heads=8, num_kv_heads=2,
                                  block_size=bs, dtype="bf16", seed=60 + bs, num_blocks=64)
    nan = np.uint16(0x7FC0)
    used = set()
    for b, c in enumerate(ctx):
        nb = -(-c // bs)
        used.update(int(x) for x in case.block_table[b, :nb])
        last, tail = int(case.block_table[b, nb - 1]), c - (nb - 1) * bs
        case.key_cache[last, :, tail:, :] = nan
        case.value_cache[last, :, tail:, :] = nan
    unused = [i for i in range(case.key_cache.shape[0]) if i not in used]
    case.key_cache[unused] = nan
    case.value_cache[unused] = nan
    t = h.attention_tensors(case, gpu)
    exp = h.oracle_attention(case)
    attn = make_attention(bs, 8, 128, 2)
    for kw in (dict(path="mfma"), dict(path="mfma", num_splits=2), dict(schedule="balanced")):
        out = attn.forward(t["query"], t["key_cache"], t["value_cache"], t["block_table"], t["context_lens"],
                           q_start_loc=t["q_start_loc"], **kw)
        h.assert_attention_close(out, case, exp, h.ATOL_BF16)
    case = wl.make_attention_case(context_lens=[9000, 20000, 700], q_lens=[8, 8, 8], num_heads=32, num_kv_heads=8,
                                  block_size=bs, dtype="bf16", seed=70 + bs)
    t = h.attention_tensors(case, gpu)
    attn = make_attention(bs, 32, 128, 8)
    exp = h.oracle_attention(case)
    for kw in (dict(schedule="grid"), dict(schedule="balanced")):
        out = attn.forward(t["query"], t["key_cache"], t["value_cache"], t["block_table"], t["context_lens"],
                           q_start_loc=t["q_start_loc"], out_dtype=torch.bfloat16, **kw)
        h.assert_attention_close(out, case, exp, h.ATOL_BF16)
    # GQA 64/8 with up to 64 rows per kv head: the four-tile kernel
    case = wl.make_attention_case(context_lens=[3000, 700, 50], q_lens=[8, 5, 1], num_heads=64, num_kv_heads=8,
                                  block_size=bs, dtype="bf16", seed=80 + bs)
    t = h.attention_tensors(case, gpu)
    attn = make_attention(bs, 64, 128, 8)
    exp = h.oracle_attention(case)
    for kw in (dict(schedule="grid"), dict(schedule="balanced")):
        out = attn.forward(t["query"], t["key_cache"], t["value_cache"], t["block_table"], t["context_lens"],
                           q_start_loc=t["q_start_loc"], **kw)
        h.assert_attention_close(out, case, exp, h.ATOL_BF16)


@pytest.mark.parametrize("bs", [16, 64])
@pytest.mark.parametrize("schedule,splits", [("grid", 1), ("grid", 3), ("auto", 0), ("balanced", 0)])
def test_five_tile_row_groups(gpu, schedule, splits, bs):
    """Units of 65-80 query rows per kv head (GQA 64/8 with 8 drafts: 72 rows) take one five-tile
    row group, and units of 129-160 rows (GQA 32/2 with 9 or 10 query rows) two, when most units
    of the batch are that long; the shorter units of the same launches fill part of a group or
    none of the second. Every cache policy, on the grid with and without splits and under the
    balanced schedule, in 16- and 64-token blocks, against the oracle."""
    for (H, Hkv), ctx, ql in (((64, 8), [3000, 700, 50, 1200, 0, 4100, 33, 260, 1500, 17, 800, 2047, 129],
                               [9, 9, 9, 9, 9, 9, 9, 9, 9, 9, 9, 9, 3]),
                              ((32, 2), [2500, 300, 47, 900, 1, 1200], [10, 10, 9, 10, 10, 6])):
        text = describe_attention(make_attention(bs, H, 128, Hkv), batch=len(ctx), total_q=sum(ql),
                                  max_q_len=max(ql), max_blocks_per_seq=512, num_blocks=4096)
        assert "row tiles 5," in text, text
        case = wl.make_attention_case(context_lens=ctx, q_lens=ql, num_heads=H, num_kv_heads=Hkv,
                                      block_size=bs, dtype="bf16", seed=90 + H + bs)
        t = h.attention_tensors(case, gpu)
        attn = make_attention(bs, H, 128, Hkv)
        exp = h.oracle_attention(case)
        for reuse in ("auto", "shared", "stream"):
            for out_dtype in (torch.float32, torch.bfloat16):
                out = attn.forward(t["query"], t["key_cache"], t["value_cache"], t["block_table"],
                                   t["context_lens"], q_start_loc=t["q_start_loc"], path="mfma",
                                   num_splits=splits, schedule=schedule, kv_reuse=reuse, out_dtype=out_dtype)
                h.assert_attention_close(out, case, exp, h.ATOL_BF16)


def test_long_context_in_one_split(gpu):
    """Contexts of 16384 and 16000 tokens in a single split: 1024 blocks, 128 block pairs per
    wave, so the block ids of a wave's pairs fill both slots of its lane-held table."""
    case = wl.make_attention_case(context_lens=[16384, 16000], q_lens=[3, 1], num_heads=8,
                                  num_kv_heads=2, dtype="bf16", seed=31)
    t = h.attention_tensors(case, gpu)
    attn = make_attention(16, 8, 128, 2)
    exp = h.oracle_attention(case)
    for splits in (1, 0):
        out = attn.forward(t["query"], t["key_cache"], t["value_cache"], t["block_table"],
                           t["context_lens"], q_start_loc=t["q_start_loc"], path="mfma",
                           num_splits=splits)
        h.assert_attention_close(out, case, exp, h.ATOL_BF16)


# ------------------------------------------------------------------ balanced schedule

BALANCED = [
    # (heads, kv heads, ctx lens, q lens): skew, empty contexts, sequences without rows, odd
    # kv head counts (one kv head per workgroup), three row groups, one split-clamped context
    ((32, 8), [3000, 17, 0, 512, 9000, 33, 1], [8, 8, 3, 0, 5, 1, 8]),
    ((64, 8), [260, 4100, 9, 700, 1, 2049], [9, 1, 4, 6, 9, 9]),
    ((12, 3), [5000, 40, 16, 1500], [2, 5, 1, 3]),
    ((8, 2), [20000, 100], [3, 1]),
    ((32, 8), [64], [8]),
    ((16, 2), [3000, 40, 0, 900, 17], [8, 5, 3, 8, 1]),
]


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("shape", BALANCED, ids=lambda s: f"{s[0][0]}x{s[0][1]}b{len(s[1])}")
def test_balanced_schedule_parity(gpu, shape, dtype):
    """The persistent balanced schedule against the oracle on every sequence, and against the
    grid schedule (same rows up to the rounding of split merges)."""
    (H, Hkv), ctx, ql = shape
    case = wl.make_attention_case(context_lens=ctx, q_lens=ql, num_heads=H, num_kv_heads=Hkv,
                                  dtype=dtype, seed=17)
    t = h.attention_tensors(case, gpu)
    attn = make_attention(16, H, 128, Hkv)
    args = (t["query"], t["key_cache"], t["value_cache"], t["block_table"], t["context_lens"])
    out = attn.forward(*args, q_start_loc=t["q_start_loc"], path="mfma", schedule="balanced")
    tol = h.ATOL_BF16 if dtype == "bf16" else h.ATOL_F32
    h.assert_attention_close(out, case, h.oracle_attention(case), tol)
    grid = attn.forward(*args, q_start_loc=t["q_start_loc"], path="mfma", schedule="grid")
    assert (out - grid).abs().max().item() < (1e-2 if dtype == "bf16" else 1e-4)
    again = attn.forward(*args, q_start_loc=t["q_start_loc"], path="mfma", schedule="balanced")
    assert torch.equal(out, again)


@pytest.mark.parametrize("seed", range(12))
def test_balanced_schedule_random_batches(gpu, seed):
    """Seeded random batches under the balanced schedule against the oracle on every sequence:
    1-40 sequences, kv head counts 1-8 (odd ones: one kv head per workgroup), GQA groups 1-8,
    0-9 query rows, contexts from 0 to 6000 tokens with a few long ones (so the plan splits
    some and not others), bf16 and f32."""
    rng = np.random.default_rng(1000 + seed)
    B = int(rng.integers(1, 41))
    Hkv = int(rng.choice([1, 2, 3, 4, 8]))
    H = Hkv * int(rng.choice([1, 2, 4, 8]))
    ql = rng.integers(0, 10, size=B)
    ctx = np.where(rng.random(B) < 0.15, rng.integers(2000, 6001, size=B), rng.integers(0, 400, size=B))
    ctx = np.maximum(ctx, 0)
    dtype = "bf16" if seed % 3 else "f32"
    case = wl.make_attention_case(context_lens=ctx.tolist(), q_lens=ql.tolist(), num_heads=H, num_kv_heads=Hkv,
                                  dtype=dtype, seed=seed)
    t = h.attention_tensors(case, gpu)
    attn = make_attention(16, H, 128, Hkv)
    out = attn.forward(t["query"], t["key_cache"], t["value_cache"], t["block_table"], t["context_lens"],
                       q_start_loc=t["q_start_loc"], path="mfma", schedule="balanced")
    h.assert_attention_close(out, case, h.oracle_attention(case), h.ATOL_BF16 if dtype == "bf16" else h.ATOL_F32)


@pytest.mark.parametrize("batch", [256, 1024])
def test_balanced_schedule_large_batches(gpu, batch):
    """256 sequences (ordered longest first by the plan) and 1024 (four per plan thread, kept in
    their order), lengths from 1 to 600 tokens with every 97th sequence at 3000; 1025 sequences
    are refused under "balanced" and run on the grid under "auto"."""
    rng = np.random.default_rng(3)
    ctx = rng.integers(1, 600, size=batch)
    ctx[::97] = 3000
    ctx = ctx.tolist()
    ql = rng.integers(1, 6, size=batch).tolist()
    case = wl.make_attention_case(context_lens=ctx, q_lens=ql, num_heads=8, num_kv_heads=2,
                                  dtype="bf16", seed=4)
    t = h.attention_tensors(case, gpu)
    attn = make_attention(16, 8, 128, 2)
    args = (t["query"], t["key_cache"], t["value_cache"], t["block_table"], t["context_lens"])
    out = attn.forward(*args, q_start_loc=t["q_start_loc"], path="mfma", schedule="balanced")
    h.assert_attention_close(out, case, h.oracle_attention(case), h.ATOL_BF16)
    if batch < 1024:
        return
    case2 = wl.make_attention_case(context_lens=ctx + [500], q_lens=ql + [2], num_heads=8, num_kv_heads=2,
                                   dtype="bf16", seed=4)
    t2 = h.attention_tensors(case2, gpu)
    args2 = (t2["query"], t2["key_cache"], t2["value_cache"], t2["block_table"], t2["context_lens"])
    with pytest.raises(kyro_amd.KyroError, match="at most 1024"):
        attn.forward(*args2, q_start_loc=t2["q_start_loc"], path="mfma", schedule="balanced")
    out2 = attn.forward(*args2, q_start_loc=t2["q_start_loc"], path="mfma")
    h.assert_attention_close(out2, case2, h.oracle_attention(case2, [0, 1023, 1024]), h.ATOL_BF16)


@pytest.mark.parametrize("H,ql", [(32, (8, 8, 3, 1, 5, 8)), (64, (8, 8, 3, 1, 5, 8)), (64, (9, 9, 9, 9, 9, 8))])
def test_balanced_schedule_replays_from_a_graph(gpu, H, ql):
    """A balanced launch (plan, per-lane claim counters, combine pass) captured in a HIP graph
    after an eager call on the same stream (so the arena is already large enough): every replay,
    with eager launches of another shape and synchronisations in between, equals the eager
    result bit for bit. GQA 32/8 runs the two-tile kernel, GQA 64/8 (up to 64 rows per kv head)
    the four-tile one, and GQA 64/8 with 72 rows on most sequences the five-tile one."""
    case = wl.make_attention_case(context_lens=[3000, 17, 0, 900, 5000, 33], q_lens=list(ql),
                                  num_heads=H, num_kv_heads=8, dtype="bf16", seed=23)
    other = wl.make_attention_case(context_lens=[700, 2100], q_lens=[2, 3], num_heads=H, num_kv_heads=8,
                                   dtype="bf16", seed=24)
    t = h.attention_tensors(case, gpu)
    t2 = h.attention_tensors(other, gpu)
    attn = make_attention(16, H, 128, 8)
    args = (t["query"], t["key_cache"], t["value_cache"], t["block_table"], t["context_lens"])
    args2 = (t2["query"], t2["key_cache"], t2["value_cache"], t2["block_table"], t2["context_lens"])
    s = torch.cuda.Stream(gpu)
    with torch.cuda.stream(s):
        eager = attn.forward(*args, q_start_loc=t["q_start_loc"], schedule="balanced")
        eager2 = attn.forward(*args2, q_start_loc=t2["q_start_loc"], schedule="balanced")
        out = torch.empty_like(eager)
    torch.cuda.synchronize()
    h.assert_attention_close(eager, case, h.oracle_attention(case), h.ATOL_BF16)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        attn.forward_async(*args, q_start_loc=t["q_start_loc"], schedule="balanced", out=out, max_q_len=max(ql))
    for _ in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        with torch.cuda.stream(s):
            again = attn.forward(*args2, q_start_loc=t2["q_start_loc"], schedule="balanced")
        torch.cuda.synchronize()
        assert torch.equal(again, eager2)


def test_balanced_schedule_slot_overflow_latches_an_error(gpu):
    """With fewer partial-state slots sized than the plan needs (forced from the host through
    the test-only kyro_testing_set_plan_slot_cap), the device plan latches an error and runs no
    item instead of writing past the workspace; the next call, sized normally, gives the
    oracle's result."""
    from kyro_amd import _lib

    case = wl.make_attention_case(context_lens=[5000, 40, 3000, 700], q_lens=[8, 3, 5, 1], num_heads=32,
                                  num_kv_heads=8, dtype="bf16", seed=31)
    t = h.attention_tensors(case, gpu)
    attn = make_attention(16, 32, 128, 8)
    args = (t["query"], t["key_cache"], t["value_cache"], t["block_table"], t["context_lens"])
    assert _lib.lib().kyro_testing_set_plan_slot_cap(3) == 0
    try:
        with pytest.raises(kyro_amd.KyroError, match="partial-state slots"):
            attn.forward(*args, q_start_loc=t["q_start_loc"], schedule="balanced")
    finally:
        assert _lib.lib().kyro_testing_set_plan_slot_cap(0) == 3
    out = attn.forward(*args, q_start_loc=t["q_start_loc"], schedule="balanced")
    h.assert_attention_close(out, case, h.oracle_attention(case), h.ATOL_BF16)


def test_arena_growth_is_refused_during_graph_capture(gpu):
    """A call whose scratch exceeds the context's arena while the stream captures a graph fails
    with a message naming the bytes to reserve (growing would free memory that captured kernels
    address); after kyro_ctx_reserve with the size query's answer the same capture succeeds and
    replays to the eager result."""
    from kyro_amd import _lib

    case = wl.make_attention_case(context_lens=[3000, 17, 900, 5000], q_lens=[8, 8, 1, 5], num_heads=32,
                                  num_kv_heads=8, dtype="bf16", seed=25)
    t = h.attention_tensors(case, gpu)
    attn = make_attention(16, 32, 128, 8)
    args = (t["query"], t["key_cache"], t["value_cache"], t["block_table"], t["context_lens"])
    ctx = _lib.Context(gpu.index or 0)
    s = torch.cuda.Stream(gpu)
    with torch.cuda.stream(s):
        # binds the fresh context to s; a one-split call uses no arena
        tiny = attn.forward_async(*args, q_start_loc=t["q_start_loc"], schedule="grid", num_splits=1, context=ctx)
        out = torch.zeros_like(tiny)
    ctx.sync()
    g = torch.cuda.CUDAGraph()
    with pytest.raises(kyro_amd.KyroError, match="kyro_ctx_reserve"):
        with torch.cuda.graph(g, stream=s):
            attn.forward_async(*args, q_start_loc=t["q_start_loc"], schedule="balanced", out=out, max_q_len=8,
                               context=ctx)
    params = _lib.PagedAttentionParams(16, 32, 128, 8, 4, int(case.q_start_loc[-1]), case.block_table.shape[1],
                                       case.key_cache.shape[0], _lib.KYRO_BF16, _lib.KYRO_F32, 1, 0.0, 0, 0, 8, 0,
                                       _lib.KYRO_ATTN_SCHEDULE_BALANCED)
    need = ctypes.c_size_t()
    _lib.check(_lib.lib().kyro_paged_attention_workspace(ctx.handle, ctypes.byref(params), 1, ctypes.byref(need)))
    assert need.value > 0
    ctx.reserve(need.value)
    with torch.cuda.stream(s):
        eager = attn.forward_async(*args, q_start_loc=t["q_start_loc"], schedule="balanced", max_q_len=8,
                                   context=ctx)
    ctx.sync()
    h.assert_attention_close(eager, case, h.oracle_attention(case), h.ATOL_BF16)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        attn.forward_async(*args, q_start_loc=t["q_start_loc"], schedule="balanced", out=out, max_q_len=8,
                           context=ctx)
    for _ in range(2):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
    del g
    ctx.close()


def test_balanced_schedule_errors(gpu):
    case = wl.make_attention_case(context_lens=[300, 40], q_lens=[2, 3], num_heads=8, num_kv_heads=2,
                                  dtype="bf16", seed=6)
    t = h.attention_tensors(case, gpu)
    attn = make_attention(16, 8, 128, 2)
    args = (t["query"], t["key_cache"], t["value_cache"], t["block_table"])
    with pytest.raises(kyro_amd.KyroError, match="num_splits"):
        attn.forward(*args, t["context_lens"], q_start_loc=t["q_start_loc"], schedule="balanced", num_splits=2)
    with pytest.raises(kyro_amd.KyroError, match="MFMA"):
        attn.forward(*args, t["context_lens"], q_start_loc=t["q_start_loc"], schedule="balanced", path="vector")
    # a context length beyond the table latches an error; the other sequence is still computed
    # and the context recovers on the next call
    bad = t["context_lens"].clone()
    bad[0] = case.block_table.shape[1] * 16 + 1
    with pytest.raises(kyro_amd.KyroError, match="context length"):
        attn.forward(*args, bad, q_start_loc=t["q_start_loc"], schedule="balanced")
    out = attn.forward(*args, t["context_lens"], q_start_loc=t["q_start_loc"], schedule="balanced")
    h.assert_attention_close(out, case, h.oracle_attention(case), h.ATOL_BF16)


# ---------------------------------------------------------------- full-size workloads


def _full(case, gpu, **kw):
    """Runs a full-size workload and compares every sequence with the oracle. Returns the device
    tensors, the attention object, the output and the oracle rows."""
    t = h.attention_tensors(case, gpu)
    attn = make_attention(case.block_size, case.num_heads, case.head_dim, case.num_kv_heads)
    out = attn.forward(t["query"], t["key_cache"], t["value_cache"], t["block_table"],
                       t["context_lens"], q_start_loc=t["q_start_loc"], **kw)
    exp = h.oracle_attention(case)
    h.assert_attention_close(out, case, exp, h.ATOL_BF16)
    return t, attn, out, exp


def test_full_mha_llama2_7b(gpu):
    """Llama-2-7B layer shape (MHA 32/32, B 16, ctx 512-2048, 5 rows): AUTO, the vector kernel
    and the MFMA kernel under both schedules, every sequence against the oracle."""
    case = wl.mha_llama2_7b()
    t, attn, out, exp = _full(case, gpu)
    args = (t["query"], t["key_cache"], t["value_cache"], t["block_table"], t["context_lens"])
    for kw in (dict(path="vector"), dict(path="mfma"), dict(schedule="balanced")):
        other = attn.forward(*args, q_start_loc=t["q_start_loc"], **kw)
        h.assert_attention_close(other, case, exp, h.ATOL_BF16)


def test_full_mha_llama2_7b_f32(gpu):
    """The reference's dtype at the Llama-2-7B layer shape: f32 Q/K/V on the f32 MFMA kernel
    (AUTO) and on the vector kernel, both against the oracle within the f32 tolerance."""
    case = wl.make_attention_case(context_lens=[512, 1000, 2048, 1777], q_lens=[5] * 4, num_heads=32,
                                  num_kv_heads=32, dtype="f32", seed=3)
    t = h.attention_tensors(case, gpu)
    attn = make_attention(16, 32, 128, 32)
    exp = h.oracle_attention(case)
    for path in ("auto", "vector"):
        out = attn.forward(t["query"], t["key_cache"], t["value_cache"], t["block_table"],
                           t["context_lens"], q_start_loc=t["q_start_loc"], path=path)
        h.assert_attention_close(out, case, exp, h.ATOL_F32)


def test_full_gqa_llama3_8b_properties(gpu):
    """Full Llama-3-8B verify shape: every sequence against the oracle, under AUTO, both explicit
    split counts, the balanced schedule and the vector kernel; permuting the physical blocks does
    not change the result bit for bit."""
    case = wl.gqa_llama3_8b()
    t, attn, out, exp = _full(case, gpu, out_dtype=torch.float32)
    args = (t["query"], t["key_cache"], t["value_cache"], t["block_table"], t["context_lens"])
    for kw in (dict(num_splits=1), dict(num_splits=16), dict(schedule="balanced"),
               dict(path="vector", num_splits=2)):
        other = attn.forward(*args, q_start_loc=t["q_start_loc"], **kw)
        h.assert_attention_close(other, case, exp, h.ATOL_BF16)
    nb = t["key_cache"].shape[0]
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(0)).to(gpu)
    k2 = torch.empty_like(t["key_cache"])
    v2 = torch.empty_like(t["value_cache"])
    k2[perm] = t["key_cache"]
    v2[perm] = t["value_cache"]
    out2 = attn.forward(t["query"], k2, v2, perm[t["block_table"]], t["context_lens"],
                        q_start_loc=t["q_start_loc"])
    assert torch.equal(out, out2)
    # The benchmark's exact call: bf16 output, max_q_len 8, AUTO path, schedule and kv_reuse,
    # into a preallocated output (forward_async, then the synchronising check).
    outb = torch.empty(out.shape, dtype=torch.bfloat16, device=gpu)
    attn.forward_async(*args, q_start_loc=t["q_start_loc"], max_q_len=8, out_dtype=torch.bfloat16, out=outb)
    kyro_amd.sync(0)
    h.assert_attention_close(outb, case, exp, h.ATOL_BF16)
    # bf16 rounding of the f32 result, nothing more
    assert torch.equal(outb, out.to(torch.bfloat16))


def test_full_skewed_prefix(gpu):
    """Skewed long-context batch with a 64-block prefix shared by all 32 sequences: every
    sequence against the oracle under AUTO (balanced schedule) and on the grid."""
    case = wl.skewed_prefix()
    t, attn, out, exp = _full(case, gpu)
    other = attn.forward(t["query"], t["key_cache"], t["value_cache"], t["block_table"], t["context_lens"],
                         q_start_loc=t["q_start_loc"], schedule="grid")
    h.assert_attention_close(other, case, exp, h.ATOL_BF16)


def test_full_mixed_llama3_70b(gpu):
    """Mixed batch at the Llama-3-70B layer shape (GQA 64/8, B 128, ragged 1-9 rows): every
    sequence against the oracle under AUTO (balanced schedule) and on the grid."""
    case, _ = wl.mixed_llama3_70b()
    t, attn, out, exp = _full(case, gpu)
    other = attn.forward(t["query"], t["key_cache"], t["value_cache"], t["block_table"], t["context_lens"],
                         q_start_loc=t["q_start_loc"], schedule="grid")
    h.assert_attention_close(other, case, exp, h.ATOL_BF16)


# ------------------------------------------------------------------------- error paths


def test_bad_block_id_and_context_length_raise(gpu):
    attn = make_attention(16, 8, 64, 2)
    q = torch.ones((1, 8, 64), device=gpu)
    kv = torch.ones((4, 2, 16, 64), device=gpu)
    with pytest.raises(kyro_amd.KyroError, match="block_table"):
        attn.forward(q, kv, kv, torch.tensor([[0, 9]], device=gpu), torch.tensor([20], device=gpu))
    with pytest.raises(kyro_amd.KyroError, match="context length"):
        attn.forward(q, kv, kv, torch.tensor([[0, 1]], device=gpu), torch.tensor([33], device=gpu))
    # the context recovers: the next valid call succeeds
    out = attn.forward(q, kv, kv, torch.tensor([[0, 1]], device=gpu), torch.tensor([20], device=gpu))
    torch.testing.assert_close(out, torch.ones_like(out))


def test_host_validation(gpu):
    attn = make_attention(16, 8, 64, 2)
    q = torch.ones((1, 8, 64), device=gpu)
    kv = torch.ones((4, 2, 16, 64), device=gpu)
    with pytest.raises(TypeError):
        attn.forward(q, kv.half(), kv.half(), torch.zeros((1, 4), dtype=torch.int64, device=gpu),
                     torch.tensor([4], device=gpu))
    with pytest.raises(kyro_amd.KyroError, match="MFMA"):
        attn.forward(q, kv, kv, torch.zeros((1, 4), dtype=torch.int64, device=gpu),
                     torch.tensor([4], device=gpu), path="mfma")


@pytest.mark.parametrize("path", ["vector", "mfma"])
def test_mha_b2_matches_golden_fixture(gpu, path):
    """Committed expected outputs (tests/golden/attention_mha_b2.npz): Llama-2-7B heads, bf16."""
    import os

    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "attention_mha_b2.npz"))
    case = wl.make_attention_case(context_lens=[17, 40], q_lens=[5, 5], num_heads=32, num_kv_heads=32,
                                  dtype="bf16", seed=0)
    t = h.attention_tensors(case, gpu)
    out = make_attention(16, 32, 128, 32).forward(
        t["query"], t["key_cache"], t["value_cache"], t["block_table"], t["context_lens"],
        q_start_loc=t["q_start_loc"], path=path)
    err = (out.cpu().numpy() - z["expected"]).__abs__().max()
    assert err <= h.ATOL_BF16, err
