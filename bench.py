#!/usr/bin/env python3
"""Verify-step benchmark on one MI355X: paged attention (one layer) + acceptance sampling.

Workload: the Llama-3-8B verify step — batch 64, k = 7 drafts (8 query rows per sequence), every
context 4096 tokens, GQA 32 query / 8 kv heads, head_dim 128, bf16 KV in 16-token blocks through
a shuffled block table, then acceptance over a 128256-entry vocabulary at temperature 0.8 with
target logits ~ N(0, 3) and draft logits = target + N(0, 1). Synthetic data of seed 0
(kyro_amd.workloads: numpy Philox4x64-10 bit generators keyed (seed, stream), numpy's ziggurat
normals), resident in HBM before timing starts.

One step = kyro_paged_attention_mq + kyro_spec_verify on the same stream. W warm-up steps, then
K timed steps. ``value`` is verified tokens per second, sum_b (accepted_b + 1) / seconds per step,
where a step's time is the mean over K steps each timed by HIP events on the launch stream after a
512 MiB read that evicts the L2s and the MALL (cold caches, as between two layers' worth of other
work). ``value_warm`` times K steps back to back between two synchronisations. A third pass of K
warm steps records HIP events around each part; those time the attention kernel for the roofline
entry and the per-part figures. The CPU oracle (f32 build) is timed on a bounded sample of the
same workload for the cpu_baseline entry.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
METRIC = "verified tok/s at bs64 k=7; paged-attn + sampling HBM GB/s (% of peak)"

B, HQ, HKV, D, BS, CTX, K_DRAFT, VOCAB, TEMP = 64, 32, 8, 128, 16, 4096, 7, 128256, 0.8


def make_inputs(dev, seed=0):
    """The Llama-3-8B verify-step inputs of kyro_amd.workloads: a numpy Philox4x64-10 generator
    per (seed, stream) (one stream per tensor), numpy's ziggurat normals, bf16 by round-to-nearest-
    even, draft tokens drawn from softmax(draft / T) by inverse CDF. Built on the host (a few
    seconds) and uploaded before any timing."""
    import numpy as np
    import torch

    from kyro_amd import workloads as wl

    a = wl.gqa_llama3_8b(batch=B, ctx=CTX, seed=seed)
    v = wl.verify_llama3_8b(batch=B, vocab=VOCAB, seed=seed)

    def up(x, bf16=False):
        t = torch.from_numpy(np.ascontiguousarray(x))
        return (t.view(torch.bfloat16) if bf16 else t).to(dev)

    return dict(q=up(a.query, True), kc=up(a.key_cache, True), vc=up(a.value_cache, True),
                table=up(a.block_table), ctx=up(a.context_lens), q_start=up(a.q_start_loc.astype(np.int32)),
                target=up(v.target), draft=up(v.draft), tokens=up(v.draft_tokens.astype(np.int32)),
                u_acc=up(v.u_accept), u_res=up(v.u_resample), nd=up(v.num_draft.astype(np.int32)),
                temp=up(v.temperature.astype(np.float32)))


def attention_bytes():
    kv = B * CTX * HKV * D * 2 * 2
    q = B * (K_DRAFT + 1) * HQ * D * 2
    return kv + q + q  # bf16 out has the query's size


def sampler_bytes(accepted=None):
    """Logit bytes of every row (accepted None), or of the rows the acceptance scan evaluates:
    target and draft rows 0 .. j of a sequence rejected at j, and every row (target 0 .. k,
    draft 0 .. k - 1) of a fully accepted one. Each row counted once."""
    if accepted is None:
        return B * (2 * K_DRAFT + 1) * VOCAB * 4
    j = accepted.cpu().long()
    rows = (j + 1) + j.clamp(max=K_DRAFT - 1) + 1
    return int(rows.sum().item()) * VOCAB * 4


def cpu_baseline(sample: int, threads: int):
    """Times the f32 build of the CPU oracle on `sample` sequences of the same workload."""
    import numpy as np

    import oracle
    from kyro_amd import workloads as wl

    acase = wl.gqa_llama3_8b(batch=sample, ctx=CTX)
    vcase = wl.verify_llama3_8b(batch=sample, vocab=VOCAB)
    t0 = time.perf_counter()
    oracle.paged_attention_mq(acase.query, acase.key_cache, acase.value_cache, acase.block_table,
                              acase.context_lens, num_heads=HQ, num_kv_heads=HKV, head_dim=D,
                              block_size=BS, q_start_loc=acase.q_start_loc, threads=threads,
                              precision="f32")
    t1 = time.perf_counter()
    r = oracle.spec_verify(vcase.target, vcase.draft, vcase.draft_tokens, vcase.num_draft,
                           vcase.temperature, vcase.u_accept, vcase.u_resample, precision="f32")
    t2 = time.perf_counter()
    tokens = int(np.sum(r["accepted"] + 1))
    # The same step on one core, over the first `sample1` sequences (the oracle's per-sequence
    # work does not depend on the batch it sits in).
    sample1 = max(1, min(sample, 16))
    acase1 = wl.gqa_llama3_8b(batch=sample1, ctx=CTX)
    vcase1 = wl.verify_llama3_8b(batch=sample1, vocab=VOCAB)
    t3 = time.perf_counter()
    oracle.paged_attention_mq(acase1.query, acase1.key_cache, acase1.value_cache, acase1.block_table,
                              acase1.context_lens, num_heads=HQ, num_kv_heads=HKV, head_dim=D,
                              block_size=BS, q_start_loc=acase1.q_start_loc, threads=1,
                              precision="f32")
    r1 = oracle.spec_verify(vcase1.target, vcase1.draft, vcase1.draft_tokens, vcase1.num_draft,
                            vcase1.temperature, vcase1.u_accept, vcase1.u_resample, precision="f32")
    t4 = time.perf_counter()
    tokens1 = int(np.sum(r1["accepted"] + 1))
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), model)
    except OSError:
        pass
    return {
        "value": tokens / (t2 - t0),
        "unit": "tok/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{sample} of {B} sequences of the same step (attention over ctx {CTX}, "
                   f"GQA {HQ}/{HKV}, then acceptance over V {VOCAB}); f32 CPU oracle, attention on "
                   f"{threads} threads ({t1 - t0:.2f} s), acceptance on 1 thread ({t2 - t1:.2f} s)"),
        "cpu_model": model,
        "host_cpus": os.cpu_count(),
        "one_core": {"value": tokens1 / (t4 - t3), "unit": "tok/s", "cores": 1,
                     "sample": f"{sample1} sequences of the same step on 1 thread ({t4 - t3:.2f} s)"},
    }


def _median_us(fn, warmup, steps):
    """Median per-call time of fn() in µs from HIP events on the current stream. The stream is
    first held by a short spin kernel while every timed call is queued behind it, so the events
    measure the GPU work and not the host's time to enqueue a small call."""
    import numpy as np
    import torch

    import kyro_amd

    for _ in range(warmup):
        fn()
    kyro_amd.sync(0)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    torch.cuda._sleep(int(5e6) * max(1, steps // 20))  # a few ms at gfx950 clocks
    for e0, e1 in ev:
        e0.record()
        fn()
        e1.record()
    torch.cuda.synchronize()
    kyro_amd.sync(0)
    return float(np.median([e0.elapsed_time(e1) for e0, e1 in ev])) * 1e3


def _roofline(nbytes, us, bound="hbm"):
    """Roofline entry for one kernel chain on its algorithmic bytes (bound "hbm": 8 TB/s peak)."""
    achieved = nbytes / us / 1e3
    return {"bound": bound, "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": achieved / PEAK_HBM_GBS}


def _cpu_seconds(fn, min_seconds=0.5):
    """Seconds per call of fn() on the host, repeated until min_seconds have passed."""
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        t = time.perf_counter() - t0
        if t >= min_seconds:
            return t / n


def kv_append_workload(warmup, steps):
    """One JSON line for the paged KV write (kyro_paged_kv_append): the verify step's 8 new rows per
    sequence of the Llama-3-8B workload, and a prefill of 4 x 2048 f32 rows into a bf16 cache.
    Algorithmic bytes: rows read (K and V) + rows written into the cache; block ids, context lengths
    and q_start_loc are a few KB."""
    import torch

    import kyro_amd

    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(0)
    res = {"workload": "kv-append"}
    for label, b, q, old, src in (("verify_llama3_8b", B, K_DRAFT + 1, CTX - K_DRAFT - 1, torch.bfloat16),
                                  ("prefill_4x2048_f32_rows", 4, 2048, 0, torch.float32)):
        ctx = old + q
        mb = (ctx + BS - 1) // BS
        nb = max(16384, b * mb)
        kc = torch.zeros((nb, HKV, BS, D), dtype=torch.bfloat16, device=dev)
        vc = torch.zeros_like(kc)
        table = torch.randperm(nb, generator=g, device=dev)[: b * mb].reshape(b, mb).contiguous()
        ctx_t = torch.full((b,), ctx, dtype=torch.int64, device=dev)
        qs = torch.arange(0, (b + 1) * q, q, dtype=torch.int32, device=dev)
        k = torch.randn((b * q, HKV, D), generator=g, device=dev).to(src)
        v = torch.randn((b * q, HKV, D), generator=g, device=dev).to(src)
        kv = kyro_amd.PagedKVCache(BS, HKV, D)
        us = _median_us(lambda: kv.append_kv_async(k, v, kc, vc, table, ctx_t, q_start_loc=qs, max_q_len=q),
                        warmup, steps)
        nbytes = 2 * b * q * HKV * D * (k.element_size() + 2)
        res[label] = {"us": us, "algorithmic_bytes": nbytes, "GB_s": nbytes / us / 1e3, "rows": b * q,
                      "roofline": _roofline(nbytes, us)}
    res["cpu_baseline"] = _kv_append_cpu()
    print(json.dumps(res), flush=True)


def _kv_append_cpu():
    """The oracle's KV append (C, one thread) on 8 of the verify batch's sequences: 8 new bf16
    rows each into a bf16 cache of their own blocks."""
    import numpy as np

    import oracle

    n, q, ctx = 8, K_DRAFT + 1, CTX
    mb = (ctx + BS - 1) // BS
    rng = np.random.default_rng(0)
    kc = np.zeros((n * mb, HKV, BS, D), np.uint16)
    vc = np.zeros_like(kc)
    table = rng.permutation(n * mb).reshape(n, mb).astype(np.int64)
    k = rng.integers(0, 1 << 15, size=(n * q, HKV, D)).astype(np.uint16)
    v = rng.integers(0, 1 << 15, size=(n * q, HKV, D)).astype(np.uint16)
    ctx_a = np.full(n, ctx, np.int64)
    qs = np.arange(0, (n + 1) * q, q).astype(np.int32)
    sec = _cpu_seconds(lambda: oracle.kv_append(k, v, kc, vc, table, ctx_a, block_size=BS, q_start_loc=qs))
    nbytes = 2 * n * q * HKV * D * 4
    return {"value": nbytes / sec / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{n} sequences x {q} bf16 rows of the verify step, oracle_kv_append"}


def block_tables_workload(warmup, steps):
    """One JSON line for the block-table producer: host allocation of 64 requests with 4096-token
    prompts sharing a 1000-token prefix (the prefix cache warmed by one finished request, so each
    allocation shares 62 blocks and copies one partially matched block), the device table write
    for the verify batch (64 x 256 int64 + context lengths), and the copy-on-write of 64 blocks."""
    import numpy as np
    import torch

    import kyro_amd

    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(0)
    prefix = rng.integers(0, 128256, size=1000).astype(np.uint32)
    prompts = [np.concatenate([prefix, rng.integers(0, 128256, size=CTX - 1000).astype(np.uint32)]) for _ in range(B)]
    times, copies = [], []
    for rep_i in range(max(3, warmup)):
        bm = kyro_amd.BlockManager(BS, 32768, 0)
        bm.allocate_with_prefix(10_000, prompts[0])
        bm.free(10_000)
        t0 = time.perf_counter()
        for b in range(B):
            bm.allocate_with_prefix(b, prompts[b])
        times.append((time.perf_counter() - t0) / B * 1e6)
        copies = bm.take_copies()
    table = torch.zeros((B, CTX // BS + 1), dtype=torch.int64, device=dev)
    lens = torch.zeros((B,), dtype=torch.int64, device=dev)
    write_us = _median_us(lambda: bm.write_tables(list(range(B)), table, lens), warmup, steps)
    kc = torch.zeros((32768, HKV, BS, D), dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    copy_us = _median_us(lambda: kyro_amd.copy_blocks(kc, vc, copies), warmup, steps)
    slab = HKV * BS * D * 2
    print(json.dumps({
        "workload": "block-tables",
        "allocate_with_prefix_host_us_per_request": float(np.median(times)),
        "cached_tokens_per_request": 1000,
        "write_tables": {"us": write_us, "bytes": int(table.numel() * 8 + B * 8)},
        "copy_blocks": {"us": copy_us, "pairs": len(copies), "bytes": 2 * 2 * slab * len(copies),
                        "GB_s": 2 * 2 * slab * len(copies) / copy_us / 1e3,
                        "roofline": _roofline(2 * 2 * slab * len(copies) * 2, copy_us)},
        "cpu_baseline": {"value": float(np.median(times)), "unit": "us per request", "cores": 1,
                         "kind": "port", "sample": "allocate_with_prefix is host code in the "
                         "reference and here alike; this is its time per request"},
    }), flush=True)


def decode_sample_workload(warmup, steps):
    """One JSON line for the plain-decode sampler (kyro_sample_tokens): 64 rows of V 128256 f32
    logits ~ N(0, 3), T 0.8, for each filter setting, plus one with every logit processor (bias,
    penalties from 256 generated tokens, a grammar mask on half the rows). Bytes: the logit rows
    read once (33 MB); the kernels re-read them from cache, so GB/s on these bytes is the rate at
    which a batch's rows are turned into tokens."""
    import numpy as np
    import torch

    import kyro_amd

    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(0)
    b, v = B, VOCAB
    x = (torch.randn((b, v), generator=g, device=dev) * 3).contiguous()
    u = torch.rand((b,), generator=g, device=dev)
    T = torch.full((b,), TEMP, device=dev)
    nbytes = b * v * 4
    res = {"workload": "decode-sample", "rows": b, "vocab": v, "logit_bytes": nbytes}
    rng = np.random.default_rng(0)
    settings = {
        "greedy": dict(temperature=torch.zeros((b,), device=dev)),
        "plain": {},
        # per-row settings as device tensors, built once: a host array would be copied (and the
        # host held) inside every timed call
        "top_k_50": dict(top_k=torch.full((b,), 50, dtype=torch.int32, device=dev)),
        "top_p_0.9": dict(top_p=torch.full((b,), 0.9, dtype=torch.float32, device=dev)),
        "top_k_50_top_p_0.9": dict(top_k=torch.full((b,), 50, dtype=torch.int32, device=dev),
                                   top_p=torch.full((b,), 0.9, dtype=torch.float32, device=dev)),
        "processors_plain": dict(
            bias=[{int(t): 1.0 for t in rng.integers(0, v, size=8)} for _ in range(b)],
            penalty=[kyro_amd.penalty_adds(rng.integers(0, v, size=256), 0.5, 0.2, v) for _ in range(b)],
            masks=np.stack([kyro_amd.grammar_mask(rng.choice(v, size=20000, replace=False), v)]),
            mask_row=np.where(np.arange(b) % 2 == 0, 0, -1).astype(np.int32)),
    }
    for name, kw in settings.items():
        kw = dict(kw)
        temp = kw.pop("temperature", T)
        if "bias" in kw:  # device tensors built once, outside the timed calls
            kw = {"processors": kyro_amd.sampling.Processors(b, v, dev, **kw)}
        out = torch.empty(b, dtype=torch.int32, device=dev)
        us = _median_us(lambda: kyro_amd.sample_tokens_async(x, temp, u, out=out, **kw), warmup, steps)
        res[name] = {"us": us, "GB_s": nbytes / us / 1e3, "roofline": _roofline(nbytes, us)}
    # CPU: the oracle's decode step (C, f32 build, one thread) on 4 of the rows
    import oracle

    xs = x[:4].cpu().numpy()
    us_np, T_np = u[:4].cpu().numpy(), T[:4].cpu().numpy()
    cpu = {}
    for name, kw in (("plain", {}), ("top_p_0.9", {"top_p": np.full(4, 0.9, np.float32)})):
        sec = _cpu_seconds(lambda: oracle.sample_decode(xs, T_np, us_np, precision="f32", **kw))
        cpu[name] = {"value": 4 / sec, "unit": "tok/s"}
    res["cpu_baseline"] = {"value": cpu["plain"]["value"], "unit": "tok/s", "cores": 1, "kind": "port",
                           "sample": "4 rows of V 128256, oracle_sample_decode (f32), plain; top-p 0.9: "
                                     f"{cpu['top_p_0.9']['value']:.0f} tok/s"}
    print(json.dumps(res), flush=True)


def ngram_draft_workload(warmup, steps):
    """One JSON line for n-gram drafting: a table of order 3 built on the host from a 1M-token
    corpus (vocabulary 128256, drawn so that prefixes repeat), then drafts of up to 7 tokens for
    the 64 sequences of the verify batch on the GPU."""
    import numpy as np
    import torch

    import kyro_amd

    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(0)
    corpus = [rng.integers(0, 2000, size=1 << 14).astype(np.uint32) for _ in range(64)]
    t0 = time.perf_counter()
    table = kyro_amd.NgramTable(corpus, 3)
    build_s = time.perf_counter() - t0
    contexts = [c[: int(rng.integers(100, 4000))] for c in corpus]
    tail, lens = kyro_amd.context_tails(contexts, 3, dev)
    toks = torch.empty((B, K_DRAFT), dtype=torch.int32, device=dev)
    nd = torch.empty((B,), dtype=torch.int32, device=dev)
    us = _median_us(lambda: table.draft(tail, lens, K_DRAFT, out=(toks, nd)), warmup, steps)
    # CPU: the oracle's dict table (built outside the timing) drafting for the same 64 contexts
    import oracle

    ref = oracle.ngram_build(corpus, 3)
    sec = _cpu_seconds(lambda: [oracle.ngram_draft(ref, c, 3, K_DRAFT) for c in contexts])
    print(json.dumps({"workload": "ngram-draft", "corpus_tokens": int(sum(c.size for c in corpus)),
                      "table_entries": len(table), "host_build_ms": build_s * 1e3, "draft_us": us,
                      "mean_drafts": float(nd.float().mean().item()),
                      "roofline": {"bound": "latency", "note": "one wave per sequence, 7 dependent "
                                   "lookups of one round of loads each (64 probe slots at once)"},
                      "cpu_baseline": {"value": sec * 1e6, "unit": "us per batch", "cores": 1,
                                       "kind": "port", "sample": "the same 64 contexts, Python dict "
                                       "table of the oracle"}}), flush=True)


def _cold_median_us(fn, steps, scratch):
    """Median per-call time of fn() in µs from HIP events on the current stream, each call after a
    read of `scratch` (512 MiB) that evicts the L2s and the MALL, as for the headline step."""
    import numpy as np
    import torch

    import kyro_amd

    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    torch.cuda.synchronize()
    for e0, e1 in ev:
        scratch.sum()
        e0.record()
        fn()
        e1.record()
    torch.cuda.synchronize()
    kyro_amd.sync(0)
    return float(np.median([e0.elapsed_time(e1) for e0, e1 in ev])) * 1e3


CONFIG_WORKLOADS = {
    "rejection-b8": "rejection sampling only: batch 8, k 4, V 32000, T 1.0",
    "mha-llama2-7b": "paged attention, Llama-2-7B layer: MHA 32/32, head_dim 128, batch 16, ctx U[512, 2048], q 5",
    "skewed-prefix": "skewed long-context verify: batch 32, ctx log-U[128, 32768], 64 shared prefix blocks, "
                     "GQA 32/8, k 4, V 128256, T 1.0",
    "mixed-llama3-70b": "mixed batch: 128 sequences, k U{0..8}, ctx U[256, 8192], GQA 64/8, V 128256, "
                        "half greedy, half T 0.7",
}


def measure_config(name, warmup, steps, detailed=False, scratch=None):
    """Attention (when the workload has one) and sampler (when it has one) of a non-default
    workload, each on its algorithmic bytes, as a dict. With `scratch` (a 512 MiB tensor) each
    part is also timed cold, after a cache-evicting read. `detailed` adds the vector and MFMA
    paths, the "shared" kv_reuse hint and the CPU oracle. Inputs come from kyro_amd.workloads
    (seeded numpy), uploaded before timing."""
    import torch

    import kyro_amd
    from kyro_amd import workloads as wl
    from kyro_amd.attention import describe_attention
    from kyro_amd.speculative import describe_verify

    dev = torch.device("cuda", 0)

    def up(a, bf16=False):
        t = torch.from_numpy(a)
        return (t.view(torch.bfloat16) if bf16 else t).to(dev)

    acase = vcase = None
    if name == "mha-llama2-7b":
        acase = wl.mha_llama2_7b()
    elif name == "rejection-b8":
        vcase = wl.rejection_only_b8()
    elif name == "skewed-prefix":
        acase, vcase = wl.skewed_prefix(), wl.verify_skewed()
    elif name == "mixed-llama3-70b":
        acase, k = wl.mixed_llama3_70b()
        vcase = wl.verify_mixed(k)
    else:
        raise SystemExit(f"unknown workload {name}")
    line = {"workload": name, "description": CONFIG_WORKLOADS[name]}
    total_us = 0.0
    if acase is not None:
        bf16 = acase.dtype == "bf16"
        t = dict(q=up(acase.query, bf16), kc=up(acase.key_cache, bf16), vc=up(acase.value_cache, bf16),
                 table=up(acase.block_table), ctx=up(acase.context_lens), qs=up(acase.q_start_loc))
        attn = kyro_amd.PagedAttention(acase.block_size, acase.num_heads, acase.head_dim, acase.num_kv_heads)
        out = torch.empty(t["q"].shape, dtype=torch.bfloat16, device=dev)
        logical = acase.kv_bytes() + acase.q_out_bytes(2)
        unique = acase.unique_kv_bytes() + acase.q_out_bytes(2)
        # The library's default kv_reuse hint (AUTO). Where tables share blocks (a common prefix)
        # the "shared" hint, which keeps K/V loads cacheable, is timed beside it.
        res = {"logical_bytes": logical, "unique_bytes": unique, "context_tokens": int(acase.context_lens.sum()),
               "kv_reuse": "auto",
               "launch": describe_attention(attn, batch=acase.batch, total_q=int(acase.q_start_loc[-1]),
                                            max_q_len=acase.max_q_len, max_blocks_per_seq=acase.block_table.shape[1],
                                            num_blocks=acase.key_cache.shape[0],
                                            dtype=torch.bfloat16 if bf16 else torch.float32, device=0)}
        runs = [("auto", "auto")]
        if detailed:
            runs += [("vector", "auto"), ("mfma", "auto")]
            if acase.unique_kv_bytes() < acase.kv_bytes():
                runs.append(("auto", "shared"))
        for path, reuse in runs:
            fn = lambda: attn.forward_async(  # noqa: E731
                t["q"], t["kc"], t["vc"], t["table"], t["ctx"], q_start_loc=t["qs"],
                max_q_len=acase.max_q_len, out_dtype=torch.bfloat16, out=out, path=path, kv_reuse=reuse)
            us = _median_us(fn, warmup, steps)
            entry = {"us": us, "GB_s_unique": unique / us / 1e3, "frac_unique": unique / us / 1e3 / PEAK_HBM_GBS,
                     "GB_s_logical": logical / us / 1e3}
            if scratch is not None and path == "auto" and reuse == "auto":
                cus = _cold_median_us(fn, steps, scratch)
                entry.update({"us_cold": cus, "frac_unique_cold": unique / cus / 1e3 / PEAK_HBM_GBS})
            res[path if reuse == "auto" else f"{path}_kv_reuse_{reuse}"] = entry
        res["roofline"] = _roofline(unique, res["auto"]["us"])
        if detailed:
            # CPU: the oracle's attention (f32 build, 16 threads) on the first two sequences
            import oracle

            n2 = min(2, acase.batch)
            nb2 = int(((acase.context_lens[:n2] + acase.block_size - 1) // acase.block_size).max())
            q2 = int(acase.q_start_loc[n2])
            sec = _cpu_seconds(lambda: oracle.paged_attention_mq(
                acase.query[:q2], acase.key_cache, acase.value_cache, acase.block_table[:n2, :nb2],
                acase.context_lens[:n2], num_heads=acase.num_heads, num_kv_heads=acase.num_kv_heads,
                head_dim=acase.head_dim, block_size=acase.block_size, q_start_loc=acase.q_start_loc[:n2 + 1],
                threads=16, precision="f32"), min_seconds=1.0)
            kv2 = int(acase.context_lens[:n2].sum()) * acase.num_kv_heads * acase.head_dim * 2 * 2
            res["cpu_baseline"] = {"value": kv2 / sec / 1e9, "unit": "GB/s of KV", "cores": 16, "kind": "port",
                                   "sample": f"the first {n2} sequences, oracle paged attention (f32)"}
        line["attention"] = res
        total_us += res["auto"]["us"]
    if vcase is not None:
        vt = dict(target_logits=up(vcase.target), draft_logits=up(vcase.draft),
                  draft_tokens=up(vcase.draft_tokens.astype("int32")), num_draft=up(vcase.num_draft),
                  temperature=up(vcase.temperature), u_accept=up(vcase.u_accept), u_resample=up(vcase.u_resample))
        fn = lambda: kyro_amd.verify_drafts_async(**vt)  # noqa: E731
        us = _median_us(fn, warmup, steps)
        r = kyro_amd.verify_drafts(**vt)
        emitted = int((r.accepted.cpu() + 1).sum().item())
        s_bytes = vcase.logit_bytes(r.accepted.cpu().numpy())
        line["sampler"] = {"us": us, "algorithmic_bytes": s_bytes, "all_rows_bytes": int(vcase.target.nbytes + vcase.draft.nbytes),
                           "GB_s": s_bytes / us / 1e3, "tokens": emitted, "mean_accepted": emitted / vcase.batch - 1,
                           "roofline": _roofline(s_bytes, us),
                           "launch": describe_verify(vcase.batch, vcase.draft_tokens.shape[1], vcase.target.shape[2])}
        if scratch is not None:
            line["sampler"]["us_cold"] = _cold_median_us(fn, steps, scratch)
        if detailed:
            # CPU: the oracle's acceptance (f32 build, one thread) on up to 8 sequences
            import oracle

            n8 = min(8, vcase.batch)
            sec = _cpu_seconds(lambda: oracle.spec_verify(
                vcase.target[:n8], vcase.draft[:n8], vcase.draft_tokens[:n8], vcase.num_draft[:n8],
                vcase.temperature[:n8], vcase.u_accept[:n8], vcase.u_resample[:n8], precision="f32"), min_seconds=1.0)
            r8 = oracle.spec_verify(vcase.target[:n8], vcase.draft[:n8], vcase.draft_tokens[:n8],
                                    vcase.num_draft[:n8], vcase.temperature[:n8], vcase.u_accept[:n8],
                                    vcase.u_resample[:n8], precision="f32")
            line["sampler"]["cpu_baseline"] = {"value": float((r8["accepted"] + 1).sum()) / sec, "unit": "tok/s",
                                               "cores": 1, "kind": "port",
                                               "sample": f"the first {n8} sequences, oracle acceptance (f32)"}
        total_us += us
        line["verified_tok_s_at_measured_parts"] = emitted / (total_us * 1e-6)
    return line


def shape_sweep_workload(kind, warmup, steps):
    """One JSON line: the attention on the Llama-3-8B verify shape (GQA 32/8, batch 64, ctx 4096,
    8 query rows, bf16 KV and out) at other head dims ("head-dims": 64, 80, 96, 112, 128, 160, 192,
    224 and 256 with 16-token blocks; AUTO takes the MFMA kernel at each of them)
    or other block sizes ("block-sizes": 8, 16, 32, 64 at head_dim 128; AUTO takes the MFMA
    kernel at every multiple of 16, the vector kernel at 8), AUTO and the vector kernel, each on
    its algorithmic bytes; or ("row-tiles") GQA 64/8 at head_dim 128 with 1, 2, 4, 8 and 9 query
    rows per sequence (8 to 72 rows per kv head: the one-, two-, four- and five-tile MFMA
    kernels), AUTO only."""
    import torch

    import kyro_amd
    from kyro_amd import workloads as wl
    from kyro_amd.attention import describe_attention

    dev = torch.device("cuda", 0)
    H = 64 if kind == "row-tiles" else 32
    res = {"workload": kind, "shape": f"GQA {H}/8, batch 64, ctx 4096, "
           + ("1-9" if kind == "row-tiles" else "8") + " query rows, bf16 KV and out"}
    if kind == "head-dims":
        points = [(D, 16, 8) for D in (64, 80, 96, 112, 128, 160, 192, 224, 256)]
    elif kind == "block-sizes":
        points = [(128, bs, 8) for bs in (8, 16, 32, 64)]
    else:
        points = [(128, 16, q) for q in (1, 2, 4, 8, 9)]
    for D, bs, ql in points:
        case = wl.make_attention_case(context_lens=[4096] * 64, q_lens=[ql] * 64, num_heads=H, num_kv_heads=8,
                                      head_dim=D, block_size=bs, dtype="bf16", seed=D + bs + ql)
        up = lambda x: torch.from_numpy(x).view(torch.bfloat16).to(dev)  # noqa: E731
        t = dict(q=up(case.query), kc=up(case.key_cache), vc=up(case.value_cache),
                 table=torch.from_numpy(case.block_table).to(dev), ctx=torch.from_numpy(case.context_lens).to(dev),
                 qs=torch.from_numpy(case.q_start_loc).to(dev))
        attn = kyro_amd.PagedAttention(bs, H, D, 8)
        out = torch.empty(t["q"].shape, dtype=torch.bfloat16, device=dev)
        nbytes = case.kv_bytes() + case.q_out_bytes(2)
        entry = {"algorithmic_bytes": nbytes}
        for path in (("auto",) if kind == "row-tiles" else ("auto", "vector")):
            us = _median_us(lambda: attn.forward_async(
                t["q"], t["kc"], t["vc"], t["table"], t["ctx"], q_start_loc=t["qs"], max_q_len=ql,
                out_dtype=torch.bfloat16, out=out, path=path), warmup, steps)
            entry[path] = {"us": us, "GB_s": nbytes / us / 1e3, "frac": nbytes / us / 1e3 / PEAK_HBM_GBS,
                           "launch": describe_attention(attn, batch=64, total_q=64 * ql, max_q_len=ql,
                                                        max_blocks_per_seq=case.block_table.shape[1],
                                                        num_blocks=case.key_cache.shape[0], path=path, device=0)}
        res[{"head-dims": f"d{D}", "block-sizes": f"bs{bs}"}.get(kind, f"q{ql}")] = entry
        del t, out
        torch.cuda.empty_cache()
    print(json.dumps(res), flush=True)


def other_workload(name, warmup, steps):
    """One JSON line for a non-default workload (measure_config with the vector and MFMA paths,
    the "shared" hint and the CPU oracle)."""
    print(json.dumps(measure_config(name, warmup, steps, detailed=True)), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    # 200 steps (about 55 ms): with 50, the launch of the first step and the final
    # synchronisation added about 4 us to every step's share.
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--path", default="auto", choices=["auto", "vector", "mfma"])
    ap.add_argument("--splits", type=int, default=0, help="context splits (0 = automatic)")
    ap.add_argument("--window", type=int, default=0,
                    help="draft positions read before the first acceptance scan (0 = library default)")
    ap.add_argument("--cpu-sample", type=int, default=64, help="sequences in the CPU-baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the other four workloads' figures in the benchmark line")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run 5 device-to-device copies of MIB MiB (the known-size kernel that "
                         "scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings), then exit")
    ap.add_argument("--workload", default="llama3-8b",
                    choices=["llama3-8b", "mha-llama2-7b", "rejection-b8", "skewed-prefix",
                             "mixed-llama3-70b", "kv-append", "block-tables", "decode-sample", "ngram-draft",
                             "head-dims", "block-sizes", "row-tiles", "others"],
                    help="llama3-8b (default) prints the benchmark line; the others print one "
                         "informational line each (attention and sampler on their algorithmic bytes)")
    args = ap.parse_args()
    if args.workload != "llama3-8b":
        names = (["mha-llama2-7b", "rejection-b8", "skewed-prefix", "mixed-llama3-70b", "kv-append", "block-tables",
                  "decode-sample", "ngram-draft", "head-dims", "block-sizes", "row-tiles"] if args.workload == "others"
                 else [args.workload])
        for n in names:
            if n == "kv-append":
                kv_append_workload(args.warmup, args.steps)
            elif n == "block-tables":
                block_tables_workload(args.warmup, args.steps)
            elif n == "decode-sample":
                decode_sample_workload(args.warmup, args.steps)
            elif n == "ngram-draft":
                ngram_draft_workload(args.warmup, args.steps)
            elif n in ("head-dims", "block-sizes", "row-tiles"):
                shape_sweep_workload(n, args.warmup, args.steps)
            else:
                other_workload(n, args.warmup, args.steps)
        return
    if args.calibrate_copy:
        import torch

        n = args.calibrate_copy << 20
        src = torch.ones(n // 4, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes": n, "copies": 5}))
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} (WORLD_SIZE {world}) is not supported; "
              "the verify step shards by sequence or kv head with no exchange, so the one-GPU "
              "figure is the per-GPU rate.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import kyro_amd

    dev = torch.device("cuda", 0)
    kyro_amd.lib()
    x = make_inputs(dev)
    attn = kyro_amd.PagedAttention(BS, HQ, D, HKV)
    out = torch.empty((B * (K_DRAFT + 1), HQ, D), dtype=torch.bfloat16, device=dev)
    acc = torch.empty((B,), dtype=torch.int32, device=dev)
    toks = torch.empty((B, K_DRAFT + 1), dtype=torch.int32, device=dev)

    def step(ev=None):
        if ev is not None:
            ev[0].record()
        attn.forward_async(x["q"], x["kc"], x["vc"], x["table"], x["ctx"], q_start_loc=x["q_start"],
                           max_q_len=K_DRAFT + 1, out_dtype=torch.bfloat16, out=out, path=args.path,
                           num_splits=args.splits)
        if ev is not None:
            ev[1].record()
        kyro_amd.verify_drafts_async(x["target"], x["draft"], x["tokens"], x["nd"], x["temp"],
                                     x["u_acc"], x["u_res"], out=(acc, toks), window=args.window)
        if ev is not None:
            ev[2].record()

    for _ in range(args.warmup):
        step()
    kyro_amd.sync(0)
    torch.cuda.synchronize()

    def spread(vals):
        return {"median": float(np.median(vals)), "p10": float(np.percentile(vals, 10)),
                "p90": float(np.percentile(vals, 90))}

    def summary(evs):
        return {"step_us": spread([e[0].elapsed_time(e[2]) * 1e3 for e in evs]),
                "attention_us": spread([e[0].elapsed_time(e[1]) * 1e3 for e in evs]),
                "sampler_us": spread([e[1].elapsed_time(e[2]) * 1e3 for e in evs])}

    # `value`: K cold steps. Before each, a 512 MiB read evicts the L2s and the 256 MiB MALL, as a
    # model's other layers would between two verify steps; HIP events on the launch stream bracket
    # the step alone. (A flushing write would leave dirty lines whose write-back lands in the step.)
    scratch = torch.ones(128 << 20, dtype=torch.float32, device=dev)
    for _ in range(2):
        scratch.sum()
    cold_events = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    for ev in cold_events:
        scratch.sum()
        step(ev)
    torch.cuda.synchronize()
    kyro_amd.sync(0)
    del scratch
    cold_steps_ms = [e[0].elapsed_time(e[2]) for e in cold_events]
    sec_per_step = float(np.mean(cold_steps_ms)) * 1e-3

    # Warm rate: the same K steps back to back with nothing else on the stream (logit rows partly
    # served from the MALL, which the benchmark loop re-reads every step).
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    kyro_amd.sync(0)
    warm_sec_per_step = (t1 - t0) / args.steps

    # Per-part times and the attention launch duration behind `roofline`: K more warm steps with
    # HIP events on the launch stream before the attention kernel, between it and the sampler, and
    # after the sampler (each record costs the stream a few microseconds).
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    t2 = time.perf_counter()
    for i in range(args.steps):
        step(events[i])
    torch.cuda.synchronize()
    t3 = time.perf_counter()
    kyro_amd.sync(0)
    instrumented_sec_per_step = (t3 - t2) / args.steps
    cold = dict(steps=args.steps, **summary(cold_events))
    attn_ms = float(np.mean([e[0].elapsed_time(e[1]) for e in events]))
    samp_ms = float(np.mean([e[1].elapsed_time(e[2]) for e in events]))
    emitted = int((acc.cpu() + 1).sum().item())
    a_bytes, s_bytes = attention_bytes(), sampler_bytes(acc)
    achieved = a_bytes / (attn_ms * 1e-3) / 1e9
    step_gbs = (a_bytes + s_bytes) / sec_per_step / 1e9
    # The step's bytes as a sampler that reads every logit row would move them (KV, Q, out, all
    # target and draft rows): 1,574,633,472 B on this workload. The step never reads the rows
    # after a sequence's first rejected draft, so this over-counts what it needs.
    all_rows_gbs = (a_bytes + sampler_bytes()) / sec_per_step / 1e9

    traffic = None
    # HBM bytes per attention launch from the rocprofv3 FETCH_SIZE / WRITE_SIZE runs recorded
    # in profiles/ (counters need runs of their own, so they are not read live here).
    pmc_path = os.path.join(ROOT, "profiles", "attention_llama3_8b_pmc.md")
    if os.path.exists(pmc_path):
        with open(pmc_path) as f:
            m = re.search(r"^hbm_bytes_per_launch:\s*(\d+)", f.read(), flags=re.M)
        traffic = int(m.group(1)) if m else None

    # The other four workloads of the benchmark's configuration list, timed the same way (cold:
    # after a cache-evicting read; warm: back to back), so that the one JSON line carries every
    # configuration. The Llama-3-8B step's inputs are freed first.
    from kyro_amd.attention import describe_attention
    from kyro_amd.speculative import describe_verify

    del x
    torch.cuda.empty_cache()
    configs = {}
    if not args.no_configs:
        scratch = torch.ones(128 << 20, dtype=torch.float32, device=dev)
        for n in ("rejection-b8", "mha-llama2-7b", "skewed-prefix", "mixed-llama3-70b"):
            configs[n] = measure_config(n, 10, 50, scratch=scratch)
            torch.cuda.empty_cache()
        del scratch
    configs["llama3-8b"] = {
        "workload": "llama3-8b",
        "description": "full verify step, Llama-3-8B: GQA 32/8, head_dim 128, batch 64, ctx 4096, k 7, "
                       "V 128256, T 0.8 (the headline)",
        "attention": {"logical_bytes": a_bytes, "unique_bytes": a_bytes, "us": attn_ms * 1e3,
                      "us_cold": cold["attention_us"]["median"],
                      "frac_unique": a_bytes / (attn_ms * 1e-3) / 1e9 / PEAK_HBM_GBS,
                      "frac_unique_cold": a_bytes / (cold["attention_us"]["median"] * 1e-6) / 1e9 / PEAK_HBM_GBS,
                      "launch": describe_attention(attn, batch=B, total_q=B * (K_DRAFT + 1), max_q_len=K_DRAFT + 1,
                                                   max_blocks_per_seq=CTX // BS, num_blocks=16384, device=0,
                                                   path=args.path, num_splits=args.splits)},
        "sampler": {"us": samp_ms * 1e3, "us_cold": cold["sampler_us"]["median"], "algorithmic_bytes": s_bytes,
                    "all_rows_bytes": sampler_bytes(), "GB_s": s_bytes / (samp_ms * 1e-3) / 1e9,
                    "tokens": emitted, "mean_accepted": emitted / B - 1,
                    "launch": describe_verify(B, K_DRAFT, VOCAB, args.window)},
    }

    baseline = None
    if not args.no_cpu_baseline:
        threads = max(1, min(16, os.cpu_count() or 1))
        baseline = cpu_baseline(args.cpu_sample, threads)

    line = {
        "metric": METRIC,
        "value": emitted / sec_per_step,
        "value_warm": emitted / warm_sec_per_step,
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": sec_per_step * 1e3,
        "ms_per_step_warm": warm_sec_per_step * 1e3,
        "timing": "value and ms_per_step: mean of K steps each timed by HIP events after a 512 MiB "
                  "cache-evicting read; value_warm: K steps back to back between two synchronisations",
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic, seed 0 (kyro_amd.workloads): numpy Philox4x64-10 bit generators keyed "
                "(seed, stream), numpy ziggurat normals; KV, Q ~ N(0,1) bf16; target logits ~ N(0,3); "
                "draft = target + N(0,1); draft tokens ~ softmax(draft/T) by inverse CDF; tables: one "
                "shuffled pool of 16384 blocks",
        "config": {
            "workload": "Llama-3-8B verify step: paged attention (1 layer) + acceptance sampling",
            "batch": B, "draft_k": K_DRAFT, "context": CTX, "q_heads": HQ, "kv_heads": HKV,
            "head_dim": D, "block_size": BS, "kv_dtype": "bf16", "vocab": VOCAB,
            "temperature": TEMP, "logits_dtype": "f32", "attention_path": args.path,
            "splits": args.splits, "window": args.window,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "attn_mfma_kernel" if args.path != "vector" else "attn_vector_kernel",
            "achieved": achieved,
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": achieved / PEAK_HBM_GBS,
            "traffic": traffic,
            "algorithmic_bytes": a_bytes,
            "avg_launch_us": attn_ms * 1e3,
        },
        "cpu_baseline": baseline,
        "step": {
            "algorithmic_bytes": a_bytes + s_bytes,
            "GB_s": step_gbs,
            "frac_of_peak": step_gbs / PEAK_HBM_GBS,
            "bytes_note": "algorithmic_bytes / GB_s / frac_of_peak count the logit rows the acceptance scan "
                          "evaluates (each once); all_rows_* count every logit row, including the rows after "
                          "each sequence's first rejection that the step never reads",
            "all_rows_bytes": a_bytes + sampler_bytes(),
            "all_rows_GB_s": all_rows_gbs,
            "all_rows_frac_of_peak": all_rows_gbs / PEAK_HBM_GBS,
            "instrumented_ms_per_step": instrumented_sec_per_step * 1e3,
            "attention_us": attn_ms * 1e3,
            "sampler_us": samp_ms * 1e3,
            "sampler_GB_s": s_bytes / (samp_ms * 1e-3) / 1e9,
            "sampler_bytes_evaluated_rows": s_bytes,
            "sampler_bytes_all_rows": sampler_bytes(),
            "tokens_per_step": emitted,
            "mean_accepted": emitted / B - 1,
            "accepted_histogram": torch.bincount(acc.cpu().long(), minlength=K_DRAFT + 1).tolist(),
            "warm_instrumented": summary(events),
            "cold_cache": cold,
        },
        "configs_note": "every configuration of the benchmark list: attention (with its combine pass) and "
                        "sampler timed separately by HIP events, median of 50 calls; us_cold after a 512 MiB "
                        "cache-evicting read, us back to back; frac_unique on the unique KV + Q + out bytes "
                        "(shared prefix blocks counted once); sampler bytes are the logit rows the acceptance "
                        "scan evaluates, each once",
        "configs": configs,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
