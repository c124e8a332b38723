"""Writes the golden fixtures under tests/golden/ (run from the repository root:
``python tests/golden/make_golden.py``).

* ``reference_kats.json`` — the known-answer tests the reference's own test suites hold for this
  path: ``sample_token`` (src/worker.rs:395-457) and the PagedAttention shape/value cases
  (src/model/attention_kernel.rs:154-227). Inputs and expected outputs only.
* ``rejection_b8.json`` — the rejection-sampling-only workload (B 8, k 4, V 32000, target ~ N(0, 2),
  draft = target + N(0, 0.5), T 1, seed 0). Inputs are regenerated from the recipe by
  kyro_amd.workloads, and their SHA-256 digests are stored to detect drift. Expected outputs come
  from the f64 oracle. Before writing, this script re-derives every acceptance decision, p_i(x_i)
  and q_i(x_i) with scipy's softmax, and every draw with numpy's searchsorted.
* ``attention_mha_b2.npz`` — a reduced Llama-2-7B attention case (32/32 heads, D 128, bf16,
  contexts 17 and 40, 5 causal query rows each, seed 0). Expected f32 outputs come from the
  oracle, cross-checked against torch's CPU scaled_dot_product_attention.
"""
import hashlib
import json
import os
import sys

import numpy as np
import scipy.special
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from kyro_amd import workloads as wl  # noqa: E402


def digest(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def reference_kats():
    return {
        "source": "src/worker.rs:395-457 (sample_token) and src/model/attention_kernel.rs:154-227",
        "sample_token": [
            {"logits": [0.1, 0.2, 0.3, 0.4, 0.5, 10.0, 0.1, 0.2], "temperature": 0.0, "top_p": 1.0,
             "top_k": None, "expect": [5]},
            {"logits": [1.0, 2.0, 3.0, 0.5, 0.1], "temperature": 0.0, "top_p": 1.0, "top_k": None,
             "expect": [2]},
            {"logits": [0.1, 0.2, 5.0, 0.4], "temperature": 0.0, "top_p": 1.0, "top_k": None,
             "expect": [2]},
            {"logits": [100.0, 0.0, 0.0, 0.0, 0.0], "temperature": 2.0, "top_p": 1.0, "top_k": None,
             "expect": [0]},
            {"logits": [100.0, 0.0, 0.0, 0.0, 0.0], "temperature": 1.0, "top_p": 0.5, "top_k": None,
             "expect": [0]},
            {"logits": [1.0, 2.0, 10.0, 0.5, 0.1], "temperature": 1.0, "top_p": 1.0, "top_k": 2,
             "expect": [1, 2]},
        ],
        "paged_attention": [
            {"name": "zero_context", "block_size": 16, "num_heads": 8, "head_dim": 64, "num_kv_heads": 2,
             "num_blocks": 4, "fill": 0.0, "block_table": [[0, 0, 0, 0]], "context_lens": [0],
             "expect_shape": [1, 8, 64], "expect_value": 0.0},
            {"name": "mha_single_block", "block_size": 16, "num_heads": 8, "head_dim": 64, "num_kv_heads": 8,
             "num_blocks": 4, "fill": 1.0, "block_table": [[0, 0, 0, 0]], "context_lens": [8],
             "expect_shape": [1, 8, 64], "expect_value": 1.0},
            {"name": "mha_multi_block_aliased", "block_size": 16, "num_heads": 8, "head_dim": 64,
             "num_kv_heads": 8, "num_blocks": 4, "fill": 1.0, "block_table": [[0, 0, 0, 0]],
             "context_lens": [24], "expect_shape": [1, 8, 64], "expect_value": 1.0},
        ],
    }


def rejection_b8():
    case = wl.rejection_only_b8()
    r = oracle.spec_verify(case.target, case.draft, case.draft_tokens, case.num_draft,
                           case.temperature, case.u_accept, case.u_resample)
    B, k = case.draft_tokens.shape
    # independent re-derivation with scipy / numpy
    for b in range(B):
        j = 0
        while j < k:
            x = case.draft_tokens[b, j]
            p = scipy.special.softmax(case.target[b, j].astype(np.float64))
            q = scipy.special.softmax(case.draft[b, j].astype(np.float64))
            assert abs(r["p_draft"][b, j] - p[x]) <= 1e-12 * p[x] + 1e-300
            assert abs(r["q_draft"][b, j] - q[x]) <= 1e-12 * q[x] + 1e-300
            if not case.u_accept[b, j] < min(1.0, p[x] / q[x]):
                break
            j += 1
        assert j == r["accepted"][b]
        if j < k:
            p = scipy.special.softmax(case.target[b, j].astype(np.float64))
            q = scipy.special.softmax(case.draft[b, j].astype(np.float64))
            w = np.maximum(p - q, 0.0)
        else:
            w = scipy.special.softmax(case.target[b, k].astype(np.float64))
        cdf = np.cumsum(w)
        want = int(np.searchsorted(cdf, case.u_resample[b] * cdf[-1], side="left"))
        assert want == r["tokens"][b, j] or r["resample_margin"][b] < 1e-9
    return {
        "workload": "rejection_only_b8 (B 8, k 4, V 32000, target N(0,2), draft = target + N(0,0.5), T 1, seed 0)",
        "generator": "kyro_amd.workloads.rejection_only_b8()",
        "sha256": {
            "target": digest(case.target), "draft": digest(case.draft),
            "draft_tokens": digest(case.draft_tokens), "u_accept": digest(case.u_accept),
            "u_resample": digest(case.u_resample),
        },
        "draft_tokens": case.draft_tokens.tolist(),
        "accepted": r["accepted"].tolist(),
        "tokens": r["tokens"].astype(np.int64).tolist(),
        "p_draft": [[None if np.isnan(v) else float(v) for v in row] for row in r["p_draft"]],
        "q_draft": [[None if np.isnan(v) else float(v) for v in row] for row in r["q_draft"]],
        "accept_margin": [[None if np.isnan(v) else float(v) for v in row] for row in r["accept_margin"]],
        "resample_margin": [float(v) for v in r["resample_margin"]],
    }


def attention_mha_b2():
    case = wl.make_attention_case(context_lens=[17, 40], q_lens=[5, 5], num_heads=32, num_kv_heads=32,
                                  dtype="bf16", seed=0)
    out = oracle.paged_attention_mq(case.query, case.key_cache, case.value_cache, case.block_table,
                                    case.context_lens, num_heads=32, num_kv_heads=32, head_dim=128,
                                    block_size=16, q_start_loc=case.q_start_loc)
    # cross-check against torch SDPA on the gathered context
    q_all = wl.bf16_bits_to_f32(case.query)
    kc, vc = wl.bf16_bits_to_f32(case.key_cache), wl.bf16_bits_to_f32(case.value_cache)
    for b in range(2):
        ctx = int(case.context_lens[b])
        blocks = case.block_table[b, : -(-ctx // 16)]
        k = torch.from_numpy(np.ascontiguousarray(kc[blocks].transpose(1, 0, 2, 3).reshape(32, -1, 128)[:, :ctx])).double()
        v = torch.from_numpy(np.ascontiguousarray(vc[blocks].transpose(1, 0, 2, 3).reshape(32, -1, 128)[:, :ctx])).double()
        q = torch.from_numpy(np.ascontiguousarray(q_all[5 * b:5 * b + 5].transpose(1, 0, 2))).double()
        mask = torch.arange(ctx)[None, :] <= (ctx - 5 + torch.arange(5)[:, None])
        ref = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=mask).transpose(0, 1).numpy()
        assert np.max(np.abs(ref - out[5 * b:5 * b + 5])) < 1e-9
    return case, out


def main():
    with open(os.path.join(HERE, "reference_kats.json"), "w") as f:
        json.dump(reference_kats(), f, indent=1)
    with open(os.path.join(HERE, "rejection_b8.json"), "w") as f:
        json.dump(rejection_b8(), f, indent=1)
    case, out = attention_mha_b2()
    np.savez_compressed(os.path.join(HERE, "attention_mha_b2.npz"), expected=out.astype(np.float32),
                        query_sha256=np.array(digest(case.query)),
                        kv_sha256=np.array(digest(case.key_cache, case.value_cache)),
                        block_table=case.block_table, context_lens=case.context_lens,
                        q_start_loc=case.q_start_loc)
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
