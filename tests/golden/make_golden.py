"""Writes the golden fixtures under tests/golden/ from the CPU oracle.  TEST INFRASTRUCTURE ONLY.

The reference ships no golden vectors and cannot be imported here (model/cuda.py imports tvm, which
is absent).  So these fixtures are written by the oracle after tests/test_oracle_pinning.py has
pinned it against the local transformers Qwen2, torch SDPA and closed forms.
tests/test_golden.py checks the fixtures against transformers independently of the oracle.

cfg1_tiny.npz   BASELINE cfg1: tiny fp32 model, seed 0, prompt of 16 ids in [0, 510), mask id 511.
                The decode loop (fast_dllm_relax/runtime.py:591-880) runs with max_new_tokens 80: a
                stateless first block, then a cached block refined in sub-blocks of 8 with partial
                steps (rp0/8/16/24) and threshold 0.9.  The fixture holds the per-call trace and the
                tokens, plus logits of one cached refinement step and one partial step.
hd128_bf16.npz  A small head_dim-128 model (the HIP attention's head size) in bf16 and fp32, seed 5:
                prefix of 64 through build_prefix_cache, one 32-row cached step, its logits and
                confidence, and a partial rp8 step.  The GPU parity test compares the HIP path
                with it.

Usage: python tests/golden/make_golden.py
"""

from __future__ import annotations

import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import confidence as oconf  # noqa: E402
from oracle.model import OracleConfig, OracleModel, build_prefix_block_attention_bias, random_params  # noqa: E402
from oracle.runtime import (build_prefix_cache_from_ids, greedy_generate, score_active_block_partial_perlayer,  # noqa: E402
                            score_active_block_refine)

CFG1 = dict(vocab_size=512, hidden_size=64, intermediate_size=128, num_hidden_layers=2, num_attention_heads=4,
            num_key_value_heads=2, head_dim=16)
HD128 = dict(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
             num_key_value_heads=2, head_dim=128)
CFG1_MASK = 511
CFG1_NEW = 80


def cfg1_fixture() -> dict:
    cfg = OracleConfig(**CFG1)
    model = OracleModel(cfg, random_params(cfg, 0, "float32"), "float32")
    prompt = np.random.default_rng(0).integers(0, 510, 16)
    trace: list = []
    tokens, stats = greedy_generate(model, prompt.tolist(), max_new_tokens=CFG1_NEW, block_size=32,
                                    small_block_size=8, threshold=0.9, mask_id=CFG1_MASK, stop_token=None,
                                    trace=trace)
    seq = prompt.tolist() + list(tokens)
    # one cached refinement step of the second block (first token known, 31 masks), then a partial
    # step over rows 8..15 of that block with one of them unmasked
    cache = build_prefix_cache_from_ids(model, seq[:32], block_size=32, capacity=96)
    active = seq[32:33] + [CFG1_MASK] * 31
    h_full = model.forward_cached(model.embed(active)[None], cache.k, cache.v, 32, 32)
    logits_full = model.get_logits(h_full)[0]
    ids_full, maxp_full = score_active_block_refine(model, active, cache)
    ids_p, maxp_p = score_active_block_partial_perlayer(model, active[8:15] + [seq[47]], cache, 8, block_size=32)
    kinds = {"full": 0, "partial": 1, "stateless": 2, "append": 3}
    # one row per model call: kind, sub-block offset (append: prefix length), number of rows unmasked
    # (append: the appended token), then up to 8 rows and their 8 tokens; -1 pads
    tr = np.full((len(trace), 19), -1, np.int64)
    for i, item in enumerate(trace):
        tr[i, 0] = kinds[item[0]]
        tr[i, 1] = item[1]
        if item[0] == "append":
            tr[i, 2] = item[2]
            continue
        rows, toks = item[2], item[3]
        tr[i, 2] = len(rows)
        tr[i, 3:3 + len(rows)] = rows
        tr[i, 11:11 + len(toks)] = toks
    return dict(prompt=prompt.astype(np.int64), tokens=np.asarray(tokens, np.int64), trace=tr,
                stats=np.asarray([stats[k] for k in ("unmask_updates", "block_recomputes", "partial_recomputes",
                                                      "block_appends")], np.int64),
                refine_active=np.asarray(active, np.int64), refine_hidden=h_full[0].astype(np.float32),
                refine_logits=logits_full.astype(np.float32),
                refine_ids=np.asarray(ids_full, np.int64), refine_maxp=np.asarray(maxp_full, np.float32),
                partial_ids=np.asarray(ids_p, np.int64), partial_maxp=np.asarray(maxp_p, np.float32))


def hd128_fixture() -> dict:
    cfg = OracleConfig(**HD128)
    rng = np.random.default_rng(11)
    P, R, cap = 64, 32, 128
    ids = rng.integers(0, HD128["vocab_size"] - 1, P + R)
    arrays = random_params(cfg, 5, "bfloat16")
    out = dict(ids=ids.astype(np.int64), P=np.int64(P), cap=np.int64(cap))
    for tag, dtype in (("bf16", "bfloat16"), ("f32", "float32")):
        model = OracleModel(cfg, arrays, dtype)
        kc = np.zeros((2, 1, cap, 2, 128), np.float32)
        vc = kc.copy()
        model.build_prefix_cache(model.embed(ids[:P])[None], build_prefix_block_attention_bias(0, P, block_size=32),
                                 kc, vc)
        h = model.forward_cached(model.embed(ids[P:])[None], kc, vc, P, P)
        out[f"hidden_{tag}"] = h[0].astype(np.float32)
        lg = model.get_logits(h)[0]
        out[f"logits_{tag}"] = lg.astype(np.float32)
        if tag == "bf16":
            cid, cp = oconf.confidence(lg)
            out["conf_ids"], out["conf_maxp"] = cid.astype(np.int64), cp.astype(np.float32)
        hp = model.forward_block_partial(8, model.embed(ids[P + 8:P + 16])[None], kc, vc, P + 8, P)
        out[f"partial8_{tag}"] = hp[0].astype(np.float32)
    return out


def main() -> None:
    np.savez_compressed(HERE / "cfg1_tiny.npz", **cfg1_fixture())
    np.savez_compressed(HERE / "hd128_bf16.npz", **hd128_fixture())
    for f in ("cfg1_tiny.npz", "hd128_bf16.npz"):
        print(f, (HERE / f).stat().st_size, "bytes")


if __name__ == "__main__":
    main()
