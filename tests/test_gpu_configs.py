"""BASELINE.json's configs 4 and 5 at their own sizes (two layers of the 1.5B shapes) against the oracle.
Marked gpu; every model call goes through the C ABI.  (Config 3's decode loop at full depth is in
test_gpu_loop.py; config 2 at full depth in test_gpu_fulldepth.py.)

* Config 4: fp16, seed 3, 16 sequences with bench.py's prefixes (U[128, 1024] from seed 3), each block
  starting at its prefix rounded down to 32 (the prompt's tail, then masks).  The full 32-row step runs the
  batched path's default attention (the RoPE / KV-append pass and attn_seq_kernel with key splits over the
  idle compute units, merged by the last split to arrive), the 8-row partial step the chunk kernel; each
  sequence's hidden states and appended K/V rows meet the per-sequence fp16 oracle.
* Config 5: bf16, seed 4, an 8192-token prefix through build_prefix_cache (the paired-query-block prefill
  attention in its default regime and the register-weight GEMMs at M = 8192) against the oracle's caches,
  then the 64-token continuation scored by score_masked_continuation (64 cached rows: 24 query tiles per
  kv head, the long-block attention kernel with key splits) and its per-token log-probabilities.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import WIDE2, bf16_parity, log, make_pair, to_np
from oracle.model import build_prefix_block_attention_bias

pytestmark = pytest.mark.gpu


def _dev_ids(ids):
    return torch.tensor(np.asarray(ids), dtype=torch.int32, device="cuda")


@pytest.mark.timeout(900)
def test_cfg4_batched_step_fp16_bench_prefixes():
    from fast_dllm_relax_amd.config import DEFAULT_MASK_ID

    kw = dict(WIDE2, tie_word_embeddings=False)
    log("setup: 1.5B shapes, 2 layers, fp16, seed 3, untied lm_head N(0, 0.5)")
    ref, vm = make_pair(kw, 3, "float16", lm_head_std=0.5, max_rows=1024)
    rng = np.random.default_rng(3)
    prefixes = [int(p) for p in rng.integers(128, 1025, 16)]
    prompts = [rng.integers(0, 150000, p).tolist() for p in prefixes]
    a0s = [p - p % 32 for p in prefixes]
    blocks = [prompts[b][a0s[b]:] + [DEFAULT_MASK_ID] * (32 - (prefixes[b] - a0s[b])) for b in range(16)]
    L, nkv, hd = kw["num_hidden_layers"], kw["num_key_value_heads"], kw["head_dim"]
    cap = max(a0s) + 32
    log(f"  prefixes {prefixes}; block starts {a0s}")
    want_h, want_k, want_v = [], [], []
    for b in range(16):
        kc = np.zeros((L, 1, cap, nkv, hd), np.float32)
        vc = kc.copy()
        if a0s[b]:
            ref.build_prefix_cache(ref.embed(prompts[b][:a0s[b]])[None],
                                   build_prefix_block_attention_bias(0, a0s[b], block_size=32), kc, vc)
        want_h.append(ref.forward_cached(ref.embed(blocks[b])[None], kc, vc, a0s[b], a0s[b])[0])
        want_k.append(kc[:, 0])
        want_v.append(vc[:, 0])
    log("  oracle done; HIP build_prefix_cache_seq x 16")
    k = torch.zeros((L, 16, cap, nkv, hd), dtype=torch.float16, device="cuda")
    v = torch.zeros_like(k)
    for b in range(16):
        vm.build_prefix_cache_seq(vm.embed(_dev_ids(prompts[b][:a0s[b]]))[None], None, k, v, b)
    x = torch.stack([vm.embed(_dev_ids(blocks[b])) for b in range(16)])
    off = torch.tensor(a0s, dtype=torch.int32, device="cuda")
    log("case: forward_cached_batch, 16 x 32 rows (M = 512)")
    h = vm.forward_cached_batch(x, k, v, off, a0s)
    kn, vn = to_np(k), to_np(v)
    for b in range(16):
        P = a0s[b]
        bf16_parity(f"cfg4 seq {b} hidden", to_np(h[b]), want_h[b])
        bf16_parity(f"cfg4 seq {b} K rows", kn[:, b, :P + 32], want_k[b][:, :P + 32])
        bf16_parity(f"cfg4 seq {b} V rows", vn[:, b, :P + 32], want_v[b][:, :P + 32])
    log("case: forward_block_partial_batch rp8, 16 x 8 rows (M = 128)")
    hp = vm.forward_block_partial_batch(8, x[:, 8:16].contiguous(), k, v, off + 8, a0s)
    for b in range(16):
        bf16_parity(f"cfg4 seq {b} partial rp8 hidden", to_np(hp[b]), want_h[b][8:16])
    vm.close()


@pytest.mark.timeout(900)
def test_cfg5_long_prefill_and_scoring():
    from fast_dllm_relax_amd.config import DEFAULT_MASK_ID
    from fast_dllm_relax_amd import runtime as rt
    from oracle import runtime as ort

    kw = dict(WIDE2)
    P, C = 8192, 64
    log("setup: 1.5B shapes, 2 layers, bf16, seed 4")
    ref, vm = make_pair(kw, 4, "bfloat16", max_rows=P)
    rng = np.random.default_rng(4)
    prefix = [int(t) for t in rng.integers(0, 150000, P)]
    cont = [int(t) for t in rng.integers(0, 150000, C)]
    log(f"case: build_prefix_cache {P} rows (HIP)")
    hc = rt.build_prefix_cache_from_ids(vm, prefix, block_size=32, capacity=P + C)
    torch.cuda.synchronize()
    log("  oracle prefill (2 layers) ...")
    oc = ort.build_prefix_cache_from_ids(ref, prefix, block_size=32, capacity=P + C)
    kn, vn = to_np(hc.k), to_np(hc.v)
    for layer in range(kw["num_hidden_layers"]):
        bf16_parity(f"cfg5 layer {layer} K ({P} rows)", kn[layer, 0, :P], oc.k[layer, 0, :P])
        bf16_parity(f"cfg5 layer {layer} V ({P} rows)", vn[layer, 0, :P], oc.v[layer, 0, :P])
    log(f"case: score_masked_continuation, {C} tokens after {P}")
    got, _ = rt.score_masked_continuation(vm, prefix, cont, block_size=32, mask_id=DEFAULT_MASK_ID)
    want = ort.score_masked_continuation(ref, prefix, cont, block_size=32, mask_id=DEFAULT_MASK_ID)
    got = np.asarray(got, np.float32)
    assert got.shape == want.shape == (C, kw["vocab_size"])
    bf16_parity("cfg5 continuation logits", got, want)

    def logprobs(z):
        z = z.astype(np.float64)
        zs = z - z.max(axis=-1, keepdims=True)
        lse = np.log(np.exp(zs).sum(axis=-1))
        return zs[np.arange(len(cont)), cont] - lse

    lp_h, lp_o = logprobs(got), logprobs(want)
    log(f"  per-token log-probs: max |d| {float(np.abs(lp_h - lp_o).max()):.4g}; "
        f"sums {lp_h.sum():.4f} (HIP) / {lp_o.sum():.4f} (oracle)")
    np.testing.assert_allclose(lp_h, lp_o, atol=5e-2)
    vm.close()
