#!/usr/bin/env python3
"""Benchmark of Fast-dLLM v2's cached block-diffusion step on one MI355X.

Workload (the metric's configuration): the 1.5B architecture in bf16 with random-init weights, seed 2,
lm_head N(0, 0.5), a 2048-token random prompt and 256 new tokens decoded by the block-diffusion loop
(blocks of 32 refined in sub-blocks of 8, threshold 0.9, block cache on; the loop of
fast_dllm_relax/runtime.py:591-880).  One bench step = one such generation.  The headline value is
decode tokens/s = new tokens / (generation time - prefill time), the reference's definition
(fast_dllm_relax/runners.py:748-750), summed over the timed steps.

Beside it the JSON line carries:
  block_step      synced medians (HIP events on the kernels' stream) of one 32-row refinement step
                  (forward_cached + fused lm_head/confidence) and one 8-row partial step at prefix 2048,
                  with their algorithmic HBM bytes and GB/s (weights + KV read + KV write + rows);
  roofline        the dominant kernel (the gate_up projection with the SiLU epilogue) timed alone with
                  HIP events over launches that walk the 28 layers;
  cpu_baseline    the CPU oracle's 32-row refinement step (numpy fp32 with the bf16 rounding points) at
                  the same prefix on the host's cores, scaled to tokens/s with the GPU loop's tokens per
                  model call;
  prefix512       BASELINE config 2: the 1.5B architecture in bf16 (tied head), seed 1, a 512-row prefix;
                  synced medians of forward_cached alone, of the full 32-row refinement step and of the
                  four 8-row partial steps (rp 0, 8, 16, 24) over a block of masks;
  long_context    BASELINE config 5: seed 4, an 8192-token prefix through build_prefix_cache (prefill
                  tokens/s), then a 64-token continuation scored by score_masked_continuation with the
                  per-token log-probabilities of the loglikelihood path (scoring ms);
  batched         BASELINE config 4: the 1.5B architecture in fp16, seed 3, 16 sequences with prefix
                  lengths drawn from U[128, 1024], one 32-token masked block each refined in sub-blocks
                  of 8 (threshold 0.9) by batched steps over all 16 sequences (the projections at M = 512);
                  aggregate tokens/s, the batched step times and their MFMA rate against the fp16 peak.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
"""

from __future__ import annotations

import argparse
import json
import os
import pathlib
import statistics
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBPS = 8000.0
PREFIX = 2048
NEW_TOKENS = 256
SEED = 2


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def event_ms(fn, iters: int, warmup: int = 2) -> float:
    """Median of per-call times measured with HIP events on torch's current stream."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    times = []
    for _ in range(iters):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        b.synchronize()
        times.append(a.elapsed_time(b))
    return statistics.median(times)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--new-tokens", type=int, default=NEW_TOKENS)
    ap.add_argument("--prefix", type=int, default=PREFIX)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-batched", action="store_true")
    ap.add_argument("--no-prefix512", action="store_true")
    ap.add_argument("--no-long-context", action="store_true")
    ap.add_argument("--cpu-iters", type=int, default=5)
    ap.add_argument("--profile-target", choices=("batched", "prefill8192", "decode", "decode-gaps"),
                    help="only run a short workload for rocprofv3: 'batched' = config 4's 512-row and 128-row "
                         "batched steps (5 each), 'prefill8192' = two 8192-row prefills, 'decode' = config 3's "
                         "decode loop (one warm-up and one timed generation of --new-tokens after the prompt; "
                         "--host-loop runs the loop with the host-side unmask instead of the device one); "
                         "'decode-gaps' runs three generations without a profiler and prints the GPU time between "
                         "model calls, from events recorded after each call's last launch and before the next "
                         "call's first (device loop only)")
    ap.add_argument("--host-loop", action="store_true",
                    help="decode with the host-side unmask (a readback per step) instead of the device loop")
    ap.add_argument("--trace-gaps", metavar="KERNEL_TRACE_CSV",
                    help="host only: read a rocprofv3 kernel trace of the decode loop and print the GPU idle time "
                         "between consecutive model calls")
    ap.add_argument("--traffic-probe", nargs="?", const="gate_up", choices=("gate_up", "step"),
                    help="for rocprofv3 --pmc: 'gate_up' (default) launches the dominant kernel over the 28 layers, "
                         "then a plain 256 MiB copy; 'step' builds the 2048-row prefix, copies 256 MiB, then runs one "
                         "32-row refinement step (forward_cached + lm_head + confidence)")
    ap.add_argument("--traffic-report", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="host only: per-kernel HBM bytes of the step from the two counter_collection.csv files of "
                         "`--traffic-probe step` runs, scaled by the calibration copy")
    args = ap.parse_args()

    if args.trace_gaps:
        return trace_gaps(args.trace_gaps)
    if args.traffic_report:
        return traffic_report(*args.traffic_report)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: the cached block step is batch-1 and this build has no "
              f"multi-GPU path (asked for --gpus {args.gpus})", file=sys.stderr, flush=True)
        return 2

    import numpy as np
    import torch

    import __graft_entry__

    __graft_entry__.load_package()
    if args.profile_target is not None:
        return profile_target(args.profile_target, args)
    from fast_dllm_relax_amd import _lib
    from fast_dllm_relax_amd.config import DEFAULT_MASK_ID, fast_dllm_v2_1p5b
    from fast_dllm_relax_amd.params import random_params_torch
    from fast_dllm_relax_amd.runtime import (allocate_prefix_cache, build_prefix_cache_from_ids, cache_spec_of,
                                             relax_greedy_generate, score_active_block_partial_perlayer,
                                             score_active_block_refine)
    from fast_dllm_relax_amd.vm import HipVM

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    torch.cuda.set_device(0)

    # lm_head N(0, 0.5) is an untied head: scaling a tied embedding would also scale every input row,
    # and each masked row would then predict its own (mask) token.
    cfg = fast_dllm_v2_1p5b(tie_word_embeddings=False)
    log("generating random weights on the GPU")
    params = random_params_torch(cfg, SEED, dtype="bfloat16", device="cuda", std=0.02, lm_head_std=0.5)
    vm = HipVM(cfg, params, dtype="bfloat16", max_rows=PREFIX)
    if args.traffic_probe == "step":
        return traffic_probe_step(vm, cfg)
    if args.traffic_probe:
        return traffic_probe(vm, cfg)
    rng = np.random.default_rng(SEED)
    prompt = rng.integers(0, 150000, args.prefix).tolist()
    P = args.prefix

    # ---- decode loop: the headline --------------------------------------------------------------
    def generate():
        timing: dict = {}
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        out, stats = relax_greedy_generate(vm, prompt, max_new_tokens=args.new_tokens, block_size=32,
                                           small_block_size=8, threshold=0.9, mask_id=DEFAULT_MASK_ID,
                                           stop_token=None, timing=timing, device_loop=not args.host_loop)
        torch.cuda.synchronize()
        total = time.perf_counter() - t0
        return out, stats, total, timing["prefill_latency_s"]

    for i in range(args.warmup):
        log(f"warmup generation {i + 1}/{args.warmup}")
        generate()
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    runs = []
    for i in range(args.steps):
        out, stats, total, prefill = generate()
        runs.append((len(out), stats, total, prefill))
        log(f"step {i + 1}/{args.steps}: {len(out)} tokens, total {total * 1e3:.1f} ms, prefill "
            f"{prefill * 1e3:.1f} ms, calls {stats['block_recomputes']} (partial {stats['partial_recomputes']})")
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_start
    tokens = sum(r[0] for r in runs)
    decode_s = sum(r[2] - r[3] for r in runs)
    value = tokens / decode_s
    calls = sum(r[1]["block_recomputes"] for r in runs)
    tokens_per_call = tokens / calls

    # ---- single cached block steps at prefix P ----------------------------------------------------
    log(f"block steps at prefix {P}")
    cache = build_prefix_cache_from_ids(vm, prompt, block_size=32, capacity=P + 32)
    block = rng.integers(0, 150000, 32).tolist()
    refine_ms = event_ms(lambda: score_active_block_refine(vm, block, cache), 20)
    partial_ms = event_ms(lambda: score_active_block_partial_perlayer(vm, block[8:16], cache, 8, block_size=32), 20)
    bytes_r32 = cfg.step_bytes(32, P)
    bytes_r8 = cfg.step_bytes(8, P)

    # ---- the attention callback alone (fdllm_attn_inplace): one call per layer over the same cache,
    # with rotated queries and the block's K/V rows of a refinement step ---------------------------------
    q_cb = torch.randn((1, 32, cfg.num_attention_heads, cfg.head_dim), device="cuda").to(torch.bfloat16)
    kv_cb = torch.randn((1, 32, cfg.num_key_value_heads, cfg.head_dim), device="cuda").to(torch.bfloat16)
    o_cb = vm.attn_inplace(q_cb, kv_cb, kv_cb, cache.k, cache.v, 0, P, 0, 32)[2]  # checked once, then raw calls
    cb_args = (q_cb.data_ptr(), kv_cb.data_ptr(), kv_cb.data_ptr(), 32, cache.k.data_ptr(), cache.v.data_ptr(),
               cache.capacity)
    cb_stream = torch.cuda.current_stream().cuda_stream

    def attn_layers():
        for layer in range(cfg.num_hidden_layers):
            _lib.check(vm.lib.fdllm_attn_inplace(vm.ctx, *cb_args, layer, P, 0, 32, o_cb.data_ptr(), cb_stream))

    attn_cb_us = event_ms(attn_layers, 10) / cfg.num_hidden_layers * 1e3

    # ---- dominant kernel alone (gate_up + SiLU), events on the launch stream ------------------------
    stream = torch.cuda.current_stream().cuda_stream
    lib = vm.lib
    iters = 4 * cfg.num_hidden_layers

    def gate_up():
        _lib.check(lib.fdllm_bench_op(vm.ctx, _lib.OP_GATE_UP, 32, 0, iters, None, None, 0, 0, stream))

    gu_ms = event_ms(gate_up, 10) / iters
    H, I = cfg.hidden_size, cfg.intermediate_size
    gu_bytes = 2 * I * H * 2 + 32 * H * 2 + 32 * I * 2  # weights + input rows + output rows
    gu_gbps = gu_bytes / (gu_ms * 1e-3) / 1e9
    traffic = measured_traffic()
    step_traffic = measured_step_traffic()

    # ---- CPU baseline: the oracle's refinement step on the host ------------------------------------
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(vm, params, cache, block, P, args.cpu_iters, tokens_per_call)

    # ---- the other BASELINE configurations, one model at a time ------------------------------------
    del cache
    vm.close()
    del vm, params
    torch.cuda.empty_cache()
    prefix512 = None if args.no_prefix512 else prefix512_bench()
    torch.cuda.empty_cache()
    long_context = None if args.no_long_context else long_context_bench()
    torch.cuda.empty_cache()
    batched = None if args.no_batched else batched_bench(args)

    line = {
        "metric": "decode tokens/s (1.5B bf16, bs1); block-step ms + achieved HBM GB/s",
        "value": round(value, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init weights N(0,0.02), lm_head N(0,0.5), seed 2; random prompt ids)",
        "config": {
            "workload": f"Fast-dLLM v2 block-diffusion decode: 1.5B bf16, batch 1, prompt {P}, "
                        f"{args.new_tokens} new tokens, block 32 / sub-block 8, threshold 0.9, block cache on",
            "global_batch": 1, "seq_len": P + args.new_tokens, "parallelism": "single GPU",
        },
        "decode": {"tokens": tokens, "decode_s": round(decode_s, 4), "model_calls": calls,
                   "tokens_per_call": round(tokens_per_call, 3),
                   "prefill_ms_mean": round(statistics.mean(r[3] for r in runs) * 1e3, 2)},
        "block_step": {
            "prefix": P,
            "refine_r32_ms": round(refine_ms, 4), "refine_r32_bytes": bytes_r32,
            "refine_r32_gbps": round(bytes_r32 / (refine_ms * 1e-3) / 1e9, 1),
            "partial_r8_ms": round(partial_ms, 4), "partial_r8_bytes": bytes_r8,
            "partial_r8_gbps": round(bytes_r8 / (partial_ms * 1e-3) / 1e9, 1),
        },
        "roofline": {"kernel": "gemm_os_kernel<bf16, EPI_SILU_PAIR, XF_RMS> (RMSNorm + gate_up + SiLU*up, 32 rows)",
                     "bound": "hbm", "achieved": round(gu_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gu_gbps / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "avg_launch_us": round(gu_ms * 1e3, 2), "bytes_per_launch": gu_bytes,
                     "step_traffic": step_traffic,
                     "step_traffic_ratio": round(step_traffic / bytes_r32, 4) if step_traffic else None,
                     "step_counter_gbps": round(step_traffic / (refine_ms * 1e-3) / 1e9, 1) if step_traffic else None},
        "attention_callback": {"workload": f"fdllm_attn_inplace (fast_dllm.attn_inplace): 32 rotated query rows, "
                                           f"K/V rows written at {P}, attention over {P + 32} keys, one call per "
                                           f"layer", "us_per_call": round(attn_cb_us, 2)},
        "cpu_baseline": cpu,
        "prefix512": prefix512,
        "long_context": long_context,
        "batched": batched,
    }
    print(json.dumps(line), flush=True)
    return 0


def prefix512_bench() -> dict:
    """Config 2: seed 1, tied lm_head N(0, 0.02), 512 random prefix ids; a block of 32 mask tokens."""
    import numpy as np

    from fast_dllm_relax_amd.config import DEFAULT_MASK_ID, fast_dllm_v2_1p5b
    from fast_dllm_relax_amd.params import random_params_torch
    from fast_dllm_relax_amd.runtime import (_embed, _offset_tensor, build_prefix_cache_from_ids,
                                             score_active_block_partial_perlayer, score_active_block_refine)
    from fast_dllm_relax_amd.vm import HipVM

    P = 512
    cfg = fast_dllm_v2_1p5b()
    log("prefix512: generating bf16 weights (seed 1)")
    params = random_params_torch(cfg, 1, dtype="bfloat16", device="cuda")
    vm = HipVM(cfg, params, dtype="bfloat16", max_rows=P)
    rng = np.random.default_rng(1)
    cache = build_prefix_cache_from_ids(vm, rng.integers(0, 150000, P).tolist(), block_size=32, capacity=P + 32)
    block = [DEFAULT_MASK_ID] * 32
    emb = _embed(vm, block)
    off = _offset_tensor(P)
    layers_ms = event_ms(lambda: vm.forward_cached(emb, cache.k, cache.v, off, P), 20)
    full_ms = event_ms(lambda: score_active_block_refine(vm, block, cache), 20)
    part = {}
    for rp in (0, 8, 16, 24):
        part[f"rp{rp}"] = round(event_ms(lambda: score_active_block_partial_perlayer(
            vm, block[rp:rp + 8], cache, rp, block_size=32), 20), 4)
    b32, b8 = cfg.step_bytes(32, P), cfg.step_bytes(8, P)
    res = {"workload": "BASELINE config 2: 1.5B bf16, seed 1, tied lm_head, prefix 512 via build_prefix_cache, "
                       "a block of 32 mask tokens",
           "forward_cached_ms": round(layers_ms, 4), "refine_r32_ms": round(full_ms, 4),
           "refine_r32_gbps": round(b32 / (full_ms * 1e-3) / 1e9, 1), "partial_r8_ms": part,
           "partial_r8_gbps": round(b8 / (part["rp8"] * 1e-3) / 1e9, 1)}
    log(f"prefix512: forward_cached {layers_ms:.3f} ms, refine {full_ms:.3f} ms, partial {part}")
    vm.close()
    return res


def long_context_bench() -> dict:
    """Config 5: seed 4, 8192 random prefix ids through build_prefix_cache, then a 64-token random
    continuation scored with score_masked_continuation and reduced to per-token log-probabilities."""
    import numpy as np
    import torch

    from fast_dllm_relax_amd.config import DEFAULT_MASK_ID, fast_dllm_v2_1p5b
    from fast_dllm_relax_amd.params import random_params_torch
    from fast_dllm_relax_amd.runtime import build_prefix_cache_from_ids, score_masked_continuation
    from fast_dllm_relax_amd.vm import HipVM

    P, C = 8192, 64
    cfg = fast_dllm_v2_1p5b()
    log("long_context: generating bf16 weights (seed 4)")
    params = random_params_torch(cfg, 4, dtype="bfloat16", device="cuda")
    vm = HipVM(cfg, params, dtype="bfloat16", max_rows=P)
    rng = np.random.default_rng(4)
    prefix = rng.integers(0, 150000, P).tolist()
    cont = rng.integers(0, 150000, C).tolist()

    def prefill():
        return build_prefix_cache_from_ids(vm, prefix, block_size=32, capacity=P + C)

    def timed(fn, n):
        out, ts = None, []
        for _ in range(n):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            out = fn()
            torch.cuda.synchronize()
            ts.append(time.perf_counter() - t0)
        return out, statistics.median(ts)

    prefill()  # warm-up
    cache, prefill_s = timed(prefill, 3)
    log(f"long_context: prefill {P} rows {prefill_s * 1e3:.1f} ms")

    def score():
        logits, _ = score_masked_continuation(vm, prefix, cont, block_size=32, mask_id=DEFAULT_MASK_ID,
                                              cached_prefix=(prefix, cache))
        # the reference's reduction (runners.py:876-880): fp32 log-softmax of the host logits, then a gather
        x = torch.from_numpy(np.asarray(logits, dtype=np.float32))
        return torch.log_softmax(x, dim=-1)[torch.arange(C), torch.tensor(cont)].numpy()

    score()  # warm-up
    logprobs, score_s = timed(score, 5)
    res = {"workload": f"BASELINE config 5: 1.5B bf16, seed 4, prefix {P} via build_prefix_cache, {C}-token "
                       "continuation scored by score_masked_continuation + the fp32 log-softmax and gather of "
                       "runners.py:876-880",
           "prefill_ms": round(prefill_s * 1e3, 2), "prefill_tokens_per_s": round(P / prefill_s, 1),
           "scoring_ms": round(score_s * 1e3, 3), "loglikelihood": round(float(logprobs.sum()), 4)}
    log(f"long_context: scoring {score_s * 1e3:.2f} ms")
    vm.close()
    return res


MFMA_F16_PEAK_TFLOPS = 2500.0  # dense fp16 / bf16
BATCH_SEED = 3
BATCH_SEQS = 16


def batched_bench(args) -> dict:
    """Config 4: 16 sequences of the 1.5B architecture in fp16 refined together.

    Synthetic weights N(0, 0.02) from seed 3 with an untied lm_head N(0, 0.5) (as in config 3: with the
    tied N(0, 0.02) head a masked row's strongest logit is its own mask token, and the loop would
    never unmask it).  Prefix lengths are drawn from U[128, 1024] with seed 3; each sequence's prompt
    is that many random ids, and its 32-token block starts at the prefix rounded down to 32 (the block
    holds the prompt's tail and masks, runtime.py:719-739 per sequence)."""
    import numpy as np
    import torch

    from fast_dllm_relax_amd.config import DEFAULT_MASK_ID, fast_dllm_v2_1p5b
    from fast_dllm_relax_amd.params import random_params_torch
    from fast_dllm_relax_amd.runtime import (_embed, batched_shifted_confidence, batched_shifted_confidence_rows,
                                             relax_batched_block_refine)
    from fast_dllm_relax_amd.vm import HipVM

    cfg = fast_dllm_v2_1p5b(tie_word_embeddings=False)
    log("batched: generating fp16 weights (seed 3)")
    params = random_params_torch(cfg, BATCH_SEED, dtype="float16", device="cuda", std=0.02, lm_head_std=0.5)
    vm = HipVM(cfg, params, dtype="float16", max_rows=1024)
    rng = np.random.default_rng(BATCH_SEED)
    prefixes = [int(p) for p in rng.integers(128, 1025, BATCH_SEQS)]
    prompts = [rng.integers(0, 150000, p).tolist() for p in prefixes]

    def run():
        timing: dict = {}
        blocks, stats = relax_batched_block_refine(vm, prompts, mask_id=DEFAULT_MASK_ID, block_size=32,
                                                   small_block_size=8, threshold=0.9, timing=timing)
        return stats, timing

    for i in range(args.warmup):
        log(f"batched: warmup {i + 1}/{args.warmup}")
        run()
    unmasked, refine_s, prefill_s, steps, partial_steps = 0, 0.0, 0.0, 0, 0
    for i in range(args.steps):
        stats, timing = run()
        unmasked += stats["unmasked"]
        refine_s += timing["refine_s"]
        prefill_s += timing["prefill_s"]
        steps += stats["steps"]
        partial_steps += stats["partial_steps"]
        log(f"batched: run {i + 1}/{args.steps}: {stats['unmasked']} tokens in {stats['steps']} steps "
            f"({stats['partial_steps']} partial), refine {timing['refine_s'] * 1e3:.1f} ms, "
            f"prefill {timing['prefill_s'] * 1e3:.1f} ms")

    # synced batched steps over a freshly built batched cache
    a0s = [p - p % 32 for p in prefixes]  # the block start of relax_batched_block_refine
    cap = max(a0s) + 32
    shape = (cfg.num_hidden_layers, BATCH_SEQS, cap, cfg.num_key_value_heads, cfg.head_dim)
    k = torch.zeros(shape, dtype=torch.float16, device="cuda")
    v = torch.zeros_like(k)
    for b in range(BATCH_SEQS):
        vm.build_prefix_cache_seq(_embed(vm, prompts[b][:a0s[b]]), None, k, v, b)
    ids = rng.integers(0, 150000, BATCH_SEQS * 32).tolist()
    emb = _embed(vm, ids).view(BATCH_SEQS, 32, -1)
    emb8 = emb[:, 8:16].contiguous()
    off = torch.tensor(a0s, dtype=torch.int32, device="cuda")
    off8 = off + 8
    full_ms = event_ms(lambda: batched_shifted_confidence(vm, vm.forward_cached_batch(emb, k, v, off, a0s)), 10)
    part_ms = event_ms(lambda: batched_shifted_confidence(
        vm, vm.forward_block_partial_batch(8, emb8, k, v, off8, a0s)), 10)
    # the loop's full step: the same forward, the confidence of one 8-row sub-block per sequence only
    sub_ms = event_ms(lambda: batched_shifted_confidence_rows(vm, vm.forward_cached_batch(emb, k, v, off, a0s), 8, 16), 10)

    H, I, V, L = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size, cfg.num_hidden_layers
    qkv = (cfg.num_attention_heads + 2 * cfg.num_key_value_heads) * cfg.head_dim
    gemm_params = L * (qkv * H + H * cfg.num_attention_heads * cfg.head_dim + 2 * I * H + H * I) + V * H

    def flops(rows, attend):
        att = sum(L * 4 * cfg.num_attention_heads * rows * (a0 + attend) * cfg.head_dim for a0 in a0s)
        return 2.0 * BATCH_SEQS * rows * gemm_params + att

    f_full, f_part = flops(32, 32), flops(8, 32)
    tf_full = f_full / (full_ms * 1e-3) / 1e12
    tf_part = f_part / (part_ms * 1e-3) / 1e12
    res = {
        "workload": f"BASELINE config 4: 1.5B fp16, seed 3, {BATCH_SEQS} sequences, prefixes U[128, 1024], one "
                    f"32-token block each starting at the prefix rounded down to 32 (the prompt's tail + masks), "
                    f"sub-blocks of 8, threshold 0.9, untied lm_head N(0, 0.5) (BASELINE.json: tied head); the loop's "
                    f"full steps score only the sub-block's rows (step_full_ms: confidence of all 512 rows; "
                    f"step_full_subblock_ms: of rows 8..15 of each sequence, as the loop's full steps do)",
        "prefixes": prefixes,
        "tokens_per_s": round(unmasked / refine_s, 2), "tokens": unmasked, "refine_s": round(refine_s, 4),
        "steps": steps, "partial_steps": partial_steps,
        "prefill_ms_mean": round(prefill_s / args.steps * 1e3, 2),
        "step_full_ms": round(full_ms, 4), "step_full_rows": BATCH_SEQS * 32,
        "step_full_subblock_ms": round(sub_ms, 4),
        "step_full_tflops": round(tf_full, 1), "step_full_mfma_frac": round(tf_full / MFMA_F16_PEAK_TFLOPS, 4),
        "step_partial_ms": round(part_ms, 4), "step_partial_rows": BATCH_SEQS * 8,
        "step_partial_tflops": round(tf_part, 1),
        "mfma_peak_tflops": MFMA_F16_PEAK_TFLOPS,
    }
    log(f"batched: {res['tokens_per_s']} tokens/s, full step {full_ms:.3f} ms = {tf_full:.1f} TFLOP/s, "
        f"partial {part_ms:.3f} ms")
    vm.close()
    return res


def profile_target(which: str, args) -> int:
    """Short workloads for rocprofv3 (the commands in profiles/ name them)."""
    import numpy as np
    import torch

    from fast_dllm_relax_amd.config import DEFAULT_MASK_ID, fast_dllm_v2_1p5b
    from fast_dllm_relax_amd.params import random_params_torch
    from fast_dllm_relax_amd.runtime import (_embed, batched_shifted_confidence, build_prefix_cache_from_ids,
                                             relax_greedy_generate)
    from fast_dllm_relax_amd.vm import HipVM

    if which == "decode":
        cfg = fast_dllm_v2_1p5b(tie_word_embeddings=False)
        params = random_params_torch(cfg, SEED, dtype="bfloat16", device="cuda", std=0.02, lm_head_std=0.5)
        vm = HipVM(cfg, params, dtype="bfloat16", max_rows=args.prefix)
        prompt = np.random.default_rng(SEED).integers(0, 150000, args.prefix).tolist()
        for i in range(2):
            out, stats = relax_greedy_generate(vm, prompt, max_new_tokens=args.new_tokens, block_size=32,
                                               small_block_size=8, threshold=0.9, mask_id=DEFAULT_MASK_ID,
                                               stop_token=None, device_loop=not args.host_loop)
            torch.cuda.synchronize()
            log(f"profile target: generation {i + 1}/2 done ({len(out)} tokens, {stats['block_recomputes']} calls)")
        return 0

    if which == "decode-gaps":
        return decode_gap_events(args)

    if which == "prefill8192":
        cfg = fast_dllm_v2_1p5b()
        vm = HipVM(cfg, random_params_torch(cfg, 4, dtype="bfloat16", device="cuda"), dtype="bfloat16", max_rows=8192)
        ids = np.random.default_rng(4).integers(0, 150000, 8192).tolist()
        for i in range(2):
            build_prefix_cache_from_ids(vm, ids, block_size=32, capacity=8192 + 64)
            torch.cuda.synchronize()
            log(f"profile target: prefill {i + 1}/2 done")
        return 0
    # config 4's batched steps over the config's prefixes (fp16, seed 3)
    cfg = fast_dllm_v2_1p5b(tie_word_embeddings=False)
    vm = HipVM(cfg, random_params_torch(cfg, BATCH_SEED, dtype="float16", device="cuda", lm_head_std=0.5),
               dtype="float16", max_rows=1024)
    rng = np.random.default_rng(BATCH_SEED)
    prefixes = [int(p) for p in rng.integers(128, 1025, BATCH_SEQS)]
    a0s = [p - p % 32 for p in prefixes]
    shape = (cfg.num_hidden_layers, BATCH_SEQS, max(a0s) + 32, cfg.num_key_value_heads, cfg.head_dim)
    k = torch.zeros(shape, dtype=torch.float16, device="cuda")
    v = torch.zeros_like(k)
    for b in range(BATCH_SEQS):
        vm.build_prefix_cache_seq(_embed(vm, rng.integers(0, 150000, a0s[b]).tolist()), None, k, v, b)
    emb = _embed(vm, rng.integers(0, 150000, BATCH_SEQS * 32).tolist()).view(BATCH_SEQS, 32, -1)
    emb8 = emb[:, 8:16].contiguous()
    off = torch.tensor(a0s, dtype=torch.int32, device="cuda")
    for _ in range(5):
        batched_shifted_confidence(vm, vm.forward_cached_batch(emb, k, v, off, a0s))
    for _ in range(5):
        batched_shifted_confidence(vm, vm.forward_block_partial_batch(8, emb8, k, v, off + 8, a0s))
    torch.cuda.synchronize()
    log("profile target: 5 full + 5 partial batched steps done")
    return 0


def decode_gap_events(args) -> int:
    """GPU time between the decode loop's model calls without a profiler: the C ABI calls of the device
    loop go through a wrapper that records an event on the stream right after each call's fused
    confidence + unmask launch and right before the next call's first launch.  The time between the two
    events is the GPU's idle time plus what the stream runs in between (the embedding of the next rows),
    and the events' own recording adds about a microsecond."""
    import numpy as np
    import torch

    from fast_dllm_relax_amd.config import DEFAULT_MASK_ID, fast_dllm_v2_1p5b
    from fast_dllm_relax_amd.params import random_params_torch
    from fast_dllm_relax_amd.runtime import relax_greedy_generate
    from fast_dllm_relax_amd.vm import HipVM

    cfg = fast_dllm_v2_1p5b(tie_word_embeddings=False)
    params = random_params_torch(cfg, SEED, dtype="bfloat16", device="cuda", std=0.02, lm_head_std=0.5)
    vm = HipVM(cfg, params, dtype="bfloat16", max_rows=args.prefix)
    prompt = np.random.default_rng(SEED).integers(0, 150000, args.prefix).tolist()
    lib, marks = vm.lib, []

    def mark(kind):
        e = torch.cuda.Event(enable_timing=True)
        e.record()
        marks.append((kind, e))

    class Marked:
        def __getattr__(self, name):
            return getattr(lib, name)

        def fdllm_get_confidence_unmask(self, *a):
            rc = lib.fdllm_get_confidence_unmask(*a)
            mark("end")
            return rc

        def fdllm_forward_cached(self, *a):
            mark("start")
            return lib.fdllm_forward_cached(*a)

        def fdllm_forward_block_partial(self, *a):
            mark("start")
            return lib.fdllm_forward_block_partial(*a)

    vm.lib = Marked()
    res = []
    for i in range(3):
        marks.clear()
        _, stats = relax_greedy_generate(vm, prompt, max_new_tokens=args.new_tokens, block_size=32,
                                         small_block_size=8, threshold=0.9, mask_id=DEFAULT_MASK_ID, stop_token=None)
        torch.cuda.synchronize()
        gaps = sorted(e1.elapsed_time(e2) * 1e3 for (k1, e1), (k2, e2) in zip(marks, marks[1:])
                      if k1 == "end" and k2 == "start")
        q = lambda v, f: v[min(len(v) - 1, int(f * len(v)))]  # noqa: E731
        res.append({"generation": i, "calls": stats["block_recomputes"], "gaps": len(gaps),
                    "gap_us_median": round(statistics.median(gaps), 1), "gap_us_p10": round(q(gaps, 0.1), 1),
                    "gap_us_p90": round(q(gaps, 0.9), 1), "gap_ms_sum": round(sum(gaps) / 1e3, 3)})
        log(json.dumps(res[-1]))
    print(json.dumps({"decode_gaps": res}))
    return 0


def trace_gaps(path: str) -> int:
    """GPU idle time between model calls of the decode loop, from a rocprofv3 kernel trace (csv).

    A model call starts with its first layer-loop kernel (load_rows_kernel) and ends with the confidence
    reduction (confidence_unmask_kernel on the device loop, confidence_combine_kernel on the host loop).
    The gap is the time from the end of one call's last kernel to the start of the next call's first,
    over the calls of the last generation in the trace (the loop's steady state); it holds whatever the
    host does in between (readback, unmask, uploads, the embedding of the next rows, the launch of the
    next call)."""
    import csv

    rows = []
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"]))
    rows.sort()
    calls, cur = [], None
    for s, e, n in rows:
        if "load_rows_kernel" in n:
            cur = [s, None, 0]
        if cur is None:
            continue
        cur[2] += e - s
        if "confidence_unmask_kernel" in n or "confidence_combine_kernel" in n:
            cur[1] = e
            calls.append(cur)
            cur = None
    # the last generation: calls after the last prefill-sized gap (> 5 ms)
    start = 0
    for i in range(1, len(calls)):
        if calls[i][0] - calls[i - 1][1] > 5_000_000:
            start = i
    calls = calls[start:]
    gaps = sorted((b[0] - a[1]) / 1e3 for a, b in zip(calls, calls[1:]))
    spans = [(c[1] - c[0]) / 1e3 for c in calls]
    busy = [c[2] / 1e3 for c in calls]
    if not gaps:
        print(json.dumps({"calls": len(calls), "error": "fewer than two model calls in the trace"}))
        return 1
    q = lambda v, f: v[min(len(v) - 1, int(f * len(v)))]  # noqa: E731
    out = {"calls": len(calls), "gap_us_median": round(statistics.median(gaps), 1),
           "gap_us_mean": round(statistics.mean(gaps), 1), "gap_us_p10": round(q(gaps, 0.1), 1),
           "gap_us_p90": round(q(gaps, 0.9), 1), "call_span_us_median": round(statistics.median(spans), 1),
           "call_kernel_busy_us_median": round(statistics.median(busy), 1),
           "gap_share_of_loop": round(sum(gaps) / (sum(spans) + sum(gaps)), 4)}
    print(json.dumps(out))
    return 0


def traffic_probe(vm, cfg) -> int:
    """One pass of the dominant kernel over the layers, then a plain copy of 256 MiB (the counter scale)."""
    import torch

    stream = torch.cuda.current_stream().cuda_stream
    _lib = vm_lib()
    _lib.check(vm.lib.fdllm_bench_op(vm.ctx, _lib.OP_GATE_UP, 32, 0, cfg.num_hidden_layers, None, None, 0, 0, stream))
    src = torch.ones(128 << 20, dtype=torch.bfloat16, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    log("traffic probe done: 28 gate_up launches, 3 copies of 256 MiB")
    return 0


def traffic_probe_step(vm, cfg) -> int:
    """The 2048-row prefix, a plain 256 MiB copy (the counters' scale), then one 32-row refinement step."""
    import numpy as np
    import torch

    from fast_dllm_relax_amd.runtime import build_prefix_cache_from_ids, score_active_block_refine

    rng = np.random.default_rng(SEED)
    cache = build_prefix_cache_from_ids(vm, rng.integers(0, 150000, PREFIX).tolist(), block_size=32,
                                        capacity=PREFIX + 32)
    block = rng.integers(0, 150000, 32).tolist()
    score_active_block_refine(vm, block, cache)  # warm-up: every buffer of the step allocated
    src = torch.ones(128 << 20, dtype=torch.bfloat16, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    score_active_block_refine(vm, block, cache)
    torch.cuda.synchronize()
    log("traffic probe done: prefix, one 256 MiB copy, one 32-row refinement step")
    return 0


def traffic_report(fetch_csv: str, write_csv: str) -> int:
    """Per-kernel FETCH_SIZE / WRITE_SIZE of the refinement step that follows the last 256 MiB copy in two
    `--traffic-probe step` counter runs, each scaled by what the counter reads for that copy."""
    import csv

    import __graft_entry__

    __graft_entry__.load_package()
    from fast_dllm_relax_amd.config import fast_dllm_v2_1p5b

    copy_bytes = 256 << 20

    def load(path, counter):
        rows = []
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                if r["Counter_Name"] == counter:
                    rows.append((int(r["Dispatch_Id"]), r["Kernel_Name"], float(r["Counter_Value"]) * 1024.0))
        rows.sort()
        # the calibration copy: the largest dispatch of a copy kernel (the step's own readback is tiny)
        copies = [i for i, (_, n, _) in enumerate(rows) if "copyBuffer" in n]
        if not copies:
            raise SystemExit(f"{path}: no calibration copy found")
        cal = max(copies, key=lambda i: rows[i][2])
        return rows[cal][2], rows[cal + 1:]

    fcopy, fstep = load(fetch_csv, "FETCH_SIZE")
    wcopy, wstep = load(write_csv, "WRITE_SIZE")
    fs, ws = copy_bytes / fcopy, copy_bytes / wcopy

    def short(n):
        n = n.split("(")[0].replace("void ", "").replace("fdllm::", "")
        return n[:60]

    per = {}
    for _, n, v in fstep:
        e = per.setdefault(short(n), [0, 0.0, 0.0])
        e[0] += 1
        e[1] += v * fs
    for _, n, v in wstep:
        per.setdefault(short(n), [0, 0.0, 0.0])[2] += v * ws
    total = sum(e[1] + e[2] for e in per.values())
    cfg = fast_dllm_v2_1p5b(tie_word_embeddings=False)
    algo = cfg.step_bytes(32, PREFIX)
    print("| kernel | dispatches | fetched MB | written MB |")
    print("|---|---|---|---|")
    for n, (cnt, fb, wb) in sorted(per.items(), key=lambda kv: -(kv[1][1] + kv[1][2])):
        print(f"| `{n}` | {cnt} | {fb / 1e6:.2f} | {wb / 1e6:.2f} |")
    print(json.dumps({"fetch_scale": round(fs, 4), "write_scale": round(ws, 4), "step_traffic_bytes": int(total),
                      "algorithmic_bytes": algo, "ratio": round(total / algo, 4)}))
    return 0


def vm_lib():
    from fast_dllm_relax_amd import _lib

    return _lib


def measured_step_traffic():
    """HBM bytes of one 32-row refinement step at prefix 2048 from the committed rocprofv3 --pmc summary
    (profiles/step_traffic_p2048.md, line 'step_traffic_bytes: N'), or None."""
    path = ROOT / "profiles" / "step_traffic_p2048.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.strip().startswith("step_traffic_bytes:"):
            return int(line.split(":", 1)[1].strip().strip("`"))
    return None


def measured_traffic():
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3 --pmc summary
    (profiles/gate_up_traffic.md, line 'traffic_bytes_per_launch: N'), or None."""
    path = ROOT / "profiles" / "gate_up_traffic.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.strip().startswith("traffic_bytes_per_launch:"):
            return int(line.split(":", 1)[1].strip().strip("`"))
    return None


def hf_reference_model(cfg, params, dtype):
    """transformers' Qwen2ForCausalLM built from a Qwen2Config (no download) with the weights of ``params``
    (host tensors in the packed parameter order), q/k/v and gate/up split back out of the fused tensors:
    the reference model's HF counterpart on the host.  Constructed on the meta device and then given the
    weights, so no random initialisation is spent on 1.5B parameters."""
    import torch
    from transformers import Qwen2Config, Qwen2ForCausalLM

    from fast_dllm_relax_amd.params import param_names

    hc = Qwen2Config(vocab_size=cfg.vocab_size, hidden_size=cfg.hidden_size, intermediate_size=cfg.intermediate_size,
                     num_hidden_layers=cfg.num_hidden_layers, num_attention_heads=cfg.num_attention_heads,
                     num_key_value_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim, rms_norm_eps=cfg.rms_norm_eps,
                     rope_theta=cfg.rope_theta, tie_word_embeddings=cfg.tie_word_embeddings,
                     max_position_embeddings=max(4096, 2 * cfg.bd_size), attn_implementation="sdpa")
    with torch.device("meta"):
        model = Qwen2ForCausalLM(hc)
    model = model.to_empty(device="cpu")
    arr = dict(zip(param_names(cfg), params))
    qd, kd = cfg.num_attention_heads * cfg.head_dim, cfg.num_key_value_heads * cfg.head_dim
    inter = cfg.intermediate_size
    sd = {"model.embed_tokens.weight": arr["model.embed_tokens.weight"], "model.norm.weight": arr["model.norm.weight"]}
    if not cfg.tie_word_embeddings:
        sd["lm_head.weight"] = arr["lm_head.weight"]
    for i in range(cfg.num_hidden_layers):
        pre = f"model.layers.{i}"
        w, b = arr[f"{pre}.self_attn.qkv_proj.weight"], arr[f"{pre}.self_attn.qkv_proj.bias"]
        sd[f"{pre}.self_attn.q_proj.weight"], sd[f"{pre}.self_attn.q_proj.bias"] = w[:qd], b[:qd]
        sd[f"{pre}.self_attn.k_proj.weight"], sd[f"{pre}.self_attn.k_proj.bias"] = w[qd:qd + kd], b[qd:qd + kd]
        sd[f"{pre}.self_attn.v_proj.weight"], sd[f"{pre}.self_attn.v_proj.bias"] = w[qd + kd:], b[qd + kd:]
        sd[f"{pre}.self_attn.o_proj.weight"] = arr[f"{pre}.self_attn.o_proj.weight"]
        gu = arr[f"{pre}.mlp.gate_up_proj.weight"]
        sd[f"{pre}.mlp.gate_proj.weight"], sd[f"{pre}.mlp.up_proj.weight"] = gu[:inter], gu[inter:]
        sd[f"{pre}.mlp.down_proj.weight"] = arr[f"{pre}.mlp.down_proj.weight"]
        sd[f"{pre}.input_layernorm.weight"] = arr[f"{pre}.input_layernorm.weight"]
        sd[f"{pre}.post_attention_layernorm.weight"] = arr[f"{pre}.post_attention_layernorm.weight"]
    sd = {k: v.to(dtype).contiguous() for k, v in sd.items()}
    missing, unexpected = model.load_state_dict(sd, strict=False, assign=True)
    if unexpected or not set(missing) <= {"lm_head.weight"}:
        raise RuntimeError(f"HF weight mapping: missing {missing}, unexpected {unexpected}")
    if cfg.tie_word_embeddings:
        model.tie_weights()
    # the rotary buffers were left uninitialised by to_empty: rebuild them from the config
    model.model.rotary_emb = type(model.model.rotary_emb)(config=hc)
    return model.to(dtype).eval()


def hf_cached_step(model, k_prefix, v_prefix, block_ids, P):
    """One HF cached refinement step: a DynamicCache holding the P-row prefix (k/v [L, 1, P, nkv, hd], the
    reference's inplace_bsnh layout, after RoPE as HF caches keys), then the 32-row block forward with the
    all-allowed mask of the cached step and RoPE positions P.. (runtime.py:333-343), lm_head included.
    Returns (logits [rows, vocab] fp32, the forward's seconds)."""
    import torch
    from transformers import DynamicCache

    dt = next(model.parameters()).dtype
    cache = DynamicCache(config=model.config)
    for layer in range(k_prefix.shape[0]):
        cache.update(k_prefix[layer, 0].transpose(0, 1)[None].to(dt), v_prefix[layer, 0].transpose(0, 1)[None].to(dt),
                     layer)
    rows = len(block_ids)
    ids = torch.tensor([block_ids], dtype=torch.long)
    mask = {"full_attention": torch.zeros((1, 1, rows, P + rows), dtype=dt)}
    with torch.no_grad():
        t0 = time.perf_counter()
        out = model(input_ids=ids, position_ids=torch.arange(P, P + rows)[None], past_key_values=cache,
                    attention_mask=mask, use_cache=True)
        sec = time.perf_counter() - t0
    return out.logits[0].float(), sec


def cpu_baseline(vm, params, cache, block, P, iters, tokens_per_call):
    """The CPU baseline: the reference model's step on the host, on the same weights and KV-cache prefix as the GPU run,
    all host cores: the HF reference forward (transformers' Qwen2, one 32-row cached forward + lm_head
    against the P-row prefix) in bf16 and fp32, and this build's numpy oracle for the same step.  Medians
    of ``iters`` (>= 5) after one warm-up each; tokens/s uses the GPU loop's tokens per model call."""
    import numpy as np
    import torch
    from threadpoolctl import threadpool_info

    from oracle import confidence as oconf
    from oracle.model import OracleConfig, OracleModel, param_names

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    c = vm.cfg
    log("cpu baseline: copying weights and cache to the host")
    host = [p.cpu() for p in params]
    kpre = cache.k[:, :, :P].cpu()
    vpre = cache.v[:, :, :P].cpu()
    res = {}

    def med(fn, n):
        fn()  # warm-up
        ts = []
        for i in range(n):
            ts.append(fn())
            log(f"cpu baseline step {i + 1}/{n}: {ts[-1]:.3f} s")
        return statistics.median(ts)

    for name, dt in (("bf16", torch.bfloat16), ("fp32", torch.float32)):
        log(f"cpu baseline: HF Qwen2 {name}")
        model = hf_reference_model(c, host, dt)
        res[name] = med(lambda: hf_cached_step(model, kpre, vpre, block, P)[1], iters)
        del model
    log("cpu baseline: numpy oracle")
    ocfg = OracleConfig(vocab_size=c.vocab_size, hidden_size=c.hidden_size, intermediate_size=c.intermediate_size,
                        num_hidden_layers=c.num_hidden_layers, num_attention_heads=c.num_attention_heads,
                        num_key_value_heads=c.num_key_value_heads, head_dim=c.head_dim,
                        tie_word_embeddings=c.tie_word_embeddings)
    arrays = {n: p.float().numpy() for n, p in zip(param_names(ocfg), host)}
    model = OracleModel(ocfg, arrays, "bfloat16")
    kc = torch.cat([kpre, torch.zeros_like(kpre[:, :, :32])], 2).float().numpy()
    vc = torch.cat([vpre, torch.zeros_like(vpre[:, :, :32])], 2).float().numpy()
    emb = model.embed(block)[None]

    def oracle_step():
        t0 = time.perf_counter()
        h = model.forward_cached(emb, kc, vc, P, P)
        oconf.shifted_confidence(model.get_logits(h)[0])
        return time.perf_counter() - t0

    port_s = med(oracle_step, max(2, iters // 2))
    blas = max([d.get("num_threads", 1) for d in threadpool_info()] or [1])
    del arrays, model, host
    torch.cuda.empty_cache()
    return {"value": round(tokens_per_call / res["bf16"], 3), "unit": "tokens/s", "cores": threads,
            "kind": "reference",
            "step_s_bf16": round(res["bf16"], 4), "step_s_fp32": round(res["fp32"], 4),
            "value_fp32": round(tokens_per_call / res["fp32"], 3),
            "port_step_s": round(port_s, 4), "port_value": round(tokens_per_call / port_s, 3), "port_cores": int(blas),
            "host_cpus": os.cpu_count(),
            "sample": f"HF reference forward: transformers {_hf_version()} Qwen2ForCausalLM "
                      f"from a Qwen2Config with the bench weights, one 32-row cached forward + lm_head against a "
                      f"{P}-row DynamicCache (the GPU-built prefix), torch threads = {threads}; median of {iters} "
                      f"after 1 warm-up, bf16 (value) and fp32; tokens/s = {tokens_per_call:.3f} tokens per model "
                      f"call (the GPU loop's) / step time.  port_*: this build's numpy oracle, same step"}


def _hf_version():
    import transformers

    return transformers.__version__


if __name__ == "__main__":
    sys.exit(main())
