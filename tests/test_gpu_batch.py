"""Batched cached steps (a build extension: the reference's entry points are batch 1, cuda.py:796-836).

Each sequence of a batched call follows the batch-1 semantics exactly, so the oracle is the batch-1
oracle run per sequence; calls go through the C ABI."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import TINY, WIDE2, bf16_parity, log, make_pair, to_np
from oracle.model import build_prefix_block_attention_bias

pytestmark = pytest.mark.gpu

SENTINEL = 7.0


def _dev_ids(ids):
    return torch.tensor(np.asarray(ids), dtype=torch.int32, device="cuda")


def _batched_case(ref, vm, kw, prefixes, seed, label):
    rng = np.random.default_rng(seed)
    L, nkv, hd = kw["num_hidden_layers"], kw["num_key_value_heads"], kw["head_dim"]
    B, R = len(prefixes), 32
    cap = max(prefixes) + 2 * R
    ids = [rng.integers(0, kw["vocab_size"] - 1, P + R) for P in prefixes]

    want_h, want_k, want_v = [], [], []
    for b, P in enumerate(prefixes):
        kc = np.zeros((L, 1, cap, nkv, hd), np.float32)
        vc = kc.copy()
        ref.build_prefix_cache(ref.embed(ids[b][:P])[None], build_prefix_block_attention_bias(0, P, block_size=32),
                               kc, vc)
        want_h.append(ref.forward_cached(ref.embed(ids[b][P:])[None], kc, vc, P, P)[0])
        want_k.append(kc[:, 0])
        want_v.append(vc[:, 0])

    k = torch.full((L, B, cap, nkv, hd), SENTINEL, dtype=vm.torch_dtype, device="cuda")
    v = torch.full_like(k, SENTINEL)
    log(f"case: {label} build_prefix_cache_seq x {B} (prefixes {prefixes})")
    for b, P in enumerate(prefixes):
        vm.build_prefix_cache_seq(vm.embed(_dev_ids(ids[b][:P]))[None], None, k, v, b)
    x = torch.stack([vm.embed(_dev_ids(ids[b][P:])) for b, P in enumerate(prefixes)])
    off = torch.tensor(prefixes, dtype=torch.int32, device="cuda")
    log(f"case: {label} forward_cached_batch nseq={B} rows={R}")
    h = vm.forward_cached_batch(x, k, v, off, prefixes)
    kn, vn = to_np(k), to_np(v)
    for b, P in enumerate(prefixes):
        bf16_parity(f"{label} seq {b} hidden", to_np(h[b]), want_h[b])
        bf16_parity(f"{label} seq {b} K", kn[:, b, :P + R], want_k[b][:, :P + R])
        bf16_parity(f"{label} seq {b} V", vn[:, b, :P + R], want_v[b][:, :P + R])
        assert (kn[:, b, P + R:] == SENTINEL).all() and (vn[:, b, P + R:] == SENTINEL).all(), \
            f"sequence {b}: rows past its window were written"

    # the partial step reproduces the full step's rows for the same tokens (cuda.py:740-756)
    rp = 8
    xp = x[:, rp:rp + 8].contiguous()
    offp = torch.tensor([P + rp for P in prefixes], dtype=torch.int32, device="cuda")
    log(f"case: {label} forward_block_partial_batch rp={rp}")
    hp = vm.forward_block_partial_batch(rp, xp, k, v, offp, prefixes)
    # the two calls run their projections at different M (different k splits), so bf16 roundings
    # can differ by an ulp: the bf16 criterion, not an element-wise bound
    bf16_parity(f"{label} partial rows vs full-step rows", to_np(hp), to_np(h[:, rp:rp + 8]))
    return h


@pytest.fixture(scope="module")
def tiny():
    log("setup: tiny bf16 model seed 0")
    return make_pair(TINY, 0)


def test_batched_step_matches_oracle_per_sequence(tiny):
    ref, vm = tiny
    _batched_case(ref, vm, TINY, [32, 96, 64], 21, "tiny")


def test_batched_window_errors(tiny):
    _, vm = tiny
    c = vm.cfg
    k = torch.zeros((c.num_hidden_layers, 2, 96, c.num_key_value_heads, c.head_dim), dtype=vm.torch_dtype,
                    device="cuda")
    v = torch.zeros_like(k)
    x = torch.zeros((2, 32, c.hidden_size), dtype=vm.torch_dtype, device="cuda")
    off = torch.tensor([32, 80], dtype=torch.int32, device="cuda")
    log("case: batched write past capacity names the sequence")
    with pytest.raises(ValueError, match="sequence 1"):
        vm.forward_cached_batch(x, k, v, off, [32, 80])
    with pytest.raises(ValueError):
        vm.forward_block_partial_batch(8, x, k, v, off, [32, 32])  # 32 rows where 8 are required
    with pytest.raises(ValueError):
        vm.forward_cached_batch(x, k, v, off, [32])  # one prefix length for two sequences


def test_batched_loop_equals_batch1_loop(tiny):
    """One sequence through the batched loop runs the batch-1 kernels, so its tokens equal the batch-1
    loop's (relax_greedy_generate over the same block) exactly; several sequences unmask every row."""
    from fast_dllm_relax_amd.runtime import relax_batched_block_refine, relax_greedy_generate

    _, vm = tiny
    rng = np.random.default_rng(5)
    mask_id = TINY["vocab_size"] - 1
    prompt = [int(t) for t in rng.integers(0, mask_id, 45)]
    log("case: batched loop, one sequence vs relax_greedy_generate")
    blocks, stats = relax_batched_block_refine(vm, [prompt], mask_id=mask_id)
    n_new = 64 - len(prompt)
    # the batch-1 loop counts masked rows as generated (runtime.py:841-843): ask for one more block so that
    # the first block is refined to the end
    cont, _ = relax_greedy_generate(vm, prompt, max_new_tokens=n_new + 32, mask_id=mask_id, stop_token=None)
    got = [int(t) for t in blocks[0]]
    assert got[:len(prompt) - 32] == prompt[32:]
    want = [int(t) for t in cont]
    assert got[len(prompt) - 32:] == want[:n_new], (got, want)
    log("case: batched loop, three sequences")
    prompts = [[int(t) for t in rng.integers(0, mask_id, n)] for n in (33, 64, 90)]
    blocks, stats = relax_batched_block_refine(vm, prompts, mask_id=mask_id)
    assert stats["steps"] >= 4
    for p, blk in zip(prompts, blocks):
        a0 = len(p) - len(p) % 32 if len(p) % 32 else len(p)
        assert mask_id not in blk
        assert blk[:len(p) - a0] == p[a0:]


@pytest.fixture(scope="module")
def wide2():
    log("setup: 1.5B-shape 2-layer bf16 model seed 1")
    return make_pair(WIDE2, 1)


def test_wide_batched_step_16_sequences(wide2):
    """16 sequences x 32 rows: the projections run at M = 512 (the MFMA block kernel, with k splits)."""
    ref, vm = wide2
    rng = np.random.default_rng(3)
    prefixes = [int(p) for p in 32 * rng.integers(1, 5, 16)]
    h = _batched_case(ref, vm, WIDE2, prefixes, 31, "wide")
    # the confidence of all 512 rows (the lm_head at M = 512) is bit-exact given its own logits
    from oracle import confidence as oconf

    rows = h.shape[0] * h.shape[1]
    logits = torch.empty((1, rows, WIDE2["vocab_size"]), dtype=torch.float32, device="cuda")
    log("case: wide fused lm_head + confidence, 512 rows")
    ids, maxp = vm.get_confidence(h.view(1, rows, -1), logits=logits)
    wid, wp = oconf.confidence(to_np(logits)[0])
    np.testing.assert_array_equal(ids.cpu().numpy()[0], wid)
    np.testing.assert_array_equal(maxp.cpu().numpy()[0].view(np.uint32), wp.view(np.uint32))
    # the batched loop's full steps take the confidence of the sub-block's logit rows only (the lm_head at
    # M = 112 or 128): the same bits as the shifted confidence of all 512 rows, sliced
    from fast_dllm_relax_amd.runtime import batched_shifted_confidence, batched_shifted_confidence_rows

    all_ids, all_p = batched_shifted_confidence(vm, h)
    for s0 in (0, 8, 16, 24):
        log(f"case: shifted confidence of rows [{s0}, {s0 + 8}) of 16 sequences vs all rows")
        sid, sp = batched_shifted_confidence_rows(vm, h, s0, s0 + 8)
        np.testing.assert_array_equal(sid, all_ids[:, s0:s0 + 8])
        np.testing.assert_array_equal(sp.view(np.uint32), all_p[:, s0:s0 + 8].view(np.uint32))


def test_seq_attention_kernel_matches_chunk_kernel(monkeypatch):
    """Batched calls take attn_seq_kernel by default: a workgroup streams its sequence's key blocks (the
    longest sequences' blocks split over the compute units the others leave idle, the splits merged by the
    last to arrive, in split order); FDLLM_SEQ_SPLIT=0 streams every key of a sequence through one
    workgroup, and FDLLM_SEQ_ATTN=0 keeps the chunk kernel with key splits and the merge launch.  All three
    append the same RoPE'd K/V rows at layer 0 (bit for bit) and agree on the hidden states, and so on later
    layers' appended rows, to the bf16 criterion (their fp32 softmax sums run in different orders).  The
    split kernel gives the same bits when the call is repeated (the arrival counters return to zero, and
    which split arrives last does not matter).  Prefixes off the 64-key block grid, up to 1000 keys, full
    (32-row) and partial (8-row) steps; 16 sequences of the 1.5B width."""
    from fast_dllm_relax_amd.config import FastDLLMConfig
    from fast_dllm_relax_amd.params import from_numpy
    from fast_dllm_relax_amd.vm import HipVM
    from oracle.model import OracleConfig, random_params

    kw = WIDE2
    params = from_numpy(random_params(OracleConfig(**kw), 4, "bfloat16"), FastDLLMConfig(**kw), dtype="bfloat16")
    vms = {}
    for name, on, split in (("seq", "1", "1"), ("nosplit", "1", "0"), ("chunk", "0", "1")):
        monkeypatch.setenv("FDLLM_SEQ_ATTN", on)
        monkeypatch.setenv("FDLLM_SEQ_SPLIT", split)
        vms[name] = HipVM(FastDLLMConfig(**kw), params, dtype="bfloat16", max_rows=512)
        monkeypatch.delenv("FDLLM_SEQ_ATTN")
        monkeypatch.delenv("FDLLM_SEQ_SPLIT")
    rng = np.random.default_rng(41)
    prefixes = [1000, 32, 96, 511, 200, 64, 992, 130, 700, 33, 257, 960, 448, 5, 640, 801]
    L, nkv, hd = kw["num_hidden_layers"], kw["num_key_value_heads"], kw["head_dim"]
    B, R = len(prefixes), 32
    cap = max(prefixes) + 2 * R
    ids = [rng.integers(0, kw["vocab_size"] - 1, P + R) for P in prefixes]
    out = {}
    for name, vm in vms.items():
        k = torch.full((L, B, cap, nkv, hd), SENTINEL, dtype=torch.bfloat16, device="cuda")
        v = torch.full_like(k, SENTINEL)
        log(f"case: {name} attention, build_prefix_cache_seq x {B}")
        for b, P in enumerate(prefixes):
            vm.build_prefix_cache_seq(vm.embed(_dev_ids(ids[b][:P]))[None], None, k, v, b)
        x = torch.stack([vm.embed(_dev_ids(ids[b][P:])) for b, P in enumerate(prefixes)])
        off = torch.tensor(prefixes, dtype=torch.int32, device="cuda")
        log(f"case: {name} attention, forward_cached_batch nseq={B} rows={R}")
        h = vm.forward_cached_batch(x, k, v, off, prefixes)
        if name == "seq":
            log("case: seq attention, the same call again (same bits)")
            h2 = vm.forward_cached_batch(x, k, v, off, prefixes)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(to_np(h2).view(np.uint16), to_np(h).view(np.uint16))
        kf, vf = to_np(k), to_np(v)
        offp = torch.tensor([P + 8 for P in prefixes], dtype=torch.int32, device="cuda")
        log(f"case: {name} attention, forward_block_partial_batch rp=8")
        hp = vm.forward_block_partial_batch(8, x[:, 8:16].contiguous(), k, v, offp, prefixes)
        torch.cuda.synchronize()
        out[name] = (to_np(h), kf, vf, to_np(hp))
    for other in ("chunk", "nosplit"):
        for i, what in ((1, "K cache"), (2, "V cache")):
            # layer 0's appended rows and every prefix row are the same bits; later layers' appended rows
            # follow hidden states that agree to the bf16 criterion
            np.testing.assert_array_equal(out["seq"][i][0], out[other][i][0], err_msg=f"{what}, layer 0")
            for b, P in enumerate(prefixes):
                np.testing.assert_array_equal(out["seq"][i][:, b, :P], out[other][i][:, b, :P],
                                              err_msg=f"{what}, sequence {b} prefix rows")
                assert (out["seq"][i][:, b, P + R:] == SENTINEL).all(), f"{what}, sequence {b}: rows past its window"
            bf16_parity(f"seq vs {other} attention, {what} appended rows",
                        np.stack([out["seq"][i][1:, b, P:P + R] for b, P in enumerate(prefixes)]),
                        np.stack([out[other][i][1:, b, P:P + R] for b, P in enumerate(prefixes)]))
        bf16_parity(f"seq vs {other} attention, full step hidden", out["seq"][0], out[other][0])
        bf16_parity(f"seq vs {other} attention, partial step hidden", out["seq"][3], out[other][3])
    assert np.isfinite(out["seq"][0]).all() and np.isfinite(out["seq"][3]).all()
    for vm in vms.values():
        vm.close()


def test_batched_step_beyond_one_step_key_split_plan(wide2):
    """A batched call whose longest prefix (8300 keys) is past the chunk kernel's one-step plan (64 chunks of
    128 keys): attn_seq_kernel streams every key, so the call runs; each sequence's hidden states match the
    batch-1 cached forward of the same sequence (the long-block loop kernel) to the bf16 criterion."""
    _, vm = wide2
    kw = WIDE2
    rng = np.random.default_rng(43)
    prefixes = [8300, 100]
    L, nkv, hd = kw["num_hidden_layers"], kw["num_key_value_heads"], kw["head_dim"]
    R = 32
    cap = max(prefixes) + R
    ids = [rng.integers(0, kw["vocab_size"] - 1, P + R) for P in prefixes]
    k = torch.zeros((L, len(prefixes), cap, nkv, hd), dtype=vm.torch_dtype, device="cuda")
    v = torch.zeros_like(k)
    log(f"case: batched step over prefixes {prefixes} (build_prefix_cache_seq)")
    for b, P in enumerate(prefixes):
        vm.build_prefix_cache_seq(vm.embed(_dev_ids(ids[b][:P]))[None], None, k, v, b)
    x = torch.stack([vm.embed(_dev_ids(ids[b][P:])) for b, P in enumerate(prefixes)])
    k1, v1 = k.clone(), v.clone()
    off = torch.tensor(prefixes, dtype=torch.int32, device="cuda")
    h = vm.forward_cached_batch(x, k, v, off, prefixes)
    torch.cuda.synchronize()
    for b, P in enumerate(prefixes):
        log(f"case: batch-1 forward_cached of sequence {b} (prefix {P})")
        kb = k1[:, b:b + 1].contiguous()
        vb = v1[:, b:b + 1].contiguous()
        hb = vm.forward_cached(x[b:b + 1], kb, vb, torch.tensor(P, dtype=torch.int32, device="cuda"), P)
        torch.cuda.synchronize()
        bf16_parity(f"batched vs batch-1, sequence {b} hidden", to_np(h[b]), to_np(hb[0]))
        bf16_parity(f"batched vs batch-1, sequence {b} K rows", to_np(k[:, b, P:P + R]), to_np(kb[:, 0, P:P + R]))


def test_batched_step_ragged_query_tiles(wide2):
    """40 rows per sequence: 240 stacked query rows per kv head, so the last query tile is part padding (and
    the chunk plan, at most 12 tiles, does not cover it); each sequence's hidden states and appended K rows
    match its batch-1 cached forward to the bf16 criterion."""
    _, vm = wide2
    kw = WIDE2
    rng = np.random.default_rng(47)
    prefixes, R = [64, 250, 97], 40
    L, nkv, hd = kw["num_hidden_layers"], kw["num_key_value_heads"], kw["head_dim"]
    cap = max(prefixes) + R
    ids = [rng.integers(0, kw["vocab_size"] - 1, P + R) for P in prefixes]
    k = torch.zeros((L, len(prefixes), cap, nkv, hd), dtype=vm.torch_dtype, device="cuda")
    v = torch.zeros_like(k)
    for b, P in enumerate(prefixes):
        vm.build_prefix_cache_seq(vm.embed(_dev_ids(ids[b][:P]))[None], None, k, v, b)
    x = torch.stack([vm.embed(_dev_ids(ids[b][P:])) for b, P in enumerate(prefixes)])
    k1, v1 = k.clone(), v.clone()
    log(f"case: batched step, {R} rows per sequence, prefixes {prefixes}")
    h = vm.forward_cached_batch(x, k, v, torch.tensor(prefixes, dtype=torch.int32, device="cuda"), prefixes)
    torch.cuda.synchronize()
    for b, P in enumerate(prefixes):
        kb, vb = k1[:, b:b + 1].contiguous(), v1[:, b:b + 1].contiguous()
        hb = vm.forward_cached(x[b:b + 1], kb, vb, torch.tensor(P, dtype=torch.int32, device="cuda"), P)
        torch.cuda.synchronize()
        bf16_parity(f"{R}-row batched vs batch-1, sequence {b} hidden", to_np(h[b]), to_np(hb[0]))
        bf16_parity(f"{R}-row batched vs batch-1, sequence {b} K rows", to_np(k[:, b, P:P + R]),
                    to_np(kb[:, 0, P:P + R]))
