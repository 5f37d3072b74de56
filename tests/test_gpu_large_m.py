"""The register-weight large-M GEMM against the LDS-staged and streaming large-M GEMMs.

By default gate_up and down run gemm_wr_kernel's 128 x 256 blocks from 2048 rows and qkv and o_proj from
4096 (FDLLM_WR_OPS selects the projections, one bit per GemmCfg; FDLLM_WR_MIN_ROWS lowers the threshold,
here to 256 so that ragged and small row counts take it too); below that qkv, and o_proj below 2048 rows,
run its 64 x 128 blocks, or up to 512 rows its 64 x 64 blocks (FDLLM_WR_SMALL, bits of qkv and o_proj).  Every large-M kernel accumulates each
output element's k steps in order in one MFMA chain and shares the epilogues, so with k splits off
(FDLLM_MM_TARGET_WGS=1) the hidden states must agree bit for bit whichever kernel ran.  Parity of the default configuration with the oracle is
established by the prefill, forward_hidden and batched-step tests."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import WIDE2, bf16_parity, log

pytestmark = pytest.mark.gpu


def _vm(kw, params, dtype, monkeypatch, wr_ops, max_rows, wr_small=0, wt8=0, wt256=0):
    from fast_dllm_relax_amd.config import FastDLLMConfig
    from fast_dllm_relax_amd.vm import HipVM

    monkeypatch.setenv("FDLLM_WR_OPS", str(wr_ops))
    monkeypatch.setenv("FDLLM_WR_MIN_ROWS", "256")
    monkeypatch.setenv("FDLLM_MM_TARGET_WGS", "1")
    monkeypatch.setenv("FDLLM_WR_SMALL", str(wr_small))
    monkeypatch.setenv("FDLLM_WT8", str(wt8))
    monkeypatch.setenv("FDLLM_WT256", str(wt256))
    vm = HipVM(FastDLLMConfig(**kw), params, dtype=dtype, max_rows=max_rows)
    for k in ("FDLLM_WR_OPS", "FDLLM_WR_MIN_ROWS", "FDLLM_MM_TARGET_WGS", "FDLLM_WR_SMALL", "FDLLM_WT8", "FDLLM_WT256"):
        monkeypatch.delenv(k)
    return vm


def _bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy()


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_register_weight_kernel_bit_identical(dtype, monkeypatch):
    from fast_dllm_relax_amd.config import FastDLLMConfig
    from fast_dllm_relax_amd.params import from_numpy
    from oracle.model import OracleConfig, random_params

    kw = WIDE2
    params = from_numpy(random_params(OracleConfig(**kw), 5, dtype), FastDLLMConfig(**kw), dtype=dtype)
    sizes = (300, 512, 1056)  # 64 x 64 blocks for qkv / o_proj up to 512 rows, 64 x 128 above
    vm_wr = _vm(kw, params, dtype, monkeypatch, 15, max(sizes))
    vm_old = _vm(kw, params, dtype, monkeypatch, 0, max(sizes))
    vm_small = _vm(kw, params, dtype, monkeypatch, 0, max(sizes), wr_small=3)  # 64 x 128 blocks for qkv, o_proj
    # gate_up and down on the LDS-staged kernel's eight-wave 128 x 192 blocks (waves copy 3 or 2 blocks a stage)
    vm_wt8 = _vm(kw, params, dtype, monkeypatch, 0, max(sizes), wt8=3)
    # gate_up up to 512 rows on 256 x 192 blocks of eight waves (waves copy 4 or 3 of a stage's 28 blocks)
    vm_256 = _vm(kw, params, dtype, monkeypatch, 0, max(sizes), wt256=512)  # (the default; vm_old: 0)
    rng = np.random.default_rng(17)
    for S in sizes:
        log(f"case: forward_hidden {S} rows, 1.5B width, 2 layers, {dtype}, register-weight vs LDS-staged")
        ids = torch.tensor(rng.integers(0, kw["vocab_size"] - 1, S), dtype=torch.int32, device="cuda")
        x = vm_old.embed(ids)[None]
        h_old = vm_old.forward_hidden(x, None)
        h_wr = vm_wr.forward_hidden(x, None)
        h_small = vm_small.forward_hidden(x, None)
        h_wt8 = vm_wt8.forward_hidden(x, None)
        h_256 = vm_256.forward_hidden(x, None)
        torch.cuda.synchronize()
        assert torch.isfinite(h_wr.float()).all()
        np.testing.assert_array_equal(_bits(h_wr), _bits(h_old), err_msg=f"S={S}")
        np.testing.assert_array_equal(_bits(h_small), _bits(h_old), err_msg=f"S={S}, 64 x 128 blocks")
        np.testing.assert_array_equal(_bits(h_wt8), _bits(h_old), err_msg=f"S={S}, eight-wave LDS-staged blocks")
        np.testing.assert_array_equal(_bits(h_256), _bits(h_old), err_msg=f"S={S}, 256 x 192 LDS-staged blocks")


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_small_m_ffn_register_weight_bit_identical(dtype, monkeypatch):
    """Below 256 rows gate_up and down take the register-weight kernel's 64 x 128 or 128 x 128 blocks by
    default (FDLLM_WR_FFN: bits 0 / 1 the 64 x 128 blocks for gate_up / down, bits 2 / 3 the 128 x 128 ones,
    0 the LDS-staged gemm_mm_kernel); with k splits off all three accumulate each output's k steps in
    order, so the hidden states agree bit for bit."""
    from fast_dllm_relax_amd.config import FastDLLMConfig
    from fast_dllm_relax_amd.params import from_numpy
    from fast_dllm_relax_amd.vm import HipVM
    from oracle.model import OracleConfig, random_params

    kw = WIDE2
    params = from_numpy(random_params(OracleConfig(**kw), 9, dtype), FastDLLMConfig(**kw), dtype=dtype)
    vms = {}
    for name, ffn in (("mm", 0), ("64x128", 3), ("128x128", 12)):
        monkeypatch.setenv("FDLLM_WR_FFN", str(ffn))
        monkeypatch.setenv("FDLLM_MM_TARGET_WGS", "1")
        vms[name] = HipVM(FastDLLMConfig(**kw), params, dtype=dtype, max_rows=256)
        monkeypatch.delenv("FDLLM_WR_FFN")
        monkeypatch.delenv("FDLLM_MM_TARGET_WGS")
    rng = np.random.default_rng(19)
    for S in (40, 100, 200):
        log(f"case: forward_hidden {S} rows, 1.5B width, 2 layers, {dtype}, FFN register-weight blocks vs gemm_mm")
        ids = torch.tensor(rng.integers(0, kw["vocab_size"] - 1, S), dtype=torch.int32, device="cuda")
        x = vms["mm"].embed(ids)[None]
        h = {name: vm.forward_hidden(x, None) for name, vm in vms.items()}
        torch.cuda.synchronize()
        assert torch.isfinite(h["64x128"].float()).all()
        for name in ("64x128", "128x128"):
            np.testing.assert_array_equal(_bits(h[name]), _bits(h["mm"]), err_msg=f"S={S}, {name}")
    for vm in vms.values():
        vm.close()


def _prefill_vm(kw, params, dtype, monkeypatch, pair, max_rows):
    from fast_dllm_relax_amd.config import FastDLLMConfig
    from fast_dllm_relax_amd.vm import HipVM

    monkeypatch.setenv("FDLLM_PREFILL_PAIR", str(pair))
    vm = HipVM(FastDLLMConfig(**kw), params, dtype=dtype, max_rows=max_rows)
    monkeypatch.delenv("FDLLM_PREFILL_PAIR")
    return vm


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_prefill_pair_kernel_bit_identical(dtype, monkeypatch):
    """The paired-query-block prefill attention, with all six heads of a kv head per workgroup
    (FDLLM_PREFILL_PAIR=2 forces it at every size; by default it runs once its workgroups fill the chip,
    from 4096 rows) and with the heads split over three workgroups (=3 forces it; by default from 32
    query blocks below that), against attn_prefill_kernel: the same key blocks in the same order per query,
    so hidden states and caches agree bit for bit.  Odd and even query-block counts, a ragged last block,
    the block-causal mask (forward_hidden, build_prefix_cache) and the unmasked form (a cached forward of
    200 rows after a prefix)."""
    from fast_dllm_relax_amd.config import FastDLLMConfig
    from fast_dllm_relax_amd.params import from_numpy
    from oracle.model import OracleConfig, random_params

    kw = WIDE2
    tdt = torch.bfloat16 if dtype == "bfloat16" else torch.float16
    params = from_numpy(random_params(OracleConfig(**kw), 6, dtype), FastDLLMConfig(**kw), dtype=dtype)
    vm_pair = _prefill_vm(kw, params, dtype, monkeypatch, 2, 2080)
    vm_split = _prefill_vm(kw, params, dtype, monkeypatch, 3, 2080)
    vm_old = _prefill_vm(kw, params, dtype, monkeypatch, 0, 2080)
    rng = np.random.default_rng(23)
    for S in (300, 1056, 2080):
        log(f"case: forward_hidden {S} rows, 1.5B width, 2 layers, {dtype}, paired (whole / split) vs one-block")
        ids = torch.tensor(rng.integers(0, kw["vocab_size"] - 1, S), dtype=torch.int32, device="cuda")
        x = vm_old.embed(ids)[None]
        h_old = vm_old.forward_hidden(x, None)
        h_pair = vm_pair.forward_hidden(x, None)
        h_split = vm_split.forward_hidden(x, None)
        torch.cuda.synchronize()
        assert torch.isfinite(h_pair.float()).all()
        np.testing.assert_array_equal(_bits(h_pair), _bits(h_old), err_msg=f"forward_hidden S={S}")
        np.testing.assert_array_equal(_bits(h_split), _bits(h_old), err_msg=f"forward_hidden S={S}, split")

    P, R = 1000, 200
    L, nkv, hd = kw["num_hidden_layers"], kw["num_key_value_heads"], kw["head_dim"]
    log(f"case: build_prefix_cache {P} rows + forward_cached {R} rows, {dtype}, paired vs one-block")
    ids = torch.tensor(rng.integers(0, kw["vocab_size"] - 1, P + R), dtype=torch.int32, device="cuda")
    caches = {}
    for name, vm in (("pair", vm_pair), ("split", vm_split), ("old", vm_old)):
        k = torch.zeros((L, 1, P + R + 32, nkv, hd), dtype=tdt, device="cuda")
        v = torch.zeros_like(k)
        vm.build_prefix_cache(vm.embed(ids[:P])[None], None, k, v)
        off = torch.tensor(P, dtype=torch.int32, device="cuda")
        h = vm.forward_cached(vm.embed(ids[P:])[None], k, v, off, P)
        torch.cuda.synchronize()
        caches[name] = (k, v, h)
    for i, what in enumerate(("k cache", "v cache", "cached-forward hidden")):
        np.testing.assert_array_equal(_bits(caches["pair"][i]), _bits(caches["old"][i]), err_msg=what)
        np.testing.assert_array_equal(_bits(caches["split"][i]), _bits(caches["old"][i]), err_msg=f"{what}, split")


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_lm_head_register_weight_bit_identical(dtype, monkeypatch):
    """The lm_head with its confidence statistics on the register-weight kernel (from 256 rows by default;
    FDLLM_WR_MIN_ROWS=128 here) against gemm_mm_kernel (FDLLM_WR_OPS without the lm_head bit): logits, ids
    and maxp bit for bit, at ragged and whole row counts, with and without the fp32 logits output."""
    from fast_dllm_relax_amd.config import FastDLLMConfig
    from fast_dllm_relax_amd.params import from_numpy
    from fast_dllm_relax_amd.vm import HipVM
    from oracle.model import OracleConfig, random_params

    kw = dict(WIDE2, tie_word_embeddings=False)
    params = from_numpy(random_params(OracleConfig(**kw), 8, dtype, lm_head_std=0.5), FastDLLMConfig(**kw),
                        dtype=dtype)
    vms = {}
    for name, ops in (("wr", 16), ("mm", 0)):
        monkeypatch.setenv("FDLLM_WR_OPS", str(ops))
        monkeypatch.setenv("FDLLM_WR_MIN_ROWS", "128")
        vms[name] = HipVM(FastDLLMConfig(**kw), params, dtype=dtype, max_rows=512)
        monkeypatch.delenv("FDLLM_WR_OPS")
        monkeypatch.delenv("FDLLM_WR_MIN_ROWS")
    tdt = torch.bfloat16 if dtype == "bfloat16" else torch.float16
    g = torch.Generator(device="cuda").manual_seed(31)
    for rows in (130, 300, 512):
        log(f"case: lm_head + confidence, {rows} rows, 1.5B vocab, {dtype}, register-weight vs gemm_mm")
        h = torch.randn((1, rows, kw["hidden_size"]), generator=g, device="cuda").to(tdt)
        out = {}
        for name, vm in vms.items():
            logits = torch.empty((1, rows, kw["vocab_size"]), dtype=torch.float32, device="cuda")
            ids, maxp = vm.get_confidence(h, logits)
            ids2, maxp2 = vm.get_confidence(h)
            torch.cuda.synchronize()
            out[name] = (logits, ids, maxp, ids2, maxp2)
        assert torch.isfinite(out["wr"][0]).all()
        for i, what in enumerate(("logits", "ids", "maxp", "ids (no logits)", "maxp (no logits)")):
            np.testing.assert_array_equal(out["wr"][i].cpu().numpy(), out["mm"][i].cpu().numpy(),
                                          err_msg=f"{what}, rows={rows}")
    for vm in vms.values():
        vm.close()


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_fused_down_norm_bit_identical(dtype, monkeypatch):
    """A large-M down launch that splits k hands its split sums, row-major, to resid_norm_kernel, which adds
    them, applies the residual epilogue and the next RMSNorm (the next layer's qkv input, or the final norm)
    in one launch; up to 256 rows o_proj does the same with three k splits (the post-attention norm).  The
    arithmetic is the split-sum kernel's and norm_rows_kernel's, and k splits add their sums in split order,
    so the results match the separate launches (FDLLM_FUSE_DOWN=0, FDLLM_FUSE_OPROJ=0) except where o_proj's
    forced split regroups its fp32 sums: the hidden states at sizes that fuse only down, and the caches and
    hidden states of a 16-sequence batched step (512 rows), must agree bit for bit; the 128-row partial step
    and the 100-row forward to the bf16 criterion."""
    from fast_dllm_relax_amd.config import FastDLLMConfig
    from fast_dllm_relax_amd.params import from_numpy
    from fast_dllm_relax_amd.vm import HipVM
    from oracle.model import OracleConfig, random_params

    kw = WIDE2
    params = from_numpy(random_params(OracleConfig(**kw), 12, dtype), FastDLLMConfig(**kw), dtype=dtype)
    tdt = torch.bfloat16 if dtype == "bfloat16" else torch.float16
    vms = {}
    for name, on in (("fused", "1"), ("separate", "0")):
        monkeypatch.setenv("FDLLM_FUSE_DOWN", on)
        monkeypatch.setenv("FDLLM_FUSE_OPROJ", "" if on == "1" else "0")
        vms[name] = HipVM(FastDLLMConfig(**kw), params, dtype=dtype, max_rows=1024)
        monkeypatch.delenv("FDLLM_FUSE_DOWN")
        monkeypatch.delenv("FDLLM_FUSE_OPROJ")
    rng = np.random.default_rng(29)
    for S in (100, 300, 512, 1056):
        log(f"case: forward_hidden {S} rows, {dtype}, fused down epilogue + norm vs separate launches")
        ids = torch.tensor(rng.integers(0, kw["vocab_size"] - 1, S), dtype=torch.int32, device="cuda")
        x = vms["separate"].embed(ids)[None]
        h = {name: vm.forward_hidden(x, None) for name, vm in vms.items()}
        torch.cuda.synchronize()
        assert torch.isfinite(h["fused"].float()).all()
        if S <= 256:  # o_proj's forced k split
            bf16_parity(f"fused vs separate, S={S}", h["fused"].float().cpu().numpy(), h["separate"].float().cpu().numpy())
        else:
            np.testing.assert_array_equal(_bits(h["fused"]), _bits(h["separate"]), err_msg=f"S={S}")

    L, nkv, hd = kw["num_hidden_layers"], kw["num_key_value_heads"], kw["head_dim"]
    prefixes = [int(p) for p in 32 * rng.integers(1, 9, 16)]
    cap = max(prefixes) + 32
    ids = [rng.integers(0, kw["vocab_size"] - 1, P + 32) for P in prefixes]
    # one set of prefix caches for both (prefixes up to 256 rows take the fused o_proj)
    k0 = torch.zeros((L, 16, cap, nkv, hd), dtype=tdt, device="cuda")
    v0 = torch.zeros_like(k0)
    for b, P in enumerate(prefixes):
        vms["separate"].build_prefix_cache_seq(
            vms["separate"].embed(torch.tensor(ids[b][:P], dtype=torch.int32, device="cuda"))[None], None, k0, v0, b)
    out = {}
    for name, vm in vms.items():
        log(f"case: batched step of 16 x 32 rows + partial step, {dtype}, {name}")
        k, v = k0.clone(), v0.clone()
        x = torch.stack([vm.embed(torch.tensor(ids[b][P:], dtype=torch.int32, device="cuda"))
                         for b, P in enumerate(prefixes)])
        hf = vm.forward_cached_batch(x, k, v, torch.tensor(prefixes, dtype=torch.int32, device="cuda"), prefixes)
        kf, vf = k.clone(), v.clone()
        hp = vm.forward_block_partial_batch(8, x[:, 8:16].contiguous(), k, v,
                                            torch.tensor([P + 8 for P in prefixes], dtype=torch.int32, device="cuda"),
                                            prefixes)
        torch.cuda.synchronize()
        out[name] = (hf, kf, vf, hp, k, v)
    for i, what in enumerate(("full-step hidden", "full-step K cache", "full-step V cache")):
        np.testing.assert_array_equal(_bits(out["fused"][i]), _bits(out["separate"][i]), err_msg=what)
    # 128 rows: o_proj's forced k split
    for i, what in ((3, "partial-step hidden"), (4, "K cache after the partial step"), (5, "V cache after the partial step")):
        bf16_parity(what, out["fused"][i].float().cpu().numpy(), out["separate"][i].float().cpu().numpy())
    for vm in vms.values():
        vm.close()


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_qkv_rope_epilogue_bit_identical(dtype, monkeypatch):
    """Calls whose attention starts with the RoPE / KV-append pass (prefill and forward_hidden from 128 rows,
    the batched-sequence kernel) have qkv's register-weight epilogue do that pass instead: rope_kv_kernel's
    arithmetic on the rounded qkv values, with the tiles taken in perm8 order so that both halves of each
    rotation pair are in one block (64 x 64 blocks up to 512 rows, 64 x 128 below 4096, 128 x 256 above).
    Hidden states, caches and the batched step must agree bit for bit with the separate pass
    (FDLLM_QKV_ROPE=0), at ragged row counts too."""
    from fast_dllm_relax_amd.config import FastDLLMConfig
    from fast_dllm_relax_amd.params import from_numpy
    from fast_dllm_relax_amd.vm import HipVM
    from oracle.model import OracleConfig, random_params, build_prefix_block_attention_bias

    kw = WIDE2
    params = from_numpy(random_params(OracleConfig(**kw), 14, dtype), FastDLLMConfig(**kw), dtype=dtype)
    tdt = torch.bfloat16 if dtype == "bfloat16" else torch.float16
    vms = {}
    for name, on in (("epilogue", "1"), ("separate", "0")):
        monkeypatch.setenv("FDLLM_QKV_ROPE", on)
        vms[name] = HipVM(FastDLLMConfig(**kw), params, dtype=dtype, max_rows=4200)
        monkeypatch.delenv("FDLLM_QKV_ROPE")
    rng = np.random.default_rng(37)
    L, nkv, hd = kw["num_hidden_layers"], kw["num_key_value_heads"], kw["head_dim"]
    for S in (130, 300, 512, 2080, 4160):
        log(f"case: forward_hidden {S} rows and build_prefix_cache, {dtype}, RoPE in qkv's epilogue vs rope_kv")
        ids = torch.tensor(rng.integers(0, kw["vocab_size"] - 1, S), dtype=torch.int32, device="cuda")
        x = vms["separate"].embed(ids)[None]
        h = {name: vm.forward_hidden(x, None) for name, vm in vms.items()}
        caches = {}
        for name, vm in vms.items():
            k = torch.zeros((L, 1, S, nkv, hd), dtype=tdt, device="cuda")
            v = torch.zeros_like(k)
            vm.build_prefix_cache(x, None, k, v)
            caches[name] = (k, v)
        torch.cuda.synchronize()
        assert torch.isfinite(h["epilogue"].float()).all()
        np.testing.assert_array_equal(_bits(h["epilogue"]), _bits(h["separate"]), err_msg=f"hidden S={S}")
        for i, what in enumerate(("K", "V")):
            np.testing.assert_array_equal(_bits(caches["epilogue"][i]), _bits(caches["separate"][i]),
                                          err_msg=f"{what} cache S={S}")
    prefixes = [int(p) for p in 32 * rng.integers(1, 9, 16)]
    cap = max(prefixes) + 32
    ids = [rng.integers(0, kw["vocab_size"] - 1, P + 32) for P in prefixes]
    k0 = torch.zeros((L, 16, cap, nkv, hd), dtype=tdt, device="cuda")
    v0 = torch.zeros_like(k0)
    for b, P in enumerate(prefixes):
        vms["separate"].build_prefix_cache_seq(
            vms["separate"].embed(torch.tensor(ids[b][:P], dtype=torch.int32, device="cuda"))[None], None, k0, v0, b)
    out = {}
    for name, vm in vms.items():
        log(f"case: batched step of 16 x 32 rows, {dtype}, {name}")
        k, v = k0.clone(), v0.clone()
        x = torch.stack([vm.embed(torch.tensor(ids[b][P:], dtype=torch.int32, device="cuda"))
                         for b, P in enumerate(prefixes)])
        hf = vm.forward_cached_batch(x, k, v, torch.tensor(prefixes, dtype=torch.int32, device="cuda"), prefixes)
        torch.cuda.synchronize()
        out[name] = (hf, k, v)
    for i, what in enumerate(("batched hidden", "K cache", "V cache")):
        np.testing.assert_array_equal(_bits(out["epilogue"][i]), _bits(out["separate"][i]), err_msg=what)
    for vm in vms.values():
        vm.close()
