"""The down projection's k splits summed inside their own launch against the separate split-sum launch.

A call of at most 32 rows sums the one-shot down projection's k splits inside the launch that produces
them (the splits of each tile group meet at a counter, then each sums a share of the group's outputs),
when the launch's whole grid is resident at once; FDLLM_GROUP_WAITS=0 keeps the separate
gemm_os_epilogue_kernel launch.  The arithmetic and its order are the same, so hidden states and cache
rows must agree bit for bit, over consecutive calls (the counter banks alternate and each launch clears
the other).  fdllm_group_wait_launches shows which path ran.  A wait that timed out would be reported by
the next entry point, which every case calls last."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import TINY, WIDE2, log

pytestmark = pytest.mark.gpu


def _pair_of_vms(kw, seed, monkeypatch, dtype):
    from fast_dllm_relax_amd.config import FastDLLMConfig
    from fast_dllm_relax_amd.params import from_numpy
    from fast_dllm_relax_amd.vm import HipVM
    from oracle.model import OracleConfig, random_params

    cfg = FastDLLMConfig(**kw)
    params = from_numpy(random_params(OracleConfig(**kw), seed, dtype), cfg, dtype=dtype)
    monkeypatch.delenv("FDLLM_GROUP_WAITS", raising=False)
    vm_g = HipVM(cfg, params, dtype=dtype, max_rows=64)
    monkeypatch.setenv("FDLLM_GROUP_WAITS", "0")
    vm_s = HipVM(cfg, params, dtype=dtype, max_rows=64)
    monkeypatch.delenv("FDLLM_GROUP_WAITS")
    return vm_g, vm_s


def _bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy()


def _same(a, b, what):
    np.testing.assert_array_equal(_bits(a), _bits(b), err_msg=what)


def _run_case(kw, seed, P, monkeypatch, dtype="bfloat16"):
    vm_g, vm_s = _pair_of_vms(kw, seed, monkeypatch, dtype)
    tdt = torch.bfloat16 if dtype == "bfloat16" else torch.float16
    L, nkv, hd = kw["num_hidden_layers"], kw["num_key_value_heads"], kw["head_dim"]
    cap = (P + 32 + 31) // 32 * 32 + 32
    rng = np.random.default_rng(seed + 300)
    ids = torch.tensor(rng.integers(0, kw["vocab_size"] - 1, P + 32), dtype=torch.int32, device="cuda")
    k = torch.zeros((L, 1, cap, nkv, hd), dtype=tdt, device="cuda")
    v = torch.zeros_like(k)
    log(f"case: prefix {P} rows, L={L}, H={kw['hidden_size']}, {dtype}")
    vm_s.build_prefix_cache(vm_s.embed(ids[:P])[None], None, k, v)
    caches = {"g": (k.clone(), v.clone()), "s": (k.clone(), v.clone())}
    off = torch.tensor(P, dtype=torch.int32, device="cuda")
    x = vm_s.embed(ids[P:])[None]

    log("  forward_cached R=32")
    n0 = vm_g.lib.fdllm_group_wait_launches(vm_g.ctx)
    hg = vm_g.forward_cached(x, *caches["g"], off, P)
    hs = vm_s.forward_cached(x, *caches["s"], off, P)
    torch.cuda.synchronize()
    ran = vm_g.lib.fdllm_group_wait_launches(vm_g.ctx) - n0
    assert ran == L, ran  # down in every layer
    assert vm_s.lib.fdllm_group_wait_launches(vm_s.ctx) == 0
    _same(hg, hs, "hidden R=32")
    _same(caches["g"][0], caches["s"][0], "K cache")
    _same(caches["g"][1], caches["s"][1], "V cache")
    for rp in (0, 8, 16, 24):
        log(f"  forward_block_partial_rp{rp} R=8")
        xs = x[:, rp:rp + 8]
        hg = getattr(vm_g, f"forward_block_partial_rp{rp}")(xs, *caches["g"], off, P)
        hs = getattr(vm_s, f"forward_block_partial_rp{rp}")(xs, *caches["s"], off, P)
        _same(hg, hs, f"hidden rp{rp}")
        _same(caches["g"][0], caches["s"][0], f"K cache rp{rp}")
        _same(caches["g"][1], caches["s"][1], f"V cache rp{rp}")
    # a second full step on the same context: each launch zeroed the bank the launch before it used
    log("  forward_cached R=32 again")
    _same(vm_g.forward_cached(x, *caches["g"], off, P), vm_s.forward_cached(x, *caches["s"], off, P), "hidden again")
    torch.cuda.synchronize()
    assert bool(torch.isfinite(hg.float()).all())
    # the next entry point reports a timed-out wait of any launch above
    vm_g.get_logits(hg[:, :1])
    torch.cuda.synchronize()


def test_group_waits_tiny_bf16(monkeypatch):
    """Tiny shapes: 4 tile groups of 8 k splits."""
    _run_case(TINY, 0, 96, monkeypatch)


def test_group_waits_tiny_fp16(monkeypatch):
    _run_case(dict(TINY, num_hidden_layers=3), 3, 700, monkeypatch, "float16")


def test_group_waits_wide(monkeypatch):
    """1.5B layer shapes (two layers), prefix 2048: 24 tile groups of 10 k splits (240 workgroups)."""
    _run_case(WIDE2, 1, 2048, monkeypatch)


def test_group_waits_wide_long_prefix(monkeypatch):
    """Prefix 6000: the attention merges 48 key splits with its separate launch."""
    _run_case(WIDE2, 2, 6000, monkeypatch)
