"""The persistent cached step (every layer in one cooperative launch) against the per-operator kernels.

Both paths run the same arithmetic in the same order (k partitions, wave-order and split-order sums,
epilogues, attention bodies), so hidden states and the appended cache rows must agree bit for bit.
Each case also checks that the persistent launch really ran (fdllm_persistent_steps) and, with
FDLLM_STEP_CHECK=1, that no grid-barrier wait timed out.  The persistent path is opt-in
(FDLLM_PERSISTENT=1); the per-operator path it is compared with is the default one, whose parity with
the oracle test_gpu_parity.py checks, so the persistent path's parity follows bit for bit."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import TINY, WIDE2, log

pytestmark = pytest.mark.gpu

TINY4 = dict(TINY, num_hidden_layers=4)


def _pair_of_vms(kw, seed, monkeypatch, dtype="bfloat16"):
    """Two contexts over one set of device weights: persistent step on, and off."""
    from fast_dllm_relax_amd.config import FastDLLMConfig
    from fast_dllm_relax_amd.params import from_numpy
    from fast_dllm_relax_amd.vm import HipVM
    from oracle.model import OracleConfig, random_params

    cfg = FastDLLMConfig(**kw)
    params = from_numpy(random_params(OracleConfig(**kw), seed, dtype), cfg, dtype=dtype)
    monkeypatch.setenv("FDLLM_PERSISTENT", "1")
    monkeypatch.setenv("FDLLM_STEP_CHECK", "1")
    vm_p = HipVM(cfg, params, dtype=dtype, max_rows=64)
    monkeypatch.setenv("FDLLM_PERSISTENT", "0")
    vm_o = HipVM(cfg, params, dtype=dtype, max_rows=64)
    monkeypatch.delenv("FDLLM_STEP_CHECK")
    return vm_p, vm_o


def _bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy()


def _run_case(kw, seed, P, monkeypatch, dtype="bfloat16"):
    vm_p, vm_o = _pair_of_vms(kw, seed, monkeypatch, dtype)
    tdt = torch.bfloat16 if dtype == "bfloat16" else torch.float16
    L, nkv, hd = kw["num_hidden_layers"], kw["num_key_value_heads"], kw["head_dim"]
    cap = (P + 32 + 31) // 32 * 32 + 32
    rng = np.random.default_rng(seed + 100)
    ids = torch.tensor(rng.integers(0, kw["vocab_size"] - 1, P + 32), dtype=torch.int32, device="cuda")
    k = torch.zeros((L, 1, cap, nkv, hd), dtype=tdt, device="cuda")
    v = torch.zeros_like(k)
    log(f"case: prefix {P} rows, L={L}, H={kw['hidden_size']}, {dtype}")
    vm_o.build_prefix_cache(vm_o.embed(ids[:P])[None], None, k, v)
    caches = {"p": (k.clone(), v.clone()), "o": (k.clone(), v.clone())}
    off = torch.tensor(P, dtype=torch.int32, device="cuda")
    x = vm_o.embed(ids[P:])[None]
    before = vm_p.lib.fdllm_persistent_steps(vm_p.ctx)
    log("  forward_cached R=32")
    hp = vm_p.forward_cached(x, *caches["p"], off, P)
    ho = vm_o.forward_cached(x, *caches["o"], off, P)
    torch.cuda.synchronize()
    assert vm_p.lib.fdllm_persistent_steps(vm_p.ctx) == before + 1, "the persistent launch did not run"
    assert vm_o.lib.fdllm_persistent_steps(vm_o.ctx) == 0
    np.testing.assert_array_equal(_bits(hp), _bits(ho))
    for name, i in (("K", 0), ("V", 1)):
        np.testing.assert_array_equal(_bits(caches["p"][i]), _bits(caches["o"][i]), err_msg=f"{name} cache")
    for rp in (0, 8, 16, 24):
        log(f"  forward_block_partial_rp{rp} R=8")
        xs = x[:, rp:rp + 8]
        hp = getattr(vm_p, f"forward_block_partial_rp{rp}")(xs, *caches["p"], off, P)
        ho = getattr(vm_o, f"forward_block_partial_rp{rp}")(xs, *caches["o"], off, P)
        np.testing.assert_array_equal(_bits(hp), _bits(ho))
        np.testing.assert_array_equal(_bits(caches["p"][0]), _bits(caches["o"][0]))
        np.testing.assert_array_equal(_bits(caches["p"][1]), _bits(caches["o"][1]))
    torch.cuda.synchronize()
    assert vm_p.lib.fdllm_persistent_steps(vm_p.ctx) == before + 5
    assert bool(torch.isfinite(hp.float()).all())


def test_persistent_step_tiny(monkeypatch):
    _run_case(TINY, 0, 96, monkeypatch)


def test_persistent_step_tiny_4_layers_fp16(monkeypatch):
    _run_case(TINY4, 3, 200, monkeypatch, "float16")


def test_persistent_step_wide(monkeypatch):
    """1.5B layer shapes (two layers), prefix 512: 9 key chunks of 64."""
    _run_case(WIDE2, 1, 512, monkeypatch)


def test_persistent_step_wide_long_prefix(monkeypatch):
    """Prefix 3000: 24 key chunks of 128 (the merge's one-round register path ends at 24 chunks)."""
    _run_case(WIDE2, 2, 3000, monkeypatch)


def test_persistent_step_wide_longer_prefix(monkeypatch):
    """Prefix 4000: 32 key chunks of 128, merged in the two-pass loop."""
    _run_case(WIDE2, 5, 4000, monkeypatch)
