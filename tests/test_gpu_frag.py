"""Activations in MFMA-fragment order against the row-major layout (and the one-shot GEMMs' half-row
m-chunks against whole 32-row chunks, the same way).

A call of at most 32 rows whose four projections all take the one-shot GEMM keeps h, the attention
output and SiLU * up in the order the GEMMs load their operand fragments (the default); FDLLM_XFRAG=0
keeps them row-major.  The kernels and their arithmetic are the same, only the addresses differ, so
hidden states and cache rows must agree bit for bit.  The row-major layout is the one whose parity
with the oracle the other GPU tests establish for the large-row paths (prefill, batched steps), and
fdllm_frag_calls shows that the fragment-order path really ran."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import TINY, WIDE2, log

pytestmark = pytest.mark.gpu


def _pair_of_vms(kw, seed, monkeypatch, dtype, env="FDLLM_XFRAG"):
    """The default context and one with the switch `env` set to 0, on the same weights."""
    from fast_dllm_relax_amd.config import FastDLLMConfig
    from fast_dllm_relax_amd.params import from_numpy
    from fast_dllm_relax_amd.vm import HipVM
    from oracle.model import OracleConfig, random_params

    cfg = FastDLLMConfig(**kw)
    params = from_numpy(random_params(OracleConfig(**kw), seed, dtype), cfg, dtype=dtype)
    monkeypatch.delenv(env, raising=False)
    vm_f = HipVM(cfg, params, dtype=dtype, max_rows=64)
    monkeypatch.setenv(env, "0")
    vm_r = HipVM(cfg, params, dtype=dtype, max_rows=64)
    monkeypatch.delenv(env)
    return vm_f, vm_r


def _bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy()


def _same(a, b, what):
    np.testing.assert_array_equal(_bits(a), _bits(b), err_msg=what)


def _run_case(kw, seed, P, monkeypatch, dtype="bfloat16", env="FDLLM_XFRAG"):
    vm_f, vm_r = _pair_of_vms(kw, seed, monkeypatch, dtype, env)
    frag_r = 0 if env == "FDLLM_XFRAG" else 1  # the other switches keep the fragment order
    tdt = torch.bfloat16 if dtype == "bfloat16" else torch.float16
    L, nkv, hd = kw["num_hidden_layers"], kw["num_key_value_heads"], kw["head_dim"]
    cap = (P + 32 + 31) // 32 * 32 + 32
    rng = np.random.default_rng(seed + 200)
    ids = torch.tensor(rng.integers(0, kw["vocab_size"] - 1, P + 32), dtype=torch.int32, device="cuda")
    k = torch.zeros((L, 1, cap, nkv, hd), dtype=tdt, device="cuda")
    v = torch.zeros_like(k)
    log(f"case: prefix {P} rows, L={L}, H={kw['hidden_size']}, {dtype}")
    vm_r.build_prefix_cache(vm_r.embed(ids[:P])[None], None, k, v)
    caches = {"f": (k.clone(), v.clone()), "r": (k.clone(), v.clone())}
    off = torch.tensor(P, dtype=torch.int32, device="cuda")
    x = vm_r.embed(ids[P:])[None]

    log("  forward_cached R=32")
    hf = vm_f.forward_cached(x, *caches["f"], off, P)
    hr = vm_r.forward_cached(x, *caches["r"], off, P)
    torch.cuda.synchronize()
    assert vm_f.lib.fdllm_frag_calls(vm_f.ctx) == 1, "the fragment-order path did not run"
    assert vm_r.lib.fdllm_frag_calls(vm_r.ctx) == frag_r
    _same(hf, hr, "hidden R=32")
    _same(caches["f"][0], caches["r"][0], "K cache")
    _same(caches["f"][1], caches["r"][1], "V cache")
    for rp in (0, 8, 16, 24):
        log(f"  forward_block_partial_rp{rp} R=8")
        xs = x[:, rp:rp + 8]
        hf = getattr(vm_f, f"forward_block_partial_rp{rp}")(xs, *caches["f"], off, P)
        hr = getattr(vm_r, f"forward_block_partial_rp{rp}")(xs, *caches["r"], off, P)
        _same(hf, hr, f"hidden rp{rp}")
        _same(caches["f"][0], caches["r"][0], f"K cache rp{rp}")
        _same(caches["f"][1], caches["r"][1], f"V cache rp{rp}")

    # short stateless forwards: block-causal (20 rows: a partial second block), then an additive bias
    xs = vm_r.embed(ids[:20])[None]
    log("  forward_hidden 20 rows, block-causal")
    _same(vm_f.forward_hidden(xs, None), vm_r.forward_hidden(xs, None), "forward_hidden block-causal")
    bias = torch.tensor(rng.normal(0.0, 1.0, (1, 1, 20, 20)), dtype=torch.float32, device="cuda")
    bias[..., 5:, 17:] = float("-inf")
    log("  forward_hidden 20 rows, additive bias")
    _same(vm_f.forward_hidden(xs, bias), vm_r.forward_hidden(xs, bias), "forward_hidden bias")
    torch.cuda.synchronize()
    assert vm_f.lib.fdllm_frag_calls(vm_f.ctx) == 7
    assert vm_r.lib.fdllm_frag_calls(vm_r.ctx) == 7 * frag_r
    assert bool(torch.isfinite(hf.float()).all())


def test_frag_tiny_bf16(monkeypatch):
    _run_case(TINY, 0, 96, monkeypatch)


def test_frag_tiny_fp16(monkeypatch):
    _run_case(dict(TINY, num_hidden_layers=3), 3, 200, monkeypatch, "float16")


def test_frag_tiny_short_prefix(monkeypatch):
    """Prefix 16: one key chunk, the chunk kernel writes the attention output itself."""
    _run_case(TINY, 4, 16, monkeypatch)


def test_frag_wide(monkeypatch):
    """1.5B layer shapes (two layers), prefix 512."""
    _run_case(WIDE2, 1, 512, monkeypatch)


def test_frag_wide_long_prefix(monkeypatch):
    """Prefix 3000: 24 key chunks, the split merge writes the attention output."""
    _run_case(WIDE2, 2, 3000, monkeypatch)


def test_half_row_chunks_bit_identical(monkeypatch):
    """One-shot qkv and o_proj of 17 to 32 rows as two 16-row m-chunks (the default for bf16) against one
    32-row chunk (FDLLM_OS_HALF=0): each row's arithmetic is the same, so every result is the same bits."""
    _run_case(WIDE2, 5, 700, monkeypatch, env="FDLLM_OS_HALF")
    _run_case(dict(TINY, num_hidden_layers=3), 6, 130, monkeypatch, env="FDLLM_OS_HALF")
