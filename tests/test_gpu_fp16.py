"""The fp16 model dtype (config 4 runs in fp16) vs the oracle with fp16 rounding points, through the C ABI:
the cached step, logits and confidence, the large-M stateless forward and the batched step."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import TINY, WIDE2, bf16_parity, log, make_pair, to_np
from oracle import confidence as oconf
from oracle.model import OracleModel, build_prefix_block_attention_bias

pytestmark = pytest.mark.gpu


def _dev_ids(ids):
    return torch.tensor(np.asarray(ids), dtype=torch.int32, device="cuda")


def _off(v):
    return torch.tensor(int(v), dtype=torch.int32, device="cuda")


@pytest.fixture(scope="module")
def tiny16():
    log("setup: tiny fp16 model seed 7")
    return make_pair(TINY, 7, dtype="float16")


@pytest.fixture(scope="module")
def wide16():
    log("setup: 1.5B-shape 2-layer fp16 model seed 8")
    return make_pair(WIDE2, 8, dtype="float16")


def _cached_case(ref, vm, kw, P, seed, label):
    from oracle.model import OracleModel as _OM

    ref32 = _OM(ref.cfg, ref.p, "float32")
    rng = np.random.default_rng(seed)
    L, nkv, hd = kw["num_hidden_layers"], kw["num_key_value_heads"], kw["head_dim"]
    cap = P + 64
    ids = rng.integers(0, kw["vocab_size"] - 1, P + 32)
    outs = {}
    for name, model in (("f16", ref), ("f32", ref32)):
        kc = np.zeros((L, 1, cap, nkv, hd), np.float32)
        vc = kc.copy()
        model.build_prefix_cache(model.embed(ids[:P])[None], build_prefix_block_attention_bias(0, P, block_size=32), kc, vc)
        h = model.forward_cached(model.embed(ids[P:])[None], kc, vc, P, P)
        outs[name] = (h, model.get_logits(h), kc)
    k = torch.zeros((L, 1, cap, nkv, hd), dtype=torch.float16, device="cuda")
    v = torch.zeros_like(k)
    log(f"case: {label} fp16 build_prefix_cache P={P} + forward_cached R=32")
    vm.build_prefix_cache(vm.embed(_dev_ids(ids[:P]))[None], None, k, v)
    bf16_parity(f"{label} fp16 prefix K", to_np(k)[:, :, :P + 32][:, :, :P], outs["f16"][2][:, :, :P], outs["f32"][2][:, :, :P])
    h = vm.forward_cached(vm.embed(_dev_ids(ids[P:]))[None], k, v, _off(P), P)
    bf16_parity(f"{label} fp16 hidden", to_np(h), outs["f16"][0], outs["f32"][0])
    lg = to_np(vm.get_logits(h))
    bf16_parity(f"{label} fp16 logits", lg, outs["f16"][1], outs["f32"][1])
    ids_d, maxp_d = vm.get_confidence(h)
    wid, wp = oconf.confidence(lg[0])
    np.testing.assert_array_equal(ids_d.cpu().numpy()[0], wid)
    np.testing.assert_array_equal(maxp_d.cpu().numpy()[0].view(np.uint32), wp.view(np.uint32))


def test_fp16_cached_step_logits_confidence(tiny16):
    ref, vm = tiny16
    _cached_case(ref, vm, TINY, 64, 21, "tiny")


def test_fp16_large_m_forward_hidden(tiny16):
    ref, vm = tiny16
    ref32 = OracleModel(ref.cfg, ref.p, "float32")
    rng = np.random.default_rng(22)
    for S in (45, 160):
        ids = rng.integers(0, TINY["vocab_size"] - 1, S)
        bias = build_prefix_block_attention_bias(0, S, block_size=32)
        log(f"case: tiny fp16 forward_hidden S={S}")
        got = to_np(vm.forward_hidden(vm.embed(_dev_ids(ids))[None], None))
        bf16_parity(f"fp16 hidden S={S}", got, ref.forward_hidden(ref.embed(ids)[None], bias),
                    ref32.forward_hidden(ref32.embed(ids)[None], bias))


def test_fp16_wide_cached_step(wide16):
    ref, vm = wide16
    _cached_case(ref, vm, WIDE2, 256, 23, "wide")


def test_fp16_wide_batched_step(wide16):
    """16 sequences x 32 rows in fp16 (config 4's dtype and row count) vs the fp16 oracle per sequence."""
    ref, vm = wide16
    rng = np.random.default_rng(24)
    kw = WIDE2
    L, nkv, hd = kw["num_hidden_layers"], kw["num_key_value_heads"], kw["head_dim"]
    prefixes = [int(p) for p in 32 * rng.integers(1, 4, 16)]
    B, R = len(prefixes), 32
    cap = max(prefixes) + 2 * R
    ids = [rng.integers(0, kw["vocab_size"] - 1, P + R) for P in prefixes]
    want = []
    for b, P in enumerate(prefixes):
        kc = np.zeros((L, 1, cap, nkv, hd), np.float32)
        vc = kc.copy()
        ref.build_prefix_cache(ref.embed(ids[b][:P])[None], build_prefix_block_attention_bias(0, P, block_size=32), kc, vc)
        want.append(ref.forward_cached(ref.embed(ids[b][P:])[None], kc, vc, P, P)[0])
    k = torch.zeros((L, B, cap, nkv, hd), dtype=torch.float16, device="cuda")
    v = torch.zeros_like(k)
    for b, P in enumerate(prefixes):
        vm.build_prefix_cache_seq(vm.embed(_dev_ids(ids[b][:P]))[None], None, k, v, b)
    x = torch.stack([vm.embed(_dev_ids(ids[b][P:])) for b, P in enumerate(prefixes)])
    log(f"case: wide fp16 forward_cached_batch nseq={B}")
    h = vm.forward_cached_batch(x, k, v, torch.tensor(prefixes, dtype=torch.int32, device="cuda"), prefixes)
    for b in range(B):
        bf16_parity(f"fp16 seq {b} hidden", to_np(h[b]), want[b])
