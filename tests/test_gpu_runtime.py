"""The host runtime's step functions and cache helpers on the HIP path, against the oracle's functions of the
same names (fast_dllm_relax/runtime.py), and the reference's own tests of them restated on HIP
(tests/test_tiny_compile.py:293-329).  Marked gpu; every model call goes through the C ABI.

* score_active_block_cached_fast / _refine / _partial_perlayer (runtime.py:346-436): their shifted ids
  and probabilities are bit-exact with the oracle's confidence (oracle/confidence.c) applied to the HIP
  path's own logits, and match oracle.runtime's functions on the oracle model wherever the oracle's
  decision is not within the measured logit error of a tie.
* PrefixCache.ensure_capacity keeps the committed rows bit for bit (test_tiny_compile.py:293-308).
* chunked_prefill (runtime.py:282-307) equals the one-shot prefill to the bf16 criterion, and so does the
  cached step after it; an unaligned prefix raises the reference's error.
* get_logits with a tied head equals an untied head holding the same array, bit for bit
  (test_tiny_compile.py:311-329).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import log, make_pair, to_np
from oracle import confidence as oconf
from oracle import runtime as ort

pytestmark = pytest.mark.gpu

SMALL = dict(vocab_size=1000, hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
             num_key_value_heads=2, head_dim=128, tie_word_embeddings=False)
MASK = 999


@pytest.fixture(scope="module")
def pair():
    return make_pair(SMALL, 31, "bfloat16", lm_head_std=1.25, max_rows=256)


def _rt():
    from fast_dllm_relax_amd import runtime

    return runtime


def _agree(name, ids_h, p_h, ids_o, p_o, logits_o, delta):
    """ids equal wherever the oracle's top-2 logit gap exceeds twice the logit error; probabilities within
    the band that error allows."""
    lo = np.asarray(logits_o, np.float32)
    sh = np.concatenate([lo[:1], lo[:-1]])
    top2 = np.sort(sh, axis=-1)[:, -2:]
    firm = (top2[:, 1] - top2[:, 0]) > 2 * delta
    np.testing.assert_array_equal(np.asarray(ids_h)[firm], np.asarray(ids_o)[firm], err_msg=name)
    band = np.expm1(2 * delta)
    np.testing.assert_array_less(np.abs(np.asarray(p_h, np.float64) - p_o), band * np.maximum(p_o, 1e-30) + 1e-6,
                                 err_msg=name)
    log(f"  {name}: ids agree on {int(firm.sum())}/{len(firm)} firm rows, max |dp| "
        f"{float(np.abs(np.asarray(p_h, np.float64) - p_o).max()):.3g}")


def test_step_functions_match_oracle(pair):
    ref, vm = pair
    rt = _rt()
    rng = np.random.default_rng(32)
    P = 64
    prefix = [int(t) for t in rng.integers(0, MASK, P)]
    block = [int(t) for t in rng.integers(0, MASK, 6)] + [MASK] * 26
    hc = rt.build_prefix_cache_from_ids(vm, prefix, block_size=32, capacity=P + 64)
    oc = ort.build_prefix_cache_from_ids(ref, prefix, block_size=32, capacity=P + 64)

    log("case: score_active_block_refine")
    ids_h, p_h = rt.score_active_block_refine(vm, block, hc)
    logits_h = to_np(vm.get_logits(rt._forward_cached(vm, block, hc)))[0]
    ci, cp, _ = oconf.shifted_confidence(logits_h)
    np.testing.assert_array_equal(ids_h, ci)
    np.testing.assert_array_equal(p_h.view(np.int32), cp.view(np.int32))
    logits_o = ref.get_logits(ort.forward_cached(ref, block, oc))[0]
    delta = float(np.abs(logits_h - logits_o).max())
    log(f"  measured logit error of the step: {delta:.4g}")
    ids_o, p_o = ort.score_active_block_refine(ref, block, oc)
    _agree("refine", ids_h, p_h, ids_o, p_o, logits_o, delta)
    assert hc.prefix_len == oc.prefix_len == P  # refine does not commit

    for rp in (0, 8, 16, 24):
        log(f"case: score_active_block_partial_perlayer rp{rp}")
        small = block[rp:rp + 8]
        ids_h, p_h = rt.score_active_block_partial_perlayer(vm, small, hc, rp, block_size=32)
        hid = vm[f"forward_block_partial_rp{rp}"](rt._embed(vm, small), hc.k, hc.v, rt._offset_tensor(P + rp), P)
        lh = to_np(vm.get_logits(hid))[0]
        ci, cp, _ = oconf.shifted_confidence(lh)
        np.testing.assert_array_equal(ids_h, ci)
        np.testing.assert_array_equal(p_h.view(np.int32), cp.view(np.int32))
        ids_o, p_o = ort.score_active_block_partial_perlayer(ref, small, oc, rp, block_size=32)
        lo = ref.get_logits(ref.forward_block_partial(rp, ref.embed(small)[None], oc.k, oc.v, P + rp, P))[0]
        _agree(f"partial rp{rp}", ids_h, p_h, ids_o, p_o, lo, delta)

    log("case: score_active_block_cached_fast (commits the block)")
    k_before = hc.k[:, :, :P].clone()
    ids_h, p_h, last_h, hc2 = rt.score_active_block_cached_fast(vm, block, hc)
    ids_o, p_o, last_o, oc2 = ort.score_active_block_cached_fast(ref, block, oc)
    assert hc2 is hc and hc.prefix_len == oc2.prefix_len == P + 32
    assert torch.equal(hc.k[:, :, :P], k_before), "the committed prefix rows changed"
    _agree("cached_fast", ids_h, p_h, ids_o, p_o, logits_o, delta)
    top2 = np.sort(logits_o[-1])[-2:]
    if top2[1] - top2[0] > 2 * delta:
        assert last_h == last_o
    # the appended block's K/V rows match the oracle's to the bf16 criterion
    np.testing.assert_allclose(to_np(hc.k[:, :, P:P + 32]), oc.k[:, :, P:P + 32], rtol=2e-2, atol=2e-2)
    np.testing.assert_allclose(to_np(hc.v[:, :, P:P + 32]), oc.v[:, :, P:P + 32], rtol=2e-2, atol=2e-2)


def test_ensure_capacity_preserves_prefix(pair):
    """PrefixCache.ensure_capacity keeps rows [0, P) (test_tiny_compile.py:293-308)."""
    _, vm = pair
    rt = _rt()
    prefix = [int(t) for t in np.random.default_rng(33).integers(0, MASK, 64)]
    cache = rt.allocate_prefix_cache(rt.cache_spec_of(vm), "cuda", 64)
    rt._prefill(vm, prefix, cache, block_size=32)
    before = (cache.k.clone(), cache.v.clone())
    cache.ensure_capacity(160)
    assert cache.capacity == 160 and cache.prefix_len == 64
    for old, new in zip(before, (cache.k, cache.v)):
        assert torch.equal(new[:, :, :64], old)
    # a cached step on the grown cache attends the kept rows
    h = rt._forward_cached(vm, [MASK] * 32, cache)
    assert bool(torch.isfinite(h.float()).all())


def test_chunked_prefill_matches_one_shot(pair):
    """build_prefix_cache_from_ids(chunked_prefill=True) (runtime.py:282-307): the first block by
    build_prefix_cache, every later one by a cached step that is then committed."""
    ref, vm = pair
    rt = _rt()
    prefix = [int(t) for t in np.random.default_rng(34).integers(0, MASK, 128)]
    one = rt.build_prefix_cache_from_ids(vm, prefix, block_size=32, capacity=192)
    chk = rt.build_prefix_cache_from_ids(vm, prefix, block_size=32, capacity=192, chunked_prefill=True)
    oc = ort.build_prefix_cache_from_ids(ref, prefix, block_size=32, capacity=192)
    assert one.prefix_len == chk.prefix_len == 128
    for name, a, b, o in (("K", one.k, chk.k, oc.k), ("V", one.v, chk.v, oc.v)):
        np.testing.assert_allclose(to_np(b[:, :, :128]), to_np(a[:, :, :128]), rtol=2e-2, atol=2e-2, err_msg=name)
        np.testing.assert_allclose(to_np(b[:, :, :128]), o[:, :, :128], rtol=2e-2, atol=2e-2, err_msg=name)
    blk = [MASK] * 32
    h1 = to_np(vm.get_logits(rt._forward_cached(vm, blk, one)))[0]
    h2 = to_np(vm.get_logits(rt._forward_cached(vm, blk, chk)))[0]
    ho = ref.get_logits(ort.forward_cached(ref, blk, oc))[0]
    d12, d2o, d1o = (float(np.abs(h1 - h2).max()), float(np.abs(h2 - ho).max()), float(np.abs(h1 - ho).max()))
    log(f"  logits after the prefill: |one - chunked| {d12:.4g}, |chunked - oracle| {d2o:.4g}, |one - oracle| {d1o:.4g}")
    assert d2o <= 2 * d1o + 0.05
    with pytest.raises(ValueError, match="block-aligned"):
        rt.build_prefix_cache_from_ids(vm, prefix[:100], block_size=32, chunked_prefill=True)


def test_tied_get_logits_matches_untied():
    """Tied get_logits (embed_tokens.weight) == an untied lm_head holding the same array, bit for bit."""
    from fast_dllm_relax_amd.config import FastDLLMConfig
    from fast_dllm_relax_amd.params import from_numpy
    from fast_dllm_relax_amd.vm import HipVM
    from oracle.model import OracleConfig, random_params

    kw = dict(SMALL, tie_word_embeddings=True)
    arrays = random_params(OracleConfig(**kw), 35, "bfloat16")
    cfg_t, cfg_u = FastDLLMConfig(**kw), FastDLLMConfig(**dict(kw, tie_word_embeddings=False))
    untied = dict(arrays, **{"lm_head.weight": arrays["model.embed_tokens.weight"]})
    vm_t = HipVM(cfg_t, from_numpy(arrays, cfg_t), dtype="bfloat16")
    vm_u = HipVM(cfg_u, from_numpy(untied, cfg_u), dtype="bfloat16")
    rng = np.random.default_rng(2)
    for rows in (8, 32, 45):
        hidden = torch.from_numpy(rng.standard_normal((1, rows, kw["hidden_size"])).astype(np.float32)).to(
            "cuda", torch.bfloat16)
        lt, lu = vm_t.get_logits(hidden), vm_u.get_logits(hidden)
        assert torch.equal(lt.view(torch.int32), lu.view(torch.int32)), rows
    log("  tied and untied heads agree bit for bit at 8, 32 and 45 rows")
