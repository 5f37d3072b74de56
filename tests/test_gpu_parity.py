"""HIP path vs the CPU oracle on the same seeded weights and inputs (calls go through the C ABI)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import TINY, WIDE2, bf16_parity, log, make_pair, to_np
from oracle import confidence as oconf
from oracle.model import build_prefix_block_attention_bias

pytestmark = pytest.mark.gpu

TOL = dict(rtol=2e-2, atol=2e-2)  # bf16 activations; the reference's own tests use 2e-2 (test_tiny_compile.py:282)


def _ids(rng, n, vocab):
    return rng.integers(0, vocab - 1, n)


def _dev_ids(ids):
    return torch.tensor(np.asarray(ids), dtype=torch.int32, device="cuda")


def _off(v):
    return torch.tensor(int(v), dtype=torch.int32, device="cuda")


@pytest.fixture(scope="module")
def tiny():
    log("setup: tiny bf16 model seed 0")
    return make_pair(TINY, 0)


def test_embed_bit_exact(tiny):
    ref, vm = tiny
    ids = _ids(np.random.default_rng(1), 37, TINY["vocab_size"])
    log("case: embed 37 rows")
    got = to_np(vm.embed(_dev_ids(ids)))
    np.testing.assert_array_equal(got, ref.embed(ids))


def test_get_logits_matches_oracle(tiny):
    ref, vm = tiny
    rng = np.random.default_rng(2)
    for rows in (8, 32, 45):
        log(f"case: get_logits rows={rows}")
        h = ref.rnd(rng.standard_normal((1, rows, TINY["hidden_size"])).astype(np.float32))
        got = to_np(vm.get_logits(torch.from_numpy(h).to("cuda", torch.bfloat16)))
        want = ref.get_logits(h)
        # fp32 accumulation order differs; the bf16 rounding of the logits may flip by one ulp
        np.testing.assert_allclose(got, want, rtol=1e-2, atol=1e-2)
        assert np.mean(got == want) > 0.98


def test_prefill_and_cached_step_match_oracle(tiny):
    ref, vm = tiny
    rng = np.random.default_rng(3)
    P, R, cap = 64, 32, 128
    ids = _ids(rng, P + R, TINY["vocab_size"])
    kc = np.full((2, 1, cap, 2, 128), 7.0, np.float32)
    vc = kc.copy()
    ref.build_prefix_cache(ref.embed(ids[:P])[None], build_prefix_block_attention_bias(0, P, block_size=32), kc, vc)
    h_ref = ref.forward_cached(ref.embed(ids[P:])[None], kc, vc, P, P)
    k = torch.full((2, 1, cap, 2, 128), 7.0, dtype=torch.bfloat16, device="cuda")
    v = k.clone()
    log("case: build_prefix_cache P=64 (arithmetic block-causal)")
    vm.build_prefix_cache(vm.embed(_dev_ids(ids[:P]))[None], None, k, v)
    kn = to_np(k)
    np.testing.assert_allclose(kn[:, :, :P], kc[:, :, :P], **TOL)
    assert (kn[:, :, P:] == 7.0).all(), "build_prefix_cache wrote past the prefix"
    log("case: forward_cached R=32 at P=64")
    h = to_np(vm.forward_cached(vm.embed(_dev_ids(ids[P:]))[None], k, v, _off(P), P))
    np.testing.assert_allclose(h, h_ref, **TOL)
    kn = to_np(k)
    np.testing.assert_allclose(kn[:, :, P:P + R], kc[:, :, P:P + R], **TOL)
    assert (kn[:, :, P + R:] == 7.0).all(), "forward_cached wrote past the block"
    for rp in (0, 8, 16, 24):
        log(f"case: forward_block_partial_rp{rp}")
        small = ids[P + rp:P + rp + 8]
        kc2, vc2 = kc.copy(), vc.copy()
        h_ref_p = ref.forward_block_partial(rp, ref.embed(small)[None], kc2, vc2, P + rp, P)
        before = to_np(k)
        h_p = to_np(vm[f"forward_block_partial_rp{rp}"](vm.embed(_dev_ids(small))[None], k, v, _off(P + rp), P))
        np.testing.assert_allclose(h_p, h_ref_p, **TOL)
        # same tokens at the same rows: the partial step reproduces the full step's rows (cuda.py:740-756)
        np.testing.assert_allclose(h_p, h_ref[:, rp:rp + 8], **TOL)
        after = to_np(k)
        outside = np.ones(cap, bool)
        outside[P + rp:P + rp + 8] = False
        np.testing.assert_array_equal(after[:, :, outside], before[:, :, outside])


def test_forward_hidden_matches_oracle_and_dense_equals_cached(tiny):
    """forward_hidden against the oracle (explicit bias and the arithmetic block-causal rule), and the
    HIP path's cached and partial rows against its own dense block-causal rows."""
    ref, vm = tiny
    rng = np.random.default_rng(4)
    S = 96
    ids = _ids(rng, S, TINY["vocab_size"])
    bias = build_prefix_block_attention_bias(0, S, block_size=32)
    log("case: forward_hidden S=96 with explicit bias")
    h_ref = ref.forward_hidden(ref.embed(ids)[None], bias)
    x = vm.embed(_dev_ids(ids))[None]
    h = to_np(vm.forward_hidden(x, torch.from_numpy(bias).cuda()))
    np.testing.assert_allclose(h, h_ref, **TOL)
    log("case: forward_hidden S=96 arithmetic block-causal")
    h2 = to_np(vm.forward_hidden(x, None))
    np.testing.assert_allclose(h2, h, rtol=1e-2, atol=1e-2)
    # the reference's invariant (tests/test_tiny_compile.py:264-290): the cached step's rows equal the
    # dense block-causal forward's rows, and each partial step equals the full cached step's rows for its
    # sub-block (the cached path runs other attention kernels, hence the bf16 tolerance)
    log("case: cached rows == dense block-causal rows, partial rows == cached rows")
    P, L, nkv = 64, TINY["num_hidden_layers"], TINY["num_key_value_heads"]
    k = torch.zeros((L, 1, 128, nkv, 128), dtype=torch.bfloat16, device="cuda")
    v = torch.zeros_like(k)
    vm.build_prefix_cache(x[:, :P], None, k, v)
    hc = to_np(vm.forward_cached(x[:, P:], k, v, _off(P), P))
    np.testing.assert_allclose(hc, h2[:, P:], **TOL)
    for rp in (0, 8, 16, 24):
        hp = to_np(vm[f"forward_block_partial_rp{rp}"](x[:, P + rp:P + rp + 8].contiguous(), k, v, _off(P + rp), P))
        np.testing.assert_allclose(hp, hc[:, rp:rp + 8], **TOL, err_msg=f"rp{rp}")


def test_write_window_errors(tiny):
    _, vm = tiny
    k = torch.zeros((2, 1, 64, 2, 128), dtype=torch.bfloat16, device="cuda")
    v = torch.zeros_like(k)
    x = torch.zeros((1, 32, TINY["hidden_size"]), dtype=torch.bfloat16, device="cuda")
    log("case: window errors")
    with pytest.raises(ValueError, match="outside cache capacity"):
        vm.forward_cached(x, k, v, _off(48), 48)
    with pytest.raises(ValueError):
        vm.forward_block_partial_rp8(x, k, v, _off(8), 0)  # 32 rows where 8 are required
    xs = torch.zeros((1, 8, TINY["hidden_size"]), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="outside cache capacity"):
        vm.forward_block_partial_rp24(xs, k, v, _off(56), 40)


def test_misaligned_arguments_rejected(tiny):
    """fdllm_bind_weights checks that every parameter is 16-byte aligned (the kernels read norm weights,
    biases and embedding rows in 16-byte units): a 2-byte-offset view is rejected with FDLLM_EINVAL, and
    the context keeps the weights it had (its logits are unchanged).  The entry points that take
    activations, caches or logits refuse such views the same way."""
    _, vm = tiny
    ids = _dev_ids(np.arange(32) % (TINY["vocab_size"] - 1))
    h = vm.embed(ids)[None]
    before = vm.get_logits(h).float().cpu()
    params = list(vm.params)
    i = 2  # a norm weight
    shifted = torch.empty(params[i].numel() + 1, dtype=params[i].dtype, device="cuda")[1:].view_as(params[i])
    shifted.copy_(params[i])
    bad = params[:i] + [shifted] + params[i + 1:]
    log("case: bind with a 2-byte-offset parameter")
    with pytest.raises(ValueError, match="not 16-byte aligned"):
        vm.bind(bad)
    vm.params = params
    after = vm.get_logits(h).float().cpu()
    assert torch.equal(before, after)
    log("case: forward_hidden / forward_cached with a 2-byte-offset activation view")
    xs = torch.empty(h.numel() + 1, dtype=h.dtype, device="cuda")[1:].view_as(h)
    xs.copy_(h)
    with pytest.raises(ValueError, match="16-byte aligned"):
        vm.forward_hidden(xs, None)
    k = torch.zeros((2, 1, 64, 2, 128), dtype=torch.bfloat16, device="cuda")
    v = torch.zeros_like(k)
    with pytest.raises(ValueError, match="16-byte aligned"):
        vm.forward_cached(xs, k, v, _off(0), 0)


def test_confidence_bit_exact_given_logits(tiny):
    ref, vm = tiny
    rng = np.random.default_rng(5)
    for rows, scale in ((32, 1.0), (8, 20.0), (3, 0.01)):
        log(f"case: confidence_from_logits rows={rows} scale={scale}")
        logits = ref.rnd(scale * rng.standard_normal((1, rows, TINY["vocab_size"])).astype(np.float32))
        logits[0, 0, 17] = logits[0, 0].max()  # a tie: the first index wins
        ids, maxp = vm.confidence_from_logits(torch.from_numpy(logits).cuda())
        wid, wp = oconf.confidence(logits[0])
        np.testing.assert_array_equal(ids.cpu().numpy()[0], wid)
        np.testing.assert_array_equal(maxp.cpu().numpy()[0].view(np.uint32), wp.view(np.uint32))


def test_fused_confidence_equals_confidence_of_get_logits(tiny):
    ref, vm = tiny
    rng = np.random.default_rng(6)
    for rows in (32, 8, 96, 130):  # 96 and 130 rows take the MFMA block kernel's logits epilogue
        log(f"case: fused lm_head+confidence rows={rows}")
        h = torch.from_numpy(ref.rnd(rng.standard_normal((1, rows, TINY["hidden_size"])).astype(np.float32)))
        h = h.to("cuda", torch.bfloat16)
        logits = torch.empty((1, rows, TINY["vocab_size"]), dtype=torch.float32, device="cuda")
        ids, maxp = vm.get_confidence(h, logits=logits)
        np.testing.assert_array_equal(to_np(logits), to_np(vm.get_logits(h)))
        wid, wp = oconf.confidence(to_np(logits)[0])
        np.testing.assert_array_equal(ids.cpu().numpy()[0], wid)
        np.testing.assert_array_equal(maxp.cpu().numpy()[0].view(np.uint32), wp.view(np.uint32))


@pytest.fixture(scope="module")
def wide2():
    log("setup: 1.5B-shape 2-layer bf16 model seed 1")
    return make_pair(WIDE2, 1)


def test_wide_cached_step_and_logits(wide2):
    """1.5B layer shapes: cached 32-row step at P=512 and its logits vs the bf16 oracle and the fp32
    oracle (same bf16-representable weights, no rounding anywhere)."""
    from oracle.model import OracleModel

    ref, vm = wide2
    ref32 = OracleModel(ref.cfg, ref.p, "float32")
    rng = np.random.default_rng(7)
    P, R, cap = 512, 32, 576
    ids = _ids(rng, P + R, WIDE2["vocab_size"])
    outs = {}
    for name, model in (("bf16", ref), ("f32", ref32)):
        kc = np.zeros((2, 1, cap, 2, 128), np.float32)
        vc = kc.copy()
        model.build_prefix_cache(model.embed(ids[:P])[None], build_prefix_block_attention_bias(0, P, block_size=32),
                                 kc, vc)
        h = model.forward_cached(model.embed(ids[P:])[None], kc, vc, P, P)
        outs[name] = (h, model.get_logits(h), kc)
    k = torch.zeros((2, 1, cap, 2, 128), dtype=torch.bfloat16, device="cuda")
    v = torch.zeros_like(k)
    log("case: wide build_prefix_cache P=512")
    vm.build_prefix_cache(vm.embed(_dev_ids(ids[:P]))[None], None, k, v)
    bf16_parity("prefix K", to_np(k)[:, :, :P], outs["bf16"][2][:, :, :P], outs["f32"][2][:, :, :P])
    log("case: wide forward_cached R=32")
    h = vm.forward_cached(vm.embed(_dev_ids(ids[P:]))[None], k, v, _off(P), P)
    bf16_parity("hidden", to_np(h), outs["bf16"][0], outs["f32"][0])
    log("case: wide logits")
    lg = to_np(vm.get_logits(h))
    # The reference's own bf16 precision order is ~0.04 from fp32 at the max over 4.9M logits (bf16
    # hidden-state rounding through the layers), so the bound is relative to it, not an absolute 3e-2.
    bf16_parity("logits", lg, outs["bf16"][1], outs["f32"][1])
    ids_d, maxp_d = vm.get_confidence(h)
    wid, wp = oconf.confidence(lg[0])
    np.testing.assert_array_equal(ids_d.cpu().numpy()[0], wid)
    np.testing.assert_array_equal(maxp_d.cpu().numpy()[0].view(np.uint32), wp.view(np.uint32))



def test_lm_head_tail_split(wide2, monkeypatch):
    """The lm_head of up to 32 rows runs its 256-column groups in whole rounds of one per compute unit and
    splits the groups past the last round three ways in k (1.5B: 82 of 594 groups on 256 units).  The
    other groups' logits are the unsplit kernel's bits; the split groups' differ only by the fp32 order
    of the three partial sums, so an entry can move to the neighbouring bf16 value, and few do.  The
    confidence stays bit-exact given the logits."""
    from fast_dllm_relax_amd.config import FastDLLMConfig
    from fast_dllm_relax_amd.params import from_numpy
    from fast_dllm_relax_amd.vm import HipVM

    ref, vm = wide2
    cfg = FastDLLMConfig(**WIDE2)
    monkeypatch.setenv("FDLLM_LM_TAIL", "0")
    vm_off = HipVM(cfg, from_numpy(ref.p, cfg, dtype="bfloat16"), dtype="bfloat16", max_rows=64)
    monkeypatch.delenv("FDLLM_LM_TAIL")
    ncu = torch.cuda.get_device_properties(0).multi_processor_count
    groups = -(-WIDE2["vocab_size"] // 256)
    c0 = groups // ncu * ncu * 256  # first column of the split groups
    assert 0 < c0 < WIDE2["vocab_size"]
    g = torch.Generator(device="cuda").manual_seed(13)
    try:
        for rows in (32, 17, 8, 1):
            log(f"case: lm_head tail split, {rows} rows, split from column {c0}")
            h = (torch.randn((1, rows, WIDE2["hidden_size"]), generator=g, device="cuda") * 2).to(torch.bfloat16)
            lg = to_np(vm.get_logits(h))
            lg0 = to_np(vm_off.get_logits(h))
            np.testing.assert_array_equal(lg[..., :c0], lg0[..., :c0])
            d = np.abs(lg[..., c0:] - lg0[..., c0:])
            moved = float(np.mean(d > 0))
            log(f"  split groups: {moved:.2e} of the entries moved, max |d| {d.max():.3g}")
            # a moved entry is the neighbouring bf16 value, or, where the sum cancels to near zero, within
            # the fp32 sums' own error
            u1 = (lg[..., c0:].view(np.uint32) >> 16).astype(np.int64)
            u0 = (lg0[..., c0:].view(np.uint32) >> 16).astype(np.int64)
            adjacent = ((u1 >> 15) == (u0 >> 15)) & (np.abs(u1 - u0) <= 1)
            assert np.all(adjacent | (d <= 1e-4)), "moved by more than one bf16 step"
            assert moved < 1e-2
            if rows == 32:
                assert moved > 0, "the split groups gave the unsplit bits everywhere: was the split taken?"
            logits = torch.empty((1, rows, WIDE2["vocab_size"]), dtype=torch.float32, device="cuda")
            ids, maxp = vm.get_confidence(h, logits=logits)
            np.testing.assert_array_equal(to_np(logits), lg)
            wid, wp = oconf.confidence(lg[0])
            np.testing.assert_array_equal(ids.cpu().numpy()[0], wid)
            np.testing.assert_array_equal(maxp.cpu().numpy()[0].view(np.uint32), wp.view(np.uint32))
    finally:
        vm_off.close()


def test_wide_forward_hidden_large_m(wide2):
    """Large-M projections (the MFMA block kernel) at the 1.5B layer shapes: a stateless block-causal
    forward over 160 rows (64-row blocks with k splits) and 1056 rows (128-row blocks, ragged last
    block) vs the bf16 and fp32 oracles."""
    from oracle.model import OracleModel

    ref, vm = wide2
    ref32 = OracleModel(ref.cfg, ref.p, "float32")
    rng = np.random.default_rng(11)
    for S in (160, 1056, 2080):
        ids = _ids(rng, S, WIDE2["vocab_size"])
        bias = build_prefix_block_attention_bias(0, S, block_size=32)
        want = ref.forward_hidden(ref.embed(ids)[None], bias)
        want32 = ref32.forward_hidden(ref32.embed(ids)[None], bias)
        log(f"case: wide forward_hidden S={S} arithmetic block-causal")
        got = to_np(vm.forward_hidden(vm.embed(_dev_ids(ids))[None], None))
        bf16_parity(f"hidden S={S}", got, want, want32)


def _log_softmax(x: np.ndarray) -> np.ndarray:
    x = x.astype(np.float64)
    m = x.max(axis=-1, keepdims=True)
    return x - m - np.log(np.exp(x - m).sum(axis=-1, keepdims=True))


def test_score_masked_continuation_matches_oracle(tiny):
    """Masked-continuation scoring (runtime.py:485-588) and the per-token log-probabilities the
    loglikelihood path takes from it (runners.py:839-881) vs the oracle: a prefix shorter than a block
    (the stateless path), a prefix with a partial last block, and a continuation longer than a block."""
    from fast_dllm_relax_amd.runtime import score_masked_continuation
    from oracle import runtime as ort

    ref, vm = tiny
    rng = np.random.default_rng(12)
    mask_id = TINY["vocab_size"] - 1
    for plen, clen in ((20, 5), (70, 9), (64, 40)):
        prefix = [int(t) for t in rng.integers(0, mask_id, plen)]
        cont = [int(t) for t in rng.integers(0, mask_id, clen)]
        log(f"case: score_masked_continuation prefix={plen} continuation={clen}")
        got, _ = score_masked_continuation(vm, prefix, cont, block_size=32, mask_id=mask_id)
        want = ort.score_masked_continuation(ref, prefix, cont, block_size=32, mask_id=mask_id)
        assert got.shape == want.shape == (clen, TINY["vocab_size"])
        np.testing.assert_allclose(got, want, **TOL)
        lp_got = _log_softmax(got)[np.arange(clen), cont]
        lp_want = _log_softmax(want)[np.arange(clen), cont]
        np.testing.assert_allclose(lp_got, lp_want, rtol=0, atol=2e-2)


def test_prefill_attention_configs_agree(wide2, monkeypatch):
    """The prefill attention kernel gives every query the same arithmetic whatever the number of query
    heads per workgroup (1, 2, 3 or 6 of a kv head's 6), so all four give bit-identical outputs."""
    from fast_dllm_relax_amd.config import FastDLLMConfig
    from fast_dllm_relax_amd.params import from_numpy
    from fast_dllm_relax_amd.vm import HipVM

    ref, vm0 = wide2
    rng = np.random.default_rng(13)
    S = 352
    ids = _ids(rng, S, WIDE2["vocab_size"])
    x = vm0.embed(_dev_ids(ids))[None]
    outs = {}
    for hpw in (1, 2, 3, 6):
        monkeypatch.setenv("FDLLM_PREFILL_HPW", str(hpw))
        cfg = FastDLLMConfig(**WIDE2)
        vm = HipVM(cfg, from_numpy(ref.p, cfg, dtype="bfloat16"), dtype="bfloat16", max_rows=S)
        log(f"case: prefill attention, {hpw} query heads per workgroup, S={S}")
        outs[hpw] = to_np(vm.forward_hidden(x, None))
        vm.close()
    for hpw in (2, 3, 6):
        np.testing.assert_array_equal(outs[hpw], outs[1])


def test_vm_from_artifact_equals_vm_from_tensors(tiny, tmp_path):
    """HipVM.from_artifact (the reference artifact's weight files) binds exactly the weights it was
    written from: a stateless forward is bit-identical."""
    from fast_dllm_relax_amd import params as P
    from fast_dllm_relax_amd.config import FastDLLMConfig
    from fast_dllm_relax_amd.vm import HipVM

    ref, vm = tiny
    cfg = FastDLLMConfig(**TINY)
    tensors = P.from_numpy(ref.p, cfg, dtype="bfloat16")
    P.save_artifact(tmp_path, cfg, tensors, "bfloat16")
    log("case: HipVM.from_artifact vs HipVM(tensors)")
    vm2 = HipVM.from_artifact(tmp_path, max_rows=64)
    ids = _dev_ids(np.random.default_rng(14).integers(0, TINY["vocab_size"] - 1, 64))
    a = to_np(vm.forward_hidden(vm.embed(ids)[None], None))
    b = to_np(vm2.forward_hidden(vm2.embed(ids)[None], None))
    vm2.close()
    np.testing.assert_array_equal(a, b)


def test_long_context_prefill_and_cached_step(tiny):
    """A prefix past 64 key chunks of 128 (P = 8200, ragged): the prefill kernel over 8200 rows, then a
    32-row cached step whose attention takes the split loop kernel (more than 64 chunks), vs the oracle."""
    ref, vm = tiny
    from oracle.model import OracleModel

    ref32 = OracleModel(ref.cfg, ref.p, "float32")
    rng = np.random.default_rng(15)
    P, R = 8200, 32
    cap = P + 64
    ids = _ids(rng, P + R, TINY["vocab_size"])
    L, nkv, hd = TINY["num_hidden_layers"], TINY["num_key_value_heads"], TINY["head_dim"]
    outs = {}
    for name, model in (("bf16", ref), ("f32", ref32)):
        kc = np.zeros((L, 1, cap, nkv, hd), np.float32)
        vc = kc.copy()
        model.build_prefix_cache(model.embed(ids[:P])[None], build_prefix_block_attention_bias(0, P, block_size=32),
                                 kc, vc)
        outs[name] = (model.forward_cached(model.embed(ids[P:])[None], kc, vc, P, P), kc)
    k = torch.zeros((L, 1, cap, nkv, hd), dtype=torch.bfloat16, device="cuda")
    v = torch.zeros_like(k)
    log(f"case: build_prefix_cache P={P}")
    vm.build_prefix_cache(vm.embed(_dev_ids(ids[:P]))[None], None, k, v)
    bf16_parity("long prefix K", to_np(k)[:, :, :P], outs["bf16"][1][:, :, :P], outs["f32"][1][:, :, :P])
    log(f"case: forward_cached R={R} over {P + R} keys")
    h = vm.forward_cached(vm.embed(_dev_ids(ids[P:]))[None], k, v, _off(P), P)
    bf16_parity("long-context hidden", to_np(h), outs["bf16"][0], outs["f32"][0])
