"""The decode loop with the on-device threshold unmask (fdllm_unmask / fdllm_get_confidence_unmask,
include/fdllm.h), against the oracle.  Marked gpu; every call goes through the C ABI.

* The rule itself is bit-exact with oracle/confidence.c's fd_unmask (runtime.py:794-805) on random
  probabilities, including values exactly at the fp32 threshold, ties and all-masked / no-masked rows.
* The fused lm_head + confidence + unmask returns the same bits as fdllm_get_confidence.
* relax_greedy_generate on the device loop against oracle.runtime.greedy_generate in the same dtype:
  every device decision equals fd_unmask applied to that step's own probabilities, and the token trace
  equals the oracle's, or first diverges at a step where the oracle's own decision sits within the
  measured logit error of a tie (a top-2 logit gap or a probability at the threshold), which no
  implementation with different accumulation order can be required to reproduce.
"""

from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest
import torch

from oracle import confidence as oconf
from oracle.runtime import build_prefix_cache_from_ids as o_build
from oracle.runtime import forward_cached as o_forward_cached
from oracle.runtime import greedy_generate
from helpers import WIDE2, log, make_pair, to_np

pytestmark = pytest.mark.gpu

THR = 0.9
SMALL = dict(vocab_size=1000, hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
             num_key_value_heads=2, head_dim=128, tie_word_embeddings=False)


def _rt():
    from fast_dllm_relax_amd import _lib, runtime

    return _lib, runtime


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


@pytest.fixture(scope="module")
def small_pair():
    return make_pair(SMALL, 21, "bfloat16", lm_head_std=1.25, max_rows=256)


def _expected(ids, maxp, block, row0, s0, sub, mask_id):
    src = [max(row0 + r - 1, 0) for r in range(sub)]
    p = maxp[src].astype(np.float32)
    masked = block[s0:s0 + sub] == mask_id
    sel = oconf.unmask(p, masked, THR)
    out = block.copy()
    out[s0:s0 + sub][sel] = ids[src][sel]
    return out, sel, masked, p


def test_unmask_rule_bit_exact_random(small_pair):
    _lib, rt = _rt()
    _, vm = small_pair
    rng = np.random.default_rng(31)
    n, bd, sub, mask_id = 600, 32, 8, 999
    thr32 = np.float32(rt.threshold_f32(THR))
    cases = []
    ids_h = np.zeros((n, 32), np.int32)
    p_h = np.zeros((n, 32), np.float32)
    blk_h = np.zeros((n, bd), np.int32)
    for i in range(n):
        full = bool(rng.random() < 0.5)
        rows = 32 if full else 8
        s0 = int(rng.integers(0, 4)) * 8
        row0 = s0 if full else 0
        ids_h[i, :rows] = rng.integers(0, 999, rows)
        p = rng.random(rows).astype(np.float32)
        kind = rng.integers(0, 4)
        if kind == 1:  # values at the fp32 threshold and one ulp either side
            for j in rng.integers(0, rows, 3):
                p[j] = [thr32, np.nextafter(thr32, np.float32(1)), np.nextafter(thr32, np.float32(0))][rng.integers(0, 3)]
        elif kind == 2:  # ties below the threshold: the fallback takes the first
            p[:] = np.float32(0.25)
        elif kind == 3:
            p = (0.9 + 0.1 * rng.random(rows)).astype(np.float32)
        p_h[i, :rows] = p
        blk = rng.integers(0, 999, bd).astype(np.int32)
        mk = rng.random(bd) < [0.0, 1.0, 0.5, 0.3][rng.integers(0, 4)]
        blk[mk] = mask_id
        blk_h[i] = blk
        cases.append((rows, row0, s0))
    words = 4 + bd + 2 * sub + 4
    ids_d = torch.from_numpy(ids_h).cuda()
    p_d = torch.from_numpy(p_h).cuda()
    blk_d = torch.from_numpy(blk_h).cuda()
    rep_d = torch.zeros((n, words), dtype=torch.int32, device="cuda")
    for i, (rows, row0, s0) in enumerate(cases):
        _lib.check(vm.lib.fdllm_unmask(vm.ctx, ids_d[i].data_ptr(), p_d[i].data_ptr(), rows, row0, blk_d[i].data_ptr(),
                                       s0, sub, mask_id, float(thr32), rep_d[i].data_ptr(), i + 1, _stream()))
    torch.cuda.synchronize()
    got_blk, rep = blk_d.cpu().numpy(), rep_d.cpu().numpy()
    for i, (rows, row0, s0) in enumerate(cases):
        want, sel, masked, p = _expected(ids_h[i, :rows], p_h[i, :rows], blk_h[i], row0, s0, sub, mask_id)
        np.testing.assert_array_equal(got_blk[i], want, err_msg=f"case {i} {cases[i]}")
        r = rep[i]
        assert r[0] == i + 1
        np.testing.assert_array_equal(r[4:4 + bd], want)
        assert r[1] == int((masked & ~sel).sum()) and r[2] == int(sel.sum())
        assert r[3] == ids_h[i, rows - 1]
        np.testing.assert_array_equal(r[4 + bd + sub:4 + bd + 2 * sub].view(np.float32), p)
        m64 = (int(r[4 + bd + 2 * sub]) & 0xFFFFFFFF) | (int(r[4 + bd + 2 * sub + 1]) & 0xFFFFFFFF) << 32
        s64 = (int(r[4 + bd + 2 * sub + 2]) & 0xFFFFFFFF) | (int(r[4 + bd + 2 * sub + 3]) & 0xFFFFFFFF) << 32
        assert m64 == sum(1 << j for j in range(sub) if masked[j])
        assert s64 == sum(1 << j for j in range(sub) if sel[j])
    log(f"  {n} random unmask cases bit-exact with fd_unmask")


def test_unmask_sub_block_past_32_rows():
    """A 64-row block refined as one 64-row sub-block: the report's masked / selected masks carry all 64
    rows (a low and a high word each), and the block update matches fd_unmask."""
    _lib, rt = _rt()
    _, vm = make_pair(dict(SMALL, bd_size=64), 25, "bfloat16", max_rows=64)
    rng = np.random.default_rng(26)
    thr32 = np.float32(rt.threshold_f32(THR))
    bd = sub = 64
    for i, frac in enumerate((0.6, 1.0, 0.2)):
        ids_h = rng.integers(0, 999, 64).astype(np.int32)
        p_h = rng.random(64).astype(np.float32)
        p_h[rng.integers(32, 64, 5)] = np.float32(0.95)  # rows past 32 crossing the threshold
        blk_h = rng.integers(0, 999, bd).astype(np.int32)
        blk_h[rng.random(bd) < frac] = 999
        ids_d, p_d, blk_d = (torch.from_numpy(a).cuda() for a in (ids_h, p_h, blk_h))
        rep_d = torch.zeros(4 + bd + 2 * sub + 4, dtype=torch.int32, device="cuda")
        _lib.check(vm.lib.fdllm_unmask(vm.ctx, ids_d.data_ptr(), p_d.data_ptr(), 64, 0, blk_d.data_ptr(), 0, sub, 999,
                                       float(thr32), rep_d.data_ptr(), i + 1, _stream()))
        torch.cuda.synchronize()
        want, sel, masked, _ = _expected(ids_h, p_h, blk_h, 0, 0, sub, 999)
        r = rep_d.cpu().numpy()
        np.testing.assert_array_equal(blk_d.cpu().numpy(), want)
        m64 = (int(r[4 + bd + 2 * sub]) & 0xFFFFFFFF) | (int(r[4 + bd + 2 * sub + 1]) & 0xFFFFFFFF) << 32
        s64 = (int(r[4 + bd + 2 * sub + 2]) & 0xFFFFFFFF) | (int(r[4 + bd + 2 * sub + 3]) & 0xFFFFFFFF) << 32
        assert m64 == sum(1 << j for j in range(sub) if masked[j])
        assert s64 == sum(1 << j for j in range(sub) if sel[j])
        assert r[1] == int((masked & ~sel).sum()) and r[2] == int(sel.sum())
    vm.close()


def test_unmask_rejects_bad_windows(small_pair):
    _lib, _ = _rt()
    _, vm = small_pair
    ids = torch.zeros(32, dtype=torch.int32, device="cuda")
    p = torch.zeros(32, dtype=torch.float32, device="cuda")
    blk = torch.zeros(32, dtype=torch.int32, device="cuda")
    for rows, row0, s0, sub in [(8, 1, 0, 8), (32, 0, 28, 8), (0, 0, 0, 8), (8, 0, -1, 8)]:
        with pytest.raises(ValueError):
            _lib.check(vm.lib.fdllm_unmask(vm.ctx, ids.data_ptr(), p.data_ptr(), rows, row0, blk.data_ptr(), s0, sub,
                                           999, 0.9, None, 1, _stream()))


def test_fused_confidence_unmask_equals_confidence(small_pair):
    _lib, rt = _rt()
    _, vm = small_pair
    torch.manual_seed(3)
    for rows, row0, s0 in [(32, 8, 8), (8, 0, 16), (32, 0, 0)]:
        hidden = (torch.randn((1, rows, 256)) * 2).to(torch.bfloat16).cuda()
        ids_u, p_u = vm.get_confidence(hidden)
        blk = torch.full((32,), 999, dtype=torch.int32, device="cuda")
        blk[::3] = 5
        blk0 = blk.cpu().numpy()
        ids_f = torch.empty(rows, dtype=torch.int32, device="cuda")
        p_f = torch.empty(rows, dtype=torch.float32, device="cuda")
        thr = rt.threshold_f32(THR)
        _lib.check(vm.lib.fdllm_get_confidence_unmask(vm.ctx, hidden.data_ptr(), rows, row0, blk.data_ptr(), s0, 8, 999,
                                                      thr, ids_f.data_ptr(), p_f.data_ptr(), None, 1, _stream()))
        torch.cuda.synchronize()
        np.testing.assert_array_equal(ids_f.cpu().numpy(), ids_u.cpu().numpy()[0])
        np.testing.assert_array_equal(p_f.cpu().numpy().view(np.int32), p_u.cpu().numpy()[0].view(np.int32))
        want, *_ = _expected(ids_u.cpu().numpy()[0], p_u.cpu().numpy()[0], blk0, row0, s0, 8, 999)
        np.testing.assert_array_equal(blk.cpu().numpy(), want)


def test_fused_unmask_without_confidence_outputs(small_pair):
    """Without the ids / maxp outputs the fused kernel combines only the rows the rule reads (the shifted
    sub-block and, for the report, the last row): the block update and the report equal the rule applied
    to the full confidence, including the report-only call (sub 0)."""
    _lib, rt = _rt()
    _, vm = small_pair
    torch.manual_seed(4)
    thr = rt.threshold_f32(THR)
    bd = 32
    for rows, row0, s0, sub in [(32, 0, 0, 8), (32, 8, 8, 8), (32, 24, 24, 8), (8, 0, 16, 8), (32, 5, 3, 20),
                                (32, 0, 0, 0), (8, 0, 0, 0)]:
        log(f"case: fused unmask rows={rows} row0={row0} s0={s0} sub={sub}")
        hidden = (torch.randn((1, rows, 256)) * 2).to(torch.bfloat16).cuda()
        ids_u, p_u = vm.get_confidence(hidden)
        ids_h, p_h = ids_u.cpu().numpy()[0], p_u.cpu().numpy()[0]
        blk = torch.full((bd,), 999, dtype=torch.int32, device="cuda")
        blk[::3] = 5
        blk0 = blk.cpu().numpy()
        rep = torch.zeros(4 + bd + 2 * sub + 4, dtype=torch.int32, device="cuda")
        _lib.check(vm.lib.fdllm_get_confidence_unmask(vm.ctx, hidden.data_ptr(), rows, row0, blk.data_ptr(), s0, sub,
                                                      999, thr, None, None, rep.data_ptr(), 7, _stream()))
        torch.cuda.synchronize()
        if sub:
            want, sel, masked, _ = _expected(ids_h, p_h, blk0, row0, s0, sub, 999)
        else:
            want, sel, masked = blk0, np.zeros(0, bool), np.zeros(0, bool)
        np.testing.assert_array_equal(blk.cpu().numpy(), want)
        r = rep.cpu().numpy()
        assert r[0] == 7 and r[3] == ids_h[rows - 1]
        np.testing.assert_array_equal(r[4:4 + bd], want)
        src = [max(row0 + j - 1, 0) for j in range(sub)]
        np.testing.assert_array_equal(r[4 + bd:4 + bd + sub], ids_h[src])
        np.testing.assert_array_equal(r[4 + bd + sub:4 + bd + 2 * sub], p_h[src].view(np.int32))
        assert r[2] == int(sel.sum()) and r[1] == int((masked & ~sel).sum())


def _check_decisions(decisions):
    """Every cached decision is fd_unmask of that step's own fp32 probabilities (bit-exact given the
    logits); a stateless one (runtime.py:806-837) unmasks the masked rows whose float64 probability
    exceeds the threshold, else the first of the largest."""
    n = 0
    for d in decisions:
        if d["kind"] == "append":
            continue
        sub = len(d["ids"])
        masked = np.zeros(sub, bool)
        masked[d["masked"]] = True
        if d["kind"] == "stateless":
            p = np.asarray(d["probs"], np.float64)
            sel = [r for r in d["masked"] if p[r] > THR]
            if not sel:
                g = np.where(masked, p, -np.inf)
                sel = [int(np.argmax(g))]
            assert list(sel) == list(d["selected"]), d
        else:
            sel = oconf.unmask(np.asarray(d["probs"], np.float32), masked, THR)
            assert list(np.nonzero(sel)[0]) == list(d["selected"]), d
        n += 1
    return n


def _fragile(od, delta):
    """Whether the oracle's decision at this step lies within the logit error `delta` of another one: a
    selected or candidate row whose top-2 logit gap is below 2 delta, a masked row whose probability is
    within the corresponding band of the threshold, or a fallback between rows of near-equal probability."""
    if od["kind"] == "append":
        return od["gap"] <= 2 * delta
    band = math.expm1(2 * delta)
    masked = list(od["masked"])
    p = np.asarray(od["probs"], np.float64)
    gap = np.asarray(od["gap"], np.float64)
    if any(gap[r] <= 2 * delta for r in masked):
        return True
    if any(abs(p[r] - THR) <= band * p[r] for r in masked):
        return True
    if all(p[r] <= THR for r in masked) and len(masked) > 1:
        top = sorted((p[r] for r in masked), reverse=True)
        return top[0] - top[1] <= band * top[0]
    return False


class _LoggedTrace(list):
    """A trace list that prints each call as it is logged (a long oracle loop then shows progress)."""

    def __init__(self, name):
        super().__init__()
        self.name = name

    def append(self, item):
        super().append(item)
        if len(self) % 8 == 1:
            log(f"    {self.name} call {len(self)}: {item[0]}")


def _loop_vs_oracle(ref, vm, prompt, new_tokens, mask_id, delta, device_loop=True, verbose=False):
    _, rt = _rt()
    common = dict(max_new_tokens=new_tokens, block_size=32, small_block_size=8, threshold=THR, mask_id=mask_id,
                  stop_token=None)
    tr_h, dec_h = [], []
    out_h, st_h = rt.relax_greedy_generate(vm, prompt, trace=tr_h, decisions=dec_h, device_loop=device_loop, **common)
    log(f"  HIP loop ({'device' if device_loop else 'host'} rule): {len(out_h)} tokens, {st_h}")
    n = _check_decisions(dec_h)
    log(f"  {n} unmask decisions equal the rule applied to their own probabilities")
    assert sum(len(d["selected"]) > 1 for d in dec_h if d["kind"] != "append") > 0, "no step crossed the threshold"
    tr_o, dec_o = (_LoggedTrace("oracle") if verbose else []), []
    out_o, st_o = greedy_generate(ref, prompt, trace=tr_o, decisions=dec_o, **common)
    log(f"  oracle loop: {len(out_o)} tokens, {st_o}")
    first = next((i for i, (a, b) in enumerate(zip(tr_h, tr_o)) if a != b), None)
    if first is None:
        assert len(tr_h) == len(tr_o) and out_h == out_o
        log(f"  traces identical over {len(tr_h)} calls")
        return
    # decisions line up with trace entries after the aligned-prompt append
    off = len(tr_o) - len(dec_o)
    od = dec_o[first - off]
    log(f"  traces diverge at call {first}/{len(tr_o)}: HIP {tr_h[first]} oracle {tr_o[first]} (oracle decision {od})")
    assert first >= off and _fragile(od, delta), "divergence at a decision the logit error cannot explain"


def _measured_logit_error(ref, vm, prompt, mask_id):
    """max |logit_HIP - logit_oracle| of one cached 32-row step after the prompt's prefix."""
    _, rt = _rt()
    P = len(prompt) // 32 * 32
    blk = list(prompt[P - 32:P])[:1] + [mask_id] * 31
    oc = o_build(ref, list(prompt[:P - 32]), block_size=32, capacity=P + 32)
    lo = ref.get_logits(o_forward_cached(ref, blk, oc))[0]
    hc = rt.build_prefix_cache_from_ids(vm, list(prompt[:P - 32]), block_size=32, capacity=P + 32)
    lh = to_np(vm.get_logits(rt._forward_cached(vm, blk, hc)))[0]
    delta = float(np.abs(lh - lo).max())
    log(f"  measured logit error of one cached step: max |dlogit| = {delta:.4g} (logit scale {np.abs(lo).max():.1f})")
    return delta


def test_decode_loop_small_matches_oracle(small_pair):
    ref, vm = small_pair
    prompt = [int(t) for t in np.random.default_rng(22).integers(0, 999, 64)]
    delta = _measured_logit_error(ref, vm, prompt, 999)
    _loop_vs_oracle(ref, vm, prompt, 96, 999, delta)


def test_decode_loop_small_unaligned_prompt(small_pair):
    """An unaligned prompt: the first cached block holds prompt tokens (partial steps start at rp0)."""
    ref, vm = small_pair
    prompt = [int(t) for t in np.random.default_rng(23).integers(0, 999, 77)]
    delta = _measured_logit_error(ref, vm, prompt, 999)
    _loop_vs_oracle(ref, vm, prompt, 64, 999, delta)


@pytest.mark.timeout(600)
def test_decode_loop_cfg3_shape_matches_oracle():
    """BASELINE cfg3's regime at two layers: the 1.5B widths, seed 2, untied lm_head N(0, 0.5), a 2048-token
    prompt and 64 new tokens."""
    from fast_dllm_relax_amd.config import DEFAULT_MASK_ID

    kw = dict(WIDE2, tie_word_embeddings=False)
    ref, vm = make_pair(kw, 2, "bfloat16", lm_head_std=0.5, max_rows=2048)
    prompt = [int(t) for t in np.random.default_rng(2).integers(0, 150000, 2048)]
    delta = _measured_logit_error(ref, vm, prompt, DEFAULT_MASK_ID)
    _loop_vs_oracle(ref, vm, prompt, 64, DEFAULT_MASK_ID, delta)
    vm.close()


def test_host_loop_small_matches_oracle(small_pair):
    """relax_greedy_generate with the reference's host rule (device_loop=False): score_active_block_refine /
    _partial_perlayer / _cached_fast and the threshold decision on the host, as runtime.py:794-805."""
    ref, vm = small_pair
    prompt = [int(t) for t in np.random.default_rng(22).integers(0, 999, 64)]
    delta = _measured_logit_error(ref, vm, prompt, 999)
    _loop_vs_oracle(ref, vm, prompt, 96, 999, delta, device_loop=False)


def test_host_loop_small_unaligned_prompt(small_pair):
    ref, vm = small_pair
    prompt = [int(t) for t in np.random.default_rng(23).integers(0, 999, 77)]
    delta = _measured_logit_error(ref, vm, prompt, 999)
    _loop_vs_oracle(ref, vm, prompt, 64, 999, delta, device_loop=False)


@pytest.mark.parametrize("device_loop", [True, False])
def test_loop_short_prompt_stateless_first_block(small_pair, device_loop):
    """A 20-token prompt: the first block is refined statelessly (score_sequence_block, float64 probabilities
    and the gated argmax, runtime.py:719-721, 806-837), then the block is appended and the loop turns to
    the cache."""
    ref, vm = small_pair
    prompt = [int(t) for t in np.random.default_rng(24).integers(0, 999, 20)]
    # the stateless block's logit error: a dense forward over the prompt and its masks
    from oracle.runtime import score_sequence_block as o_ssb

    _, rt = _rt()
    seq = prompt + [999] * 12
    _, sh_o = o_ssb(ref, seq, block_size=32)
    _, sh_h = rt.score_sequence_block(vm, seq, block_size=32)
    delta = float(np.abs(np.asarray(sh_h, np.float32) - sh_o).max())
    log(f"  stateless block logit error: max |dlogit| = {delta:.4g}")
    _loop_vs_oracle(ref, vm, prompt, 64, 999, delta, device_loop=device_loop)


@pytest.mark.timeout(900)
def test_decode_loop_cfg3_full_depth():
    """BASELINE cfg3 at full depth: the 28-layer 1.5B model with bench.py's weights (seed 2, untied lm_head
    N(0, 0.5)), a 2048-token prompt and 64 new tokens, on the device loop, against the bf16 oracle loop
    under the divergence rule above (the measured logit error of one cached step at this depth sets it)."""
    from fast_dllm_relax_amd.config import DEFAULT_MASK_ID, fast_dllm_v2_1p5b
    from fast_dllm_relax_amd.params import param_names, random_params_torch
    from fast_dllm_relax_amd.vm import HipVM
    from oracle.model import OracleConfig, OracleModel

    cfg = fast_dllm_v2_1p5b(tie_word_embeddings=False)
    log("setup: 1.5B bf16, 28 layers, seed 2, lm_head N(0, 0.5)")
    params = random_params_torch(cfg, 2, dtype="bfloat16", device="cuda", lm_head_std=0.5)
    vm = HipVM(cfg, params, dtype="bfloat16", max_rows=2048)
    ocfg = OracleConfig(vocab_size=cfg.vocab_size, hidden_size=cfg.hidden_size, intermediate_size=cfg.intermediate_size,
                        num_hidden_layers=cfg.num_hidden_layers, num_attention_heads=cfg.num_attention_heads,
                        num_key_value_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim, tie_word_embeddings=False)
    ref = OracleModel(ocfg, {n: p.float().cpu().numpy() for n, p in zip(param_names(cfg), params)}, "bfloat16")
    prompt = [int(t) for t in np.random.default_rng(2).integers(0, 150000, 2048)]
    delta = _measured_logit_error(ref, vm, prompt, DEFAULT_MASK_ID)
    _loop_vs_oracle(ref, vm, prompt, 64, DEFAULT_MASK_ID, delta, verbose=True)
    vm.close()
