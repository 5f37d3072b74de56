"""Golden fixtures (tests/golden/, written by tests/golden/make_golden.py).

CPU: the oracle still reproduces the fixtures bit for bit (a change to the oracle that moves any
trace, token or logit fails here), and the cfg1 fixture's logits agree with the local transformers
Qwen2 on the same weights, which pins the fixture independently of the oracle.  GPU: the HIP path,
through the C ABI, against the hd128 fixture (bf16 and fp32 oracle outputs) with the bf16 parity
criterion of tests/helpers.py, and the confidence of its logits bit-exact with the C oracle's.
"""

from __future__ import annotations

import pathlib
import sys

import numpy as np
import pytest
import torch

from helpers import bf16_parity, log, make_pair, to_np

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))

import make_golden  # noqa: E402


def _load(name):
    with np.load(GOLDEN / name) as d:
        return {k: d[k] for k in d.files}


def test_cfg1_oracle_reproduces_fixture():
    want = _load("cfg1_tiny.npz")
    got = make_golden.cfg1_fixture()
    assert set(got) == set(want)
    for k in ("prompt", "tokens", "trace", "stats", "refine_active", "refine_ids", "partial_ids"):
        np.testing.assert_array_equal(got[k], want[k], err_msg=k)
    for k in ("refine_hidden", "refine_logits", "refine_maxp", "partial_maxp"):
        np.testing.assert_allclose(got[k], want[k], rtol=0, atol=1e-6, err_msg=k)
    # the loop took all four kinds of call: stateless first block, full refinement, partial, append
    assert set(want["trace"][:, 0].tolist()) == {0, 1, 2, 3}
    assert want["stats"][2] > 0, "no partial (block-cache) step in the fixture"


def test_cfg1_fixture_matches_transformers():
    """The fixture's cached refinement logits against transformers' Qwen2 over the dense sequence
    (prefix block-causal, the active block sees everything: the cached step's attention)."""
    from oracle.model import OracleConfig, build_prefix_block_attention_bias, random_params
    from test_oracle_pinning import _hf_model

    want = _load("cfg1_tiny.npz")
    cfg = OracleConfig(**make_golden.CFG1)
    hf = _hf_model(cfg, random_params(cfg, 0, "float32"))
    seq = np.concatenate([want["prompt"], want["tokens"]])[:32]
    ids = np.concatenate([seq, want["refine_active"]])
    bias = build_prefix_block_attention_bias(0, 64, block_size=32)
    with torch.no_grad():
        logits = hf(input_ids=torch.from_numpy(ids)[None], attention_mask={"full_attention": torch.from_numpy(bias)},
                    position_ids=torch.arange(64)[None]).logits.numpy()[0, 32:]
    np.testing.assert_allclose(want["refine_logits"], logits, rtol=0, atol=1e-5)
    # shifted confidence of those logits (runtime.py:176-181) in float64
    shifted = np.concatenate([logits[:1], logits[:-1]]).astype(np.float64)
    np.testing.assert_array_equal(want["refine_ids"], shifted.argmax(-1))
    e = np.exp(shifted - shifted.max(-1, keepdims=True))
    np.testing.assert_allclose(want["refine_maxp"], 1.0 / e.sum(-1), rtol=1e-5)


def test_hd128_oracle_reproduces_fixture():
    want = _load("hd128_bf16.npz")
    got = make_golden.hd128_fixture()
    assert set(got) == set(want)
    for k in want:
        if want[k].dtype.kind in "iu":
            np.testing.assert_array_equal(got[k], want[k], err_msg=k)
        else:
            np.testing.assert_allclose(got[k], want[k], rtol=0, atol=1e-6, err_msg=k)


@pytest.mark.gpu
def test_hd128_fixture_hip():
    from oracle import confidence as oconf

    g = _load("hd128_bf16.npz")
    _, vm = make_pair(make_golden.HD128, 5)
    ids, P, cap = g["ids"], int(g["P"]), int(g["cap"])
    dev = torch.tensor(ids, dtype=torch.int32, device="cuda")
    k = torch.zeros((2, 1, cap, 2, 128), dtype=torch.bfloat16, device="cuda")
    v = torch.zeros_like(k)
    log("case: golden hd128 prefix 64 + cached step R=32")
    vm.build_prefix_cache(vm.embed(dev[:P])[None], None, k, v)
    off = torch.tensor(P, dtype=torch.int32, device="cuda")
    h = vm.forward_cached(vm.embed(dev[P:])[None], k, v, off, P)
    bf16_parity("golden hidden", to_np(h)[0], g["hidden_bf16"], g["hidden_f32"])
    lg = to_np(vm.get_logits(h))[0]
    bf16_parity("golden logits", lg, g["logits_bf16"], g["logits_f32"])
    cid, cp = vm.get_confidence(h)
    wid, wp = oconf.confidence(lg)
    np.testing.assert_array_equal(cid.cpu().numpy()[0], wid)
    np.testing.assert_array_equal(cp.cpu().numpy()[0].view(np.uint32), wp.view(np.uint32))
    log("case: golden hd128 partial rp8")
    off8 = torch.tensor(P + 8, dtype=torch.int32, device="cuda")
    hp = vm.forward_block_partial_rp8(vm.embed(dev[P + 8:P + 16])[None], k, v, off8, P)
    bf16_parity("golden partial rp8", to_np(hp)[0], g["partial8_bf16"], g["partial8_f32"])
