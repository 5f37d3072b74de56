"""fdllm_attn_inplace and fdllm_kv_write, the reference's attention callbacks fast_dllm.attn_inplace and
fast_dllm.kv_write (fast_dllm_relax/runtime.py:19-80), against the oracle's restatement
(OracleModel.attn_inplace / kv_write), through the C ABI.  Every case names the kernel family its row
count takes: the chunk kernel (up to 32 rows), the loop kernel (33 to 127) and the prefill kernel (128
rows and more, queries staged in the output buffer)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import TINY, log, make_pair, to_np

pytestmark = pytest.mark.gpu

# the 1.5B attention shapes (12 query heads on 2 kv heads, head_dim 128) with small projections
HEADS12 = dict(vocab_size=1000, hidden_size=1536, intermediate_size=512, num_hidden_layers=2,
               num_attention_heads=12, num_key_value_heads=2, head_dim=128)
TDT = {"bfloat16": torch.bfloat16, "float16": torch.float16}


@pytest.fixture(scope="module")
def heads12():
    log("setup: 12/2-head bf16 model seed 21")
    return make_pair(HEADS12, 21)


def _inputs(ref, rows, cap, seed):
    c = ref.cfg
    rng = np.random.default_rng(seed)
    q = ref.rnd(rng.standard_normal((1, rows, c.num_attention_heads, c.head_dim)).astype(np.float32))
    k = ref.rnd(rng.standard_normal((1, rows, c.num_key_value_heads, c.head_dim)).astype(np.float32))
    v = ref.rnd(rng.standard_normal((1, rows, c.num_key_value_heads, c.head_dim)).astype(np.float32))
    shape = (c.num_hidden_layers, 1, cap, c.num_key_value_heads, c.head_dim)
    kc = ref.rnd(rng.standard_normal(shape).astype(np.float32))
    vc = ref.rnd(rng.standard_normal(shape).astype(np.float32))
    return q, k, v, kc, vc


def _dev(a, tdt):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda", tdt)


def _case(ref, vm, rows, P, write_rel, attend_rel, cap, seed, layer):
    tdt = TDT[vm.dtype]
    log(f"case: attn_inplace rows={rows} prefix={P} write_rel={write_rel} attend_rel={attend_rel} cap={cap} "
        f"layer={layer} {vm.dtype}")
    q, k, v, kc, vc = _inputs(ref, rows, cap, seed)
    dq, dk, dv, dkc, dvc = (_dev(a, tdt) for a in (q, k, v, kc, vc))
    kc_out, vc_out, got = vm.attn_inplace(dq, dk, dv, dkc, dvc, layer, P, write_rel, attend_rel)
    assert kc_out is dkc and vc_out is dvc
    _, _, want = ref.attn_inplace(q, k, v, kc, vc, layer, P, write_rel, attend_rel)
    # the caches: the written rows byte for byte, every other row untouched
    np.testing.assert_array_equal(to_np(dkc), kc)
    np.testing.assert_array_equal(to_np(dvc), vc)
    got = to_np(got)
    assert got.shape == want.shape
    # the reference's tolerance (tests/test_tiny_compile.py:282); then a tighter bound: the kernels round
    # the probabilities to the model dtype for the P.V product (as flash attention does) and sum in
    # another order than the oracle's fp32 softmax, so an output may sit a few units in the last place
    # of the largest output away, no more
    np.testing.assert_allclose(got, want, rtol=2e-2, atol=2e-2)
    d = np.abs(got - want)
    big = float(np.abs(want).max())
    ulp = 2.0 ** (np.floor(np.log2(big)) - (7 if vm.dtype == "bfloat16" else 10))
    log(f"  identical elements {float(np.mean(d == 0)):.4f}, max |d| {float(d.max()):.3g} = "
        f"{float(d.max()) / ulp:.2f} ulp of the largest output, mean |d| {float(d.mean()):.3g}")
    assert d.max() <= 4 * ulp


@pytest.mark.parametrize("rows,P,write_rel,attend_rel,cap", [
    (32, 96, 0, 32, 160),      # the full block step's call: chunk kernel
    (8, 96, 8, 32, 160),       # a partial step (rp 8): chunk kernel
    (32, 2016, 0, 32, 2080),   # the config-3 prefix: chunk kernel, 16 key chunks + merge
    (64, 40, 0, 64, 128),      # a scoring tail: loop kernel
    (160, 32, 0, 160, 192),    # prefill kernel with the queries staged in out
    (32, 64, 0, 80, 128),      # attended rows past the capacity: the reference's slice stops at cap
    (20, 50, 3, 30, 96),       # unaligned window and row count
])
def test_attn_inplace_matches_oracle(heads12, rows, P, write_rel, attend_rel, cap):
    ref, vm = heads12
    _case(ref, vm, rows, P, write_rel, attend_rel, cap, seed=rows + P, layer=1)


def test_attn_inplace_other_grouping_and_fp16():
    ref, vm = make_pair(TINY, 22)  # 4 query heads on 2 kv heads
    _case(ref, vm, 32, 64, 0, 32, 96, seed=1, layer=0)
    _case(ref, vm, 8, 64, 24, 32, 96, seed=2, layer=1)
    ref, vm = make_pair(HEADS12, 23, dtype="float16")
    _case(ref, vm, 32, 200, 0, 32, 256, seed=3, layer=0)
    _case(ref, vm, 96, 100, 0, 96, 224, seed=4, layer=1)


def test_kv_write_byte_exact_and_errors(heads12):
    ref, vm = heads12
    c = ref.cfg
    log("case: kv_write 13 rows at 50, special values")
    q, k, v, kc, vc = _inputs(ref, 13, 80, 7)
    k[0, 0, 0, :4] = [-0.0, np.inf, -np.inf, np.nan]
    dk, dv, dkc, dvc = (_dev(a, torch.bfloat16) for a in (k, v, kc, vc))
    bits_k = dk.view(torch.int16).clone()
    vm.kv_write(dk, dv, dkc, dvc, 1, 50)
    want_k = dkc.clone()
    assert torch.equal(dkc[1, 0, 50:63].reshape(13, -1).view(torch.int16), bits_k[0].reshape(13, -1))
    ref.kv_write(k, v, kc, vc, 1, 50)
    np.testing.assert_array_equal(to_np(dvc), vc)
    np.testing.assert_array_equal(np.isnan(to_np(dkc)), np.isnan(kc))
    log("case: kv_write from rows that are not 16-byte aligned (the two-copy path)")
    flat = torch.zeros(13 * 2 * 128 + 8, dtype=torch.bfloat16, device="cuda")
    ku = flat[1:1 + 13 * 2 * 128].view(1, 13, 2, 128)
    ku.copy_(dk)
    assert ku.data_ptr() % 16 != 0
    vm.kv_write(ku, dv, dkc, dvc, 0, 20)
    assert torch.equal(dkc[0, 0, 20:33].reshape(13, -1).view(torch.int16), bits_k[0].reshape(13, -1))
    assert torch.equal(dvc[0, 0, 20:33], dv[0])
    want_k = dkc.clone()
    log("case: window errors")
    with pytest.raises(ValueError, match=r"KV write \[70, 83\) outside cache capacity 80"):
        vm.kv_write(dk, dv, dkc, dvc, 0, 70)
    with pytest.raises(ValueError, match=r"KV write \[-1, 12\) outside cache capacity 80"):
        vm.kv_write(dk, dv, dkc, dvc, 0, -1)
    with pytest.raises(ValueError, match="layer 2 outside"):
        vm.kv_write(dk, dv, dkc, dvc, 2, 0)
    dq = _dev(q, torch.bfloat16)
    with pytest.raises(ValueError, match=r"KV write \[40, 53\) past the attended rows \[0, 50\)"):
        vm.attn_inplace(dq, dk, dv, dkc, dvc, 0, 32, 8, 18)
    with pytest.raises(ValueError, match=r"KV write \[72, 85\) outside cache capacity 80"):
        vm.attn_inplace(dq, dk, dv, dkc, dvc, 0, 64, 8, 30)
    torch.cuda.synchronize()
    assert torch.equal(dkc.view(torch.int16), want_k.view(torch.int16)), "a refused call wrote the cache"
    assert c.num_key_value_heads == 2
