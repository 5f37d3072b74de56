"""The allocation-free cached step (fdllm_forward_cached_noalloc, include/fdllm.h) against
fdllm_forward_cached: the same hidden states and cache rows, bit for bit, on calls in a row, each
smaller than the one before (the first at the documented limit of 8192 attended keys), called through
the C ABI.  Marked gpu."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import WIDE2, log, make_pair

pytestmark = pytest.mark.gpu


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _step_both(vm, lib, _lib, prompt, block, cap):
    from fast_dllm_relax_amd.runtime import _embed, _offset_tensor, build_prefix_cache_from_ids

    P = len(prompt)
    ca = build_prefix_cache_from_ids(vm, prompt, block_size=32, capacity=cap)
    cb = build_prefix_cache_from_ids(vm, prompt, block_size=32, capacity=cap)
    emb = _embed(vm, block)
    off = _offset_tensor(P)
    want = vm.forward_cached(emb, ca.k, ca.v, off, P)
    got = torch.empty_like(want)
    _lib.check(lib.fdllm_forward_cached_noalloc(vm.ctx, emb.data_ptr(), len(block), cb.k.data_ptr(), cb.v.data_ptr(),
                                                int(cb.k.shape[2]), off.data_ptr(), P, got.data_ptr(), _stream()))
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    assert torch.equal(cb.k[:, :, :P + len(block)].view(torch.int16), ca.k[:, :, :P + len(block)].view(torch.int16))
    assert torch.equal(cb.v[:, :, :P + len(block)].view(torch.int16), ca.v[:, :, :P + len(block)].view(torch.int16))


def test_noalloc_step_equals_forward_cached():
    from fast_dllm_relax_amd import _lib

    ref, vm = make_pair(WIDE2, 7, "bfloat16", max_rows=2048)
    lib = vm.lib
    rng = np.random.default_rng(7)
    long_prompt = [int(t) for t in rng.integers(0, 150000, 8160)]
    log("case: noalloc 32 rows at prefix 8160 (8192 keys, the documented limit: 64 key chunks of partials)")
    _step_both(vm, lib, _lib, long_prompt, [int(t) for t in rng.integers(0, 150000, 32)], 8192)
    prompt = [int(t) for t in rng.integers(0, 150000, 2016)]
    log("case: noalloc 32 rows at prefix 2016 (a smaller call after it)")
    _step_both(vm, lib, _lib, prompt, [int(t) for t in rng.integers(0, 150000, 32)], 2048)
    log("case: noalloc 8 rows at prefix 480 (a smaller second call)")
    _step_both(vm, lib, _lib, prompt[:480], [int(t) for t in rng.integers(0, 150000, 8)], 512)
    # beyond the maximum: a clear error, nothing launched
    emb = torch.zeros((1, 33, WIDE2["hidden_size"]), dtype=torch.bfloat16, device="cuda")
    k = torch.zeros((2, 1, 64, 2, 128), dtype=torch.bfloat16, device="cuda")
    off = torch.zeros((), dtype=torch.int32, device="cuda")
    with pytest.raises(ValueError, match="allocation-free"):
        _lib.check(lib.fdllm_forward_cached_noalloc(vm.ctx, emb.data_ptr(), 33, k.data_ptr(), k.data_ptr(), 64,
                                                    off.data_ptr(), 0, emb.data_ptr(), _stream()))
    vm.close()
