"""bench.py's CPU baseline computes the step it claims to time (CPU only): the HF reference forward
(transformers' Qwen2 built from the packed weights, a cached 32-row step against a DynamicCache prefix)
gives the oracle's logits on a small head_dim-128 model, in fp32, with an untied head and a tied one."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import bench
from oracle.model import OracleConfig, OracleModel, build_prefix_block_attention_bias, random_params

KW = dict(vocab_size=1000, hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
          num_key_value_heads=2, head_dim=128)


@pytest.mark.parametrize("tied", [False, True])
def test_hf_cached_step_matches_oracle(tied):
    from fast_dllm_relax_amd.config import FastDLLMConfig
    from fast_dllm_relax_amd.params import param_names

    kw = dict(KW, tie_word_embeddings=tied)
    ocfg, cfg = OracleConfig(**kw), FastDLLMConfig(**kw)
    arrays = random_params(ocfg, 3, "float32", lm_head_std=None if tied else 0.5)
    ref = OracleModel(ocfg, arrays, "float32")
    P = 64
    ids = np.random.default_rng(4).integers(0, 999, P + 32)
    kc = np.zeros((2, 1, P + 32, 2, 128), np.float32)
    vc = np.zeros_like(kc)
    ref.build_prefix_cache(ref.embed(ids[:P])[None], build_prefix_block_attention_bias(0, P, block_size=32), kc, vc)
    want = ref.get_logits(ref.forward_cached(ref.embed(ids[P:])[None], kc, vc, P, P))[0]
    params = [torch.from_numpy(np.ascontiguousarray(arrays[n])) for n in param_names(cfg)]
    model = bench.hf_reference_model(cfg, params, torch.float32)
    got, sec = bench.hf_cached_step(model, torch.from_numpy(kc[:, :, :P]), torch.from_numpy(vc[:, :, :P]),
                                    [int(t) for t in ids[P:]], P)
    assert sec > 0
    np.testing.assert_allclose(got.numpy(), want, rtol=0, atol=4e-6 * float(np.abs(want).max()) + 1e-5)
