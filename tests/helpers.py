"""Shared test helpers: matched oracle / HIP models on the same seeded weights."""

from __future__ import annotations

import numpy as np

from oracle.model import OracleConfig, OracleModel, random_params

TINY = dict(vocab_size=1000, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
            num_attention_heads=4, num_key_value_heads=2, head_dim=128)
# the 1.5B shapes with two layers (the per-layer work is identical for all 28)
WIDE2 = dict(vocab_size=151936, hidden_size=1536, intermediate_size=8960, num_hidden_layers=2,
             num_attention_heads=12, num_key_value_heads=2, head_dim=128)


def make_pair(kw: dict, seed: int, dtype: str = "bfloat16", embed_std=None, max_rows: int = 64):
    import torch  # noqa: F401

    from fast_dllm_relax_amd.config import FastDLLMConfig
    from fast_dllm_relax_amd.params import from_numpy
    from fast_dllm_relax_amd.vm import HipVM

    arrays = random_params(OracleConfig(**kw), seed, dtype, embed_std=embed_std)
    ref = OracleModel(OracleConfig(**kw), arrays, dtype)
    cfg = FastDLLMConfig(**kw)
    vm = HipVM(cfg, from_numpy(arrays, cfg, dtype=dtype), dtype=dtype, max_rows=max_rows)
    return ref, vm


def to_np(t) -> np.ndarray:
    return t.float().cpu().numpy()


def log(msg: str) -> None:
    print(msg, flush=True)
