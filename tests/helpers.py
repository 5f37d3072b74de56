"""Shared test helpers: matched oracle / HIP models on the same seeded weights."""

from __future__ import annotations

import numpy as np

from oracle.model import OracleConfig, OracleModel, random_params

TINY = dict(vocab_size=1000, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
            num_attention_heads=4, num_key_value_heads=2, head_dim=128)
# the 1.5B shapes with two layers (the per-layer work is identical for all 28)
WIDE2 = dict(vocab_size=151936, hidden_size=1536, intermediate_size=8960, num_hidden_layers=2,
             num_attention_heads=12, num_key_value_heads=2, head_dim=128)


def make_pair(kw: dict, seed: int, dtype: str = "bfloat16", embed_std=None, max_rows: int = 64, lm_head_std=None):
    import torch  # noqa: F401

    from fast_dllm_relax_amd.config import FastDLLMConfig
    from fast_dllm_relax_amd.params import from_numpy
    from fast_dllm_relax_amd.vm import HipVM

    arrays = random_params(OracleConfig(**kw), seed, dtype, embed_std=embed_std, lm_head_std=lm_head_std)
    ref = OracleModel(OracleConfig(**kw), arrays, dtype)
    cfg = FastDLLMConfig(**kw)
    vm = HipVM(cfg, from_numpy(arrays, cfg, dtype=dtype), dtype=dtype, max_rows=max_rows)
    return ref, vm



def to_np(t) -> np.ndarray:
    return t.float().cpu().numpy()


def log(msg: str) -> None:
    print(msg, flush=True)


def bf16_parity(name: str, got: np.ndarray, want_bf16: np.ndarray, want_f32: np.ndarray | None = None, *,
                rtol: float = 2e-2, atol: float = 2e-2, max_outside: float = 5e-3, max_abs: float = 0.1,
                factor: float = 1.5) -> dict:
    """Parity of a bf16 result with the oracle.

    ``want_bf16`` is the oracle with the reference's bf16 rounding points; accumulation orders differ,
    so a bf16 rounding can flip by one ulp and propagate: at most ``max_outside`` of the elements may
    fall outside rtol/atol (2e-2, the reference's own tolerance, tests/test_tiny_compile.py:282) and
    none by more than ``max_abs``.  With ``want_f32`` (the oracle without rounding on the same weights),
    the HIP error against fp32 must stay within ``factor`` x the bf16 oracle's own error against fp32:
    the HIP path is as accurate as the reference's precision order."""
    got = np.asarray(got, np.float32)
    d = np.abs(got - want_bf16)
    outside = float(np.mean(d > atol + rtol * np.abs(want_bf16)))
    stats = {"max_abs": float(d.max()), "mean_abs": float(d.mean()), "outside": outside}
    if want_f32 is not None:
        e_hip = np.abs(got - want_f32)
        e_ora = np.abs(want_bf16 - want_f32)
        stats.update(hip_vs_f32_max=float(e_hip.max()), oracle_vs_f32_max=float(e_ora.max()),
                     hip_vs_f32_mean=float(e_hip.mean()), oracle_vs_f32_mean=float(e_ora.mean()))
    log(f"  {name}: " + ", ".join(f"{k}={v:.4g}" for k, v in stats.items()))
    assert outside <= max_outside, (name, stats)
    assert stats["max_abs"] <= max_abs, (name, stats)
    if want_f32 is not None:
        assert stats["hip_vs_f32_mean"] <= factor * stats["oracle_vs_f32_mean"] + 1e-6, (name, stats)
        assert stats["hip_vs_f32_max"] <= factor * stats["oracle_vs_f32_max"] + 1e-6, (name, stats)
    return stats
