"""Reference artifact weight files (export_cuda.py:162-168, export_utils.py:25-34, 56-66) written and read
back; the reference runner's load-time checks (runners.py:597-603, 819-831, 947-963).  CPU only."""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from helpers import TINY
from fast_dllm_relax_amd import params as P
from fast_dllm_relax_amd.config import FastDLLMConfig


def _cfg(tied=True):
    return FastDLLMConfig(**TINY, tie_word_embeddings=tied)


@pytest.mark.parametrize("dtype,tied", [("bfloat16", True), ("float16", True), ("bfloat16", False)])
def test_round_trip_is_bit_exact(tmp_path, dtype, tied):
    cfg = _cfg(tied)
    params = P.random_params_torch(cfg, 3, dtype=dtype, device="cpu")
    P.save_artifact(tmp_path, cfg, params, dtype)
    assert P.config_from_artifact(tmp_path) == cfg
    loaded, got_dtype = P.load_artifact(tmp_path, device="cpu")
    assert got_dtype == dtype
    assert len(loaded) == len(params)
    for a, b in zip(loaded, params):
        assert a.dtype == b.dtype and a.shape == b.shape
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_file_format_matches_the_exporter(tmp_path):
    cfg = _cfg()
    params = P.random_params_torch(cfg, 4, dtype="bfloat16", device="cpu")
    P.save_artifact(tmp_path, cfg, params, "bfloat16")
    names = P.param_names(cfg)
    with np.load(tmp_path / "fast_dllm_relax_nn_params.npz", allow_pickle=False) as z:
        assert sorted(z.files) == sorted(f"arr_{i}" for i in range(len(names)))
        for i, (n, t) in enumerate(zip(names, params)):
            a = z[f"arr_{i}"]
            assert a.dtype == np.uint16  # bf16 bits (export_utils.py:56-66)
            assert tuple(a.shape) == tuple(t.shape)
            # the bits are the bf16 value's upper 16 float32 bits
            f32 = t.float().numpy().view(np.uint32)
            assert np.array_equal(a, (f32 >> 16).astype(np.uint16))
    assert (tmp_path / "fast_dllm_relax_nn_param_names.txt").read_text() == "\n".join(names) + "\n"
    assert (tmp_path / "fast_dllm_relax_nn_dtype.txt").read_text() == "bfloat16\n"
    manifest = json.loads((tmp_path / "fast_dllm_relax_nn_kv_cache.json").read_text())
    assert manifest == {"kv_cache": "inplace_bsnh_v1", "num_layers": cfg.num_hidden_layers,
                        "num_kv_heads": cfg.num_key_value_heads, "head_dim": cfg.head_dim, "dtype": "bfloat16"}


def test_loader_errors_follow_the_runner(tmp_path):
    cfg = _cfg()
    params = P.random_params_torch(cfg, 5, dtype="bfloat16", device="cpu")
    P.save_artifact(tmp_path, cfg, params, "bfloat16")
    man = tmp_path / "fast_dllm_relax_nn_kv_cache.json"
    good = man.read_text()
    man.write_text(json.dumps({"kv_cache": "stacked_bhsd"}))
    with pytest.raises(RuntimeError, match="in-place KV cache"):
        P.load_artifact(tmp_path, cfg, device="cpu")
    man.unlink()
    with pytest.raises(RuntimeError, match="in-place KV cache"):
        P.load_artifact(tmp_path, cfg, device="cpu")
    man.write_text(good)
    # no dtype sidecar: the runner assumes float16 (runners.py:947-949), and these bf16 bits then load
    # as float16 values
    (tmp_path / "fast_dllm_relax_nn_dtype.txt").unlink()
    assert P.artifact_dtype(tmp_path) == "float16"
    loaded, dtype = P.load_artifact(tmp_path, cfg, device="cpu")
    assert dtype == "float16" and loaded[0].dtype == torch.float16
    # an archive short of arrays
    names = P.param_names(cfg)
    with np.load(tmp_path / "fast_dllm_relax_nn_params.npz") as z:
        kept = [z[f"arr_{i}"] for i in range(len(names) - 1)]
    np.savez(tmp_path / "fast_dllm_relax_nn_params.npz", *kept)
    with pytest.raises(ValueError, match="missing expected arrays"):
        P.load_artifact(tmp_path, cfg, device="cpu")
    (tmp_path / "fast_dllm_relax_nn_params.npz").unlink()
    with pytest.raises(FileNotFoundError, match="Missing Relax artifact"):
        P.load_artifact(tmp_path, cfg, device="cpu")


def test_names_must_match_the_configuration(tmp_path):
    cfg = _cfg()
    P.save_artifact(tmp_path, cfg, P.random_params_torch(cfg, 6, dtype="bfloat16", device="cpu"), "bfloat16")
    other = FastDLLMConfig(**{**TINY, "num_hidden_layers": 3})
    with pytest.raises(ValueError, match="names do not match"):
        P.load_artifact(tmp_path, other, device="cpu")
