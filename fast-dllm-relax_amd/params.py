"""Packed parameter list: names, shapes, synthetic initialisation and the reference artifact format.

Order and fusion follow the reference: param_names.txt order (runners.py:947-972), fused qkv
[q; k; v] and gate_up [gate; up] (export_utils.py:76-115), tied lm_head = embed_tokens.weight.
Artifacts store bf16 as uint16 bits with a dtype.txt sidecar (export_utils.py:56-66,
export_cuda.py:162-168) and a KV-cache manifest (export_utils.py:25-34).
"""

from __future__ import annotations

import json
import pathlib

import numpy as np
import torch

from .config import KV_CACHE_CONTRACT, FastDLLMConfig

TORCH_DTYPES = {"bfloat16": torch.bfloat16, "float16": torch.float16}


def param_names(cfg: FastDLLMConfig) -> list[str]:
    names = ["model.embed_tokens.weight"]
    for i in range(cfg.num_hidden_layers):
        p = f"model.layers.{i}"
        names += [f"{p}.self_attn.qkv_proj.weight", f"{p}.self_attn.qkv_proj.bias", f"{p}.self_attn.o_proj.weight",
                  f"{p}.mlp.gate_up_proj.weight", f"{p}.mlp.down_proj.weight",
                  f"{p}.input_layernorm.weight", f"{p}.post_attention_layernorm.weight"]
    names.append("model.norm.weight")
    if not cfg.tie_word_embeddings:
        names.append("lm_head.weight")
    return names


def param_shapes(cfg: FastDLLMConfig) -> dict[str, tuple[int, ...]]:
    c = cfg
    shapes = {"model.embed_tokens.weight": (c.vocab_size, c.hidden_size), "model.norm.weight": (c.hidden_size,)}
    for i in range(c.num_hidden_layers):
        p = f"model.layers.{i}"
        shapes[f"{p}.self_attn.qkv_proj.weight"] = (c.qkv_dim, c.hidden_size)
        shapes[f"{p}.self_attn.qkv_proj.bias"] = (c.qkv_dim,)
        shapes[f"{p}.self_attn.o_proj.weight"] = (c.hidden_size, c.num_attention_heads * c.head_dim)
        shapes[f"{p}.mlp.gate_up_proj.weight"] = (2 * c.intermediate_size, c.hidden_size)
        shapes[f"{p}.mlp.down_proj.weight"] = (c.hidden_size, c.intermediate_size)
        shapes[f"{p}.input_layernorm.weight"] = (c.hidden_size,)
        shapes[f"{p}.post_attention_layernorm.weight"] = (c.hidden_size,)
    if not c.tie_word_embeddings:
        shapes["lm_head.weight"] = (c.vocab_size, c.hidden_size)
    return shapes


def random_params_torch(cfg: FastDLLMConfig, seed: int, *, dtype: str = "bfloat16", device: str = "cuda",
                        std: float = 0.02, embed_std: float | None = None,
                        lm_head_std: float | None = None) -> list[torch.Tensor]:
    """Synthetic weights N(0, std) (norm weights = 1, the reference's test convention,
    tests/test_tiny_compile.py:45-55) generated on ``device`` from ``seed``; ``embed_std`` scales the
    embedding (the lm_head too when tied) and ``lm_head_std`` an untied lm_head separately."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    td = TORCH_DTYPES[dtype]
    out = []
    shapes = param_shapes(cfg)
    for name in param_names(cfg):
        shape = shapes[name]
        if name.endswith("norm.weight"):
            out.append(torch.ones(shape, dtype=td, device=device))
            continue
        s = std
        if embed_std is not None and name == "model.embed_tokens.weight":
            s = embed_std
        elif lm_head_std is not None and name == "lm_head.weight":
            s = lm_head_std
        t = torch.empty(shape, dtype=torch.float32, device=device)
        t.normal_(0.0, 1.0, generator=gen)
        out.append((t * s).to(td))
        del t
    return out


def from_numpy(arrays: dict[str, np.ndarray], cfg: FastDLLMConfig, *, dtype: str = "bfloat16",
               device: str = "cuda") -> list[torch.Tensor]:
    """Packed device list from name -> fp32 arrays (values already representable in ``dtype``)."""
    td = TORCH_DTYPES[dtype]
    return [torch.from_numpy(np.ascontiguousarray(arrays[n], dtype=np.float32)).to(device=device, dtype=td)
            for n in param_names(cfg)]


def load_artifact(artifact_dir, cfg: FastDLLMConfig, *, device: str = "cuda") -> tuple[list[torch.Tensor], str]:
    """Load a reference artifact directory: fast_dllm_relax_nn_params.npz, _param_names.txt, _dtype.txt
    and the KV-cache manifest (export_cuda.py:143-168).  Returns (packed params, dtype)."""
    d = pathlib.Path(artifact_dir)
    dtype = (d / "fast_dllm_relax_nn_dtype.txt").read_text().strip()
    if dtype not in TORCH_DTYPES:
        raise ValueError(f"artifact dtype {dtype!r} is not supported (bfloat16, float16)")
    manifest = d / "fast_dllm_relax_nn_kv_cache.json"
    if manifest.exists():
        info = json.loads(manifest.read_text())
        if info.get("kv_cache") != KV_CACHE_CONTRACT:
            raise ValueError(f"artifact KV-cache contract {info.get('kv_cache')!r} != {KV_CACHE_CONTRACT!r}")
    names = (d / "fast_dllm_relax_nn_param_names.txt").read_text().split()
    if names != param_names(cfg):
        raise ValueError("artifact parameter names do not match the configuration's packed order")
    shapes = param_shapes(cfg)
    td = TORCH_DTYPES[dtype]
    out = []
    with np.load(d / "fast_dllm_relax_nn_params.npz", allow_pickle=False) as z:
        missing = [f"arr_{i}" for i in range(len(names)) if f"arr_{i}" not in z.files]
        if missing:  # runners.py:953-963
            raise ValueError(f"Parameter archive is missing expected arrays: {', '.join(missing[:10])}")
        for i, name in enumerate(names):
            arr = z[f"arr_{i}"]
            if tuple(arr.shape) != shapes[name]:
                raise ValueError(f"{name}: shape {arr.shape} != {shapes[name]}")
            if dtype == "bfloat16":
                t = torch.from_numpy(arr.view(np.int16).copy()).view(torch.bfloat16)
            else:
                t = torch.from_numpy(arr.astype(np.float16))
            out.append(t.to(device=device, dtype=td))
    return out, dtype
