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


# Artifact file names (export_cuda.py:9-11, 162-168; export_utils.py:22).
PARAMS_NPZ = "fast_dllm_relax_nn_params.npz"
PARAM_NAMES_TXT = "fast_dllm_relax_nn_param_names.txt"
DTYPE_TXT = "fast_dllm_relax_nn_dtype.txt"
KV_CACHE_MANIFEST = "fast_dllm_relax_nn_kv_cache.json"


def save_artifact(artifact_dir, cfg: FastDLLMConfig, params: list[torch.Tensor], dtype: str) -> pathlib.Path:
    """Write the weight files of a reference artifact: the packed params as positional npz arrays arr_i in
    param_names order (bf16 as its uint16 bits, export_utils.py:56-66), the names one per line, the
    dtype sidecar and the KV-cache manifest (export_cuda.py:162-168, export_utils.py:25-34).  The Relax
    executable itself (fast_dllm_relax_nn.so) is not written: this build's kernels replace it."""
    if dtype not in TORCH_DTYPES:
        raise ValueError(f"dtype {dtype!r} is not supported (bfloat16, float16)")
    names = param_names(cfg)
    if len(params) != len(names):
        raise ValueError(f"{len(params)} tensors for {len(names)} parameter names")
    d = pathlib.Path(artifact_dir)
    d.mkdir(parents=True, exist_ok=True)
    arrays = []
    for t in params:
        t = t.detach().to(TORCH_DTYPES[dtype]).contiguous().cpu()
        arrays.append(t.view(torch.int16).numpy().view(np.uint16) if dtype == "bfloat16" else t.numpy())
    np.savez(d / PARAMS_NPZ, *arrays)
    (d / PARAM_NAMES_TXT).write_text("\n".join(names) + "\n", encoding="utf-8")
    (d / DTYPE_TXT).write_text(dtype + "\n", encoding="utf-8")
    manifest = {"kv_cache": KV_CACHE_CONTRACT, "num_layers": cfg.num_hidden_layers,
                "num_kv_heads": cfg.num_key_value_heads, "head_dim": cfg.head_dim, "dtype": dtype}
    (d / KV_CACHE_MANIFEST).write_text(json.dumps(manifest, indent=2) + "\n", encoding="utf-8")
    return d


def _artifact_checks(d: pathlib.Path) -> dict:
    """The reference runner's checks at load (runners.py:597-603, 819-831): the weight files exist and
    the KV-cache manifest names the in-place contract."""
    missing = [p for p in (d / PARAMS_NPZ, d / PARAM_NAMES_TXT) if not p.exists()]
    if missing:
        formatted = "\n".join(f"- {p}" for p in missing)
        raise FileNotFoundError(f"Missing Relax artifact file(s):\n{formatted}")
    manifest_path = d / KV_CACHE_MANIFEST
    manifest = json.loads(manifest_path.read_text(encoding="utf-8")) if manifest_path.exists() else {}
    if manifest.get("kv_cache") != KV_CACHE_CONTRACT:
        raise RuntimeError(f"Relax artifact {d} does not use the in-place KV cache (no {KV_CACHE_MANIFEST} with "
                           f"kv_cache={KV_CACHE_CONTRACT!r}).")
    return manifest


def artifact_dtype(artifact_dir) -> str:
    """The artifact's semantic dtype; float16 when dtype.txt is absent (runners.py:947-949)."""
    path = pathlib.Path(artifact_dir) / DTYPE_TXT
    return path.read_text().strip() if path.exists() else "float16"


def config_from_artifact(artifact_dir, **overrides) -> FastDLLMConfig:
    """Model dimensions read from an artifact: layers, kv heads and head dim from the KV-cache manifest,
    the rest from the parameter shapes (embedding [V, H], gate_up [2I, H], qkv [(nq + 2 nkv) hd, H]) and
    whether lm_head.weight is listed.  rms_norm_eps, rope_theta and the block size are not stored in
    the weight files: the defaults (the 1.5B model's) apply unless given in ``overrides``."""
    d = pathlib.Path(artifact_dir)
    manifest = _artifact_checks(d)
    names = (d / PARAM_NAMES_TXT).read_text(encoding="utf-8").splitlines()
    index = {n: i for i, n in enumerate(names)}
    with np.load(d / PARAMS_NPZ, allow_pickle=False) as z:
        def shape(name):
            if name not in index:
                raise ValueError(f"artifact has no parameter {name}")
            return tuple(z[f"arr_{index[name]}"].shape)
        vocab, hidden = shape("model.embed_tokens.weight")
        inter = shape("model.layers.0.mlp.gate_up_proj.weight")[0] // 2
        qkv = shape("model.layers.0.self_attn.qkv_proj.weight")[0]
    nkv, hd = int(manifest["num_kv_heads"]), int(manifest["head_dim"])
    base = dict(vocab_size=vocab, hidden_size=hidden, intermediate_size=inter,
                num_hidden_layers=int(manifest["num_layers"]), num_attention_heads=qkv // hd - 2 * nkv,
                num_key_value_heads=nkv, head_dim=hd, tie_word_embeddings="lm_head.weight" not in index)
    base.update(overrides)
    return FastDLLMConfig(**base)


def load_artifact(artifact_dir, cfg: FastDLLMConfig | None = None, *,
                  device: str = "cuda") -> tuple[list[torch.Tensor], str]:
    """Load a reference artifact's weights (runners.py:938-968): the packed param list in param_names
    order on ``device`` and the artifact dtype.  With ``cfg`` the names and shapes are checked against it;
    without, the configuration is config_from_artifact's."""
    d = pathlib.Path(artifact_dir)
    _artifact_checks(d)
    dtype = artifact_dtype(d)
    if dtype not in TORCH_DTYPES:
        raise ValueError(f"artifact dtype {dtype!r} is not supported (bfloat16, float16)")
    if cfg is None:
        cfg = config_from_artifact(d)
    names = (d / PARAM_NAMES_TXT).read_text(encoding="utf-8").splitlines()
    if names != param_names(cfg):
        raise ValueError("artifact parameter names do not match the configuration's packed order")
    shapes = param_shapes(cfg)
    td = TORCH_DTYPES[dtype]
    out = []
    with np.load(d / PARAMS_NPZ, allow_pickle=False) as z:
        missing = [f"arr_{i}" for i in range(len(names)) if f"arr_{i}" not in z.files]
        if missing:  # runners.py:953-960
            suffix = "..." if len(missing) > 10 else ""
            raise ValueError(f"Parameter archive is missing expected arrays: {', '.join(missing[:10])}{suffix}")
        for i, name in enumerate(names):
            arr = z[f"arr_{i}"]
            if tuple(arr.shape) != shapes[name]:
                raise ValueError(f"{name}: shape {arr.shape} != {shapes[name]}")
            if dtype == "bfloat16":
                t = torch.from_numpy(np.ascontiguousarray(arr).view(np.int16).copy()).view(torch.bfloat16)
            else:
                t = torch.from_numpy(np.ascontiguousarray(arr).astype(np.float16))
            out.append(t.to(device=device, dtype=td))
    return out, dtype
