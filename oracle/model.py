"""numpy restatement of the reference model's nine entry points.  TEST INFRASTRUCTURE ONLY.

Follows ``fast_dllm_relax/model/cuda.py`` of the reference:

* embed                                  cuda.py:698-699
* FastDLLMRMSNorm.forward                cuda.py:257-275  (fp32 normalize -> cast -> x weight in model dtype)
* fused qkv projection + bias            cuda.py:389-399  (one rounding of acc + bias, cuBLAS bias epilogue)
* RoPE tables with offset / apply        cuda.py:278-316, _rotate_half 207-209
* cached attention (attn_inplace)        runtime.py:51-73, in-graph restatement metal.py:378-439
  (fp32 scores, fp32 softmax, fp32 P.V, one cast at the end; no mask; GQA head h -> kv head h // group)
* dense attention with additive bias     cuda.py:401-466 (forward / forward_and_collect_kv)
* MLP with _silu_fp32                    cuda.py:319-348
* decoder layer / model loops            cuda.py:545-666
* get_logits (tied)                      cuda.py:704-711  (model-dtype GEMM -> rounded -> fp32)
* build_prefix_block_attention_bias      cuda.py:148-177
* extract_shifted_block_logits           cuda.py:180-204

``dtype`` selects the rounding emulation: ``"bfloat16"`` / ``"float16"`` round every tensor the
reference materialises in the model dtype (round-to-nearest-even, as torch / cuBLAS / TVM casts do);
``"float32"`` rounds nothing (the fp32 reference the logit tolerance is quoted against).

Pinned by tests/test_oracle_pinning.py against: the local ``transformers`` Qwen2 implementation
(an independent restatement of the same architecture) in fp32, torch's scaled_dot_product_attention,
closed forms (RoPE at position 0 is the identity and preserves norms; RMSNorm output has unit RMS),
and the reference's own invariants (cached rows == dense block-causal rows; partial rows == full rows).
"""

from __future__ import annotations

import dataclasses
import math

import numpy as np

F32 = np.float32


@dataclasses.dataclass(frozen=True)
class OracleConfig:
    """Model constants (mirror of FastDLLMRelaxConfig, cuda.py:15-29)."""

    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6
    tie_word_embeddings: bool = True
    bd_size: int = 32


def bf16_round(x: np.ndarray) -> np.ndarray:
    """fp32 -> nearest-even bfloat16 -> fp32 (what ``tensor.to(torch.bfloat16)`` does)."""
    x = np.ascontiguousarray(x, dtype=F32)
    u = x.view(np.uint32)
    out = u + (((u >> 16) & np.uint32(1)) + np.uint32(0x7FFF))  # wraps only for NaN, fixed below
    out &= np.uint32(0xFFFF0000)
    nan = np.isnan(x)
    if nan.any():
        out[nan] = 0x7FC00000
    return out.view(F32)


def f16_round(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=F32).astype(np.float16).astype(F32)


def rounder(dtype: str):
    if dtype == "bfloat16":
        return bf16_round
    if dtype == "float16":
        return f16_round
    if dtype == "float32":
        return lambda x: np.asarray(x, dtype=F32)
    raise ValueError(f"unsupported dtype {dtype!r}")


def build_prefix_block_attention_bias(prefix_len: int, block_len: int, *, block_size: int | None = None,
                                      blocked_value: float = -1e9) -> np.ndarray:
    """Block-causal additive bias [1,1,T,T]: allowed iff q//bs >= k//bs (cuda.py:148-177)."""
    if prefix_len < 0:
        raise ValueError("prefix_len must be non-negative")
    if block_len <= 0:
        raise ValueError("block_len must be positive")
    total = prefix_len + block_len
    bs = block_len if block_size is None else int(block_size)
    if bs <= 0:
        raise ValueError("block_size must be positive when provided")
    pos = np.arange(total, dtype=np.int32)
    allowed = (pos[:, None] // bs) >= (pos[None, :] // bs)
    return np.where(allowed, 0.0, blocked_value).astype(F32)[None, None]


def extract_shifted_block_logits(logits: np.ndarray, *, prefix_len: int, block_len: int) -> np.ndarray:
    """Position i is predicted from logits at i-1 (cuda.py:180-204)."""
    if logits.ndim != 3:
        raise ValueError(f"Expected logits to have rank 3, got shape {logits.shape}")
    if block_len <= 0:
        raise ValueError("block_len must be positive")
    if prefix_len + block_len > logits.shape[1]:
        raise ValueError(f"Requested prefix_len={prefix_len} and block_len={block_len} "
                         f"for logits of length {logits.shape[1]}")
    if prefix_len > 0:
        src = [prefix_len - 1] + list(range(prefix_len, prefix_len + block_len - 1))
    else:
        src = [0] + list(range(0, block_len - 1))
    return logits[:, src, :]


def param_names(cfg: OracleConfig) -> list[str]:
    """Packed parameter order of the reference artifact (02_relax_frontend_model.ipynb cell 9)."""
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


class OracleModel:
    """The reference's entry points on numpy arrays.

    ``params``: name -> fp32 array holding values representable in ``dtype`` (the caller rounds them).
    Activations are ``[1, S, H]`` fp32 arrays; caches are ``[L, 1, cap, nkv, hd]`` fp32 arrays,
    mutated in place exactly where the reference writes them.
    """

    def __init__(self, cfg: OracleConfig, params: dict[str, np.ndarray], dtype: str = "bfloat16"):
        self.cfg = cfg
        self.dtype = dtype
        self.rnd = rounder(dtype)
        self.p = {k: np.asarray(v, dtype=F32) for k, v in params.items()}
        self.scale = F32(cfg.head_dim ** -0.5)  # cuda.py:362

    # ---- building blocks -------------------------------------------------------------------
    def rmsnorm(self, x: np.ndarray, w: np.ndarray) -> np.ndarray:
        """cuda.py:269-275."""
        xf = x.astype(F32)
        var = np.mean(np.square(xf), axis=-1, keepdims=True, dtype=F32)
        y = xf * (F32(1.0) / np.sqrt(var + F32(self.cfg.rms_norm_eps)))
        return self.rnd(w * self.rnd(y))

    def linear(self, x: np.ndarray, w: np.ndarray, b: np.ndarray | None = None) -> np.ndarray:
        acc = np.matmul(x.astype(F32), w.T.astype(F32))
        if b is not None:
            acc = acc + b
        return self.rnd(acc)

    def rope_tables(self, n: int, offset: int) -> tuple[np.ndarray, np.ndarray]:
        """cuda.py:288-299: inv_freq = exp(-ln(theta) * i / half); pos = r + offset; emb = [f, f]."""
        hd = self.cfg.head_dim
        half = hd // 2
        exponent = F32(-math.log(self.cfg.rope_theta)) * np.arange(half, dtype=F32)
        exponent = (exponent / F32(half)).astype(F32)
        inv_freq = np.exp(exponent).astype(F32)
        pos = np.arange(n, dtype=F32) + F32(offset)
        freqs = (pos[:, None] * inv_freq[None, :]).astype(F32)
        emb = np.concatenate([freqs, freqs], axis=-1)
        return self.rnd(np.cos(emb)), self.rnd(np.sin(emb))

    def apply_rope(self, x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
        """x [n, heads, hd]; cos/sin [n, hd] (cuda.py:314-315, _rotate_half 207-209)."""
        half = x.shape[-1] // 2
        rot = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
        c, s = cos[:, None, :], sin[:, None, :]
        return self.rnd(self.rnd(x * c) + self.rnd(rot * s))

    def attend(self, q: np.ndarray, k: np.ndarray, v: np.ndarray, bias: np.ndarray | None = None) -> np.ndarray:
        """q [n, nq, hd]; k/v [m, nkv, hd]; bias [n, m] or None.  fp32 throughout, one cast at the end."""
        nq, nkv = self.cfg.num_attention_heads, self.cfg.num_key_value_heads
        grp = nq // nkv
        out = np.empty(q.shape, dtype=F32)
        for h in range(nq):
            g = h // grp
            s = np.matmul(q[:, h, :], k[:, g, :].T).astype(F32) * self.scale
            if bias is not None:
                s = s + bias
            s = s - s.max(axis=-1, keepdims=True)
            e = np.exp(s)
            pr = e / e.sum(axis=-1, keepdims=True, dtype=F32)
            out[:, h, :] = np.matmul(pr, v[:, g, :])
        return self.rnd(out)

    def _qkv(self, i: int, xn: np.ndarray, offset: int):
        c = self.cfg
        n = xn.shape[0]
        pre = f"model.layers.{i}.self_attn"
        qkv = self.linear(xn, self.p[f"{pre}.qkv_proj.weight"], self.p[f"{pre}.qkv_proj.bias"])
        qd, kd = c.num_attention_heads * c.head_dim, c.num_key_value_heads * c.head_dim
        q = qkv[:, :qd].reshape(n, c.num_attention_heads, c.head_dim)
        k = qkv[:, qd:qd + kd].reshape(n, c.num_key_value_heads, c.head_dim)
        v = qkv[:, qd + kd:].reshape(n, c.num_key_value_heads, c.head_dim)
        cos, sin = self.rope_tables(n, offset)
        return self.apply_rope(q, cos, sin), self.apply_rope(k, cos, sin), v

    def _mlp(self, i: int, x: np.ndarray) -> np.ndarray:
        pre = f"model.layers.{i}.mlp"
        gu = self.linear(x, self.p[f"{pre}.gate_up_proj.weight"])
        inter = self.cfg.intermediate_size
        g, u = gu[:, :inter], gu[:, inter:]
        silu = self.rnd(g * (F32(1.0) / (F32(1.0) + np.exp(-g))))  # _silu_fp32, cuda.py:319-328
        return self.linear(self.rnd(silu * u), self.p[f"{pre}.down_proj.weight"])

    def _layer_tail(self, i: int, h: np.ndarray, attn: np.ndarray) -> np.ndarray:
        pre = f"model.layers.{i}"
        n = h.shape[0]
        o = self.linear(attn.reshape(n, -1), self.p[f"{pre}.self_attn.o_proj.weight"])
        h = self.rnd(h + o)
        m = self._mlp(i, self.rmsnorm(h, self.p[f"{pre}.post_attention_layernorm.weight"]))
        return self.rnd(h + m)

    # ---- entry points (cuda.py:698-788) ------------------------------------------------------
    def embed(self, ids) -> np.ndarray:
        ids = np.asarray(ids, dtype=np.int64)
        return self.p["model.embed_tokens.weight"][ids].copy()

    def forward_hidden(self, input_embed: np.ndarray, attention_bias: np.ndarray) -> np.ndarray:
        h = np.asarray(input_embed, dtype=F32)[0]
        bias = np.asarray(attention_bias, dtype=F32)[0, 0]
        for i in range(self.cfg.num_hidden_layers):
            xn = self.rmsnorm(h, self.p[f"model.layers.{i}.input_layernorm.weight"])
            q, k, v = self._qkv(i, xn, 0)
            h = self._layer_tail(i, h, self.attend(q, k, v, bias))
        return self.rmsnorm(h, self.p["model.norm.weight"])[None]

    def get_logits(self, hidden: np.ndarray) -> np.ndarray:
        w = self.p["model.embed_tokens.weight"] if self.cfg.tie_word_embeddings else self.p["lm_head.weight"]
        return self.rnd(np.matmul(np.asarray(hidden, dtype=F32), w.T)).astype(F32)

    def build_prefix_cache(self, prefix_embed: np.ndarray, prefix_bias: np.ndarray,
                           k_cache: np.ndarray, v_cache: np.ndarray) -> None:
        h = np.asarray(prefix_embed, dtype=F32)[0]
        n = h.shape[0]
        if n > k_cache.shape[2]:
            raise ValueError(f"KV write [0, {n}) outside cache capacity {k_cache.shape[2]}")
        bias = np.asarray(prefix_bias, dtype=F32)[0, 0]
        for i in range(self.cfg.num_hidden_layers):
            xn = self.rmsnorm(h, self.p[f"model.layers.{i}.input_layernorm.weight"])
            q, k, v = self._qkv(i, xn, 0)
            k_cache[i, 0, :n] = k
            v_cache[i, 0, :n] = v
            h = self._layer_tail(i, h, self.attend(q, k, v, bias))

    @staticmethod
    def kv_write(k: np.ndarray, v: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray, layer: int, start: int):
        """fast_dllm.kv_write (runtime.py:76-80) with _write_rows (:51-60): k / v [1, rows, nkv, hd] copied
        to cache rows [start, start + rows) of `layer` (caches [L, 1, cap, nkv, hd])."""
        rows = k.shape[1]
        if start < 0 or start + rows > k_cache.shape[2]:
            raise ValueError(f"KV write [{start}, {start + rows}) outside cache capacity {k_cache.shape[2]}")
        k_cache[layer, :, start:start + rows] = k
        v_cache[layer, :, start:start + rows] = v
        return k_cache, v_cache

    def attn_inplace(self, q: np.ndarray, k: np.ndarray, v: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                     layer: int, prefix_len: int, write_rel: int, attend_rel: int):
        """fast_dllm.attn_inplace (runtime.py:63-73): write k / v at rows [prefix_len + write_rel, + rows),
        then attend q [1, rows, nq, hd] (already rotated) over the cache slice [0, prefix_len + attend_rel)
        of `layer` (a slice: past the capacity it stops there), no mask (_attend, runtime.py:30-48).
        Returns (k_cache, v_cache, out [1, rows, nq, hd])."""
        write_start, attend_len = prefix_len + write_rel, prefix_len + attend_rel
        rows = k.shape[1]
        if write_start + rows > attend_len:
            raise ValueError(f"KV write [{write_start}, {write_start + rows}) past the attended rows [0, {attend_len})")
        self.kv_write(k, v, k_cache, v_cache, layer, write_start)
        out = self.attend(q[0], k_cache[layer, 0, :attend_len], v_cache[layer, 0, :attend_len])
        return k_cache, v_cache, out[None]

    def forward_cached(self, active_embed: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                       cache_offset: int, prefix_len: int, write_rel: int = 0,
                       attend_rel: int | None = None) -> np.ndarray:
        """cuda.py:639-666: per layer, the projections and RoPE, then the attn_inplace callback
        (runtime.py:51-73)."""
        h = np.asarray(active_embed, dtype=F32)[0]
        rows = h.shape[0]
        attend_rel = rows if attend_rel is None else attend_rel
        for i in range(self.cfg.num_hidden_layers):
            xn = self.rmsnorm(h, self.p[f"model.layers.{i}.input_layernorm.weight"])
            q, k, v = self._qkv(i, xn, int(cache_offset))
            _, _, attn = self.attn_inplace(q[None], k[None], v[None], k_cache, v_cache, i, prefix_len, write_rel,
                                           attend_rel)
            h = self._layer_tail(i, h, attn[0])
        return self.rmsnorm(h, self.p["model.norm.weight"])[None]

    def forward_block_partial(self, rp: int, active_embed, k_cache, v_cache, cache_offset, prefix_len):
        """cuda.py:740-788: write_rel = rp, attend_rel = bd_size."""
        return self.forward_cached(active_embed, k_cache, v_cache, cache_offset, prefix_len,
                                   write_rel=rp, attend_rel=self.cfg.bd_size)


def random_params(cfg: OracleConfig, seed: int, dtype: str = "bfloat16", std: float = 0.02,
                  embed_std: float | None = None, lm_head_std: float | None = None) -> dict[str, np.ndarray]:
    """Seeded N(0, std) weights in packed order, norm weights = 1 (tests/test_tiny_compile.py:45-55).

    ``embed_std`` scales the (tied) embedding separately; ``lm_head_std`` scales an untied lm_head
    separately (a peaked head, as BASELINE cfg3's N(0, 0.5), so that rows cross the 0.9 threshold).
    Values are rounded to ``dtype`` and returned as fp32 arrays.
    """
    rnd = rounder(dtype)
    rng = np.random.default_rng(seed)
    shapes = param_shapes(cfg)
    out = {}
    for name in param_names(cfg):
        shape = shapes[name]
        if name.endswith("norm.weight"):
            out[name] = np.ones(shape, dtype=F32)
        else:
            s = std
            if embed_std is not None and name == "model.embed_tokens.weight":
                s = embed_std
            if lm_head_std is not None and name == "lm_head.weight":
                s = lm_head_std
            out[name] = rnd((F32(s) * rng.standard_normal(shape, dtype=F32)).astype(F32))
    return out


def param_shapes(cfg: OracleConfig) -> dict[str, tuple[int, ...]]:
    c = cfg
    qkv = (c.num_attention_heads + 2 * c.num_key_value_heads) * c.head_dim
    shapes = {"model.embed_tokens.weight": (c.vocab_size, c.hidden_size), "model.norm.weight": (c.hidden_size,)}
    for i in range(c.num_hidden_layers):
        p = f"model.layers.{i}"
        shapes[f"{p}.self_attn.qkv_proj.weight"] = (qkv, c.hidden_size)
        shapes[f"{p}.self_attn.qkv_proj.bias"] = (qkv,)
        shapes[f"{p}.self_attn.o_proj.weight"] = (c.hidden_size, c.num_attention_heads * c.head_dim)
        shapes[f"{p}.mlp.gate_up_proj.weight"] = (2 * c.intermediate_size, c.hidden_size)
        shapes[f"{p}.mlp.down_proj.weight"] = (c.hidden_size, c.intermediate_size)
        shapes[f"{p}.input_layernorm.weight"] = (c.hidden_size,)
        shapes[f"{p}.post_attention_layernorm.weight"] = (c.hidden_size,)
    if not c.tie_word_embeddings:
        shapes["lm_head.weight"] = (c.vocab_size, c.hidden_size)
    return shapes
