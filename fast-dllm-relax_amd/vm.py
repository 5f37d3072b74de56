"""The nine-entry-point function table over libfdllm.so.

``HipVM`` stands where the reference holds ``tvm.relax.VirtualMachine`` (fast_dllm_relax/runners.py:614-615):
``vm["forward_cached"](embedded, k_cache, v_cache, cache_offset, prefix_len)`` and so on for every name of
REQUIRED_FNS (export_utils.py:13-17), plus ``get_confidence_m{rows}`` (model/metal.py:505-528).
Tensors are torch device tensors (PyTorch owns the memory); the packed weights are bound once at
construction instead of being passed on every call.  Work runs on torch's current stream, the stream
the reference's attention callbacks use (runtime.py:19-27).
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .config import FastDLLMConfig
from .params import TORCH_DTYPES, param_names

REQUIRED_FNS = (
    "embed", "forward_hidden", "get_logits", "build_prefix_cache", "forward_cached",
    "forward_block_partial_rp0", "forward_block_partial_rp8",
    "forward_block_partial_rp16", "forward_block_partial_rp24",
)


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


class HipVM:
    def __init__(self, cfg: FastDLLMConfig, params: list[torch.Tensor], *, dtype: str = "bfloat16",
                 max_rows: int = 64):
        if dtype not in TORCH_DTYPES:
            raise ValueError(f"unsupported dtype {dtype!r}")
        self.cfg = cfg
        self.dtype = dtype
        self.torch_dtype = TORCH_DTYPES[dtype]
        self.lib = _lib.load()
        c = _lib.FdllmConfig(cfg.vocab_size, cfg.hidden_size, cfg.intermediate_size, cfg.num_hidden_layers,
                             cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, cfg.rms_norm_eps,
                             cfg.rope_theta, int(cfg.tie_word_embeddings), cfg.bd_size,
                             _lib.DTYPE_BF16 if dtype == "bfloat16" else _lib.DTYPE_F16, max_rows)
        h = ctypes.c_void_p()
        _lib.check(self.lib.fdllm_create(ctypes.byref(c), ctypes.byref(h)))
        self.ctx = h
        names = [self.lib.fdllm_param_name(h, i).decode() for i in range(self.lib.fdllm_num_params(h))]
        if names != param_names(cfg):
            raise RuntimeError("libfdllm parameter order differs from params.param_names")
        self.bind(params)

    @classmethod
    def from_artifact(cls, artifact_dir, *, max_rows: int = 64, device: str = "cuda", **config_overrides) -> "HipVM":
        """A function table over the weights of a reference artifact directory (the params npz, names,
        dtype and KV-cache manifest of scripts/export_cuda.py; runners.py:597-639 loads the same files)."""
        from .params import config_from_artifact, load_artifact

        cfg = config_from_artifact(artifact_dir, **config_overrides)
        params, dtype = load_artifact(artifact_dir, cfg, device=device)
        return cls(cfg, params, dtype=dtype, max_rows=max_rows)

    def bind(self, params: list[torch.Tensor]) -> None:
        names = param_names(self.cfg)
        if len(params) != len(names):
            raise ValueError(f"expected {len(names)} params, got {len(params)}")
        for n, p in zip(names, params):
            if not p.is_cuda or p.dtype != self.torch_dtype or not p.is_contiguous():
                raise ValueError(f"param {n} must be a contiguous {self.torch_dtype} device tensor")
        self.params = list(params)
        arr = (ctypes.c_void_p * len(params))(*[p.data_ptr() for p in params])
        _lib.check(self.lib.fdllm_bind_weights(self.ctx, arr, len(params)))

    def close(self) -> None:
        if getattr(self, "ctx", None):
            self.lib.fdllm_destroy(self.ctx)
            self.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001 -- interpreter shutdown
            pass

    # ---- function table -------------------------------------------------------------------
    def __getitem__(self, name: str):
        if name in REQUIRED_FNS:
            return getattr(self, name)
        if name.startswith("get_confidence_m"):
            return self.get_confidence
        raise KeyError(name)

    def _check_cache(self, k: torch.Tensor, v: torch.Tensor) -> int:
        c = self.cfg
        exp = (c.num_hidden_layers, 1, k.shape[2], c.num_key_value_heads, c.head_dim)
        for t in (k, v):
            if tuple(t.shape) != exp or t.dtype != self.torch_dtype or not t.is_contiguous() or not t.is_cuda:
                raise ValueError(f"KV cache must be a contiguous {self.torch_dtype} device tensor of shape {exp}")
        if v.shape != k.shape:
            raise ValueError("k_cache and v_cache shapes differ")
        return int(k.shape[2])

    def _check_rows(self, x: torch.Tensor) -> int:
        if x.dim() != 3 or x.shape[0] != 1 or x.shape[2] != self.cfg.hidden_size or x.dtype != self.torch_dtype:
            raise ValueError(f"expected [1, rows, {self.cfg.hidden_size}] {self.torch_dtype}, got "
                             f"{tuple(x.shape)} {x.dtype}")
        if not x.is_contiguous():
            raise ValueError("activation tensor must be contiguous")
        return int(x.shape[1])

    def embed(self, input_ids: torch.Tensor) -> torch.Tensor:
        """ids [seq_len] int32 -> [seq_len, hidden] (cuda.py:698-699)."""
        ids = input_ids.to(dtype=torch.int32).contiguous()
        n = ids.numel()
        if n > 0:
            lo, hi = int(ids.min()), int(ids.max())
            if lo < 0 or hi >= self.cfg.vocab_size:
                raise ValueError(f"token id out of range [0, {self.cfg.vocab_size}): {lo if lo < 0 else hi}")
        out = torch.empty((n, self.cfg.hidden_size), dtype=self.torch_dtype, device=ids.device)
        _lib.check(self.lib.fdllm_embed(self.ctx, _ptr(ids), n, _ptr(out), _stream()))
        return out

    def embed_unchecked(self, ids: torch.Tensor) -> torch.Tensor:
        """embed of ids the caller has range-checked on the host (no device readback)."""
        out = torch.empty((ids.numel(), self.cfg.hidden_size), dtype=self.torch_dtype, device=ids.device)
        _lib.check(self.lib.fdllm_embed(self.ctx, _ptr(ids), ids.numel(), _ptr(out), _stream()))
        return out

    def forward_hidden(self, input_embed: torch.Tensor, attention_bias: torch.Tensor | None) -> torch.Tensor:
        s = self._check_rows(input_embed)
        if attention_bias is not None:
            if tuple(attention_bias.shape) != (1, 1, s, s) or attention_bias.dtype != torch.float32:
                raise ValueError(f"attention_bias must be [1, 1, {s}, {s}] float32")
            attention_bias = attention_bias.contiguous()
        out = torch.empty_like(input_embed)
        _lib.check(self.lib.fdllm_forward_hidden(self.ctx, _ptr(input_embed), s, _ptr(attention_bias), _ptr(out),
                                                 _stream()))
        return out

    def get_logits(self, hidden_states: torch.Tensor) -> torch.Tensor:
        rows = self._check_rows(hidden_states)
        out = torch.empty((1, rows, self.cfg.vocab_size), dtype=torch.float32, device=hidden_states.device)
        _lib.check(self.lib.fdllm_get_logits(self.ctx, _ptr(hidden_states), rows, _ptr(out), _stream()))
        return out

    def build_prefix_cache(self, prefix_embed: torch.Tensor, prefix_bias: torch.Tensor | None,
                           k_cache: torch.Tensor, v_cache: torch.Tensor):
        p = self._check_rows(prefix_embed)
        cap = self._check_cache(k_cache, v_cache)
        if prefix_bias is not None:
            if tuple(prefix_bias.shape) != (1, 1, p, p) or prefix_bias.dtype != torch.float32:
                raise ValueError(f"prefix_bias must be [1, 1, {p}, {p}] float32")
            prefix_bias = prefix_bias.contiguous()
        _lib.check(self.lib.fdllm_build_prefix_cache(self.ctx, _ptr(prefix_embed), p, _ptr(prefix_bias),
                                                     _ptr(k_cache), _ptr(v_cache), cap, _stream()))
        return k_cache, v_cache

    def forward_cached(self, active_embed: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                       cache_offset: torch.Tensor, prefix_len: int) -> torch.Tensor:
        rows = self._check_rows(active_embed)
        cap = self._check_cache(k_cache, v_cache)
        off = self._offset(cache_offset)
        out = torch.empty_like(active_embed)
        _lib.check(self.lib.fdllm_forward_cached(self.ctx, _ptr(active_embed), rows, _ptr(k_cache), _ptr(v_cache),
                                                 cap, _ptr(off), int(prefix_len), _ptr(out), _stream()))
        return out

    def _offset(self, cache_offset: torch.Tensor) -> torch.Tensor:
        if cache_offset.numel() != 1 or cache_offset.dtype != torch.int32 or not cache_offset.is_cuda:
            raise ValueError("cache_offset must be a 0-d int32 device tensor")
        return cache_offset

    def _partial(self, rp: int, active_embed, k_cache, v_cache, cache_offset, prefix_len):
        rows = self._check_rows(active_embed)
        cap = self._check_cache(k_cache, v_cache)
        off = self._offset(cache_offset)
        out = torch.empty_like(active_embed)
        _lib.check(self.lib.fdllm_forward_block_partial(self.ctx, rp, _ptr(active_embed), rows, _ptr(k_cache),
                                                        _ptr(v_cache), cap, _ptr(off), int(prefix_len), _ptr(out),
                                                        _stream()))
        return out

    def forward_block_partial_rp0(self, active_embed, k_cache, v_cache, cache_offset, prefix_len):
        return self._partial(0, active_embed, k_cache, v_cache, cache_offset, prefix_len)

    def forward_block_partial_rp8(self, active_embed, k_cache, v_cache, cache_offset, prefix_len):
        return self._partial(8, active_embed, k_cache, v_cache, cache_offset, prefix_len)

    def forward_block_partial_rp16(self, active_embed, k_cache, v_cache, cache_offset, prefix_len):
        return self._partial(16, active_embed, k_cache, v_cache, cache_offset, prefix_len)

    def forward_block_partial_rp24(self, active_embed, k_cache, v_cache, cache_offset, prefix_len):
        return self._partial(24, active_embed, k_cache, v_cache, cache_offset, prefix_len)

    # ---- batched steps (no reference counterpart: the reference is batch 1, cuda.py:796-836) ----
    # ---- the reference's attention callbacks (runtime.py:19-80) ------------------------------
    def _check_bsnh(self, t: torch.Tensor, heads: int, name: str) -> int:
        hd = self.cfg.head_dim
        if (t.dim() != 4 or t.shape[0] != 1 or t.shape[2] != heads or t.shape[3] != hd or t.dtype != self.torch_dtype
                or not t.is_cuda or not t.is_contiguous()):
            raise ValueError(f"{name} must be a contiguous {self.torch_dtype} device tensor [1, rows, {heads}, {hd}], "
                             f"got {tuple(t.shape)} {t.dtype}")
        return int(t.shape[1])

    def kv_write(self, k: torch.Tensor, v: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, layer: int,
                 start: int):
        """fast_dllm.kv_write (runtime.py:76-80): k / v [1, rows, nkv, hd] into cache rows [start, + rows) of
        `layer`, byte for byte; returns the caches (aliases)."""
        nkv = self.cfg.num_key_value_heads
        rows = self._check_bsnh(k, nkv, "k")
        if self._check_bsnh(v, nkv, "v") != rows:
            raise ValueError("k and v rows differ")
        cap = self._check_cache(k_cache, v_cache)
        _lib.check(self.lib.fdllm_kv_write(self.ctx, _ptr(k), _ptr(v), rows, _ptr(k_cache), _ptr(v_cache), cap,
                                           int(layer), int(start), _stream()))
        return k_cache, v_cache

    def attn_inplace(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, k_cache: torch.Tensor,
                     v_cache: torch.Tensor, layer: int, prefix_len: int, write_rel: int, attend_rel: int):
        """fast_dllm.attn_inplace (runtime.py:63-73): write k / v at cache rows [prefix_len + write_rel,
        + rows), then attend the rotated queries q [1, rows, nq, hd] over rows [0, prefix_len + attend_rel)
        with no mask.  Returns (k_cache, v_cache, out [1, rows, nq, hd])."""
        c = self.cfg
        rows = self._check_bsnh(q, c.num_attention_heads, "q")
        if self._check_bsnh(k, c.num_key_value_heads, "k") != rows or \
                self._check_bsnh(v, c.num_key_value_heads, "v") != rows:
            raise ValueError("q, k and v rows differ")
        cap = self._check_cache(k_cache, v_cache)
        out = torch.empty_like(q)
        _lib.check(self.lib.fdllm_attn_inplace(self.ctx, _ptr(q), _ptr(k), _ptr(v), rows, _ptr(k_cache), _ptr(v_cache),
                                               cap, int(layer), int(prefix_len), int(write_rel), int(attend_rel),
                                               _ptr(out), _stream()))
        return k_cache, v_cache, out

    def _check_batch_cache(self, k: torch.Tensor, v: torch.Tensor, nseq: int) -> int:
        c = self.cfg
        exp = (c.num_hidden_layers, nseq, k.shape[2] if k.dim() == 5 else -1, c.num_key_value_heads, c.head_dim)
        for t in (k, v):
            if tuple(t.shape) != exp or t.dtype != self.torch_dtype or not t.is_contiguous() or not t.is_cuda:
                raise ValueError(f"batched KV cache must be a contiguous {self.torch_dtype} device tensor of shape {exp}")
        return int(k.shape[2])

    def _check_batch_rows(self, x: torch.Tensor) -> tuple[int, int]:
        if x.dim() != 3 or x.shape[2] != self.cfg.hidden_size or x.dtype != self.torch_dtype or not x.is_contiguous():
            raise ValueError(f"expected a contiguous [nseq, rows, {self.cfg.hidden_size}] {self.torch_dtype} tensor, "
                             f"got {tuple(x.shape)} {x.dtype}")
        return int(x.shape[0]), int(x.shape[1])

    @staticmethod
    def _batch_offsets(cache_offset: torch.Tensor, nseq: int) -> torch.Tensor:
        if cache_offset.shape != (nseq,) or cache_offset.dtype != torch.int32 or not cache_offset.is_cuda:
            raise ValueError(f"cache_offset must be an int32 device tensor of shape ({nseq},)")
        return cache_offset.contiguous()

    @staticmethod
    def _prefix_lens(prefix_lens, nseq: int):
        lens = [int(p) for p in prefix_lens]
        if len(lens) != nseq:
            raise ValueError(f"prefix_lens has {len(lens)} entries for {nseq} sequences")
        return (ctypes.c_int64 * nseq)(*lens)

    def forward_cached_batch(self, active_embed: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                             cache_offset: torch.Tensor, prefix_lens) -> torch.Tensor:
        """forward_cached of nseq sequences at once: active_embed [nseq, rows, H], caches
        [L, nseq, cap, nkv, hd], cache_offset int32 [nseq], prefix_lens nseq host ints."""
        nseq, rows = self._check_batch_rows(active_embed)
        cap = self._check_batch_cache(k_cache, v_cache, nseq)
        off = self._batch_offsets(cache_offset, nseq)
        out = torch.empty_like(active_embed)
        _lib.check(self.lib.fdllm_forward_cached_batch(self.ctx, _ptr(active_embed), nseq, rows, _ptr(k_cache),
                                                       _ptr(v_cache), cap, _ptr(off), self._prefix_lens(prefix_lens, nseq),
                                                       _ptr(out), _stream()))
        return out

    def forward_block_partial_batch(self, replace_position: int, active_embed: torch.Tensor, k_cache: torch.Tensor,
                                    v_cache: torch.Tensor, cache_offset: torch.Tensor, prefix_lens) -> torch.Tensor:
        """forward_block_partial_rp{replace_position} of nseq sequences at once (shapes as forward_cached_batch)."""
        nseq, rows = self._check_batch_rows(active_embed)
        cap = self._check_batch_cache(k_cache, v_cache, nseq)
        off = self._batch_offsets(cache_offset, nseq)
        out = torch.empty_like(active_embed)
        _lib.check(self.lib.fdllm_forward_block_partial_batch(
            self.ctx, int(replace_position), _ptr(active_embed), nseq, rows, _ptr(k_cache), _ptr(v_cache), cap,
            _ptr(off), self._prefix_lens(prefix_lens, nseq), _ptr(out), _stream()))
        return out

    def build_prefix_cache_seq(self, prefix_embed: torch.Tensor, prefix_bias: torch.Tensor | None,
                               k_cache: torch.Tensor, v_cache: torch.Tensor, seq: int):
        """build_prefix_cache of sequence `seq` into its slice of a batched cache [L, nseq, cap, nkv, hd]."""
        p = self._check_rows(prefix_embed)
        nseq = int(k_cache.shape[1]) if k_cache.dim() == 5 else -1
        cap = self._check_batch_cache(k_cache, v_cache, nseq)
        if prefix_bias is not None:
            if tuple(prefix_bias.shape) != (1, 1, p, p) or prefix_bias.dtype != torch.float32:
                raise ValueError(f"prefix_bias must be [1, 1, {p}, {p}] float32")
            prefix_bias = prefix_bias.contiguous()
        _lib.check(self.lib.fdllm_build_prefix_cache_seq(self.ctx, _ptr(prefix_embed), p, _ptr(prefix_bias),
                                                         _ptr(k_cache), _ptr(v_cache), cap, nseq, int(seq), _stream()))
        return k_cache, v_cache

    def get_confidence(self, hidden_states: torch.Tensor, logits: torch.Tensor | None = None, out=None):
        """(ids [1, rows] int32, maxp [1, rows] fp32), unshifted (metal.py:505-528).  out: an optional
        contiguous [1, 2 rows] int32 device tensor that receives ids then maxp (bit-cast), so that one
        copy brings both back to the host."""
        rows = self._check_rows(hidden_states)
        if out is None:
            ids = torch.empty((1, rows), dtype=torch.int32, device=hidden_states.device)
            maxp = torch.empty((1, rows), dtype=torch.float32, device=hidden_states.device)
        else:
            if tuple(out.shape) != (1, 2 * rows) or out.dtype != torch.int32 or not out.is_contiguous():
                raise ValueError(f"out must be a contiguous [1, {2 * rows}] int32 tensor")
            ids, maxp = out[:, :rows], out[:, rows:].view(torch.float32)
        if logits is not None and (tuple(logits.shape) != (1, rows, self.cfg.vocab_size)
                                   or logits.dtype != torch.float32 or not logits.is_contiguous()):
            raise ValueError("logits must be a contiguous [1, rows, vocab] float32 tensor")
        _lib.check(self.lib.fdllm_get_confidence(self.ctx, _ptr(hidden_states), rows, _ptr(ids), _ptr(maxp),
                                                 _ptr(logits), _stream()))
        return ids, maxp

    def confidence_from_logits(self, logits: torch.Tensor):
        """Device confidence of given fp32 logits [1, rows, vocab] (runtime.py:176-181 restated)."""
        if logits.dim() != 3 or logits.shape[2] != self.cfg.vocab_size or logits.dtype != torch.float32:
            raise ValueError("logits must be [1, rows, vocab] float32")
        logits = logits.contiguous()
        rows = int(logits.shape[1])
        ids = torch.empty((1, rows), dtype=torch.int32, device=logits.device)
        maxp = torch.empty((1, rows), dtype=torch.float32, device=logits.device)
        _lib.check(self.lib.fdllm_confidence_from_logits(self.ctx, _ptr(logits), rows, self.cfg.vocab_size,
                                                         self.cfg.vocab_size, _ptr(ids), _ptr(maxp), _stream()))
        return ids, maxp
