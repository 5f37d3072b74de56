"""Prefix KV cache, step functions and the Fast-dLLM v2 decode loop over the HIP function table.

Mirror of fast_dllm_relax/runtime.py with ``vm`` a ``HipVM``: the same names, arguments, cache
contract, window checks and exceptions, so the reference's loop reads the same here.
  PrefixCache / allocate_prefix_cache / _check_write        runtime.py:196-263
  build_prefix_cache_from_ids / _prefill / _embed            runtime.py:266-330
  _forward_cached                                            runtime.py:333-343
  shifted_confidence                                         runtime.py:158-181 (device confidence path)
  score_active_block_cached_fast / _refine / _partial        runtime.py:346-436
  score_sequence_block / score_masked_continuation           runtime.py:439-588
  relax_greedy_generate                                      runtime.py:591-880
Differences: prefill passes no host-built bias when block_size is the model's bd_size (the kernels
apply the same block-causal rule arithmetically, build_prefix_block_attention_bias semantics,
cuda.py:148-177); the cached-step
confidence always runs on the device (fused lm_head + argmax + max-softmax), reading back 2 x rows values.
"""

from __future__ import annotations

import dataclasses
import time
from typing import Any

import numpy as np
import torch

from .vm import HipVM, _stream


@dataclasses.dataclass(frozen=True)
class CacheSpec:
    num_layers: int
    num_kv_heads: int
    head_dim: int
    dtype: str


def cache_spec_of(vm: HipVM) -> CacheSpec:
    c = vm.cfg
    return CacheSpec(c.num_hidden_layers, c.num_key_value_heads, c.head_dim, vm.dtype)


@dataclasses.dataclass
class PrefixCache:
    """In-place KV cache of one sequence: k / v [num_layers, 1, capacity, num_kv_heads, head_dim].
    Rows [0, prefix_len) hold the committed prefix and are never rewritten."""

    k: torch.Tensor
    v: torch.Tensor
    prefix_len: int
    spec: CacheSpec

    @property
    def capacity(self) -> int:
        return int(self.k.shape[2])

    def commit(self, rows: int) -> None:
        if self.prefix_len + rows > self.capacity:
            raise ValueError(f"commit past capacity: {self.prefix_len} + {rows} > {self.capacity}")
        self.prefix_len += rows

    def ensure_capacity(self, rows: int, dev: Any = None) -> None:
        """Grow (reallocate, copy the committed rows) so that ``rows`` rows fit."""
        if rows <= self.capacity:
            return
        bigger = allocate_prefix_cache(self.spec, self.k.device, rows)
        bigger.k[:, :, :self.prefix_len].copy_(self.k[:, :, :self.prefix_len])
        bigger.v[:, :, :self.prefix_len].copy_(self.v[:, :, :self.prefix_len])
        self.k, self.v = bigger.k, bigger.v


def allocate_prefix_cache(spec: CacheSpec, dev: Any, rows: int, *, block_size: int = 32) -> PrefixCache:
    """An empty PrefixCache with capacity ``rows`` rounded up to a multiple of block_size."""
    from .params import TORCH_DTYPES

    capacity = -(-max(int(rows), 1) // block_size) * block_size
    shape = (spec.num_layers, 1, capacity, spec.num_kv_heads, spec.head_dim)
    td = TORCH_DTYPES[spec.dtype]
    return PrefixCache(k=torch.empty(shape, dtype=td, device=dev), v=torch.empty(shape, dtype=td, device=dev),
                       prefix_len=0, spec=spec)


def _check_write(cache: PrefixCache, write_start: int, attend_len: int) -> None:
    if write_start < cache.prefix_len:
        raise ValueError(f"KV write at row {write_start} would overwrite the committed prefix [0, {cache.prefix_len})")
    if attend_len > cache.capacity:
        raise ValueError(f"cached call needs {attend_len} rows; cache capacity is {cache.capacity}")


def _ids_tensor(vm: HipVM, ids) -> torch.Tensor:
    arr = np.asarray(ids, dtype=np.int64)
    if arr.size and (arr.min() < 0 or arr.max() >= vm.cfg.vocab_size):
        raise ValueError(f"token id out of range [0, {vm.cfg.vocab_size})")
    return torch.from_numpy(arr.astype(np.int32)).pin_memory().to("cuda", non_blocking=True)


def _embed(vm: HipVM, ids) -> torch.Tensor:
    """vm.embed of ``ids`` reshaped to [1, len(ids), hidden] (runtime.py:326-330)."""
    return vm.embed_unchecked(_ids_tensor(vm, ids))[None]


def _to_host(t: torch.Tensor) -> np.ndarray:
    """Device tensor -> numpy through page-locked memory (torch's caching host allocator, so repeated
    calls reuse the staging blocks): a pageable copy of the 64 x 151936 fp32 scoring logits ran at
    4 GB/s (9.4 ms), a pinned one at the link's rate."""
    host = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
    host.copy_(t)
    return host.numpy()


def _offset_tensor(value: int) -> torch.Tensor:
    return torch.tensor(int(value), dtype=torch.int32).pin_memory().to("cuda", non_blocking=True)


def build_prefix_cache_from_ids(vm: HipVM, prefix_ids, *, block_size: int, cache_spec: CacheSpec | None = None,
                                capacity: int | None = None, chunked_prefill: bool = False) -> PrefixCache:
    spec = cache_spec or cache_spec_of(vm)
    prefix_len = len(prefix_ids)
    cache = allocate_prefix_cache(spec, "cuda", max(prefix_len, capacity or 0), block_size=block_size)
    if prefix_len == 0:
        return cache
    if chunked_prefill and prefix_len > block_size:
        if prefix_len % block_size != 0:
            raise ValueError(f"chunked_prefill requires a block-aligned prefix; got {prefix_len} tokens "
                             f"with block_size={block_size}.")
        _prefill(vm, list(prefix_ids[:block_size]), cache, block_size=block_size)
        for start in range(block_size, prefix_len, block_size):
            _forward_cached(vm, list(prefix_ids[start:start + block_size]), cache)
            cache.commit(block_size)
        return cache
    _prefill(vm, list(prefix_ids), cache, block_size=block_size)
    return cache


def _prefill(vm: HipVM, prefix_ids, cache: PrefixCache, *, block_size: int) -> None:
    """build_prefix_cache into an empty cache (runtime.py:312-323).  The kernels apply the block-causal
    rule of build_prefix_block_attention_bias arithmetically with the model's bd_size; another
    block_size passes the reference's explicit bias instead."""
    if cache.prefix_len != 0:
        raise ValueError("build_prefix_cache writes from row 0; the cache already has a prefix")
    _check_write(cache, 0, len(prefix_ids))
    bias = None
    if block_size != vm.cfg.bd_size:
        bias = torch.from_numpy(build_prefix_block_attention_bias(0, len(prefix_ids), block_size=block_size)).cuda()
    vm.build_prefix_cache(_embed(vm, prefix_ids), bias, cache.k, cache.v)
    cache.commit(len(prefix_ids))


def _forward_cached(vm: HipVM, active_ids, cache: PrefixCache) -> torch.Tensor:
    _check_write(cache, cache.prefix_len, cache.prefix_len + len(active_ids))
    return vm.forward_cached(_embed(vm, active_ids), cache.k, cache.v, _offset_tensor(cache.prefix_len),
                             cache.prefix_len)


def shifted_confidence(vm: HipVM, hidden: torch.Tensor) -> tuple[np.ndarray, np.ndarray, int]:
    """(shifted ids [rows] int64, shifted max probs [rows] fp32, unshifted last-row argmax).

    Device path of runtime.py:168-174: the fused lm_head + confidence kernel reduces the logits, only
    2 x rows values come back."""
    rows = hidden.shape[1]
    both_d = torch.empty((1, 2 * rows), dtype=torch.int32, device=hidden.device)
    vm.get_confidence(hidden, out=both_d)
    both = both_d.cpu().numpy()[0].view(np.float32)
    ids = both[:rows].view(np.int32).astype(np.int64)
    maxp = both[rows:].astype(np.float32)
    return np.concatenate([ids[:1], ids[:-1]]), np.concatenate([maxp[:1], maxp[:-1]]), int(ids[-1])


def score_active_block_cached_fast(vm: HipVM, active_ids, prefix_cache: PrefixCache):
    hidden = _forward_cached(vm, active_ids, prefix_cache)
    prefix_cache.commit(len(active_ids))
    ids, probs, last = shifted_confidence(vm, hidden)
    return ids, probs, last, prefix_cache


def score_active_block_refine(vm: HipVM, active_ids, prefix_cache: PrefixCache):
    ids, probs, _ = shifted_confidence(vm, _forward_cached(vm, active_ids, prefix_cache))
    return ids, probs


def score_active_block_partial_perlayer(vm: HipVM, small_block_ids, prefix_cache: PrefixCache,
                                        replace_position: int, *, block_size: int):
    write_start = prefix_cache.prefix_len + replace_position
    _check_write(prefix_cache, write_start, prefix_cache.prefix_len + block_size)
    fn = vm[f"forward_block_partial_rp{replace_position}"]
    hidden = fn(_embed(vm, small_block_ids), prefix_cache.k, prefix_cache.v, _offset_tensor(write_start),
                prefix_cache.prefix_len)
    ids, probs, _ = shifted_confidence(vm, hidden)
    return ids, probs


def threshold_f32(threshold: float) -> float:
    """Largest fp32 value <= threshold: the device's fp32 `p > t` then decides exactly as the reference's
    numpy `p > threshold` on an fp32 probability (runtime.py:796)."""
    t = np.float32(threshold)
    if float(t) > threshold:
        t = np.nextafter(t, np.float32(-np.inf))
    return float(t)


@dataclasses.dataclass
class UnmaskReport:
    """What one device step reports (include/fdllm.h, fdllm_unmask): the block after the update, the
    selected rows of the sub-block, and the sub-block's shifted ids / probabilities."""

    block: list
    selected: list
    masked: list
    ids: list
    probs: np.ndarray
    left: int
    last: int


class DeviceBlock:
    """The active block of the decode loop (runtime.py:748-843) held on the device.

    The block's ids and its RoPE offsets live in device memory, uploaded once per block.  Each model
    call embeds its rows straight from there, and fdllm_get_confidence_unmask applies the threshold
    rule on the device and writes a report into pinned host memory, which the host polls: no readback
    copy and no upload per step."""

    REPORT_TIMEOUT_S = 60.0

    def __init__(self, vm: HipVM, block_size: int, sub_rows: int, mask_id: int, threshold: float):
        import ctypes

        from . import _lib

        self.vm, self.lib, self._lib = vm, vm.lib, _lib
        self.bd, self.sub = int(block_size), int(sub_rows)
        self.mask_id, self.thr = int(mask_id), threshold_f32(threshold)
        self.buf = torch.zeros(self.bd + 1 + self.bd // self.sub, dtype=torch.int32, device="cuda")
        self.block = self.buf[:self.bd]
        self._stage = torch.empty(self.buf.numel(), dtype=torch.int32, pin_memory=True)
        self._stage_np = self._stage.numpy()
        self.words = 4 + self.bd + 2 * self.sub + 4
        host, dev = ctypes.c_void_p(), ctypes.c_void_p()
        _lib.check(self.lib.fdllm_host_alloc(self.words * 4, ctypes.byref(host), ctypes.byref(dev)))
        self._host, self._dev = host, dev
        self.rep = np.ctypeslib.as_array(ctypes.cast(host, ctypes.POINTER(ctypes.c_int32)), shape=(self.words,))
        self.seq = int(self.rep[0])
        self._pre = torch.empty((self.bd, vm.cfg.hidden_size), dtype=vm.torch_dtype, device="cuda")
        self._pre_ok = False  # whether self._pre holds the block's rows as the last update left them
        self._st = None       # the stream of the block's calls (torch's current stream at load())
        self._ck = self._cv = None  # the cache the prepared pointers belong to
        self._kcv = (0, 0, 0)
        self._outs: dict = {}

    def close(self) -> None:
        if self._host is not None:
            torch.cuda.synchronize()
            self.lib.fdllm_host_free(self._host)
            self._host = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001 - interpreter shutdown
            pass

    def load(self, ids, prefix_len: int) -> None:
        """Upload the block's ids and the RoPE offsets of its full step (prefix_len) and partial steps
        (prefix_len + rp)."""
        vals = [int(t) for t in ids] + [prefix_len] + [prefix_len + rp for rp in range(0, self.bd, self.sub)]
        if len(vals) != self.buf.numel():
            raise ValueError(f"block of {len(ids)} ids, expected {self.bd}")
        # one pinned staging buffer for every load: the previous load's copy has run long before (the
        # host has waited for the device's reports since)
        self._stage_np[:] = vals
        self.buf.copy_(self._stage, non_blocking=True)
        self._pre_ok = False
        self._st = _stream()

    # The model calls of the loop go straight to the C ABI with arguments prepared once: the block's
    # embedded rows (self._pre), the cache pointers (checked by HipVM the first time a cache is seen), the
    # offsets in self.buf and one output buffer per call kind, which the next call of that kind
    # overwrites after the stream has consumed it (the unmask that follows every call).  Between two
    # calls the host's work is on the GPU's critical path: this takes it from about 25 to about 10 us.
    def _bind(self, cache: PrefixCache) -> None:
        if cache.k is not self._ck or cache.v is not self._cv:
            cap = self.vm._check_cache(cache.k, cache.v)
            self._ck, self._cv, self._kcv = cache.k, cache.v, (cache.k.data_ptr(), cache.v.data_ptr(), cap)
        if self._st is None:
            self._st = _stream()
        if not self._pre_ok:
            self._embed_block()

    def _embed_block(self) -> None:
        """The block's rows, embedded from its ids on the device into self._pre (stream-ordered: the
        previous model call has read the buffer by the time this overwrites it)."""
        self._lib.check(self.lib.fdllm_embed(self.vm.ctx, self.block.data_ptr(), self.bd, self._pre.data_ptr(),
                                             self._st))
        self._pre_ok = True

    def _out(self, rows: int) -> torch.Tensor:
        out = self._outs.get(rows)
        if out is None:
            out = self._outs[rows] = torch.empty((1, rows, self.vm.cfg.hidden_size), dtype=self.vm.torch_dtype,
                                                 device="cuda")
        return out

    def forward_full(self, cache: PrefixCache) -> torch.Tensor:
        """forward_cached over the whole block at the cache frontier (runtime.py:333-343)."""
        _check_write(cache, cache.prefix_len, cache.prefix_len + self.bd)
        self._bind(cache)
        kp, vp, cap = self._kcv
        out = self._out(self.bd)
        self._lib.check(self.lib.fdllm_forward_cached(self.vm.ctx, self._pre.data_ptr(), self.bd, kp, vp, cap,
                                                      self.buf.data_ptr() + 4 * self.bd, cache.prefix_len,
                                                      out.data_ptr(), self._st))
        return out

    def forward_partial(self, cache: PrefixCache, rp: int) -> torch.Tensor:
        """forward_block_partial_rp{rp} over rows [rp, rp + sub) (runtime.py:401-436)."""
        _check_write(cache, cache.prefix_len + rp, cache.prefix_len + self.bd)
        self._bind(cache)
        kp, vp, cap = self._kcv
        out = self._out(self.sub)
        x = self._pre.data_ptr() + rp * self.vm.cfg.hidden_size * self._pre.element_size()
        off = self.buf.data_ptr() + 4 * (self.bd + 1 + rp // self.sub)
        self._lib.check(self.lib.fdllm_forward_block_partial(self.vm.ctx, rp, x, self.sub, kp, vp, cap, off,
                                                             cache.prefix_len, out.data_ptr(), self._st))
        return out

    def unmask(self, hidden: torch.Tensor, row0: int, s0: int, sub: int) -> UnmaskReport:
        """lm_head + confidence + the threshold rule on block rows [s0, s0 + sub) (sub = 0: report only),
        then wait for the report."""
        rows = hidden.shape[1] if any(hidden is o for o in self._outs.values()) else self.vm._check_rows(hidden)
        if self._st is None:
            self._st = _stream()
        self.seq = (self.seq + 1) & 0x7FFFFFFF
        seq = self.seq
        self._lib.check(self.lib.fdllm_get_confidence_unmask(
            self.vm.ctx, hidden.data_ptr(), rows, row0, self.block.data_ptr(), s0, sub, self.mask_id, self.thr,
            None, None, self._dev, seq, self._st))
        # the next step of this block embeds rows of the block as this update leaves it: embedding all of
        # them now, behind the update on the stream, takes the embed launch off the host's path between
        # two model calls (a new block's load() embeds again at its first call)
        if sub > 0:
            self._embed_block()
        else:
            self._pre_ok = False
        rep = self.rep
        if rep[0] != seq:
            deadline = time.perf_counter() + self.REPORT_TIMEOUT_S
            n = 0
            while rep[0] != seq:
                n += 1
                if n & 0xFFFF == 0 and time.perf_counter() > deadline:
                    torch.cuda.synchronize()  # surfaces a device error, if there is one
                    if rep[0] != seq:
                        raise RuntimeError(f"device unmask report {seq} did not arrive")
        words = rep[:4 + self.bd + 2 * sub + 4].copy()
        b = 4 + self.bd

        def mask64(i):  # a (low, high) word pair
            return (int(words[i]) & 0xFFFFFFFF) | (int(words[i + 1]) & 0xFFFFFFFF) << 32

        masked_bits, sel_bits = mask64(b + 2 * sub), mask64(b + 2 * sub + 2)
        return UnmaskReport(block=words[4:b].tolist(), selected=[r for r in range(sub) if sel_bits >> r & 1],
                            masked=[r for r in range(sub) if masked_bits >> r & 1], ids=words[b:b + sub].tolist(),
                            probs=words[b + sub:b + 2 * sub].view(np.float32).copy(), left=int(words[1]),
                            last=int(words[3]))


def _device_block(vm: HipVM, block_size: int, sub_rows: int, mask_id: int, threshold: float) -> DeviceBlock:
    """The vm's DeviceBlock for these loop parameters (kept across calls: its pinned report buffer is
    allocated once)."""
    key = (block_size, sub_rows, mask_id, threshold_f32(threshold))
    cache = vm.__dict__.setdefault("_device_blocks", {})
    if key not in cache:
        cache[key] = DeviceBlock(vm, block_size, sub_rows, mask_id, threshold)
    return cache[key]


def build_prefix_block_attention_bias(prefix_len: int, block_len: int, *, block_size: int | None = None,
                                      blocked_value: float = -1e9) -> np.ndarray:
    """[1, 1, T, T] block-causal bias (cuda.py:148-177)."""
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
    return np.where(allowed, 0.0, blocked_value).astype(np.float32)[None, None]


def extract_shifted_block_logits(logits, *, prefix_len: int, block_len: int):
    """Position i is predicted from logits at i-1 (cuda.py:180-204)."""
    if logits.ndim != 3:
        raise ValueError(f"Expected logits to have rank 3, got shape {tuple(logits.shape)}")
    if block_len <= 0:
        raise ValueError("block_len must be positive")
    if prefix_len + block_len > logits.shape[1]:
        raise ValueError(f"Requested prefix_len={prefix_len} and block_len={block_len} "
                         f"for logits of length {logits.shape[1]}")
    src = ([prefix_len - 1] + list(range(prefix_len, prefix_len + block_len - 1)) if prefix_len > 0
           else [0] + list(range(0, block_len - 1)))
    return logits[:, src, :]


def score_sequence_block(vm: HipVM, sequence_ids, *, block_size: int):
    """Raw active-block logits and shifted block logits of a token sequence (runtime.py:439-482),
    as host numpy arrays."""
    if len(sequence_ids) <= block_size:
        prefix_ids, active = [], list(sequence_ids)
    else:
        plen = ((len(sequence_ids) - 1) // block_size) * block_size
        prefix_ids, active = list(sequence_ids[:plen]), list(sequence_ids[plen:])
    bias = torch.from_numpy(build_prefix_block_attention_bias(len(prefix_ids), len(active),
                                                              block_size=block_size)).cuda()
    hidden = vm.forward_hidden(_embed(vm, prefix_ids + active), bias)
    logits = _to_host(vm.get_logits(hidden))
    cur = logits[:, -len(active):, :]
    shifted = extract_shifted_block_logits(logits, prefix_len=len(prefix_ids), block_len=len(active))
    return cur, shifted


def score_masked_continuation(vm: HipVM, prefix_ids, continuation_ids, *, block_size: int, mask_id: int,
                              eos_token_id: int | None = None, cached_prefix=None, chunked_prefill: bool = False):
    """Masked-continuation scoring (runtime.py:485-588): returns (logits [len(cont), vocab] numpy,
    (aligned prefix ids, PrefixCache) or None)."""
    if not continuation_ids:
        return np.empty((0, 0), dtype=np.float32), cached_prefix
    pcl = (len(prefix_ids) // block_size) * block_size
    if pcl == 0:
        seq = list(prefix_ids) + [mask_id] * len(continuation_ids)
        _, shifted = score_sequence_block(vm, seq, block_size=block_size)
        return shifted[0, -len(continuation_ids):, :], None
    aligned = list(prefix_ids[:pcl])
    tail_rows = max(len(prefix_ids) - pcl + len(continuation_ids), block_size)
    if cached_prefix is not None and cached_prefix[0] == aligned:
        cache = cached_prefix[1]
        cache.ensure_capacity(pcl + tail_rows)
    else:
        cache = build_prefix_cache_from_ids(vm, aligned, block_size=block_size, capacity=pcl + tail_rows,
                                            chunked_prefill=chunked_prefill)
    real = list(prefix_ids[cache.prefix_len:])
    active = real + [mask_id] * len(continuation_ids)
    if len(active) <= block_size:
        pad = block_size - len(active)
        if pad:
            active = active + [mask_id] * pad
            if eos_token_id is not None:
                active[len(real) + len(continuation_ids)] = eos_token_id
    hidden = _forward_cached(vm, active, cache)
    logits = vm.get_logits(hidden)
    shifted = torch.cat([logits[:, :1, :], logits[:, :-1, :]], dim=1)
    end = len(real) + len(continuation_ids)
    return _to_host(shifted[0, len(real):end, :]), (aligned, cache)


def relax_greedy_generate(vm: HipVM, prompt_token_ids, *, max_new_tokens: int, block_size: int = 32,
                          small_block_size: int = 8, threshold: float = 0.9, temperature: float = 0.0,
                          top_p: float = 0.95, use_block_cache: bool = True, mask_id: int,
                          stop_token: int | None, timing: dict | None = None, chunked_prefill: bool = False,
                          trace: list | None = None, decisions: list | None = None, device_loop: bool = True):
    """Fast-dLLM v2 block-diffusion generation (runtime.py:591-880), temperature 0.

    ``trace`` (optional) receives one tuple per model call, as oracle.runtime.greedy_generate logs.
    With ``device_loop`` (the default, when block_size is the model's bd_size, at most 64, and a multiple
    of small_block_size) the cached block's ids stay on the device: each refinement step embeds from
    there and ends with the fused lm_head + confidence + threshold unmask (fdllm_get_confidence_unmask),
    and the host reads only the step's report.  ``decisions`` (optional) then receives, per cached
    refinement step, the report's sub-block view: the rows that were masked, their shifted probabilities
    and ids, and the rows the device selected (and {"kind": "append", "token": t} per block append).  Without it, each step reads the confidence back and
    applies the rule on the host, as the reference does, and ``decisions`` receives the same view of the
    host's decision; a stateless step (the first block of a prompt shorter than a block) records
    {"kind": "stateless", ...} with its float64 probabilities."""
    if temperature != 0.0:
        raise NotImplementedError("Fast-dLLM Relax runner currently supports only temperature=0.")
    if top_p <= 0:
        raise ValueError("top_p must be positive.")
    if max_new_tokens < 0:
        raise ValueError("max_new_tokens must be non-negative.")
    if block_size <= 0 or small_block_size <= 0:
        raise ValueError("block_size and small_block_size must be positive.")

    t_start = time.perf_counter()
    prefill_recorded = False
    dblk = None
    if (device_loop and block_size == vm.cfg.bd_size and block_size <= 64 and small_block_size <= block_size
            and block_size % small_block_size == 0):
        dblk = _device_block(vm, block_size, small_block_size, mask_id, threshold)
    generated = list(prompt_token_ids)
    plen0 = len(generated)
    unmask_updates = block_recomputes = partial_recomputes = block_appends = 0
    prefix_cache: PrefixCache | None = None
    block_kv_valid = False
    capacity = -(-(plen0 + max_new_tokens) // block_size) * block_size + block_size

    def has_completed_stop(seq, plen):
        if stop_token is None:
            return False
        suffix = seq[plen:]
        if stop_token not in suffix:
            return False
        return mask_id not in suffix[:suffix.index(stop_token)]

    def make_continuation(tokens):
        raw = tokens[plen0:plen0 + max_new_tokens]
        first = next((i for i, t in enumerate(raw) if t == mask_id), len(raw))
        return raw[:first]

    def stats():
        return {"unmask_updates": unmask_updates, "block_recomputes": block_recomputes,
                "partial_recomputes": partial_recomputes, "block_appends": block_appends}

    def log(*item):
        if trace is not None:
            trace.append(item)

    if plen0 % block_size == 0 and plen0 > 0 and max_new_tokens > 0:
        last_start = plen0 - block_size
        prefix_cache = build_prefix_cache_from_ids(vm, generated[:last_start], block_size=block_size,
                                                   capacity=capacity, chunked_prefill=chunked_prefill)
        _, _, nxt, prefix_cache = score_active_block_cached_fast(vm, generated[last_start:], prefix_cache)
        log("append", prefix_cache.prefix_len, nxt)
        block_recomputes += 1
        block_appends += 1
        generated.append(nxt)
        if stop_token is not None and nxt == int(stop_token):
            if timing is not None:
                timing["prefill_latency_s"] = time.perf_counter() - t_start
            return make_continuation(generated), stats()

    while len(generated) - plen0 < max_new_tokens:
        prompt_length = len(generated)
        x_t = generated + [mask_id] * (block_size - prompt_length % block_size)
        a0 = len(x_t) - block_size
        if a0 == 0:
            use_cache = False
        else:
            use_cache = True
            if a0 != (prefix_cache.prefix_len if prefix_cache is not None else 0):
                prefix_cache = build_prefix_cache_from_ids(vm, x_t[:a0], block_size=block_size, capacity=capacity,
                                                           chunked_prefill=chunked_prefill)
                block_kv_valid = False
        if not prefill_recorded:
            if timing is not None:
                torch.cuda.synchronize()
                timing["prefill_latency_s"] = time.perf_counter() - t_start
            prefill_recorded = True
        if use_cache and dblk is not None:
            dblk.load(x_t[a0:], prefix_cache.prefix_len)

        for s0 in range(0, block_size, small_block_size):
            s1 = min(block_size, s0 + small_block_size)
            while True:
                local = [i for i, t in enumerate(x_t[a0 + s0:a0 + s1]) if t == mask_id]
                if not local:
                    break
                if has_completed_stop(x_t, prompt_length):
                    return make_continuation(x_t), stats()
                if use_cache and dblk is not None:
                    use_partial = use_block_cache and block_kv_valid and x_t[a0 + s0] != mask_id
                    if use_partial:
                        hidden = dblk.forward_partial(prefix_cache, s0)
                    else:
                        hidden = dblk.forward_full(prefix_cache)
                        block_kv_valid = use_block_cache
                    block_recomputes += 1
                    if use_partial:
                        partial_recomputes += 1
                    rep = dblk.unmask(hidden, 0 if use_partial else s0, s0, s1 - s0)
                    x_t[a0:a0 + block_size] = rep.block
                    rows = rep.selected
                    unmask_updates += len(rows)
                    if trace is not None:
                        log("partial" if use_partial else "full", s0, tuple(rows), tuple(rep.ids[r] for r in rows))
                    if decisions is not None:
                        decisions.append({"kind": "partial" if use_partial else "full", "s0": s0,
                                          "masked": rep.masked, "probs": rep.probs, "ids": rep.ids,
                                          "selected": rows})
                elif use_cache:
                    use_partial = use_block_cache and block_kv_valid and x_t[a0 + s0] != mask_id
                    if use_partial:
                        ids, probs = score_active_block_partial_perlayer(vm, x_t[a0 + s0:a0 + s1], prefix_cache,
                                                                         s0, block_size=block_size)
                    else:
                        ids, probs = score_active_block_refine(vm, x_t[a0:], prefix_cache)
                        block_kv_valid = use_block_cache
                    block_recomputes += 1
                    if use_partial:
                        partial_recomputes += 1
                    bids = ids if use_partial else ids[s0:s1]
                    bp = probs if use_partial else probs[s0:s1]
                    rows = [r for r in local if bp[r] > threshold]
                    if not rows:
                        rows = [local[int(np.argmax([bp[r] for r in local]))]]
                    for r in rows:
                        x_t[a0 + s0 + r] = int(bids[r])
                        unmask_updates += 1
                    log("partial" if use_partial else "full", s0, tuple(rows), tuple(int(bids[r]) for r in rows))
                    if decisions is not None:
                        decisions.append({"kind": "partial" if use_partial else "full", "s0": s0, "masked": local,
                                          "probs": np.asarray(bp, np.float32), "ids": [int(t) for t in bids],
                                          "selected": rows})
                else:
                    _, shifted = score_sequence_block(vm, x_t, block_size=block_size)
                    block_recomputes += 1
                    small = shifted[:, s0:s1, :][0]
                    chosen = small.argmax(axis=-1)
                    cp = np.empty(small.shape[0], dtype=np.float64)
                    for r in range(small.shape[0]):
                        z = small[r].astype(np.float64)
                        e = np.exp(z - z.max())
                        cp[r] = e[chosen[r]] / e.sum()
                    gated = np.full_like(cp, -np.inf, dtype=np.float64)
                    for r in local:
                        gated[r] = cp[r]
                    rows = [r for r in local if gated[r] > threshold]
                    if not rows:
                        rows = [int(np.argmax(gated))]
                    for r in rows:
                        x_t[a0 + s0 + r] = int(chosen[r])
                        unmask_updates += 1
                    log("stateless", s0, tuple(rows), tuple(int(chosen[r]) for r in rows))
                    if decisions is not None:
                        decisions.append({"kind": "stateless", "s0": s0, "masked": local, "probs": cp,
                                          "ids": [int(t) for t in chosen], "selected": rows})
                if len(x_t) - plen0 >= max_new_tokens:
                    break
            if len(x_t) - plen0 >= max_new_tokens:
                break

        generated = x_t
        if len(generated) - plen0 >= max_new_tokens:
            break
        if has_completed_stop(generated, plen0):
            break
        if use_cache and dblk is not None:
            hidden = dblk.forward_full(prefix_cache)
            prefix_cache.commit(block_size)
            nxt = dblk.unmask(hidden, 0, 0, 0).last
            block_kv_valid = False
            if decisions is not None:
                decisions.append({"kind": "append", "token": nxt})
        elif use_cache:
            _, _, nxt, prefix_cache = score_active_block_cached_fast(vm, generated[a0:], prefix_cache)
            block_kv_valid = False
            if decisions is not None:
                decisions.append({"kind": "append", "token": nxt})
        else:
            cur, _ = score_sequence_block(vm, generated, block_size=block_size)
            nxt = int(cur[0, -1, :].argmax())
            if decisions is not None:
                decisions.append({"kind": "append", "token": nxt})
        log("append", prefix_cache.prefix_len if use_cache else 0, nxt)
        block_recomputes += 1
        generated.append(nxt)
        block_appends += 1
        if stop_token is not None and nxt == int(stop_token):
            break

    return make_continuation(generated), stats()


# ---- batched block refinement (a build extension; the reference is batch 1) --------------------------
def batched_shifted_confidence(vm: HipVM, hidden: torch.Tensor) -> tuple[np.ndarray, np.ndarray]:
    """shifted_confidence of each sequence of hidden [nseq, rows, H]: ids / probs [nseq, rows], the shift
    of runtime.py:172-174 applied within each sequence (row 0 keeps its own prediction)."""
    nseq, rows = int(hidden.shape[0]), int(hidden.shape[1])
    both_d = torch.empty((1, 2 * nseq * rows), dtype=torch.int32, device=hidden.device)
    vm.get_confidence(hidden.view(1, nseq * rows, -1), out=both_d)
    both = both_d.cpu().numpy()[0].view(np.float32)
    ids = both[:nseq * rows].view(np.int32).astype(np.int64).reshape(nseq, rows)
    maxp = both[nseq * rows:].astype(np.float32).reshape(nseq, rows)
    return (np.concatenate([ids[:, :1], ids[:, :-1]], axis=1), np.concatenate([maxp[:, :1], maxp[:, :-1]], axis=1))


def batched_shifted_confidence_rows(vm: HipVM, hidden: torch.Tensor, s0: int, s1: int) -> tuple[np.ndarray, np.ndarray]:
    """Columns [s0, s1) of batched_shifted_confidence(vm, hidden), bit for bit, through the lm_head of only
    the rows they read: shifted row i takes logit row i - 1 (row 0 its own), so rows max(s0 - 1, 0) ..
    s1 - 2 of each sequence.  A row's logits and confidence do not depend on the other rows of the call
    (the lm_head never splits k), so the values are the full call's."""
    nseq, rows = int(hidden.shape[0]), int(hidden.shape[1])
    if not 0 <= s0 < s1 <= rows:
        raise ValueError(f"rows [{s0}, {s1}) outside [0, {rows})")
    lo, hi = max(s0 - 1, 0), max(s1 - 1, 1)
    sub = hidden[:, lo:hi].contiguous()
    n = hi - lo
    both_d = torch.empty((1, 2 * nseq * n), dtype=torch.int32, device=hidden.device)
    vm.get_confidence(sub.view(1, nseq * n, -1), out=both_d)
    both = both_d.cpu().numpy()[0].view(np.float32)
    ids = both[:nseq * n].view(np.int32).astype(np.int64).reshape(nseq, n)
    maxp = both[nseq * n:].astype(np.float32).reshape(nseq, n)
    src = [max(i - 1, 0) - lo for i in range(s0, s1)]
    return ids[:, src], maxp[:, src]


def relax_batched_block_refine(vm: HipVM, prompts, *, mask_id: int, block_size: int = 32,
                               small_block_size: int = 8, threshold: float = 0.9, use_block_cache: bool = True,
                               timing: dict | None = None):
    """Refine one block of masks for every sequence of ``prompts`` together, as the batch-1 loop refines
    one block (runtime.py:748-843), with each model call a batched step over all sequences.

    Per sequence the block is laid out as in runtime.py:719-739: x_t = prompt + masks up to the next
    multiple of block_size, prefix = x_t[:a0] with a0 = len(x_t) - block_size (the prompt must reach
    a full block, a0 > 0), built with build_prefix_cache into that sequence's slice of one batched
    cache.  Sub-blocks are refined in order; a step is a partial step at rp = s0 when the block KV is
    valid and every sequence's row s0 is unmasked (the batch-1 condition, runtime.py:765, for all
    sequences at once), else a full 32-row step.  Each sequence takes the threshold rule with the top-1
    fallback (runtime.py:794-805) on its own rows; sequences whose sub-block is complete ride along
    unchanged.  Returns (blocks [nseq][block_size] token ids, stats)."""
    c = vm.cfg
    nseq = len(prompts)
    if nseq == 0:
        raise ValueError("no sequences")
    xs, a0s = [], []
    for p in prompts:
        x_t = [int(t) for t in p]
        x_t += [mask_id] * (block_size - len(x_t) % block_size)
        a0 = len(x_t) - block_size
        if a0 <= 0:
            raise ValueError("every prompt must fill at least one block (the batched path is cached only)")
        xs.append(x_t)
        a0s.append(a0)
    dev = torch.device("cuda")
    t0 = time.perf_counter()
    cap = max(a0s) + block_size
    shape = (c.num_hidden_layers, nseq, cap, c.num_key_value_heads, c.head_dim)
    k = torch.zeros(shape, dtype=vm.torch_dtype, device=dev)
    v = torch.zeros_like(k)
    for b in range(nseq):
        vm.build_prefix_cache_seq(_embed(vm, xs[b][:a0s[b]]), None, k, v, b)
    off_full = torch.tensor(a0s, dtype=torch.int32, device=dev)
    # the partial steps' RoPE offsets, uploaded once (one host-to-device copy per step otherwise)
    off_part = {s0: off_full + s0 for s0 in range(0, block_size, small_block_size)}
    if timing is not None:
        torch.cuda.synchronize()
        timing["prefill_s"] = time.perf_counter() - t0
    t1 = time.perf_counter()
    steps = partial_steps = unmasked = 0
    block_kv_valid = False
    for s0 in range(0, block_size, small_block_size):
        s1 = min(block_size, s0 + small_block_size)
        while True:
            local = [[i for i, t in enumerate(x[a0 + s0:a0 + s1]) if t == mask_id] for x, a0 in zip(xs, a0s)]
            if not any(local):
                break
            use_partial = use_block_cache and block_kv_valid and all(x[a0 + s0] != mask_id for x, a0 in zip(xs, a0s))
            if use_partial:
                ids = [t for x, a0 in zip(xs, a0s) for t in x[a0 + s0:a0 + s1]]
                emb = _embed(vm, ids).view(nseq, s1 - s0, -1)
                hidden = vm.forward_block_partial_batch(s0, emb, k, v, off_part[s0], a0s)
                partial_steps += 1
                sids, sprobs = batched_shifted_confidence(vm, hidden)
            else:
                ids = [t for x, a0 in zip(xs, a0s) for t in x[a0:a0 + block_size]]
                emb = _embed(vm, ids).view(nseq, block_size, -1)
                hidden = vm.forward_cached_batch(emb, k, v, off_full, a0s)
                block_kv_valid = use_block_cache
                # the rule reads the sub-block's rows only: the lm_head runs on the 8 logit rows they take
                sids, sprobs = batched_shifted_confidence_rows(vm, hidden, s0, s1)
            steps += 1
            for b in range(nseq):
                if not local[b]:
                    continue
                bids, bp = sids[b], sprobs[b]
                rows = [r for r in local[b] if bp[r] > threshold]
                if not rows:
                    rows = [local[b][int(np.argmax([bp[r] for r in local[b]]))]]
                for r in rows:
                    xs[b][a0s[b] + s0 + r] = int(bids[r])
                    unmasked += 1
            if steps > 4 * block_size:
                # every step unmasks at least one row per unfinished sequence unless the model predicts
                # the mask token itself
                raise RuntimeError(f"no progress after {steps} steps: the model keeps predicting mask id {mask_id}")
    if timing is not None:
        torch.cuda.synchronize()
        timing["refine_s"] = time.perf_counter() - t1
    stats = {"steps": steps, "partial_steps": partial_steps, "unmasked": unmasked, "nseq": nseq}
    return [x[a0:a0 + block_size] for x, a0 in zip(xs, a0s)], stats
