"""Restatement of the reference's prefix cache and decode loop over ``oracle.model``.  TEST INFRASTRUCTURE ONLY.

Follows ``fast_dllm_relax/runtime.py``:
  PrefixCache / allocate_prefix_cache / _check_write      runtime.py:196-263
  build_prefix_cache_from_ids / _prefill                   runtime.py:266-323
  _forward_cached                                          runtime.py:333-343
  score_active_block_cached_fast / _refine / _partial      runtime.py:346-436
  score_sequence_block                                     runtime.py:439-482
  score_masked_continuation                                runtime.py:485-588
  relax_greedy_generate                                    runtime.py:591-880
The confidence of a cached step is ``oracle.confidence`` (maxp = 1 / sum exp(x - max), metal.py:316-374);
the stateless first block keeps the reference's float64 host formula (runtime.py:820-833).

Pinned by (tests/test_oracle_pinning.py):
  * greedy_generate with the block cache off is token- and trace-identical with a transcription of the
    reference's traced loop, docs/notebooks/_helpers.py:890-1021 (which the reference verified
    token-identical to relax_greedy_generate, 06_runtime_and_decode_loop.ipynb:261), on the cfg1 model
    and on a head_dim-128 model with a peaked lm_head (aligned and unaligned prompts, a stop token);
  * with the block cache on, on the near-uniform cfg1 model, it picks the same tokens as with it off
    (partial rows reproduce full-step rows for identical tokens, runtime.py:762-766);
  * score_masked_continuation equals one dense forward of transformers' Qwen2 over prefix + tail with an
    explicit block mask, shifted (runtime.py:505-515), for aligned and partial prefixes, continuations
    longer than a block, the eos pad and the stateless short branch.
"""

from __future__ import annotations

import dataclasses

import numpy as np

from . import confidence as conf
from .model import OracleModel, build_prefix_block_attention_bias, extract_shifted_block_logits


@dataclasses.dataclass
class PrefixCache:
    k: np.ndarray
    v: np.ndarray
    prefix_len: int

    @property
    def capacity(self) -> int:
        return int(self.k.shape[2])

    def commit(self, rows: int) -> None:
        if self.prefix_len + rows > self.capacity:
            raise ValueError(f"commit past capacity: {self.prefix_len} + {rows} > {self.capacity}")
        self.prefix_len += rows

    def ensure_capacity(self, rows: int) -> None:
        if rows <= self.capacity:
            return
        cap = -(-rows // 32) * 32
        k = np.zeros(self.k.shape[:2] + (cap,) + self.k.shape[3:], np.float32)
        v = np.zeros_like(k)
        k[:, :, :self.prefix_len] = self.k[:, :, :self.prefix_len]
        v[:, :, :self.prefix_len] = self.v[:, :, :self.prefix_len]
        self.k, self.v = k, v


def allocate_prefix_cache(model: OracleModel, rows: int, block_size: int = 32) -> PrefixCache:
    c = model.cfg
    cap = -(-max(int(rows), 1) // block_size) * block_size
    shape = (c.num_hidden_layers, 1, cap, c.num_key_value_heads, c.head_dim)
    return PrefixCache(np.zeros(shape, np.float32), np.zeros(shape, np.float32), 0)


def _check_write(cache: PrefixCache, write_start: int, attend_len: int) -> None:
    if write_start < cache.prefix_len:
        raise ValueError(f"KV write at row {write_start} would overwrite the committed prefix [0, {cache.prefix_len})")
    if attend_len > cache.capacity:
        raise ValueError(f"cached call needs {attend_len} rows; cache capacity is {cache.capacity}")


def build_prefix_cache_from_ids(model: OracleModel, prefix_ids, *, block_size: int, capacity: int | None = None):
    cache = allocate_prefix_cache(model, max(len(prefix_ids), capacity or 0), block_size)
    if prefix_ids:
        _check_write(cache, 0, len(prefix_ids))
        emb = model.embed(prefix_ids)[None]
        bias = build_prefix_block_attention_bias(0, len(prefix_ids), block_size=block_size)
        model.build_prefix_cache(emb, bias, cache.k, cache.v)
        cache.commit(len(prefix_ids))
    return cache


def forward_cached(model: OracleModel, active_ids, cache: PrefixCache) -> np.ndarray:
    _check_write(cache, cache.prefix_len, cache.prefix_len + len(active_ids))
    return model.forward_cached(model.embed(active_ids)[None], cache.k, cache.v, cache.prefix_len, cache.prefix_len)


def shifted_confidence(model: OracleModel, hidden: np.ndarray):
    return conf.shifted_confidence(model.get_logits(hidden)[0])


def score_active_block_cached_fast(model, active_ids, cache):
    hidden = forward_cached(model, active_ids, cache)
    cache.commit(len(active_ids))
    ids, p, last = shifted_confidence(model, hidden)
    return ids, p, last, cache


def score_active_block_refine(model, active_ids, cache):
    ids, p, _ = shifted_confidence(model, forward_cached(model, active_ids, cache))
    return ids, p


def score_active_block_partial_perlayer(model, small_ids, cache, replace_position, *, block_size):
    ws = cache.prefix_len + replace_position
    _check_write(cache, ws, cache.prefix_len + block_size)
    hidden = model.forward_block_partial(replace_position, model.embed(small_ids)[None], cache.k, cache.v, ws,
                                         cache.prefix_len)
    ids, p, _ = shifted_confidence(model, hidden)
    return ids, p


def score_sequence_block(model, sequence_ids, *, block_size):
    if len(sequence_ids) <= block_size:
        prefix_ids, active = [], list(sequence_ids)
    else:
        plen = ((len(sequence_ids) - 1) // block_size) * block_size
        prefix_ids, active = list(sequence_ids[:plen]), list(sequence_ids[plen:])
    bias = build_prefix_block_attention_bias(len(prefix_ids), len(active), block_size=block_size)
    hidden = model.forward_hidden(model.embed(prefix_ids + active)[None], bias)
    logits = model.get_logits(hidden)
    cur = logits[:, -len(active):, :]
    shifted = extract_shifted_block_logits(logits, prefix_len=len(prefix_ids), block_len=len(active))
    return cur, shifted


def score_masked_continuation(model, prefix_ids, continuation_ids, *, block_size, mask_id, eos_token_id=None):
    """runtime.py:485-588 (without the cross-call memo, which does not change the result)."""
    if not continuation_ids:
        return np.empty((0, 0), np.float32)
    pcl = (len(prefix_ids) // block_size) * block_size
    if pcl == 0:
        seq = list(prefix_ids) + [mask_id] * len(continuation_ids)
        _, shifted = score_sequence_block(model, seq, block_size=block_size)
        return shifted[0, -len(continuation_ids):, :]
    tail_rows = max(len(prefix_ids) - pcl + len(continuation_ids), block_size)
    cache = build_prefix_cache_from_ids(model, list(prefix_ids[:pcl]), block_size=block_size, capacity=pcl + tail_rows)
    real = list(prefix_ids[cache.prefix_len:])
    active = real + [mask_id] * len(continuation_ids)
    if len(active) <= block_size:
        pad = block_size - len(active)
        if pad:
            active = active + [mask_id] * pad
            if eos_token_id is not None:
                active[len(real) + len(continuation_ids)] = eos_token_id
    hidden = forward_cached(model, active, cache)
    logits = model.get_logits(hidden)
    shifted = np.concatenate([logits[:, :1], logits[:, :-1]], axis=1)
    return shifted[0, len(real):len(real) + len(continuation_ids)]


def greedy_generate(model: OracleModel, prompt_ids, *, max_new_tokens: int, block_size: int = 32,
                    small_block_size: int = 8, threshold: float = 0.9, use_block_cache: bool = True,
                    mask_id: int, stop_token: int | None, trace: list | None = None, decisions: list | None = None):
    """relax_greedy_generate (runtime.py:591-880), temperature 0.  ``trace`` collects one tuple per call;
    ``decisions`` (optional) one dict per refinement step (cached or stateless): the sub-block's masked
    rows, shifted probabilities (float64 on the stateless path) and ids, the selected rows, and each row's
    gap between its two largest logits; and one per block append after the first call."""
    generated = list(prompt_ids)
    plen0 = len(generated)
    stats = dict(unmask_updates=0, block_recomputes=0, partial_recomputes=0, block_appends=0)
    cache = None
    block_kv_valid = False
    capacity = -(-(plen0 + max_new_tokens) // block_size) * block_size + block_size

    def stop_done(seq, plen):
        if stop_token is None:
            return False
        suffix = seq[plen:]
        if stop_token not in suffix:
            return False
        return mask_id not in suffix[:suffix.index(stop_token)]

    def cont(tokens):
        raw = tokens[plen0:plen0 + max_new_tokens]
        first = next((i for i, t in enumerate(raw) if t == mask_id), len(raw))
        return raw[:first]

    def log(*item):
        if trace is not None:
            trace.append(item)

    if plen0 % block_size == 0 and plen0 > 0 and max_new_tokens > 0:
        cache = build_prefix_cache_from_ids(model, generated[:plen0 - block_size], block_size=block_size,
                                            capacity=capacity)
        _, _, nxt, cache = score_active_block_cached_fast(model, generated[plen0 - block_size:], cache)
        log("append", cache.prefix_len, nxt)
        stats["block_recomputes"] += 1
        stats["block_appends"] += 1
        generated.append(nxt)
        if stop_token is not None and nxt == int(stop_token):
            return cont(generated), stats

    while len(generated) - plen0 < max_new_tokens:
        plen = len(generated)
        x_t = generated + [mask_id] * (block_size - plen % block_size)
        a0 = len(x_t) - block_size
        if a0 == 0:
            use_cache = False
        else:
            use_cache = True
            if a0 != (cache.prefix_len if cache is not None else 0):
                cache = build_prefix_cache_from_ids(model, x_t[:a0], block_size=block_size, capacity=capacity)
                block_kv_valid = False
        for s0 in range(0, block_size, small_block_size):
            s1 = min(block_size, s0 + small_block_size)
            while True:
                local = [i for i, t in enumerate(x_t[a0 + s0:a0 + s1]) if t == mask_id]
                if not local:
                    break
                if stop_done(x_t, plen):
                    return cont(x_t), stats
                if use_cache:
                    use_partial = use_block_cache and block_kv_valid and x_t[a0 + s0] != mask_id
                    if use_partial:
                        ws = cache.prefix_len + s0
                        _check_write(cache, ws, cache.prefix_len + block_size)
                        hidden = model.forward_block_partial(s0, model.embed(x_t[a0 + s0:a0 + s1])[None], cache.k,
                                                             cache.v, ws, cache.prefix_len)
                    else:
                        hidden = forward_cached(model, x_t[a0:], cache)
                        block_kv_valid = use_block_cache
                    logits = model.get_logits(hidden)[0]
                    ids, probs, _ = conf.shifted_confidence(logits)
                    stats["block_recomputes"] += 1
                    if use_partial:
                        stats["partial_recomputes"] += 1
                    bids = ids if use_partial else ids[s0:s1]
                    bp = probs if use_partial else probs[s0:s1]
                    rows = [r for r in local if bp[r] > threshold]
                    if not rows:
                        rows = [local[int(np.argmax([bp[r] for r in local]))]]
                    for r in rows:
                        x_t[a0 + s0 + r] = int(bids[r])
                        stats["unmask_updates"] += 1
                    log("partial" if use_partial else "full", s0, tuple(rows), tuple(int(bids[r]) for r in rows))
                    if decisions is not None:
                        sh = np.concatenate([logits[:1], logits[:-1]])[(0 if use_partial else s0):][:s1 - s0]
                        top2 = np.sort(sh, axis=-1)[:, -2:]
                        decisions.append({"kind": "partial" if use_partial else "full", "s0": s0, "masked": local,
                                          "probs": np.asarray(bp, np.float32), "ids": [int(t) for t in bids],
                                          "selected": rows, "gap": top2[:, 1] - top2[:, 0]})
                else:
                    _, shifted = score_sequence_block(model, x_t, block_size=block_size)
                    stats["block_recomputes"] += 1
                    small = shifted[:, s0:s1, :][0]
                    chosen = small.argmax(axis=-1)
                    cp = np.empty(small.shape[0], np.float64)
                    for r in range(small.shape[0]):
                        z = small[r].astype(np.float64)
                        e = np.exp(z - z.max())
                        cp[r] = e[chosen[r]] / e.sum()
                    gated = np.full_like(cp, -np.inf)
                    for r in local:
                        gated[r] = cp[r]
                    rows = [r for r in local if gated[r] > threshold]
                    if not rows:
                        rows = [int(np.argmax(gated))]
                    for r in rows:
                        x_t[a0 + s0 + r] = int(chosen[r])
                        stats["unmask_updates"] += 1
                    log("stateless", s0, tuple(rows), tuple(int(chosen[r]) for r in rows))
                    if decisions is not None:
                        top2 = np.sort(small, axis=-1)[:, -2:]
                        decisions.append({"kind": "stateless", "s0": s0, "masked": local, "probs": cp,
                                          "ids": [int(t) for t in chosen], "selected": rows,
                                          "gap": top2[:, 1] - top2[:, 0]})
                if len(x_t) - plen0 >= max_new_tokens:
                    break
            if len(x_t) - plen0 >= max_new_tokens:
                break
        generated = x_t
        if len(generated) - plen0 >= max_new_tokens or stop_done(generated, plen0):
            break
        if use_cache:
            hidden = forward_cached(model, generated[a0:], cache)
            cache.commit(len(generated[a0:]))
            last = model.get_logits(hidden)[0, -1]
            nxt = int(np.argmax(last))
            block_kv_valid = False
            if decisions is not None:
                top2 = np.sort(last)[-2:]
                decisions.append({"kind": "append", "token": nxt, "gap": float(top2[1] - top2[0])})
        else:
            cur, _ = score_sequence_block(model, generated, block_size=block_size)
            nxt = int(cur[0, -1, :].argmax())
            if decisions is not None:
                top2 = np.sort(cur[0, -1, :])[-2:]
                decisions.append({"kind": "append", "token": nxt, "gap": float(top2[1] - top2[0])})
        log("append", cache.prefix_len if use_cache else 0, nxt)
        stats["block_recomputes"] += 1
        generated.append(nxt)
        stats["block_appends"] += 1
        if stop_token is not None and nxt == int(stop_token):
            break
    return cont(generated), stats
