"""Pins the CPU oracle to checks independent of its own formulas (CPU only).

* the local ``transformers`` Qwen2 implementation (an independent restatement of the architecture the
  reference's model/cuda.py follows) on the same weights, in fp32: dense block-causal forward and a
  cached block step against a DynamicCache prefix;
* the reference's own invariants (tests/test_tiny_compile.py:264-290): cached rows equal the dense
  block-causal rows, and each partial rp step equals the full step's rows for the same tokens;
* closed forms: RoPE at position 0 is the identity, preserves norms and makes q.k depend only on the
  position difference; RMSNorm with unit weights has unit RMS; torch's GQA scaled_dot_product_attention;
* the confidence / unmask rules against float64 softmax, numpy argmax and a brute-force restatement of
  runtime.py:794-805.
A planted mistake in the oracle (a dropped bias, a wrong RoPE sign, a transposed projection, the wrong
KV head for a query head, a shift in the wrong direction) fails at least one of these.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import confidence as oconf
from oracle.model import (OracleConfig, OracleModel, build_prefix_block_attention_bias, extract_shifted_block_logits,
                          random_params)
from oracle.runtime import greedy_generate

CFG1 = dict(vocab_size=512, hidden_size=64, intermediate_size=128, num_hidden_layers=2, num_attention_heads=4,
            num_key_value_heads=2, head_dim=16)


@pytest.fixture(scope="module")
def tiny32():
    cfg = OracleConfig(**CFG1)
    arrays = random_params(cfg, 0, "float32")
    return cfg, arrays, OracleModel(cfg, arrays, "float32")


def _hf_model(cfg: OracleConfig, arrays):
    from transformers import Qwen2Config, Qwen2ForCausalLM

    hc = Qwen2Config(vocab_size=cfg.vocab_size, hidden_size=cfg.hidden_size, intermediate_size=cfg.intermediate_size,
                     num_hidden_layers=cfg.num_hidden_layers, num_attention_heads=cfg.num_attention_heads,
                     num_key_value_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim, rms_norm_eps=cfg.rms_norm_eps,
                     rope_theta=cfg.rope_theta, tie_word_embeddings=cfg.tie_word_embeddings, max_position_embeddings=4096,
                     attn_implementation="eager")
    model = Qwen2ForCausalLM(hc).eval()
    qd, kd, inter = cfg.num_attention_heads * cfg.head_dim, cfg.num_key_value_heads * cfg.head_dim, cfg.intermediate_size
    sd = {"model.embed_tokens.weight": arrays["model.embed_tokens.weight"], "model.norm.weight": arrays["model.norm.weight"]}
    if not cfg.tie_word_embeddings:
        sd["lm_head.weight"] = arrays["lm_head.weight"]
    for i in range(cfg.num_hidden_layers):
        p = f"model.layers.{i}"
        w, b = arrays[f"{p}.self_attn.qkv_proj.weight"], arrays[f"{p}.self_attn.qkv_proj.bias"]
        sd[f"{p}.self_attn.q_proj.weight"], sd[f"{p}.self_attn.q_proj.bias"] = w[:qd], b[:qd]
        sd[f"{p}.self_attn.k_proj.weight"], sd[f"{p}.self_attn.k_proj.bias"] = w[qd:qd + kd], b[qd:qd + kd]
        sd[f"{p}.self_attn.v_proj.weight"], sd[f"{p}.self_attn.v_proj.bias"] = w[qd + kd:], b[qd + kd:]
        sd[f"{p}.self_attn.o_proj.weight"] = arrays[f"{p}.self_attn.o_proj.weight"]
        gu = arrays[f"{p}.mlp.gate_up_proj.weight"]
        sd[f"{p}.mlp.gate_proj.weight"], sd[f"{p}.mlp.up_proj.weight"] = gu[:inter], gu[inter:]
        sd[f"{p}.mlp.down_proj.weight"] = arrays[f"{p}.mlp.down_proj.weight"]
        sd[f"{p}.input_layernorm.weight"] = arrays[f"{p}.input_layernorm.weight"]
        sd[f"{p}.post_attention_layernorm.weight"] = arrays[f"{p}.post_attention_layernorm.weight"]
    missing, unexpected = model.load_state_dict({k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in sd.items()},
                                                strict=False)
    assert not unexpected and set(missing) <= {"lm_head.weight"}
    return model


def test_dense_forward_matches_transformers_qwen2(tiny32):
    cfg, arrays, model = tiny32
    hf = _hf_model(cfg, arrays)
    ids = np.random.default_rng(0).integers(0, 510, 48)
    bias = build_prefix_block_attention_bias(0, 48, block_size=32)
    logits = model.get_logits(model.forward_hidden(model.embed(ids)[None], bias))
    with torch.no_grad():
        want = hf(input_ids=torch.from_numpy(ids)[None], attention_mask={"full_attention": torch.from_numpy(bias)},
                  position_ids=torch.arange(48)[None]).logits.numpy()
    # RoPE inverse frequencies differ by formula (exp(-ln theta * i / 64) vs theta^(-2i/d)) at fp32 rounding
    np.testing.assert_allclose(logits, want, rtol=0, atol=1e-5)


def test_cached_step_matches_transformers_dynamic_cache(tiny32):
    from transformers import DynamicCache

    cfg, arrays, model = tiny32
    hf = _hf_model(cfg, arrays)
    P, R = 32, 32
    ids = np.random.default_rng(1).integers(0, 510, P + R)
    kc = np.zeros((cfg.num_hidden_layers, 1, P + R, cfg.num_key_value_heads, cfg.head_dim), np.float32)
    vc = np.zeros_like(kc)
    model.build_prefix_cache(model.embed(ids[:P])[None], build_prefix_block_attention_bias(0, P, block_size=32), kc, vc)
    got = model.get_logits(model.forward_cached(model.embed(ids[P:])[None], kc, vc, P, P))
    with torch.no_grad():
        cache = DynamicCache()
        pre_bias = torch.from_numpy(build_prefix_block_attention_bias(0, P, block_size=32))
        hf(input_ids=torch.from_numpy(ids[:P])[None], attention_mask={"full_attention": pre_bias},
           position_ids=torch.arange(P)[None], past_key_values=cache, use_cache=True)
        # the cached block sees the whole prefix and the whole block: an all-zero additive mask
        want = hf(input_ids=torch.from_numpy(ids[P:])[None],
                  attention_mask={"full_attention": torch.zeros((1, 1, R, P + R))},
                  position_ids=torch.arange(P, P + R)[None], past_key_values=cache, use_cache=True).logits.numpy()
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-5)


def test_cached_rows_equal_dense_block_causal_rows(tiny32):
    """tests/test_tiny_compile.py:264-290, in fp32 (where the two paths agree to rounding)."""
    cfg, _, model = tiny32
    P, R = 64, 32
    ids = np.random.default_rng(2).integers(0, 510, P + R)
    dense = model.forward_hidden(model.embed(ids)[None], build_prefix_block_attention_bias(0, P + R, block_size=32))
    kc = np.zeros((cfg.num_hidden_layers, 1, P + R, cfg.num_key_value_heads, cfg.head_dim), np.float32)
    vc = np.zeros_like(kc)
    model.build_prefix_cache(model.embed(ids[:P])[None], build_prefix_block_attention_bias(0, P, block_size=32), kc, vc)
    cached = model.forward_cached(model.embed(ids[P:])[None], kc, vc, P, P)
    np.testing.assert_allclose(cached, dense[:, P:], rtol=0, atol=2e-6)
    for rp in (0, 8, 16, 24):
        part = model.forward_block_partial(rp, model.embed(ids[P + rp:P + rp + 8])[None], kc, vc, P + rp, P)
        np.testing.assert_allclose(part, cached[:, rp:rp + 8], rtol=0, atol=2e-6)


def test_rope_closed_forms(tiny32):
    cfg, _, model = tiny32
    rng = np.random.default_rng(3)
    x = rng.standard_normal((1, 2, cfg.head_dim)).astype(np.float32)
    cos, sin = model.rope_tables(1, 0)
    np.testing.assert_array_equal(model.apply_rope(x, cos, sin), x)  # position 0: identity
    cos, sin = model.rope_tables(1, 777)
    y = model.apply_rope(x, cos, sin)
    np.testing.assert_allclose(np.linalg.norm(y, axis=-1), np.linalg.norm(x, axis=-1), rtol=1e-5)
    # q(m).k(n) depends on m - n only, and the rotation direction matters (a sign flip breaks this)
    q, k = rng.standard_normal((2, 1, 1, cfg.head_dim)).astype(np.float32)

    def dot(m, n):
        cm, sm = model.rope_tables(1, m)
        cn, sn = model.rope_tables(1, n)
        return float((model.apply_rope(q, cm, sm) * model.apply_rope(k, cn, sn)).sum())

    assert abs(dot(10, 3) - dot(107, 100)) < 1e-4
    # against the textbook rotation with theta^(-2i/d) frequencies
    m = 5
    half = cfg.head_dim // 2
    inv = cfg.rope_theta ** (-np.arange(half, dtype=np.float64) * 2 / cfg.head_dim)
    ang = m * inv
    x1, x2 = x[0, 0, :half].astype(np.float64), x[0, 0, half:].astype(np.float64)
    want = np.concatenate([x1 * np.cos(ang) - x2 * np.sin(ang), x2 * np.cos(ang) + x1 * np.sin(ang)])
    cos, sin = model.rope_tables(1, m)
    np.testing.assert_allclose(model.apply_rope(x[:, :1], cos, sin)[0, 0], want, rtol=0, atol=2e-5)


def test_rmsnorm_unit_rms(tiny32):
    cfg, _, model = tiny32
    x = np.random.default_rng(4).standard_normal((5, cfg.hidden_size)).astype(np.float32) * 3
    y = model.rmsnorm(x, np.ones(cfg.hidden_size, np.float32))
    np.testing.assert_allclose(np.sqrt(np.mean(y.astype(np.float64) ** 2, axis=-1)), 1.0, rtol=1e-5)


def test_attention_matches_torch_sdpa_gqa(tiny32):
    cfg, _, model = tiny32
    rng = np.random.default_rng(5)
    n, m = 7, 19
    q = rng.standard_normal((n, cfg.num_attention_heads, cfg.head_dim)).astype(np.float32)
    k = rng.standard_normal((m, cfg.num_key_value_heads, cfg.head_dim)).astype(np.float32)
    v = rng.standard_normal((m, cfg.num_key_value_heads, cfg.head_dim)).astype(np.float32)
    got = model.attend(q, k, v)
    want = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q).transpose(0, 1)[None], torch.from_numpy(k).transpose(0, 1)[None],
        torch.from_numpy(v).transpose(0, 1)[None], enable_gqa=True)[0].transpose(0, 1).numpy()
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-6)


def _torch_callbacks(q, k, v, kc, vc, layer, prefix_len, write_rel, attend_rel):
    """fast_dllm.attn_inplace's body (runtime.py:51-73) on torch tensors: torch's slice-assignment for the
    write, torch's slice for the attended rows and torch's SDPA with GQA (the reference's fallback
    _attend, runtime.py:38-48)."""
    kc, vc = torch.from_numpy(kc.copy()), torch.from_numpy(vc.copy())
    start, attend_len, rows = prefix_len + write_rel, prefix_len + attend_rel, k.shape[1]
    kc[layer, :, start:start + rows].copy_(torch.from_numpy(k))
    vc[layer, :, start:start + rows].copy_(torch.from_numpy(v))
    out = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q).transpose(1, 2), kc[layer, :, :attend_len].transpose(1, 2),
        vc[layer, :, :attend_len].transpose(1, 2), enable_gqa=True).transpose(1, 2)
    return kc.numpy(), vc.numpy(), out.numpy()


@pytest.mark.parametrize("rows,P,write_rel,attend_rel,cap", [
    (8, 40, 0, 8, 64), (8, 40, 16, 32, 96), (5, 10, 3, 9, 32),
    (8, 40, 0, 30, 56),  # attended rows past the capacity: the slice stops at 56
])
def test_attn_callbacks_against_torch(tiny32, rows, P, write_rel, attend_rel, cap):
    cfg, _, model = tiny32
    rng = np.random.default_rng(rows * 100 + P)
    q = rng.standard_normal((1, rows, cfg.num_attention_heads, cfg.head_dim)).astype(np.float32)
    k, v = rng.standard_normal((2, 1, rows, cfg.num_key_value_heads, cfg.head_dim)).astype(np.float32)
    shape = (cfg.num_hidden_layers, 1, cap, cfg.num_key_value_heads, cfg.head_dim)
    kc, vc = rng.standard_normal((2,) + shape).astype(np.float32)
    want_k, want_v, want = _torch_callbacks(q, k, v, kc, vc, 1, P, write_rel, attend_rel)
    got_k, got_v, got = model.attn_inplace(q, k, v, kc, vc, 1, P, write_rel, attend_rel)
    assert got_k is kc and got_v is vc  # written in place, returned as aliases
    np.testing.assert_array_equal(kc, want_k)
    np.testing.assert_array_equal(vc, want_v)
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-6)


def test_attn_callback_errors(tiny32):
    cfg, _, model = tiny32
    k = np.zeros((1, 8, cfg.num_key_value_heads, cfg.head_dim), np.float32)
    q = np.zeros((1, 8, cfg.num_attention_heads, cfg.head_dim), np.float32)
    kc = np.zeros((cfg.num_hidden_layers, 1, 32, cfg.num_key_value_heads, cfg.head_dim), np.float32)
    vc = kc.copy()
    # the reference's messages (runtime.py:56-57, 69-70)
    with pytest.raises(ValueError, match=r"^KV write \[20, 28\) past the attended rows \[0, 24\)$"):
        model.attn_inplace(q, k, k, kc, vc, 0, 16, 4, 8)
    with pytest.raises(ValueError, match=r"^KV write \[28, 36\) outside cache capacity 32$"):
        model.attn_inplace(q, k, k, kc, vc, 0, 24, 4, 12)
    with pytest.raises(ValueError, match=r"^KV write \[-2, 6\) outside cache capacity 32$"):
        model.kv_write(k, k, kc, vc, 0, -2)
    assert not kc.any()


def test_shift_and_block_bias_closed_forms():
    bias = build_prefix_block_attention_bias(0, 96, block_size=32)[0, 0]
    q, k = np.meshgrid(np.arange(96), np.arange(96), indexing="ij")
    np.testing.assert_array_equal(bias == 0, (q // 32) >= (k // 32))
    logits = np.arange(2 * 6 * 3, dtype=np.float32).reshape(1, 6, 6)[:, :, :3]
    sh = extract_shifted_block_logits(logits, prefix_len=2, block_len=4)
    np.testing.assert_array_equal(sh[0], logits[0, [1, 2, 3, 4]])
    sh0 = extract_shifted_block_logits(logits, prefix_len=0, block_len=4)
    np.testing.assert_array_equal(sh0[0], logits[0, [0, 0, 1, 2]])


def test_exp_within_two_ulp_of_float64():
    x = np.concatenate([-np.logspace(-8, math.log10(86.0), 2000), [0.0, -1e-30, -85.99]]).astype(np.float32)
    got = oconf.exp_neg_array(x).astype(np.float64)
    want = np.exp(x.astype(np.float64))
    ulp = np.spacing(want.astype(np.float32)).astype(np.float64)
    assert np.max(np.abs(got - want) / ulp) <= 2.0
    assert oconf.exp_neg(-87.0) == 0.0


@pytest.mark.parametrize("scale", [0.01, 1.0, 20.0])
def test_confidence_against_float64_softmax(scale):
    rng = np.random.default_rng(7)
    rows, vocab = 9, 151936
    x = (scale * rng.standard_normal((rows, vocab))).astype(np.float32)
    x[3, 5] = x[3, 100000] = x[3].max() + 1  # tie: the first index wins
    ids, maxp = oconf.confidence(x)
    np.testing.assert_array_equal(ids, np.argmax(x, axis=-1))
    z = x.astype(np.float64)
    p = np.exp(z - z.max(-1, keepdims=True))
    np.testing.assert_allclose(maxp, p.max(-1) / p.sum(-1), rtol=2e-6)


def test_unmask_rule_brute_force():
    rng = np.random.default_rng(8)
    for _ in range(2000):
        n = int(rng.integers(1, 9))
        p = rng.random(n).astype(np.float32)
        if rng.random() < 0.3:
            p[rng.integers(0, n)] = np.float32(0.9)  # exactly at the threshold: not selected
        masked = rng.random(n) < 0.6
        got = oconf.unmask(p, masked, 0.9)
        local = [i for i in range(n) if masked[i]]
        rows = [r for r in local if p[r] > 0.9]
        if not rows and local:
            rows = [local[int(np.argmax([p[r] for r in local]))]]
        want = np.zeros(n, bool)
        want[rows] = True
        np.testing.assert_array_equal(got, want)


def test_decode_loop_block_cache_on_off_agree(tiny32):
    """In fp32 the partial (block-cache) steps reproduce the full steps' rows, so the decode loop must
    pick the same tokens with the block cache on or off (runtime.py:762-766)."""
    cfg, _, model = tiny32
    prompt = list(np.random.default_rng(9).integers(0, 510, 40))
    common = dict(max_new_tokens=40, block_size=32, small_block_size=8, threshold=0.9, mask_id=511, stop_token=None)
    on, st_on = greedy_generate(model, prompt, use_block_cache=True, **common)
    off, st_off = greedy_generate(model, prompt, use_block_cache=False, **common)
    # random weights may predict the mask id itself; the continuation then ends at it (runtime.py make_continuation)
    assert on == off and len(on) > 0 and 511 not in on
    assert st_on["partial_recomputes"] > 0 and st_off["partial_recomputes"] == 0
    assert st_on["unmask_updates"] == st_off["unmask_updates"]


# ---- the decode loop, against a transcription of the reference's own traced restatement ----------------
HD128_F32 = dict(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
                 num_key_value_heads=2, head_dim=128, tie_word_embeddings=False)


def _traced_generate(model, prompt_ids, *, max_new_tokens, bs=32, sbs=8, thr=0.9, mask_id, stop=None):
    """Control flow of ``relax_traced_generate`` (docs/notebooks/_helpers.py:890-1021; block cache off),
    which the reference verified token-identical to relax_greedy_generate (06_runtime_and_decode_loop.ipynb:261).

    Written from the helper, not from oracle.runtime.greedy_generate: it shares only the oracle's step
    functions (each pinned above against transformers and the reference's invariants).  Returns
    (continuation, events) with events ("prefill", cache_len) / ("full"|"stateless", s0, rows, tokens) /
    ("append", cache_len, token)."""
    import oracle.runtime as rt

    gen = list(prompt_ids)
    n0 = len(gen)
    cap = -(-(n0 + max_new_tokens) // bs) * bs + bs
    pc = None
    ev = []

    def finished(seq, plen):
        tail = seq[plen:]
        if stop is None or stop not in tail:
            return False
        return mask_id not in tail[:tail.index(stop)]

    def continuation(toks):
        raw = toks[n0:n0 + max_new_tokens]
        cut = next((i for i, t in enumerate(raw) if t == mask_id), len(raw))
        return raw[:cut]

    if n0 % bs == 0 and max_new_tokens > 0:
        pc = rt.build_prefix_cache_from_ids(model, gen[:n0 - bs], block_size=bs, capacity=cap)
        ev.append(("prefill", pc.prefix_len))
        _, _, nxt, pc = rt.score_active_block_cached_fast(model, gen[n0 - bs:], pc)
        gen.append(nxt)
        ev.append(("append", pc.prefix_len, nxt))
        if stop is not None and nxt == stop:
            return continuation(gen), ev
    while len(gen) - n0 < max_new_tokens:
        plen = len(gen)
        x = gen + [mask_id] * (bs - plen % bs)
        a0 = len(x) - bs
        cached = a0 != 0
        if cached and (pc is None or pc.prefix_len != a0):
            pc = rt.build_prefix_cache_from_ids(model, x[:a0], block_size=bs, capacity=cap)
            ev.append(("prefill", pc.prefix_len))
        for s0 in range(0, bs, sbs):
            s1 = min(bs, s0 + sbs)
            while True:
                masked = [i for i, t in enumerate(x[a0 + s0:a0 + s1]) if t == mask_id]
                if not masked:
                    break
                if finished(x, plen):
                    return continuation(x), ev
                if cached:
                    ids, p = rt.score_active_block_refine(model, x[a0:], pc)
                    blk_ids, blk_p = ids[s0:s1], p[s0:s1]
                    pick = [r for r in masked if blk_p[r] > thr] or [masked[int(np.argmax([blk_p[r] for r in masked]))]]
                    kind = "full"
                else:
                    _, shifted = rt.score_sequence_block(model, x, block_size=bs)
                    small = shifted[0, s0:s1, :]
                    blk_ids = small.argmax(axis=-1)
                    blk_p = np.empty(small.shape[0], np.float64)
                    for r in range(small.shape[0]):
                        z = small[r].astype(np.float64)
                        e = np.exp(z - z.max())
                        blk_p[r] = e[blk_ids[r]] / e.sum()
                    gated = np.full_like(blk_p, -np.inf)
                    gated[masked] = blk_p[masked]
                    pick = [r for r in masked if gated[r] > thr] or [int(np.argmax(gated))]
                    kind = "stateless"
                for r in pick:
                    x[a0 + s0 + r] = int(blk_ids[r])
                ev.append((kind, s0, tuple(pick), tuple(int(blk_ids[r]) for r in pick)))
                if len(x) - n0 >= max_new_tokens:
                    break
            if len(x) - n0 >= max_new_tokens:
                break
        gen = x
        if len(gen) - n0 >= max_new_tokens or finished(gen, n0):
            break
        if cached:
            _, _, nxt, pc = rt.score_active_block_cached_fast(model, gen[a0:], pc)
        else:
            cur, _ = rt.score_sequence_block(model, gen, block_size=bs)
            nxt = int(cur[0, -1, :].argmax())
        gen.append(nxt)
        ev.append(("append", pc.prefix_len if cached else 0, nxt))
        if stop is not None and nxt == stop:
            break
    return continuation(gen), ev


@pytest.fixture(scope="module")
def hd128_peaked():
    """A head_dim-128 fp32 model with an untied, peaked lm_head: N(0, 1.25) at hidden 256 gives logits of
    std ~20, as BASELINE cfg3's N(0, 0.5) head does at hidden 1536, so several rows per sub-block cross
    the 0.9 threshold."""
    cfg = OracleConfig(**HD128_F32)
    return OracleModel(cfg, random_params(cfg, 11, "float32", lm_head_std=1.25), "float32")


@pytest.mark.parametrize("case", ["cfg1_unaligned", "hd128_aligned", "hd128_unaligned", "hd128_stop"])
def test_decode_loop_matches_reference_transcription(case, tiny32, hd128_peaked):
    """oracle.runtime.greedy_generate (block cache off) is token- and trace-identical with the
    transcription of the reference's traced loop: same calls in the same order, same unmasked rows and
    tokens, same appends."""
    if case == "cfg1_unaligned":
        model, prompt, new, mask, stop = tiny32[2], list(np.random.default_rng(0).integers(0, 510, 16)), 80, 511, None
    else:
        model, mask = hd128_peaked, 511
        n = 64 if case == "hd128_aligned" else 40
        prompt = list(np.random.default_rng(12).integers(0, 510, n))
        new, stop = 72, None
    if case == "hd128_stop":
        # a stop token the loop is known to produce: the first appended token of the unaligned run
        _, ev0 = _traced_generate(model, prompt, max_new_tokens=new, mask_id=mask)
        stop = next(e[2] for e in ev0 if e[0] == "append")
    want_tokens, want_ev = _traced_generate(model, prompt, max_new_tokens=new, mask_id=mask, stop=stop)
    trace: list = []
    got_tokens, stats = greedy_generate(model, prompt, max_new_tokens=new, block_size=32, small_block_size=8,
                                        threshold=0.9, use_block_cache=False, mask_id=mask, stop_token=stop,
                                        trace=trace)
    assert got_tokens == want_tokens
    assert trace == [e for e in want_ev if e[0] != "prefill"]
    assert stats["unmask_updates"] == sum(len(e[2]) for e in trace if e[0] != "append")
    assert stats["block_appends"] == sum(e[0] == "append" for e in trace)
    if case != "cfg1_unaligned":
        # the regime the test is for: the threshold rule, not only its top-1 fallback, picks rows
        assert any(e[0] != "append" and len(e[2]) > 1 for e in trace), trace
    if case == "hd128_stop":
        assert got_tokens and got_tokens[-1] == stop or stop in got_tokens


# ---- masked-continuation scoring: cached scoring equals a dense forward (runtime.py:505-515) -------------
def _hf_dense_logits(hf, ids, allowed):
    bias = np.where(allowed, 0.0, -1e9).astype(np.float32)[None, None]
    with torch.no_grad():
        return hf(input_ids=torch.from_numpy(np.asarray(ids, np.int64))[None],
                  attention_mask={"full_attention": torch.from_numpy(bias)},
                  position_ids=torch.arange(len(ids))[None]).logits.numpy()[0]


@pytest.mark.parametrize("plen,clen,eos", [(70, 40, None), (64, 10, None), (45, 5, 7), (64, 32, None), (10, 12, None)])
def test_masked_continuation_equals_dense_forward(hd128_peaked, plen, clen, eos):
    """score_masked_continuation scores the tail (context remainder + masked continuation, padded to a
    block) with forward_cached over the block-aligned prefix cache.  The same logits come from one dense
    forward of transformers' Qwen2 over prefix + tail with an explicit mask: prefix rows block-causal in
    blocks of 32, tail rows attending to every prefix row and every tail row; the token at tail row t is
    read from logits row t - 1 (row 0 from itself).  Covers a partial last prefix block, a continuation
    longer than one block (the tail is not padded and attends as one window), the eos pad and the short
    stateless branch (prefix shorter than a block)."""
    from oracle.runtime import score_masked_continuation

    model = hd128_peaked
    hf = _hf_model(model.cfg, model.p)
    rng = np.random.default_rng(100 + plen + clen)
    prefix = [int(t) for t in rng.integers(0, 510, plen)]
    cont = [int(t) for t in rng.integers(0, 510, clen)]
    got = score_masked_continuation(model, prefix, cont, block_size=32, mask_id=511, eos_token_id=eos)
    assert got.shape == (clen, model.cfg.vocab_size)
    pcl = plen // 32 * 32
    real = prefix[pcl:]
    tail = real + [511] * clen
    if pcl and len(tail) < 32:
        tail = tail + [511] * (32 - len(tail))
        if eos is not None:
            tail[len(real) + clen] = eos
    seq = prefix[:pcl] + tail
    T = len(seq)
    q, k = np.meshgrid(np.arange(T), np.arange(T), indexing="ij")
    if pcl:
        allowed = np.where(q < pcl, (k < pcl) & (q // 32 >= k // 32), True)
    else:
        allowed = q // 32 >= k // 32  # the stateless branch: plain block-causal over the sequence
    L = _hf_dense_logits(hf, seq, allowed)[pcl:]
    want = np.stack([L[max(len(real) + j - 1, 0)] for j in range(clen)])
    # fp32 rounding of two implementations (RoPE frequency formulas differ, see above) at logits of
    # magnitude ~80; a wrong shift, row or mask moves logits by their spread (~20)
    np.testing.assert_allclose(got, want, rtol=0, atol=4e-6 * float(np.abs(want).max()))
