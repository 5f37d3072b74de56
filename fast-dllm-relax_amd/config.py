"""Model constants and decode defaults.

``FastDLLMConfig`` mirrors FastDLLMRelaxConfig (fast_dllm_relax/model/cuda.py:15-29); the decode
defaults are the reference's (fast_dllm_relax/common.py:24-31).
"""

from __future__ import annotations

import dataclasses

DEFAULT_BLOCK_SIZE = 32
DEFAULT_SMALL_BLOCK_SIZE = 8
DEFAULT_THRESHOLD = 0.9
DEFAULT_MASK_ID = 151665
DEFAULT_STOP_TOKEN = 151645

KV_CACHE_CONTRACT = "inplace_bsnh_v1"  # export_utils.py:21


@dataclasses.dataclass(frozen=True)
class FastDLLMConfig:
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
    bd_size: int = DEFAULT_BLOCK_SIZE
    pad_token_id: int = 0
    context_window_size: int = 32768

    @property
    def qkv_dim(self) -> int:
        return (self.num_attention_heads + 2 * self.num_key_value_heads) * self.head_dim

    @property
    def small_block_size(self) -> int:
        return self.bd_size // 4

    def layer_bytes(self, elem: int = 2) -> int:
        """Weight bytes of one decoder layer (qkv + bias, o, gate_up, down, two norms)."""
        h, i, q = self.hidden_size, self.intermediate_size, self.num_attention_heads * self.head_dim
        n = self.qkv_dim * h + self.qkv_dim + h * q + 2 * i * h + h * i + 2 * h
        return n * elem

    def step_bytes(self, rows: int, prefix: int, elem: int = 2) -> int:
        """Algorithmic HBM bytes of one cached step + lm_head + confidence (batch 1): every layer
        weight and the lm_head once, the K/V of [0, prefix + bd_size) read, the step's K/V rows
        written, and about 4 bytes per activation element of the row stream."""
        kv_row = self.num_hidden_layers * 2 * self.num_key_value_heads * self.head_dim * elem
        return (self.num_hidden_layers * self.layer_bytes(elem) + self.vocab_size * self.hidden_size * elem
                + kv_row * (prefix + self.bd_size) + kv_row * rows + 4 * rows * self.hidden_size)

    def step_flops(self, rows: int, prefix: int) -> int:
        lin = (self.num_hidden_layers * (self.qkv_dim * self.hidden_size
                                         + self.hidden_size * self.num_attention_heads * self.head_dim
                                         + 3 * self.intermediate_size * self.hidden_size)
               + self.vocab_size * self.hidden_size)
        attn = self.num_hidden_layers * 4 * self.num_attention_heads * (prefix + self.bd_size) * self.head_dim
        return 2 * rows * lin + rows * attn


def fast_dllm_v2_1p5b(**overrides) -> FastDLLMConfig:
    """Fast-dLLM v2 1.5B (01_eager_hf_model.ipynb cell 2; cuda.py:351-387)."""
    base = dict(vocab_size=151936, hidden_size=1536, intermediate_size=8960, num_hidden_layers=28,
                num_attention_heads=12, num_key_value_heads=2, head_dim=128)
    base.update(overrides)
    return FastDLLMConfig(**base)
