"""MI355X-native cached block-diffusion step of Fast-dLLM v2 (gfx950 HIP kernels behind a C ABI).

Modules:
  config   -- model constants and decode defaults (FastDLLMRelaxConfig / common.py of the reference)
  params   -- packed parameter order, synthetic weights, reference artifact loading
  vm       -- HipVM: the nine entry points (REQUIRED_FNS) + device confidence over libfdllm.so
  runtime  -- prefix KV cache, step functions and the decode loop (mirror of fast_dllm_relax/runtime.py)
"""

from .config import (DEFAULT_BLOCK_SIZE, DEFAULT_MASK_ID, DEFAULT_SMALL_BLOCK_SIZE, DEFAULT_STOP_TOKEN,
                     DEFAULT_THRESHOLD, FastDLLMConfig, fast_dllm_v2_1p5b)

__all__ = ["FastDLLMConfig", "fast_dllm_v2_1p5b", "DEFAULT_BLOCK_SIZE", "DEFAULT_SMALL_BLOCK_SIZE",
           "DEFAULT_THRESHOLD", "DEFAULT_MASK_ID", "DEFAULT_STOP_TOKEN"]
