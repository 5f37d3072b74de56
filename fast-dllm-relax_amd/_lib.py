"""ctypes binding of libfdllm.so (the C ABI declared in include/fdllm.h).

There is no fallback: if the library is missing or fails to load, every entry point raises.
Error codes map to the reference's exceptions: FDLLM_EINVAL -> ValueError (the reference's window
checks, runtime.py:56-57, 69-70, 258-263, and VM shape errors), anything else -> RuntimeError.
"""

from __future__ import annotations

import ctypes
import pathlib

LIB_PATH = pathlib.Path(__file__).resolve().parent / "libfdllm.so"

FDLLM_OK, FDLLM_EINVAL, FDLLM_EHIP, FDLLM_ESTATE = 0, 1, 2, 3
DTYPE_BF16, DTYPE_F16 = 0, 1

# every entry point declared in include/fdllm.h
EXPORTS = (
    "fdllm_create", "fdllm_destroy", "fdllm_num_params", "fdllm_param_name", "fdllm_bind_weights",
    "fdllm_embed", "fdllm_forward_hidden", "fdllm_get_logits", "fdllm_build_prefix_cache",
    "fdllm_forward_cached", "fdllm_forward_cached_noalloc", "fdllm_forward_block_partial", "fdllm_forward_block_partial_rp0",
    "fdllm_forward_block_partial_rp8", "fdllm_forward_block_partial_rp16", "fdllm_forward_block_partial_rp24",
    "fdllm_kv_write", "fdllm_attn_inplace",
    "fdllm_forward_cached_batch", "fdllm_forward_block_partial_batch", "fdllm_build_prefix_cache_seq",
    "fdllm_get_confidence", "fdllm_confidence_from_logits", "fdllm_unmask", "fdllm_get_confidence_unmask",
    "fdllm_host_alloc", "fdllm_host_free", "fdllm_bench_op", "fdllm_group_wait_launches",
    "fdllm_frag_calls",
    "fdllm_last_error",
)

OP_QKV, OP_O_PROJ, OP_GATE_UP, OP_DOWN, OP_ATTENTION, OP_LM_HEAD_CONFIDENCE = range(6)


class FdllmConfig(ctypes.Structure):
    _fields_ = [
        ("vocab_size", ctypes.c_int32), ("hidden_size", ctypes.c_int32), ("intermediate_size", ctypes.c_int32),
        ("num_hidden_layers", ctypes.c_int32), ("num_attention_heads", ctypes.c_int32),
        ("num_key_value_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32), ("rms_norm_eps", ctypes.c_float),
        ("rope_theta", ctypes.c_float), ("tie_word_embeddings", ctypes.c_int32), ("bd_size", ctypes.c_int32),
        ("dtype", ctypes.c_int32), ("max_rows", ctypes.c_int32),
    ]


_lib: ctypes.CDLL | None = None

_P, _I, _I64, _F = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
_SIGS = {
    "fdllm_create": ([ctypes.POINTER(FdllmConfig), ctypes.POINTER(ctypes.c_void_p)], _I),
    "fdllm_destroy": ([_P], None),
    "fdllm_num_params": ([_P], _I),
    "fdllm_param_name": ([_P, _I], ctypes.c_char_p),
    "fdllm_bind_weights": ([_P, ctypes.POINTER(ctypes.c_void_p), _I], _I),
    "fdllm_embed": ([_P, _P, _I, _P, _P], _I),
    "fdllm_forward_hidden": ([_P, _P, _I, _P, _P, _P], _I),
    "fdllm_get_logits": ([_P, _P, _I, _P, _P], _I),
    "fdllm_build_prefix_cache": ([_P, _P, _I, _P, _P, _P, _I, _P], _I),
    "fdllm_forward_cached": ([_P, _P, _I, _P, _P, _I, _P, _I64, _P, _P], _I),
    "fdllm_forward_cached_noalloc": ([_P, _P, _I, _P, _P, _I, _P, _I64, _P, _P], _I),
    "fdllm_forward_block_partial": ([_P, _I, _P, _I, _P, _P, _I, _P, _I64, _P, _P], _I),
    "fdllm_forward_block_partial_rp0": ([_P, _P, _I, _P, _P, _I, _P, _I64, _P, _P], _I),
    "fdllm_forward_block_partial_rp8": ([_P, _P, _I, _P, _P, _I, _P, _I64, _P, _P], _I),
    "fdllm_forward_block_partial_rp16": ([_P, _P, _I, _P, _P, _I, _P, _I64, _P, _P], _I),
    "fdllm_forward_block_partial_rp24": ([_P, _P, _I, _P, _P, _I, _P, _I64, _P, _P], _I),
    "fdllm_kv_write": ([_P, _P, _P, _I, _P, _P, _I, _I, _I64, _P], _I),
    "fdllm_attn_inplace": ([_P, _P, _P, _P, _I, _P, _P, _I, _I, _I64, _I, _I, _P, _P], _I),
    "fdllm_forward_cached_batch": ([_P, _P, _I, _I, _P, _P, _I, _P, ctypes.POINTER(_I64), _P, _P], _I),
    "fdllm_forward_block_partial_batch": ([_P, _I, _P, _I, _I, _P, _P, _I, _P, ctypes.POINTER(_I64), _P, _P], _I),
    "fdllm_build_prefix_cache_seq": ([_P, _P, _I, _P, _P, _P, _I, _I, _I, _P], _I),
    "fdllm_get_confidence": ([_P, _P, _I, _P, _P, _P, _P], _I),
    "fdllm_confidence_from_logits": ([_P, _P, _I, _I, _I, _P, _P, _P], _I),
    "fdllm_unmask": ([_P, _P, _P, _I, _I, _P, _I, _I, ctypes.c_int32, _F, _P, ctypes.c_int32, _P], _I),
    "fdllm_get_confidence_unmask": ([_P, _P, _I, _I, _P, _I, _I, ctypes.c_int32, _F, _P, _P, _P, ctypes.c_int32, _P], _I),
    "fdllm_host_alloc": ([ctypes.c_size_t, ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_void_p)], _I),
    "fdllm_host_free": ([_P], None),
    "fdllm_bench_op": ([_P, _I, _I, _I, _I, _P, _P, _I, _I, _P], _I),
    "fdllm_group_wait_launches": ([_P], ctypes.c_longlong),
    "fdllm_frag_calls": ([_P], ctypes.c_longlong),
    "fdllm_last_error": ([], ctypes.c_char_p),
}


def load() -> ctypes.CDLL:
    """Load libfdllm.so; raises if it is absent (build it with __graft_entry__.build() or make)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built; the HIP path has no fallback "
                               "(run `make -C fast-dllm-relax_amd` or __graft_entry__.build())")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (args, res) in _SIGS.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _lib = lib
    return _lib


def check(rc: int) -> None:
    if rc == FDLLM_OK:
        return
    msg = (load().fdllm_last_error() or b"").decode()
    if rc == FDLLM_EINVAL:
        raise ValueError(msg)
    raise RuntimeError(f"libfdllm error {rc}: {msg}")
