"""ctypes wrapper of oracle/confidence.c.  TEST INFRASTRUCTURE ONLY.

``confidence(logits)`` -> (ids int32 [rows], maxp fp32 [rows]), unshifted (as metal.py:505-528 returns
them); ``shifted_confidence(logits)`` applies runtime.py:172-174 (row i takes row i-1; row 0 its own)
and also returns the unshifted argmax of the last row (runtime.py:181).
``unmask(p, masked, threshold)`` is runtime.py:794-805.
"""

from __future__ import annotations

import ctypes
import pathlib
import subprocess

import numpy as np

_HERE = pathlib.Path(__file__).resolve().parent
_LIB_PATH = _HERE / "liboracle_conf.so"
_lib = None


def build() -> pathlib.Path:
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        lib = ctypes.CDLL(str(_LIB_PATH))
        f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
        i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
        u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
        lib.fd_exp_neg.argtypes = [ctypes.c_float]
        lib.fd_exp_neg.restype = ctypes.c_float
        lib.fd_confidence.argtypes = [f32p, ctypes.c_int, ctypes.c_int, i32p, f32p, f32p, i32p, f32p]
        lib.fd_confidence.restype = None
        lib.fd_tile_stats.argtypes = [f32p, ctypes.c_int, f32p, i32p, f32p]
        lib.fd_tile_stats.restype = None
        lib.fd_unmask.argtypes = [f32p, u8p, ctypes.c_int, ctypes.c_float, u8p]
        lib.fd_unmask.restype = ctypes.c_int
        _lib = lib
    return _lib


def exp_neg(x: float) -> float:
    return float(_load().fd_exp_neg(float(x)))


def exp_neg_array(x: np.ndarray) -> np.ndarray:
    lib = _load()
    flat = np.asarray(x, dtype=np.float32).ravel()
    return np.array([lib.fd_exp_neg(float(v)) for v in flat], dtype=np.float32).reshape(np.shape(x))


def tile_stats(row: np.ndarray):
    row = np.ascontiguousarray(row, dtype=np.float32)
    tiles = (row.size + 255) // 256
    m = np.empty(tiles, np.float32)
    a = np.empty(tiles, np.int32)
    s = np.empty(tiles, np.float32)
    _load().fd_tile_stats(row, row.size, m, a, s)
    return m, a, s


def confidence(logits: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    x = np.ascontiguousarray(np.asarray(logits, dtype=np.float32).reshape(-1, np.shape(logits)[-1]))
    rows, vocab = x.shape
    tiles = (vocab + 255) // 256
    ids = np.empty(rows, np.int32)
    maxp = np.empty(rows, np.float32)
    _load().fd_confidence(x, rows, vocab, ids, maxp, np.empty(tiles, np.float32), np.empty(tiles, np.int32),
                          np.empty(tiles, np.float32))
    return ids, maxp


def shift(ids: np.ndarray, maxp: np.ndarray):
    """runtime.py:172-174: row i takes row i-1's prediction, row 0 keeps its own."""
    return np.concatenate([ids[:1], ids[:-1]]).astype(np.int64), np.concatenate([maxp[:1], maxp[:-1]])


def shifted_confidence(logits: np.ndarray):
    ids, maxp = confidence(logits)
    sid, sp = shift(ids, maxp)
    return sid, sp, int(ids[-1])


def threshold_f32(threshold: float) -> np.float32:
    """Largest float32 <= threshold: `p32 > t32` then decides exactly like numpy's `p32 > threshold`."""
    t = np.float32(threshold)
    if float(t) > threshold:
        t = np.nextafter(t, np.float32(-np.inf))
    return np.float32(t)


def unmask(p: np.ndarray, masked: np.ndarray, threshold: float) -> np.ndarray:
    p = np.ascontiguousarray(p, dtype=np.float32)
    m = np.ascontiguousarray(masked, dtype=np.uint8)
    sel = np.zeros(p.size, np.uint8)
    _load().fd_unmask(p, m, p.size, float(threshold_f32(threshold)), sel)
    return sel.astype(bool)
