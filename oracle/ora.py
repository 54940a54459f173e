"""ctypes binding of oracle/rc_oracle.c (TEST INFRASTRUCTURE ONLY; see oracle/__init__.py).

Each function cites the reference lines it restates in rc_oracle.c.  The shared object is built by
``make -C oracle`` (``__graft_entry__.build()`` runs it).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None

_u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            build()
        L = ctypes.CDLL(_SO)
        i64, c_int = ctypes.c_int64, ctypes.c_int
        L.ora_encode_tables.argtypes = [c_int, _u32p, c_int, _i32p, i64, _u32p, i64]
        L.ora_encode_tables.restype = i64
        L.ora_decode_tables.argtypes = [c_int, _u32p, c_int, i64, _u32p, i64, _i32p]
        L.ora_encode_probs_q2.argtypes = [c_int, _f32p, c_int, _i32p, i64, _u32p, i64]
        L.ora_encode_probs_q2.restype = i64
        L.ora_decode_probs_q2.argtypes = [c_int, _f32p, c_int, i64, _u32p, i64, _i32p]
        L.ora_encode_logits_xq.argtypes = [c_int, _f32p, c_int, _i32p, i64, _u32p, i64]
        L.ora_encode_logits_xq.restype = i64
        L.ora_decode_logits_xq.argtypes = [c_int, _f32p, c_int, i64, _u32p, i64, _i32p]
        L.ora_q2_cdf_rows.argtypes = [_f32p, i64, c_int, c_int, _u32p]
        L.ora_xq_cdf_rows.argtypes = [_f32p, i64, c_int, c_int, _u32p]
        L.ora_expf_rows.argtypes = [_f32p, i64, _f32p]
        _lib = L
    return _lib


def _cap(T: int) -> int:
    # word capacity of a stream of T symbols: at most one word per coded symbol plus the few finalize
    # words; the device pitch uses the same T + 8 bound
    return int(T) + 8


def encode_tables(P: int, cdf: np.ndarray, syms: np.ndarray) -> np.ndarray:
    """One stream: cdf [T, K+1] uint32, syms [T] -> words (uint32)."""
    cdf = np.ascontiguousarray(cdf, dtype=np.uint32)
    syms = np.ascontiguousarray(syms, dtype=np.int32)
    T, K1 = cdf.shape
    out = np.zeros(_cap(T), dtype=np.uint32)
    n = lib().ora_encode_tables(P, cdf.reshape(-1), K1 - 1, syms, T, out, out.size)
    assert n <= out.size
    return out[:n].copy()


def decode_tables(P: int, cdf: np.ndarray, words: np.ndarray) -> np.ndarray:
    cdf = np.ascontiguousarray(cdf, dtype=np.uint32)
    words = np.ascontiguousarray(words, dtype=np.uint32)
    T, K1 = cdf.shape
    syms = np.zeros(T, dtype=np.int32)
    w = words if words.size else np.zeros(1, dtype=np.uint32)
    lib().ora_decode_tables(P, cdf.reshape(-1), K1 - 1, T, w, words.size, syms)
    return syms


def encode_probs_q2(P: int, probs: np.ndarray, syms: np.ndarray) -> np.ndarray:
    probs = np.ascontiguousarray(probs, dtype=np.float32)
    syms = np.ascontiguousarray(syms, dtype=np.int32)
    T, K = probs.shape
    out = np.zeros(_cap(T), dtype=np.uint32)
    n = lib().ora_encode_probs_q2(P, probs.reshape(-1), K, syms, T, out, out.size)
    return out[:n].copy()


def decode_probs_q2(P: int, probs: np.ndarray, words: np.ndarray) -> np.ndarray:
    probs = np.ascontiguousarray(probs, dtype=np.float32)
    words = np.ascontiguousarray(words, dtype=np.uint32)
    T, K = probs.shape
    syms = np.zeros(T, dtype=np.int32)
    w = words if words.size else np.zeros(1, dtype=np.uint32)
    lib().ora_decode_probs_q2(P, probs.reshape(-1), K, T, w, words.size, syms)
    return syms


def encode_logits_xq(P: int, logits: np.ndarray, syms: np.ndarray) -> np.ndarray:
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    syms = np.ascontiguousarray(syms, dtype=np.int32)
    T, K = logits.shape
    out = np.zeros(_cap(T), dtype=np.uint32)
    n = lib().ora_encode_logits_xq(P, logits.reshape(-1), K, syms, T, out, out.size)
    return out[:n].copy()


def decode_logits_xq(P: int, logits: np.ndarray, words: np.ndarray) -> np.ndarray:
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    words = np.ascontiguousarray(words, dtype=np.uint32)
    T, K = logits.shape
    syms = np.zeros(T, dtype=np.int32)
    w = words if words.size else np.zeros(1, dtype=np.uint32)
    lib().ora_decode_logits_xq(P, logits.reshape(-1), K, T, w, words.size, syms)
    return syms


def q2_cdf(probs: np.ndarray, P: int) -> np.ndarray:
    """probs [..., K] float32 -> cdf [..., K+1] uint32 (gpu_range_coder.py:57-79)."""
    probs = np.ascontiguousarray(probs, dtype=np.float32)
    K = probs.shape[-1]
    rows = probs.size // K
    out = np.zeros(probs.shape[:-1] + (K + 1,), dtype=np.uint32)
    lib().ora_q2_cdf_rows(probs.reshape(-1), rows, K, P, out.reshape(-1))
    return out


def xq_cdf(logits: np.ndarray, P: int) -> np.ndarray:
    """logits [..., K] float32 -> cdf [..., K+1] uint32 (this build's fused quantiser)."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    K = logits.shape[-1]
    rows = logits.size // K
    out = np.zeros(logits.shape[:-1] + (K + 1,), dtype=np.uint32)
    lib().ora_xq_cdf_rows(logits.reshape(-1), rows, K, P, out.reshape(-1))
    return out


def expf(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().ora_expf_rows(x.reshape(-1), x.size, y.reshape(-1))
    return y
