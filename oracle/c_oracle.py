"""ctypes wrapper for ``oracle/liboracle_q8.so`` (the plain-C restatement).

TEST INFRASTRUCTURE ONLY (see ``oracle/q8_oracle.py``)."""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

_DT = {np.dtype(np.float32): 0, np.dtype(np.float16): 1, np.dtype(np.uint16): 2}


def build() -> None:
    subprocess.check_call(["make", "-s", "-C", _HERE, "oracle"])


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle_q8.so")
        if not os.path.exists(path):
            build()
        L = ctypes.CDLL(path)
        P, I, I64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
        L.q8_ref_quantize_rows.argtypes = [P, I, P, I64, I]
        L.q8_ref_reshape_and_cache.argtypes = [P, I, P, P, I, I, I, I, I64, I64, I64, I64, I64]
        L.q8_ref_gather.argtypes = [P, P, P, P, P, P, I, I, I, I, I, I, I,
                                    I64, I64, I64, I64, I64, I64]
        _LIB = L
    return _LIB


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def quantize_rows(x: np.ndarray) -> np.ndarray:
    """x [..., D] fp16 / bf16 bits (uint16) / fp32 -> uint8 [..., D/32*34]."""
    x = np.ascontiguousarray(x)
    D = x.shape[-1]
    N = x.size // D
    y = np.empty(x.shape[:-1] + (D // 32 * 34,), dtype=np.uint8)
    lib().q8_ref_quantize_rows(_p(x), _DT[x.dtype], _p(y), N, D)
    return y


def reshape_and_cache(key: np.ndarray, slot_mapping: np.ndarray, cache: np.ndarray) -> None:
    """cache: uint8 [NB, bs, Hkv, bpr] C-contiguous, written in place."""
    key = np.ascontiguousarray(key)
    sm = np.ascontiguousarray(slot_mapping, dtype=np.int64)
    assert cache.flags.c_contiguous
    T, Hkv, D = key.shape
    NB, bs, _, bpr = cache.shape
    lib().q8_ref_reshape_and_cache(_p(key), _DT[key.dtype], _p(sm), _p(cache), T, Hkv, D, bs,
                                   Hkv * D, D, bs * Hkv * bpr, Hkv * bpr, bpr)


def gather(k_cache: np.ndarray, v_cache: np.ndarray, block_table: np.ndarray,
           seq_lens: np.ndarray, Sk: int, k_out: np.ndarray | None = None):
    """Reference gather contract over C-contiguous AoS caches
    k [NB, bs, Hkv, kb], v [NB, bs, Hkv, vb(bytes)]."""
    NB, bs, Hkv, kb = k_cache.shape
    vb = v_cache.shape[-1] * v_cache.itemsize
    B, M = block_table.shape
    bt = np.ascontiguousarray(block_table, dtype=np.int32)
    sl = np.ascontiguousarray(seq_lens, dtype=np.int32)
    if k_out is None:
        k_out = np.zeros((B, Hkv, Sk, kb), dtype=np.uint8)
    v_out = np.empty((B, Hkv, Sk, v_cache.shape[-1]), dtype=v_cache.dtype)
    lib().q8_ref_gather(_p(k_cache), _p(v_cache), _p(bt), _p(sl), _p(k_out), _p(v_out),
                        B, Hkv, Sk, kb, vb, bs, M,
                        bs * Hkv * kb, Hkv * kb, kb, bs * Hkv * vb, Hkv * vb, vb)
    return k_out, v_out
