"""ctypes binding of ``qmm_ref.c`` (the C restatement) and ``qmm_fast.c`` (the
vectorised CPU restatement timed as the CPU baseline) — TEST INFRASTRUCTURE ONLY.

``build()`` compiles it with gcc through ``oracle/Makefile``; ``load()`` opens the
built library.  Used by the tests as a second, independent implementation of
the oracle and by ``bench.py`` as the timed CPU baseline.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "liboracle_ref.so")
_lib = None


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def available():
    return os.path.exists(LIB_PATH)


def load():
    global _lib
    if _lib is None:
        if not available():
            raise RuntimeError(f"C oracle not built: {LIB_PATH} (run oracle.cref.build())")
        lib = ctypes.CDLL(LIB_PATH)
        p, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        lib.oref_qmm_bf16.argtypes = [p, p, p, p, p, p, i64, i64, i64, i32, i32, i32]
        lib.oref_qmm_bf16.restype = i32
        lib.oref_qmm_fast_bf16.argtypes = [p, p, p, p, p, p, i64, i64, i64, i32, i32, i32]
        lib.oref_qmm_fast_bf16.restype = i32
        lib.oref_vocab_gather_bf16.argtypes = [p, i32, i64, p, i64, i64, i64, p, i32]
        lib.oref_vocab_gather_bf16.restype = i32
        _lib = lib
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def default_threads():
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, 16))


def qmm_bf16(x, wq, scales, biases, bias=None, group_size=64, bits=4, threads=None):
    """x uint16 [M, K]; wq uint32 [N, K*bits/32]; s, b uint16 [N, G] -> uint16 [M, N]."""
    lib = load()
    x = np.ascontiguousarray(x, dtype=np.uint16)
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    s = np.ascontiguousarray(scales, dtype=np.uint16)
    b = np.ascontiguousarray(biases, dtype=np.uint16)
    M, K = x.shape
    N = wq.shape[0]
    y = np.empty((M, N), dtype=np.uint16)
    bptr = None
    if bias is not None:
        bias = np.ascontiguousarray(bias, dtype=np.uint16)
        bptr = _ptr(bias)
    rc = lib.oref_qmm_bf16(_ptr(x), _ptr(wq), _ptr(s), _ptr(b), bptr, _ptr(y), M, N, K, bits,
                           group_size, threads or default_threads())
    if rc != 0:
        raise ValueError(f"oref_qmm_bf16 failed with {rc}")
    return y


def qmm_fast_bf16(x, wq, scales, biases, bias=None, group_size=64, bits=4, threads=None):
    """The vectorised fp32 CPU restatement (qmm_fast.c): the timed CPU baseline."""
    lib = load()
    x = np.ascontiguousarray(x, dtype=np.uint16)
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    s = np.ascontiguousarray(scales, dtype=np.uint16)
    b = np.ascontiguousarray(biases, dtype=np.uint16)
    M, K = x.shape
    N = wq.shape[0]
    y = np.empty((M, N), dtype=np.uint16)
    bptr = None
    if bias is not None:
        bias = np.ascontiguousarray(bias, dtype=np.uint16)
        bptr = _ptr(bias)
    rc = lib.oref_qmm_fast_bf16(_ptr(x), _ptr(wq), _ptr(s), _ptr(b), bptr, _ptr(y), M, N, K, bits,
                                group_size, threads or default_threads())
    if rc != 0:
        raise ValueError(f"oref_qmm_fast_bf16 failed with {rc}")
    return y


def vocab_gather_bf16(ids, table, vocab_start, threads=None):
    lib = load()
    ids = np.ascontiguousarray(ids)
    is64 = 1 if ids.dtype == np.int64 else 0
    if not is64:
        ids = ids.astype(np.int32)
    table = np.ascontiguousarray(table, dtype=np.uint16)
    out = np.empty(ids.shape + (table.shape[1],), dtype=np.uint16)
    rc = lib.oref_vocab_gather_bf16(_ptr(ids), is64, ids.size, _ptr(table), table.shape[0],
                                    table.shape[1], vocab_start, _ptr(out),
                                    threads or default_threads())
    if rc != 0:
        raise ValueError(f"oref_vocab_gather_bf16 failed with {rc}")
    return out
