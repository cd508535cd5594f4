"""ctypes binding of ``oracle/rowdot.c`` (TEST INFRASTRUCTURE ONLY).

Mirrors the PyO3 surface of the reference Rust module ``epure_kernel``:
``dequant_matmul(x, packed, scales, cb, group, four_bit)`` and ``threads()``
(kernel/src/lib.rs:94-104, :155-157).

Pinning: bit-exact against ``oracle.ref.rust_dequant_matmul`` (an independent
numpy restatement), against fp64 brute force within a derived bound, and on
closed-form special cases (tests/test_oracle.py).
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_rowdot.so")
_lib = None


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        lib.oracle_dequant_matmul_f32.restype = ctypes.c_longlong
        lib.oracle_dequant_matmul_f32.argtypes = [
            ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_size_t,
            ctypes.c_size_t, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
            ctypes.c_size_t, ctypes.c_size_t, ctypes.c_int, ctypes.c_void_p, ctypes.c_int]
        lib.oracle_threads.restype = ctypes.c_size_t
        _lib = lib
    return _lib


def threads():
    return int(_load().oracle_threads())


def dequant_matmul(x, packed, scales, cb, group, four_bit, nthreads=0):
    """out[m, n] = x[m, k] @ dequant(packed)[n, k].T, Rust summation order.

    x: f32 (any shape, flattened like ``as_slice``); packed: u8 [n, row_bytes];
    scales: f32 [n, n_groups]; cb: f32 [levels].
    """
    lib = _load()
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    cb = np.ascontiguousarray(cb, dtype=np.float32).ravel()
    n, row_bytes = packed.shape
    k = row_bytes * 2 if four_bit else row_bytes
    m = x.size // k if k else 0
    out = np.empty((max(m, 0), n), dtype=np.float32)
    rc = lib.oracle_dequant_matmul_f32(
        x.ctypes.data, x.size, packed.ctypes.data, n, row_bytes, scales.ctypes.data,
        scales.shape[1], cb.ctypes.data, cb.size, group, int(bool(four_bit)),
        out.ctypes.data, int(nthreads))
    if rc < 0:
        raise ValueError(f"oracle_dequant_matmul_f32 failed with code {rc}")
    return out
