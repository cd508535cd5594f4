"""CPU backend: the fused dequant-matmul on host cores (``libepure_cpu.so``).

Contract of the reference's ``epure/kernels/cpu.py:29-70``: ``available()``,
``threads()`` and ``linear(x, store, cache=None) -> Tensor | None`` where
``None`` declines and the caller materializes.  It serves what the
reference's Rust path serves -- a CPU ``x`` in float32, a rank-2 store with
at most 16 levels (4-bit indices) -- and declines the rest (a bf16/fp16
``x`` would cost more to convert than the kernel saves, cpu.py:51-55).
The result is bit-identical to the Rust kernel (kernel/src/lib.rs:36-151):
same per-group LUT, same k order, products rounded then added, no FMA.

The per-store host copies (packed rows, f32 scales, f32 codebook) live in
``cache`` keyed by the store's identity, as the reference does
(runtime.py:24, cpu.py:57-67); unlike the reference, an entry is rebuilt
when the store's ``packed``/``scale``/``cb`` tensors were replaced or
modified in place (``make_trainable`` swaps them for Parameters, training
updates them), so a stale copy is never used.
"""
import ctypes
import os

import numpy as np
import torch

LIB_NAME = "libepure_cpu.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "_lib",
                        LIB_NAME)

_lib = None
LOAD_ERROR = None


def _load():
    global _lib, LOAD_ERROR
    if _lib is None and LOAD_ERROR is None:
        try:
            lib = ctypes.CDLL(LIB_PATH)
            lib.ep_cpu_dequant_matmul_f32.restype = ctypes.c_int
            lib.ep_cpu_dequant_matmul_f32.argtypes = [
                ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64,
                ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_int]
            lib.ep_cpu_threads.restype = ctypes.c_size_t
            lib.ep_cpu_threads.argtypes = []
            _lib = lib
        except OSError as exc:
            LOAD_ERROR = exc
    return _lib


def available():
    """True when libepure_cpu.so is loaded."""
    return _load() is not None


def threads():
    """Worker threads a call uses by default (0 when the library is absent)."""
    lib = _load()
    return int(lib.ep_cpu_threads()) if lib is not None else 0


_ERRORS = {-1: "levels > 256", -2: "fewer scale columns than groups",
           -3: "bad pointer, size or group", -4: "out of memory"}


def dequant_matmul(x, packed, scales, cb, group, four_bit, nthreads=0):
    """numpy surface of the reference's ``epure_kernel.dequant_matmul``
    (lib.rs:94-151): x f32 (flattened, m = x.size // k), packed u8
    [n, row_bytes], scales f32 [n, n_groups], cb f32 [levels] -> f32 [m, n].
    Raises ValueError where the Rust code raises."""
    lib = _load()
    if lib is None:
        raise RuntimeError(f"{LIB_NAME} is not available: {LOAD_ERROR}")
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    cb = np.ascontiguousarray(cb, dtype=np.float32).reshape(-1)
    if packed.ndim != 2 or scales.ndim != 2:
        raise ValueError("packed and scales must be 2-D")
    n, row_bytes = packed.shape
    k = row_bytes * 2 if four_bit else row_bytes
    m = x.size // k if k else 0
    out = np.empty((m, n), dtype=np.float32)
    rc = lib.ep_cpu_dequant_matmul_f32(
        x.ctypes.data, x.size, packed.ctypes.data, n, row_bytes, scales.ctypes.data,
        scales.shape[1], cb.ctypes.data, cb.size, int(group), int(bool(four_bit)),
        out.ctypes.data, int(nthreads))
    if rc != 0:
        raise ValueError(f"ep_cpu_dequant_matmul_f32: {_ERRORS.get(rc, rc)}")
    return out


def _version(t):
    return (id(t), t._version, t.data_ptr())


def _host_copies(store, cache):
    key = id(store)
    stamp = (_version(store.packed), _version(store.scale), _version(store.cb))
    entry = cache.get(key) if cache is not None else None
    if entry is None or entry[0] != stamp:
        entry = (stamp,
                 np.ascontiguousarray(store.packed_2d().detach().numpy()),
                 np.ascontiguousarray(store.scale.detach().to(torch.float32).numpy()),
                 np.ascontiguousarray(store.cb.detach().to(torch.float32).numpy()).reshape(-1))
        if cache is not None:
            cache[key] = entry
    return entry[1:]


def linear(x, store, cache=None):
    """``x @ dequant(store).T`` on the host cores, or ``None`` to decline."""
    if _load() is None or x.is_cuda or store.levels > 16 or len(store.shape) != 2:
        return None
    if x.dtype != torch.float32 or store.packed.is_cuda:
        return None
    if torch.is_grad_enabled() and (x.requires_grad or store.cb.requires_grad
                                    or store.scale.requires_grad):
        return None  # no backward here: the differentiable route materializes
    shape = x.shape
    packed, scale, cb = _host_copies(store, cache)
    out = dequant_matmul(x.detach().reshape(-1, shape[-1]).numpy(), packed, scale, cb,
                         store.group, True)
    return torch.from_numpy(out).reshape(*shape[:-1], store.out_features)
