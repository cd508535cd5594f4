"""Fused dequantize-and-matmul backends (contract of the reference's
``epure/kernels/__init__.py:1-15``):

    linear(x, store, ...) -> Tensor | None

``None`` means "this backend cannot serve this call" and the caller falls
back to materializing the weight.

``cuda`` is the gfx950 HIP backend (libepure_hip.so); ``cpu`` is the host
backend (libepure_cpu.so), bit-identical to the reference's Rust kernel.
"""
from . import cpu, cuda

__all__ = ["cpu", "cuda"]
