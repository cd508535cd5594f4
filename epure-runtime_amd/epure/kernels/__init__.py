"""Fused dequantize-and-matmul backends (contract of the reference's
``epure/kernels/__init__.py:1-15``):

    linear(x, store, ...) -> Tensor | None

``None`` means "this backend cannot serve this call" and the caller falls
back to materializing the weight.

``cuda`` is the gfx950 HIP backend.  ``cpu`` keeps the reference's CPU
backend interface but always declines: the CPU kernel is outside this
build's scope (the reference's own CPU path is reproduced only as the test
oracle), exactly like a reference install without its Rust extension.
"""
from . import cpu, cuda

__all__ = ["cpu", "cuda"]
