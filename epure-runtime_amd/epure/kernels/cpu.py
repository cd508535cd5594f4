"""CPU backend interface (reference ``epure/kernels/cpu.py``) -- always declines.

The reference serves CPU activations with its Rust kernel
(kernel/src/lib.rs); this build targets the GPU only, so ``available()`` is
False and ``linear`` returns ``None``, which makes the caller materialize:
the same behaviour as a reference install without the extension
(cpu.py:29-45).
"""


def available():
    return False


def threads():
    return 0


def linear(x, store, cache=None):
    return None
