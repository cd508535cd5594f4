"""CPU oracle for the fused codebook dequant-matmul.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports this
module; only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` use it, and only as the checker or the timed CPU
baseline.

Contents
--------
``ref``      numpy restatements of the reference's packing, dequantisation,
             Rust-order GEMV and backward closed forms.
``rowdot``   ctypes binding of ``rowdot.c``, the plain-C restatement of the
             reference Rust kernel (``kernel/src/lib.rs``).
``decoder``  dense float32 restatement of the decoder the reference runs
             through transformers (materialize + ``F.linear``), used for the
             greedy-decode parity checks.

Parity pinning (what checks each function) is listed in each module header.
"""
