"""Writes the small seeded fixtures in this directory.

The reference holds no test vectors for this path (it has no tests and its
.ebin files are git-ignored), so these fixtures come from the CPU oracle
after it has been pinned by tests/test_oracle.py (brute force, closed forms,
library routines).  They freeze the oracle's answers so GPU runs can be
checked against committed data as well as against a live oracle call.

Each .npz holds: idx [N, K] u8, packed (flat, runtime.py:34-45 layout),
scale [N, G] f16, cb [L] f16, x_bf16 [M, K] bf16 bit patterns,
tile_f32 [N, K] (container.py:70-88), y_rust [M, N] (kernel/src/lib.rs
order, float32), y_f64 [M, N] (exact), levels, group.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import ref, rowdot  # noqa: E402

CASES = {
    "gemv4_n96_k512_g128_m1": (96, 512, 16, 128, 1, 101),
    "gemv4_n64_k256_g64_m4": (64, 256, 16, 64, 4, 102),
    "gemv8_n48_k256_g128_m2": (48, 256, 256, 128, 2, 103),
    "gemv4_n40_k96_g32_m3_lv10": (40, 96, 10, 32, 3, 104),
}


def make(name, n, k, levels, group, m, seed):
    idx, packed, scale, cb = ref.synth_linear(n, k, levels, group, seed=seed)
    r = np.random.Generator(np.random.PCG64(seed + 1000))
    x_bits = ref.f32_to_bf16_bits(r.standard_normal((m, k)).astype(np.float32))
    x = ref.bf16_bits_to_f32(x_bits)
    tile = ref.dequant_tile_f32(idx, scale, cb, group)
    y_rust = rowdot.dequant_matmul(x, ref.packed_2d(packed, n, k, levels),
                                   scale.astype(np.float32), cb.astype(np.float32), group,
                                   levels <= 16)
    y64 = ref.linear_f64(x, tile)
    np.savez_compressed(os.path.join(HERE, name + ".npz"), idx=idx, packed=packed, scale=scale,
                        cb=cb, x_bf16=x_bits, tile_f32=tile, y_rust=y_rust, y_f64=y64,
                        levels=np.int64(levels), group=np.int64(group))


if __name__ == "__main__":
    for name, args in CASES.items():
        make(name, *args)
        print("wrote", name)
