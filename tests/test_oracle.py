"""Pins the CPU oracle (oracle/ref.py, oracle/rowdot.c) before anything is
checked against it.  The reference ships no tests or fixtures for this path
(no tests/ directory; .ebin files are git-ignored), so every check here is a
brute-force computation, a closed form, or an independent library routine.
"""
import hashlib
import os

import numpy as np
import pytest
import torch

from oracle import ref, rowdot

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


# ------------------------------------------------------------------ packing
def test_pack_known_bytes():
    assert ref.pack4([1, 2], 16).tolist() == [0x21]
    assert ref.pack4([1, 2, 3], 16).tolist() == [0x21, 0x03]       # odd count: zero pad
    assert ref.pack4([15, 0, 7, 9], 16).tolist() == [0x0F, 0x97]
    assert ref.pack4([200, 17], 256).tolist() == [200, 17]          # identity above 16 levels


def test_unpack_brute_force():
    r = rng(1)
    b = r.integers(0, 256, 301, dtype=np.uint8)
    for n in (0, 1, 601, 602):
        got = ref.unpack4(b, n, 16)
        want = []
        for byte in b.tolist():
            want += [byte % 16, byte // 16]
        assert got.tolist() == want[:n]
    assert ref.unpack4(b, 100, 256).tolist() == b[:100].tolist()


@pytest.mark.parametrize("n", [1, 2, 7, 1000, 1001])
def test_pack_roundtrip(n):
    idx = rng(n).integers(0, 16, n, dtype=np.uint8)
    assert np.array_equal(ref.unpack4(ref.pack4(idx, 16), n, 16), idx)


def test_packed_2d_view():
    p = np.arange(12, dtype=np.uint8)
    assert ref.packed_2d(p, 3, 8, 16).shape == (3, 4)
    assert ref.packed_2d(p, 3, 4, 256).shape == (3, 4)


# ------------------------------------------------------------------ dequant
def test_dequant_tile_pure_python():
    idx, _, scale, cb = ref.synth_linear(5, 40, 16, 16, seed=3)
    w = ref.dequant_tile_f32(idx, scale, cb, 16)
    for n in range(5):
        for k in range(40):
            exact = float(cb[idx[n, k]]) * float(scale[n, k // 16])    # python double
            assert w[n, k] == np.float32(exact)
            # fp16 x fp16 products are exact in f32: no rounding happened
            assert float(w[n, k]) == exact


def test_dequant_tile_reads_zero_beyond_levels():
    idx = np.array([[0, 3, 9, 15]], np.uint8)
    cb = np.arange(1, 11, dtype=np.float32)            # 10 levels
    w = ref.dequant_tile_f32(idx, np.ones((1, 1), np.float32), cb, 4)
    assert w.tolist() == [[1.0, 4.0, 10.0, 0.0]]


@pytest.mark.parametrize("levels,n,k,group,f32_scale", [
    (16, 7, 256, 128, False),     # 4-bit, two groups per row
    (16, 5, 101, 32, False),      # odd K: rows straddle bytes of the flat stream
    (16, 3, 77, 16, True),        # odd K, f32 scales (after make_trainable)
    (10, 6, 96, 32, False),       # levels < 16: indices 10..15 read 0
    (256, 4, 300, 128, False),    # 8-bit, partial last group
    (256, 5, 129, 64, True),      # 8-bit, odd K, f32 scales
    (200, 3, 64, 64, False),      # 8-bit with levels < 256
])
def test_dense_tile_matches_dequant_tile(levels, n, k, group, f32_scale):
    """oracle/decoder.py dense_tile (the torch tile the large-shape GPU tests
    and the decoder oracle use) equals dequant_tile_f32 (pinned above
    against the pure-Python product) bit for bit."""
    from oracle.decoder import dense_tile

    r = rng(n * 1000 + k)
    # indices over the whole nibble/byte range, so idx >= levels occurs
    idx = r.integers(0, 16 if levels <= 16 else 256, (n, k), dtype=np.uint8)
    packed = ref.pack4(idx, levels)
    cb = np.sort(r.standard_normal(levels)).astype(np.float16)
    g = (k + group - 1) // group
    scale = (np.abs(r.normal(0.0, 0.02, (n, g))) + 1e-3).astype(np.float16)
    if f32_scale:
        scale = scale.astype(np.float32) * np.float32(1.0 + 2.0 ** -20)   # not fp16-valued
    want = ref.dequant_tile_f32(ref.unpack4(packed, n * k, levels).reshape(n, k), scale, cb, group)
    got = dense_tile(torch.from_numpy(packed), torch.from_numpy(scale), torch.from_numpy(cb),
                     n, k, group, levels).numpy()
    assert got.dtype == np.float32 and got.shape == (n, k)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    if levels < (16 if levels <= 16 else 256):
        assert (got[idx >= levels] == 0).all() and (idx >= levels).any()


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_materialize_matches_torch_expression(dtype):
    tdt = {"f16": torch.float16, "bf16": torch.bfloat16}[dtype]
    idx, packed, scale, _ = ref.synth_linear(16, 256, 16, 128, seed=4)
    cb = rng(5).standard_normal(16).astype(np.float32)          # not fp16-valued
    sc32 = scale.astype(np.float32) * np.float32(1.0001)         # not fp16-valued
    got = ref.materialize(packed, sc32, cb, 16, 256, 128, 16, dtype)
    t_idx = torch.from_numpy(idx.astype(np.int64))
    w = torch.from_numpy(cb).to(tdt)[t_idx]
    w = w * torch.from_numpy(sc32).to(tdt).repeat_interleave(128, dim=1)
    assert np.array_equal(got, w.float().numpy())


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("levels,k", [(16, 256), (16, 37), (256, 96), (12, 64)])
def test_embedding_rows_are_materialize_rows(dtype, levels, k):
    # PackedEmbedding (runtime.py:139-156) and materialize (runtime.py:78-89)
    # apply the same per-element rounding; the oracle computes them by two
    # routes (row gather of the flat stream vs whole-matrix unpack)
    n = 50
    idx = rng(20).integers(0, 16 if levels == 12 else levels, (n, k)).astype(np.uint8)
    packed = ref.pack4(idx.ravel(), levels)
    cb = rng(21).standard_normal(levels).astype(np.float32)
    scale = (np.abs(rng(22).standard_normal((n, -(-k // 32)))) * 0.02 + 1e-3).astype(np.float32)
    ids = np.array([0, 49, 7, 7, 23, 1], np.int64)
    got = ref.embedding_rows(packed, scale, cb, n, k, 32, levels, ids, dtype)
    full = ref.materialize(packed, scale, cb, n, k, 32, levels, dtype)
    assert np.array_equal(got, full[ids])


def test_embedding_rows_brute_force():
    n, k, levels, group = 6, 10, 16, 4
    idx = rng(23).integers(0, 16, (n, k)).astype(np.uint8)
    packed = ref.pack4(idx.ravel(), levels)
    cb = rng(24).standard_normal(levels).astype(np.float32)
    scale = rng(25).uniform(0.5, 2.0, (n, 3)).astype(np.float32)
    got = ref.embedding_rows(packed, scale, cb, n, k, group, levels, [5, 2], "f16")
    for i, r in enumerate([5, 2]):
        for c in range(k):
            a = np.float16(cb[idx[r, c]])
            b = np.float16(scale[r, c // group])
            assert got[i, c] == np.float32(np.float16(np.float32(a) * np.float32(b)))


def test_bf16_rounding_matches_torch():
    x = rng(6).standard_normal(10000).astype(np.float32) * 1000
    x[:4] = [np.inf, -np.inf, 0.0, -0.0]
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(ref.round_bf16(x), want)


# ------------------------------------------------------------------ Rust-order GEMV
CASES = [  # (n, k, levels, group, m)
    (64, 256, 16, 128, 1), (33, 96, 16, 32, 3), (17, 130, 16, 64, 2),
    (40, 256, 256, 128, 1), (9, 48, 200, 16, 4), (5, 6, 16, 2, 1),
]


@pytest.mark.parametrize("n,k,levels,group,m", CASES)
def test_rust_c_matches_numpy_bitwise(n, k, levels, group, m):
    four = levels <= 16
    idx, packed, scale, cb = ref.synth_linear(n, k, levels, group, seed=n + k)
    x = ref.round_bf16(rng(k).standard_normal((m, k)).astype(np.float32))
    p2 = ref.packed_2d(packed, n, k, levels)
    a = rowdot.dequant_matmul(x, p2, scale.astype(np.float32), cb.astype(np.float32), group, four)
    b = ref.rust_dequant_matmul(x, p2, scale.astype(np.float32), cb.astype(np.float32), group,
                                four)
    assert a.shape == (m, n)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    # thread count must not change the bits (rows are independent)
    c = rowdot.dequant_matmul(x, p2, scale.astype(np.float32), cb.astype(np.float32), group,
                              four, nthreads=1)
    assert np.array_equal(a.view(np.uint32), c.view(np.uint32))


@pytest.mark.parametrize("n,k,levels,group,m", CASES[:5])
def test_rust_within_fp64_bound(n, k, levels, group, m):
    idx, packed, scale, cb = ref.synth_linear(n, k, levels, group, seed=2 * n + k)
    x = ref.round_bf16(rng(7).standard_normal((m, k)).astype(np.float32))
    p2 = ref.packed_2d(packed, n, k, levels)
    y = rowdot.dequant_matmul(x, p2, scale.astype(np.float32), cb.astype(np.float32), group,
                              levels <= 16)
    w = ref.dequant_tile_f32(idx, scale, cb, group)
    exact = ref.linear_f64(x, w)
    # serial float32 summation: |err| <= (group + G) * 2^-24 * sum|x w| (first order)
    bound = (group + k / group + 2) * 2.0 ** -24 * (np.abs(x).astype(np.float64) @
                                                  np.abs(w).astype(np.float64).T)
    assert np.all(np.abs(y - exact) <= bound + 1e-30)


@pytest.mark.parametrize("levels", [16, 256])
def test_rust_single_term_is_exact_product(levels):
    n, k, group = 7, 64, 16
    idx, packed, scale, cb = ref.synth_linear(n, k, levels, group, seed=9)
    p2 = ref.packed_2d(packed, n, k, levels)
    for kk in (0, 1, 17, 62, 63):
        x = np.zeros((1, k), np.float32)
        x[0, kk] = 1.0
        y = rowdot.dequant_matmul(x, p2, scale.astype(np.float32), cb.astype(np.float32), group,
                                  levels <= 16)
        want = cb.astype(np.float64)[idx[:, kk]] * scale.astype(np.float64)[:, kk // group]
        assert np.array_equal(y[0].astype(np.float64), want)


def test_rust_integer_sums_exact():
    n, k, group = 6, 64, 32
    r = rng(10)
    idx = r.integers(0, 16, (n, k), dtype=np.uint8)
    cb = (2.0 ** np.arange(-4, 12)).astype(np.float32)
    scale = np.ones((n, 2), np.float32)
    x = r.integers(-3, 4, (2, k)).astype(np.float32)
    y = rowdot.dequant_matmul(x, ref.pack4(idx, 16).reshape(n, k // 2), scale, cb, group, True)
    exact = x.astype(np.float64) @ cb.astype(np.float64)[idx].T
    assert np.array_equal(y.astype(np.float64), exact)


def test_rust_odd_group_pairs_nibbles_shifted():
    """kernel/src/lib.rs:71-77 with an odd group start reads the low nibble of
    byte k>>1 for x[k]; the oracle keeps that quirk."""
    idx = np.array([[1, 2, 3, 4, 5, 6]], np.uint8)
    cb = np.arange(16, dtype=np.float32)
    scale = np.ones((1, 2), np.float32)
    x = np.array([[1, 10, 100, 1000, 10000, 100000]], np.float32)
    y = rowdot.dequant_matmul(x, ref.pack4(idx, 16).reshape(1, 3), scale, cb, 3, True)
    # group 0 (k 0..2): 1*1 + 10*2 + 100*3; group 1 starts at k=3 (odd):
    # kk=3 -> byte 1 = (3, 4): x[3]*3 + x[4]*4; kk=5 -> byte 2 = (5, 6): x[5]*5
    assert y[0, 0] == 321 + 1000 * 3 + 10000 * 4 + 100000 * 5
    assert np.array_equal(ref.rust_dequant_matmul(x, ref.pack4(idx, 16).reshape(1, 3), scale,
                                                  cb, 3, True), y)


def test_rust_truncates_m_and_zero_beyond_levels():
    n, k = 4, 8
    idx = np.full((n, k), 12, np.uint8)
    cb = np.ones(10, np.float32)                   # 10 levels: idx 12 reads 0
    x = np.ones(2 * k + 3, np.float32)             # m = 19 // 8 = 2
    y = rowdot.dequant_matmul(x, ref.pack4(idx, 16).reshape(n, k // 2),
                              np.ones((n, 1), np.float32), cb, 8, True)
    assert y.shape == (2, n) and not y.any()


def test_rust_rejects_narrow_scales():
    with pytest.raises(ValueError):
        rowdot.dequant_matmul(np.ones(8, np.float32), np.zeros((1, 4), np.uint8),
                              np.ones((1, 1), np.float32), np.ones(16, np.float32), 4, True)


# ------------------------------------------------------------------ backward
def test_backward_closed_form_matches_autograd():
    n, k, group, m = 12, 48, 16, 5
    idx, _, scale, cb = ref.synth_linear(n, k, 16, group, seed=11)
    r = rng(12)
    x = r.standard_normal((m, k))
    gy = r.standard_normal((m, n))
    gx, gcb, gsc = ref.backward_f64(gy, x, idx, scale, cb, group)

    tcb = torch.tensor(cb.astype(np.float64), requires_grad=True)
    tsc = torch.tensor(scale.astype(np.float64), requires_grad=True)
    tx = torch.tensor(x, requires_grad=True)
    w = tcb[torch.from_numpy(idx.astype(np.int64))] * tsc.repeat_interleave(group, 1)
    y = tx @ w.T
    (y * torch.from_numpy(gy)).sum().backward()
    assert np.allclose(gx, tx.grad.numpy(), rtol=1e-12, atol=1e-12)
    assert np.allclose(gcb, tcb.grad.numpy(), rtol=1e-12, atol=1e-12)
    assert np.allclose(gsc, tsc.grad.numpy(), rtol=1e-12, atol=1e-12)


# ------------------------------------------------------------------ index freeze
def test_snapshot_digest_known_answer():
    assert ref.snapshot_digest(np.zeros(0, np.uint8)) == \
        hashlib.blake2b(b"", digest_size=16).hexdigest() == "cae66941d9efbd404e4d88758ea67670"
    a = np.arange(10, dtype=np.uint8)
    b = a.copy()
    b[[3, 4]] = b[[4, 3]]                         # a swap keeps the sum, not the digest
    assert ref.snapshot_digest(a) != ref.snapshot_digest(b)


# ------------------------------------------------------------------ golden fixtures
def _goldens():
    return sorted(f for f in os.listdir(GOLDEN) if f.endswith(".npz"))


@pytest.mark.parametrize("name", _goldens())
def test_oracle_reproduces_golden(name):
    g = np.load(os.path.join(GOLDEN, name))
    n, k = g["idx"].shape
    levels, group = int(g["levels"]), int(g["group"])
    assert np.array_equal(ref.pack4(g["idx"], levels), g["packed"])
    assert np.array_equal(ref.unpack4(g["packed"], n * k, levels).reshape(n, k), g["idx"])
    tile = ref.dequant_tile_f32(g["idx"], g["scale"], g["cb"], group)
    assert np.array_equal(tile, g["tile_f32"])
    x = ref.bf16_bits_to_f32(g["x_bf16"])
    y = rowdot.dequant_matmul(x, ref.packed_2d(g["packed"], n, k, levels),
                              g["scale"].astype(np.float32), g["cb"].astype(np.float32), group,
                              levels <= 16)
    assert np.array_equal(y.view(np.uint32), g["y_rust"].view(np.uint32))
    assert np.allclose(ref.linear_f64(x, tile), g["y_f64"], rtol=0, atol=0)
