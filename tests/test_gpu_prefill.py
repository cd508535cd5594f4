"""GPU parity of the prefill path (more than 64 activation rows) through the C ABI.

Oracles: the C restatement of the reference Rust kernel (kernel/src/lib.rs,
oracle/rowdot.c) where it finishes in seconds, and the closed form
y = x . (cb[idx] * scale)^T in float64 on the GPU (the exact f32 tile of
container.py:70-88, oracle/decoder.py dense_tile) for the large shapes.
Bar: max relative error 2e-3, normwise and per element with an rms floor.
The cases cover both tile heights (64 and 128 rows), K split into several
partial sums, N past the last 256-row tile, every x and output dtype,
accumulation, group sizes, and rows of very different magnitude.
"""
import numpy as np
import pytest
import torch

from epure import PackedWeight
from epure.kernels import _abi, cuda
from oracle import ref, rowdot
from oracle.decoder import dense_tile

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TOL = 2e-3
# A bf16 output adds its own rounding on top: bf16 keeps 8 significant bits,
# so round-to-nearest moves a value by at most 2^-8 of itself (half an ulp of
# 2^-7) -- hence TOL + 2^-8 for bf16 outputs (normwise, so |y| <= max|y|).


def rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def assert_close(y, r, tol=TOL):
    y = np.asarray(y, np.float64)
    r = np.asarray(r, np.float64)
    assert y.shape == r.shape
    assert np.isfinite(y).all()
    err = np.abs(y - r)
    scale = np.abs(r).max()
    assert err.max() <= tol * scale, f"normwise {err.max() / scale:.3e}"
    floor = np.sqrt(np.mean(r ** 2))
    rel = (err / np.maximum(np.abs(r), floor)).max()
    assert rel <= tol, f"per-element {rel:.3e}"


def make(n, k, levels=16, group=128, seed=0):
    idx, packed, scale, cb = ref.synth_linear(n, k, levels, group, seed=seed)
    s = PackedWeight((n, k), packed, scale, cb.astype(np.float32), group, levels).to(DEV)
    return idx, packed, scale, cb, s


def rust_ref(x32, packed, scale, cb, n, k, levels, group):
    return rowdot.dequant_matmul(x32, ref.packed_2d(packed, n, k, levels),
                                 np.asarray(scale, np.float32), np.asarray(cb, np.float32), group,
                                 levels <= 16)


def f64_ref(x, s):
    """x . W^T in float64 on the GPU, W the exact f32 dequantized tile."""
    w = dense_tile(s.packed, s.scale, s.cb, s.out_features, s.in_features, s.group, s.levels)
    return (x.double() @ w.double().t()).cpu().numpy()


def x_bf16(m, k, seed, scale=1.0):
    x32 = ref.round_bf16((rng(seed).standard_normal((m, k)) * scale).astype(np.float32))
    return x32, torch.from_numpy(x32).to(DEV).to(torch.bfloat16)


def run(s, x, out_dtype=torch.float32, accumulate=False, out=None):
    print(f"case: N={s.out_features} K={s.in_features} M={x.shape[0]} levels={s.levels} "
          f"group={s.group} x={x.dtype} y={out_dtype} acc={accumulate}", flush=True)
    h = cuda._hot(s)
    if out is None:
        out = torch.empty((x.shape[0], s.out_features), device=DEV, dtype=out_dtype)
    y = cuda.forward(x, h, out=out, accumulate=accumulate)
    assert y is not None, f"declined: {_abi.last_error()}"
    torch.cuda.synchronize()
    return y


@pytest.mark.parametrize("levels", [16, 256])
@pytest.mark.parametrize("m", [65, 100, 256])
def test_prefill_vs_rust_order(levels, m):
    n, k = 300, 1024
    _, packed, scale, cb, s = make(n, k, levels, seed=m + levels)
    x32, x = x_bf16(m, k, m)
    assert_close(run(s, x).cpu().numpy(), rust_ref(x32, packed, scale, cb, n, k, levels, 128))


@pytest.mark.parametrize("levels", [16, 256])
@pytest.mark.parametrize("m,n,k", [(1024, 1024, 4096), (1500, 520, 2048), (128, 256, 8192),
                                   (2048, 256, 14336)])
def test_prefill_large_and_split(levels, m, n, k):
    """128-row tiles (4-bit, M >= 1024), ragged M and N, and small grids
    whose K is split into partial sums."""
    _, _, _, _, s = make(n, k, levels, seed=n + k + m)
    _, x = x_bf16(m, k, k + m)
    assert_close(run(s, x).cpu().numpy(), f64_ref(x, s))


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,k", [(96, 512), (160, 8192)])
def test_prefill_accumulate_and_out_dtypes(out_dtype, m, k):
    """One split (accumulation in the epilogue) and several (through the
    ordered reduction)."""
    n = 384
    _, _, _, _, s = make(n, k, seed=k + 1)
    _, x = x_bf16(m, k, k + 2)
    want = f64_ref(x, s)
    out_tol = TOL if out_dtype == torch.float32 else TOL + 2.0 ** -8
    assert_close(run(s, x, out_dtype).float().cpu().numpy(), want, out_tol)
    base = torch.from_numpy(rng(k + 3).standard_normal((m, n)).astype(np.float32)).to(DEV)
    out = base.to(out_dtype)
    start = out.float().cpu().numpy()
    run(s, x, out_dtype, accumulate=True, out=out)
    assert_close(out.float().cpu().numpy(), want + start, out_tol)


@pytest.mark.parametrize("xdt", [torch.float16, torch.float32])
def test_prefill_x_dtypes(xdt):
    n, k, m = 512, 2048, 200
    _, packed, scale, cb, s = make(n, k, seed=31)
    x32 = rng(32).standard_normal((m, k)).astype(np.float32)
    x = torch.from_numpy(x32).to(DEV).to(xdt)
    assert_close(run(s, x).cpu().numpy(), f64_ref(x, s))


@pytest.mark.parametrize("m", [80, 300])
@pytest.mark.parametrize("group,levels", [(32, 16), (64, 16), (16, 256), (256, 256), (96, 16), (48, 256)])
def test_prefill_groups(group, levels, m):
    """Both tilings: 64 activation rows x 64 weight rows per wave, and 128
    activation rows x 32 weight rows per wave (M >= 256).  Groups that
    neither divide the 64-wide k step nor are 64 * 2^i (96, 48) are served by
    the generic MFMA path."""
    n, k = 300, 1024 if 1024 % group == 0 else 1152
    _, packed, scale, cb, s = make(n, k, levels, group=group, seed=group)
    x32, x = x_bf16(m, k, group)
    assert_close(run(s, x).cpu().numpy(), rust_ref(x32, packed, scale, cb, n, k, levels, group))


def test_prefill_levels_below_16_read_zero():
    n, k, m = 64, 512, 70
    idx = rng(3).integers(0, 16, (n, k), dtype=np.uint8)
    packed = ref.pack4(idx, 16)
    cb = np.sort(rng(4).standard_normal(10)).astype(np.float16)
    scale = (np.abs(rng(5).normal(0, 0.02, (n, 4))) + 1e-3).astype(np.float16)
    s = PackedWeight((n, k), packed, scale, cb.astype(np.float32), 128, 10).to(DEV)
    x32, x = x_bf16(m, k, 6)
    assert_close(run(s, x).cpu().numpy(), rust_ref(x32, packed, scale, cb, n, k, 10, 128))


def test_prefill_rows_of_very_different_magnitude():
    n, k, m = 256, 2048, 80
    _, _, _, _, s = make(n, k, seed=41)
    mags = np.ones(m, np.float32)
    mags[:4] = [3e5, 1e-12, 1e-30, 0.0]
    x32 = ref.round_bf16((rng(42).standard_normal((m, k)) * mags[:, None]).astype(np.float32))
    x = torch.from_numpy(x32).to(DEV).to(torch.bfloat16)
    y = run(s, x).cpu().numpy()
    want = f64_ref(x, s)
    for r in [0, 1, 2] + list(range(4, m)):
        assert_close(y[r:r + 1], want[r:r + 1])
    assert np.all(y[3] == 0.0)


def test_prefill_deterministic():
    n, k, m = 512, 8192, 128  # split K
    _, _, _, _, s = make(n, k, seed=51)
    _, x = x_bf16(m, k, 52)
    a = run(s, x).cpu().numpy()
    b = run(s, x).cpu().numpy()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_batch1_8bit_long_k_stays_on_the_gemv():
    """Batch-1 8-bit at K = 14336 is served by the LUT GEMV (~22 us per
    4096 x 14336 launch); a shape-check slip once routed it to the MFMA tile
    path (~450 us).  The bar leaves 2.5x headroom over the GEMV's time."""
    n, k = 4096, 14336
    _, packed, scale, cb = ref.synth_linear(n, k, 256, 128, seed=77)
    s = PackedWeight((n, k), packed, scale, cb.astype(np.float32), 128, 256).to(DEV)
    x = torch.randn(1, k, device=DEV).to(torch.bfloat16)
    h = cuda._hot(s)
    for _ in range(3):
        cuda.forward(x, h)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(20):
        cuda.forward(x, h)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) / 20 * 1e3
    assert us < 60.0, f"{us:.1f} us per launch"
