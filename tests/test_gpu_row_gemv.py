"""GPU parity of the row GEMV (`gemv_row_kernel`) at every row length it
serves: rows of 4, 8, 12, 16, 24, 28 and 32 slabs of 256 bytes (and 56 with
8-bit indices), i.e. K = 2048 .. 16384 with 4-bit indices and 1024 .. 14336
with 8-bit.  A wave owns whole rows: 1, 2 or 4 rows per wave and 3 to 14
loads per lane, activations staged by 1 or 2 chunks per thread; rows of 4, 8
and 16 slabs also take 2..4 activation rows per launch, which share each
load's table lookups.

Oracle: the C restatement of the reference Rust kernel (kernel/src/lib.rs:
36-151, oracle/rowdot.c).  Bar: max relative error 2e-3, normwise and per
element with an rms floor (bf16 / fp16 outputs add their own rounding).
"""
import numpy as np
import pytest
import torch

from epure import PackedWeight
from epure.kernels import _abi, cuda
from oracle import ref, rowdot

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TOL = 2e-3


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


def case(n, k, levels, x_dtype, scale_f32, seed, out_dtype=torch.float32, accumulate=False):
    _, packed, scale, cb = ref.synth_linear(n, k, levels, 128, seed=seed)
    s = PackedWeight((n, k), packed, scale.astype(np.float32 if scale_f32 else np.float16),
                     cb.astype(np.float32), 128, levels).to(DEV)
    x32 = rng(seed + 1).standard_normal((1, k)).astype(np.float32)
    if x_dtype == torch.bfloat16:
        x32 = ref.round_bf16(x32)
    x = torch.from_numpy(x32).to(DEV).to(x_dtype)
    x_in = x.float().cpu().numpy()
    want = rowdot.dequant_matmul(x_in, ref.packed_2d(packed, n, k, levels), np.asarray(scale, np.float32),
                                 np.asarray(cb, np.float32), 128, levels <= 16)
    print(f"case: row GEMV N={n} K={k} levels={levels} x={x_dtype} f32 scales={scale_f32} "
          f"y={out_dtype} acc={accumulate}", flush=True)
    h = cuda._hot(s)
    out = torch.from_numpy(rng(seed + 2).standard_normal((1, n)).astype(np.float32)).to(DEV).to(out_dtype)
    start = out.float().cpu().numpy()
    y = cuda.forward(x, h, out=out, accumulate=accumulate)
    assert y is not None, f"declined: {_abi.last_error()}"
    torch.cuda.synchronize()
    tol = TOL if out_dtype == torch.float32 else TOL + 2.0 ** -8
    assert_close(out.float().cpu().numpy(), want + (start if accumulate else 0.0), tol)


# (levels, K): slabs of a row = K / 512 (4-bit) or K / 256 (8-bit)
ROWS = [(16, 2048), (16, 4096), (16, 6144), (16, 8192), (16, 12288), (16, 14336), (16, 16384),
        (256, 1024), (256, 3072), (256, 4096), (256, 6144), (256, 7168), (256, 8192), (256, 14336)]


@pytest.mark.parametrize("levels,k", ROWS)
@pytest.mark.parametrize("x_dtype", [torch.bfloat16, torch.float32])
def test_row_gemv_lengths(levels, k, x_dtype):
    """Every row length, a ragged N (not a multiple of any workgroup's rows),
    bf16 activations and f32 ones (hi and lo fp16 terms)."""
    case(300, k, levels, x_dtype, False, seed=k + levels)


@pytest.mark.parametrize("levels,k", [(16, 6144), (16, 14336), (256, 14336)])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_row_gemv_f32_scales_and_accumulate(levels, k, out_dtype):
    """f32 group scales (after make_trainable: one 32-bit load per scale) and
    accumulation into y, fp16 activations."""
    case(1000, k, levels, torch.float16, True, seed=3 * k + levels, out_dtype=out_dtype, accumulate=True)


def case_m(m, n, k, levels, x_dtype, seed, out_dtype=torch.float32, accumulate=False, ld_pad=0):
    _, packed, scale, cb = ref.synth_linear(n, k, levels, 128, seed=seed)
    s = PackedWeight((n, k), packed, scale.astype(np.float16), cb.astype(np.float32), 128, levels).to(DEV)
    x32 = rng(seed + 1).standard_normal((m, k + ld_pad)).astype(np.float32)
    if x_dtype == torch.bfloat16:
        x32 = ref.round_bf16(x32)
    wide = torch.from_numpy(x32).to(DEV).to(x_dtype)
    x = wide[:, :k]
    x_in = x.float().cpu().numpy()
    want = rowdot.dequant_matmul(np.ascontiguousarray(x_in), ref.packed_2d(packed, n, k, levels),
                                 np.asarray(scale, np.float32), np.asarray(cb, np.float32), 128, levels <= 16)
    print(f"case: row GEMV M={m} N={n} K={k} levels={levels} x={x_dtype} y={out_dtype} "
          f"acc={accumulate} ld={k + ld_pad}", flush=True)
    h = cuda._hot(s)
    out = torch.from_numpy(rng(seed + 2).standard_normal((m, n)).astype(np.float32)).to(DEV).to(out_dtype)
    start = out.float().cpu().numpy()
    y = cuda.forward(x, h, out=out, accumulate=accumulate)
    assert y is not None, f"declined: {_abi.last_error()}"
    torch.cuda.synchronize()
    tol = TOL if out_dtype == torch.float32 else TOL + 2.0 ** -8
    assert_close(out.float().cpu().numpy(), want + (start if accumulate else 0.0), tol)


# rows of 4, 8 and 16 slabs with 2..4 activation rows (the row kernel takes
# up to 4 with 4-bit indices, 2 with 4-bit rows of 16 slabs and with 8-bit
# indices; the other cases check the kernels that serve them instead)
@pytest.mark.parametrize("levels,k,m", [(16, 2048, 2), (16, 2048, 4), (16, 4096, 3), (16, 8192, 2),
                                        (256, 1024, 2), (256, 2048, 2), (256, 4096, 2), (256, 4096, 4)])
@pytest.mark.parametrize("x_dtype", [torch.bfloat16, torch.float16])
def test_row_gemv_several_rows(levels, k, m, x_dtype):
    """2, 3 (a zero-padded fourth row) and 4 activation rows share each
    load's table lookups; ragged N."""
    case_m(m, 300, k, levels, x_dtype, seed=7 * k + m + levels)


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_row_gemv_several_rows_strided_accumulate(out_dtype):
    """Activation rows further apart than K, results added into y."""
    case_m(4, 1000, 4096, 16, torch.bfloat16, seed=91, out_dtype=out_dtype, accumulate=True, ld_pad=96)
    case_m(2, 1000, 4096, 256, torch.bfloat16, seed=92, out_dtype=out_dtype, accumulate=True, ld_pad=96)
