"""GPU parity of the forward path through the C ABI, against the CPU oracle.

Bars: unpacked indices and dequantized tiles are
bit-exact; matmul outputs are within max relative error 2e-3 of the
reference's fp32-accumulated result (kernel/src/lib.rs order, computed by the
oracle), measured normwise (max|y-r| / max|r|) and per element with an
rms(r) floor.
"""
import os

import numpy as np
import pytest
import torch

from epure import PackedLinear, PackedWeight
from epure.kernels import _abi, cuda
from oracle import ref, rowdot

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TOL = 2e-3
# A bf16 output adds its own rounding on top: bf16 keeps 8 significant bits,
# so round-to-nearest moves a value by at most 2^-8 of itself (half an ulp of
# 2^-7) -- hence TOL + 2^-8 for bf16 outputs (normwise, so |y| <= max|y|).
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


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


def make(n, k, levels=16, group=128, seed=0, scale_dt=np.float16, cb_dt=np.float32):
    idx, packed, scale, cb = ref.synth_linear(n, k, levels, group, seed=seed)
    s = PackedWeight((n, k), packed, scale.astype(scale_dt), cb.astype(cb_dt), group,
                     levels).to(DEV)
    return idx, packed, scale, cb, s


def rust_ref(x32, packed, scale, cb, n, k, levels, group):
    return rowdot.dequant_matmul(x32, ref.packed_2d(packed, n, k, levels),
                                 np.asarray(scale, np.float32), np.asarray(cb, np.float32), group,
                                 levels <= 16)


def x_bf16(m, k, seed, scale=1.0):
    x32 = ref.round_bf16((rng(seed).standard_normal((m, k)) * scale).astype(np.float32))
    return x32, torch.from_numpy(x32).to(DEV).to(torch.bfloat16)


def run(s, x, out_dtype=torch.float32, accumulate=False, out=None):
    h = cuda._hot(s)
    x2 = x.reshape(-1, x.shape[-1])
    if out is None:
        out = torch.empty((x2.shape[0], s.out_features), device=DEV, dtype=out_dtype)
    y = cuda.forward(x2, h, out=out, accumulate=accumulate)
    assert y is not None, f"declined: {_abi.last_error()}"
    torch.cuda.synchronize()
    return y


def test_backend_available():
    assert cuda.available()
    assert _abi.lib is not None and os.path.exists(cuda.library_path())


# ------------------------------------------------------------------ bit-exact decode
@pytest.mark.parametrize("n,levels", [(1, 16), (2, 16), (4097, 16), (100000, 16), (999, 256)])
def test_unpack_bitexact(n, levels):
    nbytes = (n + 1) // 2 if levels <= 16 else n
    b = rng(n).integers(0, 256, nbytes, dtype=np.uint8)
    pd = torch.from_numpy(b).to(DEV)
    out = torch.full((n,), 0xAA, dtype=torch.uint8, device=DEV)
    rc = _abi.lib.ep_unpack_indices(pd.data_ptr(), n, levels, out.data_ptr(),
                                    _abi.stream_handle())
    assert rc == 0
    assert np.array_equal(out.cpu().numpy(), ref.unpack4(b, n, levels))


@pytest.mark.parametrize("dtype,name", [(torch.float32, "f32"), (torch.float16, "f16"),
                                        (torch.bfloat16, "bf16")])
@pytest.mark.parametrize("levels,n,k,group", [(16, 64, 512, 128), (256, 33, 256, 64),
                                              (16, 7, 9, 4), (10, 5, 40, 8)])
def test_dequant_tile_bitexact(dtype, name, levels, n, k, group):
    idx, packed, scale, _ = ref.synth_linear(n, k, levels, group, seed=n)
    cb = rng(k).standard_normal(levels).astype(np.float32)      # not fp16-valued
    sc = (scale.astype(np.float32) * np.float32(1.0003))        # f32 scales (trained)
    if levels == 10:
        idx = rng(1).integers(0, 16, (n, k), dtype=np.uint8)    # indices beyond levels read 0
        packed = ref.pack4(idx, 16)
    s = PackedWeight((n, k), packed, sc, cb, group, levels).to(DEV)
    w = s.materialize(dtype).float().cpu().numpy()
    want = ref.materialize(packed, sc, cb, n, k, group, levels, name)
    assert np.array_equal(w, want)


# ------------------------------------------------------------------ batch-1 GEMV
def test_gemv_config0_shape():
    n = k = 4096
    _, packed, scale, cb, s = make(n, k, seed=0)
    x32, x = x_bf16(1, k, 1)
    y = run(s, x).cpu().numpy()
    assert_close(y, rust_ref(x32, packed, scale, cb, n, k, 16, 128))
    yb = run(s, x, torch.bfloat16).float().cpu().numpy()
    assert_close(yb, y, tol=2.0 ** -8)


@pytest.mark.parametrize("levels", [16, 256])
@pytest.mark.parametrize("m", [1, 2, 3, 4])
@pytest.mark.parametrize("n,k", [(256, 512), (1000, 4096), (96, 14336), (40, 2048)])
def test_gemv_shapes(levels, m, n, k):
    _, packed, scale, cb, s = make(n, k, levels, seed=n + k + m)
    x32, x = x_bf16(m, k, m)
    assert_close(run(s, x).cpu().numpy(), rust_ref(x32, packed, scale, cb, n, k, levels, 128))


@pytest.mark.parametrize("xdt", [torch.float16, torch.float32])
def test_gemv_x_dtypes(xdt):
    n, k = 512, 2048
    _, packed, scale, cb, s = make(n, k, seed=5)
    x32 = rng(6).standard_normal((2, k)).astype(np.float32)
    x = torch.from_numpy(x32).to(DEV).to(xdt)
    xr = x.float().cpu().numpy()
    assert_close(run(s, x).cpu().numpy(), rust_ref(xr, packed, scale, cb, n, k, 16, 128))


def test_gemv_f32_scales_f16_cb():
    n, k = 384, 1024
    idx, packed, scale, cb = ref.synth_linear(n, k, 16, 128, seed=8)
    sc = scale.astype(np.float32) * np.float32(0.999)
    s = PackedWeight((n, k), packed, sc, cb.astype(np.float16), 128, 16).to(DEV)
    x32, x = x_bf16(1, k, 9)
    assert_close(run(s, x).cpu().numpy(), rust_ref(x32, packed, sc, cb, n, k, 16, 128))


def test_gemv_group_64_and_32():
    for group in (64, 32):
        _, packed, scale, cb, s = make(300, 1024, group=group, seed=group)
        x32, x = x_bf16(1, 1024, group)
        assert_close(run(s, x).cpu().numpy(),
                     rust_ref(x32, packed, scale, cb, 300, 1024, 16, group))


def test_gemv_levels_below_16_read_zero():
    n, k = 64, 512
    idx = rng(3).integers(0, 16, (n, k), dtype=np.uint8)
    packed = ref.pack4(idx, 16)
    cb = np.sort(rng(4).standard_normal(10)).astype(np.float16)
    scale = (np.abs(rng(5).normal(0, 0.02, (n, 4))) + 1e-3).astype(np.float16)
    s = PackedWeight((n, k), packed, scale, cb.astype(np.float32), 128, 10).to(DEV)
    x32, x = x_bf16(1, k, 6)
    assert_close(run(s, x).cpu().numpy(), rust_ref(x32, packed, scale, cb, n, k, 10, 128))


def test_gemv_large_and_tiny_activations():
    n, k = 256, 1024
    idx, packed, scale, cb, s = make(n, k, seed=11)
    w64 = ref.dequant_tile_f32(idx, scale, cb, 128).astype(np.float64)
    for mag in (3e5, 1e-12):
        x32, x = x_bf16(1, k, 12, scale=mag)
        y = run(s, x).cpu().numpy()
        assert_close(y, ref.linear_f64(x32, w64))


def test_gemv_accumulate_and_determinism():
    n, k = 512, 4096
    _, packed, scale, cb, s = make(n, k, seed=13)
    x32, x = x_bf16(1, k, 14)
    base = torch.from_numpy(rng(15).standard_normal((1, n)).astype(np.float32)).to(DEV)
    out = base.clone()
    run(s, x, accumulate=True, out=out)
    want = rust_ref(x32, packed, scale, cb, n, k, 16, 128) + base.cpu().numpy()
    assert_close(out.cpu().numpy(), want)
    a = run(s, x).cpu().numpy()
    b = run(s, x).cpu().numpy()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ------------------------------------------------------------------ MFMA and generic paths
@pytest.mark.parametrize("levels", [16, 256])
@pytest.mark.parametrize("m", [5, 16, 33, 64, 200])
def test_mfma_path(levels, m):
    n, k = 384, 1024
    _, packed, scale, cb, s = make(n, k, levels, seed=m)
    x32, x = x_bf16(m, k, m + 1)
    assert_close(run(s, x).cpu().numpy(), rust_ref(x32, packed, scale, cb, n, k, levels, 128))


def test_mfma_ragged_n_and_f32_x():
    n, k, m = 200, 512, 70
    _, packed, scale, cb, s = make(n, k, seed=21)
    x32 = rng(22).standard_normal((m, k)).astype(np.float32)
    x = torch.from_numpy(x32).to(DEV)
    assert_close(run(s, x).cpu().numpy(), rust_ref(x32, packed, scale, cb, n, k, 16, 128))


@pytest.mark.parametrize("n,k,group,levels,m", [(37, 100, 50, 16, 1), (8, 6, 2, 16, 3),
                                                (5, 96, 24, 256, 2), (3, 7, 7, 16, 1),
                                                (64, 160, 20, 16, 9)])
def test_generic_path(n, k, group, levels, m):
    idx, packed, scale, cb = ref.synth_linear(n, k, levels, group, seed=k)
    s = PackedWeight((n, k), packed, scale, cb.astype(np.float32), group, levels).to(DEV)
    x32, x = x_bf16(m, k, k + 1)
    w = ref.dequant_tile_f32(idx, scale, cb, group)     # flat-stream semantics (odd K too)
    assert_close(run(s, x).cpu().numpy(), ref.linear_f64(x32, w))


def test_empty_batch():
    _, _, _, _, s = make(64, 256, seed=1)
    x = torch.empty((0, 256), device=DEV, dtype=torch.bfloat16)
    assert run(s, x).shape == (0, 64)


# ------------------------------------------------------------------ fixtures, module, graphs
@pytest.mark.parametrize("name", sorted(f for f in os.listdir(GOLDEN) if f.endswith(".npz")))
def test_golden_fixture(name):
    g = np.load(os.path.join(GOLDEN, name))
    n, k = g["idx"].shape
    levels, group = int(g["levels"]), int(g["group"])
    s = PackedWeight((n, k), g["packed"], g["scale"], g["cb"].astype(np.float32), group,
                     levels).to(DEV)
    assert np.array_equal(s.materialize(torch.float32).cpu().numpy(), g["tile_f32"])
    x = torch.from_numpy(g["x_bf16"].view(np.int16)).to(DEV).view(torch.bfloat16)
    assert_close(run(s, x).cpu().numpy(), g["y_rust"])


def test_packed_linear_uses_fused_path(monkeypatch):
    n, k = 512, 1024
    _, packed, scale, cb, s = make(n, k, seed=31)
    lin = PackedLinear(s, bias=torch.ones(n, device=DEV, dtype=torch.bfloat16))

    def boom(*a, **kw):
        raise AssertionError("materialize called: fused path not taken")
    monkeypatch.setattr(s, "materialize", boom)
    x32, x = x_bf16(3, k, 32)
    y = lin(x.view(1, 3, k))
    assert y.shape == (1, 3, n) and y.dtype == torch.bfloat16
    want = rust_ref(x32, packed, scale, cb, n, k, 16, 128) + 1.0
    assert_close(y.float().cpu().numpy().reshape(3, n), want, tol=TOL + 2.0 ** -8)


def test_graph_capture_replays():
    n, k = 1024, 4096
    _, packed, scale, cb, s = make(n, k, seed=41)
    h = cuda._hot(s)
    xs = torch.zeros((1, k), device=DEV, dtype=torch.bfloat16)
    ys = torch.zeros((1, n), device=DEV, dtype=torch.float32)
    cuda.forward(xs, h, out=ys)               # warm-up outside capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        cuda.forward(xs, h, out=ys)
    for i in range(4):
        x32, x = x_bf16(1, k, 100 + i)
        xs.copy_(x)
        g.replay()
        torch.cuda.synchronize()
        eager = run(s, x).cpu().numpy()
        assert np.array_equal(ys.cpu().numpy(), eager)
        assert_close(eager, rust_ref(x32, packed, scale, cb, n, k, 16, 128))
