"""GPU parity at the exact shapes of the config-3 sweep: the 8B-shaped
linears 4096x4096, 14336x4096 and 4096x14336 with 8-bit indices (256-entry
fp16 codebook, group-128 fp16 scales), bf16 activations, and every M of the
sweep {1, 4, 16, 64, 512, 2048}.

At these N and K the launch geometry (GEMV row blocks, the one-launch
small-M tiles, the split-K depth, the prefill tiling and K split) differs
from the smaller shapes of the other test files, so each full-size case is
checked here.

Oracles: the float64 product with the exact f32 dequantized tile
(container.py:70-88, oracle/decoder.py dense_tile, pinned bit for bit to
oracle.ref.dequant_tile_f32 in tests/test_oracle.py) for every M, and the C
restatement of the reference Rust kernel (kernel/src/lib.rs:36-151,
oracle/rowdot.c) for M <= 16.  Bar: max relative error 2e-3, normwise and
per element with an rms floor (the north-star matmul tolerance).
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
SHAPES = [(4096, 4096), (14336, 4096), (4096, 14336)]   # (N, K)
MS = [1, 4, 16, 64, 512, 2048]


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


_STORES = {}


def store(n, k):
    """The config-3 weight of shape (n, k) (seeded; built once per module)."""
    key = (n, k)
    if key not in _STORES:
        _STORES.clear()     # one full-size weight resident at a time
        _, packed, scale, cb = ref.synth_linear(n, k, 256, 128, seed=n + 3 * k)
        s = PackedWeight((n, k), packed, scale, cb.astype(np.float32), 128, 256).to(DEV)
        w64 = dense_tile(s.packed, s.scale, s.cb, n, k, 128, 256).double()
        _STORES[key] = (packed, scale, cb, s, w64)
    return _STORES[key]


@pytest.mark.parametrize("m", MS)
@pytest.mark.parametrize("n,k", SHAPES)
def test_config3_shape(n, k, m):
    packed, scale, cb, s, w64 = store(n, k)
    x32 = ref.round_bf16(rng(m * 7 + n + k).standard_normal((m, k)).astype(np.float32))
    x = torch.from_numpy(x32).to(DEV).to(torch.bfloat16)
    print(f"case: config 3 N={n} K={k} M={m} 8-bit bf16 x", flush=True)
    h = cuda._hot(s)
    y = cuda.forward(x, h, out=torch.empty((m, n), device=DEV, dtype=torch.float32))
    assert y is not None, f"declined: {_abi.last_error()}"
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    want = (x.double() @ w64.t()).cpu().numpy()
    assert_close(y, want)
    if m <= 16:
        rust = rowdot.dequant_matmul(x32, ref.packed_2d(packed, n, k, 256), scale.astype(np.float32),
                                     cb.astype(np.float32), 128, False)
        assert_close(y, rust)


@pytest.fixture(scope="module", autouse=True)
def _free_stores():
    yield
    _STORES.clear()
