"""The product CPU backend (libepure_cpu.so behind epure.kernels.cpu)
against the oracle's C restatement of the reference Rust kernel
(oracle/rowdot.c, kernel/src/lib.rs:36-151): bit-identical results, the
same m truncation and the same failures; and the PackedLinear routing on
CPU (reference epure/kernels/cpu.py:37-70, runtime.py:117-118)."""
import numpy as np
import pytest
import torch

from epure import PackedLinear, PackedWeight, make_trainable
from epure import runtime
from epure.kernels import cpu
from oracle import ref, rowdot


def case(n, k, levels, group, m, seed):
    idx, packed, scale, cb = ref.synth_linear(n, k, levels, group, seed=seed)
    row = k // 2 if levels <= 16 else k
    rng = np.random.Generator(np.random.PCG64(seed + 1))
    x = rng.standard_normal((m, k)).astype(np.float32)
    return x, packed.reshape(n, row), scale.astype(np.float32), cb.astype(np.float32)


@pytest.mark.parametrize("n,k,levels,group,m", [
    (64, 256, 16, 128, 1), (37, 96, 16, 32, 3), (9, 4096, 16, 128, 2), (100, 160, 10, 64, 5),
    (24, 256, 256, 128, 4), (8, 96, 200, 96, 1), (13, 100, 16, 50, 2), (5, 7, 16, 7, 1)])
@pytest.mark.parametrize("threads", [1, 3])
def test_bit_identical_to_oracle(n, k, levels, group, m, threads):
    if levels <= 16 and k % 2:
        pytest.skip("4-bit rows of odd length have no [n, k/2] view")
    x, packed, scale, cb = case(n, k, levels, group, m, seed=n + k + m)
    got = cpu.dequant_matmul(x, packed, scale, cb, group, levels <= 16, nthreads=threads)
    want = rowdot.dequant_matmul(x, packed, scale, cb, group, levels <= 16, nthreads=1)
    assert got.dtype == np.float32 and got.shape == want.shape == (m, n)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_odd_group_end_and_nibble_guard():
    # a group boundary inside a byte: the high nibble of the group's last
    # byte is skipped and the next group starts on it (lib.rs:71-78)
    x, packed, scale, cb = case(16, 96, 16, 3, 2, seed=5)
    got = cpu.dequant_matmul(x, packed, scale, cb, 3, True)
    want = rowdot.dequant_matmul(x, packed, scale, cb, 3, True)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_m_truncates_like_the_reference():
    x, packed, scale, cb = case(8, 64, 16, 32, 3, seed=9)
    xs = x.reshape(-1)[:-5]                 # 187 floats -> m = 187 // 64 = 2
    got = cpu.dequant_matmul(xs, packed, scale, cb, 32, True)
    assert got.shape == (2, 8)
    assert np.array_equal(got, rowdot.dequant_matmul(xs, packed, scale, cb, 32, True))


def test_errors_where_the_reference_raises():
    x, packed, scale, cb = case(8, 64, 16, 32, 1, seed=2)
    with pytest.raises(ValueError, match="scale columns"):
        cpu.dequant_matmul(x, packed, scale[:, :1], cb, 32, True)
    with pytest.raises(ValueError, match="levels"):
        cpu.dequant_matmul(x, packed, scale, np.zeros(300, np.float32), 32, True)


def test_threads_reports_pool_size(monkeypatch):
    assert cpu.threads() >= 1


def _store(n, k, seed):
    idx, packed, scale, cb = ref.synth_linear(n, k, 16, 128, seed=seed)
    return PackedWeight((n, k), packed, scale, cb.astype(np.float32), 128, 16)


def test_packed_linear_routes_f32_to_the_cpu_kernel(monkeypatch):
    s = _store(48, 256, seed=11)
    x = torch.randn(2, 3, 256)
    calls = []
    real = cpu.dequant_matmul
    monkeypatch.setattr(cpu, "dequant_matmul", lambda *a, **k: calls.append(1) or real(*a, **k))
    y = PackedLinear(s)(x)
    assert calls == [1] and y.shape == (2, 3, 48)
    want = rowdot.dequant_matmul(x.reshape(-1, 256).numpy(), s.packed_2d().numpy(),
                                 s.scale.float().numpy(), s.cb.numpy(), 128, True)
    assert np.array_equal(y.reshape(-1, 48).numpy(), want)


def test_cache_follows_replaced_and_updated_tensors():
    s = _store(16, 256, seed=12)
    lin = PackedLinear(s)
    x = torch.randn(1, 256)
    with torch.no_grad():
        y0 = lin(x)
        make_trainable(torch.nn.Sequential(lin), "scale", verbose=False)  # scale swapped
        s.scale.mul_(2.0)                                                 # then updated in place
        y1 = lin(x)
    assert len(runtime._BUFFER_CACHE) >= 1
    assert torch.allclose(y1, 2 * y0, rtol=1e-6, atol=1e-6)


def test_declines_with_grad_so_gradients_flow():
    s = _store(16, 256, seed=13)
    lin = PackedLinear(s)
    make_trainable(torch.nn.Sequential(lin), "both", verbose=False)
    x = torch.randn(2, 256)
    assert cpu.linear(x, s, {}) is None      # cb/scale need grad: materialize route
    lin(x).sum().backward()
    assert s.cb.grad is not None and s.scale.grad is not None
