"""ep_dequant_matmul_noalloc (static device scratch, no allocation) against
ep_dequant_matmul with a caller workspace: the same kernels run, so the
outputs must be bit-identical; both are also held to the Rust-order oracle
bar (max relative error 2e-3).  Two calls in a row, the second smaller, so a
stale scratch from the first call cannot leak into the second."""
import numpy as np
import pytest
import torch

from epure import PackedWeight
from epure.kernels import _abi, cuda
from oracle import ref, rowdot

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _case(n, k, m, levels, seed):
    _, packed, scale, cb = ref.synth_linear(n, k, levels, 128, seed=seed)
    s = PackedWeight((n, k), packed, scale, cb.astype(np.float32), 128, levels).to(DEV)
    x32 = ref.round_bf16(np.random.Generator(np.random.PCG64(seed + 1)).standard_normal(
        (m, k)).astype(np.float32))
    x = torch.from_numpy(x32).to(DEV).to(torch.bfloat16)
    row = k // 2 if levels <= 16 else k
    want = rowdot.dequant_matmul(x32, packed.reshape(n, row), scale.astype(np.float32),
                                 cb.astype(np.float32), 128, levels <= 16)
    return s, x, want


def _run(s, x, noalloc):
    h = cuda._hot(s)
    m, k = x.shape
    y = torch.full((m, h.N), float("nan"), device=DEV, dtype=torch.float32)
    args = [x.data_ptr(), _abi.BF16, x.stride(0), h.packed.data_ptr(), h.scale.data_ptr(),
            h.scale_dt, h.ld_scale, h.cb.data_ptr(), h.cb_dt, h.levels, h.group, m, h.N, k,
            y.data_ptr(), _abi.F32, y.stride(0), 0]
    if noalloc:
        rc = _abi.lib.ep_dequant_matmul_noalloc(*args, _abi.stream_handle(DEV))
    else:
        nb = _abi.lib.ep_dequant_matmul_workspace(m, h.N, k, h.levels, h.group)
        ws = torch.empty(max(nb, 256), device=DEV, dtype=torch.uint8)
        rc = _abi.lib.ep_dequant_matmul(*args, ws.data_ptr(), ws.numel(), _abi.stream_handle(DEV))
    assert rc == 0, _abi.last_error()
    torch.cuda.synchronize()
    return y.cpu().numpy()


# (N, K, M, levels): the split-K small-M path with partials in the scratch,
# then smaller calls through the MFMA prefill, the batch-1 GEMV and again
# the small-M path
CALLS = [(4096, 4096, 48, 16), (1024, 2048, 256, 256), (768, 1024, 1, 16), (512, 1024, 20, 16)]


def test_noalloc_matches_workspace_entry_on_consecutive_calls():
    assert _abi.lib.ep_noalloc_scratch_bytes() == 32 << 20
    for i, (n, k, m, levels) in enumerate(CALLS):
        s, x, want = _case(n, k, m, levels, seed=70 + i)
        a = _run(s, x, noalloc=True)
        b = _run(s, x, noalloc=False)
        assert np.array_equal(a, b), f"call {i}: noalloc differs from the workspace entry"
        err = np.abs(a - want).max() / np.abs(want).max()
        assert err < 2e-3, f"call {i}: normwise error {err:.2e} against the Rust-order oracle"


def test_noalloc_rejects_requests_beyond_the_scratch():
    need = _abi.lib.ep_dequant_matmul_workspace(2048, 14336, 14336, 16, 128)
    assert need > _abi.lib.ep_noalloc_scratch_bytes()
    # Null x, y and weight pointers: the size check rejects the request
    # first; were it ever skipped, the null pointers are rejected with
    # EP_ERR_ARG before any launch, so no kernel can run on them.
    rc = _abi.lib.ep_dequant_matmul_noalloc(
        None, _abi.BF16, 14336, None, None, _abi.F16, 112, None, _abi.F32, 16, 128, 2048,
        14336, 14336, None, _abi.F32, 14336, 0, _abi.stream_handle(DEV))
    assert rc == -3 and "scratch" in _abi.last_error()
    rc = _abi.lib.ep_dequant_matmul_noalloc(
        None, _abi.BF16, 512, None, None, _abi.F16, 4, None, _abi.F32, 16, 128, 1, 256, 512,
        None, _abi.F32, 256, 0, _abi.stream_handle(DEV))
    assert rc == -1 and "null" in _abi.last_error()
