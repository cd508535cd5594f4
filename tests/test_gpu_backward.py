"""Fused compressed-state backward against the closed forms
(fine-tuning/README.md:62-68), float64 references.

grad_x = gy W; G = gy^T x; grad_scale[n, g] = sum_{k in g} G[n, k]
cb[idx[n, k]]; grad_cb[l] = sum_{idx == l} G[n, k] scale[n, g(k)].
Indices must be bit-identical before and after.

Two routes serve it: below 512 tokens the fused kernels (dx_kernel,
dw_kernel) keep each G tile in accumulators and never write G or W; from
512 tokens (N, K >= 256) the library route materializes W as fp16 and
writes G as f32 [N, K] into the caller's workspace.  Both are checked at
token counts on either side of the switch and at the config-4 shapes.
"""
import hashlib

import numpy as np
import pytest
import torch

from epure import PackedLinear, PackedWeight, make_trainable, snapshot_indices, verify_frozen
from epure.kernels import _abi, cuda
from oracle import ref
from oracle.decoder import dense_tile

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def make(n, k, group=128, seed=0):
    idx, packed, scale, cb = ref.synth_linear(n, k, 16, group, seed=seed)
    s = PackedWeight((n, k), packed, scale, cb.astype(np.float32), group, 16).to(DEV)
    return idx, packed, scale, cb, s


def bf16(shape, seed, std=1.0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return (torch.randn(*shape, generator=g, device=DEV) * std).to(torch.bfloat16)


def closed_forms_t64(gy, x, s):
    """float64 torch restatement of the closed forms (on the GPU)."""
    n, k, grp = s.out_features, s.in_features, s.group
    w = dense_tile(s.packed, s.scale, s.cb, n, k, grp, 16).double()
    gy64, x64 = gy.double(), x.double()
    gx = gy64 @ w
    G = gy64.t() @ x64
    both = torch.stack((s.packed & 0x0F, s.packed >> 4), -1).reshape(-1)[:n * k]
    idx = both.reshape(n, k).long()
    cbd = s.cb.double()
    gsc = (G * cbd[idx]).view(n, k // grp, grp).sum(-1)
    sfull = s.scale.double().repeat_interleave(grp, 1)
    gcb = torch.zeros(16, dtype=torch.float64, device=DEV).index_add_(
        0, idx.reshape(-1), (G * sfull).reshape(-1))
    return gx, gcb, gsc


def rel(a, b):
    return float((a.double() - b).abs().max() / b.abs().max())


def run_bwd(s, gy, x, gx_dtype=torch.float32):
    h = cuda._hot(s)
    r = cuda.backward(gy, x, h, gx_dtype=gx_dtype)
    assert r is not None, _abi.last_error()
    torch.cuda.synchronize()
    return r


@pytest.mark.parametrize("n,k,m,group", [(256, 512, 64, 128), (384, 1024, 100, 64),
                                         (208, 256, 33, 32), (128, 128, 1, 128),
                                         (320, 640, 130, 128)])
def test_backward_small_vs_closed_forms(n, k, m, group):
    idx, packed, scale, cb, s = make(n, k, group, seed=n + k)
    x, gy = bf16((m, k), 1), bf16((m, n), 2, 1e-2)
    gx, gcb, gsc = run_bwd(s, gy, x)
    # numpy float64 oracle (oracle/ref.py backward_f64) on the same bf16 values
    wgx, wgcb, wgsc = ref.backward_f64(gy.float().cpu().numpy(), x.float().cpu().numpy(), idx,
                                       scale, cb, group)
    assert rel(gx.float().cpu(), torch.from_numpy(wgx)) < 2e-3
    assert rel(gsc.cpu(), torch.from_numpy(wgsc)) < 1e-4
    assert rel(gcb.cpu(), torch.from_numpy(wgcb)) < 1e-4


@pytest.mark.parametrize("n,k,m,group", [(512, 1024, 131, 128), (384, 768, 257, 64),
                                         (256, 2048, 384, 32), (1024, 512, 511, 128)])
def test_backward_fused_route_mid_tokens(n, k, m, group):
    """Token counts 131..511: the fused kernels (G kept in accumulators) with
    several 128-token tiles, ragged last tiles and the grad_x K split."""
    idx, packed, scale, cb, s = make(n, k, group, seed=n + 2 * k + m)
    x, gy = bf16((m, k), 13), bf16((m, n), 14, 1e-2)
    print(f"case: fused backward N={n} K={k} M={m} group={group}", flush=True)
    gx, gcb, gsc = run_bwd(s, gy, x)
    wgx, wgcb, wgsc = ref.backward_f64(gy.float().cpu().numpy(), x.float().cpu().numpy(), idx,
                                       scale, cb, group)
    assert rel(gx.float().cpu(), torch.from_numpy(wgx)) < 2e-3
    assert rel(gsc.cpu(), torch.from_numpy(wgsc)) < 1e-4
    assert rel(gcb.cpu(), torch.from_numpy(wgcb)) < 1e-4


@pytest.mark.parametrize("m", [384, 511])
@pytest.mark.parametrize("n,k", [(2048, 6144), (6144, 2048)])
def test_backward_config4_shapes_fused_route(n, k, m):
    """The config-4 weights below 512 tokens (the fused route) against the
    float64 closed forms; deterministic; indices untouched."""
    _, _, _, _, s = make(n, k, seed=17)
    before = hashlib.blake2b(s.packed.cpu().numpy().tobytes(), digest_size=16).hexdigest()
    x, gy = bf16((m, k), 23), bf16((m, n), 24, 1e-2)
    print(f"case: fused backward config-4 N={n} K={k} M={m}", flush=True)
    gx, gcb, gsc = run_bwd(s, gy, x)
    wgx, wgcb, wgsc = closed_forms_t64(gy, x, s)
    assert rel(gx.float(), wgx) < 2e-3
    assert rel(gsc, wgsc) < 1e-4
    assert rel(gcb, wgcb) < 1e-4
    a = run_bwd(s, gy, x)
    assert all(torch.equal(p, q) for p, q in zip((gx, gcb, gsc), a))   # deterministic
    after = hashlib.blake2b(s.packed.cpu().numpy().tobytes(), digest_size=16).hexdigest()
    assert before == after


@pytest.mark.parametrize("n,k,m,group", [(384, 640, 600, 64), (256, 384, 512, 32),
                                         (272, 1152, 1030, 128)])
def test_backward_library_route_vs_closed_forms(n, k, m, group):
    """From 512 tokens grad_x and G are library GEMMs (W materialized to
    fp16, gy prescaled per row) finished by this library's kernels; K not a
    multiple of 256 exercises the epilogue's partial steps."""
    idx, packed, scale, cb, s = make(n, k, group, seed=n + k + m)
    x, gy = bf16((m, k), 11), bf16((m, n), 12, 1e-2)
    gx, gcb, gsc = run_bwd(s, gy, x)
    wgx, wgcb, wgsc = ref.backward_f64(gy.float().cpu().numpy(), x.float().cpu().numpy(), idx,
                                       scale, cb, group)
    assert rel(gx.float().cpu(), torch.from_numpy(wgx)) < 2e-3
    assert rel(gsc.cpu(), torch.from_numpy(wgsc)) < 1e-4
    assert rel(gcb.cpu(), torch.from_numpy(wgcb)) < 1e-4
    again = run_bwd(s, gy, x)
    assert all(torch.equal(p, q) for p, q in zip((gx, gcb, gsc), again))   # deterministic


@pytest.mark.parametrize("n,k", [(2048, 6144), (6144, 2048)])
def test_backward_config4(n, k):
    _, packed, _, _, s = make(n, k, seed=7)
    before = hashlib.blake2b(s.packed.cpu().numpy().tobytes(), digest_size=16).hexdigest()
    x, gy = bf16((2048, k), 3), bf16((2048, n), 4, 1e-2)
    gx, gcb, gsc = run_bwd(s, gy, x)
    wgx, wgcb, wgsc = closed_forms_t64(gy, x, s)
    assert rel(gx.float(), wgx) < 2e-3
    assert rel(gsc, wgsc) < 1e-4
    assert rel(gcb, wgcb) < 1e-4
    after = hashlib.blake2b(s.packed.cpu().numpy().tobytes(), digest_size=16).hexdigest()
    assert before == after
    a = run_bwd(s, gy, x)
    assert all(torch.equal(p, q) for p, q in zip((gx, gcb, gsc), a))   # deterministic
    gxb = run_bwd(s, gy, x, torch.bfloat16)[0]
    assert rel(gxb.float(), wgx) < 2e-3 + 2.0 ** -8


def test_autograd_through_packed_linear(monkeypatch):
    n, k, m = 512, 1024, 48
    _, _, _, _, s = make(n, k, seed=9)
    lin = PackedLinear(s)
    model = torch.nn.Sequential(lin)
    snap = snapshot_indices(model)
    make_trainable(model, "both", verbose=False)

    def boom(*a, **kw):
        raise AssertionError("materialize called: fused forward/backward not taken")
    monkeypatch.setattr(s, "materialize", boom)
    x = bf16((m, k), 5).requires_grad_(True)
    gy = bf16((m, n), 6, 1e-2)
    y = lin(x)
    y.backward(gy)
    monkeypatch.undo()
    # reference: autograd through a float64 materialize of the same weight
    cb64 = s.cb.detach().double().requires_grad_(True)
    sc64 = s.scale.detach().double().requires_grad_(True)
    both = torch.stack((s.packed & 0x0F, s.packed >> 4), -1).reshape(-1)[:n * k]
    w = cb64[both.reshape(n, k).long()] * sc64.repeat_interleave(128, 1)
    x64 = x.detach().double().requires_grad_(True)
    (x64 @ w.t()).backward(gy.double())
    assert rel(x.grad.float(), x64.grad) < 2e-3 + 2.0 ** -8    # bf16 output
    assert rel(s.cb.grad, cb64.grad) < 1e-4
    assert rel(s.scale.grad, sc64.grad) < 1e-4
    assert verify_frozen(model, snap)


def test_backward_declines_unserved():
    _, _, _, _, s = make(128, 256, seed=1)
    h = cuda._hot(s)
    x = torch.randn(4, 256, device=DEV)                 # f32 activations: declined
    gy = torch.randn(4, 128, device=DEV)
    assert cuda.backward(gy, x, h) is None
    assert cuda.linear(x.requires_grad_(True), s) is None   # autograd: falls back to materialize


def test_autograd_zero_rows_gives_zero_grads():
    """An empty batch through a trainable bf16 PackedLinear: grads are the
    sums over no tokens (zeros), grad_x is empty."""
    _, _, _, _, s = make(256, 512, seed=31)
    lin = PackedLinear(s)
    make_trainable(torch.nn.Sequential(lin), "both", verbose=False)
    s.cb.grad = torch.full_like(s.cb, 7.0)           # stale values must be replaced,
    s.scale.grad = None                              # not accumulated into
    x = torch.zeros((0, 512), device=DEV, dtype=torch.bfloat16, requires_grad=True)
    y = lin(x)
    assert y.shape == (0, 256)
    y.float().sum().backward()
    torch.cuda.synchronize()
    assert x.grad.shape == (0, 512)
    assert torch.all(s.scale.grad == 0)
    assert torch.all(s.cb.grad == 7.0)               # autograd accumulates a zero grad


def test_fp32_activations_take_the_exact_route():
    """fp32 x is declined by the fused backend (the kernels use fp16
    operands), so PackedLinear computes it with the fp32 materialized
    weight: float32 accuracy, not fp16-operand accuracy."""
    idx, packed, scale, cb, s = make(384, 1024, seed=33)
    g = torch.Generator(device=DEV).manual_seed(34)
    x = torch.randn(3, 1024, generator=g, device=DEV)
    assert cuda.linear(x, s) is None
    with torch.no_grad():
        y = PackedLinear(s)(x).double()
    w = dense_tile(s.packed, s.scale, s.cb, 384, 1024, 128, 16).double()
    want = x.double() @ w.t()
    assert rel(y, want) < 1e-5


def test_backward_library_route_graph_replays():
    """The library route's two chains (grad_x on the caller's stream, the
    scale/codebook gradients on a forked side stream joined back) captured
    in a HIP graph: every replay, with x and gy rewritten in place between
    them, equals the eager call bit for bit."""
    n, k, m = 256, 384, 512
    _, _, _, _, s = make(n, k, 128, seed=5)
    h = cuda._hot(s)
    x, gy = bf16((m, k), 21), bf16((m, n), 22, 1e-2)
    for _ in range(2):                       # first call in order, then forked
        run_bwd(s, gy, x)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        cuda.backward(gy, x, h, gx_dtype=torch.float32)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = cuda.backward(gy, x, h, gx_dtype=torch.float32)
    assert out is not None
    for r in range(3):
        x.copy_(bf16((m, k), 30 + r))
        gy.copy_(bf16((m, n), 40 + r, 1e-2))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        eager = run_bwd(s, gy, x)
        assert all(torch.equal(p, q) for p, q in zip(out, eager)), r


def test_backward_library_route_many_token_counts():
    """A new token count on every call (70 counts from 512 up): each count
    gets its own library GEMM plans -- the cache keeps at most 64 and drops
    the least recently used -- and reuses its shape bucket's timed
    algorithm.  Every call matches the closed forms, and the first count,
    run again after its plans were dropped, gives the same bits."""
    n, k = 256, 384
    _, _, _, _, s = make(n, k, 128, seed=55)
    first = None
    for i, m in enumerate(range(512, 582)):
        x, gy = bf16((m, k), 200 + i), bf16((m, n), 300 + i, 1e-2)
        gx, gcb, gsc = run_bwd(s, gy, x)
        wgx, wgcb, wgsc = closed_forms_t64(gy, x, s)
        assert rel(gx.float(), wgx) < 2e-3, m
        assert rel(gsc, wgsc) < 1e-4, m
        assert rel(gcb, wgcb) < 1e-4, m
        if first is None:
            first = (x, gy, gx, gcb, gsc)
    x, gy = first[0], first[1]
    again = run_bwd(s, gy, x)
    assert all(torch.equal(p, q) for p, q in zip(first[2:], again))
