"""Stacked experts (epure/runtime.py:163-186): the expert-indexed packed
linear (experts kept packed) and the reference-style holder that attaches
the dense slab only while its module runs.  Held to the packed-linear bar:
max relative error 2e-3 against the Rust-order float32 result per expert
(plus the output rounding)."""
import numpy as np
import pytest
import torch

from epure import ExpertHolder, PackedExperts, PackedWeight
from oracle import ref, rowdot

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def experts(E, n, k, levels, group, seed):
    rng = np.random.Generator(np.random.PCG64(seed))
    idx = rng.integers(0, levels, E * n * k).astype(np.uint8)
    packed = ref.pack4(idx, levels)
    cb = np.sort(rng.standard_normal(levels)).astype(np.float16).astype(np.float32)
    scale = (np.abs(rng.normal(0, 0.02, (E * n, k // group))) + 1e-3).astype(np.float16)
    s = PackedWeight((E, n, k), packed, scale, cb, group, levels).to(DEV)
    return s, packed, scale, cb


def want_rows(x32, ids, packed, scale, cb, E, n, k, group, levels):
    rb = k // 2 if levels <= 16 else k
    p2 = packed.reshape(E * n, rb)
    out = np.empty((len(ids), n), np.float32)
    for t, e in enumerate(ids):
        out[t] = rowdot.dequant_matmul(x32[t:t + 1], p2[e * n:(e + 1) * n],
                                       scale[e * n:(e + 1) * n].astype(np.float32), cb, group,
                                       levels <= 16)[0]
    return out


@pytest.mark.parametrize("E,n,k,levels,T", [(4, 256, 512, 16, 10), (8, 512, 1024, 16, 300),
                                            (3, 128, 256, 256, 7)])
def test_packed_experts_vs_oracle(E, n, k, levels, T):
    group = 128
    s, packed, scale, cb = experts(E, n, k, levels, group, seed=E + n)
    g = torch.Generator(device=DEV).manual_seed(T)
    x = torch.randn(T, k, generator=g, device=DEV).to(torch.bfloat16)
    ids = torch.randint(0, E - 1, (T,), generator=g, device=DEV)   # the last expert unused
    y = PackedExperts(s)(x, ids)
    assert y.shape == (T, n) and y.dtype == torch.bfloat16
    want = want_rows(x.float().cpu().numpy(), ids.cpu().tolist(), packed, scale, cb, E, n, k,
                     group, levels)
    got = y.float().cpu().numpy()
    err = np.abs(got - want).max() / np.abs(want).max()
    assert err < 2e-3 + 2.0 ** -8, err


def test_packed_experts_rejects_bad_ids():
    s, *_ = experts(2, 64, 128, 16, 128, seed=1)
    with pytest.raises(IndexError):
        PackedExperts(s)(torch.zeros(2, 128, device=DEV, dtype=torch.bfloat16),
                         torch.tensor([0, 2], device=DEV))


def test_expert_holder_attaches_only_during_forward():
    s, *_ = experts(4, 64, 128, 16, 64, seed=2)

    class Moe(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.weight = torch.nn.Parameter(torch.zeros(4, 64, 128))
            self.seen = None

        def forward(self, x):
            self.seen = self.weight
            # a plain reduction over the attached slab (no batched product)
            return x.float().sum(1)[:, None, None] * self.weight.float().sum(-1)[None]

    m = Moe().to(DEV)
    ExpertHolder(m, "weight", s, torch.bfloat16)
    assert m.weight is None
    y = m(torch.randn(3, 128, device=DEV))
    assert m.weight is None and y.shape == (3, 4, 64)
    assert torch.equal(m.seen, s.materialize(torch.bfloat16))


@pytest.mark.parametrize("E,n,k,levels,T,dt", [(4, 256, 512, 16, 1, torch.bfloat16),
                                               (6, 512, 2048, 16, 8, torch.float16),
                                               (8, 384, 1024, 16, 5, torch.bfloat16),
                                               (3, 128, 256, 256, 4, torch.float16)])
def test_gathered_experts_vs_oracle(E, n, k, levels, T, dt):
    """T <= GATHER_MAX_TOKENS: one ep_expert_matmul launch, ids on the device
    (repeated and out-of-order ids included)."""
    group = 128
    s, packed, scale, cb = experts(E, n, k, levels, group, seed=3 * E + T)
    g = torch.Generator(device=DEV).manual_seed(100 + T)
    x = torch.randn(T, k, generator=g, device=DEV).to(dt)
    ids = torch.randint(0, E, (T,), generator=g, device=DEV)
    if T > 2:
        ids[1] = ids[0]                     # two tokens on one expert
    y = PackedExperts(s)(x, ids)
    assert y.shape == (T, n) and y.dtype == dt
    want = want_rows(x.float().cpu().numpy(), ids.cpu().tolist(), packed, scale, cb, E, n, k,
                     group, levels)
    err = np.abs(y.float().cpu().numpy() - want).max() / np.abs(want).max()
    assert err < 2e-3 + 2.0 ** -8, err


def test_gathered_experts_match_grouped_path():
    """The gathered launch and the per-expert host-grouped route agree bit
    for bit on the same rows (both run the batch-1 GEMV per token row)."""
    s, *_ = experts(5, 512, 1024, 16, 128, seed=7)
    g = torch.Generator(device=DEV).manual_seed(9)
    x = torch.randn(6, 1024, generator=g, device=DEV).to(torch.bfloat16)
    ids = torch.tensor([4, 0, 2, 2, 1, 3], device=DEV)
    m = PackedExperts(s)
    y_g = m(x, ids)
    m.GATHER_MAX_TOKENS = 0                 # this instance groups per expert on the host
    m.GROUP_ON_DEVICE = False
    ys = [m(x[t:t + 1], ids[t:t + 1]) for t in range(6)]
    assert torch.equal(y_g, torch.cat(ys))


def test_gathered_experts_graph_replay_follows_ids():
    """Captured once, the gathered call follows ids and x rewritten in place
    between replays (no host synchronization inside the call)."""
    E, n, k, T = 6, 256, 1024, 4
    s, packed, scale, cb = experts(E, n, k, 16, 128, seed=11)
    m = PackedExperts(s, check_ids=False)
    g = torch.Generator(device=DEV).manual_seed(5)
    x = torch.randn(T, k, generator=g, device=DEV).to(torch.bfloat16)
    ids = torch.tensor([0, 1, 2, 3], device=DEV, dtype=torch.int32)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        m(x, ids)                           # warm-up outside capture
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y = m(x, ids)
    for r in range(4):
        new_ids = torch.randint(0, E, (T,), generator=g, device=DEV, dtype=torch.int32)
        ids.copy_(new_ids)
        x.copy_(torch.randn(T, k, generator=g, device=DEV).to(torch.bfloat16))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        eager = PackedExperts(s)(x, ids)
        assert torch.equal(y, eager), r


def test_gathered_experts_f32_scales_and_bf16_codebook():
    """The gathered launch with float32 group scales and a bfloat16 codebook
    (per-expert scale stride in 4-byte units)."""
    E, n, k, T, group = 5, 256, 1024, 6, 128
    rng = np.random.Generator(np.random.PCG64(21))
    idx = rng.integers(0, 16, E * n * k).astype(np.uint8)
    packed = ref.pack4(idx, 16)
    cb = torch.tensor(np.sort(rng.standard_normal(16)), dtype=torch.bfloat16)
    scale = (np.abs(rng.normal(0, 0.02, (E * n, k // group))) + 1e-3).astype(np.float32)
    s = PackedWeight((E, n, k), packed, scale, cb, group, 16).to(DEV)
    assert s.scale.dtype == torch.float32 and s.cb.dtype == torch.bfloat16
    g = torch.Generator(device=DEV).manual_seed(4)
    x = torch.randn(T, k, generator=g, device=DEV).to(torch.bfloat16)
    ids = torch.tensor([4, 0, 3, 3, 1, 2], device=DEV)
    y = PackedExperts(s)(x, ids)
    want = want_rows(x.float().cpu().numpy(), ids.cpu().tolist(), packed, scale,
                     cb.float().numpy(), E, n, k, group, 16)
    err = np.abs(y.float().cpu().numpy() - want).max() / np.abs(want).max()
    assert err < 2e-3 + 2.0 ** -8, err


def test_gathered_experts_clamp_ids_without_check():
    """With check_ids=False ids outside [0, E) are clamped on the device
    (-3 -> expert 0, E + 2 -> expert E - 1): the rows equal those of the
    clamped ids."""
    E, n, k = 4, 128, 512
    s, *_ = experts(E, n, k, 16, 128, seed=13)
    g = torch.Generator(device=DEV).manual_seed(6)
    x = torch.randn(3, k, generator=g, device=DEV).to(torch.float16)
    y = PackedExperts(s, check_ids=False)(x, torch.tensor([-3, 1, E + 2], device=DEV))
    want = PackedExperts(s)(x, torch.tensor([0, 1, E - 1], device=DEV))
    assert torch.equal(y, want)


@pytest.mark.parametrize("pad", [3, 8])
def test_gathered_experts_strided_rows(pad):
    """Activation rows at a stride of k + pad elements (a column slice of a
    wider buffer).  The gathered launch reads each row with 16-byte loads,
    so a stride that is not a multiple of 8 bf16 elements is declined
    (the grouped path serves it); a multiple of 8 runs gathered.  Both
    match the oracle."""
    from epure.kernels import _abi
    from epure.kernels import cuda as cuda_kernel

    E, n, k, T = 4, 256, 512, 5
    s, packed, scale, cb = experts(E, n, k, 16, 128, seed=40 + pad)
    g = torch.Generator(device=DEV).manual_seed(41)
    wide = torch.randn(T, k + pad, generator=g, device=DEV).to(torch.bfloat16)
    x = wide[:, :k]
    assert x.stride() == (k + pad, 1)
    ids = torch.tensor([3, 0, 1, 1, 2], device=DEV)
    h = cuda_kernel._hot(s)
    y_try = torch.empty(T, n, device=DEV, dtype=torch.bfloat16)
    rc = _abi.lib.ep_expert_matmul(
        x.data_ptr(), _abi.dtype_code(x.dtype), x.stride(0),
        ids.to(torch.int32).contiguous().data_ptr(), T, h.packed.data_ptr(), h.scale.data_ptr(),
        h.scale_dt, h.ld_scale, h.cb.data_ptr(), h.cb_dt, h.levels, h.group, E, n, k,
        y_try.data_ptr(), _abi.dtype_code(y_try.dtype), y_try.stride(0), _abi.stream_handle(DEV))
    torch.cuda.synchronize()
    assert (rc > 0) == (pad % 8 != 0), (rc, _abi.last_error())
    y = PackedExperts(s)(x, ids)
    want = want_rows(x.float().cpu().numpy(), ids.cpu().tolist(), packed, scale, cb, E, n, k,
                     128, 16)
    err = np.abs(y.float().cpu().numpy() - want).max() / np.abs(want).max()
    assert err < 2e-3 + 2.0 ** -8, err


def skewed_ids(T, E, g, kind):
    if kind == "uniform":
        return torch.randint(0, E, (T,), generator=g, device=DEV)
    if kind == "skewed":                    # most tokens on one expert, the rest spread
        ids = torch.randint(0, E, (T,), generator=g, device=DEV)
        hot = torch.rand(T, generator=g, device=DEV) < 0.8
        return torch.where(hot, torch.full_like(ids, E // 2), ids)
    if kind == "sparse":                    # every other expert empty
        return 2 * torch.randint(0, (E + 1) // 2, (T,), generator=g, device=DEV)
    return torch.full((T,), E - 1, device=DEV, dtype=torch.int64)   # one expert takes all


@pytest.mark.parametrize("E,n,k,levels,T,dt,kind", [
    # the prefill kernel over the sorted runs (fp16 scales): 64-row tiles
    # below 128 tokens per expert, 128-row tiles from there
    (8, 256, 512, 16, 100, torch.bfloat16, "uniform"),
    (4, 384, 1024, 16, 300, torch.float16, "skewed"),      # one long run
    (16, 128, 256, 256, 37, torch.bfloat16, "sparse"),     # 8-bit, empty experts
    (64, 128, 512, 16, 2048, torch.bfloat16, "uniform"),   # many experts
    (2, 256, 512, 256, 700, torch.float16, "one"),         # all tokens on the last expert, 128 rows
    (6, 192, 512, 16, 90, torch.float32, "uniform"),       # f32 activations
    (3, 512, 1024, 16, 400, torch.bfloat16, "uniform"),    # 4-bit, 128-row tiles
    (4, 256, 2048, 256, 260, torch.bfloat16, "skewed"),    # 8-bit
    (4, 320, 1024, 16, 300, torch.float16, "sparse"),      # empty experts
    (2, 128, 512, 16, 300, torch.float32, "uniform"),      # f32 activations, 128-row tiles
    (16, 256, 2048, 16, 40, torch.bfloat16, "uniform"),
    (8, 384, 4096, 16, 50, torch.float16, "skewed"),       # one expert's run over two tiles
    (12, 128, 2048, 256, 30, torch.bfloat16, "sparse"),
    (6, 256, 8192, 16, 20, torch.bfloat16, "uniform"),
])
def test_grouped_experts_vs_oracle(E, n, k, levels, T, dt, kind):
    """T > GATHER_MAX_TOKENS: tokens sorted by expert on the device, one
    grouped MFMA launch over each expert's row tiles (ep_expert_matmul_grouped),
    results at the tokens' own rows."""
    group = 128
    s, packed, scale, cb = experts(E, n, k, levels, group, seed=5 * E + T)
    g = torch.Generator(device=DEV).manual_seed(200 + T)
    x = torch.randn(T, k, generator=g, device=DEV).to(dt)
    ids = skewed_ids(T, E, g, kind)
    print(f"case: grouped experts E={E} n={n} k={k} levels={levels} T={T} x={dt} ids={kind}", flush=True)
    y = PackedExperts(s)(x, ids)
    assert y.shape == (T, n) and y.dtype == dt
    want = want_rows(x.float().cpu().numpy(), ids.cpu().tolist(), packed, scale, cb, E, n, k,
                     group, levels)
    got = y.float().cpu().numpy()
    tol = 2e-3 + (0.0 if dt == torch.float32 else 2.0 ** -8)
    err = np.abs(got - want).max() / np.abs(want).max()
    assert err < tol, err
    floor = np.sqrt(np.mean(want ** 2))
    rel = (np.abs(got - want) / np.maximum(np.abs(want), floor)).max()
    assert rel < 2 * tol, rel


@pytest.mark.parametrize("E,T,k", [(12, 64, 1024), (4, 512, 1024), (32, 64, 2048)])
def test_grouped_experts_graph_replay_follows_ids(E, T, k):
    """Captured once, the grouped call (device sort + the prefill kernel over
    the sorted runs: 64-row tiles at 12 and 32 experts x 64 tokens, 128-row
    tiles at 4 x 512) follows ids and x rewritten in place between replays;
    every replay equals an eager call bit for bit."""
    n = 256
    s, *_ = experts(E, n, k, 16, 128, seed=17)
    m = PackedExperts(s, check_ids=False)
    g = torch.Generator(device=DEV).manual_seed(8)
    x = torch.randn(T, k, generator=g, device=DEV).to(torch.bfloat16)
    ids = torch.randint(0, E, (T,), generator=g, device=DEV, dtype=torch.int32)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        m(x, ids)                           # warm-up outside capture
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y = m(x, ids)
    for r in range(4):
        ids.copy_(skewed_ids(T, E, g, ["uniform", "skewed", "sparse", "one"][r]).to(torch.int32))
        x.copy_(torch.randn(T, k, generator=g, device=DEV).to(torch.bfloat16))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        eager = PackedExperts(s)(x, ids)
        assert torch.equal(y, eager), r


@pytest.mark.parametrize("E,T", [(6, 40), (3, 200)])
def test_grouped_experts_f32_scales_generic_kernel(E, T):
    """float32 group scales and a bfloat16 codebook (after make_trainable)
    take the generic MFMA kernel over the sorted runs (32- / 64-row tiles;
    per-expert scale stride in 4-byte units)."""
    n, k, group = 256, 1024, 128
    rng = np.random.Generator(np.random.PCG64(31 + T))
    idx = rng.integers(0, 16, E * n * k).astype(np.uint8)
    packed = ref.pack4(idx, 16)
    cb = torch.tensor(np.sort(rng.standard_normal(16)), dtype=torch.bfloat16)
    scale = (np.abs(rng.normal(0, 0.02, (E * n, k // group))) + 1e-3).astype(np.float32)
    s = PackedWeight((E, n, k), packed, scale, cb, group, 16).to(DEV)
    g = torch.Generator(device=DEV).manual_seed(T)
    x = torch.randn(T, k, generator=g, device=DEV).to(torch.bfloat16)
    ids = skewed_ids(T, E, g, "skewed")
    y = PackedExperts(s)(x, ids)
    want = want_rows(x.float().cpu().numpy(), ids.cpu().tolist(), packed, scale,
                     cb.float().numpy(), E, n, k, group, 16)
    err = np.abs(y.float().cpu().numpy() - want).max() / np.abs(want).max()
    assert err < 2e-3 + 2.0 ** -8, err


def test_grouped_experts_clamp_ids_and_strided_rows():
    """check_ids=False clamps ids outside [0, E) on the device; activation
    rows at a stride of k + 8 elements; two calls give the same bits."""
    E, n, k, T = 5, 128, 512, 40
    s, *_ = experts(E, n, k, 16, 128, seed=19)
    g = torch.Generator(device=DEV).manual_seed(12)
    wide = torch.randn(T, k + 8, generator=g, device=DEV).to(torch.bfloat16)
    x = wide[:, :k]
    ids = torch.randint(0, E, (T,), generator=g, device=DEV)
    bad = ids.clone()
    bad[0], bad[1] = -3, E + 2
    ids[0], ids[1] = 0, E - 1
    y = PackedExperts(s, check_ids=False)(x, bad)
    want = PackedExperts(s)(x.contiguous(), ids)
    assert torch.equal(y, want)
    assert torch.equal(PackedExperts(s)(x, ids), want)
    with pytest.raises(IndexError):
        PackedExperts(s)(x, bad)
