"""GPU parity of the small-M (2..64 rows) split-K path through the C ABI.

The oracle is the C restatement of the reference Rust kernel
(kernel/src/lib.rs:36-151, oracle/rowdot.c): fp32, group-then-k order.  Bar:
max relative error 2e-3, normwise and per element with an rms floor (the
GPU multiplies fp16 operands, fp32 accumulation, like the reference's
Triton table kernel, epure/kernels/_triton.py:95-103).  The cases cover the
edges of the split-K tiling: K not a multiple of the split, N not a multiple
of the 128-row tile, several tiles per workgroup, accumulation through the
split reduction, every output dtype, activations far outside fp16's range.
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


def x_bf16(m, k, seed, scale=1.0):
    x32 = ref.round_bf16((rng(seed).standard_normal((m, k)) * scale).astype(np.float32))
    return x32, torch.from_numpy(x32).to(DEV).to(torch.bfloat16)


def run(s, x, out_dtype=torch.float32, accumulate=False, out=None):
    print(f"case: N={s.out_features} K={s.in_features} M={x.shape[0]} levels={s.levels} "
          f"x={x.dtype} y={out_dtype} acc={accumulate}", flush=True)
    h = cuda._hot(s)
    if out is None:
        out = torch.empty((x.shape[0], s.out_features), device=DEV, dtype=out_dtype)
    y = cuda.forward(x, h, out=out, accumulate=accumulate)
    assert y is not None, f"declined: {_abi.last_error()}"
    torch.cuda.synchronize()
    return y


@pytest.mark.parametrize("levels", [16, 256])
@pytest.mark.parametrize("m", [2, 7, 16, 17, 32, 48, 64])
def test_skinny_rows(levels, m):
    n, k = 1000, 4096
    _, packed, scale, cb, s = make(n, k, levels, seed=m + levels)
    x32, x = x_bf16(m, k, m)
    assert_close(run(s, x).cpu().numpy(), rust_ref(x32, packed, scale, cb, n, k, levels, 128))


@pytest.mark.parametrize("levels", [16, 256])
@pytest.mark.parametrize("n,k", [(200, 1056), (130, 96), (4096, 1024), (14336, 512), (64, 14336)])
def test_skinny_ragged_splits_and_tiles(levels, n, k):
    """K past the last full split, N past the last full tile, and (at 14336
    rows) several row tiles per workgroup."""
    m = 5
    _, packed, scale, cb, s = make(n, k, levels, seed=n + k)
    x32, x = x_bf16(m, k, n)
    assert_close(run(s, x).cpu().numpy(), rust_ref(x32, packed, scale, cb, n, k, levels, 128))


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("k", [512, 4096])
def test_skinny_accumulate_and_out_dtypes(out_dtype, k):
    """One split (K = 512, results straight from the workgroups or through
    the reduction when accumulating) and eight splits (K = 4096)."""
    n, m = 384, 12
    _, packed, scale, cb, s = make(n, k, seed=k + 1)
    x32, x = x_bf16(m, k, k + 2)
    want = rust_ref(x32, packed, scale, cb, n, k, 16, 128)
    out_tol = TOL if out_dtype == torch.float32 else TOL + 2.0 ** -8
    y = run(s, x, out_dtype).float().cpu().numpy()
    assert_close(y, want, out_tol)
    base = torch.from_numpy(rng(k + 3).standard_normal((m, n)).astype(np.float32)).to(DEV)
    out = base.to(out_dtype)
    start = out.float().cpu().numpy()  # the accumulator's initial contents
    run(s, x, out_dtype, accumulate=True, out=out)
    assert_close(out.float().cpu().numpy(), want + start, out_tol)


@pytest.mark.parametrize("xdt", [torch.float16, torch.float32])
def test_skinny_x_dtypes(xdt):
    n, k, m = 512, 2048, 9
    _, packed, scale, cb, s = make(n, k, seed=31)
    x32 = rng(32).standard_normal((m, k)).astype(np.float32)
    x = torch.from_numpy(x32).to(DEV).to(xdt)
    xr = x.float().cpu().numpy()
    assert_close(run(s, x).cpu().numpy(), rust_ref(xr, packed, scale, cb, n, k, 16, 128))


@pytest.mark.parametrize("group,levels", [(32, 16), (64, 16), (16, 256), (256, 256)])
def test_skinny_groups(group, levels):
    n, k, m = 300, 1024, 6
    _, packed, scale, cb, s = make(n, k, levels, group=group, seed=group)
    x32, x = x_bf16(m, k, group)
    assert_close(run(s, x).cpu().numpy(), rust_ref(x32, packed, scale, cb, n, k, levels, group))


def test_skinny_levels_below_16_read_zero():
    n, k, m = 64, 512, 5
    idx = rng(3).integers(0, 16, (n, k), dtype=np.uint8)
    packed = ref.pack4(idx, 16)
    cb = np.sort(rng(4).standard_normal(10)).astype(np.float16)
    scale = (np.abs(rng(5).normal(0, 0.02, (n, 4))) + 1e-3).astype(np.float16)
    s = PackedWeight((n, k), packed, scale, cb.astype(np.float32), 128, 10).to(DEV)
    x32, x = x_bf16(m, k, 6)
    assert_close(run(s, x).cpu().numpy(), rust_ref(x32, packed, scale, cb, n, k, 10, 128))


def test_skinny_rows_of_very_different_magnitude():
    """Each row of each split gets its own power-of-two factor: rows at
    3e5, 1, 1e-12, 1e-30 and 0 all stay exact relative to their own size."""
    n, k = 256, 2048
    idx, packed, scale, cb, s = make(n, k, seed=41)
    w64 = ref.dequant_tile_f32(idx, scale, cb, 128).astype(np.float64)
    mags = np.array([3e5, 1.0, 1e-12, 1e-30, 0.0], np.float32)
    x32 = ref.round_bf16((rng(42).standard_normal((5, k)) * mags[:, None]).astype(np.float32))
    x = torch.from_numpy(x32).to(DEV).to(torch.bfloat16)
    y = run(s, x).cpu().numpy()
    want = ref.linear_f64(x32, w64)
    for r in range(4):
        assert_close(y[r:r + 1], want[r:r + 1])
    assert np.all(y[4] == 0.0)


def test_skinny_deterministic():
    n, k, m = 1024, 4096, 16
    _, packed, scale, cb, s = make(n, k, seed=51)
    _, x = x_bf16(m, k, 52)
    a = run(s, x).cpu().numpy()
    b = run(s, x).cpu().numpy()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# Loads per lane and row tile of the small-M path, at most (the staged
# activation rows x K split fit the LDS); a split is 64 bytes of a row per
# load, and the launch takes the longest split whose grid (one 128-row tile
# per workgroup at most) still fills the CUs.
LD_MAX = {(16, 16): 16, (16, 32): 8, (16, 64): 4, (256, 16): 16, (256, 32): 16, (256, 64): 8}


def skinny_splits(m, n, k, levels):
    mb = 16 if m <= 16 else (32 if m <= 32 else 64)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    per_load = 128 if levels <= 16 else 64  # k values per load's 64 bytes
    tiles = -(-n // 128)
    ld = LD_MAX[(levels, mb)]
    while ld > 4 and tiles * -(-k // (ld * per_load)) < cus:
        ld //= 2
    return -(-k // (ld * per_load))


@pytest.mark.parametrize("m", [2, 16, 17, 32, 33, 64])
@pytest.mark.parametrize("levels", [16, 256])
@pytest.mark.parametrize("n,k", [(14336, 4096 + 64), (4096, 4096), (4096, 14336)])
def test_skinny_workspace_covers_partials(m, levels, n, k):
    """The workspace query covers every split's partial sums."""
    need = _abi.lib.ep_dequant_matmul_workspace(m, n, k, levels, 128)
    assert need >= skinny_splits(m, n, k, levels) * m * n * 4


# The one-launch path: 16-bit activations, enough 16-row tiles to fill 3/4
# of the CUs (N >= 12 x CUs, at most 4 tiles per CU) and M <= 16 x the
# tiles per workgroup (one tile up to N = 16 x CUs, two up to 32 x CUs,
# four above); 8-bit indices up to M = 64 (bf16 x on the bf16 path, whose
# groups are multiples of 64 values; else up to M = 32), 4-bit indices up
# to M = 8 (M <= 4 at K <= 4096 stays on the GEMV).  On a 256-CU device:
# 8-bit at M <= 16, (32, 8200), (24, 14336), (20, 6144), (64, 14336) and
# (48, 12000); 4-bit at (5, 4096), (8, 8200), (7, 4096); the others take
# the split-K kernel.
@pytest.mark.parametrize("levels", [16, 256])
@pytest.mark.parametrize("m,n,k", [(2, 4096, 4096), (16, 4096, 4096 + 32), (9, 8200, 2048),
                                   (4, 14336, 1024), (13, 4100, 1568), (17, 4096, 4096),
                                   (32, 8200, 2048), (24, 14336, 1024), (20, 6144, 2048 + 32),
                                   (33, 4100, 1568), (64, 4096, 4096 + 32), (5, 4096, 4096 + 32),
                                   (8, 8200, 2048), (7, 4096, 14336), (64, 14336, 1024),
                                   (48, 12000, 2048 + 64)])
def test_skinny_one_launch(levels, m, n, k):
    """All of K in one workgroup per row tile: K past the last full round
    of a wave (and a last group of 32 values), N past the last 16-row tile,
    one, two and four row tiles per workgroup, one, two and four 16-row
    activation blocks."""
    _, packed, scale, cb, s = make(n, k, levels, seed=n + k + m)
    x32, x = x_bf16(m, k, m + levels)
    assert_close(run(s, x).cpu().numpy(), rust_ref(x32, packed, scale, cb, n, k, levels, 128))


@pytest.mark.parametrize("m,n", [(11, 4096), (28, 8192), (60, 14336)])
@pytest.mark.parametrize("levels", [16, 256])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_skinny_one_launch_accumulate_f16_x(out_dtype, levels, m, n):
    """fp16 activations (the operand as they are); results written, then
    added to y in the same launch."""
    k = 2048
    _, packed, scale, cb, s = make(n, k, levels, seed=61)
    x32 = rng(62).standard_normal((m, k)).astype(np.float32)
    x = torch.from_numpy(x32).to(DEV).to(torch.float16)
    want = rust_ref(x.float().cpu().numpy(), packed, scale, cb, n, k, levels, 128)
    out_tol = TOL if out_dtype == torch.float32 else TOL + 2.0 ** -8
    assert_close(run(s, x, out_dtype).float().cpu().numpy(), want, out_tol)
    out = torch.from_numpy(rng(63).standard_normal((m, n)).astype(np.float32)).to(DEV).to(out_dtype)
    start = out.float().cpu().numpy()
    run(s, x, out_dtype, accumulate=True, out=out)
    assert_close(out.float().cpu().numpy(), want + start, out_tol)


@pytest.mark.parametrize("m,n,k", [(5, 8200, 2048), (8, 4096, 14336)])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_skinny_one_launch_4bit_accumulate_f16_x(out_dtype, m, n, k):
    """The 4-bit one-launch kernel (M 5..8) with fp16 activations: results
    written, then added to y in the same launch, for every output dtype."""
    _, packed, scale, cb, s = make(n, k, 16, seed=64 + m)
    x32 = rng(65 + m).standard_normal((m, k)).astype(np.float32)
    x = torch.from_numpy(x32).to(DEV).to(torch.float16)
    want = rust_ref(x.float().cpu().numpy(), packed, scale, cb, n, k, 16, 128)
    out_tol = TOL if out_dtype == torch.float32 else TOL + 2.0 ** -8
    assert_close(run(s, x, out_dtype).float().cpu().numpy(), want, out_tol)
    out = torch.from_numpy(rng(66 + m).standard_normal((m, n)).astype(np.float32)).to(DEV).to(out_dtype)
    start = out.float().cpu().numpy()
    run(s, x, out_dtype, accumulate=True, out=out)
    assert_close(out.float().cpu().numpy(), want + start, out_tol)


@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,n,k", [(6, 8184, 1104), (16, 8184, 2112), (5, 12300, 1104), (16, 12300, 2112)])
def test_skinny_one_launch_whole_line_rounds(xdt, m, n, k):
    """The one-launch kernel at two (N = 8184) and four (N = 12300) tiles
    per workgroup on 256 CUs, 8-bit indices, M >= 5 (the GEMV takes M <= 4):
    rounds of 128 values (two 16-byte pieces per row) over a K that ends
    inside a round's second piece (1104 = 8 x 128 + 80) or first (2112 = 16
    x 128 + 64)."""
    _, packed, scale, cb, s = make(n, k, 256, 64, seed=n + k + m)
    x32, x = x_bf16(m, k, 7 * m + k)
    x = x.to(xdt)
    xr = x.float().cpu().numpy()
    y = run(s, x).cpu().numpy()
    want = rust_ref(xr, packed, scale, cb, n, k, 256, 64)
    if xdt == torch.bfloat16:
        assert_close(y, want)
    else:  # fp16 x: the products take fp16(cb[idx] * scale) (_triton.py:95-103)
        assert_close(y, ref.linear_f64(xr, ref.materialize(packed, scale, cb, n, k, 64, 256, "f16")), 1e-4)


@pytest.mark.parametrize("group,m", [(64, 24), (256, 24), (64, 40), (256, 64)])
def test_skinny_one_launch_bf16_path_groups(group, m):
    """The bf16 path (8-bit indices, bf16 x) scales each 64-value piece's
    sums by its group's scale: groups of one piece and of four, two and
    four activation blocks (four tiles per workgroup)."""
    n, k = 8200, 2048
    _, packed, scale, cb, s = make(n, k, 256, group=group, seed=111 + group + m)
    x32, x = x_bf16(m, k, 112 + group + m)
    assert_close(run(s, x).cpu().numpy(), rust_ref(x32, packed, scale, cb, n, k, 256, group))


def test_skinny_one_launch_rows_of_very_different_magnitude():
    """Rows at 3e5, 1, 1e-12, 1e-30 and 0 stay exact relative to their own
    size (the same five again in the second 16-row block): the bf16 path
    keeps bf16's range, the fp16 one rescales each row by a power of two
    per round."""
    n, k = 8192, 2048
    idx, packed, scale, cb, s = make(n, k, levels=256, seed=71)
    w64 = ref.dequant_tile_f32(idx, scale, cb, 128).astype(np.float64)
    mags = np.array([3e5, 1.0, 1e-12, 1e-30, 0.0] + [1.0] * 11 + [3e5, 1.0, 1e-12, 1e-30, 0.0],
                    np.float32)
    x32 = ref.round_bf16((rng(72).standard_normal((21, k)) * mags[:, None]).astype(np.float32))
    x = torch.from_numpy(x32).to(DEV).to(torch.bfloat16)
    y = run(s, x).cpu().numpy()
    want = ref.linear_f64(x32, w64)
    for r in list(range(4)) + list(range(16, 20)):
        assert_close(y[r:r + 1], want[r:r + 1])
    assert np.all(y[4] == 0.0) and np.all(y[20] == 0.0)


@pytest.mark.parametrize("m,n", [(16, 4096), (32, 8192)])
def test_skinny_one_launch_deterministic(m, n):
    k = 4096
    _, packed, scale, cb, s = make(n, k, 256, seed=81)
    _, x = x_bf16(m, k, 82)
    a = run(s, x).cpu().numpy()
    b = run(s, x).cpu().numpy()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("m,k", [(3, 16), (5, 256), (16, 1040)])
def test_skinny_one_launch_short_k(m, k):
    """K of one 16-value chunk, of two rounds (most of the 16 waves own no
    round and add zeros), and one chunk past a full round."""
    n = 4096
    _, packed, scale, cb, s = make(n, k, 256, group=16, seed=91 + k)
    x32, x = x_bf16(m, k, 92 + k)
    assert_close(run(s, x).cpu().numpy(), rust_ref(x32, packed, scale, cb, n, k, 256, 16))


@pytest.mark.parametrize("m", [4, 24])
def test_skinny_one_launch_strided_x(m):
    """Activation rows further apart than K (a column slice of a wider
    tensor): every row read at its own stride."""
    n, k = 8192, 2048
    _, packed, scale, cb, s = make(n, k, 256, seed=101)
    x32 = ref.round_bf16(rng(102).standard_normal((m, k + 96)).astype(np.float32))
    wide = torch.from_numpy(x32).to(DEV).to(torch.bfloat16)
    x = wide[:, :k]
    assert x.stride(0) == k + 96
    assert_close(run(s, x).cpu().numpy(), rust_ref(np.ascontiguousarray(x32[:, :k]), packed, scale, cb, n,
                                                    k, 256, 128))


# The register-resident split-K kernel: 8-bit indices, 33 <= M <= 64 (17 <=
# M on layers of at least 2^25 weights), fp16 x or bf16 x with groups of a
# multiple of 64 values (the bf16 path).  A split is 4096 values of K (M <= 32) or 2048;
# a workgroup streams every gtiles-th 16-row tile of its split.
@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,n,k,group,levels", [
    (17, 8200, 4096 + 64, 128, 256),   # two splits, the second of 64 values; N past the last tile
    (33, 8200, 4096 + 64, 64, 200),    # three activation blocks; levels below 256
    (48, 2056, 16384 + 64, 256, 256),  # nine splits (the last of 64 values), 129 tiles
    (64, 16400, 2048, 128, 256),       # one split: straight into y, several tiles per workgroup
    (32, 4104, 8192 + 128, 128, 256),  # two blocks, three splits (the last of 128 values)
    (20, 4104, 8192 + 32, 64, 256),    # K past the last whole 64-value piece
])
def test_skinny_register_resident(xdt, m, n, k, group, levels):
    _, packed, scale, cb, s = make(n, k, levels, group, seed=n + k + m)
    x32, x = x_bf16(m, k, m + levels)
    x = x.to(xdt)
    want = rust_ref(x.float().cpu().numpy(), packed, scale, cb, n, k, levels, group)
    assert_close(run(s, x).cpu().numpy(), want)


@pytest.mark.parametrize("m,n,k", [(24, 16400, 2048), (64, 8200, 4096 + 64)])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_skinny_register_resident_accumulate(out_dtype, m, n, k):
    """Results written, then added to y: in the kernel with one split,
    through the split reduction with three."""
    _, packed, scale, cb, s = make(n, k, 256, seed=71 + m)
    x32, x = x_bf16(m, k, 72 + m)
    want = rust_ref(x32, packed, scale, cb, n, k, 256, 128)
    out_tol = TOL if out_dtype == torch.float32 else TOL + 2.0 ** -8
    assert_close(run(s, x, out_dtype).float().cpu().numpy(), want, out_tol)
    out = torch.from_numpy(rng(73 + m).standard_normal((m, n)).astype(np.float32)).to(DEV).to(out_dtype)
    start = out.float().cpu().numpy()
    run(s, x, out_dtype, accumulate=True, out=out)
    assert_close(out.float().cpu().numpy(), want + start, out_tol)


def test_skinny_register_resident_rows_of_very_different_magnitude():
    """bf16 rows from 1e30 down to 1e-30 and 0 are exact MFMA operands on
    the bf16 path: each row stays exact relative to its own size."""
    n, k = 8200, 4096 + 64
    idx, packed, scale, cb, s = make(n, k, 256, seed=81)
    w64 = ref.dequant_tile_f32(idx, scale, cb, 128).astype(np.float64)
    mags = np.array([1e30, 3e5, 1.0, 1e-12, 1e-30, 0.0] * 3, np.float32)
    x32 = ref.round_bf16((rng(82).standard_normal((len(mags), k)) * mags[:, None]).astype(np.float32))
    x = torch.from_numpy(x32).to(DEV).to(torch.bfloat16)
    y = run(s, x).cpu().numpy()
    want = ref.linear_f64(x32, w64)
    for r in range(len(mags)):
        if mags[r] == 0.0:
            assert np.all(y[r] == 0.0)
        else:
            assert_close(y[r:r + 1], want[r:r + 1])


def test_skinny_register_resident_deterministic():
    n, k, m = 8200, 4096 + 64, 40
    _, packed, scale, cb, s = make(n, k, 256, seed=91)
    _, x = x_bf16(m, k, 92)
    a = run(s, x).cpu().numpy()
    b = run(s, x).cpu().numpy()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("m,n,k", [(16, 4096, 2048), (48, 2056, 4096 + 64), (24, 8200, 4096 + 64)])
def test_skinny_graph_replays_match_eager(m, n, k):
    """Captured once, replayed with new activations copied in: every replay
    equals the eager call bit for bit (the one-launch kernel; the
    register-resident kernel with three and with two splits and their
    reduction launch)."""
    _, packed, scale, cb, s = make(n, k, 256, seed=95 + m)
    h = cuda._hot(s)
    xs = torch.zeros((m, k), device=DEV, dtype=torch.bfloat16)
    ys = torch.zeros((m, n), device=DEV, dtype=torch.float32)
    cuda.forward(xs, h, out=ys)  # warm-up outside capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        cuda.forward(xs, h, out=ys)
    for i in range(3):
        x32, x = x_bf16(m, k, 200 + i)
        xs.copy_(x)
        g.replay()
        torch.cuda.synchronize()
        eager = run(s, x).cpu().numpy()
        assert np.array_equal(ys.cpu().numpy(), eager)
        assert_close(eager, rust_ref(x32, packed, scale, cb, n, k, 256, 128))


def _random_register_resident_cases(count=8, seed=2024):
    """Seeded shapes the register-resident kernel serves: M 33..64 at any
    size (and 17..32 at >= 2^25 weights), N and K ragged (K a multiple of
    16; of 64 for groups of 64), groups of 64, 128 or 256, levels 17..256."""
    g = rng(seed)
    cases = []
    while len(cases) < count:
        m = int(g.integers(17, 65))
        group = int(g.choice([64, 128, 256]))
        k = int(g.integers(2, 80)) * 64
        n = int(g.integers(1, 600)) * 8 + int(g.integers(0, 8))
        if m <= 32 and n * k < 2 ** 25:
            n = 2 ** 25 // k + 1 + int(g.integers(0, 64))
        if n * k > 40_000_000:
            continue
        cases.append((m, n, k, group, int(g.integers(17, 257))))
    return cases


@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,n,k,group,levels", _random_register_resident_cases())
def test_skinny_register_resident_random_shapes(xdt, m, n, k, group, levels):
    """Seeded random shapes.  bf16 x: the products take the f32 weights (a
    hi/lo bf16 pair of the codebook), held to the Rust-order result.  fp16 x:
    the products take fp16(cb[idx] * scale), the operands of the reference's
    Triton kernel (_triton.py:95-103), so the result is held to 1e-4 of the
    fp64 product of those operands, and normwise to the Rust order.  Against
    the Rust order per element, fp16 weight rounding (2^-11 of each weight)
    reaches 2.5e-3 of max(|y|, rms y) at 28 x 58274 outputs, K = 576."""
    _, packed, scale, cb, s = make(n, k, levels, group, seed=n + k + m + group)
    x32, x = x_bf16(m, k, 3 * m + levels)
    x = x.to(xdt)
    xr = x.float().cpu().numpy()
    want = rust_ref(xr, packed, scale, cb, n, k, levels, group)
    y = run(s, x).cpu().numpy()
    if xdt == torch.bfloat16:
        assert_close(y, want)
        return
    w16 = ref.materialize(packed, scale, cb, n, k, group, levels, "f16")
    assert_close(y, ref.linear_f64(xr, w16), 1e-4)
    err = np.abs(y.astype(np.float64) - want).max()
    assert err <= TOL * np.abs(want).max(), f"normwise {err / np.abs(want).max():.3e}"
