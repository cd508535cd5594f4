"""C ABI checks that need no GPU: the library loads, exports every symbol
include/epure_hip.h declares, and rejects bad arguments on the host side
before any launch."""
import ctypes
import os
import re

import pytest

import torch  # noqa: F401  (load torch's HIP runtime first, as the package does)

from epure.kernels import _abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", f) for f in os.listdir(os.path.join(ROOT, "include"))
           if f.endswith(".h")]


# which library exports the entry points a header declares
LIBRARY_OF = {"epure_cpu.h": "libepure_cpu.so"}


def declared_functions():
    names = set()
    for h in HEADERS:
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        lib = LIBRARY_OF.get(os.path.basename(h), "libepure_hip.so")
        for m in re.finditer(r"\b(ep_[a-z0-9_]+)\s*\(", text):
            names.add((m.group(1), lib))
    return sorted(names)


@pytest.fixture(scope="module")
def lib():
    handle = _abi._load()
    assert handle is not None, f"libepure_hip.so failed to load: {_abi.LOAD_ERROR}"
    return handle


def test_header_declares_entry_points():
    names = [n for n, _ in declared_functions()]
    for required in ("ep_dequant_matmul", "ep_dequant_matmul_bwd", "ep_unpack_indices",
                     "ep_dequant_tile", "ep_hip_available", "ep_last_error", "ep_abi_version"):
        assert required in names


@pytest.mark.parametrize("name,libname", declared_functions())
def test_library_exports_declared_symbol(lib, name, libname):
    raw = ctypes.CDLL(os.path.join(os.path.dirname(_abi.LIB_PATH), libname))
    assert hasattr(raw, name), f"{name} declared in include/ but not exported by {libname}"


def test_version(lib):
    assert lib.ep_abi_version() == _abi.ABI_VERSION == 1


def test_available_is_boolean(lib):
    assert lib.ep_hip_available() in (0, 1)
    if not torch.cuda.is_available():
        assert lib.ep_hip_available() == 0


def _matmul(lib, levels=16, group=128, M=1, N=8, K=256, xdt=_abi.BF16, sdt=_abi.F16, cb_dt=_abi.F32,
            ld_scale=2, x=1, y=1):
    # Host-side validation runs before any device access, so dummy non-null
    # pointers are never dereferenced on these paths.
    dummy = ctypes.c_void_p(16)
    return lib.ep_dequant_matmul(
        dummy if x else None, xdt, K, dummy, dummy, sdt, ld_scale, dummy, cb_dt, levels, group,
        M, N, K, dummy if y else None, _abi.BF16, N, 0, None, 0, None)


def test_rejects_levels_out_of_range(lib):
    assert _matmul(lib, levels=0) == 3
    assert _matmul(lib, levels=257) == 3
    assert "levels" in _abi.last_error()


def test_rejects_bad_dtype(lib):
    assert _matmul(lib, xdt=7) == 1
    assert _matmul(lib, sdt=9) == 1


def test_rejects_bad_args(lib):
    assert _matmul(lib, group=0) < 0
    assert _matmul(lib, ld_scale=1) < 0          # ceil(256/128) = 2 > 1
    assert _matmul(lib, M=-1) < 0
    assert _matmul(lib, x=0) < 0
    assert _matmul(lib, M=0) == 0                # empty: nothing to do
    assert _matmul(lib, N=0) == 0


def test_check_maps_codes(lib):
    assert _abi.check(0, "x") is True
    assert _abi.check(2, "x") is False
    with pytest.raises(RuntimeError):
        _abi.check(-1, "x")


def test_workspace_sizes(lib):
    assert lib.ep_dequant_matmul_workspace(1, 4096, 4096, 16, 128) >= 4
    assert lib.ep_dequant_matmul_workspace(512, 4096, 4096, 16, 128) >= 512 * 4


# ---- persistent decode step (include/epure_decode.h): host-side contract
LLAMA8B = dict(H=4096, I=14336, Hq=32, Hkv=8, D=128)
QWEN17B = dict(H=2048, I=6144, Hq=16, Hkv=8, D=128)


def _serves(lib, H, I, Hq, Hkv, D, max_pos=448, levels=16, group=128, sdt=_abi.F16, cdt=_abi.F32):
    return lib.ep_decode_step_serves(H, I, Hq, Hkv, D, max_pos, levels, group, sdt, cdt)


def test_decode_step_layer_descriptor_is_27_pointers(lib):
    assert lib.ep_decode_step_layer_bytes() == 27 * 8


def test_decode_step_workspace_size(lib):
    # 8-byte tagged values, each buffer 256-byte aligned: sync, residual
    # (2 x 32 ring slots), q, k, v, attention output (f32, 32 slots),
    # SwiGLU output (32 slots), split-KV partials
    def r(n):
        return (n * 8 + 255) // 256 * 256
    H, I, Hq, Hkv, D, P = 4096, 14336, 32, 8, 128, 448
    want = r(8) + r(64 * H) + r(Hq * D) + 2 * r(Hkv * D) + r(32 * Hq * D) + r(32 * I) + \
        r(Hq * (P // 64 + 1) * (D + 2))
    assert lib.ep_decode_step_workspace(H, I, Hq, Hkv, D, P) == want
    assert lib.ep_decode_step_workspace(H, I, 0, Hkv, D, P) == 0


@pytest.mark.parametrize("shape", [LLAMA8B, QWEN17B], ids=["llama3-8b", "qwen3-1.7b"])
def test_decode_step_serves_baseline_shapes(lib, shape):
    assert _serves(lib, **shape) == 1
    assert _serves(lib, **shape, cdt=_abi.F16) == 1


QWEN8B = dict(H=4096, I=12288, Hq=32, Hkv=8, D=128)
LLAMA3B = dict(H=3072, I=8192, Hq=24, Hkv=8, D=128)


@pytest.mark.parametrize("shape", [QWEN8B, LLAMA3B], ids=["qwen3-8b", "llama3.2-3b"])
def test_decode_step_serves_more_shapes(lib, shape):
    assert _serves(lib, **shape) == 1


@pytest.mark.parametrize("change", [
    dict(H=1024), dict(I=8192), dict(Hq=16), dict(sdt=_abi.F32), dict(H=2560, I=6656, Hq=20, Hkv=4),
    dict(Hq=8, Hkv=8)])
def test_decode_step_serves_generic_shapes(lib, change):
    """Shapes outside the tuned list (and f32 group scales) take the generic
    one-launch variants: hidden and query width <= 4096, intermediate
    <= 16384, multiples of 512, up to 8 query heads per kv head."""
    shape = dict(LLAMA8B)
    kw = {k: v for k, v in change.items() if k in ("sdt",)}
    shape.update({k: v for k, v in change.items() if k in shape})
    assert _serves(lib, **shape, **kw) == 1


@pytest.mark.parametrize("change", [
    dict(D=64), dict(levels=256), dict(group=64), dict(max_pos=100), dict(max_pos=32),
    dict(H=4352), dict(I=14592), dict(H=8192), dict(I=20480), dict(Hq=48), dict(Hkv=2),
    dict(sdt=_abi.BF16)])
def test_decode_step_declines_other_shapes(lib, change):
    """Head dim other than 128, 8-bit indices, groups below 128, a cache not
    of whole 64-position chunks, rows that are not whole 512-value slabs,
    shapes past the generic maxima, more than 8 query heads per kv head,
    bf16 scales."""
    shape = dict(LLAMA8B)
    kw = {k: v for k, v in change.items() if k in ("max_pos", "levels", "group", "sdt", "cdt")}
    shape.update({k: v for k, v in change.items() if k in shape})
    assert _serves(lib, **shape, **kw) == 0


def test_decode_step_rejects_bad_arguments_without_launch(lib):
    rc = lib.ep_decode_step(None, 32, None, None, 0, None, None, None, 4096, 14336, 32, 8, 128,
                            448, 16, 128, _abi.F16, _abi.F32, 1e-5, 1e-5, 0.088, None, None)
    assert rc < 0 and "bad arguments" in _abi.last_error()


def test_backward_workspace_empty_batch(lib):
    # no tokens: no workspace, and no division by the zero tile count
    assert lib.ep_dequant_matmul_bwd_workspace(0, 2048, 6144, 16, 128) == 0
    assert lib.ep_dequant_matmul_bwd_workspace(4, 0, 6144, 16, 128) == 0
    assert lib.ep_dequant_matmul_bwd_workspace(64, 256, 512, 16, 128) > 0
