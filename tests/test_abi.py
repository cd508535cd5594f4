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


def declared_functions():
    names = set()
    for h in HEADERS:
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b(ep_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return sorted(names)


@pytest.fixture(scope="module")
def lib():
    handle = _abi._load()
    assert handle is not None, f"libepure_hip.so failed to load: {_abi.LOAD_ERROR}"
    return handle


def test_header_declares_entry_points():
    names = declared_functions()
    for required in ("ep_dequant_matmul", "ep_dequant_matmul_bwd", "ep_unpack_indices",
                     "ep_dequant_tile", "ep_hip_available", "ep_last_error", "ep_abi_version"):
        assert required in names


@pytest.mark.parametrize("name", declared_functions())
def test_library_exports_declared_symbol(lib, name):
    raw = ctypes.CDLL(_abi.LIB_PATH)
    assert hasattr(raw, name), f"{name} declared in include/ but not exported"


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
