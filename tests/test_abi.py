"""The C-ABI library: it loads, and exports exactly what include/mace_hip.h declares.

No compute call is made here (this suite also runs without a GPU)."""

import ctypes
import re
from pathlib import Path

import pytest

from mace_mlx_amd import _ffi

HEADER = Path(__file__).resolve().parents[1] / "include" / "mace_hip.h"


def _declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(mace_[a-z_]+)\s*\(", text)))


@pytest.mark.parametrize("channels", _ffi.ENGINE_WIDTHS)
def test_library_loads_and_exports_every_declared_symbol(channels):
    """Each channel width's library (libmace_hip.so, libmace_hip_c192.so, libmace_hip_c256.so)."""
    lib = _ffi.load_library(channels=channels)
    declared = _declared()
    assert set(declared) == set(_ffi.EXPORTED_SYMBOLS)
    for name in declared:
        assert isinstance(getattr(lib, name), ctypes._CFuncPtr), name


def test_model_dims_struct_matches_header():
    text = HEADER.read_text()
    body = text[text.index("typedef struct mace_model_dims"):text.index("} mace_model_dims;")]
    fields = re.findall(r"^\s*(int32_t|double)\s+(\w+)(\[\d+\])?;", body, re.M)
    names = [f[1] for f in fields]
    assert names == [f[0] for f in _ffi.ModelDims._fields_]
    size = 0
    for ty, _, arr in fields:
        n = int(arr[1:-1]) if arr else 1
        sz = 4 if ty == "int32_t" else 8
        size = (size + sz - 1) // sz * sz + sz * n
    assert ctypes.sizeof(_ffi.ModelDims) == (size + 7) // 8 * 8


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(ImportError):
        _ffi.load_library(str(tmp_path / "nope.so"))


def _symcheck():
    import importlib.util
    p = Path(__file__).resolve().parents[1] / "mace-mlx_amd" / "csrc" / "check_kernel_symbols.py"
    spec = importlib.util.spec_from_file_location("check_kernel_symbols", p)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_every_registered_kernel_is_in_the_gfx950_code_object():
    """The HIP runtime aborts at the first launch of a kernel whose host-registered
    (mangled) name is absent from the device code object; host and device mangle
    differently when a kernel parameter type depends on an unnamed enum."""
    chk = _symcheck()
    assert chk.check(_ffi.LIB_PATH) == []


def test_symbol_check_detects_a_missing_kernel():
    """Plant a mismatch: drop one kernel from the device-name set the check compares with."""
    chk = _symcheck()
    data = Path(_ffi.LIB_PATH).read_bytes()
    host, dev = chk.host_kernels(data), chk.device_kernels(data)
    assert host and host <= dev
    victim = sorted(host)[0]
    assert sorted(host - (dev - {victim})) == [victim]
    assert any("k_tp_bwd_recv" in h for h in host) and any("k_mlp_out" in h for h in host)
