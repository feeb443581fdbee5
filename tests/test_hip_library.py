"""CPU-side checks of the product library (no compute calls)."""
from __future__ import annotations

import ctypes
import re
import subprocess

import pytest

from conftest import PKG_DIR, ROOT


def declared_functions() -> set[str]:
    names = set()
    for header in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names |= set(re.findall(r"^\s*(?:BNN_Status|void|const char\*)\s+(BNNX?_\w+)\s*\(", text, flags=re.M))
    return names


def test_headers_declare_the_eleven_api_functions():
    api = {n for n in declared_functions() if n.startswith("BNN_")}
    assert api == {"BNN_DeviceOpen", "BNN_DeviceClose", "BNN_DeviceGetCaps", "BNN_MatrixCreate",
                   "BNN_MatrixDestroy", "BNN_BufferAlloc", "BNN_BufferFree", "BNN_BufferWrite",
                   "BNN_BufferRead", "BNN_Execute", "BNN_StatusString"}


def test_library_loads_and_exports_every_declared_symbol(pkg):
    lib = ctypes.CDLL(str(pkg.HIP_LIBRARY))
    missing = [n for n in sorted(declared_functions()) if not hasattr(lib, n)]
    assert not missing, missing


def test_library_exports_nothing_else(pkg):
    out = subprocess.run(["nm", "-D", "--defined-only", str(pkg.HIP_LIBRARY)], capture_output=True,
                         text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    assert exported == declared_functions()


def test_product_does_not_touch_the_oracle(pkg):
    needed = subprocess.run(["readelf", "-d", str(pkg.HIP_LIBRARY)], capture_output=True, text=True,
                            check=True).stdout
    assert "oracle" not in needed
    for src in list((PKG_DIR / "csrc").glob("*")) + list(PKG_DIR.glob("*.py")):
        assert "oracle" not in src.read_text().lower(), src


def test_gfx950_code_object_present(pkg):
    # the fat binary carries a gfx950 code object
    data = pkg.HIP_LIBRARY.read_bytes()
    assert b"gfx950" in data


def test_status_strings_without_gpu(pkg, hip):
    assert hip.status_string(0) == "success"
    assert hip.status_string(-7) == "device timeout"
    assert hip.status_string(99) == "unknown status"


def test_device_open_arguments(pkg, hip):
    assert hip.BNN_DeviceOpen(0, None) == pkg.Status.EINVAL
    h = ctypes.c_void_p(1234)
    assert hip.BNN_DeviceOpen(2**32 - 1, ctypes.byref(h)) == pkg.Status.ENOTSUP
    assert h.value is None
    # index != 0 is rejected before any device is touched (soft-bnn-accelerator.c:317-318)
    h = ctypes.c_void_p(1234)
    assert hip.BNN_DeviceOpen(1, ctypes.byref(h)) == pkg.Status.ENOTSUP
    assert h.value is None
    fn = hip.lib.BNNX_DeviceOpenOrdinal
    assert fn(ctypes.c_uint32(0), None) == pkg.Status.EINVAL
    h = ctypes.c_void_p(1234)
    assert fn(ctypes.c_uint32(2**32 - 1), ctypes.byref(h)) == pkg.Status.ENOTSUP
    assert h.value is None
    assert hip.BNN_DeviceClose(None) == pkg.Status.EINVAL
    caps = pkg.Caps()
    assert hip.BNN_DeviceGetCaps(None, ctypes.byref(caps)) == pkg.Status.EINVAL


def test_no_gpu_means_enotsup(pkg, hip):
    h = ctypes.c_void_p()
    st = hip.BNN_DeviceOpen(0, ctypes.byref(h))
    if st == pkg.Status.OK:
        assert hip.BNN_DeviceClose(h) == pkg.Status.OK
        pytest.skip("a GPU is present")
    assert st == pkg.Status.ENOTSUP and h.value is None
