"""Shared fixtures.  GPU tests are marked `gpu`; everything else runs on a CPU-only host."""
from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG_DIR = ROOT / "bnn-train-infer_amd"
GOLDEN = ROOT / "tests" / "golden"
ORACLE_LIB = ROOT / "oracle" / "lib" / "liboracle_cpu.so"
REF_DIR = ROOT / "oracle" / "_ref"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def load_pkg():
    name = "bnn_train_infer_amd"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, PKG_DIR / "__init__.py",
                                                  submodule_search_locations=[str(PKG_DIR)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def pkg():
    return load_pkg()


@pytest.fixture(scope="session")
def oracle(pkg):
    """The CPU oracle (test infrastructure, never part of the product)."""
    if not ORACLE_LIB.exists():
        pytest.fail(f"oracle not built: {ORACLE_LIB} (make -C oracle)")
    return pkg.Api(ORACLE_LIB)


@pytest.fixture(scope="session")
def oracle_fast(oracle):
    """oracle_execute_parallel(op, bits, half, k, n, rows, input, out, threads)."""
    import ctypes
    fn = oracle.lib.oracle_execute_parallel
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32,
                   ctypes.c_uint32, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
    return fn


@pytest.fixture(scope="session")
def hip(pkg):
    """The product library; GPU tests fail (not skip) when it is missing."""
    return pkg.load_hip()


@pytest.fixture()
def hipdev(pkg, hip):
    dev = pkg.Device(hip, 0)
    yield dev
    dev.close()
