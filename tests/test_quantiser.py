"""The reciprocal quantiser the kernels use (csrc/bnn_quant.h, quantize_rcp) against the
reference formula clamp(roundf(F32(x / s)), -127, 127) (soft-bnn-accelerator.c:175-211),
on the host: every finite x for a set of row scales s (normal, near FLT_MIN, subnormal,
FLT_TRUE_MIN, FLT_MAX / 127), and the floats nearest to every half-integer multiple
(k + 0.5) * s for thousands of seeded scales, with the reciprocal F32(1 / s) and with
neighbours up to two ulps away (the device multiplies by an estimate within 7 * 2^-24).
The row scale (quant_row_scale: a corrected product instead of the division) against
F32(absmax / 127) for every finite absmax >= 0.  Planted mistakes (the reciprocal product
without the division fallback; the row-scale product without its correction) must be
found by the same checker."""
from __future__ import annotations

import subprocess

import numpy as np
import pytest

from conftest import PKG_DIR, ROOT

SRC = ROOT / "tests" / "quant_sweep.cpp"
FLAGS = ["-O2", "-std=c++17", "-fno-fast-math", "-ffp-contract=off", "-I", str(PKG_DIR / "csrc")]


def _f32_bits(v) -> str:
    return f"{int(np.float32(v).view(np.uint32)):08x}"


@pytest.fixture(scope="module")
def sweep(tmp_path_factory):
    d = tmp_path_factory.mktemp("quant")
    exe, planted, planted_scale = d / "quant_sweep", d / "quant_planted", d / "quant_planted_scale"
    subprocess.run(["g++", *FLAGS, str(SRC), "-o", str(exe), "-lpthread"], check=True)
    subprocess.run(["g++", *FLAGS, "-DPLANTED_NO_DIVISION", str(SRC), "-o", str(planted), "-lpthread"],
                   check=True)
    subprocess.run(["g++", *FLAGS, "-DPLANTED_NO_CORRECTION", str(SRC), "-o", str(planted_scale), "-lpthread"],
                   check=True)
    return exe, planted, planted_scale


def _run(exe, *args):
    r = subprocess.run([str(exe), *args], capture_output=True, text=True, timeout=600)
    last = r.stdout.strip().splitlines()[-1]
    checked, bad = int(last.split()[1]), int(last.split()[3])
    return r.returncode, checked, bad, r.stdout


SCALES = {
    "1/127": np.float32(1.0) / np.float32(127.0),
    "57.3/127 (outlier row)": np.float32(57.3) / np.float32(127.0),
    "3.0": 3.0,
    "1.0 (zero row)": 1.0,
    "FLT_MIN": np.float32(2.0 ** -126),
    "FLT_MIN+1ulp": np.nextafter(np.float32(2.0 ** -126), np.float32(1)),
    "largest subnormal": np.float32(2.0 ** -126) - np.float32(2.0 ** -149),
    "FLT_TRUE_MIN": np.float32(2.0 ** -149),
    "FLT_MAX/127": np.float32(np.finfo(np.float32).max) / np.float32(127.0),
}


@pytest.mark.parametrize("name", list(SCALES))
def test_every_finite_x(sweep, name):
    rc, checked, bad, out = _run(sweep[0], "full", _f32_bits(SCALES[name]))
    assert checked == 2 ** 32 - 2 ** 24, checked  # all patterns but the Inf/NaN exponent
    assert bad == 0 and rc == 0, out


def test_half_integer_neighbourhoods(sweep):
    rc, checked, bad, out = _run(sweep[0], "near", "20000", "7")
    assert checked > 3_000_000_000  # five reciprocals per x
    assert bad == 0 and rc == 0, out


def test_row_scale_every_absmax(sweep):
    rc, checked, bad, out = _run(sweep[0], "scale")
    assert checked == 2 ** 31 - 2 ** 23, checked  # every finite absmax >= 0
    assert bad == 0 and rc == 0, out


def test_checker_finds_a_planted_scale_mistake(sweep):
    rc, checked, bad, out = _run(sweep[2], "scale")
    assert rc == 1 and bad > 0, out


def test_checker_finds_a_planted_mistake(sweep):
    rc, checked, bad, out = _run(sweep[1], "near", "2000", "7")
    assert rc == 1 and bad > 0, out
