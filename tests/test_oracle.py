"""Pins the CPU oracle (oracle/bnn_cpu.c) before anything is compared against it.

Checks, each chosen so that a plausible mistake fails one of them:
  - the reference's own contract test (tests/accelerator/test_bnn_accelerator.c,
    with its independent scalar oracle) passes against the oracle, and its raw
    output dump is byte-identical to the one it produces against the reference soft backend;
  - the reference's RTL golden case (bnn-hw-v2/simple_test/tests/case) is reproduced bit-exactly;
  - soft-backend outputs at every benchmark shape (tests/golden/soft_fixtures.json) match;
  - binary16 -> binary32 conversion, exhaustively against numpy's float16;
  - the quantiser against exact rational arithmetic (round half away from zero, ties included);
  - D against a brute-force signed-product sum, including the +-16256 extremes;
  - the fast row-parallel evaluation is bit-identical to the scalar path.
"""
from __future__ import annotations

import ctypes
import json
import subprocess
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

from bnn_cases import CASES, case_inputs, fast_oracle, first_mismatch, input_sha, run_chunks, sha
from conftest import GOLDEN, REF_DIR, ROOT


def _run(path: Path, *args):
    return subprocess.run([str(path), *map(str, args)], capture_output=True, text=True, timeout=300)


def test_reference_contract_suite_passes_on_oracle(tmp_path):
    exe = REF_DIR / "test_ref_vs_oracle"
    if not exe.exists():
        pytest.skip("oracle/_ref not built (reference tree absent when building)")
    dump = tmp_path / "dump.bin"
    r = _run(exe, dump)
    assert r.returncode == 0, r.stderr
    assert "453 successful jobs" in r.stdout
    want = json.loads((GOLDEN / "ref_suite.json").read_text())
    data = dump.read_bytes()
    assert len(data) == want["bytes"]
    import hashlib
    assert hashlib.sha256(data).hexdigest() == want["sha256"]


def test_abi_layout_matches_reference_header():
    own = _run(ROOT / "oracle/lib/abi_probe_own")
    assert own.returncode == 0
    assert own.stdout == (GOLDEN / "abi_layout.txt").read_text()
    ref = REF_DIR / "abi_probe_ref"
    if ref.exists():
        assert _run(ref).stdout == own.stdout


def _rtl(pkg, dev):
    case = np.load(GOLDEN / "rtl_case.npz")
    bits, scales = case["bits"], case["scales"]
    full = dev.matrix(bits, scales)
    tile = dev.matrix(np.ascontiguousarray(bits[:, :16]), np.ascontiguousarray(scales[:, :1]))
    try:
        got = {
            "golden_full_i8": dev.run(pkg.Op.GEMM, full, case["q_full"]),
            "golden_tile_i8": dev.run(pkg.Op.GEMM, tile, case["q_tile"]),
            "golden_tile_f32": dev.run(pkg.Op.GEMM_F32, tile, case["f32_tile"]),
        }
    finally:
        full.destroy()
        tile.destroy()
    return case, got


def test_rtl_golden_case_bit_exact(pkg, oracle):
    with pkg.Device(oracle, 0) as dev:
        case, got = _rtl(pkg, dev)
    for name, out in got.items():
        assert np.array_equal(out.view(np.uint32), case[name]), (name, first_mismatch(out.view(np.uint32), case[name]))


FIXTURES = json.loads((GOLDEN / "soft_fixtures.json").read_text())
# the multi-row M=1024 cases take ~1 min each on the scalar oracle; the fast path covers them
SCALAR_CASES = [c for c in CASES if c[4] <= 64 and c[0] != "lm_head_2048x151669"]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_oracle_fast_path_matches_soft_fixtures(pkg, oracle_fast, case):
    name, op, k, n, rows, seed = case
    rec = FIXTURES[name]
    chunks, x = case_inputs(pkg, op, k, n, rows, seed)
    assert input_sha(chunks, x) == rec["input_sha256"], "synthetic generator drifted"
    out = np.concatenate([fast_oracle(pkg, oracle_fast, op, b, s, x, threads=8) for b, s in chunks], axis=1)
    assert sha(out) == rec["output_sha256"]


@pytest.mark.parametrize("case", SCALAR_CASES[:6], ids=[c[0] for c in SCALAR_CASES[:6]])
def test_oracle_scalar_path_matches_soft_fixtures(pkg, oracle, case):
    name, op, k, n, rows, seed = case
    chunks, x = case_inputs(pkg, op, k, n, rows, seed)
    with pkg.Device(oracle, 0) as dev:
        out = run_chunks(pkg, dev, op, chunks, x)
    assert sha(out) == FIXTURES[name]["output_sha256"]
    small = np.load(GOLDEN / "soft_small.npz")
    if name in small.files:
        assert np.array_equal(out.view(np.uint8), small[name].view(np.uint8))


def _half_to_float(oracle):
    fn = oracle.lib.oracle_half_to_float
    fn.restype = ctypes.c_float
    fn.argtypes = [ctypes.c_uint16]
    return fn


def test_half_to_float_exhaustive(oracle):
    fn = _half_to_float(oracle)
    got = np.array([fn(h) for h in range(65536)], np.float32)
    want = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    # literal table of the reference test (test_bnn_accelerator.c:28-35)
    table = {0x3c00: 1.0, 0xbc00: -1.0, 0x3800: 0.5, 0x4000: 2.0, 0x0001: 2.0**-24, 0x8001: -2.0**-24,
             0x03ff: 1023 * 2.0**-24, 0x0400: 2.0**-14, 0x8000: -0.0, 0x3c01: 1 + 2.0**-10, 0x7bff: 65504.0}
    for h, v in table.items():
        assert np.float32(fn(h)).tobytes() == np.float32(v).tobytes()


def _exact_quantize(x: np.ndarray):
    """Independent restatement by exact rationals of the contract (bnn-accelerator.h:141-149)."""
    x = x.astype(np.float32)
    a = np.float32(np.max(np.abs(x)))
    if a == 0:
        s = np.float32(1)
    else:
        s = np.float32(a) / np.float32(127)  # IEEE binary32 division (numpy), correctly rounded
        if s == 0:
            s = np.float32(2.0**-149)
    q = []
    for v in x:
        y = np.float32(v) / s  # one correctly rounded binary32 division
        f = Fraction(float(y))
        mag = int((abs(f) + Fraction(1, 2)).__floor__())  # half away from zero
        r = mag if f >= 0 else -mag
        q.append(max(-127, min(127, r)))
    return np.array(q, np.int8), s


def _quantize(oracle):
    fn = oracle.lib.oracle_quantize_row
    fn.restype = ctypes.c_float
    fn.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_void_p]

    def q(x):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty(x.size, np.int8)
        s = fn(x.ctypes.data, x.size, out.ctypes.data)
        return out, np.float32(s)
    return q


def _quant_rows():
    rng = np.random.default_rng(0)  # test-only randomness; results are compared exactly
    rows = [
        np.array([127.0, -127.0] + [k % 8 + 0.5 for k in range(126)], np.float32),  # exact ties
        np.array([(-1) ** k * (k % 8 + 0.5) for k in range(128)] + [127.0], np.float32),
        np.ldexp(np.arange(-125, 126, dtype=np.float32), -149).astype(np.float32),  # subnormal inputs
        np.array([2.0**-149, -(2.0**-149)] * 64, np.float32),  # a/127 underflows: s = FLT_TRUE_MIN
        np.zeros(128, np.float32),
        np.array([np.finfo(np.float32).max, -np.finfo(np.float32).max, 1e30, -3e37], np.float32),
        np.array([0.49999997, 0.5, 1.5, 2.5, -0.5, -2.5, 126.5, 127.0], np.float32),
        rng.standard_normal(512).astype(np.float32),
        (rng.standard_normal(384) * 1e-38).astype(np.float32),
    ]
    # values that land exactly on .5 after division by a non-trivial scale
    s = np.float32(3.0) / np.float32(127)
    rows.append(np.array([3.0] + [np.float32(np.float32(j + 0.5) * s) for j in range(-20, 20)], np.float32))
    return rows


@pytest.mark.parametrize("i", range(10))
def test_quantizer_matches_exact_rationals(oracle, i):
    x = _quant_rows()[i]
    got_q, got_s = _quantize(oracle)(x)
    want_q, want_s = _exact_quantize(x)
    assert got_s.tobytes() == np.float32(want_s).tobytes()
    assert np.array_equal(got_q, want_q)


def _brute_dot(bits, q, n, g):
    w = np.unpackbits(bits[n, g * 16:(g + 1) * 16], bitorder="little").astype(np.int32) * 2 - 1
    return int(np.dot(w, q[g * 128:(g + 1) * 128].astype(np.int32)))


def test_dot_groups_brute_force_and_extremes(pkg, oracle):
    bits, scales = pkg.synth.matrix(5, 384, seed=9)
    q = pkg.synth.int8_uniform(3, 384, seed=9)
    # row 2: the +-16256 extremes (test_bnn_accelerator.c:493-517)
    w0 = np.unpackbits(bits[0], bitorder="little").astype(np.int32) * 2 - 1
    q[2] = (w0 * np.where((np.arange(384) // 128) % 2 == 0, 127, -127)).astype(np.int8)
    with pkg.Device(oracle, 0) as dev:
        m = dev.matrix(bits, scales)
        out = dev.run(pkg.Op.DOT_GROUPS, m, q)
        m.destroy()
    for r in range(3):
        for n in range(5):
            for g in range(3):
                assert out[r, n, g] == _brute_dot(bits, q[r], n, g)
    assert list(out[2, 0]) == [16256, -16256, 16256]


def _h(v: float) -> int:
    return int(np.float16(v).view(np.uint16))


def sum_order_case():
    """Row 0 separates sequential from pairwise/reversed sums; row 1 separates round-then-add from FMA.

    Row 0: D = [127, 1, 127, 1], scales [2048, 2^-14, -2048, 2^-14]:
      sequential ((((0 + 260096) + 2^-14) - 260096) + 2^-14) = 2^-14   (first 2^-14 absorbed)
      pairwise   (260096 + 2^-14) + (-260096 + 2^-14)        = 0
      reversed   (((2^-14 - 260096) + 2^-14) + 260096)        = 0
    Row 1: D = [16255, 16255], scales [-2047/1024, 2047/1024]: the product 16255*2047/1024
      needs 25 bits and rounds to 33273984/1024, so round-then-add gives 0 while
      fma(s1, D1, acc) gives 2^-10.
    Returns (bits, scales, q [2][512] int8, expected Z [2] float32 with N = 2 rows of weights).
    """
    k = 512
    bits = np.full((2, k // 8), 0xFF, np.uint8)  # all +1
    scales = np.array([[_h(2048.0), _h(2.0**-14), _h(-2048.0), _h(2.0**-14)],
                       [_h(-2047 / 1024), _h(2047 / 1024), _h(0.0), _h(0.0)]], np.uint16)
    q = np.zeros((2, k), np.int8)
    q[0, 0], q[0, 128], q[0, 256], q[0, 384] = 127, 1, 127, 1
    q[1, 0:128] = 127
    q[1, 0] = 126
    q[1, 128:256] = q[1, 0:128]
    return bits, scales, q, np.array([2.0**-14, 0.0], np.float32)


def test_fp32_accumulation_order_is_sequential(pkg, oracle):
    bits, scales, q, want = sum_order_case()
    with pkg.Device(oracle, 0) as dev:
        m = dev.matrix(bits, scales)
        z = dev.run(pkg.Op.GEMM, m, q)
        m.destroy()
    assert z[0, 0] == want[0]  # weights row 0 against activation row 0
    assert z[1, 1] == want[1]  # weights row 1 against activation row 1
    # the alternatives really differ on these inputs
    p = np.float32(16255) * np.float32(2047 / 1024)
    assert np.float32(np.float32(-p) + p) == 0.0
    assert np.float64(16255) * (2047 / 1024) - float(p) != 0.0


@pytest.mark.parametrize("op", ["DOT_GROUPS", "GEMV", "GEMM", "GEMV_F32", "GEMM_F32"])
def test_fast_path_equals_scalar_path(pkg, oracle, oracle_fast, op):
    rows = 1 if op.startswith("GEMV") else 5
    k, n = 1024, 37
    bits, _ = pkg.synth.matrix(n, k, seed=11)
    # every finite fp16 class: normal, subnormal, signed zero, max
    specials = np.array([0x3c00, 0x8001, 0x0001, 0x03ff, 0x8000, 0x0000, 0x7bff, 0xfbff, 0x2e66], np.uint16)
    scales = specials[np.arange(n * (k // 128)) % specials.size].reshape(n, k // 128)
    x = (pkg.synth.normal_f32(rows, k, seed=11) if op.endswith("F32") else pkg.synth.int8_uniform(rows, k, seed=11))
    with pkg.Device(oracle, 0) as dev:
        want = run_chunks(pkg, dev, op, [(bits, scales)], x)
    got = fast_oracle(pkg, oracle_fast, op, bits, scales, x, threads=3)
    assert np.array_equal(got.view(np.uint8), want.view(np.uint8)), first_mismatch(got, want)


def test_soft_live_random_cases(pkg, oracle):
    """Direct comparison with the reference soft backend built from source, where present."""
    soft_path = REF_DIR / "libbnn_soft_ref.so"
    if not soft_path.exists():
        pytest.skip("oracle/_ref/libbnn_soft_ref.so not built")
    soft = pkg.Api(soft_path)
    with pkg.Device(soft, 0) as ds, pkg.Device(oracle, 0) as do:
        for seed, (k, n, rows) in enumerate([(128, 1, 1), (256, 9, 2), (1152, 70, 3), (8192, 5, 2)]):
            bits, scales = pkg.synth.matrix(n, k, seed=100 + seed)
            for op in ("DOT_GROUPS", "GEMM", "GEMM_F32"):
                x = (pkg.synth.normal_f32(rows, k, seed=seed) if op.endswith("F32")
                     else pkg.synth.int8_uniform(rows, k, seed=seed))
                a = run_chunks(pkg, ds, op, [(bits, scales)], x)
                b = run_chunks(pkg, do, op, [(bits, scales)], x)
                assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), (op, k, n, rows)
