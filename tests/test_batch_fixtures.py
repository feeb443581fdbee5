"""The batched dot kernels against the reference's own outputs.

Every single-row benchmark case of tests/bnn_cases.py runs through BNNX_ExecuteBatch
and through a prepared BNNX_BatchLaunch, and each output's SHA-256 is compared with
the soft backend's (tests/golden/soft_fixtures.json, written by the reference compiled
from source): the small batches take the group-split kernel (k_dot), the lm_head's 19
chunks as one table-mapped batch included.  Full-chip forms -- hundreds of copies of
a case's matrix, each its own resident allocation with its own input row and output --
take the one-wave-per-item kernels the headline times (k_dot_wave for K <= 2048,
k_dot_wave_long for 6144 -> 2048), uniform and table-mapped, with and without scale
reads (DOT_GROUPS-only batches read none).  No comparison goes through another HIP
entry point (soft-bnn-accelerator.c:219-276 is the function; linear.c:104-125 the
chunking).
"""
from __future__ import annotations

import ctypes
import hashlib
import json

import numpy as np
import pytest

from bnn_cases import CASES, case_inputs, input_sha, sha
from conftest import GOLDEN

pytestmark = pytest.mark.gpu
FIXTURES = json.loads((GOLDEN / "soft_fixtures.json").read_text())
ONE_ROW = [c for c in CASES if c[4] == 1]


def _row_bytes(op, n, k):
    return n * (k // 128) * 2 if op == "DOT_GROUPS" else 4 * n


def _place(pkg, dev, specs):
    """specs: [(op, matrix, x, out_row_bytes)] -> one input and one output buffer and
    the jobs, each job's input and output at its own 256-byte aligned offset."""
    ioff, ooff, jobs_io = 0, 0, []
    for op, m, x, orow in specs:
        jobs_io.append((ioff, ooff))
        ioff += -(-x.nbytes // 256) * 256
        ooff += -(-orow // 256) * 256
    bi, bo = dev.buffer(ioff), dev.buffer(ooff)
    raw = np.zeros(ioff, np.uint8)
    for (op, m, x, orow), (io, oo) in zip(specs, jobs_io):
        raw[io:io + x.nbytes] = x.view(np.uint8).reshape(-1)
    bi.write(raw)
    jobs = (pkg.Job * len(specs))()
    for i, ((op, m, x, orow), (io, oo)) in enumerate(zip(specs, jobs_io)):
        in_t, out_t = pkg.api.OP_TYPES[pkg.Op[op]]
        jobs[i] = pkg.Job(int(pkg.Op[op]), m.handle.value, bi.view(in_t, io), bo.view(out_t, oo), 1)
    return bi, bo, jobs, [oo for _, oo in jobs_io]


def _run_both(pkg, dev, jobs, bo):
    """The outputs of one BNNX_ExecuteBatch and of three prepared launches (sentinel-
    filled output before each form)."""
    api = dev.api
    outs = []
    bo.write(np.full(bo.nbytes, 0xA5, np.uint8))
    assert api.BNNX_ExecuteBatch(dev.handle, jobs, len(jobs)) == pkg.Status.OK
    outs.append(bo.read())
    bo.write(np.full(bo.nbytes, 0x5A, np.uint8))
    b = ctypes.c_void_p()
    assert api.BNNX_BatchCreate(dev.handle, jobs, len(jobs), ctypes.byref(b)) == pkg.Status.OK
    try:
        for _ in range(3):
            assert api.BNNX_BatchLaunch(b) == pkg.Status.OK
        assert api.BNNX_DeviceSynchronize(dev.handle) == pkg.Status.OK
        outs.append(bo.read())
    finally:
        api.BNNX_BatchDestroy(b)
    return outs


@pytest.mark.parametrize("case", ONE_ROW, ids=[c[0] for c in ONE_ROW])
def test_small_batch_matches_soft(pkg, hipdev, case):
    """The case's chunks as one batch (one job per chunk of at most 8192 outputs): the
    group-split kernel; its concatenated output equals the soft backend's."""
    name, op, k, n, rows, seed = case
    print(f"batch fixture {name}", flush=True)
    rec = FIXTURES[name]
    chunks, x = case_inputs(pkg, op, k, n, rows, seed)
    assert input_sha(chunks, x) == rec["input_sha256"], "synthetic generator drifted"
    mats = [hipdev.matrix(b, s) for b, s in chunks]
    widths = [b.shape[0] for b, _ in chunks]
    try:
        bi, bo, jobs, oo = _place(pkg, hipdev, [(op, m, x, _row_bytes(op, w, k)) for m, w in zip(mats, widths)])
        for form, raw in zip(("ExecuteBatch", "BatchLaunch"), _run_both(pkg, hipdev, jobs, bo)):
            out = b"".join(raw[o:o + _row_bytes(op, w, k)].tobytes() for o, w in zip(oo, widths))
            assert len(out) == rec["output_bytes"]
            assert hashlib.sha256(out).hexdigest() == rec["output_sha256"], (name, form)
        bi.free()
        bo.free()
    finally:
        for m in mats:
            m.destroy()


# (case name, copies): enough 64-feature items to fill the chip 16 times over -- the
# one-wave-per-item kernels; 608 copies of a 2048 -> 6144 matrix are the headline's
# 1.0 GiB step
FULL_CHIP = [
    ("gemv_f32_2048x6144", 608),   # k_dot_wave, uniform (the headline's form)
    ("dot_2048x6144", 100),        # k_dot_wave without scale reads
    ("gemv_i8_2048x6144", 100),    # k_dot_wave, integer input
    ("gemv_f32_2048x1024", 300),   # k_dot_wave, 16 tiles per job
    ("gemv_f32_6144x2048", 400),   # k_dot_wave_long (48 groups)
]


@pytest.mark.parametrize("name,copies", FULL_CHIP, ids=[c[0] for c in FULL_CHIP])
def test_full_chip_copies_match_soft(pkg, hipdev, name, copies):
    case = next(c for c in CASES if c[0] == name)
    _, op, k, n, rows, seed = case
    rec = FIXTURES[name]
    chunks, x = case_inputs(pkg, op, k, n, rows, seed)
    assert len(chunks) == 1 and input_sha(chunks, x) == rec["input_sha256"]
    print(f"batch fixture {name} x {copies} copies", flush=True)
    mats = []
    try:
        for _ in range(copies):
            mats.append(hipdev.matrix(*chunks[0]))
        orow = _row_bytes(op, n, k)
        bi, bo, jobs, oo = _place(pkg, hipdev, [(op, m, x, orow) for m in mats])
        for form, raw in zip(("ExecuteBatch", "BatchLaunch"), _run_both(pkg, hipdev, jobs, bo)):
            bad = [i for i, o in enumerate(oo) if sha(raw[o:o + orow]) != rec["output_sha256"]]
            assert not bad, (name, form, f"{len(bad)} of {copies} outputs differ, first job {bad[0]}")
        bi.free()
        bo.free()
    finally:
        for m in mats:
            m.destroy()


def test_full_chip_mixed_table_batch_matches_soft(pkg, hipdev):
    """Copies of four cases in one table-mapped batch (jobs of 96, 96, 96 and 32 tiles,
    one with int16 outputs): every output equals its case's soft output."""
    mix = [("gemv_f32_2048x6144", 20), ("dot_2048x6144", 12), ("gemv_i8_2048x6144", 12), ("gemv_f32_2048x2048", 20)]
    specs, names, mats = [], [], []
    try:
        for name, copies in mix:
            _, op, k, n, rows, seed = next(c for c in CASES if c[0] == name)
            chunks, x = case_inputs(pkg, op, k, n, rows, seed)
            assert input_sha(chunks, x) == FIXTURES[name]["input_sha256"]
            for _ in range(copies):
                m = hipdev.matrix(*chunks[0])
                mats.append(m)
                specs.append((op, m, x, _row_bytes(op, n, k)))
                names.append(name)
        # interleave the cases so that neighbouring items belong to different jobs
        order = np.random.default_rng(5).permutation(len(specs))
        specs = [specs[i] for i in order]
        names = [names[i] for i in order]
        assert sum(-(-(s[3] // (32 if s[0] == "DOT_GROUPS" else 4)) // 64) for s in specs) >= 256 * 16
        print(f"batch fixture mixed table batch, {len(specs)} jobs", flush=True)
        bi, bo, jobs, oo = _place(pkg, hipdev, specs)
        for form, raw in zip(("ExecuteBatch", "BatchLaunch"), _run_both(pkg, hipdev, jobs, bo)):
            for i, (o, s) in enumerate(zip(oo, specs)):
                assert sha(raw[o:o + s[3]]) == FIXTURES[names[i]]["output_sha256"], (form, i, names[i])
        bi.free()
        bo.free()
    finally:
        for m in mats:
            m.destroy()

