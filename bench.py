#!/usr/bin/env python3
"""Headline benchmark: GEMV_F32 at 2048 -> 6144 (Qwen3-1.7B gate/up shape), rows = 1.

One step = one pass of the hot path over one batch of synthetic input: 608
GEMV_F32 jobs, each on its own resident 2048 -> 6144 matrix (1.0 GiB of sign
bits + scales in total, 4x the 256 MB Infinity Cache) with its own input row,
issued as one BNNX_ExecuteBatch call (one prep launch + one group-dot launch).
Inputs are resident in HBM before timing starts.

  value            algorithmic bytes of the step / wall time of the step (GB/s);
                   per GEMV_F32 job 1,802,240 B = 1.125 bit per weight + 4K + 4N
  roofline         the dot kernel: algorithmic bytes per launch / its average
                   duration from HIP events on the device stream, against 8 TB/s
  per_call         the same operation through the reference's synchronous
                   BNN_Execute, one job per call (latency-bound at this size)
  cpu_baseline     the reference soft backend (compiled from its source into
                   oracle/_ref) or else this project's C restatement of it, one
                   host core, on a bounded sample of the same jobs

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
PKG_DIR = ROOT / "bnn-train-infer_amd"
K_IN, N_OUT = 2048, 6144
MATRICES = 608
BYTES_PER_JOB = N_OUT * K_IN // 8 + N_OUT * (K_IN // 128) * 2 + 4 * K_IN + 4 * N_OUT  # 1,802,240
HBM_PEAK_GBS = 8000.0


def load_pkg():
    name = "bnn_train_infer_amd"
    spec = importlib.util.spec_from_file_location(name, PKG_DIR / "__init__.py",
                                                  submodule_search_locations=[str(PKG_DIR)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def traffic_from_profiles():
    """HBM bytes per dot launch from the committed rocprofv3 --pmc summary, if any."""
    path = ROOT / "profiles" / "gemv_f32_2048x6144_batch608_traffic.txt"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def copy_calibration(mib: int = 256) -> None:
    """One device-to-device hipMemcpy of known size through the HIP runtime (no product
    code): rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE over this run gives the factors that
    turn those counters into bytes."""
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so")
    a, b = ctypes.c_void_p(), ctypes.c_void_p()
    n = mib << 20
    assert hip.hipMalloc(ctypes.byref(a), ctypes.c_size_t(n)) == 0
    assert hip.hipMalloc(ctypes.byref(b), ctypes.c_size_t(n)) == 0
    assert hip.hipMemset(a, 1, ctypes.c_size_t(n)) == 0
    assert hip.hipMemcpy(b, a, ctypes.c_size_t(n), 3) == 0  # hipMemcpyDeviceToDevice
    assert hip.hipDeviceSynchronize() == 0
    hip.hipFree(a)
    hip.hipFree(b)
    print(f"copy calibration: {mib} MiB device-to-device", flush=True)


def cpu_baseline(pkg, seconds: float = 12.0):
    """Bounded single-core sample of the same jobs on the host (checker-side code)."""
    ref = ROOT / "oracle" / "_ref" / "libbnn_soft_ref.so"
    port = ROOT / "oracle" / "lib" / "liboracle_cpu.so"
    path, kind = (ref, "reference") if ref.exists() else (port, "port")
    if not path.exists():
        return None
    core = sorted(os.sched_getaffinity(0))[0]
    os.sched_setaffinity(0, {core})
    api = pkg.Api(path)
    bits, scales = pkg.synth.matrix(N_OUT, K_IN, seed=3)
    x = pkg.synth.normal_f32(1, K_IN, seed=3)
    with pkg.Device(api, 0) as dev:
        m = dev.matrix(bits, scales)
        bi, bo = dev.buffer(x.nbytes), dev.buffer(4 * N_OUT)
        bi.write(x)
        job = pkg.Job(int(pkg.Op.GEMV_F32), m.handle.value, bi.view(pkg.Type.F32), bo.view(pkg.Type.F32), 1)
        calls, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < seconds:
            assert dev.execute(job) == 0
            calls += 1
        dt = time.perf_counter() - t0
        bi.free()
        bo.free()
        m.destroy()
    cpu_name = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_name = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(calls * BYTES_PER_JOB / dt / 1e9, 5), "unit": "GB/s", "cores": 1, "kind": kind,
            "sample": f"{calls} GEMV_F32 {K_IN}->{N_OUT} rows=1 calls in {dt:.1f} s on core {core} "
                      f"({cpu_name}, nproc {os.cpu_count()}), {dt / calls * 1e3:.1f} ms/call",
            "library": str(path.relative_to(ROOT))}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run one 256 MiB device-to-device copy (counter calibration)")
    args = ap.parse_args()
    if args.copy_calibration:
        copy_calibration()
        return
    if args.gpus != 1:
        print("bench.py: this build runs on exactly one GPU (the BNN_* path has no multi-GPU form here; "
              "see DESIGN.md for how it would shard).", file=sys.stderr)
        sys.exit(2)

    pkg = load_pkg()
    hip = pkg.load_hip()
    dev = pkg.Device(hip, 0)
    name, arch = dev.name()
    print(f"device: {name} {arch}", flush=True)

    # ---- resident inputs: 608 distinct matrices, input rows and output rows ----
    t0 = time.perf_counter()
    mats = []
    for i in range(MATRICES):
        bits, scales = pkg.synth.matrix(N_OUT, K_IN, seed=1000 + i)
        mats.append(dev.matrix(bits, scales))
    x = pkg.synth.normal_f32(MATRICES, K_IN, seed=3)
    bin_ = dev.buffer(x.nbytes)
    bin_.write(x)
    bout = dev.buffer(MATRICES * N_OUT * 4)
    jobs = (pkg.Job * MATRICES)()
    for i, m in enumerate(mats):
        jobs[i] = pkg.Job(int(pkg.Op.GEMV_F32), m.handle.value, bin_.view(pkg.Type.F32, i * K_IN * 4),
                          bout.view(pkg.Type.F32, i * N_OUT * 4), 1)
    print(f"setup: {MATRICES} matrices resident in {time.perf_counter() - t0:.1f} s", flush=True)

    def step():
        st = hip.BNNX_ExecuteBatch(dev.handle, jobs, MATRICES)
        if st != 0:
            raise pkg.BnnError(st, "BNNX_ExecuteBatch")

    for _ in range(args.warmup):
        step()

    # spot check the batch against the single-job path on a few jobs
    y_batch = bout.read().view(np.float32).reshape(MATRICES, N_OUT)
    for i in (0, MATRICES // 2, MATRICES - 1):
        y1 = dev.run(pkg.Op.GEMV_F32, mats[i], x[i:i + 1])
        assert np.array_equal(y1[0].view(np.uint32), y_batch[i].view(np.uint32)), f"batch job {i} differs"

    # ---- timed region (synchronous API: each call returns with its results readable) ----
    dev.kernel_timing(True)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    wall = time.perf_counter() - t0
    dot_ms, dot_n = dev.kernel_timing_read(1)
    prep_ms, prep_n = dev.kernel_timing_read(0)
    dev.kernel_timing(False)
    print(f"timed: {args.steps} steps in {wall:.3f} s", flush=True)

    step_bytes = MATRICES * BYTES_PER_JOB
    value = step_bytes * args.steps / wall / 1e9
    dot_avg_s = dot_ms / 1e3 / max(dot_n, 1)
    achieved = step_bytes / dot_avg_s / 1e9

    # ---- per-call path through BNN_Execute (one job per call), same matrices ----
    per_call_jobs = min(MATRICES, 200)
    dev.kernel_timing(True)
    t0 = time.perf_counter()
    for i in range(per_call_jobs):
        st = dev.execute(jobs[i])
        if st != 0:
            raise pkg.BnnError(st, "BNN_Execute")
    call_wall = time.perf_counter() - t0
    single_ms, single_n = dev.kernel_timing_read(1)
    single_prep_ms, _ = dev.kernel_timing_read(0)
    dev.kernel_timing(False)
    per_call = {
        "us_per_call": round(call_wall / per_call_jobs * 1e6, 2),
        "GBps_api": round(per_call_jobs * BYTES_PER_JOB / call_wall / 1e9, 2),
        "dot_kernel_us": round(single_ms / max(single_n, 1) * 1e3, 3),
        "prep_kernel_us": round(single_prep_ms / max(single_n, 1) * 1e3, 3),
        "dot_kernel_GBps": round(BYTES_PER_JOB / (single_ms / 1e3 / max(single_n, 1)) / 1e9, 1),
        "calls": per_call_jobs,
    }

    for m in mats:
        m.destroy()
    bin_.free()
    bout.free()
    dev.close()

    result = {
        "metric": "GEMV_F32 GB/s (% HBM peak) at 2048->6144",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "w1a8",
        "data": "synthetic",
        "config": {
            "workload": f"GEMV_F32 {K_IN}->{N_OUT} rows=1 (Qwen3-1.7B gate/up), {MATRICES} distinct resident "
                        f"matrices (1.0 GiB) per step in one BNNX_ExecuteBatch",
            "bytes_per_job": BYTES_PER_JOB,
            "bytes_per_step": step_bytes,
            "hbm_fraction": round(value / HBM_PEAK_GBS, 4),
            "device": f"{name} {arch}",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic_from_profiles(),
            "kernel": "k_dot_wave (batched group-dot, one wave per 64-feature tile)",
            "kernel_avg_us": round(dot_avg_s * 1e6, 2),
            "prep_kernel_avg_us": round(prep_ms / max(prep_n, 1) * 1e3, 2),
        },
        "per_call": per_call,
        "cpu_baseline": None if args.no_cpu else cpu_baseline(pkg),
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
