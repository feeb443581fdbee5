#!/usr/bin/env python3
"""Headline benchmark: GEMV_F32 at 2048 -> 6144 (Qwen3-1.7B gate/up shape), rows = 1.

One step = one pass of the hot path over one batch of synthetic input: 608
GEMV_F32 jobs, each on its own resident 2048 -> 6144 matrix (1.0 GiB of sign
bits + scales in total, 4x the 256 MB Infinity Cache) with its own input row,
issued as one prepared batch launch (one prep launch + one group-dot launch).
Inputs are resident in HBM before timing starts.  The GPU is pre-warmed with
0.5 s of back-to-back steps (it leaves its idle clocks only after some
milliseconds of work), then the declared warmup steps, a kernel pass (K steps
with HIP events on every dispatch), and the K timed steps, launched back to
back and closed by one BNNX_DeviceSynchronize.

  value            algorithmic bytes of the step / wall time of the step (GB/s);
                   per GEMV_F32 job 1,802,240 B = 1.125 bit per weight + 4K + 4N;
                   config.sync_GBps is the same step through the synchronous
                   BNNX_ExecuteBatch (one host round trip per step)
  roofline         the dot kernel: algorithmic bytes per launch / its average
                   duration from HIP events on the device stream (kernel pass),
                   against 8 TB/s; step_frac is value / 8 TB/s
  per_call         the same operation through the reference's synchronous
                   BNN_Execute, one job per call (latency-bound at this size)
  cpu_baseline     the reference soft backend (compiled from its source into
                   oracle/_ref) or else this project's C restatement of it, one
                   host core, on a bounded sample of the same jobs; `configs` holds
                   the same for every benchmark configuration (per-shape samples
                   composed into samples/s, GB/s, TOPS and tok/s)

Secondary legs (the other benchmark configurations; --no-extra skips them):
  ops              configs 2/3: DOT_GROUPS, GEMV_I8 and the GEMV_F32 Qwen3 shapes,
                   per call (BNN_Execute) and sustained over >= 1 GiB of distinct
                   resident matrices in one BNNX_ExecuteBatch per step
  gemm             config 4: GEMM_F32 / GEMM_I8 at rows 64/256/1024 (and 8/32, prefill-sized)
                   on the matrix cores: TOPS and utilisation of the 5.0 POPS dense int8 peak
  e2e              config 5: Qwen3-1.7B-shape greedy decode (random-init Q1_0 model,
                   32 prompt + 128 new tokens) through the engine: the device path
                   (fused batches), the device path with prepared batches, and the
                   reference call pattern; tok/s, backend share of step time,
                   token agreement with the reference engine + soft backend (fixture)
  mlp              config 1: bnn-mlp classifier, 1000 samples in batches of 64

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-extra] [--only LEG]
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import os
import sys
import threading
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


def alg_bytes(op: str, k: int, n: int, rows: int = 1) -> int:
    """Algorithmic bytes of one job: sign bits + fp16 scales (not read by DOT_GROUPS) +
    input rows + output rows."""
    weights = n * k // 8 + (0 if op == "DOT_GROUPS" else n * (k // 128) * 2)
    in_row = 4 * k if op.endswith("F32") else k
    out_row = n * (k // 128) * 2 if op == "DOT_GROUPS" else 4 * n
    return weights + rows * (in_row + out_row)


# Per decode token at the Qwen3-1.7B shape, the reference caller's BNN_Execute calls by
# shape (bnne_linear_forward, linear.c:161-216): per layer q, k, v, o, gate, up, down; the
# lm_head as 18 chunks of 8192 outputs and one of 4213 (bnne_linear_init, linear.c:104-125).
DECODE_CALLS = [((2048, 2048), 56), ((2048, 1024), 56), ((2048, 6144), 56), ((6144, 2048), 28),
                ((2048, 8192), 18), ((2048, 4213), 1)]
MLP_SHAPES = [(896, 512), (512, 512), (512, 10)]  # bnn-mlp blocks, one GEMV_F32 each per sample


def cpu_all_cores(pkg, api, cores, seconds: float = 3.0):
    """The headline job on every allowed host core at once: one thread per core, each
    pinned to its core with its own device handle (the backend's devices are independent)
    and its own matrix, calling BNN_Execute for `seconds` after a common start; aggregate
    GB/s = all calls' algorithmic bytes / the slowest thread's time.  The threads are joined
    before this returns."""
    results = [None] * len(cores)
    start = threading.Barrier(len(cores))

    def work(i, core):
        os.sched_setaffinity(0, {core})  # this thread only
        with pkg.Device(api, 0) as dev:
            bits, scales = pkg.synth.matrix(N_OUT, K_IN, seed=3)
            x = pkg.synth.normal_f32(1, K_IN, seed=3)
            m = dev.matrix(bits, scales)
            bi, bo = dev.buffer(x.nbytes), dev.buffer(4 * N_OUT)
            bi.write(x)
            job = pkg.Job(int(pkg.Op.GEMV_F32), m.handle.value, bi.view(pkg.Type.F32), bo.view(pkg.Type.F32), 1)
            start.wait()
            calls, t0 = 0, time.perf_counter()
            while calls == 0 or time.perf_counter() - t0 < seconds:
                if dev.execute(job) != 0:
                    break
                calls += 1
            results[i] = (calls, time.perf_counter() - t0)
            bi.free()
            bo.free()
            m.destroy()

    threads = [threading.Thread(target=work, args=(i, c)) for i, c in enumerate(cores)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    if any(r is None for r in results):
        return None
    calls = sum(c for c, _ in results)
    wall = max(w for _, w in results)
    return {"value": round(calls * BYTES_PER_JOB / wall / 1e9, 5), "unit": "GB/s", "cores": len(cores),
            "sample": f"{calls} GEMV_F32 {K_IN}->{N_OUT} rows=1 calls over {len(cores)} threads, one per core "
                      f"(cores {cores[0]}..{cores[-1]}), in {wall:.1f} s"}


def cpu_baseline(pkg, seconds: float = 6.0, per_shape: float = 0.8):
    """Bounded single-core samples on the host (checker-side code): the headline job for
    `seconds`, then every benchmark configuration -- each distinct job shape timed for
    about `per_shape` seconds (at least one call) and composed into the configuration's
    unit (samples/s, GB/s, TOPS, tok/s); beside them the headline job on all allowed
    cores at once (`all_cores`)."""
    ref = ROOT / "oracle" / "_ref" / "libbnn_soft_ref.so"
    port = ROOT / "oracle" / "lib" / "liboracle_cpu.so"
    path, kind = (ref, "reference") if ref.exists() else (port, "port")
    if not path.exists():
        return None
    api = pkg.Api(path)
    allowed = sorted(os.sched_getaffinity(0))
    all_cores = cpu_all_cores(pkg, api, allowed)
    core = allowed[0]
    os.sched_setaffinity(0, {core})
    t_all = time.perf_counter()

    def per_call(dev, op, k, n, rows, seed, budget):
        """Seconds per BNN_Execute of one job of this shape, over `budget` seconds."""
        bits, scales = pkg.synth.matrix(n, k, seed=seed)
        f32 = op.endswith("F32")
        x = pkg.synth.normal_f32(rows, k, seed=seed) if f32 else pkg.synth.int8_uniform(rows, k, seed=seed)
        in_t, out_t = pkg.api.OP_TYPES[pkg.Op[op]]
        out_row = n * (k // 128) * 2 if op == "DOT_GROUPS" else 4 * n
        m = dev.matrix(bits, scales)
        bi, bo = dev.buffer(x.nbytes), dev.buffer(rows * out_row)
        bi.write(x)
        job = pkg.Job(int(pkg.Op[op]), m.handle.value, bi.view(in_t), bo.view(out_t), rows)
        calls, t0 = 0, time.perf_counter()
        while calls == 0 or time.perf_counter() - t0 < budget:
            assert dev.execute(job) == 0
            calls += 1
        dt = time.perf_counter() - t0
        bi.free()
        bo.free()
        m.destroy()
        return dt / calls, calls

    configs = {}
    with pkg.Device(api, 0) as dev:
        head, calls = per_call(dev, "GEMV_F32", K_IN, N_OUT, 1, 3, seconds)
        shape_s = {}

        def gemv_f32(k, n):
            if (k, n) not in shape_s:
                shape_s[(k, n)] = per_call(dev, "GEMV_F32", k, n, 1, 3, per_shape)[0]
            return shape_s[(k, n)]

        shape_s[(K_IN, N_OUT)] = head
        # config 1: bnn-mlp, the reference engine's pattern (one GEMV_F32 per block and sample)
        per_sample = sum(gemv_f32(k, n) for k, n in MLP_SHAPES)
        configs["1 bnn-mlp 896->512->512->10, one GEMV_F32 per block and sample"] = {
            "samples_per_s": round(1.0 / per_sample, 2), "ms_per_sample": round(per_sample * 1e3, 3),
            "bytes_per_sample": sum(alg_bytes("GEMV_F32", k, n) for k, n in MLP_SHAPES)}
        # config 2: single-op microbench at one row
        for op in ("DOT_GROUPS", "GEMV"):
            t, c = per_call(dev, op, 2048, 6144, 1, 2, per_shape)
            configs[f"2 {op} 2048->6144"] = {"ms_per_call": round(t * 1e3, 3),
                                             "GBps": round(alg_bytes(op, 2048, 6144) / t / 1e9, 5), "calls": c}
        # config 3: the GEMV_F32 sweep; the lm_head as its 19 chunks
        for k, n in ((2048, 2048), (2048, 1024), (2048, 6144), (6144, 2048)):
            t = gemv_f32(k, n)
            configs[f"3 GEMV_F32 {k}->{n}"] = {"ms_per_call": round(t * 1e3, 3),
                                               "GBps": round(alg_bytes("GEMV_F32", k, n) / t / 1e9, 5)}
        lm = 18 * gemv_f32(2048, 8192) + gemv_f32(2048, 4213)
        lm_bytes = 18 * alg_bytes("GEMV_F32", 2048, 8192) + alg_bytes("GEMV_F32", 2048, 4213)
        configs["3 GEMV_F32 2048->151669 (19 chunks)"] = {"ms_per_call": round(lm * 1e3, 2),
                                                          "GBps": round(lm_bytes / lm / 1e9, 5)}
        # config 4: one multi-row job per op at 64 rows
        for op in ("GEMM", "GEMM_F32"):
            t, c = per_call(dev, op, 2048, 6144, 64, 4, 0.0)
            configs[f"4 {op} 2048->6144 rows=64"] = {"ms_per_call": round(t * 1e3, 1),
                                                     "TOPS": round(2.0 * 64 * 2048 * 6144 / t / 1e12, 6)}
        # config 5: one decode token's 215 calls, composed from the per-shape times
        token = sum(gemv_f32(k, n) * count for (k, n), count in DECODE_CALLS)
        configs["5 Qwen3-1.7B-shape decode, 215 GEMV_F32 calls per token"] = {
            "tok_per_s": round(1.0 / token, 4), "s_per_token": round(token, 2),
            "calls_per_token": sum(c for _, c in DECODE_CALLS)}
    cpu_name = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_name = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(BYTES_PER_JOB / head / 1e9, 5), "unit": "GB/s", "cores": 1, "kind": kind,
            "sample": f"{calls} GEMV_F32 {K_IN}->{N_OUT} rows=1 calls in {head * calls:.1f} s on core {core} "
                      f"({cpu_name}, nproc {os.cpu_count()}), {head * 1e3:.1f} ms/call; per config below, each "
                      f"job shape timed for ~{per_shape} s (one call at least); {time.perf_counter() - t_all:.0f} s "
                      f"in all",
            "library": str(path.relative_to(ROOT)), "configs": configs, "all_cores": all_cores}


def _timed_calls(dev, job, reps):
    """Average wall time of `reps` BNN_Execute calls (no timing events: they slow each
    dispatch), then of the dot/gemm kernels over `reps` more calls with events."""
    t0 = time.perf_counter()
    for _ in range(reps):
        st = dev.execute(job)
        if st != 0:
            raise RuntimeError(f"BNN_Execute: {st}")
    wall = (time.perf_counter() - t0) / reps
    dev.kernel_timing(True)
    for _ in range(reps):
        st = dev.execute(job)
        if st != 0:
            raise RuntimeError(f"BNN_Execute: {st}")
    dot_ms, dot_n = dev.kernel_timing_read(1)
    gemm_ms, gemm_n = dev.kernel_timing_read(3)
    prep_ms, prep_n = dev.kernel_timing_read(0)
    dev.kernel_timing(False)
    kern = (dot_ms + gemm_ms) / max(dot_n + gemm_n, 1) / 1e3
    return wall, kern, prep_ms / max(prep_n, 1) / 1e3


def ops_leg(pkg, hip):
    """Configs 2 and 3 per call and sustained."""
    out = {}
    shapes = [("DOT_GROUPS", 2048, 6144), ("GEMV", 2048, 6144), ("GEMV_F32", 2048, 2048), ("GEMV_F32", 2048, 1024),
              ("GEMV_F32", 2048, 6144), ("GEMV_F32", 6144, 2048)]
    with pkg.Device(hip, 0) as dev:
        for op, k, n in shapes:
            f32 = op.endswith("F32")
            in_t, out_t = pkg.api.OP_TYPES[pkg.Op[op]]
            bits, scales = pkg.synth.matrix(n, k, seed=2)
            x = pkg.synth.normal_f32(1, k, seed=3) if f32 else pkg.synth.int8_uniform(1, k, seed=2)
            out_row = n * (k // 128) * 2 if op == "DOT_GROUPS" else 4 * n
            in_row = 4 * k if f32 else k
            weight_bytes = n * k // 8 + (0 if op == "DOT_GROUPS" else n * (k // 128) * 2)
            unit = weight_bytes + in_row + out_row  # algorithmic bytes per call
            count = max(64, -(-(1 << 30) // weight_bytes))  # >= 1 GiB of distinct matrices
            mats = [dev.matrix(bits, scales) for _ in range(count)]
            bi = dev.buffer(in_row * count)
            bi.write(np.concatenate([x.reshape(-1).view(np.uint8)] * count))
            bo = dev.buffer(out_row * count)
            jobs = (pkg.Job * count)()
            for i, m in enumerate(mats):
                jobs[i] = pkg.Job(int(pkg.Op[op]), m.handle.value, bi.view(in_t, i * in_row), bo.view(out_t, i * out_row), 1)
            for _ in range(5):  # first-launch costs out of the timing
                assert dev.execute(jobs[0]) == 0
            wall, kern, prep = _timed_calls(dev, jobs[0], 50)
            for _ in range(20):  # sustained: past the clock ramp of a fresh burst
                assert hip.BNNX_ExecuteBatch(dev.handle, jobs, count) == 0
            reps, t0 = 50, time.perf_counter()
            for _ in range(reps):
                assert hip.BNNX_ExecuteBatch(dev.handle, jobs, count) == 0
            bwall = (time.perf_counter() - t0) / reps
            dev.kernel_timing(True)  # kernel durations in a second pass (events slow each dispatch)
            for _ in range(reps):
                assert hip.BNNX_ExecuteBatch(dev.handle, jobs, count) == 0
            dms, dn = dev.kernel_timing_read(1)
            dev.kernel_timing(False)
            out[f"{op} {k}->{n}"] = {
                "bytes_per_call": unit, "per_call_us": round(wall * 1e6, 2), "kernel_us": round(kern * 1e6, 2),
                "prep_us": round(prep * 1e6, 2),
                "sustained_GBps": round(count * unit / bwall / 1e9, 1),
                "sustained_kernel_GBps": round(count * unit / (dms / dn / 1e3) / 1e9, 1),
                "matrices": count}
            for m in mats:
                m.destroy()
            bi.free()
            bo.free()
        # lm_head: 2048 -> 151669 as 19 chunks of <= 8192 outputs in one batch
        k, n_total, chunk = 2048, 151669, 8192
        bits, scales = pkg.synth.matrix(chunk, k, seed=3)
        x = pkg.synth.normal_f32(1, k, seed=3)
        bi = dev.buffer(4 * k)
        bi.write(x)
        bo = dev.buffer(4 * n_total)
        sizes = [min(chunk, n_total - o) for o in range(0, n_total, chunk)]
        mats = [dev.matrix(bits[:sz], scales[:sz]) for sz in sizes]
        jobs = (pkg.Job * len(sizes))()
        for i, (m, sz) in enumerate(zip(mats, sizes)):
            jobs[i] = pkg.Job(int(pkg.Op.GEMV_F32), m.handle.value, bi.view(pkg.Type.F32),
                              bo.view(pkg.Type.F32, 4 * i * chunk), 1)
        for _ in range(3):
            assert hip.BNNX_ExecuteBatch(dev.handle, jobs, len(sizes)) == 0
        reps, t0 = 50, time.perf_counter()
        for _ in range(reps):
            assert hip.BNNX_ExecuteBatch(dev.handle, jobs, len(sizes)) == 0
        bwall = (time.perf_counter() - t0) / reps
        dev.kernel_timing(True)
        for _ in range(reps):
            assert hip.BNNX_ExecuteBatch(dev.handle, jobs, len(sizes)) == 0
        dms, dn = dev.kernel_timing_read(1)
        pms, pn = dev.kernel_timing_read(0)
        dev.kernel_timing(False)
        unit = n_total * k // 8 + n_total * (k // 128) * 2 + len(sizes) * 4 * k + 4 * n_total  # 19 chunks
        out["GEMV_F32 2048->151669 (19 chunks, one batch)"] = {
            "bytes_per_call": unit, "us_per_call": round(bwall * 1e6, 2), "GBps": round(unit / bwall / 1e9, 1),
            "dot_kernel_us": round(dms / dn * 1e3, 2), "prep_kernel_us": round(pms / pn * 1e3, 2),
            "dot_kernel_GBps": round(unit / (dms / dn / 1e3) / 1e9, 1)}
        for m in mats:
            m.destroy()
        bi.free()
        bo.free()
    return out


def gemm_leg(pkg, hip):
    """Config 4: multi-row GEMM_F32 / GEMM_I8 on the matrix cores."""
    out, best = {}, 0.0
    with pkg.Device(hip, 0) as dev:
        for op in ("GEMM_F32", "GEMM"):
            for k, n in ((2048, 6144), (6144, 2048)):
                bits, scales = pkg.synth.matrix(n, k, seed=4)
                m = dev.matrix(bits, scales)
                for rows in (8, 32, 64, 256, 1024):
                    f32 = op.endswith("F32")
                    x = pkg.synth.normal_f32(rows, k, seed=4) if f32 else pkg.synth.int8_uniform(rows, k, seed=4)
                    in_t, out_t = pkg.api.OP_TYPES[pkg.Op[op]]
                    bi, bo = dev.buffer(x.nbytes), dev.buffer(rows * n * 4)
                    bi.write(x)
                    job = pkg.Job(int(pkg.Op[op]), m.handle.value, bi.view(in_t), bo.view(out_t), rows)
                    _timed_calls(dev, job, 3)
                    wall, kern, prep = _timed_calls(dev, job, 20)
                    ops = 2.0 * rows * n * k
                    tops = ops / kern / 1e12
                    best = max(best, tops)
                    out[f"{op} {k}->{n} rows={rows}"] = {"kernel_us": round(kern * 1e6, 1), "TOPS": round(tops, 1),
                                                         "mfma_util": round(tops / 5000.0, 4),
                                                         "call_us": round(wall * 1e6, 1), "prep_us": round(prep * 1e6, 1)}
                    bi.free()
                    bo.free()
                m.destroy()
    return {"peak_TOPS": 5000.0, "best_TOPS": round(best, 1), "cases": out}


# device_greedy: the device path with the greedy loop on the device (BNNEX_DecodeGreedy,
# one host wait for all the steps); the others return logits to the host every step
E2E_PATHS = {"device": 1, "device_greedy": 1, "prepared": 2, "host": 0}


def e2e_leg(pkg, hip, paths=tuple(E2E_PATHS), new=128):
    """Config 5: Qwen3-1.7B-shape greedy decode through the engine (BNNE_* API)."""
    import tempfile
    fixture_path = ROOT / "tests" / "golden" / "e2e_qwen3_1p7b.json"
    fixture = json.loads(fixture_path.read_text()) if fixture_path.exists() else None
    eng = pkg.engine.EngineLib()
    res = {}
    with tempfile.TemporaryDirectory() as d:
        path = Path(d) / "qwen3.gguf"
        t0 = time.perf_counter()
        info = pkg.gguf.qwen3_random(path)
        prompt = pkg.gguf.prompt_ids(32, info["vocab"], seed=5)
        gen_s = time.perf_counter() - t0
        with pkg.Device(hip, 0) as dev:
            t0 = time.perf_counter()
            model = pkg.engine.Model(eng, dev, path)
            load_s = time.perf_counter() - t0
            for name in paths:
                mode = E2E_PATHS[name]
                ctx = pkg.engine.Context(model, n_ctx=1024)
                ctx.set_resident(mode)
                assert ctx.resident() == mode, f"{name} path not available"
                logits = np.empty(info["vocab"], np.float32)  # one buffer for every step, as bnn-infer-v2.c
                t0 = time.perf_counter()
                tokens = [int(np.argmax(ctx.decode(prompt, out=logits)))]
                t1 = time.perf_counter()
                ctx.reset_stats()
                if name == "device_greedy":
                    tokens += ctx.decode_greedy(tokens[-1], new - 1)
                else:
                    for _ in range(new - 1):
                        tokens.append(int(np.argmax(ctx.decode([tokens[-1]], out=logits))))
                t2 = time.perf_counter()
                st = ctx.stats()
                ctx.free()
                steps = new - 1
                entry = {"prefill_tok_s": round(32 / (t1 - t0), 1), "decode_tok_s": round(steps / (t2 - t1), 1),
                         "ms_per_token": round((t2 - t1) / steps * 1e3, 3),
                         "backend_share": round((st["transfer_ns"] + st["execute_ns"]) / max(st["total_ns"], 1), 4),
                         "weight_GBps": round(info["weight_bytes"] * steps / (t2 - t1) / 1e9, 1)}
                if fixture:
                    want = [row[1] for row in fixture["steps"]][:new]
                    same = sum(a == b for a, b in zip(tokens, want))
                    entry["token_agreement"] = f"{same}/{len(want)}"
                res[name] = entry
            model.free()
    out = {"model": "random-init Qwen3-1.7B shape (28 layers, 2048, 16/8 heads, FFN 6144, vocab 151669), Q1_0",
           "tokens": f"32 prompt + {new} greedy", "gguf_write_s": round(gen_s, 1), "load_s": round(load_s, 1),
           "weight_bytes_per_token": info["weight_bytes"], "paths": res}
    if fixture and fixture.get("soft_seconds"):
        # the fixture run: 32 prompt steps + 127 decode steps on one host core of the build container
        out["reference_soft_1core_tok_s"] = round((len(fixture["prompt"]) + fixture["steps_arg"]) /
                                                  fixture["soft_seconds"], 4)
    return out


def mlp_leg(pkg, hip):
    """Config 1: bnn-mlp classifier through the engine, 1000 samples in classify calls of
    64.  The default is the engine's device path: a call's rows are copied to the device
    once, each block runs there as one prepared batch of GEMM_F32 jobs (every row of it is
    that sample's GEMV_F32) plus the post-operation kernel, and only the logits come back.
    `host_rows` is the host call pattern with the same GEMM_F32 jobs (per block a write,
    a synchronous BNN_Execute and a read, the post-operation on the host); `per_sample` is
    the reference engine's call pattern (bnn-mlp.c:173-198: one GEMV_F32 per sample and
    block), through contexts of one sample per call (so it also carries one ctypes
    classify call per sample).  Each path runs the 1000 samples twice in one context and
    times the second pass (the device path builds a chunk size's batches on its first
    call of that size)."""
    import tempfile
    eng = pkg.engine.EngineLib()
    fixture_path = ROOT / "tests" / "golden" / "e2e_bnn_mlp.json"
    want = json.loads(fixture_path.read_text())["argmax"] if fixture_path.exists() else None

    def run(model, x, batch, path):
        ctx = pkg.engine.Context(model, n_batch=batch)
        ctx.set_resident(path)
        for s0 in range(0, len(x), batch):  # warm-up pass: every chunk size's batches built
            ctx.classify(x[s0:s0 + batch])
        st0 = ctx.stats()
        t0 = time.perf_counter()
        preds = []
        for s0 in range(0, len(x), batch):
            preds.extend(ctx.classify(x[s0:s0 + batch]).argmax(axis=1).tolist())
        dt = time.perf_counter() - t0
        st = {k: v - st0[k] for k, v in ctx.stats().items()}  # the timed pass only
        ctx.free()
        agree = f"{sum(a == b for a, b in zip(preds, want))}/{len(want)}" if want else None
        return {"path": "device" if path else "host",
                "samples_per_s": round(len(x) / dt, 1), "us_per_sample": round(dt / len(x) * 1e6, 1),
                "device_calls_per_sample": round(st["device_calls"] / len(x), 4),
                "backend_share": round((st["transfer_ns"] + st["execute_ns"]) / st["total_ns"], 4),
                "argmax_agreement": agree}

    with tempfile.TemporaryDirectory() as d:
        path = Path(d) / "mlp.gguf"
        pkg.gguf.bnn_mlp_random(path)
        x = pkg.gguf.bnn_mlp_inputs(1000)
        with pkg.Device(hip, 0) as dev:
            model = pkg.engine.Model(eng, dev, path)
            out = run(model, x, 64, 2)
            out["host_rows"] = run(model, x, 64, 0)
            out["per_sample"] = run(model, x, 1, 0)
            model.free()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--prewarm", type=float, default=0.5,
                    help="seconds of back-to-back steps before the declared warmup (GPU clock ramp)")
    ap.add_argument("--timed-events", action="store_true",
                    help="also record HIP events in the timed steps (kernel durations from them)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-extra", action="store_true", help="skip the secondary legs (ops, gemm, e2e, mlp)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run one 256 MiB device-to-device copy (counter calibration)")
    ap.add_argument("--only", choices=("ops", "gemm", "e2e", "mlp"),
                    help="run one secondary leg alone and print its JSON (for profiling)")
    ap.add_argument("--e2e-paths", default=",".join(E2E_PATHS),
                    help="decode paths of the e2e leg (comma list of device, prepared, host)")
    ap.add_argument("--e2e-new", type=int, default=128, help="greedy tokens per path in the e2e leg (2..128)")
    args = ap.parse_args()
    if args.copy_calibration:
        copy_calibration()
        return
    if args.gpus != 1:
        print("bench.py: this build runs on exactly one GPU. The BNN_* path has no multi-GPU form here: "
              "it would shard on output features (each matrix chunk on its own GPU, the input row "
              "broadcast and the outputs gathered, no floating-point reduction across GPUs).",
              file=sys.stderr)
        sys.exit(2)

    pkg = load_pkg()
    hip = pkg.load_hip()
    if args.only:
        e2e_paths = tuple(p for p in args.e2e_paths.split(",") if p)
        if not e2e_paths or any(p not in E2E_PATHS for p in e2e_paths) or not 2 <= args.e2e_new <= 128:
            ap.error("--e2e-paths takes " + ", ".join(E2E_PATHS) + "; --e2e-new 2..128")
        legs = {"ops": ops_leg, "gemm": gemm_leg, "mlp": mlp_leg,
                "e2e": lambda pkg, hip: e2e_leg(pkg, hip, e2e_paths, args.e2e_new)}
        print(json.dumps({args.only: legs[args.only](pkg, hip)}), flush=True)
        return
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

    # ---- timed region: the step as a prepared batch, launched back to back ----
    # BNNX_BatchCreate checks the 608 jobs once; every step is then one
    # BNNX_BatchLaunch (one prep launch + one group-dot launch, no host wait), and
    # BNNX_DeviceSynchronize closes the timed region (it also reports any input error).
    import ctypes
    batch = ctypes.c_void_p()
    st = hip.BNNX_BatchCreate(dev.handle, jobs, MATRICES, ctypes.byref(batch))
    if st != 0:
        raise pkg.BnnError(st, "BNNX_BatchCreate")

    def launch():
        st = hip.BNNX_BatchLaunch(batch)
        if st != 0:
            raise pkg.BnnError(st, "BNNX_BatchLaunch")

    def synchronize():
        st = hip.BNNX_DeviceSynchronize(dev.handle)
        if st != 0:
            raise pkg.BnnError(st, "BNNX_DeviceSynchronize")

    # Pre-warm: the GPU leaves its idle clocks only after some milliseconds of work, so
    # steps are launched back to back (in bursts closed by a synchronisation) until
    # PREWARM_S seconds have passed; then the declared warmup steps, one
    # synchronisation, and the timed steps.
    t0, prewarm_steps = time.perf_counter(), 0
    while time.perf_counter() - t0 < args.prewarm:
        for _ in range(64):
            launch()
        synchronize()
        prewarm_steps += 64
    for _ in range(args.warmup):
        launch()
    synchronize()
    # Kernel pass: the same K steps with HIP events on every kernel launch of the device
    # stream (the dispatches' own start and end timestamps, recorded through
    # hipExtLaunchKernel by the library and resolved at the synchronisation).  Timing
    # every dispatch slows a step by ~5% (config.event_overhead), so the timed steps
    # that follow run without events; --timed-events puts them in the timed steps.
    dev.kernel_timing(True)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        launch()
    synchronize()
    event_wall = time.perf_counter() - t0
    dot_ms, dot_n = dev.kernel_timing_read(1)
    prep_ms, prep_n = dev.kernel_timing_read(0)
    dev.kernel_timing(bool(args.timed_events))
    t0 = time.perf_counter()
    for _ in range(args.steps):
        launch()
    synchronize()
    wall = time.perf_counter() - t0
    if args.timed_events:
        dot_ms, dot_n = dev.kernel_timing_read(1)
        prep_ms, prep_n = dev.kernel_timing_read(0)
        dev.kernel_timing(False)
    print(f"timed: {args.steps} steps in {wall:.4f} s after {prewarm_steps} pre-warm steps "
          f"(kernel pass with events: {event_wall:.4f} s)", flush=True)
    y_stream = bout.read().view(np.float32).reshape(MATRICES, N_OUT)
    assert np.array_equal(y_stream.view(np.uint32), y_batch.view(np.uint32)), "streamed steps differ"

    hip.BNNX_BatchDestroy(batch)

    # the same step through the synchronous BNNX_ExecuteBatch (returns with results readable)
    sync_steps = max(1, args.steps // 4)
    t0 = time.perf_counter()
    for _ in range(sync_steps):
        step()
    sync_wall = time.perf_counter() - t0

    step_bytes = MATRICES * BYTES_PER_JOB
    value = step_bytes * args.steps / wall / 1e9
    dot_avg_s = dot_ms / 1e3 / max(dot_n, 1)
    achieved = step_bytes / dot_avg_s / 1e9

    # ---- per-call path through BNN_Execute (one job per call), same matrices ----
    per_call_jobs = min(MATRICES, 200)
    t0 = time.perf_counter()
    for i in range(per_call_jobs):
        st = dev.execute(jobs[i])
        if st != 0:
            raise pkg.BnnError(st, "BNN_Execute")
    call_wall = time.perf_counter() - t0
    dev.kernel_timing(True)  # kernel durations in a second pass (events slow each dispatch)
    for i in range(per_call_jobs):
        st = dev.execute(jobs[i])
        if st != 0:
            raise pkg.BnnError(st, "BNN_Execute")
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
            "step": "one prepared batch launch (BNNX_BatchLaunch: prep + group-dot), back to back, "
                    "one BNNX_DeviceSynchronize at the end",
            "prewarm_s": args.prewarm,
            "timed_events": bool(args.timed_events),
            "kernel_pass": "the same K steps right before the timed ones, HIP events on every dispatch",
            "event_overhead": round(event_wall / wall - 1.0, 4),
            "kernel_pass_GBps": round(step_bytes * args.steps / event_wall / 1e9, 2),
            "sync_GBps": round(step_bytes * sync_steps / sync_wall / 1e9, 2),
            "sync_ms_per_step": round(sync_wall / sync_steps * 1e3, 4),
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
            "kernel_launches_timed": dot_n,
            "prep_kernel_avg_us": round(prep_ms / max(prep_n, 1) * 1e3, 2),
            "step_frac": round(value / HBM_PEAK_GBS, 4),
        },
        "per_call": per_call,
    }
    if not args.no_extra:
        for leg_name, leg in (("ops", ops_leg), ("gemm", gemm_leg), ("e2e", e2e_leg), ("mlp", mlp_leg)):
            t0 = time.perf_counter()
            result[leg_name] = leg(pkg, hip)
            print(f"leg {leg_name}: {time.perf_counter() - t0:.1f} s", flush=True)
    result["cpu_baseline"] = None if args.no_cpu else cpu_baseline(pkg)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
