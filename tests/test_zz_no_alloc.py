"""BNNX_ExecuteNoAlloc: BNN_Execute's results without any allocation, its scratch in
one fixed device array per GPU.  Each case runs two calls in a row, the second on a
smaller input, and compares both with BNN_Execute bit for bit."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _views(pkg, dev, op, k, n, rows, shift_in, shift_out, stride_pad):
    in_t, out_t = pkg.api.OP_TYPES[pkg.Op[op]]
    isz = 4 if in_t == pkg.Type.F32 else 1
    osz = 2 if op == "DOT_GROUPS" else 4
    orow = n * (k // 128) * osz if op == "DOT_GROUPS" else n * osz
    istride, ostride = k * isz + stride_pad, orow + stride_pad
    bi = dev.buffer(shift_in + rows * istride + 64)
    bo = dev.buffer(shift_out + rows * ostride + 64)
    return in_t, out_t, isz, orow, istride, ostride, bi, bo


def _inputs(pkg, op, rows, k, seed):
    if op.endswith("F32"):
        x = pkg.synth.normal_f32(rows, k, seed=seed)
        x[0, seed % k] *= 20.0
        return x
    return pkg.synth.int8_uniform(rows, k, seed=seed)


def _run(pkg, dev, fn, op, m, k, n, rows, x, shift_in, shift_out, stride_pad):
    in_t, out_t, isz, orow, istride, ostride, bi, bo = _views(pkg, dev, op, k, n, rows, shift_in, shift_out,
                                                              stride_pad)
    try:
        raw = np.zeros(bi.nbytes, np.uint8)
        xb = x.view(np.uint8).reshape(rows, -1)
        for r in range(rows):
            raw[shift_in + r * istride:shift_in + r * istride + xb.shape[1]] = xb[r]
        bi.write(raw)
        bo.write(np.full(bo.nbytes, 0xA5, np.uint8))
        job = pkg.Job(int(pkg.Op[op]), m.handle.value, bi.view(in_t, shift_in, istride if stride_pad else 0),
                      bo.view(out_t, shift_out, ostride if stride_pad else 0), rows)
        st = fn(dev.handle, ctypes.byref(job))
        return st, bo.read()  # the whole buffer: padding must stay untouched too
    finally:
        bi.free()
        bo.free()


CASES = [
    # op, K, N, rows (first call), rows (second call), shift_in, shift_out, stride pad
    ("GEMV_F32", 2048, 6144, 1, 1, 0, 0, 0),
    ("DOT_GROUPS", 2048, 6144, 1, 1, 0, 0, 0),
    ("GEMV_F32", 8192, 700, 1, 1, 0, 0, 0),            # K > fused width: one row through the scratch
    ("GEMM_F32", 2048, 6144, 64, 17, 0, 0, 0),
    ("GEMM", 6144, 2048, 256, 9, 0, 0, 0),
    ("DOT_GROUPS", 1024, 1000, 40, 3, 0, 0, 0),
    ("GEMM_F32", 8192, 512, 1500, 700, 0, 0, 0),       # 2 chunks of the 8 MiB array, then 1
    ("GEMM_F32", 384, 70, 5, 2, 3, 6, 12),             # unaligned input and output: staging rows
    ("DOT_GROUPS", 8192, 8192, 9, 2, 1, 1, 2),          # 1 MiB staged output per row: chunks of 7
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}_{c[1]}x{c[2]}_r{c[3]}" for c in CASES])
def test_no_alloc_equals_execute(pkg, hip, case):
    op, k, n, rows1, rows2, si, so, pad = case
    fn = hip.lib.BNNX_ExecuteNoAlloc
    with pkg.Device(hip, 0) as dev:
        m = dev.matrix(*pkg.synth.matrix(n, k, seed=k + n))
        try:
            for call, rows in enumerate((rows1, rows2)):
                x = _inputs(pkg, op, rows, k, seed=31 * call + rows)
                st_ref, want = _run(pkg, dev, hip.BNN_Execute, op, m, k, n, rows, x, si, so, pad)
                st, got = _run(pkg, dev, fn, op, m, k, n, rows, x, si, so, pad)
                assert st_ref == pkg.Status.OK and st == pkg.Status.OK, (call, st_ref, st)
                assert got.tobytes() == want.tobytes(), (op, k, n, rows, call)
        finally:
            m.destroy()


def test_no_alloc_errors_and_device_memory(pkg, hip):
    """Statuses as BNN_Execute (argument errors, an illegal value with the output left
    untouched), and no device memory taken by the calls."""
    rt = ctypes.CDLL("libamdhip64.so")
    fn = hip.lib.BNNX_ExecuteNoAlloc
    k, n, rows = 2048, 1024, 300
    with pkg.Device(hip, 0) as dev:
        m = dev.matrix(*pkg.synth.matrix(n, k, seed=5))
        x = pkg.synth.normal_f32(rows, k, seed=5)
        bi, bo = dev.buffer(x.nbytes), dev.buffer(4 * n * rows)
        try:
            bi.write(x)
            job = pkg.Job(int(pkg.Op.GEMM_F32), m.handle.value, bi.view(pkg.Type.F32), bo.view(pkg.Type.F32), rows)
            assert fn(None, ctypes.byref(job)) == pkg.Status.EINVAL
            assert fn(dev.handle, None) == pkg.Status.EINVAL
            bad_op = pkg.Job(99, m.handle.value, bi.view(pkg.Type.F32), bo.view(pkg.Type.F32), rows)
            assert fn(dev.handle, ctypes.byref(bad_op)) == pkg.Status.ENOTSUP
            too_far = pkg.Job(int(pkg.Op.GEMM_F32), m.handle.value, bi.view(pkg.Type.F32, 4), bo.view(pkg.Type.F32),
                              rows)
            assert fn(dev.handle, ctypes.byref(too_far)) == pkg.Status.ERANGE
            free0, total = ctypes.c_size_t(), ctypes.c_size_t()
            assert fn(dev.handle, ctypes.byref(job)) == pkg.Status.OK  # first use after open
            assert rt.hipMemGetInfo(ctypes.byref(free0), ctypes.byref(total)) == 0
            for _ in range(3):
                assert fn(dev.handle, ctypes.byref(job)) == pkg.Status.OK
            free1 = ctypes.c_size_t()
            assert rt.hipMemGetInfo(ctypes.byref(free1), ctypes.byref(total)) == 0
            assert free1.value == free0.value
            good = bo.read()
            bad = x.copy()
            bad[rows - 1, k - 1] = np.nan  # the last value of the last row: checked before any chunk writes
            bi.write(bad)
            assert fn(dev.handle, ctypes.byref(job)) == pkg.Status.ERANGE
            assert bo.read().tobytes() == good.tobytes()
            bi.write(x)
            assert fn(dev.handle, ctypes.byref(job)) == pkg.Status.OK
            assert bo.read().tobytes() == good.tobytes()
        finally:
            bi.free()
            bo.free()
            m.destroy()


def test_no_alloc_two_handles_two_threads(pkg, hip):
    """Devices are independent (bnn-accelerator.h:166-168) although every handle on a GPU
    shares that GPU's one scratch array: two threads, each with its own handle on GPU 0,
    run multi-row NoAlloc jobs (which stage their quantised rows in the array) at the
    same time; every result equals BNN_Execute's."""
    import threading
    fn = hip.lib.BNNX_ExecuteNoAlloc
    specs = [("GEMM_F32", 2048, 2048, 700, 1), ("GEMM", 6144, 1024, 400, 2)]  # rows staged in the array
    results = {}

    def worker(t, op, k, n, rows, seed):
        try:
            with pkg.Device(hip, 0) as dev:
                m = dev.matrix(*pkg.synth.matrix(n, k, seed=seed))
                try:
                    xs = [_inputs(pkg, op, rows, k, seed=seed * 10 + i) for i in range(2)]
                    want = [_run(pkg, dev, hip.BNN_Execute, op, m, k, n, rows, x, 0, 0, 0) for x in xs]
                    barrier.wait(timeout=60)
                    for it in range(6):
                        i = it % 2
                        st, got = _run(pkg, dev, fn, op, m, k, n, rows, xs[i], 0, 0, 0)
                        assert want[i][0] == pkg.Status.OK and st == pkg.Status.OK, (t, it, st)
                        assert got.tobytes() == want[i][1].tobytes(), (t, it, op)
                finally:
                    m.destroy()
            results[t] = "ok"
        except BaseException as e:  # reported by the main thread
            results[t] = e

    barrier = threading.Barrier(len(specs))
    threads = [threading.Thread(target=worker, args=(t, *spec)) for t, spec in enumerate(specs)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=300)
    assert not any(th.is_alive() for th in threads), "a NoAlloc thread did not finish"
    for t in range(len(specs)):
        if results.get(t) != "ok":
            raise AssertionError(f"thread {t}: {results.get(t)!r}")
