"""BNNX_ExecuteBatch (HIP-backend extension): every job's output equals the CPU
oracle's (bit for bit), all-or-nothing input checks, concurrency rules, and
table-cache invalidation."""
from __future__ import annotations

import numpy as np
import pytest

from bnn_cases import fast_oracle, first_mismatch

pytestmark = pytest.mark.gpu


def _mk_batch(pkg, dev, specs, seed=0):
    """specs: [(op, K, N, rows)] -> matrices, one input and one output buffer, jobs."""
    mats, xs, in_off, out_off, layouts = [], [], [], [], []
    ioff = ooff = 0
    for i, (op, k, n, rows) in enumerate(specs):
        host = pkg.synth.matrix(n, k, seed=seed * 100 + i)
        mats.append(dev.matrix(*host))
        mats[-1].host = host  # the oracle's copy
        f32 = op.endswith("F32")
        x = pkg.synth.normal_f32(rows, k, seed=seed + i) if f32 else pkg.synth.int8_uniform(rows, k, seed=seed + i)
        xs.append(x)
        in_off.append(ioff)
        ioff += -(-x.nbytes // 64) * 64
        shape, dtype = ((rows, n, k // 128), np.int16) if op == "DOT_GROUPS" else ((rows, n), np.float32)
        layouts.append((shape, dtype))
        out_off.append(ooff)
        ooff += -(-int(np.prod(shape)) * np.dtype(dtype).itemsize // 64) * 64
    ioff += 64  # slack so that views can be shifted inside the buffers
    ooff += 64
    bi, bo = dev.buffer(ioff), dev.buffer(ooff)
    raw = np.zeros(ioff, np.uint8)
    for x, o in zip(xs, in_off):
        raw[o:o + x.nbytes] = x.view(np.uint8).reshape(-1)
    bi.write(raw)
    jobs = (pkg.Job * len(specs))()
    for i, (op, k, n, rows) in enumerate(specs):
        in_t, out_t = pkg.api.OP_TYPES[pkg.Op[op]]
        jobs[i] = pkg.Job(int(pkg.Op[op]), mats[i].handle.value, bi.view(in_t, in_off[i]), bo.view(out_t, out_off[i]),
                          rows)
    return mats, xs, bi, bo, jobs, out_off, layouts


def _oracle(pkg, oracle_fast, specs, mats, xs):
    """Every job's expected output from the CPU oracle (never from another HIP path)."""
    return [fast_oracle(pkg, oracle_fast, op, *mats[i].host, xs[i]) for i, (op, k, n, rows) in enumerate(specs)]


def _outputs(bo, out_off, layouts):
    raw = bo.read()
    res = []
    for o, (shape, dtype) in zip(out_off, layouts):
        nb = int(np.prod(shape)) * np.dtype(dtype).itemsize
        res.append(raw[o:o + nb].view(dtype).reshape(shape))
    return res


def _free(mats, bi, bo):
    bi.free()
    bo.free()
    for m in mats:
        m.destroy()


@pytest.mark.parametrize("specs", [
    [("GEMV_F32", 2048, 6144, 1)] * 12,                                   # uniform
    [("GEMV_F32", 2048, 2048, 1), ("GEMV", 6144, 2048, 1), ("DOT_GROUPS", 384, 70, 3),
     ("GEMM_F32", 8192, 129, 5), ("GEMM", 128, 1, 2), ("GEMV_F32", 2048, 8192, 1)],  # mixed
    [("GEMV_F32", 2048, 2048, 1), ("GEMV", 1024, 100, 1), ("DOT_GROUPS", 384, 70, 3),
     ("GEMM_F32", 2048, 129, 5), ("GEMM", 128, 1, 2), ("DOT_GROUPS", 2048, 64, 2)],  # mixed, K <= 2048
    [("GEMV_F32", 6144, 2048, 1)] * 32,                                   # long K: one wave per tile, 6 blocks
    [("GEMV_F32", 6144, 2048, 1)] * 16 + [("GEMV", 2176, 4100, 1)] * 8 + [("DOT_GROUPS", 8192, 640, 1)] * 4
    + [("GEMV_F32", 3072, 1000, 1)] * 8,                                  # long K, table-mapped: 17..64 groups
], ids=["uniform", "mixed", "mixed_small", "long_k", "long_k_mixed"])
def test_batch_equals_oracle(pkg, hipdev, oracle_fast, specs):
    mats, xs, bi, bo, jobs, out_off, layouts = _mk_batch(pkg, hipdev, specs)
    assert hipdev.api.BNNX_ExecuteBatch(hipdev.handle, jobs, len(specs)) == pkg.Status.OK
    got = _outputs(bo, out_off, layouts)
    wants = _oracle(pkg, oracle_fast, specs, mats, xs)
    for i, (op, k, n, rows) in enumerate(specs):
        want = wants[i]
        assert np.array_equal(got[i].view(np.uint8), want.view(np.uint8)), (i, op, first_mismatch(got[i], want))
    # a second, cached call on new input data
    xs2 = [(-x if x.dtype == np.float32 else np.negative(x)) for x in xs]
    raw = bi.read()
    for x, o in zip(xs2, [j.input.offset for j in jobs]):
        raw[o:o + x.nbytes] = x.view(np.uint8).reshape(-1)
    bi.write(raw)
    assert hipdev.api.BNNX_ExecuteBatch(hipdev.handle, jobs, len(specs)) == pkg.Status.OK
    got = _outputs(bo, out_off, layouts)
    wants = _oracle(pkg, oracle_fast, specs, mats, xs2)
    for i, (op, k, n, rows) in enumerate(specs):
        assert np.array_equal(got[i].view(np.uint8), wants[i].view(np.uint8)), (i, op)
    _free(mats, bi, bo)


def test_batch_cache_follows_resource_changes(pkg, hipdev, oracle_fast):
    specs = [("GEMV_F32", 256, 100, 1)] * 3
    mats, xs, bi, bo, jobs, out_off, layouts = _mk_batch(pkg, hipdev, specs, seed=5)
    assert hipdev.api.BNNX_ExecuteBatch(hipdev.handle, jobs, 3) == pkg.Status.OK
    # replace matrix 1 by a different one; the job array may even hold the same handle value
    mats[1].destroy()
    host = pkg.synth.matrix(100, 256, seed=999)
    mats[1] = hipdev.matrix(*host)
    jobs[1].matrix = mats[1].handle.value
    assert hipdev.api.BNNX_ExecuteBatch(hipdev.handle, jobs, 3) == pkg.Status.OK
    got = _outputs(bo, out_off, layouts)
    want = fast_oracle(pkg, oracle_fast, "GEMV_F32", *host, xs[1])
    assert np.array_equal(got[1].view(np.uint32), want.view(np.uint32))
    _free(mats, bi, bo)


def test_batch_illegal_input_writes_nothing(pkg, hipdev):
    specs = [("GEMV_F32", 512, 64, 1), ("DOT_GROUPS", 256, 10, 2), ("GEMM", 128, 7, 3)]
    mats, xs, bi, bo, jobs, out_off, layouts = _mk_batch(pkg, hipdev, specs, seed=2)
    raw = bi.read()
    raw[jobs[2].input.offset + 2 * 128 + 5] = 0x80  # -128 in the last row of the last job
    bi.write(raw)
    sentinel = np.full(bo.nbytes, 0x5A, np.uint8)
    bo.write(sentinel)
    assert hipdev.api.BNNX_ExecuteBatch(hipdev.handle, jobs, 3) == pkg.Status.ERANGE
    assert np.array_equal(bo.read(), sentinel)
    raw[jobs[2].input.offset + 2 * 128 + 5] = 0x01
    bi.write(raw)
    assert hipdev.api.BNNX_ExecuteBatch(hipdev.handle, jobs, 3) == pkg.Status.OK
    _free(mats, bi, bo)


def test_batch_rejections(pkg, hipdev):
    specs = [("GEMV_F32", 256, 16, 1), ("GEMV_F32", 256, 16, 1)]
    mats, xs, bi, bo, jobs, out_off, layouts = _mk_batch(pkg, hipdev, specs, seed=3)
    api = hipdev.api
    assert api.BNNX_ExecuteBatch(hipdev.handle, jobs, 0) == pkg.Status.EINVAL
    assert api.BNNX_ExecuteBatch(None, jobs, 2) == pkg.Status.EINVAL
    bad = (pkg.Job * 2)(*jobs)
    bad[1].output.offset = jobs[0].output.offset + 4  # overlapping outputs
    assert api.BNNX_ExecuteBatch(hipdev.handle, bad, 2) == pkg.Status.EINVAL
    own_in = hipdev.buffer(bi.nbytes)
    own_in.write(bi.read())
    bad = (pkg.Job * 2)(*jobs)
    bad[1].input.buffer = own_in.handle.value
    bad[1].output.buffer = jobs[0].input.buffer  # job 1 would write what job 0 reads
    bad[1].output.offset = 0
    assert api.BNNX_ExecuteBatch(hipdev.handle, bad, 2) == pkg.Status.EINVAL
    bad[1].output.buffer = jobs[1].output.buffer  # same views, own input: accepted
    bad[1].output.offset = jobs[1].output.offset
    assert api.BNNX_ExecuteBatch(hipdev.handle, bad, 2) == pkg.Status.OK
    own_in.free()
    bad = (pkg.Job * 2)(*jobs)
    bad[1].output.offset += 2  # unaligned F32 output: single jobs only
    assert api.BNNX_ExecuteBatch(hipdev.handle, bad, 2) == pkg.Status.ENOTSUP
    bad = (pkg.Job * 2)(*jobs)
    bad[0].rows = 2  # the first failing job's own status (GEMV with rows != 1)
    bad[1].operation = 99
    assert api.BNNX_ExecuteBatch(hipdev.handle, bad, 2) == pkg.Status.EINVAL
    assert api.BNNX_ExecuteBatch(hipdev.handle, jobs, 2) == pkg.Status.OK
    _free(mats, bi, bo)


def test_prepared_batch_launches(pkg, hipdev, oracle_fast):
    """BNNX_BatchCreate/Launch/DeviceSynchronize: same results as single jobs, input
    errors reported at the synchronisation, batches invalidated by destroys."""
    api = hipdev.api
    specs = [("GEMV_F32", 2048, 1024, 1), ("GEMV", 1024, 100, 1), ("DOT_GROUPS", 384, 70, 3), ("GEMM_F32", 256, 129, 5)]
    mats, xs, bi, bo, jobs, out_off, layouts = _mk_batch(pkg, hipdev, specs, seed=7)
    import ctypes
    want = _oracle(pkg, oracle_fast, specs, mats, xs)
    b = ctypes.c_void_p()
    assert api.BNNX_BatchCreate(hipdev.handle, jobs, len(specs), ctypes.byref(b)) == pkg.Status.OK
    for rep in range(3):  # launched repeatedly without waiting in between
        assert api.BNNX_BatchLaunch(b) == pkg.Status.OK
    assert api.BNNX_DeviceSynchronize(hipdev.handle) == pkg.Status.OK
    got = _outputs(bo, out_off, layouts)
    for i, (op, k, n, rows) in enumerate(specs):
        assert np.array_equal(got[i].view(np.uint8), want[i].view(np.uint8)), (i, op)
    # an illegal F32 input: the device skips the batch, the synchronisation reports it
    raw = bi.read()
    raw[jobs[0].input.offset:jobs[0].input.offset + 4] = np.frombuffer(np.float32(np.nan).tobytes(), np.uint8)
    bi.write(raw)
    sentinel = np.full(bo.nbytes, 0x3C, np.uint8)
    bo.write(sentinel)
    assert api.BNNX_BatchLaunch(b) == pkg.Status.OK
    assert api.BNNX_DeviceSynchronize(hipdev.handle) == pkg.Status.ERANGE
    assert np.array_equal(bo.read(), sentinel)
    assert api.BNNX_DeviceSynchronize(hipdev.handle) == pkg.Status.OK  # reported once
    # device pointers of buffers are distinct and non-null
    p1, p2 = ctypes.c_void_p(), ctypes.c_void_p()
    assert api.BNNX_BufferDevicePointer(bi.handle, ctypes.byref(p1)) == pkg.Status.OK
    assert api.BNNX_BufferDevicePointer(bo.handle, ctypes.byref(p2)) == pkg.Status.OK
    assert p1.value and p2.value and p1.value != p2.value
    assert api.BNNX_BufferDevicePointer(None, ctypes.byref(p1)) == pkg.Status.EINVAL
    # any destroy invalidates prepared batches; a live batch keeps the device open
    assert api.BNNX_BatchCheck(b) == pkg.Status.OK
    extra = hipdev.buffer(64)
    extra.free()
    assert api.BNNX_BatchCheck(b) == pkg.Status.EINVAL
    assert api.BNNX_BatchLaunch(b) == pkg.Status.EINVAL
    api.BNNX_BatchDestroy(b)
    bad = (pkg.Job * 2)(*jobs[:2])
    bad[1].output.buffer = jobs[0].input.buffer
    bad[1].output.offset = 0
    assert api.BNNX_BatchCreate(hipdev.handle, bad, 2, ctypes.byref(b)) == pkg.Status.EINVAL
    assert not b.value
    _free(mats, bi, bo)


def test_async_status_is_separate_from_synchronous_calls(pkg, hipdev):
    """An illegal input met by a synchronous call after an asynchronous launch is that
    call's own BNN_ERANGE; the next BNNX_DeviceSynchronize reports only the launches
    (and the other way round: a failed launch is not hidden by a later good call)."""
    import ctypes
    api = hipdev.api
    specs = [("GEMV_F32", 2048, 1024, 1), ("GEMV_F32", 2048, 512, 1)]
    mats, xs, bi, bo, jobs, out_off, layouts = _mk_batch(pkg, hipdev, specs, seed=9)
    b = ctypes.c_void_p()
    assert api.BNNX_BatchCreate(hipdev.handle, jobs, 1, ctypes.byref(b)) == pkg.Status.OK
    bad = xs[1].copy()
    bad[0, 7] = np.nan
    raw = bi.read()
    o1 = jobs[1].input.offset
    raw[o1:o1 + bad.nbytes] = bad.view(np.uint8).reshape(-1)
    bi.write(raw)
    assert api.BNNX_BatchLaunch(b) == pkg.Status.OK             # job 0: legal
    assert hipdev.execute(jobs[1]) == pkg.Status.ERANGE         # synchronous, illegal
    assert api.BNNX_DeviceSynchronize(hipdev.handle) == pkg.Status.OK
    # the reverse order: a failed launch, then a good synchronous call
    raw[o1:o1 + xs[1].nbytes] = xs[1].view(np.uint8).reshape(-1)
    o0 = jobs[0].input.offset
    bad0 = xs[0].copy()
    bad0[0, 3] = np.inf
    raw[o0:o0 + bad0.nbytes] = bad0.view(np.uint8).reshape(-1)
    bi.write(raw)
    assert api.BNNX_BatchLaunch(b) == pkg.Status.OK
    assert hipdev.execute(jobs[1]) == pkg.Status.OK
    assert api.BNNX_DeviceSynchronize(hipdev.handle) == pkg.Status.ERANGE
    assert api.BNNX_DeviceSynchronize(hipdev.handle) == pkg.Status.OK
    api.BNNX_BatchDestroy(b)
    _free(mats, bi, bo)


def test_batches_drop_the_single_row_mirror(pkg, hipdev):
    """A single-row F32 BNN_Execute output is mirrored in host memory; a later
    BNNX_ExecuteBatch or prepared batch launch that rewrites the same range must make
    BNN_BufferRead return the new device contents."""
    import ctypes
    api = hipdev.api
    k, n = 2048, 700
    mats = [hipdev.matrix(*pkg.synth.matrix(n, k, seed=s)) for s in (21, 22, 23)]
    x = pkg.synth.normal_f32(1, k, seed=21)
    bi, bo = hipdev.buffer(x.nbytes), hipdev.buffer(4 * n)
    bi.write(x)
    want = [hipdev.run(pkg.Op.GEMV_F32, m, x)[0] for m in mats]
    jobs = [pkg.Job(int(pkg.Op.GEMV_F32), m.handle.value, bi.view(pkg.Type.F32), bo.view(pkg.Type.F32), 1)
            for m in mats]
    f = lambda raw: np.frombuffer(raw, np.float32).view(np.uint32)
    assert hipdev.execute(jobs[0]) == pkg.Status.OK
    assert np.array_equal(f(bo.read()), want[0].view(np.uint32))
    one = (pkg.Job * 1)(jobs[1])
    assert api.BNNX_ExecuteBatch(hipdev.handle, one, 1) == pkg.Status.OK
    assert np.array_equal(f(bo.read()), want[1].view(np.uint32))
    assert hipdev.execute(jobs[0]) == pkg.Status.OK
    assert np.array_equal(f(bo.read(40, 80)), want[0][20:30].view(np.uint32))
    b = ctypes.c_void_p()
    three = (pkg.Job * 1)(jobs[2])
    assert api.BNNX_BatchCreate(hipdev.handle, three, 1, ctypes.byref(b)) == pkg.Status.OK
    assert hipdev.execute(jobs[0]) == pkg.Status.OK                 # mirror valid again
    assert api.BNNX_BatchLaunch(b) == pkg.Status.OK
    assert api.BNNX_DeviceSynchronize(hipdev.handle) == pkg.Status.OK
    assert np.array_equal(f(bo.read()), want[2].view(np.uint32))
    api.BNNX_BatchDestroy(b)
    bi.free()
    bo.free()
    for m in mats:
        m.destroy()


def test_device_index_contract(pkg, hip):
    """BNN_DeviceOpen takes index 0 only (soft-bnn-accelerator.c:317-318); other GPUs
    are opened through BNNX_DeviceOpenOrdinal."""
    import ctypes
    h = ctypes.c_void_p(1234)
    assert hip.BNN_DeviceOpen(1, ctypes.byref(h)) == pkg.Status.ENOTSUP and h.value is None
    count = ctypes.c_int()
    assert ctypes.CDLL("libamdhip64.so").hipGetDeviceCount(ctypes.byref(count)) == 0 and count.value >= 1
    h = ctypes.c_void_p(1234)
    assert hip.lib.BNNX_DeviceOpenOrdinal(ctypes.c_uint32(count.value), ctypes.byref(h)) == pkg.Status.ENOTSUP
    assert h.value is None
    assert hip.lib.BNNX_DeviceOpenOrdinal(ctypes.c_uint32(0), ctypes.byref(h)) == pkg.Status.OK and h.value
    caps = pkg.Caps()
    assert hip.BNN_DeviceGetCaps(h, ctypes.byref(caps)) == pkg.Status.OK and caps.max_in_features == 8192
    assert hip.BNN_DeviceClose(h) == pkg.Status.OK


@pytest.mark.parametrize("specs", [
    [("GEMV_F32", 2048, 6144, 1)] * 45,                                   # uniform, 45 rows (not a multiple of 8)
    [("GEMV_F32", 2048, 6144, 1)] * 24 + [("GEMV", 1024, 8192, 1)] * 12 + [("DOT_GROUPS", 2048, 4096, 1)] * 6
    + [("GEMV_F32", 640, 1000, 1)] * 3,                                   # mixed one-row jobs, table-mapped
], ids=["uniform45", "mixed"])
def test_full_chip_one_row_batch(pkg, hipdev, oracle_fast, specs):
    """Batches of one-row jobs with K <= 2048 and a full chip of 64-feature items (the
    headline's form, on the one-wave-per-item kernel): the same results as single jobs,
    through BNNX_ExecuteBatch and through repeated prepared launches, and an illegal row
    writes nothing while the next launch works again."""
    import ctypes
    api = hipdev.api
    mats, xs, bi, bo, jobs, out_off, layouts = _mk_batch(pkg, hipdev, specs, seed=11)
    items = sum(-(-n // 64) for _, _, n, _ in specs)
    assert items >= 256 * 16  # enough items for the one-wave-per-item kernel
    want = _oracle(pkg, oracle_fast, specs, mats, xs)
    for rep in range(2):
        assert api.BNNX_ExecuteBatch(hipdev.handle, jobs, len(specs)) == pkg.Status.OK
        got = _outputs(bo, out_off, layouts)
        for i, (op, k, n, rows) in enumerate(specs):
            assert np.array_equal(got[i].view(np.uint8), want[i].view(np.uint8)), (rep, i, op, first_mismatch(got[i], want[i]))
    b = ctypes.c_void_p()
    assert api.BNNX_BatchCreate(hipdev.handle, jobs, len(specs), ctypes.byref(b)) == pkg.Status.OK
    bo.write(np.zeros(bo.nbytes, np.uint8))
    for rep in range(5):
        assert api.BNNX_BatchLaunch(b) == pkg.Status.OK
    assert api.BNNX_DeviceSynchronize(hipdev.handle) == pkg.Status.OK
    got = _outputs(bo, out_off, layouts)
    for i, (op, k, n, rows) in enumerate(specs):
        assert np.array_equal(got[i].view(np.uint8), want[i].view(np.uint8)), ("prepared", i, op)
    # one illegal value in the last job's row: no output of the launch is written
    raw = bi.read()
    o = jobs[len(specs) - 1].input.offset
    bad = np.frombuffer(np.float32(np.inf).tobytes(), np.uint8) if specs[-1][0].endswith("F32") else np.array([0x80], np.uint8)
    raw[o:o + bad.size] = bad
    bi.write(raw)
    sentinel = np.full(bo.nbytes, 0x5A, np.uint8)
    bo.write(sentinel)
    assert api.BNNX_BatchLaunch(b) == pkg.Status.OK
    assert api.BNNX_DeviceSynchronize(hipdev.handle) == pkg.Status.ERANGE
    assert np.array_equal(bo.read(), sentinel)
    assert api.BNNX_ExecuteBatch(hipdev.handle, jobs, len(specs)) == pkg.Status.ERANGE
    assert np.array_equal(bo.read(), sentinel)
    # the row made legal again: the next launches compute everything
    raw[o:o + bad.size] = np.frombuffer(xs[-1].view(np.uint8).reshape(-1)[:bad.size].tobytes(), np.uint8)
    bi.write(raw)
    assert api.BNNX_BatchLaunch(b) == pkg.Status.OK
    assert api.BNNX_DeviceSynchronize(hipdev.handle) == pkg.Status.OK
    got = _outputs(bo, out_off, layouts)
    for i, (op, k, n, rows) in enumerate(specs):
        assert np.array_equal(got[i].view(np.uint8), want[i].view(np.uint8)), ("after error", i, op)
    api.BNNX_BatchDestroy(b)
    _free(mats, bi, bo)
