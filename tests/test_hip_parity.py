"""GPU parity of the HIP backend against the reference's fixtures and the CPU oracle.

Every comparison is bit-exact (integer, I16 and F32 outputs alike): the kernels
keep the reference's sequential per-group FP32 accumulation, so no tolerance is
needed or allowed.
"""
from __future__ import annotations

import ctypes
import hashlib
import json
import subprocess

import numpy as np
import pytest

from bnn_cases import CASES, case_inputs, fast_oracle, first_mismatch, input_sha, run_chunks, sha
from conftest import GOLDEN, REF_DIR
from test_oracle import _quant_rows, _rtl, sum_order_case

pytestmark = pytest.mark.gpu
FIXTURES = json.loads((GOLDEN / "soft_fixtures.json").read_text())


def test_reference_contract_suite_on_hip(tmp_path):
    """The reference's own API test (tests/accelerator/test_bnn_accelerator.c), unchanged,
    linked against libbnn_hip.so: 453 jobs byte-compared with its independent scalar
    oracle, every error path, view layout, ownership, busy and isolation rule."""
    exe = REF_DIR / "test_ref_vs_hip"
    assert exe.exists(), "oracle/_ref/test_ref_vs_hip missing (built by __graft_entry__.build())"
    dump = tmp_path / "dump.bin"
    print(f"running {exe}", flush=True)
    r = subprocess.run([str(exe), str(dump)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    assert "453 successful jobs" in r.stdout
    want = json.loads((GOLDEN / "ref_suite.json").read_text())
    data = dump.read_bytes()
    assert len(data) == want["bytes"]
    assert hashlib.sha256(data).hexdigest() == want["sha256"]


def test_rtl_golden_case(pkg, hipdev):
    case, got = _rtl(pkg, hipdev)
    for name, out in got.items():
        assert np.array_equal(out.view(np.uint32), case[name]), (name, first_mismatch(out.view(np.uint32), case[name]))


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_benchmark_shapes_match_soft_fixtures(pkg, hipdev, oracle_fast, case):
    name, op, k, n, rows, seed = case
    print(f"case {name}", flush=True)
    rec = FIXTURES[name]
    chunks, x = case_inputs(pkg, op, k, n, rows, seed)
    assert input_sha(chunks, x) == rec["input_sha256"], "synthetic generator drifted"
    out = run_chunks(pkg, hipdev, op, chunks, x)
    if sha(out) != rec["output_sha256"]:
        want = np.concatenate([fast_oracle(pkg, oracle_fast, op, b, s, x) for b, s in chunks], axis=1)
        pytest.fail(f"{name}: {first_mismatch(out, want)}")
    small = np.load(GOLDEN / "soft_small.npz")
    if name in small.files:
        assert np.array_equal(out.view(np.uint8), small[name].view(np.uint8))


def test_every_finite_fp16_scale_converts_exactly(pkg, hipdev):
    """GEMV with D = 1 returns F32(scale) (test_bnn_accelerator.c:473-491), for all 63488
    finite binary16 patterns; -0 sums to +0."""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    h = h[(h & 0x7C00) != 0x7C00]
    x = np.zeros((1, 128), np.int8)
    x[0, 0] = 1
    got = []
    for off in range(0, h.size, 8192):
        hs = h[off:off + 8192]
        bits = np.zeros((hs.size, 16), np.uint8)
        bits[:, 0] = 1  # weight 0 is +1, the rest -1 but multiplied by zero activations
        m = hipdev.matrix(bits, hs.reshape(-1, 1))
        got.append(hipdev.run(pkg.Op.GEMV, m, x)[0])
        m.destroy()
    got = np.concatenate(got)
    want = h.view(np.float16).astype(np.float32) + np.float32(0.0)  # -0 -> +0 like 0 + (-0)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), first_mismatch(got, want)


def test_fp32_accumulation_order_and_no_fma(pkg, hipdev):
    bits, scales, q, want = sum_order_case()
    m = hipdev.matrix(bits, scales)
    z = hipdev.run(pkg.Op.GEMM, m, q)
    m.destroy()
    assert z[0, 0] == want[0]
    assert z[1, 1] == want[1]


@pytest.mark.parametrize("i", range(10))
def test_quantiser_edge_rows(pkg, hipdev, oracle, i):
    x = _quant_rows()[i]
    k = -(-x.size // 128) * 128
    xr = np.zeros((1, k), np.float32)
    xr[0, :x.size] = x
    bits, scales = pkg.synth.matrix(70, k, seed=i)
    got = run_chunks(pkg, hipdev, "GEMV_F32", [(bits, scales)], xr)
    with pkg.Device(oracle, 0) as dev:
        want = run_chunks(pkg, dev, "GEMV_F32", [(bits, scales)], xr)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), first_mismatch(got, want)


@pytest.mark.parametrize("op", ["GEMM", "GEMM_F32"])
@pytest.mark.parametrize("rows,k,n", [
    (1000, 384, 4100), (2049, 128, 2000),                      # 128 x 128 workgroup tiles, two per CU
    (400, 640, 6100),                                          # 128 x 128, one workgroup per CU
    (1000, 640, 2000),                                         # 64 x 128
    (250, 1152, 6100),                                         # 64 x 64
    (100, 640, 7000),                                          # 64 x 64, three quarters of a round
    (120, 640, 5000),                                          # 32 x 64
    (8, 2048, 6144), (13, 1152, 1000),                         # K split, operands by DMA: 16 x 32, <= 16 rows
    (17, 640, 1000), (50, 640, 1000), (24, 2048, 8100),        # the same, 32 x 32 in one round (5..16 groups)
    (30, 1152, 7000), (32, 1408, 2050), (120, 1152, 2040),
    (80, 1408, 3500), (150, 2048, 2000),                       # the same, 32 x 64 in one round (16 waves)
    (190, 1024, 2040),                                         # the same, 8 waves (<= 8 groups)
    (380, 2048, 2000), (100, 1152, 6100),                      # the same, 32 x 32 past one round
    (40, 2304, 1500),                                          # the same, 16 x 32, 17..32 groups
    (100, 3200, 2000), (180, 4096, 2040), (150, 3200, 2000),   # the same, 32 x 32, 17..32 groups
    (24, 6144, 2048), (56, 4608, 1000),                        # the same, 16 x 32, 33..48 groups
    (100, 4224, 2000), (110, 6144, 1900),                      # running sums over two K slices, 16 x 64
    (30, 8192, 2000), (9, 6400, 700),                          # the same, eight slices, 16 x 16 (50: empty slice)
    (20, 6272, 5000),                                          # a wave per 16 x 16 block, operands in registers
    (20, 6272, 7000), (40, 6272, 1500),                        # K split over 8 / 4 waves in registers: 32x32, 32x16
    (330, 4224, 2040), (300, 4480, 2000),                      # a wave per 32 x 32 block, long K
    (250, 6144, 2000), (300, 8192, 1000),                      # K split over 8 waves per 32 x 64 tile, long K
    (60, 4480, 6100),                                          # K split over 4 waves per 32 x 64 tile, 17..47 groups
    (380, 6144, 2000), (120, 6272, 6100),                      # the same, >= 48 groups, one to two rounds
    (1000, 2048, 6100), (777, 1152, 8000), (1152, 640, 8128),  # 128 x 192, operands per wave (9 groups: odd)
    (1000, 6272, 2000), (1024, 4096, 2048),                    # 64 x 128, operands per wave, long K
])
def test_gemm_tilings_ragged_edges(pkg, hipdev, oracle_fast, op, rows, k, n):
    """Shapes that select each multi-row tiling, with a partial last row tile, a last
    column tile that ends inside a 64-feature scale tile or past it, odd and even
    group counts, fewer groups than waves, and round counts that do not fill the
    prefetch ring."""
    print(f"case {op} rows={rows} k={k} n={n}", flush=True)
    bits, scales = pkg.synth.matrix(n, k, seed=rows + n)
    f32 = op.endswith("F32")
    x = pkg.synth.normal_f32(rows, k, seed=k) if f32 else pkg.synth.int8_uniform(rows, k, seed=k)
    got = run_chunks(pkg, hipdev, op, [(bits, scales)], x)
    want = fast_oracle(pkg, oracle_fast, op, bits, scales, x)
    assert np.array_equal(got.view(np.uint8), want.view(np.uint8)), first_mismatch(got, want)


@pytest.mark.parametrize("op", ["DOT_GROUPS", "GEMM", "GEMM_F32"])
def test_row_chunking_and_late_illegal_row(pkg, hipdev, oracle_fast, op):
    """More rows than one launch chunk: all rows are validated before any chunk writes."""
    rows, k, n = 5000, 256, 67
    bits, scales = pkg.synth.matrix(n, k, seed=21)
    f32 = op.endswith("F32")
    x = pkg.synth.normal_f32(rows, k, seed=21) if f32 else pkg.synth.int8_uniform(rows, k, seed=21)
    got = run_chunks(pkg, hipdev, op, [(bits, scales)], x)
    want = fast_oracle(pkg, oracle_fast, op, bits, scales, x)
    assert np.array_equal(got.view(np.uint8), want.view(np.uint8)), first_mismatch(got, want)

    # illegal value in the last row: ERANGE and the output buffer untouched
    bad = x.copy()
    bad[-1, 200] = np.nan if f32 else -128
    m = hipdev.matrix(bits, scales)
    in_t, out_t = pkg.api.OP_TYPES[pkg.Op[op]]
    bi, bo = hipdev.buffer(bad.nbytes), hipdev.buffer(got.nbytes)
    sentinel = np.full(got.nbytes, 0x5A, np.uint8)
    bi.write(bad)
    bo.write(sentinel)
    job = pkg.Job(int(pkg.Op[op]), m.handle.value, bi.view(in_t), bo.view(out_t), rows)
    assert hipdev.execute(job) == pkg.Status.ERANGE
    assert np.array_equal(bo.read(), sentinel)
    # recovery on the same buffers
    bi.write(x)
    assert hipdev.execute(job) == pkg.Status.OK
    assert np.array_equal(bo.read().view(got.dtype).reshape(got.shape).view(np.uint8), got.view(np.uint8))
    bi.free()
    bo.free()
    m.destroy()


@pytest.mark.parametrize("seed", range(4))
def test_odd_views_random(pkg, hipdev, oracle, seed):
    """Unaligned offsets and strides on both sides, padding never written."""
    rng = np.random.default_rng(seed)
    for op in ("DOT_GROUPS", "GEMM", "GEMM_F32", "GEMV", "GEMV_F32"):
        k = int(rng.integers(1, 9)) * 128
        n = int(rng.integers(1, 200))
        rows = 1 if op.startswith("GEMV") else int(rng.integers(1, 6))
        bits, scales = pkg.synth.matrix(n, k, seed=seed * 10 + 1)
        in_t, out_t = pkg.api.OP_TYPES[pkg.Op[op]]
        esz = 4 if in_t == pkg.Type.F32 else 1
        in_row = k * esz
        out_row = n * (k // 128) * 2 if op == "DOT_GROUPS" else n * 4
        in_off, out_off = int(rng.integers(0, 9)), int(rng.integers(0, 9))
        in_stride = in_row + int(rng.integers(0, 13))
        out_stride = out_row + int(rng.integers(0, 13))
        in_bytes = in_off + rows * in_stride + 5
        out_bytes = out_off + rows * out_stride + 7
        x = pkg.synth.normal_f32(rows, k, seed=seed) if esz == 4 else pkg.synth.int8_uniform(rows, k, seed=seed)
        raw = np.full(in_bytes, 0xFF if esz == 4 else 0x80, np.uint8)  # NaN / -128 padding is legal
        for r in range(rows):
            raw[in_off + r * in_stride: in_off + r * in_stride + in_row] = x[r].view(np.uint8)
        results = []
        with pkg.Device(oracle, 0) as odev:
            for dev in (hipdev, odev):
                m = dev.matrix(bits, scales)
                bi, bo = dev.buffer(in_bytes), dev.buffer(out_bytes)
                bi.write(raw)
                bo.write(np.full(out_bytes, 0xA5, np.uint8))
                job = pkg.Job(int(pkg.Op[op]), m.handle.value, bi.view(in_t, in_off, in_stride),
                              bo.view(out_t, out_off, out_stride), rows)
                assert dev.execute(job) == pkg.Status.OK
                results.append(bo.read())
                assert np.array_equal(bi.read(), raw)  # input untouched
                bi.free()
                bo.free()
                m.destroy()
        assert np.array_equal(results[0], results[1]), (op, k, n, rows, in_off, in_stride, out_off, out_stride)


def test_two_devices_are_isolated(pkg, hip):
    a, b = pkg.Device(hip, 0), pkg.Device(hip, 0)
    bits, scales = pkg.synth.matrix(10, 256, seed=3)
    ma, mb = a.matrix(bits, scales), b.matrix(bits, scales)
    bi = a.buffer(256)
    bo = b.buffer(40)
    job = pkg.Job(int(pkg.Op.GEMV), ma.handle.value, bi.view(pkg.Type.I8), bo.view(pkg.Type.F32), 1)
    assert a.execute(job) == pkg.Status.EINVAL  # output buffer of another device
    assert a.api.BNN_DeviceClose(a.handle) == pkg.Status.EBUSY
    bi.free()
    bo.free()
    ma.destroy()
    mb.destroy()
    a.close()
    b.close()


@pytest.mark.parametrize("op", ["GEMV_F32", "GEMV", "DOT_GROUPS"])
@pytest.mark.parametrize("k", [128, 1152, 6144, 6272, 8192])
def test_single_row_both_paths(pkg, hipdev, oracle, k, op):
    """BNN_Execute with one row: K <= 6144 runs as one fused launch, wider rows as prep +
    dot.  Both against the oracle on ragged tile counts, with outliers and a row of one
    non-zero value; an illegal input (Inf; -128 for int8 rows) is ERANGE with the output
    left untouched, and the next call succeeds."""
    rng = np.random.default_rng(k)
    f32 = op == "GEMV_F32"
    in_t, out_t = pkg.api.OP_TYPES[pkg.Op[op]]
    for n in (1, 65, 8192):
        print(f"{op} k={k} n={n}", flush=True)
        bits, scales = pkg.synth.matrix(n, k, seed=k + n)
        if f32:
            x = pkg.synth.normal_f32(3, k, seed=k)
            x[0, rng.integers(0, k, 8)] *= 20.0
            x[1] = 0.0
            x[1, k // 2] = -3.5
        else:
            x = pkg.synth.int8_uniform(3, k, seed=k)
            x[1] = 0
            x[1, k // 2] = -127
        out_bytes = n * (k // 128) * 2 if op == "DOT_GROUPS" else 4 * n
        with pkg.Device(oracle, 0) as odev:
            mh, mo = hipdev.matrix(bits, scales), odev.matrix(bits, scales)
            try:
                for r in range(3):
                    got = hipdev.run(pkg.Op[op], mh, x[r:r + 1])
                    want = odev.run(pkg.Op[op], mo, x[r:r + 1])
                    assert got.tobytes() == want.tobytes(), (op, k, n, r)
                bad = x[:1].copy()
                bad[0, k - 1] = np.inf if f32 else -128
                bi, bo = hipdev.buffer(bad.nbytes), hipdev.buffer(out_bytes)
                try:
                    bi.write(bad)
                    bo.write(np.full(out_bytes, 0x5A, np.uint8))
                    job = pkg.Job(int(pkg.Op[op]), mh.handle.value, bi.view(in_t), bo.view(out_t), 1)
                    assert hipdev.execute(job) == pkg.Status.ERANGE
                    assert np.all(bo.read() == 0x5A)
                    bi.write(x[:1])
                    assert hipdev.execute(job) == pkg.Status.OK  # recovers on the next call
                finally:
                    bi.free()
                    bo.free()
            finally:
                mh.destroy()
                mo.destroy()


def test_read_after_single_row_execute(pkg, hipdev, oracle):
    """A single-row F32 output is also written to host memory by the kernel; a read of
    (part of) it right after the call is served from there.  Every other call that can
    change buffers must drop that copy: later writes, other jobs on the same buffer, an
    error, and a buffer whose device pointer was handed out."""
    k, n = 2048, 300
    bits, scales = pkg.synth.matrix(n, k, seed=11)
    x = pkg.synth.normal_f32(2, k, seed=11)
    with pkg.Device(oracle, 0) as odev:
        mo = odev.matrix(bits, scales)
        want = [odev.run(pkg.Op.GEMV_F32, mo, x[r:r + 1])[0] for r in range(2)]
        mo.destroy()
    m = hipdev.matrix(bits, scales)
    bi, bo = hipdev.buffer(x.nbytes), hipdev.buffer(4 * 2 * n + 64)
    try:
        bi.write(x)
        jobs = [pkg.Job(int(pkg.Op.GEMV_F32), m.handle.value, bi.view(pkg.Type.F32, r * 4 * k),
                        bo.view(pkg.Type.F32, 64 + r * 4 * n), 1) for r in range(2)]
        f = lambda raw: np.frombuffer(raw, np.float32)
        assert hipdev.execute(jobs[0]) == pkg.Status.OK
        assert np.array_equal(f(bo.read(4 * n, 64)).view(np.uint32), want[0].view(np.uint32))
        assert np.array_equal(f(bo.read(80, 64 + 40)).view(np.uint32), want[0][10:30].view(np.uint32))
        # a write to the output buffer: the next read sees the write
        bo.write(np.full(16, 7.0, np.float32), 64 + 8)
        got = f(bo.read(4 * n, 64))
        assert np.all(got[2:18] == 7.0) and np.array_equal(got[18:].view(np.uint32), want[0][18:].view(np.uint32))
        # a second job into the same buffer: both rows read back from the device
        assert hipdev.execute(jobs[0]) == pkg.Status.OK
        assert hipdev.execute(jobs[1]) == pkg.Status.OK
        both = f(bo.read(8 * n, 64))
        assert np.array_equal(both[:n].view(np.uint32), want[0].view(np.uint32))
        assert np.array_equal(both[n:].view(np.uint32), want[1].view(np.uint32))
        # an illegal input: ERANGE, the output keeps the previous row
        bad = x[1].copy()
        bad[5] = np.nan
        bi.write(bad, 4 * k)
        assert hipdev.execute(jobs[1]) == pkg.Status.ERANGE
        assert np.array_equal(f(bo.read(4 * n, 64 + 4 * n)).view(np.uint32), want[1].view(np.uint32))
        # a buffer whose device address is known may change behind the library's back
        bi.write(x[1], 4 * k)
        assert hipdev.execute(jobs[1]) == pkg.Status.OK
        dptr = bo.device_pointer()
        rt = ctypes.CDLL("libamdhip64.so")
        zeros = np.zeros(n, np.float32)
        assert rt.hipMemcpy(ctypes.c_void_p(dptr + 64 + 4 * n), zeros.ctypes.data_as(ctypes.c_void_p),
                            ctypes.c_size_t(4 * n), 1) == 0
        assert np.all(f(bo.read(4 * n, 64 + 4 * n)) == 0.0)
        assert hipdev.execute(jobs[1]) == pkg.Status.OK  # never mirrored again
        assert rt.hipMemcpy(ctypes.c_void_p(dptr + 64 + 4 * n), zeros.ctypes.data_as(ctypes.c_void_p),
                            ctypes.c_size_t(4 * n), 1) == 0
        assert np.all(f(bo.read(4 * n, 64 + 4 * n)) == 0.0)
    finally:
        bi.free()
        bo.free()
        m.destroy()


def test_batches_drop_the_host_copy(pkg, hipdev, oracle):
    """A single-row F32 output read from its host copy must not outlive a batch that
    rewrites the same bytes: BNNX_ExecuteBatch, and a prepared BNNX_BatchLaunch read
    after BNNX_DeviceSynchronize."""
    k, n = 2048, 300
    bits, scales = pkg.synth.matrix(n, k, seed=12)
    x = pkg.synth.normal_f32(3, k, seed=12)
    with pkg.Device(oracle, 0) as odev:
        mo = odev.matrix(bits, scales)
        want = [odev.run(pkg.Op.GEMV_F32, mo, x[r:r + 1])[0].view(np.uint32) for r in range(3)]
        mo.destroy()
    assert not np.array_equal(want[0], want[1]) and not np.array_equal(want[0], want[2])
    api = hipdev.api
    m = hipdev.matrix(bits, scales)
    bi, bo = hipdev.buffer(x.nbytes), hipdev.buffer(4 * n)
    batch = ctypes.c_void_p()
    try:
        bi.write(x)
        job = lambda r: pkg.Job(int(pkg.Op.GEMV_F32), m.handle.value, bi.view(pkg.Type.F32, r * 4 * k),
                                bo.view(pkg.Type.F32, 0), 1)
        out = lambda: bo.read().view(np.uint32)
        prepared = (pkg.Job * 1)(job(2))
        assert api.BNNX_BatchCreate(hipdev.handle, prepared, 1, ctypes.byref(batch)) == pkg.Status.OK
        # row 0 through BNN_Execute (host copy), then row 1 through BNNX_ExecuteBatch
        assert hipdev.execute(job(0)) == pkg.Status.OK
        assert np.array_equal(out(), want[0])
        assert api.BNNX_ExecuteBatch(hipdev.handle, (pkg.Job * 1)(job(1)), 1) == pkg.Status.OK
        assert np.array_equal(out(), want[1])
        # row 0 again, then the prepared batch (row 2) and the synchronisation
        assert hipdev.execute(job(0)) == pkg.Status.OK
        assert np.array_equal(out(), want[0])
        assert api.BNNX_BatchCheck(batch) == pkg.Status.OK
        assert api.BNNX_BatchLaunch(batch) == pkg.Status.OK
        assert api.BNNX_DeviceSynchronize(hipdev.handle) == pkg.Status.OK
        assert np.array_equal(out(), want[2])
    finally:
        if batch.value:
            api.BNNX_BatchDestroy(batch)
        bi.free()
        bo.free()
        m.destroy()
