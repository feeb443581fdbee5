"""GPU parity of fused batches (BNNX_BatchCreateFused): the input row produced on
the device by a pre-operation, quantised and multiplied in one launch, must give
exactly what GEMV_F32 gives for the row computed on the host in the reference
engine's operation order (bnn-sw-v2/qwen3/qwen3.c:342-353 RMSNorm, :491-495
SiLU(gate)*up, :497-498 / :510-511 the residual adds).  The expected outputs come
from the CPU oracle fed with that host row."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from bnn_cases import first_mismatch

pytestmark = pytest.mark.gpu

_libm = ctypes.CDLL("libm.so.6")
_libm.expf.restype = ctypes.c_float
_libm.expf.argtypes = [ctypes.c_float]


def host_rmsnorm(a, b, gain, eps):
    """x = a (+ b); sum of x*x in index order; x / rms * gain -- all binary32."""
    x = (a + b) if b is not None else a.copy()
    total = np.cumsum(x * x, dtype=np.float32)[-1]  # sequential accumulation
    rms = np.sqrt(np.float32(total) / np.float32(x.size) + np.float32(eps))
    return x, (x / rms) * gain, rms


def host_silu_mul(a, b):
    e = np.array([_libm.expf(float(-v)) for v in a], np.float32)
    return (a / (np.float32(1.0) + e)) * b


def f32(rng, n, scale=1.0):
    return (rng.standard_normal(n) * scale).astype(np.float32)


class Fused:
    """Device objects of one fused batch: matrices, output buffers, operand buffers."""

    def __init__(self, pkg, dev, k, ns, seed):
        self.pkg, self.dev, self.k, self.ns = pkg, dev, k, ns
        self.chunks = [pkg.synth.matrix(n, k, seed=seed, stream=i) for i, n in enumerate(ns)]
        self.mats = [dev.matrix(b, s) for b, s in self.chunks]
        self.outs = [dev.buffer(4 * n) for n in ns]
        self.row = dev.buffer(4 * k)  # the jobs' input view (the produced row for PRE_ROW)
        self.ops = {name: dev.buffer(4 * k) for name in ("a", "b", "gain", "a_out")}
        self.err = dev.buffer(4)
        self.err.write(np.zeros(1, np.int32))
        self.batch = ctypes.c_void_p()

    def jobs(self):
        jobs = (self.pkg.Job * len(self.mats))()
        for i, m in enumerate(self.mats):
            jobs[i] = self.pkg.Job(int(self.pkg.Op.GEMV_F32), m.handle.value, self.row.view(self.pkg.Type.F32),
                                   self.outs[i].view(self.pkg.Type.F32), 1)
        return jobs

    def pre(self, kind, with_b=True, with_out=True, eps=1e-6, code=7, width=None):
        p = self.pkg.api.PreOp()
        p.kind, p.width, p.eps = kind, self.k if width is None else width, eps
        if kind != p.ROW:
            p.a = self.ops["a"].device_pointer()
            p.b = self.ops["b"].device_pointer() if with_b else None
        if kind == p.RMSNORM:
            p.gain = self.ops["gain"].device_pointer()
            p.a_out = self.ops["a_out"].device_pointer() if with_out else None
            p.err, p.err_code = self.err.device_pointer(), code
        return p

    def create(self, pre, jobs=None):
        jobs = self.jobs() if jobs is None else jobs
        return self.dev.api.BNNX_BatchCreateFused(self.dev.handle, jobs, len(jobs), ctypes.byref(pre),
                                                  ctypes.byref(self.batch))

    def run(self):
        assert self.dev.api.BNNX_BatchLaunch(self.batch) == 0
        return self.dev.api.BNNX_DeviceSynchronize(self.dev.handle)

    def outputs(self):
        return [o.read().view(np.float32) for o in self.outs]

    def free(self):
        if self.batch:
            self.dev.api.BNNX_BatchDestroy(self.batch)
            self.batch = ctypes.c_void_p()
        for m in self.mats:
            m.destroy()
        for b in self.outs + [self.row, self.err] + list(self.ops.values()):
            b.free()


def expected(pkg, oracle, chunks, row):
    with pkg.Device(oracle, 0) as ref:
        out = []
        for bits, scales in chunks:
            m = ref.matrix(bits, scales)
            out.append(ref.run(pkg.Op.GEMV_F32, m, row.reshape(1, -1))[0])
            m.destroy()
    return out


def check(got, want):
    for g, w in zip(got, want):
        assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), first_mismatch(g, w)


@pytest.mark.parametrize("k,ns", [(2048, [2048, 1000, 64]), (6144, [2048]), (128, [130])])
def test_fused_row(pkg, hipdev, oracle, k, ns):
    rng = np.random.default_rng(k)
    f = Fused(pkg, hipdev, k, ns, seed=k)
    try:
        x = f32(rng, k)
        f.row.write(x)
        assert f.create(f.pre(pkg.api.PreOp.ROW)) == 0
        assert f.run() == 0
        check(f.outputs(), expected(pkg, oracle, f.chunks, x))
    finally:
        f.free()


@pytest.mark.parametrize("k,ns,with_b,with_out", [
    (2048, [2048, 1024, 1024], True, True),   # a Qwen3-1.7B q/k/v layer
    (2048, [6144, 6144], False, True),        # gate/up shape, first layer (no residual)
    (2048, [512], True, False),
    (6144, [2048, 96], True, True),           # the wide template
])
def test_fused_rmsnorm(pkg, hipdev, oracle, k, ns, with_b, with_out):
    rng = np.random.default_rng(k + len(ns))
    f = Fused(pkg, hipdev, k, ns, seed=7)
    try:
        a, b = f32(rng, k, 3.0), f32(rng, k, 0.5)
        gain = (1.0 + 0.02 * rng.standard_normal(k)).astype(np.float32)
        f.ops["a"].write(a)
        f.ops["b"].write(b)
        f.ops["gain"].write(gain)
        f.ops["a_out"].write(np.full(k, 5.0, np.float32))
        assert f.create(f.pre(pkg.api.PreOp.RMSNORM, with_b, with_out, eps=1e-6)) == 0
        for rep in range(2):  # the batch relaunches on new operand values
            if rep:
                a = f32(rng, k, 0.1)
                f.ops["a"].write(a)
            assert f.run() == 0
            x, row, _ = host_rmsnorm(a, b if with_b else None, gain, 1e-6)
            check(f.outputs(), expected(pkg, oracle, f.chunks, row))
            stored = f.ops["a_out"].read().view(np.float32)
            want = x if with_out else np.full(k, 5.0, np.float32)
            assert np.array_equal(stored.view(np.uint32), want.view(np.uint32))
        assert f.err.read().view(np.int32)[0] == 0
    finally:
        f.free()


@pytest.mark.parametrize("ns,kind,k", [
    ([8192, 8192, 8192], "rms", 2048),          # 384 tiles: workgroups walk tiles, jobs at multiples of 128 tiles
    ([8192, 3000, 8192, 4213], "row", 2048),    # 394 tiles: jobs at irregular tiles (the table walk)
    ([6144] * 4 + [4096], "rms", 2048),         # 448 tiles
    ([8192] * 18 + [4213], "rms", 2048),        # the lm_head's 2370 tiles (~9 per workgroup)
    ([8192] * 8 + [3000, 4213], "row", 1152),   # 1137 tiles of 9 groups, irregular job starts
    ([8192] * 36, "row", 128),                  # 4608 tiles of one group
])
def test_fused_many_tiles(pkg, hipdev, oracle, ns, kind, k):
    """Batches with more tiles than workgroups (one per CU): each workgroup walks several
    tiles with a ring of weights in flight, finding each tile's job in one step when the
    jobs start at multiples of a power of two and by walking the table otherwise."""
    rng = np.random.default_rng(len(ns))
    f = Fused(pkg, hipdev, k, ns, seed=17)
    try:
        print(f"fused batch: {len(ns)} jobs, {sum((n + 63) // 64 for n in ns)} tiles, pre {kind}", flush=True)
        if kind == "rms":
            a, b = f32(rng, k, 2.0), f32(rng, k, 0.5)
            gain = (1.0 + 0.02 * rng.standard_normal(k)).astype(np.float32)
            f.ops["a"].write(a)
            f.ops["b"].write(b)
            f.ops["gain"].write(gain)
            assert f.create(f.pre(pkg.api.PreOp.RMSNORM, True, False, eps=1e-6)) == 0
            _, row, _ = host_rmsnorm(a, b, gain, 1e-6)
        else:
            row = f32(rng, k)
            f.row.write(row)
            assert f.create(f.pre(pkg.api.PreOp.ROW)) == 0
        for _ in range(2):
            assert f.run() == 0
            check(f.outputs(), expected(pkg, oracle, f.chunks, row))
    finally:
        f.free()


def sum_pattern(name, k, rng):
    """Rows chosen for the sum of squares: rounding that drifts far from the exact
    prefix sums, terms across many binades, subnormal terms, long zero runs."""
    if name == "constant":  # the same rounding at every step: hundreds of ulps of drift
        return np.full(k, 1.1, np.float32)
    if name == "ramp":  # squares from 2^-70 to 2^20 in index order
        sign = rng.choice(np.array([-1.0, 1.0], np.float32), k)
        return (np.exp2(np.linspace(-35.0, 10.0, k)) * sign).astype(np.float32)
    if name == "tiny":  # subnormal and vanishing squares
        return f32(rng, k, 1e-22)
    if name == "zero_head":
        a = f32(rng, k)
        a[: k * 3 // 4] = 0.0
        return a
    if name == "spikes":  # a few large terms among small ones
        a = f32(rng, k, 1e-3)
        a[rng.integers(0, k, 5)] = 300.0
        return a
    raise ValueError(name)


@pytest.mark.parametrize("pattern", ["constant", "ramp", "tiny", "zero_head", "spikes"])
@pytest.mark.parametrize("k", [2048, 1152, 6144, 128])
def test_fused_rmsnorm_sum_patterns(pkg, hipdev, oracle, k, pattern):
    """The sum of squares is evaluated in parallel segments and resolved exactly;
    these rows make the resolution fall back to term-by-term addition."""
    rng = np.random.default_rng(k)
    f = Fused(pkg, hipdev, k, [64], seed=13)
    try:
        a = sum_pattern(pattern, k, rng)
        gain = np.ones(k, np.float32)
        f.ops["a"].write(a)
        f.ops["gain"].write(gain)
        assert f.create(f.pre(pkg.api.PreOp.RMSNORM, with_b=False, with_out=False)) == 0
        assert f.run() == 0
        _, row, _ = host_rmsnorm(a, None, gain, 1e-6)
        check(f.outputs(), expected(pkg, oracle, f.chunks, row))
    finally:
        f.free()


@pytest.mark.parametrize("k,ns", [(6144, [2048]), (1024, [300, 64])])
def test_fused_silu_mul(pkg, hipdev, oracle, k, ns):
    rng = np.random.default_rng(k)
    f = Fused(pkg, hipdev, k, ns, seed=11)
    try:
        a, b = f32(rng, k, 4.0), f32(rng, k)
        a[:4] = [0.0, -0.0, 88.5, -104.0]  # expf overflow and underflow on the way
        f.ops["a"].write(a)
        f.ops["b"].write(b)
        assert f.create(f.pre(pkg.api.PreOp.SILU_MUL)) == 0
        assert f.run() == 0
        check(f.outputs(), expected(pkg, oracle, f.chunks, host_silu_mul(a, b)))
    finally:
        f.free()


@pytest.mark.parametrize("k,ns,kind", [
    (2048, [640, 640], "rmsnorm"),           # the gate/up shape, scaled down
    (2048, [256, 96, 256, 96], "rmsnorm"),   # two pairs of different lengths
    (1024, [100, 100], "row"),               # a partial last tile, the ROW input
    (6144, [128, 128], "rmsnorm"),           # the wide template
])
def test_fused_post_silu_mul(pkg, hipdev, oracle, k, ns, kind):
    """SiLU(y_p) * y_(m+p) of the pairs stored next to the jobs' own outputs."""
    rng = np.random.default_rng(k + len(ns))
    f = Fused(pkg, hipdev, k, ns, seed=17)
    m = len(ns) // 2
    post_buf = hipdev.buffer(4 * sum(ns[:m]))
    try:
        post = pkg.api.PostOp()
        post.kind, post.out = post.SILU_MUL, post_buf.device_pointer()
        if kind == "rmsnorm":
            a, b = f32(rng, k, 3.0), f32(rng, k, 0.5)
            gain = (1.0 + 0.02 * rng.standard_normal(k)).astype(np.float32)
            f.ops["a"].write(a)
            f.ops["b"].write(b)
            f.ops["gain"].write(gain)
            pre = f.pre(pkg.api.PreOp.RMSNORM, True, False)
            _, row, _ = host_rmsnorm(a, b, gain, 1e-6)
        else:
            row = f32(rng, k, 2.0)
            f.row.write(row)
            pre = f.pre(pkg.api.PreOp.ROW)
        jobs = f.jobs()
        st = hipdev.api.BNNX_BatchCreateFusedPost(hipdev.handle, jobs, len(jobs), ctypes.byref(pre),
                                                  ctypes.byref(post), ctypes.byref(f.batch))
        assert st == 0
        assert f.run() == 0
        want = expected(pkg, oracle, f.chunks, row)
        check(f.outputs(), want)
        prod = np.concatenate([host_silu_mul(want[p], want[m + p]) for p in range(m)])
        got = post_buf.read().view(np.float32)
        assert np.array_equal(got.view(np.uint32), prod.view(np.uint32)), first_mismatch(got, prod)
    finally:
        f.free()
        post_buf.free()


def test_fused_post_create_checks(pkg, hipdev):
    S = pkg.Status
    f = Fused(pkg, hipdev, 1024, [128, 128, 64], seed=19)
    post_buf = hipdev.buffer(4 * 256)
    try:
        P = pkg.api.PreOp
        post = pkg.api.PostOp()
        post.kind, post.out = post.SILU_MUL, post_buf.device_pointer()

        def create(jobs, post_op):
            return hipdev.api.BNNX_BatchCreateFusedPost(hipdev.handle, jobs, len(jobs), ctypes.byref(f.pre(P.ROW)),
                                                        ctypes.byref(post_op), ctypes.byref(f.batch))
        jobs = f.jobs()
        assert create(jobs, post) == S.EINVAL  # three jobs: no pairs
        two = (pkg.Job * 2)(jobs[0], jobs[2])
        assert create(two, post) == S.EINVAL  # a pair of unequal lengths
        two = (pkg.Job * 2)(jobs[0], jobs[1])
        bad = pkg.api.PostOp()
        bad.kind, bad.out = 7, post_buf.device_pointer()
        assert create(two, bad) == S.EINVAL
        bad.kind, bad.out = bad.SILU_MUL, None
        assert create(two, bad) == S.EINVAL
        bad.out = f.outs[1].device_pointer()  # the products may not overlap a job output
        assert create(two, bad) == S.EINVAL
        bad.out = f.row.device_pointer()  # nor the input row
        assert create(two, bad) == S.EINVAL
        assert not f.batch
        none = pkg.api.PostOp()
        assert create(f.jobs(), none) == 0  # POST_NONE: a plain fused batch
    finally:
        f.free()
        post_buf.free()


def test_fused_illegal_rows_write_nothing(pkg, hipdev):
    """A failed RMSNorm divisor stores err_code and raises the device error; a
    non-finite produced row raises it without err_code; outputs stay untouched and
    the next clean launch succeeds."""
    k = 2048
    f = Fused(pkg, hipdev, k, [256], seed=3)
    try:
        sentinel = np.full(256, 0x5A5A5A5A, np.uint32).view(np.float32)
        f.outs[0].write(sentinel)
        f.ops["a"].write(np.zeros(k, np.float32))
        f.ops["gain"].write(np.ones(k, np.float32))
        assert f.create(f.pre(pkg.api.PreOp.RMSNORM, with_b=False, eps=0.0, code=41)) == 0
        assert f.run() == pkg.Status.ERANGE  # rms = sqrt(0 + 0) = 0
        assert f.err.read().view(np.int32)[0] == 41
        assert np.array_equal(f.outputs()[0].view(np.uint32), sentinel.view(np.uint32))
        f.err.write(np.zeros(1, np.int32))
        a = np.ones(k, np.float32)
        a[100] = np.inf
        f.ops["a"].write(a)
        assert f.run() == pkg.Status.ERANGE  # rms is inf: the divisor check again
        assert f.err.read().view(np.int32)[0] == 41
        f.err.write(np.zeros(1, np.int32))
        f.ops["a"].write(np.full(k, 1.5e19, np.float32))  # finite squares, the sum overflows
        assert f.run() == pkg.Status.ERANGE
        assert f.err.read().view(np.int32)[0] == 41
        f.err.write(np.zeros(1, np.int32))
        a[100] = 1.0
        a[7] = 4.0
        gain = np.ones(k, np.float32)
        gain[7] = np.float32(3e38)  # x[7] / rms is about 4: the product overflows
        f.ops["a"].write(a * np.float32(1e3))
        f.ops["gain"].write(gain)
        assert f.run() == pkg.Status.ERANGE  # finite divisor, an infinite input value
        assert f.err.read().view(np.int32)[0] == 0
        assert np.array_equal(f.outputs()[0].view(np.uint32), sentinel.view(np.uint32))
        f.ops["gain"].write(np.ones(k, np.float32))
        assert f.run() == 0
        assert not np.array_equal(f.outputs()[0].view(np.uint32), sentinel.view(np.uint32))
    finally:
        f.free()
    f = Fused(pkg, hipdev, 1024, [64], seed=4)
    try:
        a = np.zeros(1024, np.float32)
        a[5] = np.nan
        f.ops["a"].write(a)
        f.ops["b"].write(np.ones(1024, np.float32))
        f.outs[0].write(np.zeros(64, np.float32))
        assert f.create(f.pre(pkg.api.PreOp.SILU_MUL)) == 0
        assert f.run() == pkg.Status.ERANGE
        assert np.array_equal(f.outputs()[0], np.zeros(64, np.float32))
    finally:
        f.free()


def test_fused_create_checks(pkg, hipdev):
    S = pkg.Status
    f = Fused(pkg, hipdev, 2048, [128, 64], seed=5)
    try:
        P = pkg.api.PreOp
        assert f.create(f.pre(P.RMSNORM, width=1024)) == S.EINVAL  # the matrices' K is 2048
        bad = f.pre(P.RMSNORM)
        bad.kind = 9
        assert f.create(bad) == S.EINVAL
        bad = f.pre(P.RMSNORM)
        bad.a_out = bad.a  # the stored sum may not overlap what is read
        assert f.create(bad) == S.EINVAL
        bad = f.pre(P.RMSNORM)
        bad.b = f.outs[1].device_pointer()  # an output may not overlap an operand
        assert f.create(bad) == S.EINVAL
        bad = f.pre(P.SILU_MUL)
        bad.b = None
        assert f.create(bad) == S.EINVAL
        jobs = f.jobs()
        jobs[1].input = f.ops["b"].view(pkg.Type.F32)  # ROW: every job must read the same row
        assert f.create(f.pre(P.ROW), jobs) == S.EINVAL
        jobs = f.jobs()
        jobs[0].rows = 2  # GEMV_F32 takes one row (BNN_Execute's check)
        assert f.create(f.pre(P.ROW), jobs) == S.EINVAL
        jobs = f.jobs()
        jobs[0].operation = int(pkg.Op.GEMV)
        jobs[0].input = f.row.view(pkg.Type.I8)
        assert f.create(f.pre(P.ROW), jobs) == S.ENOTSUP
        assert not f.batch
    finally:
        f.free()
    wide = Fused(pkg, hipdev, 6272, [64], seed=6)  # 49 groups: wider than a fused batch takes
    try:
        assert wide.create(wide.pre(pkg.api.PreOp.ROW)) == S.ENOTSUP
    finally:
        wide.free()
