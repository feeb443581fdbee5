"""Benchmark-shape cases shared by the fixture generator and the parity tests."""
from __future__ import annotations

import hashlib

import numpy as np

# (name, op, K, N, rows, seed).  Seeds follow the benchmark configs (2: single-op
# microbench, 3: GEMV_F32 sweep, 4: multi-row).  lm_head is split into matrices of
# at most 8192 output features, as bnne_linear_init does (bnn-sw-v2/linear.c:104-125).
CASES = [
    ("dot_2048x6144", "DOT_GROUPS", 2048, 6144, 1, 2),
    ("gemv_i8_2048x6144", "GEMV", 2048, 6144, 1, 2),
    ("gemv_f32_2048x2048", "GEMV_F32", 2048, 2048, 1, 3),
    ("gemv_f32_2048x1024", "GEMV_F32", 2048, 1024, 1, 3),
    ("gemv_f32_2048x6144", "GEMV_F32", 2048, 6144, 1, 3),
    ("gemv_f32_6144x2048", "GEMV_F32", 6144, 2048, 1, 3),
    ("lm_head_2048x151669", "GEMV_F32", 2048, 151669, 1, 3),
] + [
    (f"{op.lower()}_m{m}_{k}x{n}", op, k, n, m, 4)
    for op in ("GEMM", "GEMM_F32") for (k, n) in ((2048, 6144), (6144, 2048)) for m in (64, 256, 1024)
] + [
    ("dot_m64_2048x6144", "DOT_GROUPS", 2048, 6144, 64, 4),
]

MAX_OUT = 8192  # BNN_Caps.max_out_features of every backend here


def case_inputs(pkg, op, k, n, rows, seed):
    """Matrix chunks [(bits, scales)] and the input rows of one case."""
    chunks = []
    for c, off in enumerate(range(0, n, MAX_OUT)):
        chunks.append(pkg.synth.matrix(min(MAX_OUT, n - off), k, seed=seed, stream=c))
    if op in ("GEMV_F32", "GEMM_F32"):
        x = pkg.synth.normal_f32(rows, k, seed=seed)
    else:
        x = pkg.synth.int8_uniform(rows, k, seed=seed)
    return chunks, x


def input_sha(chunks, x) -> str:
    h = hashlib.sha256()
    for bits, scales in chunks:
        h.update(bits.tobytes())
        h.update(scales.tobytes())
    h.update(x.tobytes())
    return h.hexdigest()


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def out_shape(op, n, rows, groups):
    if op == "DOT_GROUPS":
        return (rows, n, groups), np.int16
    return (rows, n), np.float32


def fast_oracle(pkg, oracle_fast, op, bits, scales, x, threads=16):
    """Row-parallel exact CPU evaluation of one job (test infrastructure)."""
    n, k = bits.shape[0], bits.shape[1] * 8
    rows = x.shape[0]
    shape, dtype = out_shape(op, n, rows, k // 128)
    out = np.empty(shape, dtype)
    bits = np.ascontiguousarray(bits)
    scales = np.ascontiguousarray(scales)
    x = np.ascontiguousarray(x)
    st = oracle_fast(int(pkg.Op[op]), bits.ctypes.data, scales.ctypes.data, k, n, rows, x.ctypes.data,
                     out.ctypes.data, threads)
    if st != 0:
        raise pkg.BnnError(st, "oracle_execute_parallel")
    return out


def run_chunks(pkg, dev, op, chunks, x):
    """Runs one case through a device (any backend) chunk by chunk; concatenates outputs."""
    outs = []
    for bits, scales in chunks:
        m = dev.matrix(bits, scales)
        try:
            outs.append(dev.run(pkg.Op[op], m, x))
        finally:
            m.destroy()
    return np.concatenate(outs, axis=1)


def first_mismatch(got: np.ndarray, want: np.ndarray) -> str:
    g = got.reshape(-1).view(np.uint8)
    w = want.reshape(-1).view(np.uint8)
    if g.size != w.size:
        return f"size {g.size} != {w.size}"
    bad = np.flatnonzero(g != w)
    if bad.size == 0:
        return "equal"
    item = bad[0] // got.itemsize
    return (f"{bad.size} differing bytes; first element {item}: got {got.reshape(-1)[item]!r} "
            f"want {want.reshape(-1)[item]!r}")
