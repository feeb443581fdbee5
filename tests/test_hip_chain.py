"""BNNX_BatchCreateChain (HIP-backend extension): GEMM_F32 layers applied in turn to every
row, each layer's outputs optionally mapped (post_scale * y, then + post_bias, then ReLU)
before the next layer, in one launch.  Every output is compared bit for bit with the CPU
oracle run layer by layer: one GEMM_F32 per layer, the mapping in float32 on the host
(each operation rounded on its own, as bnn-mlp.c:173-198 and this engine's host loop do)."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from bnn_cases import fast_oracle

pytestmark = pytest.mark.gpu


def _map(y, scale, bias, relu):
    if scale is not None:
        y = (scale * y).astype(np.float32)
        y = (y + bias).astype(np.float32)
    if relu:
        y = np.where(y < 0, np.float32(0), y).astype(np.float32)  # -0.0 and NaN pass, as "v < 0 ? 0 : v"
    return y


class Chain:
    """Matrices, mapping parameters (one device buffer), input and output buffers."""

    def __init__(self, pkg, dev, dims, posts, rows, seed, in_pad=0, out_pad=0, in_off=64, out_off=128):
        self.pkg, self.dev, self.dims, self.rows = pkg, dev, dims, rows
        rng = np.random.default_rng(seed)
        self.hosts = [pkg.synth.matrix(dims[i + 1], dims[i], seed=seed * 10 + i) for i in range(len(dims) - 1)]
        self.mats = [dev.matrix(*h) for h in self.hosts]
        self.params = []
        blob = []
        for i, (affine, relu) in enumerate(posts):
            n = dims[i + 1]
            if affine:
                sc = rng.uniform(0.5, 1.5, n).astype(np.float32)
                bi = rng.normal(0.0, 0.1, n).astype(np.float32)
                self.params.append((sc, bi, relu))
                blob += [sc, bi]
            else:
                self.params.append((None, None, relu))
        raw = np.concatenate(blob) if blob else np.zeros(1, np.float32)
        self.pbuf = dev.buffer(raw.nbytes)
        self.pbuf.write(raw)
        base = self.pbuf.device_pointer()
        self.layers = (pkg.api.ChainLayer * len(self.mats))()
        at = 0
        for i, (sc, bi, relu) in enumerate(self.params):
            ps = pb = None
            if sc is not None:
                ps, pb = base + at * 4, base + (at + len(sc)) * 4
                at += 2 * len(sc)
            self.layers[i] = pkg.api.ChainLayer(self.mats[i].handle.value, ps, pb, 1 if relu else 0)
        self.in_stride = dims[0] * 4 + in_pad
        self.out_stride = dims[-1] * 4 + out_pad
        self.in_off, self.out_off = in_off, out_off
        self.bi = dev.buffer(in_off + rows * self.in_stride)
        self.bo = dev.buffer(out_off + rows * self.out_stride)

    def write_input(self, x):
        raw = np.zeros(self.bi.nbytes, np.uint8)
        for r in range(self.rows):
            o = self.in_off + r * self.in_stride
            raw[o:o + x.shape[1] * 4] = x[r].view(np.uint8)
        self.bi.write(raw)

    def output(self):
        raw = self.bo.read()
        n = self.dims[-1]
        return np.stack([raw[self.out_off + r * self.out_stride:self.out_off + r * self.out_stride + 4 * n]
                         .view(np.float32) for r in range(self.rows)])

    def create(self, count=None, rows=None, in_view=None, out_view=None):
        pkg = self.pkg
        b = ctypes.c_void_p()
        iv = in_view or self.bi.view(pkg.Type.F32, self.in_off, self.in_stride)
        ov = out_view or self.bo.view(pkg.Type.F32, self.out_off, self.out_stride)
        st = self.dev.api.BNNX_BatchCreateChain(self.dev.handle, self.layers, len(self.mats) if count is None else count,
                                                iv, ov, self.rows if rows is None else rows, ctypes.byref(b))
        return st, b

    def expected(self, oracle_fast, x):
        y = x
        for (bits, scales), (sc, bi, relu) in zip(self.hosts, self.params):
            y = _map(fast_oracle(self.pkg, oracle_fast, "GEMM_F32", bits, scales, y), sc, bi, relu)
        return y

    def free(self):
        for m in self.mats:
            m.destroy()
        for b in (self.pbuf, self.bi, self.bo):
            b.free()


CASES = [
    ("bnn-mlp", [896, 512, 512, 10], [(1, 1), (1, 1), (1, 0)], 64, 0, 0),
    ("one layer, one row", [128, 64], [(0, 0)], 1, 0, 0),
    ("widest", [4096, 4096, 130], [(0, 1), (1, 0)], 3, 0, 0),
    ("strided views", [256, 1024, 384, 72], [(1, 0), (0, 1), (1, 1)], 17, 12, 20),
    ("sixteen layers", [128] * 17, [(1, 1)] * 15 + [(1, 0)], 2, 0, 4),
    ("long K then narrow", [3968, 128, 1], [(1, 1), (0, 0)], 5, 4, 0),
]


@pytest.mark.parametrize("name,dims,posts,rows,in_pad,out_pad", CASES, ids=[c[0] for c in CASES])
def test_chain_equals_layerwise_oracle(pkg, hipdev, oracle_fast, name, dims, posts, rows, in_pad, out_pad):
    print(f"chain {name}: dims {dims[:4]}{'...' if len(dims) > 4 else ''} rows {rows}", flush=True)
    c = Chain(pkg, hipdev, dims, posts, rows, seed=len(dims) * 7 + rows, in_pad=in_pad, out_pad=out_pad)
    x = pkg.synth.normal_f32(rows, dims[0], seed=rows + 3)
    x[0, : min(5, dims[0])] = [3.5, -3.5, 0.0, -0.0, 1e-30][: min(5, dims[0])]
    c.write_input(x)
    want = c.expected(oracle_fast, x)
    st, b = c.create()
    assert st == pkg.Status.OK
    api = hipdev.api
    for _ in range(2):  # launched twice without a wait in between
        assert api.BNNX_BatchLaunch(b) == pkg.Status.OK
    assert api.BNNX_DeviceSynchronize(hipdev.handle) == pkg.Status.OK
    got = c.output()
    assert got.view(np.uint32).tolist() == want.view(np.uint32).tolist()
    api.BNNX_BatchDestroy(b)
    c.free()


def test_chain_illegal_rows(pkg, hipdev, oracle_fast):
    """A non-finite input value: that row writes nothing, the others their results, and
    the synchronisation reports BNN_ERANGE once.  A mapping that overflows to infinity
    makes the next layer's input illegal: every row stops there."""
    api = hipdev.api
    dims, rows = [256, 256, 128, 20], 6
    c = Chain(pkg, hipdev, dims, [(1, 1), (1, 1), (1, 0)], rows, seed=3)
    x = pkg.synth.normal_f32(rows, dims[0], seed=9)
    x[2, 17] = np.nan
    c.write_input(x)
    ok = [0, 1, 3, 4, 5]
    want = c.expected(oracle_fast, x[ok])
    sentinel = np.full(c.bo.nbytes, 0x5A, np.uint8)
    c.bo.write(sentinel)
    st, b = c.create()
    assert st == pkg.Status.OK
    assert api.BNNX_BatchLaunch(b) == pkg.Status.OK
    assert api.BNNX_DeviceSynchronize(hipdev.handle) == pkg.Status.ERANGE
    assert api.BNNX_DeviceSynchronize(hipdev.handle) == pkg.Status.OK  # reported once
    got = c.output()
    assert got[ok].view(np.uint32).tolist() == want.view(np.uint32).tolist()
    assert got[2].view(np.uint32).tolist() == [0x5A5A5A5A] * dims[-1]
    api.BNNX_BatchDestroy(b)
    c.free()

    c = Chain(pkg, hipdev, [256, 256, 20], [(1, 0), (0, 0)], rows, seed=4)
    c.pbuf.write(np.full(256, 3.0e38, np.float32))  # layer 0's post_scale: its products overflow
    c.write_input(pkg.synth.normal_f32(rows, 256, seed=10))
    c.bo.write(np.full(c.bo.nbytes, 0x5A, np.uint8))
    st, b = c.create()
    assert st == pkg.Status.OK
    assert api.BNNX_BatchLaunch(b) == pkg.Status.OK
    assert api.BNNX_DeviceSynchronize(hipdev.handle) == pkg.Status.ERANGE
    assert c.output().view(np.uint32).tolist() == [[0x5A5A5A5A] * 20] * rows
    api.BNNX_BatchDestroy(b)
    c.free()


def test_chain_argument_checks(pkg, hipdev):
    api = hipdev.api
    S = pkg.Status
    c = Chain(pkg, hipdev, [256, 128, 10], [(1, 1), (0, 0)], 4, seed=5)
    st, b = c.create()
    assert st == S.OK
    # stale once any buffer or matrix of the device is destroyed
    assert api.BNNX_BatchCheck(b) == S.OK
    extra = hipdev.buffer(64)
    extra.free()
    assert api.BNNX_BatchCheck(b) == S.EINVAL and api.BNNX_BatchLaunch(b) == S.EINVAL
    api.BNNX_BatchDestroy(b)
    assert c.create(rows=0)[0] == S.EINVAL
    assert c.create(count=0)[0] == S.EINVAL
    assert c.create(rows=4097)[0] == S.ENOTSUP
    # the same buffer for input and output
    assert c.create(out_view=c.bi.view(pkg.Type.F32, 0, 0))[0] == S.EINVAL
    # a misaligned input row, an output view that does not fit, a wrong view type
    assert c.create(in_view=c.bi.view(pkg.Type.F32, 2, c.in_stride))[0] == S.ENOTSUP
    assert c.create(out_view=c.bo.view(pkg.Type.F32, c.bo.nbytes - 8, 0))[0] == S.ERANGE
    assert c.create(in_view=c.bi.view(pkg.Type.I8, c.in_off, c.in_stride))[0] == S.EINVAL
    # a mapping with a scale but no bias
    bad = (pkg.api.ChainLayer * 2)(*c.layers)
    bad[0].post_bias = None
    b2 = ctypes.c_void_p()
    assert api.BNNX_BatchCreateChain(hipdev.handle, bad, 2, c.bi.view(pkg.Type.F32, c.in_off, c.in_stride),
                                     c.bo.view(pkg.Type.F32, c.out_off, c.out_stride), 4, ctypes.byref(b2)) == S.EINVAL
    # layers that do not connect (K of layer 1 != N of layer 0), a layer wider than 4096
    m_other = hipdev.matrix(*pkg.synth.matrix(10, 256, seed=1))
    m_wide = hipdev.matrix(*pkg.synth.matrix(8192, 256, seed=2))
    for second, want in ((m_other, S.EINVAL),):
        lay = (pkg.api.ChainLayer * 2)(c.layers[0], pkg.api.ChainLayer(second.handle.value, None, None, 0))
        assert api.BNNX_BatchCreateChain(hipdev.handle, lay, 2, c.bi.view(pkg.Type.F32, c.in_off, c.in_stride),
                                         c.bo.view(pkg.Type.F32, c.out_off, c.out_stride), 4, ctypes.byref(b2)) == want
    wide = (pkg.api.ChainLayer * 1)(pkg.api.ChainLayer(m_wide.handle.value, None, None, 0))
    big_out = hipdev.buffer(4 * 8192 * 4)
    assert api.BNNX_BatchCreateChain(hipdev.handle, wide, 1, c.bi.view(pkg.Type.F32, c.in_off, c.in_stride),
                                     big_out.view(pkg.Type.F32, 0, 0), 4, ctypes.byref(b2)) == S.ENOTSUP
    many = (pkg.api.ChainLayer * 17)()
    assert api.BNNX_BatchCreateChain(hipdev.handle, many, 17, c.bi.view(pkg.Type.F32, c.in_off, c.in_stride),
                                     c.bo.view(pkg.Type.F32, c.out_off, c.out_stride), 4, ctypes.byref(b2)) == S.ENOTSUP
    big_out.free()
    m_other.destroy()
    m_wide.destroy()
    c.free()
