"""ctypes mirror of the BNN accelerator API v2 (reference bnn-accelerator/bnn-accelerator.h).

`Api(path)` binds the eleven BNN_* entry points of any shared library that
exports them.  The product library is libbnn_hip.so (see `load_hip`); the
binding is the same one a Python caller of the reference's C API would write,
so the tests read like the reference's own contract test
(tests/accelerator/test_bnn_accelerator.c).

The high-level helpers (`Device`, `Matrix`, `Buffer`) raise `BnnError` on any
status other than BNN_OK, mirroring how the reference's engine turns statuses
into errors (bnn-sw-v2/common.c:76-88).
"""
from __future__ import annotations

import ctypes
import enum
import os
from pathlib import Path

import numpy as np

PKG_DIR = Path(__file__).resolve().parent
HIP_LIBRARY = PKG_DIR / "lib" / "libbnn_hip.so"

API_VERSION = 2  # bnn-accelerator.h:12
GROUP = 128


class Status(enum.IntEnum):  # bnn-accelerator.h:18-27
    OK = 0
    EINVAL = -1
    ENOMEM = -2
    ENOTSUP = -3
    ERANGE = -4
    EBUSY = -5
    EIO = -6
    ETIMEOUT = -7


class Op(enum.IntEnum):  # bnn-accelerator.h:35-41
    GEMV = 1
    GEMM = 2
    DOT_GROUPS = 3
    GEMV_F32 = 4
    GEMM_F32 = 5


class Type(enum.IntEnum):  # bnn-accelerator.h:43
    I8 = 1
    F32 = 2
    I16 = 3


class Cap(enum.IntFlag):  # bnn-accelerator.h:46-52
    GEMV = 1 << 0
    GEMM = 1 << 1
    DOT_GROUPS = 1 << 2
    GEMV_F32 = 1 << 3
    GEMM_F32 = 1 << 4


ALL_CAPS = Cap.GEMV | Cap.GEMM | Cap.DOT_GROUPS | Cap.GEMV_F32 | Cap.GEMM_F32

# (input type, output type) per operation (soft-bnn-accelerator.c:153-172)
OP_TYPES = {
    Op.GEMV: (Type.I8, Type.F32),
    Op.GEMM: (Type.I8, Type.F32),
    Op.DOT_GROUPS: (Type.I8, Type.I16),
    Op.GEMV_F32: (Type.F32, Type.F32),
    Op.GEMM_F32: (Type.F32, Type.F32),
}


class Caps(ctypes.Structure):  # bnn-accelerator.h:62-69
    _fields_ = [
        ("api_version", ctypes.c_uint32),
        ("max_in_features", ctypes.c_uint32),
        ("max_out_features", ctypes.c_uint32),
        ("max_rows", ctypes.c_uint32),
        ("group_size", ctypes.c_uint32),
        ("supported_ops", ctypes.c_uint32),
    ]


class MatrixDesc(ctypes.Structure):  # bnn-accelerator.h:92-102
    _fields_ = [
        ("in_features", ctypes.c_uint32),
        ("out_features", ctypes.c_uint32),
        ("group_size", ctypes.c_uint32),
        ("weight_bits", ctypes.c_void_p),
        ("weight_bytes", ctypes.c_size_t),
        ("scale_fp16", ctypes.c_void_p),
        ("scale_count", ctypes.c_size_t),
    ]


class BufferView(ctypes.Structure):  # bnn-accelerator.h:114-119
    _fields_ = [
        ("buffer", ctypes.c_void_p),
        ("type", ctypes.c_int),
        ("offset", ctypes.c_size_t),
        ("row_stride", ctypes.c_size_t),
    ]


class Job(ctypes.Structure):  # bnn-accelerator.h:155-161
    _fields_ = [
        ("operation", ctypes.c_int),
        ("matrix", ctypes.c_void_p),
        ("input", BufferView),
        ("output", BufferView),
        ("rows", ctypes.c_uint32),
    ]


class PreOp(ctypes.Structure):  # include/bnn-accelerator-hip.h (BNNX_PreOp)
    ROW, RMSNORM, SILU_MUL = 0, 1, 2
    _fields_ = [
        ("kind", ctypes.c_int32),
        ("width", ctypes.c_uint32),
        ("a", ctypes.c_void_p),
        ("b", ctypes.c_void_p),
        ("gain", ctypes.c_void_p),
        ("a_out", ctypes.c_void_p),
        ("eps", ctypes.c_float),
        ("err", ctypes.c_void_p),
        ("err_code", ctypes.c_int32),
    ]


class PostOp(ctypes.Structure):  # include/bnn-accelerator-hip.h (BNNX_PostOp)
    NONE, SILU_MUL = 0, 1
    _fields_ = [
        ("kind", ctypes.c_int32),
        ("out", ctypes.c_void_p),
    ]


class ChainLayer(ctypes.Structure):  # include/bnn-accelerator-hip.h (BNNX_ChainLayer)
    _fields_ = [
        ("matrix", ctypes.c_void_p),
        ("post_scale", ctypes.c_void_p),
        ("post_bias", ctypes.c_void_p),
        ("relu", ctypes.c_int32),
    ]


class BnnError(RuntimeError):
    def __init__(self, status: int, what: str = ""):
        self.status = Status(status) if status in Status._value2member_map_ else status
        super().__init__(f"{what}: {self.status!r}" if what else repr(self.status))


def _check(status: int, what: str) -> None:
    if status != Status.OK:
        raise BnnError(status, what)


class Api:
    """Raw binding of one library exporting the BNN_* C ABI."""

    def __init__(self, path: os.PathLike | str):
        self.path = str(path)
        lib = ctypes.CDLL(self.path)
        self.lib = lib
        V, S, P, U32, SZ = ctypes.c_void_p, ctypes.c_int, ctypes.POINTER, ctypes.c_uint32, ctypes.c_size_t
        sig = {
            "BNN_DeviceOpen": (S, [U32, P(V)]),
            "BNN_DeviceClose": (S, [V]),
            "BNN_DeviceGetCaps": (S, [V, P(Caps)]),
            "BNN_MatrixCreate": (S, [V, P(MatrixDesc), P(V)]),
            "BNN_MatrixDestroy": (None, [V]),
            "BNN_BufferAlloc": (S, [V, SZ, P(V)]),
            "BNN_BufferFree": (None, [V]),
            "BNN_BufferWrite": (S, [V, SZ, V, SZ]),
            "BNN_BufferRead": (S, [V, SZ, V, SZ]),
            "BNN_Execute": (S, [V, P(Job)]),
            "BNN_StatusString": (ctypes.c_char_p, [S]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
            setattr(self, name, fn)
        # HIP-backend extensions (include/bnn-accelerator-hip.h); absent elsewhere.
        ext = {
            "BNNX_DeviceOpenOrdinal": (S, [U32, P(V)]),
            "BNNX_DeviceStream": (S, [V, P(V)]),
            "BNNX_KernelTiming": (S, [V, ctypes.c_int]),
            "BNNX_KernelTimingRead": (S, [V, U32, P(ctypes.c_double), P(ctypes.c_uint64)]),
            "BNNX_DeviceName": (S, [V, ctypes.c_char_p, SZ, ctypes.c_char_p, SZ]),
            "BNNX_ExecuteBatch": (S, [V, P(Job), U32]),
            "BNNX_BatchCreate": (S, [V, P(Job), U32, P(V)]),
            "BNNX_BatchCreateFused": (S, [V, P(Job), U32, P(PreOp), P(V)]),
            "BNNX_BatchCreateFusedPost": (S, [V, P(Job), U32, P(PreOp), P(PostOp), P(V)]),
            "BNNX_BatchCreateChain": (S, [V, P(ChainLayer), U32, BufferView, BufferView, U32, P(V)]),
            "BNNX_BatchLaunch": (S, [V]),
            "BNNX_BatchCheck": (S, [V]),
            "BNNX_BatchDestroy": (None, [V]),
            "BNNX_DeviceSynchronize": (S, [V]),
            "BNNX_BufferDevicePointer": (S, [V, P(V)]),
        }
        self.extensions = set()
        for name, (res, args) in ext.items():
            fn = getattr(lib, name, None)
            if fn is None:
                continue
            fn.restype = res
            fn.argtypes = args
            setattr(self, name, fn)
            self.extensions.add(name)

    def status_string(self, status: int) -> str:
        return self.BNN_StatusString(int(status)).decode()


def load_hip() -> Api:
    """The product library.  Fails loudly when it has not been built."""
    if not HIP_LIBRARY.exists():
        raise RuntimeError(
            f"HIP backend library missing: {HIP_LIBRARY} (run __graft_entry__.build() "
            "or make -C bnn-train-infer_amd/csrc)")
    return Api(HIP_LIBRARY)


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


class Buffer:
    def __init__(self, device: "Device", nbytes: int):
        self.device = device
        self.nbytes = int(nbytes)
        h = ctypes.c_void_p()
        _check(device.api.BNN_BufferAlloc(device.handle, self.nbytes, ctypes.byref(h)), "BNN_BufferAlloc")
        self.handle = h

    def write(self, data, offset: int = 0) -> None:
        a = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        _check(self.device.api.BNN_BufferWrite(self.handle, offset, _ptr(a), a.nbytes), "BNN_BufferWrite")

    def read(self, nbytes: int | None = None, offset: int = 0) -> np.ndarray:
        n = self.nbytes - offset if nbytes is None else int(nbytes)
        out = np.empty(n, dtype=np.uint8)
        _check(self.device.api.BNN_BufferRead(self.handle, offset, _ptr(out), n), "BNN_BufferRead")
        return out

    def view(self, type_: Type, offset: int = 0, row_stride: int = 0) -> BufferView:
        return BufferView(self.handle.value, int(type_), offset, row_stride)

    def device_pointer(self) -> int:
        """Device address of the buffer (HIP backend extension)."""
        p = ctypes.c_void_p()
        _check(self.device.api.BNNX_BufferDevicePointer(self.handle, ctypes.byref(p)), "BNNX_BufferDevicePointer")
        return p.value

    def free(self) -> None:
        if self.handle:
            self.device.api.BNN_BufferFree(self.handle)
            self.handle = ctypes.c_void_p()


class Matrix:
    """Weights [out][in] as packed sign bits [out][in/8] + fp16 bit patterns [out][in/128]."""

    def __init__(self, device: "Device", bits: np.ndarray, scales: np.ndarray):
        bits = np.ascontiguousarray(bits, dtype=np.uint8)
        scales = np.ascontiguousarray(scales).view(np.uint16)
        n, kb = bits.shape
        self.device, self.k, self.n = device, kb * 8, n
        self.groups = self.k // GROUP
        d = MatrixDesc(self.k, n, GROUP, _ptr(bits), bits.nbytes, _ptr(scales), scales.size)
        h = ctypes.c_void_p()
        _check(device.api.BNN_MatrixCreate(device.handle, ctypes.byref(d), ctypes.byref(h)), "BNN_MatrixCreate")
        self.handle = h

    def destroy(self) -> None:
        if self.handle:
            self.device.api.BNN_MatrixDestroy(self.handle)
            self.handle = ctypes.c_void_p()


class Device:
    def __init__(self, api: Api, index: int = 0):
        self.api = api
        h = ctypes.c_void_p()
        _check(api.BNN_DeviceOpen(index, ctypes.byref(h)), "BNN_DeviceOpen")
        self.handle = h

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def close(self) -> None:
        if self.handle:
            _check(self.api.BNN_DeviceClose(self.handle), "BNN_DeviceClose")
            self.handle = ctypes.c_void_p()

    def caps(self) -> Caps:
        c = Caps()
        _check(self.api.BNN_DeviceGetCaps(self.handle, ctypes.byref(c)), "BNN_DeviceGetCaps")
        return c

    def matrix(self, bits: np.ndarray, scales: np.ndarray) -> Matrix:
        return Matrix(self, bits, scales)

    def buffer(self, nbytes: int) -> Buffer:
        return Buffer(self, nbytes)

    def execute(self, job: Job) -> int:
        return self.api.BNN_Execute(self.handle, ctypes.byref(job))

    def run(self, op: Op, matrix: Matrix, x: np.ndarray) -> np.ndarray:
        """One job with tight views: x is [rows][K] int8 or float32; returns the output array."""
        op = Op(op)
        in_t, out_t = OP_TYPES[op]
        x = np.ascontiguousarray(x, dtype=np.int8 if in_t == Type.I8 else np.float32)
        rows = x.shape[0] if x.ndim == 2 else 1
        if op == Op.DOT_GROUPS:
            shape, dtype = (rows, matrix.n, matrix.groups), np.int16
        else:
            shape, dtype = (rows, matrix.n), np.float32
        out_bytes = int(np.prod(shape)) * np.dtype(dtype).itemsize
        bin_, bout = self.buffer(x.nbytes), self.buffer(out_bytes)
        try:
            bin_.write(x)
            job = Job(int(op), matrix.handle.value, bin_.view(in_t), bout.view(out_t), rows)
            _check(self.execute(job), "BNN_Execute")
            return bout.read().view(dtype).reshape(shape)
        finally:
            bin_.free()
            bout.free()

    # ---- HIP extensions ----
    def stream(self) -> int:
        s = ctypes.c_void_p()
        _check(self.api.BNNX_DeviceStream(self.handle, ctypes.byref(s)), "BNNX_DeviceStream")
        return s.value or 0

    def kernel_timing(self, enable: bool) -> None:
        _check(self.api.BNNX_KernelTiming(self.handle, int(enable)), "BNNX_KernelTiming")

    def kernel_timing_read(self, kind: int) -> tuple[float, int]:
        ms, n = ctypes.c_double(), ctypes.c_uint64()
        _check(self.api.BNNX_KernelTimingRead(self.handle, kind, ctypes.byref(ms), ctypes.byref(n)),
               "BNNX_KernelTimingRead")
        return ms.value, n.value

    def name(self) -> tuple[str, str]:
        a, b = ctypes.create_string_buffer(256), ctypes.create_string_buffer(64)
        _check(self.api.BNNX_DeviceName(self.handle, a, 256, b, 64), "BNNX_DeviceName")
        return a.value.decode(), b.value.decode()
