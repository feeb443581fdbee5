"""ctypes binding of the model engine library (lib/libbnn_engine.so, include/bnn-engine.h).

The engine is the caller of the accelerator API: it loads a GGUF model (qwen3 or
bnn-mlp), creates the BNN_Matrix objects on the device it is given, and runs every
linear layer through BNN_Execute.  Use it with a Device from api.py; both load the
same libbnn_hip.so.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

from .api import PKG_DIR, Device

ENGINE_LIBRARY = PKG_DIR / "lib" / "libbnn_engine.so"
TASK_CLASSIFY, TASK_LLM = 1, 2
STATUS = {0: "OK", -1: "EINVAL", -2: "ENOMEM", -3: "ENOTSUP", -4: "ERANGE", -5: "EIO", -6: "EFORMAT", -7: "ECOMPUTE"}


class ModelInfo(ctypes.Structure):
    _fields_ = [("task", ctypes.c_int), ("arch", ctypes.c_char_p), ("load_ns", ctypes.c_uint64),
                ("input_rank", ctypes.c_uint32), ("input_dims", ctypes.c_uint32 * 4),
                ("input_size", ctypes.c_uint32), ("n_classes", ctypes.c_uint32), ("n_vocab", ctypes.c_uint32),
                ("n_ctx_train", ctypes.c_uint32), ("bos_token", ctypes.c_int32), ("eos_token", ctypes.c_int32)]


class ContextParams(ctypes.Structure):
    _fields_ = [("n_ctx", ctypes.c_uint32), ("n_batch", ctypes.c_uint32), ("enable_stats", ctypes.c_int)]


STAT_FIELDS = ("calls", "items", "total_ns", "quantize_ns", "transfer_ns", "execute_ns", "host_ns", "device_calls",
               "bytes_written", "bytes_read", "logical_macs", "executed_macs")


class Stats(ctypes.Structure):
    _fields_ = [(name, ctypes.c_uint64) for name in STAT_FIELDS]

    def as_dict(self) -> dict:
        return {name: int(getattr(self, name)) for name in STAT_FIELDS}


class EngineError(RuntimeError):
    def __init__(self, status: int, what: str, detail: str):
        super().__init__(f"{what}: {STATUS.get(status, status)}: {detail}")
        self.status = status


class EngineLib:
    def __init__(self, path: os.PathLike | str = ENGINE_LIBRARY):
        if not Path(path).exists():
            raise FileNotFoundError(f"engine library missing: {path} (run __graft_entry__.build())")
        lib = ctypes.CDLL(str(path))
        vp, u32, i32 = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_int32
        sig = {
            "BNNE_ModelLoad": (ctypes.c_int, [vp, ctypes.c_char_p, ctypes.POINTER(vp)]),
            "BNNE_ModelFree": (None, [vp]),
            "BNNE_ModelGetInfo": (ctypes.c_int, [vp, ctypes.POINTER(ModelInfo)]),
            "BNNE_Tokenize": (ctypes.c_int, [vp, ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(i32), u32,
                                             ctypes.POINTER(u32)]),
            "BNNE_TokenIsEog": (ctypes.c_int, [vp, i32]),
            "BNNE_ContextParamsInit": (None, [ctypes.POINTER(ContextParams)]),
            "BNNE_ContextCreate": (ctypes.c_int, [vp, ctypes.POINTER(ContextParams), ctypes.POINTER(vp)]),
            "BNNE_ContextFree": (None, [vp]),
            "BNNE_Classify": (ctypes.c_int, [vp, ctypes.POINTER(ctypes.c_float), u32, ctypes.POINTER(ctypes.c_float)]),
            "BNNE_Decode": (ctypes.c_int, [vp, ctypes.POINTER(i32), u32, ctypes.POINTER(ctypes.c_float)]),
            "BNNE_ContextPos": (u32, [vp]),
            "BNNE_ContextTruncate": (ctypes.c_int, [vp, u32]),
            "BNNE_ContextGetStats": (ctypes.c_int, [vp, ctypes.POINTER(Stats)]),
            "BNNE_ContextResetStats": (ctypes.c_int, [vp]),
            "BNNE_StatusString": (ctypes.c_char_p, [ctypes.c_int]),
            "BNNE_LastError": (ctypes.c_char_p, []),
            "BNNEX_ContextSetResident": (ctypes.c_int, [vp, ctypes.c_int]),
            "BNNEX_ContextIsResident": (ctypes.c_int, [vp]),
            "BNNEX_DecodeGreedy": (ctypes.c_int, [vp, i32, u32, ctypes.POINTER(i32)]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args
            setattr(self, name, fn)
        self.lib = lib

    def check(self, status: int, what: str) -> None:
        if status != 0:
            raise EngineError(status, what, (self.BNNE_LastError() or b"").decode())


class Model:
    def __init__(self, eng: EngineLib, device: Device, path: os.PathLike | str):
        self.eng = eng
        h = ctypes.c_void_p()
        eng.check(eng.BNNE_ModelLoad(device.handle, str(path).encode(), ctypes.byref(h)), "BNNE_ModelLoad")
        self.handle = h
        self.info = ModelInfo()
        eng.check(eng.BNNE_ModelGetInfo(h, ctypes.byref(self.info)), "BNNE_ModelGetInfo")

    def free(self) -> None:
        if self.handle:
            self.eng.BNNE_ModelFree(self.handle)
            self.handle = None


class Context:
    def __init__(self, model: Model, n_ctx: int = 0, n_batch: int = 0, stats: bool = True):
        self.model, self.eng = model, model.eng
        p = ContextParams(n_ctx, n_batch, 1 if stats else 0)
        h = ctypes.c_void_p()
        self.eng.check(self.eng.BNNE_ContextCreate(model.handle, ctypes.byref(p), ctypes.byref(h)),
                       "BNNE_ContextCreate")
        self.handle = h

    def decode(self, tokens, want_logits: bool = True, out: np.ndarray | None = None) -> np.ndarray | None:
        """BNNE_Decode; the logits go into `out` when given (a caller's buffer reused across
        steps, as bnn-infer-v2.c:246-279 reuses one), else into a new array."""
        ids = np.ascontiguousarray(tokens, dtype=np.int32)
        if want_logits and out is not None:
            if out.dtype != np.float32 or out.shape != (self.model.info.n_vocab,) or not out.flags.c_contiguous:
                raise ValueError("out: a contiguous float32 array of n_vocab elements")
        elif want_logits:
            out = np.empty(self.model.info.n_vocab, np.float32)
        else:
            out = None
        self.eng.check(self.eng.BNNE_Decode(self.handle, ids.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                                            ids.size,
                                            out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)) if want_logits
                                            else None), "BNNE_Decode")
        return out

    def decode_greedy(self, token: int, steps: int) -> list[int]:
        """BNNEX_DecodeGreedy: `steps` one-token decode steps from `token`, each next token
        the argmax of the previous logits; the argmax after every step."""
        out = np.empty(steps, np.int32)
        self.eng.check(self.eng.BNNEX_DecodeGreedy(self.handle, int(token), int(steps),
                                                   out.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))),
                       "BNNEX_DecodeGreedy")
        return out.tolist()

    def classify(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        n = x.shape[0]
        out = np.empty((n, self.model.info.n_classes), np.float32)
        self.eng.check(self.eng.BNNE_Classify(self.handle, x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), n,
                                              out.ctypes.data_as(ctypes.POINTER(ctypes.c_float))), "BNNE_Classify")
        return out

    def set_resident(self, mode: int) -> None:
        """Execution path.  qwen3, only before the first token: 1 device with fused
        batches (the default), 2 device with prepared batches, 0 the host call pattern.
        bnn-mlp, between any two calls: 1 or 2 the device path (the default), 0 the host
        call pattern.  True and False mean 1 and 0."""
        self.eng.check(self.eng.BNNEX_ContextSetResident(self.handle, int(mode)), "BNNEX_ContextSetResident")

    def resident(self) -> int:
        """The path in effect: 1 device (fused), 2 device (prepared batches), 0 host;
        a bnn-mlp context's device path reports 2."""
        return int(self.eng.BNNEX_ContextIsResident(self.handle))

    def pos(self) -> int:
        return int(self.eng.BNNE_ContextPos(self.handle))

    def stats(self) -> dict:
        s = Stats()
        self.eng.check(self.eng.BNNE_ContextGetStats(self.handle, ctypes.byref(s)), "BNNE_ContextGetStats")
        return s.as_dict()

    def reset_stats(self) -> None:
        self.eng.check(self.eng.BNNE_ContextResetStats(self.handle), "BNNE_ContextResetStats")

    def free(self) -> None:
        if self.handle:
            self.eng.BNNE_ContextFree(self.handle)
            self.handle = None
