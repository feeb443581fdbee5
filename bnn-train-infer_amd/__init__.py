"""bnn-train-infer_amd: MI355X (gfx950) HIP backend for the BNN accelerator API v2.

The product is the C-ABI library lib/libbnn_hip.so (sources in csrc/, public
headers in the repository's include/).  This Python package only binds it:
  api    -- ctypes mirror of the eleven BNN_* entry points (+ BNNX_* extensions)
  synth  -- deterministic synthetic inputs of the benchmark configurations
  gguf   -- GGUF v3 writer, Q1_0 blocks, the seeded random models (qwen3, bnn-mlp)
  engine -- ctypes binding of lib/libbnn_engine.so (BNNE_* model engine API)
The directory name has hyphens, so load it by path, e.g.
  importlib.util.spec_from_file_location("bnn_train_infer_amd", ".../__init__.py",
                                         submodule_search_locations=[...])
"""
from . import api, engine, gguf, synth  # noqa: F401
from .api import (ALL_CAPS, GROUP, HIP_LIBRARY, Api, BnnError, Buffer, BufferView, Cap, Caps, Device,  # noqa: F401
                  Job, Matrix, MatrixDesc, Op, Status, Type, load_hip)
