#!/usr/bin/env python3
"""Writes the committed golden fixtures of tests/golden/.  Run in the build
container (where the reference tree exists), after `make -C oracle`:

    python tests/golden/make_fixtures.py

Outputs (data only: inputs and expected outputs):
  rtl_case.npz      -- the reference's RTL golden case
                       (bnn-hw-v2/simple_test/tests/case/{memory.img,golden_*.hex}, layout per
                       gen_model_case.py:220-232, 291-301), unpacked into API arrays: the matrix
                       blk.0.attn_q K=512 N=512, int8 rows q_full [16][512], q_tile [16][128],
                       f32 rows f32_tile [16][128], goldens as binary32 bits [16][512].
  soft_fixtures.json -- outputs of the reference soft backend (compiled from its source into
                       oracle/_ref/libbnn_soft_ref.so) on the seeded benchmark-shape inputs of
                       bnn-train-infer_amd/synth.py: sha256 of every output, plus the sha256 of the
                       inputs so generator drift is caught separately.
  soft_small.npz     -- full outputs of the cases whose outputs are at most 200 KB.
  ref_suite.json     -- sha256 of the raw outputs the reference's own contract test
                       (tests/accelerator/test_bnn_accelerator.c) dumps when run against soft.
  abi_layout.txt     -- oracle/_ref/abi_probe_ref output (layout of the reference header).
"""
from __future__ import annotations

import concurrent.futures as cf
import hashlib
import importlib.util
import json
import subprocess
import sys
import tempfile
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
REF = Path("/root/reference")
CASE = REF / "bnn-hw-v2/simple_test/tests/case"
SOFT = ROOT / "oracle/_ref/libbnn_soft_ref.so"

sys.path.insert(0, str(ROOT / "tests"))
from bnn_cases import CASES, case_inputs, input_sha, sha  # noqa: E402


def load_pkg():
    pkg_dir = ROOT / "bnn-train-infer_amd"
    spec = importlib.util.spec_from_file_location("bnn_train_infer_amd", pkg_dir / "__init__.py",
                                                  submodule_search_locations=[str(pkg_dir)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["bnn_train_infer_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def rtl_case() -> dict:
    img = (CASE / "memory.img").read_bytes()
    meta = json.loads((CASE / "meta.json").read_text())
    k, n, rows = meta["matrix"]["in_features"], meta["matrix"]["out_features"], meta["rows"]
    groups = k // 128
    addr = meta["addresses"]
    bits = np.zeros((n, k // 8), np.uint8)
    scales = np.zeros((n, groups), np.uint16)
    # weight records: [n_block][k_group][channel] x 18 bytes = fp16 LE scale + 16 sign-bit bytes
    for nb in range(n // 128):
        for g in range(groups):
            for ch in range(128):
                off = addr["weights"] + ((nb * groups + g) * 128 + ch) * 18
                rec = img[off:off + 18]
                row = nb * 128 + ch
                scales[row, g] = rec[0] | (rec[1] << 8)
                bits[row, g * 16:(g + 1) * 16] = np.frombuffer(rec[2:18], np.uint8)

    def i8(a, kk):
        return np.frombuffer(img[a:a + rows * kk], np.int8).reshape(rows, kk).copy()

    f32_tile = np.frombuffer(img[addr["f32_tile_input"]:addr["f32_tile_input"] + rows * 128 * 4],
                             "<f4").reshape(rows, 128).astype(np.float32)

    def golden(name):
        words = [ln for ln in (CASE / name).read_text().split("\n") if ln and not ln.startswith("#")]
        return np.array([int(w, 16) for w in words], np.uint32).reshape(rows, n)

    return dict(bits=bits, scales=scales, q_full=i8(addr["int8_full_input"], k),
                q_tile=i8(addr["int8_tile_input"], 128), f32_tile=f32_tile,
                golden_full_i8=golden("golden_full_i8.hex"), golden_tile_i8=golden("golden_tile_i8.hex"),
                golden_tile_f32=golden("golden_tile_f32.hex"))


def run_case(args):
    name, op, k, n, rows, seed = args
    pkg = load_pkg()
    soft = pkg.Api(SOFT)
    chunks, x = case_inputs(pkg, op, k, n, rows, seed)
    outs = []
    with pkg.Device(soft, 0) as dev:
        for bits, scales in chunks:
            m = dev.matrix(bits, scales)
            try:
                outs.append(dev.run(pkg.Op[op], m, x))
            finally:
                m.destroy()
    out = np.concatenate(outs, axis=1)
    return name, dict(op=op, k=k, n=n, rows=rows, seed=seed, chunks=len(chunks),
                      input_sha256=input_sha(chunks, x), output_sha256=sha(out),
                      output_bytes=int(out.nbytes)), (out if out.nbytes <= 200 * 1024 else None)


def ref_suite_dump() -> dict:
    with tempfile.TemporaryDirectory() as tmp:
        path = Path(tmp) / "dump.bin"
        subprocess.run([str(ROOT / "oracle/_ref/test_ref_vs_soft"), str(path)], check=True,
                       stdout=subprocess.DEVNULL)
        data = path.read_bytes()
    return {"bytes": len(data), "sha256": hashlib.sha256(data).hexdigest()}


def main():
    if not SOFT.exists():
        raise SystemExit("build the reference soft library first: make -C oracle")
    np.savez_compressed(HERE / "rtl_case.npz", **rtl_case())
    (HERE / "abi_layout.txt").write_text(
        subprocess.run([str(ROOT / "oracle/_ref/abi_probe_ref")], check=True, capture_output=True,
                       text=True).stdout)
    (HERE / "ref_suite.json").write_text(json.dumps(ref_suite_dump(), indent=1) + "\n")
    fixtures, small = {}, {}
    with cf.ProcessPoolExecutor(max_workers=8) as ex:
        for name, rec, out in ex.map(run_case, CASES):
            fixtures[name] = rec
            if out is not None:
                small[name] = out
            print(name, rec["output_sha256"][:16], flush=True)
    (HERE / "soft_fixtures.json").write_text(json.dumps(fixtures, indent=1, sort_keys=True) + "\n")
    np.savez_compressed(HERE / "soft_small.npz", **small)


if __name__ == "__main__":
    main()
