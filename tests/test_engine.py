"""The model engine (lib/libbnn_engine.so): the caller of the accelerator API.

CPU: the restated bnn-engine.h ABI, the exported symbols, the GGUF writer (format
and determinism), format errors of the engine's GGUF reader, and the reference
engine (soft backend) reproducing the committed fixtures from the same seeded models.
GPU: this engine on the HIP backend (and the reference engine on the HIP backend)
reproduces the reference engine + soft backend: every decode step's greedy token and
the FNV-1a-64 hash of all logits bytes (bit-exact logits), every classifier logit.
"""
from __future__ import annotations

import ctypes
import hashlib
import json
import re
import struct
import subprocess

import numpy as np
import pytest

from conftest import GOLDEN, PKG_DIR, REF_DIR, ROOT

ENGINE_RUN_OWN = ROOT / "oracle" / "lib" / "engine_run_own"
ENGINE_RUN_SOFT = REF_DIR / "engine_run_soft"
ENGINE_RUN_REFHIP = REF_DIR / "engine_run_refhip"
TINY = json.loads((GOLDEN / "e2e_qwen3_tiny.json").read_text())
MLP = json.loads((GOLDEN / "e2e_bnn_mlp.json").read_text())
LONG = json.loads((GOLDEN / "e2e_qwen3_long.json").read_text())
ROPE = json.loads((GOLDEN / "e2e_qwen3_rope.json").read_text())
ERR = json.loads((GOLDEN / "e2e_qwen3_error.json").read_text())
SHAPES = json.loads((GOLDEN / "e2e_qwen3_shapes.json").read_text())
FULL_FIXTURE = GOLDEN / "e2e_qwen3_1p7b.json"


def engine_declared() -> set[str]:
    names = set()
    for h in ("bnn-engine.h", "bnn-engine-hip.h"):
        text = re.sub(r"/\*.*?\*/", "", (ROOT / "include" / h).read_text(), flags=re.S)
        names |= set(re.findall(r"(BNNEX?_\w+)\s*\(", text))
    return names


def parse_path(text: str) -> str:
    return next((ln.split()[1] for ln in text.splitlines() if ln.startswith("path ")), "")


def parse_llm(text: str) -> list[list]:
    return [[int(f[1]), int(f[2]), f[3]] for f in (ln.split() for ln in text.splitlines()) if f and f[0] == "step"]


def parse_greedy(text: str) -> list[int] | None:
    """The tokens of engine_run's BNNEX_DecodeGreedy pass (this engine's builds only)."""
    for f in (ln.split() for ln in text.splitlines()):
        if f and f[0] == "greedy":
            return [int(t) for t in f[1:]]
    return None


def write_tiny(pkg, tmp_path):
    model, ids = tmp_path / "tiny.gguf", tmp_path / "ids.txt"
    pkg.gguf.qwen3_random(model, **TINY["model"])
    ids.write_text(" ".join(map(str, TINY["prompt"])) + "\n")
    return model, ids


def write_rope(pkg, tmp_path, name):
    """The tiny model with one of the fixtures' RoPE scalings (YaRN or linear)."""
    rec = ROPE[name]
    model, ids = tmp_path / f"rope_{name}.gguf", tmp_path / f"rope_{name}.txt"
    pkg.gguf.qwen3_random(model, **rec["model"])
    ids.write_text(" ".join(map(str, rec["prompt"])) + "\n")
    return rec, model, ids


def write_shape(pkg, tmp_path, name):
    """One of the fixtures' models with head_dim 20 or 72 (context 61)."""
    rec = SHAPES[name]
    model, ids = tmp_path / f"shape_{name}.gguf", tmp_path / f"shape_{name}.txt"
    pkg.gguf.qwen3_random(model, **rec["model"])
    ids.write_text(" ".join(map(str, rec["prompt"])) + "\n")
    return rec, model, ids


def write_error_model(pkg, tmp_path):
    """The tiny model on which decoding ERR["error_token"] fails (BNNE_ECOMPUTE) and
    every other token decodes normally; ids files of the prompt with and without it."""
    model, ids, bad = tmp_path / "err.gguf", tmp_path / "ids.txt", tmp_path / "bad.txt"
    pkg.gguf.qwen3_random(model, **ERR["model"], tweak=pkg.gguf.qwen3_overflow_tweak(ERR["error_token"]))
    ids.write_text(" ".join(map(str, ERR["prompt"])) + "\n")
    bad.write_text(" ".join(map(str, ERR["prompt"] + [ERR["error_token"]])) + "\n")
    return model, ids, bad


def write_mlp(pkg, tmp_path):
    model, inp = tmp_path / "mlp.gguf", tmp_path / "in.f32"
    pkg.gguf.bnn_mlp_random(model, dims=tuple(MLP["dims"]), seed=MLP["seed"])
    pkg.gguf.bnn_mlp_inputs(MLP["samples"]).tofile(inp)
    return model, inp


def check_mlp_output(text: str):
    rows = [r.split() for r in text.splitlines()]
    logits = np.array([[int(h, 16) for h in r] for r in rows], dtype=np.uint32)
    assert [" ".join(r) for r in rows[:4]] == MLP["first_rows_hex"]
    assert [int(i) for i in logits.view(np.float32).argmax(axis=1)] == MLP["argmax"]
    assert hashlib.sha256(logits.tobytes()).hexdigest() == MLP["logits_sha256"]


# ----------------------------------------------------------------------------- CPU


def test_engine_header_abi_matches_reference():
    probe = ROOT / "oracle" / "lib" / "engine_abi_probe_own"
    own = subprocess.run([str(probe)], capture_output=True, text=True, check=True).stdout
    assert own == (GOLDEN / "engine_abi_layout.txt").read_text()


def test_engine_library_exports_exactly_the_header(pkg):
    lib = pkg.engine.ENGINE_LIBRARY
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib)], capture_output=True, text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    assert exported == engine_declared()
    needed = subprocess.run(["readelf", "-d", str(lib)], capture_output=True, text=True, check=True).stdout
    assert "libbnn_hip.so" in needed and "oracle" not in needed
    for src in (PKG_DIR / "engine").glob("*"):
        assert "oracle" not in src.read_text().lower(), src


def read_gguf(path):
    """Independent minimal GGUF v3 parser (metadata scalars/strings, tensor table)."""
    data = path.read_bytes()
    pos = 0

    def take(fmt):
        nonlocal pos
        v = struct.unpack_from(fmt, data, pos)
        pos += struct.calcsize(fmt)
        return v if len(v) > 1 else v[0]

    def string():
        n = take("<Q")
        nonlocal pos
        s = data[pos:pos + n]
        pos += n
        return s.decode("utf-8")

    scalar = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<B", 10: "<Q", 11: "<q", 12: "<d"}

    def value(t):
        if t == 8:
            return string()
        if t == 9:
            et, n = take("<I"), take("<Q")
            return [value(et) for _ in range(n)]
        return take(scalar[t])

    assert data[:4] == b"GGUF"
    pos = 4
    version, n_tensors, n_kv = take("<I"), take("<Q"), take("<Q")
    kv = {}
    for _ in range(n_kv):
        k = string()
        kv[k] = value(take("<I"))
    tensors = {}
    for _ in range(n_tensors):
        name = string()
        rank = take("<I")
        dims = [take("<Q") for _ in range(rank)]
        ttype, off = take("<I"), take("<Q")
        tensors[name] = (dims, ttype, off)
    align = kv.get("general.alignment", 32)
    base = (pos + align - 1) // align * align
    return version, kv, tensors, base, data


def test_gguf_writer_format(pkg, tmp_path):
    path = tmp_path / "m.gguf"
    pkg.gguf.qwen3_random(path, **TINY["model"])
    version, kv, tensors, base, data = read_gguf(path)
    m = TINY["model"]
    assert version == 3 and kv["general.architecture"] == "qwen3"
    assert kv["qwen3.block_count"] == m["layers"] and kv["qwen3.embedding_length"] == m["hidden"]
    assert len(kv["tokenizer.ggml.tokens"]) == m["vocab"]
    assert len(set(kv["tokenizer.ggml.tokens"][:256])) == 256
    assert len(tensors) == 2 + 11 * m["layers"]
    dims, ttype, off = tensors["blk.1.ffn_down.weight"]
    assert dims == [m["ffn"], m["hidden"]] and ttype == 41 and off % 32 == 0
    payload = data[base + off: base + off + m["hidden"] * (m["ffn"] // 128) * 18]
    bits, scales = pkg.gguf.q1_0_split(payload, m["ffn"], m["hidden"])
    assert pkg.gguf.q1_0_blocks(bits, scales) == payload
    assert np.all(scales == np.float16(1 / np.sqrt(m["ffn"])).view(np.uint16))
    # deterministic: the same seed writes the same bytes
    path2 = tmp_path / "m2.gguf"
    pkg.gguf.qwen3_random(path2, **TINY["model"])
    assert path.read_bytes() == path2.read_bytes()


def _engine_lib(pkg):
    return pkg.engine.EngineLib()


@pytest.mark.parametrize("case", ["missing", "magic", "version", "truncated", "no_tensors", "arch", "tensor_type"])
def test_engine_format_errors_without_device(pkg, tmp_path, case):
    """Malformed files fail inside the GGUF reader, before the device is used."""
    eng = _engine_lib(pkg)
    w = pkg.gguf.Writer()
    w.string("general.architecture", "nosuch" if case == "arch" else "qwen3")
    if case == "tensor_type":
        w.tensors.append(("t", (4,), 2, b"\0" * 8))  # Q4_0 and others are not accepted
    elif case != "no_tensors":
        w.tensor("t", (4,), pkg.gguf.TYPE_F32, b"\0" * 16)
    path = tmp_path / "bad.gguf"
    w.write(path)
    raw = bytearray(path.read_bytes())
    if case == "magic":
        raw[0:4] = b"GGUX"
    elif case == "version":
        raw[4:8] = struct.pack("<I", 2)
    elif case == "truncated":
        raw = raw[:40]
    path.write_bytes(bytes(raw))
    if case == "missing":
        path = tmp_path / "absent.gguf"
    fake_device = ctypes.c_void_p(1)  # never dereferenced on these paths
    h = ctypes.c_void_p()
    st = eng.BNNE_ModelLoad(fake_device, str(path).encode(), ctypes.byref(h))
    want = {"missing": -5, "arch": -3, "tensor_type": -3}.get(case, -6)
    assert st == want, (case, st, eng.BNNE_LastError())
    assert not h.value
    assert eng.BNNE_ModelLoad(None, str(path).encode(), ctypes.byref(h)) == -1


def test_engine_status_strings(pkg):
    eng = _engine_lib(pkg)
    assert eng.BNNE_StatusString(0) == b"success"
    assert eng.BNNE_StatusString(-6) == b"invalid or truncated model"
    assert eng.BNNE_StatusString(5) == b"unknown status"


@pytest.mark.skipif(not ENGINE_RUN_SOFT.exists(), reason="reference engine not built (no reference tree)")
def test_reference_engine_reproduces_fixtures(pkg, tmp_path):
    """The committed fixtures are what the reference engine + soft backend compute on
    the models this package writes (pins the writer and the fixture together)."""
    model, ids = write_tiny(pkg, tmp_path)
    out = subprocess.run([str(ENGINE_RUN_SOFT), "llm", str(model), str(ids), str(TINY["steps_arg"]),
                          str(TINY["ctx"])], capture_output=True, text=True, check=True).stdout
    assert parse_llm(out) == TINY["steps"]
    model, inp = write_mlp(pkg, tmp_path)
    out = subprocess.run([str(ENGINE_RUN_SOFT), "classify", str(model), str(inp), str(MLP["samples"]),
                          str(MLP["batch"])], capture_output=True, text=True, check=True).stdout
    check_mlp_output(out)


@pytest.mark.skipif(not ENGINE_RUN_SOFT.exists(), reason="reference engine not built (no reference tree)")
@pytest.mark.parametrize("name", sorted(ROPE))
def test_reference_engine_reproduces_rope_fixtures(pkg, tmp_path, name):
    """The RoPE-scaling fixtures (YaRN ramp and mscale, qwen3.c:116-142 and :298-319;
    original context defaulting to the trained one, gguf.c:483-486; linear scaling) are
    what the reference engine + soft backend compute on the models written here."""
    rec, model, ids = write_rope(pkg, tmp_path, name)
    out = subprocess.run([str(ENGINE_RUN_SOFT), "llm", str(model), str(ids), str(rec["steps_arg"]),
                          str(rec["ctx"])], capture_output=True, text=True, check=True).stdout
    assert parse_llm(out) == rec["steps"]


@pytest.mark.skipif(not ENGINE_RUN_SOFT.exists(), reason="reference engine not built (no reference tree)")
@pytest.mark.parametrize("name", sorted(SHAPES))
def test_reference_engine_reproduces_shape_fixtures(pkg, tmp_path, name):
    """The head-width fixtures (head_dim 20 and 72, a context of 61 positions) are what the
    reference engine + soft backend compute on the models written here."""
    rec, model, ids = write_shape(pkg, tmp_path, name)
    out = subprocess.run([str(ENGINE_RUN_SOFT), "llm", str(model), str(ids), str(rec["steps_arg"]),
                          str(rec["ctx"])], capture_output=True, text=True, check=True).stdout
    assert parse_llm(out) == rec["steps"]


def test_rope_fixtures_differ_from_unscaled():
    """Each scaling changes the logits (the fixtures would otherwise pin nothing of it)."""
    plain = [row[2] for row in TINY["steps"]]
    hashes = {name: [row[2] for row in rec["steps"]] for name, rec in ROPE.items()}
    for name, h in hashes.items():
        assert all(a != b for a, b in zip(h, plain)), name
    assert hashes["yarn"][1:] != hashes["yarn_default_original"][1:]


ENGINE_RUN_CPU = ROOT / "oracle" / "lib" / "engine_run_cpu"
ENGINE_RUN_ASAN = ROOT / "oracle" / "lib" / "engine_run_asan"
ASAN_ENV = {"ASAN_OPTIONS": "detect_leaks=1:abort_on_error=0:exitcode=99", "UBSAN_OPTIONS": "print_stacktrace=1"}


@pytest.mark.parametrize("exe", [ENGINE_RUN_CPU, ENGINE_RUN_ASAN], ids=["plain", "sanitized"])
def test_engine_host_step_on_cpu_oracle(pkg, tmp_path, exe):
    """This engine's host code (GGUF reader, Q1_0 layers, the Qwen3 host step, bnn-mlp)
    linked to the CPU oracle backend reproduces the reference engine + soft backend:
    every step's token and logits hash of the tiny model, all 1000x10 classifier logits.
    The sanitized build runs the same under AddressSanitizer + UndefinedBehaviorSanitizer."""
    import os
    env = dict(os.environ, **ASAN_ENV)
    model, ids = write_tiny(pkg, tmp_path)
    out = subprocess.run([str(exe), "llm", str(model), str(ids), str(TINY["steps_arg"]), str(TINY["ctx"]), "host"],
                         capture_output=True, text=True, timeout=300, env=env)
    assert out.returncode == 0, out.stderr[-2000:]
    assert parse_path(out.stdout) == "host"
    assert parse_llm(out.stdout) == TINY["steps"]
    assert parse_greedy(out.stdout) == [row[1] for row in TINY["steps"][1:]]
    model, inp = write_mlp(pkg, tmp_path)
    out = subprocess.run([str(exe), "classify", str(model), str(inp), str(MLP["samples"]), str(MLP["batch"])],
                         capture_output=True, text=True, timeout=300, env=env)
    assert out.returncode == 0, out.stderr[-2000:]
    check_mlp_output(out.stdout)


@pytest.mark.parametrize("name", sorted(ROPE))
def test_engine_rope_scaling_host_step_on_cpu_oracle(pkg, tmp_path, name):
    """This engine's RoPE tables (YaRN / linear scaling) in its host step, on the CPU
    oracle backend: every step's token and logits hash equal the reference's."""
    rec, model, ids = write_rope(pkg, tmp_path, name)
    out = subprocess.run([str(ENGINE_RUN_CPU), "llm", str(model), str(ids), str(rec["steps_arg"]), str(rec["ctx"]),
                          "host"], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr[-2000:]
    assert parse_llm(out.stdout) == rec["steps"]
    assert parse_greedy(out.stdout) == [row[1] for row in rec["steps"][1:]]


@pytest.mark.parametrize("exe", [ENGINE_RUN_CPU, ENGINE_RUN_ASAN], ids=["plain", "sanitized"])
@pytest.mark.parametrize("name", sorted(SHAPES))
def test_engine_head_widths_host_step_on_cpu_oracle(pkg, tmp_path, name, exe):
    """The host step's attention by lanes at head widths that leave partial lane groups
    (20 = 2 x 8 + 4, 72 = 64 + 8) over a 61-position context (a partial block of eight
    cached keys), on the CPU oracle backend: every step's token and logits hash equal the
    reference's; the sanitized build runs the same under AddressSanitizer +
    UndefinedBehaviorSanitizer."""
    import os
    rec, model, ids = write_shape(pkg, tmp_path, name)
    env = dict(os.environ, **ASAN_ENV)
    out = subprocess.run([str(exe), "llm", str(model), str(ids), str(rec["steps_arg"]), str(rec["ctx"]), "host"],
                         capture_output=True, text=True, timeout=300, env=env)
    assert out.returncode == 0, out.stderr[-2000:]
    assert parse_llm(out.stdout) == rec["steps"]
    assert parse_greedy(out.stdout) == [row[1] for row in rec["steps"][1:]]


@pytest.mark.parametrize("exe", [ENGINE_RUN_SOFT, ENGINE_RUN_CPU], ids=["reference", "own-host"])
def test_engine_error_model_on_cpu(pkg, tmp_path, exe):
    """The error-path model: the prompt decodes to the fixture's tokens and hashes, and a
    prompt ending in the error token fails with BNNE_ECOMPUTE, for the reference engine
    (soft backend) and this engine's host step (CPU oracle backend)."""
    if not exe.exists():
        pytest.skip(f"{exe.name} not built")
    model, ids, bad = write_error_model(pkg, tmp_path)
    mode = ["host"] if exe == ENGINE_RUN_CPU else []
    out = subprocess.run([str(exe), "llm", str(model), str(ids), str(ERR["steps_arg"]), str(ERR["ctx"])] + mode,
                         capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr[-2000:]
    assert parse_llm(out.stdout) == ERR["steps"]
    out = subprocess.run([str(exe), "llm", str(model), str(bad), "1", str(ERR["ctx"])] + mode, capture_output=True,
                         text=True, timeout=120)
    assert out.returncode == 2 and "computation failed or produced non-finite values" in out.stderr


def _classify(exe, model, inp, samples, batch, env=None):
    out = subprocess.run([str(exe), "classify", str(model), str(inp), str(samples), str(batch)],
                         capture_output=True, text=True, timeout=300, env=env)
    assert out.returncode == 0, out.stderr[-2000:]
    return out.stdout


def write_wide_mlp(pkg, tmp_path, samples):
    """One block of 256 -> 8320 outputs: two accelerator shards (8192 + 128 outputs)."""
    model, inp = tmp_path / "wide.gguf", tmp_path / "wide.f32"
    pkg.gguf.bnn_mlp_random(model, dims=(256, 8320), seed=5, input_pixels=200)
    pkg.gguf.bnn_mlp_inputs(samples, features=256, pixels=200, seed=5).tofile(inp)
    return model, inp


@pytest.mark.parametrize("exe", [ENGINE_RUN_CPU, ENGINE_RUN_ASAN], ids=["plain", "sanitized"])
def test_engine_classify_rows_match_per_sample_on_cpu_oracle(pkg, tmp_path, exe):
    """A classify call's samples go through each block as one GEMM_F32 job per shard, in
    chunks of at most 256 rows; the logits are bit-identical to one sample per call (one
    GEMV_F32 per sample, the reference's pattern), including a layer split into two
    shards and a last chunk of 44 rows (300 samples per call)."""
    import os
    env = dict(os.environ, **ASAN_ENV)
    model, inp = write_wide_mlp(pkg, tmp_path, 300)
    rows = _classify(exe, model, inp, 300, 300, env)
    single = _classify(exe, model, inp, 300, 1, env)
    assert len(rows.splitlines()) == 300
    assert rows == single


@pytest.mark.parametrize("exe", [ENGINE_RUN_CPU, ENGINE_RUN_ASAN], ids=["plain", "sanitized"])
def test_engine_classify_respects_backend_max_rows(pkg, tmp_path, exe):
    """A backend that takes at most 100 rows per job (as the reference's remote backend
    takes 128: remote-bnn-accelerator.c:39,624; the CPU oracle's ORACLE_MAX_ROWS hook
    reports and enforces such a limit): chunks of 256 rows run as jobs of <= 100 rows,
    with the same logits as one sample per call."""
    import os
    env = dict(os.environ, **ASAN_ENV, ORACLE_MAX_ROWS="100")
    model, inp = write_wide_mlp(pkg, tmp_path, 300)
    rows = _classify(exe, model, inp, 300, 300, env)
    single = _classify(exe, model, inp, 300, 1, dict(os.environ, **ASAN_ENV))
    assert len(rows.splitlines()) == 300
    assert rows == single


def _run_sanitized(args, env):
    out = subprocess.run([str(ENGINE_RUN_ASAN), *args], capture_output=True, text=True, timeout=60, env=env)
    report = "AddressSanitizer" in out.stderr or "runtime error" in out.stderr or "LeakSanitizer" in out.stderr
    return out.returncode, report, out.stderr


@pytest.mark.parametrize("case", ["missing", "magic", "version", "truncated", "no_tensors", "arch", "tensor_type"])
def test_engine_format_errors_sanitized(pkg, tmp_path, case):
    """The malformed files of test_engine_format_errors_without_device, read by the
    sanitized host build: an engine error (exit 2), no sanitizer report."""
    import os
    w = pkg.gguf.Writer()
    w.string("general.architecture", "nosuch" if case == "arch" else "qwen3")
    if case == "tensor_type":
        w.tensors.append(("t", (4,), 2, b"\0" * 8))
    elif case != "no_tensors":
        w.tensor("t", (4,), pkg.gguf.TYPE_F32, b"\0" * 16)
    path = tmp_path / "bad.gguf"
    w.write(path)
    raw = bytearray(path.read_bytes())
    if case == "magic":
        raw[0:4] = b"GGUX"
    elif case == "version":
        raw[4:8] = struct.pack("<I", 2)
    elif case == "truncated":
        raw = raw[:40]
    path.write_bytes(bytes(raw))
    if case == "missing":
        path = tmp_path / "absent.gguf"
    ids = tmp_path / "ids.txt"
    ids.write_text("1 2\n")
    rc, report, err = _run_sanitized(["llm", str(path), str(ids), "1", "8", "host"], dict(os.environ, **ASAN_ENV))
    assert rc == 2 and not report, err[-2000:]


def test_engine_gguf_mutation_fuzz_sanitized(pkg, tmp_path):
    """Bounded mutation fuzz of the GGUF reader and model loaders under ASan/UBSan: the
    tiny Qwen3 and bnn-mlp files with bytes of their header, metadata and tensor table
    overwritten, lengths and counts set to extremes, or the file cut short.  Each run
    must end with success or an engine error -- never a sanitizer report, a crash or a
    hang.  Stops at the first failure."""
    import os
    import random
    env = dict(os.environ, **ASAN_ENV)
    model, ids = write_tiny(pkg, tmp_path)
    mlp, inp = write_mlp(pkg, tmp_path)
    rng = random.Random(20261202)
    extremes = [b"\xff" * 8, b"\x00" * 8, struct.pack("<Q", 2 ** 32), struct.pack("<Q", 2 ** 63 + 1),
                struct.pack("<I", 0xffffffff), struct.pack("<I", 13), struct.pack("<I", 9)]
    for base, run in ((model, ["llm", None, str(ids), "1", "16", "host"]),
                      (mlp, ["classify", None, str(inp), "2", "2"])):
        pristine = base.read_bytes()
        # the header, metadata and tensor table: everything before the first tensor's data
        _, _, _, data_start, _ = read_gguf(base)
        for trial in range(60):
            raw = bytearray(pristine)
            kind = trial % 3
            if kind == 0:
                for _ in range(rng.randint(1, 8)):
                    raw[rng.randrange(data_start)] = rng.randrange(256)
            elif kind == 1:
                at = rng.randrange(data_start - 8)
                v = rng.choice(extremes)
                raw[at:at + len(v)] = v
            else:
                raw = raw[:rng.randrange(1, len(raw))]
            path = tmp_path / "fuzz.gguf"
            path.write_bytes(bytes(raw))
            args = list(run)
            args[1] = str(path)
            rc, report, err = _run_sanitized(args, env)
            assert rc in (0, 2) and not report, (base.name, trial, kind, rc, err[-2000:])


# ----------------------------------------------------------------------------- GPU


@pytest.mark.gpu
@pytest.mark.parametrize("runner", ["own-device", "own-prepared", "own-host", "refhip"])
def test_engine_qwen3_tiny_bit_exact(pkg, tmp_path, runner):
    exe = ENGINE_RUN_REFHIP if runner == "refhip" else ENGINE_RUN_OWN
    if runner == "refhip" and not exe.exists():
        pytest.skip("reference engine on HIP not built")
    model, ids = write_tiny(pkg, tmp_path)
    print(f"engine qwen3 tiny via {exe.name} {runner}", flush=True)
    args = [str(exe), "llm", str(model), str(ids), str(TINY["steps_arg"]), str(TINY["ctx"])]
    out = subprocess.run(args + ([runner.split("-")[1]] if runner != "refhip" else []), capture_output=True,
                         text=True, timeout=120, check=True).stdout
    if runner != "refhip":
        assert parse_path(out) == runner.split("-")[1]
        assert parse_greedy(out) == [row[1] for row in TINY["steps"][1:]]
    assert parse_llm(out) == TINY["steps"]


@pytest.mark.gpu
@pytest.mark.parametrize("path", ["device", "prepared", "host"])
@pytest.mark.parametrize("name", sorted(ROPE))
def test_engine_rope_scaling_bit_exact(pkg, tmp_path, name, path):
    """YaRN and linear RoPE scaling on every decode path (the device paths read the
    host-computed tables): every step's token and logits hash, and the greedy loop's
    tokens, equal the reference engine + soft backend's."""
    rec, model, ids = write_rope(pkg, tmp_path, name)
    print(f"engine qwen3 rope {name}, {path} path", flush=True)
    out = subprocess.run([str(ENGINE_RUN_OWN), "llm", str(model), str(ids), str(rec["steps_arg"]), str(rec["ctx"]),
                          path], capture_output=True, text=True, timeout=120, check=True).stdout
    assert parse_path(out) == path
    assert parse_llm(out) == rec["steps"]
    assert parse_greedy(out) == [row[1] for row in rec["steps"][1:]]


@pytest.mark.gpu
@pytest.mark.parametrize("path", ["prepared", "host"])
@pytest.mark.parametrize("name", sorted(SHAPES))
def test_engine_head_widths_bit_exact(pkg, tmp_path, name, path):
    """head_dim 20 and 72 over 61 positions: the host step's attention by lanes, and the
    device step's per-head kernels for head widths other than the fused step's 128 (such a
    model runs the device step with prepared batches), against the reference engine + soft
    backend."""
    rec, model, ids = write_shape(pkg, tmp_path, name)
    print(f"engine qwen3 head width {name}, {path} path", flush=True)
    out = subprocess.run([str(ENGINE_RUN_OWN), "llm", str(model), str(ids), str(rec["steps_arg"]), str(rec["ctx"]),
                          path], capture_output=True, text=True, timeout=120, check=True).stdout
    assert parse_path(out) == path
    assert parse_llm(out) == rec["steps"]
    assert parse_greedy(out) == [row[1] for row in rec["steps"][1:]]


@pytest.mark.gpu
@pytest.mark.parametrize("path", ["device", "prepared"])
def test_engine_qwen3_long_context_bit_exact(pkg, tmp_path, path):
    """Decoding past 4096 positions: the device attention's multi-pass V rows (more
    than 1024 positions) and its probabilities recomputed beyond the LDS capacity
    (more than 4096), against the reference engine + soft backend."""
    model, ids = tmp_path / "long.gguf", tmp_path / "ids.txt"
    pkg.gguf.qwen3_random(model, **LONG["model"])
    prompt = pkg.gguf.prompt_ids(LONG["prompt_count"], LONG["model"]["vocab"], seed=LONG["prompt_seed"])
    ids.write_text(" ".join(map(str, prompt)) + "\n")
    print(f"engine qwen3 long context, {path} path", flush=True)
    out = subprocess.run([str(ENGINE_RUN_OWN), "llm", str(model), str(ids), str(LONG["steps_arg"]), str(LONG["ctx"]),
                          path], capture_output=True, text=True, timeout=300, check=True).stdout
    assert parse_path(out) == path
    assert parse_llm(out) == LONG["steps"]


@pytest.mark.gpu
@pytest.mark.parametrize("cli", ["bnn-infer-v2-own", "bnn-infer-v2-hip"])
def test_reference_cli_on_this_build(pkg, tmp_path, cli):
    """The reference CLI (bnn-infer-v2.c, unchanged) linked against this engine
    (-own) or the reference engine on this backend (-hip) prints the same token
    pieces as the reference CLI with the soft backend."""
    exe = REF_DIR / cli
    if not exe.exists():
        pytest.skip(f"{cli} not built")
    model, ids = write_tiny(pkg, tmp_path)
    out = subprocess.run([str(exe), "llm", str(model), "--ids", str(ids), "--steps", str(TINY["cli_steps"]),
                          "--ctx", str(TINY["ctx"])], capture_output=True, timeout=120, check=True).stdout
    assert out.hex() == TINY["cli_stdout_hex"]


@pytest.mark.gpu
@pytest.mark.parametrize("runner", ["own-device", "own-host", "refhip"])
def test_engine_bnn_mlp_bit_exact(pkg, tmp_path, runner):
    """The bnn-mlp fixture (1000 samples in calls of 64, reference engine + soft backend)
    on this engine's device path (the default), its host call pattern and the reference
    engine on this backend."""
    exe = ENGINE_RUN_OWN if runner.startswith("own") else ENGINE_RUN_REFHIP
    if runner == "refhip" and not exe.exists():
        pytest.skip("reference engine on HIP not built")
    model, inp = write_mlp(pkg, tmp_path)
    print(f"engine bnn-mlp via {exe.name} {runner}", flush=True)
    mode = [runner.split("-")[1]] if runner.startswith("own") else []
    out = subprocess.run([str(exe), "classify", str(model), str(inp), str(MLP["samples"]), str(MLP["batch"])] + mode,
                         capture_output=True, text=True, timeout=120, check=True)
    if mode:
        assert f"path {mode[0]}" in out.stderr
    check_mlp_output(out.stdout)


@pytest.mark.gpu
@pytest.mark.parametrize("form", ["chain", "per-block"])
def test_engine_mlp_device_path_matches_host(pkg, hip, tmp_path, form):
    """bnn-mlp classify on the device path: a chunk's rows are copied to the device once,
    the blocks run there -- as one chained batch (every block and its post_scale * y +
    post_bias and ReLU in one launch), or, with a block wider than a chain takes (4224
    outputs), as a prepared batch of GEMM_F32 jobs per block plus the engine's
    post-operation kernel -- and only the logits come back.  Bit-identical to the host
    call pattern for call sizes 1..300 (a context of 300 stages chunks of 256 + 44), with
    more chunk sizes than the path keeps batches for (evicted and rebuilt), after another
    context's buffers were freed (its batches stale and rebuilt), and when the path
    changes between calls; the statistics count the same jobs and MACs."""
    if form == "chain":
        model_path, _ = write_mlp(pkg, tmp_path)
        x = pkg.gguf.bnn_mlp_inputs(300, seed=7)
    else:
        model_path = tmp_path / "wide_block.gguf"
        pkg.gguf.bnn_mlp_random(model_path, dims=(256, 4224, 10), seed=6, input_pixels=200)
        x = pkg.gguf.bnn_mlp_inputs(300, features=256, pixels=200, seed=7)
    eng = _engine_lib(pkg)
    sizes = [1, 7, 64, 300, 2, 3, 4, 5, 300, 64]
    with pkg.Device(hip, 0) as dev:
        m = pkg.engine.Model(eng, dev, model_path)
        host = pkg.engine.Context(m, n_batch=300)
        host.set_resident(0)
        assert host.resident() == 0
        device = pkg.engine.Context(m, n_batch=300)
        assert device.resident() == 2  # the default: prepared batches on the device
        print(f"engine bnn-mlp device path ({form}) vs host, sizes", sizes, flush=True)
        s0 = 0
        for n in sizes:
            rows = x[s0:s0 + n] if s0 + n <= len(x) else x[:n]
            want = host.classify(rows)
            got = device.classify(rows)
            assert got.shape == (n, 10) and got.view(np.uint32).tolist() == want.view(np.uint32).tolist(), n
            s0 = (s0 + n) % 200
            if n == 4:  # another context's buffers freed: the device path's batches go stale
                other = pkg.engine.Context(m, n_batch=8)
                other.free()
        hs, ds = host.stats(), device.stats()
        for field in ("calls", "items", "device_calls", "logical_macs", "executed_macs"):
            assert hs[field] == ds[field], field
        # the path changes between calls, both ways
        device.set_resident(0)
        assert device.resident() == 0
        assert device.classify(x[:9]).view(np.uint32).tolist() == host.classify(x[:9]).view(np.uint32).tolist()
        device.set_resident(1)
        assert device.resident() == 2
        assert device.classify(x[:9]).view(np.uint32).tolist() == host.classify(x[:9]).view(np.uint32).tolist()
        with pytest.raises(pkg.engine.EngineError) as e:
            device.set_resident(3)
        assert e.value.status == -1 and device.resident() == 2
        host.free()
        device.free()
        m.free()


@pytest.mark.gpu
def test_engine_mlp_sharded_block_stays_on_host(pkg, hip, tmp_path):
    """A block split over two accelerator shards (256 -> 8320): the device path declines
    (BNNE_ENOTSUP), the context classifies with the host call pattern."""
    model_path, _ = write_wide_mlp(pkg, tmp_path, 4)
    eng = _engine_lib(pkg)
    with pkg.Device(hip, 0) as dev:
        m = pkg.engine.Model(eng, dev, model_path)
        c = pkg.engine.Context(m, n_batch=4)
        assert c.resident() == 0
        with pytest.raises(pkg.engine.EngineError) as e:
            c.set_resident(2)
        assert e.value.status == -3 and c.resident() == 0
        c.set_resident(0)
        c.free()
        m.free()


@pytest.mark.gpu
def test_engine_classify_rows_match_per_sample(pkg, tmp_path):
    """On the HIP backend: the multi-row classify path (GEMM_F32 on the matrix cores,
    two shards, chunks of 256 + 44 rows) equals one GEMV_F32 per sample, bit for bit."""
    model, inp = write_wide_mlp(pkg, tmp_path, 300)
    print("engine classify 256->8320, 300 samples, rows vs per sample", flush=True)
    assert _classify(ENGINE_RUN_OWN, model, inp, 300, 300) == _classify(ENGINE_RUN_OWN, model, inp, 300, 1)


@pytest.mark.gpu
@pytest.mark.parametrize("resident", [1, 2, 0], ids=["device", "prepared", "host"])
def test_engine_api_behaviour(pkg, hip, tmp_path, resident):
    """Argument and range checks of the public API on a loaded model (engine.c:241-338)."""
    model_path, _ = write_tiny(pkg, tmp_path)
    eng = _engine_lib(pkg)
    with pkg.Device(hip, 0) as dev:
        m = pkg.engine.Model(eng, dev, model_path)
        assert m.info.task == pkg.engine.TASK_LLM and m.info.n_vocab == TINY["model"]["vocab"]
        assert m.info.n_ctx_train == TINY["model"]["context"] and m.info.eos_token == -1
        with pytest.raises(pkg.engine.EngineError) as e:
            pkg.engine.Context(m, n_ctx=TINY["model"]["context"] + 1)
        assert e.value.status == -4
        c = pkg.engine.Context(m, n_ctx=16, n_batch=4)
        assert c.resident() == 1  # fused batches by default
        c.set_resident(resident)
        assert c.resident() == resident
        with pytest.raises(pkg.engine.EngineError) as e:
            c.set_resident(3)
        assert e.value.status == -1 and c.resident() == resident
        prompt = TINY["prompt"]
        with pytest.raises(pkg.engine.EngineError) as e:
            c.decode(prompt[:5])  # more than n_batch
        assert e.value.status == -4
        with pytest.raises(pkg.engine.EngineError) as e:
            c.decode([TINY["model"]["vocab"]])  # outside the vocabulary
        assert e.value.status == -4 and c.pos() == 0
        with pytest.raises(pkg.engine.EngineError) as e:
            c.classify(np.zeros((1, 4), np.float32))
        assert e.value.status == -3
        logits = None
        for i in range(0, 8, 4):
            logits = c.decode(prompt[i:i + 4])
        assert c.pos() == 8 and int(np.argmax(logits)) == TINY["steps"][0][1]
        with pytest.raises(pkg.engine.EngineError) as e:
            c.set_resident(0 if resident else 1)  # only before the first token
        assert e.value.status == -1
        s = c.stats()
        assert s["calls"] == 2 and s["items"] == 8
        assert s["device_calls"] == 8 * 2 * 7 + 2  # 7 linears per layer per token, lm_head once per call
        assert s["total_ns"] >= s["transfer_ns"] + s["execute_ns"]
        assert eng.BNNE_ContextTruncate(c.handle, 9) == -1
        assert eng.BNNE_ContextTruncate(c.handle, 4) == 0 and c.pos() == 4
        c.reset_stats()
        assert c.stats()["calls"] == 0
        tok = (ctypes.c_int32 * 4)()
        n = ctypes.c_uint32()
        assert eng.BNNE_Tokenize(m.handle, b"hi", 1, tok, 4, ctypes.byref(n)) == -3
        piece, plen = ctypes.c_char_p(), ctypes.c_size_t()
        eng.lib.BNNE_TokenPiece.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.POINTER(ctypes.c_char_p),
                                            ctypes.POINTER(ctypes.c_size_t)]
        assert eng.lib.BNNE_TokenPiece(m.handle, 300, ctypes.byref(piece), ctypes.byref(plen)) == 0
        assert piece.value == b"<t300>" and plen.value == 6
        assert eng.lib.BNNE_TokenPiece(m.handle, 33, ctypes.byref(piece), ctypes.byref(plen)) == 0
        assert piece.value == b"!"  # byte tokens stand for their byte
        assert eng.lib.BNNE_TokenPiece(m.handle, TINY["model"]["vocab"], ctypes.byref(piece),
                                       ctypes.byref(plen)) == -4
        c.free()
        m.free()


@pytest.mark.gpu
@pytest.mark.skipif(not FULL_FIXTURE.exists(), reason="full-size fixture not generated")
@pytest.mark.parametrize("path", ["device", "prepared", "host"])
def test_engine_qwen3_1p7b_matches_reference(pkg, tmp_path, path):
    """Benchmark configuration 5 at full Qwen3-1.7B shape: 32 prompt tokens, 128
    greedy tokens; every step's token and logits hash equal the reference engine's."""
    full = json.loads(FULL_FIXTURE.read_text())
    model, ids = tmp_path / "q.gguf", tmp_path / "ids.txt"
    pkg.gguf.qwen3_random(model)
    ids.write_text(" ".join(map(str, full["prompt"])) + "\n")
    print(f"engine qwen3 1.7B-shape decode, 32 + 128 tokens, {path} path", flush=True)
    out = subprocess.run([str(ENGINE_RUN_OWN), "llm", str(model), str(ids), str(full["steps_arg"]),
                          str(full["ctx"]), path], capture_output=True, text=True, timeout=600, check=True).stdout
    assert parse_path(out) == path
    assert parse_llm(out) == full["steps"]


def _prefill(ctx, prompt, n_batch):
    logits = None
    for i in range(0, len(prompt), n_batch):
        logits = ctx.decode(prompt[i:i + n_batch])
    return int(np.argmax(logits))


@pytest.mark.gpu
@pytest.mark.parametrize("resident", [1, 2, 0], ids=["device", "prepared", "host"])
def test_engine_greedy_decode(pkg, hip, tmp_path, resident):
    """BNNEX_DecodeGreedy: the tokens of the reference loop (bnn-infer-v2.c:246-279, its
    argmax at :48-54) over the tiny model, the position advanced by the steps taken, and
    its argument checks leaving the position alone."""
    model_path, _ = write_tiny(pkg, tmp_path)
    eng = _engine_lib(pkg)
    want = [row[1] for row in TINY["steps"]]
    with pkg.Device(hip, 0) as dev:
        m = pkg.engine.Model(eng, dev, model_path)
        c = pkg.engine.Context(m, n_ctx=TINY["ctx"])
        c.set_resident(resident)
        print(f"greedy decode, tiny model, path {resident}", flush=True)
        first = _prefill(c, TINY["prompt"], len(TINY["prompt"]))
        assert first == want[0]
        got = c.decode_greedy(first, len(want) - 1)
        assert [first] + got == want
        pos = len(TINY["prompt"]) + len(want) - 1
        assert c.pos() == pos
        s = c.stats()
        assert s["items"] == len(TINY["prompt"]) + len(want) - 1
        for token, steps in ((TINY["model"]["vocab"], 1), (-1, 1), (0, TINY["ctx"] - pos + 1)):
            with pytest.raises(pkg.engine.EngineError) as e:
                c.decode_greedy(token, steps)
            assert e.value.status == -4 and c.pos() == pos
        out = (ctypes.c_int32 * 1)()
        assert eng.BNNEX_DecodeGreedy(c.handle, 0, 0, out) == -1
        assert eng.BNNEX_DecodeGreedy(c.handle, 0, 1, None) == -1
        # the same steps again from a truncated context
        assert eng.BNNE_ContextTruncate(c.handle, len(TINY["prompt"]) + 3) == 0
        assert c.decode_greedy(want[3], len(want) - 4) == want[4:]
        c.free()
        m.free()


@pytest.mark.gpu
@pytest.mark.parametrize("resident", [1, 2, 0], ids=["device", "prepared", "host"])
def test_engine_greedy_recovers_after_compute_error(pkg, hip, tmp_path, resident):
    """A greedy call that fails with BNNE_ECOMPUTE (its first token overflows a head
    RMSNorm, so the logits come out NaN too) leaves nothing behind: after truncating,
    the next greedy calls return the reference's tokens (the error word and the logits
    flag are cleared by each call's first launch)."""
    model_path, _, _ = write_error_model(pkg, tmp_path)
    eng = _engine_lib(pkg)
    want = [row[1] for row in ERR["steps"]]
    prompt = ERR["prompt"]
    with pkg.Device(hip, 0) as dev:
        m = pkg.engine.Model(eng, dev, model_path)
        c = pkg.engine.Context(m, n_ctx=ERR["ctx"])
        c.set_resident(resident)
        print(f"greedy after a compute error, path {resident}", flush=True)
        first = _prefill(c, prompt, len(prompt))
        assert first == want[0]
        for rep in range(2):  # twice in a row: each failure is reported once
            with pytest.raises(pkg.engine.EngineError) as e:
                c.decode_greedy(ERR["error_token"], 3)
            assert e.value.status == -7
            assert eng.BNNE_ContextTruncate(c.handle, len(prompt)) == 0
        assert [first] + c.decode_greedy(first, 5) == want[:6]
        assert c.decode_greedy(want[5], len(want) - 6) == want[6:]
        # a failed per-token decode, then greedy again
        with pytest.raises(pkg.engine.EngineError) as e:
            c.decode([ERR["error_token"]])
        assert e.value.status == -7
        assert eng.BNNE_ContextTruncate(c.handle, len(prompt)) == 0
        assert c.decode_greedy(first, 4) == want[1:5]
        c.free()
        m.free()


@pytest.mark.gpu
@pytest.mark.parametrize("resident", [1, 2], ids=["device", "prepared"])
def test_engine_greedy_decode_long_context(pkg, hip, tmp_path, resident):
    """Greedy steps past position 4160 (the device attention's multi-block form), against
    the reference engine + soft backend's tokens."""
    model_path = tmp_path / "long.gguf"
    pkg.gguf.qwen3_random(model_path, **LONG["model"])
    prompt = pkg.gguf.prompt_ids(LONG["prompt_count"], LONG["model"]["vocab"], seed=LONG["prompt_seed"])
    want = [row[1] for row in LONG["steps"]]
    eng = _engine_lib(pkg)
    with pkg.Device(hip, 0) as dev:
        m = pkg.engine.Model(eng, dev, model_path)
        c = pkg.engine.Context(m, n_ctx=LONG["ctx"], n_batch=512)
        c.set_resident(resident)
        print(f"greedy decode, long context, path {resident}", flush=True)
        first = _prefill(c, prompt, 512)
        assert first == want[0]
        assert [first] + c.decode_greedy(first, len(want) - 1) == want
        c.free()
        m.free()


@pytest.mark.gpu
@pytest.mark.skipif(not FULL_FIXTURE.exists(), reason="full-size fixture not generated")
def test_engine_greedy_decode_1p7b(pkg, hip, tmp_path):
    """Benchmark configuration 5 as one greedy call on the device path: the 128 tokens of
    the reference engine's run."""
    full = json.loads(FULL_FIXTURE.read_text())
    model_path = tmp_path / "q.gguf"
    pkg.gguf.qwen3_random(model_path)
    want = [row[1] for row in full["steps"]]
    eng = _engine_lib(pkg)
    with pkg.Device(hip, 0) as dev:
        m = pkg.engine.Model(eng, dev, model_path)
        c = pkg.engine.Context(m, n_ctx=full["ctx"])
        print("greedy decode, 1.7B shape, 32 + 128 tokens, device path", flush=True)
        first = _prefill(c, full["prompt"], len(full["prompt"]))
        assert [first] + c.decode_greedy(first, len(want) - 1) == want
        c.free()
        m.free()


def test_device_expf_restatement_matches_host_libm():
    """The device expf (csrc/libc_expf.h, shared by the backend and engine kernels) and the
    host step's four-lane form of it (engine/host_expf.h, on processors with AVX2 and FMA)
    return what the host C library's expf returns: every 13th float bit pattern here (the
    full 2^32 sweep is the same program with stride 1)."""
    exe = ROOT / "oracle" / "lib" / "libc_expf_check"
    out = subprocess.run([str(exe), "13"], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0 and out.stdout.strip().endswith("mismatches 0"), out.stdout
