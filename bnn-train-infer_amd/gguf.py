"""GGUF v3 writer and the seeded random models of the benchmark configurations.

File format (what the engine reads, bnn-sw-v2/gguf.c:404-490): "GGUF", version 3,
tensor count, metadata count; metadata entries (key string, type, value); the tensor
table (name, rank, dims, type, offset relative to the data section); padding to the
alignment (32); the tensor data, each tensor at an aligned offset.

Tensor types: F32 (0), F16 (1), Q1_0 (41).  A Q1_0 tensor of dims [in, out] holds
out x (in / 128) blocks of 18 bytes: the group's fp16 scale (little-endian), then its
128 sign bits, 16 bytes, LSB first (bit 1 = +scale) -- bnn-sw-v2/linear.c:26-62.

Random models (benchmark configurations 1 and 5) draw everything from the repository's
counter-based generator (synth.u64), so every machine writes the same bytes.
"""
from __future__ import annotations

import struct
from pathlib import Path

import numpy as np

from . import synth

TYPE_F32, TYPE_F16, TYPE_Q1_0 = 0, 1, 41
_U32, _F32, _BOOL, _STRING, _ARRAY, _I32, _U64 = 4, 6, 7, 8, 9, 5, 10
ALIGNMENT = 32
GROUP = 128


def _str(value) -> bytes:
    data = value.encode("utf-8") if isinstance(value, str) else bytes(value)
    return struct.pack("<Q", len(data)) + data


class Writer:
    """Collects metadata and tensors, then writes one GGUF v3 file."""

    def __init__(self):
        self.kvs: list[bytes] = []
        self.tensors: list[tuple[str, tuple[int, ...], int, bytes]] = []

    def _kv(self, key: str, vtype: int, payload: bytes):
        self.kvs.append(_str(key) + struct.pack("<I", vtype) + payload)

    def u32(self, key, v):
        self._kv(key, _U32, struct.pack("<I", int(v)))

    def u64(self, key, v):
        self._kv(key, _U64, struct.pack("<Q", int(v)))

    def f32(self, key, v):
        self._kv(key, _F32, struct.pack("<f", float(v)))

    def boolean(self, key, v):
        self._kv(key, _BOOL, struct.pack("<B", 1 if v else 0))

    def string(self, key, v):
        self._kv(key, _STRING, _str(v))

    def strings(self, key, values):
        self._kv(key, _ARRAY, struct.pack("<IQ", _STRING, len(values)) + b"".join(_str(v) for v in values))

    def i32s(self, key, values):
        arr = np.asarray(values, dtype="<i4")
        self._kv(key, _ARRAY, struct.pack("<IQ", _I32, arr.size) + arr.tobytes())

    def tensor(self, name: str, dims, ttype: int, payload: bytes):
        dims = tuple(int(d) for d in dims)
        if ttype == TYPE_Q1_0:
            assert len(dims) == 2 and dims[0] % GROUP == 0
            expected = dims[1] * (dims[0] // GROUP) * 18
        else:
            expected = int(np.prod(dims)) * (4 if ttype == TYPE_F32 else 2)
        if len(payload) != expected:
            raise ValueError(f"{name}: {len(payload)} bytes, expected {expected}")
        self.tensors.append((name, dims, ttype, payload))

    def write(self, path):
        path = Path(path)
        path.parent.mkdir(parents=True, exist_ok=True)
        header = b"GGUF" + struct.pack("<IQQ", 3, len(self.tensors), len(self.kvs))
        table, offsets, off = [], [], 0
        for name, dims, ttype, payload in self.tensors:
            off += (-off) % ALIGNMENT
            offsets.append(off)
            table.append(_str(name) + struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims) +
                         struct.pack("<IQ", ttype, off))
            off += len(payload)
        head = header + b"".join(self.kvs) + b"".join(table)
        with open(path, "wb") as f:
            f.write(head)
            f.write(b"\0" * ((-len(head)) % ALIGNMENT))
            pos = 0
            for (name, dims, ttype, payload), start in zip(self.tensors, offsets):
                f.write(b"\0" * (start - pos))
                f.write(payload)
                pos = start + len(payload)


def q1_0_blocks(bits: np.ndarray, scales: np.ndarray) -> bytes:
    """bits [out][in/8] uint8 and scales [out][in/128] uint16 -> Q1_0 payload."""
    out, row = bits.shape
    groups = row // 16
    blocks = np.empty((out, groups, 18), np.uint8)
    blocks[:, :, 0:2] = scales.astype("<u2").view(np.uint8).reshape(out, groups, 2)
    blocks[:, :, 2:] = bits.reshape(out, groups, 16)
    return blocks.tobytes()


def q1_0_split(payload: bytes, in_features: int, out_features: int) -> tuple[np.ndarray, np.ndarray]:
    """Inverse of q1_0_blocks."""
    groups = in_features // GROUP
    blocks = np.frombuffer(payload, np.uint8).reshape(out_features, groups, 18)
    scales = blocks[:, :, 0:2].copy().view("<u2").reshape(out_features, groups)
    bits = blocks[:, :, 2:].reshape(out_features, groups * 16).copy()
    return bits, scales


def _uniform(seed: int, stream: int, count: int, lo: float, hi: float) -> np.ndarray:
    u = (synth.u64(seed, stream, count) >> np.uint64(11)).astype(np.float64) * 2.0**-53
    return lo + (hi - lo) * u


def _normal(seed: int, stream: int, count: int, mean: float, std: float) -> np.ndarray:
    """Irwin-Hall(12) approximation of N(mean, std) (exact integer sums, one rounding)."""
    w = synth.u64(seed, stream, 6 * count).reshape(count, 6)
    m24 = np.uint64(0xFFFFFF)
    s = (w & m24).astype(np.int64).sum(axis=1) + ((w >> np.uint64(24)) & m24).astype(np.int64).sum(axis=1)
    return mean + std * (s.astype(np.float64) * 2.0**-24 - 6.0)


def byte_vocabulary() -> list[str]:
    """The 256 byte-level tokens (GPT-2 byte-to-codepoint map) a BPE vocabulary must hold."""
    direct = list(range(33, 127)) + list(range(161, 173)) + list(range(174, 256))
    cp, extra = {}, 0
    for b in range(256):
        if b in direct:
            cp[b] = b
        else:
            cp[b] = 256 + extra
            extra += 1
    return [chr(cp[b]) for b in range(256)]


def qwen3_random(path, *, layers=28, hidden=2048, heads=16, kv_heads=8, head_dim=128, ffn=6144, vocab=151669,
                 context=40960, seed=5, rope_scaling=None, tweak=None) -> dict:
    """Random-init Qwen3-architecture Q1_0 model (benchmark configuration 5).

    Sign bits uniform; every Q1_0 scale of a tensor with input width `in` is
    fp16(1/sqrt(in)) (the choice of the reference's random writer); RMSNorm gains
    N(1, 0.02); eps 1e-6; rope base 1e6, no rope scaling.  The vocabulary table holds
    the 256 byte tokens and placeholders, enough for a BPE tokenizer to load; there is
    no EOS token, so generation never stops early.

    rope_scaling: None, or {"type": "yarn" | "linear" | ..., "factor": f,
    "original_context_length": n (optional)} written as the qwen3.rope.scaling.* keys
    the reference reads (bnn-sw-v2/gguf.c:272-280).
    tweak: None, or a function (tensor name, data) -> data applied before a tensor is
    written; data is (bits [out][in/8] u8, scales [out][in/128] u16) for Q1_0 tensors
    and a float32 array for gains (tests build models with chosen values this way).
    """
    w = Writer()
    w.string("general.architecture", "qwen3")
    w.u32("general.alignment", ALIGNMENT)
    w.u32("qwen3.block_count", layers)
    w.u32("qwen3.context_length", context)
    w.u32("qwen3.embedding_length", hidden)
    w.u32("qwen3.feed_forward_length", ffn)
    w.u32("qwen3.attention.head_count", heads)
    w.u32("qwen3.attention.head_count_kv", kv_heads)
    w.u32("qwen3.attention.key_length", head_dim)
    w.u32("qwen3.attention.value_length", head_dim)
    w.f32("qwen3.attention.layer_norm_rms_epsilon", 1e-6)
    w.f32("qwen3.rope.freq_base", 1e6)
    if rope_scaling is None:
        w.string("qwen3.rope.scaling.type", "none")
        w.f32("qwen3.rope.scaling.factor", 1.0)
    else:
        w.string("qwen3.rope.scaling.type", rope_scaling["type"])
        w.f32("qwen3.rope.scaling.factor", rope_scaling["factor"])
        if "original_context_length" in rope_scaling:
            w.u32("qwen3.rope.scaling.original_context_length", rope_scaling["original_context_length"])
    w.string("tokenizer.ggml.model", "gpt2")
    toks = byte_vocabulary() + [f"<t{i}>" for i in range(256, vocab)]
    w.strings("tokenizer.ggml.tokens", toks[:vocab])

    stream = [0]

    def q1(name, in_f, out_f):
        stream[0] += 1
        bits = synth.sign_bits(out_f, in_f, seed, stream=stream[0])
        scale = np.float16(1.0 / np.sqrt(in_f)).view(np.uint16)
        scales = np.full((out_f, in_f // GROUP), scale, np.uint16)
        if tweak is not None:
            bits, scales = tweak(name, (bits, scales))
        w.tensor(name, (in_f, out_f), TYPE_Q1_0, q1_0_blocks(bits, scales))

    def gains(name, n):
        stream[0] += 1
        g = _normal(seed, 7000 + stream[0], n, 1.0, 0.02).astype("<f4")
        if tweak is not None:
            g = np.asarray(tweak(name, g), "<f4")
        w.tensor(name, (n,), TYPE_F32, g.tobytes())

    q1("token_embd.weight", hidden, vocab)
    gains("output_norm.weight", hidden)
    kv = kv_heads * head_dim
    for layer in range(layers):
        gains(f"blk.{layer}.attn_norm.weight", hidden)
        gains(f"blk.{layer}.ffn_norm.weight", hidden)
        gains(f"blk.{layer}.attn_q_norm.weight", head_dim)
        gains(f"blk.{layer}.attn_k_norm.weight", head_dim)
        q1(f"blk.{layer}.attn_q.weight", hidden, hidden)
        q1(f"blk.{layer}.attn_k.weight", hidden, kv)
        q1(f"blk.{layer}.attn_v.weight", hidden, kv)
        q1(f"blk.{layer}.attn_output.weight", hidden, hidden)
        q1(f"blk.{layer}.ffn_gate.weight", hidden, ffn)
        q1(f"blk.{layer}.ffn_up.weight", hidden, ffn)
        q1(f"blk.{layer}.ffn_down.weight", ffn, hidden)
    w.write(path)
    weights = vocab * hidden + layers * (2 * hidden * hidden + 2 * hidden * kv + 3 * hidden * ffn)
    return {"layers": layers, "hidden": hidden, "heads": heads, "kv_heads": kv_heads, "head_dim": head_dim,
            "ffn": ffn, "vocab": vocab, "context": context, "seed": seed, "weights": weights,
            "weight_bytes": weights // 8 + weights // 64}


def qwen3_overflow_tweak(token: int, gain: float = 2.19e19):
    """A `tweak` for qwen3_random: the model decodes every token normally except `token`,
    whose step fails with a non-finite head RMSNorm divisor (BNNE_ECOMPUTE) in layer 0.

    Layer 0's attention RMSNorm gain of feature 0 is `gain`, so that the normalised row's
    absmax -- and with it every q/k value of the layer (its other quantised values round
    to 0) -- is `gain` times feature 0's normalised value.  That value is ~1 for a token
    whose two embedding groups have equal scales, and sqrt(2) for `token`, whose second
    group's scale is the smallest fp16 subnormal; the head norm's sum of squares
    (128 * (absmax / 16)^2 for hidden 256) then stays below FLT_MAX for every other token
    and overflows for `token`.  Layer 0's value weights get the smallest fp16 scale, so
    that the residual stream stays far from overflow.  Meant for the tiny shape
    (hidden 256, head_dim 128).
    """
    def tweak(name, data):
        if name == "token_embd.weight":
            bits, scales = data
            scales = scales.copy()
            scales[token, 1:] = 0x0001
            return bits, scales
        if name == "blk.0.attn_v.weight":
            bits, scales = data
            return bits, np.full_like(scales, 0x0001)
        if name == "blk.0.attn_norm.weight":
            g = np.array(data, np.float32)
            g[0] = np.float32(gain)
            return g
        return data
    return tweak


def prompt_ids(count: int, vocab: int, seed: int = 5) -> list[int]:
    """Seeded random prompt token IDs in [0, vocab)."""
    return [int(v) for v in synth.u64(seed, 9000, count) % np.uint64(vocab)]


def bnn_mlp_random(path, *, dims=(896, 512, 512, 10), seed=1, input_pixels=784) -> dict:
    """Random bnn-mlp classifier (benchmark configuration 1): sign bits uniform, fp16
    scales U[0.01, 0.1], post_scale U[0.5, 1.5], post_bias N(0, 0.1), ReLU on every
    block but the last."""
    w = Writer()
    blocks = len(dims) - 1
    w.string("general.architecture", "bnn-mlp")
    w.u32("general.alignment", ALIGNMENT)
    w.u32("bnn-mlp.block_count", blocks)
    w.u32("bnn-mlp.input_features", dims[0])
    w.u32("bnn-mlp.input_pixels", input_pixels)
    w.u32("bnn-mlp.class_count", dims[-1])
    w.f32("bnn-mlp.input_mean", 0.0)
    w.f32("bnn-mlp.input_std", 1.0)
    for i in range(blocks):
        w.string(f"bnn-mlp.block.{i}.activation", "relu" if i + 1 < blocks else "none")
    for i in range(blocks):
        k, n = dims[i], dims[i + 1]
        bits, scales = synth.matrix(n, k, seed, stream=10 + i)
        w.tensor(f"blk.{i}.weight", (k, n), TYPE_Q1_0, q1_0_blocks(bits, scales))
        w.tensor(f"blk.{i}.post_scale", (n,), TYPE_F32,
                 _uniform(seed, 7100 + i, n, 0.5, 1.5).astype("<f4").tobytes())
        w.tensor(f"blk.{i}.post_bias", (n,), TYPE_F32, _normal(seed, 7200 + i, n, 0.0, 0.1).astype("<f4").tobytes())
    w.write(path)
    return {"dims": list(dims), "seed": seed}


def bnn_mlp_inputs(samples: int, features: int = 896, pixels: int = 784, seed: int = 1) -> np.ndarray:
    """[samples][features] float32: N(0, 1) on the first `pixels` features, zeros after."""
    x = np.zeros((samples, features), np.float32)
    x[:, :pixels] = _normal(seed, 7300, samples * pixels, 0.0, 1.0).astype(np.float32).reshape(samples, pixels)
    return x
