"""The `.ll2c` weight container: reader, writer, quantisers and a seeded
synthetic-model generator.

Format (kurulav1/cpi src/model/weight_loader.cpp:10-242, tools/pack_ll2c.py:21-278):
``LL2CUDA\\0`` magic, a V1-V4 header, a table of ``(name[64], int64 offset,
int64 bytes)`` entries (offsets absolute from the file start) and the raw
tensor bytes.  Low-bit tensors follow tools/pack_ll2c.py:102-146 and
src/engine/llama_engine_lowbit_utils.cpp:25-29: ``<base>.int8`` ``[R, K]`` or
``<base>.int4`` ``[R, ceil(K/2)]`` (low nibble = even column, two's complement)
plus ``<base>.scale`` fp32 ``[R]`` (or ``[1]``, a global scale).

Extension used by the group-32 configurations: ``<base>.int4`` with
``<base>.gscale`` fp16 ``[R, K/32]`` (one scale per 32 consecutive columns).
"""
from __future__ import annotations

import dataclasses
import hashlib
import mmap
import os
import struct
from typing import Callable, Dict, Iterable, List, Optional, Tuple

import numpy as np

MAGIC = b"LL2CUDA\x00"
HEADER_V4 = "<8siiiiiiiiiiqffiiiiii"
ENTRY = "<64sqq"

# model_family ids (include/model/llama_config.hpp:17-25)
FAMILY = {"unknown": 0, "llama2": 1, "llama3": 2, "mistral": 3, "phi3": 4, "qwen2": 5, "mixtral": 6}


@dataclasses.dataclass
class Config:
    vocab_size: int = 32000
    hidden_size: int = 4096
    intermediate_size: int = 11008
    num_layers: int = 32
    num_heads: int = 32
    num_kv_heads: int = 32
    max_seq_len: int = 4096
    tensor_parallel: int = 1
    rope_theta: float = 0.0
    norm_eps: float = 1e-5
    sliding_window: int = 0
    tie_word_embeddings: bool = False
    has_qkv_bias: bool = False
    use_layernorm: bool = False
    model_family: int = 0
    num_local_experts: int = 0
    num_experts_per_tok: int = 0
    expert_intermediate_size: int = 0

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_heads

    def effective_rope_theta(self) -> float:
        # llama_config.hpp:27-33,63-66
        if self.rope_theta > 0:
            return self.rope_theta
        return {2: 500000.0, 5: 1000000.0}.get(self.model_family, 10000.0)


# ----------------------------------------------------------------- reading
class Reader:
    """mmap'd reader; tensor(name) returns a read-only uint8 numpy view."""

    def __init__(self, path: str):
        self.path = path
        self._f = open(path, "rb")
        self._mm = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ)
        mm = self._mm
        if len(mm) < 48 or mm[:7] != MAGIC[:7]:
            raise ValueError("unsupported weights format. expected LL2CUDA manifest")
        (version,) = struct.unpack_from("<i", mm, 8)
        c = Config()
        if version >= 2:
            (c.vocab_size, c.hidden_size, c.intermediate_size, c.num_layers, c.num_heads,
             c.num_kv_heads, c.max_seq_len, c.tensor_parallel, count) = struct.unpack_from("<9i", mm, 12)
            (table,) = struct.unpack_from("<q", mm, 48)
            if version >= 3:
                theta, eps, sw, flags, fam = struct.unpack_from("<ffiii", mm, 56)
                c.rope_theta, c.norm_eps, c.sliding_window = theta, (eps if eps > 0 else 1e-5), sw
                c.tie_word_embeddings = bool(flags & 1)
                c.has_qkv_bias = bool(flags & 2)
                c.use_layernorm = bool(flags & 4)
                c.model_family = fam
            if version >= 4:
                (c.num_local_experts, c.num_experts_per_tok,
                 c.expert_intermediate_size) = struct.unpack_from("<3i", mm, 76)
        else:
            (c.vocab_size, c.hidden_size, c.intermediate_size, c.num_layers, c.num_heads,
             c.max_seq_len, c.tensor_parallel, count) = struct.unpack_from("<8i", mm, 12)
            c.num_kv_heads = c.num_heads
            (table,) = struct.unpack_from("<q", mm, 44)
        if c.num_kv_heads <= 0 or c.num_heads <= 0 or c.num_heads % c.num_kv_heads:
            raise ValueError("invalid attention head config in model header")
        self.version = version
        self.config = c
        self.entries: Dict[str, Tuple[int, int]] = {}
        for i in range(count):
            name, off, nbytes = struct.unpack_from(ENTRY, mm, table + i * 80)
            self.entries[name.split(b"\x00", 1)[0].decode()] = (off, nbytes)

    def has(self, name: str) -> bool:
        return name in self.entries

    def tensor(self, name: str) -> np.ndarray:
        if name not in self.entries:
            raise KeyError(f"tensor not found: {name}")
        off, nbytes = self.entries[name]
        return np.frombuffer(self._mm, dtype=np.uint8, count=nbytes, offset=off)

    def close(self):
        self._mm.close()
        self._f.close()


# ---------------------------------------------------------------- writing
def write(path: str, cfg: Config, tensors: Iterable[Tuple[str, int, Callable[[], bytes]]]) -> None:
    """Write a V4 file.  `tensors` yields (name, nbytes, producer) so large
    models are generated and written one tensor at a time."""
    items = list(tensors)
    header = struct.calcsize(HEADER_V4)
    cursor = header + len(items) * struct.calcsize(ENTRY)
    entries = []
    for name, nbytes, _ in items:
        raw = name.encode()
        if len(raw) >= 64:
            raise ValueError(f"Tensor name too long: {name}")
        entries.append(struct.pack(ENTRY, raw + b"\x00" * (64 - len(raw)), cursor, nbytes))
        cursor += nbytes
    flags = (1 if cfg.tie_word_embeddings else 0) | (2 if cfg.has_qkv_bias else 0) | (4 if cfg.use_layernorm else 0)
    with open(path, "wb") as f:
        f.write(struct.pack(HEADER_V4, MAGIC, 4, cfg.vocab_size, cfg.hidden_size, cfg.intermediate_size,
                            cfg.num_layers, cfg.num_heads, cfg.num_kv_heads, cfg.max_seq_len,
                            cfg.tensor_parallel, len(items), header, float(cfg.rope_theta),
                            float(cfg.norm_eps), cfg.sliding_window, flags, cfg.model_family,
                            cfg.num_local_experts, cfg.num_experts_per_tok, cfg.expert_intermediate_size))
        for e in entries:
            f.write(e)
        for name, nbytes, prod in items:
            blob = prod()
            if len(blob) != nbytes:
                raise ValueError(f"{name}: produced {len(blob)} bytes, expected {nbytes}")
            f.write(blob)


# ------------------------------------------------------------- quantisers
def quantize_int8_rowwise(w: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """tools/pack_ll2c.py:102-118: s = max(absmax/127, 1e-8), q = rint(clip(w/s))."""
    w = w.astype(np.float32)
    s = np.maximum(np.max(np.abs(w), axis=1) / 127.0, 1.0e-8).astype(np.float32)
    q = np.rint(np.clip(w / s[:, None], -127.0, 127.0)).astype(np.int8)
    return q, s


def pack_int4(q: np.ndarray) -> np.ndarray:
    """Two signed nibbles per byte, low nibble = even column (pack_ll2c.py:134-143)."""
    rows, cols = q.shape
    q = q.astype(np.int16)
    even = q[:, 0::2]
    odd = np.zeros_like(even)
    odd[:, : q[:, 1::2].shape[1]] = q[:, 1::2]
    return ((even & 0x0F) | ((odd & 0x0F) << 4)).astype(np.uint8)


def unpack_int4(packed: np.ndarray, cols: int) -> np.ndarray:
    """Inverse of pack_int4 by sign extension (independent of the oracle's
    nibble-compare formulation)."""
    p = packed.astype(np.uint8)
    lo = ((p << 4).astype(np.int8) >> 4)
    hi = (p.astype(np.int8) >> 4)
    out = np.empty((p.shape[0], p.shape[1] * 2), dtype=np.int8)
    out[:, 0::2] = lo
    out[:, 1::2] = hi
    return out[:, :cols]


def quantize_int4_rowwise(w: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """tools/pack_ll2c.py:121-146: s = max(absmax/7, 1e-8), q = rint(clip(w/s, -7, 7))."""
    w = w.astype(np.float32)
    s = np.maximum(np.max(np.abs(w), axis=1) / 7.0, 1.0e-8).astype(np.float32)
    q = np.rint(np.clip(w / s[:, None], -7.0, 7.0)).astype(np.int8)
    return pack_int4(q), s


def quantize_int4_g32(w: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """Group-32 extension: one fp16 scale per 32 columns, s = fp16(max(absmax/7, 1e-8)),
    q = rint(clip(w / s, -8, 7))."""
    rows, cols = w.shape
    assert cols % 32 == 0
    g = w.astype(np.float32).reshape(rows, cols // 32, 32)
    s = np.maximum(np.max(np.abs(g), axis=2) / 7.0, 1.0e-8).astype(np.float16)
    q = np.rint(np.clip(g / s.astype(np.float32)[:, :, None], -8.0, 7.0)).astype(np.int8)
    return pack_int4(q.reshape(rows, cols)), s


def dequant(fmt: str, w: np.ndarray, scales: Optional[np.ndarray], rows: int, cols: int) -> np.ndarray:
    """fp32 weights from a stored tensor (uint8 views accepted)."""
    if fmt == "f16":
        return w.view(np.float16).reshape(rows, cols).astype(np.float32)
    if fmt == "i8":
        s = scales.view(np.float32)
        s = s if s.size > 1 else np.full(rows, s[0], np.float32)
        return w.view(np.int8).reshape(rows, cols).astype(np.float32) * s[:, None]
    q = unpack_int4(w.view(np.uint8).reshape(rows, (cols + 1) // 2), cols).astype(np.float32)
    if fmt == "i4":
        s = scales.view(np.float32)
        s = s if s.size > 1 else np.full(rows, s[0], np.float32)
        return q * s[:, None]
    if fmt == "i4g32":
        s = scales.view(np.float16).reshape(rows, cols // 32).astype(np.float32)
        return q * np.repeat(s, 32, axis=1)
    raise ValueError(fmt)


# ------------------------------------------------------- synthetic models
@dataclasses.dataclass
class SynthSpec:
    cfg: Config
    attn_fmt: str = "f16"     # f16 | i8 | i4 | i4g32
    mlp_fmt: str = "f16"
    lm_fmt: str = "f16"
    seed: int = 0
    std: float = 0.02         # fp16 / quantise-from weights ~ N(0, std^2)
    gscale_std: float = 0.01  # group-32 random form: scales |N(0, gscale_std^2)|
    random_lowbit: bool = True  # i4g32: uniform nibbles + random scales
    norm_jitter: float = 0.0    # norm weights 1 + N(0, jitter^2)


def _linear_tensors(name: str, rows: int, cols: int, fmt: str, spec: SynthSpec, rng_for) -> List:
    out = []
    if fmt == "f16":
        out.append((name, rows * cols * 2, lambda: _normal_f16(rng_for(name), rows * cols, spec.std)))
        return out
    if fmt == "i4g32" and spec.random_lowbit:
        assert cols % 32 == 0
        out.append((name + ".int4", rows * cols // 2,
                    lambda: rng_for(name + ".int4").integers(0, 256, rows * cols // 2, dtype=np.uint8).tobytes()))
        out.append((name + ".gscale", rows * (cols // 32) * 2,
                    lambda: np.abs(rng_for(name + ".gscale").standard_normal(rows * (cols // 32), dtype=np.float32)
                                   * spec.gscale_std).astype(np.float16).tobytes()))
        return out
    # quantised from an fp16 N(0, std^2) matrix (the reference packer pipeline)
    cache: Dict[str, Tuple[np.ndarray, np.ndarray]] = {}

    def q():
        if "v" not in cache:
            w = np.frombuffer(_normal_f16(rng_for(name), rows * cols, spec.std), np.float16).reshape(rows, cols)
            if fmt == "i8":
                cache["v"] = quantize_int8_rowwise(w)
            elif fmt == "i4":
                cache["v"] = quantize_int4_rowwise(w)
            else:
                cache["v"] = quantize_int4_g32(w)
        return cache["v"]

    if fmt == "i8":
        out.append((name + ".int8", rows * cols, lambda: q()[0].tobytes()))
        out.append((name + ".scale", rows * 4, lambda: q()[1].tobytes()))
    elif fmt == "i4":
        out.append((name + ".int4", rows * ((cols + 1) // 2), lambda: q()[0].tobytes()))
        out.append((name + ".scale", rows * 4, lambda: q()[1].tobytes()))
    elif fmt == "i4g32":
        out.append((name + ".int4", rows * ((cols + 1) // 2), lambda: q()[0].tobytes()))
        out.append((name + ".gscale", rows * (cols // 32) * 2, lambda: q()[1].tobytes()))
    else:
        raise ValueError(fmt)
    return out


def _normal_f16(rng: np.random.Generator, n: int, std: float) -> bytes:
    return (rng.standard_normal(n, dtype=np.float32) * np.float32(std)).astype(np.float16).tobytes()


def synth_tensors(spec: SynthSpec) -> List:
    """(name, nbytes, producer) list for a random-init Llama-family model."""
    c = spec.cfg
    H, I, V = c.hidden_size, c.intermediate_size, c.vocab_size
    hd = c.head_dim
    qd, kvd = c.num_heads * hd, c.num_kv_heads * hd

    def rng_for(name: str) -> np.random.Generator:
        h = int.from_bytes(hashlib.sha256(name.encode()).digest()[:8], "little")
        return np.random.default_rng([spec.seed, h])

    def norm(name: str):
        def p():
            w = np.ones(H, np.float32)
            if spec.norm_jitter > 0:
                w += rng_for(name).standard_normal(H, dtype=np.float32) * np.float32(spec.norm_jitter)
            return w.astype(np.float16).tobytes()
        return (name, H * 2, p)

    t = [("tok_embeddings.weight", V * H * 2, lambda: _normal_f16(rng_for("tok_embeddings.weight"), V * H, spec.std))]
    for l in range(c.num_layers):
        p = f"layers.{l}."
        t.append(norm(p + "attention_norm.weight"))
        t.append(norm(p + "ffn_norm.weight"))
        t += _linear_tensors(p + "attention.wq", qd, H, spec.attn_fmt, spec, rng_for)
        t += _linear_tensors(p + "attention.wk", kvd, H, spec.attn_fmt, spec, rng_for)
        t += _linear_tensors(p + "attention.wv", kvd, H, spec.attn_fmt, spec, rng_for)
        t += _linear_tensors(p + "attention.wo", H, qd, spec.attn_fmt, spec, rng_for)
        if c.num_local_experts > 0:
            EI = c.expert_intermediate_size or I
            t += _linear_tensors(p + "feed_forward.router", c.num_local_experts, H, "f16", spec, rng_for)
            for e in range(c.num_local_experts):
                b = p + f"feed_forward.experts.{e}."
                t += _linear_tensors(b + "w1", EI, H, spec.mlp_fmt, spec, rng_for)
                t += _linear_tensors(b + "w2", H, EI, spec.mlp_fmt, spec, rng_for)
                t += _linear_tensors(b + "w3", EI, H, spec.mlp_fmt, spec, rng_for)
        else:
            t += _linear_tensors(p + "feed_forward.w1", I, H, spec.mlp_fmt, spec, rng_for)
            t += _linear_tensors(p + "feed_forward.w2", H, I, spec.mlp_fmt, spec, rng_for)
            t += _linear_tensors(p + "feed_forward.w3", I, H, spec.mlp_fmt, spec, rng_for)
    t.append(norm("norm.weight"))
    if not c.tie_word_embeddings:
        t += _linear_tensors("output.weight", V, H, spec.lm_fmt, spec, rng_for)
    return t


def write_synthetic(path: str, spec: SynthSpec) -> str:
    """Write a deterministic random-init model; returns its SHA-256."""
    write(path, spec.cfg, synth_tensors(spec))
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for blk in iter(lambda: f.read(1 << 24), b""):
            h.update(blk)
    return h.hexdigest()


# Named shapes from the benchmark configurations.
def tinyllama_config(**kw) -> Config:
    return Config(vocab_size=32000, hidden_size=2048, intermediate_size=5632, num_layers=22, num_heads=32,
                  num_kv_heads=4, max_seq_len=2048, rope_theta=10000.0, norm_eps=1e-5,
                  model_family=FAMILY["llama2"], **kw)


def llama2_7b_config(**kw) -> Config:
    base = dict(vocab_size=32000, hidden_size=4096, intermediate_size=11008, num_layers=32, num_heads=32,
                num_kv_heads=32, max_seq_len=4096, rope_theta=10000.0, norm_eps=1e-5,
                model_family=FAMILY["llama2"])
    base.update(kw)
    return Config(**base)


def mixtral_config(**kw) -> Config:
    base = dict(vocab_size=32000, hidden_size=4096, intermediate_size=14336, num_layers=32, num_heads=32,
                num_kv_heads=8, max_seq_len=4096, rope_theta=10000.0, norm_eps=1e-5,
                model_family=FAMILY["mixtral"], num_local_experts=8, num_experts_per_tok=2,
                expert_intermediate_size=14336)
    base.update(kw)
    return Config(**base)
