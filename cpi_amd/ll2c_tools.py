"""Command-line tools for the `.ll2c` weight container.

    python -m cpi_amd.ll2c_tools convert  --hf-dir DIR --output F.ll2c [--quant ...]
    python -m cpi_amd.ll2c_tools pack     --input-dir BINS --output F.ll2c [--emit-streaming-int4 ...]
    python -m cpi_amd.ll2c_tools quantize --input F.ll2c --output G.ll2c --mode int8|int4|int4-g32
    python -m cpi_amd.ll2c_tools validate F.ll2c

They cover the reference's conversion pipeline:
* `convert` = tools/convert_hf_to_bins.py + tools/pack_ll2c.py in one pass:
  HF config -> model family and header fields (convert_hf_to_bins.py:57-235),
  HF tensor names -> container names (:242-320), Q/K/V biases fused into
  `bqkv` (:383-396), tied embeddings copied to `output.weight` (:398-403),
  F16/BF16/F32 safetensors read as fp16 (:128-165).  Tensors are streamed one
  at a time into the file (no `.bin` intermediate).
* `pack` = tools/pack_ll2c.py:149-274 on a directory of `<name>.bin` fp16
  blobs plus `model_config.json`: same tensor order (sorted file names, each
  packed tensor followed by its low-bit copy), same header, same
  `--emit-streaming-int8/int4` and `--omit-fp16-layer-tensors` semantics.
* `quantize` = tools/quantize_ll2c_streaming.py: add low-bit copies of the
  linears of an existing file.
* `validate` = tools/validate_ll2c.py:23-340: header, table bounds, head
  topology and every layer tensor's byte size, for fp16 and packed forms.

Extension beyond the reference: `--quant int4-g32` writes `<base>.int4` with
`<base>.gscale` (fp16, one scale per 32 columns), and `--quant-scope all`
also quantises the attention projections (the resident engine serves every
projection in its stored format).  Quantisation formulas are those of
`cpi_amd.ll2c` (pack_ll2c.py:102-146 for the row-scale forms).
"""
from __future__ import annotations

import argparse
import json
import re
import struct
import sys
from pathlib import Path
from typing import Callable, Dict, List, Optional, Tuple

import numpy as np

from cpi_amd import ll2c

# ------------------------------------------------------------------ families
# model-family ids of the header (include/model/llama_config.hpp:17-25)
FAMILY_ID = {"unknown": 0, "llama2": 1, "llama3": 2, "mistral": 3, "phi3": 4, "qwen2": 5, "mixtral": 6}
DEFAULT_THETA = {"llama2": 10000.0, "llama3": 500000.0, "mistral": 10000.0, "mixtral": 10000.0,
                 "phi3": 10000.0, "qwen2": 1000000.0}


def detect_family(hf: dict) -> str:
    """Model family from HF `config.json` (convert_hf_to_bins.py:57-97)."""
    mt = str(hf.get("model_type", "")).lower()
    if mt in ("llama", "llama2"):
        big = int(hf.get("vocab_size", 32000)) > 100000 or float(hf.get("rope_theta", 10000.0)) > 100000
        return "llama3" if big else "llama2"
    if mt == "mixtral":
        return "mixtral"
    if mt == "mistral":
        return "mixtral" if int(hf.get("num_local_experts", 0) or 0) > 0 else "mistral"
    if mt in ("phi", "phi3", "phi-3", "phi-msft", "phimoe"):
        return "phi3"
    if mt == "qwen2":
        return "qwen2"
    for key, fam in (("qwen", "qwen2"), ("phi", "phi3"), ("mistral", "mistral"), ("mixtral", "mixtral")):
        if key in mt:
            return fam
    print(f"[warn] unknown model_type '{mt}', using llama2", file=sys.stderr)
    return "llama2"


def model_config(hf: dict, family: str) -> dict:
    """Header fields from HF `config.json` (convert_hf_to_bins.py:172-235)."""
    nh = int(hf["num_attention_heads"])
    experts = int(hf.get("num_local_experts", 0) or 0)
    per_tok = int(hf.get("num_experts_per_tok", 0) or 0)
    e_inter = int(hf.get("expert_intermediate_size", 0) or 0)
    if family == "mixtral" and experts <= 0:
        experts = 8
    if experts > 0:
        per_tok = per_tok if per_tok > 0 else 2
        e_inter = e_inter if e_inter > 0 else int(hf.get("intermediate_size", 0) or 0)
    kind = str(hf.get("norm_type", hf.get("normalization", ""))).lower()
    if "layernorm" in kind:
        layernorm = True
    elif "rmsnorm" in kind:
        layernorm = False
    else:
        layernorm = "layer_norm_eps" in hf and "rms_norm_eps" not in hf
    return {
        "model_family": family,
        "model_family_id": FAMILY_ID.get(family, 0),
        "vocab_size": int(hf["vocab_size"]),
        "hidden_size": int(hf["hidden_size"]),
        "intermediate_size": int(hf["intermediate_size"]),
        "num_layers": int(hf["num_hidden_layers"]),
        "num_heads": nh,
        "num_kv_heads": int(hf.get("num_key_value_heads", nh)),
        "max_seq_len": int(hf.get("max_position_embeddings", 4096)),
        "rope_theta": float(hf.get("rope_theta", DEFAULT_THETA.get(family, 10000.0))),
        "norm_eps": float(hf.get("rms_norm_eps", hf.get("layer_norm_eps", 1e-5))),
        "sliding_window": int(hf.get("sliding_window", 0) or 0),
        "tie_word_embeddings": bool(hf.get("tie_word_embeddings", False)),
        "has_qkv_bias": family == "qwen2" or bool(hf.get("attention_bias", False)),
        "use_layernorm": layernorm,
        "num_local_experts": experts,
        "num_experts_per_tok": per_tok,
        "expert_intermediate_size": e_inter,
    }


def config_from_dict(d: dict, tensor_parallel: int = 1) -> ll2c.Config:
    """`ll2c.Config` from a model_config dict; absent fields take
    pack_ll2c.py:43-74's defaults."""
    return ll2c.Config(
        vocab_size=int(d.get("vocab_size", 32000)), hidden_size=int(d.get("hidden_size", 4096)),
        intermediate_size=int(d.get("intermediate_size", 11008)), num_layers=int(d.get("num_layers", 32)),
        num_heads=int(d.get("num_heads", 32)), num_kv_heads=int(d.get("num_kv_heads", d.get("num_heads", 32))),
        max_seq_len=int(d.get("max_seq_len", 4096)), tensor_parallel=tensor_parallel,
        rope_theta=float(d.get("rope_theta", 0.0)), norm_eps=float(d.get("norm_eps", 1e-5)),
        sliding_window=int(d.get("sliding_window", 0)), tie_word_embeddings=bool(d.get("tie_word_embeddings", False)),
        has_qkv_bias=bool(d.get("has_qkv_bias", False)), use_layernorm=bool(d.get("use_layernorm", False)),
        model_family=int(d.get("model_family_id", 0)), num_local_experts=int(d.get("num_local_experts", 0) or 0),
        num_experts_per_tok=int(d.get("num_experts_per_tok", 0) or 0),
        expert_intermediate_size=int(d.get("expert_intermediate_size", 0) or 0))


def name_map(layers: int, experts: int, qkv_bias: bool) -> List[Tuple[str, str, bool]]:
    """(HF name, container name, required) in the converter's order
    (convert_hf_to_bins.py:242-320)."""
    out = [("model.embed_tokens.weight", "tok_embeddings.weight", True),
           ("model.norm.weight", "norm.weight", True),
           ("model.norm.bias", "norm.bias", False),
           ("lm_head.weight", "output.weight", False),
           ("lm_head.bias", "output.bias", False)]
    for i in range(layers):
        hp, p = f"model.layers.{i}.", f"layers.{i}."
        out += [(hp + "input_layernorm.weight", p + "attention_norm.weight", True),
                (hp + "input_layernorm.bias", p + "attention_norm.bias", False),
                (hp + "self_attn.q_proj.weight", p + "attention.wq", True),
                (hp + "self_attn.k_proj.weight", p + "attention.wk", True),
                (hp + "self_attn.v_proj.weight", p + "attention.wv", True),
                (hp + "self_attn.o_proj.weight", p + "attention.wo", True),
                (hp + "self_attn.o_proj.bias", p + "attention.bo", False),
                (hp + "post_attention_layernorm.weight", p + "ffn_norm.weight", True),
                (hp + "post_attention_layernorm.bias", p + "ffn_norm.bias", False)]
        if experts > 0:
            out.append((hp + "block_sparse_moe.gate.weight", p + "feed_forward.router", True))
            for e in range(experts):
                for w in ("w1", "w2", "w3"):
                    out.append((hp + f"block_sparse_moe.experts.{e}.{w}.weight",
                                p + f"feed_forward.experts.{e}.{w}", True))
        else:
            out += [(hp + "mlp.gate_proj.weight", p + "feed_forward.w1", True),
                    (hp + "mlp.down_proj.weight", p + "feed_forward.w2", True),
                    (hp + "mlp.up_proj.weight", p + "feed_forward.w3", True)]
        if qkv_bias:
            out += [(hp + "self_attn.q_proj.bias", p + "attention.bq", False),
                    (hp + "self_attn.k_proj.bias", p + "attention.bk", False),
                    (hp + "self_attn.v_proj.bias", p + "attention.bv", False)]
    return out


# --------------------------------------------------------------- safetensors
class SafeTensors:
    """Lazy reader over a single-file or sharded HF safetensors checkpoint."""

    def __init__(self, hf_dir: Path):
        self.dir = hf_dir
        index = hf_dir / "model.safetensors.index.json"
        if index.exists():
            self.where = dict(json.loads(index.read_text())["weight_map"])
        elif (hf_dir / "model.safetensors").exists():
            self.where = {k: "model.safetensors" for k in self._header(hf_dir / "model.safetensors")[0]
                          if k != "__metadata__"}
        else:
            raise FileNotFoundError(f"missing {index} and {hf_dir / 'model.safetensors'}")
        self._headers: Dict[str, Tuple[dict, int]] = {}

    @staticmethod
    def _header(path: Path) -> Tuple[dict, int]:
        with path.open("rb") as f:
            (n,) = struct.unpack("<Q", f.read(8))
            return json.loads(f.read(n).decode("utf-8")), 8 + n

    def meta(self, name: str) -> Tuple[Path, dict, int]:
        shard = self.where[name]
        if shard not in self._headers:
            self._headers[shard] = self._header(self.dir / shard)
        hdr, base = self._headers[shard]
        if name not in hdr:
            raise KeyError(f"tensor {name} not found in {shard}")
        return self.dir / shard, hdr[name], base

    def nbytes_f16(self, name: str) -> int:
        _, m, _ = self.meta(name)
        return 2 * int(np.prod(m.get("shape", [])) if m.get("shape") else 1)

    def shape(self, name: str) -> List[int]:
        return list(self.meta(name)[1].get("shape", []))

    def f16(self, name: str) -> np.ndarray:
        """The tensor as fp16 (BF16 widened to fp32 first, F32 rounded to
        nearest even), flattened."""
        path, m, base = self.meta(name)
        start, end = m["data_offsets"]
        raw = np.memmap(path, dtype=np.uint8, mode="r", offset=base + start, shape=(end - start,))
        dt = m.get("dtype")
        if dt == "F16":
            return np.array(raw.view(np.float16))
        if dt == "BF16":
            return (raw.view(np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32).astype(np.float16)
        if dt == "F32":
            return raw.view(np.float32).astype(np.float16)
        raise ValueError(f"tensor {name} dtype {dt}, expected F16/BF16/F32")


# ------------------------------------------------------------ quantisation
FFN_RE = re.compile(r"layers\.\d+\.feed_forward\.(experts\.\d+\.)?w[123]")
ATTN_RE = re.compile(r"layers\.\d+\.attention\.w[qkvo]")


def quantizable(name: str, scope: str) -> bool:
    """FFN weights (tools/pack_ll2c.py:77-82), plus the attention projections
    with scope 'all'."""
    return bool(FFN_RE.fullmatch(name)) or (scope == "all" and bool(ATTN_RE.fullmatch(name)))


def linear_shape(name: str, c: ll2c.Config) -> Tuple[int, int]:
    """[rows, cols] of a quantisable linear (pack_ll2c.py:85-99 for the FFN)."""
    H, I = c.hidden_size, c.intermediate_size
    EI = c.expert_intermediate_size if c.expert_intermediate_size > 0 else I
    hd = H // c.num_heads
    m = re.fullmatch(r"layers\.\d+\.feed_forward\.(experts\.\d+\.)?(w[123])", name)
    if m:
        inter = EI if m.group(1) else I
        return (H, inter) if m.group(2) == "w2" else (inter, H)
    m = re.fullmatch(r"layers\.\d+\.attention\.(w[qkvo])", name)
    if m:
        return {"wq": (c.num_heads * hd, H), "wk": (c.num_kv_heads * hd, H),
                "wv": (c.num_kv_heads * hd, H), "wo": (H, c.num_heads * hd)}[m.group(1)]
    raise ValueError(f"no linear shape for {name}")


def lowbit(mode: str, w16: np.ndarray, rows: int, cols: int) -> List[Tuple[str, bytes]]:
    """Low-bit copies of an fp16 matrix: [(suffix, bytes)]."""
    w = w16.reshape(rows, cols).astype(np.float32)
    if mode == "int8":
        q, s = ll2c.quantize_int8_rowwise(w)
        return [(".int8", q.tobytes()), (".scale", s.astype(np.float32).tobytes())]
    if mode == "int4":
        q, s = ll2c.quantize_int4_rowwise(w)
        return [(".int4", q.tobytes()), (".scale", s.astype(np.float32).tobytes())]
    if mode == "int4-g32":
        if cols % 32:
            raise ValueError(f"int4-g32 needs columns % 32 == 0, got {cols}")
        q, s = ll2c.quantize_int4_g32(w)
        return [(".int4", q.tobytes()), (".gscale", s.astype(np.float16).tobytes())]
    raise ValueError(mode)


def lowbit_sizes(mode: str, rows: int, cols: int) -> List[Tuple[str, int]]:
    if mode == "int8":
        return [(".int8", rows * cols), (".scale", 4 * rows)]
    if mode == "int4":
        return [(".int4", rows * ((cols + 1) // 2)), (".scale", 4 * rows)]
    return [(".int4", rows * ((cols + 1) // 2)), (".gscale", 2 * rows * (cols // 32))]


Producer = Tuple[str, int, Callable[[], bytes]]


def with_lowbit(items: List[Producer], c: ll2c.Config, mode: Optional[str], scope: str, omit: bool) -> List[Producer]:
    """Insert each quantisable tensor's low-bit copy right after it (and drop
    its fp16 form with `omit`).  The fp16 source of a copy is produced once
    more when the copy is written, so memory stays at one tensor."""
    out: List[Producer] = []
    for name, nbytes, prod in items:
        q = mode is not None and quantizable(name, scope)
        if not (q and omit):
            out.append((name, nbytes, prod))
        if q:
            rows, cols = linear_shape(name, c)
            if nbytes != 2 * rows * cols:
                raise ValueError(f"{name}: {nbytes} bytes, expected fp16 [{rows}, {cols}]")
            cache: Dict[str, List[Tuple[str, bytes]]] = {}

            def part(suffix, prod=prod, rows=rows, cols=cols, cache=cache):
                if "v" not in cache:
                    cache["v"] = lowbit(mode, np.frombuffer(prod(), np.float16), rows, cols)
                blob = dict(cache["v"])[suffix]
                if suffix != lowbit_sizes(mode, rows, cols)[0][0]:
                    cache.clear()  # scales are written last: free the copy
                return blob

            for suffix, size in lowbit_sizes(mode, rows, cols):
                out.append((name + suffix, size, lambda s=suffix, part=part: part(s)))
    return out


# ---------------------------------------------------------------- commands
def cmd_convert(a) -> int:
    src = Path(a.hf_dir)
    hf = json.loads((src / "config.json").read_text())
    family = a.family or detect_family(hf)
    if family == "phimoe":
        family = "phi3"
    mc = model_config(hf, family)
    c = config_from_dict(mc, a.tensor_parallel)
    st = SafeTensors(src)
    items: List[Producer] = []
    names = set()
    for hf_name, name, required in name_map(c.num_layers, c.num_local_experts, c.has_qkv_bias):
        if hf_name not in st.where:
            if required:
                raise KeyError(f"missing required tensor: {hf_name}")
            continue
        items.append((name, st.nbytes_f16(hf_name), lambda n=hf_name: st.f16(n).tobytes()))
        names.add(name)
    if c.has_qkv_bias:
        fused = []
        for i in range(c.num_layers):
            parts = [f"layers.{i}.attention.b{x}" for x in "qkv"]
            if all(p in names for p in parts):
                prods = {n: (b, p) for n, b, p in items if n in parts}
                total = sum(prods[p][0] for p in parts)
                fused.append((f"layers.{i}.attention.bqkv", total,
                              lambda ps=[prods[p][1] for p in parts]: b"".join(f() for f in ps)))
                items = [it for it in items if it[0] not in parts]
            elif any(p in names for p in parts):
                print(f"[warn] layer {i}: incomplete Q/K/V biases, left out", file=sys.stderr)
                items = [it for it in items if it[0] not in parts]
        items += fused
    if c.tie_word_embeddings and "output.weight" not in names:
        emb = next(it for it in items if it[0] == "tok_embeddings.weight")
        items.append(("output.weight", emb[1], emb[2]))
    mode = None if a.quant == "none" else a.quant
    items = with_lowbit(items, c, mode, a.quant_scope, a.omit_fp16)
    ll2c.write(a.output, c, items)
    print(f"[convert] family={family} layers={c.num_layers} hidden={c.hidden_size} experts={c.num_local_experts} "
          f"tensors={len(items)} quant={a.quant}/{a.quant_scope} -> {a.output}")
    return 0


def cmd_pack(a) -> int:
    if a.omit_fp16_layer_tensors and not (a.emit_streaming_int8 or a.emit_streaming_int4):
        raise ValueError("--omit-fp16-layer-tensors requires --emit-streaming-int8 or --emit-streaming-int4")
    if a.emit_streaming_int8 and a.emit_streaming_int4:
        raise ValueError("choose only one low-bit packing mode: --emit-streaming-int8 or --emit-streaming-int4")
    src = Path(a.input_dir)
    cfg_path = src / "model_config.json"
    d = json.loads(cfg_path.read_text()) if cfg_path.exists() else {}
    for k in ("vocab_size", "hidden_size", "intermediate_size", "num_layers", "num_heads", "num_kv_heads",
              "max_seq_len"):
        v = getattr(a, k)
        if v is not None:
            d[k] = v
    c = config_from_dict(d, a.tensor_parallel)
    bins = sorted(src.glob("*.bin"))
    if not bins:
        raise RuntimeError(f"no .bin files found in {src}")
    items = [(p.stem, p.stat().st_size, lambda p=p: p.read_bytes()) for p in bins]
    mode = "int8" if a.emit_streaming_int8 else ("int4" if a.emit_streaming_int4 else None)
    items = with_lowbit(items, c, mode, "ffn", a.omit_fp16_layer_tensors)
    ll2c.write(a.output, c, items)
    print(f"Packed tensors: {len(items)}")
    print(f"Wrote {a.output} ({Path(a.output).stat().st_size} bytes)")
    return 0


def cmd_quantize(a) -> int:
    """Existing entries keep their order; the new low-bit pairs are appended
    (tools/quantize_ll2c_streaming.py:340-360).  Low-bit copies already in the
    file for a re-quantised linear are replaced."""
    if Path(a.output).resolve() == Path(a.input).resolve():
        raise ValueError("output must differ from input")
    r = ll2c.Reader(a.input)
    c = r.config
    bases = [n for n in r.entries if quantizable(n, a.scope)]
    stale = {n + s for n in bases for s in (".int8", ".int4", ".scale", ".gscale")}
    keep: List[Producer] = [(n, nb, lambda n=n: r.tensor(n).tobytes())
                            for n, (_, nb) in r.entries.items()
                            if n not in stale and not (a.omit_fp16 and n in bases)]
    fresh = with_lowbit([(n, r.entries[n][1], lambda n=n: r.tensor(n).tobytes()) for n in bases],
                        c, a.mode, a.scope, omit=True)
    ll2c.write(a.output, c, keep + fresh)
    print(f"[quantize] {len(bases)} linears -> {a.mode} ({a.scope}); {len(keep) + len(fresh)} tensors -> {a.output}")
    return 0


class ValidationError(ValueError):
    pass


def validate(path: str) -> dict:
    """tools/validate_ll2c.py:23-340 for the dense/MoE tensors, plus the
    group-32 form (`.int4` + `.gscale`).  Raises ValidationError."""
    data = Path(path).read_bytes()
    if len(data) < 48:
        raise ValidationError("file too small for header")
    try:
        r = ll2c.Reader(path)
    except ValueError as e:
        raise ValidationError(str(e))
    c = r.config
    if data[:8] != ll2c.MAGIC:
        raise ValidationError("bad magic, expected LL2CUDA")
    H, I, L, nh, nkv, V = c.hidden_size, c.intermediate_size, c.num_layers, c.num_heads, c.num_kv_heads, c.vocab_size
    if H <= 0 or I <= 0 or L <= 0 or nh <= 0 or nkv <= 0:
        raise ValidationError("invalid model config in header")
    if nh % nkv:
        raise ValidationError("invalid head topology")
    ent = {}
    for name, (off, nbytes) in r.entries.items():
        if off < 0 or nbytes < 0 or off + nbytes > len(data):
            raise ValidationError(f"tensor {name} has invalid offset/size")
        ent[name] = nbytes

    def expect(name, got, want):
        if got != want:
            raise ValidationError(f"{name}: expected {want} bytes, got {got} bytes")

    def rows_of(name, cols):
        for suffix, per_row in (("", 2 * cols), (".int8", cols), (".int4", (cols + 1) // 2)):
            if name + suffix in ent:
                if per_row == 0 or ent[name + suffix] % per_row:
                    raise ValidationError(f"{name + suffix}: invalid matrix byte size")
                return ent[name + suffix] // per_row
        raise ValidationError(f"missing tensor: {name} (or packed int8/int4 alternative)")

    q_rows = rows_of("layers.0.attention.wq", H)
    if q_rows <= 0 or q_rows % nh:
        raise ValidationError("invalid q_proj shape: rows must be positive and divisible by heads")
    hd = q_rows // nh
    kv_rows = nkv * hd
    if rows_of("layers.0.attention.wk", H) != kv_rows or rows_of("layers.0.attention.wv", H) != kv_rows:
        raise ValidationError("invalid k_proj/v_proj shape for inferred attention head_dim")
    packed = 0

    def req(name, want):
        if name not in ent:
            raise ValidationError(f"missing tensor: {name}")
        expect(name, ent[name], want)

    def opt(name, want):
        if name in ent:
            expect(name, ent[name], want)

    def linear(name, rows, cols):
        nonlocal packed
        if name in ent:
            expect(name, ent[name], 2 * rows * cols)
            return
        if name + ".int8" in ent and name + ".scale" in ent:
            expect(name + ".int8", ent[name + ".int8"], rows * cols)
        elif name + ".int4" in ent and name + ".scale" in ent:
            expect(name + ".int4", ent[name + ".int4"], rows * ((cols + 1) // 2))
        elif name + ".int4" in ent and name + ".gscale" in ent:
            expect(name + ".int4", ent[name + ".int4"], rows * ((cols + 1) // 2))
            if cols % 32:
                raise ValidationError(f"{name}.gscale: columns {cols} not a multiple of 32")
            expect(name + ".gscale", ent[name + ".gscale"], 2 * rows * (cols // 32))
            packed += 1
            return
        else:
            raise ValidationError(f"missing tensor: {name} (or packed int8/int4 alternative)")
        if ent[name + ".scale"] not in (4, 4 * rows):
            raise ValidationError(f"{name}.scale: expected 4 or {4 * rows} bytes, got {ent[name + '.scale']} bytes")
        packed += 1

    req("tok_embeddings.weight", 2 * V * H)
    req("norm.weight", 2 * H)
    opt("norm.bias", 2 * H)
    opt("output.weight", 2 * V * H)
    opt("output.bias", 2 * V)
    EI = c.expert_intermediate_size if c.expert_intermediate_size > 0 else I
    for l in range(L):
        p = f"layers.{l}."
        req(p + "attention_norm.weight", 2 * H)
        opt(p + "attention_norm.bias", 2 * H)
        linear(p + "attention.wq", q_rows, H)
        linear(p + "attention.wk", kv_rows, H)
        linear(p + "attention.wv", kv_rows, H)
        linear(p + "attention.wo", H, q_rows)
        opt(p + "attention.bqkv", 2 * (q_rows + 2 * kv_rows))
        opt(p + "attention.bo", 2 * H)
        req(p + "ffn_norm.weight", 2 * H)
        opt(p + "ffn_norm.bias", 2 * H)
        dense = [p + f"feed_forward.w{k}" for k in (1, 2, 3)]
        has_dense = any(n + s in ent for n in dense for s in ("", ".int8", ".int4"))
        pat = re.compile(rf"^{re.escape(p)}feed_forward\.experts\.(\d+)\.w[123](\.int8|\.int4)?$")
        experts = {int(m.group(1)) for m in (pat.match(n) for n in ent) if m}
        has_moe = bool(experts) or p + "feed_forward.router" in ent
        if has_dense and has_moe:
            raise ValidationError(f"layer {l}: mixed dense and MoE feed-forward tensors are not allowed")
        if has_moe:
            E = c.num_local_experts if c.num_local_experts > 0 else len(experts)
            linear(p + "feed_forward.router", E, H)
            if not experts:
                raise ValidationError(f"layer {l}: MoE layer has no experts")
            if c.num_local_experts > 0 and len(experts) != c.num_local_experts:
                raise ValidationError(f"layer {l}: expected {c.num_local_experts} experts from header, "
                                      f"found {len(experts)}")
            for e in sorted(experts):
                b = p + f"feed_forward.experts.{e}."
                linear(b + "w1", EI, H)
                linear(b + "w2", H, EI)
                linear(b + "w3", EI, H)
        else:
            linear(dense[0], I, H)
            linear(dense[1], H, I)
            linear(dense[2], I, H)
    r.close()
    return {"version": r.version, "vocab": V, "hidden": H, "inter": I, "expert_inter": c.expert_intermediate_size,
            "layers": L, "heads": nh, "q_hidden": q_rows, "kv_heads": nkv, "max_seq": c.max_seq_len,
            "tensors": len(ent), "packed_layer_tensors": packed, "experts": c.num_local_experts,
            "topk": c.num_experts_per_tok}


def cmd_validate(a) -> int:
    try:
        info = validate(a.model)
    except ValidationError as e:
        print(f"error: {e}", file=sys.stderr)
        return 1
    print("OK")
    print(" ".join(f"{k}={v}" for k, v in info.items()))
    return 0


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(prog="python -m cpi_amd.ll2c_tools", description=__doc__.split("\n")[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    q_choices = ["none", "int8", "int4", "int4-g32"]

    c = sub.add_parser("convert", help="HF safetensors directory -> .ll2c")
    c.add_argument("--hf-dir", required=True)
    c.add_argument("--output", required=True)
    c.add_argument("--family", default=None, help="llama2|llama3|mistral|mixtral|phi3|phimoe|qwen2")
    c.add_argument("--quant", choices=q_choices, default="none")
    c.add_argument("--quant-scope", choices=["ffn", "all"], default="ffn",
                   help="ffn: the feed-forward weights (the reference's packing); all: also wq/wk/wv/wo")
    c.add_argument("--omit-fp16", action="store_true", help="drop the fp16 form of quantised tensors")
    c.add_argument("--tensor-parallel", type=int, default=1)
    c.set_defaults(fn=cmd_convert)

    p = sub.add_parser("pack", help="directory of <name>.bin fp16 blobs + model_config.json -> .ll2c")
    p.add_argument("--input-dir", required=True)
    p.add_argument("--output", required=True)
    for k in ("vocab-size", "hidden-size", "intermediate-size", "num-layers", "num-heads", "num-kv-heads",
              "max-seq-len"):
        p.add_argument(f"--{k}", type=int)
    p.add_argument("--tensor-parallel", type=int, default=1)
    p.add_argument("--emit-streaming-int8", action="store_true")
    p.add_argument("--emit-streaming-int4", action="store_true")
    p.add_argument("--omit-fp16-layer-tensors", action="store_true")
    p.set_defaults(fn=cmd_pack)

    q = sub.add_parser("quantize", help="add low-bit copies of the linears of an .ll2c file")
    q.add_argument("--input", required=True)
    q.add_argument("--output", required=True)
    q.add_argument("--mode", choices=q_choices[1:], required=True)
    q.add_argument("--scope", choices=["ffn", "all"], default="ffn")
    q.add_argument("--omit-fp16", action="store_true")
    q.set_defaults(fn=cmd_quantize)

    v = sub.add_parser("validate", help="check an .ll2c file's header and tensor sizes")
    v.add_argument("model")
    v.set_defaults(fn=cmd_validate)

    a = ap.parse_args(argv)
    return a.fn(a)


if __name__ == "__main__":
    sys.exit(main())
