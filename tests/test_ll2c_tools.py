"""The `.ll2c` tools (cpi_amd/ll2c_tools.py): HF checkpoint conversion,
bin-directory packing, quantisation and validation (tools/convert_hf_to_bins.py,
tools/pack_ll2c.py, tools/quantize_ll2c_streaming.py, tools/validate_ll2c.py).

Checkpoints are written here as safetensors files in F16, BF16 and F32, single
and sharded.  Converted tensors are compared bit for bit against fp16 values
computed independently from the source dtype (BF16 -> fp32 by a 16-bit
shift, then numpy's round-to-nearest-even fp32 -> fp16); quantised tensors
against the bounds their scales imply; whole models through the C oracle
engine against the float64 decoder of tests/numpy_ref.py."""
import json
import struct

import numpy as np
import pytest

import oracle
from cpi_amd import ll2c, ll2c_tools as T
from tests.numpy_ref import RefModel

HF_LLAMA = dict(model_type="llama", vocab_size=96, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64, rms_norm_eps=1e-5,
                rope_theta=10000.0)


def _bf16_bits(x):
    """fp32 -> bf16 bit patterns (round to nearest even)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def write_safetensors(path, tensors):
    """{name: (dtype, np array)} -> safetensors file (our own writer)."""
    header, blobs, off = {}, [], 0
    for name, (dt, a) in tensors.items():
        raw = {"F16": lambda a: a.astype(np.float16).tobytes(), "F32": lambda a: a.astype(np.float32).tobytes(),
               "BF16": lambda a: _bf16_bits(a).tobytes()}[dt](a)
        header[name] = {"dtype": dt, "shape": list(a.shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    h = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + b"".join(blobs))


def expected_f16(dt, a):
    if dt == "BF16":
        return (_bf16_bits(a).astype(np.uint32) << 16).view(np.float32).astype(np.float16)
    return a.astype(np.float32).astype(np.float16) if dt == "F32" else a.astype(np.float16)


def hf_tensors(cfg, rng, dtype="F16", experts=0, qkv_bias=False, lm_head=True):
    H, I, V, L = cfg["hidden_size"], cfg["intermediate_size"], cfg["vocab_size"], cfg["num_hidden_layers"]
    nh, nkv = cfg["num_attention_heads"], cfg["num_key_value_heads"]
    hd = H // nh
    t = {}
    n = lambda *s: (rng.standard_normal(s) * 0.08).astype(np.float32)
    t["model.embed_tokens.weight"] = (dtype, n(V, H))
    t["model.norm.weight"] = (dtype, 1 + n(H))
    if lm_head:
        t["lm_head.weight"] = (dtype, n(V, H))
    for i in range(L):
        p = f"model.layers.{i}."
        t[p + "input_layernorm.weight"] = (dtype, 1 + n(H))
        t[p + "post_attention_layernorm.weight"] = (dtype, 1 + n(H))
        t[p + "self_attn.q_proj.weight"] = (dtype, n(nh * hd, H))
        t[p + "self_attn.k_proj.weight"] = (dtype, n(nkv * hd, H))
        t[p + "self_attn.v_proj.weight"] = (dtype, n(nkv * hd, H))
        t[p + "self_attn.o_proj.weight"] = (dtype, n(H, nh * hd))
        if qkv_bias:
            t[p + "self_attn.q_proj.bias"] = (dtype, n(nh * hd))
            t[p + "self_attn.k_proj.bias"] = (dtype, n(nkv * hd))
            t[p + "self_attn.v_proj.bias"] = (dtype, n(nkv * hd))
        if experts:
            t[p + "block_sparse_moe.gate.weight"] = (dtype, n(experts, H))
            for e in range(experts):
                q = p + f"block_sparse_moe.experts.{e}."
                t[q + "w1.weight"] = (dtype, n(I, H))
                t[q + "w2.weight"] = (dtype, n(H, I))
                t[q + "w3.weight"] = (dtype, n(I, H))
        else:
            t[p + "mlp.gate_proj.weight"] = (dtype, n(I, H))
            t[p + "mlp.down_proj.weight"] = (dtype, n(H, I))
            t[p + "mlp.up_proj.weight"] = (dtype, n(I, H))
    return t


def make_hf(d, cfg, tensors, shards=1):
    d.mkdir(parents=True, exist_ok=True)
    (d / "config.json").write_text(json.dumps(cfg))
    names = list(tensors)
    if shards == 1:
        write_safetensors(d / "model.safetensors", tensors)
        return
    wmap = {}
    for s in range(shards):
        part = {k: tensors[k] for k in names[s::shards]}
        fn = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
        write_safetensors(d / fn, part)
        wmap.update({k: fn for k in part})
    (d / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wmap}))


def f16_of(r, name):
    return r.tensor(name).view(np.float16)


@pytest.mark.parametrize("dtype,shards", [("F16", 1), ("BF16", 2), ("F32", 3)])
def test_convert_dense_tensors_bit_exact(tmp_path, dtype, shards):
    rng = np.random.default_rng(1)
    t = hf_tensors(HF_LLAMA, rng, dtype)
    make_hf(tmp_path / "hf", HF_LLAMA, t, shards)
    out = str(tmp_path / "m.ll2c")
    assert T.main(["convert", "--hf-dir", str(tmp_path / "hf"), "--output", out]) == 0
    info = T.validate(out)
    assert info["q_hidden"] == 64 and info["kv_heads"] == 2 and info["packed_layer_tensors"] == 0
    r = ll2c.Reader(out)
    c = r.config
    assert (c.vocab_size, c.hidden_size, c.intermediate_size, c.num_layers, c.num_heads, c.num_kv_heads) == \
        (96, 64, 128, 2, 4, 2)
    assert c.model_family == 1 and c.rope_theta == 10000.0 and abs(c.norm_eps - 1e-5) < 1e-12
    for hf_name, name, _ in T.name_map(2, 0, False):
        if hf_name not in t:
            assert not r.has(name)
            continue
        dt, a = t[hf_name]
        assert np.array_equal(f16_of(r, name).view(np.uint16), expected_f16(dt, a).ravel().view(np.uint16)), name


def test_convert_int4_g32_runs_in_the_oracle(tmp_path):
    """All projections to int4-g32 (fp16 forms dropped): validator accepts it,
    every group obeys |w - q s| <= s/2, and the C oracle engine decodes the
    file exactly as the float64 decoder does."""
    rng = np.random.default_rng(2)
    t = hf_tensors(HF_LLAMA, rng, "F16")
    make_hf(tmp_path / "hf", HF_LLAMA, t)
    out = str(tmp_path / "q.ll2c")
    assert T.main(["convert", "--hf-dir", str(tmp_path / "hf"), "--output", out, "--quant", "int4-g32",
                   "--quant-scope", "all", "--omit-fp16"]) == 0
    assert T.validate(out)["packed_layer_tensors"] == 2 * 7
    r = ll2c.Reader(out)
    for hf_name, name, _ in T.name_map(2, 0, False):
        if not T.quantizable(name, "all"):
            continue
        assert not r.has(name) and r.has(name + ".int4") and r.has(name + ".gscale")
        w = t[hf_name][1].astype(np.float16).astype(np.float32)
        rows, cols = w.shape
        s = r.tensor(name + ".gscale").view(np.float16).astype(np.float32).reshape(rows, cols // 32)
        q = ll2c.unpack_int4(r.tensor(name + ".int4").reshape(rows, cols // 2), cols).astype(np.float32)
        assert q.min() >= -8 and q.max() <= 7
        err = np.abs(w - q * np.repeat(s, 32, axis=1))
        assert np.all(err <= np.repeat(s, 32, axis=1) * (0.5 + 2e-3) + 1e-7), name
    prompt = np.array([3, 17, 5, 90, 41])
    ids, lg = oracle.Engine(out, 64).generate(prompt, 6, eos=-1, logit_steps=6)
    rids, rlg = RefModel(out).generate(prompt, 6)
    np.testing.assert_allclose(lg, rlg, atol=2e-5 * max(np.abs(rlg).max(), 1))
    assert (ids == rids).all()


def test_convert_mixtral_qwen2_tied(tmp_path):
    rng = np.random.default_rng(3)
    mix = dict(HF_LLAMA, model_type="mixtral", num_local_experts=4, num_experts_per_tok=2, sliding_window=8)
    t = hf_tensors(mix, rng, "BF16", experts=4)
    make_hf(tmp_path / "mix", mix, t, 2)
    out = str(tmp_path / "mix.ll2c")
    assert T.main(["convert", "--hf-dir", str(tmp_path / "mix"), "--output", out, "--quant", "int4"]) == 0
    info = T.validate(out)
    # fp16 forms are present, so (as in validate_ll2c.py) the packed copies are not counted
    assert info["experts"] == 4 and info["topk"] == 2 and info["packed_layer_tensors"] == 0
    r = ll2c.Reader(out)
    assert r.config.model_family == 6 and r.config.sliding_window == 8 and r.config.expert_intermediate_size == 128
    # fp16 form kept next to the int4 copy; row scales s = absmax / 7
    name = "layers.1.feed_forward.experts.3.w2"
    w = f16_of(r, name).astype(np.float32).reshape(64, 128)
    s = r.tensor(name + ".scale").view(np.float32)
    np.testing.assert_array_equal(s, np.maximum(np.abs(w).max(axis=1) / np.float32(7), np.float32(1e-8)))
    q = ll2c.unpack_int4(r.tensor(name + ".int4").reshape(64, 64), 128)
    assert np.abs(q).max() == 7 and np.all(np.abs(q).max(axis=1) == 7)
    # the engine's own MoE file runs too
    prompt = np.array([1, 2, 3])
    ids, lg = oracle.Engine(out, 32).generate(prompt, 4, eos=-1, logit_steps=4)
    rids, rlg = RefModel(out).generate(prompt, 4)
    np.testing.assert_allclose(lg, rlg, atol=2e-5 * max(np.abs(rlg).max(), 1))

    qw = dict(HF_LLAMA, model_type="qwen2", tie_word_embeddings=True)
    t = hf_tensors(qw, rng, "F32", qkv_bias=True, lm_head=False)
    make_hf(tmp_path / "qw", qw, t)
    out = str(tmp_path / "qw.ll2c")
    assert T.main(["convert", "--hf-dir", str(tmp_path / "qw"), "--output", out]) == 0
    T.validate(out)
    r = ll2c.Reader(out)
    assert r.config.has_qkv_bias and r.config.tie_word_embeddings and r.config.model_family == 5
    assert r.config.rope_theta == 10000.0  # config value wins over the family default
    for i in range(2):
        p = f"model.layers.{i}.self_attn."
        want = np.concatenate([expected_f16("F32", t[p + x + "_proj.bias"][1]) for x in "qkv"])
        assert np.array_equal(f16_of(r, f"layers.{i}.attention.bqkv"), want)
        assert not r.has(f"layers.{i}.attention.bq")
    assert np.array_equal(f16_of(r, "output.weight"), f16_of(r, "tok_embeddings.weight"))


def test_family_detection_and_defaults():
    assert T.detect_family({"model_type": "llama", "vocab_size": 128256}) == "llama3"
    assert T.detect_family({"model_type": "llama", "rope_theta": 500000.0}) == "llama3"
    assert T.detect_family({"model_type": "llama"}) == "llama2"
    assert T.detect_family({"model_type": "mistral", "num_local_experts": 8}) == "mixtral"
    assert T.detect_family({"model_type": "phimoe"}) == "phi3"
    assert T.detect_family({"model_type": "qwen2_moe"}) == "qwen2"
    base = dict(num_attention_heads=8, vocab_size=10, hidden_size=8, intermediate_size=16, num_hidden_layers=1)
    mc = T.model_config(dict(base), "llama3")
    assert mc["rope_theta"] == 500000.0 and mc["num_kv_heads"] == 8 and mc["max_seq_len"] == 4096
    mc = T.model_config(dict(base), "mixtral")
    assert (mc["num_local_experts"], mc["num_experts_per_tok"], mc["expert_intermediate_size"]) == (8, 2, 16)
    assert T.model_config(dict(base, layer_norm_eps=1e-6), "phi3")["use_layernorm"]
    assert not T.model_config(dict(base, layer_norm_eps=1e-6, rms_norm_eps=1e-6), "phi3")["use_layernorm"]


def test_pack_bins_order_header_and_int8(tmp_path):
    """pack_ll2c semantics: sorted .bin names; each FFN weight followed by its
    low-bit copy; header from model_config.json with CLI overrides."""
    rng = np.random.default_rng(4)
    d = tmp_path / "bins"
    d.mkdir()
    H, I = 32, 64
    shapes = {"tok_embeddings.weight": (10, H), "norm.weight": (H,), "layers.0.attention_norm.weight": (H,),
              "layers.0.ffn_norm.weight": (H,), "layers.0.attention.wq": (H, H), "layers.0.attention.wk": (H, H),
              "layers.0.attention.wv": (H, H), "layers.0.attention.wo": (H, H),
              "layers.0.feed_forward.w1": (I, H), "layers.0.feed_forward.w2": (H, I),
              "layers.0.feed_forward.w3": (I, H)}
    vals = {}
    for n, s in shapes.items():
        vals[n] = (rng.standard_normal(s) * 0.1).astype(np.float16)
        (d / f"{n}.bin").write_bytes(vals[n].tobytes())
    (d / "model_config.json").write_text(json.dumps(dict(vocab_size=10, hidden_size=H, intermediate_size=I,
                                                         num_layers=1, num_heads=4, rope_theta=0.0)))
    out = str(tmp_path / "p.ll2c")
    assert T.main(["pack", "--input-dir", str(d), "--output", out, "--emit-streaming-int8",
                   "--max-seq-len", "128"]) == 0
    r = ll2c.Reader(out)
    names = list(r.entries)
    want = []
    for n in sorted(shapes):
        want.append(n)
        if "feed_forward" in n:
            want += [n + ".int8", n + ".scale"]
    assert names == want
    assert r.config.max_seq_len == 128 and r.config.num_kv_heads == 4 and r.config.tensor_parallel == 1
    offs = [r.entries[n][0] for n in names]
    assert offs[0] == struct.calcsize(ll2c.HEADER_V4) + len(names) * 80  # table right after the header
    assert all(offs[i + 1] == offs[i] + r.entries[names[i]][1] for i in range(len(names) - 1))
    w = vals["layers.0.feed_forward.w2"].astype(np.float32)
    q = r.tensor("layers.0.feed_forward.w2.int8").view(np.int8).reshape(H, I).astype(np.float32)
    s = r.tensor("layers.0.feed_forward.w2.scale").view(np.float32)
    assert np.all(np.abs(q).max(axis=1) == 127)
    assert np.all(np.abs(w - q * s[:, None]) <= s[:, None] * 0.5 * (1 + 1e-5))
    T.validate(out)
    with pytest.raises(ValueError):
        T.main(["pack", "--input-dir", str(d), "--output", out, "--omit-fp16-layer-tensors"])


def test_quantize_appends_and_replaces(tmp_path):
    cfg = ll2c.Config(vocab_size=64, hidden_size=64, intermediate_size=96, num_layers=1, num_heads=4,
                      num_kv_heads=4, max_seq_len=32)
    src = str(tmp_path / "f.ll2c")
    ll2c.write_synthetic(src, ll2c.SynthSpec(cfg, attn_fmt="f16", mlp_fmt="i8", seed=1))
    out = str(tmp_path / "g.ll2c")
    before = list(ll2c.Reader(src).entries)
    assert T.main(["quantize", "--input", src, "--output", out, "--mode", "int4", "--scope", "all"]) == 0
    after = list(ll2c.Reader(out).entries)
    kept = [n for n in before if not n.endswith((".int8", ".int4", ".scale", ".gscale"))
            or n.rsplit(".", 1)[0] not in before]
    assert after[:len(kept)] == kept
    assert all(n.endswith((".int4", ".scale")) for n in after[len(kept):])
    assert len(after) - len(kept) == 2 * 4  # wq wk wv wo (w1..w3 are stored only as int8 in the source)
    T.validate(out)


def test_validate_rejects(tmp_path, capsys):
    cfg = ll2c.Config(vocab_size=64, hidden_size=64, intermediate_size=96, num_layers=1, num_heads=4,
                      num_kv_heads=2, max_seq_len=32)
    good = str(tmp_path / "ok.ll2c")
    ll2c.write_synthetic(good, ll2c.SynthSpec(cfg, attn_fmt="i4g32", mlp_fmt="i4g32", seed=1))
    assert T.main(["validate", good]) == 0
    assert capsys.readouterr().out.startswith("OK")
    data = open(good, "rb").read()
    bad = tmp_path / "bad.ll2c"
    bad.write_bytes(data[: len(data) - 10])
    with pytest.raises(T.ValidationError, match="invalid offset/size"):
        T.validate(str(bad))
    assert T.main(["validate", str(bad)]) == 1
    r = ll2c.Reader(good)
    items = [(n, nb, lambda n=n: r.tensor(n).tobytes()) for n, (_, nb) in r.entries.items()
             if n != "layers.0.feed_forward.w2.gscale"]
    miss = str(tmp_path / "miss.ll2c")
    ll2c.write(miss, cfg, items)
    with pytest.raises(T.ValidationError, match="feed_forward.w2"):
        T.validate(miss)
    wrong = dict((n, (nb, p)) for n, nb, p in [(n, nb, lambda n=n: r.tensor(n).tobytes())
                                              for n, (_, nb) in r.entries.items()])
    nb, _ = wrong["layers.0.attention.wo.gscale"]
    wrong["layers.0.attention.wo.gscale"] = (nb - 2, lambda: b"\x00" * (nb - 2))
    bad2 = str(tmp_path / "wrong.ll2c")
    ll2c.write(bad2, cfg, [(n, v[0], v[1]) for n, v in wrong.items()])
    with pytest.raises(T.ValidationError, match="attention.wo.gscale"):
        T.validate(bad2)
    topo = ll2c.Config(**{**cfg.__dict__, "num_kv_heads": 3})
    bad3 = str(tmp_path / "topo.ll2c")
    ll2c.write(bad3, topo, [(n, nb, lambda n=n: r.tensor(n).tobytes()) for n, (_, nb) in r.entries.items()])
    with pytest.raises(T.ValidationError):
        T.validate(bad3)
