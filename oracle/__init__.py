"""CPU oracle (TEST INFRASTRUCTURE ONLY): a C restatement of kurulav1/cpi's
reference CPU decode path (src/engine/cpu_engine.cpp).  Loaded only by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg, as the checker —
never by the product path.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(_HERE, "liboracle.so")
_lib = None

_f = ctypes.c_float
_i = ctypes.c_int
_p = ctypes.c_void_p


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        L = ctypes.CDLL(LIB)
        L.oracle_fp16_to_fp32.restype = _f
        L.oracle_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        L.oracle_int4_nibble.restype = _i
        L.oracle_int4_nibble.argtypes = [ctypes.c_uint8, _i]
        L.oracle_gemv.argtypes = [_i, _p, _p, ctypes.c_long, _i, _i, _p, _p]
        L.oracle_rmsnorm.argtypes = [_p, _p, _p, _f, _i, _p, _i]
        L.oracle_rope_tables.argtypes = [_i, _i, _f, _p, _p]
        L.oracle_rope.argtypes = [_p, _p, _i, _i, _i, _i, _p, _p]
        L.oracle_attention.argtypes = [_p, _p, _p, _i, _i, _i, _i, _i, _p, _p]
        L.oracle_silu.restype = _f
        L.oracle_silu.argtypes = [_f]
        L.oracle_router_topk.argtypes = [_p, _i, _i, _p, _p]
        L.oracle_argmax.restype = _i
        L.oracle_argmax.argtypes = [_p, _i]
        L.oracle_sample.restype = _i
        L.oracle_sample.argtypes = [_p, _i, _f, _i, _f, _f, _i, _p, _i, _f]
        L.oracle_engine_open.restype = _p
        L.oracle_engine_open.argtypes = [ctypes.c_char_p, _i, _f]
        L.oracle_engine_free.argtypes = [_p]
        L.oracle_engine_dims.argtypes = [_p, _p]
        L.oracle_engine_forward.restype = _i
        L.oracle_engine_forward.argtypes = [_p, _i, _i, _p]
        L.oracle_engine_generate.restype = _i
        L.oracle_engine_generate.argtypes = [_p, _p, _i, _i, _i, _p, _p, _i]
        L.oracle_num_threads.restype = _i
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(_p)


FMT = {"f16": 0, "i8": 1, "i4": 2, "i4g32": 3, "f32": 4}


def gemv(fmt: str, w: np.ndarray, scales, R: int, K: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.zeros(R, np.float32)
    w = np.ascontiguousarray(w)
    if scales is None:
        sp, sc = None, 0
    else:
        scales = np.ascontiguousarray(scales)
        sp, sc = _ptr(scales), scales.size
    lib().oracle_gemv(FMT[fmt], _ptr(w), sp, sc, R, K, _ptr(x), _ptr(y))
    return y


def rmsnorm(x, w_f16, eps, bias=None, layernorm=False):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w_f16, np.float16)
    out = np.zeros_like(x)
    b = None if bias is None else np.ascontiguousarray(bias, np.float16)
    lib().oracle_rmsnorm(_ptr(x), _ptr(w), None if b is None else _ptr(b), eps, int(layernorm), _ptr(out), x.size)
    return out


def rope_tables(max_ctx, hd, theta):
    c = np.zeros((max_ctx, hd // 2), np.float32)
    s = np.zeros_like(c)
    lib().oracle_rope_tables(max_ctx, hd, theta, _ptr(c), _ptr(s))
    return c, s


def rope(q, k, pos, nh, nkv, hd, cos_t, sin_t):
    q = np.array(q, np.float32)
    k = np.array(k, np.float32)
    lib().oracle_rope(_ptr(q), _ptr(k), pos, nh, nkv, hd, _ptr(np.ascontiguousarray(cos_t)),
                      _ptr(np.ascontiguousarray(sin_t)))
    return q, k


def attention(q, kc, vc, seq, nh, nkv, hd, window=0):
    q = np.ascontiguousarray(q, np.float32)
    kc = np.ascontiguousarray(kc, np.float32)
    vc = np.ascontiguousarray(vc, np.float32)
    out = np.zeros(nh * hd, np.float32)
    scores = np.zeros(nh * max(seq, 1), np.float32)
    lib().oracle_attention(_ptr(q), _ptr(kc), _ptr(vc), seq, window, nh, nkv, hd, _ptr(out), _ptr(scores))
    return out


def router_topk(logits, top_k):
    logits = np.ascontiguousarray(logits, np.float32)
    idx = np.zeros(top_k, np.int32)
    prob = np.zeros(top_k, np.float32)
    lib().oracle_router_topk(_ptr(logits), logits.size, top_k, _ptr(idx), _ptr(prob))
    return idx, prob


def sample(logits, temperature, top_k=0, top_p=1.0, rep_penalty=1.0, ngram=0, history=(), r=0.5):
    """The resident engine's sampler (llama_engine_sampling_utils.cpp:10-189)
    for one uniform draw r in [0, 1)."""
    lg = np.array(logits, np.float32)
    h = np.ascontiguousarray(np.asarray(history, np.int32))
    return lib().oracle_sample(_ptr(lg), lg.size, temperature, top_k, top_p, rep_penalty, ngram,
                               _ptr(h) if h.size else None, int(h.size), float(r))


def argmax(x):
    x = np.ascontiguousarray(x, np.float32)
    return lib().oracle_argmax(_ptr(x), x.size)


class Engine:
    """Reference-CPU-path restatement over an .ll2c file."""

    def __init__(self, path: str, max_ctx: int, theta_override: float = 0.0):
        self.h = lib().oracle_engine_open(path.encode(), max_ctx, theta_override)
        if not self.h:
            raise RuntimeError(f"oracle could not open {path}")
        d = np.zeros(10, np.int32)
        lib().oracle_engine_dims(self.h, _ptr(d))
        self.vocab, self.hidden, self.inter, self.layers, self.heads, self.kv_heads, self.head_dim, \
            self.max_ctx, self.experts, self.experts_per_tok = (int(v) for v in d)

    def forward(self, token: int, pos: int) -> np.ndarray:
        out = np.zeros(self.vocab, np.float32)
        if lib().oracle_engine_forward(self.h, token, pos, _ptr(out)) != 0:
            raise RuntimeError("oracle forward failed")
        return out

    def generate(self, prompt, max_new: int, eos: int = -1, logit_steps: int = 0):
        p = np.ascontiguousarray(prompt, np.int32)
        ids = np.zeros(max_new, np.int32)
        lg = np.zeros((max(logit_steps, 1), self.vocab), np.float32)
        n = lib().oracle_engine_generate(self.h, _ptr(p), p.size, max_new, eos, _ptr(ids), _ptr(lg), logit_steps)
        if n < 0:
            raise RuntimeError("oracle generate failed")
        return ids[:n], lg[:logit_steps]

    def close(self):
        if self.h:
            lib().oracle_engine_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
