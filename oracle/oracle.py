"""ctypes binding of the CPU oracle (oracle/libshs_oracle.so).

Test infrastructure only: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker, never as the product path.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libshs_oracle.so"

F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0 = 0, 1, 2, 3, 6, 7, 8
TYPE_NAMES = {"Q4_0": Q4_0, "Q4_1": Q4_1, "Q5_0": Q5_0, "Q5_1": Q5_1, "Q8_0": Q8_0, "F32": F32}
TYPE_SIZE = {Q4_0: 18, Q4_1: 20, Q5_0: 22, Q5_1: 24, Q8_0: 34, F32: 128}


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = C.CDLL(str(LIB_PATH))
        _declare(_lib)
    return _lib


P = C.c_void_p


class Config(C.Structure):
    _fields_ = [
        ("n_layer", C.c_int), ("hidden", C.c_int), ("n_head", C.c_int), ("n_kv_head", C.c_int),
        ("head_dim", C.c_int), ("ffn", C.c_int), ("vocab", C.c_int),
        ("eps", C.c_float), ("rope_theta", C.c_float), ("rope_dim", C.c_int),
        ("rope_scale", C.c_float), ("rope_orig_ctx", C.c_int),
        ("yarn_beta_fast", C.c_float), ("yarn_beta_slow", C.c_float), ("yarn_ext_factor", C.c_float),
        ("yarn_mscale", C.c_float), ("yarn_mscale_all_dim", C.c_float), ("rope_attn_factor", C.c_float),
        ("attn_temperature", C.c_float), ("yarn_active", C.c_int),
    ]


class Layer(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("type_q", "type_k", "type_v", "type_o", "type_gate", "type_up", "type_down")] + \
               [(n, P) for n in ("q", "k", "v", "o", "gate", "up", "down")] + \
               [("attn_norm", P), ("ffn_norm", P)]


class Model(C.Structure):
    _fields_ = [("cfg", Config), ("embd_type", C.c_int), ("token_embd", P), ("output_norm", P), ("layers", P)]


class KV(C.Structure):
    _fields_ = [("k", P), ("v", P), ("cap", C.c_int), ("len", C.c_int)]


CAPTURE_FN = C.CFUNCTYPE(None, C.c_char_p, C.POINTER(C.c_float), C.c_int, C.c_int, C.c_void_p)


def _declare(L: C.CDLL) -> None:
    L.ora_half_to_float.argtypes = [C.c_uint16]
    L.ora_half_to_float.restype = C.c_float
    L.ora_float_to_half.argtypes = [C.c_float]
    L.ora_float_to_half.restype = C.c_uint16
    L.ora_dequantize.argtypes = [C.c_int, P, P, C.c_int64]
    L.ora_quantize.argtypes = [C.c_int, P, P, C.c_int64]
    L.ora_quantize_activations.argtypes = [P, C.c_int64, P, P, P]
    L.ora_quantize_activations_q8.argtypes = [P, C.c_int64, P, P, P]
    L.ora_block_sums.argtypes = [C.c_int, P, C.c_int, C.c_int, P, P, C.c_int, P]
    L.ora_matmul_q.argtypes = [C.c_int, P, C.c_int, C.c_int, P, P, P, C.c_int, P, C.c_int, P, C.c_int]
    L.ora_matmul.argtypes = [C.c_int, P, C.c_int, C.c_int, P, C.c_int, P, C.c_int, P, C.c_int, C.c_int]
    L.ora_gather_rows.argtypes = [C.c_int, P, C.c_int, C.c_int, P, C.c_int, P]
    L.ora_rmsnorm.argtypes = [P, P, C.c_float, C.c_int, P]
    L.ora_swiglu.argtypes = [P, P, P, C.c_int64]
    L.ora_softmax.argtypes = [P, C.c_int]
    L.ora_dot4.argtypes = [P, P, P, P, P, C.c_int, P]
    L.ora_add_scaled4.argtypes = [P, P, P, P, P, P, C.c_int]
    L.ora_rope_freqs.argtypes = [C.POINTER(Config), P, P]
    L.ora_rope_apply.argtypes = [P, C.c_float, C.c_int, P, C.c_int, C.c_int, C.c_int]
    L.ora_forward.argtypes = [C.POINTER(Model), C.POINTER(KV), P, C.c_int, C.c_int, P, C.c_int, P,
                              CAPTURE_FN, P, C.c_int]
    L.ora_score.argtypes = [P, C.c_int, C.c_int, P, P, P]
    L.ora_expf.argtypes = [C.c_float]
    L.ora_expf.restype = C.c_float
    L.ora_expf_n.argtypes = [P, C.c_int64, P]
    L.ora_layer_forward.argtypes = [C.POINTER(Model), C.POINTER(KV), C.c_int, P, C.c_int, P, C.c_int]


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ------------------------------------------------------------------ wrappers

def half_to_float(bits: int) -> float:
    return lib().ora_half_to_float(bits)


def dequantize(qtype: int, raw: bytes | np.ndarray, n: int) -> np.ndarray:
    src = np.frombuffer(bytes(raw), dtype=np.uint8) if not isinstance(raw, np.ndarray) else _c(raw, np.uint8)
    out = np.empty(n, np.float32)
    if lib().ora_dequantize(qtype, _p(src), _p(out), n):
        raise ValueError("dequantize failed")
    return out


def quantize(qtype: int, x: np.ndarray) -> np.ndarray:
    x = _c(x, np.float32).reshape(-1)
    out = np.empty(x.size // 32 * TYPE_SIZE[qtype], np.uint8)
    if lib().ora_quantize(qtype, _p(x), _p(out), x.size):
        raise ValueError("quantize failed")
    return out


def quantize_activations(x: np.ndarray, semantics: int = 0):
    x = _c(x, np.float32).reshape(-1)
    q = np.empty(x.size, np.int8)
    d = np.empty(x.size // 32, np.float32)
    s = np.empty(x.size // 32, np.int32)
    fn = lib().ora_quantize_activations if semantics == 0 else lib().ora_quantize_activations_q8
    fn(_p(x), x.size, _p(q), _p(d), _p(s))
    return q, d, s


def block_sums(qtype: int, w: np.ndarray, rows: int, cols: int, q: np.ndarray, tokens: int,
               s: np.ndarray | None = None) -> np.ndarray:
    """s: the quantizer's int32 block sums; when omitted, the sums of the codes (the same
    for every block whose codes did not saturate)."""
    w = _c(w, np.uint8)
    q = _c(q, np.int8)
    if s is None:
        s = q.reshape(tokens, cols // 32, 32).astype(np.int64).sum(axis=2)
    s = _c(np.asarray(s).astype(np.int64).astype(np.int32), np.int32)
    out = np.empty((tokens, rows, cols // 32), np.int32)
    if lib().ora_block_sums(qtype, _p(w), rows, cols, _p(q), _p(s), tokens, _p(out)):
        raise ValueError("block_sums failed")
    return out


def matmul(qtype: int, w: np.ndarray, rows: int, cols: int, x: np.ndarray, tokens: int,
           row_ids=None, semantics: int = 0, threads: int = 0) -> np.ndarray:
    w = _c(w, np.uint8)
    x = _c(x, np.float32)
    ids = None if row_ids is None else _c(row_ids, np.int32)
    n_out = rows if ids is None else ids.size
    y = np.empty((tokens, n_out), np.float32)
    rc = lib().ora_matmul(qtype, _p(w), rows, cols, _p(x), tokens, _p(ids), 0 if ids is None else ids.size,
                          _p(y), semantics, threads)
    if rc == -2:
        raise IndexError("row id outside the matrix")
    if rc:
        raise ValueError(f"matmul failed ({rc})")
    return y


def matmul_q(qtype, w, rows, cols, q, d, s, tokens, row_ids=None, threads=0):
    w = _c(w, np.uint8)
    q, d, s = _c(q, np.int8), _c(d, np.float32), _c(s, np.int32)
    ids = None if row_ids is None else _c(row_ids, np.int32)
    n_out = rows if ids is None else ids.size
    y = np.empty((tokens, n_out), np.float32)
    if lib().ora_matmul_q(qtype, _p(w), rows, cols, _p(q), _p(d), _p(s), tokens, _p(ids),
                          0 if ids is None else ids.size, _p(y), threads):
        raise ValueError("matmul_q failed")
    return y


def gather_rows(qtype, table, rows, cols, ids):
    table = _c(table, np.uint8)
    ids = _c(ids, np.int32)
    out = np.empty((ids.size, cols), np.float32)
    rc = lib().ora_gather_rows(qtype, _p(table), rows, cols, _p(ids), ids.size, _p(out))
    if rc == -2:
        raise IndexError("token id outside the table")
    return out


def rmsnorm(x, w, eps):
    x, w = _c(x, np.float32), _c(w, np.float32)
    y = np.empty_like(x)
    lib().ora_rmsnorm(_p(x), _p(w), eps, x.size, _p(y))
    return y


def swiglu(g, u):
    g, u = _c(g, np.float32).copy(), _c(u, np.float32).copy()
    out = np.empty_like(g)
    lib().ora_swiglu(_p(g), _p(u), _p(out), g.size)
    return out


def expf(x):
    """ora_expf elementwise."""
    x = _c(x, np.float32).reshape(-1)
    y = np.empty_like(x)
    lib().ora_expf_n(_p(x), x.size, _p(y))
    return y


def softmax(x):
    x = _c(x, np.float32).copy()
    lib().ora_softmax(_p(x), x.size)
    return x


def dot4(shared, a):
    shared = _c(shared, np.float32)
    a = [_c(v, np.float32) for v in a]
    r = np.empty(4, np.float32)
    lib().ora_dot4(_p(shared), _p(a[0]), _p(a[1]), _p(a[2]), _p(a[3]), shared.size, _p(r))
    return r


def add_scaled4(src, dst, w):
    src = _c(src, np.float32)
    dst = [_c(v, np.float32).copy() for v in dst]
    w = _c(w, np.float32)
    lib().ora_add_scaled4(_p(src), _p(dst[0]), _p(dst[1]), _p(dst[2]), _p(dst[3]), _p(w), src.size)
    return dst


def make_config(**kw) -> Config:
    c = Config()
    defaults = dict(n_layer=26, hidden=3072, n_head=32, n_kv_head=8, head_dim=128, ffn=9216, vocab=131072,
                    eps=1e-5, rope_theta=1e6, rope_dim=128, rope_scale=1.0, rope_orig_ctx=0,
                    yarn_beta_fast=32.0, yarn_beta_slow=1.0, yarn_ext_factor=1.0, yarn_mscale=0.0,
                    yarn_mscale_all_dim=0.0, rope_attn_factor=1.0, attn_temperature=0.0, yarn_active=0)
    defaults.update(kw)
    for k, v in defaults.items():
        setattr(c, k, v)
    return c


def rope_freqs(cfg: Config):
    f = np.empty(cfg.rope_dim // 2, np.float32)
    ms = np.empty(1, np.float32)
    lib().ora_rope_freqs(C.byref(cfg), _p(f), _p(ms))
    return f, float(ms[0])


def rope_apply(freqs, mscale, rope_dim, data, heads, head_dim, position):
    data = _c(data, np.float32).copy()
    freqs = _c(freqs, np.float32)
    lib().ora_rope_apply(_p(freqs), mscale, rope_dim, _p(data), heads, head_dim, position)
    return data


def score(logits, n_yes, n_no):
    logits = _c(logits, np.float32)
    out = np.empty(3, np.float32)
    lib().ora_score(_p(logits), n_yes, n_no, _p(out[0:]), _p(out[1:]), _p(out[2:]))
    return float(out[0]), float(out[1]), float(out[2])


class OracleModel:
    """Holds a synthetic model's tensors (the same bytes the GPU consumes) for ora_forward."""

    def __init__(self, cfg: Config, tensors: dict, types: dict, cap: int = 512):
        self.cfg = cfg
        self.tensors = {k: np.ascontiguousarray(v) for k, v in tensors.items()}
        self.types = types
        L = cfg.n_layer
        self._layers = (Layer * L)()
        for l in range(L):
            lay = self._layers[l]
            for short, name in (("q", "attn_q"), ("k", "attn_k"), ("v", "attn_v"), ("o", "attn_output"),
                                ("gate", "ffn_gate"), ("up", "ffn_up"), ("down", "ffn_down")):
                key = f"blk.{l}.{name}.weight"
                setattr(lay, "type_" + short, types[key])
                setattr(lay, short, self.tensors[key].ctypes.data)
            lay.attn_norm = self.tensors[f"blk.{l}.attn_norm.weight"].ctypes.data
            lay.ffn_norm = self.tensors[f"blk.{l}.ffn_norm.weight"].ctypes.data
        self.model = Model()
        self.model.cfg = cfg
        self.model.embd_type = types["token_embd.weight"]
        self.model.token_embd = self.tensors["token_embd.weight"].ctypes.data
        self.model.output_norm = self.tensors["output_norm.weight"].ctypes.data
        self.model.layers = C.cast(self._layers, C.c_void_p)
        self.cap = 0
        self.kv = KV()
        self._ensure(cap)

    def _ensure(self, cap):
        if cap <= self.cap:
            return
        c = self.cfg
        shape = (c.n_layer, c.n_kv_head, cap, c.head_dim)
        k = np.zeros(shape, np.float32)
        v = np.zeros(shape, np.float32)
        if self.cap:
            k[:, :, : self.cap] = self._k
            v[:, :, : self.cap] = self._v
        self._k, self._v, self.cap = k, v, cap
        self.kv.k, self.kv.v, self.kv.cap = k.ctypes.data, v.ctypes.data, cap

    @property
    def kv_len(self):
        return self.kv.len

    def reset(self):
        self.kv.len = 0

    def snapshot(self, length=None):
        """KvCache.Snapshot layout (KvCache.cs:94-112): keys [layer][head][pos][dim], then values."""
        n = self.kv.len if length is None else length
        return np.concatenate([self._k[:, :, :n].reshape(-1), self._v[:, :, :n].reshape(-1)])

    def restore(self, snap, length):
        c = self.cfg
        self._ensure(length)
        per = c.n_layer * c.n_kv_head * length * c.head_dim
        self._k[:, :, :length] = snap[:per].reshape(c.n_layer, c.n_kv_head, length, c.head_dim)
        self._v[:, :, :length] = snap[per:].reshape(c.n_layer, c.n_kv_head, length, c.head_dim)
        self.kv.len = length

    def layer_forward(self, layer, x, threads=0):
        """One decoder layer on hidden state x [n, hidden] at positions 0..n-1."""
        x = _c(x, np.float32).reshape(-1, self.cfg.hidden)
        self._ensure(x.shape[0])
        y = np.empty_like(x)
        if lib().ora_layer_forward(C.byref(self.model), C.byref(self.kv), layer, _p(x), x.shape[0], _p(y), threads):
            raise ValueError("ora_layer_forward failed")
        return y

    def forward(self, tokens, head_mode=1, vocab_ids=None, capture=None, threads=0):
        tokens = _c(tokens, np.int32)
        self._ensure(self.kv.len + tokens.size)
        ids = None if vocab_ids is None else _c(vocab_ids, np.int32)
        if head_mode == 2:
            logits = np.empty(self.cfg.vocab, np.float32)
        elif head_mode == 1:
            logits = np.empty(ids.size, np.float32)
        else:
            logits = np.empty(1, np.float32)
        cb = CAPTURE_FN(0)
        if capture is not None:
            def _cb(name, data, rows, cols, user):
                arr = np.ctypeslib.as_array(data, shape=(rows * cols,)).copy().reshape(rows, cols)
                capture(name.decode(), arr)
            cb = CAPTURE_FN(_cb)
        rc = lib().ora_forward(C.byref(self.model), C.byref(self.kv), _p(tokens), tokens.size, head_mode,
                               _p(ids), 0 if ids is None else ids.size, _p(logits), cb, None, threads)
        if rc:
            raise ValueError(f"ora_forward failed ({rc})")
        return logits
