"""Host side of the Shieldstral prefill path over libshieldstral_hip's C ABI.

Mirrors llm-shield's public surface for this path with the same names, argument
meaning and error behaviour (paths are in the llm-shield repository):

* ShieldstralModerator / ModerationResult  (src/LlmShield.Shieldstral/ShieldstralModerator.cs)
* MinistralModel, KvCache                  (Model/MinistralModel.cs, Model/KvCache.cs)
* SystemPromptCache ("SHKV" v1 files)     (SystemPromptCache.cs)
* QuantMatMul over a WeightMatrix          (Numerics/QuantMatMul.cs)

Tokenization and chat-template rendering stay with the caller (they are host string
work); every entry point here takes token ids. All arithmetic runs in the HIP
library: there is no CPU fallback, and importing this module without the built
library raises.
"""
from __future__ import annotations

import ctypes as C
import hashlib
import io
import os
import struct
import threading
from dataclasses import dataclass, field
from pathlib import Path
from typing import Callable, Iterable, Optional, Sequence

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libshieldstral_hip.so"

F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0 = 0, 1, 2, 3, 6, 7, 8
TYPE_IDS = {"F32": F32, "F16": F16, "Q4_0": Q4_0, "Q4_1": Q4_1, "Q5_0": Q5_0, "Q5_1": Q5_1, "Q8_0": Q8_0}
TYPE_SIZE = {Q4_0: 18, Q4_1: 20, Q5_0: 22, Q5_1: 24, Q8_0: 34}


# ----------------------------------------------------------------- errors

class ShieldstralError(Exception):
    """Base of the errors the C ABI reports."""


class ArgumentError(ShieldstralError, ValueError):
    """ArgumentException."""


class ArgumentOutOfRangeError(ShieldstralError, IndexError):
    """ArgumentOutOfRangeException (token id ≥ vocab, row id outside the matrix)."""


class InvalidDataError(ShieldstralError, ValueError):
    """InvalidDataException (shapes that disagree with the hyperparameters)."""


class TensorNotFoundError(ShieldstralError, KeyError):
    """KeyNotFoundException (a tensor the model needs is absent)."""


class NotSupportedError(ShieldstralError, NotImplementedError):
    """NotSupportedException (a weight type without an integer kernel)."""


class ModelIOError(ShieldstralError, OSError):
    """IOException (unreadable or truncated file)."""


class OperationCanceledError(ShieldstralError):
    """OperationCanceledException."""


class DeviceError(ShieldstralError, RuntimeError):
    """HIP failure, or no gfx950 device."""


_ERRORS = {1: ArgumentError, 2: ArgumentOutOfRangeError, 3: InvalidDataError, 4: TensorNotFoundError,
           5: NotSupportedError, 6: ModelIOError, 7: OperationCanceledError, 8: DeviceError}


# ---------------------------------------------------------------- binding

class shs_config(C.Structure):
    _fields_ = [
        ("n_layer", C.c_int32), ("hidden", C.c_int32), ("n_head", C.c_int32), ("n_kv_head", C.c_int32),
        ("head_dim", C.c_int32), ("ffn", C.c_int32), ("vocab", C.c_int32),
        ("rms_eps", C.c_float), ("rope_theta", C.c_float), ("rope_dim", C.c_int32),
        ("rope_scale", C.c_float), ("rope_orig_ctx", C.c_int32),
        ("yarn_beta_fast", C.c_float), ("yarn_beta_slow", C.c_float), ("yarn_ext_factor", C.c_float),
        ("yarn_mscale", C.c_float), ("yarn_mscale_all_dim", C.c_float), ("rope_attn_factor", C.c_float),
        ("attn_temperature", C.c_float), ("yarn_active", C.c_int32), ("architecture", C.c_char * 32),
    ]


class shs_tensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("type", C.c_int32), ("ne0", C.c_int64), ("ne1", C.c_int64), ("data", C.c_void_p)]


CAPTURE_FN = C.CFUNCTYPE(None, C.c_char_p, C.POINTER(C.c_float), C.c_int32, C.c_int32, C.c_void_p)

#: Every symbol include/shieldstral_hip.h declares.
EXPORTS = (
    "shs_last_error", "shs_open_tensors", "shs_open", "shs_read_config", "shs_open_synthetic", "shs_tensor_download",
    "shs_close",
    "shs_get_config", "shs_kv_reset", "shs_kv_length", "shs_kv_capacity", "shs_kv_snapshot", "shs_kv_restore",
    "shs_forward", "shs_forward_batch", "shs_set_capture", "shs_layer_forward", "shs_matrix_create",
    "shs_matrix_free", "shs_matmul", "shs_matmul_rows", "shs_matmul_block_sums", "shs_matmul_device",
    "shs_matmul_device_noalloc",
    "shs_profile_enable", "shs_profile_read", "shs_profile_reset", "shs_synchronize",
    "shs_debug_expf",
)

_lib = None
_lib_lock = threading.Lock()


def load_library(path: Optional[os.PathLike] = None) -> C.CDLL:
    """Loads libshieldstral_hip.so (built in-tree by __graft_entry__.build())."""
    global _lib
    with _lib_lock:
        if _lib is None:
            p = Path(path) if path else LIB_PATH
            if not p.exists():
                raise ImportError(f"{p} is missing: build it first (python -c 'import __graft_entry__ as g; g.build()')")
            lib = C.CDLL(str(p))
            _declare(lib)
            _lib = lib
    return _lib


def _declare(L: C.CDLL) -> None:
    P, I32, I64 = C.c_void_p, C.c_int32, C.c_int64
    PP = C.POINTER(C.c_void_p)
    L.shs_last_error.restype = C.c_char_p
    L.shs_last_error.argtypes = []
    sigs = {
        "shs_open_tensors": [C.POINTER(shs_config), C.POINTER(shs_tensor), I32, I32, I32, PP],
        "shs_open": [C.c_char_p, I32, I32, PP],
        "shs_read_config": [C.c_char_p, C.POINTER(shs_config)],
        "shs_open_synthetic": [C.POINTER(shs_config), I32, I32, C.c_uint64, I32, I32, PP],
        "shs_tensor_download": [P, C.c_char_p, P, C.c_size_t],
        "shs_get_config": [P, C.POINTER(shs_config)],
        "shs_kv_reset": [P],
        "shs_kv_length": [P, C.POINTER(I32)],
        "shs_kv_capacity": [P, C.POINTER(I32)],
        "shs_kv_snapshot": [P, I32, P, C.c_size_t],
        "shs_kv_restore": [P, P, C.c_size_t, I32],
        "shs_forward": [P, P, I32, I32, P, I32, P, P],
        "shs_forward_batch": [P, P, P, I32, P, I32, P],
        "shs_set_capture": [P, CAPTURE_FN, P],
        "shs_layer_forward": [P, I32, P, I32, P],
        "shs_matrix_create": [I32, I32, I32, P, I32, PP],
        "shs_matmul": [P, P, I32, P, I32],
        "shs_matmul_rows": [P, P, I32, P, I32, P],
        "shs_matmul_block_sums": [P, P, I32, P],
        "shs_matmul_device": [P, P, I32, P],
        "shs_matmul_device_noalloc": [P, P, I32, P],
        "shs_profile_enable": [P, I32],
        "shs_profile_read": [P, C.c_char_p, C.POINTER(I64), C.POINTER(C.c_double), C.POINTER(C.c_double)],
        "shs_profile_reset": [P],
        "shs_synchronize": [P],
        "shs_debug_expf": [P, I32, P, I32],
    }
    for name, args in sigs.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = C.c_int
    L.shs_close.argtypes = [P]
    L.shs_close.restype = None
    L.shs_matrix_free.argtypes = [P]
    L.shs_matrix_free.restype = None


def _check(status: int) -> None:
    if status != 0:
        msg = _lib.shs_last_error().decode(errors="replace")
        raise _ERRORS.get(status, ShieldstralError)(msg)


def _ptr(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data


def _arr(a, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


# ------------------------------------------------------------------ config

@dataclass
class ModelConfig:
    """ModelConfig (Model/ModelConfig.cs:12-60)."""
    layer_count: int = 26
    hidden_size: int = 3072
    head_count: int = 32
    kv_head_count: int = 8
    head_dim: int = 128
    feed_forward_size: int = 9216
    vocab_size: int = 131072
    rms_norm_eps: float = 1e-5
    rope_freq_base: float = 1e6
    rope_dim: int = 128
    rope_scale_factor: float = 1.0
    rope_original_context_length: int = 0
    yarn_beta_fast: float = 32.0
    yarn_beta_slow: float = 1.0
    yarn_ext_factor: float = 1.0
    yarn_mscale: float = 0.0
    yarn_mscale_all_dim: float = 0.0
    rope_attn_factor: float = 1.0
    attention_temperature_scale: float = 0.0
    yarn_active: bool = False
    architecture: str = "mistral3"

    @property
    def group_size(self) -> int:
        return self.head_count // self.kv_head_count

    @property
    def q_dim(self) -> int:
        return self.head_count * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.kv_head_count * self.head_dim

    def to_c(self) -> shs_config:
        c = shs_config()
        c.n_layer, c.hidden, c.n_head, c.n_kv_head = self.layer_count, self.hidden_size, self.head_count, self.kv_head_count
        c.head_dim, c.ffn, c.vocab = self.head_dim, self.feed_forward_size, self.vocab_size
        c.rms_eps, c.rope_theta, c.rope_dim = self.rms_norm_eps, self.rope_freq_base, self.rope_dim
        c.rope_scale, c.rope_orig_ctx = self.rope_scale_factor, self.rope_original_context_length
        c.yarn_beta_fast, c.yarn_beta_slow, c.yarn_ext_factor = self.yarn_beta_fast, self.yarn_beta_slow, self.yarn_ext_factor
        c.yarn_mscale, c.yarn_mscale_all_dim = self.yarn_mscale, self.yarn_mscale_all_dim
        c.rope_attn_factor, c.attn_temperature = self.rope_attn_factor, self.attention_temperature_scale
        c.yarn_active = int(self.yarn_active)
        c.architecture = self.architecture.encode()[:31]
        return c

    @classmethod
    def from_c(cls, c: shs_config) -> "ModelConfig":
        return cls(c.n_layer, c.hidden, c.n_head, c.n_kv_head, c.head_dim, c.ffn, c.vocab, c.rms_eps, c.rope_theta,
                   c.rope_dim, c.rope_scale, c.rope_orig_ctx, c.yarn_beta_fast, c.yarn_beta_slow, c.yarn_ext_factor,
                   c.yarn_mscale, c.yarn_mscale_all_dim, c.rope_attn_factor, c.attn_temperature, bool(c.yarn_active),
                   c.architecture.decode() or "mistral3")

    @classmethod
    def from_gguf(cls, gguf_path) -> "ModelConfig":
        """ModelConfig.FromGguf (ModelConfig.cs:62-112): the header alone, no device."""
        lib = load_library()
        c = shs_config()
        _check(lib.shs_read_config(str(gguf_path).encode(), C.byref(c)))
        return cls.from_c(c)

    def tensor_shapes(self, weight_type: int, embd_type: int):
        """GGUF tensor table (MinistralModel.cs:74-96): name → (type, ne0, ne1)."""
        t = {"token_embd.weight": (embd_type, self.hidden_size, self.vocab_size),
             "output_norm.weight": (F32, self.hidden_size, 1)}
        for l in range(self.layer_count):
            p = f"blk.{l}."
            t[p + "attn_norm.weight"] = (F32, self.hidden_size, 1)
            t[p + "attn_q.weight"] = (weight_type, self.hidden_size, self.q_dim)
            t[p + "attn_k.weight"] = (weight_type, self.hidden_size, self.kv_dim)
            t[p + "attn_v.weight"] = (weight_type, self.hidden_size, self.kv_dim)
            t[p + "attn_output.weight"] = (weight_type, self.q_dim, self.hidden_size)
            t[p + "ffn_norm.weight"] = (F32, self.hidden_size, 1)
            t[p + "ffn_gate.weight"] = (weight_type, self.hidden_size, self.feed_forward_size)
            t[p + "ffn_up.weight"] = (weight_type, self.hidden_size, self.feed_forward_size)
            t[p + "ffn_down.weight"] = (weight_type, self.feed_forward_size, self.hidden_size)
        return t


SHIELDSTRAL_3B = ModelConfig()


# ---------------------------------------------------------------- matmul

class WeightMatrix:
    """A quantized weight uploaded once to HBM (WeightMatrix + QuantMatMul integer path)."""

    def __init__(self, qtype: int, rows: int, cols: int, data: np.ndarray, device: int = 0):
        lib = load_library()
        self.type, self.rows, self.cols = qtype, rows, cols
        raw = _arr(data, np.uint8)
        h = C.c_void_p()
        _check(lib.shs_matrix_create(qtype, rows, cols, _ptr(raw), device, C.byref(h)))
        self._h = h

    def close(self):
        if getattr(self, "_h", None):
            _lib.shs_matrix_free(self._h)
            self._h = None

    __del__ = close

    def forward(self, x: np.ndarray, semantics: int = 0) -> np.ndarray:
        """QuantMatMul.ForwardAsync (QuantMatMul.cs:71-85): y[t, r] = x[t]·W[r]."""
        x = _arr(x, np.float32).reshape(-1, self.cols)
        y = np.empty((x.shape[0], self.rows), np.float32)
        _check(_lib.shs_matmul(self._h, _ptr(x), x.shape[0], _ptr(y), semantics))
        return y

    def forward_rows(self, row_ids: Sequence[int], x: np.ndarray) -> np.ndarray:
        """QuantMatMul.ForwardRowsAsync (QuantMatMul.cs:98-110)."""
        ids = _arr(row_ids, np.int32)
        x = _arr(x, np.float32).reshape(-1, self.cols)
        y = np.empty((x.shape[0], ids.size), np.float32)
        _check(_lib.shs_matmul_rows(self._h, _ptr(ids), ids.size, _ptr(x), x.shape[0], _ptr(y)))
        return y

    def block_sums(self, x: np.ndarray) -> np.ndarray:
        """The exact int32 per-block dot products, [tokens, rows, cols/32]."""
        x = _arr(x, np.float32).reshape(-1, self.cols)
        out = np.empty((x.shape[0], self.rows, self.cols // 32), np.int32)
        _check(_lib.shs_matmul_block_sums(self._h, _ptr(x), x.shape[0], _ptr(out)))
        return out

    def forward_device(self, x_ptr: int, tokens: int, y_ptr: int) -> None:
        """y_dev = x_dev·Wᵀ for activations already in HBM (device pointers)."""
        _check(_lib.shs_matmul_device(self._h, C.c_void_p(x_ptr), tokens, C.c_void_p(y_ptr)))

    def forward_device_noalloc(self, x_ptr: int, tokens: int, y_ptr: int) -> None:
        """forward_device with the activation codes in the library's fixed per-GPU scratch:
        allocates nothing. Calls that overlap on one GPU race on that scratch."""
        _check(_lib.shs_matmul_device_noalloc(self._h, C.c_void_p(x_ptr), tokens, C.c_void_p(y_ptr)))


# ------------------------------------------------------------------ model

class KvCache:
    """The model's device KV cache, as KvCache (Model/KvCache.cs) exposes it."""

    def __init__(self, model: "MinistralModel"):
        self._m = model

    @property
    def length(self) -> int:
        n = C.c_int32()
        _check(_lib.shs_kv_length(self._m._h, C.byref(n)))
        return n.value

    @property
    def capacity(self) -> int:
        n = C.c_int32()
        _check(_lib.shs_kv_capacity(self._m._h, C.byref(n)))
        return n.value

    @property
    def bytes_per_position(self) -> int:
        c = self._m.config
        return c.layer_count * c.kv_head_count * c.head_dim * 4 * 2

    def reset(self) -> None:
        _check(_lib.shs_kv_reset(self._m._h))

    def snapshot(self, length: int) -> np.ndarray:
        """KvCache.Snapshot: keys [layer][head][pos][dim] for all layers, then values."""
        c = self._m.config
        n = 2 * c.layer_count * c.kv_head_count * length * c.head_dim
        out = np.empty(n, np.float32)
        _check(_lib.shs_kv_snapshot(self._m._h, length, _ptr(out), n))
        return out

    def restore(self, snapshot: np.ndarray, length: int) -> None:
        s = _arr(snapshot, np.float32)
        _check(_lib.shs_kv_restore(self._m._h, _ptr(s), s.size, length))


class ActivationSink:
    """IActivationSink (MinistralModel.cs:494-501): observe(name, rows×cols array)."""

    def observe(self, name: str, values: np.ndarray) -> None:  # pragma: no cover - interface
        raise NotImplementedError


class MinistralModel:
    """MinistralModel over libshieldstral_hip: weights in HBM, one KV cache, not thread-safe."""

    def __init__(self, handle: C.c_void_p, path: str = ""):
        self._h = handle
        self.model_path = path
        cfg = shs_config()
        _check(_lib.shs_get_config(handle, C.byref(cfg)))
        self.config = ModelConfig.from_c(cfg)
        self.kv_cache = KvCache(self)
        self._capture_cb = None

    @classmethod
    def open(cls, gguf_path: str, device: int = 0, initial_cache_capacity: int = 512) -> "MinistralModel":
        lib = load_library()
        h = C.c_void_p()
        _check(lib.shs_open(str(gguf_path).encode(), device, initial_cache_capacity, C.byref(h)))
        return cls(h, str(gguf_path))

    @classmethod
    def from_tensors(cls, config: ModelConfig, tensors: dict, types: dict, device: int = 0,
                     initial_cache_capacity: int = 512) -> "MinistralModel":
        """tensors: name → array of native GGUF bytes (matrices) or float32 (norms)."""
        lib = load_library()
        keep = {k: np.ascontiguousarray(v) for k, v in tensors.items()}
        shapes = {}
        for name, arr in keep.items():
            t = types[name]
            if t in (F32, F16):
                shapes[name] = (t, arr.size, 1)
        full = config.tensor_shapes(Q4_0, Q4_0)
        table = (shs_tensor * len(keep))()
        names = []
        for i, (name, arr) in enumerate(keep.items()):
            t = types[name]
            if name in shapes:
                _, ne0, ne1 = shapes[name]
            elif name in full:
                _, ne0, ne1 = full[name]
            else:
                ne0, ne1 = config.hidden_size, config.vocab_size
            names.append(name.encode())
            table[i].name = names[-1]
            table[i].type = t
            table[i].ne0 = ne0
            table[i].ne1 = ne1
            table[i].data = arr.ctypes.data
        h = C.c_void_p()
        _check(lib.shs_open_tensors(C.byref(config.to_c()), table, len(keep), device, initial_cache_capacity, C.byref(h)))
        return cls(h)

    @classmethod
    def synthetic(cls, config: ModelConfig, weight_type: int = Q4_0, embd_type: Optional[int] = None, seed: int = 0,
                  device: int = 0, initial_cache_capacity: int = 512) -> "MinistralModel":
        lib = load_library()
        h = C.c_void_p()
        _check(lib.shs_open_synthetic(C.byref(config.to_c()), weight_type,
                                      weight_type if embd_type is None else embd_type, seed, device,
                                      initial_cache_capacity, C.byref(h)))
        return cls(h, f"synthetic:{seed}")

    def close(self) -> None:
        if getattr(self, "_h", None):
            _lib.shs_close(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def cached_token_count(self) -> int:
        return self.kv_cache.length

    def reset_kv_cache(self) -> None:
        self.kv_cache.reset()

    def download(self, name: str) -> np.ndarray:
        """A tensor back in native GGUF bytes (matrices) or fp32 (norm gains)."""
        c = self.config
        shapes = c.tensor_shapes(Q4_0, Q4_0)
        if name not in shapes:
            raise TensorNotFoundError(name)
        if name.endswith("norm.weight"):
            out = np.empty(c.hidden_size, np.float32)
        else:
            out = None
            for t in (Q4_0, Q4_1, Q5_0, Q5_1, Q8_0):
                _, ne0, ne1 = shapes[name]
                cand = np.empty(ne1 * (ne0 // 32) * TYPE_SIZE[t], np.uint8)
                if _lib.shs_tensor_download(self._h, name.encode(), _ptr(cand), cand.size) == 0:
                    return cand
            raise InvalidDataError(_lib.shs_last_error().decode())
        _check(_lib.shs_tensor_download(self._h, name.encode(), _ptr(out), out.nbytes))
        return out

    def set_capture(self, sink: Optional[Callable[[str, np.ndarray], None]]) -> None:
        """Attach an IActivationSink-like callable(name, array) or None."""
        if sink is None:
            self._capture_cb = None
            _check(_lib.shs_set_capture(self._h, CAPTURE_FN(0), None))
            return

        def _cb(name, data, rows, cols, user):
            arr = np.ctypeslib.as_array(data, shape=(rows * cols,)).copy().reshape(rows, cols)
            sink(name.decode(), arr)

        self._capture_cb = CAPTURE_FN(_cb)
        _check(_lib.shs_set_capture(self._h, self._capture_cb, None))

    def _forward(self, tokens, head_mode: int, vocab_ids=None, cancel: Optional["CancellationFlag"] = None):
        toks = _arr(tokens, np.int32).reshape(-1)
        if toks.size == 0:
            raise ArgumentError("No tokens to forward.")
        ids = None if vocab_ids is None else _arr(vocab_ids, np.int32)
        if head_mode == 2:
            out = np.empty(self.config.vocab_size, np.float32)
        elif head_mode == 1:
            out = np.empty(ids.size, np.float32)
        else:
            out = None
        flag = None if cancel is None else cancel._ptr
        _check(_lib.shs_forward(self._h, _ptr(toks), toks.size, head_mode, _ptr(ids), 0 if ids is None else ids.size,
                                _ptr(out), flag))
        return out

    def forward(self, tokens, cancel=None) -> np.ndarray:
        """ForwardAsync: full logits for the last position."""
        return self._forward(tokens, 2, cancel=cancel)

    def forward_selected(self, tokens, vocabulary_ids, cancel=None) -> np.ndarray:
        """ForwardSelectedAsync: logits of vocabulary_ids only (bit-identical to the full head)."""
        return self._forward(tokens, 1, vocabulary_ids, cancel)

    def prefill(self, tokens, cancel=None) -> None:
        """PrefillAsync: KV state only, no head."""
        self._forward(tokens, 0, cancel=cancel)

    def forward_batch(self, sequences: Sequence[Sequence[int]], vocabulary_ids) -> np.ndarray:
        """Independent prompts packed into one ragged prefill: [n_seq, n_ids] logits."""
        seqs = [np.asarray(s, np.int32) for s in sequences]
        cu = np.zeros(len(seqs) + 1, np.int32)
        cu[1:] = np.cumsum([s.size for s in seqs])
        toks = np.concatenate(seqs).astype(np.int32)
        ids = _arr(vocabulary_ids, np.int32)
        out = np.empty((len(seqs), ids.size), np.float32)
        _check(_lib.shs_forward_batch(self._h, _ptr(toks), _ptr(cu), len(seqs), _ptr(ids), ids.size, _ptr(out)))
        return out

    def layer_forward(self, layer: int, x: np.ndarray) -> np.ndarray:
        x = _arr(x, np.float32).reshape(-1, self.config.hidden_size)
        y = np.empty_like(x)
        _check(_lib.shs_layer_forward(self._h, layer, _ptr(x), x.shape[0], _ptr(y)))
        return y

    def synchronize(self) -> None:
        """Waits until all work queued on the model's stream has finished."""
        _check(_lib.shs_synchronize(self._h))

    # kernel-class timing (HIP events on the model's stream)
    def profile(self, enable: bool) -> None:
        _check(_lib.shs_profile_enable(self._h, int(enable)))

    def profile_reset(self) -> None:
        _check(_lib.shs_profile_reset(self._h))

    def profile_read(self, kernel_class: str):
        n, ms, ops = C.c_int64(), C.c_double(), C.c_double()
        _check(_lib.shs_profile_read(self._h, kernel_class.encode(), C.byref(n), C.byref(ms), C.byref(ops)))
        return n.value, ms.value, ops.value


def device_expf(x, device: int = 0) -> np.ndarray:
    """The device's softmax/sigmoid exponential on x (parity instrumentation)."""
    lib = load_library()
    x = _arr(x, np.float32).reshape(-1)
    y = np.empty_like(x)
    _check(lib.shs_debug_expf(_ptr(x), x.size, _ptr(y), device))
    return y


class CancellationFlag:
    """A host int the library polls between layers while they run (the CancellationToken):
    a cancellable pass keeps at most two layers queued ahead of the GPU and checks the
    flag while it waits for them, so a cancel set from another thread mid-pass is seen
    within about two layers."""

    def __init__(self):
        self._v = C.c_int32(0)
        self._ptr = C.cast(C.pointer(self._v), C.c_void_p)

    def cancel(self) -> None:
        self._v.value = 1

    @property
    def is_cancellation_requested(self) -> bool:
        return self._v.value != 0


# ------------------------------------------------------- moderator layer

@dataclass(frozen=True)
class ModerationResult:
    """ModerationResult (ShieldstralModerator.cs:22-33)."""
    score: float
    yes_logit: float
    no_logit: float
    prompt_tokens: int
    prefilled_tokens: int

    @property
    def is_unsafe(self) -> bool:
        return self.score > 0.5

    def is_unsafe_at(self, threshold: float) -> bool:
        return self.score > threshold

    def __str__(self) -> str:
        return f"{'UNSAFE' if self.is_unsafe else 'safe'} score={self.score:.6f} (yes={self.yes_logit:.4f} no={self.no_logit:.4f})"


def score(verdict_logits: np.ndarray, n_yes: int, prompt_tokens: int, prefilled: int) -> ModerationResult:
    """ShieldstralModerator.Score (ShieldstralModerator.cs:348-364), in float32 like the reference."""
    v = np.asarray(verdict_logits, np.float32)
    yes = np.float32(-np.inf)
    for x in v[:n_yes]:
        if x > yes:
            yes = x
    no = np.float32(-np.inf)
    for x in v[n_yes:]:
        if x > no:
            no = x
    mx = np.float32(max(yes, no))
    e_yes = np.float32(np.exp(np.float32(yes - mx)))
    e_no = np.float32(np.exp(np.float32(no - mx)))
    s = np.float32(e_yes / np.float32(e_yes + e_no))
    return ModerationResult(float(s), float(yes), float(no), int(prompt_tokens), int(prefilled))


class SystemPromptCache:
    """SystemPromptCache (SystemPromptCache.cs): the fixed prefix's KV state, "SHKV" v1 on disk."""

    MAGIC = 0x53484B56
    VERSION = 1

    def __init__(self, tokens: np.ndarray, state: np.ndarray, fingerprint: str):
        self.tokens = np.asarray(tokens, np.int32)
        self.state = np.asarray(state, np.float32)
        self.fingerprint = fingerprint

    @property
    def token_count(self) -> int:
        return int(self.tokens.size)

    @property
    def byte_size(self) -> int:
        return self.state.size * 4

    @staticmethod
    def compute_fingerprint(model: MinistralModel, tokens: Iterable[int]) -> str:
        """ComputeFingerprint (SystemPromptCache.cs:90-105)."""
        toks = [int(t) for t in tokens]
        path = model.model_path
        if path and os.path.exists(path):
            st = os.stat(path)
            ticks = int(st.st_mtime_ns // 100) + 621355968000000000  # DateTime ticks (UTC)
            ident = f"{os.path.basename(path)}|{st.st_size}|{ticks}|"
        else:
            ident = f"{os.path.basename(path)}|-1|-1|"
        c = model.config
        s = (ident + f"{c.architecture}|{c.layer_count}x{c.kv_head_count}x{c.head_dim}|{len(toks)}:"
             + "".join(f"{t}," for t in toks))
        return hashlib.sha256(s.encode()).hexdigest()

    @classmethod
    def capture(cls, model: MinistralModel, tokens) -> "SystemPromptCache":
        toks = np.asarray(tokens, np.int32)
        model.reset_kv_cache()
        model.prefill(toks)
        return cls(toks, model.kv_cache.snapshot(toks.size), cls.compute_fingerprint(model, toks))

    def restore_into(self, model: MinistralModel) -> None:
        expected = self.compute_fingerprint(model, self.tokens)
        if expected != self.fingerprint:
            raise RuntimeError(f"This snapshot was captured for a different model or prefix "
                               f"(fingerprint {self.fingerprint}, model reports {expected}).")
        model.kv_cache.restore(self.state, self.token_count)

    def is_prefix_of(self, tokens) -> bool:
        t = np.asarray(tokens)
        return t.size >= self.tokens.size and bool(np.array_equal(t[: self.tokens.size], self.tokens))

    def save(self, path) -> None:
        """SHKV v1: magic, version, fingerprint (7-bit length-prefixed UTF-8), tokens, then fp32 state."""
        fp = self.fingerprint.encode()
        n, pre = len(fp), bytearray()
        while True:
            b = n & 0x7F
            n >>= 7
            pre.append(b | (0x80 if n else 0))
            if not n:
                break
        with open(path, "wb") as f:
            f.write(struct.pack("<Ii", self.MAGIC, self.VERSION))
            f.write(bytes(pre) + fp)
            f.write(struct.pack("<i", self.token_count))
            f.write(self.tokens.astype("<i4").tobytes())
            f.write(struct.pack("<q", self.state.size))
            f.write(self.state.astype("<f4").tobytes())

    @classmethod
    def try_load(cls, path, model: MinistralModel) -> Optional["SystemPromptCache"]:
        try:
            with open(path, "rb") as f:
                data = f.read()
        except OSError:
            return None
        try:
            r = io.BytesIO(data)
            magic, ver = struct.unpack("<Ii", r.read(8))
            if magic != cls.MAGIC or ver != cls.VERSION:
                return None
            n, shift = 0, 0
            while True:
                b = r.read(1)
                if not b:
                    return None
                n |= (b[0] & 0x7F) << shift
                shift += 7
                if not b[0] & 0x80:
                    break
            fp = r.read(n).decode()
            (count,) = struct.unpack("<i", r.read(4))
            if count < 0 or count > 1_000_000:
                return None
            raw_tokens = r.read(4 * count)
            if len(raw_tokens) != 4 * count:
                return None
            tokens = np.frombuffer(raw_tokens, "<i4").astype(np.int32)
            (length,) = struct.unpack("<q", r.read(8))
            if length < 0 or length > 2**31 - 1:
                return None
            raw = r.read(4 * length)
            if len(raw) != 4 * length or tokens.size != count:
                return None
            state = np.frombuffer(raw, "<f4").astype(np.float32)
        except (struct.error, UnicodeDecodeError):
            return None
        cache = cls(tokens, state, fp)
        if cls.compute_fingerprint(model, tokens) != fp:
            return None
        return cache

    @classmethod
    def load_or_capture(cls, model: MinistralModel, tokens, path) -> "SystemPromptCache":
        cached = cls.try_load(path, model)
        if cached is not None and np.array_equal(cached.tokens, np.asarray(tokens, np.int32)):
            return cached
        fresh = cls.capture(model, tokens)
        try:
            fresh.save(path)
        except OSError:
            pass
        return fresh


class ShieldstralModerator:
    """ShieldstralModerator (ShieldstralModerator.cs) over token ids: prefix-cached prefill,
    the yes/no rows of the LM head, and the two-way Score. Not thread-safe."""

    def __init__(self, model: MinistralModel, yes_tokens: Sequence[int], no_tokens: Sequence[int],
                 system_prefix_tokens: Optional[Sequence[int]] = None, cache_system_prompt: bool = True,
                 prefix_cache_path: Optional[str] = None, owns_model: bool = False):
        if len(yes_tokens) == 0 or len(no_tokens) == 0:
            raise InvalidDataError("The model's vocabulary has no 'yes'/'no' tokens; "
                                   "this does not look like a Shieldstral checkpoint.")
        self.model = model
        self._owns = owns_model
        self._yes = np.asarray(yes_tokens, np.int32)
        self._no = np.asarray(no_tokens, np.int32)
        self._verdict = np.concatenate([self._yes, self._no]).astype(np.int32)
        self._prefix: Optional[SystemPromptCache] = None
        if cache_system_prompt and system_prefix_tokens is not None and len(system_prefix_tokens) > 0:
            if prefix_cache_path:
                self._prefix = SystemPromptCache.load_or_capture(model, system_prefix_tokens, prefix_cache_path)
            else:
                self._prefix = SystemPromptCache.capture(model, system_prefix_tokens)

    @property
    def config(self) -> ModelConfig:
        return self.model.config

    @property
    def cached_prefix_tokens(self) -> int:
        return 0 if self._prefix is None else self._prefix.token_count

    @property
    def verdict_tokens(self) -> np.ndarray:
        return self._verdict

    def _prepare_cache(self, tokens: np.ndarray) -> int:
        """PrepareCache (ShieldstralModerator.cs:314-323)."""
        if self._prefix is not None and self._prefix.is_prefix_of(tokens):
            self._prefix.restore_into(self.model)
            return self._prefix.token_count
        self.model.reset_kv_cache()
        return 0

    def moderate_tokens(self, tokens: Sequence[int], cancel: Optional[CancellationFlag] = None) -> ModerationResult:
        """ModerateAsync (ShieldstralModerator.cs:251-263) on an already tokenized prompt."""
        if cancel is not None and cancel.is_cancellation_requested:
            raise OperationCanceledError("The operation was canceled.")
        toks = np.asarray(tokens, np.int32)
        prefilled = self._prepare_cache(toks)
        if prefilled == toks.size:
            raise ArgumentError("No tokens to forward.")
        logits = self.model.forward_selected(toks[prefilled:], self._verdict, cancel)
        return score(logits, self._yes.size, toks.size, prefilled)

    def moderate_batch(self, prompts: Sequence[Sequence[int]]) -> list:
        """Scores several prompts in one packed prefill (no prefix cache; the model's KV is untouched)."""
        logits = self.model.forward_batch(prompts, self._verdict)
        return [score(row, self._yes.size, len(p), 0) for row, p in zip(logits, prompts)]

    def verdict_logits(self, tokens: Sequence[int], cancel: Optional[CancellationFlag] = None) -> np.ndarray:
        """VerdictLogitsAsync (ShieldstralModerator.cs:269-277): the full distribution."""
        toks = np.asarray(tokens, np.int32)
        prefilled = self._prepare_cache(toks)
        return self.model.forward(toks[prefilled:], cancel)

    def top_verdict_token(self, tokens: Sequence[int], cancel: Optional[CancellationFlag] = None) -> int:
        """TopVerdictTokenAsync (ShieldstralModerator.cs:370-378), as a token id (ties → lowest)."""
        return int(np.argmax(self.verdict_logits(tokens, cancel)))

    def close(self) -> None:
        if self._owns:
            self.model.close()
