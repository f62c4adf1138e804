"""ctypes binding of the CPU oracle (oracle/svl_oracle.c).

TEST INFRASTRUCTURE ONLY: this module is the checker. Only tests/, the smoke
check in __graft_entry__.py and the CPU-baseline leg of bench.py import it;
the product library never does.

The config resolution below restates the parts of src/model/config.rs that
the forward pass consumes (config.rs:112-269: layer_types, per_layer_config
overrides, rope_parameters, eps as f64 -> f32) independently of the product's
own parser, so a parser mistake cannot hide behind a shared helper.
"""
from __future__ import annotations

import ctypes
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libsvl_oracle.so")
_lib = None

GLOBAL_TENSORS = 5
LAYER_TENSORS = 17
LAYER_NAMES = [
    "input_layernorm.weight",
    "post_attention_layernorm.weight",
    "pre_feedforward_layernorm.weight",
    "post_feedforward_layernorm.weight",
    "layer_scalar",
    "mlp.gate_proj.weight",
    "mlp.up_proj.weight",
    "mlp.down_proj.weight",
    "ple_block.per_layer_input_gate.weight",
    "ple_block.per_layer_projection.weight",
    "ple_block.post_per_layer_input_norm.weight",
    "self_attn.q_proj.weight",
    "self_attn.k_proj.weight",
    "self_attn.v_proj.weight",
    "self_attn.o_proj.weight",
    "self_attn.q_norm.weight",
    "self_attn.k_norm.weight",
]
GLOBAL_NAMES = [
    "language_model.embed_tokens.weight",
    "language_model.embedding_projection.weight",
    "language_model.norm.weight",
    "language_model.ple.per_layer_model_projection.weight",
    "language_model.ple.per_layer_projection_norm.weight",
]


def tensor_names(num_layers: int) -> list[str]:
    """Names in TextConfig::tensor_shapes order (config.rs:394-484)."""
    names = list(GLOBAL_NAMES)
    for i in range(num_layers):
        names += [f"language_model.layers.{i}.{n}" for n in LAYER_NAMES]
    return names


class _Cfg(ctypes.Structure):
    _fields_ = [
        ("vocab_size", ctypes.c_int64),
        ("hidden_size", ctypes.c_int64),
        ("intermediate_size", ctypes.c_int64),
        ("num_hidden_layers", ctypes.c_int64),
        ("num_attention_heads", ctypes.c_int64),
        ("hidden_size_per_layer_input", ctypes.c_int64),
        ("embedding_dim", ctypes.c_int64),
        ("max_position_embeddings", ctypes.c_int64),
        ("sliding_window", ctypes.c_int64),
        ("pad_token_id", ctypes.c_int64),
        ("rms_norm_eps", ctypes.c_float),
        ("full_rope_theta", ctypes.c_float),
        ("sliding_rope_theta", ctypes.c_float),
        ("layer_type", ctypes.POINTER(ctypes.c_int32)),
        ("head_dim", ctypes.POINTER(ctypes.c_int64)),
        ("num_kv_heads", ctypes.POINTER(ctypes.c_int64)),
    ]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle library missing: {_LIB_PATH} (run make -C oracle)")
        _lib = ctypes.CDLL(_LIB_PATH)
        f = ctypes.POINTER(ctypes.c_float)
        sz = ctypes.c_size_t
        _lib.svlo_dot.restype = ctypes.c_float
        _lib.svlo_gelu_tanh_value.restype = ctypes.c_float
        _lib.svlo_gelu_tanh_value.argtypes = [ctypes.c_float]
        _lib.svlo_rope_inv_freq.argtypes = [sz, ctypes.c_float, f]
        _lib.svlo_rms_norm_rows.argtypes = [f, f, sz, sz, ctypes.c_float, f]
        _lib.svlo_rms_norm_rows_unscaled.argtypes = [f, sz, sz, ctypes.c_float, f]
        _lib.svlo_bidirectional_attention.argtypes = [f, f, f, sz, sz, sz, sz, ctypes.c_int64,
                                                      ctypes.c_float, f]
        _lib.svlo_text_forward.argtypes = [
            ctypes.POINTER(_Cfg), ctypes.POINTER(f), ctypes.POINTER(ctypes.c_uint32), sz, f, sz, sz,
            sz, f, f, f, f, ctypes.c_char_p, sz]
    return _lib


def _fp(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


class OracleError(RuntimeError):
    def __init__(self, status, message=""):
        super().__init__(f"oracle status {status}: {message}")
        self.status = status


def _check(status, what=""):
    if status != 0:
        raise OracleError(status, what)


# ---- kernels.rs scalar functions -------------------------------------------------

def linear(x, w, rows, in_f, out_f):
    x, w = _f32(x), _f32(w)
    out = np.empty(rows * out_f, np.float32)
    _check(lib().svlo_linear(_fp(x), _fp(w), ctypes.c_size_t(rows), ctypes.c_size_t(in_f),
                             ctypes.c_size_t(out_f), _fp(out)), "linear")
    return out


def matmul(a, b, m, k, n):
    a, b = _f32(a), _f32(b)
    out = np.empty(m * n, np.float32)
    _check(lib().svlo_matmul(_fp(a), _fp(b), ctypes.c_size_t(m), ctypes.c_size_t(k),
                             ctypes.c_size_t(n), _fp(out)), "matmul")
    return out


def rms_norm_rows(x, w, rows, width, eps):
    x, w = _f32(x), _f32(w)
    out = np.empty(rows * width, np.float32)
    _check(lib().svlo_rms_norm_rows(_fp(x), _fp(w), rows, width, eps, _fp(out)), "rms_norm_rows")
    return out


def rms_norm_rows_unscaled(x, rows, width, eps):
    x = _f32(x)
    out = np.empty(rows * width, np.float32)
    _check(lib().svlo_rms_norm_rows_unscaled(_fp(x), rows, width, eps, _fp(out)), "rms unscaled")
    return out


def softmax(v):
    v = _f32(v)
    out = np.empty(v.size, np.float32)
    _check(lib().svlo_softmax(_fp(v), ctypes.c_size_t(v.size), _fp(out)), "softmax")
    return out


def gelu_tanh_value(x):
    return lib().svlo_gelu_tanh_value(float(x))


def geglu(g, u):
    g, u = _f32(g), _f32(u)
    out = np.empty(g.size, np.float32)
    _check(lib().svlo_geglu(_fp(g), _fp(u), ctypes.c_size_t(g.size), _fp(out)), "geglu")
    return out


def l2_normalize(v):
    v = _f32(v)
    out = np.empty(v.size, np.float32)
    _check(lib().svlo_l2_normalize(_fp(v), ctypes.c_size_t(v.size), _fp(out)), "l2")
    return out


def mean_pool(v, rows, width):
    v = _f32(v)
    out = np.empty(width, np.float32)
    _check(lib().svlo_mean_pool(_fp(v), ctypes.c_size_t(rows), ctypes.c_size_t(width), _fp(out)),
           "mean_pool")
    return out


def truncate_and_normalize(v, dim):
    v = _f32(v)
    out = np.empty(dim, np.float32)
    _check(lib().svlo_truncate_and_normalize(_fp(v), ctypes.c_size_t(v.size), ctypes.c_size_t(dim),
                                             _fp(out)), "truncate")
    return out


def rope_inv_freq(head_dim, base):
    out = np.empty(max(head_dim // 2, 1), np.float32)
    _check(lib().svlo_rope_inv_freq(head_dim, base, _fp(out)), "rope_inv_freq")
    return out[: head_dim // 2]


def rope_with_inv_freq(values, seq, heads, head_dim, inv_freq, offset=0):
    values = _f32(values).copy()
    inv = _f32(inv_freq)
    _check(lib().svlo_rope_with_inv_freq(_fp(values), ctypes.c_size_t(seq), ctypes.c_size_t(heads),
                                         ctypes.c_size_t(head_dim), _fp(inv),
                                         ctypes.c_size_t(inv.size), ctypes.c_size_t(offset)), "rope")
    return values


def bidirectional_attention(q, k, v, seq, nh, nkv, hd, window, scale=1.0):
    q, k, v = _f32(q), _f32(k), _f32(v)
    out = np.empty(seq * nh * hd, np.float32)
    _check(lib().svlo_bidirectional_attention(_fp(q), _fp(k), _fp(v), seq, nh, nkv, hd,
                                              -1 if window is None else int(window), scale,
                                              _fp(out)), "attention")
    return out


# ---- config resolution and the text forward pass ----------------------------------

def resolve_config(config: dict) -> dict:
    """Resolved per-layer layout of an EmbeddingGemma-2 text config dict."""
    text = config.get("text_config", config)
    n = int(text["num_hidden_layers"])
    types = [1 if t == "full_attention" else 0 for t in text["layer_types"]]
    hd = [int(text["head_dim"])] * n
    kv = [int(text["num_key_value_heads"])] * n
    for key, ov in (text.get("per_layer_config") or {}).items():
        hd[int(key)] = int(ov["head_dim"])
        kv[int(key)] = int(ov["num_key_value_heads"])
    rp = text["rope_parameters"]
    return dict(
        vocab_size=int(text["vocab_size"]), hidden_size=int(text["hidden_size"]),
        intermediate_size=int(text["intermediate_size"]), num_hidden_layers=n,
        num_attention_heads=int(text["num_attention_heads"]),
        hidden_size_per_layer_input=int(text["hidden_size_per_layer_input"]),
        embedding_dim=int(text["embedding_dim"]),
        max_position_embeddings=int(text["max_position_embeddings"]),
        sliding_window=int(text["sliding_window"]),
        pad_token_id=-1 if text.get("pad_token_id") is None else int(text["pad_token_id"]),
        rms_norm_eps=float(np.float32(float(text["rms_norm_eps"]))),
        full_rope_theta=float(np.float32(float(rp["full_attention"]["rope_theta"]))),
        sliding_rope_theta=float(np.float32(float(rp["sliding_attention"]["rope_theta"]))),
        layer_type=types, head_dim=hd, num_kv_heads=kv)


class OracleTextModel:
    """The reference TextModel restated on the CPU (text.rs:77-555)."""

    def __init__(self, config: dict, weights: dict):
        self.cfg = resolve_config(config)
        c = self.cfg
        self._lt = np.asarray(c["layer_type"], np.int32)
        self._hd = np.asarray(c["head_dim"], np.int64)
        self._kv = np.asarray(c["num_kv_heads"], np.int64)
        self._c = _Cfg(c["vocab_size"], c["hidden_size"], c["intermediate_size"],
                       c["num_hidden_layers"], c["num_attention_heads"],
                       c["hidden_size_per_layer_input"], c["embedding_dim"],
                       c["max_position_embeddings"], c["sliding_window"], c["pad_token_id"],
                       c["rms_norm_eps"], c["full_rope_theta"], c["sliding_rope_theta"],
                       self._lt.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                       self._hd.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)),
                       self._kv.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)))
        names = tensor_names(c["num_hidden_layers"])
        self._arrays = [_f32(weights[n]).reshape(-1) for n in names]
        self._ptrs = (ctypes.POINTER(ctypes.c_float) * len(names))(*[_fp(a) for a in self._arrays])

    def forward(self, ids, capture_hidden=False, features=None, feature_start=0,
                feature_count=0):
        """Returns dict(projected, pooled, normalized, hidden_states)."""
        c = self.cfg
        ids = np.ascontiguousarray(ids, np.uint32)
        seq = ids.size
        H, E, L = c["hidden_size"], c["embedding_dim"], c["num_hidden_layers"]
        projected = np.empty(max(seq, 1) * E, np.float32)
        pooled = np.empty(E, np.float32)
        normalized = np.empty(E, np.float32)
        hidden = np.empty((L + 1) * max(seq, 1) * H, np.float32) if capture_hidden else None
        feats = None if features is None else _f32(features).reshape(-1)
        msg = ctypes.create_string_buffer(256)
        st = lib().svlo_text_forward(
            ctypes.byref(self._c), self._ptrs,
            ids.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), seq,
            None if feats is None else _fp(feats), feature_start, feature_count,
            0 if feats is None else feats.size, _fp(projected), _fp(pooled), _fp(normalized),
            None if hidden is None else _fp(hidden), msg, 256)
        if st != 0:
            raise OracleError(st, msg.value.decode())
        out = dict(projected=projected.reshape(seq, E), pooled=pooled, normalized=normalized)
        if capture_hidden:
            out["hidden_states"] = hidden.reshape(L + 1, seq, H)
        return out

    def forward_rows(self, rows, threads=None):
        """One forward per row, rows spread over threads (the reference's
        request-level concurrency, tests/text_bench.rs:58-72)."""
        threads = threads or min(len(rows), os.cpu_count() or 1)
        with ThreadPoolExecutor(max_workers=threads) as ex:
            return list(ex.map(lambda r: self.forward(r), rows))
