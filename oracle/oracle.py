"""ctypes binding of the CPU oracle (oracle/svl_oracle.c).

TEST INFRASTRUCTURE ONLY: this module is the oracle that the HIP path is
compared against. Only tests/, the smoke
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


# ---- vision tower (src/model/vision.rs) -------------------------------------------

VISION_GLOBAL_TENSORS = 2
VISION_LAYER_TENSORS = 13
VISION_LAYER_NAMES = [
    "input_layernorm.weight",
    "post_attention_layernorm.weight",
    "pre_feedforward_layernorm.weight",
    "post_feedforward_layernorm.weight",
    "self_attn.q_proj.linear.weight",
    "self_attn.k_proj.linear.weight",
    "self_attn.v_proj.linear.weight",
    "self_attn.o_proj.linear.weight",
    "self_attn.q_norm.weight",
    "self_attn.k_norm.weight",
    "mlp.gate_proj.linear.weight",
    "mlp.up_proj.linear.weight",
    "mlp.down_proj.linear.weight",
]


def vision_tensor_names(num_layers: int) -> list[str]:
    """Names in VisionConfig::tensor_shapes order (vision.rs:345-414)."""
    names = ["vision_tower.patch_embedder.input_proj.weight",
             "vision_tower.patch_embedder.position_embedding_table"]
    for i in range(num_layers):
        names += [f"vision_tower.encoder.layers.{i}.{n}" for n in VISION_LAYER_NAMES]
    names.append("embed_vision.embedding_projection.weight")
    return names


class _VisCfg(ctypes.Structure):
    _fields_ = [
        ("hidden_size", ctypes.c_int64),
        ("intermediate_size", ctypes.c_int64),
        ("num_hidden_layers", ctypes.c_int64),
        ("num_attention_heads", ctypes.c_int64),
        ("num_key_value_heads", ctypes.c_int64),
        ("head_dim", ctypes.c_int64),
        ("position_embedding_size", ctypes.c_int64),
        ("rms_norm_eps", ctypes.c_float),
        ("rope_theta", ctypes.c_float),
    ]


def _vision_lib():
    L = lib()
    if not getattr(L, "_vision_ready", False):
        f = ctypes.POINTER(ctypes.c_float)
        i32 = ctypes.POINTER(ctypes.c_int32)
        sz = ctypes.c_size_t
        L.svlo_axial_inv_freq.argtypes = [sz, ctypes.c_float, f]
        L.svlo_axial_rope.argtypes = [f, sz, sz, sz, i32, sz, f, sz]
        L.svlo_pool_patches.argtypes = [f, i32, sz, sz, sz, sz, sz, f]
        L.svlo_vision_forward.argtypes = [ctypes.POINTER(_VisCfg), ctypes.POINTER(f), sz, f, i32,
                                          sz, sz, sz, sz, sz, f, f, ctypes.c_char_p, sz]
        L.svlo_vision_layer.argtypes = [ctypes.POINTER(_VisCfg), ctypes.POINTER(f), sz, f, i32, sz,
                                        f, ctypes.c_char_p, sz]
        L._vision_ready = True
    return L


def _ip(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))


def axial_inv_freq(head_dim, theta):
    out = np.empty(max(head_dim // 4, 1), np.float32)
    _check(_vision_lib().svlo_axial_inv_freq(head_dim, theta, _fp(out)), "axial_inv_freq")
    return out[: head_dim // 4]


def axial_rope(values, seq, heads, head_dim, positions, inv_freq):
    values = _f32(values).copy()
    pos = np.ascontiguousarray(positions, np.int32).reshape(-1)
    inv = _f32(inv_freq)
    _check(_vision_lib().svlo_axial_rope(_fp(values), seq, heads, head_dim, _ip(pos),
                                         pos.size // 2, _fp(inv), inv.size), "axial_rope")
    return values


def pool_patches(hidden, positions, valid, grid_w, grid_h, soft, width):
    hidden = _f32(hidden)
    pos = np.ascontiguousarray(positions, np.int32).reshape(-1)
    out = np.empty(max(soft * width, 1), np.float32)
    _check(_vision_lib().svlo_pool_patches(_fp(hidden), _ip(pos), valid, grid_w, grid_h, soft,
                                           width, _fp(out)), "pool_patches")
    return out[: soft * width]


def resolve_vision_config(config: dict) -> dict:
    """The fields of VisionConfig (vision.rs:84-273) that the forward pass uses."""
    v = config["vision_config"]
    return dict(
        hidden_size=int(v["hidden_size"]), intermediate_size=int(v["intermediate_size"]),
        num_hidden_layers=int(v["num_hidden_layers"]),
        num_attention_heads=int(v["num_attention_heads"]),
        num_key_value_heads=int(v["num_key_value_heads"]), head_dim=int(v["head_dim"]),
        position_embedding_size=int(v["position_embedding_size"]),
        rms_norm_eps=float(np.float32(float(v["rms_norm_eps"]))),
        rope_theta=float(np.float32(float(v["rope_parameters"]["rope_theta"]))))


class OracleVisionModel:
    """The reference VisionModel restated on the CPU (vision.rs:686-959).

    `patches` is any object with the ImagePatches accessors of
    media/preprocess.rs:87-147: pixel_values [>= valid, 768],
    positions [>= valid, 2], valid_patches, max_patches, patch_grid, soft_tokens.
    """

    def __init__(self, config: dict, weights: dict, text_hidden: int):
        self.cfg = c = resolve_vision_config(config)
        self.text_hidden = int(text_hidden)
        self._c = _VisCfg(c["hidden_size"], c["intermediate_size"], c["num_hidden_layers"],
                          c["num_attention_heads"], c["num_key_value_heads"], c["head_dim"],
                          c["position_embedding_size"], c["rms_norm_eps"], c["rope_theta"])
        names = vision_tensor_names(c["num_hidden_layers"])
        self._arrays = [_f32(weights[n]).reshape(-1) for n in names]
        self._ptrs = (ctypes.POINTER(ctypes.c_float) * len(names))(*[_fp(a) for a in self._arrays])

    def forward(self, patches, capture_hidden=False):
        """Returns dict(pooled [soft, text_hidden], hidden_states, soft_tokens)."""
        c = self.cfg
        valid = int(patches.valid_patches)
        pix = _f32(np.asarray(patches.pixel_values, np.float32).reshape(-1)[: valid * 768])
        pos = np.ascontiguousarray(np.asarray(patches.positions, np.int32).reshape(-1, 2)[:valid])
        gw, gh = patches.patch_grid
        soft = int(patches.soft_tokens)
        H, L = c["hidden_size"], c["num_hidden_layers"]
        pooled = np.empty(max(soft, 1) * self.text_hidden, np.float32)
        hidden = np.empty((L + 1) * max(valid, 1) * H, np.float32) if capture_hidden else None
        msg = ctypes.create_string_buffer(256)
        st = _vision_lib().svlo_vision_forward(
            ctypes.byref(self._c), self._ptrs, self.text_hidden, _fp(pix), _ip(pos), valid,
            int(patches.max_patches), int(gw), int(gh), soft, _fp(pooled),
            None if hidden is None else _fp(hidden), msg, 256)
        if st != 0:
            raise OracleError(st, msg.value.decode())
        out = dict(pooled=pooled[: soft * self.text_hidden].reshape(soft, self.text_hidden),
                   soft_tokens=soft)
        if capture_hidden:
            out["hidden_states"] = hidden.reshape(L + 1, valid, H)
        return out

    def layer(self, layer, hidden, positions):
        """Encoder layer `layer` alone (vision.rs:816-935) applied to hidden
        [rows, hidden_size] with patch positions [rows, 2] (x, y); the code
        the forward pass runs per layer."""
        h = _f32(hidden)
        rows = h.shape[0]
        pos = np.ascontiguousarray(np.asarray(positions, np.int32).reshape(-1, 2)[:rows])
        assert pos.shape[0] == rows
        out = np.empty_like(h)
        msg = ctypes.create_string_buffer(256)
        st = _vision_lib().svlo_vision_layer(ctypes.byref(self._c), self._ptrs, int(layer), _fp(h),
                                             _ip(pos), rows, _fp(out), msg, 256)
        if st != 0:
            raise OracleError(st, msg.value.decode())
        return out


# ---- audio tower (src/model/audio.rs) ---------------------------------------------

AUDIO_GLOBAL_TENSORS = 5
AUDIO_LAYER_TENSORS = 62
_BOUNDS = ["input_min", "input_max", "output_min", "output_max"]


def audio_tensor_names(num_layers: int) -> list[str]:
    """Names in AudioConfig::tensor_shapes order (audio.rs:394-498)."""
    p = "audio_tower.subsample_conv_projection."
    names = [p + "layer0.conv.weight", p + "layer0.norm.weight", p + "layer1.conv.weight",
             p + "layer1.norm.weight", p + "input_proj_linear.weight"]
    for i in range(num_layers):
        q = f"audio_tower.layers.{i}."
        for ff in ("feed_forward1", "feed_forward2"):
            b = q + ff + "."
            names += [b + "pre_layer_norm.weight", b + "post_layer_norm.weight",
                      b + "ffw_layer_1.linear.weight", b + "ffw_layer_2.linear.weight"]
            for lin in ("ffw_layer_1", "ffw_layer_2"):
                names += [f"{b}{lin}.{x}" for x in _BOUNDS]
        for proj in ("q_proj", "k_proj", "v_proj", "post"):
            names.append(f"{q}self_attn.{proj}.linear.weight")
            names += [f"{q}self_attn.{proj}.{x}" for x in _BOUNDS]
        names += [q + "self_attn.relative_k_proj.weight", q + "self_attn.per_dim_scale",
                  q + "lconv1d.pre_layer_norm.weight", q + "lconv1d.linear_start.linear.weight",
                  q + "lconv1d.linear_end.linear.weight"]
        for lin in ("linear_start", "linear_end"):
            names += [f"{q}lconv1d.{lin}.{x}" for x in _BOUNDS]
        names += [q + "lconv1d.depthwise_conv1d.weight", q + "lconv1d.conv_norm.weight",
                  q + "norm_pre_attn.weight", q + "norm_post_attn.weight", q + "norm_out.weight"]
    names += ["audio_tower.output_proj.weight", "audio_tower.output_proj.bias",
              "embed_audio.embedding_projection.weight"]
    return names


class _AudCfg(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int64) for n in (
        "hidden_size", "intermediate_size", "num_hidden_layers", "num_attention_heads", "head_dim",
        "conv_kernel_size", "conv_channels0", "conv_channels1", "attention_chunk_size",
        "attention_context_left", "attention_context_right", "output_proj_dims")] + [
        (n, ctypes.c_float) for n in ("attention_logit_cap", "rms_norm_eps", "residual_weight",
                                      "gradient_clipping")]


def _audio_lib():
    L = lib()
    if not getattr(L, "_audio_ready", False):
        f = ctypes.POINTER(ctypes.c_float)
        sz = ctypes.c_size_t
        L.svlo_silu_value.restype = ctypes.c_float
        L.svlo_silu_value.argtypes = [ctypes.c_float]
        L.svlo_sigmoid_value.restype = ctypes.c_float
        L.svlo_sigmoid_value.argtypes = [ctypes.c_float]
        L.svlo_softplus_value.restype = ctypes.c_float
        L.svlo_softplus_value.argtypes = [ctypes.c_float]
        L.svlo_clamp_value.restype = ctypes.c_float
        L.svlo_clamp_value.argtypes = [ctypes.c_float] * 3
        L.svlo_clipped_linear.argtypes = [f, f, f, sz, sz, sz, f]
        L.svlo_audio_position_embeddings.argtypes = [sz, sz, f]
        L.svlo_audio_attention_core.argtypes = [f, f, f, f, ctypes.POINTER(ctypes.c_ubyte), sz, sz,
                                                sz, sz, sz, sz, ctypes.c_float, f]
        L.svlo_audio_subsampled_frames.restype = sz
        L.svlo_audio_subsampled_frames.argtypes = [sz]
        L.svlo_audio_forward.argtypes = [ctypes.POINTER(_AudCfg), ctypes.POINTER(f), sz, f,
                                         ctypes.POINTER(ctypes.c_ubyte), sz,
                                         ctypes.POINTER(sz), f, f, f, ctypes.c_char_p, sz]
        L.svlo_audio_layer.argtypes = [ctypes.POINTER(_AudCfg), ctypes.POINTER(f), sz, f,
                                       ctypes.POINTER(ctypes.c_ubyte), sz, f, ctypes.c_char_p, sz]
        L._audio_ready = True
    return L


def silu_value(x):
    return _audio_lib().svlo_silu_value(float(x))


def sigmoid_value(x):
    return _audio_lib().svlo_sigmoid_value(float(x))


def softplus_value(x):
    return _audio_lib().svlo_softplus_value(float(x))


def clipped_linear(x, w, bounds, rows, in_f, out_f):
    x, w, b = _f32(x), _f32(w), _f32(bounds)
    out = np.empty(rows * out_f, np.float32)
    _check(_audio_lib().svlo_clipped_linear(_fp(x), _fp(w), _fp(b), rows, in_f, out_f, _fp(out)),
           "clipped_linear")
    return out


def audio_position_embeddings(hidden, positions):
    out = np.empty(positions * hidden, np.float32)
    _check(_audio_lib().svlo_audio_position_embeddings(hidden, positions, _fp(out)), "positions")
    return out.reshape(positions, hidden)


def audio_attention_core(q, k, v, relk, mask, heads, chunk, left, right, cap):
    """q, k, v [rows, heads * hd] (already projected and scaled), relk
    [positions, heads * hd], mask [rows]."""
    q, k, v, relk = _f32(q), _f32(k), _f32(v), _f32(relk)
    m = np.ascontiguousarray(np.asarray(mask, np.uint8).reshape(-1))
    rows, width = q.shape
    out = np.empty((rows, width), np.float32)
    _check(_audio_lib().svlo_audio_attention_core(
        _fp(q), _fp(k), _fp(v), _fp(relk), m.ctypes.data_as(ctypes.POINTER(ctypes.c_ubyte)), rows,
        heads, width // heads, chunk, left, right, cap, _fp(out)), "audio attention")
    return out


def resolve_audio_config(config: dict) -> dict:
    """The fields of AudioConfig (audio.rs:94-294) that the forward pass uses."""
    a = config["audio_config"]
    H, NH = int(a["hidden_size"]), int(a["num_attention_heads"])
    c0, c1 = (int(x) for x in a["subsampling_conv_channels"])
    f32 = lambda k: float(np.float32(float(a[k])))
    return dict(hidden_size=H, intermediate_size=4 * H, num_hidden_layers=int(a["num_hidden_layers"]),
                num_attention_heads=NH, head_dim=H // NH, conv_kernel_size=int(a["conv_kernel_size"]),
                conv_channels0=c0, conv_channels1=c1,
                attention_chunk_size=int(a["attention_chunk_size"]),
                attention_context_left=int(a["attention_context_left"]),
                attention_context_right=int(a["attention_context_right"]),
                output_proj_dims=int(a["output_proj_dims"]),
                attention_logit_cap=f32("attention_logit_cap"), rms_norm_eps=f32("rms_norm_eps"),
                residual_weight=f32("residual_weight"), gradient_clipping=f32("gradient_clipping"))


class OracleAudioModel:
    """The reference AudioModel restated on the CPU (audio.rs:932-1134)."""

    def __init__(self, config: dict, weights: dict, text_hidden: int):
        self.cfg = c = resolve_audio_config(config)
        self.text_hidden = int(text_hidden)
        self._c = _AudCfg(*[c[n] for n, _ in _AudCfg._fields_])
        names = audio_tensor_names(c["num_hidden_layers"])
        self._arrays = [_f32(weights[n]).reshape(-1) for n in names]
        self._ptrs = (ctypes.POINTER(ctypes.c_float) * len(names))(*[_fp(a) for a in self._arrays])

    def forward(self, features, mask, capture_hidden=False):
        """features [frames, 128] log-mel, mask [frames] bool. Returns
        dict(pooled [tokens, text_hidden], audio_tokens, sscp_output, hidden_states)."""
        c = self.cfg
        feats = _f32(features).reshape(-1)
        m = np.ascontiguousarray(np.asarray(mask, np.uint8).reshape(-1))
        frames = m.size
        rows = _audio_lib().svlo_audio_subsampled_frames(frames)
        H, L = c["hidden_size"], c["num_hidden_layers"]
        pooled = np.empty(max(rows, 1) * self.text_hidden, np.float32)
        sscp = np.empty(max(rows, 1) * H, np.float32) if capture_hidden else None
        hidden = np.empty(max(L, 1) * max(rows, 1) * H, np.float32) if capture_hidden else None
        tokens = ctypes.c_size_t(0)
        msg = ctypes.create_string_buffer(256)
        st = _audio_lib().svlo_audio_forward(
            ctypes.byref(self._c), self._ptrs, self.text_hidden, _fp(feats),
            m.ctypes.data_as(ctypes.POINTER(ctypes.c_ubyte)), frames, ctypes.byref(tokens),
            _fp(pooled), None if sscp is None else _fp(sscp), None if hidden is None else _fp(hidden),
            msg, 256)
        if st != 0:
            raise OracleError(st, msg.value.decode())
        n = tokens.value
        out = dict(pooled=pooled[: n * self.text_hidden].reshape(n, self.text_hidden),
                   audio_tokens=n)
        if capture_hidden:
            out["sscp_output"] = sscp[: n * H].reshape(n, H)
            out["hidden_states"] = hidden[: L * n * H].reshape(L, n, H)
        return out


    def layer(self, layer, hidden, row_mask):
        """Encoder layer `layer` alone (audio.rs:1001-1083) applied to hidden
        [rows, hidden_size] with the subsampled row mask [rows]; the code the
        forward pass runs per layer."""
        h = _f32(hidden)
        rows = h.shape[0]
        m = np.ascontiguousarray(np.asarray(row_mask, np.uint8).reshape(-1))
        assert m.size == rows
        out = np.empty_like(h)
        msg = ctypes.create_string_buffer(256)
        st = _audio_lib().svlo_audio_layer(ctypes.byref(self._c), self._ptrs, int(layer), _fp(h),
                                           m.ctypes.data_as(ctypes.POINTER(ctypes.c_ubyte)), rows,
                                           _fp(out), msg, 256)
        if st != 0:
            raise OracleError(st, msg.value.decode())
        return out


# ---- audio_preprocess.rs log-mel front end ----------------------------------------

MEL_FEATURES = 128


def _mel_lib():
    L = lib()
    if not getattr(L, "_mel_ready", False):
        sz = ctypes.c_size_t
        d = ctypes.POINTER(ctypes.c_double)
        L.svlo_hann_window.restype = None
        L.svlo_hann_window.argtypes = [ctypes.POINTER(ctypes.c_float)]
        L.svlo_mel_filter_bank.argtypes = [d]
        L.svlo_fft.argtypes = [d, sz]
        L.svlo_log_mel_layout.argtypes = [sz, ctypes.POINTER(sz), ctypes.POINTER(sz),
                                          ctypes.POINTER(sz), ctypes.c_char_p, sz]
        L.svlo_log_mel.argtypes = [ctypes.POINTER(ctypes.c_float), sz,
                                   ctypes.POINTER(ctypes.c_float),
                                   ctypes.POINTER(ctypes.c_ubyte), ctypes.c_char_p, sz]
        L._mel_ready = True
    return L


def hann_window():
    out = np.zeros(320, np.float32)
    _mel_lib().svlo_hann_window(_fp(out))
    return out


def mel_filter_bank():
    """[257 bins, 128 filters] float64."""
    out = np.zeros((257, MEL_FEATURES), np.float64)
    _check(_mel_lib().svlo_mel_filter_bank(out.ctypes.data_as(ctypes.POINTER(ctypes.c_double))),
           "filter bank")
    return out


def fft(values):
    """FftPlan::forward on a complex vector of power-of-two length."""
    v = np.ascontiguousarray(values, np.complex128).copy()
    _check(_mel_lib().svlo_fft(v.ctypes.data_as(ctypes.POINTER(ctypes.c_double)), v.size), "fft")
    return v


def log_mel_layout(samples):
    """(frames, padded_samples, valid_frames) for a clip of `samples` samples."""
    sz = ctypes.c_size_t
    f, p, v = sz(), sz(), sz()
    msg = ctypes.create_string_buffer(256)
    _check(_mel_lib().svlo_log_mel_layout(samples, ctypes.byref(f), ctypes.byref(p),
                                          ctypes.byref(v), msg, 256), msg.value.decode())
    return f.value, p.value, v.value


def log_mel(samples):
    """log_mel (audio_preprocess.rs:94-200): (features [frames, 128] f32,
    mask [frames] bool, padded_samples, valid_frames)."""
    x = _f32(samples).ravel()
    msg = ctypes.create_string_buffer(256)
    if x.size == 0:
        _check(_mel_lib().svlo_log_mel(_fp(np.zeros(1, np.float32)), 0, None, None, msg, 256),
               msg.value.decode())
    try:
        frames, padded, valid = log_mel_layout(min(x.size, 480000))
    except OracleError:
        frames, padded, valid = 1, 0, 0
    feats = np.zeros((frames, MEL_FEATURES), np.float32)
    mask = np.zeros(frames, np.uint8)
    _check(_mel_lib().svlo_log_mel(_fp(x), x.size, _fp(feats),
                                   mask.ctypes.data_as(ctypes.POINTER(ctypes.c_ubyte)), msg, 256),
           msg.value.decode())
    return feats, mask.astype(bool), padded, valid


# ---- index/vector.rs exact cosine ranking -------------------------------------------

def vector_rank(query, embeddings, chunk_ids, mask=None, has_dim=None):
    """vector::rank (vector.rs:17-97): the full ranking as (indices, scores)."""
    L = lib()
    if not getattr(L, "_search_ready", False):
        sz = ctypes.c_size_t
        L.svlo_vector_rank.argtypes = [ctypes.POINTER(ctypes.c_float), sz,
                                       ctypes.POINTER(ctypes.c_float),
                                       ctypes.POINTER(ctypes.c_uint64), sz, sz, ctypes.c_int,
                                       ctypes.POINTER(ctypes.c_ubyte), ctypes.POINTER(sz),
                                       ctypes.POINTER(ctypes.c_double), ctypes.POINTER(sz),
                                       ctypes.c_char_p, sz]
        L._search_ready = True
    q = _f32(query).ravel()
    e = _f32(embeddings)
    n = e.shape[0] if e.ndim == 2 else 0
    dim = e.shape[1] if e.ndim == 2 else 0
    e = e.reshape(-1) if e.size else np.zeros(1, np.float32)
    ids = np.ascontiguousarray(chunk_ids, np.uint64)
    if ids.size == 0:
        ids = np.zeros(1, np.uint64)
    m = None if mask is None else np.ascontiguousarray(mask, np.uint8)
    out_i = np.zeros(max(n, 1), np.uintp)
    out_s = np.zeros(max(n, 1), np.float64)
    cnt = ctypes.c_size_t()
    msg = ctypes.create_string_buffer(256)
    qq = q if q.size else np.zeros(1, np.float32)
    _check(L.svlo_vector_rank(_fp(qq), q.size, _fp(e), ids.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64)),
                              n, dim, int(n > 0 if has_dim is None else has_dim),
                              None if m is None else m.ctypes.data_as(ctypes.POINTER(ctypes.c_ubyte)),
                              out_i.ctypes.data_as(ctypes.POINTER(ctypes.c_size_t)),
                              out_s.ctypes.data_as(ctypes.POINTER(ctypes.c_double)),
                              ctypes.byref(cnt), msg, 256), msg.value.decode())
    return out_i[: cnt.value].astype(np.int64), out_s[: cnt.value]
