"""Python binding of libsvl_hip.so (include/svl_hip.h), shaped like the
reference crate's model API so callers and tests read like the reference's:

* ``TextConfig.from_json_str`` — the strict parser of src/model/config.rs:112-269
* ``TextModel`` — src/model/text.rs:77-555 (``forward``, ``forward_with_features``,
  ``embed_ids``) plus ``forward_batch`` (many independent rows, one launch
  sequence)
* ``ForwardOutput`` — text.rs:38-75 (``projected``, ``pooled``, ``normalized``,
  ``hidden_states``, ``embedding(dim)``)
* the kernel seam of src/tensor/kernels.rs on device tensors (``linear``,
  ``rms_norm_rows``, ``rope_with_inv_freq``, ``bidirectional_attention`` ...)

Errors raise ``SvlError`` whose ``kind`` follows src/error.rs. The compute
runs only in the HIP library: if it is missing or no gfx950 device is
visible, every model call raises; nothing here falls back to the CPU.
"""
from __future__ import annotations

import ctypes
import json
import math
import os
import struct
import threading

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libsvl_hip.so")

STATUS = {0: "Ok", 2: "Usage", 3: "Io", 4: "Corrupt", 5: "LimitExceeded", 6: "Unsupported",
          7: "Internal", 8: "Device"}

# src/model/config.rs:20-51
MAX_CONFIG_BYTES = 1024 * 1024
MAX_TEXT_TOKENS = 8192
MAX_HIDDEN_SIZE = 16384
MAX_LAYERS = 128
MAX_HEADS = 128
MAX_HEAD_DIM = 1024
MAX_INTERMEDIATE_SIZE = 65536
MAX_VOCAB_SIZE = 1_000_000
MAX_EMBEDDING_DIM = 16384
MAX_POSITIONS = 1_048_576


class SvlError(RuntimeError):
    """Error with the reference's taxonomy (src/error.rs:24-37)."""

    def __init__(self, status: int, message: str):
        self.status = status
        self.kind = STATUS.get(status, f"status{status}")
        super().__init__(f"{self.kind}: {message}")


def _corrupt(msg):
    return SvlError(4, msg)


def _limit(msg):
    return SvlError(5, msg)


def _unsupported(msg):
    return SvlError(6, msg)


# ---------------------------------------------------------------------------
# ctypes declarations

class _TensorView(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("dtype", ctypes.c_int32), ("ndim", ctypes.c_int32),
                ("shape", ctypes.c_int64 * 8), ("data", ctypes.c_void_p),
                ("nbytes", ctypes.c_size_t)]


class _Config(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int64) for n in (
        "vocab_size", "hidden_size", "intermediate_size", "num_hidden_layers",
        "num_attention_heads", "hidden_size_per_layer_input", "embedding_dim",
        "max_position_embeddings", "sliding_window", "pad_token_id")] + [
        ("rms_norm_eps", ctypes.c_double), ("full_rope_theta", ctypes.c_double),
        ("sliding_rope_theta", ctypes.c_double),
        ("layer_type", ctypes.POINTER(ctypes.c_int32)),
        ("head_dim", ctypes.POINTER(ctypes.c_int64)),
        ("num_kv_heads", ctypes.POINTER(ctypes.c_int64))]


class _FeatureSpan(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("start", ctypes.c_int64), ("count", ctypes.c_int64),
                ("len", ctypes.c_int64)]


EXPORTED = [
    "svl_init", "svl_shutdown", "svl_last_error", "svl_text_model_create",
    "svl_text_model_destroy", "svl_text_forward_batch", "svl_text_forward_device",
    "svl_text_embed_ids", "svl_truncate_and_normalize", "svl_text_model_set_stream_split",
    "svl_text_model_set_pass_tokens", "svl_text_model_set_kernel_timing",
    "svl_kernel_class_count", "svl_kernel_class_name", "svl_text_model_kernel_stats",
    "svl_linear", "svl_rms_norm_rows", "svl_rope_with_inv_freq", "svl_rope_inv_freq",
    "svl_bidirectional_attention", "svl_gelu_tanh", "svl_geglu", "svl_add", "svl_mean_pool",
    "svl_l2_normalize", "svl_synth_uniform", "svl_synth_ids", "svl_synth_lengths",
    "svl_vision_model_create", "svl_vision_model_destroy", "svl_vision_model_set_stream_split",
    "svl_vision_model_set_pass_patches", "svl_vision_forward_batch",
    "svl_vision_forward_device", "svl_image_embed_batch", "svl_image_embed_device",
    "svl_audio_model_create", "svl_audio_model_destroy", "svl_audio_token_count",
    "svl_audio_forward_batch", "svl_audio_forward_device", "svl_audio_embed_batch",
    "svl_audio_embed_device", "svl_log_mel_layout", "svl_log_mel_create", "svl_log_mel_destroy",
    "svl_log_mel_batch", "svl_log_mel_device", "svl_audio_embed_samples",
    "svl_audio_embed_samples_device", "svl_tokenizer_create", "svl_tokenizer_destroy",
    "svl_tokenizer_encode", "svl_tokenizer_encode_batch", "svl_tokenizer_decode",
    "svl_tokenizer_token_id", "svl_tokenizer_token", "svl_tokenizer_vocab_size",
    "svl_tokenizer_max_token_id", "svl_tokenizer_bos_id", "svl_tokenizer_eos_id",
    "svl_tokenizer_unk_id", "svl_tokenizer_pad_id", "svl_tokenizer_is_special_id",
    "svl_text_embed_texts", "svl_vector_index_create", "svl_vector_index_destroy",
    "svl_vector_index_size", "svl_vector_index_dimension", "svl_vector_rank",
    "svl_vector_rank_device", "svl_tensor_to_f32", "svl_bidirectional_attention_noalloc",
    "svl_measure_peaks", "svl_measure_fp64_peak", "svl_set_attention_path",
]

_lib = None
_lib_lock = threading.Lock()


def _share_torch_hip_runtime():
    """PyTorch-ROCm ships its own libamdhip64.so (SONAME libamdhip64.so.7,
    the same as /opt/rocm's). Loading torch's HIP library first makes this
    library bind to that already-loaded runtime, so a process that also uses
    torch for device buffers and streams has exactly one HIP runtime; two
    runtimes in one process cannot share streams and torch cannot initialise
    after another runtime has claimed the device. Without torch the library
    uses the system ROCm runtime."""
    try:
        import torch  # noqa: F401
    except ImportError:
        return
    tlib = os.path.join(os.path.dirname(torch.__file__), "lib", "libamdhip64.so")
    if os.path.exists(tlib):
        ctypes.CDLL(tlib, mode=ctypes.RTLD_GLOBAL)


def lib():
    """Loads libsvl_hip.so; raises if it has not been built."""
    global _lib
    with _lib_lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"HIP extension missing: {LIB_PATH} (build with make -C "
                               f"seldon-vault-lite-rust_amd or __graft_entry__.build())")
        _share_torch_hip_runtime()
        L = ctypes.CDLL(LIB_PATH)
        vp, i64, i32, f32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_float
        fptr = ctypes.POINTER(ctypes.c_float)
        L.svl_last_error.restype = ctypes.c_char_p
        L.svl_kernel_class_name.restype = ctypes.c_char_p
        L.svl_kernel_class_name.argtypes = [i32]
        L.svl_init.argtypes = [ctypes.c_int, ctypes.POINTER(vp)]
        L.svl_shutdown.argtypes = [vp]
        L.svl_text_model_create.argtypes = [vp, ctypes.POINTER(_Config),
                                            ctypes.POINTER(_TensorView), ctypes.c_size_t,
                                            ctypes.POINTER(vp)]
        L.svl_text_model_destroy.argtypes = [vp]
        L.svl_text_forward_batch.argtypes = [vp, vp, vp, i32, vp, vp, vp, vp, vp]
        L.svl_text_forward_device.argtypes = [vp, vp, vp, i32, vp, i32, vp, vp]
        L.svl_text_embed_ids.argtypes = [vp, vp, i64, i64, vp]
        L.svl_truncate_and_normalize.argtypes = [vp, ctypes.c_size_t, ctypes.c_size_t, vp]
        L.svl_tensor_to_f32.argtypes = [ctypes.POINTER(_TensorView), vp, i64]
        L.svl_measure_peaks.argtypes = [vp, ctypes.POINTER(ctypes.c_double),
                                        ctypes.POINTER(ctypes.c_double)]
        L.svl_measure_fp64_peak.argtypes = [vp, ctypes.POINTER(ctypes.c_double)]
        L.svl_text_model_set_kernel_timing.argtypes = [vp, ctypes.c_int]
        L.svl_text_model_set_stream_split.argtypes = [vp, ctypes.c_int]
        L.svl_text_model_set_pass_tokens.argtypes = [vp, i64]
        L.svl_text_model_kernel_stats.argtypes = [vp, vp, vp, vp]
        L.svl_linear.argtypes = [vp, vp, i64, i64, i64, vp, vp]
        L.svl_rms_norm_rows.argtypes = [vp, vp, i64, i64, f32, vp, vp]
        L.svl_rope_with_inv_freq.argtypes = [vp, i64, i64, i64, vp, i64, i64, vp]
        L.svl_rope_inv_freq.argtypes = [i64, f32, vp]
        L.svl_bidirectional_attention.argtypes = [vp, vp, vp, i64, i64, i64, i64, i64, f32, vp, vp]
        L.svl_bidirectional_attention_noalloc.argtypes = [vp, vp, vp, i64, i64, i64, i64, i64,
                                                          f32, vp, vp]
        L.svl_set_attention_path.argtypes = [ctypes.c_int]
        L.svl_gelu_tanh.argtypes = [vp, i64, vp, vp]
        L.svl_geglu.argtypes = [vp, vp, i64, vp, vp]
        L.svl_add.argtypes = [vp, vp, i64, vp, vp]
        L.svl_mean_pool.argtypes = [vp, i64, i64, vp, vp]
        L.svl_l2_normalize.argtypes = [vp, i64, vp, vp]
        L.svl_synth_uniform.argtypes = [ctypes.c_uint64, ctypes.c_uint64, f32, f32,
                                        ctypes.c_size_t, vp]
        L.svl_synth_ids.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint32,
                                    ctypes.c_size_t, vp]
        L.svl_synth_lengths.argtypes = [ctypes.c_uint64, ctypes.c_uint64, i64, i64,
                                        ctypes.c_size_t, vp]
        L.svl_vision_model_create.argtypes = [vp, vp, i64, ctypes.POINTER(_TensorView),
                                              ctypes.c_size_t, ctypes.POINTER(vp)]
        L.svl_vision_model_destroy.argtypes = [vp]
        L.svl_vision_model_set_stream_split.argtypes = [vp, ctypes.c_int]
        L.svl_vision_model_set_pass_patches.argtypes = [vp, i64]
        L.svl_vision_forward_batch.argtypes = [vp, vp, i32, vp, vp]
        L.svl_vision_forward_device.argtypes = [vp, vp, vp, i32, vp, vp]
        L.svl_image_embed_batch.argtypes = [vp, vp, vp, vp, i32, i64, vp]
        L.svl_image_embed_device.argtypes = [vp, vp, vp, vp, vp, i32, i64, vp]
        _lib = L
        return L


def _check(status):
    if status != 0:
        raise SvlError(status, lib().svl_last_error().decode(errors="replace"))


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else None


# ---------------------------------------------------------------------------
# Configuration: src/model/config.rs:112-269

class TextConfig:
    """Validated EmbeddingGemma-2 text configuration (config.rs:76-95)."""

    def __init__(self, **kw):
        self.__dict__.update(kw)

    @classmethod
    def from_json_str(cls, text: str) -> "TextConfig":
        if len(text.encode()) > MAX_CONFIG_BYTES:
            raise _limit("configuration file is too large")
        try:
            value = json.loads(text)
        except json.JSONDecodeError as e:
            raise _corrupt(f"configuration is not valid JSON: {e}")
        return cls.from_json_value(value)

    @classmethod
    def from_file(cls, path: str) -> "TextConfig":
        with open(path, "rb") as f:
            data = f.read(MAX_CONFIG_BYTES + 1)
        return cls.from_json_str(data.decode("utf-8"))

    @classmethod
    def from_json_value(cls, value) -> "TextConfig":
        if not isinstance(value, dict):
            raise _corrupt("model configuration must be a JSON object")
        text = value.get("text_config", value)
        if not isinstance(text, dict):
            raise _corrupt("text_config must be a JSON object")
        if "model_type" in text:
            if not isinstance(text["model_type"], str):
                raise _corrupt("model_type must be a string")
            if text["model_type"] != "embedding_gemma2_text":
                raise _unsupported(f"text model type {text['model_type']} is not embedding_gemma2_text")
        if "dtype" in text:
            d = text["dtype"]
            if not isinstance(d, str):
                raise _corrupt("dtype must be a string")
            if d == "float16":
                raise _unsupported("float16 is forbidden for EmbeddingGemma 2 activations")
            if d not in ("bfloat16", "float32"):
                raise _unsupported(f"model dtype {d} is not supported")

        def unsigned(obj, key):
            if key not in obj:
                raise _corrupt(f"configuration is missing {key}")
            v = obj[key]
            if isinstance(v, bool) or not isinstance(v, int) or v < 0:
                raise _corrupt(f"{key} must be a non-negative integer")
            return v

        def number(obj, key):
            if key not in obj:
                raise _corrupt(f"configuration is missing {key}")
            v = obj[key]
            if isinstance(v, bool) or not isinstance(v, (int, float)):
                raise _corrupt(f"{key} must be a number")
            return float(v)

        H = unsigned(text, "hidden_size")
        I = unsigned(text, "intermediate_size")
        L = unsigned(text, "num_hidden_layers")
        NH = unsigned(text, "num_attention_heads")
        KV = unsigned(text, "num_key_value_heads")
        HD = unsigned(text, "head_dim")
        P = unsigned(text, "hidden_size_per_layer_input")
        E = unsigned(text, "embedding_dim")
        V = unsigned(text, "vocab_size")
        MP = unsigned(text, "max_position_embeddings")
        SW = unsigned(text, "sliding_window")
        eps = number(text, "rms_norm_eps")
        if not math.isfinite(float(np.float32(eps))):
            raise _corrupt("RMSNorm epsilon does not fit a finite f32 value")
        act = text.get("hidden_activation")
        if not isinstance(act, str):
            raise _corrupt("configuration is missing hidden_activation")
        if act != "gelu_pytorch_tanh":
            raise _unsupported(f"hidden activation {act} is not gelu_pytorch_tanh")
        if text.get("attention_bias", False):
            raise _unsupported("attention bias is not part of the frozen model")
        drop = text.get("attention_dropout")
        if drop is not None and float(drop) != 0.0:
            raise _unsupported("attention dropout is not implemented by the inference engine")
        for v, hi, what in [(H, MAX_HIDDEN_SIZE, "hidden size"), (I, MAX_INTERMEDIATE_SIZE,
                            "intermediate size"), (L, MAX_LAYERS, "layer count"),
                            (NH, MAX_HEADS, "attention head count"),
                            (P, MAX_HIDDEN_SIZE, "per-layer input size"),
                            (E, MAX_EMBEDDING_DIM, "embedding dimension"),
                            (V, MAX_VOCAB_SIZE, "vocabulary size"),
                            (MP, MAX_POSITIONS, "position count"), (SW, MP, "sliding window")]:
            if v == 0 or v > hi:
                raise _limit(f"{what} {v} is outside 1..={hi}")
        if not math.isfinite(eps) or eps < 0:
            raise _corrupt("RMSNorm epsilon must be finite and non-negative")
        _head_layout(NH, KV, HD)
        types = text.get("layer_types")
        if types is None:
            raise _corrupt("layer_types is missing")
        if not isinstance(types, list):
            raise _corrupt("layer_types must be an array")
        if len(types) != L:
            raise _corrupt(f"layer_types has {len(types)} entries, expected {L}")
        lt = []
        for i, t in enumerate(types):
            if not isinstance(t, str):
                raise _corrupt(f"layer_types[{i}] must be a string")
            if t not in ("sliding_attention", "full_attention"):
                raise _unsupported(f"layer type {t} is not sliding_attention or full_attention")
            lt.append(1 if t == "full_attention" else 0)
        if lt[-1] != 1:
            raise _unsupported("the last layer must use full attention")
        hd = [HD] * L
        kv = [KV] * L
        plc = text.get("per_layer_config")
        if plc is not None:
            if not isinstance(plc, dict):
                raise _corrupt("per_layer_config must be an object")
            for key, entry in plc.items():
                digits = key[1:] if key.startswith("+") else key
                if not digits or not digits.isascii() or not digits.isdigit():
                    raise _corrupt(f"per_layer_config key {key} is not an index")
                idx = int(digits)
                if idx >= L:
                    raise _corrupt(f"per_layer_config index {idx} is outside {L} layers")
                if not isinstance(entry, dict):
                    raise _corrupt(f"per_layer_config[{idx}] must be an object")
                hd[idx] = unsigned(entry, "head_dim")
                kv[idx] = unsigned(entry, "num_key_value_heads")
        for i in range(L):
            _head_layout(NH, kv[i], hd[i])
        for t in (0, 1):
            dims = {hd[i] for i in range(L) if lt[i] == t}
            if len(dims) > 1:
                raise _unsupported("layers of the same attention type must share one head dimension")
        rp = text.get("rope_parameters")
        if rp is None:
            raise _corrupt("rope_parameters is missing")
        if not isinstance(rp, dict):
            raise _corrupt("rope_parameters must be an object")
        thetas = {}
        for key, entry in rp.items():
            if not isinstance(entry, dict):
                raise _corrupt(f"rope_parameters.{key} must be an object")
            rt = entry.get("rope_type")
            if not isinstance(rt, str):
                raise _corrupt("configuration is missing rope_type")
            if rt != "default":
                raise _unsupported(f"RoPE type {rt} is not supported")
            th = number(entry, "rope_theta")
            if not math.isfinite(th) or th <= 1.0:
                raise _corrupt(f"RoPE theta {th} must be finite and greater than one")
            if key not in ("full_attention", "sliding_attention"):
                raise _unsupported(f"RoPE parameters for {key} are not supported")
            thetas[key] = th
        if set(thetas) != {"full_attention", "sliding_attention"}:
            raise _corrupt("rope_parameters must declare full_attention and sliding_attention")
        special = {}
        for key in ("pad_token_id", "bos_token_id", "eos_token_id"):
            v = text.get(key)
            if v is None:
                special[key] = None
                continue
            if isinstance(v, bool) or not isinstance(v, int) or v < 0 or v > 0xFFFFFFFF:
                raise _corrupt(f"{key} must be a token id")
            if v >= V:
                raise _corrupt(f"special token id {v} is outside the vocabulary of {V} entries")
            special[key] = v
        return cls(vocab_size=V, hidden_size=H, intermediate_size=I, num_hidden_layers=L,
                   num_attention_heads=NH, hidden_size_per_layer_input=P, embedding_dim=E,
                   max_position_embeddings=MP, sliding_window=SW, rms_norm_eps=eps,
                   full_rope_theta=thetas["full_attention"],
                   sliding_rope_theta=thetas["sliding_attention"], layer_type=lt, head_dim=hd,
                   num_kv_heads=kv, **special)

    def tensor_shapes(self):
        """config.rs:394-484."""
        H, P, I = self.hidden_size, self.hidden_size_per_layer_input, self.intermediate_size
        out = [("language_model.embed_tokens.weight", (self.vocab_size, H)),
               ("language_model.embedding_projection.weight", (self.embedding_dim, H)),
               ("language_model.norm.weight", (H,)),
               ("language_model.ple.per_layer_model_projection.weight", (self.num_hidden_layers * P, H)),
               ("language_model.ple.per_layer_projection_norm.weight", (P,))]
        for i in range(self.num_hidden_layers):
            p = f"language_model.layers.{i}."
            qd = self.num_attention_heads * self.head_dim[i]
            kd = self.num_kv_heads[i] * self.head_dim[i]
            out += [(p + "input_layernorm.weight", (H,)), (p + "post_attention_layernorm.weight", (H,)),
                    (p + "pre_feedforward_layernorm.weight", (H,)),
                    (p + "post_feedforward_layernorm.weight", (H,)), (p + "layer_scalar", (1,)),
                    (p + "mlp.gate_proj.weight", (I, H)), (p + "mlp.up_proj.weight", (I, H)),
                    (p + "mlp.down_proj.weight", (H, I)),
                    (p + "ple_block.per_layer_input_gate.weight", (P, H)),
                    (p + "ple_block.per_layer_projection.weight", (H, P)),
                    (p + "ple_block.post_per_layer_input_norm.weight", (H,)),
                    (p + "self_attn.q_proj.weight", (qd, H)), (p + "self_attn.k_proj.weight", (kd, H)),
                    (p + "self_attn.v_proj.weight", (kd, H)), (p + "self_attn.o_proj.weight", (H, qd)),
                    (p + "self_attn.q_norm.weight", (self.head_dim[i],)),
                    (p + "self_attn.k_norm.weight", (self.head_dim[i],))]
        return out

    def _c(self):
        self._lt = np.asarray(self.layer_type, np.int32)
        self._hd = np.asarray(self.head_dim, np.int64)
        self._kv = np.asarray(self.num_kv_heads, np.int64)
        return _Config(self.vocab_size, self.hidden_size, self.intermediate_size,
                       self.num_hidden_layers, self.num_attention_heads,
                       self.hidden_size_per_layer_input, self.embedding_dim,
                       self.max_position_embeddings, self.sliding_window,
                       -1 if self.pad_token_id is None else self.pad_token_id,
                       self.rms_norm_eps, self.full_rope_theta, self.sliding_rope_theta,
                       self._lt.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                       self._hd.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)),
                       self._kv.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)))


def _head_layout(nh, kv, hd):
    """config.rs:571-598."""
    if kv == 0 or kv > nh:
        raise _corrupt(f"key/value head count {kv} is not in 1..={nh}")
    if nh % kv:
        raise _corrupt(f"attention head count {nh} is not a multiple of key/value head count {kv}")
    if hd == 0 or hd > MAX_HEAD_DIM or hd % 2:
        raise _corrupt(f"head dimension {hd} must be a positive even value at most {MAX_HEAD_DIM}")


# ---------------------------------------------------------------------------
# Safetensors (src/binary/safetensors.rs:123-222): F32 and BF16 views.

class RawTensor:
    """A little-endian tensor payload: dtype 'F32' or 'BF16'."""

    def __init__(self, dtype, shape, data: np.ndarray):
        self.dtype, self.shape, self.data = dtype, tuple(shape), data

    def to_f32(self) -> np.ndarray:
        """TensorEntry::to_f32 (safetensors.rs:69-110), decoded by the library:
        F32 as stored, BF16 widened exactly (bf16.rs:13-15)."""
        numel = int(np.prod(self.shape, dtype=np.int64)) if self.shape else 1
        out = np.zeros(max(numel, 1), np.float32)
        data = np.ascontiguousarray(self.data)
        v = _TensorView()
        v.name = b"tensor"
        v.dtype = 1 if self.dtype == "BF16" else (0 if self.dtype == "F32" else 99)
        v.ndim = len(self.shape)
        for i, d in enumerate(self.shape):
            v.shape[i] = int(d)
        v.data = data.ctypes.data if data.size else None
        v.nbytes = data.nbytes
        _check(lib().svl_tensor_to_f32(ctypes.byref(v), _ptr(out), out.size))
        return out[:numel].reshape(self.shape)


def read_safetensors(path: str) -> dict:
    with open(path, "rb") as f:
        raw = f.read()
    if len(raw) < 8:
        raise _corrupt("safetensors file is truncated")
    (n,) = struct.unpack("<Q", raw[:8])
    if 8 + n > len(raw):
        raise _corrupt("safetensors header is truncated")
    header = json.loads(raw[8:8 + n].decode("utf-8"))
    body = memoryview(raw)[8 + n:]
    out = {}
    for name, meta in header.items():
        if name == "__metadata__":
            continue
        dt = meta["dtype"]
        a, b = meta["data_offsets"]
        if dt == "F32":
            arr = np.frombuffer(body[a:b], dtype="<f4")
        elif dt == "BF16":
            arr = np.frombuffer(body[a:b], dtype="<u2")
        elif dt == "F16":
            raise _unsupported(f"tensor {name} is F16, which is forbidden")
        else:
            raise _unsupported(f"tensor {name} has unsupported dtype {dt}")
        out[name] = RawTensor(dt, meta["shape"], arr)
    return out


# ---------------------------------------------------------------------------
# Device context

class Device:
    """One HIP device (gfx950)."""

    _cache = {}

    def __init__(self, ordinal=0):
        self.ordinal = ordinal
        h = ctypes.c_void_p()
        _check(lib().svl_init(ordinal, ctypes.byref(h)))
        self.handle = h

    @classmethod
    def get(cls, ordinal=0):
        if ordinal not in cls._cache:
            cls._cache[ordinal] = cls(ordinal)
        return cls._cache[ordinal]

    def measure_peaks(self):
        """(FP32 MFMA TFLOP/s, HBM copy GB/s) measured on this device."""
        t, b = ctypes.c_double(), ctypes.c_double()
        _check(lib().svl_measure_peaks(self.handle, ctypes.byref(t), ctypes.byref(b)))
        return t.value, b.value

    def measure_fp64_peak(self):
        """FP64 MFMA TFLOP/s measured on this device."""
        t = ctypes.c_double()
        _check(lib().svl_measure_fp64_peak(self.handle, ctypes.byref(t)))
        return t.value


def tensor_views(weights: dict):
    """svl_tensor_view array over a name -> RawTensor / array mapping.
    Returns (array, count, keep-alive list); F32 and BF16 payloads pass
    through unchanged, F16 is rejected (src/tensor/dtype.rs)."""
    views, keep = [], []
    for name, t in weights.items():
        if isinstance(t, RawTensor):
            dtype, shape, data = (1 if t.dtype == "BF16" else 0), t.shape, t.data
        else:
            a = np.asarray(t)
            if a.dtype == np.float16:
                raise _unsupported(f"tensor {name} is F16, which is forbidden")
            # shape first: ascontiguousarray turns a rank-0 scalar into shape (1,)
            dtype, shape, data = 0, a.shape, np.ascontiguousarray(a, dtype=np.float32)
        data = np.ascontiguousarray(data)
        bname = name.encode()
        keep += [data, bname]
        v = _TensorView()
        v.name = bname
        v.dtype = dtype
        v.ndim = len(shape)
        for i, d in enumerate(shape):
            v.shape[i] = int(d)
        v.data = data.ctypes.data
        v.nbytes = data.nbytes
        views.append(v)
    return (_TensorView * len(views))(*views), len(views), keep


class ForwardOutput:
    """text.rs:38-75."""

    def __init__(self, projected, pooled, normalized, hidden_states):
        self._projected, self._pooled = projected, pooled
        self._normalized, self._hidden = normalized, hidden_states

    def projected(self):
        return self._projected

    def pooled(self):
        return self._pooled

    def normalized(self):
        return self._normalized

    def hidden_states(self):
        return self._hidden

    def embedding(self, dimension: int):
        return truncate_and_normalize(self._normalized, dimension)


class TextModel:
    """The reference TextModel (text.rs:77-555) with its forward pass on the GPU."""

    def __init__(self, config: TextConfig, weights: dict, device: Device | None = None):
        self.config = config
        self.device = device or Device.get(0)
        arr, n, keep = tensor_views(weights)  # alive until the library has copied them
        cfg = config._c()
        h = ctypes.c_void_p()
        _check(lib().svl_text_model_create(self.device.handle, ctypes.byref(cfg), arr, n,
                                           ctypes.byref(h)))
        self.handle = h
        self.row_groups = 3   # the library's default split of large batches

    @classmethod
    def load(cls, model_dir: str, device: Device | None = None) -> "TextModel":
        """TextModel::load (text.rs:93-108): config.json + model.safetensors."""
        cfg = TextConfig.from_file(os.path.join(model_dir, "config.json"))
        w = read_safetensors(os.path.join(model_dir, "model.safetensors"))
        return cls(cfg, w, device)

    def close(self):
        if getattr(self, "handle", None):
            lib().svl_text_model_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # text.rs:150-152
    def forward(self, input_ids, capture_hidden=False) -> ForwardOutput:
        return self.forward_batch([input_ids], capture_hidden=capture_hidden)[0]

    # text.rs:167-180
    def forward_with_features(self, input_ids, features, feature_start, feature_count,
                              capture_hidden=False) -> ForwardOutput:
        return self.forward_batch([input_ids], capture_hidden=capture_hidden,
                                  features=[(features, feature_start, feature_count)])[0]

    def forward_batch(self, rows, capture_hidden=False, features=None):
        """Independent forward passes of `rows` (each a token-id sequence),
        packed into one launch sequence. Returns one ForwardOutput per row."""
        c = self.config
        lens = [len(r) for r in rows]
        offsets = np.zeros(len(rows) + 1, np.int64)
        offsets[1:] = np.cumsum(lens)
        T = int(offsets[-1])
        ids = np.zeros(max(T, 1), np.uint32)
        for i, r in enumerate(rows):
            ids[offsets[i]:offsets[i + 1]] = np.asarray(r, dtype=np.int64).astype(np.uint32) \
                if len(r) else []
        E, H, L = c.embedding_dim, c.hidden_size, c.num_hidden_layers
        B = len(rows)
        normalized = np.zeros((B, E), np.float32)
        pooled = np.zeros((B, E), np.float32)
        projected = np.zeros((max(T, 1), E), np.float32)
        hidden = np.zeros((L + 1, max(T, 1), H), np.float32) if capture_hidden else None
        spans = None
        keep = []
        if features is not None:
            spans = (_FeatureSpan * B)()
            for i, f in enumerate(features):
                if f is None:
                    continue
                data, start, count = f
                data = np.ascontiguousarray(data, np.float32).reshape(-1)
                keep.append(data)
                spans[i] = _FeatureSpan(data.ctypes.data, start, count, data.size)
        _check(lib().svl_text_forward_batch(
            self.handle, _ptr(ids), _ptr(offsets), B, spans, _ptr(normalized), _ptr(pooled),
            _ptr(projected), _ptr(hidden)))
        outs = []
        for i in range(B):
            a, b = int(offsets[i]), int(offsets[i + 1])
            hs = hidden[:, a:b, :] if capture_hidden else []
            outs.append(ForwardOutput(projected[a:b], pooled[i], normalized[i], hs))
        return outs

    def embed_batch(self, rows, dims):
        """embed_ids (text.rs:546-554) over many rows in one call: ids on the
        host, one forward pass of the packed batch returning only the
        normalized embeddings, then truncate_and_normalize on the host at
        every dim. Returns [len(rows), sum(dims)]."""
        lens = [len(r) for r in rows]
        offsets = np.zeros(len(rows) + 1, np.int64)
        offsets[1:] = np.cumsum(lens)
        ids = np.concatenate([np.asarray(r, np.int64) for r in rows]).astype(np.uint32) \
            if rows else np.zeros(1, np.uint32)
        E = self.config.embedding_dim
        normalized = np.zeros((len(rows), E), np.float32)
        _check(lib().svl_text_forward_batch(self.handle, _ptr(ids), _ptr(offsets), len(rows),
                                            None, _ptr(normalized), None, None, None))
        out = np.zeros((len(rows), sum(dims)), np.float32)
        for i in range(len(rows)):
            off = 0
            for d in dims:
                _check(lib().svl_truncate_and_normalize(_ptr(normalized[i]), E, int(d),
                                                        _ptr(out[i, off:off + d])))
                off += d
        return out

    def forward_device(self, ids_dev_ptr: int, offsets, dims, out_dev_ptr: int, stream=0):
        """Device-resident batch: ids already in HBM, Matryoshka outputs to HBM."""
        offsets = np.ascontiguousarray(offsets, np.int64)
        dims = np.ascontiguousarray(dims, np.int32)
        _check(lib().svl_text_forward_device(self.handle, ctypes.c_void_p(ids_dev_ptr),
                                             _ptr(offsets), len(offsets) - 1, _ptr(dims),
                                             dims.size, ctypes.c_void_p(out_dev_ptr),
                                             ctypes.c_void_p(stream)))

    # text.rs:546-554
    def embed_ids(self, input_ids, dimension: int):
        ids = np.ascontiguousarray(input_ids, np.uint32)
        out = np.zeros(max(int(dimension), 1), np.float32)
        _check(lib().svl_text_embed_ids(self.handle, _ptr(ids) if ids.size else None, ids.size,
                                        int(dimension), _ptr(out)))
        return out[:dimension]

    def set_stream_split(self, groups):
        """Row groups (1..4, each on its own stream) for batches of 4096+
        tokens; True = 3 (the default), False = 1."""
        g = 3 if groups is True else (1 if groups is False else int(groups))
        _check(lib().svl_text_model_set_stream_split(self.handle, g))
        self.row_groups = max(1, min(g, 4))

    def set_pass_tokens(self, tokens: int):
        """Largest pass of consecutive rows a batch runs in (0: sized to about
        32 GiB of device workspace); results do not depend on it."""
        _check(lib().svl_text_model_set_pass_tokens(self.handle, int(tokens)))

    def set_kernel_timing(self, enable: bool):
        _check(lib().svl_text_model_set_kernel_timing(self.handle, 1 if enable else 0))

    def kernel_stats(self):
        n = lib().svl_kernel_class_count()
        ms = np.zeros(n, np.float64)
        launches = np.zeros(n, np.int64)
        work = np.zeros(n, np.float64)
        _check(lib().svl_text_model_kernel_stats(self.handle, _ptr(ms), _ptr(launches), _ptr(work)))
        return {lib().svl_kernel_class_name(i).decode(): dict(ms=float(ms[i]), launches=int(launches[i]),
                                                               work=float(work[i])) for i in range(n)}


def truncate_and_normalize(values, dimension):
    """kernels.rs:916-927 (host)."""
    v = np.ascontiguousarray(values, np.float32)
    out = np.zeros(max(int(dimension), 1), np.float32)
    _check(lib().svl_truncate_and_normalize(_ptr(v), v.size, int(dimension), _ptr(out)))
    return out[:dimension]


# ---------------------------------------------------------------------------
# Kernel seam on device tensors (torch tensors on cuda, used as plain
# device memory: data_ptr() and the current stream).

def _dp(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _stream():
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def linear(x, w, rows, in_f, out_f, out):
    _check(lib().svl_linear(_dp(x), _dp(w), rows, in_f, out_f, _dp(out), _stream()))


def rms_norm_rows(x, w, rows, width, eps, out):
    _check(lib().svl_rms_norm_rows(_dp(x), _dp(w), rows, width, eps, _dp(out), _stream()))


def rope_with_inv_freq(values, seq, heads, hd, inv_freq, offset=0):
    inv = np.ascontiguousarray(inv_freq, np.float32)
    _check(lib().svl_rope_with_inv_freq(_dp(values), seq, heads, hd, _ptr(inv), inv.size, offset,
                                        _stream()))


def rope_inv_freq(head_dim, base):
    out = np.zeros(max(head_dim // 2, 1), np.float32)
    _check(lib().svl_rope_inv_freq(head_dim, base, _ptr(out)))
    return out[: head_dim // 2]


def bidirectional_attention(q, k, v, seq, nh, nkv, hd, window, scale, out):
    _check(lib().svl_bidirectional_attention(_dp(q), _dp(k), _dp(v), seq, nh, nkv, hd,
                                             -1 if window is None else int(window), scale,
                                             _dp(out), _stream()))


def bidirectional_attention_noalloc(q, k, v, seq, nh, nkv, hd, window, scale, out):
    """bidirectional_attention without device allocation (the library's
    per-GPU scratch array; at most 8192 keys)."""
    _check(lib().svl_bidirectional_attention_noalloc(
        _dp(q), _dp(k), _dp(v), seq, nh, nkv, hd, -1 if window is None else int(window), scale,
        _dp(out), _stream()))


ATTENTION_PATHS = {"auto": 0, "fallback": 1, "generic": 2}


def set_attention_path(path: str):
    """Test hook: which attention kernel every later launch of the process
    uses ("auto" by shape, "fallback" as for rows whose K/V window passes
    2 GiB, "generic")."""
    _check(lib().svl_set_attention_path(ATTENTION_PATHS[path]))


def gelu_tanh(x, n, out):
    _check(lib().svl_gelu_tanh(_dp(x), n, _dp(out), _stream()))


def geglu(g, u, n, out):
    _check(lib().svl_geglu(_dp(g), _dp(u), n, _dp(out), _stream()))


def add(a, b, n, out):
    _check(lib().svl_add(_dp(a), _dp(b), n, _dp(out), _stream()))


def mean_pool(x, rows, width, out):
    _check(lib().svl_mean_pool(_dp(x), rows, width, _dp(out), _stream()))


def l2_normalize(x, n, out):
    _check(lib().svl_l2_normalize(_dp(x), n, _dp(out), _stream()))


# ---------------------------------------------------------------------------
# Deterministic synthetic data (counter-based SplitMix64; see svl_hip.h).

def synth_uniform(seed, stream, lo, hi, n):
    out = np.empty(n, np.float32)
    lib().svl_synth_uniform(seed, stream, lo, hi, n, _ptr(out))
    return out


def synth_ids(seed, stream, vocab, n):
    out = np.empty(n, np.uint32)
    lib().svl_synth_ids(seed, stream, vocab, n, _ptr(out))
    return out


def synth_lengths(seed, stream, lo, hi, n):
    out = np.empty(n, np.int64)
    lib().svl_synth_lengths(seed, stream, lo, hi, n, _ptr(out))
    return out
