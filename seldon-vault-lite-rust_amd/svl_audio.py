"""Audio tower and audio embedder on the MI355X backend, shaped like the
reference crate's API:

* ``AudioConfig.from_json_str`` — the strict parser of src/model/audio.rs:94-294
* ``MelSpectrogram`` — the log-mel input of src/media/audio_preprocess.rs:50-90
* ``AudioModel`` — audio.rs:932-1134 (``forward`` -> ``AudioOutput``), plus
  ``forward_batch`` (many clips, one launch sequence) and ``forward_device``
* ``log_mel`` / ``LogMel`` — the log-mel front end of
  src/media/audio_preprocess.rs:94-200 on the GPU (bit-exact with the
  reference's double-precision FFT and mel projection)
* ``AudioEmbedder`` — src/model/audio_embedder.rs:100-267, from 16 kHz samples
  (``embed``: log-mel, tower and text model without the features leaving
  HBM) or from mel spectrograms (``embed_mel``)

Compute runs only in libsvl_hip.so; there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import json
import math
from dataclasses import dataclass

import numpy as np

import svl_amd
from svl_amd import SvlError, _check, lib, tensor_views

# audio.rs:30-60; audio_preprocess.rs:34-46
MAX_AUDIO_HIDDEN = 16_384
MAX_AUDIO_INTERMEDIATE = 65_536
MAX_AUDIO_LAYERS = 128
MAX_AUDIO_HEADS = 128
MAX_AUDIO_HEAD_DIM = 1_024
MAX_AUDIO_CONV_CHANNELS = 4_096
MAX_AUDIO_OUTPUT_DIMS = 16_384
MAX_AUDIO_CONTEXT = 4_096
MAX_AUDIO_CONFIG_BYTES = 1024 * 1024
FEATURE_SIZE = 128
MAX_MEL_FRAMES = 3_000
MAX_AUDIO_SAMPLES = 480_000  # media/audio.rs:19, 30 s at 16 kHz
_BOUNDS = ("input_min", "input_max", "output_min", "output_max")


def _corrupt(m):
    return SvlError(4, m)


def _limit(m):
    return SvlError(5, m)


def _unsupported(m):
    return SvlError(6, m)


class _AudioConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int64) for n in (
        "hidden_size", "num_hidden_layers", "num_attention_heads", "conv_kernel_size",
        "conv_channels0", "conv_channels1", "attention_chunk_size", "attention_context_left",
        "attention_context_right", "output_proj_dims")] + [
        (n, ctypes.c_double) for n in ("attention_logit_cap", "rms_norm_eps", "residual_weight",
                                       "gradient_clipping")]


class _Mel(ctypes.Structure):
    _fields_ = [("features", ctypes.c_void_p), ("mask", ctypes.c_void_p),
                ("frames", ctypes.c_int64)]


class _SpecialTokens(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in ("bos", "eos", "pad", "boa", "audio", "eoa")]


def _load():
    L = lib()
    if not getattr(L, "_audio_ready", False):
        vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32
        L.svl_audio_model_create.argtypes = [vp, vp, i64, ctypes.POINTER(svl_amd._TensorView),
                                             ctypes.c_size_t, ctypes.POINTER(vp)]
        L.svl_audio_model_destroy.argtypes = [vp]
        L.svl_audio_token_count.restype = i64
        L.svl_audio_token_count.argtypes = [vp, i64]
        L.svl_audio_forward_batch.argtypes = [vp, vp, i32, vp, vp, vp, vp]
        L.svl_audio_forward_device.argtypes = [vp, vp, vp, i32, vp, vp]
        L.svl_audio_embed_batch.argtypes = [vp, vp, vp, vp, i32, i64, vp]
        L.svl_audio_embed_device.argtypes = [vp, vp, vp, vp, vp, i32, i64, vp]
        L.svl_log_mel_layout.argtypes = [i64, vp, vp, vp]
        L.svl_log_mel_create.argtypes = [vp, ctypes.POINTER(vp)]
        L.svl_log_mel_destroy.argtypes = [vp]
        L.svl_log_mel_batch.argtypes = [vp, vp, vp, i32, vp, vp]
        L.svl_log_mel_device.argtypes = [vp, vp, vp, i32, vp, vp, vp]
        L.svl_audio_embed_samples.argtypes = [vp, vp, vp, vp, vp, i32, i64, vp]
        L.svl_audio_embed_samples_device.argtypes = [vp, vp, vp, vp, vp, i32, i64, vp]
        L._audio_ready = True
    return L


class AudioConfig:
    """Validated Gemma 4 audio configuration (audio.rs:62-80)."""

    def __init__(self, **kw):
        self.__dict__.update(kw)

    @classmethod
    def from_json_str(cls, text: str) -> "AudioConfig":
        if len(text.encode()) > MAX_AUDIO_CONFIG_BYTES:
            raise _limit("audio configuration file is too large")
        try:
            value = json.loads(text)
        except json.JSONDecodeError as e:
            raise _corrupt(f"configuration is not valid JSON: {e}")
        return cls.from_json_value(value)

    @classmethod
    def from_json_value(cls, value) -> "AudioConfig":
        """audio.rs:94-294, in the reference's order of checks."""
        if not isinstance(value, dict):
            raise _corrupt("model configuration must be a JSON object")
        if "audio_config" not in value:
            raise _unsupported("the model has no audio_config; audio embeddings are unavailable")
        a = value["audio_config"]
        if not isinstance(a, dict):
            raise _corrupt("audio_config must be a JSON object")
        if "model_type" in a:
            if not isinstance(a["model_type"], str):
                raise _corrupt("audio model_type must be a string")
            if a["model_type"] != "gemma4_audio":
                raise _unsupported(f"audio model type {a['model_type']} is not gemma4_audio")
        if "dtype" in a:
            d = a["dtype"]
            if not isinstance(d, str):
                raise _corrupt("audio dtype must be a string")
            if d == "float16":
                raise _unsupported("float16 is forbidden for EmbeddingGemma 2 activations")
            if d not in ("bfloat16", "float32"):
                raise _unsupported(f"audio dtype {d} is not supported")

        def unsigned(key):
            if key not in a:
                raise _corrupt(f"audio configuration is missing {key}")
            x = a[key]
            if isinstance(x, bool) or not isinstance(x, (int, float)):
                raise _corrupt(f"{key} must be a number")
            if isinstance(x, float) or x < 0:
                raise _corrupt(f"{key} must be a non-negative integer")
            return x

        def number(key):
            x = a.get(key)
            if isinstance(x, bool) or not isinstance(x, (int, float)):
                raise _corrupt(f"{key} must be a number")
            return float(np.float32(float(x)))

        H = unsigned("hidden_size")
        L = unsigned("num_hidden_layers")
        NH = unsigned("num_attention_heads")
        K = unsigned("conv_kernel_size")
        chunk = unsigned("attention_chunk_size")
        left = unsigned("attention_context_left")
        right = unsigned("attention_context_right")
        P = unsigned("output_proj_dims")
        eps = number("rms_norm_eps")
        cap = number("attention_logit_cap")
        rw = number("residual_weight")
        clip = number("gradient_clipping")
        act = a.get("hidden_act")
        if not isinstance(act, str):
            raise _corrupt("hidden_act must be a string")
        if act != "silu":
            raise _unsupported(f"audio activation {act} is not silu")
        ucl = a.get("use_clipped_linears")
        if ucl is not None and not isinstance(ucl, bool):
            raise _corrupt("use_clipped_linears must be a boolean")
        if not ucl:
            raise _unsupported("audio clipped linear layers are required by the frozen model")
        if "attention_dropout" in a:
            drop = a["attention_dropout"]
            if isinstance(drop, bool) or not isinstance(drop, (int, float)):
                raise _corrupt("attention_dropout must be a number")
            if float(drop) != 0.0:
                raise _unsupported("audio attention dropout is not implemented")
        if H % 2:
            raise _corrupt("audio hidden size must be even for sinusoidal relative positions")
        if NH == 0 or H % NH:
            raise _corrupt("audio hidden size must be divisible by a positive head count")
        hd = H // NH
        if hd == 0 or hd > MAX_AUDIO_HEAD_DIM:
            raise _limit(f"audio head dimension {hd} is outside 1..={MAX_AUDIO_HEAD_DIM}")
        if (H > MAX_AUDIO_HIDDEN or 4 * H > MAX_AUDIO_INTERMEDIATE or L > MAX_AUDIO_LAYERS
                or NH > MAX_AUDIO_HEADS or P == 0 or P > MAX_AUDIO_OUTPUT_DIMS):
            raise _limit("audio dimensions exceed their documented caps")
        if K == 0 or K > 31:
            raise _limit(f"audio convolution kernel {K} is outside 1..=31")
        if chunk == 0 or left < 2:
            raise _corrupt("audio chunked attention requires a positive chunk and at least two "
                           "context positions on the left")
        context = chunk + left - 1 + right
        if context == 0 or context > MAX_AUDIO_CONTEXT:
            raise _limit(f"audio attention context {context} is outside 1..={MAX_AUDIO_CONTEXT}")
        if not math.isfinite(eps) or eps < 0:
            raise _corrupt("audio RMSNorm epsilon must be finite and non-negative")
        if not math.isfinite(cap) or cap <= 0:
            raise _corrupt("audio attention logit cap must be finite and positive")
        if not math.isfinite(rw):
            raise _corrupt("audio residual weight must be finite")
        if not math.isfinite(clip) or clip <= 0:
            raise _corrupt("audio gradient clipping must be finite and positive")
        ch = a.get("subsampling_conv_channels")
        if not isinstance(ch, list):
            raise _corrupt("audio subsampling_conv_channels must be an array")
        if len(ch) != 2:
            raise _unsupported("audio subsampling requires exactly two convolution channels")
        for x in ch:
            if isinstance(x, bool) or not isinstance(x, int) or x < 0:
                raise _corrupt("audio conv channel must be a non-negative integer")
        c0, c1 = ch
        if (c0 == 0 or c1 == 0 or c0 > MAX_AUDIO_CONV_CHANNELS or c1 > MAX_AUDIO_CONV_CHANNELS
                or c0 % 4):
            raise _limit("audio subsampling channels exceed their documented caps or are not "
                         "divisible by four")
        if (c0 // 4) * c1 == 0:
            raise _corrupt("audio subsampling projection has no input features")
        return cls(hidden_size=H, intermediate_size=4 * H, num_hidden_layers=L,
                   num_attention_heads=NH, head_dim=hd, conv_kernel_size=K,
                   conv_channels=(c0, c1), attention_chunk_size=chunk,
                   attention_context_left=left, attention_context_right=right,
                   attention_logit_cap=cap, rms_norm_eps=eps, output_proj_dims=P,
                   residual_weight=rw, gradient_clipping=clip)

    def context_size(self):
        return self.attention_chunk_size + self.attention_context_left - 1 + \
            self.attention_context_right

    def position_count(self):
        return self.context_size() // 2 + 1

    def subsampling_projection_input(self):
        return (self.conv_channels[0] // 4) * self.conv_channels[1]

    def tensor_shapes(self, text_hidden: int):
        """audio.rs:394-498."""
        H, I, hd = self.hidden_size, self.intermediate_size, self.head_dim
        c0, c1 = self.conv_channels
        p = "audio_tower.subsample_conv_projection."
        out = [(p + "layer0.conv.weight", (c0, 1, 3, 3)), (p + "layer0.norm.weight", (c0,)),
               (p + "layer1.conv.weight", (c1, c0, 3, 3)), (p + "layer1.norm.weight", (c1,)),
               (p + "input_proj_linear.weight", (H, self.subsampling_projection_input()))]
        for i in range(self.num_hidden_layers):
            q = f"audio_tower.layers.{i}."
            for ff in ("feed_forward1", "feed_forward2"):
                b = q + ff + "."
                out += [(b + "pre_layer_norm.weight", (H,)), (b + "post_layer_norm.weight", (H,)),
                        (b + "ffw_layer_1.linear.weight", (I, H)),
                        (b + "ffw_layer_2.linear.weight", (H, I))]
                for lin in ("ffw_layer_1", "ffw_layer_2"):
                    out += [(f"{b}{lin}.{x}", ()) for x in _BOUNDS]
            for proj in ("q_proj", "k_proj", "v_proj", "post"):
                out.append((f"{q}self_attn.{proj}.linear.weight", (H, H)))
                out += [(f"{q}self_attn.{proj}.{x}", ()) for x in _BOUNDS]
            out += [(q + "self_attn.relative_k_proj.weight", (H, H)),
                    (q + "self_attn.per_dim_scale", (hd,)),
                    (q + "lconv1d.pre_layer_norm.weight", (H,)),
                    (q + "lconv1d.linear_start.linear.weight", (2 * H, H)),
                    (q + "lconv1d.linear_end.linear.weight", (H, H))]
            for lin in ("linear_start", "linear_end"):
                out += [(f"{q}lconv1d.{lin}.{x}", ()) for x in _BOUNDS]
            out += [(q + "lconv1d.depthwise_conv1d.weight", (H, 1, self.conv_kernel_size)),
                    (q + "lconv1d.conv_norm.weight", (H,)), (q + "norm_pre_attn.weight", (H,)),
                    (q + "norm_post_attn.weight", (H,)), (q + "norm_out.weight", (H,))]
        out += [("audio_tower.output_proj.weight", (self.output_proj_dims, H)),
                ("audio_tower.output_proj.bias", (self.output_proj_dims,)),
                ("embed_audio.embedding_projection.weight", (text_hidden, self.output_proj_dims))]
        return out

    def _c(self):
        return _AudioConfig(self.hidden_size, self.num_hidden_layers, self.num_attention_heads,
                            self.conv_kernel_size, self.conv_channels[0], self.conv_channels[1],
                            self.attention_chunk_size, self.attention_context_left,
                            self.attention_context_right, self.output_proj_dims,
                            self.attention_logit_cap, self.rms_norm_eps, self.residual_weight,
                            self.gradient_clipping)


class MelSpectrogram:
    """Row-major [frames, 128] log-mel features with the frame mask
    (audio_preprocess.rs:50-90)."""

    def __init__(self, features, mask, padded_samples=None):
        self.features = np.ascontiguousarray(features, np.float32).reshape(-1, FEATURE_SIZE)
        self.mask = np.ascontiguousarray(np.asarray(mask, bool).reshape(-1).astype(np.uint8))
        if self.mask.size != self.features.shape[0]:
            raise SvlError(7, "audio mel mask does not match the frame count")
        self._padded = padded_samples

    def padded_samples(self):
        """16 kHz samples after right-padding to a multiple of 128 (None when
        the spectrogram was not computed here)."""
        return self._padded

    @property
    def frames(self):
        return int(self.mask.size)

    def valid_frames(self):
        return int(self.mask.sum())

    def audio_tokens(self):
        """Valid tokens after the two stride-2 subsamplings."""
        return int(_load().svl_audio_token_count(ctypes.c_void_p(self.mask.ctypes.data),
                                                 self.frames))

    def _c(self, with_features=True):
        return _Mel(self.features.ctypes.data if with_features else None, self.mask.ctypes.data,
                    self.frames)


def _lengths(clips):
    xs = [np.ascontiguousarray(np.asarray(c, np.float32).reshape(-1)) for c in clips]
    lengths = np.array([x.size for x in xs], np.int64)
    ptrs = (ctypes.c_void_p * max(len(xs), 1))(*[x.ctypes.data for x in xs])
    return xs, lengths, ptrs


def log_mel_layout(samples: int):
    """(frames, padded_samples, valid_frames) of a clip of `samples` 16 kHz
    samples (audio_preprocess.rs:94-131)."""
    f, p, v = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    _check(_load().svl_log_mel_layout(int(samples), ctypes.byref(f), ctypes.byref(p),
                                      ctypes.byref(v)))
    return f.value, p.value, v.value


class LogMel:
    """The log-mel front end (audio_preprocess.rs:94-200) on one device."""

    _cache = {}

    def __init__(self, device: svl_amd.Device | None = None):
        self.device = device or svl_amd.Device.get(0)
        h = ctypes.c_void_p()
        _check(_load().svl_log_mel_create(self.device.handle, ctypes.byref(h)))
        self.handle = h

    @classmethod
    def get(cls, ordinal=0):
        if ordinal not in cls._cache:
            cls._cache[ordinal] = cls(svl_amd.Device.get(ordinal))
        return cls._cache[ordinal]

    def __del__(self):
        if getattr(self, "handle", None):
            _load().svl_log_mel_destroy(self.handle)
            self.handle = None

    def compute(self, samples) -> MelSpectrogram:
        return self.compute_batch([samples])[0]

    def compute_batch(self, clips) -> list:
        xs, lengths, ptrs = _lengths(clips)
        layouts = [log_mel_layout(n) if n > 0 else (0, 0, 0) for n in lengths]
        total = sum(l[0] for l in layouts)
        feats = np.empty((max(total, 1), FEATURE_SIZE), np.float32)
        mask = np.empty(max(total, 1), np.uint8)
        _check(_load().svl_log_mel_batch(self.handle, ptrs, ctypes.c_void_p(lengths.ctypes.data),
                                         len(xs), ctypes.c_void_p(feats.ctypes.data),
                                         ctypes.c_void_p(mask.ctypes.data)))
        out, o = [], 0
        for f, p, _ in layouts:
            out.append(MelSpectrogram(feats[o:o + f].copy(), mask[o:o + f].astype(bool), p))
            o += f
        return out

    def compute_device(self, samples_dev_ptr: int, lengths, features_dev_ptr: int, stream=None):
        """Clips back to back in HBM -> features [sum frames, 128] in HBM;
        returns the host frame masks, one array per clip."""
        lengths = np.ascontiguousarray(lengths, np.int64)
        layouts = [log_mel_layout(n) if n > 0 else (0, 0, 0) for n in lengths]
        mask = np.empty(max(sum(l[0] for l in layouts), 1), np.uint8)
        _check(_load().svl_log_mel_device(self.handle, ctypes.c_void_p(samples_dev_ptr),
                                          ctypes.c_void_p(lengths.ctypes.data), len(lengths),
                                          ctypes.c_void_p(features_dev_ptr),
                                          ctypes.c_void_p(mask.ctypes.data),
                                          ctypes.c_void_p(stream) if stream else None))
        out, o = [], 0
        for f, _, _ in layouts:
            out.append(mask[o:o + f].astype(bool))
            o += f
        return out


def log_mel(samples) -> MelSpectrogram:
    """log_mel (audio_preprocess.rs:94-200) of 16 kHz mono samples on device 0."""
    return LogMel.get(0).compute(samples)


class AudioOutput:
    """audio.rs:893-930."""

    def __init__(self, pooled, hidden_states, sscp_output, audio_tokens, text_hidden):
        self._pooled, self._hidden, self._sscp = pooled, hidden_states, sscp_output
        self._tokens, self._text_hidden = audio_tokens, text_hidden

    def pooled(self):
        return self._pooled

    def hidden_states(self):
        return self._hidden

    def sscp_output(self):
        return self._sscp

    def audio_tokens(self):
        return self._tokens

    def text_hidden(self):
        return self._text_hidden


def _mels(mels, with_features=True):
    structs = [m._c(with_features) for m in mels]
    keep = [x for m in mels for x in (m.features, m.mask)]
    return (_Mel * max(len(structs), 1))(*structs), keep


class AudioModel:
    """The reference AudioModel (audio.rs:932-1134) with its forward pass on the GPU."""

    def __init__(self, config: AudioConfig, weights: dict, text_hidden: int,
                 device: svl_amd.Device | None = None):
        self.config = config
        self.text_hidden = int(text_hidden)
        self.device = device or svl_amd.Device.get(0)
        arr, n, keep = tensor_views(weights)  # alive until the library has copied them
        cfg = config._c()
        h = ctypes.c_void_p()
        _check(_load().svl_audio_model_create(self.device.handle, ctypes.byref(cfg),
                                              self.text_hidden, arr, n, ctypes.byref(h)))
        self.handle = h

    def close(self):
        if getattr(self, "handle", None):
            _load().svl_audio_model_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def forward(self, mel: MelSpectrogram, capture_hidden=False) -> AudioOutput:
        """audio.rs:981-1134."""
        return self.forward_batch([mel], capture_hidden)[0]

    def forward_batch(self, mels, capture_hidden=False):
        arr, keep = _mels(mels)
        toks = [m.audio_tokens() for m in mels]
        N, H, L = sum(toks), self.config.hidden_size, self.config.num_hidden_layers
        counts = np.zeros(max(len(mels), 1), np.int64)
        soft = np.empty((max(N, 1), self.text_hidden), np.float32)
        sscp = np.empty((max(N, 1), H), np.float32) if capture_hidden else None
        hidden = np.empty((max(L, 1), max(N, 1), H), np.float32) if capture_hidden else None
        _check(_load().svl_audio_forward_batch(
            self.handle, arr, len(mels), ctypes.c_void_p(counts.ctypes.data),
            ctypes.c_void_p(soft.ctypes.data),
            None if sscp is None else ctypes.c_void_p(sscp.ctypes.data),
            None if hidden is None else ctypes.c_void_p(hidden.ctypes.data)))
        out, t0 = [], 0
        for i, m in enumerate(mels):
            n = int(counts[i])
            hs = [hidden[l, t0:t0 + n].copy() for l in range(L)] if capture_hidden else None
            out.append(AudioOutput(soft[t0:t0 + n].copy(), hs,
                                   sscp[t0:t0 + n].copy() if capture_hidden else None, n,
                                   self.text_hidden))
            t0 += n
        return out

    def forward_device(self, features_dev_ptr: int, mels, out_dev_ptr: int, stream=0):
        """Mel frames already in HBM ([sum frames, 128]); soft tokens written
        to HBM [sum tokens, text_hidden]."""
        arr, keep = _mels(mels, with_features=False)
        _check(_load().svl_audio_forward_device(self.handle, ctypes.c_void_p(features_dev_ptr),
                                                arr, len(mels), ctypes.c_void_p(out_dev_ptr),
                                                ctypes.c_void_p(stream) if stream else None))


@dataclass(frozen=True)
class AudioSpecialTokens:
    """audio_embedder.rs:32-46 (defaults: tests/audio_embeddings.rs:100-107)."""
    bos: int = 2
    eos: int = 1
    pad: int = 0
    boa: int = 256_000
    audio: int = 258_881
    eoa: int = 258_883

    def _c(self):
        return _SpecialTokens(self.bos, self.eos, self.pad, self.boa, self.audio, self.eoa)


class AudioEmbedder:
    """AudioEmbedder (audio_embedder.rs:100-267) over log-mel spectrograms:
    the tower, the audio-only prompt and the text encoder with the soft
    tokens substituted, kept in HBM between the two models."""

    def __init__(self, model: svl_amd.TextModel, audio: AudioModel,
                 tokens: AudioSpecialTokens = AudioSpecialTokens()):
        self.model, self.audio, self.tokens = model, audio, tokens

    def special_tokens(self):
        return self.tokens

    def embed(self, samples, dimension: int):
        """AudioEmbedder::embed (audio_embedder.rs:214-267) of 16 kHz mono
        samples: log-mel, tower and text model on the device."""
        return self.embed_samples_batch([samples], dimension)[0]

    def embed_samples_batch(self, clips, dimension: int):
        xs, lengths, ptrs = _lengths(clips)
        out = np.empty((max(len(xs), 1), int(dimension)), np.float32)
        tok = self.tokens._c()
        _check(_load().svl_audio_embed_samples(self.audio.handle, self.model.handle,
                                               ctypes.byref(tok), ptrs,
                                               ctypes.c_void_p(lengths.ctypes.data), len(xs),
                                               int(dimension), ctypes.c_void_p(out.ctypes.data)))
        return out[: len(xs)]

    def embed_samples_device(self, samples_dev_ptr: int, lengths, dimension: int):
        lengths = np.ascontiguousarray(lengths, np.int64)
        out = np.empty((max(len(lengths), 1), int(dimension)), np.float32)
        tok = self.tokens._c()
        _check(_load().svl_audio_embed_samples_device(
            self.audio.handle, self.model.handle, ctypes.byref(tok),
            ctypes.c_void_p(samples_dev_ptr), ctypes.c_void_p(lengths.ctypes.data), len(lengths),
            int(dimension), ctypes.c_void_p(out.ctypes.data)))
        return out[: len(lengths)]

    def embed_mel(self, mel: MelSpectrogram, dimension: int):
        return self.embed_batch([mel], dimension)[0]

    def embed_batch(self, mels, dimension: int):
        arr, keep = _mels(mels)
        out = np.empty((max(len(mels), 1), int(dimension)), np.float32)
        tok = self.tokens._c()
        _check(_load().svl_audio_embed_batch(self.audio.handle, self.model.handle,
                                             ctypes.byref(tok), arr, len(mels), int(dimension),
                                             ctypes.c_void_p(out.ctypes.data)))
        return out[: len(mels)]

    def embed_device(self, features_dev_ptr: int, mels, dimension: int):
        arr, keep = _mels(mels, with_features=False)
        out = np.empty((max(len(mels), 1), int(dimension)), np.float32)
        tok = self.tokens._c()
        _check(_load().svl_audio_embed_device(self.audio.handle, self.model.handle,
                                              ctypes.byref(tok), ctypes.c_void_p(features_dev_ptr),
                                              arr, len(mels), int(dimension),
                                              ctypes.c_void_p(out.ctypes.data)))
        return out[: len(mels)]
