"""Vision tower and image embedder on the MI355X backend, shaped like the
reference crate's API:

* ``VisionConfig.from_json_str`` — the strict parser of src/model/vision.rs:84-273
* ``ImagePatches`` — the preprocessed image of src/media/preprocess.rs:87-147
* ``VisionModel`` — vision.rs:686-959 (``forward`` -> ``VisionOutput``), plus
  ``forward_batch`` (many images, one launch sequence) and ``forward_device``
* ``ImageEmbedder`` — src/model/image.rs:100-253 over ``ImagePatches``
  (decoding and resizing images is preprocessing, not part of this backend)

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

# vision.rs:29-56; media/preprocess.rs:22-43
MAX_VISION_HIDDEN = 16_384
MAX_VISION_INTERMEDIATE = 65_536
MAX_VISION_LAYERS = 128
MAX_VISION_HEADS = 128
MAX_VISION_HEAD_DIM = 1_024
MAX_POSITION_EMBEDDINGS = 1_048_576
MAX_VISION_CONFIG_BYTES = 1024 * 1024
PATCH_SIZE = 16
POOLING_KERNEL_SIZE = 3
PATCH_VALUES = PATCH_SIZE * PATCH_SIZE * 3
MAX_PATCHES = 1120 * POOLING_KERNEL_SIZE * POOLING_KERNEL_SIZE
# media/preprocess.rs: 1/255 evaluated in f32
RESCALE_FACTOR = np.float32(1.0) / np.float32(255.0)


def _corrupt(m):
    return SvlError(4, m)


def _limit(m):
    return SvlError(5, m)


def _unsupported(m):
    return SvlError(6, m)


class _VisionConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int64) for n in (
        "hidden_size", "intermediate_size", "num_hidden_layers", "num_attention_heads",
        "num_key_value_heads", "head_dim", "position_embedding_size")] + [
        ("rms_norm_eps", ctypes.c_double), ("rope_theta", ctypes.c_double)]


class _ImagePatches(ctypes.Structure):
    _fields_ = [("pixel_values", ctypes.c_void_p), ("positions", ctypes.c_void_p),
                ("valid_patches", ctypes.c_int64), ("max_patches", ctypes.c_int64),
                ("grid_width", ctypes.c_int64), ("grid_height", ctypes.c_int64),
                ("soft_tokens", ctypes.c_int64)]


class _SpecialTokens(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in ("bos", "eos", "pad", "boi", "image", "eoi")]


class VisionConfig:
    """Validated Gemma 4 vision configuration (vision.rs:58-70)."""

    def __init__(self, **kw):
        self.__dict__.update(kw)

    @classmethod
    def from_json_str(cls, text: str) -> "VisionConfig":
        if len(text.encode()) > MAX_VISION_CONFIG_BYTES:
            raise _limit("vision configuration file is too large")
        try:
            value = json.loads(text)
        except json.JSONDecodeError as e:
            raise _corrupt(f"configuration is not valid JSON: {e}")
        return cls.from_json_value(value)

    @classmethod
    def from_json_value(cls, value) -> "VisionConfig":
        """vision.rs:84-273, in the reference's order of checks."""
        if not isinstance(value, dict):
            raise _corrupt("model configuration must be a JSON object")
        if "vision_config" not in value:
            raise _unsupported("the model has no vision_config; image embeddings are unavailable")
        v = value["vision_config"]
        if not isinstance(v, dict):
            raise _corrupt("vision_config must be a JSON object")
        if "model_type" in v:
            if not isinstance(v["model_type"], str):
                raise _corrupt("vision model_type must be a string")
            if v["model_type"] != "gemma4_vision":
                raise _unsupported(f"vision model type {v['model_type']} is not gemma4_vision")
        if "dtype" in v:
            d = v["dtype"]
            if not isinstance(d, str):
                raise _corrupt("vision dtype must be a string")
            if d == "float16":
                raise _unsupported("float16 is forbidden for EmbeddingGemma 2 activations")
            if d not in ("bfloat16", "float32"):
                raise _unsupported(f"vision dtype {d} is not supported")

        def unsigned(key):
            if key not in v:
                raise _corrupt(f"vision configuration is missing {key}")
            x = v[key]
            if isinstance(x, bool) or not isinstance(x, (int, float)):
                raise _corrupt(f"{key} must be a number")
            if isinstance(x, float) or x < 0:
                raise _corrupt(f"{key} must be a non-negative integer")
            return x

        def number(obj, key, what=None):
            x = obj.get(key)
            if isinstance(x, bool) or not isinstance(x, (int, float)):
                raise _corrupt(what or f"{key} must be a number")
            return float(x)

        def opt_bool(key):
            if key not in v:
                return None
            if not isinstance(v[key], bool):
                raise _corrupt(f"{key} must be a boolean")
            return v[key]

        H = unsigned("hidden_size")
        I = unsigned("intermediate_size")
        L = unsigned("num_hidden_layers")
        NH = unsigned("num_attention_heads")
        KV = unsigned("num_key_value_heads")
        HD = unsigned("head_dim")
        PS = unsigned("patch_size")
        PK = unsigned("pooling_kernel_size")
        POS = unsigned("position_embedding_size")
        eps = number(v, "rms_norm_eps")
        eps32 = float(np.float32(eps))
        if not math.isfinite(eps32) or eps32 < 0:
            raise _corrupt("vision RMSNorm epsilon must be finite and non-negative")
        act = v.get("hidden_activation")
        if not isinstance(act, str):
            raise _corrupt("hidden_activation must be a string")
        if act != "gelu_pytorch_tanh":
            raise _unsupported(f"vision activation {act} is not gelu_pytorch_tanh")
        if opt_bool("attention_bias"):
            raise _unsupported("vision attention bias is not part of the frozen model")
        if "attention_dropout" in v:
            drop = v["attention_dropout"]
            if isinstance(drop, bool) or not isinstance(drop, (int, float)):
                raise _corrupt("attention_dropout must be a number")
            if float(drop) != 0.0:
                raise _unsupported("vision attention dropout is not implemented")
        if opt_bool("use_clipped_linears"):
            raise _unsupported("clipped vision linear layers are not part of the frozen model")
        if opt_bool("standardize"):
            raise _unsupported("vision feature standardization is not part of the frozen model")
        if PS != PATCH_SIZE:
            raise _unsupported(f"vision patch size {PS} is not the frozen {PATCH_SIZE}")
        if PK != POOLING_KERNEL_SIZE:
            raise _unsupported(f"vision pooling kernel {PK} is not the frozen {POOLING_KERNEL_SIZE}")
        if HD == 0 or HD % 4:
            raise _unsupported("vision head dimension must be positive and divisible by four for axial RoPE")
        if NH == 0 or KV == 0:
            raise _corrupt("vision attention head counts must be positive")
        if NH % KV:
            raise _corrupt("vision query head count is not a multiple of the key/value head count")
        if H > MAX_VISION_HIDDEN or NH * HD > MAX_VISION_HIDDEN or KV * HD > MAX_VISION_HIDDEN:
            raise _limit(f"vision dimensions exceed the {MAX_VISION_HIDDEN}-element hidden cap")
        if I > MAX_VISION_INTERMEDIATE:
            raise _limit(f"vision intermediate size {I} exceeds the {MAX_VISION_INTERMEDIATE} cap")
        if L > MAX_VISION_LAYERS:
            raise _limit(f"vision layer count {L} exceeds the {MAX_VISION_LAYERS} cap")
        if NH > MAX_VISION_HEADS or HD > MAX_VISION_HEAD_DIM:
            raise _limit("vision attention layout exceeds its documented cap")
        if POS == 0 or POS > MAX_POSITION_EMBEDDINGS:
            raise _limit(f"vision position table size {POS} is outside 1..={MAX_POSITION_EMBEDDINGS}")
        rope = v.get("rope_parameters")
        if not isinstance(rope, dict):
            raise _corrupt("vision rope_parameters must be an object")
        rt = rope.get("rope_type")
        if not isinstance(rt, str):
            raise _corrupt("vision rope_type must be a string")
        if rt != "axial":
            raise _unsupported(f"vision RoPE type {rt} is not axial")
        theta = number(rope, "rope_theta", "vision rope_theta must be a number")
        theta32 = float(np.float32(theta))
        if not math.isfinite(theta32) or theta32 <= 0.0:
            raise _corrupt("vision RoPE theta must be finite and positive")
        return cls(hidden_size=H, intermediate_size=I, num_hidden_layers=L,
                   num_attention_heads=NH, num_key_value_heads=KV, head_dim=HD,
                   patch_size=PS, pooling_kernel_size=PK, position_embedding_size=POS,
                   rms_norm_eps=eps32, rope_theta=theta32)

    @property
    def query_dim(self):
        return self.num_attention_heads * self.head_dim

    @property
    def key_value_dim(self):
        return self.num_key_value_heads * self.head_dim

    def tensor_shapes(self, text_hidden: int):
        """vision.rs:345-414."""
        H, I, hd = self.hidden_size, self.intermediate_size, self.head_dim
        out = [("vision_tower.patch_embedder.input_proj.weight", (H, PATCH_VALUES)),
               ("vision_tower.patch_embedder.position_embedding_table",
                (2, self.position_embedding_size, H))]
        for i in range(self.num_hidden_layers):
            p = f"vision_tower.encoder.layers.{i}."
            out += [(p + "input_layernorm.weight", (H,)),
                    (p + "post_attention_layernorm.weight", (H,)),
                    (p + "pre_feedforward_layernorm.weight", (H,)),
                    (p + "post_feedforward_layernorm.weight", (H,)),
                    (p + "self_attn.q_proj.linear.weight", (self.query_dim, H)),
                    (p + "self_attn.k_proj.linear.weight", (self.key_value_dim, H)),
                    (p + "self_attn.v_proj.linear.weight", (self.key_value_dim, H)),
                    (p + "self_attn.o_proj.linear.weight", (H, self.query_dim)),
                    (p + "self_attn.q_norm.weight", (hd,)),
                    (p + "self_attn.k_norm.weight", (hd,)),
                    (p + "mlp.gate_proj.linear.weight", (I, H)),
                    (p + "mlp.up_proj.linear.weight", (I, H)),
                    (p + "mlp.down_proj.linear.weight", (H, I))]
        out.append(("embed_vision.embedding_projection.weight", (text_hidden, H)))
        return out

    def _c(self):
        return _VisionConfig(self.hidden_size, self.intermediate_size, self.num_hidden_layers,
                             self.num_attention_heads, self.num_key_value_heads, self.head_dim,
                             self.position_embedding_size, self.rms_norm_eps, self.rope_theta)


class ImagePatches:
    """A preprocessed image (media/preprocess.rs:87-147): padded patch
    values [max_patches, 768] and (x, y) grid positions, of which the first
    valid_patches rows are real (padding rows carry position (-1, -1))."""

    def __init__(self, pixel_values, positions, valid_patches, soft_tokens, max_patches,
                 patch_grid):
        self.pixel_values = np.ascontiguousarray(pixel_values, np.float32).reshape(-1, PATCH_VALUES)
        self.positions = np.ascontiguousarray(positions, np.int32).reshape(-1, 2)
        self.valid_patches = int(valid_patches)
        self.soft_tokens = int(soft_tokens)
        self.max_patches = int(max_patches)
        self.patch_grid = (int(patch_grid[0]), int(patch_grid[1]))

    @classmethod
    def from_grid(cls, pixel_values, grid_width, grid_height, max_patches=None):
        """Patches of a grid_width x grid_height image in the reference's row-major
        patch order (preprocess.rs:217-242): patch y * grid_width + x at (x, y)."""
        valid = grid_width * grid_height
        max_patches = valid if max_patches is None else max_patches
        pix = np.zeros((max_patches, PATCH_VALUES), np.float32)
        pix[:valid] = np.asarray(pixel_values, np.float32).reshape(valid, PATCH_VALUES)
        pos = np.full((max_patches, 2), -1, np.int32)
        ys, xs = np.divmod(np.arange(valid), grid_width)
        pos[:valid, 0], pos[:valid, 1] = xs, ys
        pooled = POOLING_KERNEL_SIZE * POOLING_KERNEL_SIZE
        return cls(pix, pos, valid, valid // pooled, max_patches, (grid_width, grid_height))

    def _c(self, with_pixels=True):
        keep = [self.pixel_values, self.positions]
        return _ImagePatches(self.pixel_values.ctypes.data if with_pixels else None,
                             self.positions.ctypes.data, self.valid_patches, self.max_patches,
                             self.patch_grid[0], self.patch_grid[1], self.soft_tokens), keep


class VisionOutput:
    """vision.rs:638-676."""

    def __init__(self, pooled, hidden_states, soft_tokens, text_hidden):
        self._pooled, self._hidden = pooled, hidden_states
        self._soft, self._text_hidden = soft_tokens, text_hidden

    def pooled(self):
        return self._pooled

    def hidden_states(self):
        return self._hidden

    def soft_tokens(self):
        return self._soft

    def text_hidden(self):
        return self._text_hidden


def _images(patches_list, with_pixels=True):
    keep = []
    structs = []
    for p in patches_list:
        c, k = p._c(with_pixels)
        structs.append(c)
        keep += k
    return (_ImagePatches * max(len(structs), 1))(*structs), keep


class VisionModel:
    """The reference VisionModel (vision.rs:686-959) with its forward pass on the GPU."""

    def __init__(self, config: VisionConfig, weights: dict, text_hidden: int,
                 device: svl_amd.Device | None = None):
        self.config = config
        self.text_hidden = int(text_hidden)
        self.device = device or svl_amd.Device.get(0)
        arr, n, keep = tensor_views(weights)  # alive until the library has copied them
        cfg = config._c()
        h = ctypes.c_void_p()
        _check(lib().svl_vision_model_create(self.device.handle, ctypes.byref(cfg),
                                             self.text_hidden, arr, n, ctypes.byref(h)))
        self.handle = h

    def close(self):
        if getattr(self, "handle", None):
            lib().svl_vision_model_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_stream_split(self, groups):
        """Image groups of a batch's encoder layers on concurrent streams (1 or
        2; results are bit-identical either way)."""
        g = 2 if groups is True else 1 if groups is False else int(groups)
        _check(lib().svl_vision_model_set_stream_split(self.handle, g))

    def set_pass_patches(self, patches: int):
        """Largest pass of consecutive images a batch runs in, in real
        patches (0: sized to about 32 GiB of device workspace); results do not
        depend on it."""
        _check(lib().svl_vision_model_set_pass_patches(self.handle, int(patches)))

    def forward(self, patches: ImagePatches, capture_hidden=False) -> VisionOutput:
        """vision.rs:742-959."""
        return self.forward_batch([patches], capture_hidden)[0]

    def forward_batch(self, patches_list, capture_hidden=False):
        """One VisionOutput per image, all images in one launch sequence."""
        arr, keep = _images(patches_list)
        S = sum(p.soft_tokens for p in patches_list)
        T = sum(p.valid_patches for p in patches_list)
        soft = np.empty((max(S, 1), self.text_hidden), np.float32)
        L, H = self.config.num_hidden_layers, self.config.hidden_size
        hidden = np.empty((L + 1, max(T, 1), H), np.float32) if capture_hidden else None
        _check(lib().svl_vision_forward_batch(
            self.handle, arr, len(patches_list), ctypes.c_void_p(soft.ctypes.data),
            None if hidden is None else ctypes.c_void_p(hidden.ctypes.data)))
        out, s0, t0 = [], 0, 0
        for p in patches_list:
            hs = None
            if capture_hidden:
                hs = [hidden[l, t0:t0 + p.valid_patches].copy() for l in range(L + 1)]
            out.append(VisionOutput(soft[s0:s0 + p.soft_tokens].copy(), hs, p.soft_tokens,
                                    self.text_hidden))
            s0 += p.soft_tokens
            t0 += p.valid_patches
        return out

    def forward_device(self, pixels_dev_ptr: int, patches_list, out_dev_ptr: int, stream=0):
        """Patches already in HBM ([sum valid, 768], rescaled in place);
        soft tokens written to HBM [sum soft, text_hidden]."""
        arr, keep = _images(patches_list, with_pixels=False)
        _check(lib().svl_vision_forward_device(self.handle, ctypes.c_void_p(pixels_dev_ptr), arr,
                                               len(patches_list), ctypes.c_void_p(out_dev_ptr),
                                               ctypes.c_void_p(stream) if stream else None))


@dataclass(frozen=True)
class ImageSpecialTokens:
    """image.rs:30-44."""
    bos: int = 2
    eos: int = 1
    pad: int = 0
    boi: int = 255_999
    image: int = 258_880
    eoi: int = 258_882

    def _c(self):
        return _SpecialTokens(self.bos, self.eos, self.pad, self.boi, self.image, self.eoi)


class ImageEmbedder:
    """ImageEmbedder (image.rs:100-253) over preprocessed patches: the vision
    tower, the image-only prompt and the text encoder with the soft tokens
    substituted, kept in HBM between the two models."""

    def __init__(self, model: svl_amd.TextModel, vision: VisionModel,
                 tokens: ImageSpecialTokens = ImageSpecialTokens()):
        self.model, self.vision, self.tokens = model, vision, tokens

    def special_tokens(self):
        return self.tokens

    def embed_patches(self, patches: ImagePatches, dimension: int):
        return self.embed_batch([patches], dimension)[0]

    def embed_batch(self, patches_list, dimension: int):
        arr, keep = _images(patches_list)
        out = np.empty((max(len(patches_list), 1), int(dimension)), np.float32)
        tok = self.tokens._c()
        _check(lib().svl_image_embed_batch(self.vision.handle, self.model.handle,
                                           ctypes.byref(tok), arr, len(patches_list),
                                           int(dimension), ctypes.c_void_p(out.ctypes.data)))
        return out[: len(patches_list)]

    def embed_device(self, pixels_dev_ptr: int, patches_list, dimension: int):
        """embed_batch with the patches already in HBM ([sum valid, 768],
        rescaled in place); returns [batch, dimension] on the host."""
        arr, keep = _images(patches_list, with_pixels=False)
        out = np.empty((max(len(patches_list), 1), int(dimension)), np.float32)
        tok = self.tokens._c()
        _check(lib().svl_image_embed_device(self.vision.handle, self.model.handle,
                                            ctypes.byref(tok), ctypes.c_void_p(pixels_dev_ptr),
                                            arr, len(patches_list), int(dimension),
                                            ctypes.c_void_p(out.ctypes.data)))
        return out[: len(patches_list)]
