"""Deterministic synthetic EmbeddingGemma-2 text models and inputs.

Shape A is the headline benchmark shape (hidden 768, 3 query heads sharing
one KV head of dim 256, GeGLU FFN 1152, 24 layers, vocab 262144, PLE 256);
shape B is the reference's frozen manifest shape (fixtures/model/
manifest.json:137-204: hidden 512, 4 heads, 2 KV heads of dim 256 on sliding
layers and 1 of dim 512 on full layers 5/11/17/23, FFN 2048, PLE 512). Both
are legal configurations of the reference's TextConfig (config.rs:112-269).

Weights come from the library's counter-based SplitMix64 generator, one
stream per tensor in TextConfig::tensor_shapes order:
  linear [out, in]        U(-sqrt(3/in), +sqrt(3/in))
  embed_tokens            U(-sqrt(3/H), +sqrt(3/H))   (rms ~ 1 after x sqrt(H))
  RMSNorm weights         1 + U(-0.1, 0.1)
  q_norm, k_norm          U(0.2, 0.3)   (score std ~ 1 at head_dim 256, scale 1.0)
  layer_scalar            U(0.5, 1.0)
Inputs: token ids floor(u * vocab) (seed, stream 0); row lengths
lo + floor(u * (hi - lo + 1)) (seed, stream 1).
"""
from __future__ import annotations

import json
import math

import numpy as np

import svl_amd


def _layer_types(n, every=6):
    """Five sliding layers then one full layer, repeated; the last layer is
    always full (config.rs:647-649)."""
    return ["full_attention" if (i + 1) % every == 0 or i == n - 1 else "sliding_attention"
            for i in range(n)]


def config_a(layers=24, vocab=262144) -> dict:
    return {"model_type": "embedding_gemma2_text", "dtype": "float32", "vocab_size": vocab,
            "hidden_size": 768, "intermediate_size": 1152, "num_hidden_layers": layers,
            "num_attention_heads": 3, "num_key_value_heads": 1, "head_dim": 256,
            "hidden_size_per_layer_input": 256, "embedding_dim": 768,
            "hidden_activation": "gelu_pytorch_tanh", "max_position_embeddings": 8192,
            "rms_norm_eps": 1e-06, "pad_token_id": 0, "bos_token_id": 2, "eos_token_id": 1,
            "attention_bias": False, "attention_dropout": 0.0, "sliding_window": 512,
            "layer_types": _layer_types(layers),
            "rope_parameters": {"full_attention": {"rope_theta": 1000000.0, "rope_type": "default"},
                                "sliding_attention": {"rope_theta": 10000.0, "rope_type": "default"}}}


def config_b(layers=24, vocab=262144) -> dict:
    c = config_a(layers, vocab)
    c.update(hidden_size=512, intermediate_size=2048, num_attention_heads=4, num_key_value_heads=2,
             head_dim=256, hidden_size_per_layer_input=512)
    c["per_layer_config"] = {f"{i:02d}": {"head_dim": 512, "num_key_value_heads": 1}
                             for i, t in enumerate(c["layer_types"]) if t == "full_attention"}
    return c


def weights(config: dict, seed: int = 0) -> dict:
    """name -> float32 array for every tensor of the config."""
    cfg = svl_amd.TextConfig.from_json_value(config)
    H = cfg.hidden_size
    out = {}
    for stream, (name, shape) in enumerate(cfg.tensor_shapes()):
        n = int(np.prod(shape))
        if name.endswith("embed_tokens.weight"):
            b = math.sqrt(3.0 / H)
            lo, hi = -b, b
        elif name.endswith("layer_scalar"):
            lo, hi = 0.5, 1.0
        elif name.endswith("q_norm.weight") or name.endswith("k_norm.weight"):
            lo, hi = 0.2, 0.3
        elif len(shape) == 1:
            lo, hi = 0.9, 1.1
        else:
            b = math.sqrt(3.0 / shape[1])
            lo, hi = -b, b
        out[name] = svl_amd.synth_uniform(seed, stream, lo, hi, n).reshape(shape)
    return out


def token_rows(vocab: int, lengths, seed: int = 1):
    """Rows of uniform token ids, one id stream shared across rows."""
    lengths = [int(x) for x in lengths]
    ids = svl_amd.synth_ids(seed, 0, vocab, int(sum(lengths)))
    rows, a = [], 0
    for n in lengths:
        rows.append(ids[a:a + n])
        a += n
    return rows


def row_lengths(batch: int, lo: int, hi: int, seed: int = 1):
    return svl_amd.synth_lengths(seed, 1, lo, hi, batch)


def dumps(config: dict) -> str:
    return json.dumps(config)


# ---- vision tower -------------------------------------------------------------
#
# Config V is the frozen gemma4_vision shape (docs/architecture.md:553-558:
# hidden 768, 16 layers, 12 heads of dim 64, FFN 3072, axial theta 100, eps
# 1e-6, patch 16, pool 3). position_embedding_size is not stated there; 10240
# entries per axis covers every patch grid the preprocessing can produce and
# only sets the size of the position table. Weights, one SplitMix64 stream per
# tensor in VisionConfig::tensor_shapes order after an offset of 100000:
#   linear [out, in]        U(-sqrt(3/in), +sqrt(3/in))
#   position table          U(-0.5, 0.5)
#   RMSNorm weights         1 + U(-0.1, 0.1)
#   q_norm, k_norm          U(0.3, 0.4)   (score std ~ 1 at head_dim 64, scale 1.0)
# Images: uint8 uniform noise rescaled by 1/255 (as preprocess.rs does),
# generated directly per patch value (iid noise, so the patch cut does not
# change the distribution).

VISION_STREAM_BASE = 100_000


def config_v(layers=16, text=None) -> dict:
    """Composite config: text config (shape A by default) plus vision_config V."""
    c = {"text_config": text or config_a()}
    c["vision_config"] = {
        "model_type": "gemma4_vision", "dtype": "float32", "hidden_size": 768,
        "intermediate_size": 3072, "num_hidden_layers": layers, "num_attention_heads": 12,
        "num_key_value_heads": 12, "head_dim": 64, "patch_size": 16, "pooling_kernel_size": 3,
        "position_embedding_size": 10240, "rms_norm_eps": 1e-06,
        "hidden_activation": "gelu_pytorch_tanh", "attention_bias": False,
        "attention_dropout": 0.0, "use_clipped_linears": False, "standardize": False,
        "rope_parameters": {"rope_type": "axial", "rope_theta": 100.0}}
    return c


def vision_weights(config: dict, text_hidden: int, seed: int = 0) -> dict:
    import svl_vision
    vc = svl_vision.VisionConfig.from_json_value(config)
    out = {}
    for k, (name, shape) in enumerate(vc.tensor_shapes(text_hidden)):
        n = int(np.prod(shape))
        if name.endswith("position_embedding_table"):
            lo, hi = -0.5, 0.5
        elif name.endswith("q_norm.weight") or name.endswith("k_norm.weight"):
            lo, hi = 0.3, 0.4
        elif len(shape) == 1:
            lo, hi = 0.9, 1.1
        else:
            b = math.sqrt(3.0 / shape[-1])
            lo, hi = -b, b
        out[name] = svl_amd.synth_uniform(seed, VISION_STREAM_BASE + k, lo, hi, n).reshape(shape)
    return out


def image_patches(batch: int, grid_width: int = 48, grid_height: int = 48, seed: int = 2,
                  max_patches: int | None = None):
    """`batch` noise images of grid_width x grid_height patches (768 x 768
    pixels at the default 48 x 48), one id stream per image."""
    import svl_vision
    out = []
    valid = grid_width * grid_height
    for i in range(batch):
        u8 = svl_amd.synth_ids(seed, 10 + i, 256, valid * svl_vision.PATCH_VALUES)
        pix = u8.astype(np.float32) * svl_vision.RESCALE_FACTOR
        out.append(svl_vision.ImagePatches.from_grid(pix, grid_width, grid_height, max_patches))
    return out


# ---- audio tower --------------------------------------------------------------
#
# Config AU is the frozen gemma4_audio shape (docs/architecture.md:566-578:
# hidden 1024, 12 layers, 8 heads, conv kernel 5, SSCP channels [128, 32],
# chunk 12, left context 13, right 0, logit cap 50, output projection 1536,
# residual weight 0.5, clipping 1e10, SiLU). Weights, one SplitMix64 stream
# per tensor in AudioConfig::tensor_shapes order after an offset of 200000:
#   linear / conv weights   U(-sqrt(3/fan_in), +sqrt(3/fan_in))
#   RMSNorm / LayerNorm     1 + U(-0.1, 0.1)
#   per_dim_scale           U(-0.5, 0.5)
#   output_proj bias        U(-0.1, 0.1)
#   clipping bounds         input/output min -U(2.5, 4), max +U(2.5, 4)
# Mel input: log-mel-shaped frames U(-7, 2) per bin (one stream per clip),
# every frame valid unless a mask is given; 30 s at 16 kHz is 2999 frames.

AUDIO_STREAM_BASE = 200_000


def config_au(layers=12, text=None) -> dict:
    c = {"text_config": text or config_a()}
    c["audio_config"] = {
        "model_type": "gemma4_audio", "dtype": "float32", "hidden_size": 1024,
        "num_hidden_layers": layers, "num_attention_heads": 8, "conv_kernel_size": 5,
        "subsampling_conv_channels": [128, 32], "attention_chunk_size": 12,
        "attention_context_left": 13, "attention_context_right": 0,
        "attention_logit_cap": 50.0, "rms_norm_eps": 1e-06, "output_proj_dims": 1536,
        "residual_weight": 0.5, "gradient_clipping": 1e10, "hidden_act": "silu",
        "use_clipped_linears": True, "attention_invalid_logits_value": -1e9}
    return c


def audio_weights(config: dict, text_hidden: int, seed: int = 0) -> dict:
    import svl_audio
    ac = svl_audio.AudioConfig.from_json_value(config)
    out = {}
    for k, (name, shape) in enumerate(ac.tensor_shapes(text_hidden)):
        n = int(np.prod(shape)) if shape else 1
        stream = AUDIO_STREAM_BASE + k
        if name.endswith(("input_min", "output_min")):
            v = -svl_amd.synth_uniform(seed, stream, 2.5, 4.0, 1)
        elif name.endswith(("input_max", "output_max")):
            v = svl_amd.synth_uniform(seed, stream, 2.5, 4.0, 1)
        elif name.endswith("per_dim_scale"):
            v = svl_amd.synth_uniform(seed, stream, -0.5, 0.5, n)
        elif name.endswith("output_proj.bias"):
            v = svl_amd.synth_uniform(seed, stream, -0.1, 0.1, n)
        elif len(shape) == 1:
            v = svl_amd.synth_uniform(seed, stream, 0.9, 1.1, n)
        else:
            fan_in = int(np.prod(shape[1:]))
            b = math.sqrt(3.0 / fan_in)
            v = svl_amd.synth_uniform(seed, stream, -b, b, n)
        out[name] = np.asarray(v, np.float32).reshape(shape)
    return out


def sine_clips(n_clip: int, seed: int = 3, seconds: float = 30.0, rate: int = 16000):
    """Synthetic 16 kHz mono clips: per clip, three sines of amplitude 0.3 at
    frequencies uniform in [100, 4000) Hz plus Gaussian noise of sigma 0.05,
    drawn from numpy default_rng(seed) clip by clip (3 frequencies, then the
    noise)."""
    rng = np.random.default_rng(seed)
    t = np.arange(int(seconds * rate), dtype=np.float64) / rate
    clips = []
    for _ in range(n_clip):
        f = rng.uniform(100.0, 4000.0, 3)
        x = 0.3 * np.sin(2 * np.pi * f[:, None] * t[None, :]).sum(axis=0)
        x += rng.normal(0.0, 0.05, t.size)
        clips.append(x.astype(np.float32))
    return clips


def mel_clips(frames, seed: int = 3, masks=None):
    """Synthetic log-mel spectrograms, one per entry of `frames`."""
    import svl_audio
    out = []
    for i, f in enumerate(frames):
        feats = svl_amd.synth_uniform(seed, 20 + i, -7.0, 2.0, int(f) * 128).reshape(int(f), 128)
        mask = np.ones(int(f), bool) if masks is None else np.asarray(masks[i], bool)
        out.append(svl_audio.MelSpectrogram(feats, mask))
    return out
