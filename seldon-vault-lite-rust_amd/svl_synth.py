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
