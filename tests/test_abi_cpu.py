"""CPU-only checks of the product library: it loads, it exports every entry
point include/svl_hip.h declares, the host mirror of config.rs is as strict
as the reference's parser (config.rs:837-967), and the host-side helpers
(truncate_and_normalize, synthetic data) behave. No compute call here needs
a GPU."""
import json
import os
import re

import numpy as np
import pytest

import svl_amd
import svl_synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "svl_hip.h")

MINI = """{
    "model_type": "embedding_gemma2_text", "dtype": "bfloat16", "vocab_size": 64,
    "hidden_size": 16, "intermediate_size": 32, "num_hidden_layers": 3,
    "num_attention_heads": 2, "num_key_value_heads": 1, "head_dim": 8,
    "hidden_size_per_layer_input": 8, "embedding_dim": 8,
    "hidden_activation": "gelu_pytorch_tanh", "max_position_embeddings": 64,
    "rms_norm_eps": 1e-6, "pad_token_id": 0, "bos_token_id": 1, "eos_token_id": 2,
    "attention_bias": false, "attention_dropout": 0.0, "sliding_window": 2,
    "layer_types": ["sliding_attention", "sliding_attention", "full_attention"],
    "per_layer_config": {"2": {"head_dim": 16, "num_key_value_heads": 1}},
    "rope_parameters": {
        "sliding_attention": {"rope_theta": 10000.0, "rope_type": "default"},
        "full_attention": {"rope_theta": 1000000.0, "rope_type": "default"}
    }
}"""


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(svl_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_entry_point():
    lib = svl_amd.lib()
    syms = declared_symbols()
    assert len(syms) >= 20
    for name in syms:
        assert hasattr(lib, name), f"{name} declared in svl_hip.h but not exported"
    assert set(syms) == set(svl_amd.EXPORTED)


def test_attention_path_hook_rejects_unknown_paths():
    with pytest.raises(svl_amd.SvlError) as e:
        svl_amd._check(svl_amd.lib().svl_set_attention_path(3))
    assert e.value.kind == "Usage"
    svl_amd.set_attention_path("auto")


def test_pass_size_setter_checks_its_arguments():
    lib = svl_amd.lib()
    with pytest.raises(svl_amd.SvlError) as e:
        svl_amd._check(lib.svl_text_model_set_pass_tokens(None, 5))
    assert e.value.kind == "Usage"


def test_library_has_a_single_gfx950_code_object():
    data = open(svl_amd.LIB_PATH, "rb").read()
    assert data.count(b"amdgcn-amd-amdhsa--gfx950") >= 1
    for other in (b"gfx942", b"gfx90a", b"gfx1100", b"sm_"):
        assert b"amdgcn-amd-amdhsa--" + other not in data


def test_config_parses_consistent_configuration():  # config.rs:838-852
    c = svl_amd.TextConfig.from_json_str(MINI)
    assert (c.vocab_size, c.hidden_size, c.num_hidden_layers, c.embedding_dim) == (64, 16, 3, 8)
    assert c.head_dim == [8, 8, 16] and c.num_kv_heads == [1, 1, 1]
    assert c.layer_type == [0, 0, 1]
    assert len(c.tensor_shapes()) == 5 + 3 * 17
    c2 = svl_amd.TextConfig.from_json_str('{"text_config": %s}' % MINI)
    assert c2.hidden_size == 16


def test_config_rejects_unsupported_choices():  # config.rs:883-915
    for old, new in [('"gelu_pytorch_tanh"', '"silu"'), ('"bfloat16"', '"float16"'),
                     ('"attention_bias": false', '"attention_bias": true'),
                     ('"attention_dropout": 0.0', '"attention_dropout": 0.1'),
                     ('"sliding_attention"', '"causal"'),
                     ('"rope_type": "default"', '"rope_type": "linear"')]:
        with pytest.raises(svl_amd.SvlError) as e:
            svl_amd.TextConfig.from_json_str(MINI.replace(old, new, 1))
        assert e.value.kind in ("Unsupported", "Corrupt")


def test_config_rejects_missing_and_inconsistent_fields():  # config.rs:916-940
    for old, new in [('"hidden_size": 16,', ''), ('"num_hidden_layers": 3', '"num_hidden_layers": 4'),
                     ('"sliding_window": 2', '"sliding_window": 0'), ('"head_dim": 8', '"head_dim": 7'),
                     ('"num_key_value_heads": 1', '"num_key_value_heads": 3'),
                     ('"2": {"head_dim"', '"3": {"head_dim"'),
                     ('"rms_norm_eps": 1e-6', '"rms_norm_eps": 1e300')]:
        with pytest.raises(svl_amd.SvlError) as e:
            svl_amd.TextConfig.from_json_str(MINI.replace(old, new, 1))
        assert e.value.kind in ("Corrupt", "Unsupported", "LimitExceeded")


def test_config_rejects_non_full_last_layer():  # config.rs:941-949
    doc = MINI.replace('["sliding_attention", "sliding_attention", "full_attention"]',
                       '["sliding_attention", "sliding_attention", "sliding_attention"]')
    with pytest.raises(svl_amd.SvlError) as e:
        svl_amd.TextConfig.from_json_str(doc)
    assert e.value.kind == "Unsupported"


def test_tensor_inventory_matches_reference():  # config.rs:951-966
    shapes = dict(svl_amd.TextConfig.from_json_str(MINI).tensor_shapes())
    assert shapes["language_model.embed_tokens.weight"] == (64, 16)
    assert shapes["language_model.embedding_projection.weight"] == (8, 16)
    assert shapes["language_model.ple.per_layer_model_projection.weight"] == (24, 16)
    assert shapes["language_model.layers.0.self_attn.k_proj.weight"] == (8, 16)
    assert shapes["language_model.layers.2.self_attn.q_proj.weight"] == (32, 16)


def test_benchmark_shapes_are_legal_reference_configs():
    a = svl_amd.TextConfig.from_json_value(svl_synth.config_a())
    assert (a.hidden_size, a.num_attention_heads, a.head_dim[0], a.num_kv_heads[0]) == (768, 3, 256, 1)
    assert a.layer_type.count(1) == 4 and a.layer_type[-1] == 1
    b = svl_amd.TextConfig.from_json_value(svl_synth.config_b())
    assert b.head_dim[5] == 512 and b.num_kv_heads[5] == 1 and b.num_kv_heads[0] == 2
    nparams = sum(int(np.prod(s)) for _, s in a.tensor_shapes())
    assert nparams == 317_627_416


def test_truncate_and_normalize_host():  # kernels.rs:1480-1491
    np.testing.assert_allclose(svl_amd.truncate_and_normalize([3, 4, 12], 2), [0.6, 0.8], atol=1e-7)
    for bad in (0, 4):
        with pytest.raises(svl_amd.SvlError) as e:
            svl_amd.truncate_and_normalize([3, 4, 12], bad)
        assert e.value.kind == "Internal"
    with pytest.raises(svl_amd.SvlError):
        svl_amd.truncate_and_normalize([0, 0], 2)


def test_synthetic_data_is_deterministic_and_in_range():
    a = svl_amd.synth_uniform(0, 7, -0.5, 0.5, 100000)
    b = svl_amd.synth_uniform(0, 7, -0.5, 0.5, 100000)
    assert a.tobytes() == b.tobytes()
    assert a.min() >= -0.5 and a.max() < 0.5 and abs(a.mean()) < 0.01
    c = svl_amd.synth_uniform(0, 8, -0.5, 0.5, 1000)
    assert not np.array_equal(a[:1000], c)
    ids = svl_amd.synth_ids(1, 0, 262144, 50000)
    assert ids.max() < 262144 and ids.min() >= 0
    lens = svl_amd.synth_lengths(1, 1, 64, 512, 10000)
    assert lens.min() >= 64 and lens.max() <= 512 and 270 < lens.mean() < 306


def test_safetensors_reader_matches_fixture():
    w = svl_amd.read_safetensors(os.path.join(ROOT, "tests", "golden", "tiny_text", "model.safetensors"))
    assert len(w) == 56
    t = w["language_model.embed_tokens.weight"]
    assert t.dtype == "F32" and t.shape == (64, 16) and t.data.size == 1024
