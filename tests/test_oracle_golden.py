"""Pins the oracle's whole text forward pass against the official
Transformers golden of the reference's tiny model
(fixtures/model/tiny_text/golden.json, copied to tests/golden/tiny_text) at
the reference tolerances (tests/text_embeddings.rs:83-230)."""
import json
import os

import numpy as np
import pytest
from safetensors.numpy import load_file

from oracle import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
TINY = os.path.join(HERE, "golden", "tiny_text")


def load_tiny():
    cfg = json.load(open(os.path.join(TINY, "config.json")))
    w = load_file(os.path.join(TINY, "model.safetensors"))
    g = json.load(open(os.path.join(TINY, "golden.json")))
    return cfg, w, g


def assert_close(actual, expected, atol, rtol, label):
    actual = np.asarray(actual, np.float32)
    expected = np.asarray(expected, np.float32)
    diff = np.abs(actual - expected)
    tol = atol + rtol * np.abs(expected)
    assert (diff <= tol).all(), f"{label}: max diff {diff.max()}"


def assert_embedding(actual, expected, label):  # text_embeddings.rs:106-125
    assert_close(actual, expected, 1e-4, 1e-4, label)
    assert abs(float(np.dot(actual, actual)) - 1) <= 1e-4
    cos = float(np.dot(actual, expected) / (np.linalg.norm(actual) * np.linalg.norm(expected)))
    assert cos >= 0.9999, f"{label} cosine {cos}"


def test_tiny_model_matches_official_layer_and_embedding_outputs():
    cfg, w, g = load_tiny()
    m = O.OracleTextModel(cfg, w)
    for ci, case in enumerate(g["cases"]):
        out = m.forward(case["input_ids"], capture_hidden=True)
        hs = out["hidden_states"]
        assert hs.shape[0] == 1 + cfg["num_hidden_layers"]
        for layer in range(hs.shape[0]):
            assert_close(hs[layer].mean(0), case["hidden_state_means"][layer], 2e-5, 1e-4,
                         f"case {ci} layer {layer} mean")
            assert_close(hs[layer][-1], case["hidden_state_last"][layer], 2e-5, 1e-4,
                         f"case {ci} layer {layer} last")
        assert_close(out["projected"].mean(0), case["projected_mean"], 2e-4, 1e-4, "projected mean")
        assert_close(out["projected"][-1], case["projected_last"], 2e-4, 1e-4, "projected last")
        assert_embedding(out["normalized"], case["embedding"], f"case {ci}")
        t = O.truncate_and_normalize(out["normalized"], 4)
        assert abs(float(np.dot(t, t)) - 1) <= 1e-4


def test_oracle_is_deterministic():  # text_embeddings.rs:388-405
    cfg, w, g = load_tiny()
    m = O.OracleTextModel(cfg, w)
    a = m.forward([1, 5, 7, 9, 2])["normalized"]
    b = m.forward([1, 5, 7, 9, 2])["normalized"]
    assert a.tobytes() == b.tobytes()


def test_oracle_rejections():  # text.rs:188-218, text_embeddings.rs:407-431
    cfg, w, g = load_tiny()
    m = O.OracleTextModel(cfg, w)
    with pytest.raises(O.OracleError) as e:
        m.forward([])
    assert e.value.status == 4
    with pytest.raises(O.OracleError) as e:
        m.forward([1, 64])
    assert e.value.status == 4
    with pytest.raises(O.OracleError) as e:
        m.forward([1] * 65)  # above max_position_embeddings = 64
    assert e.value.status == 5


def test_planted_mistakes_fail_the_golden():
    """A (1 + w) norm convention, a doubled post-attention norm or an
    unscaled V would move the output outside the golden tolerance."""
    cfg, w, g = load_tiny()
    case = g["cases"][0]
    for name in ["language_model.layers.1.self_attn.q_norm.weight",
                 "language_model.layers.2.self_attn.k_norm.weight",
                 "language_model.layers.0.post_attention_layernorm.weight",
                 "language_model.layers.1.ple_block.post_per_layer_input_norm.weight"]:
        w2 = dict(w)
        w2[name] = w[name] + 1.0
        out = O.OracleTextModel(cfg, w2).forward(case["input_ids"])
        with pytest.raises(AssertionError):
            assert_embedding(out["normalized"], case["embedding"], name)


def test_oracle_matches_float64_restatement_with_nontrivial_1d_weights():
    """The golden's 1-D weights are all ones; random norm weights and layer
    scalars pin weight alignment and the layer_scalar multiply (text.rs:510-513)."""
    import ref64
    cfg, w, g = load_tiny()
    rc = O.resolve_config(cfg)
    for seed in (1, 2):
        w2 = ref64.randomize_1d(w, seed)
        m = O.OracleTextModel(cfg, w2)
        for case in g["cases"]:
            a = m.forward(case["input_ids"], capture_hidden=True)
            b = ref64.forward(rc, w2, case["input_ids"])
            np.testing.assert_allclose(a["hidden_states"], b["hidden_states"], atol=5e-5, rtol=1e-4)
            np.testing.assert_allclose(a["normalized"], b["normalized"], atol=1e-5)
    # planted: skipping layer_scalar in the float64 side is detected
    w2 = ref64.randomize_1d(w, 1)
    w3 = dict(w2)
    for l in range(cfg["num_hidden_layers"]):
        w3[f"language_model.layers.{l}.layer_scalar"] = np.ones(1, np.float32)
    a = O.OracleTextModel(cfg, w2).forward(g["cases"][0]["input_ids"])
    b = ref64.forward(rc, w3, g["cases"][0]["input_ids"])
    assert np.abs(a["normalized"] - b["normalized"]).max() > 1e-3


def test_features_overwrite_rows():  # text.rs:226-275
    cfg, w, g = load_tiny()
    m = O.OracleTextModel(cfg, w)
    H = cfg["hidden_size"]
    feats = np.linspace(-1, 1, 2 * H, dtype=np.float32)
    out = m.forward([1, 5, 7, 9, 2], capture_hidden=True, features=feats, feature_start=1,
                    feature_count=2)
    np.testing.assert_array_equal(out["hidden_states"][0][1:3].reshape(-1), feats)
    with pytest.raises(O.OracleError) as e:
        m.forward([1, 5, 7], features=feats, feature_start=2, feature_count=2)
    assert e.value.status == 4
