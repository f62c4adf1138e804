"""GPU parity of the whole text forward pass (TextModel::forward_impl,
src/model/text.rs:182-538) through the C ABI.

* tiny official model: against the official Transformers golden at the
  reference tolerances (tests/text_embeddings.rs:83-230) and against the
  CPU oracle;
* benchmark shapes (A: hidden 768 / 3 q heads / 1 KV head of 256; B: the
  reference manifest shape with 2 KV heads and head_dim 512 on full layers)
  with random-init weights: against the oracle row by row, per embedding
  max-abs <= 1e-4 and cosine >= 0.99999;
* batching semantics: a packed ragged batch equals independent calls bit for
  bit; sliding windows beyond 512 tokens; multimodal feature rows; the
  device-resident Matryoshka outputs; error taxonomy and determinism."""
import json
import os
import threading

import numpy as np
import pytest
from safetensors.numpy import load_file

import svl_amd as S
import svl_synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
TINY = os.path.join(HERE, "golden", "tiny_text")

MAX_ABS = 1e-4      # north-star tolerance per pooled embedding
MIN_COS = 0.99999


def tiny():
    cfg = json.load(open(os.path.join(TINY, "config.json")))
    w = load_file(os.path.join(TINY, "model.safetensors"))
    g = json.load(open(os.path.join(TINY, "golden.json")))
    return cfg, w, g


def model(cfg, w):
    return S.TextModel(S.TextConfig.from_json_value(cfg), w)


def cosine(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def assert_close(actual, expected, atol, rtol, label):
    actual = np.asarray(actual, np.float32)
    expected = np.asarray(expected, np.float32)
    diff = np.abs(actual - expected)
    assert (diff <= atol + rtol * np.abs(expected)).all(), f"{label}: max diff {diff.max()}"


def assert_embedding_parity(got, ref, label):
    d = float(np.abs(np.asarray(got) - np.asarray(ref)).max())
    c = cosine(got, ref)
    assert d <= MAX_ABS and c >= MIN_COS, f"{label}: max-abs {d:.3g} cosine {c:.8f}"


def test_tiny_model_matches_official_golden():
    cfg, w, g = tiny()
    m = model(cfg, w)
    for ci, case in enumerate(g["cases"]):
        out = m.forward(case["input_ids"], capture_hidden=True)
        hs = out.hidden_states()
        assert hs.shape[0] == 1 + cfg["num_hidden_layers"]
        for layer in range(hs.shape[0]):
            assert_close(hs[layer].mean(0), case["hidden_state_means"][layer], 2e-5, 1e-4,
                         f"case {ci} layer {layer} mean")
            assert_close(hs[layer][-1], case["hidden_state_last"][layer], 2e-5, 1e-4,
                         f"case {ci} layer {layer} last")
        proj = out.projected()
        assert_close(proj.mean(0), case["projected_mean"], 2e-4, 1e-4, "projected mean")
        assert_close(proj[-1], case["projected_last"], 2e-4, 1e-4, "projected last")
        emb = out.normalized()
        assert_close(emb, case["embedding"], 1e-4, 1e-4, "embedding")
        assert abs(float(emb @ emb) - 1) <= 1e-4
        assert cosine(emb, case["embedding"]) >= 0.9999
        t = out.embedding(4)
        assert abs(float(t @ t) - 1) <= 1e-4


def test_tiny_model_matches_oracle_with_nontrivial_weights():
    import ref64
    cfg, w, g = tiny()
    for seed in (0, 1):
        w2 = ref64.randomize_1d(w, seed)
        m, o = model(cfg, w2), O.OracleTextModel(cfg, w2)
        rows = [c["input_ids"] for c in g["cases"]] + [list(range(1, 60))]
        outs = m.forward_batch(rows, capture_hidden=True)
        for r, got in zip(rows, outs):
            ref = o.forward(r, capture_hidden=True)
            np.testing.assert_allclose(got.hidden_states(), ref["hidden_states"], atol=2e-5, rtol=1e-4)
            np.testing.assert_allclose(got.pooled(), ref["pooled"], atol=2e-5, rtol=1e-4)
            assert_embedding_parity(got.normalized(), ref["normalized"], f"tiny seed {seed}")


def _shape_parity(cfg, lengths, seed=1, capture=False):
    w = svl_synth.weights(cfg, seed=0)
    rows = svl_synth.token_rows(cfg["vocab_size"], lengths, seed=seed)
    m = model(cfg, w)
    got = m.forward_batch(rows, capture_hidden=capture)
    ref = O.OracleTextModel(cfg, w).forward_rows(rows)
    for i, (g_, r_) in enumerate(zip(got, ref)):
        assert_embedding_parity(g_.normalized(), r_["normalized"], f"row {i} len {lengths[i]}")
        for d in (512, 256, 128):
            assert_embedding_parity(g_.embedding(d), O.truncate_and_normalize(r_["normalized"], d),
                                    f"row {i} dim {d}")
    return m, rows, got


def test_shape_a_reduced_depth_ragged_rows_match_oracle():
    # 6 layers (5 sliding + 1 full); rows straddle the 32-key tiles, the
    # 128-vector attention blocks and the 512-token sliding window.
    cfg = svl_synth.config_a(layers=6, vocab=4096)
    _shape_parity(cfg, [1, 31, 129, 300, 515, 700])


@pytest.mark.parametrize("path", ["fallback", "generic"])
def test_forward_on_the_fallback_attention_kernels_matches_oracle(path):
    """The whole forward pass with its attention forced onto the kernels that
    rows past a 2 GiB K/V window take (the register-staged MFMA kernel at
    head_dim 256) and onto the generic kernel: shape A at reduced depth with
    ragged rows across the 512-token window, and shape B (two KV heads, and
    head_dim 512 on its full layer)."""
    try:
        S.set_attention_path(path)
        _shape_parity(svl_synth.config_a(layers=6, vocab=4096), [1, 31, 129, 300, 515, 700])
        _shape_parity(svl_synth.config_b(layers=6, vocab=4096), [77, 600])
    finally:
        S.set_attention_path("auto")


def test_shape_a_full_depth_t1_matches_oracle():
    # 24 layers at the reference-sized config, batch 1 x 128 tokens.
    cfg = svl_synth.config_a(layers=24, vocab=262144)
    _shape_parity(cfg, [128])


def test_long_context_rows_match_oracle():
    # The long-context row length: two 2048-token rows through a sliding layer
    # (window 512: every query's window is cut on both sides) and a full one
    # (the 2048 x 2048 score matrix).
    cfg = svl_synth.config_a(layers=2, vocab=4096)
    _shape_parity(cfg, [2048, 2047])


def test_long_context_batch_is_batch_invariant():
    # The full long-context shape (8 x 2048 tokens, 24 layers): every row of the batch
    # equals the same row run alone, bit for bit, and is a finite unit vector.
    cfg = svl_synth.config_a(layers=24, vocab=262144)
    w = svl_synth.weights(cfg, seed=0)
    m = model(cfg, w)
    del w
    rows = svl_synth.token_rows(cfg["vocab_size"], [2048] * 8, seed=4)
    batch = m.forward_batch(rows)
    for i in (0, 5):
        one = m.forward_batch([rows[i]])[0]
        assert np.array_equal(one.normalized(), batch[i].normalized()), f"row {i}"
    for b in batch:
        e = b.normalized()
        assert np.isfinite(e).all() and abs(float(e.astype(np.float64) @ e) - 1.0) < 1e-5


def test_longest_row_matches_oracle():
    # A row of 8192 tokens, the most the reference accepts (text.rs:188-202),
    # beside a short row, on a narrow two-layer model (hidden 128, 2 q heads
    # sharing one KV head of dim 64, so the oracle finishes in seconds): the
    # sliding layer cuts every window of the long row, the full layer scores
    # 8192 x 8192 keys per head. One token more is LimitExceeded.
    cfg = svl_synth.config_a(layers=2, vocab=4096)
    cfg.update(hidden_size=128, intermediate_size=256, num_attention_heads=2,
               num_key_value_heads=1, head_dim=64, hidden_size_per_layer_input=32,
               embedding_dim=128)
    w = svl_synth.weights(cfg, seed=5)
    rows = svl_synth.token_rows(4096, [8192, 77], seed=6)
    m = model(cfg, w)
    got = m.forward_batch(rows)
    ref = O.OracleTextModel(cfg, w).forward_rows(rows)
    for i, (g_, r_) in enumerate(zip(got, ref)):
        assert_embedding_parity(g_.normalized(), r_["normalized"], f"row {i} len {len(rows[i])}")
    assert m.forward(rows[0]).normalized().tobytes() == got[0].normalized().tobytes()
    with pytest.raises(S.SvlError) as e:
        m.forward(np.concatenate([rows[0], rows[1][:1]]))
    assert e.value.kind == "LimitExceeded"


def test_shape_b_manifest_shape_matches_oracle():
    # 2 KV heads on sliding layers, 1 KV head of head_dim 512 on the full layer.
    cfg = svl_synth.config_b(layers=6, vocab=4096)
    _shape_parity(cfg, [40, 257])


def test_shape_b_long_rows_match_oracle():
    # Rows past the 512 window on the sliding layers and a 1100 x 1100 score
    # matrix at head_dim 512 on the full layer (layer 6 of 6).
    cfg = svl_synth.config_b(layers=6, vocab=4096)
    _shape_parity(cfg, [1100, 700])


def test_packed_batch_equals_independent_calls_bit_for_bit():
    cfg = svl_synth.config_a(layers=3, vocab=4096)
    w = svl_synth.weights(cfg)
    m = model(cfg, w)
    rows = svl_synth.token_rows(4096, [5, 200, 64, 333])
    batch = m.forward_batch(rows)
    for r, b in zip(rows, batch):
        single = m.forward(r)
        assert single.normalized().tobytes() == b.normalized().tobytes()
        assert single.pooled().tobytes() == b.pooled().tobytes()
    again = m.forward_batch(rows)  # determinism (text_embeddings.rs:388-405)
    for a, b in zip(batch, again):
        assert a.normalized().tobytes() == b.normalized().tobytes()


def test_two_stream_row_groups_are_bit_identical():
    # Batches above 4096 tokens run as row groups on concurrent streams (a
    # batch whose rows are all longer than the 512 window runs as one group).
    cfg = svl_synth.config_a(layers=2, vocab=4096)
    w = svl_synth.weights(cfg)
    m = model(cfg, w)
    rows = svl_synth.token_rows(4096, [512, 300, 500, 400, 100, 480, 500, 513, 64, 512, 300, 400,
                                       700])
    assert sum(len(r) for r in rows) >= 4096
    split = m.forward_batch(rows, capture_hidden=True)
    m.set_stream_split(False)
    single = m.forward_batch(rows, capture_hidden=True)
    m.set_stream_split(True)
    for a, b in zip(split, single):
        assert a.normalized().tobytes() == b.normalized().tobytes()
        assert a.hidden_states().tobytes() == b.hidden_states().tobytes()
    for r, a in zip(rows[:3], split[:3]):
        assert m.forward(r).normalized().tobytes() == a.normalized().tobytes()


def test_row_groups_in_grouped_tile_order_are_bit_identical():
    # About 16,000 tokens: each of the three row groups' GEMMs has 80 or more
    # 64-row M blocks, so the shared launches take the grouped tile order
    # (odd groups of 8 M blocks run their N blocks in reverse, the last group
    # is partial); the single-stream launches of the whole batch take it too,
    # and one row alone runs small tiles in the plain order.
    cfg = svl_synth.config_a(layers=2, vocab=4096)
    w = svl_synth.weights(cfg)
    m = model(cfg, w)
    lengths = [300 + (97 * i) % 213 for i in range(40)]
    rows = svl_synth.token_rows(4096, lengths, seed=5)
    split = m.forward_batch(rows, capture_hidden=True)
    m.set_stream_split(False)
    single = m.forward_batch(rows, capture_hidden=True)
    m.set_stream_split(True)
    for a, b in zip(split, single):
        assert a.normalized().tobytes() == b.normalized().tobytes()
        assert a.hidden_states().tobytes() == b.hidden_states().tobytes()
    for i in (0, 13, 39):
        assert m.forward(rows[i]).normalized().tobytes() == split[i].normalized().tobytes()


def test_batches_run_in_passes_bit_for_bit():
    """A batch whose workspace would pass the budget runs as passes of
    consecutive rows. At a 700-token budget the 13 rows below take ten passes
    (the 900-token row alone); the host outputs, hidden states included, with
    feature rows in two of the passes, and the device entry point's Matryoshka
    outputs equal the one-pass run bit for bit."""
    import torch
    cfg = svl_synth.config_a(layers=2, vocab=4096)
    w = svl_synth.weights(cfg)
    m = model(cfg, w)
    lens = [512, 300, 500, 400, 100, 480, 900, 513, 64, 512, 300, 400, 37]
    rows = svl_synth.token_rows(4096, lens)
    rng = np.random.default_rng(3)
    feats = [None] * len(rows)
    feats[2] = ((rng.standard_normal((10, 768)) * 0.5).astype(np.float32), 5, 10)
    feats[9] = ((rng.standard_normal((4, 768)) * 0.5).astype(np.float32), 500, 4)
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    ids = torch.from_numpy(np.concatenate(rows).astype(np.int32)).to("cuda:0")
    dims = [768, 256]
    outs, dev = [], []
    for budget in (0, 700):
        m.set_pass_tokens(budget)
        outs.append(m.forward_batch(rows, capture_hidden=True, features=feats))
        d = torch.zeros((len(rows), sum(dims)), dtype=torch.float32, device="cuda:0")
        m.forward_device(ids.data_ptr(), offsets, dims, d.data_ptr(),
                         torch.cuda.current_stream().cuda_stream)
        dev.append(d.cpu().numpy())
    for i, (a, b) in enumerate(zip(*outs)):
        for part in ("normalized", "pooled", "projected", "hidden_states"):
            assert getattr(a, part)().tobytes() == getattr(b, part)().tobytes(), (i, part)
    np.testing.assert_array_equal(outs[1][2].hidden_states()[0][5:15], feats[2][0])
    assert dev[0].tobytes() == dev[1].tobytes()
    with pytest.raises(S.SvlError) as e:
        m.set_pass_tokens(-1)
    assert e.value.kind == "Usage"
    m.set_pass_tokens(0)


def test_features_replace_rows_like_the_reference():  # text.rs:226-275
    cfg = svl_synth.config_a(layers=3, vocab=4096)
    w = svl_synth.weights(cfg)
    m, o = model(cfg, w), O.OracleTextModel(cfg, w)
    ids = svl_synth.token_rows(4096, [40])[0]
    feats = (np.random.default_rng(0).standard_normal((10, 768)) * 0.5).astype(np.float32)
    got = m.forward_with_features(ids, feats, 5, 10, capture_hidden=True)
    ref = o.forward(ids, capture_hidden=True, features=feats, feature_start=5, feature_count=10)
    np.testing.assert_array_equal(got.hidden_states()[0][5:15], feats)
    assert_embedding_parity(got.normalized(), ref["normalized"], "features")
    with pytest.raises(S.SvlError) as e:
        m.forward_with_features(ids, feats, 35, 10)
    assert e.value.kind == "Corrupt"
    with pytest.raises(S.SvlError) as e:
        m.forward_with_features(ids, feats[:9], 5, 10)
    assert e.value.kind == "Corrupt"


def test_device_resident_matryoshka_outputs():
    import torch
    cfg = svl_synth.config_a(layers=3, vocab=4096)
    w = svl_synth.weights(cfg)
    m = model(cfg, w)
    rows = svl_synth.token_rows(4096, [10, 99, 256])
    host = m.forward_batch(rows)
    offsets = np.concatenate([[0], np.cumsum([len(r) for r in rows])]).astype(np.int64)
    ids = torch.from_numpy(np.concatenate(rows).astype(np.int32)).to("cuda:0")
    dims = [768, 512, 256, 128]
    out = torch.zeros((3, sum(dims)), dtype=torch.float32, device="cuda:0")
    m.forward_device(ids.data_ptr(), offsets, dims, out.data_ptr(),
                     torch.cuda.current_stream().cuda_stream)
    got = out.cpu().numpy()
    for i, h in enumerate(host):
        off = 0
        for d in dims:
            np.testing.assert_allclose(got[i, off:off + d], h.embedding(d), atol=1e-6)
            off += d
    bad = torch.from_numpy(np.array([1, 2, 5000], np.int32)).to("cuda:0")
    with pytest.raises(S.SvlError) as e:
        m.forward_device(bad.data_ptr(), np.array([0, 3], np.int64), [768], out.data_ptr())
    assert e.value.kind == "Corrupt"


def test_error_taxonomy_matches_reference():  # text.rs:188-218, 546-554
    cfg, w, g = tiny()
    m = model(cfg, w)
    cases = [([], "Corrupt"), ([1, 64], "Corrupt"), ([1] * 65, "LimitExceeded")]
    for ids, kind in cases:
        with pytest.raises(S.SvlError) as e:
            m.forward(ids)
        assert e.value.kind == kind, ids
    for dim in (0, 9):
        with pytest.raises(S.SvlError) as e:
            m.embed_ids([1, 2], dim)
        assert e.value.kind == "Internal"
    v = m.embed_ids([1, 5, 7, 9, 2], 4)
    assert v.shape == (4,) and abs(float(v @ v) - 1) <= 1e-4


def test_concurrent_calls_are_safe_and_identical():  # text_embeddings.rs:439-457
    cfg, w, g = tiny()
    m = model(cfg, w)
    ref = m.forward([1, 5, 7, 9, 2]).normalized().tobytes()
    errors = []

    def work():
        try:
            for _ in range(5):
                assert m.forward([1, 5, 7, 9, 2]).normalized().tobytes() == ref
        except Exception as e:  # noqa
            errors.append(e)

    ts = [threading.Thread(target=work) for _ in range(4)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errors


def test_weight_inventory_is_validated():  # weights.rs:130-166
    cfg, w, g = tiny()
    c = S.TextConfig.from_json_value(cfg)
    w2 = dict(w)
    del w2["language_model.norm.weight"]
    with pytest.raises(S.SvlError) as e:
        S.TextModel(c, w2)
    assert e.value.kind == "Corrupt"
    w3 = dict(w)
    w3["language_model.extra.weight"] = np.zeros(3, np.float32)
    with pytest.raises(S.SvlError) as e:
        S.TextModel(c, w3)
    assert e.value.kind == "Corrupt"
    w4 = dict(w)
    bad = w["language_model.norm.weight"].copy()
    bad[0] = np.nan
    w4["language_model.norm.weight"] = bad
    with pytest.raises(S.SvlError) as e:
        S.TextModel(c, w4)
    assert e.value.kind == "Internal"
    # a payload one element short of its shape (safetensors.rs:79-88)
    w5 = dict(w)
    short = np.ascontiguousarray(w["language_model.norm.weight"], np.float32)[:-1]
    w5["language_model.norm.weight"] = S.RawTensor("F32", (cfg["hidden_size"],), short)
    with pytest.raises(S.SvlError) as e:
        S.TextModel(c, w5)
    assert e.value.kind == "Corrupt"


def _to_bf16_bits(a):
    """f32_to_bf16 (bf16.rs:21-40): round to nearest, ties to even."""
    b = np.ascontiguousarray(a, np.float32).view(np.uint32)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def test_bf16_weights_equal_their_f32_widening():
    """The tiny model with every weight rounded to BF16 and passed as BF16
    views (widened by the library, safetensors.rs:69-110) gives the same bits
    as the widened values passed as F32, and matches the oracle on them."""
    cfg, w, g = tiny()
    bf = {k: S.RawTensor("BF16", np.shape(v), _to_bf16_bits(v)) for k, v in w.items()}
    wide = {k: t.to_f32() for k, t in bf.items()}
    for k, v in w.items():
        assert np.abs(wide[k] - v).max() <= np.abs(v).max() * 2.0 ** -8, k
    a, b = model(cfg, bf), model(cfg, wide)
    ref = O.OracleTextModel(cfg, wide)
    for case in g["cases"]:
        x, y = a.forward(case["input_ids"]), b.forward(case["input_ids"])
        assert x.normalized().tobytes() == y.normalized().tobytes()
        assert x.projected().tobytes() == y.projected().tobytes()
        assert_embedding_parity(x.normalized(), ref.forward(case["input_ids"])["normalized"],
                                "BF16 tiny model")
