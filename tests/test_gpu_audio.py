"""GPU parity of the audio tower (AudioModel::forward, src/model/audio.rs:
981-1134) and of the audio prompt glue (AudioEmbedder::embed_impl,
src/model/audio_embedder.rs:223-267) through the C ABI.

* the official tiny audio fixture: SSCP output, both layer outputs, the audio
  features and the final embedding at the tolerances of
  tests/audio_tiny.rs:78-200, and against the CPU oracle chain;
* config AU (hidden 1024, 8 heads of 128, SSCP [128, 32], chunk 12 / left 13)
  at 2 layers against the oracle over a ragged batch with masked frames, and
  a full 30 s clip (2999 frames, 750 tokens) at 1 layer;
* batching and the device-resident variants bit-identical to single calls;
* the audio embedder against the oracle chain; the error taxonomy."""
import json
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
from safetensors.numpy import load_file

import svl_amd as S
import svl_audio as A
import svl_synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
TINY = os.path.join(HERE, "golden", "tiny_audio")

MAX_ABS = 1e-4
MIN_COS = 0.99999


def cosine(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def close(actual, expected, atol=2e-4, rtol=2e-4):
    a = np.asarray(actual, np.float32)
    e = np.asarray(expected, np.float32)
    return a.shape == e.shape and bool((np.abs(a - e) <= atol + rtol * np.abs(e)).all())


def check(got, want, label, max_abs=MAX_ABS):
    d = float(np.abs(np.asarray(got) - np.asarray(want)).max())
    c = cosine(got, want)
    print(f"{label}: max-abs {d:.3g} cosine {c:.9f}", flush=True)
    assert d <= max_abs and c >= MIN_COS, f"{label}: max-abs {d:.3g} cosine {c:.9f}"


@pytest.fixture(scope="module")
def tiny():
    cfg = json.load(open(os.path.join(TINY, "config.json")))
    g = json.load(open(os.path.join(TINY, "golden.json")))
    w = load_file(os.path.join(TINY, "model.safetensors"))
    tm = S.TextModel(S.TextConfig.from_json_value(cfg), w)
    am = A.AudioModel(A.AudioConfig.from_json_value(cfg), w, 16)
    return cfg, g, w, tm, am


def test_tiny_audio_matches_the_official_fixture(tiny):
    cfg, g, w, tm, am = tiny
    mel = A.MelSpectrogram(np.array(g["mel_features"], np.float32), g["mel_mask"])
    out = am.forward(mel, capture_hidden=True)
    assert out.audio_tokens() == g["audio_tokens"] == 3
    assert close(out.sscp_output(), g["sscp_output"])
    assert len(out.hidden_states()) == 2
    for l in range(2):
        assert close(out.hidden_states()[l], g["layer_outputs"][l]), f"layer {l}"
    assert close(out.pooled(), g["audio_features"])
    ref = O.OracleAudioModel(cfg, w, 16).forward(mel.features, mel.mask.astype(bool), True)
    check(out.pooled(), ref["pooled"], "tiny soft tokens vs oracle")
    np.testing.assert_allclose(np.stack(out.hidden_states()), ref["hidden_states"], atol=1e-5,
                               rtol=1e-5)

    tokens = A.AudioSpecialTokens(bos=1, eos=2, pad=0, boa=3, audio=4, eoa=5)
    emb = A.AudioEmbedder(tm, am, tokens)
    e = emb.embed_mel(mel, 8)
    exp = np.array(g["embedding"], np.float64)
    assert cosine(e, exp) >= 0.9999 and np.abs(e - exp).max() <= 1e-4
    assert abs(float(e @ e) - 1.0) <= 1e-5
    fwd = O.OracleTextModel(cfg, w).forward(g["input_ids"], features=ref["pooled"],
                                            feature_start=2, feature_count=3)
    for dim in (8, 4, 2, 1):
        check(emb.embed_mel(mel, dim), O.truncate_and_normalize(fwd["normalized"], dim),
              f"tiny embedding dim {dim}")


@pytest.fixture(scope="module")
def au2():
    c = svl_synth.config_au(2)
    w = svl_synth.audio_weights(c, 768, seed=5)
    return c, w, A.AudioModel(A.AudioConfig.from_json_value(c), w, 768), O.OracleAudioModel(c, w, 768)


def _masked_clips():
    masks = [np.ones(200, bool), np.ones(157, bool), np.ones(13, bool)]
    masks[1][117:] = False        # padded tail: the last 10 tokens are invalid
    masks[2][4] = False           # an interior masked frame
    return svl_synth.mel_clips([200, 157, 13], seed=9, masks=masks)


def test_config_au_two_layers_matches_oracle(au2):
    c, w, gpu, om = au2
    mels = _masked_clips()
    got = gpu.forward_batch(mels, capture_hidden=True)
    with ThreadPoolExecutor(max_workers=3) as ex:
        want = list(ex.map(lambda m: om.forward(m.features, m.mask.astype(bool), True), mels))
    for i, (g_, o) in enumerate(zip(got, want)):
        assert g_.audio_tokens() == o["audio_tokens"] == mels[i].audio_tokens()
        np.testing.assert_allclose(g_.sscp_output(), o["sscp_output"], atol=1e-4, rtol=1e-4)
        hs = np.stack(g_.hidden_states())
        print(f"clip {i}: per-layer hidden max-abs {np.abs(hs - o['hidden_states']).max(axis=(1, 2))}",
              flush=True)
        np.testing.assert_allclose(hs, o["hidden_states"], atol=2e-4, rtol=1e-4)
        check(g_.pooled(), o["pooled"], f"config AU clip {i} soft tokens")


def test_batch_and_device_paths_are_bit_identical(au2):
    import torch
    c, w, gpu, om = au2
    mels = _masked_clips()
    batch = gpu.forward_batch(mels)
    for i, m in enumerate(mels):
        assert np.array_equal(gpu.forward(m).pooled(), batch[i].pooled()), f"clip {i}"
    rev = gpu.forward_batch(mels[::-1])
    for i in range(3):
        assert np.array_equal(rev[i].pooled(), batch[2 - i].pooled())
    feats = torch.from_numpy(np.concatenate([m.features for m in mels])).to("cuda:0")
    n = sum(m.audio_tokens() for m in mels)
    d_out = torch.empty((n, 768), device="cuda:0")
    torch.cuda.synchronize()
    gpu.forward_device(feats.data_ptr(), mels, d_out.data_ptr())
    assert np.array_equal(d_out.cpu().numpy(), np.concatenate([b.pooled() for b in batch]))


def test_subsampling_width_mismatch_fails_the_forward_pass_like_the_reference():
    """A legal configuration whose first subsampling layer has 36 channels
    loads, but its input projection takes (36 / 4) * C1 features per row
    while layer 1 yields 32 * C1, so the forward pass fails with Internal,
    in the reference (audio.rs:1244-1248) as here, after the subsampling
    caps and before the no-token check."""
    c = svl_synth.config_au(1)
    c["audio_config"]["subsampling_conv_channels"] = [36, 20]
    w = svl_synth.audio_weights(c, 768, seed=12)
    gpu = A.AudioModel(A.AudioConfig.from_json_value(c), w, 768)
    om = O.OracleAudioModel(c, w, 768)
    mel = _masked_clips()[0]
    with pytest.raises(S.SvlError) as e:
        gpu.forward(mel)
    assert e.value.kind == "Internal"
    assert "projection input width" in str(e.value)
    with pytest.raises(O.OracleError) as e:
        om.forward(mel.features, mel.mask.astype(bool))
    assert e.value.status == 7
    empty = svl_synth.mel_clips([9], seed=3, masks=[np.zeros(9, bool)])[0]
    with pytest.raises(S.SvlError) as e:   # width before the no-token check, as in audio.rs
        gpu.forward(empty)
    assert e.value.kind == "Internal"
    gpu.close()


def test_batch_past_one_pass_runs_in_passes():
    """44 clips of 2999 frames put 66,000 layer-0 rows of 64 x 128 floats in
    one batch, past the 2 GiB that one pass of the tower takes (43 clips), so
    the batch runs as two passes. Every clip's soft tokens equal a single
    call bit for bit, on the host path and on the device path."""
    import torch
    c = svl_synth.config_au(1)
    w = svl_synth.audio_weights(c, 64, seed=13)
    gpu = A.AudioModel(A.AudioConfig.from_json_value(c), w, 64)
    mels = svl_synth.mel_clips([2999] * 44, seed=14)
    batch = gpu.forward_batch(mels)
    assert [b.audio_tokens() for b in batch] == [750] * 44
    for i in (0, 42, 43):
        assert np.array_equal(gpu.forward(mels[i]).pooled(), batch[i].pooled()), f"clip {i}"
    feats = torch.from_numpy(np.concatenate([m.features for m in mels])).to("cuda:0")
    d_out = torch.empty((44 * 750, 64), device="cuda:0")
    torch.cuda.synchronize()
    gpu.forward_device(feats.data_ptr(), mels, d_out.data_ptr())
    assert np.array_equal(d_out.cpu().numpy(), np.concatenate([b.pooled() for b in batch]))
    one = gpu.forward(mels[43], capture_hidden=True)
    cap = gpu.forward_batch(mels, capture_hidden=True)
    assert np.array_equal(cap[43].hidden_states()[0], one.hidden_states()[0])
    assert np.array_equal(cap[43].sscp_output(), one.sscp_output())
    gpu.close()


# Attention shapes beyond config AU: a head_dim of 15 (rows not 16-byte
# aligned) with 20-row blocks and a 61-entry context (a full wave of lanes
# per query, two passes over each block's queries, right context), and a
# head_dim of 256 with a 35-entry context.
@pytest.mark.parametrize("hidden,heads,chunk,left,right", [(60, 4, 20, 40, 2), (512, 2, 6, 30, 0)])
def test_attention_shapes_match_oracle(hidden, heads, chunk, left, right):
    c = svl_synth.config_au(2)
    c["audio_config"].update(hidden_size=hidden, num_attention_heads=heads,
                             attention_chunk_size=chunk, attention_context_left=left,
                             attention_context_right=right, output_proj_dims=40)
    w = svl_synth.audio_weights(c, 768, seed=11)
    gpu = A.AudioModel(A.AudioConfig.from_json_value(c), w, 768)
    om = O.OracleAudioModel(c, w, 768)
    masks = [np.ones(300, bool), np.ones(157, bool), np.ones(13, bool)]
    masks[0][41:45] = False       # interior masked frames inside a block
    masks[1][130:] = False        # padded tail
    mels = svl_synth.mel_clips([300, 157, 13], seed=9, masks=masks)
    got = gpu.forward_batch(mels, capture_hidden=True)
    for i, (g_, m) in enumerate(zip(got, mels)):
        o = om.forward(m.features, m.mask.astype(bool), True)
        np.testing.assert_allclose(np.stack(g_.hidden_states()), o["hidden_states"], atol=2e-4,
                                   rtol=1e-4)
        check(g_.pooled(), o["pooled"], f"hidden {hidden} clip {i} soft tokens")


def test_full_30_second_clip_one_layer():
    """2999 mel frames -> 1500 -> 750 tokens: every chunk block of a real clip."""
    c = svl_synth.config_au(1)
    w = svl_synth.audio_weights(c, 768, seed=6)
    gpu = A.AudioModel(A.AudioConfig.from_json_value(c), w, 768)
    mel = svl_synth.mel_clips([2999], seed=3)[0]
    out = gpu.forward(mel, capture_hidden=True)
    assert out.audio_tokens() == 750
    ref = O.OracleAudioModel(c, w, 768).forward(mel.features, mel.mask.astype(bool), True)
    np.testing.assert_allclose(out.sscp_output(), ref["sscp_output"], atol=1e-4, rtol=1e-4)
    np.testing.assert_allclose(out.hidden_states()[0], ref["hidden_states"][0], atol=2e-4,
                               rtol=1e-4)
    check(out.pooled(), ref["pooled"], "30 s clip soft tokens")


TOKENS = A.AudioSpecialTokens(bos=2, eos=1, pad=0, boa=1000, audio=1001, eoa=1002)


def test_audio_embedder_matches_oracle():
    import torch
    tc = svl_synth.config_a(layers=2, vocab=1024)
    c = svl_synth.config_au(2, text=tc)
    tw = svl_synth.weights(tc, seed=3)
    aw = svl_synth.audio_weights(c, 768, seed=8)
    tm = S.TextModel(S.TextConfig.from_json_value(tc), tw)
    am = A.AudioModel(A.AudioConfig.from_json_value(c), aw, 768)
    emb = A.AudioEmbedder(tm, am, TOKENS)
    mels = svl_synth.mel_clips([120, 61], seed=4)
    ot, oa = O.OracleTextModel(tc, tw), O.OracleAudioModel(c, aw, 768)
    for dim in (768, 128):
        got = emb.embed_batch(mels, dim)
        for i, m in enumerate(mels):
            soft = oa.forward(m.features, m.mask.astype(bool))["pooled"]
            n = soft.shape[0]
            ids = [TOKENS.bos, TOKENS.boa] + [TOKENS.audio] * n + [TOKENS.eoa, TOKENS.eos]
            ref = ot.forward(ids, features=soft, feature_start=2, feature_count=n)["normalized"]
            check(got[i], O.truncate_and_normalize(ref, dim), f"clip {i} dim {dim}")
    one = emb.embed_mel(mels[1], 768)
    batch = emb.embed_batch(mels, 768)
    assert np.array_equal(one, batch[1])
    # the prompts through the text encoder in one pass each (a 20-token pass budget)
    tm.set_pass_tokens(20)
    try:
        assert emb.embed_batch(mels, 768).tobytes() == batch.tobytes()
    finally:
        tm.set_pass_tokens(0)
    feats = torch.from_numpy(np.concatenate([m.features for m in mels])).to("cuda:0")
    torch.cuda.synchronize()
    assert np.array_equal(emb.embed_device(feats.data_ptr(), mels, 768), batch)
    for dim in (0, 769):
        with pytest.raises(S.SvlError) as e:
            emb.embed_mel(mels[0], dim)
        assert e.value.kind == "Internal"


def test_audio_error_taxonomy(tiny):
    cfg, g, w, tm, am = tiny
    feats = np.array(g["mel_features"], np.float32)
    with pytest.raises(S.SvlError) as e:
        am.forward(A.MelSpectrogram(feats[:0], np.zeros(0, bool)))
    assert e.value.kind == "Corrupt"
    mask = np.ones(12, bool)
    mask[::4] = False  # every subsampled row reads a masked frame
    with pytest.raises(S.SvlError) as e:
        am.forward(A.MelSpectrogram(feats, mask))
    assert e.value.kind == "Corrupt"
    ok = am.forward(A.MelSpectrogram(feats, np.ones(12, bool))).pooled()
    assert np.isfinite(ok).all()

    ac = A.AudioConfig.from_json_value(cfg)
    bad = dict(w)
    bad["audio_tower.layers.0.self_attn.q_proj.input_min"] = np.array(30.0, np.float32)
    with pytest.raises(S.SvlError) as e:
        A.AudioModel(ac, bad, 16)
    assert e.value.kind == "Corrupt" and "inverted" in str(e.value)
    missing = dict(w)
    del missing["audio_tower.layers.1.lconv1d.conv_norm.weight"]
    with pytest.raises(S.SvlError) as e:
        A.AudioModel(ac, missing, 16)
    assert e.value.kind == "Corrupt"
    extra = dict(w)
    extra["audio_tower.layers.2.norm_out.weight"] = np.ones(16, np.float32)
    with pytest.raises(S.SvlError) as e:
        A.AudioModel(ac, extra, 16)
    assert e.value.kind == "Corrupt"


def test_config_au_full_depth_on_30_second_clips():
    """Config AU at its full 12 layers on the audio workload's own input:
    four 30 s clips of three sines plus noise (seed 3) through the GPU log-mel
    front end (2999 frames, 750 tokens each), then the 754-token audio prompt
    through the 24-layer shape-A text encoder (vocab 262144).

    Each stage is checked from the GPU's own input to that stage, as the scalar
    oracle needs minutes for the whole tower: the SSCP output and layer 1
    against the oracle's one-layer tower, layers 6 and 12 against the oracle's
    single-layer path (the forward pass's own per-layer code) applied to the
    GPU's layer 5 and 11 outputs, and the output projection + unscaled norm +
    text projection (audio.rs:1085-1133) in float64 from the GPU's layer-12
    output. The four-clip batch equals single calls bit for bit, and the
    prompt's embedding at dims 768 and 128 matches the text oracle run on the
    GPU's soft tokens (audio_embedder.rs:223-267)."""
    tc = svl_synth.config_a()
    c = svl_synth.config_au(12, text=tc)
    aw = svl_synth.audio_weights(c, 768, seed=0)
    am = A.AudioModel(A.AudioConfig.from_json_value(c), aw, 768)
    clips = svl_synth.sine_clips(4, seed=3)
    mels = A.LogMel.get().compute_batch(clips)
    assert all(m.frames == 2999 and m.audio_tokens() == 750 for m in mels)

    batch = am.forward_batch(mels)
    out = am.forward(mels[0], capture_hidden=True)
    assert np.array_equal(out.pooled(), batch[0].pooled())
    assert np.array_equal(am.forward(mels[3]).pooled(), batch[3].pooled())
    hs = out.hidden_states()
    assert len(hs) == 12 and hs[0].shape == (750, 1024)
    for h in hs:
        assert np.isfinite(h).all()

    tw = svl_synth.weights(tc, seed=0)
    tm = S.TextModel(S.TextConfig.from_json_value(tc), tw)
    emb = A.AudioEmbedder(tm, am, A.AudioSpecialTokens())
    got = {d: emb.embed_mel(mels[0], d) for d in (768, 128)}
    soft = out.pooled()
    tokens = A.AudioSpecialTokens()
    ids = [tokens.bos, tokens.boa] + [tokens.audio] * 750 + [tokens.eoa, tokens.eos]

    om12 = O.OracleAudioModel(c, aw, 768)
    om1 = O.OracleAudioModel(svl_synth.config_au(1, text=tc), aw, 768)
    ot = O.OracleTextModel(tc, tw)
    valid = np.ones(750, bool)
    with ThreadPoolExecutor(max_workers=4) as ex:
        f_text = ex.submit(lambda: ot.forward(ids, features=soft, feature_start=2,
                                              feature_count=750)["normalized"])
        f_one = ex.submit(lambda: om1.forward(mels[0].features, mels[0].mask.astype(bool), True))
        f_l6 = ex.submit(lambda: om12.layer(5, hs[4], valid))
        f_l12 = ex.submit(lambda: om12.layer(11, hs[10], valid))

        def rel(g, r):
            return float(np.abs(np.asarray(g, np.float64) - r).max() / np.abs(r).max())

        one = f_one.result()
        e = rel(out.sscp_output(), one["sscp_output"])
        print(f"SSCP output: relative max error {e:.3g}", flush=True)
        assert e <= 1e-4
        for label, g_, r_ in (("layer 1", hs[0], one["hidden_states"][0]),
                              ("layer 6", hs[5], f_l6.result()),
                              ("layer 12", hs[11], f_l12.result())):
            e = rel(g_, r_)
            print(f"{label}: relative max error {e:.3g}", flush=True)
            assert e <= 1e-4, label

        G = "audio_tower.output_proj"
        p = hs[11].astype(np.float64) @ aw[G + ".weight"].astype(np.float64).T + \
            aw[G + ".bias"].astype(np.float64)
        p = p / np.sqrt((p * p).mean(1, keepdims=True) + 1e-6)
        want = p @ aw["embed_audio.embedding_projection.weight"].astype(np.float64).T
        check(soft, want, "soft tokens from the layer-12 output")

        ref = f_text.result()
    for d in (768, 128):
        check(got[d], O.truncate_and_normalize(ref, d), f"754-token audio prompt dim {d}")
