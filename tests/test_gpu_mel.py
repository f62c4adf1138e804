"""GPU parity of the log-mel front end (log_mel, src/media/audio_preprocess.rs:
94-200) and of the audio embedder fed with 16 kHz samples
(AudioEmbedder::embed, src/model/audio_embedder.rs:214-267), through the
C ABI.

The bar is bit-exactness against the oracle: the kernel evaluates the
reference's double-precision FFT, magnitudes and mel sums in the same order
with the same twiddles and filter weights. Cases: the six official WAV
fixtures (and their first values at tests/audio.rs:87-93's 1e-5), the tiny
audio fixture's 12 frames (tests/audio_tiny.rs:95-110), full 30 s clips of
noise, a batch of 30 s clips of sines plus noise, a 35 s clip (truncated), a
ragged batch with every layout boundary, the device-resident variant, the
error taxonomy, and the embedding of the tiny fixture's samples against its
golden embedding."""
import json
import os

import numpy as np
import pytest
from safetensors.numpy import load_file

import svl_amd as S
import svl_audio as A
import svl_synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
PRE = os.path.join(HERE, "golden", "audio_preprocess")
TINY = os.path.join(HERE, "golden", "tiny_audio")


def read_wav(name):
    import wave
    with wave.open(os.path.join(PRE, name + ".wav")) as w:
        raw = np.frombuffer(w.readframes(w.getnframes()), "<i2")
    return raw.astype(np.float32) / np.float32(32768.0)


def assert_bit_exact(mel, x, label):
    feats, mask, padded, _ = O.log_mel(x)
    diff = np.flatnonzero(mel.features.view(np.uint32) != feats.view(np.uint32))
    print(f"{label}: {mel.frames} frames, {diff.size} differing values", flush=True)
    assert mel.features.shape == feats.shape, label
    assert diff.size == 0, f"{label}: first differences at {diff[:5]}"
    assert np.array_equal(mel.mask.astype(bool), mask) and mel.padded_samples() == padded


@pytest.fixture(scope="module")
def lm():
    return A.LogMel.get(0)


def test_official_wav_fixtures_bit_exact(lm):
    cases = json.load(open(os.path.join(PRE, "golden.json")))["cases"]
    clips = [read_wav(c["name"]) for c in cases]
    mels = lm.compute_batch(clips)
    for c, x, mel in zip(cases, clips, mels):
        assert_bit_exact(mel, x, c["name"])
        assert mel.frames == c["mel_frames"] and mel.valid_frames() == c["valid_mel_frames"]
        first = np.array(c["mel_features_first"], np.float32)
        assert np.abs(mel.features.ravel()[: first.size] - first).max() <= 1e-5


def test_tiny_fixture_and_single_clip_api(lm):
    g = json.load(open(os.path.join(TINY, "golden.json")))
    x = np.array(g["samples"], np.float32)
    mel = A.log_mel(x)
    assert_bit_exact(mel, x, "tiny")
    e = np.array(g["mel_features"], np.float32)
    assert np.all(np.abs(mel.features - e) <= 2e-5 + 2e-5 * np.abs(e))
    assert np.array_equal(lm.compute(x).features, mel.features)


def test_full_and_truncated_clips(lm):
    rng = np.random.default_rng(11)
    noise = rng.uniform(-1, 1, 480000).astype(np.float32)
    loud = (rng.standard_normal(480000) * 30).astype(np.float32)   # large magnitudes
    t = np.arange(560000) / 16000
    tone = (0.5 * np.sin(2 * np.pi * 997 * t)).astype(np.float32)  # 35 s -> truncated
    for x, label in ((noise, "noise 30 s"), (loud, "loud 30 s"), (tone, "tone 35 s")):
        mel = lm.compute(x)
        assert mel.frames == 2999
        assert_bit_exact(mel, x, label)


def test_sine_and_noise_batch(lm):
    # The audio throughput workload: 4 x 30 s of three sines (100-4000 Hz)
    # plus N(0, 0.05^2) noise, computed as one batch.
    clips = svl_synth.sine_clips(4, seed=3)
    mels = lm.compute_batch(clips)
    for i, (x, mel) in enumerate(zip(clips, mels)):
        assert mel.frames == 2999 and mel.valid_frames() == 2999
        assert_bit_exact(mel, x, f"sine clip {i}")


def test_ragged_batch_and_device_path(lm):
    import torch
    rng = np.random.default_rng(12)
    lengths = [1600, 161, 2000, 481, 12345, 480001, 320, 16000]
    clips = [rng.uniform(-0.8, 0.8, n).astype(np.float32) for n in lengths]
    mels = lm.compute_batch(clips)
    for i, (x, mel) in enumerate(zip(clips, mels)):
        assert_bit_exact(mel, x, f"clip {i} ({x.size} samples)")
    d_x = torch.from_numpy(np.concatenate(clips)).to("cuda:0")
    total = sum(m.frames for m in mels)
    d_f = torch.full((total, 128), float("nan"), device="cuda:0")
    torch.cuda.synchronize()
    masks = lm.compute_device(d_x.data_ptr(), lengths, d_f.data_ptr())
    got = d_f.cpu().numpy()
    assert np.array_equal(got.view(np.uint32),
                          np.concatenate([m.features for m in mels]).view(np.uint32))
    for m, mask in zip(mels, masks):
        assert np.array_equal(m.mask.astype(bool), mask)
    assert lm.compute_batch([]) == []


def test_error_taxonomy(lm):
    import torch
    for bad in ([], [0.0] * 10, [0.0] * 150):
        with pytest.raises(S.SvlError) as e:
            lm.compute(np.array(bad, np.float32))
        assert e.value.kind == "Corrupt"
    x = np.zeros(480005, np.float32)
    x[480002] = np.nan  # beyond the 30 s cap, still rejected (audio_preprocess.rs:98-100)
    with pytest.raises(S.SvlError) as e:
        lm.compute(x)
    assert e.value.kind == "Corrupt" and "non-finite" in str(e.value)
    d = torch.from_numpy(np.concatenate([np.zeros(1600, np.float32), x])).to("cuda:0")
    out = torch.empty((20 + 2999, 128), device="cuda:0")
    torch.cuda.synchronize()
    with pytest.raises(S.SvlError) as e:
        lm.compute_device(d.data_ptr(), [1600, x.size], out.data_ptr())
    assert e.value.kind == "Corrupt"
    ok = lm.compute(np.zeros(1600, np.float32))   # the object stays usable
    assert ok.frames == 10


def test_embedding_from_samples_matches_the_official_fixture():
    """tests/audio_tiny.rs:95-200: samples -> log-mel -> tower -> embedding."""
    cfg = json.load(open(os.path.join(TINY, "config.json")))
    g = json.load(open(os.path.join(TINY, "golden.json")))
    w = load_file(os.path.join(TINY, "model.safetensors"))
    tm = S.TextModel(S.TextConfig.from_json_value(cfg), w)
    am = A.AudioModel(A.AudioConfig.from_json_value(cfg), w, 16)
    emb = A.AudioEmbedder(tm, am, A.AudioSpecialTokens(bos=1, eos=2, pad=0, boa=3, audio=4,
                                                       eoa=5))
    x = np.array(g["samples"], np.float32)
    e = emb.embed(x, 8)
    exp = np.array(g["embedding"], np.float64)
    cos = float(e @ exp / (np.linalg.norm(e) * np.linalg.norm(exp)))
    print(f"tiny embedding from samples: cosine {cos:.9f} max-abs {np.abs(e - exp).max():.3g}",
          flush=True)
    assert cos >= 0.9999 and np.abs(e - exp).max() <= 1e-4
    # the same bits as the mel route with the oracle's spectrogram
    feats, mask, _, _ = O.log_mel(x)
    assert np.array_equal(e, emb.embed_mel(A.MelSpectrogram(feats, mask), 8))


def test_batched_and_device_sample_embedding():
    import torch
    tc = svl_synth.config_a(layers=2, vocab=1024)
    c = svl_synth.config_au(2, text=tc)
    tm = S.TextModel(S.TextConfig.from_json_value(tc), svl_synth.weights(tc, seed=3))
    am = A.AudioModel(A.AudioConfig.from_json_value(c), svl_synth.audio_weights(c, 768, seed=8),
                      768)
    emb = A.AudioEmbedder(tm, am, A.AudioSpecialTokens(bos=2, eos=1, pad=0, boa=1000,
                                                       audio=1001, eoa=1002))
    rng = np.random.default_rng(13)
    clips = [rng.uniform(-0.5, 0.5, n).astype(np.float32) for n in (16000, 4321, 48000)]
    got = emb.embed_samples_batch(clips, 768)
    ref = emb.embed_batch([O_mel(x) for x in clips], 768)
    assert np.array_equal(got, ref)
    assert np.array_equal(emb.embed(clips[1], 768), got[1])
    d = torch.from_numpy(np.concatenate(clips)).to("cuda:0")
    torch.cuda.synchronize()
    assert np.array_equal(emb.embed_samples_device(d.data_ptr(), [x.size for x in clips], 768),
                          got)
    with pytest.raises(S.SvlError) as e:
        emb.embed_samples_batch([clips[0], np.zeros(100, np.float32)], 768)
    assert e.value.kind == "Corrupt"


def O_mel(x):
    feats, mask, _, _ = O.log_mel(x)
    return A.MelSpectrogram(feats, mask)
