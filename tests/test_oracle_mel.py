"""Pins of the log-mel oracle (oracle/svl_oracle_mel.c, a restatement of
src/media/audio_preprocess.rs):

* the six WAV cases of fixtures/media/audio_preprocess_golden.json (produced
  by the official feature extractor): sample counts, padded lengths, frame
  and valid-frame counts, and the first mel values at the 1e-5 bar of
  tests/audio.rs:44-100;
* the tiny audio fixture's full 12x128 mel matrix at the 2e-5 bar of
  tests/audio_tiny.rs:95-110 (every filter of the bank);
* the unit tests of audio_preprocess.rs:335-423 (Hann window values, FFT
  against a direct DFT, filter-bank shape, error kinds, the semicausal frame
  layout);
* the periodic Hann window against scipy.signal.get_window, the FFT against
  numpy.fft.fft, and whole spectrograms against a second pipeline built on
  numpy.fft.rfft and a matrix product (a different FFT algorithm and a
  different summation order must agree to float rounding).

The golden's SHA-256 of the features was computed from NumPy's FFT; it is
reproduced exactly for the all-silent clip only, as the reference's own test
only prints the hash (tests/audio.rs:94-99)."""
import hashlib
import json
import os
import wave

import numpy as np
import pytest

from oracle import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
PRE = os.path.join(HERE, "golden", "audio_preprocess")
TINY = os.path.join(HERE, "golden", "tiny_audio", "golden.json")


def read_wav(name):
    """16-bit PCM mono 16 kHz fixture -> f32 samples (wav.rs:294-297: i16 / 32768)."""
    with wave.open(os.path.join(PRE, name + ".wav")) as w:
        assert (w.getnchannels(), w.getsampwidth(), w.getframerate()) == (1, 2, 16000)
        raw = np.frombuffer(w.readframes(w.getnframes()), "<i2")
    return raw.astype(np.float32) / np.float32(32768.0)


def golden_cases():
    return json.load(open(os.path.join(PRE, "golden.json")))["cases"]


@pytest.mark.parametrize("case", golden_cases(), ids=lambda c: c["name"])
def test_official_preprocessing_fixtures(case):
    x = read_wav(case["name"])
    assert x.size == case["samples"]
    feats, mask, padded, valid = O.log_mel(x)
    assert padded == case["padded_samples"]
    assert feats.shape == (case["mel_frames"], 128)
    assert valid == case["valid_mel_frames"] == int(mask.sum())
    first = np.array(case["mel_features_first"], np.float32)
    assert np.abs(feats.ravel()[: first.size] - first).max() <= 1e-5
    if case["name"] == "silence_1s":
        sha = hashlib.sha256(feats.astype("<f4").tobytes()).hexdigest()
        assert sha == case["mel_features_sha256"]


def test_tiny_audio_mel_matrix():
    g = json.load(open(TINY))
    feats, mask, padded, valid = O.log_mel(np.array(g["samples"], np.float32))
    expected = np.array(g["mel_features"], np.float32)
    assert feats.shape == expected.shape == (12, 128) and valid == 12 and mask.all()
    assert np.all(np.abs(feats - expected) <= 2e-5 + 2e-5 * np.abs(expected))
    assert [bool(v) for v in mask] == g["mel_mask"]


def test_hann_window():
    # audio_preprocess.rs:339-345 and the periodic Hann of scipy
    from scipy.signal import get_window
    w = O.hann_window()
    assert abs(w[0]) <= 1e-7 and abs(w[160] - 1.0) <= 1e-6 and abs(w[319] - 0.000096) <= 1e-5
    ref = get_window("hann", 320, fftbins=True)
    assert np.abs(w.astype(np.float64) - ref).max() <= 6e-8


def test_fft_matches_direct_dft_and_numpy():
    # audio_preprocess.rs:348-372
    x = np.sin(np.arange(16) * 0.7).astype(np.complex128)
    got = O.fft(x)
    k = np.arange(16)
    dft = (x[None, :] * np.exp(-2j * np.pi * np.outer(k, k) / 16)).sum(axis=1)
    assert np.abs(got - dft).max() <= 1e-9
    rng = np.random.default_rng(0)
    y = rng.standard_normal(512) + 1j * rng.standard_normal(512)
    assert np.abs(O.fft(y) - np.fft.fft(y)).max() <= 1e-9 * np.abs(np.fft.fft(y)).max()


def test_filter_bank_shape():
    # audio_preprocess.rs:375-384
    f = O.mel_filter_bank()
    assert f.shape == (257, 128)
    assert (f >= 0).all() and (f <= 1).all() and f[0, 0] == 0.0 and (f > 0).any()
    # the non-zero weights of a filter form one run of bins; the lowest
    # filters are narrower than the 31.25 Hz bin spacing and can be empty
    # (their energy is exactly 0, their feature ln(0.001))
    empty = 0
    for j in range(128):
        nz = np.flatnonzero(f[:, j])
        empty += nz.size == 0
        assert nz.size == 0 or nz[-1] - nz[0] + 1 == nz.size
        assert nz.size > 0 or j < 4
    assert 1 <= empty <= 4
    assert (f[:, 64:] > 0).sum(axis=0).min() >= 2


def test_rejects_empty_non_finite_and_short_audio():
    # audio_preprocess.rs:386-391
    for bad in ([], [np.nan], [0.0] * 10):
        with pytest.raises(O.OracleError) as e:
            O.log_mel(np.array(bad, np.float32))
        assert e.value.status == 4
    with pytest.raises(O.OracleError) as e:   # 150 samples: one frame, no complete window
        O.log_mel(np.zeros(150, np.float32))
    assert e.value.status == 4
    x = np.zeros(480001, np.float32)
    x[-1] = np.inf                               # checked before the 30 s truncation
    with pytest.raises(O.OracleError):
        O.log_mel(x)


def test_semicausal_layout():
    # audio_preprocess.rs:393-406
    feats, mask, padded, valid = O.log_mel(np.zeros(1600, np.float32))
    assert feats.shape == (10, 128) and valid == 9 and padded == 1664
    assert list(mask) == [True] * 9 + [False]
    assert (feats[9] == 0).all()
    assert np.all(feats[:9] == np.float32(np.log(0.001)))


@pytest.mark.parametrize("n", [161, 320, 481, 1600, 2000, 16000, 479999, 480000, 480001, 600000])
def test_layout_closed_form(n):
    frames, padded, valid = O.log_mel_layout(n)
    m = min(n, 480000)
    assert padded == -(-m // 128) * 128
    assert frames == (padded + 160 - 321) // 160 + 1
    assert valid == sum(1 for t in range(frames) if t * 160 + 160 < m)


def numpy_log_mel(x):
    """Second pipeline: frames gathered with numpy, numpy.fft.rfft, |X| and
    one matrix product with the oracle's filter bank."""
    m = min(x.size, 480000)
    x = x[:m]
    frames, padded, valid = O.log_mel_layout(m)
    w = O.hann_window()
    buf = np.zeros(160 + padded + 512, np.float32)
    buf[160:160 + m] = x
    idx = np.arange(frames)[:, None] * 160 + np.arange(320)[None, :]
    windowed = (buf[idx] * w[None, :]).astype(np.float64)
    spec = np.abs(np.fft.rfft(windowed, n=512, axis=1))
    out = np.log(spec @ O.mel_filter_bank() + 0.001).astype(np.float32)
    mask = np.arange(frames) * 160 + 160 < m
    out[~mask] = 0
    return out, mask


@pytest.mark.parametrize("source", ["french_speech", "rain_noise_2s", "noise_30s", "tone_35s"])
def test_whole_spectrogram_against_numpy_fft(source):
    rng = np.random.default_rng(7)
    if source == "noise_30s":
        x = rng.uniform(-1, 1, 480000).astype(np.float32)
    elif source == "tone_35s":
        t = np.arange(560000) / 16000
        x = (0.4 * np.sin(2 * np.pi * 440 * t) + 0.01 * rng.standard_normal(t.size)).astype(
            np.float32)
    else:
        x = read_wav(source)
    got, mask, _, _ = O.log_mel(x)
    ref, ref_mask = numpy_log_mel(x)
    assert np.array_equal(mask, ref_mask)
    assert np.abs(got - ref).max() <= 4e-6
