/*
 * CPU oracle, audio front end: a C restatement of the log-mel spectrogram of
 * src/media/audio_preprocess.rs (log_mel :94-200, hann_window :203-210,
 * mel_filter_bank :212-244, the radix-2 FftPlan :279-333).
 *
 * TEST INFRASTRUCTURE ONLY: the oracle for the HIP log-mel kernel, never part
 * of the product library. Built with -ffp-contract=off and no fast-math; the
 * FFT, the magnitudes and the mel projection run in double in the reference's
 * order with the platform libm (cos, sin, pow, log10, log), and each feature
 * is rounded to float once.
 *
 * Parity pins (tests/test_oracle_mel.py): the tiny audio fixture's 12x128 mel
 * matrix (tests/audio_tiny.rs:95-110, 2e-5), the first values, frame counts
 * and padded lengths of the six WAV cases of
 * fixtures/media/audio_preprocess_golden.json (tests/audio.rs:44-100, 1e-5),
 * the unit tests of audio_preprocess.rs:335-423, the FFT against a direct DFT
 * and against numpy.fft, and the whole spectrogram against an independent
 * numpy restatement built on numpy.fft.rfft.
 */
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "svl_oracle.h"

#define MEL_PI 3.14159265358979323846264338327950288

static int mel_fail(char *msg, size_t msg_len, int code, const char *fmt, ...) {
    if (msg && msg_len) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(msg, msg_len, fmt, ap);
        va_end(ap);
    }
    return code;
}

/* audio_preprocess.rs:203-210, periodic Hann window rounded to float. */
void svlo_hann_window(float *out) {
    for (size_t i = 0; i < SVLO_MEL_FRAME_LENGTH; ++i) {
        const double angle = 2.0 * MEL_PI * (double)i / (double)SVLO_MEL_FRAME_LENGTH;
        out[i] = (float)(0.5 - 0.5 * cos(angle));
    }
}

static double hertz_to_mel(double f) { return 2595.0 * log10(1.0 + f / 700.0); }
static double mel_to_hertz(double m) { return 700.0 * (pow(10.0, m / 2595.0) - 1.0); }

/* audio_preprocess.rs:212-244; out [257 bins, 128 filters]. */
int svlo_mel_filter_bank(double *out) {
    const double nyquist = 16000.0 / 2.0;
    const double mel_min = hertz_to_mel(0.0), mel_max = hertz_to_mel(8000.0);
    double freqs[SVLO_MEL_FEATURES + 2];
    for (size_t i = 0; i <= SVLO_MEL_FEATURES + 1; ++i) {
        const double fraction = (double)i / (double)(SVLO_MEL_FEATURES + 1);
        freqs[i] = mel_to_hertz(mel_min + (mel_max - mel_min) * fraction);
    }
    for (size_t bin = 0; bin < SVLO_MEL_BINS; ++bin) {
        const double frequency = nyquist * (double)bin / (double)(SVLO_MEL_BINS - 1);
        for (size_t f = 0; f < SVLO_MEL_FEATURES; ++f) {
            const double lower = freqs[f], center = freqs[f + 1], upper = freqs[f + 2];
            const double down = (frequency - lower) / (center - lower);
            const double up = (upper - frequency) / (upper - center);
            /* f64::min / f64::max: neither operand is NaN here */
            double v = down < up ? down : up;
            v = v > 0.0 ? v : 0.0;
            if (!isfinite(v)) return SVLO_INTERNAL;
            out[bin * SVLO_MEL_FEATURES + f] = v;
        }
    }
    return SVLO_OK;
}

static size_t reverse_bits(size_t v, unsigned bits) {
    size_t r = 0;
    for (unsigned b = 0; b < bits; ++b) r |= ((v >> b) & 1u) << (bits - 1 - b);
    return r;
}

/* FftPlan::new + forward (audio_preprocess.rs:279-333): in-place iterative
 * radix-2 on interleaved (re, im) doubles; n a power of two. */
int svlo_fft(double *values, size_t n) {
    if (n == 0 || (n & (n - 1))) return SVLO_INTERNAL;
    unsigned bits = 0;
    while (((size_t)1 << bits) < n) ++bits;
    double *tw = (double *)malloc(sizeof(double) * (n > 1 ? n : 2));
    if (!tw) return SVLO_INTERNAL;
    for (size_t i = 0; i < n / 2; ++i) {
        const double angle = -2.0 * MEL_PI * (double)i / (double)n;
        tw[2 * i] = cos(angle);
        tw[2 * i + 1] = sin(angle);
    }
    for (size_t i = 0; i < n; ++i) {
        const size_t t = reverse_bits(i, bits);
        if (i < t) {
            const double r = values[2 * i], im = values[2 * i + 1];
            values[2 * i] = values[2 * t];
            values[2 * i + 1] = values[2 * t + 1];
            values[2 * t] = r;
            values[2 * t + 1] = im;
        }
    }
    for (size_t span = 2; span <= n; span *= 2) {
        const size_t half = span / 2, step = n / span;
        for (size_t start = 0; start < n; start += span)
            for (size_t off = 0; off < half; ++off) {
                const double tr = tw[2 * off * step], ti = tw[2 * off * step + 1];
                double *e = values + 2 * (start + off), *o = values + 2 * (start + off + half);
                const double odr = o[0] * tr - o[1] * ti;
                const double odi = o[0] * ti + o[1] * tr;
                const double er = e[0], ei = e[1];
                e[0] = er + odr;
                e[1] = ei + odi;
                o[0] = er - odr;
                o[1] = ei - odi;
            }
    }
    free(tw);
    return SVLO_OK;
}

/* Frame layout of log_mel (audio_preprocess.rs:103-131). */
int svlo_log_mel_layout(size_t samples, size_t *frames, size_t *padded_samples,
                        size_t *valid_frames, char *msg, size_t msg_len) {
    if (samples == 0) return mel_fail(msg, msg_len, SVLO_CORRUPT, "audio contains no samples");
    if (samples > SVLO_MEL_MAX_SAMPLES) samples = SVLO_MEL_MAX_SAMPLES;
    const size_t padded = (samples + SVLO_MEL_PAD_TO - 1) / SVLO_MEL_PAD_TO * SVLO_MEL_PAD_TO;
    const size_t padded_len = padded + SVLO_MEL_FRAME_LENGTH / 2;
    if (padded_len < SVLO_MEL_FRAME_LENGTH + 1)
        return mel_fail(msg, msg_len, SVLO_CORRUPT,
                        "audio has %zu samples, too short for one analysis frame", samples);
    const size_t n = (padded_len - (SVLO_MEL_FRAME_LENGTH + 1)) / SVLO_MEL_HOP + 1;
    if (n > SVLO_MEL_MAX_FRAMES)
        return mel_fail(msg, msg_len, SVLO_LIMIT, "audio produces %zu mel frames", n);
    size_t valid = 0;
    for (size_t t = 0; t < n; ++t)
        if (t * SVLO_MEL_HOP + SVLO_MEL_FRAME_LENGTH / 2 < samples) ++valid;
    if (frames) *frames = n;
    if (padded_samples) *padded_samples = padded;
    if (valid_frames) *valid_frames = valid;
    return SVLO_OK;
}

/*
 * log_mel (audio_preprocess.rs:94-200). samples are the 16 kHz mono input
 * (truncated at SVLO_MEL_MAX_SAMPLES); features receives [frames, 128] and
 * mask [frames] (0/1), with frames from svlo_log_mel_layout.
 */
int svlo_log_mel(const float *samples, size_t n_samples, float *features, unsigned char *mask,
                 char *msg, size_t msg_len) {
    if (n_samples == 0) return mel_fail(msg, msg_len, SVLO_CORRUPT, "audio contains no samples");
    for (size_t i = 0; i < n_samples; ++i)
        if (!isfinite(samples[i]))
            return mel_fail(msg, msg_len, SVLO_CORRUPT, "audio contains a non-finite sample");
    if (n_samples > SVLO_MEL_MAX_SAMPLES) n_samples = SVLO_MEL_MAX_SAMPLES;
    size_t frames = 0, padded = 0, valid_frames = 0;
    int st = svlo_log_mel_layout(n_samples, &frames, &padded, &valid_frames, msg, msg_len);
    if (st) return st;

    float window[SVLO_MEL_FRAME_LENGTH];
    svlo_hann_window(window);
    double *filters = (double *)malloc(sizeof(double) * SVLO_MEL_BINS * SVLO_MEL_FEATURES);
    double *spectrum = (double *)malloc(sizeof(double) * 2 * SVLO_MEL_FFT);
    if (!filters || !spectrum) {
        free(filters);
        free(spectrum);
        return mel_fail(msg, msg_len, SVLO_INTERNAL, "out of memory");
    }
    st = svlo_mel_filter_bank(filters);
    if (st) {
        free(filters);
        free(spectrum);
        return mel_fail(msg, msg_len, st, "mel filter bank produced a non-finite value");
    }
    double magnitudes[SVLO_MEL_BINS];
    for (size_t t = 0; t < frames; ++t) {
        const size_t start = t * SVLO_MEL_HOP;
        const int valid = start + SVLO_MEL_FRAME_LENGTH / 2 < n_samples;
        mask[t] = (unsigned char)valid;
        float *row = features + t * SVLO_MEL_FEATURES;
        if (!valid) {
            memset(row, 0, sizeof(float) * SVLO_MEL_FEATURES);
            continue;
        }
        for (size_t i = 0; i < SVLO_MEL_FFT; ++i) {
            float v = 0.0f;
            if (i < SVLO_MEL_FRAME_LENGTH && start + i >= SVLO_MEL_FRAME_LENGTH / 2) {
                const size_t src = start + i - SVLO_MEL_FRAME_LENGTH / 2;
                const float s = (src < padded && src < n_samples) ? samples[src] : 0.0f;
                v = s * window[i];
            }
            spectrum[2 * i] = (double)v;
            spectrum[2 * i + 1] = 0.0;
        }
        svlo_fft(spectrum, SVLO_MEL_FFT);
        for (size_t b = 0; b < SVLO_MEL_BINS; ++b) {
            const double re = spectrum[2 * b], im = spectrum[2 * b + 1];
            magnitudes[b] = sqrt(re * re + im * im);
        }
        for (size_t f = 0; f < SVLO_MEL_FEATURES; ++f) {
            double energy = 0.0;
            for (size_t b = 0; b < SVLO_MEL_BINS; ++b)
                energy += magnitudes[b] * filters[b * SVLO_MEL_FEATURES + f];
            row[f] = (float)log(energy + SVLO_MEL_FLOOR);
        }
    }
    free(filters);
    free(spectrum);
    if (valid_frames == 0)
        return mel_fail(msg, msg_len, SVLO_CORRUPT,
                        "audio has no complete analysis window and cannot be embedded");
    for (size_t i = 0; i < frames * SVLO_MEL_FEATURES; ++i)
        if (!isfinite(features[i]))
            return mel_fail(msg, msg_len, SVLO_INTERNAL,
                            "audio preprocessing produced a non-finite mel value");
    return SVLO_OK;
}
