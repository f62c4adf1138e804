// Host runtime of the log-mel front end (the svl_log_mel_* part of
// include/svl_hip.h): the reference's log_mel (src/media/audio_preprocess.rs:
// 94-200) with the per-frame FFT and mel projection on the GPU.
//
// The constant tables are built once per object on the host in double with
// the platform libm, exactly as the reference builds them (Hann window :203-
// 210, FFT twiddles :288-297, HTK filter bank :212-244), so the device
// pipeline sees the same operands; the filter bank is stored sparsely (the
// non-zero weights of each triangular filter, in bin order).
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <memory>
#include <vector>

#include "../../include/svl_hip.h"
#include "mel_host.hpp"

namespace {

using namespace svl;

// audio_preprocess.rs:24-46, media/audio.rs:16-19.
constexpr int64_t FRAME_LENGTH = 320;
constexpr int64_t HOP_LENGTH = 160;
constexpr int64_t FFT_LENGTH = 512;
constexpr int64_t FEATURE_SIZE = 128;
constexpr int64_t FREQUENCY_BINS = FFT_LENGTH / 2 + 1;
constexpr int64_t PAD_TO_MULTIPLE = 128;
constexpr int64_t MAX_MEL_FRAMES = 3000;
constexpr int64_t MAX_AUDIO_SAMPLES = 480000;
constexpr double SAMPLE_RATE = 16000.0;
constexpr double PI = 3.14159265358979323846264338327950288;

double hertz_to_mel(double f) { return 2595.0 * std::log10(1.0 + f / 700.0); }
double mel_to_hertz(double m) { return 700.0 * (std::pow(10.0, m / 2595.0) - 1.0); }

// [bins, filters] dense HTK bank (audio_preprocess.rs:212-244).
svl_status filter_bank(std::vector<double> &out) {
    const double nyquist = SAMPLE_RATE / 2.0;
    const double lo = hertz_to_mel(0.0), hi = hertz_to_mel(8000.0);
    std::vector<double> edges((size_t)FEATURE_SIZE + 2);
    for (int64_t i = 0; i <= FEATURE_SIZE + 1; ++i)
        edges[(size_t)i] = mel_to_hertz(lo + (hi - lo) * ((double)i / (double)(FEATURE_SIZE + 1)));
    out.assign((size_t)(FREQUENCY_BINS * FEATURE_SIZE), 0.0);
    for (int64_t b = 0; b < FREQUENCY_BINS; ++b) {
        const double freq = nyquist * (double)b / (double)(FREQUENCY_BINS - 1);
        for (int64_t f = 0; f < FEATURE_SIZE; ++f) {
            const double rise = (freq - edges[(size_t)f]) / (edges[(size_t)f + 1] - edges[(size_t)f]);
            const double fall =
                (edges[(size_t)f + 2] - freq) / (edges[(size_t)f + 2] - edges[(size_t)f + 1]);
            const double v = std::max(std::min(rise, fall), 0.0);
            if (!std::isfinite(v)) return fail(SVL_INTERNAL, "mel filter bank produced a non-finite value");
            out[(size_t)(b * FEATURE_SIZE + f)] = v;
        }
    }
    return SVL_OK;
}

svl_status layout(int64_t n, int64_t *frames, int64_t *padded, int64_t *valid) {
    if (n <= 0) return fail(SVL_CORRUPT, "audio contains no samples");
    n = std::min(n, MAX_AUDIO_SAMPLES);
    const int64_t pad = (n + PAD_TO_MULTIPLE - 1) / PAD_TO_MULTIPLE * PAD_TO_MULTIPLE;
    const int64_t padded_len = pad + FRAME_LENGTH / 2;
    if (padded_len < FRAME_LENGTH + 1)
        return fail(SVL_CORRUPT,
                    "audio has %lld samples, too short for one %lld-sample analysis frame",
                    (long long)n, (long long)FRAME_LENGTH);
    const int64_t f = (padded_len - (FRAME_LENGTH + 1)) / HOP_LENGTH + 1;
    if (f > MAX_MEL_FRAMES)
        return fail(SVL_LIMIT, "audio produces %lld mel frames, above the %lld-frame cap",
                    (long long)f, (long long)MAX_MEL_FRAMES);
    // frame t is valid when t * hop + frame / 2 < n
    const int64_t v = std::min(f, n > FRAME_LENGTH / 2
                                      ? (n - FRAME_LENGTH / 2 - 1) / HOP_LENGTH + 1
                                      : (int64_t)0);
    if (frames) *frames = f;
    if (padded) *padded = pad;
    if (valid) *valid = v;
    return SVL_OK;
}

}  // namespace

svl_log_mel::~svl_log_mel() {
    if (device >= 0) (void)hipSetDevice(device);
    window.release(); twiddle.release(); weight.release(); start.release(); bin.release();
    samples.release(); features.release(); clips.release(); flag.release();
    if (h_flag) (void)hipHostFree(h_flag);
    if (stream) (void)hipStreamDestroy(stream);
}

namespace svl {

svl_status mel_create_on(int device, svl_log_mel **out) {
    if (!out) return fail(SVL_USAGE, "output handle is required");
    *out = nullptr;
    std::unique_ptr<svl_log_mel> lm(new svl_log_mel());
    lm->device = device;
    HIP_TRY(hipSetDevice(device));
    HIP_TRY(hipStreamCreateWithFlags(&lm->stream, hipStreamNonBlocking));
    HIP_TRY(hipHostMalloc((void **)&lm->h_flag, 2 * sizeof(int), hipHostMallocDefault));

    std::vector<float> window((size_t)FRAME_LENGTH);
    for (int64_t i = 0; i < FRAME_LENGTH; ++i) {
        const double angle = 2.0 * PI * (double)i / (double)FRAME_LENGTH;
        window[(size_t)i] = (float)(0.5 - 0.5 * std::cos(angle));
    }
    std::vector<double> tw((size_t)FFT_LENGTH);  // (cos, sin) pairs
    for (int64_t i = 0; i < FFT_LENGTH / 2; ++i) {
        const double angle = -2.0 * PI * (double)i / (double)FFT_LENGTH;
        tw[(size_t)(2 * i)] = std::cos(angle);
        tw[(size_t)(2 * i + 1)] = std::sin(angle);
    }
    std::vector<double> bank;
    ST_TRY(filter_bank(bank));
    std::vector<int32_t> start(1, 0), bins;
    std::vector<double> weights;
    for (int64_t f = 0; f < FEATURE_SIZE; ++f) {
        for (int64_t b = 0; b < FREQUENCY_BINS; ++b) {
            const double v = bank[(size_t)(b * FEATURE_SIZE + f)];
            if (v != 0.0) {
                bins.push_back((int32_t)b);
                weights.push_back(v);
            }
        }
        start.push_back((int32_t)bins.size());
    }
    HIP_TRY(lm->window.ensure(window.size()));
    HIP_TRY(lm->twiddle.ensure(tw.size()));
    HIP_TRY(lm->start.ensure(start.size()));
    HIP_TRY(lm->bin.ensure(bins.size()));
    HIP_TRY(lm->weight.ensure(weights.size()));
    HIP_TRY(lm->flag.ensure(2));
    HIP_TRY(hipMemcpy(lm->window.p, window.data(), window.size() * 4, hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(lm->twiddle.p, tw.data(), tw.size() * 8, hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(lm->start.p, start.data(), start.size() * 4, hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(lm->bin.p, bins.data(), bins.size() * 4, hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(lm->weight.p, weights.data(), weights.size() * 8, hipMemcpyHostToDevice));
    *out = lm.release();
    return SVL_OK;
}

svl_status mel_plan(const int64_t *lengths, int32_t clips, MelBatch &b) {
    if (clips < 0) return fail(SVL_USAGE, "negative clip count");
    if (clips > 0 && !lengths) return fail(SVL_USAGE, "clip lengths are null");
    b.clips.clear();
    b.mask.clear();
    b.frame_off.assign(1, 0);
    b.input_off.assign(1, 0);
    for (int32_t i = 0; i < clips; ++i) {
        int64_t frames = 0, padded = 0, valid = 0;
        const svl_status st = layout(lengths[i], &frames, &padded, &valid);
        if (st != SVL_OK) return fail(st, "clip %d: %s", i, g_err.c_str());
        if (valid == 0)
            return fail(SVL_CORRUPT,
                        "clip %d: audio has no complete analysis window and cannot be embedded", i);
        const int64_t used = std::min(lengths[i], MAX_AUDIO_SAMPLES);
        b.clips.push_back({0, b.frame_off.back(), (int32_t)used, (int32_t)frames});
        for (int64_t t = 0; t < frames; ++t) b.mask.push_back((uint8_t)(t < valid));
        b.frame_off.push_back(b.frame_off.back() + frames);
        b.input_off.push_back(b.input_off.back() + lengths[i]);
    }
    b.total_frames = b.frame_off.back();
    if (b.total_frames > (int64_t)INT32_MAX / FEATURE_SIZE)
        return fail(SVL_LIMIT, "batch holds too many mel frames");
    return SVL_OK;
}

svl_status mel_compute(svl_log_mel *lm, MelBatch &b, const float *const *h_samples,
                       const float *d_samples, const int64_t *lengths, float *d_out,
                       hipStream_t s) {
    const int32_t B = (int32_t)b.clips.size();
    if (B == 0) return SVL_OK;
    HIP_TRY(hipSetDevice(lm->device));
    HIP_TRY(hipMemsetAsync(lm->flag.p, 0, 2 * sizeof(int), s));
    const float *x = d_samples;
    if (h_samples) {
        int64_t packed = 0;
        for (int32_t i = 0; i < B; ++i) {
            if (!h_samples[i]) return fail(SVL_USAGE, "clip %d: samples are null", i);
            for (int64_t k = 0; k < lengths[i]; ++k)
                if (!std::isfinite(h_samples[i][k]))
                    return fail(SVL_CORRUPT, "clip %d: audio contains a non-finite sample", i);
            b.clips[(size_t)i].sample_base = packed;
            packed += b.clips[(size_t)i].samples;
        }
        HIP_TRY(lm->samples.ensure((size_t)packed));
        for (int32_t i = 0; i < B; ++i)
            HIP_TRY(hipMemcpyAsync(lm->samples.p + b.clips[(size_t)i].sample_base, h_samples[i],
                                   (size_t)b.clips[(size_t)i].samples * 4, hipMemcpyHostToDevice,
                                   s));
        x = lm->samples.p;
    } else {
        for (int32_t i = 0; i < B; ++i) b.clips[(size_t)i].sample_base = b.input_off[(size_t)i];
        HIP_TRY(launch_finite_check(d_samples, b.input_off.back(), lm->flag.p + 1, s));
    }
    HIP_TRY(lm->clips.ensure((size_t)B));
    HIP_TRY(hipMemcpyAsync(lm->clips.p, b.clips.data(), (size_t)B * sizeof(MelClip),
                           hipMemcpyHostToDevice, s));
    const MelTables t{lm->window.p, lm->twiddle.p, lm->start.p, lm->bin.p, lm->weight.p};
    HIP_TRY(launch_log_mel(x, lm->clips.p, B, b.total_frames, t, d_out, lm->flag.p, s));
    HIP_TRY(hipMemcpyAsync(lm->h_flag, lm->flag.p, 2 * sizeof(int), hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    if (lm->h_flag[1]) return fail(SVL_CORRUPT, "audio contains a non-finite sample");
    if (lm->h_flag[0])
        return fail(SVL_INTERNAL, "audio preprocessing produced a non-finite mel value");
    return SVL_OK;
}

}  // namespace svl

extern "C" {

svl_status svl_log_mel_layout(int64_t samples, int64_t *frames, int64_t *padded_samples,
                              int64_t *valid_frames) {
    int64_t f = 0, p = 0, v = 0;
    ST_TRY(layout(samples, &f, &p, &v));
    if (v == 0)
        return fail(SVL_CORRUPT, "audio has no complete analysis window and cannot be embedded");
    if (frames) *frames = f;
    if (padded_samples) *padded_samples = p;
    if (valid_frames) *valid_frames = v;
    return SVL_OK;
}

svl_status svl_log_mel_create(svl_ctx *ctx, svl_log_mel **out) {
    if (!ctx) return fail(SVL_USAGE, "context is required");
    return mel_create_on(ctx->device, out);
}

svl_status svl_log_mel_destroy(svl_log_mel *lm) {
    delete lm;
    return SVL_OK;
}

svl_status svl_log_mel_batch(svl_log_mel *lm, const float *const *samples,
                             const int64_t *lengths, int32_t clips, float *features,
                             uint8_t *mask) {
    if (!lm || (clips > 0 && (!samples || !features || !mask)))
        return fail(SVL_USAGE, "object, samples, features and mask are required");
    std::lock_guard<std::mutex> lock(lm->mu);
    MelBatch b;
    ST_TRY(mel_plan(lengths, clips, b));
    if (clips == 0) return SVL_OK;
    HIP_TRY(hipSetDevice(lm->device));
    HIP_TRY(lm->features.ensure((size_t)(b.total_frames * FEATURE_SIZE)));
    ST_TRY(mel_compute(lm, b, samples, nullptr, lengths, lm->features.p, lm->stream));
    HIP_TRY(hipMemcpy(features, lm->features.p, (size_t)(b.total_frames * FEATURE_SIZE) * 4,
                      hipMemcpyDeviceToHost));
    std::copy(b.mask.begin(), b.mask.end(), mask);
    return SVL_OK;
}

svl_status svl_log_mel_device(svl_log_mel *lm, const float *d_samples, const int64_t *lengths,
                              int32_t clips, float *d_features, uint8_t *mask, void *stream) {
    if (!lm || (clips > 0 && (!d_samples || !d_features || !mask)))
        return fail(SVL_USAGE, "object, samples, features and mask are required");
    std::lock_guard<std::mutex> lock(lm->mu);
    MelBatch b;
    ST_TRY(mel_plan(lengths, clips, b));
    if (clips == 0) return SVL_OK;
    hipStream_t s = stream ? (hipStream_t)stream : lm->stream;
    ST_TRY(mel_compute(lm, b, nullptr, d_samples, lengths, d_features, s));
    std::copy(b.mask.begin(), b.mask.end(), mask);
    return SVL_OK;
}

}  // extern "C"
