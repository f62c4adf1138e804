// Log-mel spectrogram of 16 kHz clips (src/media/audio_preprocess.rs:94-200):
// periodic Hann window over 320 samples, semicausal 160-sample left pad, a
// 512-point radix-2 FFT in double, magnitudes, 128 HTK mel filters, ln(e +
// 0.001) rounded to float once.
//
// One wave (= one workgroup) per frame. The windowed frame is written to LDS
// in bit-reversed order and the nine butterfly stages run in LDS, each lane
// owning four butterflies per stage. Every double operation is the
// reference's (same twiddles from the host, same operand order, no
// contraction into FMA), so the features are bit-identical to its f64
// pipeline. The mel projection sums only the non-zero filter weights, in
// bin order: every skipped term is an exact +0.0, so the sum is unchanged.
#include "dev_common.hpp"
#include "svl_internal.hpp"

namespace svl {

constexpr int MEL_FFT = 512;
constexpr int MEL_HALF_FRAME = 160;  // left pad and hop
constexpr int MEL_FRAME = 320;
constexpr int MEL_BINS_FFT = MEL_FFT / 2 + 1;
constexpr int MEL_FILTERS = 128;

__global__ __launch_bounds__(64) void log_mel_kernel(
    const float *__restrict__ x, const MelClip *__restrict__ clips, int n_clips,
    int64_t total_frames, const float *__restrict__ window, const double2 *__restrict__ twiddle,
    const int32_t *__restrict__ filt_start, const int32_t *__restrict__ filt_bin,
    const double *__restrict__ filt_weight, float *__restrict__ out, int *flag) {
#pragma clang fp contract(off)
    __shared__ double2 buf[MEL_FFT];
    __shared__ double mag[MEL_BINS_FFT];
    const int lane = threadIdx.x;
    const int64_t g = blockIdx.x;
    if (g >= total_frames) return;
    // the clip holding global frame g: last clip with frame_base <= g
    int lo = 0, hi = n_clips - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (clips[mid].frame_base <= g) lo = mid;
        else hi = mid - 1;
    }
    const MelClip c = clips[lo];
    const int64_t t = g - c.frame_base;
    const int64_t start = t * MEL_HALF_FRAME;
    float *row = out + g * MEL_FILTERS;
    if (start + MEL_HALF_FRAME >= (int64_t)c.samples) {  // incomplete window: zero row
        row[lane] = 0.0f;
        row[lane + 64] = 0.0f;
        return;
    }
    const float *src = x + c.sample_base;
    for (int i = lane; i < MEL_FFT; i += 64) {
        float v = 0.0f;
        if (i < MEL_FRAME) {
            const int64_t k = start + i - MEL_HALF_FRAME;
            if (k >= 0 && k < (int64_t)c.samples) v = src[k] * window[i];
        }
        buf[__builtin_bitreverse32((uint32_t)i) >> 23] = make_double2((double)v, 0.0);
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < 9; ++s) {
        const int half = 1 << s, step = MEL_FFT >> (s + 1);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int j = lane + 64 * q;
            const int off = j & (half - 1);
            const int e = ((j >> s) << (s + 1)) + off;
            const double2 tw = twiddle[off * step];
            const double2 ev = buf[e], od = buf[e + half];
            const double mr = od.x * tw.x - od.y * tw.y;
            const double mi = od.x * tw.y + od.y * tw.x;
            buf[e] = make_double2(ev.x + mr, ev.y + mi);
            buf[e + half] = make_double2(ev.x - mr, ev.y - mi);
        }
        __syncthreads();
    }
    for (int b = lane; b < MEL_BINS_FFT; b += 64) {
        const double2 v = buf[b];
        mag[b] = sqrt(v.x * v.x + v.y * v.y);
    }
    __syncthreads();
    bool ok = true;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int f = lane + 64 * h;
        double energy = 0.0;
        for (int k = filt_start[f]; k < filt_start[f + 1]; ++k)
            energy = energy + mag[filt_bin[k]] * filt_weight[k];
        const float y = (float)log(energy + 0.001);
        ok = ok && isfinite(y);
        row[f] = y;
    }
    if (!ok) raise_flag(flag, FLAG_NONFINITE);
}

hipError_t launch_log_mel(const float *x, const MelClip *clips, int n_clips, int64_t total_frames,
                          const MelTables &t, float *out, int *flag, hipStream_t s) {
    if (total_frames <= 0) return hipSuccess;
    if (n_clips <= 0 || total_frames > INT32_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL(log_mel_kernel, dim3((unsigned)total_frames), dim3(64), 0, s, x, clips,
                       n_clips, total_frames, t.window, (const double2 *)t.twiddle, t.filt_start,
                       t.filt_bin, t.filt_weight, out, flag);
    return hipGetLastError();
}

}  // namespace svl
