// Host side of the log-mel front end shared by mel.cpp (svl_log_mel_*) and
// audio.cpp (the audio embedder's sample entry points).
#pragma once

#include <hip/hip_runtime_api.h>

#include <mutex>
#include <vector>

#include "host_common.hpp"
#include "svl_internal.hpp"

struct svl_log_mel {
    int device = -1;
    hipStream_t stream = nullptr;
    svl::DevBuf<float> window;
    svl::DevBuf<double> twiddle, weight;
    svl::DevBuf<int32_t> start, bin;
    svl::DevBuf<float> samples, features;  // staging for host clips / host results
    svl::DevBuf<svl::MelClip> clips;
    svl::DevBuf<int> flag;  // [0] non-finite feature, [1] non-finite input sample
    int *h_flag = nullptr;
    std::mutex mu;
    ~svl_log_mel();
};

namespace svl {

// Frame layout of a batch of clips, validated clip by clip in the order
// log_mel meets each condition (audio_preprocess.rs:94-131, 186-190).
struct MelBatch {
    std::vector<MelClip> clips;     // sample_base filled by mel_compute
    std::vector<uint8_t> mask;      // [total_frames]
    std::vector<int64_t> frame_off;  // [B + 1]
    std::vector<int64_t> input_off;  // [B + 1] over the callers' full lengths
    int64_t total_frames = 0;
};

svl_status mel_plan(const int64_t *lengths, int32_t clips, MelBatch &b);
// Features of the planned batch into d_out ([total_frames, 128]) on stream s,
// from host clips (h_samples) or from the packed device buffer d_samples.
// Returns after the stream drained, with input / output finiteness checked.
svl_status mel_compute(svl_log_mel *lm, MelBatch &b, const float *const *h_samples,
                       const float *d_samples, const int64_t *lengths, float *d_out,
                       hipStream_t s);
svl_status mel_create_on(int device, svl_log_mel **out);

}  // namespace svl
