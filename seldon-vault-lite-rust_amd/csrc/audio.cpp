// Host runtime of the audio tower and the audio prompt glue: the
// svl_audio_* part of include/svl_hip.h.
//
// It plays the role of the reference's AudioModel (src/model/audio.rs:
// 932-1134) and AudioEmbedder::embed_impl (src/model/audio_embedder.rs:
// 223-267). Weights are validated like AudioWeights::decode (audio.rs:
// 717-794, including the inverted-bounds check of :850-870) and packed once:
// fused Q/K/V, interleaved light-conv start projection, and each layer's
// relative keys (the sinusoidal table
// times relative_k_proj, input-independent) computed on the GPU at load.
// A forward call packs every clip's mel frames back to back and runs the
// tower as one launch sequence; the subsampled rows of all clips are
// processed (padding rows included, as the reference's light convolution
// reads them) and only valid tokens are projected and returned.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/svl_hip.h"
#include "host_common.hpp"
#include "mel_host.hpp"
#include "svl_internal.hpp"

namespace {

using namespace svl;

// audio.rs:30-60; media/audio_preprocess.rs:34.
constexpr int64_t MAX_AUDIO_HIDDEN = 16384;
constexpr int64_t MAX_AUDIO_INTERMEDIATE = 65536;
constexpr int64_t MAX_AUDIO_LAYERS = 128;
constexpr int64_t MAX_AUDIO_HEADS = 128;
constexpr int64_t MAX_AUDIO_HEAD_DIM = 1024;
constexpr int64_t MAX_AUDIO_CONV_CHANNELS = 4096;
constexpr int64_t MAX_AUDIO_OUTPUT_DIMS = 16384;
constexpr int64_t MAX_AUDIO_CONTEXT = 4096;
constexpr int64_t MAX_AUDIO_WEIGHT_ELEMENTS = int64_t(1) << 30;
constexpr int64_t FEATURE_SIZE = 128;
constexpr int64_t FREQ0 = 64, FREQ1 = 32;
constexpr int64_t MAX_TEXT_TOKENS = 8192;
// std::f64::consts::LN_2 and E
constexpr double LN_2 = 0.693147180559945309417232121458176568;
constexpr double EULER = 2.71828182845904523536028747135266250;

struct Bounds {
    float v[4];  // input min, input max, output min, output max
};

struct AuLayer {
    float *ff_pre[2] = {}, *ff_post[2] = {}, *ff_w1[2] = {}, *ff_w2[2] = {};
    Bounds ff_b1[2] = {}, ff_b2[2] = {};
    float *w_qkv = nullptr, *w_post = nullptr;
    Bounds bq = {}, bk = {}, bv = {}, bpost = {};
    float *relk = nullptr, *qf = nullptr;
    float *lc_pre = nullptr, *w_start = nullptr, *w_end = nullptr, *dw = nullptr,
          *lc_norm = nullptr;
    Bounds bstart = {}, bend = {};
    float *norm_pre_attn = nullptr, *norm_post_attn = nullptr, *norm_out = nullptr;
};

// Typed view into the model's metadata block (set by upload_au_meta).
template <typename T>
struct AuView {
    T *p = nullptr;
};

}  // namespace

struct svl_audio_model {
    int device = 0;
    int64_t H = 0, I = 0, L = 0, NH = 0, hd = 0, K = 0, C0 = 0, C1 = 0, chunk = 0, left = 0,
            right = 0, P = 0, text_hidden = 0, context = 0, positions = 0, H_pad = 0;
    float cap = 0.f, eps = 0.f, rw = 0.f, clip = 0.f, k_scale = 0.f;
    std::vector<float *> allocations;
    float *w_conv0 = nullptr, *ln0 = nullptr, *w_conv1 = nullptr, *ln1 = nullptr,
          *w_in = nullptr, *w_out = nullptr, *b_out = nullptr, *w_emb = nullptr;
    std::vector<AuLayer> layers;
    // workspace
    DevBuf<float> mel, l0, l1, h, n, tmp, act, qkv, att, gated, proj, projn, soft;
    DevBuf<int32_t> pos, rowlen;
    // A pass's metadata in one device block, filled by one copy from pinned
    // host memory: the error flag, the frame mask, the subsampling masks and
    // rows, the valid-token index, the attention blocks and the row offsets
    // (the views below). Every pass of a call has its own staging region.
    DevBuf<unsigned char> meta;
    unsigned char *h_meta = nullptr;  // pinned staging
    size_t h_meta_n = 0;
    hipEvent_t ev_meta = nullptr;     // after the last copy out of h_meta
    AuView<int> flag;
    AuView<uint8_t> mask, mask0, mask1;
    AuView<SscpRow> rows0, rows1;
    AuView<int32_t> valid_idx, att_blocks;
    AuView<int64_t> offsets;
    int *h_flag = nullptr;
    hipStream_t stream = nullptr;
    svl_log_mel *lm = nullptr;  // log-mel tables, created by the first sample call
    std::mutex mu;

    ~svl_audio_model() {
        delete lm;
        if (device >= 0) (void)hipSetDevice(device);
        for (float *p : allocations) (void)hipFree(p);
        mel.release(); l0.release(); l1.release(); h.release(); n.release(); tmp.release();
        act.release(); qkv.release(); att.release(); gated.release(); proj.release();
        projn.release(); soft.release(); pos.release(); rowlen.release(); meta.release();
        if (ev_meta) {
            (void)hipEventSynchronize(ev_meta);
            (void)hipEventDestroy(ev_meta);
        }
        if (h_meta) (void)hipHostFree(h_meta);
        if (h_flag) (void)hipHostFree(h_flag);
        if (stream) (void)hipStreamDestroy(stream);
    }
};

namespace {

// AudioConfig invariants (audio.rs:129-278) on an already parsed config.
svl_status validate_audio_config(const svl_audio_config *c, int64_t text_hidden) {
    if (!c) return fail(SVL_USAGE, "audio configuration is null");
    const int64_t H = c->hidden_size, NH = c->num_attention_heads;
    if (H % 2) return fail(SVL_CORRUPT, "audio hidden size must be even for sinusoidal relative positions");
    if (NH <= 0 || H <= 0 || H % NH)
        return fail(SVL_CORRUPT, "audio hidden size must be divisible by a positive head count");
    const int64_t hd = H / NH;
    if (hd == 0 || hd > MAX_AUDIO_HEAD_DIM)
        return fail(SVL_LIMIT, "audio head dimension %lld is outside 1..=%lld", (long long)hd,
                    (long long)MAX_AUDIO_HEAD_DIM);
    if (H > MAX_AUDIO_HIDDEN || 4 * H > MAX_AUDIO_INTERMEDIATE ||
        c->num_hidden_layers < 0 || c->num_hidden_layers > MAX_AUDIO_LAYERS ||
        NH > MAX_AUDIO_HEADS || c->output_proj_dims <= 0 ||
        c->output_proj_dims > MAX_AUDIO_OUTPUT_DIMS)
        return fail(SVL_LIMIT, "audio dimensions exceed their documented caps");
    if (c->conv_kernel_size <= 0 || c->conv_kernel_size > 31)
        return fail(SVL_LIMIT, "audio convolution kernel %lld is outside 1..=31",
                    (long long)c->conv_kernel_size);
    if (c->attention_chunk_size <= 0 || c->attention_context_left < 2)
        return fail(SVL_CORRUPT, "audio chunked attention requires a positive chunk and at least "
                                 "two context positions on the left");
    if (c->attention_context_right < 0)
        return fail(SVL_CORRUPT, "audio right context must be non-negative");
    const int64_t context =
        c->attention_chunk_size + c->attention_context_left - 1 + c->attention_context_right;
    if (context <= 0 || context > MAX_AUDIO_CONTEXT)
        return fail(SVL_LIMIT, "audio attention context %lld is outside 1..=%lld",
                    (long long)context, (long long)MAX_AUDIO_CONTEXT);
    if (!std::isfinite((float)c->rms_norm_eps) || (float)c->rms_norm_eps < 0.f)
        return fail(SVL_CORRUPT, "audio RMSNorm epsilon must be finite and non-negative");
    if (!std::isfinite((float)c->attention_logit_cap) || (float)c->attention_logit_cap <= 0.f)
        return fail(SVL_CORRUPT, "audio attention logit cap must be finite and positive");
    if (!std::isfinite((float)c->residual_weight))
        return fail(SVL_CORRUPT, "audio residual weight must be finite");
    if (!std::isfinite((float)c->gradient_clipping) || (float)c->gradient_clipping <= 0.f)
        return fail(SVL_CORRUPT, "audio gradient clipping must be finite and positive");
    const int64_t c0 = c->conv_channels0, c1 = c->conv_channels1;
    if (c0 <= 0 || c1 <= 0 || c0 > MAX_AUDIO_CONV_CHANNELS || c1 > MAX_AUDIO_CONV_CHANNELS ||
        c0 % 4)
        return fail(SVL_LIMIT, "audio subsampling channels exceed their documented caps or are "
                               "not divisible by four");
    if (text_hidden <= 0 || text_hidden > MAX_AUDIO_HIDDEN)
        return fail(SVL_LIMIT, "text hidden size %lld is out of range", (long long)text_hidden);
    return SVL_OK;
}

const char *kBoundNames[4] = {"input_min", "input_max", "output_min", "output_max"};

// AudioConfig::tensor_shapes (audio.rs:394-498).
ShapeList audio_tensor_shapes(const svl_audio_config *c, int64_t text_hidden) {
    const int64_t H = c->hidden_size, I = 4 * H, hd = H / c->num_attention_heads;
    const int64_t c0 = c->conv_channels0, c1 = c->conv_channels1;
    ShapeList s;
    const std::string sp = "audio_tower.subsample_conv_projection.";
    s.push_back({sp + "layer0.conv.weight", {c0, 1, 3, 3}});
    s.push_back({sp + "layer0.norm.weight", {c0}});
    s.push_back({sp + "layer1.conv.weight", {c1, c0, 3, 3}});
    s.push_back({sp + "layer1.norm.weight", {c1}});
    s.push_back({sp + "input_proj_linear.weight", {H, (c0 / 4) * c1}});
    for (int64_t l = 0; l < c->num_hidden_layers; ++l) {
        const std::string p = "audio_tower.layers." + std::to_string(l) + ".";
        for (const char *ff : {"feed_forward1", "feed_forward2"}) {
            const std::string b = p + ff + ".";
            s.push_back({b + "pre_layer_norm.weight", {H}});
            s.push_back({b + "post_layer_norm.weight", {H}});
            s.push_back({b + "ffw_layer_1.linear.weight", {I, H}});
            s.push_back({b + "ffw_layer_2.linear.weight", {H, I}});
            for (const char *lin : {"ffw_layer_1", "ffw_layer_2"})
                for (const char *bn : kBoundNames) s.push_back({b + lin + "." + bn, {}});
        }
        for (const char *proj : {"q_proj", "k_proj", "v_proj", "post"}) {
            s.push_back({p + "self_attn." + proj + ".linear.weight", {H, H}});
            for (const char *bn : kBoundNames) s.push_back({p + "self_attn." + proj + "." + bn, {}});
        }
        s.push_back({p + "self_attn.relative_k_proj.weight", {H, H}});
        s.push_back({p + "self_attn.per_dim_scale", {hd}});
        s.push_back({p + "lconv1d.pre_layer_norm.weight", {H}});
        s.push_back({p + "lconv1d.linear_start.linear.weight", {2 * H, H}});
        s.push_back({p + "lconv1d.linear_end.linear.weight", {H, H}});
        for (const char *lin : {"linear_start", "linear_end"})
            for (const char *bn : kBoundNames) s.push_back({p + "lconv1d." + lin + "." + bn, {}});
        s.push_back({p + "lconv1d.depthwise_conv1d.weight", {H, 1, c->conv_kernel_size}});
        s.push_back({p + "lconv1d.conv_norm.weight", {H}});
        s.push_back({p + "norm_pre_attn.weight", {H}});
        s.push_back({p + "norm_post_attn.weight", {H}});
        s.push_back({p + "norm_out.weight", {H}});
    }
    s.push_back({"audio_tower.output_proj.weight", {c->output_proj_dims, H}});
    s.push_back({"audio_tower.output_proj.bias", {c->output_proj_dims}});
    s.push_back({"embed_audio.embedding_projection.weight", {text_hidden, c->output_proj_dims}});
    return s;
}

// build_clipped_linear (audio.rs:850-870): four scalars, not inverted.
svl_status read_bounds(const TensorIndex &by_name, const std::string &prefix, Bounds &b) {
    std::vector<float> a;
    for (int k = 0; k < 4; ++k) {
        ST_TRY(decode_named(by_name, prefix + "." + kBoundNames[k], a));
        if (a.size() != 1) return fail(SVL_INTERNAL, "%s.%s is not a scalar", prefix.c_str(), kBoundNames[k]);
        b.v[k] = a[0];
    }
    if (b.v[0] > b.v[1] || b.v[2] > b.v[3])
        return fail(SVL_CORRUPT, "audio clipping bounds for %s are inverted", prefix.c_str());
    return SVL_OK;
}

// audio.rs:1366-1372.
float softplus_host(float v) { return v > 20.0f ? v : std::log(1.0f + std::exp(v)); }

// AudioModel::position_embeddings (audio.rs:1257-1288).
std::vector<float> position_table(int64_t hidden, int64_t positions) {
    const int64_t ts = hidden / 2;
    const double increment = ts > 1 ? std::log(10000.0) / (double)(ts - 1) : 0.0;
    std::vector<float> inv((size_t)ts), out((size_t)(positions * hidden));
    for (int64_t i = 0; i < ts; ++i) inv[(size_t)i] = (float)std::exp(-(double)i * increment);
    for (int64_t p = 0; p < positions; ++p) {
        const float id = (float)(positions - 1 - p);
        for (int64_t i = 0; i < ts; ++i) {
            const float scaled = id * inv[(size_t)i];
            out[(size_t)(p * hidden + i)] = std::sin(scaled);
            out[(size_t)(p * hidden + ts + i)] = std::cos(scaled);
        }
    }
    return out;
}

// A clipped linear (audio.rs:558-601). Its A operand is written already
// clamped to b's input bounds by the kernel that produces it (in_clamp).
GemmArgs clipped(const float *A, int64_t lda, const float *W, int64_t ldw, float *C, int64_t ldc,
                 int64_t M, int64_t N, int64_t K, int epi, const Bounds &b) {
    GemmArgs g{A, lda, W, ldw, C, ldc, (int)M, (int)N, (int)K, epi, 1.f, nullptr, 0, 0};
    for (int k = 0; k < 4; ++k) g.clip[0][k] = b.v[k];
    return g;
}

// Store clamp that makes a row kernel's output the A operand of the clipped
// linears with input bounds b[0 .. n-1] (one copy each, `stride` floats apart).
OutClamp in_clamp(const Bounds *const *b, int n, int64_t stride) {
    OutClamp oc;
    oc.copies = n;
    oc.stride = stride;
    for (int k = 0; k < n; ++k) {
        oc.lo[k] = b[k]->v[0];
        oc.hi[k] = b[k]->v[1];
    }
    return oc;
}

OutClamp in_clamp(const Bounds &b) {
    const Bounds *p = &b;
    return in_clamp(&p, 1, 0);
}

// The FFN up projection's SiLU output is the down projection's A operand.
GemmArgs ffn_up(const float *A, int64_t lda, const float *W, float *C, int64_t M, int64_t N,
                int64_t K, const Bounds &up, const Bounds &down) {
    GemmArgs g = clipped(A, lda, W, K, C, N, M, N, K, EPI_CLIP_SILU, up);
    g.post_lo = down.v[0];
    g.post_hi = down.v[1];
    return g;
}

// Per-call geometry of a batch of clips.
struct AuBatch {
    int32_t B = 0;
    int64_t F = 0, T0 = 0, T = 0, tokens = 0;  // frames, layer-0 rows, layer-1 rows, tokens
    std::vector<int64_t> frame_off, row_off;   // [B + 1]
    std::vector<int64_t> tokens_per_clip;
    std::vector<SscpRow> rows0, rows1;
    std::vector<uint8_t> mask0, mask1;
    std::vector<int32_t> valid_idx;
    std::vector<int32_t> att_blocks;  // first row of each attention block
};

// Validation in the order AudioModel::forward meets each condition
// (audio.rs:981-1010, subsample :1136-1166) and the batch layout.
svl_status prepare_clips(const svl_audio_model *m, const svl_mel *mels, int32_t batch,
                         bool need_features, AuBatch &b) {
    if (batch < 0) return fail(SVL_USAGE, "negative batch");
    if (batch > 0 && !mels) return fail(SVL_USAGE, "mel spectrograms are null");
    b.B = batch;
    b.frame_off.assign(1, 0);
    b.row_off.assign(1, 0);
    int64_t row0_off = 0;
    for (int i = 0; i < batch; ++i) {
        const svl_mel &mel = mels[i];
        const int64_t F = mel.frames;
        if (F < 0) return fail(SVL_USAGE, "clip %d: negative frame count", i);
        if (F > 0 && (!mel.mask || (need_features && !mel.features)))
            return fail(SVL_USAGE, "clip %d: mel features or mask are null", i);
        const int64_t f1 = (F + 1) / 2, f2 = (f1 + 1) / 2;
        if (f2 == 0) return fail(SVL_CORRUPT, "clip %d: audio subsampling produced no frames", i);
        if (f1 * FREQ0 * m->C0 > MAX_ACTIVATION_ELEMENTS || f2 * FREQ1 * m->C1 > MAX_ACTIVATION_ELEMENTS)
            return fail(SVL_LIMIT, "clip %d: audio subsampling would allocate more than the "
                                   "%lld-element cap", i, (long long)MAX_ACTIVATION_ELEMENTS);
        // The input projection takes (C0 / 4) * C1 features per row and layer 1
        // yields 32 * C1 (audio.rs:1244-1248): only C0 = 128 can run.
        if ((m->C0 / 4) * m->C1 != FREQ1 * m->C1)
            return fail(SVL_INTERNAL,
                        "audio subsampling output does not match the projection input width");
        for (int64_t t = 0; t < f1; ++t) {
            b.rows0.push_back({(int32_t)b.frame_off.back(), (int32_t)t, (int32_t)F});
            b.mask0.push_back(2 * t < F ? (uint8_t)(mel.mask[2 * t] != 0) : (uint8_t)0);
        }
        for (int64_t t = 0; t < f2; t += m->chunk) b.att_blocks.push_back((int32_t)(b.row_off.back() + t));
        int64_t tok = 0;
        for (int64_t t = 0; t < f2; ++t) {
            b.rows1.push_back({(int32_t)row0_off, (int32_t)t, (int32_t)f1});
            const uint8_t v = 2 * t < f1 ? b.mask0[(size_t)(row0_off + 2 * t)] : (uint8_t)0;
            b.mask1.push_back(v);
            if (v) {
                b.valid_idx.push_back((int32_t)(b.row_off.back() + t));
                ++tok;
            }
        }
        if (tok == 0)
            return fail(SVL_CORRUPT, "clip %d: audio tower received no valid subsampled token", i);
        const int64_t widest = std::max({m->I, 2 * m->H, m->P, m->text_hidden});
        if (f2 * widest > MAX_ACTIVATION_ELEMENTS)
            return fail(SVL_LIMIT, "clip %d: audio linear output would allocate %lld elements", i,
                        (long long)(f2 * widest));
        b.tokens_per_clip.push_back(tok);
        row0_off += f1;
        b.frame_off.push_back(b.frame_off.back() + F);
        b.row_off.push_back(b.row_off.back() + f2);
    }
    b.F = b.frame_off.back();
    b.T0 = row0_off;
    b.T = b.row_off.back();
    b.tokens = (int64_t)b.valid_idx.size();
    return SVL_OK;
}

// One pass of the tower keeps its layer-0 activations below 2 GiB: the
// implicit-im2col convolution reads them through one 32-bit buffer window,
// and the packed frame and row offsets are 32-bit. One clip always fits
// (its layer-0 output is at most MAX_ACTIVATION_ELEMENTS floats).
bool au_pass_fits(const svl_audio_model *m, int64_t t0) {
    return t0 * FREQ0 * m->C0 * 4 < 0x7FFFFFF0;
}

size_t au_meta_layout(const AuBatch &b, size_t off[9]);

svl_status ensure_au_workspace(svl_audio_model *m, const AuBatch &b) {
    const int64_t F = std::max<int64_t>(b.F, 1), T0 = std::max<int64_t>(b.T0, 1),
                  T = std::max<int64_t>(b.T, 1), N = std::max<int64_t>(b.tokens, 1);
    HIP_TRY(m->mel.ensure(F * FEATURE_SIZE));
    HIP_TRY(m->l0.ensure(T0 * FREQ0 * m->C0));
    HIP_TRY(m->l1.ensure(T * FREQ1 * m->C1));
    HIP_TRY(m->h.ensure(T * m->H));
    HIP_TRY(m->n.ensure(3 * T * m->H));  // three clamped copies feed the Q/K/V projection
    HIP_TRY(m->tmp.ensure(T * m->H));
    HIP_TRY(m->act.ensure(T * m->I));
    HIP_TRY(m->qkv.ensure(T * 3 * m->H));
    HIP_TRY(m->att.ensure(T * m->H));
    HIP_TRY(m->gated.ensure(T * m->H));
    HIP_TRY(m->proj.ensure(T * m->P));
    HIP_TRY(m->projn.ensure(N * m->P));
    HIP_TRY(m->soft.ensure(N * m->text_hidden));
    HIP_TRY(m->pos.ensure(T));
    HIP_TRY(m->rowlen.ensure(T));
    size_t off[9];
    HIP_TRY(m->meta.ensure(au_meta_layout(b, off)));
    return SVL_OK;
}

// Byte offsets in a pass's metadata block (each array 256-byte aligned):
// flag, frame mask, mask0, mask1, rows0, rows1, valid_idx, att_blocks,
// offsets; returns the block's size.
size_t au_meta_layout(const AuBatch &b, size_t off[9]) {
    auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
    const size_t bytes[9] = {sizeof(int), (size_t)b.F, b.mask0.size(), b.mask1.size(),
                             b.rows0.size() * sizeof(SscpRow), b.rows1.size() * sizeof(SscpRow),
                             b.valid_idx.size() * 4, b.att_blocks.size() * 4,
                             b.row_off.size() * 8};
    size_t at = 0;
    for (int i = 0; i < 9; ++i) {
        off[i] = at;
        at += up(std::max<size_t>(bytes[i], 1));
    }
    return at;
}

// Pinned staging for the passes of one call, `bytes` in all; waits for the
// copies of the call before out of it.
svl_status au_staging(svl_audio_model *m, size_t bytes) {
    if (m->ev_meta) HIP_TRY(hipEventSynchronize(m->ev_meta));
    else HIP_TRY(hipEventCreateWithFlags(&m->ev_meta, hipEventDisableTiming));
    if (m->h_meta_n >= bytes) return SVL_OK;
    if (m->h_meta) HIP_TRY(hipHostFree(m->h_meta));
    m->h_meta = nullptr;
    m->h_meta_n = 0;
    HIP_TRY(hipHostMalloc((void **)&m->h_meta, bytes, hipHostMallocDefault));
    m->h_meta_n = bytes;
    return SVL_OK;
}

// One pass's metadata (the frame masks of its clips `mels`, the batch
// layout, the flag cleared on the first pass only, so a later pass keeps an
// earlier one's error) through its staging region at `stage` by one copy.
svl_status upload_au_meta(svl_audio_model *m, const AuBatch &b, const svl_mel *mels, hipStream_t s,
                          bool reset_flag, size_t stage) {
    size_t off[9];
    const size_t total = au_meta_layout(b, off);
    unsigned char *h = m->h_meta + stage, *d = m->meta.p;
    std::memset(h, 0, total);
    for (int32_t i = 0; i < b.B; ++i)
        if (mels[i].frames > 0)
            std::memcpy(h + off[1] + b.frame_off[(size_t)i], mels[i].mask, (size_t)mels[i].frames);
    std::memcpy(h + off[2], b.mask0.data(), b.mask0.size());
    std::memcpy(h + off[3], b.mask1.data(), b.mask1.size());
    std::memcpy(h + off[4], b.rows0.data(), b.rows0.size() * sizeof(SscpRow));
    std::memcpy(h + off[5], b.rows1.data(), b.rows1.size() * sizeof(SscpRow));
    std::memcpy(h + off[6], b.valid_idx.data(), b.valid_idx.size() * 4);
    std::memcpy(h + off[7], b.att_blocks.data(), b.att_blocks.size() * 4);
    std::memcpy(h + off[8], b.row_off.data(), b.row_off.size() * 8);
    m->flag.p = (int *)d;
    m->mask.p = d + off[1];
    m->mask0.p = d + off[2];
    m->mask1.p = d + off[3];
    m->rows0.p = (SscpRow *)(d + off[4]);
    m->rows1.p = (SscpRow *)(d + off[5]);
    m->valid_idx.p = (int32_t *)(d + off[6]);
    m->att_blocks.p = (int32_t *)(d + off[7]);
    m->offsets.p = (int64_t *)(d + off[8]);
    const size_t from = reset_flag ? 0 : off[1];
    HIP_TRY(hipMemcpyAsync(d + from, h + from, total - from, hipMemcpyHostToDevice, s));
    HIP_TRY(hipEventRecord(m->ev_meta, s));
    return SVL_OK;
}

// Valid rows of a captured [T, H] host copy, clip by clip (select_valid,
// audio.rs:1671-1685).
void select_valid(const AuBatch &b, int64_t H, const float *all, float *out) {
    for (size_t j = 0; j < b.valid_idx.size(); ++j)
        std::copy(all + (int64_t)b.valid_idx[j] * H, all + ((int64_t)b.valid_idx[j] + 1) * H,
                  out + j * H);
}

// The tower over the packed mel frames in d_mel (audio.rs:981-1133); soft
// tokens of the valid rows land in d_soft. Captures (all rows, [T, H]; the
// caller selects the valid ones after the stream drains): h_sscp after the
// subsampling, h_hidden [L, T, H] after every layer.
svl_status enqueue_audio(svl_audio_model *m, const AuBatch &b, const float *d_mel, hipStream_t s,
                         float *d_soft, float *h_sscp, float *h_hidden) {
    const int64_t T = b.T, H = m->H, I = m->I;
    const int W = (int)H;
    int *flag = m->flag.p;
    const float inf = INFINITY;
    HIP_TRY(launch_positions(m->offsets.p, b.B, m->pos.p, m->rowlen.p, s));
    // Subsampling (audio.rs:1136-1255).
    HIP_TRY(launch_sscp_conv0(d_mel, m->mask.p, m->rows0.p, b.T0, m->w_conv0, m->ln0, (int)m->C0,
                              m->eps, m->l0.p, flag, s));
    // layer 1: the 3x3 stride-2 convolution as an implicit-im2col GEMM against
    // the tap-major [C1, 9 C0] weight, then LayerNorm + ReLU. C0 is 128 in
    // every configuration that reaches this point (prepare_clips), and a pass
    // keeps the layer-0 output inside the kernel's buffer window
    // (au_pass_fits), so gemm_conv_ok holds.
    {
        const int64_t K = 9 * m->C0;
        GemmArgs g{m->l0.p, K, m->w_conv1, K, m->l1.p, m->C1, (int)(T * FREQ1), (int)m->C1,
                   (int)K, EPI_STORE, 1.f, nullptr, 0, 0};
        g.conv_rows = reinterpret_cast<const int32_t *>(m->rows1.p);
        g.conv_mask = m->mask0.p;
        g.conv_c0 = (int)m->C0;
        g.conv_f0 = (int)FREQ0;
        g.conv_f1 = (int)FREQ1;
        g.conv_a_floats = b.T0 * FREQ0 * m->C0;
        if (!gemm_conv_ok(g)) return fail(SVL_INTERNAL, "audio subsampling launch out of bounds");
        HIP_TRY(launch_gemm_conv(g, s));
    }
    HIP_TRY(launch_sscp_ln_relu(m->l1.p, m->ln1, (int)m->C1, T * FREQ1, m->eps, flag, s));
    {
        const int64_t K = FREQ1 * m->C1;
        GemmArgs g{m->l1.p, K, m->w_in, K, m->h.p, H, (int)T, (int)H, (int)K, EPI_STORE, 1.f,
                   nullptr, 0, 0};
        HIP_TRY(launch_gemm(g, s));
    }
    if (h_sscp)
        HIP_TRY(hipMemcpyAsync(h_sscp, m->h.p, (size_t)(T * H) * 4, hipMemcpyDeviceToHost, s));
    if (m->L > 0)  // feed_forward1's input clamp + pre norm of layer 0
        HIP_TRY(launch_audio_rows(m->h.p, m->clip, m->layers[0].ff_pre[0], nullptr, 1.f, m->n.p,
                                  inf, nullptr, nullptr, T, W, m->eps, flag, s,
                                  in_clamp(m->layers[0].ff_b1[0])));
    for (int64_t l = 0; l < m->L; ++l) {
        const AuLayer &ly = m->layers[(size_t)l];
        // feed_forward1 (audio.rs:1374-1433): n holds rms(clamp(h), pre).
        HIP_TRY(launch_gemm(ffn_up(m->n.p, H, ly.ff_w1[0], m->act.p, T, I, H, ly.ff_b1[0],
                                   ly.ff_b2[0]), s));
        HIP_TRY(launch_gemm(clipped(m->act.p, I, ly.ff_w2[0], I, m->tmp.p, H, T, H, I,
                                    EPI_CLIP_STORE, ly.ff_b2[0]), s));
        // h += rms(clamp(ff), post) * rw; n = rms(h, norm_pre_attn), one copy
        // per projection of Q, K and V, each clamped to its input bounds
        const Bounds *bs[3] = {&ly.bq, &ly.bk, &ly.bv};
        HIP_TRY(launch_audio_rows(m->tmp.p, m->clip, ly.ff_post[0], m->h.p, m->rw, m->h.p, inf,
                                  ly.norm_pre_attn, m->n.p, T, W, m->eps, flag, s,
                                  in_clamp(bs, 3, T * H)));
        // chunked attention (audio.rs:1529-1669)
        if (H % 128 == 0) {
            GemmArgs g = clipped(m->n.p, H, ly.w_qkv, H, m->qkv.p, 3 * H, T, 3 * H, H,
                                 EPI_CLIP_STORE, ly.bq);
            g.clip_cols = (int)H;
            g.a_seg = T * H;
            for (int k = 0; k < 4; ++k) {
                g.clip[1][k] = ly.bk.v[k];
                g.clip[2][k] = ly.bv.v[k];
            }
            HIP_TRY(launch_gemm(g, s));
        } else {
            for (int j = 0; j < 3; ++j)
                HIP_TRY(launch_gemm(clipped(m->n.p + (int64_t)j * T * H, H,
                                            ly.w_qkv + (int64_t)j * H * H, H,
                                            m->qkv.p + (int64_t)j * H, 3 * H, T, H, H,
                                            EPI_CLIP_STORE, *bs[j]), s));
        }
        {
            AudioAttnArgs a{};
            a.q = m->qkv.p;
            a.k = m->qkv.p + H;
            a.v = m->qkv.p + 2 * H;
            a.ldq = a.ldk = a.ldv = 3 * H;
            a.relk = ly.relk;
            a.qf = ly.qf;
            a.k_scale = m->k_scale;
            a.cap = m->cap;
            a.mask = m->mask1.p;
            a.pos = m->pos.p;
            a.rowlen = m->rowlen.p;
            a.out = m->att.p;
            a.ldo = H;
            a.blocks = m->att_blocks.p;
            a.n_blocks = (int64_t)b.att_blocks.size();
            a.heads = (int)m->NH;
            a.head_dim = (int)m->hd;
            a.chunk = (int)m->chunk;
            a.left = (int)m->left;
            a.context = (int)m->context;
            a.positions = (int)m->positions;
            a.flag = flag;
            a.out_lo = ly.bpost.v[0];
            a.out_hi = ly.bpost.v[1];
            HIP_TRY(launch_audio_attention(a, s));
        }
        HIP_TRY(launch_gemm(clipped(m->att.p, H, ly.w_post, H, m->tmp.p, H, T, H, H, EPI_CLIP_STORE,
                                    ly.bpost), s));
        // h += rms(post, norm_post_attn); n = rms(h, lconv pre)
        HIP_TRY(launch_audio_rows(m->tmp.p, inf, ly.norm_post_attn, m->h.p, 1.f, m->h.p, inf,
                                  ly.lc_pre, m->n.p, T, W, m->eps, flag, s, in_clamp(ly.bstart)));
        // light conv (audio.rs:1448-1527)
        {
            GemmArgs g = clipped(m->n.p, H, ly.w_start, H, m->gated.p, H, T, 2 * m->H_pad, H,
                                 EPI_CLIP_GLU, ly.bstart);
            g.n_out = (int)H;
            HIP_TRY(launch_gemm(g, s));
        }
        HIP_TRY(launch_lconv(m->gated.p, ly.dw, (int)m->K, m->pos.p, m->clip, ly.lc_norm, m->n.p,
                             T, W, m->eps, flag, s, ly.bend.v[0], ly.bend.v[1]));
        HIP_TRY(launch_gemm(clipped(m->n.p, H, ly.w_end, H, m->tmp.p, H, T, H, H, EPI_CLIP_STORE,
                                    ly.bend), s));
        // h += end; n = rms(clamp(h), feed_forward2 pre)
        HIP_TRY(launch_audio_rows(m->tmp.p, inf, nullptr, m->h.p, 1.f, m->h.p, m->clip,
                                  ly.ff_pre[1], m->n.p, T, W, m->eps, flag, s, in_clamp(ly.ff_b1[1])));
        // feed_forward2
        HIP_TRY(launch_gemm(ffn_up(m->n.p, H, ly.ff_w1[1], m->act.p, T, I, H, ly.ff_b1[1],
                                   ly.ff_b2[1]), s));
        HIP_TRY(launch_gemm(clipped(m->act.p, I, ly.ff_w2[1], I, m->tmp.p, H, T, H, I,
                                    EPI_CLIP_STORE, ly.ff_b2[1]), s));
        // h = rms(h + rms(clamp(ff), post) * rw, norm_out)
        HIP_TRY(launch_audio_rows(m->tmp.p, m->clip, ly.ff_post[1], m->h.p, m->rw, nullptr, inf,
                                  ly.norm_out, m->h.p, T, W, m->eps, flag, s));
        if (h_hidden)
            HIP_TRY(hipMemcpyAsync(h_hidden + (size_t)(l * T * H), m->h.p, (size_t)(T * H) * 4,
                                   hipMemcpyDeviceToHost, s));
        if (l + 1 < m->L)
            HIP_TRY(launch_audio_rows(m->h.p, m->clip, m->layers[(size_t)l + 1].ff_pre[0], nullptr,
                                      1.f, m->n.p, inf, nullptr, nullptr, T, W, m->eps, flag, s,
                                      in_clamp(m->layers[(size_t)l + 1].ff_b1[0])));
    }
    // Output projection + bias, unscaled RMSNorm of the valid rows, text
    // projection (audio.rs:1085-1133).
    {
        GemmArgs g{m->h.p, H, m->w_out, H, m->proj.p, m->P, (int)T, (int)m->P, (int)H, EPI_BIAS,
                   1.f, m->b_out, 0, 0};
        HIP_TRY(launch_gemm(g, s));
    }
    HIP_TRY(launch_finite_check(m->proj.p, T * m->P, flag, s));
    HIP_TRY(launch_compact_rms(m->proj.p, m->valid_idx.p, m->projn.p, b.tokens, (int)m->P, m->eps,
                               flag, s));
    {
        GemmArgs g{m->projn.p, m->P, m->w_emb, m->P, d_soft, m->text_hidden, (int)b.tokens,
                   (int)m->text_hidden, (int)m->P, EPI_STORE, 1.f, nullptr, 0, 0};
        HIP_TRY(launch_gemm(g, s));
    }
    HIP_TRY(launch_finite_check(d_soft, b.tokens * m->text_hidden, flag, s));
    return SVL_OK;
}

svl_status au_finish(svl_audio_model *m, hipStream_t s) {
    HIP_TRY(hipMemcpyAsync(m->h_flag, m->flag.p, sizeof(int), hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    if (*m->h_flag & FLAG_NONFINITE)
        return fail(SVL_INTERNAL, "the audio tower produced a non-finite value");
    return SVL_OK;
}

// Runs the tower; soft tokens stay in m->soft, clip after clip. Mel frames
// come from the host spectrograms, or from d_features ([sum frames, 128] in
// HBM). A batch whose layer-0 activations would pass au_pass_fits runs as
// consecutive passes over groups of whole clips on the same stream; every
// clip is an independent reference call, so its output does not depend on
// the grouping. Caller holds m->mu.
svl_status run_audio(svl_audio_model *m, const svl_mel *mels, int32_t batch,
                     const float *d_features, hipStream_t s, AuBatch &b, int64_t *out_tokens,
                     float *out_soft, float *out_sscp, float *out_hidden) {
    HIP_TRY(hipSetDevice(m->device));
    ST_TRY(prepare_clips(m, mels, batch, d_features == nullptr, b));
    if (batch == 0) return SVL_OK;
    std::vector<int32_t> first(1, 0);  // first clip of each pass, then batch
    for (int32_t i = 0, t0 = 0; i < batch; ++i) {
        const int64_t f1 = (mels[i].frames + 1) / 2;
        if (i > first.back() && !au_pass_fits(m, t0 + f1)) {
            first.push_back(i);
            t0 = 0;
        }
        t0 += (int32_t)f1;
    }
    first.push_back(batch);
    const size_t passes = first.size() - 1;
    std::vector<AuBatch> parts(passes > 1 ? passes : 0);
    for (size_t g = 0; g < parts.size(); ++g)
        ST_TRY(prepare_clips(m, mels + first[g], first[g + 1] - first[g], d_features == nullptr,
                             parts[g]));
    // every workspace is sized before the first launch, so no buffer moves
    // while an earlier pass still reads it
    for (size_t g = 0; g < passes; ++g) ST_TRY(ensure_au_workspace(m, passes > 1 ? parts[g] : b));
    HIP_TRY(m->soft.ensure((size_t)std::max<int64_t>(b.tokens, 1) * m->text_hidden));
    // each pass's metadata has its own staging region: the passes are
    // enqueued back to back, so no region is rewritten before its copy ran
    std::vector<size_t> stage(passes + 1, 0);
    for (size_t g = 0; g < passes; ++g) {
        size_t off[9];
        stage[g + 1] = stage[g] + au_meta_layout(passes > 1 ? parts[g] : b, off);
    }
    ST_TRY(au_staging(m, stage[passes]));
    std::vector<std::vector<float>> cap_sscp(passes), cap_hidden(passes);
    int64_t tok_off = 0;
    for (size_t g = 0; g < passes; ++g) {
        const AuBatch &pb = passes > 1 ? parts[g] : b;
        const int32_t c0 = first[g], nc = first[g + 1] - first[g];
        const float *feats = d_features ? d_features + b.frame_off[(size_t)c0] * FEATURE_SIZE
                                        : m->mel.p;
        for (int32_t i = 0; i < nc; ++i) {
            const svl_mel &mel = mels[c0 + i];
            if (mel.frames <= 0 || d_features) continue;
            HIP_TRY(hipMemcpyAsync(m->mel.p + pb.frame_off[(size_t)i] * FEATURE_SIZE,
                                   mel.features, (size_t)(mel.frames * FEATURE_SIZE) * 4,
                                   hipMemcpyHostToDevice, s));
        }
        ST_TRY(upload_au_meta(m, pb, mels + c0, s, g == 0, stage[g]));
        if (out_sscp) cap_sscp[g].resize((size_t)(pb.T * m->H));
        if (out_hidden) cap_hidden[g].resize((size_t)(m->L * pb.T * m->H));
        ST_TRY(enqueue_audio(m, pb, feats, s, m->soft.p + tok_off * m->text_hidden,
                             out_sscp ? cap_sscp[g].data() : nullptr,
                             out_hidden ? cap_hidden[g].data() : nullptr));
        tok_off += pb.tokens;
    }
    if (out_soft)
        HIP_TRY(hipMemcpyAsync(out_soft, m->soft.p, (size_t)(b.tokens * m->text_hidden) * 4,
                               hipMemcpyDeviceToHost, s));
    ST_TRY(au_finish(m, s));
    tok_off = 0;
    for (size_t g = 0; g < passes; ++g) {
        const AuBatch &pb = passes > 1 ? parts[g] : b;
        if (out_sscp) select_valid(pb, m->H, cap_sscp[g].data(), out_sscp + tok_off * m->H);
        for (int64_t l = 0; out_hidden && l < m->L; ++l)
            select_valid(pb, m->H, cap_hidden[g].data() + (size_t)(l * pb.T * m->H),
                         out_hidden + (size_t)((l * b.tokens + tok_off) * m->H));
        tok_off += pb.tokens;
    }
    if (out_tokens)
        for (int i = 0; i < batch; ++i) out_tokens[i] = b.tokens_per_clip[(size_t)i];
    return SVL_OK;
}

// AudioEmbedder::embed_impl (audio_embedder.rs:223-267) for a batch.
svl_status embed_checks(svl_audio_model *m, svl_text_model *text,
                        const svl_audio_special_tokens *tokens, int64_t dimension, float *out) {
    if (!m || !text || !tokens || !out)
        return fail(SVL_USAGE, "models, special tokens and output are required");
    const int64_t E = text_embedding_dim(text);
    if (dimension <= 0 || dimension > E)
        return fail(SVL_INTERNAL, "embedding dimension %lld is outside 1..=%lld",
                    (long long)dimension, (long long)E);
    if (text_device(text) != m->device)
        return fail(SVL_USAGE, "the audio and text models live on different devices");
    if (text_hidden_size(text) != m->text_hidden)
        return fail(SVL_USAGE, "the audio projection width %lld is not the text hidden size %lld",
                    (long long)m->text_hidden, (long long)text_hidden_size(text));
    return SVL_OK;
}

// The embedder body; caller holds m->mu and ran embed_checks.
svl_status audio_embed_locked(svl_audio_model *m, svl_text_model *text,
                              const svl_audio_special_tokens *tokens, const svl_mel *mels,
                              int32_t batch, const float *d_features, int64_t dimension,
                              float *out) {
    const int64_t E = text_embedding_dim(text);
    AuBatch b;
    ST_TRY(run_audio(m, mels, batch, d_features, m->stream, b, nullptr, nullptr, nullptr, nullptr));
    if (batch == 0) return SVL_OK;
    std::vector<int64_t> offsets(1, 0);
    for (int i = 0; i < batch; ++i) {
        const int64_t seq = b.tokens_per_clip[(size_t)i] + 4;
        if (seq > MAX_TEXT_TOKENS)
            return fail(SVL_LIMIT, "clip %d: audio prompt has %lld tokens, above the %lld-token context",
                        i, (long long)seq, (long long)MAX_TEXT_TOKENS);
        offsets.push_back(offsets.back() + seq);
    }
    std::vector<uint32_t> ids((size_t)offsets.back());
    std::vector<int32_t> featmap((size_t)offsets.back(), -1);
    int64_t soft_off = 0;
    for (int i = 0; i < batch; ++i) {
        const int64_t o = offsets[i], n = b.tokens_per_clip[(size_t)i];
        ids[(size_t)o] = tokens->bos;
        ids[(size_t)o + 1] = tokens->boa;
        for (int64_t k = 0; k < n; ++k) {
            ids[(size_t)(o + 2 + k)] = tokens->audio;
            featmap[(size_t)(o + 2 + k)] = (int32_t)(soft_off + k);
        }
        ids[(size_t)(o + 2 + n)] = tokens->eoa;
        ids[(size_t)(o + 3 + n)] = tokens->eos;
        soft_off += n;
    }
    std::vector<float> normalized((size_t)(batch * E));
    ST_TRY(text_forward_with_device_features(text, ids.data(), offsets.data(), batch,
                                             featmap.data(), m->soft.p, normalized.data()));
    for (int i = 0; i < batch; ++i)
        ST_TRY(svl_truncate_and_normalize(normalized.data() + (size_t)i * E, (size_t)E,
                                          (size_t)dimension, out + (size_t)i * dimension));
    return SVL_OK;
}

svl_status audio_embed(svl_audio_model *m, svl_text_model *text,
                       const svl_audio_special_tokens *tokens, const svl_mel *mels, int32_t batch,
                       const float *d_features, int64_t dimension, float *out) {
    ST_TRY(embed_checks(m, text, tokens, dimension, out));
    std::lock_guard<std::mutex> lock(m->mu);
    return audio_embed_locked(m, text, tokens, mels, batch, d_features, dimension, out);
}

// AudioEmbedder::embed from 16 kHz samples (audio_embedder.rs:235-237): the
// log-mel features are computed into HBM on the model's stream and feed the
// tower directly.
svl_status audio_embed_samples(svl_audio_model *m, svl_text_model *text,
                               const svl_audio_special_tokens *tokens,
                               const float *const *h_samples, const float *d_samples,
                               const int64_t *lengths, int32_t clips, int64_t dimension,
                               float *out) {
    ST_TRY(embed_checks(m, text, tokens, dimension, out));
    std::lock_guard<std::mutex> lock(m->mu);
    HIP_TRY(hipSetDevice(m->device));
    if (!m->lm) ST_TRY(mel_create_on(m->device, &m->lm));
    MelBatch mb;
    ST_TRY(mel_plan(lengths, clips, mb));
    if (clips == 0) return SVL_OK;
    HIP_TRY(m->lm->features.ensure((size_t)(mb.total_frames * FEATURE_SIZE)));
    ST_TRY(mel_compute(m->lm, mb, h_samples, d_samples, lengths, m->lm->features.p, m->stream));
    std::vector<svl_mel> mels((size_t)clips);
    for (int32_t i = 0; i < clips; ++i)
        mels[(size_t)i] = {nullptr, mb.mask.data() + mb.frame_off[(size_t)i],
                           mb.frame_off[(size_t)i + 1] - mb.frame_off[(size_t)i]};
    return audio_embed_locked(m, text, tokens, mels.data(), clips, m->lm->features.p, dimension,
                              out);
}

}  // namespace

extern "C" {

svl_status svl_audio_model_create(svl_ctx *ctx, const svl_audio_config *cfg, int64_t text_hidden,
                                  const svl_tensor_view *tensors, size_t n_tensors,
                                  svl_audio_model **out) {
    if (!ctx || !out) return fail(SVL_USAGE, "context or output pointer is null");
    ST_TRY(validate_audio_config(cfg, text_hidden));
    HIP_TRY(hipSetDevice(ctx->device));
    const ShapeList shapes = audio_tensor_shapes(cfg, text_hidden);
    TensorIndex by_name;
    ST_TRY(check_inventory(tensors, n_tensors, shapes, {"audio_tower.", "embed_audio."}, "audio",
                           MAX_AUDIO_WEIGHT_ELEMENTS, by_name));

    auto m = new svl_audio_model();
    std::unique_ptr<svl_audio_model> guard(m);
    m->device = ctx->device;
    m->H = cfg->hidden_size;
    m->I = 4 * m->H;
    m->L = cfg->num_hidden_layers;
    m->NH = cfg->num_attention_heads;
    m->hd = m->H / m->NH;
    m->K = cfg->conv_kernel_size;
    m->C0 = cfg->conv_channels0;
    m->C1 = cfg->conv_channels1;
    m->chunk = cfg->attention_chunk_size;
    m->left = cfg->attention_context_left;
    m->right = cfg->attention_context_right;
    m->P = cfg->output_proj_dims;
    m->text_hidden = text_hidden;
    m->context = m->chunk + m->left - 1 + m->right;
    m->positions = m->context / 2 + 1;
    m->cap = (float)cfg->attention_logit_cap;
    m->eps = (float)cfg->rms_norm_eps;
    m->rw = (float)cfg->residual_weight;
    m->clip = (float)cfg->gradient_clipping;
    m->k_scale = (float)(std::log(1.0 + EULER) / LN_2);
    m->H_pad = (m->H + 31) / 32 * 32;
    // Backend limits (one wave per row, registers for a head).
    if (m->H % 4 || m->H > 2048 || m->P % 4 || m->P > 2048)
        return fail(SVL_UNSUPPORTED, "audio hidden and projection widths must be multiples of 4 up to 2048");
    if (m->hd > 256 || m->context > 64)
        return fail(SVL_UNSUPPORTED, "audio head dimension above 256 or attention context above 64");
    if (m->C0 > 512)
        return fail(SVL_UNSUPPORTED, "audio subsampling channels above 512 are not supported");

    std::vector<float> a, b2;
    auto up = [&](const std::string &name, float **dst) -> svl_status {
        ST_TRY(decode_named(by_name, name, a));
        return upload_owned(m->allocations, a.data(), a.size(), dst);
    };
    const std::string sp = "audio_tower.subsample_conv_projection.";
    ST_TRY(up(sp + "layer0.conv.weight", &m->w_conv0));
    ST_TRY(up(sp + "layer0.norm.weight", &m->ln0));
    // Layer-1 convolution weight [C1][C0][3][3]; the implicit-im2col GEMM
    // takes it tap-major, [C1][3 x 3][C0].
    ST_TRY(decode_named(by_name, sp + "layer1.conv.weight", a));
    b2.assign(a.size(), 0.f);
    for (int64_t o = 0; o < m->C1; ++o)
        for (int64_t c = 0; c < m->C0; ++c)
            for (int64_t t = 0; t < 9; ++t)
                b2[(size_t)((o * 9 + t) * m->C0 + c)] = a[(size_t)((o * m->C0 + c) * 9 + t)];
    a.swap(b2);
    ST_TRY(upload_owned(m->allocations, a.data(), a.size(), &m->w_conv1));
    ST_TRY(up(sp + "layer1.norm.weight", &m->ln1));
    ST_TRY(up(sp + "input_proj_linear.weight", &m->w_in));
    ST_TRY(up("audio_tower.output_proj.weight", &m->w_out));
    ST_TRY(up("audio_tower.output_proj.bias", &m->b_out));
    ST_TRY(up("embed_audio.embedding_projection.weight", &m->w_emb));

    const std::vector<float> table = position_table(m->H, m->positions);
    float *d_table = nullptr;
    ST_TRY(upload_owned(m->allocations, table.data(), table.size(), &d_table));
    const float q_scale = (float)(std::pow((double)m->hd, -0.5) / LN_2);
    m->layers.resize((size_t)m->L);
    for (int64_t l = 0; l < m->L; ++l) {
        AuLayer &ly = m->layers[(size_t)l];
        const std::string p = "audio_tower.layers." + std::to_string(l) + ".";
        const char *ffs[2] = {"feed_forward1.", "feed_forward2."};
        for (int f = 0; f < 2; ++f) {
            const std::string q = p + ffs[f];
            ST_TRY(up(q + "pre_layer_norm.weight", &ly.ff_pre[f]));
            ST_TRY(up(q + "post_layer_norm.weight", &ly.ff_post[f]));
            ST_TRY(up(q + "ffw_layer_1.linear.weight", &ly.ff_w1[f]));
            ST_TRY(up(q + "ffw_layer_2.linear.weight", &ly.ff_w2[f]));
            ST_TRY(read_bounds(by_name, q + "ffw_layer_1", ly.ff_b1[f]));
            ST_TRY(read_bounds(by_name, q + "ffw_layer_2", ly.ff_b2[f]));
        }
        std::vector<float> qkv((size_t)(3 * m->H * m->H));
        const char *projs[3] = {"q_proj", "k_proj", "v_proj"};
        Bounds *bs[3] = {&ly.bq, &ly.bk, &ly.bv};
        for (int j = 0; j < 3; ++j) {
            ST_TRY(decode_named(by_name, p + "self_attn." + projs[j] + ".linear.weight", a));
            std::copy(a.begin(), a.end(), qkv.begin() + (int64_t)j * m->H * m->H);
            ST_TRY(read_bounds(by_name, p + "self_attn." + projs[j], *bs[j]));
        }
        ST_TRY(upload_owned(m->allocations, qkv.data(), qkv.size(), &ly.w_qkv));
        ST_TRY(up(p + "self_attn.post.linear.weight", &ly.w_post));
        ST_TRY(read_bounds(by_name, p + "self_attn.post", ly.bpost));
        // per-dimension query scale q_scale * softplus(per_dim_scale) (audio.rs:1565-1576)
        ST_TRY(decode_named(by_name, p + "self_attn.per_dim_scale", a));
        std::vector<float> qf((size_t)m->hd);
        for (int64_t d = 0; d < m->hd; ++d) {
            const float sc = softplus_host(a[(size_t)d]);
            if (!std::isfinite(sc)) return fail(SVL_INTERNAL, "audio per-dimension scale is not finite");
            qf[(size_t)d] = q_scale * sc;
        }
        ST_TRY(upload_owned(m->allocations, qf.data(), qf.size(), &ly.qf));
        // relative keys: position table x relative_k_proj^T (audio.rs:1035-1041)
        float *w_rel = nullptr;
        ST_TRY(up(p + "self_attn.relative_k_proj.weight", &w_rel));
        {
            float *relk = nullptr;
            HIP_TRY(hipMalloc((void **)&relk, (size_t)(m->positions * m->H) * 4));
            m->allocations.push_back(relk);
            GemmArgs g{d_table, m->H, w_rel, m->H, relk, m->H, (int)m->positions, (int)m->H,
                       (int)m->H, EPI_STORE, 1.f, nullptr, 0, 0};
            HIP_TRY(launch_gemm(g, nullptr));
            HIP_TRY(hipDeviceSynchronize());
            ly.relk = relk;
        }
        ST_TRY(up(p + "lconv1d.pre_layer_norm.weight", &ly.lc_pre));
        ST_TRY(decode_named(by_name, p + "lconv1d.linear_start.linear.weight", a));
        {   // rows [0, H) are the gated values, [H, 2H) the gates
            std::vector<float> first(a.begin(), a.begin() + m->H * m->H),
                second(a.begin() + m->H * m->H, a.end());
            const std::vector<float> il = interleave_gate_up(first, second, m->H, m->H_pad, m->H);
            ST_TRY(upload_owned(m->allocations, il.data(), il.size(), &ly.w_start));
        }
        ST_TRY(read_bounds(by_name, p + "lconv1d.linear_start", ly.bstart));
        ST_TRY(up(p + "lconv1d.linear_end.linear.weight", &ly.w_end));
        ST_TRY(read_bounds(by_name, p + "lconv1d.linear_end", ly.bend));
        // depthwise weight [H, 1, K] uploaded tap-major, [K, H]: the kernel
        // reads four channels' weights of one tap as one float4
        ST_TRY(decode_named(by_name, p + "lconv1d.depthwise_conv1d.weight", a));
        if ((int64_t)a.size() != m->K * m->H)
            return fail(SVL_INTERNAL, "audio depthwise weight has %zu elements, expected %lld",
                        a.size(), (long long)(m->K * m->H));
        {
            std::vector<float> dwt((size_t)(m->K * m->H));
            for (int64_t c = 0; c < m->H; ++c)
                for (int64_t t = 0; t < m->K; ++t) dwt[(size_t)(t * m->H + c)] = a[(size_t)(c * m->K + t)];
            ST_TRY(upload_owned(m->allocations, dwt.data(), dwt.size(), &ly.dw));
        }
        ST_TRY(up(p + "lconv1d.conv_norm.weight", &ly.lc_norm));
        ST_TRY(up(p + "norm_pre_attn.weight", &ly.norm_pre_attn));
        ST_TRY(up(p + "norm_post_attn.weight", &ly.norm_post_attn));
        ST_TRY(up(p + "norm_out.weight", &ly.norm_out));
    }
    HIP_TRY(hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking));
    HIP_TRY(hipHostMalloc((void **)&m->h_flag, sizeof(int), hipHostMallocDefault));
    *out = guard.release();
    return SVL_OK;
}

svl_status svl_audio_model_destroy(svl_audio_model *model) {
    delete model;
    return SVL_OK;
}

int64_t svl_audio_token_count(const uint8_t *mask, int64_t frames) {
    if (frames <= 0 || !mask) return 0;
    const int64_t f1 = (frames + 1) / 2, f2 = (f1 + 1) / 2;
    int64_t n = 0;
    for (int64_t t = 0; t < f2; ++t)
        if (2 * t < f1 && 4 * t < frames && mask[4 * t]) ++n;
    return n;
}

svl_status svl_audio_forward_batch(svl_audio_model *m, const svl_mel *mels, int32_t batch,
                                   int64_t *out_tokens, float *out_soft, float *out_sscp,
                                   float *out_hidden) {
    if (!m || !out_soft) return fail(SVL_USAGE, "model and out_soft are required");
    std::lock_guard<std::mutex> lock(m->mu);
    AuBatch b;
    return run_audio(m, mels, batch, nullptr, m->stream, b, out_tokens, out_soft, out_sscp,
                     out_hidden);
}

svl_status svl_audio_forward_device(svl_audio_model *m, const float *d_features,
                                    const svl_mel *mels, int32_t batch, float *d_out,
                                    void *stream) {
    if (!m || !d_features || !d_out) return fail(SVL_USAGE, "model, features and output are required");
    std::lock_guard<std::mutex> lock(m->mu);
    hipStream_t s = stream ? (hipStream_t)stream : m->stream;
    AuBatch b;
    ST_TRY(run_audio(m, mels, batch, d_features, s, b, nullptr, nullptr, nullptr, nullptr));
    if (batch == 0) return SVL_OK;
    HIP_TRY(hipMemcpyAsync(d_out, m->soft.p, (size_t)(b.tokens * m->text_hidden) * 4,
                           hipMemcpyDeviceToDevice, s));
    HIP_TRY(hipStreamSynchronize(s));
    return SVL_OK;
}

svl_status svl_audio_embed_batch(svl_audio_model *m, svl_text_model *text,
                                 const svl_audio_special_tokens *tokens, const svl_mel *mels,
                                 int32_t batch, int64_t dimension, float *out) {
    return audio_embed(m, text, tokens, mels, batch, nullptr, dimension, out);
}

svl_status svl_audio_embed_device(svl_audio_model *m, svl_text_model *text,
                                  const svl_audio_special_tokens *tokens, const float *d_features,
                                  const svl_mel *mels, int32_t batch, int64_t dimension,
                                  float *out) {
    if (!d_features) return fail(SVL_USAGE, "features are required");
    return audio_embed(m, text, tokens, mels, batch, d_features, dimension, out);
}

svl_status svl_audio_embed_samples(svl_audio_model *audio, svl_text_model *text,
                                   const svl_audio_special_tokens *tokens,
                                   const float *const *samples, const int64_t *lengths,
                                   int32_t clips, int64_t dimension, float *out) {
    if (clips > 0 && !samples) return fail(SVL_USAGE, "samples are required");
    return audio_embed_samples(audio, text, tokens, samples, nullptr, lengths, clips, dimension,
                               out);
}

svl_status svl_audio_embed_samples_device(svl_audio_model *audio, svl_text_model *text,
                                          const svl_audio_special_tokens *tokens,
                                          const float *d_samples, const int64_t *lengths,
                                          int32_t clips, int64_t dimension, float *out) {
    if (clips > 0 && !d_samples) return fail(SVL_USAGE, "samples are required");
    return audio_embed_samples(audio, text, tokens, nullptr, d_samples, lengths, clips, dimension,
                               out);
}

}  // extern "C"
