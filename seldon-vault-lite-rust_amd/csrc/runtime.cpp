// Host runtime of the MI355X encoder backend: the C ABI of include/svl_hip.h.
//
// It plays the role of the reference's TextModel (src/model/text.rs) with
// the forward pass moved to HBM: weights are validated like
// src/model/weights.rs:125-241 and packed once at model creation; every
// forward call packs the rows of a batch back to back (no padding), runs the
// whole encoder as one launch sequence on one stream, and reads back only
// the pooled / normalised vectors (plus optional captures).
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/svl_hip.h"
#include "host_common.hpp"
#include "svl_internal.hpp"

namespace {

using namespace svl;

// src/model/config.rs:27-51, text.rs:34, tensor/owned.rs MAX_TENSOR_ELEMENTS,
// weights.rs MAX_WEIGHT_ELEMENTS.
constexpr int64_t MAX_TEXT_TOKENS = 8192;
constexpr int64_t MAX_HIDDEN_SIZE = 16384;
constexpr int64_t MAX_LAYERS = 128;
constexpr int64_t MAX_HEADS = 128;
constexpr int64_t MAX_HEAD_DIM = 1024;
constexpr int64_t MAX_INTERMEDIATE_SIZE = 65536;
constexpr int64_t MAX_VOCAB_SIZE = 1000000;
constexpr int64_t MAX_EMBEDDING_DIM = 16384;
constexpr int64_t MAX_POSITIONS = 1048576;
constexpr int64_t MAX_WEIGHT_ELEMENTS = int64_t(1) << 30;

// ---------------------------------------------------------------------------
// Kernel timing classes.
enum KernelClass : int {
    KC_GEMM_QKV = 0,
    KC_GEMM_O,
    KC_GEMM_GATE_UP,
    KC_GEMM_DOWN,
    KC_GEMM_PLE_GATE,
    KC_GEMM_PLE_PROJ,
    KC_GEMM_PLE_MODEL,
    KC_GEMM_OUT,
    KC_ATTENTION,
    KC_QKV_POST,
    KC_RESNORM,
    KC_GATHER,
    KC_PLE_NORM,
    KC_POOL,
    KC_COUNT
};
const char *kClassNames[KC_COUNT] = {
    "gemm_qkv",      "gemm_o",         "gemm_gate_up", "gemm_down", "gemm_ple_gate",
    "gemm_ple_proj", "gemm_ple_model", "gemm_out",     "attention", "qkv_norm_rope",
    "resnorm",       "gather",         "ple_norm",     "pool"};

struct DevLayer {
    float *w_qkv = nullptr, *w_o = nullptr, *w_gu = nullptr, *w_down = nullptr;
    float *w_pg = nullptr, *w_pp = nullptr;
    float *ln_in = nullptr, *ln_post_attn = nullptr, *ln_pre_ff = nullptr, *ln_post_ff = nullptr,
          *ln_post_ple = nullptr, *q_norm = nullptr, *k_norm = nullptr;
    float scalar = 1.f;
    int hd = 0, nkv = 0, full = 0;
};

struct TimedLaunch {
    int cls;
    double work;
    hipEvent_t a, b;
};

// Typed view into the model's metadata block (set by upload_batch_meta).
template <typename T>
struct MetaView {
    T *p = nullptr;
};

}  // namespace

struct svl_text_model {
    int device = 0;
    // configuration (config.rs:76-95)
    int64_t V = 0, H = 0, I = 0, L = 0, NH = 0, P = 0, E = 0, max_pos = 0, window = 0, pad = -1;
    float eps = 0.f, full_theta = 0.f, slide_theta = 0.f;
    float embedding_scale = 1.f, ple_scale = 1.f;
    int64_t I_pad = 0;
    std::vector<DevLayer> layers;
    std::vector<float *> allocations;
    float *embed = nullptr, *out_proj = nullptr, *final_norm = nullptr, *ple_model = nullptr,
          *ple_norm = nullptr;
    // RoPE tables [rope_positions, hd/2] per layer type (0 sliding, 1 full)
    float *cos_t[2] = {nullptr, nullptr}, *sin_t[2] = {nullptr, nullptr};
    int64_t rope_positions = 0;
    int type_hd[2] = {0, 0};

    int64_t max_qkv = 0, max_q = 0;  // widest per-layer QKV / query row
    hipStream_t stream = nullptr;
    static constexpr int MAX_GROUPS = 4;
    hipStream_t extra[MAX_GROUPS - 1] = {};  // streams of row groups 1..3
    hipEvent_t ev_fork = nullptr, ev_join[MAX_GROUPS - 1] = {};
    int row_groups = 3;                      // row groups per large batch
    int64_t pass_tokens = 0;                 // tokens per pass (0: from PASS_BYTES)
    std::mutex mu;

    // workspace
    DevBuf<float> h, n, tmp, qkv, attn, act, ple, pg, proj, feats, pooled, normalized, trunc;
    DevBuf<int32_t> pos, rowlen, featmap;
    DevBuf<uint32_t> ids;
    // A pass's metadata in one device block, filled by one copy from pinned
    // host memory: the error flag (cleared), the Matryoshka dims, the row
    // offsets and the attention work items (the views below).
    DevBuf<unsigned char> meta;
    unsigned char *h_meta = nullptr;  // pinned staging of `meta`
    size_t h_meta_n = 0;
    hipEvent_t ev_meta = nullptr;     // after the last copy out of h_meta
    MetaView<int> flag;
    MetaView<int32_t> dims;
    MetaView<int64_t> offsets;
    MetaView<AttnTile> tiles;
    int *h_flag = nullptr;  // pinned

    // kernel timing
    bool timing = false;
    std::vector<TimedLaunch> pending;
    std::vector<hipEvent_t> event_pool;
    double stat_ms[KC_COUNT] = {0};
    int64_t stat_launches[KC_COUNT] = {0};
    double stat_work[KC_COUNT] = {0};

    ~svl_text_model() {
        if (device >= 0) (void)hipSetDevice(device);
        for (float *p : allocations) (void)hipFree(p);
        for (int t = 0; t < 2; ++t) {
            if (cos_t[t]) (void)hipFree(cos_t[t]);
            if (sin_t[t]) (void)hipFree(sin_t[t]);
        }
        h.release(); n.release(); tmp.release(); qkv.release(); attn.release(); act.release();
        ple.release(); pg.release(); proj.release(); feats.release(); pooled.release();
        normalized.release(); trunc.release(); pos.release(); rowlen.release();
        featmap.release(); ids.release(); meta.release();
        if (ev_meta) {
            (void)hipEventSynchronize(ev_meta);
            (void)hipEventDestroy(ev_meta);
        }
        if (h_meta) (void)hipHostFree(h_meta);
        if (h_flag) (void)hipHostFree(h_flag);
        for (auto &e : event_pool) (void)hipEventDestroy(e);
        for (auto &t : pending) {
            (void)hipEventDestroy(t.a);
            (void)hipEventDestroy(t.b);
        }
        if (ev_fork) (void)hipEventDestroy(ev_fork);
        for (int i = 0; i < MAX_GROUPS - 1; ++i) {
            if (ev_join[i]) (void)hipEventDestroy(ev_join[i]);
            if (extra[i]) (void)hipStreamDestroy(extra[i]);
        }
        if (stream) (void)hipStreamDestroy(stream);
    }
};

namespace {

// ---------------------------------------------------------------------------
// Configuration validation (config.rs:503-616, 647-649, 695-736).

svl_status validate_config(const svl_text_config *c) {
    if (!c) return fail(SVL_USAGE, "configuration is null");
    auto cap = [](int64_t v, int64_t hi, const char *what) -> svl_status {
        if (v <= 0 || v > hi) return fail(SVL_LIMIT, "%s %lld is outside 1..=%lld", what,
                                          (long long)v, (long long)hi);
        return SVL_OK;
    };
    ST_TRY(cap(c->hidden_size, MAX_HIDDEN_SIZE, "hidden size"));
    ST_TRY(cap(c->intermediate_size, MAX_INTERMEDIATE_SIZE, "intermediate size"));
    ST_TRY(cap(c->num_hidden_layers, MAX_LAYERS, "layer count"));
    ST_TRY(cap(c->num_attention_heads, MAX_HEADS, "attention head count"));
    ST_TRY(cap(c->hidden_size_per_layer_input, MAX_HIDDEN_SIZE, "per-layer input size"));
    ST_TRY(cap(c->embedding_dim, MAX_EMBEDDING_DIM, "embedding dimension"));
    ST_TRY(cap(c->vocab_size, MAX_VOCAB_SIZE, "vocabulary size"));
    ST_TRY(cap(c->max_position_embeddings, MAX_POSITIONS, "position count"));
    ST_TRY(cap(c->sliding_window, c->max_position_embeddings, "sliding window"));
    if (!std::isfinite(c->rms_norm_eps) || c->rms_norm_eps < 0)
        return fail(SVL_CORRUPT, "RMSNorm epsilon must be finite and non-negative");
    if (!std::isfinite((float)c->rms_norm_eps))
        return fail(SVL_CORRUPT, "RMSNorm epsilon does not fit a finite f32 value");
    if (!c->layer_type || !c->head_dim || !c->num_kv_heads)
        return fail(SVL_USAGE, "per-layer arrays are null");
    const int64_t nh = c->num_attention_heads;
    int type_hd[2] = {0, 0};
    for (int64_t l = 0; l < c->num_hidden_layers; ++l) {
        const int64_t kv = c->num_kv_heads[l], hd = c->head_dim[l];
        if (c->layer_type[l] != 0 && c->layer_type[l] != 1)
            return fail(SVL_UNSUPPORTED, "layer %lld has an unsupported attention type",
                        (long long)l);
        if (kv <= 0 || kv > nh)
            return fail(SVL_CORRUPT, "key/value head count %lld is not in 1..=%lld",
                        (long long)kv, (long long)nh);
        if (nh % kv)
            return fail(SVL_CORRUPT,
                        "attention head count %lld is not a multiple of key/value head count %lld",
                        (long long)nh, (long long)kv);
        if (hd <= 0 || hd > MAX_HEAD_DIM || hd % 2)
            return fail(SVL_CORRUPT, "head dimension %lld must be a positive even value at most %lld",
                        (long long)hd, (long long)MAX_HEAD_DIM);
        int &t = type_hd[c->layer_type[l]];
        if (t == 0) t = (int)hd;
        else if (t != hd)
            return fail(SVL_UNSUPPORTED,
                        "layers of the same attention type must share one head dimension");
    }
    if (c->layer_type[c->num_hidden_layers - 1] != 1)
        return fail(SVL_UNSUPPORTED, "the last layer must use full attention");
    for (double th : {c->full_rope_theta, c->sliding_rope_theta})
        if (!std::isfinite(th) || th <= 1.0)
            return fail(SVL_CORRUPT, "RoPE theta %g must be finite and greater than one", th);
    if (c->pad_token_id >= c->vocab_size)
        return fail(SVL_CORRUPT, "special token id %lld is outside the vocabulary",
                    (long long)c->pad_token_id);
    return SVL_OK;
}

// TextConfig::tensor_shapes (config.rs:394-484).
std::vector<std::pair<std::string, std::vector<int64_t>>> tensor_shapes(const svl_text_config *c) {
    const int64_t H = c->hidden_size, P = c->hidden_size_per_layer_input,
                  I = c->intermediate_size;
    std::vector<std::pair<std::string, std::vector<int64_t>>> s;
    s.push_back({"language_model.embed_tokens.weight", {c->vocab_size, H}});
    s.push_back({"language_model.embedding_projection.weight", {c->embedding_dim, H}});
    s.push_back({"language_model.norm.weight", {H}});
    s.push_back({"language_model.ple.per_layer_model_projection.weight",
                 {c->num_hidden_layers * P, H}});
    s.push_back({"language_model.ple.per_layer_projection_norm.weight", {P}});
    for (int64_t l = 0; l < c->num_hidden_layers; ++l) {
        const std::string p = "language_model.layers." + std::to_string(l);
        const int64_t qd = c->num_attention_heads * c->head_dim[l];
        const int64_t kd = c->num_kv_heads[l] * c->head_dim[l];
        s.push_back({p + ".input_layernorm.weight", {H}});
        s.push_back({p + ".post_attention_layernorm.weight", {H}});
        s.push_back({p + ".pre_feedforward_layernorm.weight", {H}});
        s.push_back({p + ".post_feedforward_layernorm.weight", {H}});
        s.push_back({p + ".layer_scalar", {1}});
        s.push_back({p + ".mlp.gate_proj.weight", {I, H}});
        s.push_back({p + ".mlp.up_proj.weight", {I, H}});
        s.push_back({p + ".mlp.down_proj.weight", {H, I}});
        s.push_back({p + ".ple_block.per_layer_input_gate.weight", {P, H}});
        s.push_back({p + ".ple_block.per_layer_projection.weight", {H, P}});
        s.push_back({p + ".ple_block.post_per_layer_input_norm.weight", {H}});
        s.push_back({p + ".self_attn.q_proj.weight", {qd, H}});
        s.push_back({p + ".self_attn.k_proj.weight", {kd, H}});
        s.push_back({p + ".self_attn.v_proj.weight", {kd, H}});
        s.push_back({p + ".self_attn.o_proj.weight", {H, qd}});
        s.push_back({p + ".self_attn.q_norm.weight", {c->head_dim[l]}});
        s.push_back({p + ".self_attn.k_norm.weight", {c->head_dim[l]}});
    }
    return s;
}

svl_status upload(svl_text_model *m, const float *host, size_t count, float **dst) {
    return upload_owned(m->allocations, host, count, dst);
}

// RoPE cos/sin tables with the reference's exact f32 angles
// (kernels.rs:974-976: angle = (pos as f32) * inv_freq[j], sin_cos) and
// inverse frequencies (kernels.rs:1005-1008).
void rope_tables(int hd, float theta, int64_t positions, int64_t pos0, std::vector<float> &c,
                 std::vector<float> &s) {
    const int half = hd / 2;
    std::vector<float> inv(half);
    for (int j = 0; j < half; ++j) {
        const float exponent = (float)(2 * j) / (float)hd;
        inv[j] = 1.0f / std::pow(theta, exponent);
    }
    c.resize((size_t)(positions * half));
    s.resize((size_t)(positions * half));
    for (int64_t p = 0; p < positions; ++p)
        for (int j = 0; j < half; ++j) {
            const float angle = (float)(pos0 + p) * inv[j];
            c[(size_t)(p * half + j)] = std::cos(angle);
            s[(size_t)(p * half + j)] = std::sin(angle);
        }
}

// ---------------------------------------------------------------------------
// Kernel timing helpers.

struct Timer {
    svl_text_model *m;
    hipStream_t s;
    int cls;
    double work;
    hipEvent_t a = nullptr;
    Timer(svl_text_model *m_, hipStream_t s_, int cls_, double work_)
        : m(m_), s(s_), cls(cls_), work(work_) {
        if (!m->timing) return;
        a = take();
        (void)hipEventRecord(a, s);
    }
    hipEvent_t take() {
        if (!m->event_pool.empty()) {
            hipEvent_t e = m->event_pool.back();
            m->event_pool.pop_back();
            return e;
        }
        hipEvent_t e = nullptr;
        (void)hipEventCreate(&e);
        return e;
    }
    ~Timer() {
        if (!m->timing || !a) return;
        hipEvent_t b = take();
        (void)hipEventRecord(b, s);
        m->pending.push_back({cls, work, a, b});
    }
};

void collect_timing(svl_text_model *m) {
    for (auto &t : m->pending) {
        float ms = 0.f;
        if (hipEventElapsedTime(&ms, t.a, t.b) == hipSuccess) {
            m->stat_ms[t.cls] += ms;
            m->stat_launches[t.cls] += 1;
            m->stat_work[t.cls] += t.work;
        }
        m->event_pool.push_back(t.a);
        m->event_pool.push_back(t.b);
    }
    m->pending.clear();
}

// ---------------------------------------------------------------------------
// Per-call geometry.
//
// A large batch is cut into a few groups of consecutive rows with about the
// same number of tokens. Each group runs the whole encoder on its own stream
// (all at the default priority), on its own token range of every workspace
// buffer, so the streams' kernels fill each other's partial last rounds of
// workgroups and the bandwidth-bound norm kernels of one group overlap the
// MFMA-bound GEMMs of another. Every row's arithmetic is unchanged.

constexpr int64_t SPLIT_MIN_TOKENS = 4096;

struct Group {
    int32_t r0 = 0, nrows = 0;  // rows [r0, r0 + nrows)
    int64_t t0 = 0, T = 0;      // tokens [t0, t0 + T)
    int64_t off_slot = 0;       // first entry of this group's rebased offsets
    int64_t shortest = 0;       // shortest row of the group
    // attention work lists per distinct (nkv, hd): (first tile, count)
    std::map<std::pair<int, int>, std::pair<int, int>> tile_ranges;
    double attn_flops[2] = {0, 0};  // algorithmic attention FLOPs per layer type
};

struct Batch {
    int32_t B = 0;
    int64_t T = 0;
    std::vector<int64_t> offsets;      // host copy, global
    std::vector<int64_t> dev_offsets;  // per group: nrows + 1 offsets rebased to the group
    std::vector<AttnTile> tiles;       // all groups, tok0 relative to the group
    std::vector<Group> groups;
    int64_t hidden_stride = 0;         // tokens per layer block of captured states (0: T)
};

void build_group(const svl_text_model *m, Batch &b, Group &g) {
    g.off_slot = (int64_t)b.dev_offsets.size();
    for (int r = 0; r <= g.nrows; ++r) b.dev_offsets.push_back(b.offsets[g.r0 + r] - g.t0);
    for (int r = 0; r < g.nrows; ++r) {
        const int64_t len = b.offsets[g.r0 + r + 1] - b.offsets[g.r0 + r];
        g.shortest = r == 0 ? len : std::min(g.shortest, len);
    }
    std::vector<int> order(g.nrows);
    for (int r = 0; r < g.nrows; ++r) order[r] = g.r0 + r;
    // longest rows first: the attention cost of a work item grows with its row
    std::stable_sort(order.begin(), order.end(), [&](int x, int y) {
        return b.offsets[x + 1] - b.offsets[x] > b.offsets[y + 1] - b.offsets[y];
    });
    for (const DevLayer &ly : m->layers) {
        const auto key = std::make_pair(ly.nkv, ly.hd);
        if (g.tile_ranges.count(key)) continue;
        const int bv = attn_block_vectors(ly.hd);
        const int first = (int)b.tiles.size();
        if (bv > 0) {
            const int G = (int)(m->NH / ly.nkv);
            for (int r : order) {
                const int64_t len = b.offsets[r + 1] - b.offsets[r];
                const int32_t tok0 = (int32_t)(b.offsets[r] - g.t0);
                for (int kv = 0; kv < ly.nkv; ++kv)
                    for (int64_t v0 = 0; v0 < len * G; v0 += bv)
                        b.tiles.push_back({tok0, (int32_t)len, kv, (int32_t)v0});
            }
        }
        g.tile_ranges[key] = {first, (int)b.tiles.size() - first};
    }
    // algorithmic attention FLOPs: 4 * hd * nh * sum_i keys(i) per layer
    for (int t = 0; t < 2; ++t) {
        double f = 0;
        const int hd = m->type_hd[t];
        if (!hd) continue;
        for (int r = g.r0; r < g.r0 + g.nrows; ++r) {
            const int64_t len = b.offsets[r + 1] - b.offsets[r];
            double keys = 0;
            if (t == 1 || m->window >= len) {
                keys = (double)len * (double)len;
            } else {
                for (int64_t i = 0; i < len; ++i)
                    keys += (double)(std::min(len - 1, i + m->window) -
                                     std::max<int64_t>(0, i - m->window) + 1);
            }
            f += 4.0 * hd * (double)m->NH * keys;
        }
        g.attn_flops[t] = f;
    }
}

void build_groups(const svl_text_model *m, Batch &b, int max_groups) {
    b.groups.clear();
    b.tiles.clear();
    b.dev_offsets.clear();
    int ng = 1;
    if (b.T >= SPLIT_MIN_TOKENS) ng = std::max(1, std::min<int>(max_groups, b.B));
    // When every row is longer than the sliding window, the sliding layers'
    // attention gives each XCD a contiguous range of its work items
    // (launch_attention). Concurrent row groups interleave their workgroups
    // over the XCDs and lose that placement, which is worth more than their
    // overlap: 8 x 2048 tokens take 43.2 ms as one group, 44.3 ms as three.
    bool windowed = false;
    for (const DevLayer &ly : m->layers) windowed = windowed || !ly.full;
    if (windowed && m->window >= 0 && b.B > 0) {
        int64_t shortest = b.offsets[1] - b.offsets[0];
        for (int32_t i = 1; i < b.B; ++i) shortest = std::min(shortest, b.offsets[i + 1] - b.offsets[i]);
        if (shortest > m->window + 1) ng = 1;
    }
    // group k starts at the first row boundary at or past k/ng of the tokens,
    // every group keeping at least one row
    int32_t r = 0;
    for (int k = 0; k < ng; ++k) {
        int32_t end = b.B;
        if (k + 1 < ng) {
            end = std::max(r + 1, 1);
            while (end < b.B - (ng - 1 - k) && (int64_t)ng * b.offsets[end] < (int64_t)(k + 1) * b.T)
                ++end;
        }
        Group g;
        g.r0 = r;
        g.nrows = end - r;
        b.groups.push_back(g);
        r = end;
    }
    for (Group &g : b.groups) {
        g.t0 = b.offsets[g.r0];
        g.T = b.offsets[g.r0 + g.nrows] - g.t0;
        build_group(m, b, g);
    }
}

svl_status ensure_workspace(svl_text_model *m, const Batch &b, int64_t feat_floats,
                            bool need_featmap, int dims_total) {
    const int64_t T = std::max<int64_t>(b.T, 1);
    HIP_TRY(m->h.ensure(T * m->H));
    HIP_TRY(m->n.ensure(T * m->H));
    HIP_TRY(m->tmp.ensure(T * m->H));
    HIP_TRY(m->qkv.ensure(T * m->max_qkv));
    HIP_TRY(m->attn.ensure(T * m->max_q));
    HIP_TRY(m->act.ensure(T * m->I));
    HIP_TRY(m->ple.ensure(T * m->L * m->P));
    HIP_TRY(m->pg.ensure(T * m->P));
    HIP_TRY(m->proj.ensure(T * m->E));
    HIP_TRY(m->pos.ensure(T));
    HIP_TRY(m->rowlen.ensure(T));
    HIP_TRY(m->ids.ensure(T));
    HIP_TRY(m->pooled.ensure((size_t)b.B * m->E));
    HIP_TRY(m->normalized.ensure((size_t)b.B * m->E));
    if (feat_floats > 0) HIP_TRY(m->feats.ensure(feat_floats));
    if (need_featmap) HIP_TRY(m->featmap.ensure(T));
    if (dims_total > 0) HIP_TRY(m->trunc.ensure((size_t)b.B * dims_total));
    return SVL_OK;
}

// The whole encoder for one group of rows, enqueued on `s`
// (text.rs:209-531). Inputs already in m->ids / m->offsets / m->tiles (and
// m->featmap / m->feats when has_features). Every buffer is addressed at the
// group's token (or row) range; the per-layer-width QKV and attention
// buffers are carved at their widest layer so the groups never overlap.
// d_featmap (per token: feature row or -1) and d_feats are null without
// multimodal features.
svl_status enqueue_group(svl_text_model *m, const Batch &b, const Group &grp, hipStream_t s,
                         const uint32_t *d_ids, const int32_t *d_featmap, const float *d_feats,
                         const int32_t *d_dims,
                         int n_dims, int dims_total, float *d_trunc, float *h_hidden) {
    const int64_t T = grp.T, H = m->H, P = m->P, L = m->L, E = m->E, t0 = grp.t0;
    if (T == 0) return SVL_OK;
    int *flag = m->flag.p;
    const double Td = (double)T;
    float *h = m->h.p + t0 * H, *n = m->n.p + t0 * H, *tmp = m->tmp.p + t0 * H;
    float *qkv = m->qkv.p + t0 * m->max_qkv, *attn = m->attn.p + t0 * m->max_q;
    float *act = m->act.p + t0 * m->I, *ple = m->ple.p + t0 * L * P, *pg = m->pg.p + t0 * P;
    float *proj = m->proj.p + t0 * E;
    int32_t *pos = m->pos.p + t0, *rowlen = m->rowlen.p + t0;
    const int64_t *offs = m->offsets.p + grp.off_slot;
    const int64_t T_all = b.hidden_stride > 0 ? b.hidden_stride : b.T;
    // CUs each launch can expect while the batch's groups run side by side
    const int cus = b.groups.size() > 1 ? (int)(256 / b.groups.size()) : 0;

    HIP_TRY(launch_positions(offs, grp.nrows, pos, rowlen, s));
    {
        Timer tm(m, s, KC_GATHER, Td * H * 4 * 3);
        HIP_TRY(launch_gather(d_ids + t0, m->embed, m->V, d_featmap ? d_featmap + t0 : nullptr,
                              d_feats, m->embedding_scale,
                              m->layers[0].ln_in, h, n, T, (int)H, m->eps, flag, s));
    }
    if (h_hidden)
        HIP_TRY(hipMemcpyAsync(h_hidden + t0 * H, h, (size_t)(T * H) * 4, hipMemcpyDeviceToHost,
                               s));

    // Projection-only per-layer embeddings (text.rs:285-306).
    {
        GemmArgs g{h, H, m->ple_model, H, ple, L * P, (int)T, (int)(L * P), (int)H, EPI_SCALE,
                   m->ple_scale, nullptr, 0, 0};
        g.cus = cus;
        Timer tm(m, s, KC_GEMM_PLE_MODEL, 2.0 * Td * H * L * P);
        HIP_TRY(launch_gemm(g, s));
    }
    {
        Timer tm(m, s, KC_PLE_NORM, Td * L * P * 8);
        HIP_TRY(launch_rms_rows(ple, m->ple_norm, ple, T * L, (int)P, m->eps, flag, s));
    }

    for (int64_t l = 0; l < L; ++l) {
        const DevLayer &ly = m->layers[(size_t)l];
        const int64_t qd = m->NH * ly.hd, kd = (int64_t)ly.nkv * ly.hd, ldqkv = qd + 2 * kd;
        {
            GemmArgs g{n, H, ly.w_qkv, H, qkv, ldqkv, (int)T, (int)ldqkv, (int)H, EPI_STORE, 1.f,
                       nullptr, 0, 0};
            g.cus = cus;
            Timer tm(m, s, KC_GEMM_QKV, 2.0 * Td * H * ldqkv);
            HIP_TRY(launch_gemm(g, s));
        }
        {
            Timer tm(m, s, KC_QKV_POST, Td * ldqkv * 8);
            HIP_TRY(launch_qkv_post(qkv, ldqkv, T, (int)m->NH, ly.nkv, ly.hd, ly.q_norm, ly.k_norm,
                                    m->cos_t[ly.full], m->sin_t[ly.full], pos, m->eps, flag, s));
        }
        {
            const auto range = grp.tile_ranges.at(std::make_pair(ly.nkv, ly.hd));
            AttnArgs a{};
            a.q = qkv;
            a.k = qkv + qd;
            a.v = qkv + qd + kd;
            a.out = attn;
            a.ldq = a.ldk = a.ldv = ldqkv;
            a.ldo = qd;
            a.nh = (int)m->NH;
            a.nkv = ly.nkv;
            a.hd = ly.hd;
            a.window = ly.full ? -1 : (int)m->window;
            a.scale = 1.0f;  // text.rs:421
            a.tiles = m->tiles.p + range.first;
            a.n_tiles = range.second;
            a.pos = pos;
            a.rowlen = rowlen;
            a.tokens = T;
            a.flag = flag;
            a.max_len = std::min<int64_t>(T, MAX_TEXT_TOKENS);  // validate_row caps every row
            a.shortest = grp.shortest;
            Timer tm(m, s, KC_ATTENTION, grp.attn_flops[ly.full]);
            HIP_TRY(launch_attention(a, s));
        }
        {
            GemmArgs g{attn, qd, ly.w_o, qd, tmp, H, (int)T, (int)H, (int)qd, EPI_STORE, 1.f,
                       nullptr, 0, 0};
            g.cus = cus;
            Timer tm(m, s, KC_GEMM_O, 2.0 * Td * qd * H);
            HIP_TRY(launch_gemm(g, s));
        }
        {
            Timer tm(m, s, KC_RESNORM, Td * H * 4 * 4);
            HIP_TRY(launch_resnorm(tmp, ly.ln_post_attn, h, h, ly.ln_pre_ff, n, 1.0f, T, (int)H,
                                   m->eps, flag, s));
        }
        {
            GemmArgs g{n, H, ly.w_gu, H, act, m->I, (int)T, (int)(2 * m->I_pad), (int)H, EPI_GEGLU,
                       1.f, nullptr, 0, (int)m->I};
            g.cus = cus;
            Timer tm(m, s, KC_GEMM_GATE_UP, 2.0 * Td * H * 2 * m->I);
            HIP_TRY(launch_gemm(g, s));
        }
        {
            GemmArgs g{act, m->I, ly.w_down, m->I, tmp, H, (int)T, (int)H, (int)m->I, EPI_STORE,
                       1.f, nullptr, 0, 0};
            g.cus = cus;
            Timer tm(m, s, KC_GEMM_DOWN, 2.0 * Td * m->I * H);
            HIP_TRY(launch_gemm(g, s));
        }
        {
            Timer tm(m, s, KC_RESNORM, Td * H * 4 * 3);
            HIP_TRY(launch_resnorm(tmp, ly.ln_post_ff, h, h, nullptr, nullptr, 1.0f, T, (int)H,
                                   m->eps, flag, s));
        }
        {
            GemmArgs g{h, H, ly.w_pg, H, pg, P, (int)T, (int)P, (int)H, EPI_GELU_MUL, 1.f,
                       ple + l * P, L * P, 0};
            g.cus = cus;
            Timer tm(m, s, KC_GEMM_PLE_GATE, 2.0 * Td * H * P);
            HIP_TRY(launch_gemm(g, s));
        }
        {
            GemmArgs g{pg, P, ly.w_pp, P, tmp, H, (int)T, (int)H, (int)P, EPI_STORE, 1.f, nullptr,
                       0, 0};
            g.cus = cus;
            Timer tm(m, s, KC_GEMM_PLE_PROJ, 2.0 * Td * P * H);
            HIP_TRY(launch_gemm(g, s));
        }
        {
            const float *next = l + 1 < L ? m->layers[(size_t)l + 1].ln_in : m->final_norm;
            Timer tm(m, s, KC_RESNORM, Td * H * 4 * 4);
            HIP_TRY(launch_resnorm(tmp, ly.ln_post_ple, h, h, next, n, ly.scalar, T, (int)H,
                                   m->eps, flag, s));
        }
        if (h_hidden)
            HIP_TRY(hipMemcpyAsync(h_hidden + (size_t)((l + 1) * T_all * H + t0 * H), h,
                                   (size_t)(T * H) * 4, hipMemcpyDeviceToHost, s));
    }

    // Final norm (fused above), projection, pooling (text.rs:520-531).
    {
        GemmArgs g{n, H, m->out_proj, H, proj, E, (int)T, (int)E, (int)H, EPI_STORE, 1.f, nullptr,
                   0, 0};
        g.cus = cus;
        Timer tm(m, s, KC_GEMM_OUT, 2.0 * Td * H * E);
        HIP_TRY(launch_gemm(g, s));
    }
    {
        Timer tm(m, s, KC_POOL, Td * E * 4);
        HIP_TRY(launch_pool(proj, (int)E, offs, grp.nrows, d_dims, n_dims, dims_total,
                            m->pooled.p + (int64_t)grp.r0 * E,
                            m->normalized.p + (int64_t)grp.r0 * E,
                            d_trunc ? d_trunc + (int64_t)grp.r0 * dims_total : nullptr, flag, s));
    }
    return SVL_OK;
}

// Enqueues every group: group 0 on s0, group k > 0 on the model's stream k,
// which waits for everything s0 has enqueued so far and is joined back into
// s0 at the end.
svl_status enqueue_forward(svl_text_model *m, const Batch &b, hipStream_t s0,
                           const uint32_t *d_ids, const int32_t *d_featmap, const float *d_feats,
                           const int32_t *d_dims,
                           int n_dims, int dims_total, float *d_trunc, float *h_hidden) {
    const size_t ng = b.groups.size();
    if (ng > 1) {
        HIP_TRY(hipEventRecord(m->ev_fork, s0));
        for (size_t gi = 1; gi < ng; ++gi)
            HIP_TRY(hipStreamWaitEvent(m->extra[gi - 1], m->ev_fork, 0));
    }
    for (size_t gi = 0; gi < ng; ++gi)
        ST_TRY(enqueue_group(m, b, b.groups[gi], gi == 0 ? s0 : m->extra[gi - 1], d_ids,
                             d_featmap, d_feats, d_dims, n_dims, dims_total, d_trunc, h_hidden));
    for (size_t gi = 1; gi < ng; ++gi) {
        HIP_TRY(hipEventRecord(m->ev_join[gi - 1], m->extra[gi - 1]));
        HIP_TRY(hipStreamWaitEvent(s0, m->ev_join[gi - 1], 0));
    }
    return SVL_OK;
}

// Row validation in the order of text.rs:188-218 (lengths, then ids) plus
// the checked_len activation caps (text.rs:209-343, 629-639).
svl_status validate_row(const svl_text_model *m, int r, const uint32_t *ids, int64_t len) {
    if (len <= 0) return fail(SVL_CORRUPT, "row %d: cannot embed an empty token sequence", r);
    if (len > MAX_TEXT_TOKENS)
        return fail(SVL_LIMIT, "row %d: sequence has %lld tokens, above the %lld-token context", r,
                    (long long)len, (long long)MAX_TEXT_TOKENS);
    if (len > m->max_pos)
        return fail(SVL_LIMIT, "row %d: sequence has %lld tokens, above the %lld declared positions",
                    r, (long long)len, (long long)m->max_pos);
    auto chk = [&](int64_t rows, int64_t width, const char *label) -> svl_status {
        if (width != 0 && rows > INT64_MAX / width)
            return fail(SVL_LIMIT, "row %d: %s size overflow", r, label);
        if (rows * width > MAX_ACTIVATION_ELEMENTS)
            return fail(SVL_LIMIT, "row %d: %s would allocate %lld elements, above the cap", r,
                        label, (long long)(rows * width));
        return SVL_OK;
    };
    ST_TRY(chk(len, m->H, "embedding buffer"));
    ST_TRY(chk(len, m->L * m->P, "per-layer projection buffer"));
    ST_TRY(chk(len, m->I, "feed-forward buffer"));
    for (const DevLayer &ly : m->layers) {
        ST_TRY(chk(len, m->NH * ly.hd, "query buffer"));
        ST_TRY(chk(len, (int64_t)ly.nkv * ly.hd, "key/value buffer"));
    }
    if (ids)
        for (int64_t i = 0; i < len; ++i)
            if (ids[i] >= (uint64_t)m->V)
                return fail(SVL_CORRUPT,
                            "row %d: token id %u is outside the vocabulary of %lld entries", r,
                            ids[i], (long long)m->V);
    return SVL_OK;
}

svl_status finish(svl_text_model *m, hipStream_t s) {
    HIP_TRY(hipMemcpyAsync(m->h_flag, m->flag.p, sizeof(int), hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    if (m->timing) collect_timing(m);
    const int f = *m->h_flag;
    if (f & FLAG_BAD_TOKEN) return fail(SVL_CORRUPT, "a token id is outside the vocabulary");
    if (f & FLAG_NONFINITE)
        return fail(SVL_INTERNAL, "the forward pass produced a non-finite value");
    return SVL_OK;
}

svl_status check_offsets(const int64_t *offsets, int32_t batch) {
    if (batch < 0) return fail(SVL_USAGE, "negative batch");
    if (!offsets) return fail(SVL_USAGE, "offsets are null");
    if (offsets[0] != 0) return fail(SVL_USAGE, "offsets must start at 0");
    for (int r = 0; r < batch; ++r)
        if (offsets[r + 1] < offsets[r]) return fail(SVL_USAGE, "offsets must not decrease");
    return SVL_OK;
}

// One pass over rows r0 .. r1 - 1 of a checked batch (offsets rebased to the
// pass's first token).
svl_status prepare_batch(svl_text_model *m, const int64_t *offsets, int32_t r0, int32_t r1,
                         Batch &b) {
    b.B = r1 - r0;
    b.offsets.resize((size_t)b.B + 1);
    for (int32_t r = r0; r <= r1; ++r) b.offsets[(size_t)(r - r0)] = offsets[r] - offsets[r0];
    b.T = b.offsets.back();
    if (b.T > (int64_t)INT32_MAX / 8) return fail(SVL_LIMIT, "batch holds too many tokens");
    build_groups(m, b, m->row_groups);
    return SVL_OK;
}

// Every workspace buffer grows with the batch's tokens, so a batch runs in
// passes of consecutive rows whose workspace stays within PASS_BYTES (a row
// longer than a pass runs alone). Rows are independent and a row's bits do
// not depend on the rows beside it, so the outputs equal those of one pass.
constexpr int64_t PASS_BYTES = (int64_t)32 << 30;
constexpr int64_t MAX_PASS_TOKENS = (int64_t)INT32_MAX / 8;

int64_t pass_token_budget(const svl_text_model *m) {
    if (m->pass_tokens > 0) return m->pass_tokens;
    const int64_t per_token =
        4 * (3 * m->H + m->max_qkv + m->max_q + m->I + m->L * m->P + m->P + m->E + 4);
    return std::min(MAX_PASS_TOKENS, std::max(MAX_TEXT_TOKENS, PASS_BYTES / per_token));
}

std::vector<std::pair<int32_t, int32_t>> row_passes(const svl_text_model *m,
                                                    const int64_t *offsets, int32_t batch) {
    std::vector<std::pair<int32_t, int32_t>> passes;
    const int64_t cap = pass_token_budget(m);
    int32_t r0 = 0;
    for (int32_t r = 0; r < batch; ++r)
        if (r > r0 && offsets[r + 1] - offsets[r0] > cap) {
            passes.emplace_back(r0, r);
            r0 = r;
        }
    if (batch > 0) passes.emplace_back(r0, batch);
    return passes;
}

// The pass's metadata as one block: the error flag (zero), `n_dims`
// Matryoshka dims, the row offsets and the attention work items, staged in
// pinned host memory and sent by one copy on `s` (a copy or fill per array
// costs a transfer each on the stream, about 10 us apiece at one row). The
// staging is rewritten only once the copy before has left it.
svl_status upload_batch_meta(svl_text_model *m, const Batch &b, hipStream_t s,
                             const int32_t *dims = nullptr, int n_dims = 0) {
    auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
    const size_t off_dims = 256;
    const size_t off_offs = off_dims + up((size_t)n_dims * sizeof(int32_t));
    const size_t off_tiles = off_offs + up(b.dev_offsets.size() * sizeof(int64_t));
    const size_t used = off_tiles + b.tiles.size() * sizeof(AttnTile);
    HIP_TRY(m->meta.ensure(up(used)));
    if (m->ev_meta) HIP_TRY(hipEventSynchronize(m->ev_meta));
    else HIP_TRY(hipEventCreateWithFlags(&m->ev_meta, hipEventDisableTiming));
    if (m->h_meta_n < used) {
        if (m->h_meta) HIP_TRY(hipHostFree(m->h_meta));
        m->h_meta = nullptr;
        m->h_meta_n = 0;
        HIP_TRY(hipHostMalloc((void **)&m->h_meta, up(used), hipHostMallocDefault));
        m->h_meta_n = up(used);
    }
    unsigned char *h = m->h_meta, *d = m->meta.p;
    std::memset(h, 0, off_offs);
    if (n_dims > 0) std::memcpy(h + off_dims, dims, (size_t)n_dims * sizeof(int32_t));
    std::memcpy(h + off_offs, b.dev_offsets.data(), b.dev_offsets.size() * sizeof(int64_t));
    if (!b.tiles.empty())
        std::memcpy(h + off_tiles, b.tiles.data(), b.tiles.size() * sizeof(AttnTile));
    m->flag.p = (int *)d;
    m->dims.p = n_dims > 0 ? (int32_t *)(d + off_dims) : nullptr;
    m->offsets.p = (int64_t *)(d + off_offs);
    m->tiles.p = (AttnTile *)(d + off_tiles);
    HIP_TRY(hipMemcpyAsync(d, h, used, hipMemcpyHostToDevice, s));
    HIP_TRY(hipEventRecord(m->ev_meta, s));
    return SVL_OK;
}

// ---------------------------------------------------------------------------
// Kernel seam state (one flag per device, serialised).

std::mutex g_seam_mu;
std::map<int, int *> g_seam_flag;

svl_status seam_flag(int **out) {
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    auto it = g_seam_flag.find(dev);
    if (it == g_seam_flag.end()) {
        int *f = nullptr;
        HIP_TRY(hipMalloc((void **)&f, sizeof(int)));
        it = g_seam_flag.emplace(dev, f).first;
    }
    *out = it->second;
    return SVL_OK;
}

svl_status seam_finish(hipStream_t s, int *flag, const char *what) {
    int h = 0;
    HIP_TRY(hipGetLastError());
    HIP_TRY(hipMemcpyAsync(&h, flag, sizeof(int), hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    if (h & FLAG_NONFINITE) return fail(SVL_INTERNAL, "%s produced a non-finite value", what);
    return SVL_OK;
}

uint64_t splitmix64(uint64_t x) {
    uint64_t z = x + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

inline float unit(uint64_t seed, uint64_t stream, uint64_t i) {
    const uint64_t key = seed ^ (stream * 0x9E3779B97F4A7C15ull);
    return (float)(splitmix64(key + i) >> 40) * (1.0f / 16777216.0f);
}

template <class F>
void parallel_for(size_t n, F f) {
    unsigned nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    if (n < (size_t)1 << 16) nt = 1;
    std::vector<std::thread> th;
    const size_t chunk = (n + nt - 1) / nt;
    for (unsigned t = 0; t < nt; ++t) {
        const size_t a = t * chunk, b = std::min(n, a + chunk);
        if (a >= b) break;
        th.emplace_back([=] { f(a, b); });
    }
    for (auto &x : th) x.join();
}

}  // namespace

namespace svl {

int text_device(const svl_text_model *m) { return m->device; }
int64_t text_hidden_size(const svl_text_model *m) { return m->H; }
int64_t text_embedding_dim(const svl_text_model *m) { return m->E; }
int64_t text_pad_token(const svl_text_model *m) { return m->pad; }

svl_status text_forward_with_device_features(svl_text_model *m, const uint32_t *ids,
                                             const int64_t *offsets, int32_t batch,
                                             const int32_t *featmap, const float *d_feats,
                                             float *out_normalized) {
    std::lock_guard<std::mutex> lock(m->mu);
    HIP_TRY(hipSetDevice(m->device));
    ST_TRY(check_offsets(offsets, batch));
    if (batch == 0) return SVL_OK;
    for (int r = 0; r < batch; ++r)
        ST_TRY(validate_row(m, r, ids + offsets[r], offsets[r + 1] - offsets[r]));
    if (m->pad < 0)
        return fail(SVL_UNSUPPORTED, "model has no padding token for multimodal inputs");
    // featmap holds rows of d_feats, so a pass reads its tokens' entries as they are
    for (const auto &pr : row_passes(m, offsets, batch)) {
        const int64_t t0 = offsets[pr.first];
        Batch b;
        ST_TRY(prepare_batch(m, offsets, pr.first, pr.second, b));
        ST_TRY(ensure_workspace(m, b, 0, true, 0));
        hipStream_t s = m->stream;
        HIP_TRY(hipMemcpyAsync(m->ids.p, ids + t0, (size_t)b.T * 4, hipMemcpyHostToDevice, s));
        HIP_TRY(hipMemcpyAsync(m->featmap.p, featmap + t0, (size_t)b.T * 4,
                               hipMemcpyHostToDevice, s));
        ST_TRY(upload_batch_meta(m, b, s));
        ST_TRY(enqueue_forward(m, b, s, m->ids.p, m->featmap.p, d_feats, nullptr, 0, 0, nullptr,
                               nullptr));
        HIP_TRY(hipMemcpyAsync(out_normalized + (size_t)pr.first * m->E, m->normalized.p,
                               (size_t)(b.B * m->E) * 4, hipMemcpyDeviceToHost, s));
        ST_TRY(finish(m, s));
    }
    return SVL_OK;
}

}  // namespace svl

// ===========================================================================
// C ABI
// ===========================================================================

extern "C" {

svl_status svl_init(int device_ordinal, svl_ctx **out) {
    if (!out) return fail(SVL_USAGE, "output pointer is null");
    int count = 0;
    HIP_TRY(hipGetDeviceCount(&count));
    if (device_ordinal < 0 || device_ordinal >= count)
        return fail(SVL_USAGE, "device %d is outside the %d visible devices", device_ordinal,
                    count);
    hipDeviceProp_t prop;
    HIP_TRY(hipGetDeviceProperties(&prop, device_ordinal));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(SVL_UNSUPPORTED, "device %d is %s; this library is built for gfx950",
                    device_ordinal, prop.gcnArchName);
    HIP_TRY(hipSetDevice(device_ordinal));
    void *scratch = nullptr;  // the allocation-free entry points' device scratch
    HIP_TRY(noalloc_scratch(device_ordinal, &scratch));
    *out = new svl_ctx{device_ordinal};
    return SVL_OK;
}

svl_status svl_shutdown(svl_ctx *ctx) {
    delete ctx;
    return SVL_OK;
}

const char *svl_last_error(void) { return g_err.c_str(); }

svl_status svl_text_model_create(svl_ctx *ctx, const svl_text_config *cfg,
                                 const svl_tensor_view *tensors, size_t n_tensors,
                                 svl_text_model **out) {
    if (!ctx || !out) return fail(SVL_USAGE, "context or output pointer is null");
    ST_TRY(validate_config(cfg));
    HIP_TRY(hipSetDevice(ctx->device));

    // Inventory (weights.rs:130-165).
    const auto shapes = tensor_shapes(cfg);
    TensorIndex by_name;
    ST_TRY(check_inventory(tensors, n_tensors, shapes, {"language_model."}, "text",
                           MAX_WEIGHT_ELEMENTS, by_name));

    auto m = new svl_text_model();
    std::unique_ptr<svl_text_model> guard(m);
    m->device = ctx->device;
    m->V = cfg->vocab_size;
    m->H = cfg->hidden_size;
    m->I = cfg->intermediate_size;
    m->L = cfg->num_hidden_layers;
    m->NH = cfg->num_attention_heads;
    m->P = cfg->hidden_size_per_layer_input;
    m->E = cfg->embedding_dim;
    m->max_pos = cfg->max_position_embeddings;
    m->window = cfg->sliding_window;
    m->pad = cfg->pad_token_id;
    m->eps = (float)cfg->rms_norm_eps;
    m->full_theta = (float)cfg->full_rope_theta;
    m->slide_theta = (float)cfg->sliding_rope_theta;
    // config.rs:241-242
    m->embedding_scale = std::sqrt((float)m->H);
    m->ple_scale = 1.0f / m->embedding_scale;
    m->I_pad = (m->I + 31) / 32 * 32;
    if (m->H % 4 || m->H > 2048)
        return fail(SVL_UNSUPPORTED, "hidden size %lld is not a multiple of 4 up to 2048",
                    (long long)m->H);
    if (m->E > 4096) return fail(SVL_UNSUPPORTED, "embedding dimension above 4096");

    auto get = [&](const std::string &name, std::vector<float> &buf) -> svl_status {
        return decode_named(by_name, name, buf);
    };
    std::vector<float> a, b2, c2;
    ST_TRY(get("language_model.embed_tokens.weight", a));
    ST_TRY(upload(m, a.data(), a.size(), &m->embed));
    ST_TRY(get("language_model.embedding_projection.weight", a));
    ST_TRY(upload(m, a.data(), a.size(), &m->out_proj));
    ST_TRY(get("language_model.norm.weight", a));
    ST_TRY(upload(m, a.data(), a.size(), &m->final_norm));
    ST_TRY(get("language_model.ple.per_layer_model_projection.weight", a));
    ST_TRY(upload(m, a.data(), a.size(), &m->ple_model));
    ST_TRY(get("language_model.ple.per_layer_projection_norm.weight", a));
    ST_TRY(upload(m, a.data(), a.size(), &m->ple_norm));

    m->layers.resize((size_t)m->L);
    for (int64_t l = 0; l < m->L; ++l) {
        DevLayer &ly = m->layers[(size_t)l];
        const std::string p = "language_model.layers." + std::to_string(l) + ".";
        ly.hd = (int)cfg->head_dim[l];
        ly.nkv = (int)cfg->num_kv_heads[l];
        ly.full = cfg->layer_type[l];
        m->type_hd[ly.full] = ly.hd;
        const int64_t H = m->H, qd = m->NH * ly.hd, kd = (int64_t)ly.nkv * ly.hd;
        // fused QKV weight: rows [q; k; v]
        std::vector<float> qkv((size_t)((qd + 2 * kd) * H));
        ST_TRY(get(p + "self_attn.q_proj.weight", a));
        std::copy(a.begin(), a.end(), qkv.begin());
        ST_TRY(get(p + "self_attn.k_proj.weight", a));
        std::copy(a.begin(), a.end(), qkv.begin() + qd * H);
        ST_TRY(get(p + "self_attn.v_proj.weight", a));
        std::copy(a.begin(), a.end(), qkv.begin() + (qd + kd) * H);
        ST_TRY(upload(m, qkv.data(), qkv.size(), &ly.w_qkv));
        ST_TRY(get(p + "self_attn.o_proj.weight", a));
        ST_TRY(upload(m, a.data(), a.size(), &ly.w_o));
        ST_TRY(get(p + "mlp.gate_proj.weight", b2));
        ST_TRY(get(p + "mlp.up_proj.weight", c2));
        const std::vector<float> gu = interleave_gate_up(b2, c2, m->I, m->I_pad, m->H);
        ST_TRY(upload(m, gu.data(), gu.size(), &ly.w_gu));
        ST_TRY(get(p + "mlp.down_proj.weight", a));
        ST_TRY(upload(m, a.data(), a.size(), &ly.w_down));
        ST_TRY(get(p + "ple_block.per_layer_input_gate.weight", a));
        ST_TRY(upload(m, a.data(), a.size(), &ly.w_pg));
        ST_TRY(get(p + "ple_block.per_layer_projection.weight", a));
        ST_TRY(upload(m, a.data(), a.size(), &ly.w_pp));
        struct {
            const char *name;
            float **dst;
        } norms[] = {{"input_layernorm.weight", &ly.ln_in},
                     {"post_attention_layernorm.weight", &ly.ln_post_attn},
                     {"pre_feedforward_layernorm.weight", &ly.ln_pre_ff},
                     {"post_feedforward_layernorm.weight", &ly.ln_post_ff},
                     {"ple_block.post_per_layer_input_norm.weight", &ly.ln_post_ple},
                     {"self_attn.q_norm.weight", &ly.q_norm},
                     {"self_attn.k_norm.weight", &ly.k_norm}};
        for (auto &nm : norms) {
            ST_TRY(get(p + nm.name, a));
            ST_TRY(upload(m, a.data(), a.size(), nm.dst));
        }
        ST_TRY(get(p + "layer_scalar", a));
        ly.scalar = a[0];
    }

    // RoPE tables for every position a row may use.
    m->rope_positions = std::min<int64_t>(m->max_pos, MAX_TEXT_TOKENS);
    const float thetas[2] = {m->slide_theta, m->full_theta};
    for (int t = 0; t < 2; ++t) {
        if (!m->type_hd[t]) continue;
        std::vector<float> cs, sn;
        rope_tables(m->type_hd[t], thetas[t], m->rope_positions, 0, cs, sn);
        HIP_TRY(hipMalloc((void **)&m->cos_t[t], cs.size() * 4));
        HIP_TRY(hipMalloc((void **)&m->sin_t[t], sn.size() * 4));
        HIP_TRY(hipMemcpy(m->cos_t[t], cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
        HIP_TRY(hipMemcpy(m->sin_t[t], sn.data(), sn.size() * 4, hipMemcpyHostToDevice));
    }
    for (const DevLayer &ly : m->layers) {
        m->max_qkv = std::max<int64_t>(m->max_qkv, m->NH * ly.hd + 2 * (int64_t)ly.nkv * ly.hd);
        m->max_q = std::max<int64_t>(m->max_q, m->NH * ly.hd);
    }
    HIP_TRY(hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking));
    HIP_TRY(hipEventCreateWithFlags(&m->ev_fork, hipEventDisableTiming));
    for (int i = 0; i < svl_text_model::MAX_GROUPS - 1; ++i) {
        HIP_TRY(hipStreamCreateWithFlags(&m->extra[i], hipStreamNonBlocking));
        HIP_TRY(hipEventCreateWithFlags(&m->ev_join[i], hipEventDisableTiming));
    }
    HIP_TRY(hipHostMalloc((void **)&m->h_flag, sizeof(int), hipHostMallocDefault));
    *out = guard.release();
    return SVL_OK;
}

svl_status svl_text_model_destroy(svl_text_model *model) {
    delete model;
    return SVL_OK;
}

svl_status svl_text_forward_batch(svl_text_model *m, const uint32_t *ids, const int64_t *offsets,
                                  int32_t batch, const svl_feature_span *features,
                                  float *out_normalized, float *out_pooled, float *out_projected,
                                  float *out_hidden) {
    if (!m || !ids || !offsets || !out_normalized)
        return fail(SVL_USAGE, "model, ids, offsets and out_normalized are required");
    std::lock_guard<std::mutex> lock(m->mu);
    HIP_TRY(hipSetDevice(m->device));
    ST_TRY(check_offsets(offsets, batch));
    if (batch == 0) return SVL_OK;
    for (int r = 0; r < batch; ++r)
        ST_TRY(validate_row(m, r, ids + offsets[r], offsets[r + 1] - offsets[r]));

    // Multimodal feature spans (text.rs:226-275), every row checked before
    // any pass runs.
    if (features) {
        for (int r = 0; r < batch; ++r) {
            const svl_feature_span &f = features[r];
            if (!f.data) continue;
            const int64_t len = offsets[r + 1] - offsets[r];
            if (f.count <= 0)
                return fail(SVL_CORRUPT,
                            "row %d: multimodal feature replacement requires at least one token", r);
            if (f.start < 0 || f.start > INT64_MAX - f.count)
                return fail(SVL_LIMIT, "row %d: multimodal feature range overflow", r);
            if (f.start + f.count > len)
                return fail(SVL_CORRUPT, "row %d: multimodal feature range is outside the sequence",
                            r);
            if (f.len != f.count * m->H)
                return fail(SVL_CORRUPT, "row %d: multimodal features have %lld values, expected %lld",
                            r, (long long)f.len, (long long)(f.count * m->H));
            if (m->pad < 0)
                return fail(SVL_UNSUPPORTED, "model has no padding token for multimodal inputs");
        }
    }

    const int64_t T_all = offsets[batch];
    for (const auto &pr : row_passes(m, offsets, batch)) {
        const int32_t r0 = pr.first, r1 = pr.second;
        const int64_t t0 = offsets[r0];
        Batch b;
        ST_TRY(prepare_batch(m, offsets, r0, r1, b));
        b.hidden_stride = T_all;
        // per token of the pass: its row of the pass's feature values, or -1
        int64_t feat_floats = 0;
        std::vector<int32_t> featmap;
        if (features) {
            featmap.assign((size_t)b.T, -1);
            for (int r = r0; r < r1; ++r) {
                const svl_feature_span &f = features[r];
                if (!f.data) continue;
                for (int64_t i = 0; i < f.count; ++i)
                    featmap[(size_t)(offsets[r] - t0 + f.start + i)] =
                        (int32_t)(feat_floats / m->H + i);
                feat_floats += f.len;
            }
            if (feat_floats == 0) featmap.clear();
        }
        ST_TRY(ensure_workspace(m, b, feat_floats, feat_floats > 0, 0));
        hipStream_t s = m->stream;
        HIP_TRY(hipMemcpyAsync(m->ids.p, ids + t0, (size_t)b.T * 4, hipMemcpyHostToDevice, s));
        if (feat_floats > 0) {
            HIP_TRY(hipMemcpyAsync(m->featmap.p, featmap.data(), featmap.size() * 4,
                                   hipMemcpyHostToDevice, s));
            int64_t off = 0;
            for (int r = r0; r < r1; ++r) {
                const svl_feature_span &f = features[r];
                if (!f.data) continue;
                HIP_TRY(hipMemcpyAsync(m->feats.p + off, f.data, (size_t)f.len * 4,
                                       hipMemcpyHostToDevice, s));
                off += f.len;
            }
        }
        ST_TRY(upload_batch_meta(m, b, s));
        ST_TRY(enqueue_forward(m, b, s, m->ids.p, feat_floats > 0 ? m->featmap.p : nullptr,
                               feat_floats > 0 ? m->feats.p : nullptr, nullptr, 0, 0, nullptr,
                               out_hidden ? out_hidden + (size_t)t0 * m->H : nullptr));
        HIP_TRY(hipMemcpyAsync(out_normalized + (size_t)r0 * m->E, m->normalized.p,
                               (size_t)(b.B * m->E) * 4, hipMemcpyDeviceToHost, s));
        if (out_pooled)
            HIP_TRY(hipMemcpyAsync(out_pooled + (size_t)r0 * m->E, m->pooled.p,
                                   (size_t)(b.B * m->E) * 4, hipMemcpyDeviceToHost, s));
        if (out_projected)
            HIP_TRY(hipMemcpyAsync(out_projected + (size_t)t0 * m->E, m->proj.p,
                                   (size_t)(b.T * m->E) * 4, hipMemcpyDeviceToHost, s));
        ST_TRY(finish(m, s));
    }
    return SVL_OK;
}

svl_status svl_text_forward_device(svl_text_model *m, const uint32_t *d_ids,
                                   const int64_t *offsets, int32_t batch, const int32_t *dims,
                                   int32_t n_dims, float *d_out, void *stream) {
    if (!m || !d_ids || !offsets || !dims || n_dims <= 0 || !d_out)
        return fail(SVL_USAGE, "model, ids, offsets, dims and output are required");
    std::lock_guard<std::mutex> lock(m->mu);
    HIP_TRY(hipSetDevice(m->device));
    int dims_total = 0;
    for (int i = 0; i < n_dims; ++i) {
        if (dims[i] <= 0 || dims[i] > m->E)
            return fail(SVL_INTERNAL, "embedding dimension %d is outside 1..=%lld", dims[i],
                        (long long)m->E);
        dims_total += dims[i];
    }
    ST_TRY(check_offsets(offsets, batch));
    if (batch == 0) return SVL_OK;
    for (int r = 0; r < batch; ++r)
        ST_TRY(validate_row(m, r, nullptr, offsets[r + 1] - offsets[r]));
    hipStream_t s = stream ? (hipStream_t)stream : m->stream;
    for (const auto &pr : row_passes(m, offsets, batch)) {
        Batch b;
        ST_TRY(prepare_batch(m, offsets, pr.first, pr.second, b));
        ST_TRY(ensure_workspace(m, b, 0, false, dims_total));
        ST_TRY(upload_batch_meta(m, b, s, dims, n_dims));
        ST_TRY(enqueue_forward(m, b, s, d_ids + offsets[pr.first], nullptr, nullptr, m->dims.p,
                               n_dims, dims_total, d_out + (size_t)pr.first * dims_total,
                               nullptr));
        ST_TRY(finish(m, s));
    }
    return SVL_OK;
}

svl_status svl_truncate_and_normalize(const float *values, size_t n, size_t dimension,
                                      float *out) {
    // kernels.rs:916-927 then l2_normalize_scalar (kernels.rs:424-444).
    if (dimension == 0) return fail(SVL_INTERNAL, "embedding dimension must be positive");
    if (dimension > n)
        return fail(SVL_INTERNAL, "cannot truncate %zu elements to %zu", n, dimension);
    float sum = 0.f;
    for (size_t i = 0; i < dimension; ++i) {
        if (!std::isfinite(values[i]))
            return fail(SVL_INTERNAL, "L2 normalization input contains a non-finite value");
        sum += values[i] * values[i];
    }
    if (!std::isfinite(sum) || sum <= 0.f)
        return fail(SVL_INTERNAL, "cannot normalize a zero or non-finite vector");
    const float inv = 1.0f / std::sqrt(sum);
    for (size_t i = 0; i < dimension; ++i) out[i] = values[i] * inv;
    return SVL_OK;
}

svl_status svl_tensor_to_f32(const svl_tensor_view *t, float *out, int64_t capacity) {
    // TensorEntry::to_f32 (safetensors.rs:69-110): element cap, then F32
    // little-endian or BF16 widened exactly (bf16.rs:13-15).
    if (!t) return fail(SVL_USAGE, "tensor view is null");
    if (t->ndim < 0 || t->ndim > 8) return fail(SVL_CORRUPT, "tensor %s has rank %d", t->name, t->ndim);
    int64_t numel = 1;
    for (int d = 0; d < t->ndim; ++d) {
        if (t->shape[d] < 0) return fail(SVL_CORRUPT, "tensor %s has a negative dimension", t->name);
        if (t->shape[d] && numel > MAX_TENSOR_ELEMENTS / t->shape[d])
            return fail(SVL_LIMIT, "tensor %s has more elements than the cap", t->name);
        numel *= t->shape[d];
    }
    if (numel > MAX_TENSOR_ELEMENTS)
        return fail(SVL_LIMIT, "tensor %s has %lld elements, above the cap", t->name, (long long)numel);
    if (numel > capacity)
        return fail(SVL_USAGE, "tensor %s has %lld elements, the output holds %lld", t->name,
                    (long long)numel, (long long)capacity);
    if (numel == 0) return widen_f32(*t, 0, out);
    if (!t->data || !out) return fail(SVL_USAGE, "tensor %s has no data", t->name);
    return widen_f32(*t, numel, out);
}

svl_status svl_measure_peaks(svl_ctx *ctx, double *fp32_mfma_tflops, double *hbm_copy_gbs) {
    if (!ctx || !fp32_mfma_tflops || !hbm_copy_gbs) return fail(SVL_USAGE, "null argument");
    HIP_TRY(hipSetDevice(ctx->device));
    const hipError_t e = probe_peaks(fp32_mfma_tflops, hbm_copy_gbs);
    if (e != hipSuccess) return fail(SVL_DEVICE, "peak probe: %s", hipGetErrorString(e));
    return SVL_OK;
}

svl_status svl_measure_fp64_peak(svl_ctx *ctx, double *fp64_mfma_tflops) {
    if (!ctx || !fp64_mfma_tflops) return fail(SVL_USAGE, "null argument");
    HIP_TRY(hipSetDevice(ctx->device));
    const hipError_t e = probe_fp64_peak(fp64_mfma_tflops);
    if (e != hipSuccess) return fail(SVL_DEVICE, "FP64 peak probe: %s", hipGetErrorString(e));
    return SVL_OK;
}

svl_status svl_text_embed_ids(svl_text_model *m, const uint32_t *ids, int64_t n,
                              int64_t dimension, float *out) {
    if (!m || !out) return fail(SVL_USAGE, "model and output are required");
    if (dimension <= 0 || dimension > m->E)
        return fail(SVL_INTERNAL, "embedding dimension %lld is outside 1..=%lld",
                    (long long)dimension, (long long)m->E);
    std::vector<float> normalized((size_t)m->E);
    const int64_t offs[2] = {0, n};
    static const uint32_t empty_ids[1] = {0};
    ST_TRY(svl_text_forward_batch(m, ids ? ids : empty_ids, offs, 1, nullptr, normalized.data(),
                                  nullptr, nullptr, nullptr));
    return svl_truncate_and_normalize(normalized.data(), (size_t)m->E, (size_t)dimension, out);
}

svl_status svl_text_model_set_stream_split(svl_text_model *m, int enable) {
    if (!m) return fail(SVL_USAGE, "model is null");
    std::lock_guard<std::mutex> lock(m->mu);
    m->row_groups = std::max(1, std::min(enable, svl_text_model::MAX_GROUPS));
    return SVL_OK;
}

svl_status svl_text_model_set_pass_tokens(svl_text_model *m, int64_t tokens) {
    if (!m) return fail(SVL_USAGE, "model is null");
    if (tokens < 0 || tokens > MAX_PASS_TOKENS)
        return fail(SVL_USAGE, "pass size %lld is outside 0..=%lld tokens", (long long)tokens,
                    (long long)MAX_PASS_TOKENS);
    std::lock_guard<std::mutex> lock(m->mu);
    m->pass_tokens = tokens;
    return SVL_OK;
}

svl_status svl_text_model_set_kernel_timing(svl_text_model *m, int enable) {
    if (!m) return fail(SVL_USAGE, "model is null");
    std::lock_guard<std::mutex> lock(m->mu);
    m->timing = enable != 0;
    for (int c = 0; c < KC_COUNT; ++c) {
        m->stat_ms[c] = 0;
        m->stat_launches[c] = 0;
        m->stat_work[c] = 0;
    }
    return SVL_OK;
}

int32_t svl_kernel_class_count(void) { return KC_COUNT; }

const char *svl_kernel_class_name(int32_t cls) {
    return cls >= 0 && cls < KC_COUNT ? kClassNames[cls] : "";
}

svl_status svl_text_model_kernel_stats(svl_text_model *m, double *ms, int64_t *launches,
                                       double *work) {
    if (!m) return fail(SVL_USAGE, "model is null");
    std::lock_guard<std::mutex> lock(m->mu);
    for (int c = 0; c < KC_COUNT; ++c) {
        if (ms) ms[c] = m->stat_ms[c];
        if (launches) launches[c] = m->stat_launches[c];
        if (work) work[c] = m->stat_work[c];
    }
    return SVL_OK;
}

// ---- kernel seam ------------------------------------------------------------

svl_status svl_linear(const float *d_in, const float *d_w, int64_t rows, int64_t in_features,
                      int64_t out_features, float *d_out, void *stream) {
    if (rows < 0 || in_features < 0 || out_features < 0)
        return fail(SVL_INTERNAL, "linear shape is negative");
    if (rows * out_features > MAX_TENSOR_ELEMENTS)
        return fail(SVL_LIMIT, "linear would allocate %lld elements, above the cap",
                    (long long)(rows * out_features));
    if (rows > INT32_MAX || in_features > INT32_MAX || out_features > INT32_MAX)
        return fail(SVL_LIMIT, "linear dimension above 2^31");
    std::lock_guard<std::mutex> lock(g_seam_mu);
    int *flag;
    ST_TRY(seam_flag(&flag));
    hipStream_t s = (hipStream_t)stream;
    HIP_TRY(hipMemsetAsync(flag, 0, sizeof(int), s));
    GemmArgs g{d_in, in_features, d_w, in_features, d_out, out_features, (int)rows,
               (int)out_features, (int)in_features, EPI_STORE, 1.f, nullptr, 0, 0};
    if (in_features == 0) {
        HIP_TRY(hipMemsetAsync(d_out, 0, (size_t)(rows * out_features) * 4, s));
    } else {
        HIP_TRY(launch_gemm(g, s));
    }
    HIP_TRY(launch_finite_check(d_out, rows * out_features, flag, s));
    return seam_finish(s, flag, "linear projection");
}

svl_status svl_rms_norm_rows(const float *d_in, const float *d_weight, int64_t rows,
                             int64_t width, float eps, float *d_out, void *stream) {
    if (width <= 0) return fail(SVL_INTERNAL, "RMSNorm row width must be positive");
    if (!std::isfinite(eps) || eps < 0)
        return fail(SVL_INTERNAL, "RMSNorm epsilon must be finite and non-negative");
    if (rows < 0 || rows * width > MAX_TENSOR_ELEMENTS)
        return fail(SVL_LIMIT, "RMSNorm would allocate above the cap");
    std::lock_guard<std::mutex> lock(g_seam_mu);
    int *flag;
    ST_TRY(seam_flag(&flag));
    hipStream_t s = (hipStream_t)stream;
    HIP_TRY(hipMemsetAsync(flag, 0, sizeof(int), s));
    HIP_TRY(launch_rms_rows(d_in, d_weight, d_out, rows, (int)width, eps, flag, s));
    return seam_finish(s, flag, "RMSNorm");
}

svl_status svl_rope_inv_freq(int64_t head_dim, float base, float *out) {
    if (head_dim <= 0 || head_dim % 2)
        return fail(SVL_INTERNAL, "RoPE head dimension must be a positive even number");
    if (!std::isfinite(base) || base <= 1.0f)
        return fail(SVL_INTERNAL, "RoPE base must be finite and greater than one");
    for (int64_t j = 0; j < head_dim / 2; ++j) {
        const float exponent = (float)(2 * j) / (float)head_dim;
        out[j] = 1.0f / std::pow(base, exponent);
    }
    return SVL_OK;
}

svl_status svl_rope_with_inv_freq(float *d_values, int64_t seq_len, int64_t num_heads,
                                  int64_t head_dim, const float *inv_freq, int64_t n_inv_freq,
                                  int64_t position_offset, void *stream) {
    if (head_dim <= 0 || head_dim % 2)
        return fail(SVL_INTERNAL, "RoPE head dimension must be a positive even number");
    if (n_inv_freq != head_dim / 2)
        return fail(SVL_INTERNAL, "RoPE expects %lld inverse frequencies for head_dim %lld, got %lld",
                    (long long)(head_dim / 2), (long long)head_dim, (long long)n_inv_freq);
    if (seq_len < 0 || num_heads < 0 || position_offset < 0)
        return fail(SVL_INTERNAL, "RoPE shape is negative");
    if (seq_len == 0 || num_heads == 0) return SVL_OK;
    const int half = (int)(head_dim / 2);
    std::vector<float> c((size_t)(seq_len * half)), sn((size_t)(seq_len * half));
    for (int64_t p = 0; p < seq_len; ++p)
        for (int j = 0; j < half; ++j) {
            const float angle = (float)(position_offset + p) * inv_freq[j];
            c[(size_t)(p * half + j)] = std::cos(angle);
            sn[(size_t)(p * half + j)] = std::sin(angle);
        }
    std::lock_guard<std::mutex> lock(g_seam_mu);
    int *flag;
    ST_TRY(seam_flag(&flag));
    hipStream_t s = (hipStream_t)stream;
    float *dc = nullptr, *ds = nullptr;
    HIP_TRY(hipMalloc((void **)&dc, c.size() * 4));
    HIP_TRY(hipMalloc((void **)&ds, sn.size() * 4));
    svl_status st = SVL_OK;
    if (hipMemcpyAsync(dc, c.data(), c.size() * 4, hipMemcpyHostToDevice, s) != hipSuccess ||
        hipMemcpyAsync(ds, sn.data(), sn.size() * 4, hipMemcpyHostToDevice, s) != hipSuccess ||
        hipMemsetAsync(flag, 0, sizeof(int), s) != hipSuccess ||
        launch_rope(d_values, seq_len, (int)num_heads, (int)head_dim, dc, ds, flag, s) !=
            hipSuccess)
        st = fail(SVL_DEVICE, "RoPE launch failed");
    if (st == SVL_OK) st = seam_finish(s, flag, "RoPE");
    (void)hipStreamSynchronize(s);
    (void)hipFree(dc);
    (void)hipFree(ds);
    return st;
}

static svl_status check_attention_shape(int64_t seq_len, int64_t num_heads, int64_t num_kv_heads,
                                        int64_t head_dim, float scale) {
    if (head_dim <= 0) return fail(SVL_INTERNAL, "attention head dimension must be positive");
    if (num_heads <= 0 || num_kv_heads <= 0)
        return fail(SVL_INTERNAL, "attention head counts must be positive");
    if (num_heads % num_kv_heads)
        return fail(SVL_INTERNAL,
                    "attention head count is not a multiple of the key/value head count");
    if (!std::isfinite(scale)) return fail(SVL_INTERNAL, "attention scale must be finite");
    if (seq_len < 0 || seq_len * num_heads * head_dim > MAX_TENSOR_ELEMENTS)
        return fail(SVL_LIMIT, "attention would allocate above the cap");
    if (seq_len > 8192 && attn_block_vectors((int)head_dim) == 0)
        return fail(SVL_UNSUPPORTED, "sequence above 8192 keys for head_dim %lld",
                    (long long)head_dim);
    return SVL_OK;
}

// One row of seq_len keys, q/k/v/out packed [seq, heads, head_dim].
static AttnArgs seam_attention_args(const float *d_q, const float *d_k, const float *d_v,
                                    int64_t seq_len, int64_t num_heads, int64_t num_kv_heads,
                                    int64_t head_dim, int64_t sliding_window, float scale,
                                    float *d_out) {
    AttnArgs a{};
    a.q = d_q;
    a.k = d_k;
    a.v = d_v;
    a.out = d_out;
    a.ldq = num_heads * head_dim;
    a.ldk = a.ldv = num_kv_heads * head_dim;
    a.ldo = num_heads * head_dim;
    a.nh = (int)num_heads;
    a.nkv = (int)num_kv_heads;
    a.hd = (int)head_dim;
    a.window = sliding_window < 0 ? -1 : (int)std::min<int64_t>(sliding_window, INT32_MAX);
    a.scale = scale;
    a.tokens = seq_len;
    a.max_len = seq_len;
    a.shortest = seq_len;
    return a;
}

svl_status svl_bidirectional_attention(const float *d_q, const float *d_k, const float *d_v,
                                       int64_t seq_len, int64_t num_heads, int64_t num_kv_heads,
                                       int64_t head_dim, int64_t sliding_window, float scale,
                                       float *d_out, void *stream) {
    ST_TRY(check_attention_shape(seq_len, num_heads, num_kv_heads, head_dim, scale));
    if (seq_len == 0) return SVL_OK;
    const int bv = attn_block_vectors((int)head_dim);
    const int G = (int)(num_heads / num_kv_heads);
    std::vector<AttnTile> tiles;
    if (bv > 0)
        for (int g = 0; g < num_kv_heads; ++g)
            for (int64_t v0 = 0; v0 < seq_len * G; v0 += bv)
                tiles.push_back({0, (int32_t)seq_len, g, (int32_t)v0});
    std::vector<int32_t> pos((size_t)seq_len), rl((size_t)seq_len, (int32_t)seq_len);
    for (int64_t i = 0; i < seq_len; ++i) pos[(size_t)i] = (int32_t)i;
    std::lock_guard<std::mutex> lock(g_seam_mu);
    int *flag;
    ST_TRY(seam_flag(&flag));
    hipStream_t s = (hipStream_t)stream;
    AttnTile *dt = nullptr;
    int32_t *dp = nullptr, *dl = nullptr;
    HIP_TRY(hipMalloc((void **)&dt, std::max<size_t>(tiles.size(), 1) * sizeof(AttnTile)));
    HIP_TRY(hipMalloc((void **)&dp, pos.size() * 4));
    HIP_TRY(hipMalloc((void **)&dl, rl.size() * 4));
    AttnArgs a = seam_attention_args(d_q, d_k, d_v, seq_len, num_heads, num_kv_heads, head_dim,
                                     sliding_window, scale, d_out);
    a.tiles = dt;
    a.n_tiles = (int)tiles.size();
    a.pos = dp;
    a.rowlen = dl;
    a.flag = flag;
    svl_status st = SVL_OK;
    if ((!tiles.empty() && hipMemcpyAsync(dt, tiles.data(), tiles.size() * sizeof(AttnTile),
                                          hipMemcpyHostToDevice, s) != hipSuccess) ||
        hipMemcpyAsync(dp, pos.data(), pos.size() * 4, hipMemcpyHostToDevice, s) != hipSuccess ||
        hipMemcpyAsync(dl, rl.data(), rl.size() * 4, hipMemcpyHostToDevice, s) != hipSuccess ||
        hipMemsetAsync(flag, 0, sizeof(int), s) != hipSuccess ||
        launch_attention(a, s) != hipSuccess)
        st = fail(SVL_DEVICE, "attention launch failed");
    if (st == SVL_OK) st = seam_finish(s, flag, "attention");
    (void)hipStreamSynchronize(s);
    (void)hipFree(dt);
    (void)hipFree(dp);
    (void)hipFree(dl);
    return st;
}

std::mutex g_noalloc_mu;

svl_status svl_bidirectional_attention_noalloc(const float *d_q, const float *d_k,
                                               const float *d_v, int64_t seq_len,
                                               int64_t num_heads, int64_t num_kv_heads,
                                               int64_t head_dim, int64_t sliding_window,
                                               float scale, float *d_out, void *stream) {
    ST_TRY(check_attention_shape(seq_len, num_heads, num_kv_heads, head_dim, scale));
    if (seq_len == 0) return SVL_OK;
    if (seq_len > NOALLOC_MAX_KEYS)
        return fail(SVL_LIMIT, "%lld keys: the allocation-free attention takes at most %d",
                    (long long)seq_len, NOALLOC_MAX_KEYS);
    const int bv = attn_block_vectors((int)head_dim);
    const int64_t G = num_heads / num_kv_heads;
    const int64_t per_head = bv > 0 ? (seq_len * G + bv - 1) / bv : 0;
    if (per_head * num_kv_heads > NOALLOC_MAX_TILES)
        return fail(SVL_LIMIT, "%lld attention work items: the allocation-free attention takes "
                    "at most %d", (long long)(per_head * num_kv_heads), NOALLOC_MAX_TILES);
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    void *base = nullptr;
    HIP_TRY(noalloc_scratch(dev, &base));
    char *b = (char *)base;
    AttnArgs a = seam_attention_args(d_q, d_k, d_v, seq_len, num_heads, num_kv_heads, head_dim,
                                     sliding_window, scale, d_out);
    a.tiles = (const AttnTile *)(b + NOALLOC_TILES_OFF);
    a.n_tiles = (int)(per_head * num_kv_heads);
    a.pos = (const int32_t *)(b + NOALLOC_POS_OFF);
    a.rowlen = (const int32_t *)(b + NOALLOC_LEN_OFF);
    a.flag = (int *)(b + NOALLOC_FLAG_OFF);
    hipStream_t s = (hipStream_t)stream;
    // one call at a time per process: every call on a GPU shares its scratch
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    HIP_TRY(launch_noalloc_attn_setup(base, (int)seq_len, (int)per_head, bv, a.n_tiles, s));
    if (launch_attention(a, s) != hipSuccess) return fail(SVL_DEVICE, "attention launch failed");
    return seam_finish(s, a.flag, "attention");
}

svl_status svl_set_attention_path(int path) {
    if (path != ATTN_PATH_AUTO && path != ATTN_PATH_FALLBACK && path != ATTN_PATH_GENERIC)
        return fail(SVL_USAGE, "attention path %d is not 0, 1 or 2", path);
    set_attention_path(path);
    return SVL_OK;
}

static svl_status seam_elementwise(const char *what, int kind, const float *a, const float *b,
                                   int64_t n, float *out, void *stream) {
    if (n < 0 || n > MAX_TENSOR_ELEMENTS) return fail(SVL_LIMIT, "%s above the cap", what);
    std::lock_guard<std::mutex> lock(g_seam_mu);
    hipStream_t s = (hipStream_t)stream;
    hipError_t e = kind == 0 ? launch_gelu(a, out, n, s)
                             : (kind == 1 ? launch_geglu(a, b, out, n, s) : launch_add(a, b, out, n, s));
    if (e != hipSuccess) return fail(SVL_DEVICE, "%s launch: %s", what, hipGetErrorString(e));
    HIP_TRY(hipStreamSynchronize(s));
    return SVL_OK;
}

svl_status svl_gelu_tanh(const float *d_in, int64_t n, float *d_out, void *stream) {
    return seam_elementwise("gelu_tanh", 0, d_in, nullptr, n, d_out, stream);
}
svl_status svl_geglu(const float *d_gate, const float *d_up, int64_t n, float *d_out,
                     void *stream) {
    return seam_elementwise("geglu", 1, d_gate, d_up, n, d_out, stream);
}
svl_status svl_add(const float *d_a, const float *d_b, int64_t n, float *d_out, void *stream) {
    return seam_elementwise("add", 2, d_a, d_b, n, d_out, stream);
}

svl_status svl_mean_pool(const float *d_values, int64_t rows, int64_t width, float *d_out,
                         void *stream) {
    if (rows <= 0) return fail(SVL_INTERNAL, "mean pooling of an empty sequence");
    if (width <= 0 || width > 4096) return fail(SVL_UNSUPPORTED, "pool width outside 1..=4096");
    std::lock_guard<std::mutex> lock(g_seam_mu);
    int *flag;
    ST_TRY(seam_flag(&flag));
    hipStream_t s = (hipStream_t)stream;
    int64_t *doff = nullptr;
    const int64_t offs[2] = {0, rows};
    HIP_TRY(hipMalloc((void **)&doff, sizeof offs));
    svl_status st = SVL_OK;
    if (hipMemcpyAsync(doff, offs, sizeof offs, hipMemcpyHostToDevice, s) != hipSuccess ||
        hipMemsetAsync(flag, 0, sizeof(int), s) != hipSuccess ||
        launch_pool(d_values, (int)width, doff, 1, nullptr, 0, 0, d_out, nullptr, nullptr, nullptr,
                    s) != hipSuccess ||
        launch_finite_check(d_out, width, flag, s) != hipSuccess)
        st = fail(SVL_DEVICE, "mean pool launch failed");
    if (st == SVL_OK) st = seam_finish(s, flag, "mean pooling");
    (void)hipStreamSynchronize(s);
    (void)hipFree(doff);
    return st;
}

svl_status svl_l2_normalize(const float *d_in, int64_t n, float *d_out, void *stream) {
    if (n <= 0) return fail(SVL_INTERNAL, "cannot normalize an empty vector");
    if (n > 4096) return fail(SVL_UNSUPPORTED, "vector longer than 4096");
    std::lock_guard<std::mutex> lock(g_seam_mu);
    int *flag;
    ST_TRY(seam_flag(&flag));
    hipStream_t s = (hipStream_t)stream;
    // The pool-normalisation kernel on one already pooled row applies
    // l2_normalize_scalar's arithmetic.
    svl_status st = SVL_OK;
    if (hipMemsetAsync(flag, 0, sizeof(int), s) != hipSuccess ||
        launch_pool_norm(d_in, (int)n, 1, nullptr, 0, 0, d_out, nullptr, flag, s) != hipSuccess)
        st = fail(SVL_DEVICE, "l2 launch failed");
    if (st == SVL_OK) st = seam_finish(s, flag, "L2 normalization");
    (void)hipStreamSynchronize(s);
    if (st == SVL_INTERNAL) g_err = "cannot normalize a zero or non-finite vector";
    return st;
}

// ---- synthetic data -----------------------------------------------------------

void svl_synth_uniform(uint64_t seed, uint64_t stream, float lo, float hi, size_t n, float *out) {
    const float span = hi - lo;
    parallel_for(n, [=](size_t a, size_t b) {
        for (size_t i = a; i < b; ++i) out[i] = lo + span * unit(seed, stream, i);
    });
}

void svl_synth_ids(uint64_t seed, uint64_t stream, uint32_t vocab, size_t n, uint32_t *out) {
    for (size_t i = 0; i < n; ++i) {
        uint32_t v = (uint32_t)(unit(seed, stream, i) * (float)vocab);
        out[i] = v < vocab ? v : vocab - 1;
    }
}

void svl_synth_lengths(uint64_t seed, uint64_t stream, int64_t lo, int64_t hi, size_t n,
                       int64_t *out) {
    const double span = (double)(hi - lo + 1);
    for (size_t i = 0; i < n; ++i) {
        int64_t v = lo + (int64_t)((double)unit(seed, stream, i) * span);
        out[i] = v > hi ? hi : v;
    }
}

}  // extern "C"
