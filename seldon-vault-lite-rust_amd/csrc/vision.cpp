// Host runtime of the vision tower and the image prompt glue: the
// svl_vision_* / svl_image_* part of include/svl_hip.h.
//
// It plays the role of the reference's VisionModel (src/model/vision.rs:
// 686-959) and ImageEmbedder::embed_impl (src/model/image.rs:209-253). The
// weights are validated like VisionWeights::decode (vision.rs:556-610) and
// packed once (fused QKV, interleaved gate/up). A forward call packs the
// real patches of every image of the batch back to back, runs the whole
// tower as one launch sequence on the model's stream, and reads back only
// the projected soft tokens (plus optional captures). Padding patches are
// never uploaded: like the reference, only the first valid_patches rows of
// each image take part.
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
#include "svl_internal.hpp"

namespace {

using namespace svl;

// vision.rs:29-56 caps; media/preprocess.rs:22-43 patch geometry.
constexpr int64_t MAX_VISION_HIDDEN = 16384;
constexpr int64_t MAX_VISION_INTERMEDIATE = 65536;
constexpr int64_t MAX_VISION_LAYERS = 128;
constexpr int64_t MAX_VISION_HEADS = 128;
constexpr int64_t MAX_VISION_HEAD_DIM = 1024;
constexpr int64_t MAX_POSITION_EMBEDDINGS = 1048576;
constexpr int64_t MAX_VISION_WEIGHT_ELEMENTS = int64_t(1) << 30;
constexpr int64_t PATCH_VALUES = 16 * 16 * 3;
constexpr int64_t POOL = 3;
// image.rs: the text context of an image prompt (config.rs:27).
constexpr int64_t MAX_TEXT_TOKENS = 8192;
// attn_simple_kernel bound for head dims without an MFMA attention kernel.
constexpr int64_t SIMPLE_ATTENTION_MAX_KEYS = 8192;

struct VisLayer {
    float *w_qkv = nullptr, *w_o = nullptr, *w_gu = nullptr, *w_down = nullptr;
    float *ln_in = nullptr, *ln_post_attn = nullptr, *ln_pre_ff = nullptr, *ln_post_ff = nullptr,
          *q_norm = nullptr, *k_norm = nullptr;
};

}  // namespace

struct svl_vision_model {
    int device = 0;
    int64_t H = 0, I = 0, L = 0, NH = 0, NKV = 0, hd = 0, pos_size = 0, text_hidden = 0;
    int64_t I_pad = 0, qd = 0, kd = 0;
    float eps = 0.f, theta = 0.f;
    std::vector<float> inv_freq;  // axial_inv_freq, hd / 4 entries
    std::vector<float *> allocations;
    float *w_in = nullptr, *pos_table = nullptr, *w_proj = nullptr;
    std::vector<VisLayer> layers;
    // axial RoPE angle tables [n_coord, hd/4] for coordinates 0..n_coord-1
    DevBuf<float> cos_t, sin_t;
    int64_t n_coord = 0;
    // workspace
    DevBuf<float> pix, h, n, tmp, qkv, attn, act, pooled, soft;
    DevBuf<int32_t> apos, rowlen;
    // A call's metadata in one device block, filled by one copy from pinned
    // host memory: the error flag (cleared), the patch coordinates, the
    // pooling bins, the image offsets and the attention work items.
    DevBuf<unsigned char> meta;
    unsigned char *h_meta = nullptr;  // pinned staging of `meta`
    size_t h_meta_n = 0;
    hipEvent_t ev_meta = nullptr;     // after the last copy out of h_meta
    struct {
        int *p = nullptr;
    } flag;
    struct {
        int32_t *p = nullptr;
    } coord, bin_start, bin_patch;
    struct {
        int64_t *p = nullptr;
    } offsets;
    struct {
        AttnTile *p = nullptr;
    } tiles;
    int *h_flag = nullptr;
    hipStream_t stream = nullptr;
    // image groups: the encoder layers of the second group run on `extra`
    int groups = 2;
    int64_t pass_patches = 0;  // patches per pass (0: from VIS_PASS_BYTES)
    hipStream_t extra = nullptr;
    hipEvent_t ev_fork = nullptr, ev_join = nullptr;
    std::mutex mu;

    ~svl_vision_model() {
        if (device >= 0) (void)hipSetDevice(device);
        for (float *p : allocations) (void)hipFree(p);
        cos_t.release(); sin_t.release();
        pix.release(); h.release(); n.release(); tmp.release(); qkv.release(); attn.release();
        act.release(); pooled.release(); soft.release();
        apos.release(); rowlen.release(); meta.release();
        if (ev_meta) {
            (void)hipEventSynchronize(ev_meta);
            (void)hipEventDestroy(ev_meta);
        }
        if (h_meta) (void)hipHostFree(h_meta);
        if (h_flag) (void)hipHostFree(h_flag);
        if (stream) (void)hipStreamDestroy(stream);
        if (extra) (void)hipStreamDestroy(extra);
        if (ev_fork) (void)hipEventDestroy(ev_fork);
        if (ev_join) (void)hipEventDestroy(ev_join);
    }
};

namespace {

// VisionConfig invariants (vision.rs:128-272) on an already parsed config.
svl_status validate_vision_config(const svl_vision_config *c, int64_t text_hidden) {
    if (!c) return fail(SVL_USAGE, "vision configuration is null");
    if (!std::isfinite((float)c->rms_norm_eps) || c->rms_norm_eps < 0)
        return fail(SVL_CORRUPT, "vision RMSNorm epsilon must be finite and non-negative");
    if (c->head_dim <= 0 || c->head_dim % 4)
        return fail(SVL_UNSUPPORTED,
                    "vision head dimension must be positive and divisible by four for axial RoPE");
    if (c->num_attention_heads <= 0 || c->num_key_value_heads <= 0)
        return fail(SVL_CORRUPT, "vision attention head counts must be positive");
    if (c->num_attention_heads % c->num_key_value_heads)
        return fail(SVL_CORRUPT,
                    "vision query head count is not a multiple of the key/value head count");
    const int64_t qd = c->num_attention_heads * c->head_dim;
    const int64_t kd = c->num_key_value_heads * c->head_dim;
    if (c->hidden_size <= 0 || c->hidden_size > MAX_VISION_HIDDEN || qd > MAX_VISION_HIDDEN ||
        kd > MAX_VISION_HIDDEN)
        return fail(SVL_LIMIT, "vision dimensions exceed the %lld-element hidden cap",
                    (long long)MAX_VISION_HIDDEN);
    if (c->intermediate_size <= 0 || c->intermediate_size > MAX_VISION_INTERMEDIATE)
        return fail(SVL_LIMIT, "vision intermediate size %lld exceeds the %lld cap",
                    (long long)c->intermediate_size, (long long)MAX_VISION_INTERMEDIATE);
    if (c->num_hidden_layers < 0 || c->num_hidden_layers > MAX_VISION_LAYERS)
        return fail(SVL_LIMIT, "vision layer count %lld exceeds the %lld cap",
                    (long long)c->num_hidden_layers, (long long)MAX_VISION_LAYERS);
    if (c->num_attention_heads > MAX_VISION_HEADS || c->head_dim > MAX_VISION_HEAD_DIM)
        return fail(SVL_LIMIT, "vision attention layout exceeds its documented cap");
    if (c->position_embedding_size <= 0 || c->position_embedding_size > MAX_POSITION_EMBEDDINGS)
        return fail(SVL_LIMIT, "vision position table size %lld is outside 1..=%lld",
                    (long long)c->position_embedding_size, (long long)MAX_POSITION_EMBEDDINGS);
    if (!std::isfinite((float)c->rope_theta) || (float)c->rope_theta <= 0.f)
        return fail(SVL_CORRUPT, "vision RoPE theta must be finite and positive");
    if (text_hidden <= 0 || text_hidden > MAX_VISION_HIDDEN)
        return fail(SVL_LIMIT, "text hidden size %lld is outside 1..=%lld", (long long)text_hidden,
                    (long long)MAX_VISION_HIDDEN);
    return SVL_OK;
}

// VisionConfig::tensor_shapes (vision.rs:345-414).
ShapeList vision_tensor_shapes(const svl_vision_config *c, int64_t text_hidden) {
    const int64_t H = c->hidden_size, I = c->intermediate_size, hd = c->head_dim;
    const int64_t qd = c->num_attention_heads * hd, kd = c->num_key_value_heads * hd;
    ShapeList s;
    s.push_back({"vision_tower.patch_embedder.input_proj.weight", {H, PATCH_VALUES}});
    s.push_back({"vision_tower.patch_embedder.position_embedding_table",
                 {2, c->position_embedding_size, H}});
    for (int64_t l = 0; l < c->num_hidden_layers; ++l) {
        const std::string p = "vision_tower.encoder.layers." + std::to_string(l);
        s.push_back({p + ".input_layernorm.weight", {H}});
        s.push_back({p + ".post_attention_layernorm.weight", {H}});
        s.push_back({p + ".pre_feedforward_layernorm.weight", {H}});
        s.push_back({p + ".post_feedforward_layernorm.weight", {H}});
        s.push_back({p + ".self_attn.q_proj.linear.weight", {qd, H}});
        s.push_back({p + ".self_attn.k_proj.linear.weight", {kd, H}});
        s.push_back({p + ".self_attn.v_proj.linear.weight", {kd, H}});
        s.push_back({p + ".self_attn.o_proj.linear.weight", {H, qd}});
        s.push_back({p + ".self_attn.q_norm.weight", {hd}});
        s.push_back({p + ".self_attn.k_norm.weight", {hd}});
        s.push_back({p + ".mlp.gate_proj.linear.weight", {I, H}});
        s.push_back({p + ".mlp.up_proj.linear.weight", {I, H}});
        s.push_back({p + ".mlp.down_proj.linear.weight", {H, I}});
    }
    s.push_back({"embed_vision.embedding_projection.weight", {text_hidden, H}});
    return s;
}

// axial_inv_freq (vision.rs:1047-1065) and the per-coordinate angle tables
// of axial_rope (vision.rs:1105-1121): angle = (coord as f32) * inv_freq[i],
// cos / sin in f32 on the host, exactly as the reference evaluates them.
svl_status ensure_axial_tables(svl_vision_model *v, int64_t n_coord) {
    if (n_coord <= v->n_coord) return SVL_OK;
    const int64_t q = v->hd / 4;
    std::vector<float> c((size_t)(n_coord * q)), s((size_t)(n_coord * q));
    for (int64_t p = 0; p < n_coord; ++p)
        for (int64_t i = 0; i < q; ++i) {
            const float angle = (float)p * v->inv_freq[(size_t)i];
            c[(size_t)(p * q + i)] = std::cos(angle);
            s[(size_t)(p * q + i)] = std::sin(angle);
        }
    v->cos_t.release();
    v->sin_t.release();
    v->n_coord = 0;
    HIP_TRY(v->cos_t.ensure(c.size()));
    HIP_TRY(v->sin_t.ensure(s.size()));
    HIP_TRY(hipMemcpy(v->cos_t.p, c.data(), c.size() * 4, hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(v->sin_t.p, s.data(), s.size() * 4, hipMemcpyHostToDevice));
    v->n_coord = n_coord;
    return SVL_OK;
}

// Per-call geometry of a batch of images.
struct VisBatch {
    int32_t B = 0;
    int64_t T = 0, S = 0;                 // real patches, soft tokens
    std::vector<int64_t> offsets;         // patch offsets per image [B + 1]
    std::vector<int64_t> soft_offsets;    // soft-token offsets per image [B + 1]
    std::vector<int32_t> coord;           // [T, 2] (x, y)
    std::vector<int32_t> bin_start;       // [S + 1]
    std::vector<int32_t> bin_patch;       // [T] global patch index, bin-major, patch order
    std::vector<AttnTile> tiles;
    int64_t max_coord = 0;
    double attn_flops = 0;
    int64_t hidden_stride = 0;            // patches per layer block of captured states (0: T)
    // image groups for the encoder layers: patches [t0, t1), attention work
    // items [w0, w1) of `tiles`
    struct Group {
        int64_t t0, t1, w0, w1;
    };
    std::vector<Group> groups;
};

svl_status checked_len(int i, int64_t rows, int64_t width, const char *label) {
    if (width != 0 && rows > INT64_MAX / width)
        return fail(SVL_LIMIT, "image %d: %s size overflow", i, label);
    if (rows * width > MAX_ACTIVATION_ELEMENTS)
        return fail(SVL_LIMIT, "image %d: %s would allocate %lld elements, above the cap", i,
                    label, (long long)(rows * width));
    return SVL_OK;
}

// Validation of image i in the order VisionModel::forward meets each
// condition (vision.rs:743-809, then pool_patches :981-1032).
svl_status check_image(const svl_vision_model *v, const svl_image_patches &p, int i,
                       bool need_pixels) {
    const int64_t valid = p.valid_patches;
    if (valid <= 0) return fail(SVL_CORRUPT, "image %d: vision tower received zero real patches", i);
    if (valid > p.max_patches)
        return fail(SVL_INTERNAL,
                    "image %d: vision tower received more real patches than the padded tensor", i);
    ST_TRY(checked_len(i, valid, PATCH_VALUES, "vision patch tensor"));
    ST_TRY(checked_len(i, valid, v->H, "vision hidden state"));
    ST_TRY(checked_len(i, valid, v->qd, "vision query rows"));
    ST_TRY(checked_len(i, valid, v->kd, "vision key rows"));
    ST_TRY(checked_len(i, valid, v->I, "vision feed-forward buffer"));
    if (need_pixels && !p.pixel_values)
        return fail(SVL_USAGE, "image %d: pixel values are null", i);
    if (!p.positions) return fail(SVL_USAGE, "image %d: positions are null", i);
    for (int64_t k = 0; k < valid; ++k) {
        const int32_t x = p.positions[2 * k], y = p.positions[2 * k + 1];
        if (x < 0) return fail(SVL_INTERNAL, "image %d: vision patch x position is negative", i);
        if (y < 0) return fail(SVL_INTERNAL, "image %d: vision patch y position is negative", i);
        if (x >= v->pos_size || y >= v->pos_size)
            return fail(SVL_CORRUPT,
                        "image %d: vision patch position (%d, %d) is outside the %lld-entry table",
                        i, x, y, (long long)v->pos_size);
    }
    if (v->hd != 0 && attn_block_vectors((int)v->hd) == 0 && valid > SIMPLE_ATTENTION_MAX_KEYS)
        return fail(SVL_UNSUPPORTED, "image %d: %lld patches at head dimension %lld", i,
                    (long long)valid, (long long)v->hd);
    // pool_patches geometry (vision.rs:981-1032)
    if (p.grid_width < 0 || p.grid_height < 0 || p.grid_width % POOL || p.grid_height % POOL)
        return fail(SVL_INTERNAL, "image %d: vision patch grid is not divisible by the pooling kernel", i);
    const int64_t pw = p.grid_width / POOL, ph = p.grid_height / POOL;
    if (ph != 0 && pw > INT64_MAX / ph)
        return fail(SVL_LIMIT, "image %d: vision pooled grid overflow", i);
    if (pw * ph != p.soft_tokens)
        return fail(SVL_INTERNAL,
                    "image %d: vision pooler produces %lld tokens, preprocessing declared %lld",
                    i, (long long)(pw * ph), (long long)p.soft_tokens);
    ST_TRY(checked_len(i, p.soft_tokens, v->H, "vision pooled state"));
    for (int64_t k = 0; k < valid; ++k) {
        const int64_t x = p.positions[2 * k], y = p.positions[2 * k + 1];
        if (x / POOL + pw * (y / POOL) >= p.soft_tokens)
            return fail(SVL_INTERNAL, "image %d: vision pooler computed an out-of-range bin", i);
    }
    return SVL_OK;
}

svl_status check_images(const svl_image_patches *im, int32_t batch) {
    if (batch < 0) return fail(SVL_USAGE, "negative batch");
    if (batch > 0 && !im) return fail(SVL_USAGE, "images are null");
    return SVL_OK;
}

// Validation (check_image) and the layout of a batch of images.
svl_status prepare_images(const svl_vision_model *v, const svl_image_patches *im, int32_t batch,
                          bool need_pixels, VisBatch &b, bool single) {
    ST_TRY(check_images(im, batch));
    b.B = batch;
    b.offsets.assign(1, 0);
    b.soft_offsets.assign(1, 0);
    for (int i = 0; i < batch; ++i) {
        ST_TRY(check_image(v, im[i], i, need_pixels));
        b.offsets.push_back(b.offsets.back() + im[i].valid_patches);
        b.soft_offsets.push_back(b.soft_offsets.back() + im[i].soft_tokens);
    }
    b.T = b.offsets.back();
    b.S = b.soft_offsets.back();
    if (b.T > (int64_t)INT32_MAX / 8 || b.S > (int64_t)INT32_MAX / 8)
        return fail(SVL_LIMIT, "batch holds too many patches");
    b.coord.resize((size_t)(2 * b.T));
    b.bin_start.assign((size_t)b.S + 1, 0);
    b.bin_patch.resize((size_t)b.T);
    std::vector<int32_t> bin_of((size_t)b.T);
    for (int i = 0; i < batch; ++i) {
        const svl_image_patches &p = im[i];
        const int64_t t0 = b.offsets[i], s0 = b.soft_offsets[i], pw = p.grid_width / POOL;
        for (int64_t k = 0; k < p.valid_patches; ++k) {
            const int32_t x = p.positions[2 * k], y = p.positions[2 * k + 1];
            b.coord[(size_t)(2 * (t0 + k))] = x;
            b.coord[(size_t)(2 * (t0 + k) + 1)] = y;
            b.max_coord = std::max<int64_t>(b.max_coord, std::max(x, y));
            const int64_t bin = s0 + x / POOL + pw * (y / POOL);
            bin_of[(size_t)(t0 + k)] = (int32_t)bin;
            b.bin_start[(size_t)bin + 1] += 1;
        }
    }
    for (int64_t s = 0; s < b.S; ++s) b.bin_start[(size_t)s + 1] += b.bin_start[(size_t)s];
    {
        std::vector<int32_t> fill(b.bin_start.begin(), b.bin_start.end() - 1);
        for (int64_t t = 0; t < b.T; ++t) b.bin_patch[(size_t)fill[(size_t)bin_of[(size_t)t]]++] = (int32_t)t;
    }
    // Image groups: consecutive images in two groups of about equal patch
    // counts when there are two or more images and 4096 or more patches
    // (and the MFMA attention applies); otherwise one group.
    const int bv = attn_block_vectors((int)v->hd);
    int cut = 0;  // first image of the second group
    if (!single && v->groups >= 2 && batch >= 2 && b.T >= 4096 && bv > 0) {
        int64_t best = b.T;
        for (int c = 1; c < batch; ++c) {
            const int64_t d = std::llabs(2 * b.offsets[(size_t)c] - b.T);
            if (d < best) {
                best = d;
                cut = c;
            }
        }
    }
    // attention work items of each group, longest images first
    const int G = (int)(v->NH / v->NKV);
    auto add_group = [&](int i0, int i1) {
        const int64_t w0 = (int64_t)b.tiles.size();
        std::vector<int> order;
        for (int i = i0; i < i1; ++i) order.push_back(i);
        std::stable_sort(order.begin(), order.end(), [&](int x, int y) {
            return im[x].valid_patches > im[y].valid_patches;
        });
        if (bv > 0)
            for (int i : order) {
                const int64_t len = im[i].valid_patches;
                for (int kv = 0; kv < v->NKV; ++kv)
                    for (int64_t v0 = 0; v0 < len * G; v0 += bv)
                        b.tiles.push_back({(int32_t)b.offsets[i], (int32_t)len, kv, (int32_t)v0});
            }
        b.groups.push_back({b.offsets[(size_t)i0], b.offsets[(size_t)i1], w0, (int64_t)b.tiles.size()});
    };
    if (cut > 0) {
        add_group(0, cut);
        add_group(cut, batch);
    } else {
        add_group(0, batch);
    }
    for (int i = 0; i < batch; ++i) {
        const double len = (double)im[i].valid_patches;
        b.attn_flops += 4.0 * (double)v->hd * (double)v->NH * len * len;
    }
    return SVL_OK;
}

svl_status ensure_vis_workspace(svl_vision_model *v, const VisBatch &b) {
    const int64_t T = std::max<int64_t>(b.T, 1), S = std::max<int64_t>(b.S, 1);
    HIP_TRY(v->pix.ensure(T * PATCH_VALUES));
    HIP_TRY(v->h.ensure(T * v->H));
    HIP_TRY(v->n.ensure(T * v->H));
    HIP_TRY(v->tmp.ensure(T * v->H));
    HIP_TRY(v->qkv.ensure(T * (v->qd + 2 * v->kd)));
    HIP_TRY(v->attn.ensure(T * v->qd));
    HIP_TRY(v->act.ensure(T * v->I));
    HIP_TRY(v->pooled.ensure(S * v->H));
    HIP_TRY(v->soft.ensure(S * v->text_hidden));
    HIP_TRY(v->apos.ensure(T));
    HIP_TRY(v->rowlen.ensure(T));
    return SVL_OK;
}

// The call's metadata (flag cleared, patch coordinates, pooling bins, image
// offsets, attention work items) staged in pinned host memory and sent by
// one copy on `s` instead of a copy or fill per array. The staging is
// rewritten only once the copy before has left it.
svl_status upload_vis_meta(svl_vision_model *v, const VisBatch &b, hipStream_t s) {
    auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
    const size_t bytes[6] = {sizeof(int), b.coord.size() * 4, b.bin_start.size() * 4,
                             b.bin_patch.size() * 4, b.offsets.size() * 8,
                             b.tiles.size() * sizeof(AttnTile)};
    size_t off[6], total = 0;
    for (int i = 0; i < 6; ++i) {
        off[i] = total;
        total += up(std::max<size_t>(bytes[i], 1));
    }
    HIP_TRY(v->meta.ensure(total));
    if (v->ev_meta) HIP_TRY(hipEventSynchronize(v->ev_meta));
    else HIP_TRY(hipEventCreateWithFlags(&v->ev_meta, hipEventDisableTiming));
    if (v->h_meta_n < total) {
        if (v->h_meta) HIP_TRY(hipHostFree(v->h_meta));
        v->h_meta = nullptr;
        v->h_meta_n = 0;
        HIP_TRY(hipHostMalloc((void **)&v->h_meta, total, hipHostMallocDefault));
        v->h_meta_n = total;
    }
    unsigned char *h = v->h_meta, *d = v->meta.p;
    std::memset(h, 0, total);
    std::memcpy(h + off[1], b.coord.data(), bytes[1]);
    std::memcpy(h + off[2], b.bin_start.data(), bytes[2]);
    std::memcpy(h + off[3], b.bin_patch.data(), bytes[3]);
    std::memcpy(h + off[4], b.offsets.data(), bytes[4]);
    if (bytes[5]) std::memcpy(h + off[5], b.tiles.data(), bytes[5]);
    v->flag.p = (int *)d;
    v->coord.p = (int32_t *)(d + off[1]);
    v->bin_start.p = (int32_t *)(d + off[2]);
    v->bin_patch.p = (int32_t *)(d + off[3]);
    v->offsets.p = (int64_t *)(d + off[4]);
    v->tiles.p = (AttnTile *)(d + off[5]);
    HIP_TRY(hipMemcpyAsync(d, h, total, hipMemcpyHostToDevice, s));
    HIP_TRY(hipEventRecord(v->ev_meta, s));
    return SVL_OK;
}

// The encoder layers (vision.rs:852-930) over patches [g.t0, g.t1) of the
// batch on stream s; every kernel works row by row or within the group's
// images, so the rows get the same arithmetic as one launch over the batch.
// h_hidden: the batch's first patch in a [L + 1, hidden_stride, H] host
// capture (one group only).
svl_status enqueue_vis_layers(svl_vision_model *v, const VisBatch &b, const VisBatch::Group &g,
                              hipStream_t s, float *h_hidden) {
    const int64_t T = b.T, H = v->H, R = g.t1 - g.t0;
    const int64_t Ts = b.hidden_stride > 0 ? b.hidden_stride : T;
    if (R <= 0) return SVL_OK;
    int *flag = v->flag.p;
    const int64_t ldqkv = v->qd + 2 * v->kd;
    const int cus = b.groups.size() > 1 ? (int)(256 / b.groups.size()) : 0;
    float *h = v->h.p + g.t0 * H, *n = v->n.p + g.t0 * H, *tmp = v->tmp.p + g.t0 * H,
          *qkv = v->qkv.p + g.t0 * ldqkv, *attn = v->attn.p + g.t0 * v->qd, *act = v->act.p + g.t0 * v->I;
    for (int64_t l = 0; l < v->L; ++l) {
        const VisLayer &ly = v->layers[(size_t)l];
        {
            GemmArgs ga{n, H, ly.w_qkv, H, qkv, ldqkv, (int)R, (int)ldqkv, (int)H, EPI_STORE, 1.f,
                        nullptr, 0, 0};
            ga.cus = cus;
            HIP_TRY(launch_gemm(ga, s));
        }
        HIP_TRY(launch_qkv_post_axial(qkv, ldqkv, R, (int)v->NH, (int)v->NKV, (int)v->hd,
                                      ly.q_norm, ly.k_norm, v->cos_t.p, v->sin_t.p,
                                      v->coord.p + 2 * g.t0, v->eps, flag, s));
        {
            AttnArgs a{};
            a.q = v->qkv.p;
            a.k = v->qkv.p + v->qd;
            a.v = v->qkv.p + v->qd + v->kd;
            a.out = v->attn.p;
            a.ldq = a.ldk = a.ldv = ldqkv;
            a.ldo = v->qd;
            a.nh = (int)v->NH;
            a.nkv = (int)v->NKV;
            a.hd = (int)v->hd;
            a.window = -1;   // vision.rs:880 sliding_window: None
            a.scale = 1.0f;  // vision.rs:881
            a.tiles = v->tiles.p + g.w0;  // absolute first patches of the group's images
            a.n_tiles = (int)(g.w1 - g.w0);
            a.pos = v->apos.p;
            a.rowlen = v->rowlen.p;
            a.tokens = T;
            a.flag = flag;
            HIP_TRY(launch_attention(a, s));
        }
        {
            GemmArgs ga{attn, v->qd, ly.w_o, v->qd, tmp, H, (int)R, (int)H, (int)v->qd, EPI_STORE,
                        1.f, nullptr, 0, 0};
            ga.cus = cus;
            HIP_TRY(launch_gemm(ga, s));
        }
        HIP_TRY(launch_resnorm(tmp, ly.ln_post_attn, h, h, ly.ln_pre_ff, n, 1.0f, R, (int)H, v->eps,
                               flag, s));
        {
            GemmArgs ga{n, H, ly.w_gu, H, act, v->I, (int)R, (int)(2 * v->I_pad), (int)H, EPI_GEGLU,
                        1.f, nullptr, 0, (int)v->I};
            ga.cus = cus;
            HIP_TRY(launch_gemm(ga, s));
        }
        {
            GemmArgs ga{act, v->I, ly.w_down, v->I, tmp, H, (int)R, (int)H, (int)v->I, EPI_STORE,
                        1.f, nullptr, 0, 0};
            ga.cus = cus;
            HIP_TRY(launch_gemm(ga, s));
        }
        const float *next = l + 1 < v->L ? v->layers[(size_t)l + 1].ln_in : nullptr;
        HIP_TRY(launch_resnorm(tmp, ly.ln_post_ff, h, h, next, next ? n : nullptr, 1.0f, R, (int)H,
                               v->eps, flag, s));
        if (h_hidden)
            HIP_TRY(hipMemcpyAsync(h_hidden + (size_t)((l + 1) * Ts * H), v->h.p,
                                   (size_t)(T * H) * 4, hipMemcpyDeviceToHost, s));
    }

    return SVL_OK;
}

// The tower over the packed patches in d_pix (overwritten with the rescaled
// values), enqueued on s (vision.rs:760-951). Soft tokens land in v->soft.
svl_status enqueue_vision(svl_vision_model *v, const VisBatch &b, float *d_pix, hipStream_t s,
                          float *h_hidden) {
    const int64_t T = b.T, H = v->H, S = b.S;
    if (T == 0) return SVL_OK;
    int *flag = v->flag.p;
    HIP_TRY(launch_positions(v->offsets.p, b.B, v->apos.p, v->rowlen.p, s));
    HIP_TRY(launch_patch_scale(d_pix, d_pix, T * PATCH_VALUES, s));
    {
        GemmArgs g{d_pix, PATCH_VALUES, v->w_in, PATCH_VALUES, v->h.p, H, (int)T, (int)H,
                   (int)PATCH_VALUES, EPI_STORE, 1.f, nullptr, 0, 0};
        HIP_TRY(launch_gemm(g, s));
    }
    // position add fused with layer 0's input norm (the model has >= 1 layer)
    HIP_TRY(launch_patch_pos(v->h.p, v->coord.p, v->pos_table, v->pos_size, v->layers[0].ln_in,
                             v->n.p, T, (int)H, v->eps, flag, s));
    if (h_hidden)
        HIP_TRY(hipMemcpyAsync(h_hidden, v->h.p, (size_t)(T * H) * 4, hipMemcpyDeviceToHost, s));

    if (b.groups.size() > 1) {
        // the second image group runs its layers on the model's second stream
        HIP_TRY(hipEventRecord(v->ev_fork, s));
        HIP_TRY(hipStreamWaitEvent(v->extra, v->ev_fork, 0));
        ST_TRY(enqueue_vis_layers(v, b, b.groups[1], v->extra, nullptr));
        ST_TRY(enqueue_vis_layers(v, b, b.groups[0], s, nullptr));
        HIP_TRY(hipEventRecord(v->ev_join, v->extra));
        HIP_TRY(hipStreamWaitEvent(s, v->ev_join, 0));
    } else {
        ST_TRY(enqueue_vis_layers(v, b, b.groups[0], s, h_hidden));
    }

    // pool_patches + rms_norm_rows_unscaled + embedding projection
    // (vision.rs:937-951).
    HIP_TRY(launch_pool_bins(v->h.p, v->bin_start.p, v->bin_patch.p, S, (int)H, (float)(POOL * POOL),
                             std::sqrt((float)H), v->eps, v->pooled.p, flag, s));
    {
        GemmArgs g{v->pooled.p, H, v->w_proj, H, v->soft.p, v->text_hidden, (int)S,
                   (int)v->text_hidden, (int)H, EPI_STORE, 1.f, nullptr, 0, 0};
        HIP_TRY(launch_gemm(g, s));
    }
    HIP_TRY(launch_finite_check(v->soft.p, S * v->text_hidden, flag, s));
    return SVL_OK;
}

svl_status vis_finish(svl_vision_model *v, hipStream_t s) {
    HIP_TRY(hipMemcpyAsync(v->h_flag, v->flag.p, sizeof(int), hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    if (*v->h_flag & FLAG_NONFINITE)
        return fail(SVL_INTERNAL, "the vision tower produced a non-finite value");
    return SVL_OK;
}

// Every workspace buffer grows with the batch's patches, so a batch runs in
// passes of consecutive images whose workspace stays within VIS_PASS_BYTES
// (an image larger than a pass runs alone). An image's bits do not depend on
// the images beside it, so the outputs equal those of one pass.
constexpr int64_t VIS_PASS_BYTES = (int64_t)32 << 30;
constexpr int64_t MAX_PASS_PATCHES = (int64_t)INT32_MAX / 8;

int64_t vis_pass_budget(const svl_vision_model *v) {
    if (v->pass_patches > 0) return v->pass_patches;
    const int64_t per_patch = 4 * (PATCH_VALUES + 3 * v->H + 2 * v->qd + 2 * v->kd + v->I + 6);
    return std::min(MAX_PASS_PATCHES, std::max<int64_t>(1, VIS_PASS_BYTES / per_patch));
}

// Images [first, last) of each pass, after check_image has passed for all.
std::vector<std::pair<int32_t, int32_t>> image_passes(const svl_vision_model *v,
                                                      const svl_image_patches *im,
                                                      int32_t batch) {
    std::vector<std::pair<int32_t, int32_t>> passes;
    const int64_t cap = vis_pass_budget(v);
    int32_t i0 = 0;
    int64_t patches = 0;
    for (int32_t i = 0; i < batch; ++i) {
        if (i > i0 && patches + im[i].valid_patches > cap) {
            passes.emplace_back(i0, i);
            i0 = i;
            patches = 0;
        }
        patches += im[i].valid_patches;
    }
    if (batch > 0) passes.emplace_back(i0, batch);
    return passes;
}

// check_image for every image of a batch (image indices of the whole batch
// in the messages); *patches = their real patches.
svl_status check_batch(const svl_vision_model *v, const svl_image_patches *im, int32_t batch,
                       bool need_pixels, int64_t *patches) {
    ST_TRY(check_images(im, batch));
    *patches = 0;
    for (int i = 0; i < batch; ++i) {
        ST_TRY(check_image(v, im[i], i, need_pixels));
        *patches += im[i].valid_patches;
    }
    return SVL_OK;
}

// Runs the tower for one pass; the soft tokens stay in v->soft (and are
// copied to out_soft when given). Pixels come from the host images, or from
// d_pixels ([sum valid, 768] in HBM, rescaled in place) when it is given.
// out_hidden: the pass's first patch in a [L + 1, hidden_stride, H] capture.
// Caller holds v->mu.
svl_status run_vision(svl_vision_model *v, const svl_image_patches *images, int32_t batch,
                      float *d_pixels, hipStream_t s, VisBatch &b, float *out_soft,
                      float *out_hidden, int64_t hidden_stride) {
    HIP_TRY(hipSetDevice(v->device));
    ST_TRY(prepare_images(v, images, batch, d_pixels == nullptr, b, out_hidden != nullptr));
    if (batch == 0) return SVL_OK;
    b.hidden_stride = hidden_stride;
    ST_TRY(ensure_axial_tables(v, b.max_coord + 1));
    ST_TRY(ensure_vis_workspace(v, b));
    if (!d_pixels) {
        for (int i = 0; i < batch; ++i)
            HIP_TRY(hipMemcpyAsync(v->pix.p + b.offsets[i] * PATCH_VALUES, images[i].pixel_values,
                                   (size_t)(images[i].valid_patches * PATCH_VALUES) * 4,
                                   hipMemcpyHostToDevice, s));
        d_pixels = v->pix.p;
    }
    ST_TRY(upload_vis_meta(v, b, s));
    ST_TRY(enqueue_vision(v, b, d_pixels, s, out_hidden));
    if (out_soft)
        HIP_TRY(hipMemcpyAsync(out_soft, v->soft.p, (size_t)(b.S * v->text_hidden) * 4,
                               hipMemcpyDeviceToHost, s));
    return vis_finish(v, s);
}

// ImageEmbedder::embed_impl (image.rs:209-253) for a batch; see
// svl_image_embed_batch.
svl_status image_embed(svl_vision_model *v, svl_text_model *text,
                       const svl_image_special_tokens *tokens, const svl_image_patches *images,
                       int32_t batch, float *d_pixels, int64_t dimension, float *out) {
    if (!v || !text || !tokens || !out)
        return fail(SVL_USAGE, "models, special tokens and output are required");
    // image.rs:215-221
    const int64_t E = text_embedding_dim(text);
    if (dimension <= 0 || dimension > E)
        return fail(SVL_INTERNAL, "embedding dimension %lld is outside 1..=%lld",
                    (long long)dimension, (long long)E);
    if (text_device(text) != v->device)
        return fail(SVL_USAGE, "the vision and text models live on different devices");
    if (text_hidden_size(text) != v->text_hidden)
        return fail(SVL_USAGE, "the vision projection width %lld is not the text hidden size %lld",
                    (long long)v->text_hidden, (long long)text_hidden_size(text));
    std::lock_guard<std::mutex> lock(v->mu);
    int64_t patches = 0;
    ST_TRY(check_batch(v, images, batch, d_pixels == nullptr, &patches));
    if (batch == 0) return SVL_OK;
    // image.rs:224-244: <bos> <boi> <image> x soft <eoi> <eos>, features at 2.
    for (int i = 0; i < batch; ++i) {
        const int64_t seq = images[i].soft_tokens + 4;
        if (seq > MAX_TEXT_TOKENS)
            return fail(SVL_LIMIT, "image %d: image prompt has %lld tokens, above the %lld-token context",
                        i, (long long)seq, (long long)MAX_TEXT_TOKENS);
    }
    int64_t first_patch = 0;
    for (const auto &pr : image_passes(v, images, batch)) {
        const int32_t i0 = pr.first, n = pr.second - pr.first;
        VisBatch b;
        ST_TRY(run_vision(v, images + i0, n, d_pixels ? d_pixels + first_patch * PATCH_VALUES : nullptr,
                          v->stream, b, nullptr, nullptr, 0));
        first_patch += b.T;
        std::vector<int64_t> offsets(1, 0);
        for (int i = 0; i < n; ++i) offsets.push_back(offsets.back() + images[i0 + i].soft_tokens + 4);
        std::vector<uint32_t> ids((size_t)offsets.back());
        std::vector<int32_t> featmap((size_t)offsets.back(), -1);
        for (int i = 0; i < n; ++i) {
            const int64_t o = offsets[i], soft = images[i0 + i].soft_tokens;
            ids[(size_t)o] = tokens->bos;
            ids[(size_t)o + 1] = tokens->boi;
            for (int64_t k = 0; k < soft; ++k) {
                ids[(size_t)(o + 2 + k)] = tokens->image;
                featmap[(size_t)(o + 2 + k)] = (int32_t)(b.soft_offsets[i] + k);
            }
            ids[(size_t)(o + 2 + soft)] = tokens->eoi;
            ids[(size_t)(o + 3 + soft)] = tokens->eos;
        }
        std::vector<float> normalized((size_t)(n * E));
        ST_TRY(text_forward_with_device_features(text, ids.data(), offsets.data(), n,
                                                 featmap.data(), v->soft.p, normalized.data()));
        for (int i = 0; i < n; ++i)
            ST_TRY(svl_truncate_and_normalize(normalized.data() + (size_t)i * E, (size_t)E,
                                              (size_t)dimension,
                                              out + (size_t)(i0 + i) * dimension));
    }
    return SVL_OK;
}

}  // namespace

extern "C" {

svl_status svl_vision_model_create(svl_ctx *ctx, const svl_vision_config *cfg, int64_t text_hidden,
                                   const svl_tensor_view *tensors, size_t n_tensors,
                                   svl_vision_model **out) {
    if (!ctx || !out) return fail(SVL_USAGE, "context or output pointer is null");
    ST_TRY(validate_vision_config(cfg, text_hidden));
    const int device = ctx->device;
    HIP_TRY(hipSetDevice(device));
    const ShapeList shapes = vision_tensor_shapes(cfg, text_hidden);
    TensorIndex by_name;
    ST_TRY(check_inventory(tensors, n_tensors, shapes, {"vision_tower.", "embed_vision."}, "vision",
                           MAX_VISION_WEIGHT_ELEMENTS, by_name));

    auto v = new svl_vision_model();
    std::unique_ptr<svl_vision_model> guard(v);
    v->device = device;
    v->H = cfg->hidden_size;
    v->I = cfg->intermediate_size;
    v->L = cfg->num_hidden_layers;
    v->NH = cfg->num_attention_heads;
    v->NKV = cfg->num_key_value_heads;
    v->hd = cfg->head_dim;
    v->pos_size = cfg->position_embedding_size;
    v->text_hidden = text_hidden;
    v->eps = (float)cfg->rms_norm_eps;
    v->theta = (float)cfg->rope_theta;
    v->I_pad = (v->I + 31) / 32 * 32;
    v->qd = v->NH * v->hd;
    v->kd = v->NKV * v->hd;
    if (v->H % 4 || v->H > 2048)
        return fail(SVL_UNSUPPORTED, "vision hidden size %lld is not a multiple of 4 up to 2048",
                    (long long)v->H);
    if (v->L == 0) return fail(SVL_UNSUPPORTED, "a vision tower without layers is not supported");
    // axial_inv_freq (vision.rs:1047-1065)
    const int64_t spatial = v->hd / 2;
    for (int64_t i = 0; i < spatial / 2; ++i) {
        const float exponent = (float)(2 * i) / (float)spatial;
        const float value = 1.0f / std::pow(v->theta, exponent);
        if (!std::isfinite(value)) return fail(SVL_INTERNAL, "axial RoPE frequency is not finite");
        v->inv_freq.push_back(value);
    }

    auto up = [&](const std::string &name, float **dst) -> svl_status {
        std::vector<float> a;
        ST_TRY(decode_named(by_name, name, a));
        return upload_owned(v->allocations, a.data(), a.size(), dst);
    };
    ST_TRY(up("vision_tower.patch_embedder.input_proj.weight", &v->w_in));
    ST_TRY(up("vision_tower.patch_embedder.position_embedding_table", &v->pos_table));
    ST_TRY(up("embed_vision.embedding_projection.weight", &v->w_proj));
    v->layers.resize((size_t)v->L);
    std::vector<float> a, b2, c2;
    for (int64_t l = 0; l < v->L; ++l) {
        VisLayer &ly = v->layers[(size_t)l];
        const std::string p = "vision_tower.encoder.layers." + std::to_string(l) + ".";
        std::vector<float> qkv((size_t)((v->qd + 2 * v->kd) * v->H));
        ST_TRY(decode_named(by_name, p + "self_attn.q_proj.linear.weight", a));
        std::copy(a.begin(), a.end(), qkv.begin());
        ST_TRY(decode_named(by_name, p + "self_attn.k_proj.linear.weight", a));
        std::copy(a.begin(), a.end(), qkv.begin() + v->qd * v->H);
        ST_TRY(decode_named(by_name, p + "self_attn.v_proj.linear.weight", a));
        std::copy(a.begin(), a.end(), qkv.begin() + (v->qd + v->kd) * v->H);
        ST_TRY(upload_owned(v->allocations, qkv.data(), qkv.size(), &ly.w_qkv));
        ST_TRY(up(p + "self_attn.o_proj.linear.weight", &ly.w_o));
        ST_TRY(decode_named(by_name, p + "mlp.gate_proj.linear.weight", b2));
        ST_TRY(decode_named(by_name, p + "mlp.up_proj.linear.weight", c2));
        const std::vector<float> gu = interleave_gate_up(b2, c2, v->I, v->I_pad, v->H);
        ST_TRY(upload_owned(v->allocations, gu.data(), gu.size(), &ly.w_gu));
        ST_TRY(up(p + "mlp.down_proj.linear.weight", &ly.w_down));
        ST_TRY(up(p + "input_layernorm.weight", &ly.ln_in));
        ST_TRY(up(p + "post_attention_layernorm.weight", &ly.ln_post_attn));
        ST_TRY(up(p + "pre_feedforward_layernorm.weight", &ly.ln_pre_ff));
        ST_TRY(up(p + "post_feedforward_layernorm.weight", &ly.ln_post_ff));
        ST_TRY(up(p + "self_attn.q_norm.weight", &ly.q_norm));
        ST_TRY(up(p + "self_attn.k_norm.weight", &ly.k_norm));
    }
    HIP_TRY(hipStreamCreateWithFlags(&v->stream, hipStreamNonBlocking));
    HIP_TRY(hipStreamCreateWithFlags(&v->extra, hipStreamNonBlocking));
    HIP_TRY(hipEventCreateWithFlags(&v->ev_fork, hipEventDisableTiming));
    HIP_TRY(hipEventCreateWithFlags(&v->ev_join, hipEventDisableTiming));
    HIP_TRY(hipHostMalloc((void **)&v->h_flag, sizeof(int), hipHostMallocDefault));
    *out = guard.release();
    return SVL_OK;
}

svl_status svl_vision_model_set_stream_split(svl_vision_model *model, int groups) {
    if (!model) return fail(SVL_USAGE, "vision model is null");
    if (groups < 1 || groups > 2) return fail(SVL_USAGE, "image groups must be 1 or 2");
    std::lock_guard<std::mutex> lock(model->mu);
    model->groups = groups;
    return SVL_OK;
}

svl_status svl_vision_model_set_pass_patches(svl_vision_model *model, int64_t patches) {
    if (!model) return fail(SVL_USAGE, "vision model is null");
    if (patches < 0 || patches > MAX_PASS_PATCHES)
        return fail(SVL_USAGE, "pass size %lld is outside 0..=%lld patches", (long long)patches,
                    (long long)MAX_PASS_PATCHES);
    std::lock_guard<std::mutex> lock(model->mu);
    model->pass_patches = patches;
    return SVL_OK;
}

svl_status svl_vision_model_destroy(svl_vision_model *model) {
    delete model;
    return SVL_OK;
}

svl_status svl_vision_forward_batch(svl_vision_model *v, const svl_image_patches *images,
                                    int32_t batch, float *out_soft, float *out_hidden) {
    if (!v || !out_soft) return fail(SVL_USAGE, "model and out_soft are required");
    std::lock_guard<std::mutex> lock(v->mu);
    int64_t patches = 0;
    ST_TRY(check_batch(v, images, batch, true, &patches));
    int64_t t0 = 0, s0 = 0;
    for (const auto &pr : image_passes(v, images, batch)) {
        VisBatch b;
        ST_TRY(run_vision(v, images + pr.first, pr.second - pr.first, nullptr, v->stream, b,
                          out_soft + (size_t)(s0 * v->text_hidden),
                          out_hidden ? out_hidden + (size_t)(t0 * v->H) : nullptr, patches));
        t0 += b.T;
        s0 += b.S;
    }
    return SVL_OK;
}

svl_status svl_vision_forward_device(svl_vision_model *v, float *d_pixels,
                                     const svl_image_patches *images, int32_t batch, float *d_out,
                                     void *stream) {
    if (!v || !d_pixels || !d_out) return fail(SVL_USAGE, "model, pixels and output are required");
    std::lock_guard<std::mutex> lock(v->mu);
    hipStream_t s = stream ? (hipStream_t)stream : v->stream;
    int64_t patches = 0;
    ST_TRY(check_batch(v, images, batch, false, &patches));
    int64_t t0 = 0, s0 = 0;
    for (const auto &pr : image_passes(v, images, batch)) {
        VisBatch b;
        ST_TRY(run_vision(v, images + pr.first, pr.second - pr.first,
                          d_pixels + (size_t)(t0 * PATCH_VALUES), s, b, nullptr, nullptr, 0));
        HIP_TRY(hipMemcpyAsync(d_out + (size_t)(s0 * v->text_hidden), v->soft.p,
                               (size_t)(b.S * v->text_hidden) * 4, hipMemcpyDeviceToDevice, s));
        HIP_TRY(hipStreamSynchronize(s));
        t0 += b.T;
        s0 += b.S;
    }
    return SVL_OK;
}

svl_status svl_image_embed_batch(svl_vision_model *v, svl_text_model *text,
                                 const svl_image_special_tokens *tokens,
                                 const svl_image_patches *images, int32_t batch, int64_t dimension,
                                 float *out) {
    return image_embed(v, text, tokens, images, batch, nullptr, dimension, out);
}

svl_status svl_image_embed_device(svl_vision_model *v, svl_text_model *text,
                                  const svl_image_special_tokens *tokens, float *d_pixels,
                                  const svl_image_patches *images, int32_t batch, int64_t dimension,
                                  float *out) {
    if (!d_pixels) return fail(SVL_USAGE, "pixels are required");
    return image_embed(v, text, tokens, images, batch, d_pixels, dimension, out);
}

}  // extern "C"
