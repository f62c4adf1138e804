/*
 * CPU oracle, vision tower: a C restatement of src/model/vision.rs.
 *
 * TEST INFRASTRUCTURE ONLY: the oracle for the HIP vision path, never part
 * of the product library. Same build rules as svl_oracle.c (-O2,
 * -ffp-contract=off, no fast-math) and the same kernels (svlo_linear,
 * svlo_rms_norm_rows, svlo_bidirectional_attention, ...).
 *
 * Parity pins (tests/test_oracle_vision.py):
 *  - svlo_axial_inv_freq / svlo_axial_rope against the known answers of
 *    src/model/vision.rs:1154-1182 and a float64 rotation restatement;
 *  - svlo_pool_patches against a float64 bin average;
 *  - svlo_vision_forward by closed forms of degenerate weight sets (zero
 *    projections: every layer is the identity; identical patches: attention
 *    returns the value row), by a brute-force softmax over two patches that
 *    fixes the q_norm / k_norm / axial RoPE wiring (tests/test_oracle_wiring.py),
 *    and against an independent float64 numpy forward with random weights.
 *    No offline golden exists for the vision tower (the reference's image
 *    golden needs the full released weights).
 *  - svlo_vision_layer is the forward pass's own per-layer code; chaining it
 *    reproduces svlo_vision_forward bit for bit.
 */
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "svl_oracle.h"

/* text.rs:34 MAX_ACTIVATION_ELEMENTS (vision.rs:962-972 reuses it). */
#define VIS_MAX_ACTIVATION_ELEMENTS ((size_t)1 << 28)
/* media/preprocess.rs:22-43 */
#define VIS_PATCH_VALUES (16 * 16 * 3)
#define VIS_POOL 3

static int vis_all_finite(const float *v, size_t n) {
    for (size_t i = 0; i < n; ++i)
        if (!isfinite(v[i])) return 0;
    return 1;
}

static int vis_fail(char *msg, size_t msg_len, int code, const char *fmt, ...) {
    if (msg && msg_len) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(msg, msg_len, fmt, ap);
        va_end(ap);
    }
    return code;
}

/* vision.rs:962-972 checked_len. */
static int vis_checked_len(size_t rows, size_t width, size_t *out) {
    if (width != 0 && rows > SIZE_MAX / width) return SVLO_LIMIT;
    size_t n = rows * width;
    if (n > VIS_MAX_ACTIVATION_ELEMENTS) return SVLO_LIMIT;
    *out = n;
    return SVLO_OK;
}

/* vision.rs:1047-1065 axial_inv_freq: head_dim/4 frequencies
 * 1 / theta^((2i) / (head_dim/2)). */
int svlo_axial_inv_freq(size_t head_dim, float theta, float *out) {
    if (head_dim == 0 || head_dim % 4) return SVLO_INTERNAL;
    size_t spatial = head_dim / 2, count = spatial / 2;
    for (size_t i = 0; i < count; ++i) {
        float exponent = (float)(2 * i) / (float)spatial;
        float value = 1.0f / powf(theta, exponent);
        if (!isfinite(value)) return SVLO_INTERNAL;
        out[i] = value;
    }
    return SVLO_OK;
}

/* vision.rs:1073-1148 axial_rope: the first half of each head rotates with
 * x, the second with y; within a half, quarter i pairs with quarter i + q. */
int svlo_axial_rope(float *values, size_t sequence, size_t heads, size_t head_dim,
                    const int32_t *positions, size_t n_positions, const float *inv_freq,
                    size_t n_inv_freq) {
    if (head_dim % 4) return SVLO_INTERNAL;
    if (n_inv_freq != head_dim / 4) return SVLO_INTERNAL;
    if (n_positions < sequence) return SVLO_INTERNAL;
    const size_t half = head_dim / 2, quarter = head_dim / 4;
    float *cos_h = (float *)malloc((sequence * quarter + 1) * sizeof(float));
    float *sin_h = (float *)malloc((sequence * quarter + 1) * sizeof(float));
    float *cos_w = (float *)malloc((sequence * quarter + 1) * sizeof(float));
    float *sin_w = (float *)malloc((sequence * quarter + 1) * sizeof(float));
    int st = SVLO_OK;
    if (!cos_h || !sin_h || !cos_w || !sin_w) {
        st = SVLO_LIMIT;
        goto done;
    }
    for (size_t p = 0; p < sequence; ++p) {
        if (positions[2 * p] < 0 || positions[2 * p + 1] < 0) {
            st = SVLO_INTERNAL;
            goto done;
        }
        float x = (float)positions[2 * p], y = (float)positions[2 * p + 1];
        for (size_t i = 0; i < quarter; ++i) {
            float ah = x * inv_freq[i], aw = y * inv_freq[i];
            cos_h[p * quarter + i] = cosf(ah);
            sin_h[p * quarter + i] = sinf(ah);
            cos_w[p * quarter + i] = cosf(aw);
            sin_w[p * quarter + i] = sinf(aw);
        }
    }
    for (size_t p = 0; p < sequence; ++p)
        for (size_t h = 0; h < heads; ++h) {
            float *base = values + (p * heads + h) * head_dim;
            float *wide = base + half;
            for (size_t i = 0; i < quarter; ++i) {
                float c = cos_h[p * quarter + i], s = sin_h[p * quarter + i];
                float f = base[i], g = base[i + quarter];
                base[i] = f * c - g * s;
                base[i + quarter] = g * c + f * s;
                c = cos_w[p * quarter + i];
                s = sin_w[p * quarter + i];
                f = wide[i];
                g = wide[i + quarter];
                wide[i] = f * c - g * s;
                wide[i + quarter] = g * c + f * s;
            }
        }
    if (!vis_all_finite(values, sequence * heads * head_dim)) st = SVLO_INTERNAL;
done:
    free(cos_h);
    free(sin_h);
    free(cos_w);
    free(sin_w);
    return st;
}

/* vision.rs:980-1040 pool_patches: bin = x/3 + pooled_width * (y/3); rows are
 * summed into their bin in patch order, then (sum / 9) * sqrt(hidden). */
int svlo_pool_patches(const float *hidden, const int32_t *positions, size_t valid,
                      size_t grid_width, size_t grid_height, size_t soft_tokens,
                      size_t hidden_size, float *out) {
    if (grid_width % VIS_POOL || grid_height % VIS_POOL) return SVLO_INTERNAL;
    size_t pw = grid_width / VIS_POOL, ph = grid_height / VIS_POOL;
    if (ph != 0 && pw > SIZE_MAX / ph) return SVLO_LIMIT;
    if (pw * ph != soft_tokens) return SVLO_INTERNAL;
    size_t n_out;
    if (vis_checked_len(soft_tokens, hidden_size, &n_out)) return SVLO_LIMIT;
    memset(out, 0, n_out * sizeof(float));
    const float divisor = (float)(VIS_POOL * VIS_POOL);
    for (size_t p = 0; p < valid; ++p) {
        if (positions[2 * p] < 0 || positions[2 * p + 1] < 0) return SVLO_INTERNAL;
        size_t x = (size_t)positions[2 * p], y = (size_t)positions[2 * p + 1];
        size_t bin = x / VIS_POOL + pw * (y / VIS_POOL);
        if (bin >= soft_tokens) return SVLO_INTERNAL;
        const float *src = hidden + p * hidden_size;
        float *dst = out + bin * hidden_size;
        for (size_t c = 0; c < hidden_size; ++c) dst[c] += src[c];
    }
    const float scale = sqrtf((float)hidden_size);
    if (!isfinite(scale) || scale <= 0.0f) return SVLO_INTERNAL;
    for (size_t i = 0; i < n_out; ++i) out[i] = (out[i] / divisor) * scale;
    if (!vis_all_finite(out, n_out)) return SVLO_INTERNAL;
    return SVLO_OK;
}

enum {
    V_INPUT_LN = 0,
    V_POST_ATTN_LN,
    V_PRE_FF_LN,
    V_POST_FF_LN,
    V_Q,
    V_K,
    V_V,
    V_O,
    V_QNORM,
    V_KNORM,
    V_GATE,
    V_UP,
    V_DOWN
};
#define VW(layer, idx) weights[SVLO_VISION_GLOBAL_TENSORS + (size_t)(layer)*SVLO_VISION_LAYER_TENSORS + (idx)]

/* Work buffers of one encoder layer over `valid` rows. */
typedef struct {
    float *residual, *normed, *tmp, *tmp2, *query, *query_n, *key, *key_n, *value, *value_n,
        *attn, *gate, *up, *act;
} vis_layer_bufs;

static void vis_layer_free(vis_layer_bufs *b) {
    free(b->residual);
    free(b->normed);
    free(b->tmp);
    free(b->tmp2);
    free(b->query);
    free(b->query_n);
    free(b->key);
    free(b->key_n);
    free(b->value);
    free(b->value_n);
    free(b->attn);
    free(b->gate);
    free(b->up);
    free(b->act);
    memset(b, 0, sizeof(*b));
}

static int vis_layer_alloc(vis_layer_bufs *b, size_t n_hidden, size_t n_q, size_t n_kv,
                           size_t n_ff) {
    b->residual = (float *)malloc(n_hidden * sizeof(float));
    b->normed = (float *)malloc(n_hidden * sizeof(float));
    b->tmp = (float *)malloc(n_hidden * sizeof(float));
    b->tmp2 = (float *)malloc(n_hidden * sizeof(float));
    b->query = (float *)malloc(n_q * sizeof(float));
    b->query_n = (float *)malloc(n_q * sizeof(float));
    b->key = (float *)malloc(n_kv * sizeof(float));
    b->key_n = (float *)malloc(n_kv * sizeof(float));
    b->value = (float *)malloc(n_kv * sizeof(float));
    b->value_n = (float *)malloc(n_kv * sizeof(float));
    b->attn = (float *)malloc(n_q * sizeof(float));
    b->gate = (float *)malloc(n_ff * sizeof(float));
    b->up = (float *)malloc(n_ff * sizeof(float));
    b->act = (float *)malloc(n_ff * sizeof(float));
    if (b->residual && b->normed && b->tmp && b->tmp2 && b->query && b->query_n && b->key &&
        b->key_n && b->value && b->value_n && b->attn && b->gate && b->up && b->act)
        return 1;
    vis_layer_free(b);
    return 0;
}

/* One encoder layer (vision.rs:816-935) in place on hidden [valid, H]; inv
 * holds the head_dim / 4 axial frequencies. */
static int vis_layer(const svlo_vision_config *cfg, const float *const *weights, size_t l,
                     float *hidden, const int32_t *positions, size_t valid, const float *inv,
                     vis_layer_bufs *b) {
    const size_t H = (size_t)cfg->hidden_size, I = (size_t)cfg->intermediate_size;
    const size_t NH = (size_t)cfg->num_attention_heads, NKV = (size_t)cfg->num_key_value_heads;
    const size_t hd = (size_t)cfg->head_dim, qd = NH * hd, kd = NKV * hd;
    const size_t n_hidden = valid * H, n_ff = valid * I;
    const float eps = cfg->rms_norm_eps;
    int st;
    memcpy(b->residual, hidden, n_hidden * sizeof(float));
    if ((st = svlo_rms_norm_rows(hidden, VW(l, V_INPUT_LN), valid, H, eps, b->normed))) return st;
    if ((st = svlo_linear(b->normed, VW(l, V_Q), valid, H, qd, b->query))) return st;
    if ((st = svlo_linear(b->normed, VW(l, V_K), valid, H, kd, b->key))) return st;
    if ((st = svlo_linear(b->normed, VW(l, V_V), valid, H, kd, b->value))) return st;
    if ((st = svlo_rms_norm_rows(b->query, VW(l, V_QNORM), valid * NH, hd, eps, b->query_n)))
        return st;
    if ((st = svlo_rms_norm_rows(b->key, VW(l, V_KNORM), valid * NKV, hd, eps, b->key_n)))
        return st;
    if ((st = svlo_rms_norm_rows_unscaled(b->value, valid * NKV, hd, eps, b->value_n))) return st;
    if ((st = svlo_axial_rope(b->query_n, valid, NH, hd, positions, valid, inv, hd / 4))) return st;
    if ((st = svlo_axial_rope(b->key_n, valid, NKV, hd, positions, valid, inv, hd / 4))) return st;
    if ((st = svlo_bidirectional_attention(b->query_n, b->key_n, b->value_n, valid, NH, NKV, hd, -1,
                                           1.0f, b->attn)))
        return st;
    if ((st = svlo_linear(b->attn, VW(l, V_O), valid, qd, H, b->tmp))) return st;
    if ((st = svlo_rms_norm_rows(b->tmp, VW(l, V_POST_ATTN_LN), valid, H, eps, b->tmp2))) return st;
    svlo_add(b->residual, b->tmp2, n_hidden, hidden);

    memcpy(b->residual, hidden, n_hidden * sizeof(float));
    if ((st = svlo_rms_norm_rows(hidden, VW(l, V_PRE_FF_LN), valid, H, eps, b->normed))) return st;
    if ((st = svlo_linear(b->normed, VW(l, V_GATE), valid, H, I, b->gate))) return st;
    if ((st = svlo_linear(b->normed, VW(l, V_UP), valid, H, I, b->up))) return st;
    if ((st = svlo_geglu(b->gate, b->up, n_ff, b->act))) return st;
    if ((st = svlo_linear(b->act, VW(l, V_DOWN), valid, I, H, b->tmp))) return st;
    if ((st = svlo_rms_norm_rows(b->tmp, VW(l, V_POST_FF_LN), valid, H, eps, b->tmp2))) return st;
    svlo_add(b->residual, b->tmp2, n_hidden, hidden);
    return SVLO_OK;
}

int svlo_vision_layer(const svlo_vision_config *cfg, const float *const *weights, size_t layer,
                      const float *hidden_in, const int32_t *positions, size_t rows, float *out,
                      char *msg, size_t msg_len) {
    if (msg && msg_len) msg[0] = 0;
    if (layer >= (size_t)cfg->num_hidden_layers || rows == 0)
        return vis_fail(msg, msg_len, SVLO_INTERNAL, "vision layer %zu of %lld over %zu rows", layer,
                        (long long)cfg->num_hidden_layers, rows);
    const size_t H = (size_t)cfg->hidden_size, hd = (size_t)cfg->head_dim;
    size_t n_hidden, n_q, n_kv, n_ff;
    if (vis_checked_len(rows, H, &n_hidden) ||
        vis_checked_len(rows, (size_t)cfg->num_attention_heads * hd, &n_q) ||
        vis_checked_len(rows, (size_t)cfg->num_key_value_heads * hd, &n_kv) ||
        vis_checked_len(rows, (size_t)cfg->intermediate_size, &n_ff))
        return vis_fail(msg, msg_len, SVLO_LIMIT, "vision activation above the element cap");
    for (size_t p = 0; p < rows; ++p)
        if (positions[2 * p] < 0 || positions[2 * p + 1] < 0)
            return vis_fail(msg, msg_len, SVLO_INTERNAL, "vision patch position is negative");
    vis_layer_bufs b;
    float *inv = (float *)malloc((hd / 4 + 1) * sizeof(float));
    if (!inv || !vis_layer_alloc(&b, n_hidden, n_q, n_kv, n_ff)) {
        free(inv);
        return vis_fail(msg, msg_len, SVLO_LIMIT, "allocation failed");
    }
    int st = svlo_axial_inv_freq(hd, cfg->rope_theta, inv);
    if (st == SVLO_OK) {
        memcpy(out, hidden_in, n_hidden * sizeof(float));
        st = vis_layer(cfg, weights, layer, out, positions, rows, inv, &b);
    }
    if (st) vis_fail(msg, msg_len, st, "vision kernel failed with status %d (non-finite value or limit)", st);
    vis_layer_free(&b);
    free(inv);
    return st;
}

/* VisionModel::forward (vision.rs:742-959). */
int svlo_vision_forward(const svlo_vision_config *cfg, const float *const *weights,
                        size_t text_hidden, const float *pixel_values, const int32_t *positions,
                        size_t valid, size_t max_patches, size_t grid_width, size_t grid_height,
                        size_t soft_tokens, float *out_pooled, float *out_hidden, char *msg,
                        size_t msg_len) {
    if (msg && msg_len) msg[0] = 0;
    if (valid == 0) return vis_fail(msg, msg_len, SVLO_CORRUPT, "vision tower received zero real patches");
    if (valid > max_patches)
        return vis_fail(msg, msg_len, SVLO_INTERNAL,
                        "vision tower received more real patches than the padded tensor");
    const size_t H = (size_t)cfg->hidden_size, I = (size_t)cfg->intermediate_size;
    const size_t L = (size_t)cfg->num_hidden_layers, NH = (size_t)cfg->num_attention_heads;
    const size_t NKV = (size_t)cfg->num_key_value_heads, hd = (size_t)cfg->head_dim;
    const size_t qd = NH * hd, kd = NKV * hd;
    const size_t pos_size = (size_t)cfg->position_embedding_size;
    const float eps = cfg->rms_norm_eps;

    size_t n_patch, n_hidden, n_q, n_kv, n_ff, n_pool;
    if (vis_checked_len(valid, VIS_PATCH_VALUES, &n_patch) || vis_checked_len(valid, H, &n_hidden) ||
        vis_checked_len(valid, qd, &n_q) || vis_checked_len(valid, kd, &n_kv) ||
        vis_checked_len(valid, I, &n_ff) || vis_checked_len(soft_tokens, H, &n_pool))
        return vis_fail(msg, msg_len, SVLO_LIMIT, "vision activation above the element cap");

    int st = SVLO_OK;
    vis_layer_bufs b;
    memset(&b, 0, sizeof(b));
    float *scaled = (float *)malloc(n_patch * sizeof(float));
    float *hidden = (float *)malloc(n_hidden * sizeof(float));
    float *pooled = (float *)malloc((n_pool + 1) * sizeof(float));
    float *pooled_n = (float *)malloc((n_pool + 1) * sizeof(float));
    float *inv = (float *)malloc((hd / 4 + 1) * sizeof(float));
    if (!scaled || !hidden || !pooled || !pooled_n || !inv ||
        !vis_layer_alloc(&b, n_hidden, n_q, n_kv, n_ff)) {
        st = vis_fail(msg, msg_len, SVLO_LIMIT, "allocation failed");
        goto done;
    }

    /* vision.rs:767-777 patch scale and input projection. */
    for (size_t i = 0; i < n_patch; ++i) scaled[i] = 2.0f * (pixel_values[i] - 0.5f);
    if ((st = svlo_linear(scaled, weights[0], valid, VIS_PATCH_VALUES, H, hidden))) goto knl;

    /* vision.rs:779-809 two-axis position embeddings. */
    for (size_t p = 0; p < valid; ++p) {
        int32_t px = positions[2 * p], py = positions[2 * p + 1];
        if (px < 0 || py < 0) {
            st = vis_fail(msg, msg_len, SVLO_INTERNAL, "vision patch position is negative");
            goto done;
        }
        if ((size_t)px >= pos_size || (size_t)py >= pos_size) {
            st = vis_fail(msg, msg_len, SVLO_CORRUPT,
                          "vision patch position (%d, %d) is outside the %zu-entry table", px, py,
                          pos_size);
            goto done;
        }
        const float *xr = weights[1] + (size_t)px * H;
        const float *yr = weights[1] + pos_size * H + (size_t)py * H;
        float *dst = hidden + p * H;
        for (size_t c = 0; c < H; ++c) dst[c] += xr[c] + yr[c];
    }
    if (out_hidden) memcpy(out_hidden, hidden, n_hidden * sizeof(float));

    if ((st = svlo_axial_inv_freq(hd, cfg->rope_theta, inv))) goto knl;
    /* vision.rs:816-935 encoder layers. */
    for (size_t l = 0; l < L; ++l) {
        if ((st = vis_layer(cfg, weights, l, hidden, positions, valid, inv, &b))) goto knl;
        if (out_hidden) memcpy(out_hidden + (l + 1) * n_hidden, hidden, n_hidden * sizeof(float));
    }

    /* vision.rs:937-951 pool, unscaled norm, projection to the text width. */
    if ((st = svlo_pool_patches(hidden, positions, valid, grid_width, grid_height, soft_tokens, H,
                                pooled)))
        goto knl;
    if ((st = svlo_rms_norm_rows_unscaled(pooled, soft_tokens, H, eps, pooled_n))) goto knl;
    if ((st = svlo_linear(pooled_n, weights[SVLO_VISION_GLOBAL_TENSORS + L * SVLO_VISION_LAYER_TENSORS],
                          soft_tokens, H, text_hidden, out_pooled)))
        goto knl;
    if (!vis_all_finite(out_pooled, soft_tokens * text_hidden)) {
        st = vis_fail(msg, msg_len, SVLO_INTERNAL, "vision projection produced a non-finite soft token");
        goto done;
    }
    goto done;

knl:
    vis_fail(msg, msg_len, st, "vision kernel failed with status %d (non-finite value or limit)", st);
done:
    vis_layer_free(&b);
    free(scaled);
    free(hidden);
    free(pooled);
    free(pooled_n);
    free(inv);
    return st;
}
