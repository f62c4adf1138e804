/*
 * CPU oracle: a C restatement of the reference crate's scalar FP32 path.
 *
 * TEST INFRASTRUCTURE ONLY: the oracle for the HIP path, never part of the
 * product library. Built with -O2 -ffp-contract=off and no fast-math so that
 * every f32 operation is rounded in the same order as the Rust scalar code.
 *
 * Parity pins (tests/test_oracle_*.py):
 *  - every kernel below against the known-answer tests of
 *    src/tensor/kernels.rs:1151-1593 and closed forms;
 *  - svlo_text_forward against fixtures/model/tiny_text/golden.json, produced
 *    by the official Transformers implementation, at the reference tolerances
 *    of tests/text_embeddings.rs:83-230.
 */
#include "svl_oracle.h"

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* src/tensor/owned.rs MAX_TENSOR_ELEMENTS and text.rs:34 MAX_ACTIVATION_ELEMENTS. */
#define MAX_TENSOR_ELEMENTS ((size_t)1 << 30)
#define MAX_ACTIVATION_ELEMENTS ((size_t)1 << 28)
/* config.rs:27 */
#define MAX_TEXT_TOKENS 8192

static int all_finite(const float *v, size_t n) {
    for (size_t i = 0; i < n; ++i)
        if (!isfinite(v[i])) return 0;
    return 1;
}

/* kernels.rs:105-111 dot_scalar: sequential f32 accumulation. */
float svlo_dot(const float *a, const float *b, size_t n) {
    float sum = 0.0f;
    for (size_t i = 0; i < n; ++i) sum += a[i] * b[i];
    return sum;
}

/* kernels.rs:39-52 add_scalar. */
int svlo_add(const float *a, const float *b, size_t n, float *out) {
    if (n > MAX_TENSOR_ELEMENTS) return SVLO_LIMIT;
    for (size_t i = 0; i < n; ++i) out[i] = a[i] + b[i];
    return SVLO_OK;
}

/* kernels.rs:655-685 linear_into_scalar: out[r,c] = sum_k in[r,k] * w[c,k]. */
int svlo_linear(const float *input, const float *weight, size_t rows, size_t in_features,
                size_t out_features, float *out) {
    if (rows * out_features > MAX_TENSOR_ELEMENTS) return SVLO_LIMIT;
    for (size_t row = 0; row < rows; ++row) {
        const float *x = input + row * in_features;
        float *y = out + row * out_features;
        for (size_t col = 0; col < out_features; ++col) {
            const float *w = weight + col * in_features;
            float sum = 0.0f;
            for (size_t k = 0; k < in_features; ++k) sum += x[k] * w[k];
            y[col] = sum;
        }
    }
    if (!all_finite(out, rows * out_features)) return SVLO_INTERNAL;
    return SVLO_OK;
}

/* kernels.rs:234-260 matmul_into_scalar: C = A * B, row-major, k-outer accumulation. */
int svlo_matmul(const float *left, const float *right, size_t m, size_t k, size_t n, float *out) {
    if (m * n > MAX_TENSOR_ELEMENTS) return SVLO_LIMIT;
    memset(out, 0, m * n * sizeof(float));
    for (size_t row = 0; row < m; ++row) {
        for (size_t inner = 0; inner < k; ++inner) {
            float a = left[row * k + inner];
            const float *b = right + inner * n;
            float *c = out + row * n;
            for (size_t j = 0; j < n; ++j) c[j] += a * b[j];
        }
    }
    if (!all_finite(out, m * n)) return SVLO_INTERNAL;
    return SVLO_OK;
}

/* kernels.rs:688-720 validate_rms_norm_rows (weight length is the caller's contract). */
static int validate_rms_rows(size_t rows, size_t width, float eps) {
    if (width == 0) return SVLO_INTERNAL;
    if (!isfinite(eps) || eps < 0.0f) return SVLO_INTERNAL;
    if (rows * width > MAX_TENSOR_ELEMENTS) return SVLO_LIMIT;
    return SVLO_OK;
}

/* kernels.rs:743-776 rms_norm_rows_scalar. */
int svlo_rms_norm_rows(const float *input, const float *weight, size_t rows, size_t width,
                       float eps, float *out) {
    int st = validate_rms_rows(rows, width, eps);
    if (st) return st;
    for (size_t row = 0; row < rows; ++row) {
        const float *x = input + row * width;
        float *y = out + row * width;
        float sum = 0.0f;
        for (size_t i = 0; i < width; ++i) {
            if (!isfinite(x[i])) return SVLO_INTERNAL;
            sum += x[i] * x[i];
        }
        if (!isfinite(sum)) return SVLO_INTERNAL;
        float inverse = 1.0f / sqrtf(sum / (float)width + eps);
        for (size_t i = 0; i < width; ++i) y[i] = x[i] * inverse * weight[i];
    }
    if (!all_finite(out, rows * width)) return SVLO_INTERNAL;
    return SVLO_OK;
}

/* kernels.rs:825-857 rms_norm_rows_unscaled_scalar. */
int svlo_rms_norm_rows_unscaled(const float *input, size_t rows, size_t width, float eps,
                                float *out) {
    int st = validate_rms_rows(rows, width, eps);
    if (st) return st;
    for (size_t row = 0; row < rows; ++row) {
        const float *x = input + row * width;
        float *y = out + row * width;
        float sum = 0.0f;
        for (size_t i = 0; i < width; ++i) {
            if (!isfinite(x[i])) return SVLO_INTERNAL;
            sum += x[i] * x[i];
        }
        if (!isfinite(sum)) return SVLO_INTERNAL;
        float inverse = 1.0f / sqrtf(sum / (float)width + eps);
        for (size_t i = 0; i < width; ++i) y[i] = x[i] * inverse;
    }
    if (!all_finite(out, rows * width)) return SVLO_INTERNAL;
    return SVLO_OK;
}

/* kernels.rs:267-321 softmax: max-subtract, exp, divide by the sum. */
int svlo_softmax(const float *values, size_t n, float *out) {
    if (n == 0) return SVLO_INTERNAL;
    if (n > MAX_TENSOR_ELEMENTS) return SVLO_LIMIT;
    float maximum = -INFINITY;
    for (size_t i = 0; i < n; ++i) {
        if (isnan(values[i])) return SVLO_INTERNAL;
        if (values[i] > maximum) maximum = values[i];
    }
    if (maximum == -INFINITY) return SVLO_INTERNAL;
    if (maximum == INFINITY) {
        size_t count = 0;
        for (size_t i = 0; i < n; ++i)
            if (values[i] == INFINITY) ++count;
        float probability = 1.0f / (float)count;
        for (size_t i = 0; i < n; ++i) out[i] = values[i] == INFINITY ? probability : 0.0f;
        return SVLO_OK;
    }
    float sum = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        float e = expf(values[i] - maximum);
        sum += e;
        out[i] = e;
    }
    if (sum == 0.0f || !isfinite(sum)) return SVLO_INTERNAL;
    for (size_t i = 0; i < n; ++i) out[i] /= sum;
    return SVLO_OK;
}

/* kernels.rs:380-383 gelu_tanh_value: 0.5*v*(1+tanh(0.7978846*(v+0.044715*v^3))). */
float svlo_gelu_tanh_value(float v) {
    float cubic = v * v * v;
    return 0.5f * v * (1.0f + tanhf(0.7978846f * (v + 0.044715f * cubic)));
}

/* kernels.rs:386-388 gelu_tanh. */
void svlo_gelu_tanh(const float *values, size_t n, float *out) {
    for (size_t i = 0; i < n; ++i) out[i] = svlo_gelu_tanh_value(values[i]);
}

/* kernels.rs:391-400 geglu: gelu(gate) * up. */
int svlo_geglu(const float *gate, const float *up, size_t n, float *out) {
    if (n > MAX_TENSOR_ELEMENTS) return SVLO_LIMIT;
    for (size_t i = 0; i < n; ++i) out[i] = svlo_gelu_tanh_value(gate[i]) * up[i];
    return SVLO_OK;
}

/* kernels.rs:424-444 l2_normalize_scalar. */
int svlo_l2_normalize(const float *input, size_t n, float *out) {
    if (n == 0) return SVLO_INTERNAL;
    if (n > MAX_TENSOR_ELEMENTS) return SVLO_LIMIT;
    float sum = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        if (!isfinite(input[i])) return SVLO_INTERNAL;
        sum += input[i] * input[i];
    }
    if (!isfinite(sum) || sum <= 0.0f) return SVLO_INTERNAL;
    float inverse = 1.0f / sqrtf(sum);
    for (size_t i = 0; i < n; ++i) out[i] = input[i] * inverse;
    return SVLO_OK;
}

/* kernels.rs:892-909 mean_pool_scalar: row-ordered sums times 1/rows. */
int svlo_mean_pool(const float *values, size_t rows, size_t width, float *out) {
    if (rows == 0) return SVLO_INTERNAL;
    if (width > MAX_TENSOR_ELEMENTS) return SVLO_LIMIT;
    for (size_t c = 0; c < width; ++c) out[c] = 0.0f;
    for (size_t r = 0; r < rows; ++r)
        for (size_t c = 0; c < width; ++c) out[c] += values[r * width + c];
    float inverse = 1.0f / (float)rows;
    for (size_t c = 0; c < width; ++c) {
        out[c] *= inverse;
        if (!isfinite(out[c])) return SVLO_INTERNAL;
    }
    return SVLO_OK;
}

/* kernels.rs:916-927 truncate_and_normalize. */
int svlo_truncate_and_normalize(const float *values, size_t n, size_t dim, float *out) {
    if (dim == 0) return SVLO_INTERNAL;
    if (dim > n) return SVLO_INTERNAL;
    return svlo_l2_normalize(values, dim, out);
}

/* kernels.rs:991-1010 rope_inv_freq: 1 / base^((2j)/head_dim) in f32. */
int svlo_rope_inv_freq(size_t head_dim, float base, float *out) {
    if (head_dim == 0 || head_dim % 2) return SVLO_INTERNAL;
    if (!isfinite(base) || base <= 1.0f) return SVLO_INTERNAL;
    size_t half = head_dim / 2;
    for (size_t pair = 0; pair < half; ++pair) {
        float exponent = (float)(2 * pair) / (float)head_dim;
        out[pair] = 1.0f / powf(base, exponent);
    }
    return SVLO_OK;
}

/* kernels.rs:936-988 rope_with_inv_freq: rotate-half pairing j with j + head_dim/2. */
int svlo_rope_with_inv_freq(float *values, size_t seq_len, size_t num_heads, size_t head_dim,
                            const float *inv_freq, size_t n_inv_freq, size_t position_offset) {
    if (head_dim == 0 || head_dim % 2) return SVLO_INTERNAL;
    if (n_inv_freq != head_dim / 2) return SVLO_INTERNAL;
    size_t half = head_dim / 2;
    for (size_t position = 0; position < seq_len; ++position) {
        size_t absolute = position_offset + position;
        for (size_t head = 0; head < num_heads; ++head) {
            size_t offset = (position * num_heads + head) * head_dim;
            for (size_t pair = 0; pair < half; ++pair) {
                float angle = (float)absolute * inv_freq[pair];
                float sine = sinf(angle);
                float cosine = cosf(angle);
                float first = values[offset + pair];
                float second = values[offset + pair + half];
                values[offset + pair] = first * cosine - second * sine;
                values[offset + pair + half] = first * sine + second * cosine;
            }
        }
    }
    if (!all_finite(values, seq_len * num_heads * head_dim)) return SVLO_INTERNAL;
    return SVLO_OK;
}

/*
 * kernels.rs:1037-1135 bidirectional_attention: query head h reads key/value
 * head h / (num_heads / num_kv_heads); window |i - j| <= r or full; scores are
 * dot * scale, softmax over the window, then p-weighted value rows summed in
 * key order, skipping exact zeros.
 */
int svlo_bidirectional_attention(const float *q, const float *k, const float *v, size_t seq_len,
                                 size_t num_heads, size_t num_kv_heads, size_t head_dim,
                                 int64_t sliding_window, float scale, float *out) {
    if (head_dim == 0) return SVLO_INTERNAL;
    if (num_heads == 0 || num_kv_heads == 0) return SVLO_INTERNAL;
    if (num_heads % num_kv_heads) return SVLO_INTERNAL;
    if (!isfinite(scale)) return SVLO_INTERNAL;
    size_t query_len = seq_len * num_heads * head_dim;
    if (query_len > MAX_TENSOR_ELEMENTS) return SVLO_LIMIT;
    if (seq_len == 0) return SVLO_OK;
    size_t groups = num_heads / num_kv_heads;
    float *scores = (float *)malloc(seq_len * sizeof(float));
    float *probs = (float *)malloc(seq_len * sizeof(float));
    if (!scores || !probs) {
        free(scores);
        free(probs);
        return SVLO_LIMIT;
    }
    memset(out, 0, query_len * sizeof(float));
    int st = SVLO_OK;
    for (size_t position = 0; position < seq_len && st == SVLO_OK; ++position) {
        size_t start, end;
        if (sliding_window >= 0) {
            size_t w = (size_t)sliding_window;
            start = position > w ? position - w : 0;
            end = position + w < seq_len - 1 ? position + w : seq_len - 1;
        } else {
            start = 0;
            end = seq_len - 1;
        }
        size_t width = end - start + 1;
        for (size_t head = 0; head < num_heads; ++head) {
            size_t key_head = head / groups;
            const float *qrow = q + (position * num_heads + head) * head_dim;
            for (size_t c = 0; c < width; ++c) {
                size_t off = start + c;
                const float *krow = k + (off * num_kv_heads + key_head) * head_dim;
                float score = svlo_dot(qrow, krow, head_dim) * scale;
                if (!isfinite(score)) {
                    st = SVLO_INTERNAL;
                    break;
                }
                scores[c] = score;
            }
            if (st) break;
            st = svlo_softmax(scores, width, probs);
            if (st) break;
            float *orow = out + (position * num_heads + head) * head_dim;
            for (size_t c = 0; c < width; ++c) {
                float p = probs[c];
                if (p == 0.0f) continue;
                const float *vrow = v + ((start + c) * num_kv_heads + key_head) * head_dim;
                for (size_t d = 0; d < head_dim; ++d) orow[d] += p * vrow[d];
            }
        }
    }
    free(scores);
    free(probs);
    if (st) return st;
    if (!all_finite(out, query_len)) return SVLO_INTERNAL;
    return SVLO_OK;
}

/* ------------------------------------------------------------------------- */
/* Text forward pass: src/model/text.rs:182-538.                              */

static int fail(char *msg, size_t msg_len, int code, const char *fmt, ...) {
    if (msg && msg_len) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(msg, msg_len, fmt, ap);
        va_end(ap);
    }
    return code;
}

/* text.rs:629-639 checked_len against MAX_ACTIVATION_ELEMENTS. */
static int checked_len(size_t rows, size_t width, size_t *out) {
    if (width != 0 && rows > SIZE_MAX / width) return SVLO_LIMIT;
    size_t n = rows * width;
    if (n > MAX_ACTIVATION_ELEMENTS) return SVLO_LIMIT;
    *out = n;
    return SVLO_OK;
}

#define W_EMBED 0
#define W_OUTPROJ 1
#define W_NORM 2
#define W_PLE_MODEL 3
#define W_PLE_NORM 4
enum {
    L_INPUT_LN = 0,
    L_POST_ATTN_LN,
    L_PRE_FF_LN,
    L_POST_FF_LN,
    L_SCALAR,
    L_GATE,
    L_UP,
    L_DOWN,
    L_PLE_GATE,
    L_PLE_PROJ,
    L_POST_PLE_LN,
    L_Q,
    L_K,
    L_V,
    L_O,
    L_QNORM,
    L_KNORM
};

#define LW(layer, idx) weights[SVLO_GLOBAL_TENSORS + (size_t)(layer)*SVLO_LAYER_TENSORS + (idx)]

int svlo_text_forward(const svlo_text_config *cfg, const float *const *weights,
                      const uint32_t *ids, size_t seq, const float *features,
                      size_t feature_start, size_t feature_count, size_t features_len,
                      float *out_projected, float *out_pooled, float *out_normalized,
                      float *out_hidden, char *msg, size_t msg_len) {
    if (msg && msg_len) msg[0] = 0;
    /* text.rs:188-202 */
    if (seq == 0) return fail(msg, msg_len, SVLO_CORRUPT, "cannot embed an empty token sequence");
    if (seq > MAX_TEXT_TOKENS)
        return fail(msg, msg_len, SVLO_LIMIT, "sequence has %zu tokens, above the %d-token context",
                    seq, MAX_TEXT_TOKENS);
    if (seq > (size_t)cfg->max_position_embeddings)
        return fail(msg, msg_len, SVLO_LIMIT, "sequence has %zu tokens, above the declared positions",
                    seq);

    const size_t H = (size_t)cfg->hidden_size;
    const size_t P = (size_t)cfg->hidden_size_per_layer_input;
    const size_t L = (size_t)cfg->num_hidden_layers;
    const size_t E = (size_t)cfg->embedding_dim;
    const size_t I = (size_t)cfg->intermediate_size;
    const size_t NH = (size_t)cfg->num_attention_heads;
    const float eps = cfg->rms_norm_eps;
    /* config.rs:241-242 */
    const float embedding_scale = sqrtf((float)H);
    const float ple_scale = 1.0f / embedding_scale;

    size_t n_hidden, n_ple, n_ff;
    if (checked_len(seq, H, &n_hidden)) return fail(msg, msg_len, SVLO_LIMIT, "embedding buffer");
    if (checked_len(L, P, &n_ple) || checked_len(seq, n_ple, &n_ple))
        return fail(msg, msg_len, SVLO_LIMIT, "per-layer projection buffer");
    if (checked_len(seq, I, &n_ff)) return fail(msg, msg_len, SVLO_LIMIT, "feed-forward buffer");

    size_t max_q = 0, max_kv = 0;
    for (size_t l = 0; l < L; ++l) {
        size_t qd = NH * (size_t)cfg->head_dim[l];
        size_t kd = (size_t)cfg->num_kv_heads[l] * (size_t)cfg->head_dim[l];
        if (qd > max_q) max_q = qd;
        if (kd > max_kv) max_kv = kd;
    }
    size_t max_hd = 0;
    for (size_t l = 0; l < L; ++l)
        if ((size_t)cfg->head_dim[l] > max_hd) max_hd = (size_t)cfg->head_dim[l];

    int st = SVLO_OK;
    float *hidden = (float *)calloc(n_hidden, sizeof(float));
    float *residual = (float *)malloc(n_hidden * sizeof(float));
    float *normed = (float *)malloc(n_hidden * sizeof(float));
    float *tmp_h = (float *)malloc(n_hidden * sizeof(float));
    float *tmp_h2 = (float *)malloc(n_hidden * sizeof(float));
    float *per_layer_raw = (float *)malloc(n_ple * sizeof(float));
    float *per_layer = (float *)malloc(n_ple * sizeof(float));
    float *query = (float *)malloc(seq * max_q * sizeof(float));
    float *query_n = (float *)malloc(seq * max_q * sizeof(float));
    float *key = (float *)malloc(seq * max_kv * sizeof(float));
    float *key_n = (float *)malloc(seq * max_kv * sizeof(float));
    float *value = (float *)malloc(seq * max_kv * sizeof(float));
    float *value_n = (float *)malloc(seq * max_kv * sizeof(float));
    float *attn = (float *)malloc(seq * max_q * sizeof(float));
    float *gate = (float *)malloc(n_ff * sizeof(float));
    float *up = (float *)malloc(n_ff * sizeof(float));
    float *act = (float *)malloc(n_ff * sizeof(float));
    float *pgate = (float *)malloc(seq * P * sizeof(float));
    float *pgated = (float *)malloc(seq * P * sizeof(float));
    float *inv_full = (float *)malloc(max_hd * sizeof(float));
    float *inv_slide = (float *)malloc(max_hd * sizeof(float));
    if (!hidden || !residual || !normed || !tmp_h || !tmp_h2 || !per_layer_raw || !per_layer ||
        !query || !query_n || !key || !key_n || !value || !value_n || !attn || !gate || !up ||
        !act || !pgate || !pgated || !inv_full || !inv_slide) {
        st = fail(msg, msg_len, SVLO_LIMIT, "allocation failed");
        goto done;
    }

    /* text.rs:209-224 embedding gather scaled by sqrt(H). */
    for (size_t row = 0; row < seq; ++row) {
        size_t index = ids[row];
        if (index >= (size_t)cfg->vocab_size) {
            st = fail(msg, msg_len, SVLO_CORRUPT, "token id %u is outside the vocabulary",
                      ids[row]);
            goto done;
        }
        const float *src = weights[W_EMBED] + index * H;
        for (size_t c = 0; c < H; ++c) hidden[row * H + c] = src[c] * embedding_scale;
    }

    /* text.rs:226-275 multimodal feature overwrite. */
    if (features) {
        if (feature_count == 0) {
            st = fail(msg, msg_len, SVLO_CORRUPT, "multimodal feature replacement requires at least one token");
            goto done;
        }
        size_t end = feature_start + feature_count;
        if (end < feature_start) {
            st = fail(msg, msg_len, SVLO_LIMIT, "multimodal feature range overflow");
            goto done;
        }
        if (end > seq) {
            st = fail(msg, msg_len, SVLO_CORRUPT, "multimodal feature range is outside the sequence");
            goto done;
        }
        if (features_len != feature_count * H) {
            st = fail(msg, msg_len, SVLO_CORRUPT, "multimodal features have the wrong length");
            goto done;
        }
        if (cfg->pad_token_id < 0) {
            st = fail(msg, msg_len, SVLO_UNSUPPORTED, "model has no padding token for multimodal inputs");
            goto done;
        }
        size_t pad = (size_t)cfg->pad_token_id;
        if (pad >= (size_t)cfg->vocab_size) {
            st = fail(msg, msg_len, SVLO_CORRUPT, "padding token id is outside the vocabulary");
            goto done;
        }
        const float *pad_emb = weights[W_EMBED] + pad * H;
        for (size_t row = feature_start; row < end; ++row)
            for (size_t c = 0; c < H; ++c) hidden[row * H + c] = pad_emb[c] * embedding_scale;
        for (size_t off = 0; off < feature_count; ++off)
            memcpy(hidden + (feature_start + off) * H, features + off * H, H * sizeof(float));
        if (!all_finite(hidden, n_hidden)) {
            st = fail(msg, msg_len, SVLO_INTERNAL, "multimodal features contain a non-finite activation");
            goto done;
        }
    }

    if (out_hidden) memcpy(out_hidden, hidden, n_hidden * sizeof(float));

    /* text.rs:285-306 projection-only per-layer embeddings. */
    if ((st = svlo_linear(hidden, weights[W_PLE_MODEL], seq, H, L * P, per_layer_raw))) goto knl;
    for (size_t i = 0; i < n_ple; ++i) per_layer_raw[i] *= ple_scale;
    if ((st = svlo_rms_norm_rows(per_layer_raw, weights[W_PLE_NORM], seq * L, P, eps, per_layer)))
        goto knl;

    /* text.rs:314-333 RoPE inverse frequencies per layer type (config.rs:366-388). */
    {
        size_t full_hd = 0, slide_hd = 0;
        int has_full = 0, has_slide = 0;
        for (size_t l = 0; l < L; ++l) {
            if (cfg->layer_type[l] == 1 && !has_full) {
                has_full = 1;
                full_hd = (size_t)cfg->head_dim[l];
            }
            if (cfg->layer_type[l] == 0 && !has_slide) {
                has_slide = 1;
                slide_hd = (size_t)cfg->head_dim[l];
            }
        }
        if (has_full && (st = svlo_rope_inv_freq(full_hd, cfg->full_rope_theta, inv_full))) goto knl;
        if (has_slide && (st = svlo_rope_inv_freq(slide_hd, cfg->sliding_rope_theta, inv_slide)))
            goto knl;
    }

    /* text.rs:335-518 encoder layers. */
    for (size_t l = 0; l < L; ++l) {
        const size_t hd = (size_t)cfg->head_dim[l];
        const size_t nkv = (size_t)cfg->num_kv_heads[l];
        const size_t qd = NH * hd, kd = nkv * hd;
        const int full = cfg->layer_type[l] == 1;

        memcpy(residual, hidden, n_hidden * sizeof(float));
        if ((st = svlo_rms_norm_rows(hidden, LW(l, L_INPUT_LN), seq, H, eps, normed))) goto knl;
        if ((st = svlo_linear(normed, LW(l, L_Q), seq, H, qd, query))) goto knl;
        if ((st = svlo_linear(normed, LW(l, L_K), seq, H, kd, key))) goto knl;
        if ((st = svlo_linear(normed, LW(l, L_V), seq, H, kd, value))) goto knl;
        if ((st = svlo_rms_norm_rows(query, LW(l, L_QNORM), seq * NH, hd, eps, query_n))) goto knl;
        if ((st = svlo_rms_norm_rows(key, LW(l, L_KNORM), seq * nkv, hd, eps, key_n))) goto knl;
        if ((st = svlo_rms_norm_rows_unscaled(value, seq * nkv, hd, eps, value_n))) goto knl;
        const float *inv = full ? inv_full : inv_slide;
        if ((st = svlo_rope_with_inv_freq(query_n, seq, NH, hd, inv, hd / 2, 0))) goto knl;
        if ((st = svlo_rope_with_inv_freq(key_n, seq, nkv, hd, inv, hd / 2, 0))) goto knl;
        if ((st = svlo_bidirectional_attention(query_n, key_n, value_n, seq, NH, nkv, hd,
                                               full ? -1 : cfg->sliding_window, 1.0f, attn)))
            goto knl;
        if ((st = svlo_linear(attn, LW(l, L_O), seq, qd, H, tmp_h))) goto knl;
        if ((st = svlo_rms_norm_rows(tmp_h, LW(l, L_POST_ATTN_LN), seq, H, eps, tmp_h2))) goto knl;
        svlo_add(residual, tmp_h2, n_hidden, hidden);

        memcpy(residual, hidden, n_hidden * sizeof(float));
        if ((st = svlo_rms_norm_rows(hidden, LW(l, L_PRE_FF_LN), seq, H, eps, normed))) goto knl;
        if ((st = svlo_linear(normed, LW(l, L_GATE), seq, H, I, gate))) goto knl;
        if ((st = svlo_linear(normed, LW(l, L_UP), seq, H, I, up))) goto knl;
        svlo_geglu(gate, up, n_ff, act);
        if ((st = svlo_linear(act, LW(l, L_DOWN), seq, I, H, tmp_h))) goto knl;
        if ((st = svlo_rms_norm_rows(tmp_h, LW(l, L_POST_FF_LN), seq, H, eps, tmp_h2))) goto knl;
        svlo_add(residual, tmp_h2, n_hidden, hidden);

        memcpy(residual, hidden, n_hidden * sizeof(float));
        if ((st = svlo_linear(hidden, LW(l, L_PLE_GATE), seq, H, P, pgate))) goto knl;
        svlo_gelu_tanh(pgate, seq * P, pgate);
        for (size_t row = 0; row < seq; ++row) {
            const float *g = pgate + row * P;
            const float *in = per_layer + row * L * P + l * P;
            float *dst = pgated + row * P;
            for (size_t c = 0; c < P; ++c) dst[c] = g[c] * in[c];
        }
        if ((st = svlo_linear(pgated, LW(l, L_PLE_PROJ), seq, P, H, tmp_h))) goto knl;
        if ((st = svlo_rms_norm_rows(tmp_h, LW(l, L_POST_PLE_LN), seq, H, eps, tmp_h2))) goto knl;
        svlo_add(residual, tmp_h2, n_hidden, hidden);
        const float layer_scalar = LW(l, L_SCALAR)[0];
        for (size_t i = 0; i < n_hidden; ++i) hidden[i] *= layer_scalar;

        if (out_hidden) memcpy(out_hidden + (l + 1) * n_hidden, hidden, n_hidden * sizeof(float));
    }

    /* text.rs:520-531 final norm, projection, mean pool, L2 normalisation. */
    if ((st = svlo_rms_norm_rows(hidden, weights[W_NORM], seq, H, eps, normed))) goto knl;
    if ((st = svlo_linear(normed, weights[W_OUTPROJ], seq, H, E, out_projected))) goto knl;
    if ((st = svlo_mean_pool(out_projected, seq, E, out_pooled))) goto knl;
    if ((st = svlo_l2_normalize(out_pooled, E, out_normalized))) goto knl;
    goto done;

knl:
    fail(msg, msg_len, st, "kernel failed with status %d (non-finite value or limit)", st);
done:
    free(hidden);
    free(residual);
    free(normed);
    free(tmp_h);
    free(tmp_h2);
    free(per_layer_raw);
    free(per_layer);
    free(query);
    free(query_n);
    free(key);
    free(key_n);
    free(value);
    free(value_n);
    free(attn);
    free(gate);
    free(up);
    free(act);
    free(pgate);
    free(pgated);
    free(inv_full);
    free(inv_slide);
    return st;
}
