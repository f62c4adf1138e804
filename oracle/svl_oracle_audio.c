/*
 * CPU oracle, audio tower: a C restatement of src/model/audio.rs.
 *
 * TEST INFRASTRUCTURE ONLY: the oracle for the HIP audio path, never part of
 * the product library. Same build rules as svl_oracle.c (-O2,
 * -ffp-contract=off, no fast-math); the reference's f32 operations are
 * evaluated in its order with the platform libm (expf, logf, tanhf, sinf,
 * cosf, sqrtf), and its f64 constants are computed in double and rounded
 * once, as the Rust code does.
 *
 * Parity pins (tests/test_oracle_audio.py): the official tiny audio fixture
 * (fixtures/model/tiny_audio/golden.json, produced by Transformers): SSCP
 * output, both layer outputs, the projected audio features and the final
 * embedding through the text oracle, at the tolerances of
 * tests/audio_tiny.rs:78-200; plus the unit tests of audio.rs:1692-1740 and
 * closed forms for the activations and the relative position table.
 */
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "svl_oracle.h"

#define AU_MAX_ACTIVATION_ELEMENTS ((size_t)1 << 28)
#define AU_FEATURE_SIZE 128
/* std::f64::consts::LN_2 and E */
#define AU_LN_2 0.693147180559945309417232121458176568
#define AU_E 2.71828182845904523536028747135266250

static int au_fail(char *msg, size_t msg_len, int code, const char *fmt, ...) {
    if (msg && msg_len) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(msg, msg_len, fmt, ap);
        va_end(ap);
    }
    return code;
}

/* audio.rs:1339-1347 */
float svlo_clamp_value(float value, float minimum, float maximum) {
    if (value < minimum) return minimum;
    if (value > maximum) return maximum;
    return value;
}

/* audio.rs:1349-1355 */
float svlo_silu_value(float value) {
    if (value >= 0.0f) return value / (1.0f + expf(-value));
    return value * expf(value) / (1.0f + expf(value));
}

/* audio.rs:1357-1364 */
float svlo_sigmoid_value(float value) {
    if (value >= 0.0f) return 1.0f / (1.0f + expf(-value));
    float e = expf(value);
    return e / (1.0f + e);
}

/* audio.rs:1366-1372 */
float svlo_softplus_value(float value) {
    if (value > 20.0f) return value;
    return logf(1.0f + expf(value));
}

/* audio.rs:558-601 ClippedLinear::apply; bounds = {in_min, in_max, out_min, out_max}. */
int svlo_clipped_linear(const float *input, const float *weight, const float *bounds,
                        size_t rows, size_t in_features, size_t out_features, float *out) {
    if (rows * out_features > AU_MAX_ACTIVATION_ELEMENTS) return SVLO_LIMIT;
    for (size_t r = 0; r < rows; ++r) {
        const float *x = input + r * in_features;
        for (size_t c = 0; c < out_features; ++c) {
            const float *w = weight + c * in_features;
            float sum = 0.0f;
            for (size_t k = 0; k < in_features; ++k)
                sum += svlo_clamp_value(x[k], bounds[0], bounds[1]) * w[k];
            out[r * out_features + c] = svlo_clamp_value(sum, bounds[2], bounds[3]);
        }
    }
    for (size_t i = 0; i < rows * out_features; ++i)
        if (!isfinite(out[i])) return SVLO_INTERNAL;
    return SVLO_OK;
}

/* audio.rs:1435-1446 clamp_if_needed (in place on a copy). */
static void au_clamp_if_needed(float *values, size_t n, float bound) {
    int any = 0;
    for (size_t i = 0; i < n; ++i)
        if (fabsf(values[i]) > bound) any = 1;
    if (!any) return;
    for (size_t i = 0; i < n; ++i) values[i] = svlo_clamp_value(values[i], -bound, bound);
}

/* audio.rs:1257-1288 sinusoidal relative positions, out [positions, hidden]. */
int svlo_audio_position_embeddings(size_t hidden, size_t positions, float *out) {
    if (hidden % 2) return SVLO_INTERNAL;
    size_t timescales = hidden / 2;
    if (timescales == 0) return SVLO_INTERNAL;
    double increment = timescales > 1 ? log(10000.0) / (double)(timescales - 1) : 0.0;
    float *inverse = (float *)malloc(timescales * sizeof(float));
    if (!inverse) return SVLO_LIMIT;
    for (size_t i = 0; i < timescales; ++i) inverse[i] = (float)exp(-(double)i * increment);
    for (size_t p = 0; p < positions; ++p) {
        float id = (float)(positions - 1 - p);
        for (size_t i = 0; i < timescales; ++i) {
            float scaled = id * inverse[i];
            out[p * hidden + i] = sinf(scaled);
            out[p * hidden + timescales + i] = cosf(scaled);
        }
    }
    free(inverse);
    return SVLO_OK;
}

/* audio.rs:1290-1322 normalize_subsample: LayerNorm without bias, then ReLU. */
static int au_normalize_subsample(float *values, const float *weight, size_t width, float eps) {
    float sum = 0.0f;
    for (size_t i = 0; i < width; ++i) {
        if (!isfinite(values[i])) return SVLO_INTERNAL;
        sum += values[i];
    }
    float mean = sum / (float)width;
    float variance = 0.0f;
    for (size_t i = 0; i < width; ++i) {
        float d = values[i] - mean;
        variance += d * d;
    }
    variance /= (float)width;
    float inverse = 1.0f / sqrtf(variance + eps);
    if (!isfinite(inverse)) return SVLO_INTERNAL;
    for (size_t i = 0; i < width; ++i) {
        float v = (values[i] - mean) * inverse * weight[i];
        values[i] = fmaxf(v, 0.0f);
    }
    return SVLO_OK;
}

/* Layer weights inside the tensor_shapes order (audio.rs:394-498). */
enum {
    A_FF_PRE = 0, A_FF_POST = 1, A_FF_W1 = 2, A_FF_W2 = 3, A_FF_B1 = 4, A_FF_B2 = 8,
    A_FF1 = 0, A_FF2 = 12,
    A_ATT = 24, /* + 5 * projection (q, k, v, post): weight, then 4 bounds */
    A_RELK = 44, A_PDS = 45, A_LC_PRE = 46, A_LC_START = 47, A_LC_END = 48,
    A_LC_START_B = 49, A_LC_END_B = 53, A_LC_DW = 57, A_LC_NORM = 58,
    A_NORM_PRE_ATTN = 59, A_NORM_POST_ATTN = 60, A_NORM_OUT = 61
};
#define AW(l, i) weights[SVLO_AUDIO_GLOBAL_TENSORS + (size_t)(l)*SVLO_AUDIO_LAYER_TENSORS + (i)]

/* Four scalar bounds starting at tensor index i of layer l. */
static void au_bounds(const float *const *weights, size_t l, size_t i, float b[4]) {
    for (int k = 0; k < 4; ++k) b[k] = AW(l, i + (size_t)k)[0];
}

/* audio.rs:1374-1433 feed_forward; out may not alias hidden. */
static int au_feed_forward(const svlo_audio_config *c, const float *const *weights, size_t l,
                           size_t base, const float *hidden, size_t rows, float *tmp_h,
                           float *tmp_i, float *tmp_i2, float *out) {
    const size_t H = (size_t)c->hidden_size, I = (size_t)c->intermediate_size;
    int st;
    float b1[4], b2[4];
    au_bounds(weights, l, base + A_FF_B1, b1);
    au_bounds(weights, l, base + A_FF_B2, b2);
    memcpy(tmp_h, hidden, rows * H * sizeof(float));
    au_clamp_if_needed(tmp_h, rows * H, c->gradient_clipping);
    if ((st = svlo_rms_norm_rows(tmp_h, AW(l, base + A_FF_PRE), rows, H, c->rms_norm_eps, out)))
        return st;
    if ((st = svlo_clipped_linear(out, AW(l, base + A_FF_W1), b1, rows, H, I, tmp_i))) return st;
    for (size_t i = 0; i < rows * I; ++i) {
        float s = svlo_silu_value(tmp_i[i]);
        if (!isfinite(s)) return SVLO_INTERNAL;
        tmp_i2[i] = s;
    }
    if ((st = svlo_clipped_linear(tmp_i2, AW(l, base + A_FF_W2), b2, rows, I, H, tmp_h))) return st;
    au_clamp_if_needed(tmp_h, rows * H, c->gradient_clipping);
    if ((st = svlo_rms_norm_rows(tmp_h, AW(l, base + A_FF_POST), rows, H, c->rms_norm_eps, out)))
        return st;
    for (size_t i = 0; i < rows * H; ++i) {
        float scaled = out[i] * c->residual_weight;
        float sum = hidden[i] + scaled;
        if (!isfinite(sum)) return SVLO_INTERNAL;
        out[i] = sum;
    }
    return SVLO_OK;
}

/* audio.rs:1448-1527 light_conv; out may not alias hidden. */
static int au_light_conv(const svlo_audio_config *c, const float *const *weights, size_t l,
                         const float *hidden, size_t rows, float *tmp_h, float *tmp_2h,
                         float *tmp_h2, float *out) {
    const size_t H = (size_t)c->hidden_size, K = (size_t)c->conv_kernel_size;
    int st;
    float bs[4], be[4];
    au_bounds(weights, l, A_LC_START_B, bs);
    au_bounds(weights, l, A_LC_END_B, be);
    if ((st = svlo_rms_norm_rows(hidden, AW(l, A_LC_PRE), rows, H, c->rms_norm_eps, tmp_h))) return st;
    if ((st = svlo_clipped_linear(tmp_h, AW(l, A_LC_START), bs, rows, H, 2 * H, tmp_2h))) return st;
    for (size_t r = 0; r < rows; ++r)
        for (size_t col = 0; col < H; ++col) {
            float first = tmp_2h[r * 2 * H + col], second = tmp_2h[r * 2 * H + H + col];
            float v = first * svlo_sigmoid_value(second);
            if (!isfinite(v)) return SVLO_INTERNAL;
            tmp_h[r * H + col] = v; /* gated */
        }
    const float *dw = AW(l, A_LC_DW);
    for (size_t r = 0; r < rows; ++r)
        for (size_t col = 0; col < H; ++col) {
            float sum = 0.0f;
            for (size_t tap = 0; tap < K; ++tap) {
                long long src = (long long)r - ((long long)K - 1) + (long long)tap;
                if (src < 0 || src >= (long long)rows) continue;
                sum += tmp_h[(size_t)src * H + col] * dw[col * K + tap];
            }
            tmp_h2[r * H + col] = sum;
        }
    au_clamp_if_needed(tmp_h2, rows * H, c->gradient_clipping);
    if ((st = svlo_rms_norm_rows(tmp_h2, AW(l, A_LC_NORM), rows, H, c->rms_norm_eps, tmp_h)))
        return st;
    for (size_t i = 0; i < rows * H; ++i) {
        float s = svlo_silu_value(tmp_h[i]);
        if (!isfinite(s)) return SVLO_INTERNAL;
        tmp_h[i] = s;
    }
    if ((st = svlo_clipped_linear(tmp_h, AW(l, A_LC_END), be, rows, H, H, tmp_h2))) return st;
    for (size_t i = 0; i < rows * H; ++i) {
        float sum = hidden[i] + tmp_h2[i];
        if (!isfinite(sum)) return SVLO_INTERNAL;
        out[i] = sum;
    }
    return SVLO_OK;
}

/* audio.rs:1579-1661: the chunked local attention on already projected and
 * scaled q, k (and v), [rows, heads * head_dim]; relk [positions, heads *
 * head_dim]; att [rows, heads * head_dim] (rows the mask drops stay zero). */
int svlo_audio_attention_core(const float *q, const float *k, const float *v, const float *relk,
                              const unsigned char *mask, size_t rows, size_t heads,
                              size_t head_dim, size_t chunk, size_t context_left,
                              size_t context_right, float cap, float *att) {
    const size_t H = heads * head_dim;
    if (chunk == 0 || context_left < 2) return SVLO_INTERNAL;
    const size_t context = chunk + context_left - 1 + context_right;
    const size_t positions = context / 2 + 1;
    const long long max_past = (long long)context_left - 1;
    const long long left_window = (long long)context_left - 1;
    const float invalid = -1.0e9f;
    float *scores = (float *)malloc(heads * context * sizeof(float));
    float *den = (float *)malloc(heads * sizeof(float));
    if (!scores || !den) {
        free(scores);
        free(den);
        return SVLO_LIMIT;
    }
    int st = SVLO_OK;
    memset(att, 0, rows * H * sizeof(float));
    size_t blocks = (rows + chunk - 1) / chunk;
    for (size_t b = 0; b < blocks; ++b)
        for (size_t off = 0; off < chunk; ++off) {
            size_t qi = b * chunk + off;
            if (qi >= rows || !mask[qi]) continue;
            for (size_t h = 0; h < heads; ++h) {
                float maximum = -INFINITY;
                for (size_t ci = 0; ci < context; ++ci) {
                    long long ki = (long long)(b * chunk) + (long long)ci - max_past;
                    int valid = ki >= 0 && ki < (long long)rows && mask[ki] &&
                                (long long)qi - ki >= 0 && (long long)qi - ki < left_window;
                    float score;
                    if (valid) {
                        float dot = 0.0f;
                        for (size_t d = 0; d < head_dim; ++d)
                            dot += q[qi * H + h * head_dim + d] * k[(size_t)ki * H + h * head_dim + d];
                        long long rel = (long long)ci - (long long)off;
                        if (rel >= 0 && (size_t)rel < positions)
                            for (size_t d = 0; d < head_dim; ++d)
                                dot += q[qi * H + h * head_dim + d] *
                                       relk[((size_t)rel * heads + h) * head_dim + d];
                        score = tanhf(dot / cap) * cap;
                    } else {
                        score = invalid;
                    }
                    scores[h * context + ci] = score;
                    maximum = fmaxf(maximum, score);
                }
                if (maximum <= invalid / 2.0f) {
                    den[h] = 0.0f;
                    continue;
                }
                float sum = 0.0f;
                for (size_t ci = 0; ci < context; ++ci) {
                    float e = expf(scores[h * context + ci] - maximum);
                    scores[h * context + ci] = e;
                    sum += e;
                }
                if (!isfinite(sum) || sum <= 0.0f) {
                    st = SVLO_INTERNAL;
                    goto done;
                }
                den[h] = sum;
            }
            for (size_t h = 0; h < heads; ++h) {
                float sum = den[h];
                if (sum == 0.0f) continue;
                for (size_t ci = 0; ci < context; ++ci) {
                    float w = scores[h * context + ci] / sum;
                    if (w == 0.0f) continue;
                    long long ki = (long long)(b * chunk) + (long long)ci - max_past;
                    if (ki < 0 || ki >= (long long)rows) continue;
                    for (size_t d = 0; d < head_dim; ++d)
                        att[qi * H + h * head_dim + d] += w * v[(size_t)ki * H + h * head_dim + d];
                }
            }
        }
    for (size_t i = 0; i < rows * H; ++i)
        if (!isfinite(att[i])) st = SVLO_INTERNAL;
done:
    free(scores);
    free(den);
    return st;
}

/* audio.rs:1529-1669 chunked_attention over all rows (mask marks valid rows):
 * q/k/v clipped linears, the per-dimension query scale and key scale, the
 * attention core, then the post clipped linear into out. */
static int au_chunked_attention(const svlo_audio_config *c, const float *const *weights, size_t l,
                                const float *hidden, const unsigned char *mask, size_t rows,
                                const float *relk, float *q, float *k, float *v, float *att,
                                float *out) {
    const size_t H = (size_t)c->hidden_size, NH = (size_t)c->num_attention_heads;
    const size_t hd = (size_t)c->head_dim;
    const float q_scale = (float)(pow((double)hd, -0.5) / AU_LN_2);
    const float k_scale = (float)(log(1.0 + AU_E) / AU_LN_2);
    int st;
    float bq[4], bk[4], bv[4], bp[4];
    au_bounds(weights, l, A_ATT + 1, bq);
    au_bounds(weights, l, A_ATT + 6, bk);
    au_bounds(weights, l, A_ATT + 11, bv);
    au_bounds(weights, l, A_ATT + 16, bp);
    if ((st = svlo_clipped_linear(hidden, AW(l, A_ATT + 0), bq, rows, H, H, q))) return st;
    if ((st = svlo_clipped_linear(hidden, AW(l, A_ATT + 5), bk, rows, H, H, k))) return st;
    if ((st = svlo_clipped_linear(hidden, AW(l, A_ATT + 10), bv, rows, H, H, v))) return st;
    const float *pds = AW(l, A_PDS);
    for (size_t r = 0; r < rows; ++r)
        for (size_t h = 0; h < NH; ++h)
            for (size_t d = 0; d < hd; ++d) {
                size_t i = r * H + h * hd + d;
                float scale = svlo_softplus_value(pds[d]);
                if (!isfinite(scale)) return SVLO_INTERNAL;
                q[i] *= q_scale * scale;
                k[i] *= k_scale;
            }
    if ((st = svlo_audio_attention_core(q, k, v, relk, mask, rows, NH, hd,
                                        (size_t)c->attention_chunk_size,
                                        (size_t)c->attention_context_left,
                                        (size_t)c->attention_context_right,
                                        c->attention_logit_cap, att)))
        return st;
    return svlo_clipped_linear(att, AW(l, A_ATT + 15), bp, rows, H, H, out);
}

/* AudioModel::subsample (audio.rs:1136-1255); out_hidden [second_frames, H],
 * mask1 [second_frames]. */
static int au_subsample(const svlo_audio_config *c, const float *const *weights,
                        const float *features, const unsigned char *mask, size_t frames,
                        float *out_hidden, unsigned char *mask1, char *msg, size_t msg_len) {
    const size_t C0 = (size_t)c->conv_channels0, C1 = (size_t)c->conv_channels1;
    const size_t H = (size_t)c->hidden_size;
    const size_t f1 = (frames + 1) / 2, f2 = (f1 + 1) / 2;
    const size_t q1 = (AU_FEATURE_SIZE + 1) / 2, q2 = (q1 + 1) / 2;
    if (f2 == 0) return au_fail(msg, msg_len, SVLO_CORRUPT, "audio subsampling produced no frames");
    if (f1 * q1 * C0 > AU_MAX_ACTIVATION_ELEMENTS || f2 * q2 * C1 > AU_MAX_ACTIVATION_ELEMENTS)
        return au_fail(msg, msg_len, SVLO_LIMIT, "audio subsampling above the element cap");
    float *l0 = (float *)calloc(f1 * q1 * C0, sizeof(float));
    float *l1 = (float *)calloc(f2 * q2 * C1, sizeof(float));
    unsigned char *mask0 = (unsigned char *)calloc(f1 + 1, 1);
    int st = SVLO_OK;
    if (!l0 || !l1 || !mask0) {
        st = SVLO_LIMIT;
        goto done;
    }
    const float *w0 = weights[0], *n0 = weights[1], *w1 = weights[2], *n1 = weights[3];
    for (size_t t = 0; t < f1; ++t)
        for (size_t f = 0; f < q1; ++f) {
            float *dst = l0 + (t * q1 + f) * C0;
            for (size_t oc = 0; oc < C0; ++oc) {
                float sum = 0.0f;
                for (long long kt = 0; kt < 3; ++kt)
                    for (long long kf = 0; kf < 3; ++kf) {
                        long long it = (long long)t * 2 + kt - 1, iff = (long long)f * 2 + kf - 1;
                        if (it < 0 || it >= (long long)frames || iff < 0 ||
                            iff >= AU_FEATURE_SIZE || !mask[it])
                            continue;
                        sum += features[(size_t)it * AU_FEATURE_SIZE + (size_t)iff] *
                               w0[oc * 9 + (size_t)(kt * 3 + kf)];
                    }
                dst[oc] = sum;
            }
            if ((st = au_normalize_subsample(dst, n0, C0, c->rms_norm_eps))) goto done;
        }
    for (size_t i = 0; i < f1; ++i) mask0[i] = (2 * i < frames) ? mask[2 * i] : 0;
    for (size_t t = 0; t < f2; ++t)
        for (size_t f = 0; f < q2; ++f) {
            float *dst = l1 + (t * q2 + f) * C1;
            for (size_t oc = 0; oc < C1; ++oc) {
                float sum = 0.0f;
                for (size_t ic = 0; ic < C0; ++ic)
                    for (long long kt = 0; kt < 3; ++kt)
                        for (long long kf = 0; kf < 3; ++kf) {
                            long long it = (long long)t * 2 + kt - 1,
                                      iff = (long long)f * 2 + kf - 1;
                            if (it < 0 || it >= (long long)f1 || iff < 0 || iff >= (long long)q1 ||
                                !mask0[it])
                                continue;
                            sum += l0[((size_t)it * q1 + (size_t)iff) * C0 + ic] *
                                   w1[((oc * C0 + ic) * 3 + (size_t)kt) * 3 + (size_t)kf];
                        }
                dst[oc] = sum;
            }
            if ((st = au_normalize_subsample(dst, n1, C1, c->rms_norm_eps))) goto done;
        }
    for (size_t i = 0; i < f2; ++i) mask1[i] = (2 * i < f1) ? mask0[2 * i] : 0;
    if (q2 * C1 != (size_t)(c->conv_channels0 / 4 * c->conv_channels1)) {
        st = SVLO_INTERNAL;
        goto done;
    }
    st = svlo_linear(l1, weights[4], f2, q2 * C1, H, out_hidden);
done:
    if (st && st != SVLO_CORRUPT)
        au_fail(msg, msg_len, st, "audio subsampling failed with status %d", st);
    free(l0);
    free(l1);
    free(mask0);
    return st;
}

size_t svlo_audio_subsampled_frames(size_t frames) {
    size_t f1 = (frames + 1) / 2;
    return (f1 + 1) / 2;
}

/* Scratch of one encoder layer over `rows` subsampled rows. */
typedef struct {
    float *h2, *t1, *t2, *t3, *ti, *ti2, *t2h, *qb, *kb, *vb, *relk;
} au_layer_bufs;

/* One conformer layer of AudioModel::forward (audio.rs:1001-1083): feed-forward
 * 1, attention sandwich, light conv, feed-forward 2, norm_out; `hidden` [rows,
 * H] is read and overwritten. */
static int au_layer(const svlo_audio_config *c, const float *const *weights, size_t l,
                    float *hidden, const unsigned char *mask1, size_t rows, const float *posemb,
                    const au_layer_bufs *b) {
    const size_t H = (size_t)c->hidden_size;
    const size_t context = (size_t)(c->attention_chunk_size + c->attention_context_left - 1 +
                                    c->attention_context_right);
    const size_t positions = context / 2 + 1;
    int st;
    if ((st = au_feed_forward(c, weights, l, A_FF1, hidden, rows, b->t1, b->ti, b->ti2, b->h2)))
        return st;
    /* residual = h2 */
    if ((st = svlo_rms_norm_rows(b->h2, AW(l, A_NORM_PRE_ATTN), rows, H, c->rms_norm_eps, b->t1)))
        return st;
    if ((st = svlo_linear(posemb, AW(l, A_RELK), positions, H, H, b->relk))) return st;
    if ((st = au_chunked_attention(c, weights, l, b->t1, mask1, rows, b->relk, b->qb, b->kb, b->vb,
                                   b->t2, b->t3)))
        return st;
    if ((st = svlo_rms_norm_rows(b->t3, AW(l, A_NORM_POST_ATTN), rows, H, c->rms_norm_eps, b->t2)))
        return st;
    svlo_add(b->h2, b->t2, rows * H, hidden);
    if ((st = au_light_conv(c, weights, l, hidden, rows, b->t1, b->t2h, b->t3, b->h2))) return st;
    if ((st = au_feed_forward(c, weights, l, A_FF2, b->h2, rows, b->t1, b->ti, b->ti2, b->t2)))
        return st;
    return svlo_rms_norm_rows(b->t2, AW(l, A_NORM_OUT), rows, H, c->rms_norm_eps, hidden);
}

static au_layer_bufs au_layer_alloc(size_t rows, size_t H, size_t I, size_t positions) {
    au_layer_bufs b;
    b.h2 = (float *)malloc(rows * H * sizeof(float));
    b.t1 = (float *)malloc(rows * H * sizeof(float));
    b.t2 = (float *)malloc(rows * H * sizeof(float));
    b.t3 = (float *)malloc(rows * H * sizeof(float));
    b.ti = (float *)malloc(rows * I * sizeof(float));
    b.ti2 = (float *)malloc(rows * I * sizeof(float));
    b.t2h = (float *)malloc(rows * 2 * H * sizeof(float));
    b.qb = (float *)malloc(rows * H * sizeof(float));
    b.kb = (float *)malloc(rows * H * sizeof(float));
    b.vb = (float *)malloc(rows * H * sizeof(float));
    b.relk = (float *)malloc(positions * H * sizeof(float));
    return b;
}

static int au_layer_ok(const au_layer_bufs *b) {
    return b->h2 && b->t1 && b->t2 && b->t3 && b->ti && b->ti2 && b->t2h && b->qb && b->kb &&
           b->vb && b->relk;
}

static void au_layer_free(au_layer_bufs *b) {
    free(b->h2);
    free(b->t1);
    free(b->t2);
    free(b->t3);
    free(b->ti);
    free(b->ti2);
    free(b->t2h);
    free(b->qb);
    free(b->kb);
    free(b->vb);
    free(b->relk);
}

/* One encoder layer alone, from a given hidden state [rows, H] and the
 * subsampled row mask (0/1 bytes), into out [rows, H]. */
int svlo_audio_layer(const svlo_audio_config *c, const float *const *weights, size_t layer,
                     const float *hidden_in, const unsigned char *mask, size_t rows, float *out,
                     char *msg, size_t msg_len) {
    if (msg && msg_len) msg[0] = 0;
    const size_t H = (size_t)c->hidden_size, I = (size_t)c->intermediate_size;
    const size_t context = (size_t)(c->attention_chunk_size + c->attention_context_left - 1 +
                                    c->attention_context_right);
    const size_t positions = context / 2 + 1;
    if (layer >= (size_t)c->num_hidden_layers || rows == 0)
        return au_fail(msg, msg_len, SVLO_INTERNAL, "audio layer %zu of %lld over %zu rows", layer,
                       (long long)c->num_hidden_layers, rows);
    au_layer_bufs b = au_layer_alloc(rows, H, I, positions);
    float *posemb = (float *)malloc(positions * H * sizeof(float));
    int st = SVLO_OK;
    if (!au_layer_ok(&b) || !posemb) {
        st = au_fail(msg, msg_len, SVLO_LIMIT, "allocation failed");
    } else if ((st = svlo_audio_position_embeddings(H, positions, posemb)) == SVLO_OK) {
        memcpy(out, hidden_in, rows * H * sizeof(float));
        st = au_layer(c, weights, layer, out, mask, rows, posemb, &b);
    }
    if (st && msg && msg_len && !msg[0])
        au_fail(msg, msg_len, st, "audio layer failed with status %d", st);
    au_layer_free(&b);
    free(posemb);
    return st;
}

/* AudioModel::forward (audio.rs:981-1134). */
int svlo_audio_forward(const svlo_audio_config *c, const float *const *weights,
                       size_t text_hidden, const float *features, const unsigned char *mask,
                       size_t frames, size_t *out_tokens, float *out_pooled, float *out_sscp,
                       float *out_hidden, char *msg, size_t msg_len) {
    if (msg && msg_len) msg[0] = 0;
    const size_t H = (size_t)c->hidden_size, L = (size_t)c->num_hidden_layers;
    const size_t I = (size_t)c->intermediate_size, P = (size_t)c->output_proj_dims;
    const size_t context = (size_t)(c->attention_chunk_size + c->attention_context_left - 1 +
                                    c->attention_context_right);
    const size_t positions = context / 2 + 1;
    const size_t rows = svlo_audio_subsampled_frames(frames);
    if (rows == 0) return au_fail(msg, msg_len, SVLO_CORRUPT, "audio subsampling produced no frames");
    int st = SVLO_OK;
    float *hidden = (float *)malloc(rows * H * sizeof(float));
    au_layer_bufs lb = au_layer_alloc(rows, H, I, positions);
    float *posemb = (float *)malloc(positions * H * sizeof(float));
    float *proj = (float *)malloc(rows * P * sizeof(float));
    float *projn = (float *)malloc(rows * P * sizeof(float));
    float *pooled_all = (float *)malloc(rows * text_hidden * sizeof(float));
    unsigned char *mask1 = (unsigned char *)calloc(rows + 1, 1);
    if (!hidden || !au_layer_ok(&lb) || !posemb || !proj || !projn || !pooled_all || !mask1) {
        st = au_fail(msg, msg_len, SVLO_LIMIT, "allocation failed");
        goto done;
    }
    if ((st = au_subsample(c, weights, features, mask, frames, hidden, mask1, msg, msg_len)))
        goto done;
    size_t tokens = 0;
    for (size_t r = 0; r < rows; ++r) tokens += mask1[r] != 0;
    if (tokens == 0) {
        st = au_fail(msg, msg_len, SVLO_CORRUPT, "audio tower received no valid subsampled token");
        goto done;
    }
    *out_tokens = tokens;
    if ((st = svlo_audio_position_embeddings(H, positions, posemb))) goto knl;
    if (out_sscp) {
        size_t o = 0;
        for (size_t r = 0; r < rows; ++r)
            if (mask1[r]) memcpy(out_sscp + (o++) * H, hidden + r * H, H * sizeof(float));
    }
    for (size_t l = 0; l < L; ++l) {
        if ((st = au_layer(c, weights, l, hidden, mask1, rows, posemb, &lb))) goto knl;
        if (out_hidden) {
            size_t o = 0;
            for (size_t r = 0; r < rows; ++r)
                if (mask1[r])
                    memcpy(out_hidden + (l * tokens + o++) * H, hidden + r * H, H * sizeof(float));
        }
    }
    /* audio.rs:1085-1133 output projection + bias, unscaled norm, text projection. */
    {
        const size_t G = SVLO_AUDIO_GLOBAL_TENSORS + L * SVLO_AUDIO_LAYER_TENSORS;
        if ((st = svlo_linear(hidden, weights[G], rows, H, P, proj))) goto knl;
        const float *bias = weights[G + 1];
        for (size_t r = 0; r < rows; ++r)
            for (size_t col = 0; col < P; ++col) proj[r * P + col] += bias[col];
        for (size_t i = 0; i < rows * P; ++i)
            if (!isfinite(proj[i])) {
                st = au_fail(msg, msg_len, SVLO_INTERNAL,
                             "audio output projection produced a non-finite value");
                goto done;
            }
        if ((st = svlo_rms_norm_rows_unscaled(proj, rows, P, c->rms_norm_eps, projn))) goto knl;
        if ((st = svlo_linear(projn, weights[G + 2], rows, P, text_hidden, pooled_all))) goto knl;
        size_t o = 0;
        for (size_t r = 0; r < rows; ++r)
            if (mask1[r])
                memcpy(out_pooled + (o++) * text_hidden, pooled_all + r * text_hidden,
                       text_hidden * sizeof(float));
    }
    goto done;
knl:
    au_fail(msg, msg_len, st, "audio kernel failed with status %d (non-finite value or limit)", st);
done:
    free(hidden);
    au_layer_free(&lb);
    free(posemb);
    free(proj);
    free(projn);
    free(pooled_all);
    free(mask1);
    return st;
}
