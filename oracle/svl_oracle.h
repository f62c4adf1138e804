/*
 * CPU oracle for the EmbeddingGemma-2 text encoder forward pass.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the oracle that the HIP path is
 * compared against; it is never linked into, loaded by, or called from the
 * product library. Only tests, the smoke check and the CPU-baseline leg of
 * bench.py load it.
 *
 * Every function restates one scalar function of the reference crate
 * (src/tensor/kernels.rs, src/model/text.rs, src/model/config.rs) with the
 * same loop order, the same f32 evaluation order and no FMA contraction
 * (compiled with -ffp-contract=off), using the platform libm for
 * expf/tanhf/sinf/cosf/powf/sqrtf as the reference does on Linux.
 *
 * Status codes mirror src/error.rs:24-37.
 */
#ifndef SVL_ORACLE_H
#define SVL_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    SVLO_OK = 0,
    SVLO_USAGE = 2,
    SVLO_IO = 3,
    SVLO_CORRUPT = 4,
    SVLO_LIMIT = 5,
    SVLO_UNSUPPORTED = 6,
    SVLO_INTERNAL = 7
};

/* kernels.rs scalar functions (device-free, caller-owned buffers). */
float svlo_dot(const float *a, const float *b, size_t n);
int svlo_add(const float *a, const float *b, size_t n, float *out);
int svlo_linear(const float *input, const float *weight, size_t rows, size_t in_features,
                size_t out_features, float *out);
int svlo_matmul(const float *left, const float *right, size_t m, size_t k, size_t n, float *out);
int svlo_rms_norm_rows(const float *input, const float *weight, size_t rows, size_t width,
                       float eps, float *out);
int svlo_rms_norm_rows_unscaled(const float *input, size_t rows, size_t width, float eps,
                                float *out);
int svlo_softmax(const float *values, size_t n, float *out);
float svlo_gelu_tanh_value(float v);
void svlo_gelu_tanh(const float *values, size_t n, float *out);
int svlo_geglu(const float *gate, const float *up, size_t n, float *out);
int svlo_l2_normalize(const float *input, size_t n, float *out);
int svlo_mean_pool(const float *values, size_t rows, size_t width, float *out);
int svlo_truncate_and_normalize(const float *values, size_t n, size_t dim, float *out);
int svlo_rope_inv_freq(size_t head_dim, float base, float *out);
int svlo_rope_with_inv_freq(float *values, size_t seq_len, size_t num_heads, size_t head_dim,
                            const float *inv_freq, size_t n_inv_freq, size_t position_offset);
/* sliding_window < 0 means full attention. */
int svlo_bidirectional_attention(const float *q, const float *k, const float *v, size_t seq_len,
                                 size_t num_heads, size_t num_kv_heads, size_t head_dim,
                                 int64_t sliding_window, float scale, float *out);

/* Validated text configuration (src/model/config.rs:76-95). */
typedef struct {
    int64_t vocab_size;
    int64_t hidden_size;
    int64_t intermediate_size;
    int64_t num_hidden_layers;
    int64_t num_attention_heads;
    int64_t hidden_size_per_layer_input;
    int64_t embedding_dim;
    int64_t max_position_embeddings;
    int64_t sliding_window;
    int64_t pad_token_id; /* -1 when absent */
    float rms_norm_eps;
    float full_rope_theta;
    float sliding_rope_theta;
    const int32_t *layer_type; /* [layers], 0 = sliding, 1 = full */
    const int64_t *head_dim;   /* [layers] */
    const int64_t *num_kv_heads; /* [layers] */
} svlo_text_config;

/*
 * Weights in the order of TextConfig::tensor_shapes (config.rs:394-484):
 * [0] embed_tokens, [1] embedding_projection, [2] norm,
 * [3] ple.per_layer_model_projection, [4] ple.per_layer_projection_norm,
 * then 17 per layer: input_layernorm, post_attention_layernorm,
 * pre_feedforward_layernorm, post_feedforward_layernorm, layer_scalar,
 * gate_proj, up_proj, down_proj, per_layer_input_gate, per_layer_projection,
 * post_per_layer_input_norm, q_proj, k_proj, v_proj, o_proj, q_norm, k_norm.
 */
#define SVLO_GLOBAL_TENSORS 5
#define SVLO_LAYER_TENSORS 17

/*
 * TextModel::forward_impl (text.rs:182-538). features may be NULL.
 * out_projected [seq, embedding_dim], out_pooled and out_normalized
 * [embedding_dim] are required; out_hidden [(layers+1), seq, hidden] is
 * optional. msg (optional, msg_len bytes) receives the error text.
 */
int svlo_text_forward(const svlo_text_config *cfg, const float *const *weights,
                      const uint32_t *ids, size_t seq, const float *features,
                      size_t feature_start, size_t feature_count, size_t features_len,
                      float *out_projected, float *out_pooled, float *out_normalized,
                      float *out_hidden, char *msg, size_t msg_len);

/* ---- vision tower (src/model/vision.rs) --------------------------------- */

/* Validated vision configuration (vision.rs:58-70). */
typedef struct {
    int64_t hidden_size;
    int64_t intermediate_size;
    int64_t num_hidden_layers;
    int64_t num_attention_heads;
    int64_t num_key_value_heads;
    int64_t head_dim;
    int64_t position_embedding_size;
    float rms_norm_eps;
    float rope_theta;
} svlo_vision_config;

/*
 * Weights in the order of VisionConfig::tensor_shapes (vision.rs:345-414):
 * [0] patch_embedder.input_proj [hidden, 768],
 * [1] patch_embedder.position_embedding_table [2, pos, hidden],
 * then 13 per layer: input_layernorm, post_attention_layernorm,
 * pre_feedforward_layernorm, post_feedforward_layernorm, q_proj, k_proj,
 * v_proj, o_proj, q_norm, k_norm, gate_proj, up_proj, down_proj,
 * and last embed_vision.embedding_projection [text_hidden, hidden].
 */
#define SVLO_VISION_GLOBAL_TENSORS 2
#define SVLO_VISION_LAYER_TENSORS 13

/* vision.rs:1047-1065; out has head_dim / 4 entries. */
int svlo_axial_inv_freq(size_t head_dim, float theta, float *out);
/* vision.rs:1073-1148 on [sequence, heads, head_dim]; positions [n, 2] (x, y). */
int svlo_axial_rope(float *values, size_t sequence, size_t heads, size_t head_dim,
                    const int32_t *positions, size_t n_positions, const float *inv_freq,
                    size_t n_inv_freq);
/* vision.rs:980-1040; out [soft_tokens, hidden_size]. */
int svlo_pool_patches(const float *hidden, const int32_t *positions, size_t valid,
                      size_t grid_width, size_t grid_height, size_t soft_tokens,
                      size_t hidden_size, float *out);
/*
 * VisionModel::forward (vision.rs:742-959) over the first `valid` patches:
 * pixel_values [valid, 768], positions [valid, 2]. out_pooled
 * [soft_tokens, text_hidden] (VisionOutput::pooled); out_hidden
 * [(layers + 1), valid, hidden] optional.
 */
int svlo_vision_forward(const svlo_vision_config *cfg, const float *const *weights,
                        size_t text_hidden, const float *pixel_values, const int32_t *positions,
                        size_t valid, size_t max_patches, size_t grid_width, size_t grid_height,
                        size_t soft_tokens, float *out_pooled, float *out_hidden, char *msg,
                        size_t msg_len);
/* One encoder layer of VisionModel::forward (vision.rs:816-935) alone, from a
 * given hidden state [rows, hidden] and patch positions [rows, 2] (x, y), into
 * out [rows, hidden]; the same code the forward pass runs per layer. */
int svlo_vision_layer(const svlo_vision_config *cfg, const float *const *weights, size_t layer,
                      const float *hidden_in, const int32_t *positions, size_t rows, float *out,
                      char *msg, size_t msg_len);

/* ---- audio tower (src/model/audio.rs) ----------------------------------- */

/* Validated audio configuration (audio.rs:62-80). */
typedef struct {
    int64_t hidden_size;
    int64_t intermediate_size; /* 4 * hidden_size */
    int64_t num_hidden_layers;
    int64_t num_attention_heads;
    int64_t head_dim; /* hidden_size / num_attention_heads */
    int64_t conv_kernel_size;
    int64_t conv_channels0;
    int64_t conv_channels1;
    int64_t attention_chunk_size;
    int64_t attention_context_left;
    int64_t attention_context_right;
    int64_t output_proj_dims;
    float attention_logit_cap;
    float rms_norm_eps;
    float residual_weight;
    float gradient_clipping;
} svlo_audio_config;

/*
 * Weights in the order of AudioConfig::tensor_shapes (audio.rs:394-498):
 * 5 subsampling tensors (layer0 conv [C0,1,3,3], layer0 norm [C0], layer1 conv
 * [C1,C0,3,3], layer1 norm [C1], input_proj_linear [H, C0/4*C1]), 62 per layer
 * (feed_forward1 and feed_forward2: pre/post norms, two linears, 4 bounds each;
 * q/k/v/post: weight + 4 bounds each; relative_k_proj; per_dim_scale; light
 * conv: pre norm, start/end linears, their bounds, depthwise weight, conv
 * norm; norm_pre_attn, norm_post_attn, norm_out), then output_proj weight and
 * bias and embed_audio.embedding_projection. Scalars are 1-element arrays.
 */
#define SVLO_AUDIO_GLOBAL_TENSORS 5
#define SVLO_AUDIO_LAYER_TENSORS 62

float svlo_clamp_value(float value, float minimum, float maximum); /* audio.rs:1339 */
float svlo_silu_value(float value);                                /* audio.rs:1349 */
float svlo_sigmoid_value(float value);                             /* audio.rs:1357 */
float svlo_softplus_value(float value);                            /* audio.rs:1366 */
/* audio.rs:558-601; bounds = {input_min, input_max, output_min, output_max}. */
int svlo_clipped_linear(const float *input, const float *weight, const float *bounds, size_t rows,
                        size_t in_features, size_t out_features, float *out);
/* audio.rs:1257-1288; out [positions, hidden]. */
int svlo_audio_position_embeddings(size_t hidden, size_t positions, float *out);
/* audio.rs:1579-1661 chunked local attention on projected, scaled q and k:
 * [rows, heads * head_dim] each, relk [positions, heads * head_dim], mask
 * [rows] (0/1). att [rows, heads * head_dim]. */
int svlo_audio_attention_core(const float *q, const float *k, const float *v, const float *relk,
                              const unsigned char *mask, size_t rows, size_t heads,
                              size_t head_dim, size_t chunk, size_t context_left,
                              size_t context_right, float cap, float *att);
/* Rows after the two stride-2 subsampling convolutions: ceil(ceil(frames/2)/2). */
size_t svlo_audio_subsampled_frames(size_t frames);
/*
 * AudioModel::forward (audio.rs:981-1134) on log-mel features [frames, 128]
 * with the frame mask (0/1 bytes). out_pooled [subsampled frames, text_hidden]
 * receives the valid tokens first (*out_tokens of them, AudioOutput::pooled);
 * out_sscp (optional, [tokens, hidden]) the subsampling output and out_hidden
 * (optional, [layers, tokens, hidden]) each layer's output, valid rows only.
 */
int svlo_audio_forward(const svlo_audio_config *cfg, const float *const *weights,
                       size_t text_hidden, const float *features, const unsigned char *mask,
                       size_t frames, size_t *out_tokens, float *out_pooled, float *out_sscp,
                       float *out_hidden, char *msg, size_t msg_len);

/* One encoder layer of AudioModel::forward (audio.rs:1001-1083) alone, from a
 * given hidden state [rows, hidden] and subsampled row mask (0/1 bytes), into
 * out [rows, hidden]; the same code the forward pass runs per layer. */
int svlo_audio_layer(const svlo_audio_config *cfg, const float *const *weights, size_t layer,
                     const float *hidden_in, const unsigned char *mask, size_t rows, float *out,
                     char *msg, size_t msg_len);

/* Log-mel front end, src/media/audio_preprocess.rs:24-46 constants. */
#define SVLO_MEL_FRAME_LENGTH 320
#define SVLO_MEL_HOP 160
#define SVLO_MEL_FFT 512
#define SVLO_MEL_FEATURES 128
#define SVLO_MEL_BINS (SVLO_MEL_FFT / 2 + 1)
#define SVLO_MEL_FLOOR 0.001
#define SVLO_MEL_PAD_TO 128
#define SVLO_MEL_MAX_FRAMES 3000
/* src/media/audio.rs:19: 30 s at 16 kHz */
#define SVLO_MEL_MAX_SAMPLES 480000

void svlo_hann_window(float *out);
int svlo_mel_filter_bank(double *out);
int svlo_fft(double *values, size_t n);
int svlo_log_mel_layout(size_t samples, size_t *frames, size_t *padded_samples,
                        size_t *valid_frames, char *msg, size_t msg_len);
int svlo_log_mel(const float *samples, size_t n_samples, float *features, unsigned char *mask,
                 char *msg, size_t msg_len);

/* Exact vector search, src/index/vector.rs:17-97 (storage/model.rs:35 cap). */
#define SVLO_MAX_EMBEDDING_DIMENSION 8192
/* vector::rank over chunks emb [n, dim] with ids [n] (has_dim: the index has a
 * dimension); mask NULL or [n] 0/1. out_index / out_score [n] receive the full
 * ranking, *out_count its length. */
int svlo_vector_rank(const float *query, size_t qlen, const float *emb, const uint64_t *ids,
                     size_t n, size_t dim, int has_dim, const unsigned char *mask,
                     size_t *out_index, double *out_score, size_t *out_count, char *msg,
                     size_t msg_len);

#ifdef __cplusplus
}
#endif

#endif
