/*
 * svl_hip.h — C ABI of the MI355X (gfx950) encoder backend.
 *
 * The boundary sits at the whole text forward pass: weights stay resident in
 * HBM, token ids and row offsets go in, pooled / normalised embeddings come
 * out. It replaces the body of TextModel::forward_impl
 * (src/model/text.rs:182-538) behind the unchanged TextModel / TextEmbedder
 * API, the way src/tensor/neon.rs sits behind src/tensor/kernels.rs.
 *
 * A second group of entry points mirrors the kernel seam of
 * src/tensor/kernels.rs on device pointers, so each kernel can be checked on
 * its own against the reference's known answers.
 *
 * Conventions:
 *  - Status codes mirror src/error.rs:24-37 (Usage, Io, Corrupt,
 *    LimitExceeded, Unsupported, Internal) plus SVL_DEVICE for HIP failures.
 *  - The caller owns every buffer it passes; the library never retains a
 *    caller pointer past the call. The library owns device weights and
 *    workspaces.
 *  - svl_last_error() returns the calling thread's last message.
 *  - A model may be called from several threads; calls are serialised per
 *    model, and repeated calls are bit-identical (fixed reduction orders,
 *    no floating-point atomics).
 *  - Streams are passed as void* (a hipStream_t); NULL selects the model's
 *    own stream (model entry points) or the null stream (kernel seam).
 */
#ifndef SVL_HIP_H
#define SVL_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* src/error.rs:24-37 */
typedef enum {
    SVL_OK = 0,
    SVL_USAGE = 2,
    SVL_IO = 3,
    SVL_CORRUPT = 4,
    SVL_LIMIT = 5,
    SVL_UNSUPPORTED = 6,
    SVL_INTERNAL = 7,
    SVL_DEVICE = 8
} svl_status;

/* src/tensor/dtype.rs:11-57 (FP16 is rejected as in the reference). */
typedef enum { SVL_F32 = 0, SVL_BF16 = 1 } svl_dtype;

typedef struct svl_ctx svl_ctx;
typedef struct svl_text_model svl_text_model;

/* One named weight tensor, borrowed for the duration of the call
 * (src/binary/safetensors.rs:69-110 TensorEntry: name, dtype, shape and its
 * byte slice). A payload whose length is not numel * 4 (F32) or numel * 2
 * (BF16) is Corrupt, as in TensorEntry::to_f32 and bf16::decode_bf16. */
typedef struct {
    const char *name;
    int32_t dtype; /* svl_dtype */
    int32_t ndim;
    int64_t shape[8];
    const void *data; /* host memory, little-endian */
    size_t nbytes;    /* bytes at data */
} svl_tensor_view;

/* Validated text configuration (src/model/config.rs:76-95 TextConfig and
 * :64-72 LayerConfig). Arrays have num_hidden_layers entries. */
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
    int64_t pad_token_id; /* -1 when the config declares none */
    double rms_norm_eps;
    double full_rope_theta;
    double sliding_rope_theta;
    const int32_t *layer_type; /* 0 = sliding_attention, 1 = full_attention */
    const int64_t *head_dim;
    const int64_t *num_kv_heads;
} svl_text_config;

/* Multimodal soft tokens for one row (text.rs:167-180, 226-275):
 * rows [start, start + count) of that row's hidden state are replaced by
 * data[count, hidden_size]. data == NULL means no replacement. */
typedef struct {
    const float *data;
    int64_t start;
    int64_t count;
    int64_t len; /* number of floats in data */
} svl_feature_span;

/* ---- context and model lifetime ------------------------------------------ */

/* Selects one HIP device; gfx950 only. */
svl_status svl_init(int device_ordinal, svl_ctx **out);
svl_status svl_shutdown(svl_ctx *ctx);
/* Thread-local message of the last failing call on this thread. */
const char *svl_last_error(void);

/* Validates the inventory like src/model/weights.rs:125-189 (missing,
 * unexpected or mis-shaped tensors -> CORRUPT, non-finite -> CORRUPT, BF16
 * widened exactly), copies the weights to HBM in the backend's packed
 * layouts, and returns a model. Replaces TextModel::new / from_files
 * (text.rs:104-126). */
svl_status svl_text_model_create(svl_ctx *ctx, const svl_text_config *cfg,
                                 const svl_tensor_view *tensors, size_t n_tensors,
                                 svl_text_model **out);
svl_status svl_text_model_destroy(svl_text_model *model);

/* ---- whole forward pass -------------------------------------------------- */

/* Runs `batch` independent forward passes (text.rs:150-180, 182-538), one
 * per row; row r is ids[offsets[r] .. offsets[r+1]). Row r of every output
 * equals TextModel::forward(row r). Host buffers.
 *  features        NULL or [batch] spans (forward_with_features)
 *  out_normalized  [batch, embedding_dim]   (ForwardOutput::normalized)
 *  out_pooled      NULL or [batch, embedding_dim]   (::pooled)
 *  out_projected   NULL or [total_tokens, embedding_dim] (::projected)
 *  out_hidden      NULL or [num_hidden_layers + 1, total_tokens, hidden]
 *                  (::hidden_states, capture_hidden = true)
 * Validation order per row follows text.rs:188-218: empty -> CORRUPT,
 * > 8192 or > max_position_embeddings -> LIMIT, id >= vocab -> CORRUPT; a
 * non-finite intermediate -> INTERNAL. */
svl_status svl_text_forward_batch(svl_text_model *model, const uint32_t *ids,
                                  const int64_t *offsets, int32_t batch,
                                  const svl_feature_span *features, float *out_normalized,
                                  float *out_pooled, float *out_projected, float *out_hidden);

/* Device-resident variant for serving loops: d_ids already in HBM, row
 * offsets on the host, Matryoshka outputs written to HBM as
 * d_out[batch, sum(dims)] (each block = truncate_and_normalize(normalized,
 * dims[i]), kernels.rs:916-927; dims[i] == embedding_dim gives normalized).
 * Enqueued on `stream` (NULL = the model's stream); the call returns after
 * the stream has drained and the device error flags have been read. */
svl_status svl_text_forward_device(svl_text_model *model, const uint32_t *d_ids,
                                   const int64_t *offsets, int32_t batch, const int32_t *dims,
                                   int32_t n_dims, float *d_out, void *stream);

/* TextModel::embed_ids (text.rs:546-554): one row, Matryoshka dimension. */
svl_status svl_text_embed_ids(svl_text_model *model, const uint32_t *ids, int64_t n,
                              int64_t dimension, float *out);

/* ForwardOutput::embedding / kernels::truncate_and_normalize
 * (text.rs:72-74, kernels.rs:916-927); host buffers. */
svl_status svl_truncate_and_normalize(const float *values, size_t n, size_t dimension,
                                      float *out);

/* TensorEntry::to_f32 (src/binary/safetensors.rs:69-110): decodes one view
 * into `out` (capacity floats): F32 read little-endian, BF16 widened exactly
 * (bits << 16, src/binary/bf16.rs:13-15). LimitExceeded above the element
 * cap, Corrupt when the payload length does not match the shape,
 * Unsupported for another dtype. Host only; no device is needed. */
svl_status svl_tensor_to_f32(const svl_tensor_view *tensor, float *out, int64_t capacity);

/* No counterpart in the reference (a measurement aid): the device's FP32
 * matrix rate from register-only MFMA chains on every SIMD, and its HBM
 * bandwidth from a 1 GiB device-to-device copy (read + written bytes per
 * second); best of a few timed launches each. Takes well under a second. */
svl_status svl_measure_peaks(svl_ctx *ctx, double *fp32_mfma_tflops, double *hbm_copy_gbs);
/* No counterpart in the reference (a measurement aid): the device's FP64
 * matrix rate from register-only v_mfma_f64_16x16x4f64 chains in four waves
 * on every SIMD; best of three timed launches of about 12 ms each. */
svl_status svl_measure_fp64_peak(svl_ctx *ctx, double *fp64_mfma_tflops);

/* Batches of 4096 tokens or more run as `groups` groups of rows (1..4,
 * default 3), group 0 on the caller's stream and the others on streams of
 * the model that wait for it and are joined back into it, so one group's
 * kernels fill the GPU while another's drain. groups <= 1 runs every batch
 * as one group on one stream. Results are bit-identical for any setting. */
svl_status svl_text_model_set_stream_split(svl_text_model *model, int groups);

/* Every forward entry point (svl_text_forward_batch, svl_text_forward_device,
 * the image and audio prompts) runs a batch as passes of consecutive rows of
 * at most `tokens` tokens each, one after another (a longer row runs alone),
 * so the device workspace stays bounded whatever the batch: row r of every
 * output still equals TextModel::forward(row r), bit for bit, like the
 * reference's loop over rows (text.rs:150-180). 0 (the default) sizes passes
 * to about 32 GiB of workspace (677,617 tokens at EmbeddingGemma's shape).
 * Usage error outside 0..=268435455. No counterpart in the reference, which
 * holds one row at a time. */
svl_status svl_text_model_set_pass_tokens(svl_text_model *model, int64_t tokens);

/* Per-kernel GPU time of the last forward call, when enabled: one entry per
 * kernel class (see svl_kernel_class_name). Used by the benchmark to relate
 * a kernel's algorithmic work to its measured duration. */
svl_status svl_text_model_set_kernel_timing(svl_text_model *model, int enable);
int32_t svl_kernel_class_count(void);
const char *svl_kernel_class_name(int32_t cls);
/* ms[cls] = summed milliseconds, launches[cls] = number of launches and
 * flops[cls] = algorithmic FLOPs (GEMMs, attention) or bytes (bandwidth
 * kernels) accumulated since timing was enabled. */
svl_status svl_text_model_kernel_stats(svl_text_model *model, double *ms, int64_t *launches,
                                       double *work);

/* ---- kernel seam: src/tensor/kernels.rs on device pointers --------------- */
/* Each call validates like its reference function, runs on `stream`, waits
 * for it, and returns INTERNAL if the output holds a non-finite value where
 * the reference checks for one. */

/* kernels.rs:577-685 linear: out[r, c] = sum_k in[r, k] * w[c, k]. */
svl_status svl_linear(const float *d_in, const float *d_w, int64_t rows, int64_t in_features,
                      int64_t out_features, float *d_out, void *stream);
/* kernels.rs:727-776 rms_norm_rows; d_weight == NULL gives
 * rms_norm_rows_unscaled (kernels.rs:810-857). */
svl_status svl_rms_norm_rows(const float *d_in, const float *d_weight, int64_t rows,
                             int64_t width, float eps, float *d_out, void *stream);
/* kernels.rs:936-988 rope_with_inv_freq on [seq, heads, head_dim], in place;
 * inv_freq is a host array of head_dim / 2 values. */
svl_status svl_rope_with_inv_freq(float *d_values, int64_t seq_len, int64_t num_heads,
                                  int64_t head_dim, const float *inv_freq, int64_t n_inv_freq,
                                  int64_t position_offset, void *stream);
/* kernels.rs:991-1010 rope_inv_freq (host). */
svl_status svl_rope_inv_freq(int64_t head_dim, float base, float *out);
/* kernels.rs:1037-1135 bidirectional_attention; sliding_window < 0 = full. */
svl_status svl_bidirectional_attention(const float *d_q, const float *d_k, const float *d_v,
                                       int64_t seq_len, int64_t num_heads,
                                       int64_t num_kv_heads, int64_t head_dim,
                                       int64_t sliding_window, float scale, float *d_out,
                                       void *stream);
/* No counterpart in the reference: svl_bidirectional_attention for callers
 * that cannot allocate device memory (tight serving loops, harnesses that
 * forbid hipMalloc). Same arguments, kernels and results; its work items,
 * position arrays and non-finite flag live in a 320 KiB device array of the
 * library, one per GPU, instead of per-call allocations. At most 8192 keys
 * and 16384 work items (LimitExceeded beyond). The call waits for its stream
 * and reads the non-finite flag back before it returns, so it cannot be
 * recorded into a HIP graph. Every call on a GPU shares that GPU's array:
 * calls in one process are serialised by a lock and return after their
 * stream has finished, and calls that overlap on one GPU by other means
 * race. */
svl_status svl_bidirectional_attention_noalloc(const float *d_q, const float *d_k,
                                               const float *d_v, int64_t seq_len,
                                               int64_t num_heads, int64_t num_kv_heads,
                                               int64_t head_dim, int64_t sliding_window,
                                               float scale, float *d_out, void *stream);
/* Test hook, no counterpart in the reference: fixes which attention kernel
 * every later attention launch of the process uses (the model forward passes
 * and the entry points above), so that tests can check the kernels that only
 * rows whose K/V operand window passes 2 GiB would otherwise reach.
 * 0 = by shape (the default), 1 = the fallback for such rows (the
 * register-staged MFMA kernel at head_dim 64 / 128 / 256, the generic kernel
 * otherwise), 2 = the generic kernel (one wave per query row and head; rows of
 * at most 8192 keys). Other values are Usage. Results stay within the
 * reference tolerance but are not bit-identical across paths; calls in flight
 * on other threads race with a change. */
svl_status svl_set_attention_path(int path);
/* kernels.rs:386-400 gelu_tanh / geglu, kernels.rs:44-52 add. */
svl_status svl_gelu_tanh(const float *d_in, int64_t n, float *d_out, void *stream);
svl_status svl_geglu(const float *d_gate, const float *d_up, int64_t n, float *d_out,
                     void *stream);
svl_status svl_add(const float *d_a, const float *d_b, int64_t n, float *d_out, void *stream);
/* kernels.rs:882-909 mean_pool and kernels.rs:414-444 l2_normalize. */
svl_status svl_mean_pool(const float *d_values, int64_t rows, int64_t width, float *d_out,
                         void *stream);
svl_status svl_l2_normalize(const float *d_in, int64_t n, float *d_out, void *stream);

/* ---- vision tower and image prompts --------------------------------------- */

typedef struct svl_vision_model svl_vision_model;

/* Validated vision configuration (src/model/vision.rs:58-70 VisionConfig;
 * patch_size 16 and pooling_kernel_size 3 are fixed, vision.rs:174-183). */
typedef struct {
    int64_t hidden_size;
    int64_t intermediate_size;
    int64_t num_hidden_layers;
    int64_t num_attention_heads;
    int64_t num_key_value_heads;
    int64_t head_dim;
    int64_t position_embedding_size;
    double rms_norm_eps;
    double rope_theta;
} svl_vision_config;

/* One preprocessed image (src/media/preprocess.rs:87-147 ImagePatches).
 * Only the first valid_patches rows are read, as VisionModel::forward does
 * (vision.rs:742-809): pixel_values [valid_patches, 768] (16x16x3 values per
 * patch), positions [valid_patches, 2] patch-grid (x, y). */
typedef struct {
    const float *pixel_values;
    const int32_t *positions;
    int64_t valid_patches;
    int64_t max_patches;
    int64_t grid_width;
    int64_t grid_height;
    int64_t soft_tokens;
} svl_image_patches;

/* src/model/image.rs:30-44 ImageSpecialTokens. */
typedef struct {
    uint32_t bos, eos, pad, boi, image, eoi;
} svl_image_special_tokens;

/* Validates the inventory like VisionWeights::decode (vision.rs:556-610):
 * unexpected vision_tower. / embed_vision. tensors, missing or mis-shaped
 * ones -> CORRUPT; packs the weights into HBM. Replaces VisionModel::new
 * (vision.rs:701-723) with its weights; text_hidden is the width of the
 * embedding projection's output. */
svl_status svl_vision_model_create(svl_ctx *ctx, const svl_vision_config *cfg,
                                   int64_t text_hidden, const svl_tensor_view *tensors,
                                   size_t n_tensors, svl_vision_model **out);
svl_status svl_vision_model_destroy(svl_vision_model *model);

/* Batches of two or more images and 4096 or more patches run the encoder
 * layers as `groups` groups of consecutive images (1..2, default 2), group 0
 * on the caller's stream and group 1 on a stream of the model, so that one
 * group's attention and norms overlap the other's projections. groups 1 runs
 * every batch on one stream; so does a call that captures hidden states.
 * Results are bit-identical for any setting. No reference counterpart (the
 * reference encodes one image at a time). */
svl_status svl_vision_model_set_stream_split(svl_vision_model *model, int groups);

/* Every vision and image entry point runs a batch as passes of consecutive
 * images of at most `patches` real patches each, one after another (a larger
 * image runs alone), so the device workspace stays bounded whatever the
 * batch; every output equals the one-pass run bit for bit (captured hidden
 * states keep the whole batch's [L + 1, patches, H] layout). 0 (the default)
 * sizes passes to about 32 GiB of workspace (931,461 patches, 404 images of
 * 2304 patches, at the EmbeddingGemma tower's shape). Usage error outside
 * 0..=268435455. No counterpart in the reference, which encodes one image at
 * a time. */
svl_status svl_vision_model_set_pass_patches(svl_vision_model *model, int64_t patches);

/* VisionModel::forward (vision.rs:742-959) for `batch` images at once; image
 * i's result equals the reference's forward(image i).
 *  out_soft    [sum soft_tokens, text_hidden]  (VisionOutput::pooled of each
 *              image, images back to back)
 *  out_hidden  NULL or [num_hidden_layers + 1, sum valid_patches, hidden]
 *              (VisionOutput::hidden_states, images back to back per layer)
 * Validation follows the reference's order: zero patches -> CORRUPT, a
 * position outside the table -> CORRUPT, negative positions and an
 * inconsistent pooling geometry -> INTERNAL, a non-finite value -> INTERNAL. */
svl_status svl_vision_forward_batch(svl_vision_model *model, const svl_image_patches *images,
                                    int32_t batch, float *out_soft, float *out_hidden);

/* Device-resident variant: d_pixels holds the images' patches back to back
 * in HBM ([sum valid_patches, 768]; the library rescales them in place);
 * images[i].pixel_values is ignored, positions stay on the host. Soft tokens
 * go to d_out [sum soft_tokens, text_hidden] on `stream` (NULL = the model's
 * stream); the call returns after the stream has drained. */
svl_status svl_vision_forward_device(svl_vision_model *model, float *d_pixels,
                                     const svl_image_patches *images, int32_t batch,
                                     float *d_out, void *stream);

/* ImageEmbedder::embed_impl (image.rs:209-253) for `batch` images: the
 * vision tower, then the prompt <bos> <boi> <image> x soft_tokens <eoi>
 * <eos> through the text model with the soft tokens replacing positions
 * [2, 2 + soft_tokens) (text.rs forward_with_features), then
 * ForwardOutput::embedding(dimension). out [batch, dimension]. The soft
 * tokens stay in HBM between the two models. */
svl_status svl_image_embed_batch(svl_vision_model *vision, svl_text_model *text,
                                 const svl_image_special_tokens *tokens,
                                 const svl_image_patches *images, int32_t batch,
                                 int64_t dimension, float *out);

/* The same with the images' patches already in HBM: d_pixels as in
 * svl_vision_forward_device (rescaled in place; images[i].pixel_values is
 * ignored). out [batch, dimension] on the host. */
svl_status svl_image_embed_device(svl_vision_model *vision, svl_text_model *text,
                                  const svl_image_special_tokens *tokens, float *d_pixels,
                                  const svl_image_patches *images, int32_t batch,
                                  int64_t dimension, float *out);

/* ---- audio tower and audio prompts ---------------------------------------- */

typedef struct svl_audio_model svl_audio_model;

/* Validated audio configuration (src/model/audio.rs:62-80 AudioConfig; the
 * intermediate size is 4 * hidden_size and head_dim hidden / heads, as
 * audio.rs:185-192 derives them). */
typedef struct {
    int64_t hidden_size;
    int64_t num_hidden_layers;
    int64_t num_attention_heads;
    int64_t conv_kernel_size;
    int64_t conv_channels0; /* subsampling_conv_channels[0] */
    int64_t conv_channels1; /* subsampling_conv_channels[1] */
    int64_t attention_chunk_size;
    int64_t attention_context_left;
    int64_t attention_context_right;
    int64_t output_proj_dims;
    double attention_logit_cap;
    double rms_norm_eps;
    double residual_weight;
    double gradient_clipping;
} svl_audio_config;

/* One clip's log-mel spectrogram (src/media/audio_preprocess.rs:50-90
 * MelSpectrogram): features [frames, 128] row-major, mask [frames] (1 for
 * frames whose window holds real audio). */
typedef struct {
    const float *features;
    const uint8_t *mask;
    int64_t frames;
} svl_mel;

/* src/model/audio_embedder.rs:32-46 AudioSpecialTokens. */
typedef struct {
    uint32_t bos, eos, pad, boa, audio, eoa;
} svl_audio_special_tokens;

/* Validates the inventory like AudioWeights::decode (audio.rs:717-794):
 * unexpected audio_tower. / embed_audio. tensors, missing or mis-shaped ones
 * and inverted clipping bounds -> CORRUPT; packs the weights into HBM and
 * computes each layer's relative keys once. Replaces AudioModel::new
 * (audio.rs:940-964) with its weights. */
svl_status svl_audio_model_create(svl_ctx *ctx, const svl_audio_config *cfg,
                                  int64_t text_hidden, const svl_tensor_view *tensors,
                                  size_t n_tensors, svl_audio_model **out);
svl_status svl_audio_model_destroy(svl_audio_model *model);

/* Number of valid audio tokens of a clip: subsampled row t is valid when
 * mask[4 t] is set (the two stride-2 subsamplings of audio.rs:1187-1240). */
int64_t svl_audio_token_count(const uint8_t *mask, int64_t frames);

/* AudioModel::forward (audio.rs:981-1134) for `batch` clips at once; clip
 * i's result equals the reference's forward(clip i).
 *  out_tokens  NULL or [batch] valid tokens per clip (AudioOutput::audio_tokens)
 *  out_soft    [sum tokens, text_hidden] (AudioOutput::pooled, clips back to back)
 *  out_sscp    NULL or [sum tokens, hidden] (AudioOutput::sscp_output)
 *  out_hidden  NULL or [num_hidden_layers, sum tokens, hidden] (hidden_states)
 * Validation follows the reference: zero frames or no valid subsampled token
 * -> CORRUPT, activation caps -> LIMIT, a non-finite value -> INTERNAL. */
svl_status svl_audio_forward_batch(svl_audio_model *model, const svl_mel *mels, int32_t batch,
                                   int64_t *out_tokens, float *out_soft, float *out_sscp,
                                   float *out_hidden);

/* Device-resident variant: d_features holds the clips' mel frames back to
 * back in HBM ([sum frames, 128]); mels[i].features is ignored, the masks
 * stay on the host. Soft tokens go to d_out [sum tokens, text_hidden] on
 * `stream` (NULL = the model's stream); the call returns after it drained. */
svl_status svl_audio_forward_device(svl_audio_model *model, const float *d_features,
                                    const svl_mel *mels, int32_t batch, float *d_out,
                                    void *stream);

/* AudioEmbedder::embed_impl (audio_embedder.rs:223-267) for `batch` clips:
 * the tower, then <bos> <boa> <audio> x tokens <eoa> <eos> through the text
 * model with the soft tokens replacing positions [2, 2 + tokens), then
 * ForwardOutput::embedding(dimension). out [batch, dimension]. The soft
 * tokens stay in HBM between the two models. */
svl_status svl_audio_embed_batch(svl_audio_model *audio, svl_text_model *text,
                                 const svl_audio_special_tokens *tokens, const svl_mel *mels,
                                 int32_t batch, int64_t dimension, float *out);
/* The same with the mel frames already in HBM (d_features as in
 * svl_audio_forward_device). */
svl_status svl_audio_embed_device(svl_audio_model *audio, svl_text_model *text,
                                  const svl_audio_special_tokens *tokens, const float *d_features,
                                  const svl_mel *mels, int32_t batch, int64_t dimension,
                                  float *out);

/* ---- log-mel front end ------------------------------------------------------ */

typedef struct svl_log_mel svl_log_mel;

/* Frame layout of log_mel (src/media/audio_preprocess.rs:94-131) for a clip
 * of `samples` 16 kHz samples (truncated at 480000, the 30 s cap of
 * src/media/audio.rs:19): mel frames, samples after right-padding to a
 * multiple of 128, and frames whose analysis window holds real audio.
 * Empty or too-short clips, and clips with no complete window -> CORRUPT. */
svl_status svl_log_mel_layout(int64_t samples, int64_t *frames, int64_t *padded_samples,
                              int64_t *valid_frames);

/* Uploads the Hann window, FFT twiddles and mel filter bank to the current
 * device of ctx. */
svl_status svl_log_mel_create(svl_ctx *ctx, svl_log_mel **out);
svl_status svl_log_mel_destroy(svl_log_mel *lm);

/* log_mel (audio_preprocess.rs:94-200) for `clips` clips of 16 kHz mono
 * samples: clip i is samples[i][0 .. lengths[i]). features receives the
 * clips' [frames_i, 128] spectrograms back to back and mask their frame
 * masks (1 = complete window), frames_i from svl_log_mel_layout. Bit-exact
 * with the reference's double-precision pipeline. An empty, too-short or
 * non-finite clip -> CORRUPT; a non-finite feature -> INTERNAL. */
svl_status svl_log_mel_batch(svl_log_mel *lm, const float *const *samples,
                             const int64_t *lengths, int32_t clips, float *features,
                             uint8_t *mask);
/* Device-resident variant: d_samples holds the clips back to back in HBM
 * (clip i at offset lengths[0] + ... + lengths[i - 1], all lengths[i]
 * samples checked for finiteness); d_features [sum frames_i, 128] is
 * written on `stream` (NULL = the object's stream); mask stays on the host.
 * Returns after the stream drained. */
svl_status svl_log_mel_device(svl_log_mel *lm, const float *d_samples, const int64_t *lengths,
                              int32_t clips, float *d_features, uint8_t *mask, void *stream);

/* AudioEmbedder::embed (audio_embedder.rs:214-267) from 16 kHz samples: the
 * log-mel spectrogram, the tower and the text model back to back on the
 * device, without the features leaving HBM. Clips as in svl_log_mel_batch;
 * out [clips, dimension]. */
svl_status svl_audio_embed_samples(svl_audio_model *audio, svl_text_model *text,
                                   const svl_audio_special_tokens *tokens,
                                   const float *const *samples, const int64_t *lengths,
                                   int32_t clips, int64_t dimension, float *out);
/* The same with the samples already in HBM (d_samples as in
 * svl_log_mel_device). */
svl_status svl_audio_embed_samples_device(svl_audio_model *audio, svl_text_model *text,
                                          const svl_audio_special_tokens *tokens,
                                          const float *d_samples, const int64_t *lengths,
                                          int32_t clips, int64_t dimension, float *out);

/* ---- tokenizer and text embedding from strings ---------------------------- */

typedef struct svl_tokenizer svl_tokenizer;

/* Tokenizer::from_json_str (src/model/tokenizer.rs:96-334): parses a
 * tokenizer.json document (UTF-8, at most 64 MiB, the JSON limits of
 * :569-578) and validates the BPE pipeline strictly: an inconsistent
 * document -> CORRUPT, a pipeline other than the frozen model's ->
 * UNSUPPORTED, a cap -> LIMIT. */
svl_status svl_tokenizer_create(const char *json, size_t len, svl_tokenizer **out);
svl_status svl_tokenizer_destroy(svl_tokenizer *tokenizer);

/* Tokenizer::encode (tokenizer.rs:339-389) of `len` bytes of UTF-8 text
 * (invalid UTF-8 -> CORRUPT). *count receives the number of ids; when it
 * exceeds `capacity` the call returns USAGE and writes nothing. Input above
 * 1 MiB or more than 262144 tokens -> LIMIT. */
svl_status svl_tokenizer_encode(const svl_tokenizer *tokenizer, const char *text, size_t len,
                                int add_special_tokens, uint32_t *ids, size_t capacity,
                                size_t *count);
/* encode for `n` texts on several host threads: text i's ids land in
 * ids[offsets[i] .. offsets[i + 1]) (offsets [n + 1]). The first failing
 * text, in order, gives the status. */
svl_status svl_tokenizer_encode_batch(const svl_tokenizer *tokenizer, const char *const *texts,
                                      const size_t *lens, int32_t n, int add_special_tokens,
                                      uint32_t *ids, size_t capacity, int64_t *offsets);
/* Tokenizer::decode (tokenizer.rs:391-425): an unknown id or invalid UTF-8
 * output -> CORRUPT; *len as in encode. */
svl_status svl_tokenizer_decode(const svl_tokenizer *tokenizer, const uint32_t *ids, size_t n,
                                int skip_special_tokens, char *out, size_t capacity, size_t *len);
/* tokenizer.rs:427-471 accessors; -1 / NULL where the reference returns
 * None. svl_tokenizer_token's string lives as long as the tokenizer. */
int64_t svl_tokenizer_token_id(const svl_tokenizer *tokenizer, const char *token, size_t len);
const char *svl_tokenizer_token(const svl_tokenizer *tokenizer, uint32_t id, size_t *len);
int64_t svl_tokenizer_vocab_size(const svl_tokenizer *tokenizer);
int64_t svl_tokenizer_max_token_id(const svl_tokenizer *tokenizer);
int64_t svl_tokenizer_bos_id(const svl_tokenizer *tokenizer);
int64_t svl_tokenizer_eos_id(const svl_tokenizer *tokenizer);
int64_t svl_tokenizer_unk_id(const svl_tokenizer *tokenizer);
int64_t svl_tokenizer_pad_id(const svl_tokenizer *tokenizer);
int svl_tokenizer_is_special_id(const svl_tokenizer *tokenizer, uint32_t id);

/* Prompt roles of src/model/prompt.rs:38-55, in that order. */
typedef enum {
    SVL_PROMPT_SEARCH_QUERY = 0,
    SVL_PROMPT_DOCUMENT = 1,
    SVL_PROMPT_CLASSIFICATION = 2,
    SVL_PROMPT_CLUSTERING = 3,
    SVL_PROMPT_CODE_RETRIEVAL = 4,
    SVL_PROMPT_FACT_CHECKING = 5,
    SVL_PROMPT_SENTENCE_SIMILARITY = 6,
    SVL_PROMPT_QUESTION_ANSWERING = 7
} svl_prompt;

/* TextEmbedder::embed (src/model/text.rs:610-626) for `n` texts: the
 * prompt's prefix, encode with <bos>/<eos> (host threads), more than 8192
 * tokens -> LIMIT, then one batched forward pass and
 * ForwardOutput::embedding(dimension) (dimension outside 1..=embedding_dim
 * -> INTERNAL). out [n, dimension]. */
svl_status svl_text_embed_texts(svl_text_model *model, const svl_tokenizer *tokenizer,
                                const char *const *texts, const size_t *lens, int32_t n,
                                int32_t prompt, int64_t dimension, float *out);

/* ---- exact vector search ---------------------------------------------------- */

typedef struct svl_vector_index svl_vector_index;

/* The vector view of Index::build (src/index/mod.rs:251-309): `n` chunk
 * embeddings [n, dimension] (host, caller order) with their chunk ids,
 * copied into HBM. An empty index has no dimension. dimension outside
 * 1..=8192 (storage/model.rs:35) -> LIMIT. */
svl_status svl_vector_index_create(svl_ctx *ctx, const float *embeddings,
                                   const uint64_t *chunk_ids, int64_t n, int64_t dimension,
                                   svl_vector_index **out);
svl_status svl_vector_index_destroy(svl_vector_index *index);
int64_t svl_vector_index_size(const svl_vector_index *index);
int64_t svl_vector_index_dimension(const svl_vector_index *index);

/* vector::rank (src/index/vector.rs:17-97) for `nq` queries [nq, query_dim]
 * and the pagination slice of Index::search (mod.rs:347-359): entries
 * [offset, offset + limit) of each query's ranking by descending cosine
 * score (computed in double exactly as the reference computes it), ties by
 * ascending chunk id. mask: NULL (no filter) or bytes in caller order, row
 * q at mask + q * mask_stride (mask_stride 0: one row for every query);
 * only chunks with a non-zero byte are ranked (Filters::matches).
 *  out_index  [nq, limit] caller indices of the hits
 *  out_score  [nq, limit] cosine scores
 *  out_count  [nq] hits written for each query
 * Validation per query in the reference's order: empty -> USAGE, more than
 * 8192 dimensions -> LIMIT, a non-finite value or a zero norm -> USAGE, a
 * dimension other than the index's -> USAGE; an admitted chunk with a zero
 * or non-finite norm -> INTERNAL. */
svl_status svl_vector_rank(svl_vector_index *index, const float *queries, int32_t nq,
                           int64_t query_dim, const uint8_t *mask, int64_t mask_stride,
                           int64_t offset, int64_t limit, int64_t *out_index, double *out_score,
                           int64_t *out_count);
/* The same with the queries already in HBM (d_queries [nq, query_dim], for
 * example the text embedder's device output); their norms and checks run on
 * `stream` (NULL = the index's stream). */
svl_status svl_vector_rank_device(svl_vector_index *index, const float *d_queries, int32_t nq,
                                  int64_t query_dim, const uint8_t *mask, int64_t mask_stride,
                                  int64_t offset, int64_t limit, int64_t *out_index,
                                  double *out_score, int64_t *out_count, void *stream);

/* ---- deterministic synthetic data (benchmark and tests) ------------------ */
/* Counter-based SplitMix64: element i of stream s under seed k is
 * u = (splitmix64(k ^ (s * 0x9E3779B97F4A7C15) + i) >> 40) / 2^24 in [0, 1),
 * scaled to [lo, hi). Host buffers; multithreaded. */
void svl_synth_uniform(uint64_t seed, uint64_t stream, float lo, float hi, size_t n, float *out);
/* floor(u * vocab) token ids and lo + floor(u * (hi - lo + 1)) lengths. */
void svl_synth_ids(uint64_t seed, uint64_t stream, uint32_t vocab, size_t n, uint32_t *out);
void svl_synth_lengths(uint64_t seed, uint64_t stream, int64_t lo, int64_t hi, size_t n,
                       int64_t *out);

#ifdef __cplusplus
}
#endif

#endif /* SVL_HIP_H */
