// Internal declarations shared by the host runtime (text_model.cpp, api.cpp)
// and the device translation unit (svl_device.hip). Kernel launchers take
// device pointers and a stream and return the launch status.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>

namespace svl {

// Device error flag bits (one int per model, read after every forward).
enum : int {
    FLAG_NONFINITE = 1,   // a non-finite activation (reference: Error::Internal)
    FLAG_BAD_TOKEN = 2,   // id >= vocab in the device-resident path (Error::Corrupt)
};

// GEMM epilogues: C = epilogue(A[M,K] . W[N,K]^T).
enum GemmEpi : int {
    EPI_STORE = 0,     // C[m,n] = acc
    EPI_SCALE = 1,     // C[m,n] = acc * alpha
    EPI_GEGLU = 2,     // W rows interleaved in 32-blocks (gate, up); C[m,j] = gelu(g) * u
    EPI_GELU_MUL = 3,  // C[m,n] = gelu(acc) * aux[m * ldaux + n]
    EPI_BIAS = 4,      // C[m,n] = acc + aux[n]
    // Clipped linears (audio tower): the sum is clamped to
    // [clip[s][2], clip[s][3]], s = n / clip_cols (0 when clip_cols == 0).
    // The A operand must already hold values clamped to the segment's input
    // bounds [clip[s][0], clip[s][1]]: the kernel that writes A applies that
    // clamp as it stores (the same operation on the same value, so the
    // product is unchanged), instead of every tile clamping every fragment
    // it reads. Segment s reads A + s * a_seg.
    EPI_CLIP_STORE = 5,  // C[m,n] = clamp(acc)
    EPI_CLIP_SILU = 6,   // C[m,n] = clamp(silu(clamp(acc)), post_lo, post_hi)
    EPI_CLIP_GLU = 7,    // W rows interleaved in 32-blocks (x, y); C[m,j] = clamp(x) * sigmoid(clamp(y))
};

struct GemmArgs {
    const float *A;
    int64_t lda;
    const float *W;
    int64_t ldw;
    float *C;
    int64_t ldc;
    int M, N, K;
    int epi;
    float alpha;
    const float *aux;
    int64_t ldaux;
    int n_out;  // EPI_GEGLU / EPI_CLIP_GLU: number of real output columns
    int cus = 0;               // > 0: the launch shares the GPU with other streams
    int clip_cols = 0;         // output columns per clip segment (0: one segment)
    float clip[4][4] = {};     // per segment: input min, input max, output min, output max
    int64_t a_seg = 0;         // floats from one clip segment's A operand to the next's
    // EPI_CLIP_SILU: bounds of the next clipped linear's input, applied as
    // the result is stored (the identity by default)
    float post_lo = -__builtin_huge_valf(), post_hi = __builtin_huge_valf();
    // launch_gemm_conv: implicit im2col for the audio subsampling's layer-1
    // 3x3 stride-2 convolution. A is the layer-0 output [rows0, conv_f0,
    // conv_c0]; row m of the virtual A is output position (r, f) = (m /
    // conv_f1, m % conv_f1) of layer-1 row conv_rows[r] = {base, t, len}, and
    // its column k = tap * conv_c0 + c (tap = 3 kt + kf) holds layer-0 row
    // base + 2 t + kt - 1, frequency 2 f + kf - 1, channel c, or zero outside
    // the clip, on a masked row (conv_mask[base + row] == 0) or outside the
    // frequencies. W is [N][9][conv_c0].
    const int32_t *conv_rows = nullptr;
    const uint8_t *conv_mask = nullptr;
    int conv_c0 = 0, conv_f0 = 0, conv_f1 = 0;
    int64_t conv_a_floats = 0;  // floats of the layer-0 output (A's window)
};

hipError_t launch_gemm(const GemmArgs &a, hipStream_t s);
// True when launch_gemm_conv can take the convolution (conv_c0 % 32 == 0,
// windows below 2 GiB).
bool gemm_conv_ok(const GemmArgs &a);
hipError_t launch_gemm_conv(const GemmArgs &a, hipStream_t s);
// Plain scalar-FMA fallback for shapes the MFMA kernel does not take
// (K % 4 != 0); same epilogues.
hipError_t launch_gemm_simple(const GemmArgs &a, hipStream_t s);

// out = rms_norm_rows(x, w) (w == nullptr: unscaled).
hipError_t launch_rms_rows(const float *x, const float *w, float *out, int64_t rows, int width,
                           float eps, int *flag, hipStream_t s);

// h_out = (res + rms(x, w1)) * scale ; if w2: n_out = rms(h_out, w2).
hipError_t launch_resnorm(const float *x, const float *w1, const float *res, float *h_out,
                          const float *w2, float *n_out, float scale, int64_t rows, int width,
                          float eps, int *flag, hipStream_t s);

// h[t] = table[ids[t]] * scale, or feats[featmap[t]] when featmap[t] >= 0;
// n[t] = rms(h[t], w_in).
hipError_t launch_gather(const uint32_t *ids, const float *table, int64_t vocab,
                         const int32_t *featmap, const float *feats, float scale,
                         const float *w_in, float *h, float *n, int64_t tokens, int width,
                         float eps, int *flag, hipStream_t s);

// In place on qkv[T, ld]: per-head q RMSNorm(q_norm) + RoPE, k RMSNorm(k_norm)
// + RoPE, v unscaled RMSNorm. cos/sin tables are [positions, hd/2].
hipError_t launch_qkv_post(float *qkv, int64_t ld, int64_t tokens, int nh, int nkv, int hd,
                           const float *qn, const float *kn, const float *cos_t,
                           const float *sin_t, const int32_t *pos, float eps, int *flag,
                           hipStream_t s);

// RoPE only (kernel seam): values [T, heads, hd], position = pos0 + t.
hipError_t launch_rope(float *x, int64_t tokens, int heads, int hd, const float *cos_t,
                       const float *sin_t, int *flag, hipStream_t s);

// Work item of the attention kernel: one kv head of one row, a block of
// query vectors [qv0, qv0 + block) where vector v = (pos v / G, head kvh*G + v % G).
struct AttnTile {
    int32_t tok0;  // first token of the row in the packed layout
    int32_t len;   // row length
    int32_t kvh;   // key/value head
    int32_t qv0;   // first query vector of the block
};

struct AttnArgs {
    const float *q;  // token t, head h at q + t * ldq + h * hd
    const float *k;  // token t, kv head g at k + t * ldk + g * hd
    const float *v;
    float *out;      // token t, head h at out + t * ldo + h * hd
    int64_t ldq, ldk, ldv, ldo;
    int nh, nkv, hd;
    int window;      // < 0: full attention
    float scale;
    const AttnTile *tiles;  // MFMA kernel work items
    int n_tiles;
    const int32_t *pos;     // per token: position in its row (simple kernel)
    const int32_t *rowlen;  // per token: length of its row (simple kernel)
    int64_t tokens;
    int *flag;
    int64_t max_len = 0;    // bound on the row length (0: unknown, bounded by tokens)
    int64_t shortest = 0;   // shortest row of the launch (0: unknown)
};
// Query vectors per work item of the MFMA kernel (0 if hd has no MFMA kernel).
int attn_block_vectors(int hd);
hipError_t launch_attention(const AttnArgs &a, hipStream_t s);
// Attention kernel choice for every later launch in the process (a test
// hook): by shape (the DMA kernel whenever a row's operand window fits 2 GiB),
// the fallback that longer windows take (the register-staged MFMA kernel at
// head_dim 64 / 128 / 256, the generic kernel at 512), or the generic kernel.
constexpr int ATTN_PATH_AUTO = 0, ATTN_PATH_FALLBACK = 1, ATTN_PATH_GENERIC = 2;
void set_attention_path(int path);

// Scratch of the allocation-free attention entry point (noalloc.hip), one
// copy per GPU: work items, then per-token positions and row lengths, then
// the non-finite flag. 320 KiB in all.
constexpr int NOALLOC_MAX_KEYS = 8192;
constexpr int NOALLOC_MAX_TILES = 16384;
constexpr size_t NOALLOC_TILES_OFF = 0;
constexpr size_t NOALLOC_POS_OFF = NOALLOC_TILES_OFF + NOALLOC_MAX_TILES * sizeof(AttnTile);
constexpr size_t NOALLOC_LEN_OFF = NOALLOC_POS_OFF + NOALLOC_MAX_KEYS * sizeof(int32_t);
constexpr size_t NOALLOC_FLAG_OFF = NOALLOC_LEN_OFF + NOALLOC_MAX_KEYS * sizeof(int32_t);
constexpr size_t NOALLOC_SCRATCH_BYTES = NOALLOC_FLAG_OFF + 256;
// Device address of `device`'s scratch (looked up once per device).
hipError_t noalloc_scratch(int device, void **out);
// Work items of one row of `seq` keys (per_head per KV head, bv query
// vectors each), positions 0..seq-1, row lengths seq, flag cleared.
hipError_t launch_noalloc_attn_setup(void *base, int seq, int per_head, int bv, int n_tiles,
                                     hipStream_t s);

// Measured FP32 MFMA rate (register-only chains on every SIMD) and HBM copy
// bandwidth of the current device (probe.hip).
hipError_t probe_peaks(double *fp32_mfma_tflops, double *hbm_copy_gbs);
hipError_t probe_fp64_peak(double *fp64_mfma_tflops);

// Per row r of [offsets[r], offsets[r+1]): pos[t] = t - offsets[r] and
// rowlen[t] = offsets[r+1] - offsets[r] (rowlen may be null).
hipError_t launch_positions(const int64_t *offsets, int batch, int32_t *pos, int32_t *rowlen,
                            hipStream_t s);

// Mean pool + L2 + Matryoshka per row (masked segmented reduction).
// pooled [batch, width] is required; normalized and trunc_out
// [batch, sum(dims)] may be null.
hipError_t launch_pool(const float *proj, int width, const int64_t *offsets, int batch,
                       const int32_t *dims, int n_dims, int dims_total, float *pooled,
                       float *normalized, float *trunc_out, int *flag, hipStream_t s);
// L2 normalisation and Matryoshka truncations of already pooled rows.
hipError_t launch_pool_norm(const float *pooled, int width, int batch, const int32_t *dims,
                            int n_dims, int dims_total, float *normalized, float *trunc_out,
                            int *flag, hipStream_t s);

// Elementwise seam kernels.
hipError_t launch_gelu(const float *x, float *y, int64_t n, hipStream_t s);
hipError_t launch_geglu(const float *g, const float *u, float *y, int64_t n, hipStream_t s);
hipError_t launch_add(const float *a, const float *b, float *y, int64_t n, hipStream_t s);
hipError_t launch_finite_check(const float *x, int64_t n, int *flag, hipStream_t s);

// ---- vision tower row kernels ------------------------------------------------
// y = 2 * (x - 0.5), n % 4 == 0.
hipError_t launch_patch_scale(const float *x, float *y, int64_t n, hipStream_t s);
// h[t] += table[0][x_t] + table[1][y_t] with pos [T, 2] (x, y) and table
// [2, pos_size, width]; n[t] = rms(h[t], w). width % 4 == 0, <= 2048.
hipError_t launch_patch_pos(float *h, const int32_t *pos, const float *table, int64_t pos_size,
                            const float *w, float *n, int64_t rows, int width, float eps,
                            int *flag, hipStream_t s);
// In place on qkv[T, ld]: per-head q RMSNorm(qn) + axial RoPE, k RMSNorm(kn)
// + axial RoPE, v unscaled RMSNorm. cos/sin tables are [coordinate, hd/4].
hipError_t launch_qkv_post_axial(float *qkv, int64_t ld, int64_t tokens, int nh, int nkv, int hd,
                                 const float *qn, const float *kn, const float *cos_t,
                                 const float *sin_t, const int32_t *pos, float eps, int *flag,
                                 hipStream_t s);
// out[s] = unscaled_rms((sum of h over bin s in patch order / divisor) * scale).
hipError_t launch_pool_bins(const float *h, const int32_t *bin_start, const int32_t *bin_patch,
                            int64_t soft_tokens, int width, float divisor, float scale, float eps,
                            float *out, int *flag, hipStream_t s);

// ---- audio tower kernels -----------------------------------------------------

// One output row of a subsampling convolution: its input rows are
// [base, base + len) of the packed input (the clip's rows), and it is row t
// of the clip's output.
struct SscpRow {
    int32_t base;
    int32_t t;
    int32_t len;
};
static_assert(sizeof(SscpRow) == 3 * sizeof(int32_t), "GemmArgs::conv_rows reads SscpRow triplets");

// Mel [frames, 128] -> layer 0 [rows, 64, C0] (conv 3x3 stride 2 pad 1,
// masked frames skipped, LayerNorm + ReLU). C0 <= 512.
hipError_t launch_sscp_conv0(const float *mel, const uint8_t *mask, const SscpRow *rows,
                             int64_t n_rows, const float *w, const float *ln, int C0, float eps,
                             float *out, int *flag, hipStream_t s);
// In place: x[p] = relu(layernorm(x[p], ln)) over C channels, n positions.
hipError_t launch_sscp_ln_relu(float *x, const float *ln, int C, int64_t n, float eps, int *flag,
                               hipStream_t s);
// Clamped stores of a row kernel's last output (the A operand of a clipped
// linear): copy c goes to out + c * stride clamped to [lo[c], hi[c]]. The
// default is one unclamped copy.
struct OutClamp {
    int copies = 1;
    int64_t stride = 0;
    float lo[3] = {-__builtin_huge_valf(), -__builtin_huge_valf(), -__builtin_huge_valf()};
    float hi[3] = {__builtin_huge_valf(), __builtin_huge_valf(), __builtin_huge_valf()};
};
// t = w1 ? rms(clamp(x, +-c1), w1) : x; h = res ? res + t * rw : t (-> h_out);
// if w2: n_out = rms(clamp(h, +-c2), w2). `oc` applies to the last output
// written: n_out when w2 is given, else h_out.
hipError_t launch_audio_rows(const float *x, float c1, const float *w1, const float *res, float rw,
                             float *h_out, float c2, const float *w2, float *n_out, int64_t rows,
                             int width, float eps, int *flag, hipStream_t s,
                             const OutClamp &oc = OutClamp());

struct AudioAttnArgs {
    const float *q, *k, *v;      // head h of row i at q + i * ldq + h * head_dim
    int64_t ldq, ldk, ldv;
    const float *relk;           // [positions, heads * head_dim]
    const float *qf;             // [head_dim] query scale per dimension
    float k_scale, cap;
    const uint8_t *mask;         // [rows] valid rows
    const int32_t *pos, *rowlen; // row index within its clip, clip length
    float *out;
    int64_t ldo;
    const int32_t *blocks;       // first row of each block of `chunk` rows of a clip
    int64_t n_blocks;
    int heads, head_dim, chunk, left, context, positions;
    int *flag;
    // the output projection's input bounds, applied as the output is stored
    float out_lo = -__builtin_huge_valf(), out_hi = __builtin_huge_valf();
};
hipError_t launch_audio_attention(const AudioAttnArgs &a, hipStream_t s);
// Causal depthwise conv (dw tap-major, [K, width]) within each clip, clamp, RMSNorm(w), SiLU,
// stored clamped to [out_lo, out_hi] (the next linear's input bounds).
hipError_t launch_lconv(const float *gated, const float *dw, int K, const int32_t *pos, float clip,
                        const float *w, float *out, int64_t rows, int width, float eps, int *flag,
                        hipStream_t s, float out_lo = -__builtin_huge_valf(),
                        float out_hi = __builtin_huge_valf());
// out[j] = unscaled_rms(x[idx[j]]).
hipError_t launch_compact_rms(const float *x, const int32_t *idx, float *out, int64_t rows,
                              int width, float eps, int *flag, hipStream_t s);

// ---- log-mel front end ---------------------------------------------------------
// One clip of packed 16 kHz samples: samples [sample_base, sample_base +
// samples) (already truncated to 30 s), frames [frame_base, frame_base + frames).
struct MelClip {
    int64_t sample_base;
    int64_t frame_base;
    int32_t samples;
    int32_t frames;
};
// Device tables: Hann window [320] f32, twiddles [256] (cos, sin) f64, and the
// non-zero mel filter weights in CSR form: filter f owns entries
// [filt_start[f], filt_start[f + 1]) of (filt_bin, filt_weight), bins ascending.
struct MelTables {
    const float *window;
    const double *twiddle;
    const int32_t *filt_start;
    const int32_t *filt_bin;
    const double *filt_weight;
};
// out [total_frames, 128]; frames whose window is incomplete are zero rows.
hipError_t launch_log_mel(const float *x, const MelClip *clips, int n_clips, int64_t total_frames,
                          const MelTables &t, float *out, int *flag, hipStream_t s);

// ---- exact cosine search ---------------------------------------------------------
// keys[q, c] = descending total-order key of dot(Q[q], V[c]) / (qnorm[q] *
// cnorm[c]) accumulated in double in d order; all ones when mask (indexed
// mask[q * mask_stride + perm[c]]) is given and zero.
// Qd: scratch of D * round_up(nq, cosine_query_block(nq)) doubles.
int cosine_query_block(int nq);
hipError_t launch_cosine_keys(const float *V, const double *cnorm, const float *Q,
                              const double *qnorm, int nq, int64_t n, int D, const uint8_t *mask,
                              int64_t mask_stride, const int64_t *perm, double *Qd,
                              uint64_t *keys, hipStream_t s);
// qnorm[q] = sqrt(sum Q[q, d]^2) in d order; flag bit 1: a non-finite value,
// bit 2: a zero or non-finite norm (per query: flags[q]).
hipError_t launch_query_norms(const float *Q, int nq, int D, double *qnorm, int *flags,
                              hipStream_t s);
// Stable ranking of all nq * n keys by (query, key, position). With tmp ==
// nullptr only *tmp_bytes is computed. *sorted receives the buffer (idx or
// idx_alt) that holds the flat pair indices q * n + c in ranked order.
hipError_t rank_sort(const uint64_t *keys, uint64_t *keys_alt, uint32_t *idx, uint32_t *idx_alt,
                     uint32_t *qkey, int nq, int64_t n, void *tmp, size_t *tmp_bytes,
                     const uint32_t **sorted, hipStream_t s);
// Top-K selection for pages far smaller than the index: SAMPLE_COUNT samples
// per query (every (n / SAMPLE_COUNT)-th key, n >= SAMPLE_COUNT), sorted per
// query into sorted[q * SAMPLE_COUNT ...]; candidates are the admitted keys
// <= sorted sample `rank`, in position order (at most cap stored per query,
// cnt[q] counts all); the candidates sorted by (key, position); and the page
// gathered.
constexpr int SAMPLE_COUNT = 4096;
hipError_t sort_samples(const uint64_t *keys, int nq, int64_t n, uint64_t *sorted,
                        hipStream_t s);
// Only the sample of rank `rank` (into sorted[q * SAMPLE_COUNT + rank]), by
// counting; the faster choice up to SELECT_SAMPLE_MAX_QUERIES queries.
constexpr int SELECT_SAMPLE_MAX_QUERIES = 4;
hipError_t select_sample(const uint64_t *keys, int nq, int64_t n, int rank, uint64_t *sorted,
                         hipStream_t s);
// blk_count: candidate_blocks(n) * nq counters.
int candidate_blocks(int64_t n);
hipError_t launch_compact_keys(const uint64_t *keys, int nq, int64_t n,
                               const uint64_t *sorted_samples, int S, int rank, int64_t cap,
                               unsigned int *blk_count, unsigned int *cnt, uint64_t *cand_key,
                               uint32_t *cand_idx, hipStream_t s);
// Candidates sorted on chip when every query has at most CAND_LDS of them
// (cnt[q] <= min(cap, most), most = the longest list <= CAND_LDS), into
// key_alt / idx_alt.
constexpr int CAND_LDS = 8192;
hipError_t sort_candidates_lds(const uint64_t *cand_key, const uint32_t *cand_idx,
                               uint64_t *key_alt, uint32_t *idx_alt, const unsigned int *cnt,
                               int nq, int64_t cap, int64_t most, hipStream_t s);
// Stable sort of each query's candidates by key into key_alt / idx_alt.
hipError_t sort_candidates(const uint64_t *cand_key, const uint32_t *cand_idx, uint64_t *key_alt,
                           uint32_t *idx_alt, const unsigned int *cnt, unsigned int *begin,
                           unsigned int *end, int nq, int64_t cap, void *tmp, size_t *tmp_bytes,
                           hipStream_t s);
hipError_t launch_gather_candidates(const uint64_t *cand_key, const uint32_t *cand_idx, int nq,
                                    int64_t n, int64_t cap, const int64_t *perm, int64_t offset,
                                    int64_t limit, const int64_t *take, int64_t *out_index,
                                    double *out_score, hipStream_t s);
// out_index / out_score [nq, limit]: ranked entries [offset, offset + take[q]).
hipError_t launch_gather_hits(const uint64_t *keys, const uint32_t *sidx, int nq, int64_t n,
                              const int64_t *perm, int64_t offset, int64_t limit,
                              const int64_t *take, int64_t *out_index, double *out_score,
                              hipStream_t s);

}  // namespace svl
