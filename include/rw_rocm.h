/*
 * rw_rocm.h -- C ABI of librw_rocm.so, the MI355X (gfx950) implementation of
 * rusty_whisper's quantized linear-layer matmul.
 *
 * The reference computes y = x W^T (+ b) with W held in ggml blocks
 * (Q4_0 / Q4_1 / Q5_0 / Q5_1 / Q8_0, 32 elements per block) and x an f32
 * Tensor, through:
 *   QTensor::new            src/quant.rs:553-563
 *   QTensor::{row_f32,to_dense}  src/quant.rs:566-576
 *   matmul_t_q              src/quant.rs:754-1051
 *   linear_w                src/quant.rs:1054-1063
 * Each entry below names the reference function it replaces.  Activations
 * are quantized per 32-block to int8 exactly as quantize_acts_i8
 * (src/quant.rs:691-716) does, and each output is
 *     sum_bl d_a*d_b*S + m_b*d_a*sum(q_a)   (+ bias, added last)
 * with S = sum(q_a*q_b) the per-block integer sum.  Decode-shape products
 * (m <= 8) form S exactly and combine in f32 as the reference does.
 * Encoder-shape products (m > 8) multiply the same values as f16 operands
 * d_a*q_a and d_b*q_b + m_b (one rounding each; each activation row and each
 * weight row scaled by its own power of two first, so no operand overflows
 * or loses precision to f16 subnormals whatever the block scales are) with
 * exact products and f32 accumulation on the matrix cores: within
 * 2^-10 * sum|a||w| plus f32 accumulation error of the exact result, far
 * inside the 1e-3 (row-L2) agreement with the reference CPU path.  So the
 * exact per-block integer sums S are formed on the product path for m <= 8
 * only; for m > 8 the validation entry rw_rocm_block_dots (below) forms them,
 * bit for bit, off the product path.
 *
 * Conventions (the crate's existing C ABI, src/wasm.rs:25-110, returns an
 * i32 status and keeps error text separately):
 *   - every function returns RW_OK (0) or a negative RW_E* code;
 *   - rw_rocm_last_error() copies the calling thread's last error text;
 *   - no function aborts the process on bad input; the reference panics on
 *     the same conditions (src/quant.rs:757-758, 129), and its Rust binding
 *     turns a non-zero status back into that panic.
 * Thread safety: every entry point may be called concurrently from several
 * threads on shared rw_weight handles (the reference shares &Model across
 * transcription threads, src/transcribe.rs:1525-1552).  Host-pointer entries
 * are synchronous.  Device-pointer entries are asynchronous on the stream
 * passed in; called without a workspace they use one buffer of the
 * library's per (device, stream), which a call holds until its launches are
 * queued, so concurrent calls on one stream queue one after the other and
 * never share it.  Calls that pass one caller workspace race on it unless
 * the caller orders them.  An rw_decoder is one decoding state: its calls
 * must not overlap.
 */
#ifndef RW_ROCM_H
#define RW_ROCM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RW_OK 0
#define RW_EINVAL (-1)  /* bad dtype, k % 32 != 0, shape or length mismatch, NULL */
#define RW_ENODEV (-2)  /* no usable gfx950 device / bad device index */
#define RW_EHIP (-3)    /* a HIP runtime call failed */
#define RW_ENOMEM (-4)  /* device allocation failed */
#define RW_EIO (-5)     /* a model file cannot be opened, read or mapped */

/* ggml dtype ids (src/quant.rs:43-52) */
#define RW_Q4_0 2
#define RW_Q4_1 3
#define RW_Q5_0 6
#define RW_Q5_1 7
#define RW_Q8_0 8

typedef struct rw_weight rw_weight;

/* Library version, e.g. 0x000100 for 0.1.0. */
int rw_rocm_version(void);

/* Number of visible devices this library can run on (gfx950 only), or a
 * negative RW_E* code. */
int rw_rocm_device_count(void);

/* Select and initialise `device` for the calling thread.  Fails with
 * RW_ENODEV when it is absent or not gfx950.  Replaces nothing in the
 * reference (the CPU path needs no set-up); the Rust binding calls it once,
 * from the OnceLock that guards device use. */
int rw_rocm_init(int device);

/* Bytes per ggml block of `dtype` (18/20/22/24/34), or RW_EINVAL.
 * Replaces block_bytes, src/quant.rs:43-52. */
int rw_rocm_block_bytes(int dtype);

/* Upload an [n, k] ggml-quantized matrix (n rows of k/32 consecutive blocks,
 * src/quant.rs:493-494) to the current device.  The blocks are repacked once,
 * on the device, into the resident layout the kernels read; they stay in HBM
 * until rw_rocm_weight_free.  raw_len must equal n*(k/32)*block_bytes(dtype).
 * Replaces QTensor::new (src/quant.rs:553-563) plus its lazily packed int8
 * cache (src/quant.rs:589-639). */
int rw_rocm_weight_upload(int dtype, size_t n, size_t k, const uint8_t *raw, size_t raw_len,
                          rw_weight **out);

/* Release a weight (the Rust Drop of the device handle). NULL is a no-op. */
int rw_rocm_weight_free(rw_weight *w);

/* dtype, rows, cols and resident device bytes of an uploaded weight. */
int rw_rocm_weight_info(const rw_weight *w, int *dtype, size_t *n, size_t *k, size_t *device_bytes);

/* out[m, n] = a[m, k] W^T (+ bias[n] when bias != NULL), host pointers,
 * synchronous.  Replaces matmul_t_q (src/quant.rs:754-1051) and, with a
 * bias, linear_w's Quant arm (src/quant.rs:1054-1063).  m == 0 is valid and
 * writes nothing. */
int rw_rocm_matmul_t_q(const rw_weight *w, const float *a, size_t m, size_t k, const float *bias,
                       float *out);

/* The dense f32 tier: out[m, n] = a[m, k] b[n, k]^T (+ bias[n] when bias
 * != NULL), host pointers, synchronous, on the calling thread's current
 * device.  Replaces tensor::matmul_t (src/tensor.rs:194-238) and, with a
 * bias, linear_w's Dense arm (src/quant.rs:1054-1063): every element is the
 * reference's tensor::dot (8 lane accumulators, products and sums rounded
 * separately, lanes and tail summed from -0.0) plus the bias, so results
 * are bit-identical.  m == 0 is valid and writes nothing. */
int rw_rocm_matmul_t_f32(const float *a, size_t m, size_t k, const float *b, size_t n, const float *bias,
                         float *out);
/* The same with device pointers (a, b, bias, out on the current device),
 * queued on `stream` without waiting.  No reference counterpart as such. */
int rw_rocm_matmul_t_f32_dev(const float *a, size_t m, size_t k, const float *b, size_t n, const float *bias,
                             float *out, void *stream);

/* Device-resident form of rw_rocm_matmul_t_q: a, bias and out are device
 * pointers on the weight's device; the work is queued on `stream` (a
 * hipStream_t; NULL = the default stream) and the call returns without
 * waiting.  For m > 8, `workspace` (device memory, >=
 * rw_rocm_matmul_workspace_size(m, k) bytes) holds the quantized
 * activations; NULL makes the library use a buffer of its own for this
 * stream (grown as needed, so it may allocate).  For m <= 8 the activations
 * are quantized inside the product's one launch and `workspace` is not
 * used.
 * Has no reference counterpart as such: it is matmul_t_q without the host
 * copies, for callers that keep activations on the device. */
int rw_rocm_matmul_t_q_dev(const rw_weight *w, const float *a, size_t m, size_t k,
                           const float *bias, float *out, void *workspace, size_t workspace_len,
                           void *stream);

/* Workspace bytes rw_rocm_matmul_t_q_dev needs for an [m, k] activation. */
size_t rw_rocm_matmul_workspace_size(size_t m, size_t k);

/* rw_rocm_matmul_t_q_dev without any allocation: the same kernels and bit
 * for bit the same results, with the quantized activation kept in a fixed
 * RW_NOALLOC_SCRATCH_BYTES array of device memory that each GPU running the
 * library holds until the process ends.  No hipMalloc, hipFree or other
 * allocating call happens inside it.  Inputs whose workspace
 * (rw_rocm_matmul_workspace_size) exceeds the array are rejected with
 * RW_EINVAL; 16 MiB covers m = 1500 rows at k = 5120.  Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (two streams, or
 * two threads) race on it, so a caller orders them.  Call rw_rocm_init for
 * the device first where possible (it looks the array's address up; the
 * first call on a device does otherwise).  Has no counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid it). */
#define RW_NOALLOC_SCRATCH_BYTES (16 << 20)
int rw_rocm_matmul_t_q_dev_noalloc(const rw_weight *w, const float *a, size_t m, size_t k,
                                   const float *bias, float *out, void *stream);

/* The two halves of rw_rocm_matmul_t_q_dev, for callers that reuse one
 * quantized activation across several weights.  rw_rocm_quantize_dev runs
 * quantize_acts_i8 (src/quant.rs:691-716) on device a[m, k] into `workspace`;
 * rw_rocm_matmul_prequant_dev then computes out = a W^T (+ bias) from that
 * workspace (same m, and W's k must equal the k it was quantized with).
 * The reference quantizes inside every matmul_t_q call
 * (src/quant.rs:766); its Q, K and V projections share their input
 * (src/encoder.rs:130-141, src/decoder.rs:148-158), so quantizing once and
 * running three products gives bitwise the same three results. */
int rw_rocm_quantize_dev(const float *a, size_t m, size_t k, void *workspace, size_t workspace_len,
                         void *stream);
int rw_rocm_matmul_prequant_dev(const rw_weight *w, const void *workspace, size_t m, const float *bias,
                                float *out, void *stream);

/* Several products from one quantized activation in one launch:
 * out[i][m, n_i] = a W_i^T (+ bias[i]) for i < count, 1 <= count <= 4, with
 * `workspace` filled by rw_rocm_quantize_dev (same m and k).  The weights
 * share dtype, k and device; `bias` may be NULL (no biases) or hold NULL
 * entries.  Replaces the linear_w calls on one input of src/encoder.rs:130-141
 * (Q, K and V of the self-attention; Q/K/V of src/decoder.rs:148-158 in the
 * decode shape).  For m > 8 the weights' column tiles share one GEMM launch
 * whose k split is chosen from all of them, so a result can differ from
 * rw_rocm_matmul_prequant_dev's in the last bits of the f32 sums (within
 * the same error bound); it never depends on m.  For m <= 8 each weight
 * runs its own decode launch, bitwise rw_rocm_matmul_prequant_dev. */
int rw_rocm_matmul_prequant_multi_dev(const rw_weight *const *w, size_t count, const void *workspace, size_t m,
                                      const float *const *bias, float *const *out, void *stream);

/* The encoder MLP's middle (src/encoder.rs:161-171, gelu src/tensor.rs:
 * 289-305): y = gelu(a W^T + bias) from `workspace` filled by
 * rw_rocm_quantize_dev (m rows, W's k), quantized (quantize_acts_i8) into
 * `next_workspace` as rw_rocm_quantize_dev would leave it for y -- ready for
 * rw_rocm_matmul_prequant_dev with the next weight (k = W's n).  y itself is
 * never written: the product's epilogue applies the bias and GELU and
 * quantizes each 32-column block, one more launch builds the next product's
 * f16 operand, and that operand is bitwise the one rw_rocm_quantize_dev makes
 * from the f32 y, so the next product's result is too.  The f32 y is never
 * in memory (at m = 1500, n = 5120 that is 31 MB not written and read back);
 * on large-v3 the pair costs about what the product, an f32 y and
 * rw_rocm_quantize_dev cost.  m > 8 (the encoder shape), W's n a multiple of
 * 32; next_workspace holds rw_rocm_gelu_quantize_workspace_size(m, n) bytes
 * (0 for shapes it does not take). */
size_t rw_rocm_gelu_quantize_workspace_size(size_t m, size_t n);
int rw_rocm_matmul_prequant_gelu_quantize_dev(const rw_weight *w, const void *workspace, size_t m,
                                              const float *bias, void *next_workspace, size_t next_len,
                                              void *stream);

/* One entry of a grouped launch: out_g[m_g, n_g] = a_g W_g^T (+ bias_g). */
typedef struct rw_linear {
    const rw_weight *w;
    const float *a;    /* device [m, k] */
    const float *bias; /* device [n] or NULL */
    float *out;        /* device [m, n] */
    size_t m;
} rw_linear;

/* Run `count` independent linears, each with m <= 8 (the decode-GEMV
 * regime), in two launches per distinct (dtype, m): every linear's
 * activation is quantized once, then all products run; entries with m == 0
 * are skipped.  Device pointers, asynchronous on `stream`.  Each result
 * has the same exact per-block integer sums and the same per-block combine
 * as the same linear run alone through rw_rocm_matmul_t_q_dev, and agrees
 * with it within a few f32 roundings: a single linear's launch splits a
 * row's blocks over more wavefronts (it is short of workgroups at decode
 * sizes), so the parts' f32 sums are added in another order.  Results of one
 * call do not depend on the other items of the call.  The launch tables go
 * to `workspace` (>=
 * rw_rocm_grouped_workspace_size bytes; NULL = a buffer of the library's own
 * for this stream) through pinned host memory on `stream`, and the quantized
 * activations are kept there; calls that overlap on one workspace race.
 * Replaces a
 * sequence of independent linear_w calls (src/quant.rs:1054-1063): the
 * Q/K/V projections of src/decoder.rs:148-158 share x, the cross K/V of
 * every layer at src/decoder.rs:44-53 are independent. */
int rw_rocm_matmul_grouped_dev(const rw_linear *items, size_t count, void *workspace,
                               size_t workspace_len, void *stream);

/* Workspace bytes rw_rocm_matmul_grouped_dev needs for these items. */
size_t rw_rocm_grouped_workspace_size(const rw_linear *items, size_t count);

/* A prepared group: the same launches as rw_rocm_matmul_grouped_dev over
 * the same items (so bitwise the same results), with the launch tables
 * uploaded once by rw_rocm_group_create, which also allocates the group's
 * buffer for quantized activations.  rw_rocm_group_run then only launches,
 * queued on `stream`: no copy, no allocation, no host wait; runs of one group
 * that overlap (two streams) race on that buffer.  For
 * decode loops whose activation and output buffers stay put from token to
 * token (src/decoder.rs:148-196 runs the same linears every step); the
 * pointers in `items` are captured at creation.  Has no reference
 * counterpart. */
typedef struct rw_group rw_group;
int rw_rocm_group_create(const rw_linear *items, size_t count, rw_group **out);
int rw_rocm_group_run(const rw_group *g, void *stream);
void rw_rocm_group_free(rw_group *g);

/* Dequantize rows [row0, row0+nrows) of W to f32 into host `out`
 * (nrows*k floats): x = d*q + m exactly as dequant_row_scalar
 * (src/quant.rs:528-537), bit for bit.  Replaces QTensor::row_f32
 * (src/quant.rs:566-570) and, over all rows, QTensor::to_dense
 * (src/quant.rs:572-576). */
int rw_rocm_dequant_rows(const rw_weight *w, size_t row0, size_t nrows, float *out);

/* Validation entry: quantize host activations a[m, k] on the device and
 * return q[m*k] (natural element order), d[m*k/32], sum[m*k/32] -- the QActs
 * of quantize_acts_i8 (src/quant.rs:679-716), bit for bit. */
int rw_rocm_quantize_acts(const float *a, size_t m, size_t k, int8_t *q, float *d, int32_t *sum);

/* Validation entry: the exact per-block integer sums
 * S[i, j, bl] = sum_e qa[i, bl*32+e] * q_b[j, bl*32+e] for host int8
 * activations qa[m, k] (natural order) against W, computed on the device's
 * int8 matrix cores (v_mfma_i32_32x32x32_i8) from the resident weight
 * planes.  S is host [m, n, k/32]. */
int rw_rocm_block_dots(const rw_weight *w, const int8_t *qa, size_t m, int32_t *S);

/* ---- Multi-head attention ----
 *
 * out[t_q, n_state] = concat over heads h of softmax(q_h k_h^T / sqrt(dh)
 * + mask) v_h, with q_h the h-th group of dh = n_state / n_head columns.
 * Replaces encoder::multi_head_attention / mha_split_kv
 * (src/encoder.rs:48-80, 109-119): with `causal`, query row i sits at
 * absolute position t_kv - t_q + i and sees kv rows up to it.  Computed in
 * f32-equivalent precision (f16 hi/lo pairs on the matrix cores, f32
 * softmax); within 1e-3 row-L2 of the reference (in practice a few f32
 * roundings).  Heads of 64 values only (every whisper model); |q|, |k|, |v|
 * below 65504.  RW_EINVAL for other head sizes, n_state % n_head != 0,
 * causal with t_q > t_kv, or rows not 16-byte aligned.
 *
 * _dev: device pointers (16-byte aligned), row strides ld* in floats
 * (>= n_state, multiples of 4), queued on `stream`; the workspace (NULL: one kept
 * per (device, stream)) holds rw_rocm_attention_workspace_size bytes.
 * rw_rocm_attention: host arrays, dense rows, synchronous. */
size_t rw_rocm_attention_workspace_size(size_t t_q, size_t t_kv, size_t n_state);
int rw_rocm_attention_dev(const float *q, size_t ldq, const float *k, size_t ldk, const float *v, size_t ldv,
                          size_t t_q, size_t t_kv, size_t n_state, int n_head, int causal, float *out, size_t ldo,
                          void *workspace, size_t workspace_len, void *stream);
int rw_rocm_attention(const float *q, const float *k, const float *v, size_t t_q, size_t t_kv, size_t n_state,
                      int n_head, int causal, float *out);

/* ---- One encoder layer on the device ----
 *
 * x[t, n_state] (device, row-major) <- x + attn(ln1(x)), then
 * x <- x + fc2(gelu(fc1(ln2(x)))): self_attention_block and mlp_block of
 * src/encoder.rs:121-175 for one non-causal layer, every activation
 * resident.  The layernorms are fused into the activation quantization of
 * the product that follows them, GELU and the residual adds into the
 * products' epilogues, and q, k and v come from one GEMM launch.  Weights
 * are resident (rw_rocm_weight_upload / rw_rocm_model_weight); q, k, v and
 * out are [n_state, n_state] of one dtype, fc1 [f, n_state], fc2 [n_state, f];
 * vectors are device f32 (16-byte aligned), biases may be NULL.
 * n_state = 64 n_head.  t must exceed 8 (the encoder has t = n_audio_ctx).
 * The workspace (NULL: one kept per (device, stream)) holds
 * rw_rocm_encoder_layer_workspace_size bytes; calls that share it must not
 * overlap.  Outputs within the products' and attention's tolerances of the
 * reference (1e-3 row-L2 per product).  With the environment variable
 * RW_ENCODER_MLP=fused, fc1's epilogue quantizes gelu(fc1) for fc2 (as
 * rw_rocm_matmul_prequant_gelu_quantize_dev does) instead of writing it in
 * f32: bitwise the same output, a few microseconds slower per large-v3
 * layer. */
typedef struct rw_encoder_layer {
  const float *attn_ln_w, *attn_ln_b;
  const rw_weight *q, *k, *v, *out;
  const float *q_b, *k_b, *v_b, *out_b; /* whisper's key has no bias: k_b NULL */
  const float *mlp_ln_w, *mlp_ln_b;
  const rw_weight *fc1, *fc2;
  const float *fc1_b, *fc2_b;
  int n_head;
} rw_encoder_layer;
size_t rw_rocm_encoder_layer_workspace_size(const rw_encoder_layer *layer, size_t t);
int rw_rocm_encoder_layer_dev(const rw_encoder_layer *layer, float *x, size_t t, void *workspace,
                              size_t workspace_len, void *stream);

/* ---- The decoder step on the device ----
 *
 * rw_decoder is the reference's Decoder (src/decoder.rs:26-213) with its
 * state resident: per-layer self-attention K/V caches of n_ctx rows, and
 * cross-attention K/V computed once per audio window (kept as the
 * attention kernel's f16 hi/lo planes).  forward_hidden runs tokens at
 * positions n_past .. n_past + n_tok through the embedding, every layer
 * (causal self-attention over cache + new rows, cross-attention, MLP) and
 * the final layernorm, extending the caches; the logits are then
 * rw_rocm_matmul_t_q_dev(token_embedding, hidden) as project_logits does.
 * Weights are resident rw_weight handles; vectors are device f32, 16-byte
 * aligned; biases may be NULL.  The token embedding must be quantized (as
 * in every quantized ggml model).  Replaces Decoder::new (:36-67),
 * fork (:70-79), reset (:86-95) and forward_hidden (:110-213).  A decoder
 * is used by one stream at a time. */
typedef struct rw_decoder_layer {
  const float *attn_ln_w, *attn_ln_b;
  const rw_weight *q, *k, *v, *out;
  const float *q_b, *v_b, *out_b;
  const float *cross_ln_w, *cross_ln_b;
  const rw_weight *cq, *ck, *cv, *cout;
  const float *cq_b, *cv_b, *cout_b;
  const float *mlp_ln_w, *mlp_ln_b;
  const rw_weight *fc1, *fc2;
  const float *fc1_b, *fc2_b;
} rw_decoder_layer;
typedef struct rw_decoder_params {
  int n_layer, n_head, n_ctx;       /* n_text_layer, n_text_head, n_text_ctx */
  const rw_decoder_layer *layers;   /* n_layer entries, copied at create */
  const rw_weight *token_embedding; /* [n_vocab, n_state] */
  const float *positional;          /* [n_ctx, n_state] */
  const float *ln_w, *ln_b;         /* decoder.ln */
} rw_decoder_params;
typedef struct rw_decoder rw_decoder;
int rw_rocm_decoder_create(const rw_decoder_params *params, size_t n_audio_ctx, rw_decoder **out);
void rw_rocm_decoder_free(rw_decoder *d);
/* cross K/V of every layer from the encoder output [n_audio_ctx, n_state]
 * (device), and n_past = 0 */
int rw_rocm_decoder_set_audio_dev(rw_decoder *d, const float *enc_out, void *stream);
int rw_rocm_decoder_reset(rw_decoder *d);
int rw_rocm_decoder_n_past(const rw_decoder *d, size_t *n_past);
/* an independent branch: copies the self-attention caches (on `stream`),
 * shares the cross K/V */
int rw_rocm_decoder_fork(const rw_decoder *d, void *stream, rw_decoder **out);
/* tokens: host array of n_tok ids; hidden: device [n_tok, n_state] */
int rw_rocm_decoder_forward_hidden_dev(rw_decoder *d, const uint32_t *tokens, size_t n_tok, float *hidden,
                                       void *stream);

/* One step of a beam search for up to RW_MAX_BEAMS beams at once: beam i
 * forwards its one new token tokens[i] (host array) and hidden row i (device
 * [n_beams, n_state]) receives its final hidden state, as n_beams separate
 * rw_rocm_decoder_forward_hidden_dev calls of one token would (within f32
 * rounding: the products see n_beams rows, and the attention's kv split is
 * chosen for all beams together).  Replaces the per-beam forward_hidden calls
 * of the beam search (src/transcribe.rs:931-949); the beams' logits are then
 * one rw_rocm_matmul_t_q_dev of the token embedding on the n_beams hidden
 * rows, as the reference's stacked project_logits (src/transcribe.rs:965-978).
 * The beams are distinct decoders forked from one decoder (they share its
 * cross K/V) with equal n_past; every linear runs once over the n_beams rows,
 * and the beams' self-attentions run as one launch, each over its own cache.
 * Each beam's n_past grows by one.  The step uses beam 0's scratch, so steps
 * that involve one decoder must not overlap. */
#define RW_MAX_BEAMS 8
int rw_rocm_decoder_forward_beams_dev(rw_decoder *const *beams, size_t n_beams, const uint32_t *tokens,
                                      float *hidden, void *stream);

/* log_softmax (src/transcribe.rs:482-486) and top_k (src/transcribe.rs:672-
 * 685) of every row of logits [rows, n_vocab] (device): ids[rows * k] and
 * logprobs[rows * k] (device) get the list the reference's insertion scan
 * keeps: exactly -inf is skipped; an entry is inserted ahead of equal
 * log-probs while the list has room or it beats the last entry, and the
 * list is cut to k, so of the entries tied at the k-th log-prob those
 * admitted while there was room stay, oldest pushed out first; the list runs
 * by log-prob, equal ones later id first.  A row holding NaN or +inf, or
 * only -inf, has NaN log-probs throughout (as in the reference), and its
 * list is ids min(k, n_vocab) - 1 .. 0 with NaN.  A row with fewer than k
 * candidates ends with id 0xFFFFFFFF and -inf.  1 <= k <=
 * 16, n_vocab <= 131072, rows <= 65535.  The log-sum-exp is summed in tree
 * order, so a log-prob can differ from the reference's in its last bit.
 * `workspace` (>= rw_rocm_logits_topk_workspace_size bytes; NULL = a buffer
 * of the library's own for this stream) holds per-chunk partial results.  On
 * the current device, asynchronous on `stream`. */
int rw_rocm_logits_topk_dev(const float *logits, size_t rows, size_t n_vocab, size_t k, uint32_t *ids,
                            float *logprobs, void *workspace, size_t workspace_len, void *stream);
size_t rw_rocm_logits_topk_workspace_size(size_t rows, size_t n_vocab, size_t k);

/* ---- Model files straight to resident weights ----
 *
 * rw_rocm_model_load reads a whisper model in either container the reference
 * loads -- the legacy ggml ".bin" (src/model.rs:145-275) or GGUF with the
 * reference's metadata mapping (src/gguf.rs:156-300) -- chosen by the magic,
 * from a read-only memory map.  Every 2-D block-quantized matrix goes to the
 * current device through rw_rocm_weight_upload straight from the mapped bytes
 * (the reference's Weight::Quant); every other tensor becomes host f32 as the
 * reference's Weight::Dense (f16 by the exact conversion of
 * src/model.rs:68-86, quantized tensors of other ranks by d*q + m).  Shapes
 * are row-major (the file's innermost-first dims flipped).  A malformed file
 * fails with RW_EINVAL and the reference's message; an unreadable one with
 * RW_EIO.  RW_MODEL_PARSE_ONLY skips the uploads (no device needed): the
 * quantized matrices are then reachable only as their blocks
 * (rw_rocm_model_raw).  Replaces model::load_model and gguf::load.  Pointers
 * returned by the accessors live until rw_rocm_model_free, which also frees
 * the uploaded weights. */
typedef struct rw_model rw_model;
#define RW_MODEL_PARSE_ONLY 1
int rw_rocm_model_load(const char *path, int flags, rw_model **out);
void rw_rocm_model_free(rw_model *m);

/* The 11 hyperparameters in the order of HParams (src/model.rs:24-37):
 * n_vocab, n_audio_ctx, n_audio_state, n_audio_head, n_audio_layer,
 * n_text_ctx, n_text_state, n_text_head, n_text_layer, n_mels, ftype. */
int rw_rocm_model_hparams(const rw_model *m, int32_t *hp);

/* The embedded mel filterbank, n_mel x n_fft row-major f32 (Model::mel_filters). */
int rw_rocm_model_mel_filters(const rw_model *m, const float **data, size_t *n_mel, size_t *n_fft);

/* Vocabulary (Model::vocab): n_vocab tokens as raw bytes, the ids past the
 * file's own tokens named "[_extra_token_<id>]" as the reference names them. */
int rw_rocm_model_vocab_size(const rw_model *m, size_t *n);
int rw_rocm_model_token(const rw_model *m, size_t id, const uint8_t **bytes, size_t *len);

/* Tensors (Model::tensors): count, name by index (file order; a repeated name
 * keeps the last tensor, as the reference's map does), and by name the ggml
 * dtype, rank and row-major shape (unused dims 1).  rw_rocm_model_tensor
 * returns 1 for a quantized matrix (Weight::Quant), 0 for a dense tensor. */
int rw_rocm_model_tensor_count(const rw_model *m, size_t *n);
int rw_rocm_model_tensor_name(const rw_model *m, size_t i, const char **name);
int rw_rocm_model_tensor(const rw_model *m, const char *name, int *dtype, int *ndims, size_t *shape);

/* A quantized matrix's resident device weight (RW_EINVAL for a dense tensor
 * or a parse-only load). */
int rw_rocm_model_weight(const rw_model *m, const char *name, const rw_weight **w);

/* A dense tensor's host f32 data (RW_EINVAL for a quantized matrix). */
int rw_rocm_model_dense(const rw_model *m, const char *name, const float **data, size_t *len);

/* A tensor's bytes as stored in the file (ggml blocks for quantized ones). */
int rw_rocm_model_raw(const rw_model *m, const char *name, const uint8_t **raw, size_t *len);

/* Copy the calling thread's last error text (NUL-terminated, truncated to
 * len).  Returns the full text length. */
int rw_rocm_last_error(char *buf, size_t len);

#ifdef __cplusplus
}
#endif
#endif
