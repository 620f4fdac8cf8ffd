/* trit_hip: Trit's decoder token loop on MI355X (gfx950), behind a C ABI.
 *
 * This library replaces, for one GPU, the products and the token loop that
 * Trit runs on its CPU kernels. Each entry point names the reference
 * interface it stands in for (paths into Hi9841/trit).
 *
 * Rules for every function (as in the reference's include/trit.h:8-17 and
 * ffi/src/lib.rs:1-46):
 * - A call that fails returns -1 (or NULL) and sets the calling thread's
 *   error text, which trit_hip_last_error() returns. No C++ exception
 *   crosses the ABI.
 * - Pointers named host_* or taking plain `const float*` inputs in the
 *   layer and session calls are host memory; *_device calls take device
 *   pointers and a hipStream_t (NULL: the library's stream).
 * - Layer and decoder handles are immutable after creation and may be
 *   shared across threads. A session belongs to one thread at a time.
 * - Weights are copied into device memory at creation; the handle owns
 *   them. A decoder keeps its layers alive: the caller may free its layer
 *   handles right after trit_hip_decoder_new.
 */
#ifndef TRIT_HIP_H
#define TRIT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct TritHipLayer TritHipLayer;
typedef struct TritHipDecoder TritHipDecoder;
typedef struct TritHipSession TritHipSession;

/* Library version text. Static. */
const char *trit_hip_version(void);

/* Error of the last failed call on this thread, "" after a success.
 * Mirrors trit_last_error (reference include/trit.h:44-46,
 * ffi/src/lib.rs:20-46). */
const char *trit_hip_last_error(void);

/* Selects and initialises `device` for this thread and creates the
 * library's stream on it. Stands in for gpu::Gpu::get
 * (reference src/gpu/mod.rs:36-128). 0 on success. */
int trit_hip_init(int device);

/* ---- Layers: the Dense seam (reference src/cpu/gemm.rs:15-35,500-542) --- */

enum {
    TRIT_HIP_Q8_0 = 1,    /* ggml Q8_0: 32 int8 codes + f16 scale per block   */
    TRIT_HIP_INT8 = 2,    /* Trit int8: one f32 scale per row and 128 inputs  */
    TRIT_HIP_TERNARY = 3, /* codes 0..2, w = scale * (code - 1), 128 groups   */
    TRIT_HIP_Q4_K = 4,    /* ggml Q4_K super-blocks, run as Trit's Q8_0 codes */
    TRIT_HIP_F16 = 5,     /* f16 weights, f32 math (token tables, the head)   */
    TRIT_HIP_F32 = 6,     /* f32 weights, f32 math                            */
    TRIT_HIP_Q8 = 7       /* int8 storage, f32 scale per 32, f32 math         */
};

/* ggml Q8_0 weights as stored in GGUF: n*k/32 blocks of 34 bytes (f16 d,
 * little endian, then 32 int8 codes), row-major n x k. bias: n floats or
 * NULL. Replaces Dense::q8_0 + Int8::from_q8_0
 * (reference src/cpu/gemm.rs:225-247, src/cpu/int8.rs:234-236,256-289,
 * src/cpu/tensors.rs:282-305): int8 activations when n % 32 == 0, else
 * (a shape Trit's int8 kernels refuse) the codes with f32 math, as
 * trit_hip_layer_q8_0_f32. k % 32 == 0. */
int trit_hip_layer_q8_0(int n, int k, const void *blocks, const float *bias, TritHipLayer **out);

/* Trit int8 weights: codes row-major n x k, scales n x (k/128).
 * Replaces Int8::quantize's layer (reference src/cpu/int8.rs:292-369). */
int trit_hip_layer_int8(int n, int k, const int8_t *codes, const float *scales, const float *bias,
                        TritHipLayer **out);

/* Ternary weights: codes 0..2 row-major n x k, scales n x (k/128).
 * Replaces Ternary::from_rows (reference src/cpu/kernels.rs:136-202). */
int trit_hip_layer_ternary(int n, int k, const uint8_t *codes, const float *scales, TritHipLayer **out);

/* Ternary weights as the model file stores them: ceil(k/5) base-3 bytes per
 * row, five digits each, least significant first. Replaces
 * Ternary::from_base3 (reference src/cpu/kernels.rs:91-130). */
int trit_hip_layer_ternary_base3(int n, int k, const uint8_t *packed, const float *scales,
                                 TritHipLayer **out);

/* ggml Q4_K weights as stored in GGUF: n*k/256 super-blocks of 144 bytes.
 * Results are Trit's: the device expands the super-blocks and requantizes
 * each 32 values to Q8_0 codes at creation, as expand-then-Blocks::quantize
 * does (reference src/cpu/ggml_quants.rs:168-196, src/cpu/gemm.rs:58-76,
 * src/cpu/tensors.rs:263-286); products then run on those codes.
 * k % 256 == 0. */
int trit_hip_layer_q4_k(int n, int k, const void *blocks, TritHipLayer **out);

/* A GGUF tensor of ggml type `ggml_type` as Trit loads it under Auto
 * precision (Tensors::precision_of / q8_0, reference src/cpu/tensors.rs:
 * 262-305; Dense::load / Dense::table, src/cpu/gemm.rs:225-247,287-409):
 * Q8_0 (8) as stored; Q4_0 (2), Q4_1 (3), Q5_0 (6), Q5_1 (7), Q4_K (12),
 * Q5_K (13) and Q6_K (14) expanded as ggml's dequantize_row_* and
 * requantized to Q8_0 codes (src/cpu/ggml_quants.rs:103-245, gemm.rs:58-76),
 * on the device. Then int8 activations, unless f32_math (a token table) or
 * n % 32 != 0 ask for the codes with f32 math. k a multiple of the type's
 * block (32, or 256 for the K types). bias: n floats or NULL. */
int trit_hip_layer_ggml(int n, int k, int ggml_type, const void *blocks, const float *bias, int f32_math,
                        TritHipLayer **out);

/* f32 weights, row-major n x k, f32 math in Trit's 16-lane order.
 * Replaces Dense::new / Weights::F32 and Dense::table under F32
 * (reference src/cpu/gemm.rs:190-204,395). Any k: the 16-lane tail padded with zeros. */
int trit_hip_layer_f32(int n, int k, const float *weights, const float *bias, TritHipLayer **out);

/* Int8 storage with f32 math (Weights::Q8, reference src/cpu/gemm.rs:37-44,
 * 117-187): codes row-major n x k, scales n x (k/32) f32; the product
 * widens each weight to f32(code) * scale (one rounding) and runs the f32
 * product. Replaces Q8::quantize's layer and Dense::table under Int8 or
 * Auto (:396-399). k % 32 == 0. */
int trit_hip_layer_q8(int n, int k, const int8_t *codes, const float *scales, const float *bias,
                      TritHipLayer **out);

/* ggml Q8_0 blocks (as trit_hip_layer_q8_0) held with f32 math: Dense::table
 * under Q8_0 (reference src/cpu/gemm.rs:386-393) -- a token table or an
 * untied head never takes int8 activations. k % 32 == 0. */
int trit_hip_layer_q8_0_f32(int n, int k, const void *blocks, const float *bias, TritHipLayer **out);

/* f16 weights (bits), row-major n x k. Replaces Dense::half / Dense::table
 * with F16 weights (reference src/cpu/gemm.rs:206-221,383-409). Any k: the 16-lane tail padded with zeros. */
int trit_hip_layer_f16(int n, int k, const uint16_t *weights, const float *bias, TritHipLayer **out);

/* y = x * W^T (+ bias, then max(y, 0) when relu): x is m x k f32, y m x n
 * f32, host memory. Replaces Dense::forward / forward_relu
 * (reference src/cpu/gemm.rs:500-542). Up to 8 rows run on the small-batch
 * GEMV kernels; more rows of a Q8_0, Q4_K or int8 layer with n % 128 == 0
 * run on the matrix cores (int8 MFMA), with the same bits. */
int trit_hip_layer_forward(const TritHipLayer *layer, const float *x, int m, int relu, float *y);

/* The same on device pointers, enqueued on `stream` (a hipStream_t; NULL:
 * the library's stream), without a wait. Products of 2 or more rows use a
 * scratch buffer of the calling thread: calls from one thread must not
 * overlap on different streams. */
int trit_hip_layer_forward_device(const TritHipLayer *layer, const float *x, int m, int relu, float *y,
                                  void *stream);

/* trit_hip_layer_forward_device that allocates nothing. It has no
 * counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid it). The activations of 2 or more rows are
 * quantized into one 4 MiB array per device that is part of the library
 * (its address found by trit_hip_init on that device, else by the first
 * call there), not into a per-thread buffer the library grows. A product
 * whose quantized rows need more than that fails with an error naming the
 * bytes it needs. All calls on one device share the array and it keeps the
 * last call's contents: calls on one device must not overlap (queue them
 * on one stream). Results are trit_hip_layer_forward_device's, bit for
 * bit. Call trit_hip_init on the calling thread first (it creates the
 * library's stream), or pass a stream. */
int trit_hip_layer_forward_device_noalloc(const TritHipLayer *layer, const float *x, int m, int relu, float *y,
                                          void *stream);

/* The measurement hook (the counterpart of Trit's kernel bench timing,
 * src/cpu/v2/bench.rs:42-54): trit_hip_layer_forward_device with the
 * product kernel's launch stamped with start_event and stop_event
 * (hipEvent_t, either may be NULL) at the kernel's start and end. One row
 * (and f16 layers) is one launch; 2..8 rows of an integer layer quantize
 * their activations in a pass of their own first, and start_event then
 * stamps that pass's start, so the interval covers the whole call. A
 * matrix-core product stamps its GEMM kernel (the activation quantization
 * runs before it, unstamped). Fails for more than 8 rows of a layer the
 * matrix cores do not take. */
int trit_hip_layer_forward_timed(const TritHipLayer *layer, const float *x, int m, int relu, float *y,
                                 void *stream, void *start_event, void *stop_event);

/* Shape and kind of a layer; device_bytes: the bytes its weights hold. */
int trit_hip_layer_info(const TritHipLayer *layer, int *n, int *k, int *kind, int64_t *device_bytes);

/* Row `index` of a token table as f32 (Dense::row, reference
 * src/cpu/gemm.rs:412-429). F16 layers only. */
int trit_hip_layer_row(const TritHipLayer *layer, int index, float *out);

void trit_hip_layer_free(TritHipLayer *layer);

/* ---- f16 conversions (reference src/cpu/tensors.rs:542-595) ------------ */

/* f32_to_f16 / f16_to_f32 of n values (host arrays) by the device's
 * conversion -- the one the kernels use for Q8_0 scales, f16 weights and
 * the f16 key/value caches: round to nearest even with subnormals and
 * infinities, bit for bit Trit's for every value but NaN (a NaN stays a
 * NaN; its payload bits are the hardware's). */
int trit_hip_f32_to_f16(const float *in, int64_t n, uint16_t *out);
int trit_hip_f16_to_f32(const uint16_t *in, int64_t n, float *out);

/* ---- Decoder: CausalLm (reference src/models/parts/causal_lm.rs) ------- */

typedef struct {
    int d, ffn, layers, heads, kv_heads, head_dim, vocab;
    float eps;        /* rms_norm_eps, 1e-6 when the config has none       */
    float rope_base;  /* rope_theta, 1e6 when the config has none          */
    int qk_norm;      /* Qwen3's per-head q and k norms                     */
    /* Granite's multipliers (Config, reference causal_lm.rs:17-27,62-65):
     * on the input embeddings, on q in place of 1/sqrt(head_dim) (0: none),
     * on each residual branch, and (as a divisor) on the logits. 0 in
     * embedding_multiplier, residual_multiplier or logits_scaling means 1,
     * so a zeroed tail describes a Qwen3 / Llama decoder. */
    float embedding_multiplier, attention_multiplier, residual_multiplier, logits_scaling;
} TritHipLmConfig;

/* A decoder from its layers (CausalLm::from_tensors, reference
 * causal_lm.rs:141-198). linears: 4 per layer, in order qkv (q, k, v rows
 * stacked), o, gate_up (gate rows then up rows), down. norms (host f32):
 * per layer norm_attn[d], norm_mlp[d], q_norm[hd], k_norm[hd] (the last two
 * only with qk_norm), then the final norm[d]. embed: an F16 vocab x d
 * table; head: the output projection, or NULL when tied to embed. */
int trit_hip_decoder_new(const TritHipLmConfig *config, const TritHipLayer *const *linears,
                         const float *norms, const TritHipLayer *embed, const TritHipLayer *head,
                         TritHipDecoder **out);
void trit_hip_decoder_free(TritHipDecoder *decoder);

/* The device weight-cache file (the role of Trit's Store cache file,
 * reference src/cpu/store.rs:1-16,369-428,508-524): _save writes a
 * decoder's device layouts (repacked and requantized as they sit in HBM)
 * to `path`, keyed by this library's version and target; _load uploads
 * them into a new decoder without converting anything, and fails on a file
 * of another key or format, or one whose checksum does not hold (a stale
 * or damaged cache never changes a product). config (optional) receives
 * the decoder's config. MLP scales are not part of the file. */
int trit_hip_decoder_save(const TritHipDecoder *decoder, const char *path);
int trit_hip_decoder_load(const char *path, TritHipLmConfig *config, TritHipDecoder **out);

/* CausalLm::set_ffn_scales (reference causal_lm.rs:304-307,458-464):
 * layers x d f32 scales on each layer's normed MLP input (Voxtral
 * Realtime's 1 + ada(t)); NULL removes them. Sessions see the change from
 * their next call; not while a session of the decoder runs a call. */
int trit_hip_decoder_set_ffn_scales(TritHipDecoder *decoder, const float *scales);

/* Session flags. Every sum runs in Trit's order unless TRIT_HIP_TREE_SUMS
 * is given: the default (0) is Trit's arithmetic with f16 keys and values
 * (each appended key and value rounded through f16), bit for bit. */
enum {
    TRIT_HIP_EXACT = 1,     /* Trit's arithmetic throughout: f32 keys and values */
    TRIT_HIP_KV_F32 = 2,    /* f32 keys and values                              */
    TRIT_HIP_TREE_SUMS = 4  /* RMSNorm, q/k norm and attention sums as parallel
                               trees (faster; the int8 activation codes then
                               differ from Trit's where a value lies within
                               rounding of a code boundary)                     */
};

/* Per-call state: the key/value caches of up to max_positions positions
 * (the Vec caches of CausalLm::generate, reference causal_lm.rs:224-240). */
int trit_hip_session_new(const TritHipDecoder *decoder, int max_positions, int flags, TritHipSession **out);

/* Runs `n` tokens at the next positions and extends the caches; logits
 * (vocab floats, host) after the last token, or NULL. CausalLm::forward
 * (reference causal_lm.rs:363-371). */
int trit_hip_session_prefill(TritHipSession *session, const int32_t *tokens, int n, float *logits);

/* As trit_hip_session_prefill from embeddings, n x d host floats
 * (CausalLm::forward_rows, reference causal_lm.rs:374-389; the rows of
 * generate_rows and answer, :254-282). */
int trit_hip_session_prefill_rows(TritHipSession *session, const float *rows, int n, float *logits);

/* Greedy tokens from the last logits (CausalLm::greedy, reference
 * causal_lm.rs:284-302): argmax (the first of equal values), stop check,
 * forward of the kept token, until a stop token or max_new tokens. The loop
 * stays on the device. Returns the token count written to out. */
int trit_hip_session_generate(TritHipSession *session, int max_new, const int32_t *stop, int n_stop,
                              int32_t *out);

/* The measurement hook for the token loop: trit_hip_session_generate with
 * start_event / stop_event (hipEvent_t, either may be NULL) recorded on the
 * library's stream right before the first step launch and right after the
 * last, so their interval is the device time of the steps. *persistent (may
 * be NULL) tells whether the steps ran as the persistent decode step (one
 * kernel launch for all the call's tokens: nonzero, bit 0 set) or as the
 * per-kernel loop (0); on the step, bit 1 is set when the attention runs
 * on every block, the q/k/v rows and scores of each key/value head passing
 * through the L2 of the XCD that attends to it. The counterpart of
 * Trit's decode timing (src/cpu/v2/bench.rs:42-54). */
int trit_hip_session_generate_timed(TritHipSession *session, int max_new, const int32_t *stop, int n_stop,
                                    int32_t *out, void *start_event, void *stop_event, int *persistent);

/* Measurement only; no counterpart in the reference. A library built with
 * `python -m trit_amd.build --stamps` (libtrit_hip_stamps.so) stamps the
 * persistent step's phases for one (step, layer) of each launch (layer ==
 * layers: the final norm and the head): thread 0 of every block writes the
 * device wall clock (100 MHz) and its shader clock at fixed points.
 * _stamps chooses the (step, layer) (-1: none) for later launches; _read
 * copies the stamps of the first `blocks` blocks (NSTAMP = 32 a block, the
 * return value). The product library returns -1 from both. */
int trit_hip_step_stamps(int step, int layer);
int trit_hip_step_stamps_read(uint64_t *wall, uint64_t *clock, int blocks);

/* Clears the caches (a new call). */
int trit_hip_session_reset(TritHipSession *session);

/* CausalLm::generate_additive (reference causal_lm.rs:313-345): greedy
 * tokens with audio rows added to every input -- the prompt's embeddings
 * plus audio rows 0..n, then each new token's embedding plus the row of
 * its position -- until a stop token or the rows end. audio: rows x d
 * host f32. Starts from a fresh (or reset) session, whose positions must
 * hold `rows`; out holds rows - n + 1 tokens. Returns the count (0 when
 * n is 0 or rows < n, as Trit does), or -1. */
int trit_hip_session_generate_additive(TritHipSession *session, const int32_t *prompt, int n, const float *audio,
                                       int rows, const int32_t *stop, int n_stop, int32_t *out);

/* A prompt start that many calls share (CausalLm::prefix and Prefix,
 * reference causal_lm.rs:118-122,200-215): its keys and values, computed
 * once in a session of the given flags. */
typedef struct TritHipPrefix TritHipPrefix;
int trit_hip_prefix_new(const TritHipDecoder *decoder, const int32_t *tokens, int n, int flags, TritHipPrefix **out);
void trit_hip_prefix_free(TritHipPrefix *prefix);
/* The prompt `tokens` of a fresh (or reset) session that may begin with
 * `prefix` (CausalLm::generate with Some(prefix), causal_lm.rs:217-249):
 * when it is longer than the prefix and starts with its tokens, the
 * session takes the prefix's keys and values and runs only the rest;
 * otherwise the whole prompt. The prefix must come from the session's
 * decoder and flags. Logits as trit_hip_session_prefill. */
int trit_hip_session_prefill_prefixed(TritHipSession *session, const TritHipPrefix *prefix, const int32_t *tokens,
                                      int n, float *logits);

/* Position count the caches hold. */
int trit_hip_session_position(const TritHipSession *session);

void trit_hip_session_free(TritHipSession *session);

/* ---- Audio encoder (reference src/models/parts/audio_encoder.rs) ------- */

/* Whisper's audio encoder, which Voxtral and MOSS run (Encoder,
 * reference src/models/parts/audio_encoder.rs:18-139). */
typedef struct {
    int d, layers, heads, ffn, mels, positions; /* EncoderShape (:40-60) */
} TritHipEncoderConfig;
typedef struct TritHipEncoder TritHipEncoder;
/* Encoder::load (:62-108) from device layers with their biases: conv1
 * (d x 3*mels) and conv2 (d x 3*d), their weights [out][in][kernel] as
 * rows; per layer qkv (3d x d, q/k/v stacked, k's bias zero), out (d x d),
 * fc1 (ffn x d), fc2 (d x ffn), 4 a layer in that order; positions
 * (positions x d); norms per layer attn weight, attn bias, ffn weight, ffn
 * bias (d each), then the final weight and bias. Layer kinds as the
 * decoder takes them (int8 activations, or f32 math). */
int trit_hip_encoder_new(const TritHipEncoderConfig *config, const TritHipLayer *conv1, const TritHipLayer *conv2,
                         const float *positions, const TritHipLayer *const *linears, const float *norms,
                         TritHipEncoder **out);
void trit_hip_encoder_free(TritHipEncoder *encoder);
/* Encoder::encode (:111-138): the positions x d output of one window of
 * 2 * positions x mels features (host memory), with Trit's arithmetic:
 * im2col, the products in their kinds' orders (biases after the chains),
 * the exact GELU, layer norm in 32-lane order, Trit's attention over every
 * position. */
int trit_hip_encoder_encode(const TritHipEncoder *encoder, const float *mel, float *out);

/* The Qwen3-ASR audio encoder (AudioEncoder, reference
 * src/models/families/qwen3_asr.rs:284-405); sizes as AudioConfig
 * (:71-118): chunk = 2 * n_window mel frames, window_chunks =
 * n_window_infer / chunk, out = output_dim. */
typedef struct {
    int d, layers, heads, ffn, mels, channels, chunk, window_chunks, out, max_positions;
} TritHipAsrEncoderConfig;
typedef struct TritHipAsrEncoder TritHipAsrEncoder;
/* AudioEncoder::load (:284-317) from device layers with their biases:
 * convs = conv2d1 (channels x 9), conv2d2 and conv2d3 (channels x 9 *
 * channels), weights [out][in][bin tap][time tap] as rows; conv_out (d x
 * channels * ceil^3(mels / 2)); per layer qkv (3d x d, q/k/v stacked),
 * out (d x d), fc1 (ffn x d), fc2 (d x ffn), 4 a layer; norms per layer
 * attn weight, attn bias, ffn weight, ffn bias (d each), then ln_post's
 * weight and bias; proj1 (d x d), proj2 (out x d). The sinusoid positions
 * (max_positions x d, src/layers.rs:257-270) are made here. Any layer kind
 * (the first convolution's 9 inputs take f16 or f32). */
int trit_hip_asr_encoder_new(const TritHipAsrEncoderConfig *config, const TritHipLayer *const *convs,
                             const TritHipLayer *conv_out, const TritHipLayer *const *linears, const float *norms,
                             const TritHipLayer *proj1, const TritHipLayer *proj2, TritHipAsrEncoder **out);
void trit_hip_asr_encoder_free(TritHipAsrEncoder *encoder);
/* Rows encode makes of `frames` mel frames (ceil^3(length / 2) of each
 * chunk), or -1. */
int trit_hip_asr_encoder_rows(const TritHipAsrEncoder *encoder, int frames);
/* The sinusoid table the encoder holds (max_positions x d floats). */
int trit_hip_asr_encoder_positions(const TritHipAsrEncoder *encoder, float *out);
/* AudioEncoder::encode (:321-373): frames x mels log-mel features (host
 * memory) to rows x out (host memory, rows as trit_hip_asr_encoder_rows);
 * returns rows or -1. Chunks zero padded to the longest, the three
 * convolutions with the exact GELU, the channel-major time columns,
 * conv_out, the positions, layers whose attention sees only the rows of
 * its window, ln_post, proj1, GELU, proj2 -- Trit's arithmetic throughout. */
int trit_hip_asr_encoder_encode(const TritHipAsrEncoder *encoder, const float *mel, int frames, float *out);

/* ---- Attention (reference src/layers.rs:343-504) ---------------------- */

/* Grouped-query attention of tq query rows over tk keys, host memory:
 * layers::attention (src/layers.rs:343-504,571-587). q rows have stride qs
 * floats (heads * hd values each), k and v rows stride kvs (kv_heads * hd);
 * query head h reads key head h / (heads / kv_heads); out is tq rows of
 * heads * hd floats. causal: row i sees keys 0 .. tk - tq + i; else every
 * key. flags TRIT_HIP_EXACT: Trit's order and sums with f32 keys and
 * values, bit for bit (head_dim up to 256, tk up to 16000); 0: the fast
 * form of the prompt path, keys and values rounded to f16 as the f16 caches
 * hold them and the products on the matrix cores (head_dim 128; 1, 2 or 4
 * query heads per key head). */
int trit_hip_attention(const float *q, int qs, const float *k, const float *v, int kvs, int tq, int tk, int heads,
                       int kv_heads, int hd, int causal, int flags, float *out);

/* The self-attention of one decoder step for several sequences (beams):
 * layers::attention_steps (src/layers.rs:505-562). Sequence b asks its one
 * query (row b of q, stride qs floats, heads * hd values, hd = d / heads)
 * over its own tk[b] keys and values (keys[b], values[b]: tk[b] rows of
 * kv_heads * hd f32 each, the rows of Trit's per-sequence caches); out is
 * sequences x d. Trit's orders and sums, bit for bit (the values of
 * trit_hip_attention with EXACT on each sequence alone). 1 to 32
 * sequences; head_dim a multiple of 8 up to 256; up to 16000 keys. Host
 * memory. */
int trit_hip_attention_steps(const float *q, int qs, const float *const *keys, const float *const *values,
                             const int *tk, int sequences, int d, int heads, int kv_heads, float *out);
/* The same on device memory (q, out and each keys[b] / values[b], 16-byte
 * aligned; the pointer arrays and tk in host memory), queued on `stream`
 * (a hipStream_t; NULL: the calling thread's stream) without waiting.
 * Allocates nothing. */
int trit_hip_attention_steps_device(const float *q, int qs, const float *const *keys, const float *const *values,
                                    const int *tk, int sequences, int d, int heads, int kv_heads, float *out,
                                    void *stream);

/* ---- Tokenizer (reference src/text/bpe.rs, src/text/mod.rs) ----------- */

/* Byte-level BPE from a Hugging Face tokenizer.json (Bpe::open / Bpe::parse,
 * reference src/text/bpe.rs:76-174): the vocabulary, the merges in rank
 * order, the added (special) tokens, and Trit's Qwen or GPT-2 word split
 * (chosen as Trit chooses it, by the Qwen regex in pre_tokenizer). Host
 * code. */
typedef struct TritHipBpe TritHipBpe;
int trit_hip_bpe_open(const char *path, TritHipBpe **out);
int trit_hip_bpe_parse(const char *json, size_t len, TritHipBpe **out);
void trit_hip_bpe_free(TritHipBpe *bpe);
/* Bpe::id (:176-183): the id of a token as the vocabulary writes it, or -1. */
int trit_hip_bpe_id(const TritHipBpe *bpe, const char *token);
/* Bpe::encode (:197-227; plain != 0: encode_plain, :229-237): the ids of
 * `len` bytes of UTF-8 text, special tokens written in it becoming their
 * ids unless plain. Writes up to cap ids and returns the count (which may
 * exceed cap: call again with room), or -1. */
int trit_hip_bpe_encode(const TritHipBpe *bpe, const char *text, size_t len, int plain, int32_t *out, int cap);
/* Bpe::decode (:185-195): the text of ids without special tokens, a last
 * character cut short dropped and other invalid bytes as U+FFFD. Writes up
 * to cap - 1 bytes and a NUL; returns the text's length, or -1. */
int64_t trit_hip_bpe_decode(const TritHipBpe *bpe, const int32_t *ids, int n, char *out, size_t cap);

/* The prompt of Trit's transcript cleanup with S1-mini (Cleaner,
 * reference src/cleanup.rs:19-21,156-158,199-215,280-301). _system: the
 * ids of the fixed system turn that every call shares (the Prefix the
 * cleaner makes once). _prompt: the ids of one call -- the system turn and
 * the control line ("[Styling: ...] [Structure: ...] [Context: ...]";
 * styling 0 casual, 1 semi-casual, 2 semi-formal, 3 formal; structure 0
 * prose, 1 lists; context 0 general, 1 email), the transcript as plain text
 * (a spoken "<|im_end|>" cannot end the turn), then the assistant turn with
 * thinking off. Counts and capacity as trit_hip_bpe_encode. */
int trit_hip_cleanup_system(const TritHipBpe *bpe, int32_t *out, int cap);
int trit_hip_cleanup_prompt(const TritHipBpe *bpe, const char *transcript, size_t len, int styling, int structure,
                            int context, int32_t *out, int cap);
/* Cleaner::parts (reference src/cleanup.rs:240-278) of the trimmed
 * transcript: whole sentences, or words of a sentence longer alone, joined
 * with one space into parts of at most `limit` tokens (Trit's PART_TOKENS
 * is 800). Writes up to cap bytes of the parts, each followed by a NUL, and
 * returns their total bytes, or -1. */
int64_t trit_hip_cleanup_parts(const TritHipBpe *bpe, const char *transcript, size_t len, int limit, char *out,
                               size_t cap);

/* ---- GGUF files (reference src/models/gguf/mod.rs:130-300) ------------- */

typedef struct TritHipGguf TritHipGguf;

/* Opens and checks a GGUF v2/v3 file: the magic, the version, the metadata
 * (strings and arrays of at most 2^24 entries, arrays nested at most 4
 * deep), a tensor count the file can hold, general.alignment (32 when
 * absent, never 0), and every tensor's byte range for its ggml type (F32,
 * F16, BF16, Q8_0, Q4_0, Q4_1, Q5_0, Q5_1, Q4_K, Q5_K, Q6_K). Replaces
 * Gguf::open (gguf/mod.rs:155-226) with ggml_quants::layout
 * (src/cpu/ggml_quants.rs:51-75); the error texts are the reference's,
 * prefixed by the path. Host only: needs no device. */
int trit_hip_gguf_open(const char *path, TritHipGguf **out);
void trit_hip_gguf_free(TritHipGguf *gguf);
int trit_hip_gguf_tensor_count(const TritHipGguf *gguf);

/* Tensor `index` in file order: its name, ggml type name, dims (ne0 first,
 * up to 4 written), and byte range [start, end) of the file. Any output
 * may be NULL; the strings live as long as the handle. */
int trit_hip_gguf_tensor(const TritHipGguf *gguf, int index, const char **name, const char **dtype, int *n_dims,
                         int64_t *dims, int64_t *start, int64_t *end);

/* Metadata of `key`: an integer (unsigned, or signed and not negative), a
 * number, or a string (living as long as the handle). -1 when the key is
 * absent or of another kind (Gguf::get / num, gguf/mod.rs:242-249). */
int trit_hip_gguf_meta_u64(const TritHipGguf *gguf, const char *key, uint64_t *out);
int trit_hip_gguf_meta_f64(const TritHipGguf *gguf, const char *key, double *out);
int trit_hip_gguf_meta_str(const TritHipGguf *gguf, const char *key, const char **out);

/* A decoder from the language model of a GGUF file as transcribe.cpp
 * writes it: the shape under `prefix` (NULL: from general.architecture,
 * `stt.qwen3_asr.decoder` for qwen3_asr; keys hidden_size,
 * intermediate_size, n_layers, n_heads, n_kv_heads, head_dim, vocab_size,
 * rms_norm_eps, rope_theta, tie_word_embeddings, gguf/blocks.rs:25-45) and
 * the `dec.*` tensors (gguf/qwen3_asr.rs:103-136; qk_norm when
 * attn.q_norm is there). Q8_0 and Q4_K linears (q, k, v stacked; gate, up
 * stacked), F32/F16 norms, an F16 or F32 token table; output.weight only
 * when the head is untied. The config read is written to *config (may be
 * NULL). Replaces the GGUF branch of CausalLm::from_tensors
 * (causal_lm.rs:141-198) for these files. */
int trit_hip_decoder_from_gguf(const char *path, const char *prefix, TritHipLmConfig *config, TritHipDecoder **out);

#ifdef __cplusplus
}
#endif

#endif
