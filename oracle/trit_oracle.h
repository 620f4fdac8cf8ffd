/* CPU restatement of Trit's decoder-loop numerics.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT CODE. Only the tests, the smoke check
 * and the CPU-baseline leg of the benchmark load this library, and only as
 * the checker (or, in the benchmark, as the timed CPU baseline). The HIP
 * library never links or calls it.
 *
 * Every function restates a function of the Rust reference (Hi9841/trit);
 * the citation beside each declaration is the file:line it follows. The
 * "contract" path (isa 0) is the portable scalar statement of the bits that
 * Trit's default x86 path (AVX-512 VNNI, first kernel set) produces; isa 1
 * (AVX2) and isa 2 (AVX-512 VNNI) are SIMD restatements of Trit's tiles,
 * timed as the CPU baseline and checked bit for bit against isa 0.
 */
#ifndef TRIT_ORACLE_H
#define TRIT_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { OR_SCALAR = 0, OR_AVX2 = 1, OR_AVX512 = 2 };

/* Fastest path this CPU runs (src/cpu/isa.rs:16-115). */
int or_isa_best(void);

/* Worker team (src/cpu/team.rs:900-976, src/cpu/mod.rs:127-161,281-292):
 * spread 0 = physical cores of the largest L3 domain, pinned; 1 = all
 * allowed cores. threads > 0 overrides the count and turns pinning off.
 * Returns the team size. */
int or_team_start(int spread, int threads);
int or_team_size(void);
/* int8 multiply-adds per second of the team on independent vpdpbusd chains
 * (no memory traffic), `iters` rounds of 12 x 64 per thread; 0 without
 * AVX-512 VNNI. The yardstick of the baseline's fairness check. */
double or_vnni_peak(int64_t iters);

/* src/cpu/tensors.rs:542-573 and :575-595. */
uint16_t or_f32_to_f16(float value);
float or_f16_to_f32(uint16_t half);

/* Cephes expf as Trit's fused paths compute it
 * (src/cpu/activation.rs:8-38,357-375; src/cpu/v2/activation.rs:27-56). */
float or_exp(float x);
/* v / (1 + exp(0 - v)) (src/cpu/activation.rs:54-56,330). */
void or_silu(float* values, int64_t n);

/* Activation quantizer (src/cpu/kernels.rs:661-737,769-846;
 * src/cpu/v2/quantize.rs:71-171): m rows of k values in groups of `group`;
 * codes m*k, scales and sums m*(k/group). half_scales rounds each stored
 * scale through f16 after the codes are made. */
void or_quantize(int isa, const float* x, int m, int k, int group, int half_scales,
                 int8_t* codes, float* scales, int32_t* sums);

/* ggml Q8_0 quantization of f32 values, as Blocks::quantize
 * (src/cpu/gemm.rs:58-76): count is a multiple of 32. */
void or_q8_0_quantize(const float* values, int64_t count, int8_t* codes, float* scales);
/* GGUF Q8_0 block bytes (34 per block) to codes and f32 scales
 * (src/cpu/tensors.rs:282-305). */
void or_q8_0_parse(const uint8_t* blocks, int64_t nblocks, int8_t* codes, float* scales);
/* GGUF Q4_K super-blocks (144 bytes per 256 values) to f32
 * (src/cpu/ggml_quants.rs:168-196). */
void or_q4_k_expand(const uint8_t* blocks, int64_t nblocks, float* out);
/* The audio encoder's pieces (src/models/parts/audio_encoder.rs): the exact
 * GELU (src/cpu/v2/activation.rs:33-39), layer norm (src/layers.rs:50-121),
 * im2col (src/layers.rs:613-634). */
void or_gelu(float* values, int64_t n);
void or_layer_norm(const float* x, int rows, int d, const float* w, const float* b, float eps, float* out);
void or_conv_columns(const float* x, int frames, int channels, int kernel, int stride, int pad, int out_frames,
                     float* out);
/* f32_to_f16 / f16_to_f32 over arrays (src/cpu/tensors.rs:542-595). */
void or_f32_to_f16_n(const float* in, int64_t n, uint16_t* out);
void or_f16_to_f32_n(const uint16_t* in, int64_t n, float* out);
/* ggml's block types expanded to f32 (src/cpu/ggml_quants.rs:103-245):
 * Q4_0 2, Q4_1 3, Q5_0 6, Q5_1 7, Q4_K 12, Q5_K 13, Q6_K 14; -1 for others. */
int or_ggml_expand(int type, const uint8_t* blocks, int64_t nblocks, float* out);

/* Int8 layer with i8 activations (src/cpu/int8.rs:155-289,425-584;
 * src/cpu/v2/product.rs:156-423): codes row-major n*k, scales n*(k/group).
 * group 32 with half_scales 1 is ggml Q8_0; group 128 is Trit's int8. */
void* or_int8_new(int isa, int n, int k, int group, int half_scales,
                  const int8_t* codes, const float* scales);
void or_int8_forward(const void* layer, const float* x, int m, float* out);
void or_int8_free(void* layer);

/* Ternary layer (src/cpu/kernels.rs:72-307,353-420): codes 0..2 row-major
 * n*k (w = scale * (code - 1)), scales n*(k/128). */
void* or_ternary_new(int isa, int n, int k, const uint8_t* codes, const float* scales);
void or_ternary_forward(const void* layer, const float* x, int m, float* out);
void or_ternary_free(void* layer);
/* Base-3 file bytes (5 digits per byte, least significant first) to codes
 * 0..2 (src/cpu/kernels.rs:91-130,630-643). Returns -1 for a byte > 242. */
int or_ternary_from_base3(const uint8_t* packed, int n, int k, uint8_t* codes);

/* out = x * w^T with w as f16 bits, the 16-lane contract
 * (src/cpu/fgemm.rs:213-246,413-455; src/cpu/v2/float.rs:1-30,255-270). */
void or_matmul_f16(int isa, const float* x, int m, int k, const uint16_t* w, int n, float* out);
/* The same with f32 weights. */
void or_matmul_f32(int isa, const float* x, int m, int k, const float* w, int n, float* out);

/* RMSNorm in place over rows of d (src/layers.rs:136-144). */
void or_rmsnorm(const float* weight, int d, float eps, float* x, int rows);
/* Rotary halves table: sin/cos of pos * base^(-2i/dims), positions
 * [0, positions), pairs dims/2 (src/layers.rs:287-299,318). */
void or_rope_table(int dims, float base, int positions, float* sin_out, float* cos_out);
/* Rotary halves on `heads` heads of `rows` rows, row r at position first+r
 * (src/layers.rs:303-334). */
void or_rope(float* x, int rows, int stride, int heads, int hd, int first, float base);
/* Causal/non-causal GQA attention of tq queries over tk keys
 * (src/layers.rs:343-504,571-587): q rows of stride qs, k/v rows of stride
 * kvs; out tq*(heads*hd). */
void or_attention(const float* q, int qs, const float* k, const float* v, int kvs,
                  int tq, int tk, int heads, int kv_heads, int hd, int causal, float* out);
/* First index of the largest value (src/layers.rs:604-612). */
int or_argmax(const float* values, int n);

/* Decoder of the Llama plan with Qwen3 q/k norms and Granite's multipliers
 * (src/models/parts/causal_lm.rs:17-481). Linears are GGUF Q8_0 blocks or
 * Trit's int8 weights; the embedding and the head are token tables. */
typedef struct {
    int d, ffn, layers, heads, kv_heads, head_dim, vocab;
    float eps, rope_base;
    int qk_norm;
    /* Keys and values rounded through f16 where they are appended (the
     * device's f16 caches); 0 keeps Trit's f32 caches. */
    int kv_f16;
    /* Granite's multipliers (causal_lm.rs:17-78): 1 (attention: 0) is none. */
    float embedding_multiplier, attention_multiplier, residual_multiplier, logits_scaling;
} or_lm_config;

/* Token table kinds (Dense::table, src/cpu/gemm.rs:383-409). */
enum { OR_TABLE_F16 = 0, OR_TABLE_F32 = 1, OR_TABLE_Q8 = 2 };

void* or_lm_new(int isa, const or_lm_config* cfg);
/* One layer. qkv: (heads+2*kv_heads)*hd rows of d; o: d rows of heads*hd;
 * gate_up: 2*ffn rows of d; down: d rows of ffn; all as Q8_0 block bytes. */
int or_lm_set_layer(void* lm, int layer, const uint8_t* qkv, const uint8_t* o,
                    const uint8_t* gate_up, const uint8_t* down, const float* norm_attn,
                    const float* norm_mlp, const float* q_norm, const float* k_norm);
int or_lm_set_embed(void* lm, const uint16_t* embed_f16, const float* final_norm);
/* Linear `which` (0 qkv, 1 o, 2 gate_up, 3 down) of `layer` as Trit's int8
 * weights: codes row-major, one f32 scale per row and 128 inputs
 * (Int8::quantize's layer, src/cpu/int8.rs:292-369). */
int or_lm_set_linear_int8(void* lm, int layer, int which, const int8_t* codes, const float* scales);
/* Linear `which` as f16 bits (OR_TABLE_F16) or f32 (OR_TABLE_F32) weights,
 * row-major, with f32 math in the 16-lane order (Dense::half / Dense::new,
 * src/cpu/gemm.rs:189-221,500-525). */
int or_lm_set_linear_float(void* lm, int layer, int which, int kind, const void* weights);
/* Table `which` (0 the embedding, 1 the untied head) of kind OR_TABLE_*:
 * f16 bits, f32, or int8 codes with an f32 scale per 32 values (`scales`).
 * A head with data NULL is tied to the embedding again. */
int or_lm_set_table(void* lm, int which, int kind, const void* data, const float* scales);
/* Per-layer scales on the normed MLP input, layers x d, or NULL for none
 * (CausalLm::set_ffn_scales, causal_lm.rs:303-306,456-462). */
int or_lm_set_ffn_scales(void* lm, const float* scales);
/* Logits after rows of embeddings (n x d) at the next positions
 * (CausalLm::forward_rows, causal_lm.rs:374-389). */
int or_lm_forward_rows(void* lm, const float* rows, int n, float* logits);
/* Keeps the first `position` positions of the caches. */
int or_lm_truncate(void* lm, int position);
int or_lm_position(void* lm);
/* Embedding row of `token` as f32 (Dense::row, gemm.rs:412-429). */
int or_lm_embed_row(void* lm, int token, float* out);
/* Greedy tokens after `prompt` (CausalLm::generate with no prefix,
 * causal_lm.rs:217-249,284-302). Writes up to max_new tokens to out and
 * returns their count; logits (optional) receives the logits after the
 * prompt. */
int or_lm_generate(void* lm, const int32_t* prompt, int n_prompt, int max_new,
                   const int32_t* stop, int n_stop, int32_t* out, float* logits);
/* Logits after running `tokens` at positions [first, first+n) on an
 * explicit session cache; or_lm_reset clears it. */
int or_lm_forward(void* lm, const int32_t* tokens, int n, float* logits);
void or_lm_reset(void* lm);
void or_lm_free(void* lm);

#ifdef __cplusplus
}
#endif

#endif
