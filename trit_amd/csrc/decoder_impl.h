// Decoder and session structures shared by the per-kernel token loop
// (decoder.hip) and the persistent decode step (decode_step.hip).
#pragma once

#include <memory>
#include <mutex>
#include <vector>

#include "../../include/trit_hip.h"
#include "internal.h"

namespace trit {

constexpr int MAX_STOP = 64;

// Device state of a session.
struct State {
    int pos;        // positions in the caches
    int done;       // nonzero: the decode loop has ended
    int n_out;      // tokens written by the loop
    int max_new;    // loop limit
    int n_stop;     // stop tokens
    int token;      // the last token chosen
    unsigned int arrived;  // blocks of the greedy choice that are done (back to 0 after)
    int err;               // nonzero: a decode-step block waited past its deadline
    int stop[MAX_STOP];
};

struct DecoderImpl {
    TritHipLmConfig c{};
    std::vector<LayerRef> qkv, o, gate_up, down;
    LayerRef embed, head;
    DeviceMemory norms;  // per layer: attn[d] mlp[d] q[hd] k[hd]; then final[d]
    size_t layer_norm_stride = 0;
    const float* norm_attn(int l) const { return norms.as<float>() + l * layer_norm_stride; }
    const float* norm_mlp(int l) const { return norm_attn(l) + c.d; }
    const float* q_norm(int l) const { return norm_attn(l) + 2 * c.d; }
    const float* k_norm(int l) const { return q_norm(l) + c.head_dim; }
    const float* final_norm() const { return norms.as<float>() + c.layers * layer_norm_stride; }
    // The head in the persistent step's tiled f16 layout, made on first use.
    mutable DeviceMemory step_head;
    mutable std::once_flag step_head_once;
    // Some layer's gate_up takes f32 math (its SwiGLU is a kernel of its own).
    bool float_gate_up = false;
    // Per layer, d scales on the normed MLP input (set_ffn_scales); a
    // counter of their changes (sessions rebuild what depends on them).
    DeviceMemory ffn_scales;
    bool has_ffn_scales = false;
    int ffn_version = 0;
    // Granite's multipliers (1, and 0 for the attention's, elsewhere).
    bool granite() const {
        return c.embedding_multiplier != 1.0f || c.attention_multiplier != 0.0f || c.residual_multiplier != 1.0f ||
               c.logits_scaling != 1.0f;
    }
};

struct SessionImpl {
    std::shared_ptr<DecoderImpl> dec;
    int max_pos = 0, flags = 0;
    bool exact = false, kv32 = false;
    int rows_cap = 0;
    DeviceMemory kcache, vcache, rope_sin, rope_cos;
    DeviceMemory x, qkv, att, hid, inv, normed, logits, state, tokens_in, tokens_out, partials;
    DeviceMemory att_part, att_arrived;  // split attention: chunk partials, per (row, kv head) counters
    DeviceMemory gemm_scratch;           // quantized rows of the matrix-core products
    DeviceMemory xn;                     // rows x d: normed rows, a residual branch
    DeviceMemory wide;                   // rows x 2 ffn: a float-math gate_up's product
    // generate_additive: rows x d f32 added to each input, by position.
    DeviceMemory additive;
    int additive_rows = 0;
    // What the captured step was built with.
    int graph_ffn_version = -1;
    bool graph_additive = false;
    int max_splits = 0;
    int host_pos = 0;
    hipGraphExec_t graph = nullptr;
    int graph_out_cap = 0;
    // The persistent decode step: exchange words, per-block candidates of
    // the greedy choice, per-layer pointer table; a launch counter makes
    // each launch's exchange tags unique.
    DeviceMemory step_words, step_cand, step_table;
    uint32_t step_seq = 0;
    bool step_cand_fresh = false;  // candidates newer than `logits`
    // A decode step missed its deadline: the caches and the device state
    // hold a partial step, so the session refuses work until it is reset.
    bool broken = false;

    ~SessionImpl() {
        if (graph) (void)hipGraphExecDestroy(graph);
    }
    State* st() const { return state.as<State>(); }
};

// Prefill attention on the matrix cores (attention_mfma.hip): fast mode
// with f16 caches; rows of the forward at positions pos0.., layer `layer`.
bool flash_prefill_supported(const SessionImpl& S);
void flash_prefill(SessionImpl& S, int layer, int rows, int pos0, hipStream_t s);
// The same kernel on any queries and f16 caches ([kv head][max_pos][128]):
// rows query rows (stride qs floats) at positions pos0.., over tk keys;
// causal, or every key for every row; out rows of heads * 128 floats.
void flash_attention(const float* q, int qs, const _Float16* kc, const _Float16* vc, int max_pos, int heads,
                     int kv_heads, int rows, int pos0, int tk, int causal, float* out, hipStream_t s);

// Trit's attention (exact kernel) over device rows: q rows of stride qs,
// k and v rows of stride kvs; kc / vc scratch of kv_heads x tk x hd floats;
// st a device State with pos = tk - tq, done = 0 (decoder.hip).
void exact_attention(const float* q, int qs, const float* k, const float* v, int kvs, int tq, int tk, int heads,
                     int kv_heads, int hd, int causal, float* out, float* kc, float* vc, State* st, hipStream_t s);

// The persistent decode step (decode_step.hip).
// Whether the session's model and mode run on it.
bool decode_step_supported(const SessionImpl& S);
// How the step runs the session: 1, or 3 when its attention runs on every
// block with each key/value head's exchanges in one XCD's L2; 0 when the
// session does not run on the step.
int decode_step_layout(const SessionImpl& S);
// Prepares the exchange buffers and, when the last logits are newer than
// the step's candidates, the candidates from the logits.
void decode_step_prepare(SessionImpl& S, hipStream_t s);
// Greedy steps `step` .. `step + nsteps - 1` of a generate call (choice,
// forward, head each) in one launch, the first at cache position `pos`.
void decode_step_launch(SessionImpl& S, int step, int pos, int nsteps, hipStream_t s);

}  // namespace trit
