// The persistent decode step: one launch runs a generate call's greedy
// tokens, each its choice, every layer and the head
// (src/models/parts/causal_lm.rs:284-302,410-481), on all CUs at once, one
// block per CU.
//
// Blocks hand activations to each other through exchange words: 8 bytes
// holding an f32 value and a 32-bit tag, written with one agent-scope store
// and polled with agent-scope loads until the tag is the one the reader
// waits for. The tag names the token step and the phase, so a word is never
// mistaken for an older one, and no barrier, fence or cache flush is
// needed between phases. The key and value caches are written with
// agent-scope stores (through the L2) and read with plain loads: each
// appending wave waits for its stores before the block barrier that
// precedes the block's next put, so a reader that saw a later tag reads
// them from memory (no XCD has their lines cached before they are
// written: a key's lines hold only that key). A phase's weights do not depend on its inputs:
// each block issues their loads before it waits, so the weight stream
// overlaps the hand-over instead of following it.
//
// Per layer (tags in order): qkv product -> attention partials (32 key
// splits per key/value head, one per block) -> combined attention -> o
// product + residual -> gate_up product + SwiGLU -> down product +
// residual. Then the final RMSNorm, the f16 head and each block's best
// logit, published as two more exchange words; the next step's first act
// is the greedy choice over those candidates (first maximum wins,
// src/layers.rs:604-612). The first step of a launch takes them from where
// the previous launch, or the prompt's logits, left them.
//
// Products use the one-row kernel's arithmetic (gemv_decode.hip): Trit's
// quantizer, exact i32 block dots and the f32 group chain in order, so
// their values are Trit's bit for bit given the same input. The default
// instance keeps Trit's sum orders (the serial RMSNorm, q/k norm, softmax
// and p.V chains, bit for bit the f16-cache oracle); the tree-sum instance
// sums those as trees. Every wait has a deadline: a block that misses it
// marks the session's error flag and the launch drains.
#include "decoder_impl.h"
#include "device.h"

#include <algorithm>
#include <climits>
#include <cstdio>
#include <type_traits>

namespace trit {
namespace {

constexpr int T = 512;         // threads per block
constexpr int NW = T / WAVE;   // waves per block
constexpr int HD = 128;        // head_dim
constexpr int MAXC = 4;        // 32-key chunks of a split held in registers
constexpr int MAXF = 12;       // 32-key chunks of the one-pass attention (384 positions)
constexpr int MAXT = 4096;     // positions of a Trit-order session on the step (the long attention)
constexpr int MAXD = 2048;     // largest d
constexpr int MAXK = 6144;     // largest product input
constexpr int PH = 6;          // exchange phases per layer
constexpr int MAXL = 41;       // layers: the exchange tags of a step fit in 8 bits
constexpr int BPH = 16;        // the wide attention: blocks a query head
constexpr int WD = HD / BPH;   // its output dims a block

constexpr int cmax(int x, int y) { return x > y ? x : y; }

// Phase stamps (a measurement build, TRIT_HIP_STEP_STAMPS): thread 0 of
// each block writes the device wall clock (100 MHz, the same on every XCD)
// and its shader clock at fixed points of one chosen (step, layer) of a
// launch; trit_hip_step_stamps_read copies them out. Stamp points:
//   0 layer start, 1 x gathered, 2 RMSNorm, 3 quantized, 4 qkv rows put;
//   attention blocks: 5 before the qkv gather, 6 gathered, 7 q/k norm,
//   rotary and append, 8 scores, max and exp, 9 softmax sum, 10 p.V put;
//   11 attention gathered (o input), 12 quantized, 13 o rows put,
//   14 x gathered, 15 RMSNorm, 16 quantized, 17 gate_up put, 18 h gathered,
//   19 quantized, 20 down put; the head (layer = layers): 21 x gathered,
//   22 normed, 23 passes done, 24 candidates put.
#ifdef TRIT_HIP_STEP_STAMPS
constexpr int NSTAMP = 32;
constexpr int MAX_STAMP_BLOCKS = 1024;
__device__ unsigned long long g_stamp_wall[MAX_STAMP_BLOCKS][NSTAMP];
__device__ unsigned long long g_stamp_clk[MAX_STAMP_BLOCKS][NSTAMP];
#define STAMP(k)                                                            \
    do {                                                                    \
        if (threadIdx.x == 0 && sm.stamp) {                                 \
            g_stamp_wall[blockIdx.x][k] = wall_clock64();                   \
            g_stamp_clk[blockIdx.x][k] = __builtin_readcyclecounter();      \
        }                                                                   \
    } while (0)
#define STAMP_BY(k, thr)                                                    \
    do {                                                                    \
        if ((int)threadIdx.x == (thr) && sm.stamp) {                        \
            g_stamp_wall[blockIdx.x][k] = wall_clock64();                   \
            g_stamp_clk[blockIdx.x][k] = __builtin_readcyclecounter();      \
        }                                                                   \
    } while (0)
#define STAMP_WHEN(cond)                         \
    do {                                         \
        if (threadIdx.x == 0) sm.stamp = (cond); \
    } while (0)
#else
#define STAMP_BY(k, thr) \
    do {                 \
    } while (0)
#define STAMP(k) \
    do {         \
    } while (0)
#define STAMP_WHEN(cond) \
    do {                 \
    } while (0)
#endif

// The linears' kinds the step takes: Q8_0 (and Q4_K after requantization):
// 32-groups with f16 scales; Trit's int8: 128-groups with f32 scales. Codes
// are row-major n x k int8 and scales row-major n x (k / group) either way.
enum : int { WK_Q8_0 = 0, WK_INT8 = 1 };
// The head's kinds: an f16 table, or int8 storage with an f32 scale per 32
// (Q8, f32 math).
enum : int { HK_F16 = 0, HK_Q8 = 1 };

struct LayerPtrs {
    const uint8_t* codes[4];  // qkv, o, gate_up, down: int8 codes n x k
    const void* scales[4];    // f16 bits (WK_Q8_0) or f32 (WK_INT8)
    const float* norm_attn;
    const float* norm_mlp;
    const float* q_norm;
    const float* k_norm;
    // [kv head][position][HD], f16 -- or f32 in the f32-cache instance,
    // whose attention reads them as float (attention_exact32).
    _Float16* kcache;
    _Float16* vcache;
};

struct StepArgs {
    const LayerPtrs* layers;
    int n_layers, d, qd, ffn, heads, kvh, vocab, qk_norm, max_pos;
    float eps;
    const void* embed;         // lane-chain table, vocab x d: f16 bits, or int8 codes (embed_q8)
    const float* embed_scales; // the int8 table's scales, vocab x d / 32
    int embed_q8;
    const void* head;          // the head in 4-row tiles (head_tile_kernel): f16 bits or int8 codes
    const float* head_scales;  // the int8 head's scales, vocab x d / 32
    const float* final_norm;
    const float* rope_sin;  // [position][HD / 2]
    const float* rope_cos;
    uint64_t* X;     // d words: the residual stream after o / down
    uint64_t* QKV;   // (heads + 2 kvh) * HD words
    uint64_t* PART;  // heads * splits * (HD + 2) words: max, sum, p.V
    uint64_t* ATT;   // heads * HD words
    uint64_t* H;     // ffn words
    uint64_t* CAND;  // 2 words per block: its best logit and that row's index
    uint64_t* SC;    // the wide attention's scores: T words a query head
    float2* cand;    // per block: best logit, its index (int bits)
    int* out;
    State* st;
    int splits;               // key splits per key/value head (blocks / kvh)
    int comb;                 // combined attention outputs per block
    int rq, ro, rgu, rd;      // rows per block (gate_up: pairs), multiples of 4
    int rh;                   // head rows per block
    unsigned long long ticks; // wall-clock ticks a block may wait in a step
    int norm_window;          // RMSNorm and softmax sums: candidate starts on either side of the estimate
    // Granite's multipliers (1 where a model has none): the embedding rows
    // times em, q times q_scale after the rotary, the residual adds x + rm y,
    // the logits times logit_w; and per-layer MLP input scales (d a layer)
    // or null. The Trit-order instance only.
    float em, q_scale, rm, logit_w;
    const float* ffn_scales;
    // generate_additive: rows x d added to the input at their positions
    // (before em, as the per-kernel loop adds them), or null.
    const float* additive;
    int additive_rows;
    int stamp_step, stamp_layer;  // the stamped (step, layer); layer == n_layers: the head
    // Nonzero: the q/k/v rows of key/value head x are made by the blocks on
    // XCD x, the attention of head x runs on them (attention_wide_a/_b),
    // and the qkv rows and the scores pass through that XCD's L2
    // (put_local). Set by the host where the model and the device allow it
    // (the Trit-order instance of up to T positions, one key/value head an
    // XCD). xcd_count: NX counters, zero at the launch, that give each
    // block its rank on its XCD.
    int local_qkv;
    unsigned int* xcd_count;
};

struct Smem {
    // The per-layer pointers, copied from the table at the launch's start:
    // reading them from LDS waits for nothing else, where a vector load of
    // the table would wait for every weight load in flight.
    LayerPtrs layers[MAXL];
    alignas(16) float xres[MAXD];  // the residual stream, this phase's copy
    alignas(16) float xin[MAXK];   // a product's input / gathered partials
    alignas(16) int8_t xq[MAXK];
    alignas(16) float xs[MAXK / 32];
    alignas(16) float qkv[6 * HD];  // a key/value head's q heads, k, v
    alignas(16) float kvn[2][HD];   // the new key and value, as cached
    alignas(16) uint16_t knew[HD];  // the new key's f16 bits
    union {
        alignas(16) float gpart[32][2 * HD];  // attention: per 16-lane group p.V of two heads
        struct {
            alignas(16) float sq[MAXD];  // RMSNorm: the squares
            float part[NW];              // each segment's sum as a tree
            float res[NW][WAVE];         // each segment's chain, lane L from candidate L
        } ns;
        // The exact attention: the cached values of the block's 64 dims,
        // row-major (key j's 64 values: 128 contiguous bytes).
        alignas(16) _Float16 vs[T][HD / 2];
        // The head of a wide model: the normed x by lane chain, chain i at
        // [i (d / 16 + 4)] (padded: the 16 chains' reads fall in distinct banks).
        alignas(16) float xt[16 * (MAXD / 16 + 4)];
        // The wide attention: the cached values of the block's WD dims (f16
        // bits), dim-major (row d: the T keys, padded so that the lanes'
        // reads of a row fall in distinct banks).
        alignas(16) uint16_t vth[WD][T + 8];
    };
    alignas(16) float probs[MAXT];        // the exact attention's scores, then probabilities
    float spart[NW];                      // its sum: each segment's tree sum
    float sres[NW][WAVE];                 // its sum: each segment's chain from candidate L
    float carry[WAVE];                    // its p.V sums, passed from wave to wave
    float ppos;                           // the new key's probability
    float wmax[NW];
    float gmax[32][2];
    float gl[32][2];
    float bv[T];
    int bi[T];
    float dcarry[4 * NW];  // a down product in two rounds: the first round's row totals
    float inv;
    int abort;
    int token;
    int stamp;  // thread 0: this layer is the stamped one
    int xcd, xrank;  // with local_qkv: the block's XCD and its rank there
};
static_assert(sizeof(Smem) <= 160 * 1024, "the step's LDS fits one block a CU");

__device__ __forceinline__ uint32_t tag_of(uint32_t tag0, int layer, int phase) {
    return tag0 + (uint32_t)(layer * PH + phase + 1);
}

__device__ __forceinline__ void put(uint64_t* p, float v, uint32_t tag) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t peek(const uint64_t* p) {
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// XCDs of the device. The dispatcher deals workgroups to the XCDs in turn,
// but not always from XCD 0, so a block learns its XCD from the hardware
// and its rank there from a counter (the step's launch start).
constexpr int NX = 8;
__device__ __forceinline__ int xcc_id() {
    return __builtin_amdgcn_s_getreg((3 << 11) | 20) & 0xf;  // HW_REG_XCC_ID, bits 3:0
}

// An exchange word for readers on the writer's XCD only: a store without
// scope bits goes through the CU's write-through L1 into the XCD's L2 and
// stays there; an agent-scope load (peek) from a CU of the same XCD
// returns that line (about 0.13 us from store to sight on MI355X, against
// 0.5-0.6 us for an agent-scope store, which writes through to memory).
// Readers on other XCDs would not see it until the line leaves the L2, so
// a word written with put_local is read on its writer's XCD only, and no
// other XCD writes its 128-byte line in the same launch.
__device__ __forceinline__ void put_local(uint64_t* p, float v, uint32_t tag) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
}

// Reductions over a wave: DPP inside each row of 16 lanes (every lane gets
// its row's result), then the four rows by readlane (uniform result).
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp<DPP_XOR1>(v);
    v += dpp<DPP_XOR2>(v);
    v += dpp<DPP_HALF_MIRROR>(v);
    v += dpp<DPP_MIRROR>(v);
    return v;
}
__device__ __forceinline__ float row8_sum(float v) {
    v += dpp<DPP_XOR1>(v);
    v += dpp<DPP_XOR2>(v);
    v += dpp<DPP_HALF_MIRROR>(v);
    return v;
}
__device__ __forceinline__ float row16_max(float v) {
    v = __builtin_fmaxf(v, dpp<DPP_XOR1>(v));
    v = __builtin_fmaxf(v, dpp<DPP_XOR2>(v));
    v = __builtin_fmaxf(v, dpp<DPP_HALF_MIRROR>(v));
    v = __builtin_fmaxf(v, dpp<DPP_MIRROR>(v));
    return v;
}
// s_waitcnt vmcnt(0), the other counters left alone (gfx9 encoding:
// vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
constexpr int VMCNT0 = 0x0f70;

__device__ __forceinline__ float lane_f(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
__device__ __forceinline__ float wave_sum(float v) {
    v = row16_sum(v);
    return ((lane_f(v, 0) + lane_f(v, 16)) + lane_f(v, 32)) + lane_f(v, 48);
}
__device__ __forceinline__ float wave_max(float v) {
    v = row16_max(v);
    return __builtin_fmaxf(__builtin_fmaxf(lane_f(v, 0), lane_f(v, 16)), __builtin_fmaxf(lane_f(v, 32), lane_f(v, 48)));
}

// A block that missed a deadline leaves the launch where it finds out
// (every wave of the block reads the same flag after a barrier). Ending
// the program there, rather than returning through the layer loop, keeps
// the abort paths out of the loop's control flow: joined to it, their
// loads in flight would make the compiler wait for everything a wave has
// in flight (its exchange stores too) on the paths that go on.
[[noreturn]] __device__ __forceinline__ void leave() { __builtin_amdgcn_endpgm(); }

// Whether the block has given up (one LDS word; read into a scalar
// register, so that the branch on it is uniform to the compiler too).
__device__ __forceinline__ bool aborted(Smem& sm) {
    return __builtin_amdgcn_readfirstlane(__hip_atomic_load(&sm.abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) !=
           0;
}

// Waits for n exchange words tagged `tag` (word i at src[index(i)]) and
// stores their values in dst[i]. Wave p0 + k polls words
// [k WAVE MW, (k + 1) WAVE MW), lane l word l + WAVE j of them (one base
// address, constant offsets), so ceil(n / (WAVE MW)) waves from p0 poll
// and the rest only wait at the barrier. A wave's vector memory operations
// complete in order, so a wave that has just stored exchange words or
// issued weight loads sees its polls late: each phase picks p0 and MW to
// poll from waves without such work in flight (measured on the device).
// Ends with a block barrier; false when a word missed the deadline (the
// block then leaves the launch).
template <int MW, typename Index>
__device__ __forceinline__ bool gather(int t, const uint64_t* src, int n, Index index, uint32_t tag, float* dst, Smem& sm,
                       unsigned long long deadline, State* st, int p0 = 0) {
    const int i0 = (t / WAVE - p0) * WAVE * MW + t % WAVE;
    if (i0 >= 0 && i0 < n) {  // uniform per wave: whether the wave polls
        uint64_t w[MW];
#pragma unroll
        for (int j = 0; j < MW; ++j) w[j] = 0;  // tag 0 is never waited for
        unsigned spins = 0;
        if (deadline == 0) {
            // A deadline of zero ticks (set only by the host's test override)
            // has passed before the first poll.
            __hip_atomic_store(&sm.abort, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            atomicOr(&st->err, 1);
        }
        while (deadline != 0) {
            bool ok = true;
#pragma unroll
            for (int j = 0; j < MW; ++j) {
                const int i = i0 + WAVE * j;
                if (i < n && (uint32_t)(w[j] >> 32) != tag) w[j] = peek(src + index(i));
            }
#pragma unroll
            for (int j = 0; j < MW; ++j) {
                const int i = i0 + WAVE * j;
                if (i < n && (uint32_t)(w[j] >> 32) != tag) ok = false;
            }
            if (ok) break;
            if ((++spins & 31) == 0) {
                if (aborted(sm)) break;
                if (wall_clock64() > deadline) {
                    __hip_atomic_store(&sm.abort, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                    atomicOr(&st->err, 1);
                    break;
                }
            }
        }
#pragma unroll
        for (int j = 0; j < MW; ++j) {
            const int i = i0 + WAVE * j;
            if (i < n) dst[i] = __uint_as_float((uint32_t)w[j]);
        }
    }
    __syncthreads();
    return !aborted(sm);
}


struct Linear {
    __device__ int operator()(int i) const { return i; }
};

// ---- products -----------------------------------------------------------

// A wave's four rows of one product (SwiGLU: four gate rows and their up
// rows): lane l of a row holds 16-byte chunks l + 16j of it and the scales
// of their blocks, as the one-row kernel loads them. A wave holds one
// product's rows at a time, so every product shares one register set:
// N chunks and NS scale words, product (J, P) using w[p J + j] and
// ws[p J + j].
template <int N, int NS>
struct Rows {
    uint4 w[N];
    // f16 scale bits, one a register, each the destination of its own load:
    // no arithmetic touches a loaded value before the product needs it
    // (packing two loaded halves into one register would wait for the
    // loads, and with them for every load issued before).
    uint32_t ws[NS];
};

// Lane l of a row takes chunk l + 16 j: for Q8_0 the scale of its 32-block
// (l / 2 + 8 j), for int8 that of its 128-group (l / 8 + 2 j). Rows of JT
// chunks a lane (256 JT inputs); the set takes chunks J0 .. J0 + J - 1 (a
// product in rounds).
template <int J, int P, int WK, int N, int NS, int JT = J, int J0 = 0>
__device__ __forceinline__ void load_rows(int t, const uint8_t* codes, const void* scales, int part_rows, int row,
                                          Rows<N, NS>& r) {
    static_assert(P * J <= N && P * J <= NS, "the row registers hold the product");
    static_assert(J0 + J <= JT, "the round lies in the row");
    constexpr int K = JT * 256;
    const int l = t & 15;
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const uint8_t* src = codes + (size_t)(p * part_rows + row) * K;
#pragma unroll
        for (int j = 0; j < J; ++j) r.w[p * J + j] = load_stream(src + (size_t)(l + 16 * (J0 + j)) * 16);
        if constexpr (WK == WK_Q8_0) {
            const TRIT_GLOBAL uint16_t* sc = gmem((const uint16_t*)scales) + (size_t)(p * part_rows + row) * (K / 32) + (l >> 1);
#pragma unroll
            for (int j = 0; j < J; ++j) r.ws[p * J + j] = sc[8 * (J0 + j)];
        } else {
            const TRIT_GLOBAL uint32_t* sc = gmem((const uint32_t*)scales) + (size_t)(p * part_rows + row) * (K / 128) + (l >> 3);
#pragma unroll
            for (int j = 0; j < J; ++j) r.ws[p * J + j] = sc[2 * (J0 + j)];
        }
    }
    // The rest of the set is zeroed: after any load no earlier rows stay live.
#pragma unroll
    for (int i = P * J; i < N; ++i) r.w[i] = make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int i = P * J; i < NS; ++i) r.ws[i] = 0;
}

// The row set zeroed, in the waves that load no rows in a phase: every path
// then writes the whole set before a product reads it, so no earlier rows
// stay live through the phases in between (the attention needs the room).
template <int N, int NS>
__device__ __forceinline__ void zero_rows(Rows<N, NS>& r) {
#pragma unroll
    for (int i = 0; i < N; ++i) r.w[i] = make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < NS; ++i) r.ws[i] = 0;
}

// RMSNorm factor of x (K = 256 J values in LDS) by one wave, the one-row
// kernel's tree: every block gets the same bits.
template <int J>
__device__ __forceinline__ float norm_inv_wave(int t, const float* x, float eps) {
    constexpr int K = J * 256;
    const int lane = t % WAVE;
    float part = 0.0f;
#pragma unroll
    for (int i = 0; i < J; ++i) {
        const float4 v = *(const float4*)(x + (size_t)(lane + WAVE * i) * 4);
        part += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
    }
    part += dpp<DPP_XOR1>(part);
    part += dpp<DPP_XOR2>(part);
    part += dpp<DPP_HALF_MIRROR>(part);
    part += dpp<DPP_MIRROR>(part);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, part), 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, part), 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, part), 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, part), 48));
    const float sum = ((r0 + r1) + r2) + r3;
    return 1.0f / __builtin_sqrtf(sum / (float)K + eps);
}

// The serial chain of a wave's values in lane order: lane L holds values
// N L .. N L + N - 1 of the chain in v[]; returns (in every lane) the sum
// ((c0 + v_0) + v_1) + ... in that order, for `lanes` lanes. Each round
// every lane runs the chain of its own values from the same carry, and the
// carry becomes lane L's result: the chain after lanes 0..L, bit for bit,
// with every operand in registers (a dependent add per value).
template <int N>
__device__ __forceinline__ float lane_chain(const float (&v)[N], float c0, int lanes) {
    float carry = c0;
    for (int L = 0; L < lanes; ++L) {
        float s = carry;
#pragma unroll
        for (int i = 0; i < N; ++i) s = s + v[i];
        carry = lane_f(s, L);
    }
    return carry;
}

// The serial chain ((c + p_0) + p_1) + ... over n4 float4 of LDS that
// every lane of the wave reads alike (broadcast reads), with D reads in
// flight: each read's result is used D reads after it issues, so the adds
// do not wait on the LDS latency between reads.
template <int D>
__device__ __forceinline__ float lds_chain(float c, const float* p, int n4) {
    float4 buf[D];
#pragma unroll
    for (int j = 0; j < D; ++j)
        if (j < n4) buf[j] = ((const float4*)p)[j];
    for (int i = 0; i < n4; i += D) {
#pragma unroll
        for (int j = 0; j < D; ++j) {
            if (i + j < n4) {
                const float4 v = buf[j];
                if (i + j + D < n4) buf[j] = ((const float4*)p)[i + j + D];
                // The refill issues before these adds (the scheduler would
                // otherwise sink it next to its use).
                __builtin_amdgcn_sched_barrier(0);
                c = c + v.x;
                c = c + v.y;
                c = c + v.z;
                c = c + v.w;
            }
        }
    }
    return c;
}

// RMSNorm factor of x (K = 256 J values in LDS) with Trit's sum -- the
// squares added one after another from 0 (src/layers.rs:138-139) -- bit
// for bit, by all the waves at once. Wave w chains segment w (values
// [S w, S w + S), S = K / NW) in order: wave 0 from 0, and each other wave,
// whose true start (the chain's value after the segments before) is not
// known yet, from 64 candidate starts at once, lane L from the float L - 32
// steps from an estimate of that start (the earlier segments' sums as
// trees, within a few steps of the chain: each add of the chain rounds by
// at most half a step of its value). The segments are then joined in
// order: the lane of segment w whose start equals the chain's value after
// segment w - 1 holds the chain's value after segment w; when no lane of
// the `window` lanes on either side does (the estimate that far off), the
// segment is chained again from that value. Every wave joins the segments
// itself and returns the factor.
template <int J>
__device__ float norm_inv_spec(int t, const float* x, float eps, int window, Smem& sm) {
    constexpr int K = J * 256, S = K / NW, PER = S / WAVE;
    static_assert(S % WAVE == 0 && PER <= 4, "a wave's segment: PER values a lane");
    const int w = __builtin_amdgcn_readfirstlane(t / WAVE), lane = t % WAVE;
    float* sq = sm.ns.sq;
    float part = 0.0f;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const float v = x[S * w + PER * lane + i];
        const float q = v * v;
        sq[S * w + PER * lane + i] = q;
        part += q;
    }
    const float seg = wave_sum(part);
    if (lane == 0) sm.ns.part[w] = seg;
    __syncthreads();
    float est[NW];
    est[0] = 0.0f;
#pragma unroll
    for (int q = 1; q < NW; ++q) est[q] = est[q - 1] + sm.ns.part[q - 1];
    const auto cand = [&](int q) {
        const int off = lane - WAVE / 2;
        if (q == 0) return 0.0f;
        if (off < -window || off > window) return __builtin_nanf("");
        const int bits = (int)__float_as_uint(est[q]) + off;
        return __uint_as_float((uint32_t)(bits < 0 ? 0 : bits));
    };
    float c = cand(0);
#pragma unroll
    for (int q = 1; q < NW; ++q)
        if (w == q) c = cand(q);
    c = lds_chain<8>(c, sq + S * w, S / 4);
    sm.ns.res[w][lane] = c;
    __syncthreads();
    float r[NW];
#pragma unroll
    for (int q = 0; q < NW; ++q) r[q] = sm.ns.res[q][lane];
    float sum = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, r[0])));
#pragma unroll
    for (int q = 1; q < NW; ++q) {
        const unsigned long long m = __ballot(cand(q) == sum);
        if (m) {
            sum = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, r[q]), __builtin_ctzll(m)));
        } else {
            for (int i = 0; i < S; ++i) sum = sum + sq[S * q + i];
        }
    }
    return 1.0f / __builtin_sqrtf(sum / (float)K + eps);
}

// The RMSNorm weights of the quantizer items a thread takes (item t + T i),
// loaded ahead of the phase's wait.
template <int J>
struct NormRegs {
    static constexpr int N = (J * 64 + T - 1) / T;
    float4 w[N];
};

template <int J>
__device__ __forceinline__ void load_norm(int t, const float* norm_w, NormRegs<J>& r) {
#pragma unroll
    for (int i = 0; i < NormRegs<J>::N; ++i) {
        const int item = t + T * i;
        r.w[i] = item < J * 64 ? gload_f4(norm_w + (size_t)item * 4) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
}

// Trit's activation quantizer over x (K values in LDS), optionally after
// RMSNorm x * (inv * w), into sm.xq / sm.xs; ends with a block barrier.
// Q8_0: 32-groups (8 lanes), the scale stored f16-rounded; int8: 128-groups
// (32 lanes), the f32 scale (src/cpu/kernels.rs:661-737).
template <int J, int WK>
__device__ void quantize_block(int t, const float* x, const NormRegs<J>* nr, float inv_in, Smem& sm,
                               const NormRegs<J>* fs = nullptr, bool inv_lds = false) {
    constexpr int ITEMS = J * 64;  // float4 items; a multiple of 64: whole waves
    const float inv = inv_lds ? sm.inv : inv_in;
#pragma unroll
    for (int i = 0; i < NormRegs<J>::N; ++i) {
        const int item = t + T * i;
        if (item >= ITEMS) break;  // uniform per wave
        float4 v = *(const float4*)(x + (size_t)item * 4);
        if (nr) {
            const float4 nw = nr->w[i];
            v.x = v.x * (inv * nw.x);
            v.y = v.y * (inv * nw.y);
            v.z = v.z * (inv * nw.z);
            v.w = v.w * (inv * nw.w);
        }
        if (fs) {  // the normed values times the layer's MLP scales
            const float4 f = fs->w[i];
            v.x = v.x * f.x;
            v.y = v.y * f.y;
            v.z = v.z * f.z;
            v.w = v.w * f.w;
        }
        float peak = __builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(v.x), __builtin_fabsf(v.y)),
                                     __builtin_fmaxf(__builtin_fabsf(v.z), __builtin_fabsf(v.w)));
        peak = __builtin_fmaxf(peak, dpp<DPP_XOR1>(peak));
        peak = __builtin_fmaxf(peak, dpp<DPP_XOR2>(peak));
        peak = __builtin_fmaxf(peak, dpp<DPP_HALF_MIRROR>(peak));
        if constexpr (WK == WK_INT8) {
            peak = __builtin_fmaxf(peak, dpp<DPP_MIRROR>(peak));
            peak = __builtin_fmaxf(peak, __shfl_xor(peak, 16));
        }
        const float scale = peak > 0.0f ? peak / 127.0f : 1.0f;
        const float q = 1.0f / scale;
        *(uint32_t*)(sm.xq + item * 4) =
            pack4(act_code(v.x * q), act_code(v.y * q), act_code(v.z * q), act_code(v.w * q));
        if constexpr (WK == WK_INT8) {
            if ((item & 31) == 0) sm.xs[item >> 5] = scale;
        } else {
            if ((item & 7) == 0) sm.xs[item >> 3] = f16_round(scale);
        }
    }
    __syncthreads();
}

// The one-row kernel's dots and f32 chain for a wave's rows; the total of
// each row lands in lane 14 of its 16 lanes. Trit's chain: total =
// fma(f32(dot_g), ws_g * xs_g, total) over the groups in order from 0
// (src/cpu/v2/product.rs:392-423). Q8_0: a block's two lanes add their
// dots, and the chain passes through the 8 blocks of a chunk by row_ror:2;
// int8: a group's 8 lanes add theirs, and the chain passes the chunk's two
// groups by row_ror:8 (ending in lanes 8..15). A round that starts at chunk
// J0 > 0 continues the chain from `start` (the total after the chunks
// before, in every lane of the row).
template <int J, int P, int WK, int N, int NS, int J0 = 0>
__device__ __forceinline__ void row_chain(int t, const Rows<N, NS>& r, const Smem& sm, float (&acc)[P],
                                          const float* start = nullptr) {
    const int l = t & 15;
#pragma unroll
    for (int p = 0; p < P; ++p) acc[p] = 0.0f;
    // The first step's input: 0 at the row's start, else the carried total.
    auto first_in = [&](int p) { return J0 == 0 ? 0.0f : start[p]; };
    if constexpr (WK == WK_INT8) {
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const uint4 xc = *(const uint4*)(sm.xq + (l + 16 * (J0 + j)) * 16);
            const float sc = sm.xs[(l >> 3) + 2 * (J0 + j)];
            float df[P], prod[P];
#pragma unroll
            for (int p = 0; p < P; ++p) {
                const uint4 wc = r.w[p * J + j];
                int d = sdot4(wc.x, xc.x, 0);
                d = sdot4(wc.y, xc.y, d);
                d = sdot4(wc.z, xc.z, d);
                d = sdot4(wc.w, xc.w, d);
                d += dpp<DPP_XOR1>(d);
                d += dpp<DPP_XOR2>(d);
                d += dpp<DPP_HALF_MIRROR>(d);
                df[p] = (float)d;
                prod[p] = __uint_as_float(r.ws[p * J + j]) * sc;
            }
#pragma unroll
            for (int q = 0; q < 2; ++q)
#pragma unroll
                for (int p = 0; p < P; ++p) {
                    const float in = (j == 0 && q == 0) ? first_in(p) : dpp<DPP_ROR8>(acc[p]);
                    acc[p] = __builtin_fmaf(df[p], prod[p], in);
                }
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < J; ++j) {
        // Chunk j's dots (the block's two halves meet by DPP), then the
        // chain's steps over blocks 8j .. 8j + 7.
        const uint4 xc = *(const uint4*)(sm.xq + (l + 16 * (J0 + j)) * 16);
        const float sc = sm.xs[(l >> 1) + 8 * (J0 + j)];
        float df[P], prod[P];
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const uint4 wc = r.w[p * J + j];
            int d = sdot4(wc.x, xc.x, 0);
            d = sdot4(wc.y, xc.y, d);
            d = sdot4(wc.z, xc.z, d);
            d = sdot4(wc.w, xc.w, d);
            d += dpp<DPP_XOR1>(d);
            df[p] = (float)d;
            prod[p] = f16_to_f32((uint16_t)r.ws[p * J + j]) * sc;
        }
#pragma unroll
        for (int q = 0; q < 8; ++q)
#pragma unroll
            for (int p = 0; p < P; ++p) {
                const float in = (j == 0 && q == 0) ? first_in(p) : dpp<DPP_ROR2>(acc[p]);
                acc[p] = __builtin_fmaf(df[p], prod[p], in);
            }
    }
}

// ---- attention ------------------------------------------------------------

// The keys of a split this lane holds: 16-lane group G takes keys
// j0 + G + 32i, lane l16 dims [8 l16, 8 l16 + 8).
struct KvRegs {
    uint4 k[MAXC], v[MAXC];
};

__device__ __forceinline__ void kv_prefetch(int t, const _Float16* K, const _Float16* V, int j0, int j1, int pos,
                                            KvRegs& kv) {
    const int G = t >> 4, l16 = t & 15;
#pragma unroll
    for (int i = 0; i < MAXC; ++i) {
        kv.k[i] = kv.v[i] = make_uint4(0, 0, 0, 0);
        if (j0 + 32 * i >= j1) continue;  // past the split's keys (uniform)
        const int j = j0 + G + 32 * i;
        if (j < j1 && j != pos) {  // the new key comes from the qkv product
            kv.k[i] = gload_u4(K + (size_t)j * HD + l16 * 8);
            kv.v[i] = gload_u4(V + (size_t)j * HD + l16 * 8);
        }
    }
}

__device__ __forceinline__ void unpack8(const uint4 r, float (&out)[8]) {
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        out[2 * i] = f16_to_f32((uint16_t)(w[i] & 0xffff));
        out[2 * i + 1] = f16_to_f32((uint16_t)(w[i] >> 16));
    }
}

// Block (kv head g, split s): q/k norm and rotary of the heads of g, the
// cache append (by the split that holds the new position), scores,
// softmax and p.V over the split's keys, written as partials (max, sum,
// unnormalised p.V) per query head.
template <int GROUP>
__device__ bool attention(int t, const StepArgs& a, const LayerPtrs& L, int pos, uint32_t tag_in, uint32_t tag_out,
                          Smem& sm, unsigned long long deadline) {
    const int b = blockIdx.x, g = b / a.splits, s = b % a.splits;
    const int tk = pos + 1, span = (tk + a.splits - 1) / a.splits;
    const int j0 = s * span, j1 = min(j0 + span, tk);
    const int heads = a.heads, kvh = a.kvh;
    const auto index = [g, heads, kvh](int i) {
        if (i < GROUP * HD) return g * GROUP * HD + i;
        if (i < (GROUP + 1) * HD) return (heads + g) * HD + (i - GROUP * HD);
        return (heads + kvh + g) * HD + (i - (GROUP + 1) * HD);
    };
    // The split's cached keys and values, the q/k norm weights and the
    // rotary values load while the qkv rows arrive.
    KvRegs kv;
    kv_prefetch(t, L.kcache + (size_t)g * a.max_pos * HD, L.vcache + (size_t)g * a.max_pos * HD, j0, j1, pos, kv);
    const int hh = t / WAVE, i = t % WAVE;
    float nw0 = 1.0f, nw1 = 1.0f, sn = 0.0f, cs = 1.0f;
    if (hh <= GROUP) {
        if (a.qk_norm) {
            const TRIT_GLOBAL float* nw = gmem(hh < GROUP ? L.q_norm : L.k_norm);
            nw0 = nw[i];
            nw1 = nw[i + HD / 2];
        }
        sn = gmem(a.rope_sin)[(size_t)pos * (HD / 2) + i];
        cs = gmem(a.rope_cos)[(size_t)pos * (HD / 2) + i];
    }
    // One wave polls: the first whose 16-lane groups load no key and that
    // stored no qkv value (the qkv rows sit in the last a.rq / 4 waves).
    const int kw = (j1 - j0 + 3) / 4, nqw = a.rq / 4;
    if (!gather<8>(t, a.QKV, (GROUP + 2) * HD, index, tag_in, sm.qkv, sm, deadline, a.st, kw < NW - nqw ? kw : 0))
        return false;

    // Wave hh takes head hh (the q heads, then k, then v), lane i its dims
    // i and i + 64 (a rotary pair): Qwen3's per-head RMSNorm (a shuffle
    // tree) and the rotary halves run in registers
    // (src/models/parts/causal_lm.rs:428-446, src/layers.rs:136-144,303-334).
    if (hh < GROUP + 2) {
        float x0 = sm.qkv[hh * HD + i], x1 = sm.qkv[hh * HD + i + HD / 2];
        if (hh <= GROUP) {
            if (a.qk_norm) {
                const float sum = wave_sum(x0 * x0 + x1 * x1);
                const float inv = 1.0f / __builtin_sqrtf(sum / (float)HD + a.eps);
                x0 = x0 * (inv * nw0);
                x1 = x1 * (inv * nw1);
            }
            const float ac = x0 * cs, bs = x1 * sn, bc = x1 * cs, as = x0 * sn;
            x0 = ac - bs;
            x1 = bc + as;
        }
        if (hh < GROUP) {
            const float scale = 1.0f / __builtin_sqrtf((float)HD);
            sm.qkv[hh * HD + i] = x0 * scale;
            sm.qkv[hh * HD + i + HD / 2] = x1 * scale;
        } else {
            // The new key (wave GROUP) or value (wave GROUP + 1), as cached.
            const int which = hh - GROUP;
            const _Float16 c0 = (_Float16)x0, c1 = (_Float16)x1;
            if (j0 <= pos && pos < j1) {
                // Later steps of this launch read them from other CUs: the
                // stores are agent-scope (written through to where every CU
                // reads).
                TRIT_GLOBAL uint16_t* cache =
                    gmem((uint16_t*)(which == 0 ? L.kcache : L.vcache)) + ((size_t)g * a.max_pos + pos) * HD;
                __hip_atomic_store(cache + i, __builtin_bit_cast(uint16_t, c0), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(cache + i + HD / 2, __builtin_bit_cast(uint16_t, c1), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            }
            sm.kvn[which][i] = (float)c0;
            sm.kvn[which][i + HD / 2] = (float)c1;
        }
    }
    __syncthreads();

    const int G = t >> 4, l16 = t & 15;
    float q[GROUP][8], kn[8], vn[8];
#pragma unroll
    for (int hl = 0; hl < GROUP; ++hl)
#pragma unroll
        for (int u = 0; u < 8; ++u) q[hl][u] = sm.qkv[hl * HD + l16 * 8 + u];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        kn[u] = sm.kvn[0][l16 * 8 + u];
        vn[u] = sm.kvn[1][l16 * 8 + u];
    }
    // Only the chunks the split's keys reach (uniform over the block).
    const int chunks = (j1 - j0 + 31) / 32;
    float sc[MAXC][GROUP], mx[GROUP];
#pragma unroll
    for (int hl = 0; hl < GROUP; ++hl) mx[hl] = -INFINITY;
#pragma unroll
    for (int i = 0; i < MAXC; ++i) {
#pragma unroll
        for (int hl = 0; hl < GROUP; ++hl) sc[i][hl] = -INFINITY;
        if (i >= chunks) continue;
        const int j = j0 + G + 32 * i;
        float k8[8];
        if (j == pos) {
#pragma unroll
            for (int u = 0; u < 8; ++u) k8[u] = kn[u];
        } else {
            unpack8(kv.k[i], k8);
        }
#pragma unroll
        for (int hl = 0; hl < GROUP; ++hl) {
            float acc = 0.0f;
#pragma unroll
            for (int u = 0; u < 8; ++u) acc = __builtin_fmaf(q[hl][u], k8[u], acc);
            acc += dpp<DPP_XOR1>(acc);
            acc += dpp<DPP_XOR2>(acc);
            acc += dpp<DPP_HALF_MIRROR>(acc);
            acc += dpp<DPP_MIRROR>(acc);
            sc[i][hl] = j < j1 ? acc : -INFINITY;
            mx[hl] = __builtin_fmaxf(mx[hl], sc[i][hl]);
        }
    }
    // 16-lane group G holds keys j0 + G + 32i: the groups' maxima, the
    // split's maximum, then each group's exp sums and p.V into LDS, summed
    // over the live groups in order.
    const int live = min(32, j1 - j0);
    static_assert(GROUP <= 2, "the group partials hold two query heads");
    if (l16 == 0)
#pragma unroll
        for (int hl = 0; hl < GROUP; ++hl) sm.gmax[G][hl] = mx[hl];
    __syncthreads();
    float M[GROUP];
#pragma unroll
    for (int hl = 0; hl < GROUP; ++hl) {
        M[hl] = -INFINITY;
        int q = 0;
        for (; q + 4 <= live; q += 4) {
            const float a0 = sm.gmax[q][hl], a1 = sm.gmax[q + 1][hl], a2 = sm.gmax[q + 2][hl], a3 = sm.gmax[q + 3][hl];
            M[hl] = __builtin_fmaxf(__builtin_fmaxf(M[hl], __builtin_fmaxf(a0, a1)), __builtin_fmaxf(a2, a3));
        }
        for (; q < live; ++q) M[hl] = __builtin_fmaxf(M[hl], sm.gmax[q][hl]);
    }
    float l[GROUP], acc[GROUP][8];
#pragma unroll
    for (int hl = 0; hl < GROUP; ++hl) {
        l[hl] = 0.0f;
#pragma unroll
        for (int u = 0; u < 8; ++u) acc[hl][u] = 0.0f;
    }
#pragma unroll
    for (int i = 0; i < MAXC; ++i) {
        if (i >= chunks) continue;
        const int j = j0 + G + 32 * i;
        float v8[8];
        if (j == pos) {
#pragma unroll
            for (int u = 0; u < 8; ++u) v8[u] = vn[u];
        } else {
            unpack8(kv.v[i], v8);
        }
#pragma unroll
        for (int hl = 0; hl < GROUP; ++hl) {
            const float p = sc[i][hl] == -INFINITY ? 0.0f : exp_trit(sc[i][hl] - M[hl]);
            l[hl] += p;
#pragma unroll
            for (int u = 0; u < 8; ++u) acc[hl][u] = __builtin_fmaf(p, v8[u], acc[hl][u]);
        }
    }
    if (G < live) {
#pragma unroll
        for (int hl = 0; hl < GROUP; ++hl) {
            if (l16 == 0) sm.gl[G][hl] = l[hl];
            *(float4*)(&sm.gpart[G][hl * HD + l16 * 8]) = make_float4(acc[hl][0], acc[hl][1], acc[hl][2], acc[hl][3]);
            *(float4*)(&sm.gpart[G][hl * HD + l16 * 8 + 4]) = make_float4(acc[hl][4], acc[hl][5], acc[hl][6], acc[hl][7]);
        }
    }
    __syncthreads();
    if (t < GROUP * HD) {
        const int hl = t / HD, ee = t % HD;
        float o = 0.0f;
        // In group order; four loads issued ahead of their adds.
        int q = 0;
        for (; q + 4 <= live; q += 4) {
            const float a0 = sm.gpart[q][hl * HD + ee], a1 = sm.gpart[q + 1][hl * HD + ee];
            const float a2 = sm.gpart[q + 2][hl * HD + ee], a3 = sm.gpart[q + 3][hl * HD + ee];
            o += a0;
            o += a1;
            o += a2;
            o += a3;
        }
        for (; q < live; ++q) o += sm.gpart[q][hl * HD + ee];
        const size_t base = ((size_t)(g * GROUP + hl) * a.splits + s) * (HD + 2);
        put(a.PART + base + 2 + ee, o, tag_out);
        if (ee == 0) {
            float lsum = 0.0f;
            for (int q2 = 0; q2 < live; ++q2) lsum += sm.gl[q2][hl];
            put(a.PART + base, M[hl], tag_out);
            put(a.PART + base + 1, lsum, tag_out);
        }
    }
    return true;
}

// Block b merges the splits of `comb` attention outputs (one query head's
// dims [e0, e0 + comb)) with the usual rescaling: wave e takes output e,
// lane s split s, and the sums are shuffle trees in a fixed order.
__device__ bool combine(int t, const StepArgs& a, uint32_t tag_in, uint32_t tag_out, Smem& sm,
                        unsigned long long deadline, int p0) {
    const int o0 = blockIdx.x * a.comb, h = o0 / HD, e0 = o0 % HD, per = 2 + a.comb;
    const int splits = a.splits;
    const auto index = [h, e0, per, splits](int i) {
        const int s = i / per, r = i - s * per;
        const int base = (h * splits + s) * (HD + 2);
        return r < 2 ? base + r : base + 2 + e0 + (r - 2);
    };
    // The qkv waves poll: the attention partials were stored by the first
    // waves, and the o rows are loading into the waves after gate_up's.
    if (!gather<2>(t, a.PART, splits * per, index, tag_in, sm.xin, sm, deadline, a.st, NW - a.rq / 4)) return false;
    const int e = t / WAVE, s = t % WAVE;
    if (e < a.comb) {
        const bool live = s < splits;
        const float m = live ? sm.xin[s * per] : -INFINITY;
        const float M = wave_max(m);
        const float w = m == -INFINITY ? 0.0f : exp_trit(m - M);
        const float Ls = wave_sum(live ? sm.xin[s * per + 1] * w : 0.0f);
        const float O = wave_sum(live ? sm.xin[s * per + 2 + e] * w : 0.0f);
        if (s == 0) put(a.ATT + o0 + e, O / Ls, tag_out);
    }
    return true;
}

// One pass over every key (sessions of up to 32 MAXF positions): block b
// takes key/value head g = b % kvh -- so a head's blocks share an XCD and its
// L2 -- and, of query head h = (b / kvh) % GROUP of that group, output dims
// [DPB s, DPB s + DPB), s = b / (kvh GROUP). Every block scores all the
// head's keys for its query head (8-lane group G the keys G + 64 i, lane
// l8 dims [16 l8, 16 l8 + 16)), so it finishes the softmax itself and
// stores its outputs as the o product's input: no partials and no combine
// hand-over. Lane l8 of a group takes the probability and value of the
// group's round l8; the 64 groups' own maxima, sums and p.V meet in LDS,
// and the first two waves rescale them (Measured: 8-lane groups score in
// half the instructions of 16-lane ones, whose 8-dim pieces spent as many
// lane moves on each key's sum as multiplies.) (Measured: sparing the polling wave the key
// loads, with 28 key groups, was slower; so was giving a head's blocks
// consecutive indices, spread over the XCDs.)
template <int GROUP, int DPB>
__device__ bool attention_all(int t, const StepArgs& a, const LayerPtrs& L, int pos, uint32_t tag_in,
                              uint32_t tag_out, Smem& sm, unsigned long long deadline) {
    static_assert(DPB == 4 || DPB == 8, "4 or 8 dims a block");
    const int b = blockIdx.x, kvh = a.kvh, g = b % kvh, hq = (b / kvh) % GROUP, e0 = DPB * (b / (kvh * GROUP));
    const int tk = pos + 1;
    const int heads = a.heads;
    const auto index = [g, heads, kvh](int i) {
        if (i < GROUP * HD) return g * GROUP * HD + i;
        if (i < (GROUP + 1) * HD) return (heads + g) * HD + (i - GROUP * HD);
        return (heads + kvh + g) * HD + (i - (GROUP + 1) * HD);
    };
    // Every cached key and this block's value dims load while the qkv rows
    // arrive; so do the q/k norm weights and the rotary values.
    const _Float16* K = L.kcache + (size_t)g * a.max_pos * HD;
    const _Float16* V = L.vcache + (size_t)g * a.max_pos * HD;
    // 64 groups of 8 lanes: group G takes keys G + 64 i, lane l8 dims
    // 16 l8 .. 16 l8 + 15 of each.
    const int G = t >> 3, l8 = t & 7, rounds = (tk + 63) / 64;
    uint4 kr[MAXF / 2][2];
#pragma unroll
    for (int i = 0; i < MAXF / 2; ++i) {
        kr[i][0] = kr[i][1] = make_uint4(0, 0, 0, 0);
        if (i >= rounds) continue;  // uniform
        const int j = G + 64 * i;
        if (j < tk && j != pos) {
            const _Float16* src = K + (size_t)j * HD + l8 * 16;
            kr[i][0] = gload_u4(src);
            kr[i][1] = gload_u4(src + 8);
        }
    }
    using VT = typename std::conditional<DPB == 8, uint4, uint2>::type;
    VT vr{};
    const int jv = G + 64 * l8;  // the key of this lane's probability
    if (l8 < rounds && jv < tk && jv != pos) {
        if constexpr (DPB == 8)
            vr = gload_u4(V + (size_t)jv * HD + e0);
        else
            vr = gload_u2(V + (size_t)jv * HD + e0);
    }
    const int hh = t / WAVE, i = t % WAVE;
    float nw0 = 1.0f, nw1 = 1.0f, sn = 0.0f, cs = 1.0f;
    if (hh <= GROUP) {
        if (a.qk_norm) {
            const TRIT_GLOBAL float* nw = gmem(hh < GROUP ? L.q_norm : L.k_norm);
            nw0 = nw[i];
            nw1 = nw[i + HD / 2];
        }
        sn = gmem(a.rope_sin)[(size_t)pos * (HD / 2) + i];
        cs = gmem(a.rope_cos)[(size_t)pos * (HD / 2) + i];
    }
    if (!gather<8>(t, a.QKV, (GROUP + 2) * HD, index, tag_in, sm.qkv, sm, deadline, a.st, NW - a.rq / 4 - 1))
        return false;

    // Qwen3's per-head RMSNorm and the rotary halves, wave hh head hh, lane
    // i dims i and i + 64 (src/models/parts/causal_lm.rs:428-446,
    // src/layers.rs:136-144,303-334); the first block of the head appends
    // the new key and value (agent scope: later steps read them elsewhere).
    if (hh < GROUP + 2) {
        float x0 = sm.qkv[hh * HD + i], x1 = sm.qkv[hh * HD + i + HD / 2];
        if (hh <= GROUP) {
            if (a.qk_norm) {
                const float sum = wave_sum(x0 * x0 + x1 * x1);
                const float inv = 1.0f / __builtin_sqrtf(sum / (float)HD + a.eps);
                x0 = x0 * (inv * nw0);
                x1 = x1 * (inv * nw1);
            }
            const float ac = x0 * cs, bs = x1 * sn, bc = x1 * cs, as = x0 * sn;
            x0 = ac - bs;
            x1 = bc + as;
        }
        if (hh < GROUP) {
            const float scale = 1.0f / __builtin_sqrtf((float)HD);
            sm.qkv[hh * HD + i] = x0 * scale;
            sm.qkv[hh * HD + i + HD / 2] = x1 * scale;
        } else {
            const int which = hh - GROUP;
            const _Float16 c0 = (_Float16)x0, c1 = (_Float16)x1;
            if (b < kvh) {
                TRIT_GLOBAL uint16_t* cache =
                    gmem((uint16_t*)(which == 0 ? L.kcache : L.vcache)) + ((size_t)g * a.max_pos + pos) * HD;
                __hip_atomic_store(cache + i, __builtin_bit_cast(uint16_t, c0), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(cache + i + HD / 2, __builtin_bit_cast(uint16_t, c1), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            }
            sm.kvn[which][i] = (float)c0;
            sm.kvn[which][i + HD / 2] = (float)c1;
        }
    }
    __syncthreads();

    // Scores of the group's keys for query head hq, and their maximum.
    // The new key (the key at pos: group pos % 64, round pos / 64, a round
    // the block knows) is taken as cached, its f16 bits selected into that
    // round's registers.
    float q[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) q[u] = sm.qkv[hq * HD + l8 * 16 + u];
    {
        const bool gf = G == (pos & 63);
#pragma unroll
        for (int c = 0; c < MAXF / 2; ++c) {
            if (c != (pos >> 6)) continue;  // uniform
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                uint32_t nb[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int d = l8 * 16 + 8 * h + 2 * u;
                    nb[u] = (uint32_t)f32_to_f16(sm.kvn[0][d]) | ((uint32_t)f32_to_f16(sm.kvn[0][d + 1]) << 16);
                }
                kr[c][h] = make_uint4(gf ? nb[0] : kr[c][h].x, gf ? nb[1] : kr[c][h].y, gf ? nb[2] : kr[c][h].z,
                                      gf ? nb[3] : kr[c][h].w);
            }
        }
    }
    float sc[MAXF / 2], mx = -INFINITY;
#pragma unroll
    for (int c = 0; c < MAXF / 2; ++c) {
        sc[c] = -INFINITY;
        if (c >= rounds) continue;
        const int j = G + 64 * c;
        float acc = 0.0f;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float k8[8];
            unpack8(kr[c][h], k8);
#pragma unroll
            for (int u = 0; u < 8; ++u) acc = __builtin_fmaf(q[8 * h + u], k8[u], acc);
        }
        acc = row8_sum(acc);
        sc[c] = j < tk ? acc : -INFINITY;
        mx = __builtin_fmaxf(mx, sc[c]);
    }
    // Lane l8: the probability of round l8's key against the group's
    // maximum, times its value dims; then the group's sums.
    float vv[DPB];
    {
        const uint32_t* vw = (const uint32_t*)&vr;
        const bool fresh_value = jv == pos;
#pragma unroll
        for (int d = 0; d < DPB; ++d) {
            const float loaded = f16_to_f32((uint16_t)(vw[d / 2] >> (16 * (d & 1))));
            vv[d] = fresh_value ? sm.kvn[1][e0 + d] : loaded;
        }
    }
    float mine = -INFINITY;
#pragma unroll
    for (int c = 0; c < MAXF / 2; ++c)
        if (c == l8) mine = sc[c];
    const float p = mine == -INFINITY ? 0.0f : exp_trit(mine - mx);
    float part[DPB + 1];
#pragma unroll
    for (int d = 0; d < DPB; ++d) part[d] = row8_sum(p * vv[d]);
    part[DPB] = row8_sum(p);
    // Group G's maximum, sum and p.V, flat in the attention scratch.
    float* gmax = &sm.gmax[0][0];
    float* gl = &sm.gl[0][0];
    float* gpart = &sm.gpart[0][0];
    if (l8 == 0) {
        gmax[G] = mx;
        gl[G] = part[DPB];
#pragma unroll
        for (int d = 0; d < DPB; ++d) gpart[G * DPB + d] = part[d];
    }
    __syncthreads();

    // The first two waves, DPB / 2 outputs each: lane G rescales group G by
    // exp(max_G - max); the sums are wave trees; o / l is the output.
    if (t < 2 * WAVE) {
        const int gg = t & (WAVE - 1), half = t / WAVE;
        const float m = gmax[gg];
        const float M = wave_max(m);
        const float f = m == -INFINITY ? 0.0f : exp_trit(m - M);
        const float l = wave_sum(f * gl[gg]);
        constexpr int DH = DPB / 2;
        float o[DH];
#pragma unroll
        for (int d = 0; d < DH; ++d) o[d] = wave_sum(f * gpart[gg * DPB + DH * half + d]);
        if (gg == 0) {
#pragma unroll
            for (int d = 0; d < DH; ++d)
                put(a.ATT + (size_t)(g * GROUP + hq) * HD + e0 + DH * half + d, o[d] / l, tag_out);
        }
    }
    return true;
}

// The chain sum ((0 + v_0) + v_1) + ... of the T values in LDS (zeros
// past the n that matter add nothing to these non-negative sums), bit for
// bit, by all the waves at once: norm_inv_spec's candidate-start segments.
// Wave w chains segment w (S values, S * NW <= T) from 64 candidate starts
// around the tree estimate of the chain before it; the segments are joined
// in order, and a segment whose true start no candidate holds is chained
// again from it. The join is the same in every wave (the same values and
// ballots), so its barrier is uniform. Every thread returns the sum.
__device__ float chain_sum_spec(int t, const float* v, int n, int window, Smem& sm) {
    const int w = __builtin_amdgcn_readfirstlane(t / WAVE), lane = t % WAVE;
    const int S = ((n + NW - 1) / NW + 3) & ~3;
    const float* seg = v + S * w;
    float part = 0.0f;
    for (int i = lane; i < S; i += WAVE) part += seg[i];
    const float ps = wave_sum(part);
    if (lane == 0) sm.spart[w] = ps;
    __syncthreads();
    float est[NW];
    est[0] = 0.0f;
#pragma unroll
    for (int q = 1; q < NW; ++q) est[q] = est[q - 1] + sm.spart[q - 1];
    const auto cand = [&](int q) {
        const int off = lane - WAVE / 2;
        if (q == 0) return 0.0f;
        if (off < -window || off > window) return __builtin_nanf("");
        const int bits = (int)__float_as_uint(est[q]) + off;
        return __uint_as_float((uint32_t)(bits < 0 ? 0 : bits));
    };
    float c = cand(0);
#pragma unroll
    for (int q = 1; q < NW; ++q)
        if (w == q) c = cand(q);
    for (int i = 0; i < S; i += 4) {
        const float4 x = *(const float4*)(seg + i);
        c = c + x.x;
        c = c + x.y;
        c = c + x.z;
        c = c + x.w;
    }
    sm.sres[w][lane] = c;
    __syncthreads();
    float sum = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, sm.sres[0][lane])));
    bool again = false;
#pragma unroll
    for (int q = 1; q < NW; ++q) {
        const unsigned long long m = __ballot(cand(q) == sum);
        if (m) {
            sum = __builtin_bit_cast(float,
                                     __builtin_amdgcn_readlane(__builtin_bit_cast(int, sm.sres[q][lane]), __builtin_ctzll(m)));
        } else {
            again = true;
            for (int i = 0; i < S; ++i) sum = sum + v[S * q + i];
        }
    }
    if (again) __syncthreads();  // the values stay read until every wave is done
    return sum;
}

// The cached keys and values that the next attention of a key/value head
// reads come into the L2 of the XCD its blocks share while the rest of the
// layer runs (from memory they arrive too slowly for one block to wait on):
// block r of the head's nb blocks loads one word of every nb-th 128-byte
// line of the head's n_keys keys and values, from `threads` threads, NT
// words a thread. The words stay in registers until the caller consumes
// them (a load whose value is dropped is not made).
// ESZ: bytes of a cached value (2: f16, 4: f32).
template <int NT, int ESZ = 2>
__device__ __forceinline__ void touch_kv(int t, int threads, const LayerPtrs& L, int g, int r, int nb, int n_keys,
                                         int max_pos, uint32_t (&v)[NT]) {
    const uint8_t* kb = (const uint8_t*)L.kcache + (size_t)g * max_pos * HD * ESZ;
    const uint8_t* vb = (const uint8_t*)L.vcache + (size_t)g * max_pos * HD * ESZ;
    constexpr int LINE = 128, PER_KEY = HD * ESZ / LINE;
    const int lines = PER_KEY * n_keys;
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        const int i = r + nb * (t + threads * j);
        if (i < 2 * lines) v[j] = *gmem((const uint32_t*)(i < lines ? kb + (size_t)LINE * i : vb + (size_t)LINE * (i - lines)));
    }
}

// Attention in Trit's order (src/layers.rs:442-504,571-587; the orders of
// src/cpu/fgemm.rs:665-793 and src/cpu/activation.rs exp_sums), on
// 2 * heads blocks: block b < 2 heads takes key/value head g = b % kvh (so
// a head's blocks share an XCD and its L2), query head g GROUP + (b / kvh)
// % GROUP, and output dims [64 h2, 64 h2 + 64), h2 = b / (kvh GROUP). The
// other blocks go on to the o product. Thread j scores key j (up to T
// keys) as one fused chain over the 128 dims of q * (1/sqrt(hd)), the f16
// key bits widened inside each multiply-add; the maximum (order-free);
// e_j = exp(s_j - max); their sum in key order from 0; p_j = e_j *
// (1/sum); and lane d of wave 0 chains p_j * v_j over the keys in order for
// dim 64 h2 + d, the values loaded straight into LDS while the qkv rows
// arrive. The q/k norm sums are serial chains too. The values are Trit's
// with the f16 caches, bit for bit.
template <int GROUP, int DPB>
__device__ bool attention_exact(int t, const StepArgs& a, const LayerPtrs& L, int pos, uint32_t tag_in,
                                uint32_t tag_out, Smem& sm, unsigned long long deadline) {
    const int b = blockIdx.x, kvh = a.kvh;
    if (b >= 2 * a.heads) {  // uniform over the block
        // These blocks wait for the attention's outputs: waiting for their
        // own stores now is free, and leaves the code after the attention
        // nothing in flight to wait for (see the end of this function).
        __builtin_amdgcn_s_waitcnt(VMCNT0);
        return true;
    }
    const int g = b % kvh, hq = g * GROUP + (b / kvh) % GROUP, h2 = b / (kvh * GROUP);
    const int tk = pos + 1;  // at most T (the host's plan)
    const int heads = a.heads;
    // Exchange word i: q head hq, then k head g, then v head g.
    const auto index = [hq, g, heads, kvh](int i) {
        if (i < HD) return hq * HD + i;
        if (i < 2 * HD) return (heads + g) * HD + (i - HD);
        return (heads + kvh + g) * HD + (i - 2 * HD);
    };
    const _Float16* K = L.kcache + (size_t)g * a.max_pos * HD;
    const _Float16* V = L.vcache + (size_t)g * a.max_pos * HD;
    const int w = t / WAVE, lane = t % WAVE;
    // The first half of key t (dims 0 .. 63) and the cached values'
    // 16-byte chunks (the block's 64 dims: chunk c is key c / 8, dims
    // 64 h2 + 8 (c % 8) ..) t, t + VT, ... of the first VT threads load
    // while the qkv rows arrive; the values go to LDS once the rows are
    // there, and the keys' second halves load then.
    constexpr int VT = T - WAVE, VC = (8 * T + VT - 1) / VT;
    uint4 kk[HD / 8];
#pragma unroll
    for (int i = 0; i < HD / 8; ++i) kk[i] = make_uint4(0, 0, 0, 0);
    uint32_t touch = 0;
    if (t < pos) {
#pragma unroll
        for (int i = 0; i < HD / 16; ++i) kk[i] = gload_u4(K + (size_t)t * HD + 8 * i);
        // One word of the key's second 128-byte line: the line comes to the
        // caches now, and the loads of that half after the hand-over hit them.
        touch = *gmem((const uint32_t*)(K + (size_t)t * HD + HD / 2));
    }
    uint4 vr[VC];
#pragma unroll
    for (int i = 0; i < VC; ++i) {
        vr[i] = make_uint4(0, 0, 0, 0);
        const int c = t + VT * i;
        if (t < VT && c < 8 * pos) vr[i] = gload_u4(V + (size_t)(c / 8) * HD + 64 * h2 + 8 * (c % 8));
    }
    // Wave 0 the q head, 1 the k head, 2 the v head; lane i dims i, i + 64.
    float nw0 = 1.0f, nw1 = 1.0f, sn = 0.0f, cs = 1.0f;
    if (w <= 1) {
        if (a.qk_norm) {
            const TRIT_GLOBAL float* nw = gmem(w == 0 ? L.q_norm : L.k_norm);
            nw0 = nw[lane];
            nw1 = nw[lane + HD / 2];
        }
        sn = gmem(a.rope_sin)[(size_t)pos * (HD / 2) + lane];
        cs = gmem(a.rope_cos)[(size_t)pos * (HD / 2) + lane];
    }
    // The last wave polls: it loads no value, and no key while the session
    // has at most (NW - 1) * 64 positions.
    const int p0 = pos <= VT ? NW - 1 : NW - a.rq / 4 - 1;
    STAMP(5);
    if (!gather<8>(t, a.QKV, 3 * HD, index, tag_in, sm.qkv, sm, deadline, a.st, p0)) leave();
    STAMP(6);
    asm volatile("" ::"v"(touch));
    // The cached values into LDS, row-major [key][64 dims].
#pragma unroll
    for (int i = 0; i < VC; ++i) {
        const int c = t + VT * i;
        if (t < VT && c < 8 * pos) *(uint4*)&sm.vs[c / 8][8 * (c % 8)] = vr[i];
    }
    if (t < pos) {
#pragma unroll
        for (int i = HD / 16; i < HD / 8; ++i) kk[i] = gload_u4(K + (size_t)t * HD + 8 * i);
    }

    // Qwen3's per-head RMSNorm (Trit's serial sum of the squares) and the
    // rotary halves, wave 0 the q head and wave 1 the k head, lane i dims i
    // and i + 64 (src/models/parts/causal_lm.rs:428-446, src/layers.rs:
    // 136-144,303-334); v as cached. The blocks with h2 = 0 and the first
    // query head of a group append the new key and value (agent scope:
    // later steps read them elsewhere).
    if (w < 3) {
        float x0 = sm.qkv[w * HD + lane], x1 = sm.qkv[w * HD + lane + HD / 2];
        if (w <= 1) {
            if (a.qk_norm) {
                float sq[16];
#pragma unroll
                for (int i = 0; i < 16; i += 4) {
                    const float4 f = lane < 8 ? *(const float4*)(sm.qkv + w * HD + 16 * lane + i)
                                              : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                    sq[i] = f.x * f.x, sq[i + 1] = f.y * f.y, sq[i + 2] = f.z * f.z, sq[i + 3] = f.w * f.w;
                }
                const float sum = lane_chain<16>(sq, 0.0f, HD / 16);
                const float inv = 1.0f / __builtin_sqrtf(sum / (float)HD + a.eps);
                x0 = x0 * (inv * nw0);
                x1 = x1 * (inv * nw1);
            }
            const float ac = x0 * cs, bs = x1 * sn, bc = x1 * cs, as = x0 * sn;
            x0 = ac - bs;
            x1 = bc + as;
        }
        if (w == 0) {
            // Granite: q times attention_multiplier * sqrt(hd) after the
            // rotary, then the attention's 1/sqrt(hd).
            if (a.q_scale != 1.0f) {
                x0 = x0 * a.q_scale;
                x1 = x1 * a.q_scale;
            }
            const float scale = 1.0f / __builtin_sqrtf((float)HD);
            x0 = x0 * scale;
            x1 = x1 * scale;
        } else {
            const int which = w - 1;
            const _Float16 c0 = (_Float16)x0, c1 = (_Float16)x1;
            if (b < kvh) {
                TRIT_GLOBAL uint16_t* cache =
                    gmem((uint16_t*)(which == 0 ? L.kcache : L.vcache)) + ((size_t)g * a.max_pos + pos) * HD;
                __hip_atomic_store(cache + lane, __builtin_bit_cast(uint16_t, c0), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(cache + lane + HD / 2, __builtin_bit_cast(uint16_t, c1), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            }
            sm.kvn[which][lane] = (float)c0;
            sm.kvn[which][lane + HD / 2] = (float)c1;
            if (which == 0) {
                sm.knew[lane] = __builtin_bit_cast(uint16_t, c0);
                sm.knew[lane + HD / 2] = __builtin_bit_cast(uint16_t, c1);
            }
        }
        // The norm's chain read the raw values of this head: rewrite them
        // only after every lane of the wave has read its values.
        __builtin_amdgcn_wave_barrier();
        if (w == 0) {
            sm.qkv[lane] = x0;
            sm.qkv[lane + HD / 2] = x1;
        }
    }
    __syncthreads();
    STAMP(7);

    // Scores: thread t key t, the fused chain over the dims in order (the
    // new key as cached: its f16 bits). q is read from LDS 16 values at a
    // time, the next 16 values' loads in flight during the current ones'
    // multiply-adds.
    if (t == pos) {
#pragma unroll
        for (int c = 0; c < HD / 8; ++c) kk[c] = *(const uint4*)&sm.knew[8 * c];
    }
    float score = -INFINITY;
    if (t < tk) {
        float acc = 0.0f;
        float4 qc[4], qn[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) qc[i] = *(const float4*)(sm.qkv + 4 * i);
#pragma unroll
        for (int part = 0; part < HD / 16; ++part) {
            if (part + 1 < HD / 16) {
#pragma unroll
                for (int i = 0; i < 4; ++i) qn[i] = *(const float4*)(sm.qkv + 16 * (part + 1) + 4 * i);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const uint4 kw = kk[2 * part + c];
                const uint32_t wd[4] = {kw.x, kw.y, kw.z, kw.w};
                const float q8[8] = {qc[2 * c].x, qc[2 * c].y, qc[2 * c].z, qc[2 * c].w,
                                     qc[2 * c + 1].x, qc[2 * c + 1].y, qc[2 * c + 1].z, qc[2 * c + 1].w};
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    acc = __builtin_fmaf(q8[u], f16_to_f32((uint16_t)(wd[u >> 1] >> (16 * (u & 1)))), acc);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < 4; ++i) qc[i] = qn[i];
        }
        score = acc;
    }
    // The cached values for p.V: wave w holds keys [64 w, 64 w + 64) before
    // pos, lane d the block's dim 64 h2 + d, read from the LDS rows by
    // transposing reads (ds_read_b64_tr_b16: in each 16-lane group, lane r
    // gives the address of 4 halves, and lane i receives half i % 4 of the
    // rows of lanes i / 4, 4 + i / 4, 8 + i / 4, 12 + i / 4): lane r of group
    // G points at key 4 j + r / 4, dims 16 G + 4 (r % 4) .., so lane i gets
    // dim i of keys 4 j .. 4 j + 3. The values past the last cached key are
    // zeroed before use.
    const int nkw = (pos + WAVE - 1) / WAVE;  // the waves that hold cached keys
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
    f16x4 vv[WAVE / 4];
    if (__builtin_amdgcn_readfirstlane(w) < nkw) {
        const int r = lane % 16, grp = lane / 16;
        typedef __attribute__((address_space(3))) s16x4 LdsS16x4;
#pragma unroll
        for (int j = 0; j < WAVE / 4; ++j) {
            const _Float16* row = &sm.vs[WAVE * w + 4 * j + r / 4][16 * grp + 4 * (r % 4)];
            vv[j] = __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((LdsS16x4*)row));
        }
    }
    const float m_w = wave_max(score);
    if (lane == 0) sm.wmax[w] = m_w;
    __syncthreads();
    float mx = sm.wmax[0];
#pragma unroll
    for (int q = 1; q < NW; ++q) mx = __builtin_fmaxf(mx, sm.wmax[q]);
    const float e = t < tk ? exp_trit(score - mx) : 0.0f;
    sm.probs[t] = e;
    __syncthreads();
    // Their sum in key order from 0, by every wave, then p_j = e_j *
    // (1/sum); the chain below reads -0 (adding nothing) past the cached
    // keys, and the new key's probability on its own.
    STAMP(8);
    const float p = e * (1.0f / chain_sum_spec(t, sm.probs, tk, a.norm_window, sm));
    STAMP(9);
    sm.probs[t] = t < pos ? p : -0.0f;
    if (t == pos) sm.ppos = p;
    // p.V in key order: lane d chains dim 64 h2 + d, wave w over keys
    // [64 w, 64 w + 64) from the sums wave w - 1 left in LDS (a block
    // barrier between turns), its values in registers and its 64
    // probabilities read (one broadcast read per four) before its turn; the
    // new key's value (position pos = tk - 1) comes last, from the qkv
    // product.
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    f32x4 pr[WAVE / 4];
    // The wave index as the compiler can see it: uniform over the wave.
    const int wu = __builtin_amdgcn_readfirstlane(w);
    if (wu < nkw) {
        const int nv = min(pos - WAVE * wu, WAVE);
#pragma unroll
        for (int i = 0; i < WAVE / 4; ++i) pr[i] = *(const f32x4*)(sm.probs + WAVE * w + 4 * i);
        if (nv < WAVE) {  // the last wave: the slots past the last key
            typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
#pragma unroll
            for (int j = 0; j < WAVE / 4; ++j) {
                u32x2 bits = __builtin_bit_cast(u32x2, vv[j]);
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int k = 4 * j + 2 * h;
                    bits[h] &= (k < nv ? 0xffffu : 0u) | (k + 1 < nv ? 0xffff0000u : 0u);
                }
                vv[j] = __builtin_bit_cast(f16x4, bits);
            }
        }
#pragma unroll
        for (int j = 0; j < WAVE / 4; ++j) asm volatile("" : "+v"(vv[j]));
#pragma unroll
        for (int i = 0; i < WAVE / 4; ++i) asm volatile("" : "+v"(pr[i]));
    }
    // The appended key and value are acknowledged (agent-scope stores write
    // through the L2) before the barriers below, so before this block's
    // attention outputs are put: whoever reads them in a later layer or step
    // waited, through the tags, for that put. Issued microseconds ago, they
    // have landed; the wait costs nothing.
    if (b < kvh && (w == 1 || w == 2)) __builtin_amdgcn_s_waitcnt(VMCNT0);
    if (nkw == 0) __syncthreads();  // no turns: still a barrier before the put
    // Every wave passes nkw barriers: the turns before its own, then its
    // turn's end and the rest.
    float acc = 0.0f;
    for (int cw = 0; cw < min(wu, nkw); ++cw) __syncthreads();
    if (wu < nkw) {
        if (wu > 0) acc = sm.carry[lane];
#pragma unroll
        for (int i = 0; i < WAVE; ++i) acc = __builtin_fmaf(pr[i / 4][i & 3], (float)vv[i / 4][i & 3], acc);
        if (wu + 1 < nkw) sm.carry[lane] = acc;
    }
    for (int cw = wu; cw < nkw; ++cw) __syncthreads();
    // Every load of the attention has arrived: the explicit wait costs
    // nothing here, and the compiler's later waits (for registers that its
    // analysis may see as loading) no longer wait for the put's store.
    __builtin_amdgcn_s_waitcnt(VMCNT0);
    // After a barrier (or in the wave that wrote it): the new key's term.
    if (wu == (nkw > 0 ? nkw - 1 : 0))
        put(a.ATT + (size_t)hq * HD + 64 * h2 + lane, __builtin_fmaf(sm.ppos, sm.kvn[1][64 * h2 + lane], acc), tag_out);
    STAMP(10);
    return true;
}

// The score of one key: the fused chain over the 128 dims in order of q
// (LDS, already times 1/sqrt(hd)) by the key's f16 bits widened inside each
// multiply-add; q is read 16 values at a time, the next 16 in flight.
__device__ __forceinline__ float score_of(const uint4 (&kk)[HD / 8], const float* q) {
    float acc = 0.0f;
    float4 qc[4], qn[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) qc[i] = *(const float4*)(q + 4 * i);
#pragma unroll
    for (int part = 0; part < HD / 16; ++part) {
        if (part + 1 < HD / 16) {
            // The next part's q loads wait for the chain's value so far: the
            // compiler can neither gather every load of q ahead of the chain
            // (128 registers in a loop over keys) nor sink the chain below them.
            int off = 16 * (part + 1);
            asm volatile("" : "+v"(off) : "v"(acc));
#pragma unroll
            for (int i = 0; i < 4; ++i) qn[i] = *(const float4*)(q + off + 4 * i);
        }
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const uint4 kw = kk[2 * part + c];
            const uint32_t wd[4] = {kw.x, kw.y, kw.z, kw.w};
            const float q8[8] = {qc[2 * c].x,     qc[2 * c].y,     qc[2 * c].z,     qc[2 * c].w,
                                 qc[2 * c + 1].x, qc[2 * c + 1].y, qc[2 * c + 1].z, qc[2 * c + 1].w};
#pragma unroll
            for (int u = 0; u < 8; ++u)
                acc = __builtin_fmaf(q8[u], f16_to_f32((uint16_t)(wd[u >> 1] >> (16 * (u & 1)))), acc);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) qc[i] = qn[i];
    }
    return acc;
}

// Attention in Trit's order on every block, for models with one key/value
// head per XCD (StepArgs::local_qkv): XCD x's 32 blocks take head g = x,
// BPH blocks a query head -- the block of rank r there query head
// g GROUP + r / BPH, slot s = r % BPH. Everything a head exchanges stays in
// that XCD's L2, and each block reads a slice of the cache instead of all
// of it (the attention of one block per head half was bound by what one CU
// can read: the keys and values of a head, 100-150 KB).
//   part a: the q/k/v rows (local exchange), Qwen3's q/k norms and the
//   rotary, the append; slot s scores keys [s kn, s kn + kn), kn =
//   ceil(tk / BPH), one thread a key, each score the fused chain over the
//   128 dims in order (as attention_exact), and puts them (local exchange,
//   tag_sc).
//   part b: every block of the head gathers the tk scores, takes their
//   maximum, e_j = exp(s_j - max), their sum in key order from 0, p_j =
//   e_j * (1/sum) -- the same bits in every block -- and chains p_j v_j
//   over the keys in order for its WD dims [WD s, WD s + WD), the new key
//   last; the outputs are the o product's input.
// The block's values load before the qkv rows arrive (thread j key j, 16
// bytes), and go to LDS as f32 by dim. Sessions of up to T positions.
template <int GROUP>
__device__ bool attention_wide_a(int t, const StepArgs& a, const LayerPtrs& L, int pos, uint32_t tag_in,
                                 uint32_t tag_sc, Smem& sm, unsigned long long deadline) {
    static_assert(WD == 8, "a block's value dims are one 16-byte load of f16");
    const int r = sm.xrank, g = sm.xcd;
    const int hq = g * GROUP + r / BPH, s = r % BPH;
    const int tk = pos + 1, kn = (tk + BPH - 1) / BPH, j0 = s * kn;
    const int heads = a.heads, kvh = a.kvh;
    const auto index = [hq, g, heads, kvh](int i) {
        if (i < HD) return hq * HD + i;
        if (i < 2 * HD) return (heads + g) * HD + (i - HD);
        return (heads + kvh + g) * HD + (i - 2 * HD);
    };
    const _Float16* K = L.kcache + (size_t)g * a.max_pos * HD;
    const _Float16* V = L.vcache + (size_t)g * a.max_pos * HD;
    const int w = t / WAVE, lane = t % WAVE;
    // The slot's keys: thread t (t < kn) key j0 + t, all 128 dims.
    uint4 kk[HD / 8];
#pragma unroll
    for (int i = 0; i < HD / 8; ++i) kk[i] = make_uint4(0, 0, 0, 0);
    const int jk = j0 + t;
    if (t < kn && jk < pos) {
#pragma unroll
        for (int i = 0; i < HD / 8; ++i) kk[i] = gload_u4(K + (size_t)jk * HD + 8 * i);
    }
    // The block's value dims of key t.
    uint4 vr = make_uint4(0, 0, 0, 0);
    if (t < pos) vr = gload_u4(V + (size_t)t * HD + WD * s);
    float nw0 = 1.0f, nw1 = 1.0f, sn = 0.0f, cs = 1.0f;
    if (w <= 1) {
        if (a.qk_norm) {
            const TRIT_GLOBAL float* nw = gmem(w == 0 ? L.q_norm : L.k_norm);
            nw0 = nw[lane];
            nw1 = nw[lane + HD / 2];
        }
        sn = gmem(a.rope_sin)[(size_t)pos * (HD / 2) + lane];
        cs = gmem(a.rope_cos)[(size_t)pos * (HD / 2) + lane];
    }
    // Polled by the last wave: its threads load a value only past 448
    // positions, and no key.
    STAMP(5);
    if (!gather<8>(t, a.QKV, 3 * HD, index, tag_in, sm.qkv, sm, deadline, a.st, NW - 1)) leave();
    STAMP(6);

    // Qwen3's per-head RMSNorm (Trit's serial sum of the squares) and the
    // rotary halves, wave 0 the q head and wave 1 the k head, lane i dims i
    // and i + 64 (src/models/parts/causal_lm.rs:428-446, src/layers.rs:
    // 136-144,303-334); v as cached. Block r = 0 of the XCD appends the new
    // key and value (agent scope: later steps read them on this XCD, the
    // per-kernel loop anywhere).
    if (w < 3) {
        float x0 = sm.qkv[w * HD + lane], x1 = sm.qkv[w * HD + lane + HD / 2];
        if (w <= 1) {
            if (a.qk_norm) {
                float sq[16];
#pragma unroll
                for (int i = 0; i < 16; i += 4) {
                    const float4 f = lane < 8 ? *(const float4*)(sm.qkv + w * HD + 16 * lane + i)
                                              : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                    sq[i] = f.x * f.x, sq[i + 1] = f.y * f.y, sq[i + 2] = f.z * f.z, sq[i + 3] = f.w * f.w;
                }
                const float sum = lane_chain<16>(sq, 0.0f, HD / 16);
                const float inv = 1.0f / __builtin_sqrtf(sum / (float)HD + a.eps);
                x0 = x0 * (inv * nw0);
                x1 = x1 * (inv * nw1);
            }
            const float ac = x0 * cs, bs = x1 * sn, bc = x1 * cs, as = x0 * sn;
            x0 = ac - bs;
            x1 = bc + as;
        }
        if (w == 0) {
            if (a.q_scale != 1.0f) {
                x0 = x0 * a.q_scale;
                x1 = x1 * a.q_scale;
            }
            const float scale = 1.0f / __builtin_sqrtf((float)HD);
            x0 = x0 * scale;
            x1 = x1 * scale;
        } else {
            const int which = w - 1;
            const _Float16 c0 = (_Float16)x0, c1 = (_Float16)x1;
            if (r == 0) {
                TRIT_GLOBAL uint16_t* cache =
                    gmem((uint16_t*)(which == 0 ? L.kcache : L.vcache)) + ((size_t)g * a.max_pos + pos) * HD;
                __hip_atomic_store(cache + lane, __builtin_bit_cast(uint16_t, c0), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(cache + lane + HD / 2, __builtin_bit_cast(uint16_t, c1), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            }
            sm.kvn[which][lane] = (float)c0;
            sm.kvn[which][lane + HD / 2] = (float)c1;
            if (which == 0) {
                sm.knew[lane] = __builtin_bit_cast(uint16_t, c0);
                sm.knew[lane + HD / 2] = __builtin_bit_cast(uint16_t, c1);
            }
        }
        // The norm's chain read the raw values of this head: rewrite them
        // only after every lane of the wave has read its values.
        __builtin_amdgcn_wave_barrier();
        if (w == 0) {
            sm.qkv[lane] = x0;
            sm.qkv[lane + HD / 2] = x1;
        }
    }
    __syncthreads();
    // The values by dim (f16 bits): the cached ones, the new key's (as
    // cached), zeros past it.
    {
        const uint32_t wv[4] = {vr.x, vr.y, vr.z, vr.w};
#pragma unroll
        for (int d = 0; d < WD; ++d) {
            const uint16_t cached = (uint16_t)(wv[d / 2] >> (16 * (d & 1)));
            sm.vth[d][t] = t < pos ? cached : t == pos ? f32_to_f16(sm.kvn[1][WD * s + d]) : (uint16_t)0;
        }
    }
    // The appended key and value are acknowledged before the block's
    // attention outputs are put (after barriers in part b): whoever reads
    // them later waited, through the tags, for that put.
    if (r == 0 && (w == 1 || w == 2)) __builtin_amdgcn_s_waitcnt(VMCNT0);
    STAMP(7);
    // The slot's scores (the new key as cached: its f16 bits).
    if (t < kn && jk < tk) {
        if (jk == pos) {
#pragma unroll
            for (int c = 0; c < HD / 8; ++c) kk[c] = *(const uint4*)&sm.knew[8 * c];
        }
        put_local(a.SC + (size_t)hq * T + jk, score_of(kk, sm.qkv), tag_sc);
    }
    STAMP(25);
    return true;
}

template <int GROUP>
__device__ bool attention_wide_b(int t, const StepArgs& a, int pos, uint32_t tag_sc, uint32_t tag_out, Smem& sm,
                                 unsigned long long deadline, int p0) {
    const int r = sm.xrank, g = sm.xcd;
    const int hq = g * GROUP + r / BPH, s = r % BPH;
    const int tk = pos + 1;
    const int w = t / WAVE, lane = t % WAVE;
    // The head's scores, from its BPH blocks on this XCD.
    STAMP(26);
    if (!gather<T / (4 * WAVE)>(t, a.SC + (size_t)hq * T, tk, Linear(), tag_sc, sm.probs, sm, deadline, a.st, p0))
        leave();
    STAMP(27);
    const float score = t < tk ? sm.probs[t] : -INFINITY;
    const float m_w = wave_max(score);
    if (lane == 0) sm.wmax[w] = m_w;
    __syncthreads();
    float mx = sm.wmax[0];
#pragma unroll
    for (int q = 1; q < NW; ++q) mx = __builtin_fmaxf(mx, sm.wmax[q]);
    const float e = t < tk ? exp_trit(score - mx) : 0.0f;
    sm.probs[t] = e;
    __syncthreads();
    STAMP(8);
    // Their sum in key order from 0, by every wave; p_j = e_j * (1/sum),
    // -0 past the keys (adding nothing to the chains below).
    const float p = e * (1.0f / chain_sum_spec(t, sm.probs, tk, a.norm_window, sm));
    STAMP(9);
    sm.probs[t] = t < tk ? p : -0.0f;
    __syncthreads();
    // p.V in key order: wave w takes keys [64 w, 64 w + 64), lane d its
    // dim's values (lane l: dim l % WD; lanes from WD on are not used) and
    // their probabilities (every lane alike), read from LDS PD fours ahead
    // of the multiply-adds; the waves chain in turn, the carry passing
    // through LDS, the new key last.
    const int nkw = (tk + WAVE - 1) / WAVE;  // the waves that hold keys
    const int wu = __builtin_amdgcn_readfirstlane(w);
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
    constexpr int PD = 6;
    f32x4 pq[PD];
    f16x4 vq[PD];
    const float* pw = sm.probs + WAVE * wu;
    const uint16_t* vw = sm.vth[lane % WD] + WAVE * wu;
    if (wu < nkw) {
#pragma unroll
        for (int i = 0; i < PD; ++i) {
            pq[i] = *(const f32x4*)(pw + 4 * i);
            vq[i] = *(const f16x4*)(vw + 4 * i);
        }
    }
    float acc = 0.0f;
    for (int cw = 0; cw < min(wu, nkw); ++cw) __syncthreads();
    if (wu < nkw) {
        if (wu > 0) acc = sm.carry[lane];
#pragma unroll
        for (int i = 0; i < WAVE / 4; ++i) {
            const f32x4 pc = pq[i % PD];
            const f16x4 vc = vq[i % PD];
            if (i + PD < WAVE / 4) {
                // The reads issue after the chain so far: PD of each in
                // flight, not all of them hoisted to the turn's start.
                int off = 4 * (i + PD);
                asm volatile("" : "+v"(off) : "v"(acc));
                pq[i % PD] = *(const f32x4*)(pw + off);
                vq[i % PD] = *(const f16x4*)(vw + off);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) acc = __builtin_fmaf(pc[u], (float)vc[u], acc);
        }
        if (wu + 1 < nkw) sm.carry[lane] = acc;
    }
    for (int cw = wu; cw < nkw; ++cw) __syncthreads();
    if (wu == nkw - 1 && lane < WD) put(a.ATT + (size_t)hq * HD + WD * s + lane, acc, tag_out);
    STAMP_BY(10, WAVE * (nkw - 1));
    return true;
}

// attention_exact with Trit's own f32 keys and values (TRIT_HIP_EXACT,
// TRIT_HIP_KV_F32): the same blocks, phases and orders, the keys and values
// as f32 (each appended value as computed, no f16 rounding). Thread t scores
// key t in two halves of 64 dims: the first half loads while the qkv rows
// arrive, the second right after them, under the q/k norms. For p.V, wave w
// loads the values of keys [64 w, 64 w + 64), lane d its dim 64 h2 + d, from
// the cache (its lines came to this XCD's L2 with the layer's touches) into
// registers while the softmax sum runs, and chains them in its turn as
// attention_exact does. Sessions of up to T positions.
template <int GROUP, int DPB>
__device__ bool attention_exact32(int t, const StepArgs& a, const LayerPtrs& L, int pos, uint32_t tag_in,
                                  uint32_t tag_out, Smem& sm, unsigned long long deadline) {
    const int b = blockIdx.x, kvh = a.kvh;
    if (b >= 2 * a.heads) {  // uniform over the block
        __builtin_amdgcn_s_waitcnt(VMCNT0);
        return true;
    }
    const int g = b % kvh, hq = g * GROUP + (b / kvh) % GROUP, h2 = b / (kvh * GROUP);
    const int tk = pos + 1;  // at most T (the host's plan)
    const int heads = a.heads;
    const auto index = [hq, g, heads, kvh](int i) {
        if (i < HD) return hq * HD + i;
        if (i < 2 * HD) return (heads + g) * HD + (i - HD);
        return (heads + kvh + g) * HD + (i - 2 * HD);
    };
    const float* K = (const float*)L.kcache + (size_t)g * a.max_pos * HD;
    const float* V = (const float*)L.vcache + (size_t)g * a.max_pos * HD;
    const int w = t / WAVE, lane = t % WAVE;
    // Key t's first 64 dims (16 units of 4), and one word of each line of its
    // second half: those lines come to the caches now.
    uint4 kk[HD / 8];
#pragma unroll
    for (int i = 0; i < HD / 8; ++i) kk[i] = make_uint4(0, 0, 0, 0);
    uint32_t touch0 = 0, touch1 = 0;
    if (t < pos) {
#pragma unroll
        for (int i = 0; i < HD / 8; ++i) kk[i] = gload_u4(K + (size_t)t * HD + 4 * i);
        touch0 = *gmem((const uint32_t*)(K + (size_t)t * HD + HD / 2));
        touch1 = *gmem((const uint32_t*)(K + (size_t)t * HD + 3 * HD / 4));
    }
    float nw0 = 1.0f, nw1 = 1.0f, sn = 0.0f, cs = 1.0f;
    if (w <= 1) {
        if (a.qk_norm) {
            const TRIT_GLOBAL float* nw = gmem(w == 0 ? L.q_norm : L.k_norm);
            nw0 = nw[lane];
            nw1 = nw[lane + HD / 2];
        }
        sn = gmem(a.rope_sin)[(size_t)pos * (HD / 2) + lane];
        cs = gmem(a.rope_cos)[(size_t)pos * (HD / 2) + lane];
    }
    const int p0 = pos <= T - WAVE ? NW - 1 : NW - a.rq / 4 - 1;
    STAMP(5);
    if (!gather<8>(t, a.QKV, 3 * HD, index, tag_in, sm.qkv, sm, deadline, a.st, p0)) leave();
    STAMP(6);
    asm volatile("" ::"v"(touch0), "v"(touch1));

    // Qwen3's per-head RMSNorm and the rotary halves, as attention_exact;
    // the new key and value appended as f32.
    if (w < 3) {
        float x0 = sm.qkv[w * HD + lane], x1 = sm.qkv[w * HD + lane + HD / 2];
        if (w <= 1) {
            if (a.qk_norm) {
                float sq[16];
#pragma unroll
                for (int i = 0; i < 16; i += 4) {
                    const float4 f = lane < 8 ? *(const float4*)(sm.qkv + w * HD + 16 * lane + i)
                                              : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                    sq[i] = f.x * f.x, sq[i + 1] = f.y * f.y, sq[i + 2] = f.z * f.z, sq[i + 3] = f.w * f.w;
                }
                const float sum = lane_chain<16>(sq, 0.0f, HD / 16);
                const float inv = 1.0f / __builtin_sqrtf(sum / (float)HD + a.eps);
                x0 = x0 * (inv * nw0);
                x1 = x1 * (inv * nw1);
            }
            const float ac = x0 * cs, bs = x1 * sn, bc = x1 * cs, as = x0 * sn;
            x0 = ac - bs;
            x1 = bc + as;
        }
        if (w == 0) {
            if (a.q_scale != 1.0f) {
                x0 = x0 * a.q_scale;
                x1 = x1 * a.q_scale;
            }
            const float scale = 1.0f / __builtin_sqrtf((float)HD);
            x0 = x0 * scale;
            x1 = x1 * scale;
        } else {
            const int which = w - 1;
            if (b < kvh) {
                TRIT_GLOBAL uint32_t* cache =
                    gmem((uint32_t*)(which == 0 ? L.kcache : L.vcache)) + ((size_t)g * a.max_pos + pos) * HD;
                __hip_atomic_store(cache + lane, __float_as_uint(x0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(cache + lane + HD / 2, __float_as_uint(x1), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            }
            sm.kvn[which][lane] = x0;
            sm.kvn[which][lane + HD / 2] = x1;
        }
        __builtin_amdgcn_wave_barrier();
        if (w == 0) {
            sm.qkv[lane] = x0;
            sm.qkv[lane + HD / 2] = x1;
        }
    }
    __syncthreads();
    STAMP(7);
    uint4 kh[HD / 8];
#pragma unroll
    for (int i = 0; i < HD / 8; ++i) kh[i] = make_uint4(0, 0, 0, 0);
    if (t < pos) {
#pragma unroll
        for (int i = 0; i < HD / 8; ++i) kh[i] = gload_u4(K + (size_t)t * HD + HD / 2 + 4 * i);
    }

    // Scores: thread t key t, the fused chain over the dims in order (the
    // new key from LDS).
    if (t == pos) {
#pragma unroll
        for (int c = 0; c < HD / 8; ++c) {
            kk[c] = *(const uint4*)&sm.kvn[0][4 * c];
            kh[c] = *(const uint4*)&sm.kvn[0][HD / 2 + 4 * c];
        }
    }
    float score = -INFINITY;
    if (t < tk) {
        float acc = 0.0f;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
#pragma unroll
            for (int part = 0; part < HD / 32; ++part) {
                // q dims 64 half + 16 part .. + 15, in four loads
                const int q0 = HD / 2 * half + 16 * part;
                float4 qc[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) qc[i] = *(const float4*)(sm.qkv + q0 + 4 * i);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint4 kw = half == 0 ? kk[4 * part + i] : kh[4 * part + i];
                    acc = __builtin_fmaf(qc[i].x, __uint_as_float(kw.x), acc);
                    acc = __builtin_fmaf(qc[i].y, __uint_as_float(kw.y), acc);
                    acc = __builtin_fmaf(qc[i].z, __uint_as_float(kw.z), acc);
                    acc = __builtin_fmaf(qc[i].w, __uint_as_float(kw.w), acc);
                }
            }
        }
        score = acc;
    }
    // The values for p.V: wave w keys [64 w, 64 w + 64) before pos, lane d
    // the block's dim 64 h2 + d (256 contiguous bytes a key across the
    // wave), zero past the last cached key.
    const int nkw = (pos + WAVE - 1) / WAVE;
    const int wu = __builtin_amdgcn_readfirstlane(w);
    const float m_w = wave_max(score);
    if (lane == 0) sm.wmax[w] = m_w;
    float vf[WAVE];
    if (wu < nkw) {
        const float* vcol = V + 64 * h2 + lane;
#pragma unroll
        for (int i = 0; i < WAVE; ++i) {
            const int j = WAVE * wu + i;
            vf[i] = j < pos ? *gmem(vcol + (size_t)j * HD) : 0.0f;
        }
    }
    __syncthreads();
    float mx = sm.wmax[0];
#pragma unroll
    for (int q = 1; q < NW; ++q) mx = __builtin_fmaxf(mx, sm.wmax[q]);
    const float e = t < tk ? exp_trit(score - mx) : 0.0f;
    sm.probs[t] = e;
    __syncthreads();
    STAMP(8);
    const float p = e * (1.0f / chain_sum_spec(t, sm.probs, tk, a.norm_window, sm));
    STAMP(9);
    sm.probs[t] = t < pos ? p : -0.0f;
    if (t == pos) sm.ppos = p;
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    f32x4 pr[WAVE / 4];
    if (wu < nkw) {
#pragma unroll
        for (int i = 0; i < WAVE / 4; ++i) pr[i] = *(const f32x4*)(sm.probs + WAVE * w + 4 * i);
#pragma unroll
        for (int i = 0; i < WAVE; ++i) asm volatile("" : "+v"(vf[i]));
#pragma unroll
        for (int i = 0; i < WAVE / 4; ++i) asm volatile("" : "+v"(pr[i]));
    }
    if (b < kvh && (w == 1 || w == 2)) __builtin_amdgcn_s_waitcnt(VMCNT0);
    if (nkw == 0) __syncthreads();
    float acc = 0.0f;
    for (int cw = 0; cw < min(wu, nkw); ++cw) __syncthreads();
    if (wu < nkw) {
        if (wu > 0) acc = sm.carry[lane];
#pragma unroll
        for (int i = 0; i < WAVE; ++i) acc = __builtin_fmaf(pr[i / 4][i & 3], vf[i], acc);
        if (wu + 1 < nkw) sm.carry[lane] = acc;
    }
    for (int cw = wu; cw < nkw; ++cw) __syncthreads();
    __builtin_amdgcn_s_waitcnt(VMCNT0);
    if (wu == (nkw > 0 ? nkw - 1 : 0))
        put(a.ATT + (size_t)hq * HD + 64 * h2 + lane, __builtin_fmaf(sm.ppos, sm.kvn[1][64 * h2 + lane], acc), tag_out);
    STAMP(10);
    return true;
}

// attention_exact for sessions of up to MAXT positions: the same orders and
// bits, over the keys in rounds of T. Scores: round r, thread t scores key
// r T + t into sm.probs (the next round's keys load meanwhile); the maximum
// over all of them, e_j = exp(s_j - max), their sum in key order from 0
// (the candidate-start segments over all tk values), p_j = e_j * (1/sum).
// p.V in stages of T cached keys: a stage's values (the block's 64 dims)
// sit in LDS row-major, the waves chain their 64 keys in turn as in
// attention_exact, the carry passes from the last wave of a stage to the
// first of the next, and the next stage's values load into registers
// during the turns. The new key's value comes last, from the qkv product.
template <int GROUP, int DPB>
__device__ bool attention_exact_long(int t, const StepArgs& a, const LayerPtrs& L, int pos, uint32_t tag_in,
                                     uint32_t tag_out, Smem& sm, unsigned long long deadline) {
    const int b = blockIdx.x, kvh = a.kvh;
    if (b >= 2 * a.heads) {  // uniform over the block
        __builtin_amdgcn_s_waitcnt(VMCNT0);
        return true;
    }
    const int g = b % kvh, hq = g * GROUP + (b / kvh) % GROUP, h2 = b / (kvh * GROUP);
    const int tk = pos + 1;  // at most MAXT (the host's plan)
    const int heads = a.heads;
    const auto index = [hq, g, heads, kvh](int i) {
        if (i < HD) return hq * HD + i;
        if (i < 2 * HD) return (heads + g) * HD + (i - HD);
        return (heads + kvh + g) * HD + (i - 2 * HD);
    };
    const _Float16* K = L.kcache + (size_t)g * a.max_pos * HD;
    const _Float16* V = L.vcache + (size_t)g * a.max_pos * HD;
    const int w = t / WAVE, lane = t % WAVE;
    const int wu = __builtin_amdgcn_readfirstlane(w);
    // Round 0's keys (the first half now, the second after the hand-over)
    // and stage 0's values (threads below VT) load while the qkv rows arrive.
    constexpr int VT = T - WAVE, VC = (8 * T + VT - 1) / VT, SC = 8 * T / T;  // SC: value chunks a thread, later stages
    const int n0 = min(pos, T);  // cached keys of round / stage 0
    uint4 kk[HD / 8];
#pragma unroll
    for (int i = 0; i < HD / 8; ++i) kk[i] = make_uint4(0, 0, 0, 0);
    uint32_t touch = 0;
    if (t < n0) {
#pragma unroll
        for (int i = 0; i < HD / 16; ++i) kk[i] = gload_u4(K + (size_t)t * HD + 8 * i);
        touch = *gmem((const uint32_t*)(K + (size_t)t * HD + HD / 2));
    }
    uint4 vr[VC];
#pragma unroll
    for (int i = 0; i < VC; ++i) {
        vr[i] = make_uint4(0, 0, 0, 0);
        const int c = t + VT * i;
        if (t < VT && c < 8 * n0) vr[i] = gload_u4(V + (size_t)(c / 8) * HD + 64 * h2 + 8 * (c % 8));
    }
    float nw0 = 1.0f, nw1 = 1.0f, sn = 0.0f, cs = 1.0f;
    if (w <= 1) {
        if (a.qk_norm) {
            const TRIT_GLOBAL float* nw = gmem(w == 0 ? L.q_norm : L.k_norm);
            nw0 = nw[lane];
            nw1 = nw[lane + HD / 2];
        }
        sn = gmem(a.rope_sin)[(size_t)pos * (HD / 2) + lane];
        cs = gmem(a.rope_cos)[(size_t)pos * (HD / 2) + lane];
    }
    // The last wave polls: it loads no value, and no key while round 0
    // leaves it none.
    const int p0 = n0 <= VT ? NW - 1 : NW - a.rq / 4 - 1;
    STAMP(5);
    if (!gather<8>(t, a.QKV, 3 * HD, index, tag_in, sm.qkv, sm, deadline, a.st, p0)) leave();
    STAMP(6);
    asm volatile("" ::"v"(touch));
#pragma unroll
    for (int i = 0; i < VC; ++i) {
        const int c = t + VT * i;
        if (t < VT && c < 8 * n0) *(uint4*)&sm.vs[c / 8][8 * (c % 8)] = vr[i];
    }
    if (t < n0) {
#pragma unroll
        for (int i = HD / 16; i < HD / 8; ++i) kk[i] = gload_u4(K + (size_t)t * HD + 8 * i);
    }
    // q/k norm, rotary, append: as attention_exact.
    if (w < 3) {
        float x0 = sm.qkv[w * HD + lane], x1 = sm.qkv[w * HD + lane + HD / 2];
        if (w <= 1) {
            if (a.qk_norm) {
                float sq[16];
#pragma unroll
                for (int i = 0; i < 16; i += 4) {
                    const float4 f = lane < 8 ? *(const float4*)(sm.qkv + w * HD + 16 * lane + i)
                                              : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                    sq[i] = f.x * f.x, sq[i + 1] = f.y * f.y, sq[i + 2] = f.z * f.z, sq[i + 3] = f.w * f.w;
                }
                const float sum = lane_chain<16>(sq, 0.0f, HD / 16);
                const float inv = 1.0f / __builtin_sqrtf(sum / (float)HD + a.eps);
                x0 = x0 * (inv * nw0);
                x1 = x1 * (inv * nw1);
            }
            const float ac = x0 * cs, bs = x1 * sn, bc = x1 * cs, as = x0 * sn;
            x0 = ac - bs;
            x1 = bc + as;
        }
        if (w == 0) {
            if (a.q_scale != 1.0f) {
                x0 = x0 * a.q_scale;
                x1 = x1 * a.q_scale;
            }
            const float scale = 1.0f / __builtin_sqrtf((float)HD);
            x0 = x0 * scale;
            x1 = x1 * scale;
        } else {
            const int which = w - 1;
            const _Float16 c0 = (_Float16)x0, c1 = (_Float16)x1;
            if (b < kvh) {
                TRIT_GLOBAL uint16_t* cache =
                    gmem((uint16_t*)(which == 0 ? L.kcache : L.vcache)) + ((size_t)g * a.max_pos + pos) * HD;
                __hip_atomic_store(cache + lane, __builtin_bit_cast(uint16_t, c0), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(cache + lane + HD / 2, __builtin_bit_cast(uint16_t, c1), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            }
            sm.kvn[which][lane] = (float)c0;
            sm.kvn[which][lane + HD / 2] = (float)c1;
            if (which == 0) {
                sm.knew[lane] = __builtin_bit_cast(uint16_t, c0);
                sm.knew[lane + HD / 2] = __builtin_bit_cast(uint16_t, c1);
            }
        }
        __builtin_amdgcn_wave_barrier();
        if (w == 0) {
            sm.qkv[lane] = x0;
            sm.qkv[lane + HD / 2] = x1;
        }
    }
    __syncthreads();
    STAMP(7);

    // Scores by rounds; each thread keeps the maximum of its keys.
    const int rounds = (tk + T - 1) / T;
    float mx = -INFINITY;
    for (int r = 0; r < rounds; ++r) {
        const int j = r * T + t;
        // The first half of the next round's key loads during this round's
        // chain; its second half after it.
        uint4 kn[HD / 16];
        const bool more = r + 1 < rounds;  // uniform
        const int jn = j + T;
        if (more) {
#pragma unroll
            for (int i = 0; i < HD / 16; ++i)
                kn[i] = jn < pos ? gload_u4(K + (size_t)jn * HD + 8 * i) : make_uint4(0, 0, 0, 0);
        }
        if (j == pos) {
#pragma unroll
            for (int c = 0; c < HD / 8; ++c) kk[c] = *(const uint4*)&sm.knew[8 * c];
        }
        const float score = j < tk ? score_of(kk, sm.qkv) : -INFINITY;
        sm.probs[j] = score;
        mx = __builtin_fmaxf(mx, score);
        if (more) {
#pragma unroll
            for (int i = 0; i < HD / 16; ++i) kk[i] = kn[i];
#pragma unroll
            for (int i = HD / 16; i < HD / 8; ++i)
                kk[i] = jn < pos ? gload_u4(K + (size_t)jn * HD + 8 * i) : make_uint4(0, 0, 0, 0);
        }
    }
    const float m_w = wave_max(mx);
    if (lane == 0) sm.wmax[w] = m_w;
    __syncthreads();
    mx = sm.wmax[0];
#pragma unroll
    for (int q = 1; q < NW; ++q) mx = __builtin_fmaxf(mx, sm.wmax[q]);
    // Each thread rewrites its own keys: e_j, zero past the keys (the sum's
    // segments read up to rounds T values).
    for (int r = 0; r < rounds; ++r) {
        const int j = r * T + t;
        sm.probs[j] = j < tk ? exp_trit(sm.probs[j] - mx) : 0.0f;
    }
    __syncthreads();
    STAMP(8);
    const float inv = 1.0f / chain_sum_spec(t, sm.probs, tk, a.norm_window, sm);
    STAMP(9);
    __syncthreads();  // every wave has read the sum's values
    for (int r = 0; r < rounds; ++r) {
        const int j = r * T + t;
        const float p = sm.probs[j] * inv;
        sm.probs[j] = j < pos ? p : -0.0f;
        if (j == pos) sm.ppos = p;
    }
    __syncthreads();

    // p.V by stages of T cached keys.
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    typedef __attribute__((address_space(3))) s16x4 LdsS16x4;
    const int stages = (pos + T - 1) / T;
    if (b < kvh && (w == 1 || w == 2)) __builtin_amdgcn_s_waitcnt(VMCNT0);
    float acc = 0.0f;
    int last_w = 0;  // the wave that chains the last cached key
    for (int s = 0; s < stages; ++s) {
        const int ns = min(pos - s * T, T);  // keys of this stage
        const int nkw = (ns + WAVE - 1) / WAVE;
        const bool more = s + 1 < stages;  // uniform
        // The next stage's values, into registers during this stage's turns.
        uint4 nv[SC];
        if (more) {
            const int nn = min(pos - (s + 1) * T, T);
#pragma unroll
            for (int i = 0; i < SC; ++i) {
                const int c = t + T * i;
                nv[i] = c < 8 * nn ? gload_u4(V + (size_t)((s + 1) * T + c / 8) * HD + 64 * h2 + 8 * (c % 8))
                                   : make_uint4(0, 0, 0, 0);
            }
        }
        f16x4 vv[WAVE / 4];
        f32x4 pr[WAVE / 4];
        if (wu < nkw) {
            const int r = lane % 16, grp = lane / 16;
#pragma unroll
            for (int j = 0; j < WAVE / 4; ++j) {
                const _Float16* row = &sm.vs[WAVE * w + 4 * j + r / 4][16 * grp + 4 * (r % 4)];
                vv[j] = __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((LdsS16x4*)row));
            }
            const int nvk = min(ns - WAVE * wu, WAVE);
#pragma unroll
            for (int i = 0; i < WAVE / 4; ++i) pr[i] = *(const f32x4*)(sm.probs + s * T + WAVE * w + 4 * i);
            if (nvk < WAVE) {  // the stage's last wave: the slots past its last key
#pragma unroll
                for (int j = 0; j < WAVE / 4; ++j) {
                    u32x2 bits = __builtin_bit_cast(u32x2, vv[j]);
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const int k = 4 * j + 2 * h;
                        bits[h] &= (k < nvk ? 0xffffu : 0u) | (k + 1 < nvk ? 0xffff0000u : 0u);
                    }
                    vv[j] = __builtin_bit_cast(f16x4, bits);
                }
            }
#pragma unroll
            for (int j = 0; j < WAVE / 4; ++j) asm volatile("" : "+v"(vv[j]));
#pragma unroll
            for (int i = 0; i < WAVE / 4; ++i) asm volatile("" : "+v"(pr[i]));
        }
        for (int cw = 0; cw < min(wu, nkw); ++cw) __syncthreads();
        if (wu < nkw) {
            if (s > 0 || wu > 0) acc = sm.carry[lane];
#pragma unroll
            for (int i = 0; i < WAVE; ++i) acc = __builtin_fmaf(pr[i / 4][i & 3], (float)vv[i / 4][i & 3], acc);
            if (wu + 1 < nkw || more) sm.carry[lane] = acc;
        }
        for (int cw = wu; cw < nkw; ++cw) __syncthreads();
        last_w = nkw - 1;
        if (more) {
            // Every wave has read this stage's values: the next stage's go in.
#pragma unroll
            for (int i = 0; i < SC; ++i) {
                const int c = t + T * i;
                *(uint4*)&sm.vs[c / 8][8 * (c % 8)] = nv[i];
            }
            __syncthreads();
        }
    }
    if (stages == 0) __syncthreads();  // no turns: still a barrier before the put
    __builtin_amdgcn_s_waitcnt(VMCNT0);
    if (wu == last_w)
        put(a.ATT + (size_t)hq * HD + 64 * h2 + lane, __builtin_fmaf(sm.ppos, sm.kvn[1][64 * h2 + lane], acc), tag_out);
    STAMP(10);
    return true;
}

__device__ __forceinline__ void better(float& bv, int& bi, float v, int i) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

// The best (value, index) pair of a wave, in every lane: shuffle tree.
template <int CTRL>
__device__ __forceinline__ void better_dpp(float& bv, int& bi) {
    const float v = dpp<CTRL>(bv);
    const int i = dpp<CTRL>(bi);
    better(bv, bi, v, i);
}

__device__ __forceinline__ void best_of_wave(float& bv, int& bi) {
    better_dpp<DPP_XOR1>(bv, bi);
    better_dpp<DPP_XOR2>(bv, bi);
    better_dpp<DPP_HALF_MIRROR>(bv, bi);
    better_dpp<DPP_MIRROR>(bv, bi);
    // The four rows' results, read before any is overwritten.
    float v[4];
    int i[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        v[r] = lane_f(bv, 16 * r);
        i[r] = __builtin_amdgcn_readlane(bi, 16 * r);
    }
    bv = v[0];
    bi = i[0];
#pragma unroll
    for (int r = 1; r < 4; ++r) better(bv, bi, v[r], i[r]);
}

// LONG: Trit-order sessions of more than T positions (attention_exact_long).
// KV32: Trit's own f32 keys and values (attention_exact32; T positions).
template <int JD, int JO, int JF, int GROUP, int DPB, bool EXACT, int WK, int HK, bool LONG = false,
          bool KV32 = false>
__global__ __launch_bounds__(T, 1) void step_kernel(StepArgs a, int step0, int pos0, uint32_t seq0, int nsteps) {
    static_assert(!KV32 || (EXACT && !LONG && DPB > 0), "f32 caches: the one-pass Trit-order attention");
    __shared__ Smem sm;
    State* st = a.st;
    if (st->done) return;
    const int b = blockIdx.x;
    if (a.local_qkv) {
        // The block's XCD and its rank among the XCD's blocks (each XCD
        // holds gridDim / NX of them: one a CU). Were it otherwise, the
        // launch fails here (the others' waits reach their deadlines)
        // rather than run with a role taken twice.
        if (threadIdx.x == 0) {
            const int x = xcc_id();
            sm.xcd = x;
            sm.xrank = x < NX ? (int)atomicAdd(a.xcd_count + x, 1u) : INT_MAX;
        }
        __syncthreads();
        if (__builtin_amdgcn_readfirstlane(sm.xrank) >= (int)gridDim.x / NX) {
            if (threadIdx.x == 0) atomicOr(&st->err, 2);
            leave();
        }
    }
    if (threadIdx.x == 0) sm.abort = 0;
    for (int i = threadIdx.x; i < a.n_layers * (int)(sizeof(LayerPtrs) / 8); i += T)
        ((uint64_t*)sm.layers)[i] = gmem((const uint64_t*)a.layers)[i];
    __syncthreads();

    // Waves by product, four rows a wave: gate_up [0, nu), o [nu, nu + no),
    // down [nu, nu + DR nd), qkv [NW - nqw, NW). Each product's rows load
    // during the hand-over just before it (o's during the attention
    // outputs', gate_up's during x's after o, down's during h's, the next
    // layer's qkv during x's after down); a wave holds one product's rows
    // at a time, so all share one register set. Where those
    // ranges do not fit in the waves (wide MLPs), gate_up moves to the last
    // nu waves and o / down to the first: gate_up's rows then load during
    // the attention in waves that also poll for its outputs (every wave has
    // loads in flight there), and no two sets live at once in one wave.
    // A down product of more than 16 chunks a lane (ffn > 4096) runs in DR =
    // 2 rounds of JF / 2 chunks, held by two sets of nd waves and chained
    // one after the other (the first round's totals pass through LDS).
    constexpr int DR = JF > 16 ? 2 : 1, JFR = JF / DR;
    static_assert(JF % DR == 0, "down rounds of whole chunks");
    const int nu = a.rgu / 4, no = a.ro / 4, nd = a.rd / 4, nqw = a.rq / 4;
    const bool packed = nu + cmax(no, DR * nd) + nqw <= NW;
    const int u0 = packed ? 0 : NW - nu, od0 = packed ? nu : 0;
    // The one row register set (see Rows); the first layer's qkv rows
    // stream in during the choice.
    constexpr int RN = cmax(cmax(2 * JD, JO), JFR);
    constexpr int RS = RN;
    // Words a lane of a gather takes for a product input of up to
    // max(JF, 12) chunks.
    constexpr int MWK = cmax(JF, 12) * 256 / T;
    const Linear lin;

    // Token steps: step it forwards the token chosen from step it - 1's
    // candidates (exchange words) -- the first from the candidates the
    // previous launch or the prompt's logits left in a.cand.
    for (int it = 0; it < nsteps; ++it) {
    const int step = step0 + it, pos = pos0 + it;
    const uint32_t tag0 = (seq0 + (uint32_t)it) << 8;
    const unsigned long long deadline = a.ticks ? wall_clock64() + a.ticks : 0ull;
    // The thread index, made opaque to the optimizer at the top of the step,
    // of each layer and of the head: what derives from it (the wave's
    // product, a lane's rows) is computed within that part, rather than
    // hoisted out of the loops and held in registers through the others
    // (the head needs them).
    int t, w, lane, rowq, rowo, rowgu, rowd, dround;
    bool aq, agu, ao, ad;
    // The RMSNorm factor of sm.xres. The exact instances with registers to
    // spare take it in every thread from Trit's serial sum, which every wave
    // joins and returns itself: no barrier before the quantizer, which
    // touches none of the norm's LDS. The others pass it through LDS
    // (sm.inv, read by the quantizer: INV_LDS).
    constexpr bool INV_LDS = !EXACT || KV32 || LONG;
    auto fresh = [&] {
        t = threadIdx.x;
        asm volatile("" : "+v"(t));
        t &= T - 1;  // its range, for the arithmetic derived from it
        w = t / WAVE;
        lane = t % WAVE;
        aq = w >= NW - nqw;
        agu = w >= u0 && w < u0 + nu;
        ao = w >= od0 && w < od0 + no;
        ad = w >= od0 && w < od0 + DR * nd;
        dround = ad ? (w - od0) / nd : 0;
        rowq = b * a.rq + 4 * (w - (NW - nqw)) + (lane >> 4);
        rowo = b * a.ro + 4 * (w - od0) + (lane >> 4);
        rowgu = b * a.rgu + 4 * (w - u0) + (lane >> 4);
        rowd = b * a.rd + 4 * ((w - od0) % nd) + (lane >> 4);
    };
    fresh();
    // The qkv row a lane of the qkv waves takes: row rowq, or with the
    // XCD-local exchange, the block of rank r on XCD x makes rows
    // [r rq, r rq + rq) of key/value head x's (GROUP + 2) HD rows -- its
    // GROUP query heads, its key, its value (the host's plan: the rows of a
    // head fill its XCD's blocks). Computed where it is used.
    auto qkv_row = [&]() {
        if (!a.local_qkv) return rowq;
        const int x = sm.xcd, lr = sm.xrank * a.rq + (rowq - b * a.rq), gq = GROUP * HD;
        return lr < gq ? x * gq + lr
             : lr < gq + HD ? (a.heads + x) * HD + (lr - gq)
                            : (a.heads + a.kvh + x) * HD + (lr - gq - HD);
    };

    // The first layer's qkv rows stream in during the choice. (Declared per
    // step so that nothing of it stays live through the head.)
    Rows<RN, RS> rr{};
    if (aq) load_rows<JD, 1, WK>(t, sm.layers[0].codes[0], sm.layers[0].scales[0], 0, qkv_row(), rr);

    // ---- the greedy choice over the blocks' candidates -------------------
    {
        float best = -INFINITY;
        int index = INT_MAX;
        if (it > 0) {
            const uint32_t tag_c = ((seq0 + (uint32_t)it - 1) << 8) + (uint32_t)(a.n_layers * PH + 1);
            if (!gather<MAXD / T>(t, a.CAND, 2 * (int)gridDim.x, lin, tag_c, sm.xin, sm, deadline, st)) leave();
            if (t < (int)gridDim.x) {
                best = sm.xin[2 * t];
                index = __float_as_int(sm.xin[2 * t + 1]);
            }
        } else if (t < (int)gridDim.x) {
            const float2 c = gload_f2(a.cand + t);
            best = c.x;
            index = __float_as_int(c.y);
        }
        best_of_wave(best, index);
        if (lane == 0) {
            sm.bv[w] = best;
            sm.bi[w] = index;
        }
        __syncthreads();
        float bv = sm.bv[0];
        int bi = sm.bi[0];
        for (int q = 1; q < NW; ++q) better(bv, bi, sm.bv[q], sm.bi[q]);
        const int token = bi == INT_MAX ? 0 : bi;
        bool stop = false;
        for (int s = 0; s < st->n_stop; ++s) stop |= st->stop[s] == token;
        const bool append = !stop && step < st->max_new;
        const bool forward = append && step + 1 < st->max_new;
        if (b == 0 && t == 0) {
            st->token = token;
            if (append) {
                a.out[step] = token;
                st->n_out = step + 1;
            }
            if (!forward) st->done = 1;
        }
        if (!forward) return;
        // Dense::row of the token (src/cpu/gemm.rs:412-429) is layer 0's input:
        // the f16 value widened, or an int8 table's f32(code) * scale
        // (widen_q8, :171-179).
        const int s_count = a.d / 16;
        for (int kk = t; kk < a.d; kk += T) {
            const int s = kk / 16, i = kk % 16;
            const size_t at = ((size_t)token * 16 + i) * s_count + s;
            float v = a.embed_q8 ? (float)gmem((const int8_t*)a.embed)[at] *
                                       gmem(a.embed_scales)[(size_t)token * (a.d / 32) + kk / 32]
                                 : f16_to_f32(gmem((const uint16_t*)a.embed)[at]);
            if (a.additive && pos < a.additive_rows) v = v + *gmem(a.additive + (size_t)pos * a.d + kk);
            sm.xres[kk] = a.em != 1.0f ? v * a.em : v;
        }
        __syncthreads();
    }

    // Each product's rows are loaded one phase ahead of it: the loads run
    // while the block waits for that phase's inputs. (Zero-initialised so
    // that no register stays live across the layer loop.)
    for (int layer = 0; layer < a.n_layers; ++layer) {
        fresh();
        const LayerPtrs& L = sm.layers[layer];
        STAMP_WHEN(layer == a.stamp_layer && it == a.stamp_step);
        STAMP(0);
        // qkv: x (gathered, or the embedding) -> RMSNorm -> quantize -> rows.
        NormRegs<JD> nq;
        load_norm<JD>(t, L.norm_attn, nq);
        // The touched words (see touch_kv); left unset where nothing is
        // touched: zeroing them would wait for whatever the registers last
        // loaded, and for the stores issued since.
        uint32_t kvt[4];
        // Polled by the first waves (the down rows' wave stored x).
        if (layer > 0 && !gather<6>(t, a.X, a.d, lin, tag_of(tag0, layer - 1, 5), sm.xres, sm, deadline, st))
            leave();
        STAMP(1);
        float inv = 0.0f;
        if constexpr (!INV_LDS) {
            inv = norm_inv_spec<JD>(t, sm.xres, a.eps, a.norm_window, sm);
        } else {
            if constexpr (EXACT) {
                const float v = norm_inv_spec<JD>(t, sm.xres, a.eps, a.norm_window, sm);
                if (t == 0) sm.inv = v;
            } else if (w == 0) {
                const float v = norm_inv_wave<JD>(t, sm.xres, a.eps);
                if (lane == 0) sm.inv = v;
            }
            __syncthreads();
        }
        STAMP(2);
        quantize_block<JD, WK>(t, sm.xres, &nq, inv, sm, nullptr, INV_LDS);
        STAMP(3);
        if (aq) {
            float acc[1];
            row_chain<JD, 1, WK>(t, rr, sm, acc);
            if ((lane & 15) == 14) {
                if (a.local_qkv)
                    put_local(a.QKV + qkv_row(), acc[0], tag_of(tag0, layer, 0));
                else
                    put(a.QKV + rowq, acc[0], tag_of(tag0, layer, 0));
            }
        }
        // No barrier here: the attention's first writes to LDS (the
        // gathered q/k/v, the values) touch nothing the qkv product reads.
        STAMP(4);
        if constexpr (DPB > 0) {
            // attention in one pass: its outputs are the o product's input.
            bool ok;
            // The attention on every block (one key/value head an XCD).
            const bool wide = EXACT && !LONG && !KV32 && a.local_qkv;
            if (wide)
                ok = attention_wide_a<GROUP>(t, a, L, pos, tag_of(tag0, layer, 0), tag_of(tag0, layer, 1), sm,
                                             deadline) &&
                     attention_wide_b<GROUP>(t, a, pos, tag_of(tag0, layer, 1), tag_of(tag0, layer, 2), sm, deadline,
                                             NW - nqw);
            else if constexpr (KV32)
                ok = attention_exact32<GROUP, DPB>(t, a, L, pos, tag_of(tag0, layer, 0), tag_of(tag0, layer, 2), sm,
                                                   deadline);
            else if constexpr (EXACT && LONG)
                ok = attention_exact_long<GROUP, DPB>(t, a, L, pos, tag_of(tag0, layer, 0), tag_of(tag0, layer, 2), sm,
                                                      deadline);
            else if constexpr (EXACT)
                ok = attention_exact<GROUP, DPB>(t, a, L, pos, tag_of(tag0, layer, 0), tag_of(tag0, layer, 2), sm,
                                                 deadline);
            else
                ok = attention_all<GROUP, DPB>(t, a, L, pos, tag_of(tag0, layer, 0), tag_of(tag0, layer, 2), sm,
                                               deadline);
            if (!ok) leave();
            // o + residual; the o and gate_up rows stream in meanwhile, and
            // the qkv waves (nothing in flight) poll.
            if (ao)
                load_rows<JO, 1, WK>(t, L.codes[1], L.scales[1], 0, rowo, rr);
            else
                zero_rows(rr);
            // (Packed: the gate_up rows load after the o product instead,
            // but in the f32-cache instance, where that spills registers.)
            if ((!packed || KV32) && agu) load_rows<JD, 2, WK>(t, L.codes[2], L.scales[2], a.ffn, rowgu, rr);
            // Then the attention waves before the qkv waves load the next
            // attention's keys and values into L2 (with the wide attention,
            // every block of the XCD a share).
            if (EXACT && w < NW - nqw) {
                const bool last = layer + 1 == a.n_layers;
                const int kvh = a.kvh;
                if (wide)
                    touch_kv<4, 2>(t, (NW - nqw) * WAVE, sm.layers[last ? 0 : layer + 1], sm.xcd, sm.xrank,
                                   (int)gridDim.x / NX, last ? pos + 1 : pos, a.max_pos, kvt);
                else if (b < 2 * a.heads)
                    touch_kv<4, KV32 ? 4 : 2>(t, (NW - nqw) * WAVE, sm.layers[last ? 0 : layer + 1], b % kvh, b / kvh,
                                              2 * a.heads / kvh, last ? pos + 1 : pos, a.max_pos, kvt);
            }
            __syncthreads();
            if (!gather<8>(t, a.ATT, a.qd, lin, tag_of(tag0, layer, 2), sm.xin, sm, deadline, st, NW - nqw))
                leave();
            STAMP(11);
        } else {
            // attention partials.
            if (!attention<GROUP>(t, a, L, pos, tag_of(tag0, layer, 0), tag_of(tag0, layer, 1), sm, deadline))
                leave();
            // combine; the o rows stream in meanwhile.
            if (ao)
                load_rows<JO, 1, WK>(t, L.codes[1], L.scales[1], 0, rowo, rr);
            else
                zero_rows(rr);
            __syncthreads();
            if (!combine(t, a, tag_of(tag0, layer, 1), tag_of(tag0, layer, 2), sm, deadline, nu + no)) leave();
            // o + residual; the gate_up rows stream in meanwhile.
            if (agu)
                load_rows<JD, 2, WK>(t, L.codes[2], L.scales[2], a.ffn, rowgu, rr);
            else if (!ao)  // the o rows are still to be used
                zero_rows(rr);
            __syncthreads();
            // Polled from the first o wave on: the gate_up waves' loads are
            // in flight.
            if (!gather<8>(t, a.ATT, a.qd, lin, tag_of(tag0, layer, 2), sm.xin, sm, deadline, st, nu)) leave();
        }
        quantize_block<JO, WK>(t, sm.xin, (const NormRegs<JO>*)nullptr, 1.0f, sm);
        STAMP(12);
        if (ao) {
            float acc[1];
            row_chain<JO, 1, WK>(t, rr, sm, acc);
            if ((lane & 15) == 14) put(a.X + rowo, sm.xres[rowo] + a.rm * acc[0], tag_of(tag0, layer, 3));
        }
        STAMP(13);
        // The touched words are consumed here, where they have long arrived
        // (before the polls of the gather below).
        asm volatile("" ::"v"(kvt[0]), "v"(kvt[1]), "v"(kvt[2]), "v"(kvt[3]));
        // gate_up + SwiGLU.
        // Each product's rows stream in during the hand-over just before it:
        // o's during the attention outputs', gate_up's here (packed: their
        // waves hold no other rows), down's during h's, the next qkv's
        // during x's after down. (Measured: with gate_up's and the next
        // qkv's loads a hand-over earlier, each hand-over with two loads in
        // flight took 2.0-2.7 us; 675 -> 635 us a forward.) This gather is
        // then polled by the last waves, clear of the gate_up waves [0, nu).
        constexpr bool GU_LATE = DPB > 0 && !KV32;
        if (GU_LATE && packed && agu) load_rows<JD, 2, WK>(t, L.codes[2], L.scales[2], a.ffn, rowgu, rr);
        const int need = (a.d + WAVE * MWK - 1) / (WAVE * MWK);
        const int px = GU_LATE && packed && NW - need >= nu ? NW - need : 0;
        NormRegs<JD> ngu, nfs;
        load_norm<JD>(t, L.norm_mlp, ngu);
        if (a.ffn_scales) load_norm<JD>(t, a.ffn_scales + (size_t)layer * a.d, nfs);
        __syncthreads();
        if (!gather<MWK>(t, a.X, a.d, lin, tag_of(tag0, layer, 3), sm.xres, sm, deadline, st, px)) leave();
        STAMP(14);
        float inv_gu = 0.0f;
        if constexpr (!INV_LDS) {
            inv_gu = norm_inv_spec<JD>(t, sm.xres, a.eps, a.norm_window, sm);
        } else {
            if constexpr (EXACT) {
                const float v = norm_inv_spec<JD>(t, sm.xres, a.eps, a.norm_window, sm);
                if (t == 0) sm.inv = v;
            } else if (w == 0) {
                const float v = norm_inv_wave<JD>(t, sm.xres, a.eps);
                if (lane == 0) sm.inv = v;
            }
            __syncthreads();
        }
        STAMP(15);
        quantize_block<JD, WK>(t, sm.xres, &ngu, inv_gu, sm, a.ffn_scales ? &nfs : nullptr, INV_LDS);
        STAMP(16);
        if (agu) {
            float acc[2];
            row_chain<JD, 2, WK>(t, rr, sm, acc);
            if ((lane & 15) == 14) put(a.H + rowgu, silu_trit(acc[0]) * acc[1], tag_of(tag0, layer, 4));
        }
        STAMP(17);
        // down + residual.
        if (ad && dround == 0)
            load_rows<JFR, 1, WK, RN, RS, JF, 0>(t, L.codes[3], L.scales[3], 0, rowd, rr);
        else if (DR > 1 && ad)
            load_rows<JFR, 1, WK, RN, RS, JF, (DR > 1 ? JFR : 0)>(t, L.codes[3], L.scales[3], 0, rowd, rr);
        else
            zero_rows(rr);

        __syncthreads();
        if (!gather<MWK>(t, a.H, a.ffn, lin, tag_of(tag0, layer, 4), sm.xin, sm, deadline, st)) leave();
        STAMP(18);
        quantize_block<JF, WK>(t, sm.xin, (const NormRegs<JF>*)nullptr, 1.0f, sm);
        STAMP(19);
        if constexpr (DR == 1) {
            if (ad) {
                float acc[1];
                row_chain<JF, 1, WK>(t, rr, sm, acc);
                if ((lane & 15) == 14) put(a.X + rowd, sm.xres[rowd] + a.rm * acc[0], tag_of(tag0, layer, 5));
            }
        } else {
            // The first round's waves chain inputs [0, 256 JFR) and leave each
            // row's total in LDS; the second round's continue from it.
            if (ad && dround == 0) {
                float acc[1];
                row_chain<JFR, 1, WK>(t, rr, sm, acc);
                if ((lane & 15) == 14) sm.dcarry[rowd - b * a.rd] = acc[0];
            }
            __syncthreads();
            if (ad && dround == 1) {
                float acc[1];
                const float start[1] = {sm.dcarry[rowd - b * a.rd]};
                row_chain<JFR, 1, WK, RN, RS, JFR>(t, rr, sm, acc, start);
                if ((lane & 15) == 14) put(a.X + rowd, sm.xres[rowd] + a.rm * acc[0], tag_of(tag0, layer, 5));
            }
        }
        // The next layer's qkv rows stream in during the x hand-over.
        if (aq && layer + 1 < a.n_layers)
            load_rows<JD, 1, WK>(t, sm.layers[layer + 1].codes[0], sm.layers[layer + 1].scales[0], 0, qkv_row(), rr);
        __syncthreads();
        STAMP(20);
    }

    // ---- final RMSNorm, the head, the block's best logit ----------------
    // Pass p of block b covers head rows [32 (p nb + b), +32), 16-lane
    // group r row 32 (p nb + b) + r: the blocks sweep the table together.
    // Three passes of weights are in flight at a time, and each lane keeps
    // the normed x values of its lane chain in registers.
    // 16-byte units per lane chain: d / 128 (f16) or d / 256 (int8). An int8
    // head's row has d / 32 f32 scales, SC a lane: lane i of a row holds
    // scales SC i .. SC i + SC - 1, and the chain's step s, in group s / 2,
    // reads its scale from lane (s / 2) / SC of the row by a row broadcast.
    constexpr int SU = HK == HK_F16 ? JD * 2 : JD;
    constexpr int SC = HK == HK_F16 ? 1 : JD / 2;
    static_assert(HK == HK_F16 || JD % 2 == 0, "an int8 head's scales split over the row's lanes");
    struct Pass {
        uint4 w[SU];
        float sc[SC];
    };
    fresh();
    const int l16 = t & 15;
    const int rows_pass = T / 16, nb = (int)gridDim.x;
    const int passes = (a.vocab + rows_pass * nb - 1) / (rows_pass * nb);
    auto row_of = [&](int p) { return (p * nb + b) * rows_pass + (t >> 4); };
    // Wave w of pass p reads 4-row tile (p nb + b) 8 + w: instruction j
    // reads the tile's 1 KB run j, in which lane 16g + i finds unit j of
    // lane chain i of the tile's row g.
    const int tiles = (a.vocab + 3) / 4;
    const size_t tile_bytes = (size_t)4 * a.d * (HK == HK_F16 ? 2 : 1);
    auto load_pass = [&](int p, Pass& wv) {
        const int tile = (p * nb + b) * (rows_pass / 4) + w;
        const uint4* src = (const uint4*)((const uint8_t*)a.head + (size_t)(tile < tiles ? tile : 0) * tile_bytes);
#pragma unroll
        for (int j = 0; j < SU; ++j) wv.w[j] = load_stream(src + j * WAVE + lane);
        if constexpr (HK == HK_Q8) {
            const int row = row_of(p);
            const TRIT_GLOBAL float* sc =
                gmem(a.head_scales) + (size_t)(row < a.vocab ? row : 0) * (a.d / 32) + SC * l16;
#pragma unroll
            for (int c = 0; c < SC; ++c) wv.sc[c] = sc[c];
        }
    };
    // Passes in flight: three, or two in the long-session instances (their
    // attention leaves fewer registers; three would spill), one for d > 1024
    // (a pass of 2048 f16 weights a row is 64 registers; the chip then has
    // 32 MB of head rows in flight, past HBM's bandwidth-latency product).
    constexpr int RING = LONG ? 2 : JD > 4 ? 1 : 3;
    // The normed x of the lane's chain: in registers up to d = 1024, else
    // read from LDS (sm.xt) as the chain goes.
    constexpr bool XLDS = JD > 4;
    constexpr int XS = JD * 16 + 4;
    Pass ring[RING];
#pragma unroll
    for (int q = 0; q < RING; ++q)
        if (q < passes) load_pass(q, ring[q]);
    float fn[(MAXD + T - 1) / T];
#pragma unroll
    for (int q = 0; q < (MAXD + T - 1) / T; ++q) fn[q] = t + T * q < a.d ? gmem(a.final_norm)[t + T * q] : 0.0f;
    STAMP_WHEN(a.stamp_layer == a.n_layers && it == a.stamp_step);
    if (!gather<MAXD / T>(t, a.X, a.d, lin, tag_of(tag0, a.n_layers - 1, 5), sm.xres, sm, deadline, st)) return;
    STAMP(21);
    if constexpr (EXACT) {
        const float inv = norm_inv_spec<JD>(t, sm.xres, a.eps, a.norm_window, sm);
        if (t == 0) sm.inv = inv;
    } else if (w == 0) {
        const float inv = norm_inv_wave<JD>(t, sm.xres, a.eps);
        if (lane == 0) sm.inv = inv;
    }
    __syncthreads();
    // RMSNorm as src/layers.rs:136-144: x * (inv * w).
#pragma unroll
    for (int q = 0; q < (MAXD + T - 1) / T; ++q)
        if (t + T * q < a.d) sm.xin[t + T * q] = sm.xres[t + T * q] * (sm.inv * fn[q]);
    __syncthreads();
    STAMP(22);
    float xr[XLDS ? 1 : JD * 16];  // lane chain l16 of the normed x
    if constexpr (XLDS) {
        for (int kk = t; kk < a.d; kk += T) sm.xt[(kk & 15) * XS + (kk >> 4)] = sm.xin[kk];
        __syncthreads();
    } else {
#pragma unroll
        for (int s = 0; s < JD * 16; ++s) xr[s] = sm.xin[16 * s + l16];
    }
    // Values s0 .. s0 + N - 1 of the lane's chain.
    auto chain_x = [&](int s0, auto& out) {
        constexpr int N = sizeof(out) / sizeof(float);
        if constexpr (XLDS) {
#pragma unroll
            for (int q = 0; q < N; q += 4) {
                const float4 v = *(const float4*)(sm.xt + l16 * XS + s0 + q);
                out[q] = v.x;
                out[q + 1] = v.y;
                out[q + 2] = v.z;
                out[q + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int q = 0; q < N; ++q) out[q] = xr[s0 + q];
        }
    };
    float best = -INFINITY;
    int index = INT_MAX;
    auto head_pass = [&](int p, Pass& wv) {
        // Trit's 16-lane order (gemv_float.hip): lane chain, then the tree.
        // The weight is the f16 value widened, or f32(code) * scale of its
        // 32-group, one rounding (widen_q8).
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < SU; ++j) {
            const uint32_t words[4] = {wv.w[j].x, wv.w[j].y, wv.w[j].z, wv.w[j].w};
            if constexpr (HK == HK_F16) {
                float xx[8];
                chain_x(j * 8, xx);
#pragma unroll
                for (int hh = 0; hh < 8; ++hh) {
                    const float wf = f16_to_f32((uint16_t)(words[hh >> 1] >> ((hh & 1) * 16)));
                    acc = __builtin_fmaf(xx[hh], wf, acc);
                }
            } else {
                float xx[16];
                chain_x(16 * j, xx);
#pragma unroll
                for (int u = 0; u < 16; u += 2) {
                    const int g = 8 * j + u / 2;  // the group of steps 16 j + u, + u + 1
                    const float scale = row_bcast(wv.sc[g % SC], g / SC);
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        const int h = u + e;
                        const float wf = (float)(int8_t)(uint8_t)(words[h >> 2] >> ((h & 3) * 8)) * scale;
                        acc = __builtin_fmaf(xx[h], wf, acc);
                    }
                }
            }
        }
        // Lane i adds lane i - 8, - 4, - 2, - 1 of its row (rotations): in
        // lane 0 that is the xor tree of gemv_float.hip, bit for bit (the
        // pairs it adds are the same sums with their operands swapped).
        float v = acc;
        v = v + dpp<0x128>(v);
        v = v + dpp<0x124>(v);
        v = v + dpp<DPP_ROR2>(v);
        v = v + dpp<0x121>(v);
        if (a.logit_w != 1.0f) v = v * a.logit_w;  // Granite's 1 / logits_scaling
        const int row = row_of(p);
        if (l16 == 0 && row < a.vocab && (index == INT_MAX || v > best)) {
            best = v;
            index = row;
        }
        if (p + RING < passes) load_pass(p + RING, wv);
    };
    for (int p = 0; p < passes; p += RING) {
        head_pass(p, ring[0]);
        if constexpr (RING > 1)
            if (p + 1 < passes) head_pass(p + 1, ring[1 % RING]);
        if constexpr (RING > 2)
            if (p + 2 < passes) head_pass(p + 2, ring[2 % RING]);
    }
    STAMP(23);
    // The block's first maximum: the lanes of a row group agree; waves by
    // shuffles, then one thread over the waves.
    best_of_wave(best, index);
    if (lane == 0) {
        sm.bv[w] = best;
        sm.bi[w] = index;
    }
    // Every store of the block in this step (the cache appends among them)
    // is acknowledged before the candidates are put: the next step reads
    // the caches only after it has polled every block's candidates.
    __builtin_amdgcn_s_waitcnt(VMCNT0);
    __syncthreads();
    if (t == 0) {
        float bv = sm.bv[0];
        int bi = sm.bi[0];
        for (int q = 1; q < NW; ++q) better(bv, bi, sm.bv[q], sm.bi[q]);
        a.cand[b] = make_float2(bv, __int_as_float(bi));
        const uint32_t tag_c = tag0 + (uint32_t)(a.n_layers * PH + 1);
        put(a.CAND + 2 * b, bv, tag_c);
        put(a.CAND + 2 * b + 1, __int_as_float(bi), tag_c);
        if (b == 0) st->pos = pos + 1;
    }
    STAMP(24);
    __syncthreads();  // sm.bv / sm.bi are the next choice's
    }
}

// The head's tiled layout: rows in tiles of four; in a tile, 16-byte run
// (j, g, i) holds unit j of lane chain i of row g (values 8j .. 8j + 7 of
// an f16 chain, 16j .. 16j + 15 of an int8 one; element kk = 16 s + i of
// the row is value s of chain i), runs ordered j, then g, then i. From the
// lane-chain layout [row][i][s] of an F16 or Q8 layer; s8 16-byte units a
// chain.
__global__ void head_tile_kernel(const uint4* __restrict__ src, int n, int s8, uint4* __restrict__ dst) {
    const size_t chunks = (size_t)n * 16 * s8;
    for (size_t q = blockIdx.x * (size_t)blockDim.x + threadIdx.x; q < chunks; q += (size_t)gridDim.x * blockDim.x) {
        const size_t r = q / (16 * s8);
        const int rem = (int)(q - r * 16 * s8), i = rem / s8, j = rem % s8;
        const size_t to = (r / 4) * (size_t)(4 * 16 * s8) + (size_t)(j * 4 + (int)(r % 4)) * 16 + i;
        dst[to] = src[q];
    }
}

// The blocks' candidates from a logits row (after a prefill), with the
// head phase's row split.
__global__ __launch_bounds__(256) void cand_kernel(const float* __restrict__ logits, int vocab, int rh,
                                                   float2* __restrict__ cand) {
    __shared__ float bv[256];
    __shared__ int bi[256];
    const int r0 = blockIdx.x * rh, r1 = min(r0 + rh, vocab);
    float best = -INFINITY;
    int index = INT_MAX;
    for (int i = r0 + (int)threadIdx.x; i < r1; i += 256) {
        const float v = logits[i];
        if (index == INT_MAX || v > best) {
            best = v;
            index = i;
        }
    }
    bv[threadIdx.x] = best;
    bi[threadIdx.x] = index;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) better(bv[threadIdx.x], bi[threadIdx.x], bv[threadIdx.x + s], bi[threadIdx.x + s]);
        __syncthreads();
    }
    if (threadIdx.x == 0) cand[blockIdx.x] = make_float2(bv[0], __int_as_float(bi[0]));
}

using StepFn = void (*)(StepArgs, int, int, uint32_t, int);

// The instantiated shapes: (d/256, heads*hd/256, ffn/256, q heads per kv head).
// dpb: output dims of one query head a block takes in the one-pass
// attention, 0 for the split attention and its combine.
// wk, hk: the linears' and the head's kinds (WK_*, HK_*); the tree-sum
// instances take Q8_0 linears and an f16 head only.
// lng: sessions of more than T positions, instantiated for Qwen3-0.6B's
// shape with Q8_0 linears and an f16 head, and with int8 linears and a Q8
// head (S1-mini).
template <int JD, int JO, int JF, int GROUP, int DPB>
StepFn exact_fn(int wk, int hk, bool lng) {
    if (lng) {
        if constexpr (JD == 4 && JO == 8 && JF == 12) {
            if (wk == WK_Q8_0 && hk == HK_F16) return step_kernel<JD, JO, JF, GROUP, DPB, true, WK_Q8_0, HK_F16, true>;
            if (wk == WK_INT8 && hk == HK_Q8) return step_kernel<JD, JO, JF, GROUP, DPB, true, WK_INT8, HK_Q8, true>;
        }
        return nullptr;
    }
    if (wk == WK_Q8_0) return hk == HK_F16 ? step_kernel<JD, JO, JF, GROUP, DPB, true, WK_Q8_0, HK_F16>
                                           : step_kernel<JD, JO, JF, GROUP, DPB, true, WK_Q8_0, HK_Q8>;
    return hk == HK_F16 ? step_kernel<JD, JO, JF, GROUP, DPB, true, WK_INT8, HK_F16>
                        : step_kernel<JD, JO, JF, GROUP, DPB, true, WK_INT8, HK_Q8>;
}

StepFn step_fn(int jd, int jo, int jf, int group, int dpb, bool exact, int wk, int hk, bool lng = false,
               bool kv32 = false) {
    if (!exact && (wk != WK_Q8_0 || hk != HK_F16 || lng)) return nullptr;
    if (kv32) {
        // Trit's f32 caches: Qwen3-0.6B's shape, Q8_0 / Q4_K linears, an f16
        // table, Trit's orders, up to T positions.
        if (jd == 4 && jo == 8 && jf == 12 && group == 2 && exact && dpb == 8 && !lng && wk == WK_Q8_0 &&
            hk == HK_F16)
            return step_kernel<4, 8, 12, 2, 8, true, WK_Q8_0, HK_F16, false, true>;
        return nullptr;
    }
    if (jd == 4 && jo == 8 && jf == 12 && group == 2) {  // Qwen3-0.6B
        if (exact) return dpb == 8 ? exact_fn<4, 8, 12, 2, 8>(wk, hk, lng) : nullptr;
        if (dpb == 0) return step_kernel<4, 8, 12, 2, 0, false, WK_Q8_0, HK_F16>;
        if (dpb == 8) return step_kernel<4, 8, 12, 2, 8, false, WK_Q8_0, HK_F16>;
    }
    if (jd == 4 && jo == 4 && jf == 8 && group == 2) {
        if (exact) return dpb == 4 ? exact_fn<4, 4, 8, 2, 4>(wk, hk, lng) : nullptr;
        if (dpb == 0) return step_kernel<4, 4, 8, 2, 0, false, WK_Q8_0, HK_F16>;
        if (dpb == 4) return step_kernel<4, 4, 8, 2, 4, false, WK_Q8_0, HK_F16>;
    }
    // Qwen3-1.7B (d 2048, ffn 6144): Trit's orders, Q8_0 / Q4_K linears, an
    // f16 table, sessions of up to T positions.
    if (jd == 8 && jo == 8 && jf == 24 && group == 2 && exact && dpb == 8 && !lng && wk == WK_Q8_0 && hk == HK_F16)
        return step_kernel<8, 8, 24, 2, 8, true, WK_Q8_0, HK_F16>;
    return nullptr;
}

int device_blocks() {
    int dev = 0;
    TRIT_HIP(hipGetDevice(&dev));
    int cus = 0;
    TRIT_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    return cus;
}

struct Plan {
    int blocks, splits, comb, dpb, rq, ro, rgu, rd, rh, wk, hk;
    int local_qkv;
    StepFn fn;
};

// The one-pass attention unless TRIT_HIP_STEP_SPLIT=1 asks for the split
// attention and its combine (which also serve longer sessions).
bool split_forced() {
    const char* v = getenv("TRIT_HIP_STEP_SPLIT");
    return v && v[0] == '1';
}

// The attention on every block with each key/value head's exchanges in one
// XCD's L2 (StepArgs::local_qkv): the Trit-order instance of up to T
// positions with f16 caches, one key/value head an XCD whose (group + 2) HD
// qkv rows fill that XCD's blocks at rq rows each, BPH blocks a query head,
// and the head's scores polled by the qkv waves (two words a lane).
// TRIT_HIP_STEP_LOCAL=0 keeps the attention on two blocks a query head and
// every exchange at agent scope.
bool local_fits(const SessionImpl& S, const Plan& p) {
    const char* v = getenv("TRIT_HIP_STEP_LOCAL");
    if (v && v[0] == '0') return false;
    const auto& c = S.dec->c;
    const int group = c.heads / c.kv_heads, nbx = p.blocks / NX, nqw = p.rq / 4;
    constexpr int mw = T / (4 * WAVE);  // attention_wide_b's gather
    return S.exact && !S.kv32 && S.max_pos <= T && p.dpb > 0 && c.kv_heads == NX && p.blocks % NX == 0 &&
           nbx * p.rq == (group + 2) * HD && nbx == group * BPH && NW - nqw + (T + WAVE * mw - 1) / (WAVE * mw) <= NW;
}

bool plan(const SessionImpl& S, Plan& p) {
    const DecoderImpl& D = *S.dec;
    const auto& c = D.c;
    // f32 caches: the Trit-order instance of up to T positions only.
    if (S.kv32 && (!S.exact || S.max_pos > T)) return false;
    // Granite's multipliers, per-layer MLP scales and added input rows run
    // on the Trit-order instance only.
    if ((D.granite() || D.has_ffn_scales || S.additive_rows) && !S.exact) return false;
    if (c.head_dim != HD || c.kv_heads <= 0 || c.heads % c.kv_heads != 0) return false;
    const int group = c.heads / c.kv_heads, qd = c.heads * HD;
    if (c.d % 256 || qd % 256 || c.ffn % 256 || c.d > MAXD || qd > MAXK || c.ffn > MAXK) return false;
    if (c.layers <= 0 || c.layers > MAXL || c.layers * PH + PH >= 256) return false;
    // Every linear Q8_0 / Q4_K (32-groups, f16 scales), or every linear
    // Trit's int8 (128-groups, f32 scales); no bias.
    auto wk_of = [](const LayerRef& L) {
        if (L->bias.ptr) return -1;
        if (L->kind == Q8_0 || L->kind == Q4_K) return (int)WK_Q8_0;
        if (L->kind == INT8 && L->group == 128) return (int)WK_INT8;
        return -1;
    };
    p.wk = wk_of(D.qkv[0]);
    if (p.wk < 0) return false;
    for (int l = 0; l < c.layers; ++l)
        if (wk_of(D.qkv[l]) != p.wk || wk_of(D.o[l]) != p.wk || wk_of(D.gate_up[l]) != p.wk || wk_of(D.down[l]) != p.wk)
            return false;
    // An f16 or int8-storage (Q8) head, and such a table for the embeddings.
    const Layer& head = D.head ? *D.head : *D.embed;
    if (head.k != c.d || head.bias.ptr || (D.embed->kind != F16 && D.embed->kind != Q8_F32)) return false;
    if (head.kind == F16) p.hk = HK_F16;
    else if (head.kind == Q8_F32 && c.d % 512 == 0) p.hk = HK_Q8;
    else return false;
    p.blocks = device_blocks();
    if (p.blocks < c.kv_heads || p.blocks % c.kv_heads) return false;
    const int nq = (c.heads + 2 * c.kv_heads) * HD;
    auto rows = [&](int n, int& r) {
        if (n % (4 * p.blocks)) return false;
        r = n / p.blocks;
        return r <= 4 * NW;
    };
    if (!rows(nq, p.rq) || !rows(c.d, p.ro) || !rows(c.ffn, p.rgu) || !rows(c.d, p.rd)) return false;
    // The kernel's wave ranges by product (disjoint where rows are live
    // together; the kernel derives the same layout) and the waves each
    // gather polls with. A down product of more than 16 chunks a lane runs
    // in two rounds on two sets of waves.
    const int nu = p.rgu / 4, no = p.ro / 4, nd = p.rd / 4, nqw = p.rq / 4;
    const int dr = c.ffn / 256 > 16 ? 2 : 1;
    const bool packed = nu + std::max(no, dr * nd) + nqw <= NW;
    // Otherwise gate_up takes the last waves (the one-pass Trit-order
    // attention only): gate_up beside o, down beside qkv.
    if (!packed && (!S.exact || nu + no > NW || dr * nd + nqw > NW)) return false;
    auto fits = [](int n, int p0, int mw) { return p0 + (n + WAVE * mw - 1) / (WAVE * mw) <= NW; };
    if (!fits((group + 2) * HD, NW - nqw - 1, 8)) return false;
    const int mwk = std::max(c.ffn / 256, 12) * 256 / T;  // the kernel's MWK
    if (!fits(c.d, 0, 6) || !fits(c.ffn, 0, mwk) || !fits(c.d, 0, mwk)) return false;
    if (!fits(2 * p.blocks, 0, MAXD / T)) return false;  // the candidates' words
    p.splits = p.blocks / c.kv_heads;
    p.comb = qd / p.blocks;
    // The one-pass attention: every key of the session in registers, each
    // block dpb dims of one query head.
    p.dpb = (qd % p.blocks) ? 0 : qd / p.blocks;
    if (S.exact) {
        // Trit's sum orders: the one-pass attention with a thread per key
        // (up to T positions), wave w output dim w of the block's DPB; the
        // long form (keys in rounds of T) up to MAXT positions.
        if (S.max_pos > MAXT || (p.dpb != 4 && p.dpb != 8) || p.blocks % (c.kv_heads * group) ||
            !fits(qd, NW - nqw, 8))
            return false;
        p.fn = step_fn(c.d / 256, qd / 256, c.ffn / 256, group, p.dpb, true, p.wk, p.hk, S.max_pos > T, S.kv32);
        if (!p.fn) return false;
        p.rh = (c.vocab + p.blocks - 1) / p.blocks;
        p.local_qkv = local_fits(S, p);
        return true;
    }
    const bool one_pass = !split_forced() && S.max_pos <= 32 * MAXF && (p.dpb == 4 || p.dpb == 8) &&
                          p.blocks % (c.kv_heads * group) == 0 && fits(qd, NW - nqw, 8);
    if (one_pass) {
        p.fn = step_fn(c.d / 256, qd / 256, c.ffn / 256, group, p.dpb, false, p.wk, p.hk);
    } else {
        p.dpb = 0;
        if (S.max_pos > p.splits * 32 * MAXC) return false;
        if ((qd % p.blocks) || HD % p.comb) return false;
        if (p.splits > WAVE || p.comb > NW || p.splits * (2 + p.comb) > MAXK) return false;
        if (!fits(p.splits * (2 + p.comb), NW - nqw, 2) || !fits(qd, nu, 8)) return false;
        p.fn = step_fn(c.d / 256, qd / 256, c.ffn / 256, group, 0, false, p.wk, p.hk);
    }
    if (!p.fn) return false;
    p.rh = (c.vocab + p.blocks - 1) / p.blocks;
    p.local_qkv = 0;
    return true;
}

}  // namespace

// Where the wide attention's score words start in the exchange buffer:
// after every other region, on a 128-byte line of their own (no line of
// them is written from another XCD).
size_t sc_words(const TritHipLmConfig& c, const Plan& p) {
    const int nq = (c.heads + 2 * c.kv_heads) * HD, qd = c.heads * HD;
    const size_t end = (size_t)c.d + nq + (size_t)c.heads * p.splits * (HD + 2) + qd + c.ffn + 2 * (size_t)p.blocks;
    return (end + 15) / 16 * 16;
}

bool decode_step_supported(const SessionImpl& S) {
    Plan p;
    return plan(S, p);
}

int decode_step_layout(const SessionImpl& S) {
    Plan p;
    if (!plan(S, p)) return 0;
    return 1 | (p.local_qkv ? 2 : 0);
}

void decode_step_prepare(SessionImpl& S, hipStream_t s) {
    Plan p;
    if (!plan(S, p)) fail("decode step: the session's model does not fit the persistent step");
    const DecoderImpl& D = *S.dec;
    const auto& c = D.c;
    const size_t words = sc_words(c, p) + (size_t)c.heads * T + 16;  // + the XCD rank counters' line
    if (!S.step_words.ptr) {
        S.step_words.alloc(words * 8);
        TRIT_HIP(hipMemsetAsync(S.step_words.ptr, 0, words * 8, s));
        S.step_cand.alloc((size_t)p.blocks * sizeof(float2));
        std::vector<LayerPtrs> table(c.layers);
        for (int l = 0; l < c.layers; ++l) {
            const LayerRef* ls[4] = {&D.qkv[l], &D.o[l], &D.gate_up[l], &D.down[l]};
            for (int i = 0; i < 4; ++i) {
                table[l].codes[i] = (*ls[i])->codes.as<uint8_t>();
                table[l].scales[i] = (*ls[i])->scales.ptr;
            }
            table[l].norm_attn = D.norm_attn(l);
            table[l].norm_mlp = D.norm_mlp(l);
            table[l].q_norm = D.q_norm(l);
            table[l].k_norm = D.k_norm(l);
            // A layer's caches in bytes: f16 values, or f32 (S.kv32).
            const size_t layer_bytes = (size_t)c.kv_heads * S.max_pos * HD * (S.kv32 ? 4 : 2);
            table[l].kcache = (_Float16*)(S.kcache.as<uint8_t>() + (size_t)l * layer_bytes);
            table[l].vcache = (_Float16*)(S.vcache.as<uint8_t>() + (size_t)l * layer_bytes);
        }
        const Layer& head = D.head ? *D.head : *D.embed;
        std::call_once(D.step_head_once, [&] {
            const size_t rows = (size_t)(c.vocab + 3) / 4 * 4, elem = head.kind == F16 ? 2 : 1;
            D.step_head.alloc(rows * c.d * elem);
            TRIT_HIP(hipMemsetAsync(D.step_head.ptr, 0, rows * c.d * elem, s));
            hipLaunchKernelGGL(head_tile_kernel, dim3(4096), dim3(256), 0, s, head.codes.as<uint4>(), c.vocab,
                               (int)(c.d * elem / 256), D.step_head.as<uint4>());
            TRIT_HIP(hipGetLastError());
            TRIT_HIP(hipStreamSynchronize(s));
        });
        S.step_table.alloc(table.size() * sizeof(LayerPtrs));
        TRIT_HIP(hipMemcpy(S.step_table.ptr, table.data(), table.size() * sizeof(LayerPtrs), hipMemcpyHostToDevice));
        S.step_seq = 0;
    }
    if (!S.step_cand_fresh) {
        hipLaunchKernelGGL(cand_kernel, dim3(p.blocks), dim3(256), 0, s, S.logits.as<float>(), c.vocab, p.rh,
                           S.step_cand.as<float2>());
        TRIT_HIP(hipGetLastError());
    }
}

// The (step, layer) the measurement build stamps (-1: none).
int g_stamp_step = -1, g_stamp_layer = -1;

void decode_step_launch(SessionImpl& S, int step, int pos, int nsteps, hipStream_t s) {
    Plan p;
    if (!plan(S, p)) fail("decode step: the session's model does not fit the persistent step");
    if (nsteps < 1 || nsteps >= (1 << 20)) fail("decode step: 1 to 2^20 - 1 steps a launch");
    const DecoderImpl& D = *S.dec;
    const auto& c = D.c;
    const int nq = (c.heads + 2 * c.kv_heads) * HD, qd = c.heads * HD;
    // Tags: step counter in the high 24 bits, phase in the low 8. When the
    // counter would wrap, the words start over from zero.
    if (S.step_seq + (uint32_t)nsteps >= (1u << 24)) {
        const size_t words =
            sc_words(c, p) + (size_t)c.heads * T + 16;  // + the XCD rank counters' line
        TRIT_HIP(hipMemsetAsync(S.step_words.ptr, 0, words * 8, s));
        S.step_seq = 0;
    }
    const uint32_t seq0 = S.step_seq + 1;
    S.step_seq += (uint32_t)nsteps;
    StepArgs a{};
    a.layers = S.step_table.as<LayerPtrs>();
    a.n_layers = c.layers;
    a.d = c.d;
    a.qd = qd;
    a.ffn = c.ffn;
    a.heads = c.heads;
    a.kvh = c.kv_heads;
    a.vocab = c.vocab;
    a.qk_norm = c.qk_norm;
    a.max_pos = S.max_pos;
    a.eps = c.eps;
    a.embed = D.embed->codes.ptr;
    a.embed_q8 = D.embed->kind == Q8_F32;
    a.embed_scales = D.embed->kind == Q8_F32 ? D.embed->scales.as<float>() : nullptr;
    a.head = D.step_head.ptr;
    const Layer& head = D.head ? *D.head : *D.embed;
    a.head_scales = head.kind == Q8_F32 ? head.scales.as<float>() : nullptr;
    a.final_norm = D.final_norm();
    a.rope_sin = S.rope_sin.as<float>();
    a.rope_cos = S.rope_cos.as<float>();
    uint64_t* w = S.step_words.as<uint64_t>();
    a.X = w;
    a.QKV = a.X + c.d;
    a.PART = a.QKV + nq;
    a.ATT = a.PART + (size_t)c.heads * p.splits * (HD + 2);
    a.H = a.ATT + qd;
    a.CAND = a.H + c.ffn;
    a.SC = w + sc_words(c, p);
    a.cand = S.step_cand.as<float2>();
    a.out = S.tokens_out.as<int>();
    a.st = S.st();
    a.splits = p.splits;
    a.comb = p.comb;
    a.rq = p.rq;
    a.ro = p.ro;
    a.rgu = p.rgu;
    a.rd = p.rd;
    a.rh = p.rh;
    int rate_khz = 0, dev = 0;
    TRIT_HIP(hipGetDevice(&dev));
    TRIT_HIP(hipDeviceGetAttribute(&rate_khz, hipDeviceAttributeWallClockRate, dev));
    a.ticks = (unsigned long long)(rate_khz > 0 ? rate_khz : 100000) * 200ull;  // 200 ms
    // TRIT_HIP_STEP_DEADLINE_US overrides the deadline (tests of the abort
    // path: 0 makes every block's first wait give up, and the launch drains).
    if (const char* v = getenv("TRIT_HIP_STEP_DEADLINE_US"))
        a.ticks = (unsigned long long)(rate_khz > 0 ? rate_khz : 100000) * strtoull(v, nullptr, 10) / 1000ull;
    // TRIT_HIP_NORM_WINDOW narrows the candidate starts of the RMSNorm and
    // softmax sums (tests of the path that chains a segment again: 0 leaves
    // only the estimate, -1 none).
    a.norm_window = 31;
    if (const char* v = getenv("TRIT_HIP_NORM_WINDOW")) a.norm_window = (int)strtol(v, nullptr, 10);
    // Granite (the per-kernel loop's factors, causal_lm.rs:387,420,438-442,456).
    a.em = c.embedding_multiplier;
    a.q_scale = c.attention_multiplier != 0.0f ? c.attention_multiplier * sqrtf((float)HD) : 1.0f;
    a.rm = c.residual_multiplier;
    a.logit_w = 1.0f / c.logits_scaling;
    a.ffn_scales = D.has_ffn_scales ? D.ffn_scales.as<float>() : nullptr;
    a.additive = S.additive_rows ? S.additive.as<float>() : nullptr;
    a.additive_rows = S.additive_rows;
    a.stamp_step = g_stamp_step;
    a.stamp_layer = g_stamp_layer;
    a.local_qkv = p.local_qkv;
    // The XCD rank counters, zeroed for this launch.
    a.xcd_count = (unsigned int*)(w + sc_words(c, p) + (size_t)c.heads * T);
    if (p.local_qkv) TRIT_HIP(hipMemsetAsync(a.xcd_count, 0, NX * sizeof(unsigned int), s));
    void* args[] = {&a, &step, &pos, (void*)&seq0, &nsteps};
    // TRIT_HIP_STEP_LAUNCH=plain (measurement only: profilers that end badly
    // after cooperative launches): the same grid by an ordinary launch. One
    // block fits a CU (its LDS), so the grid of one block a CU is resident
    // on an otherwise idle device; were it not, the waits reach their
    // deadlines and the call fails.
    const char* how = getenv("TRIT_HIP_STEP_LAUNCH");
    if (how && std::string(how) == "plain")
        TRIT_HIP(hipLaunchKernel((const void*)p.fn, dim3(p.blocks), dim3(T), args, 0, s));
    else
        TRIT_HIP(hipLaunchCooperativeKernel((const void*)p.fn, dim3(p.blocks), dim3(T), args, 0, s));
}

}  // namespace trit

extern "C" {

int trit_hip_step_stamps(int step, int layer) {
    return trit::guard(-1, [&] {
#ifdef TRIT_HIP_STEP_STAMPS
        trit::g_stamp_step = step;
        trit::g_stamp_layer = layer;
        return 0;
#else
        (void)step;
        (void)layer;
        trit::fail("step stamps: this library was built without them (python -m trit_amd.build --stamps)");
        return -1;
#endif
    });
}

int trit_hip_step_stamps_read(uint64_t* wall, uint64_t* clock, int blocks) {
    return trit::guard(-1, [&] {
#ifdef TRIT_HIP_STEP_STAMPS
        if (!wall || !clock || blocks < 1 || blocks > trit::MAX_STAMP_BLOCKS) trit::fail("step stamps: bad arguments");
        const size_t bytes = (size_t)blocks * trit::NSTAMP * 8;
        TRIT_HIP(hipMemcpyFromSymbol(wall, HIP_SYMBOL(trit::g_stamp_wall), bytes, 0, hipMemcpyDeviceToHost));
        TRIT_HIP(hipMemcpyFromSymbol(clock, HIP_SYMBOL(trit::g_stamp_clk), bytes, 0, hipMemcpyDeviceToHost));
        return trit::NSTAMP;
#else
        (void)wall;
        (void)clock;
        (void)blocks;
        trit::fail("step stamps: this library was built without them (python -m trit_amd.build --stamps)");
        return -1;
#endif
    });
}

}  // extern "C"
