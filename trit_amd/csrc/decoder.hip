// The decoder half of the C ABI: CausalLm's token loop on the device
// (src/models/parts/causal_lm.rs:17-481).
//
// A session owns the key/value caches and the activations. Every kernel
// reads the cache position from device memory, so one decode step
// (argmax + stop check + embedding + 28 layers + head) is position-free and
// is captured once as a HIP graph, then replayed per token without a trip
// to the host. A `done` flag in device memory turns the rest of the replays
// into no-ops after a stop token or max_new tokens.
//
// Per layer and step: [RMSNorm factor] -> qkv product (RMSNorm and the
// activation quantizer fused in its prologue) -> q/k norm + RoPE + cache
// append -> attention -> o product (+ residual) -> [RMSNorm factor] ->
// gate_up product (SwiGLU fused in its epilogue) -> down product
// (+ residual). The bracketed kernels run in exact mode only: there the
// RMSNorm sum is Trit's serial chain; in fast mode each product block
// computes it with a fixed tree.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "../../include/trit_hip.h"
#include "decoder_impl.h"
#include "device.h"
#include "internal.h"

namespace trit {
namespace {

constexpr int MAX_HD = 256;
constexpr int ATT_THREADS = 256;


constexpr int CHOOSE_THREADS = 256;
constexpr int CHOOSE_SPAN = CHOOSE_THREADS * 4;  // logits per block

// ---- small kernels ----------------------------------------------------

// RMSNorm factor of each row with Trit's sum -- the squares added one
// after another from 0 (src/layers.rs:136-144) -- bit for bit, by the 8
// waves of a 512-thread block at once: wave w chains segment w (S values,
// zeros past d adding nothing) from 64 candidate starts, lane L from the
// float L - 32 steps from the tree estimate of the chain before the
// segment (within a few steps of it: each add of the chain rounds by at
// most half a step); the segments are then joined in order -- the lane
// whose start equals the chain so far holds the chain after the segment --
// and a segment whose true start no candidate within `window` steps holds
// is chained again from it.
constexpr int NI_THREADS = 512, NI_WAVES = NI_THREADS / 64;

__host__ __device__ inline int norm_inv_segment(int d) { return ((d + NI_WAVES - 1) / NI_WAVES + 3) & ~3; }

__global__ __launch_bounds__(NI_THREADS) void norm_inv_kernel(const float* __restrict__ x, int d, float eps,
                                                              float* __restrict__ inv, const State* st, int window) {
    if (st && st->done) return;
    extern __shared__ __align__(16) float sq[];  // S * NI_WAVES squares
    __shared__ float part[NI_WAVES];
    __shared__ float res[NI_WAVES][64];
    const int t = threadIdx.x, w = t / 64, lane = t % 64;
    const int S = norm_inv_segment(d);
    const float* row = x + (size_t)blockIdx.x * d;
    for (int i = t; i < S * NI_WAVES; i += NI_THREADS) {
        const float v = i < d ? row[i] : 0.0f;
        sq[i] = v * v;
    }
    __syncthreads();
    const float* seg = sq + S * w;
    float p = 0.0f;
    for (int i = lane; i < S; i += 64) p += seg[i];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) p += __shfl_xor(p, off);
    if (lane == 0) part[w] = p;
    __syncthreads();
    float est[NI_WAVES];
    est[0] = 0.0f;
#pragma unroll
    for (int q = 1; q < NI_WAVES; ++q) est[q] = est[q - 1] + part[q - 1];
    const auto cand = [&](int q) {
        const int off = lane - 32;
        if (q == 0) return 0.0f;
        if (off < -window || off > window) return __builtin_nanf("");
        const int bits = (int)__float_as_uint(est[q]) + off;
        return __uint_as_float((uint32_t)(bits < 0 ? 0 : bits));
    };
    float c = 0.0f;
#pragma unroll
    for (int q = 1; q < NI_WAVES; ++q)
        if (w == q) c = cand(q);  // (est[] indexed by constants: registers)
#pragma unroll 4
    for (int i = 0; i < S; i += 4) {
        const float4 v = *(const float4*)(seg + i);
        c = c + v.x;
        c = c + v.y;
        c = c + v.z;
        c = c + v.w;
    }
    res[w][lane] = c;
    __syncthreads();
    if (w != 0) return;
    float sum = __shfl(res[0][lane], 0);
    for (int q = 1; q < NI_WAVES; ++q) {
        const unsigned long long m = __ballot(cand(q) == sum);
        if (m) {
            sum = __shfl(res[q][lane], __builtin_ctzll(m));
        } else {
            for (int i = 0; i < S; ++i) sum = sum + sq[S * q + i];
        }
    }
    if (lane == 0) inv[blockIdx.x] = 1.0f / __builtin_sqrtf(sum / (float)d + eps);
}

// The candidate window (TRIT_HIP_NORM_WINDOW narrows it: tests of the path
// that chains a segment again; 0 leaves only the estimate, -1 none).
int norm_window() {
    const char* v = getenv("TRIT_HIP_NORM_WINDOW");
    return v && *v ? (int)strtol(v, nullptr, 10) : 31;
}

void launch_norm_inv(const float* x, int rows, int d, float eps, float* inv, const State* st, hipStream_t s) {
    hipLaunchKernelGGL(norm_inv_kernel, dim3(rows), dim3(NI_THREADS), (size_t)norm_inv_segment(d) * NI_WAVES * 4, s,
                       x, d, eps, inv, st, norm_window());
}

// out = x * (inv * w), inv from `inv` (exact) or a fixed tree (fast); then,
// with `scale`, out *= scale (the MLP scales, causal_lm.rs:458-464).
__global__ void rmsnorm_kernel(const float* __restrict__ x, int d, const float* __restrict__ w, float eps,
                               const float* __restrict__ inv_in, float* __restrict__ out, const State* st,
                               const float* __restrict__ scale = nullptr) {
    if (st && st->done) return;
    __shared__ float red[256];
    __shared__ float inv_s;
    const float* row = x + (size_t)blockIdx.x * d;
    if (inv_in) {
        if (threadIdx.x == 0) inv_s = inv_in[blockIdx.x];
    } else {
        float part = 0.0f;
        for (int i = threadIdx.x; i < d; i += 256) {
            const float v = row[i];
            part += v * v;
        }
        red[threadIdx.x] = part;
        __syncthreads();
        for (int s = 128; s > 0; s >>= 1) {
            if ((int)threadIdx.x < s) red[threadIdx.x] += red[threadIdx.x + s];
            __syncthreads();
        }
        if (threadIdx.x == 0) inv_s = 1.0f / __builtin_sqrtf(red[0] / (float)d + eps);
    }
    __syncthreads();
    const float inv = inv_s;
    for (int i = threadIdx.x; i < d; i += 256) {
        float v = row[i] * (inv * w[i]);
        if (scale) v = v * scale[i];
        out[(size_t)blockIdx.x * d + i] = v;
    }
}

// x *= w (scale_all, src/layers.rs:219-223; the caller skips w == 1).
__global__ void scale_kernel(float* __restrict__ x, int n, float w, const State* st) {
    if (st && st->done) return;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) x[i] = x[i] * w;
}

// The first qd values (q) of each row of the qkv product times w, after
// the rotary (causal_lm.rs:438-442).
__global__ void scale_q_kernel(float* __restrict__ qkv, int stride, int rows, int qd, float w, const State* st) {
    if (st && st->done) return;
    const int n = rows * qd;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        float* v = qkv + (size_t)(i / qd) * stride + i % qd;
        *v = *v * w;
    }
}

// x += w * y, two roundings (add_scaled_into, src/layers.rs:226-236, for
// w != 1).
__global__ void add_scaled_kernel(float* __restrict__ x, const float* __restrict__ y, int n, float w,
                                  const State* st) {
    if (st && st->done) return;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) x[i] = x[i] + w * y[i];
}

// x += rows of `add` (add_into, src/layers.rs:245-252): the n x d rows at `add`, or
// with `by_pos` the one row at position st->pos (a decode step's input).
__global__ void add_rows_kernel(float* __restrict__ x, const float* __restrict__ add, int n, int d, int by_pos,
                                const State* st) {
    if (st->done) return;
    const float* a = by_pos ? add + (size_t)st->pos * d : add;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) x[i] = x[i] + a[i];
}

// A token table in the lane-chain layout (f16 bits, f32, or int8 codes
// with f32 scales n x k/32).
struct TableRef {
    int kind;
    const void* codes;
    const float* scales;
};

TableRef table_ref(const Layer& L) { return TableRef{L.kind, L.codes.ptr, L.scales.as<float>()}; }

// Value kk of row `token` as f32 (Dense::row, src/cpu/gemm.rs:412-429; Q8:
// f32(code) * scale, widen_q8 :171-179).
__device__ __forceinline__ float table_value(const TableRef& t, int token, int kk, int k) {
    const int s_count = k / 16;
    const size_t at = ((size_t)token * 16 + (kk & 15)) * s_count + (kk >> 4);
    if (t.kind == F16) return f16_to_f32(((const uint16_t*)t.codes)[at]);
    if (t.kind == F32) return ((const float*)t.codes)[at];
    return (float)((const int8_t*)t.codes)[at] * t.scales[(size_t)token * (k / 32) + kk / 32];
}

// Embedding rows of `tokens` (or of st->token when tokens is null).
__global__ void embed_kernel(TableRef table, int k, const int* __restrict__ tokens, float* __restrict__ x,
                             const State* st) {
    if (st->done) return;
    const int token = tokens ? tokens[blockIdx.x] : st->token;
    for (int kk = threadIdx.x; kk < k; kk += blockDim.x) x[(size_t)blockIdx.x * k + kk] = table_value(table, token, kk, k);
}

// SwiGLU of the stacked gate_up product's rows (2 * ffn wide): h = silu(gate)
// * up (causal_lm.rs:464-473), for float-math gate_up layers.
__global__ void silu_pair_kernel(const float* __restrict__ wide, int rows, int ffn, float* __restrict__ h,
                                 const State* st) {
    if (st && st->done) return;
    const int n = rows * ffn;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        const int r = i / ffn, j = i - r * ffn;
        h[i] = silu_trit(wide[(size_t)r * 2 * ffn + j]) * wide[(size_t)r * 2 * ffn + ffn + j];
    }
}

// Per (row, head) of the qkv product: Qwen3's per-head RMSNorm of q and k
// (serial sums, causal_lm.rs:428-433), the rotary halves at the row's
// position (src/layers.rs:303-334, no fused steps), then k and v appended
// to the caches at that position (causal_lm.rs:443-446); q is rotated in
// place. Heads: [0, heads) q, [heads, heads+kvh) k, then v.
template <typename KV>
__global__ void qk_rope_kernel(float* __restrict__ qkv, int stride, int heads, int kvh, int hd, int qk_norm,
                               const float* __restrict__ q_norm, const float* __restrict__ k_norm, float eps,
                               const float* __restrict__ rope_sin, const float* __restrict__ rope_cos,
                               KV* __restrict__ kcache, KV* __restrict__ vcache, int max_pos,
                               const State* st) {
    if (st->done) return;
    __shared__ float v[MAX_HD];
    __shared__ float inv_s;
    const int row = blockIdx.x / (heads + 2 * kvh);
    const int head = blockIdx.x % (heads + 2 * kvh);
    const int e = threadIdx.x;
    const int pos = st->pos + row;
    float* src = qkv + (size_t)row * stride + (size_t)head * hd;
    const bool is_q = head < heads, is_k = !is_q && head < heads + kvh;
    if (e < hd) v[e] = src[e];
    __syncthreads();
    if (qk_norm && (is_q || is_k)) {
        __shared__ __align__(16) float sq[MAX_HD];
        if (e < hd) sq[e] = v[e] * v[e];
        __syncthreads();
        if (e == 0) {
            // Trit's serial sum of the rounded squares (src/layers.rs:139).
            float sum = 0.0f;
            for (int i = 0; i < hd; i += 4) {
                const float4 q4 = *(const float4*)(sq + i);
                sum = sum + q4.x;
                sum = sum + q4.y;
                sum = sum + q4.z;
                sum = sum + q4.w;
            }
            inv_s = 1.0f / __builtin_sqrtf(sum / (float)hd + eps);
        }
        __syncthreads();
        const float* w = is_q ? q_norm : k_norm;
        float t = 0.0f;
        if (e < hd) t = v[e] * (inv_s * w[e]);
        __syncthreads();
        if (e < hd) v[e] = t;
        __syncthreads();
    }
    float out = 0.0f;
    if (e < hd) {
        out = v[e];
        if (is_q || is_k) {
            const int half = hd / 2;
            const int i = e < half ? e : e - half;
            const float s = rope_sin[(size_t)pos * half + i], c = rope_cos[(size_t)pos * half + i];
            if (e < half) {
                const float a = v[e], b = v[e + half];
                const float ac = a * c, bs = b * s;
                out = ac - bs;
            } else {
                const float a = v[e - half], b = v[e];
                const float bc = b * c, as = a * s;
                out = bc + as;
            }
        }
    }
    if (e < hd) {
        if (is_q) {
            src[e] = out;
        } else {
            const int g = is_k ? head - heads : head - heads - kvh;
            KV* cache = is_k ? kcache : vcache;
            cache[((size_t)g * max_pos + pos) * hd + e] = (KV)out;
        }
    }
}

// Fast mode, head_dim 128: the same step with one wave per (row, head),
// lane i holding dims i and i + 64 (a rotary pair), the norm's sum a DPP
// tree (fast mode: tree sums) -- four heads a 256-thread block instead of
// a block a head with a serial sum.
template <typename KV>
__global__ __launch_bounds__(256) void qk_rope_wave_kernel(float* __restrict__ qkv, int stride, int rows, int heads,
                                                            int kvh, int qk_norm, const float* __restrict__ q_norm,
                                                            const float* __restrict__ k_norm, float eps,
                                                            const float* __restrict__ rope_sin,
                                                            const float* __restrict__ rope_cos,
                                                            KV* __restrict__ kcache, KV* __restrict__ vcache,
                                                            int max_pos, const State* st) {
    constexpr int HD = 128, HALF = 64;
    if (st->done) return;
    const int per_row = heads + 2 * kvh;
    const int item = (int)(blockIdx.x * (blockDim.x / WAVE) + threadIdx.x / WAVE);
    if (item >= rows * per_row) return;  // a whole wave
    const int row = item / per_row, head = item % per_row, lane = threadIdx.x % WAVE;
    const int pos = st->pos + row;
    float* src = qkv + (size_t)row * stride + (size_t)head * HD;
    const bool is_q = head < heads, is_k = !is_q && head < heads + kvh;
    float x0 = src[lane], x1 = src[lane + HALF];
    if (is_q || is_k) {
        if (qk_norm) {
            float sq = x0 * x0 + x1 * x1;
            sq += dpp<DPP_XOR1>(sq);
            sq += dpp<DPP_XOR2>(sq);
            sq += dpp<DPP_HALF_MIRROR>(sq);
            sq += dpp<DPP_MIRROR>(sq);
            const float sum = (__shfl(sq, 0) + __shfl(sq, 16)) + (__shfl(sq, 32) + __shfl(sq, 48));
            const float inv = 1.0f / __builtin_sqrtf(sum / (float)HD + eps);
            const float* w = is_q ? q_norm : k_norm;
            x0 = x0 * (inv * w[lane]);
            x1 = x1 * (inv * w[lane + HALF]);
        }
        const float sn = rope_sin[(size_t)pos * HALF + lane], cs = rope_cos[(size_t)pos * HALF + lane];
        const float a = x0, b = x1;
        x0 = a * cs - b * sn;
        x1 = b * cs + a * sn;
    }
    if (is_q) {
        src[lane] = x0;
        src[lane + HALF] = x1;
    } else {
        const int g = is_k ? head - heads : head - heads - kvh;
        KV* cache = (is_k ? kcache : vcache) + ((size_t)g * max_pos + pos) * HD;
        cache[lane] = (KV)x0;
        cache[lane + HALF] = (KV)x1;
    }
}

__device__ __forceinline__ float kv_load(const float* p) { return *p; }
__device__ __forceinline__ float kv_load(const _Float16* p) { return (float)*p; }

// Eight consecutive cache values (16- or 32-byte aligned) as f32.
__device__ __forceinline__ void kv_load8(const float* p, float* out) {
    const float4 a = ((const float4*)p)[0], b = ((const float4*)p)[1];
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
    out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
}
template <typename KV>
__device__ __forceinline__ void kv_unpack8(const uint4* u, float* out);
template <>
__device__ __forceinline__ void kv_unpack8<float>(const uint4* u, float* out) {
    const uint4 a = u[0], b = u[1];
    out[0] = __uint_as_float(a.x); out[1] = __uint_as_float(a.y); out[2] = __uint_as_float(a.z); out[3] = __uint_as_float(a.w);
    out[4] = __uint_as_float(b.x); out[5] = __uint_as_float(b.y); out[6] = __uint_as_float(b.z); out[7] = __uint_as_float(b.w);
}
template <>
__device__ __forceinline__ void kv_unpack8<_Float16>(const uint4* u, float* out) {
    const uint32_t w[4] = {u[0].x, u[0].y, u[0].z, u[0].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        out[2 * i] = f16_to_f32((uint16_t)(w[i] & 0xffff));
        out[2 * i + 1] = f16_to_f32((uint16_t)(w[i] >> 16));
    }
}

__device__ __forceinline__ void kv_load8(const _Float16* p, float* out) {
    const uint4 v = *(const uint4*)p;
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        out[2 * i] = f16_to_f32((uint16_t)(w[i] & 0xffff));
        out[2 * i + 1] = f16_to_f32((uint16_t)(w[i] >> 16));
    }
}

// Attention of row `row` of this forward for query head blockIdx.x over
// the cache (src/layers.rs:442-504,571-587 with the AVX-512 orders): qh =
// q * (1/sqrt(hd)); score_j = fused chain over e from 0; keys past the
// row's position are -inf; max; e_j = exp(s_j - max); sum over j (serial
// in exact mode); p_j = e_j * (1/sum); out_e = fused chain of p_j * v_je
// over every key of the forward, from 0.
template <typename KV>
__global__ __launch_bounds__(ATT_THREADS) void attention_kernel(
    const float* __restrict__ qkv, int stride, int heads, int kvh, int hd, const KV* __restrict__ kcache,
    const KV* __restrict__ vcache, int max_pos, int rows, float* __restrict__ out, int exact, const State* st,
    int causal = 1) {
    if (st->done) return;
    extern __shared__ float sm[];  // qh[hd] | probs[tk] | red[ATT_THREADS]
    const int h = blockIdx.x;
    const int row = blockIdx.y;
    const int g = h / (heads / kvh);
    const int tk = st->pos + rows;       // keys in the caches for this forward
    const int visible = causal ? st->pos + row + 1 : tk;
    float* qh = sm;
    float* probs = sm + MAX_HD;
    float* red = probs + tk;
    const float scale = 1.0f / __builtin_sqrtf((float)hd);
    const float* q = qkv + (size_t)row * stride + (size_t)h * hd;
    for (int e = threadIdx.x; e < hd; e += ATT_THREADS) qh[e] = q[e] * scale;
    __syncthreads();
    const KV* K = kcache + (size_t)g * max_pos * hd;
    const KV* V = vcache + (size_t)g * max_pos * hd;
    float best = -INFINITY;
    for (int j = threadIdx.x; j < tk; j += ATT_THREADS) {
        float acc = 0.0f;
        if (j < visible) {
            const KV* kr = K + (size_t)j * hd;
            for (int e = 0; e < hd; e += 8) {
                float kv[8];
                kv_load8(kr + e, kv);
#pragma unroll
                for (int u = 0; u < 8; ++u) acc = __builtin_fmaf(qh[e + u], kv[u], acc);
            }
        } else {
            acc = -INFINITY;
        }
        probs[j] = acc;
        best = __builtin_fmaxf(best, acc);
    }
    red[threadIdx.x] = best;
    __syncthreads();
    for (int s = ATT_THREADS / 2; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) red[threadIdx.x] = __builtin_fmaxf(red[threadIdx.x], red[threadIdx.x + s]);
        __syncthreads();
    }
    const float mx = red[0];
    __syncthreads();
    float part = 0.0f;
    for (int j = threadIdx.x; j < tk; j += ATT_THREADS) {
        const float e = exp_trit(probs[j] - mx);
        probs[j] = e;
        part += e;
    }
    red[threadIdx.x] = part;
    __syncthreads();
    if (exact) {
        if (threadIdx.x == 0) {
            float sum = 0.0f;
            int j = 0;
            for (; j + 4 <= tk; j += 4) {
                const float4 p4 = *(const float4*)(probs + j);
                sum = sum + p4.x;
                sum = sum + p4.y;
                sum = sum + p4.z;
                sum = sum + p4.w;
            }
            for (; j < tk; ++j) sum = sum + probs[j];
            red[0] = sum;
        }
        __syncthreads();
    } else {
        for (int s = ATT_THREADS / 2; s > 0; s >>= 1) {
            if ((int)threadIdx.x < s) red[threadIdx.x] += red[threadIdx.x + s];
            __syncthreads();
        }
    }
    const float inv = 1.0f / red[0];
    __syncthreads();
    for (int j = threadIdx.x; j < tk; j += ATT_THREADS) probs[j] = probs[j] * inv;
    __syncthreads();
    for (int e = threadIdx.x; e < hd; e += ATT_THREADS) {
        float acc = 0.0f;
        int j = 0;
        for (; j + 16 <= tk; j += 16) {
            float v[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) v[u] = kv_load(V + (size_t)(j + u) * hd + e);
#pragma unroll
            for (int u = 0; u < 16; ++u) acc = __builtin_fmaf(probs[j + u], v[u], acc);
        }
        for (; j < tk; ++j) acc = __builtin_fmaf(probs[j], kv_load(V + (size_t)j * hd + e), acc);
        out[(size_t)row * heads * hd + (size_t)h * hd + e] = acc;
    }
}

// Keys per block of the split attention: 64 with f16 caches, 32 with f32,
// so the staged chunk of keys and values is 32 KB either way.
template <typename KV>
struct Split {
    static constexpr int CH = sizeof(KV) == 2 ? 64 : 32;
};

// Qwen3's per-head RMSNorm (serial sum of the rounded squares, as
// src/layers.rs:139) and the rotary halves (src/layers.rs:303-334) of one
// head held in LDS `v` (hd values), by the block's first hd threads.
__device__ void norm_rope_head(float* v, float* sq, const float* w, int hd, float eps, const float* sn,
                               const float* cs, bool norm, bool rope, float* inv_slot) {
    const int e = threadIdx.x;
    if (norm) {
        if (e < hd) sq[e] = v[e] * v[e];
        __syncthreads();
        if (e == 0) {
            float sum = 0.0f;
            for (int i = 0; i < hd; i += 4) {
                const float4 q4 = *(const float4*)(sq + i);
                sum = sum + q4.x;
                sum = sum + q4.y;
                sum = sum + q4.z;
                sum = sum + q4.w;
            }
            *inv_slot = 1.0f / __builtin_sqrtf(sum / (float)hd + eps);
        }
        __syncthreads();
        float t = 0.0f;
        if (e < hd) t = v[e] * (*inv_slot * w[e]);
        __syncthreads();
        if (e < hd) v[e] = t;
        __syncthreads();
    }
    if (rope) {
        const int half = hd / 2;
        float out = 0.0f;
        if (e < hd) {
            const int i = e < half ? e : e - half;
            const float s_ = sn[i], c = cs[i];
            if (e < half) {
                const float ac = v[e] * c, bs = v[e + half] * s_;
                out = ac - bs;
            } else {
                const float bc = v[e] * c, as = v[e - half] * s_;
                out = bc + as;
            }
        }
        __syncthreads();
        if (e < hd) v[e] = out;
        __syncthreads();
    }
}

// Fast-mode attention (split over the keys, "flash decoding"): block
// (g, split, row) stages keys and values [split*CH, split*CH+CH) of
// key/value head g in LDS with one round of 16-byte loads, scores them
// against the query heads that share g (16 lanes per dot product, DPP
// sums), takes the chunk's softmax with one wave per query head, and keeps
// the chunk's maximum, sum of exp(s - max) and unnormalised p.V. The last
// block of (row, g) merges the chunks with the usual rescaling. Keys past
// the row's position get no weight. The sums run in parallel, so the values
// are within rounding of the exact kernel's, not equal to them.
//
// FUSED (one decode row): the block also does the q/k norm and rotary of
// its heads from the raw qkv product, and the block whose chunk holds the
// new position appends that key and value to the caches.
template <typename KV, bool FUSED>
__global__ __launch_bounds__(ATT_THREADS) void attention_split_kernel(
    const float* __restrict__ qkv, int stride, int heads, int kvh, int hd, KV* __restrict__ kcache,
    KV* __restrict__ vcache, int max_pos, int rows, float* __restrict__ out, float* __restrict__ part,
    unsigned int* __restrict__ arrived, int max_splits, const State* st, int qk_norm,
    const float* __restrict__ q_norm, const float* __restrict__ k_norm, float eps,
    const float* __restrict__ rope_sin, const float* __restrict__ rope_cos) {
    constexpr int CH = Split<KV>::CH;
    constexpr int PER = 16 / sizeof(KV);  // cache values per 16-byte load
    if (st->done) return;
    extern __shared__ __align__(16) char smem[];
    KV* Ks = (KV*)smem;
    KV* Vs = Ks + CH * hd;
    __shared__ __align__(16) float qh[4 * 128];
    __shared__ __align__(16) float kv_new[2][128];
    __shared__ __align__(16) float sq[128];
    __shared__ float inv_slot;
    __shared__ float sc[4][CH];
    __shared__ float mrow[4], lrow[4];
    __shared__ bool last;
    const int g = blockIdx.x, split = blockIdx.y, row = blockIdx.z;
    const int group = heads / kvh;
    const int pos = st->pos;
    const int tk = pos + rows;
    const int visible = pos + row + 1;
    const int j0 = split * CH;
    const int splits = (tk + CH - 1) / CH;
    if (split >= splits) return;
    const int nk = min(CH, tk - j0);
    // With FUSED, the new position is not in the cache yet: stage one key less.
    const int nstage = FUSED && split == splits - 1 ? nk - 1 : nk;
    const uint4* K = (const uint4*)(kcache + ((size_t)g * max_pos + j0) * hd);
    const uint4* V = (const uint4*)(vcache + ((size_t)g * max_pos + j0) * hd);
    const int units = nstage * hd / PER;
    constexpr int UPT = CH * 128 / (16 / (int)sizeof(KV)) / ATT_THREADS;
    uint4 kr[UPT], vr[UPT];
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
        // Past the staged keys, re-read the first unit (in bounds); the store skips it.
        const int u = (int)threadIdx.x + i * ATT_THREADS;
        const int uc = u < units ? u : 0;
        kr[i] = K[uc];
        vr[i] = V[uc];
    }
    const float scale = 1.0f / __builtin_sqrtf((float)hd);
    const float* qsrc = qkv + (size_t)row * stride;
    const bool holds_new = FUSED && split == splits - 1;
    // The raw q (and new k, v) values this thread needs, fetched with the chunk.
    const int t = threadIdx.x;
    float qreg[4] = {0.0f, 0.0f, 0.0f, 0.0f}, kreg = 0.0f, vreg = 0.0f;
    if (t < hd) {
#pragma unroll
        for (int hl = 0; hl < 4; ++hl)
            if (hl < group) qreg[hl] = qsrc[(size_t)(g * group + hl) * hd + t];
        if (holds_new) {
            kreg = qsrc[(size_t)(heads + g) * hd + t];
            vreg = qsrc[(size_t)(heads + kvh + g) * hd + t];
        }
    }
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
        const int u = t + i * ATT_THREADS;
        if (u < units) {
            ((uint4*)Ks)[u] = kr[i];
            ((uint4*)Vs)[u] = vr[i];
        }
    }
    for (int u = t + UPT * ATT_THREADS; u < units; u += ATT_THREADS) {
        ((uint4*)Ks)[u] = K[u];
        ((uint4*)Vs)[u] = V[u];
    }
    if (FUSED) {
        const float* sn = rope_sin + (size_t)pos * (hd / 2);
        const float* cs = rope_cos + (size_t)pos * (hd / 2);
        for (int hl = 0; hl < group; ++hl) {
            float* v = qh + hl * hd;
            if (t < hd) v[t] = qreg[hl];
            __syncthreads();
            norm_rope_head(v, sq, q_norm, hd, eps, sn, cs, qk_norm != 0, true, &inv_slot);
        }
        if (holds_new) {
            float* kn = kv_new[0];
            if (t < hd) kn[t] = kreg;
            __syncthreads();
            norm_rope_head(kn, sq, k_norm, hd, eps, sn, cs, qk_norm != 0, true, &inv_slot);
            if (t < hd) {
                const size_t at = ((size_t)g * max_pos + pos) * hd + t;
                const KV kq = (KV)kn[t], vq = (KV)vreg;
                kcache[at] = kq;
                vcache[at] = vq;
                // The new key and value, rounded as the cache holds them.
                Ks[(size_t)nstage * hd + t] = kq;
                Vs[(size_t)nstage * hd + t] = vq;
            }
        }
        for (int i = t; i < group * hd; i += ATT_THREADS) qh[i] = qh[i] * scale;
    } else {
        for (int i = t; i < group * hd; i += ATT_THREADS) {
            const int h = g * group + i / hd;
            qh[i] = qsrc[(size_t)h * hd + i % hd] * scale;
        }
    }
    __syncthreads();
    // Scores: 16 lanes per (head, key), 8 dims per lane and step.
    const int lane16 = threadIdx.x & 15;
    for (int pi = threadIdx.x >> 4; pi < group * CH; pi += ATT_THREADS / 16) {
        const int hl = pi / CH, j = pi % CH;
        float acc = 0.0f;
        if (j < nk) {
            const float* q = qh + hl * hd;
            for (int e = lane16 * 8; e < hd; e += 128) {
                float kv[8];
                kv_load8(Ks + (size_t)j * hd + e, kv);
#pragma unroll
                for (int u = 0; u < 8; ++u) acc = __builtin_fmaf(q[e + u], kv[u], acc);
            }
        }
        acc += dpp<DPP_XOR1>(acc);
        acc += dpp<DPP_XOR2>(acc);
        acc += dpp<DPP_HALF_MIRROR>(acc);
        acc += dpp<DPP_MIRROR>(acc);
        if (lane16 == 0) sc[hl][j] = (j < nk && j0 + j < visible) ? acc : -INFINITY;
    }
    __syncthreads();
    // The chunk's softmax, one wave per query head: lane j holds key j (and j+64).
    {
        const int w = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
        if (w < group) {
            const float a = lane < CH ? sc[w][lane] : -INFINITY;
            const float b = lane + WAVE < CH ? sc[w][lane + WAVE] : -INFINITY;
            float mx = __builtin_fmaxf(a, b);
            mx = __builtin_fmaxf(mx, dpp<DPP_XOR1>(mx));
            mx = __builtin_fmaxf(mx, dpp<DPP_XOR2>(mx));
            mx = __builtin_fmaxf(mx, dpp<DPP_HALF_MIRROR>(mx));
            mx = __builtin_fmaxf(mx, dpp<DPP_MIRROR>(mx));
            mx = __builtin_fmaxf(__builtin_fmaxf(__shfl(mx, 0), __shfl(mx, 16)),
                                 __builtin_fmaxf(__shfl(mx, 32), __shfl(mx, 48)));
            const float ea = a == -INFINITY ? 0.0f : exp_trit(a - mx);
            const float eb = b == -INFINITY ? 0.0f : exp_trit(b - mx);
            if (lane < CH) sc[w][lane] = ea;
            if (lane + WAVE < CH) sc[w][lane + WAVE] = eb;
            float l = ea + eb;
            l += dpp<DPP_XOR1>(l);
            l += dpp<DPP_XOR2>(l);
            l += dpp<DPP_HALF_MIRROR>(l);
            l += dpp<DPP_MIRROR>(l);
            l = (__shfl(l, 0) + __shfl(l, 16)) + (__shfl(l, 32) + __shfl(l, 48));
            if (lane == 0) {
                mrow[w] = mx;
                lrow[w] = l;
            }
        }
    }
    __syncthreads();
    const size_t slot = ((size_t)row * heads + g * group) * max_splits;
    for (int t = threadIdx.x; t < group * hd; t += ATT_THREADS) {
        const int hl = t / hd, e = t % hd;
        float acc = 0.0f;
        int j = 0;
        for (; j + 8 <= nk; j += 8) {
            float vv[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) vv[u] = kv_load(Vs + (size_t)(j + u) * hd + e);
#pragma unroll
            for (int u = 0; u < 8; ++u) acc = __builtin_fmaf(sc[hl][j + u], vv[u], acc);
        }
        for (; j < nk; ++j) acc = __builtin_fmaf(sc[hl][j], kv_load(Vs + (size_t)j * hd + e), acc);
        if (splits == 1) {
            out[(size_t)row * heads * hd + (size_t)(g * group + hl) * hd + e] = acc / lrow[hl];
            continue;
        }
        float* p = part + (slot + (size_t)hl * max_splits + split) * (hd + 2);
        p[2 + e] = acc;
        if (e == 0) {
            p[0] = mrow[hl];
            p[1] = lrow[hl];
        }
    }
    if (splits == 1) return;
    __syncthreads();
    if (threadIdx.x == 0) {
        __threadfence();
        unsigned int* ctr = arrived + (size_t)row * kvh + g;
        last = atomicAdd(ctr, 1u) == (unsigned)splits - 1;
        if (last) *ctr = 0;
    }
    __syncthreads();
    if (!last) return;
    __threadfence();
    for (int t = threadIdx.x; t < group * hd; t += ATT_THREADS) {
        const int hl = t / hd, e = t % hd;
        const float* base = part + (slot + (size_t)hl * max_splits) * (hd + 2);
        float M = -INFINITY;
        for (int s2 = 0; s2 < splits; ++s2) M = __builtin_fmaxf(M, base[(size_t)s2 * (hd + 2)]);
        float L = 0.0f, O = 0.0f;
        for (int s2 = 0; s2 < splits; ++s2) {
            const float* p = base + (size_t)s2 * (hd + 2);
            if (p[0] == -INFINITY) continue;
            const float w = exp_trit(p[0] - M);
            L = __builtin_fmaf(p[1], w, L);
            O = __builtin_fmaf(p[2 + e], w, O);
        }
        out[(size_t)row * heads * hd + (size_t)(g * group + hl) * hd + e] = O / L;
    }
}

constexpr int DEC_THREADS = 512;
constexpr int DEC_GROUPS = DEC_THREADS / 16;  // 16-lane groups, one key row each at a time

// Fast-mode attention of one decode row, one block per key/value head g,
// every key in one round of loads. 16-lane group G holds keys G, G+32,
// G+64, ... straight from the caches, lane l16 dims [8*l16, 8*l16+8) of
// each: the dot products against the query heads of g reduce over the 16
// lanes by DPP, the softmax and p.V reduce over the block through LDS, so
// nothing goes back to memory between the scores and the output. The block
// also does the q/k norm and rotary of its heads and appends the new key
// and value (src/models/parts/causal_lm.rs:428-446). The sums run in
// parallel: values within rounding of the exact kernel's.
template <typename KV, int MAXI, int GROUP>  // MAXI: keys per group (at most 32*MAXI keys); GROUP: q heads per kv head
__global__ __launch_bounds__(DEC_THREADS) void attention_decode_kernel(
    const float* __restrict__ qkv, int heads, int kvh, int hd, KV* __restrict__ kcache, KV* __restrict__ vcache,
    int max_pos, float* __restrict__ out, const State* st, int qk_norm, const float* __restrict__ q_norm,
    const float* __restrict__ k_norm, float eps, const float* __restrict__ rope_sin,
    const float* __restrict__ rope_cos) {
    if (st->done) return;
    __shared__ __align__(16) float qh[4 * 128];
    __shared__ __align__(16) float kv_new[2][128];
    __shared__ __align__(16) float sq[4][128];
    __shared__ float inv_s[4];
    __shared__ float red[DEC_THREADS / WAVE][4];
    __shared__ float stat[2][4];
    __shared__ __align__(16) float part[DEC_THREADS / WAVE][4 * 128];
    const int g = blockIdx.x;
    constexpr int group = GROUP;
    const int pos = st->pos;
    const int tk = pos + 1;
    const int t = threadIdx.x;
    const int G = t >> 4, l16 = t & 15;
    const bool dims = l16 * 8 < hd;
    const KV* K = kcache + (size_t)g * max_pos * hd;
    const KV* V = vcache + (size_t)g * max_pos * hd;
    constexpr int PER = 16 / (int)sizeof(KV);  // values per 16 bytes
    constexpr int U = 8 / PER;                  // 16-byte loads per 8 values
    // Every key this lane holds, and the raw q / new k, v and norm values.
    uint4 kr[MAXI][U], vr[MAXI][U];
#pragma unroll
    for (int i = 0; i < MAXI; ++i) {
        const int j = G + DEC_GROUPS * i;
        const int jc = (j < pos && dims) ? j : 0;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            kr[i][u] = ((const uint4*)(K + (size_t)jc * hd + l16 * 8))[u];
            vr[i][u] = ((const uint4*)(V + (size_t)jc * hd + l16 * 8))[u];
        }
    }
    const float* src = qkv;
    const int hh = t / hd, e = t % hd;  // threads [0, (group+1)*hd): q heads, then k
    float raw = 0.0f, vraw = 0.0f, nw = 1.0f, sn = 0.0f, cs = 1.0f;
    if (hh < group + 1) {
        raw = hh < group ? src[(size_t)(g * group + hh) * hd + e] : src[(size_t)(heads + g) * hd + e];
        if (hh == group) vraw = src[(size_t)(heads + kvh + g) * hd + e];
        nw = qk_norm ? (hh < group ? q_norm[e] : k_norm[e]) : 1.0f;
        const int half = hd / 2;
        sn = rope_sin[(size_t)pos * half + (e % half)];
        cs = rope_cos[(size_t)pos * half + (e % half)];
    }
    // q and k: Trit's per-head norm (serial sum), then the rotary halves.
    float* vv = hh < group ? qh + hh * hd : kv_new[0];
    if (hh < group + 1) {
        vv[e] = raw;
        sq[hh][e] = raw * raw;
    }
    __syncthreads();
    if (qk_norm && e == 0 && hh < group + 1) {
        float sum = 0.0f;
        for (int i = 0; i < hd; i += 4) {
            const float4 q4 = *(const float4*)(&sq[hh][i]);
            sum = sum + q4.x;
            sum = sum + q4.y;
            sum = sum + q4.z;
            sum = sum + q4.w;
        }
        inv_s[hh] = 1.0f / __builtin_sqrtf(sum / (float)hd + eps);
    }
    __syncthreads();
    float nv = raw;
    if (hh < group + 1 && qk_norm) nv = raw * (inv_s[hh] * nw);
    __syncthreads();
    if (hh < group + 1) vv[e] = nv;
    __syncthreads();
    float rot = 0.0f;
    if (hh < group + 1) {
        const int half = hd / 2;
        if (e < half) {
            const float ac = vv[e] * cs, bs = vv[e + half] * sn;
            rot = ac - bs;
        } else {
            const float bc = vv[e] * cs, as = vv[e - half] * sn;
            rot = bc + as;
        }
    }
    __syncthreads();
    const float scale = 1.0f / __builtin_sqrtf((float)hd);
    if (hh < group) qh[hh * hd + e] = rot * scale;
    if (hh == group) {
        const KV kq = (KV)rot, vq = (KV)vraw;
        kcache[((size_t)g * max_pos + pos) * hd + e] = kq;
        vcache[((size_t)g * max_pos + pos) * hd + e] = vq;
        kv_new[0][e] = (float)kq;
        kv_new[1][e] = (float)vq;
    }
    __syncthreads();
    // The new key and value replace the lane's stale copy of position pos.
    float q[GROUP][8];
#pragma unroll
    for (int hl = 0; hl < GROUP; ++hl)
#pragma unroll
        for (int u = 0; u < 8; ++u) q[hl][u] = (dims) ? qh[hl * hd + l16 * 8 + u] : 0.0f;
    float kn[8], vn[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        kn[u] = dims ? kv_new[0][l16 * 8 + u] : 0.0f;
        vn[u] = dims ? kv_new[1][l16 * 8 + u] : 0.0f;
    }
    // Scores.
    float sc[MAXI][GROUP];
    float mx[GROUP];
#pragma unroll
    for (int hl = 0; hl < GROUP; ++hl) mx[hl] = -INFINITY;
#pragma unroll
    for (int i = 0; i < MAXI; ++i) {
        const int j = G + DEC_GROUPS * i;
        float k8[8];
        if (j == pos) {
#pragma unroll
            for (int u = 0; u < 8; ++u) k8[u] = kn[u];
        } else {
            kv_unpack8<KV>(kr[i], k8);
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
            sc[i][hl] = j < tk ? acc : -INFINITY;
            mx[hl] = __builtin_fmaxf(mx[hl], sc[i][hl]);
        }
    }
    // Block maximum per head: rows of 16 lanes agree; combine the 4 rows of
    // each wave, then the waves.
    const int wave = t / WAVE, wl = t % WAVE;
#pragma unroll
    for (int hl = 0; hl < GROUP; ++hl) {
        float m = mx[hl];
        m = __builtin_fmaxf(__builtin_fmaxf(__shfl(m, 0), __shfl(m, 16)), __builtin_fmaxf(__shfl(m, 32), __shfl(m, 48)));
        if (wl == 0) red[wave][hl] = m;
    }
    __syncthreads();
    if (t < GROUP) {
        float m = -INFINITY;
        for (int w = 0; w < DEC_THREADS / WAVE; ++w) m = __builtin_fmaxf(m, red[w][t]);
        stat[0][t] = m;
    }
    __syncthreads();
    float l[GROUP];
#pragma unroll
    for (int hl = 0; hl < GROUP; ++hl) l[hl] = 0.0f;
#pragma unroll
    for (int i = 0; i < MAXI; ++i)
#pragma unroll
        for (int hl = 0; hl < GROUP; ++hl) {
            const float p = sc[i][hl] == -INFINITY ? 0.0f : exp_trit(sc[i][hl] - stat[0][hl]);
            sc[i][hl] = p;
            l[hl] += p;
        }
    // p.V over this lane's keys, then the block sums.
    float acc[GROUP][8];
#pragma unroll
    for (int hl = 0; hl < GROUP; ++hl)
#pragma unroll
        for (int u = 0; u < 8; ++u) acc[hl][u] = 0.0f;
#pragma unroll
    for (int i = 0; i < MAXI; ++i) {
        const int j = G + DEC_GROUPS * i;
        float v8[8];
        if (j == pos) {
#pragma unroll
            for (int u = 0; u < 8; ++u) v8[u] = vn[u];
        } else {
            kv_unpack8<KV>(vr[i], v8);
        }
#pragma unroll
        for (int hl = 0; hl < GROUP; ++hl)
#pragma unroll
            for (int u = 0; u < 8; ++u) acc[hl][u] = __builtin_fmaf(sc[i][hl], v8[u], acc[hl][u]);
    }
    __syncthreads();
#pragma unroll
    for (int hl = 0; hl < GROUP; ++hl) {
        // A row's 16 lanes hold the same l: count it from lane 0 of each row.
        float lw = l[hl];
        lw = (__shfl(lw, 0) + __shfl(lw, 16)) + (__shfl(lw, 32) + __shfl(lw, 48));
        if (wl == 0) red[wave][hl] = lw;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            float a = acc[hl][u];
            a += __shfl_xor(a, 16);
            a += __shfl_xor(a, 32);
            if (wl < 16 && dims) part[wave][hl * hd + l16 * 8 + u] = a;
        }
    }
    __syncthreads();
    if (t < GROUP) {
        float s2 = 0.0f;
        for (int w = 0; w < DEC_THREADS / WAVE; ++w) s2 += red[w][t];
        stat[1][t] = s2;
    }
    __syncthreads();
    if (t < group * hd) {
        const int hl = t / hd, ee = t % hd;
        float o = 0.0f;
        for (int w = 0; w < DEC_THREADS / WAVE; ++w) o += part[w][hl * hd + ee];
        out[(size_t)(g * group + hl) * hd + ee] = o / stat[1][hl];
    }
}

// Greedy choice (CausalLm::greedy, causal_lm.rs:284-302): the first index
// of the largest logit (src/layers.rs:604-612); a stop token ends the loop
// without being kept; max_new kept tokens end it too. Each block takes
// CHOOSE_SPAN logits; the last block to arrive reduces the blocks' winners,
// commits the token and writes its embedding row (the next forward's input).
__device__ __forceinline__ void better(float& bv, int& bi, float v, int i) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

__global__ __launch_bounds__(CHOOSE_THREADS) void choose_kernel(const float* __restrict__ logits, int n, State* st,
                                                                 int* __restrict__ out, float2* __restrict__ part,
                                                                 TableRef table, int d, float* __restrict__ x) {
    if (st->done) return;
    __shared__ float bv[CHOOSE_THREADS];
    __shared__ int bi[CHOOSE_THREADS];
    __shared__ bool last;
    const int i0 = blockIdx.x * CHOOSE_SPAN + (int)threadIdx.x * 4;
    float best = -INFINITY;
    int index = 0x7fffffff;
    for (int j = 0; j < 4; ++j) {
        const int i = i0 + j;
        if (i < n) {
            const float v = logits[i];
            if (index == 0x7fffffff || v > best) {
                best = v;
                index = i;
            }
        }
    }
    bv[threadIdx.x] = best;
    bi[threadIdx.x] = index;
    __syncthreads();
    for (int s = CHOOSE_THREADS / 2; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) better(bv[threadIdx.x], bi[threadIdx.x], bv[threadIdx.x + s], bi[threadIdx.x + s]);
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        part[blockIdx.x] = make_float2(bv[0], __int_as_float(bi[0]));
        __threadfence();
        last = atomicAdd(&st->arrived, 1u) == gridDim.x - 1;
    }
    __syncthreads();
    if (!last) return;
    __threadfence();
    best = -INFINITY;
    index = 0x7fffffff;
    for (int b = threadIdx.x; b < (int)gridDim.x; b += CHOOSE_THREADS) {
        const float2 p = part[b];
        better(best, index, p.x, __float_as_int(p.y));
    }
    bv[threadIdx.x] = best;
    bi[threadIdx.x] = index;
    __syncthreads();
    for (int s = CHOOSE_THREADS / 2; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) better(bv[threadIdx.x], bi[threadIdx.x], bv[threadIdx.x + s], bi[threadIdx.x + s]);
        __syncthreads();
    }
    __shared__ int commit;
    if (threadIdx.x == 0) {
        st->arrived = 0;
        const int token = bi[0];
        st->token = token;
        bool stop = false;
        for (int s = 0; s < st->n_stop; ++s) stop |= st->stop[s] == token;
        commit = 0;
        if (stop || st->n_out >= st->max_new) {
            st->done = 1;
        } else {
            out[st->n_out] = token;
            st->n_out += 1;
            // The forward of the last kept token gives logits nobody reads.
            if (st->n_out >= st->max_new) st->done = 1;
            else commit = 1;
        }
    }
    __syncthreads();
    if (!commit) return;
    // Dense::row of the chosen token (src/cpu/gemm.rs:412-429).
    const int token = bi[0];
    for (int kk = threadIdx.x; kk < d; kk += CHOOSE_THREADS) x[kk] = table_value(table, token, kk, d);
}

__global__ void advance_kernel(State* st, int rows) {
    if (st->done) return;
    st->pos += rows;
}

// The sequences of one decoder step with several sequences (beams): each
// its own keys and values, tk rows of kv_heads * hd f32 (the row layout of
// the reference's per-sequence caches).
constexpr int STEPS_MAX = 32;
struct StepsSeq {
    const float* k;
    const float* v;
    int tk;
};
struct StepsTable {
    StepsSeq s[STEPS_MAX];
};

// layers::attention_steps (src/layers.rs:505-562): block (h, b) is query
// head h of sequence b, its one query over all of the sequence's keys, in
// attention_kernel's orders (qh = q * (1/sqrt(hd)); score_j a fused chain
// over e; max; e_j = exp(s_j - max); a serial sum over j; p_j = e_j *
// (1/sum); out_e a fused chain of p_j * v_je over j). out row b holds
// heads * hd values at stride d.
__global__ __launch_bounds__(ATT_THREADS) void attention_steps_kernel(const float* __restrict__ q, int qs,
                                                                      StepsTable table, int heads, int kvh, int hd,
                                                                      int d, float* __restrict__ out) {
    extern __shared__ float sm[];  // qh[MAX_HD] | probs[tk] | red[ATT_THREADS]
    const int h = blockIdx.x, b = blockIdx.y;
    const StepsSeq seq = table.s[b];
    const int tk = seq.tk, stride = kvh * hd;
    const int g = h / (heads / kvh);
    float* qh = sm;
    float* probs = sm + MAX_HD;
    float* red = probs + tk;
    const float scale = 1.0f / __builtin_sqrtf((float)hd);
    for (int e = threadIdx.x; e < hd; e += ATT_THREADS) qh[e] = q[(size_t)b * qs + (size_t)h * hd + e] * scale;
    __syncthreads();
    float best = -INFINITY;
    for (int j = threadIdx.x; j < tk; j += ATT_THREADS) {
        const float* kr = seq.k + (size_t)j * stride + (size_t)g * hd;
        float acc = 0.0f;
        for (int e = 0; e < hd; e += 8) {
            float kv[8];
            kv_load8(kr + e, kv);
#pragma unroll
            for (int u = 0; u < 8; ++u) acc = __builtin_fmaf(qh[e + u], kv[u], acc);
        }
        probs[j] = acc;
        best = __builtin_fmaxf(best, acc);
    }
    red[threadIdx.x] = best;
    __syncthreads();
    for (int s = ATT_THREADS / 2; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) red[threadIdx.x] = __builtin_fmaxf(red[threadIdx.x], red[threadIdx.x + s]);
        __syncthreads();
    }
    const float mx = red[0];
    __syncthreads();
    for (int j = threadIdx.x; j < tk; j += ATT_THREADS) probs[j] = exp_trit(probs[j] - mx);
    __syncthreads();
    if (threadIdx.x == 0) {
        float sum = 0.0f;
        for (int j = 0; j < tk; ++j) sum = sum + probs[j];
        red[0] = sum;
    }
    __syncthreads();
    const float inv = 1.0f / red[0];
    for (int j = threadIdx.x; j < tk; j += ATT_THREADS) probs[j] = probs[j] * inv;
    __syncthreads();
    const float* V = seq.v + (size_t)g * hd;
    for (int e = threadIdx.x; e < hd; e += ATT_THREADS) {
        float acc = 0.0f;
        for (int j = 0; j < tk; ++j) acc = __builtin_fmaf(probs[j], V[(size_t)j * stride + e], acc);
        out[(size_t)b * d + (size_t)h * hd + e] = acc;
    }
}

// attention_kernel's arithmetic for one query row (a decode step; every
// key visible), same bits, with the values' memory latency hidden: the
// values of the first VB bytes of keys are loaded into registers before
// the scores are made, and p.V runs stage by stage -- the registers stored
// to LDS, the next stage's loads issued, then lane e chains dim e over the
// stage's keys in order. The serial sum reads 16 values ahead.
constexpr int ONE_VB = 32768;  // bytes of values a stage: 8 16-byte pieces a thread

size_t attention_one_lds(int max_pos) { return ONE_VB + (size_t)(MAX_HD + ((max_pos + 3) & ~3) + 8) * 4; }

// HD: the head size as a constant (its loops unrolled, so each key's loads
// are issued together), or 0 for the size in hd.
template <typename KV, int HD>
__global__ __launch_bounds__(ATT_THREADS) void attention_one_kernel(const float* __restrict__ qkv, int heads, int kvh,
                                                                    int hd_arg, const KV* __restrict__ kcache,
                                                                    const KV* __restrict__ vcache, int max_pos,
                                                                    float* __restrict__ out, const State* st) {
    if (st->done) return;
    const int hd = HD ? HD : hd_arg;
    extern __shared__ __align__(16) float sm[];  // values[ONE_VB bytes] | qh[MAX_HD] | probs[tk] | red | inv
    const int t = threadIdx.x, h = blockIdx.x;
    const int g = h / (heads / kvh);
    const int tk = st->pos + 1;
    const int vch = ONE_VB / (hd * (int)sizeof(KV));  // keys a stage
    char* vbuf = (char*)sm;
    float* qh = sm + ONE_VB / 4;
    float* probs = qh + MAX_HD;
    float* red = probs + ((tk + 3) & ~3);
    const KV* K = kcache + (size_t)g * max_pos * hd;
    const KV* V = vcache + (size_t)g * max_pos * hd;
    constexpr int PIECES = ONE_VB / 16 / ATT_THREADS;
    uint4 vr[PIECES];
    auto load_stage = [&](int s0) {
        const int nbytes = min(tk - s0, vch) * hd * (int)sizeof(KV);
        const char* src = (const char*)(V + (size_t)s0 * hd);
#pragma unroll
        for (int i = 0; i < PIECES; ++i) {
            const int p = t + ATT_THREADS * i;
            vr[i] = 16 * p < nbytes ? *(const uint4*)(src + 16 * p) : make_uint4(0, 0, 0, 0);
        }
    };
    load_stage(0);
    const float scale = 1.0f / __builtin_sqrtf((float)hd);
    const float* q = qkv + (size_t)h * hd;
    for (int e = t; e < hd; e += ATT_THREADS) qh[e] = q[e] * scale;
    __syncthreads();
    float best = -INFINITY;
    for (int j = t; j < tk; j += ATT_THREADS) {
        float acc = 0.0f;
        const KV* kr = K + (size_t)j * hd;
        if constexpr (HD > 0) {
            float kv[HD];
#pragma unroll
            for (int e = 0; e < HD; e += 8) kv_load8(kr + e, kv + e);
#pragma unroll
            for (int e = 0; e < HD; ++e) acc = __builtin_fmaf(qh[e], kv[e], acc);
        } else {
            for (int e = 0; e < hd; e += 8) {
                float kv[8];
                kv_load8(kr + e, kv);
#pragma unroll
                for (int u = 0; u < 8; ++u) acc = __builtin_fmaf(qh[e + u], kv[u], acc);
            }
        }
        probs[j] = acc;
        best = __builtin_fmaxf(best, acc);
    }
    const int wave = t / 64, lane = t % 64;
    for (int o = 32; o > 0; o >>= 1) best = __builtin_fmaxf(best, __shfl_xor(best, o));
    if (lane == 0) red[wave] = best;
    __syncthreads();
    float mx = red[0];
    for (int w = 1; w < ATT_THREADS / 64; ++w) mx = __builtin_fmaxf(mx, red[w]);
    for (int j = t; j < tk; j += ATT_THREADS) probs[j] = exp_trit(probs[j] - mx);
    __syncthreads();
    if (t == 0) {
        float sum = 0.0f;
        int j = 0;
        float4 cur[4], nxt[4];
        if (tk >= 16) {
#pragma unroll
            for (int k = 0; k < 4; ++k) cur[k] = *(const float4*)(probs + 4 * k);
        }
        for (; j + 16 <= tk; j += 16) {
            if (j + 32 <= tk) {
#pragma unroll
                for (int k = 0; k < 4; ++k) nxt[k] = *(const float4*)(probs + j + 16 + 4 * k);
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                sum = sum + cur[k].x;
                sum = sum + cur[k].y;
                sum = sum + cur[k].z;
                sum = sum + cur[k].w;
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) cur[k] = nxt[k];
        }
        for (; j < tk; ++j) sum = sum + probs[j];
        red[ATT_THREADS / 64] = 1.0f / sum;
    }
    __syncthreads();
    const float inv = red[ATT_THREADS / 64];
    for (int j = t; j < tk; j += ATT_THREADS) probs[j] = probs[j] * inv;
    float acc = 0.0f;
    for (int s0 = 0; s0 < tk; s0 += vch) {
        __syncthreads();  // the probabilities are scaled; the last stage's reads are done
#pragma unroll
        for (int i = 0; i < PIECES; ++i) *(uint4*)(vbuf + 16 * (t + ATT_THREADS * i)) = vr[i];
        __syncthreads();
        if (s0 + vch < tk) load_stage(s0 + vch);  // in flight while this stage chains
        if (t < hd) {
            const int n = min(tk - s0, vch);
            const KV* vs = (const KV*)vbuf + t;
            const float* pj = probs + s0;
#pragma unroll 8
            for (int j = 0; j < n; ++j) acc = __builtin_fmaf(pj[j], (float)vs[(size_t)j * hd], acc);
        }
    }
    if (t < hd) out[(size_t)h * hd + t] = acc;
}

// attention_kernel's arithmetic for R query rows of one head per block:
// every row's scores, maximum, exponentials, serial sum and p.V chains in
// the same orders (same bits), with each key and value read once for the R
// rows. Scores: thread j chains its key against the R rows; p.V: thread
// (e, group) chains dim e of rows group, group + G, ... (G = 256 / hd) from
// values it loads once for its rows. probs rows have a pitch of tk rounded
// up to 4 floats.
template <typename KV, int R>
__global__ __launch_bounds__(ATT_THREADS) void attention_rows_kernel(
    const float* __restrict__ qkv, int stride, int heads, int kvh, int hd, const KV* __restrict__ kcache,
    const KV* __restrict__ vcache, int max_pos, int rows, float* __restrict__ out, const State* st, int causal) {
    if (st->done) return;
    extern __shared__ float sm[];  // qh[R][MAX_HD] | probs[R][pitch] | red[R][ATT_THREADS / 64] | inv[R]
    const int h = blockIdx.x, row0 = blockIdx.y * R;
    const int nr = min(R, rows - row0);
    const int g = h / (heads / kvh);
    const int tk = st->pos + rows;
    const int pitch = (tk + 3) & ~3;
    // Causal rows see no key past kmax (the block's last row's position):
    // there every row's weight is exp_trit(-inf) ~ 1.2e-38, which leaves a
    // sum of at least 1 (the maximum key's exp(0)) unchanged, so scores,
    // exponentials and the sums stop at kmax; the p.V chains too where that
    // is exact (below).
    const int kmax = causal ? min(tk, st->pos + row0 + nr) : tk;
    float* qh = sm;
    float* probs = sm + R * MAX_HD;
    float* red = probs + R * pitch;
    float* inv = red + R * (ATT_THREADS / 64);
    const float scale = 1.0f / __builtin_sqrtf((float)hd);
    for (int i = threadIdx.x; i < R * hd; i += ATT_THREADS) {
        const int r = i / hd, e = i - r * hd;
        qh[r * MAX_HD + e] = r < nr ? qkv[(size_t)(row0 + r) * stride + (size_t)h * hd + e] * scale : 0.0f;
    }
    __syncthreads();
    const KV* K = kcache + (size_t)g * max_pos * hd;
    const KV* V = vcache + (size_t)g * max_pos * hd;
    float best[R];
#pragma unroll
    for (int r = 0; r < R; ++r) best[r] = -INFINITY;
    for (int j = threadIdx.x; j < kmax; j += ATT_THREADS) {
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.0f;
        const KV* kr = K + (size_t)j * hd;
        for (int e = 0; e < hd; e += 8) {
            float kv[8];
            kv_load8(kr + e, kv);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float4 qa = *(const float4*)(qh + r * MAX_HD + e), qb = *(const float4*)(qh + r * MAX_HD + e + 4);
                const float qv[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
                for (int u = 0; u < 8; ++u) acc[r] = __builtin_fmaf(qv[u], kv[u], acc[r]);
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int visible = causal ? st->pos + row0 + r + 1 : tk;
            const float v = j < visible ? acc[r] : -INFINITY;
            probs[r * pitch + j] = v;
            best[r] = __builtin_fmaxf(best[r], v);
        }
    }
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float m = best[r];
        for (int o = 32; o > 0; o >>= 1) m = __builtin_fmaxf(m, __shfl_xor(m, o));
        if (lane == 0) red[r * (ATT_THREADS / 64) + wave] = m;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < nr * kmax; i += ATT_THREADS) {
        const int r = i / kmax, j = i - r * kmax;
        float mx = red[r * (ATT_THREADS / 64)];
        for (int w = 1; w < ATT_THREADS / 64; ++w) mx = __builtin_fmaxf(mx, red[r * (ATT_THREADS / 64) + w]);
        probs[r * pitch + j] = exp_trit(probs[r * pitch + j] - mx);
    }
    __syncthreads();
    // The serial sum of each row (thread r), in key order from 0: 16
    // values a step, the next 16 read while the current ones are added.
    if ((int)threadIdx.x < nr) {
        const float* pr = probs + threadIdx.x * pitch;
        float sum = 0.0f;
        int j = 0;
        float4 cur[4], nxt[4];
        if (kmax >= 16) {
#pragma unroll
            for (int q = 0; q < 4; ++q) cur[q] = *(const float4*)(pr + 4 * q);
        }
        for (; j + 16 <= kmax; j += 16) {
            if (j + 32 <= kmax) {
#pragma unroll
                for (int q = 0; q < 4; ++q) nxt[q] = *(const float4*)(pr + j + 16 + 4 * q);
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                sum = sum + cur[q].x;
                sum = sum + cur[q].y;
                sum = sum + cur[q].z;
                sum = sum + cur[q].w;
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) cur[q] = nxt[q];
        }
        for (; j < kmax; ++j) sum = sum + pr[j];
        inv[threadIdx.x] = 1.0f / sum;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < nr * kmax; i += ATT_THREADS) {
        const int r = i / kmax, j = i - r * kmax;
        probs[r * pitch + j] = probs[r * pitch + j] * inv[r];
    }
    __syncthreads();
    // p.V: dim e of the rows group, group + G, ...; each value loaded once.
    const int G = ATT_THREADS / hd;  // hd divides ATT_THREADS (8, 16, ..., 256)
    const int e = threadIdx.x % hd, group = threadIdx.x / hd;
    if (group < G) {
        constexpr int MR = R;  // at most R rows a thread
        float acc[MR];
#pragma unroll
        for (int k = 0; k < MR; ++k) acc[k] = 0.0f;
        int j = 0;
        for (; j + 16 <= kmax; j += 16) {
            float v[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) v[u] = kv_load(V + (size_t)(j + u) * hd + e);
#pragma unroll
            for (int k = 0; k < MR; ++k) {
                const int r = group + k * G;
                if (r >= nr) break;
                const float4* p4 = (const float4*)(probs + r * pitch + j);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float4 pq = p4[q];
                    acc[k] = __builtin_fmaf(pq.x, v[4 * q], acc[k]);
                    acc[k] = __builtin_fmaf(pq.y, v[4 * q + 1], acc[k]);
                    acc[k] = __builtin_fmaf(pq.z, v[4 * q + 2], acc[k]);
                    acc[k] = __builtin_fmaf(pq.w, v[4 * q + 3], acc[k]);
                }
            }
        }
        for (; j < kmax; ++j) {
            const float v = kv_load(V + (size_t)j * hd + e);
#pragma unroll
            for (int k = 0; k < MR; ++k) {
                const int r = group + k * G;
                if (r >= nr) break;
                acc[k] = __builtin_fmaf(probs[r * pitch + j], v, acc[k]);
            }
        }
        // Keys past kmax: weight pm = exp_trit(-inf) * (1/sum) <= 1.2e-38.
        // With f16 values (|v| <= 65504) each term is below 7.7e-34, under
        // half a step of any |acc| >= 2^-80, so it leaves acc as it is;
        // a chain nearer 0, or f32 values, takes the terms in order.
        if (kmax < tk) {
#pragma unroll
            for (int k = 0; k < MR; ++k) {
                const int r = group + k * G;
                if (r >= nr) break;
                if (sizeof(KV) == 2 && __builtin_fabsf(acc[k]) >= 0x1p-80f) continue;
                const float pm = exp_trit(-INFINITY) * inv[r];
                for (int jj = kmax; jj < tk; ++jj) acc[k] = __builtin_fmaf(pm, kv_load(V + (size_t)jj * hd + e), acc[k]);
            }
        }
#pragma unroll
        for (int k = 0; k < MR; ++k) {
            const int r = group + k * G;
            if (r >= nr) break;
            out[(size_t)(row0 + r) * heads * hd + (size_t)h * hd + e] = acc[k];
        }
    }
}

// Shared memory of attention_rows_kernel for R rows over tk keys.
size_t rows_lds(int R, int tk) {
    return (size_t)(R * MAX_HD + R * ((tk + 3) & ~3) + R * (ATT_THREADS / 64) + R) * 4;
}

// Trit's attention of `rows` query rows (exact kernel's arithmetic) over
// caches of max_tk positions: 4 rows a block (measured best: 8 rows share
// more key reads but halve the resident blocks), 2 when 4 rows' scores do
// not fit 64 KB of shared memory; false when not even two rows do.
template <typename KV>
bool launch_attention_rows(const float* qkv, int stride, int heads, int kvh, int hd, const KV* kc, const KV* vc,
                           int max_pos, int rows, int max_tk, float* out, const State* st, int causal,
                           hipStream_t s) {
    constexpr size_t LIMIT = 64 * 1024;
    auto go = [&](auto R_) {
        constexpr int R = decltype(R_)::value;
        hipLaunchKernelGGL((attention_rows_kernel<KV, R>), dim3(heads, (rows + R - 1) / R), dim3(ATT_THREADS),
                           rows_lds(R, max_tk), s, qkv, stride, heads, kvh, hd, kc, vc, max_pos, rows, out, st, causal);
        return true;
    };
    if (rows >= 4 && rows_lds(4, max_tk) <= LIMIT) return go(std::integral_constant<int, 4>{});
    if (rows >= 2 && rows_lds(2, max_tk) <= LIMIT) return go(std::integral_constant<int, 2>{});
    return false;
}

// Rows of keys and values (tk x kvs floats each, head g at g * hd) into the
// cache layout [g][position][hd] of type KV.
template <typename KV>
__global__ void rows_to_cache_kernel(const float* __restrict__ k, const float* __restrict__ v, int kvs, int tk,
                                     int kvh, int hd, KV* __restrict__ kc, KV* __restrict__ vc) {
    const size_t total = (size_t)tk * kvh * hd;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        const int e = (int)(i % hd);
        const size_t jg = i / hd;
        const int g = (int)(jg % kvh), j = (int)(jg / kvh);
        const size_t to = ((size_t)g * tk + j) * hd + e;
        kc[to] = (KV)k[(size_t)j * kvs + (size_t)g * hd + e];
        vc[to] = (KV)v[(size_t)j * kvs + (size_t)g * hd + e];
    }
}

}  // namespace

// Trit's attention over device rows (q rows of stride qs; k, v rows of
// stride kvs): the rows go into head-major caches kc, vc (kv_heads x tk x
// hd floats each) and the exact kernel runs per (head, query row). `st`
// holds pos = tk - tq and done = 0.
void exact_attention(const float* q, int qs, const float* k, const float* v, int kvs, int tq, int tk, int heads,
                     int kv_heads, int hd, int causal, float* out, float* kc, float* vc, State* st, hipStream_t s) {
    if ((size_t)(MAX_HD + tk + ATT_THREADS) * 4 > 64 * 1024)
        fail("attention: more keys than the exact kernel's shared memory holds (16000)");
    const int grid = (int)std::min<size_t>(4096, ((size_t)tk * kv_heads * hd + 255) / 256);
    hipLaunchKernelGGL(rows_to_cache_kernel<float>, dim3(grid), dim3(256), 0, s, k, v, kvs, tk, kv_heads, hd, kc, vc);
    if (!launch_attention_rows<float>(q, qs, heads, kv_heads, hd, kc, vc, tk, tq, tk, out, st, causal, s)) {
        const size_t lds = (size_t)(MAX_HD + tk + ATT_THREADS) * 4;
        hipLaunchKernelGGL(attention_kernel<float>, dim3(heads, tq), dim3(ATT_THREADS), lds, s, q, qs, heads, kv_heads,
                           hd, kc, vc, tk, tq, out, 1, st, causal);
    }
    TRIT_HIP(hipGetLastError());
}

// ---- host side ------------------------------------------------------------


namespace {

// Host rotary table, the glibc calls Trit makes on Linux (src/layers.rs:
// 291-299,318): inv_freq[i] = base^(-(2i)/dims), angle = pos * inv_freq[i].
void rope_table(int dims, float base, int positions, std::vector<float>& sn, std::vector<float>& cs) {
    float (*volatile f_pow)(float, float) = powf;
    float (*volatile f_sin)(float) = sinf;
    float (*volatile f_cos)(float) = cosf;
    const int half = dims / 2;
    std::vector<float> inv(half);
    for (int i = 0; i < half; ++i) inv[i] = f_pow(base, -(float)(2 * i) / (float)dims);
    sn.resize((size_t)positions * half);
    cs.resize((size_t)positions * half);
    for (int p = 0; p < positions; ++p)
        for (int i = 0; i < half; ++i) {
            const float angle = (float)p * inv[i];
            sn[(size_t)p * half + i] = f_sin(angle);
            cs[(size_t)p * half + i] = f_cos(angle);
        }
}

void drop_graph(SessionImpl& S) {
    if (S.graph) (void)hipGraphExecDestroy(S.graph);
    S.graph = nullptr;
}

void ensure_rows(SessionImpl& S, int rows) {
    if (rows <= S.rows_cap) return;
    const auto& c = S.dec->c;
    const int qd = c.heads * c.head_dim, kv = c.kv_heads * c.head_dim;
    S.x.alloc((size_t)rows * c.d * 4);
    S.qkv.alloc((size_t)rows * (qd + 2 * kv) * 4);
    S.att.alloc((size_t)rows * qd * 4);
    S.hid.alloc((size_t)rows * c.ffn * 4);
    S.inv.alloc((size_t)rows * 4);
    S.xn.alloc((size_t)rows * c.d * 4);
    if (S.dec->float_gate_up) S.wide.alloc((size_t)rows * 2 * c.ffn * 4);
    S.normed.alloc((size_t)c.d * 4);
    S.tokens_in.alloc((size_t)rows * 4);
    S.max_splits = (S.max_pos + Split<float>::CH - 1) / Split<float>::CH;
    S.att_part.alloc((size_t)rows * c.heads * S.max_splits * (c.head_dim + 2) * 4);
    S.att_arrived.alloc((size_t)rows * c.kv_heads * 4);
    const int kmax = std::max(std::max(c.d, qd), c.ffn);
    S.gemm_scratch.alloc(std::max(gemm_scratch_bytes(rows, kmax), gemv_scratch_bytes(8, kmax)));
    TRIT_HIP(hipMemset(S.att_arrived.ptr, 0, (size_t)rows * c.kv_heads * 4));
    S.rows_cap = rows;
    drop_graph(S);
}

// TRIT_HIP_QK_WAVE=0 runs the prompt's q/k norm and rotary one block a
// head (qk_rope_kernel) at head_dim 128 too.
bool use_qk_wave() {
    const char* v = getenv("TRIT_HIP_QK_WAVE");
    return !(v && v[0] == '0');
}

// TRIT_HIP_FLASH=0 keeps prompt attention on the split kernel.
bool use_flash() {
    const char* v = getenv("TRIT_HIP_FLASH");
    return !(v && v[0] == '0');
}

// Integer product of `rows` rows: on the matrix cores for more than 8 rows
// (same bits), else in launches of up to 8.
void product(SessionImpl& S, const Layer& L, GemvArgs a, int rows, hipStream_t s, int y_stride) {
    a.m = rows;
    if (rows > 8 && gemm_supported(L, a)) return gemm_int(L, a, S.gemm_scratch.ptr, s);
    a.scratch = S.gemm_scratch.ptr;
    a.scratch_bytes = S.gemm_scratch.bytes;
    for (int r0 = 0; r0 < rows; r0 += 8) {
        GemvArgs b = a;
        b.m = rows - r0 < 8 ? rows - r0 : 8;
        b.x = a.x + (size_t)r0 * L.k;
        b.y = a.y + (size_t)r0 * y_stride;
        if (a.residual) b.residual = a.residual + (size_t)r0 * y_stride;
        if (a.norm_inv) b.norm_inv = a.norm_inv + r0;
        layer_forward(L, b, s);
    }
}

template <typename KV, int MAXI, int GROUP>
void launch_decode_g(SessionImpl& S, int l, hipStream_t s) {
    const DecoderImpl& D = *S.dec;
    const auto& c = D.c;
    const int hd = c.head_dim;
    KV* kc = S.kcache.as<KV>() + (size_t)l * c.kv_heads * S.max_pos * hd;
    KV* vc = S.vcache.as<KV>() + (size_t)l * c.kv_heads * S.max_pos * hd;
    hipLaunchKernelGGL((attention_decode_kernel<KV, MAXI, GROUP>), dim3(c.kv_heads), dim3(DEC_THREADS), 0, s,
                       S.qkv.as<float>(), c.heads, c.kv_heads, hd, kc, vc, S.max_pos, S.att.as<float>(), S.st(),
                       c.qk_norm, D.q_norm(l), D.k_norm(l), c.eps, S.rope_sin.as<float>(), S.rope_cos.as<float>());
}

template <typename KV, int MAXI>
void launch_decode_i(SessionImpl& S, int l, hipStream_t s) {
    switch (S.dec->c.heads / S.dec->c.kv_heads) {
        case 1: return launch_decode_g<KV, MAXI, 1>(S, l, s);
        case 2: return launch_decode_g<KV, MAXI, 2>(S, l, s);
        default: return launch_decode_g<KV, MAXI, 4>(S, l, s);
    }
}

// Decode attention sized for the session: every key in one round of loads.
template <typename KV>
bool launch_decode(SessionImpl& S, int l, hipStream_t s) {
    const int per_group = (S.max_pos + DEC_GROUPS - 1) / DEC_GROUPS;
    const int group = S.dec->c.heads / S.dec->c.kv_heads;
    // The q heads and the new key take one thread per value.
    if (group != 1 && group != 2 && group != 4) return false;
    if ((group + 1) * S.dec->c.head_dim > DEC_THREADS) return false;
    if (per_group <= 4) return launch_decode_i<KV, 4>(S, l, s), true;
    if (per_group <= 8) return launch_decode_i<KV, 8>(S, l, s), true;
    if (per_group <= 12) return launch_decode_i<KV, 12>(S, l, s), true;
    return false;
}

template <typename KV>
void launch_split(SessionImpl& S, int l, int rows, bool fused, hipStream_t s) {
    const DecoderImpl& D = *S.dec;
    const auto& c = D.c;
    const int hd = c.head_dim, stride = (c.heads + 2 * c.kv_heads) * hd;
    const dim3 grid(c.kv_heads, (S.max_pos + Split<KV>::CH - 1) / Split<KV>::CH, rows);
    const size_t lds = (size_t)2 * Split<KV>::CH * hd * sizeof(KV);
    KV* kc = S.kcache.as<KV>() + (size_t)l * c.kv_heads * S.max_pos * hd;
    KV* vc = S.vcache.as<KV>() + (size_t)l * c.kv_heads * S.max_pos * hd;
    if (fused)
        hipLaunchKernelGGL((attention_split_kernel<KV, true>), grid, dim3(ATT_THREADS), lds, s, S.qkv.as<float>(),
                           stride, c.heads, c.kv_heads, hd, kc, vc, S.max_pos, rows, S.att.as<float>(),
                           S.att_part.as<float>(), S.att_arrived.as<unsigned int>(), S.max_splits, S.st(),
                           c.qk_norm, D.q_norm(l), D.k_norm(l), c.eps, S.rope_sin.as<float>(),
                           S.rope_cos.as<float>());
    else
        hipLaunchKernelGGL((attention_split_kernel<KV, false>), grid, dim3(ATT_THREADS), lds, s, S.qkv.as<float>(),
                           stride, c.heads, c.kv_heads, hd, kc, vc, S.max_pos, rows, S.att.as<float>(),
                           S.att_part.as<float>(), S.att_arrived.as<unsigned int>(), S.max_splits, S.st(),
                           c.qk_norm, D.q_norm(l), D.k_norm(l), c.eps, S.rope_sin.as<float>(),
                           S.rope_cos.as<float>());
}

// One forward of `rows` rows whose embeddings are in S.x, at positions
// st->pos.., ending with the logits of the last row.
void forward(SessionImpl& S, int rows, hipStream_t s) {
    const DecoderImpl& D = *S.dec;
    const auto& c = D.c;
    const int hd = c.head_dim, qd = c.heads * hd, kv = c.kv_heads * hd, stride = qd + 2 * kv;
    State* st = S.st();
    float* x = S.x.as<float>();
    const int ew = 256, eblocks = std::min((rows * c.d + 255) / 256, 1024);
    // Granite: the input rows times embedding_multiplier (causal_lm.rs:420).
    if (c.embedding_multiplier != 1.0f)
        hipLaunchKernelGGL(scale_kernel, dim3(eblocks), dim3(ew), 0, s, x, rows * c.d, c.embedding_multiplier, st);
    // q times attention_multiplier * sqrt(head_dim) after the rotary
    // (causal_lm.rs:422-424,438-442); off without the multiplier.
    const float q_scale = c.attention_multiplier != 0.0f ? c.attention_multiplier * sqrtf((float)hd) : 1.0f;
    const float rm = c.residual_multiplier;
    const float* ffn_scales = D.has_ffn_scales ? D.ffn_scales.as<float>() : nullptr;
    float* xn = S.xn.as<float>();
    for (int l = 0; l < c.layers; ++l) {
        GemvArgs a;
        a.eps = c.eps;
        a.skip = &st->done;
        // qkv with the attention norm in the prologue (a float-math qkv
        // takes the normed rows).
        if (S.exact) {
            launch_norm_inv(x, rows, c.d, c.eps, S.inv.as<float>(), st, s);
            a.norm_inv = S.inv.as<float>();
        }
        if (float_kind(D.qkv[l]->kind)) {
            hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(256), 0, s, x, c.d, D.norm_attn(l), c.eps,
                               S.exact ? S.inv.as<float>() : nullptr, xn, st, nullptr);
            a.x = xn;
            a.norm_inv = nullptr;
        } else {
            a.x = x;
            a.norm_w = D.norm_attn(l);
        }
        a.y = S.qkv.as<float>();
        product(S, *D.qkv[l], a, rows, s, stride);
        // q/k norm, rotary, cache append, attention.
        const bool fused = !S.exact && rows == 1 && q_scale == 1.0f;
        if (!fused) {
            if (S.exact && !S.kv32) {
                // Trit's serial q/k norm sums, f16 caches.
                hipLaunchKernelGGL(qk_rope_kernel<_Float16>, dim3(rows * (c.heads + 2 * c.kv_heads)),
                                   dim3(hd < 64 ? 64 : hd), 0, s, S.qkv.as<float>(), stride, c.heads, c.kv_heads, hd,
                                   c.qk_norm, D.q_norm(l), D.k_norm(l), c.eps, S.rope_sin.as<float>(),
                                   S.rope_cos.as<float>(),
                                   S.kcache.as<_Float16>() + (size_t)l * c.kv_heads * S.max_pos * hd,
                                   S.vcache.as<_Float16>() + (size_t)l * c.kv_heads * S.max_pos * hd, S.max_pos, st);
            } else if (S.kv32) {
                hipLaunchKernelGGL(qk_rope_kernel<float>, dim3(rows * (c.heads + 2 * c.kv_heads)),
                                   dim3(hd < 64 ? 64 : hd), 0, s, S.qkv.as<float>(), stride, c.heads, c.kv_heads, hd,
                                   c.qk_norm, D.q_norm(l), D.k_norm(l), c.eps, S.rope_sin.as<float>(),
                                   S.rope_cos.as<float>(),
                                   S.kcache.as<float>() + (size_t)l * c.kv_heads * S.max_pos * hd,
                                   S.vcache.as<float>() + (size_t)l * c.kv_heads * S.max_pos * hd, S.max_pos, st);
            } else if (hd == 128 && use_qk_wave()) {
                const int items = rows * (c.heads + 2 * c.kv_heads);
                hipLaunchKernelGGL(qk_rope_wave_kernel<_Float16>, dim3((items + 3) / 4), dim3(256), 0, s,
                                   S.qkv.as<float>(), stride, rows, c.heads, c.kv_heads, c.qk_norm, D.q_norm(l),
                                   D.k_norm(l), c.eps, S.rope_sin.as<float>(), S.rope_cos.as<float>(),
                                   S.kcache.as<_Float16>() + (size_t)l * c.kv_heads * S.max_pos * hd,
                                   S.vcache.as<_Float16>() + (size_t)l * c.kv_heads * S.max_pos * hd, S.max_pos, st);
            } else {
                hipLaunchKernelGGL(qk_rope_kernel<_Float16>, dim3(rows * (c.heads + 2 * c.kv_heads)),
                                   dim3(hd < 64 ? 64 : hd), 0, s, S.qkv.as<float>(), stride, c.heads, c.kv_heads, hd,
                                   c.qk_norm, D.q_norm(l), D.k_norm(l), c.eps, S.rope_sin.as<float>(),
                                   S.rope_cos.as<float>(),
                                   S.kcache.as<_Float16>() + (size_t)l * c.kv_heads * S.max_pos * hd,
                                   S.vcache.as<_Float16>() + (size_t)l * c.kv_heads * S.max_pos * hd, S.max_pos, st);
            }
            TRIT_HIP(hipGetLastError());
            if (q_scale != 1.0f)
                hipLaunchKernelGGL(scale_q_kernel, dim3(std::min((rows * qd + 255) / 256, 1024)), dim3(256), 0, s,
                                   S.qkv.as<float>(), stride, rows, qd, q_scale, st);
        }
        if (S.exact) {
            // The host sizes shared memory for the largest key count this forward can see.
            const size_t lds = (size_t)(MAX_HD + S.max_pos + ATT_THREADS) * 4;
            const size_t lo = (size_t)l * c.kv_heads * S.max_pos * hd;
            const bool multi =
                rows > 1 && (S.kv32 ? launch_attention_rows<float>(S.qkv.as<float>(), stride, c.heads, c.kv_heads, hd,
                                                                  S.kcache.as<float>() + lo, S.vcache.as<float>() + lo,
                                                                  S.max_pos, rows, S.max_pos, S.att.as<float>(), st,
                                                                  1, s)
                                    : launch_attention_rows<_Float16>(
                                          S.qkv.as<float>(), stride, c.heads, c.kv_heads, hd,
                                          S.kcache.as<_Float16>() + lo, S.vcache.as<_Float16>() + lo, S.max_pos,
                                          rows, S.max_pos, S.att.as<float>(), st, 1, s));
            if (multi) {
                // R query rows a block.
            } else if (rows == 1 && hd <= MAX_HD && ATT_THREADS % hd == 0 && attention_one_lds(S.max_pos) <= 64 * 1024) {
                // One decode row: the values' loads hidden behind the scores.
                if (S.kv32)
                    hipLaunchKernelGGL((hd == 128 ? attention_one_kernel<float, 128> : attention_one_kernel<float, 0>),
                                       dim3(c.heads), dim3(ATT_THREADS),
                                       attention_one_lds(S.max_pos), s, S.qkv.as<float>(), c.heads, c.kv_heads, hd,
                                       S.kcache.as<float>() + lo, S.vcache.as<float>() + lo, S.max_pos,
                                       S.att.as<float>(), st);
                else
                    hipLaunchKernelGGL((hd == 128 ? attention_one_kernel<_Float16, 128> : attention_one_kernel<_Float16, 0>),
                                       dim3(c.heads), dim3(ATT_THREADS),
                                       attention_one_lds(S.max_pos), s, S.qkv.as<float>(), c.heads, c.kv_heads, hd,
                                       S.kcache.as<_Float16>() + lo, S.vcache.as<_Float16>() + lo, S.max_pos,
                                       S.att.as<float>(), st);
            } else if (S.kv32)
                hipLaunchKernelGGL(attention_kernel<float>, dim3(c.heads, rows), dim3(ATT_THREADS), lds, s,
                                   S.qkv.as<float>(), stride, c.heads, c.kv_heads, hd, S.kcache.as<float>() + lo,
                                   S.vcache.as<float>() + lo, S.max_pos, rows, S.att.as<float>(), 1, st, 1);
            else
                hipLaunchKernelGGL(attention_kernel<_Float16>, dim3(c.heads, rows), dim3(ATT_THREADS), lds, s,
                                   S.qkv.as<float>(), stride, c.heads, c.kv_heads, hd, S.kcache.as<_Float16>() + lo,
                                   S.vcache.as<_Float16>() + lo, S.max_pos, rows, S.att.as<float>(), 1, st, 1);
        } else if (fused && (S.kv32 ? launch_decode<float>(S, l, s) : launch_decode<_Float16>(S, l, s))) {
            // One block per key/value head.
        } else if (!fused && rows > 1 && flash_prefill_supported(S) && use_flash()) {
            // Prompt rows (never inside the captured step): positions from the host.
            flash_prefill(S, l, rows, S.host_pos, s);
        } else if (S.kv32) {
            launch_split<float>(S, l, rows, fused, s);
        } else {
            launch_split<_Float16>(S, l, rows, fused, s);
        }
        TRIT_HIP(hipGetLastError());
        // o with the residual add; with Granite's residual_multiplier the
        // product is stored and added times it (causal_lm.rs:456).
        auto residual = [&](const LayerRef& L, const float* in) {
            GemvArgs r;
            r.skip = &st->done;
            r.x = in;
            if (rm == 1.0f) {
                r.y = x;
                r.residual = x;
                r.epilogue = EPI_RESIDUAL;
                product(S, *L, r, rows, s, c.d);
            } else {
                r.y = xn;
                product(S, *L, r, rows, s, c.d);
                hipLaunchKernelGGL(add_scaled_kernel, dim3(eblocks), dim3(ew), 0, s, x, xn, rows * c.d, rm, st);
            }
        };
        residual(D.o[l], S.att.as<float>());
        // gate_up with the MLP norm in the prologue and SwiGLU after; with
        // MLP scales the normed rows are made first and scaled
        // (causal_lm.rs:457-464).
        GemvArgs gu;
        gu.skip = &st->done;
        gu.eps = c.eps;
        if (S.exact) {
            launch_norm_inv(x, rows, c.d, c.eps, S.inv.as<float>(), st, s);
            gu.norm_inv = S.inv.as<float>();
        }
        const bool float_gu = float_kind(D.gate_up[l]->kind);
        if (ffn_scales || float_gu) {
            hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(256), 0, s, x, c.d, D.norm_mlp(l), c.eps,
                               S.exact ? S.inv.as<float>() : nullptr, xn, st,
                               ffn_scales ? ffn_scales + (size_t)l * c.d : nullptr);
            gu.x = xn;
            gu.norm_inv = nullptr;
        } else {
            gu.x = x;
            gu.norm_w = D.norm_mlp(l);
        }
        if (float_gu) {
            // The stacked product, then SwiGLU.
            gu.y = S.wide.as<float>();
            product(S, *D.gate_up[l], gu, rows, s, 2 * c.ffn);
            hipLaunchKernelGGL(silu_pair_kernel, dim3(std::min((rows * c.ffn + 255) / 256, 1024)), dim3(256), 0, s,
                               S.wide.as<float>(), rows, c.ffn, S.hid.as<float>(), st);
        } else {
            gu.y = S.hid.as<float>();
            gu.epilogue = EPI_SILU_PAIR;
            product(S, *D.gate_up[l], gu, rows, s, c.ffn);
        }
        // down with the residual add.
        residual(D.down[l], S.hid.as<float>());
    }
    // Final norm of the last row, then the head.
    const float* last = x + (size_t)(rows - 1) * c.d;
    if (S.exact) {
        launch_norm_inv(last, 1, c.d, c.eps, S.inv.as<float>(), st, s);
    }
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(1), dim3(256), 0, s, last, c.d, D.final_norm(), c.eps,
                       S.exact ? S.inv.as<float>() : nullptr, S.normed.as<float>(), st);
    TRIT_HIP(hipGetLastError());
    GemvArgs h;
    h.skip = &st->done;
    h.x = S.normed.as<float>();
    h.y = S.logits.as<float>();
    layer_forward(D.head ? *D.head : *D.embed, h, s);
    // Granite: logits times 1 / logits_scaling (causal_lm.rs:387).
    const float lw = 1.0f / c.logits_scaling;
    if (lw != 1.0f)
        hipLaunchKernelGGL(scale_kernel, dim3((c.vocab + 255) / 256), dim3(256), 0, s, S.logits.as<float>(), c.vocab,
                           lw, st);
    hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(1), 0, s, st, rows);
    TRIT_HIP(hipGetLastError());
}

void read_logits(SessionImpl& S, float* logits) {
    hipStream_t s = stream();
    if (logits)
        TRIT_HIP(hipMemcpyAsync(logits, S.logits.ptr, (size_t)S.dec->c.vocab * 4, hipMemcpyDeviceToHost, s));
    TRIT_HIP(hipStreamSynchronize(s));
}

void reset_state(SessionImpl& S) {
    State init{};
    TRIT_HIP(hipMemcpy(S.state.ptr, &init, sizeof(State), hipMemcpyHostToDevice));
    S.host_pos = 0;
    S.broken = false;
    S.step_cand_fresh = false;
}

void check_usable(const SessionImpl& S) {
    if (S.broken) fail("session: a decode step was abandoned at its deadline; reset the session before using it");
}

// Clears `done` and sets the loop limits for a generate call, keeping pos.
void arm_state(SessionImpl& S, int max_new, const int32_t* stop, int n_stop) {
    State h{};
    TRIT_HIP(hipMemcpy(&h, S.state.ptr, sizeof(State), hipMemcpyDeviceToHost));
    h.done = 0;
    h.n_out = 0;
    h.err = 0;
    h.max_new = max_new;
    h.n_stop = n_stop;
    for (int i = 0; i < n_stop; ++i) h.stop[i] = stop[i];
    TRIT_HIP(hipMemcpy(S.state.ptr, &h, sizeof(State), hipMemcpyHostToDevice));
}

// One greedy step: choose, embed the chosen token, forward it.
void step(SessionImpl& S, hipStream_t s) {
    const auto& c = S.dec->c;
    const int blocks = (c.vocab + CHOOSE_SPAN - 1) / CHOOSE_SPAN;
    hipLaunchKernelGGL(choose_kernel, dim3(blocks), dim3(CHOOSE_THREADS), 0, s, S.logits.as<float>(), c.vocab,
                       S.st(), S.tokens_out.as<int>(), S.partials.as<float2>(), table_ref(*S.dec->embed), c.d,
                       S.x.as<float>());
    if (S.additive_rows)
        hipLaunchKernelGGL(add_rows_kernel, dim3((c.d + 255) / 256), dim3(256), 0, s, S.x.as<float>(),
                           S.additive.as<float>(), c.d, c.d, 1, S.st());
    forward(S, 1, s);
}

// TRIT_HIP_GRAPH=0 launches each step's kernels one by one instead of
// replaying a captured graph (same kernels, same results).
bool use_graph() {
    const char* v = getenv("TRIT_HIP_GRAPH");
    return !(v && v[0] == '0');
}

// Fast-mode sessions whose model fits it decode on the persistent step
// (decode_step.hip); TRIT_HIP_STEP=0 keeps them on the per-kernel loop.
bool use_step(const SessionImpl& S) {
    const char* v = getenv("TRIT_HIP_STEP");
    if (v && v[0] == '0') return false;
    return decode_step_supported(S);
}

void build_graph(SessionImpl& S) {
    // The captured step holds the MLP scales' buffer and whether rows are
    // added to its input.
    const bool additive = S.additive_rows != 0;
    if (S.graph && S.graph_ffn_version == S.dec->ffn_version && S.graph_additive == additive) return;
    drop_graph(S);
    hipStream_t s = stream();
    hipGraph_t g = nullptr;
    TRIT_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    try {
        step(S, s);
    } catch (...) {
        (void)hipStreamEndCapture(s, &g);
        if (g) (void)hipGraphDestroy(g);
        throw;
    }
    TRIT_HIP(hipStreamEndCapture(s, &g));
    hipGraphExec_t exec = nullptr;
    hipError_t e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    TRIT_HIP(e);
    S.graph = exec;
    S.graph_ffn_version = S.dec->ffn_version;
    S.graph_additive = additive;
}

}  // namespace
}  // namespace trit

struct TritHipDecoder {
    std::shared_ptr<trit::DecoderImpl> impl;
};
struct TritHipSession {
    trit::SessionImpl impl;
};
// Prefix (causal_lm.rs:118-122): the tokens and, per layer and key/value
// head, their n keys and values in the cache type of the flags it was made
// with.
struct TritHipPrefix {
    std::shared_ptr<trit::DecoderImpl> dec;
    std::vector<int32_t> tokens;
    bool exact = false, kv32 = false;
    trit::DeviceMemory keys, values;  // [layer][kv head][n][head_dim]
};

namespace trit {
namespace {

// A session's caches and buffers for `max_positions` positions.
void init_session(SessionImpl& s, std::shared_ptr<DecoderImpl> dec, int max_positions, int flags) {
    if (max_positions <= 0) fail("session: max_positions must be positive");
    s.dec = std::move(dec);
    const auto& c = s.dec->c;
    s.max_pos = max_positions;
    s.flags = flags;
    // Trit's sum orders unless tree sums are asked for; f32 caches
    // with EXACT (Trit's own arithmetic) or KV_F32.
    s.exact = (flags & TRIT_HIP_EXACT) != 0 || (flags & TRIT_HIP_TREE_SUMS) == 0;
    s.kv32 = (flags & (TRIT_HIP_EXACT | TRIT_HIP_KV_F32)) != 0;
    if ((flags & TRIT_HIP_EXACT) && (flags & TRIT_HIP_TREE_SUMS))
        fail("session: EXACT and TREE_SUMS exclude each other");
    const size_t lds = (size_t)(MAX_HD + max_positions + ATT_THREADS) * 4;
    if (lds > 64 * 1024) fail("session: max_positions above the attention kernel's limit (16000)");
    const size_t kvb = (size_t)c.layers * c.kv_heads * max_positions * c.head_dim * (s.kv32 ? 4 : 2);
    s.kcache.alloc(kvb);
    s.vcache.alloc(kvb);
    std::vector<float> sn, cs;
    rope_table(c.head_dim, c.rope_base, max_positions, sn, cs);
    s.rope_sin.alloc(sn.size() * 4);
    s.rope_sin.upload(sn.data(), sn.size() * 4);
    s.rope_cos.alloc(cs.size() * 4);
    s.rope_cos.upload(cs.data(), cs.size() * 4);
    s.logits.alloc((size_t)c.vocab * 4);
    s.partials.alloc((size_t)((c.vocab + CHOOSE_SPAN - 1) / CHOOSE_SPAN) * 8);
    s.state.alloc(sizeof(State));
    ensure_rows(s, 8);
    reset_state(s);
}

}  // namespace
}  // namespace trit

using namespace trit;

extern "C" {

int trit_hip_decoder_new(const TritHipLmConfig* config, const TritHipLayer* const* linears, const float* norms,
                         const TritHipLayer* embed, const TritHipLayer* head, TritHipDecoder** out) {
    return guard(-1, [&] {
        if (!config || !linears || !norms || !embed || !out) fail("decoder: a required argument is NULL");
        const TritHipLmConfig& c = *config;
        if (c.heads <= 0 || c.kv_heads <= 0 || c.heads % c.kv_heads != 0)
            fail("decoder: the query heads do not share the key heads evenly");
        if (c.head_dim <= 0 || c.head_dim > 128 || c.head_dim % 8 != 0)
            fail("decoder: head_dim must be a multiple of 8 and at most 128");
        if (c.heads / c.kv_heads > 4) fail("decoder: at most 4 query heads per key/value head");
        auto D = std::make_shared<DecoderImpl>();
        D->c = c;
        // Zeros in the Granite fields mean none.
        if (D->c.embedding_multiplier == 0.0f) D->c.embedding_multiplier = 1.0f;
        if (D->c.residual_multiplier == 0.0f) D->c.residual_multiplier = 1.0f;
        if (D->c.logits_scaling == 0.0f) D->c.logits_scaling = 1.0f;
        const int hd = c.head_dim, qkv_rows = (c.heads + 2 * c.kv_heads) * hd;
        auto want = [&](const TritHipLayer* h, int n, int k, const char* what, int l) {
            LayerRef L = layer_ref(h);
            if (!L) fail(std::string("decoder: layer ") + std::to_string(l) + " " + what + " is NULL");
            if (L->n != n || L->k != k)
                fail(std::string("decoder: layer ") + std::to_string(l) + " " + what + " is " + std::to_string(L->n) +
                     "x" + std::to_string(L->k) + ", expected " + std::to_string(n) + "x" + std::to_string(k));
            if (L->kind == TERNARY)
                fail(std::string("decoder: layer ") + std::to_string(l) + " " + what +
                     " must be Q8_0, Q4_K, int8, f16, f32 or Q8");
            return L;
        };
        for (int l = 0; l < c.layers; ++l) {
            D->qkv.push_back(want(linears[4 * l], qkv_rows, c.d, "qkv", l));
            D->o.push_back(want(linears[4 * l + 1], c.d, c.heads * hd, "o", l));
            D->gate_up.push_back(want(linears[4 * l + 2], 2 * c.ffn, c.d, "gate_up", l));
            D->down.push_back(want(linears[4 * l + 3], c.d, c.ffn, "down", l));
        }
        for (int l = 0; l < c.layers; ++l) D->float_gate_up |= float_kind(D->gate_up[l]->kind);
        // Token tables take f32 math, never int8 activations (Dense::table,
        // src/cpu/gemm.rs:376-409).
        D->embed = layer_ref(embed);
        if (!float_kind(D->embed->kind) || D->embed->n != c.vocab || D->embed->k != c.d)
            fail("decoder: embed must be a vocab x d table of f16, f32 or Q8 weights");
        if (head) {
            D->head = layer_ref(head);
            if (D->head->n != c.vocab || D->head->k != c.d) fail("decoder: head must be vocab x d");
            if (!float_kind(D->head->kind))
                fail("decoder: head must be a table of f16, f32 or Q8 weights (f32 math; for Q8_0 blocks "
                     "trit_hip_layer_q8_0_f32)");
        }
        D->layer_norm_stride = (size_t)2 * c.d + (c.qk_norm ? 2 * hd : 0);
        const size_t count = D->layer_norm_stride * c.layers + c.d;
        // q/k norm slots exist even without qk_norm so the pointers stay valid.
        D->layer_norm_stride = (size_t)2 * c.d + 2 * hd;
        std::vector<float> packed(D->layer_norm_stride * c.layers + c.d, 1.0f);
        const float* src = norms;
        for (int l = 0; l < c.layers; ++l) {
            float* dst = packed.data() + l * D->layer_norm_stride;
            std::memcpy(dst, src, (size_t)2 * c.d * 4);
            src += 2 * c.d;
            if (c.qk_norm) {
                std::memcpy(dst + 2 * c.d, src, (size_t)2 * hd * 4);
                src += 2 * hd;
            }
        }
        std::memcpy(packed.data() + D->layer_norm_stride * c.layers, src, (size_t)c.d * 4);
        (void)count;
        D->norms.alloc(packed.size() * 4);
        D->norms.upload(packed.data(), packed.size() * 4);
        *out = new TritHipDecoder{D};
        return 0;
    });
}

void trit_hip_decoder_free(TritHipDecoder* decoder) { delete decoder; }

// ---- The device weight-cache file --------------------------------------
//
// A decoder's device layouts as they sit in HBM (codes repacked, Q4_K and
// the other block types already requantized, f16 tables in lane chains),
// so a later load uploads them without converting. Layout: "TRITHIPW", a
// format version, the library's key (its version and target), the config,
// the norms as trit_hip_decoder_new takes them, the 4 linears of each layer,
// the embedding and the head (when untied), each as kind, n, k, group and
// the byte runs of its codes, scales and bias; then a 64-bit checksum of
// everything before it. Stale or damaged files fail the load.

}  // extern "C"

namespace trit {
namespace {

constexpr char CACHE_MAGIC[8] = {'T', 'R', 'I', 'T', 'H', 'I', 'P', 'W'};
constexpr uint32_t CACHE_FORMAT = 2;
// The version of the device layouts the file holds (the row-major integer
// codes and scales, the float kinds' lane-chain layout, the 2-bit ternary
// spans): bumped whenever a repack changes, so an older file is refused
// by its key instead of handing the kernels buffers of another layout.
constexpr int LAYOUT_VERSION = 2;

struct Hash {
    uint64_t h = 0x9E3779B97F4A7C15ull;
    uint64_t tail = 0;
    int tail_bytes = 0;
    void add(const void* data, size_t n) {
        const uint8_t* p = (const uint8_t*)data;
        while (n && tail_bytes) {
            tail |= (uint64_t)*p++ << (8 * tail_bytes);
            --n;
            if (++tail_bytes == 8) {
                word(tail);
                tail = 0;
                tail_bytes = 0;
            }
        }
        for (; n >= 8; n -= 8, p += 8) {
            uint64_t w;
            std::memcpy(&w, p, 8);
            word(w);
        }
        while (n--) tail |= (uint64_t)*p++ << (8 * tail_bytes++);
    }
    void word(uint64_t w) {
        h ^= w;
        h *= 0x100000001B3ull;
        h ^= h >> 29;
    }
    uint64_t value() const {
        uint64_t v = h;
        if (tail_bytes) {
            v ^= tail;
            v *= 0x100000001B3ull;
        }
        return v ^ (v >> 32);
    }
};

struct CacheWriter {
    FILE* f;
    Hash hash;
    void put(const void* p, size_t n) {
        if (n && std::fwrite(p, 1, n, f) != n) fail("cache: write failed");
        hash.add(p, n);
    }
    template <class T>
    void val(T v) {
        put(&v, sizeof v);
    }
    void device(const DeviceMemory& m) {
        val<uint64_t>(m.bytes);
        std::vector<uint8_t> host(std::min<size_t>(m.bytes, (size_t)64 << 20));
        for (size_t at = 0; at < m.bytes; at += host.size()) {
            const size_t c = std::min(host.size(), m.bytes - at);
            TRIT_HIP(hipMemcpy(host.data(), (const uint8_t*)m.ptr + at, c, hipMemcpyDeviceToHost));
            put(host.data(), c);
        }
    }
    void layer(const Layer& L) {
        val<int32_t>(L.kind);
        val<int32_t>(L.n);
        val<int32_t>(L.k);
        val<int32_t>(L.group);
        device(L.codes);
        device(L.scales);
        device(L.bias);
    }
};

// The exact device bytes of a layer's codes and scales for its kind, n, k
// and group (the layouts the layer calls make); false for a combination no
// layer call makes.
bool layout_bytes(int kind, int n, int k, int group, uint64_t* codes, uint64_t* scales) {
    const uint64_t N = (uint64_t)n, K = (uint64_t)k, steps = (uint64_t)chain_steps(k);
    switch (kind) {
        case Q8_0:
        case Q4_K:
            if (group != 32 || k % 32) return false;
            *codes = N * K, *scales = N * (K / 32) * 2;
            return true;
        case INT8:
            if (group != 128 || k % 128) return false;
            *codes = N * K, *scales = N * (K / 128) * 4;
            return true;
        case TERNARY:
            if (group != 128 || k % 128) return false;
            *codes = N * K / 4, *scales = N * (K / 128) * 4;
            return true;
        case F16: *codes = N * 16 * steps * 2, *scales = 0; return true;
        case F32: *codes = N * 16 * steps * 4, *scales = 0; return true;
        case Q8_F32:
            if (k % 32) return false;
            *codes = N * 16 * steps, *scales = N * (K / 32) * 4;
            return true;
        default: return false;
    }
}

struct CacheReader {
    FILE* f;
    Hash hash;
    const char* path;
    void get(void* p, size_t n) {
        if (n && std::fread(p, 1, n, f) != n) fail(std::string(path) + ": the cache file is cut short");
        hash.add(p, n);
    }
    template <class T>
    T val() {
        T v;
        get(&v, sizeof v);
        return v;
    }
    // A buffer of exactly `want` bytes (`alt`, when nonzero, is the one
    // other size allowed: a bias may be absent).
    void device(DeviceMemory& m, uint64_t want, uint64_t alt = UINT64_MAX) {
        const uint64_t bytes = val<uint64_t>();
        if (bytes != want && bytes != alt)
            fail(std::string(path) + ": a buffer of the cache file does not have its layer's size");
        m.alloc(bytes);
        std::vector<uint8_t> host(std::min<size_t>(bytes, (size_t)64 << 20));
        for (size_t at = 0; at < bytes; at += host.size()) {
            const size_t c = std::min<size_t>(host.size(), bytes - at);
            get(host.data(), c);
            TRIT_HIP(hipMemcpy((uint8_t*)m.ptr + at, host.data(), c, hipMemcpyHostToDevice));
        }
    }
    LayerRef layer() {
        auto L = std::make_shared<Layer>();
        L->kind = val<int32_t>();
        L->n = val<int32_t>();
        L->k = val<int32_t>();
        L->group = val<int32_t>();
        uint64_t codes = 0, scales = 0;
        if (L->n <= 0 || L->k <= 0 || !layout_bytes(L->kind, L->n, L->k, L->group, &codes, &scales))
            fail(std::string(path) + ": a layer of the cache file is not valid");
        // The three buffers' sizes are checked before any is uploaded.
        const off_t at = ftello(f);
        const uint64_t want[3] = {codes, scales, (uint64_t)L->n * 4};
        for (int i = 0; i < 3; ++i) {
            uint64_t bytes = 0;
            if (std::fread(&bytes, 8, 1, f) != 1) fail(std::string(path) + ": the cache file is cut short");
            if (bytes != want[i] && !(i == 2 && bytes == 0))
                fail(std::string(path) + ": a buffer of the cache file does not have its layer's size");
            if (bytes > (uint64_t)INT64_MAX || fseeko(f, (off_t)bytes, SEEK_CUR) != 0)
                fail(std::string(path) + ": the cache file is cut short");
        }
        if (fseeko(f, at, SEEK_SET) != 0) fail(std::string(path) + ": cannot read the cache file");
        device(L->codes, codes);
        device(L->scales, scales);
        device(L->bias, (uint64_t)L->n * 4, 0);
        return L;
    }
};

std::string cache_key() { return std::string(trit_hip_version()) + " layout " + std::to_string(LAYOUT_VERSION); }

}  // namespace
}  // namespace trit

extern "C" {

int trit_hip_decoder_save(const TritHipDecoder* decoder, const char* path) {
    return guard(-1, [&] {
        if (!decoder || !path) fail("cache: decoder or path is NULL");
        const DecoderImpl& D = *decoder->impl;
        const auto& c = D.c;
        const std::string tmp = std::string(path) + ".tmp";
        FILE* f = std::fopen(tmp.c_str(), "wb");
        if (!f) fail(std::string("cache: cannot write ") + tmp);
        try {
            CacheWriter w{f};
            w.put(CACHE_MAGIC, 8);
            w.val<uint32_t>(CACHE_FORMAT);
            const std::string key = cache_key();
            w.val<uint32_t>((uint32_t)key.size());
            w.put(key.data(), key.size());
            w.val<uint32_t>((uint32_t)sizeof(TritHipLmConfig));
            w.put(&c, sizeof c);
            // The norms as the caller gave them: attn, mlp, [q, k] a layer; final.
            std::vector<float> all(D.norms.bytes / 4), norms;
            TRIT_HIP(hipMemcpy(all.data(), D.norms.ptr, D.norms.bytes, hipMemcpyDeviceToHost));
            for (int l = 0; l < c.layers; ++l) {
                const float* at = all.data() + l * D.layer_norm_stride;
                norms.insert(norms.end(), at, at + 2 * c.d + (c.qk_norm ? 2 * c.head_dim : 0));
            }
            const float* fin = all.data() + c.layers * D.layer_norm_stride;
            norms.insert(norms.end(), fin, fin + c.d);
            w.val<uint64_t>(norms.size());
            w.put(norms.data(), norms.size() * 4);
            for (int l = 0; l < c.layers; ++l) {
                w.layer(*D.qkv[l]);
                w.layer(*D.o[l]);
                w.layer(*D.gate_up[l]);
                w.layer(*D.down[l]);
            }
            w.layer(*D.embed);
            w.val<uint8_t>(D.head ? 1 : 0);
            if (D.head) w.layer(*D.head);
            const uint64_t sum = w.hash.value();
            if (std::fwrite(&sum, 8, 1, f) != 1) fail("cache: write failed");
        } catch (...) {
            std::fclose(f);
            std::remove(tmp.c_str());
            throw;
        }
        if (std::fclose(f) != 0 || std::rename(tmp.c_str(), path) != 0) {
            std::remove(tmp.c_str());
            fail(std::string("cache: cannot write ") + path);
        }
        return 0;
    });
}

int trit_hip_decoder_load(const char* path, TritHipLmConfig* config, TritHipDecoder** out) {
    return guard(-1, [&] {
        if (!path || !out) fail("cache: path or out is NULL");
        FILE* f = std::fopen(path, "rb");
        if (!f) fail(std::string("cache: cannot read ") + path);
        std::vector<TritHipLayer*> handles;
        auto cleanup = [&] {
            for (TritHipLayer* h : handles) trit_hip_layer_free(h);
            std::fclose(f);
        };
        try {
            CacheReader r{f, {}, path};
            char magic[8];
            r.get(magic, 8);
            if (std::memcmp(magic, CACHE_MAGIC, 8) != 0) fail(std::string(path) + ": not a trit_hip weight cache");
            if (r.val<uint32_t>() != CACHE_FORMAT) fail(std::string(path) + ": another cache format");
            const uint32_t klen = r.val<uint32_t>();
            if (klen > 256) fail(std::string(path) + ": not a trit_hip weight cache");
            std::string key(klen, '\0');
            r.get(key.data(), klen);
            if (key != cache_key())
                fail(std::string(path) + ": made by " + key + ", not by " + cache_key() + " (build it again)");
            if (r.val<uint32_t>() != sizeof(TritHipLmConfig)) fail(std::string(path) + ": another config layout");
            TritHipLmConfig c;
            r.get(&c, sizeof c);
            if (c.layers <= 0 || c.layers > 4096 || c.d <= 0) fail(std::string(path) + ": a bad config");
            // attn, mlp and (with QK-norm) q, k a layer, then the final norm:
            // exactly what trit_hip_decoder_new reads.
            if (c.d > (1 << 20) || c.head_dim < 0 || c.head_dim > (1 << 16)) fail(std::string(path) + ": a bad config");
            const uint64_t per_layer = 2 * (uint64_t)c.d + (c.qk_norm ? 2 * (uint64_t)c.head_dim : 0);
            const uint64_t nn = r.val<uint64_t>();
            if (nn != (uint64_t)c.layers * per_layer + (uint64_t)c.d) fail(std::string(path) + ": a bad norm count");
            std::vector<float> norms(nn);
            r.get(norms.data(), nn * 4);
            for (int i = 0; i < 4 * c.layers + 1; ++i) handles.push_back(layer_handle(r.layer()));
            if (r.val<uint8_t>()) handles.push_back(layer_handle(r.layer()));
            const uint64_t want = r.hash.value();
            uint64_t sum = 0;
            if (std::fread(&sum, 8, 1, f) != 1 || sum != want)
                fail(std::string(path) + ": the cache file is damaged (checksum)");
            TritHipDecoder* dec = nullptr;
            const TritHipLayer* head = handles.size() > (size_t)(4 * c.layers + 1) ? handles.back() : nullptr;
            if (trit_hip_decoder_new(&c, handles.data(), norms.data(), handles[4 * c.layers], head, &dec) != 0)
                fail(error_text());
            if (config) *config = c;
            *out = dec;
        } catch (...) {
            cleanup();
            throw;
        }
        cleanup();  // the decoder holds its layers
        return 0;
    });
}

int trit_hip_decoder_set_ffn_scales(TritHipDecoder* decoder, const float* scales) {
    return guard(-1, [&] {
        if (!decoder) fail("decoder is NULL");
        DecoderImpl& D = *decoder->impl;
        if (scales) {
            const size_t bytes = (size_t)D.c.layers * D.c.d * 4;
            if (D.ffn_scales.bytes != bytes) D.ffn_scales.alloc(bytes);
            D.ffn_scales.upload(scales, bytes);
            D.has_ffn_scales = true;
        } else {
            D.has_ffn_scales = false;
        }
        D.ffn_version += 1;
        return 0;
    });
}

int trit_hip_session_new(const TritHipDecoder* decoder, int max_positions, int flags, TritHipSession** out) {
    return guard(-1, [&] {
        if (!decoder || !out) fail("session: decoder or out is NULL");
        auto* S = new TritHipSession();
        try {
            init_session(S->impl, decoder->impl, max_positions, flags);
        } catch (...) {
            delete S;
            throw;
        }
        *out = S;
        return 0;
    });
}

// The prompt's rows (embeddings of `tokens`, or host `rows`) plus, with
// `add`, n x d device rows, at the next positions.
static int prefill_common(TritHipSession* session, int n, float* logits, const int32_t* tokens, const float* rows,
                          const float* add = nullptr) {
    if (!session) fail("session is NULL");
    if (n <= 0) fail("prefill: no rows");
    SessionImpl& S = session->impl;
    check_usable(S);
    const auto& c = S.dec->c;
    if (S.host_pos + n > S.max_pos)
        fail("prefill: " + std::to_string(S.host_pos + n) + " positions exceed the session's " +
             std::to_string(S.max_pos));
    ensure_rows(S, n);
    hipStream_t s = stream();
    // A forward after a finished loop continues from the kept positions.
    State h{};
    TRIT_HIP(hipMemcpy(&h, S.state.ptr, sizeof(State), hipMemcpyDeviceToHost));
    h.done = 0;
    TRIT_HIP(hipMemcpy(S.state.ptr, &h, sizeof(State), hipMemcpyHostToDevice));
    if (tokens) {
        for (int i = 0; i < n; ++i)
            if (tokens[i] < 0 || tokens[i] >= c.vocab) fail("prefill: token " + std::to_string(tokens[i]) + " out of range");
        TRIT_HIP(hipMemcpyAsync(S.tokens_in.ptr, tokens, (size_t)n * 4, hipMemcpyHostToDevice, s));
        hipLaunchKernelGGL(embed_kernel, dim3(n), dim3(256), 0, s, table_ref(*S.dec->embed), c.d,
                           S.tokens_in.as<int>(), S.x.as<float>(), S.st());
        TRIT_HIP(hipGetLastError());
    } else {
        TRIT_HIP(hipMemcpyAsync(S.x.ptr, rows, (size_t)n * c.d * 4, hipMemcpyHostToDevice, s));
    }
    if (add) {
        hipLaunchKernelGGL(add_rows_kernel, dim3(std::min((n * c.d + 255) / 256, 1024)), dim3(256), 0, s,
                           S.x.as<float>(), add, n * c.d, c.d, 0, S.st());
        TRIT_HIP(hipGetLastError());
    }
    forward(S, n, s);
    S.host_pos += n;
    S.step_cand_fresh = false;
    read_logits(S, logits);
    return 0;
}

int trit_hip_session_prefill(TritHipSession* session, const int32_t* tokens, int n, float* logits) {
    return guard(-1, [&] {
        if (!tokens) fail("prefill: tokens is NULL");
        return prefill_common(session, n, logits, tokens, nullptr);
    });
}

int trit_hip_session_prefill_rows(TritHipSession* session, const float* rows, int n, float* logits) {
    return guard(-1, [&] {
        if (!rows) fail("prefill: rows is NULL");
        return prefill_common(session, n, logits, nullptr, rows);
    });
}

static int generate_common(TritHipSession* session, int max_new, const int32_t* stop, int n_stop, int32_t* out,
                           hipEvent_t ev_start, hipEvent_t ev_stop) {
    if (!session) fail("session is NULL");
    SessionImpl& S = session->impl;
    check_usable(S);
    if (S.host_pos == 0) fail("generate: prefill a prompt first");
    if (max_new <= 0) return 0;
    if (!out) fail("generate: out is NULL");
    if (n_stop < 0 || n_stop > MAX_STOP) fail("generate: at most 64 stop tokens");
    if (n_stop && !stop) fail("generate: stop is NULL");
    // The loop forwards up to max_new - 1 new tokens.
    if (S.host_pos + max_new - 1 > S.max_pos)
        fail("generate: " + std::to_string(max_new) + " tokens exceed the session's positions");
    if (S.graph_out_cap < max_new) {
        S.tokens_out.alloc((size_t)max_new * 4);
        S.graph_out_cap = max_new;
        drop_graph(S);
    }
    arm_state(S, max_new, stop, n_stop);
    hipStream_t s = stream();
    const bool persistent = use_step(S);
    if (persistent) decode_step_prepare(S, s);
    else if (use_graph()) build_graph(S);
    if (ev_start) TRIT_HIP(hipEventRecord(ev_start, s));
    if (persistent) {
        decode_step_launch(S, 0, S.host_pos, max_new, s);
        S.step_cand_fresh = true;
    } else if (use_graph()) {
        for (int i = 0; i < max_new; ++i) TRIT_HIP(hipGraphLaunch(S.graph, s));
    } else {
        for (int i = 0; i < max_new; ++i) step(S, s);
    }
    if (ev_stop) TRIT_HIP(hipEventRecord(ev_stop, s));
    State h{};
    TRIT_HIP(hipMemcpyAsync(&h, S.state.ptr, sizeof(State), hipMemcpyDeviceToHost, s));
    TRIT_HIP(hipStreamSynchronize(s));
    if (h.err) {
        // Blocks left the launch at different points: the caches may hold a
        // partial step and the device position may have moved.
        S.broken = true;
        S.host_pos = h.pos;
        S.step_cand_fresh = false;
        if (h.err & 2)
            fail("generate: a decode-step block ran on another XCD than its local exchange needs (the step was "
                 "abandoned; reset the session, with TRIT_HIP_STEP_LOCAL=0)");
        fail("generate: a decode-step block waited past its deadline (the step was abandoned; reset the session)");
    }
    TRIT_HIP(hipMemcpy(out, S.tokens_out.ptr, (size_t)h.n_out * 4, hipMemcpyDeviceToHost));
    S.host_pos = h.pos;
    return h.n_out;
}

int trit_hip_session_generate(TritHipSession* session, int max_new, const int32_t* stop, int n_stop, int32_t* out) {
    return guard(-1, [&] { return generate_common(session, max_new, stop, n_stop, out, nullptr, nullptr); });
}

int trit_hip_session_generate_timed(TritHipSession* session, int max_new, const int32_t* stop, int n_stop,
                                    int32_t* out, void* start_event, void* stop_event, int* persistent) {
    return guard(-1, [&] {
        if (persistent) *persistent = session && use_step(session->impl) ? decode_step_layout(session->impl) : 0;
        return generate_common(session, max_new, stop, n_stop, out, (hipEvent_t)start_event, (hipEvent_t)stop_event);
    });
}

int trit_hip_session_generate_additive(TritHipSession* session, const int32_t* prompt, int n, const float* audio,
                                       int rows, const int32_t* stop, int n_stop, int32_t* out) {
    return guard(-1, [&] {
        if (!session) fail("session is NULL");
        SessionImpl& S = session->impl;
        check_usable(S);
        if (n < 0 || rows < 0) fail("generate_additive: negative sizes");
        // Trit returns no tokens for an empty prompt or too few rows.
        if (n == 0 || rows < n) return 0;
        if (!prompt || !audio || !out) fail("generate_additive: prompt, audio or out is NULL");
        if (S.host_pos != 0) fail("generate_additive: the session holds positions; reset it first");
        if (rows > S.max_pos)
            fail("generate_additive: " + std::to_string(rows) + " rows exceed the session's " +
                 std::to_string(S.max_pos) + " positions");
        const auto& c = S.dec->c;
        const size_t bytes = (size_t)rows * c.d * 4;
        if (S.additive.bytes < bytes) {
            // The captured step holds the old buffer.
            drop_graph(S);
            S.additive.alloc(bytes);
        }
        S.additive.upload(audio, bytes);
        struct Off {
            SessionImpl& S;
            ~Off() { S.additive_rows = 0; }
        } off{S};
        S.additive_rows = rows;
        prefill_common(session, n, nullptr, prompt, nullptr, S.additive.as<float>());
        // The choice after the prompt, then one per row n..rows-1.
        return generate_common(session, rows - n + 1, stop, n_stop, out, nullptr, nullptr);
    });
}

int trit_hip_prefix_new(const TritHipDecoder* decoder, const int32_t* tokens, int n, int flags, TritHipPrefix** out) {
    return guard(-1, [&] {
        if (!decoder || !out) fail("prefix: decoder or out is NULL");
        if (n < 0) fail("prefix: negative token count");
        if (n && !tokens) fail("prefix: tokens is NULL");
        auto P = std::make_unique<TritHipPrefix>();
        P->dec = decoder->impl;
        P->tokens.assign(tokens, tokens + n);
        const auto& c = decoder->impl->c;
        if (n) {
            auto* T = new TritHipSession();
            std::unique_ptr<TritHipSession> own(T);
            init_session(T->impl, decoder->impl, n, flags);
            prefill_common(T, n, nullptr, tokens, nullptr);
            SessionImpl& S = T->impl;
            const size_t es = S.kv32 ? 4 : 2, run = (size_t)n * c.head_dim * es;
            const size_t bytes = run * c.layers * c.kv_heads;
            P->keys.alloc(bytes);
            P->values.alloc(bytes);
            // The session holds exactly n positions: its caches are the prefix's.
            TRIT_HIP(hipMemcpy(P->keys.ptr, S.kcache.ptr, bytes, hipMemcpyDeviceToDevice));
            TRIT_HIP(hipMemcpy(P->values.ptr, S.vcache.ptr, bytes, hipMemcpyDeviceToDevice));
            P->exact = S.exact;
            P->kv32 = S.kv32;
        } else {
            // The session flags' modes, as init_session reads them.
            P->exact = (flags & TRIT_HIP_EXACT) != 0 || (flags & TRIT_HIP_TREE_SUMS) == 0;
            P->kv32 = (flags & (TRIT_HIP_EXACT | TRIT_HIP_KV_F32)) != 0;
        }
        *out = P.release();
        return 0;
    });
}

void trit_hip_prefix_free(TritHipPrefix* prefix) { delete prefix; }

int trit_hip_session_prefill_prefixed(TritHipSession* session, const TritHipPrefix* prefix, const int32_t* tokens,
                                      int n, float* logits) {
    return guard(-1, [&] {
        if (!session || !prefix || !tokens) fail("prefill_prefixed: session, prefix or tokens is NULL");
        SessionImpl& S = session->impl;
        check_usable(S);
        if (prefix->dec != S.dec) fail("prefill_prefixed: the prefix belongs to another decoder");
        if (prefix->exact != S.exact || prefix->kv32 != S.kv32)
            fail("prefill_prefixed: the prefix was made with other session flags");
        if (S.host_pos != 0) fail("prefill_prefixed: the session holds positions; reset it first");
        const int p = (int)prefix->tokens.size();
        // Trit takes the prefix only for a longer prompt that starts with it.
        const bool take = n > p && std::equal(prefix->tokens.begin(), prefix->tokens.end(), tokens);
        if (!take || p == 0) return prefill_common(session, n, logits, tokens, nullptr);
        if (n > S.max_pos)
            fail("prefill: " + std::to_string(n) + " positions exceed the session's " + std::to_string(S.max_pos));
        const auto& c = S.dec->c;
        const size_t es = S.kv32 ? 4 : 2, run = (size_t)p * c.head_dim * es;
        const size_t pitch = (size_t)S.max_pos * c.head_dim * es;
        hipStream_t s = stream();
        TRIT_HIP(hipMemcpy2DAsync(S.kcache.ptr, pitch, prefix->keys.ptr, run, run, (size_t)c.layers * c.kv_heads,
                                  hipMemcpyDeviceToDevice, s));
        TRIT_HIP(hipMemcpy2DAsync(S.vcache.ptr, pitch, prefix->values.ptr, run, run, (size_t)c.layers * c.kv_heads,
                                  hipMemcpyDeviceToDevice, s));
        TRIT_HIP(hipStreamSynchronize(s));
        State h{};
        TRIT_HIP(hipMemcpy(&h, S.state.ptr, sizeof(State), hipMemcpyDeviceToHost));
        h.pos = p;
        TRIT_HIP(hipMemcpy(S.state.ptr, &h, sizeof(State), hipMemcpyHostToDevice));
        S.host_pos = p;
        return prefill_common(session, n - p, logits, tokens + p, nullptr);
    });
}

int trit_hip_session_reset(TritHipSession* session) {
    return guard(-1, [&] {
        if (!session) fail("session is NULL");
        reset_state(session->impl);
        return 0;
    });
}

int trit_hip_session_position(const TritHipSession* session) {
    return guard(-1, [&] {
        if (!session) fail("session is NULL");
        return session->impl.host_pos;
    });
}

void trit_hip_session_free(TritHipSession* session) { delete session; }

// Checks of attention_steps' arguments; returns head_dim and the shared
// memory of the largest sequence.
static int steps_check(const float* q, int qs, const float* const* keys, const float* const* values, const int* tk,
                       int sequences, int d, int heads, int kv_heads, const float* out, size_t* lds) {
    if (!q || !keys || !values || !tk || !out) fail("attention_steps: q, keys, values, tk or out is NULL");
    if (sequences <= 0 || sequences > STEPS_MAX) fail("attention_steps: 1 to 32 sequences");
    if (heads <= 0 || kv_heads <= 0 || heads % kv_heads)
        fail("attention_steps: the query heads do not share the key heads evenly");
    if (d <= 0 || d % heads) fail("attention_steps: d is not a multiple of the heads");
    const int hd = d / heads;
    if (hd > MAX_HD || hd % 8) fail("attention_steps: head_dim must be a multiple of 8 and at most 256");
    if (qs < d) fail("attention_steps: the query stride is shorter than d");
    int most = 0;
    for (int b = 0; b < sequences; ++b) {
        if (tk[b] <= 0) fail("attention_steps: sequence " + std::to_string(b) + " has no keys");
        if (!keys[b] || !values[b]) fail("attention_steps: sequence " + std::to_string(b) + " has NULL keys or values");
        most = std::max(most, tk[b]);
    }
    *lds = (size_t)(MAX_HD + most + ATT_THREADS) * 4;
    if (*lds > 64 * 1024) fail("attention_steps: more keys than one block's shared memory holds (16000)");
    return hd;
}

int trit_hip_attention_steps(const float* q, int qs, const float* const* keys, const float* const* values,
                             const int* tk, int sequences, int d, int heads, int kv_heads, float* out) {
    return guard(-1, [&] {
        size_t lds = 0;
        const int hd = steps_check(q, qs, keys, values, tk, sequences, d, heads, kv_heads, out, &lds);
        const size_t kvs = (size_t)kv_heads * hd;
        size_t rows = 0;
        for (int b = 0; b < sequences; ++b) rows += (size_t)tk[b];
        hipStream_t s = stream();
        const size_t qb = ((size_t)(sequences - 1) * qs + d) * 4, ob = (size_t)sequences * d * 4;
        DeviceMemory dq(qb), dk(rows * kvs * 4), dv(rows * kvs * 4), dout(ob);
        TRIT_HIP(hipMemcpyAsync(dq.ptr, q, qb, hipMemcpyHostToDevice, s));
        StepsTable table{};
        size_t at = 0;
        for (int b = 0; b < sequences; ++b) {
            const size_t bytes = (size_t)tk[b] * kvs * 4;
            TRIT_HIP(hipMemcpyAsync(dk.as<float>() + at, keys[b], bytes, hipMemcpyHostToDevice, s));
            TRIT_HIP(hipMemcpyAsync(dv.as<float>() + at, values[b], bytes, hipMemcpyHostToDevice, s));
            table.s[b] = StepsSeq{dk.as<float>() + at, dv.as<float>() + at, tk[b]};
            at += (size_t)tk[b] * kvs;
        }
        hipLaunchKernelGGL(attention_steps_kernel, dim3(heads, sequences), dim3(ATT_THREADS), lds, s, dq.as<float>(),
                           qs, table, heads, kv_heads, hd, d, dout.as<float>());
        TRIT_HIP(hipGetLastError());
        TRIT_HIP(hipMemcpyAsync(out, dout.ptr, ob, hipMemcpyDeviceToHost, s));
        TRIT_HIP(hipStreamSynchronize(s));
        return 0;
    });
}

int trit_hip_attention_steps_device(const float* q, int qs, const float* const* keys, const float* const* values,
                                    const int* tk, int sequences, int d, int heads, int kv_heads, float* out,
                                    void* stream_) {
    return guard(-1, [&] {
        size_t lds = 0;
        const int hd = steps_check(q, qs, keys, values, tk, sequences, d, heads, kv_heads, out, &lds);
        const size_t kvs = (size_t)kv_heads * hd;
        StepsTable table{};
        for (int b = 0; b < sequences; ++b) {
            // float4 loads of each key row.
            if (((uintptr_t)keys[b] | (uintptr_t)values[b]) % 16 || kvs % 4)
                fail("attention_steps: keys and values must be 16-byte aligned");
            table.s[b] = StepsSeq{keys[b], values[b], tk[b]};
        }
        hipStream_t s = stream_ ? (hipStream_t)stream_ : stream();
        hipLaunchKernelGGL(attention_steps_kernel, dim3(heads, sequences), dim3(ATT_THREADS), lds, s, q, qs, table,
                           heads, kv_heads, hd, d, out);
        TRIT_HIP(hipGetLastError());
        return 0;
    });
}

int trit_hip_attention(const float* q, int qs, const float* k, const float* v, int kvs, int tq, int tk, int heads,
                       int kv_heads, int hd, int causal, int flags, float* out) {
    return guard(-1, [&] {
        if (!q || !k || !v || !out) fail("attention: q, k, v or out is NULL");
        if (tq <= 0 || tk <= 0) fail("attention: no rows");
        if (heads <= 0 || kv_heads <= 0 || heads % kv_heads)
            fail("attention: the query heads do not share the key heads evenly");
        if (hd <= 0 || hd > MAX_HD || hd % 8) fail("attention: head_dim must be a multiple of 8 and at most 256");
        if (qs < heads * hd || kvs < kv_heads * hd) fail("attention: a row stride is shorter than its heads");
        if (causal && tq > tk) fail("attention: causal attention with more queries than keys");
        const bool exact = (flags & TRIT_HIP_EXACT) != 0;
        const int group = heads / kv_heads;
        if (!exact && (hd != 128 || (group != 1 && group != 2 && group != 4)))
            fail("attention: the fast form takes head_dim 128 and 1, 2 or 4 query heads per key head");
        if (exact && (size_t)(MAX_HD + tk + ATT_THREADS) * 4 > 64 * 1024)
            fail("attention: more keys than the exact kernel's shared memory holds (16000)");
        hipStream_t s = stream();
        const size_t qb = (size_t)tq * qs * 4, kb = (size_t)tk * kvs * 4, ob = (size_t)tq * heads * hd * 4;
        const size_t cache = (size_t)kv_heads * tk * hd * (exact ? 4 : 2);
        DeviceMemory dq(qb), dk(kb), dv(kb), dkc(cache), dvc(cache), dout(ob), dst(sizeof(State));
        TRIT_HIP(hipMemcpyAsync(dq.ptr, q, qb, hipMemcpyHostToDevice, s));
        TRIT_HIP(hipMemcpyAsync(dk.ptr, k, kb, hipMemcpyHostToDevice, s));
        TRIT_HIP(hipMemcpyAsync(dv.ptr, v, kb, hipMemcpyHostToDevice, s));
        const int grid = (int)std::min<size_t>(4096, ((size_t)tk * kv_heads * hd + 255) / 256);
        if (exact) {
            State st{};
            st.pos = tk - tq;
            TRIT_HIP(hipMemcpyAsync(dst.ptr, &st, sizeof(State), hipMemcpyHostToDevice, s));
            exact_attention(dq.as<float>(), qs, dk.as<float>(), dv.as<float>(), kvs, tq, tk, heads, kv_heads, hd,
                            causal, dout.as<float>(), dkc.as<float>(), dvc.as<float>(), dst.as<State>(), s);
        } else {
            hipLaunchKernelGGL(rows_to_cache_kernel<_Float16>, dim3(grid), dim3(256), 0, s, dk.as<float>(),
                               dv.as<float>(), kvs, tk, kv_heads, hd, dkc.as<_Float16>(), dvc.as<_Float16>());
            flash_attention(dq.as<float>(), qs, dkc.as<_Float16>(), dvc.as<_Float16>(), tk, heads, kv_heads, tq,
                            tk - tq, tk, causal, dout.as<float>(), s);
        }
        TRIT_HIP(hipGetLastError());
        TRIT_HIP(hipMemcpyAsync(out, dout.ptr, ob, hipMemcpyDeviceToHost, s));
        TRIT_HIP(hipStreamSynchronize(s));
        return 0;
    });
}

}  // extern "C"
