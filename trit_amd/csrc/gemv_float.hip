// Float-math products (f16, f32 and int8-storage weights: token tables, the
// LM head, f16/f32 linears) in Trit's 16-lane sum order, bit for bit
// (src/cpu/fgemm.rs:413-455, src/cpu/v2/float.rs:1-30, 255-270): output j
// is reduce16(lanes) where lane i is the fused chain acc_i = fma(x[16s+i],
// w[16s+i], acc_i) over s in order from +0, and reduce16 adds lane i and
// i+8, then i+4, then i+2, then the last two. The weight is the f16 value
// widened (exact), the f32 value, or for int8 storage (Q8, gemm.rs:37-44,
// 117-187) f32(code) * scale of its 32-group, one rounding, as widen_q8
// makes the panel the f32 product reads.
//
// The device layout keeps each lane chain contiguous: element kk = 16s + i
// of row j lives at [j][i][s], so one thread streams its chain with 16-byte
// loads (8 f16, 4 f32 or 16 int8 values each) and 16 threads cover a row;
// Q8 scales stay row-major [j][kk / 32] (step s of any lane is in group
// s / 2). The tree is four cross-lane shuffles inside each 16-lane group;
// f32 addition commutes, so both lanes of a pair hold the same bits.
#include "device.h"
#include "internal.h"

#include <type_traits>

namespace trit {
namespace {

constexpr int THREADS = 256;
constexpr int MAXF = 8;
constexpr int ROWS = THREADS / 16;  // rows per block step

// Weight kinds: element type and elements per 16-byte unit.
enum WKind { WK_F16, WK_F32, WK_Q8 };
template <int K>
struct WT;
template <>
struct WT<WK_F16> {
    using E = uint16_t;
    static constexpr int PER = 8;
};
template <>
struct WT<WK_F32> {
    using E = float;
    static constexpr int PER = 4;
};
template <>
struct WT<WK_Q8> {
    using E = int8_t;
    static constexpr int PER = 16;
};

// Element h of a 16-byte unit as f32 (a Q8 code before its scale).
template <int K>
__device__ __forceinline__ float elem(const uint32_t (&words)[4], int h) {
    if constexpr (K == WK_F16) return f16_to_f32((uint16_t)(words[h >> 1] >> ((h & 1) * 16)));
    else if constexpr (K == WK_F32) return __uint_as_float(words[h]);
    else return (float)(int8_t)(uint8_t)(words[h >> 2] >> ((h & 3) * 8));
}

// One element of a chain, widened: w[s] (f16, f32) or f32(code) * scale.
template <int K>
__device__ __forceinline__ float widen1(const typename WT<K>::E* chain, const float* row_scales, int s) {
    if constexpr (K == WK_F16) return f16_to_f32(chain[s]);
    else if constexpr (K == WK_F32) return chain[s];
    else return (float)chain[s] * row_scales[s >> 1];
}

__device__ __forceinline__ void store_out(const GemvArgs& a, const float* __restrict__ bias, int n, int f, int row,
                                          float v) {
    if (bias) v = v + bias[row];
    if (a.relu) v = __builtin_fmaxf(v, 0.0f);
    const size_t at = (size_t)f * n + row;
    a.y[at] = a.epilogue == EPI_RESIDUAL ? a.residual[at] + v : v;
}

__device__ __forceinline__ float tree16(float v) {
    v = v + __shfl_xor(v, 8);
    v = v + __shfl_xor(v, 4);
    v = v + __shfl_xor(v, 2);
    v = v + __shfl_xor(v, 1);
    return v;
}

// f16 weights, k 1024 or 2048 (S8 = k / 128 16-byte loads a chain, all in
// registers), the rows staged in shared memory: the LM head's product.
template <int S8>
__global__ __launch_bounds__(THREADS) void f16_kernel(const uint16_t* __restrict__ w, const float* __restrict__ bias,
                                                      int n, int k, GemvArgs a) {
    extern __shared__ __align__(16) float xs[];  // m x k
    if (a.skip && *a.skip) return;
    const int m = a.m;
    for (int i = threadIdx.x; i < m * k; i += THREADS) xs[i] = a.x[i];
    __syncthreads();
    const int lane = threadIdx.x & 15;
    const int s_count = k / 16;
    const int steps = (n + ROWS - 1) / ROWS;
    for (int step = blockIdx.x; step < steps; step += gridDim.x) {
        const int row = step * ROWS + (int)(threadIdx.x >> 4);
        const bool live = row < n;
        const uint16_t* chain = w + ((size_t)(live ? row : 0) * 16 + lane) * (size_t)s_count;
        uint4 wv[S8];
#pragma unroll
        for (int j = 0; j < S8; ++j) wv[j] = ((const uint4*)chain)[j];
        // Rows one after the other: the chain's weights stay in registers.
#pragma unroll 1
        for (int f = 0; f < m; ++f) {
            const float* xf = xs + (size_t)f * k + lane;
            float acc = 0.0f;
#pragma unroll
            for (int j = 0; j < S8; ++j) {
                const uint32_t words[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
#pragma unroll
                for (int h = 0; h < 8; ++h) acc = __builtin_fmaf(xf[16 * (j * 8 + h)], elem<WK_F16>(words, h), acc);
            }
            const float v = tree16(acc);
            if (live && lane == 0) store_out(a, bias, n, f, row, v);
        }
    }
}

// Any kind and k (any k for f16 and f32, a multiple of 32 for Q8): one
// element load a step, the rows read in place (shared memory when they
// fit, else global memory, where they stay in the caches). Past k the
// chains add 0 * 0 (zero weights in the layout, the inputs masked): Trit's
// tail padded with zeros.
template <int K, bool LDS>
__global__ __launch_bounds__(THREADS) void float_any_kernel(const typename WT<K>::E* __restrict__ w,
                                                            const float* __restrict__ scales,
                                                            const float* __restrict__ bias, int n, int k, GemvArgs a) {
    extern __shared__ __align__(16) float xs_lds[];  // m x k
    if (a.skip && *a.skip) return;
    const int m = a.m;
    const float* xs = a.x;
    if constexpr (LDS) {
        for (int i = threadIdx.x; i < m * k; i += THREADS) xs_lds[i] = a.x[i];
        __syncthreads();
        xs = xs_lds;
    }
    const int lane = threadIdx.x & 15;
    const int s_count = chain_steps(k);
    const int steps = (n + ROWS - 1) / ROWS;
    for (int step = blockIdx.x; step < steps; step += gridDim.x) {
        const int row = step * ROWS + (int)(threadIdx.x >> 4);
        const bool live = row < n;
        const int rr = live ? row : 0;
        const typename WT<K>::E* chain = w + ((size_t)rr * 16 + lane) * (size_t)s_count;
        const float* row_scales = scales ? scales + (size_t)rr * (k / 32) : nullptr;
#pragma unroll 1
        for (int f = 0; f < m; ++f) {
            const float* xf = xs + (size_t)f * k + lane;
            float acc = 0.0f;
            for (int sidx = 0; sidx < s_count; ++sidx) {
                const float xv = 16 * sidx + lane < k ? xf[16 * sidx] : 0.0f;
                acc = __builtin_fmaf(xv, widen1<K>(chain, row_scales, sidx), acc);
            }
            const float v = tree16(acc);
            if (live && lane == 0) store_out(a, bias, n, f, row, v);
        }
    }
}

// Any kind, k a multiple of 16 * PER (rows 16-byte aligned). With SPLIT a
// block takes R = 16 / m output rows, and each 16-lane group of its
// threads one (row, input row) pair: the chains of the m input rows run on
// different threads, so a few output rows still fill many waves; else a
// block takes 16 rows and each thread runs the chains of all m input rows
// (for many output rows, where the staging below is the cost). The m
// input rows are staged in shared memory in segments of `seg` chain steps,
// transposed so that lane i's values of consecutive steps s are contiguous
// ([row][i][s], the pitch padded to spread the lanes over the banks); the
// chains continue across segments in s order, their weights (and Q8
// scales) streamed in batches of CH 16-byte units with the next batch in
// flight (weights shared by the m threads of a row come from the caches).
template <int K, int CH, bool SPLIT, int SB = 8>
__global__ __launch_bounds__(THREADS) void float_chunked_kernel(const typename WT<K>::E* __restrict__ w,
                                                                const float* __restrict__ scales,
                                                                const float* __restrict__ bias, int n, int k, int seg,
                                                                GemvArgs a) {
    constexpr int PER = WT<K>::PER;
    extern __shared__ __align__(16) float xt[];  // m x 16 x (seg + 4)
    if (a.skip && *a.skip) return;
    const int m = a.m, R = SPLIT ? ROWS / m : ROWS;
    const int lane = threadIdx.x & 15, slot = threadIdx.x >> 4;
    const int r = SPLIT ? slot / m : slot, f0 = SPLIT ? slot - r * m : 0, nf = SPLIT ? 1 : m;
    constexpr int NF = SPLIT ? 1 : MAXF;
    constexpr int NS = K == WK_Q8 ? 2 : 1;  // float4s of scales a unit (8 groups)
    const int s_count = k / 16, pitch = seg + 4;
    const int steps = (n + R - 1) / R;
    for (int step = blockIdx.x; step < steps; step += gridDim.x) {
        const int row = step * R + r;
        const bool live = r < R && row < n;
        const int rr = live ? row : 0;
        const uint4* chain = (const uint4*)(w + ((size_t)rr * 16 + lane) * (size_t)s_count);
        const float4* row_scales = (const float4*)(scales + (K == WK_Q8 ? (size_t)rr * (k / 32) : 0));
        const float* xrow = xt + (f0 * 16 + lane) * pitch;
        float acc[NF];
#pragma unroll
        for (int ff = 0; ff < NF; ++ff) acc[ff] = 0.0f;
        const int total = s_count / PER;  // units in the chain
        uint4 cur[CH], nxt[CH];
        float4 scur[CH][NS], snxt[CH][NS];
#pragma unroll
        for (int j = 0; j < CH; ++j)
            if (j < total) {
                cur[j] = chain[j];
                if constexpr (K == WK_Q8) {
                    scur[j][0] = row_scales[2 * j];
                    scur[j][1] = row_scales[2 * j + 1];
                }
            }
        int at = 0;
        for (int s0 = 0; s0 < s_count; s0 += seg) {
            const int sn = s_count - s0 < seg ? s_count - s0 : seg;
            __syncthreads();  // the previous segment is read
            // 16-byte loads (4 lanes of one step), SB of them in flight.
            const int total4 = m * 4 * sn;
            for (int base = 0; base < total4; base += THREADS * SB) {
                float4 v[SB];
#pragma unroll
                for (int u = 0; u < SB; ++u) {
                    const int idx = base + u * THREADS + (int)threadIdx.x;
                    if (idx < total4) {
                        const int ff = idx / (4 * sn), q = idx - ff * 4 * sn;
                        v[u] = *(const float4*)(a.x + (size_t)ff * k + 16 * (s0 + (q >> 2)) + (q & 3) * 4);
                    }
                }
#pragma unroll
                for (int u = 0; u < SB; ++u) {
                    const int idx = base + u * THREADS + (int)threadIdx.x;
                    if (idx < total4) {
                        const int ff = idx / (4 * sn), q = idx - ff * 4 * sn;
                        float* to = xt + (ff * 16 + (q & 3) * 4) * pitch + (q >> 2);
                        to[0] = v[u].x;
                        to[pitch] = v[u].y;
                        to[2 * pitch] = v[u].z;
                        to[3 * pitch] = v[u].w;
                    }
                }
            }
            __syncthreads();
            // Batches never straddle segments (seg is a multiple of PER * CH).
            const int end = (s0 + sn) / PER;
            for (; at < end; at += CH) {
#pragma unroll
                for (int j = 0; j < CH; ++j)
                    if (at + CH + j < total) {
                        nxt[j] = chain[at + CH + j];
                        if constexpr (K == WK_Q8) {
                            snxt[j][0] = row_scales[2 * (at + CH + j)];
                            snxt[j][1] = row_scales[2 * (at + CH + j) + 1];
                        }
                    }
#pragma unroll
                for (int j = 0; j < CH; ++j) {
                    if (at + j >= end) break;
                    const uint32_t words[4] = {cur[j].x, cur[j].y, cur[j].z, cur[j].w};
                    float wf[PER];
#pragma unroll
                    for (int h = 0; h < PER; ++h) {
                        wf[h] = elem<K>(words, h);
                        if constexpr (K == WK_Q8) {
                            const float sc[8] = {scur[j][0].x, scur[j][0].y, scur[j][0].z, scur[j][0].w,
                                                 scur[j][1].x, scur[j][1].y, scur[j][1].z, scur[j][1].w};
                            wf[h] = wf[h] * sc[h >> 1];
                        }
                    }
#pragma unroll
                    for (int ff = 0; ff < NF; ++ff) {
                        if (ff >= nf) break;
                        const float4* xp = (const float4*)(xrow + ff * 16 * pitch + (at + j) * PER - s0);
#pragma unroll
                        for (int q = 0; q < PER / 4; ++q) {
                            const float4 xq = xp[q];
                            acc[ff] = __builtin_fmaf(xq.x, wf[4 * q], acc[ff]);
                            acc[ff] = __builtin_fmaf(xq.y, wf[4 * q + 1], acc[ff]);
                            acc[ff] = __builtin_fmaf(xq.z, wf[4 * q + 2], acc[ff]);
                            acc[ff] = __builtin_fmaf(xq.w, wf[4 * q + 3], acc[ff]);
                        }
                    }
                }
#pragma unroll
                for (int j = 0; j < CH; ++j) {
                    cur[j] = nxt[j];
                    if constexpr (K == WK_Q8) {
                        scur[j][0] = snxt[j][0];
                        scur[j][1] = snxt[j][1];
                    }
                }
            }
        }
#pragma unroll
        for (int ff = 0; ff < NF; ++ff) {
            if (ff >= nf) break;
            const float v = tree16(acc[ff]);
            if (live && lane == 0) store_out(a, bias, n, f0 + ff, row, v);
        }
    }
}

// Many input rows of a layer with few inputs (k <= 16 S; an audio stem's
// first convolution): block (x, y) takes 256 output columns and RB input
// rows; a thread holds its column's 16 lane chains (S steps each) in
// registers and runs them over the rows, then the tree16 order of the
// small-batch kernels, so every row gets their bits.
template <int K, int S>
__global__ __launch_bounds__(THREADS) void float_rows_kernel(const typename WT<K>::E* __restrict__ w,
                                                             const float* __restrict__ scales,
                                                             const float* __restrict__ bias, int n, int k, GemvArgs a) {
    constexpr int RB = 64;
    const int col = blockIdx.x * THREADS + (int)threadIdx.x;
    if (col >= n) return;
    const int s_count = chain_steps(k);  // <= S
    float wr[16][S];
#pragma unroll
    for (int i = 0; i < 16; ++i)
#pragma unroll
        for (int st = 0; st < S; ++st)
            wr[i][st] = st < s_count ? widen1<K>(w + ((size_t)col * 16 + i) * s_count,
                                                 scales ? scales + (size_t)col * (k / 32) : nullptr, st)
                                     : 0.0f;
    const int f1 = min(a.m, (int)(blockIdx.y + 1) * RB);
    for (int f = blockIdx.y * RB; f < f1; ++f) {
        const float* xf = a.x + (size_t)f * k;
        float l[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float acc = 0.0f;
#pragma unroll
            for (int st = 0; st < S; ++st) {
                const int kk = 16 * st + i;
                acc = __builtin_fmaf(kk < k ? xf[kk] : 0.0f, wr[i][st], acc);
            }
            l[i] = acc;
        }
        float h[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) h[i] = l[i] + l[i + 8];
        const float v = ((h[0] + h[4]) + (h[2] + h[6])) + ((h[1] + h[5]) + (h[3] + h[7]));
        store_out(a, bias, n, f, col, v);
    }
}

// Lane-chain layout from row-major weights (the padding past k is left as
// the caller cleared it).
template <typename E>
__global__ void repack_kernel(const E* __restrict__ src, int n, int k, E* __restrict__ dst) {
    const size_t total = (size_t)n * k;
    const int s_count = chain_steps(k);
    for (size_t e = blockIdx.x * (size_t)blockDim.x + threadIdx.x; e < total; e += (size_t)gridDim.x * blockDim.x) {
        const size_t row = e / k;
        const int kk = (int)(e - row * k);
        const int sidx = kk / 16, i = kk % 16;
        dst[(row * 16 + i) * s_count + sidx] = src[e];
    }
}

// Row `index` widened (Dense::row, src/cpu/gemm.rs:412-429).
template <int K>
__global__ void row_kernel(const typename WT<K>::E* __restrict__ w, const float* __restrict__ scales, int k,
                           int index, float* __restrict__ out) {
    const int s_count = chain_steps(k);
    const typename WT<K>::E* base = w + (size_t)index * 16 * s_count;
    const float* row_scales = scales ? scales + (size_t)index * (k / 32) : nullptr;
    for (int kk = threadIdx.x; kk < k; kk += blockDim.x) {
        const int sidx = kk / 16, i = kk % 16;
        if constexpr (K == WK_Q8) out[kk] = (float)base[i * s_count + sidx] * row_scales[kk / 32];
        else out[kk] = widen1<K>(base + i * s_count, nullptr, sidx);
    }
}

template <int K>
void launch_float(const Layer& L, const GemvArgs& a, hipStream_t s) {
    using E = typename WT<K>::E;
    constexpr int PER = WT<K>::PER, CH = 4;
    const E* w = L.codes.as<E>();
    const float* sc = K == WK_Q8 ? L.scales.as<float>() : nullptr;
    const float* b = L.bias.as<float>();
    const size_t bytes = (size_t)a.m * L.k * 4;
    const bool in_lds = bytes <= 64 * 1024;
    const int steps = (L.n + ROWS - 1) / ROWS;
    const int grid = steps < 4096 ? steps : 4096;
    // (The chunked kernel stages the rows with 16-byte loads.)
    const bool aligned = ((uintptr_t)a.x & 15) == 0;
    if constexpr (K == WK_F16) {
        if (in_lds && (L.k == 1024 || L.k == 2048)) {
            if (L.k == 1024)
                launch_timed(a, f16_kernel<8>, dim3(grid), dim3(THREADS), bytes, s, w, b, L.n, L.k, a);
            else
                launch_timed(a, f16_kernel<16>, dim3(grid), dim3(THREADS), bytes, s, w, b, L.n, L.k, a);
            return;
        }
    }
    if (L.k % (16 * PER) == 0 && aligned) {
        // Segments of chain steps whose m x 16 x (seg + 4) floats fit 64 KB.
        int seg = (1024 / a.m - 4) / (PER * CH) * (PER * CH);
        if (seg > L.k / 16) seg = L.k / 16;
        const size_t seg_lds = (size_t)a.m * 16 * (seg + 4) * 4;
        // Split the input rows over threads while that makes at most 1024
        // blocks (each stages the input rows).
        const int R = ROWS / a.m, csteps = (L.n + R - 1) / R;
        if (a.m > 1 && csteps <= 1024)
            launch_timed(a, float_chunked_kernel<K, CH, true>, dim3(csteps < 4096 ? csteps : 4096), dim3(THREADS),
                         seg_lds, s, w, sc, b, L.n, L.k, seg, a);
        else
            launch_timed(a, float_chunked_kernel<K, CH, false>, dim3(grid), dim3(THREADS), seg_lds, s, w, sc, b, L.n,
                         L.k, seg, a);
        return;
    }
    if (in_lds)
        launch_timed(a, float_any_kernel<K, true>, dim3(grid), dim3(THREADS), bytes, s, w, sc, b, L.n, L.k, a);
    else
        launch_timed(a, float_any_kernel<K, false>, dim3(grid), dim3(THREADS), 0, s, w, sc, b, L.n, L.k, a);
}

}  // namespace

void gemv_float(const Layer& L, const GemvArgs& a, hipStream_t s) {
    if (a.m < 1 || a.m > MAXF) fail("float gemv: 1 to 8 rows per call");
    if (a.epilogue == EPI_SILU_PAIR) fail("float gemv: no SwiGLU pair epilogue");
    if (a.norm_w) fail("float gemv: no RMSNorm prologue");
    switch (L.kind) {
        case F16: launch_float<WK_F16>(L, a, s); break;
        case F32: launch_float<WK_F32>(L, a, s); break;
        case Q8_F32: launch_float<WK_Q8>(L, a, s); break;
        default: fail("float gemv: not a float-math layer");
    }
    TRIT_HIP(hipGetLastError());
}

bool gemm_float_supported(const Layer& L, const GemvArgs& a) {
    return float_kind(L.kind) && L.k <= 128 && a.m >= 1 && !a.norm_w && a.epilogue != EPI_SILU_PAIR;
}

void gemm_float(const Layer& L, const GemvArgs& a, hipStream_t s) {
    if (!gemm_float_supported(L, a)) fail("float rows: a float-math layer of k <= 128, no prologue or pair");
    auto go = [&](auto K_, auto S_) {
        constexpr int K = decltype(K_)::value, S = decltype(S_)::value;
        using E = typename WT<K>::E;
        const dim3 grid((L.n + THREADS - 1) / THREADS, (a.m + 63) / 64);
        launch_timed(a, float_rows_kernel<K, S>, grid, dim3(THREADS), 0, s, L.codes.as<E>(),
                     K == WK_Q8 ? L.scales.as<float>() : nullptr, L.bias.as<float>(), L.n, L.k, a);
    };
    auto by_steps = [&](auto K_) {
        const int steps = chain_steps(L.k);
        if (steps <= 1) go(K_, std::integral_constant<int, 1>{});
        else if (steps <= 2) go(K_, std::integral_constant<int, 2>{});
        else if (steps <= 4) go(K_, std::integral_constant<int, 4>{});
        else go(K_, std::integral_constant<int, 8>{});
    };
    switch (L.kind) {
        case F16: by_steps(std::integral_constant<int, WK_F16>{}); break;
        case F32: by_steps(std::integral_constant<int, WK_F32>{}); break;
        default: by_steps(std::integral_constant<int, WK_Q8>{}); break;
    }
    TRIT_HIP(hipGetLastError());
}

void float_repack(const void* src, int kind, int n, int k, void* dst, hipStream_t s) {
    if (kind == F16)
        hipLaunchKernelGGL(repack_kernel<uint16_t>, dim3(4096), dim3(256), 0, s, (const uint16_t*)src, n, k,
                           (uint16_t*)dst);
    else if (kind == F32)
        hipLaunchKernelGGL(repack_kernel<float>, dim3(4096), dim3(256), 0, s, (const float*)src, n, k, (float*)dst);
    else
        hipLaunchKernelGGL(repack_kernel<int8_t>, dim3(4096), dim3(256), 0, s, (const int8_t*)src, n, k,
                           (int8_t*)dst);
    TRIT_HIP(hipGetLastError());
}

void float_row(const Layer& L, int index, float* out, hipStream_t s) {
    if (L.kind == F16)
        hipLaunchKernelGGL(row_kernel<WK_F16>, dim3(1), dim3(256), 0, s, L.codes.as<uint16_t>(), nullptr, L.k, index,
                           out);
    else if (L.kind == F32)
        hipLaunchKernelGGL(row_kernel<WK_F32>, dim3(1), dim3(256), 0, s, L.codes.as<float>(), nullptr, L.k, index,
                           out);
    else if (L.kind == Q8_F32)
        hipLaunchKernelGGL(row_kernel<WK_Q8>, dim3(1), dim3(256), 0, s, L.codes.as<int8_t>(), L.scales.as<float>(),
                           L.k, index, out);
    else
        fail("row: not a token table");
    TRIT_HIP(hipGetLastError());
}

}  // namespace trit
