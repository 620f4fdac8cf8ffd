// f16-weight GEMV (token tables, the tied LM head) in Trit's 16-lane sum
// order, bit for bit (src/cpu/fgemm.rs:413-455, src/cpu/v2/float.rs:1-30,
// 255-270): output j is reduce16(lanes) where lane i is the fused chain
// acc_i = fma(x[16s+i], w[16s+i], acc_i) over s in order from +0, and
// reduce16 adds lane i and i+8, then i+4, then i+2, then the last two.
//
// The device layout keeps each lane chain contiguous: element kk = 16s + i
// of row j lives at [j][i][s], so one thread streams its chain with 16-byte
// loads (8 f16 values each) and 16 threads cover a row. The tree is four
// cross-lane shuffles inside each 16-lane group; f32 addition commutes, so
// both lanes of a pair hold the same bits.
#include "device.h"
#include "internal.h"

namespace trit {
namespace {

constexpr int THREADS = 256;
constexpr int MAXF = 8;
constexpr int ROWS = THREADS / 16;  // rows per block step

// S8 = 16-byte loads per chain (k / 128); 0: any k (2-byte loads). LDS:
// the rows are staged in shared memory; else (m x k above 64 KB) every
// block reads them from global memory, where they stay in the caches.
template <int S8, bool LDS>
__global__ __launch_bounds__(THREADS) void f16_kernel(const uint16_t* __restrict__ w, const float* __restrict__ bias,
                                                      int n, int k, GemvArgs a) {
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
    const int s_count = k / 16;
    const int steps = (n + ROWS - 1) / ROWS;
    for (int step = blockIdx.x; step < steps; step += gridDim.x) {
        const int row = step * ROWS + (int)(threadIdx.x >> 4);
        const bool live = row < n;
        const uint16_t* chain = w + ((size_t)(live ? row : 0) * 16 + lane) * (size_t)s_count;
        uint4 wv[S8 > 0 ? S8 : 1];
        if constexpr (S8 > 0) {
#pragma unroll
            for (int j = 0; j < S8; ++j) wv[j] = ((const uint4*)chain)[j];
        }
        // Frames one after the other: the chain's weights stay in registers.
#pragma unroll 1
        for (int f = 0; f < m; ++f) {
            const float* xf = xs + (size_t)f * k + lane;
            float acc = 0.0f;
            if constexpr (S8 > 0) {
#pragma unroll
                for (int j = 0; j < S8; ++j) {
                    const uint32_t words[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
#pragma unroll
                    for (int h = 0; h < 8; ++h) {
                        const int s = j * 8 + h;
                        const float wf = f16_to_f32((uint16_t)(words[h >> 1] >> ((h & 1) * 16)));
                        acc = __builtin_fmaf(xf[16 * s], wf, acc);
                    }
                }
            } else {
                for (int s = 0; s < s_count; ++s) acc = __builtin_fmaf(xf[16 * s], f16_to_f32(chain[s]), acc);
            }
            float v = acc;
            v = v + __shfl_xor(v, 8);
            v = v + __shfl_xor(v, 4);
            v = v + __shfl_xor(v, 2);
            v = v + __shfl_xor(v, 1);
            if (live && lane == 0) {
                if (bias) v = v + bias[row];
                if (a.relu) v = __builtin_fmaxf(v, 0.0f);
                const size_t at = (size_t)f * n + row;
                a.y[at] = a.epilogue == EPI_RESIDUAL ? a.residual[at] + v : v;
            }
        }
    }
}

// Any k that is a multiple of 128 (rows 16-byte aligned). With SPLIT a
// block takes R = 16 / m output rows, and each 16-lane group of its
// threads one (row, input row) pair: the chains of the m input rows run on
// different threads, so a few output rows still fill many waves; else a
// block takes 16 rows and each thread runs the chains of all m input rows
// (for many output rows, where the staging below is the cost). The m input rows
// are staged in shared memory in segments of `seg` chain steps,
// transposed so that lane i's values of 8 consecutive steps s are 32
// contiguous bytes ([row][i][s], the pitch padded to spread the lanes over
// the banks); the chains continue across segments in s order, their
// weights streamed in batches of CH 16-byte loads with the next batch in
// flight (weights shared by the m threads of a row come from the caches).
template <int CH, bool SPLIT, int SB = 8>
__global__ __launch_bounds__(THREADS) void f16_chunked_kernel(const uint16_t* __restrict__ w,
                                                              const float* __restrict__ bias, int n, int k, int seg,
                                                              GemvArgs a) {
    extern __shared__ __align__(16) float xt[];  // m x 16 x (seg + 4)
    if (a.skip && *a.skip) return;
    const int m = a.m, R = SPLIT ? ROWS / m : ROWS;
    const int lane = threadIdx.x & 15, slot = threadIdx.x >> 4;
    const int r = SPLIT ? slot / m : slot, f0 = SPLIT ? slot - r * m : 0, nf = SPLIT ? 1 : m;
    constexpr int NF = SPLIT ? 1 : MAXF;
    const int s_count = k / 16, pitch = seg + 4;
    const int steps = (n + R - 1) / R;
    for (int step = blockIdx.x; step < steps; step += gridDim.x) {
        const int row = step * R + r;
        const bool live = r < R && row < n;
        const uint4* chain = (const uint4*)(w + ((size_t)(live ? row : 0) * 16 + lane) * (size_t)s_count);
        const float* xrow = xt + (f0 * 16 + lane) * pitch;
        float acc[NF];
#pragma unroll
        for (int ff = 0; ff < NF; ++ff) acc[ff] = 0.0f;
        const int total = s_count / 8;
        uint4 cur[CH], nxt[CH];
#pragma unroll
        for (int j = 0; j < CH; ++j)
            if (j < total) cur[j] = chain[j];
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
                        const int ff = idx / (4 * sn), rr = idx - ff * 4 * sn;
                        v[u] = *(const float4*)(a.x + (size_t)ff * k + 16 * (s0 + (rr >> 2)) + (rr & 3) * 4);
                    }
                }
#pragma unroll
                for (int u = 0; u < SB; ++u) {
                    const int idx = base + u * THREADS + (int)threadIdx.x;
                    if (idx < total4) {
                        const int ff = idx / (4 * sn), rr = idx - ff * 4 * sn;
                        float* to = xt + (ff * 16 + (rr & 3) * 4) * pitch + (rr >> 2);
                        to[0] = v[u].x;
                        to[pitch] = v[u].y;
                        to[2 * pitch] = v[u].z;
                        to[3 * pitch] = v[u].w;
                    }
                }
            }
            __syncthreads();
            // Batches never straddle segments (seg is a multiple of 8 * CH).
            const int end = (s0 + sn) / 8;
            for (; at < end; at += CH) {
#pragma unroll
                for (int j = 0; j < CH; ++j)
                    if (at + CH + j < total) nxt[j] = chain[at + CH + j];
#pragma unroll
                for (int j = 0; j < CH; ++j) {
                    if (at + j >= end) break;
                    const uint32_t words[4] = {cur[j].x, cur[j].y, cur[j].z, cur[j].w};
                    float wf[8];
#pragma unroll
                    for (int h = 0; h < 8; ++h) wf[h] = f16_to_f32((uint16_t)(words[h >> 1] >> ((h & 1) * 16)));
#pragma unroll
                    for (int ff = 0; ff < NF; ++ff) {
                        if (ff >= nf) break;
                        const float4* xp = (const float4*)(xrow + ff * 16 * pitch + (at + j) * 8 - s0);
                        const float4 x0 = xp[0], x1 = xp[1];
                        const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                        for (int h = 0; h < 8; ++h) acc[ff] = __builtin_fmaf(xv[h], wf[h], acc[ff]);
                    }
                }
#pragma unroll
                for (int j = 0; j < CH; ++j) cur[j] = nxt[j];
            }
        }
#pragma unroll
        for (int ff = 0; ff < NF; ++ff) {
            if (ff >= nf) break;
            float v = acc[ff];
            v = v + __shfl_xor(v, 8);
            v = v + __shfl_xor(v, 4);
            v = v + __shfl_xor(v, 2);
            v = v + __shfl_xor(v, 1);
            if (live && lane == 0) {
                if (bias) v = v + bias[row];
                if (a.relu) v = __builtin_fmaxf(v, 0.0f);
                const size_t at_y = (size_t)(f0 + ff) * n + row;
                a.y[at_y] = a.epilogue == EPI_RESIDUAL ? a.residual[at_y] + v : v;
            }
        }
    }
}

// Lane-chain layout from row-major f16.
__global__ void repack_kernel(const uint16_t* __restrict__ src, int n, int k, uint16_t* __restrict__ dst) {
    const size_t total = (size_t)n * k;
    const int s_count = k / 16;
    for (size_t e = blockIdx.x * (size_t)blockDim.x + threadIdx.x; e < total; e += (size_t)gridDim.x * blockDim.x) {
        const size_t row = e / k;
        const int kk = (int)(e - row * k);
        const int s = kk / 16, i = kk % 16;
        dst[(row * 16 + i) * s_count + s] = src[e];
    }
}

__global__ void row_kernel(const uint16_t* __restrict__ w, int k, int index, float* __restrict__ out) {
    const int s_count = k / 16;
    for (int kk = threadIdx.x; kk < k; kk += blockDim.x) {
        const int s = kk / 16, i = kk % 16;
        out[kk] = f16_to_f32(w[((size_t)index * 16 + i) * s_count + s]);
    }
}

}  // namespace

void gemv_f16(const Layer& L, const GemvArgs& a, hipStream_t s) {
    if (a.m < 1 || a.m > MAXF) fail("f16 gemv: 1 to 8 rows per call");
    if (a.epilogue == EPI_SILU_PAIR) fail("f16 gemv: no SwiGLU pair epilogue");
    const size_t bytes = (size_t)a.m * L.k * 4;
    const bool in_lds = bytes <= 64 * 1024;
    const size_t lds = in_lds ? bytes : 0;
    const int steps = (L.n + ROWS - 1) / ROWS;
    const int grid = steps < 4096 ? steps : 4096;
    const uint16_t* w = L.codes.as<uint16_t>();
    const float* b = L.bias.as<float>();
    // (The chunked kernel stages the rows with 16-byte loads.)
    const bool aligned = ((uintptr_t)a.x & 15) == 0;
    if (L.k % 128 == 0 && aligned && ((L.k != 1024 && L.k != 2048) || !in_lds)) {
        // Segments of chain steps whose m x 16 x (seg + 4) floats fit 64 KB.
        constexpr int CH = 4;
        int seg = (1024 / a.m - 4) / (8 * CH) * (8 * CH);
        if (seg > L.k / 16) seg = L.k / 16;
        const size_t seg_lds = (size_t)a.m * 16 * (seg + 4) * 4;
        // Split the input rows over threads while that makes at most 1024
        // blocks (each stages the input rows).
        const int R = ROWS / a.m, csteps = (L.n + R - 1) / R;
        if (a.m > 1 && csteps <= 1024) {
            launch_timed(a, f16_chunked_kernel<CH, true>, dim3(csteps < 4096 ? csteps : 4096), dim3(THREADS),
                         seg_lds, s, w, b, L.n, L.k, seg, a);
        } else {
            launch_timed(a, f16_chunked_kernel<CH, false>, dim3(grid), dim3(THREADS), seg_lds, s, w, b, L.n, L.k,
                         seg, a);
        }
    } else if (!in_lds)
        launch_timed(a, f16_kernel<0, false>, dim3(grid), dim3(THREADS), lds, s, w, b, L.n, L.k, a);
    else if (L.k == 1024)
        launch_timed(a, f16_kernel<8, true>, dim3(grid), dim3(THREADS), lds, s, w, b, L.n, L.k, a);
    else if (L.k == 2048)
        launch_timed(a, f16_kernel<16, true>, dim3(grid), dim3(THREADS), lds, s, w, b, L.n, L.k, a);
    else
        launch_timed(a, f16_kernel<0, true>, dim3(grid), dim3(THREADS), lds, s, w, b, L.n, L.k, a);
    TRIT_HIP(hipGetLastError());
}

void f16_repack(const uint16_t* src, int n, int k, uint16_t* dst, hipStream_t s) {
    hipLaunchKernelGGL(repack_kernel, dim3(4096), dim3(256), 0, s, src, n, k, dst);
    TRIT_HIP(hipGetLastError());
}

void f16_row(const Layer& L, int index, float* out, hipStream_t s) {
    hipLaunchKernelGGL(row_kernel, dim3(1), dim3(256), 0, s, L.codes.as<uint16_t>(), L.k, index, out);
    TRIT_HIP(hipGetLastError());
}

}  // namespace trit
