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
    if (!in_lds)
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
