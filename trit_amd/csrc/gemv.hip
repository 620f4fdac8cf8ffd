// Integer GEMV for decode (batch 1..8): Q8_0 (and Q4_K requantized to it),
// Trit int8 with 128-value groups, and ternary 2-bit codes.
//
// The values are Trit's, bit for bit (src/cpu/int8.rs:525-584,
// src/cpu/kernels.rs:353-420, src/cpu/v2/product.rs:389-423):
//   y[f][r] = chain over groups g in order of
//             total = fma(f32(dot_g), ws[r][g] * xs[f][g], total), from +0,
// where dot_g is the exact i32 dot product of the group's weight codes and
// the activation codes of Trit's quantizer (src/cpu/kernels.rs:661-807).
//
// Work split (one workgroup of 256 threads, 4 waves):
//  1. the block quantizes the m activation rows into LDS (optionally after
//     Trit's RMSNorm, src/layers.rs:136-144);
//  2. it walks tiles of R rows (P parts of R rows for the SwiGLU pair);
//     each thread streams 16-byte chunks of weight codes (a wave reads
//     1 KB per instruction, rows contiguous), dots them with the LDS codes
//     by sdot4, and the lanes of one group add their partial i32 sums with
//     cross-lane shuffles; the group's leader lane parks the exact dot in
//     LDS;
//  3. one thread per (row, frame) runs the f32 chain over the groups in
//     Trit's order and applies the epilogue.
#include "device.h"
#include "internal.h"

namespace trit {
namespace {

constexpr int THREADS = 256;
constexpr int MAXF = 8;
constexpr int BATCH = 4;  // 16-byte chunks a thread has in flight

// Weight kinds: G inputs per scale, KPC inputs per 16-byte chunk, LPG
// chunks (lanes) per group.
struct Q8 {
    static constexpr int G = 32, KPC = 16, LPG = 2, ROW_DIV = 1;
    static constexpr bool HALF = true, TERN = false;
    __device__ static float scale(const void* s, size_t i) { return f16_to_f32(((const uint16_t*)s)[i]); }
};
struct I8 {
    static constexpr int G = 128, KPC = 16, LPG = 8, ROW_DIV = 1;
    static constexpr bool HALF = false, TERN = false;
    __device__ static float scale(const void* s, size_t i) { return ((const float*)s)[i]; }
};
struct T2 {
    static constexpr int G = 128, KPC = 64, LPG = 2, ROW_DIV = 4;
    static constexpr bool HALF = false, TERN = true;
    __device__ static float scale(const void* s, size_t i) { return ((const float*)s)[i]; }
};

struct Smem {
    int8_t* xq;    // m x k codes
    float* xs;     // m x G scales
    int* xsum;     // m x G code sums (ternary)
    float* inv;    // m norm factors
    float* red;    // THREADS floats of scratch
    int* dots;     // (P*R*m) x (G+1)
    float* ws;     // P*R x G weight scales
    float* res;    // P*R*m chain results (pair epilogue)
};

__device__ __forceinline__ size_t align16(size_t v) { return (v + 15) & ~(size_t)15; }

// Quantizes the m rows of x into LDS with Trit's rule, optionally after
// RMSNorm: x * (inv * w).
template <class W>
__device__ void quantize_rows(const GemvArgs& a, int k, const Smem& sm) {
    constexpr int TPG = W::G / 4;
    const int groups = k / W::G;
    const int m = a.m;
    if (a.norm_w) {
        if (a.norm_inv) {
            if (threadIdx.x < m) sm.inv[threadIdx.x] = a.norm_inv[threadIdx.x];
        } else if (k % 256 == 0) {
            // A fixed tree: each wave sums 256 values of one row with
            // shuffles, one thread adds a row's wave sums in order. Every
            // block gets the same bits.
            const int per_row = k / 256;
            for (int base = 0; base < m * per_row; base += THREADS / WAVE) {
                const int chunk = base + (int)(threadIdx.x / WAVE);
                float part = 0.0f;
                if (chunk < m * per_row) {
                    const int row = chunk / per_row, c = chunk - row * per_row;
                    const float4 v = *(const float4*)(a.x + (size_t)row * k + c * 256 + (threadIdx.x % WAVE) * 4);
                    part = (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
                }
#pragma unroll
                for (int off = WAVE / 2; off > 0; off >>= 1) part += __shfl_xor(part, off);
                if (threadIdx.x % WAVE == 0 && chunk < m * per_row) sm.red[chunk] = part;
            }
            __syncthreads();
            if (threadIdx.x < m) {
                float sum = 0.0f;
                for (int c = 0; c < per_row; ++c) sum += sm.red[threadIdx.x * per_row + c];
                sm.inv[threadIdx.x] = 1.0f / __builtin_sqrtf(sum / (float)k + a.eps);
            }
        } else {
            // A fixed tree over the block: every block gets the same bits.
            for (int f = 0; f < m; ++f) {
                const float* row = a.x + (size_t)f * k;
                float part = 0.0f;
                for (int i = threadIdx.x; i < k; i += THREADS) {
                    float v = row[i];
                    part += v * v;
                }
                sm.red[threadIdx.x] = part;
                __syncthreads();
                for (int s = THREADS / 2; s > 0; s >>= 1) {
                    if (threadIdx.x < s) sm.red[threadIdx.x] += sm.red[threadIdx.x + s];
                    __syncthreads();
                }
                if (threadIdx.x == 0) sm.inv[f] = 1.0f / __builtin_sqrtf(sm.red[0] / (float)k + a.eps);
                __syncthreads();
            }
        }
        __syncthreads();
    }
    const int total = m * groups * TPG;
    for (int base = 0; base < total; base += THREADS) {
        const int i = base + (int)threadIdx.x;
        const bool live = i < total;
        const int item = live ? i : 0;
        const int row = item / (groups * TPG);
        const int rem = item - row * groups * TPG;
        const int g = rem / TPG, part = rem - g * TPG;
        const int col = g * W::G + part * 4;
        float4 v = *(const float4*)(a.x + (size_t)row * k + col);
        if (a.norm_w) {
            const float inv = sm.inv[row];
            const float4 w = *(const float4*)(a.norm_w + col);
            v.x = v.x * (inv * w.x);
            v.y = v.y * (inv * w.y);
            v.z = v.z * (inv * w.z);
            v.w = v.w * (inv * w.w);
        }
        float peak = __builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(v.x), __builtin_fabsf(v.y)),
                                     __builtin_fmaxf(__builtin_fabsf(v.z), __builtin_fabsf(v.w)));
#pragma unroll
        for (int off = TPG / 2; off > 0; off >>= 1) peak = __builtin_fmaxf(peak, __shfl_xor(peak, off));
        const float scale = peak > 0.0f ? peak / 127.0f : 1.0f;
        const float inv = 1.0f / scale;
        const int c0 = act_code(v.x * inv), c1 = act_code(v.y * inv);
        const int c2 = act_code(v.z * inv), c3 = act_code(v.w * inv);
        int sum = c0 + c1 + c2 + c3;
        if (W::TERN) {
#pragma unroll
            for (int off = TPG / 2; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
        }
        if (live) {
            *(uint32_t*)(sm.xq + (size_t)row * k + col) = pack4(c0, c1, c2, c3);
            if (part == 0) {
                sm.xs[row * ((groups + 4) & ~3) + g] = W::HALF ? f16_round(scale) : scale;
                if (W::TERN) sm.xsum[row * ((groups + 4) & ~3) + g] = sum;
            }
        }
    }
}

constexpr int XI = 4;  // float4 activation items a thread holds in the one-trip prologue

// The one-trip prologue: the activation rows (and RMSNorm weights) were
// loaded into registers with the weights, so this only computes. Requires
// m*k/4 <= XI*THREADS, and k % 256 == 0 when the norm sum is made here.
template <class W>
__device__ void quantize_regs(const GemvArgs& a, int k, const Smem& sm, const float4* xv, const float4* nv,
                              float inv_in) {
    constexpr int TPG = W::G / 4;
    const int groups = k / W::G;
    const int gsx = (groups + 4) & ~3;
    const int m = a.m;
    const int items = m * k / 4;
    const int ipr = k / 4;  // items per row
    if (a.norm_w) {
        if (a.norm_inv) {
            if (threadIdx.x < m) sm.inv[threadIdx.x] = inv_in;
        } else {
            // Each wave's 64 items are 256 values of one row: shuffle sums,
            // then one thread adds a row's wave sums in order.
#pragma unroll
            for (int i = 0; i < XI; ++i) {
                const int item = (int)threadIdx.x + i * THREADS;
                float part = 0.0f;
                if (item < items) {
                    const float4 v = xv[i];
                    part = (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
                }
#pragma unroll
                for (int off = WAVE / 2; off > 0; off >>= 1) part += __shfl_xor(part, off);
                if (threadIdx.x % WAVE == 0 && item < items) sm.red[item / WAVE] = part;
            }
            __syncthreads();
            if (threadIdx.x < m) {
                const int per_row = ipr / WAVE;
                float sum = 0.0f;
                for (int c = 0; c < per_row; ++c) sum += sm.red[threadIdx.x * per_row + c];
                sm.inv[threadIdx.x] = 1.0f / __builtin_sqrtf(sum / (float)k + a.eps);
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < XI; ++i) {
        const int base = i * THREADS;
        if (base >= items) break;  // uniform
        const int item = base + (int)threadIdx.x;
        const bool live = item < items;
        const int row = live ? item / ipr : 0;
        const int col = (live ? item - row * ipr : 0) * 4;
        float4 v = xv[i];
        if (a.norm_w) {
            const float inv = sm.inv[row];
            const float4 w = nv[i];
            v.x = v.x * (inv * w.x);
            v.y = v.y * (inv * w.y);
            v.z = v.z * (inv * w.z);
            v.w = v.w * (inv * w.w);
        }
        float peak = __builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(v.x), __builtin_fabsf(v.y)),
                                     __builtin_fmaxf(__builtin_fabsf(v.z), __builtin_fabsf(v.w)));
#pragma unroll
        for (int off = TPG / 2; off > 0; off >>= 1) peak = __builtin_fmaxf(peak, __shfl_xor(peak, off));
        const float scale = peak > 0.0f ? peak / 127.0f : 1.0f;
        const float inv = 1.0f / scale;
        const int c0 = act_code(v.x * inv), c1 = act_code(v.y * inv);
        const int c2 = act_code(v.z * inv), c3 = act_code(v.w * inv);
        int sum = c0 + c1 + c2 + c3;
        if (W::TERN) {
#pragma unroll
            for (int off = TPG / 2; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
        }
        if (live) {
            *(uint32_t*)(sm.xq + (size_t)row * k + col) = pack4(c0, c1, c2, c3);
            const int g = col / W::G;
            if (col % W::G == 0) {
                sm.xs[row * gsx + g] = W::HALF ? f16_round(scale) : scale;
                if (W::TERN) sm.xsum[row * gsx + g] = sum;
            }
        }
    }
}

template <class W>
__device__ __forceinline__ int chunk_dot(const uint4& w, const int8_t* xq, int kc) {
    if constexpr (W::TERN) {
        // 64 codes: word j holds 16 codes; (word >> 2s) & 0x03030303 are the
        // codes of inputs 16j + 4s .. 16j + 4s + 3.
        const uint4* xp = (const uint4*)(xq + (size_t)kc * 64);
        int d = 0;
        const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint4 xv = xp[j];
            const uint32_t xs[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
            for (int s = 0; s < 4; ++s) d = sdot4((words[j] >> (2 * s)) & 0x03030303u, xs[s], d);
        }
        return d;
    } else {
        const uint4 xv = *(const uint4*)(xq + (size_t)kc * 16);
        int d = sdot4(w.x, xv.x, 0);
        d = sdot4(w.y, xv.y, d);
        d = sdot4(w.z, xv.z, d);
        d = sdot4(w.w, xv.w, d);
        return d;
    }
}

// Row stride (ints) of a (row, frame) pair's group dots in LDS: 16-byte rows.
__host__ __device__ __forceinline__ int dot_stride(int groups) { return (groups + 4) & ~3; }

template <class W, int R, int P>
__global__ __launch_bounds__(THREADS) void gemv_kernel(const uint8_t* __restrict__ codes,
                                                        const void* __restrict__ scales,
                                                        const float* __restrict__ bias, int n, int k,
                                                        GemvArgs a) {
    extern __shared__ __align__(16) char smem_raw[];
    if (a.skip && *a.skip) return;
    const int m = a.m;
    const int groups = k / W::G;
    const int gs = dot_stride(groups);
    constexpr int rows_tile = P * R;
    const int part_rows = n / P;  // rows of one part (the SwiGLU pair's half)
    const int cpr = k / W::KPC;   // chunks per row
    const size_t row_bytes = (size_t)k / W::ROW_DIV;
    const int tiles = part_rows / R;
    int tile = blockIdx.x;
    if (tile >= tiles) return;

    Smem sm;
    {
        char* p = smem_raw;
        sm.xq = (int8_t*)p;
        p += align16((size_t)m * k);
        sm.xs = (float*)p;
        p += align16((size_t)m * gs * 4);
        sm.xsum = (int*)p;
        p += align16((size_t)m * gs * 4);
        sm.inv = (float*)p;
        p += align16((size_t)MAXF * 4);
        sm.red = (float*)p;
        p += align16((size_t)THREADS * 4);
        sm.dots = (int*)p;
        p += align16((size_t)rows_tile * m * gs * 4);
        sm.ws = (float*)p;
        p += align16((size_t)rows_tile * gs * 4);
        sm.res = (float*)p;
    }

    const int total = rows_tile * cpr;
    uint4 w[BATCH];
    auto load_batch = [&](int t, int base) {
        const int row0 = t * R;
#pragma unroll
        for (int u = 0; u < BATCH; ++u) {
            const int c = base + u * THREADS + (int)threadIdx.x;
            if (c < total) {
                const int pr = c / cpr, kc = c - pr * cpr;
                const int row = (pr / R) * part_rows + row0 + pr % R;
                w[u] = load_stream(codes + (size_t)row * row_bytes + (size_t)kc * 16);
            } else {
                w[u] = make_uint4(0, 0, 0, 0);
            }
        }
    };
    auto stage_scales = [&](int t) {
        const int row0 = t * R;
        for (int i = threadIdx.x; i < rows_tile * groups; i += THREADS) {
            const int pr = i / groups, g = i - pr * groups;
            const int row = (pr / R) * part_rows + row0 + pr % R;
            sm.ws[pr * gs + g] = W::scale(scales, (size_t)row * groups + g);
        }
    };

    // One memory round trip: the first weights, the activations, the norm
    // weights and the tile's scales are all in flight before any is used.
    load_batch(tile, 0);
    const int items = m * k / 4;
    const bool one_trip = items <= XI * THREADS && (!a.norm_w || a.norm_inv || k % 256 == 0) &&
                          rows_tile * groups <= XI * THREADS;
    if (one_trip) {
        float4 xv[XI], nv[XI];
        float sv[XI];
#pragma unroll
        for (int i = 0; i < XI; ++i) {
            const int item = (int)threadIdx.x + i * THREADS;
            xv[i] = item < items ? *(const float4*)(a.x + (size_t)item * 4) : make_float4(0, 0, 0, 0);
            nv[i] = (a.norm_w && item < items) ? *(const float4*)(a.norm_w + (item * 4) % k)
                                                : make_float4(0, 0, 0, 0);
            const int si = (int)threadIdx.x + i * THREADS;
            if (si < rows_tile * groups) {
                const int pr = si / groups, g = si - pr * groups;
                const int row = (pr / R) * part_rows + tile * R + pr % R;
                sv[i] = W::scale(scales, (size_t)row * groups + g);
            }
        }
        const float inv_in = (a.norm_w && a.norm_inv && (int)threadIdx.x < m) ? a.norm_inv[threadIdx.x] : 0.0f;
#pragma unroll
        for (int i = 0; i < XI; ++i) {
            const int si = (int)threadIdx.x + i * THREADS;
            if (si < rows_tile * groups) {
                const int pr = si / groups, g = si - pr * groups;
                sm.ws[pr * gs + g] = sv[i];
            }
        }
        quantize_regs<W>(a, k, sm, xv, nv, inv_in);
    } else {
        stage_scales(tile);
        quantize_rows<W>(a, k, sm);
    }
    __syncthreads();

    for (;;) {
        const int row0 = tile * R;
        for (int base = 0; base < total; base += THREADS * BATCH) {
            if (base > 0) load_batch(tile, base);
#pragma unroll
            for (int u = 0; u < BATCH; ++u) {
                const int c0 = base + u * THREADS;
                if (c0 >= total) break;  // uniform across the block
                const int c = c0 + (int)threadIdx.x;
                const bool live = c < total;
                const int cc = live ? c : 0;
                const int pr = cc / cpr, kc = cc - pr * cpr;
                const int g = kc / W::LPG;
                for (int f = 0; f < m; ++f) {
                    int d = chunk_dot<W>(w[u], sm.xq + (size_t)f * k, kc);
#pragma unroll
                    for (int off = 1; off < W::LPG; off <<= 1) d += __shfl_xor(d, off);
                    if (live && (kc % W::LPG) == 0) sm.dots[(pr * m + f) * gs + g] = d;
                }
            }
        }
        const int next = tile + gridDim.x;
        __syncthreads();
        // The next tile's weights stream in while this one's chains run.
        if (next < tiles) load_batch(next, 0);
        // The f32 chain, one thread per (row, frame), four groups per step.
        for (int t = threadIdx.x; t < rows_tile * m; t += THREADS) {
            const int pr = t / m, f = t - pr * m;
            const int* dots = sm.dots + (pr * m + f) * gs;
            const float* ws = sm.ws + pr * gs;
            const float* xs = sm.xs + f * gs;
            const int* xsum = sm.xsum + f * gs;
            float acc = 0.0f;
            int g = 0;
            for (; g + 4 <= groups; g += 4) {
                int4 d = *(const int4*)(dots + g);
                const float4 wv = *(const float4*)(ws + g);
                const float4 xv = *(const float4*)(xs + g);
                if (W::TERN) {
                    const int4 sv = *(const int4*)(xsum + g);
                    d.x -= sv.x;
                    d.y -= sv.y;
                    d.z -= sv.z;
                    d.w -= sv.w;
                }
                acc = __builtin_fmaf((float)d.x, wv.x * xv.x, acc);
                acc = __builtin_fmaf((float)d.y, wv.y * xv.y, acc);
                acc = __builtin_fmaf((float)d.z, wv.z * xv.z, acc);
                acc = __builtin_fmaf((float)d.w, wv.w * xv.w, acc);
            }
            for (; g < groups; ++g) {
                int d = dots[g];
                if (W::TERN) d -= xsum[g];
                acc = __builtin_fmaf((float)d, ws[g] * xs[g], acc);
            }
            const int row = (pr / R) * part_rows + row0 + pr % R;
            if (bias) acc = acc + bias[row];
            if (a.relu) acc = __builtin_fmaxf(acc, 0.0f);
            if (P == 2) {
                sm.res[t] = acc;
            } else if (a.epilogue == EPI_RESIDUAL) {
                a.y[(size_t)f * n + row] = a.residual[(size_t)f * n + row] + acc;
            } else {
                a.y[(size_t)f * n + row] = acc;
            }
        }
        if (P == 2) {
            __syncthreads();
            // SwiGLU: h = silu(gate) * up (src/models/parts/causal_lm.rs:464-473).
            for (int t = threadIdx.x; t < R * m; t += THREADS) {
                const int r = t / m, f = t - r * m;
                const float gate = sm.res[r * m + f];
                const float up = sm.res[(R + r) * m + f];
                a.y[(size_t)f * part_rows + row0 + r] = silu_trit(gate) * up;
            }
        }
        if (next >= tiles) break;
        __syncthreads();
        tile = next;
        stage_scales(tile);
        __syncthreads();
    }
}

size_t smem_bytes(int m, int k, int G, int rows_tile) {
    const int groups = k / G;
    const int gs = dot_stride(groups);
    auto al = [](size_t v) { return (v + 15) & ~(size_t)15; };
    return al((size_t)m * k) + 2 * al((size_t)m * gs * 4) + al((size_t)MAXF * 4) + al((size_t)THREADS * 4) +
           al((size_t)rows_tile * m * gs * 4) + al((size_t)rows_tile * gs * 4) + al((size_t)rows_tile * m * 4);
}

template <class W, int R, int P>
void launch(const Layer& L, const GemvArgs& a, hipStream_t s) {
    const int tiles = L.n / P / R;
    const size_t lds = smem_bytes(a.m, L.k, W::G, P * R);
    const int grid = tiles < 2048 ? tiles : 2048;
    launch_timed(a, gemv_kernel<W, R, P>, dim3(grid), dim3(THREADS), lds, s, L.codes.as<uint8_t>(),
                 (const void*)L.scales.ptr, L.bias.as<float>(), L.n, L.k, a);
    TRIT_HIP(hipGetLastError());
}

// The largest tile that leaves at least 512 tiles (a full chip at two per
// CU), down to 4 rows, within 64 KB of LDS.
template <class W, int P>
void dispatch_rows(const Layer& L, const GemvArgs& a, hipStream_t s) {
    const int rows = L.n / P;
    auto fits = [&](int R) {
        return rows % R == 0 && smem_bytes(a.m, L.k, W::G, P * R) <= 64 * 1024;
    };
    if (rows / 32 >= 512 && fits(32)) return launch<W, 32, P>(L, a, s);
    if (rows / 16 >= 512 && fits(16)) return launch<W, 16, P>(L, a, s);
    if (rows / 8 >= 512 && fits(8)) return launch<W, 8, P>(L, a, s);
    if (fits(4)) return launch<W, 4, P>(L, a, s);
    if (fits(2)) return launch<W, 2, P>(L, a, s);
    if (fits(1)) return launch<W, 1, P>(L, a, s);
    fail("gemv: layer " + std::to_string(L.n) + "x" + std::to_string(L.k) + " with " + std::to_string(a.m) +
         " rows does not fit the kernel's shared memory");
}

template <class W>
void dispatch(const Layer& L, const GemvArgs& a, hipStream_t s) {
    if (a.epilogue == EPI_SILU_PAIR) return dispatch_rows<W, 2>(L, a, s);
    return dispatch_rows<W, 1>(L, a, s);
}

}  // namespace

void gemv_int(const Layer& L, const GemvArgs& a, hipStream_t s) {
    if (a.m < 1 || a.m > MAXF) fail("gemv: 1 to 8 rows per call");
    if (gemv_row(L, a, s)) return;
    if (a.epilogue == EPI_SILU_PAIR && (L.n % 2 != 0)) fail("gemv: the SwiGLU pair needs an even row count");
    switch (L.kind) {
        case Q8_0:
        case Q4_K:
            return dispatch<Q8>(L, a, s);
        case INT8:
            return dispatch<I8>(L, a, s);
        case TERNARY:
            return dispatch<T2>(L, a, s);
        default:
            fail("gemv: not an integer layer");
    }
}

}  // namespace trit
