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

#include <algorithm>
#include <type_traits>
#include <map>
#include <mutex>

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
    static constexpr int G = 128, KPC = 16, LPG = 8, ROW_DIV = 1;  // LPG: 2 or 8
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


// Maximum and sum over the TPG consecutive lanes of a quantizer group
// (TPG = 8 or 32): DPP inside rows of 16 lanes, one cross-row shuffle for
// 32. Order-free (max, integer sums), so any lane order gives Trit's values.
template <int TPG>
__device__ __forceinline__ float group_max(float v) {
    v = __builtin_fmaxf(v, dpp<DPP_XOR1>(v));
    v = __builtin_fmaxf(v, dpp<DPP_XOR2>(v));
    v = __builtin_fmaxf(v, dpp<DPP_HALF_MIRROR>(v));
    if (TPG >= 16) v = __builtin_fmaxf(v, dpp<DPP_MIRROR>(v));
    if (TPG >= 32) v = __builtin_fmaxf(v, __shfl_xor(v, 16));
    return v;
}
template <int TPG>
__device__ __forceinline__ int group_sum(int v) {
    v += dpp<DPP_XOR1>(v);
    v += dpp<DPP_XOR2>(v);
    v += dpp<DPP_HALF_MIRROR>(v);
    if (TPG >= 16) v += dpp<DPP_MIRROR>(v);
    if (TPG >= 32) v += __shfl_xor(v, 16);
    return v;
}

constexpr int QB = 8;  // float4 items a thread has in flight in the prologue

// Where a row's activation code `col` sits in LDS (k codes a row). Ternary
// products read 64 codes a lane (one 16-byte weight chunk): their codes are
// stored as four planes of 16-byte pieces, piece j of chunk c at
// (j k / 64 + c) 16, so the lanes of a wave, holding consecutive chunks,
// read consecutive 16-byte pieces. Other kinds keep the row order.
template <class W>
__device__ __forceinline__ int code_pos(int col, int k) {
    if constexpr (W::TERN) return ((col >> 4) & 3) * (k >> 2) + (col >> 6) * 16 + (col & 15);
    return col;
}

// Trit's quantizer on one float4 item (values col .. col + 3 of a row): the
// group's TPG lanes (consecutive, aligned) find the peak together; the
// codes go to xq (at code_pos), and the group's first lane stores its scale
// (f16 rounded for Q8_0) and code sum at xs[col / G], xsum[col / G]. Every
// lane of the wave calls it (the DPP steps read neighbours); `live` lanes
// store.
template <class W>
__device__ __forceinline__ void quantize_item(float4 v, bool live, int col, int k, int8_t* xq, float* xs,
                                              int* xsum) {
    constexpr int TPG = W::G / 4;
    float peak = __builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(v.x), __builtin_fabsf(v.y)),
                                 __builtin_fmaxf(__builtin_fabsf(v.z), __builtin_fabsf(v.w)));
    peak = group_max<TPG>(peak);
    const float scale = peak > 0.0f ? peak / 127.0f : 1.0f;
    const float qi = 1.0f / scale;
    const int c0 = act_code(v.x * qi), c1 = act_code(v.y * qi);
    const int c2 = act_code(v.z * qi), c3 = act_code(v.w * qi);
    int sum = c0 + c1 + c2 + c3;
    if (W::TERN) sum = group_sum<TPG>(sum);
    if (live) {
        *(uint32_t*)(xq + code_pos<W>(col, k)) = pack4(c0, c1, c2, c3);
        if (col % W::G == 0) {
            xs[col / W::G] = W::HALF ? f16_round(scale) : scale;
            if (W::TERN) xsum[col / W::G] = sum;
        }
    }
}

// Quantizes the m rows of x into LDS with Trit's rule, optionally after
// RMSNorm: x * (inv * w). Loads go out QB at a time, so a thread waits
// for the caches once per batch rather than once per item.
template <class W>
__device__ void quantize_rows(const GemvArgs& a, int k, const Smem& sm) {
    constexpr int TPG = W::G / 4;
    static_assert(TPG == 8 || TPG == 32, "group lanes");
    const int groups = k / W::G;
    const int m = a.m;
    if (a.norm_w) {
        if (a.norm_inv) {
            if (threadIdx.x < m) sm.inv[threadIdx.x] = a.norm_inv[threadIdx.x];
        } else if (k % 256 == 0) {
            // A fixed tree: each wave sums 256 values of one row with
            // shuffles, one thread adds a row's wave sums in order. Every
            // block gets the same bits.
            const int per_row = k / 256, chunks = m * per_row, nw = THREADS / WAVE;
            const int lane = threadIdx.x % WAVE;
            for (int base = (int)(threadIdx.x / WAVE); base < chunks; base += nw * QB) {
                float4 v[QB];
#pragma unroll
                for (int q = 0; q < QB; ++q) {
                    const int chunk = base + q * nw;
                    v[q] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                    if (chunk < chunks) {
                        const int row = chunk / per_row, c = chunk - row * per_row;
                        v[q] = *(const float4*)(a.x + (size_t)row * k + c * 256 + lane * 4);
                    }
                }
#pragma unroll
                for (int q = 0; q < QB; ++q) {
                    const int chunk = base + q * nw;
                    if (chunk >= chunks) break;  // uniform per wave
                    float part = (v[q].x * v[q].x + v[q].y * v[q].y) + (v[q].z * v[q].z + v[q].w * v[q].w);
#pragma unroll
                    for (int off = WAVE / 2; off > 0; off >>= 1) part += __shfl_xor(part, off);
                    if (lane == 0) sm.red[chunk] = part;
                }
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
    // Items are float4s in row-major order; a group's TPG items are TPG
    // consecutive lanes (whole waves: k % 256 == 0 is not needed, since
    // TPG divides 64 and a row's items divide into whole groups).
    const int total = m * groups * TPG;
    const int ipr = k / 4;  // items per row
    for (int base = 0; base < total; base += THREADS * QB) {
        float4 v[QB], nv[QB];
#pragma unroll
        for (int q = 0; q < QB; ++q) {
            const int i = base + q * THREADS + (int)threadIdx.x;
            v[q] = nv[q] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (i < total) {
                v[q] = *(const float4*)(a.x + (size_t)i * 4);
                if (a.norm_w) nv[q] = *(const float4*)(a.norm_w + (size_t)(i % ipr) * 4);
            }
        }
#pragma unroll
        for (int q = 0; q < QB; ++q) {
            const int i0 = base + q * THREADS;
            if (i0 >= total) break;  // uniform across the block
            const int i = i0 + (int)threadIdx.x;
            const bool live = i < total;
            const int row = live ? i / ipr : 0;
            const int col = (live ? i - row * ipr : 0) * 4;
            float4 x = v[q];
            if (a.norm_w) {
                const float inv = sm.inv[row];
                x.x = x.x * (inv * nv[q].x);
                x.y = x.y * (inv * nv[q].y);
                x.z = x.z * (inv * nv[q].z);
                x.w = x.w * (inv * nv[q].w);
            }
            const int gsx = (groups + 4) & ~3;
            quantize_item<W>(x, live, col, k, sm.xq + (size_t)row * k, sm.xs + row * gsx, sm.xsum + row * gsx);
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
        quantize_item<W>(v, live, col, k, sm.xq + (size_t)row * k, sm.xs + row * gsx, sm.xsum + row * gsx);
    }
}

// A 16-byte weight chunk ready for its dots: ternary chunks unpacked once
// into 16 words of four codes (word 4j + s holds the codes of inputs
// 16j + 4s .. +3: (word j >> 2s) & 0x03030303 of the stored chunk), other
// kinds as stored.
template <class W>
struct Chunk {
    uint32_t v[W::TERN ? 16 : 4];
};

template <class W>
__device__ __forceinline__ Chunk<W> chunk_codes(const uint4& w) {
    Chunk<W> c;
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
    if constexpr (W::TERN) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int s = 0; s < 4; ++s) c.v[4 * j + s] = (words[j] >> (2 * s)) & 0x03030303u;
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) c.v[j] = words[j];
    }
    return c;
}

// The exact i32 dot of chunk kc with one row of activation codes (xq, k
// codes, laid out by code_pos).
template <class W>
__device__ __forceinline__ int chunk_dot(const Chunk<W>& c, const int8_t* xq, int kc, int k) {
    int d = 0;
    if constexpr (W::TERN) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint4 xv = *(const uint4*)(xq + (size_t)j * (k >> 2) + (size_t)kc * 16);
            d = sdot4(c.v[4 * j], xv.x, d);
            d = sdot4(c.v[4 * j + 1], xv.y, d);
            d = sdot4(c.v[4 * j + 2], xv.z, d);
            d = sdot4(c.v[4 * j + 3], xv.w, d);
        }
    } else {
        const uint4 xv = *(const uint4*)(xq + (size_t)kc * 16);
        d = sdot4(c.v[0], xv.x, d);
        d = sdot4(c.v[1], xv.y, d);
        d = sdot4(c.v[2], xv.z, d);
        d = sdot4(c.v[3], xv.w, d);
    }
    return d;
}



// RMSNorm factor of one row by the whole block, with the sum trees of
// quantize_rows (so both paths give a row the same bits); every thread
// returns it.
__device__ float row_inv_block(const float* x, int k, float eps, float* red) {
    float sum = 0.0f;
    if (k % 256 == 0) {
        const int per_row = k / 256, nw = THREADS / WAVE, lane = threadIdx.x % WAVE;
        for (int base = (int)(threadIdx.x / WAVE); base < per_row; base += nw * QB) {
            float4 v[QB];
#pragma unroll
            for (int q = 0; q < QB; ++q)
                v[q] = base + q * nw < per_row ? *(const float4*)(x + (size_t)(base + q * nw) * 256 + lane * 4)
                                               : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
            for (int q = 0; q < QB; ++q) {
                if (base + q * nw >= per_row) break;  // uniform per wave
                float part = (v[q].x * v[q].x + v[q].y * v[q].y) + (v[q].z * v[q].z + v[q].w * v[q].w);
#pragma unroll
                for (int off = WAVE / 2; off > 0; off >>= 1) part += __shfl_xor(part, off);
                if (lane == 0) red[base + q * nw] = part;
            }
        }
        __syncthreads();
        for (int c = 0; c < per_row; ++c) sum += red[c];
    } else {
        float part = 0.0f;
        for (int i = threadIdx.x; i < k; i += THREADS) {
            const float v = x[i];
            part += v * v;
        }
        red[threadIdx.x] = part;
        __syncthreads();
        for (int st = THREADS / 2; st > 0; st >>= 1) {
            if ((int)threadIdx.x < st) red[threadIdx.x] += red[threadIdx.x + st];
            __syncthreads();
        }
        sum = red[0];
    }
    return 1.0f / __builtin_sqrtf(sum / (float)k + eps);
}

constexpr int PRE_ITEMS = 2;  // float4 items a thread quantizes in the quantization pass

// The quantization pass for 2..8 rows: Trit's quantizer (after RMSNorm when
// the product has one) runs once per call instead of once per product
// block. Block (row, slice) writes items [slice THREADS PRE_ITEMS, ...) of
// the row into the image (pre_bytes) the product kernel copies into LDS.
template <class W>
__global__ __launch_bounds__(THREADS) void prequant_kernel(GemvArgs a, int k, uint8_t* __restrict__ img) {
    __shared__ float red[THREADS];
    if (a.skip && *a.skip) return;
    const int m = a.m, row = blockIdx.x, gs = dot_stride(k / W::G);
    int8_t* xq = (int8_t*)img + (size_t)row * k;
    float* xs = (float*)(img + align16((size_t)m * k)) + (size_t)row * gs;
    int* xsum = (int*)(img + align16((size_t)m * k) + align16((size_t)m * gs * 4)) + (size_t)row * gs;
    const float* x = a.x + (size_t)row * k;
    const int ipr = k / 4, base = blockIdx.y * THREADS * PRE_ITEMS;
    float4 v[PRE_ITEMS], nv[PRE_ITEMS];
#pragma unroll
    for (int q = 0; q < PRE_ITEMS; ++q) {
        const int i = base + q * THREADS + (int)threadIdx.x;
        v[q] = nv[q] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (i < ipr) {
            v[q] = *(const float4*)(x + (size_t)i * 4);
            if (a.norm_w) nv[q] = *(const float4*)(a.norm_w + (size_t)i * 4);
        }
    }
    float inv = 1.0f;
    if (a.norm_w) inv = a.norm_inv ? a.norm_inv[row] : row_inv_block(x, k, a.eps, red);
#pragma unroll
    for (int q = 0; q < PRE_ITEMS; ++q) {
        if (base + q * THREADS >= ipr) break;  // uniform across the block
        const int i = base + q * THREADS + (int)threadIdx.x;
        float4 xv = v[q];
        if (a.norm_w) {
            xv.x = xv.x * (inv * nv[q].x);
            xv.y = xv.y * (inv * nv[q].y);
            xv.z = xv.z * (inv * nv[q].z);
            xv.w = xv.w * (inv * nv[q].w);
        }
        quantize_item<W>(xv, i < ipr, i * 4, k, xq, xs, xsum);
    }
}

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
    uint4 wn[BATCH];  // the next batch, in flight while this one computes
    auto load_into = [&](uint4 (&dst)[BATCH], int t, int base) {
        const int row0 = t * R;
#pragma unroll
        for (int u = 0; u < BATCH; ++u) {
            const int c = base + u * THREADS + (int)threadIdx.x;
            if (c < total) {
                const int pr = c / cpr, kc = c - pr * cpr;
                const int row = (pr / R) * part_rows + row0 + pr % R;
                dst[u] = load_stream(codes + (size_t)row * row_bytes + (size_t)kc * 16);
            } else {
                dst[u] = make_uint4(0, 0, 0, 0);
            }
        }
    };
    auto load_batch = [&](int t, int base) { load_into(w, t, base); };
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
    const bool one_trip = !a.pre && items <= XI * THREADS && (!a.norm_w || a.norm_inv || k % 256 == 0) &&
                          rows_tile * groups <= XI * THREADS;
    if (a.pre) {
        // The rows were quantized by the quantization pass: one copy of
        // its image into the first bytes of LDS.
        // Up to IB pieces a thread are in flight at once (with the tile's
        // weight scales), so most images take one memory round trip.
        constexpr int IB = 12;
        const int n16 = (int)(pre_bytes(m, k, W::G) / 16);
        const uint4* src = (const uint4*)a.pre;
        uint4* dst = (uint4*)smem_raw;
        for (int base = 0; base < n16; base += THREADS * IB) {
            uint4 v[IB];
#pragma unroll
            for (int q = 0; q < IB; ++q) {
                const int i = base + q * THREADS + (int)threadIdx.x;
                v[q] = i < n16 ? src[i] : make_uint4(0, 0, 0, 0);
            }
            if (base == 0) stage_scales(tile);
#pragma unroll
            for (int q = 0; q < IB; ++q) {
                const int i = base + q * THREADS + (int)threadIdx.x;
                if (i < n16) dst[i] = v[q];
            }
        }
    } else if (one_trip) {
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
            const bool more = base + THREADS * BATCH < total;  // uniform
            if (more) load_into(wn, tile, base + THREADS * BATCH);
#pragma unroll
            for (int u = 0; u < BATCH; ++u) {
                const int c0 = base + u * THREADS;
                if (c0 >= total) break;  // uniform across the block
                const int c = c0 + (int)threadIdx.x;
                const bool live = c < total;
                const int cc = live ? c : 0;
                const int pr = cc / cpr, kc = cc - pr * cpr;
                const int g = kc / W::LPG;
                const Chunk<W> ch = chunk_codes<W>(w[u]);
                for (int f = 0; f < m; ++f) {
                    int d = chunk_dot<W>(ch, sm.xq + (size_t)f * k, kc, k);
                    // The group's LPG lanes (2 or 8, aligned) add their dots.
                    d += dpp<DPP_XOR1>(d);
                    if (W::LPG >= 4) d += dpp<DPP_XOR2>(d);
                    if (W::LPG >= 8) d += dpp<DPP_HALF_MIRROR>(d);
                    if (live && (kc % W::LPG) == 0) sm.dots[(pr * m + f) * gs + g] = d;
                }
            }
            if (more) {
#pragma unroll
                for (int u = 0; u < BATCH; ++u) w[u] = wn[u];
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
            // Unrolled so that later groups' loads issue ahead of the
            // dependent FMAs (the chain itself is serial).
#pragma unroll 4
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

// Blocks of `kernel` the device holds at once (cached per kernel and LDS
// size).
int resident_blocks(const void* kernel, int threads, size_t lds) {
    static std::mutex mu;
    static std::map<std::pair<const void*, size_t>, int> cache;
    std::lock_guard<std::mutex> lock(mu);
    const auto key = std::make_pair(kernel, lds);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    int per_cu = 0, dev = 0, cus = 0;
    TRIT_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, lds));
    TRIT_HIP(hipGetDevice(&dev));
    TRIT_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    const int n = std::max(1, per_cu) * std::max(1, cus);
    cache[key] = n;
    return n;
}

template <class W, int R, int P>
void launch(const Layer& L, const GemvArgs& a, hipStream_t s) {
    const int tiles = L.n / P / R;
    const size_t lds = smem_bytes(a.m, L.k, W::G, P * R);
    int grid = tiles < 2048 ? tiles : 2048;
    // With the rows quantized ahead, each block copies their image once:
    // no more blocks than are resident together, looping over the tiles.
    if (a.pre) grid = std::min(grid, resident_blocks((const void*)gemv_kernel<W, R, P>, THREADS, lds));
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
void dispatch(const Layer& L, const GemvArgs& a0, hipStream_t s) {
    GemvArgs a = a0;
    // Two or more rows: quantize once in a pass of its own when the caller
    // gave scratch for the image (a timed call then starts its interval at
    // that pass's start).
    if (a.m >= 2 && !a.pre && a.scratch && a.scratch_bytes >= pre_bytes(a.m, L.k, W::G)) {
        const dim3 grid(a.m, (L.k / 4 + THREADS * PRE_ITEMS - 1) / (THREADS * PRE_ITEMS));
        GemvArgs t = a;
        t.ev_stop = nullptr;  // the start event, if any, stamps this pass's start
        launch_timed(t, prequant_kernel<W>, grid, dim3(THREADS), 0, s, a, L.k, (uint8_t*)a.scratch);
        TRIT_HIP(hipGetLastError());
        a.pre = (const uint8_t*)a.scratch;
        a.ev_start = nullptr;
    }
    if ((std::is_same<W, Q8>::value || std::is_same<W, T2>::value) && gemv_stream(L, a, s)) return;
    if (a.epilogue == EPI_SILU_PAIR) return dispatch_rows<W, 2>(L, a, s);
    return dispatch_rows<W, 1>(L, a, s);
}

}  // namespace

size_t gemv_scratch_bytes(int m, int k) { return pre_bytes(m, k, 32) > pre_bytes(m, k, 128) ? pre_bytes(m, k, 32) : pre_bytes(m, k, 128); }

void gemv_int(const Layer& L, const GemvArgs& a, hipStream_t s) {
    if (a.m < 1 || a.m > MAXF) fail("gemv: 1 to 8 rows per call");
    if (gemv_stream(L, a, s)) return;  // rows quantized in the block
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
