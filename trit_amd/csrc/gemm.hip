// Integer products of many rows (prompt prefill) on the matrix cores:
// Q8_0 (and Q4_K requantized to it) with 32-value groups, Trit int8 with
// 128-value groups.
//
// The values are Trit's, bit for bit, as in the small-batch kernels
// (src/cpu/int8.rs:525-584, src/cpu/v2/product.rs:389-423):
//   y[f][r] = chain over groups g in order of
//             total = fma(f32(dot_g), ws[r][g] * xs[f][g], total), from +0,
// where dot_g is the exact i32 dot of the group's weight codes and the
// activation codes of Trit's quantizer (src/cpu/kernels.rs:661-807). The
// matrix cores make the i32 group dots (v_mfma_i32_32x32x32_i8: one 32-wide
// step is one Q8_0 group, four steps one int8 group); the f32 chain runs on
// the vector ALUs in group order, per output, in the MFMA's own register
// layout.
//
// Passes:
//  1. (RMSNorm rows) row_norm_kernel: each row's factor, with the same sum
//     tree as the small-batch kernel's prologue;
//  2. quantize_kernel: Trit's activation quantizer over all rows into codes
//     (m x k) and group scales stored group-major (g x mpad), so that a
//     lane's four consecutive output rows read one 16-byte load;
//  3. gemm_kernel: 256 threads = 2 x 2 waves; a wave owns 32 rows of x by
//     two 32-row MFMA tiles of weights (or, for the SwiGLU pair, the gate
//     tile and its up tile), so every (row, output) total stays in one
//     lane's registers from the first group to the epilogue.
#include "device.h"
#include "internal.h"

namespace trit {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int GEMM_THREADS = 256;
constexpr int BM = 64;  // rows of x per block: two waves of 32

int round_up(int v, int to) { return (v + to - 1) / to * to; }

// RMSNorm factor per row: each 256-value chunk's squares summed by a
// shuffle butterfly over one wave, the chunks added in order from lane 0 --
// the bits of the small-batch kernel's prologue (gemv.hip), so a prompt row
// gets the same factor on either path. One wave per row, k % 256 == 0.
__global__ __launch_bounds__(WAVE) void row_norm_kernel(const float* __restrict__ x, int k, float eps,
                                                         float* __restrict__ inv, const int* skip) {
    if (skip && *skip) return;
    const int row = blockIdx.x, lane = threadIdx.x;
    float sum = 0.0f;
    for (int c = 0; c < k / 256; ++c) {
        const float4 v = *(const float4*)(x + (size_t)row * k + c * 256 + lane * 4);
        float part = (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
#pragma unroll
        for (int off = WAVE / 2; off > 0; off >>= 1) part += __shfl_xor(part, off);
        sum += __shfl(part, 0);
    }
    if (lane == 0) inv[row] = 1.0f / __builtin_sqrtf(sum / (float)k + eps);
}

// Trit's activation quantizer (src/cpu/kernels.rs:661-737), G/4 threads per
// group, four values a thread; rows [m, mpad) get zero scales.
template <int G, bool HALF>
__global__ __launch_bounds__(256) void quantize_kernel(const float* __restrict__ x, int m, int mpad, int k,
                                                       const float* __restrict__ norm_w,
                                                       const float* __restrict__ inv, int8_t* __restrict__ xq,
                                                       float* __restrict__ xs, const int* skip) {
    if (skip && *skip) return;
    constexpr int TPG = G / 4;
    const int ipr = k / 4;  // items per row
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    const bool live = i < (size_t)mpad * ipr;
    const int row = live ? (int)(i / ipr) : 0;
    const int col = live ? (int)(i - (size_t)row * ipr) * 4 : 0;
    const bool real = live && row < m;
    float4 v = real ? *(const float4*)(x + (size_t)row * k + col) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (norm_w && real) {
        const float f = inv[row];
        const float4 w = *(const float4*)(norm_w + col);
        v.x = v.x * (f * w.x);
        v.y = v.y * (f * w.y);
        v.z = v.z * (f * w.z);
        v.w = v.w * (f * w.w);
    }
    float peak = __builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(v.x), __builtin_fabsf(v.y)),
                                 __builtin_fmaxf(__builtin_fabsf(v.z), __builtin_fabsf(v.w)));
#pragma unroll
    for (int off = TPG / 2; off > 0; off >>= 1) peak = __builtin_fmaxf(peak, __shfl_xor(peak, off));
    const float scale = peak > 0.0f ? peak / 127.0f : 1.0f;
    const float q = 1.0f / scale;
    const int c0 = act_code(v.x * q), c1 = act_code(v.y * q);
    const int c2 = act_code(v.z * q), c3 = act_code(v.w * q);
    if (real) *(uint32_t*)(xq + (size_t)row * k + col) = pack4(c0, c1, c2, c3);
    if (live && col % G == 0) xs[(size_t)(col / G) * mpad + row] = real ? (HALF ? f16_round(scale) : scale) : 0.0f;
}

template <bool HALF>
__device__ __forceinline__ float weight_scale(const void* s, size_t i) {
    if (HALF) return f16_to_f32(((const uint16_t*)s)[i]);
    return ((const float*)s)[i];
}

// One group's operands: per 32-wide step, the x tile's 16 bytes and the
// two weight tiles'; the x scales of the lane's 16 output rows and the two
// weight rows' scales.
template <int CH>
struct Operands {
    v4i a[CH], b0[CH], b1[CH];
    float4 xv[4];
    float w0, w1;
};

template <int G, bool HALF, int P>
__global__ __launch_bounds__(GEMM_THREADS) void gemm_kernel(const int8_t* __restrict__ xq,
                                                            const float* __restrict__ xs, int m, int mpad,
                                                            const int8_t* __restrict__ codes,
                                                            const void* __restrict__ scales,
                                                            const float* __restrict__ bias, int n, int k, int nb,
                                                            int mb, GemvArgs a) {
    constexpr int CH = G / 32;  // MFMA steps per group
    if (a.skip && *a.skip) return;
    const int groups = k / G;
    // Tiles in XCD order: block b runs on XCD b % 8; the blocks of one XCD
    // share weight tiles, which then stay in that XCD's L2.
    const int b = blockIdx.x;
    int bn, bm;
    if (nb % 8 == 0) {
        const int t = b / 8;
        bn = b % 8 + 8 * (t / mb);
        bm = t % mb;
    } else {
        bn = b % nb;
        bm = b / nb;
    }
    const int lane = threadIdx.x % WAVE, w = threadIdx.x / WAVE;
    const int lr = lane % 32, h = lane / 32;
    const int m0 = bm * BM + (w % 2) * 32;
    int r0, r1;  // first weight rows of the wave's two tiles
    if (P == 1) {
        r0 = bn * 128 + (w / 2) * 64;
        r1 = r0 + 32;
    } else {
        r0 = bn * 64 + (w / 2) * 32;
        r1 = n / 2 + r0;
    }
    const int arow = m0 + lr < m ? m0 + lr : m - 1;
    const int8_t* ap = xq + (size_t)arow * k + 16 * h;
    const int8_t* bp0 = codes + (size_t)(r0 + lr) * k + 16 * h;
    const int8_t* bp1 = codes + (size_t)(r1 + lr) * k + 16 * h;
    const float* xp = xs + m0 + 4 * h;
    const size_t s0 = (size_t)(r0 + lr) * groups, s1 = (size_t)(r1 + lr) * groups;

    float t0[16], t1[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) t0[r] = t1[r] = 0.0f;

    // Operands of group g: lane (lr, h) holds bytes [16h, 16h + 16) of each
    // 32-wide step in x row m0 + lr and in weight rows r0 + lr, r1 + lr.
    // Everything a group needs is loaded one group ahead, so the wait for a
    // group's loads never waits for the next group's.
    auto load = [&](int g, Operands<CH>& o) {
#pragma unroll
        for (int s = 0; s < CH; ++s) {
            const size_t off = (size_t)g * G + 32 * s;
            o.a[s] = *(const v4i*)(ap + off);
            o.b0[s] = *(const v4i*)(bp0 + off);
            o.b1[s] = *(const v4i*)(bp1 + off);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) o.xv[q] = *(const float4*)(xp + (size_t)g * mpad + 8 * q);
        o.w0 = weight_scale<HALF>(scales, s0 + g);
        o.w1 = weight_scale<HALF>(scales, s1 + g);
    };
    Operands<CH> cur, nxt;
    load(0, cur);
    for (int g = 0; g < groups; ++g) {
        if (g + 1 < groups) load(g + 1, nxt);
        v16i d0 = {}, d1 = {};
#pragma unroll
        for (int s = 0; s < CH; ++s) {
            d0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(cur.a[s], cur.b0[s], d0, 0, 0, 0);
            d1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(cur.a[s], cur.b1[s], d1, 0, 0, 0);
        }
        // Output (row 8*(r/4) + 4h + r%4, column lr) of a tile is register r.
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float4 x4 = cur.xv[r / 4];
            const float xsv = r % 4 == 0 ? x4.x : r % 4 == 1 ? x4.y : r % 4 == 2 ? x4.z : x4.w;
            t0[r] = __builtin_fmaf((float)d0[r], cur.w0 * xsv, t0[r]);
            t1[r] = __builtin_fmaf((float)d1[r], cur.w1 * xsv, t1[r]);
        }
        cur = nxt;
    }

    // Epilogue, as the small-batch kernel's: bias, relu, then the residual
    // add or the SwiGLU pair (src/models/parts/causal_lm.rs:464-473).
    const int ldy = n / P;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int row = m0 + 8 * (r / 4) + 4 * h + r % 4;
        if (row >= m) continue;
        float v0 = t0[r], v1 = t1[r];
        if (bias) {
            v0 = v0 + bias[r0 + lr];
            v1 = v1 + bias[r1 + lr];
        }
        if (a.relu) {
            v0 = __builtin_fmaxf(v0, 0.0f);
            v1 = __builtin_fmaxf(v1, 0.0f);
        }
        if (P == 2) {
            a.y[(size_t)row * ldy + r0 + lr] = silu_trit(v0) * v1;
        } else if (a.epilogue == EPI_RESIDUAL) {
            const size_t i0 = (size_t)row * ldy + r0 + lr, i1 = (size_t)row * ldy + r1 + lr;
            a.y[i0] = a.residual[i0] + v0;
            a.y[i1] = a.residual[i1] + v1;
        } else {
            a.y[(size_t)row * ldy + r0 + lr] = v0;
            a.y[(size_t)row * ldy + r1 + lr] = v1;
        }
    }
}

int group_of(const Layer& L) { return L.kind == INT8 ? 128 : 32; }

struct Scratch {
    int8_t* xq;
    float* xs;
    float* inv;
    int mpad;
};

Scratch carve(void* base, int m, int k) {
    const int mpad = round_up(m, BM);
    auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
    char* p = (char*)base;
    Scratch s;
    s.mpad = mpad;
    s.xq = (int8_t*)p;
    p += al((size_t)m * k);
    s.xs = (float*)p;
    p += al((size_t)(k / 32) * mpad * 4);
    s.inv = (float*)p;
    return s;
}

template <int G, bool HALF, int P>
void launch_gemm(const Layer& L, const GemvArgs& a, const Scratch& sc, hipStream_t s) {
    const int nb = P == 1 ? L.n / 128 : (L.n / 2) / 64;
    const int mb = sc.mpad / BM;
    launch_timed(a, gemm_kernel<G, HALF, P>, dim3(nb * mb), dim3(GEMM_THREADS), 0, s, (const int8_t*)sc.xq,
                 (const float*)sc.xs, a.m, sc.mpad, L.codes.as<int8_t>(), (const void*)L.scales.ptr,
                 L.bias.as<float>(), L.n, L.k, nb, mb, a);
    TRIT_HIP(hipGetLastError());
}

}  // namespace

bool gemm_supported(const Layer& L, const GemvArgs& a) {
    if (L.kind != Q8_0 && L.kind != Q4_K && L.kind != INT8) return false;
    if (L.n % 128 != 0 || L.k % group_of(L) != 0) return false;
    if (a.norm_w && !a.norm_inv && L.k % 256 != 0) return false;
    return a.m >= 1;
}

size_t gemm_scratch_bytes(int m, int k) {
    const size_t mpad = (size_t)round_up(m, BM);
    auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
    return al((size_t)m * k) + al((size_t)(k / 32) * mpad * 4) + al(mpad * 4);
}

void gemm_int(const Layer& L, const GemvArgs& a, void* scratch, hipStream_t s) {
    if (!gemm_supported(L, a)) fail("gemm: layer " + std::to_string(L.n) + "x" + std::to_string(L.k) +
                                    " is not a shape the matrix-core product takes");
    const Scratch sc = carve(scratch, a.m, L.k);
    const float* inv = a.norm_inv;
    if (a.norm_w && !inv) {
        hipLaunchKernelGGL(row_norm_kernel, dim3(a.m), dim3(WAVE), 0, s, a.x, L.k, a.eps, sc.inv, a.skip);
        TRIT_HIP(hipGetLastError());
        inv = sc.inv;
    }
    const int G = group_of(L);
    const size_t items = (size_t)sc.mpad * (L.k / 4);
    const int qblocks = (int)((items + 255) / 256);
    if (G == 32)
        hipLaunchKernelGGL((quantize_kernel<32, true>), dim3(qblocks), dim3(256), 0, s, a.x, a.m, sc.mpad, L.k,
                           a.norm_w, inv, sc.xq, sc.xs, a.skip);
    else
        hipLaunchKernelGGL((quantize_kernel<128, false>), dim3(qblocks), dim3(256), 0, s, a.x, a.m, sc.mpad, L.k,
                           a.norm_w, inv, sc.xq, sc.xs, a.skip);
    TRIT_HIP(hipGetLastError());
    const bool pair = a.epilogue == EPI_SILU_PAIR;
    if (G == 32) {
        if (pair) return launch_gemm<32, true, 2>(L, a, sc, s);
        return launch_gemm<32, true, 1>(L, a, sc, s);
    }
    if (pair) return launch_gemm<128, false, 2>(L, a, sc, s);
    return launch_gemm<128, false, 1>(L, a, sc, s);
}

}  // namespace trit
