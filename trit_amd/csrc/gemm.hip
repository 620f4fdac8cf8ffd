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
//  3. gemm_kernel: 256 threads = 2 x 2 waves over 64 rows of x and 128
//     weight rows. K runs in 256-byte chunks staged through LDS (the last
//     one zero past k when k % 256 != 0): 16 threads
//     read a row's 256 contiguous bytes, and the next chunk's loads are in
//     flight while this one computes. A wave owns 32 rows of x by two
//     32-row MFMA tiles of weights (or, for the SwiGLU pair, the gate tile
//     and its up tile), so every (row, output) total stays in one lane's
//     registers from the first group to the epilogue.
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

constexpr int KC = 256;           // bytes of K per LDS chunk
constexpr int ROW_LDS = KC + 16;  // padded LDS row: rows 8 apart start 4 banks apart
constexpr int BN_ROWS = 128;      // weight rows per block

// One K chunk in LDS: the block's 64 x rows and 128 weight rows, and their
// group scales (weight scales widened to f32).
template <int G>
struct alignas(16) Stage {
    static constexpr int GPC = KC / G;  // groups per chunk
    alignas(16) int8_t a[BM * ROW_LDS];
    alignas(16) int8_t b[BN_ROWS * ROW_LDS];
    alignas(16) float xs[GPC][BM];
    alignas(16) float ws[GPC][BN_ROWS];
};

// A group's operand fragments: lane (lr, h) holds bytes [16h, 16h + 16) of
// each 32-wide step of x row lr and weight rows lr of the two tiles.
template <int CH>
struct Frags {
    v4i a[CH], b0[CH], b1[CH];
};

template <int G>
__device__ __forceinline__ void read_frags(const int8_t* la, const int8_t* lb0, const int8_t* lb1, int gi,
                                           Frags<G / 32>& f) {
#pragma unroll
    for (int s = 0; s < G / 32; ++s) {
        const int off = gi * G + 32 * s;
        f.a[s] = *(const v4i*)(la + off);
        f.b0[s] = *(const v4i*)(lb0 + off);
        f.b1[s] = *(const v4i*)(lb1 + off);
    }
}

// The i32 dots of a group for the wave's two weight tiles.
template <int G>
__device__ __forceinline__ void mfma_group(const Frags<G / 32>& f, v16i& d0, v16i& d1) {
#pragma unroll
    for (int s = 0; s < G / 32; ++s) {
        d0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a[s], f.b0[s], d0, 0, 0, 0);
        d1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a[s], f.b1[s], d1, 0, 0, 0);
    }
}

// A group's scales for the lane: x scales of its 16 output rows (four
// runs of four), weight scales of its two columns.
struct Scales {
    float4 x[4];
    float w0, w1;
};

__device__ __forceinline__ void read_scales(const float* xs, const float* ws, int xrow, int c0, int c1, Scales& s) {
#pragma unroll
    for (int q = 0; q < 4; ++q) s.x[q] = *(const float4*)(xs + xrow + 8 * q);
    s.w0 = ws[c0];
    s.w1 = ws[c1];
}

template <int G, bool HALF, int P, bool TAIL>
__global__ __launch_bounds__(GEMM_THREADS, 2) void gemm_kernel(const int8_t* __restrict__ xq,
                                                               const float* __restrict__ xs, int m, int mpad,
                                                               const int8_t* __restrict__ codes,
                                                               const void* __restrict__ scales,
                                                               const float* __restrict__ bias, int n, int k,
                                                               int nb, int mb, GemvArgs a) {
    constexpr int GPC = KC / G;  // groups per chunk
    constexpr int CH = G / 32;   // MFMA steps per group
    __shared__ __align__(16) Stage<G> st;
    if (a.skip && *a.skip) return;
    // TAIL: k is not a multiple of KC; the last chunk holds k % KC bytes,
    // zero past them, and chains only its real groups.
    const int groups = k / G, chunks = (k + KC - 1) / KC;
    // Tiles in XCD order: block b runs on XCD b % 8; the blocks of one XCD
    // share weight tiles, which then stay in that XCD's L2.
    const int blk = blockIdx.x;
    int bn, bm;
    if (nb % 8 == 0) {
        const int q = blk / 8;
        bn = blk % 8 + 8 * (q / mb);
        bm = q % mb;
    } else {
        bn = blk % nb;
        bm = blk / nb;
    }
    const int t = threadIdx.x;
    const int lane = t % WAVE, w = t / WAVE;
    const int lr = lane % 32, h = lane / 32;
    const int mbase = bm * BM;
    // LDS weight row i holds weight row brow(i): 128 rows, or for the
    // SwiGLU pair 64 gate rows then their 64 up rows.
    // Rows past n (the last tile when n % 128 != 0) load row n - 1 and
    // store nothing.
    auto brow = [&](int i) {
        const int r = P == 1 ? bn * 128 + i : (i < 64 ? bn * 64 + i : n / 2 + bn * 64 + (i - 64));
        return r < n ? r : n - 1;
    };

    // Global loads of a chunk, 16 bytes a piece, 16 threads a row (256
    // contiguous bytes): 4 x pieces and 8 weight pieces per thread; threads
    // [0, 16*GPC) one float4 of x scales, threads [128, 256) one weight row's
    // GPC scales.
    // Byte offsets of the thread's pieces in row 0 of the chunk; rows are
    // k bytes apart (x: at most m*k < 2^31 bytes, weights: n*k).
    uint32_t ag[4], bg[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int p = t + GEMM_THREADS * i, row = p / 16;
        const int mrow = mbase + row < m ? mbase + row : m - 1;
        ag[i] = (uint32_t)mrow * (uint32_t)k + 16 * (p % 16);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int p = t + GEMM_THREADS * i;
        bg[i] = (uint32_t)brow(p / 16) * (uint32_t)k + 16 * (p % 16);
    }
    const bool xs_thread = t < 16 * GPC;
    const bool ws_thread = t >= 128;
    const int ws_row = t - 128;
    const size_t ws_base = ws_thread ? (size_t)brow(ws_row) * groups : 0;

    v4i ra[4], rb[8];
    float4 rx = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    uint4 rw = make_uint4(0, 0, 0, 0);  // HALF: 8 f16 scales; else 2 f32 in .x .y
    auto fetch = [&](int c) {
        const size_t off = (size_t)c * KC;
        // Every piece of the thread sits at byte 16 (t % 16) of its row's chunk.
        const bool in_k = !TAIL || 16 * (t % 16) < k - c * KC;
#pragma unroll
        for (int i = 0; i < 4; ++i) ra[i] = in_k ? *(const v4i*)(xq + ag[i] + off) : v4i{0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 8; ++i) rb[i] = in_k ? *(const v4i*)(codes + bg[i] + off) : v4i{0, 0, 0, 0};
        if (xs_thread) {
            if (!TAIL || c * GPC + t / 16 < groups)
                rx = *(const float4*)(xs + (size_t)(c * GPC + t / 16) * mpad + mbase + 4 * (t % 16));
            else
                rx = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
        if (ws_thread && TAIL) {
            // A row's scales start anywhere: one load a scale, none past the row.
            uint32_t v[4] = {0, 0, 0, 0};
            if (HALF) {
#pragma unroll
                for (int j = 0; j < GPC; ++j)
                    if (c * GPC + j < groups)
                        v[j / 2] |= (uint32_t)((const uint16_t*)scales)[ws_base + c * GPC + j] << (16 * (j % 2));
            } else {
#pragma unroll
                for (int j = 0; j < GPC; ++j)
                    if (c * GPC + j < groups)
                        v[j] = __builtin_bit_cast(uint32_t, ((const float*)scales)[ws_base + c * GPC + j]);
            }
            rw = make_uint4(v[0], v[1], v[2], v[3]);
        } else if (ws_thread) {
            if (HALF) {
                rw = *(const uint4*)((const uint16_t*)scales + ws_base + c * GPC);
            } else {
                const float2 f = *(const float2*)((const float*)scales + ws_base + c * GPC);
                rw.x = __builtin_bit_cast(uint32_t, f.x);
                rw.y = __builtin_bit_cast(uint32_t, f.y);
            }
        }
    };
    auto stash = [&]() {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int p = t + GEMM_THREADS * i;
            *(v4i*)(st.a + (p / 16) * ROW_LDS + 16 * (p % 16)) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int p = t + GEMM_THREADS * i;
            *(v4i*)(st.b + (p / 16) * ROW_LDS + 16 * (p % 16)) = rb[i];
        }
        if (xs_thread) *(float4*)(&st.xs[t / 16][4 * (t % 16)]) = rx;
        if (ws_thread) {
            if (HALF) {
                const uint32_t v[4] = {rw.x, rw.y, rw.z, rw.w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    st.ws[2 * j][ws_row] = f16_to_f32((uint16_t)(v[j] & 0xffff));
                    st.ws[2 * j + 1][ws_row] = f16_to_f32((uint16_t)(v[j] >> 16));
                }
            } else {
                st.ws[0][ws_row] = __builtin_bit_cast(float, rw.x);
                st.ws[1][ws_row] = __builtin_bit_cast(float, rw.y);
            }
        }
    };

    // The wave's tiles: x rows [32 (w % 2), +32) of the block; weight LDS
    // rows sub0 and sub1 (+32 each).
    const int wn = w / 2;
    const int sub0 = P == 1 ? wn * 64 : wn * 32;
    const int sub1 = P == 1 ? wn * 64 + 32 : 64 + wn * 32;
    const int8_t* la = st.a + ((w % 2) * 32 + lr) * ROW_LDS + 16 * h;
    const int8_t* lb0 = st.b + (sub0 + lr) * ROW_LDS + 16 * h;
    const int8_t* lb1 = st.b + (sub1 + lr) * ROW_LDS + 16 * h;
    const int xrow = (w % 2) * 32 + 4 * h;

    float t0[16], t1[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) t0[r] = t1[r] = 0.0f;

    fetch(0);
    for (int c = 0; c < chunks; ++c) {
        __syncthreads();  // the previous chunk's reads are done
        stash();
        __syncthreads();
        if (c + 1 < chunks) fetch(c + 1);  // lands while this chunk computes
        // Software pipeline over the chunk's groups: at step gi the matrix
        // cores run group gi + 1 from fragments read one step earlier, LDS
        // reads for group gi + 2 are in flight, and the vector ALUs run
        // group gi's f32 chain. Scheduling barriers keep the compiler from
        // folding the stages back together.
        Frags<CH> f, fn;
        v16i d0 = {}, d1 = {};
        read_frags<G>(la, lb0, lb1, 0, f);
        mfma_group<G>(f, d0, d1);
        if (GPC > 1) read_frags<G>(la, lb0, lb1, 1, f);
#pragma unroll
        for (int gi = 0; gi < GPC; ++gi) {
            v16i n0 = {}, n1 = {};
            if (gi + 1 < GPC) mfma_group<G>(f, n0, n1);
            if (gi + 2 < GPC) read_frags<G>(la, lb0, lb1, gi + 2, fn);
            Scales sc;
            read_scales(st.xs[gi], st.ws[gi], xrow, sub0 + lr, sub1 + lr, sc);
            __builtin_amdgcn_sched_barrier(0);
            // Output (row 8*(r/4) + 4h + r%4, column lr) of a tile is register r.
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if (TAIL && c * GPC + gi >= groups) break;  // past k: no chain step
                const float xv[4] = {sc.x[q].x, sc.x[q].y, sc.x[q].z, sc.x[q].w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int r = 4 * q + j;
                    t0[r] = __builtin_fmaf((float)d0[r], sc.w0 * xv[j], t0[r]);
                    t1[r] = __builtin_fmaf((float)d1[r], sc.w1 * xv[j], t1[r]);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            d0 = n0;
            d1 = n1;
            f = fn;
        }
    }

    // Epilogue, as the small-batch kernel's: bias, relu, then the residual
    // add or the SwiGLU pair (src/models/parts/causal_lm.rs:464-473).
    const int r0 = P == 1 ? bn * 128 + sub0 : bn * 64 + wn * 32;
    const int r1 = P == 1 ? bn * 128 + sub1 : n / 2 + r0;
    const int m0 = mbase + (w % 2) * 32;
    const int ldy = n / P;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int row = m0 + 8 * (r / 4) + 4 * h + r % 4;
        if (row >= m) continue;
        float v0 = t0[r], v1 = t1[r];
        if (bias) {
            v0 = v0 + bias[min(r0 + lr, n - 1)];  // columns past n are not stored
            v1 = v1 + bias[min(r1 + lr, n - 1)];
        }
        if (a.relu) {
            v0 = __builtin_fmaxf(v0, 0.0f);
            v1 = __builtin_fmaxf(v1, 0.0f);
        }
        if (P == 2) {
            a.y[(size_t)row * ldy + r0 + lr] = silu_trit(v0) * v1;
            continue;
        }
        const size_t i0 = (size_t)row * ldy + r0 + lr, i1 = (size_t)row * ldy + r1 + lr;
        if (r0 + lr < n) a.y[i0] = a.epilogue == EPI_RESIDUAL ? a.residual[i0] + v0 : v0;
        if (r1 + lr < n) a.y[i1] = a.epilogue == EPI_RESIDUAL ? a.residual[i1] + v1 : v1;
    }
}

// The same product with the K stages loaded straight into LDS
// (global_load_lds_dwordx4: no staging registers) and double-buffered, so
// one barrier a stage suffices and several blocks share a CU: the vector
// ALUs, which bound this bit-exact product, stay busy while waves wait on
// LDS, the matrix cores or a barrier. A stage holds 128 bytes of K (four
// Q8_0 groups or one int8 group) of the block's 64 x rows and 64 TW weight
// rows, and the stage's scales as they lie in memory (x scales f32
// group-major, weight scales f16 or f32 per row). A row's eight 16-byte
// pieces sit in LDS in the order piece ^ ((row >> 1) & 7), so the 32 rows
// a wave's MFMA operand reads start in different banks. Waves 2 x 2: a wave
// owns 32 x rows by TW 32-row weight tiles (TW = 2: 128-row blocks, 3 a CU,
// 52 KB of LDS each; TW = 1: 64-row blocks, 4 a CU, 35 KB -- for products
// too narrow to give every CU the same number of wide blocks). The SwiGLU
// pair takes TW = 2 (a lane holds the gate and the up output it joins).
// k must be a multiple of 128.
constexpr int KD = 128;
typedef __attribute__((address_space(3))) void LdsVoid;

template <int TW>
struct alignas(16) DStage {
    alignas(16) int8_t a[BM * KD];
    alignas(16) int8_t b[64 * TW * KD];
    alignas(16) float xs[4 * BM];            // [group of the stage][x row]
    alignas(16) uint32_t ws[2 * 64 * TW];    // f16: row r's four at [2r, 2r + 2); f32: row r's one at [r]
};

__device__ __forceinline__ int piece_swizzle(int row) { return (row >> 1) & 7; }

// Loads of 16 (4) bytes a lane from g into LDS at l + 16 (4) x lane (l the
// same for the wave). Written out rather than as the compiler's builtin,
// whose wait counting, unable to tell the stages apart, can wait for every
// load in flight before a read of the other stage; the kernel waits for
// these loads itself (vmcnt).
__device__ __forceinline__ uint32_t lds_address(const void* l) { return (uint32_t)(uintptr_t)(const LdsVoid*)l; }

__device__ __forceinline__ void load16_to_lds(const void* g, void* l) {
    asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(lds_address(l)) : "memory");
}

__device__ __forceinline__ void load4_to_lds(const void* g, void* l) {
    asm volatile("global_load_lds_dword %0, off" ::"v"(g), "{m0}"(lds_address(l)) : "memory");
}

template <int G, bool HALF, int P, int TW>
__global__ __launch_bounds__(GEMM_THREADS, TW == 2 ? 3 : 4) void gemm_dma_kernel(
    const int8_t* __restrict__ xq, const float* __restrict__ xs, int m, int mpad, const int8_t* __restrict__ codes,
    const void* __restrict__ scales, const float* __restrict__ bias, int n, int k, int nb, int mb, GemvArgs a) {
    constexpr int GPC = KD / G;  // groups per stage
    constexpr int CH = G / 32;   // MFMA steps per group
    constexpr int BN = 64 * TW;  // weight rows per block
    static_assert(GPC * CH == 4, "a stage is four 32-byte MFMA steps");
    static_assert(P == 1 || TW == 2, "the SwiGLU pair: gate and up tiles in one wave");
    __shared__ DStage<TW> st0, st1;
    if (a.skip && *a.skip) return;
    const int groups = k / G, chunks = k / KD;
    const int blk = blockIdx.x;
    int bn, bm;
    if (nb % 8 == 0) {
        const int q = blk / 8;
        bn = blk % 8 + 8 * (q / mb);
        bm = q % mb;
    } else {
        bn = blk % nb;
        bm = blk / nb;
    }
    const int t = threadIdx.x;
    const int lane = t % WAVE, w = __builtin_amdgcn_readfirstlane(t / WAVE);
    const int lr = lane % 32, h = lane / 32;
    const int mbase = bm * BM;
    // LDS weight row i holds weight row brow(i); for the SwiGLU pair, 64
    // gate rows then their 64 up rows. Rows past n load row n - 1.
    auto brow = [&](int i) {
        const int r = P == 1 ? bn * BN + i : (i < 64 ? bn * 64 + i : n / 2 + bn * 64 + (i - 64));
        return r < n ? r : n - 1;
    };

    // The wave's loads of a stage: 1 KB an instruction (eight rows of 128
    // bytes), x rows [16w, +16) and weight rows [16 TW w, +16 TW); then SPW
    // scale loads: item 0 the x scales (1 KB: four groups of 64 rows, or one
    // group and copies), items 1.. the weight scales (f16: 32 rows an item,
    // two dwords a row; f32: 64 rows an item, one dword a row), items
    // w, w + 4, ... for wave w (a wave past the last item repeats it: the
    // same bytes to the same place).
    uint32_t ag[2], bg[2 * TW];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int rl = 8 * (2 * w + i) + lane / 8;
        const int mrow = mbase + rl < m ? mbase + rl : m - 1;
        ag[i] = (uint32_t)mrow * (uint32_t)k + 16 * ((lane % 8) ^ piece_swizzle(rl));
    }
#pragma unroll
    for (int i = 0; i < 2 * TW; ++i) {
        const int rl = 8 * (2 * TW * w + i) + lane / 8;
        bg[i] = (uint32_t)brow(rl) * (uint32_t)k + 16 * ((lane % 8) ^ piece_swizzle(rl));
    }
    constexpr int NWS = HALF ? 2 * TW : TW;  // weight-scale items
    constexpr int SPW = (1 + NWS + 3) / 4;   // scale loads a wave
    int item[SPW];
    size_t soff[SPW];
#pragma unroll
    for (int j = 0; j < SPW; ++j) {
        const int it = w + 4 * j < 1 + NWS ? w + 4 * j : NWS;
        item[j] = it;
        if (it == 0)
            soff[j] = (size_t)(GPC == 4 ? lane / 16 : 0) * mpad + mbase + 4 * (lane % 16);
        else if (HALF)
            soff[j] = (size_t)brow(32 * (it - 1) + lane / 2) * (groups / 2) + lane % 2;
        else
            soff[j] = (size_t)brow(64 * (it - 1) + lane) * groups;
    }
    auto issue = [&](int c, DStage<TW>& s) {
        const size_t off = (size_t)c * KD;
#pragma unroll
        for (int i = 0; i < 2; ++i) load16_to_lds(xq + ag[i] + off, s.a + 1024 * (2 * w + i));
#pragma unroll
        for (int i = 0; i < 2 * TW; ++i) load16_to_lds(codes + bg[i] + off, s.b + 1024 * (2 * TW * w + i));
#pragma unroll
        for (int j = 0; j < SPW; ++j) {
            if (item[j] == 0)
                load16_to_lds(xs + soff[j] + (size_t)c * GPC * mpad, s.xs);
            else if (HALF)
                load4_to_lds((const uint32_t*)scales + soff[j] + 2 * c, s.ws + 64 * (item[j] - 1));
            else
                load4_to_lds((const float*)scales + soff[j] + c, s.ws + 64 * (item[j] - 1));
        }
    };

    // The wave's tiles: x rows [32 (w % 2), +32); weight LDS rows sub0 (and
    // sub1 for TW = 2), 32 each. Lane (lr, h) reads piece 2 s + h of its
    // rows for step s; its rows all share (lr >> 1) & 7.
    const int wn = w / 2;
    const int sub0 = TW == 1 ? wn * 32 : P == 1 ? wn * 64 : wn * 32;
    const int sub1 = TW == 1 ? sub0 : P == 1 ? wn * 64 + 32 : 64 + wn * 32;
    const int xrow = (w % 2) * 32 + 4 * h;
    uint32_t pa[4], pb[4];
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
        const int po = 16 * ((2 * s4 + h) ^ piece_swizzle(lr));
        pa[s4] = ((w % 2) * 32 + lr) * KD + po;
        pb[s4] = (sub0 + lr) * KD + po;
    }
    constexpr int B1 = (P == 1 ? 32 : 64) * KD;  // sub1 - sub0 rows, in bytes (TW = 2)

    float t0[16], t1[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) t0[r] = t1[r] = 0.0f;

    auto compute = [&](const DStage<TW>& s) {
        const int8_t* sa = s.a;
        const int8_t* sb = s.b;
        // The stage's weight scales of the lane's columns.
        float wsc0[GPC], wsc1[GPC];
        if (HALF) {
            const uint2 u0 = *(const uint2*)(s.ws + 2 * (sub0 + lr));
            const uint2 u1 = TW == 2 ? *(const uint2*)(s.ws + 2 * (sub1 + lr)) : u0;
            const uint32_t v0[2] = {u0.x, u0.y}, v1[2] = {u1.x, u1.y};
#pragma unroll
            for (int g = 0; g < GPC; ++g) {
                wsc0[g] = f16_to_f32((uint16_t)(v0[g / 2] >> (16 * (g % 2))));
                wsc1[g] = f16_to_f32((uint16_t)(v1[g / 2] >> (16 * (g % 2))));
            }
        } else {
            wsc0[0] = __builtin_bit_cast(float, s.ws[sub0 + lr]);
            wsc1[0] = __builtin_bit_cast(float, s.ws[sub1 + lr]);
        }
        Frags<CH> f;
#pragma unroll
        for (int c4 = 0; c4 < CH; ++c4) {
            f.a[c4] = *(const v4i*)(sa + pa[c4]);
            f.b0[c4] = *(const v4i*)(sb + pb[c4]);
            if (TW == 2) f.b1[c4] = *(const v4i*)(sb + pb[c4] + B1);
        }
#pragma unroll
        for (int gi = 0; gi < GPC; ++gi) {
            v16i d0 = {}, d1 = {};
#pragma unroll
            for (int c4 = 0; c4 < CH; ++c4) {
                d0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a[c4], f.b0[c4], d0, 0, 0, 0);
                if (TW == 2) d1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a[c4], f.b1[c4], d1, 0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            if (gi + 1 < GPC) {
#pragma unroll
                for (int c4 = 0; c4 < CH; ++c4) {
                    const int s4 = (gi + 1) * CH + c4;
                    f.a[c4] = *(const v4i*)(sa + pa[s4]);
                    f.b0[c4] = *(const v4i*)(sb + pb[s4]);
                    if (TW == 2) f.b1[c4] = *(const v4i*)(sb + pb[s4] + B1);
                }
            }
            float4 xv4[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) xv4[q] = *(const float4*)(s.xs + gi * BM + xrow + 8 * q);
            __builtin_amdgcn_sched_barrier(0);
            // Output (row 8*(r/4) + 4h + r%4, column lr) of a tile is register r.
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float xv[4] = {xv4[q].x, xv4[q].y, xv4[q].z, xv4[q].w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int r = 4 * q + j;
                    t0[r] = __builtin_fmaf((float)d0[r], wsc0[gi] * xv[j], t0[r]);
                    if (TW == 2) t1[r] = __builtin_fmaf((float)d1[r], wsc1[gi] * xv[j], t1[r]);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // Three stages in a ring, two in flight while one computes: a stage
    // takes about a microsecond to arrive, longer than one stage's work.
    // Before computing stage c a wave waits for its own loads of stage c
    // (those of stage c + 1 may stay in flight: the wave's loads a stage
    // are counted below), then the barrier makes every wave's loads of c
    // visible and frees the buffer of stage c - 1 for stage c + 2.
    // Two stages: stage c + 1 loads while stage c computes. (A third stage
    // in flight, with a block fewer a CU for its LDS, measured slower.)
    auto step = [&](int c, DStage<TW>& cur, DStage<TW>& next) {
        // This wave's loads of stage c (the only ones in flight) landed; the
        // barrier: every wave's, and every wave is done with stage c - 1,
        // whose buffer stage c + 1 takes. A bare barrier: __syncthreads
        // would add nothing the wait does not already give.
        __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
        asm volatile("s_barrier" ::: "memory");
        if (c + 1 < chunks) issue(c + 1, next);
        compute(cur);
    };
    issue(0, st0);
    for (int c = 0; c < chunks; c += 2) {
        step(c, st0, st1);
        if (c + 1 >= chunks) break;
        step(c + 1, st1, st0);
    }

    // Epilogue, as gemm_kernel's (src/models/parts/causal_lm.rs:464-473).
    const int r0 = P == 1 ? bn * BN + sub0 : bn * 64 + wn * 32;
    const int r1 = P == 1 ? bn * BN + sub1 : n / 2 + r0;
    const int m0 = mbase + (w % 2) * 32;
    const int ldy = n / P;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int row = m0 + 8 * (r / 4) + 4 * h + r % 4;
        if (row >= m) continue;
        float v0 = t0[r], v1 = t1[r];
        if (bias) {
            v0 = v0 + bias[min(r0 + lr, n - 1)];
            v1 = v1 + bias[min(r1 + lr, n - 1)];
        }
        if (a.relu) {
            v0 = __builtin_fmaxf(v0, 0.0f);
            v1 = __builtin_fmaxf(v1, 0.0f);
        }
        if (P == 2) {
            a.y[(size_t)row * ldy + r0 + lr] = silu_trit(v0) * v1;
            continue;
        }
        const size_t i0 = (size_t)row * ldy + r0 + lr, i1 = (size_t)row * ldy + r1 + lr;
        if (r0 + lr < n) a.y[i0] = a.epilogue == EPI_RESIDUAL ? a.residual[i0] + v0 : v0;
        if (TW == 2 && r1 + lr < n) a.y[i1] = a.epilogue == EPI_RESIDUAL ? a.residual[i1] + v1 : v1;
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

// Whether 64-row weight blocks (four a CU) spread the product more evenly
// than 128-row ones (three a CU) -- TRIT_HIP_GEMM_TILE=64 or 128 forces one.
bool narrow(int n, int mb) {
    static const int forced = [] {
        const char* v = getenv("TRIT_HIP_GEMM_TILE");
        return v && *v ? (int)strtol(v, nullptr, 10) : 0;
    }();
    if (forced) return forced == 64;
    return true;
}

template <int G, bool HALF, int P>
void launch_gemm(const Layer& L, const GemvArgs& a, const Scratch& sc, hipStream_t s) {
    const int nb = P == 1 ? (L.n + 127) / 128 : (L.n / 2) / 64;
    const int mb = sc.mpad / BM;
    if constexpr (P == 1) {
        if (L.k % KD == 0 && narrow(L.n, mb)) {
            const int nb1 = (L.n + 63) / 64;
            launch_timed(a, gemm_dma_kernel<G, HALF, P, 1>, dim3(nb1 * mb), dim3(GEMM_THREADS), 0, s,
                         (const int8_t*)sc.xq, (const float*)sc.xs, a.m, sc.mpad, L.codes.as<int8_t>(),
                         (const void*)L.scales.ptr, L.bias.as<float>(), L.n, L.k, nb1, mb, a);
            TRIT_HIP(hipGetLastError());
            return;
        }
    }
    if (L.k % KD == 0)
        launch_timed(a, gemm_dma_kernel<G, HALF, P, 2>, dim3(nb * mb), dim3(GEMM_THREADS), 0, s,
                     (const int8_t*)sc.xq, (const float*)sc.xs, a.m, sc.mpad, L.codes.as<int8_t>(),
                     (const void*)L.scales.ptr, L.bias.as<float>(), L.n, L.k, nb, mb, a);
    else if (L.k % KC == 0)
        launch_timed(a, gemm_kernel<G, HALF, P, false>, dim3(nb * mb), dim3(GEMM_THREADS), 0, s,
                     (const int8_t*)sc.xq, (const float*)sc.xs, a.m, sc.mpad, L.codes.as<int8_t>(),
                     (const void*)L.scales.ptr, L.bias.as<float>(), L.n, L.k, nb, mb, a);
    else
        launch_timed(a, gemm_kernel<G, HALF, P, true>, dim3(nb * mb), dim3(GEMM_THREADS), 0, s,
                     (const int8_t*)sc.xq, (const float*)sc.xs, a.m, sc.mpad, L.codes.as<int8_t>(),
                     (const void*)L.scales.ptr, L.bias.as<float>(), L.n, L.k, nb, mb, a);
    TRIT_HIP(hipGetLastError());
}

}  // namespace

bool gemm_supported(const Layer& L, const GemvArgs& a) {
    if (L.kind != Q8_0 && L.kind != Q4_K && L.kind != INT8) return false;
    // k a multiple of the group (a partial last chunk of K is zero past k);
    // RMSNorm computed here takes whole 256-value chunks.
    if (L.k % group_of(L) != 0) return false;
    if (a.epilogue == EPI_SILU_PAIR && (L.n / 2) % 64 != 0) return false;
    if (a.norm_w && !a.norm_inv && L.k % KC != 0) return false;
    // 32-bit byte offsets into the codes of x and of the weights.
    if ((int64_t)a.m * L.k >= (int64_t)1 << 31 || (int64_t)L.n * L.k >= (int64_t)1 << 32) return false;
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
