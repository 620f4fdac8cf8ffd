// Q8_0 and ternary GEMV for 1..8 rows (Q4_K held as Q8_0 too): persistent
// waves that stream their weight rows.
//
// Same values as the other integer products, bit for bit: exact i32 group
// dots and Trit's f32 chain total = fma(f32(dot_g), ws_g * xs_g, total) over
// the groups in order (src/cpu/int8.rs:525-584); for ternary codes the dot
// is sum(code * x) - sum(x), codes 0..2 standing for -1..1
// (src/cpu/v2/product.rs:389-423).
//
// The one-row kernel (gemv_decode.hip) gives each wave one quad of weight
// rows and ends; over 3072+ quads its waves come in rounds, and every wave
// quantizes the activations again. Here a block of four waves quantizes the
// activations into LDS once (or copies the rows' image that the
// quantization pass made, for 2..8 rows), and each wave then walks its
// quads in segments (1024 inputs of Q8_0, 2048 of ternary): sixteen lanes a
// row, lane l loading 16-byte chunks l, l+16, ... of the segment (every
// load instruction reads 256 contiguous bytes of each of the four rows). D
// segments are in flight at once, so the loads of the next segments overlap
// the dots and the chain of this one, across quads as well as within a row.
//
// Dots and chain follow the one-row kernel: two chunks make a group, a DPP
// swap adds the group's two halves, leaving group g = l/2 + 8j in even lane
// l; the chain is a systolic pass (row_ror:2) that visits the groups in
// order, and lane 14 of each row ends with the row's total.
#include "device.h"
#include "internal.h"

#include <cstdlib>
#include <map>
#include <mutex>
#include <tuple>

namespace trit {
namespace {

constexpr int THREADS = 256;
constexpr int WAVES = THREADS / 64;
// Inputs (rows x k) a block quantizes itself; more come from the pass
// (measured: 8 x 4096 ternary inputs in every block took 21 us against
// 15 us with the pass).
constexpr size_t IN_BLOCK = 16384;

// Weight kinds. A 16-byte chunk holds KPC inputs; two chunks make a group
// of G inputs with one weight scale, so in both kinds the lanes 2i, 2i+1 of
// a row hold the halves of group i + 8j. S chunks a lane make a segment.
struct Q8S {  // Q8_0 (and Q4_K held as Q8_0): codes row-major, f16 scales
    static constexpr int KPC = 16, G = 32, S = 4, DIV = 1;
    static constexpr bool TERN = false;
    __device__ static float scale(const void* s, size_t i) { return f16_to_f32(((const uint16_t*)s)[i]); }
    // Exact dot of chunk c (inputs 16c..16c+15) with one row's codes.
    __device__ static int dot(const uint4& w, const int8_t* xq, int c, int k) {
        const uint4 xc = *(const uint4*)(xq + c * 16);
        int d = sdot4(w.x, xc.x, 0);
        d = sdot4(w.y, xc.y, d);
        d = sdot4(w.z, xc.z, d);
        return sdot4(w.w, xc.w, d);
    }
};
struct T2S {  // ternary 2-bit codes (k/4 bytes a row), f32 scales per 128
    static constexpr int KPC = 64, G = 128, S = 2, DIV = 4;
    static constexpr bool TERN = true;
    __device__ static float scale(const void* s, size_t i) { return ((const float*)s)[i]; }
    // Word j of the chunk holds inputs 16j..16j+15 of the chunk's 64, input
    // 16j + 4s + b in bits 2s..2s+1 of byte b; the activation codes sit in
    // four planes of k/4 bytes, plane j holding inputs 16j..16j+15 of chunk
    // c at byte 16c (the quantizer's layout).
    __device__ static int dot(const uint4& w, const int8_t* xq, int c, int k) {
        const uint32_t words[4] = {w.x, w.y, w.z, w.w};
        int d = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint4 xc = *(const uint4*)(xq + j * (k >> 2) + c * 16);
            d = sdot4(words[j] & 0x03030303u, xc.x, d);
            d = sdot4((words[j] >> 2) & 0x03030303u, xc.y, d);
            d = sdot4((words[j] >> 4) & 0x03030303u, xc.z, d);
            d = sdot4((words[j] >> 6) & 0x03030303u, xc.w, d);
        }
        return d;
    }
};

template <class W, int P>
struct Seg {
    uint4 w[P][W::S];
    float ws[P][W::S];
};

// Chunk index in its row of lane l's chunk jj of segment `seg`.
template <class W>
__device__ __forceinline__ int chunk_of(int seg, int jj, int l) {
    return seg * (W::S * 16) + l + 16 * jj;
}

template <class W, int P>
__device__ __forceinline__ void load_seg(Seg<W, P>& b, const uint8_t* __restrict__ codes,
                                         const void* __restrict__ scales, int part_rows, int k, int row, int seg,
                                         int l) {
    const int groups = k / W::G;
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const size_t r = (size_t)(p * part_rows + row);
        const uint8_t* src = codes + r * (size_t)(k / W::DIV);
#pragma unroll
        for (int jj = 0; jj < W::S; ++jj) b.w[p][jj] = load_stream(src + (size_t)chunk_of<W>(seg, jj, l) * 16);
#pragma unroll
        for (int jj = 0; jj < W::S; ++jj) b.ws[p][jj] = W::scale(scales, r * groups + (chunk_of<W>(seg, jj, l) >> 1));
    }
}

// Segment `seg` of a quad: its dots against every activation row, and the
// chain steps of its 8S groups.
template <class W, int F, int P>
__device__ __forceinline__ void chain_seg(const Seg<W, P>& b, const int8_t* xq, const float* xs, const int* xsum,
                                          int k, int gs, int seg, int l, float (&acc)[P][F]) {
#pragma unroll
    for (int jj = 0; jj < W::S; ++jj) {
        const int c = chunk_of<W>(seg, jj, l), g = c >> 1;
        float df[P][F], pr[P][F];
#pragma unroll
        for (int f = 0; f < F; ++f) {
            const float sx = xs[f * gs + g];
#pragma unroll
            for (int p = 0; p < P; ++p) {
                int d = W::dot(b.w[p][jj], xq + (size_t)f * k, c, k);
                d += dpp<DPP_XOR1>(d);
                if (W::TERN) d -= xsum[f * gs + g];
                df[p][f] = (float)d;
                pr[p][f] = b.ws[p][jj] * sx;
            }
        }
        const bool first = seg == 0 && jj == 0;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
#pragma unroll
            for (int p = 0; p < P; ++p)
#pragma unroll
                for (int f = 0; f < F; ++f) {
                    const float in = (first && q == 0) ? 0.0f : dpp<DPP_ROR2>(acc[p][f]);
                    acc[p][f] = __builtin_fmaf(df[p][f], pr[p][f], in);
                }
        }
    }
}

template <int F, int P>
__device__ __forceinline__ void finish(const float (&acc)[P][F], const float* __restrict__ bias, int out_n,
                                       int row, const GemvArgs& a) {
#pragma unroll
    for (int f = 0; f < F; ++f) {
        const size_t o = (size_t)f * out_n + row;
        if (P == 2) {
            a.y[o] = silu_trit(acc[0][f]) * acc[P - 1][f];
            continue;
        }
        float y = acc[0][f];
        if (bias) y = y + bias[row];
        if (a.relu) y = __builtin_fmaxf(y, 0.0f);
        a.y[o] = a.epilogue == EPI_RESIDUAL ? a.residual[o] + y : y;
    }
}

// Trit's quantizer for the block's rows into LDS, in the layout of the
// quantization pass, after RMSNorm with the caller's factors when `nw` is
// given. Float4 item i holds inputs 4i..4i+3 of the rows laid end to end;
// the G/4 lanes of a group find its peak (and, for ternary, its code sum)
// by lane moves. Each thread loads QB items before it quantizes them, so
// their latencies overlap (a load per item in turn cost 8 us over 16 items).
template <class W>
__device__ __forceinline__ void quantize_rows(const float* __restrict__ x, const float* __restrict__ nw,
                                              const float* __restrict__ inv, int rows, int k, int8_t* xq,
                                              float* xs, int* xsum, int gs, int nt = THREADS) {
    constexpr int QB = 8;
    const int ipr = k / 4, items = rows * ipr;  // a multiple of the block's nt threads
    for (int base = 0; base < items; base += nt * QB) {
        float4 v[QB];
#pragma unroll
        for (int q = 0; q < QB; ++q) {
            const int item = base + q * nt + (int)threadIdx.x;
            if (base + q * nt < items) v[q] = *(const float4*)(x + (size_t)item * 4);
        }
#pragma unroll
        for (int q = 0; q < QB; ++q) {
            if (base + q * nt >= items) break;  // uniform across the block
            const int item = base + q * nt + (int)threadIdx.x;
            const int f = item / ipr, col = (item - f * ipr) * 4;
            float4 xv = v[q];
            if (nw) {
                const float4 w = *(const float4*)(nw + col);
                const float r = inv[f];
                xv.x = xv.x * (r * w.x);
                xv.y = xv.y * (r * w.y);
                xv.z = xv.z * (r * w.z);
                xv.w = xv.w * (r * w.w);
            }
            float peak = __builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(xv.x), __builtin_fabsf(xv.y)),
                                         __builtin_fmaxf(__builtin_fabsf(xv.z), __builtin_fabsf(xv.w)));
            peak = __builtin_fmaxf(peak, dpp<DPP_XOR1>(peak));
            peak = __builtin_fmaxf(peak, dpp<DPP_XOR2>(peak));
            peak = __builtin_fmaxf(peak, dpp<DPP_HALF_MIRROR>(peak));
            if (W::TERN) {
                peak = __builtin_fmaxf(peak, dpp<DPP_MIRROR>(peak));
                peak = __builtin_fmaxf(peak, __shfl_xor(peak, 16));
            }
            const float scale = peak > 0.0f ? peak / 127.0f : 1.0f;
            const float qi = 1.0f / scale;
            const int c0 = act_code(xv.x * qi), c1 = act_code(xv.y * qi);
            const int c2 = act_code(xv.z * qi), c3 = act_code(xv.w * qi);
            int8_t* rq = xq + (size_t)f * k;
            if (W::TERN) {
                int sum = c0 + c1 + c2 + c3;
                sum += dpp<DPP_XOR1>(sum);
                sum += dpp<DPP_XOR2>(sum);
                sum += dpp<DPP_HALF_MIRROR>(sum);
                sum += dpp<DPP_MIRROR>(sum);
                sum += __shfl_xor(sum, 16);
                *(uint32_t*)(rq + ((col >> 4) & 3) * (k >> 2) + (col >> 6) * 16 + (col & 15)) = pack4(c0, c1, c2, c3);
                if (col % W::G == 0) {
                    xs[f * gs + col / W::G] = scale;
                    xsum[f * gs + col / W::G] = sum;
                }
            } else {
                *(uint32_t*)(rq + col) = pack4(c0, c1, c2, c3);
                if (col % W::G == 0) xs[f * gs + col / W::G] = f16_round(scale);
            }
        }
    }
}

// F activation rows, P = 2: the SwiGLU pair (gate rows, then up rows), D
// segments in flight a wave. LDS: codes F x k, f32 scales F x gs, then (for
// ternary) i32 code sums F x gs: the quantization pass's image.
template <class W, int F, int P, int D>
__global__ __launch_bounds__(THREADS) void gemv_stream_kernel(const uint8_t* __restrict__ codes,
                                                              const void* __restrict__ scales,
                                                              const float* __restrict__ bias, int n, int k,
                                                              GemvArgs a) {
    extern __shared__ __align__(16) char smem_raw[];
    if (a.skip && *a.skip) return;
    const int gs = dot_stride(k / W::G);
    int8_t* xq = (int8_t*)smem_raw;
    float* xs = (float*)(smem_raw + align16((size_t)F * k));
    int* xsum = (int*)(smem_raw + align16((size_t)F * k) + align16((size_t)F * gs * 4));
    const int lane = threadIdx.x & 63, l = lane & 15;
    const int wave = threadIdx.x >> 6, waves = (int)blockDim.x >> 6;
    const int part_rows = n / P;
    const int quads = part_rows / 4;
    const int gw = blockIdx.x * waves + wave, nw = gridDim.x * waves;
    const int nseg = k / (W::S * 16 * W::KPC);
    const int total = gw < quads ? ((quads - 1 - gw) / nw + 1) * nseg : 0;

    // The first D segments' loads, then the activations under them.
    Seg<W, P> buf[D];
    int lq = gw, ls = 0;  // quad and segment of the next load
#pragma unroll
    for (int d = 0; d < D; ++d) {
        if (d < total) {
            load_seg<W, P>(buf[d], codes, scales, part_rows, k, lq * 4 + (lane >> 4), ls, l);
            if (++ls == nseg) ls = 0, lq += nw;
        }
    }
    if (a.pre) {
        // 2..8 rows: the image the quantization pass wrote, in this layout.
        const size_t bytes = align16((size_t)F * k) + (W::TERN ? 2 : 1) * align16((size_t)F * gs * 4);
#pragma unroll 8
        for (int i = threadIdx.x; i < (int)(bytes / 16); i += (int)blockDim.x) ((uint4*)smem_raw)[i] = ((const uint4*)a.pre)[i];
    } else {
        // The rows in the block (few inputs in all): no RMSNorm, or with the
        // caller's factors.
        quantize_rows<W>(a.x, a.norm_w, a.norm_inv, F, k, xq, xs, xsum, gs, (int)blockDim.x);
    }
    __syncthreads();

    float acc[P][F];
#pragma unroll
    for (int p = 0; p < P; ++p)
#pragma unroll
        for (int f = 0; f < F; ++f) acc[p][f] = 0.0f;
    int cq = gw, cs = 0;  // quad and segment being chained
    for (int t0 = 0; t0 < total; t0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            if (t0 + d < total) {
                chain_seg<W, F, P>(buf[d], xq, xs, xsum, k, gs, cs, l, acc);
                if (cs == nseg - 1 && l == 14) finish<F, P>(acc, bias, part_rows, cq * 4 + (lane >> 4), a);
                if (++cs == nseg) cs = 0, cq += nw;
                if (t0 + d + D < total) {
                    load_seg<W, P>(buf[d], codes, scales, part_rows, k, lq * 4 + (lane >> 4), ls, l);
                    if (++ls == nseg) ls = 0, lq += nw;
                }
            }
        }
    }
}

template <class W>
size_t stream_lds(int m, int k) {
    return align16((size_t)m * k) + (W::TERN ? 2 : 1) * align16((size_t)m * dot_stride(k / W::G) * 4);
}

int resident(const void* kernel, size_t lds, int threads = THREADS) {
    static std::mutex mu;
    static std::map<std::tuple<const void*, size_t, int>, int> cache;
    std::lock_guard<std::mutex> lock(mu);
    const auto key = std::make_tuple(kernel, lds, threads);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    int per_cu = 0, dev = 0, cus = 0;
    TRIT_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, lds));
    TRIT_HIP(hipGetDevice(&dev));
    TRIT_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    return cache[key] = (per_cu > 0 ? per_cu : 1) * (cus > 0 ? cus : 1);
}

template <class W, int F, int P>
void launch(const Layer& L, const GemvArgs& a, hipStream_t s) {
    constexpr int D = P == 2 ? 2 : F <= 2 ? 4 : F <= 4 ? 3 : 2;
    auto kernel = gemv_stream_kernel<W, F, P, D>;
    const size_t lds = stream_lds<W>(F, L.k);
    const int quads = L.n / P / 4;
    // Four waves a block: measured against one and two (more blocks, each
    // quantizing the rows itself), four is faster at every C1 / C4 shape.
    const int waves = WAVES, threads = 64 * waves;
    int grid = resident((const void*)kernel, lds, threads);
    if (grid * waves > quads) grid = (quads + waves - 1) / waves;
    launch_timed(a, kernel, dim3(grid), dim3(threads), lds, s, L.codes.as<uint8_t>(), (const void*)L.scales.ptr,
                 L.bias.as<float>(), L.n, L.k, a);
    TRIT_HIP(hipGetLastError());
}

template <class W, int P>
void launch_rows(const Layer& L, const GemvArgs& a, hipStream_t s) {
    switch (a.m) {
        case 1: return launch<W, 1, P>(L, a, s);
        case 2: return launch<W, 2, P>(L, a, s);
        case 3: return launch<W, 3, P>(L, a, s);
        case 4: return launch<W, 4, P>(L, a, s);
        case 5: return launch<W, 5, P>(L, a, s);
        case 6: return launch<W, 6, P>(L, a, s);
        case 7: return launch<W, 7, P>(L, a, s);
        default: return launch<W, 8, P>(L, a, s);
    }
}

// TRIT_HIP_GEMV_STREAM: 0 never, 1 whenever the shape fits, unset: by size
// (read at each call, so that tests can switch it).
int stream_mode() {
    const char* v = getenv("TRIT_HIP_GEMV_STREAM");
    return v && *v ? atoi(v) : -1;
}

template <class W>
bool stream(const Layer& L, const GemvArgs& a, hipStream_t s) {
    if (a.m < 1 || a.m > 8 || L.k % (W::S * 16 * W::KPC) != 0) return false;
    const int P = a.epilogue == EPI_SILU_PAIR ? 2 : 1;
    if (L.n % (4 * P) != 0 || (P == 2 && L.bias.ptr)) return false;
    // Up to 16384 inputs in all quantize in the block (without RMSNorm, or
    // with the caller's factors); more take the quantization pass's image.
    const bool in_block = (size_t)a.m * L.k <= IN_BLOCK && (!a.norm_w || a.norm_inv);
    if (!a.pre && !in_block) return false;
    if (stream_lds<W>(a.m, L.k) > 64 * 1024) return false;
    const int mode = stream_mode();
    if (mode == 0) return false;
    if (mode < 0 && a.pre) {
        // After the quantization pass, by size (measured on MI355X): Q8_0
        // from 4M weights (2..4 rows) and 12M (5..8 rows), ternary from 48M
        // for 5..8 rows; below that the tiled kernel's blocks finish sooner.
        const size_t weights = (size_t)L.n * L.k;
        const size_t least = W::TERN ? (a.m <= 4 ? 0 : (size_t)48 << 20) : (a.m <= 4 ? (size_t)4 << 20 : (size_t)12 << 20);
        if (weights < least) return false;
    }
    if (P == 2)
        launch_rows<W, 2>(L, a, s);
    else
        launch_rows<W, 1>(L, a, s);
    return true;
}

// ---- Q4_K from the super-blocks as stored --------------------------------
//
// Trit expands a Q4_K super-block (f16 d and dmin, twelve bytes of 6-bit
// scales and mins, 256 4-bit codes; src/cpu/ggml_quants.rs:168-196) into
// y = d sc q - dmin m and requantizes every 32 values as Q8_0
// (Blocks::quantize, src/cpu/gemm.rs:58-76) before its int8 product. This
// product reads the 144-byte blocks (0.5625 B a weight instead of the Q8_0
// codes' 1.0625) and rebuilds the same Q8_0 codes in registers:
//  - y is affine in the 4-bit code q (d sc q is exact in f32, so the
//    expansion's rounded difference is fma(d sc, q, -dmin m)), so the
//    sub-block's peak |y| is at its smallest or largest code and its 32
//    Q8_0 codes take at most 16 values: a 16-byte code table per sub-block,
//    read with byte permutes;
//  - round(y / d8) half away from zero is (trunc(2|t|) + 1) >> 1 with
//    t = y * (1/d8) and the sign of y: exact for every finite t (2t is an
//    exact f32 scaling); blocks whose d or dmin is not finite take the
//    reference's own expression (their y can be NaN or infinite; Rust's
//    `as i8` takes a NaN code to 0).
// The exact i32 dots of those codes and the activation codes then enter
// Trit's chain total = fma(f32(dot_g), ws_g * xs_g, total) in group order.
//
// A block takes a tile of R weight rows (of each SwiGLU part): each thread
// rebuilds one or more pairs of sub-blocks (the 32 bytes holding the codes
// of sub-blocks 2j (low nibbles) and 2j + 1 (high nibbles)), writes each
// pair's (f32 dot, ws * xs) per activation row into LDS, and after a barrier
// one wave runs the tile's chains, a lane per (row, activation row) -- the
// serial part of the product, on the wave that owns the tile while the
// others rebuild the next tile (double-buffered LDS, the tiles' weights
// loaded one tile ahead).

constexpr int QK_BYTES = 144;  // a super-block: 256 weights

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ u16x2 as_u16x2(uint32_t v) { return __builtin_bit_cast(u16x2, v); }
__device__ __forceinline__ uint32_t as_u32(u16x2 v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ uint32_t as_u32(float v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ uint32_t pk_max16(uint32_t a, uint32_t b) {
    return as_u32(__builtin_elementwise_max(as_u16x2(a), as_u16x2(b)));
}
__device__ __forceinline__ uint32_t pk_min16(uint32_t a, uint32_t b) {
    return as_u32(__builtin_elementwise_min(as_u16x2(a), as_u16x2(b)));
}

// One thread's pair of sub-blocks: the super-block's first 16 bytes (d,
// dmin, the scale bytes) and the pair's 32 code bytes.
struct QkPair {
    uint4 h, c0, c1;
};

__device__ __forceinline__ void qk_load(QkPair& b, const uint8_t* __restrict__ raw, size_t row, int spr, int pair) {
    const uint8_t* sb = raw + (row * spr + (pair >> 2)) * QK_BYTES;
    b.h = load_stream(sb);
    b.c0 = load_stream(sb + 16 + (pair & 3) * 32);
    b.c1 = load_stream(sb + 32 + (pair & 3) * 32);
}

// Scale and min of sub-blocks 2jp and 2jp + 1 (ggml's get_scale_min_k4,
// src/cpu/ggml_quants.rs:150-166): scale bytes q[0..11] at header bytes 4..15.
__device__ __forceinline__ void qk_scale_min(const uint4& h, int jp, int (&sc)[2], int (&mn)[2]) {
    const int sh = 16 * (jp & 1);
    const uint32_t a = h.y >> sh, b = h.z >> sh, c = h.w >> sh;  // q[j], q[j + 4], q[j + 8] for j = 2jp & 3
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t ai = (a >> (8 * i)) & 0xFF, bi = (b >> (8 * i)) & 0xFF, ci = (c >> (8 * i)) & 0xFF;
        if (jp < 2) {
            sc[i] = (int)(ai & 63);
            mn[i] = (int)(bi & 63);
        } else {
            sc[i] = (int)((ci & 0xF) | ((ai >> 6) << 4));
            mn[i] = (int)((ci >> 4) | ((bi >> 6) << 4));
        }
    }
}

// Smallest and largest 4-bit code of each sub-block of the pair. Each
// 16-bit half of a shifted word holds one code in its top 4 bits (over
// lower bits that cannot change the order), so packed u16 max / min find
// them: low nibbles via w << 4 and w << 12, high nibbles via w and w << 8.
__device__ __forceinline__ void qk_range(const QkPair& b, int (&lo)[2], int (&hi)[2]) {
    const uint32_t w[8] = {b.c0.x, b.c0.y, b.c0.z, b.c0.w, b.c1.x, b.c1.y, b.c1.z, b.c1.w};
    uint32_t mx0 = 0, mn0 = 0xFFFFFFFFu, mx1 = 0, mn1 = 0xFFFFFFFFu;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t l4 = w[i] << 4, l12 = w[i] << 12, h8 = w[i] << 8;
        mx0 = pk_max16(pk_max16(mx0, l4), l12);
        mn0 = pk_min16(pk_min16(mn0, l4), l12);
        mx1 = pk_max16(pk_max16(mx1, w[i]), h8);
        mn1 = pk_min16(pk_min16(mn1, w[i]), h8);
    }
    auto top = [](uint32_t v, bool most) {
        const uint32_t a = v >> 28, b = (v >> 12) & 15;
        return (int)(most ? (a > b ? a : b) : (a < b ? a : b));
    };
    hi[0] = top(mx0, true);
    lo[0] = top(mn0, false);
    hi[1] = top(mx1, true);
    lo[1] = top(mn1, false);
}

// The 16 Q8_0 codes of y(q) = fma(d1, q, -m1), q = 0..15, as bytes of four
// words, with `inv` = 1 / d8 (0 when d8 is 0).
__device__ __forceinline__ void qk_table(float d1, float m1, float inv, bool finite, uint32_t (&t)[4]) {
    if (__builtin_expect(finite, 1)) {
        const float inv2 = inv * 2.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t half[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const float q = (float)(4 * i + 2 * h);
                const float ya = __builtin_fmaf(d1, q, -m1), yb = __builtin_fmaf(d1, q + 1.0f, -m1);
                const uint32_t ta = (uint32_t)__builtin_fabsf(ya * inv2), tb = (uint32_t)__builtin_fabsf(yb * inv2);
                // (trunc(2|t|) + 1) >> 1 in each half, then the sign of y.
                u16x2 mag = as_u16x2(ta | (tb << 16));
                mag = (mag + (u16x2)1) >> (u16x2)1;
                const uint32_t neg = __builtin_amdgcn_perm(as_u32(yb), as_u32(ya), 0x0B0B0909u);
                half[h] = as_u32(as_u16x2(as_u32(mag) ^ neg) - as_u16x2(neg));
            }
            t[i] = __builtin_amdgcn_perm(half[1], half[0], 0x06040200u);  // the low bytes of the four halves
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            int c[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float y = __builtin_fmaf(d1, (float)(4 * i + e), -m1);
                const float r = __builtin_roundf(y * inv);
                c[e] = r != r ? 0 : (int)__builtin_fminf(__builtin_fmaxf(r, -128.0f), 127.0f);
            }
            t[i] = pack4(c[0], c[1], c[2], c[3]);
        }
    }
}

// Code word of four 4-bit codes (at bit offset `shift` of each byte) read
// from the table: bytes 0..7 by the low three bits, 8..15 likewise, picked
// by bit 3 (a byte mask made by a permute of the constant selectors 12 and
// 13, which give 0x00 and 0xFF).
template <int SHIFT>
__device__ __forceinline__ uint32_t qk_lookup(uint32_t w, const uint32_t (&t)[4]) {
    const uint32_t sel = (w >> SHIFT) & 0x07070707u;
    const uint32_t upper = __builtin_amdgcn_perm(0u, 0u, ((w >> (SHIFT + 3)) & 0x01010101u) | 0x0C0C0C0Cu);
    const uint32_t lo = __builtin_amdgcn_perm(t[1], t[0], sel), hi = __builtin_amdgcn_perm(t[3], t[2], sel);
    return (hi & upper) | (lo & ~upper);
}

// One pair: the Q8_0 codes of both sub-blocks, their f16 scales, and the
// (f32 dot, ws * xs) of each against the F activation rows into `out`
// (float4 {dot_2j, pr_2j, dot_2j+1, pr_2j+1} per row, rows `stride` floats apart).
template <int F>
__device__ __forceinline__ void qk_pair(const QkPair& b, int pair, const int8_t* xq, const float* xs, int k, int gs,
                                        float* out, int stride) {
    const int jp = pair & 3;
    int sc[2], mn[2], qlo[2], qhi[2];
    qk_scale_min(b.h, jp, sc, mn);
    qk_range(b, qlo, qhi);
    const float d = f16_to_f32((uint16_t)(b.h.x & 0xFFFF)), dmin = f16_to_f32((uint16_t)(b.h.x >> 16));
    const bool finite = __builtin_isfinite(d) && __builtin_isfinite(dmin);
    const uint32_t w[8] = {b.c0.x, b.c0.y, b.c0.z, b.c0.w, b.c1.x, b.c1.y, b.c1.z, b.c1.w};
    int dots[2][F];
    float ws[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        const float d1 = d * (float)sc[s], m1 = dmin * (float)mn[s];
        const float ya = __builtin_fmaf(d1, (float)qlo[s], -m1), yb = __builtin_fmaf(d1, (float)qhi[s], -m1);
        const float peak = __builtin_fmaxf(__builtin_fmaxf(0.0f, __builtin_fabsf(ya)), __builtin_fabsf(yb));
        const float d8 = peak / 127.0f;
        const float inv = d8 != 0.0f ? 1.0f / d8 : 0.0f;
        ws[s] = f16_round(d8);
        uint32_t t[4];
        qk_table(d1, m1, inv, finite, t);
        uint32_t code[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) code[i] = s == 0 ? qk_lookup<0>(w[i], t) : qk_lookup<4>(w[i], t);
#pragma unroll
        for (int f = 0; f < F; ++f) {
            const uint4* xv = (const uint4*)(xq + (size_t)f * k + pair * 64 + s * 32);
            const uint4 x0 = xv[0], x1 = xv[1];
            int dt = sdot4(code[0], x0.x, 0);
            dt = sdot4(code[1], x0.y, dt);
            dt = sdot4(code[2], x0.z, dt);
            dt = sdot4(code[3], x0.w, dt);
            dt = sdot4(code[4], x1.x, dt);
            dt = sdot4(code[5], x1.y, dt);
            dt = sdot4(code[6], x1.z, dt);
            dots[s][f] = sdot4(code[7], x1.w, dt);
        }
    }
#pragma unroll
    for (int f = 0; f < F; ++f) {
        const float2 sx = *(const float2*)(xs + f * gs + 2 * pair);
        *(float4*)(out + (size_t)f * stride) =
            make_float4((float)dots[0][f], ws[0] * sx.x, (float)dots[1][f], ws[1] * sx.y);
    }
}

// LDS of the tile kernel: the activation image (codes F x k, f32 scales
// F x gs), then two buffers of F x RP rows of `stride` floats.
__host__ __device__ __forceinline__ int qk_stride(int k) { return 2 * (k / 32) + 4; }
__host__ __device__ __forceinline__ size_t qk_image(int F, int k) {
    return align16((size_t)F * k) + align16((size_t)F * dot_stride(k / 32) * 4);
}
__host__ __device__ __forceinline__ size_t qk_lds(int F, int k, int rp) {
    return qk_image(F, k) + 2 * (size_t)F * rp * qk_stride(k) * 4;
}

// Tiles of R rows of each of the P parts; I pairs a thread (blockDim.x x I
// = R P k / 64); a block walks tiles blockIdx.x, + gridDim.x, ...
template <int F, int P, int I>
__global__ __launch_bounds__(THREADS) void gemv_q4k_kernel(const uint8_t* __restrict__ raw,
                                                           const float* __restrict__ bias, int n, int k, int R,
                                                           GemvArgs a) {
    extern __shared__ __align__(16) char smem_raw[];
    if (a.skip && *a.skip) return;
    const int gs = dot_stride(k / 32), spr = k / 256, ppr = k / 64, stride = qk_stride(k);
    int8_t* xq = (int8_t*)smem_raw;
    float* xs = (float*)(smem_raw + align16((size_t)F * k));
    float* pairs = (float*)(smem_raw + qk_image(F, k));
    const int part_rows = n / P, rp = R * P, tiles = part_rows / R;
    const int nthreads = (int)blockDim.x, waves = nthreads / 64, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const size_t buf_floats = (size_t)F * rp * stride;

    auto row_of = [&](int tile, int item, int& local) {
        local = item / ppr;
        const int part = local / R, r = local - part * R;
        return (size_t)part * part_rows + (size_t)tile * R + r;
    };
    QkPair cur[I], nxt[I];
    int tile = blockIdx.x;
    if (tile >= tiles) return;
#pragma unroll
    for (int i = 0; i < I; ++i) {
        const int item = threadIdx.x + i * nthreads;
        int local;
        const size_t row = row_of(tile, item, local);
        qk_load(cur[i], raw, row, spr, item - local * ppr);
    }
    if (a.pre) {
        const size_t bytes = qk_image(F, k);
#pragma unroll 8
        for (int i = threadIdx.x; i < (int)(bytes / 16); i += nthreads) ((uint4*)smem_raw)[i] = ((const uint4*)a.pre)[i];
    } else {
        quantize_rows<Q8S>(a.x, a.norm_w, a.norm_inv, F, k, xq, xs, nullptr, gs, nthreads);
    }
    __syncthreads();

    for (int step = 0; tile < tiles; ++step, tile += gridDim.x) {
        const int next = tile + gridDim.x;
        if (next < tiles) {
#pragma unroll
            for (int i = 0; i < I; ++i) {
                const int item = threadIdx.x + i * nthreads;
                int local;
                const size_t row = row_of(next, item, local);
                qk_load(nxt[i], raw, row, spr, item - local * ppr);
            }
        }
        float* buf = pairs + (step & 1) * buf_floats;
#pragma unroll
        for (int i = 0; i < I; ++i) {
            const int item = threadIdx.x + i * nthreads;
            const int local = item / ppr, pair = item - local * ppr;
            qk_pair<F>(cur[i], pair, xq, xs, k, gs, buf + (size_t)local * stride + 4 * pair, rp * stride);
        }
        __syncthreads();
        // The tile's chains: wave (step mod waves), lane (row r, activation row f).
        if (wave == step % waves && lane < R * F) {
            const int r = lane % R, f = lane / R;
            float acc[P];
#pragma unroll
            for (int p = 0; p < P; ++p) {
                const float* src = buf + ((size_t)f * rp + p * R + r) * stride;
                float t = 0.0f;
                for (int g = 0; g < ppr; ++g) {
                    const float4 v = *(const float4*)(src + 4 * g);
                    t = __builtin_fmaf(v.x, v.y, t);
                    t = __builtin_fmaf(v.z, v.w, t);
                }
                acc[p] = t;
            }
            const size_t o = (size_t)f * part_rows + (size_t)tile * R + r;
            if (P == 2) {
                a.y[o] = silu_trit(acc[0]) * acc[P - 1];
            } else {
                float y = acc[0];
                if (bias) y = y + bias[(size_t)tile * R + r];
                if (a.relu) y = __builtin_fmaxf(y, 0.0f);
                a.y[o] = a.epilogue == EPI_RESIDUAL ? a.residual[o] + y : y;
            }
        }
#pragma unroll
        for (int i = 0; i < I; ++i) cur[i] = nxt[i];
    }
}

// A tile shape for the layer: R rows of each part, waves a block and pairs
// a thread with waves x 64 x I = R P k / 64, R F <= 64 (one wave's chains),
// LDS within 64 KB; the largest R that leaves 512 tiles, else the smallest.
struct QkShape {
    int R = 0, waves = 0, I = 0;
};
QkShape qk_shape(int part_rows, int k, int F, int P) {
    QkShape best;
    const int ppr = k / 64;
    for (int R = 1; R * F <= 64 && R <= part_rows; R *= 2) {
        if (part_rows % R) continue;
        const int items = R * P * ppr;
        if (items % 64 || qk_lds(F, k, R * P) > 64 * 1024) continue;
        QkShape s;
        for (int w = 4; w >= 1 && !s.R; --w)
            for (int i = 1; i <= 4 && !s.R; ++i)
                if (w * 64 * i == items) s = QkShape{R, w, i};
        if (!s.R) continue;
        if (!best.R || part_rows / R >= 512) best = s;
    }
    return best;
}

template <int F, int P, int I>
void qk_launch(const Layer& L, const GemvArgs& a, const QkShape& sh, hipStream_t s) {
    auto kernel = gemv_q4k_kernel<F, P, I>;
    const size_t lds = qk_lds(F, L.k, sh.R * P);
    const int threads = sh.waves * 64, tiles = L.n / P / sh.R;
    const int grid = std::min(resident((const void*)kernel, lds, threads), tiles);
    launch_timed(a, kernel, dim3(grid), dim3(threads), lds, s, L.raw.as<uint8_t>(), L.bias.as<float>(), L.n, L.k,
                 sh.R, a);
    TRIT_HIP(hipGetLastError());
}

template <int F, int P>
void qk_items(const Layer& L, const GemvArgs& a, const QkShape& sh, hipStream_t s) {
    switch (sh.I) {
        case 1: return qk_launch<F, P, 1>(L, a, sh, s);
        case 2: return qk_launch<F, P, 2>(L, a, sh, s);
        case 3: return qk_launch<F, P, 3>(L, a, sh, s);
        default: return qk_launch<F, P, 4>(L, a, sh, s);
    }
}

template <int P>
void qk_rows(const Layer& L, const GemvArgs& a, const QkShape& sh, hipStream_t s) {
    switch (a.m) {
        case 1: return qk_items<1, P>(L, a, sh, s);
        case 2: return qk_items<2, P>(L, a, sh, s);
        case 3: return qk_items<3, P>(L, a, sh, s);
        default: return qk_items<4, P>(L, a, sh, s);
    }
}

// The native product runs for layers made with TRIT_HIP_Q4K=1 (which hold
// their super-blocks) whenever the shape fits; TRIT_HIP_Q4K=0 at a call
// sends it to the requantized codes (read at each call, so that tests can
// compare both).
int q4k_mode() {
    const char* v = getenv("TRIT_HIP_Q4K");
    return v && *v ? atoi(v) : -1;
}

bool q4k(const Layer& L, const GemvArgs& a, hipStream_t s) {
    if (L.kind != Q4_K || !L.raw.ptr || a.m < 1 || a.m > 4 || L.k % 256 != 0) return false;
    const int mode = q4k_mode();
    if (mode == 0) return false;
    const int P = a.epilogue == EPI_SILU_PAIR ? 2 : 1;
    if (L.n % P != 0 || (P == 2 && L.bias.ptr)) return false;
    // The activations: quantized in the block (no RMSNorm, or with the
    // caller's factors, up to 16384 inputs in all), else the pass's image.
    const QkShape sh = qk_shape(L.n / P, L.k, a.m, P);
    if (!sh.R) return false;
    const bool in_block = (size_t)a.m * L.k <= IN_BLOCK && (a.m * L.k / 4) % (sh.waves * 64) == 0 &&
                          (!a.norm_w || a.norm_inv);
    if (!a.pre && !in_block) return false;
    if (P == 2)
        qk_rows<2>(L, a, sh, s);
    else
        qk_rows<1>(L, a, sh, s);
    return true;
}

}  // namespace

bool gemv_stream(const Layer& L, const GemvArgs& a, hipStream_t s) {
    if (L.kind == Q4_K && q4k(L, a, s)) return true;
    if (L.kind == Q8_0 || L.kind == Q4_K) return stream<Q8S>(L, a, s);
    if (L.kind == TERNARY) return stream<T2S>(L, a, s);
    return false;
}

}  // namespace trit
