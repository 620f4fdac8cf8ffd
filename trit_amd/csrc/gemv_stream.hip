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
                                              float* xs, int* xsum, int gs) {
    constexpr int QB = 8;
    const int ipr = k / 4, items = rows * ipr;  // a multiple of THREADS
    for (int base = 0; base < items; base += THREADS * QB) {
        float4 v[QB];
#pragma unroll
        for (int q = 0; q < QB; ++q) {
            const int item = base + q * THREADS + (int)threadIdx.x;
            if (base + q * THREADS < items) v[q] = *(const float4*)(x + (size_t)item * 4);
        }
#pragma unroll
        for (int q = 0; q < QB; ++q) {
            if (base + q * THREADS >= items) break;  // uniform across the block
            const int item = base + q * THREADS + (int)threadIdx.x;
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
    const int wave = threadIdx.x >> 6;
    const int part_rows = n / P;
    const int quads = part_rows / 4;
    const int gw = blockIdx.x * WAVES + wave, nw = gridDim.x * WAVES;
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
        for (int i = threadIdx.x; i < (int)(bytes / 16); i += THREADS) ((uint4*)smem_raw)[i] = ((const uint4*)a.pre)[i];
    } else {
        // The rows in the block (few inputs in all): no RMSNorm, or with the
        // caller's factors.
        quantize_rows<W>(a.x, a.norm_w, a.norm_inv, F, k, xq, xs, xsum, gs);
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

int resident(const void* kernel, size_t lds) {
    static std::mutex mu;
    static std::map<std::pair<const void*, size_t>, int> cache;
    std::lock_guard<std::mutex> lock(mu);
    const auto key = std::make_pair(kernel, lds);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    int per_cu = 0, dev = 0, cus = 0;
    TRIT_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, THREADS, lds));
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
    int grid = resident((const void*)kernel, lds);
    if (grid * WAVES > quads) grid = (quads + WAVES - 1) / WAVES;
    launch_timed(a, kernel, dim3(grid), dim3(THREADS), lds, s, L.codes.as<uint8_t>(), (const void*)L.scales.ptr,
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

}  // namespace

bool gemv_stream(const Layer& L, const GemvArgs& a, hipStream_t s) {
    if (L.kind == Q8_0 || L.kind == Q4_K) return stream<Q8S>(L, a, s);
    if (L.kind == TERNARY) return stream<T2S>(L, a, s);
    return false;
}

}  // namespace trit
