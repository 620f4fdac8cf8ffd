// Q8_0 GEMV for 1..8 rows over large weights (Q4_K held as Q8_0 too):
// persistent waves that stream their rows.
//
// Same values as the other integer products, bit for bit: exact i32 block
// dots and Trit's f32 chain total = fma(f32(dot_g), ws_g * xs_g, total) over
// the groups in order (src/cpu/int8.rs:525-584), for every activation row.
//
// The one-row kernel (gemv_decode.hip) gives each wave one quad of weight
// rows and ends; over 3072+ quads its waves come in rounds, and every wave
// quantizes the activations again. Here a block of four waves quantizes the
// activations into LDS once (or copies the rows' image that the
// quantization pass made, for 2..8 rows), and each wave then walks its
// quads in segments of 1024 inputs: sixteen lanes a row, lane l loading
// chunks l, l+16, l+32, l+48 of the segment (every load instruction reads
// 256 contiguous bytes of each of the four rows). D segments are in flight
// at once, so the loads of the next segments overlap the dots and the chain
// of this one, across quads as well as within a row.
//
// Dots and chain follow the one-row kernel: a DPP swap adds the two halves
// of each 32-value block, leaving block g = l/2 + 8j in even lane l; the
// chain is a systolic pass (row_ror:2) that visits the blocks in order, and
// lane 14 of each row ends with the row's total.
#include "device.h"
#include "internal.h"

#include <cstdlib>
#include <map>
#include <mutex>

namespace trit {
namespace {

constexpr int THREADS = 256;
constexpr int WAVES = THREADS / 64;
constexpr int S = 4;            // 16-byte chunks a lane loads per segment
constexpr int SEG = S * 256;    // inputs of a row per segment

template <int P>
struct Seg {
    uint4 w[P][S];
    float ws[P][S];
};

template <int P>
__device__ __forceinline__ void load_seg(Seg<P>& b, const uint8_t* __restrict__ codes,
                                         const uint16_t* __restrict__ scales, int part_rows, int k, int row,
                                         int seg, int l) {
    const int groups = k / 32;
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const size_t r = (size_t)(p * part_rows + row);
        const uint8_t* src = codes + r * k + (size_t)seg * SEG;
#pragma unroll
        for (int jj = 0; jj < S; ++jj) b.w[p][jj] = load_stream(src + (size_t)(l + 16 * jj) * 16);
        const uint16_t* sc = scales + r * groups + seg * (S * 8) + (l >> 1);
#pragma unroll
        for (int jj = 0; jj < S; ++jj) b.ws[p][jj] = f16_to_f32(sc[8 * jj]);
    }
}

// Segment `seg` of a quad: its dots against every activation row, and the
// chain steps of its 8S blocks.
template <int F, int P>
__device__ __forceinline__ void chain_seg(const Seg<P>& b, const int8_t* xq, const float* xs, int k, int gs,
                                          int seg, int l, float (&acc)[P][F]) {
#pragma unroll
    for (int jj = 0; jj < S; ++jj) {
        const int j = seg * S + jj;
        float df[P][F], pr[P][F];
#pragma unroll
        for (int f = 0; f < F; ++f) {
            const uint4 xc = *(const uint4*)(xq + (size_t)f * k + (l + 16 * j) * 16);
            const float sx = xs[f * gs + (l >> 1) + 8 * j];
#pragma unroll
            for (int p = 0; p < P; ++p) {
                int d = sdot4(b.w[p][jj].x, xc.x, 0);
                d = sdot4(b.w[p][jj].y, xc.y, d);
                d = sdot4(b.w[p][jj].z, xc.z, d);
                d = sdot4(b.w[p][jj].w, xc.w, d);
                d += dpp<DPP_XOR1>(d);
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

// F activation rows, P = 2: the SwiGLU pair (gate rows, then up rows), D
// segments in flight a wave. LDS: codes F x k, then f32 scales F x gs.
template <int F, int P, int D>
__global__ __launch_bounds__(THREADS) void gemv_stream_kernel(const uint8_t* __restrict__ codes,
                                                              const uint16_t* __restrict__ scales,
                                                              const float* __restrict__ bias, int n, int k,
                                                              GemvArgs a) {
    extern __shared__ __align__(16) char smem_raw[];
    if (a.skip && *a.skip) return;
    const int gs = dot_stride(k / 32);
    int8_t* xq = (int8_t*)smem_raw;
    float* xs = (float*)(smem_raw + align16((size_t)F * k));
    const int lane = threadIdx.x & 63, l = lane & 15;
    const int wave = threadIdx.x >> 6;
    const int part_rows = n / P;
    const int quads = part_rows / 4;
    const int gw = blockIdx.x * WAVES + wave, nw = gridDim.x * WAVES;
    const int nseg = k / SEG;
    const int total = gw < quads ? ((quads - 1 - gw) / nw + 1) * nseg : 0;

    // The first D segments' loads, then the activations under them.
    Seg<P> buf[D];
    int lq = gw, ls = 0;  // quad and segment of the next load
#pragma unroll
    for (int d = 0; d < D; ++d) {
        if (d < total) {
            load_seg<P>(buf[d], codes, scales, part_rows, k, lq * 4 + (lane >> 4), ls, l);
            if (++ls == nseg) ls = 0, lq += nw;
        }
    }
    if (a.pre) {
        // 2..8 rows: the image the quantization pass wrote, in this layout.
        const int n16 = (int)((align16((size_t)F * k) + align16((size_t)F * gs * 4)) / 16);
        for (int i = threadIdx.x; i < n16; i += THREADS) ((uint4*)smem_raw)[i] = ((const uint4*)a.pre)[i];
    } else {
        // One row (F == 1, no RMSNorm): Trit's quantizer.
        for (int item = threadIdx.x; item < k / 4; item += THREADS) {
            const float4 v = *(const float4*)(a.x + (size_t)item * 4);
            float peak = __builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(v.x), __builtin_fabsf(v.y)),
                                         __builtin_fmaxf(__builtin_fabsf(v.z), __builtin_fabsf(v.w)));
            peak = __builtin_fmaxf(peak, dpp<DPP_XOR1>(peak));
            peak = __builtin_fmaxf(peak, dpp<DPP_XOR2>(peak));
            peak = __builtin_fmaxf(peak, dpp<DPP_HALF_MIRROR>(peak));
            const float scale = peak > 0.0f ? peak / 127.0f : 1.0f;
            const float q = 1.0f / scale;
            *(uint32_t*)(xq + item * 4) =
                pack4(act_code(v.x * q), act_code(v.y * q), act_code(v.z * q), act_code(v.w * q));
            if ((item & 7) == 0) xs[item >> 3] = f16_round(scale);
        }
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
                chain_seg<F, P>(buf[d], xq, xs, k, gs, cs, l, acc);
                if (cs == nseg - 1 && l == 14) finish<F, P>(acc, bias, part_rows, cq * 4 + (lane >> 4), a);
                if (++cs == nseg) cs = 0, cq += nw;
                if (t0 + d + D < total) {
                    load_seg<P>(buf[d], codes, scales, part_rows, k, lq * 4 + (lane >> 4), ls, l);
                    if (++ls == nseg) ls = 0, lq += nw;
                }
            }
        }
    }
}

size_t stream_lds(int m, int k) { return align16((size_t)m * k) + align16((size_t)m * dot_stride(k / 32) * 4); }

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

template <int F, int P>
void launch(const Layer& L, const GemvArgs& a, hipStream_t s) {
    constexpr int D = P == 2 ? 2 : F <= 2 ? 4 : F <= 4 ? 3 : 2;
    auto kernel = gemv_stream_kernel<F, P, D>;
    const size_t lds = stream_lds(F, L.k);
    const int quads = L.n / P / 4;
    int grid = resident((const void*)kernel, lds);
    if (grid * WAVES > quads) grid = (quads + WAVES - 1) / WAVES;
    launch_timed(a, kernel, dim3(grid), dim3(THREADS), lds, s, L.codes.as<uint8_t>(), L.scales.as<uint16_t>(),
                 L.bias.as<float>(), L.n, L.k, a);
    TRIT_HIP(hipGetLastError());
}

template <int P>
void launch_rows(const Layer& L, const GemvArgs& a, hipStream_t s) {
    switch (a.m) {
        case 1: return launch<1, P>(L, a, s);
        case 2: return launch<2, P>(L, a, s);
        case 3: return launch<3, P>(L, a, s);
        case 4: return launch<4, P>(L, a, s);
        case 5: return launch<5, P>(L, a, s);
        case 6: return launch<6, P>(L, a, s);
        case 7: return launch<7, P>(L, a, s);
        default: return launch<8, P>(L, a, s);
    }
}

// TRIT_HIP_GEMV_STREAM: 0 never, 1 whenever the shape fits, unset: by size.
int stream_mode() {
    static const int mode = [] {
        const char* v = getenv("TRIT_HIP_GEMV_STREAM");
        return v && *v ? atoi(v) : -1;
    }();
    return mode;
}

}  // namespace

bool gemv_stream(const Layer& L, const GemvArgs& a, hipStream_t s) {
    if (L.kind != Q8_0 && L.kind != Q4_K) return false;
    if (a.m < 1 || a.m > 8 || L.k % SEG != 0) return false;
    const int P = a.epilogue == EPI_SILU_PAIR ? 2 : 1;
    if (L.n % (4 * P) != 0 || (P == 2 && L.bias.ptr)) return false;
    // One row without RMSNorm quantizes in the block; more rows take the
    // quantization pass's image (normalized there).
    if (a.m == 1 ? a.norm_w != nullptr : !a.pre) return false;
    if (stream_lds(a.m, L.k) > 64 * 1024) return false;
    const int mode = stream_mode();
    if (mode == 0) return false;
    if (mode < 0) {
        // By size (measured on MI355X): one row streams at every size; 2..4
        // rows from 4M weights and 5..8 rows from 12M, below which the tiled
        // kernel's blocks (more of them, each a few rows) finish sooner.
        const size_t weights = (size_t)L.n * L.k;
        if (a.m >= 2 && weights < (a.m <= 4 ? ((size_t)4 << 20) : ((size_t)12 << 20))) return false;
    }
    if (P == 2)
        launch_rows<2>(L, a, s);
    else
        launch_rows<1>(L, a, s);
    return true;
}

}  // namespace trit
