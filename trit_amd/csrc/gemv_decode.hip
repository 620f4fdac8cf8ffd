// Q8_0 GEMV for one decode row (m = 1), k in {1024, 2048, 3072}.
//
// Same values as the general kernel (gemv.hip), bit for bit: exact i32
// block dots and Trit's f32 chain total = fma(f32(dot_g), ws_g * xs_g,
// total) over the groups in order (src/cpu/int8.rs:525-584).
//
// One wave per block, four rows per wave, sixteen lanes per row. Lane l of
// a row streams chunks l, l+16, l+32, ... (16 bytes each, so every load
// instruction reads 256 contiguous bytes of the row) and keeps the matching
// activation codes in registers. A DPP swap adds the two halves of each
// 32-value block, leaving block g = l/2 + 8j in even lane l. The f32 chain
// is then a systolic pass: at step t the running total moves two lanes
// (row_ror:2) and the lane that holds block t folds it in, so the chain
// visits blocks 0, 1, 2, ... in order without leaving registers.
//
// The prologue (RMSNorm, Trit's activation quantizer) runs once per wave
// into LDS while the weight loads are in flight; its reductions are DPP
// moves in a fixed order, so every block gets the same bits.
#include "device.h"
#include "internal.h"

namespace trit {
namespace {

constexpr int LANES = 64;

template <int J, int P>  // J = k / 256 chunks per lane; P = 2: SwiGLU pair
__global__ __launch_bounds__(LANES) void gemv_row_kernel(const uint8_t* __restrict__ codes,
                                                         const uint16_t* __restrict__ scales,
                                                         const float* __restrict__ bias, int n, GemvArgs a) {
    constexpr int K = J * 256;
    constexpr int G = K / 32;
    __shared__ __align__(16) int8_t xq[K];
    __shared__ float xs[G];
    if (a.skip && *a.skip) return;
    const int lane = threadIdx.x;
    const int l = lane & 15;
    const int part_rows = n / P;
    const int row = blockIdx.x * 4 + (lane >> 4);

    // Weights and scales first: their latency overlaps the prologue.
    uint4 w[P][J];
    float ws[P][J];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const uint8_t* src = codes + (size_t)(p * part_rows + row) * K;
#pragma unroll
        for (int j = 0; j < J; ++j) w[p][j] = load_stream(src + (size_t)(l + 16 * j) * 16);
        const uint16_t* sc = scales + (size_t)(p * part_rows + row) * G + (l >> 1);
#pragma unroll
        for (int j = 0; j < J; ++j) ws[p][j] = f16_to_f32(sc[8 * j]);
    }

    // Prologue: x (and the RMSNorm factor), then Trit's quantizer, into LDS.
    float4 xv[J];
#pragma unroll
    for (int i = 0; i < J; ++i) xv[i] = *(const float4*)(a.x + (size_t)(lane + LANES * i) * 4);
    float inv = 0.0f;
    if (a.norm_w) {
        if (a.norm_inv) {
            inv = a.norm_inv[0];
        } else {
            float part = 0.0f;
#pragma unroll
            for (int i = 0; i < J; ++i)
                part += (xv[i].x * xv[i].x + xv[i].y * xv[i].y) + (xv[i].z * xv[i].z + xv[i].w * xv[i].w);
            part += dpp<DPP_XOR1>(part);
            part += dpp<DPP_XOR2>(part);
            part += dpp<DPP_HALF_MIRROR>(part);
            part += dpp<DPP_MIRROR>(part);
            const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, part), 0));
            const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, part), 16));
            const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, part), 32));
            const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, part), 48));
            const float sum = ((r0 + r1) + r2) + r3;
            inv = 1.0f / __builtin_sqrtf(sum / (float)K + a.eps);
        }
    }
#pragma unroll
    for (int i = 0; i < J; ++i) {
        const int item = lane + LANES * i;
        float4 v = xv[i];
        if (a.norm_w) {
            const float4 nw = *(const float4*)(a.norm_w + item * 4);
            v.x = v.x * (inv * nw.x);
            v.y = v.y * (inv * nw.y);
            v.z = v.z * (inv * nw.z);
            v.w = v.w * (inv * nw.w);
        }
        float peak = __builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(v.x), __builtin_fabsf(v.y)),
                                     __builtin_fmaxf(__builtin_fabsf(v.z), __builtin_fabsf(v.w)));
        peak = __builtin_fmaxf(peak, dpp<DPP_XOR1>(peak));
        peak = __builtin_fmaxf(peak, dpp<DPP_XOR2>(peak));
        peak = __builtin_fmaxf(peak, dpp<DPP_HALF_MIRROR>(peak));
        const float scale = peak > 0.0f ? peak / 127.0f : 1.0f;
        const float q = 1.0f / scale;
        *(uint32_t*)(xq + item * 4) = pack4(act_code(v.x * q), act_code(v.y * q), act_code(v.z * q), act_code(v.w * q));
        if ((item & 7) == 0) xs[item >> 3] = f16_round(scale);
    }
    __syncthreads();

    // Dots: lane l, chunk c = l + 16j; the block's two halves meet by DPP.
    float df[P][J], sc[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const uint4 xc = *(const uint4*)(xq + (l + 16 * j) * 16);
        sc[j] = xs[(l >> 1) + 8 * j];
#pragma unroll
        for (int p = 0; p < P; ++p) {
            int d = sdot4(w[p][j].x, xc.x, 0);
            d = sdot4(w[p][j].y, xc.y, d);
            d = sdot4(w[p][j].z, xc.z, d);
            d = sdot4(w[p][j].w, xc.w, d);
            d += dpp<DPP_XOR1>(d);
            df[p][j] = (float)d;
        }
    }
    float prod[P][J];
#pragma unroll
    for (int p = 0; p < P; ++p)
#pragma unroll
        for (int j = 0; j < J; ++j) prod[p][j] = ws[p][j] * sc[j];

    // The chain: block t = 8j + q lives in lane 2q, step j.
    float acc[P];
#pragma unroll
    for (int p = 0; p < P; ++p) acc[p] = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
#pragma unroll
            for (int p = 0; p < P; ++p) {
                const float in = (j == 0 && q == 0) ? 0.0f : dpp<DPP_ROR2>(acc[p]);
                acc[p] = __builtin_fmaf(df[p][j], prod[p][j], in);
            }
        }
    }
    // Lane 14 of each row holds the last block's total.
    if (l == 14) {
        float y = acc[0];
        if (P == 2) {
            a.y[row] = silu_trit(acc[0]) * acc[1];
            return;
        }
        if (bias) y = y + bias[row];
        if (a.relu) y = __builtin_fmaxf(y, 0.0f);
        a.y[row] = a.epilogue == EPI_RESIDUAL ? a.residual[row] + y : y;
    }
}

template <int J>
void launch_row(const Layer& L, const GemvArgs& a, hipStream_t s) {
    const int P = a.epilogue == EPI_SILU_PAIR ? 2 : 1;
    const int blocks = L.n / P / 4;
    const uint8_t* c = L.codes.as<uint8_t>();
    const uint16_t* sc = L.scales.as<uint16_t>();
    const float* b = L.bias.as<float>();
    if (P == 2)
        launch_timed(a, gemv_row_kernel<J, 2>, dim3(blocks), dim3(LANES), 0, s, c, sc, b, L.n, a);
    else
        launch_timed(a, gemv_row_kernel<J, 1>, dim3(blocks), dim3(LANES), 0, s, c, sc, b, L.n, a);
    TRIT_HIP(hipGetLastError());
}

}  // namespace

bool gemv_row(const Layer& L, const GemvArgs& a, hipStream_t s) {
    if (a.m != 1 || (L.kind != Q8_0 && L.kind != Q4_K)) return false;
    const int P = a.epilogue == EPI_SILU_PAIR ? 2 : 1;
    if ((L.n / P) % 4 != 0) return false;
    if (P == 2 && L.bias.ptr) return false;
    switch (L.k) {
        case 1024: launch_row<4>(L, a, s); return true;
        case 2048: launch_row<8>(L, a, s); return true;
        case 3072: launch_row<12>(L, a, s); return true;
        default: return false;
    }
}

}  // namespace trit
