// Prefill attention on the matrix cores (fast mode, f16 key/value caches):
// causal GQA over the caches after the prompt rows were appended
// (src/layers.rs:343-504 for the mathematics; the sums run in other orders,
// so the values are within rounding of the exact kernel's).
//
// Block (key/value head g, query tile qt) takes query rows
// [32 qt, 32 qt + 32) of every query head that shares g: wave 2 hl + half
// holds 16 rows of head g*GROUP + hl. Keys stream through LDS in tiles of
// 64 (K row-major, V transposed); per tile a wave makes its 16 x 64 scores
// with v_mfma_f32_16x16x32_f16 (q in f16, scaled by 1/sqrt(hd)), masks the
// keys past each row's position, updates the running max and sum
// (flash-attention rescaling, Trit's Cephes exp) and adds P.V, P through
// LDS in f16, with the same instruction. The output is O / sum in f32.
//
// Lane layouts of the 16x16x32 f16 instruction (checked on the device): an
// operand lane l holds row (or column) l % 16, elements 8 (l / 16) .. +7 of
// the 32-wide K step; result lane l holds column l % 16, rows 4 (l / 16) + r.
#include "decoder_impl.h"
#include "device.h"

namespace trit {
namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int HD = 128;
constexpr int QT = 32;      // query rows per block and head
constexpr int KT = 64;      // keys per tile
constexpr int KS = HD + 8;  // LDS row stride of K, in halves
constexpr int VS = KT + 8;  // LDS row stride of V^T
constexpr int PS = KT + 8;  // LDS row stride of P

template <int GROUP>
__global__ __launch_bounds__(GROUP * 128) void flash_prefill_kernel(const float* __restrict__ qkv, int stride,
                                                                    int rows, int pos0,
                                                                    const _Float16* __restrict__ kcache,
                                                                    const _Float16* __restrict__ vcache, int max_pos,
                                                                    float* __restrict__ out, int qd) {
    constexpr int NT = GROUP * 128;
    __shared__ __align__(16) _Float16 Ks[KT * KS];
    __shared__ __align__(16) _Float16 Vt[HD * VS];
    __shared__ __align__(16) _Float16 Ps[GROUP * 2][16 * PS];
    const int g = blockIdx.x, qt = blockIdx.y;
    const int t = threadIdx.x, w = t / WAVE, l = t % WAVE;
    const int hl = w / 2, half = w % 2, h = g * GROUP + hl;
    const int r0 = qt * QT + half * 16;  // the wave's first query row
    const int lr = l % 16, lq = l / 16;

    // Q fragments: row r0 + lr, dims 32 ks + 8 lq + i.
    const float scale = 1.0f / __builtin_sqrtf((float)HD);
    v8h qf[4];
    {
        const int row = r0 + lr;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f), b = a;
            if (row < rows) {
                const float* src = qkv + (size_t)row * stride + (size_t)h * HD + 32 * ks + 8 * lq;
                a = *(const float4*)src;
                b = *(const float4*)(src + 4);
            }
            qf[ks][0] = (_Float16)(a.x * scale);
            qf[ks][1] = (_Float16)(a.y * scale);
            qf[ks][2] = (_Float16)(a.z * scale);
            qf[ks][3] = (_Float16)(a.w * scale);
            qf[ks][4] = (_Float16)(b.x * scale);
            qf[ks][5] = (_Float16)(b.y * scale);
            qf[ks][6] = (_Float16)(b.z * scale);
            qf[ks][7] = (_Float16)(b.w * scale);
        }
    }

    // Running max and sum of rows 4 lq + r; output columns n*16 + lr.
    float m[4], lsum[4];
    v4f o[8];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        m[r] = -INFINITY;
        lsum[r] = 0.0f;
    }
#pragma unroll
    for (int n = 0; n < 8; ++n) o[n] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

    const int last_row = min(qt * QT + QT, rows) - 1;
    const int kend = pos0 + last_row + 1;  // keys the block's last row sees
    const int tiles = (kend + KT - 1) / KT;
    const _Float16* K = kcache + (size_t)g * max_pos * HD;
    const _Float16* V = vcache + (size_t)g * max_pos * HD;
    for (int kt = 0; kt < tiles; ++kt) {
        __syncthreads();  // the previous tile's K, V^T reads are done
        // K: 16 threads a key (coalesced 256-byte rows).
        for (int u = t; u < KT * HD / 8; u += NT) {
            const int key = u / (HD / 8), c8 = u % (HD / 8);
            const int j = kt * KT + key;
            const uint4 kv = *(const uint4*)(K + (size_t)(j < kend ? j : 0) * HD + c8 * 8);
            *(uint4*)(Ks + key * KS + c8 * 8) = kv;
        }
        // V^T: 64 threads a chunk column (consecutive keys write consecutive halves).
        for (int u = t; u < KT * HD / 8; u += NT) {
            const int key = u % KT, c8 = u / KT;
            const int j = kt * KT + key;
            const uint4 vv = *(const uint4*)(V + (size_t)(j < kend ? j : 0) * HD + c8 * 8);
            const uint32_t wds[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint16_t bits = (uint16_t)(wds[i >> 1] >> ((i & 1) * 16));
                Vt[(c8 * 8 + i) * VS + key] = __builtin_bit_cast(_Float16, bits);
            }
        }
        __syncthreads();

        // Scores: 4 key subtiles of 16.
        v4f s[4];
#pragma unroll
        for (int sub = 0; sub < 4; ++sub) {
            s[sub] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const v8h kb = *(const v8h*)(Ks + (sub * 16 + lr) * KS + 32 * ks + 8 * lq);
                s[sub] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qf[ks], kb, s[sub], 0, 0, 0);
            }
        }
        // Mask, running max, exp, running sum, rescale.
        float p[4][4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = r0 + 4 * lq + r;
            const int seen = row < rows ? pos0 + row : -1;  // last key the row sees
            float mt = -INFINITY;
#pragma unroll
            for (int sub = 0; sub < 4; ++sub) {
                const int key = kt * KT + sub * 16 + lr;
                if (key > seen) s[sub][r] = -INFINITY;
                mt = __builtin_fmaxf(mt, s[sub][r]);
            }
            mt = __builtin_fmaxf(mt, __shfl_xor(mt, 1));
            mt = __builtin_fmaxf(mt, __shfl_xor(mt, 2));
            mt = __builtin_fmaxf(mt, __shfl_xor(mt, 4));
            mt = __builtin_fmaxf(mt, __shfl_xor(mt, 8));
            const float mn = __builtin_fmaxf(m[r], mt);
            const float alpha = (m[r] == -INFINITY) ? 0.0f : exp_trit(m[r] - mn);
            float rs = 0.0f;
#pragma unroll
            for (int sub = 0; sub < 4; ++sub) {
                p[sub][r] = s[sub][r] == -INFINITY ? 0.0f : exp_trit(s[sub][r] - mn);
                rs += p[sub][r];
            }
            rs += __shfl_xor(rs, 1);
            rs += __shfl_xor(rs, 2);
            rs += __shfl_xor(rs, 4);
            rs += __shfl_xor(rs, 8);
            lsum[r] = __builtin_fmaf(lsum[r], alpha, rs);
            m[r] = mn;
#pragma unroll
            for (int n = 0; n < 8; ++n) o[n][r] *= alpha;
        }
        // P (16 x 64, f16) through this wave's LDS rows, read back as A fragments.
        _Float16* P = Ps[w];
#pragma unroll
        for (int sub = 0; sub < 4; ++sub)
#pragma unroll
            for (int r = 0; r < 4; ++r) P[(4 * lq + r) * PS + sub * 16 + lr] = (_Float16)p[sub][r];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const v8h pa = *(const v8h*)(P + lr * PS + 32 * ks + 8 * lq);
#pragma unroll
            for (int n = 0; n < 8; ++n) {
                const v8h vb = *(const v8h*)(Vt + (n * 16 + lr) * VS + 32 * ks + 8 * lq);
                o[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, vb, o[n], 0, 0, 0);
            }
        }
    }

#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int row = r0 + 4 * lq + r;
        if (row >= rows) continue;
        const float inv = 1.0f / lsum[r];
#pragma unroll
        for (int n = 0; n < 8; ++n) out[(size_t)row * qd + (size_t)h * HD + n * 16 + lr] = o[n][r] * inv;
    }
}

}  // namespace

bool flash_prefill_supported(const SessionImpl& S) {
    const auto& c = S.dec->c;
    if (S.exact || S.kv32 || c.head_dim != HD || c.heads % c.kv_heads) return false;
    const int group = c.heads / c.kv_heads;
    return group == 1 || group == 2 || group == 4;
}

void flash_prefill(SessionImpl& S, int layer, int rows, int pos0, hipStream_t s) {
    const auto& c = S.dec->c;
    const int group = c.heads / c.kv_heads, stride = (c.heads + 2 * c.kv_heads) * HD, qd = c.heads * HD;
    const _Float16* kc = S.kcache.as<_Float16>() + (size_t)layer * c.kv_heads * S.max_pos * HD;
    const _Float16* vc = S.vcache.as<_Float16>() + (size_t)layer * c.kv_heads * S.max_pos * HD;
    const dim3 grid(c.kv_heads, (rows + QT - 1) / QT);
    switch (group) {
        case 1:
            hipLaunchKernelGGL(flash_prefill_kernel<1>, grid, dim3(128), 0, s, S.qkv.as<float>(), stride, rows, pos0,
                               kc, vc, S.max_pos, S.att.as<float>(), qd);
            break;
        case 2:
            hipLaunchKernelGGL(flash_prefill_kernel<2>, grid, dim3(256), 0, s, S.qkv.as<float>(), stride, rows, pos0,
                               kc, vc, S.max_pos, S.att.as<float>(), qd);
            break;
        default:
            hipLaunchKernelGGL(flash_prefill_kernel<4>, grid, dim3(512), 0, s, S.qkv.as<float>(), stride, rows, pos0,
                               kc, vc, S.max_pos, S.att.as<float>(), qd);
            break;
    }
    TRIT_HIP(hipGetLastError());
}

}  // namespace trit
