// Prefill attention on the matrix cores (fast mode, f16 key/value caches):
// causal GQA over the caches after the prompt rows were appended
// (src/layers.rs:343-504 for the mathematics; the sums run in other orders
// and exp is the hardware exp2, so the values are within rounding of the
// exact kernel's).
//
// Block (key/value head g, query tile qt) takes query rows
// [32 qt, 32 qt + 32) of every query head that shares g: wave 2 hl + half
// holds 16 rows of head g*GROUP + hl. Keys stream through LDS in tiles of
// 64 (K row-major, V transposed), each tile loaded into registers while
// the previous one computes; the blocks with the longest causal rows start
// first.
//
// The wave works on transposed products, so that the probabilities never
// leave registers: S^T = K Q^T (v_mfma_f32_16x16x32_f16 with the keys as
// rows) gives lane l the scores of query l % 16 for keys 4 (l / 16) + r of
// each 16-key subtile; after the mask and the online softmax (running max
// and sum per query, q pre-scaled by log2(e) / sqrt(hd)) those values,
// converted to f16, are already the B operand of O^T = V^T P^T for a K
// step of 32 keys taken in the order
//   slot 8 j + i -> key 4 j + i (i < 4), 16 + 4 j + (i - 4) (i >= 4),
// and the A operand reads V^T rows in that same order (two 8-byte pieces).
// Lane l ends with O^T[16 n + 4 (l / 16) + r][query l % 16].
//
// The keys and values are f16 as cached, so only q and p are rounded to
// reach the f16 products: each is carried as two f16 parts, hi = f16(v)
// and lo = f16(v - hi), and each product runs twice (lo, then hi) into the
// f32 accumulator. The parts hold v to about 2^-22 of its size, so the
// scores and outputs are those of f32 q and p against the cached keys and
// values up to f32 rounding of the sums.
//
// Lane layouts of the 16x16x32 f16 instruction (checked on the device): an
// operand lane l holds row (or column) l % 16, elements 8 (l / 16) .. +7 of
// the 32-wide K step; result lane l holds column l % 16, rows 4 (l / 16) + r.
#include "decoder_impl.h"
#include "device.h"

namespace trit {
namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int HD = 128;
constexpr int QT = 32;      // query rows per block and head
constexpr int KT = 64;      // keys per tile
constexpr int KS = HD + 8;  // LDS row stride of K, in halves
constexpr int VS = KT + 8;  // LDS row stride of V^T

template <int GROUP>
__global__ __launch_bounds__(GROUP * 128) void flash_prefill_kernel(const float* __restrict__ qkv, int stride,
                                                                    int rows, int pos0,
                                                                    const _Float16* __restrict__ kcache,
                                                                    const _Float16* __restrict__ vcache, int max_pos,
                                                                    float* __restrict__ out, int qd, int tk_all) {
    constexpr int NT = GROUP * 128;
    constexpr int KP = KT * HD / 8;          // 16-byte pieces of a K tile
    constexpr int KPT = (KP + NT - 1) / NT;  // a thread's K pieces
    constexpr int VI = (KT / 4) * (HD / 8);  // V items: 4 keys x 8 dims
    constexpr int VPT = (VI + NT - 1) / NT;  // a thread's V items
    __shared__ __align__(16) _Float16 Ks[KT * KS];
    __shared__ __align__(16) _Float16 Vt[HD * VS];
    const int g = blockIdx.x, qt = gridDim.y - 1 - blockIdx.y;
    const int t = threadIdx.x, w = t / WAVE, l = t % WAVE;
    const int hl = w / 2, half = w % 2, h = g * GROUP + hl;
    const int r0 = qt * QT + half * 16;  // the wave's first query row
    const int lr = l % 16, lq = l / 16;
    const int row = r0 + lr;  // this lane's query
    // The last key it sees: causal, its own position; with tk_all > 0
    // (attention without a mask), every one of the tk_all keys.
    const int seen = row < rows ? (tk_all > 0 ? tk_all - 1 : pos0 + row) : -1;

    // Q^T fragments (B operand): query lr, dims 32 ks + 8 lq + i, scaled by
    // log2(e) / sqrt(hd) so that the scores are exp2 exponents.
    const float scale = 1.4426950408889634f / __builtin_sqrtf((float)HD);
    v8h qf[4], ql[4];  // hi and lo parts
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f), b = a;
        if (row < rows) {
            const float* src = qkv + (size_t)row * stride + (size_t)h * HD + 32 * ks + 8 * lq;
            a = *(const float4*)src;
            b = *(const float4*)(src + 4);
        }
        const float v[8] = {a.x * scale, a.y * scale, a.z * scale, a.w * scale,
                            b.x * scale, b.y * scale, b.z * scale, b.w * scale};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const _Float16 hi = (_Float16)v[i];
            qf[ks][i] = hi;
            ql[ks][i] = (_Float16)(v[i] - (float)hi);
        }
    }

    float m = -INFINITY, lsum = 0.0f;  // of query lr (the same in its 4 lanes)
    v4f o[8];                          // O^T rows 16 n + 4 lq + r, column lr
#pragma unroll
    for (int n = 0; n < 8; ++n) o[n] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

    const int last_row = min(qt * QT + QT, rows) - 1;
    const int kend = tk_all > 0 ? tk_all : pos0 + last_row + 1;  // keys the block's last row sees
    const int tiles = (kend + KT - 1) / KT;
    const _Float16* K = kcache + (size_t)g * max_pos * HD;
    const _Float16* V = vcache + (size_t)g * max_pos * HD;

    // Tile loads, one tile ahead: K piece u = key u / 16, dims 8 (u % 16)..;
    // V item u = keys 4 (u / 16) .. +3, dims 8 (u % 16) .. (keys past kend
    // read key 0: in bounds, masked in the scores).
    uint4 kr[KPT], vr[VPT][4];
#pragma unroll
    for (int i = 0; i < KPT; ++i) kr[i] = make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < VPT; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) vr[i][q] = make_uint4(0, 0, 0, 0);
#define TRIT_FETCH(KT_)                                                                                     \
    do {                                                                                                    \
        _Pragma("unroll") for (int i = 0; i < KPT; ++i) {                                                   \
            const int u = t + NT * i;                                                                       \
            if (u < KP) {                                                                                   \
                const int j = (KT_) * KT + u / (HD / 8);                                                    \
                kr[i] = *(const uint4*)(K + (size_t)(j < kend ? j : 0) * HD + (u % (HD / 8)) * 8);          \
            }                                                                                               \
        }                                                                                                   \
        _Pragma("unroll") for (int i = 0; i < VPT; ++i) {                                                   \
            const int u = t + NT * i;                                                                       \
            if (u < VI) {                                                                                   \
                _Pragma("unroll") for (int q = 0; q < 4; ++q) {                                             \
                    const int j = (KT_) * KT + 4 * (u / (HD / 8)) + q;                                      \
                    vr[i][q] = *(const uint4*)(V + (size_t)(j < kend ? j : 0) * HD + (u % (HD / 8)) * 8);   \
                }                                                                                           \
            }                                                                                               \
        }                                                                                                   \
    } while (0)

    TRIT_FETCH(0);
    for (int kt = 0; kt < tiles; ++kt) {
        __syncthreads();  // the previous tile's K, V^T reads are done
        // K row-major; V transposed: a thread's four keys' halves of dim d
        // go to Vt[d][4 kq ..] as one 8-byte store (halves paired by byte
        // perms: low halves of word d / 2 for even d, high for odd).
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int u = t + NT * i;
            if (u < KP) *(uint4*)(Ks + (u / (HD / 8)) * KS + (u % (HD / 8)) * 8) = kr[i];
        }
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int u = t + NT * i;
            if (u < VI) {
                const int kq = u / (HD / 8), c8 = u % (HD / 8);
                const uint32_t k0[4] = {vr[i][0].x, vr[i][0].y, vr[i][0].z, vr[i][0].w};
                const uint32_t k1[4] = {vr[i][1].x, vr[i][1].y, vr[i][1].z, vr[i][1].w};
                const uint32_t k2[4] = {vr[i][2].x, vr[i][2].y, vr[i][2].z, vr[i][2].w};
                const uint32_t k3[4] = {vr[i][3].x, vr[i][3].y, vr[i][3].z, vr[i][3].w};
#pragma unroll
                for (int d = 0; d < 8; ++d) {
                    const uint32_t sel = (d & 1) ? 0x07060302u : 0x05040100u;
                    uint2 v;
                    v.x = __builtin_amdgcn_perm(k1[d / 2], k0[d / 2], sel);
                    v.y = __builtin_amdgcn_perm(k3[d / 2], k2[d / 2], sel);
                    *(uint2*)(Vt + (c8 * 8 + d) * VS + 4 * kq) = v;
                }
            }
        }
        __syncthreads();
        if (kt + 1 < tiles) TRIT_FETCH(kt + 1);  // lands while this tile computes

        // S^T for 4 subtiles of 16 keys: lane holds keys 16 sub + 4 lq + r.
        v4f s[4];
#pragma unroll
        for (int sub = 0; sub < 4; ++sub) {
            s[sub] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const v8h ka = *(const v8h*)(Ks + (sub * 16 + lr) * KS + 32 * ks + 8 * lq);
                s[sub] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, ql[ks], s[sub], 0, 0, 0);
                s[sub] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qf[ks], s[sub], 0, 0, 0);
            }
        }
        // Mask, the tile's maximum for the query (its 16 values here, then
        // the lanes lr + 16 j), the running max and sum, rescale.
        float mt = -INFINITY;
#pragma unroll
        for (int sub = 0; sub < 4; ++sub)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int key = kt * KT + sub * 16 + 4 * lq + r;
                if (key > seen) s[sub][r] = -INFINITY;
                mt = __builtin_fmaxf(mt, s[sub][r]);
            }
        mt = __builtin_fmaxf(mt, __shfl_xor(mt, 16));
        mt = __builtin_fmaxf(mt, __shfl_xor(mt, 32));
        const float mn = __builtin_fmaxf(m, mt);
        const float alpha = __builtin_amdgcn_exp2f(m - mn);  // 0 on the first tile (m = -inf)
        float rs = 0.0f;
        v4h pk[4], pl[4];  // exp2(s - mn) as hi and lo f16 parts, per subtile
#pragma unroll
        for (int sub = 0; sub < 4; ++sub)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float p = __builtin_amdgcn_exp2f(s[sub][r] - mn);  // masked: exp2(-inf) = 0
                rs += p;
                const _Float16 hi = (_Float16)p;
                pk[sub][r] = hi;
                pl[sub][r] = (_Float16)(p - (float)hi);
            }
        rs += __shfl_xor(rs, 16);
        rs += __shfl_xor(rs, 32);
        lsum = __builtin_fmaf(lsum, alpha, rs);
        m = mn;
#pragma unroll
        for (int n = 0; n < 8; ++n) o[n] *= alpha;
        // O^T += V^T P^T over two K steps of 32 keys (subtiles 2c, 2c + 1).
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const v8h pb = {pk[2 * c][0], pk[2 * c][1], pk[2 * c][2], pk[2 * c][3],
                            pk[2 * c + 1][0], pk[2 * c + 1][1], pk[2 * c + 1][2], pk[2 * c + 1][3]};
            const v8h plb = {pl[2 * c][0], pl[2 * c][1], pl[2 * c][2], pl[2 * c][3],
                             pl[2 * c + 1][0], pl[2 * c + 1][1], pl[2 * c + 1][2], pl[2 * c + 1][3]};
#pragma unroll
            for (int n = 0; n < 8; ++n) {
                const _Float16* vrow = Vt + (n * 16 + lr) * VS + 32 * c + 4 * lq;
                const v4h lo = *(const v4h*)vrow, hi = *(const v4h*)(vrow + 16);
                const v8h va = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                o[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, plb, o[n], 0, 0, 0);
                o[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb, o[n], 0, 0, 0);
            }
        }
    }
#undef TRIT_FETCH

    if (row < rows) {
        const float inv = 1.0f / lsum;
        float* dst = out + (size_t)row * qd + (size_t)h * HD + 4 * lq;
#pragma unroll
        for (int n = 0; n < 8; ++n)
            *(float4*)(dst + 16 * n) = make_float4(o[n][0] * inv, o[n][1] * inv, o[n][2] * inv, o[n][3] * inv);
    }
}

}  // namespace

bool flash_prefill_supported(const SessionImpl& S) {
    const auto& c = S.dec->c;
    if (S.exact || S.kv32 || c.head_dim != HD || c.heads % c.kv_heads) return false;
    const int group = c.heads / c.kv_heads;
    return group == 1 || group == 2 || group == 4;
}

void flash_attention(const float* q, int qs, const _Float16* kc, const _Float16* vc, int max_pos, int heads,
                     int kv_heads, int rows, int pos0, int tk, int causal, float* out, hipStream_t s) {
    const int group = heads / kv_heads, qd = heads * HD, tk_all = causal ? 0 : tk;
    const dim3 grid(kv_heads, (rows + QT - 1) / QT);
    switch (group) {
        case 1:
            hipLaunchKernelGGL(flash_prefill_kernel<1>, grid, dim3(128), 0, s, q, qs, rows, pos0, kc, vc, max_pos, out,
                               qd, tk_all);
            break;
        case 2:
            hipLaunchKernelGGL(flash_prefill_kernel<2>, grid, dim3(256), 0, s, q, qs, rows, pos0, kc, vc, max_pos, out,
                               qd, tk_all);
            break;
        default:
            hipLaunchKernelGGL(flash_prefill_kernel<4>, grid, dim3(512), 0, s, q, qs, rows, pos0, kc, vc, max_pos, out,
                               qd, tk_all);
            break;
    }
    TRIT_HIP(hipGetLastError());
}

void flash_prefill(SessionImpl& S, int layer, int rows, int pos0, hipStream_t s) {
    const auto& c = S.dec->c;
    const int stride = (c.heads + 2 * c.kv_heads) * HD;
    const _Float16* kc = S.kcache.as<_Float16>() + (size_t)layer * c.kv_heads * S.max_pos * HD;
    const _Float16* vc = S.vcache.as<_Float16>() + (size_t)layer * c.kv_heads * S.max_pos * HD;
    flash_attention(S.qkv.as<float>(), stride, kc, vc, S.max_pos, c.heads, c.kv_heads, rows, pos0, pos0 + rows, 1,
                    S.att.as<float>(), s);
}

}  // namespace trit
