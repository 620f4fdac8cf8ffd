// The audio encoder of Whisper, which Voxtral and MOSS run too
// (src/models/parts/audio_encoder.rs:1-138): a conv stem (kernel 3, stride
// 1 then 2, each with GELU) as im2col + product, learned positions,
// pre-norm layers (stacked q/k/v, attention with no mask, an exact-GELU
// MLP), a final layer norm. The prefill before the decoder: every product
// of more than 8 rows runs on the matrix cores (Q8_0, Q4_K, int8 with the
// shapes they take; other kinds and shapes in launches of 8 rows), the
// same bits as the small-batch kernels; layer norm in Trit's 32-lane order,
// the exact GELU, Trit's attention.
#include <algorithm>
#include <cstring>

#include "../../include/trit_hip.h"
#include "decoder_impl.h"
#include "device.h"
#include "internal.h"

namespace trit {
namespace {

constexpr float NORM_EPS = 1e-5f;  // Norm::load (src/layers.rs:6,29-40)

// conv_columns (src/layers.rs:613-634): row t of `out` holds x[t*stride +
// tap - pad][c] at c*kernel + tap; zero outside the frames.
__global__ void im2col_kernel(const float* __restrict__ x, int frames, int channels, int kernel, int stride, int pad,
                              int out_frames, float* __restrict__ out) {
    const size_t total = (size_t)out_frames * channels * kernel;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        const int tap = (int)(i % kernel);
        const size_t tc = i / kernel;
        const int c = (int)(tc % channels);
        const int t = (int)(tc / channels);
        const int src = t * stride + tap - pad;
        out[i] = src >= 0 && src < frames ? x[(size_t)src * channels + c] : 0.0f;
    }
}

__global__ void gelu_kernel(float* __restrict__ x, size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        x[i] = gelu_trit(x[i]);
}

__global__ void add_kernel(float* __restrict__ x, const float* __restrict__ y, size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        x[i] = x[i] + y[i];
}

// Norm::apply (src/layers.rs:50-64,84-121), one 64-lane wave a row: lane j
// < 32 chains the values j, j + 32, ... of the mean's (then the
// variance's) sum; lane 0 adds the 32 lane sums in order and then the
// tail; out = (v - mean) * inv * w + b.
__global__ __launch_bounds__(64) void layer_norm_kernel(const float* __restrict__ x, int d, const float* __restrict__ w,
                                                        const float* __restrict__ b, float eps, float* __restrict__ out) {
    __shared__ float lanes[32];
    __shared__ float stat[2];
    const float* row = x + (size_t)blockIdx.x * d;
    const int lane = threadIdx.x;
    const int whole = d / 32 * 32;
    const float n = (float)d;
    for (int pass = 0; pass < 2; ++pass) {
        const float mean = pass ? stat[0] : 0.0f;
        if (lane < 32) {
            float acc = 0.0f;
            for (int i = lane; i < whole; i += 32) {
                const float v = row[i];
                acc += pass ? (v - mean) * (v - mean) : v;
            }
            lanes[lane] = acc;
        }
        __syncthreads();
        if (lane == 0) {
            float s = 0.0f;
            for (int j = 0; j < 32; ++j) s += lanes[j];
            float t = 0.0f;
            for (int i = whole; i < d; ++i) {
                const float v = row[i];
                t += pass ? (v - mean) * (v - mean) : v;
            }
            stat[pass] = (s + t) / n;
        }
        __syncthreads();
    }
    const float mean = stat[0];
    const float inv = 1.0f / __builtin_sqrtf(stat[1] + eps);
    float* o = out + (size_t)blockIdx.x * d;
    for (int i = lane; i < d; i += 64) o[i] = (row[i] - mean) * inv * w[i] + b[i];
}

int blocks_for(size_t n) { return (int)std::min<size_t>((n + 255) / 256, 4096); }

}  // namespace

struct EncoderImpl {
    TritHipEncoderConfig c{};
    LayerRef conv1, conv2;
    std::vector<LayerRef> layers;  // qkv, out, fc1, fc2 per layer
    DeviceMemory positions;        // positions x d
    DeviceMemory norms;            // per layer: attn w, b, ffn w, b (d each); then final w, b
    const float* norm(int l, int i) const { return norms.as<float>() + ((size_t)4 * l + i) * c.d; }
};

}  // namespace trit

struct TritHipEncoder {
    trit::EncoderImpl impl;
};

using namespace trit;

namespace {

// x W^T (+ bias) of m rows into y (+ residual): the matrix cores for more
// than 8 rows where the layer allows it, else launches of up to 8 rows.
void encoder_product(const Layer& L, const float* x, int m, float* y, const float* residual, DeviceMemory& scratch,
                     hipStream_t s) {
    GemvArgs a;
    a.x = x;
    a.y = y;
    a.m = m;
    if (residual) {
        a.residual = residual;
        a.epilogue = EPI_RESIDUAL;
    }
    if (m > 8 && gemm_supported(L, a)) {
        const size_t need = gemm_scratch_bytes(m, L.k);
        if (scratch.bytes < need) scratch.alloc(need);
        return gemm_int(L, a, scratch.ptr, s);
    }
    if (!float_kind(L.kind)) {
        const size_t need = gemv_scratch_bytes(8, L.k);
        if (scratch.bytes < need) scratch.alloc(need);
        a.scratch = scratch.ptr;
        a.scratch_bytes = scratch.bytes;
    }
    for (int r0 = 0; r0 < m; r0 += 8) {
        GemvArgs b = a;
        b.m = m - r0 < 8 ? m - r0 : 8;
        b.x = x + (size_t)r0 * L.k;
        b.y = y + (size_t)r0 * L.n;
        if (residual) b.residual = residual + (size_t)r0 * L.n;
        layer_forward(L, b, s);
    }
}

}  // namespace

extern "C" {

int trit_hip_encoder_new(const TritHipEncoderConfig* config, const TritHipLayer* conv1, const TritHipLayer* conv2,
                         const float* positions, const TritHipLayer* const* linears, const float* norms,
                         TritHipEncoder** out) {
    return guard(-1, [&] {
        if (!config || !conv1 || !conv2 || !positions || !linears || !norms || !out)
            fail("encoder: a required argument is NULL");
        const TritHipEncoderConfig& c = *config;
        if (c.d <= 0 || c.layers <= 0 || c.heads <= 0 || c.ffn <= 0 || c.mels <= 0 || c.positions <= 0)
            fail("encoder: a size is not positive");
        if (c.d % c.heads) fail("encoder: d is not a multiple of the heads");
        const int hd = c.d / c.heads;
        if (hd % 8 || hd > 256) fail("encoder: head_dim must be a multiple of 8 and at most 256");
        auto want = [&](const TritHipLayer* h, int n, int k, const std::string& what) {
            LayerRef L = layer_ref(h);
            if (!L) fail("encoder: " + what + " is NULL");
            if (L->n != n || L->k != k)
                fail("encoder: " + what + " is " + std::to_string(L->n) + "x" + std::to_string(L->k) + ", expected " +
                     std::to_string(n) + "x" + std::to_string(k));
            return L;
        };
        auto* E = new TritHipEncoder();
        try {
            EncoderImpl& e = E->impl;
            e.c = c;
            e.conv1 = want(conv1, c.d, 3 * c.mels, "conv1");
            e.conv2 = want(conv2, c.d, 3 * c.d, "conv2");
            for (int l = 0; l < c.layers; ++l) {
                const std::string p = "layer " + std::to_string(l) + " ";
                e.layers.push_back(want(linears[4 * l], 3 * c.d, c.d, p + "qkv"));
                e.layers.push_back(want(linears[4 * l + 1], c.d, c.d, p + "out"));
                e.layers.push_back(want(linears[4 * l + 2], c.ffn, c.d, p + "fc1"));
                e.layers.push_back(want(linears[4 * l + 3], c.d, c.ffn, p + "fc2"));
            }
            e.positions.alloc((size_t)c.positions * c.d * 4);
            e.positions.upload(positions, (size_t)c.positions * c.d * 4);
            const size_t nb = ((size_t)4 * c.layers + 2) * c.d * 4;
            e.norms.alloc(nb);
            e.norms.upload(norms, nb);
        } catch (...) {
            delete E;
            throw;
        }
        *out = E;
        return 0;
    });
}

void trit_hip_encoder_free(TritHipEncoder* encoder) { delete encoder; }

int trit_hip_encoder_encode(const TritHipEncoder* encoder, const float* mel, float* out) {
    return guard(-1, [&] {
        if (!encoder || !mel || !out) fail("encoder: encoder, mel or out is NULL");
        const EncoderImpl& e = encoder->impl;
        const auto& c = e.c;
        const int P = c.positions, frames = 2 * P, d = c.d, hd = d / c.heads;
        hipStream_t s = stream();
        DeviceMemory dmel((size_t)frames * c.mels * 4), cols((size_t)frames * 3 * std::max(c.mels, d) * 4);
        DeviceMemory h((size_t)frames * d * 4), x((size_t)P * d * 4), xn((size_t)P * d * 4);
        DeviceMemory qkv((size_t)P * 3 * d * 4), att((size_t)P * d * 4), hid((size_t)P * c.ffn * 4);
        DeviceMemory kc((size_t)P * d * 4), vc((size_t)P * d * 4), st(sizeof(State)), scratch;
        TRIT_HIP(hipMemcpyAsync(dmel.ptr, mel, dmel.bytes, hipMemcpyHostToDevice, s));
        State h0{};  // pos = tk - tq = 0: every query sees every key (no mask)
        TRIT_HIP(hipMemcpyAsync(st.ptr, &h0, sizeof(State), hipMemcpyHostToDevice, s));
        // The stem (audio_encoder.rs:116-123).
        size_t n = (size_t)frames * c.mels * 3;
        hipLaunchKernelGGL(im2col_kernel, dim3(blocks_for(n)), dim3(256), 0, s, dmel.as<float>(), frames, c.mels, 3, 1,
                           1, frames, cols.as<float>());
        encoder_product(*e.conv1, cols.as<float>(), frames, h.as<float>(), nullptr, scratch, s);
        hipLaunchKernelGGL(gelu_kernel, dim3(blocks_for((size_t)frames * d)), dim3(256), 0, s, h.as<float>(),
                           (size_t)frames * d);
        n = (size_t)P * d * 3;
        hipLaunchKernelGGL(im2col_kernel, dim3(blocks_for(n)), dim3(256), 0, s, h.as<float>(), frames, d, 3, 2, 1, P,
                           cols.as<float>());
        encoder_product(*e.conv2, cols.as<float>(), P, x.as<float>(), nullptr, scratch, s);
        hipLaunchKernelGGL(gelu_kernel, dim3(blocks_for((size_t)P * d)), dim3(256), 0, s, x.as<float>(),
                           (size_t)P * d);
        hipLaunchKernelGGL(add_kernel, dim3(blocks_for((size_t)P * d)), dim3(256), 0, s, x.as<float>(),
                           e.positions.as<float>(), (size_t)P * d);
        // The layers (audio_encoder.rs:124-136).
        for (int l = 0; l < c.layers; ++l) {
            const Layer& Lqkv = *e.layers[4 * l];
            const Layer& Lout = *e.layers[4 * l + 1];
            const Layer& Lfc1 = *e.layers[4 * l + 2];
            const Layer& Lfc2 = *e.layers[4 * l + 3];
            hipLaunchKernelGGL(layer_norm_kernel, dim3(P), dim3(64), 0, s, x.as<float>(), d, e.norm(l, 0),
                               e.norm(l, 1), NORM_EPS, xn.as<float>());
            encoder_product(Lqkv, xn.as<float>(), P, qkv.as<float>(), nullptr, scratch, s);
            exact_attention(qkv.as<float>(), 3 * d, qkv.as<float>() + d, qkv.as<float>() + 2 * d, 3 * d, P, P, c.heads,
                            c.heads, hd, 0, att.as<float>(), kc.as<float>(), vc.as<float>(), st.as<State>(), s);
            encoder_product(Lout, att.as<float>(), P, x.as<float>(), x.as<float>(), scratch, s);
            hipLaunchKernelGGL(layer_norm_kernel, dim3(P), dim3(64), 0, s, x.as<float>(), d, e.norm(l, 2),
                               e.norm(l, 3), NORM_EPS, xn.as<float>());
            encoder_product(Lfc1, xn.as<float>(), P, hid.as<float>(), nullptr, scratch, s);
            hipLaunchKernelGGL(gelu_kernel, dim3(blocks_for((size_t)P * c.ffn)), dim3(256), 0, s, hid.as<float>(),
                               (size_t)P * c.ffn);
            encoder_product(Lfc2, hid.as<float>(), P, x.as<float>(), x.as<float>(), scratch, s);
        }
        hipLaunchKernelGGL(layer_norm_kernel, dim3(P), dim3(64), 0, s, x.as<float>(), d, e.norm(c.layers, 0),
                           e.norm(c.layers, 1), NORM_EPS, xn.as<float>());
        TRIT_HIP(hipGetLastError());
        TRIT_HIP(hipMemcpyAsync(out, xn.ptr, (size_t)P * d * 4, hipMemcpyDeviceToHost, s));
        TRIT_HIP(hipStreamSynchronize(s));
        return 0;
    });
}

}  // extern "C"
