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
#include <cmath>
#include <cstring>
#include <mutex>

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

// AudioEncoder::chunk's first map (src/models/families/qwen3_asr.rs:
// 391-398), for every chunk at once: map c is [bin][time] (one channel) of
// the frames c * chunk + time, zero past the chunk's own length and out to
// `longest` time steps (every chunk padded to the longest).
__global__ void mel_maps_kernel(const float* __restrict__ mel, int frames, int mels, int chunk, int maps, int longest,
                                float* __restrict__ out) {
    const size_t total = (size_t)maps * mels * longest;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        const int time = (int)(i % longest);
        const size_t rest = i / longest;
        const int bin = (int)(rest % mels);
        const int f = (int)(rest / mels) * chunk + time;
        out[i] = f < frames ? mel[(size_t)f * mels + bin] : 0.0f;
    }
}

// conv2d's im2col (qwen3_asr.rs:408-428) over `maps` [bin][time][channel]
// maps laid end to end: row (map, bin', time') holds map[2 bin' + dy -
// 1][2 time' + dx - 1][c] at column c * 9 + 3 dy + dx, zero outside.
__global__ void conv2d_columns_kernel(const float* __restrict__ in, int maps, int bins, int times, int channels,
                                      float* __restrict__ out) {
    const int ob = (bins + 1) / 2, ot = (times + 1) / 2;
    const size_t total = (size_t)maps * ob * ot * channels * 9;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        const int tap = (int)(i % 9);
        const size_t rest = i / 9;
        const int c = (int)(rest % channels);
        const size_t pos = rest / channels;
        const int x = (int)(pos % ot), y = (int)(pos / ot % ob);
        const size_t map = pos / ((size_t)ot * ob);
        const int sy = 2 * y + tap / 3 - 1, sx = 2 * x + tap % 3 - 1;
        out[i] = sy >= 0 && sy < bins && sx >= 0 && sx < times
                     ? in[((map * bins + sy) * times + sx) * channels + c]
                     : 0.0f;
    }
}

// Per time step the channel-major columns (qwen3_asr.rs:380-388): row
// (map, time) of the first `rows` holds map[bin][time][c] at c * bins + bin.
__global__ void time_columns_kernel(const float* __restrict__ in, int bins, int times, int channels, int rows,
                                    float* __restrict__ out) {
    const size_t total = (size_t)rows * channels * bins;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        const int bin = (int)(i % bins);
        const size_t rest = i / bins;
        const int c = (int)(rest % channels);
        const size_t r = rest / channels;
        const size_t map = r / times;
        const int t = (int)(r % times);
        out[i] = in[((map * bins + bin) * times + t) * channels + c];
    }
}

// x[r] += positions[r % times]: each chunk's rows take the table from row 0.
__global__ void add_positions_kernel(float* __restrict__ x, const float* __restrict__ pos, int rows, int times,
                                     int d) {
    const size_t total = (size_t)rows * d;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        const size_t r = i / d;
        x[i] = x[i] + pos[(r % times) * d + i % d];
    }
}

int blocks_for(size_t n) { return (int)std::min<size_t>((n + 255) / 256, 4096); }

}  // namespace

// Device buffers an encoder keeps between calls, grown on demand: an
// encode allocates only when it needs more than the calls before it. Calls
// on one encoder take turns (the mutex); the buffers are the encoder's
// until it is freed.
struct Workspace {
    std::mutex mu;
    DeviceMemory bufs[16];
    DeviceMemory& get(int i, size_t bytes) {
        if (bufs[i].bytes < bytes) bufs[i].alloc(bytes);
        return bufs[i];
    }
};

struct EncoderImpl {
    TritHipEncoderConfig c{};
    LayerRef conv1, conv2;
    std::vector<LayerRef> layers;  // qkv, out, fc1, fc2 per layer
    DeviceMemory positions;        // positions x d
    DeviceMemory norms;            // per layer: attn w, b, ffn w, b (d each); then final w, b
    const float* norm(int l, int i) const { return norms.as<float>() + ((size_t)4 * l + i) * c.d; }
    mutable Workspace ws;
};

struct AsrEncoderImpl {
    TritHipAsrEncoderConfig c{};
    LayerRef convs[3], conv_out, proj1, proj2;
    std::vector<LayerRef> layers;  // qkv, out, fc1, fc2 per layer
    DeviceMemory positions;        // max_positions x d
    DeviceMemory norms;            // per layer: attn w, b, ffn w, b (d each); then ln_post w, b
    const float* norm(int l, int i) const { return norms.as<float>() + ((size_t)4 * l + i) * c.d; }
    mutable Workspace ws;
};

// Length after a kernel-3, stride-2, padding-1 convolution (qwen3_asr.rs:
// 120-123), and after three.
int half_len(int n) { return (n + 1) / 2; }
int half3(int n) { return half_len(half_len(half_len(n))); }

}  // namespace trit

struct TritHipEncoder {
    trit::EncoderImpl impl;
};

struct TritHipAsrEncoder {
    trit::AsrEncoderImpl impl;
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
    if (m > 8 && gemm_float_supported(L, a)) return gemm_float(L, a, s);
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

// sinusoids (src/layers.rs:257-270): row p is [sin | cos] of (first + p)
// * exp(-i * ln_timescale / (d/2 - 1)), times scale, in double with the C
// library's exp, sin and cos (the calls Rust's f64 methods make on Linux),
// rounded to f32.
std::vector<float> sinusoids(int rows, int d, int first, double ln_timescale, double scale) {
    double (*volatile f_exp)(double) = exp;
    double (*volatile f_sin)(double) = sin;
    double (*volatile f_cos)(double) = cos;
    const int half = d / 2;
    const double inc = ln_timescale / ((double)half - 1.0);
    std::vector<float> t((size_t)rows * d, 0.0f);
    for (int p = 0; p < rows; ++p) {
        const double pos = (double)(first + p);
        for (int i = 0; i < half; ++i) {
            const double angle = pos * f_exp(-inc * (double)i);
            t[(size_t)p * d + i] = (float)(f_sin(angle) * scale);
            t[(size_t)p * d + half + i] = (float)(f_cos(angle) * scale);
        }
    }
    return t;
}

// The rows a Qwen3-ASR encoder makes of `frames` mel frames: half^3 of
// each chunk's length.
int asr_rows(const TritHipAsrEncoderConfig& c, int frames) {
    int rows = 0;
    for (int s = 0; s < frames; s += c.chunk) rows += half3(std::min(c.chunk, frames - s));
    return rows;
}

LayerRef want_layer(const TritHipLayer* h, int n, int k, const std::string& what) {
    LayerRef L = layer_ref(h);
    if (!L) fail("encoder: " + what + " is NULL");
    if (L->n != n || L->k != k)
        fail("encoder: " + what + " is " + std::to_string(L->n) + "x" + std::to_string(L->k) + ", expected " +
             std::to_string(n) + "x" + std::to_string(k));
    return L;
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
        std::lock_guard<std::mutex> lock(e.ws.mu);
        Workspace& ws = e.ws;
        DeviceMemory& dmel = ws.get(0, (size_t)frames * c.mels * 4);
        DeviceMemory& cols = ws.get(1, (size_t)frames * 3 * std::max(c.mels, d) * 4);
        DeviceMemory& h = ws.get(2, (size_t)frames * d * 4);
        DeviceMemory& x = ws.get(3, (size_t)P * d * 4);
        DeviceMemory& xn = ws.get(4, (size_t)P * d * 4);
        DeviceMemory& qkv = ws.get(5, (size_t)P * 3 * d * 4);
        DeviceMemory& att = ws.get(6, (size_t)P * d * 4);
        DeviceMemory& hid = ws.get(7, (size_t)P * c.ffn * 4);
        DeviceMemory& kc = ws.get(8, (size_t)P * d * 4);
        DeviceMemory& vc = ws.get(9, (size_t)P * d * 4);
        DeviceMemory& st = ws.get(10, sizeof(State));
        DeviceMemory& scratch = ws.bufs[11];
        TRIT_HIP(hipMemcpyAsync(dmel.ptr, mel, (size_t)frames * c.mels * 4, hipMemcpyHostToDevice, s));
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

int trit_hip_asr_encoder_new(const TritHipAsrEncoderConfig* config, const TritHipLayer* const* convs,
                             const TritHipLayer* conv_out, const TritHipLayer* const* linears, const float* norms,
                             const TritHipLayer* proj1, const TritHipLayer* proj2, TritHipAsrEncoder** out) {
    return guard(-1, [&] {
        if (!config || !convs || !conv_out || !linears || !norms || !proj1 || !proj2 || !out)
            fail("asr encoder: a required argument is NULL");
        const TritHipAsrEncoderConfig& c = *config;
        if (c.d <= 0 || c.layers <= 0 || c.heads <= 0 || c.ffn <= 0 || c.mels <= 0 || c.channels <= 0 ||
            c.chunk <= 0 || c.window_chunks <= 0 || c.out <= 0 || c.max_positions <= 0)
            fail("asr encoder: a size is not positive");
        if (c.d % c.heads) fail("asr encoder: d is not a multiple of the heads");
        const int hd = c.d / c.heads;
        if (hd % 8 || hd > 256) fail("asr encoder: head_dim must be a multiple of 8 and at most 256");
        if (c.d % 2 || c.d < 4) fail("asr encoder: d must be even and at least 4 (the sinusoid table)");
        if (half3(c.chunk) > c.max_positions) fail("asr encoder: a chunk makes more rows than max_positions");
        auto* E = new TritHipAsrEncoder();
        try {
            AsrEncoderImpl& e = E->impl;
            e.c = c;
            e.convs[0] = want_layer(convs[0], c.channels, 9, "conv2d1");
            e.convs[1] = want_layer(convs[1], c.channels, 9 * c.channels, "conv2d2");
            e.convs[2] = want_layer(convs[2], c.channels, 9 * c.channels, "conv2d3");
            e.conv_out = want_layer(conv_out, c.d, c.channels * half3(c.mels), "conv_out");
            for (int l = 0; l < c.layers; ++l) {
                const std::string p = "layer " + std::to_string(l) + " ";
                e.layers.push_back(want_layer(linears[4 * l], 3 * c.d, c.d, p + "qkv"));
                e.layers.push_back(want_layer(linears[4 * l + 1], c.d, c.d, p + "out"));
                e.layers.push_back(want_layer(linears[4 * l + 2], c.ffn, c.d, p + "fc1"));
                e.layers.push_back(want_layer(linears[4 * l + 3], c.d, c.ffn, p + "fc2"));
            }
            e.proj1 = want_layer(proj1, c.d, c.d, "proj1");
            e.proj2 = want_layer(proj2, c.out, c.d, "proj2");
            const std::vector<float> table = sinusoids(c.max_positions, c.d, 0, log(10000.0), 1.0);
            e.positions.alloc(table.size() * 4);
            e.positions.upload(table.data(), table.size() * 4);
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

void trit_hip_asr_encoder_free(TritHipAsrEncoder* encoder) { delete encoder; }

int trit_hip_asr_encoder_rows(const TritHipAsrEncoder* encoder, int frames) {
    return guard(-1, [&] {
        if (!encoder) fail("asr encoder: encoder is NULL");
        if (frames <= 0) fail("asr encoder: frames must be positive");
        return asr_rows(encoder->impl.c, frames);
    });
}

int trit_hip_asr_encoder_positions(const TritHipAsrEncoder* encoder, float* out) {
    return guard(-1, [&] {
        if (!encoder || !out) fail("asr encoder: encoder or out is NULL");
        const auto& e = encoder->impl;
        TRIT_HIP(hipMemcpy(out, e.positions.ptr, e.positions.bytes, hipMemcpyDeviceToHost));
        return 0;
    });
}

int trit_hip_asr_encoder_encode(const TritHipAsrEncoder* encoder, const float* mel, int frames, float* out) {
    return guard(-1, [&] {
        if (!encoder || !mel || !out) fail("asr encoder: encoder, mel or out is NULL");
        if (frames <= 0) fail("asr encoder: frames must be positive");
        const AsrEncoderImpl& e = encoder->impl;
        const auto& c = e.c;
        const int d = c.d, hd = d / c.heads, ch = c.channels;
        const int maps = (frames + c.chunk - 1) / c.chunk;
        const int longest = std::min(c.chunk, frames);
        const int t = asr_rows(c, frames);
        // The convolutions' map sizes: [bin][time] of the padded chunk, then
        // halved three times.
        int bins[4] = {c.mels}, times[4] = {longest};
        for (int i = 1; i < 4; ++i) bins[i] = half_len(bins[i - 1]), times[i] = half_len(times[i - 1]);
        const int window = times[3] * c.window_chunks;
        hipStream_t s = stream();
        size_t col_floats = (size_t)t * ch * bins[3], map_floats = (size_t)maps * c.mels * longest;
        for (int i = 1; i < 4; ++i) {
            const size_t positions = (size_t)maps * bins[i] * times[i];
            col_floats = std::max(col_floats, positions * (i == 1 ? 9 : 9 * ch));
            map_floats = std::max(map_floats, positions * ch);
        }
        std::lock_guard<std::mutex> lock(e.ws.mu);
        Workspace& ws = e.ws;
        DeviceMemory& dmel = ws.get(0, (size_t)frames * c.mels * 4);
        DeviceMemory& cols = ws.get(1, col_floats * 4);
        DeviceMemory& map = ws.get(2, map_floats * 4);
        DeviceMemory& x = ws.get(3, (size_t)t * d * 4);
        DeviceMemory& xn = ws.get(4, (size_t)t * d * 4);
        DeviceMemory& qkv = ws.get(5, (size_t)t * 3 * d * 4);
        DeviceMemory& att = ws.get(6, (size_t)t * d * 4);
        DeviceMemory& hid = ws.get(7, (size_t)t * std::max(c.ffn, c.out) * 4);
        DeviceMemory& kc = ws.get(8, (size_t)window * d * 4);
        DeviceMemory& vc = ws.get(9, (size_t)window * d * 4);
        DeviceMemory& st = ws.get(10, sizeof(State));
        DeviceMemory& scratch = ws.bufs[11];
        TRIT_HIP(hipMemcpyAsync(dmel.ptr, mel, (size_t)frames * c.mels * 4, hipMemcpyHostToDevice, s));
        State h0{};  // pos = tk - tq = 0: every row of a window sees the whole window
        TRIT_HIP(hipMemcpyAsync(st.ptr, &h0, sizeof(State), hipMemcpyHostToDevice, s));
        // The chunks (qwen3_asr.rs:389-405): three convolutions with GELU over
        // every chunk's map at once, the time columns of the kept rows,
        // conv_out, the positions.
        hipLaunchKernelGGL(mel_maps_kernel, dim3(blocks_for((size_t)maps * c.mels * longest)), dim3(256), 0, s,
                           dmel.as<float>(), frames, c.mels, c.chunk, maps, longest, map.as<float>());
        for (int i = 0; i < 3; ++i) {
            const int cin = i == 0 ? 1 : ch;
            const size_t rows = (size_t)maps * bins[i + 1] * times[i + 1];
            hipLaunchKernelGGL(conv2d_columns_kernel, dim3(blocks_for(rows * cin * 9)), dim3(256), 0, s,
                               map.as<float>(), maps, bins[i], times[i], cin, cols.as<float>());
            encoder_product(*e.convs[i], cols.as<float>(), (int)rows, map.as<float>(), nullptr, scratch, s);
            hipLaunchKernelGGL(gelu_kernel, dim3(blocks_for(rows * ch)), dim3(256), 0, s, map.as<float>(),
                               rows * ch);
        }
        hipLaunchKernelGGL(time_columns_kernel, dim3(blocks_for((size_t)t * ch * bins[3])), dim3(256), 0, s,
                           map.as<float>(), bins[3], times[3], ch, t, cols.as<float>());
        encoder_product(*e.conv_out, cols.as<float>(), t, x.as<float>(), nullptr, scratch, s);
        hipLaunchKernelGGL(add_positions_kernel, dim3(blocks_for((size_t)t * d)), dim3(256), 0, s, x.as<float>(),
                           e.positions.as<float>(), t, times[3], d);
        // The layers (qwen3_asr.rs:344-368): attention within windows.
        for (int l = 0; l < c.layers; ++l) {
            hipLaunchKernelGGL(layer_norm_kernel, dim3(t), dim3(64), 0, s, x.as<float>(), d, e.norm(l, 0),
                               e.norm(l, 1), NORM_EPS, xn.as<float>());
            encoder_product(*e.layers[4 * l], xn.as<float>(), t, qkv.as<float>(), nullptr, scratch, s);
            for (int w0 = 0; w0 < t; w0 += window) {
                const int n = std::min(window, t - w0);
                const float* q = qkv.as<float>() + (size_t)w0 * 3 * d;
                exact_attention(q, 3 * d, q + d, q + 2 * d, 3 * d, n, n, c.heads, c.heads, hd, 0,
                                att.as<float>() + (size_t)w0 * d, kc.as<float>(), vc.as<float>(), st.as<State>(), s);
            }
            encoder_product(*e.layers[4 * l + 1], att.as<float>(), t, x.as<float>(), x.as<float>(), scratch, s);
            hipLaunchKernelGGL(layer_norm_kernel, dim3(t), dim3(64), 0, s, x.as<float>(), d, e.norm(l, 2),
                               e.norm(l, 3), NORM_EPS, xn.as<float>());
            encoder_product(*e.layers[4 * l + 2], xn.as<float>(), t, hid.as<float>(), nullptr, scratch, s);
            hipLaunchKernelGGL(gelu_kernel, dim3(blocks_for((size_t)t * c.ffn)), dim3(256), 0, s, hid.as<float>(),
                               (size_t)t * c.ffn);
            encoder_product(*e.layers[4 * l + 3], hid.as<float>(), t, x.as<float>(), x.as<float>(), scratch, s);
        }
        // ln_post, proj1, GELU, proj2 (qwen3_asr.rs:369-372).
        hipLaunchKernelGGL(layer_norm_kernel, dim3(t), dim3(64), 0, s, x.as<float>(), d, e.norm(c.layers, 0),
                           e.norm(c.layers, 1), NORM_EPS, xn.as<float>());
        encoder_product(*e.proj1, xn.as<float>(), t, att.as<float>(), nullptr, scratch, s);
        hipLaunchKernelGGL(gelu_kernel, dim3(blocks_for((size_t)t * d)), dim3(256), 0, s, att.as<float>(),
                           (size_t)t * d);
        encoder_product(*e.proj2, att.as<float>(), t, hid.as<float>(), nullptr, scratch, s);
        TRIT_HIP(hipGetLastError());
        TRIT_HIP(hipMemcpyAsync(out, hid.ptr, (size_t)t * c.out * 4, hipMemcpyDeviceToHost, s));
        TRIT_HIP(hipStreamSynchronize(s));
        return t;
    });
}

}  // extern "C"
