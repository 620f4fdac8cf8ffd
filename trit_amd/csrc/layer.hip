// The layer half of the C ABI (include/trit_hip.h): construction of the
// device weight cache for each weight kind, and the products.
#include <cstdlib>
#include <cstring>
#include <mutex>

#include "../../include/trit_hip.h"
#include "device.h"
#include "internal.h"

namespace trit {

namespace {
thread_local std::string g_error;
thread_local int g_device = -1;
thread_local hipStream_t g_stream = nullptr;
}  // namespace

[[noreturn]] void fail(const std::string& message) { throw Error(message); }

std::string& error_text() { return g_error; }

int device_id() {
    if (g_device < 0) {
        int count = 0;
        if (hipGetDeviceCount(&count) != hipSuccess || count == 0) fail("no HIP device is visible");
        TRIT_HIP(hipGetDevice(&g_device));
    }
    return g_device;
}

hipStream_t stream() {
    if (!g_stream) {
        device_id();
        TRIT_HIP(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking));
    }
    return g_stream;
}

namespace {

__device__ __forceinline__ float half_at(const uint8_t* p, int at) {
    return f16_to_f32((uint16_t)(p[at] | (p[at + 1] << 8)));
}

// The 6-bit scale and min j of a K-quant block's 12 scale bytes.
__device__ __forceinline__ void scale_min_k4(int j, const uint8_t* q, int& sc, int& m) {
    if (j < 4) {
        sc = q[j] & 63;
        m = q[j + 4] & 63;
    } else {
        sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

// The 32 values of output block `sb` (32 consecutive weights) of ggml type
// T, expanded as ggml's dequantize_row_* in the same float order
// (src/cpu/ggml_quants.rs:125-245): Q4_0 2, Q4_1 3, Q5_0 6, Q5_1 7 (one
// 32-value block each); Q4_K 12, Q5_K 13, Q6_K 14 (eight per 256-value
// super-block).
template <int T>
__device__ void expand32(const uint8_t* __restrict__ blocks, int64_t sb, float (&y)[32]) {
    if constexpr (T == 2 || T == 3 || T == 6 || T == 7) {
        constexpr int size = T == 2 ? 18 : T == 3 ? 20 : T == 6 ? 22 : 24;
        const uint8_t* p = blocks + sb * size;
        const float d = half_at(p, 0);
        const float m = (T == 3 || T == 7) ? half_at(p, 2) : 0.0f;
        if constexpr (T == 2 || T == 3) {
            const uint8_t* qs = p + (T == 2 ? 2 : 4);
            for (int j = 0; j < 16; ++j) {
                if constexpr (T == 2) {
                    y[j] = (float)((qs[j] & 0x0F) - 8) * d;
                    y[j + 16] = (float)((qs[j] >> 4) - 8) * d;
                } else {
                    const float a = (float)(qs[j] & 0x0F) * d, c = (float)(qs[j] >> 4) * d;
                    y[j] = a + m;
                    y[j + 16] = c + m;
                }
            }
        } else {
            const uint8_t* h = p + (T == 6 ? 2 : 4);
            const uint32_t qh = (uint32_t)h[0] | ((uint32_t)h[1] << 8) | ((uint32_t)h[2] << 16) | ((uint32_t)h[3] << 24);
            const uint8_t* qs = h + 4;
            for (int j = 0; j < 16; ++j) {
                const int q0 = (qs[j] & 0x0F) | (int)(((qh >> j) << 4) & 0x10);
                const int q1 = (qs[j] >> 4) | (int)((qh >> (j + 12)) & 0x10);
                if constexpr (T == 6) {
                    y[j] = (float)(q0 - 16) * d;
                    y[j + 16] = (float)(q1 - 16) * d;
                } else {
                    const float a = (float)q0 * d, c = (float)q1 * d;
                    y[j] = a + m;
                    y[j + 16] = c + m;
                }
            }
        }
    } else if constexpr (T == 12 || T == 13) {
        const int64_t super = sb / 8;
        const int j = (int)(sb % 8);
        const uint8_t* p = blocks + super * (T == 12 ? 144 : 176);
        const float d = half_at(p, 0), dmin = half_at(p, 2);
        int sc, mn;
        scale_min_k4(j, p + 4, sc, mn);
        const float d1 = d * (float)sc, m1 = dmin * (float)mn;
        const int shift = (j & 1) * 4;
        if constexpr (T == 12) {
            const uint8_t* q = p + 16 + (j / 2) * 32;
            for (int l = 0; l < 32; ++l) {
                const float t = d1 * (float)((q[l] >> shift) & 0xF);
                y[l] = t - m1;
            }
        } else {
            const uint8_t* qh = p + 16;
            const uint8_t* ql = p + 48 + (j / 2) * 32;
            for (int l = 0; l < 32; ++l) {
                const int high = (qh[l] >> j) & 1 ? 16 : 0;
                const float t = d1 * (float)(((ql[l] >> shift) & 0xF) + high);
                y[l] = t - m1;
            }
        }
    } else {
        static_assert(T == 14, "ggml type");
        const int64_t super = sb / 8;
        const int j = (int)(sb % 8), half = j / 4, quarter = j % 4;
        const uint8_t* p = blocks + super * 210;
        const float d = half_at(p, 208);
        const uint8_t* ql = p + half * 64 + (quarter & 1) * 32;
        const uint8_t* qh = p + 128 + half * 32;
        const int8_t* scales = (const int8_t*)(p + 192 + half * 8);
        const int lshift = (quarter >> 1) * 4, hshift = quarter * 2;
        for (int l = 0; l < 32; ++l) {
            const int q = (int)(int8_t)(((ql[l] >> lshift) & 0xF) | (((qh[l] >> hshift) & 3) << 4)) - 32;
            y[l] = d * (float)scales[l / 16 + 2 * quarter] * (float)q;
        }
    }
}

// Output blocks of ggml type T, each requantized as Blocks::quantize
// (src/cpu/gemm.rs:58-76): d8 = max|y| / 127, code = round(y * (1/d8))
// half away from zero, cast as Rust's `as i8` (saturating, NaN to 0), d8
// stored as f16. One thread per 32-value block.
template <int T>
__global__ void requant_kernel(const uint8_t* __restrict__ blocks, int64_t nsub, int8_t* __restrict__ codes,
                               uint16_t* __restrict__ scales) {
    for (int64_t sb = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; sb < nsub;
         sb += (int64_t)gridDim.x * blockDim.x) {
        float y[32];
        expand32<T>(blocks, sb, y);
        float mx = 0.0f;
        for (int l = 0; l < 32; ++l) mx = __builtin_fmaxf(mx, __builtin_fabsf(y[l]));
        const float d8 = mx / 127.0f;
        const float inverse = d8 != 0.0f ? 1.0f / d8 : 0.0f;
        for (int l = 0; l < 32; ++l) {
            const float r = __builtin_roundf(y[l] * inverse);
            codes[sb * 32 + l] = r != r ? 0 : (int8_t)(int)__builtin_fminf(__builtin_fmaxf(r, -128.0f), 127.0f);
        }
        scales[sb] = f32_to_f16(d8);
    }
}

// The library's f16 conversions (the hardware's, round to nearest even)
// over arrays.
__global__ void f32_to_f16_kernel(const float* __restrict__ in, int64_t n, uint16_t* __restrict__ out) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = f32_to_f16(in[i]);
}
__global__ void f16_to_f32_kernel(const uint16_t* __restrict__ in, int64_t n, float* __restrict__ out) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = f16_to_f32(in[i]);
}

__global__ void widen_scales_kernel(const uint16_t* __restrict__ in, int64_t n, float* __restrict__ out) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = f16_to_f32(in[i]);
}

}  // namespace

bool ggml_block_type(int type, int* values, int* bytes) {
    switch (type) {
        case 2: *values = 32, *bytes = 18; return true;
        case 3: *values = 32, *bytes = 20; return true;
        case 6: *values = 32, *bytes = 22; return true;
        case 7: *values = 32, *bytes = 24; return true;
        case 12: *values = 256, *bytes = 144; return true;
        case 13: *values = 256, *bytes = 176; return true;
        case 14: *values = 256, *bytes = 210; return true;
        default: return false;
    }
}

void ggml_requantize(const uint8_t* blocks, int type, int n, int k, int8_t* codes, uint16_t* scales, hipStream_t s) {
    const int64_t nsub = (int64_t)n * k / 32;
    const dim3 grid(2048), block(256);
    switch (type) {
        case 2: hipLaunchKernelGGL(requant_kernel<2>, grid, block, 0, s, blocks, nsub, codes, scales); break;
        case 3: hipLaunchKernelGGL(requant_kernel<3>, grid, block, 0, s, blocks, nsub, codes, scales); break;
        case 6: hipLaunchKernelGGL(requant_kernel<6>, grid, block, 0, s, blocks, nsub, codes, scales); break;
        case 7: hipLaunchKernelGGL(requant_kernel<7>, grid, block, 0, s, blocks, nsub, codes, scales); break;
        case 12: hipLaunchKernelGGL(requant_kernel<12>, grid, block, 0, s, blocks, nsub, codes, scales); break;
        case 13: hipLaunchKernelGGL(requant_kernel<13>, grid, block, 0, s, blocks, nsub, codes, scales); break;
        case 14: hipLaunchKernelGGL(requant_kernel<14>, grid, block, 0, s, blocks, nsub, codes, scales); break;
        default: fail("ggml type " + std::to_string(type) + " is not a block type the loader expands");
    }
    TRIT_HIP(hipGetLastError());
}

void q4_k_requantize(const uint8_t* blocks, int n, int k, Layer& L, hipStream_t s) {
    const int64_t nsub = (int64_t)n * k / 32;
    L.codes.alloc((size_t)n * k);
    L.scales.alloc((size_t)nsub * 2);
    ggml_requantize(blocks, 12, n, k, L.codes.as<int8_t>(), L.scales.as<uint16_t>(), s);
}

void widen_scales(const uint16_t* in, int64_t n, float* out, hipStream_t s) {
    hipLaunchKernelGGL(widen_scales_kernel, dim3(1024), dim3(256), 0, s, in, n, out);
    TRIT_HIP(hipGetLastError());
}

void layer_forward(const Layer& L, const GemvArgs& a, hipStream_t s) {
    if (float_kind(L.kind)) return gemv_float(L, a, s);
    return gemv_int(L, a, s);
}

// Per-thread staging buffers of the host-pointer forward, and the scratch
// of the calling thread's many-row products. A thread holds one set from a
// pool; when the thread ends, its set goes back to the pool (no HIP call)
// and the next thread to need one takes it after a device synchronisation.
// Nothing frees device memory from a destructor: the main thread's
// thread-local destructors run inside exit(), where the HIP runtime (or a
// profiler wrapped around it) may already have shut down.
struct Staging {
    int device = -1;
    DeviceMemory x, y, scratch;
};

struct StagingPool {
    std::mutex mu;
    std::vector<Staging*> idle;
};

StagingPool& staging_pool() {
    static StagingPool* pool = new StagingPool();  // never destroyed
    return *pool;
}

struct StagingSlot {
    Staging* set = nullptr;
    ~StagingSlot() {
        if (!set) return;
        StagingPool& p = staging_pool();
        std::lock_guard<std::mutex> lock(p.mu);
        p.idle.push_back(set);
    }
};
thread_local StagingSlot g_slot;

Staging& staging() {
    if (!g_slot.set) {
        const int dev = device_id();
        Staging* got = nullptr;
        {
            StagingPool& p = staging_pool();
            std::lock_guard<std::mutex> lock(p.mu);
            for (size_t i = 0; i < p.idle.size(); ++i)
                if (p.idle[i]->device == dev) {
                    got = p.idle[i];
                    p.idle.erase(p.idle.begin() + (ptrdiff_t)i);
                    break;
                }
        }
        if (got) {
            // Work its previous thread queued may still use it.
            TRIT_HIP(hipDeviceSynchronize());
        } else {
            got = new Staging();
            got->device = dev;
        }
        g_slot.set = got;
    }
    return *g_slot.set;
}

// Rows above this many run on the matrix cores when the layer allows it.
constexpr int GEMM_MIN_ROWS = 9;

// The scratch of trit_hip_layer_forward_device_noalloc: one array per
// device in the library's own code object, so that call allocates nothing.
// Every such call on a device shares that device's array (calls that
// overlap on one device race), and it keeps the last call's contents: the
// products write all of it they read before reading it.
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)4 << 20;
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

// The device address of `scratch` per device, found once per device with
// that device current (in host code the array's name is no device address).
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[MAX_DEVICES] = {};

void resolve_noalloc_scratch(int dev) {
    if (dev < 0 || dev >= MAX_DEVICES) fail("device " + std::to_string(dev) + " is beyond the library's table");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev]) return;
    void* ptr = nullptr;
    TRIT_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    if (!ptr) fail("no device address for the no-allocation scratch");
    g_scratch_ptr[dev] = ptr;
}

void* noalloc_scratch(int dev) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    return g_scratch_ptr[dev];
}

// Grows the calling thread's scratch to `need` bytes.
void* staging_scratch(size_t need) {
    Staging& g = staging();
    if (g.scratch.bytes < need) {
        // Work already queued may still use the old scratch.
        TRIT_HIP(hipDeviceSynchronize());
        g.scratch.alloc(need);
    }
    return g.scratch.ptr;
}

// One product of m rows: the matrix-core product for many rows, else the
// small-batch kernels in calls of up to 8 rows (2..8 rows of an integer
// layer with their activations quantized once, in the scratch). `get`
// gives the scratch of `need` bytes (staging_scratch, or the no-allocation
// array).
template <class Scratch>
void forward_rows(const Layer& L, GemvArgs a, int m, hipStream_t s, Scratch get) {
    a.m = m;
    if (m >= GEMM_MIN_ROWS && gemm_supported(L, a)) return gemm_int(L, a, get(gemm_scratch_bytes(m, L.k)), s);
    if (m > 8 && !a.ev_start && !a.ev_stop && gemm_float_supported(L, a)) return gemm_float(L, a, s);
    if (m >= 2 && !float_kind(L.kind)) {
        a.scratch_bytes = gemv_scratch_bytes(m < 8 ? m : 8, L.k);
        a.scratch = get(a.scratch_bytes);
    }
    if (a.ev_start || a.ev_stop) {
        if (m > 8) fail("timed forward: more than 8 rows of this layer take several launches");
    }
    const float* x = a.x;
    float* y = a.y;
    for (int r0 = 0; r0 < m; r0 += 8) {
        a.x = x + (size_t)r0 * L.k;
        a.y = y + (size_t)r0 * L.n;
        a.m = m - r0 < 8 ? m - r0 : 8;
        layer_forward(L, a, s);
    }
}

}  // namespace trit

struct TritHipLayer {
    trit::LayerRef layer;
};

using namespace trit;

namespace {

void upload_bias(Layer& L, const float* bias) {
    if (!bias) return;
    L.bias.alloc((size_t)L.n * 4);
    L.bias.upload(bias, (size_t)L.n * 4);
}

void check_shape(int n, int k, int k_multiple, const char* what) {
    if (n <= 0 || k <= 0) fail(std::string(what) + ": empty layer");
    if (k % k_multiple != 0)
        fail(std::string(what) + ": k = " + std::to_string(k) + " is not a multiple of " + std::to_string(k_multiple));
}

int finish(std::shared_ptr<Layer> L, TritHipLayer** out) {
    if (!out) fail("out is NULL");
    TRIT_HIP(hipStreamSynchronize(stream()));
    *out = new TritHipLayer{std::move(L)};
    return 0;
}

// The lane-chain layout of a float-math layer's row-major device weights,
// the steps past k (when k is not a multiple of 16) zero.
void chain_layout(Layer& L, const void* raw, size_t elem) {
    const size_t bytes = (size_t)L.n * 16 * chain_steps(L.k) * elem;
    L.codes.alloc(bytes);
    if (L.k % 16) TRIT_HIP(hipMemsetAsync(L.codes.ptr, 0, bytes, stream()));
    float_repack(raw, L.kind, L.n, L.k, L.codes.ptr, stream());
}

// A float-math layer (F32, or Q8 with f32 scales n x k/32) from row-major
// host weights, repacked into the lane-chain layout.
int float_layer(int kind, int n, int k, const void* weights, const float* scales, const float* bias,
                TritHipLayer** out, const char* what) {
    check_shape(n, k, kind == Q8_F32 ? 32 : 1, what);
    if (!weights) fail(std::string(what) + ": weights is NULL");
    auto L = std::make_shared<Layer>();
    L->kind = kind;
    L->n = n;
    L->k = k;
    const size_t elem = kind == F32 ? 4 : 1;
    const size_t bytes = (size_t)n * k * elem;
    DeviceMemory raw(bytes);
    raw.upload(weights, bytes);
    chain_layout(*L, raw.ptr, elem);
    if (kind == Q8_F32) {
        L->scales.alloc((size_t)n * (k / 32) * 4);
        L->scales.upload(scales, (size_t)n * (k / 32) * 4);
    }
    upload_bias(*L, bias);
    TRIT_HIP(hipStreamSynchronize(stream()));
    return finish(L, out);
}

// A layer from ggml blocks of another type (not Q8_0): expanded and
// requantized to Q8_0 codes on the device (Tensors::q8_0 of such a tensor,
// src/cpu/tensors.rs:262-305), then held as Dense::q8_0 holds them -- int8
// activations when n % 32 == 0 and f32_math is false, else the codes with
// f32 math (a table, or a shape the int8 kernels refuse).
int ggml_layer(int n, int k, int type, const void* blocks, const float* bias, bool f32_math, TritHipLayer** out) {
    int values = 0, size = 0;
    if (!ggml_block_type(type, &values, &size))
        fail("ggml layer: type " + std::to_string(type) + " is not Q4_0, Q4_1, Q5_0, Q5_1, Q4_K, Q5_K or Q6_K");
    check_shape(n, k, values, "ggml layer");
    const size_t bytes = (size_t)n * k / values * size;
    DeviceMemory raw(bytes);
    raw.upload(blocks, bytes);
    const int64_t nsub = (int64_t)n * k / 32;
    auto L = std::make_shared<Layer>();
    L->n = n;
    L->k = k;
    if (!f32_math && n % 32 == 0) {
        L->kind = type == 12 ? Q4_K : Q8_0;
        L->group = 32;
        L->codes.alloc((size_t)n * k);
        L->scales.alloc((size_t)nsub * 2);
        ggml_requantize(raw.as<uint8_t>(), type, n, k, L->codes.as<int8_t>(), L->scales.as<uint16_t>(), stream());
        // TRIT_HIP_Q4K=1: the super-blocks stay too, for the native product
        // (measured slower than the requantized codes on MI355X, so opt-in).
        const char* native = getenv("TRIT_HIP_Q4K");
        if (type == 12 && native && native[0] == '1') std::swap(L->raw.ptr, raw.ptr), std::swap(L->raw.bytes, raw.bytes);
    } else {
        L->kind = Q8_F32;
        DeviceMemory codes((size_t)n * k), half((size_t)nsub * 2);
        ggml_requantize(raw.as<uint8_t>(), type, n, k, codes.as<int8_t>(), half.as<uint16_t>(), stream());
        L->codes.alloc((size_t)n * k);
        float_repack(codes.ptr, Q8_F32, n, k, L->codes.ptr, stream());
        L->scales.alloc((size_t)nsub * 4);
        widen_scales(half.as<uint16_t>(), nsub, L->scales.as<float>(), stream());
        TRIT_HIP(hipStreamSynchronize(stream()));  // before the temporaries go
    }
    upload_bias(*L, bias);
    TRIT_HIP(hipStreamSynchronize(stream()));
    return finish(L, out);
}

// Q8_0 blocks as int8 storage with f32 math: the codes as stored and each
// block's f16 scale widened to f32 (Q8 built from Blocks, src/cpu/gemm.rs:
// 238-244,386-393).
int q8_from_blocks(int n, int k, const void* blocks, const float* bias, TritHipLayer** out) {
    const size_t nb = (size_t)n * k / 32;
    std::vector<int8_t> codes((size_t)n * k);
    std::vector<float> scales(nb);
    const uint8_t* p = static_cast<const uint8_t*>(blocks);
    for (size_t b = 0; b < nb; ++b) {
        scales[b] = f16_bits_to_f32((uint16_t)(p[b * 34] | (p[b * 34 + 1] << 8)));
        std::memcpy(&codes[b * 32], p + b * 34 + 2, 32);
    }
    return float_layer(Q8_F32, n, k, codes.data(), scales.data(), bias, out, "Q8_0 table");
}

}  // namespace

namespace {

// Host arrays through the device in chunks of 16 Mi values.
template <typename In, typename Out, typename K>
int convert(const In* in, int64_t n, Out* out, K kernel, const char* what) {
    if (n < 0) fail(std::string(what) + ": negative count");
    if (n && (!in || !out)) fail(std::string(what) + ": in or out is NULL");
    const int64_t chunk = (int64_t)1 << 24;
    const int64_t first = n < chunk ? n : chunk;
    DeviceMemory din((size_t)first * sizeof(In)), dout((size_t)first * sizeof(Out));
    hipStream_t s = stream();
    for (int64_t at = 0; at < n; at += chunk) {
        const int64_t c = n - at < chunk ? n - at : chunk;
        TRIT_HIP(hipMemcpyAsync(din.ptr, in + at, (size_t)c * sizeof(In), hipMemcpyHostToDevice, s));
        hipLaunchKernelGGL(kernel, dim3(1024), dim3(256), 0, s, din.as<In>(), c, dout.as<Out>());
        TRIT_HIP(hipGetLastError());
        TRIT_HIP(hipMemcpyAsync(out + at, dout.ptr, (size_t)c * sizeof(Out), hipMemcpyDeviceToHost, s));
    }
    TRIT_HIP(hipStreamSynchronize(s));
    return 0;
}

}  // namespace

extern "C" {

const char* trit_hip_version(void) { return "trit_hip 0.1.0 (gfx950)"; }

const char* trit_hip_last_error(void) { return g_error.c_str(); }

int trit_hip_init(int device) {
    return guard(-1, [&] {
        int count = 0;
        TRIT_HIP(hipGetDeviceCount(&count));
        if (device < 0 || device >= count)
            fail("device " + std::to_string(device) + " does not exist (" + std::to_string(count) + " visible)");
        TRIT_HIP(hipSetDevice(device));
        g_device = device;
        stream();
        resolve_noalloc_scratch(device);
        return 0;
    });
}

int trit_hip_layer_q8_0(int n, int k, const void* blocks, const float* bias, TritHipLayer** out) {
    return guard(-1, [&] {
        check_shape(n, k, 32, "Q8_0 layer");
        if (!blocks) fail("Q8_0 layer: blocks is NULL");
        // Dense::q8_0: int8 activations where the int8 kernels take the
        // shape (Int8::fits_group: n % 32 == 0), else int8 storage with f32
        // math (src/cpu/gemm.rs:225-247, src/cpu/int8.rs:234-236).
        if (n % 32) return q8_from_blocks(n, k, blocks, bias, out);
        auto L = std::make_shared<Layer>();
        L->kind = Q8_0;
        L->n = n;
        L->k = k;
        L->group = 32;
        const size_t nb = (size_t)n * k / 32;
        std::vector<int8_t> codes((size_t)n * k);
        std::vector<uint16_t> scales(nb);
        const uint8_t* p = static_cast<const uint8_t*>(blocks);
        for (size_t b = 0; b < nb; ++b) {
            scales[b] = (uint16_t)(p[b * 34] | (p[b * 34 + 1] << 8));
            std::memcpy(&codes[b * 32], p + b * 34 + 2, 32);
        }
        L->codes.alloc(codes.size());
        L->codes.upload(codes.data(), codes.size());
        L->scales.alloc(nb * 2);
        L->scales.upload(scales.data(), nb * 2);
        upload_bias(*L, bias);
        return finish(L, out);
    });
}

int trit_hip_layer_int8(int n, int k, const int8_t* codes, const float* scales, const float* bias,
                        TritHipLayer** out) {
    return guard(-1, [&] {
        check_shape(n, k, 128, "int8 layer");
        if (!codes || !scales) fail("int8 layer: codes or scales is NULL");
        auto L = std::make_shared<Layer>();
        L->kind = INT8;
        L->n = n;
        L->k = k;
        L->group = 128;
        L->codes.alloc((size_t)n * k);
        L->codes.upload(codes, (size_t)n * k);
        L->scales.alloc((size_t)n * (k / 128) * 4);
        L->scales.upload(scales, (size_t)n * (k / 128) * 4);
        upload_bias(*L, bias);
        return finish(L, out);
    });
}

static int ternary_from_codes(int n, int k, const uint8_t* codes, const float* scales, TritHipLayer** out) {
    check_shape(n, k, 128, "ternary layer");
    if (!codes || !scales) fail("ternary layer: codes or scales is NULL");
    auto L = std::make_shared<Layer>();
    L->kind = TERNARY;
    L->n = n;
    L->k = k;
    L->group = 128;
    std::vector<uint8_t> packed((size_t)n * k / 4);
    for (int r = 0; r < n; ++r) {
        for (int span = 0; span < k / 16; ++span) {
            const uint8_t* c = codes + (size_t)r * k + span * 16;
            for (int j = 0; j < 4; ++j) {
                for (int t = 0; t < 4; ++t)
                    if (c[4 * t + j] > 2) fail("ternary layer: a code above 2 in row " + std::to_string(r));
                packed[(size_t)r * (k / 4) + span * 4 + j] =
                    (uint8_t)(c[j] | (c[4 + j] << 2) | (c[8 + j] << 4) | (c[12 + j] << 6));
            }
        }
    }
    L->codes.alloc(packed.size());
    L->codes.upload(packed.data(), packed.size());
    L->scales.alloc((size_t)n * (k / 128) * 4);
    L->scales.upload(scales, (size_t)n * (k / 128) * 4);
    return finish(L, out);
}

int trit_hip_layer_ternary(int n, int k, const uint8_t* codes, const float* scales, TritHipLayer** out) {
    return guard(-1, [&] { return ternary_from_codes(n, k, codes, scales, out); });
}

int trit_hip_layer_ternary_base3(int n, int k, const uint8_t* packed, const float* scales, TritHipLayer** out) {
    return guard(-1, [&] {
        if (!packed) fail("ternary layer: packed is NULL");
        check_shape(n, k, 128, "ternary layer");
        const int row_bytes = (k + 4) / 5;
        std::vector<uint8_t> codes((size_t)n * k);
        for (int r = 0; r < n; ++r) {
            for (int b = 0; b < row_bytes; ++b) {
                int v = packed[(size_t)r * row_bytes + b];
                if (v > 242) fail("ternary byte above 242 in row " + std::to_string(r));
                for (int digit = 0; digit < 5; ++digit) {
                    const int kk = b * 5 + digit;
                    if (kk < k) codes[(size_t)r * k + kk] = (uint8_t)(v % 3);
                    v /= 3;
                }
            }
        }
        return ternary_from_codes(n, k, codes.data(), scales, out);
    });
}

int trit_hip_f32_to_f16(const float* in, int64_t n, uint16_t* out) {
    return guard(-1, [&] { return convert(in, n, out, f32_to_f16_kernel, "f32_to_f16"); });
}

int trit_hip_f16_to_f32(const uint16_t* in, int64_t n, float* out) {
    return guard(-1, [&] { return convert(in, n, out, f16_to_f32_kernel, "f16_to_f32"); });
}

int trit_hip_layer_q4_k(int n, int k, const void* blocks, TritHipLayer** out) {
    return guard(-1, [&] {
        if (!blocks) fail("Q4_K layer: blocks is NULL");
        return ggml_layer(n, k, 12, blocks, nullptr, false, out);
    });
}

int trit_hip_layer_ggml(int n, int k, int ggml_type, const void* blocks, const float* bias, int f32_math,
                        TritHipLayer** out) {
    return guard(-1, [&] {
        if (!blocks) fail("ggml layer: blocks is NULL");
        if (ggml_type == 8) {
            check_shape(n, k, 32, "Q8_0 layer");
            if (f32_math || n % 32) return q8_from_blocks(n, k, blocks, bias, out);
            if (trit_hip_layer_q8_0(n, k, blocks, bias, out) != 0) fail(error_text());
            return 0;
        }
        return ggml_layer(n, k, ggml_type, blocks, bias, f32_math != 0, out);
    });
}
int trit_hip_layer_f32(int n, int k, const float* weights, const float* bias, TritHipLayer** out) {
    return guard(-1, [&] { return float_layer(F32, n, k, weights, nullptr, bias, out, "f32 layer"); });
}

int trit_hip_layer_q8(int n, int k, const int8_t* codes, const float* scales, const float* bias,
                      TritHipLayer** out) {
    return guard(-1, [&] {
        if (!scales) fail("q8 layer: scales is NULL");
        return float_layer(Q8_F32, n, k, codes, scales, bias, out, "q8 layer");
    });
}

int trit_hip_layer_q8_0_f32(int n, int k, const void* blocks, const float* bias, TritHipLayer** out) {
    return guard(-1, [&] {
        check_shape(n, k, 32, "Q8_0 table");
        if (!blocks) fail("Q8_0 table: blocks is NULL");
        return q8_from_blocks(n, k, blocks, bias, out);
    });
}

int trit_hip_layer_f16(int n, int k, const uint16_t* weights, const float* bias, TritHipLayer** out) {
    return guard(-1, [&] {
        check_shape(n, k, 1, "f16 layer");
        if (!weights) fail("f16 layer: weights is NULL");
        auto L = std::make_shared<Layer>();
        L->kind = F16;
        L->n = n;
        L->k = k;
        const size_t bytes = (size_t)n * k * 2;
        DeviceMemory raw(bytes);
        raw.upload(weights, bytes);
        chain_layout(*L, raw.ptr, 2);
        upload_bias(*L, bias);
        TRIT_HIP(hipStreamSynchronize(stream()));
        return finish(L, out);
    });
}

int trit_hip_layer_forward_device(const TritHipLayer* layer, const float* x, int m, int relu, float* y,
                                  void* s) {
    return guard(-1, [&] {
        if (!layer || !x || !y) fail("layer, x or y is NULL");
        GemvArgs a;
        a.x = x;
        a.m = m;
        a.y = y;
        a.relu = relu;
        if (m <= 0) fail("m must be positive");
        forward_rows(*layer->layer, a, m, s ? (hipStream_t)s : stream(), staging_scratch);
        return 0;
    });
}

int trit_hip_layer_forward_device_noalloc(const TritHipLayer* layer, const float* x, int m, int relu, float* y,
                                          void* s) {
    return guard(-1, [&] {
        if (!layer || !x || !y) fail("layer, x or y is NULL");
        if (m <= 0) fail("m must be positive");
        const int dev = device_id();
        if (dev < 0 || dev >= MAX_DEVICES) fail("device " + std::to_string(dev) + " is beyond the library's table");
        void* base = noalloc_scratch(dev);
        if (!base) {
            // trit_hip_init found it for the devices it set up; otherwise the
            // first call on this device does.
            resolve_noalloc_scratch(dev);
            base = noalloc_scratch(dev);
        }
        GemvArgs a;
        a.x = x;
        a.m = m;
        a.y = y;
        a.relu = relu;
        const Layer& L = *layer->layer;
        forward_rows(L, a, m, s ? (hipStream_t)s : stream(), [&](size_t need) -> void* {
            if (need > NOALLOC_SCRATCH_BYTES)
                fail("no-allocation forward: " + std::to_string(m) + " rows of a " + std::to_string(L.n) + "x" +
                     std::to_string(L.k) + " layer need " + std::to_string(need) + " bytes of scratch, more than the " +
                     std::to_string(NOALLOC_SCRATCH_BYTES) + " it holds");
            return base;
        });
        return 0;
    });
}

int trit_hip_layer_forward_timed(const TritHipLayer* layer, const float* x, int m, int relu, float* y, void* s,
                                 void* start_event, void* stop_event) {
    return guard(-1, [&] {
        if (!layer || !x || !y) fail("layer, x or y is NULL");
        if (m <= 0) fail("m must be positive");
        GemvArgs a;
        a.x = x;
        a.y = y;
        a.relu = relu;
        a.ev_start = (hipEvent_t)start_event;
        a.ev_stop = (hipEvent_t)stop_event;
        forward_rows(*layer->layer, a, m, s ? (hipStream_t)s : stream(), staging_scratch);
        return 0;
    });
}

int trit_hip_layer_forward(const TritHipLayer* layer, const float* x, int m, int relu, float* y) {
    return guard(-1, [&] {
        if (!layer || !x || !y) fail("layer, x or y is NULL");
        if (m <= 0) fail("m must be positive");
        const Layer& L = *layer->layer;
        const size_t xb = (size_t)m * L.k * 4, yb = (size_t)m * L.n * 4;
        Staging& g = staging();
        if (g.x.bytes < xb) g.x.alloc(xb);
        if (g.y.bytes < yb) g.y.alloc(yb);
        hipStream_t st = stream();
        TRIT_HIP(hipMemcpyAsync(g.x.ptr, x, xb, hipMemcpyHostToDevice, st));
        if (trit_hip_layer_forward_device(layer, g.x.as<float>(), m, relu, g.y.as<float>(), st) != 0)
            fail(g_error);
        TRIT_HIP(hipMemcpyAsync(y, g.y.ptr, yb, hipMemcpyDeviceToHost, st));
        TRIT_HIP(hipStreamSynchronize(st));
        return 0;
    });
}

int trit_hip_layer_info(const TritHipLayer* layer, int* n, int* k, int* kind, int64_t* device_bytes) {
    return guard(-1, [&] {
        if (!layer) fail("layer is NULL");
        const Layer& L = *layer->layer;
        if (n) *n = L.n;
        if (k) *k = L.k;
        if (kind) *kind = L.kind;
        if (device_bytes) *device_bytes = L.weight_bytes();
        return 0;
    });
}

int trit_hip_layer_row(const TritHipLayer* layer, int index, float* out) {
    return guard(-1, [&] {
        if (!layer || !out) fail("layer or out is NULL");
        const Layer& L = *layer->layer;
        if (!float_kind(L.kind)) fail("row: only F16, F32 and Q8 token tables");
        if (index < 0 || index >= L.n) fail("row: index out of range");
        DeviceMemory d((size_t)L.k * 4);
        float_row(L, index, d.as<float>(), stream());
        TRIT_HIP(hipMemcpyAsync(out, d.ptr, (size_t)L.k * 4, hipMemcpyDeviceToHost, stream()));
        TRIT_HIP(hipStreamSynchronize(stream()));
        return 0;
    });
}

void trit_hip_layer_free(TritHipLayer* layer) { delete layer; }

}  // extern "C"

namespace trit {
LayerRef layer_ref(const TritHipLayer* h) { return h ? h->layer : nullptr; }
TritHipLayer* layer_handle(LayerRef L) { return new TritHipLayer{std::move(L)}; }
}  // namespace trit
