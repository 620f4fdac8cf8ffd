// Internal declarations of the trit_hip library (gfx950).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace trit {

struct Error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

[[noreturn]] void fail(const std::string& message);

// The calling thread's error text (trit_hip_last_error).
std::string& error_text();

// Runs `body`; an exception becomes the thread's error text and `failed`
// (the reference's guard, ffi/src/lib.rs:29-46). No exception crosses the ABI.
template <class T, class F>
T guard(T failed, F&& body) {
    error_text().clear();
    try {
        return body();
    } catch (const std::exception& e) {
        error_text() = e.what();
    } catch (...) {
        error_text() = "unknown error";
    }
    return failed;
}

#define TRIT_HIP(expr)                                                                               \
    do {                                                                                             \
        hipError_t trit_e_ = (expr);                                                                 \
        if (trit_e_ != hipSuccess) ::trit::fail(std::string(#expr) + ": " + hipGetErrorString(trit_e_)); \
    } while (0)

// The stream of the calling thread's device (created by trit_hip_init or on
// first use).
hipStream_t stream();
int device_id();

// Device memory owned by one object.
struct DeviceMemory {
    void* ptr = nullptr;
    size_t bytes = 0;
    DeviceMemory() = default;
    explicit DeviceMemory(size_t n) { alloc(n); }
    DeviceMemory(const DeviceMemory&) = delete;
    DeviceMemory& operator=(const DeviceMemory&) = delete;
    ~DeviceMemory() { release(); }
    void alloc(size_t n) {
        release();
        if (n) TRIT_HIP(hipMalloc(&ptr, n));
        bytes = n;
    }
    void release() {
        if (ptr) (void)hipFree(ptr);
        ptr = nullptr;
        bytes = 0;
    }
    template <class T>
    T* as() const {
        return static_cast<T*>(ptr);
    }
    void upload(const void* host, size_t n, size_t offset = 0) {
        TRIT_HIP(hipMemcpy(static_cast<char*>(ptr) + offset, host, n, hipMemcpyHostToDevice));
    }
};

// Host f16 conversions, round to nearest even with subnormals, infinities
// and NaN (Trit's f32_to_f16 / f16_to_f32, src/cpu/tensors.rs:542-595): the
// compiler's _Float16 conversions.
inline uint16_t f32_to_f16_bits(float v) {
    const _Float16 h = (_Float16)v;
    uint16_t b;
    __builtin_memcpy(&b, &h, 2);
    return b;
}
inline float f16_bits_to_f32(uint16_t b) {
    _Float16 h;
    __builtin_memcpy(&h, &b, 2);
    return (float)h;
}

// A layer's weights in device memory. Layouts:
//  Q8_0, Q4_K (after requantization), INT8: codes int8 row-major n x k;
//    scales row-major n x (k/group): f16 bits for Q8_0/Q4_K, f32 for INT8.
//  TERNARY: codes 2 bits each, row-major n x k/4 bytes; in each 16-code
//    span (4 bytes) byte j holds codes j, 4+j, 8+j, 12+j at bits 0,2,4,6;
//    scales f32 n x (k/128).
//  F16, F32, Q8 (f32 math): for each row, the 16 lane chains of the 16-lane
//    sum order: element kk = 16*s + i at [row][i][s] (k/16 values per
//    chain; f16 bits, f32, or int8 codes); Q8 scales f32 n x (k/32).
enum Kind { Q8_0 = 1, INT8 = 2, TERNARY = 3, Q4_K = 4, F16 = 5, F32 = 6, Q8_F32 = 7 };
inline bool float_kind(int kind) { return kind == F16 || kind == F32 || kind == Q8_F32; }

struct Layer {
    int kind = 0, n = 0, k = 0, group = 0;
    DeviceMemory codes, scales, bias;
    // Q4_K made with TRIT_HIP_Q4K=1: the 144-byte super-blocks as stored,
    // row-major n x k/256, for the native product (codes / scales hold
    // Trit's Q8_0 requantization either way).
    DeviceMemory raw;
    int64_t weight_bytes() const { return (int64_t)(codes.bytes + scales.bytes + raw.bytes); }
};

using LayerRef = std::shared_ptr<Layer>;

// ---- GEMV launches -------------------------------------------------------

// Epilogues a product can fuse.
enum Epilogue {
    EPI_STORE = 0,     // y = x W^T (+ bias, relu)
    EPI_RESIDUAL = 1,  // y = residual + x W^T (may alias)
    EPI_SILU_PAIR = 2  // rows r and r + n/2: y[r] = silu(a_r) * b_r, y is m x n/2
};

struct GemvArgs {
    const float* x = nullptr;  // m x k f32 (device)
    int m = 1;
    // RMSNorm applied to each row of x before quantization: x * (inv * w).
    const float* norm_w = nullptr;    // k floats or null
    const float* norm_inv = nullptr;  // m floats (exact mode) or null: computed in the block
    float eps = 1e-6f;
    float* y = nullptr;
    const float* residual = nullptr;
    int epilogue = EPI_STORE;
    int relu = 0;
    // Device flag: nonzero skips the launch (a finished decode loop).
    const int* skip = nullptr;
    // Measurement: events stamped at the product kernel's start and end
    // (hipExtLaunchKernel), or null.
    hipEvent_t ev_start = nullptr, ev_stop = nullptr;
    // Device memory the product may overwrite (scratch_bytes of it), or
    // null: 2..8 rows then quantize in one pass of their own
    // (gemv_scratch_bytes) instead of in every product block.
    void* scratch = nullptr;
    size_t scratch_bytes = 0;
    // Set by the integer products: the quantized rows' image.
    const uint8_t* pre = nullptr;
};

// Launches `kernel`, with the start/stop events of `a` when it has them.
template <typename K, typename... Args>
void launch_timed(const GemvArgs& a, K kernel, dim3 grid, dim3 block, size_t lds, hipStream_t s, Args... args) {
    if (a.ev_start || a.ev_stop)
        hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)lds, s, a.ev_start, a.ev_stop, 0u, args...);
    else
        hipLaunchKernelGGL(kernel, grid, block, lds, s, args...);
}

__host__ __device__ __forceinline__ size_t align16(size_t v) { return (v + 15) & ~(size_t)15; }
// Row stride (ints) of a (row, frame) pair's group dots in LDS: 16-byte rows.
__host__ __device__ __forceinline__ int dot_stride(int groups) { return (groups + 4) & ~3; }
// Bytes of the quantized rows' image: codes m x k, then f32 scales and i32
// code sums m x dot_stride(k / G) each, every part 16-byte aligned -- the
// first bytes of the product kernel's LDS, in the same layout.
__host__ __device__ __forceinline__ size_t pre_bytes(int m, int k, int G) {
    const size_t gs = (size_t)dot_stride(k / G);
    return align16((size_t)m * k) + 2 * align16((size_t)m * gs * 4);
}

// Integer products (Q8_0, Q4_K, INT8, TERNARY), m <= 8.
void gemv_int(const Layer& L, const GemvArgs& a, hipStream_t s);
// Scratch bytes that let gemv_int quantize m rows of k inputs once.
size_t gemv_scratch_bytes(int m, int k);
// Q8_0 / Q4_K / ternary products of 1..8 rows by persistent streaming
// waves (Q4_K of 1..4 rows from its super-blocks when L.raw holds them and
// TRIT_HIP_Q4K allows); false when the shape, the kind or the size is not
// one it takes.
// Rows of more than 16384 inputs in all, and RMSNorm without the caller's
// factors, need the quantization pass's image in a.pre.
bool gemv_stream(const Layer& L, const GemvArgs& a, hipStream_t s);
// The one-row Q8_0 decode product (k 1024, 2048 or 3072); false when the
// shape or kind is not one it takes.
bool gemv_row(const Layer& L, const GemvArgs& a, hipStream_t s);
// Chain steps of a float-math layer's lane-chain layout ([row][16][steps],
// element 16 s + i at lane i, step s): k / 16 rounded up, the tail zero.
__host__ __device__ inline int chain_steps(int k) { return (k + 15) >> 4; }
// Float-math products (F16, F32, Q8), m <= 8; no RMSNorm prologue, no
// SwiGLU epilogue.
void gemv_float(const Layer& L, const GemvArgs& a, hipStream_t s);
// Float-math products of any row count for k <= 128 (no prologue, no
// SwiGLU pair): the same bits row by row.
bool gemm_float_supported(const Layer& L, const GemvArgs& a);
void gemm_float(const Layer& L, const GemvArgs& a, hipStream_t s);
// Integer products of any row count on the matrix cores (Q8_0, Q4_K, INT8;
// k a multiple of the weight group, any n; the SwiGLU pair needs n / 2 a
// multiple of 64). `scratch` holds gemm_scratch_bytes(m, k) bytes of
// device memory the product may overwrite.
bool gemm_supported(const Layer& L, const GemvArgs& a);
size_t gemm_scratch_bytes(int m, int k);
void gemm_int(const Layer& L, const GemvArgs& a, void* scratch, hipStream_t s);
// Any layer kind.
void layer_forward(const Layer& L, const GemvArgs& a, hipStream_t s);

// Requantizes Q4_K super-blocks (device bytes) into Q8_0 codes and f16
// scales in L.codes / L.scales.
void q4_k_requantize(const uint8_t* blocks, int n, int k, Layer& L, hipStream_t s);
// ggml's other block types: values and bytes per block (false for a type
// that is not one of Q4_0 2, Q4_1 3, Q5_0 6, Q5_1 7, Q4_K 12, Q5_K 13, Q6_K 14).
bool ggml_block_type(int type, int* values, int* bytes);
// Blocks of such a type (device bytes, n x k values) expanded and
// requantized into Q8_0 codes (n x k) and f16 scales (n x k/32).
void ggml_requantize(const uint8_t* blocks, int type, int n, int k, int8_t* codes, uint16_t* scales, hipStream_t s);
// f16 scales widened to f32 (device).
void widen_scales(const uint16_t* in, int64_t n, float* out, hipStream_t s);
// Repacks row-major weights of a float kind (device; f16 bits, f32 or int8
// codes) into the lane-chain layout.
void float_repack(const void* src, int kind, int n, int k, void* dst, hipStream_t s);
// Row `index` of a float-kind layer as f32 (device out).
void float_row(const Layer& L, int index, float* out, hipStream_t s);

}  // namespace trit

struct TritHipLayer;
namespace trit {
LayerRef layer_ref(const TritHipLayer* handle);
TritHipLayer* layer_handle(LayerRef layer);
}  // namespace trit
