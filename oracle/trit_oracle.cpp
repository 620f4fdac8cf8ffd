// CPU restatement of Trit's decoder-loop numerics.
//
// TEST INFRASTRUCTURE, NOT PRODUCT CODE: the tests, the smoke check and the
// benchmark's CPU-baseline leg load it as the checker; the HIP library never
// does. Each function cites the Rust file:line of Hi9841/trit it restates.
//
// Bits: Trit's default x86 path (AVX-512 VNNI, first kernel set) defines
// the values. Path 0 ("contract") states them one value at a time; paths 1
// (AVX2) and 2 (AVX-512 VNNI) restate Trit's tiles for the timed baseline.
// Integer products agree on all paths; f32 products (the f16 head, attention)
// follow the 16-lane contract on paths 0 and 2 and Trit's 8-lane AVX2 tiles
// on path 1 (which Trit itself gives other bits for, src/cpu/v2/float.rs:10-14).
//
// Build with -ffp-contract=off: every fused multiply-add is an explicit fmaf.

#include "trit_oracle.h"

#include <immintrin.h>
#include <pthread.h>
#include <sched.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <functional>
#include <set>
#include <sstream>
#include <string>
#include <thread>
#include <vector>

#define AVX512 __attribute__((target("avx512f,avx512bw,avx512vl,avx512vnni,fma,f16c,avx2")))
#define AVX2T __attribute__((target("avx2,fma,f16c")))

namespace {

// ---------------------------------------------------------------- f16 ---
// src/cpu/tensors.rs:542-573: round to nearest even, subnormals kept,
// out of range to infinity, NaN stays a quiet NaN.
uint16_t f32_to_f16(float value) {
    uint32_t bits;
    std::memcpy(&bits, &value, 4);
    uint16_t sign = (uint16_t)((bits >> 16) & 0x8000);
    int32_t exponent = (int32_t)((bits >> 23) & 0xff);
    uint32_t mantissa = bits & 0x7fffff;
    if (exponent == 0xff) return sign | 0x7c00 | (mantissa ? 0x200 : 0);
    int32_t he = exponent - 127 + 15;
    if (he >= 0x1f) return sign | 0x7c00;
    if (he <= 0) {
        if (he < -10) return sign;
        uint32_t full = mantissa | 0x800000;
        uint32_t shift = (uint32_t)(14 - he);
        uint32_t half = full >> shift;
        uint32_t rest = full & ((1u << shift) - 1);
        uint32_t mid = 1u << (shift - 1);
        bool up = rest > mid || (rest == mid && (half & 1));
        return sign | (uint16_t)(half + (up ? 1 : 0));
    }
    uint32_t half = ((uint32_t)he << 10) | (mantissa >> 13);
    uint32_t rest = mantissa & 0x1fff;
    bool up = rest > 0x1000 || (rest == 0x1000 && (half & 1));
    return sign | (uint16_t)(half + (up ? 1 : 0));
}

// src/cpu/tensors.rs:575-595.
float f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff, bits;
    if (e == 0 && m == 0) {
        bits = sign;
    } else if (e == 0) {
        uint32_t ex = 127 - 15 + 1;
        while (!(m & 0x400)) {
            m <<= 1;
            ex -= 1;
        }
        bits = sign | (ex << 23) | ((m & 0x3ff) << 13);
    } else if (e == 0x1f) {
        bits = sign | 0x7f800000 | (m << 13);
    } else {
        bits = sign | ((e + 127 - 15) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

float f16r(float v) { return f16_to_f32(f32_to_f16(v)); }

// ------------------------------------------------------------ exp/silu ---
// Constants of src/cpu/activation.rs:8-38 (Cephes expf, Moshier's method).
constexpr float LOG2E = 1.44269504088896340736f;
constexpr float LN2_HI = 0.693359375f;
constexpr float LN2_LO = -2.12194440e-4f;
constexpr float EXP_LOW = -87.3f;
constexpr float EXP_HIGH = 88.0f;
constexpr float POLY[6] = {1.9875691e-4f, 1.3981999e-3f, 8.333452e-3f,
                           4.1665796e-2f, 0.16666665f, 0.5f};

// The AVX-512 exp of src/cpu/activation.rs:357-375 (= src/cpu/v2/activation.rs:45-56):
// max then min clamp, n = cvtps (ties to even), two fused reductions,
// Horner with fused steps from 0, y = fma(p, r*r, r+1), times 2^n.
float exp_contract(float x) {
    x = std::fmin(std::fmax(x, EXP_LOW), EXP_HIGH);
    if (std::isnan(x)) x = EXP_LOW;
    float t = x * LOG2E;
    int n_int = (int)std::nearbyint(t);
    float n = (float)n_int;
    float r = std::fmaf(-n, LN2_HI, x);
    r = std::fmaf(-n, LN2_LO, r);
    float p = 0.0f;
    for (float c : POLY) p = std::fmaf(p, r, c);
    float y = std::fmaf(p, r * r, r + 1.0f);
    uint32_t bits = (uint32_t)(n_int + 127) << 23;
    float two;
    std::memcpy(&two, &bits, 4);
    return y * two;
}

float silu_one(float v) { return v / (1.0f + exp_contract(0.0f - v)); }

// Numerical Recipes' erfcc coefficients, Horner order (src/cpu/activation.rs:15-28).
constexpr float ERFC[10] = {0.17087277f, -0.82215223f, 1.4885159f, -1.135204f, 0.27886807f,
                            -0.18628806f, 0.09678418f, 0.37409196f, 1.0000237f, -1.2655122f};
constexpr float FRAC_1_SQRT_2 = 0.70710678118654752440f;

// The exact GELU in the fused form every path gives (src/cpu/v2/activation.rs:
// 33-39): v * erfc(-v / sqrt 2) / 2, erfc(z) = t * exp(-z^2 + P(t)).
float gelu_one(float v) {
    const float z = std::fabs(v) * FRAC_1_SQRT_2;
    const float t = 1.0f / std::fmaf(z, 0.5f, 1.0f);
    float p = 0.0f;
    for (float c : ERFC) p = std::fmaf(p, t, c);
    const float tail = t * exp_contract(std::fmaf(-z, z, p));
    return (0.5f * v) * (v >= 0.0f ? 2.0f - tail : tail);
}

AVX512 __m512 exp512(__m512 x) {
    x = _mm512_min_ps(_mm512_max_ps(x, _mm512_set1_ps(EXP_LOW)), _mm512_set1_ps(EXP_HIGH));
    __m512i n_int = _mm512_cvtps_epi32(_mm512_mul_ps(x, _mm512_set1_ps(LOG2E)));
    __m512 n = _mm512_cvtepi32_ps(n_int);
    __m512 r = _mm512_fnmadd_ps(n, _mm512_set1_ps(LN2_HI), x);
    r = _mm512_fnmadd_ps(n, _mm512_set1_ps(LN2_LO), r);
    __m512 p = _mm512_setzero_ps();
    for (float c : POLY) p = _mm512_fmadd_ps(p, r, _mm512_set1_ps(c));
    __m512 y = _mm512_fmadd_ps(p, _mm512_mul_ps(r, r), _mm512_add_ps(r, _mm512_set1_ps(1.0f)));
    __m512i two = _mm512_slli_epi32(_mm512_add_epi32(n_int, _mm512_set1_epi32(127)), 23);
    return _mm512_mul_ps(y, _mm512_castsi512_ps(two));
}

// ---------------------------------------------------------------- team ---
// A spinning worker team in the manner of src/cpu/team.rs:1-130,900-976:
// the calling thread takes tasks too; workers pinned one per core.
struct Team {
    std::vector<std::thread> workers;
    std::atomic<uint64_t> generation{0};
    std::atomic<int> next{0}, done{0}, active{0};
    std::atomic<bool> stop{false};
    const std::function<void(int)>* job = nullptr;
    int tasks = 0;
    int size = 1;

    void work() {
        for (;;) {
            int t = next.fetch_add(1, std::memory_order_acq_rel);
            if (t >= tasks) break;
            (*job)(t);
            done.fetch_add(1, std::memory_order_acq_rel);
        }
    }

    void worker_loop() {
        uint64_t seen = 0;
        int idle = 0;
        while (!stop.load(std::memory_order_acquire)) {
            uint64_t g = generation.load(std::memory_order_acquire);
            if (g == seen) {
                if (++idle < 20000) {
                    _mm_pause();
                } else {
                    std::this_thread::yield();
                }
                continue;
            }
            idle = 0;
            active.fetch_add(1, std::memory_order_acq_rel);
            if (generation.load(std::memory_order_acquire) == g) work();
            active.fetch_sub(1, std::memory_order_acq_rel);
            seen = g;
        }
    }

    void run(int n, const std::function<void(int)>& fn) {
        if (n <= 0) return;
        if (size <= 1 || n == 1) {
            for (int t = 0; t < n; ++t) fn(t);
            return;
        }
        while (active.load(std::memory_order_acquire) != 0) _mm_pause();
        job = &fn;
        tasks = n;
        done.store(0, std::memory_order_release);
        next.store(0, std::memory_order_release);
        generation.fetch_add(1, std::memory_order_acq_rel);
        work();
        while (done.load(std::memory_order_acquire) < n) _mm_pause();
        while (active.load(std::memory_order_acquire) != 0) _mm_pause();
    }

    ~Team() {
        stop.store(true);
        for (auto& w : workers) w.join();
    }
};

Team* g_team = nullptr;

std::vector<int> parse_list(const std::string& s) {
    std::vector<int> out;
    std::stringstream ss(s);
    std::string part;
    while (std::getline(ss, part, ',')) {
        size_t dash = part.find('-');
        if (dash == std::string::npos) {
            if (!part.empty()) out.push_back(std::atoi(part.c_str()));
        } else {
            int a = std::atoi(part.substr(0, dash).c_str()), b = std::atoi(part.substr(dash + 1).c_str());
            for (int i = a; i <= b; ++i) out.push_back(i);
        }
    }
    return out;
}

std::string read_line(const std::string& path) {
    std::ifstream f(path);
    std::string s;
    std::getline(f, s);
    return s;
}

// One CPU per physical core of the largest L3 domain that this process may
// use (src/cpu/mod.rs:127-161,281-292), capped by the cgroup CPU quota.
std::vector<int> team_cpus(int spread) {
    cpu_set_t set;
    CPU_ZERO(&set);
    sched_getaffinity(0, sizeof(set), &set);
    std::vector<int> allowed;
    for (int c = 0; c < CPU_SETSIZE; ++c)
        if (CPU_ISSET(c, &set)) allowed.push_back(c);
    std::set<int> allowed_set(allowed.begin(), allowed.end());
    // Physical cores: the first CPU of each sibling list.
    std::set<int> cores;
    for (int c : allowed) {
        auto sib = parse_list(read_line("/sys/devices/system/cpu/cpu" + std::to_string(c) +
                                        "/topology/thread_siblings_list"));
        int first = c;
        for (int s : sib)
            if (allowed_set.count(s)) first = std::min(first, s);
        cores.insert(first);
    }
    std::vector<int> chosen(cores.begin(), cores.end());
    if (spread == 0) {
        // L3 domains by shared_cpu_list; take the one with the most cores.
        std::set<std::vector<int>> domains;
        for (int c : allowed) {
            std::string l = read_line("/sys/devices/system/cpu/cpu" + std::to_string(c) +
                                      "/cache/index3/shared_cpu_list");
            if (!l.empty()) domains.insert(parse_list(l));
        }
        std::vector<int> best;
        for (auto& d : domains) {
            std::vector<int> in;
            for (int c : d)
                if (cores.count(c)) in.push_back(c);
            if (in.size() > best.size()) best = in;
        }
        if (!best.empty()) chosen = best;
    }
    // cgroup v2 quota.
    std::string quota = read_line("/sys/fs/cgroup/cpu.max");
    if (!quota.empty() && quota.rfind("max", 0) != 0) {
        double q = 0, p = 1;
        if (std::sscanf(quota.c_str(), "%lf %lf", &q, &p) == 2 && p > 0) {
            size_t cap = (size_t)std::max(1.0, std::ceil(q / p));
            if (chosen.size() > cap) chosen.resize(cap);
        }
    }
    if (chosen.empty()) chosen.push_back(0);
    return chosen;
}

void parallel(int n, const std::function<void(int)>& fn) {
    if (!g_team) {
        for (int t = 0; t < n; ++t) fn(t);
        return;
    }
    g_team->run(n, fn);
}

int team_threads() { return g_team ? g_team->size : 1; }

// ----------------------------------------------------------- quantizer ---
int group_code(float scaled) {
    // cvtps2dq then the limits (src/cpu/v2/quantize.rs:140-149).
    float r = std::nearbyint(scaled);
    int whole = (r >= -2147483648.0f && r < 2147483648.0f) ? (int)r : INT32_MIN;
    return std::min(127, std::max(-127, whole));
}

float group_step(float peak) { return peak > 0.0f ? peak / 127.0f : 1.0f; }

// src/cpu/v2/quantize.rs:150-171 (= src/cpu/kernels.rs:769-779 for finite values).
void quantize_group_scalar(const float* src, int n, int8_t* dst, float* scale, int32_t* sum) {
    float peak = 0.0f;
    for (int i = 0; i < n; ++i) peak = std::fmax(peak, std::fabs(src[i]));
    float s = group_step(peak);
    float inv = 1.0f / s;
    int32_t total = 0;
    for (int i = 0; i < n; ++i) {
        int c = group_code(src[i] * inv);
        dst[i] = (int8_t)c;
        total += c;
    }
    *scale = s;
    *sum = total;
}

// src/cpu/kernels.rs:783-807.
AVX512 void quantize_group_avx512(const float* src, int n, int8_t* dst, float* scale, int32_t* sum) {
    __m512 vmax = _mm512_setzero_ps();
    for (int i = 0; i < n; i += 16) vmax = _mm512_max_ps(vmax, _mm512_abs_ps(_mm512_loadu_ps(src + i)));
    float s = group_step(_mm512_reduce_max_ps(vmax));
    __m512 inv = _mm512_set1_ps(1.0f / s);
    __m512i hi = _mm512_set1_epi32(127), lo = _mm512_set1_epi32(-127);
    __m512i vsum = _mm512_setzero_si512();
    for (int i = 0; i < n; i += 16) {
        __m512i q = _mm512_cvtps_epi32(_mm512_mul_ps(_mm512_loadu_ps(src + i), inv));
        q = _mm512_max_epi32(_mm512_min_epi32(q, hi), lo);
        vsum = _mm512_add_epi32(vsum, q);
        _mm_storeu_si128((__m128i*)(dst + i), _mm512_cvtsepi32_epi8(q));
    }
    *scale = s;
    *sum = _mm512_reduce_add_epi32(vsum);
}

// src/cpu/kernels.rs:811-846 (codes stored in order; the sum is order-free).
AVX2T void quantize_group_avx2(const float* src, int n, int8_t* dst, float* scale, int32_t* sum) {
    const __m256 sign = _mm256_set1_ps(-0.0f);
    __m256 vmax = _mm256_setzero_ps();
    for (int i = 0; i < n; i += 8) vmax = _mm256_max_ps(vmax, _mm256_andnot_ps(sign, _mm256_loadu_ps(src + i)));
    float lanes[8];
    _mm256_storeu_ps(lanes, vmax);
    float peak = 0.0f;
    for (float l : lanes) peak = std::fmax(peak, l);
    float s = group_step(peak);
    __m256 inv = _mm256_set1_ps(1.0f / s);
    __m256i hi = _mm256_set1_epi32(127), lo = _mm256_set1_epi32(-127);
    int32_t total = 0;
    for (int i = 0; i < n; i += 8) {
        __m256i q = _mm256_cvtps_epi32(_mm256_mul_ps(_mm256_loadu_ps(src + i), inv));
        q = _mm256_max_epi32(_mm256_min_epi32(q, hi), lo);
        int32_t c[8];
        _mm256_storeu_si256((__m256i*)c, q);
        for (int j = 0; j < 8; ++j) {
            dst[i + j] = (int8_t)c[j];
            total += c[j];
        }
    }
    *scale = s;
    *sum = total;
}

struct Quantized {
    int m = 0, k = 0, group = 0;
    std::vector<int8_t> values;
    std::vector<float> scales;
    std::vector<int32_t> sums;
};

// src/cpu/kernels.rs:661-737: rows in tasks of 8; the stored scale is
// rounded through f16 after the codes are made (half_scales, ggml Q8_0).
void quantize_rows(int isa, const float* x, int m, int k, int group, bool half_scales, Quantized& q) {
    int groups = k / group;
    q.m = m;
    q.k = k;
    q.group = group;
    q.values.resize((size_t)m * k);
    q.scales.resize((size_t)m * groups);
    q.sums.resize((size_t)m * groups);
    parallel((m + 7) / 8, [&](int task) {
        for (int row = task * 8; row < std::min(m, task * 8 + 8); ++row) {
            for (int g = 0; g < groups; ++g) {
                const float* src = x + (size_t)row * k + (size_t)g * group;
                int8_t* dst = q.values.data() + (size_t)row * k + (size_t)g * group;
                float s;
                int32_t sum;
                if (isa == OR_AVX512) {
                    quantize_group_avx512(src, group, dst, &s, &sum);
                } else if (isa == OR_AVX2) {
                    quantize_group_avx2(src, group, dst, &s, &sum);
                } else {
                    quantize_group_scalar(src, group, dst, &s, &sum);
                }
                q.scales[(size_t)row * groups + g] = half_scales ? f16r(s) : s;
                q.sums[(size_t)row * groups + g] = sum;
            }
        }
    });
}

// Tasks of at least MIN_TASK_WORK multiply-adds while each thread still
// gets two (src/cpu/int8.rs:849-873).
constexpr size_t MIN_TASK_WORK = 800000;
void grouped(int units, size_t work, const std::function<void(int)>& run) {
    size_t per = (MIN_TASK_WORK + std::max<size_t>(work, 1) - 1) / std::max<size_t>(work, 1);
    size_t cap = std::max<size_t>(1, (size_t)units / (2 * (size_t)team_threads()));
    per = std::min(std::max<size_t>(per, 1), cap);
    int tasks = (int)((units + per - 1) / per);
    parallel(tasks, [&](int task) {
        for (int u = task * (int)per; u < std::min(units, (task + 1) * (int)per); ++u) run(u);
    });
}

// --------------------------------------------------------- int8 layer ---
// src/cpu/int8.rs:155-289: AVX-512 VNNI packs [n/16][k/4][16][4] bytes as
// w+128, AVX2 [n/8][k/4][8][4]; scales [n/rows][k/group][rows]. The
// contract path keeps row-major codes and scales.
struct Int8Layer {
    int isa, n, k, group;
    bool half_scales;
    std::vector<int8_t> weights;
    std::vector<float> scales;
    int rows() const { return isa == OR_AVX512 ? 16 : isa == OR_AVX2 ? 8 : 1; }
};

Int8Layer* int8_new(int isa, int n, int k, int group, bool half, const int8_t* codes, const float* scales) {
    auto* L = new Int8Layer{isa, n, k, group, half, {}, {}};
    int rows = L->rows(), groups = k / group;
    L->weights.resize((size_t)n * k);
    L->scales.resize((size_t)n * groups);
    for (int row = 0; row < n; ++row) {
        int block = row / rows, r = row % rows;
        for (int g = 0; g < groups; ++g)
            L->scales[((size_t)block * groups + g) * rows + r] = scales[(size_t)row * groups + g];
        for (int kk = 0; kk < k; ++kk) {
            int8_t c = codes[(size_t)row * k + kk];
            if (isa == OR_SCALAR) {
                L->weights[(size_t)row * k + kk] = c;
            } else {
                size_t at = (((size_t)block * (k / 4) + kk / 4) * rows + r) * 4 + kk % 4;
                L->weights[at] = isa == OR_AVX512 ? (int8_t)(c ^ (int8_t)0x80) : c;
            }
        }
    }
    return L;
}

// The contract: total = fma(f32(dot_g), ws_g * xs_g, total) over groups in
// order, from +0 (src/cpu/v2/product.rs:389-423; src/cpu/int8.rs:560-569).
void int8_scalar_row(const Int8Layer& L, const Quantized& q, int row, float* out) {
    int k = L.k, group = L.group, groups = k / group;
    for (int f = 0; f < q.m; ++f) {
        float total = 0.0f;
        for (int g = 0; g < groups; ++g) {
            int32_t dot = 0;
            for (int kk = g * group; kk < (g + 1) * group; ++kk)
                dot += (int32_t)L.weights[(size_t)row * k + kk] * (int32_t)q.values[(size_t)f * k + kk];
            float scale = L.scales[(size_t)row * groups + g] * q.scales[(size_t)f * groups + g];
            total = std::fmaf((float)dot, scale, total);
        }
        out[(size_t)f * L.n + row] = total;
    }
}

// src/cpu/int8.rs:524-584: two 16-row blocks by F frames.
template <int F>
AVX512 void int8_vnni_tile(const Int8Layer& L, const Quantized& q, int task, int frame0, float* out) {
    int k = L.k, k4s = k / 4, groups = k / L.group, quads = L.group / 4;
    int blocks[2] = {2 * task, 2 * task + 1};
    __m512 acc[2][F];
    #pragma GCC unroll 16
    for (int b = 0; b < 2; ++b)
        #pragma GCC unroll 16
        for (int f = 0; f < F; ++f) acc[b][f] = _mm512_setzero_ps();
    const int8_t* W = L.weights.data();
    for (int g = 0; g < groups; ++g) {
        __m512i dots[2][F];
        #pragma GCC unroll 16
        for (int b = 0; b < 2; ++b)
            #pragma GCC unroll 16
            for (int f = 0; f < F; ++f) dots[b][f] = _mm512_setzero_si512();
        for (int k4 = g * quads; k4 < (g + 1) * quads; ++k4) {
            __m512i w0 = _mm512_loadu_si512(W + ((size_t)blocks[0] * k4s + k4) * 64);
            __m512i w1 = _mm512_loadu_si512(W + ((size_t)blocks[1] * k4s + k4) * 64);
            #pragma GCC unroll 16
            for (int f = 0; f < F; ++f) {
                int32_t xv;
                std::memcpy(&xv, q.values.data() + (size_t)(frame0 + f) * k + k4 * 4, 4);
                __m512i x = _mm512_set1_epi32(xv);
                dots[0][f] = _mm512_dpbusd_epi32(dots[0][f], w0, x);
                dots[1][f] = _mm512_dpbusd_epi32(dots[1][f], w1, x);
            }
        }
        #pragma GCC unroll 16
        for (int b = 0; b < 2; ++b) {
            __m512 ws = _mm512_loadu_ps(L.scales.data() + ((size_t)blocks[b] * groups + g) * 16);
            #pragma GCC unroll 16
            for (int f = 0; f < F; ++f) {
                size_t index = (size_t)(frame0 + f) * groups + g;
                __m512i corrected = _mm512_sub_epi32(dots[b][f], _mm512_set1_epi32(128 * q.sums[index]));
                __m512 scale = _mm512_mul_ps(ws, _mm512_set1_ps(q.scales[index]));
                acc[b][f] = _mm512_fmadd_ps(_mm512_cvtepi32_ps(corrected), scale, acc[b][f]);
            }
        }
    }
    #pragma GCC unroll 16
    for (int b = 0; b < 2; ++b)
        #pragma GCC unroll 16
        for (int f = 0; f < F; ++f) _mm512_storeu_ps(out + (size_t)(frame0 + f) * L.n + blocks[b] * 16, acc[b][f]);
}

AVX512 void int8_vnni_task(const Int8Layer& L, const Quantized& q, int task, float* out) {
    int frame = 0;
    while (frame + 6 <= q.m) {
        int8_vnni_tile<6>(L, q, task, frame, out);
        frame += 6;
    }
    switch (q.m - frame) {
        case 1: int8_vnni_tile<1>(L, q, task, frame, out); break;
        case 2: int8_vnni_tile<2>(L, q, task, frame, out); break;
        case 3: int8_vnni_tile<3>(L, q, task, frame, out); break;
        case 4: int8_vnni_tile<4>(L, q, task, frame, out); break;
        case 5: int8_vnni_tile<5>(L, q, task, frame, out); break;
        default: break;
    }
}

// src/cpu/int8.rs:615-655: 8 rows by F frames, the sign trick.
template <int F>
AVX2T void int8_avx2_tile(const Int8Layer& L, const Quantized& q, int block, int frame0, float* out) {
    int k = L.k, k4s = k / 4, groups = k / L.group, quads = L.group / 4;
    const __m256i ones = _mm256_set1_epi16(1);
    __m256 acc[F];
    #pragma GCC unroll 16
    for (int f = 0; f < F; ++f) acc[f] = _mm256_setzero_ps();
    for (int g = 0; g < groups; ++g) {
        __m256i dots[F];
        #pragma GCC unroll 16
        for (int f = 0; f < F; ++f) dots[f] = _mm256_setzero_si256();
        for (int k4 = g * quads; k4 < (g + 1) * quads; ++k4) {
            __m256i w = _mm256_loadu_si256((const __m256i*)(L.weights.data() + ((size_t)block * k4s + k4) * 32));
            __m256i mag = _mm256_abs_epi8(w);
            #pragma GCC unroll 16
            for (int f = 0; f < F; ++f) {
                int32_t xv;
                std::memcpy(&xv, q.values.data() + (size_t)(frame0 + f) * k + k4 * 4, 4);
                __m256i x = _mm256_set1_epi32(xv);
                __m256i pairs = _mm256_maddubs_epi16(mag, _mm256_sign_epi8(x, w));
                dots[f] = _mm256_add_epi32(dots[f], _mm256_madd_epi16(pairs, ones));
            }
        }
        __m256 ws = _mm256_loadu_ps(L.scales.data() + ((size_t)block * groups + g) * 8);
        #pragma GCC unroll 16
        for (int f = 0; f < F; ++f) {
            __m256 scale = _mm256_mul_ps(ws, _mm256_set1_ps(q.scales[(size_t)(frame0 + f) * groups + g]));
            acc[f] = _mm256_fmadd_ps(_mm256_cvtepi32_ps(dots[f]), scale, acc[f]);
        }
    }
    #pragma GCC unroll 16
    for (int f = 0; f < F; ++f) _mm256_storeu_ps(out + (size_t)(frame0 + f) * L.n + block * 8, acc[f]);
}

AVX2T void int8_avx2_task(const Int8Layer& L, const Quantized& q, int block, float* out) {
    int frame = 0;
    while (frame + 4 <= q.m) {
        int8_avx2_tile<4>(L, q, block, frame, out);
        frame += 4;
    }
    switch (q.m - frame) {
        case 1: int8_avx2_tile<1>(L, q, block, frame, out); break;
        case 2: int8_avx2_tile<2>(L, q, block, frame, out); break;
        case 3: int8_avx2_tile<3>(L, q, block, frame, out); break;
        default: break;
    }
}

// src/cpu/int8.rs:425-483.
void int8_forward(const Int8Layer& L, const float* x, int m, float* out) {
    Quantized q;
    quantize_rows(L.isa, x, m, L.k, L.group, L.half_scales, q);
    int rows = L.rows();
    size_t block_work = (size_t)m * L.k * rows;
    if (L.isa == OR_AVX512) {
        grouped(L.n / (2 * rows), 2 * block_work, [&](int t) { int8_vnni_task(L, q, t, out); });
    } else if (L.isa == OR_AVX2) {
        grouped(L.n / rows, block_work, [&](int b) { int8_avx2_task(L, q, b, out); });
    } else {
        grouped(L.n, (size_t)m * L.k, [&](int r) { int8_scalar_row(L, q, r, out); });
    }
}

// ------------------------------------------------------ ternary layer ---
// src/cpu/kernels.rs:620-628: bits 2s..2s+2 of byte j hold code 4s+j of a
// 16-code span.
void pack_span(const uint8_t* codes, uint8_t* out4) {
    for (int j = 0; j < 4; ++j)
        out4[j] = (uint8_t)(codes[j] | codes[4 + j] << 2 | codes[8 + j] << 4 | codes[12 + j] << 6);
}

struct TernaryLayer {
    int isa, n, k;
    std::vector<uint8_t> codes;  // contract: row-major codes; SIMD: [n/16][k/16][16][4]
    std::vector<float> scales;   // contract: row-major n*(k/128); SIMD: [n/16][G][16]
};
constexpr int TGROUP = 128;

TernaryLayer* ternary_new(int isa, int n, int k, const uint8_t* codes, const float* scales) {
    // Trit falls back to the scalar tile unless k % 128 == 0 and n % 32 == 0
    // (src/cpu/kernels.rs:156-161); AVX2 keeps the contract path here.
    if (isa != OR_SCALAR && (k % TGROUP != 0 || n % 32 != 0 || isa == OR_AVX2)) isa = OR_SCALAR;
    auto* L = new TernaryLayer{isa, n, k, {}, {}};
    int groups = k / TGROUP;
    if (isa == OR_SCALAR) {
        L->codes.assign(codes, codes + (size_t)n * k);
        L->scales.assign(scales, scales + (size_t)n * groups);
        return L;
    }
    int rows = 16;
    L->codes.resize((size_t)n * k / 4);
    L->scales.resize((size_t)n * groups);
    for (int block = 0; block < n / rows; ++block) {
        for (int k16 = 0; k16 < k / 16; ++k16)
            for (int r = 0; r < rows; ++r)
                pack_span(codes + (size_t)(block * rows + r) * k + k16 * 16,
                          L->codes.data() + (((size_t)block * (k / 16) + k16) * rows + r) * 4);
        for (int g = 0; g < groups; ++g)
            for (int r = 0; r < rows; ++r)
                L->scales[((size_t)block * groups + g) * rows + r] = scales[(size_t)(block * rows + r) * groups + g];
    }
    return L;
}

// Contract: dot = sum(code*q) - sum(q) = sum((code-1)*q), then the same
// f32 chain as the int8 product (src/cpu/kernels.rs:396-406).
void ternary_scalar_row(const TernaryLayer& L, const Quantized& q, int row, float* out) {
    int k = L.k, groups = k / TGROUP;
    for (int f = 0; f < q.m; ++f) {
        float total = 0.0f;
        for (int g = 0; g < groups; ++g) {
            int32_t s = 0;
            for (int kk = g * TGROUP; kk < (g + 1) * TGROUP; ++kk)
                s += (int32_t)L.codes[(size_t)row * k + kk] * (int32_t)q.values[(size_t)f * k + kk];
            int32_t dot = s - q.sums[(size_t)f * groups + g];
            float scale = L.scales[(size_t)row * groups + g] * q.scales[(size_t)f * groups + g];
            total = std::fmaf((float)dot, scale, total);
        }
        out[(size_t)f * L.n + row] = total;
    }
}

// src/cpu/kernels.rs:346-420.
template <int F>
AVX512 void ternary_vnni_tile(const TernaryLayer& L, const Quantized& q, int task, int frame0, float* out) {
    int k = L.k, k16s = k / 16, groups = k / TGROUP;
    int blocks[2] = {2 * task, 2 * task + 1};
    const __m512i low = _mm512_set1_epi8(3);
    __m512 acc[2][F];
    #pragma GCC unroll 16
    for (int b = 0; b < 2; ++b)
        #pragma GCC unroll 16
        for (int f = 0; f < F; ++f) acc[b][f] = _mm512_setzero_ps();
    for (int g = 0; g < groups; ++g) {
        __m512i dots[2][F];
        #pragma GCC unroll 16
        for (int b = 0; b < 2; ++b)
            #pragma GCC unroll 16
            for (int f = 0; f < F; ++f) dots[b][f] = _mm512_setzero_si512();
        for (int quad = 0; quad < TGROUP / 16; ++quad) {
            int k16 = g * (TGROUP / 16) + quad;
            __m512i w[2][4];
            #pragma GCC unroll 16
            for (int b = 0; b < 2; ++b) {
                __m512i z = _mm512_loadu_si512(L.codes.data() + ((size_t)blocks[b] * k16s + k16) * 64);
                w[b][0] = _mm512_and_si512(z, low);
                w[b][1] = _mm512_and_si512(_mm512_srli_epi16(z, 2), low);
                w[b][2] = _mm512_and_si512(_mm512_srli_epi16(z, 4), low);
                w[b][3] = _mm512_and_si512(_mm512_srli_epi16(z, 6), low);
            }
            for (int s = 0; s < 4; ++s) {
                int k4 = 4 * k16 + s;
                #pragma GCC unroll 16
                for (int f = 0; f < F; ++f) {
                    int32_t xv;
                    std::memcpy(&xv, q.values.data() + (size_t)(frame0 + f) * k + k4 * 4, 4);
                    __m512i x = _mm512_set1_epi32(xv);
                    dots[0][f] = _mm512_dpbusd_epi32(dots[0][f], w[0][s], x);
                    dots[1][f] = _mm512_dpbusd_epi32(dots[1][f], w[1][s], x);
                }
            }
        }
        #pragma GCC unroll 16
        for (int b = 0; b < 2; ++b) {
            __m512 ws = _mm512_loadu_ps(L.scales.data() + ((size_t)blocks[b] * groups + g) * 16);
            #pragma GCC unroll 16
            for (int f = 0; f < F; ++f) {
                size_t index = (size_t)(frame0 + f) * groups + g;
                __m512i corrected = _mm512_sub_epi32(dots[b][f], _mm512_set1_epi32(q.sums[index]));
                __m512 scale = _mm512_mul_ps(ws, _mm512_set1_ps(q.scales[index]));
                acc[b][f] = _mm512_fmadd_ps(_mm512_cvtepi32_ps(corrected), scale, acc[b][f]);
            }
        }
    }
    #pragma GCC unroll 16
    for (int b = 0; b < 2; ++b)
        #pragma GCC unroll 16
        for (int f = 0; f < F; ++f) _mm512_storeu_ps(out + (size_t)(frame0 + f) * L.n + blocks[b] * 16, acc[b][f]);
}

AVX512 void ternary_vnni_task(const TernaryLayer& L, const Quantized& q, int task, float* out) {
    int frame = 0;
    while (frame + 6 <= q.m) {
        ternary_vnni_tile<6>(L, q, task, frame, out);
        frame += 6;
    }
    switch (q.m - frame) {
        case 1: ternary_vnni_tile<1>(L, q, task, frame, out); break;
        case 2: ternary_vnni_tile<2>(L, q, task, frame, out); break;
        case 3: ternary_vnni_tile<3>(L, q, task, frame, out); break;
        case 4: ternary_vnni_tile<4>(L, q, task, frame, out); break;
        case 5: ternary_vnni_tile<5>(L, q, task, frame, out); break;
        default: break;
    }
}

void ternary_forward(const TernaryLayer& L, const float* x, int m, float* out) {
    Quantized q;
    quantize_rows(L.isa, x, m, L.k, TGROUP, false, q);
    if (L.isa == OR_AVX512) {
        parallel(L.n / 32, [&](int t) { ternary_vnni_task(L, q, t, out); });
    } else {
        parallel(L.n, [&](int r) { ternary_scalar_row(L, q, r, out); });
    }
}

// ----------------------------------------------------- float products ---
// The 16-lane tree of _mm512_reduce_add_ps (src/cpu/v2/float.rs:255-270).
float reduce16(const float* l) {
    float half[8];
    for (int i = 0; i < 8; ++i) half[i] = l[i] + l[i + 8];
    float q[4] = {half[0] + half[4], half[1] + half[5], half[2] + half[6], half[3] + half[7]};
    float p0 = q[0] + q[2], p1 = q[1] + q[3];
    return p0 + p1;
}

template <typename W>
float widen(W w);
template <>
float widen<uint16_t>(uint16_t w) { return f16_to_f32(w); }
template <>
float widen<float>(float w) { return w; }

// Contract (src/cpu/v2/float.rs:1-30,687-718): lane i adds
// x[16j+i]*w[16j+i] fused, in j order; tail padded with zeros; the tree.
template <typename W>
float dot16(const float* x, const W* w, int k) {
    float lanes[16] = {0};
    int j = 0;
    for (; j + 16 <= k; j += 16)
        for (int i = 0; i < 16; ++i) lanes[i] = std::fmaf(x[j + i], widen(w[j + i]), lanes[i]);
    if (j < k) {
        for (int i = 0; i < 16; ++i) {
            float xv = j + i < k ? x[j + i] : 0.0f, wv = j + i < k ? widen(w[j + i]) : 0.0f;
            lanes[i] = std::fmaf(xv, wv, lanes[i]);
        }
    }
    return reduce16(lanes);
}

AVX512 __m512 load16(const uint16_t* p) { return _mm512_cvtph_ps(_mm256_loadu_si256((const __m256i*)p)); }
AVX512 __m512 load16(const float* p) { return _mm512_loadu_ps(p); }
AVX512 __m512 load16_first(const uint16_t* p, int count) {
    return _mm512_cvtph_ps(_mm256_maskz_loadu_epi16((__mmask16)((1u << count) - 1), p));
}
AVX512 __m512 load16_first(const float* p, int count) {
    return _mm512_maskz_loadu_ps((__mmask16)((1u << count) - 1), p);
}

AVX512 float reduce512(__m512 v) {
    alignas(64) float l[16];
    _mm512_store_ps(l, v);
    return reduce16(l);
}

// src/cpu/fgemm.rs:402-455: R x C tile of 16-lane sums.
template <int R, int C, typename W>
AVX512 void f_tile512(const float* x, const W* w, int k, float* out, int n) {
    __m512 acc[R][C];
    #pragma GCC unroll 16
    for (int r = 0; r < R; ++r)
        for (int c = 0; c < C; ++c) acc[r][c] = _mm512_setzero_ps();
    int kk = 0;
    for (; kk + 16 <= k; kk += 16) {
        __m512 wv[C];
        for (int c = 0; c < C; ++c) wv[c] = load16(w + (size_t)c * k + kk);
        #pragma GCC unroll 16
        for (int r = 0; r < R; ++r) {
            __m512 xv = _mm512_loadu_ps(x + (size_t)r * k + kk);
            for (int c = 0; c < C; ++c) acc[r][c] = _mm512_fmadd_ps(xv, wv[c], acc[r][c]);
        }
    }
    if (kk < k) {
        __mmask16 mask = (__mmask16)((1u << (k - kk)) - 1);
        __m512 wv[C];
        for (int c = 0; c < C; ++c) wv[c] = load16_first(w + (size_t)c * k + kk, k - kk);
        #pragma GCC unroll 16
        for (int r = 0; r < R; ++r) {
            __m512 xv = _mm512_maskz_loadu_ps(mask, x + (size_t)r * k + kk);
            for (int c = 0; c < C; ++c) acc[r][c] = _mm512_fmadd_ps(xv, wv[c], acc[r][c]);
        }
    }
    #pragma GCC unroll 16
    for (int r = 0; r < R; ++r)
        for (int c = 0; c < C; ++c) out[(size_t)r * n + c] = reduce512(acc[r][c]);
}

template <typename W>
AVX512 void f_block512(const float* x, int k, const W* w, int n, int r0, int r1, int c0, int c1, float* out) {
    int i = r0;
    while (i < r1) {
        int left = r1 - i;
        int r = (left <= 3 || left == 5) ? left : 4;
        int j = c0;
        while (j < c1) {
            int c = std::min(3, c1 - j);
            const float* xp = x + (size_t)i * k;
            const W* wp = w + (size_t)j * k;
            float* op = out + (size_t)i * n + j;
#define TILE(RR, CC) \
    if (r == RR && c == CC) f_tile512<RR, CC, W>(xp, wp, k, op, n);
            TILE(5, 3) TILE(5, 2) TILE(5, 1) TILE(4, 3) TILE(4, 2) TILE(4, 1) TILE(3, 3) TILE(3, 2)
            TILE(3, 1) TILE(2, 3) TILE(2, 2) TILE(2, 1) TILE(1, 3) TILE(1, 2) TILE(1, 1)
#undef TILE
            j += c;
        }
        i += r;
    }
}

// src/cpu/fgemm.rs:497-560: the first set's 8-lane AVX2 tile with its
// hsum tree and a k tail added value by value.
template <typename W>
AVX2T float dot8_avx2(const float* x, const W* w, int k) {
    __m256 acc = _mm256_setzero_ps();
    int kk = 0;
    for (; kk + 8 <= k; kk += 8) {
        __m256 wv;
        if constexpr (sizeof(W) == 2) {
            wv = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(w + kk)));
        } else {
            wv = _mm256_loadu_ps((const float*)(w + kk));
        }
        acc = _mm256_fmadd_ps(_mm256_loadu_ps(x + kk), wv, acc);
    }
    __m128 pair = _mm_add_ps(_mm256_castps256_ps128(acc), _mm256_extractf128_ps(acc, 1));
    __m128 quad = _mm_add_ps(pair, _mm_movehl_ps(pair, pair));
    float total = _mm_cvtss_f32(_mm_add_ss(quad, _mm_shuffle_ps(quad, quad, 1)));
    for (; kk < k; ++kk) total += x[kk] * widen(w[kk]);
    return total;
}

template <typename W>
void matmul(int isa, const float* x, int m, int k, const W* w, int n, float* out) {
    const int B = 64;
    int rb = (m + B - 1) / B, cb = (n + B - 1) / B;
    parallel(rb * cb, [&](int task) {
        int r0 = (task / cb) * B, r1 = std::min(m, r0 + B);
        int c0 = (task % cb) * B, c1 = std::min(n, c0 + B);
        if (isa == OR_AVX512) {
            f_block512<W>(x, k, w, n, r0, r1, c0, c1, out);
            return;
        }
        for (int i = r0; i < r1; ++i)
            for (int j = c0; j < c1; ++j)
                out[(size_t)i * n + j] = isa == OR_AVX2 ? dot8_avx2(x + (size_t)i * k, w + (size_t)j * k, k)
                                                        : dot16(x + (size_t)i * k, w + (size_t)j * k, k);
    });
}

// --------------------------------------------------------------- layers ---
// src/layers.rs:136-144: a serial sum of squares, inv = 1/sqrt(sum/d + eps),
// v *= inv * w.
void rmsnorm_row(const float* w, int d, float eps, float* x) {
    float sum = 0.0f;
    for (int i = 0; i < d; ++i) sum += x[i] * x[i];
    float inv = 1.0f / std::sqrt(sum / (float)d + eps);
    for (int i = 0; i < d; ++i) x[i] *= inv * w[i];
}

void rope_table(int dims, float base, int positions, float* sn, float* cs) {
    int half = dims / 2;
    std::vector<float> inv(half);
    for (int i = 0; i < half; ++i) inv[i] = std::pow(base, -(float)(2 * i) / (float)dims);
    for (int p = 0; p < positions; ++p)
        for (int i = 0; i < half; ++i) {
            float angle = (float)p * inv[i];
            sn[(size_t)p * half + i] = std::sin(angle);
            cs[(size_t)p * half + i] = std::cos(angle);
        }
}

// src/layers.rs:303-334 (halves): a' = a*cos - b*sin, b' = b*cos + a*sin.
void rope_apply(float* x, int rows, int stride, int heads, int hd, int first, const float* sn, const float* cs) {
    int half = hd / 2;
    for (int r = 0; r < rows; ++r) {
        const float* s = sn + (size_t)(first + r) * half;
        const float* c = cs + (size_t)(first + r) * half;
        for (int h = 0; h < heads; ++h) {
            float* head = x + (size_t)r * stride + (size_t)h * hd;
            for (int i = 0; i < half; ++i) {
                float a = head[i], b = head[i + half];
                float ac = a * c[i], bs = b * s[i];
                float bc = b * c[i], as = a * s[i];
                head[i] = ac - bs;
                head[i + half] = bc + as;
            }
        }
    }
}

// src/layers.rs:442-504,571-587 with the AVX-512 tiles of
// src/cpu/fgemm.rs:665-793 and src/cpu/activation.rs:214-275: per query,
// qh = q * (1/sqrt(hd)); score_j = fused chain over e from 0; masked keys
// are -inf; max; e_j = exp(s_j - max) (masked: exp of the clamp low end);
// sum in key order from 0; p_j = e_j * (1/sum); out_e = fused chain of
// p_j * v_je over j from 0.
void attention_head_scalar(const float* qrow, const float* kbase, const float* vbase, int kvs, int tk, int visible,
                           int hd, float scale, float* out, std::vector<float>& probs) {
    std::vector<float> qh(hd);
    for (int e = 0; e < hd; ++e) qh[e] = qrow[e] * scale;
    probs.resize(tk);
    for (int j = 0; j < tk; ++j) {
        float acc = 0.0f;
        const float* kr = kbase + (size_t)j * kvs;
        for (int e = 0; e < hd; ++e) acc = std::fmaf(qh[e], kr[e], acc);
        probs[j] = j < visible ? acc : -INFINITY;
    }
    float mx = -INFINITY;
    for (int j = 0; j < tk; ++j) mx = std::fmax(mx, probs[j]);
    float sum = 0.0f;
    for (int j = 0; j < tk; ++j) {
        probs[j] = exp_contract(probs[j] - mx);
        sum += probs[j];
    }
    float inv = 1.0f / sum;
    for (int j = 0; j < tk; ++j) probs[j] *= inv;
    for (int e = 0; e < hd; ++e) {
        float acc = 0.0f;
        for (int j = 0; j < tk; ++j) acc = std::fmaf(probs[j], vbase[(size_t)j * kvs + e], acc);
        out[e] = acc;
    }
}

// The same values with keys transposed per head (HeadMajor,
// src/layers.rs:362-430) and 16-wide vectors, for the timed baseline.
AVX512 void attention_head_512(const float* qrow, const float* kt, const float* vh, int tk, int visible, int hd,
                               float scale, float* out, float* probs) {
    alignas(64) float qh[256];
    for (int e = 0; e < hd; ++e) qh[e] = qrow[e] * scale;
    int j = 0;
    for (; j < tk; j += 16) {
        int cnt = std::min(16, tk - j);
        __mmask16 mask = (__mmask16)((1u << cnt) - 1);
        __m512 acc = _mm512_setzero_ps();
        for (int e = 0; e < hd; ++e)
            acc = _mm512_fmadd_ps(_mm512_set1_ps(qh[e]), _mm512_maskz_loadu_ps(mask, kt + (size_t)e * tk + j), acc);
        _mm512_mask_storeu_ps(probs + j, mask, acc);
    }
    for (int t = visible; t < tk; ++t) probs[t] = -INFINITY;
    __m512 best = _mm512_set1_ps(-INFINITY);
    for (j = 0; j + 16 <= tk; j += 16) best = _mm512_max_ps(_mm512_loadu_ps(probs + j), best);
    float mx = _mm512_reduce_max_ps(best);
    for (; j < tk; ++j) mx = std::fmax(mx, probs[j]);
    __m512 shift = _mm512_set1_ps(mx);
    for (j = 0; j < tk; j += 16) {
        int cnt = std::min(16, tk - j);
        __mmask16 mask = (__mmask16)((1u << cnt) - 1);
        __m512 e = exp512(_mm512_sub_ps(_mm512_maskz_loadu_ps(mask, probs + j), shift));
        _mm512_mask_storeu_ps(probs + j, mask, e);
    }
    float sum = 0.0f;
    for (j = 0; j < tk; ++j) sum += probs[j];
    __m512 inv = _mm512_set1_ps(1.0f / sum);
    for (j = 0; j < tk; j += 16) {
        int cnt = std::min(16, tk - j);
        __mmask16 mask = (__mmask16)((1u << cnt) - 1);
        _mm512_mask_storeu_ps(probs + j, mask, _mm512_mul_ps(_mm512_maskz_loadu_ps(mask, probs + j), inv));
    }
    for (int e0 = 0; e0 < hd; e0 += 16) {
        int cnt = std::min(16, hd - e0);
        __mmask16 mask = (__mmask16)((1u << cnt) - 1);
        __m512 acc = _mm512_setzero_ps();
        for (j = 0; j < tk; ++j)
            acc = _mm512_fmadd_ps(_mm512_set1_ps(probs[j]), _mm512_maskz_loadu_ps(mask, vh + (size_t)j * hd + e0), acc);
        _mm512_mask_storeu_ps(out + e0, mask, acc);
    }
}

void attention(int isa, const float* q, int qs, const float* k, const float* v, int kvs, int tq, int tk, int heads,
               int kv_heads, int hd, bool causal, float* out) {
    if (tq == 0) return;
    int group = heads / kv_heads;
    float scale = 1.0f / std::sqrt((float)hd);
    int d = heads * hd;
    const int CH = 128;
    int chunk = std::min(CH, tq), chunks = (tq + chunk - 1) / chunk;
    if (isa == OR_AVX512 && hd <= 256) {
        std::vector<float> kt((size_t)kv_heads * hd * tk), vh((size_t)kv_heads * tk * hd);
        parallel(kv_heads, [&](int g) {
            for (int j = 0; j < tk; ++j)
                for (int e = 0; e < hd; ++e) {
                    kt[(size_t)g * hd * tk + (size_t)e * tk + j] = k[(size_t)j * kvs + g * hd + e];
                    vh[(size_t)g * tk * hd + (size_t)j * hd + e] = v[(size_t)j * kvs + g * hd + e];
                }
        });
        parallel(heads * chunks, [&](int task) {
            int h = task / chunks, c = task % chunks;
            std::vector<float> probs(tk);
            for (int i = c * chunk; i < std::min(tq, (c + 1) * chunk); ++i) {
                int visible = causal ? tk - tq + i + 1 : tk;
                attention_head_512(q + (size_t)i * qs + h * hd, kt.data() + (size_t)(h / group) * hd * tk,
                                   vh.data() + (size_t)(h / group) * tk * hd, tk, visible, hd, scale,
                                   out + (size_t)i * d + h * hd, probs.data());
            }
        });
        return;
    }
    parallel(heads * chunks, [&](int task) {
        int h = task / chunks, c = task % chunks;
        std::vector<float> probs;
        for (int i = c * chunk; i < std::min(tq, (c + 1) * chunk); ++i) {
            int visible = causal ? tk - tq + i + 1 : tk;
            attention_head_scalar(q + (size_t)i * qs + h * hd, k + (size_t)(h / group) * hd,
                                  v + (size_t)(h / group) * hd, kvs, tk, visible, hd, scale,
                                  out + (size_t)i * d + h * hd, probs);
        }
    });
}

int argmax(const float* v, int n) {
    int best = 0;
    for (int i = 0; i < n; ++i)
        if (v[i] > v[best]) best = i;
    return best;
}

// ------------------------------------------------------------- decoder ---
// A token table (Dense::table / Dense::row, src/cpu/gemm.rs:383-429): f16
// bits, f32, or int8 storage with one f32 scale per 32 values (Q8,
// :37-44,117-187), always with f32 math in the 16-lane order.
struct Table {
    int kind = OR_TABLE_F16, rows = 0, cols = 0;
    std::vector<uint16_t> f16;
    std::vector<float> f32;
    std::vector<int8_t> codes;
    std::vector<float> scales;  // rows x cols/32

    // widen_q8 (src/cpu/gemm.rs:171-179): f32(code) * scale, one rounding.
    void widen_rows(int r0, int r1, float* out) const {
        const int g = cols / 32;
        for (int r = r0; r < r1; ++r)
            for (int kk = 0; kk < cols; ++kk)
                out[(size_t)(r - r0) * cols + kk] =
                    (float)codes[(size_t)r * cols + kk] * scales[(size_t)r * g + kk / 32];
    }
    void row(int index, float* out) const {
        if (kind == OR_TABLE_F16) {
            for (int i = 0; i < cols; ++i) out[i] = f16_to_f32(f16[(size_t)index * cols + i]);
        } else if (kind == OR_TABLE_F32) {
            std::memcpy(out, f32.data() + (size_t)index * cols, (size_t)cols * 4);
        } else {
            widen_rows(index, index + 1, out);
        }
    }
    // out = x * table^T for one row x (Dense::forward of a table,
    // src/cpu/gemm.rs:522-525; Q8::matmul widens panels of rows and runs the
    // f32 product, fgemm.rs:263-295, so each value is the f32 product's).
    void product(int isa, const float* x, float* out) const {
        if (kind == OR_TABLE_F16) return matmul<uint16_t>(isa, x, 1, cols, f16.data(), rows, out);
        if (kind == OR_TABLE_F32) return matmul<float>(isa, x, 1, cols, f32.data(), rows, out);
        const int P = 4096;
        std::vector<float> panel((size_t)P * cols);
        for (int r0 = 0; r0 < rows; r0 += P) {
            const int r1 = std::min(rows, r0 + P);
            widen_rows(r0, r1, panel.data());
            matmul<float>(isa, x, 1, cols, panel.data(), r1 - r0, out + r0);
        }
    }
};

// A decoder linear (Dense, src/cpu/gemm.rs:15-35): int8 activations
// (Q8_0 or Trit's int8), or f16 / f32 weights with f32 math (matmul,
// fgemm.rs:213-246).
struct Linear {
    Int8Layer* int8 = nullptr;
    int fkind = -1, n = 0, k = 0;  // OR_TABLE_F16 / OR_TABLE_F32 without int8
    std::vector<uint16_t> f16;
    std::vector<float> f32;
    Linear() = default;
    Linear(const Linear&) = delete;
    Linear& operator=(const Linear&) = delete;
    Linear(Linear&& o) noexcept
        : int8(o.int8), fkind(o.fkind), n(o.n), k(o.k), f16(std::move(o.f16)), f32(std::move(o.f32)) {
        o.int8 = nullptr;
    }
    ~Linear() { delete int8; }
    void set_int8(Int8Layer* L) {
        delete int8;
        int8 = L;
        fkind = -1;
        f16.clear();
        f32.clear();
    }
    void forward(int isa, const float* x, int m, float* out) const {
        if (int8) return int8_forward(*int8, x, m, out);
        if (fkind == OR_TABLE_F16) return matmul<uint16_t>(isa, x, m, k, f16.data(), n, out);
        return matmul<float>(isa, x, m, k, f32.data(), n, out);
    }
};

struct Lm {
    int isa;
    or_lm_config c;
    struct Layer {
        Linear qkv, o, gate_up, down;
        std::vector<float> norm_attn, norm_mlp, q_norm, k_norm;
    };
    std::vector<Layer> layers;
    Table embed;
    Table head;  // rows == 0: tied to embed
    std::vector<float> final_norm;
    std::vector<std::vector<float>> ffn_scales;  // empty, or layers x d
    std::vector<float> rope_sin, rope_cos;
    int rope_positions = 0;
    // Session: f32 caches per layer, positions x (kv_heads*hd).
    std::vector<std::vector<float>> keys, values;
    int position = 0;

    void ensure_rope(int positions) {
        if (positions <= rope_positions) return;
        int n = std::max(positions, 2 * rope_positions);
        int half = c.head_dim / 2;
        rope_sin.resize((size_t)n * half);
        rope_cos.resize((size_t)n * half);
        rope_table(c.head_dim, c.rope_base, n, rope_sin.data(), rope_cos.data());
        rope_positions = n;
    }

};

Int8Layer* q8_layer(int isa, int n, int k, const uint8_t* blocks) {
    size_t nb = (size_t)n * k / 32;
    std::vector<int8_t> codes((size_t)n * k);
    std::vector<float> scales(nb);
    or_q8_0_parse(blocks, (int64_t)nb, codes.data(), scales.data());
    return int8_new(isa, n, k, 32, true, codes.data(), scales.data());
}

// add_scaled_into (src/layers.rs:224-236): x += y, or x += w * y (no fused
// multiply-add) for a multiplier other than 1.
void add_scaled(float* x, const float* y, size_t n, float w) {
    if (w == 1.0f) {
        for (size_t i = 0; i < n; ++i) x[i] += y[i];
    } else {
        for (size_t i = 0; i < n; ++i) x[i] += w * y[i];
    }
}

// scale_all (src/layers.rs:218-222): nothing for 1.
void scale_all(float* x, size_t n, float w) {
    if (w != 1.0f)
        for (size_t i = 0; i < n; ++i) x[i] *= w;
}

// src/models/parts/causal_lm.rs:374-389,410-481 for rows of embeddings x:
// CausalLm::hidden, the final norm of the last row, the head and the
// logits scaling.
void lm_forward_rows(Lm& lm, std::vector<float>& x, int m, float* logits) {
    const auto& c = lm.c;
    int d = c.d, hd = c.head_dim, qd = c.heads * hd, kv = c.kv_heads * hd, stride = qd + 2 * kv;
    int first = lm.position;
    lm.ensure_rope(first + m);
    scale_all(x.data(), x.size(), c.embedding_multiplier);
    // Granite's attention multiplier replaces 1/sqrt(head_dim)
    // (causal_lm.rs:419-424): q is scaled by multiplier * sqrt(hd) first.
    const float q_scale = c.attention_multiplier != 0.0f ? c.attention_multiplier * std::sqrt((float)hd) : 1.0f;
    std::vector<float> normed((size_t)m * d), qkv((size_t)m * stride), att((size_t)m * qd), y((size_t)m * d);
    std::vector<float> wide((size_t)m * 2 * c.ffn), hidden((size_t)m * c.ffn);
    for (int l = 0; l < c.layers; ++l) {
        auto& L = lm.layers[l];
        normed = x;
        parallel(m, [&](int r) { rmsnorm_row(L.norm_attn.data(), d, c.eps, normed.data() + (size_t)r * d); });
        L.qkv.forward(lm.isa, normed.data(), m, qkv.data());
        if (c.qk_norm) {
            parallel(m, [&](int r) {
                float* row = qkv.data() + (size_t)r * stride;
                for (int h = 0; h < c.heads; ++h) rmsnorm_row(L.q_norm.data(), hd, c.eps, row + (size_t)h * hd);
                for (int h = 0; h < c.kv_heads; ++h)
                    rmsnorm_row(L.k_norm.data(), hd, c.eps, row + qd + (size_t)h * hd);
            });
        }
        rope_apply(qkv.data(), m, stride, c.heads, hd, first, lm.rope_sin.data(), lm.rope_cos.data());
        rope_apply(qkv.data() + qd, m, stride, c.kv_heads, hd, first, lm.rope_sin.data(), lm.rope_cos.data());
        if (q_scale != 1.0f)
            for (int r = 0; r < m; ++r)
                for (int i = 0; i < qd; ++i) qkv[(size_t)r * stride + i] *= q_scale;
        auto& K = lm.keys[l];
        auto& V = lm.values[l];
        for (int r = 0; r < m; ++r) {
            const float* row = qkv.data() + (size_t)r * stride;
            K.insert(K.end(), row + qd, row + qd + kv);
            V.insert(V.end(), row + qd + kv, row + stride);
            if (c.kv_f16) {
                // The f16 cache: each appended key and value rounded through
                // binary16 (round to nearest even) where it is stored.
                for (size_t i = K.size() - kv; i < K.size(); ++i) K[i] = f16r(K[i]);
                for (size_t i = V.size() - kv; i < V.size(); ++i) V[i] = f16r(V[i]);
            }
        }
        int seen = first + m;
        attention(lm.isa, qkv.data(), stride, K.data(), V.data(), kv, m, seen, c.heads, c.kv_heads, hd, true,
                  att.data());
        L.o.forward(lm.isa, att.data(), m, y.data());
        add_scaled(x.data(), y.data(), (size_t)m * d, c.residual_multiplier);
        normed = x;
        parallel(m, [&](int r) { rmsnorm_row(L.norm_mlp.data(), d, c.eps, normed.data() + (size_t)r * d); });
        if (!lm.ffn_scales.empty()) {
            const float* s = lm.ffn_scales[l].data();
            for (int r = 0; r < m; ++r)
                for (int i = 0; i < d; ++i) normed[(size_t)r * d + i] *= s[i];
        }
        L.gate_up.forward(lm.isa, normed.data(), m, wide.data());
        parallel(m, [&](int r) {
            const float* row = wide.data() + (size_t)r * 2 * c.ffn;
            float* h = hidden.data() + (size_t)r * c.ffn;
            for (int i = 0; i < c.ffn; ++i) h[i] = silu_one(row[i]) * row[c.ffn + i];
        });
        L.down.forward(lm.isa, hidden.data(), m, y.data());
        add_scaled(x.data(), y.data(), (size_t)m * d, c.residual_multiplier);
    }
    lm.position += m;
    std::vector<float> last(x.begin() + (size_t)(m - 1) * d, x.begin() + (size_t)m * d);
    rmsnorm_row(lm.final_norm.data(), d, c.eps, last.data());
    (lm.head.rows ? lm.head : lm.embed).product(lm.isa, last.data(), logits);
    scale_all(logits, (size_t)c.vocab, 1.0f / c.logits_scaling);
}

void lm_forward_tokens(Lm& lm, const int32_t* tokens, int n, float* logits) {
    int d = lm.c.d;
    std::vector<float> x((size_t)n * d);
    for (int r = 0; r < n; ++r) lm.embed.row(tokens[r], x.data() + (size_t)r * d);
    lm_forward_rows(lm, x, n, logits);
}

bool fill_table(Table& t, int kind, int rows, int cols, const void* data, const float* scales) {
    if (!data || rows <= 0 || cols <= 0) return false;
    t = Table();
    t.kind = kind;
    t.rows = rows;
    t.cols = cols;
    const size_t n = (size_t)rows * cols;
    if (kind == OR_TABLE_F16) {
        t.f16.assign((const uint16_t*)data, (const uint16_t*)data + n);
    } else if (kind == OR_TABLE_F32) {
        t.f32.assign((const float*)data, (const float*)data + n);
    } else if (kind == OR_TABLE_Q8) {
        if (cols % 32 || !scales) return false;
        t.codes.assign((const int8_t*)data, (const int8_t*)data + n);
        t.scales.assign(scales, scales + n / 32);
    } else {
        return false;
    }
    return true;
}

}  // namespace

// =============================================================== C ABI ===
extern "C" {

int or_isa_best(void) {
    __builtin_cpu_init();
    if (__builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
        __builtin_cpu_supports("avx512vl") && __builtin_cpu_supports("avx512vnni"))
        return OR_AVX512;
    if (__builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma")) return OR_AVX2;
    return OR_SCALAR;
}

int or_team_start(int spread, int threads) {
    if (g_team) {
        delete g_team;
        g_team = nullptr;
    }
    std::vector<int> cpus;
    bool pin = threads <= 0;
    if (threads > 0) {
        cpus.resize(std::min(threads, 256));
    } else {
        cpus = team_cpus(spread);
    }
    g_team = new Team();
    g_team->size = (int)cpus.size();
    if (pin) {
        cpu_set_t set;
        CPU_ZERO(&set);
        CPU_SET(cpus[0], &set);
        pthread_setaffinity_np(pthread_self(), sizeof(set), &set);
    }
    for (size_t i = 1; i < cpus.size(); ++i) {
        int cpu = cpus[i];
        g_team->workers.emplace_back([cpu, pin] {
            if (pin) {
                cpu_set_t set;
                CPU_ZERO(&set);
                CPU_SET(cpu, &set);
                pthread_setaffinity_np(pthread_self(), sizeof(set), &set);
            }
            g_team->worker_loop();
        });
    }
    return g_team->size;
}

int or_team_size(void) { return team_threads(); }

// The host's int8 dot-product peak as the team reaches it: each thread runs
// 12 independent chains of vpdpbusd (64 multiply-adds each) for `iters`
// rounds; no memory traffic. The yardstick of the baseline's fairness check
// (a compute-bound int8 product should reach about 90 % of it).
}  // extern "C"
namespace {
AVX512 int64_t vnni_spin(int64_t iters) {
    // 24 independent chains: enough to cover vpdpbusd's latency at two
    // issues a cycle (Zen 5's 512-bit pipes), with every operand in registers.
    constexpr int CH = 24;
    __m512i acc[CH];
#pragma GCC unroll 32
    for (int i = 0; i < CH; ++i) acc[i] = _mm512_set1_epi32(i);
    const __m512i a = _mm512_set1_epi32(0x01020304), b = _mm512_set1_epi32(0x05060708);
    for (int64_t it = 0; it < iters; ++it) {
#pragma GCC unroll 32
        for (int i = 0; i < CH; ++i) acc[i] = _mm512_dpbusd_epi32(acc[i], a, b);
    }
    __m512i t = acc[0];
#pragma GCC unroll 32
    for (int i = 1; i < CH; ++i) t = _mm512_add_epi32(t, acc[i]);
    return _mm512_reduce_add_epi32(t);
}
}  // namespace
extern "C" {

double or_vnni_peak(int64_t iters) {
    if (or_isa_best() != OR_AVX512) return 0.0;
    const int n = team_threads();
    std::vector<int64_t> sink(n);
    double best = 0.0;
    for (int round = 0; round < 3; ++round) {  // the best of three
        const auto t0 = std::chrono::steady_clock::now();
        parallel(n, [&](int t) { sink[t] = vnni_spin(iters); });
        const double s = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        best = std::max(best, (double)n * (double)iters * 24.0 * 64.0 / s);
    }
    volatile int64_t keep = 0;
    for (int64_t v : sink) keep = keep + v;
    (void)keep;
    return best;
}

uint16_t or_f32_to_f16(float value) { return f32_to_f16(value); }
float or_f16_to_f32(uint16_t half) { return f16_to_f32(half); }
float or_exp(float x) { return exp_contract(x); }

void or_silu(float* values, int64_t n) {
    for (int64_t i = 0; i < n; ++i) values[i] = silu_one(values[i]);
}

void or_quantize(int isa, const float* x, int m, int k, int group, int half_scales, int8_t* codes, float* scales,
                 int32_t* sums) {
    Quantized q;
    quantize_rows(isa, x, m, k, group, half_scales != 0, q);
    std::memcpy(codes, q.values.data(), q.values.size());
    std::memcpy(scales, q.scales.data(), q.scales.size() * 4);
    std::memcpy(sums, q.sums.data(), q.sums.size() * 4);
}

// src/cpu/gemm.rs:58-76: d = max|x|/127; codes round(x * (1/d)) half away
// from zero from the f32 d, cast as Rust's `as i8` casts (saturating, NaN
// to 0: a block with an infinite value has d = inf and every code 0); d
// stored through f16.
void or_q8_0_quantize(const float* values, int64_t count, int8_t* codes, float* scales) {
    for (int64_t b = 0; b < count / 32; ++b) {
        const float* blk = values + b * 32;
        float mx = 0.0f;
        for (int i = 0; i < 32; ++i) mx = std::fmax(mx, std::fabs(blk[i]));
        float d = mx / 127.0f;
        float inverse = d != 0.0f ? 1.0f / d : 0.0f;
        for (int i = 0; i < 32; ++i) {
            const float r = std::round(blk[i] * inverse);
            codes[b * 32 + i] = std::isnan(r) ? 0 : (int8_t)std::fmin(127.0f, std::fmax(-128.0f, r));
        }
        scales[b] = f16r(d);
    }
}

void or_q8_0_parse(const uint8_t* blocks, int64_t nblocks, int8_t* codes, float* scales) {
    for (int64_t b = 0; b < nblocks; ++b) {
        const uint8_t* p = blocks + b * 34;
        scales[b] = f16_to_f32((uint16_t)(p[0] | (p[1] << 8)));
        std::memcpy(codes + b * 32, p + 2, 32);
    }
}

// src/cpu/ggml_quants.rs:168-196: y = d*sc*q - dmin*m, two roundings.
void or_q4_k_expand(const uint8_t* blocks, int64_t nblocks, float* out) {
    for (int64_t b = 0; b < nblocks; ++b) {
        const uint8_t* p = blocks + b * 144;
        float d = f16_to_f32((uint16_t)(p[0] | (p[1] << 8)));
        float dmin = f16_to_f32((uint16_t)(p[2] | (p[3] << 8)));
        const uint8_t* sc = p + 4;
        const uint8_t* q = p + 16;
        float* y = out + b * 256;
        auto scale_min = [&](int j, uint8_t* s, uint8_t* m) {
            if (j < 4) {
                *s = sc[j] & 63;
                *m = sc[j + 4] & 63;
            } else {
                *s = (uint8_t)((sc[j + 4] & 0xF) | ((sc[j - 4] >> 6) << 4));
                *m = (uint8_t)((sc[j + 4] >> 4) | ((sc[j] >> 6) << 4));
            }
        };
        for (int is = 0; is < 8; is += 2) {
            uint8_t s1, m1, s2, m2;
            scale_min(is, &s1, &m1);
            scale_min(is + 1, &s2, &m2);
            float d1 = d * (float)s1, mm1 = dmin * (float)m1;
            float d2 = d * (float)s2, mm2 = dmin * (float)m2;
            for (int l = 0; l < 32; ++l) {
                float a = d1 * (float)(q[l] & 0xF);
                float c = d2 * (float)(q[l] >> 4);
                y[l] = a - mm1;
                y[32 + l] = c - mm2;
            }
            y += 64;
            q += 32;
        }
    }
}

// ------------------------------------------------------------- encoder ---
void or_gelu(float* values, int64_t n) {
    for (int64_t i = 0; i < n; ++i) values[i] = gelu_one(values[i]);
}

// Norm::apply (src/layers.rs:50-64,84-121): mean and variance each summed
// in 32 lanes (lane j takes values j, j+32, ... in order), the lanes added
// in order, then the tail; out = (v - mean) * inv * w + b.
void or_layer_norm(const float* x, int rows, int d, const float* w, const float* b, float eps, float* out) {
    auto lane_sum = [&](const float* row, auto term) {
        float lanes[32] = {0};
        const int whole = d / 32 * 32;
        for (int i = 0; i < whole; i += 32)
            for (int j = 0; j < 32; ++j) lanes[j] += term(row[i + j]);
        float s = 0.0f;
        for (int j = 0; j < 32; ++j) s += lanes[j];
        float t = 0.0f;
        for (int i = whole; i < d; ++i) t += term(row[i]);
        return s + t;
    };
    for (int r = 0; r < rows; ++r) {
        const float* row = x + (size_t)r * d;
        const float n = (float)d;
        const float mean = lane_sum(row, [](float v) { return v; }) / n;
        const float var = lane_sum(row, [&](float v) { return (v - mean) * (v - mean); }) / n;
        const float inv = 1.0f / std::sqrt(var + eps);
        float* o = out + (size_t)r * d;
        for (int i = 0; i < d; ++i) o[i] = (row[i] - mean) * inv * w[i] + b[i];
    }
}

// conv_columns (src/layers.rs:613-634): output row t holds x[t*stride + tap
// - pad][c] at c*kernel + tap; outside the frames, zero.
void or_conv_columns(const float* x, int frames, int channels, int kernel, int stride, int pad, int out_frames,
                     float* out) {
    for (int t = 0; t < out_frames; ++t)
        for (int tap = 0; tap < kernel; ++tap) {
            const long src = (long)t * stride + tap - pad;
            for (int c = 0; c < channels; ++c)
                out[((size_t)t * channels + c) * kernel + tap] =
                    src >= 0 && src < frames ? x[(size_t)src * channels + c] : 0.0f;
        }
}

// f32_to_f16 / f16_to_f32 (src/cpu/tensors.rs:542-595) over arrays.
void or_f32_to_f16_n(const float* in, int64_t n, uint16_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = f32_to_f16(in[i]);
}
void or_f16_to_f32_n(const uint16_t* in, int64_t n, float* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = f16_to_f32(in[i]);
}

// ggml's other block types expanded to f32 (src/cpu/ggml_quants.rs:103-245,
// ggml's dequantize_row_* in the same float order): Q4_0 (2), Q4_1 (3),
// Q5_0 (6), Q5_1 (7), Q4_K (12), Q5_K (13), Q6_K (14). Returns 0, or -1
// for another type.
int or_ggml_expand(int type, const uint8_t* blocks, int64_t nblocks, float* out) {
    auto half = [](const uint8_t* b, int at) { return f16_to_f32((uint16_t)(b[at] | (b[at + 1] << 8))); };
    auto scale_min = [](int j, const uint8_t* q, int* sc, int* m) {
        if (j < 4) {
            *sc = q[j] & 63;
            *m = q[j + 4] & 63;
        } else {
            *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
            *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
        }
    };
    switch (type) {
        case 2:  // Q4_0: f16 d, 16 bytes; (q - 8) * d (:125-132)
            for (int64_t b = 0; b < nblocks; ++b) {
                const uint8_t* p = blocks + b * 18;
                float* y = out + b * 32;
                const float d = half(p, 0);
                for (int j = 0; j < 16; ++j) {
                    y[j] = (float)((p[2 + j] & 0x0F) - 8) * d;
                    y[j + 16] = (float)((p[2 + j] >> 4) - 8) * d;
                }
            }
            return 0;
        case 3:  // Q4_1: f16 d, f16 m, 16 bytes; q * d + m (:134-141)
            for (int64_t b = 0; b < nblocks; ++b) {
                const uint8_t* p = blocks + b * 20;
                float* y = out + b * 32;
                const float d = half(p, 0), m = half(p, 2);
                for (int j = 0; j < 16; ++j) {
                    const float a = (float)(p[4 + j] & 0x0F) * d, c = (float)(p[4 + j] >> 4) * d;
                    y[j] = a + m;
                    y[j + 16] = c + m;
                }
            }
            return 0;
        case 6:  // Q5_0: f16 d, u32 high bits, 16 bytes; (q - 16) * d (:143-153)
        case 7:  // Q5_1: f16 d, f16 m, u32 high bits, 16 bytes; q * d + m (:155-166)
            for (int64_t b = 0; b < nblocks; ++b) {
                const bool one = type == 7;
                const uint8_t* p = blocks + b * (one ? 24 : 22);
                float* y = out + b * 32;
                const float d = half(p, 0), m = one ? half(p, 2) : 0.0f;
                const uint8_t* h = p + (one ? 4 : 2);
                const uint32_t qh = (uint32_t)h[0] | ((uint32_t)h[1] << 8) | ((uint32_t)h[2] << 16) | ((uint32_t)h[3] << 24);
                const uint8_t* qs = h + 4;
                for (int j = 0; j < 16; ++j) {
                    const int xh0 = (int)(((qh >> j) << 4) & 0x10), xh1 = (int)((qh >> (j + 12)) & 0x10);
                    const int q0 = (qs[j] & 0x0F) | xh0, q1 = (qs[j] >> 4) | xh1;
                    if (one) {
                        const float a = (float)q0 * d, c = (float)q1 * d;
                        y[j] = a + m;
                        y[j + 16] = c + m;
                    } else {
                        y[j] = (float)(q0 - 16) * d;
                        y[j + 16] = (float)(q1 - 16) * d;
                    }
                }
            }
            return 0;
        case 12:
            or_q4_k_expand(blocks, nblocks, out);
            return 0;
        case 13:  // Q5_K: f16 d, f16 dmin, 12 scale bytes, 32 high-bit bytes, 128 bytes (:198-221)
            for (int64_t b = 0; b < nblocks; ++b) {
                const uint8_t* p = blocks + b * 176;
                float* y = out + b * 256;
                const float d = half(p, 0), dmin = half(p, 2);
                const uint8_t* scales = p + 4;
                const uint8_t* qh = p + 16;
                const uint8_t* ql = p + 48;
                int u1 = 1, u2 = 2;
                for (int is = 0; is < 8; is += 2) {
                    int sc, m;
                    scale_min(is, scales, &sc, &m);
                    const float d1 = d * (float)sc, m1 = dmin * (float)m;
                    scale_min(is + 1, scales, &sc, &m);
                    const float d2 = d * (float)sc, m2 = dmin * (float)m;
                    for (int l = 0; l < 32; ++l) {
                        const int h1 = (qh[l] & u1) ? 16 : 0, h2 = (qh[l] & u2) ? 16 : 0;
                        const float a = d1 * (float)((ql[l] & 0xF) + h1), c = d2 * (float)((ql[l] >> 4) + h2);
                        y[l] = a - m1;
                        y[32 + l] = c - m2;
                    }
                    y += 64;
                    ql += 32;
                    u1 <<= 2;
                    u2 <<= 2;
                }
            }
            return 0;
        case 14:  // Q6_K: 128 low bytes, 64 high-bit bytes, 16 int8 scales, f16 d (:223-245)
            for (int64_t b = 0; b < nblocks; ++b) {
                const uint8_t* p = blocks + b * 210;
                float* y = out + b * 256;
                const float d = half(p, 208);
                const uint8_t* ql = p;
                const uint8_t* qh = p + 128;
                const int8_t* sc = (const int8_t*)(p + 192);
                for (int n = 0; n < 2; ++n) {
                    for (int l = 0; l < 32; ++l) {
                        const int is = l / 16;
                        const int q1 = (int8_t)((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32;
                        const int q2 = (int8_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                        const int q3 = (int8_t)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                        const int q4 = (int8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                        y[l] = d * (float)sc[is] * (float)q1;
                        y[l + 32] = d * (float)sc[is + 2] * (float)q2;
                        y[l + 64] = d * (float)sc[is + 4] * (float)q3;
                        y[l + 96] = d * (float)sc[is + 6] * (float)q4;
                    }
                    y += 128;
                    ql += 64;
                    qh += 32;
                    sc += 8;
                }
            }
            return 0;
        default:
            return -1;
    }
}

void* or_int8_new(int isa, int n, int k, int group, int half_scales, const int8_t* codes, const float* scales) {
    if (k % group != 0 || group % 4 != 0) return nullptr;
    if (isa != OR_SCALAR && n % 32 != 0) isa = OR_SCALAR;
    return int8_new(isa, n, k, group, half_scales != 0, codes, scales);
}
void or_int8_forward(const void* layer, const float* x, int m, float* out) {
    int8_forward(*(const Int8Layer*)layer, x, m, out);
}
void or_int8_free(void* layer) { delete (Int8Layer*)layer; }

void* or_ternary_new(int isa, int n, int k, const uint8_t* codes, const float* scales) {
    if (k % TGROUP != 0) return nullptr;
    return ternary_new(isa, n, k, codes, scales);
}
void or_ternary_forward(const void* layer, const float* x, int m, float* out) {
    ternary_forward(*(const TernaryLayer*)layer, x, m, out);
}
void or_ternary_free(void* layer) { delete (TernaryLayer*)layer; }

int or_ternary_from_base3(const uint8_t* packed, int n, int k, uint8_t* codes) {
    int row_bytes = (k + 4) / 5;
    for (int r = 0; r < n; ++r) {
        for (int b = 0; b < row_bytes; ++b) {
            int v = packed[(size_t)r * row_bytes + b];
            if (v > 242) return -1;
            for (int digit = 0; digit < 5; ++digit) {
                int kk = b * 5 + digit;
                if (kk < k) codes[(size_t)r * k + kk] = (uint8_t)(v % 3);
                v /= 3;
            }
        }
    }
    return 0;
}

void or_matmul_f16(int isa, const float* x, int m, int k, const uint16_t* w, int n, float* out) {
    matmul<uint16_t>(isa, x, m, k, w, n, out);
}
void or_matmul_f32(int isa, const float* x, int m, int k, const float* w, int n, float* out) {
    matmul<float>(isa, x, m, k, w, n, out);
}

void or_rmsnorm(const float* weight, int d, float eps, float* x, int rows) {
    for (int r = 0; r < rows; ++r) rmsnorm_row(weight, d, eps, x + (size_t)r * d);
}

void or_rope_table(int dims, float base, int positions, float* sin_out, float* cos_out) {
    rope_table(dims, base, positions, sin_out, cos_out);
}

void or_rope(float* x, int rows, int stride, int heads, int hd, int first, float base) {
    std::vector<float> s((size_t)(first + rows) * (hd / 2)), c(s.size());
    rope_table(hd, base, first + rows, s.data(), c.data());
    rope_apply(x, rows, stride, heads, hd, first, s.data(), c.data());
}

void or_attention(const float* q, int qs, const float* k, const float* v, int kvs, int tq, int tk, int heads,
                  int kv_heads, int hd, int causal, float* out) {
    attention(OR_SCALAR, q, qs, k, v, kvs, tq, tk, heads, kv_heads, hd, causal != 0, out);
}

int or_argmax(const float* values, int n) { return argmax(values, n); }

void* or_lm_new(int isa, const or_lm_config* cfg) {
    if (cfg->heads <= 0 || cfg->kv_heads <= 0 || cfg->heads % cfg->kv_heads != 0) return nullptr;
    auto* lm = new Lm();
    lm->isa = isa;
    lm->c = *cfg;
    if (lm->c.logits_scaling == 0.0f) lm->c.logits_scaling = 1.0f;
    lm->layers.resize(cfg->layers);
    lm->keys.resize(cfg->layers);
    lm->values.resize(cfg->layers);
    return lm;
}

int or_lm_set_layer(void* p, int layer, const uint8_t* qkv, const uint8_t* o, const uint8_t* gate_up,
                    const uint8_t* down, const float* norm_attn, const float* norm_mlp, const float* q_norm,
                    const float* k_norm) {
    auto* lm = (Lm*)p;
    const auto& c = lm->c;
    if (layer < 0 || layer >= c.layers) return -1;
    int hd = c.head_dim, d = c.d;
    auto& L = lm->layers[layer];
    L.qkv.set_int8(q8_layer(lm->isa, (c.heads + 2 * c.kv_heads) * hd, d, qkv));
    L.o.set_int8(q8_layer(lm->isa, d, c.heads * hd, o));
    L.gate_up.set_int8(q8_layer(lm->isa, 2 * c.ffn, d, gate_up));
    L.down.set_int8(q8_layer(lm->isa, d, c.ffn, down));
    L.norm_attn.assign(norm_attn, norm_attn + d);
    L.norm_mlp.assign(norm_mlp, norm_mlp + d);
    if (c.qk_norm) {
        L.q_norm.assign(q_norm, q_norm + hd);
        L.k_norm.assign(k_norm, k_norm + hd);
    }
    return 0;
}

int or_lm_set_linear_int8(void* p, int layer, int which, const int8_t* codes, const float* scales) {
    auto* lm = (Lm*)p;
    const auto& c = lm->c;
    if (layer < 0 || layer >= c.layers || which < 0 || which > 3 || !codes || !scales) return -1;
    const int hd = c.head_dim;
    const int n[4] = {(c.heads + 2 * c.kv_heads) * hd, c.d, 2 * c.ffn, c.d};
    const int k[4] = {c.d, c.heads * hd, c.d, c.ffn};
    if (k[which] % 128) return -1;
    auto& L = lm->layers[layer];
    Linear* slot[4] = {&L.qkv, &L.o, &L.gate_up, &L.down};
    slot[which]->set_int8(int8_new(lm->isa, n[which], k[which], 128, false, codes, scales));
    return 0;
}

int or_lm_set_linear_float(void* p, int layer, int which, int kind, const void* weights) {
    auto* lm = (Lm*)p;
    const auto& c = lm->c;
    if (layer < 0 || layer >= c.layers || which < 0 || which > 3 || !weights) return -1;
    if (kind != OR_TABLE_F16 && kind != OR_TABLE_F32) return -1;
    const int hd = c.head_dim;
    const int n[4] = {(c.heads + 2 * c.kv_heads) * hd, c.d, 2 * c.ffn, c.d};
    const int k[4] = {c.d, c.heads * hd, c.d, c.ffn};
    auto& L = lm->layers[layer];
    Linear* slot[4] = {&L.qkv, &L.o, &L.gate_up, &L.down};
    Linear& q = *slot[which];
    q.set_int8(nullptr);
    q.fkind = kind;
    q.n = n[which];
    q.k = k[which];
    const size_t count = (size_t)q.n * q.k;
    if (kind == OR_TABLE_F16) q.f16.assign((const uint16_t*)weights, (const uint16_t*)weights + count);
    else q.f32.assign((const float*)weights, (const float*)weights + count);
    return 0;
}

int or_lm_set_embed(void* p, const uint16_t* embed, const float* final_norm) {
    auto* lm = (Lm*)p;
    if (!fill_table(lm->embed, OR_TABLE_F16, lm->c.vocab, lm->c.d, embed, nullptr)) return -1;
    lm->final_norm.assign(final_norm, final_norm + lm->c.d);
    return 0;
}

int or_lm_set_table(void* p, int which, int kind, const void* data, const float* scales) {
    auto* lm = (Lm*)p;
    if (which == 1 && !data) {
        lm->head = Table();
        return 0;
    }
    if (which != 0 && which != 1) return -1;
    return fill_table(which == 0 ? lm->embed : lm->head, kind, lm->c.vocab, lm->c.d, data, scales) ? 0 : -1;
}

int or_lm_set_ffn_scales(void* p, const float* scales) {
    auto* lm = (Lm*)p;
    lm->ffn_scales.clear();
    if (!scales) return 0;
    for (int l = 0; l < lm->c.layers; ++l)
        lm->ffn_scales.emplace_back(scales + (size_t)l * lm->c.d, scales + (size_t)(l + 1) * lm->c.d);
    return 0;
}

void or_lm_reset(void* p) {
    auto* lm = (Lm*)p;
    for (auto& k : lm->keys) k.clear();
    for (auto& v : lm->values) v.clear();
    lm->position = 0;
}

int or_lm_truncate(void* p, int position) {
    auto* lm = (Lm*)p;
    if (position < 0 || position > lm->position) return -1;
    const size_t kv = (size_t)lm->c.kv_heads * lm->c.head_dim;
    for (auto& k : lm->keys) k.resize((size_t)position * kv);
    for (auto& v : lm->values) v.resize((size_t)position * kv);
    lm->position = position;
    return 0;
}

int or_lm_position(void* p) { return ((Lm*)p)->position; }

int or_lm_embed_row(void* p, int token, float* out) {
    auto* lm = (Lm*)p;
    if (token < 0 || token >= lm->c.vocab) return -1;
    lm->embed.row(token, out);
    return 0;
}

int or_lm_forward(void* p, const int32_t* tokens, int n, float* logits) {
    auto* lm = (Lm*)p;
    if (n <= 0) return -1;
    for (int i = 0; i < n; ++i)
        if (tokens[i] < 0 || tokens[i] >= lm->c.vocab) return -1;
    lm_forward_tokens(*lm, tokens, n, logits);
    return 0;
}

int or_lm_forward_rows(void* p, const float* rows, int n, float* logits) {
    auto* lm = (Lm*)p;
    if (n <= 0 || !rows) return -1;
    std::vector<float> x(rows, rows + (size_t)n * lm->c.d);
    lm_forward_rows(*lm, x, n, logits);
    return 0;
}

// causal_lm.rs:217-249,284-302: forward the prompt, then argmax, stop
// check, and a forward of each kept token (also after the last one).
int or_lm_generate(void* p, const int32_t* prompt, int n_prompt, int max_new, const int32_t* stop, int n_stop,
                   int32_t* out, float* logits_out) {
    auto* lm = (Lm*)p;
    or_lm_reset(lm);
    std::vector<float> logits(lm->c.vocab);
    if (or_lm_forward(lm, prompt, n_prompt, logits.data()) != 0) return -1;
    if (logits_out) std::memcpy(logits_out, logits.data(), logits.size() * 4);
    int count = 0;
    while (count < max_new) {
        int32_t token = argmax(logits.data(), lm->c.vocab);
        bool stopped = false;
        for (int s = 0; s < n_stop; ++s) stopped |= stop[s] == token;
        if (stopped) break;
        out[count++] = token;
        lm_forward_tokens(*lm, &token, 1, logits.data());
    }
    return count;
}

void or_lm_free(void* p) { delete (Lm*)p; }

}  // extern "C"
