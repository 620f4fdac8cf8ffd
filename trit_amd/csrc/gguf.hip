// GGUF files: the container Trit reads its decoder weights from
// (src/models/gguf/mod.rs:130-300), and a decoder built from one.
//
// The reader keeps the reference's checks and their order: the magic, the
// version (2 or 3), the metadata (strings and arrays bounded in length,
// arrays nested at most four deep), a tensor count the file can hold, the
// tensor entries, general.alignment (32 when absent, never 0), and every
// tensor's byte range inside the file for its ggml type
// (src/cpu/ggml_quants.rs:51-75). Host code only: no device call.
//
// The decoder builder reads a language model laid out as transcribe.cpp
// writes it (the Qwen3 decoder of a qwen3_asr file): the shape under
// `<prefix>.{hidden_size, intermediate_size, n_layers, n_heads, n_kv_heads,
// head_dim, vocab_size, rms_norm_eps, rope_theta, tie_word_embeddings}`
// (src/models/gguf/blocks.rs:25-45) and the tensors `dec.token_embd`,
// `dec.output_norm`, `dec.blocks.<l>.{norm_attn, norm_ffn, attn.q_norm,
// attn.k_norm, attn.q, attn.k, attn.v, attn.o, ffn.gate, ffn.up, ffn.down}`
// (src/models/gguf/qwen3_asr.rs:103-136). The linears go to the device as
// the layers trit_hip_layer_q8_0 / _q4_k make (q, k, v rows stacked, then
// gate and up), the token table as an f16 layer.
#include "../../include/trit_hip.h"
#include "internal.h"

#include <cerrno>
#include <cstdio>
#include <cstring>
#include <map>

struct TritHipGguf;

namespace trit {
namespace {

// A metadata value: numbers keep their GGUF type's range; arrays nest.
struct GgufValue {
    enum Kind { U, I, F, B, S, A } kind = U;
    uint64_t u = 0;
    int64_t i = 0;
    double f = 0.0;
    bool b = false;
    std::string s;
    std::vector<GgufValue> a;
};

struct GgufTensor {
    std::string name, dtype;
    uint32_t type = 0;
    std::vector<uint64_t> dims;
    uint64_t start = 0, end = 0;
};

// ggml types the reader knows: id, name, values a block, bytes a block
// (src/cpu/ggml_quants.rs:51-63).
struct GgmlType {
    uint32_t id;
    const char* name;
    uint64_t values, bytes;
};
constexpr GgmlType kTypes[] = {
    {0, "F32", 1, 4},      {1, "F16", 1, 2},       {30, "BF16", 1, 2},     {8, "Q8_0", 32, 34},
    {2, "Q4_0", 32, 18},   {3, "Q4_1", 32, 20},    {6, "Q5_0", 32, 22},    {7, "Q5_1", 32, 24},
    {12, "Q4_K", 256, 144}, {13, "Q5_K", 256, 176}, {14, "Q6_K", 256, 210},
};

std::string type_list() {
    std::string out;
    const int n = (int)(sizeof(kTypes) / sizeof(kTypes[0]));
    for (int i = 0; i < n; ++i) {
        if (i) out += i + 1 == n ? ", and " : ", ";
        out += kTypes[i].name;
    }
    return out;
}

constexpr uint64_t kDefaultAlignment = 32;
constexpr uint64_t kMinTensorEntry = 24;  // empty name, no dims, type, offset
constexpr int kMaxArrayDepth = 4;
constexpr uint64_t kMaxLength = 1ull << 24;  // strings and arrays

// Little-endian reads from the start of the file; a short read is the
// header ending early.
struct Reader {
    FILE* f = nullptr;
    uint64_t pos = 0;
    void bytes(void* out, size_t n) {
        if (n && std::fread(out, 1, n, f) != n) throw Error("the header ends early");
        pos += n;
    }
    template <class T>
    T get() {
        T v;
        bytes(&v, sizeof(T));
        return v;
    }
    std::string string() {
        const uint64_t len = get<uint64_t>();
        if (len > kMaxLength) throw Error("a header string is too long");
        std::string s(len, '\0');
        bytes(s.data(), len);
        if (!utf8(s)) throw Error("a header string is not UTF-8");
        return s;
    }
    // Well-formed UTF-8 (no overlong forms, surrogates or values past
    // U+10FFFF), as Rust's String::from_utf8 accepts it.
    static bool utf8(const std::string& s) {
        const unsigned char* p = (const unsigned char*)s.data();
        const size_t n = s.size();
        for (size_t i = 0; i < n;) {
            const unsigned c = p[i];
            int more;
            unsigned lo = 0x80, hi = 0xBF;
            if (c < 0x80) { ++i; continue; }
            if (c >= 0xC2 && c <= 0xDF) more = 1;
            else if (c == 0xE0) more = 2, lo = 0xA0;
            else if (c == 0xED) more = 2, hi = 0x9F;
            else if (c >= 0xE1 && c <= 0xEF) more = 2;
            else if (c == 0xF0) more = 3, lo = 0x90;
            else if (c >= 0xF1 && c <= 0xF3) more = 3;
            else if (c == 0xF4) more = 3, hi = 0x8F;
            else return false;
            if (i + (size_t)more >= n) return false;  // the sequence runs past the end
            if (p[i + 1] < lo || p[i + 1] > hi) return false;
            for (int k = 2; k <= more; ++k)
                if (p[i + k] < 0x80 || p[i + k] > 0xBF) return false;
            i += (size_t)more + 1;
        }
        return true;
    }
    GgufValue value(uint32_t kind, int depth) {
        GgufValue v;
        switch (kind) {
            case 0: v.kind = GgufValue::U, v.u = get<uint8_t>(); break;
            case 1: v.kind = GgufValue::I, v.i = get<int8_t>(); break;
            case 2: v.kind = GgufValue::U, v.u = get<uint16_t>(); break;
            case 3: v.kind = GgufValue::I, v.i = get<int16_t>(); break;
            case 4: v.kind = GgufValue::U, v.u = get<uint32_t>(); break;
            case 5: v.kind = GgufValue::I, v.i = get<int32_t>(); break;
            case 6: v.kind = GgufValue::F, v.f = get<float>(); break;
            case 7: v.kind = GgufValue::B, v.b = get<uint8_t>() != 0; break;
            case 8: v.kind = GgufValue::S, v.s = string(); break;
            case 9: {
                if (depth >= kMaxArrayDepth) throw Error("the header arrays are nested too deep");
                const uint32_t item = get<uint32_t>();
                const uint64_t count = get<uint64_t>();
                if (count > kMaxLength) throw Error("a header array is too long");
                v.kind = GgufValue::A;
                v.a.reserve(count);
                for (uint64_t k = 0; k < count; ++k) v.a.push_back(value(item, depth + 1));
                break;
            }
            case 10: v.kind = GgufValue::U, v.u = get<uint64_t>(); break;
            case 11: v.kind = GgufValue::I, v.i = get<int64_t>(); break;
            case 12: v.kind = GgufValue::F, v.f = get<double>(); break;
            default: throw Error("metadata type " + std::to_string(kind) + " is not GGUF");
        }
        return v;
    }
};

}  // namespace

struct GgufFile {
    std::string path;
    std::map<std::string, GgufValue> meta;
    std::vector<GgufTensor> tensors;

    // Gguf::open (src/models/gguf/mod.rs:155-226); errors name the file.
    explicit GgufFile(const std::string& p) : path(p) {
        FILE* f = std::fopen(p.c_str(), "rb");
        if (!f) fail("Could not read " + p + ": " + std::strerror(errno));
        try {
            read(f);
        } catch (const Error& e) {
            std::fclose(f);
            fail(p + ": " + e.what());
        }
        std::fclose(f);
    }

    void read(FILE* f) {
        std::fseek(f, 0, SEEK_END);
        const uint64_t total = (uint64_t)std::ftell(f);
        std::fseek(f, 0, SEEK_SET);
        Reader r{f, 0};
        char magic[4];
        r.bytes(magic, 4);
        if (std::memcmp(magic, "GGUF", 4) != 0) throw Error("not a GGUF file");
        const uint32_t version = r.get<uint32_t>();
        if (version < 2 || version > 3)
            throw Error("GGUF version " + std::to_string(version) + "; Trit reads 2 and 3");
        const uint64_t tensor_count = r.get<uint64_t>();
        const uint64_t kv_count = r.get<uint64_t>();
        for (uint64_t k = 0; k < kv_count; ++k) {
            std::string key = r.string();
            const uint32_t kind = r.get<uint32_t>();
            meta[key] = r.value(kind, 0);
        }
        if (tensor_count > total / kMinTensorEntry) throw Error("the tensor list runs past the end of the file");
        struct Info {
            std::string name;
            std::vector<uint64_t> dims;
            uint64_t count;
            uint32_t kind;
            uint64_t offset;
        };
        std::vector<Info> infos;
        infos.reserve(tensor_count);
        for (uint64_t k = 0; k < tensor_count; ++k) {
            Info in;
            in.name = r.string();
            const uint32_t dims = r.get<uint32_t>();
            uint64_t count = 1;
            for (uint32_t d = 0; d < dims; ++d) {
                const uint64_t n = r.get<uint64_t>();
                in.dims.push_back(n);
                count = (n != 0 && count > UINT64_MAX / n) ? UINT64_MAX : count * n;  // saturating
            }
            in.count = count;
            in.kind = r.get<uint32_t>();
            in.offset = r.get<uint64_t>();
            infos.push_back(std::move(in));
        }
        uint64_t alignment = kDefaultAlignment;
        auto al = meta.find("general.alignment");
        if (al != meta.end() && al->second.kind == GgufValue::U) alignment = al->second.u;
        if (al != meta.end() && al->second.kind == GgufValue::I && al->second.i >= 0) alignment = (uint64_t)al->second.i;
        if (alignment == 0) throw Error("general.alignment is 0");
        const uint64_t here = r.pos;
        if (here > UINT64_MAX - (alignment - 1)) throw Error("the tensor data runs past the end of the file");
        const uint64_t data = (here + alignment - 1) / alignment * alignment;
        for (Info& in : infos) {
            const GgmlType* t = nullptr;
            for (const GgmlType& k : kTypes)
                if (k.id == in.kind) t = &k;
            // ggml_quants::layout: an unknown id, or a count that is not whole
            // blocks, is a type Trit does not read.
            if (!t || in.count % t->values != 0)
                throw Error("tensor " + in.name + " has ggml type " + std::to_string(in.kind) + "; Trit reads " +
                            type_list());
            const uint64_t blocks = in.count / t->values;
            bool ok = blocks <= UINT64_MAX / t->bytes;
            const uint64_t bytes = ok ? blocks * t->bytes : 0;
            ok = ok && data <= UINT64_MAX - in.offset;
            const uint64_t start = ok ? data + in.offset : 0;
            ok = ok && start <= UINT64_MAX - bytes && start + bytes <= total;
            if (!ok) throw Error("tensor " + in.name + " runs past the end of the file");
            GgufTensor g;
            g.name = std::move(in.name);
            g.dtype = t->name;
            g.type = t->id;
            g.dims = std::move(in.dims);
            g.start = start;
            g.end = start + bytes;
            tensors.push_back(std::move(g));
        }
    }

    const GgufValue* get(const std::string& key) const {
        auto it = meta.find(key);
        return it == meta.end() ? nullptr : &it->second;
    }
    const GgufTensor* tensor(const std::string& name) const {
        for (const GgufTensor& t : tensors)
            if (t.name == name) return &t;
        return nullptr;
    }
    std::vector<uint8_t> bytes(const GgufTensor& t) const {
        std::vector<uint8_t> out(t.end - t.start);
        FILE* f = std::fopen(path.c_str(), "rb");
        if (!f) fail("Could not read " + path + ": " + std::strerror(errno));
        const bool ok = std::fseek(f, (long)t.start, SEEK_SET) == 0 && std::fread(out.data(), 1, out.size(), f) == out.size();
        std::fclose(f);
        if (!ok) fail(path + ": tensor " + t.name + " could not be read");
        return out;
    }
};

namespace {

bool as_u64(const GgufValue* v, uint64_t& out) {
    if (!v) return false;
    if (v->kind == GgufValue::U) return out = v->u, true;
    if (v->kind == GgufValue::I && v->i >= 0) return out = (uint64_t)v->i, true;
    return false;
}

bool as_f64(const GgufValue* v, double& out) {
    if (!v) return false;
    if (v->kind == GgufValue::F) return out = v->f, true;
    if (v->kind == GgufValue::U) return out = (double)v->u, true;
    if (v->kind == GgufValue::I) return out = (double)v->i, true;
    return false;
}

// The decoder key block of the architectures whose language model is the
// Qwen3 plan with `dec.*` tensors.
const char* decoder_prefix(const GgufFile& g) {
    const GgufValue* arch = g.get("general.architecture");
    if (arch && arch->kind == GgufValue::S && arch->s == "qwen3_asr") return "stt.qwen3_asr.decoder";
    return nullptr;
}


struct LayerOwner {
    std::vector<TritHipLayer*> all;
    ~LayerOwner() {
        for (TritHipLayer* l : all) trit_hip_layer_free(l);
    }
    TritHipLayer* keep(TritHipLayer* l) {
        all.push_back(l);
        return l;
    }
};

}  // namespace
}  // namespace trit

struct TritHipGguf {
    trit::GgufFile file;
};

using namespace trit;

extern "C" {

int trit_hip_gguf_open(const char* path, TritHipGguf** out) {
    return guard(-1, [&] {
        if (!path || !out) fail("gguf: a required argument is NULL");
        *out = new TritHipGguf{GgufFile(path)};
        return 0;
    });
}

void trit_hip_gguf_free(TritHipGguf* g) { delete g; }

int trit_hip_gguf_tensor_count(const TritHipGguf* g) {
    return guard(-1, [&] {
        if (!g) fail("gguf: NULL handle");
        return (int)g->file.tensors.size();
    });
}

int trit_hip_gguf_tensor(const TritHipGguf* g, int index, const char** name, const char** dtype, int* n_dims,
                         int64_t* dims, int64_t* start, int64_t* end) {
    return guard(-1, [&] {
        if (!g) fail("gguf: NULL handle");
        if (index < 0 || index >= (int)g->file.tensors.size()) fail("gguf: tensor index out of range");
        const GgufTensor& t = g->file.tensors[index];
        if (name) *name = t.name.c_str();
        if (dtype) *dtype = t.dtype.c_str();
        if (n_dims) *n_dims = (int)t.dims.size();
        if (dims)
            for (size_t d = 0; d < t.dims.size() && d < 4; ++d) dims[d] = (int64_t)t.dims[d];
        if (start) *start = (int64_t)t.start;
        if (end) *end = (int64_t)t.end;
        return 0;
    });
}

int trit_hip_gguf_meta_u64(const TritHipGguf* g, const char* key, uint64_t* out) {
    return guard(-1, [&] {
        if (!g || !key || !out) fail("gguf: a required argument is NULL");
        if (!as_u64(g->file.get(key), *out)) fail(std::string("gguf: no integer ") + key);
        return 0;
    });
}

int trit_hip_gguf_meta_f64(const TritHipGguf* g, const char* key, double* out) {
    return guard(-1, [&] {
        if (!g || !key || !out) fail("gguf: a required argument is NULL");
        if (!as_f64(g->file.get(key), *out)) fail(std::string("gguf: no number ") + key);
        return 0;
    });
}

int trit_hip_gguf_meta_str(const TritHipGguf* g, const char* key, const char** out) {
    return guard(-1, [&] {
        if (!g || !key || !out) fail("gguf: a required argument is NULL");
        const GgufValue* v = g->file.get(key);
        if (!v || v->kind != GgufValue::S) fail(std::string("gguf: no string ") + key);
        *out = v->s.c_str();
        return 0;
    });
}

int trit_hip_decoder_from_gguf(const char* path, const char* prefix, TritHipLmConfig* config,
                               TritHipDecoder** out) {
    return guard(-1, [&] {
        if (!path || !out) fail("gguf decoder: a required argument is NULL");
        GgufFile g(path);
        const char* pre = prefix ? prefix : decoder_prefix(g);
        if (!pre) fail(std::string(path) + ": no language model block for this architecture (give its key prefix)");
        auto num = [&](const char* key) {
            uint64_t v = 0;
            if (!as_u64(g.get(std::string(pre) + "." + key), v))
                fail(std::string(path) + ": no " + pre + "." + key);
            if (v > (1u << 30)) fail(std::string(path) + ": " + pre + "." + key + " is out of range");
            return (int)v;
        };
        auto real = [&](const char* key, double dflt) {
            double v = dflt;
            as_f64(g.get(std::string(pre) + "." + key), v);
            return v;
        };
        TritHipLmConfig c{};
        c.d = num("hidden_size");
        c.ffn = num("intermediate_size");
        c.layers = num("n_layers");
        c.heads = num("n_heads");
        c.kv_heads = num("n_kv_heads");
        c.head_dim = num("head_dim");
        c.vocab = num("vocab_size");
        c.eps = (float)real("rms_norm_eps", 1e-6);
        c.rope_base = (float)real("rope_theta", 1e6);
        // Granite's multipliers where the file has them (granite_speech.rs:33-36).
        c.embedding_multiplier = (float)real("embedding_multiplier", 1.0);
        c.attention_multiplier = (float)real("attention_multiplier", 0.0);
        c.residual_multiplier = (float)real("residual_multiplier", 1.0);
        c.logits_scaling = (float)real("logits_scaling", 1.0);
        const GgufValue* tie_v = g.get(std::string(pre) + ".tie_word_embeddings");
        const bool tie = !(tie_v && tie_v->kind == GgufValue::B && !tie_v->b);
        c.qk_norm = g.tensor("dec.blocks.0.attn.q_norm.weight") || g.tensor("dec.layers.0.attn.q_norm.weight");

        // Fun-ASR files say dec.layers, the others dec.blocks.
        const std::string blocks = g.tensor("dec.layers.0.attn.q.weight") ? "dec.layers." : "dec.blocks.";
        auto need = [&](const std::string& name) -> const GgufTensor& {
            const GgufTensor* t = g.tensor(name);
            if (!t) fail(std::string(path) + ": no tensor " + name);
            return *t;
        };
        auto shape = [&](const GgufTensor& t, uint64_t n, uint64_t k) {
            // ggml dims: ne0 (the inputs, fastest) then ne1 (the rows).
            const uint64_t d0 = t.dims.size() > 0 ? t.dims[0] : 1, d1 = t.dims.size() > 1 ? t.dims[1] : 1;
            if (d0 != k || d1 != n || t.dims.size() > 2)
                fail(std::string(path) + ": tensor " + t.name + " is " + std::to_string(d1) + "x" +
                     std::to_string(d0) + ", expected " + std::to_string(n) + "x" + std::to_string(k));
        };
        auto vec = [&](const std::string& name, uint64_t n, std::vector<float>& dst) {
            const GgufTensor& t = need(name);
            uint64_t count = 1;
            for (uint64_t d : t.dims) count *= d;
            if (count != n) fail(std::string(path) + ": tensor " + name + " has " + std::to_string(count) + " values");
            const std::vector<uint8_t> b = g.bytes(t);
            if (t.type == 0) {
                const size_t at = dst.size();
                dst.resize(at + n);
                std::memcpy(dst.data() + at, b.data(), n * 4);
            } else if (t.type == 1) {
                for (uint64_t k = 0; k < n; ++k) {
                    uint16_t h;
                    std::memcpy(&h, b.data() + 2 * k, 2);
                    dst.push_back(f16_bits_to_f32(h));
                }
            } else {
                fail(std::string(path) + ": norm " + name + " is " + t.dtype + "; the loader reads F32 and F16");
            }
        };
        LayerOwner own;
        // One device layer from the row blocks of `parts` (stacked in order).
        auto linear = [&](const std::vector<std::string>& parts, const std::vector<uint64_t>& rows, uint64_t k) {
            const GgufTensor& first = need(parts[0]);
            uint64_t n = 0;
            std::vector<uint8_t> all;
            for (size_t i = 0; i < parts.size(); ++i) {
                const GgufTensor& t = need(parts[i]);
                shape(t, rows[i], k);
                if (t.type != first.type)
                    fail(std::string(path) + ": " + parts[i] + " is " + t.dtype + " and " + parts[0] + " " +
                         first.dtype + "; stacked rows take one type");
                const std::vector<uint8_t> b = g.bytes(t);
                all.insert(all.end(), b.begin(), b.end());
                n += rows[i];
            }
            // Dense::load under Auto (src/cpu/gemm.rs:287-333, tensors.rs:
            // 262-279): Q8_0 and ggml's other block types as Q8_0 codes; F16
            // as f16 weights and F32 as f32 weights, f32 math.
            TritHipLayer* L = nullptr;
            int rc = -1;
            int values = 0, size = 0;
            if (first.type == 8 || ggml_block_type((int)first.type, &values, &size))
                rc = trit_hip_layer_ggml((int)n, (int)k, (int)first.type, all.data(), nullptr, 0, &L);
            else if (first.type == 1)
                rc = trit_hip_layer_f16((int)n, (int)k, (const uint16_t*)all.data(), nullptr, &L);
            else if (first.type == 0)
                rc = trit_hip_layer_f32((int)n, (int)k, (const float*)all.data(), nullptr, &L);
            else
                fail(std::string(path) + ": " + parts[0] + " is " + first.dtype +
                     "; the device loader reads F32, F16, Q8_0 and ggml's Q4/Q5/Q6 block types");
            if (rc != 0) fail(error_text());
            return own.keep(L);
        };

        const uint64_t hd = c.head_dim, qd = (uint64_t)c.heads * hd, kd = (uint64_t)c.kv_heads * hd;
        std::vector<const TritHipLayer*> linears;
        std::vector<float> norms;
        for (int l = 0; l < c.layers; ++l) {
            const std::string b = blocks + std::to_string(l) + ".";
            linears.push_back(linear({b + "attn.q.weight", b + "attn.k.weight", b + "attn.v.weight"}, {qd, kd, kd},
                                     c.d));
            linears.push_back(linear({b + "attn.o.weight"}, {(uint64_t)c.d}, qd));
            linears.push_back(linear({b + "ffn.gate.weight", b + "ffn.up.weight"}, {(uint64_t)c.ffn, (uint64_t)c.ffn},
                                     c.d));
            linears.push_back(linear({b + "ffn.down.weight"}, {(uint64_t)c.d}, c.ffn));
            vec(b + "norm_attn.weight", c.d, norms);
            vec(b + "norm_ffn.weight", c.d, norms);
            if (c.qk_norm) {
                vec(b + "attn.q_norm.weight", hd, norms);
                vec(b + "attn.k_norm.weight", hd, norms);
            }
        }
        vec("dec.output_norm.weight", c.d, norms);
        // Dense::table under Auto (src/cpu/gemm.rs:376-409): F16 and F32 as
        // stored; Q8_0 and ggml's other block types as Q8_0 codes with f32
        // math -- never int8 activations.
        auto table = [&](const std::string& name) {
            const GgufTensor& t = need(name);
            shape(t, c.vocab, c.d);
            const std::vector<uint8_t> b = g.bytes(t);
            TritHipLayer* L = nullptr;
            int rc = -1;
            int values = 0, size = 0;
            if (t.type == 1)
                rc = trit_hip_layer_f16(c.vocab, c.d, (const uint16_t*)b.data(), nullptr, &L);
            else if (t.type == 0)
                rc = trit_hip_layer_f32(c.vocab, c.d, (const float*)b.data(), nullptr, &L);
            else if (t.type == 8 || ggml_block_type((int)t.type, &values, &size))
                rc = trit_hip_layer_ggml(c.vocab, c.d, (int)t.type, b.data(), nullptr, 1, &L);
            else
                fail(std::string(path) + ": " + name + " is " + t.dtype +
                     "; a token table is read as F16, F32, Q8_0 or ggml's Q4/Q5/Q6 block types");
            if (rc != 0) fail(error_text());
            return own.keep(L);
        };
        TritHipLayer* embed = table("dec.token_embd.weight");
        TritHipLayer* head = nullptr;
        if (!tie || g.tensor("dec.output.weight")) head = table("dec.output.weight");
        TritHipDecoder* dec = nullptr;
        if (trit_hip_decoder_new(&c, linears.data(), norms.data(), embed, head, &dec) != 0) fail(error_text());
        if (config) *config = c;
        *out = dec;
        return 0;  // the decoder keeps its layers alive; `own` frees the handles
    });
}

}  // extern "C"
