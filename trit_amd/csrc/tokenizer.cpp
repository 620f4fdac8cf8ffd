// Byte-level BPE from a Hugging Face tokenizer.json, as Trit's text::bpe
// runs it for Qwen3 (S1-mini, Qwen3-ASR) and Whisper (src/text/bpe.rs,
// src/text/mod.rs): every byte has a printable stand-in character, a token
// is a string of stand-ins, the text is cut into words by Trit's
// restatement of the pre-tokenizer regex, and each word's bytes are merged
// by rank. Host code: tokenization runs before and after the device loop.
// Also the prompt of Trit's transcript cleanup (src/cleanup.rs), which
// feeds the decoder.
#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <queue>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/trit_hip.h"
#include "internal.h"
#include "unicode_tables.h"

namespace trit {
namespace {

// ---- UTF-8 ------------------------------------------------------------

void put_utf8(std::string& out, uint32_t cp) {
    if (cp < 0x80) {
        out += (char)cp;
    } else if (cp < 0x800) {
        out += (char)(0xC0 | (cp >> 6));
        out += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
        out += (char)(0xE0 | (cp >> 12));
        out += (char)(0x80 | ((cp >> 6) & 0x3F));
        out += (char)(0x80 | (cp & 0x3F));
    } else {
        out += (char)(0xF0 | (cp >> 18));
        out += (char)(0x80 | ((cp >> 12) & 0x3F));
        out += (char)(0x80 | ((cp >> 6) & 0x3F));
        out += (char)(0x80 | (cp & 0x3F));
    }
}

// The length of the valid UTF-8 sequence at s[i..n), or 0: shortest forms,
// no surrogates, at most U+10FFFF (the rules of Rust's str).
int utf8_len(const unsigned char* s, size_t i, size_t n, uint32_t* cp) {
    const unsigned char b = s[i];
    if (b < 0x80) {
        *cp = b;
        return 1;
    }
    int len;
    uint32_t lo = 0x80, hi = 0xBF, v;
    if (b >= 0xC2 && b <= 0xDF) len = 2, v = b & 0x1F;
    else if (b >= 0xE0 && b <= 0xEF) {
        len = 3, v = b & 0x0F;
        if (b == 0xE0) lo = 0xA0;
        if (b == 0xED) hi = 0x9F;
    } else if (b >= 0xF0 && b <= 0xF4) {
        len = 4, v = b & 0x07;
        if (b == 0xF0) lo = 0x90;
        if (b == 0xF4) hi = 0x8F;
    } else {
        return 0;
    }
    for (int k = 1; k < len; ++k) {
        if (i + k >= n) return 0;
        const unsigned char c = s[i + k];
        if (c < (k == 1 ? lo : 0x80) || c > (k == 1 ? hi : 0xBF)) return 0;
        v = (v << 6) | (c & 0x3F);
    }
    *cp = v;
    return len;
}

// String::from_utf8_lossy: each maximal invalid subpart becomes U+FFFD.
std::string lossy_utf8(const std::string& bytes) {
    std::string out;
    const unsigned char* s = (const unsigned char*)bytes.data();
    const size_t n = bytes.size();
    size_t i = 0;
    while (i < n) {
        uint32_t cp;
        const int len = utf8_len(s, i, n, &cp);
        if (len) {
            out.append(bytes, i, len);
            i += len;
            continue;
        }
        // The maximal subpart: the lead byte and the continuation bytes that
        // a valid sequence could still have had.
        const unsigned char b = s[i];
        size_t j = i + 1;
        int need = b >= 0xC2 && b <= 0xDF ? 1 : b >= 0xE0 && b <= 0xEF ? 2 : b >= 0xF0 && b <= 0xF4 ? 3 : 0;
        for (int k = 1; k <= need && j < n; ++k, ++j) {
            const unsigned char c = s[j];
            unsigned char lo = 0x80, hi = 0xBF;
            if (k == 1) {
                if (b == 0xE0) lo = 0xA0;
                if (b == 0xED) hi = 0x9F;
                if (b == 0xF0) lo = 0x90;
                if (b == 0xF4) hi = 0x8F;
            }
            if (c < lo || c > hi) break;
        }
        put_utf8(out, 0xFFFD);
        i = j;
    }
    return out;
}

// text::lossy (src/text/mod.rs:76-96): a last character cut short is
// dropped; other invalid bytes become U+FFFD.
std::string lossy(const std::string& bytes) {
    const size_t len = bytes.size();
    size_t keep = len;
    for (size_t back = 1; back <= std::min<size_t>(len, 4); ++back) {
        const unsigned char byte = (unsigned char)bytes[len - back];
        if ((byte & 0xC0) == 0x80) continue;
        const size_t needs = byte >= 0xC0 && byte <= 0xDF ? 2 : byte >= 0xE0 && byte <= 0xEF ? 3
                             : byte >= 0xF0 && byte <= 0xF7 ? 4 : 1;
        if (needs > back) keep = len - back;
        break;
    }
    return lossy_utf8(bytes.substr(0, keep));
}

// ---- Unicode properties (Rust's char methods) ---------------------------

template <size_t N>
bool in_table(const uint32_t (&t)[N][2], uint32_t cp) {
    size_t lo = 0, hi = N;
    while (lo < hi) {
        const size_t mid = (lo + hi) / 2;
        if (cp < t[mid][0]) hi = mid;
        else if (cp > t[mid][1]) lo = mid + 1;
        else return true;
    }
    return false;
}
bool is_alphabetic(uint32_t c) { return in_table(unicode::alphabetic, c); }
bool is_numeric(uint32_t c) { return in_table(unicode::numeric, c); }
bool is_whitespace(uint32_t c) { return in_table(unicode::white_space, c); }

// ---- JSON (the parts of tokenizer.json the tokenizer reads) -------------

struct Json {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    bool b = false;
    double num = 0;
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;
    const Json* get(const char* key) const {
        if (kind != OBJ) return nullptr;
        for (const auto& kv : obj)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
};

struct JsonParser {
    const char* p;
    const char* end;
    int depth = 0;
    [[noreturn]] void bad(const char* what) { fail(std::string("tokenizer.json is not JSON: ") + what); }
    void ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
    }
    uint32_t hex4() {
        if (end - p < 4) bad("short \\u escape");
        uint32_t v = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = *p++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= c - '0';
            else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
            else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
            else bad("bad \\u escape");
        }
        return v;
    }
    std::string string() {
        if (p >= end || *p != '"') bad("expected a string");
        ++p;
        std::string out;
        while (true) {
            if (p >= end) bad("unterminated string");
            const char c = *p++;
            if (c == '"') break;
            if (c != '\\') {
                out += c;
                continue;
            }
            if (p >= end) bad("unterminated escape");
            const char e = *p++;
            switch (e) {
                case '"': out += '"'; break;
                case '\\': out += '\\'; break;
                case '/': out += '/'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'u': {
                    uint32_t cp = hex4();
                    if (cp >= 0xD800 && cp <= 0xDBFF && end - p >= 6 && p[0] == '\\' && p[1] == 'u') {
                        const char* save = p;
                        p += 2;
                        const uint32_t lo = hex4();
                        if (lo >= 0xDC00 && lo <= 0xDFFF) cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                        else p = save;
                    }
                    if (cp >= 0xD800 && cp <= 0xDFFF) cp = 0xFFFD;  // a lone surrogate
                    put_utf8(out, cp);
                    break;
                }
                default: bad("bad escape");
            }
        }
        return out;
    }
    Json value() {
        ws();
        if (p >= end) bad("unexpected end");
        Json j;
        if (*p == '{') {
            if (++depth > 64) bad("nested too deep");
            ++p;
            j.kind = Json::OBJ;
            ws();
            if (p < end && *p == '}') {
                ++p;
            } else {
                while (true) {
                    ws();
                    std::string key = string();
                    ws();
                    if (p >= end || *p != ':') bad("expected ':'");
                    ++p;
                    j.obj.emplace_back(std::move(key), value());
                    ws();
                    if (p < end && *p == ',') { ++p; continue; }
                    if (p < end && *p == '}') { ++p; break; }
                    bad("expected ',' or '}'");
                }
            }
            --depth;
        } else if (*p == '[') {
            if (++depth > 64) bad("nested too deep");
            ++p;
            j.kind = Json::ARR;
            ws();
            if (p < end && *p == ']') {
                ++p;
            } else {
                while (true) {
                    j.arr.push_back(value());
                    ws();
                    if (p < end && *p == ',') { ++p; continue; }
                    if (p < end && *p == ']') { ++p; break; }
                    bad("expected ',' or ']'");
                }
            }
            --depth;
        } else if (*p == '"') {
            j.kind = Json::STR;
            j.str = string();
        } else if (end - p >= 4 && !std::strncmp(p, "true", 4)) {
            j.kind = Json::BOOL, j.b = true, p += 4;
        } else if (end - p >= 5 && !std::strncmp(p, "false", 5)) {
            j.kind = Json::BOOL, j.b = false, p += 5;
        } else if (end - p >= 4 && !std::strncmp(p, "null", 4)) {
            p += 4;
        } else {
            const char* s = p;
            if (p < end && (*p == '-' || *p == '+')) ++p;
            while (p < end && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' || *p == '-' ||
                               *p == '+'))
                ++p;
            if (p == s) bad("unexpected character");
            j.kind = Json::NUM;
            j.num = std::strtod(std::string(s, p).c_str(), nullptr);
        }
        return j;
    }
};

// ---- BPE ----------------------------------------------------------------

// GPT-2's bytes_to_unicode (src/text/bpe.rs:356-369): printable bytes stand
// for themselves, the other 68 take U+0100 and up in byte order.
struct ByteMap {
    uint32_t to_char[256];
    std::unordered_map<uint32_t, uint8_t> to_byte;
    ByteMap() {
        uint32_t next = 0;
        for (int b = 0; b < 256; ++b) {
            const bool printable = (b >= '!' && b <= '~') || (b >= 0xA1 && b <= 0xAC) || (b >= 0xAE && b <= 0xFF);
            to_char[b] = printable ? (uint32_t)b : 255 + ++next;
            to_byte[to_char[b]] = (uint8_t)b;
        }
    }
};
const ByteMap& byte_map() {
    static const ByteMap m;
    return m;
}

enum Split { GPT2, QWEN };

}  // namespace

// The tokenizer (Bpe, src/text/bpe.rs:11-22).
struct Bpe {
    std::vector<std::string> pieces;  // id -> bytes; special tokens their text
    std::vector<bool> special;
    std::unordered_map<std::string, int> ids;  // token as written -> id
    // Merge rank of "left\0right"; the lower merges first.
    std::unordered_map<std::string, int> ranks;
    std::vector<std::pair<std::string, int>> specials;  // text, id; longest first
    Split split = GPT2;

    int rank(const std::string& left, const std::string& right) const {
        std::string key;
        key.reserve(left.size() + right.size() + 1);
        key += left;
        key += '\0';
        key += right;
        auto it = ranks.find(key);
        return it == ranks.end() ? -1 : it->second;
    }

    // text::merge_symbols (src/text/mod.rs:6-74): the lowest rank first,
    // the leftmost of equal ranks; a heap of offers, stale ones skipped.
    void merge(std::vector<std::string>& symbols) const {
        const int count = (int)symbols.size();
        if (count < 2) return;
        constexpr int NONE = -1;
        std::vector<int> next(count), before(count);
        std::vector<uint32_t> grown(count, 0);
        std::vector<bool> gone(count, false);
        for (int i = 0; i < count; ++i) {
            next[i] = i + 1 < count ? i + 1 : NONE;
            before[i] = i - 1;
        }
        using Offer = std::tuple<int, int, uint32_t, uint32_t>;  // rank, left, its growth, right's growth
        std::priority_queue<Offer, std::vector<Offer>, std::greater<Offer>> pairs;
        auto offer = [&](int left) {
            const int right = next[left];
            if (right == NONE) return;
            const int r = rank(symbols[left], symbols[right]);
            if (r >= 0) pairs.emplace(r, left, grown[left], grown[right]);
        };
        for (int left = 0; left < count - 1; ++left) offer(left);
        while (!pairs.empty()) {
            const auto [r, left, gl, gr] = pairs.top();
            pairs.pop();
            (void)r;
            const int right = next[left];
            if (gone[left] || right == NONE || grown[left] != gl || grown[right] != gr) continue;
            symbols[left] += symbols[right];
            symbols[right].clear();
            gone[right] = true;
            grown[left] += 1;
            next[left] = next[right];
            if (next[left] != NONE) before[next[left]] = left;
            if (before[left] != NONE) offer(before[left]);
            offer(left);
        }
        int w = 0;
        for (int i = 0; i < count; ++i)
            if (!gone[i]) {
                if (w != i) symbols[w] = std::move(symbols[i]);
                ++w;
            }
        symbols.resize(w);
    }

    // Bpe::merge_word (src/text/bpe.rs:239-258).
    void merge_word(const std::string& word, std::vector<int>& out) const {
        const ByteMap& m = byte_map();
        std::vector<std::string> symbols;
        symbols.reserve(word.size());
        for (unsigned char b : word) {
            std::string s;
            put_utf8(s, m.to_char[b]);
            symbols.push_back(std::move(s));
        }
        merge(symbols);
        for (const auto& s : symbols) {
            auto it = ids.find(s);
            if (it != ids.end()) out.push_back(it->second);
        }
    }

    // pretokenize (src/text/bpe.rs:260-354): the words the regex of the
    // split would cut, by Trit's restatement of it.
    std::vector<std::string> pretokenize(const std::string& text) const {
        std::vector<uint32_t> cs;
        std::vector<size_t> offs;
        const unsigned char* s = (const unsigned char*)text.data();
        for (size_t i = 0; i < text.size();) {
            uint32_t cp;
            int len = utf8_len(s, i, text.size(), &cp);
            if (!len) fail("tokenizer: the text is not UTF-8");
            cs.push_back(cp);
            offs.push_back(i);
            i += len;
        }
        const size_t n = cs.size();
        auto at = [&](size_t i, uint32_t* c) {
            if (i >= n) return false;
            *c = cs[i];
            return true;
        };
        auto offset = [&](size_t i) { return i < n ? offs[i] : text.size(); };
        auto letter = [](uint32_t c) { return is_alphabetic(c); };
        auto number = [](uint32_t c) { return is_numeric(c); };
        auto newline = [](uint32_t c) { return c == '\r' || c == '\n'; };
        auto other = [&](uint32_t c) { return !is_whitespace(c) && !letter(c) && !number(c); };
        auto run = [&](size_t j, auto f) {
            uint32_t c;
            while (at(j, &c) && f(c)) ++j;
            return j;
        };
        std::vector<std::string> words;
        size_t i = 0;
        while (i < n) {
            const uint32_t c = cs[i];
            const size_t start = i;
            if (c == '\'') {
                // Contractions 's 't 're 've 'm 'll 'd (Qwen: any case, as
                // to_lowercase gives them only from ASCII letters).
                std::string tail;
                for (size_t k = i + 1; k < std::min(n, i + 3); ++k) {
                    uint32_t t = cs[k];
                    if (split == QWEN && t >= 'A' && t <= 'Z') t += 32;
                    put_utf8(tail, t);
                }
                auto starts = [&](const char* p) { return tail.compare(0, std::strlen(p), p) == 0; };
                size_t len = (starts("re") || starts("ve") || starts("ll")) ? 2
                             : (starts("s") || starts("t") || starts("m") || starts("d")) ? 1 : 0;
                if (len) {
                    i += 1 + len;
                    words.push_back(text.substr(offset(start), offset(i) - offset(start)));
                    continue;
                }
            }
            bool matched = false;
            size_t end = 0;
            uint32_t f;
            if (split == GPT2) {
                const size_t lead = (c == ' ' && at(i + 1, &f) && !is_whitespace(f)) ? 1 : 0;
                uint32_t first = ' ';
                at(i + lead, &first);
                if (letter(first)) matched = true, end = run(i + lead, letter);
                else if (number(first)) matched = true, end = run(i + lead, number);
                else if (other(first)) matched = true, end = run(i + lead, other);
            } else {
                const size_t lead = (!newline(c) && !letter(c) && !number(c)) ? 1 : 0;
                if (at(i + lead, &f) && letter(f)) {
                    matched = true, end = run(i + lead, letter);
                } else if (number(c)) {
                    matched = true, end = i + 1;
                } else {
                    const size_t lead2 = c == ' ' ? 1 : 0;
                    if (at(i + lead2, &f) && other(f)) matched = true, end = run(run(i + lead2, other), newline);
                }
            }
            if (matched) {
                i = end;
            } else {
                // Whitespace. Qwen first takes \s*[\r\n]+: up to the last newline.
                const size_t space_end = run(i, [](uint32_t x) { return is_whitespace(x); });
                size_t last_nl = (size_t)-1;
                for (size_t j = space_end; j > i; --j)
                    if (newline(cs[j - 1])) {
                        last_nl = j - 1;
                        break;
                    }
                if (split == QWEN && last_nl != (size_t)-1) i = last_nl + 1;
                else if (space_end < n && space_end - i > 1) i = space_end - 1;  // \s+(?!\S)
                else i = space_end;
            }
            words.push_back(text.substr(offset(start), offset(i) - offset(start)));
        }
        return words;
    }

    // Bpe::encode / encode_plain (src/text/bpe.rs:197-237).
    std::vector<int> encode(const std::string& text, bool plain) const {
        std::vector<int> out;
        if (plain) {
            for (const auto& w : pretokenize(text)) merge_word(w, out);
            return out;
        }
        size_t rest = 0;
        while (rest < text.size()) {
            // The first special token in the rest; the longest at one place.
            size_t best_at = std::string::npos, best_len = 0;
            int best_id = -1;
            for (const auto& sp : specials) {
                const size_t at = text.find(sp.first, rest);
                if (at == std::string::npos) continue;
                if (at < best_at || (at == best_at && sp.first.size() > best_len))
                    best_at = at, best_len = sp.first.size(), best_id = sp.second;
            }
            const size_t plain_end = best_at == std::string::npos ? text.size() : best_at;
            for (const auto& w : pretokenize(text.substr(rest, plain_end - rest))) merge_word(w, out);
            if (best_id < 0) break;
            out.push_back(best_id);
            rest = plain_end + best_len;
        }
        return out;
    }

    // Bpe::decode (src/text/bpe.rs:185-195).
    std::string decode(const int32_t* toks, int n) const {
        std::string bytes;
        for (int i = 0; i < n; ++i) {
            const int id = toks[i];
            if (id >= 0 && id < (int)pieces.size() && !special[id]) bytes += pieces[id];
        }
        return lossy(bytes);
    }
};

namespace {

constexpr size_t MAX_ID_GAP = (size_t)1 << 16;

// Bpe::build (src/text/bpe.rs:115-174).
Bpe* build(const std::vector<std::pair<std::string, int64_t>>& vocab,
           const std::vector<std::pair<std::string, std::string>>& merges,
           const std::vector<std::tuple<int64_t, std::string, bool>>& added, Split split) {
    const ByteMap& m = byte_map();
    struct Entry {
        int64_t id;
        std::string bytes;
        bool special;
        std::string text;
    };
    std::vector<Entry> entries;
    entries.reserve(vocab.size() + added.size());
    for (const auto& [token, id] : vocab) {
        if (id < 0) fail("the vocabulary has a bad id");
        std::string bytes;
        const unsigned char* s = (const unsigned char*)token.data();
        for (size_t i = 0; i < token.size();) {
            uint32_t cp;
            const int len = utf8_len(s, i, token.size(), &cp);
            if (!len) fail("the vocabulary has a token that is not UTF-8");
            auto it = m.to_byte.find(cp);
            bytes += it == m.to_byte.end() ? '?' : (char)it->second;
            i += len;
        }
        entries.push_back({id, std::move(bytes), false, token});
    }
    auto B = std::make_unique<Bpe>();
    for (const auto& [id, content, special] : added) {
        if (id < 0) fail("an added token has a bad id");
        B->specials.emplace_back(content, (int)id);
        entries.push_back({id, content, special, content});
    }
    std::stable_sort(B->specials.begin(), B->specials.end(),
                     [](const auto& a, const auto& b) { return a.first.size() > b.first.size(); });
    int64_t largest = -1;
    for (const auto& e : entries) largest = std::max(largest, e.id);
    if (largest >= 0 && (size_t)largest >= entries.size() * 2 + MAX_ID_GAP)
        fail("the tokenizer's id " + std::to_string(largest) + " is far past its " + std::to_string(entries.size()) +
             " tokens");
    const size_t size = (size_t)(largest + 1);
    B->pieces.assign(size, std::string());
    B->special.assign(size, false);
    B->ids.reserve(size);
    for (auto& e : entries) {
        B->pieces[e.id] = e.bytes;
        B->special[e.id] = e.special;
        B->ids[e.text] = (int)e.id;
    }
    int r = 0;
    for (const auto& [left, right] : merges) {
        std::string key = left;
        key += '\0';
        key += right;
        B->ranks.emplace(std::move(key), r++);  // the first rank of a pair stays
    }
    B->split = split;
    return B.release();
}

// text::parse_merge (src/text/mod.rs:98-107): ["a", "b"] or "a b".
bool parse_merge(const Json& v, std::pair<std::string, std::string>& out) {
    if (v.kind == Json::ARR) {
        if (v.arr.size() < 2 || v.arr[0].kind != Json::STR || v.arr[1].kind != Json::STR) return false;
        out = {v.arr[0].str, v.arr[1].str};
        return true;
    }
    if (v.kind == Json::STR) {
        const size_t sp = v.str.find(' ');
        if (sp == std::string::npos) return false;
        out = {v.str.substr(0, sp), v.str.substr(sp + 1)};
        return true;
    }
    return false;
}

// Json::to_string of the pre_tokenizer as serde_json writes it: the Qwen
// test of Bpe::parse looks for the Qwen regex's text in it, escapes as JSON
// writes them ("\\p{L}" for \p{L}).
void json_text(const Json& j, std::string& out) {
    switch (j.kind) {
        case Json::NUL: out += "null"; break;
        case Json::BOOL: out += j.b ? "true" : "false"; break;
        case Json::NUM: {
            char buf[32];
            std::snprintf(buf, sizeof buf, "%.17g", j.num);
            out += buf;
            break;
        }
        case Json::STR:
            out += '"';
            for (unsigned char c : j.str) {
                if (c == '"') out += "\\\"";
                else if (c == '\\') out += "\\\\";
                else if (c == '\n') out += "\\n";
                else if (c == '\r') out += "\\r";
                else if (c == '\t') out += "\\t";
                else if (c < 0x20) {
                    char buf[8];
                    std::snprintf(buf, sizeof buf, "\\u%04x", c);
                    out += buf;
                } else out += (char)c;
            }
            out += '"';
            break;
        case Json::ARR:
            out += '[';
            for (size_t i = 0; i < j.arr.size(); ++i) {
                if (i) out += ',';
                json_text(j.arr[i], out);
            }
            out += ']';
            break;
        case Json::OBJ:
            out += '{';
            for (size_t i = 0; i < j.obj.size(); ++i) {
                if (i) out += ',';
                Json k;
                k.kind = Json::STR;
                k.str = j.obj[i].first;
                json_text(k, out);
                out += ':';
                json_text(j.obj[i].second, out);
            }
            out += '}';
            break;
    }
}

// Bpe::parse (src/text/bpe.rs:82-113).
Bpe* parse(const char* text, size_t len) {
    JsonParser P{text, text + len};
    const Json root = P.value();
    const Json* model = root.get("model");
    const Json* vocab = model ? model->get("vocab") : nullptr;
    if (!vocab || vocab->kind != Json::OBJ) fail("tokenizer.json has no model.vocab");
    std::vector<std::pair<std::string, int64_t>> v;
    v.reserve(vocab->obj.size());
    for (const auto& [token, id] : vocab->obj) {
        if (id.kind != Json::NUM || id.num < 0 || id.num != (double)(int64_t)id.num)
            fail("the vocabulary has a bad id");
        v.emplace_back(token, (int64_t)id.num);
    }
    std::vector<std::tuple<int64_t, std::string, bool>> added;
    if (const Json* a = root.get("added_tokens"); a && a->kind == Json::ARR)
        for (const Json& t : a->arr) {
            const Json* id = t.get("id");
            const Json* content = t.get("content");
            if (!id || id->kind != Json::NUM || id->num < 0 || !content || content->kind != Json::STR) continue;
            const Json* sp = t.get("special");
            added.emplace_back((int64_t)id->num, content->str, sp && sp->kind == Json::BOOL ? sp->b : true);
        }
    std::vector<std::pair<std::string, std::string>> merges;
    if (const Json* mg = model->get("merges"); mg && mg->kind == Json::ARR)
        for (const Json& m : mg->arr) {
            std::pair<std::string, std::string> pr;
            if (parse_merge(m, pr)) merges.push_back(std::move(pr));
        }
    std::string pre;
    if (const Json* pt = root.get("pre_tokenizer")) json_text(*pt, pre);
    else pre = "null";
    const bool qwen = pre.find("[^\\\\r\\\\n\\\\p{L}\\\\p{N}]?\\\\p{L}+") != std::string::npos;
    return build(v, merges, added, qwen ? QWEN : GPT2);
}

const char* SYSTEM =
    "You are a text normalizer for speech-to-text transcripts. The input begins with a control line "
    "specifying the styling, structure, and context settings; clean the transcript to match those settings "
    "and output only the cleaned text.";
const char* STYLING[] = {"casual", "semi-casual", "semi-formal", "formal"};
const char* STRUCTURE[] = {"prose", "lists"};
const char* CONTEXT[] = {"general", "email"};

std::string system_prefix() {
    return std::string("<|im_start|>system\n") + SYSTEM + "<|im_end|>\n<|im_start|>user\n";
}

// str::trim: Unicode White_Space off both ends.
std::string trim(const std::string& t) {
    const unsigned char* s = (const unsigned char*)t.data();
    size_t a = 0, b = t.size();
    while (a < b) {
        uint32_t cp;
        const int len = utf8_len(s, a, b, &cp);
        if (!len || !is_whitespace(cp)) break;
        a += len;
    }
    while (b > a) {
        size_t k = b - 1;
        while (k > a && (s[k] & 0xC0) == 0x80) --k;
        uint32_t cp;
        const int len = utf8_len(s, k, b, &cp);
        if (!len || k + len != b || !is_whitespace(cp)) break;
        b = k;
    }
    return t.substr(a, b - a);
}

// Cleaner::parts (src/cleanup.rs:240-278): whole sentences (cut after '.',
// '?' or '!' that the end or whitespace follows), joined with one space
// while the join holds at most `limit` tokens; a sentence longer alone goes
// word by word (split on whitespace).
std::vector<std::string> cleanup_parts(const Bpe& B, const std::string& text, int limit) {
    const unsigned char* s = (const unsigned char*)text.data();
    const size_t n = text.size();
    std::vector<std::string> units;
    size_t start = 0;
    for (size_t i = 0; i < n;) {
        uint32_t cp;
        const int len = utf8_len(s, i, n, &cp);
        if (!len) fail("cleanup: the transcript is not UTF-8");
        const size_t after = i + len;
        bool next_ws = true;
        if (after < n) {
            uint32_t nx;
            const int l2 = utf8_len(s, after, n, &nx);
            next_ws = l2 && is_whitespace(nx);
        }
        if ((cp == '.' || cp == '?' || cp == '!') && next_ws) {
            units.push_back(trim(text.substr(start, after - start)));
            start = after;
        }
        i = after;
    }
    units.push_back(trim(text.substr(start)));
    auto tokens = [&](const std::string& t) { return (int)B.encode(t, false).size(); };
    std::vector<std::string> parts;
    std::string current;
    for (const std::string& unit : units) {
        if (unit.empty()) continue;
        std::vector<std::string> words;
        if (tokens(unit) > limit) {
            // str::split_whitespace.
            const unsigned char* u = (const unsigned char*)unit.data();
            size_t i = 0, w = std::string::npos;
            while (i <= unit.size()) {
                uint32_t cp = ' ';
                int len = 1;
                if (i < unit.size()) {
                    len = utf8_len(u, i, unit.size(), &cp);
                    if (!len) fail("cleanup: the transcript is not UTF-8");
                }
                const bool ws = i == unit.size() || is_whitespace(cp);
                if (ws && w != std::string::npos) {
                    words.push_back(unit.substr(w, i - w));
                    w = std::string::npos;
                } else if (!ws && w == std::string::npos) {
                    w = i;
                }
                i += len;
            }
        } else {
            words.push_back(unit);
        }
        for (const std::string& piece : words) {
            const std::string joined = current.empty() ? piece : current + " " + piece;
            if (tokens(joined) > limit && !current.empty()) {
                parts.push_back(current);
                current = piece;
            } else {
                current = joined;
            }
        }
    }
    if (!current.empty()) parts.push_back(current);
    return parts;
}

int copy_ids(const std::vector<int>& ids, int32_t* out, int cap) {
    if (cap < 0) fail("tokenizer: negative capacity");
    if (cap && !out) fail("tokenizer: out is NULL");
    for (int i = 0; i < (int)ids.size() && i < cap; ++i) out[i] = ids[i];
    return (int)ids.size();
}

}  // namespace
}  // namespace trit

struct TritHipBpe {
    std::unique_ptr<trit::Bpe> bpe;
};

using namespace trit;

extern "C" {

int trit_hip_bpe_parse(const char* json, size_t len, TritHipBpe** out) {
    return guard(-1, [&] {
        if (!json || !out) fail("tokenizer: json or out is NULL");
        *out = new TritHipBpe{std::unique_ptr<Bpe>(parse(json, len))};
        return 0;
    });
}

int trit_hip_bpe_open(const char* path, TritHipBpe** out) {
    return guard(-1, [&] {
        if (!path || !out) fail("tokenizer: path or out is NULL");
        FILE* f = std::fopen(path, "rb");
        if (!f) fail(std::string("cannot read ") + path);
        std::string text;
        char buf[1 << 16];
        size_t got;
        while ((got = std::fread(buf, 1, sizeof buf, f)) > 0) text.append(buf, got);
        std::fclose(f);
        *out = new TritHipBpe{std::unique_ptr<Bpe>(parse(text.data(), text.size()))};
        return 0;
    });
}

void trit_hip_bpe_free(TritHipBpe* bpe) { delete bpe; }

int trit_hip_bpe_id(const TritHipBpe* bpe, const char* token) {
    return guard(-1, [&] {
        if (!bpe || !token) fail("tokenizer: bpe or token is NULL");
        auto it = bpe->bpe->ids.find(token);
        return it == bpe->bpe->ids.end() ? -1 : it->second;
    });
}

int trit_hip_bpe_encode(const TritHipBpe* bpe, const char* text, size_t len, int plain, int32_t* out, int cap) {
    return guard(-1, [&] {
        if (!bpe || (!text && len)) fail("tokenizer: bpe or text is NULL");
        return copy_ids(bpe->bpe->encode(std::string(text ? text : "", len), plain != 0), out, cap);
    });
}

int64_t trit_hip_bpe_decode(const TritHipBpe* bpe, const int32_t* ids, int n, char* out, size_t cap) {
    return guard((int64_t)-1, [&] {
        if (!bpe || (n && !ids) || n < 0) fail("tokenizer: bpe or ids is NULL");
        const std::string s = bpe->bpe->decode(ids, n);
        if (cap && !out) fail("tokenizer: out is NULL");
        if (cap) {
            const size_t k = std::min(cap - 1, s.size());
            std::memcpy(out, s.data(), k);
            out[k] = '\0';
        }
        return (int64_t)s.size();
    });
}

int trit_hip_cleanup_system(const TritHipBpe* bpe, int32_t* out, int cap) {
    return guard(-1, [&] {
        if (!bpe) fail("tokenizer: bpe is NULL");
        return copy_ids(bpe->bpe->encode(system_prefix(), false), out, cap);
    });
}

int trit_hip_cleanup_prompt(const TritHipBpe* bpe, const char* transcript, size_t len, int styling, int structure,
                            int context, int32_t* out, int cap) {
    return guard(-1, [&] {
        if (!bpe || (!transcript && len)) fail("tokenizer: bpe or transcript is NULL");
        if (styling < 0 || styling > 3 || structure < 0 || structure > 1 || context < 0 || context > 1)
            fail("cleanup: a style setting is out of range");
        const Bpe& B = *bpe->bpe;
        const std::string control = std::string("[Styling: ") + STYLING[styling] + "] [Structure: " +
                                    STRUCTURE[structure] + "] [Context: " + CONTEXT[context] + "]";
        std::vector<int> ids = B.encode(system_prefix() + control + "\n", false);
        const std::vector<int> body = B.encode(std::string(transcript ? transcript : "", len), true);
        ids.insert(ids.end(), body.begin(), body.end());
        const std::vector<int> tail = B.encode("<|im_end|>\n<|im_start|>assistant\n<think>\n\n</think>\n\n", false);
        ids.insert(ids.end(), tail.begin(), tail.end());
        return copy_ids(ids, out, cap);
    });
}

int64_t trit_hip_cleanup_parts(const TritHipBpe* bpe, const char* transcript, size_t len, int limit, char* out,
                               size_t cap) {
    return guard((int64_t)-1, [&] {
        if (!bpe || (!transcript && len)) fail("tokenizer: bpe or transcript is NULL");
        if (limit <= 0) fail("cleanup: the part limit must be positive");
        const std::vector<std::string> parts =
            cleanup_parts(*bpe->bpe, trim(std::string(transcript ? transcript : "", len)), limit);
        std::string all;
        for (const auto& p : parts) {
            all += p;
            all += '\0';
        }
        if (cap && !out) fail("tokenizer: out is NULL");
        if (cap) std::memcpy(out, all.data(), std::min(cap, all.size()));
        return (int64_t)all.size();
    });
}

}  // extern "C"
