// Byte-level BPE from a Hugging Face tokenizer.json, with the behaviour of
// Trit's tokenizer for Qwen3 (S1-mini, Qwen3-ASR) and Whisper
// (src/text/bpe.rs, src/text/mod.rs), and the prompt of Trit's transcript
// cleanup (src/cleanup.rs), which feeds the decoder. Host code: it runs
// before and after the device loop.
//
// What is fixed by the contract: the byte stand-in characters (GPT-2's
// table), the word split (Trit's reading of the Qwen2 / GPT-2 pre-tokenizer
// regex, which counts Alphabetic rather than \p{L}), the merge order (the
// pair of lowest rank first, the leftmost of equal ranks), the lossy decode,
// and the error texts callers match. How it is computed is this file's own:
//
//  - Every string that can be a symbol during merging (the 256 byte
//    stand-ins, both sides of each merge and their join) is interned once at
//    load, so a merge is a lookup of an (int, int) key and the merged
//    symbol's id, and no string is built while a word is merged.
//  - A word's pairs sit in an addressable binary heap keyed (rank, position):
//    a merge updates the two pairs it changes in place and deletes the one it
//    consumes, so the heap only ever holds live pairs.
//  - The text is classified once (letter / number / white space / newline
//    flags per code point), and each alternative of the split is a small
//    matcher over those flags that returns where its word ends.
#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/trit_hip.h"
#include "internal.h"
#include "unicode_tables.h"

namespace trit {
namespace {

// ---- UTF-8 ------------------------------------------------------------

void append_utf8(std::string& out, uint32_t cp) {
    char b[4];
    int n;
    if (cp < 0x80) {
        b[0] = (char)cp, n = 1;
    } else if (cp < 0x800) {
        b[0] = (char)(0xC0 | cp >> 6), b[1] = (char)(0x80 | (cp & 0x3F)), n = 2;
    } else if (cp < 0x10000) {
        b[0] = (char)(0xE0 | cp >> 12), b[1] = (char)(0x80 | (cp >> 6 & 0x3F)), b[2] = (char)(0x80 | (cp & 0x3F)), n = 3;
    } else {
        b[0] = (char)(0xF0 | cp >> 18), b[1] = (char)(0x80 | (cp >> 12 & 0x3F)), b[2] = (char)(0x80 | (cp >> 6 & 0x3F));
        b[3] = (char)(0x80 | (cp & 0x3F)), n = 4;
    }
    out.append(b, n);
}

// The range the second byte of a sequence may take after lead byte `lead`
// (shortest forms only, no surrogates, nothing past U+10FFFF); later
// continuation bytes are 0x80..0xBF.
struct Lead {
    int len;                  // sequence length, 0 for a byte that cannot lead
    unsigned char lo, hi;     // the second byte's range
};
Lead lead_of(unsigned char b) {
    if (b < 0x80) return {1, 0, 0};
    if (b >= 0xC2 && b <= 0xDF) return {2, 0x80, 0xBF};
    if (b == 0xE0) return {3, 0xA0, 0xBF};
    if (b == 0xED) return {3, 0x80, 0x9F};
    if (b >= 0xE1 && b <= 0xEF) return {3, 0x80, 0xBF};
    if (b == 0xF0) return {4, 0x90, 0xBF};
    if (b >= 0xF1 && b <= 0xF3) return {4, 0x80, 0xBF};
    if (b == 0xF4) return {4, 0x80, 0x8F};
    return {0, 0, 0};
}

// How many bytes at s[i..n) belong to the sequence that starts there:
// `valid` tells whether they form a whole character (then *cp is it), else
// they are the maximal ill-formed subpart (the lead and the continuation
// bytes that a valid character could still have had; at least one byte).
size_t scan_utf8(const unsigned char* s, size_t i, size_t n, bool* valid, uint32_t* cp) {
    const Lead L = lead_of(s[i]);
    if (L.len == 1) {
        *valid = true, *cp = s[i];
        return 1;
    }
    *valid = false;
    if (L.len == 0) return 1;
    uint32_t v = s[i] & (0x7F >> L.len);
    size_t k = 1;
    for (; k < (size_t)L.len && i + k < n; ++k) {
        const unsigned char c = s[i + k];
        const unsigned char lo = k == 1 ? L.lo : 0x80, hi = k == 1 ? L.hi : 0xBF;
        if (c < lo || c > hi) return k;
        v = v << 6 | (c & 0x3F);
    }
    if (k < (size_t)L.len) return k;  // cut short by the end
    *valid = true, *cp = v;
    return k;
}

// The code points of a text that must be UTF-8 (`what` names it in the error).
void decode_utf8(const std::string& text, std::vector<uint32_t>& cps, std::vector<uint32_t>* offsets,
                 const char* what) {
    const unsigned char* s = (const unsigned char*)text.data();
    for (size_t i = 0; i < text.size();) {
        bool ok;
        uint32_t cp;
        const size_t len = scan_utf8(s, i, text.size(), &ok, &cp);
        if (!ok) fail(std::string(what) + " is not UTF-8");
        cps.push_back(cp);
        if (offsets) offsets->push_back((uint32_t)i);
        i += len;
    }
}

bool is_utf8(const char* p, size_t n) {
    const unsigned char* s = (const unsigned char*)p;
    for (size_t i = 0; i < n;) {
        bool ok;
        uint32_t cp;
        i += scan_utf8(s, i, n, &ok, &cp);
        if (!ok) return false;
    }
    return true;
}

// Decoded bytes as text (text::lossy, src/text/mod.rs:76-96): when the
// last non-continuation byte among the final four announces more bytes
// than follow it, the bytes from it on are a character the decode stopped
// inside, and are dropped; every other ill-formed subpart becomes U+FFFD
// (String::from_utf8_lossy).
std::string bytes_to_text(const std::string& bytes) {
    size_t keep = bytes.size();
    const size_t window = std::min<size_t>(4, keep);
    for (size_t back = 1; back <= window; ++back) {
        const unsigned char b = (unsigned char)bytes[keep - back];
        if ((b & 0xC0) == 0x80) continue;
        const size_t announced = b < 0xC0 ? 1 : b < 0xE0 ? 2 : b < 0xF0 ? 3 : b < 0xF8 ? 4 : 1;
        if (announced > back) keep -= back;
        break;
    }
    std::string out;
    out.reserve(keep);
    const unsigned char* s = (const unsigned char*)bytes.data();
    for (size_t i = 0; i < keep;) {
        bool ok;
        uint32_t cp;
        const size_t len = scan_utf8(s, i, keep, &ok, &cp);
        if (ok) out.append(bytes, i, len);
        else out += "\xEF\xBF\xBD";
        i += len;
    }
    return out;
}

// ---- Unicode properties of Rust's char methods --------------------------

template <size_t N>
bool in_ranges(const uint32_t (&t)[N][2], uint32_t cp) {
    // The first range that ends at or after cp.
    const auto* it = std::lower_bound(&t[0], &t[0] + N, cp, [](const uint32_t(&r)[2], uint32_t c) { return r[1] < c; });
    return it != &t[0] + N && (*it)[0] <= cp;
}

enum CharFlag : uint8_t { LETTER = 1, NUMBER = 2, SPACE = 4, NEWLINE = 8 };

uint8_t flags_of(uint32_t cp) {
    if (cp < 0x80) {  // the common case without a table search
        if ((cp | 0x20) >= 'a' && (cp | 0x20) <= 'z') return LETTER;
        if (cp >= '0' && cp <= '9') return NUMBER;
        if (cp == '\n' || cp == '\r') return SPACE | NEWLINE;
        if (cp == ' ' || (cp >= 0x09 && cp <= 0x0D)) return SPACE;
        return 0;
    }
    uint8_t f = 0;
    if (in_ranges(unicode::alphabetic, cp)) f |= LETTER;
    if (in_ranges(unicode::numeric, cp)) f |= NUMBER;
    if (in_ranges(unicode::white_space, cp)) f |= SPACE;
    return f;
}
bool is_space_cp(uint32_t cp) { return (flags_of(cp) & SPACE) != 0; }

// ---- JSON -----------------------------------------------------------------
// A strict reader of RFC 8259 text (what serde_json accepts): no trailing
// commas, no control characters in strings, no lone surrogates, integers
// told apart from other numbers (a vocabulary id must be an integer).

struct JValue {
    enum Type : uint8_t { NUL, BOOL, INT, REAL, STR, ARR, OBJ } type = NUL;
    bool flag = false;
    uint64_t u = 0;          // INT: the value (non-negative integers only)
    bool neg_or_big = false; // INT written negative or past u64
    std::string s;
    std::vector<JValue> items;                          // ARR
    std::vector<std::pair<std::string, JValue>> members;  // OBJ, in document order

    // The member `key` as a serde_json map reads it: the last of duplicates.
    const JValue* member(const char* key) const {
        if (type != OBJ) return nullptr;
        for (auto it = members.rbegin(); it != members.rend(); ++it)
            if (it->first == key) return &it->second;
        return nullptr;
    }
    bool is_u64() const { return type == INT && !neg_or_big; }
};

class JsonReader {
   public:
    JsonReader(const char* p, size_t n) : p_(p), end_(p + n) {}

    JValue document() {
        JValue v = value(0);
        skip_ws();
        if (p_ != end_) bad("trailing characters");
        return v;
    }

   private:
    const char* p_;
    const char* end_;

    [[noreturn]] void bad(const char* why) { fail(std::string("tokenizer.json is not JSON: ") + why); }
    void skip_ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool eat(char c) {
        skip_ws();
        if (p_ < end_ && *p_ == c) {
            ++p_;
            return true;
        }
        return false;
    }
    void expect(char c, const char* why) {
        if (!eat(c)) bad(why);
    }
    bool literal(const char* word) {
        const size_t n = std::strlen(word);
        if ((size_t)(end_ - p_) >= n && std::memcmp(p_, word, n) == 0) {
            p_ += n;
            return true;
        }
        return false;
    }

    uint32_t hex4() {
        if (end_ - p_ < 4) bad("EOF while parsing a string");
        uint32_t v = 0;
        for (int i = 0; i < 4; ++i, ++p_) {
            const char c = *p_;
            const int d = c >= '0' && c <= '9' ? c - '0' : c >= 'a' && c <= 'f' ? c - 'a' + 10 : c >= 'A' && c <= 'F' ? c - 'A' + 10 : -1;
            if (d < 0) bad("invalid escape");
            v = v << 4 | (uint32_t)d;
        }
        return v;
    }

    std::string string_body() {  // after the opening quote
        std::string out;
        for (;;) {
            const char* run = p_;
            while (p_ < end_ && *p_ != '"' && *p_ != '\\' && (unsigned char)*p_ >= 0x20) ++p_;
            out.append(run, p_);
            if (p_ >= end_) bad("EOF while parsing a string");
            const char c = *p_++;
            if (c == '"') return out;
            if (c != '\\') bad("control character (\\u0000-\\u001F) found while parsing a string");
            if (p_ >= end_) bad("EOF while parsing a string");
            const char e = *p_++;
            static const char from[] = "\"\\/bfnrt", to[] = "\"\\/\b\f\n\r\t";
            if (const char* hit = e ? std::strchr(from, e) : nullptr) {
                out += to[hit - from];
                continue;
            }
            if (e != 'u') bad("invalid escape");
            uint32_t cp = hex4();
            if (cp >= 0xDC00 && cp <= 0xDFFF) bad("lone leading surrogate in hex escape");
            if (cp >= 0xD800 && cp <= 0xDBFF) {
                if (end_ - p_ < 2 || p_[0] != '\\' || p_[1] != 'u') bad("unexpected end of hex escape");
                p_ += 2;
                const uint32_t low = hex4();
                if (low < 0xDC00 || low > 0xDFFF) bad("lone leading surrogate in hex escape");
                cp = 0x10000 + ((cp - 0xD800) << 10) + (low - 0xDC00);
            }
            append_utf8(out, cp);
        }
    }

    void number(JValue& v) {
        const char* start = p_;
        const bool neg = p_ < end_ && *p_ == '-';
        if (neg) ++p_;
        auto digits = [&] {
            const char* d = p_;
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
            return (size_t)(p_ - d);
        };
        const char* int_start = p_;
        const size_t nint = digits();
        if (nint == 0 || (nint > 1 && *int_start == '0')) bad("invalid number");
        bool real = false;
        if (p_ < end_ && *p_ == '.') {
            ++p_, real = true;
            if (!digits()) bad("invalid number");
        }
        if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
            ++p_, real = true;
            if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
            if (!digits()) bad("invalid number");
        }
        if (real) {
            v.type = JValue::REAL;
            (void)start;
            return;
        }
        v.type = JValue::INT;
        v.neg_or_big = neg;
        uint64_t acc = 0;
        for (const char* d = int_start; d < p_; ++d) {
            const uint64_t digit = (uint64_t)(*d - '0');
            if (acc > (UINT64_MAX - digit) / 10) {
                v.neg_or_big = true;  // serde reads it as a float
                break;
            }
            acc = acc * 10 + digit;
        }
        v.u = acc;
        if (neg && acc == 0) v.neg_or_big = false;  // "-0" is the integer 0
    }

    JValue value(int depth) {
        if (depth > 128) bad("recursion limit exceeded");
        skip_ws();
        if (p_ >= end_) bad("EOF while parsing a value");
        JValue v;
        switch (*p_) {
            case '{':
                ++p_;
                v.type = JValue::OBJ;
                if (eat('}')) break;
                do {
                    skip_ws();
                    if (p_ >= end_ || *p_ != '"') bad("key must be a string");
                    ++p_;
                    std::string key = string_body();
                    expect(':', "expected `:`");
                    v.members.emplace_back(std::move(key), value(depth + 1));
                } while (eat(','));
                expect('}', "expected `,` or `}`");
                break;
            case '[':
                ++p_;
                v.type = JValue::ARR;
                if (eat(']')) break;
                do v.items.push_back(value(depth + 1));
                while (eat(','));
                expect(']', "expected `,` or `]`");
                break;
            case '"':
                ++p_;
                v.type = JValue::STR;
                v.s = string_body();
                break;
            default:
                if (literal("true")) v.type = JValue::BOOL, v.flag = true;
                else if (literal("false")) v.type = JValue::BOOL, v.flag = false;
                else if (literal("null")) v.type = JValue::NUL;
                else if (*p_ == '-' || (*p_ >= '0' && *p_ <= '9')) number(v);
                else bad("expected value");
        }
        return v;
    }
};

// Whether a string anywhere in `v` (keys included) contains `needle`.
bool any_string_contains(const JValue& v, const char* needle) {
    switch (v.type) {
        case JValue::STR: return v.s.find(needle) != std::string::npos;
        case JValue::ARR:
            for (const JValue& x : v.items)
                if (any_string_contains(x, needle)) return true;
            return false;
        case JValue::OBJ:
            for (const auto& m : v.members)
                if (m.first.find(needle) != std::string::npos || any_string_contains(m.second, needle)) return true;
            return false;
        default: return false;
    }
}

// ---- byte stand-ins -------------------------------------------------------

// GPT-2's byte-to-character table (src/text/bpe.rs:356-369): bytes that
// print stand for themselves; the 68 others, in byte order, for U+0100,
// U+0101, ... All stand-ins lie below U+0144.
constexpr uint32_t STANDIN_LIMIT = 0x144;

bool prints(int b) { return (b >= 0x21 && b <= 0x7E) || (b >= 0xA1 && b <= 0xFF && b != 0xAD); }

struct StandIns {
    uint32_t of_byte[256];
    int16_t byte_of[STANDIN_LIMIT];  // -1: not a stand-in
    StandIns() {
        std::fill(std::begin(byte_of), std::end(byte_of), (int16_t)-1);
        uint32_t shifted = 0x100;
        for (int b = 0; b < 256; ++b) {
            of_byte[b] = prints(b) ? (uint32_t)b : shifted++;
            byte_of[of_byte[b]] = (int16_t)b;
        }
    }
};
const StandIns& standins() {
    static const StandIns t;
    return t;
}

// ---- the word split -------------------------------------------------------

enum class Split { Gpt2, Qwen };

// The words of `text` (Trit's pre-tokenize, src/text/bpe.rs:260-354):
// from each position the first alternative that matches takes its word.
class Splitter {
   public:
    Splitter(const std::string& text, Split split) : text_(text), split_(split) {
        decode_utf8(text, cp_, &off_, "tokenizer: the text");
        fl_.resize(cp_.size());
        for (size_t i = 0; i < cp_.size(); ++i) fl_[i] = flags_of(cp_[i]);
    }

    template <class F>
    void each_word(F&& take) const {
        for (size_t i = 0, n = cp_.size(); i < n;) {
            const size_t end = word_end(i);
            take(text_.data() + off(i), off(end) - off(i));
            i = end;
        }
    }

   private:
    const std::string& text_;
    Split split_;
    std::vector<uint32_t> cp_, off_;
    std::vector<uint8_t> fl_;

    size_t size() const { return cp_.size(); }
    size_t off(size_t i) const { return i < size() ? off_[i] : text_.size(); }
    uint8_t flag(size_t i) const { return i < size() ? fl_[i] : 0; }
    bool has(size_t i, uint8_t f) const { return i < size() && (fl_[i] & f); }
    // A character that is neither white space, a letter nor a number.
    bool other(size_t i) const { return i < size() && !(fl_[i] & (SPACE | LETTER | NUMBER)); }
    template <class P>
    size_t span(size_t j, P p) const {
        while (j < size() && p(j)) ++j;
        return j;
    }
    size_t letters(size_t j) const { return span(j, [&](size_t k) { return (fl_[k] & LETTER) != 0; }); }
    size_t numbers(size_t j) const { return span(j, [&](size_t k) { return (fl_[k] & NUMBER) != 0; }); }
    size_t others(size_t j) const { return span(j, [&](size_t k) { return other(k); }); }

    // 's 't 're 've 'm 'll 'd (Qwen: letters of any case): the word's end, or 0.
    size_t contraction(size_t i) const {
        if (cp_[i] != '\'') return 0;
        auto at = [&](size_t k) -> uint32_t {
            if (k >= size()) return 0;
            const uint32_t c = cp_[k];
            return split_ == Split::Qwen && c >= 'A' && c <= 'Z' ? c + 32 : c;
        };
        const uint32_t a = at(i + 1), b = at(i + 2);
        if ((a == 'r' && b == 'e') || (a == 'v' && b == 'e') || (a == 'l' && b == 'l')) return i + 3;
        if (a == 's' || a == 't' || a == 'm' || a == 'd') return i + 2;
        return 0;
    }

    //  ?\p{L}+ |  ?\p{N}+ |  ?[^\s\p{L}\p{N}]+
    size_t gpt2(size_t i) const {
        const size_t j = i + (cp_[i] == ' ' && i + 1 < size() && !has(i + 1, SPACE));
        if (has(j, LETTER)) return letters(j);
        if (has(j, NUMBER)) return numbers(j);
        if (other(j)) return others(j);
        return 0;
    }

    // [^\r\n\p{L}\p{N}]?\p{L}+ | \p{N} |  ?[^\s\p{L}\p{N}]+[\r\n]*
    size_t qwen(size_t i) const {
        const uint8_t f = fl_[i];
        const size_t j = i + !(f & (NEWLINE | LETTER | NUMBER));
        if (has(j, LETTER)) return letters(j);
        if (f & NUMBER) return i + 1;
        const size_t k = i + (cp_[i] == ' ');
        if (other(k)) return span(others(k), [&](size_t q) { return (fl_[q] & NEWLINE) != 0; });
        return 0;
    }

    // White space: Qwen's \s*[\r\n]+ first (through the last newline of the
    // run), then \s+(?!\S) (a run that a word follows leaves its last
    // character to that word), then \s+.
    size_t spaces(size_t i) const {
        const size_t end = span(i, [&](size_t k) { return (fl_[k] & SPACE) != 0; });
        if (split_ == Split::Qwen)
            for (size_t k = end; k > i; --k)
                if (fl_[k - 1] & NEWLINE) return k;
        if (end < size() && end - i > 1) return end - 1;
        return end;
    }

    size_t word_end(size_t i) const {
        if (size_t e = contraction(i)) return e;
        if (size_t e = split_ == Split::Gpt2 ? gpt2(i) : qwen(i)) return e;
        return spaces(i);
    }
};

// ---- merges ---------------------------------------------------------------

// Pairs of a word in a binary min-heap keyed (rank, position), addressable
// by position: each symbol position has at most one entry (the pair it
// starts), so an update or a removal finds its entry through `slot`.
class PairHeap {
   public:
    explicit PairHeap(size_t positions) : slot_(positions, NONE) { heap_.reserve(positions); }
    bool empty() const { return heap_.empty(); }
    int top() const { return heap_[0].pos; }

    // Sets the pair at `pos` to `rank` (inserting it), or removes it (rank < 0).
    void set(int pos, int rank) {
        int h = slot_[pos];
        if (rank < 0) {
            if (h == NONE) return;
            const int last = (int)heap_.size() - 1;
            swap_nodes(h, last);
            heap_.pop_back();
            slot_[pos] = NONE;
            if (h < last) fix(h);
            return;
        }
        if (h == NONE) {
            h = (int)heap_.size();
            heap_.push_back({rank, pos});
            slot_[pos] = h;
        } else {
            heap_[h].rank = rank;
        }
        fix(h);
    }

   private:
    static constexpr int NONE = -1;
    struct Node {
        int rank, pos;
        bool before(const Node& o) const { return rank < o.rank || (rank == o.rank && pos < o.pos); }
    };
    std::vector<Node> heap_;
    std::vector<int> slot_;

    void swap_nodes(int a, int b) {
        std::swap(heap_[a], heap_[b]);
        slot_[heap_[a].pos] = a;
        slot_[heap_[b].pos] = b;
    }
    void fix(int h) {
        while (h > 0 && heap_[h].before(heap_[(h - 1) / 2])) {
            swap_nodes(h, (h - 1) / 2);
            h = (h - 1) / 2;
        }
        for (;;) {
            const int l = 2 * h + 1, r = l + 1;
            int m = h;
            if (l < (int)heap_.size() && heap_[l].before(heap_[m])) m = l;
            if (r < (int)heap_.size() && heap_[r].before(heap_[m])) m = r;
            if (m == h) return;
            swap_nodes(h, m);
            h = m;
        }
    }
};

}  // namespace

// The tokenizer (Trit's Bpe, src/text/bpe.rs:11-22).
struct Bpe {
    // Token id -> its bytes (special tokens: their text), and whether special.
    std::vector<std::string> piece;
    std::vector<uint8_t> is_special;
    // Token as written in the file -> id (vocabulary stand-in strings and
    // added tokens' text; for a text given twice the later entry wins).
    std::unordered_map<std::string, int> id_of_text;
    // Interned symbols: their vocabulary id (or -1); the 256 byte stand-ins
    // are symbols 0..255 in byte order.
    std::vector<int> symbol_id;
    // (left symbol, right symbol) -> the first rank of that merge and the
    // joined symbol.
    struct Merge {
        int rank, joined;
    };
    std::unordered_map<uint64_t, Merge> merge_of;
    // Added tokens by their first byte: (text, id), longest first and, among
    // equal lengths, in file order.
    std::vector<std::pair<std::string, int>> special_by_byte[256];
    Split split = Split::Gpt2;

    static uint64_t key(int l, int r) { return (uint64_t)(uint32_t)l << 32 | (uint32_t)r; }
    const Merge* find_merge(int l, int r) const {
        const auto it = merge_of.find(key(l, r));
        return it == merge_of.end() ? nullptr : &it->second;
    }

    // One word's ids: its bytes as symbols, merged lowest rank first (the
    // leftmost of equal ranks) until no neighbouring pair has a rank
    // (text::merge_symbols, src/text/mod.rs:6-74); symbols the vocabulary
    // does not hold give no id (Bpe::merge_word, src/text/bpe.rs:239-258).
    void merge_word(const char* w, size_t n, std::vector<int>& out) const {
        if (n == 1) {
            const int id = symbol_id[(unsigned char)w[0]];
            if (id >= 0) out.push_back(id);
            return;
        }
        std::vector<int> sym(n), next(n), prev(n);
        for (size_t i = 0; i < n; ++i) {
            sym[i] = (unsigned char)w[i];
            next[i] = i + 1 < n ? (int)i + 1 : -1;
            prev[i] = (int)i - 1;
        }
        PairHeap heap(n);
        auto offer = [&](int left) {
            const int right = next[left];
            const Merge* m = right < 0 ? nullptr : find_merge(sym[left], sym[right]);
            heap.set(left, m ? m->rank : -1);
        };
        for (int i = 0; i + 1 < (int)n; ++i) offer(i);
        while (!heap.empty()) {
            const int left = heap.top(), right = next[left];
            sym[left] = find_merge(sym[left], sym[right])->joined;
            heap.set(right, -1);
            next[left] = next[right];
            if (next[left] >= 0) prev[next[left]] = left;
            offer(left);
            if (prev[left] >= 0) offer(prev[left]);
        }
        for (int i = 0; i >= 0; i = next[i])
            if (symbol_id[sym[i]] >= 0) out.push_back(symbol_id[sym[i]]);
    }

    void encode_words(const std::string& text, std::vector<int>& out) const {
        Splitter(text, split).each_word([&](const char* w, size_t n) { merge_word(w, n, out); });
    }

    // Bpe::encode / encode_plain (src/text/bpe.rs:197-237): added tokens
    // written in the text become their ids (the earliest in the text, the
    // longest where several start at one place); the rest is split and merged.
    std::vector<int> encode(const std::string& text, bool plain) const {
        std::vector<int> out;
        size_t from = 0;
        if (!plain) {
            for (size_t at = 0; at < text.size(); ++at) {
                for (const auto& sp : special_by_byte[(unsigned char)text[at]]) {
                    if (text.compare(at, sp.first.size(), sp.first) != 0) continue;
                    encode_words(text.substr(from, at - from), out);
                    out.push_back(sp.second);
                    from = at + sp.first.size();
                    at = from - 1;
                    break;
                }
            }
        }
        encode_words(text.substr(from), out);
        return out;
    }

    // Bpe::decode (src/text/bpe.rs:185-195): the pieces of non-special ids
    // in range, as text.
    std::string decode(const int32_t* ids, int n) const {
        std::string bytes;
        for (int i = 0; i < n; ++i)
            if (ids[i] >= 0 && (size_t)ids[i] < piece.size() && !is_special[ids[i]]) bytes += piece[ids[i]];
        return bytes_to_text(bytes);
    }
};

namespace {

// Ids past twice the entries plus this are refused (a table that large is
// not a real vocabulary; src/text/bpe.rs:8).
constexpr uint64_t FREE_IDS = 1 << 16;

// The tokenizer of a tokenizer.json (Bpe::parse / build,
// src/text/bpe.rs:82-174).
std::unique_ptr<Bpe> load(const JValue& root) {
    const JValue* model = root.member("model");
    const JValue* vocab = model ? model->member("vocab") : nullptr;
    if (!vocab || vocab->type != JValue::OBJ) fail("tokenizer.json has no model.vocab");
    const StandIns& S = standins();
    auto B = std::make_unique<Bpe>();

    // The vocabulary as a serde_json map holds it: one entry per text (the
    // last of duplicates), in text order.
    std::vector<const std::pair<std::string, JValue>*> order;
    order.reserve(vocab->members.size());
    for (const auto& m : vocab->members) order.push_back(&m);
    std::stable_sort(order.begin(), order.end(), [](auto* a, auto* b) { return a->first < b->first; });
    struct Entry {
        uint64_t id;
        std::string bytes, text;
        bool special;
    };
    std::vector<Entry> entries;
    entries.reserve(order.size());
    for (size_t i = 0; i < order.size(); ++i) {
        if (i + 1 < order.size() && order[i + 1]->first == order[i]->first) continue;  // a later duplicate wins
        const auto& [text, id] = *order[i];
        if (!id.is_u64()) fail("the vocabulary has a bad id");
        std::vector<uint32_t> cps;
        decode_utf8(text, cps, nullptr, "the vocabulary");
        std::string bytes(cps.size(), '?');
        for (size_t c = 0; c < cps.size(); ++c)
            if (cps[c] < STANDIN_LIMIT && S.byte_of[cps[c]] >= 0) bytes[c] = (char)S.byte_of[cps[c]];
        entries.push_back({id.u, std::move(bytes), text, false});
    }
    // Added tokens: those with a non-negative integer id and a text
    // ("special" unless it says false).
    std::vector<std::pair<std::string, int>> added_texts;
    if (const JValue* added = root.member("added_tokens"); added && added->type == JValue::ARR)
        for (const JValue& a : added->items) {
            const JValue* id = a.member("id");
            const JValue* content = a.member("content");
            if (!id || !id->is_u64() || !content || content->type != JValue::STR) continue;
            const JValue* sp = a.member("special");
            entries.push_back({id->u, content->s, content->s, !(sp && sp->type == JValue::BOOL && !sp->flag)});
            added_texts.emplace_back(content->s, (int)id->u);
        }
    uint64_t top = 0;
    for (const Entry& e : entries) top = std::max(top, e.id);
    if (!entries.empty() && top >= 2 * (uint64_t)entries.size() + FREE_IDS)
        fail("the tokenizer's id " + std::to_string(top) + " is far past its " + std::to_string(entries.size()) +
             " tokens");
    const size_t table = entries.empty() ? 0 : (size_t)top + 1;
    B->piece.assign(table, std::string());
    B->is_special.assign(table, 0);
    B->id_of_text.reserve(entries.size());
    for (const Entry& e : entries) {  // later entries win a shared id or text
        B->piece[e.id] = e.bytes;
        B->is_special[e.id] = e.special;
        B->id_of_text[e.text] = (int)e.id;
    }
    // Added tokens for encode, by first byte, longest first (file order
    // among equal lengths). An empty text never matches.
    std::stable_sort(added_texts.begin(), added_texts.end(),
                     [](const auto& a, const auto& b) { return a.first.size() > b.first.size(); });
    for (auto& sp : added_texts)
        if (!sp.first.empty()) B->special_by_byte[(unsigned char)sp.first[0]].push_back(std::move(sp));

    // Symbols: the byte stand-ins first, then every side of every merge and
    // each merge's join.
    std::unordered_map<std::string, int> symbol;
    auto intern = [&](std::string text) {
        const auto it = symbol.find(text);
        if (it != symbol.end()) return it->second;
        const int s = (int)B->symbol_id.size();
        const auto id = B->id_of_text.find(text);
        B->symbol_id.push_back(id == B->id_of_text.end() ? -1 : id->second);
        symbol.emplace(std::move(text), s);
        return s;
    };
    for (int b = 0; b < 256; ++b) {
        std::string t;
        append_utf8(t, S.of_byte[b]);
        intern(std::move(t));
    }
    // A merge is ["left", "right"] (two strings first; more items are
    // ignored) or "left right" (cut at the first space), src/text/mod.rs:98-107.
    int rank = 0;
    if (const JValue* merges = model->member("merges"); merges && merges->type == JValue::ARR) {
        B->merge_of.reserve(merges->items.size());
        for (const JValue& m : merges->items) {
            std::string left, right;
            if (m.type == JValue::ARR && m.items.size() >= 2 && m.items[0].type == JValue::STR &&
                m.items[1].type == JValue::STR) {
                left = m.items[0].s, right = m.items[1].s;
            } else if (m.type == JValue::STR && m.s.find(' ') != std::string::npos) {
                const size_t cut = m.s.find(' ');
                left = m.s.substr(0, cut), right = m.s.substr(cut + 1);
            } else {
                continue;
            }
            const int l = intern(left), r = intern(right), j = intern(left + right);
            B->merge_of.emplace(Bpe::key(l, r), Bpe::Merge{rank++, j});  // the first rank of a pair stays
        }
    }
    // Qwen2's split when the pre-tokenizer holds its letter alternative.
    const JValue* pre = root.member("pre_tokenizer");
    B->split = pre && any_string_contains(*pre, "[^\\r\\n\\p{L}\\p{N}]?\\p{L}+") ? Split::Qwen : Split::Gpt2;
    return B;
}

std::unique_ptr<Bpe> parse(const char* text, size_t len) {
    if (!is_utf8(text, len)) fail("tokenizer.json is not JSON: the text is not UTF-8");
    return load(JsonReader(text, len).document());
}

// ---- the cleanup prompt (src/cleanup.rs) ----------------------------------

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
    std::vector<uint32_t> cps, offs;
    decode_utf8(t, cps, &offs, "cleanup: the transcript");
    size_t a = 0, b = cps.size();
    while (a < b && is_space_cp(cps[a])) ++a;
    while (b > a && is_space_cp(cps[b - 1])) --b;
    const size_t from = a < cps.size() ? offs[a] : t.size(), to = b < cps.size() ? offs[b] : t.size();
    return t.substr(from, to - from);
}

// Cleaner::parts (src/cleanup.rs:240-278): whole sentences (cut after '.',
// '?' or '!' that the end or whitespace follows), joined with one space
// while the join holds at most `limit` tokens; a sentence longer alone goes
// word by word (split on whitespace).
std::vector<std::string> cleanup_parts(const Bpe& B, const std::string& text, int limit) {
    std::vector<uint32_t> cps, offs;
    decode_utf8(text, cps, &offs, "cleanup: the transcript");
    auto off = [&](size_t i) { return i < cps.size() ? offs[i] : text.size(); };
    std::vector<std::string> sentences;
    size_t start = 0;
    for (size_t i = 0; i < cps.size(); ++i) {
        const uint32_t c = cps[i];
        if ((c == '.' || c == '?' || c == '!') && (i + 1 == cps.size() || is_space_cp(cps[i + 1]))) {
            sentences.push_back(trim(text.substr(off(start), off(i + 1) - off(start))));
            start = i + 1;
        }
    }
    sentences.push_back(trim(text.substr(off(start))));
    auto tokens = [&](const std::string& t) { return (int)B.encode(t, false).size(); };
    auto words_of = [&](const std::string& s) {
        std::vector<std::string> words;
        std::vector<uint32_t> c2, o2;
        decode_utf8(s, c2, &o2, "cleanup: the transcript");
        for (size_t i = 0; i < c2.size();) {
            if (is_space_cp(c2[i])) {
                ++i;
                continue;
            }
            size_t j = i;
            while (j < c2.size() && !is_space_cp(c2[j])) ++j;
            const size_t to = j < c2.size() ? o2[j] : s.size();
            words.push_back(s.substr(o2[i], to - o2[i]));
            i = j;
        }
        return words;
    };
    std::vector<std::string> parts;
    std::string current;
    for (const std::string& sentence : sentences) {
        if (sentence.empty()) continue;
        const std::vector<std::string> pieces =
            tokens(sentence) > limit ? words_of(sentence) : std::vector<std::string>{sentence};
        for (const std::string& piece : pieces) {
            std::string joined = current.empty() ? piece : current + " " + piece;
            if (!current.empty() && tokens(joined) > limit) {
                parts.push_back(std::move(current));
                current = piece;
            } else {
                current = std::move(joined);
            }
        }
    }
    if (!current.empty()) parts.push_back(std::move(current));
    return parts;
}

int copy_ids(const std::vector<int>& ids, int32_t* out, int cap) {
    if (cap < 0) fail("tokenizer: negative capacity");
    if (cap && !out) fail("tokenizer: out is NULL");
    std::copy_n(ids.begin(), std::min<size_t>(ids.size(), (size_t)cap), out);
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
        *out = new TritHipBpe{parse(json, len)};
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
        for (size_t got; (got = std::fread(buf, 1, sizeof buf, f)) > 0;) text.append(buf, got);
        std::fclose(f);
        if (!is_utf8(text.data(), text.size()))
            fail(std::string("cannot read ") + path + ": stream did not contain valid UTF-8");
        *out = new TritHipBpe{parse(text.data(), text.size())};
        return 0;
    });
}

void trit_hip_bpe_free(TritHipBpe* bpe) { delete bpe; }

int trit_hip_bpe_id(const TritHipBpe* bpe, const char* token) {
    return guard(-1, [&] {
        if (!bpe || !token) fail("tokenizer: bpe or token is NULL");
        const auto it = bpe->bpe->id_of_text.find(token);
        return it == bpe->bpe->id_of_text.end() ? -1 : it->second;
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
        // Cleaner::clean_part (src/cleanup.rs:280-301): the system turn and
        // the control line, the transcript as plain text (a spoken
        // "<|im_end|>" stays characters), the assistant turn with thinking off.
        const std::string control = std::string("[Styling: ") + STYLING[styling] + "] [Structure: " +
                                    STRUCTURE[structure] + "] [Context: " + CONTEXT[context] + "]";
        std::vector<int> ids = B.encode(system_prefix() + control + "\n", false);
        for (int id : B.encode(std::string(transcript ? transcript : "", len), true)) ids.push_back(id);
        for (int id : B.encode("<|im_end|>\n<|im_start|>assistant\n<think>\n\n</think>\n\n", false)) ids.push_back(id);
        return copy_ids(ids, out, cap);
    });
}

int64_t trit_hip_cleanup_parts(const TritHipBpe* bpe, const char* transcript, size_t len, int limit, char* out,
                               size_t cap) {
    return guard((int64_t)-1, [&] {
        if (!bpe || (!transcript && len)) fail("tokenizer: bpe or transcript is NULL");
        if (limit <= 0) fail("cleanup: the part limit must be positive");
        std::string all;
        for (const std::string& p : cleanup_parts(*bpe->bpe, trim(std::string(transcript ? transcript : "", len)), limit)) {
            all += p;
            all += '\0';
        }
        if (cap && !out) fail("tokenizer: out is NULL");
        if (cap) std::memcpy(out, all.data(), std::min(cap, all.size()));
        return (int64_t)all.size();
    });
}

}  // extern "C"
