// The Qwen3 tokenizer (tokenizer.hpp): Unicode classes and NFC, the Split pre-tokenizer, the byte map, BPE, added
// tokens and the tokenizer.json loader.
#include "tokenizer.hpp"

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <functional>
#include <mutex>
#include <queue>
#include <set>

#include "json.hpp"

namespace lrm {
namespace tok {

namespace {

struct ClassRun {
    uint32_t start;
    uint8_t cls;
};
struct ScalarRange {
    uint32_t first, last;
};
struct CccEntry {
    uint32_t cp;
    uint8_t ccc;
};
struct DecompEntry {
    uint32_t cp, off;
    uint8_t len;
};
struct CompEntry {
    uint32_t a, b, c;
};

#include "unicode_tables.inc"

template <class T, size_t N>
constexpr size_t count_of(const T (&)[N]) {
    return N;
}

[[noreturn]] void data_fail(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void data_fail(const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    throw DataError(std::string("tokenizer.json: ") + buf);
}

// The BMP part of the class table, unpacked once.
const uint8_t* bmp_classes() {
    static uint8_t table[0x10000];
    static std::once_flag once;
    std::call_once(once, [] {
        size_t r = 0;
        for (uint32_t c = 0; c < 0x10000; ++c) {
            while (r + 1 < count_of(kClassRuns) && kClassRuns[r + 1].start <= c) ++r;
            table[c] = (c >= 0xD800 && c <= 0xDFFF) ? kOther : kClassRuns[r].cls;
        }
    });
    return table;
}

constexpr uint32_t kSBase = 0xAC00, kLBase = 0x1100, kVBase = 0x1161, kTBase = 0x11A7;
constexpr uint32_t kLCount = 19, kVCount = 21, kTCount = 28, kNCount = kVCount * kTCount, kSCount = kLCount * kNCount;

uint8_t ccc_of(uint32_t cp) {
    const CccEntry* e = std::lower_bound(kCcc, kCcc + count_of(kCcc), cp,
                                         [](const CccEntry& x, uint32_t v) { return x.cp < v; });
    return (e != kCcc + count_of(kCcc) && e->cp == cp) ? e->ccc : 0;
}

void decompose_into(uint32_t cp, std::u32string& out) {
    if (cp >= kSBase && cp < kSBase + kSCount) {  // Hangul syllables, algorithmically
        const uint32_t s = cp - kSBase;
        out += char32_t(kLBase + s / kNCount);
        out += char32_t(kVBase + (s % kNCount) / kTCount);
        if (s % kTCount) out += char32_t(kTBase + s % kTCount);
        return;
    }
    const DecompEntry* e = std::lower_bound(kDecompIndex, kDecompIndex + count_of(kDecompIndex), cp,
                                            [](const DecompEntry& x, uint32_t v) { return x.cp < v; });
    if (e != kDecompIndex + count_of(kDecompIndex) && e->cp == cp) {
        for (uint32_t k = 0; k < e->len; ++k) out += char32_t(kDecompData[e->off + k]);
    } else {
        out += char32_t(cp);
    }
}

// The primary composite of (a, b), or 0.
uint32_t compose_pair(uint32_t a, uint32_t b) {
    if (a >= kLBase && a < kLBase + kLCount && b >= kVBase && b < kVBase + kVCount)
        return kSBase + ((a - kLBase) * kVCount + (b - kVBase)) * kTCount;
    if (a >= kSBase && a < kSBase + kSCount && (a - kSBase) % kTCount == 0 && b > kTBase && b < kTBase + kTCount)
        return a + (b - kTBase);
    const CompEntry* e = std::lower_bound(kComposites, kComposites + count_of(kComposites), std::make_pair(a, b),
                                          [](const CompEntry& x, std::pair<uint32_t, uint32_t> v) {
                                              return x.a != v.first ? x.a < v.first : x.b < v.second;
                                          });
    return (e != kComposites + count_of(kComposites) && e->a == a && e->b == b) ? e->c : 0;
}

// NFC of a string that holds no split point: full canonical decomposition, canonical ordering, canonical composition.
void nfc_part(const char32_t* s, size_t n, std::u32string& out) {
    std::u32string d;
    d.reserve(n + 8);
    for (size_t i = 0; i < n; ++i) decompose_into(uint32_t(s[i]), d);
    // canonical ordering: a stable sort by combining class inside each run of non-starters
    std::vector<uint8_t> cc(d.size());
    for (size_t i = 0; i < d.size(); ++i) cc[i] = ccc_of(uint32_t(d[i]));
    for (size_t i = 1; i < d.size(); ++i) {
        if (cc[i] == 0) continue;
        size_t j = i;
        while (j > 0 && cc[j - 1] > cc[j]) {
            std::swap(d[j - 1], d[j]);
            std::swap(cc[j - 1], cc[j]);
            --j;
        }
    }
    // canonical composition: a character composes with the last starter when nothing between them blocks it (no
    // starter, no mark of the same or a higher class); `last` is the class of the last character kept
    if (d.empty()) return;
    size_t sp = out.size();  // the last starter's index in out
    int last = cc[0] ? 256 : 0;  // a leading mark: nothing composes with it
    out += d[0];
    for (size_t i = 1; i < d.size(); ++i) {
        const uint32_t ch = uint32_t(d[i]);
        const int c = cc[i];
        const uint32_t comp = compose_pair(uint32_t(out[sp]), ch);
        if (comp && (last < c || last == 0)) {
            out[sp] = char32_t(comp);
            continue;
        }
        if (c == 0) sp = out.size();
        last = c;
        out += char32_t(ch);
    }
}

bool is_crlf(uint32_t c) { return c == 0x0D || c == 0x0A; }

}  // namespace

// ---------------------------------------------------------------- classes

CharClass char_class(uint32_t cp) {
    if (cp < 0x10000) return CharClass(bmp_classes()[cp]);
    if (cp > 0x10FFFF) return kOther;
    const ClassRun* e = std::upper_bound(kClassRuns, kClassRuns + count_of(kClassRuns), cp,
                                         [](uint32_t v, const ClassRun& r) { return v < r.start; });
    return CharClass((e - 1)->cls);
}

char contraction_letter(uint32_t cp) {
    switch (cp) {
        case 0x53: case 0x73: case 0x17F: return 's';
        case 0x54: case 0x74: return 't';
        case 0x52: case 0x72: return 'r';
        case 0x45: case 0x65: return 'e';
        case 0x56: case 0x76: return 'v';
        case 0x4D: case 0x6D: return 'm';
        case 0x4C: case 0x6C: return 'l';
        case 0x44: case 0x64: return 'd';
        default: return 0;
    }
}

// ---------------------------------------------------------------- UTF-8

namespace {
// The length of the well-formed sequence led by byte c and the range of its second byte; 0 when c leads none.
int lead(uint8_t c, uint8_t& lo, uint8_t& hi) {
    lo = 0x80, hi = 0xBF;
    if (c >= 0xC2 && c <= 0xDF) return 2;
    if (c >= 0xE0 && c <= 0xEF) {
        if (c == 0xE0) lo = 0xA0;
        if (c == 0xED) hi = 0x9F;
        return 3;
    }
    if (c >= 0xF0 && c <= 0xF4) {
        if (c == 0xF0) lo = 0x90;
        if (c == 0xF4) hi = 0x8F;
        return 4;
    }
    return 0;
}

// The scalar at s[i] and its length, or the length of the maximal ill-formed subpart there (as a negative number).
int next_scalar(const uint8_t* s, size_t n, size_t i, uint32_t& cp) {
    const uint8_t c = s[i];
    if (c < 0x80) {
        cp = c;
        return 1;
    }
    uint8_t lo, hi;
    const int len = lead(c, lo, hi);
    if (!len) return -1;
    int k = 1;
    uint32_t v = c & (len == 2 ? 0x1F : len == 3 ? 0x0F : 0x07);
    while (k < len && i + size_t(k) < n) {
        const uint8_t b = s[i + size_t(k)];
        if (k == 1 ? (b < lo || b > hi) : (b < 0x80 || b > 0xBF)) break;
        v = (v << 6) | (b & 0x3F);
        ++k;
    }
    if (k < len) return -k;
    cp = v;
    return len;
}
}  // namespace

bool utf8_decode(const uint8_t* s, size_t n, std::u32string& out, size_t* bad) {
    out.clear();
    out.reserve(n);
    for (size_t i = 0; i < n;) {
        uint32_t cp;
        const int k = next_scalar(s, n, i, cp);
        if (k < 0) {
            if (bad) *bad = i;
            return false;
        }
        out += char32_t(cp);
        i += size_t(k);
    }
    return true;
}

std::u32string utf8_decode_replace(const uint8_t* s, size_t n) {
    std::u32string out;
    out.reserve(n);
    for (size_t i = 0; i < n;) {
        uint32_t cp;
        const int k = next_scalar(s, n, i, cp);
        if (k < 0) {
            out += char32_t(0xFFFD);
            i += size_t(-k);
        } else {
            out += char32_t(cp);
            i += size_t(k);
        }
    }
    return out;
}

std::string utf8_encode(const std::u32string& s) {
    std::string out;
    out.reserve(s.size());
    for (char32_t c : s) json::append_utf8(out, uint32_t(c));
    return out;
}

// ---------------------------------------------------------------- NFC

bool nfc_split_point(uint32_t cp) {
    const ScalarRange* e = std::upper_bound(kSplitRanges, kSplitRanges + count_of(kSplitRanges), cp,
                                            [](uint32_t v, const ScalarRange& r) { return v < r.first; });
    return e != kSplitRanges && cp <= (e - 1)->last;
}

std::u32string nfc(const std::u32string& s) {
    std::u32string out;
    out.reserve(s.size() + 8);
    size_t start = 0;
    for (size_t i = 0; i < s.size(); ++i) {
        if (!nfc_split_point(uint32_t(s[i]))) continue;
        if (i > start) nfc_part(s.data() + start, i - start, out);
        out += s[i];
        start = i + 1;
    }
    if (start < s.size()) nfc_part(s.data() + start, s.size() - start, out);
    return out;
}

// ---------------------------------------------------------------- the Split pre-tokenizer
// The regex (?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}| ?[^\s\p{L}\p{N}]+[\r\n]*|\s*[\r\n]+|\s+(?!\S)|\s+
// tried alternative by alternative at each position, as Oniguruma does (PreTokenizer.fs:1-24): the end of the match
// at p is
//   1. p + 2 or p + 3 for U+0027 followed by s, t, m, d, or re, ve, ll (simple case folding);
//   2. the end of the letter run when p is a letter, or when p is not \r, \n or a number and p + 1 is a letter;
//   3. p + 1 for a number;
//   4. for other, or a space followed by other: the end of the run of others, then of \r and \n;
//   5. for a white-space run [p, q) holding \r or \n: just after its last \r or \n;
//   6. otherwise q when the run ends the text, q - 1 when the run has two scalars or more;
//   7. otherwise q.

std::vector<size_t> pre_split(const std::u32string& s) {
    const size_t n = s.size();
    std::vector<uint8_t> cls(n);
    for (size_t i = 0; i < n; ++i) cls[i] = char_class(uint32_t(s[i]));
    auto run_end = [&](uint8_t k, size_t from) {
        size_t i = from;
        while (i < n && cls[i] == k) ++i;
        return i;
    };
    std::vector<size_t> b{0};
    size_t p = 0;
    while (p < n) {
        const uint32_t c = uint32_t(s[p]);
        const uint8_t k = cls[p];
        size_t e = 0;
        bool done = false;
        if (c == 0x27 && p + 1 < n) {
            const char l1 = contraction_letter(uint32_t(s[p + 1]));
            const char l2 = p + 2 < n ? contraction_letter(uint32_t(s[p + 2])) : 0;
            if (l1 == 's' || l1 == 't' || l1 == 'm' || l1 == 'd') e = p + 2, done = true;
            else if ((l1 == 'r' || l1 == 'v') && l2 == 'e') e = p + 3, done = true;
            else if (l1 == 'l' && l2 == 'l') e = p + 3, done = true;
        }
        if (done) {
        } else if (k == kLetter) {
            e = run_end(kLetter, p + 1);
        } else if (k != kNumber && !is_crlf(c) && p + 1 < n && cls[p + 1] == kLetter) {
            e = run_end(kLetter, p + 2);
        } else if (k == kNumber) {
            e = p + 1;
        } else if (k == kOther || (c == 0x20 && p + 1 < n && cls[p + 1] == kOther)) {
            e = run_end(kOther, k == kOther ? p + 1 : p + 2);
            while (e < n && is_crlf(uint32_t(s[e]))) ++e;
        } else {
            size_t q = p;
            long last_crlf = -1;
            while (q < n && cls[q] == kSpace) {
                if (is_crlf(uint32_t(s[q]))) last_crlf = long(q);
                ++q;
            }
            if (last_crlf >= 0) e = size_t(last_crlf) + 1;
            else if (q == n) e = n;
            else if (q - p >= 2) e = q - 1;
            else e = q;
        }
        b.push_back(e);
        p = e;
    }
    return b;
}

// ---------------------------------------------------------------- the byte map

namespace {
struct ByteMap {
    uint32_t to_char[256];
    int16_t to_byte[0x144];
    ByteMap() {
        uint32_t next = 0x100;
        for (int i = 0; i < 0x144; ++i) to_byte[i] = -1;
        for (int b = 0; b < 256; ++b) {
            const bool printable = (b >= 0x21 && b <= 0x7E) || (b >= 0xA1 && b <= 0xAC) || (b >= 0xAE && b <= 0xFF);
            to_char[b] = printable ? uint32_t(b) : next++;
            to_byte[to_char[b]] = int16_t(b);
        }
    }
};
const ByteMap& byte_map() {
    static const ByteMap m;
    return m;
}

// The bytes of a byte-level string, or false when a scalar is outside the map.
bool byte_level_decode(const std::u32string& token, std::string& out) {
    out.clear();
    for (char32_t c : token) {
        const int b = char_byte(uint32_t(c));
        if (b < 0) return false;
        out += char(b);
    }
    return true;
}
}  // namespace

uint32_t byte_char(uint8_t b) { return byte_map().to_char[b]; }
int char_byte(uint32_t c) { return c < 0x144 ? byte_map().to_byte[c] : -1; }

// ---------------------------------------------------------------- the loader (TokenizerJson.fs)

namespace {
using json::Kind;
using json::Value;

const Value* member(const Value& o, const char* name) {
    if (o.kind != Kind::Object) return nullptr;
    const Value* found = nullptr;
    for (const auto& [k, v] : o.members)
        if (k == name) found = &v;  // the last of repeated names, as a JSON object model keeps
    return found;
}
const Value& prop(const Value& o, const std::string& path, const char* name) {
    const Value* v = member(o, name);
    if (!v) data_fail("%s has no '%s'", path.c_str(), name);
    return *v;
}
const std::string& str(const Value& o, const std::string& path, const char* name) {
    const Value& v = prop(o, path, name);
    if (v.kind != Kind::String) data_fail("%s.%s is not a string", path.c_str(), name);
    return v.text;
}
void expect_str(const Value& o, const std::string& path, const char* name, const char* want) {
    const std::string& v = str(o, path, name);
    if (v != want) data_fail("%s.%s is '%s', only '%s' is supported", path.c_str(), name, v.c_str(), want);
}
void expect_bool(const Value& o, const std::string& path, const char* name, bool want) {
    const Value& v = prop(o, path, name);
    if (v.kind != Kind::Bool || v.boolean != want)
        data_fail("%s.%s must be %s", path.c_str(), name, want ? "true" : "false");
}
bool null_or_absent(const Value& o, const char* name) {
    const Value* v = member(o, name);
    return !v || v->kind == Kind::Null;
}
void expect_null(const Value& o, const std::string& path, const char* name) {
    if (!null_or_absent(o, name)) data_fail("%s.%s must be null", path.c_str(), name);
}
void expect_empty_affix(const Value& o, const std::string& path, const char* name) {
    const Value* v = member(o, name);
    if (v && v->kind != Kind::Null && !(v->kind == Kind::String && v->text.empty()))
        data_fail("%s.%s must be empty", path.c_str(), name);
}
void expect_false_or_absent(const Value& o, const std::string& path, const char* name) {
    const Value* v = member(o, name);
    if (v && v->kind != Kind::Null && !(v->kind == Kind::Bool && !v->boolean))
        data_fail("%s.%s must be false", path.c_str(), name);
}
void check_byte_level(const Value& o, const std::string& path, bool pre_tokenizer) {
    expect_str(o, path, "type", "ByteLevel");
    expect_bool(o, path, "add_prefix_space", false);
    if (pre_tokenizer) expect_bool(o, path, "use_regex", false);
}
int32_t int_of(const Value& v, const std::string& what) {
    int64_t x;
    if (v.kind == Kind::Number && json::nonnegative_int(v, &x) && x <= INT32_MAX) return int32_t(x);
    if (v.kind == Kind::Number && !v.text.empty() && v.text[0] == '-') {
        // a negative integer: the id check below reports it
        bool digits = v.text.size() > 1 && v.text.find_first_not_of("0123456789", 1) == std::string::npos;
        if (digits && v.text.size() < 11) return int32_t(std::stol(v.text));
    }
    data_fail("%s is not an int32", what.c_str());
}
std::u32string u32(const std::string& utf8) {
    std::u32string out;
    size_t bad;
    if (!utf8_decode(reinterpret_cast<const uint8_t*>(utf8.data()), utf8.size(), out, &bad))
        data_fail("a string is not valid UTF-8");
    return out;
}
}  // namespace

// The Qwen Split regex, character for character as tokenizer.json holds it (PreTokenizer.SplitPattern).
static const char* const kSplitPattern =
    "(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\\r\\n\\p{L}\\p{N}]?\\p{L}+|\\p{N}| ?[^\\s\\p{L}\\p{N}]+[\\r\\n]*|\\s*[\\r\\n]+|"
    "\\s+(?!\\S)|\\s+";

std::unique_ptr<Tokenizer> Tokenizer::parse(const uint8_t* bytes, size_t n) {
    if (!json::utf8_valid(bytes, n)) throw DataError("tokenizer.json is not valid UTF-8");
    Value root;
    try {
        root = json::parse(bytes, n, 64);
    } catch (const json::Error& e) {
        throw DataError(std::string("tokenizer.json is not valid JSON: ") + e.what());
    }
    if (root.kind != Kind::Object) data_fail("the document is not an object");
    // the pipeline
    expect_null(root, "$", "truncation");
    expect_null(root, "$", "padding");
    expect_str(prop(root, "$", "normalizer"), "normalizer", "type", "NFC");
    const Value& pre = prop(root, "$", "pre_tokenizer");
    expect_str(pre, "pre_tokenizer", "type", "Sequence");
    const Value& steps = prop(pre, "pre_tokenizer", "pretokenizers");
    if (steps.kind != Kind::Array || steps.items.size() != 2) data_fail("pre_tokenizer.pretokenizers must be [Split, ByteLevel]");
    const Value& split = steps.items[0];
    expect_str(split, "pre_tokenizer.pretokenizers[0]", "type", "Split");
    expect_str(prop(split, "Split", "pattern"), "Split.pattern", "Regex", kSplitPattern);
    expect_str(split, "Split", "behavior", "Isolated");
    expect_bool(split, "Split", "invert", false);
    check_byte_level(steps.items[1], "pre_tokenizer.pretokenizers[1]", true);
    if (!null_or_absent(root, "post_processor")) expect_str(prop(root, "$", "post_processor"), "post_processor", "type", "ByteLevel");
    check_byte_level(prop(root, "$", "decoder"), "decoder", false);
    // the model
    const Value& model = prop(root, "$", "model");
    expect_str(model, "model", "type", "BPE");
    expect_null(model, "model", "dropout");
    expect_null(model, "model", "unk_token");
    expect_empty_affix(model, "model", "continuing_subword_prefix");
    expect_empty_affix(model, "model", "end_of_word_suffix");
    expect_false_or_absent(model, "model", "fuse_unk");
    expect_false_or_absent(model, "model", "byte_fallback");
    expect_false_or_absent(model, "model", "ignore_merges");

    std::unique_ptr<Tokenizer> t(new Tokenizer());
    const Value& vocab = prop(model, "model", "vocab");
    if (vocab.kind != Kind::Object) data_fail("model.vocab is not an object");
    const size_t nv = vocab.members.size();
    t->token_bytes_.assign(nv, std::string());
    t->token_strings_.assign(nv, std::string());
    std::vector<bool> seen(nv, false);
    for (const auto& [token, v] : vocab.members) {
        if (v.kind != Kind::Number) data_fail("model.vocab[%s] is not a number", token.c_str());
        const int32_t id = int_of(v, "model.vocab[" + token + "]");
        if (!t->vocab_.emplace(token, id).second) data_fail("model.vocab has '%s' twice", token.c_str());
        if (id < 0 || size_t(id) >= nv || seen[size_t(id)])
            data_fail("model.vocab ids are not 0..%zu, each once (%s -> %d)", nv - 1, token.c_str(), id);
        seen[size_t(id)] = true;
        std::string b;
        if (!byte_level_decode(u32(token), b) || b.empty())
            data_fail("model.vocab token '%s' is not a byte-level string", token.c_str());
        t->token_bytes_[size_t(id)] = b;
        t->token_strings_[size_t(id)] = token;
    }
    for (int b = 0; b < 256; ++b) {
        std::string ch;
        json::append_utf8(ch, byte_char(uint8_t(b)));
        auto it = t->vocab_.find(ch);
        if (it == t->vocab_.end()) data_fail("model.vocab has no token for byte 0x%02X", b);
        t->byte_ids_[b] = it->second;
    }
    const Value& merges = prop(model, "model", "merges");
    if (merges.kind != Kind::Array) data_fail("model.merges is not an array");
    t->merges_.reserve(merges.items.size() * 2);
    uint64_t rank = 0;
    for (const Value& m : merges.items) {
        std::string left, right;
        if (m.kind == Kind::Array && m.items.size() == 2 && m.items[0].kind == Kind::String &&
            m.items[1].kind == Kind::String) {
            left = m.items[0].text;
            right = m.items[1].text;
        } else if (m.kind == Kind::String) {
            const size_t sp = m.text.find(' ');
            if (sp == std::string::npos || m.text.find(' ', sp + 1) != std::string::npos)
                data_fail("model.merges[%llu] is not 'a b'", (unsigned long long)rank);
            left = m.text.substr(0, sp);
            right = m.text.substr(sp + 1);
        } else {
            data_fail("model.merges[%llu] is not a pair", (unsigned long long)rank);
        }
        auto id_of = [&](const std::string& s) {
            auto it = t->vocab_.find(s);
            if (it == t->vocab_.end())
                data_fail("model.merges[%llu] names '%s', which is not in the vocabulary", (unsigned long long)rank,
                          s.c_str());
            return uint64_t(uint32_t(it->second));
        };
        const uint64_t l = id_of(left), r = id_of(right), merged = id_of(left + right);
        if (!t->merges_.emplace((l << 32) | r, (rank << 32) | merged).second)
            data_fail("model.merges[%llu] repeats the pair '%s' '%s'", (unsigned long long)rank, left.c_str(),
                      right.c_str());
        ++rank;
    }
    // added tokens
    if (!null_or_absent(root, "added_tokens")) {
        const Value& a = prop(root, "$", "added_tokens");
        if (a.kind != Kind::Array) data_fail("added_tokens is not an array");
        for (const Value& e : a.items) {
            const int32_t id = int_of(prop(e, "added_tokens[]", "id"), "added_tokens[].id");
            const std::string path = "added_tokens[id " + std::to_string(id) + "]";
            const std::string& content = str(e, path, "content");
            expect_bool(e, path, "normalized", false);
            expect_bool(e, path, "lstrip", false);
            expect_bool(e, path, "rstrip", false);
            expect_bool(e, path, "single_word", false);
            const Value& sp = prop(e, path, "special");
            if (sp.kind != Kind::Bool) data_fail("%s.special is not a boolean", path.c_str());
            t->added_.push_back({id, u32(content), sp.boolean});
        }
        std::stable_sort(t->added_.begin(), t->added_.end(),
                         [](const AddedToken& x, const AddedToken& y) { return x.id < y.id; });
        for (size_t i = 0; i < t->added_.size(); ++i)
            if (t->added_[i].id != int32_t(nv + i))
                data_fail("added token ids must follow the vocabulary (%zu expected, %d found)", nv + i, t->added_[i].id);
    }
    // the trie of the added tokens' contents
    t->trie_.emplace_back();
    for (const AddedToken& a : t->added_) {
        if (a.content.empty()) data_fail("an added token has empty content");
        int32_t node = 0;
        for (char32_t c : a.content) {
            auto it = t->trie_[size_t(node)].next.find(uint32_t(c));
            if (it == t->trie_[size_t(node)].next.end()) {
                t->trie_.emplace_back();
                const int32_t nx = int32_t(t->trie_.size() - 1);
                t->trie_[size_t(node)].next[uint32_t(c)] = nx;
                node = nx;
            } else {
                node = it->second;
            }
        }
        if (t->trie_[size_t(node)].id >= 0) data_fail("the added token %s appears twice", utf8_encode(a.content).c_str());
        t->trie_[size_t(node)].id = a.id;
        t->added_by_content_[utf8_encode(a.content)] = a.id;
    }
    return t;
}

// ---------------------------------------------------------------- encode / decode

// Byte-level BPE of one piece (Bpe.fs:123-219): the bytes start as one symbol each; while some adjacent pair has a
// merge, the pair of the lowest rank is merged, the leftmost among equal ranks.
void Tokenizer::encode_piece(const std::u32string& s, size_t b, size_t e, std::vector<int32_t>& out) const {
    std::string bytes;
    for (size_t i = b; i < e; ++i) json::append_utf8(bytes, uint32_t(s[i]));
    const size_t m = bytes.size();
    if (m == 1) {
        out.push_back(byte_ids_[uint8_t(bytes[0])]);
        return;
    }
    std::vector<int32_t> sym(m);
    std::vector<long> next(m), prev(m);
    for (size_t i = 0; i < m; ++i) {
        sym[i] = byte_ids_[uint8_t(bytes[i])];
        next[i] = i + 1 < m ? long(i + 1) : -1;
        prev[i] = long(i) - 1;
    }
    // (rank << 32 | position of the left symbol): the lowest rank first, ties to the leftmost pair
    std::priority_queue<uint64_t, std::vector<uint64_t>, std::greater<uint64_t>> queue;
    auto merge_of = [&](long i, uint64_t& v) {
        const long j = next[size_t(i)];
        if (j < 0) return false;
        auto it = merges_.find((uint64_t(uint32_t(sym[size_t(i)])) << 32) | uint32_t(sym[size_t(j)]));
        if (it == merges_.end()) return false;
        v = it->second;
        return true;
    };
    auto push = [&](long i) {
        uint64_t v;
        if (merge_of(i, v)) queue.push(((v >> 32) << 32) | uint64_t(i));
    };
    for (size_t i = 0; i + 1 < m; ++i) push(long(i));
    while (!queue.empty()) {
        const uint64_t top = queue.top();
        queue.pop();
        const long i = long(top & 0xFFFFFFFFu);
        uint64_t v;
        // stale entries: the left symbol was absorbed, lost its right neighbour, or the pair changed (ranks are unique
        // per pair, so an unchanged rank is an unchanged pair)
        if (prev[size_t(i)] == -2 || !merge_of(i, v) || (v >> 32) != (top >> 32)) continue;
        const long j = next[size_t(i)];
        sym[size_t(i)] = int32_t(v & 0xFFFFFFFFu);
        const long k = next[size_t(j)];
        next[size_t(i)] = k;
        if (k >= 0) prev[size_t(k)] = i;
        prev[size_t(j)] = -2;
        if (prev[size_t(i)] >= 0) push(prev[size_t(i)]);
        push(i);
    }
    for (long i = 0; i >= 0; i = next[size_t(i)]) out.push_back(sym[size_t(i)]);
}

std::vector<int32_t> Tokenizer::encode_scalars(const std::u32string& text) const {
    std::vector<int32_t> ids;
    ids.reserve(text.size() / 3 + 4);
    auto segment = [&](size_t b, size_t e) {
        const std::u32string seg = nfc(text.substr(b, e - b));
        const std::vector<size_t> bounds = pre_split(seg);
        for (size_t i = 0; i + 1 < bounds.size(); ++i) encode_piece(seg, bounds[i], bounds[i + 1], ids);
    };
    // added tokens first, on the raw text: at the first position where one starts, the longest one there
    size_t start = 0, i = 0;
    while (i < text.size()) {
        int32_t node = 0, best = -1;
        size_t best_len = 0, k = i;
        while (k < text.size()) {
            auto it = trie_[size_t(node)].next.find(uint32_t(text[k]));
            if (it == trie_[size_t(node)].next.end()) break;
            node = it->second;
            ++k;
            if (trie_[size_t(node)].id >= 0) best = trie_[size_t(node)].id, best_len = k - i;
        }
        if (best >= 0) {
            if (i > start) segment(start, i);
            ids.push_back(best);
            i += best_len;
            start = i;
        } else {
            ++i;
        }
    }
    if (start < text.size()) segment(start, text.size());
    return ids;
}

std::vector<int32_t> Tokenizer::encode(const uint8_t* utf8, size_t n) const {
    std::u32string text;
    size_t bad = 0;
    if (!utf8_decode(utf8, n, text, &bad))
        throw std::invalid_argument("the text is not valid UTF-8 at byte " + std::to_string(bad) +
                                    "; only Unicode scalar values can be encoded");
    return encode_scalars(text);
}

std::vector<int32_t> Tokenizer::encode_bytes(const uint8_t* bytes, size_t n) const {
    return encode_scalars(utf8_decode_replace(bytes, n));
}

std::string Tokenizer::decode_bytes(const int32_t* ids, size_t n) const {
    std::string out;
    for (size_t i = 0; i < n; ++i) {
        const int32_t id = ids[i];
        if (id >= 0 && size_t(id) < token_bytes_.size()) {
            out += token_bytes_[size_t(id)];
        } else if (id >= 0 && size_t(id - int32_t(token_bytes_.size())) < added_.size()) {
            const std::u32string& c = added_[size_t(id) - token_bytes_.size()].content;
            std::string b;
            out += byte_level_decode(c, b) ? b : utf8_encode(c);  // the ByteLevel decoder's bytes of the content
        } else if (id >= vocab_size() && id < kModelRows) {
            // an lm_head row with no token
        } else {
            throw std::out_of_range("token id " + std::to_string(id) + " at index " + std::to_string(i) +
                                    " is outside the model's " + std::to_string(kModelRows) + " rows");
        }
    }
    return out;
}

int32_t Tokenizer::id_of(const std::string& token) const {
    auto a = added_by_content_.find(token);
    if (a != added_by_content_.end()) return a->second;
    auto v = vocab_.find(token);
    return v == vocab_.end() ? -1 : v->second;
}

bool Tokenizer::token_of(int32_t id, std::string& out) const {
    if (id >= 0 && size_t(id) < token_strings_.size()) {
        out = token_strings_[size_t(id)];
        return true;
    }
    if (id >= 0 && size_t(id - int32_t(token_strings_.size())) < added_.size()) {
        out = utf8_encode(added_[size_t(id) - token_strings_.size()].content);
        return true;
    }
    return false;
}

}  // namespace tok
}  // namespace lrm
