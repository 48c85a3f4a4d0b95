// The validating safetensors reader: header rules after SafetensorsParse (src/Lrm.Tensor/Safetensors.fs:296-498), the
// mapped file after SafetensorsFile (Safetensors.fs:504-727).
#include "safetensors.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <set>

#include "contract.hpp"
#include "json.hpp"
#include "sha256.hpp"

namespace lrm {

namespace {

[[noreturn]] void fail(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void fail(const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    throw FormatError(std::string("safetensors: ") + buf);
}

struct DtypeName {
    const char* name;
    uint32_t code;
};
// The dtypes the format names and the library reads (DType.safetensorsName, src/Lrm.Core/DType.fs:100-107); others,
// such as "BOOL", are unsupported.
const DtypeName kDtypes[] = {{"F32", F32}, {"BF16", BF16}, {"F16", F16}, {"I32", I32},
                             {"U32", U32}, {"U8", U8},     {"F64", F64}, {"I64", I64}};

const char* c(const std::string& s) { return s.c_str(); }

// Whether two names share code point order: the order of their UTF-8 bytes, unsigned.
bool code_point_less(const std::string& a, const std::string& b) {
    return std::lexicographical_compare(a.begin(), a.end(), b.begin(), b.end(),
                                        [](char x, char y) { return uint8_t(x) < uint8_t(y); });
}

StEntry entry(int64_t data_length, const std::string& name, const json::Value& v) {
    if (name.empty()) fail("empty tensor name");
    if (v.kind != json::Kind::Object) fail("%s: the entry is not an object", c(name));
    std::set<std::string> fields;
    bool has_dtype = false, has_shape = false, has_offsets = false;
    StEntry e{name, 0, {}, 0, 0};
    for (const auto& [field, fv] : v.members) {
        if (!fields.insert(field).second) fail("%s: duplicate field '%s'", c(name), c(field));
        if (field == "dtype") {
            if (fv.kind != json::Kind::String) fail("%s: dtype is not a string", c(name));
            bool found = false;
            for (const DtypeName& d : kDtypes)
                if (fv.text == d.name) {
                    e.dtype = d.code;
                    found = true;
                }
            if (!found) fail("%s: unsupported dtype '%s'", c(name), c(fv.text));
            has_dtype = true;
        } else if (field == "shape") {
            if (fv.kind != json::Kind::Array) fail("%s: shape is not an array", c(name));
            for (const json::Value& d : fv.items) {
                int64_t x;
                if (!json::nonnegative_int(d, &x)) fail("%s: shape: a dimension is not a non-negative integer", c(name));
                e.shape.push_back(x);
            }
            has_shape = true;
        } else if (field == "data_offsets") {
            if (fv.kind != json::Kind::Array || fv.items.size() != 2) fail("%s: data_offsets is not a pair", c(name));
            if (!json::nonnegative_int(fv.items[0], &e.begin) || !json::nonnegative_int(fv.items[1], &e.end))
                fail("%s: data_offsets: an offset is not a non-negative integer", c(name));
            has_offsets = true;
        } else {
            fail("%s: unknown field '%s'", c(name), c(field));
        }
    }
    if (!has_dtype || !has_shape || !has_offsets) fail("%s: the entry needs dtype, shape and data_offsets", c(name));
    // the element count and byte count must fit int64 (Shape.Of, src/Lrm.Tensor/Shape.fs:10-25)
    __int128 elements = 1;
    for (int64_t d : e.shape) {
        elements *= d;
        if (elements > INT64_MAX) fail("%s: the element count overflows int64", c(name));
    }
    const __int128 bytes = elements * dtype_size(e.dtype);
    if (bytes > INT64_MAX) fail("%s: the byte count overflows", c(name));
    if (e.end < e.begin) fail("%s: data_offsets [%lld, %lld] are reversed", c(name), (long long)e.begin, (long long)e.end);
    if (e.end - e.begin != int64_t(bytes))
        fail("%s: %lld bytes for %s (expected %lld)", c(name), (long long)(e.end - e.begin), dtype_name(e.dtype),
             (long long)bytes);
    if (e.end > data_length)
        fail("%s: data_offsets end %lld is beyond the data section (%lld bytes)", c(name), (long long)e.end,
             (long long)data_length);
    return e;
}

}  // namespace

const char* st_dtype_name(uint32_t dtype) {
    for (const DtypeName& d : kDtypes)
        if (d.code == dtype) return d.name;
    return nullptr;
}

StHeader st_validate(const uint8_t* head, uint64_t head_bytes, uint64_t length) {
    if (length < 8) fail("%llu bytes is shorter than the 8-byte header length", (unsigned long long)length);
    uint64_t n = 0;
    for (int k = 7; k >= 0; --k) n = (n << 8) | head[k];
    if (n > uint64_t(kMaxHeaderBytes)) fail("header length %llu exceeds %lld", (unsigned long long)n, (long long)kMaxHeaderBytes);
    if (n > length - 8) fail("header length %llu exceeds the file (%llu bytes)", (unsigned long long)n, (unsigned long long)length);
    if (head_bytes < 8 + n) fail("internal: %llu header bytes given, %llu needed", (unsigned long long)head_bytes, (unsigned long long)(8 + n));
    const int64_t data_length = int64_t(length - 8 - n);
    const uint8_t* h = head + 8;
    if (n == 0 || h[0] != '{') fail("the header is not a JSON object");
    if (!json::utf8_valid(h, size_t(n))) fail("the header is not valid UTF-8");
    json::Value doc;
    try {
        doc = json::parse(h, size_t(n), 8);
    } catch (const json::Error& e) {
        fail("the header is not valid JSON: %s", e.what());
    }
    if (doc.kind != json::Kind::Object) fail("the header is not a JSON object");

    StHeader out;
    out.header_length = int64_t(n);
    std::set<std::string> seen;
    for (const auto& [key, v] : doc.members) {
        if (!seen.insert(key).second) fail("duplicate key '%s'", c(key));
        if (key == "__metadata__") {
            if (v.kind != json::Kind::Object) fail("__metadata__ is not an object");
            std::set<std::string> keys;
            for (const auto& [k, mv] : v.members) {
                if (!keys.insert(k).second) fail("duplicate metadata key '%s'", c(k));
                if (mv.kind != json::Kind::String) fail("metadata '%s' is not a string", c(k));
                out.metadata.emplace_back(k, mv.text);
            }
        } else {
            out.entries.push_back(entry(data_length, key, v));
        }
    }
    // the tensors tile the data section exactly: no holes, no overlaps, nothing after the last one
    std::vector<const StEntry*> by_offset;
    for (const StEntry& e : out.entries) by_offset.push_back(&e);
    std::stable_sort(by_offset.begin(), by_offset.end(), [](const StEntry* a, const StEntry* b) {
        return a->begin != b->begin ? a->begin < b->begin : a->end < b->end;
    });
    int64_t position = 0;
    for (const StEntry* e : by_offset) {
        if (e->begin < position)
            fail("%s overlaps the previous tensor (begins at %lld, previous ends at %lld)", c(e->name),
                 (long long)e->begin, (long long)position);
        if (e->begin > position)
            fail("hole before %s (begins at %lld, previous ends at %lld)", c(e->name), (long long)e->begin,
                 (long long)position);
        position = e->end;
    }
    if (position != data_length) fail("%lld bytes after the last tensor", (long long)(data_length - position));
    std::sort(out.metadata.begin(), out.metadata.end(),
              [](const auto& a, const auto& b) { return code_point_less(a.first, b.first); });
    std::sort(out.entries.begin(), out.entries.end(),
              [](const StEntry& a, const StEntry& b) { return code_point_less(a.name, b.name); });
    return out;
}

std::unique_ptr<StFile> StFile::open(const std::string& path, int64_t expect_bytes, const char* expect_sha256) {
    char full[4096];
    const std::string shown = realpath(path.c_str(), full) ? std::string(full) : path;
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) throw std::invalid_argument(shown + ": cannot open: " + std::strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0) {
        const int err = errno;
        ::close(fd);
        throw std::invalid_argument(shown + ": cannot stat: " + std::strerror(err));
    }
    std::unique_ptr<StFile> f(new StFile());
    f->path_ = shown;
    f->length_ = uint64_t(st.st_size);
    if (expect_bytes >= 0 && uint64_t(expect_bytes) != f->length_) {
        ::close(fd);
        throw IntegrityError("integrity check failed for " + shown + ": expected " + std::to_string(expect_bytes) +
                             " bytes, found " + std::to_string(f->length_) + " bytes");
    }
    if (f->length_ > 0) {
        void* p = mmap(nullptr, f->length_, PROT_READ, MAP_PRIVATE, fd, 0);
        if (p == MAP_FAILED) {
            const int err = errno;
            ::close(fd);
            throw std::invalid_argument(shown + ": cannot map: " + std::strerror(err));
        }
        f->base_ = static_cast<const uint8_t*>(p);
        f->mapped_ = true;
    }
    ::close(fd);
    if (expect_sha256) {
        const std::string actual = Sha256::hex(Sha256::of(f->base_, f->length_));
        if (actual != expect_sha256)
            throw IntegrityError("integrity check failed for " + shown + ": expected sha256 " + expect_sha256 +
                                 ", found sha256 " + actual);
    }
    try {
        f->header_ = st_validate(f->base_, f->length_, f->length_);
    } catch (const FormatError& e) {
        // the message names the file: "safetensors: <path>: <rule>"
        throw FormatError("safetensors: " + shown + ": " + std::string(e.what()).substr(std::strlen("safetensors: ")));
    }
    for (size_t i = 0; i < f->header_.entries.size(); ++i) f->index_[f->header_.entries[i].name] = i;
    return f;
}

std::unique_ptr<StFile> StFile::from_memory(const uint8_t* bytes, uint64_t n) {
    std::unique_ptr<StFile> f(new StFile());
    f->owned_.assign(bytes, bytes + n);
    f->base_ = f->owned_.data();
    f->length_ = n;
    f->path_ = "<memory>";
    f->header_ = st_validate(f->base_, n, n);
    for (size_t i = 0; i < f->header_.entries.size(); ++i) f->index_[f->header_.entries[i].name] = i;
    return f;
}

StFile::~StFile() {
    if (mapped_ && base_) munmap(const_cast<uint8_t*>(base_), length_);
}

bool StFile::aligned() const {
    if (data_offset() % 8 != 0) return false;
    for (const StEntry& e : header_.entries)
        if (e.begin % dtype_size(e.dtype) != 0) return false;
    return true;
}

const StEntry* StFile::find(const std::string& name) const {
    auto it = index_.find(name);
    return it == index_.end() ? nullptr : &header_.entries[it->second];
}

}  // namespace lrm
