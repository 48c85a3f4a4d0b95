// Host-side contract checks of the HIP device: HeapLayout, HeapPlanner, TensorRow, TensorTable, the catalog and
// Dispatch.prepare (see contract.hpp for the reference files each part follows).
#include "contract.hpp"

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <unordered_map>

#include "sha256.hpp"

namespace lrm {

void contract_fail(const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    throw ContractError(buf);
}

int dtype_size(uint32_t c) {
    switch (c) {
        case F32: case I32: case U32: return 4;
        case BF16: case F16: return 2;
        case U8: return 1;
        case F64: case I64: return 8;
        default: return 0;
    }
}

const char* dtype_name(uint32_t c) {
    switch (c) {
        case F32: return "f32";
        case BF16: return "bf16";
        case F16: return "f16";
        case I32: return "i32";
        case U32: return "u32";
        case U8: return "u8";
        case F64: return "f64";
        case I64: return "i64";
        default: return "invalid";
    }
}

const char* arena_name(uint32_t c) {
    static const char* names[] = {"",       "weights", "rope", "kv_cache", "activations", "scratch", "logits",
                                  "taps",   "master",  "grad", "adam_m",   "adam_v",      "roslyn_in", "roslyn_out"};
    return c >= 1 && c <= 13 ? names[c] : "invalid";
}

static uint64_t align_up(uint64_t a, uint64_t x) { return (x + a - 1) / a * a; }

// ---------------------------------------------------------------- HeapLayout

HeapLayout HeapLayout::of_pages(const std::vector<std::pair<uint32_t, uint64_t>>& kb) {
    if (kb.size() > size_t(kSlotCount - 1)) contract_fail("%zu pages; a heap holds at most 63", kb.size());
    HeapLayout l;
    uint32_t last = 0;
    std::vector<int> per(14, 0);
    for (size_t i = 0; i < kb.size(); ++i) {
        uint32_t kind = kb[i].first;
        uint64_t bytes = kb[i].second;
        if (kind < 1 || kind > 13) contract_fail("page %zu: arena code %u is not an arena", i, kind);
        if (kind >= Master) contract_fail("page %zu: arena %s is reserved until contracts-v2", i, arena_name(kind));
        if (bytes < kPageGranularity || bytes > kMaxPageBytes || bytes % kPageGranularity != 0)
            contract_fail("page %zu: %llu bytes is not a multiple of 64 KiB in 64 KiB..1 GiB", i, (unsigned long long)bytes);
        if (kind < last) contract_fail("page %zu: arena %s after %s breaks contract order", i, arena_name(kind), arena_name(last));
        last = kind;
        l.pages.push_back(Page{int(i) + 1, kind, per[kind]++, bytes});
    }
    return l;
}

const Page& HeapLayout::page(int slot) const {
    if (!has_slot(slot)) contract_fail("slot %d holds no page in the layout", slot);
    return pages[size_t(slot - 1)];
}

uint64_t HeapLayout::total_bytes() const {
    uint64_t t = kTableBytes;
    for (auto& p : pages) t += p.bytes;
    return t;
}

// ---------------------------------------------------------------- HeapPlanner

HeapPlanner::HeapPlanner(uint64_t page_bytes) : page_bytes_(page_bytes), fill_(14) {
    if (page_bytes < kPageGranularity || page_bytes > kMaxPageBytes || page_bytes % kPageGranularity != 0)
        contract_fail("planner page size %llu is not a multiple of 64 KiB in 64 KiB..1 GiB", (unsigned long long)page_bytes);
}

Placement HeapPlanner::allocate(uint32_t arena, uint64_t bytes) {
    if (built_) contract_fail("the planner is built; no more allocations");
    if (arena < 1 || arena > 13) contract_fail("arena code %u is not an arena", arena);
    if (arena >= Master) contract_fail("arena %s is reserved until contracts-v2", arena_name(arena));
    if (bytes == 0 || bytes > page_bytes_) contract_fail("an allocation of %llu bytes does not fit one page", (unsigned long long)bytes);
    auto& pages = fill_[arena];
    if (!pages.empty()) {
        uint64_t off = align_up(kAllocationAlignment, pages.back());
        if (off + bytes <= page_bytes_) {
            pages.back() = off + bytes;
            return Placement{arena, int(pages.size()) - 1, off, bytes};
        }
    }
    pages.push_back(bytes);
    return Placement{arena, int(pages.size()) - 1, 0, bytes};
}

HeapLayout HeapPlanner::build() {
    if (!built_) {
        std::vector<std::pair<uint32_t, uint64_t>> kb;
        for (uint32_t a = 1; a <= 13; ++a)
            for (uint64_t f : fill_[a]) kb.emplace_back(a, align_up(kPageGranularity, f));
        layout_ = HeapLayout::of_pages(kb);
        built_ = true;
    }
    return layout_;
}

int HeapPlanner::slot_of(const Placement& p) const {
    if (!built_) contract_fail("the planner has not been built");
    for (auto& pg : layout_.pages)
        if (pg.arena == p.arena && pg.index == p.page) return pg.slot;
    contract_fail("placement (arena %s, page %d) is not in the layout", arena_name(p.arena), p.page);
}

// ---------------------------------------------------------------- TensorRow

uint32_t debug_id_of(const std::string& name) {
    if (name.empty()) return 0;
    auto d = Sha256::of(name.data(), name.size());
    return uint32_t(d[0]) | uint32_t(d[1]) << 8 | uint32_t(d[2]) << 16 | uint32_t(d[3]) << 24;
}

bool TensorRow::is_zero() const {
    for (uint32_t x : w)
        if (x) return false;
    return true;
}

uint64_t TensorRow::extent_bytes() const {
    int sz = dtype_size(dtype());
    if (!sz) return 0;
    uint64_t span = 1;
    for (uint32_t i = 0; i < rank() && i < 4; ++i) span += uint64_t(w[4 + i] - 1) * w[8 + i];
    return align_up(4, span * uint64_t(sz));
}

TensorRow TensorRow::create(int slot, uint64_t offset, uint32_t dtype, const std::vector<uint32_t>& dims, uint32_t flags,
                            const std::string& name) {
    if (dims.empty() || dims.size() > 4) contract_fail("tensor rank %zu is outside 1..4", dims.size());
    if (offset > 0xFFFFFFFFull) contract_fail("byte offset %llu does not fit in u32", (unsigned long long)offset);
    uint64_t count = 1;
    for (uint32_t d : dims) {
        if (d < 1) contract_fail("tensor dims must each be 1..2^32-1");
        count *= d;
        if (count > 0xFFFFFFFFull) contract_fail("tensor of %llu elements does not fit a u32 count", (unsigned long long)count);
    }
    TensorRow r;
    r.w[0] = uint32_t(slot);
    r.w[1] = uint32_t(offset);
    r.w[2] = dtype;
    r.w[3] = uint32_t(dims.size());
    uint64_t stride = 1;
    for (int i = 3; i >= 0; --i) {
        if (i < int(dims.size())) {
            r.w[4 + i] = dims[size_t(i)];
            r.w[8 + i] = uint32_t(stride);
            stride *= dims[size_t(i)];
        } else {
            r.w[4 + i] = 1;
            r.w[8 + i] = 0;
        }
    }
    r.w[12] = uint32_t(count);
    r.w[13] = (flags & ~uint32_t(Contiguous)) | Contiguous;
    r.w[14] = debug_id_of(name);
    r.w[15] = 0;
    return r;
}

void TensorRow::validate(const HeapLayout& layout) const {
    std::string problems;
    auto add = [&](const std::string& s) {
        if (!problems.empty()) problems += "; ";
        problems += s;
    };
    char b[256];
    if (slot() < 1 || slot() >= uint32_t(kSlotCount)) {
        snprintf(b, sizeof b, "slot %u is outside 1..63", slot());
        add(b);
    } else if (!layout.has_slot(int(slot()))) {
        snprintf(b, sizeof b, "slot %u holds no page in the layout", slot());
        add(b);
    }
    int sz = dtype_size(dtype());
    if (!sz) {
        snprintf(b, sizeof b, "dtype code %u is not a DType", dtype());
        add(b);
    } else if (offset() % uint32_t(std::max(4, sz)) != 0) {
        snprintf(b, sizeof b, "byte offset %u is not a multiple of %d", offset(), std::max(4, sz));
        add(b);
    }
    if (rank() < 1 || rank() > 4) {
        snprintf(b, sizeof b, "rank %u is outside 1..4", rank());
        add(b);
    } else {
        uint64_t product = 1;
        for (uint32_t i = 0; i < 4; ++i) {
            if (i < rank() && w[4 + i] < 1) add("a used dim is 0");
            if (i >= rank() && (w[4 + i] != 1 || w[8 + i] != 0)) add("unused dims must be 1 with stride 0");
            if (i < rank()) product *= w[4 + i];
        }
        if (product != count()) add("element count is not the product of the dims");
        bool packed = true;
        uint64_t stride = 1;
        for (int i = int(rank()) - 1; i >= 0; --i) {
            if (w[8 + i] != stride) packed = false;
            stride *= w[4 + i];
        }
        if (bool(flags() & Contiguous) != packed) add("the Contiguous flag must be set exactly when the strides are packed row-major");
    }
    if (flags() & ~uint32_t(Contiguous | ReadOnly | View)) add("flags use reserved bits");
    if (w[15] != 0) add("word 15 is reserved and must be 0");
    if (problems.empty()) {
        const Page& p = layout.page(int(slot()));
        uint64_t end = uint64_t(offset()) + extent_bytes();
        if (end > p.bytes) {
            snprintf(b, sizeof b, "extent ends at byte %llu, past the %llu-byte page in slot %u", (unsigned long long)end,
                     (unsigned long long)p.bytes, slot());
            add(b);
        }
    }
    if (!problems.empty()) throw ContractError(problems);
}

// ---------------------------------------------------------------- TensorTable

uint32_t TensorTable::add(const std::string& name, int slot, uint64_t offset, uint32_t dtype,
                          const std::vector<uint32_t>& dims, uint32_t flags) {
    if (sealed_) contract_fail("the tensor table is sealed");
    if (name.empty()) contract_fail("a tensor needs a name");
    if (find(name)) contract_fail("tensor name '%s' is already in the table", name.c_str());
    if (rows_.size() + 1 >= size_t(kTableRows)) contract_fail("the tensor table is full (%d rows)", kTableRows - 1);
    TensorRow r = TensorRow::create(slot, offset, dtype, dims, flags, name);
    try {
        r.validate(layout_);
    } catch (const ContractError& e) {
        contract_fail("tensor '%s': %s", name.c_str(), e.what());
    }
    rows_.push_back(r);
    names_.push_back(name);
    return uint32_t(rows_.size());
}

uint32_t TensorTable::add_placed(const std::string& name, const HeapPlanner& planner, const Placement& p, uint32_t dtype,
                                 const std::vector<uint32_t>& dims, uint32_t flags) {
    int slot = planner.slot_of(p);
    TensorRow probe = TensorRow::create(slot, p.offset, dtype, dims, flags, name);
    if (probe.extent_bytes() > align_up(4, p.bytes))
        contract_fail("tensor '%s' needs %llu bytes but its placement has %llu", name.c_str(),
                      (unsigned long long)probe.extent_bytes(), (unsigned long long)p.bytes);
    return add(name, slot, p.offset, dtype, dims, flags);
}

uint32_t TensorTable::add_view(const std::string& name, uint32_t source, const std::vector<uint32_t>& dims,
                               uint64_t element_offset) {
    if (source == 0 || source > rows_.size()) contract_fail("cannot view token %u", source);
    const TensorRow src = rows_[source - 1];
    uint64_t off = uint64_t(src.offset()) + element_offset * uint64_t(dtype_size(src.dtype()));
    TensorRow r = TensorRow::create(int(src.slot()), off, src.dtype(), dims, View | (src.flags() & ReadOnly), name);
    if (off + r.extent_bytes() > uint64_t(src.offset()) + src.extent_bytes())
        contract_fail("view '%s' does not lie inside its source %u", name.c_str(), source);
    return add(name, int(src.slot()), off, src.dtype(), dims, View | (src.flags() & ReadOnly));
}

void TensorTable::seal() {
    if (sealed_) contract_fail("the tensor table is sealed");
    image_.assign(kTableBytes, 0);
    for (size_t t = 0; t < rows_.size(); ++t) std::memcpy(image_.data() + (t + 1) * kRowBytes, rows_[t].w.data(), kRowBytes);
    sealed_ = true;
}

const std::vector<uint8_t>& TensorTable::image() const {
    if (!sealed_) contract_fail("the tensor table is not sealed");
    return image_;
}

uint32_t TensorTable::find(const std::string& name) const {
    for (size_t i = 0; i < names_.size(); ++i)
        if (names_[i] == name) return uint32_t(i + 1);
    return 0;
}

TensorRow SealedTableView::row(uint32_t token) const {
    if (token >= uint32_t(kTableRows)) contract_fail("token %u is not below 16,384", token);
    TensorRow r;
    std::memcpy(r.w.data(), image + size_t(token) * kRowBytes, kRowBytes);
    return r;
}

// ---------------------------------------------------------------- the catalog, ids 0..13 (catalog.json)

static int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

#define DT(x) (1u << (x))
#define TOK_R(n, m) FieldSpec{n, FieldKind::Token, Access::Read, m, nullptr}
#define TOK_W(n, m, al) FieldSpec{n, FieldKind::Token, Access::Write, m, al}
#define TOK_META(n) FieldSpec{n, FieldKind::Token, Access::Meta, 0, nullptr}
#define U32F(n) FieldSpec{n, FieldKind::U32, Access::None, 0, nullptr}
#define F32F(n) FieldSpec{n, FieldKind::F32, Access::None, 0, nullptr}

static void need(const uint32_t* counts, int field, int64_t elems, const char* kernel, const char* what) {
    if (elems < 0 || int64_t(counts[field]) < elems)
        contract_fail("%s.%s holds %u elements; the dispatch touches %lld", kernel, what, counts[field], (long long)elems);
}

static std::vector<KernelSpec> base_catalog() {
    std::vector<KernelSpec> c;
    // 0 scale_f32: x, y, n, a
    c.push_back({"scale_f32", "selftest", {256, 1, 1}, true,
                 [](const uint32_t* w) { return Grid3{cdiv(w[3], 256), 1, 1}; },
                 {TOK_R("x", DT(F32)), TOK_W("y", DT(F32), "x"), U32F("n"), F32F("a")},
                 [](const uint32_t* w, const uint32_t* c) {
                     need(c, 0, w[3], "scale_f32", "x");
                     need(c, 1, w[3], "scale_f32", "y");
                 }});
    // 1 table_echo: src (meta), y
    c.push_back({"table_echo", "selftest", {16, 1, 1}, true, [](const uint32_t*) { return Grid3{1, 1, 1}; },
                 {TOK_META("src"), TOK_W("y", DT(U32), nullptr)},
                 [](const uint32_t*, const uint32_t* c) { need(c, 1, 16, "table_echo", "y"); }});
    // 2 args_echo: y, v2..v31
    {
        std::vector<FieldSpec> f{TOK_W("y", DT(U32), nullptr)};
        static const char* names[] = {"v2",  "v3",  "v4",  "v5",  "v6",  "v7",  "v8",  "v9",  "v10", "v11",
                                      "v12", "v13", "v14", "v15", "v16", "v17", "v18", "v19", "v20", "v21",
                                      "v22", "v23", "v24", "v25", "v26", "v27", "v28", "v29", "v30", "v31"};
        for (auto n : names) f.push_back(U32F(n));
        c.push_back({"args_echo", "selftest", {32, 1, 1}, true, [](const uint32_t*) { return Grid3{1, 1, 1}; }, f,
                     [](const uint32_t*, const uint32_t* c) { need(c, 0, 32, "args_echo", "y"); }});
    }
    // 3 groups_echo: y, groups
    c.push_back({"groups_echo", "selftest", {1, 1, 1}, true, [](const uint32_t* w) { return Grid3{w[2], 1, 1}; },
                 {TOK_W("y", DT(U32), nullptr), U32F("groups")},
                 [](const uint32_t* w, const uint32_t* c) { need(c, 0, w[2], "groups_echo", "y"); }});
    // 4 bf16_unpack: x, y, n
    c.push_back({"bf16_unpack", "selftest", {256, 1, 1}, true,
                 [](const uint32_t* w) { return Grid3{cdiv(w[3], 256), 1, 1}; },
                 {TOK_R("x", DT(BF16)), TOK_W("y", DT(F32), nullptr), U32F("n")},
                 [](const uint32_t* w, const uint32_t* c) {
                     need(c, 0, w[3], "bf16_unpack", "x");
                     need(c, 1, w[3], "bf16_unpack", "y");
                 }});
    // 5 embed_gather_bf16: ids, table, y, rows, cols, vocab
    c.push_back({"embed_gather_bf16", "basic", {256, 1, 1}, false,
                 [](const uint32_t* w) { return Grid3{cdiv(w[5], 256), w[4], 1}; },
                 {TOK_R("ids", DT(U32)), TOK_R("table", DT(BF16)), TOK_W("y", DT(F32), nullptr), U32F("rows"),
                  U32F("cols"), U32F("vocab")},
                 [](const uint32_t* w, const uint32_t* c) {
                     need(c, 0, w[4], "embed_gather_bf16", "ids");
                     need(c, 1, int64_t(w[6]) * w[5], "embed_gather_bf16", "table");
                     need(c, 2, int64_t(w[4]) * w[5], "embed_gather_bf16", "y");
                 }});
    // 6 rmsnorm_rows: x, w, y, rows, cols, eps
    c.push_back({"rmsnorm_rows", "basic", {256, 1, 1}, true, [](const uint32_t* w) { return Grid3{w[4], 1, 1}; },
                 {TOK_R("x", DT(F32)), TOK_R("w", DT(BF16)), TOK_W("y", DT(F32), "x"), U32F("rows"), U32F("cols"),
                  F32F("eps")},
                 [](const uint32_t* w, const uint32_t* c) {
                     if (w[5] < 1) contract_fail("rmsnorm_rows: cols must be at least 1");
                     need(c, 0, int64_t(w[4]) * w[5], "rmsnorm_rows", "x");
                     need(c, 1, w[5], "rmsnorm_rows", "w");
                     need(c, 2, int64_t(w[4]) * w[5], "rmsnorm_rows", "y");
                 }});
    // 7 rope_apply: x, cos_table, sin_table, y, rows, heads, head_dim, pos0
    c.push_back({"rope_apply", "basic", {64, 1, 1}, true, [](const uint32_t* w) { return Grid3{w[5], 1, 1}; },
                 {TOK_R("x", DT(F32)), TOK_R("cos_table", DT(F32)), TOK_R("sin_table", DT(F32)),
                  TOK_W("y", DT(F32), "x"), U32F("rows"), U32F("heads"), U32F("head_dim"), U32F("pos0")},
                 [](const uint32_t* w, const uint32_t* c) {
                     uint32_t rows = w[5], heads = w[6], hd = w[7], pos0 = w[8];
                     if (heads < 1 || rows % heads != 0) contract_fail("rope_apply: heads must be >= 1 and divide rows");
                     if (hd < 2 || hd % 2 != 0) contract_fail("rope_apply: head_dim must be even and at least 2");
                     need(c, 0, int64_t(rows) * hd, "rope_apply", "x");
                     need(c, 1, (int64_t(pos0) + rows / heads) * (hd / 2), "rope_apply", "cos_table");
                     need(c, 2, (int64_t(pos0) + rows / heads) * (hd / 2), "rope_apply", "sin_table");
                     need(c, 3, int64_t(rows) * hd, "rope_apply", "y");
                 }});
    // 8 silu_mul: gate, up, y, n
    c.push_back({"silu_mul", "basic", {256, 1, 1}, true, [](const uint32_t* w) { return Grid3{cdiv(w[4], 256), 1, 1}; },
                 {TOK_R("gate", DT(F32)), TOK_R("up", DT(F32)), TOK_W("y", DT(F32), "gate,up"), U32F("n")},
                 [](const uint32_t* w, const uint32_t* c) {
                     for (int i = 0; i < 3; ++i) need(c, i, w[4], "silu_mul", i == 0 ? "gate" : i == 1 ? "up" : "y");
                 }});
    // 9 add: a, b, y, n
    c.push_back({"add", "basic", {256, 1, 1}, true, [](const uint32_t* w) { return Grid3{cdiv(w[4], 256), 1, 1}; },
                 {TOK_R("a", DT(F32)), TOK_R("b", DT(F32)), TOK_W("y", DT(F32), "a,b"), U32F("n")},
                 [](const uint32_t* w, const uint32_t* c) {
                     for (int i = 0; i < 3; ++i) need(c, i, w[4], "add", i == 0 ? "a" : i == 1 ? "b" : "y");
                 }});
    // 10 copy_rows: src, dst, rows, cols, src_row0, dst_row0, src_stride, dst_stride
    c.push_back({"copy_rows", "basic", {256, 1, 1}, true,
                 [](const uint32_t* w) { return Grid3{cdiv(int64_t(w[3]) * w[4], 256), 1, 1}; },
                 {TOK_R("src", DT(F32) | DT(U32) | DT(I32)), TOK_W("dst", DT(F32) | DT(U32) | DT(I32), nullptr),
                  U32F("rows"), U32F("cols"), U32F("src_row0"), U32F("dst_row0"), U32F("src_stride"),
                  U32F("dst_stride")},
                 [](const uint32_t* w, const uint32_t* c) {
                     int64_t rows = w[3], cols = w[4];
                     if (rows > 1 && cols > int64_t(w[8])) contract_fail("copy_rows: cols exceeds dst_stride");
                     need(c, 0, (int64_t(w[5]) + rows - 1) * w[7] + cols, "copy_rows", "src");
                     need(c, 1, (int64_t(w[6]) + rows - 1) * w[8] + cols, "copy_rows", "dst");
                 }});
    // 11 argmax_rows: x, y, rows, cols
    c.push_back({"argmax_rows", "basic", {256, 1, 1}, true, [](const uint32_t* w) { return Grid3{w[3], 1, 1}; },
                 {TOK_R("x", DT(F32)), TOK_W("y", DT(U32), nullptr), U32F("rows"), U32F("cols")},
                 [](const uint32_t* w, const uint32_t* c) {
                     if (w[4] < 1) contract_fail("argmax_rows: cols must be at least 1");
                     need(c, 0, int64_t(w[3]) * w[4], "argmax_rows", "x");
                     need(c, 1, w[3], "argmax_rows", "y");
                 }});
    // 12 matmul_bf16w: x, w, y, m, n, k
    c.push_back({"matmul_bf16w", "matmul", {16, 16, 1}, false,
                 [](const uint32_t* w) { return Grid3{cdiv(w[5], 64), cdiv(w[4], 64), 1}; },
                 {TOK_R("x", DT(F32)), TOK_R("w", DT(BF16)), TOK_W("y", DT(F32), nullptr), U32F("m"), U32F("n"),
                  U32F("k")},
                 [](const uint32_t* w, const uint32_t* c) {
                     need(c, 0, int64_t(w[4]) * w[6], "matmul_bf16w", "x");
                     need(c, 1, int64_t(w[5]) * w[6], "matmul_bf16w", "w");
                     need(c, 2, int64_t(w[4]) * w[5], "matmul_bf16w", "y");
                 }});
    // 13 attention_gqa_causal: q, k, v, y, rows, q_row0, past, q_heads, kv_heads, head_dim, scale
    c.push_back({"attention_gqa_causal", "attention", {64, 1, 1}, false,
                 [](const uint32_t* w) { return Grid3{w[5], w[8], 1}; },
                 {TOK_R("q", DT(F32)), TOK_R("k", DT(F32)), TOK_R("v", DT(F32)), TOK_W("y", DT(F32), nullptr),
                  U32F("rows"), U32F("q_row0"), U32F("past"), U32F("q_heads"), U32F("kv_heads"), U32F("head_dim"),
                  F32F("scale")},
                 [](const uint32_t* w, const uint32_t* c) {
                     int64_t rows = w[5], q0 = w[6], past = w[7], qh = w[8], kvh = w[9], hd = w[10];
                     if (kvh < 1 || qh % kvh != 0) contract_fail("attention_gqa_causal: kv_heads must divide q_heads");
                     if (hd < 1) contract_fail("attention_gqa_causal: head_dim must be at least 1");
                     need(c, 0, (q0 + rows) * qh * hd, "attention_gqa_causal", "q");
                     need(c, 1, (past + rows) * kvh * hd, "attention_gqa_causal", "k");
                     need(c, 2, (past + rows) * kvh * hd, "attention_gqa_causal", "v");
                     need(c, 3, (q0 + rows) * qh * hd, "attention_gqa_causal", "y");
                 }});
    return c;
}

// The appended entries of this backend (ids 14 and up), defined next to their kernels' host code.
std::vector<KernelSpec> fast_catalog();

const std::vector<KernelSpec>& catalog() {
    static const std::vector<KernelSpec> all = [] {
        auto c = base_catalog();
        auto f = fast_catalog();
        c.insert(c.end(), f.begin(), f.end());
        return c;
    }();
    return all;
}

int catalog_size() { return int(catalog().size()); }

int catalog_find(const char* name) {
    auto& c = catalog();
    for (size_t i = 0; i < c.size(); ++i)
        if (std::strcmp(c[i].name, name) == 0) return int(i);
    return -1;
}

// ---------------------------------------------------------------- grids and prepare

Physical grid_physical(bool linear, const Grid3& g) {
    if (g.x < 1 || g.y < 1 || g.z < 1)
        contract_fail("grid (%lld, %lld, %lld) is empty; callers skip empty work", (long long)g.x, (long long)g.y, (long long)g.z);
    if (g.y > 65535 || g.z > 65535) contract_fail("grid y and z must be at most 65,535");
    if (g.x <= 65535) return Physical{uint32_t(g.x), uint32_t(g.y), uint32_t(g.z)};
    if (!linear) contract_fail("grid x of %lld exceeds 65,535 and the kernel is not linear", (long long)g.x);
    if (g.x > 65535ll * 65535ll) contract_fail("grid x of %lld exceeds 65,535 squared", (long long)g.x);
    int64_t yy = cdiv(g.x, 65535);
    int64_t xx = cdiv(g.x, yy);
    return Physical{uint32_t(xx), uint32_t(yy), 1};
}

static bool writes(Access a) { return a == Access::Write || a == Access::ReadWrite; }

static bool alias_lists(const char* alias, const char* name) {
    if (!alias) return false;
    std::string s(alias);
    size_t p = 0;
    while (p <= s.size()) {
        size_t q = s.find(',', p);
        if (q == std::string::npos) q = s.size();
        if (s.compare(p, q - p, name) == 0 && std::strlen(name) == q - p) return true;
        p = q + 1;
    }
    return false;
}

static PreparedDispatch prepare_impl(const SealedTableView& table, int kernel, const uint32_t* words, int library) {
    auto& cat = catalog();
    if (kernel < 0 || kernel >= int(cat.size())) contract_fail("kernel id %d is not in the catalog", kernel);
    const KernelSpec& k = cat[size_t(kernel)];
    if (words[0] != 0) contract_fail("%s: argument word 0 is lrm_groups_x, which Dispatch writes; pass 0", k.name);
    for (size_t w = k.fields.size() + 1; w < 32; ++w)
        if (words[w] != 0) contract_fail("%s: argument word %zu is past the last field and must be 0", k.name, w);
    PreparedDispatch pd;
    pd.kernel = kernel;
    uint32_t counts[32] = {0};
    for (size_t i = 0; i < k.fields.size(); ++i) {
        const FieldSpec& f = k.fields[i];
        if (f.kind != FieldKind::Token) continue;
        uint32_t token = words[i + 1];
        if (int(i) == library) {
            if (token != 0) contract_fail("%s.%s: the library supplies this buffer; pass token 0", k.name, f.name);
            counts[i] = 0xFFFFFFFFu;
            continue;
        }
        TensorRow row = table.row(token);
        if (f.access == Access::Meta) {
            if (token != 0 && row.is_zero()) contract_fail("%s.%s: token %u is not in the table", k.name, f.name, token);
        } else {
            if (token == 0) contract_fail("%s.%s: the null token is not allowed here", k.name, f.name);
            if (row.is_zero()) contract_fail("%s.%s: token %u is not in the table", k.name, f.name, token);
            if (!(f.dtype_mask & (1u << row.dtype())))
                contract_fail("%s.%s: token %u is %s, which the kernel does not accept", k.name, f.name, token,
                              dtype_name(row.dtype()));
            if (!(row.flags() & Contiguous)) contract_fail("%s.%s: token %u is not contiguous", k.name, f.name, token);
            if (writes(f.access) && (row.flags() & ReadOnly))
                contract_fail("%s.%s: token %u is read only", k.name, f.name, token);
            counts[i] = row.count();
        }
        uint64_t start = row.offset();
        pd.tokens.push_back(TokenUse{int(i), f.access, token, row, start, start + row.extent_bytes()});
    }
    // aliasing (Dispatch.fs:104-143)
    for (size_t i = 0; i < pd.tokens.size(); ++i) {
        for (size_t j = i + 1; j < pd.tokens.size(); ++j) {
            const TokenUse &a = pd.tokens[i], &b = pd.tokens[j];
            if (a.access == Access::Meta || b.access == Access::Meta) continue;
            bool overlap = a.row.slot() == b.row.slot() && a.start < b.end && b.start < a.end;
            if (!overlap || !(writes(a.access) || writes(b.access))) continue;
            const FieldSpec &fa = k.fields[size_t(a.field)], &fb = k.fields[size_t(b.field)];
            bool same = a.start == b.start && a.end == b.end;
            bool declared = (writes(a.access) && !writes(b.access) && alias_lists(fa.alias, fb.name)) ||
                            (writes(b.access) && !writes(a.access) && alias_lists(fb.alias, fa.name));
            if (!(declared && same))
                contract_fail("%s: %s and %s overlap in slot %u, and %s", k.name, fa.name, fb.name, a.row.slot(),
                              declared ? "a declared alias must span exactly the same bytes"
                                       : "the catalog does not let them alias");
        }
    }
    pd.grid = k.grid(words);
    pd.physical = grid_physical(k.linear, pd.grid);
    if (k.check_counts) k.check_counts(words, counts);
    std::memcpy(pd.words.data(), words, 128);
    pd.words[0] = pd.physical.x;
    return pd;
}

PreparedDispatch prepare(const SealedTableView& table, int kernel, const uint32_t* words) {
    return prepare_impl(table, kernel, words, -1);
}

PreparedDispatch prepare_library_field(const SealedTableView& table, int kernel, const uint32_t* words,
                                       int library_field) {
    auto& cat = catalog();
    if (kernel < 0 || kernel >= int(cat.size())) contract_fail("kernel id %d is not in the catalog", kernel);
    const auto& fields = cat[size_t(kernel)].fields;
    if (library_field < 0 || library_field >= int(fields.size()) || fields[size_t(library_field)].kind != FieldKind::Token)
        contract_fail("%s: field %d is not a token field", cat[size_t(kernel)].name, library_field);
    return prepare_impl(table, kernel, words, library_field);
}

void check_copy(const HeapLayout& layout, int ss, uint64_t so, int ds, uint64_t dof, uint64_t bytes) {
    auto check = [&](const char* what, int slot, uint64_t off) {
        if (slot < 1 || slot >= kSlotCount) contract_fail("copy %s: slot %d is not a page slot (1..63)", what, slot);
        const Page& p = layout.page(slot);
        if (off % 4 || bytes % 4) contract_fail("copy %s: offset and size must be multiples of 4", what);
        if (off + bytes > p.bytes) contract_fail("copy %s: range ends past the page in slot %d", what, slot);
    };
    if (bytes == 0) contract_fail("copy: the size must be positive");
    check("source", ss, so);
    check("destination", ds, dof);
    if (ss == ds && so < dof + bytes && dof < so + bytes) contract_fail("copy: source and destination overlap");
}

void check_transfer(const HeapLayout& layout, int slot, uint64_t offset, uint64_t bytes, bool allow_table) {
    if (offset % 4 || bytes % 4) contract_fail("transfer: offset and size must be multiples of 4");
    if (slot == kTableSlot) {
        if (!allow_table) contract_fail("transfer: slot 0 is the table, written only by WriteTable");
        if (offset + bytes > kTableBytes) contract_fail("transfer: range ends past the table");
        return;
    }
    const Page& p = layout.page(slot);
    if (offset + bytes > p.bytes) contract_fail("transfer: range ends past the page in slot %d", slot);
}

}  // namespace lrm
