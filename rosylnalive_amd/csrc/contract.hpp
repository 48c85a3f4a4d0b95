// The host-side contract of the reference's Lrm.Gpu.Core, restated in C++ for the HIP device and its executor:
//   - heap constants, arenas and HeapLayout / HeapPlanner   (src/Lrm.Gpu.Core/HeapLayout.fs:149-525)
//   - the 64-byte TensorRow and the sealed TensorTable image (src/Lrm.Gpu.Core/TensorTable.fs:46-474)
//   - the 128-byte ArgBlock, catalog grids and folding        (src/Lrm.Gpu.Core/ArgBlock.fs:240-393)
//   - the kernel catalog (ids 0..13 as catalog.json, plus the appended bf16 kernels of this backend)
//   - Dispatch.prepare: word rules, token rules, aliasing     (src/Lrm.Gpu.Core/Dispatch.fs:48-173)
// Violations throw ContractError, the counterpart of GpuContractException (src/Lrm.Gpu.Core/Errors.fs:7-13).
#pragma once

#include <array>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

namespace lrm {

struct ContractError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

[[noreturn]] void contract_fail(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

// ---- heap constants (HeapLayout.fs:149-175) ----
constexpr int kSlotCount = 64;
constexpr int kTableSlot = 0;
constexpr int kTableRows = 16384;
constexpr int kRowBytes = 64;
constexpr uint64_t kTableBytes = uint64_t(kTableRows) * kRowBytes;  // 1 MiB
constexpr uint64_t kMaxPageBytes = 1ull << 30;
constexpr uint64_t kPageGranularity = 64ull << 10;
constexpr uint64_t kAllocationAlignment = 256;

// ---- dtype codes (LrmCore DType codes, heap-and-tensor-table.md "TensorRow") ----
enum DType : uint32_t { F32 = 1, BF16 = 2, F16 = 3, I32 = 4, U32 = 5, U8 = 6, F64 = 7, I64 = 8 };
int dtype_size(uint32_t code);  // 0 for an invalid code
const char* dtype_name(uint32_t code);

// ---- arenas (HeapLayout.fs:6-36): codes 1..7 usable, 8..13 reserved until a later contract ----
enum Arena : uint32_t {
    Weights = 1, Rope = 2, KvCache = 3, Activations = 4, Scratch = 5, Logits = 6, Taps = 7,
    Master = 8, Grad = 9, AdamM = 10, AdamV = 11, RoslynIn = 12, RoslynOut = 13
};
const char* arena_name(uint32_t code);

struct Page {
    int slot;         // 1..63
    uint32_t arena;   // Arena code
    int index;        // position within its arena
    uint64_t bytes;   // multiple of 64 KiB, 64 KiB .. 1 GiB
};

// HeapLayout.ofPages: at most 63 pages, sizes multiples of 64 KiB in 64 KiB..1 GiB, no reserved kind, kinds in
// contract order.
struct HeapLayout {
    std::vector<Page> pages;
    static HeapLayout of_pages(const std::vector<std::pair<uint32_t, uint64_t>>& kinds_and_bytes);
    const Page& page(int slot) const;  // throws for a slot that is not a page
    bool has_slot(int slot) const { return slot >= 1 && slot <= int(pages.size()); }
    uint64_t total_bytes() const;      // the table included
};

struct Placement {
    uint32_t arena;
    int page;          // index within the arena
    uint64_t offset;
    uint64_t bytes;
};

// HeapPlanner (HeapLayout.fs:433-525): an allocation goes at the end of its arena's last page, aligned to 256, when it
// fits, otherwise at offset 0 of a new page; Build rounds every page up to 64 KiB in contract order.
class HeapPlanner {
  public:
    explicit HeapPlanner(uint64_t page_bytes = kMaxPageBytes);
    Placement allocate(uint32_t arena, uint64_t bytes);
    HeapLayout build();
    int slot_of(const Placement& p) const;  // valid after build()

  private:
    uint64_t page_bytes_;
    bool built_ = false;
    std::vector<std::vector<uint64_t>> fill_;  // per arena code (index 0 unused): fill level of each page
    HeapLayout layout_;
};

// ---- TensorRow (TensorTable.fs:46-59) ----
enum Flags : uint32_t { Contiguous = 1, ReadOnly = 2, View = 4 };

struct TensorRow {
    std::array<uint32_t, 16> w{};  // the 16 little-endian words
    uint32_t slot() const { return w[0]; }
    uint32_t offset() const { return w[1]; }
    uint32_t dtype() const { return w[2]; }
    uint32_t rank() const { return w[3]; }
    uint32_t count() const { return w[12]; }
    uint32_t flags() const { return w[13]; }
    bool is_zero() const;
    uint64_t extent_bytes() const;  // (1 + sum (dims-1)*strides) * size, rounded up to 4
    static TensorRow create(int slot, uint64_t offset, uint32_t dtype, const std::vector<uint32_t>& dims,
                            uint32_t flags, const std::string& name);
    void validate(const HeapLayout& layout) const;  // TensorRow.validate
};

uint32_t debug_id_of(const std::string& name);  // first 4 bytes of SHA-256(UTF-8 name), little-endian

// TensorTable + SealedTable (TensorTable.fs:321-474): tokens 1, 2, ... in order, unique names, sealed once.
class TensorTable {
  public:
    explicit TensorTable(HeapLayout layout) : layout_(std::move(layout)) {}
    uint32_t add(const std::string& name, int slot, uint64_t offset, uint32_t dtype, const std::vector<uint32_t>& dims,
                 uint32_t flags);
    uint32_t add_placed(const std::string& name, const HeapPlanner& planner, const Placement& p, uint32_t dtype,
                        const std::vector<uint32_t>& dims, uint32_t flags);
    uint32_t add_view(const std::string& name, uint32_t source, const std::vector<uint32_t>& dims, uint64_t element_offset);
    void seal();
    bool sealed() const { return sealed_; }
    const std::vector<uint8_t>& image() const;  // 1 MiB; valid after seal()
    const HeapLayout& layout() const { return layout_; }
    uint32_t size() const { return uint32_t(rows_.size()); }
    uint32_t find(const std::string& name) const;  // 0 when absent

  private:
    HeapLayout layout_;
    std::vector<TensorRow> rows_;   // token t at rows_[t - 1]
    std::vector<std::string> names_;
    std::vector<uint8_t> image_;
    bool sealed_ = false;
};

// A read-only view of a sealed table image (as the device keeps it after WriteTable).
struct SealedTableView {
    const uint8_t* image = nullptr;  // kTableBytes
    TensorRow row(uint32_t token) const;  // zero row for token 0 / unused; throws for token >= 16384
    bool assigned(uint32_t token) const { return token != 0 && token < uint32_t(kTableRows) && !row(token).is_zero(); }
};

// ---- the catalog (kernel-abi.md "The catalog"; catalog.json) ----
enum class FieldKind : uint8_t { Token = 1, U32 = 2, I32 = 3, F32 = 4 };
enum class Access : uint8_t { None = 0, Read = 1, Write = 2, ReadWrite = 3, Meta = 4 };

struct FieldSpec {
    const char* name;
    FieldKind kind;
    Access access;
    uint32_t dtype_mask;  // bit (1 << code) per accepted dtype
    const char* alias;    // comma-separated read fields this written field may alias, or nullptr
};

struct Grid3 {
    int64_t x, y, z;
};

struct KernelSpec {
    const char* name;
    const char* family;
    int threads[3];
    bool linear;                                      // grid y and z are the literal 1
    Grid3 (*grid)(const uint32_t* w);                 // the logical grid from the argument words
    std::vector<FieldSpec> fields;                    // field i is word i + 1
    void (*check_counts)(const uint32_t* w, const uint32_t* counts);  // minimum element counts; counts[i] for field i
};

const std::vector<KernelSpec>& catalog();
int catalog_size();
int catalog_find(const char* name);  // -1 when absent

// Grid.physical (ArgBlock.fs:368-387)
struct Physical {
    uint32_t x, y, z;
};
Physical grid_physical(bool linear, const Grid3& g);

struct TokenUse {
    int field;
    Access access;
    uint32_t token;
    TensorRow row;
    uint64_t start, end;  // byte range inside row.slot()
};

struct PreparedDispatch {
    int kernel;
    Grid3 grid;
    Physical physical;
    std::array<uint32_t, 32> words;   // word 0 = physical x
    std::vector<TokenUse> tokens;
};

// Dispatch.prepare (Dispatch.fs:149-173) plus the minimum element counts of kernel-abi.md, which this device checks
// on the host before every launch so no kernel can touch memory outside its tensors.
PreparedDispatch prepare(const SealedTableView& table, int kernel, const uint32_t* words);
// The same checks for a dispatch one of whose token fields, `library_field`, is memory the library supplies rather
// than a tensor of the heap: its word must be 0 and it takes no part in the token, aliasing and minimum-count rules
// (the caller checks the bytes the launch touches against its own buffer).
PreparedDispatch prepare_library_field(const SealedTableView& table, int kernel, const uint32_t* words,
                                       int library_field);

// Dispatch.checkCopy / checkTransfer
void check_copy(const HeapLayout& layout, int src_slot, uint64_t src_off, int dst_slot, uint64_t dst_off, uint64_t bytes);
void check_transfer(const HeapLayout& layout, int slot, uint64_t offset, uint64_t bytes, bool allow_table);

}  // namespace lrm
