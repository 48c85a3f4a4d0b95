// The validating safetensors reader (SafetensorsFile, src/Lrm.Tensor/Safetensors.fs:290-727): an 8-byte little-endian
// header length N, N bytes of UTF-8 JSON {name: {dtype, shape, data_offsets}, "__metadata__": {key: string}}, then the
// data section, which the tensors must tile exactly. Open maps the file read-only and checks everything before it
// returns, so a caller only ever sees a well-formed file.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace lrm {

// A file that breaks the format rules (SafetensorsFormatException, Safetensors.fs:15-17).
struct FormatError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

// A file whose size or SHA-256 differs from the value it is pinned to (IntegrityException, Safetensors.fs:20-34).
struct IntegrityError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

struct StEntry {
    std::string name;            // UTF-8
    uint32_t dtype;              // DType code (contract.hpp)
    std::vector<int64_t> shape;  // rank 0 = scalar
    int64_t begin, end;          // byte offsets in the data section, end exclusive
    int64_t bytes() const { return end - begin; }
};

struct StHeader {
    int64_t header_length = 0;
    std::vector<std::pair<std::string, std::string>> metadata;  // in code point order of the keys
    std::vector<StEntry> entries;                                // in code point order of the names
};

// The largest header the reader accepts (Safetensors.MaxHeaderBytes, Safetensors.fs:86-88).
constexpr int64_t kMaxHeaderBytes = 100000000;

// Validates the first bytes of a file of `length` bytes (SafetensorsParse.header, Safetensors.fs:401-498). `head`
// holds at least min(length, 8 + N) bytes of it. Throws FormatError.
StHeader st_validate(const uint8_t* head, uint64_t head_bytes, uint64_t length);

// The safetensors dtype string of a DType code ("F32", "BF16", ...), or nullptr.
const char* st_dtype_name(uint32_t dtype);

class StFile {
  public:
    // Maps `path` read-only and validates it (SafetensorsFile.Open). With expect_bytes >= 0 and expect_sha256 (64 hex
    // digits) the size and the SHA-256 of the mapped bytes are checked first (OpenVerified): IntegrityError.
    static std::unique_ptr<StFile> open(const std::string& path, int64_t expect_bytes = -1,
                                        const char* expect_sha256 = nullptr);
    // Validates bytes held in memory (SafetensorsFile.Validate); the bytes are copied.
    static std::unique_ptr<StFile> from_memory(const uint8_t* bytes, uint64_t n);
    ~StFile();
    StFile(const StFile&) = delete;
    StFile& operator=(const StFile&) = delete;

    const std::string& path() const { return path_; }
    uint64_t length() const { return length_; }
    int64_t header_length() const { return header_.header_length; }
    int64_t data_offset() const { return 8 + header_.header_length; }
    const std::vector<StEntry>& entries() const { return header_.entries; }
    const std::vector<std::pair<std::string, std::string>>& metadata() const { return header_.metadata; }
    // The data section starts at a multiple of 8 and every tensor at a multiple of its element size (IsAligned).
    bool aligned() const;
    const StEntry* find(const std::string& name) const;
    // The tensor's bytes in the mapping (valid while the file is open).
    const uint8_t* data(const StEntry& e) const { return base_ + data_offset() + e.begin; }
    const uint8_t* bytes() const { return base_; }

  private:
    StFile() = default;
    std::string path_;
    const uint8_t* base_ = nullptr;
    uint64_t length_ = 0;
    bool mapped_ = false;
    std::vector<uint8_t> owned_;
    StHeader header_;
    std::map<std::string, size_t> index_;
};

}  // namespace lrm
