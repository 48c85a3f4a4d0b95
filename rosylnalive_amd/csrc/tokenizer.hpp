// The Qwen3 byte-level BPE tokenizer (QwenTokenizer, src/Lrm.Tokenizer/QwenTokenizer.fs): added tokens matched on the
// raw text (leftmost-longest), then for each stretch between them the oracle's NFC, the Split pre-tokenizer and
// byte-level BPE over merge ranks. No BOS or EOS is added. Built from tokenizer.json bytes with the reference
// loader's checks (TokenizerJson.fs): only the configuration Qwen3 uses is accepted. An instance is immutable, so every
// member may be called from many threads at once.
#pragma once

#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

namespace lrm {
namespace tok {

// tokenizer.json holds a configuration this tokenizer does not run (InvalidDataException, TokenizerJson.fs:24-25).
struct DataError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

// The class of a scalar in the Split regex (CharClass.fs:7-20).
enum CharClass : uint8_t { kLetter = 0, kNumber = 1, kSpace = 2, kOther = 3 };
CharClass char_class(uint32_t cp);
// The letter a scalar matches in the case-insensitive contraction group, or 0 (CharClass.contractionLetter).
char contraction_letter(uint32_t cp);

// UTF-8 -> scalars. Strict: false at the first ill-formed sequence (its byte offset in *bad). Replacing: one U+FFFD
// per maximal ill-formed subpart (the Unicode standard's practice, as Python's errors="replace").
bool utf8_decode(const uint8_t* s, size_t n, std::u32string& out, size_t* bad);
std::u32string utf8_decode_replace(const uint8_t* s, size_t n);
std::string utf8_encode(const std::u32string& s);

// The oracle's NFC (Nfc.fs): NFC with Unicode 13.0 data, split at the scalars the oracle's Unicode 9.0 tables leave
// inert but a newer Unicode does not (and at U+FFFE); the split scalars stay as they are.
std::u32string nfc(const std::u32string& s);
bool nfc_split_point(uint32_t cp);

// The Split pre-tokenizer (PreTokenizer.fs): piece boundaries [b[i], b[i + 1]) in scalars, b[0] = 0, b.back() = n.
std::vector<size_t> pre_split(const std::u32string& s);

// GPT-2's byte map (ByteLevel.fs): the character that stands for byte b, and back (-1 for other characters).
uint32_t byte_char(uint8_t b);
int char_byte(uint32_t c);

struct AddedToken {
    int32_t id;
    std::u32string content;
    bool special;
};

class Tokenizer {
  public:
    // The rows of Qwen3's embedding and lm_head (config.json vocab_size): ids from vocab_size() up to here decode to
    // nothing, ids outside [0, kModelRows) are refused (QwenTokenizer.ModelRows).
    static constexpr int32_t kModelRows = 151936;

    static std::unique_ptr<Tokenizer> parse(const uint8_t* json, size_t n);  // throws DataError

    // The ids of `text` (Encode); text must be valid UTF-8, the analogue of the reference's refusal of a lone
    // surrogate (std::invalid_argument naming the byte).
    std::vector<int32_t> encode(const uint8_t* utf8, size_t n) const;
    // EncodeBytes: ill-formed UTF-8 replaced first.
    std::vector<int32_t> encode_bytes(const uint8_t* bytes, size_t n) const;
    std::vector<int32_t> encode_scalars(const std::u32string& text) const;
    // DecodeBytes: each vocabulary token's bytes, an added token's content as the ByteLevel decoder gives it, nothing
    // for ids in [vocab_size(), kModelRows); std::out_of_range for other ids.
    std::string decode_bytes(const int32_t* ids, size_t n) const;

    int32_t vocab_size() const { return int32_t(token_bytes_.size() + added_.size()); }
    int32_t merge_count() const { return int32_t(merges_.size()); }
    const std::vector<AddedToken>& added() const { return added_; }
    // IdOf: an added token's content or a vocabulary token in its byte-level form (UTF-8), or -1.
    int32_t id_of(const std::string& token_utf8) const;
    // TokenOf: the byte-level vocabulary string or the added token's content (UTF-8); false for other ids.
    bool token_of(int32_t id, std::string& out) const;

  private:
    Tokenizer() = default;
    void encode_piece(const std::u32string& s, size_t b, size_t e, std::vector<int32_t>& out) const;
    std::vector<std::string> token_bytes_;     // bytes of vocabulary id i
    std::vector<std::string> token_strings_;   // byte-level string of id i (UTF-8)
    int32_t byte_ids_[256] = {};
    std::unordered_map<uint64_t, uint64_t> merges_;  // (left << 32 | right) -> (rank << 32 | merged id)
    std::unordered_map<std::string, int32_t> vocab_;  // byte-level string (UTF-8) -> id
    std::vector<AddedToken> added_;
    std::unordered_map<std::string, int32_t> added_by_content_;  // UTF-8 content -> id
    struct TrieNode {
        std::unordered_map<uint32_t, int32_t> next;
        int32_t id = -1;
    };
    std::vector<TrieNode> trie_;
};

}  // namespace tok
}  // namespace lrm
