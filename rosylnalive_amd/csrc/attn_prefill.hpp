// Workspace of the causal prefill attention (attention_prefill_f16 in kernels_fast.hip), shared by the kernel, its
// contract and the executor that sizes the buffer.
#pragma once

#include <cstdint>

namespace lrm {
namespace attn_prefill {

constexpr int kRows = 32;                   // query rows of a tile
constexpr int kSlotWords = 8192 + 256;      // one partial of a split tile: O^T (2 heads x 64 lanes x 64), then m, l
// One record of u32 words per (KV head, tile pair): the pair's counter (padded to 256 bytes), then the partials of
// its two parts. Record p sits at p * kRecordWords whatever the row count, so launches of different lengths share
// one buffer: counters are never overwritten by partials. The counters must be zero before the first launch; every
// launch leaves them zero.
constexpr int kRecordWords = 64 + 2 * kSlotWords;
constexpr int64_t pairs(int64_t rows) { return ((rows + kRows - 1) / kRows) / 2; }
constexpr int64_t workspace_words(int64_t rows, int64_t kv_heads) {
    return (kv_heads * pairs(rows) > 0 ? kv_heads * pairs(rows) : 1) * kRecordWords;
}

}  // namespace attn_prefill
}  // namespace lrm
