// Layout of the fast path's fp16 V cache, shared by its kernels and the executor that reads and writes it.
#pragma once

#include <cstddef>

namespace lrm {
namespace kv {

// A KV head's V cache holds max_pos x 128 halves as max_pos / 64 blocks of 64 positions, each block a [128 dims][64
// positions] tile (16 KiB, contiguous): element (pos, dim) at (pos / 64) 8192 + dim 64 + pos % 64. The prefill
// attention's O^T = V^T P^T takes its A operand from such a tile, and a decode split streams whole blocks, so every
// read of a 64-key block is one contiguous 16 KiB (a [128][max_pos] transpose made it 128 pieces of 128 bytes,
// max_pos x 2 bytes apart). max_pos is a multiple of 64 wherever this layout is used.
constexpr int kVBlock = 64;
constexpr size_t kVBlockHalves = size_t(kVBlock) * 128;

constexpr size_t v_at(int pos, int dim) {
    return size_t(unsigned(pos) / unsigned(kVBlock)) * kVBlockHalves + size_t(dim) * kVBlock +
           size_t(unsigned(pos) % unsigned(kVBlock));
}

}  // namespace kv
}  // namespace lrm
