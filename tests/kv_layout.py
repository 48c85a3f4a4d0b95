"""The fast path's fp16 V cache layout, for tests that build or read the cache themselves: per KV head, max_pos / 64
blocks of 64 positions, each a [128 dims][64 positions] tile (rosylnalive_amd/csrc/kv_layout.hpp)."""
import numpy as np


def v_block(vt):
    """[kv_heads, 128, max_pos] (a head's V transposed: dims x positions) -> the cache layout
    [kv_heads, max_pos / 64, 128, 64]."""
    kvh, hd, mp = vt.shape
    assert hd == 128 and mp % 64 == 0
    return np.ascontiguousarray(vt.reshape(kvh, hd, mp // 64, 64).transpose(0, 2, 1, 3))


def v_unblock(vb, kv_heads, max_pos):
    """The cache layout (any array of kv_heads * max_pos * 128 elements in that order) -> [kv_heads, 128, max_pos]."""
    return np.ascontiguousarray(np.asarray(vb).reshape(kv_heads, max_pos // 64, 128, 64).transpose(0, 2, 1, 3)
                                .reshape(kv_heads, 128, max_pos))
