// Device helpers shared by the bf16 fast-path kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace lrm {
namespace fast {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }

// Round to nearest even; a NaN narrows to 7fc0 / ffc0 by its sign (Bf16.narrowRne, src/Lrm.Core/Numerics.fs:35-45).
__device__ __forceinline__ uint16_t f2bf(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u & 0x80000000u) ? 0xFFC0 : 0x7FC0;
    return uint16_t((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ uint32_t pack2(float a, float b) { return uint32_t(f2bf(a)) | (uint32_t(f2bf(b)) << 16); }

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

// The 8 bf16 of a uint4 widened to float.
__device__ __forceinline__ void unpack8(uint4 v, float* f) {
    f[0] = __uint_as_float(v.x << 16);
    f[1] = __uint_as_float(v.x & 0xFFFF0000u);
    f[2] = __uint_as_float(v.y << 16);
    f[3] = __uint_as_float(v.y & 0xFFFF0000u);
    f[4] = __uint_as_float(v.z << 16);
    f[5] = __uint_as_float(v.z & 0xFFFF0000u);
    f[6] = __uint_as_float(v.w << 16);
    f[7] = __uint_as_float(v.w & 0xFFFF0000u);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Loads that bypass the non-coherent per-CU cache: for data another workgroup of the same launch wrote and published
// through a device-scope release (the last-arriving workgroup's fix-up step).
__device__ __forceinline__ float load_coherent(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t load_coherent_u32(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Arrival counter of a fix-up: every workgroup publishes its results (release) and increments; the one that sees
// `expected - 1` is last, acquires, and resets the counter to 0 for the next launch (graph replays reuse it).
// Every thread fences its own stores at device scope before the barrier: a fence only orders the issuing wave's
// stores, and on a chip with one L2 per XCD the device-scope release is what writes them back for other XCDs.
__device__ __forceinline__ bool arrive_last(uint32_t* counter, uint32_t expected, int* flag_lds) {
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t old = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        int last = old == expected - 1u;
        if (last) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *flag_lds = last;
    }
    __syncthreads();
    bool last = *flag_lds != 0;
    if (last) __threadfence();
    return last;
}

}  // namespace fast
}  // namespace lrm
