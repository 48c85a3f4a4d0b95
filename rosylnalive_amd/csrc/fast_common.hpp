// Device helpers shared by the bf16 fast-path kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace lrm {
namespace fast {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
// A native 16-byte vector for staging loads and LDS traffic (HIP's uint4 is a union-based struct that the
// optimiser can fail to keep in registers).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }

// Round to nearest even; a NaN narrows to 7fc0 / ffc0 by its sign (Bf16.narrowRne, src/Lrm.Core/Numerics.fs:35-45).
__device__ __forceinline__ uint16_t f2bf(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u & 0x80000000u) ? 0xFFC0 : 0x7FC0;
    return uint16_t((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ uint32_t pack2(float a, float b) { return uint32_t(f2bf(a)) | (uint32_t(f2bf(b)) << 16); }

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }
__device__ __forceinline__ f16x8 as_f16x8(uint4 v) { return __builtin_bit_cast(f16x8, v); }
__device__ __forceinline__ f16x8 as_f16x8(u32x4 v) { return __builtin_bit_cast(f16x8, v); }

// IEEE half: round to nearest even (hardware conversion), and exact widening.
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f)); }
__device__ __forceinline__ float h2f(uint16_t h) { return static_cast<float>(__builtin_bit_cast(_Float16, h)); }
// Two floats to an fp16 pair, round to nearest even (one v_cvt_pk_f16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack2h(float a, float b) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    typedef float f2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){a, b}, h2));
}

// The 8 halves of a uint4 (or u32x4) widened to float.
__device__ __forceinline__ void unpack8h(uint4 v, float* f) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[2 * i] = h2f(uint16_t(w[i] & 0xFFFFu));
        f[2 * i + 1] = h2f(uint16_t(w[i] >> 16));
    }
}
__device__ __forceinline__ void unpack8h(u32x4 v, float* f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[2 * i] = h2f(uint16_t(v[i] & 0xFFFFu));
        f[2 * i + 1] = h2f(uint16_t(v[i] >> 16));
    }
}

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

// A workgroup barrier for LDS traffic only: this wave's LDS operations complete (lgkmcnt(0)), then s_barrier. Unlike
// __syncthreads() it does not wait for outstanding global loads (gfx9 counts loads and stores in one counter, so the
// release fence would drain prefetches still in flight). The empty asm statements keep the compiler from moving
// memory operations across it.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // vmcnt and expcnt at their maxima (no wait), lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Cross-lane reductions without an LDS round trip: DPP moves inside each 16-lane row (quad_perm [1,0,3,2] and
// [2,3,0,1], row_half_mirror, row_mirror), then the gfx950 row swaps (v_permlane16_swap, v_permlane32_swap) across the
// four rows. Every step adds a lane's value to its partner's, so partners hold the same bits (a + b == b + a) and the
// result is identical in every lane of the group.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// the sum over lanes 4 (l / 4) .. + 3
__device__ __forceinline__ float quad4_sum(float v) {
    v += dpp_f<0xB1>(v);
    return v + dpp_f<0x4E>(v);
}

// the sum over the 16 lanes of the row of lane l (lanes 16 (l / 16) .. + 15)
__device__ __forceinline__ float row_sum16(float v) {
    v = quad4_sum(v);
    v += dpp_f<0x141>(v);
    return v + dpp_f<0x140>(v);
}

__device__ __forceinline__ float row_max16(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    return fmaxf(v, dpp_f<0x140>(v));
}

// the sum / maximum over the four rows of lanes that share l % 16
__device__ __forceinline__ float cross_rows_sum(float v) {
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
__device__ __forceinline__ float cross_rows_max(float v) {
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float wave_sum(float v) { return cross_rows_sum(row_sum16(v)); }

// The wave sums of R = 2, 4 or 8 values per lane at once (row k = v[k] over the 64 lanes), each exchange step swapping
// half of the rows instead of reducing every row alone: with v_permlane32_swap(A = v[i], B = v[R/2 + i]) lanes 0-31
// get the upper lane's v[i] and lanes 32-63 the lower lane's v[R/2 + i], so the sum of the two results is row i's pair
// sum in the lower half and row R/2 + i's in the upper (R/2 swaps for R rows; v_permlane16_swap likewise across the
// 16-lane rows, then one row_mirror exchange for R = 8). Returns row k's sum in lanes (64 / R) k .. + 64 / R - 1, the
// same bits in each of them.
template <int R>
__device__ __forceinline__ float wave_sum_rows(const float (&v)[R]) {
    static_assert(R == 2 || R == 4 || R == 8, "2, 4 or 8 rows");
    float a[R / 2];
#pragma unroll
    for (int i = 0; i < R / 2; ++i) {
        const auto x = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[i]), __float_as_uint(v[R / 2 + i]), false,
                                                        false);
        a[i] = __uint_as_float(x[0]) + __uint_as_float(x[1]);
    }
    if constexpr (R == 2) {
        return row_sum16(
            [&] {
                const auto x = __builtin_amdgcn_permlane16_swap(__float_as_uint(a[0]), __float_as_uint(a[0]), false,
                                                                false);
                return __uint_as_float(x[0]) + __uint_as_float(x[1]);
            }());
    } else {
        float b[R / 4];
#pragma unroll
        for (int i = 0; i < R / 4; ++i) {
            const auto x = __builtin_amdgcn_permlane16_swap(__float_as_uint(a[i]), __float_as_uint(a[R / 4 + i]), false,
                                                            false);
            b[i] = __uint_as_float(x[0]) + __uint_as_float(x[1]);
        }
        if constexpr (R == 4) {
            return row_sum16(b[0]);
        } else {
            // lanes 0-7 of a 16-lane row keep b[0] and take b[0] of lane 15 - l; lanes 8-15 keep b[1] and take b[1]
            const bool hi = (threadIdx.x & 8) != 0;
            float c = (hi ? b[1] : b[0]) + dpp_f<0x140>(hi ? b[0] : b[1]);
            c += dpp_f<0xB1>(c);
            c += dpp_f<0x4E>(c);
            return c + dpp_f<0x141>(c);
        }
    }
}

__device__ __forceinline__ float wave_max(float v) { return cross_rows_max(row_max16(v)); }

// ---------------------------------------------------------------- the fp16 range monitor
// The fast path narrows some activations and the K/V cache to fp16, whose range ends at 65,504: a value the float32
// reference keeps (a SwiGLU outlier, a large projection) becomes inf there. Every kernel that stores such a value ORs
// the bit of its site into a sticky device word when a half it stores is inf or NaN; the executor reads and clears the
// word after each forward and decode run and fails the call with the sites named, instead of passing the inf on. The
// word starts at zero (static storage) and each code object including this header holds its own, one per GPU.
enum F16Site : uint32_t {
    kF16Hidden = 1u,  // RMSNorm output rows (the GEMM input h)
    kF16Query = 2u,   // q after its norm and RoPE
    kF16Cache = 4u,   // K or V cache entries
    kF16Attn = 8u,    // the attention output o
    kF16Swiglu = 16u  // the SwiGLU output a
};
static __device__ uint32_t f16_range_word;

// 1 when a half of the pair is inf or NaN (exponent field all ones)
__device__ __forceinline__ uint32_t f16_bad2(uint32_t p) {
    return uint32_t((p & 0x7C00u) == 0x7C00u) | uint32_t((p & 0x7C000000u) == 0x7C000000u);
}
__device__ __forceinline__ uint32_t f16_bad8(u32x4 v) {
    return f16_bad2(v[0]) | f16_bad2(v[1]) | f16_bad2(v[2]) | f16_bad2(v[3]);
}
// A vector atomic, issued only by the lanes that saw a bad value (none, on finite data).
__device__ __forceinline__ void f16_note(uint32_t bad, uint32_t site) {
    if (bad) __hip_atomic_fetch_or(&f16_range_word, site, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace fast
}  // namespace lrm
