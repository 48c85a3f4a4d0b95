// The reference catalog's kernels 0..13 (docs/contracts/kernel-abi.md "The catalog at contracts-v1") for gfx950:
// fp32 activations, bf16 weights, the arithmetic of CpuRef F32 where the catalog asks for it. These are the parity
// path of the device (the executor's fp32 mode); the bf16 performance kernels are in kernels_fast.hip.
//
// Built with -ffp-contract=off: every product is rounded before the following add unless fmaf is written, as CpuRef
// does (docs/contracts/cpu-reference.md rules 2 and 4). Division and sqrtf are IEEE (hipcc's default
// -fhip-fp32-correctly-rounded-divide-sqrt).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>

#include "device.hpp"

namespace lrm {

static __device__ __forceinline__ float widen(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }
static __device__ __forceinline__ uint32_t linear_group() { return blockIdx.y * gridDim.x + blockIdx.x; }

// ---------------------------------------------------------------- 0 scale_f32: y[i] = a * x[i]
__global__ void k_scale_f32(const float* x, float* y, uint32_t n, float a) {
    uint32_t i = linear_group() * 256u + threadIdx.x;
    if (i >= n) return;
    y[i] = a * x[i];
}

// ---------------------------------------------------------------- 1 table_echo: the 16 words of a table row
__global__ void k_table_echo(const uint32_t* row, uint32_t* y) {
    uint32_t t = threadIdx.x;
    if (t < 16) y[t] = row[t];
}

// ---------------------------------------------------------------- 2 args_echo: all 32 argument words
struct Words32 {
    uint32_t w[32];
};
__global__ void k_args_echo(Words32 a, uint32_t* y) {
    uint32_t t = threadIdx.x;
    if (t < 32) y[t] = a.w[t];
}

// ---------------------------------------------------------------- 3 groups_echo: logical group g writes g
__global__ void k_groups_echo(uint32_t* y, uint32_t groups) {
    uint32_t g = linear_group();
    if (g < groups) y[g] = g;
}

// ---------------------------------------------------------------- 4 bf16_unpack
__global__ void k_bf16_unpack(const uint16_t* x, float* y, uint32_t n) {
    uint32_t i = linear_group() * 256u + threadIdx.x;
    if (i >= n) return;
    y[i] = widen(x[i]);
}

// ---------------------------------------------------------------- 5 embed_gather_bf16
__global__ void k_embed_gather(const uint32_t* ids, const uint16_t* table, float* y, uint32_t rows, uint32_t cols,
                               uint32_t vocab) {
    uint32_t r = blockIdx.y, c = blockIdx.x * 256u + threadIdx.x;
    if (r >= rows || c >= cols) return;
    uint32_t id = ids[r];
    y[size_t(r) * cols + c] = id < vocab ? widen(table[size_t(id) * cols + c]) : __uint_as_float(0x7FC00000u);
}

// Block reductions over 256 threads (4 waves of 64).
static __device__ __forceinline__ float block_sum_256(float v, float* red) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    return s;
}

// ---------------------------------------------------------------- 6 rmsnorm_rows
// y = widen(w) * (x * r), r = 1 / sqrt(sum(x^2) / cols + eps); per-thread fused partial sums, a fixed tree after.
__global__ void k_rmsnorm_rows(const float* x, const uint16_t* w, float* y, uint32_t rows, uint32_t cols, float eps) {
    __shared__ float red[4];
    uint32_t r = linear_group();
    if (r >= rows) return;
    const float* xr = x + size_t(r) * cols;
    float ss = 0.f;
    for (uint32_t c = threadIdx.x; c < cols; c += 256u) ss = fmaf(xr[c], xr[c], ss);
    ss = block_sum_256(ss, red);
    float mean = ss / float(cols);
    float rr = 1.0f / sqrtf(mean + eps);
    float* yr = y + size_t(r) * cols;
    for (uint32_t c = threadIdx.x; c < cols; c += 256u) {
        float xv = xr[c] * rr;
        yr[c] = widen(w[c]) * xv;
    }
}

// ---------------------------------------------------------------- 7 rope_apply (table driven, NeoX rotate-half)
__global__ void k_rope_apply(const float* x, const float* cos_t, const float* sin_t, float* y, uint32_t rows,
                             uint32_t heads, uint32_t hd, uint32_t pos0) {
    uint32_t r = linear_group();
    if (r >= rows) return;
    uint32_t half = hd / 2u;
    size_t pos = size_t(pos0) + r / heads;
    const float* xr = x + size_t(r) * hd;
    float* yr = y + size_t(r) * hd;
    for (uint32_t i = threadIdx.x; i < half; i += 64u) {
        float c = cos_t[pos * half + i], s = sin_t[pos * half + i];
        float a = xr[i], b = xr[i + half];
        float ac = a * c, bs = b * s, bc = b * c, as = a * s;
        yr[i] = ac - bs;
        yr[i + half] = bc + as;
    }
}

// ---------------------------------------------------------------- 8 silu_mul: y = (g / (1 + exp(-g))) * u
__global__ void k_silu_mul(const float* g, const float* u, float* y, uint32_t n) {
    uint32_t i = linear_group() * 256u + threadIdx.x;
    if (i >= n) return;
    float gv = g[i], uv = u[i];
    float den = 1.0f + expf(-gv);
    float s = gv / den;
    y[i] = s * uv;
}

// ---------------------------------------------------------------- 9 add
__global__ void k_add(const float* a, const float* b, float* y, uint32_t n) {
    uint32_t i = linear_group() * 256u + threadIdx.x;
    if (i >= n) return;
    y[i] = a[i] + b[i];
}

// ---------------------------------------------------------------- 10 copy_rows (4-byte elements)
__global__ void k_copy_rows(const uint32_t* src, uint32_t* dst, uint32_t rows, uint32_t cols, uint32_t sr0,
                            uint32_t dr0, uint32_t ss, uint32_t ds) {
    uint64_t e = uint64_t(linear_group()) * 256u + threadIdx.x;
    if (e >= uint64_t(rows) * cols) return;
    uint32_t r = uint32_t(e / cols), c = uint32_t(e % cols);
    dst[(uint64_t(dr0) + r) * ds + c] = src[(uint64_t(sr0) + r) * ss + c];
}

// ---------------------------------------------------------------- 11 argmax_rows
// The lowest index of the row maximum by '>' (+0 and -0 tie); a row holding a NaN gives 0xFFFFFFFF.
__global__ void k_argmax_rows(const float* x, uint32_t* y, uint32_t rows, uint32_t cols) {
    __shared__ float sv[256];
    __shared__ uint32_t si[256];
    __shared__ int snan;
    uint32_t r = linear_group();
    if (r >= rows) return;
    if (threadIdx.x == 0) snan = 0;
    __syncthreads();
    const float* xr = x + size_t(r) * cols;
    float best = 0.f;
    uint32_t bi = 0xFFFFFFFFu;
    bool nan = false;
    for (uint32_t c = threadIdx.x; c < cols; c += 256u) {
        float v = xr[c];
        if (v != v) nan = true;
        else if (bi == 0xFFFFFFFFu || v > best) {
            best = v;
            bi = c;
        }
    }
    if (nan) atomicOr(&snan, 1);
    sv[threadIdx.x] = best;
    si[threadIdx.x] = bi;
    __syncthreads();
    for (uint32_t s = 128; s > 0; s >>= 1) {
        if (threadIdx.x < s) {
            float ov = sv[threadIdx.x + s];
            uint32_t oi = si[threadIdx.x + s];
            uint32_t mi = si[threadIdx.x];
            if (oi != 0xFFFFFFFFu && (mi == 0xFFFFFFFFu || ov > sv[threadIdx.x] || (ov == sv[threadIdx.x] && oi < mi))) {
                sv[threadIdx.x] = ov;
                si[threadIdx.x] = oi;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) y[r] = snan ? 0xFFFFFFFFu : si[0];
}

// ---------------------------------------------------------------- 12 matmul_bf16w
// y[i, j] = sum_p fma(x[i, p], widen(w[j, p]), .) from +0 in increasing p: the same chain as CpuRef F32, so the result
// equals CpuRef's bit for bit and is the same for every m (no split-K, no m-dependent path). A block computes a
// 16 x 64 tile: thread t owns column t % 64 and rows 4 (t / 64) .. 4 (t / 64) + 3, with k staged 64 at a time.
constexpr int MM_TM = 16, MM_TN = 64, MM_KS = 64;
__global__ __launch_bounds__(256) void k_matmul_bf16w(const float* x, const uint16_t* w, float* y, uint32_t m,
                                                      uint32_t n, uint32_t k) {
    __shared__ float xs[MM_TM][MM_KS];
    __shared__ float ws[MM_TN][MM_KS + 1];
    const uint32_t t = threadIdx.x, col = t % 64u, rg = t / 64u;
    const uint32_t j0 = blockIdx.x * MM_TN, i0 = blockIdx.y * MM_TM;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (uint32_t p0 = 0; p0 < k; p0 += MM_KS) {
        uint32_t ks = k - p0 < uint32_t(MM_KS) ? k - p0 : uint32_t(MM_KS);
        for (uint32_t e = t; e < uint32_t(MM_TM * MM_KS); e += 256u) {
            uint32_t r = e / MM_KS, p = e % MM_KS;
            xs[r][p] = (i0 + r < m && p < ks) ? x[size_t(i0 + r) * k + p0 + p] : 0.f;
        }
        for (uint32_t e = t; e < uint32_t(MM_TN * MM_KS); e += 256u) {
            uint32_t c = e / MM_KS, p = e % MM_KS;
            ws[c][p] = (j0 + c < n && p < ks) ? widen(w[size_t(j0 + c) * k + p0 + p]) : 0.f;
        }
        __syncthreads();
        for (uint32_t p = 0; p < ks; ++p) {
            float wv = ws[col][p];
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[r] = fmaf(xs[rg * 4 + r][p], wv, acc[r]);
        }
        __syncthreads();
    }
    if (j0 + col < n)
        for (int r = 0; r < 4; ++r)
            if (i0 + rg * 4 + r < m) y[size_t(i0 + rg * 4 + r) * n + j0 + col] = acc[r];
}

// ---------------------------------------------------------------- 13 attention_gqa_causal
// One 64-thread group per (query row, q head), as the catalog grid. Keys in blocks of 64 anchored at position 0, the
// causal mask as the loop bound; thread t scores key j0 + t with a sequential fused dot in increasing d (CpuRef's
// order), times scale. Online softmax per block: m = the first block's maximum, then m' = max(m, block max),
// alpha = exp(m - m'), weights e = exp(s - m'), block sum and block values summed in increasing j from +0, then
// l = fma(l, alpha, sum) and o = fma(o, alpha, value); y = o / l at the end. Output dimensions in passes of 256
// (4 per thread); each pass recomputes the same scores with the same instructions.
constexpr int ATT_MAX_HD = 1024;
__global__ __launch_bounds__(64) void k_attention_f32(const float* q, const float* kc, const float* vc, float* y,
                                                      uint32_t rows, uint32_t q_row0, uint32_t past, uint32_t qh,
                                                      uint32_t kvh, uint32_t hd, float scale) {
    __shared__ float qs[ATT_MAX_HD];
    __shared__ float sc[64];
    __shared__ float wt[64];
    if (blockIdx.x >= rows || blockIdx.y >= qh) return;
    const uint32_t i = rows - 1u - blockIdx.x, h = blockIdx.y, t = threadIdx.x;
    const uint32_t kvhead = h / (qh / kvh);
    const uint32_t keys = past + i + 1u;
    const size_t kv_stride = size_t(kvh) * hd;
    const size_t qbase = (size_t(q_row0 + i) * qh + h) * hd;
    for (uint32_t d = t; d < hd; d += 64u) qs[d] = q[qbase + d];
    __syncthreads();
    for (uint32_t d0 = 0; d0 < hd; d0 += 256u) {
        float m = 0.f, l = 0.f;
        float o[4] = {0.f, 0.f, 0.f, 0.f};
        for (uint32_t j0 = 0; j0 < keys; j0 += 64u) {
            uint32_t count = keys - j0 < 64u ? keys - j0 : 64u;
            float s = 0.f;
            if (t < count) {
                const float* kr = kc + size_t(j0 + t) * kv_stride + size_t(kvhead) * hd;
                float acc = 0.f;
                for (uint32_t d = 0; d < hd; ++d) acc = fmaf(qs[d], kr[d], acc);
                s = acc * scale;
            }
            sc[t] = s;
            __syncthreads();
            float bmax = sc[0];
            for (uint32_t jm = 1; jm < count; ++jm) bmax = fmaxf(bmax, sc[jm]);
            if (j0 == 0) m = bmax;
            float mn = fmaxf(m, bmax);
            float alpha = expf(m - mn);
            m = mn;
            wt[t] = t < count ? expf(s - mn) : 0.f;
            __syncthreads();
            float bsum = 0.f;
            float acc[4] = {0.f, 0.f, 0.f, 0.f};
            for (uint32_t j = 0; j < count; ++j) {
                float e = wt[j];
                bsum += e;
                const float* vr = vc + size_t(j0 + j) * kv_stride + size_t(kvhead) * hd;
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    uint32_t d = d0 + t + 64u * u;
                    if (d < hd) acc[u] = fmaf(e, vr[d], acc[u]);
                }
            }
            l = fmaf(l, alpha, bsum);
#pragma unroll
            for (int u = 0; u < 4; ++u) o[u] = fmaf(o[u], alpha, acc[u]);
            __syncthreads();
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            uint32_t d = d0 + t + 64u * u;
            if (d < hd) y[qbase + d] = o[u] / l;
        }
    }
}

// ---------------------------------------------------------------- launchers

static float f32_of(uint32_t b) {
    float f;
    std::memcpy(&f, &b, 4);
    return f;
}

static dim3 phys(const PreparedDispatch& pd) { return dim3(pd.physical.x, pd.physical.y, pd.physical.z); }

static void l_scale(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    hipLaunchKernelGGL(k_scale_f32, phys(pd), dim3(256), 0, s, (const float*)p[0], (float*)p[1], pd.words[3], f32_of(pd.words[4]));
}
static void l_table_echo(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    hipLaunchKernelGGL(k_table_echo, phys(pd), dim3(16), 0, s, (const uint32_t*)p[0], (uint32_t*)p[1]);
}
static void l_args_echo(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    Words32 a;
    std::memcpy(a.w, pd.words.data(), 128);
    hipLaunchKernelGGL(k_args_echo, phys(pd), dim3(32), 0, s, a, (uint32_t*)p[0]);
}
static void l_groups_echo(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    hipLaunchKernelGGL(k_groups_echo, phys(pd), dim3(1), 0, s, (uint32_t*)p[0], pd.words[2]);
}
static void l_bf16_unpack(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    hipLaunchKernelGGL(k_bf16_unpack, phys(pd), dim3(256), 0, s, (const uint16_t*)p[0], (float*)p[1], pd.words[3]);
}
static void l_embed(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    hipLaunchKernelGGL(k_embed_gather, phys(pd), dim3(256), 0, s, (const uint32_t*)p[0], (const uint16_t*)p[1],
                       (float*)p[2], pd.words[4], pd.words[5], pd.words[6]);
}
static void l_rmsnorm(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    hipLaunchKernelGGL(k_rmsnorm_rows, phys(pd), dim3(256), 0, s, (const float*)p[0], (const uint16_t*)p[1],
                       (float*)p[2], pd.words[4], pd.words[5], f32_of(pd.words[6]));
}
static void l_rope(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    hipLaunchKernelGGL(k_rope_apply, phys(pd), dim3(64), 0, s, (const float*)p[0], (const float*)p[1],
                       (const float*)p[2], (float*)p[3], pd.words[5], pd.words[6], pd.words[7], pd.words[8]);
}
static void l_silu(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    hipLaunchKernelGGL(k_silu_mul, phys(pd), dim3(256), 0, s, (const float*)p[0], (const float*)p[1], (float*)p[2], pd.words[4]);
}
static void l_add(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    hipLaunchKernelGGL(k_add, phys(pd), dim3(256), 0, s, (const float*)p[0], (const float*)p[1], (float*)p[2], pd.words[4]);
}
static void l_copy_rows(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    hipLaunchKernelGGL(k_copy_rows, phys(pd), dim3(256), 0, s, (const uint32_t*)p[0], (uint32_t*)p[1], pd.words[3],
                       pd.words[4], pd.words[5], pd.words[6], pd.words[7], pd.words[8]);
}
static void l_argmax(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    hipLaunchKernelGGL(k_argmax_rows, phys(pd), dim3(256), 0, s, (const float*)p[0], (uint32_t*)p[1], pd.words[3], pd.words[4]);
}
static void l_matmul(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    uint32_t m = pd.words[4], n = pd.words[5], k = pd.words[6];
    dim3 grid((n + MM_TN - 1) / MM_TN, (m + MM_TM - 1) / MM_TM);
    hipLaunchKernelGGL(k_matmul_bf16w, grid, dim3(256), 0, s, (const float*)p[0], (const uint16_t*)p[1], (float*)p[2], m, n, k);
}
static void l_attention(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    uint32_t hd = pd.words[10];
    if (hd > uint32_t(ATT_MAX_HD)) contract_fail("attention_gqa_causal: this device supports head_dim up to %d", ATT_MAX_HD);
    hipLaunchKernelGGL(k_attention_f32, dim3(pd.words[5], pd.words[8]), dim3(64), 0, s, (const float*)p[0],
                       (const float*)p[1], (const float*)p[2], (float*)p[3], pd.words[5], pd.words[6], pd.words[7],
                       pd.words[8], pd.words[9], hd, f32_of(pd.words[11]));
}

const LaunchFn* catalog_launchers() {
    static const LaunchFn t[14] = {l_scale,  l_table_echo, l_args_echo, l_groups_echo, l_bf16_unpack,
                                   l_embed,  l_rmsnorm,    l_rope,      l_silu,        l_add,
                                   l_copy_rows, l_argmax,  l_matmul,    l_attention};
    return t;
}

}  // namespace lrm
