// The fast path of the HIP device (appended catalog ids 14 and up), gfx950 (CDNA4) only, wave64.
//
// Precision. Weights are stored bf16 (the model's format); decode streams them as bf16 with fp32 arithmetic. The
// prefill matrix units take fp16 operands: an exact fp16 copy of each bf16 weight (|w| < 65536 is checked on upload;
// bf16 values below 2^-17 lose low bits as fp16 subnormals, an absolute change under 2^-25) and fp16-rounded
// activations, 11 mantissa bits against bf16's 8, accumulated in fp32. The KV cache is fp16: the same bytes as bf16
// with 8x less rounding error (K is RMS-normalised per head and V is a projection of a normalised row, so both stay
// far inside the fp16 range).
//
// Data layout in HBM (chosen by the executor, see qwen_exec.cpp):
//   residual stream x          f32  [T, hidden]
//   prefill GEMM inputs        f16  [T, k]           (k contiguous: the MFMA A operand)
//   weights                    bf16 [n, k] (PyTorch Linear) for decode, f16 copies for prefill; q|k|v rows fused into
//                              one [QC + 2 KC, hidden], gate|up rows fused into one [2 I, hidden]
//   K cache                    f16  [kv_heads, max_pos, head_dim]   (head-major: one head's keys are contiguous)
//   V cache                    f16  [kv_heads, max_pos / 64, head_dim, 64]   (64-position blocks, each transposed: the
//                              A operand of O^T = V^T P^T, and one contiguous 16 KiB per key block; kv_layout.hpp)
//
// MFMA: v_mfma_f32_16x16x32_f16. Operand layout (lane l, g = l / 16, c = l % 16): A supplies row c, k = 8g .. 8g + 7;
// B supplies column c, k = 8g .. 8g + 7; D holds rows 4g .. 4g + 3 of column c.
//
// No kernel here synchronises the workgroups of its own launch: each cross-workgroup reduction ends its kernel, and
// the next kernel on the stream reads the partial results (kernel boundaries are the device-wide ordering points).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>
#include <type_traits>

#include "device.hpp"
#include "attn_prefill.hpp"
#include "fast_common.hpp"
#include "kv_layout.hpp"
#include "persist.hpp"

namespace lrm {
using namespace fast;

static constexpr float kLog2e = 1.4426950408889634f;

// ================================================================ 14 rmsnorm_rows_f16
// y[r, :] = f16(widen(w) * (x[row0 + r, :] * r)), r = 1 / sqrt(sum(x^2) / cols + eps). One block per row.
__global__ __launch_bounds__(256) void k_rmsnorm_f16(const float* x, const uint16_t* w, uint16_t* y, uint32_t rows,
                                                     uint32_t cols, float eps, uint32_t row0) {
    __shared__ float red[4];
    uint32_t r = blockIdx.x;
    if (r >= rows) return;
    const float* xr = x + size_t(row0 + r) * cols;
    float ss = 0.f;
    for (uint32_t c = threadIdx.x; c < cols; c += 256u) ss = fmaf(xr[c], xr[c], ss);
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = (red[0] + red[1]) + (red[2] + red[3]);
    float rr = 1.0f / sqrtf(ss / float(cols) + eps);
    uint16_t* yr = y + size_t(r) * cols;
    uint32_t bad = 0;
    for (uint32_t c = threadIdx.x; c < cols; c += 256u) {
        const uint16_t h = f2h(bf2f(w[c]) * (xr[c] * rr));
        bad |= f16_bad2(h);
        yr[c] = h;
    }
    f16_note(bad, kF16Hidden);
}

// The same for cols = 256 NC (the model widths): one wave per row, four rows per block. Each lane loads its NC float4
// of the row (lane l: columns 4 l + 256 j) at once and keeps them, so the row is read once, the sum of squares is a
// wave reduction with no barrier, and the output goes out as 8-byte packs of four halves.
template <int NC>
__global__ __launch_bounds__(256) void k_rmsnorm_f16_wave(const float* x, const uint16_t* w, uint16_t* y,
                                                          uint32_t rows, uint32_t cols, float eps, uint32_t row0) {
    const uint32_t r = blockIdx.x * 4u + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (r >= rows) return;
    const float4* xr = reinterpret_cast<const float4*>(x + size_t(row0 + r) * cols) + lane;
    const uint2* wr = reinterpret_cast<const uint2*>(w) + lane;
    float4 v[NC];
    uint2 wv[NC];
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        v[j] = xr[64 * j];
        wv[j] = wr[64 * j];
    }
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NC; ++j) ss = fmaf(v[j].x, v[j].x, fmaf(v[j].y, v[j].y, fmaf(v[j].z, v[j].z, fmaf(v[j].w, v[j].w, ss))));
    ss = wave_sum(ss);
    const float rr = 1.0f / sqrtf(ss / float(cols) + eps);
    uint2* yr = reinterpret_cast<uint2*>(y + size_t(r) * cols) + lane;
    uint32_t bad = 0;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        const float w0 = __uint_as_float(wv[j].x << 16), w1 = __uint_as_float(wv[j].x & 0xFFFF0000u);
        const float w2 = __uint_as_float(wv[j].y << 16), w3 = __uint_as_float(wv[j].y & 0xFFFF0000u);
        const uint2 h = make_uint2(pack2h(w0 * (v[j].x * rr), w1 * (v[j].y * rr)), pack2h(w2 * (v[j].z * rr), w3 * (v[j].w * rr)));
        bad |= f16_bad2(h.x) | f16_bad2(h.y);
        yr[64 * j] = h;
    }
    f16_note(bad, kF16Hidden);
}

// ================================================================ 40 residual_add_norm
// x[r, :] += p[0][r, :] + p[1][r, :] + ... (the k-split partial products of gemm_residual_split, added in split order),
// then y[r, :] = f16(widen(w) * (x[r, :] * rr)) exactly as rmsnorm_rows_f16 forms it. One wave per row (cols = 256 NC),
// blockDim / 64 rows per block; the partial rows of two splits are loaded before their adds.
template <int NC>
__global__ __launch_bounds__(256) void k_resid_add_norm(float* x, const float* part, const uint16_t* w, uint16_t* y,
                                                        uint32_t rows, uint32_t cols, uint32_t splits, float eps) {
    const uint32_t r = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (r >= rows) return;
    float4* xr = reinterpret_cast<float4*>(x + size_t(r) * cols) + lane;
    const float4* pr = reinterpret_cast<const float4*>(part + size_t(r) * cols) + lane;
    const size_t ps = size_t(rows) * cols / 4;  // float4s from one split's partial to the next
    const uint2* wr = reinterpret_cast<const uint2*>(w) + lane;
    float4 v[NC], q[2][NC];
    uint2 wv[NC];
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        v[j] = xr[64 * j];
        wv[j] = wr[64 * j];
    }
    for (uint32_t k = 0; k < splits; k += 2) {  // two splits' rows in flight at a time (splits is 1 or even)
        const bool two = k + 1 < splits;
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            q[0][j] = pr[k * ps + 64 * j];
            q[1][j] = two ? pr[(k + 1) * ps + 64 * j] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int h = 0; h < 2; ++h)
            if (h == 0 || two)
#pragma unroll
                for (int j = 0; j < NC; ++j) {
                    v[j].x += q[h][j].x;
                    v[j].y += q[h][j].y;
                    v[j].z += q[h][j].z;
                    v[j].w += q[h][j].w;
                }
    }
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        xr[64 * j] = v[j];
        ss = fmaf(v[j].x, v[j].x, fmaf(v[j].y, v[j].y, fmaf(v[j].z, v[j].z, fmaf(v[j].w, v[j].w, ss))));
    }
    ss = wave_sum(ss);
    const float rr = 1.0f / sqrtf(ss / float(cols) + eps);
    uint2* yr = reinterpret_cast<uint2*>(y + size_t(r) * cols) + lane;
    uint32_t bad = 0;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        const float w0 = __uint_as_float(wv[j].x << 16), w1 = __uint_as_float(wv[j].x & 0xFFFF0000u);
        const float w2 = __uint_as_float(wv[j].y << 16), w3 = __uint_as_float(wv[j].y & 0xFFFF0000u);
        const uint2 h = make_uint2(pack2h(w0 * (v[j].x * rr), w1 * (v[j].y * rr)), pack2h(w2 * (v[j].z * rr), w3 * (v[j].w * rr)));
        bad |= f16_bad2(h.x) | f16_bad2(h.y);
        yr[64 * j] = h;
    }
    f16_note(bad, kF16Hidden);
}

// ================================================================ GEMM (ids 15, 17, 18, 19)
// C[m, n] = sum_k A[m, k] W[n, k] on f16 operands, 128 x 128 tiles (128 x 64 for the residual GEMMs of few tiles), k
// in steps of 64, 4 waves each owning a 64 x 64 quarter as 4 x 4 MFMA tiles. Tiles are loaded from memory straight
// into two LDS stages (the lds form of the buffer load), the next k tile landing while the current one multiplies.
constexpr int GBM = 128, GBN = 128, GBK = 64;

// A raw buffer resource over `bytes` bytes at `base` (gfx9 descriptor word 3: 32-bit data format, no swizzle): loads
// through it take a per-lane byte offset and a scalar one, so a loop's changing k offset costs no vector registers.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}

// 16 bytes per lane from a buffer resource straight into LDS: lane l writes lds_block + 16 l (lds_block is uniform).
// The builtin exists only for the device target, so the host pass (which only needs the kernels' launch stubs) sees
// an empty body.
__device__ __forceinline__ void buffer_load_lds16(__amdgpu_buffer_rsrc_t r, uint16_t* lds_block, int voff, int soff) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_block, 16, voff, soff, 0, 0);
#endif
}

enum Epi { EPI_F32 = 0, EPI_RESID = 1, EPI_SWIGLU = 2, EPI_QKV = 3, EPI_PART = 4 };

struct GemmArgs {
    const uint16_t* a;
    const uint16_t* w;
    int M, N, K;
    float* y32;           // F32, RESID (in place over resid)
    const float* resid;   // RESID
    uint16_t* y16;        // SWIGLU: [M, inter] f16
    int inter;            // SWIGLU: I (the W rows are gate 0..I-1 then up I..2I-1)
    // QKV: one 128-column tile per head; q heads, then k heads, then v heads
    const uint16_t* qn;   // bf16 norm weights
    const uint16_t* kn;
    const float* cos_t;
    const float* sin_t;
    uint16_t* q_out;      // [M, qh * 128] f16
    uint16_t* kc;         // [kvh, max_pos, 128] f16
    uint16_t* vc;         // [kvh, max_pos / 64, 128, 64] f16 (kv::v_at)
    int qh, kvh, pos0, max_pos;
    float eps;
    // PART: block z multiplies k range [z ksplit, (z + 1) ksplit) and writes its f32 partial to y32 + z M N
    int ksplit;
    // SWIGLU stores a 2^-s, RESID and PART multiply their sums by 2^s: the SwiGLU output's fp16 range moved up by s
    // binades (1 for s = 0, which changes no bit)
    float ascale;
};

// The stage-timing build (LRM_GEMM_STAMPS): wave 0 of every block of the direct-to-LDS loop records constant-clock
// stamps, per GEMM kind (the epilogue), of the last launch of that kind: word 0 the hardware CU (HW_ID) and XCD
// (XCC_ID) ids, 1 the block's start, 2 + kt tile kt landed (after the step's wait and barrier, kt < kGemmStampSteps),
// 28, 29, 26 and 27 points inside the q|k|v epilogue (past the barrier that ends the main loop; its global loads
// issued; its tile staged in LDS; its rows read back and their squares summed),
// 30 the main loop's end, 31 the epilogue's end. Lane k of wave 0 keeps stamp k in a register (one select per stamp)
// and the lanes store them once, at the end, so no stamp store is in flight while the block runs; the shipped build
// has none.
#if defined(LRM_GEMM_STAMPS)
constexpr int kGemmStampWords = 32, kGemmStampSteps = 24, kGemmStampBlocks = 4096, kGemmStampKinds = 5;
__device__ uint64_t g_gemm_stamps[kGemmStampKinds][kGemmStampBlocks * kGemmStampWords];
struct GemmStampEnd {  // the epilogue's end, at whichever return the lane leaves by
    uint64_t* at;
    uint64_t& v;
    int lane;
    __device__ ~GemmStampEnd() {
        if (at && lane < kGemmStampWords) {
            const uint64_t e = wall_clock64();
            at[lane] = lane == kGemmStampWords - 1 ? e : v;
        }
    }
};
#define GSTAMP(k)                                   \
    do {                                            \
        if (gst) {                                  \
            const uint64_t now_ = wall_clock64();   \
            gsv = lane == (k) ? now_ : gsv;         \
        }                                           \
    } while (0)
#else
#define GSTAMP(k) \
    do {          \
    } while (0)
#endif

// Two main loops, chosen by the launcher: DMA (a grid of at least two blocks per CU) moves tiles from memory
// straight into two LDS stages, the two blocks on a CU hiding each other's load latency; otherwise (one block per CU)
// tiles go through two register sets into two padded LDS buffers with every load two k steps ahead.
template <int EPI, int BN, bool DMA, int BM = GBM>
__global__ __launch_bounds__(256, 2) void k_gemm(GemmArgs p) {
    static_assert(BN == 128 || (BN == 64 && (EPI == EPI_F32 || EPI == EPI_RESID || EPI == EPI_PART)) ||
                      (BN == 192 && EPI == EPI_SWIGLU && DMA),
                  "QKV takes 128 columns, SwiGLU 128 or 192 (64 or 96 gate / up pairs)");
    static_assert(BM == GBM || (BM == 64 && (EPI == EPI_QKV || EPI == EPI_PART) && !DMA),
                  "64-row tiles: the q|k|v and k-split register loops only");
    constexpr int MI = BM / 32;   // MFMA row tiles per wave: each wave owns BM / 2 rows
    constexpr int PAIR = BN / 2;  // SWIGLU: gate / up pairs per tile
    // the k range of this block: all of k, or split z of a PART launch (A and W then start kz columns in)
    const int kz = EPI == EPI_PART ? int(blockIdx.z) * p.ksplit : 0;
    const int KE = EPI == EPI_PART ? p.ksplit : p.K;
    const uint16_t* const pa = p.a + kz;
    const uint16_t* const pw = p.w + kz;
    constexpr int WN = BN / 2, JT = WN / 16;    // columns per wave, MFMA tiles per wave
    // both paths: unpadded LDS rows of GBK halves, the 16-byte chunks XOR-swizzled (row r, position q holds k chunk
    // q ^ (r % 8)), so a fragment read (16 rows, one chunk) spreads over the banks (padded 144-byte rows measured
    // 14 % of the register path's cycles stalled on bank conflicts)
    constexpr int STAGE = (BM + BN) * GBK;  // halves: the A tile then the W tile
    // LDS stages of the direct-to-LDS loop: three for 128 x 64 tiles (72 KiB, two blocks per CU still fit), else two
    constexpr int NST = DMA && BN == 64 ? 3 : 2;
    // the stages, or what the QKV epilogue needs after them (x32 32 KiB + the V^T tile 128 x 136 halves)
    constexpr int LDS_HALVES = EPI == EPI_QKV ? (NST * STAGE > 33792 ? NST * STAGE : 33792) : NST * STAGE;
    __shared__ __attribute__((aligned(16))) uint16_t lds[LDS_HALVES];
    const int t = threadIdx.x, lane = t & 63, w = t >> 6, wm = w >> 1, wn = w & 1, g = lane >> 4, c16 = lane & 15;
    // XCD-aware tile order. Blocks are dispatched round-robin over the 8 XCDs (block L, x fastest, on XCD L % 8), each
    // with its own L2. Block L takes tile T = (L % 8) (tiles / 8) + L / 8, so an XCD's blocks are consecutive tiles,
    // and tiles are numbered in groups of GM row tiles, rows fastest within a group: an XCD then covers about a
    // GM x (tiles / 8 / GM) rectangle and reads GM row tiles of A and tiles / 8 / GM column tiles of W into its L2,
    // instead of (with x fastest) every row tile of A. GM balances the two (A rows are 128 wide, W columns BN).
    constexpr int GM = BN == 64 ? 4 : 8;
    int tx = blockIdx.x, ty = blockIdx.y;
    {
        const int gx = gridDim.x, ntiles = gx * int(gridDim.y), L = int(blockIdx.y) * gx + int(blockIdx.x);
        const int T = ntiles % 8 == 0 ? (L % 8) * (ntiles / 8) + L / 8 : L;
        const int sr = T / (GM * gx), within = T - sr * GM * gx, rows = min(GM, int(gridDim.y) - sr * GM);
        ty = sr * GM + within % rows;
        tx = within / rows;
    }
    const int m0 = ty * BM;
    const int n0 = tx * BN;
#if defined(LRM_GEMM_STAMPS)
    uint64_t* gst = nullptr;  // wave 0 of a direct-to-LDS block: where its stamps go
    uint64_t gsv = 0;         // lane k: stamp k
    {
        const int Lb = (int(blockIdx.z) * int(gridDim.y) + int(blockIdx.y)) * int(gridDim.x) + int(blockIdx.x);
        if (DMA && w == 0 && Lb < kGemmStampBlocks) {
            gst = g_gemm_stamps[EPI] + size_t(Lb) * kGemmStampWords;
            const uint32_t hw = __builtin_amdgcn_s_getreg((31 << 11) | 4), xcc = __builtin_amdgcn_s_getreg((3 << 11) | 20);
            gsv = lane == 0 ? (uint64_t(xcc) << 32) | hw : 0;
        }
    }
    GSTAMP(1);
    GemmStampEnd gst_end{gst, gsv, lane};
#endif

    f32x4 acc[MI][JT];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < JT; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (DMA) {
        // Tiles go from memory straight into LDS (buffer loads with the lds flag: no registers, no LDS store
        // instructions). One load instruction moves 64 lanes x 16 B = 1 KiB = 8 rows of 128 B; lane l writes LDS bytes
        // 16 l of it, i.e. row l / 8, chunk position l % 8. Rows are unpadded and the 16-byte chunks XOR-swizzled: LDS row
        // r, position q holds k chunk q ^ (r % 8), so a fragment read (16 rows, one chunk) spreads over the banks. Each wave
        // issues instructions i = 0, 1, ... for the 1 KiB blocks 4 i + w. A row past the matrix is clamped to its last row
        // (it only feeds outputs that are never stored); the k offset is a scalar.
        constexpr int NA = BM / 32, NB = BN / 32;  // load instructions per wave per stage
        static_assert(NA + NB < 16, "vmcnt's low field");
        int aoff[NA], boff[NB];
    #pragma unroll
        for (int i = 0; i < NA; ++i) {
            const int r = 8 * (4 * i + w) + (lane >> 3), c = (lane & 7) ^ (r & 7);
            aoff[i] = (min(m0 + r, p.M - 1) * p.K + c * 8) * 2;
        }
    #pragma unroll
        for (int i = 0; i < NB; ++i) {
            const int r = 8 * (4 * i + w) + (lane >> 3), c = (lane & 7) ^ (r & 7);
            int n;
            if (EPI == EPI_SWIGLU) {
                const int j = min(tx * PAIR + (r < PAIR ? r : r - PAIR), p.inter - 1);
                n = r < PAIR ? j : p.inter + j;
            } else {
                n = min(n0 + r, p.N - 1);
            }
            boff[i] = (n * p.K + c * 8) * 2;
        }
        const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(pa, (p.M * p.K - kz) * 2);
        const __amdgpu_buffer_rsrc_t w_rsrc = make_rsrc(pw, ((EPI == EPI_SWIGLU ? 2 * p.inter : p.N) * p.K - kz) * 2);
        auto issue = [&](int buf, int k0) __attribute__((always_inline)) {
            uint16_t* st = lds + buf * STAGE;
    #pragma unroll
            for (int i = 0; i < NA; ++i) buffer_load_lds16(a_rsrc, st + (4 * i + w) * 512, aoff[i], k0 * 2);
    #pragma unroll
            for (int i = 0; i < NB; ++i) buffer_load_lds16(w_rsrc, st + BM * GBK + (4 * i + w) * 512, boff[i], k0 * 2);
        };

        // one k step of a stage: per 32-wide half, the A fragments (rows of this wave's 4 MFMA row tiles) and the W
        // fragments, read from their swizzled chunk, then the MFMAs
        auto compute = [&](int buf) __attribute__((always_inline)) {
            const uint16_t* As = lds + buf * STAGE;
            const uint16_t* Bs = As + BM * GBK;
    #pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                f16x8 af[MI], bf[JT];
    #pragma unroll
                for (int i = 0; i < MI; ++i) {
                    const int r = wm * (BM / 2) + i * 16 + c16;
                    af[i] = as_f16x8(*reinterpret_cast<const u32x4*>(As + r * GBK + (((ks * 4 + g) ^ (r & 7)) * 8)));
                }
    #pragma unroll
                for (int j = 0; j < JT; ++j) {
                    const int r = wn * WN + j * 16 + c16;
                    bf[j] = as_f16x8(*reinterpret_cast<const u32x4*>(Bs + r * GBK + (((ks * 4 + g) ^ (r & 7)) * 8)));
                }
    #pragma unroll
                for (int i = 0; i < MI; ++i)
    #pragma unroll
                    for (int j = 0; j < JT; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
            }
        };
        // NST stages: step kt waits for its tile (this wave's loads, then the barrier for everyone's, which also means
        // every wave is done reading the stage of tile kt - 1), queues tile kt + NST - 1 into that stage and multiplies
        // tile kt; NST - 1 tiles are in flight while it does. With three stages the wait leaves tile kt + 1's loads
        // (the younger NA + NB of this wave's) outstanding: loads complete in issue order.
        // The LDS-only barrier: __syncthreads() would also make every wave wait for the loads just queued.
        const int nk = KE / GBK;
        issue(0, 0);
        if (NST == 3 && nk > 1) issue(1, GBK);
        for (int kt = 0; kt < nk; ++kt) {
            if (NST == 3 && kt + 1 < nk)
                __builtin_amdgcn_s_waitcnt(0x0F70 | (NA + NB));  // vmcnt(NA + NB): tile kt has landed in LDS
            else
                __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
            lds_barrier();
#if defined(LRM_GEMM_STAMPS)
            if (kt < kGemmStampSteps) GSTAMP(2 + kt);
#endif
            if (kt + NST - 1 < nk) issue((kt + NST - 1) % NST, (kt + NST - 1) * GBK);  // uniform
            compute(kt % NST);
        }
        GSTAMP(30);
    } else {
        // the rows this thread loads: chunk c = t + 256 i -> row c / 8, 16-byte column (c % 8), as element offsets from
        // the matrix base (every matrix is under 2^31 elements). A row past the matrix is clamped to its last row: it only
        // feeds output rows / columns that are never stored, and the loads stay unconditional, so the compiler can keep
        // several tiles in flight (a guarded load makes it wait for every outstanding load).
        constexpr int BCH = BN / 32;  // B chunks per thread
        int aoff[MI], boff[BCH];  // byte offsets: the loads are buffer loads with the k offset in a scalar register
    #pragma unroll
        for (int i = 0; i < MI; ++i) {
            const int c = t + 256 * i, r = c >> 3, kc = (c & 7) * 8;
            aoff[i] = (min(m0 + r, p.M - 1) * p.K + kc) * 2;
        }
    #pragma unroll
        for (int i = 0; i < BCH; ++i) {
            const int c = t + 256 * i, r = c >> 3, kc = (c & 7) * 8;
            int n;
            if (EPI == EPI_SWIGLU) {
                const int j = min(tx * PAIR + (r < PAIR ? r : r - PAIR), p.inter - 1);
                n = r < PAIR ? j : p.inter + j;
            } else {
                n = min(n0 + r, p.N - 1);
            }
            boff[i] = (n * p.K + kc) * 2;
        }
        const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(pa, (p.M * p.K - kz) * 2);
        const __amdgpu_buffer_rsrc_t w_rsrc = make_rsrc(pw, ((EPI == EPI_SWIGLU ? 2 * p.inter : p.N) * p.K - kz) * 2);
        // Two register sets, two LDS buffers: tile j is loaded into set j % 2 at the top of iteration j - 2 and stored to
        // LDS buffer j % 2 at the end of iteration j - 1, so each load has two iterations of MFMAs to land. The loop is
        // unrolled by two so every register set is named at compile time.
        u32x4 ra[2][MI], rb[2][BCH];
        auto gload = [&](auto set, int k0) __attribute__((always_inline)) {
            constexpr int S = decltype(set)::value;
    #pragma unroll
            for (int i = 0; i < MI; ++i) ra[S][i] = __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, aoff[i], k0 * 2, 0);
    #pragma unroll
            for (int i = 0; i < BCH; ++i) rb[S][i] = __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, boff[i], k0 * 2, 0);
        };
        auto sstore = [&](auto set, int buf) __attribute__((always_inline)) {
            constexpr int S = decltype(set)::value;
            uint16_t* As = lds + buf * STAGE;
            uint16_t* Bs = As + BM * GBK;
    #pragma unroll
            for (int i = 0; i < MI; ++i) {
                const int c = t + 256 * i, r = c >> 3;
                *reinterpret_cast<u32x4*>(As + r * GBK + (((c & 7) ^ (r & 7)) * 8)) = ra[S][i];
            }
    #pragma unroll
            for (int i = 0; i < BCH; ++i) {
                const int c = t + 256 * i, r = c >> 3;
                *reinterpret_cast<u32x4*>(Bs + r * GBK + (((c & 7) ^ (r & 7)) * 8)) = rb[S][i];
            }
        };


        // MFMA operands of one 32-wide k half (ks) of an LDS buffer: two named register sets, F0 for ks 0 and F1 for
        // ks 1, so the reads of one half run under the MFMAs of the other
        f16x8 fa[2][MI], fb[2][JT];
        auto read_frags = [&](auto ksc, int buf) __attribute__((always_inline)) {
            constexpr int KS = decltype(ksc)::value;
            const uint16_t* As = lds + buf * STAGE;
            const uint16_t* Bs = As + BM * GBK;
    #pragma unroll
            for (int i = 0; i < MI; ++i) {
                const int r = wm * (BM / 2) + i * 16 + c16;
                fa[KS][i] = as_f16x8(*reinterpret_cast<const u32x4*>(As + r * GBK + (((KS * 4 + g) ^ (r & 7)) * 8)));
            }
    #pragma unroll
            for (int j = 0; j < JT; ++j) {
                const int r = wn * WN + j * 16 + c16;
                fb[KS][j] = as_f16x8(*reinterpret_cast<const u32x4*>(Bs + r * GBK + (((KS * 4 + g) ^ (r & 7)) * 8)));
            }
        };
        auto mfma_half = [&](auto ksc) __attribute__((always_inline)) {
            constexpr int KS = decltype(ksc)::value;
    #pragma unroll
            for (int i = 0; i < MI; ++i)
    #pragma unroll
                for (int j = 0; j < JT; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[KS][i], fb[KS][j], acc[i][j], 0, 0, 0);
        };
        // the MFMAs of one half interleaved with the LDS reads of the other: MPR MFMAs, then one read
        constexpr int NRD = MI + JT, NMF = MI * JT, MPR = NMF / NRD;
        auto interleave = [&]() __attribute__((always_inline)) {
    #pragma unroll
            for (int i = 0; i < NRD; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, MPR, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            if constexpr (NMF > MPR * NRD) __builtin_amdgcn_sched_group_barrier(0x008, NMF - MPR * NRD, 0);
        };
        using S0 = std::integral_constant<int, 0>;
        using S1 = std::integral_constant<int, 1>;
        using K0 = std::integral_constant<int, 0>;
        using K1 = std::integral_constant<int, 1>;
        const int nk = KE / GBK;
        // Tile t is loaded into register set t % 2 and stored to LDS buffer t % 2. Step t (parity P), with tile t in
        // buffer P and its ks-0 operands in F0, tiles t + 1 and t + 2 loaded (or landing) in sets 1 - P and P:
        //   store set 1 - P (tile t + 1) into buffer 1 - P (read up to the previous step, whose barrier every wave has
        //   passed) and load tile t + 3 into it, so every load has two steps to land; ks-0 MFMAs with the ks-1 reads of
        //   buffer P; barrier (this wave's stores and reads complete, so buffer 1 - P is whole); ks-1 MFMAs with the ks-0
        //   reads of buffer 1 - P. Loads past the last tile re-read it (clamped); the last steps' stores and reads of
        //   such tiles are never used.
        auto step = [&](auto par, int kt) __attribute__((always_inline)) {
            constexpr int P = decltype(par)::value;
            sstore(std::integral_constant<int, 1 - P>{}, 1 - P);
            gload(std::integral_constant<int, 1 - P>{}, min(kt + 3, nk - 1) * GBK);
            __builtin_amdgcn_sched_barrier(0);
            read_frags(K1{}, P);
            mfma_half(K0{});
            interleave();
            __builtin_amdgcn_sched_barrier(0);
            lds_barrier();
            read_frags(K0{}, 1 - P);
            mfma_half(K1{});
            interleave();
            __builtin_amdgcn_sched_barrier(0);
        };
        // loads issue in tile order, so each wait leaves the younger tiles in flight
        gload(S0{}, 0);
        __builtin_amdgcn_sched_barrier(0);
        gload(S1{}, min(1, nk - 1) * GBK);
        __builtin_amdgcn_sched_barrier(0);
        sstore(S0{}, 0);
        gload(S0{}, min(2, nk - 1) * GBK);
        lds_barrier();
        read_frags(K0{}, 0);
        __builtin_amdgcn_sched_barrier(0);
        // whole pairs in the loop (a conditional second step would leave the loop head with set 1 possibly the younger,
        // and the waits there would drain every load); an odd last step after it
        int kt = 0;
        for (; kt + 1 < nk; kt += 2) {
            step(S0{}, kt);
            step(S1{}, kt + 1);
        }
        if (kt < nk) step(S0{}, kt);
    }
    __syncthreads();  // the epilogues below reuse the LDS

    if (EPI == EPI_F32 || EPI == EPI_RESID || EPI == EPI_PART) {
        float* const y = EPI == EPI_PART ? p.y32 + size_t(blockIdx.z) * p.M * p.N : p.y32;
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < JT; ++j) {
                int n = n0 + wn * WN + j * 16 + c16;
                if (n >= p.N) continue;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    int m = m0 + wm * (BM / 2) + i * 16 + 4 * g + r;
                    if (m >= p.M) continue;
                    size_t o = size_t(m) * p.N + n;
                    const float v = EPI == EPI_F32 ? acc[i][j][r] : acc[i][j][r] * p.ascale;
                    y[o] = EPI == EPI_RESID ? p.resid[o] + v : v;
                }
            }
        return;
    }

    // QKV, q and k heads (head = the column tile: q heads, then k heads, then v heads; head_dim 128 = the tile's
    // columns): every wave stages its accumulators in LDS as the f32 tile [128 rows][128 dims], the 4-float unit u of row
    // r at unit u ^ (r % 16) (conflict-free both for these stores and for the row reads below), then thread t takes row
    // t / 2, dims 32 (t % 2) .. + 31 and their RoPE partners + 64: RMSNorm over the row (the other half is lane t ^ 1),
    // the rotation, and 16-byte stores of the q row or the K cache row.
    if constexpr (EPI == EPI_QKV) {
        const int head = tx;
        if (head < p.qh + p.kvh) {
            GSTAMP(28);
            const bool is_q = head < p.qh;
            const int row = t >> 1, hf = t & 1, m = m0 + row;
            // Every global load of the epilogue first: the norm weights and this row's cos / sin (the row clamped to
            // the last one for rows past M, which store nothing), so their latency runs under the staging below and is
            // paid once. (Loaded between the stores, which the compiler may not reorder them across, the four groups
            // each waited a whole load latency: 7.8 of a 24.5 us block at 2048 x 4096 x 1024.)
            const int pos = p.pos0 + min(m, p.M - 1);
            const uint16_t* nw = (is_q ? p.qn : p.kn) + hf * 32;
            const float* cst = p.cos_t + size_t(pos) * 64 + hf * 32;
            const float* snt = p.sin_t + size_t(pos) * 64 + hf * 32;
            u32x4 wlv[4], whv[4];
            f32x4 c0v[4], c1v[4], s0v[4], s1v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                wlv[u] = *reinterpret_cast<const u32x4*>(nw + 8 * u);
                whv[u] = *reinterpret_cast<const u32x4*>(nw + 64 + 8 * u);
                c0v[u] = *reinterpret_cast<const f32x4*>(cst + 8 * u);
                c1v[u] = *reinterpret_cast<const f32x4*>(cst + 8 * u + 4);
                s0v[u] = *reinterpret_cast<const f32x4*>(snt + 8 * u);
                s1v[u] = *reinterpret_cast<const f32x4*>(snt + 8 * u + 4);
            }
            GSTAMP(29);
            float* tile = reinterpret_cast<float*>(lds);
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < JT; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int rw = wm * (BM / 2) + i * 16 + 4 * g + r, col = wn * WN + j * 16 + c16;
                        tile[rw * 128 + (col ^ ((rw & 15) << 2))] = acc[i][j][r];
                    }
            lds_barrier();  // LDS only: the loads above stay in flight
            GSTAMP(26);
            if (row >= BM) return;  // 64-row tiles: threads 128 .. 255 have no row
            float x[2][32];
#pragma unroll
            for (int part = 0; part < 2; ++part)
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int unit = (part * 64 + hf * 32) / 4 + u;
                    const f32x4 v = *reinterpret_cast<const f32x4*>(tile + row * 128 + 4 * (unit ^ (row & 15)));
#pragma unroll
                    for (int e = 0; e < 4; ++e) x[part][4 * u + e] = v[e];
                }
            float ss = 0.f;
#pragma unroll
            for (int k = 0; k < 32; ++k) ss = fmaf(x[1][k], x[1][k], fmaf(x[0][k], x[0][k], ss));
            ss += dpp_f<0xB1>(ss);  // + the other half of the row (lane t ^ 1)
            GSTAMP(27);
            if (m >= p.M) return;
            const float rr = 1.0f / sqrtf(ss / 128.0f + p.eps);
            uint16_t* out = is_q ? p.q_out + size_t(m) * (p.qh * 128) + head * 128
                                 : p.kc + (size_t(head - p.qh) * p.max_pos + pos) * 128;
            out += hf * 32;
            uint32_t bad = 0;
#pragma unroll
            for (int u = 0; u < 4; ++u) {  // 8 dims d = 32 hf + 8 u + e and their partners d + 64
                const u32x4 wl = wlv[u], wh = whv[u];
                const f32x4 c0 = c0v[u], c1 = c1v[u], s0 = s0v[u], s1 = s1v[u];
                uint32_t lo[4], hi[4];
#pragma unroll
                for (int e2 = 0; e2 < 4; ++e2) {
                    float rl[2], rh[2];
#pragma unroll
                    for (int h1 = 0; h1 < 2; ++h1) {
                        const int e = 2 * e2 + h1, k = 8 * u + e;
                        const float nl = __uint_as_float(h1 ? (wl[e2] & 0xFFFF0000u) : (wl[e2] << 16));
                        const float nh = __uint_as_float(h1 ? (wh[e2] & 0xFFFF0000u) : (wh[e2] << 16));
                        const float a = nl * (x[0][k] * rr), b = nh * (x[1][k] * rr);
                        const float cs = e < 4 ? c0[e] : c1[e - 4], sn = e < 4 ? s0[e] : s1[e - 4];
                        rl[h1] = a * cs - b * sn;
                        rh[h1] = b * cs + a * sn;
                    }
                    lo[e2] = uint32_t(f2h(rl[0])) | (uint32_t(f2h(rl[1])) << 16);
                    hi[e2] = uint32_t(f2h(rh[0])) | (uint32_t(f2h(rh[1])) << 16);
                    bad |= f16_bad2(lo[e2]) | f16_bad2(hi[e2]);
                }
                *reinterpret_cast<u32x4*>(out + 8 * u) = u32x4{lo[0], lo[1], lo[2], lo[3]};
                *reinterpret_cast<u32x4*>(out + 64 + 8 * u) = u32x4{hi[0], hi[1], hi[2], hi[3]};
            }
            f16_note(bad, is_q ? kF16Query : kF16Cache);
            return;
        }
    }

    if constexpr (EPI == EPI_SWIGLU) {
        // a[m, j0 + c] = silu(gate) * up, silu(g) = g / (1 + exp(-g)). The gate column c (wave wn = 0) and its up
        // column c + PAIR (wave wn = 1, same lane and tile index) meet through LDS, half the row tiles each way, so
        // every wave computes: wave wn takes row tiles [wn MI / 2, (wn + 1) MI / 2). Values cross as 16-byte units
        // (an MFMA tile's 4 rows per lane). The products go to an fp16 tile in LDS after the exchange area (rows of
        // PAIR columns padded by 8), then out as 16-byte row chunks by all four waves. (Two waves with an IEEE
        // division per value took 6 us of a 27 us block at 2048 x 3072 x 1024.)
        constexpr int HM = MI / 2, AR = PAIR + 8, CH = PAIR / 8;  // LDS row stride (halves), 16-byte chunks per row
        f32x4* xq = reinterpret_cast<f32x4*>(lds);  // [wm][dir][HM][JT][64 lanes]: same size as 2 x MI x JT x 1 KiB
        uint16_t* As = lds + 2 * MI * 4 * JT * 64 * 2;
        auto slot = [&](int dir, int i, int j) { return ((wm * 2 + dir) * HM * JT + i * JT + j) * 64 + lane; };
        if (wn == 0) {  // dir 1: the gate values of row tiles HM .. MI - 1, to wave wn = 1
#pragma unroll
            for (int i = 0; i < HM; ++i)
#pragma unroll
                for (int j = 0; j < JT; ++j) xq[slot(1, i, j)] = acc[HM + i][j];
        } else {  // dir 0: the up values of row tiles 0 .. HM - 1, to wave wn = 0
#pragma unroll
            for (int i = 0; i < HM; ++i)
#pragma unroll
                for (int j = 0; j < JT; ++j) xq[slot(0, i, j)] = acc[i][j];
        }
        __syncthreads();
        const int rt0 = wn * HM;  // this wave's first row tile
        auto emit = [&](int i, int j, const f32x4& gv4, const f32x4& uv4) __attribute__((always_inline)) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float gv = gv4[r];
                const float sg = gv * __builtin_amdgcn_rcpf(1.0f + __expf(-gv));
                As[(wm * (BM / 2) + (rt0 + i) * 16 + 4 * g + r) * AR + j * 16 + c16] = f2h(sg * uv4[r] * p.ascale);
            }
        };
        // the partner's values first, all of them: read between the product stores, each read would wait for the
        // stores before it (the compiler cannot tell the two LDS regions apart)
        f32x4 other[HM][JT];
#pragma unroll
        for (int i = 0; i < HM; ++i)
#pragma unroll
            for (int j = 0; j < JT; ++j) other[i][j] = xq[slot(wn == 0 ? 0 : 1, i, j)];
        if (wn == 0) {
#pragma unroll
            for (int i = 0; i < HM; ++i)
#pragma unroll
                for (int j = 0; j < JT; ++j) emit(i, j, acc[i][j], other[i][j]);
        } else {
#pragma unroll
            for (int i = 0; i < HM; ++i)
#pragma unroll
                for (int j = 0; j < JT; ++j) emit(i, j, other[i][j], acc[HM + i][j]);
        }
        __syncthreads();
        uint32_t bad = 0;
#pragma unroll
        for (int k = 0; k < CH / 2; ++k) {  // 128 rows x CH chunks = 256 (CH / 2) chunks
            const int q = t + 256 * k, row = q / CH, ch = q % CH, m = m0 + row, col = tx * PAIR + ch * 8;
            if (m >= p.M || col >= p.inter) continue;
            const u32x4 v = *reinterpret_cast<const u32x4*>(As + row * AR + ch * 8);
            uint16_t* dst = p.y16 + size_t(m) * p.inter + col;
            if (col + 8 <= p.inter && (p.inter & 7) == 0) {
                bad |= f16_bad8(v);
                *reinterpret_cast<u32x4*>(dst) = v;
            } else {
                for (int e = 0; e < 8 && col + e < p.inter; ++e) {
                    const uint16_t h = uint16_t(v[e >> 1] >> (16 * (e & 1)));
                    bad |= f16_bad2(h);
                    dst[e] = h;
                }
            }
        }
        f16_note(bad, kF16Swiglu);
        return;
    }


    // The V heads of QKV pair column c (wave wn = 0) with column c + PAIR (wave wn = 1, same lane and tile index): the
    // second half goes through LDS to the first.
    float* x32 = reinterpret_cast<float*>(lds);  // 2 (wm) x 4 JT x 4 values x 64 lanes: 32 KiB (JT 4), 48 KiB (JT 6)
    if (wn == 1) {
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < JT; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) x32[((wm * MI * JT + i * JT + j) * 4 + r) * 64 + lane] = acc[i][j][r];
    }
    __syncthreads();
    const int head = tx;  // QKV: a V head (the q and k heads returned above)
    // the partner half of row tile i, read back from LDS
    auto load_hi = [&](int i, float (&hi)[JT][4]) {
#pragma unroll
        for (int j = 0; j < JT; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) hi[j][r] = x32[((wm * MI * JT + i * JT + j) * 4 + r) * 64 + lane];
    };

    if (EPI == EPI_QKV) {
        // V: the cache holds [dim][position] tiles of 64 positions (kv::v_at), so the tile is transposed through LDS
        // (after the 32 KiB of x32, rows of 128 positions padded to 136) and written as 16-byte runs of 8 positions,
        // not 2-byte stores
        uint16_t* Vs = lds + 16384;
        if (wn == 0) {
#pragma unroll
            for (int i = 0; i < MI; ++i) {
                float hi[JT][4];
                load_hi(i, hi);
#pragma unroll
                for (int j = 0; j < JT; ++j) {
                    uint16_t* vr = Vs + (j * 16 + c16) * 136 + wm * (BM / 2) + i * 16 + 4 * g;
                    *reinterpret_cast<uint2*>(vr) =
                        make_uint2(pack2h(acc[i][j][0], acc[i][j][1]), pack2h(acc[i][j][2], acc[i][j][3]));
                    *reinterpret_cast<uint2*>(vr + 64 * 136) =
                        make_uint2(pack2h(hi[j][0], hi[j][1]), pack2h(hi[j][2], hi[j][3]));
                }
            }
        }
        __syncthreads();
        const int p0 = p.pos0 + m0;
        // 16-byte aligned (8 positions in one 64-position block of the cache), every row of the tile present
        const bool whole = (p0 & 7) == 0 && m0 + BM <= p.M;
        constexpr int CHV = BM / 8, RPP = 256 / CHV;  // 16-byte chunks per V^T row, rows per pass
        const int ch = t % CHV;
        uint32_t bad = 0;
        uint16_t* vhead = p.vc + size_t(head - p.qh - p.kvh) * 128 * p.max_pos;
#pragma unroll
        for (int k = 0; k < 128 / RPP; ++k) {
            const int d = t / CHV + RPP * k;
            const u32x4 v = *reinterpret_cast<const u32x4*>(Vs + d * 136 + ch * 8);
            if (whole) {
                bad |= f16_bad8(v);
                *reinterpret_cast<u32x4*>(vhead + kv::v_at(p0 + ch * 8, d)) = v;
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    if (m0 + ch * 8 + e < p.M) {
                        const uint16_t h = uint16_t(v[e >> 1] >> (16 * (e & 1)));
                        bad |= f16_bad2(h);
                        vhead[kv::v_at(p0 + ch * 8 + e, d)] = h;
                    }
            }
        }
        f16_note(bad, kF16Cache);
        return;
    }
}

// ================================================================ 16 attention_prefill_f16
// Causal GQA flash attention on v_mfma_f32_32x32x16_f16 (32 query columns per wave: half the LDS operand bytes per
// FLOP of the 16-column form), two query heads per KV head. A tile is 32 query rows of both heads of one KV group: wave
// w owns head 2 kvhead + w % 2 (32 query columns, one MFMA column tile) and key half w / 2 (keys 32 (w / 2) .. + 31)
// of every 64-key block, so the four waves share each block's K and V^T in LDS (two stages, one barrier per block)
// and each wave runs its own online softmax over its half; the two halves of a head merge through LDS at the end.
// S^T = K Q^T (A = 32 keys x 16 dims of K from LDS, B = Q^T from registers) puts one query per lane column; lanes
// l and l + 32 hold the other 16 keys of the same column, so the row statistics take one v_permlane32_swap. The P^T
// operand of O^T = V^T P^T needs keys 8 h .. 8 h + 7 of a 16-key step in lane half h; a lane holds keys
// 4 h .. 4 h + 3 and 8 + 4 h .. 8 + 4 h + 3, and one swap of the packed halves with lane l ^ 32 gives the rest, so V^T
// stays in LDS in its natural key order. LDS rows are padded by 16 bytes (K 272, V^T 144), so the 16 lanes of each
// read phase hit distinct banks and every operand address is a per-lane base plus an immediate. The softmax keeps a
// reference maximum per column that moves (rescaling O and the sum) only when a block's maximum exceeds it by more
// than 8 in the exponent: P stays at most 2^8, and most blocks need no rescale.
//
// Causal balance: tile i needs about i / 2 key blocks, and a workgroup alone on its CU runs its blocks more slowly
// than two sharing one, so whole tiles would leave the longest tiles running alone at the end. Tiles pair up, short
// tile s = p with long tile n - 1 - p, and on grids of two workgroups per CU the pair's blocks split over two
// workgroups: X runs the first `a` key blocks of the long tile, then the whole short tile; Y runs the rest of the
// long tile. The two parts of the long
// tile meet in the workspace: each part, when done, reads the pair's counter; if the other part is already there it
// merges the other's partial (O^T, m, l) with its own and writes the rows, otherwise it stores its partial, then adds
// to the counter, and merges if the other part arrived in between. The merge combines the parts in X, Y order
// whichever workgroup runs it, so the result does not depend on timing; the merging workgroup resets the counter.
// Pair p's counter and partials form record p of the workspace (attn_prefill.hpp).
// Nothing waits for another workgroup. An odd tile count leaves the middle tile whole.
constexpr int kAttnRows = attn_prefill::kRows;
constexpr int kAttnSlotWords = attn_prefill::kSlotWords;

typedef float f32x16 __attribute__((ext_vector_type(16)));

// key blocks of tile `tile` (64-key blocks up to the last visible key of its last row)
__device__ __forceinline__ int attn_tile_blocks(int tile, int T, int past) {
    return (past + min(tile * kAttnRows + kAttnRows - 1, T - 1) + 1 + 63) / 64;
}

__global__ __launch_bounds__(256, 2) void k_attn_prefill(const uint16_t* q, const uint16_t* kc, const uint16_t* vc,
                                                      uint16_t* y, uint32_t* ws, int T, int past, int qh,
                                                      int max_pos, float scale_log2) {
    // stage s: K [64 keys][128 dims + 8] at s * kStage, V^T [128 dims][64 keys + 8] at s * kStage + kVtOff
    constexpr int kKRow = 272, kVRow = 144, kVtOff = 64 * kKRow, kStage = kVtOff + 128 * kVRow;
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * kStage];
    __shared__ int s_flag;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6, c32 = lane & 31, h = lane >> 5;
    const int cg = w & 1, kh = w >> 1;
    const int ntile = (T + kAttnRows - 1) / kAttnRows, kvh = int(gridDim.y), npairs = ntile / 2;
    const int L = int(blockIdx.y) * ntile + int(blockIdx.x);
    const int kvhead = L % kvh, u = L / kvh;
    const int head = kvhead * 2 + cg;
    const int QC = qh * 128;
    const __amdgpu_buffer_rsrc_t k_rsrc = make_rsrc(kc + size_t(kvhead) * max_pos * 128, max_pos * 256);
    const __amdgpu_buffer_rsrc_t v_rsrc = make_rsrc(vc + size_t(kvhead) * 128 * max_pos, max_pos * 256);
    // thread t moves chunks t + 256 i of a block: K row c / 16, dims 8 (c % 16) ..; V^T row (dim) c / 8, keys 8 (c % 8) ..
    // (a 64-key block of either cache is 16 KiB contiguous at 256 bytes per key)
    int koff[4], voff[4], kst[4], vst[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = t + 256 * i;
        const int kr = c >> 4, kq = c & 15, vd = c >> 3, vq = c & 7;
        koff[i] = (kr * 128 + kq * 8) * 2;
        voff[i] = (vd * 64 + vq * 8) * 2;
        kst[i] = kr * kKRow + 16 * kq;
        vst[i] = kVtOff + vd * kVRow + 16 * vq;
    }
    // read offsets of the MFMA operands: K row 32 kh + c32, chunk 2 s + h; V^T row 32 dt + c32, chunk 4 kh + 2 ks + h
    const int krd = (32 * kh + c32) * kKRow + 16 * h;
    const int vrd = kVtOff + c32 * kVRow + 16 * (4 * kh + h);

    // this workgroup's items: (tile, first key block, end key block, role: -1 whole tile, 0 part X, 1 part Y)
    int pair = 0, nitems = 1, split_a = 0, long_tile = 0, short_tile = 0;
    if (u < 2 * npairs) {
        pair = u < npairs ? u : u - npairs;
        short_tile = pair;
        long_tile = ntile - 1 - pair;
        const int ns = attn_tile_blocks(short_tile, T, past), nl = attn_tile_blocks(long_tile, T, past);
        // Only a grid of two workgroups per CU (MI355X: 256 CUs) splits: alone on its CU, X's second tile costs a
        // whole second pipeline start (T 512, 128 workgroups: 11.7 us whole, 13.5 split). Even halves, then two more
        // blocks for X: X is dispatched first, so its waves win the issue arbitration while both run, and Y finishes
        // alone at the end (T 2048: 16 / 17 blocks 36.3 us, 18 / 15 blocks 35.8 us).
        const int even = (ns + nl) / 2 - ns;
        split_a = ntile * kvh >= 512 && even > 0 ? min(even + 2, nl - 1) : 0;
        if (u < npairs && split_a > 0) nitems = 2;
    }

    f16x8 qf[8];
    float m_run, l_run;
    f32x16 o[4];
    int row0, row, kend, kb0, nb;
    u32x4 rk[2][4], rv[2][4];
    float sc[16];

    // Software pipeline over an item's blocks kb0 .. kb0 + nb - 1 (relative index j), one barrier per step: step j
    // stores K(j + 2) and V^T(j + 1), issues the scores of block j + 1 to the matrix core and runs block j's softmax
    // on the VALU while they execute, then block j's P V. K(b) lives in the K region of stage b % 2 and V^T(b) in the
    // V^T region of stage b % 2: at step j (P = j % 2) the K region of stage P takes K(j + 2) (it held K(j), read by
    // step j - 1), the V^T region of stage 1 - P takes V^T(j + 1) (it held V^T(j - 1), read by step j - 1), and the
    // step reads K(j + 1) from stage 1 - P and V^T(j) from stage P, both stored by step j - 1 before this step's
    // barrier.
    // Global loads: group g = K(g) and V^T(g - 1), loaded into register set g % 2 by step g - 4 (or the prologue) and
    // stored by step g - 2. The loads are unconditional (a block index past the item's last is clamped to it, and
    // every block of an item ends below kend <= max_pos); keys at or past kend may hold anything. Their scores are
    // masked, so K needs nothing; V is zeroed there before it is stored, since a zero weight times a NaN is still a
    // NaN.
    auto fetch = [&](auto set, int g) __attribute__((always_inline)) {
        constexpr int S = decltype(set)::value;
        const int kbk = (kb0 + min(g, nb - 1)) * 64, kbv = (kb0 + min(max(g - 1, 0), nb - 1)) * 64;
#pragma unroll
        for (int i = 0; i < 4; ++i) rk[S][i] = __builtin_amdgcn_raw_buffer_load_b128(k_rsrc, koff[i], kbk * 256, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) rv[S][i] = __builtin_amdgcn_raw_buffer_load_b128(v_rsrc, voff[i], kbv * 256, 0);
    };
    auto store_k = [&](auto set, auto stage) __attribute__((always_inline)) {
        constexpr int S = decltype(set)::value, G = decltype(stage)::value;
#pragma unroll
        for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4*>(lds + G * kStage + kst[i]) = rk[S][i];
    };
    auto store_v = [&](auto set, auto stage, int j) __attribute__((always_inline)) {
        constexpr int S = decltype(set)::value, G = decltype(stage)::value;
        const int kb = (kb0 + j) * 64;
        if (kb + 64 > kend) {  // uniform: zero V^T past kend (8 keys per chunk, two per word)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int k8 = kb + ((t + 256 * i) & 7) * 8;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t lo = k8 + 2 * e < kend ? 0x0000FFFFu : 0u;
                    const uint32_t hi = k8 + 2 * e + 1 < kend ? 0xFFFF0000u : 0u;
                    rv[S][i][e] &= lo | hi;
                }
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4*>(lds + G * kStage + vst[i]) = rv[S][i];
    };
    // S^T of the first block for this wave's 32 keys from the K region of stage 0 (one accumulation chain over the 8
    // dim steps: the matrix core chains dependent accumulations)
    auto first_scores = [&]() __attribute__((always_inline)) {
        f32x16 sa;
#pragma unroll
        for (int r = 0; r < 16; ++r) sa[r] = 0.f;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const f16x8 a0 = as_f16x8(*reinterpret_cast<const u32x4*>(lds + krd + 32 * s));
            sa = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, qf[s], sa, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) sc[r] = sa[r];
    };
    // block j's softmax on its scores sc with the scores of block j + 1 into sn, then O^T += V^T P^T with V^T from
    // stage G
    auto softmax_pv = [&](f32x16& sn, int j, auto stage) __attribute__((always_inline)) {
        constexpr int G = decltype(stage)::value;
        const int kb = (kb0 + j) * 64;
        // causal mask, only where the key block crosses the diagonal or the tile runs past T (uniform).
        // Register r holds key kb + 32 kh + 8 (r / 4) + 4 h + r % 4.
        const bool need_mask = kb + 63 > past + row0 || row0 + kAttnRows > T;
        if (need_mask) {  // a real branch (the empty asm keeps the compiler from running the mask on every block)
            asm volatile("");
            const int lim = row < T ? past + row - kb - 32 * kh - 4 * h : -1;
#pragma unroll
            for (int r = 0; r < 16; ++r) sc[r] = (8 * (r >> 2) + (r & 3) > lim) ? -INFINITY : sc[r];
        }
        float mloc = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) mloc = fmaxf(mloc, sc[r]);
        {
            auto x = __builtin_amdgcn_permlane32_swap(__float_as_uint(mloc), __float_as_uint(mloc), false, false);
            mloc = fmaxf(__uint_as_float(x[0]), __uint_as_float(x[1]));
        }
        // The reference maximum m_run moves only when this block's maximum exceeds it by more than 8 / c (the scale
        // c > 0 is folded into the exponent: p = 2^(s c - m c), one FMA per score). A column with no visible key yet
        // keeps m_run = -inf and gets p = 0.
        const bool grow = (mloc - m_run) * scale_log2 > 8.0f;  // false for NaN (both -inf)
        if (__any(grow)) {  // wave-uniform branch
            // 1 for a column that does not grow (also one with no visible key yet: -inf - -inf would be NaN), 0 for a
            // column whose first visible keys arrive
            const float alpha = grow ? __builtin_amdgcn_exp2f((m_run - mloc) * scale_log2) : 1.0f;
            const float m_new = grow ? mloc : m_run;
            l_run *= alpha;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
            m_run = m_new;
        }
        const float mc = m_run == -INFINITY ? 0.f : m_run * scale_log2;
        // the next block's scores (K from stage 1 - G), one dim step per two of this block's exponentials: the matrix
        // core runs the chain while the VALU computes the exponentials (one basic block, ordered below)
        constexpr int GN = 1 - G;
#pragma unroll
        for (int r = 0; r < 16; ++r) sn[r] = 0.f;
        float lsum = 0.f;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const f16x8 a0 = as_f16x8(*reinterpret_cast<const u32x4*>(lds + GN * kStage + krd + 32 * s));
            sn = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, qf[s], sn, 0, 0, 0);
#pragma unroll
            for (int r = 2 * s; r < 2 * s + 2; ++r) {
                sc[r] = __builtin_amdgcn_exp2f(fmaf(sc[r], scale_log2, -mc));
                lsum += sc[r];
            }
        }
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // two K operand reads
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // the MFMA of dim step s
            if (s < 6) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // the read of step s + 2
            __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);  // two exponentials, their FMAs and sums
        }
        {
            auto x = __builtin_amdgcn_permlane32_swap(__float_as_uint(lsum), __float_as_uint(lsum), false, false);
            lsum = __uint_as_float(x[0]) + __uint_as_float(x[1]);
        }
        l_run += lsum;
        // O^T += V^T P^T over the two 16-key steps of this wave's half
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const uint32_t p0a = pack2h(sc[8 * ks], sc[8 * ks + 1]), p0b = pack2h(sc[8 * ks + 2], sc[8 * ks + 3]);
            const uint32_t p1a = pack2h(sc[8 * ks + 4], sc[8 * ks + 5]), p1b = pack2h(sc[8 * ks + 6], sc[8 * ks + 7]);
            // lane half 0 keeps keys 0-3 and takes 4-7 from lane l + 32; half 1 takes 8-11 from l - 32, keeps 12-15
            const auto xa = __builtin_amdgcn_permlane32_swap(p0a, p1a, false, false);
            const auto xb = __builtin_amdgcn_permlane32_swap(p0b, p1b, false, false);
            const f16x8 bq = as_f16x8(u32x4{xa[0], xb[0], xa[1], xb[1]});
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                const f16x8 a = as_f16x8(
                    *reinterpret_cast<const u32x4*>(lds + G * kStage + vrd + dt * 32 * kVRow + 32 * ks));
                o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bq, o[dt], 0, 0, 0);
            }
        }
    };
    using A0 = std::integral_constant<int, 0>;
    using A1 = std::integral_constant<int, 1>;
    // step j with P = j % 2: the scores of block j + 1 are taken whether or not it exists (a uniform branch here
    // would split the MFMAs from the softmax they overlap); past the item's last block they read a stale stage and
    // are discarded
    auto step = [&](auto par, int j) __attribute__((always_inline)) {
        constexpr int P = decltype(par)::value;
        using Q = std::integral_constant<int, 1 - P>;
        lds_barrier();
        if (j + 2 < nb) store_k(par, par);
        if (j + 1 < nb) store_v(par, Q{}, j + 1);
        fetch(par, j + 4);
        f32x16 sn;
        softmax_pv(sn, j, par);
#pragma unroll
        for (int r = 0; r < 16; ++r) sc[r] = sn[r];
    };

    for (int item = 0; item < nitems; ++item) {
        // the item: X's first item is its part of the long tile, its second the short tile
        int tile, role;
        if (u >= 2 * npairs) {
            tile = npairs, kb0 = 0, role = -1;  // the middle tile of an odd count
            nb = attn_tile_blocks(tile, T, past);
        } else if (u < npairs) {
            if (nitems == 2 && item == 0) tile = long_tile, kb0 = 0, nb = split_a, role = 0;
            else tile = short_tile, kb0 = 0, nb = attn_tile_blocks(short_tile, T, past), role = -1;
        } else {
            tile = long_tile, kb0 = split_a, role = split_a > 0 ? 1 : -1;
            nb = attn_tile_blocks(long_tile, T, past) - split_a;
        }
        row0 = tile * kAttnRows;
        row = row0 + c32;  // this lane's query row (its column of S^T and O^T)
        kend = past + min(row0 + kAttnRows - 1, T - 1) + 1;  // keys [0, kend) are visible to some row; kend <= max_pos

        // Q^T operand of k-step s (dims 16 s .. 16 s + 15): this lane's dims 16 s + 8 h .. + 7
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            u32x4 v = u32x4{0u, 0u, 0u, 0u};
            if (row < T) v = *reinterpret_cast<const u32x4*>(q + size_t(row) * QC + head * 128 + 16 * s + 8 * h);
            qf[s] = as_f16x8(v);
        }
        m_run = -INFINITY, l_run = 0.f;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[dt][r] = 0.f;

        {  // group 0 is K(0) alone (its V^T(-1) does not exist)
            const int kbk = kb0 * 64;
#pragma unroll
            for (int i = 0; i < 4; ++i) rk[0][i] = __builtin_amdgcn_raw_buffer_load_b128(k_rsrc, koff[i], kbk * 256, 0);
        }
        __builtin_amdgcn_sched_barrier(0);  // group 0 issues before group 1, so the first wait can be partial
        fetch(A1{}, 1);
        store_k(A0{}, A0{});     // K(0)
        store_k(A1{}, A1{});     // K(1) (K(0) again when the item has one block: never read)
        store_v(A1{}, A0{}, 0);  // V^T(0)
        fetch(A0{}, 2);
        __builtin_amdgcn_sched_barrier(0);
        fetch(A1{}, 3);
        lds_barrier();
        first_scores();
        for (int j = 0;; j += 2) {
            step(A0{}, j);
            if (j + 1 >= nb) break;
            step(A1{}, j + 1);
            if (j + 2 >= nb) break;
        }

        // merge the key halves: waves 2 and 3 hand (m, l, O^T) to waves 0 and 1 (same head) through LDS
        lds_barrier();  // every wave is done with both stages
        float* xo = reinterpret_cast<float*>(lds) + cg * 4224;  // per head: 64 x 64 O words, then m and l per lane
        if (kh == 1) {
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4)
                    *reinterpret_cast<f32x4*>(xo + ((dt * 4 + r4) * 64 + lane) * 4) =
                        f32x4{o[dt][4 * r4], o[dt][4 * r4 + 1], o[dt][4 * r4 + 2], o[dt][4 * r4 + 3]};
            xo[4096 + lane] = m_run;
            xo[4160 + lane] = l_run;
        }
        lds_barrier();
        uint16_t* yr = y + size_t(row) * QC + head * 128;
        if (role < 0) {
            if (kh == 0 && row < T) {
                const float m1 = xo[4096 + lane], l1 = xo[4160 + lane];
                const float M = fmaxf(m_run, m1);
                const float Mc = M == -INFINITY ? 0.f : M * scale_log2;
                const float e0 = __builtin_amdgcn_exp2f(m_run * scale_log2 - Mc);
                const float e1 = __builtin_amdgcn_exp2f(m1 * scale_log2 - Mc);
                const float inv = 1.0f / (l_run * e0 + l1 * e1);
                const float f0 = e0 * inv, f1 = e1 * inv;
                uint32_t bad = 0;
#pragma unroll
                for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                    for (int r4 = 0; r4 < 4; ++r4) {
                        const f32x4 b = *reinterpret_cast<const f32x4*>(xo + ((dt * 4 + r4) * 64 + lane) * 4);
                        uint2 v;
                        v.x = pack2h(o[dt][4 * r4] * f0 + b[0] * f1, o[dt][4 * r4 + 1] * f0 + b[1] * f1);
                        v.y = pack2h(o[dt][4 * r4 + 2] * f0 + b[2] * f1, o[dt][4 * r4 + 3] * f0 + b[3] * f1);
                        bad |= f16_bad2(v.x) | f16_bad2(v.y);
                        // register r of tile dt: dim 32 dt + 8 (r / 4) + 4 h + r % 4
                        *reinterpret_cast<uint2*>(yr + 32 * dt + 8 * r4 + 4 * h) = v;
                    }
                f16_note(bad, kF16Attn);
            }
        } else {
            // this part of a split tile: waves 0 and 1 fold the key halves into (O^T, m, l) of their head
            if (kh == 0) {
                const float m1 = xo[4096 + lane], l1 = xo[4160 + lane];
                const float M = fmaxf(m_run, m1);
                const float Mc = M == -INFINITY ? 0.f : M * scale_log2;
                const float e0 = __builtin_amdgcn_exp2f(m_run * scale_log2 - Mc);
                const float e1 = __builtin_amdgcn_exp2f(m1 * scale_log2 - Mc);
#pragma unroll
                for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                    for (int r4 = 0; r4 < 4; ++r4) {
                        const f32x4 b = *reinterpret_cast<const f32x4*>(xo + ((dt * 4 + r4) * 64 + lane) * 4);
#pragma unroll
                        for (int e = 0; e < 4; ++e) o[dt][4 * r4 + e] = o[dt][4 * r4 + e] * e0 + b[e] * e1;
                    }
                l_run = l_run * e0 + l1 * e1;
                m_run = M;
            }
            const int pid = kvhead * npairs + pair;
            uint32_t* ctr = ws + size_t(pid) * attn_prefill::kRecordWords;
            float* slots = reinterpret_cast<float*>(ctr + 64);
            float* mine = slots + role * kAttnSlotWords + cg * 4096;
            const float* other = slots + (1 - role) * kAttnSlotWords + cg * 4096;
            float* mine_ml = slots + role * kAttnSlotWords + 8192 + cg * 128;
            const float* other_ml = slots + (1 - role) * kAttnSlotWords + 8192 + cg * 128;
            if (t == 0) s_flag = int(__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
            lds_barrier();
            int arrived = s_flag;
            if (!arrived) {
                // store this part (device-scope stores: the other part may run on another XCD), wait until they are
                // performed, then count this part in
                if (kh == 0) {
#pragma unroll
                    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                        for (int r4 = 0; r4 < 4; ++r4) {
                            uint64_t* d = reinterpret_cast<uint64_t*>(mine + ((dt * 4 + r4) * 64 + lane) * 4);
                            __hip_atomic_store(d, uint64_t(__float_as_uint(o[dt][4 * r4])) |
                                                      (uint64_t(__float_as_uint(o[dt][4 * r4 + 1])) << 32),
                                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                            __hip_atomic_store(d + 1, uint64_t(__float_as_uint(o[dt][4 * r4 + 2])) |
                                                          (uint64_t(__float_as_uint(o[dt][4 * r4 + 3])) << 32),
                                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        }
                    __hip_atomic_store(reinterpret_cast<uint32_t*>(mine_ml) + lane, __float_as_uint(m_run),
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(reinterpret_cast<uint32_t*>(mine_ml) + 64 + lane, __float_as_uint(l_run),
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0): this wave's stores are performed
                lds_barrier();
                if (t == 0)
                    s_flag = int(__hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
                lds_barrier();
                arrived = s_flag;
            }
            if (arrived) {
                // the other part is stored: merge in X, Y order and write the rows
                if (kh == 0 && row < T) {
                    float Ob[64];
#pragma unroll
                    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                        for (int r4 = 0; r4 < 4; ++r4) {
                            const uint64_t* sp = reinterpret_cast<const uint64_t*>(
                                other + ((dt * 4 + r4) * 64 + lane) * 4);
                            const uint64_t v0 = __hip_atomic_load(sp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                            const uint64_t v1 = __hip_atomic_load(sp + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                            Ob[(dt * 4 + r4) * 4 + 0] = __uint_as_float(uint32_t(v0));
                            Ob[(dt * 4 + r4) * 4 + 1] = __uint_as_float(uint32_t(v0 >> 32));
                            Ob[(dt * 4 + r4) * 4 + 2] = __uint_as_float(uint32_t(v1));
                            Ob[(dt * 4 + r4) * 4 + 3] = __uint_as_float(uint32_t(v1 >> 32));
                        }
                    const float mo = __uint_as_float(__hip_atomic_load(
                        reinterpret_cast<const uint32_t*>(other_ml) + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
                    const float lo = __uint_as_float(__hip_atomic_load(
                        reinterpret_cast<const uint32_t*>(other_ml) + 64 + lane, __ATOMIC_RELAXED,
                        __HIP_MEMORY_SCOPE_AGENT));
                    // (mx, lx) of part X and (my, ly) of part Y
                    const float mx = role == 0 ? m_run : mo, lx = role == 0 ? l_run : lo;
                    const float my = role == 0 ? mo : m_run, ly = role == 0 ? lo : l_run;
                    const float M = fmaxf(mx, my);
                    const float Mc = M == -INFINITY ? 0.f : M * scale_log2;
                    const float ex = __builtin_amdgcn_exp2f(mx * scale_log2 - Mc);
                    const float ey = __builtin_amdgcn_exp2f(my * scale_log2 - Mc);
                    const float inv = 1.0f / (lx * ex + ly * ey);
                    const float fx = ex * inv, fy = ey * inv;
                    uint32_t bad = 0;
#pragma unroll
                    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                        for (int r4 = 0; r4 < 4; ++r4) {
                            float vv[4];
#pragma unroll
                            for (int e = 0; e < 4; ++e) {
                                const float om = o[dt][4 * r4 + e], ob = Ob[(dt * 4 + r4) * 4 + e];
                                vv[e] = role == 0 ? om * fx + ob * fy : ob * fx + om * fy;
                            }
                            uint2 v;
                            v.x = pack2h(vv[0], vv[1]);
                            v.y = pack2h(vv[2], vv[3]);
                            bad |= f16_bad2(v.x) | f16_bad2(v.y);
                            *reinterpret_cast<uint2*>(yr + 32 * dt + 8 * r4 + 4 * h) = v;
                        }
                    f16_note(bad, kF16Attn);
                }
                if (t == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        lds_barrier();  // the next item's stores reuse the LDS of this one's merge
    }
}

// ================================================================ decode kernels (one token per step)
// The step state is device memory, for B sequences: state[b] = the position sequence b decodes, state[B + b] = its
// token id, state[2 B] = the step index (B = 1: position, id, step). The argmax kernel writes the next ids and advances
// the state, so a recorded step replays unchanged.
//
// The GEMVs give each wave whole rows and keep every wave independent (no LDS, no barrier): lane l covers the
// k-chunks 512 c + 8 l .. + 7, c < NCH, and issues the loads of all its weight chunks and of its slice of the input
// vector together, so the memory latency is paid once per kernel; the RMSNorm sum of squares and the dot products
// are then reduced with wave shuffles (every wave holds the whole input vector, 8 values per lane per chunk).

constexpr int kMaxHidden = 8192;

template <int NCH>
__device__ __forceinline__ void load_chunks_f32(const float* x, int K, float (&v)[NCH][8]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int k0 = 512 * c + 8 * lane;
        float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
        if (k0 < K) {
            a = *reinterpret_cast<const float4*>(x + k0);
            b = *reinterpret_cast<const float4*>(x + k0 + 4);
        }
        v[c][0] = a.x, v[c][1] = a.y, v[c][2] = a.z, v[c][3] = a.w;
        v[c][4] = b.x, v[c][5] = b.y, v[c][6] = b.z, v[c][7] = b.w;
    }
}

template <int NCH>
__device__ __forceinline__ void load_chunks_16(const uint16_t* row, int K, uint4 (&w)[NCH]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int k0 = 512 * c + 8 * lane;
        w[c] = k0 < K ? *reinterpret_cast<const uint4*>(row + k0) : make_uint4(0, 0, 0, 0);
    }
}

// v <- widen(nw) * (v * r), r = 1 / sqrt(sum(v^2) / K + eps): the RMSNorm of the whole vector (padding lanes hold 0).
template <int NCH>
__device__ __forceinline__ void rmsnorm_chunks(float (&v)[NCH][8], const uint4 (&nw)[NCH], int K, float eps) {
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = fmaf(v[c][e], v[c][e], ss);
    ss = wave_sum(ss);
    const float r = 1.0f / sqrtf(ss / float(K) + eps);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        float g[8];
        unpack8(nw[c], g);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[c][e] = g[e] * (v[c][e] * r);
    }
}

// The dot product of a bf16 row (in chunks) with the vector v, reduced over the wave.
template <int NCH>
__device__ __forceinline__ float dot_chunks(const uint4 (&w)[NCH], const float (&v)[NCH][8]) {
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        float f[8];
        unpack8(w[c], f);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc = fmaf(f[e], v[c][e], acc);
    }
    return wave_sum(acc);
}

// ---------------------------------------------------------------- 20 gemv_norm_dec: y[n] = w[n] . RMSNorm(x)
template <int NCH>
__global__ __launch_bounds__(256) void k_gemv_norm_dec(const float* x, const uint16_t* nw, const uint16_t* w, float* y,
                                                       int n, int k, float eps) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n) return;
    uint4 wv[NCH], g[NCH];
    float xv[NCH][8];
    load_chunks_16<NCH>(w + size_t(row) * k, k, wv);
    load_chunks_f32<NCH>(x, k, xv);
    load_chunks_16<NCH>(nw, k, g);
    rmsnorm_chunks<NCH>(xv, g, k, eps);
    const float out = dot_chunks<NCH>(wv, xv);
    if ((threadIdx.x & 63) == 0) y[row] = out;
}

// ---------------------------------------------------------------- 21 attention_decode_f16
// Split-KV decode attention over positions 0 .. pos = state[b]. Block (s, kv head, b) takes keys [64 C s, 64 C s +
// 64 C) for the two query heads of the group, 64 keys at a time. C = chunks per split: given by the caller (1 for one
// sequence, whose splits are its only parallelism), or, with chunks = 0, the fewest that cover 0 .. pos in the grid's
// S splits, C = ceil((pos + 1) / 64 S): every sequence's keys then spread evenly over its S blocks, so a grid sized to
// one round of resident blocks ends with them all instead of a partly filled last round. It loads the raw projections,
// issues the loads of its first two chunks, then applies the q RMSNorm and RoPE; the block whose split holds pos also
// computes the
// new key (k RMSNorm + RoPE) and value, appends them (fp16) to the caches and uses the same rounded values in place
// of the stale slot it loaded. Per chunk: scores (each key's dot over 16 lanes), an online softmax per head in the log2
// domain, and P V accumulated per thread (its 4 dims x 8 keys, rescaled when the maximum moves), with the chunk two
// ahead loading meanwhile; the 8 key groups are reduced once at the end. Each block writes, per head, (max, sum,
// unnormalised output[128]); splits past pos do nothing. Positions past pos are loaded (they lie inside max_pos) but
// masked by selects: the scores to -inf, the values to 0 (unwritten positions may hold anything).
// Every barrier orders LDS only (lds_barrier): a __syncthreads() would also wait for the chunks in flight, so each
// chunk would drain the next one's loads at its first barrier.
// MULTI = false is the one-chunk form (chunks == 1): 256 threads, no second register set and no loop, so the
// registers stay low enough for many blocks per CU, which the one-sequence decode needs (its splits are its only
// parallelism). MULTI = true streams chunks with 512 threads: a chunk's scores and P V spread over 8 waves, halving
// each wave's share of the per-chunk chain (scores, softmax, P V, two barriers) that bounds a block's rate.
template <bool MULTI>
__global__ __launch_bounds__(MULTI ? 512 : 256) void k_attn_dec(const float* qkv, const uint16_t* qn,
                                                                const uint16_t* kn, const float* cos_t,
                                                                const float* sin_t, uint16_t* kc, uint16_t* vc,
                                                                float* part, const uint32_t* state, int qh, int kvh,
                                                                int max_pos, float eps, float scale_log2, int chunks) {
    // waves per block; keys per wave and 4-key rows per thread for the scores; V^T row groups and rows per thread
    constexpr int NT = MULTI ? 512 : 256, NW = NT / 64, ITS = 64 / NW / 4, RG = NT / 8, DD = 128 / RG;
    __shared__ float qs[2][128];
    __shared__ float knew[128];
    __shared__ float vnew[128];
    __shared__ float ps[2][2][64];  // [chunk parity][query head][key]
    __shared__ float alpha_s[2][2];
    __shared__ float redq[4], redk[4];
    const int s = blockIdx.x, S = gridDim.x, kvhead = blockIdx.y, t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int b = blockIdx.z;  // the sequence: its projections, caches and partials follow the previous ones
    const int pos = int(state[b]);
    // the raw projections and the norm weights need no position: their loads go out while the position's load is in
    // flight (threads 0 .. 255 use them; the rest wait at the barriers; 4308 -> 4324 tok/s at 1.7B, 16 x 8K)
    const int hh = (t >> 7) & 1, d = t & 127;  // thread t: q head 2 kvhead + hh; new key (hh = 0) or value (hh = 1)
    const bool pro = t < 256;
    const int QC = qh * 128, KC = kvh * 128;
    qkv += size_t(b) * (qh + 2 * kvh) * 128;
    const float qv = qkv[(kvhead * 2 + hh) * 128 + d];
    const float kvv = qkv[QC + hh * KC + kvhead * 128 + d];
    const uint16_t qwb = qn[d], kwb = kn[d];
    __builtin_amdgcn_sched_barrier(0);
    if (pos < 0 || pos >= max_pos) return;  // the host keeps decode inside max_pos; never touch memory past the cache
    kc += size_t(b) * kvh * max_pos * 128;
    vc += size_t(b) * kvh * 128 * max_pos;
    part += size_t(b) * qh * S * 130;
    const int ck = chunks > 0 ? chunks : (pos + 64 * S) / (64 * S);  // chunks per split of this sequence
    const int key0 = s * 64 * ck;
    const int nkeys = min(64 * ck, pos + 1 - key0);  // keys of this split at or before pos
    if (nkeys <= 0) return;
    const int nch = (nkeys + 63) / 64;  // chunks to run; the last one ends inside max_pos (a multiple of 64)
    const bool has_pos = pos < key0 + 64 * ck;  // uniform over the block
    const int jnew = pos - key0;                 // the new key's offset in the split when has_pos

    // thread mapping: K as ITS keys (wv * 4 ITS + it * 4 + lane / 16) x 8 dims (d0); V^T as DD dims (rg + RG dd) x 8
    // keys (8 sub ..)
    const int d0 = 8 * (lane & 15), sub = t & 7, rg = t >> 3;
    const uint16_t* kb = kc + (size_t(kvhead) * max_pos + key0) * 128 + d0;
    const uint16_t* vb = vc + size_t(kvhead) * 128 * max_pos + sub * 8;  // + the chunk's block, + dim 64
    u32x4 kv4[2][ITS], vv[2][DD];
    // The streaming form loads K and V^T non-temporally: a batched step streams every sequence's cache once (1.7B,
    // 16 sequences x 8K: 537 MB per layer), far past what the last-level cache could keep for the next step, and the
    // streaming hint keeps it from filling that cache (4063 -> 4286 tok/s there). The one-chunk form's caches (one
    // sequence) can stay cached between steps.
    auto ld = [&](const uint16_t* p) __attribute__((always_inline)) {
        const u32x4* v = reinterpret_cast<const u32x4*>(p);
        if constexpr (MULTI)
            return __builtin_nontemporal_load(v);
        else
            return *v;
    };
    auto fetch = [&](auto set, int c) __attribute__((always_inline)) {
        constexpr int SET = decltype(set)::value;
        c = min(c, nch - 1) * 64;  // past the last chunk: re-read it (an L2 hit, never used)
#pragma unroll
        for (int it = 0; it < ITS; ++it) kv4[SET][it] = ld(kb + size_t(c + wv * 4 * ITS + it * 4 + (lane >> 4)) * 128);
#pragma unroll
        for (int dd = 0; dd < DD; ++dd) vv[SET][dd] = ld(vb + kv::v_at(key0 + c, rg + RG * dd));
    };
    using C0 = std::integral_constant<int, 0>;
    using C1 = std::integral_constant<int, 1>;

    // the rotation of pos, loaded (with the projections above) ahead of the first chunks: loads return in issue order,
    // so the norm, rotation and append below run while the chunks are in flight instead of after they land (1.7B, 16
    // sequences x 8K: 4283 -> 4310 tok/s)
    const float cs = cos_t[size_t(pos) * 64 + (d & 63)], sn = sin_t[size_t(pos) * 64 + (d & 63)];
    __builtin_amdgcn_sched_barrier(0);
    fetch(C0{}, 0);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (MULTI) {
        fetch(C1{}, 1);
        __builtin_amdgcn_sched_barrier(0);
    }
    const float qw = bf2f(qwb), kw = bf2f(kwb);

    // per-head RMSNorm (head hh = waves 2 hh, 2 hh + 1; the new key = waves 0, 1), then the rotation of (d, d + 64)
    const float sq = wave_sum(qv * qv), sk = wave_sum(kvv * kvv);
    if (lane == 0 && pro) {
        redq[wv] = sq;
        redk[wv] = sk;
    }
    lds_barrier();
    const float qr = qw * (qv * (1.0f / sqrtf((redq[2 * hh] + redq[2 * hh + 1]) / 128.0f + eps)));
    const float kr = kw * (kvv * (1.0f / sqrtf((redk[0] + redk[1]) / 128.0f + eps)));
    if (pro) {
        qs[hh][d] = qr;
        if (hh == 0) knew[d] = kr;
    }
    lds_barrier();
    const float qrot = d < 64 ? qr * cs - qs[hh][d + 64] * sn : qr * cs + qs[hh][d - 64] * sn;
    const float krot = d < 64 ? kr * cs - knew[d + 64] * sn : kr * cs + knew[d - 64] * sn;
    lds_barrier();
    if (pro) {
        qs[hh][d] = qrot;
        if (has_pos) {
            if (hh == 0) {
                const uint16_t kh = f2h(krot);
                knew[d] = h2f(kh);
                kc[(size_t(kvhead) * max_pos + pos) * 128 + d] = kh;
                f16_note(f16_bad2(kh), kF16Cache);
            } else {
                const uint16_t vh = f2h(kvv);
                vnew[d] = h2f(vh);
                vc[size_t(kvhead) * 128 * max_pos + kv::v_at(pos, d)] = vh;
                f16_note(f16_bad2(vh), kF16Cache);
            }
        }
    }
    lds_barrier();
    // this thread's query dims and, for the split holding pos, its slices of the new key and value (read
    // unconditionally, used only through selects: a conditional LDS read would become a branch per element)
    float q0[8], q1[8], kn8[8], vnd[DD];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        q0[e] = qs[0][d0 + e];
        q1[e] = qs[1][d0 + e];
        kn8[e] = knew[d0 + e];
    }
#pragma unroll
    for (int dd = 0; dd < DD; ++dd) vnd[dd] = vnew[rg + RG * dd];

    float m_run = -INFINITY, l_run = 0.f;  // waves 0 and 1: the running statistics of head wv
    float o0[DD], o1[DD];
#pragma unroll
    for (int dd = 0; dd < DD; ++dd) o0[dd] = o1[dd] = 0.f;
    // masked keys (past pos) and the new key (= pos, when this split holds it) lie in the split's last chunk only:
    // TAIL instantiates the selects for it, the other chunks run without them
    auto chunk = [&](auto set, auto tailc, int c) __attribute__((always_inline)) {
        constexpr int SET = decltype(set)::value;
        constexpr bool tail = decltype(tailc)::value;
        const int cb = c * 64;  // the chunk's first key, as an offset in the split
        // scores of the chunk's keys for both heads
#pragma unroll
        for (int it = 0; it < ITS; ++it) {
            const int key = wv * 4 * ITS + it * 4 + (lane >> 4);
            float kf[8];
            unpack8h(kv4[SET][it], kf);
            if constexpr (tail) {
                const bool is_new = has_pos && cb + key == jnew;
#pragma unroll
                for (int e = 0; e < 8; ++e) kf[e] = is_new ? kn8[e] : kf[e];
            }
            float a0 = 0.f, a1 = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                a0 = fmaf(q0[e], kf[e], a0);
                a1 = fmaf(q1[e], kf[e], a1);
            }
            a0 = row_sum16(a0);
            a1 = row_sum16(a1);
            if ((lane & 15) == 0) {
                const bool ok = !tail || cb + key < nkeys;
                ps[SET][0][key] = ok ? a0 * scale_log2 : -INFINITY;
                ps[SET][1][key] = ok ? a1 * scale_log2 : -INFINITY;
            }
        }
        lds_barrier();
        if (wv < 2) {  // online softmax of head wv over this chunk (key 0 of a chunk is always valid)
            const float v = ps[SET][wv][lane];
            const float m_new = fmaxf(m_run, wave_max(v));
            const float e = exp2f(v - m_new);
            const float al = exp2f(m_run - m_new);  // 0 on the first chunk
            l_run = l_run * al + wave_sum(e);
            m_run = m_new;
            ps[SET][wv][lane] = e;
            if (lane == 0) alpha_s[SET][wv] = al;
        }
        lds_barrier();
        // P V: thread t covers V^T rows rg + RG dd and keys 8 sub .. + 7 of the chunk
        float e0[8], e1[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            e0[e] = ps[SET][0][sub * 8 + e];
            e1[e] = ps[SET][1][sub * 8 + e];
        }
        const float al0 = alpha_s[SET][0], al1 = alpha_s[SET][1];
#pragma unroll
        for (int dd = 0; dd < DD; ++dd) {
            float vf[8];
            unpack8h(vv[SET][dd], vf);
            if constexpr (tail) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int key = cb + sub * 8 + e;
                    vf[e] = key >= nkeys ? 0.f : (has_pos && key == jnew ? vnd[dd] : vf[e]);
                }
            }
            float a0 = 0.f, a1 = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                a0 = fmaf(e0[e], vf[e], a0);
                a1 = fmaf(e1[e], vf[e], a1);
            }
            o0[dd] = fmaf(o0[dd], al0, a0);
            o1[dd] = fmaf(o1[dd], al1, a1);
        }
        // the accumulators materialise here: otherwise the compiler sinks this P V into the next chunk, the refilled
        // V^T registers need other registers, and the loop's end copies them back, waiting for their loads (4331 ->
        // 4338 tok/s at 1.7B, 16 x 8K)
#pragma unroll
        for (int dd = 0; dd < DD; ++dd) asm volatile("" : "+v"(o0[dd]), "+v"(o1[dd]));
        // no barrier before the next chunk: it writes the other parity's ps and alpha_s, and the chunk after it
        // writes these only past its first barrier, which every wave reaches after this P V
    };
    using Body = std::false_type;
    using Tail = std::true_type;
    if constexpr (!MULTI) {
        chunk(C0{}, Tail{}, 0);
    } else {
        int c = 0;
        for (; c + 2 < nch; c += 2) {  // whole pairs before the last chunk: the loop head has set 0 as the older load
            chunk(C0{}, Body{}, c);
            fetch(C0{}, c + 2);
            __builtin_amdgcn_sched_barrier(0);
            chunk(C1{}, Body{}, c + 1);
            fetch(C1{}, c + 3);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (c + 1 < nch) {  // two chunks left (set 0, set 1), the second the last
            chunk(C0{}, Body{}, c);
            chunk(C1{}, Tail{}, c + 1);
        } else {
            chunk(C0{}, Tail{}, c);
        }
    }

    // reduce the 8 key groups (lanes differing in t & 7) and write the partials
    float* myp = part + (size_t(kvhead * 2) * S + s) * 130;  // head 2 kvhead + hh at + hh * S * 130
#pragma unroll
    for (int dd = 0; dd < DD; ++dd) {
        float a0 = o0[dd], a1 = o1[dd];
#pragma unroll
        for (int o = 1; o < 8; o <<= 1) {
            a0 += __shfl_xor(a0, o, 64);
            a1 += __shfl_xor(a1, o, 64);
        }
        if (sub == 0) {
            myp[2 + rg + RG * dd] = a0;
            myp[size_t(S) * 130 + 2 + rg + RG * dd] = a1;
        }
    }
    if (wv < 2 && lane == 0) {
        myp[size_t(wv) * S * 130] = m_run;
        myp[size_t(wv) * S * 130 + 1] = l_run;
    }
}

// ---------------------------------------------------------------- 22 attention_combine
// y[h, d] = sum_s 2^(m_s - M) o_s[d] / sum_s 2^(m_s - M) l_s over the splits that hold keys; one block per head, the
// splits spread over the threads (every load of a pass is independent of the others). split_keys = 0: the splits of
// each sequence are the even ones of attention_decode_f16 with chunks = 0, 64 ceil((pos + 1) / 64 splits) keys each.
constexpr int kMaxSplits = 1024;
template <typename OUT>
__global__ __launch_bounds__(256) void k_attn_combine(const float* part, OUT* y, const uint32_t* state, int splits,
                                                      int split_keys, int max_pos) {
    __shared__ float sc[kMaxSplits];
    __shared__ float red[4];
    __shared__ float o_hi[128];
    const int h = blockIdx.x, b = blockIdx.y, t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const float* hp = part + (size_t(b) * gridDim.x + h) * splits * 130;
    const int d = t & 127, par = t >> 7;  // dim d over the splits of parity par
    // split t's (max, sum) and this thread's first PF output values of any split of the grid, loaded with the
    // position (one memory round instead of four: 3.36 -> 2.84 us per launch in the one-sequence decode, whose
    // kernel list then runs 1268 -> 1303 tok/s); those of splits without keys are never used
    constexpr int PF = 4;
    const float m0 = t < splits ? hp[size_t(t) * 130] : -INFINITY;
    const float l0 = t < splits ? hp[size_t(t) * 130 + 1] : 0.f;
    float ov[PF];
#pragma unroll
    for (int j = 0; j < PF; ++j) ov[j] = par + 2 * j < splits ? hp[size_t(par + 2 * j) * 130 + 2 + d] : 0.f;
    const int pos = int(state[b]);
    if (pos < 0 || pos >= max_pos) return;
    const int sk = split_keys > 0 ? split_keys : 64 * ((pos + 64 * splits) / (64 * splits));
    const int used = min(pos / sk + 1, splits);
    const bool own = t < used;
    float m = fmaxf(-INFINITY, own ? m0 : -INFINITY);
    for (int i = t + 256; i < used; i += 256) m = fmaxf(m, hp[size_t(i) * 130]);
    m = wave_max(m);
    if (lane == 0) red[wv] = m;
    __syncthreads();
    const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float l = 0.f;
    if (own) {
        const float e = exp2f(m0 - M);
        sc[t] = e;
        l = fmaf(l0, e, l);
    }
    for (int i = t + 256; i < used; i += 256) {
        const float e = exp2f(hp[size_t(i) * 130] - M);
        sc[i] = e;
        l = fmaf(hp[size_t(i) * 130 + 1], e, l);
    }
    l = wave_sum(l);
    if (lane == 0) red[wv] = l;
    __syncthreads();
    const float L = (red[0] + red[1]) + (red[2] + red[3]);
    float o = 0.f;
    int i = par;
#pragma unroll
    for (int j = 0; j < PF; ++j, i += 2)
        if (i < used) o = fmaf(ov[j], sc[i], o);
#pragma unroll 4
    for (; i < used; i += 2) o = fmaf(hp[size_t(i) * 130 + 2 + d], sc[i], o);
    if (par == 1) o_hi[d] = o;
    __syncthreads();
    if (par == 0) {
        const float v = (o + o_hi[d]) / L;
        OUT* yo = y + (size_t(b) * gridDim.x + h) * 128 + d;
        if constexpr (sizeof(OUT) == 4) {
            *yo = v;
        } else {
            const uint16_t hv = f2h(v);
            f16_note(f16_bad2(hv), kF16Attn);
            *yo = hv;
        }
    }
}

// ---------------------------------------------------------------- 23 gemv_residual_dec: x[n] += w[n] . a
template <int NCH>
__global__ __launch_bounds__(256) void k_gemv_resid_dec(const float* a, const uint16_t* w, float* x, int n, int k) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n) return;
    uint4 wv[NCH];
    float av[NCH][8];
    load_chunks_16<NCH>(w + size_t(row) * k, k, wv);
    load_chunks_f32<NCH>(a, k, av);
    const float out = dot_chunks<NCH>(wv, av);
    if ((threadIdx.x & 63) == 0) x[row] += out;
}

// ---------------------------------------------------------------- 24 gemv_swiglu_dec: a[j] = silu(g_j . h) * (u_j . h)
template <int NCH>
__global__ __launch_bounds__(256) void k_gemv_swiglu_dec(const float* x, const uint16_t* nw, const uint16_t* w,
                                                         float* y, int inter, int hidden, float eps) {
    const int j = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (j >= inter) return;
    uint4 wg[NCH], wu[NCH], g[NCH];
    float xv[NCH][8];
    load_chunks_16<NCH>(w + size_t(j) * hidden, hidden, wg);
    load_chunks_16<NCH>(w + size_t(inter + j) * hidden, hidden, wu);
    load_chunks_f32<NCH>(x, hidden, xv);
    load_chunks_16<NCH>(nw, hidden, g);
    rmsnorm_chunks<NCH>(xv, g, hidden, eps);
    const float gv = dot_chunks<NCH>(wg, xv);
    const float uv = dot_chunks<NCH>(wu, xv);
    if ((threadIdx.x & 63) == 0) y[j] = gv / (1.0f + __expf(-gv)) * uv;
}

// ---------------------------------------------------------------- 25 lmhead_dec
// logits[n] = RMSNorm(x) . E[n] (the tied embedding), rows split evenly over the blocks, 4 rows per wave at a time;
// each block writes its (max, lowest index) pair to partials, index 0xFFFFFFFE when one of its logits is NaN.
constexpr uint32_t kLmheadBlocks = 1024;
template <int NCH>
__global__ __launch_bounds__(256) void k_lmhead_dec(const float* x, const uint16_t* nw, const uint16_t* e, float* logits,
                                                    float* part, int vocab, int hidden, float eps, int write_logits) {
    __shared__ float bv[4];
    __shared__ uint32_t bi[4];
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int per_block = (vocab + int(gridDim.x) - 1) / int(gridDim.x);
    const int r0 = int(blockIdx.x) * per_block, r1 = min(vocab, r0 + per_block);
    float xv[NCH][8];
    {
        uint4 g[NCH];
        load_chunks_f32<NCH>(x, hidden, xv);
        load_chunks_16<NCH>(nw, hidden, g);
        rmsnorm_chunks<NCH>(xv, g, hidden, eps);
    }
    float best = -INFINITY;
    uint32_t besti = 0xFFFFFFFFu;
    bool nan = false;
    for (int row = r0 + wv * 4; row < r1; row += 16) {
        uint4 w4[4][NCH];
#pragma unroll
        for (int r = 0; r < 4; ++r) load_chunks_16<NCH>(e + size_t(min(row + r, vocab - 1)) * hidden, hidden, w4[r]);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float v = dot_chunks<NCH>(w4[r], xv);
            if (row + r >= r1) continue;
            if (write_logits && lane == r) logits[row + r] = v;
            if (v != v) {
                nan = true;
            } else if (besti == 0xFFFFFFFFu || v > best) {  // each wave visits its rows in increasing order
                best = v;
                besti = uint32_t(row + r);
            }
        }
    }
    if (lane == 0) {
        bv[wv] = best;
        bi[wv] = nan ? 0xFFFFFFFEu : besti;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float b = 0.f;
        uint32_t ix = 0xFFFFFFFFu;
        bool bn = false;
        for (int i = 0; i < 4; ++i) {
            if (bi[i] == 0xFFFFFFFEu)
                bn = true;
            else if (bi[i] != 0xFFFFFFFFu && (ix == 0xFFFFFFFFu || bv[i] > b || (bv[i] == b && bi[i] < ix))) {
                b = bv[i];
                ix = bi[i];
            }
        }
        part[2 * blockIdx.x] = b;
        reinterpret_cast<uint32_t*>(part)[2 * blockIdx.x + 1] = bn ? 0xFFFFFFFEu : ix;
    }
}

// ---------------------------------------------------------------- 26 argmax_dec
// The row's argmax from the lm_head partials (lowest index of the maximum; 0xFFFFFFFF when a logit is NaN), recorded
// in out_ids[state[2]] and fed back as the next step's token: state[0] += 1, state[1] = id, state[2] += 1.
__global__ __launch_bounds__(1024) void k_argmax_dec(const float* part, uint32_t* state, uint32_t* out_ids, int blocks,
                                                     int max_steps) {
    __shared__ float sv[1024];
    __shared__ uint32_t si[1024];
    __shared__ int snan;
    const int t = threadIdx.x;
    if (t == 0) snan = 0;
    __syncthreads();
    float best = 0.f;
    uint32_t bi = 0xFFFFFFFFu;
    bool nan = false;
    for (int i = t; i < blocks; i += 1024) {
        const float v = part[2 * i];
        const uint32_t j = reinterpret_cast<const uint32_t*>(part)[2 * i + 1];
        if (j == 0xFFFFFFFEu)
            nan = true;
        else if (j != 0xFFFFFFFFu && (bi == 0xFFFFFFFFu || v > best || (v == best && j < bi))) {
            best = v;
            bi = j;
        }
    }
    if (nan) snan = 1;  // every writer stores the same value
    sv[t] = best;
    si[t] = bi;
    __syncthreads();
    for (int s = 512; s > 0; s >>= 1) {
        if (t < s) {
            const float ov = sv[t + s];
            const uint32_t oi = si[t + s];
            if (oi != 0xFFFFFFFFu && (si[t] == 0xFFFFFFFFu || ov > sv[t] || (ov == sv[t] && oi < si[t]))) {
                sv[t] = ov;
                si[t] = oi;
            }
        }
        __syncthreads();
    }
    if (t == 0) {
        const uint32_t id = snan ? 0xFFFFFFFFu : si[0];
        const uint32_t step = state[2];
        if (step < uint32_t(max_steps)) out_ids[step] = id;
        state[1] = id;
        state[0] = state[0] + 1u;
        state[2] = step + 1u;
    }
}

// ---------------------------------------------------------------- 27 embed_dec: x[b] = widen(E[state.id[b]])
__global__ __launch_bounds__(256) void k_embed_dec(const uint16_t* e, const uint32_t* state, float* x, int hidden,
                                                   int vocab) {
    const int b = blockIdx.x;
    const uint32_t id = state[gridDim.x + b];
    float* xb = x + size_t(b) * hidden;
    for (int c = threadIdx.x; c < hidden; c += 256)
        xb[c] = id < uint32_t(vocab) ? bf2f(e[size_t(id) * hidden + c]) : __uint_as_float(0x7FC00000u);
}

// ---------------------------------------------------------------- 28 fill_normal_f16 (synthetic caches)
// y[i] = f16(bf16(std * N(0, 1))) from a counter-based normal: splitmix64 of (seed, stream, i / 2), Box-Muller.
__device__ __forceinline__ uint64_t splitmix(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
__global__ void k_fill_normal(uint16_t* y, uint64_t n, uint64_t seed, uint64_t stream, float std) {
    const uint64_t i = (uint64_t(blockIdx.x) * blockDim.x + threadIdx.x) * 2;
    if (i >= n) return;
    const uint64_t h = splitmix(seed ^ splitmix(stream ^ splitmix(i >> 1)));
    const double u1 = (double((h >> 11) & ((1ull << 26) - 1)) + 0.5) / double(1ull << 26);
    const double u2 = double(h >> 38) / double(1ull << 26);
    const double r = sqrt(-2.0 * log(u1));
    y[i] = f2h(bf2f(f2bf(float(std * r * cos(6.283185307179586 * u2)))));
    if (i + 1 < n) y[i + 1] = f2h(bf2f(f2bf(float(std * r * sin(6.283185307179586 * u2)))));
}

// ---------------------------------------------------------------- 29 convert_bf16_f16: y = f16(widen(x))
__global__ void k_convert_bf16_f16(const uint16_t* x, uint16_t* y, uint64_t n) {
    uint64_t i = (uint64_t(blockIdx.x) * blockDim.x + threadIdx.x) * 8;
    if (i >= n) return;
    if (i + 8 <= n) {
        float f[8];
        unpack8(*reinterpret_cast<const uint4*>(x + i), f);
        uint4 o;
        o.x = pack2h(f[0], f[1]);
        o.y = pack2h(f[2], f[3]);
        o.z = pack2h(f[4], f[5]);
        o.w = pack2h(f[6], f[7]);
        *reinterpret_cast<uint4*>(y + i) = o;
    } else {
        for (; i < n; ++i) y[i] = f2h(bf2f(x[i]));
    }
}

// ---------------------------------------------------------------- 30 argmax_rows_partial, 31 argmax_rows_final
// argmaxRows over logits rows in two passes: block (b, r) reduces columns [b per, (b + 1) per) of row r to (max, lowest
// index) or a NaN mark, then one wave per row merges the kArgmaxParts pairs: the lowest index of the row maximum, or
// 0xFFFFFFFF for a row holding a NaN (CpuRef.argmaxRows semantics, CpuRef.fs:453-467). The rows are x's rows row0 ..
// row0 + rows - 1 (row0 = 0 for all of them; a forward that needs only its last row's id reduces that row alone).
constexpr int kArgmaxParts = 64;

struct ArgBest {
    float v;
    uint32_t i;  // 0xFFFFFFFF: none yet
};

__device__ __forceinline__ ArgBest arg_merge(ArgBest a, ArgBest b) {
    if (b.i != 0xFFFFFFFFu && (a.i == 0xFFFFFFFFu || b.v > a.v || (b.v == a.v && b.i < a.i))) return b;
    return a;
}

__device__ __forceinline__ ArgBest arg_wave(ArgBest a) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        ArgBest b{__shfl_xor(a.v, o, 64), uint32_t(__shfl_xor(int(a.i), o, 64))};
        a = arg_merge(a, b);
    }
    return a;
}

__global__ __launch_bounds__(256) void k_argmax_partial(const float* x, float* part, int rows, int cols, int row0) {
    __shared__ float sv[4];
    __shared__ uint32_t si[4];
    __shared__ int snan;
    const int r = blockIdx.y, b = blockIdx.x, t = threadIdx.x;
    if (t == 0) snan = 0;
    __syncthreads();
    const int per = (cols + kArgmaxParts - 1) / kArgmaxParts;
    const int c0 = b * per, c1 = min(cols, c0 + per);
    const float* xr = x + size_t(row0 + r) * cols;
    ArgBest best{0.f, 0xFFFFFFFFu};
    bool nan = false;
    for (int c = c0 + t; c < c1; c += 256) {  // increasing per thread: the first of equal values is kept
        const float v = xr[c];
        if (v != v)
            nan = true;
        else if (best.i == 0xFFFFFFFFu || v > best.v)
            best = ArgBest{v, uint32_t(c)};
    }
    if (nan) snan = 1;
    best = arg_wave(best);
    if ((t & 63) == 0) {
        sv[t >> 6] = best.v;
        si[t >> 6] = best.i;
    }
    __syncthreads();
    if (t == 0) {
        ArgBest a{sv[0], si[0]};
        for (int i = 1; i < 4; ++i) a = arg_merge(a, ArgBest{sv[i], si[i]});
        float* pp = part + (size_t(r) * kArgmaxParts + b) * 2;
        pp[0] = a.v;
        reinterpret_cast<uint32_t*>(pp)[1] = snan ? 0xFFFFFFFEu : a.i;
    }
}

__global__ __launch_bounds__(64) void k_argmax_final(const float* part, uint32_t* out, int rows) {
    const int r = blockIdx.x, t = threadIdx.x;
    const float* pp = part + (size_t(r) * kArgmaxParts + t) * 2;
    const uint32_t i = reinterpret_cast<const uint32_t*>(pp)[1];
    const bool nan = __any(i == 0xFFFFFFFEu);
    ArgBest a = arg_wave(ArgBest{pp[0], i == 0xFFFFFFFEu ? 0xFFFFFFFFu : i});
    if (t == 0) out[r] = nan ? 0xFFFFFFFFu : a.i;
}

// ================================================================ 32-34 skinny GEMMs (batched decode)
// Y[r, n] = sum_k A[r, k] W[n, k] for M <= 16 rows (the sequences of a batched decode step), on f16 operands: the
// weights are read once for all rows. A block owns NT 16-column MFMA tiles (SwiGLU: 8 NT gate columns j0 .. and the
// matching up columns, so the block's 16 NT columns hold 8 NT pairs; two tiles also for the plain GEMM, whose wide N
// (the lm_head) would otherwise read the A rows from L2 once per 16 columns; one for the residual GEMMs, whose
// N = hidden needs the blocks) and its 8 waves
// split K in eight. Each wave streams its slice of the W rows straight into MFMA B operands (lane: row c16, 8 halves at
// k + 8g, so 64 contiguous bytes per row per 32-k step) with the A rows from L2, 128 k per iteration, and the next
// iteration's loads in flight while the current one multiplies (two named register sets). The partial tiles of the 8
// waves are summed in LDS in a fixed order (deterministic). Rows of A past M and columns past N are clamped in range
// and never stored. SK_PART (gemm_residual_split with m <= 16): block (x, z) multiplies k range z of K / gridDim.y
// and writes its partial tile to y32 + z M N.
constexpr int kSkWaves = 8;
enum SkEpi { SK_F32 = 0, SK_RESID = 1, SK_SWIGLU = 2, SK_PART = 3 };

template <int EPI, int NT>
__global__ __launch_bounds__(512) void k_gemm_skinny(const uint16_t* a, const uint16_t* w, float* y32, uint16_t* y16,
                                                     int M, int N, int K, int inter, float ascale) {
    static_assert(NT >= 1 && NT <= 3, "MFMA column tiles per block");
    static_assert(EPI != SK_SWIGLU || NT >= 2, "SwiGLU: gate and up columns of 8 NT pairs");
    static_assert(EPI == SK_SWIGLU || NT <= 2, "one output per thread: 256 NT <= 512");
    __shared__ float red[kSkWaves][NT][256];
    // the k range of this block (a part of k for SK_PART); the A and W rows are still K long
    const int KS = EPI == SK_PART ? K / int(gridDim.y) : K, kz = EPI == SK_PART ? int(blockIdx.y) * KS : 0;
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6, g = lane >> 4, c16 = lane & 15;
    // the W row of block column 16 u + c16 in tile u: SwiGLU blocks own P = 8 NT gate / up pairs, columns 0 .. P - 1
    // the gate rows j0 .. j0 + P - 1, columns P .. 2 P - 1 the matching up rows (clamped to the last pair)
    constexpr int P = 8 * NT;
    int nr[NT];
#pragma unroll
    for (int u = 0; u < NT; ++u) {
        const int lc = 16 * u + c16;
        if (EPI == SK_SWIGLU) {
            const int j = min(int(blockIdx.x) * P + (lc < P ? lc : lc - P), inter - 1);
            nr[u] = lc < P ? j : inter + j;
        } else {
            nr[u] = min(int(blockIdx.x) * (16 * NT) + lc, N - 1);
        }
    }
    const int kper = KS / kSkWaves, niter = kper / 128;  // kper a multiple of 128
    const int kb = kz + wv * kper + 8 * g;
    const uint16_t* ap = a + size_t(min(c16, M - 1)) * K + kb;
    const uint16_t* wp[NT];
#pragma unroll
    for (int u = 0; u < NT; ++u) wp[u] = w + size_t(nr[u]) * K + kb;
    f32x4 acc[NT];
#pragma unroll
    for (int u = 0; u < NT; ++u) acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
    u32x4 av[2][4], bw[2][NT][4];
    auto load = [&](auto set, int it) __attribute__((always_inline)) {
        constexpr int S = decltype(set)::value;
        const int k = it * 128;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
#pragma unroll
            for (int u = 0; u < NT; ++u) bw[S][u][s] = *reinterpret_cast<const u32x4*>(wp[u] + k + 32 * s);
            av[S][s] = *reinterpret_cast<const u32x4*>(ap + k + 32 * s);
        }
    };
    auto mma = [&](auto set) __attribute__((always_inline)) {
        constexpr int S = decltype(set)::value;
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int u = 0; u < NT; ++u)
                acc[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_f16x8(av[S][s]), as_f16x8(bw[S][u][s]), acc[u], 0, 0,
                                                                0);
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    // The scheduling barriers keep each set's loads ahead of the other set's MFMAs (left alone, the compiler sinks
    // them between the MFMAs and drains every load at the end of each iteration). The loop runs while two more
    // iterations exist, so no load is issued past the end and the loop head always has set 0 as the younger load.
    load(S0{}, 0);
    int it = 0;
    for (; it + 2 < niter; it += 2) {
        __builtin_amdgcn_sched_barrier(0);
        load(S1{}, it + 1);
        __builtin_amdgcn_sched_barrier(0);
        mma(S0{});
        __builtin_amdgcn_sched_barrier(0);
        load(S0{}, it + 2);
        __builtin_amdgcn_sched_barrier(0);
        mma(S1{});
    }
    __builtin_amdgcn_sched_barrier(0);
    if (it + 1 < niter) {
        load(S1{}, it + 1);
        __builtin_amdgcn_sched_barrier(0);
        mma(S0{});
        __builtin_amdgcn_sched_barrier(0);
        mma(S1{});
    } else {
        mma(S0{});
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int u = 0; u < NT; ++u) red[wv][u][lane * 4 + i] = acc[u][i];
    __syncthreads();
    // element e of a tile: lane e / 4, register e % 4 -> row 4 (lane / 16) + e % 4, column lane % 16
    if (EPI == SK_SWIGLU) {
        // thread t < 16 P: row t / P, pair jl = t % P (its gate at block column jl, its up at P + jl)
        if (t >= 16 * P) return;
        const int row = t / P, jl = t - row * P, col = int(blockIdx.x) * P + jl;
        auto elem = [&](int c) { return ((row >> 2) * 16 + (c & 15)) * 4 + (row & 3); };
        const int gt = jl >> 4, ge = elem(jl), ut = (P + jl) >> 4, ue = elem(P + jl);
        float gv = 0.f, uv = 0.f;
#pragma unroll
        for (int i = 0; i < kSkWaves; ++i) {
            gv += red[i][gt][ge];
            uv += red[i][ut][ue];
        }
        if (row < M && col < inter) {
            const uint16_t hv = f2h(gv / (1.0f + __expf(-gv)) * uv * ascale);
            f16_note(f16_bad2(hv), kF16Swiglu);
            y16[size_t(row) * inter + col] = hv;
        }
        return;
    }
    if (t >= 256 * NT) return;
    const int tile = t >> 8, e = t & 255;
    const int l = e >> 2, row = 4 * (l >> 4) + (e & 3), col = int(blockIdx.x) * (16 * NT) + tile * 16 + (l & 15);
    float v = 0.f;
#pragma unroll
    for (int i = 0; i < kSkWaves; ++i) v += red[i][tile][e];
    if (row >= M || col >= N) return;
    if (EPI != SK_F32) v *= ascale;
    if (EPI == SK_RESID)
        y32[size_t(row) * N + col] += v;
    else if (EPI == SK_PART)
        y32[(size_t(blockIdx.y) * M + row) * N + col] = v;
    else
        y32[size_t(row) * N + col] = v;
}

// ---------------------------------------------------------------- 36 decode_advance
// After the batched argmax: out_ids[step * B + b] = id[b] (while step < max_steps), then every sequence moves one
// position and takes its argmax as the next token; step += 1.
__global__ __launch_bounds__(256) void k_decode_advance(const uint32_t* am, uint32_t* state, uint32_t* out_ids, int B,
                                                        int max_steps) {
    const uint32_t step = state[2 * B];
    for (int b = threadIdx.x; b < B; b += 256) {
        const uint32_t id = am[b];
        if (step < uint32_t(max_steps)) out_ids[size_t(step) * B + b] = id;
        state[B + b] = id;
        state[b] = state[b] + 1u;
    }
    __syncthreads();
    if (threadIdx.x == 0) state[2 * B] = step + 1u;
}

// ---------------------------------------------------------------- 37 prefetch
// Streams up to four tensors through the caches and discards the data, so a later kernel's loads of them hit the
// last-level cache (256 MB on MI355X) instead of HBM; meant as an overlapped dispatch ahead of the kernels that read
// them (a decode GEMV on weights in that cache runs about 30 % faster than on weights in HBM). 256 blocks, eight
// 16-byte loads in flight per thread; the XOR of the data is handed to an empty asm statement so the loads stay.
__global__ __launch_bounds__(256) void k_prefetch(const u32x4* p0, uint32_t n0, const u32x4* p1, uint32_t n1,
                                                  const u32x4* p2, uint32_t n2, const u32x4* p3, uint32_t n3) {
    const uint32_t stride = gridDim.x * 256u;
    uint32_t acc = 0;
    auto run = [&](const u32x4* p, uint32_t n) __attribute__((always_inline)) {
        uint32_t i = blockIdx.x * 256u + threadIdx.x;
        for (; i + 7 * stride < n; i += 8 * stride) {
            u32x4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = p[i + u * stride];
#pragma unroll
            for (int u = 0; u < 8; ++u) acc ^= v[u].x ^ v[u].w;
        }
        for (; i < n; i += stride) acc ^= p[i].x;
    };
    run(p0, n0);
    run(p1, n1);
    run(p2, n2);
    run(p3, n3);
    asm volatile("" ::"v"(acc));
}

// ================================================================ launchers and catalog entries

static float f32_of(uint32_t b) {
    float f;
    std::memcpy(&f, &b, 4);
    return f;
}

// 14 rmsnorm_rows_f16: x, w, y, rows, cols, eps, x_row0
static void l_rmsnorm_f16(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    const uint32_t rows = pd.words[4], cols = pd.words[5];
#define L_RMS(NC)                                                                                                    \
    hipLaunchKernelGGL(k_rmsnorm_f16_wave<NC>, dim3((rows + 3) / 4), dim3(256), 0, s, (const float*)p[0],            \
                       (const uint16_t*)p[1], (uint16_t*)p[2], rows, cols, f32_of(pd.words[6]), pd.words[7])
    switch (cols % 256 == 0 ? cols / 256 : 0) {
        case 1: L_RMS(1); break;
        case 2: L_RMS(2); break;
        case 4: L_RMS(4); break;
        case 8: L_RMS(8); break;
        case 16: L_RMS(16); break;
        default:
            hipLaunchKernelGGL(k_rmsnorm_f16, dim3(rows), dim3(256), 0, s, (const float*)p[0], (const uint16_t*)p[1],
                               (uint16_t*)p[2], rows, cols, f32_of(pd.words[6]), pd.words[7]);
    }
#undef L_RMS
}

// The SwiGLU output's shift s (catalog field a_shift, at most kMaxAShift): its producers store a 2^-s, its consumers
// multiply their sums by 2^s. Powers of two scale exactly, so the results equal the unshifted ones wherever a 2^-s
// stays a normal fp16 number (|a| >= 2^(s - 14)); below that a keeps 2^(s - 24) of absolute precision.
constexpr uint32_t kMaxAShift = 24;
static_assert(fast::kF16Swiglu == kF16SiteSwiglu, "the host's SwiGLU range bit");
static float a_scale(uint32_t s) { return std::ldexp(1.0f, -int(s)); }
static float a_unscale(uint32_t s) { return std::ldexp(1.0f, int(s)); }

static GemmArgs gemm_base(void* const* p, uint32_t m, uint32_t n, uint32_t k) {
    GemmArgs a{};
    a.a = (const uint16_t*)p[0];
    a.w = (const uint16_t*)p[1];
    a.M = int(m);
    a.N = int(n);
    a.K = int(k);
    a.ascale = 1.0f;
    return a;
}

// 15 gemm_qkv_rope: h, w, q_norm, k_norm, cos, sin, q, k_cache, v_cache, m, hidden, q_heads, kv_heads, pos0, max_pos,
// The GEMM's direct-to-LDS loop needs two blocks on every CU (MI355X: 256 CUs, two 64 KiB blocks each) for the whole
// launch: grids of whole rounds of 512 tiles, or long enough (4 rounds) that a last partial round hardly counts. In a
// partial round a CU holds one block, which the register-pipelined loop (loads two k steps ahead) serves better
// (measured: the 768-tile SwiGLU GEMM of a 2048-token prefill, 42 against 44 us).
static bool two_per_cu(const dim3& g) {
    const uint64_t tiles = uint64_t(g.x) * g.y;
    return tiles >= 512 && (tiles % 512 == 0 || tiles >= 4 * 512);
}
// q|k|v tiles of 64 rows where 128-row tiles leave CUs without a tile (512 rows: 32 x 4 tiles on half the CUs, 32 x 8
// on all of them; the 512-token forward 2.40-2.41 -> 2.27 ms)
static bool qkv_rows64(uint32_t m, uint32_t heads) { return m > 64 && uint64_t(heads) * ((m + 127) / 128) < 256; }

// eps
static void l_gemm_qkv(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    const uint32_t* w = pd.words.data();
    const int qh = int(w[12]), kvh = int(w[13]);
    GemmArgs a = gemm_base(p, w[10], uint32_t((qh + 2 * kvh) * 128), w[11]);
    a.qn = (const uint16_t*)p[2];
    a.kn = (const uint16_t*)p[3];
    a.cos_t = (const float*)p[4];
    a.sin_t = (const float*)p[5];
    a.q_out = (uint16_t*)p[6];
    a.kc = (uint16_t*)p[7];
    a.vc = (uint16_t*)p[8];
    a.qh = qh;
    a.kvh = kvh;
    a.pos0 = int(w[14]);
    a.max_pos = int(w[15]);
    a.eps = f32_of(w[16]);
    const dim3 grid(uint32_t(qh + 2 * kvh), (w[10] + GBM - 1) / GBM);
    if (two_per_cu(grid))
        hipLaunchKernelGGL((k_gemm<EPI_QKV, 128, true>), grid, dim3(256), 0, s, a);
    else if (qkv_rows64(w[10], qh + 2 * kvh))
        hipLaunchKernelGGL((k_gemm<EPI_QKV, 128, false, 64>), dim3(grid.x, (w[10] + 63) / 64), dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL((k_gemm<EPI_QKV, 128, false>), grid, dim3(256), 0, s, a);
}

// 16 attention_prefill_f16: q, k_cache, v_cache, y, workspace, rows, past, q_heads, kv_heads, max_pos, scale
static void l_attn_prefill(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    const uint32_t* w = pd.words.data();
    const int T = int(w[6]);
    hipLaunchKernelGGL(k_attn_prefill, dim3(uint32_t((T + kAttnRows - 1) / kAttnRows), w[9]), dim3(256), 0, s,
                       (const uint16_t*)p[0], (const uint16_t*)p[1], (const uint16_t*)p[2], (uint16_t*)p[3],
                       (uint32_t*)p[4], T, int(w[7]), int(w[8]), int(w[10]), f32_of(w[11]) * kLog2e);
}

// Residual GEMMs with few 128 x 128 tiles (o_proj and down_proj have N = hidden) use 64-wide column tiles so the
// grid covers the CUs.
static bool resid_narrow(uint32_t m, uint32_t n) { return ((m + 127) / 128) * ((n + 127) / 128) < 512; }

// 17 gemm_residual: a, w, x, m, n, k, a_shift
static void l_gemm_resid(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    const uint32_t* w = pd.words.data();
    GemmArgs a = gemm_base(p, w[4], w[5], w[6]);
    a.y32 = (float*)p[2];
    a.resid = (const float*)p[2];
    a.ascale = a_unscale(w[7]);
    if (resid_narrow(w[4], w[5]))  // under two blocks per CU by construction
        hipLaunchKernelGGL((k_gemm<EPI_RESID, 64, false>), dim3((w[5] + 63) / 64, (w[4] + GBM - 1) / GBM), dim3(256), 0, s,
                           a);
    else
        hipLaunchKernelGGL((k_gemm<EPI_RESID, 128, true>), dim3((w[5] + GBN - 1) / GBN, (w[4] + GBM - 1) / GBM), dim3(256), 0,
                           s, a);
}

// gemm_swiglu's gate / up pairs per tile: 96 where that makes whole rounds of 512 tiles for the direct-to-LDS loop
// (Qwen3-0.6B at 2048 rows: 32 x 16 tiles, where 64 pairs give 768 tiles, one and a half rounds); else 64
static int swiglu_pairs(uint32_t m, uint32_t inter) {
    const uint64_t rows = (m + GBM - 1) / GBM;
    if (inter % 96 == 0 && (uint64_t(inter / 96) * rows) % 512 == 0) return 96;
    return 64;
}
static dim3 swiglu_grid(uint32_t m, uint32_t inter) {
    const uint32_t pairs = uint32_t(swiglu_pairs(m, inter));
    return dim3((inter + pairs - 1) / pairs, (m + GBM - 1) / GBM);
}

// 18 gemm_swiglu: a, w (2 inter rows), y, m, inter, k, a_shift
static void l_gemm_swiglu(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    const uint32_t* w = pd.words.data();
    GemmArgs a = gemm_base(p, w[4], 2 * w[5], w[6]);
    a.y16 = (uint16_t*)p[2];
    a.inter = int(w[5]);
    a.ascale = a_scale(w[7]);
    const dim3 grid = swiglu_grid(w[4], w[5]);
    const int pairs = swiglu_pairs(w[4], w[5]);
    if (pairs == 96)
        hipLaunchKernelGGL((k_gemm<EPI_SWIGLU, 192, true>), grid, dim3(256), 0, s, a);
    else if (two_per_cu(grid))
        hipLaunchKernelGGL((k_gemm<EPI_SWIGLU, 128, true>), grid, dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL((k_gemm<EPI_SWIGLU, 128, false>), grid, dim3(256), 0, s, a);
}

// 19 gemm_f32: a, w, y, m, n, k
static void l_gemm_f32(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    const uint32_t* w = pd.words.data();
    GemmArgs a = gemm_base(p, w[4], w[5], w[6]);
    a.y32 = (float*)p[2];
    const dim3 grid((w[5] + GBN - 1) / GBN, (w[4] + GBM - 1) / GBM);
    if (two_per_cu(grid))
        hipLaunchKernelGGL((k_gemm<EPI_F32, 128, true>), grid, dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL((k_gemm<EPI_F32, 128, false>), grid, dim3(256), 0, s, a);
}

// The decode GEMVs: one row (or gate/up pair) per wave, 4 waves per block; NCH, the 512-wide k-chunks per lane, is
// rounded up to one of the compiled widths.
static uint32_t gemv_blocks(uint32_t rows) { return (rows + 3) / 4; }
static int nch_bucket(uint32_t k) {
    const uint32_t c = (k + 511) / 512;
    for (int b : {1, 2, 3, 4, 6, 8, 12, 16})
        if (c <= uint32_t(b)) return b;
    return 0;
}
#define NCH_DISPATCH(K, LAUNCH)                 \
    switch (nch_bucket(K)) {                    \
        case 1: LAUNCH(1); break;               \
        case 2: LAUNCH(2); break;               \
        case 3: LAUNCH(3); break;               \
        case 4: LAUNCH(4); break;               \
        case 6: LAUNCH(6); break;               \
        case 8: LAUNCH(8); break;               \
        case 12: LAUNCH(12); break;             \
        case 16: LAUNCH(16); break;             \
        default: break;                         \
    }

// 20 gemv_norm_dec: x, norm, w, y, n, k, eps
static void l_gemv_norm(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    const uint32_t* w = pd.words.data();
#define L_NORM(N)                                                                                                    \
    hipLaunchKernelGGL(k_gemv_norm_dec<N>, dim3(gemv_blocks(w[5])), dim3(256), 0, s, (const float*)p[0],            \
                       (const uint16_t*)p[1], (const uint16_t*)p[2], (float*)p[3], int(w[5]), int(w[6]), f32_of(w[7]))
    NCH_DISPATCH(w[6], L_NORM)
#undef L_NORM
}

// 21 attention_decode_f16: qkv, q_norm, k_norm, cos, sin, k_cache, v_cache, partials, state, q_heads, kv_heads,
// max_pos, eps, scale, batch, chunks, splits
// 64-key chunks per split block: the `chunks` field, 0 meaning 1 (the field is the last one; callers that predate it
// leave its word 0)
static int dec_chunks(uint32_t w) { return w == 0 ? 1 : int(w); }
static uint32_t dec_splits(uint32_t max_pos, uint32_t chunks) {
    const uint32_t keys = 64u * uint32_t(dec_chunks(chunks));
    return (max_pos + keys - 1) / keys;
}

// the splits per sequence: the `splits` field when set (then each sequence's keys spread evenly over them), else one
// per 64 C keys of max_pos
static uint32_t dec_grid_splits(uint32_t max_pos, uint32_t chunks, uint32_t splits) {
    return splits ? splits : dec_splits(max_pos, chunks);
}
// The GEMM stamps of the stage-timing build (kind = the epilogue, 0 .. 4; words <= kGemmStampBlocks x 32): false in
// the shipped build, which records none.
bool gemm_stamps_read(int kind, uint64_t* dst, size_t words) {
#if defined(LRM_GEMM_STAMPS)
    if (kind < 0 || kind >= kGemmStampKinds || words > size_t(kGemmStampBlocks) * kGemmStampWords) return false;
    hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
    hip_check(hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_gemm_stamps), words * 8, size_t(kind) * kGemmStampBlocks * kGemmStampWords * 8,
                                  hipMemcpyDeviceToHost),
              "hipMemcpyFromSymbol(g_gemm_stamps)");
    return true;
#else
    (void)kind, (void)dst, (void)words;
    return false;
#endif
}

void* f16_range_word_fast() {
    void* p = nullptr;
    hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(fast::f16_range_word)), "hipGetSymbolAddress(f16_range_word)");
    if (!p) throw HipError("hipGetSymbolAddress(f16_range_word) returned a null address");
    return p;
}

static void l_attn_dec(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    const uint32_t* w = pd.words.data();
    const int max_pos = int(w[12]);
    const bool even = w[17] != 0;
    const dim3 grid(dec_grid_splits(w[12], w[16], w[17]), w[11], w[15]);
#define L_DEC(M)                                                                                                     \
    hipLaunchKernelGGL(k_attn_dec<M>, grid, dim3(M ? 512 : 256), 0, s, (const float*)p[0], (const uint16_t*)p[1],  \
                       (const uint16_t*)p[2], (const float*)p[3], (const float*)p[4], (uint16_t*)p[5],              \
                       (uint16_t*)p[6], (float*)p[7], (const uint32_t*)p[8], int(w[10]), int(w[11]), max_pos,       \
                       f32_of(w[13]), f32_of(w[14]) * kLog2e, even ? 0 : dec_chunks(w[16]))
    if (!even && dec_chunks(w[16]) == 1)
        L_DEC(false);
    else
        L_DEC(true);
#undef L_DEC
}

// 22 attention_combine, 35 attention_combine_f16: partials, y, state, q_heads, max_pos, batch, chunks, splits
template <typename OUT>
static void l_attn_combine_t(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    const uint32_t* w = pd.words.data();
    const int max_pos = int(w[5]);
    hipLaunchKernelGGL((k_attn_combine<OUT>), dim3(w[4], w[6]), dim3(256), 0, s, (const float*)p[0], (OUT*)p[1],
                       (const uint32_t*)p[2], int(dec_grid_splits(w[5], w[7], w[8])), w[8] ? 0 : 64 * dec_chunks(w[7]),
                       max_pos);
}
static void l_attn_combine(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    l_attn_combine_t<float>(pd, p, s);
}
static void l_attn_combine_f16(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    l_attn_combine_t<uint16_t>(pd, p, s);
}

// 23 gemv_residual_dec: a, w, x, n, k
static void l_gemv_resid(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    const uint32_t* w = pd.words.data();
#define L_RESID(N)                                                                                                   \
    hipLaunchKernelGGL(k_gemv_resid_dec<N>, dim3(gemv_blocks(w[4])), dim3(256), 0, s, (const float*)p[0],           \
                       (const uint16_t*)p[1], (float*)p[2], int(w[4]), int(w[5]))
    NCH_DISPATCH(w[5], L_RESID)
#undef L_RESID
}

// 24 gemv_swiglu_dec: x, norm, w, y, inter, hidden, eps
static void l_gemv_swiglu(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    const uint32_t* w = pd.words.data();
#define L_SWIGLU(N)                                                                                                  \
    hipLaunchKernelGGL(k_gemv_swiglu_dec<N>, dim3(gemv_blocks(w[5])), dim3(256), 0, s, (const float*)p[0],          \
                       (const uint16_t*)p[1], (const uint16_t*)p[2], (float*)p[3], int(w[5]), int(w[6]), f32_of(w[7]))
    NCH_DISPATCH(w[6], L_SWIGLU)
#undef L_SWIGLU
}

// 25 lmhead_dec: x, norm, embed, logits, partials, vocab, hidden, eps, write_logits
static void l_lmhead(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    const uint32_t* w = pd.words.data();
#define L_LM(N)                                                                                                      \
    hipLaunchKernelGGL(k_lmhead_dec<N>, dim3(kLmheadBlocks), dim3(256), 0, s, (const float*)p[0],                   \
                       (const uint16_t*)p[1], (const uint16_t*)p[2], (float*)p[3], (float*)p[4], int(w[6]), int(w[7]), \
                       f32_of(w[8]), int(w[9]))
    NCH_DISPATCH(w[7], L_LM)
#undef L_LM
}

// 26 argmax_dec: partials, state, out_ids, max_steps
static void l_argmax_dec(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    hipLaunchKernelGGL(k_argmax_dec, dim3(1), dim3(1024), 0, s, (const float*)p[0], (uint32_t*)p[1], (uint32_t*)p[2],
                       int(kLmheadBlocks), int(pd.words[4]));
}

// 27 embed_dec: embed, state, x, hidden, vocab
static void l_embed_dec(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    hipLaunchKernelGGL(k_embed_dec, dim3(pd.words[6]), dim3(256), 0, s, (const uint16_t*)p[0], (const uint32_t*)p[1],
                       (float*)p[2], int(pd.words[4]), int(pd.words[5]));
}

// 28 fill_normal_f16: y, n, seed_lo, seed_hi, stream_lo, stream_hi, std
static void l_fill_normal(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    const uint32_t* w = pd.words.data();
    const uint64_t n = w[2];
    const uint64_t seed = uint64_t(w[3]) | uint64_t(w[4]) << 32, stream = uint64_t(w[5]) | uint64_t(w[6]) << 32;
    hipLaunchKernelGGL(k_fill_normal, dim3(uint32_t((n / 2 + 255) / 256 + 1)), dim3(256), 0, s, (uint16_t*)p[0], n,
                       seed, stream, f32_of(w[7]));
}

// 29 convert_bf16_f16: x, y, n
static void l_convert(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    const uint64_t n = pd.words[3];
    hipLaunchKernelGGL(k_convert_bf16_f16, dim3(uint32_t((n / 8 + 255) / 256 + 1)), dim3(256), 0, s,
                       (const uint16_t*)p[0], (uint16_t*)p[1], n);
}

// 30 argmax_rows_partial: x, partials, rows, cols, row0
static void l_argmax_partial(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    hipLaunchKernelGGL(k_argmax_partial, dim3(kArgmaxParts, pd.words[3]), dim3(256), 0, s, (const float*)p[0],
                       (float*)p[1], int(pd.words[3]), int(pd.words[4]), int(pd.words[5]));
}

// 31 argmax_rows_final: partials, out, rows
static void l_argmax_final(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    hipLaunchKernelGGL(k_argmax_final, dim3(pd.words[3]), dim3(64), 0, s, (const float*)p[0], (uint32_t*)p[1],
                       int(pd.words[3]));
}

// 32 gemm_skinny_f32: a, w, y, m, n, k; 33 gemm_skinny_residual: a, w, y, m, n, k, a_shift; 34 gemm_skinny_swiglu:
// a, w, y, m, inter, k, a_shift
// One 16-column tile per block while that still leaves under two blocks per CU; two for wide N (the lm_head), whose
// A rows would otherwise be read from L2 once per 16 columns.
static bool skinny_one_tile(uint32_t n) { return (n + 15) / 16 < 512; }
static void l_gemm_skinny_f32(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    const uint32_t* w = pd.words.data();
    if (skinny_one_tile(w[5]))
        hipLaunchKernelGGL((k_gemm_skinny<SK_F32, 1>), dim3((w[5] + 15) / 16), dim3(512), 0, s, (const uint16_t*)p[0],
                           (const uint16_t*)p[1], (float*)p[2], (uint16_t*)nullptr, int(w[4]), int(w[5]), int(w[6]), 0, 1.0f);
    else
        hipLaunchKernelGGL((k_gemm_skinny<SK_F32, 2>), dim3((w[5] + 31) / 32), dim3(512), 0, s, (const uint16_t*)p[0],
                           (const uint16_t*)p[1], (float*)p[2], (uint16_t*)nullptr, int(w[4]), int(w[5]), int(w[6]), 0,
                           1.0f);
}
static void l_gemm_skinny_resid(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    const uint32_t* w = pd.words.data();
    hipLaunchKernelGGL((k_gemm_skinny<SK_RESID, 1>), dim3((w[5] + 15) / 16), dim3(512), 0, s, (const uint16_t*)p[0],
                       (const uint16_t*)p[1], (float*)p[2], (uint16_t*)nullptr, int(w[4]), int(w[5]), int(w[6]), 0,
                       a_unscale(w[7]));
}
// gate / up pairs per skinny SwiGLU block: 16 (two MFMA column tiles), or 24 (three) where that takes the grid from
// over one round of 256 blocks (one per CU) to one. A block's time barely depends on its k loop at these sizes, so a
// round costs about the same either way: the Qwen3-1.7B gate/up (6144 pairs at 16 rows) 384 blocks took 12.6 us, 256
// blocks of 16 pairs (4096) 7.3 us.
static int skinny_swiglu_pairs(uint32_t inter) { return (inter + 15) / 16 > 256 && (inter + 23) / 24 <= 256 ? 24 : 16; }
static void l_gemm_skinny_swiglu(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    const uint32_t* w = pd.words.data();
    if (skinny_swiglu_pairs(w[5]) == 24)
        hipLaunchKernelGGL((k_gemm_skinny<SK_SWIGLU, 3>), dim3((w[5] + 23) / 24), dim3(512), 0, s,
                           (const uint16_t*)p[0], (const uint16_t*)p[1], (float*)nullptr, (uint16_t*)p[2], int(w[4]), 0,
                           int(w[6]), int(w[5]), a_scale(w[7]));
    else
        hipLaunchKernelGGL((k_gemm_skinny<SK_SWIGLU, 2>), dim3((w[5] + 15) / 16), dim3(512), 0, s,
                           (const uint16_t*)p[0], (const uint16_t*)p[1], (float*)nullptr, (uint16_t*)p[2], int(w[4]), 0,
                           int(w[6]), int(w[5]), a_scale(w[7]));
}

// 36 decode_advance: argmax, state, out_ids, batch, max_steps
static void l_decode_advance(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    hipLaunchKernelGGL(k_decode_advance, dim3(1), dim3(256), 0, s, (const uint32_t*)p[0], (uint32_t*)p[1],
                       (uint32_t*)p[2], int(pd.words[4]), int(pd.words[5]));
}

// 37 prefetch: x0, x1, x2, x3 (each tensor's whole extent, in 16-byte units)
static void l_prefetch(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    uint32_t n[4] = {0, 0, 0, 0};
    for (const TokenUse& u : pd.tokens)
        if (u.field < 4) n[u.field] = uint32_t((u.end - u.start) / 16);
    hipLaunchKernelGGL(k_prefetch, dim3(256), dim3(256), 0, s, (const u32x4*)p[0], n[0], (const u32x4*)p[1], n[1],
                       (const u32x4*)p[2], n[2], (const u32x4*)p[3], n[3]);
}

// 39 gemm_residual_split: a, w, partials, m, n, k, splits, a_shift. 128 x 64 tiles, blockIdx.z = the k split.
// the skinny (m <= 16) form of gemm_residual_split: 8 waves over each split's k, 128 per wave per step
static bool resid_split_skinny(uint32_t m, uint32_t k, uint32_t splits) {
    return m <= 16 && (k / splits) % (kSkWaves * 128) == 0;
}
// 64-row tiles for grids of 128 x 64 tiles under one block per CU
static bool resid_rows64(uint32_t m, uint64_t blocks128) { return m > 64 && blocks128 < 256; }
static void l_gemm_resid_split(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    const uint32_t* w = pd.words.data();
    if (resid_split_skinny(w[4], w[6], w[7])) {
        hipLaunchKernelGGL((k_gemm_skinny<SK_PART, 1>), dim3((w[5] + 15) / 16, w[7]), dim3(512), 0, s,
                           (const uint16_t*)p[0], (const uint16_t*)p[1], (float*)p[2], (uint16_t*)nullptr, int(w[4]),
                           int(w[5]), int(w[6]), 0, a_unscale(w[8]));
        return;
    }
    GemmArgs a = gemm_base(p, w[4], w[5], w[6]);
    a.y32 = (float*)p[2];
    a.ksplit = int(w[6] / w[7]);
    a.ascale = a_unscale(w[8]);
    const dim3 grid((w[5] + 63) / 64, (w[4] + GBM - 1) / GBM, w[7]);
    const uint64_t blocks = uint64_t(grid.x) * grid.y * grid.z;
    if (blocks % 512 == 0)  // whole rounds of two blocks per CU: the direct-to-LDS loop
        hipLaunchKernelGGL((k_gemm<EPI_PART, 64, true>), grid, dim3(256), 0, s, a);
    else if (resid_rows64(w[4], blocks))  // 64-row tiles, twice the blocks
        hipLaunchKernelGGL((k_gemm<EPI_PART, 64, false, 64>), dim3(grid.x, (w[4] + 63) / 64, grid.z), dim3(256), 0, s,
                           a);
    else
        hipLaunchKernelGGL((k_gemm<EPI_PART, 64, false>), grid, dim3(256), 0, s, a);
}

// 40 residual_add_norm: x, partials, w, y, rows, cols, splits, eps
static void l_resid_add_norm(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    const uint32_t rows = pd.words[5], cols = pd.words[6], splits = pd.words[7];
    const float eps = f32_of(pd.words[8]);
    // a block per row for the few rows of a batched decode step (16 sequences: 16 CUs loading instead of 4; 3931 ->
    // 3973 tok/s at the 1.7B shape), else four rows per block (512 rows: 2.39-2.40 ms per forward against 2.41 with
    // one row per block)
    const uint32_t rpb = rows <= 64 ? 1 : 4;
#define L_RAN(NC)                                                                                                    \
    hipLaunchKernelGGL(k_resid_add_norm<NC>, dim3((rows + rpb - 1) / rpb), dim3(64 * rpb), 0, s, (float*)p[0],         \
                       (const float*)p[1], (const uint16_t*)p[2], (uint16_t*)p[3], rows, cols, splits, eps)
    switch (cols / 256) {
        case 1: L_RAN(1); break;
        case 2: L_RAN(2); break;
        case 4: L_RAN(4); break;
        case 8: L_RAN(8); break;
        default: L_RAN(16); break;  // 4096 (the catalog admits no other width)
    }
#undef L_RAN
}

// 38 decode_step_persistent (kernels_persist.hip)
void launch_decode_persistent(const PreparedDispatch& pd, void* const* p, hipStream_t s);

int fast_first_id() { return 14; }

const LaunchFn* fast_launchers() {
    static const LaunchFn t[] = {l_rmsnorm_f16, l_gemm_qkv,  l_attn_prefill, l_gemm_resid,   l_gemm_swiglu,
                                 l_gemm_f32,    l_gemv_norm, l_attn_dec,     l_attn_combine, l_gemv_resid,
                                 l_gemv_swiglu, l_lmhead,    l_argmax_dec,   l_embed_dec,    l_fill_normal,
                                 l_convert,     l_argmax_partial, l_argmax_final, l_gemm_skinny_f32,
                                 l_gemm_skinny_resid, l_gemm_skinny_swiglu, l_attn_combine_f16, l_decode_advance,
                                 l_prefetch,    launch_decode_persistent, l_gemm_resid_split, l_resid_add_norm};
    return t;
}

// ---------------------------------------------------------------- catalog entries (ids 14..40)

#define DT(x) (1u << (x))
#define TOK_R(n, m) FieldSpec{n, FieldKind::Token, Access::Read, m, nullptr}
#define TOK_W(n, m) FieldSpec{n, FieldKind::Token, Access::Write, m, nullptr}
#define TOK_RW(n, m) FieldSpec{n, FieldKind::Token, Access::ReadWrite, m, nullptr}
#define U32F(n) FieldSpec{n, FieldKind::U32, Access::None, 0, nullptr}
#define F32F(n) FieldSpec{n, FieldKind::F32, Access::None, 0, nullptr}

static void need(const uint32_t* counts, int field, int64_t elems, const char* kernel, const char* what) {
    if (elems < 0 || int64_t(counts[field]) < elems)
        contract_fail("%s.%s holds %u elements; the dispatch touches %lld", kernel, what, counts[field],
                      (long long)elems);
}

static void need_group2(const char* k, uint32_t qh, uint32_t kvh) {
    if (kvh < 1 || qh != 2 * kvh) contract_fail("%s: this kernel takes head_dim 128 and two query heads per KV head", k);
}

static void need_k(const char* k, uint32_t n) {
    if (n < 8 || n % 8 || n > uint32_t(kMaxHidden))
        contract_fail("%s: the reduced dimension must be a multiple of 8 in 8 .. %d", k, kMaxHidden);
}

static void need_batch(const char* k, uint32_t b) {
    if (b < 1 || b > 1024) contract_fail("%s: batch must be in 1 .. 1024", k);
}

static void need_chunks(const char* k, uint32_t chunks) {
    if (chunks > 64) contract_fail("%s: chunks must be in 0 .. 64 (0 = 1)", k);
}

// splits (0 = one per 64 chunks keys of max_pos): at most max_pos / 64, the most the partials hold
static void need_splits(const char* k, uint32_t splits, uint32_t max_pos) {
    if (splits > max_pos / 64) contract_fail("%s: splits must be in 0 .. max_pos / 64 (0 = by chunks)", k);
}

static void check_combine(const char* k, const uint32_t* w, const uint32_t* c) {
    const int64_t qh = w[4], mp = w[5], B = w[6];
    need_batch(k, w[6]);
    need_chunks(k, w[7]);
    need_splits(k, w[8], w[5]);
    if (mp < 64 || mp % 64 || mp > 64 * kMaxSplits) contract_fail("%s: max_pos must be a multiple of 64 in 64 .. %d", k, 64 * kMaxSplits);
    need(c, 0, B * qh * (mp / 64) * 130, k, "partials");
    need(c, 1, B * qh * 128, k, "y");
    need(c, 2, 2 * B + 1, k, "state");
}

static void check_skinny(const char* k, const uint32_t* w, const uint32_t* c, int64_t wrows, int64_t ycols) {
    const int64_t m = w[4], K = w[6];
    if (m < 1 || m > 16) contract_fail("%s: m must be in 1 .. 16", k);
    if (K < 1024 || K % 1024) contract_fail("%s: k must be a positive multiple of 1024", k);
    if (wrows < 1) contract_fail("%s: n must be at least 1", k);
    need(c, 0, m * K, k, "a");
    need(c, 1, wrows * K, k, "w");
    need(c, 2, m * ycols, k, "y");
}

static void need_a_shift(const char* k, uint32_t s) {
    if (s > kMaxAShift) contract_fail("%s: a_shift must be at most %u", k, kMaxAShift);
}

static void need_max_pos(const char* k, uint32_t mp) {
    if (mp < 64 || mp % 64 || mp > 64u * kMaxSplits)
        contract_fail("%s: max_pos must be a multiple of 64 in 64 .. %d", k, 64 * kMaxSplits);
}

std::vector<KernelSpec> fast_catalog() {
    std::vector<KernelSpec> c;
    // 14 rmsnorm_rows_f16: x, w, y, rows, cols, eps, x_row0
    c.push_back({"rmsnorm_rows_f16", "fast", {256, 1, 1}, true, [](const uint32_t* w) { return Grid3{w[4], 1, 1}; },
                 {TOK_R("x", DT(F32)), TOK_R("w", DT(BF16)), TOK_W("y", DT(F16)), U32F("rows"), U32F("cols"),
                  F32F("eps"), U32F("x_row0")},
                 [](const uint32_t* w, const uint32_t* c) {
                     if (w[5] < 1) contract_fail("rmsnorm_rows_f16: cols must be at least 1");
                     need(c, 0, (int64_t(w[7]) + w[4]) * w[5], "rmsnorm_rows_f16", "x");
                     need(c, 1, w[5], "rmsnorm_rows_f16", "w");
                     need(c, 2, int64_t(w[4]) * w[5], "rmsnorm_rows_f16", "y");
                 }});
    // 15 gemm_qkv_rope
    c.push_back({"gemm_qkv_rope", "fast", {256, 1, 1}, false,
                 [](const uint32_t* w) {
                     const uint32_t heads = w[12] + 2 * w[13], rows = qkv_rows64(w[10], heads) ? 64 : 128;
                     return Grid3{heads, (int64_t(w[10]) + rows - 1) / rows, 1};
                 },
                 {TOK_R("h", DT(F16)), TOK_R("w", DT(F16)), TOK_R("q_norm", DT(BF16)), TOK_R("k_norm", DT(BF16)),
                  TOK_R("cos_table", DT(F32)), TOK_R("sin_table", DT(F32)), TOK_W("q", DT(F16)),
                  TOK_W("k_cache", DT(F16)), TOK_W("v_cache", DT(F16)), U32F("m"), U32F("hidden"), U32F("q_heads"),
                  U32F("kv_heads"), U32F("pos0"), U32F("max_pos"), F32F("eps")},
                 [](const uint32_t* w, const uint32_t* c) {
                     const int64_t m = w[10], hid = w[11], qh = w[12], kvh = w[13], pos0 = w[14], mp = w[15];
                     need_group2("gemm_qkv_rope", w[12], w[13]);
                     need_max_pos("gemm_qkv_rope", w[15]);  // the V cache's 64-position blocks
                     if (hid % 64 || hid < 64) contract_fail("gemm_qkv_rope: hidden must be a positive multiple of 64");
                     if (pos0 + m > mp) contract_fail("gemm_qkv_rope: positions past max_pos");
                     need(c, 0, m * hid, "gemm_qkv_rope", "h");
                     need(c, 1, (qh + 2 * kvh) * 128 * hid, "gemm_qkv_rope", "w");
                     need(c, 2, 128, "gemm_qkv_rope", "q_norm");
                     need(c, 3, 128, "gemm_qkv_rope", "k_norm");
                     need(c, 4, (pos0 + m) * 64, "gemm_qkv_rope", "cos_table");
                     need(c, 5, (pos0 + m) * 64, "gemm_qkv_rope", "sin_table");
                     need(c, 6, m * qh * 128, "gemm_qkv_rope", "q");
                     need(c, 7, kvh * mp * 128, "gemm_qkv_rope", "k_cache");
                     need(c, 8, kvh * mp * 128, "gemm_qkv_rope", "v_cache");
                 }});
    // 16 attention_prefill_f16: q, k_cache, v_cache, y, workspace, rows, past, q_heads, kv_heads, max_pos, scale
    c.push_back({"attention_prefill_f16", "fast", {256, 1, 1}, false,
                 [](const uint32_t* w) { return Grid3{(int64_t(w[6]) + kAttnRows - 1) / kAttnRows, w[9], 1}; },
                 {TOK_R("q", DT(F16)), TOK_R("k_cache", DT(F16)), TOK_R("v_cache", DT(F16)), TOK_W("y", DT(F16)),
                  TOK_RW("workspace", DT(U32)), U32F("rows"), U32F("past"), U32F("q_heads"), U32F("kv_heads"),
                  U32F("max_pos"), F32F("scale")},
                 [](const uint32_t* w, const uint32_t* c) {
                     const int64_t rows = w[6], past = w[7], qh = w[8], kvh = w[9], mp = w[10];
                     need_group2("attention_prefill_f16", w[8], w[9]);
                     need_max_pos("attention_prefill_f16", w[10]);
                     if (past + rows > mp) contract_fail("attention_prefill_f16: positions past max_pos");
                     need(c, 0, rows * qh * 128, "attention_prefill_f16", "q");
                     need(c, 1, kvh * mp * 128, "attention_prefill_f16", "k_cache");
                     need(c, 2, kvh * mp * 128, "attention_prefill_f16", "v_cache");
                     need(c, 3, rows * qh * 128, "attention_prefill_f16", "y");
                     need(c, 4, attn_prefill::workspace_words(rows, kvh), "attention_prefill_f16", "workspace");
                 }});
    // 17 gemm_residual: a, w, x, m, n, k, a_shift
    c.push_back({"gemm_residual", "fast", {256, 1, 1}, false,
                 [](const uint32_t* w) {
                     const int64_t bn = resid_narrow(w[4], w[5]) ? 64 : 128;
                     return Grid3{(int64_t(w[5]) + bn - 1) / bn, (int64_t(w[4]) + 127) / 128, 1};
                 },
                 {TOK_R("a", DT(F16)), TOK_R("w", DT(F16)), TOK_RW("x", DT(F32)), U32F("m"), U32F("n"), U32F("k"),
                  U32F("a_shift")},
                 [](const uint32_t* w, const uint32_t* c) {
                     if (w[6] % 64 || w[6] < 64) contract_fail("gemm_residual: k must be a positive multiple of 64");
                     need_a_shift("gemm_residual", w[7]);
                     need(c, 0, int64_t(w[4]) * w[6], "gemm_residual", "a");
                     need(c, 1, int64_t(w[5]) * w[6], "gemm_residual", "w");
                     need(c, 2, int64_t(w[4]) * w[5], "gemm_residual", "x");
                 }});
    // 18 gemm_swiglu: a, w, y, m, inter, k, a_shift
    c.push_back({"gemm_swiglu", "fast", {256, 1, 1}, false,
                 [](const uint32_t* w) {
                     const dim3 g = swiglu_grid(w[4], w[5]);
                     return Grid3{g.x, g.y, 1};
                 },
                 {TOK_R("a", DT(F16)), TOK_R("w", DT(F16)), TOK_W("y", DT(F16)), U32F("m"), U32F("inter"), U32F("k"),
                  U32F("a_shift")},
                 [](const uint32_t* w, const uint32_t* c) {
                     if (w[6] % 64 || w[6] < 64) contract_fail("gemm_swiglu: k must be a positive multiple of 64");
                     need_a_shift("gemm_swiglu", w[7]);
                     need(c, 0, int64_t(w[4]) * w[6], "gemm_swiglu", "a");
                     need(c, 1, 2 * int64_t(w[5]) * w[6], "gemm_swiglu", "w");
                     need(c, 2, int64_t(w[4]) * w[5], "gemm_swiglu", "y");
                 }});
    // 19 gemm_f32: a, w, y, m, n, k
    c.push_back({"gemm_f32", "fast", {256, 1, 1}, false,
                 [](const uint32_t* w) { return Grid3{(int64_t(w[5]) + 127) / 128, (int64_t(w[4]) + 127) / 128, 1}; },
                 {TOK_R("a", DT(F16)), TOK_R("w", DT(F16)), TOK_W("y", DT(F32)), U32F("m"), U32F("n"), U32F("k")},
                 [](const uint32_t* w, const uint32_t* c) {
                     if (w[6] % 64 || w[6] < 64) contract_fail("gemm_f32: k must be a positive multiple of 64");
                     need(c, 0, int64_t(w[4]) * w[6], "gemm_f32", "a");
                     need(c, 1, int64_t(w[5]) * w[6], "gemm_f32", "w");
                     need(c, 2, int64_t(w[4]) * w[5], "gemm_f32", "y");
                 }});
    // 20 gemv_norm_dec: x, norm, w, y, n, k, eps
    c.push_back({"gemv_norm_dec", "fast", {256, 1, 1}, true,
                 [](const uint32_t* w) { return Grid3{gemv_blocks(w[5]), 1, 1}; },
                 {TOK_R("x", DT(F32)), TOK_R("norm", DT(BF16)), TOK_R("w", DT(BF16)), TOK_W("y", DT(F32)), U32F("n"),
                  U32F("k"), F32F("eps")},
                 [](const uint32_t* w, const uint32_t* c) {
                     need_k("gemv_norm_dec", w[6]);
                     if (w[5] < 1) contract_fail("gemv_norm_dec: n must be at least 1");
                     need(c, 0, w[6], "gemv_norm_dec", "x");
                     need(c, 1, w[6], "gemv_norm_dec", "norm");
                     need(c, 2, int64_t(w[5]) * w[6], "gemv_norm_dec", "w");
                     need(c, 3, w[5], "gemv_norm_dec", "y");
                 }});
    // 21 attention_decode_f16 (the catalog's block size is the one-chunk form's; the multi-chunk form, chunks > 1 or
    // splits set, launches 512 threads)
    c.push_back({"attention_decode_f16", "fast", {256, 1, 1}, false,
                 [](const uint32_t* w) { return Grid3{dec_grid_splits(w[12], w[16], w[17]), w[11], w[15]}; },
                 {TOK_R("qkv", DT(F32)), TOK_R("q_norm", DT(BF16)), TOK_R("k_norm", DT(BF16)),
                  TOK_R("cos_table", DT(F32)), TOK_R("sin_table", DT(F32)), TOK_RW("k_cache", DT(F16)),
                  TOK_RW("v_cache", DT(F16)), TOK_W("partials", DT(F32)), TOK_R("state", DT(U32)), U32F("q_heads"),
                  U32F("kv_heads"), U32F("max_pos"), F32F("eps"), F32F("scale"), U32F("batch"), U32F("chunks"),
                  U32F("splits")},
                 [](const uint32_t* w, const uint32_t* c) {
                     const int64_t qh = w[10], kvh = w[11], mp = w[12], B = w[15];
                     need_group2("attention_decode_f16", w[10], w[11]);
                     need_max_pos("attention_decode_f16", w[12]);
                     need_batch("attention_decode_f16", w[15]);
                     need_chunks("attention_decode_f16", w[16]);
                     need_splits("attention_decode_f16", w[17], w[12]);
                     need(c, 0, B * (qh + 2 * kvh) * 128, "attention_decode_f16", "qkv");
                     need(c, 1, 128, "attention_decode_f16", "q_norm");
                     need(c, 2, 128, "attention_decode_f16", "k_norm");
                     need(c, 3, mp * 64, "attention_decode_f16", "cos_table");
                     need(c, 4, mp * 64, "attention_decode_f16", "sin_table");
                     need(c, 5, B * kvh * mp * 128, "attention_decode_f16", "k_cache");
                     need(c, 6, B * kvh * mp * 128, "attention_decode_f16", "v_cache");
                     need(c, 7, B * qh * (mp / 64) * 130, "attention_decode_f16", "partials");
                     need(c, 8, 2 * B + 1, "attention_decode_f16", "state");
                 }});
    // 22 attention_combine: partials, y, state, q_heads, max_pos
    c.push_back({"attention_combine", "fast", {256, 1, 1}, false, [](const uint32_t* w) { return Grid3{w[4], w[6], 1}; },
                 {TOK_R("partials", DT(F32)), TOK_W("y", DT(F32)), TOK_R("state", DT(U32)), U32F("q_heads"),
                  U32F("max_pos"), U32F("batch"), U32F("chunks"), U32F("splits")},
                 [](const uint32_t* w, const uint32_t* c) { check_combine("attention_combine", w, c); }});
    // 23 gemv_residual_dec: a, w, x, n, k
    c.push_back({"gemv_residual_dec", "fast", {256, 1, 1}, true,
                 [](const uint32_t* w) { return Grid3{gemv_blocks(w[4]), 1, 1}; },
                 {TOK_R("a", DT(F32)), TOK_R("w", DT(BF16)), TOK_RW("x", DT(F32)), U32F("n"), U32F("k")},
                 [](const uint32_t* w, const uint32_t* c) {
                     need_k("gemv_residual_dec", w[5]);
                     if (w[4] < 1) contract_fail("gemv_residual_dec: n must be at least 1");
                     need(c, 0, w[5], "gemv_residual_dec", "a");
                     need(c, 1, int64_t(w[4]) * w[5], "gemv_residual_dec", "w");
                     need(c, 2, w[4], "gemv_residual_dec", "x");
                 }});
    // 24 gemv_swiglu_dec: x, norm, w, y, inter, hidden, eps
    c.push_back({"gemv_swiglu_dec", "fast", {256, 1, 1}, true,
                 [](const uint32_t* w) { return Grid3{gemv_blocks(w[5]), 1, 1}; },
                 {TOK_R("x", DT(F32)), TOK_R("norm", DT(BF16)), TOK_R("w", DT(BF16)), TOK_W("y", DT(F32)),
                  U32F("inter"), U32F("hidden"), F32F("eps")},
                 [](const uint32_t* w, const uint32_t* c) {
                     need_k("gemv_swiglu_dec", w[6]);
                     if (w[5] < 1) contract_fail("gemv_swiglu_dec: inter must be at least 1");
                     need(c, 0, w[6], "gemv_swiglu_dec", "x");
                     need(c, 1, w[6], "gemv_swiglu_dec", "norm");
                     need(c, 2, 2 * int64_t(w[5]) * w[6], "gemv_swiglu_dec", "w");
                     need(c, 3, w[5], "gemv_swiglu_dec", "y");
                 }});
    // 25 lmhead_dec: x, norm, embed, logits, partials, vocab, hidden, eps, write_logits
    c.push_back({"lmhead_dec", "fast", {256, 1, 1}, true, [](const uint32_t*) { return Grid3{kLmheadBlocks, 1, 1}; },
                 {TOK_R("x", DT(F32)), TOK_R("norm", DT(BF16)), TOK_R("embed", DT(BF16)), TOK_W("logits", DT(F32)),
                  TOK_W("partials", DT(F32)), U32F("vocab"), U32F("hidden"), F32F("eps"), U32F("write_logits")},
                 [](const uint32_t* w, const uint32_t* c) {
                     need_k("lmhead_dec", w[7]);
                     if (w[6] < 1) contract_fail("lmhead_dec: vocab must be at least 1");
                     need(c, 0, w[7], "lmhead_dec", "x");
                     need(c, 1, w[7], "lmhead_dec", "norm");
                     need(c, 2, int64_t(w[6]) * w[7], "lmhead_dec", "embed");
                     need(c, 3, w[9] ? int64_t(w[6]) : 0, "lmhead_dec", "logits");
                     need(c, 4, 2 * int64_t(kLmheadBlocks), "lmhead_dec", "partials");
                 }});
    // 26 argmax_dec (one sequence): partials, state, out_ids, max_steps
    c.push_back({"argmax_dec", "fast", {1024, 1, 1}, true, [](const uint32_t*) { return Grid3{1, 1, 1}; },
                 {TOK_R("partials", DT(F32)), TOK_RW("state", DT(U32)), TOK_W("out_ids", DT(U32)), U32F("max_steps")},
                 [](const uint32_t* w, const uint32_t* c) {
                     need(c, 0, 2 * int64_t(kLmheadBlocks), "argmax_dec", "partials");
                     need(c, 1, 3, "argmax_dec", "state");
                     need(c, 2, w[4], "argmax_dec", "out_ids");
                 }});
    // 27 embed_dec: embed, state, x, hidden, vocab
    c.push_back({"embed_dec", "fast", {256, 1, 1}, true, [](const uint32_t* w) { return Grid3{w[6], 1, 1}; },
                 {TOK_R("embed", DT(BF16)), TOK_R("state", DT(U32)), TOK_W("x", DT(F32)), U32F("hidden"),
                  U32F("vocab"), U32F("batch")},
                 [](const uint32_t* w, const uint32_t* c) {
                     need_batch("embed_dec", w[6]);
                     need(c, 0, int64_t(w[4]) * w[5], "embed_dec", "embed");
                     need(c, 1, 2 * int64_t(w[6]) + 1, "embed_dec", "state");
                     need(c, 2, int64_t(w[6]) * w[4], "embed_dec", "x");
                 }});
    // 28 fill_normal_f16: y, n, seed_lo, seed_hi, stream_lo, stream_hi, std
    c.push_back({"fill_normal_f16", "fast", {256, 1, 1}, true,
                 [](const uint32_t* w) { return Grid3{(int64_t(w[2]) / 2 + 255) / 256 + 1, 1, 1}; },
                 {TOK_W("y", DT(F16)), U32F("n"), U32F("seed_lo"), U32F("seed_hi"), U32F("stream_lo"),
                  U32F("stream_hi"), F32F("std")},
                 [](const uint32_t* w, const uint32_t* c) { need(c, 0, w[2], "fill_normal_f16", "y"); }});
    // 29 convert_bf16_f16: x, y, n
    c.push_back({"convert_bf16_f16", "fast", {256, 1, 1}, true,
                 [](const uint32_t* w) { return Grid3{(int64_t(w[3]) / 8 + 255) / 256 + 1, 1, 1}; },
                 {TOK_R("x", DT(BF16)), TOK_W("y", DT(F16)), U32F("n")},
                 [](const uint32_t* w, const uint32_t* c) {
                     need(c, 0, w[3], "convert_bf16_f16", "x");
                     need(c, 1, w[3], "convert_bf16_f16", "y");
                 }});
    // 30 argmax_rows_partial: x, partials, rows, cols, row0
    c.push_back({"argmax_rows_partial", "fast", {256, 1, 1}, false,
                 [](const uint32_t* w) { return Grid3{kArgmaxParts, w[3], 1}; },
                 {TOK_R("x", DT(F32)), TOK_W("partials", DT(F32)), U32F("rows"), U32F("cols"), U32F("row0")},
                 [](const uint32_t* w, const uint32_t* c) {
                     if (w[3] < 1 || w[4] < 1) contract_fail("argmax_rows_partial: rows and cols must be at least 1");
                     need(c, 0, (int64_t(w[5]) + w[3]) * w[4], "argmax_rows_partial", "x");
                     need(c, 1, int64_t(w[3]) * kArgmaxParts * 2, "argmax_rows_partial", "partials");
                 }});
    // 31 argmax_rows_final: partials, out, rows
    c.push_back({"argmax_rows_final", "fast", {64, 1, 1}, true, [](const uint32_t* w) { return Grid3{w[3], 1, 1}; },
                 {TOK_R("partials", DT(F32)), TOK_W("out", DT(U32)), U32F("rows")},
                 [](const uint32_t* w, const uint32_t* c) {
                     need(c, 0, int64_t(w[3]) * kArgmaxParts * 2, "argmax_rows_final", "partials");
                     need(c, 1, w[3], "argmax_rows_final", "out");
                 }});
    // 32 gemm_skinny_f32: a, w, y, m, n, k
    c.push_back({"gemm_skinny_f32", "fast", {512, 1, 1}, false,
                 [](const uint32_t* w) {
                     return Grid3{skinny_one_tile(w[5]) ? (int64_t(w[5]) + 15) / 16 : (int64_t(w[5]) + 31) / 32, 1, 1};
                 },
                 {TOK_R("a", DT(F16)), TOK_R("w", DT(F16)), TOK_W("y", DT(F32)), U32F("m"), U32F("n"), U32F("k")},
                 [](const uint32_t* w, const uint32_t* c) { check_skinny("gemm_skinny_f32", w, c, w[5], w[5]); }});
    // 33 gemm_skinny_residual: a, w, x, m, n, k, a_shift
    c.push_back({"gemm_skinny_residual", "fast", {512, 1, 1}, false,
                 [](const uint32_t* w) { return Grid3{(int64_t(w[5]) + 15) / 16, 1, 1}; },
                 {TOK_R("a", DT(F16)), TOK_R("w", DT(F16)), TOK_RW("x", DT(F32)), U32F("m"), U32F("n"), U32F("k"),
                  U32F("a_shift")},
                 [](const uint32_t* w, const uint32_t* c) {
                     check_skinny("gemm_skinny_residual", w, c, w[5], w[5]);
                     need_a_shift("gemm_skinny_residual", w[7]);
                 }});
    // 34 gemm_skinny_swiglu: a, w (2 inter rows), y, m, inter, k, a_shift
    c.push_back({"gemm_skinny_swiglu", "fast", {512, 1, 1}, false,
                 [](const uint32_t* w) {
                     const int64_t pairs = skinny_swiglu_pairs(w[5]);
                     return Grid3{(int64_t(w[5]) + pairs - 1) / pairs, 1, 1};
                 },
                 {TOK_R("a", DT(F16)), TOK_R("w", DT(F16)), TOK_W("y", DT(F16)), U32F("m"), U32F("inter"), U32F("k"),
                  U32F("a_shift")},
                 [](const uint32_t* w, const uint32_t* c) {
                     need_a_shift("gemm_skinny_swiglu", w[7]);
                     check_skinny("gemm_skinny_swiglu", w, c, 2 * int64_t(w[5]), w[5]);
                 }});
    // 35 attention_combine_f16: partials, y (f16), state, q_heads, max_pos, batch
    c.push_back({"attention_combine_f16", "fast", {256, 1, 1}, false,
                 [](const uint32_t* w) { return Grid3{w[4], w[6], 1}; },
                 {TOK_R("partials", DT(F32)), TOK_W("y", DT(F16)), TOK_R("state", DT(U32)), U32F("q_heads"),
                  U32F("max_pos"), U32F("batch"), U32F("chunks"), U32F("splits")},
                 [](const uint32_t* w, const uint32_t* c) { check_combine("attention_combine_f16", w, c); }});
    // 36 decode_advance: argmax, state, out_ids, batch, max_steps
    c.push_back({"decode_advance", "fast", {256, 1, 1}, true, [](const uint32_t*) { return Grid3{1, 1, 1}; },
                 {TOK_R("argmax", DT(U32)), TOK_RW("state", DT(U32)), TOK_W("out_ids", DT(U32)), U32F("batch"),
                  U32F("max_steps")},
                 [](const uint32_t* w, const uint32_t* c) {
                     need_batch("decode_advance", w[4]);
                     need(c, 0, w[4], "decode_advance", "argmax");
                     need(c, 1, 2 * int64_t(w[4]) + 1, "decode_advance", "state");
                     need(c, 2, int64_t(w[4]) * w[5], "decode_advance", "out_ids");
                 }});
    // 37 prefetch: x0, x1, x2, x3 (read through the caches, nothing written; repeat a tensor to prefetch fewer)
    c.push_back({"prefetch", "fast", {256, 1, 1}, false, [](const uint32_t*) { return Grid3{256, 1, 1}; },
                 {TOK_R("x0", DT(F32) | DT(BF16) | DT(F16) | DT(U32)), TOK_R("x1", DT(F32) | DT(BF16) | DT(F16) | DT(U32)),
                  TOK_R("x2", DT(F32) | DT(BF16) | DT(F16) | DT(U32)), TOK_R("x3", DT(F32) | DT(BF16) | DT(F16) | DT(U32))},
                 [](const uint32_t*, const uint32_t*) {}});
    // 38 decode_step_persistent: the whole one-sequence decode step in one launch of `blocks` resident workgroups.
    // Weights and caches are the layer-stacked tensors ([layers, ...]); the projection matrices and the lm_head
    // (embed16) are their exact fp16 copies; embed (bf16) feeds the embedding row. The exchange buffer holds the header
    // and the tagged hand-off entries (persist::exchange_entries 8-byte entries).
    c.push_back({"decode_step_persistent", "fast", {persist::kThreads, 1, 1}, true,
                 [](const uint32_t* w) { return Grid3{w[31], 1, 1}; },
                 {TOK_R("embed", DT(BF16)), TOK_R("final_norm", DT(BF16)), TOK_R("in_norm", DT(BF16)),
                  TOK_R("qkv", DT(F16)), TOK_R("q_norm", DT(BF16)), TOK_R("k_norm", DT(BF16)), TOK_R("o_proj", DT(F16)),
                  TOK_R("post_norm", DT(BF16)), TOK_R("gate_up", DT(F16)), TOK_R("down", DT(F16)),
                  TOK_RW("k_cache", DT(F16)), TOK_RW("v_cache", DT(F16)), TOK_R("cos", DT(F32)), TOK_R("sin", DT(F32)),
                  TOK_W("logits", DT(F32)), TOK_RW("state", DT(U32)), TOK_W("out_ids", DT(U32)),
                  TOK_RW("exchange", DT(U32)), TOK_R("embed16", DT(F16)), U32F("layers"), U32F("hidden"),
                  U32F("q_heads"), U32F("kv_heads"), U32F("inter"), U32F("vocab"), U32F("max_pos"), U32F("max_steps"),
                  U32F("write_logits"), F32F("eps"), F32F("scale"), U32F("blocks")},
                 [](const uint32_t* w, const uint32_t* c) {
                     const int64_t L = w[20], H = w[21], QH = w[22], KVH = w[23], I = w[24], V = w[25], MP = w[26];
                     const persist::Shape sh{int(H), int(QH), int(KVH), 128, int(I), int(MP), int(w[31])};
                     if (L < 1 || V < 1 || MP < 1) contract_fail("decode_step_persistent: layers, vocab and max_pos >= 1");
                     if (const char* why = persist::unsupported(sh))
                         contract_fail("decode_step_persistent: this shape is not covered (%s)", why);
                     const int64_t N1 = (QH + 2 * KVH) * 128;
                     need(c, 0, V * H, "decode_step_persistent", "embed");
                     need(c, 1, H, "decode_step_persistent", "final_norm");
                     need(c, 2, L * H, "decode_step_persistent", "in_norm");
                     need(c, 3, L * N1 * H, "decode_step_persistent", "qkv");
                     need(c, 4, L * 128, "decode_step_persistent", "q_norm");
                     need(c, 5, L * 128, "decode_step_persistent", "k_norm");
                     need(c, 6, L * H * QH * 128, "decode_step_persistent", "o_proj");
                     need(c, 7, L * H, "decode_step_persistent", "post_norm");
                     need(c, 8, L * 2 * I * H, "decode_step_persistent", "gate_up");
                     need(c, 9, L * H * I, "decode_step_persistent", "down");
                     need(c, 10, L * KVH * MP * 128, "decode_step_persistent", "k_cache");
                     need(c, 11, L * KVH * MP * 128, "decode_step_persistent", "v_cache");
                     need(c, 12, MP * 64, "decode_step_persistent", "cos");
                     need(c, 13, MP * 64, "decode_step_persistent", "sin");
                     need(c, 14, w[28] ? V : 0, "decode_step_persistent", "logits");
                     need(c, 15, 3, "decode_step_persistent", "state");
                     need(c, 16, w[27], "decode_step_persistent", "out_ids");
                     need(c, 17, 2 * int64_t(persist::exchange_entries(int(L), sh)), "decode_step_persistent", "exchange");
                     need(c, 18, V * H, "decode_step_persistent", "embed16");
                 }});
    // 39 gemm_residual_split: a, w, partials, m, n, k, splits, a_shift. partials[z] = 2^a_shift a[:, k range z] .
    // w[:, k range z]^T, the k range split in `splits` equal parts of multiples of 64; residual_add_norm adds them to
    // the residual stream. For
    // m <= 16 with 1024-multiples per split it runs as a skinny GEMM (512 threads, one block per 16 columns and split).
    c.push_back({"gemm_residual_split", "fast", {256, 1, 1}, false,
                 [](const uint32_t* w) {
                     if (resid_split_skinny(w[4], w[6], w[7])) return Grid3{(int64_t(w[5]) + 15) / 16, w[7], 1};
                     const int64_t gx = (int64_t(w[5]) + 63) / 64, g128 = (int64_t(w[4]) + 127) / 128;
                     const int64_t rows = resid_rows64(w[4], uint64_t(gx * g128 * w[7])) ? 64 : 128;
                     return Grid3{gx, (int64_t(w[4]) + rows - 1) / rows, w[7]};
                 },
                 {TOK_R("a", DT(F16)), TOK_R("w", DT(F16)), TOK_W("partials", DT(F32)), U32F("m"), U32F("n"), U32F("k"),
                  U32F("splits"), U32F("a_shift")},
                 [](const uint32_t* w, const uint32_t* c) {
                     const int64_t m = w[4], n = w[5], k = w[6], sp = w[7];
                     need_a_shift("gemm_residual_split", w[8]);
                     if (sp != 1 && sp != 2 && sp != 4 && sp != 8)
                         contract_fail("gemm_residual_split: splits must be 1, 2, 4 or 8");
                     if (k < 64 * sp || k % (64 * sp))
                         contract_fail("gemm_residual_split: k must be a positive multiple of 64 * splits");
                     if (m < 1 || n < 1) contract_fail("gemm_residual_split: m and n must be at least 1");
                     need(c, 0, m * k, "gemm_residual_split", "a");
                     need(c, 1, n * k, "gemm_residual_split", "w");
                     need(c, 2, sp * m * n, "gemm_residual_split", "partials");
                 }});
    // 40 residual_add_norm: x, partials, w, y, rows, cols, splits, eps. x += the partials in split order, then
    // y = RMSNorm(x) in f16 (as rmsnorm_rows_f16). The catalog's block size is the four-row form's; up to 64 rows
    // launch one 64-thread block per row
    c.push_back({"residual_add_norm", "fast", {256, 1, 1}, true,
                 [](const uint32_t* w) { return Grid3{w[5] <= 64 ? int64_t(w[5]) : (int64_t(w[5]) + 3) / 4, 1, 1}; },
                 {TOK_RW("x", DT(F32)), TOK_R("partials", DT(F32)), TOK_R("w", DT(BF16)), TOK_W("y", DT(F16)),
                  U32F("rows"), U32F("cols"), U32F("splits"), F32F("eps")},
                 [](const uint32_t* w, const uint32_t* c) {
                     const int64_t rows = w[5], cols = w[6], sp = w[7];
                     if (cols != 256 && cols != 512 && cols != 1024 && cols != 2048 && cols != 4096)
                         contract_fail("residual_add_norm: cols must be 256, 512, 1024, 2048 or 4096");
                     if (sp != 1 && sp != 2 && sp != 4 && sp != 8)
                         contract_fail("residual_add_norm: splits must be 1, 2, 4 or 8");
                     need(c, 0, rows * cols, "residual_add_norm", "x");
                     need(c, 1, sp * rows * cols, "residual_add_norm", "partials");
                     need(c, 2, cols, "residual_add_norm", "w");
                     need(c, 3, rows * cols, "residual_add_norm", "y");
                 }});
    return c;
}

}  // namespace lrm
