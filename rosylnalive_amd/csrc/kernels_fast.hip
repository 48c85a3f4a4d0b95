// The bf16 fast path of the HIP device (appended catalog ids 14 and up): bf16 activations into MFMA GEMMs with fused
// epilogues, an MFMA flash-attention prefill kernel, and memory-bound decode kernels. gfx950 (CDNA4) only, wave64.
//
// Data layout in HBM (chosen by the executor, see qwen_exec.cpp):
//   residual stream x          f32  [T, hidden]
//   GEMM inputs (h, o, a)      bf16 [T, k]                     (k contiguous: the MFMA A operand)
//   weights                    bf16 [n, k] (PyTorch Linear)    q|k|v rows fused into one [QC + 2 KC, hidden],
//                                                              gate|up rows fused into one [2 I, hidden]
//   K cache                    bf16 [kv_heads, max_pos, head_dim]   (head-major: one head's keys are contiguous)
//   V cache                    bf16 [kv_heads, head_dim, max_pos]   (transposed: the MFMA A operand of O^T = V^T P^T)
//
// MFMA: v_mfma_f32_16x16x32_bf16. Operand layout (lane l, g = l / 16, c = l % 16): A supplies row c, k = 8g .. 8g + 7;
// B supplies column c, k = 8g .. 8g + 7; D holds rows 4g .. 4g + 3 of column c.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>

#include "device.hpp"
#include "fast_common.hpp"

namespace lrm {
using namespace fast;

static constexpr float kLog2e = 1.4426950408889634f;

// ================================================================ 14 rmsnorm_rows_bf16
// y[r, :] = bf16(widen(w) * (x[row0 + r, :] * rsqrt-free r)), r = 1 / sqrt(sum(x^2) / cols + eps). One block per row.
__global__ __launch_bounds__(256) void k_rmsnorm_bf16(const float* x, const uint16_t* w, uint16_t* y, uint32_t rows,
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
    for (uint32_t c = threadIdx.x; c < cols; c += 256u) yr[c] = f2bf(bf2f(w[c]) * (xr[c] * rr));
}

// ================================================================ GEMM (ids 15, 17, 18, 19)
// C[m, n] = sum_k A[m, k] W[n, k], 128 x 128 tiles, k in steps of 64, 4 waves each owning a 64 x 64 quarter as 4 x 4
// MFMA tiles. The next k-tile is fetched into registers while the current one is multiplied out of LDS.
constexpr int GBM = 128, GBN = 128, GBK = 64, GLD = GBK + 8;  // LDS row stride (bf16), padded against bank conflicts

enum Epi { EPI_F32 = 0, EPI_RESID = 1, EPI_SWIGLU = 2, EPI_QKV = 3 };

struct GemmArgs {
    const uint16_t* a;
    const uint16_t* w;
    int M, N, K;
    float* y32;           // F32, RESID (in place over resid)
    const float* resid;   // RESID
    uint16_t* y16;        // SWIGLU: [M, inter]
    int inter;            // SWIGLU: I (the W rows are gate 0..I-1 then up I..2I-1)
    // QKV: one 128-column tile per head; q heads, then k heads, then v heads
    const uint16_t* qn;
    const uint16_t* kn;
    const float* cos_t;
    const float* sin_t;
    uint16_t* q_out;      // [M, qh * 128]
    uint16_t* kc;         // [kvh, max_pos, 128]
    uint16_t* vc;         // [kvh, 128, max_pos]
    int qh, kvh, pos0, max_pos;
    float eps;
};

template <int EPI>
__global__ __launch_bounds__(256) void k_gemm(GemmArgs p) {
    __shared__ __attribute__((aligned(16))) uint16_t lds[(GBM + GBN) * GLD];
    uint16_t* As = lds;
    uint16_t* Bs = lds + GBM * GLD;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6, wm = w >> 1, wn = w & 1, g = lane >> 4, c16 = lane & 15;
    const int m0 = blockIdx.y * GBM;
    const int n0 = blockIdx.x * GBN;

    uint4 ra[4], rb[4];
    auto brow = [&](int r) -> int {
        if (EPI == EPI_SWIGLU) {
            int j = blockIdx.x * 64 + (r & 63);
            if (j >= p.inter) return -1;
            return r < 64 ? j : p.inter + j;
        }
        int n = n0 + r;
        return n < p.N ? n : -1;
    };
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            int c = t + 256 * i, r = c >> 3, kc = (c & 7) * 8;
            int m = m0 + r;
            ra[i] = m < p.M ? *reinterpret_cast<const uint4*>(p.a + size_t(m) * p.K + k0 + kc) : make_uint4(0, 0, 0, 0);
            int n = brow(r);
            rb[i] = n >= 0 ? *reinterpret_cast<const uint4*>(p.w + size_t(n) * p.K + k0 + kc) : make_uint4(0, 0, 0, 0);
        }
    };
    auto sstore = [&]() {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            int c = t + 256 * i, r = c >> 3, kc = (c & 7) * 8;
            *reinterpret_cast<uint4*>(As + r * GLD + kc) = ra[i];
            *reinterpret_cast<uint4*>(Bs + r * GLD + kc) = rb[i];
        }
    };

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int nk = p.K / GBK;
    gload(0);
    for (int kt = 0; kt < nk; ++kt) {
        __syncthreads();
        sstore();
        __syncthreads();
        if (kt + 1 < nk) gload((kt + 1) * GBK);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            bf16x8 af[4], bfr[4];
            const int kof = ks * 32 + 8 * g;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                af[i] = as_bf16x8(*reinterpret_cast<const uint4*>(As + (wm * 64 + i * 16 + c16) * GLD + kof));
#pragma unroll
            for (int j = 0; j < 4; ++j)
                bfr[j] = as_bf16x8(*reinterpret_cast<const uint4*>(Bs + (wn * 64 + j * 16 + c16) * GLD + kof));
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
        }
    }

    if (EPI == EPI_F32 || EPI == EPI_RESID) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                int n = n0 + wn * 64 + j * 16 + c16;
                if (n >= p.N) continue;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    int m = m0 + wm * 64 + i * 16 + 4 * g + r;
                    if (m >= p.M) continue;
                    size_t o = size_t(m) * p.N + n;
                    p.y32[o] = EPI == EPI_RESID ? p.resid[o] + acc[i][j][r] : acc[i][j][r];
                }
            }
        return;
    }

    // SWIGLU and QKV pair column c (wave wn = 0) with column c + 64 (wave wn = 1, same lane and tile index): the
    // second half goes through LDS to the first.
    __syncthreads();
    float* x32 = reinterpret_cast<float*>(lds);  // 2 (wm) x 64 values x 64 lanes = 32 KiB
    if (wn == 1) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) x32[((wm * 16 + i * 4 + j) * 4 + r) * 64 + lane] = acc[i][j][r];
    }
    __syncthreads();
    if (wn == 1) return;
    float hi[4][4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) hi[i][j][r] = x32[((wm * 16 + i * 4 + j) * 4 + r) * 64 + lane];

    if (EPI == EPI_SWIGLU) {
        // a[m, j0 + c] = silu(gate) * up, silu(g) = g / (1 + exp(-g))
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                int col = blockIdx.x * 64 + j * 16 + c16;
                if (col >= p.inter) continue;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    int m = m0 + wm * 64 + i * 16 + 4 * g + r;
                    if (m >= p.M) continue;
                    float gv = acc[i][j][r];
                    float s = gv / (1.0f + __expf(-gv));
                    p.y16[size_t(m) * p.inter + col] = f2bf(s * hi[i][j][r]);
                }
            }
        return;
    }

    // QKV: head = blockIdx.x (q heads, then k heads, then v heads), head_dim 128 = this tile's columns.
    const int head = blockIdx.x;
    const bool is_q = head < p.qh, is_k = !is_q && head < p.qh + p.kvh;
    const uint16_t* nw = is_q ? p.qn : p.kn;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = m0 + wm * 64 + i * 16 + 4 * g + r;  // the same for the 16 lanes of group g
            float ss = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j) ss = fmaf(acc[i][j][r], acc[i][j][r], fmaf(hi[i][j][r], hi[i][j][r], ss));
            ss += __shfl_xor(ss, 1, 64);
            ss += __shfl_xor(ss, 2, 64);
            ss += __shfl_xor(ss, 4, 64);
            ss += __shfl_xor(ss, 8, 64);
            if (m >= p.M) continue;
            const int pos = p.pos0 + m;
            const float rr = 1.0f / sqrtf(ss / 128.0f + p.eps);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int c = j * 16 + c16;  // 0..63
                float lo = acc[i][j][r], h2 = hi[i][j][r];
                if (is_q || is_k) {
                    float a = bf2f(nw[c]) * (lo * rr);
                    float b = bf2f(nw[c + 64]) * (h2 * rr);
                    float cs = p.cos_t[size_t(pos) * 64 + c], sn = p.sin_t[size_t(pos) * 64 + c];
                    lo = a * cs - b * sn;
                    h2 = b * cs + a * sn;
                }
                if (is_q) {
                    uint16_t* qo = p.q_out + size_t(m) * (p.qh * 128) + head * 128;
                    qo[c] = f2bf(lo);
                    qo[c + 64] = f2bf(h2);
                } else if (is_k) {
                    uint16_t* ko = p.kc + (size_t(head - p.qh) * p.max_pos + pos) * 128;
                    ko[c] = f2bf(lo);
                    ko[c + 64] = f2bf(h2);
                } else {
                    uint16_t* vo = p.vc + size_t(head - p.qh - p.kvh) * 128 * p.max_pos + pos;
                    vo[size_t(c) * p.max_pos] = f2bf(lo);
                    vo[size_t(c + 64) * p.max_pos] = f2bf(h2);
                }
            }
        }
    }
}

// ================================================================ 16 attention_prefill_bf16
// Causal GQA flash attention, two query heads per KV head. A workgroup takes 64 query rows of both heads of one KV
// group (128 query columns, 32 per wave) and streams 64-key blocks of K and V^T through LDS, shared by both heads.
// S^T = K Q^T (A = K rows from LDS, B = Q^T from registers) puts one query per lane column, so the online-softmax
// statistics stay per lane; P^T is then already in the B-operand layout of O^T = V^T P^T once the key slots of the
// k-step are ordered {4g .. 4g + 3, 16 + 4g .. 16 + 4g + 3} — the same order is used to read V^T, so the sum is over
// the same keys.
__global__ __launch_bounds__(256) void k_attn_prefill(const uint16_t* q, const uint16_t* kc, const uint16_t* vc,
                                                      uint16_t* y, int T, int past, int qh, int kvh, int max_pos,
                                                      float scale_log2) {
    __shared__ __attribute__((aligned(16))) uint16_t Ks[64 * 136];
    __shared__ __attribute__((aligned(16))) uint16_t Vt[128 * 72];
    const int t = threadIdx.x, lane = t & 63, w = t >> 6, g = lane >> 4, c16 = lane & 15;
    const int ntile = (T + 63) / 64;
    const int row0 = (ntile - 1 - int(blockIdx.x)) * 64;  // the longest tiles start first
    const int kvhead = blockIdx.y;
    const int head = kvhead * 2 + (w >> 1);
    const int wrow0 = row0 + (w & 1) * 32;
    const int QC = qh * 128;
    (void)kvh;

    bf16x8 qf[2][4];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        int row = wrow0 + nt * 16 + c16;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            uint4 v = make_uint4(0, 0, 0, 0);
            if (row < T) v = *reinterpret_cast<const uint4*>(q + size_t(row) * QC + head * 128 + ks * 32 + 8 * g);
            qf[nt][ks] = as_bf16x8(v);
        }
    }
    float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};
    f32x4 o[8][2];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) o[dt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int last_row = min(row0 + 63, T - 1);
    const int kend = past + last_row + 1;
    const uint16_t* kbase = kc + size_t(kvhead) * max_pos * 128;
    const uint16_t* vbase = vc + size_t(kvhead) * 128 * max_pos;
    for (int kb = 0; kb < kend; kb += 64) {
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            int c = t + 256 * i, key = c >> 4, dc = (c & 15) * 8;
            uint4 v = make_uint4(0, 0, 0, 0);
            if (kb + key < kend) v = *reinterpret_cast<const uint4*>(kbase + size_t(kb + key) * 128 + dc);
            *reinterpret_cast<uint4*>(Ks + key * 136 + dc) = v;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            int c = t + 256 * i, d = c >> 3, k8 = (c & 7) * 8;
            uint4 v = make_uint4(0, 0, 0, 0);
            if (kb + k8 < kend) {
                v = *reinterpret_cast<const uint4*>(vbase + size_t(d) * max_pos + kb + k8);
                int valid = kend - (kb + k8);  // keys past kend hold anything: zero them
                if (valid < 8) {
                    uint32_t* u = reinterpret_cast<uint32_t*>(&v);
                    for (int e = 0; e < 8; ++e)
                        if (e >= valid) u[e >> 1] &= (e & 1) ? 0x0000FFFFu : 0xFFFF0000u;
                }
            }
            *reinterpret_cast<uint4*>(Vt + d * 72 + k8) = v;
        }
        __syncthreads();

        f32x4 s[4][2];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) s[kt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) {
                bf16x8 a = as_bf16x8(*reinterpret_cast<const uint4*>(Ks + (kt * 16 + c16) * 136 + ks * 32 + 8 * g));
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) s[kt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[nt][ks], s[kt][nt], 0, 0, 0);
            }

        uint32_t pb[2][2][4];  // [kk][nt]: the B operand of O^T for keys of k-step kk, packed bf16 pairs
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            const int row = wrow0 + nt * 16 + c16;
            const int qpos = past + row;
            float mloc = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    int key = kb + kt * 16 + 4 * g + r;
                    float v = s[kt][nt][r] * scale_log2;
                    if (row >= T || key > qpos) v = -INFINITY;
                    s[kt][nt][r] = v;
                    mloc = fmaxf(mloc, v);
                }
            mloc = fmaxf(mloc, __shfl_xor(mloc, 16, 64));
            mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
            const float m_new = fmaxf(m_run[nt], mloc);
            const float m_use = m_new == -INFINITY ? 0.f : m_new;
            const float alpha = exp2f(m_run[nt] - m_use);
            float lsum = 0.f;
            float pv[4][4];
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    pv[kt][r] = exp2f(s[kt][nt][r] - m_use);
                    lsum += pv[kt][r];
                }
            lsum += __shfl_xor(lsum, 16, 64);
            lsum += __shfl_xor(lsum, 32, 64);
            l_run[nt] = l_run[nt] * alpha + lsum;
            m_run[nt] = m_new;
#pragma unroll
            for (int dt = 0; dt < 8; ++dt)
#pragma unroll
                for (int r = 0; r < 4; ++r) o[dt][nt][r] *= alpha;
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                pb[kk][nt][0] = pack2(pv[2 * kk][0], pv[2 * kk][1]);
                pb[kk][nt][1] = pack2(pv[2 * kk][2], pv[2 * kk][3]);
                pb[kk][nt][2] = pack2(pv[2 * kk + 1][0], pv[2 * kk + 1][1]);
                pb[kk][nt][3] = pack2(pv[2 * kk + 1][2], pv[2 * kk + 1][3]);
            }
        }
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            bf16x8 bq[2];
#pragma unroll
            for (int nt = 0; nt < 2; ++nt)
                bq[nt] = as_bf16x8(make_uint4(pb[kk][nt][0], pb[kk][nt][1], pb[kk][nt][2], pb[kk][nt][3]));
#pragma unroll
            for (int dt = 0; dt < 8; ++dt) {
                const uint16_t* vr = Vt + (dt * 16 + c16) * 72 + kk * 32 + 4 * g;
                uint2 lo = *reinterpret_cast<const uint2*>(vr);
                uint2 hi = *reinterpret_cast<const uint2*>(vr + 16);
                bf16x8 a = as_bf16x8(make_uint4(lo.x, lo.y, hi.x, hi.y));
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) o[dt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bq[nt], o[dt][nt], 0, 0, 0);
            }
        }
    }
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const int row = wrow0 + nt * 16 + c16;
        if (row >= T) continue;
        const float inv = 1.0f / l_run[nt];
        uint16_t* yr = y + size_t(row) * QC + head * 128;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
            uint2 v;
            v.x = pack2(o[dt][nt][0] * inv, o[dt][nt][1] * inv);
            v.y = pack2(o[dt][nt][2] * inv, o[dt][nt][3] * inv);
            *reinterpret_cast<uint2*>(yr + dt * 16 + 4 * g) = v;
        }
    }
}

// ================================================================ decode kernels (one token per step)
// The step state is device memory: state[0] = the position being decoded, state[1] = its token id, state[2] = the
// step index. The lm_head kernel writes the next id and advances the state, so a recorded step replays unchanged.

// Loads x (and applies an RMSNorm with weight nw when nw != nullptr) into LDS as f32.
__device__ __forceinline__ void load_x_norm(const float* x, const uint16_t* nw, float eps, int K, float* xs, float* red) {
    float ss = 0.f;
    for (int k = threadIdx.x; k < K; k += blockDim.x) {
        float v = x[k];
        xs[k] = v;
        ss = fmaf(v, v, ss);
    }
    if (nw) {
        ss = wave_sum(ss);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
        __syncthreads();
        float tot = 0.f;
        for (int i = 0; i < int(blockDim.x >> 6); ++i) tot += red[i];
        float rr = 1.0f / sqrtf(tot / float(K) + eps);
        for (int k = threadIdx.x; k < K; k += blockDim.x) xs[k] = bf2f(nw[k]) * (xs[k] * rr);
    }
    __syncthreads();
}

// Dot products of R consecutive weight rows with xs (LDS), by one wave: lane l covers k = 512 c + 8 l .. + 7.
template <int R>
__device__ __forceinline__ void wave_rows_dot(const uint16_t* const* rows, const float* xs, int K, float* out) {
    const int lane = threadIdx.x & 63;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;
    for (int k0 = 8 * lane; k0 < K; k0 += 512) {
        uint4 wv[R];
#pragma unroll
        for (int r = 0; r < R; ++r) wv[r] = *reinterpret_cast<const uint4*>(rows[r] + k0);
        float xv[8];
        const float4 x0 = *reinterpret_cast<const float4*>(xs + k0);
        const float4 x1 = *reinterpret_cast<const float4*>(xs + k0 + 4);
        xv[0] = x0.x; xv[1] = x0.y; xv[2] = x0.z; xv[3] = x0.w;
        xv[4] = x1.x; xv[5] = x1.y; xv[6] = x1.z; xv[7] = x1.w;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float wf[8];
            unpack8(wv[r], wf);
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[r] = fmaf(wf[e], xv[e], acc[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) out[r] = wave_sum(acc[r]);
}

constexpr int kMaxHidden = 8192;

// ---------------------------------------------------------------- 20 gemv_qkv_rope_dec
// RMSNorm(x) -> [q | k | v] rows (16 per block, 4 per wave); the last block of each head applies q/k RMSNorm and RoPE
// at state[0] and writes q (f32), the K row and the V column of the cache.
__global__ __launch_bounds__(256) void k_gemv_qkv_dec(const float* x, const uint16_t* nw, const uint16_t* w,
                                                      const uint16_t* qn, const uint16_t* kn, const float* cos_t,
                                                      const float* sin_t, float* q_out, uint16_t* kc, uint16_t* vc,
                                                      float* scratch, uint32_t* counters, const uint32_t* state,
                                                      int hidden, int qh, int kvh, int max_pos, float eps) {
    __shared__ __attribute__((aligned(16))) float xs[kMaxHidden];
    __shared__ float red[4];
    __shared__ int flag;
    load_x_norm(x, nw, eps, hidden, xs, red);
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row0 = blockIdx.x * 16 + wv * 4;
    const uint16_t* rows[4] = {w + size_t(row0) * hidden, w + size_t(row0 + 1) * hidden, w + size_t(row0 + 2) * hidden,
                               w + size_t(row0 + 3) * hidden};
    float out[4];
    wave_rows_dot<4>(rows, xs, hidden, out);
    if (lane < 4) scratch[row0 + lane] = lane == 0 ? out[0] : lane == 1 ? out[1] : lane == 2 ? out[2] : out[3];
    const int head = (blockIdx.x * 16) / 128;
    if (!arrive_last(counters + head, 8u, &flag)) return;
    if (threadIdx.x >= 64) return;
    const int pos = int(state[0]);
    float lo = load_coherent(scratch + head * 128 + lane), hi = load_coherent(scratch + head * 128 + lane + 64);
    const bool is_q = head < qh, is_k = !is_q && head < qh + kvh;
    if (is_q || is_k) {
        const uint16_t* hw = is_q ? qn : kn;
        float ss = wave_sum(fmaf(lo, lo, hi * hi));
        float rr = 1.0f / sqrtf(ss / 128.0f + eps);
        float a = bf2f(hw[lane]) * (lo * rr), b = bf2f(hw[lane + 64]) * (hi * rr);
        float cs = cos_t[size_t(pos) * 64 + lane], sn = sin_t[size_t(pos) * 64 + lane];
        lo = a * cs - b * sn;
        hi = b * cs + a * sn;
    }
    if (is_q) {
        q_out[head * 128 + lane] = lo;
        q_out[head * 128 + lane + 64] = hi;
    } else if (is_k) {
        uint16_t* ko = kc + (size_t(head - qh) * max_pos + pos) * 128;
        ko[lane] = f2bf(lo);
        ko[lane + 64] = f2bf(hi);
    } else {
        uint16_t* vo = vc + size_t(head - qh - kvh) * 128 * max_pos + pos;
        vo[size_t(lane) * max_pos] = f2bf(lo);
        vo[size_t(lane + 64) * max_pos] = f2bf(hi);
    }
}

// ---------------------------------------------------------------- 21 attention_decode_bf16
// Split-KV decode attention: block (s, kv head) takes keys [64 s, 64 s + 64) of positions 0 .. state[0] for the two
// query heads of the group, writes (max, sum, unnormalised output) per head, and the last block of the KV head
// combines the splits.
__global__ __launch_bounds__(256) void k_attn_dec(const float* q, const uint16_t* kc, const uint16_t* vc, float* y,
                                                  float* part, uint32_t* counters, const uint32_t* state, int qh,
                                                  int max_pos, float scale_log2) {
    __shared__ float qs[2][128];
    __shared__ float ps[2][64];
    __shared__ float stat[2][2];
    __shared__ int flag;
    const int s = blockIdx.x, S = gridDim.x, kvhead = blockIdx.y, t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int ctx = int(state[0]) + 1;
    const int key0 = s * 64;
    const int nkeys = max(0, min(64, ctx - key0));
    const int h0 = kvhead * 2;
    qs[t >> 7][t & 127] = q[(h0 + (t >> 7)) * 128 + (t & 127)];
    __syncthreads();
    float* myp = part + (size_t(h0) * S + s) * 130;  // head h0 + hh at + hh * S * 130
    if (nkeys > 0) {
        const uint16_t* kb = kc + (size_t(kvhead) * max_pos + key0) * 128;
        const int d0 = 8 * (lane & 15);
        float q0[8], q1[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            q0[e] = qs[0][d0 + e];
            q1[e] = qs[1][d0 + e];
        }
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            int key = wv * 16 + it * 4 + (lane >> 4);
            float a0 = 0.f, a1 = 0.f;
            if (key < nkeys) {
                float kf[8];
                unpack8(*reinterpret_cast<const uint4*>(kb + size_t(key) * 128 + d0), kf);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    a0 = fmaf(q0[e], kf[e], a0);
                    a1 = fmaf(q1[e], kf[e], a1);
                }
            }
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) {
                a0 += __shfl_xor(a0, o, 64);
                a1 += __shfl_xor(a1, o, 64);
            }
            if ((lane & 15) == 0) {
                ps[0][key] = key < nkeys ? a0 * scale_log2 : -INFINITY;
                ps[1][key] = key < nkeys ? a1 * scale_log2 : -INFINITY;
            }
        }
        __syncthreads();
        if (wv < 2) {
            float v = ps[wv][lane];
            float m = wave_max(v);
            float e = exp2f(v - m);
            float l = wave_sum(e);
            ps[wv][lane] = e;
            if (lane == 0) {
                stat[wv][0] = m;
                stat[wv][1] = l;
            }
        }
        __syncthreads();
        // PV: thread t covers V^T rows d = (t >> 3) + 32 dd and keys 8 (t & 7) .. + 7 of the split
        const int sub = t & 7, rg = t >> 3;
        float e0[8], e1[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            e0[e] = ps[0][sub * 8 + e];
            e1[e] = ps[1][sub * 8 + e];
        }
        const uint16_t* vb = vc + size_t(kvhead) * 128 * max_pos + key0 + sub * 8;
#pragma unroll
        for (int dd = 0; dd < 4; ++dd) {
            const int d = rg + 32 * dd;
            float vf[8];
            unpack8(*reinterpret_cast<const uint4*>(vb + size_t(d) * max_pos), vf);
            float a0 = 0.f, a1 = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                a0 = fmaf(e0[e], vf[e], a0);
                a1 = fmaf(e1[e], vf[e], a1);
            }
#pragma unroll
            for (int o = 1; o < 8; o <<= 1) {
                a0 += __shfl_xor(a0, o, 64);
                a1 += __shfl_xor(a1, o, 64);
            }
            if (sub == 0) {
                myp[2 + d] = a0;
                myp[size_t(S) * 130 + 2 + d] = a1;
            }
        }
        if (t == 0) {
            myp[0] = stat[0][0];
            myp[1] = stat[0][1];
            myp[size_t(S) * 130] = stat[1][0];
            myp[size_t(S) * 130 + 1] = stat[1][1];
        }
    }
    if (!arrive_last(counters + kvhead, uint32_t(S), &flag)) return;
    // combine the splits that hold keys
    const int hh = t >> 7, d = t & 127;
    const int used = (ctx + 63) / 64 < S ? (ctx + 63) / 64 : S;
    const float* hp = part + size_t(h0 + hh) * S * 130;
    float M = -INFINITY;
    for (int i = 0; i < used; ++i) M = fmaxf(M, load_coherent(hp + size_t(i) * 130));
    float L = 0.f, O = 0.f;
    for (int i = 0; i < used; ++i) {
        float sc = exp2f(load_coherent(hp + size_t(i) * 130) - M);
        L = fmaf(load_coherent(hp + size_t(i) * 130 + 1), sc, L);
        O = fmaf(load_coherent(hp + size_t(i) * 130 + 2 + d), sc, O);
    }
    y[(h0 + hh) * 128 + d] = O / L;
}

// ---------------------------------------------------------------- 22 gemv_residual_dec: x[n] += a . w[n]
template <int R>
__global__ __launch_bounds__(256) void k_gemv_resid_dec(const float* a, const uint16_t* w, float* x, int n, int k) {
    __shared__ __attribute__((aligned(16))) float xs[kMaxHidden];
    load_x_norm(a, nullptr, 0.f, k, xs, nullptr);
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * 4 + wv) * R;
    if (row0 >= n) return;
    const uint16_t* rows[R];
#pragma unroll
    for (int r = 0; r < R; ++r) rows[r] = w + size_t(min(row0 + r, n - 1)) * k;
    float out[R];
    wave_rows_dot<R>(rows, xs, k, out);
#pragma unroll
    for (int r = 0; r < R; ++r)
        if (lane == r && row0 + r < n) x[row0 + r] += out[r];
}

// ---------------------------------------------------------------- 23 gemv_swiglu_dec: a[j] = silu(g . h) * (u . h)
template <int R>
__global__ __launch_bounds__(256) void k_gemv_swiglu_dec(const float* x, const uint16_t* nw, const uint16_t* w,
                                                         float* y, int inter, int hidden, float eps) {
    __shared__ __attribute__((aligned(16))) float xs[kMaxHidden];
    __shared__ float red[4];
    load_x_norm(x, nw, eps, hidden, xs, red);
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int j0 = (blockIdx.x * 4 + wv) * R;
    if (j0 >= inter) return;
    const uint16_t* rows[2 * R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        int j = min(j0 + r, inter - 1);
        rows[r] = w + size_t(j) * hidden;
        rows[R + r] = w + size_t(inter + j) * hidden;
    }
    float out[2 * R];
    wave_rows_dot<2 * R>(rows, xs, hidden, out);
#pragma unroll
    for (int r = 0; r < R; ++r)
        if (lane == r && j0 + r < inter) {
            float gv = out[r];
            y[j0 + r] = gv / (1.0f + __expf(-gv)) * out[R + r];
        }
}

// ---------------------------------------------------------------- 24 lmhead_argmax_dec
// logits[n] = RMSNorm(x) . E[n] (the tied embedding); each block keeps its (max, lowest index) and the last block picks
// the row's argmax (0xFFFFFFFF when a logit is NaN), records it in out_ids[state[2]] and advances the state.
__global__ __launch_bounds__(256) void k_lmhead_dec(const float* x, const uint16_t* nw, const uint16_t* e, float* logits,
                                                    float* part, uint32_t* counters, uint32_t* state, uint32_t* out_ids,
                                                    int vocab, int hidden, float eps, int write_logits, int max_steps) {
    __shared__ __attribute__((aligned(16))) float xs[kMaxHidden];
    __shared__ float red[4];
    __shared__ float bv[4];
    __shared__ uint32_t bi[4];
    __shared__ int flag;
    load_x_norm(x, nw, eps, hidden, xs, red);
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    float best = -INFINITY;
    uint32_t besti = 0xFFFFFFFFu;
    bool nan = false;
    const int per_block = (vocab + gridDim.x - 1) / gridDim.x;
    const int r0 = blockIdx.x * per_block, r1 = min(vocab, r0 + per_block);
    for (int row = r0 + wv * 4; row < r1; row += 16) {
        const uint16_t* rows[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) rows[r] = e + size_t(min(row + r, vocab - 1)) * hidden;
        float out[4];
        wave_rows_dot<4>(rows, xs, hidden, out);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            if (row + r >= r1) continue;
            float v = out[r];
            if (write_logits && lane == r) logits[row + r] = v;
            if (v != v) nan = true;
            else if (besti == 0xFFFFFFFFu || v > best) {  // rows visited in increasing order per wave
                best = v;
                besti = uint32_t(row + r);
            }
        }
    }
    // block reduce (value desc, index asc); a NaN anywhere marks the block
    if (lane == 0) {
        bv[wv] = nan ? NAN : best;
        bi[wv] = nan ? 0xFFFFFFFEu : besti;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float b = 0.f;
        uint32_t ix = 0xFFFFFFFFu;
        bool bn = false;
        for (int i = 0; i < 4; ++i) {
            if (bi[i] == 0xFFFFFFFEu) bn = true;
            else if (bi[i] != 0xFFFFFFFFu && (ix == 0xFFFFFFFFu || bv[i] > b || (bv[i] == b && bi[i] < ix))) {
                b = bv[i];
                ix = bi[i];
            }
        }
        part[2 * blockIdx.x] = b;
        reinterpret_cast<uint32_t*>(part)[2 * blockIdx.x + 1] = bn ? 0xFFFFFFFEu : ix;
    }
    if (!arrive_last(counters, gridDim.x, &flag)) return;
    if (threadIdx.x != 0) return;
    float b = 0.f;
    uint32_t ix = 0xFFFFFFFFu;
    bool bn = false;
    for (uint32_t i = 0; i < gridDim.x; ++i) {
        float v = load_coherent(part + 2 * i);
        uint32_t j = load_coherent_u32(reinterpret_cast<const uint32_t*>(part) + 2 * i + 1);
        if (j == 0xFFFFFFFEu) bn = true;
        else if (j != 0xFFFFFFFFu && (ix == 0xFFFFFFFFu || v > b || (v == b && j < ix))) {
            b = v;
            ix = j;
        }
    }
    uint32_t id = bn ? 0xFFFFFFFFu : ix;
    uint32_t step = state[2];
    if (int(step) < max_steps) out_ids[step] = id;
    state[1] = id;
    state[0] = state[0] + 1u;
    state[2] = step + 1u;
}

// ---------------------------------------------------------------- 25 embed_dec: x = widen(E[state[1]])
__global__ __launch_bounds__(256) void k_embed_dec(const uint16_t* e, const uint32_t* state, float* x, int hidden,
                                                   int vocab) {
    const uint32_t id = state[1];
    for (int c = threadIdx.x; c < hidden; c += 256)
        x[c] = id < uint32_t(vocab) ? bf2f(e[size_t(id) * hidden + c]) : __uint_as_float(0x7FC00000u);
}

// ---------------------------------------------------------------- 26 fill_normal_bf16 (synthetic caches/inputs)
// y[i] = bf16(std * N(0, 1)) from a counter-based generator: splitmix64 of (seed, stream, i / 2), Box-Muller.
__device__ __forceinline__ uint64_t splitmix(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
__global__ void k_fill_normal(uint16_t* y, uint64_t n, uint64_t seed, uint64_t stream, float std) {
    uint64_t i = (uint64_t(blockIdx.x) * blockDim.x + threadIdx.x) * 2;
    if (i >= n) return;
    uint64_t h = splitmix(seed ^ splitmix(stream ^ splitmix(i >> 1)));
    double u1 = (double((h >> 11) & ((1ull << 26) - 1)) + 0.5) / double(1ull << 26);
    double u2 = double(h >> 38) / double(1ull << 26);
    double r = sqrt(-2.0 * log(u1));
    y[i] = f2bf(float(std * r * cos(6.283185307179586 * u2)));
    if (i + 1 < n) y[i + 1] = f2bf(float(std * r * sin(6.283185307179586 * u2)));
}

// ================================================================ launchers and catalog entries

static float f32_of(uint32_t b) {
    float f;
    std::memcpy(&f, &b, 4);
    return f;
}

static void l_rmsnorm_bf16(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    hipLaunchKernelGGL(k_rmsnorm_bf16, dim3(pd.words[4]), dim3(256), 0, s, (const float*)p[0], (const uint16_t*)p[1],
                       (uint16_t*)p[2], pd.words[4], pd.words[5], f32_of(pd.words[6]), pd.words[7]);
}

static GemmArgs gemm_base(void* const* p, uint32_t m, uint32_t n, uint32_t k) {
    GemmArgs a{};
    a.a = (const uint16_t*)p[0];
    a.w = (const uint16_t*)p[1];
    a.M = int(m);
    a.N = int(n);
    a.K = int(k);
    return a;
}

// 15 gemm_qkv_rope: h, w, qn, kn, cos, sin, q, kc, vc, m, hidden, q_heads, kv_heads, pos0, max_pos, eps
static void l_gemm_qkv(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    const uint32_t* w = pd.words.data();
    int qh = int(w[12]), kvh = int(w[13]);
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
    dim3 grid(uint32_t(qh + 2 * kvh), (w[10] + GBM - 1) / GBM);
    hipLaunchKernelGGL(k_gemm<EPI_QKV>, grid, dim3(256), 0, s, a);
}

// 16 attention_prefill_bf16: q, kc, vc, y, rows, past, q_heads, kv_heads, max_pos, scale
static void l_attn_prefill(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    const uint32_t* w = pd.words.data();
    int T = int(w[5]);
    dim3 grid(uint32_t((T + 63) / 64), w[8]);
    hipLaunchKernelGGL(k_attn_prefill, grid, dim3(256), 0, s, (const uint16_t*)p[0], (const uint16_t*)p[1],
                       (const uint16_t*)p[2], (uint16_t*)p[3], T, int(w[6]), int(w[7]), int(w[8]), int(w[9]),
                       f32_of(w[10]) * kLog2e);
}

// 17 gemm_residual: a, w, x, m, n, k
static void l_gemm_resid(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    const uint32_t* w = pd.words.data();
    GemmArgs a = gemm_base(p, w[4], w[5], w[6]);
    a.y32 = (float*)p[2];
    a.resid = (const float*)p[2];
    dim3 grid((w[5] + GBN - 1) / GBN, (w[4] + GBM - 1) / GBM);
    hipLaunchKernelGGL(k_gemm<EPI_RESID>, grid, dim3(256), 0, s, a);
}

// 18 gemm_swiglu: a, w (2I rows), y, m, inter, k
static void l_gemm_swiglu(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    const uint32_t* w = pd.words.data();
    GemmArgs a = gemm_base(p, w[4], 2 * w[5], w[6]);
    a.y16 = (uint16_t*)p[2];
    a.inter = int(w[5]);
    dim3 grid((w[5] + 63) / 64, (w[4] + GBM - 1) / GBM);
    hipLaunchKernelGGL(k_gemm<EPI_SWIGLU>, grid, dim3(256), 0, s, a);
}

// 19 gemm_f32: a, w, y, m, n, k
static void l_gemm_f32(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    const uint32_t* w = pd.words.data();
    GemmArgs a = gemm_base(p, w[4], w[5], w[6]);
    a.y32 = (float*)p[2];
    dim3 grid((w[5] + GBN - 1) / GBN, (w[4] + GBM - 1) / GBM);
    hipLaunchKernelGGL(k_gemm<EPI_F32>, grid, dim3(256), 0, s, a);
}

// 20 gemv_qkv_rope_dec: x, nw, w, qn, kn, cos, sin, q, kc, vc, scratch, counters, state, hidden, q_heads, kv_heads,
// max_pos, eps
static void l_gemv_qkv(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    const uint32_t* w = pd.words.data();
    int qh = int(w[15]), kvh = int(w[16]);
    hipLaunchKernelGGL(k_gemv_qkv_dec, dim3(uint32_t((qh + 2 * kvh) * 8)), dim3(256), 0, s, (const float*)p[0],
                       (const uint16_t*)p[1], (const uint16_t*)p[2], (const uint16_t*)p[3], (const uint16_t*)p[4],
                       (const float*)p[5], (const float*)p[6], (float*)p[7], (uint16_t*)p[8], (uint16_t*)p[9],
                       (float*)p[10], (uint32_t*)p[11], (const uint32_t*)p[12], int(w[14]), qh, kvh, int(w[17]),
                       f32_of(w[18]));
}

// 21 attention_decode_bf16: q, kc, vc, y, part, counters, state, q_heads, kv_heads, max_pos, scale
static void l_attn_dec(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    const uint32_t* w = pd.words.data();
    int max_pos = int(w[10]);
    hipLaunchKernelGGL(k_attn_dec, dim3(uint32_t(max_pos / 64), w[9]), dim3(256), 0, s, (const float*)p[0],
                       (const uint16_t*)p[1], (const uint16_t*)p[2], (float*)p[3], (float*)p[4], (uint32_t*)p[5],
                       (const uint32_t*)p[6], int(w[8]), max_pos, f32_of(w[11]) * kLog2e);
}

// 22 gemv_residual_dec: a, w, x, n, k
static void l_gemv_resid(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    const uint32_t* w = pd.words.data();
    int n = int(w[4]), k = int(w[5]);
    if (n >= 4096) {
        hipLaunchKernelGGL(k_gemv_resid_dec<4>, dim3(uint32_t((n + 15) / 16)), dim3(256), 0, s, (const float*)p[0],
                           (const uint16_t*)p[1], (float*)p[2], n, k);
    } else {
        hipLaunchKernelGGL(k_gemv_resid_dec<1>, dim3(uint32_t((n + 3) / 4)), dim3(256), 0, s, (const float*)p[0],
                           (const uint16_t*)p[1], (float*)p[2], n, k);
    }
}

// 23 gemv_swiglu_dec: x, nw, w, y, inter, hidden, eps
static void l_gemv_swiglu(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    const uint32_t* w = pd.words.data();
    int inter = int(w[5]);
    hipLaunchKernelGGL(k_gemv_swiglu_dec<2>, dim3(uint32_t((inter + 7) / 8)), dim3(256), 0, s, (const float*)p[0],
                       (const uint16_t*)p[1], (const uint16_t*)p[2], (float*)p[3], inter, int(w[6]), f32_of(w[7]));
}

constexpr uint32_t kLmheadBlocks = 1024;

// 24 lmhead_argmax_dec: x, nw, e, logits, part, counters, state, out_ids, vocab, hidden, eps, write_logits, max_steps
static void l_lmhead(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    const uint32_t* w = pd.words.data();
    hipLaunchKernelGGL(k_lmhead_dec, dim3(kLmheadBlocks), dim3(256), 0, s, (const float*)p[0], (const uint16_t*)p[1],
                       (const uint16_t*)p[2], (float*)p[3], (float*)p[4], (uint32_t*)p[5], (uint32_t*)p[6],
                       (uint32_t*)p[7], int(w[9]), int(w[10]), f32_of(w[11]), int(w[12]), int(w[13]));
}

// 25 embed_dec: e, state, x, hidden, vocab
static void l_embed_dec(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    const uint32_t* w = pd.words.data();
    hipLaunchKernelGGL(k_embed_dec, dim3(1), dim3(256), 0, s, (const uint16_t*)p[0], (const uint32_t*)p[1],
                       (float*)p[2], int(w[4]), int(w[5]));
}

// 26 fill_normal_bf16: y, n, seed_lo, seed_hi, stream_lo, stream_hi, std
static void l_fill_normal(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    const uint32_t* w = pd.words.data();
    uint64_t n = w[2];
    uint64_t seed = uint64_t(w[3]) | uint64_t(w[4]) << 32, stream = uint64_t(w[5]) | uint64_t(w[6]) << 32;
    uint32_t blocks = uint32_t((n / 2 + 255) / 256 + 1);
    hipLaunchKernelGGL(k_fill_normal, dim3(blocks), dim3(256), 0, s, (uint16_t*)p[0], n, seed, stream, f32_of(w[7]));
}

int fast_first_id() { return 14; }

const LaunchFn* fast_launchers() {
    static const LaunchFn t[] = {l_rmsnorm_bf16, l_gemm_qkv,   l_attn_prefill, l_gemm_resid, l_gemm_swiglu,
                                 l_gemm_f32,     l_gemv_qkv,   l_attn_dec,     l_gemv_resid, l_gemv_swiglu,
                                 l_lmhead,       l_embed_dec,  l_fill_normal};
    return t;
}

// ---------------------------------------------------------------- catalog entries (ids 14..26)

#define DT(x) (1u << (x))
#define TOK_R(n, m) FieldSpec{n, FieldKind::Token, Access::Read, m, nullptr}
#define TOK_W(n, m) FieldSpec{n, FieldKind::Token, Access::Write, m, nullptr}
#define TOK_RW(n, m) FieldSpec{n, FieldKind::Token, Access::ReadWrite, m, nullptr}
#define U32F(n) FieldSpec{n, FieldKind::U32, Access::None, 0, nullptr}
#define F32F(n) FieldSpec{n, FieldKind::F32, Access::None, 0, nullptr}

static void need(const uint32_t* counts, int field, int64_t elems, const char* kernel, const char* what) {
    if (elems < 0 || int64_t(counts[field]) < elems)
        contract_fail("%s.%s holds %u elements; the dispatch touches %lld", kernel, what, counts[field], (long long)elems);
}

static void need_hd128_group2(const char* k, uint32_t qh, uint32_t kvh) {
    if (kvh < 1 || qh != 2 * kvh) contract_fail("%s: this kernel takes two query heads per KV head", k);
}

std::vector<KernelSpec> fast_catalog() {
    std::vector<KernelSpec> c;
    // 14 rmsnorm_rows_bf16: x, w, y, rows, cols, eps, x_row0
    c.push_back({"rmsnorm_rows_bf16", "fast", {256, 1, 1}, true, [](const uint32_t* w) { return Grid3{w[4], 1, 1}; },
                 {TOK_R("x", DT(F32)), TOK_R("w", DT(BF16)), TOK_W("y", DT(BF16)), U32F("rows"), U32F("cols"),
                  F32F("eps"), U32F("x_row0")},
                 [](const uint32_t* w, const uint32_t* c) {
                     if (w[5] < 1) contract_fail("rmsnorm_rows_bf16: cols must be at least 1");
                     need(c, 0, (int64_t(w[7]) + w[4]) * w[5], "rmsnorm_rows_bf16", "x");
                     need(c, 1, w[5], "rmsnorm_rows_bf16", "w");
                     need(c, 2, int64_t(w[4]) * w[5], "rmsnorm_rows_bf16", "y");
                 }});
    // 15 gemm_qkv_rope
    c.push_back({"gemm_qkv_rope", "fast", {256, 1, 1}, false,
                 [](const uint32_t* w) { return Grid3{int64_t(w[12]) + 2 * w[13], (int64_t(w[10]) + 127) / 128, 1}; },
                 {TOK_R("h", DT(BF16)), TOK_R("w", DT(BF16)), TOK_R("q_norm", DT(BF16)), TOK_R("k_norm", DT(BF16)),
                  TOK_R("cos_table", DT(F32)), TOK_R("sin_table", DT(F32)), TOK_W("q", DT(BF16)),
                  TOK_W("k_cache", DT(BF16)), TOK_W("v_cache", DT(BF16)), U32F("m"), U32F("hidden"), U32F("q_heads"),
                  U32F("kv_heads"), U32F("pos0"), U32F("max_pos"), F32F("eps")},
                 [](const uint32_t* w, const uint32_t* c) {
                     int64_t m = w[10], hid = w[11], qh = w[12], kvh = w[13], pos0 = w[14], mp = w[15];
                     need_hd128_group2("gemm_qkv_rope", w[12], w[13]);
                     if (hid % 64) contract_fail("gemm_qkv_rope: hidden must be a multiple of 64");
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
    // 16 attention_prefill_bf16: q, kc, vc, y, rows, past, q_heads, kv_heads, max_pos, scale
    c.push_back({"attention_prefill_bf16", "fast", {256, 1, 1}, false,
                 [](const uint32_t* w) { return Grid3{(int64_t(w[5]) + 63) / 64, w[8], 1}; },
                 {TOK_R("q", DT(BF16)), TOK_R("k_cache", DT(BF16)), TOK_R("v_cache", DT(BF16)), TOK_W("y", DT(BF16)),
                  U32F("rows"), U32F("past"), U32F("q_heads"), U32F("kv_heads"), U32F("max_pos"), F32F("scale")},
                 [](const uint32_t* w, const uint32_t* c) {
                     int64_t rows = w[5], past = w[6], qh = w[7], kvh = w[8], mp = w[9];
                     need_hd128_group2("attention_prefill_bf16", w[7], w[8]);
                     if (mp % 64) contract_fail("attention_prefill_bf16: max_pos must be a multiple of 64");
                     if (past + rows > mp) contract_fail("attention_prefill_bf16: positions past max_pos");
                     need(c, 0, rows * qh * 128, "attention_prefill_bf16", "q");
                     need(c, 1, kvh * mp * 128, "attention_prefill_bf16", "k_cache");
                     need(c, 2, kvh * mp * 128, "attention_prefill_bf16", "v_cache");
                     need(c, 3, rows * qh * 128, "attention_prefill_bf16", "y");
                 }});
    // 17 gemm_residual: a, w, x, m, n, k
    c.push_back({"gemm_residual", "fast", {256, 1, 1}, false,
                 [](const uint32_t* w) { return Grid3{(int64_t(w[5]) + 127) / 128, (int64_t(w[4]) + 127) / 128, 1}; },
                 {TOK_R("a", DT(BF16)), TOK_R("w", DT(BF16)), TOK_RW("x", DT(F32)), U32F("m"), U32F("n"), U32F("k")},
                 [](const uint32_t* w, const uint32_t* c) {
                     if (w[6] % 64) contract_fail("gemm_residual: k must be a multiple of 64");
                     need(c, 0, int64_t(w[4]) * w[6], "gemm_residual", "a");
                     need(c, 1, int64_t(w[5]) * w[6], "gemm_residual", "w");
                     need(c, 2, int64_t(w[4]) * w[5], "gemm_residual", "x");
                 }});
    // 18 gemm_swiglu: a, w, y, m, inter, k
    c.push_back({"gemm_swiglu", "fast", {256, 1, 1}, false,
                 [](const uint32_t* w) { return Grid3{(int64_t(w[5]) + 63) / 64, (int64_t(w[4]) + 127) / 128, 1}; },
                 {TOK_R("a", DT(BF16)), TOK_R("w", DT(BF16)), TOK_W("y", DT(BF16)), U32F("m"), U32F("inter"), U32F("k")},
                 [](const uint32_t* w, const uint32_t* c) {
                     if (w[6] % 64) contract_fail("gemm_swiglu: k must be a multiple of 64");
                     need(c, 0, int64_t(w[4]) * w[6], "gemm_swiglu", "a");
                     need(c, 1, 2 * int64_t(w[5]) * w[6], "gemm_swiglu", "w");
                     need(c, 2, int64_t(w[4]) * w[5], "gemm_swiglu", "y");
                 }});
    // 19 gemm_f32: a, w, y, m, n, k
    c.push_back({"gemm_f32", "fast", {256, 1, 1}, false,
                 [](const uint32_t* w) { return Grid3{(int64_t(w[5]) + 127) / 128, (int64_t(w[4]) + 127) / 128, 1}; },
                 {TOK_R("a", DT(BF16)), TOK_R("w", DT(BF16)), TOK_W("y", DT(F32)), U32F("m"), U32F("n"), U32F("k")},
                 [](const uint32_t* w, const uint32_t* c) {
                     if (w[6] % 64) contract_fail("gemm_f32: k must be a multiple of 64");
                     need(c, 0, int64_t(w[4]) * w[6], "gemm_f32", "a");
                     need(c, 1, int64_t(w[5]) * w[6], "gemm_f32", "w");
                     need(c, 2, int64_t(w[4]) * w[5], "gemm_f32", "y");
                 }});
    // 20 gemv_qkv_rope_dec
    c.push_back({"gemv_qkv_rope_dec", "fast", {256, 1, 1}, true,
                 [](const uint32_t* w) { return Grid3{(int64_t(w[15]) + 2 * w[16]) * 8, 1, 1}; },
                 {TOK_R("x", DT(F32)), TOK_R("norm", DT(BF16)), TOK_R("w", DT(BF16)), TOK_R("q_norm", DT(BF16)),
                  TOK_R("k_norm", DT(BF16)), TOK_R("cos_table", DT(F32)), TOK_R("sin_table", DT(F32)),
                  TOK_W("q", DT(F32)), TOK_W("k_cache", DT(BF16)), TOK_W("v_cache", DT(BF16)),
                  TOK_RW("scratch", DT(F32)), TOK_RW("counters", DT(U32)), TOK_R("state", DT(U32)), U32F("hidden"),
                  U32F("q_heads"), U32F("kv_heads"), U32F("max_pos"), F32F("eps")},
                 [](const uint32_t* w, const uint32_t* c) {
                     int64_t hid = w[14], qh = w[15], kvh = w[16], mp = w[17];
                     need_hd128_group2("gemv_qkv_rope_dec", w[15], w[16]);
                     if (hid % 512 || hid > kMaxHidden) contract_fail("gemv_qkv_rope_dec: hidden must be a multiple of 512 up to 8192");
                     need(c, 0, hid, "gemv_qkv_rope_dec", "x");
                     need(c, 1, hid, "gemv_qkv_rope_dec", "norm");
                     need(c, 2, (qh + 2 * kvh) * 128 * hid, "gemv_qkv_rope_dec", "w");
                     need(c, 3, 128, "gemv_qkv_rope_dec", "q_norm");
                     need(c, 4, 128, "gemv_qkv_rope_dec", "k_norm");
                     need(c, 5, mp * 64, "gemv_qkv_rope_dec", "cos_table");
                     need(c, 6, mp * 64, "gemv_qkv_rope_dec", "sin_table");
                     need(c, 7, qh * 128, "gemv_qkv_rope_dec", "q");
                     need(c, 8, kvh * mp * 128, "gemv_qkv_rope_dec", "k_cache");
                     need(c, 9, kvh * mp * 128, "gemv_qkv_rope_dec", "v_cache");
                     need(c, 10, (qh + 2 * kvh) * 128, "gemv_qkv_rope_dec", "scratch");
                     need(c, 11, qh + 2 * kvh, "gemv_qkv_rope_dec", "counters");
                     need(c, 12, 4, "gemv_qkv_rope_dec", "state");
                 }});
    // 21 attention_decode_bf16: q, kc, vc, y, part, counters, state, q_heads, kv_heads, max_pos, scale
    c.push_back({"attention_decode_bf16", "fast", {256, 1, 1}, false,
                 [](const uint32_t* w) { return Grid3{int64_t(w[10]) / 64, w[9], 1}; },
                 {TOK_R("q", DT(F32)), TOK_R("k_cache", DT(BF16)), TOK_R("v_cache", DT(BF16)), TOK_W("y", DT(F32)),
                  TOK_RW("partials", DT(F32)), TOK_RW("counters", DT(U32)), TOK_R("state", DT(U32)),
                  U32F("q_heads"), U32F("kv_heads"), U32F("max_pos"), F32F("scale")},
                 [](const uint32_t* w, const uint32_t* c) {
                     int64_t qh = w[8], kvh = w[9], mp = w[10];
                     need_hd128_group2("attention_decode_bf16", w[8], w[9]);
                     if (mp % 64 || mp < 64) contract_fail("attention_decode_bf16: max_pos must be a positive multiple of 64");
                     need(c, 0, qh * 128, "attention_decode_bf16", "q");
                     need(c, 1, kvh * mp * 128, "attention_decode_bf16", "k_cache");
                     need(c, 2, kvh * mp * 128, "attention_decode_bf16", "v_cache");
                     need(c, 3, qh * 128, "attention_decode_bf16", "y");
                     need(c, 4, qh * (mp / 64) * 130, "attention_decode_bf16", "partials");
                     need(c, 5, kvh, "attention_decode_bf16", "counters");
                     need(c, 6, 4, "attention_decode_bf16", "state");
                 }});
    // 22 gemv_residual_dec: a, w, x, n, k
    c.push_back({"gemv_residual_dec", "fast", {256, 1, 1}, true,
                 [](const uint32_t* w) { return Grid3{w[4] >= 4096 ? (int64_t(w[4]) + 15) / 16 : (int64_t(w[4]) + 3) / 4, 1, 1}; },
                 {TOK_R("a", DT(F32)), TOK_R("w", DT(BF16)), TOK_RW("x", DT(F32)), U32F("n"), U32F("k")},
                 [](const uint32_t* w, const uint32_t* c) {
                     if (w[5] % 512 || w[5] > uint32_t(kMaxHidden)) contract_fail("gemv_residual_dec: k must be a multiple of 512 up to 8192");
                     need(c, 0, w[5], "gemv_residual_dec", "a");
                     need(c, 1, int64_t(w[4]) * w[5], "gemv_residual_dec", "w");
                     need(c, 2, w[4], "gemv_residual_dec", "x");
                 }});
    // 23 gemv_swiglu_dec: x, nw, w, y, inter, hidden, eps
    c.push_back({"gemv_swiglu_dec", "fast", {256, 1, 1}, true,
                 [](const uint32_t* w) { return Grid3{(int64_t(w[5]) + 7) / 8, 1, 1}; },
                 {TOK_R("x", DT(F32)), TOK_R("norm", DT(BF16)), TOK_R("w", DT(BF16)), TOK_W("y", DT(F32)),
                  U32F("inter"), U32F("hidden"), F32F("eps")},
                 [](const uint32_t* w, const uint32_t* c) {
                     if (w[6] % 512 || w[6] > uint32_t(kMaxHidden)) contract_fail("gemv_swiglu_dec: hidden must be a multiple of 512 up to 8192");
                     need(c, 0, w[6], "gemv_swiglu_dec", "x");
                     need(c, 1, w[6], "gemv_swiglu_dec", "norm");
                     need(c, 2, 2 * int64_t(w[5]) * w[6], "gemv_swiglu_dec", "w");
                     need(c, 3, w[5], "gemv_swiglu_dec", "y");
                 }});
    // 24 lmhead_argmax_dec: x, nw, e, logits, part, counters, state, out_ids, vocab, hidden, eps, write_logits, max_steps
    c.push_back({"lmhead_argmax_dec", "fast", {256, 1, 1}, true,
                 [](const uint32_t*) { return Grid3{kLmheadBlocks, 1, 1}; },
                 {TOK_R("x", DT(F32)), TOK_R("norm", DT(BF16)), TOK_R("embed", DT(BF16)), TOK_W("logits", DT(F32)),
                  TOK_RW("partials", DT(F32)), TOK_RW("counters", DT(U32)), TOK_RW("state", DT(U32)),
                  TOK_RW("out_ids", DT(U32)), U32F("vocab"), U32F("hidden"), F32F("eps"), U32F("write_logits"),
                  U32F("max_steps")},
                 [](const uint32_t* w, const uint32_t* c) {
                     if (w[10] % 512 || w[10] > uint32_t(kMaxHidden)) contract_fail("lmhead_argmax_dec: hidden must be a multiple of 512 up to 8192");
                     need(c, 0, w[10], "lmhead_argmax_dec", "x");
                     need(c, 1, w[10], "lmhead_argmax_dec", "norm");
                     need(c, 2, int64_t(w[9]) * w[10], "lmhead_argmax_dec", "embed");
                     need(c, 3, w[12] ? int64_t(w[9]) : 0, "lmhead_argmax_dec", "logits");
                     need(c, 4, 2 * int64_t(kLmheadBlocks), "lmhead_argmax_dec", "partials");
                     need(c, 5, 1, "lmhead_argmax_dec", "counters");
                     need(c, 6, 4, "lmhead_argmax_dec", "state");
                     need(c, 7, w[13], "lmhead_argmax_dec", "out_ids");
                 }});
    // 25 embed_dec: e, state, x, hidden, vocab
    c.push_back({"embed_dec", "fast", {256, 1, 1}, true, [](const uint32_t*) { return Grid3{1, 1, 1}; },
                 {TOK_R("embed", DT(BF16)), TOK_R("state", DT(U32)), TOK_W("x", DT(F32)), U32F("hidden"), U32F("vocab")},
                 [](const uint32_t* w, const uint32_t* c) {
                     need(c, 0, int64_t(w[4]) * w[5], "embed_dec", "embed");
                     need(c, 1, 4, "embed_dec", "state");
                     need(c, 2, w[4], "embed_dec", "x");
                 }});
    // 26 fill_normal_bf16: y, n, seed_lo, seed_hi, stream_lo, stream_hi, std
    c.push_back({"fill_normal_bf16", "fast", {256, 1, 1}, true,
                 [](const uint32_t* w) { return Grid3{(int64_t(w[2]) / 2 + 255) / 256 + 1, 1, 1}; },
                 {TOK_W("y", DT(BF16)), U32F("n"), U32F("seed_lo"), U32F("seed_hi"), U32F("stream_lo"),
                  U32F("stream_hi"), F32F("std")},
                 [](const uint32_t* w, const uint32_t* c) { need(c, 0, w[2], "fill_normal_bf16", "y"); }});
    return c;
}

}  // namespace lrm
