// ================================================================ 38 decode_step_persistent
// The one-sequence decode step (embed, every layer, lm_head, greedy argmax, state advance) as ONE launch: 256
// workgroups of 8 waves (one per CU, all resident together) walk the layers stage by stage, each taking a fixed share
// of every stage, and hand the stage outputs to each other through tagged exchange entries in device memory instead of
// kernel boundaries. It computes what the multi-kernel step of the executor computes (embed_dec, then per layer
// gemv_norm_dec, attention_decode_f16, attention_combine, gemv_residual_dec, gemv_swiglu_dec, gemv_residual_dec, then
// lmhead_dec and argmax_dec) with the same per-lane products; the o_proj and down_proj sums run in another order (each
// XCD's columns summed alone, then the eight sums added in XCD order), and the split combine sums the splits in order.
//
// Why: batch-1 decode of a 0.6B model moves ~1.2 GB per token, ~150 us at HBM speed, but as ~170 dependent kernels
// it is bound by launch and ramp latency (4-6 us per kernel). Here each hand-off costs a store and a poll, and every
// workgroup issues the weight loads of its next stage before it waits, so the weight stream overlaps the hand-offs.
//
// XCD mapping. An MI355X has 8 XCDs, each with its own L2; the dispatcher puts workgroup b on XCD (b + c) % 8, with c
// fixed for a launch (it depends on the hardware queue), so each XCD holds 32 workgroups. A workgroup reads its XCD from
// the hardware register XCC_ID and takes role j = b / 8 on it: every (XCD, j) is taken once. That placement is the
// dispatcher's, not a documented guarantee, so each workgroup claims its role at launch (an exchange of the launch's
// tag into the role's header word): a role claimed twice aborts the step, which the host then reports, instead of
// leaving another role untaken and its readers on entries of an earlier step. A device-scope store writes
// through to memory
// and a device-scope load from another XCD fetches it there: 0.7 us one way, about 2.2 us for an all-gather between all
// 256 workgroups. A plain store stays in the writer's L2, where a device-scope load from the same XCD finds it: 0.3 us.
// So KV head h is XCD h's: its q|k|v rows, its 32 attention splits, and the o_proj and down_proj columns that read its
// outputs (o_proj columns 256 h .. + 255, SwiGLU outputs and down_proj columns 384 h .. + 383). Three of a layer's five
// hand-offs stay inside one L2; the o_proj and down_proj outputs leave as per-XCD partial sums [8][hidden] through
// memory, and every workgroup adds them to its own copy of the residual stream as it gathers them.
//
// Exchange entries carry their own ready mark, so a consumer polls the data itself. 8-byte entries (q|k|v, the lm_head
// partials): (tag << 32) | value bits; an entry is ready when it carries this launch's tag, the launch epoch + 1 (header
// word 0, advanced by workgroup 0 at the end of every step), so entries left by earlier steps never match. 4-byte
// entries (the attention partials, the SwiGLU output, the o_proj and down_proj partial sums): the value with its lowest
// mantissa bit replaced by the tag's parity; every entry that is read is written by every step (an attention split
// that holds no keys writes an empty partial), so the previous step's entries always carry the other parity (after an
// aborted step the host zeroes the area).
//
// Stages of layer l (Qwen3-0.6B: hidden 1024, 16/8 heads, intermediate 3072), workgroup b on XCD h, j = b / 8:
//   A  q|k|v of KV head h = W . RMSNorm(x): 2 of the XCD's 512 rows per wave. Waits for x, i.e. for the previous
//      layer's down_proj partial sums of all XCDs (all of x: the RMSNorm needs the whole row).
//   B  attention: split j of KV head h takes keys [j KPS, (j + 1) KPS) (KPS a multiple of 64 chosen so at most 32
//      splits cover pos + 1 keys), both query heads, 64 keys at a time with an online softmax; the split holding pos
//      also normalises, rotates and appends the new key and value. Writes (out[128], max, sum) per query head.
//   C  o_h = the combine of the splits (every workgroup of the XCD forms all 256 dims), then
//      p1[h] = W_o[:, 256 h .. + 255] . o_h: 32 rows per workgroup.
//   D  a_h = silu(W_g . r) * (W_u . r), r = RMSNorm(x + sum_h p1[h]): 12 of the XCD's 384 gate/up pairs.
//   E  p2[h] = W_d[:, 384 h .. + 383] . a_h: 32 rows per workgroup.
// Then x += sum_h p2[h], every workgroup takes 1/256 of the lm_head rows and writes its (max, lowest index); workgroup
// 0 merges them, records the id and advances the state (position, id, step) for the next launch.
//
// Every wait is bounded: a poll that waits longer than 0.2 s, or sees another workgroup's abort, sets the abort word
// (header word 1) and the stage (word 2) and the workgroup returns; so every wave ends even if a workgroup were never
// scheduled. A launch that finds the abort word set returns at once; the host reads the word after the steps and
// raises. Launches on one device must not overlap (the executor keeps them on one stream).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>
#include <type_traits>

#include "device.hpp"
#include "fast_common.hpp"
#include "kv_layout.hpp"
#include "persist.hpp"

namespace lrm {
using namespace fast;
using namespace persist;

namespace {

constexpr long long kWaitTicks = 20000000;  // 0.2 s of the 100 MHz constant clock: the default bound of a wait

// The instantiated shape (persist::unsupported): Qwen3-0.6B on 256 workgroups.
constexpr int kH = 1024, kQH = 16, kKVH = kXcds, kQPK = kQH / kKVH, kQC = kQH * 128, kKC = kKVH * 128, kI = 3072;
constexpr int kG = 256;
constexpr int kJN = kG / kXcds;                          // workgroups per XCD = attention splits per KV head
constexpr int kNCH = kH / 512;                           // 512-wide chunks of the hidden vector per lane
constexpr int kRA = (kQPK + 2) * 128 / (kJN * kWaves);  // q|k|v rows per wave
constexpr int kCW = kQPK * 128, kEW = kI / kXcds;        // o_proj / down_proj columns of one XCD
constexpr int kRowsG = kH / kJN, kRowsW = kRowsG / kWaves;  // o_proj / down_proj rows per workgroup, per wave
constexpr int kNCC = kRowsW * (kCW / 8) / 64;            // 16-byte o_proj chunks per lane
constexpr int kNCE = kRowsW * (kEW / 8) / 64;            // 16-byte down_proj chunks per lane
constexpr int kPB = kEW / kJN;                           // SwiGLU outputs per workgroup
constexpr int kUD = 2 * kPB * kNCH / kWaves;             // (gate/up row, chunk) units per wave
static_assert(kRA == 2 && kNCC == 2 && kNCE == 3 && kPB == 12 && kUD == 6 && kRowsW == 4, "the 0.6B decode shape");
static_assert(kRowsG <= 64 && kQPK * 16 == kJN, "one combine item and one row run per workgroup");

// The projection matrices and the tied lm_head are read as their fp16 copies, which hold the same values as the bf16
// weights (the executor refuses weights beyond the fp16 range; weights under 2^-17 in magnitude round to fp16's
// subnormal 2^-24 grid): a v_fma_mix_f32 takes a half of a packed pair as it is, one instruction per product where the
// bf16 pair needs a shift or a mask before each FMA.
struct PArgs {
    const uint16_t* embed;       // [V, H] bf16: the embedding row
    const uint16_t* embed16;     // [V, H] f16: the tied lm_head
    const uint16_t* final_norm;  // [H] bf16 (every norm weight is bf16)
    const uint16_t* in_norm;     // [L, H]
    const uint16_t* qkv;         // [L, QC + 2 KC, H] f16
    const uint16_t* q_norm;      // [L, 128]
    const uint16_t* k_norm;      // [L, 128]
    const uint16_t* o_proj;      // [L, H, QC] f16
    const uint16_t* post_norm;   // [L, H]
    const uint16_t* gate_up;     // [L, 2 I, H] f16 (gate rows, then up rows)
    const uint16_t* down;        // [L, H, I] f16
    uint16_t* kc;                // [L, KVH, MP, 128] f16
    uint16_t* vc;                // [L, KVH, MP / 64, 128, 64] f16 (kv::v_at)
    const float* cos_t;          // [MP, 64]
    const float* sin_t;          // [MP, 64]
    float* logits;               // [V]
    uint32_t* state;             // position, id, step
    uint32_t* out_ids;           // [max_steps]
    uint64_t* xch;               // exchange: header, then the entries
    int layers, vocab, max_pos, max_steps, write_logits;
    float eps, scale_log2;
};

__device__ __forceinline__ uint32_t word_load(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Device-wide entries (read by workgroups of every XCD): device-scope stores, written through to memory.
__device__ __forceinline__ void gstore(uint64_t* p, float v, uint32_t tag) {
    __hip_atomic_store(p, (uint64_t(tag) << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// 4-byte entries: the value with its lowest mantissa bit replaced by the launch parity (a change of at most one unit
// in the last place, which the readers of these vectors see)
__device__ __forceinline__ void gstore32(uint32_t* p, float v, uint32_t parity) {
    __hip_atomic_store(p, (__float_as_uint(v) & ~1u) | parity, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// XCD-local entries (read by the workgroups of the writer's XCD only): plain stores, which stay in the XCD's L2, where
// the readers' device-scope loads find them.
__device__ __forceinline__ void lstore(uint64_t* p, float v, uint32_t tag) {
    __hip_atomic_store(p, (uint64_t(tag) << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
}
__device__ __forceinline__ void lstore32(uint32_t* p, float v, uint32_t parity) {
    __hip_atomic_store(p, (__float_as_uint(v) & ~1u) | parity, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
}
__device__ __forceinline__ void abort_step(uint32_t* hdr, int stage) {
    __hip_atomic_store(hdr + 2, uint32_t(stage), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(hdr + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void unpack8bf(u32x4 v, float* f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[2 * i] = __uint_as_float(v[i] << 16);
        f[2 * i + 1] = __uint_as_float(v[i] & 0xFFFF0000u);
    }
}

__device__ __forceinline__ u32x4 ld16(const uint16_t* p) { return *reinterpret_cast<const u32x4*>(p); }

// The bound of a wait: true (and the step aborted, `fail` set) when this poll has waited past `limit` ticks, or every
// 16 polls, when another workgroup aborted.
__device__ __forceinline__ bool wait_over(int it, long long& start, long long limit, uint32_t* hdr, int stage,
                                          int& fail) {
    if (it == 0) {
        start = wall_clock64();
        return false;
    }
    if (wall_clock64() - start > limit || ((it & 15) == 0 && word_load(hdr + 1) != 0u)) {
        abort_step(hdr, stage);
        fail = 1;
        return true;
    }
    return false;
}

// Block-wide: waits until the 8-byte entries idx(i), i < n (1 <= n <= E * 512), carry `tag` and writes their values to
// dst[i] in LDS. Thread t polls entries t, t + 512, ..., re-reading only those not yet ready, back to back. When the
// step is aborted (this wait timed out or another workgroup aborted) it sets `fail` (the workgroup's LDS flag), which
// the caller reads after the barrier that ends the wait. `fail` must stay an LDS access: a generic (flat) read would
// also wait for every global load in flight, the prefetched weights included. Returns the number of passes this thread
// made (the stage-timing build records it).
template <int E, typename F>
__device__ __forceinline__ int gather(F idx, int n, uint32_t tag, float* dst, uint32_t* hdr, int stage, int& fail,
                                      long long limit) {
    const int t = threadIdx.x;
    if (n <= 0) {
        lds_barrier();
        return 0;
    }
    uint64_t v[E];
    bool pend[E];
#pragma unroll
    for (int e = 0; e < E; ++e) pend[e] = t + e * kThreads < n;
    long long start = 0;
    int it = 0;
    for (;; ++it) {
#pragma unroll
        for (int e = 0; e < E; ++e)
            if (pend[e]) v[e] = __hip_atomic_load(idx(t + e * kThreads), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        bool any = false;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            pend[e] = pend[e] && uint32_t(v[e] >> 32) != tag;
            any |= pend[e];
        }
        if (!any || wait_over(it, start, limit, hdr, stage, fail)) break;
    }
#pragma unroll
    for (int e = 0; e < E; ++e)
        if (t + e * kThreads < n) dst[t + e * kThreads] = __uint_as_float(uint32_t(v[e]));
    lds_barrier();
    // Nothing is in flight now (every poll waited for all older loads and stores); saying so lets the compiler's
    // wait counting start from zero after the loop instead of waiting for loads issued later.
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    return it + 1;
}

// Block-wide: waits until the 4-byte entries of the 16-byte vectors at byte offsets voff(v) from base, v < nv
// (nv <= E * 512, every offset below `bytes`), carry `parity` and writes vector v to dst[4 v .. 4 v + 3] (LDS, 16-byte
// aligned). 16-byte device-scope loads, four entries each; otherwise as gather.
template <int E, typename F>
__device__ __forceinline__ int gather32x4(const uint32_t* base, int bytes, F voff, int nv, uint32_t parity,
                                           float* dst, uint32_t* hdr, int stage, int& fail, long long limit) {
    const int t = threadIdx.x;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(base), (short)0, bytes, 0x00020000);
    constexpr int kSc1 = 16;  // the buffer load's cache policy: device scope (sc1)
    u32x4 v[E];
    int off[E];
    bool pend[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        pend[e] = t + e * kThreads < nv;
        off[e] = pend[e] ? voff(t + e * kThreads) : 0;
    }
    long long start = 0;
    int it = 0;
    for (;; ++it) {
        asm volatile("" ::: "memory");  // every pass loads again
#pragma unroll
        for (int e = 0; e < E; ++e)
            if (pend[e]) v[e] = __builtin_amdgcn_raw_buffer_load_b128(rs, off[e], 0, kSc1);
        bool any = false;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const uint32_t all = v[e][0] & v[e][1] & v[e][2] & v[e][3], some = v[e][0] | v[e][1] | v[e][2] | v[e][3];
            const bool ready = parity ? (all & 1u) != 0u : (some & 1u) == 0u;
            pend[e] = pend[e] && !ready;
            any |= pend[e];
        }
        if (!any || wait_over(it, start, limit, hdr, stage, fail)) break;
    }
#pragma unroll
    for (int e = 0; e < E; ++e)
        if (t + e * kThreads < nv) *reinterpret_cast<u32x4*>(dst + 4 * (t + e * kThreads)) = v[e];
    lds_barrier();
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0), as in gather
    return it + 1;
}

// Block-wide: waits for the per-XCD partial sums [kXcds][kH] at base (4-byte parity entries) and adds them to the
// residual stream xres: thread t polls rows 4 (t % 256) .. + 3 of XCDs 4 (t / 256) .. + 3 and sums them in XCD order in
// registers; the upper half's sums go through LDS (sc) to the lower half, which adds lower + upper to x. The same
// order in every workgroup, so the same bits. As gather otherwise.
__device__ __forceinline__ int gather_sum8(const uint32_t* base, uint32_t parity, float* xres, float* sc,
                                            uint32_t* hdr, int stage, int& fail, long long limit) {
    const int t = threadIdx.x, r4 = t & (kH / 4 - 1), x0 = (t / (kH / 4)) * 4;
    static_assert(kThreads == 2 * (kH / 4) && kXcds == 8, "two threads per 4 rows, four XCDs each");
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(base), (short)0, kXcds * kH * 4, 0x00020000);
    constexpr int kSc1 = 16;
    u32x4 v[4];
    bool pend[4];
#pragma unroll
    for (int x = 0; x < 4; ++x) pend[x] = true;
    long long start = 0;
    int it = 0;
    for (;; ++it) {
        asm volatile("" ::: "memory");
#pragma unroll
        for (int x = 0; x < 4; ++x)
            if (pend[x]) v[x] = __builtin_amdgcn_raw_buffer_load_b128(rs, ((x0 + x) * kH + 4 * r4) * 4, 0, kSc1);
        bool any = false;
#pragma unroll
        for (int x = 0; x < 4; ++x) {
            const uint32_t all = v[x][0] & v[x][1] & v[x][2] & v[x][3], some = v[x][0] | v[x][1] | v[x][2] | v[x][3];
            const bool ready = parity ? (all & 1u) != 0u : (some & 1u) == 0u;
            pend[x] = pend[x] && !ready;
            any |= pend[x];
        }
        if (!any || wait_over(it, start, limit, hdr, stage, fail)) break;
    }
    float4 sum;
    sum.x = __uint_as_float(v[0][0]), sum.y = __uint_as_float(v[0][1]);
    sum.z = __uint_as_float(v[0][2]), sum.w = __uint_as_float(v[0][3]);
#pragma unroll
    for (int x = 1; x < 4; ++x) {
        sum.x += __uint_as_float(v[x][0]), sum.y += __uint_as_float(v[x][1]);
        sum.z += __uint_as_float(v[x][2]), sum.w += __uint_as_float(v[x][3]);
    }
    if (x0) *reinterpret_cast<float4*>(sc + 4 * r4) = sum;
    lds_barrier();
    if (!x0) {
        const float4 hi = *reinterpret_cast<const float4*>(sc + 4 * r4);
        float4 xr = *reinterpret_cast<const float4*>(xres + 4 * r4);
        xr.x += sum.x + hi.x, xr.y += sum.y + hi.y, xr.z += sum.z + hi.z, xr.w += sum.w + hi.w;
        *reinterpret_cast<float4*>(xres + 4 * r4) = xr;
    }
    lds_barrier();
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0), as in gather
    return it + 1;
}

// This lane's values k = 512 c + 8 lane + e of RMSNorm(vec) (vec in LDS, 512 NCH wide): every wave reads the whole
// vector and reduces its own sum of squares, in the order of the multi-kernel GEMVs (rmsnorm_chunks).
template <int NCH>
__device__ __forceinline__ void norm_lane(const float* vec, const u32x4 (&nw)[NCH], float eps, float (&xv)[NCH][8]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const float4 lo = *reinterpret_cast<const float4*>(vec + 512 * c + 8 * lane);
        const float4 hi = *reinterpret_cast<const float4*>(vec + 512 * c + 8 * lane + 4);
        xv[c][0] = lo.x, xv[c][1] = lo.y, xv[c][2] = lo.z, xv[c][3] = lo.w;
        xv[c][4] = hi.x, xv[c][5] = hi.y, xv[c][6] = hi.z, xv[c][7] = hi.w;
    }
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = fmaf(xv[c][e], xv[c][e], ss);
    ss = wave_sum(ss);
    const float r = 1.0f / sqrtf(ss / float(512 * NCH) + eps);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        float g[8];
        unpack8bf(nw[c], g);
#pragma unroll
        for (int e = 0; e < 8; ++e) xv[c][e] = g[e] * (xv[c][e] * r);
    }
}

// sum over this lane's chunks of w . v (8 fp16 weights, f32 vector in registers), not yet reduced over the wave: the
// products in element order, each a v_fma_mix_f32 on its half of the packed pair. (Written with the halves taken by
// shifts and masks: a bit cast of the vector's element to a half pair made this compiler load only the first of the
// four words and use it for all of them.)
__device__ __forceinline__ float dot8(u32x4 wv, const float* v, float acc) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        acc = fmaf(v[2 * i], h2f(uint16_t(wv[i] & 0xFFFFu)), acc);
        acc = fmaf(v[2 * i + 1], h2f(uint16_t(wv[i] >> 16)), acc);
    }
    return acc;
}

// the same with the vector in LDS at vec[k0 .. k0 + 7]
__device__ __forceinline__ float dot8_lds(u32x4 wv, const float* vec, int k0, float acc) {
    const float4 lo = *reinterpret_cast<const float4*>(vec + k0);
    const float4 hi = *reinterpret_cast<const float4*>(vec + k0 + 4);
    const float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
    return dot8(wv, v, acc);
}

// Rows q = c / CPR of this wave's kRowsW rows, the lane's chunks c = lane + 64 i (CPR 16-byte chunks per row) dotted
// with the vector in LDS; the row sums go to red[w kRowsW + q].
template <int NC, int CPR>
__device__ __forceinline__ void rows_dot(const u32x4 (&wr)[NC], const float* vec, float* red) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    float acc[kRowsW];
#pragma unroll
    for (int q = 0; q < kRowsW; ++q) acc[q] = 0.f;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
        const int c = lane + 64 * i, q = c / CPR, kc = c - q * CPR;
        const float d = dot8_lds(wr[i], vec, 8 * kc, 0.f);
#pragma unroll
        for (int qq = 0; qq < kRowsW; ++qq)
            if (qq == q) acc[qq] += d;
    }
    const float s = wave_sum_rows<kRowsW>(acc);  // row q in lanes 16 q .. + 15
    if ((lane & (64 / kRowsW - 1)) == 0) red[w * kRowsW + lane / (64 / kRowsW)] = s;
}

// Stage stamps of the timing build (persist.hpp, LRM_PERSIST_STAMPS); nothing in the shipped build. Thread 0 keeps
// them in LDS (st_lds) and copies them to memory when the workgroup is done, so no store of theirs is in flight while
// the step runs (a wait for the loads in flight would also wait for it).
#if defined(LRM_PERSIST_STAMPS)
#define PSTAMP(k)                                                                                      \
    do {                                                                                               \
        if (t == 0 && (l == kStampLayer || l == kStampLayer + 1)) st_lds[(k) + 16 * (l - kStampLayer)] = wall_clock64(); \
    } while (0)
#define PSTAMP_AT(k)                            \
    do {                                        \
        if (t == 0) st_lds[k] = wall_clock64(); \
    } while (0)
#define PITER(k, n)                                                      \
    do {                                                                 \
        const int n_ = (n);                                              \
        if (t == 0 && l == kStampLayer) st_lds[32 + (k)] = uint64_t(n_); \
    } while (0)
#define PSUB(k)                                                           \
    do {                                                                  \
        if (t == 0 && l == kStampLayer) st_lds[48 + (k)] = wall_clock64(); \
    } while (0)
#define PFLUSH()                                                           \
    do {                                                                   \
        if (t == 0)                                                        \
            for (int k_ = 0; k_ < kStampWords; ++k_) stamps[k_] = st_lds[k_]; \
    } while (0)
#else
#define PSTAMP(k) \
    do {          \
    } while (0)
#define PSTAMP_AT(k) \
    do {             \
    } while (0)
#define PITER(k, n) \
    do {            \
        (void)(n);  \
    } while (0)
#define PSUB(k) \
    do {        \
    } while (0)
#define PFLUSH() \
    do {         \
    } while (0)
#endif

__global__ __launch_bounds__(kThreads, 1) void k_decode_persist(PArgs a) {
    __shared__ __align__(16) float vec[kVecMax];
    __shared__ __align__(16) float xres[kH];  // the residual stream: every workgroup holds all of it, the same bits
    __shared__ float red[64];
    __shared__ __align__(16) float qs[2][128];
    __shared__ float knew[128], vnew[128];
    __shared__ float ps[2][64];
    __shared__ float alpha_s[2];
    __shared__ float lmv[kWaves];
    __shared__ uint32_t lmi[kWaves];
    __shared__ int s_fail;
    // the odd chunks' scores and rescale factors (the even ones use ps and alpha_s)
    __shared__ float ps_odd[2][64];
    __shared__ float alpha_odd[2];

    const int b = blockIdx.x, t = threadIdx.x, lane = t & 63;
    const int w = __builtin_amdgcn_readfirstlane(t >> 6);  // wave-uniform: row offsets stay scalar
    // KV head xcd = this workgroup's XCD (hardware register XCC_ID); j = its index among the XCD's workgroups
    const int xcd = __builtin_amdgcn_s_getreg((3 << 11) | 20) & (kXcds - 1), j = b / kXcds;
    uint32_t* hdr = reinterpret_cast<uint32_t*>(a.xch);
    const uint32_t pos = word_load(a.state), id = word_load(a.state + 1), step = word_load(a.state + 2);
    const uint32_t tag = word_load(hdr) + 1u;
    const uint32_t par = tag & 1u;  // the tag of the 4-byte entries
    if (pos >= uint32_t(a.max_pos) || word_load(hdr + 1) != 0u) return;  // the same words for every workgroup
    const uint32_t wait_word = word_load(hdr + 3);  // the bound of every wait, in constant-clock ticks (0: default)
    const long long wait_ticks = wait_word ? (long long)wait_word : kWaitTicks;
    if (t == 0) s_fail = 0;

    const int MP = a.max_pos, S = kJN;
    const XLayout X(kQH, kKVH, kH, kI, kG);
    uint64_t* const lmp = a.xch + kHdrEntries + size_t(a.layers) * X.per_layer64;  // lm_head partials
    uint32_t* const x32 = reinterpret_cast<uint32_t*>(lmp + (2 * kG + 511) / 512 * 512);  // the 4-byte area
#if defined(LRM_PERSIST_STAMPS)
    uint64_t* const stamps = reinterpret_cast<uint64_t*>(x32 + size_t(a.layers) * X.per_layer32) + size_t(b) * kStampWords;
    __shared__ uint64_t st_lds[kStampWords];
    if (t == 0)
        for (int k = 0; k < kStampWords; ++k) st_lds[k] = 0;
#endif
    PSTAMP_AT(40);

    // attention split of this workgroup (stage B): fixed for the step
    const int hk = xcd, s = j;
    const int ntot = int(pos) + 1;
    // keys per split: whole 64-key chunks covering pos + 1 keys in 32 splits, one chunk more where that would take
    // more than 28 splits (stage C gathers the partial rows of up to 23 splits in one pass; a second pass over 29-32
    // splits costs more than the longer chain of one more chunk: per token at contexts 2000 / 4000 / 5500, 479.8 /
    // 520.7 / 550.6 us against 502.5 / 537.9 / 557.5; at 24-26 splits (contexts 1600, 3200, 4500) the extra chunk
    // measured no better, 478.8 / 513.3 / 542.8 against 467.3 / 512.8 / 543.1)
    int KPS = ((ntot + S - 1) / S + 63) / 64 * 64;
    if ((ntot + KPS - 1) / KPS > 28) KPS += 64;
    const int S_used = (ntot + KPS - 1) / KPS;
    const bool attn = s < S_used;
    const bool has_pos = s == S_used - 1;  // the split of the last key, pos
    const int k0 = s * KPS, nk = attn ? min(KPS, ntot - k0) : 0, nch = (nk + 63) / 64;
    const int jnew = int(pos) - k0;

    // stage A: the XCD's q|k|v rows, local row lr = the XCD's query heads (0 .. 255), its key (256 ..), its value
    u32x4 wa[kRA][kNCH], na[kNCH];
    auto issue_a = [&](int l) __attribute__((always_inline)) {
        const uint16_t* W = a.qkv + size_t(l) * (kQC + 2 * kKC) * kH;
#pragma unroll
        for (int r = 0; r < kRA; ++r) {
            const int lr = j * kWaves + w + r * kJN * kWaves;
            const int row = lr < kQPK * 128         ? kQPK * 128 * hk + lr
                            : lr < (kQPK + 1) * 128 ? kQC + 128 * hk + lr - kQPK * 128
                                                    : kQC + kKC + 128 * hk + lr - (kQPK + 1) * 128;
#pragma unroll
            for (int c = 0; c < kNCH; ++c) wa[r][c] = ld16(W + size_t(row) * kH + 512 * c + 8 * lane);
        }
#pragma unroll
        for (int c = 0; c < kNCH; ++c) na[c] = ld16(a.in_norm + size_t(l) * kH + 512 * c + 8 * lane);
    };

    // claim role (xcd, j) for this launch; the answer is checked after the embed, behind the loads issued before it
    uint32_t prior_claim = 0;
    if (t == 0)
        prior_claim = __hip_atomic_exchange(hdr + kClaimWord + xcd * kJN + j, tag, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);

    // x = widen(E[id]) (NaN for an id outside the vocabulary, as embed_dec)
    issue_a(0);
    for (int k = t; k < kH; k += kThreads)
        xres[k] = id < uint32_t(a.vocab) ? bf2f(a.embed[size_t(id) * kH + k]) : __uint_as_float(0x7FC00000u);
    if (t == 0 && prior_claim == tag) abort_step(hdr, kStageClaim);  // another workgroup holds this role
    lds_barrier();

    // This split's first 64-key chunks of K and V^T (one when the split holds one, else two): they do not depend on
    // this step, so layer l + 1's load during layer l (layer 0's here): the first after stage C's wait, the second at
    // the end of the layer, so neither wait for x holds back much behind them. K: thread t holds key slots t / 16 and t / 16 + 32
    // of a chunk, dims 8 (t % 16) .. + 7; V^T: dim t / 4, keys 16 (t % 4) .. + 15. Past the last chunk: re-read it
    // (never used).
    u32x4 kr[2][2], vr[2][2];
    auto fetch_k = [&](auto set, int l, int c) __attribute__((always_inline)) {
        constexpr int SET = decltype(set)::value;
        const uint16_t* kb = a.kc + ((size_t(l) * kKVH + hk) * MP + k0) * 128 + 8 * (t & 15);
        const int cc = min(c, nch - 1) * 64;
#pragma unroll
        for (int i = 0; i < 2; ++i) kr[SET][i] = ld16(kb + size_t(cc + (t >> 4) + 32 * i) * 128);
    };
    auto fetch_v = [&](auto set, int l, int c) __attribute__((always_inline)) {
        constexpr int SET = decltype(set)::value;
        const uint16_t* vb = a.vc + (size_t(l) * kKVH + hk) * 128 * MP + 16 * (t & 3);
        const int cc = min(c, nch - 1) * 64;
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) vr[SET][jj] = ld16(vb + kv::v_at(k0 + cc, t >> 2) + 8 * jj);
    };
    auto fetch = [&](auto set, int l, int c) __attribute__((always_inline)) {
        fetch_k(set, l, c);
        fetch_v(set, l, c);
    };
    using C0 = std::integral_constant<int, 0>;
    using C1 = std::integral_constant<int, 1>;
    if (attn) {
        fetch(C0{}, 0, 0);
        if (nch > 1) fetch(C1{}, 0, 1);
    }

    for (int l = 0; l < a.layers; ++l) {
        uint64_t* const q64 = a.xch + kHdrEntries + size_t(l) * X.per_layer64 + size_t(xcd) * X.blk64;  // XCD block
        uint32_t* const l32 = x32 + size_t(l) * X.per_layer32;
        uint32_t* const o32 = l32 + size_t(xcd) * X.blk32;  // this XCD's 4-byte block
        // ---------------------------------------------------------------- A: q|k|v = W_qkv . RMSNorm(x)
        PSTAMP(0);
        if (l > 0) {
            PITER(0, gather_sum8(l32 - X.per_layer32 + X.p2, par, xres, vec, hdr, 1, s_fail, wait_ticks));
            if (s_fail) return;
        }
        PSTAMP(1);
        u32x4 wc[kNCC];
        {
            float xv[kNCH][8];
            norm_lane<kNCH>(xres, na, a.eps, xv);
            PSUB(0);
            float acc[kRA];
#pragma unroll
            for (int r = 0; r < kRA; ++r) {
                acc[r] = 0.f;
#pragma unroll
                for (int c = 0; c < kNCH; ++c) acc[r] = dot8(wa[r][c], xv[c], acc[r]);
            }
            const float sr = wave_sum_rows<kRA>(acc);  // row r in lanes 32 r .. + 31
            if ((lane & (64 / kRA - 1)) == 0) red[(lane / (64 / kRA)) * kWaves + w] = sr;
            PSUB(1);
        }
        // one wave stores the workgroup's rows (runs of kWaves consecutive entries), so each run is one write of whole
        // 8-byte entries from one instruction
        lds_barrier();
        PSTAMP(2);
        if (t < kRA * kWaves) lstore(q64 + X.qkv + j * kWaves + (t % kWaves) + (t / kWaves) * kJN * kWaves, red[t], tag);
        // stage C's o_proj weights (rows 32 j + 4 w + q, the XCD's 256 columns), issued after the rows above have
        // left: a load issue that waits for room in the memory queue would otherwise hold them back
#pragma unroll
        for (int i = 0; i < kNCC; ++i) {
            const int c = lane + 64 * i, q = c / (kCW / 8), kc = c - q * (kCW / 8);
            wc[i] = ld16(a.o_proj + (size_t(l) * kH + j * kRowsG + w * kRowsW + q) * kQC + kCW * hk + 8 * kc);
        }

        // ---------------------------------------------------------------- B: attention over this split
        if (attn) {
            // the rotation of pos and the norm weights do not depend on the step's projections: load them first
            const int grp = t >> 7, d = t & 127;
            const float cs = a.cos_t[size_t(pos) * 64 + (d & 63)], sn = a.sin_t[size_t(pos) * 64 + (d & 63)];
            const float nwt = bf2f(t < 256 ? a.q_norm[l * 128 + d] : a.k_norm[l * 128 + d]);
            const float nwp = bf2f(t < 256 ? a.q_norm[l * 128 + (d ^ 64)] : a.k_norm[l * 128 + (d ^ 64)]);
            const uint64_t* src = q64 + X.qkv;  // the XCD's query heads, then its key and value
            PITER(1, gather<1>([&](int i) { return src + i; }, has_pos ? 512 : 256, tag, vec, hdr, 2, s_fail, wait_ticks));
            if (s_fail) return;
            PSTAMP(3);
            // per-head RMSNorm (q heads: threads 0-255, the new key: 256-383), then the rotation of (d, d + 64): each
            // thread normalises its partner element d ^ 64 too (the same expression as the partner's own thread, so the
            // same bits) instead of exchanging it through LDS; the split holding pos appends the rotated key and the
            // value to the caches, rounded to fp16
            const float val = (t < 256 || has_pos) ? vec[t] : 0.f;
            const float valp = (t < 256 || has_pos) ? vec[t ^ 64] : 0.f;
            const float sq = wave_sum(val * val);
            if (lane == 0) red[w] = sq;
            lds_barrier();
            PSUB(2);
            const float rn = 1.0f / sqrtf((red[2 * grp] + red[2 * grp + 1]) / 128.0f + a.eps);
            const float nr = nwt * (val * rn), np = nwp * (valp * rn);
            const float rot = d < 64 ? nr * cs - np * sn : nr * cs + np * sn;
            if (t < 256) {
                qs[grp][d] = rot;
            } else if (t < 384) {
                const uint16_t kh = f2h(rot);
                knew[d] = h2f(kh);
                if (has_pos) {
                    a.kc[((size_t(l) * kKVH + hk) * MP + pos) * 128 + d] = kh;
                    f16_note(f16_bad2(kh), kF16Cache);
                }
            } else {
                const uint16_t vh = f2h(val);
                vnew[d] = h2f(vh);
                if (has_pos) {
                    a.vc[(size_t(l) * kKVH + hk) * 128 * MP + kv::v_at(pos, d)] = vh;
                    f16_note(f16_bad2(vh), kF16Cache);
                }
            }
            lds_barrier();
            PSUB(3);
            // this thread's query dims and, for the split holding pos, its slices of the new key and value (read
            // unconditionally, used through selects)
            const int d0 = 8 * (t & 15);
            float q0[8], q1[8], kn8[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                q0[e] = qs[0][d0 + e];
                q1[e] = qs[1][d0 + e];
                kn8[e] = knew[d0 + e];
            }
            const float vn = vnew[t >> 2];
            float m_run = -INFINITY, l_run = 0.f;  // waves 0 and 1: the running statistics of head w
            float o0 = 0.f, o1 = 0.f;              // dim t / 4 of both heads over keys 16 (t % 4) .. + 15
            // chunk c from register set SET; with refill >= 0 the set's K registers take chunk refill's keys as soon as
            // the scores are taken and its V^T registers after P V, so the refill's K load has the softmax and P V to
            // land in
            auto chunk = [&](auto set, auto tailc, int c, int refill) __attribute__((always_inline)) {
                constexpr int SET = decltype(set)::value;
                constexpr bool tail = decltype(tailc)::value;
                const int cb = c * 64;
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const int key = (t >> 4) + 32 * i;
                    float kf[8];
                    unpack8h(kr[SET][i], kf);
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
                    if ((t & 15) == 0) {
                        const bool ok = !tail || cb + key < nk;
                        (SET ? ps_odd : ps)[0][key] = ok ? a0 * a.scale_log2 : -INFINITY;
                        (SET ? ps_odd : ps)[1][key] = ok ? a1 * a.scale_log2 : -INFINITY;
                    }
                }
                if (refill >= 0) fetch_k(set, l, refill);
                lds_barrier();
                if (w < 2) {  // online softmax of head w over the chunk (its key 0 is always valid)
                    const float v = (SET ? ps_odd : ps)[w][lane];
                    const float m_new = fmaxf(m_run, wave_max(v));
                    const float e = exp2f(v - m_new);
                    const float al = exp2f(m_run - m_new);  // 0 on the first chunk
                    l_run = l_run * al + wave_sum(e);
                    m_run = m_new;
                    (SET ? ps_odd : ps)[w][lane] = e;
                    if (lane == 0) (SET ? alpha_odd : alpha_s)[w] = al;
                }
                lds_barrier();
                const int kg = 16 * (t & 3);
                float a0 = 0.f, a1 = 0.f;
#pragma unroll
                for (int jj = 0; jj < 2; ++jj) {
                    float vf[8];
                    unpack8h(vr[SET][jj], vf);
                    if constexpr (tail) {
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            const int key = cb + kg + 8 * jj + e;
                            vf[e] = key >= nk ? 0.f : (has_pos && key == jnew ? vn : vf[e]);
                        }
                    }
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        a0 = fmaf((SET ? ps_odd : ps)[0][kg + 8 * jj + e], vf[e], a0);
                        a1 = fmaf((SET ? ps_odd : ps)[1][kg + 8 * jj + e], vf[e], a1);
                    }
                }
                o0 = fmaf(o0, (SET ? alpha_odd : alpha_s)[0], a0);
                o1 = fmaf(o1, (SET ? alpha_odd : alpha_s)[1], a1);
                if (refill >= 0) fetch_v(set, l, refill);
                // no barrier before the next chunk: it writes the other parity's ps and alpha_s, and the chunk after
                // it writes these only past its first barrier, which every wave reaches after this P V
            };
            using Body = std::false_type;
            using Tail = std::true_type;
            PSUB(4);
            int c = 0;
            for (; c + 2 < nch; c += 2) {  // whole pairs before the last chunk
                chunk(C0{}, Body{}, c, c + 2);
                chunk(C1{}, Body{}, c + 1, c + 3);
            }
            if (c + 1 < nch) {
                chunk(C0{}, Body{}, c, -1);
                chunk(C1{}, Tail{}, c + 1, -1);
            } else {
                chunk(C0{}, Tail{}, c, -1);
            }
            PSUB(5);
            // reduce the four key groups of each dim, then the partial rows of both heads, (out[128], max, sum) and
            // two pad entries, each written whole by one wave (wave hh: the XCD's query head hh) from LDS (qs and red
            // are free after the chunks)
            o0 = quad4_sum(o0);
            o1 = quad4_sum(o1);
            if ((t & 3) == 0) {
                qs[0][t >> 2] = o0;
                qs[1][t >> 2] = o1;
            }
            if (w < 2 && lane == 0) {
                red[2 * w] = m_run;
                red[2 * w + 1] = l_run;
            }
            lds_barrier();
            PSTAMP(4);
            if (w < 2) {
                uint32_t* pr = o32 + X.part + size_t(w * S + s) * kPartStride;
#pragma unroll
                for (int i = lane; i < 4 * kPartVecs; i += 64)
                    lstore32(pr + i, i < 128 ? qs[w][i] : i < 130 ? red[2 * w + i - 128] : 0.f, par);
            }
        } else if (w < 2) {  // no keys in this split: its rows are not read, but every step writes them (parity)
            uint32_t* pr = o32 + X.part + size_t(w * S + s) * kPartStride;
#pragma unroll
            for (int i = lane; i < 4 * kPartVecs; i += 64) lstore32(pr + i, 0.f, par);
        }

        // ---------------------------------------------------------------- C: p1[xcd] = W_o[:, the XCD's columns] . o
        PSTAMP(5);
        // o of the XCD's two query heads, formed by every workgroup from the splits' partial rows (row r = hh S_used
        // + sp of the gathered rows at vec[132 r ..]): the split weights 2^(m_sp - M), summed in split order
        lds_barrier();  // vec may still be read by stage B's waves
        {
            // up to 3 vectors per thread at once (more would spill registers); at long contexts the rest follow
            constexpr int kV1 = 3 * kThreads;
            auto voff = [&](int v) {
                const int r = v / kPartVecs, c = v - r * kPartVecs, hh = r / S_used, sp = r - hh * S_used;
                return ((hh * S + sp) * kPartStride + 4 * c) * 4;
            };
            const int nv = 2 * S_used * kPartVecs;
            PITER(2, gather32x4<3>(o32 + X.part, 2 * S * kPartStride * 4, voff, min(nv, kV1), par, vec, hdr, 4, s_fail,
                                   wait_ticks));
            if (s_fail) return;
            PSUB(12);
            if (nv > kV1) {
                static_assert(2 * kJN * kPartVecs <= kV1 + 2 * kThreads, "the partial rows in two passes");
                PITER(3, gather32x4<2>(o32 + X.part, 2 * S * kPartStride * 4, [&](int v) { return voff(v + kV1); },
                                       nv - kV1, par, vec + 4 * kV1, hdr, 4, s_fail, wait_ticks));
                if (s_fail) return;
            }
        }
        // the next layer's first K/V chunk (its registers are free once this layer's attention is done): in flight
        // through this stage's compute and the wait for the o_proj sums, away from the next layer's first wait
        PSUB(13);
        if (attn) fetch(C0{}, min(l + 1, a.layers - 1), 0);
        if (w < 2) {  // wave hh: the split weights 2^(m_sp - M) / sum_sp 2^(m_sp - M) l_sp of query head hh, a split per lane
            const bool ok = lane < S_used;
            const float* r = vec + (w * S_used + (ok ? lane : 0)) * 4 * kPartVecs;
            const float m = ok ? r[128] : -INFINITY;
            const float M = wave_max(m);
            const float e = ok ? exp2f(m - M) : 0.f;
            const float L = wave_sum(ok ? r[129] * e : 0.f);
            ps[w][lane] = e / L;
        }
        lds_barrier();
        PSTAMP(6);
        if (t < kCW) {  // in split order; four splits' weights and rows read ahead of their FMAs
            const int hh = t >> 7, d = t & 127;
            const float* rows = vec + hh * S_used * 4 * kPartVecs + d;
            float O = 0.f;
            int sp = 0;
            for (; sp + 4 <= S_used; sp += 4) {
                float pw[4], rv[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    pw[u] = ps[hh][sp + u];
                    rv[u] = rows[(sp + u) * 4 * kPartVecs];
                }
#pragma unroll
                for (int u = 0; u < 4; ++u) O = fmaf(pw[u], rv[u], O);
            }
            for (; sp < S_used; ++sp) O = fmaf(ps[hh][sp], rows[sp * 4 * kPartVecs], O);
            qs[hh][d] = O;
        }
        lds_barrier();
        PSUB(6);
        rows_dot<kNCC, kCW / 8>(wc, &qs[0][0], red);
        PSUB(7);
        lds_barrier();
        PSTAMP(8);
        if (t < kRowsG) gstore32(l32 + X.p1 + xcd * kH + j * kRowsG + t, red[t], par);
        // stage D's gate/up weights, after the rows above: unit u = w kUD + jj is (row u / kNCH of the workgroup's
        // 2 kPB, chunk jj % kNCH); rows 0 .. kPB - 1 are gate rows 384 xcd + 12 j + r, the rest the matching up rows
        u32x4 wd[kUD], nd[kNCH];
#pragma unroll
        for (int jj = 0; jj < kUD; ++jj) {
            const int ri = (w * kUD + jj) / kNCH, c = jj % kNCH;
            const int grow = ri < kPB ? kEW * hk + kPB * j + ri : kI + kEW * hk + kPB * j + (ri - kPB);
            wd[jj] = ld16(a.gate_up + (size_t(l) * 2 * kI + grow) * kH + 512 * c + 8 * lane);
        }
#pragma unroll
        for (int c = 0; c < kNCH; ++c) nd[c] = ld16(a.post_norm + size_t(l) * kH + 512 * c + 8 * lane);

        // ---------------------------------------------------------------- D: a = silu(W_g . h) * (W_u . h)
        PITER(4, gather_sum8(l32 + X.p1, par, xres, vec, hdr, 5, s_fail, wait_ticks));
        if (s_fail) return;
        PSTAMP(9);
        // stage E's down_proj weights (rows 32 j + 4 w + q, the XCD's 384 columns), before this stage computes:
        // issued after its outputs they land only after the hand-off to stage E
        u32x4 we[kNCE];
#pragma unroll
        for (int i = 0; i < kNCE; ++i) {
            const int c = lane + 64 * i, q = c / (kEW / 8), kc = c - q * (kEW / 8);
            we[i] = ld16(a.down + (size_t(l) * kH + j * kRowsG + w * kRowsW + q) * kI + kEW * hk + 8 * kc);
        }
        {
            float xv[kNCH][8];
            PSUB(8);
            norm_lane<kNCH>(xres, nd, a.eps, xv);
            PSUB(9);
            // unit jj's sum goes to red[(row ri) kNCH + chunk c] = red[w kUD + jj] (kUD is even)
            float acc[8];
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) acc[jj] = jj < kUD ? dot8(wd[jj % kUD], xv[jj % kNCH], 0.f) : 0.f;
            const float su = wave_sum_rows<8>(acc);  // unit jj in lanes 8 jj .. + 7
            if ((lane & 7) == 0 && (lane >> 3) < kUD) red[w * kUD + (lane >> 3)] = su;
            PSUB(10);
        }
        lds_barrier();
        PSTAMP(10);
        if (t < kPB) {
            float g = 0.f, u = 0.f;
#pragma unroll
            for (int c = 0; c < kNCH; ++c) {
                g += red[t * kNCH + c];
                u += red[(kPB + t) * kNCH + c];
            }
            lstore32(o32 + X.a + kPB * j + t, g / (1.0f + __expf(-g)) * u, par);
        }

        // ---------------------------------------------------------------- E: p2[xcd] = W_d[:, the XCD's columns] . a
        PITER(5, gather32x4<1>(o32 + X.a, kEW * 4, [](int v) { return 16 * v; }, kEW / 4, par, vec, hdr, 6, s_fail,
                               wait_ticks));
        if (s_fail) return;
        PSTAMP(11);
        rows_dot<kNCE, kEW / 8>(we, vec, red);
        PSUB(11);
        lds_barrier();
        PSTAMP(12);
        if (t < kRowsG) gstore32(l32 + X.p2 + xcd * kH + j * kRowsG + t, red[t], par);
        // the next layer's q|k|v rows and second K/V chunk, after the rows above (after the last layer: its q|k|v rows
        // again, never used; unconditional, so the compiler's wait counting has one path to follow)
        issue_a(min(l + 1, a.layers - 1));
        if (l + 1 < a.layers && attn && nch > 1) fetch(C1{}, l + 1, 1);
    }

    PSTAMP_AT(41);
    // ---------------------------------------------------------------- lm_head over rows [r0, r1), then the argmax
    const int V = a.vocab, per = (V + kG - 1) / kG, r0 = b * per, r1 = min(V, r0 + per);
    u32x4 ra[4][kNCH], rb4[4][kNCH], rc4[4][kNCH], nf[kNCH];
    auto load4 = [&](u32x4 (&dst)[4][kNCH], int row) __attribute__((always_inline)) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint16_t* er = a.embed16 + size_t(min(row + r, V - 1)) * kH + 8 * lane;
#pragma unroll
            for (int c = 0; c < kNCH; ++c) dst[r][c] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(er + 512 * c));
        }
    };
    // wave w visits rows r0 + 4 w + 32 j, four at a time, through three register sets (the next two sets in flight
    // while one is reduced); the first two are issued before the wait for x
    constexpr int RS = 4 * kWaves;  // rows between a wave's consecutive sets
    load4(ra, r0 + 4 * w);
    load4(rb4, r0 + 4 * w + RS);
#pragma unroll
    for (int c = 0; c < kNCH; ++c) nf[c] = ld16(a.final_norm + 512 * c + 8 * lane);
    gather_sum8(x32 + size_t(a.layers - 1) * X.per_layer32 + X.p2, par, xres, vec, hdr, 7, s_fail, wait_ticks);
    if (s_fail) return;
    PSTAMP_AT(42);
    float xv[kNCH][8];
    norm_lane<kNCH>(xres, nf, a.eps, xv);
    float best = -INFINITY;
    uint32_t besti = 0xFFFFFFFFu;
    bool nan = false;
    auto proc = [&](const u32x4 (&src)[4][kNCH], int row) __attribute__((always_inline)) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float acc = 0.f;
#pragma unroll
            for (int c = 0; c < kNCH; ++c) acc = dot8(src[r][c], xv[c], acc);
            const float v = wave_sum(acc);
            if (row + r >= r1) continue;
            if (a.write_logits && lane == r) a.logits[row + r] = v;
            if (v != v) {
                nan = true;
            } else if (besti == 0xFFFFFFFFu || v > best) {  // rows are visited in increasing order
                best = v;
                besti = uint32_t(row + r);
            }
        }
    };
    for (int row = r0 + 4 * w; row < r1; row += 3 * RS) {  // sets ra, rb4, rc4 hold rows row, + RS, + 2 RS
        if (row + 2 * RS < r1) load4(rc4, row + 2 * RS);
        proc(ra, row);
        if (row + 3 * RS < r1) load4(ra, row + 3 * RS);
        if (row + RS < r1) proc(rb4, row + RS);
        if (row + 4 * RS < r1) load4(rb4, row + 4 * RS);
        if (row + 2 * RS < r1) proc(rc4, row + 2 * RS);
    }
    if (lane == 0) {
        lmv[w] = best;
        lmi[w] = nan ? 0xFFFFFFFEu : besti;
    }
    lds_barrier();
    if (t == 0) {
        float bv = 0.f;
        uint32_t ix = 0xFFFFFFFFu;
        bool bn = false;
        for (int i = 0; i < kWaves; ++i) {
            if (lmi[i] == 0xFFFFFFFEu)
                bn = true;
            else if (lmi[i] != 0xFFFFFFFFu && (ix == 0xFFFFFFFFu || lmv[i] > bv || (lmv[i] == bv && lmi[i] < ix))) {
                bv = lmv[i];
                ix = lmi[i];
            }
        }
        gstore(lmp + 2 * b, bv, tag);
        gstore(lmp + 2 * b + 1, __uint_as_float(bn ? 0xFFFFFFFEu : ix), tag);
    }
    PSTAMP_AT(43);
    if (b != 0) {
        PFLUSH();
        return;
    }

    // workgroup 0: the lowest index of the maximum over the workgroups' pairs (0xFFFFFFFF when a logit is NaN)
    gather<1>([&](int i) { return lmp + i; }, 2 * kG, tag, vec, hdr, 8, s_fail, wait_ticks);
    if (s_fail) return;
    float bv = 0.f;
    uint32_t bi = 0xFFFFFFFFu;
    bool bn = false;
    for (int i = t; i < kG; i += kThreads) {
        const float v = vec[2 * i];
        const uint32_t jx = __float_as_uint(vec[2 * i + 1]);
        if (jx == 0xFFFFFFFEu)
            bn = true;
        else if (jx != 0xFFFFFFFFu && (bi == 0xFFFFFFFFu || v > bv || (v == bv && jx < bi))) {
            bv = v;
            bi = jx;
        }
    }
    lds_barrier();  // vec is reused for the tree below
    float* sv = vec;
    uint32_t* si = reinterpret_cast<uint32_t*>(vec + kThreads);
    sv[t] = bv;
    si[t] = bi;
    if (t == 0) s_fail = 0;
    lds_barrier();
    if (bn) s_fail = 2;  // every writer stores the same value
    for (int h = kThreads / 2; h > 0; h >>= 1) {
        if (t < h) {
            const float ov = sv[t + h];
            const uint32_t oi = si[t + h];
            if (oi != 0xFFFFFFFFu && (si[t] == 0xFFFFFFFFu || ov > sv[t] || (ov == sv[t] && oi < si[t]))) {
                sv[t] = ov;
                si[t] = oi;
            }
        }
        lds_barrier();
    }
    if (t == 0) {
        const uint32_t nid = s_fail == 2 ? 0xFFFFFFFFu : si[0];
        if (step < uint32_t(a.max_steps)) a.out_ids[step] = nid;
        a.state[1] = nid;
        a.state[0] = pos + 1u;
        a.state[2] = step + 1u;
        __hip_atomic_store(hdr, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // the next launch's epoch
#if defined(LRM_PERSIST_STAMPS)
        st_lds[44] = wall_clock64();
#endif
    }
    PFLUSH();
}

}  // namespace

// ---------------------------------------------------------------- launcher (catalog id 38)
// fields: embed, final_norm, in_norm, qkv, q_norm, k_norm, o_proj, post_norm, gate_up, down, k_cache, v_cache, cos,
// sin, logits, state, out_ids, exchange, embed16, layers, hidden, q_heads, kv_heads, inter, vocab, max_pos, max_steps,
// write_logits, eps, scale, blocks
void* f16_range_word_persist() {
    void* p = nullptr;
    hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(fast::f16_range_word)), "hipGetSymbolAddress(f16_range_word)");
    if (!p) throw HipError("hipGetSymbolAddress(f16_range_word) returned a null address");
    return p;
}

void launch_decode_persistent(const PreparedDispatch& pd, void* const* p, hipStream_t s) {
    const uint32_t* w = pd.words.data();
    auto f32 = [](uint32_t u) {
        float f;
        std::memcpy(&f, &u, 4);
        return f;
    };
    PArgs a;
    a.embed = (const uint16_t*)p[0];
    a.embed16 = (const uint16_t*)p[18];
    a.final_norm = (const uint16_t*)p[1];
    a.in_norm = (const uint16_t*)p[2];
    a.qkv = (const uint16_t*)p[3];
    a.q_norm = (const uint16_t*)p[4];
    a.k_norm = (const uint16_t*)p[5];
    a.o_proj = (const uint16_t*)p[6];
    a.post_norm = (const uint16_t*)p[7];
    a.gate_up = (const uint16_t*)p[8];
    a.down = (const uint16_t*)p[9];
    a.kc = (uint16_t*)p[10];
    a.vc = (uint16_t*)p[11];
    a.cos_t = (const float*)p[12];
    a.sin_t = (const float*)p[13];
    a.logits = (float*)p[14];
    a.state = (uint32_t*)p[15];
    a.out_ids = (uint32_t*)p[16];
    a.xch = (uint64_t*)p[17];
    a.layers = int(w[20]);
    a.vocab = int(w[25]);
    a.max_pos = int(w[26]);
    a.max_steps = int(w[27]);
    a.write_logits = int(w[28]);
    a.eps = f32(w[29]);
    a.scale_log2 = f32(w[30]) * 1.4426950408889634f;
    auto kern = k_decode_persist;
    // every workgroup must be resident at once (they wait for each other): at least one per CU, G <= CUs
    static int occupancy = -1;
    if (occupancy < 0) hip_check(hipOccupancyMaxActiveBlocksPerMultiprocessor(&occupancy, kern, kThreads, 0), "occupancy");
    int dev = 0, cus = 0;
    hip_check(hipGetDevice(&dev), "device");
    hip_check(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), "attribute");
    if (occupancy < 1 || int64_t(pd.physical.x) > int64_t(cus) * occupancy)
        throw HipError("decode_step_persistent: the grid does not fit on the device at once");
    if (pd.physical.x != uint32_t(kG)) throw HipError("decode_step_persistent: the kernel runs 256 workgroups");
    hipLaunchKernelGGL(kern, dim3(pd.physical.x), dim3(kThreads), 0, s, a);
}

}  // namespace lrm
