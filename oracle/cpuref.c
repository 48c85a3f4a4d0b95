/* The oracle (test infrastructure only; never linked by the product). Common helpers, the exact RoPE table, and the
 * two instantiations of cpuref_ops.inc (float32 = CpuRef F32, float64 = CpuRef F64). */
#define _GNU_SOURCE
#include "cpuref.h"

#include <math.h>
#include <omp.h>
#include <quadmath.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static char g_error[512];
static int g_threads = 0;

const char *orc_last_error(void) { return g_error; }

static int orc_fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof g_error, fmt, ap);
    va_end(ap);
    return code;
}

void orc_set_threads(int n) { g_threads = n < 1 ? 1 : n; }

int orc_get_threads(void) { return g_threads > 0 ? g_threads : omp_get_max_threads(); }

/* CpuExec: threads split only independent outputs (CpuExec.fs:35-49); a loop of one task runs on the caller. */
static int orc_threads_for(int64_t tasks) {
    int n = orc_get_threads();
    if (tasks < n) n = tasks < 1 ? 1 : (int)tasks;
    return n;
}

#define ORC_PARALLEL_FOR _Pragma("omp parallel for schedule(static) num_threads(orc_get_threads())")

static float orc_f32_of_bits(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* Bf16.widen (Numerics.fs:28-33): the bf16 bits become the top half of a float32. */
float orc_bf16_widen(uint16_t bits) { return orc_f32_of_bits((uint32_t)bits << 16); }

/* Bf16.narrowRne (Numerics.fs:35-45): round to nearest even; NaN -> 0x7FC0 / 0xFFC0 by sign. */
uint16_t orc_bf16_narrow_rne(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u & 0x80000000u) ? 0xFFC0 : 0x7FC0;
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

/* CpuRef.attentionScale (CpuRef.fs:56-60): head_dim ** -0.5 in float64 (pow, as Python's **), rounded once. */
double orc_attention_scale_f64(int head_dim) { return head_dim < 1 ? NAN : pow((double)head_dim, -0.5); }
float orc_attention_scale_f32(int head_dim) { return (float)orc_attention_scale_f64(head_dim); }

/* ---- The exact RoPE table (Rope.fs:8-161, 202-251) ----
 * The reference computes the correctly rounded float64 cos and sin of a float32 argument in exact fixed-point integer
 * arithmetic. Any method that yields the correctly rounded value gives the same bits; this one evaluates cos and sin
 * in binary128 (libquadmath, error about one binary128 ulp, 2^-112 relative) and accepts the float64 rounding only when
 * the binary128 value lies farther than 2^-100 (relative) from the midpoint between two float64 neighbours, so the
 * error cannot move it across. Otherwise it reports failure instead of guessing. */
static int orc_round_certain(__float128 v, double *out) {
    double d = (double)v; /* binary128 -> binary64, round to nearest even */
    if (v == (__float128)d) {
        *out = d;
        return 1;
    }
    __float128 lo = ((__float128)d + (__float128)nextafter(d, -INFINITY)) / 2;
    __float128 hi = ((__float128)d + (__float128)nextafter(d, INFINITY)) / 2;
    __float128 tol = fabsq(v) * 0x1p-100Q;
    if (v - lo > tol && hi - v > tol) {
        *out = d;
        return 1;
    }
    return 0;
}

int orc_cos_sin_exact(float x, double *c, double *s) {
    if (!isfinite(x)) {
        *c = NAN;
        *s = NAN;
        return 0;
    }
    float ax = fabsf(x);
    if (ax < 0x1p-27f) { /* Rope.fs:150-152: cos rounds to 1 and sin to x exactly */
        *c = 1.0;
        *s = (double)x;
        return 0;
    }
    __float128 cq, sq;
    sincosq((__float128)ax, &sq, &cq);
    double cd, sd;
    if (!orc_round_certain(cq, &cd) || !orc_round_certain(sq, &sd))
        return orc_fail(-5, "no certain rounding for cos/sin(%a)", (double)x);
    *c = cd;
    *s = x < 0.0f ? -sd : sd;
    return 0;
}

/* RopeTable.create (Rope.fs:218-251): freq = f32(f32(pos) * inv_freq[j]); cos/sin = f32(RN64(cos/sin freq)). */
int orc_rope_table(const uint32_t *inv_freq_bits, int half, int max_pos, float *cos_out, float *sin_out) {
    if (!inv_freq_bits || half < 1) return orc_fail(-1, "ropeTable: no inverse frequencies");
    if (max_pos < 1 || max_pos > (1 << 24)) return orc_fail(-1, "ropeTable: max_pos %d outside 1 .. 2^24", max_pos);
    for (int j = 0; j < half; ++j)
        if (!isfinite(orc_f32_of_bits(inv_freq_bits[j]))) return orc_fail(-1, "ropeTable: inv_freq %08x is not finite", inv_freq_bits[j]);
    int bad = 0;
#pragma omp parallel for schedule(dynamic, 16) num_threads(orc_get_threads())
    for (int pos = 0; pos < max_pos; ++pos) {
        for (int j = 0; j < half; ++j) {
            volatile float fpos = (float)pos;
            float angle = fpos * orc_f32_of_bits(inv_freq_bits[j]);
            double c, s;
            if (orc_cos_sin_exact(angle, &c, &s) != 0) {
#pragma omp atomic write
                bad = 1;
            }
            cos_out[(int64_t)pos * half + j] = (float)c;
            sin_out[(int64_t)pos * half + j] = (float)s;
        }
    }
    return bad ? -5 : 0;
}

/* ---- CpuRef F32 ---- */
#define T float
#define S f32
#define FMA fmaf
#define EXP expf
#define LOG logf
#define SQRT sqrtf
#define WIDEN(b) orc_bf16_widen(b)
#include "cpuref_ops.inc"
#undef T
#undef S
#undef FMA
#undef EXP
#undef LOG
#undef SQRT
#undef WIDEN

/* ---- CpuRef F64 (bf16 widened exactly through float32) ---- */
#define T double
#define S f64
#define FMA fma
#define EXP exp
#define LOG log
#define SQRT sqrt
#define WIDEN(b) ((double)orc_bf16_widen(b))
#include "cpuref_ops.inc"
