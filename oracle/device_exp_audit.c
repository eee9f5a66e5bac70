/*
 * device_exp_audit.c -- exhaustive audit of the device's binary32 exp.
 *
 * TEST INFRASTRUCTURE ONLY (part of the oracle library; see tiler_oracle.h).
 *
 * The device computes e^s for binary32 s as tiler::exp_f32_cr does
 * (tiler_amd/csrc/kernels/common.h): in binary64, k = rint(s * 64/ln2),
 * r = s - k*(HI + LO) with two FMAs, a degree-6 Taylor polynomial in Horner
 * form with FMAs, times the table value 2^((k mod 64)/64), scaled by
 * 2^(k div 64), then one rounding to binary32 (round-to-nearest-even,
 * subnormals preserved: the kernels' float mode).  Every step is an IEEE
 * binary64 operation, so this file repeats it bit for bit on the CPU (C99
 * fma, rint and the same table constants, -ffp-contract=off).
 *
 * Error of the binary64 value v against e^s, relative:
 *   * the reduction r1 = fma(-k, HI, s) is exact (k*HI fits 51 bits, and the
 *     difference is a multiple of 2^-43 below 2^-7);
 *   * r = fma(-k, LO, r1) rounds once (2^-53 |r|), and HI + LO misses ln2/64
 *     by < 2^-99, so |k| (HI + LO - ln2/64) < 2^-85: e^r differs from e^r*
 *     by < 2^-60 relative;
 *   * the Taylor remainder is |r|^7/5040 e^|r| < 2^-65 for |r| <= ln2/128;
 *     Horner rounding is < 2.5 * 2^-53 (the last two FMAs dominate);
 *   * the table value and the final product each round once (2^-53 each).
 * In total |v/e^s - 1| < 4.6 * 2^-53 < 2^-50.7.  So wherever v lies farther
 * than 2^-50.7 v from both rounding boundaries of (float)v, e^s rounds to the
 * same binary32 value and the device result is the correctly rounded one.
 * The audit uses a wider margin (2^margin_log2, -48 by default) and checks
 * every input inside it against tiler_oracle_certified_exp_f32.
 *
 * planted_log2 != 0 plants a mistake for the audit's own test: every value is
 * scaled by (1 + 2^planted_log2) before rounding, a perturbation inside the
 * margin that the comparison must catch.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "tiler_oracle.h"

#define __device__
#define __constant__
#include "../tiler_amd/csrc/kernels/exp_table.h"
#undef __device__
#undef __constant__

static double device_exp_f64(double x, int *m_out) {
    double kd = rint(x * TILER_64_OVER_LN2);
    int k = (int)kd;
    double r = fma(-kd, TILER_LN2_OVER_64_HI, x);
    r = fma(-kd, TILER_LN2_OVER_64_LO, r);
    double p = 1.0 / 720.0;
    p = fma(p, r, 1.0 / 120.0);
    p = fma(p, r, 1.0 / 24.0);
    p = fma(p, r, 1.0 / 6.0);
    p = fma(p, r, 0.5);
    p = fma(p, r, 1.0);
    p = fma(p, r, 1.0);
    *m_out = k >> 6;
    return kExp2Table64[k & 63] * p;
}

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* v * 2^m, exact for the exponents this range produces (|m| < 160). */
static double scale2(double v, int m) {
    uint64_t bits = (uint64_t)(m + 1023) << 52;
    double p;
    memcpy(&p, &bits, 8);
    return v * p;
}

/* The binary64 value the device rounds to binary32, for -104 < s < 89. */
static double device_exp_unrounded(float s) {
    int m = 0;
    double core = device_exp_f64((double)s, &m);
    return scale2(core, m);
}

float tiler_oracle_device_exp_f32(float s) {
    if (s != s) return s;
    if (s >= 89.0f) return INFINITY;
    if (s <= -104.0f) return 0.0f;
    return (float)device_exp_unrounded(s);
}

/* Rounding boundaries of the binary32 interval that v rounds into. */
static void boundaries(double v, float yf, double *lo, double *hi) {
    if (yf == 0.0f) {                 /* below half the least subnormal */
        *lo = 0.0;
        *hi = ldexp(1.0, -150);
        return;
    }
    if (isinf(yf)) {                  /* above FLT_MAX + half an ulp */
        *lo = ldexp(1.0, 128) - ldexp(1.0, 103);
        *hi = INFINITY;
        return;
    }
    float below = u2f(f2u(yf) - 1u);  /* yf > 0 here */
    double up = yf == 0x1.fffffep127f ? ldexp(1.0, 128) : (double)u2f(f2u(yf) + 1u);
    *lo = ((double)below + (double)yf) * 0.5;  /* exact: the binary32 grid is far coarser */
    *hi = ((double)yf + up) * 0.5;
}

typedef struct {
    uint64_t begin, end;  /* bit patterns [begin, end) */
    double margin;
    double planted;       /* 0, or a relative perturbation applied before rounding */
    float *hard;
    uint64_t cap;
    uint64_t n_hard, n_checked, n_mismatch;
    float first_mismatch;
    pthread_mutex_t *lock;
    uint64_t *shared_hard;
} audit_job;

static void *audit_range(void *arg) {
    audit_job *j = (audit_job *)arg;
    for (uint64_t b = j->begin; b < j->end; ++b) {
        float s = u2f((uint32_t)b);
        if (s != s || s >= 89.0f || s <= -104.0f) continue;
        ++j->n_checked;
        double v = device_exp_unrounded(s);
        if (j->planted != 0.0) v = v + v * j->planted;
        float yf = (float)v;
        double lo, hi;
        boundaries(v, yf, &lo, &hi);
        double tol = j->margin * v;
        if (v - lo > tol && hi - v > tol) continue;
        ++j->n_hard;
        pthread_mutex_lock(j->lock);
        if (*j->shared_hard < j->cap) j->hard[*j->shared_hard] = s;
        ++*j->shared_hard;
        pthread_mutex_unlock(j->lock);
        float c;
        if (tiler_oracle_certified_exp_f32(s, &c) != TILER_ORACLE_OK || f2u(c) != f2u(yf)) {
            if (j->n_mismatch == 0) j->first_mismatch = s;
            ++j->n_mismatch;
        }
    }
    return NULL;
}

int32_t tiler_oracle_audit_device_exp(int32_t margin_log2, int32_t planted_log2,
                                      uint32_t threads, float *hard,
                                      uint64_t hard_cap, uint64_t *hard_count,
                                      uint64_t *checked, uint64_t *mismatches,
                                      float *first_mismatch) {
    if (threads == 0 || threads > 256 || margin_log2 > -30) return TILER_ORACLE_INVALID_APPLICATION;
    audit_job jobs[256];
    pthread_t tids[256];
    pthread_mutex_t lock = PTHREAD_MUTEX_INITIALIZER;
    uint64_t shared = 0, span = (1ull << 32) / threads + 1;
    for (uint32_t t = 0; t < threads; ++t) {
        audit_job *j = &jobs[t];
        memset(j, 0, sizeof *j);
        j->begin = (uint64_t)t * span;
        j->end = j->begin + span > (1ull << 32) ? (1ull << 32) : j->begin + span;
        j->margin = ldexp(1.0, margin_log2);
        j->planted = planted_log2 ? ldexp(1.0, planted_log2) : 0.0;
        j->hard = hard;
        j->cap = hard_cap;
        j->lock = &lock;
        j->shared_hard = &shared;
        pthread_create(&tids[t], NULL, audit_range, j);
    }
    uint64_t nh = 0, nc = 0, nm = 0;
    float fm = 0.0f;
    for (uint32_t t = 0; t < threads; ++t) {
        pthread_join(tids[t], NULL);
        nh += jobs[t].n_hard;
        nc += jobs[t].n_checked;
        if (jobs[t].n_mismatch && nm == 0) fm = jobs[t].first_mismatch;
        nm += jobs[t].n_mismatch;
    }
    *hard_count = nh;
    *checked = nc;
    *mismatches = nm;
    *first_mismatch = fm;
    return TILER_ORACLE_OK;
}
