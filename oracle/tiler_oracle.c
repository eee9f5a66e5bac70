/*
 * tiler_oracle.c -- CPU restatement of tiler-reference for the tiler-hip hot
 * path.  TEST INFRASTRUCTURE ONLY: see tiler_oracle.h for who may call it.
 *
 * Built with gcc -O2 -ffp-contract=off -fno-fast-math so every binary32
 * operation below is one IEEE round-to-nearest-even rounding, which is the
 * arithmetic the reference fixes (ADR 0024) and that Rust's f32 provides.
 *
 * Pinning (what checks each function, so a plausible mistake fails):
 *   strict sums / partitioned / cooperative -- the conformance operand sets of
 *     tiler-conformance/src/serial_sum.rs:202-368 (exact and grouping-sensitive
 *     bit patterns) plus brute force against exact rational sums;
 *   certified exp -- silu/tests.rs:35-91 corpus, softmax/tests.rs exponentials,
 *     and an independent 60-digit decimal exp (tests/test_oracle.py);
 *   certified rsqrt -- rms_norm/tests.rs:56-136 rows and an exact integer
 *     midpoint test (tests/test_oracle.py);
 *   rms_norm / softmax / silu -- every worked example and boundary row of
 *     rms_norm/tests.rs:253-420, softmax/tests.rs:362-651, silu/tests.rs:35-91;
 *   gather -- gather_conformance.rs:181-398 rows;
 *   strict-affine U4 dequantize -- the dequantize_one and scale-domain rows of
 *     quantization.rs:638-703 and every (code, zero point) pair against exact
 *     integer arithmetic (tests/test_oracle.py);
 *   strict contraction -- the six SHA-256 digests of
 *     tiler-reference/tests/contraction_profile_cells.rs:148-200;
 *   bf16 narrowing -- closed form (ADR 0091 decision 2) checked exhaustively
 *     against exact rational rounding over all 2^32 inputs' structure classes;
 *   grouped restatements -- brute force: each equals strict_partitioned_sum /
 *     exact sums on exactly-summable operands and differs on the separating set.
 */
#include "tiler_oracle.h"

#include <math.h>
#include <pthread.h>
#include <quadmath.h>
#include <stdlib.h>
#include <string.h>

#define CANONICAL_F32_NAN_BITS 0x7fc00000u /* tiler-ir/src/semantic/operation.rs:21 */
#define CANONICAL_BF16_NAN_BITS 0x7fc0u    /* ADR 0091 decision 2 */

static inline uint32_t f2u(float v) {
    uint32_t u;
    memcpy(&u, &v, 4);
    return u;
}
static inline float u2f(uint32_t u) {
    float v;
    memcpy(&v, &u, 4);
    return v;
}

uint32_t tiler_oracle_canonical_nan_bits(void) { return CANONICAL_F32_NAN_BITS; }

/* tiler-reference/src/lib.rs:144-150 canonicalize_arithmetic_f32 */
static inline float canon(float v) { return isnan(v) ? u2f(CANONICAL_F32_NAN_BITS) : v; }

/* tiler-reference/src/conformance.rs:498-521 apply() */
float tiler_oracle_apply_subnormal_mode(int32_t mode, float value) {
    if (mode == TILER_ORACLE_PRESERVE) return value;
    if (fpclassify(value) != FP_SUBNORMAL) return value;
    if (mode == TILER_ORACLE_FLUSH_SIGN_PRESERVING) return signbit(value) ? -0.0f : 0.0f;
    return 0.0f;
}
#define OPND(v) tiler_oracle_apply_subnormal_mode(input_mode, (v))
#define RSLT(v) tiler_oracle_apply_subnormal_mode(result_mode, (v))

/* tiler-reference/src/softmax.rs:168-186 maximum_f32: NaN-propagating IEEE
 * maximum with -0 < +0 (bitwise and of equal operands). */
float tiler_oracle_maximum_f32(float left, float right) {
    if (isnan(left) || isnan(right)) return u2f(CANONICAL_F32_NAN_BITS);
    if (left == right) return u2f(f2u(left) & f2u(right));
    return left > right ? left : right;
}

/* ADR 0091 decision 2 narrowing: RNE, overflow to signed infinity at the
 * inclusive midpoint above max finite (ties-to-even sends 0x7f7f8000 up),
 * every NaN to 0x7fc0, gradual underflow, signed zero kept.  bf16 shares the
 * binary32 exponent field, so RNE on the upper 16 bits is the whole rule. */
uint16_t tiler_oracle_bf16_narrow(float value) {
    uint32_t u = f2u(value);
    if (isnan(value)) return CANONICAL_BF16_NAN_BITS;
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}
float tiler_oracle_bf16_widen(uint16_t bits) { return u2f((uint32_t)bits << 16); }
void tiler_oracle_bf16_narrow_array(const float *in, uint64_t n, uint16_t *out) {
    for (uint64_t i = 0; i < n; ++i) out[i] = tiler_oracle_bf16_narrow(in[i]);
}
void tiler_oracle_bf16_widen_array(const uint16_t *in, uint64_t n, float *out) {
    for (uint64_t i = 0; i < n; ++i) out[i] = tiler_oracle_bf16_widen(in[i]);
}

/* ------------------------------------------------------------------------ */
/* Strict serial sum, tiler-reference/src/evaluate.rs:498-589 (strict_sum):
 * per output, a left fold seeded at the FIRST contributor in ascending
 * position; each add is apply_to_result(canon(op(acc) + op(c))); an empty
 * reduction commits +0.0; the committed value is canonicalized. */
int32_t tiler_oracle_strict_sum_f32(const float *x, uint64_t outer, uint64_t extent,
                                    uint64_t inner, float *out, int32_t input_mode,
                                    int32_t result_mode) {
    for (uint64_t o = 0; o < outer; ++o) {
        for (uint64_t i = 0; i < inner; ++i) {
            float acc = 0.0f;
            int seeded = 0;
            for (uint64_t p = 0; p < extent; ++p) {
                float c = x[(o * extent + p) * inner + i];
                if (!seeded) {
                    acc = c;
                    seeded = 1;
                } else {
                    acc = RSLT(canon(OPND(acc) + OPND(c)));
                }
            }
            out[o * inner + i] = canon(seeded ? acc : 0.0f);
        }
    }
    return TILER_ORACLE_OK;
}

/* evaluate.rs:612-776 strict_partial_sums_under: partition p folds the
 * contiguous range [p*c, (p+1)*c) strictly; exact coverage required; an empty
 * partition commits +0.0; a one-contributor partition commits it unchanged
 * (canonicalized). Layout: rows x extent, partials rows x partitions. */
int32_t tiler_oracle_strict_partial_sums_f32(const float *x, uint64_t rows, uint64_t extent,
                                             uint64_t partitions, uint64_t per_partition,
                                             float *partials, int32_t input_mode,
                                             int32_t result_mode) {
    if (partitions == 0) return TILER_ORACLE_INVALID_APPLICATION;
    if (per_partition != 0 && partitions > UINT64_MAX / per_partition)
        return TILER_ORACLE_INVALID_APPLICATION;
    if (partitions * per_partition != extent) return TILER_ORACLE_INVALID_APPLICATION;
    for (uint64_t r = 0; r < rows; ++r) {
        for (uint64_t p = 0; p < partitions; ++p) {
            float acc = 0.0f;
            int seeded = 0;
            for (uint64_t w = 0; w < per_partition; ++w) {
                float c = x[r * extent + p * per_partition + w];
                if (!seeded) {
                    acc = c;
                    seeded = 1;
                } else {
                    acc = RSLT(canon(OPND(acc) + OPND(c)));
                }
            }
            partials[r * partitions + p] = canon(seeded ? acc : 0.0f);
        }
    }
    return TILER_ORACLE_OK;
}

/* evaluate.rs:788-832 strict_partitioned_sum_under: the partials, then a
 * strict serial sum of the trailing partition axis under the same contract. */
int32_t tiler_oracle_strict_partitioned_sum_f32(const float *x, uint64_t rows, uint64_t extent,
                                                uint64_t partitions, uint64_t per_partition,
                                                float *out, int32_t input_mode,
                                                int32_t result_mode) {
    if (partitions == 0) return TILER_ORACLE_INVALID_APPLICATION;
    float *partials = (float *)malloc(sizeof(float) * (rows * partitions + 1));
    if (!partials) return TILER_ORACLE_INVALID_APPLICATION;
    int32_t st = tiler_oracle_strict_partial_sums_f32(x, rows, extent, partitions, per_partition,
                                                      partials, input_mode, result_mode);
    if (st == TILER_ORACLE_OK)
        st = tiler_oracle_strict_sum_f32(partials, rows, partitions, 1, out, input_mode,
                                         result_mode);
    free(partials);
    return st;
}

/* evaluate.rs:845-1158 cooperative_grouped_sum_under / fold_cooperative_sequence:
 * participant p of round r folds the contiguous range at cell index
 * (RoundMajor r*P+p, ParticipantMajor p*R+r) seeded at its first contributor;
 * the staged partials fold in ascending p; round totals in ascending r. */
int32_t tiler_oracle_cooperative_grouped_sum_f32(const float *x, uint64_t rows, uint64_t extent,
                                                 uint64_t participants, uint64_t per_partition,
                                                 uint64_t rounds, int32_t layout, float *out,
                                                 int32_t input_mode, int32_t result_mode) {
    if (participants == 0 || per_partition == 0 || rounds == 0)
        return TILER_ORACLE_INVALID_APPLICATION;
    if (participants > UINT64_MAX / per_partition) return TILER_ORACLE_INVALID_APPLICATION;
    uint64_t per_round = participants * per_partition;
    if (per_round > UINT64_MAX / rounds) return TILER_ORACLE_INVALID_APPLICATION;
    if (per_round * rounds != extent) return TILER_ORACLE_INVALID_APPLICATION;
    for (uint64_t row = 0; row < rows; ++row) {
        const float *seq = x + row * extent;
        float total = 0.0f;
        for (uint64_t r = 0; r < rounds; ++r) {
            float staged = 0.0f;
            for (uint64_t p = 0; p < participants; ++p) {
                uint64_t cell = layout == TILER_ORACLE_ROUND_MAJOR ? r * participants + p
                                                                    : p * rounds + r;
                const float *range = seq + cell * per_partition;
                float partial = range[0];
                for (uint64_t w = 1; w < per_partition; ++w)
                    partial = RSLT(canon(OPND(partial) + OPND(range[w])));
                staged = p == 0 ? partial : RSLT(canon(OPND(staged) + OPND(partial)));
            }
            total = r == 0 ? staged : RSLT(canon(OPND(total) + OPND(staged)));
        }
        out[row] = canon(total);
    }
    return TILER_ORACLE_OK;
}

/* ------------------------------------------------------------------------ */
/* Certified transcendentals.  The reference brackets the exact value with an
 * exact-rational enclosure and admits the f64-derived candidate (or one of its
 * neighbours) only if the bracket lies strictly inside that candidate's
 * round-to-nearest interval, refusing otherwise (silu.rs:573-662,
 * rms_norm.rs:219-293).  This restatement takes the enclosure from binary128
 * arithmetic: libquadmath expq/sqrtq are within a few binary128 ulps
 * (2^-112 relative), so a relative half-width of 2^-100 is a safe bracket. */
typedef __float128 q_t;
#define ENCLOSURE_SLACK 0x1p-100Q

static q_t q_of_f32(float v) { return (q_t)v; }

/* Strict midpoint test of silu.rs:639-656 / rms_norm.rs:202-224.  lo_zero
 * lets the exp variant treat 0 as its floor, as the reference does. */
static int rounds_to(q_t lower, q_t upper, float candidate, int lo_floor_zero) {
    if (!isfinite(candidate) || candidate < 0.0f) return 0;
    q_t value = q_of_f32(candidate);
    q_t lower_mid;
    if (candidate == 0.0f) {
        if (!lo_floor_zero) return 0;
        lower_mid = 0;
    } else {
        float prev = u2f(f2u(candidate) - 1u);
        lower_mid = (value + q_of_f32(prev)) / 2;
    }
    float next = candidate == 0.0f ? u2f(1u) : u2f(f2u(candidate) + 1u);
    if (!isfinite(next)) return 0;
    q_t upper_mid = (value + q_of_f32(next)) / 2;
    return lower > lower_mid && upper < upper_mid;
}

/* silu.rs:573-630 certified_exp_strict */
int32_t tiler_oracle_certified_exp_f32(float argument, float *out) {
    if (isnan(argument)) {
        *out = u2f(CANONICAL_F32_NAN_BITS);
        return TILER_ORACLE_OK;
    }
    if (argument >= 89.0f) { /* EXPONENTIAL_OVERFLOW_GUARD, silu.rs:424 */
        *out = INFINITY;
        return TILER_ORACLE_OK;
    }
    if (argument <= -104.0f) { /* EXPONENTIAL_UNDERFLOW_GUARD, silu.rs:427 */
        *out = 0.0f;
        return TILER_ORACLE_OK;
    }
    if (argument == 0.0f) {
        *out = 1.0f;
        return TILER_ORACLE_OK;
    }
    q_t e = expq(q_of_f32(argument));
    q_t lower = e * (1 - ENCLOSURE_SLACK), upper = e * (1 + ENCLOSURE_SLACK);
    /* round-to-nearest sends every reference at or above 2^128 - 2^103 to +inf */
    q_t overflow_threshold = 0x1p128Q - 0x1p103Q;
    if (lower >= overflow_threshold) {
        *out = INFINITY;
        return TILER_ORACLE_OK;
    }
    if (upper >= overflow_threshold) return TILER_ORACLE_UNDECIDED;
    float candidate = (float)exp((double)argument);
    if (!isfinite(candidate) || candidate < 0.0f) return TILER_ORACLE_UNDECIDED;
    if (rounds_to(lower, upper, candidate, 1)) {
        *out = candidate;
        return TILER_ORACLE_OK;
    }
    float prev = candidate == 0.0f ? -u2f(1u) : u2f(f2u(candidate) - 1u);
    float next = candidate == 0.0f ? u2f(1u) : u2f(f2u(candidate) + 1u);
    float neighbours[2] = {prev, next};
    for (int i = 0; i < 2; ++i) {
        float nb = neighbours[i];
        if (isfinite(nb) && nb >= 0.0f && rounds_to(lower, upper, nb, 1)) {
            *out = nb;
            return TILER_ORACLE_OK;
        }
    }
    return TILER_ORACLE_UNDECIDED;
}

/* rms_norm.rs:232-279 certified_rsqrt_strict */
int32_t tiler_oracle_certified_rsqrt_f32(float argument, float *out) {
    if (isnan(argument)) {
        *out = u2f(CANONICAL_F32_NAN_BITS);
        return TILER_ORACLE_OK;
    }
    if (argument == INFINITY) {
        *out = 0.0f;
        return TILER_ORACLE_OK;
    }
    if (argument == 0.0f) {
        *out = signbit(argument) ? -INFINITY : INFINITY;
        return TILER_ORACLE_OK;
    }
    if (argument < 0.0f) {
        *out = u2f(CANONICAL_F32_NAN_BITS);
        return TILER_ORACLE_OK;
    }
    q_t r = 1 / sqrtq(q_of_f32(argument));
    q_t lower = r * (1 - ENCLOSURE_SLACK), upper = r * (1 + ENCLOSURE_SLACK);
    float candidate = (float)(1.0 / sqrt((double)argument));
    if (!isfinite(candidate) || candidate <= 0.0f) return TILER_ORACLE_UNDECIDED;
    if (rounds_to(lower, upper, candidate, 0)) {
        *out = candidate;
        return TILER_ORACLE_OK;
    }
    float neighbours[2] = {u2f(f2u(candidate) - 1u), u2f(f2u(candidate) + 1u)};
    for (int i = 0; i < 2; ++i) {
        float nb = neighbours[i];
        if (isfinite(nb) && nb > 0.0f && rounds_to(lower, upper, nb, 0)) {
            *out = nb;
            return TILER_ORACLE_OK;
        }
    }
    return TILER_ORACLE_UNDECIDED;
}

static int32_t certified_exp_under(float argument, float *out, int32_t input_mode,
                                   int32_t result_mode) {
    float v;
    int32_t st = tiler_oracle_certified_exp_f32(OPND(argument), &v);
    if (st) return st;
    *out = RSLT(v);
    return TILER_ORACLE_OK;
}

/* silu.rs:511-533 silu_f32_under, then the registered evaluator's
 * canonicalization (silu.rs:454). */
int32_t tiler_oracle_silu_f32(const float *x, uint64_t n, float *y, int32_t input_mode,
                              int32_t result_mode) {
    for (uint64_t i = 0; i < n; ++i) {
        float a = x[i];
        float r;
        if (isnan(a)) {
            r = NAN;
        } else if (a == INFINITY) {
            r = INFINITY;
        } else if (a == -INFINITY) {
            r = NAN;
        } else {
            a = OPND(a);
            float e;
            int32_t st = certified_exp_under(-a, &e, input_mode, result_mode);
            if (st) return st;
            float divisor = RSLT(1.0f + OPND(e));
            r = RSLT(a / OPND(divisor));
        }
        y[i] = canon(r);
    }
    return TILER_ORACLE_OK;
}

/* ------------------------------------------------------------------------ */
/* Row geometry, evaluate.rs:1229-1280: rows = outer*inner, element
 * (row, position) at ((row/inner)*extent + position)*inner + row%inner. */
static inline uint64_t elem_index(uint64_t extent, uint64_t inner, uint64_t row,
                                  uint64_t position) {
    return ((row / inner) * extent + position) * inner + row % inner;
}

/* softmax.rs:237-315 softmax_dense / row_softmax: maximum fold from the first
 * contributor; e_i = certified_exp(fl(x_i - m)); d = strict fold from e_0;
 * y_i = canon(fl(e_i * fl(1/d))). */
int32_t tiler_oracle_softmax_f32(const float *x, uint64_t outer, uint64_t extent,
                                 uint64_t inner, float *y, int32_t input_mode,
                                 int32_t result_mode) {
    if (extent == 0) return TILER_ORACLE_OK;
    uint64_t rows = outer * inner;
    float *e = (float *)malloc(sizeof(float) * extent);
    if (!e) return TILER_ORACLE_INVALID_APPLICATION;
    for (uint64_t row = 0; row < rows; ++row) {
        float m = x[elem_index(extent, inner, row, 0)];
        for (uint64_t p = 1; p < extent; ++p)
            m = tiler_oracle_maximum_f32(m, x[elem_index(extent, inner, row, p)]);
        for (uint64_t p = 0; p < extent; ++p) {
            float shifted = RSLT(OPND(x[elem_index(extent, inner, row, p)]) - OPND(m));
            int32_t st = certified_exp_under(shifted, &e[p], input_mode, result_mode);
            if (st) {
                free(e);
                return st;
            }
        }
        float d = e[0];
        for (uint64_t p = 1; p < extent; ++p) d = RSLT(OPND(d) + OPND(e[p]));
        float r = RSLT(1.0f / OPND(d));
        for (uint64_t p = 0; p < extent; ++p)
            y[elem_index(extent, inner, row, p)] = canon(RSLT(OPND(e[p]) * OPND(r)));
    }
    free(e);
    return TILER_ORACLE_OK;
}

static int32_t certified_rsqrt_under(float argument, float *out, int32_t input_mode,
                                     int32_t result_mode) {
    float v;
    int32_t st = tiler_oracle_certified_rsqrt_f32(OPND(argument), &v);
    if (st) return st;
    *out = RSLT(v);
    return TILER_ORACLE_OK;
}

/* rms_norm.rs:134-195 row_scale and :453-489 normalize_dense:
 * s = rsqrt(fl(fl(sum of fl(x^2)) / N) + eps) with the sum a strict fold from
 * the first square and a DIVISION by N; y = canon(fl(w * fl(x * s))).
 * eps must be positive and finite (rms_norm.rs:462-466). */
int32_t tiler_oracle_rms_norm_f32(const float *x, const float *w, uint64_t outer,
                                  uint64_t extent, uint64_t inner, uint32_t eps_bits, float *y,
                                  int32_t input_mode, int32_t result_mode) {
    float eps = u2f(eps_bits);
    if (!(eps > 0.0f) || !isfinite(eps)) return TILER_ORACLE_INVALID_APPLICATION;
    uint64_t rows = outer * inner;
    for (uint64_t row = 0; row < rows; ++row) {
        float acc = 0.0f;
        int seeded = 0;
        for (uint64_t p = 0; p < extent; ++p) {
            float v = OPND(x[elem_index(extent, inner, row, p)]);
            float sq = RSLT(v * v);
            acc = seeded ? RSLT(OPND(acc) + OPND(sq)) : sq;
            seeded = 1;
        }
        float mean = extent == 0 ? acc : RSLT(OPND(acc) / OPND((float)extent));
        float s;
        int32_t st = certified_rsqrt_under(RSLT(OPND(mean) + OPND(eps)), &s, input_mode,
                                           result_mode);
        if (st) return st;
        for (uint64_t p = 0; p < extent; ++p) {
            uint64_t idx = elem_index(extent, inner, row, p);
            float normalized = RSLT(OPND(x[idx]) * OPND(s));
            y[idx] = canon(RSLT(OPND(w[idx]) * OPND(normalized)));
        }
    }
    return TILER_ORACLE_OK;
}

/* ------------------------------------------------------------------------ */
/* structural.rs:513-606 GatherF32Reference::evaluate with
 * tiler-ir/src/semantic/gather.rs:438-455 decide_gather_index: output laid out
 * [outer | index | inner]; each index selects a whole inner run cloned byte
 * for byte; an index >= extent (or, for a signed index type, < 0) refuses
 * naming the first offending position; never clamped or wrapped. */
int32_t tiler_oracle_gather(const void *source, uint64_t outer, uint64_t gathered,
                            uint64_t inner, uint32_t element_bytes, const uint32_t *index,
                            uint64_t index_count, int32_t index_signed, void *out,
                            uint64_t *bad_position, int64_t *bad_value) {
    for (uint64_t i = 0; i < index_count; ++i) {
        int64_t v = index_signed ? (int64_t)(int32_t)index[i] : (int64_t)index[i];
        if (v < 0 || (uint64_t)v >= gathered) {
            if (bad_position) *bad_position = i;
            if (bad_value) *bad_value = v;
            return TILER_ORACLE_GATHER_INDEX_OUT_OF_BOUNDS;
        }
    }
    const uint8_t *src = (const uint8_t *)source;
    uint8_t *dst = (uint8_t *)out;
    uint64_t run = inner * element_bytes;
    for (uint64_t o = 0; o < outer; ++o) {
        for (uint64_t i = 0; i < index_count; ++i) {
            uint64_t sel = index_signed ? (uint64_t)(int64_t)(int32_t)index[i] : index[i];
            memcpy(dst + (o * index_count + i) * run, src + (o * gathered + sel) * run, run);
        }
    }
    return TILER_ORACLE_OK;
}

/* ------------------------------------------------------------------------ */
/* quantization.rs:318-345 read_scale_value: the scale domain is
 * positive-normal-f32 (f32::is_normal and not negative), and :347-370
 * read_zero_point_value: a U4 code, 0..=15. */
int32_t tiler_oracle_strict_affine_domain(uint32_t scale_bits, uint8_t zero_point) {
    const float scale = u2f(scale_bits);
    if (fpclassify(scale) != FP_NORMAL || signbit(scale)) return 1;
    if (zero_point > 15) return 2;
    return 0;
}

/* quantization.rs:218-246 dequantize over a dense code tensor, each element
 * by :409-419 dequantize_one: the zero point's own code is +0.0; otherwise
 * the difference of the two codes, exact in binary32, times the scale (one
 * rounding).  The codes arrive packed as the schedule's ScalarProgram reads
 * them (model.rs:682-696: U4 LSB-first in U8 carriers, zero tail), the
 * nibble the Metal emitter extracts as (carrier >> ((i & 1) * 4)) & 0x0f
 * (tiler-metal/src/emit.rs:2047). */
int32_t tiler_oracle_dequantize_u4(const uint8_t *codes, uint64_t n, uint32_t scale_bits,
                                   uint8_t zero_point, float *out) {
    if (tiler_oracle_strict_affine_domain(scale_bits, zero_point) != 0) return TILER_ORACLE_INVALID_APPLICATION;
    const float scale = u2f(scale_bits);
    for (uint64_t i = 0; i < n; ++i) {
        const int32_t code = (codes[i / 2] >> ((i & 1) * 4)) & 0x0f;
        if (code == (int32_t)zero_point) {
            out[i] = 0.0f;
            continue;
        }
        const float difference = (float)(code - (int32_t)zero_point);
        out[i] = difference * scale;
    }
    return TILER_ORACLE_OK;
}

/* ------------------------------------------------------------------------ */
/* contraction.rs:558-630 ContractionFold::evaluate_outputs for td,od->to:
 * per output, p_d = fl(a*b) (no FMA), acc seeded at the FIRST product,
 * acc = fl(acc + p_d) over ascending d; canonical NaN.  Output slabs do not
 * change values (contraction.rs:661-698), so rows are split across threads.
 * B is transposed to [k, n] so the per-output chains run side by side across
 * n -- each chain keeps its own strict order. */
typedef struct {
    const float *a;
    const float *bt;
    uint64_t n, k;
    float *c;
    uint64_t row_begin, row_end;
} contract_job;

static void *contract_worker(void *arg) {
    contract_job *job = (contract_job *)arg;
    uint64_t n = job->n, k = job->k;
    float *acc = (float *)malloc(sizeof(float) * n);
    for (uint64_t i = job->row_begin; i < job->row_end; ++i) {
        const float *arow = job->a + i * k;
        {
            float a0 = arow[0];
            const float *brow = job->bt;
            for (uint64_t j = 0; j < n; ++j) acc[j] = a0 * brow[j];
        }
        for (uint64_t d = 1; d < k; ++d) {
            float ad = arow[d];
            const float *brow = job->bt + d * n;
            for (uint64_t j = 0; j < n; ++j) {
                float p = ad * brow[j];
                acc[j] = acc[j] + p;
            }
        }
        float *crow = job->c + i * n;
        for (uint64_t j = 0; j < n; ++j) crow[j] = canon(acc[j]);
    }
    free(acc);
    return NULL;
}

int32_t tiler_oracle_contract_strict_f32(const float *a, const float *b, uint64_t m, uint64_t n,
                                         uint64_t k, float *c, uint64_t row_begin,
                                         uint64_t row_end, uint32_t threads) {
    if (k == 0) return TILER_ORACLE_INVALID_APPLICATION; /* contraction.rs:420-428 */
    if (row_end > m || row_begin > row_end) return TILER_ORACLE_INVALID_APPLICATION;
    if (threads == 0) threads = 1;
    float *bt = (float *)malloc(sizeof(float) * n * k);
    if (!bt) return TILER_ORACLE_INVALID_APPLICATION;
    for (uint64_t j = 0; j < n; ++j)
        for (uint64_t d = 0; d < k; ++d) bt[d * n + j] = b[j * k + d];
    uint64_t rows = row_end - row_begin;
    if (threads > rows) threads = rows ? (uint32_t)rows : 1;
    pthread_t tid[256];
    contract_job jobs[256];
    if (threads > 256) threads = 256;
    for (uint32_t t = 0; t < threads; ++t) {
        jobs[t].a = a;
        jobs[t].bt = bt;
        jobs[t].n = n;
        jobs[t].k = k;
        jobs[t].c = c;
        jobs[t].row_begin = row_begin + rows * t / threads;
        jobs[t].row_end = row_begin + rows * (t + 1) / threads;
        pthread_create(&tid[t], NULL, contract_worker, &jobs[t]);
    }
    for (uint32_t t = 0; t < threads; ++t) pthread_join(tid[t], NULL);
    free(bt);
    return TILER_ORACLE_OK;
}

/* ------------------------------------------------------------------------ */
/* General contraction (see header). */
typedef struct {
    uint32_t dtype;
    int32_t silu;
    int32_t input_mode, result_mode;
    const void *left, *right;
    void *out;
    uint32_t out_rank, con_rank;
    uint64_t out_dims[8], con_dims[8];
    uint64_t l_out[8], r_out[8], l_con[8], r_con[8]; /* operand strides per output / contracted axis */
    uint64_t con_count, begin, end;
    int32_t status;
} general_job;

static float general_operand(const general_job *j, int right, uint64_t off) {
    if (j->dtype == 0) return ((const float *)(right ? j->right : j->left))[off];
    uint16_t h = ((const uint16_t *)(right ? j->right : j->left))[off];
    return u2f((uint32_t)h << 16);
}

static void *general_worker(void *arg) {
    general_job *j = (general_job *)arg;
    const int32_t input_mode = j->input_mode, result_mode = j->result_mode; /* OPND / RSLT */
    for (uint64_t o = j->begin; o < j->end; ++o) {
        /* the output coordinate, row-major (contraction.rs:580-585) */
        uint64_t lbase = 0, rbase = 0, rem = o;
        for (int32_t d = (int32_t)j->out_rank - 1; d >= 0; --d) {
            uint64_t c = rem % j->out_dims[d];
            rem /= j->out_dims[d];
            lbase += c * j->l_out[d];
            rbase += c * j->r_out[d];
        }
        uint64_t coord[8] = {0};
        uint64_t lo = 0, ro = 0;
        float acc = 0.0f;
        for (uint64_t step = 0; step < j->con_count; ++step) {
            /* contraction.rs:600-625: each factor as an operand, the product and
             * every accumulation as results, the accumulator as an operand */
            float p = RSLT(canon(OPND(general_operand(j, 0, lbase + lo)) * OPND(general_operand(j, 1, rbase + ro))));
            acc = step == 0 ? p : RSLT(canon(OPND(acc) + OPND(p))); /* contraction.rs:635-652 */
            /* next contracted coordinate, ascending lexicographic */
            for (int32_t d = (int32_t)j->con_rank - 1; d >= 0; --d) {
                lo += j->l_con[d];
                ro += j->r_con[d];
                if (++coord[d] < j->con_dims[d]) break;
                lo -= coord[d] * j->l_con[d];
                ro -= coord[d] * j->r_con[d];
                coord[d] = 0;
            }
        }
        acc = canon(acc);
        if (j->dtype == 0) {
            ((float *)j->out)[o] = acc;
        } else {
            float v = acc;
            if (j->silu && tiler_oracle_silu_f32(&acc, 1, &v, input_mode, result_mode) != TILER_ORACLE_OK) {
                j->status = TILER_ORACLE_UNDECIDED;
                return NULL;
            }
            ((uint16_t *)j->out)[o] = tiler_oracle_bf16_narrow(v);
        }
    }
    return NULL;
}

int32_t tiler_oracle_contract_general(uint32_t dtype, int32_t silu, uint32_t left_rank,
                                      const uint32_t *left_idx, const uint64_t *left_dims,
                                      uint32_t right_rank, const uint32_t *right_idx,
                                      const uint64_t *right_dims, uint32_t out_rank,
                                      const uint32_t *out_idx, const void *left, const void *right,
                                      void *out, uint32_t threads, int32_t input_mode,
                                      int32_t result_mode) {
    if (dtype > 1 || (dtype == 0 && silu)) return TILER_ORACLE_INVALID_APPLICATION;
    if (left_rank > 8 || right_rank > 8 || out_rank > 8) return TILER_ORACLE_INVALID_APPLICATION;
    const uint32_t rank[2] = {left_rank, right_rank};
    const uint32_t *idx[2] = {left_idx, right_idx};
    const uint64_t *dims[2] = {left_dims, right_dims};
    /* rule: an index repeats within no operand, nor within the output */
    for (int s = 0; s < 2; ++s)
        for (uint32_t a = 0; a < rank[s]; ++a)
            for (uint32_t b = a + 1; b < rank[s]; ++b)
                if (idx[s][a] == idx[s][b]) return TILER_ORACLE_INVALID_APPLICATION;
    for (uint32_t a = 0; a < out_rank; ++a)
        for (uint32_t b = a + 1; b < out_rank; ++b)
            if (out_idx[a] == out_idx[b]) return TILER_ORACLE_INVALID_APPLICATION;
    /* extent per index, agreeing everywhere (contraction.rs:386-399) */
    uint32_t labels[16];
    uint64_t extent[16];
    uint32_t nl = 0;
    for (int s = 0; s < 2; ++s)
        for (uint32_t a = 0; a < rank[s]; ++a) {
            uint32_t i = 0;
            while (i < nl && labels[i] != idx[s][a]) ++i;
            if (i == nl) {
                labels[nl] = idx[s][a];
                extent[nl++] = dims[s][a];
            } else if (extent[i] != dims[s][a]) {
                return TILER_ORACLE_INVALID_APPLICATION;
            }
        }
    /* every output index names an operand index */
    general_job base;
    memset(&base, 0, sizeof base);
    base.dtype = dtype;
    base.silu = silu;
    base.input_mode = input_mode;
    base.result_mode = result_mode;
    base.left = left;
    base.right = right;
    base.out = out;
    base.out_rank = out_rank;
    uint64_t outputs = 1;
    for (uint32_t d = 0; d < out_rank; ++d) {
        uint32_t i = 0;
        while (i < nl && labels[i] != out_idx[d]) ++i;
        if (i == nl) return TILER_ORACLE_INVALID_APPLICATION;
        base.out_dims[d] = extent[i];
        outputs *= extent[i];
    }
    /* the contracted set: operand indices absent from the output, ascending;
     * each must name an axis of both operands */
    uint32_t con[16];
    uint32_t nc = 0;
    for (uint32_t i = 0; i < nl; ++i) {
        int in_out = 0;
        for (uint32_t d = 0; d < out_rank; ++d) in_out |= out_idx[d] == labels[i];
        if (in_out) continue;
        int in[2] = {0, 0};
        for (int s = 0; s < 2; ++s)
            for (uint32_t a = 0; a < rank[s]; ++a) in[s] |= idx[s][a] == labels[i];
        if (!in[0] || !in[1]) return TILER_ORACLE_INVALID_APPLICATION;
        uint32_t at = nc++;
        while (at > 0 && con[at - 1] > labels[i]) {
            con[at] = con[at - 1];
            --at;
        }
        con[at] = labels[i];
    }
    if (nc == 0 || nc > 8) return TILER_ORACLE_INVALID_APPLICATION;
    base.con_rank = nc;
    base.con_count = 1;
    for (uint32_t c = 0; c < nc; ++c) {
        uint32_t i = 0;
        while (labels[i] != con[c]) ++i;
        base.con_dims[c] = extent[i];
        base.con_count *= extent[i];
    }
    /* contraction.rs:420-428: an empty contracted domain has no result */
    if (base.con_count == 0) return TILER_ORACLE_INVALID_APPLICATION;
    /* per operand axis: the stride it contributes to an output or contracted axis */
    for (int s = 0; s < 2; ++s) {
        uint64_t stride = 1;
        for (int32_t a = (int32_t)rank[s] - 1; a >= 0; --a) {
            for (uint32_t d = 0; d < out_rank; ++d)
                if (out_idx[d] == idx[s][a]) (s ? base.r_out : base.l_out)[d] = stride;
            for (uint32_t c = 0; c < nc; ++c)
                if (con[c] == idx[s][a]) (s ? base.r_con : base.l_con)[c] = stride;
            stride *= dims[s][a];
        }
    }
    if (threads == 0) threads = 1;
    if (threads > 64) threads = 64;
    if (threads > outputs) threads = outputs ? (uint32_t)outputs : 1;
    pthread_t tid[64];
    general_job jobs[64];
    for (uint32_t t = 0; t < threads; ++t) {
        jobs[t] = base;
        jobs[t].begin = outputs * t / threads;
        jobs[t].end = outputs * (t + 1) / threads;
        pthread_create(&tid[t], NULL, general_worker, &jobs[t]);
    }
    int32_t st = TILER_ORACLE_OK;
    for (uint32_t t = 0; t < threads; ++t) {
        pthread_join(tid[t], NULL);
        if (jobs[t].status) st = jobs[t].status;
    }
    return st;
}

/* ------------------------------------------------------------------------ */
/* Declared groupings of the tiler-hip reassociating kernels (see header). */

/* One row under grouping (vec, waves): returns the committed sum. */
static float row_grouped_fold(const float *c, uint64_t extent, uint32_t vec, uint32_t waves) {
    if (extent == 0) return 0.0f;
    uint32_t threads = 64u * waves;
    float *part = (float *)malloc(sizeof(float) * threads);
    for (uint32_t t = 0; t < threads; ++t) part[t] = -0.0f;
    uint64_t stride = (uint64_t)threads * vec;
    for (uint64_t base = 0; base < extent; base += stride)
        for (uint32_t t = 0; t < threads; ++t)
            for (uint32_t e = 0; e < vec; ++e) {
                uint64_t p = base + (uint64_t)t * vec + e;
                if (p < extent) part[t] = part[t] + c[p];
            }
    float total = 0.0f;
    float v[64], nv[64];
    for (uint32_t w = 0; w < waves; ++w) {
        for (int l = 0; l < 64; ++l) v[l] = part[w * 64 + l];
        for (int o = 32; o >= 1; o >>= 1) {
            for (int l = 0; l < 64; ++l) nv[l] = v[l] + v[l ^ o];
            memcpy(v, nv, sizeof(v));
        }
        total = w == 0 ? v[0] : total + v[0];
    }
    free(part);
    return total;
}

int32_t tiler_oracle_row_grouped_sum_f32(const float *contributors, uint64_t rows,
                                         uint64_t extent, uint32_t vec, uint32_t waves,
                                         float *out) {
    if (vec == 0 || waves == 0 || waves > 16) return TILER_ORACLE_INVALID_APPLICATION;
    for (uint64_t r = 0; r < rows; ++r)
        out[r] = canon(row_grouped_fold(contributors + r * extent, extent, vec, waves));
    return TILER_ORACLE_OK;
}

/* In-block reduction of 256 thread partials: per-wave butterfly, then the
 * four wave results in ascending order. */
static float block_reduce256(const float *part) {
    float total = 0.0f, v[64], nv[64];
    for (int w = 0; w < 4; ++w) {
        for (int l = 0; l < 64; ++l) v[l] = part[w * 64 + l];
        for (int o = 32; o >= 1; o >>= 1) {
            for (int l = 0; l < 64; ++l) nv[l] = v[l] + v[l ^ o];
            memcpy(v, nv, sizeof(v));
        }
        total = w == 0 ? v[0] : total + v[0];
    }
    return total;
}

int32_t tiler_oracle_grid_tree_sum_f32(const float *x, uint64_t n, uint32_t blocks, float *out) {
    if (blocks == 0) return TILER_ORACLE_INVALID_APPLICATION;
    if (n == 0) {
        *out = 0.0f;
        return TILER_ORACLE_OK;
    }
    uint64_t tiles = (n + 1023) / 1024;
    float *partials = (float *)malloc(sizeof(float) * blocks);
    float part[256];
    for (uint32_t b = 0; b < blocks; ++b) {
        for (int t = 0; t < 256; ++t) part[t] = -0.0f;
        for (uint64_t tile = b; tile < tiles; tile += blocks)
            for (int t = 0; t < 256; ++t)
                for (int e = 0; e < 4; ++e) {
                    uint64_t p = tile * 1024 + (uint64_t)t * 4 + e;
                    if (p < n) part[t] = part[t] + x[p];
                }
        partials[b] = block_reduce256(part);
    }
    for (int t = 0; t < 256; ++t) {
        part[t] = -0.0f;
        for (uint64_t i = (uint64_t)t; i < blocks; i += 256) part[t] = part[t] + partials[i];
    }
    *out = canon(block_reduce256(part));
    free(partials);
    return TILER_ORACLE_OK;
}

int32_t tiler_oracle_rms_norm_grouped_f32(const float *x, const float *w, uint64_t rows,
                                          uint64_t extent, uint32_t eps_bits,
                                          int32_t weight_broadcast, uint32_t vec,
                                          uint32_t waves, float *y) {
    float eps = u2f(eps_bits);
    if (!(eps > 0.0f) || !isfinite(eps)) return TILER_ORACLE_INVALID_APPLICATION;
    if (vec == 0 || waves == 0 || waves > 16) return TILER_ORACLE_INVALID_APPLICATION;
    if (extent == 0) return TILER_ORACLE_OK;
    float *sq = (float *)malloc(sizeof(float) * extent);
    for (uint64_t r = 0; r < rows; ++r) {
        const float *xr = x + r * extent;
        const float *wr = weight_broadcast ? w : w + r * extent;
        for (uint64_t p = 0; p < extent; ++p) sq[p] = xr[p] * xr[p];
        float total = row_grouped_fold(sq, extent, vec, waves);
        float mean = total / (float)extent;
        float s;
        int32_t st = tiler_oracle_certified_rsqrt_f32(mean + eps, &s);
        if (st) {
            free(sq);
            return st;
        }
        for (uint64_t p = 0; p < extent; ++p) {
            float normalized = xr[p] * s;
            y[r * extent + p] = canon(wr[p] * normalized);
        }
    }
    free(sq);
    return TILER_ORACLE_OK;
}

/* Softmax with a segmented exponent sum: the row's exponents are cut into
 * segments of `segment` elements (0: one segment, the whole row); each
 * segment's partial is the (vec, waves) grouped fold of its elements and the
 * row total is the left fold of the partials in ascending segment order,
 * seeded by the first.  The shift, the exponent and the final scaling are
 * softmax.rs:237-315's: m = the governed maximum of the row, e = exp(x - m)
 * certified, y = canon(e * (1 / d)). */
int32_t tiler_oracle_softmax_segmented_f32(const float *x, uint64_t rows, uint64_t extent,
                                           uint64_t segment, uint32_t vec, uint32_t waves,
                                           float *y) {
    if (vec == 0 || waves == 0 || waves > 16) return TILER_ORACLE_INVALID_APPLICATION;
    if (extent == 0) return TILER_ORACLE_OK;
    if (segment == 0 || segment > extent) segment = extent;
    float *e = (float *)malloc(sizeof(float) * extent);
    for (uint64_t r = 0; r < rows; ++r) {
        const float *xr = x + r * extent;
        float m = xr[0];
        for (uint64_t p = 1; p < extent; ++p) m = tiler_oracle_maximum_f32(m, xr[p]);
        for (uint64_t p = 0; p < extent; ++p) {
            int32_t st = tiler_oracle_certified_exp_f32(xr[p] - m, &e[p]);
            if (st) {
                free(e);
                return st;
            }
        }
        float d = 0.0f;
        for (uint64_t s0 = 0; s0 < extent; s0 += segment) {
            uint64_t len = extent - s0 < segment ? extent - s0 : segment;
            float part = row_grouped_fold(e + s0, len, vec, waves);
            d = s0 == 0 ? part : d + part;
        }
        float rcp = 1.0f / d;
        for (uint64_t p = 0; p < extent; ++p) y[r * extent + p] = canon(e[p] * rcp);
    }
    free(e);
    return TILER_ORACLE_OK;
}

int32_t tiler_oracle_softmax_grouped_f32(const float *x, uint64_t rows, uint64_t extent,
                                         uint32_t vec, uint32_t waves, float *y) {
    return tiler_oracle_softmax_segmented_f32(x, rows, extent, 0, vec, waves, y);
}

/* ------------------------------------------------------------------------ */
/* Pointwise expression DAGs (tiler-ir/src/schedule/pointwise.rs:74-140 and
 * pointwise_bf16.rs:114-168; the per-node statements of tiler-metal's
 * pointwise goldens): nodes in topological order, evaluated per element.
 * f32 nodes: ADD/MULTIPLY/DIVIDE one IEEE rounding (-ffp-contract=off),
 * EXP and RSQRT the certified values (silu.rs:573-662, rms_norm.rs:219-293),
 * operand and result subnormal modes (conformance.rs:498-521), then the
 * canonical NaN.  Opcodes: 0 input (a = ordinal), 1 constant (a = bits),
 * 2 add, 3 multiply, 4 divide (a, b), 5 exp, 6 rsqrt (a).  Status 1 for a
 * malformed DAG (operand after its use, bad opcode). */
int32_t tiler_oracle_expression_f32(const uint32_t *ops, const uint32_t *as, const uint32_t *bs,
                                    uint32_t count, uint32_t root, const float *const *inputs,
                                    uint64_t n, float *y, int32_t input_mode, int32_t result_mode) {
    if (count == 0 || root >= count) return TILER_ORACLE_INVALID_APPLICATION;
    for (uint32_t i = 0; i < count; ++i) {
        if (ops[i] > 6) return TILER_ORACLE_INVALID_APPLICATION;
        if (ops[i] >= 2 && (as[i] >= i || (ops[i] <= 4 && bs[i] >= i)))
            return TILER_ORACLE_INVALID_APPLICATION;
    }
    float *v = (float *)malloc(sizeof(float) * count);
    if (!v) return TILER_ORACLE_INVALID_APPLICATION;
    for (uint64_t e = 0; e < n; ++e) {
        for (uint32_t i = 0; i < count; ++i) {
            float r;
            int32_t st = TILER_ORACLE_OK;
            switch (ops[i]) {
                case 0: r = inputs[as[i]][e]; break;
                case 1: r = u2f(as[i]); break;
                case 2: r = canon(RSLT(OPND(v[as[i]]) + OPND(v[bs[i]]))); break;
                case 3: r = canon(RSLT(OPND(v[as[i]]) * OPND(v[bs[i]]))); break;
                case 4: r = canon(RSLT(OPND(v[as[i]]) / OPND(v[bs[i]]))); break;
                case 5: {
                    float a = OPND(v[as[i]]);
                    st = isnan(a) ? (r = a, TILER_ORACLE_OK) : tiler_oracle_certified_exp_f32(a, &r);
                    r = canon(RSLT(r));
                    break;
                }
                default: {
                    float a = OPND(v[as[i]]);
                    st = tiler_oracle_certified_rsqrt_f32(a, &r);
                    r = canon(RSLT(r));
                    break;
                }
            }
            if (st) {
                free(v);
                return st;
            }
            v[i] = r;
        }
        y[e] = v[root];
    }
    free(v);
    return TILER_ORACLE_OK;
}

/* ADR 0091 narrowing of an exact binary128 value to bf16: round to nearest
 * even at the bf16 quantum of the value's binade (2^-133 below 2^-126),
 * overflow to infinity at the inclusive midpoint above the largest finite
 * bf16, signed zero kept.  The quantum scaling is exact in binary128. */
static uint16_t bf16_of_q(q_t q) {
    if (isnanq(q)) return CANONICAL_BF16_NAN_BITS;
    const uint16_t sign = signbitq(q) ? 0x8000u : 0;
    q_t a = fabsq(q);
    if (a == 0) return sign;
    int e;
    frexpq(a, &e); /* a in [2^(e-1), 2^e) */
    int ex = e - 1;
    if (ex < -126) ex = -126;
    const q_t quantum = ldexpq(1.0Q, ex - 7);
    q_t m = rintq(a / quantum); /* default rounding: to nearest, ties to even */
    q_t r = m * quantum;
    if (r >= ldexpq(1.0Q, 128)) return sign | 0x7f80u;
    float f = (float)r; /* exact: r is a bf16 value */
    return sign | (uint16_t)(f2u(f) >> 16);
}

/* bf16 expressions (pointwise_bf16.rs: INPUT, CONSTANT, ADD, MULTIPLY; each
 * node one rounding of the exact result to bf16, canonical NaN 0x7fc0;
 * bf16.rs:238-787 exact_add / exact_multiply then the ADR 0091 rounding).
 * The exact sum and product of two bf16 values are formed in binary128:
 * products are exact (16 significant bits); a sum is exact unless the
 * operands' exponents differ by more than ~104, and then the smaller lies
 * far below half a bf16 quantum of the larger and binary128 keeps it as a
 * sticky nonzero remainder, which is all the rounding reads. */
/* bf16.rs:517-533 under a Bf16SubnormalRealization: accept_operand replaces a
 * subnormal operand ENCODING by the input mode before it is decoded, commit
 * replaces a subnormal ROUNDED result by the result mode.  A bf16 encoding is
 * subnormal when its exponent field is zero and its significand is not. */
static uint16_t bf16_subnormal_mode(int32_t mode, uint16_t bits) {
    if (mode == TILER_ORACLE_PRESERVE) return bits;
    if ((bits & 0x7f80u) != 0 || (bits & 0x007fu) == 0) return bits;
    return mode == TILER_ORACLE_FLUSH_SIGN_PRESERVING ? (uint16_t)(bits & 0x8000u) : 0;
}

int32_t tiler_oracle_expression_bf16(const uint32_t *ops, const uint32_t *as, const uint32_t *bs,
                                     uint32_t count, uint32_t root, const uint16_t *const *inputs,
                                     uint64_t n, uint16_t *y, int32_t input_mode, int32_t result_mode) {
    if (count == 0 || root >= count) return TILER_ORACLE_INVALID_APPLICATION;
    for (uint32_t i = 0; i < count; ++i) {
        if (ops[i] > 3) return TILER_ORACLE_INVALID_APPLICATION;
        if (ops[i] >= 2 && (as[i] >= i || bs[i] >= i)) return TILER_ORACLE_INVALID_APPLICATION;
        if (ops[i] == 1 && as[i] > 0xffffu) return TILER_ORACLE_INVALID_APPLICATION;
    }
    uint16_t *v = (uint16_t *)malloc(sizeof(uint16_t) * count);
    if (!v) return TILER_ORACLE_INVALID_APPLICATION;
    for (uint64_t e = 0; e < n; ++e) {
        for (uint32_t i = 0; i < count; ++i) {
            switch (ops[i]) {
                case 0: v[i] = inputs[as[i]][e]; break;
                case 1: v[i] = (uint16_t)as[i]; break;
                default: {
                    const q_t x = (q_t)tiler_oracle_bf16_widen(bf16_subnormal_mode(input_mode, v[as[i]]));
                    const q_t z = (q_t)tiler_oracle_bf16_widen(bf16_subnormal_mode(input_mode, v[bs[i]]));
                    v[i] = bf16_subnormal_mode(result_mode, bf16_of_q(ops[i] == 2 ? x + z : x * z));
                }
            }
        }
        y[e] = v[root];
    }
    free(v);
    return TILER_ORACLE_OK;
}

uint16_t tiler_oracle_bf16_exact_add(uint16_t x, uint16_t z) {
    return bf16_of_q((q_t)tiler_oracle_bf16_widen(x) + (q_t)tiler_oracle_bf16_widen(z));
}
uint16_t tiler_oracle_bf16_exact_multiply(uint16_t x, uint16_t z) {
    return bf16_of_q((q_t)tiler_oracle_bf16_widen(x) * (q_t)tiler_oracle_bf16_widen(z));
}

/* ------------------------------------------------------------------------ */
/* evaluate.rs:498-589 strict_sum over any axis set, with the prologues and the
 * maximum combiner of tiler-ir/src/kernel/lower.rs:1236-1305, 2485-2500:
 * survivors in axis order give the output layout; each output folds its
 * contributors in lexicographic order of the reduced coordinates, seeded at
 * the first (transformed) contributor.  op 0 sum, 1 squared (canon(x*x)),
 * 2 scale-bias (canon(canon(x*s) + b)), 3 maximum (NaN-propagating, -0 < +0).
 * An empty sum commits +0; an empty maximum is refused (model.rs:880-906).
 * The result is canonicalized. */
int32_t tiler_oracle_fold_f32(const float *x, uint32_t rank, const uint64_t *dims,
                              uint64_t reduced_mask, uint32_t op, uint32_t scale_bits,
                              uint32_t bias_bits, float *out, int32_t input_mode,
                              int32_t result_mode) {
    if (rank > 8 || op > 3 || (reduced_mask >> rank)) return TILER_ORACLE_INVALID_APPLICATION;
    uint64_t stride[8], kept[8], red[8], kept_n = 0, red_n = 0, outputs = 1, contributors = 1;
    uint64_t total = 1;
    for (int d = (int)rank - 1; d >= 0; --d) {
        stride[d] = total;
        total *= dims[d];
    }
    for (uint32_t d = 0; d < rank; ++d) {
        if (reduced_mask >> d & 1) {
            red[red_n++] = d;
            contributors *= dims[d];
        } else {
            kept[kept_n++] = d;
            outputs *= dims[d];
        }
    }
    if (outputs && contributors == 0 && op == 3) return TILER_ORACLE_INVALID_APPLICATION;
    const float s = u2f(scale_bits), b = u2f(bias_bits);
    for (uint64_t o = 0; o < outputs; ++o) {
        uint64_t base = 0, rem = o;
        for (int k = (int)kept_n - 1; k >= 0; --k) {
            base += (rem % dims[kept[k]]) * stride[kept[k]];
            rem /= dims[kept[k]];
        }
        float acc = 0.0f;
        for (uint64_t c = 0; c < contributors; ++c) {
            uint64_t off = base, r2 = c;
            for (int k = (int)red_n - 1; k >= 0; --k) {
                off += (r2 % dims[red[k]]) * stride[red[k]];
                r2 /= dims[red[k]];
            }
            float v = x[off], t;
            switch (op) {
                case 1: t = canon(RSLT(OPND(v) * OPND(v))); break;
                case 2: t = canon(RSLT(OPND(canon(RSLT(OPND(v) * OPND(s)))) + OPND(b))); break;
                default: t = v;
            }
            if (c == 0) acc = t;
            else if (op == 3) acc = canon(tiler_oracle_maximum_f32(acc, t));
            else acc = canon(RSLT(OPND(acc) + OPND(t)));
        }
        out[o] = contributors == 0 ? 0.0f : canon(acc);
    }
    return TILER_ORACLE_OK;
}
