/*
 * tiler_oracle.h -- CPU restatement of tiler-reference for the tiler-hip hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker: it may be
 * linked or called only from tests/, from __graft_entry__.smoke() and from
 * bench.py's cpu_baseline leg.  The product (libtiler_hip.so and the
 * tiler_amd package) never calls it.
 *
 * Every function restates one reference function; the citation beside each
 * names the file:line it follows (paths relative to
 * /root/reference/crates/).  The reference is Rust and cannot be built in
 * this image, so nothing here links it; the restatement is pinned instead by
 * the reference's own golden vectors (tests/golden/) and by mathematical
 * checks (exact integer/decimal arithmetic, closed forms, brute force).
 *
 * Status codes: 0 ok, 1 invalid application, 2 undecided transcendental
 * reference, 3 gather index out of bounds, 4 iteration limit.
 */
#ifndef TILER_ORACLE_H
#define TILER_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    TILER_ORACLE_OK = 0,
    TILER_ORACLE_INVALID_APPLICATION = 1,
    TILER_ORACLE_UNDECIDED = 2,
    TILER_ORACLE_GATHER_INDEX_OUT_OF_BOUNDS = 3,
    TILER_ORACLE_ITERATION_LIMIT = 4
};

/* Subnormal modes, tiler-reference/src/conformance.rs:498-521. */
enum {
    TILER_ORACLE_PRESERVE = 0,
    TILER_ORACLE_FLUSH_SIGN_PRESERVING = 1,
    TILER_ORACLE_FLUSH_POSITIVE_ZERO = 2
};

/* Cell layouts, tiler-reference/src/evaluate.rs:395-421. */
enum { TILER_ORACLE_ROUND_MAJOR = 0, TILER_ORACLE_PARTICIPANT_MAJOR = 1 };

uint32_t tiler_oracle_canonical_nan_bits(void);
float tiler_oracle_apply_subnormal_mode(int32_t mode, float value);
float tiler_oracle_maximum_f32(float left, float right);

/* bf16 <-> f32, ADR 0091 decision 2 (narrowing RNE, NaN -> 0x7fc0). */
uint16_t tiler_oracle_bf16_narrow(float value);
float tiler_oracle_bf16_widen(uint16_t bits);
void tiler_oracle_bf16_narrow_array(const float *in, uint64_t n, uint16_t *out);
void tiler_oracle_bf16_widen_array(const uint16_t *in, uint64_t n, float *out);

/* Reductions over the single axis of a (outer, extent, inner) geometry. */
int32_t tiler_oracle_strict_sum_f32(const float *x, uint64_t outer, uint64_t extent,
                                    uint64_t inner, float *out, int32_t input_mode,
                                    int32_t result_mode);
int32_t tiler_oracle_strict_partial_sums_f32(const float *x, uint64_t rows, uint64_t extent,
                                             uint64_t partitions, uint64_t per_partition,
                                             float *partials, int32_t input_mode,
                                             int32_t result_mode);
int32_t tiler_oracle_strict_partitioned_sum_f32(const float *x, uint64_t rows, uint64_t extent,
                                                uint64_t partitions, uint64_t per_partition,
                                                float *out, int32_t input_mode,
                                                int32_t result_mode);
int32_t tiler_oracle_cooperative_grouped_sum_f32(const float *x, uint64_t rows, uint64_t extent,
                                                 uint64_t participants, uint64_t per_partition,
                                                 uint64_t rounds, int32_t layout, float *out,
                                                 int32_t input_mode, int32_t result_mode);

/* Certified transcendental steps. */
int32_t tiler_oracle_certified_exp_f32(float argument, float *out);
int32_t tiler_oracle_certified_rsqrt_f32(float argument, float *out);
int32_t tiler_oracle_silu_f32(const float *x, uint64_t n, float *y, int32_t input_mode,
                              int32_t result_mode);

/* Row families over a (outer, extent, inner) geometry. */
int32_t tiler_oracle_softmax_f32(const float *x, uint64_t outer, uint64_t extent,
                                 uint64_t inner, float *y, int32_t input_mode,
                                 int32_t result_mode);
int32_t tiler_oracle_rms_norm_f32(const float *x, const float *w, uint64_t outer,
                                  uint64_t extent, uint64_t inner, uint32_t eps_bits, float *y,
                                  int32_t input_mode, int32_t result_mode);

/* Gather: output [outer, index_count, inner]; byte moves only. */
int32_t tiler_oracle_gather(const void *source, uint64_t outer, uint64_t gathered,
                            uint64_t inner, uint32_t element_bytes, const uint32_t *index,
                            uint64_t index_count, int32_t index_signed, void *out,
                            uint64_t *bad_position, int64_t *bad_value);

/* Strict contraction td,od->to: C[m,n] = sum_k A[m,k]*B[n,k]; rows
 * [row_begin,row_end) of C are written (C is indexed from row 0). */
int32_t tiler_oracle_contract_strict_f32(const float *a, const float *b, uint64_t m, uint64_t n,
                                         uint64_t k, float *c, uint64_t row_begin,
                                         uint64_t row_end, uint32_t threads);

/* Contraction over a general binary index structure (ADR 0087):
 * tiler-reference/src/contraction.rs:346-715 (ContractionFold::plan and
 * evaluate_outputs) under a conformance: the modes at the factors, the
 * product and every accumulation (contraction.rs:600-625).  Each operand is dense
 * row-major with `*_rank` axes labelled by `*_idx` (any uint32 labels) and
 * sized by `*_dims`; the output is dense row-major over `out_idx`.  The five
 * structural rules (tiler-ir/src/semantic/contraction.rs:804-900) and extent
 * agreement are checked; the contracted set is every operand index absent
 * from the output, ascending by label, and its row-major odometer is the
 * contributor sequence: seeded at the first product, fl(a*b) and
 * fl(acc + p) each canonicalized, no FMA.  dtype 0: f32 operands and
 * result; dtype 1: bf16 operands widened exactly, the same f32 fold, then
 * (silu != 0) the reference SiLU and one bf16 narrowing. */
int32_t tiler_oracle_contract_general(uint32_t dtype, int32_t silu, uint32_t left_rank,
                                      const uint32_t *left_idx, const uint64_t *left_dims,
                                      uint32_t right_rank, const uint32_t *right_idx,
                                      const uint64_t *right_dims, uint32_t out_rank,
                                      const uint32_t *out_idx, const void *left, const void *right,
                                      void *out, uint32_t threads, int32_t input_mode,
                                      int32_t result_mode);

/* ---- Declared groupings of the tiler-hip reassociating kernels ----------
 * These restate the exact addition order each HIP kernel performs, so the
 * device result can be compared bit for bit; they are the analogue of
 * strict_partitioned_sum for a grouping the reference has no name for.
 *
 * Row grouping (vec, waves): element p of a row is held by thread
 * t = (p / vec) % (64*waves) and folded in ascending p by that thread, seeded
 * at -0.0 (the exact additive identity); each wave combines its 64 lane
 * partials by an xor butterfly over offsets 32,16,8,4,2,1 (v[l] += v[l^o]);
 * the waves' results are then folded in ascending wave order. */
int32_t tiler_oracle_row_grouped_sum_f32(const float *contributors, uint64_t rows,
                                         uint64_t extent, uint32_t vec, uint32_t waves,
                                         float *out);
/* Grid grouping of the single-output sum kernel: tile = 1024 elements
 * (256 threads x float4); block b folds tiles b, b+blocks, ... per thread in
 * ascending (tile, component) order; each block reduces its 256 thread
 * partials by the row grouping (vec 1 within a 4-wave block); the last block
 * folds the block partials with thread t taking partials t, t+256, ... and the
 * same in-block reduction. */
int32_t tiler_oracle_grid_tree_sum_f32(const float *x, uint64_t n, uint32_t blocks, float *out);
int32_t tiler_oracle_rms_norm_grouped_f32(const float *x, const float *w, uint64_t rows,
                                          uint64_t extent, uint32_t eps_bits,
                                          int32_t weight_broadcast, uint32_t vec,
                                          uint32_t waves, float *y);
int32_t tiler_oracle_softmax_grouped_f32(const float *x, uint64_t rows, uint64_t extent,
                                         uint32_t vec, uint32_t waves, float *y);
/* The same with the exponent sum folded by segments of `segment` elements
 * (0: the whole row), partials left-folded in ascending segment order. */
int32_t tiler_oracle_softmax_segmented_f32(const float *x, uint64_t rows, uint64_t extent,
                                           uint64_t segment, uint32_t vec, uint32_t waves,
                                           float *y);

/* Pointwise expression DAGs (tiler-ir/src/schedule/pointwise.rs:74-140,
 * pointwise_bf16.rs:114-168): nodes in topological order, opcodes 0 input
 * (a = ordinal), 1 constant (a = bits), 2 add, 3 multiply, 4 divide (a, b),
 * 5 exp, 6 rsqrt (a); y[e] = the root's value at element e.  bf16: opcodes
 * 0-3, each node rounded once from its exact value (binary128) to bf16. */
int32_t tiler_oracle_expression_f32(const uint32_t *ops, const uint32_t *as, const uint32_t *bs,
                                    uint32_t count, uint32_t root, const float *const *inputs,
                                    uint64_t n, float *y, int32_t input_mode, int32_t result_mode);
int32_t tiler_oracle_expression_bf16(const uint32_t *ops, const uint32_t *as, const uint32_t *bs,
                                     uint32_t count, uint32_t root, const uint16_t *const *inputs,
                                     uint64_t n, uint16_t *y, int32_t input_mode, int32_t result_mode);
uint16_t tiler_oracle_bf16_exact_add(uint16_t x, uint16_t z);
uint16_t tiler_oracle_bf16_exact_multiply(uint16_t x, uint16_t z);

/* The strict serial fold over any axis set of a dense row-major tensor:
 * op 0 sum, 1 squared, 2 scale-bias (scale_bits, bias_bits), 3 maximum. */
int32_t tiler_oracle_fold_f32(const float *x, uint32_t rank, const uint64_t *dims,
                              uint64_t reduced_mask, uint32_t op, uint32_t scale_bits,
                              uint32_t bias_bits, float *out, int32_t input_mode,
                              int32_t result_mode);

/* Audit of the device's binary32 exp (device_exp_audit.c): the device
 * algorithm restated bit for bit, and an exhaustive scan of every binary32
 * input in (-104, 89).  Inputs whose binary64 value lies within
 * 2^margin_log2 (relative) of a binary32 rounding boundary are collected in
 * `hard` (up to hard_cap) and compared with tiler_oracle_certified_exp_f32;
 * every other input is correctly rounded by the error bound stated in that
 * file.  planted_log2 != 0 perturbs every value by (1 + 2^planted_log2)
 * before rounding (a planted mistake for the audit's own test). */
float tiler_oracle_device_exp_f32(float s);
int32_t tiler_oracle_audit_device_exp(int32_t margin_log2, int32_t planted_log2,
                                      uint32_t threads, float *hard,
                                      uint64_t hard_cap, uint64_t *hard_count,
                                      uint64_t *checked, uint64_t *mismatches,
                                      float *first_mismatch);

/* Strict per-tensor affine U4 -> f32 dequantization
 * (tiler-reference/src/quantization.rs:218-246 dequantize, :409-419
 * dequantize_one; codes packed U4 LSB-first with a zero tail,
 * tiler-ir/src/schedule/model.rs:682-696).  Element i is nibble i % 2 (low
 * first) of byte i / 2.  scale must be a positive normal binary32
 * (quantization.rs:318-345) and the zero point lie in 0..=15 (:347-370), else
 * TILER_ORACLE_INVALID_APPLICATION with nothing written.  A code equal to the
 * zero point decodes to +0.0; any other to fl((code - zero_point) * scale). */
int32_t tiler_oracle_dequantize_u4(const uint8_t *codes, uint64_t n, uint32_t scale_bits,
                                   uint8_t zero_point, float *out);
/* The same domain rules alone: 0 ok, 1 scale, 2 zero point. */
int32_t tiler_oracle_strict_affine_domain(uint32_t scale_bits, uint8_t zero_point);

#ifdef __cplusplus
}
#endif

#endif
