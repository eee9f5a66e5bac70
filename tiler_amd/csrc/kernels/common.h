// Shared device helpers for the tiler-hip gfx950 kernels.
//
// Every kernel in this library is compiled with -ffp-contract=off: a written
// multiply followed by an add is two IEEE roundings, which is the arithmetic
// the reference pins (tiler-reference/src/contraction.rs:612-624 "no FMA",
// rms_norm.rs:155-162 "one rounding per square, then one per combine").
// Fused multiply-adds appear only where written as __builtin_fma/__builtin_fmaf
// (the exponential's range reduction and polynomial, which are internal to a
// correctly rounded step).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "exp_table.h"

#define TILER_CANONICAL_F32_NAN 0x7fc00000u  // tiler-ir/src/semantic/operation.rs:21
#define TILER_CANONICAL_BF16_NAN 0x7fc0u     // ADR 0091 decision 2

// Native clang vectors: the nontemporal builtins and bit casts need them
// (HIP's float4/uint4 are wrapper structs).
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

namespace tiler {

__device__ __forceinline__ float canon(float v) {
  return v != v ? __uint_as_float(TILER_CANONICAL_F32_NAN) : v;
}

// Declared subnormal modes (tiler-reference/src/conformance.rs:498-521),
// numbered as tiler_hip_region's: 0 and 1 preserve, 2 flush a subnormal to
// the zero of its own sign, 3 flush it to +0.  Zeros, normals, infinities and
// NaNs pass unchanged.  A bf16 value widened to binary32 is subnormal exactly
// when its bf16 encoding is, so the same test serves bf16 encodings
// (bf16.rs:517-533 accept_operand / commit).
__device__ __forceinline__ float subnormal(uint32_t mode, float v) {
  if (mode <= 1u) return v;
  const uint32_t b = __float_as_uint(v);
  if ((b & 0x7f800000u) != 0 || (b & 0x007fffffu) == 0) return v;  // not subnormal
  return mode == 2u ? __uint_as_float(b & 0x80000000u) : 0.0f;
}

// subnormal(mode, .) as two masks set up once: a class test (v_cmp_class,
// classes 4 and 7: negative and positive denormal), a mask keeping the sign
// (mode 2) or nothing (mode 3), and a select.
struct Flush {
  uint32_t cls, keep;
  __device__ explicit Flush(uint32_t mode) : cls(mode > 1u ? 0x90u : 0u), keep(mode == 2u ? 0x80000000u : 0u) {}
  __device__ float operator()(float v) const {
    return __builtin_amdgcn_classf(v, cls) ? __uint_as_float(__float_as_uint(v) & keep) : v;
  }
};
// subnormal(out, .) then subnormal(in, .): a result flushed, then read as an
// operand, in one flush.  A subnormal result is a zero after a flushing out
// mode, which the in mode leaves alone; otherwise the in mode decides.
__device__ __forceinline__ Flush result_as_operand(uint32_t in_mode, uint32_t out_mode) {
  return Flush(out_mode > 1u ? out_mode : in_mode);
}

// The per-contributor rule of a serial sum under a declared contract: the
// prologue (none; the square, SquaredSerialSum; x * scale + bias,
// FusedMultiplyAddSerialSum, schedule/model.rs:709-760), the two subnormal
// modes at every arithmetic site, and the combine
// apply_to_result(canon(apply_to_operand(acc) + apply_to_operand(t)))
// (evaluate.rs:575-583).  The fold is seeded at the first contributor's value,
// never at an identity: under a flushing result mode an identity add would
// flush a lone subnormal contributor the reference transports unchanged.
enum : uint32_t { kPrologueNone = 0, kPrologueSquared = 1, kPrologueFma = 2 };
struct FoldRule {
  uint32_t prologue;
  float scale, bias;
  uint32_t in_mode, out_mode;
};
__device__ __forceinline__ float fold_contributor(const FoldRule& r, float v) {
  if (r.prologue == kPrologueSquared) {
    const float o = subnormal(r.in_mode, v);
    return canon(subnormal(r.out_mode, o * o));
  }
  if (r.prologue == kPrologueFma) {
    const float p = canon(subnormal(r.out_mode, subnormal(r.in_mode, v) * subnormal(r.in_mode, r.scale)));
    return canon(subnormal(r.out_mode, subnormal(r.in_mode, p) + subnormal(r.in_mode, r.bias)));
  }
  return v;
}
__device__ __forceinline__ float fold_combine(const FoldRule& r, float acc, float t) {
  return canon(subnormal(r.out_mode, subnormal(r.in_mode, acc) + subnormal(r.in_mode, t)));
}

// bf16 <-> f32 (ADR 0091 decision 2): widening is exact; narrowing is
// round-to-nearest-even on the upper half, every NaN to 0x7fc0, signed zero
// kept, gradual underflow, overflow to infinity at the inclusive midpoint.
__device__ __forceinline__ float bf16_widen(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}
__device__ __forceinline__ uint32_t bf16_narrow(float v) {
  uint32_t u = __float_as_uint(v);
  if (v != v) return TILER_CANONICAL_BF16_NAN;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
__device__ __forceinline__ uint32_t bf16_pack2(float lo, float hi) {
  return bf16_narrow(lo) | (bf16_narrow(hi) << 16);
}
// bf16_pack2 in one v_cvt_pk_bf16_f32, which rounds to nearest even exactly
// as bf16_narrow does on every non-NaN binary32 input (the narrowing
// kernels' tests pin it at every rounding boundary); it keeps a NaN's sign
// and payload, so NaNs are made the canonical 0x7fc00000 first, which it
// narrows to 0x7fc0.
typedef float f32x2_pair __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_pair __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t bf16_pack2_rne(float lo, float hi) {
  const f32x2_pair f = {canon(lo), canon(hi)};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_pair));
}

// IEEE 754-2019 maximum with -0 < +0, NaN-propagating
// (tiler-reference/src/softmax.rs:168-186).
// Written as selects, so that a run of maxima compiles to a straight line:
// for non-NaN operands that compare equal the result is the AND of the
// encodings (+0 for {-0, +0}, the value itself otherwise), else the larger.
__device__ __forceinline__ float maximum_f32(float a, float b) {
  const float both = __uint_as_float(__float_as_uint(a) & __float_as_uint(b));
  const float r = a == b ? both : (a > b ? a : b);
  return (a != a || b != b) ? __uint_as_float(TILER_CANONICAL_F32_NAN) : r;
}

// Wave64 xor butterfly: after it every lane holds the same value,
// v[l] = v[l] + v[l ^ o] for o = 32, 16, 8, 4, 2, 1.  Addition is commutative
// bit for bit, so the order inside each pair is immaterial.
__device__ __forceinline__ float wave_sum_butterfly(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = v + __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = maximum_f32(v, __shfl_xor(v, o, 64));
  return v;
}

// Correctly rounded binary32 reciprocal square root of a binary32 argument,
// the value certified_rsqrt_f32 admits (tiler-reference/src/rms_norm.rs:219-293,
// special arguments :246-262).  The binary64 candidate 1/sqrt(t) is within
// 2^-52 relative, so its binary32 rounding is at most one step from the
// correctly rounded value; each neighbouring midpoint m is then decided
// exactly by the sign of m^2*t - 1: m^2 has at most 50 significant bits so it
// is exact in binary64, and p + e = m^2*t exactly with p = fl(m^2*t) and
// e = fma(m^2, t, -p), p - 1 exact by Sterbenz.  No midpoint is ever hit
// exactly (rms_norm.rs:22-45), so the strict sign test is total.
__device__ __forceinline__ int midpoint_sq_times_t_minus_one_sign(double m, double t) {
  double m2 = m * m;
  double p = m2 * t;
  double e = __builtin_fma(m2, t, -p);
  double d = p - 1.0;
  if (d > -e) return 1;
  if (d < -e) return -1;
  return 0;
}
__device__ __forceinline__ float rsqrt_f32_cr(float t) {
  if (t != t) return __uint_as_float(TILER_CANONICAL_F32_NAN);
  if (t == __builtin_huge_valf()) return 0.0f;
  if (t == 0.0f) return __uint_as_float(__float_as_uint(t) | 0x7f800000u);  // +-inf
  if (t < 0.0f) return __uint_as_float(TILER_CANONICAL_F32_NAN);
  double td = (double)t;
  float c = (float)(1.0 / __builtin_sqrt(td));
  uint32_t cb = __float_as_uint(c);
  double cd = (double)c;
  double up = (cd + (double)__uint_as_float(cb + 1u)) * 0.5;
  if (midpoint_sq_times_t_minus_one_sign(up, td) < 0) return __uint_as_float(cb + 1u);
  double dn = (cd + (double)__uint_as_float(cb - 1u)) * 0.5;
  if (midpoint_sq_times_t_minus_one_sign(dn, td) > 0) return __uint_as_float(cb - 1u);
  return c;
}

// binary32 e^s for the softmax and SiLU families, with the reference's guards
// (tiler-reference/src/silu.rs:573-588): NaN -> NaN, s >= 89 -> +inf,
// s <= -104 -> +0.  Between them: k = rint(s*64/ln2), r = s - k*ln2/64 with
// ln2/64 split so k*hi is exact (|r| <= 0.0055), e^r by its degree-6 Taylor
// polynomial (truncation < 2^-64), times the binary64 table entry 2^(j/64),
// scaled by 2^(k>>6), then one rounding to binary32.  The binary64 value is
// within 2^-50 relative of e^s.
// `table` is kExp2Table64 or a copy of it in LDS (divergent lookups from LDS
// keep the vector-memory path free for the streamed operands).
__device__ __forceinline__ double exp_f64_core(double x, int& m_out, const double* table) {
  double kd = __builtin_rint(x * TILER_64_OVER_LN2);
  int k = (int)kd;
  double r = __builtin_fma(-kd, TILER_LN2_OVER_64_HI, x);
  r = __builtin_fma(-kd, TILER_LN2_OVER_64_LO, r);
  double p = 1.0 / 720.0;
  p = __builtin_fma(p, r, 1.0 / 120.0);
  p = __builtin_fma(p, r, 1.0 / 24.0);
  p = __builtin_fma(p, r, 1.0 / 6.0);
  p = __builtin_fma(p, r, 0.5);
  p = __builtin_fma(p, r, 1.0);
  p = __builtin_fma(p, r, 1.0);
  m_out = k >> 6;
  return table[k & 63] * p;
}
__device__ __forceinline__ float exp_f32_cr(float s, const double* table = kExp2Table64) {
  if (s != s) return s;
  if (s >= 89.0f) return __builtin_huge_valf();
  if (s <= -104.0f) return 0.0f;
  int m;
  double v = exp_f64_core((double)s, m, table);
  v = __builtin_ldexp(v, m);
  return (float)v;
}

// exp_f32_cr for an argument s <= 0 or NaN -- the softmax's s = fl(x - m)
// with m the row's maximum -- as one straight line: the s >= 89 guard cannot
// fire, s <= -104 selects +0, and a NaN argument stays NaN through the core
// (a NaN value; its payload aside).  The same core arithmetic as
// exp_f64_core, with k = rint(fl(s * 64/ln2)) formed by adding and removing
// 1.5 * 2^52 (round to nearest even at integer granularity, the same value
// as rint for |k| < 2^51) and read from the sum's low word: for an argument
// at or below -104 (-inf included) the k read is meaningless but defined,
// its table index k & 63 in range, and the value is selected away.
__device__ __forceinline__ float exp_f32_cr_nonpositive(float s, const double* table = kExp2Table64) {
  const double x = (double)s;
  const double shifted = x * TILER_64_OVER_LN2 + 0x1.8p52;
  const double kd = shifted - 0x1.8p52;
  const int k = (int)(uint32_t)__builtin_bit_cast(uint64_t, shifted);
  double r = __builtin_fma(-kd, TILER_LN2_OVER_64_HI, x);
  r = __builtin_fma(-kd, TILER_LN2_OVER_64_LO, r);
  double p = 1.0 / 720.0;
  p = __builtin_fma(p, r, 1.0 / 120.0);
  p = __builtin_fma(p, r, 1.0 / 24.0);
  p = __builtin_fma(p, r, 1.0 / 6.0);
  p = __builtin_fma(p, r, 0.5);
  p = __builtin_fma(p, r, 1.0);
  p = __builtin_fma(p, r, 1.0);
  const float e = (float)__builtin_ldexp(table[k & 63] * p, k >> 6);
  return s <= -104.0f ? 0.0f : e;
}

// Reference SiLU, tiler-reference/src/silu.rs:511-533: x / fl(1 + exp(-x)),
// NaN -> NaN, +inf -> +inf, -inf -> NaN.  `table` as exp_f32_cr takes it.
__device__ __forceinline__ float silu_f32(float x, const double* table = kExp2Table64) {
  if (x != x) return x;
  if (x == __builtin_huge_valf()) return x;
  if (x == -__builtin_huge_valf()) return __uint_as_float(TILER_CANONICAL_F32_NAN);
  float e = exp_f32_cr(-x, table);
  float divisor = 1.0f + e;
  return x / divisor;
}

// silu_f32 as one straight line (selects instead of early returns), so that
// several evaluations interleave: the same arithmetic on every path that is
// selected, hence the same value for every binary32 x.  The guards' lanes
// compute a discarded core value (NaN or out-of-range arguments are harmless
// to the conversions involved).
__device__ __forceinline__ float silu_f32_straight(float x, const double* table = kExp2Table64) {
  const float s = -x;
  int m;
  // the core on an argument clamped into its domain (every out-of-domain or
  // NaN lane's value is selected away below)
  double core = exp_f64_core((double)__builtin_fminf(__builtin_fmaxf(s, -104.0f), 89.0f), m, table);
  const float ecore = (float)__builtin_ldexp(core, m);
  float e = s >= 89.0f ? __builtin_huge_valf() : (s <= -104.0f ? 0.0f : ecore);
  e = s != s ? s : e;
  const float r = x / (1.0f + e);
  const float special = x == -__builtin_huge_valf() ? __uint_as_float(TILER_CANONICAL_F32_NAN) : x;
  return (x != x || x == __builtin_huge_valf() || x == -__builtin_huge_valf()) ? special : r;
}

// SiLU for a result that is narrowed to bf16 next (the contraction epilogue):
// silu_for_bf16 returns a binary32 value whose bf16 narrowing equals
// bf16_narrow(silu_f32(x)) for every binary32 x -- the reference SiLU
// (silu.rs:511-533), one narrowing, no second semantics.
// * The fast value (silu_fast_f32), nine operations: e^-x = 2^(yh + yl) with
//   yh = fl(-x*log2e) and yl its rounding error (exact, by an FMA) plus the
//   constant's own, from the hardware 2^yh corrected to first order by
//   yl*ln2; then x times the hardware reciprocal of fl(1 + e).  For
//   -80 < x < 2^127 it is within a few binary32 steps of silu_f32(x).  It is
//   x itself for x >= 17 (e <= e^-17 < 2^-24, so fl(1 + e) = 1), and keeps
//   the sign of a zero (x * 0.5).
// * Only a value whose low 16 bits lie within kSiluGuard steps of the bf16
//   midpoint 0x8000 can round to a different bf16 than silu_f32(x) does;
//   those, and every x outside (-80, 2^127) (NaN, +-inf, x <= -80, the
//   largest finite x), are marked exact (silu_bf16_candidate) and take
//   silu_f32 itself.
// The equivalence is checked on the device over all 2^32 binary32 inputs,
// together with the largest distance between the two values.
constexpr uint32_t kSiluGuard = 8;
__device__ __forceinline__ float silu_fast_f32(float x) {
  const float kLog2e = 0x1.715476p+0f;       // binary32 nearest log2(e)
  const float kLog2eLo = 0x1.4ae0c0p-26f;    // binary32 nearest log2(e) - kLog2e
  const float kLn2 = 0x1.62e430p-1f;
  const float yh = x * -kLog2e;
  const float yl = __builtin_fmaf(x, -kLog2eLo, __builtin_fmaf(x, -kLog2e, -yh));
  const float p = __builtin_amdgcn_exp2f(yh);
  const float e = __builtin_fmaf(p, yl * kLn2, p);
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}
// The fast value, branch free, and whether only silu_f32(x) is known to
// narrow right.
__device__ __forceinline__ float silu_bf16_candidate(float x, bool& exact) {
  const float v = silu_fast_f32(x);
  const bool near_midpoint = (__float_as_uint(v) & 0xffffu) - (0x8000u - kSiluGuard) <= 2u * kSiluGuard;
  exact = !(x > -80.0f && x < 0x1.0p127f) || near_midpoint;
  return v;
}
// The same fast value, with the wave's lanes that must take silu_f32 (the
// lanes silu_bf16_candidate marks exact) as a ballot of the three raw
// compares: the mask stays in scalar registers.
__device__ __forceinline__ float silu_bf16_fast_marked(float x, uint64_t& mask) {
  const float v = silu_fast_f32(x);
  const uint32_t key = (__float_as_uint(v) & 0xffffu) - (0x8000u - kSiluGuard);
  mask = __builtin_amdgcn_ballot_w64(key <= 2u * kSiluGuard) | __builtin_amdgcn_ballot_w64(!(x > -80.0f)) |
         __builtin_amdgcn_ballot_w64(!(x < 0x1.0p127f));
  return v;
}
__device__ __forceinline__ float silu_for_bf16(float x) {
  bool exact;
  const float v = silu_bf16_candidate(x, exact);
  return exact ? silu_f32_straight(x) : v;
}

// f(Step<0>{}), f(Step<1>{}), ... f(Step<N - 1>{}) while f returns true: a
// loop unrolled at compile time (the index is a constant in each call, so
// register arrays indexed by it stay in registers), whatever the loop
// unroller would decide for a body that holds a loop of its own.
template <int J>
struct Step {
  static constexpr int value = J;
};
template <int J, int N, typename F>
__device__ __forceinline__ void unrolled_while(F& f) {
  if constexpr (J < N) {
    if (f(Step<J>{})) unrolled_while<J + 1, N>(f);
  }
}

// A DPP move of v across the lanes of each 16-lane row (kCtrl: row_shr:1 =
// 0x111, lane i takes lane i - 1; row_ror:9 = 0x129, lane i takes lane
// (i - 9) mod 16, so lanes 7 and 15 go to lanes 0 and 8).
template <int kCtrl>
__device__ __forceinline__ float dpp_move(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, 0xF, 0xF, true));
}

// The relay fold of one ring chunk by one wave: lane 8 g + s holds in seg the
// S4 float4 slots (4 S4 consecutive contributors, ascending) of segment s of
// row g's chunk.  Row g's running value enters the chunk in lane 8 g; each
// hop, every lane applies acc = step(acc, c) to its segment's contributors in
// order and a DPP move hands each value to the next lane of its group (the
// eighth hop back to lane 8 g), so the lane holding row g's value at hop s is
// lane 8 g + s and the chunk's 32 S4 contributors are taken in ascending
// order.  The steps read registers only, and one wave instruction advances
// the eight rows' chains.  What the other lanes compute is never read.
// kSeed: the chunk opens the row, whose first contributor is the seed (acc
// becomes it, no step), as a fold seeded at its first contributor does.
template <uint32_t S4, bool kSeed = false, typename F>
__device__ __forceinline__ float relay_fold(const f32x4 (&seg)[S4], float acc, F step) {
  auto add = [&](auto seeded) {
#pragma unroll
    for (uint32_t k = 0; k < S4; ++k) {
      acc = decltype(seeded)::value && k == 0 ? seg[0].x : step(acc, seg[k].x);
      acc = step(acc, seg[k].y);
      acc = step(acc, seg[k].z);
      acc = step(acc, seg[k].w);
    }
  };
  constexpr Step<0> plain{};
  int h = 0;
  if constexpr (kSeed) {
    add(Step<1>{});
    acc = dpp_move<0x111>(acc);
    h = 1;
  }
  // A loop, not unrolled: the callers unroll their chunk loops over the
  // resident pieces, which must stay small enough to unroll.
#pragma unroll 1
  for (; h < 7; ++h) {
    add(plain);
    acc = dpp_move<0x111>(acc);
  }
  add(plain);
  return dpp_move<0x129>(acc);
}
// The relay fold of the strict sum: step(acc, c) = fl(acc + c).
template <uint32_t S4>
__device__ __forceinline__ float relay_fold_chunk(const f32x4 (&seg)[S4], float acc) {
  return relay_fold<S4>(seg, acc, [](float a, float c) { return a + c; });
}

// The strict sum's relay fold over `passes` (at most kMaxPasses) consecutive
// 256-element passes of a row that lies contiguously in LDS at `row`
// (16-byte aligned): lane 8 g + s of the folding wave, s = lane % 8, takes
// elements 32 s .. 32 s + 31 of each pass, and the next pass's segment is
// read while the current one is folded.  Row g's sum ends in lane 8 g.
template <uint32_t kMaxPasses>
__device__ __forceinline__ float relay_fold_row(const f32x4* row, uint32_t s, uint32_t passes, float acc) {
  constexpr uint32_t S4 = 8;
  const f32x4* src = row + s * S4;
  f32x4 a[S4], b[S4];
#pragma unroll
  for (uint32_t k = 0; k < S4; ++k) a[k] = src[k];
  auto pass = [&](auto ps) -> bool {
    constexpr uint32_t p = decltype(ps)::value;
    if (p >= passes) return false;
    f32x4(&cur)[S4] = (p & 1) ? b : a;
    f32x4(&nxt)[S4] = (p & 1) ? a : b;
    const f32x4* next = src + (p + 1 < passes ? p + 1 : p) * (32u * S4 / 4u);
#pragma unroll
    for (uint32_t k = 0; k < S4; ++k) nxt[k] = next[k];
    acc = relay_fold_chunk<S4>(cur, acc);
    return true;
  };
  unrolled_while<0, kMaxPasses>(pass);
  return acc;
}

}  // namespace tiler
