// Pointwise expression DAGs (ScalarProgram::PointwiseF32 / PointwiseBf16,
// tiler-ir/src/schedule/pointwise.rs:74-140, pointwise_bf16.rs:114-168) for
// gfx950: one fused launch per expression, whatever its shape.
//
// The host compiles the verified DAG into a register program (one instruction
// per node, operands and destination in a small register file, allocated by
// last use) and binds it as a constant slot; every element runs that program.
// The instruction index is uniform across a wave, so the opcode dispatch is
// scalar work and the registers are indexed uniformly.
//
// Per node (tiler-metal's goldens emit the same: one statement per node and
// the family's canonical NaN after each arithmetic result):
//   f32   ADD/MULTIPLY/DIVIDE: one IEEE binary32 rounding (division is never a
//         reciprocal multiply: pointwise.rs:97-106); EXP: tiler::exp_f32_cr,
//         RSQRT: tiler::rsqrt_f32_cr (the correctly rounded values the
//         registered accuracy contracts admit); operands and results pass the
//         region's subnormal modes (tiler-reference/src/conformance.rs:498-521)
//         and the result is canonicalized (0x7fc00000).
//   bf16  ADD/MULTIPLY on exactly widened operands, one rounding to bf16
//         (binary32 holds every exact sum or product of two bf16 values to
//         within one binary32 rounding that cannot move the bf16 rounding), NaN
//         to 0x7fc0 (ADR 0091; tiler-metal/goldens/pointwise_scale_bias_bf16.metal).
//
// Two forms:
//   tiler_expr_{f32,bf16}_r16*  register file of 16 per element, 16-byte
//                               vectors (4 f32 / 8 bf16 per lane) or one
//                               element per lane; programs needing at most 16
//                               live values.  The vector f32 form comes twice:
//                               _r16_ with both subnormal modes preserve (the
//                               mode code compiled out, ~10% faster at 2^26)
//                               and _r16f_ with the modes read at run time.
//   tiler_expr_{f32,bf16}_mem   one element per lane, the register file in a
//                               scratch slot laid out [register][lane]; any
//                               program (up to 4096 nodes).
#include "common.h"

namespace {

// Instruction layout (12 bytes, little-endian), as the host writes it.
struct ExprInstr {
  uint16_t op, dst, a, b;
  uint32_t imm;  // CONSTANT: bits (bf16 in the low 16); INPUT: access ordinal
};

enum : uint32_t {
  kInput = 0,
  kConstant = 1,
  kAdd = 2,
  kMultiply = 3,
  kDivide = 4,
  kExp = 5,
  kRsqrt = 6,
};

constexpr uint32_t kMaxInputs = 16;

struct ExprInputs {
  const void* p[kMaxInputs];
};

typedef float f32x16v __attribute__((ext_vector_type(16)));

// Subnormal modes: 1 preserve (0 reads as 1), 2 flush to the zero of the
// same sign, 3 flush to +0 (conformance.rs:498-521).
__device__ __forceinline__ float apply_mode(uint32_t mode, float v) { return tiler::subnormal(mode, v); }

__device__ __forceinline__ float f32_node(uint32_t op, float x, float y, uint32_t in_mode,
                                          uint32_t out_mode) {
  x = apply_mode(in_mode, x);
  y = apply_mode(in_mode, y);
  float r;
  switch (op) {
    case kAdd: r = x + y; break;
    case kMultiply: r = x * y; break;
    case kDivide: r = x / y; break;
    case kExp: r = tiler::exp_f32_cr(x); break;
    default: r = tiler::rsqrt_f32_cr(x); break;
  }
  return tiler::canon(apply_mode(out_mode, r));
}

// bf16 under the modes (bf16.rs:517-533): a subnormal operand encoding is
// replaced before the operation reads it, a subnormal rounded result after
// its one rounding (a widened bf16 value is subnormal exactly when its
// encoding is).
__device__ __forceinline__ float bf16_node(uint32_t op, float x, float y, uint32_t in_mode = 1u,
                                           uint32_t out_mode = 1u) {
  x = tiler::subnormal(in_mode, x);
  y = tiler::subnormal(in_mode, y);
  const float r = op == kAdd ? x + y : x * y;
  return tiler::subnormal(out_mode, tiler::bf16_widen(tiler::bf16_narrow(r)));
}

// ---------------------------------------------------------------------------
// Register form.  kVec: E elements per lane (4 f32 / 8 bf16: one 16-byte
// vector), element i of lane chunk q is y[q*E + i]; otherwise one element
// per lane (any alignment and length).  NIN > 0: the program's first NIN
// instructions are the inputs 0..NIN-1 into registers 0..NIN-1 (the host
// orders them so); the kernel issues all NIN loads of a chunk together before
// running the rest.  NIN == 0: inputs load where their instruction stands.
template <bool kBf16, bool kVec, int NIN, bool kModes>
__device__ __forceinline__ void expr_r16_body(ExprInputs in, void* __restrict__ y,
                                              const ExprInstr* __restrict__ prog, uint32_t count,
                                              uint32_t result, uint64_t chunks, uint32_t in_mode,
                                              uint32_t out_mode) {
  constexpr int E = kVec ? (kBf16 ? 8 : 4) : 1;
  constexpr bool kPipelined = kVec && NIN > 0;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  // Pipelined form: the next chunk's NIN input loads are issued before this
  // chunk's program runs, so a wave keeps its loads in flight while it
  // interprets.
  u32x4 next[NIN > 0 ? NIN : 1];
  const uint64_t q0 = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (kPipelined && q0 < chunks) {
#pragma unroll
    for (int k = 0; k < NIN; ++k)
      next[k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(in.p[k]) + q0);
  }
  for (uint64_t q = q0; q < chunks; q += stride) {
    // One 16-register file per vector element, as vector values indexed by
    // the (uniform) register number: no stack array, so the files live in
    // VGPRs and a read or write is one indexed register move.
    f32x16v r[E];
    auto unpack = [&](u32x4 raw, float (&v)[E]) {
      if (kBf16) {
#pragma unroll
        for (int h = 0; h < E / 2; ++h) {
          v[2 * h] = tiler::bf16_widen(raw[h] & 0xffffu);
          v[2 * h + 1] = tiler::bf16_widen(raw[h] >> 16);
        }
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] = __uint_as_float(raw[e % 4]);
      }
    };
    auto load_scalar = [&](uint32_t k) -> float {
      return kBf16 ? tiler::bf16_widen(static_cast<const uint16_t*>(in.p[k])[q])
                   : static_cast<const float*>(in.p[k])[q];
    };
    if (NIN > 0) {
      if (kVec) {
        u32x4 raw[NIN > 0 ? NIN : 1];
#pragma unroll
        for (int k = 0; k < NIN; ++k) raw[k] = next[k];
        if (q + stride < chunks) {
#pragma unroll
          for (int k = 0; k < NIN; ++k)
            next[k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(in.p[k]) + q + stride);
        }
#pragma unroll
        for (int k = 0; k < NIN; ++k) {
          float v[E];
          unpack(raw[k], v);
#pragma unroll
          for (int e = 0; e < E; ++e) r[e][k] = v[e];
        }
      } else {
        float raw[NIN > 0 ? NIN : 1];
#pragma unroll
        for (int k = 0; k < NIN; ++k) raw[k] = load_scalar(k);
#pragma unroll
        for (int k = 0; k < NIN; ++k) r[0][k] = raw[k];
      }
    }
    for (uint32_t i = NIN; i < count; ++i) {
      const uint32_t w0 = __builtin_amdgcn_readfirstlane(reinterpret_cast<const uint32_t*>(prog + i)[0]);
      const uint32_t w1 = __builtin_amdgcn_readfirstlane(reinterpret_cast<const uint32_t*>(prog + i)[1]);
      const uint32_t imm = __builtin_amdgcn_readfirstlane(prog[i].imm);
      const uint32_t op = w0 & 0xffffu, dst = w0 >> 16, a = w1 & 0xffffu, b = w1 >> 16;
      float v[E];
      if (op == kInput) {
        if (kVec) unpack(__builtin_nontemporal_load(reinterpret_cast<const u32x4*>(in.p[imm]) + q), v);
        else v[0] = load_scalar(imm);
      } else if (op == kConstant) {
        const float c = kBf16 ? tiler::bf16_widen(imm & 0xffffu) : __uint_as_float(imm);
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] = c;
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e)
          v[e] = kBf16    ? (kModes ? bf16_node(op, r[e][a], r[e][b], in_mode, out_mode) : bf16_node(op, r[e][a], r[e][b]))
                 : kModes ? f32_node(op, r[e][a], r[e][b], in_mode, out_mode)
                          : f32_node(op, r[e][a], r[e][b], 1u, 1u);
      }
#pragma unroll
      for (int e = 0; e < E; ++e) r[e][dst] = v[e];
    }
    if (!kVec) {
      if (kBf16) static_cast<uint16_t*>(y)[q] = (uint16_t)tiler::bf16_narrow(r[0][result]);
      else static_cast<float*>(y)[q] = r[0][result];
      continue;
    }
    u32x4 o;
    if (kBf16) {
#pragma unroll
      for (int h = 0; h < 4; ++h)
        o[h] = tiler::bf16_narrow(r[2 * h][result]) | (tiler::bf16_narrow(r[2 * h + 1][result]) << 16);
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e) o[e % 4] = __float_as_uint(r[e][result]);
    }
    __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(y) + q);
  }
}

// A one-input f32 program over a single value (a fold's epilogue,
// ScalarProgram::SquaredSerialSumThenEpilogue, model.rs:815-830): instruction
// 0 is the input (the folded value) into register 0.
__device__ __forceinline__ float expr_epilogue_f32(const ExprInstr* __restrict__ prog, uint32_t count,
                                                   uint32_t result, float value) {
  f32x16v r;
  r[0] = value;
  for (uint32_t i = 1; i < count; ++i) {
    const uint32_t w0 = __builtin_amdgcn_readfirstlane(reinterpret_cast<const uint32_t*>(prog + i)[0]);
    const uint32_t w1 = __builtin_amdgcn_readfirstlane(reinterpret_cast<const uint32_t*>(prog + i)[1]);
    const uint32_t imm = __builtin_amdgcn_readfirstlane(prog[i].imm);
    const uint32_t op = w0 & 0xffffu, dst = w0 >> 16, a = w1 & 0xffffu, b = w1 >> 16;
    float v;
    if (op == kInput) v = value;
    else if (op == kConstant) v = __uint_as_float(imm);
    else v = f32_node(op, r[a], r[b], 1u, 1u);
    r[dst] = v;
  }
  return r[result];
}

// ---------------------------------------------------------------------------
// Value-store form: element-by-element, registers in scratch [reg][lanes].
template <bool kBf16>
__device__ __forceinline__ void expr_mem_body(ExprInputs in, void* __restrict__ y,
                                              const ExprInstr* __restrict__ prog, uint32_t count,
                                              uint32_t result, uint64_t n, uint32_t in_mode,
                                              uint32_t out_mode, float* __restrict__ store) {
  const uint64_t lanes = (uint64_t)gridDim.x * blockDim.x;
  const uint64_t lane = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (uint64_t i = lane; i < n; i += lanes) {
    for (uint32_t k = 0; k < count; ++k) {
      const uint32_t w0 = __builtin_amdgcn_readfirstlane(reinterpret_cast<const uint32_t*>(prog + k)[0]);
      const uint32_t w1 = __builtin_amdgcn_readfirstlane(reinterpret_cast<const uint32_t*>(prog + k)[1]);
      const uint32_t imm = __builtin_amdgcn_readfirstlane(prog[k].imm);
      const uint32_t op = w0 & 0xffffu, dst = w0 >> 16, a = w1 & 0xffffu, b = w1 >> 16;
      float v;
      if (op == kInput) {
        v = kBf16 ? tiler::bf16_widen(static_cast<const uint16_t*>(in.p[imm])[i])
                  : static_cast<const float*>(in.p[imm])[i];
      } else if (op == kConstant) {
        v = kBf16 ? tiler::bf16_widen(imm & 0xffffu) : __uint_as_float(imm);
      } else {
        const float x = store[(uint64_t)a * lanes + lane], z = store[(uint64_t)b * lanes + lane];
        v = kBf16 ? bf16_node(op, x, z, in_mode, out_mode) : f32_node(op, x, z, in_mode, out_mode);
      }
      store[(uint64_t)dst * lanes + lane] = v;
    }
    const float out = store[(uint64_t)result * lanes + lane];
    if (kBf16) static_cast<uint16_t*>(y)[i] = (uint16_t)tiler::bf16_narrow(out);
    else static_cast<float*>(y)[i] = out;
  }
}

}  // namespace

// tiler_expr_{f32,bf16}_r16_i{1..4} (inputs prefetched), _r16_i0 (inputs in
// place), _r16s_i{0..4} (one element per lane), _mem (value store);
// tiler_expr_f32_r16f_i{0..4}: the vector form under flushing modes.
#define TILER_EXPR_R16(TY, BF, NIN)                                                                 \
  extern "C" __global__ void __launch_bounds__(256) tiler_expr_##TY##_r16_i##NIN(                   \
      ExprInputs in, void* __restrict__ y, const ExprInstr* __restrict__ prog, uint32_t count,     \
      uint32_t result, uint64_t chunks, uint32_t in_mode, uint32_t out_mode) {                      \
    expr_r16_body<BF, true, NIN, false>(in, y, prog, count, result, chunks, in_mode, out_mode);     \
  }                                                                                                 \
  extern "C" __global__ void __launch_bounds__(256) tiler_expr_##TY##_r16s_i##NIN(                  \
      ExprInputs in, void* __restrict__ y, const ExprInstr* __restrict__ prog, uint32_t count,     \
      uint32_t result, uint64_t n, uint32_t in_mode, uint32_t out_mode) {                           \
    expr_r16_body<BF, false, NIN, true>(in, y, prog, count, result, n, in_mode, out_mode);          \
  }
#define TILER_EXPR_R16F(NIN)                                                                        \
  extern "C" __global__ void __launch_bounds__(256) tiler_expr_f32_r16f_i##NIN(                     \
      ExprInputs in, void* __restrict__ y, const ExprInstr* __restrict__ prog, uint32_t count,     \
      uint32_t result, uint64_t chunks, uint32_t in_mode, uint32_t out_mode) {                      \
    expr_r16_body<false, true, NIN, true>(in, y, prog, count, result, chunks, in_mode, out_mode);   \
  }
#define TILER_EXPR_KERNELS(TY, BF)                                                                  \
  TILER_EXPR_R16(TY, BF, 0)                                                                         \
  TILER_EXPR_R16(TY, BF, 1)                                                                         \
  TILER_EXPR_R16(TY, BF, 2)                                                                         \
  TILER_EXPR_R16(TY, BF, 3)                                                                         \
  TILER_EXPR_R16(TY, BF, 4)                                                                         \
  extern "C" __global__ void __launch_bounds__(256) tiler_expr_##TY##_mem(                          \
      ExprInputs in, void* __restrict__ y, const ExprInstr* __restrict__ prog, uint32_t count,     \
      uint32_t result, uint64_t n, uint32_t in_mode, uint32_t out_mode, float* __restrict__ store) { \
    expr_mem_body<BF>(in, y, prog, count, result, n, in_mode, out_mode, store);                     \
  }
TILER_EXPR_KERNELS(f32, false)
TILER_EXPR_KERNELS(bf16, true)
TILER_EXPR_R16F(0)
TILER_EXPR_R16F(1)
TILER_EXPR_R16F(2)
TILER_EXPR_R16F(3)
TILER_EXPR_R16F(4)
