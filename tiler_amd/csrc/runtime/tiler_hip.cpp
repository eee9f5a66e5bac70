// tiler-hip host runtime: the C ABI of include/tiler_hip.h over the HIP
// module API.  The gfx950 code object is compiled ahead of time and linked
// into this library as bytes (payload.S); bind() loads it with
// hipModuleLoadData and every launch goes through hipModuleLaunchKernel.
#include "tiler_hip.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "build_info.h"
#include "code_object.h"
#include "digest.h"
#include "envelope.h"
#include "noalloc.h"
#include "program.h"

extern "C" const uint8_t tiler_hip_code_object[];
extern "C" const uint8_t tiler_hip_code_object_end[];
extern "C" const uint8_t tiler_hip_source_bundle[];
extern "C" const uint8_t tiler_hip_source_bundle_end[];

namespace {

constexpr const char* kBackend = "tiler.hip";
constexpr const char* kRepresentation = "tiler.hip.gfx950.code-object-v1";
constexpr const char* kPayloadSchema = "tiler.hip.payload.v1";
constexpr const char* kTarget = "amdgcn-amd-amdhsa--gfx950";
constexpr const char* kProfileKey = "tiler.hip.gfx950.profile-v1";

struct EntryRow {
  const char* symbol;
  const char* family;
  uint32_t buffers;
};

// Every kernel the payload carries, in a fixed order (the entry mapping).
const EntryRow kEntries[] = {
    {"tiler_sum_f32_serial", "strict-serial-sum-f32/serial", 2},
    {"tiler_sum_f32_staged_r1", "strict-serial-sum-f32/serial", 2},
    {"tiler_sum_f32_staged_r1_u", "strict-serial-sum-f32/serial", 2},
    {"tiler_sum_f32_staged_r4", "strict-serial-sum-f32/serial", 2},
    {"tiler_sum_f32_staged_r4_u", "strict-serial-sum-f32/serial", 2},
    {"tiler_sum_f32_staged_r16", "strict-serial-sum-f32/serial", 2},
    {"tiler_sum_f32_staged_r16_u", "strict-serial-sum-f32/serial", 2},
    {"tiler_sum_f32_staged_r64", "strict-serial-sum-f32/serial", 2},
    {"tiler_sum_f32_staged_r64_u", "strict-serial-sum-f32/serial", 2},
    {"tiler_sum_f32_staged_r256", "strict-serial-sum-f32/serial", 2},
    {"tiler_sum_f32_staged_r256_u", "strict-serial-sum-f32/serial", 2},
    {"tiler_sum_f32_partials", "strict-serial-sum-f32/multipass", 2},
    {"tiler_sum_f32_cooperative", "strict-serial-sum-f32/cooperative-workgroup", 2},
    // the same folds under a rule: a flushing contract, or a fused prologue
    {"tiler_sum_f32_staged_r1_m", "serial-sum-f32/serial+rule", 2},
    {"tiler_sum_f32_staged_r1_u_m", "serial-sum-f32/serial+rule", 2},
    {"tiler_sum_f32_staged_r4_m", "serial-sum-f32/serial+rule", 2},
    {"tiler_sum_f32_staged_r4_u_m", "serial-sum-f32/serial+rule", 2},
    {"tiler_sum_f32_staged_r16_m", "serial-sum-f32/serial+rule", 2},
    {"tiler_sum_f32_staged_r16_u_m", "serial-sum-f32/serial+rule", 2},
    {"tiler_sum_f32_staged_r64_m", "serial-sum-f32/serial+rule", 2},
    {"tiler_sum_f32_staged_r64_u_m", "serial-sum-f32/serial+rule", 2},
    {"tiler_sum_f32_staged_r256_m", "serial-sum-f32/serial+rule", 2},
    {"tiler_sum_f32_staged_r256_u_m", "serial-sum-f32/serial+rule", 2},
    {"tiler_sum_f32_partials_m", "serial-sum-f32/multipass+rule", 2},
    {"tiler_sum_f32_cooperative_m", "serial-sum-f32/cooperative-workgroup+rule", 2},
    {"tiler_fold_f32_m", "serial-sum-f32/serial-any-axes+rule", 2},
    {"tiler_map_f32_m", "pointwise-f32+modes", 3},
    {"tiler_contract_general_f32_m", "tensor-contraction-f32/strict-general+modes", 4},
    {"tiler_contract_general_bf16_m", "tensor-contraction-bf16/strict-general+modes", 4},
    {"tiler_contract_general_bf16_silu_m", "tensor-contraction-bf16/strict-general+silu+modes", 4},
    {"tiler_map_bf16_m", "pointwise-bf16+modes", 3},
    {"tiler_sum_f32_grid", "strict-serial-sum-f32/tree", 2},
    {"tiler_sum_f32_grid_unaligned", "strict-serial-sum-f32/tree", 2},
    {"tiler_sum_f32_grid_final", "strict-serial-sum-f32/tree", 2},
    {"tiler_sum_f32_rows", "strict-serial-sum-f32/tree", 2},
    {"tiler_sum_f32_rows_w", "strict-serial-sum-f32/tree", 2},
    {"tiler_sum_f32_rows_w_u", "strict-serial-sum-f32/tree", 2},
    {"tiler_rms_norm_bf16_ch1", "rms-norm/bf16", 3},
    {"tiler_rms_norm_bf16_ch1_full", "rms-norm/bf16", 3},
    {"tiler_rms_norm_bf16_ch1_u", "rms-norm/bf16", 3},
    {"tiler_rms_norm_bf16_ch2", "rms-norm/bf16", 3},
    {"tiler_rms_norm_bf16_ch2_full", "rms-norm/bf16", 3},
    {"tiler_rms_norm_bf16_ch2_u", "rms-norm/bf16", 3},
    {"tiler_rms_norm_bf16_ch4", "rms-norm/bf16", 3},
    {"tiler_rms_norm_bf16_ch4_full", "rms-norm/bf16", 3},
    {"tiler_rms_norm_bf16_ch4_u", "rms-norm/bf16", 3},
    {"tiler_rms_norm_bf16_ch8", "rms-norm/bf16", 3},
    {"tiler_rms_norm_bf16_ch8_full", "rms-norm/bf16", 3},
    {"tiler_rms_norm_bf16_ch8_u", "rms-norm/bf16", 3},
    {"tiler_rms_norm_bf16_ch16", "rms-norm/bf16", 3},
    {"tiler_rms_norm_bf16_ch16_full", "rms-norm/bf16", 3},
    {"tiler_rms_norm_bf16_ch16_u", "rms-norm/bf16", 3},
    {"tiler_rms_norm_f32_ch1", "rms-norm-f32", 3},
    {"tiler_rms_norm_f32_ch1_full", "rms-norm-f32", 3},
    {"tiler_rms_norm_f32_ch1_u", "rms-norm-f32", 3},
    {"tiler_rms_norm_f32_ch2", "rms-norm-f32", 3},
    {"tiler_rms_norm_f32_ch2_full", "rms-norm-f32", 3},
    {"tiler_rms_norm_f32_ch2_u", "rms-norm-f32", 3},
    {"tiler_rms_norm_f32_ch4", "rms-norm-f32", 3},
    {"tiler_rms_norm_f32_ch4_full", "rms-norm-f32", 3},
    {"tiler_rms_norm_f32_ch4_u", "rms-norm-f32", 3},
    {"tiler_rms_norm_f32_ch8", "rms-norm-f32", 3},
    {"tiler_rms_norm_f32_ch8_full", "rms-norm-f32", 3},
    {"tiler_rms_norm_f32_ch8_u", "rms-norm-f32", 3},
    {"tiler_rms_norm_f32_ch16", "rms-norm-f32", 3},
    {"tiler_rms_norm_f32_ch16_full", "rms-norm-f32", 3},
    {"tiler_rms_norm_f32_ch16_u", "rms-norm-f32", 3},
    {"tiler_rms_norm_f32_ch32", "rms-norm-f32", 3},
    {"tiler_rms_norm_f32_ch32_full", "rms-norm-f32", 3},
    {"tiler_rms_norm_f32_ch32_u", "rms-norm-f32", 3},
    {"tiler_softmax_f32_ch1", "softmax-f32", 2},
    {"tiler_softmax_f32_ch1_full", "softmax-f32", 2},
    {"tiler_softmax_f32_ch1_u", "softmax-f32", 2},
    {"tiler_softmax_f32_ch2", "softmax-f32", 2},
    {"tiler_softmax_f32_ch2_full", "softmax-f32", 2},
    {"tiler_softmax_f32_ch2_u", "softmax-f32", 2},
    {"tiler_softmax_f32_ch4", "softmax-f32", 2},
    {"tiler_softmax_f32_ch4_full", "softmax-f32", 2},
    {"tiler_softmax_f32_ch4_u", "softmax-f32", 2},
    {"tiler_softmax_f32_ch8", "softmax-f32", 2},
    {"tiler_softmax_f32_ch8_full", "softmax-f32", 2},
    {"tiler_softmax_f32_ch8_u", "softmax-f32", 2},
    {"tiler_softmax_f32_ch16", "softmax-f32", 2},
    {"tiler_softmax_f32_ch16_full", "softmax-f32", 2},
    {"tiler_softmax_f32_ch16_u", "softmax-f32", 2},
    {"tiler_softmax_f32_ch32", "softmax-f32", 2},
    {"tiler_softmax_f32_ch32_full", "softmax-f32", 2},
    {"tiler_softmax_f32_ch32_u", "softmax-f32", 2},
    {"tiler_rms_norm_bf16_long1_a", "rms-norm-bf16/long-row", 3},
    {"tiler_rms_norm_bf16_long1_u", "rms-norm-bf16/long-row", 3},
    {"tiler_rms_norm_bf16_long2_a", "rms-norm-bf16/long-row", 3},
    {"tiler_rms_norm_bf16_long2_u", "rms-norm-bf16/long-row", 3},
    {"tiler_rms_norm_bf16_long4_a", "rms-norm-bf16/long-row", 3},
    {"tiler_rms_norm_bf16_long4_u", "rms-norm-bf16/long-row", 3},
    {"tiler_rms_norm_bf16_long8_a", "rms-norm-bf16/long-row", 3},
    {"tiler_rms_norm_bf16_long8_u", "rms-norm-bf16/long-row", 3},
    {"tiler_rms_norm_bf16_long0_a", "rms-norm-bf16/long-row", 3},
    {"tiler_rms_norm_bf16_long0_u", "rms-norm-bf16/long-row", 3},
    {"tiler_rms_norm_f32_long1_a", "rms-norm-f32/long-row", 3},
    {"tiler_rms_norm_f32_long1_u", "rms-norm-f32/long-row", 3},
    {"tiler_rms_norm_f32_long2_a", "rms-norm-f32/long-row", 3},
    {"tiler_rms_norm_f32_long2_u", "rms-norm-f32/long-row", 3},
    {"tiler_rms_norm_f32_long4_a", "rms-norm-f32/long-row", 3},
    {"tiler_rms_norm_f32_long4_u", "rms-norm-f32/long-row", 3},
    {"tiler_rms_norm_f32_long8_a", "rms-norm-f32/long-row", 3},
    {"tiler_rms_norm_f32_long8_u", "rms-norm-f32/long-row", 3},
    {"tiler_rms_norm_f32_long0_a", "rms-norm-f32/long-row", 3},
    {"tiler_rms_norm_f32_long0_u", "rms-norm-f32/long-row", 3},
    {"tiler_softmax_f32_long_r_a", "softmax-f32/long-row", 2},
    {"tiler_softmax_f32_long_r_u", "softmax-f32/long-row", 2},
    {"tiler_softmax_f32_split_max_a", "softmax-f32/split-row", 2},
    {"tiler_softmax_f32_split_max_u", "softmax-f32/split-row", 2},
    {"tiler_softmax_f32_split_sum_a", "softmax-f32/split-row", 3},
    {"tiler_softmax_f32_split_sum_u", "softmax-f32/split-row", 3},
    {"tiler_softmax_f32_split_out_a", "softmax-f32/split-row", 4},
    {"tiler_softmax_f32_split_out_u", "softmax-f32/split-row", 4},
    {"tiler_softmax_f32_rowsync_a", "softmax-f32/row-synchronized", 3},
    {"tiler_softmax_f32_rowsync_u", "softmax-f32/row-synchronized", 3},
    {"tiler_gather_u128", "gather", 4},
    {"tiler_gather_u64", "gather", 4},
    {"tiler_gather_u32", "gather", 4},
    {"tiler_gather_u16", "gather", 4},
    {"tiler_gather_u8", "gather", 4},
    {"tiler_map_f32", "pointwise-f32", 3},
    {"tiler_map_bf16", "pointwise-bf16", 3},
    {"tiler_map_f32_v4_op0", "pointwise-f32", 3},
    {"tiler_map_bf16_v8_op0", "pointwise-bf16", 3},
    {"tiler_map_f32_v4_op1", "pointwise-f32", 3},
    {"tiler_map_bf16_v8_op1", "pointwise-bf16", 3},
    {"tiler_map_f32_v4_op2", "pointwise-f32", 3},
    {"tiler_map_bf16_v8_op2", "pointwise-bf16", 3},
    {"tiler_map_f32_v4_op2_b", "pointwise-f32", 3},
    {"tiler_map_bf16_v8_op2_b", "pointwise-bf16", 3},
    {"tiler_map_f32_v4_op3", "pointwise-f32", 3},
    {"tiler_map_bf16_v8_op3", "pointwise-bf16", 3},
    {"tiler_map_f32_v4_op3_b", "pointwise-f32", 3},
    {"tiler_map_bf16_v8_op3_b", "pointwise-bf16", 3},
    {"tiler_broadcast_u32", "broadcast", 2},
    {"tiler_broadcast_u16", "broadcast", 2},
    {"tiler_broadcast_rows_u32", "broadcast", 2},
    {"tiler_broadcast_rows_u16", "broadcast", 2},
    {"tiler_fill_u32", "fill", 1},
    {"tiler_probe_subnormals", "probe", 2},
    {"tiler_narrow_f32_bf16_v8", "convert-f32-to-bf16/narrow", 2},
    {"tiler_narrow_f32_bf16", "convert-f32-to-bf16/narrow", 2},
    {"tiler_widen_bf16_f32_v8", "convert-bf16-to-f32/widen", 2},
    {"tiler_widen_bf16_f32", "convert-bf16-to-f32/widen", 2},
    {"tiler_dequantize_u4_f32_w", "dequantize-strict-affine-u4", 2},
    {"tiler_dequantize_u4_f32_v4", "dequantize-strict-affine-u4", 2},
    {"tiler_dequantize_u4_f32", "dequantize-strict-affine-u4", 2},
    {"tiler_dequantize_u4_f32_w_slots", "dequantize-strict-affine-u4", 5},
    {"tiler_dequantize_u4_f32_v4_slots", "dequantize-strict-affine-u4", 5},
    {"tiler_dequantize_u4_f32_slots", "dequantize-strict-affine-u4", 5},
    {"tiler_contract_strict_f32", "tensor-contraction-f32/strict", 3},
    {"tiler_contract_strict_f32_b16", "tensor-contraction-f32/strict", 3},
    {"tiler_contract_strict_f32_b32", "tensor-contraction-f32/strict", 3},
    {"tiler_contract_strict_f32_b64", "tensor-contraction-f32/strict", 3},
    {"tiler_contract_strict_f32_s1", "tensor-contraction-f32/strict", 3},
    {"tiler_contract_strict_f32_s1_u", "tensor-contraction-f32/strict", 3},
    {"tiler_contract_strict_f32_s4", "tensor-contraction-f32/strict", 3},
    {"tiler_contract_strict_f32_s4_u", "tensor-contraction-f32/strict", 3},
    {"tiler_contract_strict_f32_s16", "tensor-contraction-f32/strict", 3},
    {"tiler_contract_strict_f32_s16_u", "tensor-contraction-f32/strict", 3},
    {"tiler_contract_strict_f32_s64", "tensor-contraction-f32/strict", 3},
    {"tiler_contract_strict_f32_s64_u", "tensor-contraction-f32/strict", 3},
    {"tiler_contract_strict_bf16", "tensor-contraction-bf16/strict", 3},
    {"tiler_contract_strict_bf16_silu", "tensor-contraction-bf16/strict+silu", 3},
    {"tiler_contract_strict_bf16_b16", "tensor-contraction-bf16/strict", 3},
    {"tiler_contract_strict_bf16_b32", "tensor-contraction-bf16/strict", 3},
    {"tiler_contract_strict_bf16_b64", "tensor-contraction-bf16/strict", 3},
    {"tiler_contract_strict_bf16_silu_b16", "tensor-contraction-bf16/strict+silu", 3},
    {"tiler_contract_strict_bf16_silu_b32", "tensor-contraction-bf16/strict+silu", 3},
    {"tiler_contract_strict_bf16_silu_b64", "tensor-contraction-bf16/strict+silu", 3},
    {"tiler_rms_norm_f32_strict", "rms-norm-f32/strict", 3},
    {"tiler_rms_norm_bf16_strict", "rms-norm/bf16/strict", 3},
    {"tiler_rms_norm_f32_strict_r1", "rms-norm-f32/strict", 3},
    {"tiler_rms_norm_f32_strict_r1_u", "rms-norm-f32/strict", 3},
    {"tiler_rms_norm_f32_strict_r4", "rms-norm-f32/strict", 3},
    {"tiler_rms_norm_f32_strict_r4_u", "rms-norm-f32/strict", 3},
    {"tiler_rms_norm_f32_strict_r16", "rms-norm-f32/strict", 3},
    {"tiler_rms_norm_f32_strict_r16_u", "rms-norm-f32/strict", 3},
    {"tiler_rms_norm_f32_strict_r64", "rms-norm-f32/strict", 3},
    {"tiler_rms_norm_f32_strict_r64_u", "rms-norm-f32/strict", 3},
    {"tiler_rms_norm_bf16_strict_r1", "rms-norm/bf16/strict", 3},
    {"tiler_rms_norm_bf16_strict_r1_u", "rms-norm/bf16/strict", 3},
    {"tiler_rms_norm_bf16_strict_r4", "rms-norm/bf16/strict", 3},
    {"tiler_rms_norm_bf16_strict_r4_u", "rms-norm/bf16/strict", 3},
    {"tiler_rms_norm_bf16_strict_r16", "rms-norm/bf16/strict", 3},
    {"tiler_rms_norm_bf16_strict_r16_u", "rms-norm/bf16/strict", 3},
    {"tiler_rms_norm_bf16_strict_r64", "rms-norm/bf16/strict", 3},
    {"tiler_rms_norm_bf16_strict_r64_u", "rms-norm/bf16/strict", 3},
    {"tiler_rms_norm_f32_strict_rr8_p8", "rms-norm-f32/strict", 3},
    {"tiler_rms_norm_f32_strict_rr8_p16", "rms-norm-f32/strict", 3},
    {"tiler_rms_norm_bf16_strict_rr8_p8", "rms-norm/bf16/strict", 3},
    {"tiler_rms_norm_bf16_strict_rr8_p16", "rms-norm/bf16/strict", 3},
    {"tiler_rms_norm_f32_strict_rr8_p8_m", "rms-norm-f32/strict", 3},
    {"tiler_rms_norm_f32_strict_rr8_p16_m", "rms-norm-f32/strict", 3},
    {"tiler_rms_norm_bf16_strict_rr8_p8_m", "rms-norm/bf16/strict", 3},
    {"tiler_rms_norm_bf16_strict_rr8_p16_m", "rms-norm/bf16/strict", 3},
    {"tiler_softmax_f32_strict", "softmax-f32/strict", 2},
    {"tiler_softmax_f32_strict_r1", "softmax-f32/strict", 2},
    {"tiler_softmax_f32_strict_r1_u", "softmax-f32/strict", 2},
    {"tiler_softmax_f32_strict_r4", "softmax-f32/strict", 2},
    {"tiler_softmax_f32_strict_r4_u", "softmax-f32/strict", 2},
    {"tiler_softmax_f32_strict_r16", "softmax-f32/strict", 2},
    {"tiler_softmax_f32_strict_r16_u", "softmax-f32/strict", 2},
    {"tiler_softmax_f32_strict_rr8_p16", "softmax-f32/strict", 2},
    {"tiler_softmax_f32_strict_rr8_p8", "softmax-f32/strict", 2},
    {"tiler_softmax_f32_strict_rr8_p16_m", "softmax-f32/strict", 2},
    {"tiler_softmax_f32_strict_rr8_p8_m", "softmax-f32/strict", 2},
    {"tiler_softmax_f32_strict_rr8_p32", "softmax-f32/strict", 2},
    {"tiler_softmax_f32_strict_rr8_p32_m", "softmax-f32/strict", 2},
    {"tiler_rms_norm_f32_strict_r1_m", "rms-norm-f32/strict", 3},
    {"tiler_rms_norm_f32_strict_r1_u_m", "rms-norm-f32/strict", 3},
    {"tiler_rms_norm_f32_strict_r4_m", "rms-norm-f32/strict", 3},
    {"tiler_rms_norm_f32_strict_r4_u_m", "rms-norm-f32/strict", 3},
    {"tiler_rms_norm_f32_strict_r16_m", "rms-norm-f32/strict", 3},
    {"tiler_rms_norm_f32_strict_r16_u_m", "rms-norm-f32/strict", 3},
    {"tiler_rms_norm_f32_strict_r64_m", "rms-norm-f32/strict", 3},
    {"tiler_rms_norm_f32_strict_r64_u_m", "rms-norm-f32/strict", 3},
    {"tiler_rms_norm_bf16_strict_r1_m", "rms-norm/bf16/strict", 3},
    {"tiler_rms_norm_bf16_strict_r1_u_m", "rms-norm/bf16/strict", 3},
    {"tiler_rms_norm_bf16_strict_r4_m", "rms-norm/bf16/strict", 3},
    {"tiler_rms_norm_bf16_strict_r4_u_m", "rms-norm/bf16/strict", 3},
    {"tiler_rms_norm_bf16_strict_r16_m", "rms-norm/bf16/strict", 3},
    {"tiler_rms_norm_bf16_strict_r16_u_m", "rms-norm/bf16/strict", 3},
    {"tiler_rms_norm_bf16_strict_r64_m", "rms-norm/bf16/strict", 3},
    {"tiler_rms_norm_bf16_strict_r64_u_m", "rms-norm/bf16/strict", 3},
    {"tiler_softmax_f32_strict_r1_m", "softmax-f32/strict", 2},
    {"tiler_softmax_f32_strict_r1_u_m", "softmax-f32/strict", 2},
    {"tiler_softmax_f32_strict_r4_m", "softmax-f32/strict", 2},
    {"tiler_softmax_f32_strict_r4_u_m", "softmax-f32/strict", 2},
    {"tiler_softmax_f32_strict_r16_m", "softmax-f32/strict", 2},
    {"tiler_softmax_f32_strict_r16_u_m", "softmax-f32/strict", 2},
    {"tiler_fold_sum_f32", "strict-serial-sum-f32/serial-any-axes", 3},
    {"tiler_fold_squared_f32", "squared-serial-sum-f32/serial", 3},
    {"tiler_fold_fma_f32", "fused-multiply-add-serial-sum-f32/serial", 3},
    {"tiler_fold_maximum_f32", "strict-serial-maximum-f32/serial", 3},
#define TILER_EXPR_ROWS(TY, FAM)                                                                  \
  {"tiler_expr_" TY "_r16_i0", FAM, 18}, {"tiler_expr_" TY "_r16_i1", FAM, 18},                     \
      {"tiler_expr_" TY "_r16_i2", FAM, 18}, {"tiler_expr_" TY "_r16_i3", FAM, 18},                 \
      {"tiler_expr_" TY "_r16_i4", FAM, 18}, {"tiler_expr_" TY "_r16s_i0", FAM, 18},                \
      {"tiler_expr_" TY "_r16s_i1", FAM, 18}, {"tiler_expr_" TY "_r16s_i2", FAM, 18},               \
      {"tiler_expr_" TY "_r16s_i3", FAM, 18}, {"tiler_expr_" TY "_r16s_i4", FAM, 18},               \
      {"tiler_expr_" TY "_mem", FAM, 19}
    TILER_EXPR_ROWS("f32", "pointwise-f32-expression"),
    TILER_EXPR_ROWS("bf16", "pointwise-bf16-expression"),
    {"tiler_expr_f32_r16f_i0", "pointwise-f32-expression", 18},
    {"tiler_expr_f32_r16f_i1", "pointwise-f32-expression", 18},
    {"tiler_expr_f32_r16f_i2", "pointwise-f32-expression", 18},
    {"tiler_expr_f32_r16f_i3", "pointwise-f32-expression", 18},
    {"tiler_expr_f32_r16f_i4", "pointwise-f32-expression", 18},
#undef TILER_EXPR_ROWS
    {"tiler_contract_bf16_g128", "tensor-contraction-bf16/cooperative", 3},
    {"tiler_contract_bf16_silu_g128", "tensor-contraction-bf16/cooperative+silu", 3},
    {"tiler_contract_bf16_g128_k", "tensor-contraction-bf16/cooperative", 3},
    {"tiler_contract_bf16_silu_g128_k", "tensor-contraction-bf16/cooperative+silu", 3},
    {"tiler_contract_bf16_skinny1", "tensor-contraction-bf16/cooperative", 3},
    {"tiler_contract_bf16_silu_skinny1", "tensor-contraction-bf16/cooperative+silu", 3},
    {"tiler_contract_bf16_skinny2", "tensor-contraction-bf16/cooperative", 3},
    {"tiler_contract_bf16_silu_skinny2", "tensor-contraction-bf16/cooperative+silu", 3},
    {"tiler_contract_bf16_skinny3", "tensor-contraction-bf16/cooperative", 3},
    {"tiler_contract_bf16_silu_skinny3", "tensor-contraction-bf16/cooperative+silu", 3},
    {"tiler_contract_bf16_skinny4", "tensor-contraction-bf16/cooperative", 3},
    {"tiler_contract_bf16_silu_skinny4", "tensor-contraction-bf16/cooperative+silu", 3},
    {"tiler_contract_bf16_t128", "tensor-contraction-bf16/cooperative", 3},
    {"tiler_contract_bf16_silu_t128", "tensor-contraction-bf16/cooperative+silu", 3},
    {"tiler_contract_bf16_t256", "tensor-contraction-bf16/cooperative", 3},
    {"tiler_contract_bf16_silu_t256", "tensor-contraction-bf16/cooperative+silu", 3},
    {"tiler_contract_bf16_t128_kf", "tensor-contraction-bf16/cooperative", 3},
    {"tiler_contract_bf16_silu_t128_kf", "tensor-contraction-bf16/cooperative+silu", 3},
    {"tiler_contract_bf16_t256_kf", "tensor-contraction-bf16/cooperative", 3},
    {"tiler_contract_bf16_silu_t256_kf", "tensor-contraction-bf16/cooperative+silu", 3},
    // general index structures: the strict fold (geometry in a constant slot),
    // the batched MFMA forms and the right-operand transpose ahead of them
    {"tiler_contract_general_f32", "tensor-contraction-f32/strict-general", 4},
    {"tiler_contract_general_bf16", "tensor-contraction-bf16/strict-general", 4},
    {"tiler_contract_general_bf16_silu", "tensor-contraction-bf16/strict-general+silu", 4},
    {"tiler_transpose_bf16", "tensor-contraction-bf16/transpose", 2},
#define TILER_BATCHED_ROWS(K)                                                                        \
  {"tiler_contract_bf16_" K "_b", "tensor-contraction-bf16/cooperative-batched", 3},                  \
      {"tiler_contract_bf16_silu_" K "_b", "tensor-contraction-bf16/cooperative-batched+silu", 3}
    TILER_BATCHED_ROWS("t256"), TILER_BATCHED_ROWS("t128"), TILER_BATCHED_ROWS("skinny1"),
    TILER_BATCHED_ROWS("skinny2"), TILER_BATCHED_ROWS("skinny3"), TILER_BATCHED_ROWS("skinny4"),
    TILER_BATCHED_ROWS("g128"), TILER_BATCHED_ROWS("g128_k"),
#undef TILER_BATCHED_ROWS
};
constexpr uint32_t kEntryCount = sizeof(kEntries) / sizeof(kEntries[0]);

// The payload entry named `symbol`, or kEntryCount.
uint32_t entry_index(const char* symbol) {
  for (uint32_t k = 0; k < kEntryCount; ++k)
    if (std::strcmp(kEntries[k].symbol, symbol) == 0) return k;
  return kEntryCount;
}

constexpr uint32_t kMaxSumWorkgroups = tiler_rt::kMaxSumWorkgroups;
constexpr uint32_t kProfileComputeUnits = 256;

void copy_text(char* dst, uint64_t cap, const std::string& s) {
  if (!dst || cap == 0) return;
  uint64_t n = s.size() < cap - 1 ? s.size() : cap - 1;
  std::memcpy(dst, s.data(), n);
  dst[n] = 0;
}

uint64_t code_object_bytes() {
  return (uint64_t)(tiler_hip_code_object_end - tiler_hip_code_object);
}

}  // namespace

struct tiler_hip_context {
  int device = -1;
  hipStream_t stream = nullptr;
  hipModule_t module = nullptr;
  std::unordered_map<std::string, hipFunction_t> fns;
  std::vector<hipModule_t> routed_modules;
  std::vector<hipFunction_t> prepared;
  // workspace: [partials kWorkspacePartialBytes][gather_bad u64 + pad]
  //            [row-synchronized softmax area kRowSyncBytes: epoch, tagged words]
  uint8_t* workspace = nullptr;
  float* sum_partials = nullptr;
  unsigned long long* gather_bad = nullptr;
  uint8_t* row_sync = nullptr;
  // The row-synchronized softmax's wait bound (100 MHz ticks): the
  // TILER_HIP_ROW_SYNC_WAIT_TICKS environment variable at bind, else 200 us.
  // 0 makes every workgroup compute its row's maximum and sum from the row.
  uint64_t row_sync_wait_ticks = tiler_rt::kRowSyncDefaultWaitTicks;
  uint32_t compute_units = 0;
  uint64_t lds_bytes = 0;
  uint32_t max_threads = 0;
  uint64_t global_bytes = 0;
  uint32_t max_grid[3] = {0, 0, 0};
  int32_t input_subnormals = -1, result_subnormals = -1;  // measured on first query
  std::string arch;
  std::string diag;
  // Device copies of the expression register programs direct calls ran,
  // keyed by their bytes (freed at release).
  std::unordered_map<std::string, void*> expression_programs;
  // This device's copy of the no-allocation entry point's static scratch
  // array (noalloc.hip), resolved at bind; null if resolution failed
  // (noalloc_error holds the HIP error).
  void* noalloc_scratch = nullptr;
  int noalloc_error = 0;
};

namespace {

tiler_hip_status fail(tiler_hip_context* ctx, tiler_hip_status st, const std::string& what) {
  if (ctx) ctx->diag = what;
  return st;
}

hipStream_t pick(tiler_hip_context* ctx, tiler_hip_stream s) {
  return s ? static_cast<hipStream_t>(s) : ctx->stream;
}

// The context workspace (the tree and split partials, the row-synchronized
// softmax's words, the gather record) is ordered by the context's own stream
// only.  A call that would bind it on another stream could overlap a call on
// the context stream and corrupt both with no status, so it refuses before
// anything is enqueued (the single ordered stream of
// docs/decisions/0090-...md:152-154, where every unsupported case is refused).
tiler_hip_status workspace_stream(tiler_hip_context* ctx, tiler_hip_stream s, const char* what) {
  if (s && static_cast<hipStream_t>(s) != ctx->stream)
    return fail(ctx, TILER_HIP_REFUSE_UNSUPPORTED,
                std::string(what) + " binds the context workspace, which only the context's own stream orders");
  return TILER_HIP_OK;
}

hipFunction_t fn(tiler_hip_context* ctx, const char* symbol) {
  auto it = ctx->fns.find(symbol);
  return it == ctx->fns.end() ? nullptr : it->second;
}

tiler_hip_status launch(tiler_hip_context* ctx, const char* symbol, uint32_t gx, uint32_t gy,
                        uint32_t bx, hipStream_t s, void** args) {
  hipFunction_t f = fn(ctx, symbol);
  if (!f) return fail(ctx, TILER_HIP_REFUSE_NOT_PREPARED, std::string("kernel not loaded: ") + symbol);
  if (gx == 0 || gy == 0) return TILER_HIP_OK;
  hipError_t e = hipModuleLaunchKernel(f, gx, gy, 1, bx, 1, 1, 0, s, args, nullptr);
  if (e != hipSuccess)
    return fail(ctx, TILER_HIP_FAIL_LAUNCH,
                std::string("hipModuleLaunchKernel(") + symbol + "): " + hipGetErrorString(e));
  return TILER_HIP_OK;
}

// Rows longer than one wave holds run one workgroup per row, softmax's by
// segments (the grouping tiler_hip_row_grouping reports).
using tiler_rt::kWaveRowMax;

// Every live extent is a 32-bit launch field inside the range its
// realization's slots were sized for (callers check extent_ranges first).
bool live_extent_in_range(const tiler_hip_dispatch_plan* plan, uint32_t x) {
  const uint64_t v = plan->extents[x];
  return v <= 0xffffffffull && v >= plan->extent_ranges[x].minimum && v <= plan->extent_ranges[x].bound;
}

// Partials beyond the workspace are allocated on the stream; under graph
// capture that would record an allocation node, so such calls refuse there.
bool capturing(hipStream_t s) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(s, &st) == hipSuccess && st != hipStreamCaptureStatusNone;
}

tiler_rt::Target target_of(const tiler_hip_context* ctx) {
  return tiler_rt::Target{ctx ? ctx->compute_units : kProfileComputeUnits,
                          ctx ? ctx->row_sync_wait_ticks : tiler_rt::kRowSyncDefaultWaitTicks};
}

// Runs a planned program on `s`: slot addresses (plus each binding's offset)
// patched into a copy of every launch's argument segment, launched in order.
tiler_hip_status run_program(tiler_hip_context* ctx, const tiler_rt::Program& p, void* const* slots,
                             hipStream_t s) {
  for (uint32_t i = 0; i < p.nlaunches; ++i) {
    const tiler_rt::Launch& l = p.launches[i];
    if (l.overflow) return fail(ctx, TILER_HIP_REFUSE_UNSUPPORTED, std::string("argument segment overflow: ") + l.symbol);
    hipFunction_t f = fn(ctx, l.symbol);
    if (!f) return fail(ctx, TILER_HIP_REFUSE_NOT_PREPARED, std::string("kernel not loaded: ") + l.symbol);
    if (l.grid[0] == 0 || l.grid[1] == 0) continue;
    uint8_t args[tiler_rt::kMaxKernargBytes];
    std::memcpy(args, l.kernargs, l.kernarg_bytes);
    for (uint32_t b = 0; b < l.nbindings; ++b) {
      char* base = static_cast<char*>(slots[l.bindings[b].slot]);
      char* ptr = base ? base + l.bindings[b].addend : nullptr;
      std::memcpy(args + l.bindings[b].offset, &ptr, sizeof(ptr));
    }
    void* params[tiler_rt::kMaxArgs];
    for (uint32_t a = 0; a < l.nargs; ++a) params[a] = args + l.arg_offsets[a];
    hipError_t e = hipModuleLaunchKernel(f, l.grid[0], l.grid[1], 1, l.block, 1, 1, 0, s, params, nullptr);
    if (e != hipSuccess)
      return fail(ctx, TILER_HIP_FAIL_LAUNCH,
                  std::string("hipModuleLaunchKernel(") + l.symbol + "): " + hipGetErrorString(e));
  }
  return TILER_HIP_OK;
}

}  // namespace

extern "C" {

// ---------------------------------------------------------------------------
tiler_hip_status tiler_hip_profile_declare(tiler_hip_target_profile* out) try {
  if (!out) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  std::memset(out, 0, sizeof(*out));
  copy_text(out->profile_key, sizeof(out->profile_key), kProfileKey);
  copy_text(out->target_triple, sizeof(out->target_triple), kTarget);
  out->wavefront_size = 64;
  out->compute_units = kProfileComputeUnits;
  out->xcds = 8;
  out->simds_per_cu = 4;
  out->max_threads_per_workgroup = 1024;
  out->max_grid_dim[0] = 0x7fffffffu;
  out->max_grid_dim[1] = 65535;
  out->max_grid_dim[2] = 65535;
  out->lds_bytes_per_workgroup = 163840;
  out->device_memory_bytes = 288ull * 1000 * 1000 * 1000;
  out->l2_bytes_per_xcd = 4ull << 20;
  out->infinity_cache_bytes = 256ull << 20;
  out->address_bits = 64;
  out->index_u64 = 1;
  out->subgroup_width = 64;
  out->f32_subnormals_preserved = 1;
  out->hbm_bytes_per_second = 8.0e12;
  out->mfma_bf16_dense_flops = 2.5e15;
  out->mfma_fp8_dense_flops = 5.0e15;
  out->vector_f32_flops = 157.3e12;
  out->vector_f64_flops = 78.6e12;
  // Fitted P of cost = sum over stages (encoder + max(work / P, depth) * step)
  // on 22 (rows, extent) cells x 3 sum realizations (serial-or-parallel
  // verdict: 11/12 fit cells, 10/10 held-out cells; the miss, 2.02x, is one
  // row of 1024, where the staged fold's first load is as long as its chain).
  out->saturated_parallel_fold_steps = 17870;
  copy_text(out->cost_row_source, sizeof(out->cost_row_source),
            "measured: AMD Instinct MI355X gfx950:sramecc+:xnack- (256 CUs), ROCm 7.2, 2026-12-02; "
            "python -m tiler_amd.calibrate (profiles/saturated_parallel_fold_steps.md)");
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

// ---------------------------------------------------------------------------
tiler_hip_status tiler_hip_payload(tiler_hip_payload_view* out) try {
  if (!out) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  out->backend = kBackend;
  out->representation = kRepresentation;
  out->payload_schema = kPayloadSchema;
  out->target = kTarget;
  out->toolchain = TILER_HIP_BUILD_TOOLCHAIN;
  out->flags = TILER_HIP_BUILD_FLAGS;
  out->code = tiler_hip_code_object;
  out->code_bytes = code_object_bytes();
  out->entry_count = kEntryCount;
  out->source = tiler_hip_source_bundle;
  out->source_bytes = (uint64_t)(tiler_hip_source_bundle_end - tiler_hip_source_bundle);
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

// The payload's compilation subject in the artifact layer's canonical
// PayloadMetadata encoding (tiler-artifact/src/program/codec/payload.rs:
// 477-580): versioned domain, schema (1, 0) as u16 big-endian, then every
// variable-length run and collection preceded by its u64 big-endian length.
// Field order: source representation, source, toolchain, target, family,
// language, deployment major/minor (u16), components (role, version), SDK
// name/version/build, compile flags, link flags, entries (key, symbol,
// transports as u32), obligations (key, value); the unversioned platform
// appends its tag 0x00.  This payload states no SDK and no deployment
// minimum, like the reference's own unversioned backend
// (tiler-build/tests/custom_backend/backend.rs:420-438).
namespace {

constexpr char kPayloadMetadataDomain[] = "tiler.artifact-envelope.payload-metadata.v1\0";
constexpr char kPayloadIdentityDomain[] = "tiler.artifact-envelope.payload-identity.v1\0";

const std::vector<uint8_t>& payload_metadata_bytes() {
  static const std::vector<uint8_t> bytes = [] {
    using namespace tiler_rt;
    std::vector<uint8_t> b;
    b.insert(b.end(), kPayloadMetadataDomain, kPayloadMetadataDomain + sizeof(kPayloadMetadataDomain) - 1);
    push_u16(b, 1);
    push_u16(b, 0);
    push_str(b, "tiler.hip.source-bundle.v1");
    push_slice(b, tiler_hip_source_bundle, (uint64_t)(tiler_hip_source_bundle_end - tiler_hip_source_bundle));
    push_str(b, "tiler.hip.rocm-clang");
    push_str(b, kTarget);
    push_str(b, kBackend);
    push_str(b, "hip-c++17");
    push_u16(b, 0);  // deployment major: none (unversioned)
    push_u16(b, 0);  // deployment minor
    push_len(b, 1);  // components, in role order
    push_str(b, "compiler");
    push_str(b, TILER_HIP_BUILD_TOOLCHAIN);
    push_str(b, "");  // SDK name, version, build: none
    push_str(b, "");
    push_str(b, "");
    static const char* const flags[] = {TILER_HIP_BUILD_FLAG_LIST};
    push_len(b, TILER_HIP_BUILD_FLAG_COUNT);
    for (const char* f : flags) push_str(b, f);
    push_len(b, 0);  // link flags: the code object is not linked
    std::vector<uint32_t> order(kEntryCount);
    for (uint32_t i = 0; i < kEntryCount; ++i) order[i] = i;
    std::sort(order.begin(), order.end(),
              [](uint32_t x, uint32_t y) { return std::strcmp(kEntries[x].symbol, kEntries[y].symbol) < 0; });
    push_len(b, kEntryCount);  // entries, in entry-key order; the key is the symbol
    for (uint32_t i : order) {
      push_str(b, kEntries[i].symbol);
      push_str(b, kEntries[i].symbol);
      push_len(b, kEntries[i].buffers);
      for (uint32_t t = 0; t < kEntries[i].buffers; ++t) push_u32(b, t);
    }
    push_len(b, 2);  // obligations, in key order
    push_str(b, "tiler.hip.target-arch");
    push_str(b, "gfx950");
    push_str(b, "tiler.hip.wavefront-size");
    push_str(b, "64");
    b.push_back(0x00);  // PayloadPlatform::Unversioned
    return b;
  }();
  return bytes;
}

}  // namespace

tiler_hip_status tiler_hip_payload_metadata(uint8_t* out, uint64_t capacity, uint64_t* required) try {
  const std::vector<uint8_t>& m = payload_metadata_bytes();
  if (required) *required = m.size();
  if (!out) return required ? TILER_HIP_OK : TILER_HIP_REFUSE_INVALID_ARGUMENT;
  if (capacity < m.size()) return TILER_HIP_REFUSE_CAPACITY;
  std::memcpy(out, m.data(), m.size());
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

tiler_hip_status tiler_hip_payload_correspondence(const void* metadata, uint64_t byte_count, char* fact,
                                                  uint64_t fact_bytes) try {
  if (byte_count && !metadata) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  const std::vector<uint8_t>& own = payload_metadata_bytes();
  tiler_rt::PayloadSubject expected, actual;
  std::string why = tiler_rt::read_payload_metadata(own.data(), own.size(), expected, nullptr, 0);
  if (!why.empty()) {  // this library's own record always decodes; say so if it ever does not
    copy_text(fact, fact_bytes, "own metadata: " + why);
    return TILER_HIP_REFUSE_MALFORMED_PAYLOAD;
  }
  why = tiler_rt::read_payload_metadata(static_cast<const uint8_t*>(metadata), byte_count, actual, nullptr, 0);
  if (!why.empty()) {
    copy_text(fact, fact_bytes, why);
    return TILER_HIP_REFUSE_MALFORMED_PAYLOAD;
  }
  const char* first = tiler_rt::first_disagreeing_fact(expected, actual);
  copy_text(fact, fact_bytes, first);
  return first[0] ? TILER_HIP_REFUSE_PAYLOAD_MISMATCH : TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

tiler_hip_status tiler_hip_payload_identity(uint8_t* out) try {
  if (!out) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  const std::vector<uint8_t>& m = payload_metadata_bytes();
  tiler_rt::governed_digest(kPayloadIdentityDomain, sizeof(kPayloadIdentityDomain) - 1, nullptr, nullptr, 0,
                            m.data(), m.size(), out);
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

tiler_hip_status tiler_hip_digest(const void* domain, uint64_t domain_bytes, const void* const* qualifiers,
                                  const uint64_t* qualifier_bytes, uint32_t qualifier_count,
                                  const void* bytes, uint64_t byte_count, uint8_t* out) try {
  if (!out || (domain_bytes && !domain) || (byte_count && !bytes) ||
      (qualifier_count && (!qualifiers || !qualifier_bytes)))
    return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  for (uint32_t i = 0; i < qualifier_count; ++i)
    if (qualifier_bytes[i] && !qualifiers[i]) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  tiler_rt::governed_digest(domain, domain_bytes, qualifiers, qualifier_bytes, qualifier_count, bytes,
                            byte_count, out);
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

tiler_hip_status tiler_hip_payload_entry(uint32_t index, tiler_hip_entry_info* out) try {
  if (!out || index >= kEntryCount) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  tiler_hip::KernelDescriptorFacts facts;
  bool absent = false;
  std::string why = tiler_hip::inspect_code_object(tiler_hip_code_object, code_object_bytes(),
                                                   kEntries[index].symbol, &facts, &absent);
  if (!why.empty()) return absent ? TILER_HIP_REFUSE_ABSENT_SYMBOL : TILER_HIP_REFUSE_MALFORMED_PAYLOAD;
  out->symbol = kEntries[index].symbol;
  out->family = kEntries[index].family;
  out->buffer_bindings = kEntries[index].buffers;
  out->kernarg_bytes = facts.kernarg_bytes;
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

tiler_hip_status tiler_hip_validate_payload(const void* code, uint64_t code_bytes,
                                            const char* symbol, uint32_t kernarg_bytes,
                                            char* diagnostic, uint64_t diagnostic_bytes) try {
  tiler_hip::KernelDescriptorFacts facts;
  bool absent = false;
  std::string why = tiler_hip::inspect_code_object(code, code_bytes, symbol, &facts, &absent);
  if (!why.empty()) {
    copy_text(diagnostic, diagnostic_bytes, why);
    return absent ? TILER_HIP_REFUSE_ABSENT_SYMBOL : TILER_HIP_REFUSE_MALFORMED_PAYLOAD;
  }
  if (symbol && kernarg_bytes != 0 && facts.kernarg_bytes != kernarg_bytes) {
    copy_text(diagnostic, diagnostic_bytes,
              "kernel " + std::string(symbol) + " takes " + std::to_string(facts.kernarg_bytes) +
                  " kernarg bytes, the entry declares " + std::to_string(kernarg_bytes));
    return TILER_HIP_REFUSE_BINDING_MISMATCH;
  }
  copy_text(diagnostic, diagnostic_bytes, "");
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

tiler_hip_status tiler_hip_read_envelope(const void* bytes, uint64_t byte_count, tiler_hip_envelope* out,
                                         char* diagnostic, uint64_t diagnostic_bytes) try {
  if (!out || (byte_count && !bytes)) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  static_assert(tiler_rt::kMaxEnvelopeSections == sizeof(out->section_purpose), "section table width");
  static_assert(tiler_rt::kMaxEnvelopePayloads == sizeof(out->payloads) / sizeof(out->payloads[0]),
                "payload table width");
  std::memset(out, 0, sizeof(*out));
  auto* e = new (std::nothrow) tiler_rt::Envelope();  // ~2 KB of spans; kept off small host stacks
  if (!e) return TILER_HIP_REFUSE_CAPACITY;
  const std::string why = tiler_rt::read_envelope(static_cast<const uint8_t*>(bytes), byte_count, *e);
  copy_text(diagnostic, diagnostic_bytes, why);
  if (why.empty()) {
    out->total_bytes = e->total_bytes;
    out->manifest_bytes = e->manifest_bytes;
    out->manifest_schema_major = e->manifest_major;
    out->manifest_schema_minor = e->manifest_minor;
    out->section_count = e->section_count;
    std::memcpy(out->section_purpose, e->section_kind, sizeof(out->section_purpose));
    out->feature_count = e->feature_count;
    out->input_count = e->input_count;
    out->output_count = e->output_count;
    out->provider_count = e->provider_count;
    out->payload_count = e->payload_count;
    for (uint32_t i = 0; i < e->payload_count; ++i) {
      const tiler_rt::EnvelopePayload& p = e->payloads[i];
      tiler_hip_envelope_payload& o = out->payloads[i];
      o.backend = p.backend.p, o.backend_bytes = p.backend.n;
      o.representation = p.representation.p, o.representation_bytes = p.representation.n;
      o.payload_schema_major = p.schema_major, o.payload_schema_minor = p.schema_minor;
      o.digest = p.digest.p, o.digest_bytes = p.digest.n;
      o.profile_key = p.profile_key.p, o.profile_key_bytes = p.profile_key.n;
      o.profile_descriptor = p.profile_descriptor.p, o.profile_descriptor_bytes = p.profile_descriptor.n;
      o.has_environment = p.has_environment;
      o.carried = p.carried;
      o.metadata_section = p.metadata_section, o.code_section = p.code_section;
      o.metadata = p.metadata.p, o.metadata_bytes = p.metadata.n;
      o.code = p.code.p, o.code_bytes = p.code.n;
    }
    std::memcpy(out->identity_digest, e->identity_digest, 32);
  }
  delete e;
  return why.empty() ? TILER_HIP_OK : TILER_HIP_REFUSE_MALFORMED_PAYLOAD;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

tiler_hip_status tiler_hip_read_payload_metadata(const void* bytes, uint64_t byte_count,
                                                 tiler_hip_payload_subject* out,
                                                 tiler_hip_payload_mapping* mappings, uint32_t capacity,
                                                 char* diagnostic, uint64_t diagnostic_bytes) try {
  if (!out || (byte_count && !bytes) || (capacity && !mappings)) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  std::memset(out, 0, sizeof(*out));
  tiler_rt::PayloadSubject s;
  std::vector<tiler_rt::PayloadMapping> m;
  try {
    m.resize(capacity);
  } catch (...) {
    return TILER_HIP_REFUSE_CAPACITY;
  }
  const std::string why =
      tiler_rt::read_payload_metadata(static_cast<const uint8_t*>(bytes), byte_count, s, m.data(), capacity);
  copy_text(diagnostic, diagnostic_bytes, why);
  if (!why.empty()) return TILER_HIP_REFUSE_MALFORMED_PAYLOAD;
  out->source_representation = s.source_representation.p;
  out->source_representation_bytes = s.source_representation.n;
  out->source = s.source.p, out->source_bytes = s.source.n;
  out->toolchain = s.toolchain.p, out->toolchain_bytes = s.toolchain.n;
  out->target = s.target.p, out->target_bytes = s.target.n;
  out->family = s.family.p, out->family_bytes = s.family.n;
  out->language = s.language.p, out->language_bytes = s.language.n;
  out->deployment_major = s.deployment_major, out->deployment_minor = s.deployment_minor;
  out->unversioned = s.unversioned;
  out->component_count = s.component_count;
  out->compile_flag_count = s.compile_flag_count;
  out->link_flag_count = s.link_flag_count;
  out->obligation_count = s.obligation_count;
  out->entry_count = s.entry_count;
  const uint64_t n = s.entry_count < capacity ? s.entry_count : capacity;
  for (uint64_t i = 0; i < n; ++i) {
    mappings[i].key = m[i].key.p, mappings[i].key_bytes = m[i].key.n;
    mappings[i].symbol = m[i].symbol.p, mappings[i].symbol_bytes = m[i].symbol.n;
    mappings[i].transport_count = (uint32_t)m[i].transport_count;
    mappings[i].transports = m[i].transports.p;
  }
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

namespace {
tiler_hip_status select_payload(const tiler_hip_envelope* envelope, uint32_t* index, char* diagnostic,
                                uint64_t diagnostic_bytes);
}  // namespace

tiler_hip_status tiler_hip_select_payload(const tiler_hip_envelope* envelope, uint32_t* index,
                                          char* diagnostic, uint64_t diagnostic_bytes) try {
  try {
    return select_payload(envelope, index, diagnostic, diagnostic_bytes);
  } catch (...) {  // allocation failure: nothing crosses the C ABI
    return TILER_HIP_REFUSE_CAPACITY;
  }
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

namespace {
tiler_hip_status select_payload(const tiler_hip_envelope* envelope, uint32_t* index, char* diagnostic,
                                uint64_t diagnostic_bytes) {
  if (!envelope || !index || envelope->payload_count > 16) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  auto is = [](const uint8_t* p, uint64_t n, const char* s) {
    return n == std::strlen(s) && (n == 0 || std::memcmp(p, s, n) == 0);
  };
  std::string seen;
  for (uint32_t i = 0; i < envelope->payload_count; ++i) {
    const tiler_hip_envelope_payload& p = envelope->payloads[i];
    if (!seen.empty()) seen += ", ";
    seen += std::string((const char*)p.backend, p.backend_bytes) + "/" +
            std::string((const char*)p.representation, p.representation_bytes);
    if (!p.carried || !is(p.backend, p.backend_bytes, kBackend) ||
        !is(p.representation, p.representation_bytes, kRepresentation) || p.payload_schema_major != 1)
      continue;
    tiler_rt::PayloadSubject s;
    if (!tiler_rt::read_payload_metadata(p.metadata, p.metadata_bytes, s, nullptr, 0).empty()) continue;
    if (!is(s.target.p, s.target.n, kTarget)) continue;
    *index = i;
    copy_text(diagnostic, diagnostic_bytes, "");
    return TILER_HIP_OK;
  }
  copy_text(diagnostic, diagnostic_bytes,
            "no carried " + std::string(kBackend) + " payload for " + kTarget +
                (seen.empty() ? std::string(" (the envelope names no payloads)") : " among: " + seen));
  return TILER_HIP_REFUSE_FOREIGN_TARGET;
}
}  // namespace

// ---------------------------------------------------------------------------
tiler_hip_status tiler_hip_bind(int32_t ordinal, tiler_hip_context** out,
                                tiler_hip_execution_environment* env, char* diagnostic,
                                uint64_t diagnostic_bytes) try {
  if (!out) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  *out = nullptr;
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
    copy_text(diagnostic, diagnostic_bytes, "no HIP device is visible");
    return TILER_HIP_REFUSE_NO_DEVICE;
  }
  if (ordinal < 0 || ordinal >= count) {
    copy_text(diagnostic, diagnostic_bytes, "device ordinal out of range");
    return TILER_HIP_REFUSE_NO_DEVICE;
  }
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, ordinal) != hipSuccess) {
    copy_text(diagnostic, diagnostic_bytes, "hipGetDeviceProperties failed");
    return TILER_HIP_REFUSE_NO_DEVICE;
  }
  std::string arch = prop.gcnArchName;
  if (arch.rfind("gfx950", 0) != 0) {
    copy_text(diagnostic, diagnostic_bytes, "device is " + arch + ", this backend targets gfx950");
    return TILER_HIP_REFUSE_FOREIGN_TARGET;
  }
  if (hipSetDevice(ordinal) != hipSuccess) {
    copy_text(diagnostic, diagnostic_bytes, "hipSetDevice failed");
    return TILER_HIP_REFUSE_NO_DEVICE;
  }
  auto* ctx = new tiler_hip_context();
  ctx->device = ordinal;
  ctx->arch = arch;
  ctx->compute_units = (uint32_t)prop.multiProcessorCount;
  ctx->lds_bytes = prop.sharedMemPerBlock;
  ctx->max_threads = (uint32_t)prop.maxThreadsPerBlock;
  ctx->global_bytes = prop.totalGlobalMem;
  for (int d = 0; d < 3; ++d) ctx->max_grid[d] = (uint32_t)prop.maxGridSize[d];
  hipError_t e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipModuleLoadData(&ctx->module, tiler_hip_code_object);
  if (e != hipSuccess) {
    copy_text(diagnostic, diagnostic_bytes, std::string("loading the gfx950 code object: ") + hipGetErrorString(e));
    if (ctx->stream) hipStreamDestroy(ctx->stream);
    delete ctx;
    return TILER_HIP_REFUSE_MALFORMED_PAYLOAD;
  }
  for (uint32_t i = 0; i < kEntryCount; ++i) {
    hipFunction_t f = nullptr;
    if (hipModuleGetFunction(&f, ctx->module, kEntries[i].symbol) != hipSuccess || !f) {
      copy_text(diagnostic, diagnostic_bytes, std::string("absent entry symbol ") + kEntries[i].symbol);
      hipModuleUnload(ctx->module);
      hipStreamDestroy(ctx->stream);
      delete ctx;
      return TILER_HIP_REFUSE_ABSENT_SYMBOL;
    }
    ctx->fns[kEntries[i].symbol] = f;
  }
  const uint64_t ws_bytes = tiler_rt::kWorkspacePartialBytes + 256 + tiler_rt::kRowSyncBytes;
  if (hipMalloc(&ctx->workspace, ws_bytes) != hipSuccess) {
    copy_text(diagnostic, diagnostic_bytes, "workspace allocation failed");
    hipModuleUnload(ctx->module);
    hipStreamDestroy(ctx->stream);
    delete ctx;
    return TILER_HIP_REFUSE_CAPACITY;
  }
  ctx->sum_partials = reinterpret_cast<float*>(ctx->workspace);
  ctx->gather_bad = reinterpret_cast<unsigned long long*>(ctx->workspace + tiler_rt::kWorkspacePartialBytes);
  ctx->row_sync = ctx->workspace + tiler_rt::kWorkspacePartialBytes + 256;
  if (const char* w = std::getenv("TILER_HIP_ROW_SYNC_WAIT_TICKS")) ctx->row_sync_wait_ticks = std::strtoull(w, nullptr, 10);
  hipMemset(ctx->workspace, 0, ws_bytes);
  hipMemset(ctx->gather_bad, 0xff, 8);
  hipDeviceSynchronize();
  // The no-allocation entry point's scratch: this device's address of the
  // static array, resolved once here with the device current.
  ctx->noalloc_error = tiler_hip_noalloc_scratch_address(&ctx->noalloc_scratch);
  if (ctx->noalloc_error != 0) ctx->noalloc_scratch = nullptr;
  if (env) {
    std::memset(env, 0, sizeof(*env));
    env->device_ordinal = ordinal;
    copy_text(env->device_name, sizeof(env->device_name), prop.name);
    copy_text(env->gcn_arch_name, sizeof(env->gcn_arch_name), arch);
    env->compute_units = ctx->compute_units;
    env->wavefront_size = (uint32_t)prop.warpSize;
    env->max_threads_per_workgroup = ctx->max_threads;
    env->lds_bytes_per_workgroup = ctx->lds_bytes;
    env->global_memory_bytes = ctx->global_bytes;
    env->clock_khz = prop.clockRate;
    env->memory_clock_khz = prop.memoryClockRate;
    env->memory_bus_width_bits = prop.memoryBusWidth;
    int rv = 0, dv = 0;
    hipRuntimeGetVersion(&rv);
    hipDriverGetVersion(&dv);
    env->runtime_version = rv;
    env->driver_version = dv;
  }
  copy_text(diagnostic, diagnostic_bytes, "");
  *out = ctx;
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

void tiler_hip_release(tiler_hip_context* ctx) {
  if (!ctx) return;
  hipSetDevice(ctx->device);
  if (ctx->stream) hipStreamSynchronize(ctx->stream);
  for (hipModule_t m : ctx->routed_modules) hipModuleUnload(m);
  for (auto& kv : ctx->expression_programs) hipFree(kv.second);
  if (ctx->module) hipModuleUnload(ctx->module);
  if (ctx->workspace) hipFree(ctx->workspace);
  if (ctx->stream) hipStreamDestroy(ctx->stream);
  delete ctx;
}

const char* tiler_hip_last_diagnostic(const tiler_hip_context* ctx) {
  return ctx ? ctx->diag.c_str() : "";
}

namespace {

// Subnormal modes, as the reference names them (conformance.rs:269-521):
// 1 preserve, 2 flush to a zero of the same sign, 3 flush to +0; 0 a pattern
// none of them produces.
uint32_t subnormal_mode(uint32_t bits, uint32_t preserved) {
  if (bits == preserved) return 1;
  if (bits == 0x80000000u) return 2;
  if (bits == 0x00000000u) return 3;
  return 0;
}

// Runs tiler_probe_subnormals once per context on its stream and caches the
// two modes.
tiler_hip_status measure_subnormals(tiler_hip_context* ctx) {
  if (ctx->input_subnormals >= 0) return TILER_HIP_OK;
  const float in[4] = {-0x1p-149f, 0x1p30f, 0x1p-120f, -0x1p-10f};
  uint32_t out[2] = {0, 0};
  void* dev = nullptr;
  if (hipMalloc(&dev, 64) != hipSuccess) return fail(ctx, TILER_HIP_FAIL_ALLOCATION, "probe buffer");
  float* din = static_cast<float*>(dev);
  uint32_t* dout = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(dev) + 32);
  void* args[] = {&din, &dout};
  hipError_t e = hipMemcpyAsync(din, in, sizeof(in), hipMemcpyHostToDevice, ctx->stream);
  tiler_hip_status st = e == hipSuccess ? launch(ctx, "tiler_probe_subnormals", 1, 1, 64, ctx->stream, args)
                                        : TILER_HIP_FAIL_TRANSFER;
  if (st == TILER_HIP_OK && (hipMemcpyAsync(out, dout, sizeof(out), hipMemcpyDeviceToHost, ctx->stream) != hipSuccess ||
                             hipStreamSynchronize(ctx->stream) != hipSuccess))
    st = TILER_HIP_FAIL_TRANSFER;
  hipFree(dev);
  if (st != TILER_HIP_OK) return fail(ctx, st, "subnormal probe");
  ctx->input_subnormals = (int32_t)subnormal_mode(out[0], 0x80000000u | (0x7fu - 119u + 0u) << 23);
  ctx->result_subnormals = (int32_t)subnormal_mode(out[1], 0x80000000u | (1u << (149 - 130)));
  return TILER_HIP_OK;
}

}  // namespace

tiler_hip_status tiler_hip_observe_live_device(tiler_hip_context* ctx, const char* key,
                                               uint64_t* value) try {
  if (!ctx || !key || !value) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  std::string k = key;
  if (k == "f32-input-subnormals" || k == "f32-result-subnormals") {
    const tiler_hip_status st = measure_subnormals(ctx);
    if (st != TILER_HIP_OK) return st;
    *value = (uint64_t)(k == "f32-input-subnormals" ? ctx->input_subnormals : ctx->result_subnormals);
    return TILER_HIP_OK;
  }
  if (k == "wavefront-size") *value = 64;
  else if (k == "compute-units") *value = ctx->compute_units;
  else if (k == "max-threads-per-workgroup") *value = ctx->max_threads;
  else if (k == "lds-bytes-per-workgroup") *value = ctx->lds_bytes;
  else if (k == "global-memory-bytes") *value = ctx->global_bytes;
  else if (k == "target-is-gfx950") *value = ctx->arch.rfind("gfx950", 0) == 0 ? 1 : 0;
  else if (k == "max-grid-x") *value = ctx->max_grid[0];
  else if (k == "max-grid-y") *value = ctx->max_grid[1];
  else if (k == "max-grid-z") *value = ctx->max_grid[2];
  else if (k == "device-address-bits") *value = 64;
  else return fail(ctx, TILER_HIP_REFUSE_UNRECOGNIZED_KEY, "unrecognized live-device key " + k);
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

tiler_hip_status tiler_hip_prepare_entries(tiler_hip_context* ctx,
                                           const tiler_hip_routed_entry* entries, uint32_t count,
                                           uint32_t* first_index) try {
  if (!ctx || (count && !entries)) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  hipSetDevice(ctx->device);
  std::vector<hipModule_t> loaded;
  std::vector<hipFunction_t> fns;
  for (uint32_t i = 0; i < count; ++i) {
    char why[256];
    tiler_hip_status st = tiler_hip_validate_payload(entries[i].code, entries[i].code_bytes,
                                                     entries[i].symbol, 0, why, sizeof(why));
    hipModule_t m = nullptr;
    hipFunction_t f = nullptr;
    if (st == TILER_HIP_OK && hipModuleLoadData(&m, entries[i].code) != hipSuccess)
      st = TILER_HIP_REFUSE_MALFORMED_PAYLOAD;
    if (st == TILER_HIP_OK && (hipModuleGetFunction(&f, m, entries[i].symbol) != hipSuccess || !f))
      st = TILER_HIP_REFUSE_ABSENT_SYMBOL;
    if (st != TILER_HIP_OK) {
      if (m) hipModuleUnload(m);
      for (hipModule_t mm : loaded) hipModuleUnload(mm);
      return fail(ctx, st, "entry " + std::to_string(i) + " not prepared: " + std::string(why));
    }
    loaded.push_back(m);
    fns.push_back(f);
  }
  if (first_index) *first_index = (uint32_t)ctx->prepared.size();
  ctx->routed_modules.insert(ctx->routed_modules.end(), loaded.begin(), loaded.end());
  ctx->prepared.insert(ctx->prepared.end(), fns.begin(), fns.end());
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

tiler_hip_status tiler_hip_observe_prepared_entry(tiler_hip_context* ctx, uint32_t prepared,
                                                  const char* key, uint64_t* value) try {
  if (!ctx || !key || !value) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  if (prepared >= ctx->prepared.size())
    return fail(ctx, TILER_HIP_REFUSE_NOT_PREPARED, "entry not prepared");
  std::string k = key;
  hipFunction_attribute attr;
  if (k == "max-threads-per-workgroup") attr = HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK;
  else if (k == "static-lds-bytes") attr = HIP_FUNC_ATTRIBUTE_SHARED_SIZE_BYTES;
  else if (k == "private-bytes-per-lane") attr = HIP_FUNC_ATTRIBUTE_LOCAL_SIZE_BYTES;
  else if (k == "vgprs") attr = HIP_FUNC_ATTRIBUTE_NUM_REGS;
  else return fail(ctx, TILER_HIP_REFUSE_UNRECOGNIZED_KEY, "unrecognized prepared-entry key " + k);
  int v = 0;
  if (hipFuncGetAttribute(&v, attr, ctx->prepared[prepared]) != hipSuccess)
    return fail(ctx, TILER_HIP_REFUSE_NOT_PREPARED, "hipFuncGetAttribute failed");
  *value = (uint64_t)v;
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

tiler_hip_status tiler_hip_plan_dispatch(tiler_hip_context* ctx,
                                         const tiler_hip_dispatch_plan* plan) try {
  if (!ctx || !plan || (plan->entry_count && !plan->entries) ||
      (plan->slot_count && !plan->slot_bytes))
    return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  for (uint32_t s = 0; s < plan->slot_count; ++s)
    if (plan->slot_bytes[s] > ctx->global_bytes)
      return fail(ctx, TILER_HIP_REFUSE_CAPACITY, "slot " + std::to_string(s) + " exceeds device memory");
  for (uint32_t i = 0; i < plan->entry_count; ++i) {
    const tiler_hip_dispatch_entry& e = plan->entries[i];
    if (e.prepared >= ctx->prepared.size())
      return fail(ctx, TILER_HIP_REFUSE_NOT_PREPARED, "entry " + std::to_string(i) + " names an unprepared entry");
    uint64_t threads = (uint64_t)e.block[0] * e.block[1] * e.block[2];
    int maxt = 0;
    hipFuncGetAttribute(&maxt, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, ctx->prepared[e.prepared]);
    if (threads == 0 || threads > (uint64_t)maxt)
      return fail(ctx, TILER_HIP_REFUSE_CAPACITY, "entry " + std::to_string(i) + " workgroup wider than its pipeline admits");
    if (e.grid[0] == 0 || e.grid[1] == 0 || e.grid[2] == 0 || e.grid[0] > 0x7fffffffu || e.grid[1] > 65535 ||
        e.grid[2] > 65535)
      return fail(ctx, TILER_HIP_REFUSE_CAPACITY, "entry " + std::to_string(i) + " grid outside the profile");
    int slds = 0;
    hipFuncGetAttribute(&slds, HIP_FUNC_ATTRIBUTE_SHARED_SIZE_BYTES, ctx->prepared[e.prepared]);
    if ((uint64_t)slds + e.dynamic_lds_bytes > ctx->lds_bytes)
      return fail(ctx, TILER_HIP_REFUSE_CAPACITY, "entry " + std::to_string(i) + " LDS beyond the workgroup limit");
    if (e.binding_count && (!e.binding_slots || !e.binding_offsets))
      return TILER_HIP_REFUSE_INVALID_ARGUMENT;
    for (uint32_t b = 0; b < e.binding_count; ++b) {
      if (e.binding_slots[b] >= plan->slot_count)
        return fail(ctx, TILER_HIP_REFUSE_BINDING_MISMATCH, "binding names an undeclared slot");
      if ((uint64_t)e.binding_offsets[b] + 8 > e.kernarg_bytes)
        return fail(ctx, TILER_HIP_REFUSE_BINDING_MISMATCH, "binding pointer outside the kernarg segment");
    }
    if (e.extent_count && (!e.extent_ids || !e.extent_offsets)) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
    for (uint32_t x = 0; x < e.extent_count; ++x) {
      if (e.extent_ids[x] >= plan->extent_count)
        return fail(ctx, TILER_HIP_REFUSE_BINDING_MISMATCH, "entry reads a live extent the plan does not supply");
      if ((uint64_t)e.extent_offsets[x] + 4 > e.kernarg_bytes)
        return fail(ctx, TILER_HIP_REFUSE_BINDING_MISMATCH, "live extent field outside the kernarg segment");
    }
  }
  if (plan->extent_count && !plan->extents) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  // The ranges are what the realization's slots were sized for; without them
  // a value could not be told from one that reads past its operands.
  if (plan->extent_count && !plan->extent_ranges)
    return fail(ctx, TILER_HIP_REFUSE_INVALID_ARGUMENT, "live extents without the ranges they were sized for");
  for (uint32_t x = 0; x < plan->extent_count; ++x) {
    if (!live_extent_in_range(plan, x))
      return fail(ctx, TILER_HIP_REFUSE_CAPACITY,
                  "live extent " + std::to_string(x) + " = " + std::to_string(plan->extents[x]) +
                      " outside the range the realization was sized for");
  }
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

tiler_hip_status tiler_hip_allocate_dispatch(tiler_hip_context* ctx,
                                             const tiler_hip_dispatch_plan* plan,
                                             void** slot_pointers) try {
  if (!ctx || !plan || (plan->slot_count && !slot_pointers)) return TILER_HIP_FAIL_ALLOCATION;
  hipSetDevice(ctx->device);
  for (uint32_t s = 0; s < plan->slot_count; ++s) {
    if (slot_pointers[s]) continue;
    void* p = nullptr;
    uint64_t bytes = plan->slot_bytes[s] ? plan->slot_bytes[s] : 1;
    if (hipMalloc(&p, bytes) != hipSuccess || !p)
      return fail(ctx, TILER_HIP_FAIL_ALLOCATION, "allocation of slot " + std::to_string(s) + " failed");
    slot_pointers[s] = p;
  }
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

namespace {
// The entries of a planned dispatch, in order, on `s`; nothing waits.
tiler_hip_status enqueue_plan(tiler_hip_context* ctx, const tiler_hip_dispatch_plan* plan,
                              void* const* slot_pointers, hipStream_t s);
}  // namespace

tiler_hip_status tiler_hip_enqueue_dispatch(tiler_hip_context* ctx, const tiler_hip_dispatch_plan* plan,
                                            void* const* slot_pointers, tiler_hip_stream stream) try {
  if (!ctx || !plan) return TILER_HIP_FAIL_LAUNCH;
  hipSetDevice(ctx->device);
  const hipStream_t s = pick(ctx, stream);
  // A constant slot's upload from host memory has no place in captured work.
  if (plan->slot_contents && capturing(s))
    for (uint32_t i = 0; i < plan->slot_count; ++i)
      if (plan->slot_contents[i] && plan->slot_bytes[i])
        return fail(ctx, TILER_HIP_FAIL_LAUNCH, "a constant slot's upload under graph capture; upload it first");
  return enqueue_plan(ctx, plan, slot_pointers, s);
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_FAIL_ALLOCATION;
}

tiler_hip_status tiler_hip_dispatch(tiler_hip_context* ctx, const tiler_hip_dispatch_plan* plan,
                                    void* const* slot_pointers) try {
  if (!ctx || !plan) return TILER_HIP_FAIL_LAUNCH;
  hipSetDevice(ctx->device);
  tiler_hip_status st = enqueue_plan(ctx, plan, slot_pointers, ctx->stream);
  if (st != TILER_HIP_OK) return st;
  hipError_t err = hipStreamSynchronize(ctx->stream);
  if (err != hipSuccess) return fail(ctx, TILER_HIP_FAIL_DEVICE, hipGetErrorString(err));
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_FAIL_ALLOCATION;
}

namespace {
tiler_hip_status enqueue_plan(tiler_hip_context* ctx, const tiler_hip_dispatch_plan* plan,
                              void* const* slot_pointers, hipStream_t stream) {
  // The live extents again, before anything is launched: the plan that was
  // checked may not be the one dispatched, and a value past its bound would
  // make the kernels read past operands sized for the bound.
  if (plan->extent_count && (!plan->extents || !plan->extent_ranges))
    return fail(ctx, TILER_HIP_FAIL_LAUNCH, "live extents without their values or ranges");
  for (uint32_t x = 0; x < plan->extent_count; ++x)
    if (!live_extent_in_range(plan, x))
      return fail(ctx, TILER_HIP_FAIL_LAUNCH,
                  "live extent " + std::to_string(x) + " = " + std::to_string(plan->extents[x]) +
                      " outside the range the realization was sized for; nothing launched");
  // Constant slots first (an expression's register program), ordered on the
  // stream before every entry; the host bytes are the caller's for the call.
  if (plan->slot_contents) {
    for (uint32_t k = 0; k < plan->slot_count; ++k) {
      if (!plan->slot_contents[k] || !plan->slot_bytes[k]) continue;
      if (!slot_pointers[k]) return fail(ctx, TILER_HIP_FAIL_TRANSFER, "constant slot " + std::to_string(k) + " unbound");
      hipError_t err = hipMemcpyAsync(slot_pointers[k], plan->slot_contents[k], plan->slot_bytes[k],
                                      hipMemcpyHostToDevice, stream);
      if (err != hipSuccess) return fail(ctx, TILER_HIP_FAIL_TRANSFER, hipGetErrorString(err));
    }
  }
  std::vector<uint8_t> args;
  for (uint32_t i = 0; i < plan->entry_count; ++i) {
    const tiler_hip_dispatch_entry& e = plan->entries[i];
    args.assign((const uint8_t*)e.kernargs, (const uint8_t*)e.kernargs + e.kernarg_bytes);
    for (uint32_t b = 0; b < e.binding_count; ++b) {
      void* p = slot_pointers[e.binding_slots[b]];
      std::memcpy(args.data() + e.binding_offsets[b], &p, sizeof(p));
    }
    for (uint32_t x = 0; x < e.extent_count; ++x) {
      if (e.extent_ids[x] >= plan->extent_count || plan->extents[e.extent_ids[x]] > 0xffffffffull)
        return fail(ctx, TILER_HIP_FAIL_LAUNCH, "entry " + std::to_string(i) + ": live extent not supplied");
      const uint32_t v = (uint32_t)plan->extents[e.extent_ids[x]];
      std::memcpy(args.data() + e.extent_offsets[x], &v, sizeof(v));
    }
    size_t size = args.size();
    void* config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, args.data(), HIP_LAUNCH_PARAM_BUFFER_SIZE,
                      &size, HIP_LAUNCH_PARAM_END};
    hipError_t err = hipModuleLaunchKernel(ctx->prepared[e.prepared], e.grid[0], e.grid[1],
                                           e.grid[2], e.block[0], e.block[1], e.block[2],
                                           e.dynamic_lds_bytes, stream, nullptr, config);
    if (err != hipSuccess)
      return fail(ctx, TILER_HIP_FAIL_LAUNCH, "entry " + std::to_string(i) + ": " + hipGetErrorString(err));
  }
  return TILER_HIP_OK;
}
}  // namespace

tiler_hip_status tiler_hip_release_dispatch(tiler_hip_context* ctx,
                                            const tiler_hip_dispatch_plan* plan,
                                            void** slot_pointers, const void** caller_owned) try {
  if (!ctx || !plan) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  hipSetDevice(ctx->device);
  for (uint32_t s = 0; s < plan->slot_count; ++s) {
    if (!slot_pointers[s] || (caller_owned && caller_owned[s])) continue;
    hipFree(slot_pointers[s]);
    slot_pointers[s] = nullptr;
  }
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

// ---------------------------------------------------------------------------
tiler_hip_status tiler_hip_buffer_alloc(tiler_hip_context* ctx, uint64_t bytes, void** out) try {
  if (!ctx || !out) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  hipSetDevice(ctx->device);
  *out = nullptr;
  if (hipMalloc(out, bytes ? bytes : 1) != hipSuccess)
    return fail(ctx, TILER_HIP_FAIL_ALLOCATION, "hipMalloc of " + std::to_string(bytes) + " bytes failed");
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}
tiler_hip_status tiler_hip_buffer_free(tiler_hip_context* ctx, void* ptr) try {
  if (!ctx) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  hipSetDevice(ctx->device);
  if (ptr && hipFree(ptr) != hipSuccess) return fail(ctx, TILER_HIP_FAIL_DEVICE, "hipFree failed");
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}
tiler_hip_status tiler_hip_upload(tiler_hip_context* ctx, void* dst, const void* src,
                                  uint64_t bytes) try {
  if (!ctx) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  if (bytes == 0) return TILER_HIP_OK;
  hipSetDevice(ctx->device);
  if (hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream) != hipSuccess ||
      hipStreamSynchronize(ctx->stream) != hipSuccess)
    return fail(ctx, TILER_HIP_FAIL_TRANSFER, "host-to-device copy failed");
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}
tiler_hip_status tiler_hip_download(tiler_hip_context* ctx, void* dst, const void* src,
                                    uint64_t bytes) try {
  if (!ctx) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  if (bytes == 0) return TILER_HIP_OK;
  hipSetDevice(ctx->device);
  if (hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream) != hipSuccess ||
      hipStreamSynchronize(ctx->stream) != hipSuccess)
    return fail(ctx, TILER_HIP_FAIL_TRANSFER, "device-to-host copy failed");
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}
tiler_hip_status tiler_hip_fill_u32(tiler_hip_context* ctx, void* dst, uint32_t value,
                                    uint64_t words, tiler_hip_stream stream) try {
  if (!ctx || (words && !dst)) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  if (words == 0) return TILER_HIP_OK;
  uint64_t groups = (words + 255) / 256;
  if (groups > 4096) groups = 4096;
  void* args[] = {&dst, &value, &words};
  return launch(ctx, "tiler_fill_u32", (uint32_t)groups, 1, 256, pick(ctx, stream), args);
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}
tiler_hip_status tiler_hip_copy(tiler_hip_context* ctx, void* dst, const void* src, uint64_t bytes,
                                tiler_hip_stream stream) try {
  if (!ctx || (bytes && (!dst || !src))) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  if (bytes == 0) return TILER_HIP_OK;
  if (hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, pick(ctx, stream)) != hipSuccess)
    return fail(ctx, TILER_HIP_FAIL_TRANSFER, "device-to-device copy failed");
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}
tiler_hip_status tiler_hip_synchronize(tiler_hip_context* ctx) try {
  if (!ctx) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  hipError_t e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return fail(ctx, TILER_HIP_FAIL_DEVICE, hipGetErrorString(e));
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}
tiler_hip_stream tiler_hip_context_stream(tiler_hip_context* ctx) {
  return ctx ? static_cast<tiler_hip_stream>(ctx->stream) : nullptr;
}
tiler_hip_status tiler_hip_event_create(tiler_hip_context* ctx, tiler_hip_event* out) try {
  if (!ctx || !out) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return fail(ctx, TILER_HIP_FAIL_DEVICE, "hipEventCreate failed");
  *out = e;
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}
tiler_hip_status tiler_hip_event_record(tiler_hip_context* ctx, tiler_hip_event ev,
                                        tiler_hip_stream stream) try {
  if (!ctx) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  if (hipEventRecord(static_cast<hipEvent_t>(ev), pick(ctx, stream)) != hipSuccess)
    return fail(ctx, TILER_HIP_FAIL_DEVICE, "hipEventRecord failed");
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}
tiler_hip_status tiler_hip_event_elapsed_ms(tiler_hip_context* ctx, tiler_hip_event start,
                                            tiler_hip_event stop, float* ms) try {
  if (!ctx || !ms) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  if (hipEventSynchronize(static_cast<hipEvent_t>(stop)) != hipSuccess ||
      hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)) != hipSuccess)
    return fail(ctx, TILER_HIP_FAIL_DEVICE, "hipEventElapsedTime failed");
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}
tiler_hip_status tiler_hip_event_destroy(tiler_hip_context* ctx, tiler_hip_event ev) try {
  if (!ctx) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  hipEventDestroy(static_cast<hipEvent_t>(ev));
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

struct GraphHandle {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
};

tiler_hip_status tiler_hip_capture_begin(tiler_hip_context* ctx, tiler_hip_stream stream) try {
  if (!ctx) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  hipError_t e = hipStreamBeginCapture(pick(ctx, stream), hipStreamCaptureModeThreadLocal);
  if (e != hipSuccess) return fail(ctx, TILER_HIP_REFUSE_UNSUPPORTED, std::string("capture: ") + hipGetErrorString(e));
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}
tiler_hip_status tiler_hip_capture_end(tiler_hip_context* ctx, tiler_hip_stream stream,
                                       tiler_hip_graph* out) try {
  if (!ctx || !out) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  auto* g = new GraphHandle();
  hipError_t e = hipStreamEndCapture(pick(ctx, stream), &g->graph);
  if (e == hipSuccess) e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    if (g->graph) hipGraphDestroy(g->graph);
    delete g;
    return fail(ctx, TILER_HIP_FAIL_LAUNCH, std::string("graph: ") + hipGetErrorString(e));
  }
  *out = g;
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}
tiler_hip_status tiler_hip_graph_launch(tiler_hip_context* ctx, tiler_hip_graph graph,
                                        tiler_hip_stream stream) try {
  if (!ctx || !graph) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  hipError_t e = hipGraphLaunch(static_cast<GraphHandle*>(graph)->exec, pick(ctx, stream));
  if (e != hipSuccess) return fail(ctx, TILER_HIP_FAIL_LAUNCH, std::string("graph launch: ") + hipGetErrorString(e));
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}
tiler_hip_status tiler_hip_graph_destroy(tiler_hip_context* ctx, tiler_hip_graph graph) try {
  if (!ctx) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  auto* g = static_cast<GraphHandle*>(graph);
  if (g) {
    if (g->exec) hipGraphExecDestroy(g->exec);
    if (g->graph) hipGraphDestroy(g->graph);
    delete g;
  }
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

// ---------------------------------------------------------------------------
tiler_hip_status tiler_hip_row_grouping(uint32_t family, uint32_t dtype, uint64_t extent,
                                        uint32_t* vec, uint32_t* waves, uint64_t* segment) try {
  if (!vec || !waves || !segment) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  *segment = 0;
  switch (family) {
    case TILER_HIP_ROWS_RMS_NORM:
      if (dtype != TILER_HIP_F32 && dtype != TILER_HIP_BF16) return TILER_HIP_REFUSE_UNSUPPORTED;
      *vec = dtype == TILER_HIP_BF16 ? 8 : 4;
      *waves = extent > kWaveRowMax ? 16 : 1;
      return TILER_HIP_OK;
    case TILER_HIP_ROWS_SOFTMAX:
      if (dtype != TILER_HIP_F32) return TILER_HIP_REFUSE_UNSUPPORTED;
      *vec = 4;
      *waves = extent > kWaveRowMax ? 4 : 1;
      *segment = extent > kWaveRowMax ? tiler_rt::kSoftmaxSegment : 0;
      return TILER_HIP_OK;
    case TILER_HIP_ROWS_SUM:
      if (dtype != TILER_HIP_F32) return TILER_HIP_REFUSE_UNSUPPORTED;
      *vec = 4;
      *waves = 4;
      return TILER_HIP_OK;
    default:
      return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  }
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

uint32_t tiler_hip_sum_tree_workgroups(const tiler_hip_context* ctx, uint64_t n) {
  return tiler_rt::tree_workgroups(target_of(ctx), n);
}

tiler_hip_status tiler_hip_sum_f32(tiler_hip_context* ctx, const float* x, uint64_t rows,
                                   uint64_t extent, float* out, const tiler_hip_sum_plan* plan,
                                   tiler_hip_stream stream) try {
  if (!ctx || !plan || (rows && !out) || (rows && extent && !x))
    return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  tiler_rt::Program p;
  const uintptr_t addr[3] = {(uintptr_t)x, (uintptr_t)out, 0};
  tiler_hip_status st = tiler_rt::plan_sum_f32(target_of(ctx), rows, extent, *plan, addr, p);
  if (st != TILER_HIP_OK) return fail(ctx, st, p.diag);
  hipStream_t s = pick(ctx, stream);
  void* slots[tiler_rt::kMaxSlots] = {const_cast<float*>(x), out, nullptr};
  // Partials live in the context workspace when they fit (ordered on the
  // stream); only larger splits allocate, stream-ordered.
  bool own = false;
  if (p.nslots > 2 && p.nlaunches) {
    if (p.slot_bytes[2] <= tiler_rt::kWorkspacePartialBytes) {
      if ((st = workspace_stream(ctx, stream, "this sum's partials")) != TILER_HIP_OK) return st;
      slots[2] = ctx->sum_partials;
    } else {
      if (capturing(s))
        return fail(ctx, TILER_HIP_REFUSE_CAPACITY, "partials exceed the workspace under graph capture");
      if (hipMallocAsync(&slots[2], p.slot_bytes[2], s) != hipSuccess)
        return fail(ctx, TILER_HIP_FAIL_ALLOCATION, "partials allocation failed");
      own = true;
    }
  }
  st = run_program(ctx, p, slots, s);
  if (own) hipFreeAsync(slots[2], s);
  return st;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

tiler_hip_status tiler_hip_sum_f32_noalloc(tiler_hip_context* ctx, const float* x, uint64_t rows,
                                           uint64_t extent, float* out, const tiler_hip_sum_plan* plan,
                                           tiler_hip_stream stream) try {
  if (!ctx || !plan || (rows && !out) || (rows && extent && !x))
    return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  tiler_rt::Program p;
  const uintptr_t addr[3] = {(uintptr_t)x, (uintptr_t)out, 0};
  tiler_hip_status st = tiler_rt::plan_sum_f32(target_of(ctx), rows, extent, *plan, addr, p);
  if (st != TILER_HIP_OK) return fail(ctx, st, p.diag);
  void* slots[tiler_rt::kMaxSlots] = {const_cast<float*>(x), out, nullptr};
  if (p.nslots > 2 && p.nlaunches) {
    // The partials go to this device's static scratch array, through the
    // address bind resolved: nothing is allocated.  Every stage-1 launch
    // writes all the partials its second launch reads, so nothing needs
    // clearing; overlapping calls on one GPU share the array and race.
    if (!ctx->noalloc_scratch)
      return fail(ctx, TILER_HIP_REFUSE_UNSUPPORTED,
                  "the static scratch array could not be resolved at bind (HIP error " +
                      std::to_string(ctx->noalloc_error) + ")");
    if (p.slot_bytes[2] > TILER_HIP_NOALLOC_SCRATCH_BYTES)
      return fail(ctx, TILER_HIP_REFUSE_CAPACITY, "partials exceed the 8 MiB static scratch array");
    slots[2] = ctx->noalloc_scratch;
  }
  return run_program(ctx, p, slots, pick(ctx, stream));
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

tiler_hip_status tiler_hip_rms_norm(tiler_hip_context* ctx, uint32_t dtype, const void* x,
                                    const void* w, int32_t weight_broadcast, uint64_t rows,
                                    uint64_t extent, uint32_t eps_bits, void* y,
                                    tiler_hip_stream stream) try {
  if (!ctx) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  tiler_rt::Program p;
  const uintptr_t addr[3] = {(uintptr_t)x, (uintptr_t)w, (uintptr_t)y};
  tiler_hip_status st = tiler_rt::plan_rms_norm(target_of(ctx), dtype, weight_broadcast, rows, extent, eps_bits, addr, p);
  if (st != TILER_HIP_OK) return fail(ctx, st, p.diag);
  if (p.nlaunches && (!x || !w || !y)) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  void* slots[tiler_rt::kMaxSlots] = {const_cast<void*>(x), const_cast<void*>(w), y};
  return run_program(ctx, p, slots, pick(ctx, stream));
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

tiler_hip_status tiler_hip_softmax_f32(tiler_hip_context* ctx, const float* x, uint64_t rows,
                                       uint64_t extent, float* y, tiler_hip_stream stream) try {
  if (!ctx) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  tiler_rt::Program p;
  const uintptr_t addr[2] = {(uintptr_t)x, (uintptr_t)y};
  tiler_hip_status st = tiler_rt::plan_softmax_f32(tiler_rt::Mode::Direct, target_of(ctx), rows, extent, addr, p);
  if (st != TILER_HIP_OK) return fail(ctx, st, p.diag);
  if (p.nlaunches && (!x || !y)) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  hipStream_t s = pick(ctx, stream);
  void* slots[tiler_rt::kMaxSlots] = {const_cast<float*>(x), y};
  // The split form's partials (segment maxima, then sums) live in the context
  // workspace when they fit (ordered on the stream); larger ones are
  // allocated, stream-ordered.
  bool own = false;
  uint8_t* part = nullptr;
  if (p.nslots == 3) {  // the row-synchronized form: its area in the workspace
    if (p.slot_bytes[2] > tiler_rt::kRowSyncBytes) return fail(ctx, TILER_HIP_REFUSE_CAPACITY, "row-sync area");
    if ((st = workspace_stream(ctx, stream, "the row-synchronized softmax")) != TILER_HIP_OK) return st;
    slots[2] = ctx->row_sync;
  } else if (p.nslots > 2) {
    const uint64_t bytes = p.slot_bytes[2] + p.slot_bytes[3];
    if (bytes <= tiler_rt::kWorkspacePartialBytes) {
      if ((st = workspace_stream(ctx, stream, "the split softmax's partials")) != TILER_HIP_OK) return st;
      part = reinterpret_cast<uint8_t*>(ctx->sum_partials);
    } else {
      if (capturing(s))
        return fail(ctx, TILER_HIP_REFUSE_CAPACITY, "partials exceed the workspace under graph capture");
      if (hipMallocAsync(reinterpret_cast<void**>(&part), bytes, s) != hipSuccess)
        return fail(ctx, TILER_HIP_FAIL_ALLOCATION, "partials allocation failed");
      own = true;
    }
    slots[2] = part;
    slots[3] = part + p.slot_bytes[2];
  }
  st = run_program(ctx, p, slots, s);
  if (own) hipFreeAsync(part, s);
  return st;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

tiler_hip_status tiler_hip_map(tiler_hip_context* ctx, uint32_t op, uint32_t dtype,
                               const void* x, const void* x2, int32_t x2_broadcast, uint64_t n,
                               float a, float b, void* y, tiler_hip_stream stream) try {
  if (!ctx) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  const bool binary = op == TILER_HIP_MAP_ADD || op == TILER_HIP_MAP_MULTIPLY;
  tiler_rt::Program p;
  const uintptr_t addr[3] = {(uintptr_t)x, binary ? (uintptr_t)x2 : (uintptr_t)y, (uintptr_t)y};
  tiler_hip_status st = tiler_rt::plan_map(tiler_rt::Mode::Direct, op, dtype, x2_broadcast, n, a, b, addr, p);
  if (st != TILER_HIP_OK) return fail(ctx, st, p.diag);
  if (p.nlaunches && (!x || !y || (binary && !x2))) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  void* slots[tiler_rt::kMaxSlots] = {const_cast<void*>(x), binary ? const_cast<void*>(x2) : y, y};
  return run_program(ctx, p, slots, pick(ctx, stream));
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

tiler_hip_status tiler_hip_broadcast(tiler_hip_context* ctx, const void* src, uint64_t src_elements,
                                     uint32_t rank, const uint64_t* out_dims,
                                     const uint64_t* src_strides, uint32_t element_bytes, void* out,
                                     tiler_hip_stream stream) try {
  if (!ctx) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  tiler_rt::Program p;
  tiler_hip_status st = tiler_rt::plan_broadcast(src_elements, rank, out_dims, src_strides, element_bytes, p);
  if (st != TILER_HIP_OK) return fail(ctx, st, p.diag);
  if (p.nlaunches && (!src || !out)) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  void* slots[tiler_rt::kMaxSlots] = {const_cast<void*>(src), out};
  return run_program(ctx, p, slots, pick(ctx, stream));
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

tiler_hip_status tiler_hip_convert(tiler_hip_context* ctx, uint32_t direction, const void* src,
                                   uint64_t n, void* dst, tiler_hip_stream stream) try {
  if (!ctx) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  tiler_rt::Program p;
  const uintptr_t addr[2] = {(uintptr_t)src, (uintptr_t)dst};
  tiler_hip_status st = tiler_rt::plan_convert(tiler_rt::Mode::Direct, direction, n, addr, p);
  if (st != TILER_HIP_OK) return fail(ctx, st, p.diag);
  if (p.nlaunches && (!src || !dst)) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  void* slots[tiler_rt::kMaxSlots] = {const_cast<void*>(src), dst};
  return run_program(ctx, p, slots, pick(ctx, stream));
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

tiler_hip_status tiler_hip_dequantize_u4(tiler_hip_context* ctx, const uint8_t* codes, uint64_t n,
                                        uint32_t scale_bits, uint32_t zero_point, float* y,
                                        tiler_hip_stream stream) try {
  if (!ctx) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  tiler_rt::Program p;
  const uintptr_t addr[2] = {(uintptr_t)codes, (uintptr_t)y};
  tiler_hip_status st = tiler_rt::plan_dequantize_u4(tiler_rt::Mode::Direct, n, scale_bits, zero_point, addr, p);
  if (st != TILER_HIP_OK) return fail(ctx, st, p.diag);
  if (p.nlaunches && (!codes || !y)) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  void* slots[tiler_rt::kMaxSlots] = {const_cast<uint8_t*>(codes), y};
  return run_program(ctx, p, slots, pick(ctx, stream));
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

tiler_hip_status tiler_hip_validate_gather_index(const uint32_t* index, uint64_t count,
                                                 int32_t index_signed, uint64_t gathered,
                                                 uint64_t* bad_position, int64_t* bad_value) try {
  if (count && !index) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  for (uint64_t i = 0; i < count; ++i) {
    int64_t v = index_signed ? (int64_t)(int32_t)index[i] : (int64_t)index[i];
    if (v < 0 || (uint64_t)v >= gathered) {
      if (bad_position) *bad_position = i;
      if (bad_value) *bad_value = v;
      return TILER_HIP_REFUSE_GATHER_INDEX_OUT_OF_BOUNDS;
    }
  }
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

tiler_hip_status tiler_hip_gather(tiler_hip_context* ctx, const void* source, uint64_t outer,
                                  uint64_t gathered, uint64_t inner, uint32_t element_bytes,
                                  const uint32_t* index, uint64_t count, int32_t index_signed,
                                  void* out, tiler_hip_stream stream) try {
  if (!ctx) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  tiler_rt::Program p;
  const uintptr_t addr[4] = {(uintptr_t)source, (uintptr_t)index, (uintptr_t)out, 0};
  tiler_hip_status st = tiler_rt::plan_gather(tiler_rt::Mode::Direct, outer, gathered, inner, element_bytes,
                                              count, index_signed, addr, p);
  if (st != TILER_HIP_OK) return fail(ctx, st, p.diag);
  if (p.nlaunches && (!source || !index || !out)) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  if (p.nlaunches && (st = workspace_stream(ctx, stream, "the gather's out-of-range record")) != TILER_HIP_OK)
    return st;
  void* slots[tiler_rt::kMaxSlots] = {const_cast<void*>(source), const_cast<uint32_t*>(index), out,
                                      ctx->gather_bad};
  return run_program(ctx, p, slots, pick(ctx, stream));
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

tiler_hip_status tiler_hip_gather_status(tiler_hip_context* ctx, tiler_hip_stream stream,
                                         uint64_t* bad_position) try {
  if (!ctx) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  if (tiler_hip_status st = workspace_stream(ctx, stream, "the gather record's read"); st != TILER_HIP_OK)
    return st;
  hipStream_t s = pick(ctx, stream);
  unsigned long long v = 0;
  if (hipMemcpyAsync(&v, ctx->gather_bad, 8, hipMemcpyDeviceToHost, s) != hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess)
    return fail(ctx, TILER_HIP_FAIL_DEVICE, "reading the gather record failed");
  if (v == ~0ull) return TILER_HIP_OK;
  if (bad_position) *bad_position = v;
  tiler_hip_fill_u32(ctx, ctx->gather_bad, 0xffffffffu, 2, s);  // re-arm the record
  hipStreamSynchronize(s);
  return fail(ctx, TILER_HIP_FAIL_GATHER_INDEX_OUT_OF_BOUNDS,
              "gather index out of bounds at position " + std::to_string(v));
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

tiler_hip_status tiler_hip_contract_strict_f32(tiler_hip_context* ctx, const float* a,
                                               const float* b, uint64_t m, uint64_t n,
                                               uint64_t k, float* c, tiler_hip_stream stream) try {
  if (!ctx) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  tiler_rt::Program p;
  const uintptr_t addr[3] = {(uintptr_t)a, (uintptr_t)b, (uintptr_t)c};
  tiler_hip_status st = tiler_rt::plan_contract_strict_f32(target_of(ctx), m, n, k, addr, p);
  if (st != TILER_HIP_OK) return fail(ctx, st, p.diag);
  if (p.nlaunches && (!a || !b || !c)) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  void* slots[tiler_rt::kMaxSlots] = {const_cast<float*>(a), const_cast<float*>(b), c};
  return run_program(ctx, p, slots, pick(ctx, stream));
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

tiler_hip_status tiler_hip_contract_bf16(tiler_hip_context* ctx, const uint16_t* a,
                                         const uint16_t* b, uint64_t m, uint64_t n, uint64_t k,
                                         uint16_t* c, uint32_t epilogue,
                                         tiler_hip_stream stream) try {
  if (!ctx) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  tiler_rt::Program p;
  const uintptr_t addr[3] = {(uintptr_t)a, (uintptr_t)b, (uintptr_t)c};
  tiler_hip_status st = tiler_rt::plan_contract_bf16(target_of(ctx), m, n, k, epilogue, addr, p);
  if (st != TILER_HIP_OK) return fail(ctx, st, p.diag);
  if (p.nlaunches && (!a || !b || !c)) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  void* slots[tiler_rt::kMaxSlots] = {const_cast<uint16_t*>(a), const_cast<uint16_t*>(b), c};
  return run_program(ctx, p, slots, pick(ctx, stream));
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

// A program's CONSTANT slot contents (an expression's register program, a
// contraction's geometry) live on the device once per distinct contents: a
// synchronous upload on first use; under graph capture uncached contents
// refuse, so capture after one eager call.
tiler_hip_status resident_constant(tiler_hip_context* ctx, const tiler_rt::Program& p, hipStream_t s, void** out) {
  std::string key(p.constant.begin(), p.constant.end());
  auto it = ctx->expression_programs.find(key);
  if (it == ctx->expression_programs.end()) {
    if (capturing(s)) return fail(ctx, TILER_HIP_REFUSE_CAPACITY, "constant slot contents not yet resident under graph capture");
    if (ctx->expression_programs.size() >= 4096) return fail(ctx, TILER_HIP_REFUSE_CAPACITY, "too many resident constant slots");
    void* dev = nullptr;
    if (hipMalloc(&dev, p.constant.size()) != hipSuccess) return fail(ctx, TILER_HIP_FAIL_ALLOCATION, "constant slot");
    if (hipMemcpy(dev, p.constant.data(), p.constant.size(), hipMemcpyHostToDevice) != hipSuccess) {
      hipFree(dev);
      return fail(ctx, TILER_HIP_FAIL_TRANSFER, "constant slot upload");
    }
    it = ctx->expression_programs.emplace(key, dev).first;
  }
  *out = it->second;
  return TILER_HIP_OK;
}

tiler_hip_status tiler_hip_contract(tiler_hip_context* ctx, uint32_t dtype,
                                    const tiler_hip_contraction_structure* structure, uint32_t epilogue,
                                    uint32_t permissions, const void* left, const void* right, void* out,
                                    tiler_hip_stream stream) try {
  if (!ctx || !structure) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  if (permissions & ~(uint32_t)(TILER_HIP_PERMITS_REASSOCIATION | TILER_HIP_PERMITS_PERMUTATION))
    return fail(ctx, TILER_HIP_REFUSE_INVALID_ARGUMENT, "unknown permission bits");
  tiler_rt::Program p;
  const uintptr_t addr[4] = {(uintptr_t)left, (uintptr_t)right, (uintptr_t)out, 0};
  tiler_hip_status st = tiler_rt::plan_contract_general(target_of(ctx), dtype, *structure, epilogue,
                                                        !(permissions & TILER_HIP_PERMITS_REASSOCIATION), addr, p);
  if (st != TILER_HIP_OK) return fail(ctx, st, p.diag);
  if (!p.nlaunches) return TILER_HIP_OK;
  if (!left || !right || !out) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  hipStream_t s = pick(ctx, stream);
  void* slots[tiler_rt::kMaxSlots] = {const_cast<void*>(left), const_cast<void*>(right), out};
  bool own = false;
  if (p.nslots > 3) {
    if (p.slot_roles[3] == TILER_HIP_SLOT_CONSTANT) {
      st = resident_constant(ctx, p, s, &slots[3]);
      if (st != TILER_HIP_OK) return st;
    } else {  // the transposed right operand
      if (capturing(s)) return fail(ctx, TILER_HIP_REFUSE_CAPACITY, "transpose workspace allocation under graph capture");
      if (hipMallocAsync(&slots[3], p.slot_bytes[3], s) != hipSuccess)
        return fail(ctx, TILER_HIP_FAIL_ALLOCATION, "transpose workspace allocation failed");
      own = true;
    }
  }
  st = run_program(ctx, p, slots, s);
  if (own) hipFreeAsync(slots[3], s);
  return st;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

// ---------------------------------------------------------------------------
tiler_hip_status tiler_hip_expression(tiler_hip_context* ctx, uint32_t dtype,
                                      const tiler_hip_expression_node* nodes, uint32_t node_count,
                                      uint32_t root, const void* const* inputs, uint64_t n, void* y,
                                      uint32_t input_subnormals, uint32_t result_subnormals,
                                      tiler_hip_stream stream) try {
  if (!ctx) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  tiler_rt::ExpressionProgram prog;
  std::string diag;
  tiler_hip_status st = tiler_rt::compile_expression(dtype, nodes, node_count, root, false, prog, diag);
  if (st != TILER_HIP_OK) return fail(ctx, st, diag);
  if (n && (!y || (prog.inputs && !inputs))) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  for (uint32_t k = 0; n && k < prog.inputs; ++k)
    if (!inputs[k]) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  tiler_rt::Contract c;
  c.input_mode = input_subnormals ? input_subnormals : 1;
  c.result_mode = result_subnormals ? result_subnormals : 1;
  if (c.input_mode > 3 || c.result_mode > 3) return fail(ctx, TILER_HIP_REFUSE_INVALID_ARGUMENT, "unknown subnormal mode");
  uintptr_t addr[tiler_rt::kMaxSlots] = {};
  for (uint32_t k = 0; k < prog.inputs; ++k) addr[k] = inputs ? (uintptr_t)inputs[k] : 0;
  addr[prog.inputs] = (uintptr_t)y;
  tiler_rt::Program p;
  st = tiler_rt::plan_expression(target_of(ctx), dtype, n, prog, c, addr, p);
  if (st != TILER_HIP_OK) return fail(ctx, st, p.diag);
  if (!p.nlaunches) return TILER_HIP_OK;
  hipStream_t s = pick(ctx, stream);
  void* slots[tiler_rt::kMaxSlots] = {};
  st = resident_constant(ctx, p, s, &slots[prog.inputs + 1]);
  if (st != TILER_HIP_OK) return st;
  for (uint32_t k = 0; k < prog.inputs; ++k) slots[k] = const_cast<void*>(inputs[k]);
  slots[prog.inputs] = y;
  bool own = false;
  if (p.nslots > prog.inputs + 2) {  // the value store
    if (capturing(s)) return fail(ctx, TILER_HIP_REFUSE_CAPACITY, "value store allocation under graph capture");
    if (hipMallocAsync(&slots[prog.inputs + 2], p.slot_bytes[prog.inputs + 2], s) != hipSuccess)
      return fail(ctx, TILER_HIP_FAIL_ALLOCATION, "value store allocation failed");
    own = true;
  }
  st = run_program(ctx, p, slots, s);
  if (own) hipFreeAsync(slots[prog.inputs + 2], s);
  return st;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

tiler_hip_status tiler_hip_fold_f32(tiler_hip_context* ctx, uint32_t variant, const float* x, uint32_t rank,
                                    const uint64_t* dims, uint64_t reduced_mask, uint32_t scale_bits,
                                    uint32_t bias_bits, float* out, tiler_hip_stream stream) try {
  if (!ctx) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  tiler_rt::Program p;
  tiler_hip_status st = tiler_rt::plan_fold(variant, rank, dims, reduced_mask, scale_bits, bias_bits, nullptr, p);
  if (st != TILER_HIP_OK) return fail(ctx, st, p.diag);
  if (p.nlaunches && (!x || !out)) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  void* slots[tiler_rt::kMaxSlots] = {const_cast<float*>(x), out};
  return run_program(ctx, p, slots, pick(ctx, stream));
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

tiler_hip_status tiler_hip_reindex(tiler_hip_context* ctx, const void* src, uint64_t src_elements, uint32_t rank,
                                   const uint64_t* out_dims, const int64_t* strides, int64_t base,
                                   uint32_t element_bytes, void* out, tiler_hip_stream stream) try {
  if (!ctx) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  tiler_rt::Program p;
  tiler_hip_status st = tiler_rt::plan_reindex(src_elements, rank, out_dims, strides, base, element_bytes, p);
  if (st != TILER_HIP_OK) return fail(ctx, st, p.diag);
  if (p.nlaunches && (!src || !out)) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  void* slots[tiler_rt::kMaxSlots] = {const_cast<void*>(src), out};
  return run_program(ctx, p, slots, pick(ctx, stream));
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

// ---------------------------------------------------------------------------
// Target environment (adapter.rs:295-322; environment.rs:249-400).
namespace {

constexpr const char* kEnvironmentProvider = "tiler.hip.target-environment";
constexpr const char* kTargetIdPrefix = "amdgcn-amd-amdhsa--gfx950";

void put_u32_be(std::vector<uint8_t>& v, uint32_t x) {
  for (int i = 3; i >= 0; --i) v.push_back((uint8_t)(x >> (8 * i)));
}
uint32_t get_u32_be(const uint8_t* p) {
  return (uint32_t)p[0] << 24 | (uint32_t)p[1] << 16 | (uint32_t)p[2] << 8 | p[3];
}

// The canonical descriptor for a target ID's feature settings.
std::vector<uint8_t> environment_descriptor(bool sramecc, bool xnack) {
  std::string id = std::string(kTargetIdPrefix) + ":sramecc" + (sramecc ? "+" : "-") + ":xnack" + (xnack ? "+" : "-");
  std::vector<uint8_t> v;
  put_u32_be(v, (uint32_t)id.size());
  v.insert(v.end(), id.begin(), id.end());
  put_u32_be(v, 64);
  return v;
}

}  // namespace

tiler_hip_status tiler_hip_target_environment_support(tiler_hip_target_environment_schema* out) try {
  if (!out) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  std::memset(out, 0, sizeof(*out));
  copy_text(out->provider, sizeof(out->provider), kEnvironmentProvider);
  out->provider_revision = 1;
  out->schema_major = 1;
  out->schema_minor = 0;
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

tiler_hip_status tiler_hip_validate_target_environment(const void* descriptor, uint64_t bytes, char* diagnostic,
                                                       uint64_t diagnostic_bytes) try {
  if (!descriptor && bytes) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  const uint8_t* d = static_cast<const uint8_t*>(descriptor);
  auto refuse = [&](const char* what) {
    copy_text(diagnostic, diagnostic_bytes, what);
    return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  };
  if (bytes < 8) return refuse("descriptor shorter than its framing");
  const uint32_t len = get_u32_be(d);
  if ((uint64_t)len + 8 != bytes) return refuse("descriptor length does not frame the bytes exactly");
  const std::string id(reinterpret_cast<const char*>(d + 4), len);
  if (get_u32_be(d + 4 + len) != 64) return refuse("wavefront size is not 64");
  for (bool sramecc : {false, true})
    for (bool xnack : {false, true}) {
      const std::vector<uint8_t> canonical = environment_descriptor(sramecc, xnack);
      if (canonical.size() == bytes && std::memcmp(canonical.data(), d, bytes) == 0) {
        copy_text(diagnostic, diagnostic_bytes, "");
        return TILER_HIP_OK;
      }
    }
  if (id.rfind(kTargetIdPrefix, 0) != 0) return refuse("target ID is not amdgcn-amd-amdhsa--gfx950");
  return refuse("target ID features are not the canonical :sramecc(+|-):xnack(+|-) spelling");
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

tiler_hip_status tiler_hip_observe_target_environment(tiler_hip_context* ctx, uint8_t* descriptor,
                                                      uint64_t capacity, uint64_t* required, uint32_t* observed,
                                                      char* reason, uint64_t reason_bytes) try {
  if (!ctx || !observed) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  *observed = 0;
  if (required) *required = 0;
  // The runtime's gcnArchName spells the bound device's target ID features
  // (e.g. "gfx950:sramecc+:xnack-"); without both, nothing is asserted.
  const std::string& arch = ctx->arch;
  const auto feature = [&](const char* name) -> int {
    const std::string on = std::string(":") + name + "+", off = std::string(":") + name + "-";
    if (arch.find(on) != std::string::npos) return 1;
    if (arch.find(off) != std::string::npos) return 0;
    return -1;
  };
  const int sramecc = feature("sramecc"), xnack = feature("xnack");
  if (arch.rfind("gfx950", 0) != 0 || sramecc < 0 || xnack < 0) {
    copy_text(reason, reason_bytes, "the runtime's architecture name (" + arch + ") does not state both target features");
    return TILER_HIP_OK;
  }
  const std::vector<uint8_t> v = environment_descriptor(sramecc == 1, xnack == 1);
  if (required) *required = v.size();
  if (!descriptor || capacity < v.size()) return fail(ctx, TILER_HIP_REFUSE_CAPACITY, "descriptor buffer too small");
  std::memcpy(descriptor, v.data(), v.size());
  *observed = 1;
  copy_text(reason, reason_bytes, "");
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

// ---------------------------------------------------------------------------
// Realization recognizer.
namespace {

tiler_rt::Contract contract_of(const tiler_hip_region* r) {
  tiler_rt::Contract c;
  c.reassociate = (r->permissions & TILER_HIP_PERMITS_REASSOCIATION) != 0;
  c.input_mode = r->input_subnormals ? r->input_subnormals : TILER_HIP_SUBNORMALS_PRESERVE;
  c.result_mode = r->result_subnormals ? r->result_subnormals : TILER_HIP_SUBNORMALS_PRESERVE;
  return c;
}

// Programs whose arithmetic a flushing subnormal mode could change.  The
// strict-affine decode is not one: its scale is a positive normal and its
// code difference an integer of magnitude 0 or at least 1, so every operand
// and product lies outside the subnormal range and both modes have nothing to
// act on (quantization.rs:1-15, :400-408); the reference applies neither.
bool arithmetic(uint32_t program) {
  return program != TILER_HIP_PROGRAM_GATHER && program != TILER_HIP_PROGRAM_BROADCAST &&
         program != TILER_HIP_PROGRAM_REINDEX && program != TILER_HIP_PROGRAM_DEQUANTIZE_U4;
}

// Arithmetic programs whose realizations apply the declared subnormal modes.
bool realizes_modes(uint32_t program) {
  return program == TILER_HIP_PROGRAM_SERIAL_SUM || program == TILER_HIP_PROGRAM_FOLD ||
         program == TILER_HIP_PROGRAM_RMS_NORM || program == TILER_HIP_PROGRAM_SOFTMAX ||
         program == TILER_HIP_PROGRAM_POINTWISE || program == TILER_HIP_PROGRAM_EXPRESSION ||
         program == TILER_HIP_PROGRAM_CONTRACTION;
}

}  // namespace

// The program a region realizes as (the planners' own output), or the
// refusal with its diagnostic in p.diag.
static tiler_hip_status plan_region(const tiler_hip_context* ctx, const tiler_hip_region* r, tiler_rt::Program& p) {
  const bool al = (r->flags & TILER_HIP_REGION_ALIGNED16) != 0;
  const bool bc = (r->flags & TILER_HIP_REGION_OPERAND_BROADCAST) != 0;
  const bool live = (r->flags & TILER_HIP_REGION_LIVE_EXTENT) != 0;
  // A stand-in address per slot: 0 is 16-byte aligned, 1 is not.
  uintptr_t addr[tiler_rt::kMaxSlots];
  for (uint32_t i = 0; i < tiler_rt::kMaxSlots; ++i) addr[i] = al ? 0u : 1u;
  const uint64_t* e = r->extents;
  const tiler_rt::Target t = target_of(ctx);
  const tiler_rt::Contract c = contract_of(r);
  tiler_hip_status st;
  if (c.input_mode > TILER_HIP_SUBNORMALS_FLUSH_POSITIVE || c.result_mode > TILER_HIP_SUBNORMALS_FLUSH_POSITIVE)
    return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "unknown subnormal mode");
  if (r->reserved != 0) return p.refuse(TILER_HIP_REFUSE_INVALID_ARGUMENT, "reserved region field is not 0");
  // The device preserves subnormals; a flushing contract is realized where
  // the kernels apply the declared modes at every arithmetic site (the sums
  // and folds, RMSNorm, softmax, the maps and the expressions, f32 and bf16).
  // Byte moves and the strict-affine decode have no site a mode could reach;
  // the conversions refuse it.  A contraction under a flushing contract runs
  // the strict fold, whatever its permissions.
  if (c.flushes() && arithmetic(r->program) && !realizes_modes(r->program))
    return p.refuse(TILER_HIP_REFUSE_UNSUPPORTED,
                    "a flushing subnormal mode is not realized for this program (the device preserves subnormals)");
  // Forms belong to the softmax and the td,od->to bf16 contraction.
  if (r->form != TILER_HIP_FORM_AUTO && r->program != TILER_HIP_PROGRAM_SOFTMAX &&
      !(r->program == TILER_HIP_PROGRAM_CONTRACTION && !r->structure && r->dtype == TILER_HIP_BF16))
    return p.refuse(TILER_HIP_REFUSE_UNSUPPORTED, "form: this program has one form");
  // A live extent belongs to the contraction (LiveContraction, schedule/model.rs:1429-1450).
  if (live && r->program != TILER_HIP_PROGRAM_CONTRACTION)
    return p.refuse(TILER_HIP_REFUSE_UNSUPPORTED, "live-extent: only the contraction's k is live");
  auto needs_reassociation = [&](const char* what) {
    return p.refuse(TILER_HIP_REFUSE_UNSUPPORTED,
                    (std::string(what) + " regroups the fold; the contract grants no reassociation").c_str());
  };
  tiler_rt::ExpressionProgram prog;
  switch (r->program) {
    case TILER_HIP_PROGRAM_POINTWISE: {
      float a, b;
      std::memcpy(&a, &r->scalars[0], 4);
      std::memcpy(&b, &r->scalars[1], 4);
      st = tiler_rt::plan_map(tiler_rt::Mode::Realized, r->variant, r->dtype, bc ? 1 : 0, e[0], a, b, addr, p,
                              c.input_mode, c.result_mode);
      break;
    }
    case TILER_HIP_PROGRAM_EXPRESSION: {
      st = tiler_rt::compile_expression(r->dtype, r->nodes, r->node_count, r->root, false, prog, p.diag);
      if (st == TILER_HIP_OK) st = tiler_rt::plan_expression(t, r->dtype, e[0], prog, c, addr, p);
      break;
    }
    case TILER_HIP_PROGRAM_SERIAL_SUM: {
      if (r->dtype != TILER_HIP_F32) {
        st = p.refuse(TILER_HIP_REFUSE_UNSUPPORTED, "the serial sum is an f32 family");
        break;
      }
      // Tree, multi-pass and cooperative all regroup the contributor sequence
      // (model.rs:1381-1392, 1520-1531): they need permits_reassociation.
      if (r->topology != TILER_HIP_SUM_SERIAL && !c.reassociate) {
        st = needs_reassociation("a split or tree sum");
        break;
      }
      tiler_hip_sum_plan sp;
      std::memset(&sp, 0, sizeof(sp));
      sp.topology = r->topology;
      sp.participant_major = (r->flags & TILER_HIP_REGION_PARTICIPANT_MAJOR) ? 1u : 0u;
      if (r->topology == TILER_HIP_SUM_MULTIPASS) {
        sp.partitions = r->grouping[0];
        sp.per_partition = r->grouping[1];
      } else if (r->topology == TILER_HIP_SUM_COOPERATIVE) {
        sp.participants = r->grouping[0];
        sp.per_partition = r->grouping[1];
        sp.rounds = r->grouping[2];
      }
      if (c.flushes()) {
        tiler_rt::FoldRuleHost rule;
        rule.in_mode = c.input_mode;
        rule.out_mode = c.result_mode;
        st = tiler_rt::plan_sum_f32(t, e[0], e[1], sp, addr, p, &rule);
      } else {
        st = tiler_rt::plan_sum_f32(t, e[0], e[1], sp, addr, p);
      }
      break;
    }
    case TILER_HIP_PROGRAM_FOLD: {
      if (r->dtype != TILER_HIP_F32) {
        st = p.refuse(TILER_HIP_REFUSE_UNSUPPORTED, "the folds are f32 families");
        break;
      }
      const bool epi = r->node_count != 0;
      if (epi) {
        st = tiler_rt::compile_expression(TILER_HIP_F32, r->nodes, r->node_count, r->root, true, prog, p.diag);
        if (st != TILER_HIP_OK) break;
      }
      // A split or workgroup topology regroups the contributor sequence:
      // permits_reassociation required, as for the sum program.
      if (r->topology != TILER_HIP_SUM_SERIAL && !c.reassociate) {
        st = needs_reassociation("a split or workgroup fold");
        break;
      }
      tiler_hip_sum_plan sp;
      std::memset(&sp, 0, sizeof(sp));
      sp.topology = r->topology;
      sp.participant_major = (r->flags & TILER_HIP_REGION_PARTICIPANT_MAJOR) ? 1u : 0u;
      if (r->topology == TILER_HIP_SUM_MULTIPASS) {
        sp.partitions = r->grouping[1];
        sp.per_partition = r->grouping[2];
      } else if (r->topology == TILER_HIP_SUM_COOPERATIVE && r->rank >= 1) {
        // The rounds follow from exact coverage of the trailing axis.
        sp.participants = r->grouping[1];
        sp.per_partition = r->grouping[2];
        const uint64_t per_round = sp.participants * sp.per_partition;
        sp.rounds = per_round && r->extents[r->rank - 1] % per_round == 0 ? r->extents[r->rank - 1] / per_round : 0;
      }
      st = tiler_rt::plan_fold(r->variant, r->rank, r->extents, r->grouping[0], r->scalars[0], r->scalars[1],
                               epi ? &prog : nullptr, p, c, &t, &sp, addr);
      break;
    }
    case TILER_HIP_PROGRAM_RMS_NORM:
      // Without permits_reassociation the serial fold of the reference runs;
      // with it, the grouped row fold (the declared grouping).
      st = tiler_rt::plan_rms_norm(t, r->dtype, bc ? 1 : 0, e[0], e[1], r->scalars[0], addr, p, !c.reassociate,
                                   c.input_mode, c.result_mode);
      break;
    case TILER_HIP_PROGRAM_SOFTMAX:
      st = r->dtype == TILER_HIP_F32
               ? tiler_rt::plan_softmax_f32(tiler_rt::Mode::Realized, t, e[0], e[1], addr, p, !c.reassociate, r->form,
                                            c.input_mode, c.result_mode)
               : p.refuse(TILER_HIP_REFUSE_UNSUPPORTED, "softmax is an f32 family");
      break;
    case TILER_HIP_PROGRAM_CONTRACTION:
      if (c.flushes()) {
        // A flushing contract: the strict fold with the modes at every site
        // (contraction.rs:600-625), td,od->to as the structure mk,nk->mn.
        if (live) {
          st = p.refuse(TILER_HIP_REFUSE_UNSUPPORTED, "live-extent: a flushing contraction's extents are fixed");
          break;
        }
        tiler_hip_contraction_structure mk{};
        if (!r->structure) {
          mk.operand_rank[0] = mk.operand_rank[1] = mk.output_rank = 2;
          mk.operand_indices[0][0] = 0, mk.operand_indices[0][1] = 2;  // m, k
          mk.operand_indices[1][0] = 1, mk.operand_indices[1][1] = 2;  // n, k
          mk.output_indices[0] = 0, mk.output_indices[1] = 1;
          mk.operand_dims[0][0] = e[0], mk.operand_dims[0][1] = e[2];
          mk.operand_dims[1][0] = e[1], mk.operand_dims[1][1] = e[2];
          if (e[0] == 0 || e[1] == 0) {  // no outputs: nothing to dispatch (the strict plan's own answer)
            st = r->dtype == TILER_HIP_F32 ? tiler_rt::plan_contract_strict_f32(t, e[0], e[1], e[2], addr, p, false)
                                           : tiler_rt::plan_contract_bf16(t, e[0], e[1], e[2], r->variant, addr, p,
                                                                          true, r->form, false);
            break;
          }
        }
        st = tiler_rt::plan_contract_general(t, r->dtype, r->structure ? *r->structure : mk, r->variant, true, addr, p,
                                             c.input_mode, c.result_mode);
      } else if (r->structure)
        st = live ? p.refuse(TILER_HIP_REFUSE_UNSUPPORTED, "live-extent: a structured contraction's extents are fixed")
                  : tiler_rt::plan_contract_general(t, r->dtype, *r->structure, r->variant, !c.reassociate, addr, p);
      else if (r->dtype == TILER_HIP_F32)
        st = r->variant == TILER_HIP_EPILOGUE_NONE
                 ? tiler_rt::plan_contract_strict_f32(t, e[0], e[1], e[2], addr, p, live)
                 : p.refuse(TILER_HIP_REFUSE_UNSUPPORTED, "the strict f32 contraction has no epilogue");
      else if (r->dtype == TILER_HIP_BF16)
        st = tiler_rt::plan_contract_bf16(t, e[0], e[1], e[2], r->variant, addr, p, !c.reassociate, r->form, live);
      else
        st = p.refuse(TILER_HIP_REFUSE_UNSUPPORTED, "contraction dtype");
      break;
    case TILER_HIP_PROGRAM_GATHER:
      st = tiler_rt::plan_gather(tiler_rt::Mode::Realized, e[0], e[1], e[2], r->variant, e[3],
                                 (r->flags & TILER_HIP_REGION_INDEX_SIGNED) ? 1 : 0, addr, p);
      break;
    case TILER_HIP_PROGRAM_BROADCAST:
      st = tiler_rt::plan_broadcast(r->grouping[0], r->rank, r->extents, r->strides, r->variant, p);
      break;
    case TILER_HIP_PROGRAM_REINDEX: {
      int64_t strides[8];
      for (uint32_t d = 0; d < 8; ++d) strides[d] = (int64_t)r->strides[d];
      st = tiler_rt::plan_reindex(r->grouping[0], r->rank, r->extents, strides, (int64_t)r->grouping[1],
                                  r->variant, p);
      break;
    }
    case TILER_HIP_PROGRAM_CONVERT:
      st = tiler_rt::plan_convert(tiler_rt::Mode::Realized, r->variant, e[0], addr, p);
      break;
    case TILER_HIP_PROGRAM_DEQUANTIZE_U4:
      // ScalarProgram::StrictAffineU4Dequantize reads [U8 codes, F32 scale,
      // U8 zero point] (model.rs:682-696); binary32 output only.
      st = r->dtype == TILER_HIP_F32
               ? tiler_rt::plan_dequantize_u4(tiler_rt::Mode::Realized, e[0], 0, 0, addr, p)
               : p.refuse(TILER_HIP_REFUSE_UNSUPPORTED, "the strict-affine U4 decode produces f32");
      break;
    default:
      st = p.refuse(TILER_HIP_REFUSE_UNSUPPORTED, "no realization for this scalar program");
  }
  if (st != TILER_HIP_OK) return st;
  if (p.constant.size() > TILER_HIP_REALIZATION_CONSTANT_BYTES)
    return p.refuse(TILER_HIP_REFUSE_CAPACITY, "the program's constant slot exceeds the realization's capacity");
  for (uint32_t i = 0; i < p.nlaunches; ++i) {
    if (p.launches[i].overflow) return p.refuse(TILER_HIP_REFUSE_CAPACITY, "argument segment overflow");
    if (entry_index(p.launches[i].symbol) == kEntryCount)
      return p.refuse(TILER_HIP_REFUSE_ABSENT_SYMBOL, (std::string("no payload entry for ") + p.launches[i].symbol).c_str());
  }
  return TILER_HIP_OK;
}

tiler_hip_status tiler_hip_realize(const tiler_hip_context* ctx, const tiler_hip_region* r,
                                   tiler_hip_realization* out, char* diagnostic,
                                   uint64_t diagnostic_bytes) try {
  if (!r || !out) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  std::memset(out, 0, sizeof(*out));
  tiler_rt::Program p;
  const tiler_hip_status st = plan_region(ctx, r, p);
  if (st != TILER_HIP_OK) {
    copy_text(diagnostic, diagnostic_bytes, p.diag);
    return st;
  }
  const bool al = (r->flags & TILER_HIP_REGION_ALIGNED16) != 0;
  out->slot_count = p.nslots;
  for (uint32_t i = 0; i < p.nslots; ++i) {
    out->slot_roles[i] = p.slot_roles[i];
    out->slot_bytes[i] = p.slot_bytes[i];
  }
  out->slot_alignment = al ? 16 : 1;
  out->constant_slot = p.constant_slot < p.nslots ? p.constant_slot : p.nslots;
  out->constant_bytes = (uint32_t)p.constant.size();
  if (!p.constant.empty()) std::memcpy(out->constant, p.constant.data(), p.constant.size());
  for (uint32_t i = 0; i < p.nlaunches; ++i) {
    const tiler_rt::Launch& l = p.launches[i];
    tiler_hip_realized_entry& d = out->entries[i];
    d.entry = entry_index(l.symbol);
    d.grid[0] = l.grid[0];
    d.grid[1] = l.grid[1];
    d.grid[2] = 1;
    d.block[0] = l.block;
    d.block[1] = d.block[2] = 1;
    d.kernarg_bytes = l.kernarg_bytes;
    std::memcpy(d.kernargs, l.kernargs, l.kernarg_bytes);
    d.binding_count = l.nbindings;
    for (uint32_t b = 0; b < l.nbindings; ++b) {
      d.binding_slots[b] = l.bindings[b].slot;
      d.binding_offsets[b] = l.bindings[b].offset;
    }
    d.extent_count = l.nextents;
    for (uint32_t x = 0; x < l.nextents; ++x) {
      d.extent_ids[x] = l.extents[x].id;
      d.extent_offsets[x] = l.extents[x].offset;
    }
  }
  out->entry_count = p.nlaunches;
  out->live_extent_count = p.nlive;
  for (uint32_t x = 0; x < p.nlive; ++x)
    out->live_extents[x] = {p.live[x].access, p.live[x].axis, p.live[x].minimum, p.live[x].bound};
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

// ---------------------------------------------------------------------------
// Physical-implementation provider.
namespace {

constexpr uint64_t kSaturatedParallelFoldSteps = 17870;  // the profile's measured cost row
constexpr uint64_t kCombineSteps = 6 + 4;                 // a workgroup's butterfly and wave partials
constexpr uint64_t kCombineWork = 256 * 6 + 4;
constexpr char kSerialBaseline[] = "tiler.region.serial-baseline";
constexpr char kMultiPassSplit[] = "tiler.reduction.multi-pass-split";
constexpr char kWorkgroupTree[] = "tiler.reduction.single-workgroup-tree";
constexpr char kReassociation[] = "numerics.reassociation";

uint64_t sat_add(uint64_t a, uint64_t b) { return a > UINT64_MAX - b ? UINT64_MAX : a + b; }
uint64_t sat_mul(uint64_t a, uint64_t b) { return a && b > UINT64_MAX / a ? UINT64_MAX : a * b; }
uint64_t ceil_div(uint64_t a, uint64_t b) { return a / b + (a % b != 0); }
// Contributor counts beyond this hold more than a petabyte of f32: the split's
// partition search (a walk down from the square root) is not run for them.
constexpr uint64_t kMaxPartitionedExtent = 1ull << 48;

uint64_t isqrt(uint64_t n) {
  uint64_t r = (uint64_t)std::sqrt((double)n);
  while (r > 0 && (r > n / r)) --r;
  while ((r + 1) <= n / (r + 1)) ++r;
  return r;
}

// The reference's split partition (tiler-compiler/src/physical.rs:2780-2798):
// the largest divisor c <= isqrt(n) leaving at least two partitions of c.
bool governed_partition(uint64_t n, uint64_t& partitions, uint64_t& per) {
  if (n < 4) return false;
  for (uint64_t c = isqrt(n); c >= 2; --c)
    if (n % c == 0 && n / c >= 2) {
      partitions = n / c;
      per = c;
      return true;
    }
  return false;
}

struct Stage {
  uint64_t work, depth;
};

// Fold steps of each stage of a sum strategy: work summed over every
// invocation, depth the longest sequential path (the same accounting the
// calibration sweep fits the row with).
std::vector<Stage> sum_stages(const tiler_rt::Target& t, const tiler_hip_region& r) {
  const uint64_t rows = r.extents[0], extent = r.extents[1], n = sat_mul(rows, extent);
  switch (r.topology) {
    case TILER_HIP_SUM_SERIAL:
      return {{n, extent}};
    case TILER_HIP_SUM_MULTIPASS:
      return {{n, r.grouping[1]}, {sat_mul(rows, r.grouping[0]), r.grouping[0]}};
    case TILER_HIP_SUM_COOPERATIVE: {
      const uint64_t P = r.grouping[0], c = r.grouping[1], R = r.grouping[2];
      return {{sat_add(n, sat_mul(rows, sat_mul(R, P))), sat_mul(R, sat_add(c, P))}};
    }
    default:
      if (rows == 1) {
        const uint64_t g = tiler_rt::tree_workgroups(t, n);
        return {{sat_add(n, g * kCombineWork), ceil_div(n, 256 * g) + kCombineSteps},
                {g + kCombineWork, ceil_div(g, 256) + kCombineSteps}};
      }
      return {{sat_mul(rows, sat_add(extent, kCombineWork)), ceil_div(extent, 256) + kCombineSteps}};
  }
}

uint64_t measured_fold_steps(const std::vector<Stage>& st) {
  uint64_t total = 0;
  for (const Stage& s : st) {
    const uint64_t span = sat_mul(s.depth, kSaturatedParallelFoldSteps);
    total = sat_add(total, s.work > span ? s.work : span);
  }
  return total;
}

struct Offer {
  tiler_hip_provider_offer* out;
  tiler_hip_status invalid = TILER_HIP_OK;  // an INVALID_ARGUMENT refusal, if one came back
  std::string invalid_diag;

  void decline(const char* strategy, uint32_t cause, const std::string& subject, uint64_t extent) {
    if (out->declined_count >= TILER_HIP_MAX_PROPOSALS) return;
    tiler_hip_declined_strategy& d = out->declined[out->declined_count++];
    copy_text(d.strategy, sizeof(d.strategy), strategy);
    d.cause = cause;
    copy_text(d.subject, sizeof(d.subject), subject);
    d.extent = extent;
  }

  // Plans `region` for `strategy`: a proposal, or a decline named from the
  // planner's refusal (a "rule: ..." diagnostic is a shape the strategy does
  // not admit at `extent`).
  int propose(const tiler_hip_context* ctx, const char* strategy, const tiler_hip_region& region, uint64_t extent,
              bool fold_steps) {
    tiler_rt::Program p;
    const tiler_hip_status st = plan_region(ctx, &region, p);
    if (st != TILER_HIP_OK) {
      if (st == TILER_HIP_REFUSE_INVALID_ARGUMENT && invalid == TILER_HIP_OK) {
        invalid = st;
        invalid_diag = p.diag;
      }
      const std::string diag = p.diag;
      const size_t colon = diag.find(':');
      if (st == TILER_HIP_REFUSE_UNSUPPORTED && colon != std::string::npos && diag.find(' ') > colon)
        decline(strategy, TILER_HIP_DECLINE_NO_ADMISSIBLE_SHAPE, diag.substr(0, colon), extent);
      else
        decline(strategy, TILER_HIP_DECLINE_UNREPRESENTABLE, diag, extent);
      return -1;
    }
    if (out->proposal_count >= TILER_HIP_MAX_PROPOSALS) return -1;
    tiler_hip_proposal& q = out->proposals[out->proposal_count];
    copy_text(q.strategy, sizeof(q.strategy), strategy);
    q.region = region;
    q.dispatch_count = p.nlaunches;
    for (uint32_t i = 0; i < p.nlaunches; ++i) {
      const tiler_rt::Launch& l = p.launches[i];
      copy_text(q.symbols[i], sizeof(q.symbols[i]), l.symbol);
      q.workgroups[i] = (uint64_t)l.grid[0] * l.grid[1];
      q.workgroup_threads[i] = l.block;
      q.launched_threads = sat_add(q.launched_threads, sat_mul(q.workgroups[i], l.block));
    }
    for (uint32_t i = 0; i < p.nslots; ++i)
      if (p.slot_roles[i] == tiler_rt::kSlotScratch) q.temporary_bytes = sat_add(q.temporary_bytes, p.slot_bytes[i]);
    q.measured_fold_steps = fold_steps ? measured_fold_steps(sum_stages(target_of(ctx), region)) : 0;
    return (int)out->proposal_count++;
  }
};

}  // namespace

tiler_hip_status tiler_hip_propose(const tiler_hip_context* ctx, const tiler_hip_region* r,
                                   tiler_hip_provider_offer* out, char* diagnostic, uint64_t diagnostic_bytes) try {
  if (!r || !out) return TILER_HIP_REFUSE_INVALID_ARGUMENT;
  std::memset(out, 0, sizeof(*out));
  copy_text(out->provider, sizeof(out->provider), "tiler.hip.gfx950-physical-provider");
  Offer o{out};
  tiler_hip_region base = *r;
  base.form = TILER_HIP_FORM_AUTO;
  const bool reassociate = (r->permissions & TILER_HIP_PERMITS_REASSOCIATION) != 0;
  tiler_hip_region strict = base;
  strict.permissions &= ~TILER_HIP_PERMITS_REASSOCIATION;
  // A reassociating strategy: proposed under the permission, else declined for it.
  auto regrouping = [&](const char* strategy, const tiler_hip_region& region, uint64_t extent, bool steps) {
    if (!reassociate) {
      o.decline(strategy, TILER_HIP_DECLINE_NUMERICAL_PERMISSION_REFUSED, kReassociation, 0);
      return -1;
    }
    return o.propose(ctx, strategy, region, extent, steps);
  };
  int chosen = -1;
  const uint64_t* e = r->extents;
  switch (r->program) {
    case TILER_HIP_PROGRAM_SERIAL_SUM: {
      tiler_hip_region v = strict;
      v.topology = TILER_HIP_SUM_SERIAL;
      o.propose(ctx, kSerialBaseline, v, e[1], true);
      uint64_t parts = 0, per = 0;
      if (!reassociate) {
        o.decline(kMultiPassSplit, TILER_HIP_DECLINE_NUMERICAL_PERMISSION_REFUSED, kReassociation, 0);
      } else if (e[1] > kMaxPartitionedExtent) {
        o.decline(kMultiPassSplit, TILER_HIP_DECLINE_UNREPRESENTABLE, "split-extent-unrepresentable", e[1]);
      } else if (!governed_partition(e[1], parts, per)) {
        o.decline(kMultiPassSplit, TILER_HIP_DECLINE_NO_ADMISSIBLE_SHAPE, "no-admissible-partition", e[1]);
      } else {
        v = base;
        v.topology = TILER_HIP_SUM_MULTIPASS;
        v.grouping[0] = parts;
        v.grouping[1] = per;
        v.grouping[2] = 0;
        o.propose(ctx, kMultiPassSplit, v, e[1], true);
      }
      v = base;
      v.topology = TILER_HIP_SUM_TREE;
      v.grouping[0] = v.grouping[1] = v.grouping[2] = 0;
      regrouping(e[0] == 1 ? "gfx950.reduction.grid-tree" : kWorkgroupTree, v, e[1], true);
      if (!reassociate) {
        o.decline("gfx950.reduction.cooperative-workgroup", TILER_HIP_DECLINE_NUMERICAL_PERMISSION_REFUSED,
                  kReassociation, 0);
      } else if (e[1] == 0 || e[1] % 256 != 0) {
        o.decline("gfx950.reduction.cooperative-workgroup", TILER_HIP_DECLINE_NO_ADMISSIBLE_SHAPE,
                  "no-admissible-participant-count", e[1]);
      } else {
        v = base;
        v.topology = TILER_HIP_SUM_COOPERATIVE;
        v.flags &= ~TILER_HIP_REGION_PARTICIPANT_MAJOR;
        v.grouping[0] = 256;
        v.grouping[1] = e[1] / 256;
        v.grouping[2] = 1;
        o.propose(ctx, "gfx950.reduction.cooperative-workgroup", v, e[1], true);
      }
      // The measured cost row's selector: the least fold steps.
      for (uint32_t i = 0; i < out->proposal_count; ++i)
        if (chosen < 0 || out->proposals[i].measured_fold_steps < out->proposals[chosen].measured_fold_steps)
          chosen = (int)i;
      break;
    }
    case TILER_HIP_PROGRAM_RMS_NORM:
    case TILER_HIP_PROGRAM_SOFTMAX: {
      const int s0 = o.propose(ctx, kSerialBaseline, strict, e[1], false);
      const uint64_t nseg = (e[1] + tiler_rt::kSoftmaxSegment - 1) / tiler_rt::kSoftmaxSegment;
      int g = -1;
      if (r->program == TILER_HIP_PROGRAM_SOFTMAX && nseg > 4) {
        tiler_hip_region v = base;
        v.form = TILER_HIP_FORM_SOFTMAX_ROW_SYNC;
        const int sync = regrouping("gfx950.softmax.row-synchronized", v, sat_mul(e[0], nseg), false);
        v.form = TILER_HIP_FORM_SOFTMAX_SPLIT;
        const int split = regrouping("gfx950.softmax.split", v, sat_mul(e[0], nseg), false);
        g = sync >= 0 ? sync : split;
      } else {
        g = regrouping("gfx950.rows.grouped-fold", base, e[1], false);
      }
      chosen = reassociate && g >= 0 ? g : s0;
      break;
    }
    case TILER_HIP_PROGRAM_CONTRACTION: {
      const int s0 = o.propose(ctx, kSerialBaseline, strict, r->structure ? 0 : e[2], false);
      if (r->dtype != TILER_HIP_BF16) {
        chosen = s0;
        break;
      }
      if (r->structure) {
        if (!reassociate) {
          o.decline("gfx950.contraction.mfma-batched", TILER_HIP_DECLINE_NUMERICAL_PERMISSION_REFUSED,
                    kReassociation, 0);
          chosen = s0;
          break;
        }
        tiler_rt::Program p;
        if (plan_region(ctx, &base, p) == TILER_HIP_OK && p.nlaunches &&
            std::strncmp(p.launches[p.nlaunches - 1].symbol, "tiler_contract_general", 22) == 0) {
          o.decline("gfx950.contraction.mfma-batched", TILER_HIP_DECLINE_NO_ADMISSIBLE_SHAPE,
                    "batched-operand-layout", 0);
          chosen = s0;
        } else {
          const int b = o.propose(ctx, "gfx950.contraction.mfma-batched", base, 0, false);
          chosen = b >= 0 ? b : s0;
        }
        break;
      }
      static const struct {
        const char* strategy;
        uint32_t form;
      } forms[] = {{"gfx950.contraction.mfma-skinny", TILER_HIP_FORM_CONTRACT_SKINNY},
                   {"gfx950.contraction.mfma-staged-256", TILER_HIP_FORM_CONTRACT_STAGED_256},
                   {"gfx950.contraction.mfma-staged-128", TILER_HIP_FORM_CONTRACT_STAGED_128},
                   {"gfx950.contraction.mfma-general-128", TILER_HIP_FORM_CONTRACT_GENERAL_128}};
      tiler_rt::Program autop;
      const bool auto_ok = reassociate && plan_region(ctx, &base, autop) == TILER_HIP_OK;
      chosen = s0;
      for (const auto& f : forms) {
        tiler_hip_region v = base;
        v.form = f.form;
        const uint64_t extent = f.form == TILER_HIP_FORM_CONTRACT_SKINNY ? e[0] : e[1] % 8 ? e[1] : e[2];
        const int i = regrouping(f.strategy, v, extent, false);
        if (i >= 0 && auto_ok && autop.nlaunches && out->proposals[i].dispatch_count == autop.nlaunches &&
            std::strcmp(out->proposals[i].symbols[0], autop.launches[0].symbol) == 0)
          chosen = i;
      }
      break;
    }
    default:
      chosen = o.propose(ctx, kSerialBaseline, base, 0, false);
  }
  if (out->proposal_count == 0 && o.invalid != TILER_HIP_OK) {
    const std::string why = o.invalid_diag;
    std::memset(out, 0, sizeof(*out));
    copy_text(diagnostic, diagnostic_bytes, why);
    return o.invalid;
  }
  out->chosen = chosen >= 0 ? (uint32_t)chosen : 0;
  copy_text(diagnostic, diagnostic_bytes, "");
  return TILER_HIP_OK;
} catch (...) {  // host memory exhausted: nothing unwinds through the C ABI
  return TILER_HIP_REFUSE_CAPACITY;
}

}  // extern "C"
