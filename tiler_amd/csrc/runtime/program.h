// Launch programs: what each realization family dispatches, as data.
//
// A planner turns one family request (shape, grouping, dtype, and the base
// address of every storage slot, which decides the vector width a kernel may
// assume) into a Program: the storage slots the dispatches touch (inputs,
// outputs, scratch) and the launches in execution order, each with its symbol,
// grid, workgroup size, packed kernel-argument segment and the argument fields
// that hold slot addresses.  The family entry points of the C ABI execute a
// Program on the spot; tiler_hip_realize exports the same Program as a
// dispatch plan for the RuntimeAdapter route.  Everything is fixed-capacity:
// planning allocates nothing.
#pragma once

#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "tiler_hip.h"

namespace tiler_rt {

constexpr uint32_t kMaxKernargBytes = 256;
constexpr uint32_t kMaxArgs = 12;
constexpr uint32_t kMaxBindings = 18;
constexpr uint32_t kMaxSlots = 18;
// Pointwise expressions: at most this many distinct inputs (one pointer each
// in the kernel's input table) and 16 registers in the register form.
constexpr uint32_t kMaxExpressionInputs = 16;
constexpr uint32_t kExpressionRegisters = 16;
constexpr uint32_t kExpressionInstrBytes = 12;
constexpr uint32_t kMaxLaunches = 4;
constexpr uint32_t kMaxSumWorkgroups = 4096;
// Bytes of partials a context keeps in its workspace (the sum's partials, the
// split softmax's segment maxima and sums); larger scratch is allocated.
constexpr uint64_t kWorkspacePartialBytes = 256 * 1024;
// Softmax rows longer than kWaveRowMax fold by segments of this many elements.
constexpr uint64_t kWaveRowMax = 8192;
constexpr uint64_t kSoftmaxSegment = 8192;
// The row-synchronized softmax keeps its 64-bit epoch and tagged words in a
// workspace area nothing else writes (256 header bytes, then 2 words of 8
// bytes per workgroup); it runs at most this many workgroups.
constexpr uint64_t kRowSyncMaxWorkgroups = 1024;
constexpr uint64_t kRowSyncBytes = 256 + 16 * kRowSyncMaxWorkgroups;
constexpr uint64_t kRowSyncDefaultWaitTicks = 20000;  // 200 us of the 100 MHz clock

// Slot roles, as tiler_hip_realization reports them.
constexpr uint32_t kSlotInput = TILER_HIP_SLOT_INPUT;
constexpr uint32_t kSlotOutput = TILER_HIP_SLOT_OUTPUT;
constexpr uint32_t kSlotScratch = TILER_HIP_SLOT_SCRATCH;

struct Binding {
  uint32_t offset;  // byte offset of the pointer field in the kernarg segment
  uint32_t slot;
  uint64_t addend;  // bytes past the slot base (direct execution only)
};

struct ExtentBinding {
  uint32_t offset;  // byte offset of the 32-bit field in the kernarg segment
  uint32_t id;      // the program's live extent
};

// A live extent (the program reads it at dispatch): input access, axis, and
// the range its value must lie in.
struct LiveExtent {
  uint32_t access, axis;
  uint64_t minimum, bound;
};
constexpr uint32_t kMaxLiveExtents = 2;

struct Launch {
  char symbol[64];
  uint32_t grid[2];
  uint32_t block;
  uint8_t kernargs[kMaxKernargBytes];
  uint32_t kernarg_bytes;
  uint32_t arg_offsets[kMaxArgs];
  uint32_t nargs;
  Binding bindings[kMaxBindings];
  uint32_t nbindings;
  ExtentBinding extents[kMaxLiveExtents];
  uint32_t nextents;
  bool overflow;  // an argument did not fit (a planner bug; refused)

  // Kernel arguments in declaration order, each at its natural alignment
  // (the HIP kernarg layout).
  Launch& ptr(uint32_t slot, uint64_t addend = 0);  // a slot address
  Launch& null_ptr();                               // a pointer argument bound to nothing
  Launch& u32(uint32_t v);
  Launch& u64(uint64_t v);
  Launch& f32(float v);
  Launch& live_u32(uint32_t id);  // a 32-bit field the dispatch fills with live extent `id`
  Launch& blob(const void* p, uint32_t bytes, uint32_t align);
  // A table of `count` pointers to slots (NULL past count), `capacity` wide.
  Launch& ptr_table(const uint32_t* slots, uint32_t count, uint32_t capacity);
};

struct Program {
  uint64_t slot_bytes[kMaxSlots];
  uint32_t slot_roles[kMaxSlots];
  uint32_t nslots;
  Launch launches[kMaxLaunches];
  uint32_t nlaunches;
  std::string diag;
  // The CONSTANT slot's contents (an expression's register program), if any.
  uint32_t constant_slot = kMaxSlots;
  std::vector<uint8_t> constant;
  LiveExtent live[kMaxLiveExtents];
  uint32_t nlive = 0;

  Program();
  uint32_t slot(uint64_t bytes, uint32_t role);
  Launch& add(const char* symbol, uint32_t gx, uint32_t gy, uint32_t block);
  tiler_hip_status refuse(tiler_hip_status st, const char* what) {
    diag = what;
    return st;
  }
};

// What a planner may assume about the device.
struct Target {
  uint32_t compute_units;
  uint64_t row_sync_wait_ticks;  // the row-synchronized softmax's wait bound
};

// The plan's numerical contract as one region states it.  Zero-initialized
// is the strict contract.
struct Contract {
  bool reassociate = false;     // permits_reassociation
  uint32_t input_mode = 1;      // 1 preserve, 2 flush sign-preserving, 3 flush to +0
  uint32_t result_mode = 1;
  bool flushes() const { return input_mode > 1 || result_mode > 1; }
};

// Host mirror of the kernels' tiler::FoldRule (common.h): a serial sum's
// per-contributor prologue and the two subnormal modes at every site.
struct FoldRuleHost {
  uint32_t prologue = 0;  // 0 none, 1 squared, 2 scale-bias
  float scale = 1.0f, bias = 0.0f;
  uint32_t in_mode = 1, out_mode = 1;
};

// A pointwise expression compiled for the interpreter kernels (expr.hip):
// instructions in execution order (the inputs first, input k into register
// k), the result register, and the register count the program needs.
struct ExpressionProgram {
  std::vector<uint8_t> code;  // 12-byte instructions
  uint32_t count = 0, inputs = 0, registers = 0, result = 0;
};

// Checks a DAG the way the reference's verifier does
// (tiler-ir/src/schedule/pointwise.rs:185-240: operands defined before use,
// dense input ordinals each named once, every node reachable from the root,
// the node limit; pointwise_bf16.rs: the bf16 vocabulary) and compiles it.
tiler_hip_status compile_expression(uint32_t dtype, const tiler_hip_expression_node* nodes, uint32_t count,
                                    uint32_t root, bool epilogue, ExpressionProgram& out, std::string& diag);

// Direct: the program runs now, on known addresses (it may bind a slot at an
// offset, and the gather record is armed by the context).  Realized: the
// program is exported as a dispatch plan (no offsets; it arms its own record).
enum class Mode { Direct, Realized };

// Workgroups of the single-output tree for n contributors.
uint32_t tree_workgroups(const Target& t, uint64_t n);

// Planners.  Slot order is part of each contract (tiler_hip_realize documents
// it); `addr` holds each slot's base address, or a stand-in whose low bits
// carry the alignment a realization may assume.
// rule (NULL: the plain strict fold under the preserving modes) selects the
// rule-driven kernels: a flushing contract, or a fused prologue.
tiler_hip_status plan_sum_f32(const Target& t, uint64_t rows, uint64_t extent,
                              const tiler_hip_sum_plan& sp, const uintptr_t* addr, Program& p,
                              const FoldRuleHost* rule = nullptr);
tiler_hip_status plan_rms_norm(const Target& t, uint32_t dtype, int32_t weight_broadcast, uint64_t rows,
                               uint64_t extent, uint32_t eps_bits, const uintptr_t* addr,
                               Program& p, bool strict = false, uint32_t in_mode = 1, uint32_t out_mode = 1);
// `form` (TILER_HIP_FORM_SOFTMAX_*) forces the split or the row-synchronized
// launch for rows of more than four segments.
tiler_hip_status plan_softmax_f32(Mode mode, const Target& t, uint64_t rows, uint64_t extent,
                                  const uintptr_t* addr, Program& p, bool strict = false,
                                  uint32_t form = TILER_HIP_FORM_AUTO, uint32_t in_mode = 1,
                                  uint32_t out_mode = 1);
tiler_hip_status plan_map(Mode mode, uint32_t op, uint32_t dtype, int32_t x2_broadcast,
                          uint64_t n, float a, float b, const uintptr_t* addr, Program& p,
                          uint32_t in_mode = 1, uint32_t out_mode = 1);
tiler_hip_status plan_broadcast(uint64_t src_elements, uint32_t rank, const uint64_t* out_dims,
                                const uint64_t* src_strides, uint32_t element_bytes,
                                Program& p);
tiler_hip_status plan_gather(Mode mode, uint64_t outer, uint64_t gathered, uint64_t inner,
                             uint32_t element_bytes, uint64_t count, int32_t index_signed,
                             const uintptr_t* addr, Program& p);
tiler_hip_status plan_convert(Mode mode, uint32_t direction, uint64_t n, const uintptr_t* addr,
                              Program& p);
// live_k: k is read at dispatch (live extent 0, input 0 axis 1, in [1, k]);
// the slots hold operands of the bound k.
tiler_hip_status plan_dequantize_u4(Mode mode, uint64_t n, uint32_t scale_bits, uint32_t zero_point,
                                    const uintptr_t* addr, Program& p);
tiler_hip_status plan_contract_strict_f32(const Target& t, uint64_t m, uint64_t n, uint64_t k, const uintptr_t* addr,
                                          Program& p, bool live_k = false);
// Any admitted binary index structure: the strict fold (f32, or bf16 without
// reassociation), or under it the batched MFMA forms where the structure is
// [batch.., m, k] x [batch.., n, k | k, n] -> [batch.., m, n].
tiler_hip_status plan_contract_general(const Target& t, uint32_t dtype, const tiler_hip_contraction_structure& s,
                                       uint32_t epilogue, bool strict, const uintptr_t* addr, Program& p,
                                       uint32_t in_mode = 1, uint32_t out_mode = 1);
// `form` (TILER_HIP_FORM_CONTRACT_*) forces one MFMA form, refusing when the
// request does not admit it; TILER_HIP_FORM_AUTO lets the planner choose.
tiler_hip_status plan_contract_bf16(const Target& t, uint64_t m, uint64_t n, uint64_t k,
                                    uint32_t epilogue, const uintptr_t* addr, Program& p,
                                    bool strict = false, uint32_t form = TILER_HIP_FORM_AUTO,
                                    bool live_k = false);
// Pointwise expression over n elements: slots inputs 0..I-1, y, program
// (CONSTANT), and -- for programs beyond the register form -- the value
// store (SCRATCH).  `addr` covers the inputs then y.
tiler_hip_status plan_expression(const Target& t, uint32_t dtype, uint64_t n, const ExpressionProgram& prog,
                                 const Contract& c, const uintptr_t* addr, Program& p);
// Serial fold of a dense row-major tensor over the axes in `reduced_mask`.
// Slots: x, out, and the epilogue's program (CONSTANT) when one is given.
tiler_hip_status plan_fold(uint32_t op, uint32_t rank, const uint64_t* dims, uint64_t reduced_mask,
                           uint32_t scale_bits, uint32_t bias_bits, const ExpressionProgram* epilogue,
                           Program& p, const Contract& c = Contract{}, const Target* t = nullptr,
                           const tiler_hip_sum_plan* sp = nullptr, const uintptr_t* addr = nullptr);
// Reindex with signed strides: out (row-major over out_dims) reads source
// offset base + sum coord_d * strides[d].  Slots: src, out.
tiler_hip_status plan_reindex(uint64_t src_elements, uint32_t rank, const uint64_t* out_dims,
                              const int64_t* strides, int64_t base, uint32_t element_bytes, Program& p);

}  // namespace tiler_rt
