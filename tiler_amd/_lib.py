"""ctypes binding of libtiler_hip.so (the C ABI in include/tiler_hip.h).

The library is built ahead of time (``python -m tiler_amd.build``) and loaded
from ``tiler_amd/_build``.  There is no fallback: if the library is missing
every entry point raises, so nothing can silently run on the CPU.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "libtiler_hip.so")

OK = 0
REFUSE_NO_DEVICE = -1
REFUSE_FOREIGN_TARGET = -2
REFUSE_INVALID_ARGUMENT = -3
REFUSE_MALFORMED_PAYLOAD = -4
REFUSE_ABSENT_SYMBOL = -5
REFUSE_BINDING_MISMATCH = -6
REFUSE_CAPACITY = -7
REFUSE_UNSUPPORTED = -8
REFUSE_GATHER_INDEX_OUT_OF_BOUNDS = -9
REFUSE_UNRECOGNIZED_KEY = -10
REFUSE_NOT_PREPARED = -11
REFUSE_PAYLOAD_MISMATCH = -12
FAIL_ALLOCATION = 1
FAIL_LAUNCH = 2
FAIL_DEVICE = 3
FAIL_GATHER_INDEX_OUT_OF_BOUNDS = 4
FAIL_TRANSFER = 5
FAIL_VALUE_DOMAIN = 6

F32 = 0
BF16 = 1

SUM_SERIAL = 0
SUM_TREE = 1
SUM_MULTIPASS = 2
SUM_COOPERATIVE = 3

MAP_SCALE_BIAS = 0
MAP_SILU = 1
MAP_ADD = 2
MAP_MULTIPLY = 3

ROWS_RMS_NORM = 0
ROWS_SOFTMAX = 1
ROWS_SUM = 2

EPILOGUE_NONE = 0
EPILOGUE_SILU = 1

PROGRAM_POINTWISE = 1
PROGRAM_SERIAL_SUM = 2
PROGRAM_RMS_NORM = 3
PROGRAM_SOFTMAX = 4
PROGRAM_CONTRACTION = 5
PROGRAM_GATHER = 6
PROGRAM_BROADCAST = 7
PROGRAM_CONVERT = 8
PROGRAM_EXPRESSION = 9
PROGRAM_FOLD = 10
PROGRAM_REINDEX = 11
PROGRAM_DEQUANTIZE_U4 = 12

FOLD_SUM = 0
FOLD_SQUARED = 1
FOLD_FMA = 2
FOLD_MAXIMUM = 3

NODE_INPUT = 0
NODE_CONSTANT = 1
NODE_ADD = 2
NODE_MULTIPLY = 3
NODE_DIVIDE = 4
NODE_EXP = 5
NODE_RSQRT = 6
MAX_EXPRESSION_NODES = 4096

PERMITS_REASSOCIATION = 1
PERMITS_PERMUTATION = 2
SUBNORMALS_PRESERVE = 1
SUBNORMALS_FLUSH_SIGN = 2
SUBNORMALS_FLUSH_POSITIVE = 3

CONVERT_NARROW_F32_BF16 = 0
CONVERT_WIDEN_BF16_F32 = 1

FORM_AUTO = 0
FORM_CONTRACT_SKINNY = 1
FORM_CONTRACT_STAGED_256 = 2
FORM_CONTRACT_STAGED_128 = 3
FORM_CONTRACT_GENERAL_128 = 4
FORM_SOFTMAX_SPLIT = 5
FORM_SOFTMAX_ROW_SYNC = 6

MAX_PROPOSALS = 6
DECLINE_NUMERICAL_PERMISSION_REFUSED = 1
DECLINE_NO_ADMISSIBLE_SHAPE = 2
DECLINE_UNREPRESENTABLE = 3

REGION_ALIGNED16 = 1
REGION_OPERAND_BROADCAST = 2
REGION_INDEX_SIGNED = 4
REGION_PARTICIPANT_MAJOR = 8
REGION_LIVE_EXTENT = 16

SLOT_INPUT = 0
SLOT_OUTPUT = 1
SLOT_SCRATCH = 2
SLOT_CONSTANT = 3
REALIZATION_CONSTANT_BYTES = 49152
MAX_SLOTS = 18
MAX_LIVE_EXTENTS = 2


class TargetProfile(ctypes.Structure):
    _fields_ = [
        ("profile_key", ctypes.c_char * 64),
        ("target_triple", ctypes.c_char * 64),
        ("wavefront_size", ctypes.c_uint32),
        ("compute_units", ctypes.c_uint32),
        ("xcds", ctypes.c_uint32),
        ("simds_per_cu", ctypes.c_uint32),
        ("max_threads_per_workgroup", ctypes.c_uint32),
        ("max_grid_dim", ctypes.c_uint32 * 3),
        ("lds_bytes_per_workgroup", ctypes.c_uint64),
        ("device_memory_bytes", ctypes.c_uint64),
        ("l2_bytes_per_xcd", ctypes.c_uint64),
        ("infinity_cache_bytes", ctypes.c_uint64),
        ("address_bits", ctypes.c_uint32),
        ("index_u64", ctypes.c_uint32),
        ("subgroup_width", ctypes.c_uint32),
        ("f32_subnormals_preserved", ctypes.c_uint32),
        ("hbm_bytes_per_second", ctypes.c_double),
        ("mfma_bf16_dense_flops", ctypes.c_double),
        ("mfma_fp8_dense_flops", ctypes.c_double),
        ("vector_f32_flops", ctypes.c_double),
        ("vector_f64_flops", ctypes.c_double),
        ("saturated_parallel_fold_steps", ctypes.c_uint64),
        ("cost_row_source", ctypes.c_char * 192),
    ]


class PayloadView(ctypes.Structure):
    _fields_ = [
        ("backend", ctypes.c_char_p),
        ("representation", ctypes.c_char_p),
        ("payload_schema", ctypes.c_char_p),
        ("target", ctypes.c_char_p),
        ("toolchain", ctypes.c_char_p),
        ("flags", ctypes.c_char_p),
        ("code", ctypes.c_void_p),
        ("code_bytes", ctypes.c_uint64),
        ("entry_count", ctypes.c_uint32),
        ("source", ctypes.c_void_p),
        ("source_bytes", ctypes.c_uint64),
    ]


class EntryInfo(ctypes.Structure):
    _fields_ = [
        ("symbol", ctypes.c_char_p),
        ("family", ctypes.c_char_p),
        ("buffer_bindings", ctypes.c_uint32),
        ("kernarg_bytes", ctypes.c_uint32),
    ]


class ExecutionEnvironment(ctypes.Structure):
    _fields_ = [
        ("device_ordinal", ctypes.c_int32),
        ("device_name", ctypes.c_char * 64),
        ("gcn_arch_name", ctypes.c_char * 64),
        ("compute_units", ctypes.c_uint32),
        ("wavefront_size", ctypes.c_uint32),
        ("max_threads_per_workgroup", ctypes.c_uint32),
        ("lds_bytes_per_workgroup", ctypes.c_uint64),
        ("global_memory_bytes", ctypes.c_uint64),
        ("clock_khz", ctypes.c_int32),
        ("memory_clock_khz", ctypes.c_int32),
        ("memory_bus_width_bits", ctypes.c_int32),
        ("runtime_version", ctypes.c_int32),
        ("driver_version", ctypes.c_int32),
    ]


class RoutedEntry(ctypes.Structure):
    _fields_ = [
        ("code", ctypes.c_void_p),
        ("code_bytes", ctypes.c_uint64),
        ("symbol", ctypes.c_char_p),
    ]


class DispatchEntry(ctypes.Structure):
    _fields_ = [
        ("prepared", ctypes.c_uint32),
        ("grid", ctypes.c_uint32 * 3),
        ("block", ctypes.c_uint32 * 3),
        ("dynamic_lds_bytes", ctypes.c_uint32),
        ("kernargs", ctypes.c_void_p),
        ("kernarg_bytes", ctypes.c_uint32),
        ("binding_count", ctypes.c_uint32),
        ("binding_slots", ctypes.POINTER(ctypes.c_uint32)),
        ("binding_offsets", ctypes.POINTER(ctypes.c_uint32)),
        ("extent_count", ctypes.c_uint32),
        ("extent_ids", ctypes.POINTER(ctypes.c_uint32)),
        ("extent_offsets", ctypes.POINTER(ctypes.c_uint32)),
    ]


class LiveExtent(ctypes.Structure):
    _fields_ = [
        ("access", ctypes.c_uint32),
        ("axis", ctypes.c_uint32),
        ("minimum", ctypes.c_uint64),
        ("bound", ctypes.c_uint64),
    ]


class DispatchPlan(ctypes.Structure):
    _fields_ = [
        ("slot_count", ctypes.c_uint32),
        ("slot_bytes", ctypes.POINTER(ctypes.c_uint64)),
        ("entry_count", ctypes.c_uint32),
        ("entries", ctypes.POINTER(DispatchEntry)),
        ("slot_contents", ctypes.POINTER(ctypes.c_void_p)),
        ("extent_count", ctypes.c_uint32),
        ("extents", ctypes.POINTER(ctypes.c_uint64)),
        ("extent_ranges", ctypes.POINTER(LiveExtent)),
    ]


class TargetEnvironmentSchema(ctypes.Structure):
    _fields_ = [
        ("provider", ctypes.c_char * 64),
        ("provider_revision", ctypes.c_uint32),
        ("schema_major", ctypes.c_uint16),
        ("schema_minor", ctypes.c_uint16),
    ]


class SumPlan(ctypes.Structure):
    _fields_ = [
        ("topology", ctypes.c_uint32),
        ("participant_major", ctypes.c_uint32),
        ("partitions", ctypes.c_uint64),
        ("participants", ctypes.c_uint64),
        ("per_partition", ctypes.c_uint64),
        ("rounds", ctypes.c_uint64),
    ]


class ExpressionNode(ctypes.Structure):
    _fields_ = [("op", ctypes.c_uint32), ("a", ctypes.c_uint32), ("b", ctypes.c_uint32)]


class ContractionStructure(ctypes.Structure):
    _fields_ = [
        ("operand_rank", ctypes.c_uint32 * 2),
        ("output_rank", ctypes.c_uint32),
        ("reserved", ctypes.c_uint32),
        ("operand_indices", (ctypes.c_uint32 * 8) * 2),
        ("output_indices", ctypes.c_uint32 * 8),
        ("operand_dims", (ctypes.c_uint64 * 8) * 2),
    ]


def contraction_structure(left_idx, left_dims, right_idx, right_dims, out_idx) -> ContractionStructure:
    """Labels are strings of single characters or sequences of ints."""
    def labels(x):
        return [ord(c) for c in x] if isinstance(x, str) else [int(v) for v in x]
    s = ContractionStructure()
    for side, (idx, dims) in enumerate(((left_idx, left_dims), (right_idx, right_dims))):
        lab = labels(idx)
        s.operand_rank[side] = len(lab)
        for a, (v, d) in enumerate(zip(lab, dims)):
            s.operand_indices[side][a] = v
            s.operand_dims[side][a] = int(d)
    out = labels(out_idx)
    s.output_rank = len(out)
    for a, v in enumerate(out):
        s.output_indices[a] = v
    return s


class Region(ctypes.Structure):
    _fields_ = [
        ("program", ctypes.c_uint32),
        ("topology", ctypes.c_uint32),
        ("dtype", ctypes.c_uint32),
        ("variant", ctypes.c_uint32),
        ("flags", ctypes.c_uint32),
        ("rank", ctypes.c_uint32),
        ("extents", ctypes.c_uint64 * 8),
        ("strides", ctypes.c_uint64 * 8),
        ("grouping", ctypes.c_uint64 * 3),
        ("scalars", ctypes.c_uint32 * 2),
        ("permissions", ctypes.c_uint32),
        ("input_subnormals", ctypes.c_uint32),
        ("result_subnormals", ctypes.c_uint32),
        ("node_count", ctypes.c_uint32),
        ("root", ctypes.c_uint32),
        ("nodes", ctypes.POINTER(ExpressionNode)),
        ("structure", ctypes.POINTER(ContractionStructure)),
        ("form", ctypes.c_uint32),
        ("reserved", ctypes.c_uint32),
    ]


class Proposal(ctypes.Structure):
    _fields_ = [
        ("strategy", ctypes.c_char * 64),
        ("region", Region),
        ("dispatch_count", ctypes.c_uint32),
        ("launched_threads", ctypes.c_uint64),
        ("temporary_bytes", ctypes.c_uint64),
        ("symbols", (ctypes.c_char * 48) * 4),
        ("workgroups", ctypes.c_uint64 * 4),
        ("workgroup_threads", ctypes.c_uint32 * 4),
        ("measured_fold_steps", ctypes.c_uint64),
    ]


class DeclinedStrategy(ctypes.Structure):
    _fields_ = [
        ("strategy", ctypes.c_char * 64),
        ("cause", ctypes.c_uint32),
        ("subject", ctypes.c_char * 64),
        ("extent", ctypes.c_uint64),
    ]


class ProviderOffer(ctypes.Structure):
    _fields_ = [
        ("provider", ctypes.c_char * 64),
        ("proposal_count", ctypes.c_uint32),
        ("declined_count", ctypes.c_uint32),
        ("chosen", ctypes.c_uint32),
        ("proposals", Proposal * MAX_PROPOSALS),
        ("declined", DeclinedStrategy * MAX_PROPOSALS),
    ]


class RealizedEntry(ctypes.Structure):
    _fields_ = [
        ("entry", ctypes.c_uint32),
        ("grid", ctypes.c_uint32 * 3),
        ("block", ctypes.c_uint32 * 3),
        ("kernarg_bytes", ctypes.c_uint32),
        ("kernargs", ctypes.c_uint8 * 256),
        ("binding_count", ctypes.c_uint32),
        ("binding_slots", ctypes.c_uint32 * MAX_SLOTS),
        ("binding_offsets", ctypes.c_uint32 * MAX_SLOTS),
        ("extent_count", ctypes.c_uint32),
        ("extent_ids", ctypes.c_uint32 * MAX_LIVE_EXTENTS),
        ("extent_offsets", ctypes.c_uint32 * MAX_LIVE_EXTENTS),
    ]


class Realization(ctypes.Structure):
    _fields_ = [
        ("slot_count", ctypes.c_uint32),
        ("slot_roles", ctypes.c_uint32 * MAX_SLOTS),
        ("slot_bytes", ctypes.c_uint64 * MAX_SLOTS),
        ("slot_alignment", ctypes.c_uint32),
        ("entry_count", ctypes.c_uint32),
        ("entries", RealizedEntry * 4),
        ("constant_slot", ctypes.c_uint32),
        ("constant_bytes", ctypes.c_uint32),
        ("constant", ctypes.c_uint8 * REALIZATION_CONSTANT_BYTES),
        ("live_extent_count", ctypes.c_uint32),
        ("live_extents", LiveExtent * MAX_LIVE_EXTENTS),
    ]


class EnvelopePayload(ctypes.Structure):
    _fields_ = [
        ("backend", ctypes.c_void_p), ("backend_bytes", ctypes.c_uint64),
        ("representation", ctypes.c_void_p), ("representation_bytes", ctypes.c_uint64),
        ("payload_schema_major", ctypes.c_uint16), ("payload_schema_minor", ctypes.c_uint16),
        ("digest", ctypes.c_void_p), ("digest_bytes", ctypes.c_uint64),
        ("profile_key", ctypes.c_void_p), ("profile_key_bytes", ctypes.c_uint64),
        ("profile_descriptor", ctypes.c_void_p), ("profile_descriptor_bytes", ctypes.c_uint64),
        ("has_environment", ctypes.c_uint32),
        ("carried", ctypes.c_uint32),
        ("metadata_section", ctypes.c_uint32), ("code_section", ctypes.c_uint32),
        ("metadata", ctypes.c_void_p), ("metadata_bytes", ctypes.c_uint64),
        ("code", ctypes.c_void_p), ("code_bytes", ctypes.c_uint64),
    ]


class Envelope(ctypes.Structure):
    _fields_ = [
        ("total_bytes", ctypes.c_uint64), ("manifest_bytes", ctypes.c_uint64),
        ("manifest_schema_major", ctypes.c_uint16), ("manifest_schema_minor", ctypes.c_uint16),
        ("section_count", ctypes.c_uint32),
        ("section_purpose", ctypes.c_uint8 * 64),
        ("feature_count", ctypes.c_uint64), ("input_count", ctypes.c_uint64),
        ("output_count", ctypes.c_uint64), ("provider_count", ctypes.c_uint64),
        ("payload_count", ctypes.c_uint32),
        ("payloads", EnvelopePayload * 16),
        ("identity_digest", ctypes.c_uint8 * 32),
    ]


class PayloadMapping(ctypes.Structure):
    _fields_ = [
        ("key", ctypes.c_void_p), ("key_bytes", ctypes.c_uint64),
        ("symbol", ctypes.c_void_p), ("symbol_bytes", ctypes.c_uint64),
        ("transport_count", ctypes.c_uint32),
        ("transports", ctypes.c_void_p),
    ]


class PayloadSubject(ctypes.Structure):
    _fields_ = [
        ("source_representation", ctypes.c_void_p), ("source_representation_bytes", ctypes.c_uint64),
        ("source", ctypes.c_void_p), ("source_bytes", ctypes.c_uint64),
        ("toolchain", ctypes.c_void_p), ("toolchain_bytes", ctypes.c_uint64),
        ("target", ctypes.c_void_p), ("target_bytes", ctypes.c_uint64),
        ("family", ctypes.c_void_p), ("family_bytes", ctypes.c_uint64),
        ("language", ctypes.c_void_p), ("language_bytes", ctypes.c_uint64),
        ("deployment_major", ctypes.c_uint16), ("deployment_minor", ctypes.c_uint16),
        ("unversioned", ctypes.c_uint32),
        ("component_count", ctypes.c_uint64), ("compile_flag_count", ctypes.c_uint64),
        ("link_flag_count", ctypes.c_uint64), ("obligation_count", ctypes.c_uint64),
        ("entry_count", ctypes.c_uint64),
    ]


_P = ctypes.c_void_p
_U64 = ctypes.c_uint64
_U32 = ctypes.c_uint32
_I32 = ctypes.c_int32
_F = ctypes.c_float
_S = ctypes.c_int32
_CTX = ctypes.c_void_p

SIGNATURES = {
    "tiler_hip_profile_declare": (_S, [ctypes.POINTER(TargetProfile)]),
    "tiler_hip_payload": (_S, [ctypes.POINTER(PayloadView)]),
    "tiler_hip_payload_entry": (_S, [_U32, ctypes.POINTER(EntryInfo)]),
    "tiler_hip_validate_payload": (_S, [_P, _U64, ctypes.c_char_p, _U32, ctypes.c_char_p, _U64]),
    "tiler_hip_bind": (_S, [_I32, ctypes.POINTER(_CTX), ctypes.POINTER(ExecutionEnvironment),
                            ctypes.c_char_p, _U64]),
    "tiler_hip_release": (None, [_CTX]),
    "tiler_hip_last_diagnostic": (ctypes.c_char_p, [_CTX]),
    "tiler_hip_observe_live_device": (_S, [_CTX, ctypes.c_char_p, ctypes.POINTER(_U64)]),
    "tiler_hip_prepare_entries": (_S, [_CTX, ctypes.POINTER(RoutedEntry), _U32,
                                       ctypes.POINTER(_U32)]),
    "tiler_hip_observe_prepared_entry": (_S, [_CTX, _U32, ctypes.c_char_p, ctypes.POINTER(_U64)]),
    "tiler_hip_plan_dispatch": (_S, [_CTX, ctypes.POINTER(DispatchPlan)]),
    "tiler_hip_allocate_dispatch": (_S, [_CTX, ctypes.POINTER(DispatchPlan), ctypes.POINTER(_P)]),
    "tiler_hip_dispatch": (_S, [_CTX, ctypes.POINTER(DispatchPlan), ctypes.POINTER(_P)]),
    "tiler_hip_enqueue_dispatch": (_S, [_CTX, ctypes.POINTER(DispatchPlan), ctypes.POINTER(_P), _P]),
    "tiler_hip_release_dispatch": (_S, [_CTX, ctypes.POINTER(DispatchPlan), ctypes.POINTER(_P),
                                        ctypes.POINTER(_P)]),
    "tiler_hip_buffer_alloc": (_S, [_CTX, _U64, ctypes.POINTER(_P)]),
    "tiler_hip_buffer_free": (_S, [_CTX, _P]),
    "tiler_hip_upload": (_S, [_CTX, _P, _P, _U64]),
    "tiler_hip_download": (_S, [_CTX, _P, _P, _U64]),
    "tiler_hip_fill_u32": (_S, [_CTX, _P, _U32, _U64, _P]),
    "tiler_hip_copy": (_S, [_CTX, _P, _P, _U64, _P]),
    "tiler_hip_synchronize": (_S, [_CTX]),
    "tiler_hip_context_stream": (_P, [_CTX]),
    "tiler_hip_event_create": (_S, [_CTX, ctypes.POINTER(_P)]),
    "tiler_hip_event_record": (_S, [_CTX, _P, _P]),
    "tiler_hip_event_elapsed_ms": (_S, [_CTX, _P, _P, ctypes.POINTER(_F)]),
    "tiler_hip_event_destroy": (_S, [_CTX, _P]),
    "tiler_hip_capture_begin": (_S, [_CTX, _P]),
    "tiler_hip_capture_end": (_S, [_CTX, _P, ctypes.POINTER(_P)]),
    "tiler_hip_graph_launch": (_S, [_CTX, _P, _P]),
    "tiler_hip_graph_destroy": (_S, [_CTX, _P]),
    "tiler_hip_sum_f32": (_S, [_CTX, _P, _U64, _U64, _P, ctypes.POINTER(SumPlan), _P]),
    "tiler_hip_sum_f32_noalloc": (_S, [_CTX, _P, _U64, _U64, _P, ctypes.POINTER(SumPlan), _P]),
    "tiler_hip_sum_tree_workgroups": (_U32, [_CTX, _U64]),
    "tiler_hip_row_grouping": (_S, [_U32, _U32, _U64, ctypes.POINTER(_U32), ctypes.POINTER(_U32),
                                    ctypes.POINTER(_U64)]),
    "tiler_hip_rms_norm": (_S, [_CTX, _U32, _P, _P, _I32, _U64, _U64, _U32, _P, _P]),
    "tiler_hip_softmax_f32": (_S, [_CTX, _P, _U64, _U64, _P, _P]),
    "tiler_hip_map": (_S, [_CTX, _U32, _U32, _P, _P, _I32, _U64, _F, _F, _P, _P]),
    "tiler_hip_broadcast": (_S, [_CTX, _P, _U64, _U32, ctypes.POINTER(_U64), ctypes.POINTER(_U64),
                                 _U32, _P, _P]),
    "tiler_hip_gather": (_S, [_CTX, _P, _U64, _U64, _U64, _U32, _P, _U64, _I32, _P, _P]),
    "tiler_hip_convert": (_S, [_CTX, _U32, _P, _U64, _P, _P]),
    "tiler_hip_dequantize_u4": (_S, [_CTX, _P, _U64, _U32, _U32, _P, _P]),
    "tiler_hip_gather_status": (_S, [_CTX, _P, ctypes.POINTER(_U64)]),
    "tiler_hip_validate_gather_index": (_S, [_P, _U64, _I32, _U64, ctypes.POINTER(_U64),
                                             ctypes.POINTER(ctypes.c_int64)]),
    "tiler_hip_contract_strict_f32": (_S, [_CTX, _P, _P, _U64, _U64, _U64, _P, _P]),
    "tiler_hip_contract_bf16": (_S, [_CTX, _P, _P, _U64, _U64, _U64, _P, _U32, _P]),
    "tiler_hip_contract": (_S, [_CTX, _U32, ctypes.POINTER(ContractionStructure), _U32, _U32, _P, _P, _P, _P]),
    "tiler_hip_realize": (_S, [_CTX, ctypes.POINTER(Region), ctypes.POINTER(Realization),
                               ctypes.c_char_p, _U64]),
    "tiler_hip_propose": (_S, [_CTX, ctypes.POINTER(Region), ctypes.POINTER(ProviderOffer),
                               ctypes.c_char_p, _U64]),
    "tiler_hip_expression": (_S, [_CTX, _U32, ctypes.POINTER(ExpressionNode), _U32, _U32,
                                  ctypes.POINTER(_P), _U64, _P, _U32, _U32, _P]),
    "tiler_hip_fold_f32": (_S, [_CTX, _U32, _P, _U32, ctypes.POINTER(_U64), _U64, _U32, _U32, _P, _P]),
    "tiler_hip_reindex": (_S, [_CTX, _P, _U64, _U32, ctypes.POINTER(_U64), ctypes.POINTER(ctypes.c_int64),
                               ctypes.c_int64, _U32, _P, _P]),
    "tiler_hip_target_environment_support": (_S, [ctypes.POINTER(TargetEnvironmentSchema)]),
    "tiler_hip_validate_target_environment": (_S, [_P, _U64, ctypes.c_char_p, _U64]),
    "tiler_hip_observe_target_environment": (_S, [_CTX, _P, _U64, ctypes.POINTER(_U64), ctypes.POINTER(_U32),
                                                  ctypes.c_char_p, _U64]),
    "tiler_hip_payload_metadata": (_S, [_P, _U64, ctypes.POINTER(_U64)]),
    "tiler_hip_payload_identity": (_S, [_P]),
    "tiler_hip_payload_correspondence": (_S, [_P, _U64, ctypes.c_char_p, _U64]),
    "tiler_hip_digest": (_S, [_P, _U64, ctypes.POINTER(_P), ctypes.POINTER(_U64), _U32, _P, _U64, _P]),
    "tiler_hip_read_envelope": (_S, [_P, _U64, ctypes.POINTER(Envelope), ctypes.c_char_p, _U64]),
    "tiler_hip_read_payload_metadata": (_S, [_P, _U64, ctypes.POINTER(PayloadSubject),
                                             ctypes.POINTER(PayloadMapping), _U32, ctypes.c_char_p, _U64]),
    "tiler_hip_select_payload": (_S, [ctypes.POINTER(Envelope), ctypes.POINTER(_U32), ctypes.c_char_p, _U64]),
}

_lib = None


class LibraryMissing(RuntimeError):
    pass


def lib():
    """Loads libtiler_hip.so; raises LibraryMissing if it was never built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise LibraryMissing(
                f"{LIB_PATH} is not built; run `python -m tiler_amd.build` (tiler-hip has no "
                "CPU fallback)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(handle, name)
            f.restype = res
            f.argtypes = args
        _lib = handle
    return _lib
