"""Host-side mirror of the tiler-hip runtime: a bound context, device buffers,
and the realization families as launches on device storage.

`Context` plays the role of a `RuntimeAdapter` implementor's `Self`
(tiler-runtime/src/adapter.rs:260-511): it binds one device and one ordered
stream, owns the loaded gfx950 code object, and reports refusals (pre-commit,
fallback permitted) and failures (post-commit) as distinct exception types,
the split ADR 0051 draws.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _lib as L


class HipError(RuntimeError):
    """A status from the C ABI.  `fallback_permitted` mirrors
    AdapterRouteFailure::fallback_permitted (adapter.rs:738)."""

    def __init__(self, status: int, what: str, diagnostic: str = ""):
        self.status = status
        self.diagnostic = diagnostic
        super().__init__(f"{what}: status {status}" + (f" ({diagnostic})" if diagnostic else ""))

    @property
    def fallback_permitted(self) -> bool:
        return self.status < 0


class Refusal(HipError):
    pass


class Failure(HipError):
    pass


class GatherIndexOutOfBounds(HipError):
    """The gather bound refusal, naming the first offending index position
    (tiler-reference ReferenceOperationError::GatherIndexOutOfBounds)."""

    def __init__(self, status, position, value=None, extent=None, diagnostic=""):
        self.position = position
        self.value = value
        self.extent = extent
        super().__init__(status, f"gather index out of bounds at position {position}", diagnostic)


def _raise(status: int, what: str, diagnostic: str = ""):
    if status == L.OK:
        return
    cls = Refusal if status < 0 else Failure
    raise cls(status, what, diagnostic)


def profile() -> dict:
    """The gfx950 target profile (device-free)."""
    p = L.TargetProfile()
    _raise(L.lib().tiler_hip_profile_declare(ctypes.byref(p)), "profile_declare")
    out = {}
    for name, _ in L.TargetProfile._fields_:
        v = getattr(p, name)
        if isinstance(v, bytes):
            v = v.decode()
        elif hasattr(v, "__len__"):
            v = list(v)
        out[name] = v
    return out


@dataclass
class DeviceBuffer:
    ctx: "Context"
    ptr: int
    nbytes: int

    def free(self):
        if self.ptr:
            self.ctx._check(L.lib().tiler_hip_buffer_free(self.ctx.handle, self.ptr), "buffer_free")
            self.ptr = 0

    def upload(self, host: np.ndarray):
        host = np.ascontiguousarray(host)
        if host.nbytes > self.nbytes:
            raise ValueError("host array larger than the device buffer")
        self.ctx._check(L.lib().tiler_hip_upload(self.ctx.handle, self.ptr,
                                                 host.ctypes.data_as(ctypes.c_void_p), host.nbytes),
                        "upload")

    def download(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        if out.nbytes > self.nbytes:
            raise ValueError("requested more bytes than the buffer holds")
        self.ctx._check(L.lib().tiler_hip_download(self.ctx.handle,
                                                   out.ctypes.data_as(ctypes.c_void_p), self.ptr,
                                                   out.nbytes), "download")
        return out

    def offset(self, nbytes: int) -> "DeviceBuffer":
        """A non-owning view starting `nbytes` in."""
        return DeviceBuffer(self.ctx, self.ptr + nbytes, self.nbytes - nbytes)


def _ptr(buf) -> int | None:
    if buf is None:
        return None
    return buf.ptr if isinstance(buf, DeviceBuffer) else int(buf)


class Context:
    """bind_execution_context + the device half of route_with_adapter."""

    def __init__(self, device: int = 0):
        self.handle = ctypes.c_void_p()
        env = L.ExecutionEnvironment()
        diag = ctypes.create_string_buffer(512)
        st = L.lib().tiler_hip_bind(device, ctypes.byref(self.handle), ctypes.byref(env), diag,
                                    len(diag))
        if st != L.OK:
            raise Refusal(st, "bind", diag.value.decode())
        self.environment = {
            name: (getattr(env, name).decode() if isinstance(getattr(env, name), bytes)
                   else getattr(env, name))
            for name, _ in L.ExecutionEnvironment._fields_
        }

    # -- lifecycle ------------------------------------------------------------
    def close(self):
        if self.handle:
            L.lib().tiler_hip_release(self.handle)
            self.handle = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def diagnostic(self) -> str:
        d = L.lib().tiler_hip_last_diagnostic(self.handle)
        return d.decode() if d else ""

    def _check(self, status: int, what: str):
        if status != L.OK:
            _raise(status, what, self.diagnostic())

    # -- storage and timing ---------------------------------------------------
    def alloc(self, nbytes: int) -> DeviceBuffer:
        p = ctypes.c_void_p()
        self._check(L.lib().tiler_hip_buffer_alloc(self.handle, nbytes, ctypes.byref(p)), "alloc")
        return DeviceBuffer(self, p.value, nbytes)

    def to_device(self, host: np.ndarray) -> DeviceBuffer:
        host = np.ascontiguousarray(host)
        buf = self.alloc(max(host.nbytes, 1))
        buf.upload(host)
        return buf

    def synchronize(self):
        self._check(L.lib().tiler_hip_synchronize(self.handle), "synchronize")

    @property
    def stream(self) -> int:
        return L.lib().tiler_hip_context_stream(self.handle)

    def event(self) -> int:
        e = ctypes.c_void_p()
        self._check(L.lib().tiler_hip_event_create(self.handle, ctypes.byref(e)), "event_create")
        return e.value

    def record(self, event: int, stream=None):
        self._check(L.lib().tiler_hip_event_record(self.handle, event, stream), "event_record")

    def elapsed_ms(self, start: int, stop: int) -> float:
        ms = ctypes.c_float()
        self._check(L.lib().tiler_hip_event_elapsed_ms(self.handle, start, stop, ctypes.byref(ms)),
                    "event_elapsed")
        return ms.value

    def destroy_event(self, event: int):
        L.lib().tiler_hip_event_destroy(self.handle, event)

    # -- graph capture (launch-bound loops) ------------------------------------
    def capture_begin(self, stream=None):
        self._check(L.lib().tiler_hip_capture_begin(self.handle, stream), "capture_begin")

    def capture_end(self, stream=None) -> int:
        g = ctypes.c_void_p()
        self._check(L.lib().tiler_hip_capture_end(self.handle, stream, ctypes.byref(g)), "capture_end")
        return g.value

    def graph_launch(self, graph: int, stream=None):
        self._check(L.lib().tiler_hip_graph_launch(self.handle, graph, stream), "graph_launch")

    def graph_destroy(self, graph: int):
        self._check(L.lib().tiler_hip_graph_destroy(self.handle, graph), "graph_destroy")

    def copy(self, dst, src, nbytes: int, stream=None):
        """Device-to-device copy, ordered on the stream."""
        self._check(L.lib().tiler_hip_copy(self.handle, _ptr(dst), _ptr(src), nbytes, stream), "copy")

    def fill_u32(self, buf, value: int, words: int, stream=None):
        self._check(L.lib().tiler_hip_fill_u32(self.handle, _ptr(buf), value, words, stream),
                    "fill_u32")

    # -- live-device and prepared-entry observations --------------------------
    def observe_live_device(self, key: str) -> int | None:
        """None answers an unrecognized key (LiveDeviceObservation::Unrecognized)."""
        v = ctypes.c_uint64()
        st = L.lib().tiler_hip_observe_live_device(self.handle, key.encode(), ctypes.byref(v))
        if st == L.REFUSE_UNRECOGNIZED_KEY:
            return None
        self._check(st, "observe_live_device")
        return v.value

    # -- realization families (device storage, asynchronous) ------------------
    def sum_f32(self, x, rows: int, extent: int, out, topology: int = L.SUM_SERIAL,
                partitions: int = 0, participants: int = 0, per_partition: int = 0,
                rounds: int = 0, participant_major: bool = False, stream=None):
        plan = L.SumPlan(topology, 1 if participant_major else 0, partitions, participants,
                         per_partition, rounds)
        self._check(L.lib().tiler_hip_sum_f32(self.handle, _ptr(x), rows, extent, _ptr(out),
                                              ctypes.byref(plan), stream), "sum_f32")

    def sum_tree_workgroups(self, n: int) -> int:
        return L.lib().tiler_hip_sum_tree_workgroups(self.handle, n)

    def rms_norm(self, dtype: int, x, w, rows: int, extent: int, eps_bits: int, y,
                 weight_broadcast: bool = True, stream=None):
        self._check(L.lib().tiler_hip_rms_norm(self.handle, dtype, _ptr(x), _ptr(w),
                                               1 if weight_broadcast else 0, rows, extent,
                                               eps_bits, _ptr(y), stream), "rms_norm")

    def softmax_f32(self, x, rows: int, extent: int, y, stream=None):
        self._check(L.lib().tiler_hip_softmax_f32(self.handle, _ptr(x), rows, extent, _ptr(y),
                                                  stream), "softmax_f32")

    def map(self, op: int, dtype: int, x, n: int, y, x2=None, x2_broadcast: bool = False,
            a: float = 0.0, b: float = 0.0, stream=None):
        self._check(L.lib().tiler_hip_map(self.handle, op, dtype, _ptr(x), _ptr(x2),
                                          1 if x2_broadcast else 0, n, a, b, _ptr(y), stream),
                    "map")

    def broadcast(self, src, src_elements: int, out_dims, src_strides, element_bytes: int, out,
                  stream=None):
        rank = len(out_dims)
        dims = (ctypes.c_uint64 * max(rank, 1))(*out_dims)
        strides = (ctypes.c_uint64 * max(rank, 1))(*src_strides)
        self._check(L.lib().tiler_hip_broadcast(self.handle, _ptr(src), src_elements, rank, dims,
                                                strides, element_bytes, _ptr(out), stream),
                    "broadcast")

    def convert(self, direction: int, src, n: int, dst, stream=None):
        """bf16 <-> binary32 conversion (L.CONVERT_NARROW_F32_BF16 / L.CONVERT_WIDEN_BF16_F32)."""
        self._check(L.lib().tiler_hip_convert(self.handle, direction, _ptr(src), n, _ptr(dst), stream),
                    "convert")

    def dequantize_u4(self, codes, n: int, scale_bits: int, zero_point: int, y, stream=None):
        """Strict-affine U4 -> f32 (quantization.rs:218-246): n codes packed
        LSB-first in (n + 1) // 2 carriers; refuses a scale outside
        positive-normal-f32 or a zero point above 15 before commit."""
        self._check(L.lib().tiler_hip_dequantize_u4(self.handle, _ptr(codes), n, scale_bits & 0xFFFFFFFF,
                                                     zero_point, _ptr(y), stream), "dequantize_u4")

    def gather(self, source, outer: int, gathered: int, inner: int, element_bytes: int, index,
               index_count: int, out, index_signed: bool = False, stream=None):
        self._check(L.lib().tiler_hip_gather(self.handle, _ptr(source), outer, gathered, inner,
                                             element_bytes, _ptr(index), index_count,
                                             1 if index_signed else 0, _ptr(out), stream),
                    "gather")

    def gather_status(self, stream=None):
        """Raises GatherIndexOutOfBounds (a post-commit failure) if any gather
        since the last call met an out-of-range index."""
        pos = ctypes.c_uint64()
        st = L.lib().tiler_hip_gather_status(self.handle, stream, ctypes.byref(pos))
        if st == L.FAIL_GATHER_INDEX_OUT_OF_BOUNDS:
            raise GatherIndexOutOfBounds(st, pos.value, diagnostic=self.diagnostic())
        self._check(st, "gather_status")

    def contract_strict_f32(self, a, b, m: int, n: int, k: int, c, stream=None):
        self._check(L.lib().tiler_hip_contract_strict_f32(self.handle, _ptr(a), _ptr(b), m, n, k,
                                                          _ptr(c), stream), "contract_strict_f32")

    def contract_bf16(self, a, b, m: int, n: int, k: int, c, epilogue: int = L.EPILOGUE_NONE,
                      stream=None):
        self._check(L.lib().tiler_hip_contract_bf16(self.handle, _ptr(a), _ptr(b), m, n, k,
                                                    _ptr(c), epilogue, stream), "contract_bf16")

    def contract(self, dtype: int, structure, left, right, out, epilogue: int = L.EPILOGUE_NONE,
                 permissions: int = 0, stream=None):
        """A contraction over an index structure (L.contraction_structure):
        the strict fold unless `permissions` grants reassociation (bf16)."""
        self._check(L.lib().tiler_hip_contract(self.handle, dtype, ctypes.byref(structure), epilogue, permissions,
                                               _ptr(left), _ptr(right), _ptr(out), stream), "contract")

    def expression(self, dtype: int, nodes, inputs, n: int, y, root: int | None = None,
                   input_subnormals: int = 0, result_subnormals: int = 0, stream=None):
        """A pointwise expression DAG: `nodes` are (op, a, b) triples (L.NODE_*),
        `inputs` one device buffer per access ordinal."""
        arr = (L.ExpressionNode * max(1, len(nodes)))(*[L.ExpressionNode(*nd) for nd in nodes])
        ptrs = (ctypes.c_void_p * max(1, len(inputs)))(*[_ptr(b) for b in inputs])
        self._check(L.lib().tiler_hip_expression(self.handle, dtype, arr, len(nodes),
                                                 len(nodes) - 1 if root is None else root, ptrs, n, _ptr(y),
                                                 input_subnormals, result_subnormals, stream), "expression")

    def fold_f32(self, variant: int, x, dims, reduced_axes, out, scale_bits: int = 0, bias_bits: int = 0,
                 stream=None):
        """Serial fold (L.FOLD_*) of a dense f32 tensor over `reduced_axes`."""
        rank = len(dims)
        d = (ctypes.c_uint64 * max(rank, 1))(*dims)
        mask = sum(1 << a for a in reduced_axes)
        self._check(L.lib().tiler_hip_fold_f32(self.handle, variant, _ptr(x), rank, d, mask, scale_bits,
                                               bias_bits, _ptr(out), stream), "fold_f32")

    def reindex(self, src, src_elements: int, out_dims, strides, base: int, element_bytes: int, out,
                stream=None):
        rank = len(out_dims)
        d = (ctypes.c_uint64 * max(rank, 1))(*out_dims)
        s = (ctypes.c_int64 * max(rank, 1))(*strides)
        self._check(L.lib().tiler_hip_reindex(self.handle, _ptr(src), src_elements, rank, d, s, base,
                                              element_bytes, _ptr(out), stream), "reindex")

    # -- target environment (adapter.rs:295-322) ------------------------------
    def observe_target_environment(self):
        """(descriptor bytes, None) when observed, (None, reason) when
        Unavailable (which filters claimed cells, never fails the route)."""
        buf = ctypes.create_string_buffer(256)
        need, observed = ctypes.c_uint64(), ctypes.c_uint32()
        reason = ctypes.create_string_buffer(256)
        self._check(L.lib().tiler_hip_observe_target_environment(self.handle, buf, 256, ctypes.byref(need),
                                                                 ctypes.byref(observed), reason, 256),
                    "observe_target_environment")
        if not observed.value:
            return None, reason.value.decode()
        return buf.raw[:need.value], None


def target_environment_support() -> dict:
    """The one target-environment descriptor schema tiler-hip registers."""
    s = L.TargetEnvironmentSchema()
    _raise(L.lib().tiler_hip_target_environment_support(ctypes.byref(s)), "target_environment_support")
    return {"provider": s.provider.decode(), "revision": s.provider_revision,
            "schema": (s.schema_major, s.schema_minor)}


def validate_target_environment(descriptor: bytes) -> str | None:
    """None when `descriptor` is the schema's canonical spelling, else the reason."""
    diag = ctypes.create_string_buffer(256)
    st = L.lib().tiler_hip_validate_target_environment(descriptor, len(descriptor), diag, 256)
    if st == L.OK:
        return None
    if st != L.REFUSE_INVALID_ARGUMENT:
        _raise(st, "validate_target_environment")
    return diag.value.decode()


def row_grouping(family: int, dtype: int, extent: int) -> tuple[int, int, int]:
    """The declared (vec, waves, segment) grouping the row kernels use for
    `extent` (segment 0: the row folds whole)."""
    vec, waves, segment = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint64()
    _raise(L.lib().tiler_hip_row_grouping(family, dtype, extent, ctypes.byref(vec), ctypes.byref(waves),
                                          ctypes.byref(segment)), "row_grouping")
    return vec.value, waves.value, segment.value


def validate_gather_index(index: np.ndarray, gathered: int, index_signed: bool):
    """Pre-commit bound check (a Refusal naming the first offending position)."""
    idx = np.ascontiguousarray(index, dtype=np.uint32) if index.dtype != np.uint32 else \
        np.ascontiguousarray(index)
    pos = ctypes.c_uint64()
    val = ctypes.c_int64()
    st = L.lib().tiler_hip_validate_gather_index(idx.ctypes.data_as(ctypes.c_void_p), idx.size,
                                                 1 if index_signed else 0, gathered,
                                                 ctypes.byref(pos), ctypes.byref(val))
    if st == L.REFUSE_GATHER_INDEX_OUT_OF_BOUNDS:
        raise GatherIndexOutOfBounds(st, pos.value, val.value, gathered)
    _raise(st, "validate_gather_index")
