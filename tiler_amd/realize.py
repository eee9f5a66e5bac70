"""The realization recognizer and the RuntimeAdapter route over its result.

`realize` asks the C ABI (`tiler_hip_realize`) which of the library's entry
points realize one scheduled region, and with what launch geometry and
argument segment. The region names:
- the ScalarProgram (tiler-ir/src/schedule/model.rs:661-930);
- the ReductionTopology (model.rs:1327-1555);
- the geometry.

The answer is the same program the family entry point runs for that request.

`route` then executes a realization the way
`route_with_adapter` drives a RuntimeAdapter (tiler-runtime/src/adapter.rs:
545-678):
1. Prepare the payload's entries for the symbols it names (cached per
   context).
2. Plan the dispatch, acquiring nothing.
3. Check the caller's storage against the slot sizes and the alignment the
   realization assumed.
4. Allocate scratch after the commit.
5. Dispatch.
6. Release the scratch.

Every refusal raises before anything is committed. A gather's
out-of-range record raises `GatherIndexOutOfBounds` as a post-commit failure.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

from . import _lib as L
from .runtime import Failure, GatherIndexOutOfBounds, Refusal, _raise


@dataclass
class RealizedDispatch:
    symbol: str
    family: str
    grid: tuple
    block: tuple
    bindings: list  # (slot, byte offset of the pointer field)
    extents: list = field(default_factory=list)  # (live extent id, byte offset of its u32 field)


@dataclass
class Realization:
    program: int
    raw: L.Realization
    slots: list = field(default_factory=list)  # (role, bytes)
    alignment: int = 1
    dispatches: list = field(default_factory=list)
    # (input access, axis, minimum, bound) per live extent: route(extents=...)
    # supplies their values, each in [minimum, bound]
    live_extents: list = field(default_factory=list)

    @property
    def symbols(self) -> list:
        return [d.symbol for d in self.dispatches]


def _entry_info(index: int):
    info = L.EntryInfo()
    _raise(L.lib().tiler_hip_payload_entry(index, ctypes.byref(info)), "payload_entry")
    return info.symbol.decode(), info.family.decode()


def _region(program: int, extents, *, dtype: int = L.F32, topology: int = L.SUM_SERIAL, variant: int = 0,
            flags: int = L.REGION_ALIGNED16, rank: int = 0, strides=(), grouping=(), scalars=(),
            permissions: int = 0, input_subnormals: int = 0, result_subnormals: int = 0,
            nodes=(), root: int | None = None, structure=None, form: int = L.FORM_AUTO):
    """An L.Region and the objects its pointers reference (kept alive with it)."""
    r = L.Region()
    r.program, r.topology, r.dtype, r.variant, r.flags, r.rank = program, topology, dtype, variant, flags, rank
    for i, v in enumerate(extents):
        r.extents[i] = int(v)
    for i, v in enumerate(strides):
        r.strides[i] = int(v) & 0xFFFFFFFFFFFFFFFF
    for i, v in enumerate(grouping):
        r.grouping[i] = int(v) & 0xFFFFFFFFFFFFFFFF
    for i, v in enumerate(scalars):
        r.scalars[i] = int(v)
    r.permissions, r.input_subnormals, r.result_subnormals = permissions, input_subnormals, result_subnormals
    r.form = form
    node_array = (L.ExpressionNode * max(1, len(nodes)))(*[L.ExpressionNode(*nd) for nd in nodes])
    if len(nodes):
        r.node_count = len(nodes)
        r.root = len(nodes) - 1 if root is None else root
        r.nodes = node_array
    if structure is not None:
        r.structure = ctypes.pointer(structure)
    return r, (node_array, structure)


def realize(program: int, extents, *, ctx=None, **kw) -> Realization:
    """Realizes one region.  `ctx` (a runtime.Context) lets the bound device's
    CU count decide tile sizes and groupings; without it the declared
    profile's does (the call is then device-free).

    Keywords (the tiler_hip_region fields): dtype, topology, variant, flags,
    rank, strides, grouping, scalars.  The contract: `permissions`
    (L.PERMITS_*) and the two subnormal modes `input_subnormals` /
    `result_subnormals` (L.SUBNORMALS_*, 0 preserve) are the plan's numerical
    contract for this region; the defaults are the strict contract.  `nodes`
    (op, a, b) and `root` (default: the last node) give an expression's DAG,
    or a fold's epilogue.  `structure` (an L.ContractionStructure, see
    L.contraction_structure) makes a contraction region general.  `form`
    (L.FORM_*) names one form a proposal offered (default: the library's
    choice)."""
    r, keep = _region(program, **dict(kw, extents=extents))
    return _realize_region(r, ctx)


def _realize_region(r, ctx) -> Realization:
    program = r.program
    out = L.Realization()
    diag = ctypes.create_string_buffer(256)
    st = L.lib().tiler_hip_realize(ctx.handle if ctx is not None else None, ctypes.byref(r), ctypes.byref(out),
                                   diag, 256)
    _raise(st, "realize", diag.value.decode())
    res = Realization(program=program, raw=out, alignment=out.slot_alignment,
                      slots=[(out.slot_roles[i], out.slot_bytes[i]) for i in range(out.slot_count)])
    for i in range(out.entry_count):
        e = out.entries[i]
        symbol, family = _entry_info(e.entry)
        res.dispatches.append(RealizedDispatch(
            symbol, family, tuple(e.grid), tuple(e.block),
            [(e.binding_slots[b], e.binding_offsets[b]) for b in range(e.binding_count)],
            [(e.extent_ids[x], e.extent_offsets[x]) for x in range(e.extent_count)]))
    res.live_extents = [(x.access, x.axis, x.minimum, x.bound)
                        for x in out.live_extents[:out.live_extent_count]]
    return res


@dataclass
class Proposal:
    """One implementation tiler_hip_propose offered: its strategy key, the
    launches (kernel, workgroups, threads per workgroup), its structural cost
    (dispatches, launched threads, temporary bytes) and, for the sum, the
    measured row's fold steps."""
    strategy: str
    symbols: list
    workgroups: list
    workgroup_threads: list
    dispatch_count: int
    launched_threads: int
    temporary_bytes: int
    measured_fold_steps: int
    region: L.Region
    _keep: tuple = ()

    def realize(self, ctx=None) -> Realization:
        """The realization of exactly this proposal."""
        return _realize_region(self.region, ctx)


@dataclass
class Declined:
    strategy: str
    cause: int  # L.DECLINE_*
    subject: str  # the numerical dimension key, or the rule
    extent: int


@dataclass
class Offer:
    provider: str
    proposals: list
    declined: list
    chosen: int  # index into proposals

    def strategies(self) -> list:
        return [p.strategy for p in self.proposals]


def propose(program: int, extents, *, ctx=None, **kw) -> Offer:
    """Every implementation the library has for one region
    (PhysicalImplementationProvider::propose, tiler-compiler/src/frontier.rs:1507-1527),
    proposed or declined with its cause.  Keywords as for realize."""
    r, keep = _region(program, **dict(kw, extents=extents))
    offer = L.ProviderOffer()
    diag = ctypes.create_string_buffer(256)
    st = L.lib().tiler_hip_propose(ctx.handle if ctx is not None else None, ctypes.byref(r), ctypes.byref(offer),
                                   diag, 256)
    _raise(st, "propose", diag.value.decode())
    props = []
    for i in range(offer.proposal_count):
        q = offer.proposals[i]
        n = q.dispatch_count
        region = L.Region()
        ctypes.pointer(region)[0] = q.region
        props.append(Proposal(q.strategy.decode(), [q.symbols[j].value.decode() for j in range(n)],
                              list(q.workgroups[:n]), list(q.workgroup_threads[:n]), n, q.launched_threads,
                              q.temporary_bytes, q.measured_fold_steps, region, keep))
    declined = [Declined(d.strategy.decode(), d.cause, d.subject.decode(), d.extent)
                for d in offer.declined[:offer.declined_count]]
    return Offer(offer.provider.decode(), props, declined, offer.chosen)


def _payload_code():
    v = L.PayloadView()
    _raise(L.lib().tiler_hip_payload(ctypes.byref(v)), "payload")
    return ctypes.string_at(v.code, v.code_bytes)


def _prepared(ctx, symbol: str, payload=None) -> int:
    """The prepared-entry index of `symbol`, loaded from the library's own
    code object or, given a carried payload, from that payload's code bytes.
    Cached per context and per code object."""
    code = payload.code if payload is not None else None
    source = payload.digest if payload is not None else b""
    cache = ctx.__dict__.setdefault("_route_prepared", {})
    if (source, symbol) not in cache:
        codes = ctx.__dict__.setdefault("_route_code", {})
        if source not in codes:
            if code is None:
                code = _payload_code()
            codes[source] = ctypes.create_string_buffer(code, len(code))
        buf = codes[source]
        entry = L.RoutedEntry(ctypes.cast(buf, ctypes.c_void_p), len(buf.raw), symbol.encode())
        first = ctypes.c_uint32()
        _raise(L.lib().tiler_hip_prepare_entries(ctx.handle, ctypes.byref(entry), 1, ctypes.byref(first)),
               f"prepare_entries({symbol})", ctx.diagnostic())
        cache[(source, symbol)] = first.value
    return cache[(source, symbol)]


def _address(buf) -> int:
    if buf is None:
        return 0
    return int(buf.ptr) if hasattr(buf, "ptr") else int(buf)


def _capacity(buf):
    return getattr(buf, "nbytes", None)


class RoutedPlan:
    """A realization committed to its storage: planned (plan_dispatch, which
    acquires nothing), its scratch slots allocated (allocate_dispatch), ready
    to run.  `dispatch()` runs it and waits (the adapter's dispatch);
    `enqueue(stream)` only encodes it (tiler_hip_enqueue_dispatch), for a
    caller that captures it into a HIP graph or orders it itself; `release()`
    frees the scratch it allocated.  Built by `prepare_route`."""

    def __init__(self, ctx, rz, plan, ptrs, owned, keep):
        self.ctx, self.rz, self.plan, self.ptrs, self.owned, self._keep = ctx, rz, plan, ptrs, owned, keep

    def dispatch(self):
        h = self.ctx.handle
        _raise(L.lib().tiler_hip_dispatch(h, ctypes.byref(self.plan), self.ptrs), "dispatch", self.ctx.diagnostic())
        self._check_records()

    def enqueue(self, stream=None):
        _raise(L.lib().tiler_hip_enqueue_dispatch(self.ctx.handle, ctypes.byref(self.plan), self.ptrs, stream),
               "enqueue_dispatch", self.ctx.diagnostic())

    def _check_records(self):
        h, rz, ptrs = self.ctx.handle, self.rz, self.ptrs
        if rz.program == L.PROGRAM_GATHER:
            rec = ctypes.c_uint64()
            _raise(L.lib().tiler_hip_download(h, ctypes.byref(rec), ptrs[3], 8), "read gather record")
            if rec.value != 0xFFFFFFFFFFFFFFFF:
                raise GatherIndexOutOfBounds(L.FAIL_GATHER_INDEX_OUT_OF_BOUNDS, rec.value)
        elif rz.program == L.PROGRAM_DEQUANTIZE_U4:
            # the kernel's verdict on the scale and zero point it read
            # (quantization.rs:318-370): the output was not written
            rec = ctypes.c_uint32()
            _raise(L.lib().tiler_hip_download(h, ctypes.byref(rec), ptrs[4], 4), "read domain record")
            if rec.value:
                raise Failure(L.FAIL_VALUE_DOMAIN, "dispatch",
                              "scale outside positive-normal-f32" if rec.value == 1
                              else "zero point outside the U4 code domain 0..=15")

    def release(self):
        if self.plan is not None:
            L.lib().tiler_hip_release_dispatch(self.ctx.handle, ctypes.byref(self.plan), self.ptrs, self.owned)
            self.plan = None


def prepare_route(ctx, realization: Realization, storage, payload=None, extents=()) -> "RoutedPlan | None":
    """The route's steps up to dispatch (see `route`): refusals raise before
    anything is committed.  Returns None for zero work (nothing to dispatch)."""
    rz = realization
    if len(extents) != len(rz.live_extents):
        raise Refusal(L.REFUSE_BINDING_MISMATCH, "route",
                      f"{len(extents)} live extent values for {len(rz.live_extents)} live extents")
    if payload is not None:
        mapped = set(payload.subject.symbols) if payload.subject is not None else set()
        for d in rz.dispatches:
            if d.symbol not in mapped:
                raise Refusal(L.REFUSE_ABSENT_SYMBOL, "route",
                              f"{d.symbol} is not among the carried payload's entry mappings")
    if len(storage) != len(rz.slots):
        raise Refusal(L.REFUSE_BINDING_MISMATCH, "route",
                      f"{len(storage)} storage bindings for {len(rz.slots)} slots")
    if rz.raw.entry_count == 0:
        return None  # zero work: the dispatch is skipped
    for i, ((role, nbytes), buf) in enumerate(zip(rz.slots, storage)):
        if buf is None:
            if role not in (L.SLOT_SCRATCH, L.SLOT_CONSTANT):
                raise Refusal(L.REFUSE_BINDING_MISMATCH, "route", f"slot {i} needs caller storage")
            continue
        cap = _capacity(buf)
        if cap is not None and cap < nbytes:
            raise Refusal(L.REFUSE_BINDING_MISMATCH, "route", f"slot {i} holds {cap} of {nbytes} bytes")
        if _address(buf) % rz.alignment:
            raise Refusal(L.REFUSE_BINDING_MISMATCH, "route",
                          f"slot {i} is not {rz.alignment}-byte aligned as the realization assumed")
    n = rz.raw.entry_count
    entries = (L.DispatchEntry * n)()
    keep = []
    for i in range(n):
        e = rz.raw.entries[i]
        slots = (ctypes.c_uint32 * max(1, e.binding_count))(*e.binding_slots[:e.binding_count])
        offs = (ctypes.c_uint32 * max(1, e.binding_count))(*e.binding_offsets[:e.binding_count])
        kernargs = ctypes.create_string_buffer(bytes(e.kernargs[:e.kernarg_bytes]), max(1, e.kernarg_bytes))
        ids = (ctypes.c_uint32 * max(1, e.extent_count))(*e.extent_ids[:e.extent_count])
        xoffs = (ctypes.c_uint32 * max(1, e.extent_count))(*e.extent_offsets[:e.extent_count])
        keep += [slots, offs, kernargs, ids, xoffs]
        entries[i] = L.DispatchEntry(_prepared(ctx, rz.dispatches[i].symbol, payload), e.grid, e.block, 0,
                                     ctypes.cast(kernargs, ctypes.c_void_p), e.kernarg_bytes,
                                     e.binding_count, slots, offs, e.extent_count, ids, xoffs)
    slot_bytes = (ctypes.c_uint64 * len(rz.slots))(*[b for _, b in rz.slots])
    # The CONSTANT slot's contents (an expression's register program) travel
    # with the plan; dispatch uploads them before the first entry.
    contents = (ctypes.c_void_p * len(rz.slots))()
    if rz.raw.constant_slot < len(rz.slots):
        constant = ctypes.create_string_buffer(bytes(rz.raw.constant[:rz.raw.constant_bytes]),
                                               max(1, rz.raw.constant_bytes))
        keep.append(constant)
        contents[rz.raw.constant_slot] = ctypes.cast(constant, ctypes.c_void_p)
    live = len(rz.live_extents)
    values = (ctypes.c_uint64 * max(1, live))(*[int(v) for v in extents])
    ranges = (L.LiveExtent * max(1, live))(*rz.raw.live_extents[:live])
    keep += [entries, slot_bytes, contents, values, ranges]
    plan = L.DispatchPlan(len(rz.slots), slot_bytes, n, entries, contents, live, values, ranges)
    h = ctx.handle
    _raise(L.lib().tiler_hip_plan_dispatch(h, ctypes.byref(plan)), "plan_dispatch", ctx.diagnostic())
    ptrs = (ctypes.c_void_p * len(rz.slots))(*[_address(b) or None for b in storage])
    owned = (ctypes.c_void_p * len(rz.slots))(*[None if b is None else 1 for b in storage])
    _raise(L.lib().tiler_hip_allocate_dispatch(h, ctypes.byref(plan), ptrs), "allocate_dispatch",
           ctx.diagnostic())
    return RoutedPlan(ctx, rz, plan, ptrs, owned, keep)


def route(ctx, realization: Realization, storage, payload=None, extents=()) -> None:
    """Executes `realization` on `ctx`'s stream and waits for it.  `storage`
    lists one device buffer (or address) per slot, in the realization's slot
    order; scratch slots may be None (allocated here, released after).
    `payload` (from `tiler_amd.envelope.select_payload`) routes through a
    carried code object instead of the library's own: every symbol dispatched
    must be one of its PayloadEntryMappings.  `extents` gives this dispatch's
    value of each live extent (realization.live_extents, in order); the slots
    still hold the bound, and an input whose axis is live is packed at the
    value given."""
    routed = prepare_route(ctx, realization, storage, payload, extents)
    if routed is None:
        return
    try:
        routed.dispatch()
    finally:
        routed.release()
