"""Python host binding of libloom_infer_hip.so: Loom Infer's paged-KV decode path
on MI355X (gfx950).

The names and call sequence mirror the reference's Rust API so that callers and
tests read the same way:

    spec = Bf16PagedBatchDecodeSpec(batch, pool, hq, hkv, 128, 16)
    plan = DecodeProvider.load(0).plan_bf16_paged_batch(spec)
    queue = CommandQueue(torch.cuda.current_stream(), 1)
    b = queue.bindings(9); q = b.bind_read(query); ... o = b.bind_read_write(out)
    scope = queue.begin(b)
    plan.enqueue_into(scope, Bf16PagedBatchDecodeArgs(q, k, v, ip, ix, ln,
                                                      o.write(), lse.write(), ws.write()))
    b = scope.finish().wait(); out = b.take_read_write(o)

(crates/loom-infer-cuda/src/attention/decode.rs:1067-1296,
crates/loom-infer-cuda/src/rope/mod.rs:628-934,
crates/loom-infer-cuda/src/command/*.rs, crates/loom-infer-cuda/src/graph/mod.rs).

Device buffers are torch tensors used only as HIP allocations; every compute
call goes through the C ABI and there is no CPU fallback: when the library is
missing, importing the provider fails loudly.
"""
from __future__ import annotations

import ctypes as C
import threading
from dataclasses import dataclass
from typing import Any, Callable, Optional, Sequence

from . import _ffi

HEAD_DIM = 128
PAGE_SIZE = 16
PARTIAL_STATE_WIDTH = 130
PLAN_PAGE_INDICES_CAPACITY = 1
PLAN_PREFILL_TILE_16 = 2
PLAN_PREFILL_TILE_64 = 4
PLAN_PREFILL_TILE_LONG = 8
GRAPH_REPLAY_MODES = {1: "hip_graph_launch", 2: "kernel_nodes"}
PLAN_APPEND_TWO_LAUNCH = 8
PLAN_APPEND_TEST_NO_WAIT = 16


def _prefill_tile_flag(tile_cols) -> int:
    """0 (chosen from the spec), 16 (row tiles), 64 (wide tiles) or "long"
    (long tiles, paged prefill on BF16 pages)."""
    if tile_cols not in (0, 16, 64, "long"):
        raise ValueError(f"tile_cols must be 0, 16, 64 or 'long', got {tile_cols}")
    return {0: 0, 16: PLAN_PREFILL_TILE_16, 64: PLAN_PREFILL_TILE_64,
            "long": PLAN_PREFILL_TILE_LONG}[tile_cols]
# K/V page layouts (loom_kv_layout_t): NHD pages [16, Hkv, 128], HND pages
# [Hkv, 16, 128].  The reference supports NHD only.
KV_LAYOUTS = {"NHD": 0, "HND": 1}


def _layout_code(kv_layout) -> int:
    if kv_layout in KV_LAYOUTS.values():
        return int(kv_layout)
    if kv_layout not in KV_LAYOUTS:
        raise ValueError(f"kv_layout must be one of {sorted(KV_LAYOUTS)}, got {kv_layout!r}")
    return KV_LAYOUTS[kv_layout]


# K/V page element types (loom_kv_dtype_t): BF16, or OCP FP8 E4M3 bytes with
# per-tensor [k_scale, v_scale] (no reference counterpart).
KV_DTYPES = {"bf16": 0, "fp8_e4m3": 1}


def _set_paged_layout(c_paged, kv_layout, kv_dtype="bf16", kv_page_size=None):
    """Applies loom_paged_decode_spec_with_kv_{layout,dtype} and, when
    kv_page_size is given, loom_paged_decode_spec_with_page_size (16, 32 or 64
    rows per page; no reference counterpart) to an embedded paged spec."""
    if kv_page_size is not None:
        out = _ffi.PagedDecodeSpec()
        _call(lib().loom_paged_decode_spec_with_page_size, C.byref(c_paged), int(kv_page_size),
              C.byref(out))
        c_paged.page_size = out.page_size
    code = _layout_code(kv_layout)
    if code != 0:
        out = _ffi.PagedDecodeSpec()
        _call(lib().loom_paged_decode_spec_with_kv_layout, C.byref(c_paged), code, C.byref(out))
        c_paged.kv_layout = out.kv_layout
    if kv_dtype not in KV_DTYPES:
        raise ValueError(f"kv_dtype must be one of {sorted(KV_DTYPES)}, got {kv_dtype!r}")
    if KV_DTYPES[kv_dtype] != 0:
        out = _ffi.PagedDecodeSpec()
        _call(lib().loom_paged_decode_spec_with_kv_dtype, C.byref(c_paged), KV_DTYPES[kv_dtype],
              C.byref(out))
        c_paged.kv_dtype = out.kv_dtype
ROPE_PAGED_KV_APPEND_MAX_TOKENS = 64
ROPE_PAGED_KV_APPEND_MAX_TOKENS_EXTENDED = 8192

DTYPE_F32, DTYPE_F16, DTYPE_BF16, DTYPE_I32, DTYPE_U8 = range(5)

CONTRACT_VARIANTS = [
    None, "ZeroDimension", "ElementCountOverflow", "InvalidEpsilon", "UnsupportedHeadDimension",
    "UnsupportedPageSize", "InvalidHeadMapping", "InvalidPartitionCount", "InvalidIndptrStart",
    "NonMonotonicIndptr", "EmptyRaggedRequest", "RaggedQueryLongerThanKv",
    "InvalidPageIndptrStart", "NonMonotonicPageIndptr", "EmptyPagedRequest",
    "PageIndexOutOfRange", "InvalidLastPageLength", "InvalidRotaryDimension",
    "InvalidRopeScale", "InvalidRopeTheta", "NegativePositionId",
    "UnsupportedAppendTokenCount", "AppendBatchIndexOutOfRange", "AppendPositionOutOfRange",
    "DuplicatePageAppendSlot", "DuplicatePageAppendTokenSlot", "UnsupportedDType",
    "LengthMismatch",
]
COMMAND_VARIANTS = {
    40: "ZeroCommandCapacity", 41: "ZeroBindingCapacity", 42: "IdentifierSpaceExhausted",
    43: "BindingsQueueMismatch", 44: "QueuePoisoned", 45: "ScopePoisoned",
    46: "BindingCapacityExceeded", 47: "BufferContextMismatch", 48: "BindingSetMismatch",
    49: "BindingSlotOutOfRange", 50: "BindingIsReadOnly", 51: "BindingSlotVacant",
    52: "BindingTypeMismatch", 53: "DuplicateBindingSlot", 54: "CommandCapacityExceeded",
    55: "External", 56: "Driver", 57: "AliasedBinding", 58: "BindingsInUse", 59: "NullArgument",
    60: "ScopeActive", 61: "DeviceStatus",
}
PLAN_VARIANTS = {70: "StateCountOutOfRange", 71: "StateCountOverflow",
                 72: "UnsupportedHeadDimension", 73: "UnsupportedRotaryDimension",
                 74: "UnsupportedDevice", 75: "InvalidOption"}
ENQUEUE_VARIANTS = {90: "LengthMismatch", 91: "PageIndicesTooShort", 92: "MisalignedBuffer",
                    93: "PageIndicesTooLong", 94: "StaticScratchTooSmall",
                    95: "WorkspaceNotReserved", 96: "StaticScratchBusy"}
GRAPH_VARIANTS = {110: "DefaultStreamUnsupported", 111: "EmptyCapture",
                  112: "CaptureInvalidated", 113: "NullExecutableHandle",
                  114: "ExecutionPoisoned", 115: "ReplayInFlight", 116: "LaunchCountExhausted",
                  117: "TimingEventContextMismatch", 118: "Driver", 119: "Settlement"}


class LoomError(Exception):
    """Base of every error returned across the C ABI."""

    def __init__(self, code: int, variant: str, message: str, operand: Optional[str],
                 fields: tuple, value: float, hip_status: int):
        super().__init__(message)
        self.code = code
        self.variant = variant
        self.operand = operand
        self.fields = fields
        self.value = value
        self.hip_status = hip_status


class ContractError(LoomError):
    pass


class CommandError(LoomError):
    pass


class PlanError(LoomError):
    pass


class EnqueueError(LoomError):
    pass


class GraphError(LoomError):
    pass


def lib():
    return _ffi.load()


def _raise(rc: int, err: _ffi.Error):
    if rc == 0:
        return
    operand = err.operand.decode() if err.operand else None
    msg = err.message.decode(errors="replace")
    args = (rc, None, msg, operand, tuple(err.fields), err.value, err.hip_status)
    if 1 <= rc < len(CONTRACT_VARIANTS):
        cls, name = ContractError, CONTRACT_VARIANTS[rc]
    elif rc in COMMAND_VARIANTS:
        cls, name = CommandError, COMMAND_VARIANTS[rc]
    elif rc in PLAN_VARIANTS:
        cls, name = PlanError, PLAN_VARIANTS[rc]
    elif rc in ENQUEUE_VARIANTS:
        cls, name = EnqueueError, ENQUEUE_VARIANTS[rc]
    elif rc in GRAPH_VARIANTS:
        cls, name = GraphError, GRAPH_VARIANTS[rc]
    else:
        cls, name = LoomError, f"Status{rc}"
    raise cls(args[0], name, *args[2:])


def _call(fn, *args):
    err = _ffi.Error()
    rc = fn(*args, C.byref(err))
    _raise(rc, err)


_tls = threading.local()


def _enqueue(fn, plan_p, scope_p, args_ref):
    """The hot enqueue call: one preallocated error record per thread and the
    args struct built once per Args value."""
    err = getattr(_tls, "err", None)
    if err is None:
        err = _tls.err = _ffi.Error()
        _tls.err_ref = C.byref(err)
    rc = fn(plan_p, scope_p, args_ref, _tls.err_ref)
    if rc:
        _raise(rc, err)


def _i32_array(values) -> tuple:
    vals = [int(x) for x in values]
    arr = (C.c_int32 * max(1, len(vals)))(*vals)
    return arr, len(vals)


# ---- contracts --------------------------------------------------------------
class PagedBatchDecodePageTable:
    """Validated metadata view (paged_decode/mod.rs:216-279)."""

    def __init__(self, spec: "Bf16PagedBatchDecodeSpec", indptr, indices, last):
        self.spec = spec
        self.page_indptr = list(indptr)
        self.page_indices = list(indices)
        self.last_page_len = list(last)

    def request_page_range(self, request: int):
        if request >= self.spec.batch_size:
            return None
        return self.page_indptr[request], self.page_indptr[request + 1]

    def request_kv_len(self, request: int):
        ip, _ = _i32_array(self.page_indptr)
        ln, _ = _i32_array(self.last_page_len)
        out = C.c_uint64()
        rc = lib().loom_paged_decode_request_kv_len(C.byref(self.spec._c), ip, ln, request,
                                                    C.byref(out))
        return None if rc else out.value

    def physical_page_for_token(self, request: int, token: int):
        ip, _ = _i32_array(self.page_indptr)
        ix, _ = _i32_array(self.page_indices)
        ln, _ = _i32_array(self.last_page_len)
        page, off = C.c_uint64(), C.c_uint64()
        rc = lib().loom_paged_decode_physical_page_for_token(
            C.byref(self.spec._c), ip, ix, ln, request, token, C.byref(page), C.byref(off))
        return None if rc else (page.value, off.value)


class Bf16PagedBatchDecodeSpec:
    """paged_decode/mod.rs:17-149."""

    def __init__(self, batch_size, max_num_pages, num_query_heads, num_kv_heads,
                 head_dim=HEAD_DIM, page_size=PAGE_SIZE, kv_layout="NHD", kv_dtype="bf16",
                 kv_page_size=None):
        self._c = _ffi.PagedDecodeSpec()
        _call(lib().loom_paged_decode_spec_new, batch_size, max_num_pages, num_query_heads,
              num_kv_heads, head_dim, page_size, C.byref(self._c))
        _set_paged_layout(self._c, kv_layout, kv_dtype, kv_page_size)

    kv_layout = property(lambda s: {v: k for k, v in KV_LAYOUTS.items()}[s._c.kv_layout])
    kv_dtype = property(lambda s: {v: k for k, v in KV_DTYPES.items()}[s._c.kv_dtype])

    batch_size = property(lambda s: s._c.batch_size)
    max_num_pages = property(lambda s: s._c.max_num_pages)
    num_query_heads = property(lambda s: s._c.num_query_heads)
    num_kv_heads = property(lambda s: s._c.num_kv_heads)
    softmax_scale = property(lambda s: s._c.softmax_scale)
    head_dim = property(lambda s: HEAD_DIM)
    page_size = property(lambda s: s._c.page_size or PAGE_SIZE)
    gqa_group_size = property(lambda s: s.num_query_heads // s.num_kv_heads)
    query_numel = property(lambda s: s.batch_size * s.num_query_heads * HEAD_DIM)
    kv_pages_numel = property(lambda s: s.max_num_pages * s.page_size * s.num_kv_heads * HEAD_DIM)
    output_numel = property(lambda s: s.query_numel)
    lse_numel = property(lambda s: s.batch_size * s.num_query_heads)
    page_indptr_numel = property(lambda s: s.batch_size + 1)
    last_page_len_numel = property(lambda s: s.batch_size)

    def kv_head_for_query_head(self, query_head: int):
        return query_head // self.gqa_group_size if query_head < self.num_query_heads else None

    def validate_page_table(self, indptr, indices, last) -> PagedBatchDecodePageTable:
        ip, nip = _i32_array(indptr)
        ix, nix = _i32_array(indices)
        ln, nln = _i32_array(last)
        _call(lib().loom_paged_decode_validate_page_table, C.byref(self._c), ip, nip, ix, nix,
              ln, nln)
        return PagedBatchDecodePageTable(self, indptr, indices, last)


class Bf16RopePagedKvAppendSpec:
    """paged_append/mod.rs:14-131 (one token per request at kv_len-1)."""

    def __init__(self, batch_size, max_num_pages, num_query_heads, num_kv_heads,
                 head_dim=HEAD_DIM, page_size=PAGE_SIZE, kv_layout="NHD", kv_dtype="bf16",
                 kv_page_size=None):
        self._c = _ffi.RopeAppendSpec()
        _call(lib().loom_rope_append_spec_new, batch_size, max_num_pages, num_query_heads,
              num_kv_heads, head_dim, page_size, C.byref(self._c))
        _set_paged_layout(self._c.paged, kv_layout, kv_dtype, kv_page_size)
        self.paged = _wrap_paged(self._c.paged)

    batch_size = property(lambda s: s._c.paged.batch_size)
    tokens = property(lambda s: s._c.paged.batch_size)
    max_num_pages = property(lambda s: s._c.paged.max_num_pages)
    num_query_heads = property(lambda s: s._c.paged.num_query_heads)
    num_kv_heads = property(lambda s: s._c.paged.num_kv_heads)
    query_numel = property(lambda s: s.batch_size * s.num_query_heads * HEAD_DIM)
    key_numel = property(lambda s: s.batch_size * s.num_kv_heads * HEAD_DIM)
    value_numel = key_numel
    query_output_numel = query_numel
    kv_pages_numel = property(lambda s: s.paged.kv_pages_numel)

    def validate_page_table(self, indptr, indices, last) -> PagedBatchDecodePageTable:
        ip, nip = _i32_array(indptr)
        ix, nix = _i32_array(indices)
        ln, nln = _i32_array(last)
        _call(lib().loom_rope_append_validate_page_table, C.byref(self._c), ip, nip, ix, nix,
              ln, nln)
        return PagedBatchDecodePageTable(self.paged, indptr, indices, last)


class Bf16RopePagedKvAppendTokensSpec:
    """paged_append/mod.rs:134-317 (explicit tokens; T <= 64, or the extended bound)."""

    def __init__(self, tokens, batch_size, max_num_pages, num_query_heads, num_kv_heads,
                 head_dim=HEAD_DIM, page_size=PAGE_SIZE, extended: bool = False,
                 kv_layout="NHD", kv_dtype="bf16", kv_page_size=None):
        self._c = _ffi.RopeAppendTokensSpec()
        fn = (lib().loom_rope_append_tokens_spec_new_extended if extended
              else lib().loom_rope_append_tokens_spec_new)
        _call(fn, tokens, batch_size, max_num_pages, num_query_heads, num_kv_heads, head_dim,
              page_size, C.byref(self._c))
        _set_paged_layout(self._c.paged, kv_layout, kv_dtype, kv_page_size)
        self.paged = _wrap_paged(self._c.paged)

    @classmethod
    def extended(cls, *args, **kw):
        return cls(*args, extended=True, **kw)

    tokens = property(lambda s: s._c.tokens)
    batch_size = property(lambda s: s._c.paged.batch_size)
    max_num_pages = property(lambda s: s._c.paged.max_num_pages)
    num_query_heads = property(lambda s: s._c.paged.num_query_heads)
    num_kv_heads = property(lambda s: s._c.paged.num_kv_heads)
    query_numel = property(lambda s: s.tokens * s.num_query_heads * HEAD_DIM)
    key_numel = property(lambda s: s.tokens * s.num_kv_heads * HEAD_DIM)
    value_numel = key_numel
    query_output_numel = query_numel
    kv_pages_numel = property(lambda s: s.paged.kv_pages_numel)

    def validate_metadata(self, batch_indices, positions, indptr, indices, last):
        bi, nbi = _i32_array(batch_indices)
        ps, nps = _i32_array(positions)
        ip, nip = _i32_array(indptr)
        ix, nix = _i32_array(indices)
        ln, nln = _i32_array(last)
        slots = (C.c_uint64 * (2 * max(1, self.tokens)))()
        _call(lib().loom_rope_append_tokens_validate_metadata, C.byref(self._c), bi, nbi, ps,
              nps, ip, nip, ix, nix, ln, nln, slots)
        return [(slots[2 * t], slots[2 * t + 1]) for t in range(self.tokens)]


def _wrap_paged(c_spec) -> Bf16PagedBatchDecodeSpec:
    s = Bf16PagedBatchDecodeSpec.__new__(Bf16PagedBatchDecodeSpec)
    s._c = c_spec
    return s


# ---- command runtime ----------------------------------------------------------
def _torch_dtype_code(t) -> int:
    import torch
    table = {torch.float32: DTYPE_F32, torch.float16: DTYPE_F16, torch.bfloat16: DTYPE_BF16,
             torch.int32: DTYPE_I32, torch.uint8: DTYPE_U8}
    if t.dtype not in table:
        raise ContractError(26, "UnsupportedDType", f"unsupported dtype {t.dtype}", None,
                            (0, 0, 0, 0), 0.0, 0)
    return table[t.dtype]


@dataclass(frozen=True)
class Read:
    handle: _ffi.Handle


@dataclass(frozen=True)
class Write:
    handle: _ffi.Handle


@dataclass(frozen=True)
class ReadWrite:
    handle: _ffi.Handle

    def read(self) -> Read:
        return Read(self.handle)

    def write(self) -> Write:
        return Write(self.handle)


_NONE = _ffi.Handle(0, 0)


def _h(x) -> _ffi.Handle:
    return _NONE if x is None else x.handle


class CheckedBindings:
    """binding.rs:16-107.  Keeps Python references to bound tensors (the
    reference's Arc retention) so allocations outlive in-flight commands."""

    def __init__(self, ptr):
        self._p = ptr
        self._owned = {}
        # True while a scope, completion or graph owns the C binding set; the
        # owner frees it (or hands it back), never this object.
        self._moved = False

    def __len__(self):
        return lib().loom_bindings_len(self._p)

    @property
    def capacity(self):
        return lib().loom_bindings_capacity(self._p)

    def _bind(self, fn, tensor, dtype, numel):
        if tensor is None or isinstance(tensor, int):
            ptr = tensor or 0
        else:
            if not tensor.is_contiguous():
                raise ValueError("bindings require contiguous tensors")
            ptr = tensor.data_ptr()
            dtype = _torch_dtype_code(tensor) if dtype is None else dtype
            numel = tensor.numel() if numel is None else numel
        h = _ffi.Handle()
        _call(fn, self._p, C.c_void_p(ptr), numel, dtype, C.byref(h))
        self._owned[h.slot] = tensor
        return h

    def bind_read(self, tensor, dtype=None, numel=None) -> Read:
        return Read(self._bind(lib().loom_bindings_bind_read, tensor, dtype, numel))

    def bind_read_write(self, tensor, dtype=None, numel=None) -> ReadWrite:
        return ReadWrite(self._bind(lib().loom_bindings_bind_read_write, tensor, dtype, numel))

    def take_read_write(self, handle: ReadWrite):
        ptr, n = C.c_void_p(), C.c_uint64()
        _call(lib().loom_bindings_take_read_write, self._p, handle.handle, C.byref(ptr),
              C.byref(n))
        return self._owned.pop(handle.handle.slot, None)

    def __del__(self):
        try:
            if getattr(self, "_p", None) and not self._moved:
                lib().loom_bindings_free(self._p)
                self._p = None
        except Exception:  # interpreter shutdown: module globals are gone
            pass


def _stream_handle(stream) -> int:
    if stream is None:
        raise ValueError("a HIP stream is required")
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


class CommandCompletion:
    """completion.rs:8-144.  Holds the queue (the reference's &mut borrow) and
    the moved bindings until it is settled."""

    def __init__(self, ptr, bindings: CheckedBindings, queue: "CommandQueue"):
        self._p = ptr
        self._bindings = bindings
        self._queue = queue

    def submitted(self) -> int:
        return lib().loom_command_completion_submitted(self._p)

    def is_complete(self) -> bool:
        out = C.c_int()
        _call(lib().loom_command_completion_is_complete, self._p, C.byref(out))
        return bool(out.value)

    def wait(self) -> CheckedBindings:
        p, self._p = self._p, None
        out = C.c_void_p()
        b = self._bindings
        self._queue._live = False
        try:
            _call(lib().loom_command_completion_wait, p, C.byref(out))
        except LoomError:
            b._p = None  # the library dropped them (completion.rs:74-81)
            raise
        b._moved = False
        return b

    def __del__(self):
        try:
            if getattr(self, "_p", None):
                lib().loom_command_completion_free(self._p)
                self._bindings._p = None
                self._queue._live = False
                self._p = None
        except Exception:  # interpreter shutdown: module globals are gone
            pass


class CommandScope:
    """submission.rs:121-316."""

    def __init__(self, ptr, bindings: CheckedBindings, queue=None, capturing=False):
        self._p = ptr
        self._bindings = bindings
        self._queue = queue
        self._capturing = capturing

    @property
    def submitted(self) -> int:
        return lib().loom_command_scope_submitted(self._p)

    def finish(self) -> CommandCompletion:
        out = C.c_void_p()
        p, self._p = self._p, None
        _call(lib().loom_command_scope_finish, p, C.byref(out))
        return CommandCompletion(out.value, self._bindings, self._queue)

    def __del__(self):
        try:
            if getattr(self, "_p", None) and not self._capturing:
                lib().loom_command_scope_free(self._p)
                self._bindings._p = None
                self._queue._live = False
                self._p = None
        except Exception:  # interpreter shutdown: module globals are gone
            pass


class CommandQueue:
    """submission.rs:14-119: one caller-owned HIP stream, one completion event."""

    def __init__(self, stream, max_commands: int):
        self._stream = stream
        self._live = False
        out = C.c_void_p()
        _call(lib().loom_command_queue_new, C.c_void_p(_stream_handle(stream)), max_commands,
              C.byref(out))
        self._p = out.value

    @property
    def max_commands(self):
        return lib().loom_command_queue_max_commands(self._p)

    @property
    def poisoned(self):
        return bool(lib().loom_command_queue_is_poisoned(self._p))

    def stream(self):
        return self._stream

    def reserve_workspace(self, scratch_bytes: int = 0, zeroed_bytes: int = 0):
        """Allocates the queue-owned workspaces that the reference-shaped
        enqueues use, so those enqueues allocate nothing (no reference
        counterpart: the reference's plans need no workspace)."""
        _call(lib().loom_command_queue_reserve_workspace, self._p, scratch_bytes, zeroed_bytes)

    @property
    def workspace_bytes(self) -> int:
        return lib().loom_command_queue_workspace_bytes(self._p)

    def bindings(self, capacity: int) -> CheckedBindings:
        out = C.c_void_p()
        _call(lib().loom_command_queue_bindings, self._p, capacity, C.byref(out))
        return CheckedBindings(out.value)

    def begin(self, bindings: CheckedBindings) -> CommandScope:
        out = C.c_void_p()
        _call(lib().loom_command_queue_begin, self._p, bindings._p, C.byref(out))
        bindings._moved = True
        self._live = True
        return CommandScope(out.value, bindings, self)

    def __del__(self):
        try:
            # A queue still borrowed by an unsettled scope/completion (only possible
            # when a reference cycle is collected) is left allocated rather than
            # freed under its borrower.
            if getattr(self, "_p", None) and not self._live:
                lib().loom_command_queue_free(self._p)
                self._p = None
        except Exception:  # interpreter shutdown: module globals are gone
            pass


# ---- paged decode ---------------------------------------------------------------
@dataclass(frozen=True)
class Bf16PagedBatchDecodeArgs:
    """decode.rs:1452-1487.  With the reference's eight operands the split-KV
    states live in the command queue's workspace; a caller-owned `workspace`
    (and, for FP8 pages, `kv_scales`) selects the extended form."""
    query: Read
    key_pages: Read
    value_pages: Read
    page_indptr: Read
    page_indices: Read
    last_page_len: Read
    output: Write
    lse: Write
    workspace: Optional[Write] = None
    kv_scales: Optional[Read] = None  # FP8 pages: Read<f32> [k_scale, v_scale]

    @property
    def reference_shaped(self) -> bool:
        return self.workspace is None and self.kv_scales is None

    def _c(self):
        if self.reference_shaped:
            return _ffi.Bf16PagedBatchDecodeArgs(*[_h(getattr(self, f)) for f in (
                "query", "key_pages", "value_pages", "page_indptr", "page_indices",
                "last_page_len", "output", "lse")])
        return _ffi.PagedDecodeArgs(*[_h(getattr(self, f)) for f in (
            "query", "key_pages", "value_pages", "page_indptr", "page_indices",
            "last_page_len", "output", "lse", "workspace", "kv_scales")])

    def __post_init__(self):
        c = self._c()
        object.__setattr__(self, "_struct", c)
        object.__setattr__(self, "_ref", C.byref(c))


class Bf16PagedBatchDecodePlan:
    def __init__(self, ptr, spec):
        self._p = ptr
        self._spec = spec
        self.info = _ffi.PagedDecodePlanInfo()
        lib().loom_paged_decode_plan_get_info(self._p, C.byref(self.info))

    def spec(self):
        return self._spec

    @property
    def algorithm(self) -> str:
        return {1: "balanced_split_kv", 2: "direct"}[self.info.algorithm]

    @property
    def workspace_bytes(self) -> int:
        return self.info.workspace_bytes

    def enqueue_into(self, scope: CommandScope, args: Bf16PagedBatchDecodeArgs):
        fn = (_ffi.load().loom_paged_decode_enqueue_bf16 if args.reference_shaped
              else _ffi.load().loom_paged_decode_enqueue)
        _enqueue(fn, self._p, scope._p, args._ref)

    def enqueue_into_no_alloc(self, scope: CommandScope, args: Bf16PagedBatchDecodeArgs):
        """The same command with the split-KV workspace in the library's static
        per-device scratch: allocates nothing (no reference counterpart).
        Commands that overlap in time on one device race."""
        if not args.reference_shaped:
            raise TypeError("the allocation-free enqueue takes the reference's eight operands")
        _enqueue(_ffi.load().loom_paged_decode_enqueue_bf16_no_alloc, self._p, scope._p,
                 args._ref)

    def __del__(self):
        try:
            if getattr(self, "_p", None):
                lib().loom_paged_decode_plan_free(self._p)
                self._p = None
        except Exception:  # interpreter shutdown: module globals are gone
            pass


# ---- contiguous single decode -------------------------------------------------
class Bf16SingleDecodeSpec:
    """single_decode/mod.rs:15-121: Q/O [Hq, 128], K/V [kv_len, Hkv, 128]."""

    def __init__(self, kv_len, num_query_heads, num_kv_heads, head_dim=HEAD_DIM):
        self._c = _ffi.SingleDecodeSpec()
        _call(lib().loom_single_decode_spec_new, kv_len, num_query_heads, num_kv_heads,
              head_dim, C.byref(self._c))

    kv_len = property(lambda s: s._c.kv_len)
    num_query_heads = property(lambda s: s._c.num_query_heads)
    num_kv_heads = property(lambda s: s._c.num_kv_heads)
    softmax_scale = property(lambda s: s._c.softmax_scale)
    query_numel = property(lambda s: s.num_query_heads * HEAD_DIM)
    kv_numel = property(lambda s: s.kv_len * s.num_kv_heads * HEAD_DIM)
    output_numel = query_numel
    lse_numel = property(lambda s: s.num_query_heads)


class Bf16SingleDecodeSplitKSpec:
    """single_decode/mod.rs:122-194: balanced contiguous token partitions."""

    def __init__(self, decode: Bf16SingleDecodeSpec, partitions: int):
        self._c = _ffi.SingleDecodeSplitKSpec()
        _call(lib().loom_single_decode_split_k_spec_new, C.byref(decode._c), partitions,
              C.byref(self._c))
        self.decode = decode

    partitions = property(lambda s: s._c.partitions)
    partial_state_count = property(lambda s: s.decode.num_query_heads * s.partitions)
    workspace_numel = property(lambda s: s.partial_state_count * PARTIAL_STATE_WIDTH)

    def partition_token_range(self, partition: int):
        st, en = C.c_uint64(), C.c_uint64()
        rc = lib().loom_single_decode_split_k_partition_token_range(
            C.byref(self._c), partition, C.byref(st), C.byref(en))
        return None if rc else (st.value, en.value)


@dataclass(frozen=True)
class Bf16SingleDecodeArgs:
    """decode.rs:1394-1420."""
    query: Read
    key: Read
    value: Read
    output: Write
    lse: Write

    def __post_init__(self):
        c = _ffi.SingleDecodeArgs(*[_h(getattr(self, f)) for f in (
            "query", "key", "value", "output", "lse")])
        object.__setattr__(self, "_struct", c)
        object.__setattr__(self, "_ref", C.byref(c))


@dataclass(frozen=True)
class Bf16SingleDecodeSplitKArgs:
    """decode.rs:1422-1450 (workspace: ReadWrite<f32> [Hq, partitions, 130])."""
    query: Read
    key: Read
    value: Read
    workspace: "ReadWrite"
    output: Write
    lse: Write

    def __post_init__(self):
        c = _ffi.SingleDecodeSplitKArgs(*[_h(getattr(self, f)) for f in (
            "query", "key", "value", "workspace", "output", "lse")])
        object.__setattr__(self, "_struct", c)
        object.__setattr__(self, "_ref", C.byref(c))


class Bf16SingleDecodePlan:
    def __init__(self, ptr, spec):
        self._p = ptr
        self._spec = spec

    def spec(self):
        return self._spec

    def enqueue_into(self, scope: CommandScope, args: Bf16SingleDecodeArgs):
        _enqueue(_ffi.load().loom_single_decode_enqueue, self._p, scope._p, args._ref)

    def __del__(self):
        try:
            if getattr(self, "_p", None):
                lib().loom_single_decode_plan_free(self._p)
                self._p = None
        except Exception:  # interpreter shutdown: module globals are gone
            pass


class Bf16SingleDecodeSplitKPlan:
    def __init__(self, ptr, spec):
        self._p = ptr
        self._spec = spec

    def spec(self):
        return self._spec

    @property
    def workspace_required_bytes(self) -> int:
        return lib().loom_single_decode_split_k_workspace_bytes(self._p)

    @property
    def workspace_required_numel(self) -> int:
        return self.workspace_required_bytes // 4

    def enqueue_into(self, scope: CommandScope, args: Bf16SingleDecodeSplitKArgs):
        _enqueue(_ffi.load().loom_single_decode_split_k_enqueue, self._p, scope._p, args._ref)

    def __del__(self):
        try:
            if getattr(self, "_p", None):
                lib().loom_single_decode_split_k_plan_free(self._p)
                self._p = None
        except Exception:  # interpreter shutdown: module globals are gone
            pass


class DecodeProvider:
    """decode.rs:1001-1104."""

    def __init__(self, ptr, device):
        self._p = ptr
        self.device = device

    @classmethod
    def load(cls, device: int = 0) -> "DecodeProvider":
        out = C.c_void_p()
        _call(lib().loom_decode_provider_load, device, C.byref(out))
        return cls(out.value, device)

    def plan_bf16(self, spec: Bf16SingleDecodeSpec) -> Bf16SingleDecodePlan:
        """decode.rs:1016-1032."""
        out = C.c_void_p()
        _call(lib().loom_decode_provider_plan_bf16, self._p, C.byref(spec._c), C.byref(out))
        return Bf16SingleDecodePlan(out.value, spec)

    def plan_bf16_split_k(self, spec: Bf16SingleDecodeSplitKSpec) -> Bf16SingleDecodeSplitKPlan:
        """decode.rs:1034-1064."""
        out = C.c_void_p()
        _call(lib().loom_decode_provider_plan_bf16_split_k, self._p, C.byref(spec._c),
              C.byref(out))
        return Bf16SingleDecodeSplitKPlan(out.value, spec)

    def plan_bf16_paged_batch(self, spec: Bf16PagedBatchDecodeSpec, max_total_pages: int = 0,
                              teams: int = 0, indices_capacity: bool = False):
        """`teams` = number of equal page ranges (0: chosen for the device);
        `indices_capacity`: page_indices is a capacity (LOOM_PLAN_PAGE_INDICES_CAPACITY)."""
        opt = _ffi.PagedDecodePlanOptions(max_total_pages, teams,
                                          PLAN_PAGE_INDICES_CAPACITY if indices_capacity else 0)
        out = C.c_void_p()
        _call(lib().loom_decode_provider_plan_bf16_paged_batch, self._p, C.byref(spec._c),
              C.byref(opt), C.byref(out))
        return Bf16PagedBatchDecodePlan(out.value, spec)

    def __del__(self):
        try:
            if getattr(self, "_p", None):
                lib().loom_decode_provider_free(self._p)
                self._p = None
        except Exception:  # interpreter shutdown: module globals are gone
            pass


# ---- paged causal prefill ---------------------------------------------------------
class PagedPrefillMetadata:
    """Validated metadata view (paged_prefill/mod.rs:277-384)."""

    def __init__(self, spec: "Bf16PagedPrefillSpec", qo_indptr, indptr, indices, last):
        self.spec = spec
        self.qo_indptr = list(qo_indptr)
        self.page_indptr = list(indptr)
        self.page_indices = list(indices)
        self.last_page_len = list(last)

    def request_query_range(self, request: int):
        if request >= self.spec.batch_size:
            return None
        return self.qo_indptr[request], self.qo_indptr[request + 1]

    def request_page_range(self, request: int):
        if request >= self.spec.batch_size:
            return None
        return self.page_indptr[request], self.page_indptr[request + 1]

    def request_kv_len(self, request: int):
        if request >= self.spec.batch_size:
            return None
        st, en = self.request_page_range(request)
        return (en - st - 1) * self.spec.page_size + self.last_page_len[request]

    def causal_kv_end(self, request: int, query_index: int):
        qo, _ = _i32_array(self.qo_indptr)
        ip, _ = _i32_array(self.page_indptr)
        ln, _ = _i32_array(self.last_page_len)
        out = C.c_uint64()
        rc = lib().loom_paged_prefill_causal_kv_end(C.byref(self.spec._c), qo, ip, ln, request,
                                                    query_index, C.byref(out))
        return None if rc else out.value

    def physical_page_for_token(self, request: int, token: int):
        kv = self.request_kv_len(request)
        if kv is None or token >= kv:
            return None
        P = self.spec.page_size
        return self.page_indices[self.page_indptr[request] + token // P], token % P


class Bf16PagedPrefillSpec:
    """paged_prefill/mod.rs:11-159."""

    def __init__(self, batch_size, nnz_qo, max_num_pages, num_query_heads, num_kv_heads,
                 head_dim=HEAD_DIM, page_size=PAGE_SIZE, kv_layout="NHD", kv_page_size=None,
                 kv_dtype="bf16"):
        self._c = _ffi.PagedPrefillSpec()
        _call(lib().loom_paged_prefill_spec_new, batch_size, nnz_qo, max_num_pages,
              num_query_heads, num_kv_heads, head_dim, page_size, C.byref(self._c))
        code = _layout_code(kv_layout)
        if code != 0:
            out = _ffi.PagedPrefillSpec()
            _call(lib().loom_paged_prefill_spec_with_kv_layout, C.byref(self._c), code,
                  C.byref(out))
            self._c = out
        if kv_page_size is not None:
            out = _ffi.PagedPrefillSpec()
            _call(lib().loom_paged_prefill_spec_with_page_size, C.byref(self._c),
                  int(kv_page_size), C.byref(out))
            self._c = out
        if kv_dtype not in KV_DTYPES:
            raise ValueError(f"kv_dtype must be one of {sorted(KV_DTYPES)}, got {kv_dtype!r}")
        if KV_DTYPES[kv_dtype] != 0:
            out = _ffi.PagedPrefillSpec()
            _call(lib().loom_paged_prefill_spec_with_kv_dtype, C.byref(self._c),
                  KV_DTYPES[kv_dtype], C.byref(out))
            self._c = out

    kv_dtype = property(lambda s: {v: k for k, v in KV_DTYPES.items()}[s._c.kv_dtype])

    kv_layout = property(lambda s: {v: k for k, v in KV_LAYOUTS.items()}[s._c.kv_layout])

    batch_size = property(lambda s: s._c.batch_size)
    nnz_qo = property(lambda s: s._c.nnz_qo)
    max_num_pages = property(lambda s: s._c.max_num_pages)
    num_query_heads = property(lambda s: s._c.num_query_heads)
    num_kv_heads = property(lambda s: s._c.num_kv_heads)
    softmax_scale = property(lambda s: s._c.softmax_scale)
    head_dim = property(lambda s: HEAD_DIM)
    page_size = property(lambda s: s._c.page_size or PAGE_SIZE)
    gqa_group_size = property(lambda s: s.num_query_heads // s.num_kv_heads)
    query_numel = property(lambda s: s.nnz_qo * s.num_query_heads * HEAD_DIM)
    kv_pages_numel = property(lambda s: s.max_num_pages * s.page_size * s.num_kv_heads * HEAD_DIM)
    output_numel = property(lambda s: s.query_numel)
    lse_numel = property(lambda s: s.nnz_qo * s.num_query_heads)
    indptr_numel = property(lambda s: s.batch_size + 1)
    last_page_len_numel = property(lambda s: s.batch_size)

    def kv_head_for_query_head(self, query_head: int):
        return query_head // self.gqa_group_size if query_head < self.num_query_heads else None

    def validate_metadata(self, qo_indptr, indptr, indices, last) -> PagedPrefillMetadata:
        qo, nqo = _i32_array(qo_indptr)
        ip, nip = _i32_array(indptr)
        ix, nix = _i32_array(indices)
        ln, nln = _i32_array(last)
        _call(lib().loom_paged_prefill_validate_metadata, C.byref(self._c), qo, nqo, ip, nip,
              ix, nix, ln, nln)
        return PagedPrefillMetadata(self, qo_indptr, indptr, indices, last)


@dataclass(frozen=True)
class Bf16PagedPrefillArgs:
    """prefill.rs:2852-2890."""
    query: Read
    key_pages: Read
    value_pages: Read
    qo_indptr: Read
    page_indptr: Read
    page_indices: Read
    last_page_len: Read
    output: Write
    lse: Write
    kv_scales: Optional[Read] = None  # FP8 pages: Read<f32> [k_scale, v_scale]

    def __post_init__(self):
        c = _ffi.PagedPrefillArgs(*[_h(getattr(self, f)) for f in (
            "query", "key_pages", "value_pages", "qo_indptr", "page_indptr", "page_indices",
            "last_page_len", "output", "lse", "kv_scales")])
        object.__setattr__(self, "_struct", c)
        object.__setattr__(self, "_ref", C.byref(c))


class Bf16PagedPrefillPlan:
    def __init__(self, ptr, spec):
        self._p = ptr
        self._spec = spec
        self.info = _ffi.PagedPrefillPlanInfo()
        lib().loom_paged_prefill_plan_get_info(self._p, C.byref(self.info))

    def spec(self):
        return self._spec

    @property
    def algorithm(self) -> str:
        return {1: "row_tile", 2: "wide_tile", 3: "long_tile"}[self.info.algorithm]

    def enqueue_into(self, scope: CommandScope, args: Bf16PagedPrefillArgs):
        _enqueue(_ffi.load().loom_paged_prefill_enqueue, self._p, scope._p, args._ref)

    def __del__(self):
        try:
            if getattr(self, "_p", None):
                lib().loom_paged_prefill_plan_free(self._p)
                self._p = None
        except Exception:  # interpreter shutdown: module globals are gone
            pass


class RaggedPrefillMetadata:
    """Validated metadata view (ragged_prefill/mod.rs:196-243)."""

    def __init__(self, spec: "Bf16RaggedPrefillSpec", qo_indptr, kv_indptr):
        self.spec = spec
        self.qo_indptr = list(qo_indptr)
        self.kv_indptr = list(kv_indptr)

    def request_row_ranges(self, request: int):
        if request >= self.spec.batch_size:
            return None
        return ((self.qo_indptr[request], self.qo_indptr[request + 1]),
                (self.kv_indptr[request], self.kv_indptr[request + 1]))

    def causal_kv_end(self, request: int, query_index: int):
        qo, _ = _i32_array(self.qo_indptr)
        kv, _ = _i32_array(self.kv_indptr)
        out = C.c_uint64()
        rc = lib().loom_ragged_prefill_causal_kv_end(C.byref(self.spec._c), qo, kv, request,
                                                     query_index, C.byref(out))
        return None if rc else out.value


class Bf16RaggedPrefillSpec:
    """ragged_prefill/mod.rs:8-167."""

    def __init__(self, batch_size, nnz_qo, nnz_kv, num_query_heads, num_kv_heads,
                 head_dim=HEAD_DIM):
        self._c = _ffi.RaggedPrefillSpec()
        _call(lib().loom_ragged_prefill_spec_new, batch_size, nnz_qo, nnz_kv, num_query_heads,
              num_kv_heads, head_dim, C.byref(self._c))

    batch_size = property(lambda s: s._c.batch_size)
    nnz_qo = property(lambda s: s._c.nnz_qo)
    nnz_kv = property(lambda s: s._c.nnz_kv)
    num_query_heads = property(lambda s: s._c.num_query_heads)
    num_kv_heads = property(lambda s: s._c.num_kv_heads)
    softmax_scale = property(lambda s: s._c.softmax_scale)
    head_dim = property(lambda s: HEAD_DIM)
    gqa_group_size = property(lambda s: s.num_query_heads // s.num_kv_heads)
    query_numel = property(lambda s: s.nnz_qo * s.num_query_heads * HEAD_DIM)
    kv_numel = property(lambda s: s.nnz_kv * s.num_kv_heads * HEAD_DIM)
    output_numel = property(lambda s: s.query_numel)
    lse_numel = property(lambda s: s.nnz_qo * s.num_query_heads)
    indptr_numel = property(lambda s: s.batch_size + 1)

    def kv_head_for_query_head(self, query_head: int):
        return query_head // self.gqa_group_size if query_head < self.num_query_heads else None

    def validate_metadata(self, qo_indptr, kv_indptr) -> RaggedPrefillMetadata:
        qo, nqo = _i32_array(qo_indptr)
        kv, nkv = _i32_array(kv_indptr)
        _call(lib().loom_ragged_prefill_validate_metadata, C.byref(self._c), qo, nqo, kv, nkv)
        return RaggedPrefillMetadata(self, qo_indptr, kv_indptr)


@dataclass(frozen=True)
class Bf16RaggedPrefillArgs:
    """prefill.rs:2893-2931 (`workspace`: the optional with_workspace operand)."""
    query: Read
    key: Read
    value: Read
    qo_indptr: Read
    kv_indptr: Read
    output: Write
    lse: Write
    workspace: Optional["ReadWrite"] = None

    def with_workspace(self, workspace: "ReadWrite") -> "Bf16RaggedPrefillArgs":
        return Bf16RaggedPrefillArgs(self.query, self.key, self.value, self.qo_indptr,
                                     self.kv_indptr, self.output, self.lse, workspace)

    def __post_init__(self):
        c = _ffi.RaggedPrefillArgs(*[_h(getattr(self, f)) for f in (
            "query", "key", "value", "qo_indptr", "kv_indptr", "output", "lse")],
            _h(self.workspace) if self.workspace is not None else _ffi.Handle(0, 0))
        object.__setattr__(self, "_struct", c)
        object.__setattr__(self, "_ref", C.byref(c))


class Bf16RaggedPrefillPlan:
    def __init__(self, ptr, spec):
        self._p = ptr
        self._spec = spec
        self.info = _ffi.RaggedPrefillPlanInfo()
        lib().loom_ragged_prefill_plan_get_info(self._p, C.byref(self.info))

    def spec(self):
        return self._spec

    @property
    def algorithm(self) -> str:
        return {1: "row_tile", 2: "wide_tile"}[self.info.algorithm]

    @property
    def workspace_required_numel(self) -> int:
        return lib().loom_ragged_prefill_workspace_numel(self._p)

    @property
    def workspace_required_bytes(self) -> int:
        return self.workspace_required_numel * 4

    def enqueue_into(self, scope: CommandScope, args: Bf16RaggedPrefillArgs):
        _enqueue(_ffi.load().loom_ragged_prefill_enqueue, self._p, scope._p, args._ref)

    def __del__(self):
        try:
            if getattr(self, "_p", None):
                lib().loom_ragged_prefill_plan_free(self._p)
                self._p = None
        except Exception:  # interpreter shutdown: module globals are gone
            pass


class PrefillProvider:
    """prefill.rs:2278-2410 (the paged and ragged plans)."""

    def __init__(self, ptr, device):
        self._p = ptr
        self.device = device

    @classmethod
    def load(cls, device: int = 0) -> "PrefillProvider":
        out = C.c_void_p()
        _call(lib().loom_prefill_provider_load, device, C.byref(out))
        return cls(out.value, device)

    def plan_bf16_paged(self, spec: Bf16PagedPrefillSpec, waves: int = 0,
                        indices_capacity: bool = False,
                        tile_cols: int = 0) -> Bf16PagedPrefillPlan:
        """`waves` per workgroup (0: chosen from the spec; 4, 8 or 16);
        `indices_capacity`: page_indices is a capacity (LOOM_PLAN_PAGE_INDICES_CAPACITY);
        `tile_cols`: query columns per workgroup (0: chosen from the spec; 16 for
        the row-tile algorithm, 64 for the wide-tile one, "long" for the long
        tiles on BF16 pages)."""
        opt = _ffi.PagedPrefillPlanOptions(
            waves, (PLAN_PAGE_INDICES_CAPACITY if indices_capacity else 0)
            | _prefill_tile_flag(tile_cols))
        out = C.c_void_p()
        _call(lib().loom_prefill_provider_plan_bf16_paged_options, self._p, C.byref(spec._c),
              C.byref(opt), C.byref(out))
        return Bf16PagedPrefillPlan(out.value, spec)

    def plan_bf16_ragged(self, spec: Bf16RaggedPrefillSpec, waves: int = 0,
                         tile_cols: int = 0) -> Bf16RaggedPrefillPlan:
        """prefill.rs:2331-2410; `waves` per workgroup (0: four; 4, 8 or 16);
        `tile_cols` as for the paged plan."""
        opt = _ffi.PagedPrefillPlanOptions(waves, _prefill_tile_flag(tile_cols))
        out = C.c_void_p()
        _call(lib().loom_prefill_provider_plan_bf16_ragged, self._p, C.byref(spec._c),
              C.byref(opt), C.byref(out))
        return Bf16RaggedPrefillPlan(out.value, spec)

    def __del__(self):
        try:
            if getattr(self, "_p", None):
                lib().loom_prefill_provider_free(self._p)
                self._p = None
        except Exception:  # interpreter shutdown: module globals are gone
            pass


# ---- fused RoPE + append --------------------------------------------------------
@dataclass(frozen=True)
class Bf16RopePagedKvAppendArgs:
    """rope/mod.rs:963-1003.  Without a `workspace` (and `kv_scales`) this is
    the reference's struct and the validation words live in the command
    queue's workspace; a caller-owned `workspace` selects the extended form."""
    query: Read
    key: Read
    value: Read
    page_indptr: Read
    page_indices: Read
    last_page_len: Read
    query_output: Write
    key_pages: Write
    value_pages: Write
    workspace: Optional[Write] = None
    batch_indices: Optional[Read] = None
    positions: Optional[Read] = None
    kv_scales: Optional[Read] = None  # FP8 pages: Read<f32> [k_scale, v_scale]

    @property
    def reference_shaped(self) -> bool:
        return self.workspace is None and self.kv_scales is None

    def _c(self):
        if self.reference_shaped and self.batch_indices is None:
            return _ffi.Bf16RopePagedKvAppendArgs(*[_h(getattr(self, f)) for f in (
                "query", "key", "value", "page_indptr", "page_indices", "last_page_len",
                "query_output", "key_pages", "value_pages")])
        if self.reference_shaped:
            return _ffi.Bf16RopePagedKvAppendTokensArgs(*[_h(getattr(self, f)) for f in (
                "query", "key", "value", "batch_indices", "positions", "page_indptr",
                "page_indices", "last_page_len", "query_output", "key_pages", "value_pages")])
        return _ffi.RopeAppendArgs(*[_h(getattr(self, f)) for f in (
            "query", "key", "value", "batch_indices", "positions", "page_indptr",
            "page_indices", "last_page_len", "query_output", "key_pages", "value_pages",
            "workspace", "kv_scales")])

    def __post_init__(self):
        c = self._c()
        object.__setattr__(self, "_struct", c)
        object.__setattr__(self, "_ref", C.byref(c))


def Bf16RopePagedKvAppendTokensArgs(query, key, value, batch_indices, positions, page_indptr,
                                    page_indices, last_page_len, query_output, key_pages,
                                    value_pages, workspace=None, kv_scales=None):
    """rope/mod.rs:1005-1047 (same operand order as the reference)."""
    return Bf16RopePagedKvAppendArgs(query, key, value, page_indptr, page_indices,
                                     last_page_len, query_output, key_pages, value_pages,
                                     workspace, batch_indices, positions, kv_scales)


class Bf16RopePagedKvAppendPlan:
    def __init__(self, ptr, spec):
        self._p = ptr
        self._spec = spec
        self.info = _ffi.RopeAppendPlanInfo()
        lib().loom_rope_append_plan_get_info(self._p, C.byref(self.info))

    def spec(self):
        return self._spec

    @property
    def workspace_bytes(self) -> int:
        return self.info.workspace_bytes

    def enqueue_into(self, scope: CommandScope, args: Bf16RopePagedKvAppendArgs):
        if not args.reference_shaped:
            fn = _ffi.load().loom_rope_append_enqueue
        elif args.batch_indices is None:
            fn = _ffi.load().loom_rope_append_enqueue_bf16
        else:
            fn = _ffi.load().loom_rope_append_tokens_enqueue_bf16
        _enqueue(fn, self._p, scope._p, args._ref)

    def __del__(self):
        try:
            if getattr(self, "_p", None):
                lib().loom_rope_append_plan_free(self._p)
                self._p = None
        except Exception:  # interpreter shutdown: module globals are gone
            pass


class RopeProvider:
    """rope/mod.rs:581-683."""

    def __init__(self, ptr, device):
        self._p = ptr
        self.device = device

    @classmethod
    def load(cls, device: int = 0) -> "RopeProvider":
        out = C.c_void_p()
        _call(lib().loom_rope_provider_load, device, C.byref(out))
        return cls(out.value, device)

    def plan_bf16_paged_append(self, spec: Bf16RopePagedKvAppendSpec,
                               indices_capacity: bool = False, flags: int = 0):
        """rope/mod.rs:628-654.  `flags`: PLAN_APPEND_TWO_LAUNCH and
        PLAN_APPEND_TEST_NO_WAIT (no reference counterpart)."""
        out = C.c_void_p()
        _call(lib().loom_rope_provider_plan_bf16_paged_append_flags, self._p, C.byref(spec._c),
              (PLAN_PAGE_INDICES_CAPACITY if indices_capacity else 0) | flags, C.byref(out))
        return Bf16RopePagedKvAppendPlan(out.value, spec)

    def plan_bf16_paged_append_tokens(self, spec: Bf16RopePagedKvAppendTokensSpec,
                                      indices_capacity: bool = False, flags: int = 0):
        """rope/mod.rs:656-682, with the same `flags` as plan_bf16_paged_append."""
        out = C.c_void_p()
        _call(lib().loom_rope_provider_plan_bf16_paged_append_tokens_flags, self._p,
              C.byref(spec._c), (PLAN_PAGE_INDICES_CAPACITY if indices_capacity else 0) | flags,
              C.byref(out))
        return Bf16RopePagedKvAppendPlan(out.value, spec)

    def __del__(self):
        try:
            if getattr(self, "_p", None):
                lib().loom_rope_provider_free(self._p)
                self._p = None
        except Exception:  # interpreter shutdown: module globals are gone
            pass


# ---- graphs ---------------------------------------------------------------------
class GraphLaunchCompletion:
    def __init__(self, ptr):
        self._p = ptr

    def launch_index(self) -> int:
        return lib().loom_graph_completion_launch_index(self._p)

    def is_complete(self) -> bool:
        out = C.c_int()
        _call(lib().loom_graph_completion_is_complete, self._p, C.byref(out))
        return bool(out.value)

    def wait(self):
        p, self._p = self._p, None
        _call(lib().loom_graph_completion_wait, p)

    def __del__(self):
        try:
            if getattr(self, "_p", None):
                lib().loom_graph_completion_free(self._p)
                self._p = None
        except Exception:  # interpreter shutdown: module globals are gone
            pass


class GraphExec:
    """graph/mod.rs:208-463."""

    def __init__(self, ptr, bindings: CheckedBindings):
        self._p = ptr
        self._bindings = bindings

    def commands(self) -> int:
        return lib().loom_graph_exec_commands(self._p)

    def launches(self) -> int:
        return lib().loom_graph_exec_launches(self._p)

    @property
    def replay_mode(self) -> str:
        """'kernel_nodes' (the captured kernel nodes relaunched in order) or
        'hip_graph_launch' (no reference counterpart)."""
        return GRAPH_REPLAY_MODES.get(lib().loom_graph_exec_replay_mode(self._p), "unknown")

    def set_replay_mode(self, mode: str):
        code = {v: k for k, v in GRAPH_REPLAY_MODES.items()}[mode]
        _call(lib().loom_graph_exec_set_replay_mode, self._p, code)

    def launch(self) -> GraphLaunchCompletion:
        out = C.c_void_p()
        _call(lib().loom_graph_exec_launch, self._p, C.byref(out))
        return GraphLaunchCompletion(out.value)

    def measure_launch_ms(self, start_event, end_event) -> float:
        for ev in (start_event, end_event):
            if not ev.cuda_event:  # torch creates its events lazily on first record
                ev.record()
                ev.synchronize()
        ms = C.c_float()
        _call(lib().loom_graph_exec_measure_launch_ms, self._p,
              C.c_void_p(start_event.cuda_event), C.c_void_p(end_event.cuda_event),
              C.byref(ms))
        return ms.value

    def into_bindings(self) -> CheckedBindings:
        out = C.c_void_p()
        p, self._p = self._p, None
        _call(lib().loom_graph_exec_into_bindings, p, C.byref(out))
        self._bindings._moved = False
        return self._bindings

    def __del__(self):
        try:
            if getattr(self, "_p", None):
                lib().loom_graph_exec_free(self._p)
                self._bindings._p = None
                self._p = None
        except Exception:  # interpreter shutdown: module globals are gone
            pass


class CapturedGraph:
    def __init__(self, ptr, bindings):
        self._p = ptr
        self._bindings = bindings

    def commands(self) -> int:
        return lib().loom_captured_graph_commands(self._p)

    def instantiate(self) -> GraphExec:
        out = C.c_void_p()
        p, self._p = self._p, None
        _call(lib().loom_captured_graph_instantiate, p, C.byref(out))
        return GraphExec(out.value, self._bindings)

    def __del__(self):
        try:
            if getattr(self, "_p", None):
                lib().loom_captured_graph_free(self._p)
                self._bindings._p = None
                self._p = None
        except Exception:  # interpreter shutdown: module globals are gone
            pass


class GraphQueue:
    """graph/mod.rs:22-131: a private stream; one capture per queue."""

    def __init__(self, device: int = 0, max_commands: int = 1):
        out = C.c_void_p()
        _call(lib().loom_graph_queue_new, device, max_commands, C.byref(out))
        self._p = out.value

    def bindings(self, capacity: int) -> CheckedBindings:
        out = C.c_void_p()
        _call(lib().loom_graph_queue_bindings, self._p, capacity, C.byref(out))
        return CheckedBindings(out.value)

    def reserve_workspace(self, scratch_bytes: int = 0, zeroed_bytes: int = 0):
        """CommandQueue.reserve_workspace for the private queue (no reference
        counterpart): reference-shaped decode commands need it before capture."""
        _call(lib().loom_graph_queue_reserve_workspace, self._p, scratch_bytes, zeroed_bytes)

    @property
    def workspace_bytes(self) -> int:
        return lib().loom_graph_queue_workspace_bytes(self._p)

    def capture(self, bindings: CheckedBindings,
                record: Callable[[CommandScope], Any]) -> CapturedGraph:
        sp = C.c_void_p()
        _call(lib().loom_graph_queue_begin_capture, self._p, bindings._p, C.byref(sp))
        bindings._moved = True
        scope = CommandScope(sp.value, bindings, capturing=True)
        record_error = None
        try:
            record(scope)
        except LoomError as e:
            record_error = e
        out = C.c_void_p()
        p, self._p = self._p, None
        try:
            _call(lib().loom_graph_queue_end_capture, p, sp.value, C.byref(out))
        except LoomError:
            bindings._p = None
            if record_error is not None:  # graph/mod.rs:94-101: the record error wins
                raise record_error
            raise
        finally:
            scope._p = None
            lib().loom_graph_queue_free(p)
        graph = CapturedGraph(out.value, bindings)
        if record_error is not None:
            del graph
            raise record_error
        return graph

    def __del__(self):
        try:
            if getattr(self, "_p", None):
                lib().loom_graph_queue_free(self._p)
                self._p = None
        except Exception:  # interpreter shutdown: module globals are gone
            pass
