"""ctypes view of the C oracle (``oracle/libloom_oracle.so``).

TEST INFRASTRUCTURE ONLY.  This module is the parity checker: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` import
it.  The product library never calls into it.

bf16 tensors are numpy ``uint16`` arrays holding the raw bits, exactly as the
reference's ``half::bf16`` values.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# LOOM_ORACLE_LIB selects another build of the oracle (the sanitizer build of
# tests/run_sanitized.sh); the default is the in-tree build.
LIB_PATH = os.environ.get("LOOM_ORACLE_LIB") or os.path.join(_HERE, "libloom_oracle.so")

HEAD_DIM = 128
PAGE_SIZE = 16
STATE_WIDTH = 130
APPEND_MAX_TOKENS = 64

ERROR_NAMES = {
    0: "Ok", 1: "ZeroDimension", 2: "ElementCountOverflow", 3: "InvalidEpsilon",
    4: "UnsupportedHeadDimension", 5: "UnsupportedPageSize", 6: "InvalidHeadMapping",
    7: "InvalidPartitionCount", 8: "InvalidIndptrStart", 9: "NonMonotonicIndptr",
    10: "EmptyRaggedRequest", 11: "RaggedQueryLongerThanKv", 12: "InvalidPageIndptrStart",
    13: "NonMonotonicPageIndptr", 14: "EmptyPagedRequest", 15: "PageIndexOutOfRange",
    16: "InvalidLastPageLength", 17: "InvalidRotaryDimension", 18: "InvalidRopeScale",
    19: "InvalidRopeTheta", 20: "NegativePositionId", 21: "UnsupportedAppendTokenCount",
    22: "AppendBatchIndexOutOfRange", 23: "AppendPositionOutOfRange",
    24: "DuplicatePageAppendSlot", 25: "DuplicatePageAppendTokenSlot",
    26: "UnsupportedDType", 27: "LengthMismatch",
}


class OracleError(Exception):
    def __init__(self, name, buffer, fields):
        super().__init__(f"{name} buffer={buffer} fields={fields}")
        self.name = name
        self.buffer = buffer
        self.fields = fields


class _Err(C.Structure):
    _fields_ = [("code", C.c_int32), ("buffer", C.c_char_p), ("f", C.c_int64 * 4)]


class PagedSpec(C.Structure):
    _fields_ = [("batch_size", C.c_size_t), ("max_num_pages", C.c_size_t),
                ("num_query_heads", C.c_size_t), ("num_kv_heads", C.c_size_t),
                ("softmax_scale", C.c_float)]


class PrefillSpec(C.Structure):
    _fields_ = [("batch_size", C.c_size_t), ("nnz_qo", C.c_size_t),
                ("max_num_pages", C.c_size_t), ("num_query_heads", C.c_size_t),
                ("num_kv_heads", C.c_size_t), ("softmax_scale", C.c_float)]


class RaggedSpec(C.Structure):
    _fields_ = [("batch_size", C.c_size_t), ("nnz_qo", C.c_size_t), ("nnz_kv", C.c_size_t),
                ("num_query_heads", C.c_size_t), ("num_kv_heads", C.c_size_t),
                ("softmax_scale", C.c_float)]


class SingleSpec(C.Structure):
    _fields_ = [("kv_len", C.c_size_t), ("num_query_heads", C.c_size_t),
                ("num_kv_heads", C.c_size_t), ("softmax_scale", C.c_float)]


def build() -> None:
    subprocess.run(["bash", os.path.join(_HERE, "build_oracle.sh")], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing at {LIB_PATH}; run oracle/build_oracle.sh")
        _lib = C.CDLL(LIB_PATH)
        _lib.lo_bf16_from_f32.restype = C.c_uint16
        _lib.lo_bf16_from_f32.argtypes = [C.c_float]
        _lib.lo_bf16_to_f32.restype = C.c_float
        _lib.lo_bf16_to_f32.argtypes = [C.c_uint16]
        _lib.lo_digest_bf16.restype = C.c_uint64
        _lib.lo_digest_f32.restype = C.c_uint64
        _lib.lo_deterministic_bf16.argtypes = [C.c_size_t, C.c_uint64, C.c_void_p]
        _lib.lo_paged_request_kv_len.restype = C.c_int64
        _lib.lo_prefill_causal_kv_end.restype = C.c_int64
        _lib.lo_ragged_causal_kv_end.restype = C.c_int64
        _lib.lo_fp8_e4m3_from_f32.restype = C.c_uint8
        _lib.lo_fp8_e4m3_from_f32.argtypes = [C.c_float]
        _lib.lo_fp8_e4m3_to_f32.restype = C.c_float
        _lib.lo_fp8_e4m3_to_f32.argtypes = [C.c_uint8]
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _check(rc, err):
    if rc != 0:
        buf = err.buffer.decode() if err.buffer else None
        raise OracleError(ERROR_NAMES.get(rc, str(rc)), buf, tuple(err.f))


def _i32(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.int32))


# ---- storage helpers -------------------------------------------------------
def bf16_from_f32(x) -> np.ndarray:
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    out = np.empty(x.shape, dtype=np.uint16)
    lib().lo_f32_to_bf16_array(_p(x), _p(out), C.c_size_t(x.size))
    return out


def bf16_to_f32(b) -> np.ndarray:
    b = np.ascontiguousarray(np.asarray(b, dtype=np.uint16))
    out = np.empty(b.shape, dtype=np.float32)
    lib().lo_bf16_to_f32_array(_p(b), _p(out), C.c_size_t(b.size))
    return out


def deterministic_bf16(n: int, salt: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint16)
    lib().lo_deterministic_bf16(n, salt & 0xFFFFFFFFFFFFFFFF, _p(out))
    return out


def digest_bf16(a) -> int:
    a = np.ascontiguousarray(np.asarray(a, dtype=np.uint16))
    return int(lib().lo_digest_bf16(_p(a), C.c_size_t(a.size)))


def digest_f32(a) -> int:
    a = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    return int(lib().lo_digest_f32(_p(a), C.c_size_t(a.size)))


# ---- paged decode ----------------------------------------------------------
def paged_spec(batch, pool, hq, hkv, head_dim=128, page_size=16) -> PagedSpec:
    s, e = PagedSpec(), _Err()
    _check(lib().lo_paged_spec_new(C.c_size_t(batch), C.c_size_t(pool), C.c_size_t(hq),
                                   C.c_size_t(hkv), C.c_size_t(head_dim),
                                   C.c_size_t(page_size), C.byref(s), C.byref(e)), e)
    return s


def paged_validate(spec, indptr, indices, last):
    indptr, indices, last = _i32(indptr), _i32(indices), _i32(last)
    e = _Err()
    _check(lib().lo_paged_validate(C.byref(spec), _p(indptr), C.c_size_t(indptr.size),
                                   _p(indices), C.c_size_t(indices.size), _p(last),
                                   C.c_size_t(last.size), C.byref(e)), e)


def physical_page_for_token(indptr, indices, last, request, token):
    indptr, indices, last = _i32(indptr), _i32(indices), _i32(last)
    page, off = C.c_int64(), C.c_int64()
    rc = lib().lo_paged_physical_page_for_token(
        _p(indptr), _p(indices), _p(last), C.c_size_t(last.size), C.c_size_t(request),
        C.c_size_t(token), C.byref(page), C.byref(off))
    return None if rc != 0 else (page.value, off.value)


def request_kv_len(indptr, last, request):
    indptr, last = _i32(indptr), _i32(last)
    v = lib().lo_paged_request_kv_len(_p(indptr), _p(last), C.c_size_t(last.size),
                                      C.c_size_t(request))
    return None if v < 0 else int(v)


def paged_decode(spec, q, k, v, indptr, indices, last, out=None, lse=None):
    """Returns (out bf16 bits [B,Hq,128], lse f32 [B,Hq]); raises OracleError."""
    indptr, indices, last = _i32(indptr), _i32(indices), _i32(last)
    q, k, v = (np.ascontiguousarray(x, dtype=np.uint16) for x in (q, k, v))
    nq = spec.batch_size * spec.num_query_heads * HEAD_DIM
    if out is None:
        out = np.full(nq, 0x7FC0, dtype=np.uint16)
    if lse is None:
        lse = np.full(spec.batch_size * spec.num_query_heads, np.nan, dtype=np.float32)
    e = _Err()
    _check(lib().lo_paged_decode_reference(
        C.byref(spec), _p(q), C.c_size_t(q.size), _p(k), C.c_size_t(k.size), _p(v),
        C.c_size_t(v.size), _p(indptr), C.c_size_t(indptr.size), _p(indices),
        C.c_size_t(indices.size), _p(last), C.c_size_t(last.size), _p(out),
        C.c_size_t(out.size), _p(lse), C.c_size_t(lse.size), C.byref(e)), e)
    return out, lse


def paged_decode_requests(spec, q, k, v, indptr, indices, last, r0, r1, out, lse):
    """Restated loop over requests [r0, r1) (used for the bounded CPU baseline)."""
    indptr, indices, last = _i32(indptr), _i32(indices), _i32(last)
    lib().lo_paged_decode_requests(C.byref(spec), _p(q), _p(k), _p(v), _p(indptr),
                                   _p(indices), _p(last), C.c_size_t(r0), C.c_size_t(r1),
                                   _p(out), _p(lse))


def paged_decode_parallel(spec, q, k, v, indptr, indices, last, threads=None):
    """paged_decode with the requests split over host threads (ctypes releases
    the GIL); each request is the same single-threaded loop, so the result is
    bit-identical to paged_decode."""
    from concurrent.futures import ThreadPoolExecutor
    paged_validate(spec, indptr, indices, last)
    indptr, indices, last = _i32(indptr), _i32(indices), _i32(last)
    q, k, v = (np.ascontiguousarray(x, dtype=np.uint16) for x in (q, k, v))
    B, hq = spec.batch_size, spec.num_query_heads
    out = np.full(B * hq * HEAD_DIM, 0x7FC0, dtype=np.uint16)
    lse = np.full(B * hq, np.nan, dtype=np.float32)
    threads = threads or min(16, os.cpu_count() or 1)
    # cut the requests into chunks of about equal token counts
    lens = np.diff(indptr.astype(np.int64)) * PAGE_SIZE
    bounds = np.searchsorted(np.cumsum(lens), np.linspace(0, lens.sum(), 4 * threads + 1)[1:-1])
    cuts = sorted(set([0] + [int(b) + 1 for b in bounds if b + 1 < B] + [B]))
    with ThreadPoolExecutor(threads) as ex:
        list(ex.map(lambda r: paged_decode_requests(spec, q, k, v, indptr, indices, last,
                                                    r[0], r[1], out, lse),
                    zip(cuts[:-1], cuts[1:])))
    return out, lse


# ---- paged causal prefill --------------------------------------------------
def prefill_spec(batch, nnz_qo, pool, hq, hkv, head_dim=128, page_size=16) -> PrefillSpec:
    s, e = PrefillSpec(), _Err()
    _check(lib().lo_prefill_spec_new(*(C.c_size_t(x) for x in (batch, nnz_qo, pool, hq, hkv,
                                                                 head_dim, page_size)),
                                     C.byref(s), C.byref(e)), e)
    return s


def prefill_validate(spec, qo_indptr, indptr, indices, last):
    qo_indptr, indptr, indices, last = (_i32(x) for x in (qo_indptr, indptr, indices, last))
    e = _Err()
    _check(lib().lo_prefill_validate(C.byref(spec), _p(qo_indptr), C.c_size_t(qo_indptr.size),
                                     _p(indptr), C.c_size_t(indptr.size), _p(indices),
                                     C.c_size_t(indices.size), _p(last),
                                     C.c_size_t(last.size), C.byref(e)), e)


def prefill_causal_kv_end(spec, qo_indptr, indptr, last, request, query_index):
    qo_indptr, indptr, last = (_i32(x) for x in (qo_indptr, indptr, last))
    r = lib().lo_prefill_causal_kv_end(C.byref(spec), _p(qo_indptr), _p(indptr), _p(last),
                                       C.c_size_t(request), C.c_size_t(query_index))
    return None if r < 0 else int(r)


def prefill(spec, q, k, v, qo_indptr, indptr, indices, last):
    """Returns (out bf16 bits [nnz_qo,Hq,128], lse f32 [nnz_qo,Hq]); raises OracleError."""
    qo_indptr, indptr, indices, last = (_i32(x) for x in (qo_indptr, indptr, indices, last))
    q, k, v = (np.ascontiguousarray(x, dtype=np.uint16) for x in (q, k, v))
    nq = spec.nnz_qo * spec.num_query_heads * HEAD_DIM
    out = np.full(nq, 0x7FC0, dtype=np.uint16)
    lse = np.full(spec.nnz_qo * spec.num_query_heads, np.nan, dtype=np.float32)
    e = _Err()
    _check(lib().lo_prefill_reference(
        C.byref(spec), _p(q), C.c_size_t(q.size), _p(k), C.c_size_t(k.size), _p(v),
        C.c_size_t(v.size), _p(qo_indptr), C.c_size_t(qo_indptr.size), _p(indptr),
        C.c_size_t(indptr.size), _p(indices), C.c_size_t(indices.size), _p(last),
        C.c_size_t(last.size), _p(out), C.c_size_t(out.size), _p(lse), C.c_size_t(lse.size),
        C.byref(e)), e)
    return out, lse


def prefill_requests(spec, q, k, v, qo_indptr, indptr, indices, last, r0, r1, out, lse):
    """Restated loop over requests [r0, r1) (used for the bounded CPU baseline)."""
    qo_indptr, indptr, indices, last = (_i32(x) for x in (qo_indptr, indptr, indices, last))
    lib().lo_prefill_requests(C.byref(spec), _p(q), _p(k), _p(v), _p(qo_indptr), _p(indptr),
                              _p(indices), _p(last), C.c_size_t(r0), C.c_size_t(r1),
                              _p(out), _p(lse))


# ---- ragged causal prefill -------------------------------------------------
def ragged_spec(batch, nnz_qo, nnz_kv, hq, hkv, head_dim=128) -> RaggedSpec:
    s, e = RaggedSpec(), _Err()
    _check(lib().lo_ragged_spec_new(*(C.c_size_t(x) for x in (batch, nnz_qo, nnz_kv, hq, hkv,
                                                                head_dim)),
                                    C.byref(s), C.byref(e)), e)
    return s


def ragged_validate(spec, qo_indptr, kv_indptr):
    qo_indptr, kv_indptr = _i32(qo_indptr), _i32(kv_indptr)
    e = _Err()
    _check(lib().lo_ragged_validate(C.byref(spec), _p(qo_indptr), C.c_size_t(qo_indptr.size),
                                    _p(kv_indptr), C.c_size_t(kv_indptr.size), C.byref(e)), e)


def ragged_causal_kv_end(spec, qo_indptr, kv_indptr, request, query_index):
    qo_indptr, kv_indptr = _i32(qo_indptr), _i32(kv_indptr)
    r = lib().lo_ragged_causal_kv_end(C.byref(spec), _p(qo_indptr), _p(kv_indptr),
                                      C.c_size_t(request), C.c_size_t(query_index))
    return None if r < 0 else int(r)


def ragged(spec, q, k, v, qo_indptr, kv_indptr, out_len=None, lse_len=None):
    """Returns (out bf16 bits [nnz_qo,Hq,128], lse f32 [nnz_qo,Hq]); raises OracleError."""
    qo_indptr, kv_indptr = _i32(qo_indptr), _i32(kv_indptr)
    q, k, v = (np.ascontiguousarray(x, dtype=np.uint16) for x in (q, k, v))
    nq = spec.nnz_qo * spec.num_query_heads * HEAD_DIM
    out = np.full(nq if out_len is None else out_len, 0x7FC0, dtype=np.uint16)
    n_l = spec.nnz_qo * spec.num_query_heads if lse_len is None else lse_len
    lse = np.full(max(n_l, 1), np.nan, dtype=np.float32)
    e = _Err()
    _check(lib().lo_ragged_reference(
        C.byref(spec), _p(q), C.c_size_t(q.size), _p(k), C.c_size_t(k.size), _p(v),
        C.c_size_t(v.size), _p(qo_indptr), C.c_size_t(qo_indptr.size), _p(kv_indptr),
        C.c_size_t(kv_indptr.size), _p(out), C.c_size_t(out.size), _p(lse), C.c_size_t(n_l),
        C.byref(e)), e)
    return out, lse


def ragged_requests(spec, q, k, v, qo_indptr, kv_indptr, r0, r1, out, lse):
    """Restated loop over requests [r0, r1) (bounded CPU-baseline sample)."""
    qo_indptr, kv_indptr = _i32(qo_indptr), _i32(kv_indptr)
    lib().lo_ragged_requests(C.byref(spec), _p(q), _p(k), _p(v), _p(qo_indptr), _p(kv_indptr),
                             C.c_size_t(r0), C.c_size_t(r1), _p(out), _p(lse))


# ---- single decode / split-K ----------------------------------------------
def single_spec(kv_len, hq, hkv, head_dim=128) -> SingleSpec:
    s, e = SingleSpec(), _Err()
    _check(lib().lo_single_spec_new(C.c_size_t(kv_len), C.c_size_t(hq), C.c_size_t(hkv),
                                    C.c_size_t(head_dim), C.byref(s), C.byref(e)), e)
    return s


def single_decode(spec, q, k, v):
    out = np.empty(spec.num_query_heads * HEAD_DIM, dtype=np.uint16)
    lse = np.empty(spec.num_query_heads, dtype=np.float32)
    lib().lo_single_decode_reference(C.byref(spec), _p(q), _p(k), _p(v), _p(out), _p(lse))
    return out, lse


def split_k_partition(kv_len, partitions, partition):
    s, t = C.c_size_t(), C.c_size_t()
    rc = lib().lo_split_k_partition(C.c_size_t(kv_len), C.c_size_t(partitions),
                                    C.c_size_t(partition), C.byref(s), C.byref(t))
    return None if rc != 0 else (s.value, t.value)


def split_k(spec, partitions, q, k, v):
    ws = np.full(spec.num_query_heads * partitions * STATE_WIDTH, np.nan, dtype=np.float32)
    e = _Err()
    _check(lib().lo_split_k_partials_reference(C.byref(spec), C.c_size_t(partitions), _p(q),
                                               _p(k), _p(v), _p(ws), C.byref(e)), e)
    out = np.empty(spec.num_query_heads * HEAD_DIM, dtype=np.uint16)
    lse = np.empty(spec.num_query_heads, dtype=np.float32)
    _check(lib().lo_split_k_merge_reference(C.byref(spec), C.c_size_t(partitions), _p(ws),
                                            _p(out), _p(lse), C.byref(e)), e)
    return out, lse, ws


# ---- RoPE and append -------------------------------------------------------
def rope_pos_ids(tokens, qh, kh, q, k, positions, head_dim=128, rotary_dim=128,
                 scale=1.0, theta=10000.0):
    positions = _i32(positions)
    qo = np.full(tokens * qh * head_dim, 0x7FC0, dtype=np.uint16)
    ko = np.full(tokens * kh * head_dim, 0x7FC0, dtype=np.uint16)
    e = _Err()
    _check(lib().lo_rope_pos_ids_reference(
        C.c_size_t(tokens), C.c_size_t(qh), C.c_size_t(kh), C.c_size_t(head_dim),
        C.c_size_t(rotary_dim), C.c_float(scale), C.c_float(theta), _p(q), _p(k),
        _p(positions), _p(qo), _p(ko), C.byref(e)), e)
    return qo, ko


def append_validate(spec, indptr, indices, last):
    indptr, indices, last = _i32(indptr), _i32(indices), _i32(last)
    e = _Err()
    _check(lib().lo_append_validate(C.byref(spec), _p(indptr), C.c_size_t(indptr.size),
                                    _p(indices), C.c_size_t(indices.size), _p(last),
                                    C.c_size_t(last.size), C.byref(e)), e)


def append(spec, q, k, v, indptr, indices, last, k_pages, v_pages):
    """One-token-per-request append. k_pages/v_pages are updated in place."""
    indptr, indices, last = _i32(indptr), _i32(indices), _i32(last)
    qo = np.full(spec.batch_size * spec.num_query_heads * HEAD_DIM, 0x7FC0, dtype=np.uint16)
    e = _Err()
    _check(lib().lo_append_reference(
        C.byref(spec), _p(q), _p(k), _p(v), _p(indptr), C.c_size_t(indptr.size), _p(indices),
        C.c_size_t(indices.size), _p(last), C.c_size_t(last.size), _p(qo), _p(k_pages),
        _p(v_pages), C.byref(e)), e)
    return qo


def append_tokens_validate(spec, tokens, batch_indices, positions, indptr, indices, last,
                           max_tokens=APPEND_MAX_TOKENS):
    bi, pos = _i32(batch_indices), _i32(positions)
    indptr, indices, last = _i32(indptr), _i32(indices), _i32(last)
    slots = np.zeros(2 * max(tokens, 1), dtype=np.int64)
    e = _Err()
    _check(lib().lo_append_tokens_validate(
        C.byref(spec), C.c_size_t(tokens), C.c_size_t(max_tokens), _p(bi), _p(pos),
        _p(indptr), C.c_size_t(indptr.size), _p(indices), C.c_size_t(indices.size), _p(last),
        C.c_size_t(last.size), _p(slots), C.byref(e)), e)
    return [tuple(int(x) for x in slots[2 * t:2 * t + 2]) for t in range(tokens)]


def append_tokens(spec, tokens, q, k, v, batch_indices, positions, indptr, indices, last,
                  k_pages, v_pages, max_tokens=APPEND_MAX_TOKENS):
    bi, pos = _i32(batch_indices), _i32(positions)
    indptr, indices, last = _i32(indptr), _i32(indices), _i32(last)
    qo = np.full(tokens * spec.num_query_heads * HEAD_DIM, 0x7FC0, dtype=np.uint16)
    e = _Err()
    _check(lib().lo_append_tokens_reference(
        C.byref(spec), C.c_size_t(tokens), C.c_size_t(max_tokens), _p(q), _p(k), _p(v),
        _p(bi), _p(pos), _p(indptr), C.c_size_t(indptr.size), _p(indices),
        C.c_size_t(indices.size), _p(last), C.c_size_t(last.size), _p(qo), _p(k_pages),
        _p(v_pages), C.byref(e)), e)
    return qo


# ---- FP8 E4M3 KV storage (no reference counterpart) ---------------------------
def fp8_from_f32(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.size, dtype=np.uint8)
    lib().lo_fp8_e4m3_from_f32_array(_p(x), _p(out), C.c_size_t(x.size))
    return out


def fp8_to_f32(b) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint8)
    out = np.empty(b.size, dtype=np.float32)
    lib().lo_fp8_e4m3_to_f32_array(_p(b), _p(out), C.c_size_t(b.size))
    return out


def paged_decode_fp8(spec, q, k8, v8, indptr, indices, last, k_scale, v_scale):
    """Paged decode over FP8 pages (metadata must be valid: checked here with the
    BF16 contract's page-table validation)."""
    paged_validate(spec, indptr, indices, last)
    indptr, indices, last = _i32(indptr), _i32(indices), _i32(last)
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k8, v8 = (np.ascontiguousarray(x, dtype=np.uint8) for x in (k8, v8))
    out = np.empty(spec.batch_size * spec.num_query_heads * HEAD_DIM, dtype=np.uint16)
    lse = np.empty(spec.batch_size * spec.num_query_heads, dtype=np.float32)
    lib().lo_paged_decode_fp8_requests(C.byref(spec), _p(q), _p(k8), _p(v8), _p(indptr),
                                       _p(indices), _p(last), C.c_size_t(0),
                                       C.c_size_t(spec.batch_size), C.c_float(k_scale),
                                       C.c_float(v_scale), _p(out), _p(lse))
    return out, lse


def append_tokens_fp8(spec, tokens, q, k, v, batch_indices, positions, indptr, indices, last,
                      k_pages, v_pages, k_scale, v_scale, max_tokens=APPEND_MAX_TOKENS):
    """Explicit-token append writing FP8 pages in place; returns the BF16 query output."""
    bi, pos = _i32(batch_indices), _i32(positions)
    indptr, indices, last = _i32(indptr), _i32(indices), _i32(last)
    q_out = np.empty(tokens * spec.num_query_heads * HEAD_DIM, dtype=np.uint16)
    e = _Err()
    _check(lib().lo_append_tokens_fp8_reference(
        C.byref(spec), C.c_size_t(tokens), C.c_size_t(max_tokens), _p(q), _p(k), _p(v),
        _p(bi), _p(pos), _p(indptr), C.c_size_t(indptr.size), _p(indices),
        C.c_size_t(indices.size), _p(last), C.c_size_t(last.size), C.c_float(k_scale),
        C.c_float(v_scale), _p(q_out), _p(k_pages), _p(v_pages), C.byref(e)), e)
    return q_out
