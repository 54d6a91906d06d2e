"""CPU tests of the product C ABI: exports and the host contract layer.

No compute runs here (no GPU in this container): the library is loaded, every
symbol declared in include/loom_infer_hip.h is resolved, and the host-side
specifications and metadata validation are checked against the reference's
unit-test tables and, on random metadata, against the pinned oracle.
"""
import os
import re

import numpy as np
import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "loom_infer_hip.h")


@pytest.fixture(scope="module")
def L():
    import loom_infer_hip as L
    L.lib()  # raises if the library has not been built
    return L


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(loom_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol(L):
    import ctypes
    lib = ctypes.CDLL(L._ffi.LIB_PATH)
    names = declared_symbols()
    assert len(names) > 60
    missing = [n for n in names if not hasattr(lib, n)]
    assert missing == []
    # and the Python mirror declares a signature for each of them
    assert sorted(L._ffi.SIGNATURES) == names


def test_abi_version_and_status_names(L):
    assert L.lib().loom_abi_version() == 1
    assert L.lib().loom_status_name(14) == b"paged decode request 0 has no KV pages"
    assert b"capacity" in L.lib().loom_status_name(54)


def test_spec_shapes_and_mapping(L):
    # crates/loom-infer/src/attention/paged_decode/tests.rs:21-51
    s = L.Bf16PagedBatchDecodeSpec(3, 7, 8, 2, 128, 16)
    assert (s.batch_size, s.max_num_pages, s.num_query_heads, s.num_kv_heads) == (3, 7, 8, 2)
    assert (s.head_dim, s.page_size, s.gqa_group_size) == (128, 16, 4)
    assert [s.kv_head_for_query_head(i) for i in (0, 3, 4, 7, 8)] == [0, 0, 1, 1, None]
    assert s.query_numel == 3 * 8 * 128 and s.kv_pages_numel == 7 * 16 * 2 * 128
    assert s.lse_numel == 24 and s.page_indptr_numel == 4 and s.last_page_len_numel == 3
    assert s.softmax_scale == np.float32(1.0) / np.sqrt(np.float32(128.0))


def test_spec_rejections(L):
    for dims in [(0, 1, 1, 1, 128, 16), (1, 0, 1, 1, 128, 16), (1, 1, 0, 1, 128, 16),
                 (1, 1, 1, 0, 128, 16), (1, 1, 1, 1, 0, 16), (1, 1, 1, 1, 128, 0)]:
        with pytest.raises(L.ContractError) as e:
            L.Bf16PagedBatchDecodeSpec(*dims)
        assert e.value.variant == "ZeroDimension"
    with pytest.raises(L.ContractError) as e:
        L.Bf16PagedBatchDecodeSpec(1, 1, 1, 1, 64, 16)
    assert (e.value.variant, e.value.fields[:2]) == ("UnsupportedHeadDimension", (128, 64))
    with pytest.raises(L.ContractError) as e:
        L.Bf16PagedBatchDecodeSpec(1, 1, 1, 1, 128, 8)
    assert (e.value.variant, e.value.fields[:2]) == ("UnsupportedPageSize", (16, 8))
    with pytest.raises(L.ContractError) as e:
        L.Bf16PagedBatchDecodeSpec(1, 1, 6, 4)
    assert (e.value.variant, e.value.fields[:2]) == ("InvalidHeadMapping", (6, 4))
    assert str(e.value) == "query heads must be divisible by KV heads: query=6, KV=4"
    for dims in [(2 ** 64 - 1, 1, 1, 1), (1, 2 ** 64 - 1, 1, 1)]:
        with pytest.raises(L.ContractError) as e:
            L.Bf16PagedBatchDecodeSpec(*dims)
        assert e.value.variant == "ElementCountOverflow"


def test_page_table_known_answers(L):
    # crates/loom-infer/src/attention/paged_decode/tests.rs:106-133
    s = L.Bf16PagedBatchDecodeSpec(3, 8, 4, 2)
    t = s.validate_page_table([0, 2, 3, 6], [5, 1, 7, 2, 0, 6], [3, 16, 1])
    assert [t.request_kv_len(r) for r in range(4)] == [19, 16, 33, None]
    f = t.physical_page_for_token
    assert f(0, 0) == (5, 0) and f(0, 15) == (5, 15) and f(0, 16) == (1, 0)
    assert f(0, 18) == (1, 2) and f(0, 19) is None and f(1, 15) == (7, 15)
    assert f(2, 32) == (6, 0) and f(3, 0) is None
    assert t.request_page_range(1) == (2, 3) and t.request_page_range(3) is None


MALFORMED = [
    # crates/loom-infer/src/attention/paged_decode/tests.rs:135-217
    (([0, 1], [0, 1], [16, 16]), ("LengthMismatch", "page_indptr", (3, 2, 0, 0))),
    (([0, 1, 2], [0, 1], [16]), ("LengthMismatch", "last_page_len", (2, 1, 0, 0))),
    (([1, 2, 3], [0, 1, 2], [16, 16]), ("InvalidPageIndptrStart", None, (1, 0, 0, 0))),
    (([0, 2, 1], [0], [16, 16]), ("NonMonotonicPageIndptr", None, (1, 2, 1, 0))),
    (([0, 0, 1], [0], [16, 16]), ("EmptyPagedRequest", None, (0, 0, 0, 0))),
    (([0, 1, 2], [0, 1], [0, 16]), ("InvalidLastPageLength", None, (0, 0, 16, 0))),
    (([0, 1, 2], [0, 1], [16, 17]), ("InvalidLastPageLength", None, (1, 17, 16, 0))),
    (([0, 1, 2], [0], [16, 16]), ("LengthMismatch", "page_indices", (2, 1, 0, 0))),
    (([0, 1, 2], [-1, 1], [16, 16]), ("PageIndexOutOfRange", None, (0, -1, 4, 0))),
    (([0, 1, 2], [0, 4], [16, 16]), ("PageIndexOutOfRange", None, (1, 4, 4, 0))),
]


@pytest.mark.parametrize("args,expected", MALFORMED)
def test_page_table_rejections(L, args, expected):
    s = L.Bf16PagedBatchDecodeSpec(2, 4, 4, 2)
    with pytest.raises(L.ContractError) as e:
        s.validate_page_table(*args)
    assert (e.value.variant, e.value.operand, e.value.fields) == expected


def test_append_contracts_known_answers(L):
    # crates/loom-infer/src/attention/paged_append/tests.rs:72-84, :185-247
    s = L.Bf16RopePagedKvAppendSpec(2, 2, 2, 1, 128, 16)
    with pytest.raises(L.ContractError) as e:
        s.validate_page_table([0, 1, 2], [1, 1], [4, 4])
    assert (e.value.variant, e.value.fields) == ("DuplicatePageAppendSlot", (0, 1, 1, 3))
    ts = L.Bf16RopePagedKvAppendTokensSpec(6, 3, 8, 4, 2, 128, 16)
    slots = ts.validate_metadata([2, 0, 1, 0, 2, 1], [17, 3, 20, 16, 16, 19], [0, 2, 4, 6],
                                 [7, 3, 2, 6, 3, 1], [5, 8, 4])
    assert slots == [(1, 1), (7, 3), (6, 4), (3, 0), (1, 0), (6, 3)]
    ts = L.Bf16RopePagedKvAppendTokensSpec(2, 2, 4, 2, 1, 128, 16)
    md = ([0, 2, 4], [3, 1, 3, 2], [4, 4])
    for bi, pos, want in [([0, 2], [1, 17], ("AppendBatchIndexOutOfRange", (1, 2, 2, 0))),
                          ([0, 1], [1, 20], ("AppendPositionOutOfRange", (1, 1, 20, 20))),
                          ([0, 1], [2, 2], ("DuplicatePageAppendTokenSlot", (0, 1, 3, 2)))]:
        with pytest.raises(L.ContractError) as e:
            ts.validate_metadata(bi, pos, *md)
        assert (e.value.variant, e.value.fields) == want
    with pytest.raises(L.ContractError) as e:
        L.Bf16RopePagedKvAppendTokensSpec(65, 1, 1, 1, 1, 128, 16)
    assert (e.value.variant, e.value.fields[:2]) == ("UnsupportedAppendTokenCount", (64, 65))
    # the extended bulk contract admits the same shape
    assert L.Bf16RopePagedKvAppendTokensSpec.extended(65, 1, 1, 1, 1).tokens == 65
    with pytest.raises(L.ContractError):
        L.Bf16RopePagedKvAppendTokensSpec.extended(8193, 1, 1, 1, 1)


def test_duplicate_slot_reporting_matches_oracle_order(L, oracle):
    """The product finds duplicates with hash maps in O(n); the reference scans
    pairs.  Random tables with many collisions must report the same pair."""
    rng = np.random.default_rng(11)
    for trial in range(200):
        B = int(rng.integers(2, 12))
        pool = int(rng.integers(1, 6))
        pages = rng.integers(1, 3, size=B)
        indptr = np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)
        indices = rng.integers(0, pool, size=int(indptr[-1])).astype(np.int32)
        last = rng.integers(1, 4, size=B).astype(np.int32)
        s = L.Bf16RopePagedKvAppendSpec(B, pool, 2, 1)
        os_ = oracle.paged_spec(B, pool, 2, 1)
        try:
            oracle.append_validate(os_, indptr, indices, last)
            want = None
        except oracle.OracleError as e:
            want = (e.name, e.fields)
        try:
            s.validate_page_table(indptr, indices, last)
            got = None
        except L.ContractError as e:
            got = (e.variant, e.fields)
        assert got == want, (trial, indptr, indices, last)
        # explicit tokens: random requests/positions
        T = int(rng.integers(1, 10))
        bi = rng.integers(0, B, size=T).astype(np.int32)
        kv = (pages - 1) * 16 + last
        pos = np.array([rng.integers(0, kv[b]) for b in bi], np.int32)
        ts = L.Bf16RopePagedKvAppendTokensSpec(T, B, pool, 2, 1)
        try:
            oracle.append_tokens_validate(os_, T, bi, pos, indptr, indices, last)
            want = None
        except oracle.OracleError as e:
            want = (e.name, e.fields)
        try:
            ts.validate_metadata(bi, pos, indptr, indices, last)
            got = None
        except L.ContractError as e:
            got = (e.variant, e.fields)
        assert got == want, (trial, bi, pos)


def test_command_errors_before_any_device_work(L):
    # Queue construction needs a HIP stream; without a GPU the runtime reports a
    # driver error rather than crashing.
    with pytest.raises(L.CommandError) as e:
        L.CommandQueue(0, 0)
    assert e.value.variant == "ZeroCommandCapacity"


def test_single_decode_contracts(L, oracle):
    # crates/loom-infer/src/attention/single_decode/mod.rs:31-70, :131-181
    s = L.Bf16SingleDecodeSpec(127, 16, 4)
    assert (s.kv_len, s.num_query_heads, s.num_kv_heads) == (127, 16, 4)
    assert (s.query_numel, s.kv_numel, s.lse_numel) == (16 * 128, 127 * 4 * 128, 16)
    assert s.softmax_scale == np.float32(1.0 / np.sqrt(np.float32(128.0)))
    for args, variant in [((0, 8, 8), "ZeroDimension"), ((7, 8, 3), "InvalidHeadMapping")]:
        with pytest.raises(L.ContractError) as e:
            L.Bf16SingleDecodeSpec(*args)
        assert e.value.variant == variant
    with pytest.raises(L.ContractError) as e:
        L.Bf16SingleDecodeSpec(7, 8, 8, 64)
    assert e.value.variant == "UnsupportedHeadDimension"
    for p in (0, 128):
        with pytest.raises(L.ContractError) as e:
            L.Bf16SingleDecodeSplitKSpec(s, p)
        assert (e.value.variant, e.value.fields[:2]) == ("InvalidPartitionCount", (p, 127))
    for kv_len, parts in [(7, 3), (33, 6), (127, 10), (5, 5), (1, 1)]:
        sk = L.Bf16SingleDecodeSplitKSpec(L.Bf16SingleDecodeSpec(kv_len, 8, 1), parts)
        assert sk.workspace_numel == 8 * parts * 130
        for p in range(parts + 1):
            assert sk.partition_token_range(p) == oracle.split_k_partition(kv_len, parts, p)


def test_paged_prefill_contracts_match_oracle(L, oracle):
    # crates/loom-infer/src/attention/paged_prefill/mod.rs:30-383 through the
    # C ABI, against the oracle (pinned by the reference's unit tests).
    import test_oracle_prefill as P
    s = L.Bf16PagedPrefillSpec(2, 3, 6, 4, 2)
    assert (s.nnz_qo, s.query_numel, s.kv_pages_numel, s.lse_numel) == (3, 3 * 512, 6 * 16 * 256, 12)
    assert s.softmax_scale == np.float32(1.0 / np.sqrt(np.float32(128.0)))
    m = s.validate_metadata([0, 2, 3], [0, 2, 4], [4, 1, 5, 2], [3, 16])
    os_ = oracle.prefill_spec(2, 3, 6, 4, 2)
    for r in range(3):
        for i in range(3):
            assert m.causal_kv_end(r, i) == oracle.prefill_causal_kv_end(
                os_, [0, 2, 3], [0, 2, 4], [3, 16], r, i)
    assert m.physical_page_for_token(0, 18) == (1, 2) and m.physical_page_for_token(0, 19) is None
    s2 = L.Bf16PagedPrefillSpec(2, 3, 4, 4, 2)
    for args, (variant, buf, fields) in P.MALFORMED:
        with pytest.raises(L.ContractError) as e:
            s2.validate_metadata(*args)
        assert (e.value.variant, e.value.fields) == (variant, fields), args
        if buf:
            assert e.value.operand == buf
    for dims, variant in [((0, 1, 1, 1, 1), "ZeroDimension"), ((1, 1, 1, 6, 4), "InvalidHeadMapping"),
                          ((1, 2 ** 31, 1, 1, 1), "ElementCountOverflow"),
                          ((1, 1, 2 ** 64 - 1, 1, 1), "ElementCountOverflow")]:
        with pytest.raises(L.ContractError) as e:
            L.Bf16PagedPrefillSpec(*dims)
        assert e.value.variant == variant


def test_ragged_prefill_contracts_match_oracle(L, oracle):
    # crates/loom-infer/src/attention/ragged_prefill/mod.rs:27-243 through the
    # C ABI, against the oracle (pinned by the reference's unit tests).
    import test_oracle_ragged as R
    s = L.Bf16RaggedPrefillSpec(2, 3, 6, 4, 2)
    assert (s.nnz_qo, s.nnz_kv, s.query_numel, s.kv_numel, s.lse_numel) == (3, 6, 1536, 1536, 12)
    m = s.validate_metadata([0, 2, 3], [0, 4, 6])
    os_ = oracle.ragged_spec(2, 3, 6, 4, 2)
    for r in range(3):
        for i in range(3):
            assert m.causal_kv_end(r, i) == oracle.ragged_causal_kv_end(os_, [0, 2, 3],
                                                                        [0, 4, 6], r, i)
    assert m.request_row_ranges(1) == ((2, 3), (4, 6)) and m.request_row_ranges(2) is None
    s2 = L.Bf16RaggedPrefillSpec(2, 3, 5, 4, 2)
    for args, (variant, buf, fields) in R.MALFORMED:
        with pytest.raises(L.ContractError) as e:
            s2.validate_metadata(*args)
        assert (e.value.variant, e.value.fields) == (variant, fields), args
        if buf:
            assert e.value.operand == buf
    for dims, variant in [((0, 1, 1, 1, 1), "ZeroDimension"), ((1, 1, 1, 6, 4), "InvalidHeadMapping"),
                          ((1, 2 ** 31, 1, 1, 1), "ElementCountOverflow"),
                          ((1, 1, 2 ** 31, 1, 1), "ElementCountOverflow")]:
        with pytest.raises(L.ContractError) as e:
            L.Bf16RaggedPrefillSpec(*dims)
        assert e.value.variant == variant


def test_kv_layout_specs(L):
    # HND pages (no reference counterpart): the spec setters keep every other
    # field and reject unknown layouts.
    s = L.Bf16PagedBatchDecodeSpec(2, 8, 16, 4, kv_layout="HND")
    assert s.kv_layout == "HND" and (s.batch_size, s.max_num_pages, s.num_kv_heads) == (2, 8, 4)
    assert L.Bf16PagedBatchDecodeSpec(2, 8, 16, 4).kv_layout == "NHD"
    p = L.Bf16PagedPrefillSpec(2, 5, 8, 16, 4, kv_layout="HND")
    assert p.kv_layout == "HND" and p.nnz_qo == 5
    a = L.Bf16RopePagedKvAppendTokensSpec(3, 2, 8, 16, 4, kv_layout="HND")
    assert a.paged.kv_layout == "HND" and a.tokens == 3
    import ctypes as C
    out = L._ffi.PagedDecodeSpec()
    e = L._ffi.Error()
    rc = L.lib().loom_paged_decode_spec_with_kv_layout(C.byref(s._c), 2, C.byref(out), C.byref(e))
    assert rc == 75 and e.operand == b"kv_layout"
    with pytest.raises(ValueError):
        L.Bf16PagedPrefillSpec(2, 5, 8, 16, 4, kv_layout="bad")


def test_page_size_specs(L):
    """Pages of 32 and 64 rows (no reference counterpart: the reference's
    spec_new, like this library's, accepts 16 only).  The page-table contract
    scales with the page size: last_page_len in 1..page_size, token t of a
    request in page t // page_size, row t % page_size."""
    with pytest.raises(L.ContractError) as e:
        L.Bf16PagedBatchDecodeSpec(2, 8, 16, 4, 128, 32)
    assert e.value.variant == "UnsupportedPageSize" and e.value.fields[:2] == (16, 32)
    for bad in (8, 48, 128):
        with pytest.raises(L.ContractError) as e:
            L.Bf16PagedBatchDecodeSpec(2, 8, 16, 4, kv_page_size=bad)
        assert e.value.variant == "UnsupportedPageSize"
    s = L.Bf16PagedBatchDecodeSpec(2, 8, 16, 4, kv_page_size=32, kv_layout="HND")
    assert (s.page_size, s.kv_layout, s.max_num_pages) == (32, "HND", 8)
    assert s.kv_pages_numel == 8 * 32 * 4 * 128
    assert L.Bf16PagedBatchDecodeSpec(2, 8, 16, 4).page_size == 16
    t = s.validate_page_table([0, 2, 3], [5, 1, 7], [20, 32])
    assert (t.request_kv_len(0), t.request_kv_len(1)) == (52, 32)
    assert t.physical_page_for_token(0, 40) == (1, 8)
    assert t.physical_page_for_token(0, 31) == (5, 31)
    assert t.physical_page_for_token(0, 52) is None
    with pytest.raises(L.ContractError) as e:
        s.validate_page_table([0, 2, 3], [5, 1, 7], [20, 33])
    assert (e.value.variant, e.value.fields[:3]) == ("InvalidLastPageLength", (1, 33, 32))
    # a pool whose slot count does not fit 31 bits
    with pytest.raises(L.ContractError) as e:
        L.Bf16PagedBatchDecodeSpec(1, 1 << 26, 1, 1, kv_page_size=64)
    assert e.value.variant == "ElementCountOverflow"
    # append: one-token slots at kv_len - 1, explicit-token slots (page, row)
    a = L.Bf16RopePagedKvAppendSpec(2, 8, 2, 1, kv_page_size=64)
    assert a.paged.page_size == 64 and a.kv_pages_numel == 8 * 64 * 128
    with pytest.raises(L.ContractError) as e:
        a.validate_page_table([0, 1, 2], [3, 3], [10, 10])
    assert (e.value.variant, e.value.fields) == ("DuplicatePageAppendSlot", (0, 1, 3, 9))
    ts = L.Bf16RopePagedKvAppendTokensSpec(3, 2, 8, 2, 1, kv_page_size=32)
    slots = ts.validate_metadata([0, 1, 0], [33, 5, 0], [0, 2, 3], [4, 6, 2], [10, 32])
    assert slots == [(6, 1), (2, 5), (4, 0)]
    # paged prefill: spec_new keeps the reference's 16; the setter takes 32/64
    with pytest.raises(L.ContractError) as e:
        L.Bf16PagedPrefillSpec(2, 5, 8, 16, 4, 128, 32)
    assert e.value.variant == "UnsupportedPageSize"
    ps = L.Bf16PagedPrefillSpec(2, 5, 8, 16, 4, kv_page_size=64)
    assert ps.page_size == 64 and ps.kv_pages_numel == 8 * 64 * 4 * 128
    md = ps.validate_metadata([0, 2, 5], [0, 1, 3], [4, 2, 7], [60, 3])
    assert md.request_kv_len(0) == 60 and md.request_kv_len(1) == 67
    assert md.physical_page_for_token(1, 65) == (7, 1)
    assert md.causal_kv_end(1, 0) == 65
    with pytest.raises(L.ContractError) as e:
        ps.validate_metadata([0, 2, 5], [0, 1, 3], [4, 2, 7], [65, 3])
    assert (e.value.variant, e.value.fields[:3]) == ("InvalidLastPageLength", (0, 65, 64))


def test_fp8_prefill_spec_and_args(L):
    """FP8 E4M3 pages for paged prefill (no reference counterpart): the spec
    setter keeps every other field, rejects unknown element types, and the
    args carry the optional kv_scales operand."""
    s = L.Bf16PagedPrefillSpec(2, 5, 8, 16, 4, kv_dtype="fp8_e4m3", kv_page_size=32,
                               kv_layout="HND")
    assert (s.kv_dtype, s.page_size, s.kv_layout, s.nnz_qo) == ("fp8_e4m3", 32, "HND", 5)
    assert L.Bf16PagedPrefillSpec(2, 5, 8, 16, 4).kv_dtype == "bf16"
    with pytest.raises(ValueError):
        L.Bf16PagedPrefillSpec(2, 5, 8, 16, 4, kv_dtype="fp4")
    import ctypes as C
    out = L._ffi.PagedPrefillSpec()
    e = L._ffi.Error()
    rc = L.lib().loom_paged_prefill_spec_with_kv_dtype(C.byref(s._c), 9, C.byref(out), C.byref(e))
    assert rc == 75 and e.operand == b"kv_dtype"
    assert "kv_scales" in [f for f, _ in L._ffi.PagedPrefillArgs._fields_]
