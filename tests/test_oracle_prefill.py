"""Pins the paged causal prefill oracle before it is trusted as the checker.

The reference's prefill evidence records hold output digests of GPU runs that
differ from its CPU oracle in 1-2 bits, so they cannot pin the oracle.  The
pins here are independent of the oracle's formulas instead:
  * the known-answer outputs and error matrices of the reference's unit tests
    (crates/loom-infer/src/attention/paged_prefill/tests.rs);
  * the fixture digests of the reference's long-prefill evidence record
    (salts, generator and metadata of the shapes it times);
  * bit equality with the paged decode oracle, itself pinned by 0-mismatch
    golden digests, when every request has one query row (the causal end is
    then the whole KV length);
  * closed forms (Q = 0: O = mean of the visible V rows, LSE = log2(end)) that
    fix the bottom-right causal end row by row;
  * an f64 brute-force softmax over the reference's gate and timing shapes.
"""
import json
import math
import os

import numpy as np
import pytest

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                     "reference_digests.json")))
PREFILL_CASES = GOLDEN["paged_prefill"]["cases"] + GOLDEN["paged_prefill_long"]["cases"]


def h(x):
    return int(x, 16)


def fnv_i32(values):
    d = 0xcbf29ce484222325
    for v in values:
        d = ((d ^ (v & 0xFFFFFFFF)) * 0x100000001b3) & 0xFFFFFFFFFFFFFFFF
    return d


def prefill_inputs(oracle, c):
    """Reference gate fixture: Q salt s, K s^0x4b455900, V s^0x56414c554500
    (crates/loom-infer-validation/src/gates/paged_prefill.rs:52-54)."""
    s = oracle.prefill_spec(c["batch"], c["nnz_qo"], c["pool"], c["hq"], c["hkv"])
    salt = h(c["salt"])
    nkv = c["pool"] * 16 * c["hkv"] * 128
    q = oracle.deterministic_bf16(c["nnz_qo"] * c["hq"] * 128, salt)
    k = oracle.deterministic_bf16(nkv, salt ^ 0x4B455900)
    v = oracle.deterministic_bf16(nkv, salt ^ 0x5641_4C55_4500)
    return s, q, k, v


def f64_prefill(oracle, c, q, k, v):
    """One-shot f64 softmax per (row, head) over the bottom-right causal prefix."""
    hq, hkv = c["hq"], c["hkv"]
    g = hq // hkv
    qf = oracle.bf16_to_f32(q).astype(np.float64).reshape(-1, hq, 128)
    kf = oracle.bf16_to_f32(k).astype(np.float64).reshape(c["pool"], 16, hkv, 128)
    vf = oracle.bf16_to_f32(v).astype(np.float64).reshape(c["pool"], 16, hkv, 128)
    out = np.zeros((c["nnz_qo"], hq, 128))
    lse = np.zeros((c["nnz_qo"], hq))
    qo, ip, ix, last = c["qo_indptr"], c["indptr"], c["indices"], c["last"]
    for r in range(c["batch"]):
        L = (ip[r + 1] - ip[r] - 1) * 16 + last[r]
        rows = [(ix[ip[r] + t // 16], t % 16) for t in range(L)]
        kt = np.stack([kf[p, o] for p, o in rows])
        vt = np.stack([vf[p, o] for p, o in rows])
        n = qo[r + 1] - qo[r]
        for i in range(n):
            end = L - n + i + 1
            for qh in range(hq):
                sc = kt[:end, qh // g] @ qf[qo[r] + i, qh] / math.sqrt(128.0)
                w = np.exp(sc - sc.max())
                out[qo[r] + i, qh] = (w @ vt[:end, qh // g]) / w.sum()
                lse[qo[r] + i, qh] = (sc.max() + math.log(w.sum())) / math.log(2.0)
    return out, lse


# ---- fixtures and metadata ----------------------------------------------------
@pytest.mark.parametrize("case", GOLDEN["paged_prefill_long"]["cases"], ids=lambda c: c["name"])
def test_long_prefill_fixture_digests(oracle, case):
    s, q, k, v = prefill_inputs(oracle, case)
    d = case["digests"]
    assert oracle.digest_bf16(q) == h(d["query"])
    assert oracle.digest_bf16(k) == h(d["key_pages"])
    assert oracle.digest_bf16(v) == h(d["value_pages"])
    assert fnv_i32(case["qo_indptr"]) == h(d["qo_indptr"])
    assert fnv_i32(case["indptr"]) == h(d["page_indptr"])
    assert fnv_i32(case["indices"]) == h(d["page_indices"])
    assert fnv_i32(case["last"]) == h(d["last_page_len"])
    oracle.prefill_validate(s, case["qo_indptr"], case["indptr"], case["indices"], case["last"])


def test_metadata_maps_bottom_right_causal_pages(oracle):
    # paged_prefill/tests.rs:3-26
    s = oracle.prefill_spec(2, 3, 6, 4, 2)
    qo, ip, ix, ln = [0, 2, 3], [0, 2, 4], [4, 1, 5, 2], [3, 16]
    oracle.prefill_validate(s, qo, ip, ix, ln)
    assert [oracle.request_kv_len(ip, ln, r) for r in range(2)] == [19, 32]
    end = lambda r, i: oracle.prefill_causal_kv_end(s, qo, ip, ln, r, i)
    assert end(0, 0) == 18 and end(0, 1) == 19 and end(0, 2) is None
    assert end(1, 0) == 32 and end(2, 0) is None
    f = lambda r, t: oracle.physical_page_for_token(ip, ix, ln, r, t)
    assert f(0, 0) == (4, 0) and f(0, 16) == (1, 0) and f(0, 18) == (1, 2) and f(0, 19) is None


# ---- known answers of the reference's unit tests -----------------------------
def test_reference_mask_known_answer(oracle):
    # paged_prefill/tests.rs:28-68: V rows 1, 2, 3, 100 on physical page 1;
    # two query rows over kv_len 4 see 3 and 4 tokens.
    s = oracle.prefill_spec(1, 2, 2, 1, 1)
    q = np.zeros(2 * 128, np.uint16)
    k = np.zeros(2 * 16 * 128, np.uint16)
    vals = np.zeros((2, 16, 128), np.float32)
    for t, x in enumerate([1.0, 2.0, 3.0, 100.0]):
        vals[1, t] = x
    v = oracle.bf16_from_f32(vals.reshape(-1))
    out, lse = oracle.prefill(s, q, k, v, [0, 2], [0, 1], [1], [4])
    of = oracle.bf16_to_f32(out).reshape(2, 128)
    assert np.all(of[0] == 2.0) and np.all(of[1] == 26.5)
    assert np.array_equal(lse, np.array([math.log2(3.0), math.log2(4.0)], np.float32))


def test_reference_gqa_reused_pages_known_answer(oracle):
    # paged_prefill/tests.rs:70-121
    s = oracle.prefill_spec(2, 2, 2, 4, 2)
    q = np.zeros(2 * 4 * 128, np.uint16)
    k = np.zeros(2 * 16 * 2 * 128, np.uint16)
    vals = np.zeros((2, 16, 2, 128), np.float32)
    for p in range(2):
        vals[p, 0, 0] = p + 1.0
        vals[p, 0, 1] = -(p + 1.0)
    v = oracle.bf16_from_f32(vals.reshape(-1))
    out, lse = oracle.prefill(s, q, k, v, [0, 1, 2], [0, 1, 2], [1, 0], [1, 1])
    of = oracle.bf16_to_f32(out).reshape(2, 4, 128)
    for r in range(2):
        pos = 2.0 if r == 0 else 1.0
        assert np.all(of[r, :2] == pos) and np.all(of[r, 2:] == -pos)
    assert np.array_equal(lse, np.zeros(8, np.float32))


MALFORMED = [
    # paged_prefill/tests.rs:123-210 (spec 2, 3, 4, 4, 2)
    (([0, 3], [0, 1, 2], [0, 1], [16, 16]), ("LengthMismatch", "qo_indptr", (3, 2, 0, 0))),
    (([1, 2, 4], [0, 1, 2], [0, 1], [16, 16]), ("InvalidIndptrStart", "qo_indptr", (1, 0, 0, 0))),
    (([0, 2, 1], [0, 1, 2], [0, 1], [16, 16]),
     ("NonMonotonicIndptr", "qo_indptr", (1, 2, 1, 0))),
    (([0, 2, 3], [1, 2, 3], [0, 1, 2], [16, 16]), ("InvalidPageIndptrStart", None, (1, 0, 0, 0))),
    (([0, 2, 3], [0, 2, 1], [0], [16, 16]), ("NonMonotonicPageIndptr", None, (1, 2, 1, 0))),
    (([0, 2, 3], [0, 0, 1], [0], [16, 16]), ("EmptyPagedRequest", None, (0, 0, 0, 0))),
    (([0, 2, 3], [0, 1, 2], [0, 1], [16, 0]), ("InvalidLastPageLength", None, (1, 0, 16, 0))),
    (([0, 2, 3], [0, 1, 2], [0, 4], [16, 16]), ("PageIndexOutOfRange", None, (1, 4, 4, 0))),
    (([0, 2, 3], [0, 1, 2], [0, 1], [1, 16]), ("RaggedQueryLongerThanKv", None, (0, 2, 1, 0))),
    # further variants of validate_query_indptr (paged_prefill/mod.rs:235-264)
    (([0, 0, 3], [0, 1, 2], [0, 1], [16, 16]), ("EmptyRaggedRequest", "qo_indptr", (0, 0, 0, 0))),
    (([0, 1, 2], [0, 1, 2], [0, 1], [16, 16]), ("LengthMismatch", "qo_indptr", (3, 2, 0, 0))),
]


@pytest.mark.parametrize("args,expected", MALFORMED)
def test_metadata_rejections(oracle, args, expected):
    s = oracle.prefill_spec(2, 3, 4, 4, 2)
    with pytest.raises(oracle.OracleError) as e:
        oracle.prefill_validate(s, *args)
    assert (e.value.name, e.value.buffer, e.value.fields) == expected


def test_spec_rejections(oracle):
    # paged_prefill/tests.rs:212-268
    for dims in [(0, 1, 1, 1, 1, 128, 16), (1, 0, 1, 1, 1, 128, 16), (1, 1, 0, 1, 1, 128, 16),
                 (1, 1, 1, 0, 1, 128, 16), (1, 1, 1, 1, 0, 128, 16), (1, 1, 1, 1, 1, 0, 16),
                 (1, 1, 1, 1, 1, 128, 0)]:
        with pytest.raises(oracle.OracleError, match="ZeroDimension"):
            oracle.prefill_spec(*dims)
    with pytest.raises(oracle.OracleError) as e:
        oracle.prefill_spec(1, 1, 1, 1, 1, 64, 16)
    assert e.value.name == "UnsupportedHeadDimension" and e.value.fields[:2] == (128, 64)
    with pytest.raises(oracle.OracleError) as e:
        oracle.prefill_spec(1, 1, 1, 1, 1, 128, 8)
    assert e.value.name == "UnsupportedPageSize" and e.value.fields[:2] == (16, 8)
    with pytest.raises(oracle.OracleError) as e:
        oracle.prefill_spec(1, 1, 1, 6, 4)
    assert e.value.name == "InvalidHeadMapping" and e.value.fields[:2] == (6, 4)
    for dims in [(1, 2 ** 31, 1, 1, 1), (1, 1, 2 ** 64 - 1, 1, 1)]:
        with pytest.raises(oracle.OracleError, match="ElementCountOverflow"):
            oracle.prefill_spec(*dims)
    s = oracle.prefill_spec(1, 1, 1, 1, 1)
    z = np.zeros(16 * 128, np.uint16)
    with pytest.raises(oracle.OracleError) as e:
        oracle.prefill(s, np.zeros(127, np.uint16), z, z, [0, 1], [0, 1], [0], [1])
    assert (e.value.name, e.value.buffer, e.value.fields[:2]) == ("LengthMismatch", "Q", (128, 127))


# ---- reductions to pinned functions and closed forms --------------------------
def test_one_row_per_request_equals_paged_decode_bit_exact(oracle):
    # causal end = kv_len - 1 + 0 + 1 = kv_len: the paged decode loop exactly.
    rng = np.random.default_rng(11)
    B, hq, hkv, pool = 5, 16, 4, 40
    lens = [1, 16, 17, 100, 250]
    pages = [(L + 15) // 16 for L in lens]
    ip = np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)
    ix = rng.permutation(pool)[: ip[-1]].astype(np.int32)
    last = np.array([L - (p - 1) * 16 for L, p in zip(lens, pages)], np.int32)
    q = oracle.deterministic_bf16(B * hq * 128, 0x51)
    k = oracle.deterministic_bf16(pool * 16 * hkv * 128, 0x4B)
    v = oracle.deterministic_bf16(pool * 16 * hkv * 128, 0x56)
    po, pl = oracle.prefill(oracle.prefill_spec(B, B, pool, hq, hkv), q, k, v,
                            np.arange(B + 1), ip, ix, last)
    do, dl = oracle.paged_decode(oracle.paged_spec(B, pool, hq, hkv), q, k, v, ip, ix, last)
    assert np.array_equal(po, do) and np.array_equal(pl, dl)


def test_zero_query_closed_form_fixes_each_causal_end(oracle):
    # Q = 0: every visible token has weight 1, so row i of a request averages
    # exactly the first kv_len - qo_len + i + 1 V rows and LSE = log2(that count).
    rng = np.random.default_rng(3)
    B, hq, hkv, pool = 2, 4, 2, 8
    qo, ip, ix, last = [0, 5, 8], [0, 3, 5], [6, 1, 3, 0, 7], [4, 9]
    s = oracle.prefill_spec(B, 8, pool, hq, hkv)
    vals = rng.integers(-8, 8, size=pool * 16 * hkv * 128).astype(np.float32)
    k = oracle.bf16_from_f32(rng.standard_normal(vals.size).astype(np.float32))
    out, lse = oracle.prefill(s, np.zeros(8 * hq * 128, np.uint16), k,
                              oracle.bf16_from_f32(vals), qo, ip, ix, last)
    vf = vals.reshape(pool, 16, hkv, 128)
    of = oracle.bf16_to_f32(out).reshape(8, hq, 128)
    for r in range(B):
        L = (ip[r + 1] - ip[r] - 1) * 16 + last[r]
        n = qo[r + 1] - qo[r]
        rows = [(ix[ip[r] + t // 16], t % 16) for t in range(L)]
        for i in range(n):
            end = L - n + i + 1
            for qh in range(hq):
                ref = np.stack([vf[p, o, qh // 2] for p, o in rows[:end]]).mean(0)
                np.testing.assert_allclose(of[qo[r] + i, qh], ref, rtol=2 ** -8, atol=1e-6)
                assert abs(lse[(qo[r] + i) * hq + qh] - math.log2(end)) < 1e-6


@pytest.mark.parametrize("case", PREFILL_CASES, ids=lambda c: c["name"])
def test_f64_bruteforce_bound(oracle, case):
    s, q, k, v = prefill_inputs(oracle, case)
    out, lse = oracle.prefill(s, q, k, v, case["qo_indptr"], case["indptr"], case["indices"],
                              case["last"])
    ref, ref_lse = f64_prefill(oracle, case, q, k, v)
    of = oracle.bf16_to_f32(out).reshape(ref.shape)
    # bf16 output rounding (2^-9 relative) plus f32 online-softmax drift
    assert np.all(np.abs(of - ref) <= 2.0 ** -8 * np.maximum(1.0, np.abs(ref)))
    assert np.max(np.abs(lse.reshape(ref_lse.shape) - ref_lse)) < 1e-4
