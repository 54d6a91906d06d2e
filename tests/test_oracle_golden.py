"""Pins the C oracle before it is trusted as the parity checker.

Every check here is independent of the oracle's own formulas: recorded golden
digests from the reference's evidence records, known-answer tables and error
matrices from the reference's unit tests, closed forms, invariants and an f64
brute-force softmax.
"""
import json
import math
import os

import numpy as np
import pytest

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                     "reference_digests.json")))


def h(x):
    return int(x, 16)


def fnv_i32(values):
    d = 0xcbf29ce484222325
    for v in values:
        d = ((d ^ (v & 0xFFFFFFFF)) * 0x100000001b3) & 0xFFFFFFFFFFFFFFFF
    return d


# ---- storage helpers --------------------------------------------------------
def test_fnv_known_answer(oracle):
    g = GOLDEN["fnv_known_answer"]
    bits = oracle.bf16_from_f32(np.array(g["values_f32"], np.float32))
    assert oracle.digest_bf16(bits) == h(g["digest"])


def test_fixture_digests_pin_xorshift_and_bf16_rounding(oracle):
    g = GOLDEN["fixture_digests"]
    for key in ("query", "key_pages"):
        e = g[key]
        assert oracle.digest_bf16(oracle.deterministic_bf16(e["len"], h(e["salt"]))) == h(e["digest"])
    assert fnv_i32(g["page_indptr"]["values"]) == h(g["page_indptr"]["digest"])
    assert fnv_i32(g["page_indices"]["values"]) == h(g["page_indices"]["digest"])


def test_bf16_round_to_nearest_even_and_nan(oracle):
    # half::bf16::from_f32: RNE on the top 16 bits; NaN gets the quiet bit.
    cases = {1.0: 0x3F80, -2.0: 0xC000, 1.00390625: 0x3F80,   # exact tie -> even
             1.01171875: 0x3F82,                                 # tie -> round up to even
             3.0e38: 0x7F62, float("inf"): 0x7F80}
    for x, bits in cases.items():
        assert int(oracle.bf16_from_f32(np.array([x], np.float32))[0]) == bits, x
    nan_bits = np.array([0x7F800001], np.uint32).view(np.float32)
    assert int(oracle.bf16_from_f32(nan_bits)[0]) == 0x7FC0
    # every bf16 round-trips exactly
    allb = np.arange(0, 65536, dtype=np.uint32).astype(np.uint16)
    f = oracle.bf16_to_f32(allb)
    finite = np.isfinite(f)
    assert np.array_equal(oracle.bf16_from_f32(f)[finite], allb[finite])


# ---- paged decode ------------------------------------------------------------
def _paged_inputs(oracle, c):
    s = oracle.paged_spec(c["batch"], c["pool"], c["hq"], c["hkv"])
    salt = h(c["salt"])
    nq = c["batch"] * c["hq"] * 128
    nkv = c["pool"] * 16 * c["hkv"] * 128
    q = oracle.deterministic_bf16(nq, salt)
    k = oracle.deterministic_bf16(nkv, salt ^ 0x4B455900)
    v = oracle.deterministic_bf16(nkv, salt ^ 0x5641_4C55_4500)
    return s, q, k, v


@pytest.mark.parametrize("case", GOLDEN["paged_decode"]["cases"], ids=lambda c: c["name"])
def test_paged_decode_golden_output_digest(oracle, case):
    s, q, k, v = _paged_inputs(oracle, case)
    out, lse = oracle.paged_decode(s, q, k, v, case["indptr"], case["indices"], case["last"])
    assert oracle.digest_bf16(out) == h(case["output_digest"])
    # LSE bits are not pinned by a 0-mismatch record; bound it by the f64 softmax.
    ref_lse = _f64_lse(oracle, s, q, k, case)
    assert np.max(np.abs(lse.astype(np.float64) - ref_lse)) < 1e-5


def _f64_lse(oracle, s, q, k, c):
    qf = oracle.bf16_to_f32(q).astype(np.float64).reshape(c["batch"], c["hq"], 128)
    kf = oracle.bf16_to_f32(k).astype(np.float64).reshape(c["pool"], 16, c["hkv"], 128)
    g = c["hq"] // c["hkv"]
    out = np.zeros((c["batch"], c["hq"]))
    for r in range(c["batch"]):
        toks = []
        L = (c["indptr"][r + 1] - c["indptr"][r] - 1) * 16 + c["last"][r]
        for t in range(L):
            toks.append(kf[c["indices"][c["indptr"][r] + t // 16], t % 16])
        kt = np.stack(toks)  # [L, hkv, 128]
        for qh in range(c["hq"]):
            sc = kt[:, qh // g] @ qf[r, qh] / math.sqrt(128.0)
            m = sc.max()
            out[r, qh] = (m + math.log(np.exp(sc - m).sum())) / math.log(2.0)
    return out.reshape(-1)


def test_paged_decode_f64_bruteforce_output_bound(oracle):
    # Random ragged case: the f32 online softmax stays within bf16 rounding of an
    # f64 softmax computed in one shot.
    rng = np.random.default_rng(7)
    B, hq, hkv, pool = 3, 8, 2, 20
    s = oracle.paged_spec(B, pool, hq, hkv)
    lens = [5, 37, 64]
    pages = [(L + 15) // 16 for L in lens]
    indptr = np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)
    indices = rng.permutation(pool)[: indptr[-1]].astype(np.int32)
    last = np.array([L - (p - 1) * 16 for L, p in zip(lens, pages)], np.int32)
    q = oracle.bf16_from_f32(rng.standard_normal(B * hq * 128).astype(np.float32))
    k = oracle.bf16_from_f32(rng.standard_normal(pool * 16 * hkv * 128).astype(np.float32))
    v = oracle.bf16_from_f32(rng.standard_normal(pool * 16 * hkv * 128).astype(np.float32))
    out, lse = oracle.paged_decode(s, q, k, v, indptr, indices, last)
    qf = oracle.bf16_to_f32(q).astype(np.float64).reshape(B, hq, 128)
    kf = oracle.bf16_to_f32(k).astype(np.float64).reshape(pool, 16, hkv, 128)
    vf = oracle.bf16_to_f32(v).astype(np.float64).reshape(pool, 16, hkv, 128)
    of = oracle.bf16_to_f32(out).reshape(B, hq, 128)
    for r in range(B):
        rows = [(indices[indptr[r] + t // 16], t % 16) for t in range(lens[r])]
        for qh in range(hq):
            kv = qh // (hq // hkv)
            kt = np.stack([kf[p, o, kv] for p, o in rows])
            vt = np.stack([vf[p, o, kv] for p, o in rows])
            sc = kt @ qf[r, qh] / math.sqrt(128.0)
            w = np.exp(sc - sc.max())
            ref = (w @ vt) / w.sum()
            assert np.max(np.abs(of[r, qh] - ref)) <= 2.0 ** -8 * max(1.0, np.abs(ref).max())
            ref_lse = (sc.max() + math.log(w.sum())) / math.log(2.0)
            assert abs(lse[r * hq + qh] - ref_lse) < 1e-4


def test_paged_decode_closed_form_zero_query(oracle):
    # Q = 0 => uniform weights: O = mean(V), LSE = log2(kv_len)
    # (crates/loom-infer-validation/src/gates/paged_batch_decode.rs:281-293 uses 4.0 for L=16).
    s = oracle.paged_spec(2, 3, 4, 2)
    rng = np.random.default_rng(1)
    q = np.zeros(2 * 4 * 128, np.uint16)
    k = oracle.bf16_from_f32(rng.standard_normal(3 * 16 * 2 * 128).astype(np.float32))
    vals = rng.integers(-8, 8, size=3 * 16 * 2 * 128).astype(np.float32)
    v = oracle.bf16_from_f32(vals)
    out, lse = oracle.paged_decode(s, q, k, v, [0, 1, 3], [2, 0, 1], [16, 16])
    assert np.array_equal(lse, np.array([4.0] * 4 + [5.0] * 4, np.float32))
    vf = vals.reshape(3, 16, 2, 128)
    of = oracle.bf16_to_f32(out).reshape(2, 4, 128)
    for qh in range(4):
        np.testing.assert_allclose(of[0, qh], vf[2, :, qh // 2].mean(0), rtol=2 ** -8, atol=1e-6)
        ref1 = np.concatenate([vf[0, :, qh // 2], vf[1, :, qh // 2]]).mean(0)
        np.testing.assert_allclose(of[1, qh], ref1, rtol=2 ** -8, atol=1e-6)


def test_paged_equals_contiguous_single_decode_bit_exact(oracle):
    # crates/loom-infer/src/attention/paged_decode/tests.rs:219-291
    s = oracle.paged_spec(3, 7, 8, 2)
    indptr, indices, last = [0, 1, 3, 6], [4, 6, 1, 5, 0, 3], [1, 7, 16]
    q = oracle.deterministic_bf16(3 * 8 * 128, 0x5041_4745_4451)
    k = oracle.deterministic_bf16(7 * 16 * 2 * 128, 0x5041_4745_444B)
    v = oracle.deterministic_bf16(7 * 16 * 2 * 128, 0x5041_4745_4456)
    out, lse = oracle.paged_decode(s, q, k, v, indptr, indices, last)
    k4, v4 = k.reshape(7, 16, 2, 128), v.reshape(7, 16, 2, 128)
    for r in range(3):
        L = oracle.request_kv_len(indptr, last, r)
        rows = [oracle.physical_page_for_token(indptr, indices, last, r, t) for t in range(L)]
        kc = np.stack([k4[p, o] for p, o in rows]).reshape(-1)
        vc = np.stack([v4[p, o] for p, o in rows]).reshape(-1)
        ss = oracle.single_spec(L, 8, 2)
        eo, el = oracle.single_decode(ss, q[r * 1024:(r + 1) * 1024], kc, vc)
        assert np.array_equal(out[r * 1024:(r + 1) * 1024], eo)
        assert np.array_equal(lse[r * 8:(r + 1) * 8], el)


def test_page_table_known_answers(oracle):
    # crates/loom-infer/src/attention/paged_decode/tests.rs:106-133
    ip, ix, ln = [0, 2, 3, 6], [5, 1, 7, 2, 0, 6], [3, 16, 1]
    s = oracle.paged_spec(3, 8, 4, 2)
    oracle.paged_validate(s, ip, ix, ln)
    assert [oracle.request_kv_len(ip, ln, r) for r in range(4)] == [19, 16, 33, None]
    f = lambda r, t: oracle.physical_page_for_token(ip, ix, ln, r, t)
    assert f(0, 0) == (5, 0) and f(0, 15) == (5, 15) and f(0, 16) == (1, 0)
    assert f(0, 18) == (1, 2) and f(0, 19) is None and f(1, 15) == (7, 15)
    assert f(2, 32) == (6, 0) and f(3, 0) is None


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
def test_page_table_rejections(oracle, args, expected):
    s = oracle.paged_spec(2, 4, 4, 2)
    with pytest.raises(oracle.OracleError) as e:
        oracle.paged_validate(s, *args)
    assert (e.value.name, e.value.buffer, e.value.fields) == expected


def test_spec_rejections(oracle):
    # crates/loom-infer/src/attention/paged_decode/tests.rs:53-104
    for dims in [(0, 1, 1, 1, 128, 16), (1, 0, 1, 1, 128, 16), (1, 1, 0, 1, 128, 16),
                 (1, 1, 1, 0, 128, 16), (1, 1, 1, 1, 0, 16), (1, 1, 1, 1, 128, 0)]:
        with pytest.raises(oracle.OracleError, match="ZeroDimension"):
            oracle.paged_spec(*dims)
    with pytest.raises(oracle.OracleError) as e:
        oracle.paged_spec(1, 1, 1, 1, 64, 16)
    assert e.value.name == "UnsupportedHeadDimension" and e.value.fields[:2] == (128, 64)
    with pytest.raises(oracle.OracleError) as e:
        oracle.paged_spec(1, 1, 1, 1, 128, 8)
    assert e.value.name == "UnsupportedPageSize" and e.value.fields[:2] == (16, 8)
    with pytest.raises(oracle.OracleError) as e:
        oracle.paged_spec(1, 1, 6, 4)
    assert e.value.name == "InvalidHeadMapping" and e.value.fields[:2] == (6, 4)
    big = 2 ** 64 - 1
    for dims in [(big, 1, 1, 1), (1, big, 1, 1)]:
        with pytest.raises(oracle.OracleError, match="ElementCountOverflow"):
            oracle.paged_spec(*dims)


# ---- single decode / split-K -------------------------------------------------
@pytest.mark.parametrize("case", GOLDEN["single_decode_direct"]["cases"], ids=lambda c: c["name"])
def test_single_decode_golden_and_split_k_invariant(oracle, case):
    s = oracle.single_spec(case["kv_len"], case["hq"], case["hkv"])
    salt = h(case["salt"])
    n = case["kv_len"] * case["hkv"] * 128
    q = oracle.deterministic_bf16(case["hq"] * 128, salt)
    k = oracle.deterministic_bf16(n, salt ^ 0x4B455900)
    v = oracle.deterministic_bf16(n, salt ^ 0x5641_4C55_4500)
    out, lse = oracle.single_decode(s, q, k, v)
    assert oracle.digest_bf16(out) == h(case["output_digest"])
    so, sl, _ = oracle.split_k(s, case["partitions"], q, k, v)
    assert np.max(np.abs(oracle.bf16_to_f32(so) - oracle.bf16_to_f32(out))) <= 2.0 ** -8
    assert np.max(np.abs(sl - lse)) <= 1e-5


@pytest.mark.parametrize("kv_len,hq,hkv,parts,salt", [
    (1, 8, 8, 1, 0x1001), (7, 8, 1, 3, 0x2001), (33, 8, 1, 8, 0x3001), (127, 16, 4, 8, 0x4001)])
def test_split_k_matches_direct_bit_exact_on_reference_shapes(oracle, kv_len, hq, hkv, parts, salt):
    # crates/loom-infer/src/attention/single_decode/tests.rs:303-355 (its exact tuples)
    s = oracle.single_spec(kv_len, hq, hkv)
    n = kv_len * hkv * 128
    q = oracle.deterministic_bf16(hq * 128, salt)
    k = oracle.deterministic_bf16(n, salt ^ 0x4B455900)
    v = oracle.deterministic_bf16(n, salt ^ 0x5641_4C55_4500)
    out, lse = oracle.single_decode(s, q, k, v)
    so, sl, _ = oracle.split_k(s, parts, q, k, v)
    assert np.array_equal(so, out)
    assert np.max(np.abs(sl - lse)) <= 1e-6


def test_split_k_state_layout_known_answer(oracle):
    # crates/loom-infer/src/attention/single_decode/tests.rs:276-301
    s = oracle.single_spec(2, 1, 1)
    q = np.zeros(128, np.uint16)
    q[0] = oracle.bf16_from_f32(np.float32(math.sqrt(128.0)))[0]
    k = np.zeros(256, np.uint16)
    k[128] = oracle.bf16_from_f32(np.float32(1.0))[0]
    v = np.concatenate([np.full(128, oracle.bf16_from_f32(np.float32(1.5))),
                        np.full(128, oracle.bf16_from_f32(np.float32(-2.0)))]).astype(np.uint16)
    _, _, ws = oracle.split_k(s, 2, q, k, v)
    assert ws[0] == 0.0 and ws[1] == 1.0 and np.all(ws[2:130] == 1.5)
    score = np.float32(oracle.bf16_to_f32(q[:1])[0]) * np.float32(s.softmax_scale) * np.float32(
        1.44269504088896340735992468100189214)
    assert ws[130] == score and ws[131] == 1.0 and np.all(ws[132:] == -2.0)


def test_split_k_partition_is_balanced(oracle):
    # single_decode/mod.rs:171-185: base=L/P and the first L%P partitions get one more.
    for L, P in [(7, 3), (33, 6), (127, 10), (5, 5)]:
        ranges = [oracle.split_k_partition(L, P, p) for p in range(P)]
        assert ranges[0][0] == 0 and ranges[-1][1] == L
        assert all(a[1] == b[0] for a, b in zip(ranges, ranges[1:]))
        sizes = [e - b for b, e in ranges]
        assert sizes == [L // P + (1 if p < L % P else 0) for p in range(P)]
    assert oracle.split_k_partition(7, 3, 3) is None


def test_split_k_large_logits_stay_finite(oracle):
    # single_decode/tests.rs:357-387
    s = oracle.single_spec(3, 1, 1)
    q = np.full(128, oracle.bf16_from_f32(np.float32(64.0)), np.uint16)
    k = oracle.bf16_from_f32(np.concatenate([np.full(128, -64.0), np.zeros(128),
                                             np.full(128, 64.0)]).astype(np.float32))
    v = np.full(384, oracle.bf16_from_f32(np.float32(1.0)), np.uint16)
    o, l, ws = oracle.split_k(s, 3, q, k, v)
    assert np.all(np.isfinite(ws)) and np.all(np.isfinite(oracle.bf16_to_f32(o)))
    assert np.all(np.isfinite(l))


# ---- RoPE and append ----------------------------------------------------------
def test_rope_closed_form_d6_rot4(oracle):
    # crates/loom-infer/src/rope/tests.rs:3-40, with numpy float32 math.
    vals = oracle.bf16_from_f32(np.arange(1, 7, dtype=np.float32))
    qo, ko = oracle.rope_pos_ids(1, 1, 1, vals, vals, [1], head_dim=6, rotary_dim=4)
    f32 = np.float32
    c0, s0 = math.cos(1.0), math.sin(1.0)
    a1 = float(np.power(f32(10000.0), f32(-0.5)))
    c1, s1 = math.cos(a1), math.sin(a1)
    exp = [f32(1) * f32(c0) - f32(3) * f32(s0), f32(2) * f32(c1) - f32(4) * f32(s1),
           f32(3) * f32(c0) + f32(1) * f32(s0), f32(4) * f32(c1) + f32(2) * f32(s1)]
    assert list(qo[:4]) == [int(oracle.bf16_from_f32(np.array([x], f32))[0]) for x in exp]
    assert list(qo[4:]) == list(vals[4:]) and np.array_equal(qo, ko)


def test_rope_zero_position_is_identity(oracle):
    # crates/loom-infer/src/rope/tests.rs:42-59
    q = oracle.bf16_from_f32(np.arange(256, dtype=np.float32) / 256.0 - 0.5)
    k = oracle.bf16_from_f32(np.arange(128, dtype=np.float32) / 128.0 - 0.25)
    qo, ko = oracle.rope_pos_ids(1, 2, 1, q, k, [0])
    assert np.array_equal(qo, q) and np.array_equal(ko, k)


def test_rope_large_position_stays_finite(oracle):
    # crates/loom-infer/src/rope/tests.rs:61-81
    q = np.full(128, oracle.bf16_from_f32(np.array([0.25], np.float32))[0], np.uint16)
    k = np.full(128, oracle.bf16_from_f32(np.array([-0.5], np.float32))[0], np.uint16)
    qo, ko = oracle.rope_pos_ids(1, 1, 1, q, k, [32767])
    assert np.all(np.isfinite(oracle.bf16_to_f32(qo))) and np.all(np.isfinite(oracle.bf16_to_f32(ko)))
    # |rotated| <= |x1| + |x2| elementwise
    assert np.all(np.abs(oracle.bf16_to_f32(qo)) <= 0.5 + 2 ** -8)


def test_rope_rejects_negative_position(oracle):
    with pytest.raises(oracle.OracleError) as e:
        oracle.rope_pos_ids(1, 1, 1, np.zeros(2, np.uint16), np.zeros(2, np.uint16), [-1],
                            head_dim=2, rotary_dim=2)
    assert e.value.name == "NegativePositionId" and e.value.fields[:2] == (0, -1)


def _append_inputs(oracle, g, tokens_key):
    s = oracle.paged_spec(g["batch"], g["pool"], g["hq"], g["hkv"])
    n = g[tokens_key] if tokens_key else g["batch"]
    sl = {k: h(v) for k, v in g["salts"].items()}
    nkv = g["pool"] * 16 * g["hkv"] * 128
    q = oracle.deterministic_bf16(n * g["hq"] * 128, sl["query"])
    k = oracle.deterministic_bf16(n * g["hkv"] * 128, sl["key"])
    v = oracle.deterministic_bf16(n * g["hkv"] * 128, sl["value"])
    kp = oracle.deterministic_bf16(nkv, sl["key_pages"])
    vp = oracle.deterministic_bf16(nkv, sl["value_pages"])
    return s, q, k, v, kp, vp


def test_append_one_token_golden(oracle):
    g = GOLDEN["append_one_token"]
    s, q, k, v, kp, vp = _append_inputs(oracle, g, None)
    qo = oracle.append(s, q, k, v, g["indptr"], g["indices"], g["last"], kp, vp)
    assert oracle.digest_bf16(qo) == h(g["query_digest"])
    assert oracle.digest_bf16(kp) == h(g["key_pages_digest"])
    assert oracle.digest_bf16(vp) == h(g["value_pages_digest"])
    for r, slot in enumerate(g["physical_slots"]):
        pos = oracle.request_kv_len(g["indptr"], g["last"], r) - 1
        assert pos == g["positions"][r]
        assert oracle.physical_page_for_token(g["indptr"], g["indices"], g["last"], r, pos) == tuple(slot)


def test_append_tokens_t6_golden(oracle):
    g = GOLDEN["append_tokens_t6"]
    s, q, k, v, kp, vp = _append_inputs(oracle, g, "tokens")
    slots = oracle.append_tokens_validate(s, 6, g["batch_indices"], g["positions"], g["indptr"],
                                          g["indices"], g["last"])
    assert slots == [tuple(x) for x in g["physical_slots"]]
    qo = oracle.append_tokens(s, 6, q, k, v, g["batch_indices"], g["positions"], g["indptr"],
                              g["indices"], g["last"], kp, vp)
    assert oracle.digest_bf16(qo) == h(g["query_digest"])
    assert oracle.digest_bf16(vp) == h(g["value_pages_digest"])


def test_append_tokens_t64_golden(oracle):
    g = GOLDEN["append_tokens_t64"]
    s, q, k, v, kp, vp = _append_inputs(oracle, g, "tokens")
    oracle.append_tokens(s, 64, q, k, v, [0] * 64, list(range(64)), g["indptr"], g["indices"],
                         g["last"], kp, vp)
    assert oracle.digest_bf16(kp) == h(g["key_pages_digest"])
    assert oracle.digest_bf16(vp) == h(g["value_pages_digest"])


def test_append_known_slots_and_rejections(oracle):
    # crates/loom-infer/src/attention/paged_append/tests.rs:15-84, 116-247
    ip, ix, ln = [0, 1, 3, 5], [7, 2, 6, 5, 1], [3, 1, 16]
    got = [oracle.physical_page_for_token(ip, ix, ln, r, oracle.request_kv_len(ip, ln, r) - 1)
           for r in range(3)]
    assert got == [(7, 2), (6, 0), (1, 15)]
    with pytest.raises(oracle.OracleError) as e:
        oracle.append_validate(oracle.paged_spec(2, 2, 2, 1), [0, 1, 2], [1, 1], [4, 4])
    assert e.value.name == "DuplicatePageAppendSlot" and e.value.fields == (0, 1, 1, 3)
    s = oracle.paged_spec(3, 8, 4, 2)
    slots = oracle.append_tokens_validate(s, 6, [2, 0, 1, 0, 2, 1], [17, 3, 20, 16, 16, 19],
                                          [0, 2, 4, 6], [7, 3, 2, 6, 3, 1], [5, 8, 4])
    assert slots == [(1, 1), (7, 3), (6, 4), (3, 0), (1, 0), (6, 3)]
    s = oracle.paged_spec(2, 4, 2, 1)
    args = ([0, 2, 4], [3, 1, 3, 2], [4, 4])
    for bi, pos, want in [([0, 2], [1, 17], ("AppendBatchIndexOutOfRange", (1, 2, 2, 0))),
                          ([0, 1], [1, 20], ("AppendPositionOutOfRange", (1, 1, 20, 20))),
                          ([0, 1], [2, 2], ("DuplicatePageAppendTokenSlot", (0, 1, 3, 2)))]:
        with pytest.raises(oracle.OracleError) as e:
            oracle.append_tokens_validate(s, 2, bi, pos, *args)
        assert (e.value.name, e.value.fields) == want
    with pytest.raises(oracle.OracleError) as e:
        oracle.append_tokens_validate(oracle.paged_spec(1, 1, 1, 1), 65, [0] * 65, [0] * 65,
                                      [0, 1], [0], [16])
    assert e.value.name == "UnsupportedAppendTokenCount" and e.value.fields[:2] == (64, 65)


def test_parallel_paged_decode_equals_serial(oracle):
    """paged_decode_parallel (requests split over host threads, used by the
    full-size GPU parity tests) is bit-identical to the serial oracle."""
    rng = np.random.default_rng(17)
    B, hq, hkv = 9, 16, 4
    lens = rng.integers(1, 400, size=B)
    pages = (lens + 15) // 16
    pool = int(pages.sum()) + 5
    indptr = np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)
    indices = rng.permutation(pool)[: indptr[-1]].astype(np.int32)
    last = (lens - (pages - 1) * 16).astype(np.int32)
    q = oracle.bf16_from_f32(rng.standard_normal(B * hq * 128, dtype=np.float32))
    k = oracle.bf16_from_f32(rng.standard_normal(pool * 16 * hkv * 128, dtype=np.float32))
    v = oracle.bf16_from_f32(rng.standard_normal(pool * 16 * hkv * 128, dtype=np.float32))
    s = oracle.paged_spec(B, pool, hq, hkv)
    a = oracle.paged_decode(s, q, k, v, indptr, indices, last)
    b = oracle.paged_decode_parallel(s, q, k, v, indptr, indices, last, threads=4)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
