"""Pins the ragged causal prefill oracle: the output digests the reference's
ragged correctness record holds for its three short gate cases (recorded with 0
GPU bit mismatches against its CPU oracle, so they are that oracle's outputs),
the known answers and error matrices of its unit tests
(crates/loom-infer/src/attention/ragged_prefill/tests.rs), equality with the
paged prefill oracle on the same tokens laid out in pages, and an f64 brute
force on the timed shapes."""
import json
import math
import os

import numpy as np
import pytest

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                     "reference_digests.json")))
RAGGED = GOLDEN["ragged_prefill"]


def h(x):
    return int(x, 16)


def ragged_inputs(oracle, c):
    """gates/ragged_prefill.rs: Q salt s, K s^0x4b455900, V s^0x56414c554500."""
    s = oracle.ragged_spec(c["batch"], c["nnz_qo"], c["nnz_kv"], c["hq"], c["hkv"])
    salt = h(c["salt"])
    q = oracle.deterministic_bf16(c["nnz_qo"] * c["hq"] * 128, salt)
    k = oracle.deterministic_bf16(c["nnz_kv"] * c["hkv"] * 128, salt ^ 0x4B455900)
    v = oracle.deterministic_bf16(c["nnz_kv"] * c["hkv"] * 128, salt ^ 0x5641_4C55_4500)
    return s, q, k, v


@pytest.mark.parametrize("case", [c for c in RAGGED["cases"] if "output_digest" in c],
                         ids=lambda c: c["name"])
def test_golden_output_digest(oracle, case):
    s, q, k, v = ragged_inputs(oracle, case)
    out, lse = oracle.ragged(s, q, k, v, case["qo_indptr"], case["kv_indptr"])
    assert oracle.digest_bf16(out) == h(case["output_digest"])


def test_metadata_maps_bottom_right_causal_bounds(oracle):
    # ragged_prefill/tests.rs:7-19
    s = oracle.ragged_spec(2, 3, 6, 4, 2)
    qo, kv = [0, 2, 3], [0, 4, 6]
    oracle.ragged_validate(s, qo, kv)
    end = lambda r, i: oracle.ragged_causal_kv_end(s, qo, kv, r, i)
    assert (end(0, 0), end(0, 1), end(0, 2), end(1, 0), end(2, 0)) == (3, 4, None, 6, None)


def test_reference_mask_known_answer(oracle):
    # ragged_prefill/tests.rs:21-62
    s = oracle.ragged_spec(1, 2, 4, 1, 1)
    v = oracle.bf16_from_f32(np.repeat(np.array([1.0, 2.0, 3.0, 100.0], np.float32), 128))
    out, lse = oracle.ragged(s, np.zeros(256, np.uint16), np.zeros(512, np.uint16), v, [0, 2],
                             [0, 4])
    of = oracle.bf16_to_f32(out).reshape(2, 128)
    assert np.all(of[0] == 2.0) and np.all(of[1] == 26.5)
    assert np.array_equal(lse, np.array([math.log2(3.0), math.log2(4.0)], np.float32))


def test_reference_gqa_heads_known_answer(oracle):
    # ragged_prefill/tests.rs:64-100
    s = oracle.ragged_spec(2, 2, 2, 4, 2)
    vals = np.zeros((2, 2, 128), np.float32)
    for t in range(2):
        vals[t, 0], vals[t, 1] = t + 1.0, -(t + 1.0)
    out, lse = oracle.ragged(s, np.zeros(2 * 4 * 128, np.uint16), np.zeros(512, np.uint16),
                             oracle.bf16_from_f32(vals.reshape(-1)), [0, 1, 2], [0, 1, 2])
    expect = np.concatenate([np.full(256, 1.0), np.full(256, -1.0), np.full(256, 2.0),
                             np.full(256, -2.0)]).astype(np.float32)
    assert np.array_equal(out, oracle.bf16_from_f32(expect))
    assert np.array_equal(lse, np.zeros(8, np.float32))


MALFORMED = [
    # ragged_prefill/tests.rs:102-158 (spec 2, 3, 5, 4, 2)
    (([0, 3], [0, 2, 5]), ("LengthMismatch", "qo_indptr", (3, 2, 0, 0))),
    (([1, 2, 4], [0, 2, 5]), ("InvalidIndptrStart", "qo_indptr", (1, 0, 0, 0))),
    (([0, 2, 1], [0, 2, 5]), ("NonMonotonicIndptr", "qo_indptr", (1, 2, 1, 0))),
    (([0, 0, 3], [0, 2, 5]), ("EmptyRaggedRequest", "qo_indptr", (0, 0, 0, 0))),
    (([0, 1, 3], [0, 1, 4]), ("LengthMismatch", "kv_indptr", (5, 4, 0, 0))),
    (([0, 2, 3], [0, 1, 5]), ("RaggedQueryLongerThanKv", None, (0, 2, 1, 0))),
    # the kv_indptr variants of validate_indptr (ragged_prefill/mod.rs:169-193)
    (([0, 1, 3], [2, 3, 5]), ("InvalidIndptrStart", "kv_indptr", (2, 0, 0, 0))),
    (([0, 1, 3], [0, 3, 3]), ("EmptyRaggedRequest", "kv_indptr", (1, 0, 0, 0))),
]


@pytest.mark.parametrize("args,expected", MALFORMED)
def test_metadata_rejections(oracle, args, expected):
    s = oracle.ragged_spec(2, 3, 5, 4, 2)
    with pytest.raises(oracle.OracleError) as e:
        oracle.ragged_validate(s, *args)
    assert (e.value.name, e.value.buffer, e.value.fields) == expected


def test_spec_and_length_rejections(oracle):
    # ragged_prefill/tests.rs:160-295
    for dims in [(0, 1, 1, 1, 1, 128), (1, 0, 1, 1, 1, 128), (1, 1, 0, 1, 1, 128),
                 (1, 1, 1, 0, 1, 128), (1, 1, 1, 1, 0, 128), (1, 1, 1, 1, 1, 0)]:
        with pytest.raises(oracle.OracleError, match="ZeroDimension"):
            oracle.ragged_spec(*dims)
    with pytest.raises(oracle.OracleError) as e:
        oracle.ragged_spec(1, 1, 1, 1, 1, 64)
    assert e.value.name == "UnsupportedHeadDimension" and e.value.fields[:2] == (128, 64)
    with pytest.raises(oracle.OracleError) as e:
        oracle.ragged_spec(1, 1, 1, 6, 4)
    assert e.value.name == "InvalidHeadMapping"
    with pytest.raises(oracle.OracleError, match="ElementCountOverflow"):
        oracle.ragged_spec(1, 2 ** 31, 1, 1, 1)
    s = oracle.ragged_spec(1, 1, 1, 1, 1)
    z = np.zeros(128, np.uint16)
    for args, (buf, exp, act) in [((z[:127], z, z, None, None), ("Q", 128, 127)),
                                  ((z, z[:127], z, None, None), ("K", 128, 127)),
                                  ((z, z, z[:127], None, None), ("V", 128, 127)),
                                  ((z, z, z, 127, None), ("O", 128, 127)),
                                  ((z, z, z, None, 0), ("LSE", 1, 0))]:
        q, k, v, ol, ll = args
        with pytest.raises(oracle.OracleError) as e:
            oracle.ragged(s, q, k, v, [0, 1], [0, 1], out_len=ol, lse_len=ll)
        assert (e.value.name, e.value.buffer, e.value.fields[:2]) == ("LengthMismatch", buf,
                                                                      (exp, act))


def test_equals_paged_prefill_on_the_same_tokens(oracle):
    # The same causal attention with the KV rows laid out contiguously or in
    # pages: bit-exact (identical loop, identical token order).
    rng = np.random.default_rng(4)
    B, hq, hkv = 3, 8, 2
    qo_lens, kv_lens = [2, 5, 1], [20, 37, 16]
    qo = np.concatenate([[0], np.cumsum(qo_lens)]).astype(np.int32)
    kv = np.concatenate([[0], np.cumsum(kv_lens)]).astype(np.int32)
    nnz_qo, nnz_kv = int(qo[-1]), int(kv[-1])
    q = oracle.deterministic_bf16(nnz_qo * hq * 128, 0x71)
    k = oracle.deterministic_bf16(nnz_kv * hkv * 128, 0x72)
    v = oracle.deterministic_bf16(nnz_kv * hkv * 128, 0x73)
    ro, rl = oracle.ragged(oracle.ragged_spec(B, nnz_qo, nnz_kv, hq, hkv), q, k, v, qo, kv)
    pages = [(L + 15) // 16 for L in kv_lens]
    ip = np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)
    pool = int(ip[-1]) + 2
    ix = rng.permutation(pool)[: ip[-1]].astype(np.int32)
    last = np.array([L - (p - 1) * 16 for L, p in zip(kv_lens, pages)], np.int32)
    kp = np.zeros((pool, 16, hkv, 128), np.uint16)
    vp = np.zeros_like(kp)
    k3, v3 = k.reshape(nnz_kv, hkv, 128), v.reshape(nnz_kv, hkv, 128)
    for r in range(B):
        for t in range(kv_lens[r]):
            kp[ix[ip[r] + t // 16], t % 16] = k3[kv[r] + t]
            vp[ix[ip[r] + t // 16], t % 16] = v3[kv[r] + t]
    po, pl = oracle.prefill(oracle.prefill_spec(B, nnz_qo, pool, hq, hkv), q, kp.reshape(-1),
                            vp.reshape(-1), qo, ip, ix, last)
    assert np.array_equal(ro, po) and np.array_equal(rl, pl)


@pytest.mark.parametrize("case", RAGGED["timing_cases"], ids=lambda c: c["name"])
def test_f64_bruteforce_bound(oracle, case):
    s, q, k, v = ragged_inputs(oracle, case)
    out, lse = oracle.ragged(s, q, k, v, case["qo_indptr"], case["kv_indptr"])
    hq, hkv = case["hq"], case["hkv"]
    g = hq // hkv
    qf = oracle.bf16_to_f32(q).astype(np.float64).reshape(-1, hq, 128)
    kf = oracle.bf16_to_f32(k).astype(np.float64).reshape(-1, hkv, 128)
    vf = oracle.bf16_to_f32(v).astype(np.float64).reshape(-1, hkv, 128)
    of = oracle.bf16_to_f32(out).reshape(-1, hq, 128)
    lf = lse.reshape(-1, hq)
    qo, kv = case["qo_indptr"], case["kv_indptr"]
    for r in range(case["batch"]):
        n, L = qo[r + 1] - qo[r], kv[r + 1] - kv[r]
        for i in range(n):
            end = kv[r] + L - n + i + 1
            for qh in range(hq):
                sc = kf[kv[r]:end, qh // g] @ qf[qo[r] + i, qh] / math.sqrt(128.0)
                w = np.exp(sc - sc.max())
                ref = (w @ vf[kv[r]:end, qh // g]) / w.sum()
                assert np.all(np.abs(of[qo[r] + i, qh] - ref) <= 2.0 ** -8 * np.maximum(1.0, np.abs(ref)))
                assert abs(lf[qo[r] + i, qh] - (sc.max() + math.log(w.sum())) / math.log(2.0)) < 1e-4
