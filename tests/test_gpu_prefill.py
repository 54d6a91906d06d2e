"""GPU parity of paged causal prefill (libloom_infer_hip.so through the C ABI)
against the pinned CPU oracle: the reference's gate and timing fixtures, seeded
ragged shapes over every waves-per-workgroup variant, and the reference's
device-guard cases (crates/loom-infer-validation/src/gates/paged_prefill.rs)."""
import json
import os
import sys

import numpy as np
import pytest

from gpu_util import (PrefillRunner, bf16_host, compare_decode, nan_bf16, seeded_normal_bf16,
                      to_dev_bf16, to_dev_i32)

pytestmark = pytest.mark.gpu

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                     "reference_digests.json")))
GATE = GOLDEN["paged_prefill"]["cases"] + GOLDEN["paged_prefill_long"]["cases"]
WAVES = (4, 8, 16)


@pytest.fixture(scope="module")
def L():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import loom_infer_hip as L
    return L


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def gate_inputs(oracle, c):
    salt = int(c["salt"], 16)
    nkv = c["pool"] * 16 * c["hkv"] * 128
    q = oracle.deterministic_bf16(c["nnz_qo"] * c["hq"] * 128, salt)
    k = oracle.deterministic_bf16(nkv, salt ^ 0x4B455900)
    v = oracle.deterministic_bf16(nkv, salt ^ 0x5641_4C55_4500)
    return q, k, v


@pytest.mark.parametrize("case", GATE, ids=lambda c: c["name"])
def test_gate_fixtures(L, oracle, case):
    # gates/paged_prefill.rs:541-584 and benchmarks/matched.rs:1392-1425
    log(f"prefill gate fixture {case['name']}")
    q, k, v = gate_inputs(oracle, case)
    s = oracle.prefill_spec(case["batch"], case["nnz_qo"], case["pool"], case["hq"], case["hkv"])
    meta = (case["qo_indptr"], case["indptr"], case["indices"], case["last"])
    ref_out, ref_lse = oracle.prefill(s, q, k, v, *meta)
    for waves in (0,) + WAVES:
        r = PrefillRunner(L, case["batch"], case["nnz_qo"], case["pool"], case["hq"],
                          case["hkv"], waves=waves)
        out, lse = r.run(q, k, v, *meta)
        stats = compare_decode(oracle, out, lse, ref_out, ref_lse)
        log(f"  waves={r.plan.info.waves} {stats}")


def ragged_meta(rng, qo_lens, kv_lens, pool, reuse=False):
    pages = [(L + 15) // 16 for L in kv_lens]
    indptr = np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)
    if reuse:
        indices = rng.integers(0, pool, size=indptr[-1]).astype(np.int32)
    else:
        assert indptr[-1] <= pool
        indices = rng.permutation(pool)[: indptr[-1]].astype(np.int32)
    last = np.array([L - (p - 1) * 16 for L, p in zip(kv_lens, pages)], np.int32)
    qo = np.concatenate([[0], np.cumsum(qo_lens)]).astype(np.int32)
    return qo, indptr, indices, last


SHAPES = [
    # (name, hq, hkv, qo_lens, kv_lens)
    ("mha_full_causal", 8, 8, [33], [33]),
    ("gqa4_tile_edges", 16, 4, [1, 3, 4, 5, 8], [1, 17, 64, 100, 9]),
    ("gqa8_mixed", 32, 4, [2, 7, 31], [40, 300, 31]),
    ("mqa_long_rows", 8, 1, [1, 16, 64], [512, 128, 700]),
    ("group16_two_rows", 32, 2, [2, 1], [50, 1000]),
    ("group5_odd", 10, 2, [3, 9, 1], [20, 9, 77]),
    ("group3_tail_pages", 12, 4, [6, 13], [16, 33]),
    ("llama_gqa4_prompt", 32, 8, [128, 96], [128, 1000]),
]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: s[0])
@pytest.mark.parametrize("waves", WAVES)
def test_ragged_shapes(L, oracle, shape, waves):
    name, hq, hkv, qo_lens, kv_lens = shape
    log(f"prefill {name} waves={waves}")
    rng = np.random.default_rng(sum(kv_lens) + waves)
    pool = sum((L_ + 15) // 16 for L_ in kv_lens) + 3
    qo, ip, ix, last = ragged_meta(rng, qo_lens, kv_lens, pool)
    B, nnz = len(qo_lens), int(qo[-1])
    q = seeded_normal_bf16(oracle, rng, nnz * hq * 128)
    k = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    ref_out, ref_lse = oracle.prefill(oracle.prefill_spec(B, nnz, pool, hq, hkv), q, k, v,
                                      qo, ip, ix, last)
    r = PrefillRunner(L, B, nnz, pool, hq, hkv, waves=waves)
    out, lse = r.run(q, k, v, qo, ip, ix, last)
    log(f"  {compare_decode(oracle, out, lse, ref_out, ref_lse)}")


def test_reused_pages_and_nan_outside_valid_rows(L, oracle):
    # Pages shared by several requests (gqa4_reordered_reuse style) and NaN in
    # every pool row no request can see: the range-limited loads must not read
    # past a request's tail, and masked rows must not leak into the sums.
    rng = np.random.default_rng(5)
    hq, hkv, pool = 16, 4, 12
    qo_lens, kv_lens = [3, 5, 2, 7], [35, 18, 5, 60]
    qo, ip, ix, last = ragged_meta(rng, qo_lens, kv_lens, pool, reuse=True)
    B, nnz = 4, int(qo[-1])
    q = seeded_normal_bf16(oracle, rng, nnz * hq * 128)
    kf = rng.standard_normal((pool, 16, hkv, 128), dtype=np.float32)
    vf = rng.standard_normal((pool, 16, hkv, 128), dtype=np.float32)
    visible = np.zeros((pool, 16), bool)
    for r in range(B):
        for t in range(kv_lens[r]):
            visible[ix[ip[r] + t // 16], t % 16] = True
    kf[~visible] = np.nan
    vf[~visible] = np.nan
    k, v = oracle.bf16_from_f32(kf.reshape(-1)), oracle.bf16_from_f32(vf.reshape(-1))
    ref_out, ref_lse = oracle.prefill(oracle.prefill_spec(B, nnz, pool, hq, hkv), q, k, v,
                                      qo, ip, ix, last)
    for waves in WAVES:
        out, lse = PrefillRunner(L, B, nnz, pool, hq, hkv, waves=waves).run(
            q, k, v, qo, ip, ix, last)
        log(f"  reuse+nan waves={waves} {compare_decode(oracle, out, lse, ref_out, ref_lse)}")


def test_many_requests_cross_scan_blocks(L, oracle):
    # More requests than one workgroup's threads (the tile-prefix scan carries
    # across blocks) with one or two rows each.
    rng = np.random.default_rng(9)
    B, hq, hkv = 1100, 8, 2
    qo_lens = rng.integers(1, 3, size=B).tolist()
    kv_lens = [int(x) + 2 for x in rng.integers(1, 40, size=B)]
    pool = sum((L_ + 15) // 16 for L_ in kv_lens)
    qo, ip, ix, last = ragged_meta(rng, qo_lens, kv_lens, pool)
    nnz = int(qo[-1])
    q = seeded_normal_bf16(oracle, rng, nnz * hq * 128)
    k = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    ref_out, ref_lse = oracle.prefill(oracle.prefill_spec(B, nnz, pool, hq, hkv), q, k, v,
                                      qo, ip, ix, last)
    for waves in (4, 16):
        out, lse = PrefillRunner(L, B, nnz, pool, hq, hkv, waves=waves).run(
            q, k, v, qo, ip, ix, last)
        log(f"  B=1100 waves={waves} {compare_decode(oracle, out, lse, ref_out, ref_lse)}")


# ---- device guards (prefill.rs:293-342; gates/paged_prefill.rs:238-314) ------------
def _guard_setup(oracle):
    rng = np.random.default_rng(21)
    hq, hkv, pool = 8, 2, 10
    qo_lens, kv_lens = [2, 3, 1], [20, 35, 9]
    qo, ip, ix, last = ragged_meta(rng, qo_lens, kv_lens, pool)
    nnz = int(qo[-1])
    q = seeded_normal_bf16(oracle, rng, nnz * hq * 128)
    k = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    ref = oracle.prefill(oracle.prefill_spec(3, nnz, pool, hq, hkv), q, k, v, qo, ip, ix, last)
    return (hq, hkv, pool, nnz), (q, k, v), (qo, ip, ix, last), ref


def _rows(qo, r, hq):
    return slice(int(qo[r]) * hq, int(qo[r + 1]) * hq)


@pytest.mark.parametrize("waves", (4, 16))
def test_invalid_page_index_keeps_only_that_request(L, oracle, waves):
    (hq, hkv, pool, nnz), (q, k, v), (qo, ip, ix, last), (ref_out, ref_lse) = _guard_setup(oracle)
    bad = ix.copy()
    bad[ip[1] + 1] = pool  # request 1's second page, past its first row's causal pages
    out, lse = PrefillRunner(L, 3, nnz, pool, hq, hkv, waves=waves).run(
        q, k, v, qo, ip, bad, last)
    o = out.reshape(nnz * hq, 128)
    ro = ref_out.reshape(nnz * hq, 128)
    assert np.all(o[_rows(qo, 1, hq)] == 0x7FC0) and np.all(np.isnan(lse[_rows(qo, 1, hq)]))
    for r in (0, 2):
        sl = _rows(qo, r, hq)
        compare_decode(oracle, o[sl].reshape(-1), lse[sl], ro[sl].reshape(-1), ref_lse[sl])


def test_query_longer_than_kv_and_bad_tail_keep_sentinels(L, oracle):
    (hq, hkv, pool, nnz), (q, k, v), (qo, ip, ix, last), (ref_out, ref_lse) = _guard_setup(oracle)
    r = PrefillRunner(L, 3, nnz, pool, hq, hkv)
    # request 2 (one row) gets last_page_len 0; request 0 keeps its rows valid
    bad_last = last.copy()
    bad_last[2] = 0
    out, lse = r.run(q, k, v, qo, ip, ix, bad_last)
    assert np.all(np.isnan(lse[_rows(qo, 2, hq)]))
    assert np.all(np.isfinite(lse[_rows(qo, 0, hq)])) and np.all(np.isfinite(lse[_rows(qo, 1, hq)]))
    # qo_len > kv_len for request 0: 3 rows over a 2-token cache
    qo2 = np.array([0, 3, 5, 6], np.int32)
    ip2 = np.array([0, 1, 4, 5], np.int32)
    last2 = np.array([2, 3, 9], np.int32)
    out, lse = r.run(q, k, v, qo2, ip2, ix[:5], last2)
    assert np.all(np.isnan(lse[: 3 * hq])) and np.all(np.isfinite(lse[3 * hq:]))


def test_malformed_qo_range_stops_the_request_search(L, oracle):
    (hq, hkv, pool, nnz), (q, k, v), (qo, ip, ix, last), (ref_out, ref_lse) = _guard_setup(oracle)
    r = PrefillRunner(L, 3, nnz, pool, hq, hkv)
    # qo = [0, 2, 2, 6]: request 1 is empty -> request 0 computed, 1 and 2 not
    qo_bad = np.array([0, 2, 2, nnz], np.int32)
    out, lse = r.run(q, k, v, qo_bad, ip, ix, last)
    assert np.all(np.isfinite(lse[: 2 * hq])) and np.all(np.isnan(lse[2 * hq:]))
    o = out.reshape(nnz * hq, 128)
    compare_decode(oracle, o[: 2 * hq].reshape(-1), lse[: 2 * hq],
                   ref_out.reshape(nnz * hq, 128)[: 2 * hq].reshape(-1), ref_lse[: 2 * hq])


@pytest.mark.parametrize("field", ["qo_start", "qo_end", "page_start", "page_end"])
def test_invalid_global_metadata_writes_nothing(L, oracle, field):
    (hq, hkv, pool, nnz), (q, k, v), (qo, ip, ix, last), _ = _guard_setup(oracle)
    qo_b, ip_b = qo.copy(), ip.copy()
    if field == "qo_start":
        qo_b[0] = 1
    elif field == "qo_end":
        qo_b[-1] = nnz - 1
    elif field == "page_start":
        ip_b[0] = 1
    else:
        ip_b[-1] = ip[-1] - 1  # page_indptr[B] != len(page_indices)
    out, lse = PrefillRunner(L, 3, nnz, pool, hq, hkv).run(q, k, v, qo_b, ip_b, ix, last)
    assert np.all(out == 0x7FC0) and np.all(np.isnan(lse))


def test_capacity_plan_accepts_longer_page_indices(L, oracle):
    (hq, hkv, pool, nnz), (q, k, v), (qo, ip, ix, last), (ref_out, ref_lse) = _guard_setup(oracle)
    longer = np.concatenate([ix, np.full(7, 10 ** 6, np.int32)])  # junk past indptr[B]
    out, lse = PrefillRunner(L, 3, nnz, pool, hq, hkv, indices_capacity=True).run(
        q, k, v, qo, ip, longer, last)
    compare_decode(oracle, out, lse, ref_out, ref_lse)
    out, lse = PrefillRunner(L, 3, nnz, pool, hq, hkv).run(q, k, v, qo, ip, longer, last)
    assert np.all(np.isnan(lse))


def test_enqueue_rejections(L, oracle):
    # prefill.rs:2474-2505 (4-byte alignment, prefill.rs:3015-3029)
    import torch
    (hq, hkv, pool, nnz), (q, k, v), (qo, ip, ix, last), _ = _guard_setup(oracle)
    r = PrefillRunner(L, 3, nnz, pool, hq, hkv)
    dq, dk, dv = to_dev_bf16(q), to_dev_bf16(k), to_dev_bf16(v)
    dqo, dip, dix, dlast = (to_dev_i32(x) for x in (qo, ip, ix, last))
    with pytest.raises(L.EnqueueError) as e:
        r.run_dev(dq[:-1], dk, dv, dqo, dip, dix, dlast)
    assert e.value.variant == "LengthMismatch" and e.value.operand == "Q"
    with pytest.raises(L.EnqueueError) as e:
        r.run_dev(dq, dk, dv, dqo, dip, dix[:2], dlast)
    assert e.value.variant == "PageIndicesTooShort" and e.value.fields[:2] == (3, 2)
    with pytest.raises(L.EnqueueError) as e:
        r.run_dev(dq, dk, dv, dqo[:-1], dip, dix, dlast)
    assert e.value.variant == "LengthMismatch" and e.value.operand == "qo_indptr"
    big = nan_bf16(r.spec.output_numel + 8)
    with pytest.raises(L.EnqueueError) as e:
        r.run_dev(dq, dk, dv, dqo, dip, dix, dlast, out=big[1:1 + r.spec.output_numel])
    assert e.value.variant == "MisalignedBuffer" and e.value.operand == "O"
    torch.cuda.synchronize()


@pytest.mark.parametrize("tile_cols", [16, 64])
def test_prefill_graph_replays_match_eager(L, oracle, tile_cols):
    """gates/paged_prefill.rs:382-526: capture one prefill command, replay it
    with eager work and host synchronization between replays, and compare
    every replay with the eager result bit for bit."""
    import torch
    case = GOLDEN["paged_prefill"]["cases"][2]  # gqa4_reordered_reuse, as the reference's graph gate
    log(f"prefill graph replay tile_cols={tile_cols}")
    q, k, v = gate_inputs(oracle, case)
    B, nnz, pool, hq, hkv = (case[x] for x in ("batch", "nnz_qo", "pool", "hq", "hkv"))
    meta = (case["qo_indptr"], case["indptr"], case["indices"], case["last"])
    ref_out, ref_lse = oracle.prefill(oracle.prefill_spec(B, nnz, pool, hq, hkv), q, k, v, *meta)
    r = PrefillRunner(L, B, nnz, pool, hq, hkv, tile_cols=tile_cols)
    eager_o, eager_l = r.run(q, k, v, *meta)
    compare_decode(oracle, eager_o, eager_l, ref_out, ref_lse)
    ins = [to_dev_bf16(q), to_dev_bf16(k), to_dev_bf16(v)] + [to_dev_i32(m) for m in meta]
    out = nan_bf16(r.spec.output_numel)
    lse = torch.full((r.spec.lse_numel,), float("nan"), dtype=torch.float32, device="cuda")
    gq = L.GraphQueue(0, 1)
    b = gq.bindings(9)
    h = [b.bind_read(x) for x in ins] + [b.bind_read_write(out), b.bind_read_write(lse)]
    args = L.Bf16PagedPrefillArgs(*h[:7], h[7].write(), h[8].write())
    exec_ = gq.capture(b, lambda scope: r.plan.enqueue_into(scope, args)).instantiate()
    del ins
    for i in range(1, 4):
        out.fill_(float("nan"))
        lse.fill_(float("nan"))
        torch.cuda.synchronize()
        exec_.launch().wait()
        assert np.array_equal(bf16_host(out), eager_o), f"replay {i}"
        assert np.array_equal(lse.cpu().numpy(), eager_l), f"replay {i}"
    exec_.into_bindings()
