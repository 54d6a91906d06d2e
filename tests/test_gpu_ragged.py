"""GPU parity of ragged causal prefill (contiguous K/V rows) through the C ABI
against the pinned CPU oracle: the reference's gate fixtures (three of them
bit-pinned by its zero-mismatch records), seeded ragged shapes over every
waves-per-workgroup variant, and the device guards of prefill.rs:102-138
(crates/loom-infer-validation/src/gates/ragged_prefill.rs)."""
import json
import os
import sys

import numpy as np
import pytest

from gpu_util import (RaggedRunner, bf16_host, compare_decode, nan_bf16, seeded_normal_bf16,
                      to_dev_bf16, to_dev_i32)

pytestmark = pytest.mark.gpu

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                     "reference_digests.json")))["ragged_prefill"]
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


def inputs(oracle, c):
    salt = int(c["salt"], 16)
    q = oracle.deterministic_bf16(c["nnz_qo"] * c["hq"] * 128, salt)
    k = oracle.deterministic_bf16(c["nnz_kv"] * c["hkv"] * 128, salt ^ 0x4B455900)
    v = oracle.deterministic_bf16(c["nnz_kv"] * c["hkv"] * 128, salt ^ 0x5641_4C55_4500)
    return q, k, v


@pytest.mark.parametrize("case", GOLDEN["cases"] + GOLDEN["timing_cases"], ids=lambda c: c["name"])
def test_gate_fixtures(L, oracle, case):
    log(f"ragged gate fixture {case['name']}")
    q, k, v = inputs(oracle, case)
    dims = (case["batch"], case["nnz_qo"], case["nnz_kv"], case["hq"], case["hkv"])
    ref_out, ref_lse = oracle.ragged(oracle.ragged_spec(*dims), q, k, v, case["qo_indptr"],
                                     case["kv_indptr"])
    for waves in (0,) + WAVES:
        r = RaggedRunner(L, *dims, waves=waves)
        out, lse = r.run(q, k, v, case["qo_indptr"], case["kv_indptr"])
        log(f"  waves={r.plan.info.waves} {compare_decode(oracle, out, lse, ref_out, ref_lse)}")


SHAPES = [
    # (name, hq, hkv, qo_lens, kv_lens)
    ("mha_full_causal", 8, 8, [40], [40]),
    ("gqa4_tile_edges", 16, 4, [1, 3, 4, 5, 8], [1, 17, 64, 100, 9]),
    ("gqa8_long", 32, 4, [2, 31], [300, 2000]),
    ("group5_odd", 10, 2, [3, 9, 1], [20, 9, 77]),
    ("mqa_rows", 8, 1, [1, 16, 64], [512, 128, 700]),
]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: s[0])
@pytest.mark.parametrize("waves", WAVES)
def test_ragged_shapes(L, oracle, shape, waves):
    name, hq, hkv, qo_lens, kv_lens = shape
    log(f"ragged {name} waves={waves}")
    rng = np.random.default_rng(sum(kv_lens) + 7 * waves)
    qo = np.concatenate([[0], np.cumsum(qo_lens)]).astype(np.int32)
    kv = np.concatenate([[0], np.cumsum(kv_lens)]).astype(np.int32)
    B, nnz_qo, nnz_kv = len(qo_lens), int(qo[-1]), int(kv[-1])
    q = seeded_normal_bf16(oracle, rng, nnz_qo * hq * 128)
    k = seeded_normal_bf16(oracle, rng, nnz_kv * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, nnz_kv * hkv * 128)
    ref_out, ref_lse = oracle.ragged(oracle.ragged_spec(B, nnz_qo, nnz_kv, hq, hkv), q, k, v,
                                     qo, kv)
    out, lse = RaggedRunner(L, B, nnz_qo, nnz_kv, hq, hkv, waves=waves).run(q, k, v, qo, kv)
    log(f"  {compare_decode(oracle, out, lse, ref_out, ref_lse)}")


def test_invalid_metadata_guard(L, oracle):
    # gates/ragged_prefill.rs:201-258: qo_indptr [0, 2, 1] over one query row
    # (the row's request ends past nnz_qo): every sentinel survives.
    r = RaggedRunner(L, 2, 1, 2, 1, 1)
    z = np.zeros(128, np.uint16)
    out, lse = r.run(z, np.zeros(256, np.uint16), np.zeros(256, np.uint16), [0, 2, 1], [0, 1, 2])
    assert np.all(out == 0x7FC0) and np.all(np.isnan(lse))


def _setup(oracle, qo_lens=(2, 3, 1), kv_lens=(20, 35, 9), hq=8, hkv=2, seed=31):
    rng = np.random.default_rng(seed)
    qo = np.concatenate([[0], np.cumsum(qo_lens)]).astype(np.int32)
    kv = np.concatenate([[0], np.cumsum(kv_lens)]).astype(np.int32)
    nnz_qo, nnz_kv = int(qo[-1]), int(kv[-1])
    q = seeded_normal_bf16(oracle, rng, nnz_qo * hq * 128)
    k = seeded_normal_bf16(oracle, rng, nnz_kv * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, nnz_kv * hkv * 128)
    return (len(qo_lens), nnz_qo, nnz_kv, hq, hkv), (q, k, v), qo, kv


def _rows_ref(oracle, dims, q, k, v, qo_r, kv_r, rows):
    """Oracle output of the rows `rows` computed as request (qo_r, kv_r) alone."""
    B, nnz_qo, nnz_kv, hq, hkv = dims
    (s0, s1), (k0, k1) = qo_r, kv_r
    q3 = q.reshape(nnz_qo, hq, 128)
    k3, v3 = k.reshape(nnz_kv, hkv, 128), v.reshape(nnz_kv, hkv, 128)
    spec = oracle.ragged_spec(1, s1 - s0, k1 - k0, hq, hkv)
    o, l = oracle.ragged(spec, q3[s0:s1].reshape(-1), k3[k0:k1].reshape(-1),
                         v3[k0:k1].reshape(-1), [0, s1 - s0], [0, k1 - k0])
    o = o.reshape(s1 - s0, hq * 128)
    l = l.reshape(s1 - s0, hq)
    return o[[x - s0 for x in rows]], l[[x - s0 for x in rows]]


def test_row_ownership_follows_the_reference_search(L, oracle):
    # prefill.rs:111-137 on metadata the host contract would reject: a row
    # belongs to the first request whose qo range ends after it.  qo = [0, 3,
    # 2, 6]: rows 0-2 -> request 0; rows 3-5 -> request 2 (range [2, 6), so
    # they are its query indices 1-3); request 1 ([3, 2)) owns nothing.
    dims, (q, k, v), _, _ = _setup(oracle, qo_lens=(3, 1, 2), kv_lens=(20, 10, 30))
    B, nnz_qo, nnz_kv, hq, hkv = dims
    qo = np.array([0, 3, 2, 6], np.int32)
    kv = np.array([0, 20, 30, 60], np.int32)
    out, lse = RaggedRunner(L, *dims).run(q, k, v, qo, kv)
    o = out.reshape(nnz_qo, hq * 128)
    l = lse.reshape(nnz_qo, hq)
    eo, el = _rows_ref(oracle, dims, q, k, v, (0, 3), (0, 20), [0, 1, 2])
    compare_decode(oracle, o[:3].reshape(-1), l[:3].reshape(-1), eo.reshape(-1), el.reshape(-1))
    eo, el = _rows_ref(oracle, dims, q, k, v, (2, 6), (30, 60), [3, 4, 5])
    compare_decode(oracle, o[3:].reshape(-1), l[3:].reshape(-1), eo.reshape(-1), el.reshape(-1))


def test_request_guards_keep_sentinels(L, oracle):
    dims, (q, k, v), qo, kv = _setup(oracle)
    B, nnz_qo, nnz_kv, hq, hkv = dims
    r = RaggedRunner(L, *dims)
    # request 1 with qo_len 3 > kv_len 2 (kv [0, 20, 22, 64]) keeps its rows;
    # requests 0 and 2 complete
    kv_bad = np.array([0, 20, 22, nnz_kv], np.int32)
    out, lse = r.run(q, k, v, qo, kv_bad)
    l = lse.reshape(nnz_qo, hq)
    assert np.all(np.isnan(l[2:5])) and np.all(np.isfinite(l[:2])) and np.all(np.isfinite(l[5:]))
    # global guard: kv_indptr[B] != nnz_kv writes nothing
    kv_g = kv.copy()
    kv_g[-1] -= 1
    out, lse = r.run(q, k, v, qo, kv_g)
    assert np.all(out == 0x7FC0) and np.all(np.isnan(lse))


def test_workspace_operand_is_optional_and_unused(L, oracle):
    import torch
    dims, (q, k, v), qo, kv = _setup(oracle)
    ref = oracle.ragged(oracle.ragged_spec(*dims), q, k, v, qo, kv)
    r = RaggedRunner(L, *dims)
    assert r.plan.workspace_required_numel == 0
    ws = torch.full((64,), 7.0, dtype=torch.float32, device="cuda")
    out, lse = r.run_dev(to_dev_bf16(q), to_dev_bf16(k), to_dev_bf16(v), to_dev_i32(qo),
                         to_dev_i32(kv), workspace=ws)
    compare_decode(oracle, bf16_host(out), lse.cpu().numpy(), *ref)
    assert torch.all(ws == 7.0)


def test_enqueue_rejections(L, oracle):
    dims, (q, k, v), qo, kv = _setup(oracle)
    r = RaggedRunner(L, *dims)
    dq, dk, dv, dqo, dkv = to_dev_bf16(q), to_dev_bf16(k), to_dev_bf16(v), to_dev_i32(qo), to_dev_i32(kv)
    with pytest.raises(L.EnqueueError) as e:
        r.run_dev(dq, dk[:-1], dv, dqo, dkv)
    assert e.value.variant == "LengthMismatch" and e.value.operand == "K"
    with pytest.raises(L.EnqueueError) as e:
        r.run_dev(dq, dk, dv, dqo, dkv[:-1])
    assert e.value.variant == "LengthMismatch" and e.value.operand == "kv_indptr"
    big = nan_bf16(r.spec.output_numel + 8)
    with pytest.raises(L.EnqueueError) as e:
        r.run_dev(dq, dk, dv, dqo, dkv, out=big[1:1 + r.spec.output_numel])
    assert e.value.variant == "MisalignedBuffer" and e.value.operand == "O"


def test_ragged_graph_replays_match_eager(L, oracle):
    import torch
    case = GOLDEN["cases"][2]
    q, k, v = inputs(oracle, case)
    dims = (case["batch"], case["nnz_qo"], case["nnz_kv"], case["hq"], case["hkv"])
    r = RaggedRunner(L, *dims)
    eager_o, eager_l = r.run(q, k, v, case["qo_indptr"], case["kv_indptr"])
    ins = [to_dev_bf16(q), to_dev_bf16(k), to_dev_bf16(v), to_dev_i32(case["qo_indptr"]),
           to_dev_i32(case["kv_indptr"])]
    out = nan_bf16(r.spec.output_numel)
    lse = torch.full((r.spec.lse_numel,), float("nan"), dtype=torch.float32, device="cuda")
    gq = L.GraphQueue(0, 1)
    b = gq.bindings(7)
    h = [b.bind_read(x) for x in ins] + [b.bind_read_write(out), b.bind_read_write(lse)]
    args = L.Bf16RaggedPrefillArgs(*h[:5], h[5].write(), h[6].write())
    exec_ = gq.capture(b, lambda scope: r.plan.enqueue_into(scope, args)).instantiate()
    for i in range(1, 4):
        out.fill_(float("nan"))
        lse.fill_(float("nan"))
        torch.cuda.synchronize()
        exec_.launch().wait()
        assert np.array_equal(bf16_host(out), eager_o), f"replay {i}"
        assert np.array_equal(lse.cpu().numpy(), eager_l), f"replay {i}"
    exec_.into_bindings()
