"""GPU parity of paged decode (libloom_infer_hip.so through the C ABI) against
the pinned CPU oracle, on the reference's gate fixtures, seeded BASELINE-shaped
workloads and the reference's negative cases."""
import json
import os
import sys
import zlib

import numpy as np
import pytest

from gpu_util import (DecodeRunner, bf16_host, compare_decode, nan_bf16, ragged_table,
                      seeded_normal_bf16, to_dev_bf16, to_dev_i32)

pytestmark = pytest.mark.gpu

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                     "reference_digests.json")))


@pytest.fixture(scope="module")
def L():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import loom_infer_hip as L
    return L


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("case", GOLDEN["paged_decode"]["cases"], ids=lambda c: c["name"])
def test_gate_fixtures(L, oracle, case):
    # crates/loom-infer-validation/src/gates/paged_batch_decode.rs:316-358
    log(f"decode gate fixture {case['name']}")
    salt = int(case["salt"], 16)
    B, pool, hq, hkv = case["batch"], case["pool"], case["hq"], case["hkv"]
    q = oracle.deterministic_bf16(B * hq * 128, salt)
    k = oracle.deterministic_bf16(pool * 16 * hkv * 128, salt ^ 0x4B455900)
    v = oracle.deterministic_bf16(pool * 16 * hkv * 128, salt ^ 0x5641_4C55_4500)
    s = oracle.paged_spec(B, pool, hq, hkv)
    ref_out, ref_lse = oracle.paged_decode(s, q, k, v, case["indptr"], case["indices"],
                                           case["last"])
    # default plan, one team (every request finished in place), and a few teams
    # (requests split across page ranges, merged by the second kernel)
    for teams in (0, 1, 3):
        r = DecodeRunner(L, B, pool, hq, hkv, teams=teams)
        out, lse = r.run(q, k, v, case["indptr"], case["indices"], case["last"])
        stats = compare_decode(oracle, out, lse, ref_out, ref_lse)
        log(f"  teams={r.plan.info.teams} {stats}")


SHAPES = [
    # (name, B, hq, hkv, lens, teams); teams 0 = the device default
    ("mha_c1_like", 1, 32, 32, [1024], 0),
    ("gqa4_ragged", 6, 32, 8, [1, 15, 16, 17, 700, 2049], 0),
    ("gqa4_ragged_teams7", 6, 32, 8, [1, 15, 16, 17, 700, 2049], 7),
    ("gqa4_ragged_teams1", 5, 32, 8, [3000, 33, 4097, 1, 64], 1),
    ("gqa4_ragged_teams64", 5, 32, 8, [3000, 33, 4097, 1, 64], 64),
    ("gqa8_long", 1, 64, 8, [8192], 0),
    ("mqa_group8", 3, 8, 1, [16, 23, 48], 0),
    ("group16_two_tiles", 2, 16, 1, [300, 77], 0),
    ("group3", 3, 6, 2, [5, 40, 129], 4),
    ("group2", 2, 4, 2, [33, 1000], 0),
    # small page tables: the direct kernel (one workgroup per request/kv-head/tile)
    ("direct_gqa4", 5, 32, 8, [1, 15, 17, 100, 260], 0),
    ("direct_group16", 3, 16, 1, [33, 200, 7], 0),
    ("direct_mha", 2, 8, 8, [64, 190], 0),
    ("direct8_gqa4", 3, 32, 8, [500, 33, 700], 0),
    ("direct16_mha", 2, 8, 8, [900, 1000], 0),
    ("direct16_group2", 2, 4, 2, [700, 1200], 0),
    ("direct8_group16", 2, 16, 1, [1500, 17], 0),
    # more requests than the workgroup keeps in LDS: the block-wise search
    ("batch1100_small", 1100, 4, 1, [1 + (i * 37) % 70 for i in range(1100)], 0),
    ("batch1100_teams13", 1100, 8, 2, [1 + (i * 53) % 90 for i in range(1100)], 13),
]


@pytest.mark.parametrize("name,B,hq,hkv,lens,teams", SHAPES, ids=[s[0] for s in SHAPES])
def test_seeded_shapes(L, oracle, name, B, hq, hkv, lens, teams):
    log(f"decode seeded shape {name} B={B} hq={hq} hkv={hkv} teams={teams}")
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    pool = sum((x + 15) // 16 for x in lens) + 3
    indptr, indices, last = ragged_table(rng, lens, pool)
    q = seeded_normal_bf16(oracle, rng, B * hq * 128)
    k = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    s = oracle.paged_spec(B, pool, hq, hkv)
    ref_out, ref_lse = oracle.paged_decode(s, q, k, v, indptr, indices, last)
    r = DecodeRunner(L, B, pool, hq, hkv, teams=teams)
    out, lse = r.run(q, k, v, indptr, indices, last)
    log(f"  plan {r.plan.algorithm} teams={r.plan.info.teams} tile={r.plan.info.group_tile}x"
        f"{r.plan.info.group_tiles} {compare_decode(oracle, out, lse, ref_out, ref_lse)}")
    # a second call over the previous call's workspace contents is identical
    out2, lse2 = r.run(q, k, v, indptr, indices, last)
    assert np.array_equal(out2, out) and np.array_equal(lse2, lse)


def test_closed_form_zero_query(L, oracle):
    # Q = 0: O = mean(V) exactly representable inputs, LSE = log2(kv_len)
    B, hq, hkv, pool = 2, 8, 2, 12
    lens = [16, 160]
    rng = np.random.default_rng(3)
    indptr, indices, last = ragged_table(rng, lens, pool)
    q = np.zeros(B * hq * 128, np.uint16)
    k = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    v = oracle.bf16_from_f32(rng.integers(-4, 5, pool * 16 * hkv * 128).astype(np.float32))
    r = DecodeRunner(L, B, pool, hq, hkv, teams=3)
    out, lse = r.run(q, k, v, indptr, indices, last)
    np.testing.assert_allclose(lse, np.repeat(np.log2(lens), hq), atol=2e-6)
    ref_out, _ = oracle.paged_decode(oracle.paged_spec(B, pool, hq, hkv), q, k, v, indptr,
                                     indices, last)
    assert np.array_equal(out, ref_out)


def test_invalid_page_guard_preserves_sentinels(L):
    # crates/loom-infer-validation/src/gates/paged_batch_decode.rs:224-308
    torch = pytest.importorskip("torch")
    r = DecodeRunner(L, 2, 2, 4, 2)
    z = torch.zeros(r.spec.kv_pages_numel, dtype=torch.bfloat16, device="cuda")
    q = torch.zeros(r.spec.query_numel, dtype=torch.bfloat16, device="cuda")
    out, lse = r.run_dev(q, z, z.clone(), to_dev_i32([0, 1, 2]), to_dev_i32([0, 2]),
                         to_dev_i32([16, 16]))
    o = out.float().cpu().numpy()
    l = lse.cpu().numpy()
    assert np.all(o[:4 * 128] == 0.0) and np.all(l[:4] == 4.0)
    assert np.all(np.isnan(o[4 * 128:])) and np.all(np.isnan(l[4:]))


@pytest.mark.parametrize("teams", [8, 0], ids=["balanced", "direct"])
def test_invalid_page_in_split_request(L, oracle, teams):
    """An invalid page inside a request split over several teams leaves that
    request's sentinels and completes the others; the next valid call over the
    poisoned workspace is correct."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(5)
    lens = [600, 300]
    pool = 64
    indptr, indices, last = ragged_table(rng, lens, pool)
    bad = indices.copy()
    bad[20] = pool + 5  # inside request 0 (38 pages), in the second of 8 teams
    B, hq, hkv = 2, 8, 2
    q = seeded_normal_bf16(oracle, rng, B * hq * 128)
    k = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    r = DecodeRunner(L, B, pool, hq, hkv, teams=teams)
    out, lse = r.run(q, k, v, indptr, bad, last)
    o = oracle.bf16_to_f32(out).reshape(B, hq * 128)
    assert np.all(np.isnan(o[0])) and np.all(np.isnan(lse[:hq]))
    ref_out, ref_lse = oracle.paged_decode(oracle.paged_spec(B, pool, hq, hkv), q, k, v,
                                           indptr, indices, last)
    compare_decode(oracle, out.reshape(B, -1)[1], lse[hq:], ref_out.reshape(B, -1)[1],
                   ref_lse[hq:])
    out2, lse2 = r.run(q, k, v, indptr, indices, last)
    compare_decode(oracle, out2, lse2, ref_out, ref_lse)


@pytest.mark.parametrize("lens,teams", [([100, 50, 300, 20, 64], 0), ([100, 50, 300, 20, 64], 1),
                                        ([100, 50, 300, 20, 64], 5), ([20, 5, 40, 3, 30], 0),
                                        ([500, 400, 300, 200], 0)],
                         ids=["balanced", "one_team", "five_teams", "direct", "split_direct"])
def test_invalid_request_leaves_sentinels(L, oracle, lens, teams):
    """Requests failing the per-request guard (decode.rs:430-478: last page
    length outside 1..16) contribute no pages; the others are computed as
    usual, also when the pages around them are split over teams, and on the
    direct (small page table) kernel."""
    rng = np.random.default_rng(8)
    B, hq, hkv = len(lens), 8, 2
    pool = sum((x + 15) // 16 for x in lens) + 2
    indptr, indices, last = ragged_table(rng, lens, pool)
    q = seeded_normal_bf16(oracle, rng, B * hq * 128)
    k = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    ref_out, ref_lse = oracle.paged_decode(oracle.paged_spec(B, pool, hq, hkv), q, k, v,
                                           indptr, indices, last)
    bad_last = np.array(last, copy=True)
    bad_last[1] = 0
    bad_last[3] = 17
    r = DecodeRunner(L, B, pool, hq, hkv, teams=teams)
    if len(lens) == 4:  # each request over two 4-wave workgroups, states merged
        assert r.plan.algorithm == "direct" and r.plan.info.teams == 2
    out, lse = r.run(q, k, v, indptr, indices, bad_last)
    o = oracle.bf16_to_f32(out).reshape(B, hq * 128)
    l = lse.reshape(B, hq)
    for rq in (1, 3):
        assert np.all(np.isnan(o[rq])) and np.all(np.isnan(l[rq]))
    for rq in range(0, B, 2):
        compare_decode(oracle, out.reshape(B, -1)[rq], l[rq], ref_out.reshape(B, -1)[rq],
                       ref_lse.reshape(B, hq)[rq])


def test_global_indptr_guard(L):
    torch = pytest.importorskip("torch")
    r = DecodeRunner(L, 2, 4, 4, 2)
    z = torch.zeros(r.spec.kv_pages_numel, dtype=torch.bfloat16, device="cuda")
    q = torch.zeros(r.spec.query_numel, dtype=torch.bfloat16, device="cuda")
    # indptr[B] != len(page_indices): every request keeps its sentinels
    out, lse = r.run_dev(q, z, z.clone(), to_dev_i32([0, 1, 2]), to_dev_i32([0, 1, 2]),
                         to_dev_i32([16, 16]))
    assert torch.isnan(out.float()).all() and torch.isnan(lse).all()


def test_global_indptr_guard_split_direct_then_valid(L, oracle):
    """The global guard on a split direct plan (every split workgroup poisons
    its state and still counts itself in, so the queue's arrival counters
    return to zero): all sentinels kept, then a valid call on the same queue
    matches the oracle, twice."""
    rng = np.random.default_rng(21)
    lens = [1000, 700]
    B, hq, hkv = 2, 8, 2
    pool = sum((x + 15) // 16 for x in lens) + 4
    indptr, indices, last = ragged_table(rng, lens, pool)
    q = seeded_normal_bf16(oracle, rng, B * hq * 128)
    k = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    r = DecodeRunner(L, B, pool, hq, hkv)
    assert r.plan.algorithm == "direct" and r.plan.info.teams > 1
    bad_ptr = indptr.copy()
    bad_ptr[0] = 1
    out, lse = r.run(q, k, v, bad_ptr, indices, last)
    assert np.all(np.isnan(oracle.bf16_to_f32(out))) and np.all(np.isnan(lse))
    ref_out, ref_lse = oracle.paged_decode(oracle.paged_spec(B, pool, hq, hkv), q, k, v,
                                           indptr, indices, last)
    for _ in range(2):
        out, lse = r.run(q, k, v, indptr, indices, last)
        compare_decode(oracle, out, lse, ref_out, ref_lse)


def test_short_indptr_rejected_before_submission(L):
    # crates/loom-infer-validation/src/gates/paged_batch_decode.rs:150-222
    torch = pytest.importorskip("torch")
    r = DecodeRunner(L, 2, 2, 4, 2)
    s = r.spec
    z = torch.zeros(s.kv_pages_numel, dtype=torch.bfloat16, device="cuda")
    q = torch.zeros(s.query_numel, dtype=torch.bfloat16, device="cuda")
    out = torch.zeros(s.output_numel, dtype=torch.bfloat16, device="cuda")
    lse = torch.zeros(s.lse_numel, dtype=torch.float32, device="cuda")
    b, h = r.bindings(q, z, z.clone(), to_dev_i32([0, 1]), to_dev_i32([0, 0]),
                      to_dev_i32([16, 16]), out, lse)
    scope = r.queue.begin(b)
    with pytest.raises(L.EnqueueError) as e:
        r.plan.enqueue_into(scope, r.args(h))
    assert (e.value.variant, e.value.operand, e.value.fields[:2]) == (
        "LengthMismatch", "page_indptr", (3, 2))
    comp = scope.finish()
    assert comp.submitted() == 0
    comp.wait()


def test_command_runtime_checks(L):
    torch = pytest.importorskip("torch")
    r = DecodeRunner(L, 1, 1, 1, 1)
    s = r.spec
    x = torch.zeros(s.kv_pages_numel, dtype=torch.bfloat16, device="cuda")
    b = r.queue.bindings(2)
    h = b.bind_read_write(x)
    with pytest.raises(L.CommandError) as e:
        b.bind_read(x)  # overlaps a read-write lease
    assert e.value.variant == "AliasedBinding"
    b.bind_read(torch.zeros(4, dtype=torch.int32, device="cuda"))
    with pytest.raises(L.CommandError) as e:
        b.bind_read(torch.zeros(4, dtype=torch.int32, device="cuda"))
    assert e.value.variant == "BindingCapacityExceeded"
    with pytest.raises(L.CommandError) as e:
        b.bind_read(torch.zeros(4, dtype=torch.int32))  # host memory
    assert e.value.variant in ("BufferContextMismatch", "BindingCapacityExceeded")
    assert b.take_read_write(h) is x
    with pytest.raises(L.CommandError) as e:
        b.take_read_write(h)
    assert e.value.variant == "BindingSlotVacant"
    other = r.queue.bindings(1)
    scope = r.queue.begin(other)
    with pytest.raises(L.CommandError) as e:
        r.queue.begin(r.queue.bindings(1))  # one live scope per queue (Rust's &mut)
    assert e.value.variant == "ScopeActive"
    comp = scope.finish()
    comp.wait()


def test_full_c3_shape_every_request(L, oracle):
    """BASELINE config 3 at full size (64 requests, ragged 512..8192, GQA4, pool
    65536, the default balanced split-KV plan): every request and every query
    head against the oracle (the pages the batch uses, gathered in table
    order), the reference gate's protocol
    (crates/loom-infer-validation/src/gates/paged_batch_decode.rs:28-148)."""
    torch = pytest.importorskip("torch")
    log("decode full C3 shape, all 64 requests")
    rng = np.random.default_rng(0)
    B, hq, hkv, pool = 64, 32, 8, 65536
    lens = rng.integers(512, 8193, size=B)
    pages = (lens + 15) // 16
    indptr = np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)
    indices = rng.permutation(pool)[: indptr[-1]].astype(np.int32)
    last = (lens - (pages - 1) * 16).astype(np.int32)
    g = torch.Generator(device="cuda")
    g.manual_seed(0)
    q = torch.randn(B * hq * 128, generator=g, device="cuda").to(torch.bfloat16)
    k = torch.randn(pool * 16 * hkv * 128, generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn(pool * 16 * hkv * 128, generator=g, device="cuda").to(torch.bfloat16)
    r = DecodeRunner(L, B, pool, hq, hkv)
    assert r.plan.algorithm == "balanced_split_kv"
    out, lse = r.run_dev(q, k, v, to_dev_i32(indptr), to_dev_i32(indices), to_dev_i32(last))
    out_h, lse_h = bf16_host(out), lse.cpu().numpy()
    # the compact pool: the used pages in table order, so page i of the batch
    # is compact page i
    idx = torch.from_numpy(indices.astype(np.int64)).cuda()
    kh = bf16_host(k.view(pool, -1).index_select(0, idx).reshape(-1))
    vh = bf16_host(v.view(pool, -1).index_select(0, idx).reshape(-1))
    n = int(indptr[-1])
    s = oracle.paged_spec(B, n, hq, hkv)
    ref_o, ref_l = oracle.paged_decode_parallel(s, bf16_host(q), kh, vh, indptr,
                                                np.arange(n, dtype=np.int32), last)
    st = compare_decode(oracle, out_h, lse_h, ref_o, ref_l)
    log(f"  64 requests, {n} pages, teams={r.plan.info.teams}: {st}")


def test_plan_selection_and_rejections(L):
    """Planner behaviour (the reference's algorithm-selection test,
    decode.rs:1657-1698, for this build's two algorithms)."""
    prov = L.DecodeProvider.load(0)
    small = L.Bf16PagedBatchDecodeSpec(4, 8, 16, 4, 128, 16)
    p = prov.plan_bf16_paged_batch(small)
    assert p.algorithm == "direct" and p.info.grid_blocks == 4 * 4
    assert p.info.block_threads == 256
    mid = L.Bf16PagedBatchDecodeSpec(4, 60, 8, 8, 128, 16)
    p = prov.plan_bf16_paged_batch(mid)
    assert p.algorithm == "direct" and p.info.block_threads == 1024  # 16 waves, 1-head tiles
    assert p.info.teams == 0 and p.info.grid_blocks == 4 * 8
    p = prov.plan_bf16_paged_batch(L.Bf16PagedBatchDecodeSpec(4, 60, 32, 8, 128, 16))
    assert p.algorithm == "direct" and p.info.block_threads == 512
    # long requests over few workgroups: each request's blocks split over
    # 2-8 workgroups of 4 waves (teams = the split count), states merged by a
    # second kernel
    p = prov.plan_bf16_paged_batch(L.Bf16PagedBatchDecodeSpec(2, 100, 8, 8, 128, 16))
    assert p.algorithm == "direct" and p.info.teams == 4 and p.info.block_threads == 256
    assert p.info.grid_blocks == 2 * 8 * 4 and p.info.state_slots == 4 * 2
    assert p.info.workspace_bytes == 4 * 2 * 8 * 132 * 4
    c1 = prov.plan_bf16_paged_batch(L.Bf16PagedBatchDecodeSpec(1, 128, 32, 32, 128, 16))
    assert c1.algorithm == "direct" and c1.info.teams == 8 and c1.info.grid_blocks == 32 * 8
    p = prov.plan_bf16_paged_batch(L.Bf16PagedBatchDecodeSpec(2, 129, 32, 8, 128, 16))
    assert p.algorithm == "balanced_split_kv"
    p = prov.plan_bf16_paged_batch(small, teams=3)
    assert p.algorithm == "balanced_split_kv" and p.info.teams == 3
    big = L.Bf16PagedBatchDecodeSpec(64, 65536, 32, 8, 128, 16)
    p = prov.plan_bf16_paged_batch(big)
    info = p.info
    assert p.algorithm == "balanced_split_kv" and info.group_tile == 4 and info.group_tiles == 1
    # one wave per SIMD slot: teams x members waves fill the grid's XCD slices
    assert info.teams * 8 <= info.grid_blocks * 4 and info.grid_blocks % 8 == 0
    assert info.state_slots == info.teams + 64
    assert info.workspace_bytes == info.header_bytes + info.state_slots * 32 * 132 * 4
    grp = L.Bf16PagedBatchDecodeSpec(2, 64, 48, 2, 128, 16)  # group 24: 8-wide tiles x 3
    p = prov.plan_bf16_paged_batch(grp, teams=5)
    assert (p.info.group_tile, p.info.group_tiles) == (8, 3)
    with pytest.raises(L.PlanError) as e:
        prov.plan_bf16_paged_batch(big, max_total_pages=63)  # fewer pages than requests
    assert e.value.variant == "InvalidOption"
    huge = L.Bf16PagedBatchDecodeSpec(65537, 65537, 8, 8, 128, 16)
    with pytest.raises(L.PlanError) as e:
        prov.plan_bf16_paged_batch(huge)
    assert e.value.variant == "StateCountOutOfRange"


@pytest.mark.parametrize("teams", [0, 4], ids=["direct", "balanced"])
def test_enqueue_rejections_submit_nothing(L, teams):
    """Exact operand lengths, page_indices bounds and 4-byte alignment are
    checked before anything is submitted (decode.rs:1216-1251)."""
    torch = pytest.importorskip("torch")
    B, pool, hq, hkv = 2, 8, 8, 2
    r = DecodeRunner(L, B, pool, hq, hkv, teams=teams)
    s = r.spec
    dev = "cuda"

    def bufs():
        return dict(q=torch.zeros(s.query_numel, dtype=torch.bfloat16, device=dev),
                    k=torch.zeros(s.kv_pages_numel, dtype=torch.bfloat16, device=dev),
                    v=torch.zeros(s.kv_pages_numel, dtype=torch.bfloat16, device=dev),
                    ip=to_dev_i32([0, 1, 2]), ix=to_dev_i32([0, 1]), ln=to_dev_i32([16, 16]),
                    o=torch.zeros(s.output_numel, dtype=torch.bfloat16, device=dev),
                    l=torch.zeros(s.lse_numel, dtype=torch.float32, device=dev))

    def attempt(**over):
        t = bufs()
        t.update(over)
        b, h = r.bindings(t["q"], t["k"], t["v"], t["ip"], t["ix"], t["ln"], t["o"], t["l"])
        scope = r.queue.begin(b)
        try:
            with pytest.raises(L.EnqueueError) as e:
                r.plan.enqueue_into(scope, r.args(h))
        finally:
            comp = scope.finish()
            assert comp.submitted() == 0
            comp.wait()
        return e.value

    e = attempt(q=torch.zeros(s.query_numel + 8, dtype=torch.bfloat16, device=dev))
    assert (e.variant, e.operand) == ("LengthMismatch", "Q")
    e = attempt(ln=to_dev_i32([16]))
    assert (e.variant, e.operand) == ("LengthMismatch", "last_page_len")
    e = attempt(l=torch.zeros(s.lse_numel + 1, dtype=torch.float32, device=dev))
    assert (e.variant, e.operand) == ("LengthMismatch", "LSE")
    e = attempt(ix=to_dev_i32([0]))
    assert e.variant == "PageIndicesTooShort"
    e = attempt(ix=to_dev_i32(list(range(pool + 1))))
    assert e.variant == "PageIndicesTooLong"
    q2 = torch.zeros(s.query_numel + 8, dtype=torch.bfloat16, device=dev)[1:1 + s.query_numel]
    e = attempt(q=q2)
    assert (e.variant, e.operand) == ("MisalignedBuffer", "Q")


def test_max_batch_65536(L, oracle):
    """The largest admitted batch (65536 requests, 256 scan blocks): ragged
    1..3-page requests, MQA 2/1 heads, teams 0 and 97, against the oracle."""
    log("decode max batch 65536")
    rng = np.random.default_rng(65536)
    B, hq, hkv = 65536, 2, 1
    lens = rng.integers(1, 49, size=B)
    pool = int(sum((x + 15) // 16 for x in lens)) + 7
    indptr, indices, last = ragged_table(rng, list(lens), pool)
    q = seeded_normal_bf16(oracle, rng, B * hq * 128)
    k = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    ref_o, ref_l = oracle.paged_decode(oracle.paged_spec(B, pool, hq, hkv), q, k, v, indptr,
                                       indices, last)
    for teams in (0, 97):
        r = DecodeRunner(L, B, pool, hq, hkv, teams=teams)
        out, lse = r.run(q, k, v, indptr, indices, last)
        log(f"  teams={r.plan.info.teams} {compare_decode(oracle, out, lse, ref_o, ref_l)}")
