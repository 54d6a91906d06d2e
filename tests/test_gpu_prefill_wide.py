"""GPU parity of the wide-tile prefill algorithm (64 columns per workgroup,
K/V blocks staged through LDS for four waves), paged and ragged, through the
C ABI.  It has no reference counterpart: the reference runs one warp per
(row, head).  Checked against the oracle on the reference's fixtures and
seeded shapes, and against the 16-column algorithm (itself pinned to the
oracle) on long prompts, where the plan picks it by itself, on FP8, HND
and 64-row pages, and on every device-guard outcome: the same sentinel rows,
byte for byte, and the other rows within the oracle tolerance (the two
algorithms sum a column's blocks in different orders)."""
import sys

import numpy as np
import pytest

from gpu_util import (PrefillRunner, RaggedRunner, bf16_host, compare_decode, seeded_normal_bf16,
                      to_dev_bf16, to_dev_i32)
from test_gpu_prefill import GATE, SHAPES, gate_inputs, ragged_meta
from test_gpu_ragged import SHAPES as RAGGED_SHAPES

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def L():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import loom_infer_hip as L
    return L


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def paged_pair(L, B, nnz, pool, hq, hkv, q, k, v, qo, ip, ix, last, spec_kw=None, scales=None,
               tile=64):
    """(wide outputs, 16-column outputs) as raw host bits, same inputs."""
    import torch
    res = []
    for tc in (tile, 16):
        r = PrefillRunner(L, B, nnz, pool, hq, hkv)
        if spec_kw:
            r.spec = L.Bf16PagedPrefillSpec(B, nnz, pool, hq, hkv, **spec_kw)
        r.plan = r.provider.plan_bf16_paged(r.spec, tile_cols=tc)
        assert r.plan.algorithm == {64: "wide_tile", 16: "row_tile", "long": "long_tile"}[tc]
        dev = [x if isinstance(x, torch.Tensor) else to_dev_bf16(x) for x in (q, k, v)]
        out, lse = r.run_dev(*dev, *(to_dev_i32(x) for x in (qo, ip, ix, last)),
                             scales=None if scales is None else
                             torch.tensor(scales, dtype=torch.float32, device="cuda"))
        res.append((bf16_host(out), lse.view(torch.int32).cpu().numpy()))
    return res


def assert_close(oracle, res):
    """Same sentinel (NaN) positions bit for bit; elsewhere within the oracle
    tolerance of the 16-column result."""
    (o1, l1), (o2, l2) = res
    n1, n2 = np.isnan(oracle.bf16_to_f32(o1)), np.isnan(oracle.bf16_to_f32(o2))
    assert np.array_equal(n1, n2), "sentinel rows differ"
    assert np.array_equal(o1[n1], o2[n2])
    f1, f2 = l1.view(np.float32), l2.view(np.float32)
    m1 = np.isnan(f1)
    assert np.array_equal(m1, np.isnan(f2)) and np.array_equal(l1[m1], l2[m1])
    if (~n1).any():
        return compare_decode(oracle, o1[~n1], f1[~m1], o2[~n2], f2[~m1])
    return {}


@pytest.mark.parametrize("case", GATE, ids=lambda c: c["name"])
def test_gate_fixtures_wide(L, oracle, case):
    log(f"wide prefill gate fixture {case['name']}")
    q, k, v = gate_inputs(oracle, case)
    s = oracle.prefill_spec(case["batch"], case["nnz_qo"], case["pool"], case["hq"], case["hkv"])
    meta = (case["qo_indptr"], case["indptr"], case["indices"], case["last"])
    ref_out, ref_lse = oracle.prefill(s, q, k, v, *meta)
    r = PrefillRunner(L, case["batch"], case["nnz_qo"], case["pool"], case["hq"], case["hkv"],
                      tile_cols=64)
    assert r.plan.algorithm == "wide_tile"
    out, lse = r.run(q, k, v, *meta)
    log(f"  {compare_decode(oracle, out, lse, ref_out, ref_lse)}")


@pytest.mark.parametrize("shape", SHAPES + [("gqa4_long_prompt", 16, 4, [300, 200], [700, 200])],
                         ids=lambda s: s[0])
def test_paged_shapes_wide(L, oracle, shape):
    name, hq, hkv, qo_lens, kv_lens = shape
    log(f"wide prefill {name}")
    rng = np.random.default_rng(sum(kv_lens) + 64)
    pool = sum((n + 15) // 16 for n in kv_lens) + 3
    qo, ip, ix, last = ragged_meta(rng, qo_lens, kv_lens, pool)
    B, nnz = len(qo_lens), int(qo[-1])
    q = seeded_normal_bf16(oracle, rng, nnz * hq * 128)
    k = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    ref_out, ref_lse = oracle.prefill(oracle.prefill_spec(B, nnz, pool, hq, hkv), q, k, v,
                                      qo, ip, ix, last)
    out, lse = PrefillRunner(L, B, nnz, pool, hq, hkv, tile_cols=64).run(q, k, v, qo, ip, ix, last)
    log(f"  {compare_decode(oracle, out, lse, ref_out, ref_lse)}")


@pytest.mark.parametrize("shape", RAGGED_SHAPES, ids=lambda s: s[0])
def test_ragged_shapes_wide(L, oracle, shape):
    name, hq, hkv, qo_lens, kv_lens = shape
    log(f"wide ragged {name}")
    rng = np.random.default_rng(sum(kv_lens) + 65)
    qo = np.concatenate([[0], np.cumsum(qo_lens)]).astype(np.int32)
    kv = np.concatenate([[0], np.cumsum(kv_lens)]).astype(np.int32)
    B, nnz_qo, nnz_kv = len(qo_lens), int(qo[-1]), int(kv[-1])
    q = seeded_normal_bf16(oracle, rng, nnz_qo * hq * 128)
    k = seeded_normal_bf16(oracle, rng, nnz_kv * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, nnz_kv * hkv * 128)
    ref_out, ref_lse = oracle.ragged(oracle.ragged_spec(B, nnz_qo, nnz_kv, hq, hkv), q, k, v,
                                     qo, kv)
    r = RaggedRunner(L, B, nnz_qo, nnz_kv, hq, hkv, tile_cols=64)
    assert r.plan.algorithm == "wide_tile"
    out, lse = r.run(q, k, v, qo, kv)
    log(f"  {compare_decode(oracle, out, lse, ref_out, ref_lse)}")


@pytest.mark.parametrize("tile", [64, "long"], ids=["wide", "long"])
def test_long_prompt_matches_row_tiles(L, oracle, tile):
    """A 2048-row GQA4 prompt (Hq 32 / Hkv 8) over a longer cached prefix: the
    default plan is the long-tile one (BF16 pages); the wide and long plans
    equal the 16-column plan within the oracle tolerance with the same
    sentinels (they sum a column's blocks in different orders, and the long
    tiles round P to BF16, so not bit for bit), and the last query rows are
    checked against the oracle on a one-request slice."""
    import torch
    log("wide prefill long prompt")
    rng = np.random.default_rng(2048)
    B, hq, hkv, n, kvl = 1, 32, 8, 2048, 2560
    pool = (kvl + 15) // 16
    qo, ip, ix, last = ragged_meta(rng, [n], [kvl], pool)
    spec = L.Bf16PagedPrefillSpec(B, n, pool, hq, hkv)
    assert L.PrefillProvider.load(0).plan_bf16_paged(spec).algorithm == "long_tile"
    g = torch.Generator(device="cuda").manual_seed(7)
    q = torch.randn(n * hq * 128, device="cuda", generator=g).to(torch.bfloat16)
    k = torch.randn(pool * 16 * hkv * 128, device="cuda", generator=g).to(torch.bfloat16)
    v = torch.randn(pool * 16 * hkv * 128, device="cuda", generator=g).to(torch.bfloat16)
    res = paged_pair(L, B, n, pool, hq, hkv, q, k, v, qo, ip, ix, last, tile=tile)
    log(f"  {tile} vs 16-column: {assert_close(oracle, res)}")
    # oracle on the last 24 query rows (their causal ends are the largest)
    tail = 24
    qt = bf16_host(q)[(n - tail) * hq * 128:]
    qo_t = np.array([0, tail], np.int32)
    ref_out, ref_lse = oracle.prefill(oracle.prefill_spec(1, tail, pool, hq, hkv), qt,
                                      bf16_host(k), bf16_host(v), qo_t, ip, ix, last)
    o, l = res[0]
    log("  " + str(compare_decode(oracle, o[(n - tail) * hq * 128:],
                                  l.view(np.float32)[(n - tail) * hq:], ref_out, ref_lse)))


def test_fp8_pages_on_wide_tiles(L, oracle):
    """FP8 E4M3 pages on wide tiles (widened to BF16 as they are staged; the
    plan's default for long prompts is the long tiles, so they are forced
    here): the result matches the 16-column FP8 command within the oracle
    tolerance (codes up to 0x44, |x| <= 3, so outputs stay below 4 and one
    BF16 ulp is at most 1/64)."""
    import torch
    from test_gpu_fp8 import random_fp8
    log("wide prefill fp8")
    rng = np.random.default_rng(88)
    B, hq, hkv = 3, 16, 4
    qo_lens, kv_lens = [70, 5, 130], [400, 90, 130]
    pool = sum((x + 15) // 16 for x in kv_lens) + 2
    qo, ip, ix, last = ragged_meta(rng, qo_lens, kv_lens, pool)
    nnz = int(qo[-1])
    q = seeded_normal_bf16(oracle, rng, nnz * hq * 128)
    k = torch.from_numpy(random_fp8(rng, pool * 16 * hkv * 128, max_code=0x44)).to("cuda")
    v = torch.from_numpy(random_fp8(rng, pool * 16 * hkv * 128, max_code=0x44)).to("cuda")
    res = paged_pair(L, B, nnz, pool, hq, hkv, q, k, v, qo, ip, ix, last,
                     spec_kw={"kv_dtype": "fp8_e4m3"}, scales=[0.3, 0.7])
    assert not np.any(np.isnan(oracle.bf16_to_f32(res[0][0])))
    log(f"  vs 16-column: {assert_close(oracle, res)}")


@pytest.mark.parametrize("variant", ["hnd", "page64"])
def test_wide_matches_row_tiles_on_page_variants(L, oracle, variant):
    log(f"wide prefill {variant}")
    rng = np.random.default_rng(len(variant))
    B, hq, hkv = 3, 16, 4
    P = 64 if variant == "page64" else 16
    qo_lens, kv_lens = [70, 5, 130], [400, 90, 130]
    pages = [(x + P - 1) // P for x in kv_lens]
    pool = sum(pages) + 2
    ip = np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)
    ix = rng.permutation(pool)[: ip[-1]].astype(np.int32)
    last = np.array([x - (p - 1) * P for x, p in zip(kv_lens, pages)], np.int32)
    qo = np.concatenate([[0], np.cumsum(qo_lens)]).astype(np.int32)
    nnz = int(qo[-1])
    q = seeded_normal_bf16(oracle, rng, nnz * hq * 128)
    n_kv = pool * P * hkv * 128
    k = seeded_normal_bf16(oracle, rng, n_kv)
    v = seeded_normal_bf16(oracle, rng, n_kv)
    scales, kw = None, ({"kv_layout": "HND"} if variant == "hnd" else {"kv_page_size": 64})
    res = paged_pair(L, B, nnz, pool, hq, hkv, q, k, v, qo, ip, ix, last, spec_kw=kw,
                     scales=scales)
    assert not np.any(np.isnan(oracle.bf16_to_f32(res[0][0])))
    log(f"  vs 16-column: {assert_close(oracle, res)}")


def guard_inputs(oracle, rng, hq=16, hkv=4):
    qo_lens, kv_lens = [40, 7, 90], [100, 30, 200]
    pool = sum((n + 15) // 16 for n in kv_lens) + 2
    qo, ip, ix, last = ragged_meta(rng, qo_lens, kv_lens, pool)
    nnz = int(qo[-1])
    q = seeded_normal_bf16(oracle, rng, nnz * hq * 128)
    k = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    return 3, nnz, pool, hq, hkv, q, k, v, qo, ip, ix, last


@pytest.mark.parametrize("guard", ["bad_page_index", "qo_longer_than_kv", "bad_tail",
                                   "malformed_qo_range", "bad_global_qo"])
def test_wide_guards_equal_narrow(L, oracle, guard):
    """The device guards keep the same sentinels in both algorithms."""
    log(f"wide prefill guard {guard}")
    B, nnz, pool, hq, hkv, q, k, v, qo, ip, ix, last = guard_inputs(
        oracle, np.random.default_rng(11))
    qo, ip, ix, last = qo.copy(), ip.copy(), ix.copy(), last.copy()
    if guard == "bad_page_index":
        ix[ip[2] + 3] = pool + 5          # request 2 keeps its sentinels
    elif guard == "qo_longer_than_kv":
        ip[1] = ip[0] + 1                 # request 0: one page of 4 rows < its 40 query rows
        last[0] = 4
    elif guard == "bad_tail":
        last[1] = 17
    elif guard == "malformed_qo_range":
        qo[2] = qo[1] - 1                 # request 1's range is malformed
    elif guard == "bad_global_qo":
        qo[-1] = nnz - 1
    res = paged_pair(L, B, nnz, pool, hq, hkv, q, k, v, qo, ip, ix, last)
    log(f"  vs 16-column: {assert_close(oracle, res)}")
    nan_rows = int(np.isnan(oracle.bf16_to_f32(res[0][0])).reshape(nnz * hq, 128).all(1).sum())
    assert nan_rows > 0, "the guard case keeps some sentinels"
    log(f"  sentinel rows {nan_rows}")


@pytest.mark.parametrize("kind", ["paged", "ragged"])
def test_tile_flag_combinations_rejected(L, kind):
    """Planner rejections of prefill_tile_cols (paged_prefill.hip): both tile
    flags at once, and 64-column tiles with 8- or 16-wave workgroups (the wide
    algorithm runs four waves) are LOOM_PLAN_INVALID_OPTION naming the field."""
    import ctypes as C
    prov = L.PrefillProvider.load(0)
    if kind == "paged":
        spec = L.Bf16PagedPrefillSpec(1, 64, 8, 32, 8)
        fn = L.lib().loom_prefill_provider_plan_bf16_paged_options
    else:
        spec = L.Bf16RaggedPrefillSpec(1, 64, 64, 32, 8)
        fn = L.lib().loom_prefill_provider_plan_bf16_ragged
    both = L.PLAN_PREFILL_TILE_16 | L.PLAN_PREFILL_TILE_64
    for waves, flags, field in ((0, both, "flags"), (4, both, "flags"),
                                (8, L.PLAN_PREFILL_TILE_64, "waves"),
                                (16, L.PLAN_PREFILL_TILE_64, "waves")):
        opt = L._ffi.PagedPrefillPlanOptions(waves, flags)
        out = C.c_void_p()
        with pytest.raises(L.PlanError) as e:
            L._call(fn, prov._p, C.byref(spec._c), C.byref(opt), C.byref(out))
        assert e.value.code == 75 and e.value.operand == field, (waves, flags, e.value)
        assert not out.value
    # the valid single flags still plan
    for waves, flags in ((4, L.PLAN_PREFILL_TILE_64), (8, L.PLAN_PREFILL_TILE_16),
                         (16, L.PLAN_PREFILL_TILE_16)):
        opt = L._ffi.PagedPrefillPlanOptions(waves, flags)
        out = C.c_void_p()
        L._call(fn, prov._p, C.byref(spec._c), C.byref(opt), C.byref(out))
        assert out.value
        (L.lib().loom_paged_prefill_plan_free if kind == "paged"
         else L.lib().loom_ragged_prefill_plan_free)(out.value)
