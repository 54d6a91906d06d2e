"""GPU parity of the long-tile paged prefill (LOOM_PAGED_PREFILL_LONG_TILE:
the wide tiles' 64 columns per workgroup with 32-token blocks, the query in
registers, BF16 softmax weights in the P·V product and Vᵀ staged transposed
in LDS), through the C ABI.  No reference counterpart: the reference runs one
warp per (row, head).  Checked against the oracle (within the attention
tolerance: the weights are rounded to BF16) on the reference's fixtures and
seeded shapes, against the 16-column algorithm on page-layout variants and
ragged request mixes, and on every device-guard outcome (the same sentinel
rows, byte for byte)."""
import sys

import numpy as np
import pytest

from gpu_util import PrefillRunner, compare_decode, seeded_normal_bf16
from test_gpu_prefill import GATE, SHAPES, ragged_meta
from test_gpu_prefill import gate_inputs
from test_gpu_prefill_wide import assert_close, guard_inputs, paged_pair

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


@pytest.mark.parametrize("case", GATE, ids=lambda c: c["name"])
def test_gate_fixtures_long(L, oracle, case):
    log(f"long prefill gate fixture {case['name']}")
    q, k, v = gate_inputs(oracle, case)
    s = oracle.prefill_spec(case["batch"], case["nnz_qo"], case["pool"], case["hq"], case["hkv"])
    meta = (case["qo_indptr"], case["indptr"], case["indices"], case["last"])
    ref_out, ref_lse = oracle.prefill(s, q, k, v, *meta)
    r = PrefillRunner(L, case["batch"], case["nnz_qo"], case["pool"], case["hq"], case["hkv"],
                      tile_cols="long")
    assert r.plan.algorithm == "long_tile"
    out, lse = r.run(q, k, v, *meta)
    log(f"  {compare_decode(oracle, out, lse, ref_out, ref_lse)}")


LONG_SHAPES = SHAPES + [
    ("gqa4_long_prompt", 16, 4, [300, 200], [700, 200]),
    # 16-row block counts odd and even, requests shorter than one 32-token
    # block, a prompt whose causal range crosses a 64-block index window
    ("gqa4_odd_blocks", 32, 8, [17, 33, 1, 50], [17, 49, 31, 1100]),
    ("mqa_window", 8, 1, [64, 3], [1200, 40]),
    ("mha_ragged", 8, 8, [5, 90, 16], [40, 90, 530]),
]


@pytest.mark.parametrize("shape", LONG_SHAPES, ids=lambda s: s[0])
def test_paged_shapes_long(L, oracle, shape):
    name, hq, hkv, qo_lens, kv_lens = shape
    log(f"long prefill {name}")
    rng = np.random.default_rng(sum(kv_lens) + 32)
    pool = sum((n + 15) // 16 for n in kv_lens) + 3
    qo, ip, ix, last = ragged_meta(rng, qo_lens, kv_lens, pool)
    B, nnz = len(qo_lens), int(qo[-1])
    q = seeded_normal_bf16(oracle, rng, nnz * hq * 128)
    k = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    ref_out, ref_lse = oracle.prefill(oracle.prefill_spec(B, nnz, pool, hq, hkv), q, k, v,
                                      qo, ip, ix, last)
    r = PrefillRunner(L, B, nnz, pool, hq, hkv, tile_cols="long")
    assert r.plan.algorithm == "long_tile"
    out, lse = r.run(q, k, v, qo, ip, ix, last)
    log(f"  {compare_decode(oracle, out, lse, ref_out, ref_lse)}")


@pytest.mark.parametrize("variant", ["hnd", "page32", "page64"])
def test_long_matches_row_tiles_on_page_variants(L, oracle, variant):
    log(f"long prefill {variant}")
    rng = np.random.default_rng(len(variant) + 3)
    B, hq, hkv = 3, 16, 4
    P = {"page32": 32, "page64": 64}.get(variant, 16)
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
    kw = {"kv_layout": "HND"} if variant == "hnd" else {"kv_page_size": P}
    res = paged_pair(L, B, nnz, pool, hq, hkv, q, k, v, qo, ip, ix, last, spec_kw=kw,
                     tile="long")
    assert not np.any(np.isnan(oracle.bf16_to_f32(res[0][0])))
    log(f"  vs 16-column: {assert_close(oracle, res)}")


@pytest.mark.parametrize("guard", ["bad_page_index", "qo_longer_than_kv", "bad_tail",
                                   "malformed_qo_range", "bad_global_qo"])
def test_long_guards_equal_narrow(L, oracle, guard):
    """The device guards keep the same sentinels as the 16-column algorithm."""
    log(f"long prefill guard {guard}")
    B, nnz, pool, hq, hkv, q, k, v, qo, ip, ix, last = guard_inputs(
        oracle, np.random.default_rng(12))
    qo, ip, ix, last = qo.copy(), ip.copy(), ix.copy(), last.copy()
    if guard == "bad_page_index":
        ix[ip[2] + 3] = pool + 5
    elif guard == "qo_longer_than_kv":
        ip[1] = ip[0] + 1
        last[0] = 4
    elif guard == "bad_tail":
        last[1] = 17
    elif guard == "malformed_qo_range":
        qo[2] = qo[1] - 1
    elif guard == "bad_global_qo":
        qo[-1] = nnz - 1
    res = paged_pair(L, B, nnz, pool, hq, hkv, q, k, v, qo, ip, ix, last, tile="long")
    log(f"  vs 16-column: {assert_close(oracle, res)}")
    nan_rows = int(np.isnan(oracle.bf16_to_f32(res[0][0])).reshape(nnz * hq, 128).all(1).sum())
    assert nan_rows > 0, "the guard case keeps some sentinels"


def test_plan_selection_and_rejections(L):
    """Long prompts default to the long tiles (BF16 and FP8 pages); ragged
    prefill rejects the long-tile flag; it needs four waves."""
    import ctypes as C
    prov = L.PrefillProvider.load(0)
    assert prov.plan_bf16_paged(L.Bf16PagedPrefillSpec(1, 4096, 256, 32, 8)).algorithm == \
        "long_tile"
    assert prov.plan_bf16_paged(L.Bf16PagedPrefillSpec(
        1, 4096, 256, 32, 8, kv_dtype="fp8_e4m3")).algorithm == "long_tile"
    assert prov.plan_bf16_paged(L.Bf16PagedPrefillSpec(1, 4, 8, 8, 8)).algorithm == "row_tile"
    # the long tiles from a 64-column grid of 256 workgroups (GQA4 32/8: 512
    # rows), on either page type
    for dt in ("bf16", "fp8_e4m3"):
        assert prov.plan_bf16_paged(L.Bf16PagedPrefillSpec(
            1, 512, 32, 32, 8, kv_dtype=dt)).algorithm == "long_tile"
        assert prov.plan_bf16_paged(L.Bf16PagedPrefillSpec(
            1, 256, 16, 32, 8, kv_dtype=dt)).algorithm == "row_tile"
    assert prov.plan_bf16_paged(L.Bf16PagedPrefillSpec(
        1, 64, 8, 32, 8, kv_dtype="fp8_e4m3"), tile_cols="long").algorithm == "long_tile"
    # two groups of four waves split the K/V blocks when the grid fits one
    # round of two workgroups per CU (1 x 512, 1 x 1024: one tile per wave;
    # 1 x 2048: two) or, with one tile per wave, the requests average 1024
    # rows or more (1 x 1536); four waves otherwise
    for dt in ("bf16", "fp8_e4m3"):
        for (B, n), threads in (((1, 512), 512), ((1, 1024), 512), ((1, 1536), 512),
                                ((2, 512), 256), ((1, 2048), 512), ((1, 3072), 256),
                                ((1, 4096), 256)):
            p = prov.plan_bf16_paged(L.Bf16PagedPrefillSpec(B, B * n, B * n // 16, 32, 8,
                                                            kv_dtype=dt))
            assert p.algorithm == "long_tile" and p.info.block_threads == threads, (dt, B, n)
    cases = [(L.Bf16PagedPrefillSpec(1, 64, 8, 32, 8), 8, "waves", "paged"),
             (L.Bf16RaggedPrefillSpec(1, 64, 64, 32, 8), 4, "flags", "ragged")]
    for spec, waves, field, kind in cases:
        fn = (L.lib().loom_prefill_provider_plan_bf16_paged_options if kind == "paged"
              else L.lib().loom_prefill_provider_plan_bf16_ragged)
        opt = L._ffi.PagedPrefillPlanOptions(waves, L.PLAN_PREFILL_TILE_LONG)
        out = C.c_void_p()
        with pytest.raises(L.PlanError) as e:
            L._call(fn, prov._p, C.byref(spec._c), C.byref(opt), C.byref(out))
        assert e.value.operand == field, (kind, waves, e.value)


def test_two_tiles_per_wave_with_a_guarded_request(L, oracle):
    """Grids large enough for two query tiles per wave (128 columns per
    workgroup): two 1100-row GQA4 prompts (32/8 heads), the second with an
    invalid page index.  The first equals the 16-column command within the
    oracle tolerance; the second keeps every sentinel, as there."""
    import torch
    log("long prefill, two tiles per wave, one guarded request")
    rng = np.random.default_rng(1100)
    hq, hkv = 32, 8
    qo_lens, kv_lens = [1100, 1100], [1300, 1100]
    pool = sum((n + 15) // 16 for n in kv_lens) + 2
    qo, ip, ix, last = ragged_meta(rng, qo_lens, kv_lens, pool)
    ix = ix.copy()
    ix[ip[1] + 40] = pool + 9
    B, nnz = 2, int(qo[-1])
    g = torch.Generator(device="cuda").manual_seed(11)
    q = torch.randn(nnz * hq * 128, device="cuda", generator=g).to(torch.bfloat16)
    k = torch.randn(pool * 16 * hkv * 128, device="cuda", generator=g).to(torch.bfloat16)
    v = torch.randn(pool * 16 * hkv * 128, device="cuda", generator=g).to(torch.bfloat16)
    res = paged_pair(L, B, nnz, pool, hq, hkv, q, k, v, qo, ip, ix, last, tile="long")
    log(f"  vs 16-column: {assert_close(oracle, res)}")
    o = oracle.bf16_to_f32(res[0][0]).reshape(nnz, hq * 128)
    assert np.all(np.isnan(o[1100:])) and not np.any(np.isnan(o[:1100]))


FP8_CASES = [  # (name, hq, hkv, qo_lens, kv_lens, spec keywords)
    ("ragged_mix", 16, 4, [70, 5, 130], [400, 90, 130], {}),
    ("odd_blocks", 32, 8, [17, 33, 1, 50], [17, 49, 31, 1100], {}),
    ("hnd", 16, 4, [70, 5, 130], [400, 90, 130], {"kv_layout": "HND"}),
    ("page32", 16, 4, [70, 5, 130], [400, 90, 130], {"kv_page_size": 32}),
    ("page64", 8, 1, [64, 3], [1200, 40], {"kv_page_size": 64}),
]


@pytest.mark.parametrize("case", FP8_CASES, ids=lambda c: c[0])
def test_fp8_pages_on_long_tiles(L, oracle, case):
    """FP8 E4M3 pages on the long tiles (regions of 64 one-byte dims loaded
    straight into LDS, K widened to BF16 after its fragment reads, V through
    the transposing byte read), with K and V scales: the same sentinels and,
    elsewhere, the 16-column FP8 command's result within the oracle
    tolerance (codes up to 0x44, |x| <= 3)."""
    import torch
    from test_gpu_fp8 import random_fp8
    name, hq, hkv, qo_lens, kv_lens, kw = case
    log(f"long prefill fp8 {name}")
    rng = np.random.default_rng(len(name) + 880)
    P = kw.get("kv_page_size", 16)
    pages = [(x + P - 1) // P for x in kv_lens]
    pool = sum(pages) + 2
    ip = np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)
    ix = rng.permutation(pool)[: ip[-1]].astype(np.int32)
    last = np.array([x - (p - 1) * P for x, p in zip(kv_lens, pages)], np.int32)
    qo = np.concatenate([[0], np.cumsum(qo_lens)]).astype(np.int32)
    B, nnz = len(qo_lens), int(qo[-1])
    q = seeded_normal_bf16(oracle, rng, nnz * hq * 128)
    n_kv = pool * P * hkv * 128
    k = torch.from_numpy(random_fp8(rng, n_kv, max_code=0x44)).to("cuda")
    v = torch.from_numpy(random_fp8(rng, n_kv, max_code=0x44)).to("cuda")
    res = paged_pair(L, B, nnz, pool, hq, hkv, q, k, v, qo, ip, ix, last,
                     spec_kw={"kv_dtype": "fp8_e4m3", **kw}, scales=[0.3, 0.7], tile="long")
    assert not np.any(np.isnan(oracle.bf16_to_f32(res[0][0])))
    log(f"  vs 16-column: {assert_close(oracle, res)}")


def test_fp8_two_tiles_per_wave_with_a_guarded_request(L, oracle):
    """The FP8 long tiles at two query tiles per wave: two 1100-row GQA4
    prompts, the second with an invalid page index."""
    import torch
    from test_gpu_fp8 import random_fp8
    log("long prefill fp8, two tiles per wave, one guarded request")
    rng = np.random.default_rng(1101)
    hq, hkv = 32, 8
    qo_lens, kv_lens = [1100, 1100], [1300, 1100]
    pool = sum((n + 15) // 16 for n in kv_lens) + 2
    qo, ip, ix, last = ragged_meta(rng, qo_lens, kv_lens, pool)
    ix = ix.copy()
    ix[ip[1] + 40] = pool + 9
    B, nnz = 2, int(qo[-1])
    q = seeded_normal_bf16(oracle, rng, nnz * hq * 128)
    k = torch.from_numpy(random_fp8(rng, pool * 16 * hkv * 128, max_code=0x44)).to("cuda")
    v = torch.from_numpy(random_fp8(rng, pool * 16 * hkv * 128, max_code=0x44)).to("cuda")
    res = paged_pair(L, B, nnz, pool, hq, hkv, q, k, v, qo, ip, ix, last,
                     spec_kw={"kv_dtype": "fp8_e4m3"}, scales=[0.3, 0.7], tile="long")
    log(f"  vs 16-column: {assert_close(oracle, res)}")
    o = oracle.bf16_to_f32(res[0][0]).reshape(nnz, hq * 128)
    assert np.all(np.isnan(o[1100:])) and not np.any(np.isnan(o[:1100]))


def test_fp8_two_groups_of_two_tiles_at_prompt_scale(L, oracle):
    """FP8 pages at two query tiles per wave and two wave groups (a 2048-row
    GQA4 prompt: 512 workgroups, one round of two per CU), with K and V
    scales: the 16-column FP8 command agrees within the oracle tolerance."""
    import torch
    from test_gpu_fp8 import random_fp8
    n = 2048
    log(f"long prefill fp8, two wave groups of two tiles, 1 x {n} rows")
    rng = np.random.default_rng(2048 + 8)
    hq, hkv = 32, 8
    pages = n // 16
    pool = pages + 3
    qo = np.array([0, n], np.int32)
    ip = np.array([0, pages], np.int32)
    ix = rng.permutation(pool)[:pages].astype(np.int32)
    last = np.array([16], np.int32)
    plan = L.PrefillProvider.load(0).plan_bf16_paged(
        L.Bf16PagedPrefillSpec(1, n, pool, hq, hkv, kv_dtype="fp8_e4m3"))
    assert plan.algorithm == "long_tile" and plan.info.block_threads == 512
    assert plan.info.row_tiles == n * 4 // 128, plan.info.row_tiles
    q = seeded_normal_bf16(oracle, rng, n * hq * 128)
    k = torch.from_numpy(random_fp8(rng, pool * 16 * hkv * 128, max_code=0x44)).to("cuda")
    v = torch.from_numpy(random_fp8(rng, pool * 16 * hkv * 128, max_code=0x44)).to("cuda")
    res = paged_pair(L, 1, n, pool, hq, hkv, q, k, v, qo, ip, ix, last,
                     spec_kw={"kv_dtype": "fp8_e4m3"}, scales=[0.3, 0.7], tile="long")
    assert not np.any(np.isnan(oracle.bf16_to_f32(res[0][0])))
    log(f"  vs 16-column: {assert_close(oracle, res)}")


@pytest.mark.parametrize("n", [1024, 1536, 2048])
def test_two_wave_groups_at_prompt_scale(L, oracle, n):
    """Long-tile plans of these prompts run two groups of four waves that
    split each tile's K/V blocks and merge in LDS (1024 rows: one tile per
    wave, a grid of one round, one page-index window; 1536: two windows;
    2048: two tiles per wave, a grid of one round); the same command on the
    16-column algorithm agrees within the attention tolerance."""
    log(f"long prefill two wave groups, 1 x {n} rows")
    import torch
    rng = np.random.default_rng(n)
    hq, hkv = 32, 8
    pages = (n + 15) // 16
    pool = pages + 5
    qo = np.array([0, n], np.int32)
    ip = np.array([0, pages], np.int32)
    ix = rng.permutation(pool)[:pages].astype(np.int32)
    last = np.array([n - (pages - 1) * 16], np.int32)
    g = torch.Generator(device="cuda").manual_seed(n)
    q, k, v = (torch.randn(x, device="cuda", generator=g).to(torch.bfloat16)
               for x in (n * hq * 128, pool * 16 * hkv * 128, pool * 16 * hkv * 128))
    plan = L.PrefillProvider.load(0).plan_bf16_paged(L.Bf16PagedPrefillSpec(1, n, pool, hq, hkv))
    assert plan.algorithm == "long_tile" and plan.info.block_threads == 512
    assert plan.info.row_tiles == n * 4 // (128 if n == 2048 else 64), plan.info.row_tiles
    res = paged_pair(L, 1, n, pool, hq, hkv, q, k, v, qo, ip, ix, last, tile="long")
    assert not np.any(np.isnan(oracle.bf16_to_f32(res[0][0])))
    log(f"  vs 16-column: {assert_close(oracle, res)}")
