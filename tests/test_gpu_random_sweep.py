"""Seeded random sweeps of paged decode and RoPE + append shapes on the GPU
against the oracle: batch sizes, group sizes, ragged lengths, pool slack and
planner options drawn per case, so the plan choices (direct, split direct,
balanced split-KV; small and chunk-validated append) and their boundaries are
crossed in many combinations the hand-written cases do not name."""
import sys

import numpy as np
import pytest

from gpu_util import DecodeRunner, compare_decode, ragged_table, seeded_normal_bf16
from test_gpu_append import AppendRunner, check_rope

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


def decode_case(seed):
    rng = np.random.default_rng(1000 + seed)
    group = int(rng.choice([1, 2, 3, 4, 8]))
    hkv = int(rng.choice([1, 2, 4, 8]))
    B = int(rng.integers(1, 13))
    long = rng.random() < 0.5
    lens = rng.integers(1, 3001 if long else 200, size=B).tolist()
    slack = int(rng.integers(0, 21))
    teams = 0 if rng.random() < 0.5 else int(rng.integers(1, 41))
    return rng, B, group * hkv, hkv, lens, slack, teams


@pytest.mark.parametrize("seed", range(24))
def test_decode_random_shapes(L, oracle, seed):
    rng, B, hq, hkv, lens, slack, teams = decode_case(seed)
    pool = sum((x + 15) // 16 for x in lens) + slack
    log(f"decode sweep {seed}: B={B} hq={hq} hkv={hkv} pool={pool} teams={teams} "
        f"max_len={max(lens)}")
    indptr, indices, last = ragged_table(rng, lens, pool)
    q = seeded_normal_bf16(oracle, rng, B * hq * 128)
    k = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    ref = oracle.paged_decode(oracle.paged_spec(B, pool, hq, hkv), q, k, v, indptr, indices, last)
    r = DecodeRunner(L, B, pool, hq, hkv, teams=teams)
    out, lse = r.run(q, k, v, indptr, indices, last)
    log(f"  plan {r.plan.algorithm} teams={r.plan.info.teams} "
        f"{compare_decode(oracle, out, lse, *ref)}")
    out2, lse2 = r.run(q, k, v, indptr, indices, last)
    assert np.array_equal(out2, out) and np.array_equal(lse2, lse)


@pytest.mark.parametrize("seed", range(16))
def test_append_random_shapes(L, oracle, seed):
    rng = np.random.default_rng(2000 + seed)
    hkv = int(rng.choice([1, 2, 4, 8]))
    hq = hkv * int(rng.choice([1, 2, 4]))
    B = int(rng.integers(1, 9))
    lens = rng.integers(1, 600, size=B)
    T = int(min(rng.choice([1, 5, 40, 64, 65, 130, 300]), int(lens.sum())))
    pages = (lens + 15) // 16
    pool = int(pages.sum()) + int(rng.integers(0, 9))
    log(f"append sweep {seed}: B={B} hq={hq} hkv={hkv} T={T} pool={pool}")
    indptr = np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)
    indices = rng.permutation(pool)[: indptr[-1]].astype(np.int32)
    last = (lens - (pages - 1) * 16).astype(np.int32)
    flat = rng.choice(int(lens.sum()), size=T, replace=False)
    starts = np.concatenate([[0], np.cumsum(lens)])
    bi = (np.searchsorted(starts, flat, side="right") - 1).astype(np.int32)
    pos = (flat - starts[bi]).astype(np.int32)
    q = seeded_normal_bf16(oracle, rng, T * hq * 128)
    k = seeded_normal_bf16(oracle, rng, T * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, T * hkv * 128)
    kp = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    vp = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    spec = L.Bf16RopePagedKvAppendTokensSpec.extended(T, B, pool, hq, hkv)
    qo, okp, ovp = AppendRunner(L, spec, True).run(q, k, v, bi, pos, indptr, indices, last,
                                                   kp, vp)
    s = oracle.paged_spec(B, pool, hq, hkv)
    ekp, evp = kp.copy(), vp.copy()
    eq = oracle.append_tokens(s, T, q, k, v, bi, pos, indptr, indices, last, ekp, evp,
                              max_tokens=8192)
    check_rope(oracle, qo, eq, q, np.repeat(pos, hq), "query")
    assert np.array_equal(ovp, evp)
    slots = [(indices[indptr[b] + p // 16], p % 16) for b, p in zip(bi, pos)]
    rows = np.array([(pg * 16 + off) * hkv + h for pg, off in slots for h in range(hkv)])
    okr, ekr = okp.reshape(-1, 128), ekp.reshape(-1, 128)
    check_rope(oracle, okr[rows], ekr[rows], k, np.repeat(pos, hkv), "key rows")
    rest = np.ones(len(okr), bool)
    rest[rows] = False
    assert np.array_equal(okr[rest], ekr[rest])


@pytest.mark.parametrize("seed", range(12))
def test_paged_prefill_random_shapes(L, oracle, seed):
    """Paged causal prefill: random group sizes, query rows up to the KV
    length of each request, 16- or 64-column tiles (the wide tiles forced on
    shapes the planner would give row tiles)."""
    from gpu_util import PrefillRunner
    rng = np.random.default_rng(3000 + seed)
    hkv = int(rng.choice([1, 2, 4, 8]))
    hq = hkv * int(rng.choice([1, 2, 3, 4, 8]))
    B = int(rng.integers(1, 6))
    kv_lens = rng.integers(1, 700, size=B)
    qo_lens = np.array([int(rng.integers(1, min(k, 160) + 1)) for k in kv_lens])
    tile_cols = int(rng.choice([0, 16, 64]))
    pages = (kv_lens + 15) // 16
    pool = int(pages.sum()) + int(rng.integers(0, 6))
    log(f"prefill sweep {seed}: B={B} hq={hq} hkv={hkv} qo={qo_lens.tolist()} "
        f"kv={kv_lens.tolist()} tile_cols={tile_cols}")
    indptr = np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)
    indices = rng.permutation(pool)[: indptr[-1]].astype(np.int32)
    last = (kv_lens - (pages - 1) * 16).astype(np.int32)
    qo = np.concatenate([[0], np.cumsum(qo_lens)]).astype(np.int32)
    nnz = int(qo[-1])
    q = seeded_normal_bf16(oracle, rng, nnz * hq * 128)
    k = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    ref = oracle.prefill(oracle.prefill_spec(B, nnz, pool, hq, hkv), q, k, v, qo, indptr,
                         indices, last)
    r = PrefillRunner(L, B, nnz, pool, hq, hkv, tile_cols=tile_cols)
    out, lse = r.run(q, k, v, qo, indptr, indices, last)
    log(f"  plan {r.plan.algorithm} {compare_decode(oracle, out, lse, *ref)}")


@pytest.mark.parametrize("seed", range(8))
def test_paged_prefill_random_shapes_long_tiles(L, oracle, seed):
    """The long-tile algorithm forced on random shapes: random group sizes,
    ragged batches, query rows up to the KV length; one query tile per wave
    on these grids, so the two-wave-group form (the groups split each tile's
    blocks and merge in LDS) whenever the plan's grid is small."""
    from gpu_util import PrefillRunner
    rng = np.random.default_rng(4000 + seed)
    hkv = int(rng.choice([1, 2, 4, 8]))
    hq = hkv * int(rng.choice([1, 2, 4, 8]))
    B = int(rng.integers(1, 5))
    kv_lens = rng.integers(1, 1500, size=B)
    qo_lens = np.array([int(rng.integers(1, min(k, 400) + 1)) for k in kv_lens])
    pages = (kv_lens + 15) // 16
    pool = int(pages.sum()) + int(rng.integers(0, 6))
    indptr = np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)
    indices = rng.permutation(pool)[: indptr[-1]].astype(np.int32)
    last = (kv_lens - (pages - 1) * 16).astype(np.int32)
    qo = np.concatenate([[0], np.cumsum(qo_lens)]).astype(np.int32)
    nnz = int(qo[-1])
    log(f"long prefill sweep {seed}: B={B} hq={hq} hkv={hkv} qo={qo_lens.tolist()} "
        f"kv={kv_lens.tolist()}")
    q = seeded_normal_bf16(oracle, rng, nnz * hq * 128)
    k = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    ref = oracle.prefill(oracle.prefill_spec(B, nnz, pool, hq, hkv), q, k, v, qo, indptr,
                         indices, last)
    r = PrefillRunner(L, B, nnz, pool, hq, hkv, tile_cols="long")
    assert r.plan.algorithm == "long_tile"
    out, lse = r.run(q, k, v, qo, indptr, indices, last)
    log(f"  block_threads {r.plan.info.block_threads} {compare_decode(oracle, out, lse, *ref)}")


@pytest.mark.parametrize("seed", range(6))
def test_paged_prefill_random_batches_long_tiles(L, oracle, seed):
    """The long-tile algorithm forced on random batches of 3-12 ragged
    requests, whose tiles the kernel takes interleaved by their distance from
    their request's end (rank k: the k-th heaviest tile of every request);
    every tile is computed once: the result equals the oracle's."""
    from gpu_util import PrefillRunner
    rng = np.random.default_rng(5000 + seed)
    hkv = int(rng.choice([1, 2, 4]))
    hq = hkv * int(rng.choice([1, 2, 4]))
    B = int(rng.integers(3, 13))
    kv_lens = rng.integers(1, 600, size=B)
    qo_lens = np.array([int(rng.integers(1, min(k, 120) + 1)) for k in kv_lens])
    pages = (kv_lens + 15) // 16
    pool = int(pages.sum()) + int(rng.integers(0, 6))
    indptr = np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)
    indices = rng.permutation(pool)[: indptr[-1]].astype(np.int32)
    last = (kv_lens - (pages - 1) * 16).astype(np.int32)
    qo = np.concatenate([[0], np.cumsum(qo_lens)]).astype(np.int32)
    nnz = int(qo[-1])
    log(f"long prefill batch sweep {seed}: B={B} hq={hq} hkv={hkv} qo={qo_lens.tolist()} "
        f"kv={kv_lens.tolist()}")
    q = seeded_normal_bf16(oracle, rng, nnz * hq * 128)
    k = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    ref = oracle.prefill(oracle.prefill_spec(B, nnz, pool, hq, hkv), q, k, v, qo, indptr,
                         indices, last)
    r = PrefillRunner(L, B, nnz, pool, hq, hkv, tile_cols="long")
    assert r.plan.algorithm == "long_tile"
    out, lse = r.run(q, k, v, qo, indptr, indices, last)
    log(f"  block_threads {r.plan.info.block_threads} {compare_decode(oracle, out, lse, *ref)}")
