"""HND K/V page layout ([pool, Hkv, 16, 128], no reference counterpart: the
reference supports NHD only).  Every paged operation run on HND pages must
equal, bit for bit, the same operation on the NHD pages holding the same
tokens: the kernels do the same arithmetic in the same order and differ only
in the row and head strides of their loads and stores.  The NHD results are
themselves checked against the pinned oracle here."""
import sys

import numpy as np
import pytest

from gpu_util import (DecodeRunner, PrefillRunner, compare_decode, ragged_table,
                      seeded_normal_bf16)
from test_gpu_append import AppendRunner

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


def to_hnd(pages, pool, hkv):
    """NHD [pool, 16, Hkv, 128] -> HND [pool, Hkv, 16, 128] (bf16 bits)."""
    return np.ascontiguousarray(pages.reshape(pool, 16, hkv, 128).transpose(0, 2, 1, 3)).reshape(-1)


def to_nhd(pages, pool, hkv):
    return np.ascontiguousarray(pages.reshape(pool, hkv, 16, 128).transpose(0, 2, 1, 3)).reshape(-1)


def test_hnd_roundtrip_helper():
    x = np.arange(3 * 16 * 2 * 128, dtype=np.uint16)
    assert np.array_equal(to_nhd(to_hnd(x, 3, 2), 3, 2), x)
    h = to_hnd(x, 3, 2).reshape(3, 2, 16, 128)
    assert h[1, 1, 5, 7] == x.reshape(3, 16, 2, 128)[1, 5, 1, 7]


DECODE = [
    # (name, B, hq, hkv, lens, plan options)
    ("direct_gqa4", 4, 16, 4, [3, 32, 17, 41], {}),
    ("direct_mqa", 3, 8, 1, [16, 23, 48], {}),
    ("balanced_gqa4_teams7", 5, 32, 8, [40, 1000, 17, 3000, 256], {"teams": 7}),
    ("balanced_gqa8_default", 3, 64, 8, [2049, 700, 5000], {"teams": 0, "max_total_pages": 600}),
]


@pytest.mark.parametrize("case", DECODE, ids=lambda c: c[0])
def test_decode_hnd_equals_nhd(L, oracle, case):
    name, B, hq, hkv, lens, opts = case
    log(f"decode HND {name}")
    rng = np.random.default_rng(len(name))
    pool = sum((x + 15) // 16 for x in lens) + 5
    ip, ix, last = ragged_table(rng, lens, pool)
    q = seeded_normal_bf16(oracle, rng, B * hq * 128)
    k = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    ref = oracle.paged_decode(oracle.paged_spec(B, pool, hq, hkv), q, k, v, ip, ix, last)
    nhd = DecodeRunner(L, B, pool, hq, hkv, **opts)
    o1, l1 = nhd.run(q, k, v, ip, ix, last)
    compare_decode(oracle, o1, l1, *ref)
    hnd = DecodeRunner(L, B, pool, hq, hkv, **opts)
    hnd.spec = L.Bf16PagedBatchDecodeSpec(B, pool, hq, hkv, 128, 16, kv_layout="HND")
    hnd.plan = hnd.provider.plan_bf16_paged_batch(hnd.spec, **opts)
    assert hnd.plan.info.algorithm == nhd.plan.info.algorithm
    o2, l2 = hnd.run(q, to_hnd(k, pool, hkv), to_hnd(v, pool, hkv), ip, ix, last)
    assert np.array_equal(o1, o2) and np.array_equal(l1, l2)


def test_prefill_hnd_equals_nhd(L, oracle):
    log("prefill HND")
    rng = np.random.default_rng(17)
    hq, hkv = 16, 4
    qo_lens, kv_lens = [3, 7, 1], [40, 300, 16]
    pool = sum((x + 15) // 16 for x in kv_lens) + 2
    ip, ix, last = ragged_table(rng, kv_lens, pool)
    qo = np.concatenate([[0], np.cumsum(qo_lens)]).astype(np.int32)
    nnz = int(qo[-1])
    q = seeded_normal_bf16(oracle, rng, nnz * hq * 128)
    k = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    ref = oracle.prefill(oracle.prefill_spec(3, nnz, pool, hq, hkv), q, k, v, qo, ip, ix, last)
    for waves in (4, 8):
        nhd = PrefillRunner(L, 3, nnz, pool, hq, hkv, waves=waves)
        o1, l1 = nhd.run(q, k, v, qo, ip, ix, last)
        compare_decode(oracle, o1, l1, *ref)
        hnd = PrefillRunner(L, 3, nnz, pool, hq, hkv, waves=waves)
        hnd.spec = L.Bf16PagedPrefillSpec(3, nnz, pool, hq, hkv, kv_layout="HND")
        hnd.plan = hnd.provider.plan_bf16_paged(hnd.spec, waves=waves)
        o2, l2 = hnd.run(q, to_hnd(k, pool, hkv), to_hnd(v, pool, hkv), qo, ip, ix, last)
        assert np.array_equal(o1, o2) and np.array_equal(l1, l2)


@pytest.mark.parametrize("explicit", [False, True], ids=["one_token", "explicit_tokens"])
def test_append_hnd_writes_the_same_slots(L, oracle, explicit):
    log(f"append HND explicit={explicit}")
    rng = np.random.default_rng(23 + explicit)
    B, hq, hkv, pool = 4, 16, 4, 12
    ip = np.array([0, 2, 3, 6, 8], np.int32)
    ix = rng.permutation(pool)[:8].astype(np.int32)
    last = np.array([5, 16, 1, 9], np.int32)
    if explicit:
        bi = np.array([0, 2, 2, 3, 1, 0], np.int32)
        pos = np.array([17, 32, 31, 20, 15, 3], np.int32)
        T = 6
        nhd_spec = L.Bf16RopePagedKvAppendTokensSpec(T, B, pool, hq, hkv)
        hnd_spec = L.Bf16RopePagedKvAppendTokensSpec(T, B, pool, hq, hkv, kv_layout="HND")
    else:
        bi = pos = None
        T = B
        nhd_spec = L.Bf16RopePagedKvAppendSpec(B, pool, hq, hkv)
        hnd_spec = L.Bf16RopePagedKvAppendSpec(B, pool, hq, hkv, kv_layout="HND")
    assert hnd_spec.paged.kv_layout == "HND" and nhd_spec.paged.kv_layout == "NHD"
    q = seeded_normal_bf16(oracle, rng, T * hq * 128)
    k = seeded_normal_bf16(oracle, rng, T * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, T * hkv * 128)
    kp = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    vp = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    q1, k1, v1 = AppendRunner(L, nhd_spec, explicit).run(q, k, v, bi, pos, ip, ix, last, kp, vp)
    q2, k2, v2 = AppendRunner(L, hnd_spec, explicit).run(q, k, v, bi, pos, ip, ix, last,
                                                         to_hnd(kp, pool, hkv),
                                                         to_hnd(vp, pool, hkv))
    assert not np.array_equal(k1, kp)  # the NHD command wrote its slots
    assert np.array_equal(q1, q2)
    assert np.array_equal(to_nhd(k2, pool, hkv), k1) and np.array_equal(to_nhd(v2, pool, hkv), v1)


def test_unknown_layout_is_rejected(L):
    with pytest.raises(ValueError):
        L.Bf16PagedBatchDecodeSpec(1, 1, 1, 1, kv_layout="NDH")
    spec = L.Bf16PagedBatchDecodeSpec(1, 1, 1, 1)
    spec._c.kv_layout = 7  # a caller writing the C struct field directly
    with pytest.raises(L.PlanError) as e:
        L.DecodeProvider.load(0).plan_bf16_paged_batch(spec)
    assert e.value.variant == "InvalidOption" and e.value.operand == "kv_layout"


def test_append_hnd_chunked_path_writes_the_same_slots(L, oracle):
    """The chunk-validated append (T > 64 tokens) on HND pages writes the
    same bytes as on NHD pages."""
    log("append HND chunked path")
    rng = np.random.default_rng(29)
    B, hq, hkv = 5, 8, 2
    lens = np.array([40, 300, 17, 129, 64])
    pages = (lens + 15) // 16
    pool = int(pages.sum()) + 4
    ip = np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)
    ix = rng.permutation(pool)[: ip[-1]].astype(np.int32)
    last = (lens - (pages - 1) * 16).astype(np.int32)
    T = 100
    flat = rng.choice(int(lens.sum()), size=T, replace=False)
    starts = np.concatenate([[0], np.cumsum(lens)])
    bi = (np.searchsorted(starts, flat, side="right") - 1).astype(np.int32)
    pos = (flat - starts[bi]).astype(np.int32)
    nhd_spec = L.Bf16RopePagedKvAppendTokensSpec.extended(T, B, pool, hq, hkv)
    hnd_spec = L.Bf16RopePagedKvAppendTokensSpec.extended(T, B, pool, hq, hkv, kv_layout="HND")
    q = seeded_normal_bf16(oracle, rng, T * hq * 128)
    k = seeded_normal_bf16(oracle, rng, T * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, T * hkv * 128)
    kp = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    vp = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    q1, k1, v1 = AppendRunner(L, nhd_spec, True).run(q, k, v, bi, pos, ip, ix, last, kp, vp)
    q2, k2, v2 = AppendRunner(L, hnd_spec, True).run(q, k, v, bi, pos, ip, ix, last,
                                                     to_hnd(kp, pool, hkv), to_hnd(vp, pool, hkv))
    assert not np.array_equal(k1, kp)
    assert np.array_equal(q1, q2)
    assert np.array_equal(to_nhd(k2, pool, hkv), k1) and np.array_equal(to_nhd(v2, pool, hkv), v1)
