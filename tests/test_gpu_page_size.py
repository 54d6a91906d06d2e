"""Pages of 32 and 64 token rows (no reference counterpart: the reference
supports 16-row pages only).  A page of P rows is streamed as P/16 blocks of 16
rows, so every operation on P-row pages must equal, bit for bit, the same
operation on the 16-row page table that names the same bytes: with NHD pages a
[pool, P, Hkv, 128] cache is the [pool*P/16, 16, Hkv, 128] cache, block j of
page p being 16-row page p*P/16 + j.  The 16-row results are themselves checked
against the pinned oracle here."""
import sys

import numpy as np
import pytest

from gpu_util import DecodeRunner, compare_decode, seeded_normal_bf16
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


def table(rng, lens, pool, P):
    """A P-row page table drawn from a seeded permutation of the pool."""
    pages = [(n + P - 1) // P for n in lens]
    ip = np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)
    assert ip[-1] <= pool
    ix = rng.permutation(pool)[: ip[-1]].astype(np.int32)
    last = np.array([n - (p - 1) * P for n, p in zip(lens, pages)], np.int32)
    return ip, ix, last


def to_rows16(ip, ix, last, P):
    """The 16-row page table naming the same K/V bytes as a P-row NHD table."""
    m = P // 16
    ip16, ix16, last16 = [0], [], []
    for r in range(len(last)):
        pages = ix[ip[r]:ip[r + 1]]
        kv = (len(pages) - 1) * P + int(last[r])
        blocks = (kv + 15) // 16
        ix16 += [int(pages[b // m]) * m + b % m for b in range(blocks)]
        last16.append(kv - 16 * (blocks - 1))
        ip16.append(len(ix16))
    return (np.array(ip16, np.int32), np.array(ix16, np.int32), np.array(last16, np.int32))


def test_rows16_helper():
    ip, ix, last = np.array([0, 2, 3], np.int32), np.array([5, 1, 7], np.int32), \
        np.array([20, 32], np.int32)
    ip16, ix16, last16 = to_rows16(ip, ix, last, 32)
    assert ip16.tolist() == [0, 4, 6]
    assert ix16.tolist() == [10, 11, 2, 3, 14, 15] and last16.tolist() == [4, 16]


DECODE = [
    # (name, P, B, hq, hkv, lens, plan options for the P-row and the 16-row plan)
    ("direct_p32_gqa4", 32, 4, 16, 4, [3, 40, 17, 90], {"teams": 0, "max_total_pages": 64}),
    ("direct_p64_mqa", 64, 3, 8, 1, [16, 70, 129], {"teams": 0, "max_total_pages": 64}),
    ("balanced_p32_gqa4", 32, 5, 32, 8, [40, 1000, 17, 3000, 256], {"teams": 7}),
    ("balanced_p64_gqa8", 64, 3, 64, 8, [2049, 700, 5000], {"teams": 6}),
]


@pytest.mark.parametrize("case", DECODE, ids=lambda c: c[0])
def test_decode_page_size_equals_16_row_table(L, oracle, case):
    name, P, B, hq, hkv, lens, opts = case
    log(f"decode page size {name}")
    rng = np.random.default_rng(len(name) + P)
    pool = sum((n + P - 1) // P for n in lens) + 3
    ip, ix, last = table(rng, lens, pool, P)
    m = P // 16
    q = seeded_normal_bf16(oracle, rng, B * hq * 128)
    k = seeded_normal_bf16(oracle, rng, pool * P * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, pool * P * hkv * 128)
    ip16, ix16, last16 = to_rows16(ip, ix, last, P)
    ref = oracle.paged_decode(oracle.paged_spec(B, pool * m, hq, hkv), q, k, v, ip16, ix16,
                              last16)
    r16 = DecodeRunner(L, B, pool * m, hq, hkv, **opts)
    o1, l1 = r16.run(q, k, v, ip16, ix16, last16)
    compare_decode(oracle, o1, l1, *ref)
    rp = DecodeRunner(L, B, pool, hq, hkv, **opts)
    rp.spec = L.Bf16PagedBatchDecodeSpec(B, pool, hq, hkv, kv_page_size=P)
    rp.plan = rp.provider.plan_bf16_paged_batch(rp.spec, **opts)
    assert rp.plan.info.algorithm == r16.plan.info.algorithm
    o2, l2 = rp.run(q, k, v, ip, ix, last)
    assert np.array_equal(o1, o2) and np.array_equal(l1, l2)
    # the same pages in HND order ([pool, Hkv, P, 128])
    def hnd(x):
        return np.ascontiguousarray(x.reshape(pool, P, hkv, 128).transpose(0, 2, 1, 3)).reshape(-1)
    rh = DecodeRunner(L, B, pool, hq, hkv, **opts)
    rh.spec = L.Bf16PagedBatchDecodeSpec(B, pool, hq, hkv, kv_page_size=P, kv_layout="HND")
    rh.plan = rh.provider.plan_bf16_paged_batch(rh.spec, **opts)
    o3, l3 = rh.run(q, hnd(k), hnd(v), ip, ix, last)
    assert np.array_equal(o1, o3) and np.array_equal(l1, l3)


def test_decode_page_size_guards(L, oracle):
    """last_page_len up to P is valid; P + 1 fails the per-request guard
    (sentinels kept); a page index past the pool poisons only its request."""
    P, B, hq, hkv = 32, 3, 8, 2
    rng = np.random.default_rng(99)
    lens = [64, 33, 100]
    pool = 12
    ip, ix, last = table(rng, lens, pool, P)
    q = seeded_normal_bf16(oracle, rng, B * hq * 128)
    k = seeded_normal_bf16(oracle, rng, pool * P * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, pool * P * hkv * 128)
    for opts in ({"teams": 0}, {"teams": 3}):
        r = DecodeRunner(L, B, pool, hq, hkv, **opts)
        r.spec = L.Bf16PagedBatchDecodeSpec(B, pool, hq, hkv, kv_page_size=P)
        r.plan = r.provider.plan_bf16_paged_batch(r.spec, **opts)
        bad_last = last.copy()
        bad_last[1] = P + 1
        bad_ix = ix.copy()
        bad_ix[ip[2]] = pool + 4
        out, lse = r.run(q, k, v, ip, bad_ix, bad_last)
        o = oracle.bf16_to_f32(out).reshape(B, hq * 128)
        assert np.all(np.isnan(o[1])) and np.all(np.isnan(o[2]))
        ip16, ix16, last16 = to_rows16(ip, ix, last, P)
        ref_o, ref_l = oracle.paged_decode(oracle.paged_spec(B, pool * 2, hq, hkv), q, k, v,
                                           ip16, ix16, last16)
        compare_decode(oracle, out.reshape(B, -1)[0], lse[:hq], ref_o.reshape(B, -1)[0],
                       ref_l[:hq])


@pytest.mark.parametrize("P", [32, 64])
@pytest.mark.parametrize("explicit", [False, True], ids=["one_token", "explicit_tokens"])
def test_append_page_size_writes_the_same_slots(L, oracle, P, explicit):
    log(f"append page size {P} explicit={explicit}")
    rng = np.random.default_rng(P + explicit)
    B, hq, hkv = 4, 16, 4
    lens = [5, P + 3, 2 * P, 1]
    pool = 12
    ip, ix, last = table(rng, lens, pool, P)
    ip16, ix16, last16 = to_rows16(ip, ix, last, P)
    m = P // 16
    if explicit:
        bi = np.array([1, 2, 0, 3, 1, 2], np.int32)
        pos = np.array([P + 2, 2 * P - 1, 0, 0, 16, P], np.int32)
        T = len(bi)
        spec_p = L.Bf16RopePagedKvAppendTokensSpec(T, B, pool, hq, hkv, kv_page_size=P)
        spec_16 = L.Bf16RopePagedKvAppendTokensSpec(T, B, pool * m, hq, hkv)
    else:
        bi = pos = None
        T = B
        spec_p = L.Bf16RopePagedKvAppendSpec(B, pool, hq, hkv, kv_page_size=P)
        spec_16 = L.Bf16RopePagedKvAppendSpec(B, pool * m, hq, hkv)
    q = seeded_normal_bf16(oracle, rng, T * hq * 128)
    k = seeded_normal_bf16(oracle, rng, T * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, T * hkv * 128)
    kp = seeded_normal_bf16(oracle, rng, pool * P * hkv * 128)
    vp = seeded_normal_bf16(oracle, rng, pool * P * hkv * 128)
    q1, k1, v1 = AppendRunner(L, spec_16, explicit).run(q, k, v, bi, pos, ip16, ix16, last16,
                                                         kp, vp)
    assert not np.array_equal(k1, kp)  # the 16-row command wrote its slots
    q2, k2, v2 = AppendRunner(L, spec_p, explicit).run(q, k, v, bi, pos, ip, ix, last, kp, vp)
    assert np.array_equal(q1, q2) and np.array_equal(k1, k2) and np.array_equal(v1, v2)


@pytest.mark.parametrize("opts", [{"teams": 0, "max_total_pages": 64}, {"teams": 5}],
                         ids=["direct", "balanced"])
def test_fp8_decode_page_size_equals_16_row_table(L, oracle, opts):
    """FP8 E4M3 pages of 32 rows stream the same bytes as the 16-row table."""
    from test_gpu_fp8 import random_fp8, run_decode
    P, B, hq, hkv = 32, 3, 16, 4
    rng = np.random.default_rng(77)
    lens = [17, 90, 40]
    pool = sum((n + P - 1) // P for n in lens) + 2
    ip, ix, last = table(rng, lens, pool, P)
    ip16, ix16, last16 = to_rows16(ip, ix, last, P)
    q = seeded_normal_bf16(oracle, rng, B * hq * 128)
    k8 = random_fp8(rng, pool * P * hkv * 128)
    v8 = random_fp8(rng, pool * P * hkv * 128)
    scales = [0.5, 0.25]
    s16 = L.Bf16PagedBatchDecodeSpec(B, pool * 2, hq, hkv, kv_dtype="fp8_e4m3")
    sp = L.Bf16PagedBatchDecodeSpec(B, pool, hq, hkv, kv_dtype="fp8_e4m3", kv_page_size=P)
    o1, l1, p1 = run_decode(L, s16, opts, q, k8, v8, ip16, ix16, last16, scales)
    o2, l2, p2 = run_decode(L, sp, opts, q, k8, v8, ip, ix, last, scales)
    assert p1.info.algorithm == p2.info.algorithm
    assert not np.any(np.isnan(oracle.bf16_to_f32(o1)))
    assert np.array_equal(o1, o2) and np.array_equal(l1, l2)


@pytest.mark.parametrize("P", [32, 64])
@pytest.mark.parametrize("layout", ["NHD", "HND"])
def test_prefill_page_size_equals_16_row_table(L, oracle, P, layout):
    """Paged causal prefill on P-row pages equals the 16-row command on the
    table naming the same bytes (NHD), and HND P-row pages the NHD ones."""
    from gpu_util import PrefillRunner
    log(f"prefill page size {P} {layout}")
    rng = np.random.default_rng(P + len(layout))
    B, hq, hkv = 3, 16, 4
    qo_lens, kv_lens = [3, 40, 1], [40, 300, P]
    pool = sum((n + P - 1) // P for n in kv_lens) + 2
    ip, ix, last = table(rng, kv_lens, pool, P)
    ip16, ix16, last16 = to_rows16(ip, ix, last, P)
    m = P // 16
    qo = np.concatenate([[0], np.cumsum(qo_lens)]).astype(np.int32)
    nnz = int(qo[-1])
    q = seeded_normal_bf16(oracle, rng, nnz * hq * 128)
    k = seeded_normal_bf16(oracle, rng, pool * P * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, pool * P * hkv * 128)
    ref = oracle.prefill(oracle.prefill_spec(B, nnz, pool * m, hq, hkv), q, k, v, qo, ip16,
                         ix16, last16)
    r16 = PrefillRunner(L, B, nnz, pool * m, hq, hkv)
    o1, l1 = r16.run(q, k, v, qo, ip16, ix16, last16)
    compare_decode(oracle, o1, l1, *ref)
    rp = PrefillRunner(L, B, nnz, pool, hq, hkv)
    rp.spec = L.Bf16PagedPrefillSpec(B, nnz, pool, hq, hkv, kv_layout=layout, kv_page_size=P)
    rp.plan = rp.provider.plan_bf16_paged(rp.spec)
    if layout == "HND":
        def conv(x):
            return np.ascontiguousarray(
                x.reshape(pool, P, hkv, 128).transpose(0, 2, 1, 3)).reshape(-1)
        kk, vv = conv(k), conv(v)
    else:
        kk, vv = k, v
    o2, l2 = rp.run(q, kk, vv, qo, ip, ix, last)
    assert np.array_equal(o1, o2) and np.array_equal(l1, l2)


@pytest.mark.parametrize("P", [16, 32])
def test_fp8_prefill_equals_bf16_on_widened_pages(L, oracle, P):
    """FP8 E4M3 paged prefill (no reference counterpart).  E4M3 is exact in
    BF16 and power-of-two scales are exact, so with scales (0.5, 0.25) the FP8
    command must equal the BF16 command on the widened, scaled pages bit for
    bit; a non-power-of-two scale is checked against the oracle's prefill on
    the same values within the decode tolerance."""
    import torch
    from gpu_util import PrefillRunner, bf16_host, to_dev_bf16, to_dev_i32
    from test_gpu_fp8 import random_fp8
    log(f"fp8 prefill page size {P}")
    rng = np.random.default_rng(300 + P)
    B, hq, hkv = 3, 16, 4
    qo_lens, kv_lens = [5, 33, 1], [40, 200, 17]
    pool = sum((n + P - 1) // P for n in kv_lens) + 2
    ip, ix, last = table(rng, kv_lens, pool, P)
    qo = np.concatenate([[0], np.cumsum(qo_lens)]).astype(np.int32)
    nnz = int(qo[-1])
    q = seeded_normal_bf16(oracle, rng, nnz * hq * 128)
    k8 = random_fp8(rng, pool * P * hkv * 128)
    v8 = random_fp8(rng, pool * P * hkv * 128)
    kw = {} if P == 16 else {"kv_page_size": P}

    def fp8_run(scales, k8=k8, v8=v8):
        r = PrefillRunner(L, B, nnz, pool, hq, hkv)
        r.spec = L.Bf16PagedPrefillSpec(B, nnz, pool, hq, hkv, kv_dtype="fp8_e4m3", **kw)
        r.plan = r.provider.plan_bf16_paged(r.spec)
        out, lse = r.run_dev(to_dev_bf16(q), torch.from_numpy(k8).to("cuda"),
                             torch.from_numpy(v8).to("cuda"), to_dev_i32(qo), to_dev_i32(ip),
                             to_dev_i32(ix), to_dev_i32(last),
                             scales=torch.tensor(scales, dtype=torch.float32, device="cuda"))
        return bf16_host(out), lse.cpu().numpy()

    def widened(x8, scale):
        return oracle.bf16_from_f32((oracle.fp8_to_f32(x8) * np.float32(scale)).astype(np.float32))

    rb = PrefillRunner(L, B, nnz, pool, hq, hkv)
    rb.spec = L.Bf16PagedPrefillSpec(B, nnz, pool, hq, hkv, **kw)
    rb.plan = rb.provider.plan_bf16_paged(rb.spec)
    o_b, l_b = rb.run(q, widened(k8, 0.5), widened(v8, 0.25), qo, ip, ix, last)
    o_f, l_f = fp8_run([0.5, 0.25])
    assert not np.any(np.isnan(oracle.bf16_to_f32(o_f)))
    assert np.array_equal(o_b, o_f) and np.array_equal(l_b, l_f)
    # a scale that is not a power of two: the oracle on the dequantized values
    # (codes up to 0x44, |x| <= 3, so the BF16 rounding of x * scale moves the
    # scores by far less than the tolerance)
    if P == 16:
        ks = random_fp8(rng, pool * P * hkv * 128, max_code=0x44)
        vs = random_fp8(rng, pool * P * hkv * 128, max_code=0x44)
        o3, l3 = fp8_run([0.3, 0.7], ks, vs)
        kd = (oracle.fp8_to_f32(ks) * np.float32(0.3)).astype(np.float32)
        vd = (oracle.fp8_to_f32(vs) * np.float32(0.7)).astype(np.float32)
        ref = oracle.prefill(oracle.prefill_spec(B, nnz, pool, hq, hkv), q,
                             oracle.bf16_from_f32(kd), oracle.bf16_from_f32(vd), qo, ip, ix, last)
        compare_decode(oracle, o3, l3, *ref)


@pytest.mark.parametrize("P", [32, 64])
def test_append_page_size_chunked_path_writes_the_same_slots(L, oracle, P):
    """The chunk-validated append (T > 64 tokens) on P-row pages equals the
    16-row command on the table naming the same bytes."""
    log(f"append page size {P} chunked path")
    rng = np.random.default_rng(300 + P)
    B, hq, hkv = 4, 8, 2
    lens = [40, 3 * P + 5, 2 * P, 70]
    pool = sum((n + P - 1) // P for n in lens) + 3
    ip, ix, last = table(rng, lens, pool, P)
    ip16, ix16, last16 = to_rows16(ip, ix, last, P)
    m = P // 16
    T = 100
    flat = rng.choice(int(sum(lens)), size=T, replace=False)
    starts = np.concatenate([[0], np.cumsum(lens)])
    bi = (np.searchsorted(starts, flat, side="right") - 1).astype(np.int32)
    pos = (flat - starts[bi]).astype(np.int32)
    spec_p = L.Bf16RopePagedKvAppendTokensSpec.extended(T, B, pool, hq, hkv, kv_page_size=P)
    spec_16 = L.Bf16RopePagedKvAppendTokensSpec.extended(T, B, pool * m, hq, hkv)
    q = seeded_normal_bf16(oracle, rng, T * hq * 128)
    k = seeded_normal_bf16(oracle, rng, T * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, T * hkv * 128)
    kp = seeded_normal_bf16(oracle, rng, pool * P * hkv * 128)
    vp = seeded_normal_bf16(oracle, rng, pool * P * hkv * 128)
    q1, k1, v1 = AppendRunner(L, spec_16, True).run(q, k, v, bi, pos, ip16, ix16, last16, kp, vp)
    assert not np.array_equal(k1, kp)
    q2, k2, v2 = AppendRunner(L, spec_p, True).run(q, k, v, bi, pos, ip, ix, last, kp, vp)
    assert np.array_equal(q1, q2) and np.array_equal(k1, k2) and np.array_equal(v1, v2)
