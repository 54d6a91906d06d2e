"""GPU parity at the full workloads of BASELINE configs 4 and 5 (the reference's
gate protocol, crates/loom-infer-validation/src/gates/paged_batch_decode.rs:28-148:
seeded inputs, the CPU oracle on the same inputs, output/LSE tolerances).

Inputs are generated on the device (seeded torch generator) and the oracle runs
on host copies of exactly the pages the page table names, renumbered into a
compact pool: the arithmetic per request is unchanged, and the oracle never
touches the other pages of the 262144-page pool."""
import sys

import numpy as np
import pytest

from gpu_util import DecodeRunner, bf16_host, compare_decode, to_dev_i32
from test_gpu_append import check_rope

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


def shuffled_table(rng, lens, pool, page=16):
    pages = (np.asarray(lens) + page - 1) // page
    indptr = np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)
    assert indptr[-1] <= pool
    indices = rng.permutation(pool)[: indptr[-1]].astype(np.int32)
    last = (np.asarray(lens) - (pages - 1) * page).astype(np.int32)
    return indptr, indices, last


def device_normal_bf16(n, gen):
    import torch
    return torch.randn(n, generator=gen, device="cuda", dtype=torch.bfloat16)


def gather_pages(t, pool, pages):
    """Host bits of the listed pages of a flat device pool, in list order."""
    import torch
    idx = torch.from_numpy(np.asarray(pages, np.int64)).to(t.device)
    return bf16_host(t.view(pool, -1).index_select(0, idx).reshape(-1))


def test_config4_gqa8_b8_ctx32768(L, oracle):
    """Config 4: batch 8, 64 q / 8 kv heads, context 32768 per request,
    shuffled pages, the default (split-KV) plan.  Every request and every
    query head is checked against the oracle."""
    import torch
    log("config 4: GQA8 batch 8 ctx 32768")
    B, hq, hkv = 8, 64, 8
    lens = [32768] * B
    pool = B * 2048 + 64
    rng = np.random.default_rng(4)
    indptr, indices, last = shuffled_table(rng, lens, pool)
    g = torch.Generator(device="cuda")
    g.manual_seed(4)
    q = device_normal_bf16(B * hq * 128, g)
    k = device_normal_bf16(pool * 16 * hkv * 128, g)
    v = device_normal_bf16(pool * 16 * hkv * 128, g)
    r = DecodeRunner(L, B, pool, hq, hkv)
    info = r.plan.info
    assert r.plan.algorithm == "balanced_split_kv"
    # context 32768 over the plan's teams: every request crosses team ranges
    assert info.teams > B
    out, lse = r.run_dev(q, k, v, to_dev_i32(indptr), to_dev_i32(indices), to_dev_i32(last))
    out_h, lse_h = bf16_host(out), lse.cpu().numpy()
    kh = gather_pages(k, pool, indices)
    vh = gather_pages(v, pool, indices)
    n = int(indptr[-1])
    s = oracle.paged_spec(B, n, hq, hkv)
    ref_o, ref_l = oracle.paged_decode_parallel(s, bf16_host(q), kh, vh, indptr,
                                                np.arange(n, dtype=np.int32), last)
    st = compare_decode(oracle, out_h, lse_h, ref_o, ref_l)
    log(f"  teams={info.teams} tile={info.group_tile}x{info.group_tiles} {st}")
    # a second call over the first call's workspace contents is identical
    out2, lse2 = r.run_dev(q, k, v, to_dev_i32(indptr), to_dev_i32(indices), to_dev_i32(last))
    assert np.array_equal(bf16_host(out2), out_h) and np.array_equal(lse2.cpu().numpy(), lse_h)


def test_config5_full_step_graph_b256_pool262144(L, oracle):
    """Config 5: RoPE + one-token append then paged decode GQA4 (32 q / 8 kv
    heads), batch 256, lognormal lengths (median 2048, sigma 0.8, clipped to
    [16, 16384]), shuffled pages in a 262144-page pool, captured as one graph.
    The first replay is checked against the oracle's append then decode (the
    rotated query and appended K rows within one BF16 ulp or a proven sin/cos
    rounding difference, V rows and every other row of the used pages bit for
    bit, the attention output within tolerance); later replays (the append rewrites the same slots with the same
    values) are bit-equal to the first; pages outside the table are untouched."""
    import torch
    log("config 5: full decode step graph, batch 256, pool 262144")
    B, hq, hkv, pool = 256, 32, 8, 262144
    rng = np.random.default_rng(5)
    lens = np.clip(np.round(np.exp(np.log(2048) + 0.8 * rng.standard_normal(B))), 16,
                   16384).astype(np.int64)
    indptr, indices, last = shuffled_table(rng, lens, pool)
    n = int(indptr[-1])
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    qn = device_normal_bf16(B * hq * 128, g)
    kn = device_normal_bf16(B * hkv * 128, g)
    vn = device_normal_bf16(B * hkv * 128, g)
    kp = device_normal_bf16(pool * 16 * hkv * 128, g)
    vp = device_normal_bf16(pool * 16 * hkv * 128, g)
    # host copies before the step: the used pages and a sample of the others
    kp_h, vp_h = gather_pages(kp, pool, indices), gather_pages(vp, pool, indices)
    unused = np.setdiff1d(np.arange(pool), indices)
    probe = rng.choice(unused, size=2048, replace=False)
    probe_k, probe_v = gather_pages(kp, pool, probe), gather_pages(vp, pool, probe)
    qn_h, kn_h, vn_h = bf16_host(qn), bf16_host(kn), bf16_host(vn)

    dec = DecodeRunner(L, B, pool, hq, hkv)
    ap = L.RopeProvider.load(0).plan_bf16_paged_append(
        L.Bf16RopePagedKvAppendSpec(B, pool, hq, hkv))
    aws = torch.zeros(ap.workspace_bytes, dtype=torch.uint8, device="cuda")
    ip, ix, ln = to_dev_i32(indptr), to_dev_i32(indices), to_dev_i32(last)
    qrot = torch.empty(B * hq * 128, dtype=torch.bfloat16, device="cuda")
    out = torch.empty(B * hq * 128, dtype=torch.bfloat16, device="cuda")
    lse = torch.empty(B * hq, dtype=torch.float32, device="cuda")
    gq = L.GraphQueue(0, 2)
    b = gq.bindings(16)
    hq_, hk, hv = b.bind_read(qn), b.bind_read(kn), b.bind_read(vn)
    hip_, hix, hln = b.bind_read(ip), b.bind_read(ix), b.bind_read(ln)
    hqr, hkp, hvp = b.bind_read_write(qrot), b.bind_read_write(kp), b.bind_read_write(vp)
    haws = b.bind_read_write(aws)
    ho, hl, hws = b.bind_read_write(out), b.bind_read_write(lse), b.bind_read_write(dec.workspace)
    a_args = L.Bf16RopePagedKvAppendArgs(hq_, hk, hv, hip_, hix, hln, hqr.write(), hkp.write(),
                                         hvp.write(), haws.write())
    d_args = L.Bf16PagedBatchDecodeArgs(hqr.read(), hkp.read(), hvp.read(), hip_, hix, hln,
                                        ho.write(), hl.write(), hws.write())

    def record(scope):
        ap.enqueue_into(scope, a_args)
        dec.plan.enqueue_into(scope, d_args)

    exec_ = gq.capture(b, record).instantiate()
    assert exec_.commands() == 2
    log(f"  captured; decode teams={dec.plan.info.teams}, {n} pages in the table")

    # oracle step on the compact pool (page i of the compact pool = indices[i])
    s = oracle.paged_spec(B, n, hq, hkv)
    cix = np.arange(n, dtype=np.int32)
    eq = oracle.append(s, qn_h, kn_h, vn_h, indptr, cix, last, kp_h, vp_h)
    ref_o, ref_l = oracle.paged_decode_parallel(s, eq, kp_h, vp_h, indptr, cix, last)

    first = None
    for i in range(3):
        out.fill_(float("nan"))  # eager work between replays
        qrot.zero_()
        torch.cuda.synchronize()
        exec_.launch().wait()
        o, l_ = bf16_host(out), lse.cpu().numpy()
        if i == 0:
            # RoPE within one BF16 ulp, or proven sin/cos rounding differences
            pos = (lens - 1).astype(np.int64)
            check_rope(oracle, bf16_host(qrot), eq, qn_h, np.repeat(pos, hq), "query",
                       pin="c5_one_token_query")
            # the appended K rows, then every other row of the used pages bit-exact
            got_k = gather_pages(kp, pool, indices).reshape(-1, 128)
            want_k = kp_h.reshape(-1, 128)
            slot = indptr[:-1] + (pos // 16)  # compact page of each request's new token
            rows = ((slot * 16 + pos % 16)[:, None] * hkv + np.arange(hkv)).reshape(-1)
            check_rope(oracle, got_k[rows], want_k[rows], kn_h, np.repeat(pos, hkv), "key rows",
                       pin="c5_one_token_key_rows")
            got_k[rows] = 0
            want_k[rows] = 0
            assert np.array_equal(got_k, want_k), "key pages outside the appended rows"
            assert np.array_equal(gather_pages(vp, pool, indices), vp_h), "value pages"
            assert np.array_equal(gather_pages(kp, pool, probe), probe_k), "untouched K pages"
            assert np.array_equal(gather_pages(vp, pool, probe), probe_v), "untouched V pages"
            st = compare_decode(oracle, o, l_, ref_o, ref_l)
            log(f"  replay 0: {st}")
            first = (o, l_)
        else:
            assert np.array_equal(o, first[0]) and np.array_equal(l_, first[1]), f"replay {i}"
    exec_.into_bindings()
