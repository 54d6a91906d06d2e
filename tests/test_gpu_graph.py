"""hipGraph fixed-address capture and replay of the decode step (graph/mod.rs),
checked replay by replay against eager execution and the oracle."""
import sys

import numpy as np
import pytest

from gpu_util import (DecodeRunner, bf16_host, compare_decode, ragged_table,
                      seeded_normal_bf16, to_dev_bf16, to_dev_i32)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def L():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import loom_infer_hip as L
    return L


def log(msg):
    print(msg, flush=True)


@pytest.mark.parametrize("B,hq,hkv,lens,teams", [
    (5, 32, 8, [40, 1000, 17, 3000, 256], 7),  # balanced split-KV + merge kernel
    (1, 32, 32, [1024], 0),                    # direct plan split over 8 workgroups + merge
], ids=["balanced", "split_direct"])
def test_decode_graph_replays_match_eager_and_oracle(L, oracle, B, hq, hkv, lens, teams):
    """Replays with eager work and host synchronization between them; every
    replay is compared with the eager result (no memset nodes are captured; the
    split-KV workspace is scratch and needs no clearing between replays)."""
    import torch
    log(f"graph decode replay B={B} teams={teams}")
    rng = np.random.default_rng(21)
    pool = sum((x + 15) // 16 for x in lens) + 8
    indptr, indices, last = ragged_table(rng, lens, pool)
    q = seeded_normal_bf16(oracle, rng, B * hq * 128)
    k = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    ref_o, ref_l = oracle.paged_decode(oracle.paged_spec(B, pool, hq, hkv), q, k, v, indptr,
                                       indices, last)
    r = DecodeRunner(L, B, pool, hq, hkv, teams=teams)
    if teams == 0:
        assert r.plan.algorithm == "direct" and r.plan.info.teams == 8
    eager_o, eager_l = r.run(q, k, v, indptr, indices, last)
    compare_decode(oracle, eager_o, eager_l, ref_o, ref_l)

    tq, tk, tv = to_dev_bf16(q), to_dev_bf16(k), to_dev_bf16(v)
    tip, tix, tln = to_dev_i32(indptr), to_dev_i32(indices), to_dev_i32(last)
    out = torch.full((B * hq * 128,), float("nan"), dtype=torch.bfloat16, device="cuda")
    lse = torch.full((B * hq,), float("nan"), dtype=torch.float32, device="cuda")
    gq = L.GraphQueue(0, 1)
    b = gq.bindings(9)
    h = [b.bind_read(tq), b.bind_read(tk), b.bind_read(tv), b.bind_read(tip),
         b.bind_read(tix), b.bind_read(tln), b.bind_read_write(out), b.bind_read_write(lse),
         b.bind_read_write(r.workspace)]
    args = L.Bf16PagedBatchDecodeArgs(h[0], h[1], h[2], h[3], h[4], h[5], h[6].write(),
                                      h[7].write(), h[8].write())
    graph = gq.capture(b, lambda scope: r.plan.enqueue_into(scope, args))
    assert graph.commands() == 1
    # external owners dropped before replay: the graph's bindings keep them alive
    del tq, tk, tv, tip, tix, tln
    exec_ = graph.instantiate()
    # the captured kernel nodes relaunched in order (default), then the same
    # executable through hipGraphLaunch: every replay equals the eager call
    assert exec_.replay_mode == "kernel_nodes"
    for i in range(1, 7):
        if i == 4:
            exec_.set_replay_mode("hip_graph_launch")
            assert exec_.replay_mode == "hip_graph_launch"
        out.fill_(float("nan"))  # eager work between replays
        torch.cuda.synchronize()
        c = exec_.launch()
        assert c.launch_index() == i
        with pytest.raises(L.GraphError) as e:
            exec_.launch()
        assert e.value.variant == "ReplayInFlight"
        with pytest.raises(L.GraphError) as e:
            exec_.set_replay_mode("kernel_nodes")
        assert e.value.variant == "ReplayInFlight"
        c.wait()
        assert np.array_equal(bf16_host(out), eager_o), f"replay {i}"
        assert np.array_equal(lse.cpu().numpy(), eager_l), f"replay {i}"
    exec_.set_replay_mode("kernel_nodes")
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    ms = exec_.measure_launch_ms(start, end)
    assert ms > 0
    assert exec_.launches() == 7 and exec_.commands() == 1
    b = exec_.into_bindings()
    assert b.take_read_write(h[6]) is out


def test_full_decode_step_graph(L, oracle):
    """RoPE + 1-token append followed by paged decode, captured as one graph
    (BASELINE config 5 at reduced batch): replays reproduce the eager step."""
    import torch
    log("graph full decode step")
    rng = np.random.default_rng(55)
    B, hq, hkv = 8, 32, 8
    lens = np.clip(np.round(np.exp(np.log(2048) + 0.8 * rng.standard_normal(B))), 16,
                   16384).astype(int)
    pool = int(sum((x + 15) // 16 for x in lens)) + 16
    indptr, indices, last = ragged_table(rng, list(lens), pool)
    qn = seeded_normal_bf16(oracle, rng, B * hq * 128)
    kn = seeded_normal_bf16(oracle, rng, B * hkv * 128)
    vn = seeded_normal_bf16(oracle, rng, B * hkv * 128)
    kp = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    vp = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    # oracle step: append then decode with the rotated query
    s = oracle.paged_spec(B, pool, hq, hkv)
    ekp, evp = kp.copy(), vp.copy()
    eq = oracle.append(s, qn, kn, vn, indptr, indices, last, ekp, evp)
    ref_o, ref_l = oracle.paged_decode(s, eq, ekp, evp, indptr, indices, last)

    dec = DecodeRunner(L, B, pool, hq, hkv)
    ap = L.RopeProvider.load(0).plan_bf16_paged_append(L.Bf16RopePagedKvAppendSpec(B, pool, hq, hkv))
    aws = torch.zeros(ap.workspace_bytes, dtype=torch.uint8, device="cuda")
    t = dict(q=to_dev_bf16(qn), k=to_dev_bf16(kn), v=to_dev_bf16(vn), kp=to_dev_bf16(kp),
             vp=to_dev_bf16(vp), ip=to_dev_i32(indptr), ix=to_dev_i32(indices),
             ln=to_dev_i32(last))
    qrot = torch.empty(B * hq * 128, dtype=torch.bfloat16, device="cuda")
    out = torch.empty(B * hq * 128, dtype=torch.bfloat16, device="cuda")
    lse = torch.empty(B * hq, dtype=torch.float32, device="cuda")
    gq = L.GraphQueue(0, 2)
    b = gq.bindings(16)
    hq_, hk, hv = b.bind_read(t["q"]), b.bind_read(t["k"]), b.bind_read(t["v"])
    hip_, hix, hln = b.bind_read(t["ip"]), b.bind_read(t["ix"]), b.bind_read(t["ln"])
    hqr = b.bind_read_write(qrot)
    hkp, hvp = b.bind_read_write(t["kp"]), b.bind_read_write(t["vp"])
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
    assert exec_.replay_mode == "kernel_nodes"
    for i in range(6):
        if i == 3:  # the same executable through hipGraphLaunch
            exec_.set_replay_mode("hip_graph_launch")
        out.zero_()
        torch.cuda.synchronize()
        exec_.launch().wait()
        o, l = bf16_host(out), lse.cpu().numpy()
        st = compare_decode(oracle, o, l, ref_o, ref_l)
        log(f"  replay {i}: {st}")
        if i == 0:
            first = (o, l)
        else:
            assert np.array_equal(o, first[0]) and np.array_equal(l, first[1])
    exec_.into_bindings()


@pytest.mark.parametrize("cap", [200, 5000], ids=["fused_append", "chunked_append"])
def test_serving_loop_replays_one_graph_over_changing_page_tables(L, oracle, cap):
    """A decode step graph (one-token RoPE append + paged decode) captured once
    and replayed over 8 steps while the page table is rewritten in place:
    every request grows by one token per step and takes a new page when its
    last one fills.  The plans are made with LOOM_PLAN_PAGE_INDICES_CAPACITY,
    so the fixed page_indices buffer is a capacity and the entries past
    indptr[B] (left as garbage) are ignored.  Each replay is checked against
    the oracle's append + decode on host copies of the pools.  Steps 2 and 5
    first replay the graph over broken metadata, which must change nothing."""
    import torch
    log("graph serving loop with page-table updates")
    rng = np.random.default_rng(808)
    B, hq, hkv, pool = 4, 32, 8, 320
    lens = np.array([40, 15, 100, 64])
    free = list(rng.permutation(pool))
    pages = [[int(free.pop()) for _ in range((n + 15) // 16)] for n in lens]

    def table():
        indptr = np.concatenate([[0], np.cumsum([len(p) for p in pages])]).astype(np.int32)
        indices = np.concatenate(pages).astype(np.int32)
        last = np.array([n - (len(p) - 1) * 16 for n, p in zip(lens, pages)], np.int32)
        return indptr, indices, last

    kp_h = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    vp_h = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    dev = "cuda"
    t_kp, t_vp = to_dev_bf16(kp_h), to_dev_bf16(vp_h)
    t_ip = torch.zeros(B + 1, dtype=torch.int32, device=dev)
    t_ix = torch.full((cap,), -7, dtype=torch.int32, device=dev)
    t_ln = torch.zeros(B, dtype=torch.int32, device=dev)
    t_q = torch.zeros(B * hq * 128, dtype=torch.bfloat16, device=dev)
    t_k = torch.zeros(B * hkv * 128, dtype=torch.bfloat16, device=dev)
    t_v = torch.zeros(B * hkv * 128, dtype=torch.bfloat16, device=dev)
    qrot = torch.empty(B * hq * 128, dtype=torch.bfloat16, device=dev)
    out = torch.empty(B * hq * 128, dtype=torch.bfloat16, device=dev)
    lse = torch.empty(B * hq, dtype=torch.float32, device=dev)
    dspec = L.Bf16PagedBatchDecodeSpec(B, pool, hq, hkv, 128, 16)
    dplan = L.DecodeProvider.load(0).plan_bf16_paged_batch(dspec, max_total_pages=cap,
                                                           indices_capacity=True)
    aplan = L.RopeProvider.load(0).plan_bf16_paged_append(
        L.Bf16RopePagedKvAppendSpec(B, pool, hq, hkv), indices_capacity=True)
    dws = torch.zeros(dplan.workspace_bytes, dtype=torch.uint8, device=dev)
    aws = torch.zeros(aplan.workspace_bytes, dtype=torch.uint8, device=dev)
    gq = L.GraphQueue(0, 2)
    b = gq.bindings(16)
    hqn, hk, hv = b.bind_read(t_q), b.bind_read(t_k), b.bind_read(t_v)
    hip_, hix, hln = b.bind_read(t_ip), b.bind_read(t_ix), b.bind_read(t_ln)
    hqr, hkp, hvp = b.bind_read_write(qrot), b.bind_read_write(t_kp), b.bind_read_write(t_vp)
    hws_a, ho, hl = b.bind_read_write(aws), b.bind_read_write(out), b.bind_read_write(lse)
    hws_d = b.bind_read_write(dws)
    a_args = L.Bf16RopePagedKvAppendArgs(hqn, hk, hv, hip_, hix, hln, hqr.write(), hkp.write(),
                                         hvp.write(), hws_a.write())
    d_args = L.Bf16PagedBatchDecodeArgs(hqr.read(), hkp.read(), hvp.read(), hip_, hix, hln,
                                        ho.write(), hl.write(), hws_d.write())

    def record(scope):
        aplan.enqueue_into(scope, a_args)
        dplan.enqueue_into(scope, d_args)

    exec_ = gq.capture(b, record).instantiate()
    s = oracle.paged_spec(B, pool, hq, hkv)
    for step in range(8):
        lens += 1
        for r in range(B):
            if (lens[r] + 15) // 16 > len(pages[r]):
                pages[r].append(int(free.pop()))
        indptr, indices, last = table()
        qn = seeded_normal_bf16(oracle, rng, B * hq * 128)
        kn = seeded_normal_bf16(oracle, rng, B * hkv * 128)
        vn = seeded_normal_bf16(oracle, rng, B * hkv * 128)
        # rewrite the metadata and token inputs in place (fixed addresses)
        t_ip.copy_(torch.from_numpy(indptr))
        t_ix[: len(indices)].copy_(torch.from_numpy(indices))
        t_ix[len(indices):].fill_(-7)
        t_ln.copy_(torch.from_numpy(last))
        t_q.copy_(to_dev_bf16(qn))
        t_k.copy_(to_dev_bf16(kn))
        t_v.copy_(to_dev_bf16(vn))
        if step in (2, 5):
            # a replay over broken metadata (last_page_len 17) between valid
            # ones must leave the pools and the rotated queries untouched
            qrot_before = bf16_host(qrot)
            t_ln[0] = 17
            torch.cuda.synchronize()
            exec_.launch().wait()
            assert np.array_equal(bf16_host(t_kp), kp_h) and np.array_equal(bf16_host(t_vp), vp_h)
            assert np.array_equal(bf16_host(qrot), qrot_before)
            t_ln.copy_(torch.from_numpy(last))
            log(f"  step {step}: broken replay left every output untouched")
        torch.cuda.synchronize()
        exec_.launch().wait()
        eq = oracle.append(s, qn, kn, vn, indptr, indices, last, kp_h, vp_h)  # updates pools
        ref_o, ref_l = oracle.paged_decode(s, eq, kp_h, vp_h, indptr, indices, last)
        st = compare_decode(oracle, bf16_host(out), lse.cpu().numpy(), ref_o, ref_l)
        log(f"  step {step}: lens {lens.tolist()} pages {len(indices)} {st}")
    assert np.array_equal(bf16_host(t_vp), vp_h)
    exec_.into_bindings()


def test_fp8_decode_graph_replays_with_new_scales(L, oracle):
    """FP8 E4M3 decode on 32-row pages captured once; the per-tensor scales
    are a device operand, so replays after the caller rewrites them in place
    follow the new scales (each replay equals the eager command with the same
    scales, bit for bit)."""
    import torch
    from test_gpu_fp8 import dev_u8, random_fp8, run_decode
    log("graph fp8 decode replay")
    rng = np.random.default_rng(33)
    B, hq, hkv, P = 4, 16, 4, 32
    lens = [40, 700, 17, 300]
    pool = sum((x + P - 1) // P for x in lens) + 4
    pages = [(x + P - 1) // P for x in lens]
    indptr = np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)
    indices = rng.permutation(pool)[: indptr[-1]].astype(np.int32)
    last = np.array([x - (p - 1) * P for x, p in zip(lens, pages)], np.int32)
    q = seeded_normal_bf16(oracle, rng, B * hq * 128)
    k8 = random_fp8(rng, pool * P * hkv * 128, max_code=0x50)
    v8 = random_fp8(rng, pool * P * hkv * 128, max_code=0x50)
    spec = L.Bf16PagedBatchDecodeSpec(B, pool, hq, hkv, kv_dtype="fp8_e4m3", kv_page_size=P)
    opts = {"teams": 5}
    eager = [run_decode(L, spec, opts, q, k8, v8, indptr, indices, last, s)[:2]
             for s in ([0.5, 0.25], [0.125, 2.0])]
    plan = L.DecodeProvider.load(0).plan_bf16_paged_batch(spec, **opts)
    ws = torch.zeros(plan.workspace_bytes, dtype=torch.uint8, device="cuda")
    scales = torch.tensor([0.5, 0.25], dtype=torch.float32, device="cuda")
    out = torch.full((B * hq * 128,), float("nan"), dtype=torch.bfloat16, device="cuda")
    lse = torch.full((B * hq,), float("nan"), dtype=torch.float32, device="cuda")
    gq = L.GraphQueue(0, 1)
    b = gq.bindings(10)
    h = [b.bind_read(to_dev_bf16(q)), b.bind_read(dev_u8(k8)), b.bind_read(dev_u8(v8)),
         b.bind_read(to_dev_i32(indptr)), b.bind_read(to_dev_i32(indices)),
         b.bind_read(to_dev_i32(last)), b.bind_read_write(out), b.bind_read_write(lse),
         b.bind_read_write(ws), b.bind_read(scales)]
    args = L.Bf16PagedBatchDecodeArgs(h[0], h[1], h[2], h[3], h[4], h[5], h[6].write(),
                                      h[7].write(), h[8].write(), h[9])
    exec_ = gq.capture(b, lambda scope: plan.enqueue_into(scope, args)).instantiate()
    for i, (sc, (eo, el)) in enumerate(zip(([0.5, 0.25], [0.125, 2.0], [0.5, 0.25]),
                                           eager + eager[:1])):
        scales.copy_(torch.tensor(sc, dtype=torch.float32))  # eager work between replays
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        exec_.launch().wait()
        assert np.array_equal(bf16_host(out), eo), f"replay {i}"
        assert np.array_equal(lse.cpu().numpy(), el), f"replay {i}"
