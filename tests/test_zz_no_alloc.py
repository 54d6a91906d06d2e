"""The allocation-free paged-decode entry point
(loom_paged_decode_enqueue_bf16_no_alloc, no reference counterpart): its
split-KV workspace is the library's static per-device scratch.  Checked
against the caller-workspace entry point (loom_paged_decode_enqueue) bit for
bit on two calls in a row, the second with a smaller input, so the second
runs over the first call's scratch contents."""
import gc
import sys

import numpy as np
import pytest

from gpu_util import (DecodeRunner, bf16_host, nan_bf16, ragged_table, seeded_normal_bf16,
                      to_dev_bf16, to_dev_i32)

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


def no_alloc_call(L, r, q, k, v, ip, ix, ln):
    import torch
    out = nan_bf16(r.spec.output_numel)
    lse = torch.full((r.spec.lse_numel,), float("nan"), dtype=torch.float32, device="cuda")
    b = r.queue.bindings(8)
    h = [b.bind_read(x) for x in (to_dev_bf16(q), to_dev_bf16(k), to_dev_bf16(v),
                                  to_dev_i32(ip), to_dev_i32(ix), to_dev_i32(ln))]
    ho, hl = b.bind_read_write(out), b.bind_read_write(lse)
    scope = r.queue.begin(b)
    r.plan.enqueue_into_no_alloc(scope, L.Bf16PagedBatchDecodeArgs(*h, ho.write(), hl.write()))
    comp = scope.finish()
    assert comp.submitted() == 1
    b = comp.wait()
    return bf16_host(b.take_read_write(ho)), b.take_read_write(hl).cpu().numpy()


def test_no_alloc_matches_workspace_entry_point(L, oracle):
    import torch
    rng = np.random.default_rng(77)
    hq, hkv = 32, 8
    cases = [  # (lens, teams): the second call is smaller than the first
        ([3000, 40, 8000, 17, 1000, 2049, 5, 600], 0),
        ([700, 33, 1500], 0),
        ([1024], 0),  # the direct algorithm split over 8 workgroups (split states)
        ([90, 15], 0),  # the direct algorithm (no split states)
    ]
    for i, (lens, teams) in enumerate(cases):
        B = len(lens)
        pool = sum((x + 15) // 16 for x in lens) + 7
        ip, ix, ln = ragged_table(rng, lens, pool)
        q = seeded_normal_bf16(oracle, rng, B * hq * 128)
        k = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
        v = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
        log(f"no-alloc call {i}: batch {B}, {int(ip[-1])} pages")
        r = DecodeRunner(L, B, pool, hq, hkv, teams=teams)
        if lens == [1024]:
            assert r.plan.algorithm == "direct" and r.plan.info.teams == 8
        want_o, want_l = r.run(q, k, v, ip, ix, ln)
        got_o, got_l = no_alloc_call(L, r, q, k, v, ip, ix, ln)
        assert np.array_equal(got_o, want_o), f"call {i}: output"
        assert np.array_equal(got_l, want_l), f"call {i}: lse"
        log(f"  {r.plan.algorithm} (teams {r.plan.info.teams}), workspace {r.plan.workspace_bytes} B: bit-equal")
    torch.cuda.synchronize()


def test_no_alloc_rejects_plans_beyond_the_scratch(L):
    import torch
    # 2048 requests x 64 query heads of split states exceed 32 MiB
    spec = L.Bf16PagedBatchDecodeSpec(2048, 2048, 64, 8)
    plan = L.DecodeProvider.load(0).plan_bf16_paged_batch(spec)
    assert plan.workspace_bytes > 32 << 20
    queue = L.CommandQueue(torch.cuda.current_stream(), 1)
    b = queue.bindings(8)
    z = lambda n, dt: torch.zeros(n, dtype=dt, device="cuda")  # noqa: E731
    h = [b.bind_read(z(spec.query_numel, torch.bfloat16)),
         b.bind_read(z(spec.kv_pages_numel, torch.bfloat16)),
         b.bind_read(z(spec.kv_pages_numel, torch.bfloat16)),
         b.bind_read(z(2049, torch.int32)), b.bind_read(z(2048, torch.int32)),
         b.bind_read(z(2048, torch.int32))]
    ho = b.bind_read_write(z(spec.output_numel, torch.bfloat16))
    hl = b.bind_read_write(z(spec.lse_numel, torch.float32))
    scope = queue.begin(b)
    with pytest.raises(L.EnqueueError) as e:
        plan.enqueue_into_no_alloc(scope, L.Bf16PagedBatchDecodeArgs(*h, ho.write(), hl.write()))
    assert e.value.variant == "StaticScratchTooSmall"
    comp = scope.finish()
    assert comp.submitted() == 0
    comp.wait()


def test_no_alloc_from_another_stream_while_busy_is_rejected(L, oracle):
    """An eager allocation-free call on a second stream while the device's
    previous one (queued behind a bounded spin kernel on the first stream)
    has not finished is rejected with StaticScratchBusy and enqueues
    nothing; once the first completes, the same call runs and matches the
    caller-workspace entry point bit for bit."""
    import torch
    rng = np.random.default_rng(78)
    hq, hkv = 32, 8
    lens = [3000, 40, 8000, 17]
    B = len(lens)
    pool = sum((x + 15) // 16 for x in lens) + 7
    ip, ix, ln = ragged_table(rng, lens, pool)
    q = seeded_normal_bf16(oracle, rng, B * hq * 128)
    k = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    r = DecodeRunner(L, B, pool, hq, hkv)
    want_o, want_l = r.run(q, k, v, ip, ix, ln)
    ins = [to_dev_bf16(q), to_dev_bf16(k), to_dev_bf16(v), to_dev_i32(ip), to_dev_i32(ix),
           to_dev_i32(ln)]
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    q1, q2 = L.CommandQueue(s1, 1), L.CommandQueue(s2, 1)
    outs = [(nan_bf16(r.spec.output_numel),
             torch.full((r.spec.lse_numel,), float("nan"), dtype=torch.float32, device="cuda"))
            for _ in range(3)]
    torch.cuda.synchronize()

    def enqueue(queue, i):
        out, lse = outs[i]
        b = queue.bindings(8)
        h = [b.bind_read(x) for x in ins]
        ho, hl = b.bind_read_write(out), b.bind_read_write(lse)
        scope = queue.begin(b)
        err = None
        try:
            r.plan.enqueue_into_no_alloc(scope, L.Bf16PagedBatchDecodeArgs(*h, ho.write(), hl.write()))
        except L.EnqueueError as e:
            err = e
        return scope.finish(), ho, hl, err

    # Nothing may synchronize the device while stream 1 is held: freeing a
    # command queue does (hipFree of its workspaces), so earlier tests'
    # garbage is collected first and the collector is off until the check.
    gc.collect()
    gc.disable()
    try:
        log("stream 1: spin kernel, then an allocation-free decode behind it")
        with torch.cuda.stream(s1):
            torch.cuda._sleep(50_000_000)  # bounded spin (tens of ms)
        c1, ho1, hl1, e1 = enqueue(q1, 0)
        assert e1 is None and c1.submitted() == 1
        log("stream 2 while stream 1's command is pending: rejected")
        c2, _, _, e2 = enqueue(q2, 1)
    finally:
        gc.enable()
    assert e2 is not None and e2.variant == "StaticScratchBusy", e2
    assert c2.submitted() == 0
    c2.wait()
    b1 = c1.wait()
    assert np.array_equal(bf16_host(b1.take_read_write(ho1)), want_o)
    log("stream 2 after stream 1 finished: runs")
    c3, ho3, hl3, e3 = enqueue(q2, 2)
    assert e3 is None and c3.submitted() == 1
    b3 = c3.wait()
    assert np.array_equal(bf16_host(b3.take_read_write(ho3)), want_o)
    assert np.array_equal(b3.take_read_write(hl3).cpu().numpy(), want_l)
    torch.cuda.synchronize()
