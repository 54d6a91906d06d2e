"""The chunk-validated append never fails silently.

The one-launch append makes its token workgroups wait (bounded) for the
validation workgroups' verdicts, and workgroup 0 waits (bounded) for every
workgroup to start before it advances the workspace's epoch.  A wait that
gives up is reported through the command queue's device status words when the
completion settles (CommandError DeviceStatus, the queue poisoned), and a
workspace whose epoch handover gave up is marked broken, so every later
command on it writes nothing and reports that too, until it is zeroed.

The give-up is forced from the host with the test-only plan option
PLAN_APPEND_TEST_NO_WAIT (every bounded wait gives up at once), so every
kernel still exits normally.  The reference's contract for invalid metadata
(rope/mod.rs:407-466: nothing written) and its poisoning of a queue whose
submission failed (command/submission.rs:221-279) are the model.

Also here: the two-launch plan option (validation kernel, then apply kernel)
sharing one workspace with one-launch commands."""
import sys

import numpy as np
import pytest

from gpu_util import bf16_host, nan_bf16, to_dev_bf16, to_dev_i32
from test_gpu_append import check_rope, explicit_case

pytestmark = pytest.mark.gpu

VERDICT_WAIT, HANDOVER, REFUSED = 1, 2, 4
T, LONG_PAGES = 300, 4200  # chunk-validated path


@pytest.fixture(scope="module")
def L():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import loom_infer_hip as L
    return L


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def ws_words(ws):
    w = ws.cpu().numpy().view(np.uint32)
    return int(w[0]) | int(w[1]) << 32, int(w[2])


def submit(L, queue, plan, c, ws=None, graph=None):
    """One explicit-token command on `queue` (or captured on GraphQueue
    `graph`); returns (outputs, error or None).  Outputs are read from the
    device tensors whatever the completion reports."""
    import torch
    dev = dict(q=to_dev_bf16(c["q"]), k=to_dev_bf16(c["k"]), v=to_dev_bf16(c["v"]),
               bi=to_dev_i32(c["bi"]), pos=to_dev_i32(c["pos"]), ip=to_dev_i32(c["indptr"]),
               ix=to_dev_i32(c["indices"]), ln=to_dev_i32(c["last"]),
               kp=to_dev_bf16(c["kp"]), vp=to_dev_bf16(c["vp"]))
    qo = nan_bf16(len(c["bi"]) * c["hq"] * 128)
    b = (graph or queue).bindings(13)
    h = [b.bind_read(dev[n]) for n in ("q", "k", "v", "bi", "pos", "ip", "ix", "ln")]
    hqo, hkp, hvp = b.bind_read_write(qo), b.bind_read_write(dev["kp"]), b.bind_read_write(dev["vp"])
    hws = b.bind_read_write(ws) if ws is not None else None
    args = L.Bf16RopePagedKvAppendTokensArgs(*h, hqo.write(), hkp.write(), hvp.write(),
                                             hws.write() if hws else None)
    err = None
    if graph is None:
        scope = queue.begin(b)
        plan.enqueue_into(scope, args)
        comp = scope.finish()
        try:
            comp.wait()
        except L.LoomError as e:
            err = e
    else:
        exec_ = graph.capture(b, lambda scope: plan.enqueue_into(scope, args)).instantiate()
        try:
            exec_.launch().wait()
        except L.LoomError as e:
            err = e
        queue.append(exec_)  # the caller inspects the poisoned executable
    torch.cuda.synchronize()
    return [bf16_host(x) for x in (qo, dev["kp"], dev["vp"])], err


def untouched(oracle, c, out):
    qo, kp, vp = out
    return (bool(np.all(np.isnan(oracle.bf16_to_f32(qo)))) and np.array_equal(kp, c["kp"])
            and np.array_equal(vp, c["vp"]))


def expected(oracle, c):
    s = oracle.paged_spec(c["B"], c["pool"], c["hq"], c["hkv"])
    ekp, evp = c["kp"].copy(), c["vp"].copy()
    eq = oracle.append_tokens(s, len(c["bi"]), c["q"], c["k"], c["v"], c["bi"], c["pos"],
                              c["indptr"], c["indices"], c["last"], ekp, evp, max_tokens=8192)
    return eq, ekp, evp


def check_valid(oracle, c, out, want):
    qo, kp, vp = out
    eq, ekp, evp = want
    check_rope(oracle, qo, eq, c["q"], np.repeat(c["pos"], c["hq"]), "query")
    assert np.array_equal(vp, evp)


def device_status(e):
    assert e is not None, "the command reported success"
    assert e.variant == "DeviceStatus", e
    return int(e.fields[0])


def forced_bits_ok(bits):
    """A forced give-up: the handover gave up (workgroup 0 marks the workspace
    broken), and the token workgroups either gave up their verdict wait or,
    having started after workgroup 0 marked the workspace, were refused."""
    return bits & HANDOVER and bits & (VERDICT_WAIT | REFUSED) and not bits & ~7


def test_forced_give_up_fails_loudly_and_breaks_the_workspace(L, oracle):
    import torch
    c = explicit_case(oracle, 11, T, LONG_PAGES, "valid")
    want = expected(oracle, c)
    spec = L.Bf16RopePagedKvAppendTokensSpec.extended(T, c["B"], c["pool"], c["hq"], c["hkv"])
    prov = L.RopeProvider.load(0)
    forced = prov.plan_bf16_paged_append_tokens(spec, flags=L.PLAN_APPEND_TEST_NO_WAIT)
    normal = prov.plan_bf16_paged_append_tokens(spec)
    two = prov.plan_bf16_paged_append_tokens(spec, flags=L.PLAN_APPEND_TWO_LAUNCH)
    ws = torch.zeros(normal.workspace_bytes, dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream()

    log("forced give-up: every wait gives up at once")
    q1 = L.CommandQueue(stream, 1)
    out, err = submit(L, q1, forced, c, ws)
    bits = device_status(err)
    log(f"  {err}")
    assert forced_bits_ok(bits), bits
    assert q1.poisoned
    assert untouched(oracle, c, out), "a token workgroup that gave up wrote"
    epoch, broken = ws_words(ws)
    assert (epoch, broken) == (0, 1), (epoch, broken)
    b = q1.bindings(1)
    with pytest.raises(L.CommandError) as e:
        q1.begin(b)
    assert e.value.variant == "QueuePoisoned"

    log("a broken workspace refuses every later command (one- and two-launch)")
    for plan, what in ((normal, "one-launch"), (two, "two-launch")):
        q = L.CommandQueue(stream, 1)
        out, err = submit(L, q, plan, c, ws)
        assert device_status(err) == REFUSED, (what, err)
        assert q.poisoned
        assert untouched(oracle, c, out), what
        assert ws_words(ws) == (0, 1)

    log("zeroed again, the workspace serves valid commands")
    ws.zero_()
    for i, plan in enumerate((normal, two, normal)):
        q = L.CommandQueue(stream, 1)
        out, err = submit(L, q, plan, c, ws)
        assert err is None, err
        assert not q.poisoned
        check_valid(oracle, c, out, want)
    assert ws_words(ws) == (2, 0)


def test_forced_give_up_on_invalid_metadata_writes_nothing(L, oracle):
    """A give-up on a command that is also invalid: still nothing written."""
    import torch
    c = explicit_case(oracle, 12, T, LONG_PAGES, "duplicate_far")
    spec = L.Bf16RopePagedKvAppendTokensSpec.extended(T, c["B"], c["pool"], c["hq"], c["hkv"])
    forced = L.RopeProvider.load(0).plan_bf16_paged_append_tokens(
        spec, flags=L.PLAN_APPEND_TEST_NO_WAIT)
    ws = torch.zeros(forced.workspace_bytes, dtype=torch.uint8, device="cuda")
    q = L.CommandQueue(torch.cuda.current_stream(), 1)
    out, err = submit(L, q, forced, c, ws)
    assert forced_bits_ok(device_status(err))
    assert untouched(oracle, c, out)


def test_forced_give_up_reference_shaped_poisons_the_queue(L, oracle):
    """The reference-shaped args (queue-owned workspace): the completion
    fails, the queue is poisoned; a new queue (fresh workspace) runs the same
    command correctly."""
    import torch
    c = explicit_case(oracle, 13, T, LONG_PAGES, "valid")
    want = expected(oracle, c)
    spec = L.Bf16RopePagedKvAppendTokensSpec.extended(T, c["B"], c["pool"], c["hq"], c["hkv"])
    prov = L.RopeProvider.load(0)
    forced = prov.plan_bf16_paged_append_tokens(spec, flags=L.PLAN_APPEND_TEST_NO_WAIT)
    normal = prov.plan_bf16_paged_append_tokens(spec)
    stream = torch.cuda.current_stream()
    q = L.CommandQueue(stream, 2)
    out, err = submit(L, q, forced, c)
    assert forced_bits_ok(device_status(err))
    assert q.poisoned and untouched(oracle, c, out)
    q2 = L.CommandQueue(stream, 2)
    for _ in range(2):
        out, err = submit(L, q2, normal, c)
        assert err is None, err
        check_valid(oracle, c, out, want)


def test_forced_give_up_in_a_graph_poisons_the_execution(L, oracle):
    import torch
    c = explicit_case(oracle, 14, T, LONG_PAGES, "valid")
    spec = L.Bf16RopePagedKvAppendTokensSpec.extended(T, c["B"], c["pool"], c["hq"], c["hkv"])
    forced = L.RopeProvider.load(0).plan_bf16_paged_append_tokens(
        spec, flags=L.PLAN_APPEND_TEST_NO_WAIT)
    ws = torch.zeros(forced.workspace_bytes, dtype=torch.uint8, device="cuda")
    execs = []
    out, err = submit(L, execs, forced, c, ws, graph=L.GraphQueue(0, 1))
    assert forced_bits_ok(device_status(err))
    assert untouched(oracle, c, out)
    with pytest.raises(L.GraphError) as e:
        execs[0].launch()
    assert e.value.variant == "ExecutionPoisoned"


def test_one_and_two_launch_commands_share_a_workspace(L, oracle):
    """Both forms on one workspace, valid and invalid commands interleaved:
    the two-launch form leaves the epoch alone and empties the hash table it
    used, so neither form sees the other's verdicts or slot keys."""
    import torch
    cases = {brk: explicit_case(oracle, 15, T, LONG_PAGES, brk)
             for brk in ("valid", "duplicate_far", "page_index")}
    c = cases["valid"]
    want = expected(oracle, c)
    spec = L.Bf16RopePagedKvAppendTokensSpec.extended(T, c["B"], c["pool"], c["hq"], c["hkv"])
    prov = L.RopeProvider.load(0)
    plans = {"one": prov.plan_bf16_paged_append_tokens(spec),
             "two": prov.plan_bf16_paged_append_tokens(spec, flags=L.PLAN_APPEND_TWO_LAUNCH)}
    ws = torch.zeros(plans["one"].workspace_bytes, dtype=torch.uint8, device="cuda")
    q = L.CommandQueue(torch.cuda.current_stream(), 1)
    epoch = 0
    first = None
    seq = [("one", "valid"), ("two", "valid"), ("two", "duplicate_far"), ("one", "valid"),
           ("one", "duplicate_far"), ("two", "valid"), ("two", "page_index"), ("one", "valid"),
           ("two", "valid")]
    for i, (form, brk) in enumerate(seq):
        log(f"shared workspace command {i}: {form}-launch {brk}")
        x = cases[brk]
        out, err = submit(L, q, plans[form], x, ws)
        assert err is None, err
        epoch += form == "one"
        assert ws_words(ws) == (epoch, 0), i
        if brk != "valid":
            assert untouched(oracle, x, out), i
        elif first is None:
            check_valid(oracle, c, out, want)
            first = out
        else:
            assert all(np.array_equal(a, b) for a, b in zip(out, first)), i
