"""The reference's own argument structs through the C ABI.

* Bf16PagedBatchDecodeArgs (decode.rs:1452-1487, eight operands) and
  Bf16RopePagedKvAppend{,Tokens}Args (rope/mod.rs:963-1047) enqueue unchanged:
  the split-KV states and the append validation words live in a workspace the
  command queue owns.  Results equal the caller-workspace form bit for bit,
  eagerly and under graph capture.
* Operands on 4-byte boundaries (the reference's alignment contract,
  decode.rs:1585-1600, prefill.rs:3015-3029; the append checks none) give the
  same bits as 16-byte-aligned ones."""
import sys

import numpy as np
import pytest

from gpu_util import (DecodeRunner, PrefillRunner, RaggedRunner, bf16_host, compare_decode,
                      nan_bf16, ragged_table, seeded_normal_bf16, to_dev_bf16, to_dev_i32)

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


def shifted(t, elems):
    """A copy of device tensor `t` starting `elems` elements into a larger
    allocation (so its address is only 2*elems-byte aligned)."""
    import torch
    big = torch.empty(t.numel() + 16, dtype=t.dtype, device=t.device)
    v = big[elems:elems + t.numel()]
    v.copy_(t)
    return v


def decode_case(oracle, rng, B, hq, hkv, lens):
    pool = sum((x + 15) // 16 for x in lens) + 5
    indptr, indices, last = ragged_table(rng, lens, pool)
    q = seeded_normal_bf16(oracle, rng, B * hq * 128)
    k = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    return pool, (q, k, v, indptr, indices, last)


def run_decode_reference_args(L, queue, plan, spec, q, k, v, ip, ix, ln):
    """The reference's call sequence with its eight-operand args."""
    import torch
    out = nan_bf16(spec.output_numel)
    lse = torch.full((spec.lse_numel,), float("nan"), dtype=torch.float32, device="cuda")
    b = queue.bindings(8)
    h = [b.bind_read(x) for x in (q, k, v, ip, ix, ln)]
    ho, hl = b.bind_read_write(out), b.bind_read_write(lse)
    args = L.Bf16PagedBatchDecodeArgs(*h, ho.write(), hl.write())
    assert args.reference_shaped
    scope = queue.begin(b)
    plan.enqueue_into(scope, args)
    comp = scope.finish()
    assert comp.submitted() == 1
    b = comp.wait()
    return bf16_host(b.take_read_write(ho)), b.take_read_write(hl).cpu().numpy()


@pytest.mark.parametrize("name,B,hq,hkv,lens,teams", [
    ("direct_gqa4", 4, 16, 4, [3, 32, 17, 41], 0),
    ("balanced_gqa4", 5, 32, 8, [40, 1000, 17, 3000, 256], 7),
    ("balanced_gqa8_default", 3, 64, 8, [2049, 700, 5000], 0),
], ids=lambda x: x if isinstance(x, str) else None)
def test_decode_reference_args_use_the_queue_workspace(L, oracle, name, B, hq, hkv, lens, teams):
    import torch
    log(f"reference-shaped decode {name}")
    rng = np.random.default_rng(len(name))
    pool, (q, k, v, ip, ix, ln) = decode_case(oracle, rng, B, hq, hkv, lens)
    ref_o, ref_l = oracle.paged_decode(oracle.paged_spec(B, pool, hq, hkv), q, k, v, ip, ix, ln)
    r = DecodeRunner(L, B, pool, hq, hkv, teams=teams)
    want_o, want_l = r.run(q, k, v, ip, ix, ln)
    queue = L.CommandQueue(torch.cuda.current_stream(), 2)
    # the queue holds its append validation workspace from creation, no scratch
    base = queue.workspace_bytes
    assert base == append_workspace_bytes(L)
    dev = [to_dev_bf16(q), to_dev_bf16(k), to_dev_bf16(v), to_dev_i32(ip), to_dev_i32(ix),
           to_dev_i32(ln)]
    for i in range(2):  # the second command reuses the workspace the first allocated
        o, l_ = run_decode_reference_args(L, queue, r.plan, r.spec, *dev)
        assert np.array_equal(o, want_o) and np.array_equal(l_, want_l), f"call {i}"
        assert queue.workspace_bytes >= base + r.plan.workspace_bytes
    log(f"  {r.plan.algorithm} queue workspace {queue.workspace_bytes} B "
        f"{compare_decode(oracle, o, l_, ref_o, ref_l)}")


def append_workspace_bytes(L):
    spec = L.Bf16RopePagedKvAppendSpec(1, 1, 1, 1)
    return L.RopeProvider.load(0).plan_bf16_paged_append(spec).workspace_bytes


def test_reserved_workspace_is_not_regrown(L, oracle):
    import torch
    rng = np.random.default_rng(9)
    B, hq, hkv = 3, 32, 8
    pool, (q, k, v, ip, ix, ln) = decode_case(oracle, rng, B, hq, hkv, [300, 2000, 45])
    r = DecodeRunner(L, B, pool, hq, hkv, teams=5)
    want_o, want_l = r.run(q, k, v, ip, ix, ln)
    queue = L.CommandQueue(torch.cuda.current_stream(), 2)
    queue.reserve_workspace(scratch_bytes=r.plan.workspace_bytes)
    reserved = queue.workspace_bytes
    assert reserved >= r.plan.workspace_bytes
    dev = [to_dev_bf16(q), to_dev_bf16(k), to_dev_bf16(v), to_dev_i32(ip), to_dev_i32(ix),
           to_dev_i32(ln)]
    o, l_ = run_decode_reference_args(L, queue, r.plan, r.spec, *dev)
    assert np.array_equal(o, want_o) and np.array_equal(l_, want_l)
    assert queue.workspace_bytes == reserved


def test_fp8_plan_rejects_reference_args(L):
    import torch
    spec = L.Bf16PagedBatchDecodeSpec(2, 8, 8, 2, kv_dtype="fp8_e4m3")
    plan = L.DecodeProvider.load(0).plan_bf16_paged_batch(spec)
    queue = L.CommandQueue(torch.cuda.current_stream(), 1)
    b = queue.bindings(8)
    u8 = lambda n: torch.zeros(n, dtype=torch.uint8, device="cuda")  # noqa: E731
    h = [b.bind_read(torch.zeros(spec.query_numel, dtype=torch.bfloat16, device="cuda")),
         b.bind_read(u8(spec.kv_pages_numel)), b.bind_read(u8(spec.kv_pages_numel)),
         b.bind_read(to_dev_i32([0, 1, 2])), b.bind_read(to_dev_i32([0, 1])),
         b.bind_read(to_dev_i32([16, 16]))]
    ho = b.bind_read_write(torch.zeros(spec.output_numel, dtype=torch.bfloat16, device="cuda"))
    hl = b.bind_read_write(torch.zeros(spec.lse_numel, dtype=torch.float32, device="cuda"))
    scope = queue.begin(b)
    with pytest.raises(L.EnqueueError) as e:
        plan.enqueue_into(scope, L.Bf16PagedBatchDecodeArgs(*h, ho.write(), hl.write()))
    assert (e.value.variant, e.value.operand) == ("LengthMismatch", "kv_scales")
    comp = scope.finish()
    assert comp.submitted() == 0
    comp.wait()


def append_inputs(oracle, rng, B, hq, hkv, lens, T=None):
    pool = sum((x + 15) // 16 for x in lens) + 3
    indptr, indices, last = ragged_table(rng, lens, pool)
    n = B if T is None else T
    q = seeded_normal_bf16(oracle, rng, n * hq * 128)
    k = seeded_normal_bf16(oracle, rng, n * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, n * hkv * 128)
    kp = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    vp = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    return pool, (q, k, v, indptr, indices, last, kp, vp)


def run_append(L, queue, plan, spec, tokens, inputs, bi=None, pos=None, workspace=None,
               shift=0):
    """One append command; `shift` moves every BF16 operand `shift` elements
    off its allocation's alignment."""
    import torch
    q, k, v, ip, ix, ln, kp, vp = inputs
    dq, dk, dv, dkp, dvp = (to_dev_bf16(x) for x in (q, k, v, kp, vp))
    qo = nan_bf16(tokens * spec.num_query_heads * 128)
    if shift:
        dq, dk, dv, dkp, dvp, qo = (shifted(x, shift) for x in (dq, dk, dv, dkp, dvp, qo))
    b = queue.bindings(13)
    hq_, hk, hv = b.bind_read(dq), b.bind_read(dk), b.bind_read(dv)
    hbi = b.bind_read(to_dev_i32(bi)) if bi is not None else None
    hpos = b.bind_read(to_dev_i32(pos)) if pos is not None else None
    hip_, hix, hln = b.bind_read(to_dev_i32(ip)), b.bind_read(to_dev_i32(ix)), b.bind_read(
        to_dev_i32(ln))
    hqo, hkp, hvp = b.bind_read_write(qo), b.bind_read_write(dkp), b.bind_read_write(dvp)
    hws = b.bind_read_write(workspace) if workspace is not None else None
    if bi is None:
        args = L.Bf16RopePagedKvAppendArgs(hq_, hk, hv, hip_, hix, hln, hqo.write(), hkp.write(),
                                           hvp.write(), hws.write() if hws else None)
    else:
        args = L.Bf16RopePagedKvAppendTokensArgs(hq_, hk, hv, hbi, hpos, hip_, hix, hln,
                                                 hqo.write(), hkp.write(), hvp.write(),
                                                 hws.write() if hws else None)
    assert args.reference_shaped == (workspace is None)
    scope = queue.begin(b)
    plan.enqueue_into(scope, args)
    comp = scope.finish()
    assert comp.submitted() == 1
    b = comp.wait()
    return [bf16_host(b.take_read_write(h)) for h in (hqo, hkp, hvp)]


@pytest.mark.parametrize("form", ["one_token_fused", "one_token_chunked", "tokens_fused",
                                  "tokens_chunked"])
def test_append_reference_args_equal_workspace_form(L, oracle, form):
    import torch
    log(f"reference-shaped append {form}")
    rng = np.random.default_rng(len(form))
    hq, hkv = 16, 4
    chunked = form.endswith("chunked")
    B = 80 if chunked else 4  # more than 64 tokens: chunked validation
    lens = list(rng.integers(1, 200, size=B))
    prov = L.RopeProvider.load(0)
    queue = L.CommandQueue(torch.cuda.current_stream(), 2)
    if form.startswith("one_token"):
        pool, inputs = append_inputs(oracle, rng, B, hq, hkv, lens)
        spec = L.Bf16RopePagedKvAppendSpec(B, pool, hq, hkv)
        plan = prov.plan_bf16_paged_append(spec)
        T, bi, pos = B, None, None
    else:
        T = 70 if chunked else 6
        bi = rng.integers(0, B, size=T).astype(np.int32)
        lens = [x + 2 for x in lens]
        pos = np.array([rng.integers(0, lens[b]) for b in bi], np.int32)
        # distinct slots: one token per (request, position)
        keep = np.unique(np.stack([bi, pos], 1), axis=0, return_index=True)[1]
        bi, pos = bi[np.sort(keep)], pos[np.sort(keep)]
        T = len(bi)
        pool, inputs = append_inputs(oracle, rng, B, hq, hkv, lens, T)
        if T <= 64:
            spec = L.Bf16RopePagedKvAppendTokensSpec(T, B, pool, hq, hkv)
        else:
            spec = L.Bf16RopePagedKvAppendTokensSpec.extended(T, B, pool, hq, hkv)
        plan = prov.plan_bf16_paged_append_tokens(spec)
    ws = torch.zeros(plan.workspace_bytes, dtype=torch.uint8, device="cuda")
    want = run_append(L, queue, plan, spec, T, inputs, bi, pos, workspace=ws)
    for i in range(2):
        got = run_append(L, queue, plan, spec, T, inputs, bi, pos)
        for g, w, n in zip(got, want, ("query_output", "key_pages", "value_pages")):
            assert np.array_equal(g, w), f"call {i}: {n}"
    assert queue.workspace_bytes >= plan.workspace_bytes
    # and on 2-byte boundaries (the reference's append checks no alignment)
    got = run_append(L, queue, plan, spec, T, inputs, bi, pos, shift=1)
    for g, w, n in zip(got, want, ("query_output", "key_pages", "value_pages")):
        assert np.array_equal(g, w), f"2-byte aligned: {n}"


def test_decode_step_graph_with_reference_args(L, oracle):
    """Append + decode captured as one graph with the reference's args: the
    graph queue's workspaces move into the executable with its commands;
    replays equal the eager step on the caller-workspace forms."""
    import torch
    log("reference-shaped decode step graph")
    rng = np.random.default_rng(123)
    B, hq, hkv = 6, 32, 8
    lens = [40, 1000, 17, 3000, 256, 129]
    pool, (qn, kn, vn, ip, ix, ln, kp, vp) = append_inputs(oracle, rng, B, hq, hkv, lens)
    dspec = L.Bf16PagedBatchDecodeSpec(B, pool, hq, hkv)
    dplan = L.DecodeProvider.load(0).plan_bf16_paged_batch(dspec, teams=9)
    aplan = L.RopeProvider.load(0).plan_bf16_paged_append(
        L.Bf16RopePagedKvAppendSpec(B, pool, hq, hkv))
    # eager, caller workspaces
    s = oracle.paged_spec(B, pool, hq, hkv)
    ekp, evp = kp.copy(), vp.copy()
    eq = oracle.append(s, qn, kn, vn, ip, ix, ln, ekp, evp)
    ref_o, ref_l = oracle.paged_decode(s, eq, ekp, evp, ip, ix, ln)

    t = dict(q=to_dev_bf16(qn), k=to_dev_bf16(kn), v=to_dev_bf16(vn), kp=to_dev_bf16(kp),
             vp=to_dev_bf16(vp), ip=to_dev_i32(ip), ix=to_dev_i32(ix), ln=to_dev_i32(ln))
    qrot = torch.empty(B * hq * 128, dtype=torch.bfloat16, device="cuda")
    out = torch.empty(B * hq * 128, dtype=torch.bfloat16, device="cuda")
    lse = torch.empty(B * hq, dtype=torch.float32, device="cuda")
    gq = L.GraphQueue(0, 2)
    # the capture allocates nothing: the decode's split-KV workspace is
    # reserved first (the append's is held from queue creation)
    gq.reserve_workspace(scratch_bytes=dplan.workspace_bytes)
    reserved = gq.workspace_bytes
    b = gq.bindings(14)
    hq_, hk, hv = b.bind_read(t["q"]), b.bind_read(t["k"]), b.bind_read(t["v"])
    hip_, hix, hln = b.bind_read(t["ip"]), b.bind_read(t["ix"]), b.bind_read(t["ln"])
    hqr, hkp, hvp = b.bind_read_write(qrot), b.bind_read_write(t["kp"]), b.bind_read_write(t["vp"])
    ho, hl = b.bind_read_write(out), b.bind_read_write(lse)
    a_args = L.Bf16RopePagedKvAppendArgs(hq_, hk, hv, hip_, hix, hln, hqr.write(), hkp.write(),
                                         hvp.write())
    d_args = L.Bf16PagedBatchDecodeArgs(hqr.read(), hkp.read(), hvp.read(), hip_, hix, hln,
                                        ho.write(), hl.write())

    def record(scope):
        aplan.enqueue_into(scope, a_args)
        dplan.enqueue_into(scope, d_args)

    captured = gq.capture(b, record)
    assert reserved >= dplan.workspace_bytes + aplan.workspace_bytes
    exec_ = captured.instantiate()
    first = None
    for i in range(4):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        exec_.launch().wait()
        o, l_ = bf16_host(out), lse.cpu().numpy()
        if first is None:
            log(f"  replay 0 {compare_decode(oracle, o, l_, ref_o, ref_l)}")
            first = (o, l_)
        else:
            assert np.array_equal(o, first[0]) and np.array_equal(l_, first[1]), f"replay {i}"
    assert np.array_equal(bf16_host(t["vp"]), evp)
    exec_.into_bindings()


def test_four_byte_aligned_operands_decode_and_prefill(L, oracle):
    """Q, K/V, O (and LSE) two elements into their allocations: every plan
    accepts them (the reference's 4-byte contract) and returns the bits of the
    16-byte-aligned call."""
    import torch
    log("4-byte aligned operands")
    rng = np.random.default_rng(4)
    B, hq, hkv = 3, 16, 4
    for teams in (0, 5):  # direct, balanced
        pool, (q, k, v, ip, ix, ln) = decode_case(oracle, rng, B, hq, hkv, [33, 700, 5])
        r = DecodeRunner(L, B, pool, hq, hkv, teams=teams)
        want = r.run(q, k, v, ip, ix, ln)
        dq, dk, dv = (shifted(to_dev_bf16(x), 2) for x in (q, k, v))
        out = shifted(nan_bf16(r.spec.output_numel), 2)
        lse = shifted(torch.full((r.spec.lse_numel,), float("nan"), device="cuda"), 1)
        o, l_ = r.run_dev(dq, dk, dv, to_dev_i32(ip), to_dev_i32(ix), to_dev_i32(ln), out, lse)
        assert np.array_equal(bf16_host(o), want[0]), f"decode teams={teams}"
        assert np.array_equal(l_.cpu().numpy(), want[1])
    # paged prefill: 3 requests, ragged query rows
    qo = np.array([0, 4, 6, 13], np.int32)
    lens = [40, 18, 90]
    pool = sum((x + 15) // 16 for x in lens) + 2
    ip, ix, ln = ragged_table(rng, lens, pool)
    nnz = int(qo[-1])
    q = seeded_normal_bf16(oracle, rng, nnz * hq * 128)
    k = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, pool * 16 * hkv * 128)
    pr = PrefillRunner(L, 3, nnz, pool, hq, hkv)
    want = pr.run(q, k, v, qo, ip, ix, ln)
    dq, dk, dv = (shifted(to_dev_bf16(x), 2) for x in (q, k, v))
    out = shifted(nan_bf16(pr.spec.output_numel), 2)
    o, l_ = pr.run_dev(dq, dk, dv, to_dev_i32(qo), to_dev_i32(ip), to_dev_i32(ix),
                       to_dev_i32(ln), out=out)
    assert np.array_equal(bf16_host(o), want[0]) and np.array_equal(l_.cpu().numpy(), want[1])
    # ragged prefill on the same rows with contiguous K/V
    kv = np.array([0, 40, 58, 148], np.int32)
    kc = seeded_normal_bf16(oracle, rng, int(kv[-1]) * hkv * 128)
    vc = seeded_normal_bf16(oracle, rng, int(kv[-1]) * hkv * 128)
    rr = RaggedRunner(L, 3, nnz, int(kv[-1]), hq, hkv)
    want = rr.run(q, kc, vc, qo, kv)
    dk, dv = (shifted(to_dev_bf16(x), 2) for x in (kc, vc))
    out = shifted(nan_bf16(rr.spec.output_numel), 2)
    o, l_ = rr.run_dev(shifted(to_dev_bf16(q), 2), dk, dv, to_dev_i32(qo), to_dev_i32(kv),
                       out=out)
    assert np.array_equal(bf16_host(o), want[0]) and np.array_equal(l_.cpu().numpy(), want[1])
    torch.cuda.synchronize()


def test_unreserved_decode_capture_fails_typed_and_reserved_one_never_grows(L, oracle):
    """A reference-shaped split-KV decode captured on a graph queue whose
    workspace was not reserved fails with WorkspaceNotReserved (no hipMalloc
    during capture); after reserve_workspace the same capture succeeds and the
    queue's workspace does not grow; eagerly (no capture) the queue still
    grows its own."""
    import torch
    log("decode capture without a reserved workspace")
    rng = np.random.default_rng(31)
    B, hq, hkv = 3, 32, 8
    pool, (q, k, v, ip, ix, ln) = decode_case(oracle, rng, B, hq, hkv, [300, 2000, 45])
    r = DecodeRunner(L, B, pool, hq, hkv, teams=5)
    want_o, want_l = r.run(q, k, v, ip, ix, ln)
    assert r.plan.workspace_bytes > 0
    dev = [to_dev_bf16(q), to_dev_bf16(k), to_dev_bf16(v), to_dev_i32(ip), to_dev_i32(ix),
           to_dev_i32(ln)]
    out = torch.empty(r.spec.output_numel, dtype=torch.bfloat16, device="cuda")
    lse = torch.empty(r.spec.lse_numel, dtype=torch.float32, device="cuda")

    def capture(gq):
        b = gq.bindings(8)
        h = [b.bind_read(x) for x in dev]
        ho, hl = b.bind_read_write(out), b.bind_read_write(lse)
        args = L.Bf16PagedBatchDecodeArgs(*h, ho.write(), hl.write())
        return gq.capture(b, lambda scope: r.plan.enqueue_into(scope, args))

    gq = L.GraphQueue(0, 1)
    before = gq.workspace_bytes
    with pytest.raises(L.EnqueueError) as e:
        capture(gq)
    assert e.value.variant == "WorkspaceNotReserved", e.value
    log(f"  unreserved: {e.value}")

    gq = L.GraphQueue(0, 1)
    gq.reserve_workspace(scratch_bytes=r.plan.workspace_bytes)
    reserved = gq.workspace_bytes
    assert reserved >= before + r.plan.workspace_bytes
    exec_ = capture(gq).instantiate()
    for i in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        exec_.launch().wait()
        assert np.array_equal(bf16_host(out), want_o), f"replay {i}"
        assert np.array_equal(lse.cpu().numpy(), want_l), f"replay {i}"
    exec_.into_bindings()
