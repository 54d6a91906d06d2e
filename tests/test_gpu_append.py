"""GPU parity of fused RoPE + paged K/V append (C ABI) against the pinned oracle:
the reference's gate fixtures (golden digests), its sentinel guards, a
BASELINE config-2-shaped bulk append, and graph replay."""
import json
import os
import sys

import numpy as np
import pytest

from gpu_util import bf16_host, nan_bf16, to_dev_bf16, to_dev_i32

pytestmark = pytest.mark.gpu

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                     "reference_digests.json")))


@pytest.fixture(scope="module")
def L():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import loom_infer_hip as L
    return L


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def check_workspace_ready(ws, chunked_before, chunked):
    """The append workspace after a command: the one-launch chunk-validated
    path (T > 64 or more than 4096 page indices) advanced the epoch once; no
    epoch handover gave up (the broken word is clear); the hash table the
    next command inserts into is empty.  The two-launch form and the small
    one-launch path leave the epoch alone.  Layout in u32 words (one for every
    plan): 64 header words (epoch u64, broken), 8512 u64 start tags, 64 x 320
    u64 verdict copies, two 16384-entry hash tables, 320 two-launch
    verdicts."""
    w = ws.cpu().numpy().view(np.uint32)
    epoch = int(w[0]) | int(w[1]) << 32
    assert w[2] == 0, "the workspace is marked broken"
    assert epoch == chunked_before + chunked, (epoch, chunked_before, chunked)
    tables = 64 + 2 * (8192 + 320) + 2 * 64 * 320
    assert len(w) == tables + 2 * 16384 + 320
    nxt = w[tables + (epoch & 1) * 16384: tables + ((epoch & 1) + 1) * 16384]
    assert not nxt.any(), f"next command's hash table holds {np.count_nonzero(nxt)} entries"


class AppendRunner:
    def __init__(self, L, spec, explicit, flags=0):
        import torch
        self.L, self.spec, self.explicit = L, spec, explicit
        self.two_launch = bool(flags & L.PLAN_APPEND_TWO_LAUNCH)
        prov = L.RopeProvider.load(0)
        self.plan = (prov.plan_bf16_paged_append_tokens(spec, flags=flags) if explicit
                     else prov.plan_bf16_paged_append(spec, flags=flags))
        self.ws = torch.zeros(self.plan.workspace_bytes, dtype=torch.uint8, device="cuda")
        self.queue = L.CommandQueue(torch.cuda.current_stream(), 2)
        self.epochs = 0  # chunk-validated commands run on self.ws

    def bind(self, b, q, k, v, bi, pos, ip, ix, ln, qo, kp, vp):
        L = self.L
        h = dict(query=b.bind_read(q), key=b.bind_read(k), value=b.bind_read(v))
        if self.explicit:
            h["batch_indices"] = b.bind_read(bi)
            h["positions"] = b.bind_read(pos)
        h.update(page_indptr=b.bind_read(ip), page_indices=b.bind_read(ix),
                 last_page_len=b.bind_read(ln), query_output=b.bind_read_write(qo),
                 key_pages=b.bind_read_write(kp), value_pages=b.bind_read_write(vp),
                 workspace=b.bind_read_write(self.ws))
        args = L.Bf16RopePagedKvAppendArgs(
            h["query"], h["key"], h["value"], h["page_indptr"], h["page_indices"],
            h["last_page_len"], h["query_output"].write(), h["key_pages"].write(),
            h["value_pages"].write(), h["workspace"].write(), h.get("batch_indices"),
            h.get("positions"))
        return h, args

    def run(self, q, k, v, bi, pos, ip, ix, ln, kp_host, vp_host):
        tq, tk, tv = to_dev_bf16(q), to_dev_bf16(k), to_dev_bf16(v)
        tbi = to_dev_i32(bi) if self.explicit else None
        tpos = to_dev_i32(pos) if self.explicit else None
        qo = nan_bf16(self.spec.query_output_numel)
        kp, vp = to_dev_bf16(kp_host), to_dev_bf16(vp_host)
        b = self.queue.bindings(12)
        h, args = self.bind(b, tq, tk, tv, tbi, tpos, to_dev_i32(ip), to_dev_i32(ix),
                            to_dev_i32(ln), qo, kp, vp)
        scope = self.queue.begin(b)
        self.plan.enqueue_into(scope, args)
        comp = scope.finish()
        assert comp.submitted() == 1
        b = comp.wait()
        out = [bf16_host(b.take_read_write(h[n])) for n in ("query_output", "key_pages",
                                                           "value_pages")]
        b.take_read_write(h["workspace"])
        T = self.plan.info.tokens
        chunked = int(not (T <= 64 and len(ix) <= 4096) and not self.two_launch)
        check_workspace_ready(self.ws, self.epochs, chunked)
        self.epochs += chunked
        return out


def within_one_ulp(oracle, got, want):
    """Bit patterns within one BF16 ulp (same sign, |bits difference| <= 1)."""
    g, w = got.astype(np.int32), want.astype(np.int32)
    same = g == w
    a = oracle.bf16_to_f32(got)
    b = oracle.bf16_to_f32(want)
    near = (np.sign(a) == np.sign(b)) & (np.abs(g - w) <= 1)
    bad = ~(same | near)
    if bad.any():
        i = np.flatnonzero(bad)[:8]
        print(f"    beyond 1 ulp: {int(bad.sum())} of {got.size}; first {i.tolist()} "
              f"got {a[i].tolist()} want {b[i].tolist()}", flush=True)
    return bool(not bad.any()), int(np.sum(~same))


ROPE_PINS_PATH = os.path.join(os.path.dirname(__file__), "golden", "rope_beyond_one_ulp.json")


def pin_rope_counts(key, beyond, mism):
    """The number of elements beyond one BF16 ulp (all explained by the host
    sinf/cosf rounding) and of bit mismatches, pinned per case in
    tests/golden/rope_beyond_one_ulp.json: a change in the device's sin/cos
    or rotation arithmetic shifts them even when every element stays
    explainable.  With LOOM_RECORD_ROPE_COUNTS=<file> the observed counts are
    written there instead (to create the pins)."""
    rec = os.environ.get("LOOM_RECORD_ROPE_COUNTS")
    if rec:
        d = json.load(open(rec)) if os.path.exists(rec) else {}
        d[key] = {"beyond_one_ulp": beyond, "bit_mismatches": mism}
        os.makedirs(os.path.dirname(os.path.abspath(rec)), exist_ok=True)
        json.dump(d, open(rec, "w"), indent=1, sort_keys=True)
        return
    pins = json.load(open(ROPE_PINS_PATH))
    assert key in pins, f"no pinned RoPE counts for {key}"
    assert pins[key] == {"beyond_one_ulp": beyond, "bit_mismatches": mism}, (key, pins[key],
                                                                            beyond, mism)


def check_rope(oracle, got, want, inputs, positions_per_row, what, pin=None):
    """RoPE output against the oracle: within one BF16 ulp everywhere, except
    elements proven to differ only through the oracle's sin/cos rounding.

    The device evaluates sin/cos of the FP32 angle correctly rounded; the
    reference (and the oracle) calls the host C library's sinf/cosf, which
    differ from the correctly rounded value by one FP32 ulp for about 2.6% of
    the (sin, cos) pairs of these angles.  Where the rotation cancels, that
    moves the BF16 output by more than one ulp.  Every such element is
    re-evaluated on the host (tests/rope_explain.py): with sinf/cosf it must
    give the oracle's bits, with the correctly rounded pair the device's bits,
    and the two pairs must differ.  Any other difference fails.  Rows are
    [.., 128]; positions_per_row gives each row's token position."""
    from rope_explain import explain_beyond_one_ulp
    beyond, unexplained = explain_beyond_one_ulp(got, want, inputs, positions_per_row)
    mism = int(np.sum(got != want))
    log(f"    {what}: {mism} bit mismatches, {beyond} beyond 1 BF16 ulp, all explained by "
        f"sinf/cosf rounding: {not unexplained} (of {got.size})")
    assert not unexplained, (f"{what}: {len(unexplained)} of {beyond} elements beyond 1 BF16 "
                             f"ulp not explained by sin/cos rounding, first "
                             f"(row, col, pos, got, want, host, cr) {unexplained[:4]}")
    if pin:
        pin_rope_counts(pin, beyond, mism)
    return beyond


def _inputs(oracle, g, n_tokens):
    sl = {k: int(v, 16) for k, v in g["salts"].items()}
    nkv = g["pool"] * 16 * g["hkv"] * 128
    return (oracle.deterministic_bf16(n_tokens * g["hq"] * 128, sl["query"]),
            oracle.deterministic_bf16(n_tokens * g["hkv"] * 128, sl["key"]),
            oracle.deterministic_bf16(n_tokens * g["hkv"] * 128, sl["value"]),
            oracle.deterministic_bf16(nkv, sl["key_pages"]),
            oracle.deterministic_bf16(nkv, sl["value_pages"]))


def test_one_token_gate_fixture(L, oracle):
    # crates/loom-infer-validation/src/gates/rope.rs:249-365
    g = GOLDEN["append_one_token"]
    q, k, v, kp, vp = _inputs(oracle, g, g["batch"])
    s = oracle.paged_spec(g["batch"], g["pool"], g["hq"], g["hkv"])
    ekp, evp = kp.copy(), vp.copy()
    eq = oracle.append(s, q, k, v, g["indptr"], g["indices"], g["last"], ekp, evp)
    spec = L.Bf16RopePagedKvAppendSpec(g["batch"], g["pool"], g["hq"], g["hkv"])
    r = AppendRunner(L, spec, False)
    qo, okp, ovp = r.run(q, k, v, None, None, g["indptr"], g["indices"], g["last"], kp, vp)
    for got, want in ((qo, eq), (okp, ekp)):
        ok, mism = within_one_ulp(oracle, got, want)
        assert ok
        log(f"  mismatches={mism}")
    assert np.array_equal(ovp, evp)
    # the device result reproduces the reference's recorded CPU-oracle digests
    assert oracle.digest_bf16(qo) == int(g["query_digest"], 16)
    assert oracle.digest_bf16(okp) == int(g["key_pages_digest"], 16)
    assert oracle.digest_bf16(ovp) == int(g["value_pages_digest"], 16)


@pytest.mark.parametrize("name", ["append_tokens_t6", "append_tokens_t64"])
def test_explicit_token_gate_fixtures(L, oracle, name):
    # crates/loom-infer-validation/src/gates/rope.rs:369-628
    g = GOLDEN[name]
    T = g["tokens"]
    bi = g.get("batch_indices", [0] * T)
    pos = g.get("positions", list(range(T)))
    q, k, v, kp, vp = _inputs(oracle, g, T)
    s = oracle.paged_spec(g["batch"], g["pool"], g["hq"], g["hkv"])
    ekp, evp = kp.copy(), vp.copy()
    eq = oracle.append_tokens(s, T, q, k, v, bi, pos, g["indptr"], g["indices"], g["last"],
                              ekp, evp)
    spec = L.Bf16RopePagedKvAppendTokensSpec(T, g["batch"], g["pool"], g["hq"], g["hkv"])
    r = AppendRunner(L, spec, True)
    qo, okp, ovp = r.run(q, k, v, bi, pos, g["indptr"], g["indices"], g["last"], kp, vp)
    for got, want in ((qo, eq), (okp, ekp)):
        ok, mism = within_one_ulp(oracle, got, want)
        assert ok
        log(f"  {name} mismatches={mism}")
    assert np.array_equal(ovp, evp)


GUARDS_ONE = [
    # crates/loom-infer-validation/src/gates/rope.rs:936-970
    ("duplicate_final_slot", [0, 1, 2], [1, 1], [4, 4]),
    ("invalid_non_final_page", [0, 2, 3], [2, 0, 1], [4, 5]),
]


@pytest.mark.parametrize("name,ip,ix,ln", GUARDS_ONE, ids=[g[0] for g in GUARDS_ONE])
def test_one_token_guards_preserve_all_sentinels(L, oracle, name, ip, ix, ln):
    spec = L.Bf16RopePagedKvAppendSpec(2, 2, 2, 1)
    r = AppendRunner(L, spec, False)
    z = np.zeros(2 * 2 * 128, np.uint16)
    kz = np.zeros(2 * 128, np.uint16)
    ks = np.full(spec.kv_pages_numel, oracle.bf16_from_f32(np.array([-7.0], np.float32))[0],
                 np.uint16)
    vs = np.full(spec.kv_pages_numel, oracle.bf16_from_f32(np.array([9.0], np.float32))[0],
                 np.uint16)
    qo, kp, vp = r.run(z, kz, kz, None, None, ip, ix, ln, ks, vs)
    assert np.all(np.isnan(oracle.bf16_to_f32(qo)))
    assert np.array_equal(kp, ks) and np.array_equal(vp, vs)


GUARDS_TOKENS = [
    # crates/loom-infer-validation/src/gates/rope.rs:1032-1086
    ("duplicate_slot", [0, 1], [2, 2], [3, 1, 3, 2]),
    ("batch_index", [0, 2], [1, 1], [3, 1, 3, 2]),
    ("position", [0, 1], [1, 20], [3, 1, 3, 2]),
    ("page_index", [0, 1], [16, 16], [4, 1, 3, 2]),
]


@pytest.mark.parametrize("name,bi,pos,ix", GUARDS_TOKENS, ids=[g[0] for g in GUARDS_TOKENS])
def test_explicit_guards_preserve_all_sentinels(L, oracle, name, bi, pos, ix):
    spec = L.Bf16RopePagedKvAppendTokensSpec(2, 2, 4, 2, 1)
    r = AppendRunner(L, spec, True)
    z = np.zeros(2 * 2 * 128, np.uint16)
    kz = np.zeros(2 * 128, np.uint16)
    ks = np.full(spec.kv_pages_numel, oracle.bf16_from_f32(np.array([-7.0], np.float32))[0],
                 np.uint16)
    vs = np.full(spec.kv_pages_numel, oracle.bf16_from_f32(np.array([9.0], np.float32))[0],
                 np.uint16)
    qo, kp, vp = r.run(z, kz, kz, bi, pos, [0, 2, 4], ix, [4, 4], ks, vs)
    assert np.all(np.isnan(oracle.bf16_to_f32(qo)))
    assert np.array_equal(kp, ks) and np.array_equal(vp, vs)


# The two device paths of the explicit-token command: one launch in which
# every workgroup validates the whole command (T <= 64, <= 4096 page indices),
# and one launch in which the first workgroups validate one chunk each and the
# token workgroups wait for their verdicts (anything larger).
PATHS = [
    # (name, tokens, page indices of the long request)
    ("fused_small", 3, 100),
    ("chunked", 300, 4200),
    ("chunked_long_table", 300, 9000),
    ("chunked_few_tokens", 3, 4200),
    ("chunked_many_tokens", 1500, 4200),
]
BREAKS = ["valid", "duplicate_slot", "duplicate_far", "batch_index", "position", "page_index",
          "last_page_len"]


def explicit_case(oracle, seed, T, long_pages, brk):
    """Explicit-token command inputs over 3 requests (lens 40, long, 500), with
    one guard broken as `brk` names; the metadata of every break except
    page_index / last_page_len differs from the valid case only in the
    batch-index / position arrays."""
    rng = np.random.default_rng(seed)
    B, hq, hkv = 3, 4, 2
    lens = np.array([40, long_pages * 16 - 3, 500])
    pages = (lens + 15) // 16
    pool = int(pages.sum()) + 5
    indptr = np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)
    indices = rng.permutation(pool)[: indptr[-1]].astype(np.int32)
    last = (lens - (pages - 1) * 16).astype(np.int32)
    # distinct (request, position) pairs
    pairs = set()
    while len(pairs) < T:
        r = int(rng.integers(0, B))
        pairs.add((r, int(rng.integers(0, lens[r]))))
    pairs = sorted(pairs)
    rng.shuffle(pairs)
    bi = np.array([p[0] for p in pairs], np.int32)
    pos = np.array([p[1] for p in pairs], np.int32)
    j = int(rng.integers(0, T))
    if brk == "duplicate_slot":
        k2 = (j + 1) % T
        bi[k2], pos[k2] = bi[j], pos[j]
    elif brk == "duplicate_far":
        # first and last token: different validation chunks (256 tokens
        # each) once T > 256, so the two keys meet only in the shared table
        bi[T - 1], pos[T - 1] = bi[0], pos[0]
    elif brk == "batch_index":
        bi[j] = B
    elif brk == "position":
        pos[j] = lens[bi[j]]
    elif brk == "page_index":
        indices[int(rng.integers(0, len(indices)))] = pool
    elif brk == "last_page_len":
        last[1] = 17
    q = oracle.bf16_from_f32(rng.standard_normal(T * hq * 128, dtype=np.float32))
    k = oracle.bf16_from_f32(rng.standard_normal(T * hkv * 128, dtype=np.float32))
    v = oracle.bf16_from_f32(rng.standard_normal(T * hkv * 128, dtype=np.float32))
    kp = np.full(pool * 16 * hkv * 128, 0x3F80, np.uint16)
    vp = np.full(pool * 16 * hkv * 128, 0x4000, np.uint16)
    return dict(B=B, hq=hq, hkv=hkv, pool=pool, indptr=indptr, indices=indices, last=last,
                bi=bi, pos=pos, q=q, k=k, v=v, kp=kp, vp=vp)


# The two-launch plan option (validation kernel, then apply kernel) on the
# chunk-validated shapes.
PATHS_TWO_LAUNCH = [p + (True,) for p in PATHS if p[0].startswith("chunked")]


@pytest.mark.parametrize("brk", BREAKS)
@pytest.mark.parametrize("path,T,long_pages,two_launch",
                         [p + (False,) for p in PATHS] + PATHS_TWO_LAUNCH,
                         ids=[p[0] for p in PATHS] + [p[0] + "_two_launch" for p in PATHS_TWO_LAUNCH])
def test_explicit_paths_valid_and_guarded(L, oracle, path, T, long_pages, two_launch, brk):
    """Each path on valid metadata (against the oracle) and with one guard
    broken (rope/mod.rs:407-466: every output keeps its sentinels)."""
    log(f"append path {path} T={T} two_launch={two_launch} break={brk}")
    c = explicit_case(oracle, hash((path, brk)) % 2**32, T, long_pages, brk)
    B, hq, hkv, pool = c["B"], c["hq"], c["hkv"], c["pool"]
    indptr, indices, last, bi, pos = c["indptr"], c["indices"], c["last"], c["bi"], c["pos"]
    q, k, v, kp, vp = c["q"], c["k"], c["v"], c["kp"], c["vp"]
    spec = L.Bf16RopePagedKvAppendTokensSpec.extended(T, B, pool, hq, hkv)
    r = AppendRunner(L, spec, True, L.PLAN_APPEND_TWO_LAUNCH if two_launch else 0)
    for call in range(2):  # the second command runs over the first one's workspace
        qo, okp, ovp = r.run(q, k, v, bi, pos, indptr, indices, last, kp, vp)
        if brk != "valid":
            assert np.all(np.isnan(oracle.bf16_to_f32(qo))), call
            assert np.array_equal(okp, kp) and np.array_equal(ovp, vp), call
            continue
        s = oracle.paged_spec(B, pool, hq, hkv)
        ekp, evp = kp.copy(), vp.copy()
        eq = oracle.append_tokens(s, T, q, k, v, bi, pos, indptr, indices, last, ekp, evp,
                                  max_tokens=8192)
        check_rope(oracle, qo, eq, q, np.repeat(pos, hq), "query")
        slots = [(indices[indptr[b] + p // 16], p % 16) for b, p in zip(bi, pos)]
        rows = np.array([(pg * 16 + off) * hkv + h for pg, off in slots for h in range(hkv)])
        okr, ekr = okp.reshape(-1, 128), ekp.reshape(-1, 128)
        check_rope(oracle, okr[rows], ekr[rows], k, np.repeat(pos, hkv), "key rows")
        rest = np.ones(len(okr), bool)
        rest[rows] = False
        assert np.array_equal(okr[rest], ekr[rest]), call
        assert np.array_equal(ovp, evp), call


def test_chunked_path_alternating_valid_and_broken_commands(L, oracle):
    """One plan and one workspace, commands alternating valid and broken
    metadata (chunk-validated path, T = 300): a broken command must not be
    let through by an earlier command's verdicts, and a valid one must not be
    held back by an earlier broken one (the workspace's epoch tags them)."""
    T, long_pages = 300, 4200
    cases = {brk: explicit_case(oracle, 7, T, long_pages, brk)
             for brk in ("valid", "duplicate_slot", "page_index", "position")}
    c = cases["valid"]
    spec = L.Bf16RopePagedKvAppendTokensSpec.extended(T, c["B"], c["pool"], c["hq"], c["hkv"])
    r = AppendRunner(L, spec, True)
    want = None
    for i, brk in enumerate(["valid", "duplicate_slot", "valid", "page_index", "position",
                             "valid", "valid", "duplicate_slot"]):
        log(f"append alternating command {i}: {brk}")
        x = cases[brk]
        qo, okp, ovp = r.run(x["q"], x["k"], x["v"], x["bi"], x["pos"], x["indptr"],
                             x["indices"], x["last"], x["kp"], x["vp"])
        if brk != "valid":
            assert np.all(np.isnan(oracle.bf16_to_f32(qo))), i
            assert np.array_equal(okp, x["kp"]) and np.array_equal(ovp, x["vp"]), i
        elif want is None:
            s = oracle.paged_spec(c["B"], c["pool"], c["hq"], c["hkv"])
            ekp, evp = c["kp"].copy(), c["vp"].copy()
            eq = oracle.append_tokens(s, T, c["q"], c["k"], c["v"], c["bi"], c["pos"],
                                      c["indptr"], c["indices"], c["last"], ekp, evp,
                                      max_tokens=8192)
            check_rope(oracle, qo, eq, c["q"], np.repeat(c["pos"], c["hq"]), "query")
            assert np.array_equal(ovp, evp)
            want = (qo, okp, ovp)
        else:
            assert all(np.array_equal(a, b) for a, b in zip((qo, okp, ovp), want)), i


def test_bulk_append_config2_shape(L, oracle):
    """32 requests each appending U{1..64} tokens (~1040) into
    a 16384-page pool with existing lengths U[0,4095] (extended contract)."""
    log("append bulk config-2 shape")
    rng = np.random.default_rng(2)
    B, hq, hkv, pool = 32, 32, 8, 16384
    existing = rng.integers(0, 4096, size=B)
    n_new = rng.integers(1, 65, size=B)
    lens = existing + n_new
    pages = (lens + 15) // 16
    indptr = np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)
    indices = rng.permutation(pool)[: indptr[-1]].astype(np.int32)
    last = (lens - (pages - 1) * 16).astype(np.int32)
    bi = np.concatenate([np.full(n, r) for r, n in enumerate(n_new)]).astype(np.int32)
    pos = np.concatenate([np.arange(e, e + n) for e, n in zip(existing, n_new)]).astype(np.int32)
    perm = rng.permutation(len(bi))
    bi, pos = bi[perm], pos[perm]
    T = len(bi)
    q = oracle.bf16_from_f32(rng.standard_normal(T * hq * 128, dtype=np.float32))
    k = oracle.bf16_from_f32(rng.standard_normal(T * hkv * 128, dtype=np.float32))
    v = oracle.bf16_from_f32(rng.standard_normal(T * hkv * 128, dtype=np.float32))
    # only touched pages matter for the check; start from a sentinel pool
    kp = np.full(pool * 16 * hkv * 128, 0x3F80, np.uint16)
    vp = np.full(pool * 16 * hkv * 128, 0x3F80, np.uint16)
    s = oracle.paged_spec(B, pool, hq, hkv)
    ekp, evp = kp.copy(), vp.copy()
    eq = oracle.append_tokens(s, T, q, k, v, bi, pos, indptr, indices, last, ekp, evp,
                              max_tokens=8192)
    spec = L.Bf16RopePagedKvAppendTokensSpec.extended(T, B, pool, hq, hkv)
    r = AppendRunner(L, spec, True)
    qo, okp, ovp = r.run(q, k, v, bi, pos, indptr, indices, last, kp, vp)
    n_q = check_rope(oracle, qo, eq, q, np.repeat(pos, hq), "query", pin="c2_bulk_query")
    # appended K rows: gather the slots, then require the rest of the pool untouched
    slots = [(indices[indptr[b] + p // 16], p % 16) for b, p in zip(bi, pos)]
    rows = np.array([(pg * 16 + off) * hkv + h for pg, off in slots for h in range(hkv)])
    okr, ekr = okp.reshape(-1, 128), ekp.reshape(-1, 128)
    n_k = check_rope(oracle, okr[rows], ekr[rows], k, np.repeat(pos, hkv), "key rows",
                     pin="c2_bulk_key_rows")
    log(f"  config 2: {T} tokens, {n_q + n_k} elements beyond 1 BF16 ulp, every one explained")
    okr[rows] = 0
    ekr[rows] = 0
    assert np.array_equal(okr, ekr)
    assert np.array_equal(ovp, evp)


def test_large_position_stays_finite_and_matches(L, oracle):
    """One token at position 32767 (rope/tests.rs:61-81 on the device): the
    rotation at large angles stays finite and within the RoPE tolerance."""
    rng = np.random.default_rng(32767)
    B, hq, hkv = 1, 4, 2
    kv_len = 32768
    pages = kv_len // 16
    pool = pages + 3
    indptr = np.array([0, pages], np.int32)
    indices = rng.permutation(pool)[:pages].astype(np.int32)
    last = np.array([16], np.int32)
    q = oracle.bf16_from_f32(rng.standard_normal(B * hq * 128, dtype=np.float32))
    k = oracle.bf16_from_f32(rng.standard_normal(B * hkv * 128, dtype=np.float32))
    v = oracle.bf16_from_f32(rng.standard_normal(B * hkv * 128, dtype=np.float32))
    kp = np.zeros(pool * 16 * hkv * 128, np.uint16)
    vp = np.zeros(pool * 16 * hkv * 128, np.uint16)
    s = oracle.paged_spec(B, pool, hq, hkv)
    ekp, evp = kp.copy(), vp.copy()
    eq = oracle.append(s, q, k, v, indptr, indices, last, ekp, evp)
    spec = L.Bf16RopePagedKvAppendSpec(B, pool, hq, hkv)
    r = AppendRunner(L, spec, False)
    qo, okp, ovp = r.run(q, k, v, None, None, indptr, indices, last, kp, vp)
    assert np.all(np.isfinite(oracle.bf16_to_f32(qo)))
    check_rope(oracle, qo, eq, q, np.full(hq, kv_len - 1), "query")
    row = (indices[-1] * 16 + 15) * hkv
    got_k = okp.reshape(-1, 128)[row:row + hkv].reshape(-1)
    want_k = ekp.reshape(-1, 128)[row:row + hkv].reshape(-1)
    check_rope(oracle, got_k, want_k, k, np.full(hkv, kv_len - 1), "key")
    assert np.array_equal(ovp, evp)


def _many_requests_case(oracle, rng, B, T, hq, hkv):
    """B requests of 1-40 existing tokens (more when T needs them), T distinct
    (request, position) tokens among them, seeded shuffled page table."""
    lens = rng.integers(1, max(41, 4 * T // B), size=B)
    pages = (lens + 15) // 16
    pool = int(pages.sum()) + 7
    indptr = np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)
    indices = rng.permutation(pool)[: indptr[-1]].astype(np.int32)
    last = (lens - (pages - 1) * 16).astype(np.int32)
    flat = rng.choice(int(lens.sum()), size=T, replace=False)
    starts = np.concatenate([[0], np.cumsum(lens)])
    bi = (np.searchsorted(starts, flat, side="right") - 1).astype(np.int32)
    pos = (flat - starts[bi]).astype(np.int32)
    q = oracle.bf16_from_f32(rng.standard_normal(T * hq * 128, dtype=np.float32))
    k = oracle.bf16_from_f32(rng.standard_normal(T * hkv * 128, dtype=np.float32))
    v = oracle.bf16_from_f32(rng.standard_normal(T * hkv * 128, dtype=np.float32))
    return pool, indptr, indices, last, bi, pos, q, k, v


@pytest.mark.parametrize("B,T", [(3000, 300), (64, 8192), (64, 2048)],
                         ids=["batch3000_table_in_memory", "tokens8192_grid_over_residency",
                              "tokens2048"])
@pytest.mark.parametrize("brk", ["valid", "duplicate_far"])
def test_chunked_path_large_batch_and_max_tokens(L, oracle, B, T, brk):
    """The chunk-validated path where the validation workgroups read the
    request table from memory (B > 2048 requests), at the contract's largest
    command (T = 8192 tokens: 8192 + V workgroups, more than the device holds
    at once, so later token workgroups start only after earlier ones finish),
    and at 2048 tokens (eight token validation chunks); valid commands
    against the oracle, a duplicate pair in the first and last token leaving
    every output untouched."""
    log(f"append chunked B={B} T={T} break={brk}")
    rng = np.random.default_rng(B * 7 + T)
    hq, hkv = 4, 2
    pool, indptr, indices, last, bi, pos, q, k, v = _many_requests_case(oracle, rng, B, T, hq, hkv)
    if brk == "duplicate_far":
        bi[T - 1], pos[T - 1] = bi[0], pos[0]
    kp = np.full(pool * 16 * hkv * 128, 0x3F80, np.uint16)
    vp = np.full(pool * 16 * hkv * 128, 0x4000, np.uint16)
    spec = L.Bf16RopePagedKvAppendTokensSpec.extended(T, B, pool, hq, hkv)
    r = AppendRunner(L, spec, True)
    for call in range(2):
        qo, okp, ovp = r.run(q, k, v, bi, pos, indptr, indices, last, kp, vp)
        if brk != "valid":
            assert np.all(np.isnan(oracle.bf16_to_f32(qo))), call
            assert np.array_equal(okp, kp) and np.array_equal(ovp, vp), call
            continue
        s = oracle.paged_spec(B, pool, hq, hkv)
        ekp, evp = kp.copy(), vp.copy()
        eq = oracle.append_tokens(s, T, q, k, v, bi, pos, indptr, indices, last, ekp, evp,
                                  max_tokens=8192)
        check_rope(oracle, qo, eq, q, np.repeat(pos, hq), "query")
        assert np.array_equal(ovp, evp), call
        slots = [(indices[indptr[b] + p // 16], p % 16) for b, p in zip(bi, pos)]
        rows = np.array([(pg * 16 + off) * hkv + h for pg, off in slots for h in range(hkv)])
        okr, ekr = okp.reshape(-1, 128), ekp.reshape(-1, 128)
        check_rope(oracle, okr[rows], ekr[rows], k, np.repeat(pos, hkv), "key rows")
        rest = np.ones(len(okr), bool)
        rest[rows] = False
        assert np.array_equal(okr[rest], ekr[rest]), call


def test_append_plan_rejects_batches_beyond_the_validation_layout(L):
    """Append plans take batches of at most 65536 requests (the validation
    chunks and the fixed workspace layout cover that many); more is a plan
    error, before any enqueue."""
    prov = L.RopeProvider.load(0)
    prov.plan_bf16_paged_append_tokens(
        L.Bf16RopePagedKvAppendTokensSpec.extended(100, 65536, 70000, 4, 2))
    with pytest.raises(L.PlanError) as e:
        prov.plan_bf16_paged_append_tokens(
            L.Bf16RopePagedKvAppendTokensSpec.extended(100, 65537, 70000, 4, 2))
    assert e.value.variant == "StateCountOutOfRange"
