"""FP8 E4M3 K/V pages (no reference counterpart: the reference lists FP8 KV as
unsupported) through the C ABI, against the oracle's FP8 restatements (pinned
in tests/test_oracle_fp8.py against torch.float8_e4m3fn and the BF16 paths).

* Append: V bytes bit-exact (no RoPE in between); K bytes bit-exact except
  where the oracle's FP32 rotation differs from the device's by the sin/cos
  rounding discussed in test_gpu_append.check_rope, which can move
  a value across an FP8 rounding boundary: such bytes are adjacent codes, and
  rare.  Query output within the BF16 append's tolerance.
* Decode: against the oracle's FP8 decode with the BF16 decode's tolerances
  (max-abs 1/64, mean-abs 2e-3, LSE 1e-2), over the direct and balanced
  algorithms, NHD and HND pages, and pages holding every finite E4M3 code.
* Append then decode on the pages the append wrote."""
import sys

import numpy as np
import pytest

from gpu_util import (bf16_host, compare_decode, nan_bf16, ragged_table, seeded_normal_bf16,
                      to_dev_bf16, to_dev_i32)
from test_gpu_append import check_rope, within_one_ulp
from test_gpu_layout import to_hnd

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


def dev_u8(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint8)).to("cuda")


def dev_f32(a):
    import torch
    return torch.tensor(np.asarray(a, np.float32), device="cuda")


def run_decode(L, spec, opts, q, k8, v8, ip, ix, last, scales):
    import torch
    plan = L.DecodeProvider.load(0).plan_bf16_paged_batch(spec, **opts)
    ws = torch.full((plan.workspace_bytes,), 0xFF, dtype=torch.uint8, device="cuda")
    out = nan_bf16(spec.output_numel)
    lse = torch.full((spec.lse_numel,), float("nan"), dtype=torch.float32, device="cuda")
    queue = L.CommandQueue(torch.cuda.current_stream(), 2)
    b = queue.bindings(10)
    h = [b.bind_read(to_dev_bf16(q)), b.bind_read(dev_u8(k8)), b.bind_read(dev_u8(v8)),
         b.bind_read(to_dev_i32(ip)), b.bind_read(to_dev_i32(ix)), b.bind_read(to_dev_i32(last)),
         b.bind_read_write(out), b.bind_read_write(lse), b.bind_read_write(ws),
         b.bind_read(dev_f32(scales)) if scales is not None else None]
    args = L.Bf16PagedBatchDecodeArgs(h[0], h[1], h[2], h[3], h[4], h[5], h[6].write(),
                                      h[7].write(), h[8].write(), h[9])
    scope = queue.begin(b)
    plan.enqueue_into(scope, args)
    b = scope.finish().wait()
    return bf16_host(b.take_read_write(h[6])), b.take_read_write(h[7]).cpu().numpy(), plan


def random_fp8(rng, n, max_code=0x7E):
    """Finite E4M3 bytes (both signs), codes 0..max_code."""
    return (rng.integers(0, max_code + 1, n).astype(np.uint8) |
            (rng.integers(0, 2, n).astype(np.uint8) << 7))


DECODE = [
    # (name, B, hq, hkv, lens, opts, layout)
    ("direct_gqa4", 4, 16, 4, [3, 32, 17, 41], {}, "NHD"),
    ("direct_mha16", 2, 8, 8, [100, 300], {}, "NHD"),
    ("balanced_gqa4_teams7", 5, 32, 8, [40, 1000, 17, 3000, 256], {"teams": 7}, "NHD"),
    ("balanced_gqa8", 3, 64, 8, [2049, 700, 5000], {"max_total_pages": 600}, "NHD"),
    ("balanced_gqa4_hnd", 4, 32, 8, [513, 1, 4097, 64], {"teams": 9}, "HND"),
]


@pytest.mark.parametrize("case", DECODE, ids=lambda c: c[0])
def test_fp8_decode_matches_oracle(L, oracle, case):
    name, B, hq, hkv, lens, opts, layout = case
    log(f"fp8 decode {name}")
    rng = np.random.default_rng(len(name) * 7)
    pool = sum((x + 15) // 16 for x in lens) + 4
    ip, ix, last = ragged_table(rng, lens, pool)
    q = seeded_normal_bf16(oracle, rng, B * hq * 128)
    n = pool * 16 * hkv * 128
    k8, v8 = random_fp8(rng, n, 0x5F), random_fp8(rng, n)
    ks, vs = 0.0625, 0.01
    ref = oracle.paged_decode_fp8(oracle.paged_spec(B, pool, hq, hkv), q, k8, v8, ip, ix, last,
                                  ks, vs)
    spec = L.Bf16PagedBatchDecodeSpec(B, pool, hq, hkv, kv_layout=layout, kv_dtype="fp8_e4m3")
    kd, vd = (to_hnd(k8, pool, hkv), to_hnd(v8, pool, hkv)) if layout == "HND" else (k8, v8)
    out, lse, plan = run_decode(L, spec, opts, q, kd, vd, ip, ix, last, [ks, vs])
    log(f"  {plan.algorithm} teams={plan.info.teams} {compare_decode(oracle, out, lse, *ref)}")


def test_every_finite_code_decodes(L, oracle):
    # One request whose V rows hold all 254 finite codes and whose query is
    # zero: the output is the mean of the decoded V rows exactly as the oracle.
    rng = np.random.default_rng(3)
    hq = hkv = 1
    codes = np.array([c for c in range(256) if c not in (0x7F, 0xFF)], np.uint8)
    L_ = len(codes)
    pool = (L_ + 15) // 16
    ip, ix, last = ragged_table(rng, [L_], pool)
    k8 = np.zeros(pool * 16 * 128, np.uint8)
    v8 = np.zeros((pool, 16, 128), np.uint8)
    for t in range(L_):
        v8[ix[t // 16], t % 16] = np.roll(codes, t)[:128]
    ref = oracle.paged_decode_fp8(oracle.paged_spec(1, pool, 1, 1), np.zeros(128, np.uint16),
                                  k8, v8.reshape(-1), ip, ix, last, 1.0, 1.0)
    spec = L.Bf16PagedBatchDecodeSpec(1, pool, hq, hkv, kv_dtype="fp8_e4m3")
    out, lse, _ = run_decode(L, spec, {}, np.zeros(128, np.uint16), k8, v8.reshape(-1), ip, ix,
                             last, [1.0, 1.0])
    compare_decode(oracle, out, lse, *ref)


def test_fp8_plan_requires_scales(L, oracle):
    import torch
    spec = L.Bf16PagedBatchDecodeSpec(1, 2, 8, 8, kv_dtype="fp8_e4m3")
    assert spec.kv_dtype == "fp8_e4m3"
    z8 = np.zeros(2 * 16 * 8 * 128, np.uint8)
    q = np.zeros(8 * 128, np.uint16)
    with pytest.raises(L.LoomError):
        run_decode(L, spec, {}, q, z8, z8, [0, 1], [1], [1], None)
    with pytest.raises(L.EnqueueError) as e:
        run_decode(L, spec, {}, q, z8, z8, [0, 1], [1], [1], [1.0, 1.0, 1.0])
    assert e.value.variant == "LengthMismatch" and e.value.operand == "kv_scales"
    torch.cuda.synchronize()


def run_append(L, spec, explicit, q, k, v, bi, pos, ip, ix, last, kp8, vp8, scales):
    import torch
    prov = L.RopeProvider.load(0)
    plan = (prov.plan_bf16_paged_append_tokens(spec) if explicit
            else prov.plan_bf16_paged_append(spec))
    ws = torch.zeros(plan.workspace_bytes, dtype=torch.uint8, device="cuda")
    qo = nan_bf16(spec.query_output_numel)
    kp, vp = dev_u8(kp8), dev_u8(vp8)
    queue = L.CommandQueue(torch.cuda.current_stream(), 2)
    b = queue.bindings(13)
    h = dict(query=b.bind_read(to_dev_bf16(q)), key=b.bind_read(to_dev_bf16(k)),
             value=b.bind_read(to_dev_bf16(v)), page_indptr=b.bind_read(to_dev_i32(ip)),
             page_indices=b.bind_read(to_dev_i32(ix)), last_page_len=b.bind_read(to_dev_i32(last)),
             query_output=b.bind_read_write(qo), key_pages=b.bind_read_write(kp),
             value_pages=b.bind_read_write(vp), workspace=b.bind_read_write(ws),
             kv_scales=b.bind_read(dev_f32(scales)))
    if explicit:
        h["batch_indices"] = b.bind_read(to_dev_i32(bi))
        h["positions"] = b.bind_read(to_dev_i32(pos))
    args = L.Bf16RopePagedKvAppendArgs(
        h["query"], h["key"], h["value"], h["page_indptr"], h["page_indices"],
        h["last_page_len"], h["query_output"].write(), h["key_pages"].write(),
        h["value_pages"].write(), h["workspace"].write(), h.get("batch_indices"),
        h.get("positions"), h["kv_scales"])
    scope = queue.begin(b)
    plan.enqueue_into(scope, args)
    b = scope.finish().wait()
    return (bf16_host(b.take_read_write(h["query_output"])),
            b.take_read_write(h["key_pages"]).cpu().numpy(),
            b.take_read_write(h["value_pages"]).cpu().numpy())


@pytest.mark.parametrize("explicit", [False, True], ids=["one_token", "explicit_tokens"])
def test_fp8_append_matches_oracle_then_decodes(L, oracle, explicit):
    log(f"fp8 append explicit={explicit}")
    rng = np.random.default_rng(41 + explicit)
    B, hq, hkv, pool = 4, 32, 8, 24
    lens = [40, 200, 17, 90]
    ip, ix, last = ragged_table(rng, lens, pool)
    if explicit:
        bi = np.repeat(np.arange(B), 6).astype(np.int32)
        pos = np.concatenate([np.arange(L_ - 6, L_) for L_ in lens]).astype(np.int32)
        T = len(bi)
        spec = L.Bf16RopePagedKvAppendTokensSpec(T, B, pool, hq, hkv, kv_dtype="fp8_e4m3")
    else:
        bi = np.arange(B, dtype=np.int32)
        pos = np.array([L_ - 1 for L_ in lens], np.int32)
        T = B
        spec = L.Bf16RopePagedKvAppendSpec(B, pool, hq, hkv, kv_dtype="fp8_e4m3")
    q = seeded_normal_bf16(oracle, rng, T * hq * 128)
    k = seeded_normal_bf16(oracle, rng, T * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, T * hkv * 128)
    n = pool * 16 * hkv * 128
    kp8, vp8 = random_fp8(rng, n, 0x5F), random_fp8(rng, n, 0x5F)
    ks, vs = 0.02, 0.015
    ek, ev = kp8.copy(), vp8.copy()
    eq = oracle.append_tokens_fp8(oracle.paged_spec(B, pool, hq, hkv), T, q, k, v, bi, pos, ip,
                                  ix, last, ek, ev, ks, vs)
    qo, gk, gv = run_append(L, spec, explicit, q, k, v, bi, pos, ip, ix, last, kp8, vp8, [ks, vs])
    assert within_one_ulp(oracle, qo, eq)[0]
    assert np.array_equal(gv, ev), "V bytes"
    diff = gk != ek
    if diff.any():
        step = np.abs(gk[diff].astype(np.int32) - ek[diff].astype(np.int32))
        same_sign = (gk[diff] & 0x80) == (ek[diff] & 0x80)
        log(f"  K bytes differing: {int(diff.sum())} of {T * hkv * 128} written")
        assert np.all(same_sign & (step == 1)) and diff.sum() <= max(4, T * hkv * 128 // 2000)
    # decode over the pages the append wrote (the full extended requests)
    qd = seeded_normal_bf16(oracle, rng, B * hq * 128)
    ref = oracle.paged_decode_fp8(oracle.paged_spec(B, pool, hq, hkv), qd, gk, gv, ip, ix, last,
                                  ks, vs)
    dspec = L.Bf16PagedBatchDecodeSpec(B, pool, hq, hkv, kv_dtype="fp8_e4m3")
    out, lse, _ = run_decode(L, dspec, {"teams": 5}, qd, gk, gv, ip, ix, last, [ks, vs])
    log(f"  decode after append {compare_decode(oracle, out, lse, *ref)}")


def test_fp8_append_chunked_path_matches_oracle(L, oracle):
    """The chunk-validated append (T > 64 tokens) on FP8 E4M3 pages against
    the FP8 oracle (same bar as the small path: V bytes exact, K bytes within
    one code where the encode's input differs by the RoPE rounding)."""
    log("fp8 append chunked path")
    rng = np.random.default_rng(97)
    B, hq, hkv = 4, 8, 2
    lens = [40, 300, 17, 129]
    pool = sum((n + 15) // 16 for n in lens) + 4
    ip, ix, last = ragged_table(rng, lens, pool)
    T = 120
    flat = rng.choice(int(sum(lens)), size=T, replace=False)
    starts = np.concatenate([[0], np.cumsum(lens)])
    bi = (np.searchsorted(starts, flat, side="right") - 1).astype(np.int32)
    pos = (flat - starts[bi]).astype(np.int32)
    spec = L.Bf16RopePagedKvAppendTokensSpec.extended(T, B, pool, hq, hkv, kv_dtype="fp8_e4m3")
    q = seeded_normal_bf16(oracle, rng, T * hq * 128)
    k = seeded_normal_bf16(oracle, rng, T * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, T * hkv * 128)
    n = pool * 16 * hkv * 128
    kp8, vp8 = random_fp8(rng, n, 0x5F), random_fp8(rng, n, 0x5F)
    ks, vs = 0.02, 0.015
    ek, ev = kp8.copy(), vp8.copy()
    eq = oracle.append_tokens_fp8(oracle.paged_spec(B, pool, hq, hkv), T, q, k, v, bi, pos, ip,
                                  ix, last, ek, ev, ks, vs, max_tokens=8192)
    qo, gk, gv = run_append(L, spec, True, q, k, v, bi, pos, ip, ix, last, kp8, vp8, [ks, vs])
    check_rope(oracle, qo, eq, q, np.repeat(pos, hq), "query")
    assert np.array_equal(gv, ev), "V bytes"
    diff = gk != ek
    if diff.any():
        step = np.abs(gk[diff].astype(np.int32) - ek[diff].astype(np.int32))
        same_sign = (gk[diff] & 0x80) == (ek[diff] & 0x80)
        log(f"  K bytes differing: {int(diff.sum())} of {T * hkv * 128} written")
        assert np.all(same_sign & (step == 1)) and diff.sum() <= max(4, T * hkv * 128 // 2000)
