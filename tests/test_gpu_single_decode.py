"""GPU parity of contiguous single decode (direct and split-K) through the C
ABI against the pinned oracle (crates/loom-infer/src/attention/single_decode/
mod.rs:197-381), on the reference's own fixture tuples and seeded shapes."""
import json
import os
import zlib

import numpy as np
import pytest

from gpu_util import bf16_host, compare_decode, seeded_normal_bf16, to_dev_bf16

pytestmark = pytest.mark.gpu

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                     "reference_digests.json")))


@pytest.fixture(scope="module")
def L():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import loom_infer_hip as L
    return L


def run_single(L, spec, q, k, v, partitions=None, workspace_out=None):
    import torch
    prov = L.DecodeProvider.load(0)
    dev = "cuda"
    tq, tk, tv = to_dev_bf16(q), to_dev_bf16(k), to_dev_bf16(v)
    o = torch.full((spec.output_numel,), float("nan"), dtype=torch.bfloat16, device=dev)
    lse = torch.full((spec.lse_numel,), float("nan"), dtype=torch.float32, device=dev)
    queue = L.CommandQueue(torch.cuda.current_stream(), 2)
    b = queue.bindings(6)
    if partitions is None:
        plan = prov.plan_bf16(spec)
        args = L.Bf16SingleDecodeArgs(b.bind_read(tq), b.bind_read(tk), b.bind_read(tv),
                                      b.bind_read_write(o).write(), b.bind_read_write(lse).write())
    else:
        sk = L.Bf16SingleDecodeSplitKSpec(spec, partitions)
        plan = prov.plan_bf16_split_k(sk)
        assert plan.workspace_required_numel == sk.workspace_numel
        ws = torch.full((sk.workspace_numel,), float("nan"), dtype=torch.float32, device=dev)
        hws = b.bind_read_write(ws)
        args = L.Bf16SingleDecodeSplitKArgs(b.bind_read(tq), b.bind_read(tk), b.bind_read(tv),
                                            hws, b.bind_read_write(o).write(),
                                            b.bind_read_write(lse).write())
    scope = queue.begin(b)
    plan.enqueue_into(scope, args)
    comp = scope.finish()
    assert comp.submitted() == (1 if partitions is None else 2)
    comp.wait()
    if workspace_out is not None and partitions is not None:
        workspace_out.append(ws.cpu().numpy())
    return bf16_host(o), lse.cpu().numpy()


def fixture(oracle, kv_len, hq, hkv, salt):
    n = kv_len * hkv * 128
    return (oracle.deterministic_bf16(hq * 128, salt), oracle.deterministic_bf16(n, salt ^ 0x4B455900),
            oracle.deterministic_bf16(n, salt ^ 0x5641_4C55_4500))


@pytest.mark.parametrize("case", GOLDEN["single_decode_direct"]["cases"], ids=lambda c: c["name"])
def test_reference_fixtures_direct_and_split_k(L, oracle, case):
    # crates/loom-infer-validation/src/gates/single_decode.rs:146-170 fixtures
    kv_len, hq, hkv = case["kv_len"], case["hq"], case["hkv"]
    q, k, v = fixture(oracle, kv_len, hq, hkv, int(case["salt"], 16))
    s = oracle.single_spec(kv_len, hq, hkv)
    ref_o, ref_l = oracle.single_decode(s, q, k, v)
    spec = L.Bf16SingleDecodeSpec(kv_len, hq, hkv)
    o, l = run_single(L, spec, q, k, v)
    compare_decode(oracle, o, l, ref_o, ref_l)
    ws = []
    o2, l2 = run_single(L, spec, q, k, v, case["partitions"], ws)
    compare_decode(oracle, o2, l2, ref_o, ref_l)
    # the partial states follow the reference layout [Hq, P, 130]
    _, _, ref_ws = oracle.split_k(s, case["partitions"], q, k, v)
    got = ws[0].reshape(-1, 130)
    want = ref_ws.reshape(-1, 130)
    np.testing.assert_allclose(got[:, 0], want[:, 0], atol=1e-4, rtol=1e-5)
    np.testing.assert_allclose(got[:, 1], want[:, 1], rtol=1e-4)
    np.testing.assert_allclose(got[:, 2:], want[:, 2:], atol=2e-3, rtol=1e-3)


SHAPES = [
    # (kv_len, hq, hkv, partitions)
    (1, 8, 8, 1), (15, 32, 8, 2), (16, 8, 1, 3), (17, 16, 1, 5), (1000, 32, 8, 7),
    (4097, 64, 8, 16), (300, 48, 2, 9), (2049, 32, 32, 33),
]


@pytest.mark.parametrize("kv_len,hq,hkv,parts", SHAPES,
                         ids=[f"L{s[0]}_q{s[1]}_kv{s[2]}_p{s[3]}" for s in SHAPES])
def test_seeded_shapes(L, oracle, kv_len, hq, hkv, parts):
    rng = np.random.default_rng(zlib.crc32(f"{kv_len}-{hq}-{hkv}".encode()))
    q = seeded_normal_bf16(oracle, rng, hq * 128)
    k = seeded_normal_bf16(oracle, rng, kv_len * hkv * 128)
    v = seeded_normal_bf16(oracle, rng, kv_len * hkv * 128)
    s = oracle.single_spec(kv_len, hq, hkv)
    ref_o, ref_l = oracle.single_decode(s, q, k, v)
    spec = L.Bf16SingleDecodeSpec(kv_len, hq, hkv)
    compare_decode(oracle, *run_single(L, spec, q, k, v), ref_o, ref_l)
    compare_decode(oracle, *run_single(L, spec, q, k, v, parts), ref_o, ref_l)


def test_large_logits_stay_finite(L, oracle):
    # single_decode/tests.rs:357-387 on the device
    f = lambda x: oracle.bf16_from_f32(np.asarray(x, np.float32))
    q = np.full(128, f([64.0])[0], np.uint16)
    k = f(np.concatenate([np.full(128, -64.0), np.zeros(128), np.full(128, 64.0)]))
    v = np.full(384, f([1.0])[0], np.uint16)
    spec = L.Bf16SingleDecodeSpec(3, 1, 1)
    for parts in (None, 3):
        o, l = run_single(L, spec, q, k, v, parts)
        assert np.all(np.isfinite(oracle.bf16_to_f32(o))) and np.all(np.isfinite(l))


def test_split_k_rejections_submit_nothing(L):
    import torch
    spec = L.Bf16SingleDecodeSpec(64, 8, 2)
    plan = L.DecodeProvider.load(0).plan_bf16_split_k(L.Bf16SingleDecodeSplitKSpec(spec, 4))
    dev = "cuda"
    q = torch.zeros(spec.query_numel, dtype=torch.bfloat16, device=dev)
    k = torch.zeros(spec.kv_numel, dtype=torch.bfloat16, device=dev)
    o = torch.zeros(spec.output_numel, dtype=torch.bfloat16, device=dev)
    lse = torch.zeros(spec.lse_numel, dtype=torch.float32, device=dev)
    # a queue with room for one command cannot take the two-command split-K pair
    queue = L.CommandQueue(torch.cuda.current_stream(), 1)
    b = queue.bindings(6)
    ws = torch.zeros(8 * 4 * 130, dtype=torch.float32, device=dev)
    args = L.Bf16SingleDecodeSplitKArgs(b.bind_read(q), b.bind_read(k), b.bind_read(k.clone()),
                                        b.bind_read_write(ws), b.bind_read_write(o).write(),
                                        b.bind_read_write(lse).write())
    scope = queue.begin(b)
    with pytest.raises(L.CommandError) as e:
        plan.enqueue_into(scope, args)
    assert e.value.variant == "CommandCapacityExceeded"
    comp = scope.finish()
    assert comp.submitted() == 0
    comp.wait()
    # wrong workspace length
    queue = L.CommandQueue(torch.cuda.current_stream(), 2)
    b = queue.bindings(6)
    ws = torch.zeros(8 * 4 * 130 - 1, dtype=torch.float32, device=dev)
    args = L.Bf16SingleDecodeSplitKArgs(b.bind_read(q), b.bind_read(k), b.bind_read(k.clone()),
                                        b.bind_read_write(ws), b.bind_read_write(o).write(),
                                        b.bind_read_write(lse).write())
    scope = queue.begin(b)
    with pytest.raises(L.EnqueueError) as e:
        plan.enqueue_into(scope, args)
    assert (e.value.variant, e.value.operand) == ("LengthMismatch", "workspace")
    comp = scope.finish()
    assert comp.submitted() == 0
    comp.wait()
