"""Benchmark of the paged-KV decode path on one MI355X.

Headline (the JSON line's `value`): paged decode attention on BASELINE config 3
(batch 64, GQA4 32/8 heads, D128, BF16, page 16, ragged context U[512,8192],
pages scattered over a 65536-page pool) in achieved HBM GB/s, with inputs
resident in HBM.  A step is one decode call (one kernel) over that batch.

The same run reports every BASELINE config under `detail` (µs/call eager and
hipGraph replay, GB/s, fraction of the 8 TB/s roofline), the roofline of the
decode kernel measured with HIP events on its own stream, and the CPU oracle
timed on this host over a bounded sample of the same workload.

    python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--quick]
"""
import argparse
import json
import math
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "loom-kernels_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def algorithmic_decode_bytes(lens, B, hq, hkv):
    """Σ kv_len·Hkv·128·2·2 + Q read + O write + LSE + metadata (K/V counted once
    per kv-head regardless of how the kernel reads them)."""
    n_pages = int(sum((int(x) + 15) // 16 for x in lens))
    return (int(sum(int(x) for x in lens)) * hkv * 128 * 2 * 2 + 2 * B * hq * 128 * 2
            + 4 * B * hq + 4 * (2 * B + 1 + n_pages))


class DecodeCase:
    """Device-resident synthetic workload for one decode config."""

    def __init__(self, L, name, B, hq, hkv, pool, lens, seed, chunk_pages=0):
        import numpy as np
        import torch
        self.name, self.B, self.hq, self.hkv, self.pool = name, B, hq, hkv, pool
        rng = np.random.default_rng(seed)
        self.lens = np.asarray(lens, dtype=np.int64)
        pages = (self.lens + 15) // 16
        indptr = np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)
        indices = rng.permutation(pool)[: int(indptr[-1])].astype(np.int32)
        last = (self.lens - (pages - 1) * 16).astype(np.int32)
        self.indptr_h, self.indices_h, self.last_h = indptr, indices, last
        dev = "cuda"
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        self.q = torch.randn(B * hq * 128, generator=g, device=dev).to(torch.bfloat16)
        n = pool * 16 * hkv * 128
        self.k = torch.empty(n, dtype=torch.bfloat16, device=dev)
        self.v = torch.empty(n, dtype=torch.bfloat16, device=dev)
        step = 1 << 28
        for buf in (self.k, self.v):
            for s in range(0, n, step):
                e = min(n, s + step)
                buf[s:e] = torch.randn(e - s, generator=g, device=dev).to(torch.bfloat16)
        self.indptr = torch.from_numpy(indptr).to(dev)
        self.indices = torch.from_numpy(indices).to(dev)
        self.last = torch.from_numpy(last).to(dev)
        self.out = torch.empty(B * hq * 128, dtype=torch.bfloat16, device=dev)
        self.lse = torch.empty(B * hq, dtype=torch.float32, device=dev)
        self.spec = L.Bf16PagedBatchDecodeSpec(B, pool, hq, hkv, 128, 16)
        self.plan = L.DecodeProvider.load(0).plan_bf16_paged_batch(
            self.spec, max_total_pages=int(indptr[-1]), chunk_pages=chunk_pages,
            expected_kv_len=int(self.lens.mean()))
        self.ws = torch.zeros(self.plan.workspace_bytes, dtype=torch.uint8, device=dev)
        self.bytes = algorithmic_decode_bytes(self.lens, B, hq, hkv)
        self.L = L

    def bind(self, b):
        L = self.L
        h = [b.bind_read(self.q), b.bind_read(self.k), b.bind_read(self.v),
             b.bind_read(self.indptr), b.bind_read(self.indices), b.bind_read(self.last),
             b.bind_read_write(self.out), b.bind_read_write(self.lse),
             b.bind_read_write(self.ws)]
        return L.Bf16PagedBatchDecodeArgs(h[0], h[1], h[2], h[3], h[4], h[5], h[6].write(),
                                          h[7].write(), h[8].write())


def time_eager(L, case, stream, steps, warmup):
    """hipEvent pair around `steps` back-to-back enqueues on one stream, per call
    (the reference's eager_stream_batch_cuda_event, benchmarks/matched.rs:141-173)."""
    import torch
    q = L.CommandQueue(stream, steps + warmup + 1)
    b = q.bindings(9)
    args = case.bind(b)
    with torch.cuda.stream(stream):
        scope = q.begin(b)
        for _ in range(warmup):
            case.plan.enqueue_into(scope, args)
        b = scope.finish().wait()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        scope = q.begin(b)
        torch.cuda.synchronize()
        start.record(stream)
        for _ in range(steps):
            case.plan.enqueue_into(scope, args)
        end.record(stream)
        b = scope.finish().wait()
        torch.cuda.synchronize()
    return start.elapsed_time(end) * 1000.0 / steps  # µs per call


def time_graph(L, case, replays=20):
    """One fixed-address replay + its completion event per sample (graph/mod.rs:301-323);
    returns the median µs."""
    import torch
    gq = L.GraphQueue(0, 1)
    b = gq.bindings(9)
    args = case.bind(b)
    graph = gq.capture(b, lambda scope: case.plan.enqueue_into(scope, args))
    exec_ = graph.instantiate()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    samples = []
    for i in range(replays + 3):
        ms = exec_.measure_launch_ms(start, end)
        if i >= 3:
            samples.append(ms * 1000.0)
    exec_.into_bindings()
    samples.sort()
    return samples[len(samples) // 2]


def cpu_baseline(case, budget_s=12.0):
    """The oracle (single thread, the reference's loop order) on a bounded
    sample of whole requests of the same workload, scaled to GB/s."""
    import numpy as np
    import torch
    import oracle as O
    # host copies of only the pages the sample touches, renumbered
    order = np.argsort(case.lens)  # sample spans short to long requests evenly
    pick = order[np.linspace(0, len(order) - 1, num=min(len(order), 8)).astype(int)]
    done_bytes, t_total, reqs = 0, 0.0, 0
    kk = case.k.view(case.pool, -1)
    vv = case.v.view(case.pool, -1)
    for r in pick:
        pg = case.indices_h[case.indptr_h[r]:case.indptr_h[r + 1]].astype(np.int64)
        idx = torch.from_numpy(pg).cuda()
        kh = kk[idx].reshape(-1).view(torch.int16).cpu().numpy().view(np.uint16)
        vh = vv[idx].reshape(-1).view(torch.int16).cpu().numpy().view(np.uint16)
        qh = case.q[r * case.hq * 128:(r + 1) * case.hq * 128].view(torch.int16).cpu().numpy().view(np.uint16)
        n = len(pg)
        s = O.paged_spec(1, n, case.hq, case.hkv)
        out = np.empty(case.hq * 128, np.uint16)
        lse = np.empty(case.hq, np.float32)
        t0 = time.perf_counter()
        O.paged_decode_requests(s, qh, kh, vh, [0, n], np.arange(n, dtype=np.int32),
                                [int(case.last_h[r])], 0, 1, out, lse)
        t_total += time.perf_counter() - t0
        done_bytes += algorithmic_decode_bytes([case.lens[r]], 1, case.hq, case.hkv)
        reqs += 1
        if t_total > budget_s:
            break
    return {"value": done_bytes / t_total / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{reqs} whole requests of the same workload (lengths "
                      f"{sorted(int(case.lens[r]) for r in pick[:reqs])}), oracle loop "
                      f"order, {t_total:.1f} s, single thread on {platform.processor() or 'host'}"}


def make_cases(L, quick=False):
    import numpy as np
    rng = np.random.default_rng(2026)
    cases = {}
    # config 1: MHA b1 ctx 1024, 64 of a 128-page pool
    cases["c1_mha_b1_ctx1024"] = (1, 32, 32, 128, [1024])
    # config 3: batch-64 GQA4 ragged U[512,8192], pool 65536
    cases["c3_gqa4_b64_ragged"] = (64, 32, 8, 65536, list(rng.integers(512, 8193, size=64)))
    if not quick:
        # config 4: GQA8 b8 ctx 32768
        cases["c4_gqa8_b8_ctx32768"] = (8, 64, 8, 8 * 2048 + 64, [32768] * 8)
        # config 5 decode part: b256 lognormal(median 2048, sigma 0.8) clipped [16,16384]
        l5 = np.clip(np.round(np.exp(np.log(2048) + 0.8 * rng.standard_normal(256))), 16,
                     16384).astype(int)
        cases["c5_gqa4_b256_lognormal"] = (256, 32, 8, 262144, list(l5))
    return cases


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--quick", action="store_true", help="configs 1 and 3 only")
    ap.add_argument("--no-cpu", action="store_true")
    a = ap.parse_args()
    if a.gpus != 1:
        print("bench.py measures one GPU: every GPU box here has one MI355X and the path "
              "has no cross-GPU component; run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    import loom_infer_hip as L
    torch.cuda.set_device(0)
    stream = torch.cuda.Stream()  # default priority
    detail = {}
    head = None
    for name, (B, hq, hkv, pool, lens) in make_cases(L, a.quick).items():
        log(f"[bench] setting up {name}")
        case = DecodeCase(L, name, B, hq, hkv, pool, lens, seed=len(name))
        us = time_eager(L, case, stream, a.steps, a.warmup)
        g_us = time_graph(L, case)
        gbs = case.bytes / (us * 1e-6) / 1e9
        detail[name] = {"us_per_call": round(us, 3), "graph_replay_us": round(g_us, 3),
                        "GBps": round(gbs, 1), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                        "algorithmic_bytes": case.bytes,
                        "chunk_pages": case.plan.info.chunk_pages,
                        "mean_kv_len": float(case.lens.mean())}
        log(f"[bench] {name}: {detail[name]}")
        if name.startswith("c3"):
            head = case
        else:
            del case
            torch.cuda.empty_cache()
    c3 = detail["c3_gqa4_b64_ragged"]
    cpu = None if a.no_cpu else cpu_baseline(head)
    line = {
        "metric": "paged-decode achieved HBM GB/s (% of peak) + µs/call; RoPE+append µs/call",
        "value": c3["GBps"], "unit": "GB/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(c3["us_per_call"] / 1000.0, 6),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: q/K/V ~ N(0,1) cast to bf16 on device, seeded permutation page tables",
        "config": {"workload": "paged decode GQA4 batch 64, 32 q / 8 kv heads, D128, page 16, "
                               "ragged ctx U[512,8192], 65536-page pool (BASELINE config 3)",
                   "global_batch": 64, "seq_len": int(head.lens.max()), "parallelism": "none"},
        "roofline": {"bound": "hbm", "achieved": c3["GBps"], "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": c3["frac_hbm_peak"], "traffic": None},
        "cpu_baseline": cpu,
        "detail": detail,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
