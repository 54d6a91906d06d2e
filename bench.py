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
                    [--records gpurun_out/bench_records.jsonl]

Besides the one JSON line on stdout, every decode and append config writes
evidence records (JSON Lines, the reference's BenchmarkRecord schema) to
--records: raw per-sample µs, fixture digests, kernels per call and the build's
source commit.
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
# HBM bytes per decode launch on config 3 from rocprofv3 --pmc FETCH_SIZE and
# WRITE_SIZE (partial + merge kernels), each scaled by the factor the same
# counter reads for a plain copy of known size; profiles/ holds the runs.
TRAFFIC_C3 = 1.1494e9


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ---- evidence records ---------------------------------------------------------
# One JSON line per (config, measurement) in the reference's BenchmarkRecord
# schema (crates/loom-infer-validation/src/support/benchmark.rs:5-24): raw
# per-sample µs, fixture digests of the seeded inputs, kernels per call and the
# source commit of the build (loom-kernels_amd/lib/BUILD_INFO.json, written by
# build_lib.sh; the GPU box has no git metadata).
BUILD_INFO = os.path.join(ROOT, "loom-kernels_amd", "lib", "BUILD_INFO.json")
RECORDS = []


def fnv1a64(data: bytes) -> str:
    h = 0xCBF29CE484222325
    for b in data:
        h = ((h ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return f"{h:016x}"


def host_digest(a) -> str:
    """FNV-1a 64 of a host array's bytes (metadata: page tables, positions)."""
    import numpy as np
    return fnv1a64(np.ascontiguousarray(a).tobytes())


def device_digest(t) -> str:
    """A position-weighted 64-bit checksum of a device tensor's 16-bit words,
    Σ u16[i]·(i mod 65521 + 1) mod 2^64, computed on the GPU in chunks (the
    K/V pools are GBs; hashing them on the host would take minutes)."""
    import torch
    w16 = t.reshape(-1).view(torch.int16)
    n = w16.numel()
    total = 0
    step = 1 << 26
    for s0 in range(0, n, step):
        e0 = min(n, s0 + step)
        v = w16[s0:e0].to(torch.int64) & 0xFFFF
        wt = torch.arange(s0, e0, dtype=torch.int64, device=t.device) % 65521 + 1
        total = (total + int((v * wt).sum().item())) & 0xFFFFFFFFFFFFFFFF
    return f"{total:016x}"


def execution_info():
    import torch
    p = torch.cuda.get_device_properties(0)
    return {"device": p.name, "arch": getattr(p, "gcnArchName", ""), "cus": p.multi_processor_count,
            "hip": torch.version.hip, "torch": torch.__version__, "host": platform.node(),
            "stream": "one non-default stream, default priority"}


def record(operator, case, kernels_per_call, shape, fixture_id, digests, warmup, per_sample,
           samples_us, measurement, layout="NHD, page 16", dtype="bf16"):
    """Appends one BenchmarkRecord (benchmark.rs:5-24) to RECORDS."""
    info = {}
    if os.path.exists(BUILD_INFO):
        info = json.load(open(BUILD_INFO))
    RECORDS.append({
        "schema_version": 1, "provider": "loom-infer-hip",
        "provider_version": info.get("abi_version", "1"),
        "provider_commit": info.get("commit", "unknown"),
        "provider_worktree_dirty": info.get("dirty"),
        "provider_library_sha256": info.get("library_sha256"),
        "run_label": os.environ.get("LOOM_BENCH_RUN_LABEL", "bench.py"),
        "measurement": measurement, "operator": operator, "case": case, "dtype": dtype,
        "layout": layout, "execution": execution_info(), "kernels_per_call": kernels_per_call,
        "shape": shape, "fixture_id": fixture_id, "fixture_digests": digests,
        "warmup_launches": warmup, "launches_per_sample": per_sample,
        "samples_us": [round(x, 4) for x in samples_us]})


def write_records(path):
    if not path:
        return
    d = os.path.dirname(path)
    if d:
        os.makedirs(d, exist_ok=True)
    with open(path, "w") as f:
        for r in RECORDS:
            f.write(json.dumps(r) + "\n")
    log(f"[bench] wrote {len(RECORDS)} evidence records to {path}")


def decode_kernels_per_call(plan) -> int:
    """Launches per decode command: the balanced split-KV plan and a split
    direct plan add a merge kernel; an unsplit direct plan is one kernel."""
    i = plan.info
    return 1 if (plan.algorithm == "direct" and i.teams <= 1) else 2


def algorithmic_decode_bytes(lens, B, hq, hkv):
    """Σ kv_len·Hkv·128·2·2 + Q read + O write + LSE + metadata (K/V counted once
    per kv-head regardless of how the kernel reads them)."""
    n_pages = int(sum((int(x) + 15) // 16 for x in lens))
    return (int(sum(int(x) for x in lens)) * hkv * 128 * 2 * 2 + 2 * B * hq * 128 * 2
            + 4 * B * hq + 4 * (2 * B + 1 + n_pages))


class DecodeCase:
    """Device-resident synthetic workload for one decode config."""

    def __init__(self, L, name, B, hq, hkv, pool, lens, seed, teams=0, arena=None):
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
        if arena is not None:  # the config's K/V pools, allocated once (see kv_arenas)
            self.k, self.v = arena[:n], arena[n:2 * n]
        else:
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
        self.seed = seed
        self.spec = L.Bf16PagedBatchDecodeSpec(B, pool, hq, hkv, 128, 16)
        self.plan = L.DecodeProvider.load(0).plan_bf16_paged_batch(
            self.spec, max_total_pages=int(indptr[-1]), teams=teams)
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


def _timed_enqueues(L, stream, n_bind, bind, enqueue, steps, warmup, commands_per_call=1):
    """hipEvent pair around `steps` back-to-back enqueues on one stream, per call
    (the reference's eager_stream_batch_cuda_event, benchmarks/matched.rs:141-173).
    The events are recorded on the stream the kernels are launched on.
    `commands_per_call`: commands one enqueue submits (the queue's capacity)."""
    import torch
    q = L.CommandQueue(stream, (steps + warmup) * commands_per_call + 1)
    b = q.bindings(n_bind)
    args = bind(b)
    with torch.cuda.stream(stream):
        scope = q.begin(b)
        for _ in range(warmup):
            enqueue(scope, args)
        b = scope.finish().wait()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        scope = q.begin(b)
        torch.cuda.synchronize()
        start.record(stream)
        for _ in range(steps):
            enqueue(scope, args)
        end.record(stream)
        b = scope.finish().wait()
        torch.cuda.synchronize()
    return start.elapsed_time(end) * 1000.0 / steps  # µs per call


def _sampled_enqueues(L, stream, n_bind, bind, enqueue, samples, per_sample, warmup):
    """`samples` hipEvent intervals, each around `per_sample` back-to-back
    enqueues on the launch stream, divided by `per_sample`: µs per call per
    sample (the reference's raw samples_us, validation support/benchmark.rs:24)."""
    import torch
    q = L.CommandQueue(stream, samples * per_sample + warmup + 1)
    b = q.bindings(n_bind)
    args = bind(b)
    with torch.cuda.stream(stream):
        scope = q.begin(b)
        for _ in range(warmup):
            enqueue(scope, args)
        b = scope.finish().wait()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(samples)]
        scope = q.begin(b)
        torch.cuda.synchronize()
        for st, en in ev:
            st.record(stream)
            for _ in range(per_sample):
                enqueue(scope, args)
            en.record(stream)
        b = scope.finish().wait()
        torch.cuda.synchronize()
    return [st.elapsed_time(en) * 1000.0 / per_sample for st, en in ev]


def _pct(xs, q):
    xs = sorted(xs)
    i = min(len(xs) - 1, max(0, int(round(q * (len(xs) - 1)))))
    return xs[i]


def draw_lens(name, seed):
    """Request lengths of a config for one stats seed (configs 3 and 5 draw
    theirs from the stated distributions; 1 and 4 are fixed)."""
    import numpy as np
    rng = np.random.default_rng(seed)
    if name.startswith("c3"):
        return list(rng.integers(512, 8193, size=64))
    if name.startswith("c5"):
        return list(np.clip(np.round(np.exp(np.log(2048) + 0.8 * rng.standard_normal(256))), 16,
                            16384).astype(int))
    if name.startswith("c4"):
        return [32768] * 8
    return [1024]


def seed_stats(L, stream, name, B, hq, hkv, pool, seeds, samples, per_sample, warmup,
               arena=None):
    """Per-call µs over seeds 0..n-1 (each seed its own lengths, page table and
    inputs): median / p10 / p90 over every sample, and each seed's median."""
    import torch
    us_all, gbs_all, per_seed = [], [], []
    for sd in seeds:
        case = DecodeCase(L, name, B, hq, hkv, pool, draw_lens(name, sd), seed=sd, arena=arena)
        xs = _sampled_enqueues(L, stream, 9, case.bind, case.plan.enqueue_into, samples,
                               per_sample, warmup)
        us_all += xs
        gbs_all += [case.bytes / (x * 1e-6) / 1e9 for x in xs]
        per_seed.append({"seed": sd, "median_us": round(_pct(xs, 0.5), 3),
                         "mean_kv_len": round(float(case.lens.mean()), 1),
                         "algorithmic_bytes": case.bytes})
        del case
        torch.cuda.empty_cache()
    return {"samples": len(us_all), "calls_per_sample": per_sample,
            "median_us": round(_pct(us_all, 0.5), 3), "p10_us": round(_pct(us_all, 0.1), 3),
            "p90_us": round(_pct(us_all, 0.9), 3),
            "median_GBps": round(_pct(gbs_all, 0.5), 1),
            "p10_GBps": round(_pct(gbs_all, 0.1), 1), "p90_GBps": round(_pct(gbs_all, 0.9), 1),
            "median_frac_hbm_peak": round(_pct(gbs_all, 0.5) / HBM_PEAK_GBS, 4),
            "per_seed": per_seed}


def _timed_rotating(L, stream, n_bind, binders, enqueue, steps, warmup):
    """Like _timed_enqueues, but call i uses input set i % len(binders): with
    the sets together larger than the 256 MB Infinity Cache, every call reads
    its inputs from HBM (the cold-cache figure for small configs)."""
    import torch
    q = L.CommandQueue(stream, steps + warmup + 1)
    b = q.bindings(n_bind * len(binders))
    args = [bind(b) for bind in binders]
    with torch.cuda.stream(stream):
        scope = q.begin(b)
        for i in range(warmup):
            enqueue(scope, args[i % len(args)])
        b = scope.finish().wait()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        scope = q.begin(b)
        torch.cuda.synchronize()
        start.record(stream)
        for i in range(steps):
            enqueue(scope, args[i % len(args)])
        end.record(stream)
        b = scope.finish().wait()
        torch.cuda.synchronize()
    return start.elapsed_time(end) * 1000.0 / steps


def _graph_replay(L, n_bind, n_cmds, bind, record, replays=20, samples_out=None):
    """One fixed-address replay + its completion event per sample
    (graph/mod.rs:301-323); returns the median µs (and appends the raw
    samples to `samples_out` when given)."""
    import torch
    gq = L.GraphQueue(0, n_cmds)
    b = gq.bindings(n_bind)
    args = bind(b)
    exec_ = gq.capture(b, lambda scope: record(scope, args)).instantiate()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    samples = []
    for i in range(replays + 3):
        ms = exec_.measure_launch_ms(start, end)
        if i >= 3:
            samples.append(ms * 1000.0)
    exec_.into_bindings()
    if samples_out is not None:
        samples_out.extend(samples)
    samples.sort()
    return samples[len(samples) // 2]


def time_eager(L, case, stream, steps, warmup):
    return _timed_enqueues(L, stream, 9, case.bind, case.plan.enqueue_into, steps, warmup)


def time_graph(L, case, replays=20, samples_out=None):
    return _graph_replay(L, 9, 1, case.bind, case.plan.enqueue_into, replays, samples_out)


def decode_fixture(case):
    """(fixture_id, digests, shape) of a DecodeCase for its evidence records."""
    fid = (f"{case.name}: lengths and page table from numpy default_rng({case.seed}), "
           f"q/K/V torch.randn(generator seed {case.seed}) cast to bf16")
    dig = {"page_indptr": host_digest(case.indptr_h), "page_indices": host_digest(case.indices_h),
           "last_page_len": host_digest(case.last_h), "query": device_digest(case.q),
           "key_pages": device_digest(case.k), "value_pages": device_digest(case.v),
           "digest_kinds": {"metadata": "fnv1a64 of int32 bytes",
                            "tensors": "sum u16[i]*(i mod 65521 + 1) mod 2^64"}}
    shape = {"batch": case.B, "num_query_heads": case.hq, "num_kv_heads": case.hkv,
             "head_dim": 128, "page_size": 16, "max_num_pages": case.pool,
             "total_pages": int(case.indptr_h[-1]), "kv_len_sum": int(case.lens.sum()),
             "kv_len_min": int(case.lens.min()), "kv_len_max": int(case.lens.max()),
             "algorithmic_bytes": case.bytes, "plan_algorithm": case.plan.algorithm,
             "plan_teams": case.plan.info.teams}
    return fid, dig, shape


class AppendCase:
    """Device-resident fused RoPE + paged append workload.  With `n_new` None it
    is the one-token contract (token at kv_len-1 of every request); otherwise the
    explicit-token contract with n_new[r] tokens at the end of request r, given
    in a seeded shuffled order."""

    def __init__(self, L, B, hq, hkv, pool, lens, seed, n_new=None, share=None):
        import numpy as np
        import torch
        rng = np.random.default_rng(seed)
        lens = np.asarray(lens, dtype=np.int64)
        if share is not None:  # a DecodeCase: same page table and K/V pools
            indptr, indices, last = share.indptr_h, share.indices_h, share.last_h
        else:
            pages = (lens + 15) // 16
            indptr = np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)
            indices = rng.permutation(pool)[: int(indptr[-1])].astype(np.int32)
            last = (lens - (pages - 1) * 16).astype(np.int32)
        self.explicit = n_new is not None
        self.seed = seed
        if self.explicit:
            bi = np.concatenate([np.full(n, r) for r, n in enumerate(n_new)]).astype(np.int32)
            pos = np.concatenate([np.arange(l - n, l) for l, n in zip(lens, n_new)]).astype(np.int32)
            perm = rng.permutation(len(bi))
            bi, pos = bi[perm], pos[perm]
            self.bi_h, self.pos_h = bi, pos
            T = len(bi)
            self.spec = L.Bf16RopePagedKvAppendTokensSpec(T, B, pool, hq, hkv,
                                                          extended=T > 64)
        else:
            T = B
            self.spec = L.Bf16RopePagedKvAppendSpec(B, pool, hq, hkv)
        dev = "cuda"
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        self.T, self.B, self.hq, self.hkv = T, B, hq, hkv
        self.q = torch.randn(T * hq * 128, generator=g, device=dev).to(torch.bfloat16)
        self.k = torch.randn(T * hkv * 128, generator=g, device=dev).to(torch.bfloat16)
        self.v = torch.randn(T * hkv * 128, generator=g, device=dev).to(torch.bfloat16)
        if share is not None:
            self.kp, self.vp = share.k, share.v
            self.indptr, self.indices, self.last = share.indptr, share.indices, share.last
        else:
            n = pool * 16 * hkv * 128
            self.kp = torch.zeros(n, dtype=torch.bfloat16, device=dev)
            self.vp = torch.zeros(n, dtype=torch.bfloat16, device=dev)
            self.indptr = torch.from_numpy(indptr).to(dev)
            self.indices = torch.from_numpy(indices).to(dev)
            self.last = torch.from_numpy(last).to(dev)
        self.tables = (indptr, indices, last)
        if self.explicit:
            self.bi = torch.from_numpy(bi).to(dev)
            self.pos = torch.from_numpy(pos).to(dev)
        self.qo = torch.empty(T * hq * 128, dtype=torch.bfloat16, device=dev)
        prov = L.RopeProvider.load(0)
        self.plan = (prov.plan_bf16_paged_append_tokens(self.spec) if self.explicit
                     else prov.plan_bf16_paged_append(self.spec))
        self.ws = torch.zeros(self.plan.workspace_bytes, dtype=torch.uint8, device=dev)
        # bytes the append must move: q in/out, new k/v in and out, metadata
        self.bytes = (2 * T * hq * 128 * 2 + 2 * 2 * T * hkv * 128 * 2
                      + 4 * (2 * B + 1 + int(indptr[-1])) + (8 * T if self.explicit else 0))
        self.L = L

    def bind(self, b, qo=None, kp=None, vp=None):
        """Handles for the append; pass existing read-write handles to share the
        query output and K/V pools with a decode in the same command scope."""
        L = self.L
        kp = b.bind_read_write(self.kp) if kp is None else kp
        vp = b.bind_read_write(self.vp) if vp is None else vp
        qo = b.bind_read_write(self.qo) if qo is None else qo
        return L.Bf16RopePagedKvAppendArgs(
            b.bind_read(self.q), b.bind_read(self.k), b.bind_read(self.v),
            b.bind_read(self.indptr), b.bind_read(self.indices), b.bind_read(self.last),
            qo.write(), kp.write(), vp.write(), b.bind_read_write(self.ws).write(),
            b.bind_read(self.bi) if self.explicit else None,
            b.bind_read(self.pos) if self.explicit else None)


def time_append(L, case, stream, steps, warmup, graph_samples=None):
    n = 12 if case.explicit else 10
    return (_timed_enqueues(L, stream, n, case.bind, case.plan.enqueue_into, steps, warmup),
            _graph_replay(L, n, 1, case.bind, case.plan.enqueue_into, samples_out=graph_samples))


def record_append(name, app, stream, warmup, graph_samples):
    """Evidence records of an append config: raw eager samples (20 samples of
    10 back-to-back commands) and the graph replays' samples."""
    import torch
    n = 12 if app.explicit else 10
    xs = _sampled_enqueues(app.L, stream, n, app.bind, app.plan.enqueue_into, 20, 10, warmup)
    ip, ix, ln = app.tables
    dig = {"page_indptr": host_digest(ip), "page_indices": host_digest(ix),
           "last_page_len": host_digest(ln), "query": device_digest(app.q),
           "key": device_digest(app.k), "value": device_digest(app.v)}
    if app.explicit:
        dig.update(batch_indices=host_digest(app.bi_h), positions=host_digest(app.pos_h))
    fid = (f"{name}: lengths, page table and token order from numpy default_rng({app.seed}), "
           f"q/k/v torch.randn(generator seed {app.seed}) cast to bf16")
    shape = {"tokens": app.T, "batch": app.B, "num_query_heads": app.hq,
             "num_kv_heads": app.hkv, "head_dim": 128, "page_size": 16,
             "explicit_tokens": app.explicit, "algorithmic_bytes": app.bytes}
    op = "rope_paged_append_tokens" if app.explicit else "rope_paged_append"
    record(op, name, 1, shape, fid, dig, warmup, 10, xs, "eager_stream_batch_hip_event")
    record(op, name, 1, shape, fid, dig, 3, 1, graph_samples, "graph_replay_with_completion_event")
    del torch


def time_full_step(L, app, dec, samples_out=None):
    """Config 5: RoPE + one-token append writing the rotated query and the new
    K/V rows, then paged decode reading them, captured as one graph."""
    def bind(b):
        qo, kp, vp = (b.bind_read_write(app.qo), b.bind_read_write(app.kp),
                      b.bind_read_write(app.vp))
        ip, ix, ln = b.bind_read(app.indptr), b.bind_read(app.indices), b.bind_read(app.last)
        a = L.Bf16RopePagedKvAppendArgs(
            b.bind_read(app.q), b.bind_read(app.k), b.bind_read(app.v), ip, ix, ln,
            qo.write(), kp.write(), vp.write(), b.bind_read_write(app.ws).write())
        d = L.Bf16PagedBatchDecodeArgs(
            qo.read(), kp.read(), vp.read(), ip, ix, ln, b.bind_read_write(dec.out).write(),
            b.bind_read_write(dec.lse).write(), b.bind_read_write(dec.ws).write())
        return a, d

    def record(scope, args):
        app.plan.enqueue_into(scope, args[0])
        dec.plan.enqueue_into(scope, args[1])
    return _graph_replay(L, 16, 2, bind, record, samples_out=samples_out)


def cpu_baseline(case, min_s=10.0, max_s=30.0):
    """The oracle (single thread, the reference's loop order,
    crates/loom-infer/src/attention/paged_decode/mod.rs:305-363) on whole
    requests of the same workload: every request of the batch once, repeated
    until at least `min_s` of CPU work, stopping early at `max_s`.  Each
    request's pages are copied to the host (untimed) and renumbered."""
    import numpy as np
    import torch
    import oracle as O
    kk = case.k.view(case.pool, -1)
    vv = case.v.view(case.pool, -1)
    done_bytes, t_total, reqs, passes = 0, 0.0, 0, 0
    while t_total < min_s:
        for r in range(case.B):
            pg = case.indices_h[case.indptr_h[r]:case.indptr_h[r + 1]].astype(np.int64)
            idx = torch.from_numpy(pg).cuda()
            kh = kk[idx].reshape(-1).view(torch.int16).cpu().numpy().view(np.uint16)
            vh = vv[idx].reshape(-1).view(torch.int16).cpu().numpy().view(np.uint16)
            qh = (case.q[r * case.hq * 128:(r + 1) * case.hq * 128].view(torch.int16)
                  .cpu().numpy().view(np.uint16))
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
            if t_total > max_s:
                break
        passes += 1
        if t_total > max_s:
            break
    cpu = platform.processor() or platform.machine()
    try:
        with open("/proc/cpuinfo") as f:
            cpu = next(l.split(":", 1)[1].strip() for l in f if l.startswith("model name"))
    except (OSError, StopIteration):
        pass
    return {"value": round(done_bytes / t_total / 1e9, 4), "unit": "GB/s", "cores": 1,
            "kind": "port",
            "sample": f"{reqs} whole requests of the config-3 batch ({passes} pass(es) over "
                      f"its 64 requests, {done_bytes / 1e9:.2f} GB algorithmic), C oracle in "
                      f"the reference loop order, {t_total:.1f} s on 1 thread of {cpu} "
                      f"(host has {os.cpu_count()} logical CPUs)"}


def cpu_baseline_parallel(case, threads=16, min_s=3.0):
    """The same oracle over the whole config-3 batch with its requests split
    over `threads` host threads (oracle.paged_decode_parallel: each request is
    the single-threaded reference loop, so the bits are those of the serial
    oracle).  The batch's pages are gathered to the host once (untimed) and
    renumbered; the whole batch is decoded until at least `min_s` of wall
    time.  Reported beside the single-thread figure with its thread count."""
    import numpy as np
    import torch
    import oracle as O
    threads = min(threads, os.cpu_count() or 1)
    n = int(case.indptr_h[-1])
    idx = torch.from_numpy(case.indices_h.astype(np.int64)).cuda()
    kh = case.k.view(case.pool, -1)[idx].reshape(-1).view(torch.int16).cpu().numpy().view(np.uint16)
    vh = case.v.view(case.pool, -1)[idx].reshape(-1).view(torch.int16).cpu().numpy().view(np.uint16)
    qh = case.q.view(torch.int16).cpu().numpy().view(np.uint16)
    s = O.paged_spec(case.B, n, case.hq, case.hkv)
    ix = np.arange(n, dtype=np.int32)
    t_total, calls = 0.0, 0
    while t_total < min_s:
        t0 = time.perf_counter()
        O.paged_decode_parallel(s, qh, kh, vh, case.indptr_h, ix, case.last_h, threads=threads)
        t_total += time.perf_counter() - t0
        calls += 1
    return {"value": round(case.bytes * calls / t_total / 1e9, 4), "unit": "GB/s",
            "cores": threads, "kind": "port",
            "sample": f"{calls} whole config-3 batches ({case.bytes * calls / 1e9:.2f} GB "
                      f"algorithmic), C oracle in the reference loop order with the requests "
                      f"split over {threads} host threads, {t_total:.1f} s wall time"}


CAPI_BENCH = os.path.join(ROOT, "loom-kernels_amd", "lib", "capi_bench")


def capi_eager(B, pool, hq, hkv, indptr, indices, last, samples=30):
    """The same eager protocol through the C ABI alone (capi_bench, a child
    process: C++ calls of loom_paged_decode_enqueue_bf16, no Python on the
    per-call path): {"capi_eager_us", "capi_host_enqueue_us"}, or {} when the
    program is missing."""
    import subprocess
    if not os.path.exists(CAPI_BENCH):
        return {}
    lst = lambda xs: ",".join(str(int(x)) for x in xs)
    r = subprocess.run([CAPI_BENCH, str(B), str(pool), str(hq), str(hkv), lst(indptr),
                        lst(indices), lst(last), str(samples)],
                       capture_output=True, text=True, timeout=120)
    if r.returncode != 0:
        raise RuntimeError(f"capi_bench failed: {r.stderr.strip()}")
    d = json.loads(r.stdout.strip().splitlines()[-1])
    return {"capi_eager_us": d["eager_us"], "capi_host_enqueue_us": d["host_enqueue_us"]}


def reference_shapes(L, stream, samples=30):
    """The reference's own published shapes (its H20 records):
    tiny decode and append fixtures, whose time is launch latency.  Eager = the
    mean of 100 back-to-back calls between two events, median over `samples`
    batches (benchmarks/matched.rs:141-173); graph = one replay plus its
    completion event, median over `samples` (graph/mod.rs:301-323).  The page
    tables are the reference's gate fixtures; values are synthetic."""
    import numpy as np
    import torch
    g = json.load(open(os.path.join(ROOT, "tests", "golden", "reference_digests.json")))
    dev = "cuda"
    out = {}

    def med(xs):
        xs = sorted(xs)
        return round(xs[len(xs) // 2], 3)

    def eager_and_graph(n_bind, bind, enqueue):
        eg = [_timed_enqueues(L, stream, n_bind, bind, enqueue, 100, 10 if i == 0 else 2)
              for i in range(samples)]
        return med(eg), round(_graph_replay(L, n_bind, 1, bind, enqueue, replays=samples), 3)

    # Platform context: the same two measurements around one tiny torch kernel
    # (eager) and a torch-captured hipGraph of it, on the same stream.
    x = torch.zeros(16, device=dev)
    tg = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        x.add_(1)
        torch.cuda.synchronize()
        with torch.cuda.graph(tg, stream=stream):
            x.add_(1)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for key, fn in (("platform_one_kernel_graph_replay_us", tg.replay),
                    ("platform_one_kernel_eager_single_us", lambda: x.add_(1))):
        ts = []
        for i in range(samples + 3):
            with torch.cuda.stream(stream):
                ev0.record(stream)
                fn()
                ev1.record(stream)
            ev1.synchronize()
            if i >= 3:
                ts.append(ev0.elapsed_time(ev1) * 1000.0)
        out[key] = med(ts)
    del tg
    # Per-node cost of a replay: torch-captured graphs of 1..16 tiny kernels,
    # one replay + completion event per sample; the slope over the node count
    # is what each further node of a captured command adds.
    by_nodes = {}
    for nodes in (1, 2, 4, 8, 16):
        gk = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            torch.cuda.synchronize()
            with torch.cuda.graph(gk, stream=stream):
                for _ in range(nodes):
                    x.add_(1)
        torch.cuda.synchronize()
        ts = []
        for i in range(samples + 3):
            with torch.cuda.stream(stream):
                ev0.record(stream)
                gk.replay()
                ev1.record(stream)
            ev1.synchronize()
            if i >= 3:
                ts.append(ev0.elapsed_time(ev1) * 1000.0)
        by_nodes[nodes] = med(ts)
        del gk
    out["platform_graph_replay_us_by_nodes"] = by_nodes
    # Back-to-back floor: 100 tiny torch kernels between one event pair, per
    # kernel (the eager protocol of the shapes below, with no work).
    ts = []
    for i in range(samples + 3):
        with torch.cuda.stream(stream):
            ev0.record(stream)
            for _ in range(100):
                x.add_(1)
            ev1.record(stream)
        ev1.synchronize()
        if i >= 3:
            ts.append(ev0.elapsed_time(ev1) * 1000.0 / 100)
    out["platform_one_kernel_back_to_back_us"] = med(ts)
    if os.path.exists(CAPI_BENCH):
        import subprocess
        r = subprocess.run([CAPI_BENCH, "--empty-kernel", str(samples)], capture_output=True,
                           text=True, timeout=120)
        if r.returncode == 0:
            d = json.loads(r.stdout.strip().splitlines()[-1])
            out["platform_empty_kernel_back_to_back_us"] = d["eager_us"]
            out["platform_empty_kernel_host_launch_us"] = d["host_enqueue_us"]
    out["platform_graph_replay_us_per_extra_node"] = round(
        (by_nodes[16] - by_nodes[1]) / 15.0, 3)

    for c in g["paged_decode"]["cases"]:
        B, pool, hq, hkv = c["batch"], c["pool"], c["hq"], c["hkv"]
        spec = L.Bf16PagedBatchDecodeSpec(B, pool, hq, hkv, 128, 16)
        plan = L.DecodeProvider.load(0).plan_bf16_paged_batch(
            spec, max_total_pages=len(c["indices"]))
        t = [torch.randn(n, device=dev).to(torch.bfloat16) for n in
             (B * hq * 128, pool * 16 * hkv * 128, pool * 16 * hkv * 128)]
        ip, ix, ln = (torch.tensor(c[k], dtype=torch.int32, device=dev)
                      for k in ("indptr", "indices", "last"))
        o = torch.empty(B * hq * 128, dtype=torch.bfloat16, device=dev)
        lse = torch.empty(B * hq, dtype=torch.float32, device=dev)
        ws = torch.zeros(plan.workspace_bytes, dtype=torch.uint8, device=dev)

        def bind(b):
            return L.Bf16PagedBatchDecodeArgs(
                b.bind_read(t[0]), b.bind_read(t[1]), b.bind_read(t[2]), b.bind_read(ip),
                b.bind_read(ix), b.bind_read(ln), b.bind_read_write(o).write(),
                b.bind_read_write(lse).write(), b.bind_read_write(ws).write())
        e, gr = eager_and_graph(9, bind, plan.enqueue_into)
        out["decode_" + c["name"]] = {"eager_us": e, "graph_replay_us": gr,
                                      "teams": plan.info.teams}
        cap = capi_eager(B, pool, hq, hkv, c["indptr"], c["indices"], c["last"])
        if cap:
            out["decode_" + c["name"]].update(cap)
    for name in ("append_one_token", "append_tokens_t6"):
        c = g[name]
        explicit = "tokens" in c
        B, pool, hq, hkv = c["batch"], c["pool"], c["hq"], c["hkv"]
        T = c["tokens"] if explicit else B
        prov = L.RopeProvider.load(0)
        if explicit:
            plan = prov.plan_bf16_paged_append_tokens(
                L.Bf16RopePagedKvAppendTokensSpec(T, B, pool, hq, hkv))
        else:
            plan = prov.plan_bf16_paged_append(L.Bf16RopePagedKvAppendSpec(B, pool, hq, hkv))
        q, k, v = (torch.randn(T * h * 128, device=dev).to(torch.bfloat16) for h in (hq, hkv, hkv))
        kp = torch.zeros(pool * 16 * hkv * 128, dtype=torch.bfloat16, device=dev)
        vp = torch.zeros_like(kp)
        qo = torch.empty_like(q)
        ip, ix, ln = (torch.tensor(c[k], dtype=torch.int32, device=dev)
                      for k in ("indptr", "indices", "last"))
        bi = torch.tensor(c.get("batch_indices", [0]), dtype=torch.int32, device=dev)
        ps = torch.tensor(c.get("positions", [0]), dtype=torch.int32, device=dev)
        ws = torch.zeros(plan.workspace_bytes, dtype=torch.uint8, device=dev)

        def bind(b):
            return L.Bf16RopePagedKvAppendArgs(
                b.bind_read(q), b.bind_read(k), b.bind_read(v), b.bind_read(ip),
                b.bind_read(ix), b.bind_read(ln), b.bind_read_write(qo).write(),
                b.bind_read_write(kp).write(), b.bind_read_write(vp).write(),
                b.bind_read_write(ws).write(), b.bind_read(bi) if explicit else None,
                b.bind_read(ps) if explicit else None)
        e, gr = eager_and_graph(12 if explicit else 10, bind, plan.enqueue_into)
        out[name] = {"eager_us": e, "graph_replay_us": gr, "tokens": T}
    return out


# The reference's contiguous single-decode eager records (H20, median of 100
# samples; docs/results/h20-flashinfer-v0.6.16.post1-parallel-merge-eager-
# performance-20260805.json `results`): (case, kv_len, Hq, Hkv, its algorithm
# and partitions, its median µs).
SINGLE_DECODE_REFERENCE = (
    ("bf16_mha_l1_qh8_kvh8", 1, 8, 8, 0, 2.599),
    ("bf16_mqa_l33_qh8_kvh1", 33, 8, 1, 12, 6.432),
    ("bf16_gqa_l127_qh16_kvh4", 127, 16, 4, 16, 8.342),
    ("bf16_gqa_l4096_qh32_kvh4", 4096, 32, 4, 64, 35.877),
)


def single_decode_shapes(L, stream, samples=30):
    """Contiguous single decode (single_decode/mod.rs, decode.rs:1016-1450) at
    the shapes of the reference's single-decode eager records: the direct
    plan, and split-K with the reference's partition count where it used
    split-K (two kernels, as there).  Eager = the mean of 100 back-to-back
    calls between two events, median over `samples` batches; synthetic
    values."""
    import torch
    dev = "cuda"
    out = {}
    prov = L.DecodeProvider.load(0)
    for case, kv_len, hq, hkv, parts, ref_us in SINGLE_DECODE_REFERENCE:
        spec = L.Bf16SingleDecodeSpec(kv_len, hq, hkv)
        g = torch.Generator(device=dev).manual_seed(kv_len * 31 + hq)
        q, k, v = (torch.randn(n, device=dev, generator=g).to(torch.bfloat16)
                   for n in (spec.query_numel, spec.kv_numel, spec.kv_numel))
        o = torch.empty(spec.output_numel, dtype=torch.bfloat16, device=dev)
        lse = torch.empty(spec.lse_numel, dtype=torch.float32, device=dev)
        rec = {"h20_loom_eager_us": ref_us}
        plan = prov.plan_bf16(spec)

        def bind(b):
            return L.Bf16SingleDecodeArgs(b.bind_read(q), b.bind_read(k), b.bind_read(v),
                                          b.bind_read_write(o).write(),
                                          b.bind_read_write(lse).write())
        us = sorted(_timed_enqueues(L, stream, 5, bind, plan.enqueue_into, 100, 10 if i == 0 else 2)
                    for i in range(samples))[samples // 2]
        rec["direct_eager_us"] = round(us, 3)
        if parts:
            sk = L.Bf16SingleDecodeSplitKSpec(spec, parts)
            kplan = prov.plan_bf16_split_k(sk)
            ws = torch.empty(sk.workspace_numel, dtype=torch.float32, device=dev)

            def bind_k(b):
                return L.Bf16SingleDecodeSplitKArgs(
                    b.bind_read(q), b.bind_read(k), b.bind_read(v), b.bind_read_write(ws),
                    b.bind_read_write(o).write(), b.bind_read_write(lse).write())
            us = sorted(_timed_enqueues(L, stream, 6, bind_k, kplan.enqueue_into, 100,
                                        10 if i == 0 else 2, commands_per_call=2)
                        for i in range(samples))[samples // 2]
            rec["split_k_partitions"] = parts
            rec["split_k_eager_us"] = round(us, 3)
        out[case] = rec
    return out


def replay_floor(L, stream, n=200):
    """Where a graph replay's time goes (run under rocprofv3 --runtime-trace
    --kernel-trace for the per-call breakdown): the reference's T=6
    explicit-token append (its gate fixture's page table) as a captured graph,
    replayed `n` times with one completion event each (graph/mod.rs:301-323),
    the same command eagerly (enqueue, finish, wait) `n` times, and a
    torch-captured graph of one tiny kernel `n` times.  Reports the HIP-event
    µs and the host wall-clock µs of each form (median)."""
    import torch
    g = json.load(open(os.path.join(ROOT, "tests", "golden", "reference_digests.json")))
    c = g["append_tokens_t6"]
    dev = "cuda"
    B, pool, hq, hkv, T = c["batch"], c["pool"], c["hq"], c["hkv"], c["tokens"]
    plan = L.RopeProvider.load(0).plan_bf16_paged_append_tokens(
        L.Bf16RopePagedKvAppendTokensSpec(T, B, pool, hq, hkv))
    q, k, v = (torch.randn(T * h * 128, device=dev).to(torch.bfloat16) for h in (hq, hkv, hkv))
    kp = torch.zeros(pool * 16 * hkv * 128, dtype=torch.bfloat16, device=dev)
    vp = torch.zeros_like(kp)
    qo = torch.empty_like(q)
    ip, ix, ln = (torch.tensor(c[x], dtype=torch.int32, device=dev)
                  for x in ("indptr", "indices", "last"))
    bi = torch.tensor(c.get("batch_indices", [0] * T), dtype=torch.int32, device=dev)
    ps = torch.tensor(c.get("positions", list(range(T))), dtype=torch.int32, device=dev)
    ws = torch.zeros(plan.workspace_bytes, dtype=torch.uint8, device=dev)

    def bind(b):
        return L.Bf16RopePagedKvAppendTokensArgs(
            b.bind_read(q), b.bind_read(k), b.bind_read(v), b.bind_read(bi), b.bind_read(ps),
            b.bind_read(ip), b.bind_read(ix), b.bind_read(ln), b.bind_read_write(qo).write(),
            b.bind_read_write(kp).write(), b.bind_read_write(vp).write(),
            b.bind_read_write(ws).write())

    def med(xs):
        xs = sorted(xs)
        return round(xs[len(xs) // 2], 3)

    out = {}
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    gq = L.GraphQueue(0, 1)
    b = gq.bindings(12)
    args = bind(b)
    exec_ = gq.capture(b, lambda scope: plan.enqueue_into(scope, args)).instantiate()
    out["append_t6_graph_default_replay_mode"] = exec_.replay_mode
    for mode, key in (("kernel_nodes", "append_t6_graph_replay"),
                      ("hip_graph_launch", "append_t6_graph_replay_hip_graph_launch")):
        exec_.set_replay_mode(mode)
        gpu, host = [], []
        for i in range(n + 5):
            t0 = time.perf_counter()
            ms = exec_.measure_launch_ms(ev0, ev1)
            t1 = time.perf_counter()
            if i >= 5:
                gpu.append(ms * 1000.0)
                host.append((t1 - t0) * 1e6)
        out[key + "_event_us"] = med(gpu)
        out[key + "_host_us"] = med(host)
    exec_.into_bindings()
    q_ = L.CommandQueue(stream, 1)
    b = q_.bindings(12)
    args = bind(b)
    gpu, host = [], []
    with torch.cuda.stream(stream):
        for i in range(n + 5):
            t0 = time.perf_counter()
            ev0.record(stream)
            scope = q_.begin(b)
            plan.enqueue_into(scope, args)
            ev1.record(stream)
            b = scope.finish().wait()
            ev1.synchronize()
            t1 = time.perf_counter()
            if i >= 5:
                gpu.append(ev0.elapsed_time(ev1) * 1000.0)
                host.append((t1 - t0) * 1e6)
    out["append_t6_eager_single_event_us"] = med(gpu)
    out["append_t6_eager_single_host_us"] = med(host)
    x = torch.zeros(16, device=dev)
    tg = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        x.add_(1)
        torch.cuda.synchronize()
        with torch.cuda.graph(tg, stream=stream):
            x.add_(1)
    torch.cuda.synchronize()
    gpu, host = [], []
    for i in range(n + 5):
        t0 = time.perf_counter()
        with torch.cuda.stream(stream):
            ev0.record(stream)
            tg.replay()
            ev1.record(stream)
        ev1.synchronize()
        t1 = time.perf_counter()
        if i >= 5:
            gpu.append(ev0.elapsed_time(ev1) * 1000.0)
            host.append((t1 - t0) * 1e6)
    out["torch_one_kernel_graph_replay_event_us"] = med(gpu)
    out["torch_one_kernel_graph_replay_host_us"] = med(host)
    if os.path.exists(CAPI_BENCH):
        # the same forms from C++ with an empty kernel (no Python on the path)
        import subprocess
        r = subprocess.run([CAPI_BENCH, "--graph-floor", str(n)], capture_output=True, text=True,
                           timeout=120)
        if r.returncode == 0:
            out["capi_empty_kernel"] = json.loads(r.stdout.strip().splitlines()[-1])
    return out


def prefill_shapes(L, stream, samples=30):
    """Paged causal prefill at the five shapes the reference times on H20
    (benchmarks/matched.rs:1355-1425; its eager and long-eager records): eager
    and graph-replay µs as in reference_shapes, with the reference's H20 medians
    (loom-infer and FlashInfer) beside them.  Values are synthetic; the page
    tables are the reference's.  For each shape the algorithmic work is stated:
    K/V bytes of the distinct pages read once per kv-head and the causal
    QK+PV FLOPs."""
    import torch
    g = json.load(open(os.path.join(ROOT, "tests", "golden", "reference_digests.json")))
    dev = "cuda"
    out = {}
    for c in g["paged_prefill"]["cases"] + g["paged_prefill_long"]["cases"]:
        B, nnz, pool, hq, hkv = c["batch"], c["nnz_qo"], c["pool"], c["hq"], c["hkv"]
        spec = L.Bf16PagedPrefillSpec(B, nnz, pool, hq, hkv)
        plan = L.PrefillProvider.load(0).plan_bf16_paged(spec)
        t = [torch.randn(n, device=dev).to(torch.bfloat16) for n in
             (nnz * hq * 128, pool * 16 * hkv * 128, pool * 16 * hkv * 128)]
        qo, ip, ix, ln = (torch.tensor(c[k], dtype=torch.int32, device=dev)
                          for k in ("qo_indptr", "indptr", "indices", "last"))
        o = torch.empty(nnz * hq * 128, dtype=torch.bfloat16, device=dev)
        lse = torch.empty(nnz * hq, dtype=torch.float32, device=dev)

        def bind(b):
            return L.Bf16PagedPrefillArgs(
                b.bind_read(t[0]), b.bind_read(t[1]), b.bind_read(t[2]), b.bind_read(qo),
                b.bind_read(ip), b.bind_read(ix), b.bind_read(ln), b.bind_read_write(o).write(),
                b.bind_read_write(lse).write())
        eg = sorted(_timed_enqueues(L, stream, 9, bind, plan.enqueue_into, 100,
                                    10 if i == 0 else 2) for i in range(samples))
        gr = _graph_replay(L, 9, 1, bind, plan.enqueue_into, replays=samples)
        flops, kv_tokens = 0, 0
        for r in range(B):
            kv = (c["indptr"][r + 1] - c["indptr"][r] - 1) * 16 + c["last"][r]
            n = c["qo_indptr"][r + 1] - c["qo_indptr"][r]
            kv_tokens += kv
            flops += sum(kv - n + i + 1 for i in range(n)) * hq * 128 * 4
        e = eg[len(eg) // 2]
        out[c["name"]] = {
            "eager_us": round(e, 3), "graph_replay_us": round(gr, 3),
            "waves": plan.info.waves, "grid_blocks": plan.info.grid_blocks,
            "causal_gflop": round(flops / 1e9, 4), "TFLOPs": round(flops / (e * 1e-6) / 1e12, 3),
            "kv_bytes": kv_tokens * hkv * 512,
            "h20_loom_eager_us": c.get("loom_h20_eager_median_us", c.get("loom_h20_median_us")),
            "h20_flashinfer_eager_us": c.get("flashinfer_h20_eager_median_us",
                                             c.get("flashinfer_h20_median_us"))}
    return out


def ragged_shapes(L, stream, samples=30):
    """Ragged (contiguous K/V) causal prefill at the three shapes the reference
    times on H20 (benchmarks/matched.rs:1436-1465; its cp-async eager record),
    measured as prefill_shapes."""
    import torch
    g = json.load(open(os.path.join(ROOT, "tests", "golden", "reference_digests.json")))
    dev = "cuda"
    out = {}
    for c in g["ragged_prefill"]["timing_cases"]:
        B, nnz, nkv, hq, hkv = c["batch"], c["nnz_qo"], c["nnz_kv"], c["hq"], c["hkv"]
        spec = L.Bf16RaggedPrefillSpec(B, nnz, nkv, hq, hkv)
        plan = L.PrefillProvider.load(0).plan_bf16_ragged(spec)
        t = [torch.randn(n, device=dev).to(torch.bfloat16) for n in
             (nnz * hq * 128, nkv * hkv * 128, nkv * hkv * 128)]
        qo, kv = (torch.tensor(c[k], dtype=torch.int32, device=dev)
                  for k in ("qo_indptr", "kv_indptr"))
        o = torch.empty(nnz * hq * 128, dtype=torch.bfloat16, device=dev)
        lse = torch.empty(nnz * hq, dtype=torch.float32, device=dev)

        def bind(b):
            return L.Bf16RaggedPrefillArgs(
                b.bind_read(t[0]), b.bind_read(t[1]), b.bind_read(t[2]), b.bind_read(qo),
                b.bind_read(kv), b.bind_read_write(o).write(), b.bind_read_write(lse).write())
        eg = sorted(_timed_enqueues(L, stream, 7, bind, plan.enqueue_into, 100,
                                    10 if i == 0 else 2) for i in range(samples))
        gr = _graph_replay(L, 7, 1, bind, plan.enqueue_into, replays=samples)
        flops = 0
        for r in range(B):
            kvl = c["kv_indptr"][r + 1] - c["kv_indptr"][r]
            n = c["qo_indptr"][r + 1] - c["qo_indptr"][r]
            flops += sum(kvl - n + i + 1 for i in range(n)) * hq * 128 * 4
        e = eg[len(eg) // 2]
        out[c["name"]] = {
            "eager_us": round(e, 3), "graph_replay_us": round(gr, 3),
            "waves": plan.info.waves, "grid_blocks": plan.info.grid_blocks,
            "causal_gflop": round(flops / 1e9, 4), "TFLOPs": round(flops / (e * 1e-6) / 1e12, 3),
            "h20_loom_eager_us": c["loom_h20_eager_median_us"],
            "h20_flashinfer_eager_us": c["flashinfer_h20_eager_median_us"]}
    return out


def long_prefill_shapes(L, stream, samples=5, shapes=None):
    """Paged causal prefill on long prompts (no reference counterpart: its
    timed shapes stop at 64 query rows): GQA4 Hq 32 / Hkv 8, qo_len = kv_len per
    request, a seeded permutation page table; eager µs (median of `samples`
    batches of 5 enqueues) and causal TFLOP/s."""
    import torch
    dev = "cuda"
    out = {}
    for B, n in shapes or ((1, 512), (1, 1024), (1, 4096), (1, 8192), (4, 2048), (8, 256)):
        hq, hkv = 32, 8
        nnz, pages = B * n, (n + 15) // 16
        pool = B * pages
        spec = L.Bf16PagedPrefillSpec(B, nnz, pool, hq, hkv)
        plan = L.PrefillProvider.load(0).plan_bf16_paged(spec)
        g = torch.Generator(device=dev).manual_seed(B * 100000 + n)
        t = [torch.randn(x, device=dev, generator=g).to(torch.bfloat16)
             for x in (nnz * hq * 128, pool * 16 * hkv * 128, pool * 16 * hkv * 128)]
        qo = torch.arange(0, nnz + 1, n, dtype=torch.int32, device=dev)
        ip = torch.arange(0, pool + 1, pages, dtype=torch.int32, device=dev)
        ix = torch.randperm(pool, device=dev, generator=g).to(torch.int32)
        ln = torch.full((B,), n - (pages - 1) * 16, dtype=torch.int32, device=dev)
        o = torch.empty(nnz * hq * 128, dtype=torch.bfloat16, device=dev)
        lse = torch.empty(nnz * hq, dtype=torch.float32, device=dev)

        def bind(b):
            return L.Bf16PagedPrefillArgs(
                b.bind_read(t[0]), b.bind_read(t[1]), b.bind_read(t[2]), b.bind_read(qo),
                b.bind_read(ip), b.bind_read(ix), b.bind_read(ln), b.bind_read_write(o).write(),
                b.bind_read_write(lse).write())
        us = sorted(_timed_enqueues(L, stream, 9, bind, plan.enqueue_into, 5, 2)
                    for _ in range(samples))[samples // 2]
        flops = B * (n * (n + 1) // 2) * hq * 128 * 4
        rec = {"eager_us": round(us, 2), "causal_gflop": round(flops / 1e9, 2),
               "TFLOPs": round(flops / (us * 1e-6) / 1e12, 1), "algorithm": plan.algorithm,
               "grid_blocks": plan.info.grid_blocks}
        if plan.algorithm == "long_tile":
            # the wide tiles on the same command, for comparison
            wplan = L.PrefillProvider.load(0).plan_bf16_paged(spec, tile_cols=64)
            wus = sorted(_timed_enqueues(L, stream, 9, bind, wplan.enqueue_into, 5, 2)
                         for _ in range(samples))[samples // 2]
            rec.update(wide_eager_us=round(wus, 2),
                       wide_TFLOPs=round(flops / (wus * 1e-6) / 1e12, 1))
            # the same prompt on FP8 E4M3 pages (codes of |x| <= 3, scales 0.3 / 0.7)
            fspec = L.Bf16PagedPrefillSpec(B, nnz, pool, hq, hkv, kv_dtype="fp8_e4m3")
            fplan = L.PrefillProvider.load(0).plan_bf16_paged(fspec)
            k8, v8 = (torch.randint(0, 0x44, (pool * 16 * hkv * 128,), device=dev,
                                    dtype=torch.uint8, generator=g) for _ in range(2))
            sc = torch.tensor([0.3, 0.7], dtype=torch.float32, device=dev)

            def bind8(b):
                return L.Bf16PagedPrefillArgs(
                    b.bind_read(t[0]), b.bind_read(k8), b.bind_read(v8), b.bind_read(qo),
                    b.bind_read(ip), b.bind_read(ix), b.bind_read(ln),
                    b.bind_read_write(o).write(), b.bind_read_write(lse).write(),
                    b.bind_read(sc))
            fus = sorted(_timed_enqueues(L, stream, 10, bind8, fplan.enqueue_into, 5, 2)
                         for _ in range(samples))[samples // 2]
            rec.update(fp8_algorithm=fplan.algorithm, fp8_eager_us=round(fus, 2),
                       fp8_TFLOPs=round(flops / (fus * 1e-6) / 1e12, 1))
        out[f"gqa4_b{B}_q{n}_kv{n}"] = rec
    return out


def cpu_append_baseline(app, min_s=3.0):
    """The oracle's explicit-token append (rope/mod.rs + paged_append/mod.rs:
    429-489, single thread) on the config-2 command, repeated for at least
    `min_s`.  Pages no token writes are renumbered onto one shared page so the
    host pools hold only the touched pages (the work per token is unchanged)."""
    import numpy as np
    import torch
    import oracle as O
    indptr, indices, last = (np.asarray(x) for x in app.tables)
    bi = app.bi.cpu().numpy()
    pos = app.pos.cpu().numpy()
    touched = sorted({int(indices[indptr[r] + p // 16]) for r, p in zip(bi, pos)})
    remap = {pg: i + 1 for i, pg in enumerate(touched)}
    idx2 = np.array([remap.get(int(x), 0) for x in indices], np.int32)
    pool = len(touched) + 1
    s = O.paged_spec(app.B, pool, app.hq, app.hkv)
    q, k, v = (t.view(torch.int16).cpu().numpy().view(np.uint16) for t in (app.q, app.k, app.v))
    kp = np.zeros(pool * 16 * app.hkv * 128, np.uint16)
    vp = np.zeros_like(kp)
    calls, t_total = 0, 0.0
    while t_total < min_s:
        t0 = time.perf_counter()
        O.append_tokens(s, app.T, q, k, v, bi, pos, indptr, idx2, last, kp, vp, max_tokens=8192)
        t_total += time.perf_counter() - t0
        calls += 1
    return {"value": round(t_total / calls * 1e6, 1), "unit": "us/call", "cores": 1,
            "kind": "port", "sample": f"{calls} whole config-2 commands ({app.T} tokens), "
                                      f"{t_total:.1f} s, single thread"}


def kv_arenas(cases, seeds=True):
    """One K/V allocation per decode config, made before any measurement and
    kept to the end, as a serving engine reserves its cache once; every case
    of the config (the measured one and the seed statistics') views it.  The
    per-call time of the long-context config depends on where its 1.08 GB
    pool lands: on one box the same command took 163.5-164.2 µs on some
    allocations and 172-173 µs on others, stable on each, and up to 188 µs
    when the pool was allocated after the other configs' allocate/free churn.
    Two arenas per config: the measured case's (kept, e.g. for the CPU
    baseline) and one the seed statistics' cases take in turn."""
    import torch
    return {n: tuple(torch.empty(2 * pool * 16 * hkv * 128, dtype=torch.bfloat16, device="cuda")
                     for _ in range(2 if seeds else 1))
            for n, (B, hq, hkv, pool, lens) in cases.items()}


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
    ap.add_argument("--no-variants", action="store_true",
                    help="skip the HND, FP8 and 64-row page timings of config 3 (profiling runs)")
    ap.add_argument("--no-stats", action="store_true",
                    help="skip the seeds 0..4 sample statistics of the decode configs")
    ap.add_argument("--only", default=None,
                    help="run one config (prefix match, e.g. c3) and print its detail")
    ap.add_argument("--records", default=os.path.join("gpurun_out", "bench_records.jsonl"),
                    help="JSON Lines evidence records (raw samples, fixture digests, source "
                         "commit) per config; '' to skip")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run 20 plain device copies of MIB MiB (counter calibration)")
    a = ap.parse_args()
    if a.gpus != 1:
        print("bench.py measures one GPU: every GPU box here has one MI355X and the path "
              "has no cross-GPU component; run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    if a.copy_calibration:
        n = a.copy_calibration << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(20):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_per_launch": n, "launches": 20}), flush=True)
        return
    import loom_infer_hip as L
    torch.cuda.set_device(0)
    stream = torch.cuda.Stream()  # default priority
    detail = {}
    head = None
    cases = {n: c for n, c in make_cases(L, a.quick).items()
             if not a.only or n.startswith(a.only)}
    arenas = kv_arenas(cases, seeds=not a.no_stats)
    for name, (B, hq, hkv, pool, lens) in cases.items():
        log(f"[bench] setting up {name}")
        case = DecodeCase(L, name, B, hq, hkv, pool, lens, seed=len(name), arena=arenas[name][0])
        us = time_eager(L, case, stream, a.steps, a.warmup)
        g_samples = []
        g_us = time_graph(L, case, samples_out=g_samples)
        if a.records:
            fid, dig, shape = decode_fixture(case)
            xs = _sampled_enqueues(L, stream, 9, case.bind, case.plan.enqueue_into, 20, 10,
                                   a.warmup)
            kpc = decode_kernels_per_call(case.plan)
            record("paged_batch_decode", name, kpc, shape, fid, dig, a.warmup, 10, xs,
                   "eager_stream_batch_hip_event")
            record("paged_batch_decode", name, kpc, shape, fid, dig, 3, 1, g_samples,
                   "graph_replay_with_completion_event")
        gbs = case.bytes / (us * 1e-6) / 1e9
        detail[name] = {"us_per_call": round(us, 3), "graph_replay_us": round(g_us, 3),
                        "GBps": round(gbs, 1), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                        "algorithmic_bytes": case.bytes,
                        "teams": case.plan.info.teams,
                        "mean_kv_len": float(case.lens.mean())}
        if name.startswith("c3") and not a.no_variants:
            # the same command on HND pages (same bytes, head-major pages: one
            # kv-head's 16 rows are 4 KiB contiguous); the pool contents are
            # reinterpreted, which does not change the work
            hspec = L.Bf16PagedBatchDecodeSpec(B, pool, hq, hkv, 128, 16, kv_layout="HND")
            hplan = L.DecodeProvider.load(0).plan_bf16_paged_batch(
                hspec, max_total_pages=int(case.indptr_h[-1]))
            h_us = _timed_enqueues(L, stream, 9, case.bind, hplan.enqueue_into, a.steps, a.warmup)
            detail[name].update({"hnd_us_per_call": round(h_us, 3),
                                 "hnd_GBps": round(case.bytes / (h_us * 1e-6) / 1e9, 1)})
            del hplan
            # and on FP8 E4M3 pages (half the K/V bytes; finite random codes,
            # per-tensor scales): the K/V bytes per call and their rate
            n8 = pool * 16 * hkv * 128
            k8 = torch.randint(0, 0x60, (n8,), dtype=torch.uint8, device="cuda")
            v8 = torch.randint(0, 0x60, (n8,), dtype=torch.uint8, device="cuda")
            sc = torch.tensor([0.05, 0.05], dtype=torch.float32, device="cuda")
            fspec = L.Bf16PagedBatchDecodeSpec(B, pool, hq, hkv, 128, 16, kv_dtype="fp8_e4m3")
            fplan = L.DecodeProvider.load(0).plan_bf16_paged_batch(
                fspec, max_total_pages=int(case.indptr_h[-1]))
            ws8 = torch.zeros(fplan.workspace_bytes, dtype=torch.uint8, device="cuda")

            def bind8(b):
                h = [b.bind_read(case.q), b.bind_read(k8), b.bind_read(v8),
                     b.bind_read(case.indptr), b.bind_read(case.indices), b.bind_read(case.last),
                     b.bind_read_write(case.out), b.bind_read_write(case.lse),
                     b.bind_read_write(ws8), b.bind_read(sc)]
                return L.Bf16PagedBatchDecodeArgs(h[0], h[1], h[2], h[3], h[4], h[5],
                                                  h[6].write(), h[7].write(), h[8].write(), h[9])
            f_us = _timed_enqueues(L, stream, 10, bind8, fplan.enqueue_into, a.steps, a.warmup)
            kv8 = int(2 * 128 * hkv * case.lens.sum())
            f_bytes = case.bytes - kv8  # the K/V half of the BF16 bytes
            detail[name].update({"fp8_us_per_call": round(f_us, 3),
                                 "fp8_algorithmic_bytes": f_bytes,
                                 "fp8_GBps": round(f_bytes / (f_us * 1e-6) / 1e9, 1)})
            del fplan, k8, v8, ws8
            # and on 64-row pages (the same pool bytes as pool / 4 pages; the
            # same request lengths, so the same algorithmic bytes)
            import numpy as np
            P = 64
            pages64 = (case.lens + P - 1) // P
            ip64 = np.concatenate([[0], np.cumsum(pages64)]).astype(np.int32)
            ix64 = np.random.default_rng(64).permutation(pool // (P // 16))[: int(ip64[-1])]
            last64 = (case.lens - (pages64 - 1) * P).astype(np.int32)
            d_ip = torch.from_numpy(ip64).to("cuda")
            d_ix = torch.from_numpy(ix64.astype(np.int32)).to("cuda")
            d_last = torch.from_numpy(last64).to("cuda")
            pspec = L.Bf16PagedBatchDecodeSpec(B, pool // (P // 16), hq, hkv, kv_page_size=P)
            pplan = L.DecodeProvider.load(0).plan_bf16_paged_batch(
                pspec, max_total_pages=int(ip64[-1]))

            def bind64(b):
                h = [b.bind_read(case.q), b.bind_read(case.k), b.bind_read(case.v),
                     b.bind_read(d_ip), b.bind_read(d_ix), b.bind_read(d_last),
                     b.bind_read_write(case.out), b.bind_read_write(case.lse),
                     b.bind_read_write(case.ws)]
                return L.Bf16PagedBatchDecodeArgs(h[0], h[1], h[2], h[3], h[4], h[5],
                                                  h[6].write(), h[7].write(), h[8].write())
            assert pplan.workspace_bytes <= case.plan.workspace_bytes
            p_us = _timed_enqueues(L, stream, 9, bind64, pplan.enqueue_into, a.steps, a.warmup)
            detail[name].update({"page64_us_per_call": round(p_us, 3),
                                 "page64_GBps": round(case.bytes / (p_us * 1e-6) / 1e9, 1)})
            del pplan
        if name.startswith("c1"):
            detail[name].update(capi_eager(B, pool, hq, hkv, case.indptr_h, case.indices_h,
                                           case.last_h))
            # cold: 16 copies of the workload (537 MB) used round-robin
            copies = [case] + [DecodeCase(L, name, B, hq, hkv, pool, lens, seed=len(name) + i)
                               for i in range(1, 16)]
            cold = _timed_rotating(L, stream, 9, [c.bind for c in copies],
                                   case.plan.enqueue_into, a.steps, a.warmup)
            detail[name].update({"cold_us_per_call": round(cold, 3),
                                 "cold_GBps": round(case.bytes / (cold * 1e-6) / 1e9, 1)})
            del copies
        if name.startswith("c5"):
            # the one-token append of the same step, then the whole step as one graph
            app = AppendCase(L, B, hq, hkv, pool, lens, seed=5, share=case)
            ap_gs = []
            ap_us, ap_g = time_append(L, app, stream, a.steps, a.warmup, ap_gs)
            if a.records:
                record_append(name + "_one_token_append", app, stream, a.warmup, ap_gs)
            st_gs = []
            step_g = time_full_step(L, app, case, st_gs)
            if a.records:
                fid, dig, shape = decode_fixture(case)
                dig.update(new_query=device_digest(app.q), new_key=device_digest(app.k),
                           new_value=device_digest(app.v))
                record("rope_paged_append+paged_batch_decode", name + "_full_step", 1 +
                       decode_kernels_per_call(case.plan), shape, fid + "; new tokens seed 5",
                       dig, 3, 1, st_gs, "graph_replay_with_completion_event")
            detail[name].update({"append_us_per_call": round(ap_us, 3),
                                 "append_graph_replay_us": round(ap_g, 3),
                                 "full_step_graph_replay_us": round(step_g, 3)})
            del app
        if not a.no_stats:
            detail[name]["seed_stats"] = seed_stats(L, stream, name, B, hq, hkv, pool,
                                                    range(5), 10, 10, a.warmup,
                                                    arena=arenas[name][1])
        log(f"[bench] {name}: {detail[name]}")
        if name.startswith("c3"):
            head = case
        else:
            del case
            torch.cuda.empty_cache()
    if not a.quick and (not a.only or "c2_rope_append_b32_tokens".startswith(a.only)):
        log("[bench] setting up c2_rope_append_b32_tokens")
        import numpy as np
        rng = np.random.default_rng(2)
        existing = rng.integers(0, 4096, size=32)
        n_new = rng.integers(1, 65, size=32)
        app = AppendCase(L, 32, 32, 8, 16384, existing + n_new, seed=2, n_new=n_new)
        ap_gs = []
        ap_us, ap_g = time_append(L, app, stream, a.steps, a.warmup, ap_gs)
        if a.records:
            record_append("c2_rope_append_b32_tokens", app, stream, a.warmup, ap_gs)
        # cold: 24 sets of the token inputs and query outputs (each ~20 MB)
        # rotated over the same page pools
        extra = []
        for i in range(1, 24):
            x = object.__new__(AppendCase)
            x.__dict__.update(app.__dict__)
            x.q, x.k, x.v = (torch.randn_like(t) for t in (app.q, app.k, app.v))
            x.qo = torch.empty_like(app.qo)
            x.ws = torch.zeros_like(app.ws)
            extra.append(x)
        shared = {}  # the page pools are bound read-write once per binding set

        def binder(x):
            def bind(b):
                if not shared:
                    shared["kp"] = b.bind_read_write(app.kp)
                    shared["vp"] = b.bind_read_write(app.vp)
                return x.bind(b, kp=shared["kp"], vp=shared["vp"])
            return bind
        cold = _timed_rotating(L, stream, 12, [binder(x) for x in [app] + extra],
                               app.plan.enqueue_into, a.steps, a.warmup)
        del extra
        detail["c2_rope_append_b32_tokens"] = {
            "us_per_call": round(ap_us, 3), "graph_replay_us": round(ap_g, 3),
            "cold_us_per_call": round(cold, 3),
            "tokens": app.T, "algorithmic_bytes": app.bytes,
            "GBps": round(app.bytes / (ap_us * 1e-6) / 1e9, 1)}
        if not a.no_cpu:
            detail["c2_rope_append_b32_tokens"]["cpu_baseline"] = cpu_append_baseline(app)
        log(f"[bench] c2: {detail['c2_rope_append_b32_tokens']}")
        del app
    if a.only == "long_prefill":  # profiling: the 8192-row prompt alone
        detail["long_prefill"] = long_prefill_shapes(L, stream, samples=3, shapes=((1, 8192),))
    if a.only == "replay":
        detail["replay_floor"] = replay_floor(L, stream)
    elif not a.quick and (not a.only or a.only == "ref"):
        detail["replay_floor"] = replay_floor(L, stream)
        # the same in a child process with the HIP runtime's graph packet
        # capture off (read at HIP initialisation: DEBUG_CLR_GRAPH_PACKET_CAPTURE=0)
        import subprocess
        env = dict(os.environ, DEBUG_CLR_GRAPH_PACKET_CAPTURE="0")
        r = subprocess.run([sys.executable, os.path.abspath(__file__), "--only", "replay",
                            "--no-cpu", "--records", ""], capture_output=True, text=True,
                           timeout=300, env=env)
        if r.returncode == 0:
            d = json.loads(r.stdout.strip().splitlines()[-1])["replay_floor"]
            detail["replay_floor"]["packet_capture_off"] = d
    if not a.quick and (not a.only or a.only == "ref"):
        log("[bench] reference published shapes")
        detail["reference_shapes"] = reference_shapes(L, stream)
        log(f"[bench] {detail['reference_shapes']}")
        detail["single_decode"] = single_decode_shapes(L, stream)
        log(f"[bench] {detail['single_decode']}")
    if not a.quick and (not a.only or a.only == "prefill"):
        log("[bench] paged prefill at the reference's shapes")
        detail["paged_prefill"] = prefill_shapes(L, stream)
        log(f"[bench] {detail['paged_prefill']}")
        detail["ragged_prefill"] = ragged_shapes(L, stream)
        log(f"[bench] {detail['ragged_prefill']}")
        detail["long_prefill"] = long_prefill_shapes(L, stream)
        log(f"[bench] {detail['long_prefill']}")
    write_records(a.records)
    if a.only:
        print(json.dumps(detail), flush=True)
        return
    c3 = detail["c3_gqa4_b64_ragged"]
    cpu = None if a.no_cpu else cpu_baseline(head)
    if cpu is not None:
        detail["c3_gqa4_b64_ragged"]["cpu_baseline_parallel"] = cpu_baseline_parallel(head)
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
                     "unit": "GB/s", "frac": c3["frac_hbm_peak"], "traffic": TRAFFIC_C3,
                     "kernel": "decode command (split-KV partial + merge), HIP events on "
                               "its launch stream"},
        "cpu_baseline": cpu,
        "detail": detail,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
