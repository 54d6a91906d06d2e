"""Helpers for GPU parity tests: drive the product through the C ABI with the
reference's call sequence and return host copies of the outputs."""
import math

import numpy as np


def torch_dev():
    import torch
    return torch


def to_dev_bf16(u16: np.ndarray):
    torch = torch_dev()
    return torch.from_numpy(np.ascontiguousarray(u16).view(np.int16)).to("cuda").view(torch.bfloat16)


def to_dev_i32(a):
    torch = torch_dev()
    return torch.from_numpy(np.ascontiguousarray(np.asarray(a, np.int32))).to("cuda")


def bf16_host(t) -> np.ndarray:
    torch = torch_dev()
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def nan_bf16(n):
    torch = torch_dev()
    return torch.full((n,), float("nan"), dtype=torch.bfloat16, device="cuda")


def seeded_normal_bf16(oracle, rng, n):
    return oracle.bf16_from_f32(rng.standard_normal(n, dtype=np.float32))


def ragged_table(rng, lens, pool):
    """Pages drawn by a seeded permutation of the pool (each page used once)."""
    pages = [(L + 15) // 16 for L in lens]
    indptr = np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)
    assert indptr[-1] <= pool
    indices = rng.permutation(pool)[: indptr[-1]].astype(np.int32)
    last = np.array([L - (p - 1) * 16 for L, p in zip(lens, pages)], np.int32)
    return indptr, indices, last


class DecodeRunner:
    """Plans once and runs paged decode via the C ABI on torch's current stream."""

    def __init__(self, L, batch, pool, hq, hkv, **plan_opts):
        torch = torch_dev()
        self.L = L
        self.spec = L.Bf16PagedBatchDecodeSpec(batch, pool, hq, hkv, 128, 16)
        self.provider = L.DecodeProvider.load(0)
        self.plan = self.provider.plan_bf16_paged_batch(self.spec, **plan_opts)
        # deliberately not zeroed: the workspace is scratch between commands
        self.workspace = torch.full((self.plan.workspace_bytes,), 0xFF, dtype=torch.uint8,
                                    device="cuda")
        self.queue = L.CommandQueue(torch.cuda.current_stream(), 4)

    def bindings(self, q, k, v, indptr, indices, last, out, lse):
        b = self.queue.bindings(9)
        h = [b.bind_read(q), b.bind_read(k), b.bind_read(v), b.bind_read(indptr),
             b.bind_read(indices), b.bind_read(last), b.bind_read_write(out),
             b.bind_read_write(lse), b.bind_read_write(self.workspace)]
        return b, h

    def args(self, h):
        return self.L.Bf16PagedBatchDecodeArgs(h[0], h[1], h[2], h[3], h[4], h[5],
                                               h[6].write(), h[7].write(), h[8].write())

    def run_dev(self, q, k, v, indptr, indices, last, out=None, lse=None):
        torch = torch_dev()
        s = self.spec
        if out is None:
            out = nan_bf16(s.output_numel)
        if lse is None:
            lse = torch.full((s.lse_numel,), float("nan"), dtype=torch.float32, device="cuda")
        b, h = self.bindings(q, k, v, indptr, indices, last, out, lse)
        scope = self.queue.begin(b)
        self.plan.enqueue_into(scope, self.args(h))
        comp = scope.finish()
        assert comp.submitted() == 1
        b = comp.wait()
        out = b.take_read_write(h[6])
        lse = b.take_read_write(h[7])
        b.take_read_write(h[8])
        return out, lse

    def run(self, q_u16, k_u16, v_u16, indptr, indices, last):
        out, lse = self.run_dev(to_dev_bf16(q_u16), to_dev_bf16(k_u16), to_dev_bf16(v_u16),
                                to_dev_i32(indptr), to_dev_i32(indices), to_dev_i32(last))
        return bf16_host(out), lse.cpu().numpy()


def compare_decode(oracle, out, lse, ref_out, ref_lse, max_abs=0.015625, mean_abs=2e-3,
                   lse_abs=0.01):
    """The reference gate's limits (gates/paged_batch_decode.rs:18-19) and the
    target tolerance: max-abs 2e-2 / mean-abs 2e-3 against the f32 oracle."""
    a = oracle.bf16_to_f32(out).astype(np.float64)
    e = oracle.bf16_to_f32(ref_out).astype(np.float64)
    assert np.all(np.isfinite(a)), "non-finite output"
    diff = np.abs(a - e)
    ld = np.abs(lse.astype(np.float64) - ref_lse.astype(np.float64))
    assert diff.max() <= max_abs, f"output max abs {diff.max()}"
    assert diff.mean() <= mean_abs, f"output mean abs {diff.mean()}"
    assert ld.max() <= lse_abs, f"lse max abs {ld.max()}"
    return dict(max_abs=float(diff.max()), mean_abs=float(diff.mean()),
                lse_max_abs=float(ld.max()),
                bit_mismatches=int(np.sum(out != ref_out)))


class PrefillRunner:
    """Plans once and runs paged prefill via the C ABI on torch's current stream."""

    def __init__(self, L, batch, nnz_qo, pool, hq, hkv, **plan_opts):
        torch = torch_dev()
        self.L = L
        self.spec = L.Bf16PagedPrefillSpec(batch, nnz_qo, pool, hq, hkv, 128, 16)
        self.provider = L.PrefillProvider.load(0)
        self.plan = self.provider.plan_bf16_paged(self.spec, **plan_opts)
        self.queue = L.CommandQueue(torch.cuda.current_stream(), 4)

    def run_dev(self, q, k, v, qo, indptr, indices, last, out=None, lse=None, scales=None):
        torch = torch_dev()
        s = self.spec
        if out is None:
            out = nan_bf16(s.output_numel)
        if lse is None:
            lse = torch.full((s.lse_numel,), float("nan"), dtype=torch.float32, device="cuda")
        b = self.queue.bindings(10)
        h = [b.bind_read(x) for x in (q, k, v, qo, indptr, indices, last)]
        h += [b.bind_read_write(out), b.bind_read_write(lse)]
        sc = b.bind_read(scales) if scales is not None else None
        scope = self.queue.begin(b)
        self.plan.enqueue_into(scope, self.L.Bf16PagedPrefillArgs(
            h[0], h[1], h[2], h[3], h[4], h[5], h[6], h[7].write(), h[8].write(), sc))
        comp = scope.finish()
        assert comp.submitted() == 1
        b = comp.wait()
        return b.take_read_write(h[7]), b.take_read_write(h[8])

    def run(self, q_u16, k_u16, v_u16, qo, indptr, indices, last):
        out, lse = self.run_dev(to_dev_bf16(q_u16), to_dev_bf16(k_u16), to_dev_bf16(v_u16),
                                to_dev_i32(qo), to_dev_i32(indptr), to_dev_i32(indices),
                                to_dev_i32(last))
        return bf16_host(out), lse.cpu().numpy()


class RaggedRunner:
    """Plans once and runs ragged prefill via the C ABI on torch's current stream."""

    def __init__(self, L, batch, nnz_qo, nnz_kv, hq, hkv, **plan_opts):
        torch = torch_dev()
        self.L = L
        self.spec = L.Bf16RaggedPrefillSpec(batch, nnz_qo, nnz_kv, hq, hkv, 128)
        self.plan = L.PrefillProvider.load(0).plan_bf16_ragged(self.spec, **plan_opts)
        self.queue = L.CommandQueue(torch.cuda.current_stream(), 4)

    def run_dev(self, q, k, v, qo, kv, out=None, lse=None, workspace=None):
        torch = torch_dev()
        s = self.spec
        if out is None:
            out = nan_bf16(s.output_numel)
        if lse is None:
            lse = torch.full((s.lse_numel,), float("nan"), dtype=torch.float32, device="cuda")
        b = self.queue.bindings(8)
        h = [b.bind_read(x) for x in (q, k, v, qo, kv)]
        h += [b.bind_read_write(out), b.bind_read_write(lse)]
        args = self.L.Bf16RaggedPrefillArgs(h[0], h[1], h[2], h[3], h[4], h[5].write(),
                                            h[6].write())
        if workspace is not None:
            args = args.with_workspace(b.bind_read_write(workspace))
        scope = self.queue.begin(b)
        self.plan.enqueue_into(scope, args)
        comp = scope.finish()
        assert comp.submitted() == 1
        b = comp.wait()
        return b.take_read_write(h[5]), b.take_read_write(h[6])

    def run(self, q_u16, k_u16, v_u16, qo, kv):
        out, lse = self.run_dev(to_dev_bf16(q_u16), to_dev_bf16(k_u16), to_dev_bf16(v_u16),
                                to_dev_i32(qo), to_dev_i32(kv))
        return bf16_host(out), lse.cpu().numpy()
