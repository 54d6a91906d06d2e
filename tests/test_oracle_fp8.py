"""Pins the oracle's FP8 E4M3 KV storage (no reference counterpart: the
reference lists FP8 KV as unsupported) before it checks the kernels.

* The codec against torch.float8_e4m3fn (OCP E4M3, an independent
  implementation): all 256 codes decode to the same values; encoding a dense
  sweep of finite values clamped to +-448 gives the same codes (torch does
  not saturate, so the clamp is the saturation this contract adds).
* The FP8 decode loop against the pinned BF16 paged decode on values that are
  exactly representable in both formats (scales that are powers of two keep
  every product exact), so any indexing or scaling slip shows.
* The FP8 append against the pinned BF16 append: V bytes are the encoding of
  the BF16 V rows, and K bytes decode to within half an FP8 step of the BF16
  rotated K (the BF16 rotation rounds the same FP32 value)."""
import numpy as np
import pytest
import torch


def test_all_codes_decode_like_torch(oracle):
    codes = np.arange(256, dtype=np.uint8)
    ours = oracle.fp8_to_f32(codes)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan) and nan.sum() == 2
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))  # -0 too
    assert ours[0x7E] == 448.0 and ours[0x01] == 2.0 ** -9 and ours[0x08] == 2.0 ** -6


def test_encode_matches_clamped_torch(oracle):
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(2.0) ** rng.integers(-12, 10, 200000).astype(np.float32),
        oracle.fp8_to_f32(np.arange(256, dtype=np.uint8)),                 # every exact value
        (oracle.fp8_to_f32(np.arange(1, 126, dtype=np.uint8)) +
         oracle.fp8_to_f32(np.arange(2, 127, dtype=np.uint8))) / 2,        # every tie
        np.array([448.0, 449.0, 464.0, 500.0, 1e30, -1e30, np.inf, -np.inf, 1e-30, -1e-30,
                  2.0 ** -10, 3 * 2.0 ** -10, 0.0, -0.0], np.float32)]).astype(np.float32)
    x = x[np.isfinite(x) | np.isinf(x)]
    ours = oracle.fp8_from_f32(x)
    ref = torch.from_numpy(np.clip(x, -448.0, 448.0)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, ref)
    assert oracle.fp8_from_f32(np.array([np.nan], np.float32))[0] == 0x7F


def test_fp8_decode_equals_bf16_decode_on_exact_values(oracle):
    rng = np.random.default_rng(5)
    B, hq, hkv, pool = 3, 16, 4, 12
    lens = [5, 37, 60]
    pages = [(L + 15) // 16 for L in lens]
    ip = np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)
    ix = rng.permutation(pool)[: ip[-1]].astype(np.int32)
    last = np.array([L - (p - 1) * 16 for L, p in zip(lens, pages)], np.int32)
    n = pool * 16 * hkv * 128
    k8 = rng.integers(0, 0x7E, n).astype(np.uint8) | (rng.integers(0, 2, n).astype(np.uint8) << 7)
    v8 = rng.integers(0, 0x7E, n).astype(np.uint8) | (rng.integers(0, 2, n).astype(np.uint8) << 7)
    k8 = np.where((k8 & 0x7F) > 0x50, k8 & 0xD0, k8)  # keep |K| small: scores stay moderate
    ks, vs = 0.25, 2.0
    kb = oracle.bf16_from_f32(oracle.fp8_to_f32(k8) * np.float32(ks))
    vb = oracle.bf16_from_f32(oracle.fp8_to_f32(v8) * np.float32(vs))
    assert np.array_equal(oracle.bf16_to_f32(kb), oracle.fp8_to_f32(k8) * np.float32(ks))
    q = oracle.bf16_from_f32(rng.standard_normal(B * hq * 128).astype(np.float32))
    spec = oracle.paged_spec(B, pool, hq, hkv)
    o8, l8 = oracle.paged_decode_fp8(spec, q, k8, v8, ip, ix, last, ks, vs)
    ob, lb = oracle.paged_decode(spec, q, kb, vb, ip, ix, last)
    assert np.array_equal(o8, ob) and np.array_equal(l8, lb)


def test_fp8_append_against_the_bf16_append(oracle):
    rng = np.random.default_rng(9)
    B, hq, hkv, pool, T = 3, 8, 2, 8, 5
    ip, ix, last = [0, 2, 3, 6], [4, 1, 7, 0, 2, 5], [5, 16, 9]
    bi, pos = [0, 2, 1, 2, 0], [17, 40, 3, 38, 20]
    spec = oracle.paged_spec(B, pool, hq, hkv)
    q = oracle.bf16_from_f32(rng.standard_normal(T * hq * 128).astype(np.float32))
    k = oracle.bf16_from_f32(rng.standard_normal(T * hkv * 128).astype(np.float32))
    v = oracle.bf16_from_f32(rng.standard_normal(T * hkv * 128).astype(np.float32))
    kp = np.zeros(pool * 16 * hkv * 128, np.uint16)
    vp = np.zeros_like(kp)
    qo = oracle.append_tokens(spec, T, q, k, v, bi, pos, ip, ix, last, kp, vp)
    kp8 = np.zeros(kp.size, np.uint8)
    vp8 = np.zeros(kp.size, np.uint8)
    ks, vs = 0.05, 0.03
    qo8 = oracle.append_tokens_fp8(spec, T, q, k, v, bi, pos, ip, ix, last, kp8, vp8, ks, vs)
    assert np.array_equal(qo8, qo if not isinstance(qo, tuple) else qo[0])
    written = kp != 0
    assert written.sum() == T * hkv * 128
    assert np.array_equal(vp8[written], oracle.fp8_from_f32(oracle.bf16_to_f32(vp[written]) / np.float32(vs)))
    kf = oracle.fp8_to_f32(kp8[written]) * np.float32(ks)
    kr = oracle.bf16_to_f32(kp[written])
    step = np.maximum(np.abs(kr), 2.0 ** -6 * ks) * 2.0 ** -3 * 1.01
    assert np.all(np.abs(kf - kr) <= step)
    assert np.all(kp8[~written] == 0) and np.all(vp8[~written] == 0)
