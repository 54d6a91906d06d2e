"""Element-wise accounting of NeoX RoPE differences between the device and the
CPU oracle (test infrastructure).

The oracle follows the reference's rotate_tensor (crates/loom-infer/src/rope/
mod.rs:136-161): inv_freq = powf(theta, -(2p/D)) / scale, angle = pos * inv_freq
in FP32, (sin, cos) from the host C library's sinf / cosf, then
out = (x1*cos - x2*sin, x2*cos + x1*sin) with every product rounded to FP32 and
the result rounded to BF16.  The device computes the same expression with the
correctly rounded FP32 sin / cos of the same FP32 angle.  glibc's sinf / cosf
are accurate to < 1 FP32 ulp but not correctly rounded for every argument;
where they differ by one FP32 ulp and the rotation cancels, the BF16 outputs
can differ by more than one BF16 ulp.

``rotate_elements`` re-evaluates chosen output elements with either pair of
(sin, cos) values, so a test can show, element by element, that every
difference beyond one BF16 ulp is exactly that rounding of sin / cos and
nothing else."""
import ctypes as C
import math

import numpy as np

_libm = C.CDLL("libm.so.6")
for _f in ("sinf", "cosf"):
    getattr(_libm, _f).restype = C.c_float
    getattr(_libm, _f).argtypes = [C.c_float]
_libm.powf.restype = C.c_float
_libm.powf.argtypes = [C.c_float, C.c_float]


def _f32(x):
    return np.float32(x)


def _bf16_bits(x: np.float32) -> int:
    """Round-to-nearest-even FP32 -> BF16 bits (finite inputs)."""
    u = int(np.array([x], np.float32).view(np.uint32)[0])
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF


def _bf16_to_f32(bits: int) -> np.float32:
    return np.array([bits << 16], np.uint32).view(np.float32)[0]


def inv_freq(p, rotary_dim=128, scale=1.0, theta=10000.0):
    exponent = _f32(_f32(2.0) * _f32(p)) / _f32(rotary_dim)
    return _f32(_f32(_libm.powf(_f32(theta), -exponent)) / _f32(scale))


def angle(pos, p, rotary_dim=128, scale=1.0, theta=10000.0):
    return _f32(_f32(pos) * inv_freq(p, rotary_dim, scale, theta))


def host_sincos(a):
    return _f32(_libm.sinf(a)), _f32(_libm.cosf(a))


def cr_sincos(a):
    """Correctly rounded FP32 sin / cos of the FP32 angle (FP64 then one rounding)."""
    return _f32(math.sin(float(a))), _f32(math.cos(float(a)))


def rotate_element(row_bits, col, pos, sincos, rotary_dim=128):
    """BF16 bits of output element `col` of one head row (128 BF16 bits)."""
    half = rotary_dim // 2
    p = col % half
    sn, cs = sincos(angle(pos, p, rotary_dim))
    first = _bf16_to_f32(int(row_bits[p]))
    second = _bf16_to_f32(int(row_bits[half + p]))
    with np.errstate(all="ignore"):
        if col < half:
            v = _f32(_f32(first * cs) - _f32(second * sn))
        else:
            v = _f32(_f32(second * cs) + _f32(first * sn))
    return _bf16_bits(v)


def explain_beyond_one_ulp(got, want, inputs, positions_per_row):
    """For every element where the device bits `got` and the oracle bits `want`
    differ by more than one BF16 ulp, check that (1) re-evaluating the element
    with the host sinf/cosf reproduces `want`, (2) re-evaluating it with the
    correctly rounded sin/cos reproduces `got`, and (3) the two (sin, cos)
    pairs differ.  Returns (beyond_count, unexplained list)."""
    g = got.reshape(-1, 128).astype(np.int64)
    w = want.reshape(-1, 128).astype(np.int64)
    x = inputs.reshape(-1, 128)
    gf = (g << 16).astype(np.uint32).view(np.float32)
    wf = (w << 16).astype(np.uint32).view(np.float32)
    one_ulp = (g == w) | ((np.sign(gf) == np.sign(wf)) & (np.abs(g - w) <= 1))
    rows, cols = np.nonzero(~one_ulp)
    unexplained = []
    for r, c in zip(rows.tolist(), cols.tolist()):
        pos = int(positions_per_row[r])
        p = c % 64
        a = angle(pos, p)
        host = rotate_element(x[r], c, pos, host_sincos)
        cr = rotate_element(x[r], c, pos, cr_sincos)
        if not (host == w[r, c] and cr == g[r, c] and host_sincos(a) != cr_sincos(a)):
            unexplained.append((r, c, pos, int(g[r, c]), int(w[r, c]), host, cr))
    return len(rows), unexplained
