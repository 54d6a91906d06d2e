"""CPU checks of the RoPE difference accounting used by the GPU append tests
(tests/rope_explain.py): its host re-evaluation must reproduce the oracle bit
for bit, and its correctly rounded variant must be told apart from it exactly
where the sin/cos pairs differ."""
import numpy as np

import rope_explain as R


def test_host_reevaluation_reproduces_oracle(oracle):
    rng = np.random.default_rng(7)
    T, hq = 24, 4
    q = oracle.bf16_from_f32(rng.standard_normal(T * hq * 128, dtype=np.float32))
    pos = rng.integers(0, 32768, size=T).astype(np.int32)
    pos[0] = 0
    qo, _ = oracle.rope_pos_ids(T, hq, 1, q, q[:T * 128], pos)
    rows, want = q.reshape(-1, 128), qo.reshape(-1, 128)
    for r in range(T * hq):
        for c in range(128):
            assert R.rotate_element(rows[r], c, int(pos[r // hq]), R.host_sincos) == want[r, c]


def test_correctly_rounded_differences_are_all_explained(oracle):
    """A host evaluation with correctly rounded sin/cos (what the device
    computes) against the oracle: every element beyond one BF16 ulp is
    explained, and an injected two-ulp error is not."""
    rng = np.random.default_rng(11)
    T, hq = 64, 4
    q = oracle.bf16_from_f32(rng.standard_normal(T * hq * 128, dtype=np.float32))
    pos = rng.integers(0, 4160, size=T).astype(np.int32)
    # make the rotation cancel (x2 ~ x1 * cos / sin) at pairs whose sinf/cosf
    # are not correctly rounded, where the two evaluations can part by > 1 ulp
    rows = q.reshape(-1, 128)
    for r in range(T * hq):
        for p in range(64):
            a = R.angle(int(pos[r // hq]), p)
            sn, cs = R.host_sincos(a)
            if (sn, cs) != R.cr_sincos(a) and abs(sn) > 0.1:
                x1 = oracle.bf16_to_f32(rows[r, p:p + 1])[0]
                rows[r, 64 + p] = oracle.bf16_from_f32(np.array([x1 * cs / sn], np.float32))[0]
    qo, _ = oracle.rope_pos_ids(T, hq, 1, q, q[:T * 128], pos)
    rows = q.reshape(-1, 128)
    cr = np.array([[R.rotate_element(rows[r], c, int(pos[r // hq]), R.cr_sincos)
                    for c in range(128)] for r in range(T * hq)], np.uint16)
    per_row = np.repeat(pos, hq)
    beyond, unexplained = R.explain_beyond_one_ulp(cr, qo, q, per_row)
    assert not unexplained
    assert beyond > 0  # the cancelling elements do part by more than one ulp
    bad = cr.copy()
    r, c = 5, 9
    bad[r, c] = np.uint16(int(qo.reshape(-1, 128)[r, c]) + 2)
    _, unexplained = R.explain_beyond_one_ulp(bad, qo, q, per_row)
    assert [(u[0], u[1]) for u in unexplained] == [(r, c)]


def test_sincos_rounding_differs_for_a_few_percent_of_angles():
    pos = np.random.default_rng(3).integers(0, 4160, size=400)
    diff = sum(R.host_sincos(R.angle(int(P), p)) != R.cr_sincos(R.angle(int(P), p))
               for P in pos for p in range(64))
    frac = diff / (400 * 64)
    assert 0.005 < frac < 0.06, frac
