"""Randomised agreement of the C oracle with the independent pure-Python
restatement (hypothesis): random (k, m), sizes, data and erasure patterns."""
import numpy as np
from hypothesis import HealthCheck, given, settings, strategies as st

import oracle
from oracle import pyref


@st.composite
def codes(draw):
    k = draw(st.integers(1, 14))
    m = draw(st.integers(1, 5))
    n = draw(st.integers(1, 300))
    seed = draw(st.integers(0, 2**32 - 1))
    rng = np.random.default_rng(seed)
    data = [rng.integers(0, 256, n, dtype=np.uint8) for _ in range(k)]
    e = draw(st.integers(0, m))
    lost = sorted(rng.choice(k + m, e, replace=False).tolist())
    return k, m, data, lost


@settings(max_examples=60, deadline=None, suppress_health_check=[HealthCheck.too_slow])
@given(codes())
def test_encode_and_decode_agree_with_pyref(case):
    k, m, data, lost = case
    C = oracle.cauchy(k, m)
    par = oracle.rs_encode(C, data)
    for a, b in zip(par, pyref.rs_encode(k, m, data)):
        assert np.array_equal(a, b)
    cw = data + par
    want = pyref.decode(k, m, [None if g in lost else cw[g] for g in range(k + m)], lost)
    if lost:
        surv, rows = oracle.decode_matrix(C, k, m, lost)
        got = oracle.rs_encode(rows, [cw[s] for s in surv])
        for g, r in zip(lost, got):
            assert np.array_equal(r, want[g]) and np.array_equal(r, cw[g])


@settings(max_examples=40, deadline=None)
@given(st.integers(1, 9), st.integers(0, 2**32 - 1))
def test_invert_agrees_with_pyref(n, seed):
    a = np.random.default_rng(seed).integers(0, 256, (n, n), dtype=np.uint8)
    try:
        want = pyref.inverse(a)
    except np.linalg.LinAlgError:
        try:
            oracle.gf_invert(a)
        except np.linalg.LinAlgError:
            return
        raise AssertionError("oracle inverted a matrix pyref found singular")
    assert np.array_equal(oracle.gf_invert(a), want)
