"""Pins the CPU oracle (oracle/ec_oracle.c) and the SIMD CPU baseline.

The reference has no erasure coder, so nothing in it can pin these.  Each
check below comes from the mathematics, from a published vector, or from the
independent pure-Python restatement (oracle/pyref.py), chosen so that a
plausible slip (wrong polynomial, transposed coefficient index, dropped term,
wrong survivor row) fails at least one of them.
"""
import itertools
import os

import numpy as np
import pytest

import oracle
from oracle import pyref
from conftest import GOLDEN


# ------------------------------------------------------------------ field --

def test_mul_brute_force_all_pairs():
    """Every product equals the carry-less product reduced mod 0x11D
    (pyref uses polynomial long division, the oracle shift-and-reduce)."""
    t = pyref.mul_table()
    L = oracle.lib()
    got = np.array([[L.ecref_gf_mul(a, b) for b in range(256)] for a in range(256)], np.uint8)
    assert np.array_equal(got, t)


def test_field_axioms():
    t = pyref.mul_table().astype(np.int64)
    a = np.arange(256)
    assert np.array_equal(t, t.T)                                  # commutative
    assert np.array_equal(t[1], a) and not t[0].any()              # identity, zero
    rng = np.random.default_rng(0)
    x, y, z = rng.integers(0, 256, (3, 4000))
    assert np.array_equal(t[t[x, y], z], t[x, t[y, z]])            # associative
    assert np.array_equal(t[x, y ^ z], t[x, y] ^ t[x, z])          # distributive
    for v in range(1, 256):                                        # inverses
        assert t[v, oracle.gf_inv(v)] == 1
    assert oracle.gf_inv(0) == 0


def test_generator_two_is_primitive():
    seen, x = set(), 1
    for _ in range(255):
        seen.add(x)
        x = oracle.gf_mul(x, 2)
    assert x == 1 and len(seen) == 255
    # 2^8 = x^4 + x^3 + x^2 + 1 is the reduction polynomial itself.
    assert pyref.gf_mul(0x80, 2) == 0x1D


def test_iso18004_reed_solomon_example():
    """ISO/IEC 18004 (QR code) worked example, version 1-M, "01234567":
    16 data codewords -> 10 error-correction codewords, over GF(2^8)/0x11D
    with generator polynomial prod_{i<10} (x - 2^i).  A published vector for
    the field arithmetic the engine uses."""
    data = [0x10, 0x20, 0x0C, 0x56, 0x61, 0x80, 0xEC, 0x11,
            0xEC, 0x11, 0xEC, 0x11, 0xEC, 0x11, 0xEC, 0x11]
    expect = [0xA5, 0x24, 0xD4, 0xC1, 0xED, 0x36, 0xC7, 0x87, 0x2C, 0x55]
    for mul in (oracle.gf_mul, pyref.gf_mul):
        g, a = [1], 1
        for _ in range(10):
            g = [p ^ mul(c, a) for c, p in zip(g + [0], [0] + g)]  # g * (x + a), low first
            a = mul(a, 2)
        g = g[::-1]  # highest degree first
        msg = data + [0] * 10
        for i in range(len(data)):
            c = msg[i]
            if c:
                for d in range(len(g)):
                    msg[i + d] ^= mul(g[d], c)
        assert msg[-10:] == expect


# ---------------------------------------------------------------- matrices --

@pytest.mark.parametrize("k,m", [(4, 1), (6, 3), (8, 2), (12, 4), (16, 4), (1, 1), (200, 56)])
def test_cauchy_closed_form(k, m):
    c = oracle.cauchy(k, m)
    assert np.array_equal(c, pyref.cauchy(k, m))
    for i in range(m):
        for j in range(k):
            assert pyref.gf_mul(int(c[i, j]), (k + i) ^ j) == 1


@pytest.mark.parametrize("k,m,count", [(4, 1, 5), (6, 3, 84), (8, 2, 45), (12, 4, 1820)])
def test_mds_every_k_subset_invertible(k, m, count):
    """[I;C] is MDS: every k rows form an invertible matrix, and the oracle's
    inverse really is one (A @ inv(A) = I over GF(2^8))."""
    g = np.vstack([np.eye(k, dtype=np.uint8), oracle.cauchy(k, m)])
    n = 0
    for rows in itertools.combinations(range(k + m), k):
        a = g[list(rows)]
        inv = oracle.gf_invert(a)
        if n % 97 == 0:  # full product check on a spread sample (pure Python is slow)
            assert np.array_equal(pyref.mat_mul(a, inv), np.eye(k, dtype=np.uint8))
        n += 1
    assert n == count


def test_invert_rejects_singular():
    a = np.array([[1, 2], [2, 4]], np.uint8)   # row 2 = 2 * row 1
    with pytest.raises(np.linalg.LinAlgError):
        oracle.gf_invert(a)
    with pytest.raises(np.linalg.LinAlgError):
        oracle.decode_matrix(oracle.cauchy(6, 3), 6, 3, [0, 1, 2, 3])


def test_invert_random_against_pyref():
    rng = np.random.default_rng(3)
    for n in (1, 2, 5, 9):
        a = rng.integers(0, 256, (n, n), dtype=np.uint8)
        try:
            want = pyref.inverse(a)
        except np.linalg.LinAlgError:
            continue
        assert np.array_equal(oracle.gf_invert(a), want)


# ------------------------------------------------------------------ encode --

def _rand_shards(rng, k, n):
    return [rng.integers(0, 256, n, dtype=np.uint8) for _ in range(k)]


@pytest.mark.parametrize("k,m,n", [(6, 3, 4096), (4, 1, 777), (8, 2, 1), (12, 4, 300), (3, 7, 64)])
def test_rs_encode_matches_pyref(k, m, n):
    rng = np.random.default_rng(k * 100 + m)
    d = _rand_shards(rng, k, n)
    got = oracle.rs_encode(oracle.cauchy(k, m), d)
    want = pyref.rs_encode(k, m, d)
    for g, w in zip(got, want):
        assert np.array_equal(g, w)


def test_unit_vector_response():
    """One byte x at shard j, zeros elsewhere: parity_i = C[i][j] * x.  Pins
    the coefficient index order (a transposed C fails here)."""
    k, m, n = 6, 3, 256
    c = pyref.cauchy(k, m)
    for j in range(k):
        d = [np.zeros(n, np.uint8) for _ in range(k)]
        d[j][:] = np.arange(256, dtype=np.uint8)
        par = oracle.rs_encode(oracle.cauchy(k, m), d)
        for i in range(m):
            assert np.array_equal(par[i], pyref.mul_table()[c[i, j]])


def test_linearity_and_zero():
    k, m, n = 8, 2, 1000
    rng = np.random.default_rng(5)
    a, b = _rand_shards(rng, k, n), _rand_shards(rng, k, n)
    C = oracle.cauchy(k, m)
    pa, pb = oracle.rs_encode(C, a), oracle.rs_encode(C, b)
    pab = oracle.rs_encode(C, [x ^ y for x, y in zip(a, b)])
    for i in range(m):
        assert np.array_equal(pab[i], pa[i] ^ pb[i])
    assert not any(p.any() for p in oracle.rs_encode(C, [np.zeros(n, np.uint8)] * k))


def test_xor_closed_form():
    rng = np.random.default_rng(9)
    d = _rand_shards(rng, 4, 5000)
    assert np.array_equal(oracle.xor_encode(d), np.bitwise_xor.reduce(np.stack(d), axis=0))
    # XOR parity is not the m = 1 Cauchy row: inv(4 ^ j) != 1 for some j.
    assert oracle.cauchy(4, 1).tolist() != [[1, 1, 1, 1]]


# ------------------------------------------------------------------ decode --

@pytest.mark.parametrize("k,m", [(6, 3), (4, 1), (8, 2)])
def test_decode_every_erasure_pattern(k, m):
    n = 512
    rng = np.random.default_rng(k + 10 * m)
    d = _rand_shards(rng, k, n)
    C = oracle.cauchy(k, m)
    cw = d + oracle.rs_encode(C, d)
    patterns = 0
    for e in range(0, m + 1):
        for lost in itertools.combinations(range(k + m), e):
            surv, rows = oracle.decode_matrix(C, k, m, list(lost))
            assert surv == [g for g in range(k + m) if g not in lost][:k]
            rec = oracle.rs_encode(rows, [cw[s] for s in surv]) if lost else []
            for g, r in zip(lost, rec):
                assert np.array_equal(r, cw[g])
            patterns += 1
    assert patterns == sum(len(list(itertools.combinations(range(k + m), e))) for e in range(m + 1))


def test_decode_rows_match_pyref():
    k, m = 12, 4
    C = oracle.cauchy(k, m)
    g = pyref.generator(k, m)
    for lost in [(0, 5, 12, 15), (13,), (1, 2, 3, 4), (11, 12, 13, 14)]:
        surv, rows = oracle.decode_matrix(C, k, m, list(lost))
        want = pyref.mat_mul(g[list(lost)], pyref.inverse(g[surv]))
        assert np.array_equal(rows, want)


# ------------------------------------------------------- batched / update --

def _ragged(rng, k, unit, n_tensors=17):
    sizes = rng.integers(1, 5 * unit, n_tensors)
    tensors = [rng.integers(0, 256, s, dtype=np.uint8) for s in sizes]
    units, lens = [], []
    for t in tensors:
        for o in range(0, t.size, unit):
            units.append(t[o: o + unit])
            lens.append(min(unit, t.size - o))
    ns = (len(units) + k - 1) // k
    grid = [[units[s * k + j] if s * k + j < len(units) else None for j in range(k)]
            for s in range(ns)]
    glen = np.array([[lens[s * k + j] if s * k + j < len(units) else 0 for j in range(k)]
                     for s in range(ns)], np.uint32)
    return grid, glen


def test_batched_matches_padded_stripes():
    k, m, unit = 12, 4, 96
    rng = np.random.default_rng(11)
    grid, glen = _ragged(rng, k, unit)
    got = oracle.encode_batched(oracle.cauchy(k, m), grid, glen, unit)
    assert np.array_equal(got, pyref.encode_units(k, m, grid, glen, unit))


def test_parity_update_equals_reencode():
    k, m, unit = 6, 3, 64
    rng = np.random.default_rng(12)
    grid, glen = _ragged(rng, k, unit, 9)
    C = oracle.cauchy(k, m)
    par = oracle.encode_batched(C, grid, glen, unit)
    new_grid = [[None if u is None else u.copy() for u in row] for row in grid]
    newu = [[None] * k for _ in grid]
    oldu = [[None] * k for _ in grid]
    for s, row in enumerate(new_grid):
        for j, u in enumerate(row):
            if u is not None and rng.random() < 0.3:
                oldu[s][j] = u.copy()
                u[:] = rng.integers(0, 256, u.size, dtype=np.uint8)
                newu[s][j] = u
    oracle.parity_update(C, newu, oldu, glen, par, unit)
    assert np.array_equal(par, oracle.encode_batched(C, new_grid, glen, unit))


# ---------------------------------------------------------- SIMD baseline --

@pytest.mark.parametrize("isa", ["scalar", "avx2", "avx512", "gfni512"])
def test_fast_encoder_matches_oracle(isa):
    default = oracle.fast_isa()
    if not oracle.fast_force_isa(isa):
        pytest.skip(f"{isa} not supported on this host")
    try:
        rng = np.random.default_rng(21)
        for (k, m, n, threads) in [(6, 3, 100_003, 3), (12, 4, 4096, 1), (4, 1, 65, 2),
                                   (8, 2, 1 << 16, 4), (1, 1, 7, 1)]:
            d = _rand_shards(rng, k, n)
            C = oracle.cauchy(k, m)
            want = oracle.rs_encode(C, d)
            got = oracle.fast_rs_encode(C, d, nthreads=threads)
            for g, w in zip(got, want):
                assert np.array_equal(g, w)
            assert np.array_equal(oracle.fast_xor_encode(d, nthreads=threads), oracle.xor_encode(d))
    finally:
        oracle.fast_force_isa(default)


@pytest.mark.parametrize("isa", ["scalar", "avx2", "avx512", "gfni512"])
def test_fast_batched_encoder_matches_oracle(isa):
    """The SIMD batched encoder (the CPU baseline and full-size checker of
    configs 4 and 5) equals the scalar oracle's batched encode on ragged
    stripes with short and absent units, for several thread counts."""
    default = oracle.fast_isa()
    if not oracle.fast_force_isa(isa):
        pytest.skip(f"{isa} not supported on this host")
    try:
        rng = np.random.default_rng(22)
        for k, m, unit, threads in [(12, 4, 96, 3), (8, 2, 4096, 2), (6, 3, 64, 1),
                                    (4, 1, 1024, 7)]:
            grid, glen = _ragged(rng, k, unit)
            C = oracle.cauchy(k, m)
            want = oracle.encode_batched(C, grid, glen, unit)
            ns = len(grid)
            dptr = np.array([[0 if u is None else u.ctypes.data for u in row] for row in grid],
                            np.uint64).reshape(ns, k)
            got = np.full((ns, m, unit), 0xEE, np.uint8)
            pptr = np.array([[got[s, i].ctypes.data for i in range(m)] for s in range(ns)],
                            np.uint64).reshape(ns, m)
            oracle.fast_encode_batched(C, dptr, glen, pptr, unit, nthreads=threads)
            assert np.array_equal(got, want), (k, m, unit, threads)
    finally:
        oracle.fast_force_isa(default)


@pytest.mark.parametrize("isa", ["scalar", "avx2", "avx512", "gfni512"])
def test_fast_parity_update_matches_oracle(isa):
    """The SIMD incremental update (the CPU baseline beside the GPU update)
    equals the scalar oracle's update on ragged stripes with short, absent
    and unchanged units, for several thread counts, and both equal a fresh
    encode of the changed bytes."""
    default = oracle.fast_isa()
    if not oracle.fast_force_isa(isa):
        pytest.skip(f"{isa} not supported on this host")
    try:
        rng = np.random.default_rng(23)
        for k, m, unit, threads, frac in [(12, 4, 96, 3, 0.3), (8, 2, 4096, 2, 0.1),
                                          (6, 3, 64, 1, 1.0), (4, 1, 1024, 7, 0.5),
                                          (12, 4, 65536, 4, 0.05)]:
            grid, glen = _ragged(rng, k, unit, 9)
            C = oracle.cauchy(k, m)
            par0 = oracle.encode_batched(C, grid, glen, unit)
            new_grid = [[None if u is None else u.copy() for u in row] for row in grid]
            ns = len(grid)
            nptr = np.zeros((ns, k), np.uint64)
            optr = np.zeros((ns, k), np.uint64)
            newu = [[None] * k for _ in grid]
            oldu = [[None] * k for _ in grid]
            for s, row in enumerate(new_grid):
                for j, u in enumerate(row):
                    if u is not None and rng.random() < frac:
                        oldu[s][j] = grid[s][j]
                        u[:] = rng.integers(0, 256, u.size, dtype=np.uint8)
                        newu[s][j] = u
                        nptr[s, j], optr[s, j] = u.ctypes.data, grid[s][j].ctypes.data
            want = oracle.parity_update(C, newu, oldu, glen, par0.copy(), unit)
            got = par0.copy()
            pptr = np.array([[got[s, i].ctypes.data for i in range(m)] for s in range(ns)],
                            np.uint64).reshape(ns, m)
            oracle.fast_parity_update(C, nptr, optr, glen, pptr, unit, nthreads=threads)
            assert np.array_equal(got, want), (k, m, unit, threads)
            assert np.array_equal(got, oracle.encode_batched(C, new_grid, glen, unit))
    finally:
        oracle.fast_force_isa(default)


# ------------------------------------------------------------------ golden --

def _golden(name):
    return np.load(os.path.join(GOLDEN, name))


def test_golden_xor():
    g = _golden("xor_k4.npz")
    assert np.array_equal(oracle.xor_encode(list(g["data"])), g["parity"])


@pytest.mark.parametrize("name", sorted(f for f in os.listdir(GOLDEN) if f.startswith("rs_")))
def test_golden_rs(name):
    g = _golden(name)
    k, m = int(g["k"]), int(g["m"])
    assert np.array_equal(oracle.cauchy(k, m), g["coeff"])
    par = oracle.rs_encode(g["coeff"], list(g["data"]))
    assert np.array_equal(np.stack(par), g["parity"])
    cw = list(g["data"]) + list(g["parity"])
    er = [int(x) for x in g["erased"]]
    surv, rows = oracle.decode_matrix(g["coeff"], k, m, er)
    rec = oracle.rs_encode(rows, [cw[s] for s in surv])
    assert np.array_equal(np.stack(rec), g["recovered"])
    assert all(np.array_equal(r, cw[e]) for r, e in zip(rec, er))


def test_golden_ragged():
    g = _golden("ragged_12_4.npz")
    k, m, unit = int(g["k"]), int(g["m"]), int(g["unit"])
    offs = np.concatenate([[0], np.cumsum(g["sizes"])[:-1]])
    units, lens = [], []
    for o, n in zip(offs, g["sizes"]):
        for u in range(0, int(n), unit):
            units.append((o + u, min(unit, int(n) - u)))
    ns = (len(units) + k - 1) // k

    def grid_of(buf):
        return [[buf[units[s * k + j][0]: units[s * k + j][0] + units[s * k + j][1]]
                 if s * k + j < len(units) else None for j in range(k)] for s in range(ns)]
    glen = np.array([[units[s * k + j][1] if s * k + j < len(units) else 0 for j in range(k)]
                     for s in range(ns)], np.uint32)
    C = oracle.cauchy(k, m)
    par = oracle.encode_batched(C, grid_of(g["data"]), glen, unit)
    assert np.array_equal(par, g["parity"])
    newu = [[None] * k for _ in range(ns)]
    oldu = [[None] * k for _ in range(ns)]
    ng, og = grid_of(g["new"]), grid_of(g["data"])
    for u in g["changed"]:
        s, j = divmod(int(u), k)
        newu[s][j], oldu[s][j] = ng[s][j], og[s][j]
    fast = par.copy()
    oracle.parity_update(C, newu, oldu, glen, par, unit)
    assert np.array_equal(par, g["parity_after"])
    # the SIMD update over host descriptors of the same bytes
    nptr = np.array([[0 if u is None else u.ctypes.data for u in row] for row in newu],
                    np.uint64).reshape(ns, k)
    optr = np.array([[0 if u is None else u.ctypes.data for u in row] for row in oldu],
                    np.uint64).reshape(ns, k)
    pptr = np.array([[fast[s, i].ctypes.data for i in range(m)] for s in range(ns)],
                    np.uint64).reshape(ns, m)
    oracle.fast_parity_update(C, nptr, optr, glen, pptr, unit, nthreads=3)
    assert np.array_equal(fast, g["parity_after"])
