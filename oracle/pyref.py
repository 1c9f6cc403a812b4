"""Independent pure-Python restatement of the erasure code (no C, no tables
shared with ``ec_oracle.c``).

TEST INFRASTRUCTURE: used by ``tests/`` to cross-check the C oracle and by
``tests/golden/make_golden.py`` to write the golden vectors.  The reference
has no erasure coder; this follows the mathematics only:

* field multiply = polynomial product over GF(2) followed by long division by
  x^8+x^4+x^3+x^2+1 (0x11D) — a different algorithm from the shift-and-reduce
  loop of the C oracle;
* inverse = exhaustive search for b with a*b == 1;
* C[i][j] = inv((k+i) ^ j);
* decode = solve with the k x k survivor rows of [I; C] by Gaussian
  elimination on an augmented system, one right-hand side per lost shard.
Byte streams are processed with numpy gathers through a 256 x 256 product
table built from ``gf_mul`` below.
"""
from __future__ import annotations

from functools import lru_cache

import numpy as np

POLY = 0x11D


def clmul(a: int, b: int) -> int:
    """Carry-less product of two polynomials over GF(2)."""
    r = 0
    for bit in range(b.bit_length()):
        if (b >> bit) & 1:
            r ^= a << bit
    return r


def poly_mod(x: int, p: int = POLY) -> int:
    """Remainder of x divided by p over GF(2) (long division)."""
    dp = p.bit_length()
    while x.bit_length() >= dp:
        x ^= p << (x.bit_length() - dp)
    return x


def gf_mul(a: int, b: int) -> int:
    return poly_mod(clmul(a, b))


@lru_cache(maxsize=None)
def gf_inv(a: int) -> int:
    if a == 0:
        return 0
    for b in range(1, 256):
        if gf_mul(a, b) == 1:
            return b
    raise ArithmeticError("no inverse")  # impossible for an irreducible POLY


@lru_cache(maxsize=1)
def mul_table() -> np.ndarray:
    t = np.zeros((256, 256), np.uint8)
    for a in range(256):
        for b in range(256):
            t[a, b] = gf_mul(a, b)
    return t


def cauchy(k: int, m: int) -> np.ndarray:
    c = np.zeros((m, k), np.uint8)
    for i in range(m):
        for j in range(k):
            c[i, j] = gf_inv((k + i) ^ j)
    return c


def generator(k: int, m: int) -> np.ndarray:
    return np.vstack([np.eye(k, dtype=np.uint8), cauchy(k, m)])


def mat_mul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    t = mul_table()
    n, p = a.shape
    p2, q = b.shape
    assert p == p2
    out = np.zeros((n, q), np.uint8)
    for i in range(n):
        for j in range(q):
            acc = 0
            for s in range(p):
                acc ^= int(t[a[i, s], b[s, j]])
            out[i, j] = acc
    return out


def solve(a: np.ndarray, rhs: np.ndarray) -> np.ndarray:
    """Solve a @ x = rhs over GF(2^8) (a square); raises if singular."""
    t = mul_table()
    n = a.shape[0]
    aug = np.concatenate([a.astype(np.uint8), rhs.astype(np.uint8)], axis=1)
    for c in range(n):
        piv = next((r for r in range(c, n) if aug[r, c]), None)
        if piv is None:
            raise np.linalg.LinAlgError("singular")
        aug[[c, piv]] = aug[[piv, c]]
        aug[c] = t[gf_inv(int(aug[c, c]))][aug[c]]
        for r in range(n):
            if r != c and aug[r, c]:
                aug[r] ^= t[int(aug[r, c])][aug[c]]
    return aug[:, n:]


def inverse(a: np.ndarray) -> np.ndarray:
    return solve(a, np.eye(a.shape[0], dtype=np.uint8))


def xor_encode(shards) -> np.ndarray:
    out = np.zeros_like(np.asarray(shards[0]).view(np.uint8).reshape(-1))
    for s in shards:
        out ^= np.asarray(s).view(np.uint8).reshape(-1)
    return out


def matvec_bytes(mat: np.ndarray, shards) -> list:
    """out[i][b] = XOR_j mat[i][j] * shards[j][b]."""
    t = mul_table()
    shards = [np.asarray(s).view(np.uint8).reshape(-1) for s in shards]
    outs = []
    for i in range(mat.shape[0]):
        acc = np.zeros_like(shards[0])
        for j, d in enumerate(shards):
            acc ^= t[int(mat[i, j])][d]
        outs.append(acc)
    return outs


def rs_encode(k: int, m: int, shards) -> list:
    return matvec_bytes(cauchy(k, m), shards)


def decode(k: int, m: int, codeword: list, erased) -> dict:
    """Recover the erased shards of a k+m codeword (list of arrays; erased
    entries ignored).  Uses the first k surviving shards."""
    erased = sorted(set(erased))
    if len(erased) > m:
        raise np.linalg.LinAlgError("more erasures than parity shards")
    g = generator(k, m)
    surv = [s for s in range(k + m) if s not in erased][:k]
    gs = g[surv]
    # data = inv(gs) @ survivors;  lost_e = g[e] @ data
    rows = mat_mul(g[erased], inverse(gs)) if erased else np.zeros((0, k), np.uint8)
    rec = matvec_bytes(rows, [codeword[s] for s in surv])
    return dict(zip(erased, rec))


def encode_units(k: int, m: int, units, lens, unit_bytes: int) -> np.ndarray:
    """Stripe encode with zero padding: units[s][j] (or None), lens[s][j]."""
    ns = len(units)
    out = np.zeros((ns, m, unit_bytes), np.uint8)
    for s in range(ns):
        padded = []
        for j in range(k):
            p = np.zeros(unit_bytes, np.uint8)
            u = units[s][j]
            if u is not None:
                ln = int(lens[s][j])
                p[:ln] = np.asarray(u).view(np.uint8).reshape(-1)[:ln]
            padded.append(p)
        for i, par in enumerate(rs_encode(k, m, padded)):
            out[s, i] = par
    return out
