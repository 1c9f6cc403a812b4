"""Writes the golden vectors under tests/golden/ with the independent
pure-Python restatement (oracle/pyref.py).

The reference has no erasure coder, hence no vectors of its own; these pin
the C oracle and the GPU kernels to a restatement written from the
mathematics, which the CPU tests in turn pin to brute force, the field
axioms and the ISO/IEC 18004 Reed-Solomon example.  Inputs come from the
seeded generators of megatron-lm_amd/synth.py at small sizes.

    python tests/golden/make_golden.py      # rewrites the .npz files
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import __graft_entry__  # noqa: E402
from oracle import pyref  # noqa: E402

__graft_entry__.load_package()
from megatron_lm_amd import synth  # noqa: E402

SHARD = 1024


def rs_case(k, m, seed):
    shards = synth.rs_shards(seed, SHARD, k)
    parity = pyref.rs_encode(k, m, shards)
    er = synth.erasures(seed, k + m, m)
    codeword = shards + parity
    rec = pyref.decode(k, m, [None if g in er else codeword[g] for g in range(k + m)], er)
    return dict(k=np.int32(k), m=np.int32(m), data=np.stack(shards), parity=np.stack(parity),
                coeff=pyref.cauchy(k, m), erased=np.array(er, np.int32),
                recovered=np.stack([rec[g] for g in er]))


def ragged_case(seed):
    """RS(12,4) over a small ragged tensor list in 256-byte units, plus a 10%
    perturbation folded in."""
    k, m, unit = 12, 4, 256
    rng = np.random.default_rng(seed)
    sizes = (np.exp(rng.uniform(np.log(16), np.log(4096), 24)) // 4 * 4).astype(np.int64)
    data = rng.integers(0, 256, int(sizes.sum()), dtype=np.uint8)
    offs = np.concatenate([[0], np.cumsum(sizes)[:-1]])
    units, lens = [], []
    for o, n in zip(offs, sizes):
        for u in range(0, int(n), unit):
            units.append(data[o + u: o + min(n, u + unit)])
            lens.append(min(unit, int(n) - u))
    ns = (len(units) + k - 1) // k
    grid = [[units[s * k + j] if s * k + j < len(units) else None for j in range(k)]
            for s in range(ns)]
    glen = [[lens[s * k + j] if s * k + j < len(units) else 0 for j in range(k)]
            for s in range(ns)]
    parity = pyref.encode_units(k, m, grid, glen, unit)
    changed = np.sort(rng.choice(len(units), max(1, len(units) // 10), replace=False))
    new = data.copy()
    for u in changed:
        s, j = divmod(int(u), k)
        view = grid[s][j]
        start = int(view.ctypes.data - data.ctypes.data)
        new[start: start + lens[u]] = rng.integers(0, 256, lens[u], dtype=np.uint8)
    ngrid = [[None if x is None else new[int(x.ctypes.data - data.ctypes.data):
                                         int(x.ctypes.data - data.ctypes.data) + x.size]
              for x in row] for row in grid]
    parity2 = pyref.encode_units(k, m, ngrid, glen, unit)
    return dict(k=np.int32(k), m=np.int32(m), unit=np.int32(unit), sizes=sizes, data=data,
                parity=parity, changed=changed.astype(np.int64), new=new, parity_after=parity2)


def main():
    xs = synth.xor_shards(0, SHARD, 4)
    np.savez_compressed(os.path.join(HERE, "xor_k4.npz"), data=np.stack(xs),
                        parity=pyref.xor_encode(xs))
    for (k, m) in [(6, 3), (8, 2), (12, 4), (4, 1)]:
        for seed in (0, 1):
            np.savez_compressed(os.path.join(HERE, f"rs_{k}_{m}_s{seed}.npz"), **rs_case(k, m, seed))
    np.savez_compressed(os.path.join(HERE, "ragged_12_4.npz"), **ragged_case(0))
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)))


if __name__ == "__main__":
    main()
