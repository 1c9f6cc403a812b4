"""Guard-byte canaries: every buffer the kernels write lives inside one
arena, separated by gaps of a known byte, at mixed alignments; after
encode, decode and update, every byte outside the buffers must still hold
the canary (no write past a ragged tail, a misaligned head, or a unit's
valid length)."""
import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu
CANARY = 0xC3


class Arena:
    def __init__(self, dev, nbytes, seed):
        self.buf = torch.full((nbytes,), CANARY, dtype=torch.uint8, device=dev)
        self.used = np.zeros(nbytes, bool)
        self.cursor = 64
        self.rng = np.random.default_rng(seed)

    def take(self, n, align=None):
        gap = int(self.rng.integers(1, 48))
        off = self.cursor + gap
        if align is not None:
            off = (off + 15) // 16 * 16 + align
        assert off + n + 64 <= self.buf.numel()
        self.cursor = off + n
        self.used[off: off + n] = True
        return self.buf[off: off + n]

    def check(self):
        torch.cuda.synchronize()
        host = self.buf.cpu().numpy()
        bad = np.flatnonzero((host != CANARY) & ~self.used)
        assert bad.size == 0, f"{bad.size} canary bytes overwritten, first at {bad[:8]}"


@pytest.mark.parametrize("k,m", [(6, 3), (12, 4), (20, 6)])
def test_flat_paths_stay_in_bounds(pkg, dev, k, m):
    rng = np.random.default_rng(k + m)
    n = 100_003
    ar = Arena(dev, (k + 3 * m + 4) * (n + 128), k * m)
    host = [rng.integers(0, 256, n, dtype=np.uint8) for _ in range(k)]
    data = []
    for j, h in enumerate(host):
        v = ar.take(n)                      # inputs at arbitrary alignments
        v.copy_(torch.from_numpy(h))
        data.append(v)
    same = [ar.take(n, align=5) for _ in range(m)]      # outputs sharing one skew
    mixed = [ar.take(n) for _ in range(m)]              # outputs at mixed skews
    pkg.rs_encode(data, m, out=same)
    pkg.rs_encode(data, m, out=mixed)
    want = oracle.rs_encode(oracle.cauchy(k, m), host)
    for a, b, w in zip(same, mixed, want):
        assert np.array_equal(a.cpu().numpy(), w) and np.array_equal(b.cpu().numpy(), w)
    lost = [0, k] if m > 1 else [0]
    cw = data + same
    rec = [ar.take(n, align=0) for _ in lost]
    pkg.reconstruct([None if g in lost else t for g, t in enumerate(cw)], k, m, out=rec)
    assert np.array_equal(rec[0].cpu().numpy(), host[0])
    x = ar.take(n, align=3)
    pkg.xor_encode(data, out=x)
    assert np.array_equal(x.cpu().numpy(), oracle.xor_encode(host))
    ar.check()


@pytest.mark.parametrize("k,m,unit,par_align", [(8, 2, 4096, 0), (12, 4, 16384, 7),
                                                 (6, 3, 65536, 0), (20, 6, 4096, 9)])
def test_batched_paths_stay_in_bounds(pkg, dev, k, m, unit, par_align):
    rng = np.random.default_rng(unit + k)
    sizes = rng.integers(1, 4 * unit, 3 * k)
    ar = Arena(dev, int(sizes.sum()) + 64 * len(sizes) + 4 * k * m * unit * 2 + (8 << 20), unit)
    host = [rng.integers(0, 256, int(s), dtype=np.uint8) for s in sizes]
    tensors = []
    for i, h in enumerate(host):
        v = ar.take(h.size, align=None if i % 3 else 0)
        v.copy_(torch.from_numpy(h))
        tensors.append(v)
    lay = pkg.StripeLayout(tensors, k, m, unit)
    par = ar.take(lay.n_stripes * m * unit, align=par_align).view(lay.n_stripes, m, unit)
    lay.encode(par)
    want = par.clone()
    lost = [1, k + m - 1]
    for s in range(lay.n_stripes):
        u = s * k + 1
        if u < lay.n_units:
            lay.unit_view(u).fill_(0x11)
        par[s, m - 1].fill_(0x22)
    lay.decode(par, lost)
    torch.cuda.synchronize()
    assert torch.equal(par, want)
    for h, t in zip(host, tensors):
        assert np.array_equal(t.cpu().numpy(), h)
    changed = np.sort(rng.choice(lay.n_units, max(1, lay.n_units // 5), replace=False))
    olds = []
    for u in changed:
        v = lay.unit_view(int(u))
        olds.append(v.clone())
        v.copy_(torch.from_numpy(rng.integers(0, 256, v.numel(), dtype=np.uint8)))
    lay.update(par, changed, olds)
    fresh = lay.encode()
    torch.cuda.synchronize()
    assert torch.equal(par, fresh)
    ar.check()
