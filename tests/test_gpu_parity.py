"""GPU parity: the HIP kernels, called through the C ABI, against the CPU
oracle on the same seeded bytes.  Integer work, so the bar is byte equality.
"""
import itertools
import os

import numpy as np
import pytest
import torch

import oracle
from conftest import GOLDEN

pytestmark = pytest.mark.gpu


def _host(rng, k, n):
    return [rng.integers(0, 256, n, dtype=np.uint8) for _ in range(k)]


def _to_dev(arrays, dev, offset=0):
    """Device copies; with offset > 0, views starting offset bytes into a
    larger allocation (misaligned pointers)."""
    out = []
    for a in arrays:
        buf = torch.empty(a.size + offset, dtype=torch.uint8, device=dev)
        view = buf[offset:]
        view.copy_(torch.from_numpy(a))
        out.append(view)
    return out


def _eq(t, a):
    torch.cuda.synchronize()
    return np.array_equal(t.cpu().numpy(), a)


def test_rs_encode_every_instantiated_shape(pkg, dev):
    """All K in 1..16 x M in 1..4 (the template-instantiated fast kernels)."""
    rng = np.random.default_rng(0)
    n = 4096 * 3 + 16 * 5
    for k in range(1, 17):
        d = _host(rng, k, n)
        dd = _to_dev(d, dev)
        for m in range(1, 5):
            C = oracle.cauchy(k, m)
            par = pkg.rs_encode(dd, m)
            want = oracle.rs_encode(C, d)
            for i in range(m):
                assert _eq(par[i], want[i]), f"k={k} m={m} parity {i}"


@pytest.mark.parametrize("n", [1, 15, 16, 17, 255, 4096, 65536 + 7, (1 << 20) + 5, 3 << 20])
def test_rs_encode_sizes_and_tails(pkg, dev, n):
    rng = np.random.default_rng(n)
    d = _host(rng, 6, n)
    par = pkg.rs_encode(_to_dev(d, dev), 3)
    for p, w in zip(par, oracle.rs_encode(oracle.cauchy(6, 3), d)):
        assert _eq(p, w)


@pytest.mark.parametrize("offset", [1, 4, 8, 12])
def test_rs_encode_misaligned(pkg, dev, offset):
    rng = np.random.default_rng(offset)
    n = 70001
    d = _host(rng, 6, n)
    dd = _to_dev(d, dev, offset)
    out = _to_dev([np.zeros(n, np.uint8)] * 3, dev, offset)
    pkg.rs_encode(dd, 3, out=out)
    for p, w in zip(out, oracle.rs_encode(oracle.cauchy(6, 3), d)):
        assert _eq(p, w)


def test_rs_encode_mixed_misalignment(pkg, dev):
    """Shards misaligned by different amounts (byte path throughout) and by a
    common amount with the outputs aligned (byte path throughout too)."""
    rng = np.random.default_rng(31)
    n = 50_001
    d = _host(rng, 6, n)
    dd = [_to_dev([a], dev, off)[0] for a, off in zip(d, [1, 2, 3, 4, 5, 6])]
    out = [_to_dev([np.zeros(n, np.uint8)], dev, off)[0] for off in (7, 0, 9)]
    pkg.rs_encode(dd, 3, out=out)
    want = oracle.rs_encode(oracle.cauchy(6, 3), d)
    for p, w in zip(out, want):
        assert _eq(p, w)
    dd = _to_dev(d, dev, 5)
    par = pkg.rs_encode(dd, 3)
    for p, w in zip(par, want):
        assert _eq(p, w)


@pytest.mark.parametrize("k,m", [(20, 6), (32, 16), (17, 1), (5, 9), (16, 5), (32, 1), (9, 16)])
@pytest.mark.parametrize("offset", [0, 3])
def test_rs_encode_wide_codes(pkg, dev, k, m, offset):
    """Codes past the instantiated fast path (k > 16 or m > 4): the wide
    kernel on aligned shards; with a common misalignment, byte-path head
    and tail around it."""
    rng = np.random.default_rng(k * m + offset)
    n = 12345 + 4096 * 70
    d = _host(rng, k, n)
    out = _to_dev([np.zeros(n, np.uint8)] * m, dev, offset)
    pkg.rs_encode(_to_dev(d, dev, offset), m, out=out)
    for p, w in zip(out, oracle.rs_encode(oracle.cauchy(k, m), d)):
        assert _eq(p, w)


def test_rs_encode_generic_kernel_mixed_misalignment(pkg, dev):
    """Different misalignments take the byte path throughout, wide codes too."""
    k, m, n = 20, 6, 9999
    rng = np.random.default_rng(5)
    d = _host(rng, k, n)
    dd = [_to_dev([a], dev, j % 7)[0] for j, a in enumerate(d)]
    par = pkg.rs_encode(dd, m)
    for p, w in zip(par, oracle.rs_encode(oracle.cauchy(k, m), d)):
        assert _eq(p, w)


def test_rs_encode_arbitrary_coefficients(pkg, dev):
    """Any m x k matrix, including zeros and ones (decode rows look like this)."""
    rng = np.random.default_rng(7)
    n = 50000
    for k, m in [(6, 3), (12, 4), (3, 2)]:
        C = rng.integers(0, 256, (m, k), dtype=np.uint8)
        C[0, 0] = 0
        C[-1, -1] = 1
        d = _host(rng, k, n)
        par = pkg.matvec(C, _to_dev(d, dev))
        for p, w in zip(par, oracle.rs_encode(C, d)):
            assert _eq(p, w)


@pytest.mark.parametrize("k", list(range(1, 17)) + [20, 32])
def test_xor_encode(pkg, dev, k):
    rng = np.random.default_rng(100 + k)
    for n, off in [(4096 * 5 + 48, 0), (777, 0), (9999, 3), (70_000, 11), (5, 13)]:
        d = _host(rng, k, n)
        p = pkg.xor_encode(_to_dev(d, dev, off))
        assert _eq(p, oracle.xor_encode(d)), f"k={k} n={n} off={off}"
        # output at the same misalignment: head bytes, then the vector path
        q = _to_dev([np.zeros(n, np.uint8)], dev, off)[0]
        pkg.xor_encode(_to_dev(d, dev, off), out=q)
        assert _eq(q, oracle.xor_encode(d)), f"k={k} n={n} off={off} (common skew)"


@pytest.mark.parametrize("k,m", [(6, 3), (4, 1), (8, 2)])
def test_decode_every_erasure_pattern(pkg, dev, k, m):
    rng = np.random.default_rng(k * 10 + m)
    n = 65536 + 16
    d = _host(rng, k, n)
    dd = _to_dev(d, dev)
    cw = dd + pkg.rs_encode(dd, m)
    for e in range(1, m + 1):
        for lost in itertools.combinations(range(k + m), e):
            rec = pkg.reconstruct([None if g in lost else t for g, t in enumerate(cw)], k, m)
            torch.cuda.synchronize()
            for g in lost:
                assert torch.equal(rec[g], cw[g]), f"lost={lost} shard {g}"


def test_decode_12_4_sampled_patterns(pkg, dev):
    k, m = 12, 4
    rng = np.random.default_rng(44)
    dd = _to_dev(_host(rng, k, 200_000), dev)
    cw = dd + pkg.rs_encode(dd, m)
    pats = list(itertools.combinations(range(16), 4))
    for idx in rng.choice(len(pats), 60, replace=False):
        lost = pats[idx]
        rec = pkg.reconstruct([None if g in lost else t for g, t in enumerate(cw)], k, m)
        torch.cuda.synchronize()
        assert all(torch.equal(rec[g], cw[g]) for g in lost), lost


def test_too_many_erasures_rejected(pkg, dev):
    dd = _to_dev(_host(np.random.default_rng(0), 6, 64), dev)
    cw = dd + pkg.rs_encode(dd, 3)
    with pytest.raises(pkg.SingularError):
        pkg.reconstruct([None] * 4 + cw[4:], 6, 3)


def test_side_stream(pkg, dev):
    rng = np.random.default_rng(5)
    d = _host(rng, 6, 1 << 20)
    dd = _to_dev(d, dev)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        out = [torch.empty(1 << 20, dtype=torch.uint8, device=dev) for _ in range(3)]
    pkg.rs_encode(dd, 3, out=out, stream=s)
    s.synchronize()
    for p, w in zip(out, oracle.rs_encode(oracle.cauchy(6, 3), d)):
        assert np.array_equal(p.cpu().numpy(), w)


# ------------------------------------------------------------------ golden --

def test_golden_xor(pkg, dev):
    g = np.load(os.path.join(GOLDEN, "xor_k4.npz"))
    assert _eq(pkg.xor_encode(_to_dev(list(g["data"]), dev)), g["parity"])


@pytest.mark.parametrize("name", sorted(f for f in os.listdir(GOLDEN) if f.startswith("rs_")))
def test_golden_rs(pkg, dev, name):
    g = np.load(os.path.join(GOLDEN, name))
    k, m = int(g["k"]), int(g["m"])
    dd = _to_dev(list(g["data"]), dev)
    par = pkg.rs_encode(dd, m)
    for i in range(m):
        assert _eq(par[i], g["parity"][i])
    er = [int(x) for x in g["erased"]]
    cw = dd + par
    rec = pkg.reconstruct([None if x in er else t for x, t in enumerate(cw)], k, m)
    for r, e in enumerate(er):
        assert _eq(rec[e], g["recovered"][r])


# ---------------------------------------------------------------- batched --

@pytest.mark.parametrize("arena", [False, True])
def test_golden_ragged_encode_and_update(pkg, dev, arena):
    """The committed ragged fixture (RS(12,4), 256-byte units over 24 tensors,
    written by the pure-Python restatement): the batched encode equals its
    ``parity``, and the incremental update of its ``changed`` units to the
    bytes of ``new`` equals its ``parity_after``.  The tensors are separate
    allocations, or (arena) views back to back in one buffer, 4-byte aligned
    as the fixture's sizes leave them."""
    g = np.load(os.path.join(GOLDEN, "ragged_12_4.npz"))
    k, m, unit = int(g["k"]), int(g["m"]), int(g["unit"])
    sizes = [int(x) for x in g["sizes"]]
    offs = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(int)
    if arena:
        buf = torch.from_numpy(g["data"]).to(dev)
        tensors = [buf[o: o + n] for o, n in zip(offs, sizes)]
    else:
        tensors = [torch.from_numpy(g["data"][o: o + n]).to(dev) for o, n in zip(offs, sizes)]
    pset = pkg.encode(tensors, k, m, unit)
    lay = pset.layout
    torch.cuda.synchronize()
    assert np.array_equal(pset.parity.cpu().numpy(), g["parity"])
    olds = []
    for u in g["changed"]:
        u = int(u)
        v = lay.unit_view(u)
        olds.append(v.clone())
        t, i = int(lay.unit_tensor[u]), int(lay.unit_index[u])
        start = int(offs[t]) + i * unit
        v.copy_(torch.from_numpy(g["new"][start: start + v.numel()]))
    pkg.update(pset, g["changed"], olds)
    torch.cuda.synchronize()
    assert np.array_equal(pset.parity.cpu().numpy(), g["parity_after"])
    got = np.concatenate([t.cpu().numpy() for t in tensors])
    assert np.array_equal(got, g["new"])



def _ragged_device(rng, dev, n_tensors, max_bytes, misalign=False):
    """Device tensors of random byte sizes (some zero-length-free, some odd),
    optionally as views at odd offsets of one arena whose gaps hold 0xC3 (a
    kernel reading past a tensor's end would fold them into the parity)."""
    sizes = rng.integers(1, max_bytes, n_tensors)
    host = [rng.integers(0, 256, s, dtype=np.uint8) for s in sizes]
    if not misalign:
        return host, [torch.from_numpy(h).to(dev) for h in host]
    arena = torch.full((int(sizes.sum()) + 7 * n_tensors,), 0xC3, dtype=torch.uint8, device=dev)
    views, off = [], 0
    for h in host:
        off += int(rng.integers(0, 7))
        v = arena[off: off + h.size]
        v.copy_(torch.from_numpy(h))
        views.append(v)
        off += h.size
    return host, views


def _oracle_layout_parity(layout, host, unit):
    """Oracle parity of the same stripes, from host copies of the units."""
    k, m = layout.k, layout.m
    grid = []
    for s in range(layout.n_stripes):
        row = []
        for j in range(k):
            u = s * k + j
            if u >= layout.n_units:
                row.append(None)
                continue
            t, i = int(layout.unit_tensor[u]), int(layout.unit_index[u])
            row.append(host[t][i * unit: (i + 1) * unit])
        grid.append(row)
    return oracle.encode_batched(layout.coeff, grid, layout.host_len, unit)


def _perturb_units(rng, layout, host, changed):
    """New random bytes (seeded numpy) for the changed units, written into
    the device tensors and into host copies of the tensors.  Returns the
    device copies of the old bytes (the update's input) and the host copies
    of the tensors after the change."""
    unit = layout.unit_bytes
    host_new = [h.copy() for h in host]
    olds = []
    for u in changed:
        u = int(u)
        v = layout.unit_view(u)
        olds.append(v.clone())
        fresh = rng.integers(0, 256, v.numel(), dtype=np.uint8)
        v.copy_(torch.from_numpy(fresh))
        t, i = int(layout.unit_tensor[u]), int(layout.unit_index[u])
        host_new[t][i * unit: i * unit + fresh.size] = fresh
    return olds, host_new


def _oracle_update(layout, host_old, host_new, changed, par_before):
    """The oracle's incremental update (ecref_parity_update) of a copy of
    ``par_before`` over host copies of the changed units' old and new bytes."""
    k, unit = layout.k, layout.unit_bytes
    newu = [[None] * k for _ in range(layout.n_stripes)]
    oldu = [[None] * k for _ in range(layout.n_stripes)]
    for u in changed:
        s, j = divmod(int(u), k)
        t, i = int(layout.unit_tensor[u]), int(layout.unit_index[u])
        newu[s][j] = host_new[t][i * unit: (i + 1) * unit]
        oldu[s][j] = host_old[t][i * unit: (i + 1) * unit]
    return oracle.parity_update(layout.coeff, newu, oldu, layout.host_len, par_before.copy(), unit)


@pytest.mark.parametrize("k,m,unit,misalign", [(12, 4, 4096, False), (8, 2, 1024, True),
                                               (6, 3, 65536, False), (5, 1, 256, True),
                                               # misaligned units with full tiles: the
                                               # realigning fast path
                                               (12, 4, 4096, True), (8, 2, 16384, True),
                                               (6, 3, 65536, True), (3, 2, 32768, True)])
def test_batched_encode_matches_oracle(pkg, dev, k, m, unit, misalign):
    rng = np.random.default_rng(k * 7 + unit)
    host, tensors = _ragged_device(rng, dev, 40, 6 * unit, misalign)
    layout = pkg.StripeLayout(tensors, k, m, unit)
    par = layout.encode()
    torch.cuda.synchronize()
    assert np.array_equal(par.cpu().numpy(), _oracle_layout_parity(layout, host, unit))


@pytest.mark.parametrize("k,m,unit,lost", [
    (12, 4, 4096, (0,)), (12, 4, 4096, (3, 13)), (12, 4, 4096, (0, 5, 12, 15)),
    (12, 4, 4096, (12, 13, 14, 15)), (12, 4, 4096, (1, 2, 3, 4)),
    # k <= 8 runs four chunks per lane (16 KiB tiles): units shorter and
    # longer than one tile
    (8, 2, 4096, (0, 9)), (8, 2, 40960, (3, 7)), (6, 3, 65536, (0, 4, 7)), (5, 1, 1024, (2,))])
def test_batched_decode_round_trip(pkg, dev, k, m, unit, lost):
    rng = np.random.default_rng(sum(lost) + 100 * k + unit)
    host, tensors = _ragged_device(rng, dev, 50, 5 * unit, misalign=True)
    pset = pkg.encode(tensors, k, m, unit)
    par_ref = pset.parity.clone()
    # Erase: overwrite the lost positions of every stripe with junk.
    for s in range(pset.layout.n_stripes):
        for pos in lost:
            u = s * k + pos
            if pos < k and u < pset.layout.n_units:
                pset.layout.unit_view(u).fill_(0xA5)
            elif pos >= k:
                pset.parity[s, pos - k].fill_(0x5A)
    pkg.decode(pset, lost)
    torch.cuda.synchronize()
    for h, t in zip(host, tensors):
        assert np.array_equal(t.cpu().numpy(), h)
    assert torch.equal(pset.parity, par_ref)


def test_manager_default_code_every_erasure_pattern(pkg, dev):
    """The checkpoint manager's default code and unit (RS(4,2), 4 MiB units:
    the 2-slice grid order) over ragged tensors at odd offsets of an arena
    filled with 0xC3: the encode against the oracle, then every pattern of
    one or two lost positions erased (junk written over them) and decoded
    back, the other bytes of the arena untouched."""
    k, m, unit = 4, 2, 4 << 20
    rng = np.random.default_rng(42)
    host, tensors = _ragged_device(rng, dev, 9, 3 * unit + 777, misalign=True)
    pset = pkg.encode(tensors, k, m, unit)
    lay = pset.layout
    torch.cuda.synchronize()
    assert np.array_equal(pset.parity.cpu().numpy(), _oracle_layout_parity(lay, host, unit))
    par_ref = pset.parity.clone()
    arena = tensors[0]._base if tensors[0]._base is not None else None
    arena_ref = arena.clone() if arena is not None else None
    patterns = [(p,) for p in range(k + m)] + list(itertools.combinations(range(k + m), 2))
    for lost in patterns:
        for s in range(lay.n_stripes):
            for pos in lost:
                u = s * k + pos
                if pos < k and u < lay.n_units:
                    lay.unit_view(u).fill_(0xA5)
                elif pos >= k:
                    pset.parity[s, pos - k].fill_(0x5A)
        pkg.decode(pset, list(lost))
        torch.cuda.synchronize()
        assert torch.equal(pset.parity, par_ref), lost
        if arena is not None:
            assert torch.equal(arena, arena_ref), lost
        else:
            for h, t in zip(host, tensors):
                assert np.array_equal(t.cpu().numpy(), h), lost


def test_batched_decode_stripe_subset(pkg, dev):
    """Decoding a subset of stripes rebuilds exactly those stripes; stripe
    indices are checked on the host."""
    k, m, unit = 8, 2, 8192
    rng = np.random.default_rng(5)
    host, tensors = _ragged_device(rng, dev, 30, 6 * unit)
    pset = pkg.encode(tensors, k, m, unit)
    lay = pset.layout
    assert lay.n_stripes >= 4
    pick = [0, 2, lay.n_stripes - 1]
    for s in range(lay.n_stripes):
        u = s * k + 1
        if u < lay.n_units:
            lay.unit_view(u).fill_(0xA5)
    lay.decode(pset.parity, [1], stripes=pick)
    torch.cuda.synchronize()
    for s in range(lay.n_stripes):
        u = s * k + 1
        if u >= lay.n_units:
            continue
        t, i = int(lay.unit_tensor[u]), int(lay.unit_index[u])
        want = host[t].reshape(-1).view(np.uint8)[i * unit: i * unit + int(lay.host_len[s, 1])]
        got = lay.unit_view(u).cpu().numpy()
        if s in pick:
            assert np.array_equal(got, want), s
        else:
            assert (got == 0xA5).all(), s
    for bad in ([lay.n_stripes], [-1], [0, 0]):
        with pytest.raises(ValueError):
            lay.plan_decode(pset.parity, [1], stripes=bad)
    assert lay.plan_decode(pset.parity, [1], stripes=[]) is None


@pytest.mark.parametrize("k,m,unit,misalign,lost", [
    ((6, 3, (2 << 20) + 1024, False, (0, 4, 7))),   # 2049 tiles a unit: spans not a multiple of 8
    ((12, 4, (2 << 20) + 16, True, (1, 12))),       # realigned inputs, a 16-byte tail tile
    ((8, 2, 4 << 20, True, (3, 9))),
    ((4, 2, (8 << 20) + 4096, False, (1, 4)))])     # 8 slices for the encode and decode too
def test_batched_sliced_order(pkg, dev, k, m, unit, misalign, lost):
    """Units of 2 MiB and more are walked in interleaved slices of the grid
    (2 slices for an encode or decode over units below 8 MiB, else 8; the
    copying encode in 8), rounded up to whole slices; the workgroups past
    the last span do nothing.  The encode equals the oracle's, the copying
    encode into a stripe-major block writes the same parity and zero-padded
    copies, and lost positions decode back."""
    from megatron_lm_amd import _lib
    from megatron_lm_amd.checkpoint import GpuSliceCodec
    rng = np.random.default_rng(unit + k)
    host, tensors = _ragged_device(rng, dev, 7, 5 * unit, misalign)
    lay = pkg.StripeLayout(tensors, k, m, unit)
    par = lay.encode()
    torch.cuda.synchronize()
    want_par = _oracle_layout_parity(lay, host, unit)
    assert np.array_equal(par.cpu().numpy(), want_par)
    S = lay.n_stripes
    block = torch.full((S, k + m, unit), 0xC3, dtype=torch.uint8, device=dev)
    pp, cp = GpuSliceCodec._unit_ptrs(block, k, m), GpuSliceCodec._unit_ptrs(block, 0, k)
    _lib.check(_lib.lib().ec_encode_batched_copy(
        _lib.u8ptr(lay.coeff), k, m, lay.d_ptrs.data_ptr(), lay.d_len.data_ptr(),
        pp.data_ptr(), cp.data_ptr(), S, unit, None), "ec_encode_batched_copy")
    torch.cuda.synchronize()
    got = block.cpu().numpy()
    del block
    assert np.array_equal(got[:, k:], want_par)
    for s in range(S):
        for j in range(k):
            u = s * k + j
            want = np.zeros(unit, np.uint8)
            if u < lay.n_units:
                t, i = int(lay.unit_tensor[u]), int(lay.unit_index[u])
                piece = host[t][i * unit: (i + 1) * unit]
                want[: piece.size] = piece
            assert np.array_equal(got[s, j], want), (s, j)
    del got
    for s in range(S):
        for pos in lost:
            u = s * k + pos
            if pos < k and u < lay.n_units:
                lay.unit_view(u).fill_(0xA5)
            elif pos >= k:
                par[s, pos - k].fill_(0x5A)
    lay.decode(par, list(lost))
    torch.cuda.synchronize()
    for h, t in zip(host, tensors):
        assert np.array_equal(t.cpu().numpy(), h)
    assert np.array_equal(par.cpu().numpy(), want_par)


def _padded_flat_parity(pkg, lay, s):
    """Parity of stripe s by the flat kernel over zero-padded copies of its
    units (absent units are zeros)."""
    unit = lay.unit_bytes
    shards = []
    for j in range(lay.k):
        pad = torch.zeros(unit, dtype=torch.uint8, device=lay.device)
        u = s * lay.k + j
        if u < lay.n_units:
            v = lay.unit_view(u)
            pad[: v.numel()].copy_(v)
        shards.append(pad)
    return torch.stack(pkg.rs_encode(shards, lay.m, coeff=lay.coeff))


@pytest.mark.parametrize("unit,offsets", [
    (2 << 20, (0,)),                       # aligned: the full-tile kernel and the rest
    ((4 << 20) + 1024, (0, 16)),           # 4097 tiles a unit, views 16 bytes in
    (8 << 20, (0, 16, 5)),                 # aligned and misaligned stripes in one launch
    ((16 << 20) - 16, (0,))])              # the largest split unit, a short last tile
def test_batched_full_and_rest_kernels(pkg, dev, unit, offsets):
    """RS(8,2) over units of 2 to 16 MiB runs as two kernels: one codes the
    tiles where every unit and output is whole or already ended, the other
    the tiles that hold a unit's end, the outputs' short tails and every tile
    of a stripe with a misaligned address.  Tensors end on tile boundaries,
    inside tiles, on unit boundaries and one byte in; the last stripe has
    absent units.  The parity equals the flat kernel's over zero-padded units
    (and the oracle's at 2 MiB), and two lost positions (two data units; a
    data unit and a parity) decode back through the same split."""
    k, m = 8, 2
    sizes = [3 * unit, 2 * unit + 1024 * 37, unit + 777, 5 * unit - 16, 4096, 1,
             2 * unit + 3000, unit - 1024 * 5]
    g = torch.Generator(device=dev)
    g.manual_seed(unit)
    tensors = []
    for i, n in enumerate(sizes):
        off = offsets[i % len(offsets)]
        buf = torch.empty(n + off, dtype=torch.uint8, device=dev)
        v = buf[off:]
        v.copy_(torch.randint(0, 256, (n,), dtype=torch.uint8, device=dev, generator=g))
        tensors.append(v)
    keep = [t.clone() for t in tensors]
    lay = pkg.StripeLayout(tensors, k, m, unit)
    assert lay.n_units % k != 0   # the last stripe has absent units
    par = lay.encode()
    for s in range(lay.n_stripes):
        assert torch.equal(par[s], _padded_flat_parity(pkg, lay, s)), s
    if unit == 2 << 20:
        torch.cuda.synchronize()
        host = [t.cpu().numpy() for t in tensors]
        assert np.array_equal(par.cpu().numpy(), _oracle_layout_parity(lay, host, unit))
    par_ref = par.clone()
    for lost in ((2, 7), (1, 9)):
        for s in range(lay.n_stripes):
            for pos in lost:
                u = s * k + pos
                if pos < k and u < lay.n_units:
                    lay.unit_view(u).fill_(0xA5)
                elif pos >= k:
                    par[s, pos - k].fill_(0x5A)
        lay.decode(par, list(lost))
        torch.cuda.synchronize()
        for t, want in zip(tensors, keep):
            assert torch.equal(t, want), lost
        assert torch.equal(par, par_ref), lost


@pytest.mark.parametrize("seed", range(16))
def test_batched_full_and_rest_random(pkg, dev, seed):
    """Seeded random RS(8,2) layouts on the two-kernel launch: a unit size
    anywhere from 2 MiB to 16 MiB - 16 B in 16-byte steps (tiles end anywhere
    inside a unit), 2 to 9 tensors of 1 byte to 3 units at offsets of 0, 16,
    48 bytes or an odd one from 256-byte boundaries of one arena, with 4 KiB
    of 0xC3 between them.  The parity equals the flat kernel's over
    zero-padded units (a kernel reading past a unit's end would fold the
    0xC3 bytes in), and two random lost positions decode back with every
    byte of the arena, the gaps included, as before."""
    k, m = 8, 2
    r = np.random.default_rng(1000 + seed)
    unit = 16 * int(r.integers((2 << 20) // 16, (16 << 20) // 16))
    n_tensors = int(r.integers(2, 10))
    sizes = [int(r.integers(1, 3 * unit)) for _ in range(n_tensors)]
    offs = [int(r.choice([0, 0, 16, 48, int(r.integers(1, 16))])) for _ in range(n_tensors)]
    starts, pos = [], 0
    for n, off in zip(sizes, offs):
        starts.append(pos + off)
        pos = (pos + off + n + 4096 + 255) // 256 * 256
    arena = torch.full((pos,), 0xC3, dtype=torch.uint8, device=dev)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    tensors = []
    for n, a in zip(sizes, starts):
        v = arena[a:a + n]
        v.copy_(torch.randint(0, 256, (n,), dtype=torch.uint8, device=dev, generator=g))
        tensors.append(v)
    arena_before = arena.clone()
    lay = pkg.StripeLayout(tensors, k, m, unit)
    par = lay.encode()
    for s in range(lay.n_stripes):
        assert torch.equal(par[s], _padded_flat_parity(pkg, lay, s)), (seed, unit, s)
    par_ref = par.clone()
    lost = sorted(int(x) for x in r.choice(k + m, 2, replace=False))
    for s in range(lay.n_stripes):
        for pos in lost:
            u = s * k + pos
            if pos < k and u < lay.n_units:
                lay.unit_view(u).fill_(0xA5)
            elif pos >= k:
                par[s, pos - k].fill_(0x5A)
    lay.decode(par, lost)
    torch.cuda.synchronize()
    assert torch.equal(arena, arena_before), (seed, unit, lost)
    assert torch.equal(par, par_ref), (seed, unit, lost)


@pytest.mark.parametrize("k,m,unit,misalign", [(12, 4, 2048, False), (6, 3, 20480, False),
                                                (12, 4, 4096, True), (8, 2, 16384, True)])
def test_batched_update_equals_reencode(pkg, dev, k, m, unit, misalign):
    rng = np.random.default_rng(77 + k)
    host, tensors = _ragged_device(rng, dev, 60, 8 * unit, misalign)
    pset = pkg.encode(tensors, k, m, unit)
    lay = pset.layout
    par0 = _oracle_layout_parity(lay, host, unit)
    changed = np.sort(rng.choice(lay.n_units, max(1, lay.n_units // 10), replace=False))
    olds, host_new = _perturb_units(rng, lay, host, changed)
    pkg.update(pset, changed, olds)
    fresh = lay.encode()
    torch.cuda.synchronize()
    want = _oracle_update(lay, host, host_new, changed, par0)
    assert np.array_equal(pset.parity.cpu().numpy(), want)
    assert np.array_equal(want, _oracle_layout_parity(lay, host_new, unit))
    assert torch.equal(pset.parity, fresh)


@pytest.mark.parametrize("k", [2, 9])
def test_batched_largest_unit(pkg, dev, k):
    """unit_bytes at its 2 GiB maximum (the kernels' 32-bit in-unit offsets
    end there), with the last unit ending 4103 bytes short of a tile
    boundary.  Checked by size-independent properties: the batched parity
    equals the flat kernel's over the zero-padded units (the flat kernel is
    checked against the oracle above), and a lost unit decodes back."""
    unit = 1 << 31
    m = 1
    n = (k - 1) * unit + unit - 4096 - 7
    g = torch.Generator(device=dev)
    g.manual_seed(11 + k)
    data = torch.randint(0, 256, (n,), dtype=torch.uint8, device=dev, generator=g)
    pset = pkg.encode([data], k, m, unit)
    lay = pset.layout
    assert lay.n_stripes == 1 and int(lay.host_len[0, k - 1]) == unit - 4096 - 7
    last = torch.zeros(unit, dtype=torch.uint8, device=dev)
    last[: n - (k - 1) * unit].copy_(data[(k - 1) * unit:])
    shards = [data[j * unit: (j + 1) * unit] for j in range(k - 1)] + [last]
    (flat,) = pkg.rs_encode(shards, m, coeff=lay.coeff)
    torch.cuda.synchronize()
    assert torch.equal(pset.parity[0, 0], flat)
    del flat, shards
    for lost in (0, k - 1):
        keep = lay.unit_view(lost).clone()
        lay.unit_view(lost).fill_(0xA5)
        pkg.decode(pset, [lost])
        torch.cuda.synchronize()
        assert torch.equal(lay.unit_view(lost), keep), lost
        del keep


def test_zero_byte_inputs(pkg, dev):
    """Empty shards are a no-op that succeeds; zero-length tensors in a ragged
    list own no unit and the rest codes as without them."""
    empty = [torch.empty(0, dtype=torch.uint8, device=dev) for _ in range(6)]
    par = pkg.rs_encode(empty, 3)
    assert all(p.numel() == 0 for p in par)
    assert pkg.xor_encode(empty[:4]).numel() == 0
    rec = pkg.reconstruct([None, None] + empty[2:] + [par[0], None, par[2]], 6, 3)
    torch.cuda.synchronize()
    assert sorted(rec) == [0, 1, 7] and all(t.numel() == 0 for t in rec.values())
    rng = np.random.default_rng(3)
    host = [rng.integers(0, 256, n, dtype=np.uint8) for n in (5000, 0, 70000, 0, 1, 0)]
    tensors = [torch.from_numpy(h).to(dev) for h in host]
    unit = 4096
    a = pkg.encode(tensors, 4, 2, unit)
    b = pkg.encode([t for t in tensors if t.numel()], 4, 2, unit)
    torch.cuda.synchronize()
    assert a.layout.n_units == b.layout.n_units and torch.equal(a.parity, b.parity)
    assert np.array_equal(a.parity.cpu().numpy(),
                          _oracle_layout_parity(a.layout, host, unit))


@pytest.mark.parametrize("n", [5, 31, 4096 + 7, 100_003])
@pytest.mark.parametrize("k,m", [(6, 3), (4, 1), (20, 6)])
def test_rs_encode_realigned_inputs(pkg, dev, k, m, n):
    """Inputs at every misalignment 0..15 with aligned outputs: the wide
    kernel's realigning loads (two aligned loads + v_alignbyte per shard)."""
    rng = np.random.default_rng(n + 31 * k)
    d = _host(rng, k, n)
    dd = [_to_dev([a], dev, j % 16)[0] for j, a in enumerate(d)]
    par = pkg.rs_encode(dd, m)
    for p, w in zip(par, oracle.rs_encode(oracle.cauchy(k, m), d)):
        assert _eq(p, w)
    x = pkg.xor_encode(dd)
    assert _eq(x, oracle.xor_encode(d))


@pytest.mark.parametrize("n", [1_000_001, 65_537])
def test_flat_buffer_cut_into_odd_shards(pkg, dev, n):
    """k shards cut from one flat buffer at multiples of an odd size (each at
    a different misalignment), encoded and then rebuilt after 3 losses."""
    k, m = 6, 3
    rng = np.random.default_rng(n)
    flat_h = rng.integers(0, 256, k * n, dtype=np.uint8)
    flat = torch.from_numpy(flat_h).to(dev)
    shards = [flat[j * n: (j + 1) * n] for j in range(k)]
    par = pkg.rs_encode(shards, m)
    d = [flat_h[j * n: (j + 1) * n] for j in range(k)]
    for p, w in zip(par, oracle.rs_encode(oracle.cauchy(k, m), d)):
        assert _eq(p, w)
    rec = pkg.reconstruct([None, shards[1], None, shards[3], shards[4], shards[5],
                           par[0], None, par[2]], k, m)
    assert _eq(rec[0], d[0]) and _eq(rec[2], d[2]) and _eq(rec[7], oracle.rs_encode(
        oracle.cauchy(k, m), d)[1])


@pytest.mark.parametrize("k,m,unit,lost", [(20, 6, 4096, (0, 5, 19, 20, 23, 25)),
                                           (5, 9, 1024, (1, 2, 6, 13)),
                                           (32, 16, 8192, (0, 31, 32, 47))])
def test_batched_wide_codes(pkg, dev, k, m, unit, lost):
    """Batched encode, decode and update for codes past the fixed-size
    kernels, on ragged and misaligned tensor lists, against the oracle."""
    rng = np.random.default_rng(k * 100 + m)
    host, tensors = _ragged_device(rng, dev, 3 * k, 3 * unit, misalign=(k == 5))
    pset = pkg.encode(tensors, k, m, unit)
    torch.cuda.synchronize()
    assert np.array_equal(pset.parity.cpu().numpy(), _oracle_layout_parity(pset.layout, host, unit))
    lay = pset.layout
    par_ref = pset.parity.clone()
    for s in range(lay.n_stripes):
        for pos in lost:
            u = s * k + pos
            if pos < k and u < lay.n_units:
                lay.unit_view(u).fill_(0xA5)
            elif pos >= k:
                pset.parity[s, pos - k].fill_(0x5A)
    pkg.decode(pset, lost)
    torch.cuda.synchronize()
    for h, t in zip(host, tensors):
        assert np.array_equal(t.cpu().numpy(), h)
    assert torch.equal(pset.parity, par_ref)
    changed = np.sort(rng.choice(lay.n_units, max(1, lay.n_units // 7), replace=False))
    par0 = pset.parity.cpu().numpy()   # equal to the oracle's parity (checked above)
    olds, host_new = _perturb_units(rng, lay, host, changed)
    pkg.update(pset, changed, olds)
    fresh = lay.encode()
    torch.cuda.synchronize()
    assert np.array_equal(pset.parity.cpu().numpy(),
                          _oracle_update(lay, host, host_new, changed, par0))
    assert torch.equal(pset.parity, fresh)


@pytest.mark.parametrize("k,m,unit,misalign", [(12, 4, 4096, False), (6, 3, 16384, False),
                                               (8, 2, 16384, True), (5, 1, 256, True),
                                               (3, 2, 4112, False), (20, 6, 2048, True)])
def test_encode_batched_copy(pkg, dev, k, m, unit, misalign):
    """ec_encode_batched_copy: the parity equals the oracle's, and every data
    unit lands zero-padded at its copy address; units with a 0 copy address
    are skipped (their bytes keep a canary).  Covers the 16 KiB tiles
    (k <= 8, unit a multiple of 16 KiB), 4 KiB tiles, units shorter than a
    tile, realigned inputs, a unit size off the tile grid, and a wide code
    (two launches)."""
    from megatron_lm_amd import _lib
    rng = np.random.default_rng(k * 31 + unit)
    host, tensors = _ragged_device(rng, dev, 30, 5 * unit, misalign)
    lay = pkg.StripeLayout(tensors, k, m, unit)
    S = lay.n_stripes
    block = torch.full((k + m, S, unit), 0xC3, dtype=torch.uint8, device=dev)
    base = np.uint64(block.data_ptr())
    rows = np.arange(S, dtype=np.uint64)[:, None]
    pp = base + ((np.arange(m, dtype=np.uint64)[None, :] + np.uint64(k)) * np.uint64(S) + rows) \
        * np.uint64(unit)
    cp = base + (np.arange(k, dtype=np.uint64)[None, :] * np.uint64(S) + rows) * np.uint64(unit)
    skip = np.zeros((S, k), bool)
    skip[::3, 1 % k] = True                 # some units are not copied
    cp[skip] = 0
    d_pp = torch.from_numpy(pp.view(np.int64)).to(dev)
    d_cp = torch.from_numpy(np.ascontiguousarray(cp).view(np.int64)).to(dev)
    _lib.check(_lib.lib().ec_encode_batched_copy(
        _lib.u8ptr(lay.coeff), k, m, lay.d_ptrs.data_ptr(), lay.d_len.data_ptr(),
        d_pp.data_ptr(), d_cp.data_ptr(), S, unit, None), "ec_encode_batched_copy")
    torch.cuda.synchronize()
    got = block.cpu().numpy()
    want_par = _oracle_layout_parity(lay, host, unit)        # [S, m, unit]
    assert np.array_equal(got[k:].transpose(1, 0, 2), want_par)
    for s in range(S):
        for j in range(k):
            u = s * k + j
            if skip[s, j]:
                assert (got[j, s] == 0xC3).all(), (s, j)
                continue
            want = np.zeros(unit, np.uint8)
            if u < lay.n_units:
                t, i = int(lay.unit_tensor[u]), int(lay.unit_index[u])
                piece = host[t][i * unit: (i + 1) * unit]
                want[: piece.size] = piece
            assert np.array_equal(got[j, s], want), (s, j)


@pytest.mark.parametrize("unit", [4096, 16384])
def test_encode_batched_copy_every_instantiated_shape(pkg, dev, unit):
    """Every fixed-size (k, m) of the copying encode, with 4 KiB tiles and,
    for k <= 8 and 16 KiB units, 16 KiB tiles: parity against the oracle and
    the data rows against the zero-padded units."""
    from megatron_lm_amd import _lib
    rng = np.random.default_rng(unit)
    for k in range(1, 17):
        host, tensors = _ragged_device(rng, dev, k + 3, 3 * unit)
        for m in range(1, 5):
            lay = pkg.StripeLayout(tensors, k, m, unit)
            S = lay.n_stripes
            block = torch.empty((k + m, S, unit), dtype=torch.uint8, device=dev)
            base = np.uint64(block.data_ptr())
            rows = np.arange(S, dtype=np.uint64)[:, None] * np.uint64(unit)
            pp = base + (np.arange(k, k + m, dtype=np.uint64)[None, :] * np.uint64(S * unit)) + rows
            cp = base + (np.arange(k, dtype=np.uint64)[None, :] * np.uint64(S * unit)) + rows
            d_pp = torch.from_numpy(np.ascontiguousarray(pp).view(np.int64)).to(dev)
            d_cp = torch.from_numpy(np.ascontiguousarray(cp).view(np.int64)).to(dev)
            _lib.check(_lib.lib().ec_encode_batched_copy(
                _lib.u8ptr(lay.coeff), k, m, lay.d_ptrs.data_ptr(), lay.d_len.data_ptr(),
                d_pp.data_ptr(), d_cp.data_ptr(), S, unit, None), "ec_encode_batched_copy")
            torch.cuda.synchronize()
            got = block.cpu().numpy()
            assert np.array_equal(got[k:].transpose(1, 0, 2),
                                  _oracle_layout_parity(lay, host, unit)), (k, m)
            stream = np.zeros(S * k * unit, np.uint8)
            for u in range(lay.n_units):
                t, i = int(lay.unit_tensor[u]), int(lay.unit_index[u])
                piece = host[t][i * unit: (i + 1) * unit]
                stream[u * unit: u * unit + piece.size] = piece
            assert np.array_equal(got[:k].transpose(1, 0, 2).reshape(-1), stream), (k, m)


@pytest.mark.parametrize("rows,row_bytes,pitch,pinned,threads,pageable", [
    (16, (1 << 20) + 48, (1 << 20) + 64, 1 << 20, 8, False),   # many chunks, a short last one
    (3, 5000, 5000, 64, 1, False),                             # chunks narrower than a page
    (1, 4096, 8192, 1 << 16, 64, False),                       # one row, more threads than bytes/64
    (5, 70000, 70016, 1 << 16, 4, True),                       # HIP transfers: pageable "pinned"
])
def test_stage_to_host(pkg, dev, rows, row_bytes, pitch, pinned, threads, pageable):
    """ec_stage_to_host copies a pitched device region into pageable host
    memory exactly, through a pinned buffer smaller than the region, after
    the work already on the stream: on a copy engine with a pinned buffer,
    with HIP transfers when the buffer is memory the runtime did not
    allocate."""
    from megatron_lm_amd import _lib
    g = torch.Generator(device=dev)
    g.manual_seed(rows)
    src = torch.randint(0, 256, (rows, pitch), dtype=torch.uint8, device=dev, generator=g)
    out = np.full((rows, pitch + 16), 0x77, np.uint8)
    pin = np.empty(pinned, np.uint8) if pageable else torch.empty(pinned, dtype=torch.uint8,
                                                                  pin_memory=True)
    pin_ptr = pin.ctypes.data if pageable else pin.data_ptr()
    src.add_(1)   # enqueued before the call: the copy must see it
    _lib.check(_lib.lib().ec_stage_to_host(
        src.data_ptr(), pitch, out.ctypes.data, pitch + 16, rows, row_bytes, pin_ptr,
        pinned, threads, None), "ec_stage_to_host")
    assert _lib.last_stage_stats()["copy_engine"] == (0 if pageable else 1)
    want = src.cpu().numpy()
    assert np.array_equal(out[:, :row_bytes], want[:, :row_bytes])
    assert (out[:, row_bytes:] == 0x77).all()


@pytest.mark.parametrize("stripes,positions,unit,pinned,threads", [
    (300, 16, 4096 + 48, 1 << 20, 8),     # chunks end inside units, a short last one
    (5, 3, 5000, 64, 1),                  # chunks narrower than a unit and a page
    (40, 10, 1 << 16, 64 << 20, 64),      # one chunk for the whole block
    (2, 1, 7, 4096, 3),                   # one position: a plain copy
])
def test_stage_stripes_to_host(pkg, dev, stripes, positions, unit, pinned, threads):
    """ec_stage_stripes_to_host moves a stripe-major (stripes, positions,
    unit) device block into one pageable host row per position, exactly:
    row p is unit (s, p) for s = 0, 1, ..., back to back, and nothing past
    a row's end is written.  The copy follows the work already on the
    stream."""
    from megatron_lm_amd import _lib
    g = torch.Generator(device=dev)
    g.manual_seed(stripes)
    block = torch.randint(0, 256, (stripes, positions, unit), dtype=torch.uint8, device=dev,
                          generator=g)
    rows = [np.full(stripes * unit + 16, 0x77, np.uint8) for _ in range(positions)]
    pin = torch.empty(pinned, dtype=torch.uint8, pin_memory=True)
    block.add_(1)   # enqueued before the call: the copy must see it
    _lib.check(_lib.lib().ec_stage_stripes_to_host(
        block.data_ptr(), stripes, positions, unit, _lib.ptr_array([r.ctypes.data for r in rows]),
        pin.data_ptr(), pinned, threads, None), "ec_stage_stripes_to_host")
    st = _lib.last_stage_stats()
    want = block.cpu().numpy()
    for p in range(positions):
        assert np.array_equal(rows[p][:stripes * unit], want[:, p, :].reshape(-1)), p
        assert (rows[p][stripes * unit:] == 0x77).all(), p
    # the call's timings: one transfer per pinned half (whole pages when the
    # half holds at least one) of the block
    total = stripes * positions * unit
    half = pinned // 2
    half = min(half - half % 4096 if half >= 4096 else half, total)
    assert st["chunks"] == -(-total // half)
    assert 0 <= st["device_s"] <= st["wall_s"] and 0 <= st["wait_s"] <= st["wall_s"]
    if total >= 1 << 20:   # long enough for the timing events to tell apart
        assert st["device_s"] > 0
    assert 0 <= st["host_copy_s"] <= st["wall_s"] and st["max_wait_s"] <= st["wait_s"]
    assert st["copy_engine"] == 1   # runtime-allocated block and pinned buffer


def test_stage_stripes_to_host_odd_addresses(pkg, dev):
    """The copy-engine path with a block and a pinned buffer at odd
    addresses inside larger allocations, odd units and an odd pinned size
    (halves of 500 bytes): every byte lands in its row, nothing past a row's
    end is written."""
    from megatron_lm_amd import _lib
    stripes, positions, unit = 37, 5, 1001
    total = stripes * positions * unit
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    big = torch.randint(0, 256, (total + 64,), dtype=torch.uint8, device=dev, generator=g)
    block = big[5: 5 + total]
    rows = [np.full(stripes * unit + 16, 0x77, np.uint8) for _ in range(positions)]
    pin = torch.empty(1024, dtype=torch.uint8, pin_memory=True)
    _lib.check(_lib.lib().ec_stage_stripes_to_host(
        block.data_ptr(), stripes, positions, unit, _lib.ptr_array([r.ctypes.data for r in rows]),
        pin.data_ptr() + 3, 1001, 2, None), "ec_stage_stripes_to_host")
    st = _lib.last_stage_stats()
    assert st["copy_engine"] == 1 and st["chunks"] == -(-total // 500)
    want = block.cpu().numpy().reshape(stripes, positions, unit)
    for p in range(positions):
        assert np.array_equal(rows[p][:stripes * unit], want[:, p, :].reshape(-1)), p
        assert (rows[p][stripes * unit:] == 0x77).all(), p


@pytest.mark.parametrize("seed", range(6))
def test_staging_random_shapes(pkg, dev, seed):
    """Both device-to-host calls over seeded random shapes: block and region
    at random byte offsets inside larger allocations, random units, pitches,
    pinned sizes (halves from a few bytes to whole pages) and thread counts,
    pinned or pageable buffers; every byte lands where it belongs and
    nothing past a row's end is written."""
    from megatron_lm_amd import _lib
    rng = np.random.default_rng(100 + seed)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    stripes, positions = int(rng.integers(1, 40)), int(rng.integers(1, 17))
    unit = int(rng.integers(1, 70000))
    total = stripes * positions * unit
    off = int(rng.integers(0, 64))
    big = torch.randint(0, 256, (total + off + 64,), dtype=torch.uint8, device=dev, generator=g)
    block = big[off: off + total]
    pinned = int(rng.choice([int(rng.integers(2, 5000)), int(rng.integers(8192, 1 << 21))]))
    pageable = bool(rng.integers(0, 2))
    pin = np.empty(pinned + 7, np.uint8) if pageable else torch.empty(pinned + 7, dtype=torch.uint8,
                                                                      pin_memory=True)
    pin_ptr = (pin.ctypes.data if pageable else pin.data_ptr()) + int(rng.integers(0, 8))
    threads = int(rng.integers(1, 9))
    rows = [np.full(stripes * unit + 16, 0x77, np.uint8) for _ in range(positions)]
    _lib.check(_lib.lib().ec_stage_stripes_to_host(
        block.data_ptr(), stripes, positions, unit, _lib.ptr_array([r.ctypes.data for r in rows]),
        pin_ptr, pinned, threads, None), "ec_stage_stripes_to_host")
    assert _lib.last_stage_stats()["copy_engine"] == (0 if pageable else 1)
    want = block.cpu().numpy().reshape(stripes, positions, unit)
    for p in range(positions):
        assert np.array_equal(rows[p][:stripes * unit], want[:, p, :].reshape(-1)), (seed, p)
        assert (rows[p][stripes * unit:] == 0x77).all(), (seed, p)
    # the same bytes as a pitched region: rows of row_bytes at a pitch of one
    # unit (a pinned half holds at least one byte of every row)
    n_rows = max(1, min(positions * stripes, int(rng.integers(1, 12)), pinned // 2))
    row_bytes = int(rng.integers(1, unit + 1))
    out = np.full((n_rows, row_bytes + 16), 0x77, np.uint8)
    _lib.check(_lib.lib().ec_stage_to_host(
        block.data_ptr(), unit, out.ctypes.data, row_bytes + 16, n_rows, row_bytes, pin_ptr,
        pinned, threads, None), "ec_stage_to_host")
    assert _lib.last_stage_stats()["copy_engine"] == (0 if pageable else 1)
    flat = block.cpu().numpy()
    for r in range(n_rows):
        assert np.array_equal(out[r, :row_bytes], flat[r * unit: r * unit + row_bytes]), (seed, r)
        assert (out[r, row_bytes:] == 0x77).all(), (seed, r)


@pytest.mark.parametrize("pageable", [False, True])
def test_stage_stripes_to_host_follows_its_stream(pkg, dev, pageable):
    """ec_stage_stripes_to_host after work on a stream other than torch's:
    the bytes staged are those that work left.  With a pinned buffer the
    copies run on an SDMA engine once the stream's work is done; with a
    pageable one (memory the runtime did not allocate) they fall back to
    HIP transfers on the stream.  Both give the rows exactly."""
    from megatron_lm_amd import _lib
    from megatron_lm_amd.codec import stream_handle
    stripes, positions, unit, pinned = 257, 6, 12288 + 16, 3 << 20
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    block = torch.randint(0, 256, (stripes, positions, unit), dtype=torch.uint8, device=dev,
                          generator=g)
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        for _ in range(32):   # queued work the copy must wait for
            block.add_(3)
    rows = [np.full(stripes * unit, 0x77, np.uint8) for _ in range(positions)]
    if pageable:
        pin_buf = np.empty(pinned, np.uint8)
        pin_ptr = pin_buf.ctypes.data
    else:
        pin_buf = torch.empty(pinned, dtype=torch.uint8, pin_memory=True)
        pin_ptr = pin_buf.data_ptr()
    _lib.check(_lib.lib().ec_stage_stripes_to_host(
        block.data_ptr(), stripes, positions, unit, _lib.ptr_array([r.ctypes.data for r in rows]),
        pin_ptr, pinned, 4, stream_handle(side, dev)), "ec_stage_stripes_to_host")
    st = _lib.last_stage_stats()
    assert st["copy_engine"] == (0 if pageable else 1)
    side.synchronize()
    want = block.cpu().numpy()
    for p in range(positions):
        assert np.array_equal(rows[p], want[:, p, :].reshape(-1)), p


@pytest.mark.parametrize("rows,row_bytes,pitch,pinned,threads", [
    (12, (1 << 20) + 48, (1 << 20) + 64, 1 << 20, 8),
    (3, 5000, 5008, 64, 1),
    (1, 4096, 8192, 1 << 16, 64),
])
def test_stage_to_device(pkg, dev, rows, row_bytes, pitch, pinned, threads):
    """ec_stage_to_device copies separate pageable host rows into a pitched
    device region exactly, through a pinned buffer smaller than the region,
    and leaves the bytes between rows alone."""
    from megatron_lm_amd import _lib
    rng = np.random.default_rng(rows)
    host = [rng.integers(0, 256, row_bytes, dtype=np.uint8) for _ in range(rows)]
    dst = torch.full((rows, pitch), 0x5A, dtype=torch.uint8, device=dev)
    pin = torch.empty(pinned, dtype=torch.uint8, pin_memory=True)
    _lib.check(_lib.lib().ec_stage_to_device(
        _lib.ptr_array([h.ctypes.data for h in host]), rows, row_bytes, dst.data_ptr(), pitch,
        pin.data_ptr(), pinned, threads, None), "ec_stage_to_device")
    got = dst.cpu().numpy()
    for r in range(rows):
        assert np.array_equal(got[r, :row_bytes], host[r]), r
        assert (got[r, row_bytes:] == 0x5A).all(), r


@pytest.mark.parametrize("n,offset", [((1 << 20) + 5, 0), (4096 * 3 + 7, 3)])
def test_shard_plan_matches_oracle(pkg, dev, n, offset):
    """ShardPlan (a flat call prepared once): RS(6,3) encode, a 3-erasure
    decode and XOR(4), each launched twice on torch's stream and once on
    another stream, byte-equal to the oracle; a second launch after the
    inputs changed codes the new bytes."""
    rng = np.random.default_rng(n)
    d = _host(rng, 6, n)
    dd = _to_dev(d, dev, offset)
    C = oracle.cauchy(6, 3)
    enc = pkg.ShardPlan(C, dd)
    for _ in range(2):
        par = enc()
        for p, w in zip(par, oracle.rs_encode(C, d)):
            assert _eq(p, w)
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    for t in par:
        t.zero_()
    side.wait_stream(torch.cuda.current_stream(dev))
    enc(stream=side)
    side.synchronize()
    for p, w in zip(par, oracle.rs_encode(C, d)):
        assert _eq(p, w)
    lost = [1, 4, 7]
    surv, rows = pkg.decode_matrix(C, lost)
    cw = dd + par
    dec = pkg.ShardPlan(rows, [cw[s] for s in surv], what="ec_rs_decode")
    for r, g in zip(dec(), lost):
        assert _eq(r, d[g] if g < 6 else oracle.rs_encode(C, d)[g - 6])
    xp = pkg.ShardPlan(None, dd[:4], what="ec_xor_encode")
    assert _eq(xp()[0], oracle.xor_encode(d[:4]))
    d2 = _host(rng, 6, n)
    for t, a in zip(dd, d2):
        t.copy_(torch.from_numpy(a))
    assert _eq(xp()[0], oracle.xor_encode(d2[:4]))
    for p, w in zip(enc(), oracle.rs_encode(C, d2)):
        assert _eq(p, w)


def test_eager_binding_streams_and_operand_checks(pkg, dev):
    """The eager flat calls (the torch-tensor binding): outputs allocated or
    given, torch's current stream inside a stream context or an explicit
    stream, byte-equal to the oracle; operands on the wrong device kind,
    non-contiguous or of unequal size are refused before any launch."""
    rng = np.random.default_rng(11)
    n = (1 << 18) + 3
    d = _host(rng, 6, n)
    dd = _to_dev(d, dev)
    C = oracle.cauchy(6, 3)
    want = oracle.rs_encode(C, d)
    torch.cuda.synchronize()
    side = torch.cuda.Stream(dev)
    with torch.cuda.stream(side):
        assert pkg._lib.shards().current_stream(dev.index) == side.cuda_stream
        par = pkg.rs_encode(dd, 3)
        out = [torch.full((n,), 7, dtype=torch.uint8, device=dev) for _ in range(3)]
        pkg.matvec(C, dd, out=out)
        x = pkg.xor_encode(dd[:5])
    assert pkg._lib.shards().current_stream(dev.index) == \
        torch.cuda.current_stream(dev).cuda_stream
    side.synchronize()
    for a, b, w in zip(par, out, want):
        assert np.array_equal(a.cpu().numpy(), w)
        assert np.array_equal(b.cpu().numpy(), w)
    assert np.array_equal(x.cpu().numpy(), oracle.xor_encode(d[:5]))
    for t in out:
        t.zero_()
    torch.cuda.synchronize()
    pkg.rs_encode(dd, 3, out=out, stream=side)
    par2 = pkg.rs_encode(dd, 3, stream=side)  # allocated on torch's stream, written on side
    side.synchronize()
    for b, c, w in zip(out, par2, want):
        assert np.array_equal(b.cpu().numpy(), w)
        assert np.array_equal(c.cpu().numpy(), w)
    rec = pkg.reconstruct([None if g in (0, 5, 8) else t for g, t in enumerate(dd + out)], 6, 3)
    torch.cuda.synchronize()
    assert np.array_equal(rec[0].cpu().numpy(), d[0])
    assert np.array_equal(rec[5].cpu().numpy(), d[5])
    assert np.array_equal(rec[8].cpu().numpy(), want[2])
    bad = [
        dd[:5] + [torch.from_numpy(d[5])],                          # a host tensor
        dd[:5] + [torch.empty(2 * n, dtype=torch.uint8, device=dev)[::2]],  # strided
        dd[:5] + [torch.empty(n + 1, dtype=torch.uint8, device=dev)],       # one byte more
    ]
    for shards in bad:
        with pytest.raises(ValueError):
            pkg.rs_encode(shards, 3)
    with pytest.raises(ValueError):
        pkg.matvec(C, dd, out=out[:2])
    with pytest.raises(ValueError):
        pkg.matvec(C, dd, out=out[:2] + [torch.empty(n - 1, dtype=torch.uint8, device=dev)])
    with pytest.raises(ValueError):
        pkg.xor_encode(dd, out=torch.empty(n, dtype=torch.uint8))
    with pytest.raises(TypeError):
        pkg.rs_encode(dd[:5] + [d[5]], 3)


def test_shard_plan_outputs_held_for_a_launch_on_another_stream(pkg, dev):
    """A ShardPlan whose outputs it allocated (on torch's current stream)
    and that launches on another stream, given to the plan or to the call:
    dropped right after the launch, while that stream still has the launch
    queued behind a long wait, its outputs' memory is not handed out again
    (record_stream), and the launch writes the oracle's bytes."""
    rng = np.random.default_rng(12)
    n = 1 << 20
    d = _host(rng, 6, n)
    dd = _to_dev(d, dev)
    C = oracle.cauchy(6, 3)
    want = oracle.rs_encode(C, d)
    torch.cuda.synchronize()
    for how in ("plan", "call"):
        side = torch.cuda.Stream(dev)
        plan = pkg.ShardPlan(C, dd, stream=side) if how == "plan" else pkg.ShardPlan(C, dd)
        ptrs = {t.data_ptr() for t in plan.outputs}
        with torch.cuda.stream(side):
            torch.cuda._sleep(50_000_000)   # tens of milliseconds of GPU time on side
        outs = plan() if how == "plan" else plan(stream=side)
        side_done = torch.cuda.Event()
        with torch.cuda.stream(side):   # read the outputs on side, after the launch
            copies = [t.clone() for t in outs]
            side_done.record(side)
        del plan, outs
        fresh = [torch.empty(n, dtype=torch.uint8, device=dev) for _ in range(3)]
        assert not ptrs & {t.data_ptr() for t in fresh}, how
        for t in fresh:
            t.fill_(0xEE)
        side_done.synchronize()
        for c, w in zip(copies, want):
            assert np.array_equal(c.cpu().numpy(), w), how
        del fresh, copies


def test_flat_kernels_past_the_grid_cap(pkg, dev):
    """Shards of 16 GiB + 4 KiB + 48 B: more 16-byte chunks than the flat
    kernels' one-pass grid covers (2^24 one-wavefront workgroups), so the
    grid-stride loop runs a second time for the last chunks, and a byte tail
    follows.  XOR(2) and RS(2,1) with unit coefficients both equal a ^ b
    (XOR's wave-uniform loop, RS(2,1)'s per-lane loop); RS(4,1) over
    [a, b, a, b] with coefficients (1, 1, 1, 0) equals b and RS(1,1) with
    coefficient 1 equals a (the wave-uniform loop of the two pass forms of
    rs_kernel, global and sc1 stores)."""
    n = (16 << 30) + 4096 + 48
    g = torch.Generator(device=dev)
    g.manual_seed(21)
    a = torch.empty(n, dtype=torch.uint8, device=dev).random_(0, 256, generator=g)
    b = torch.empty(n, dtype=torch.uint8, device=dev).random_(0, 256, generator=g)
    want = torch.bitwise_xor(a, b)
    x = pkg.xor_encode([a, b])
    torch.cuda.synchronize()
    assert torch.equal(x, want)
    del x
    r = pkg.matvec(np.ones((1, 2), np.uint8), [a, b])[0]
    torch.cuda.synchronize()
    assert torch.equal(r, want)
    del r, want
    r = pkg.matvec(np.array([[1, 1, 1, 0]], np.uint8), [a, b, a, b])[0]
    torch.cuda.synchronize()
    assert torch.equal(r, b)
    del r
    r = pkg.matvec(np.ones((1, 1), np.uint8), [a])[0]
    torch.cuda.synchronize()
    assert torch.equal(r, a)
    del a, b, r
    torch.cuda.empty_cache()


def _random_case(seed):
    """Shape of one randomized batched case: a code (mostly the unrolled
    k <= 16, m <= 4 kernels, sometimes a wide one), a unit size that is any
    multiple of 16 up to 20 KiB (so tiles end anywhere inside a unit),
    ragged tensor sizes from 1 byte to a few units, views at odd offsets or
    separate allocations."""
    r = np.random.default_rng(seed)
    if r.random() < 0.8:
        k, m = int(r.integers(1, 17)), int(r.integers(1, 5))
    else:
        k, m = int(r.integers(2, 21)), int(r.integers(5, 9))
    unit = 16 * int(r.integers(1, 1281))
    return r, k, m, unit, int(r.integers(1, 25)), bool(r.random() < 0.5)


@pytest.mark.parametrize("seed", range(64))
def test_batched_random_layouts(pkg, dev, seed):
    """Seeded random layouts through every batched entry point: the encode
    and the copying encode against the oracle (parity, zero-padded copies),
    a decode of a random set of at most m lost positions restores the data
    and the parity, and an update of random units equals a fresh encode."""
    from megatron_lm_amd import _lib
    r, k, m, unit, n_tensors, misalign = _random_case(seed)
    host, tensors = _ragged_device(r, dev, n_tensors, int(r.integers(2, 4 * unit + 2)), misalign)
    pset = pkg.encode(tensors, k, m, unit)
    lay = pset.layout
    S = lay.n_stripes
    torch.cuda.synchronize()
    want_par = _oracle_layout_parity(lay, host, unit)
    assert np.array_equal(pset.parity.cpu().numpy(), want_par), (k, m, unit)
    # copying encode into a stripe-major block
    block = torch.full((S, k + m, unit), 0xC3, dtype=torch.uint8, device=dev)
    base = np.uint64(block.data_ptr())
    rows = np.arange(S, dtype=np.uint64)[:, None] * np.uint64((k + m) * unit)
    cp = base + rows + np.arange(k, dtype=np.uint64)[None, :] * np.uint64(unit)
    pp = base + rows + (np.arange(m, dtype=np.uint64)[None, :] + np.uint64(k)) * np.uint64(unit)
    d_cp = torch.from_numpy(np.ascontiguousarray(cp).view(np.int64)).to(dev)
    d_pp = torch.from_numpy(np.ascontiguousarray(pp).view(np.int64)).to(dev)
    _lib.check(_lib.lib().ec_encode_batched_copy(
        _lib.u8ptr(lay.coeff), k, m, lay.d_ptrs.data_ptr(), lay.d_len.data_ptr(),
        d_pp.data_ptr(), d_cp.data_ptr(), S, unit, None), "ec_encode_batched_copy")
    torch.cuda.synchronize()
    got = block.cpu().numpy()
    assert np.array_equal(got[:, k:], want_par)
    for s in range(S):
        for j in range(k):
            u = s * k + j
            want = np.zeros(unit, np.uint8)
            if u < lay.n_units:
                t, i = int(lay.unit_tensor[u]), int(lay.unit_index[u])
                piece = host[t][i * unit: (i + 1) * unit]
                want[: piece.size] = piece
            assert np.array_equal(got[s, j], want), (s, j)
    del block, d_cp, d_pp
    # decode of a random lost set
    lost = sorted(int(x) for x in r.choice(k + m, int(r.integers(1, m + 1)), replace=False))
    par_ref = pset.parity.clone()
    for s in range(S):
        for pos in lost:
            u = s * k + pos
            if pos < k and u < lay.n_units:
                lay.unit_view(u).fill_(0xA5)
            elif pos >= k:
                pset.parity[s, pos - k].fill_(0x5A)
    pkg.decode(pset, lost)
    torch.cuda.synchronize()
    for h, t in zip(host, tensors):
        assert np.array_equal(t.cpu().numpy(), h), lost
    assert torch.equal(pset.parity, par_ref), lost
    # update of random units
    changed = np.sort(r.choice(lay.n_units, max(1, lay.n_units // 4), replace=False))
    olds, host_new = _perturb_units(r, lay, host, changed)
    pkg.update(pset, changed, olds)
    fresh = lay.encode()
    torch.cuda.synchronize()
    assert np.array_equal(pset.parity.cpu().numpy(),
                          _oracle_update(lay, host, host_new, changed, want_par)), (k, m, unit)
    assert torch.equal(pset.parity, fresh)


@pytest.mark.parametrize("seed", range(48))
def test_flat_random_shards(pkg, dev, seed):
    """Seeded random flat-shard calls: codes from RS(1,1) to RS(24,8) and
    XOR, sizes from 1 byte to ~300 KiB (vector body and byte tail), each
    shard and output at its own offset 0..15 (aligned, one shared
    misalignment, or mixed: the realigning and the byte kernels), with random
    coefficient matrices as well as the Cauchy block; the encode against the
    oracle and a reconstruction of a random erasure set."""
    r = np.random.default_rng(1000 + seed)
    k = int(r.integers(1, 25))
    m = int(r.integers(1, 9)) if r.random() < 0.3 else int(r.integers(1, 5))
    n = int(r.integers(1, 300_000))
    mode = int(r.integers(0, 3))   # 0 aligned, 1 one shared offset, 2 mixed offsets
    shared = int(r.integers(1, 16))

    def off():
        return 0 if mode == 0 else shared if mode == 1 else int(r.integers(0, 16))
    d = _host(r, k, n)
    dd = [_to_dev([a], dev, off())[0] for a in d]
    if r.random() < 0.25:
        C = r.integers(0, 256, (m, k), dtype=np.uint8)
        out = [_to_dev([np.zeros(n, np.uint8)], dev, off())[0] for _ in range(m)]
        got = pkg.matvec(C, dd, out=out)
        want = oracle.rs_encode(C, d)
        for g, w in zip(got, want):
            assert _eq(g, w), (k, m, n, mode)
        return
    C = oracle.cauchy(k, m)
    out = [_to_dev([np.zeros(n, np.uint8)], dev, off())[0] for _ in range(m)]
    par = pkg.rs_encode(dd, m, out=out)
    want = oracle.rs_encode(C, d)
    for g, w in zip(par, want):
        assert _eq(g, w), (k, m, n, mode)
    if m == 1:
        assert _eq(pkg.xor_encode(dd), oracle.xor_encode(d)), (k, n, mode)
    lost = sorted(int(x) for x in r.choice(k + m, int(r.integers(1, m + 1)), replace=False))
    cw = dd + par
    rec = pkg.reconstruct([None if g in lost else t for g, t in enumerate(cw)], k, m)
    full = d + want
    for g in lost:
        assert _eq(rec[g], full[g]), (k, m, n, mode, lost)


def test_host_threads_on_their_own_streams(pkg, dev):
    """The library is re-entrant: four host threads, each on a stream of its
    own, run 10 rounds of a flat RS(6,3) encode and a batched RS(8,2) encode
    of their own tensors at the same time; every result equals the oracle's."""
    import threading
    rng = np.random.default_rng(8)
    n, unit = (1 << 20) + 3, 8192
    jobs = []
    for _ in range(4):
        d = _host(rng, 6, n)
        host, tensors = _ragged_device(rng, dev, 12, 5 * unit, misalign=True)
        jobs.append((d, _to_dev(d, dev), host, tensors))
    torch.cuda.synchronize()
    results, errors = [None] * 4, []

    def work(i):
        try:
            s = torch.cuda.Stream(dev)
            with torch.cuda.stream(s):
                for _ in range(10):
                    par = pkg.rs_encode(jobs[i][1], 3)
                    lay = pkg.StripeLayout(jobs[i][3], 8, 2, unit)
                    bpar = lay.encode()
            s.synchronize()
            results[i] = ([p.cpu().numpy() for p in par], lay, bpar.cpu().numpy())
        except Exception as e:  # reported below, in the test's thread
            errors.append((i, e))

    threads = [threading.Thread(target=work, args=(i,)) for i in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not any(t.is_alive() for t in threads)
    assert not errors, errors
    C = oracle.cauchy(6, 3)
    for (d, _, host, _), (par, lay, bpar) in zip(jobs, results):
        for p, w in zip(par, oracle.rs_encode(C, d)):
            assert np.array_equal(p, w)
        assert np.array_equal(bpar, _oracle_layout_parity(lay, host, unit))
