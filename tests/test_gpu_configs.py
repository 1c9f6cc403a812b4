"""The five benchmark configurations at full size on the GPU: XOR 4 x 64 MiB,
RS(6,3) 6 x 256 MiB encode and 3-erasure decode, RS(8,2) over a 20.8 GB rank
buffer in 4 MiB units, RS(12,4) over 3,000 ragged tensors with a 1% update.

Every output is compared byte for byte against the CPU encoder
(oracle/ec_cpu_fast.c, itself pinned to the scalar oracle by test_oracle.py)
on the same seeded numpy bytes: configs 1 and 2 whole, configs 4 and 5 stripe
by stripe over the whole buffer, the config-3 decode against the original
shards, config 5's incremental update (seeded numpy bytes) stripe by stripe
against the CPU encoder over the perturbed bytes.  On top, size-independent
properties over the whole buffer: erase -> decode round trips and update ==
full re-encode.
"""
import os

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

MiB = 1 << 20
THREADS = max(1, min(16, len(os.sched_getaffinity(0))))


def _say(msg):
    print(f"[configs] {msg}", flush=True)


@pytest.fixture(scope="module")
def synth(pkg):
    from megatron_lm_amd import synth
    return synth


def test_config1_xor_4x64MiB(pkg, dev, synth):
    _say("config 1: XOR 4 x 64 MiB bf16")
    for seed in (0, 1):
        host = synth.xor_shards(seed, 64 * MiB, 4)
        p = pkg.xor_encode([torch.from_numpy(h).to(dev) for h in host])
        torch.cuda.synchronize()
        assert np.array_equal(p.cpu().numpy(), oracle.fast_xor_encode(host, nthreads=THREADS))


@pytest.fixture(scope="module")
def rs63(pkg, dev, synth):
    _say("config 2: RS(6,3) 6 x 256 MiB fp32 optimizer state")
    host = synth.rs_shards(0, 256 * MiB, 6)
    data = [torch.from_numpy(h).to(dev) for h in host]
    parity = pkg.rs_encode(data, 3)
    torch.cuda.synchronize()
    return host, data, parity


def test_config2_rs63_256MiB_bit_exact(pkg, rs63):
    host, data, parity = rs63
    want = oracle.fast_rs_encode(oracle.cauchy(6, 3), host, nthreads=THREADS)
    for i in range(3):
        assert np.array_equal(parity[i].cpu().numpy(), want[i]), f"parity {i}"


@pytest.mark.parametrize("seed", [0, 1, 2, 3, 4])
def test_config3_decode_three_erasures(pkg, rs63, synth, seed):
    _, data, parity = rs63
    cw = data + parity
    lost = synth.erasures(seed, 9, 3)
    _say(f"config 3: seed {seed} lost {lost}")
    # The lost shards are zeroed and marked lost; the survivors are untouched.
    work = [torch.zeros_like(t) if g in lost else t for g, t in enumerate(cw)]
    rec = pkg.reconstruct([None if g in lost else t for g, t in enumerate(work)], 6, 3)
    torch.cuda.synchronize()
    for g in lost:
        assert torch.equal(rec[g], cw[g]), f"shard {g}"


def test_config3_every_erasure_pattern_full_size(pkg, rs63):
    """All 129 patterns of at most 3 lost shards among the 9, at full size."""
    import itertools
    _, data, parity = rs63
    cw = data + parity
    n = 0
    for e in (1, 2, 3):
        for lost in itertools.combinations(range(9), e):
            rec = pkg.reconstruct([None if g in lost else t for g, t in enumerate(cw)], 6, 3)
            torch.cuda.synchronize()
            for g in lost:
                assert torch.equal(rec[g], cw[g]), f"lost {lost} shard {g}"
            n += 1
    assert n == 129


def _check_every_stripe(layout, parity, host_views, what):
    """Every stripe's parity, byte for byte, against the SIMD CPU encoder
    (itself pinned to the scalar oracle by test_oracle.py) run over host
    descriptors of the same bytes, on all usable cores."""
    from megatron_lm_amd.layout import stripe_descriptors
    k, m, unit = layout.k, layout.m, layout.unit_bytes
    _, hptr, hlen = stripe_descriptors([v.ctypes.data for v in host_views],
                                       [v.size for v in host_views], k, unit)
    assert hptr.shape == (layout.n_stripes, k) and np.array_equal(hlen, layout.host_len)
    want = np.empty((layout.n_stripes, m, unit), np.uint8)
    pp = (np.uint64(want.ctypes.data) + np.arange(layout.n_stripes * m, dtype=np.uint64)
          .reshape(layout.n_stripes, m) * np.uint64(unit))
    oracle.fast_encode_batched(layout.coeff, hptr, hlen, pp, unit, nthreads=THREADS)
    got = parity.cpu().numpy()
    bad = np.flatnonzero((got != want).reshape(layout.n_stripes, -1).any(axis=1))
    assert bad.size == 0, f"{what}: {bad.size} stripes differ, first {bad[:8].tolist()}"
    _say(f"{what}: all {layout.n_stripes} stripes byte-identical to the CPU encoder")


def test_config4_gpt13b_rank_buffer_rs82(pkg, dev, synth):
    _say("config 4: 20.8 GB rank buffer, RS(8,2), 4 MiB units (numpy, seeded)")
    host = synth.gpt_rank_buffer_host(seed=4)
    buf = torch.from_numpy(host).to(dev)
    pset = pkg.encode([buf], 8, 2, 4 * MiB)
    lay = pset.layout
    assert lay.n_stripes == -(-buf.numel() // (8 * 4 * MiB))
    torch.cuda.synchronize()
    _check_every_stripe(lay, pset.parity, [host], "config 4")
    del host
    rng = np.random.default_rng(4)
    # Round trip over every stripe: lose one data and one parity position.
    lost = [int(rng.integers(0, 8)), 8 + int(rng.integers(0, 2))]
    ref_buf, ref_par = buf.clone(), pset.parity.clone()
    view = buf.view(-1)
    nfull = buf.numel() // (4 * MiB)
    for s in range(lay.n_stripes):
        u = s * 8 + lost[0]
        if u < lay.n_units:
            lay.unit_view(u).fill_(0)
    pset.parity[:, lost[1] - 8].fill_(0)
    pkg.decode(pset, lost)
    torch.cuda.synchronize()
    assert torch.equal(view, ref_buf) and torch.equal(pset.parity, ref_par), f"lost {lost}"
    _say(f"config 4: round trip with lost {lost} ok ({nfull} full units)")


def test_config5_ragged_3000_rs124_and_update(pkg, dev, synth):
    _say("config 5: 3,000 ragged tensors, RS(12,4), 64 KiB units (numpy, seeded)")
    block, views, kinds = synth.ragged_host(5)
    tensors = [torch.from_numpy(v).to(dev).view(torch.bfloat16 if kd == 0 else torch.float32)
               for v, kd in zip(views, kinds.tolist())]
    pset = pkg.encode(tensors, 12, 4, 64 << 10)
    lay = pset.layout
    _say(f"config 5: {lay.data_bytes / 1e9:.2f} GB in {lay.n_units} units, {lay.n_stripes} stripes")
    torch.cuda.synchronize()
    _check_every_stripe(lay, pset.parity, views, "config 5")
    rng = np.random.default_rng(5)
    # Incremental update after a seeded 1% perturbation: the new bytes come
    # from seeded numpy, go to the device tensors and to the host copies, and
    # the updated parity of every stripe is compared with the CPU encoder
    # over the perturbed host bytes.
    changed = synth.perturbed_units(5, lay.n_units, 0.01)
    unit = lay.unit_bytes
    fresh_bytes = synth.perturbation_bytes(5, lay.host_len.reshape(-1)[changed])
    olds = []
    for u, nb in zip(changed.tolist(), fresh_bytes):
        v = lay.unit_view(u)
        olds.append(v.clone())
        v.copy_(torch.from_numpy(nb))
        t, i = int(lay.unit_tensor[u]), int(lay.unit_index[u])
        views[t][i * unit: i * unit + nb.size] = nb
    pkg.update(pset, changed, olds)
    torch.cuda.synchronize()
    _check_every_stripe(lay, pset.parity, views, f"config 5 after the update of {changed.size} units")
    fresh = lay.encode()
    torch.cuda.synchronize()
    assert torch.equal(pset.parity, fresh)
    del block, views, fresh, olds
    # Round trip: lose 4 positions (2 data, 2 parity) of every stripe.
    lost = sorted(rng.choice(12, 2, replace=False).tolist() + (12 + rng.choice(4, 2, replace=False)).tolist())
    refs = [t.clone() for t in tensors]
    ref_par = pset.parity.clone()
    for s in range(lay.n_stripes):
        for pos in lost:
            u = s * 12 + pos
            if pos < 12 and u < lay.n_units:
                lay.unit_view(u).fill_(0)
    for pos in lost:
        if pos >= 12:
            pset.parity[:, pos - 12].fill_(0)
    pkg.decode(pset, lost)
    torch.cuda.synchronize()
    assert torch.equal(pset.parity, ref_par)
    for t, r in zip(tensors, refs):
        # byte compare: the perturbation wrote random bits, so floats may be NaN
        assert torch.equal(t.view(-1).view(torch.uint8), r.view(-1).view(torch.uint8))
    _say(f"config 5: round trip with lost {lost} ok")
