"""Encode and reconstruct captured in a HIP graph and replayed.  The C ABI
allocates nothing and issues no memset, so its launches are capturable; each
replay is checked against the eager result, with eager work and host
synchronisation between replays."""
import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


def test_graph_replays_match_eager(pkg, dev):
    k, m, n = 6, 3, (4 << 20) + 48
    rng = np.random.default_rng(9)
    host = [rng.integers(0, 256, n, dtype=np.uint8) for _ in range(k)]
    data = [torch.from_numpy(h).to(dev) for h in host]
    parity = [torch.empty(n, dtype=torch.uint8, device=dev) for _ in range(m)]
    rec = [torch.empty(n, dtype=torch.uint8, device=dev) for _ in range(3)]
    coeff = pkg.cauchy_matrix(k, m)
    lost = [0, 4, 8]
    surv, rows = pkg.decode_matrix(coeff, lost)
    cw = data + parity
    sv = [cw[s] for s in surv]
    torch.cuda.synchronize()

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):  # warm up on the capture stream
        pkg.matvec(coeff, data, out=parity)
        pkg.matvec(rows, sv, out=rec, what="ec_rs_decode")
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        pkg.matvec(coeff, data, out=parity)
        pkg.matvec(rows, sv, out=rec, what="ec_rs_decode")
    want = oracle.rs_encode(oracle.cauchy(k, m), host)
    for rep in range(4):
        # change the data eagerly, replay, check against the CPU encoder
        step = rng.integers(0, 256, n, dtype=np.uint8)
        host[rep % k] ^= step
        data[rep % k].copy_(torch.from_numpy(host[rep % k]))
        for t in parity + rec:
            t.fill_(0xEE)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        want = oracle.rs_encode(oracle.cauchy(k, m), host)
        for i in range(m):
            assert np.array_equal(parity[i].cpu().numpy(), want[i]), f"replay {rep} parity {i}"
        for r, gidx in enumerate(lost):
            ref = host[gidx] if gidx < k else want[gidx - k]
            assert np.array_equal(rec[r].cpu().numpy(), ref), f"replay {rep} shard {gidx}"


@pytest.mark.parametrize("unit", [16384, 2 << 20])
def test_graph_batched_encode_and_decode(pkg, dev, unit):
    """The batched launcher over a ragged list in a graph: encode, then
    decode of two lost positions, replayed after eager changes to the data;
    each replay checked against an eager encode and the tensors' bytes.
    RS(8,2) over 2 MiB units runs as two kernels per call (full tiles, then
    the rest), both captured."""
    k, m = 8, 2
    rng = np.random.default_rng(21)
    sizes = rng.integers(1, 5 * unit, 40)
    tensors = [torch.from_numpy(rng.integers(0, 256, int(n), dtype=np.uint8)).to(dev)
               for n in sizes]
    lay = pkg.StripeLayout(tensors, k, m, unit)
    par = lay.alloc_parity()
    plan = lay.plan_decode(par, [3, 9])   # descriptors made before capture
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        lay.encode(par, stream=s)
        lay.run(plan, stream=s)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        lay.encode(par)
        lay.run(plan)
    for rep in range(4):
        t = tensors[rep * 7 % len(tensors)]
        t.copy_(torch.from_numpy(rng.integers(0, 256, t.numel(), dtype=np.uint8)))
        truth = [x.clone() for x in tensors]
        par.fill_(0xEE)
        torch.cuda.synchronize()
        g.replay()          # encode, then rebuild positions 3 and 9 in place
        torch.cuda.synchronize()
        fresh = lay.encode()
        torch.cuda.synchronize()
        assert torch.equal(par, fresh), f"replay {rep}: parity"
        assert all(torch.equal(a, b) for a, b in zip(tensors, truth)), f"replay {rep}: data"
