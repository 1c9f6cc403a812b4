"""The bandwidth probe bench.py uses for the practical ceiling
(libec_probe.so): it must touch exactly the bytes it claims, so that its
bandwidth figures are for the RS kernel's traffic."""
import ctypes
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def probe(pkg):
    path = os.path.join(ROOT, "probe", "libec_probe.so")
    lib = ctypes.CDLL(path)
    lib.ecp_stream.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                               ctypes.c_uint64, ctypes.c_void_p, ctypes.c_void_p]
    return lib


def _pattern(n16):
    p = np.zeros((n16, 4), np.uint32)
    p[:, 0] = np.arange(n16, dtype=np.uint32)
    p[:, 1:] = [0x9E3779B9, 0x7F4A7C15, 0x85EBCA6B]
    return p.view(np.uint8).reshape(-1)


def _ptrs(ts):
    return (ctypes.c_void_p * max(1, len(ts)))(*[t.data_ptr() for t in ts])


@pytest.mark.parametrize("r,w", [(6, 0), (0, 3), (6, 3), (1, 1)])
def test_probe_bytes(probe, dev, r, w):
    n = (1 << 20) + 4096 * 3  # a grid with an odd last tile
    rng = np.random.default_rng(r * 10 + w)
    host = [rng.integers(0, 256, n, dtype=np.uint8) for _ in range(r)]
    ins = [torch.from_numpy(h).to(dev) for h in host]
    outs = [torch.zeros(n, dtype=torch.uint8, device=dev) for _ in range(w)]
    sink = torch.zeros(16, dtype=torch.uint8, device=dev)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert probe.ecp_stream(_ptrs(ins), r, _ptrs(outs), w, n, sink.data_ptr(), st) == 0
    torch.cuda.synchronize()
    want = _pattern(n // 16)
    for h in host:
        want = want ^ h
    for o in outs:
        assert np.array_equal(o.cpu().numpy(), want)
    assert not sink.any()


def test_probe_rejects_bad_arguments(probe, dev):
    a = torch.zeros(64, dtype=torch.uint8, device=dev)
    sink = torch.zeros(16, dtype=torch.uint8, device=dev)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert probe.ecp_stream(_ptrs([a]), 1, _ptrs([a[16:]]), 1, 40, sink.data_ptr(), st) == -1
    assert probe.ecp_stream(_ptrs([a[1:]]), 1, _ptrs([a]), 1, 32, sink.data_ptr(), st) == -1
    assert probe.ecp_stream(_ptrs([a, a]), 2, _ptrs([a, a]), 2, 32, sink.data_ptr(), st) == -1  # (2, 2) not built
    assert probe.ecp_stream(_ptrs([a]), 1, _ptrs([a]), 1, 32, None, st) == -1
