"""The erasure-coded checkpoint path with the real GPU codec: slices are
byte-identical to the oracle codec's, every k-subset of slices decodes, and
the multi-rank recovery scenario runs with ranks sharing the GPU (gloo for
the exchange, CPU tensors on the wire)."""
import itertools

import numpy as np
import pytest
import torch

from ec_cpu_codec import OracleSliceCodec
from ec_ckpt_worker import make_tensors, same
from test_checkpoint_cpu import launch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("k,m,unit", [(4, 2, 1024), (6, 3, 4096), (2, 1, 256), (12, 4, 65536)])
@pytest.mark.parametrize("chunk_stripes", [None, 3])
def test_gpu_slices_match_oracle_and_decode(pkg, dev, k, m, unit, chunk_stripes):
    """chunk_stripes = 3: device staging in chunks of about 3 stripes, so
    both buffers are reused and the last chunk is partial."""
    from megatron_lm_amd.checkpoint import GpuSliceCodec
    kw = {} if chunk_stripes is None else {"chunk_bytes": chunk_stripes * (k + m) * unit}
    cpu = make_tensors(3) + make_tensors(2)
    gpu = [t.to(dev) for t in cpu]
    gmeta, gs = GpuSliceCodec(k, m, unit, **kw).encode(gpu)
    ometa, os_ = OracleSliceCodec(k, m, unit).encode(cpu)
    assert gmeta == ometa
    for p, (a, b) in enumerate(zip(gs, os_)):
        assert np.array_equal(a, b), f"slice {p}"
    codec = GpuSliceCodec(k, m, unit, **kw)
    subsets = list(itertools.combinations(range(k + m), k))
    rng = np.random.default_rng(k)
    for idx in rng.choice(len(subsets), min(12, len(subsets)), replace=False):
        keep = subsets[idx]
        out = codec.decode(gmeta, {p: gs[p] for p in keep}, dev)
        assert same(out, cpu), keep


def test_gpu_checkpoint_recover_three_ranks(tmp_path):
    launch(tmp_path, "recover", world=3, k=2, m=1, unit=4096, use_gpu=True)


def test_gpu_checkpoint_cleanup_four_ranks(tmp_path):
    launch(tmp_path, "cleanup", world=4, k=2, m=2, unit=1024, use_gpu=True)


def test_gpu_checkpoint_tensor_aware_state_three_ranks(tmp_path):
    """A tensor-aware state dict comes back as itself, tensors rebuilt on the GPU."""
    launch(tmp_path, "tasd", world=3, k=2, m=1, unit=2048, use_gpu=True)


def test_gpu_empty_tensor_list(pkg, dev):
    """A rank with nothing to save still takes part: one all-zero stripe."""
    from megatron_lm_amd.checkpoint import GpuSliceCodec
    pset = pkg.encode([], 4, 2, 256)
    torch.cuda.synchronize()
    assert pset.parity.shape == (1, 2, 256) and not pset.parity.any()
    codec = GpuSliceCodec(4, 2, 256)
    meta, slices = codec.encode([])
    assert meta["n_units"] == 0 and all(not s.any() for s in slices)
    assert codec.decode(meta, {p: slices[p] for p in (1, 2, 4, 5)}, dev) == []


def test_gpu_encode_reuses_host_array_only_when_free(pkg, dev):
    """A live slice keeps its host array out of the next encode; once every
    slice is dropped the next encode of the same shape writes into it."""
    from megatron_lm_amd.checkpoint import GpuSliceCodec
    cpu = make_tensors(3)
    gpu = [t.to(dev) for t in cpu]
    codec = GpuSliceCodec(4, 2, 1024, chunk_bytes=2 * 6 * 1024)
    _, first = codec.encode(gpu)
    kept = [s.copy() for s in first]
    gpu2 = [(t + 1) if t.is_floating_point() else (t ^ 1) for t in gpu]
    meta2, second = codec.encode(gpu2)
    assert second[0].base is not first[0].base
    assert all(np.array_equal(a, b) for a, b in zip(first, kept)), "live slices were overwritten"
    base_id = id(second[0].base)  # an id, not a reference: a reference would keep it busy
    want = [s.copy() for s in second]
    del first, second
    meta3, third = codec.encode(gpu2)
    assert id(third[0].base) == base_id
    assert meta3 == meta2 and all(np.array_equal(a, b) for a, b in zip(third, want))
    _, oracle_slices = OracleSliceCodec(4, 2, 1024).encode([t.cpu() for t in gpu2])
    assert all(np.array_equal(a, b) for a, b in zip(third, oracle_slices))
