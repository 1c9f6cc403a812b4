"""The erasure-coded checkpoint path with the real GPU codec: slices are
byte-identical to the oracle codec's, every k-subset of slices decodes, and
the multi-rank recovery scenario runs with ranks sharing the GPU (gloo for
the exchange, CPU tensors on the wire)."""
import itertools
import subprocess
import sys

import numpy as np
import pytest
import torch

from conftest import ROOT
from ec_cpu_codec import OracleSliceCodec
from ec_ckpt_worker import bump, make_tensors, same
from test_checkpoint_cpu import launch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("k,m,unit", [(4, 2, 1024), (6, 3, 4096), (2, 1, 256), (12, 4, 65536)])
@pytest.mark.parametrize("chunk_stripes", [None, 3])
def test_gpu_slices_match_oracle_and_decode(pkg, dev, k, m, unit, chunk_stripes):
    """chunk_stripes = None: the one-block path; 3: the chunked path with
    chunks of about 3 stripes, so both buffers are reused and the last chunk
    is partial."""
    from megatron_lm_amd.checkpoint import GpuSliceCodec
    kw = {} if chunk_stripes is None else {"chunk_bytes": chunk_stripes * (k + m) * unit,
                                           "snapshot_bytes": 0}
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


def test_gpu_checkpoint_background_three_ranks(tmp_path):
    """Saves staged in the background with the GPU codec's snapshot: the
    tensors bumped on torch's stream right after save() do not reach the
    checkpoint; two saves in flight both land."""
    launch(tmp_path, "background", world=3, k=2, m=1, unit=4096, use_gpu=True)


def test_gpu_checkpoint_incremental_three_ranks(tmp_path):
    """Saves naming the changed tensors, through the GPU codec's kept block
    (keep_block): every save after the first takes the incremental path and
    loads back as the state of its call, also after a rank loses its
    storage."""
    launch(tmp_path, "incremental", world=3, k=2, m=1, unit=1024, use_gpu=True)


def _oracle_slices(k, m, unit, gpu):
    return OracleSliceCodec(k, m, unit).encode([t.cpu() for t in gpu])


@pytest.mark.parametrize("k,m,unit", [(6, 3, 4096), (12, 4, 1024), (4, 2, 256), (2, 1, 65536)])
def test_gpu_incremental_saves_equal_full_encodes(pkg, dev, k, m, unit):
    """A keep_block codec over a sequence of saves, each naming the tensors
    changed since the one before (none, some, all, part of one tensor), also
    through snapshot() with the next step's writes racing it: every save's
    slices equal the oracle codec's full encode of the state of its call, and
    every save after the first takes the incremental path (the kept block is
    updated in place, not reallocated)."""
    from megatron_lm_amd.checkpoint import GpuSliceCodec
    cpu = make_tensors(3) + make_tensors(1) + [torch.arange(3001, dtype=torch.int32)]
    gpu = [t.to(dev) for t in cpu]
    codec = GpuSliceCodec(k, m, unit, keep_block=True)
    calls = []
    inner = codec._snapshot_delta
    codec._snapshot_delta = lambda *a, **kw: calls.append(1) or inner(*a, **kw)
    meta, sl = codec.encode(gpu)
    assert meta == _oracle_slices(k, m, unit, gpu)[0]
    block = codec._resident[0].data_ptr()
    codec.release(sl)
    rng = np.random.default_rng(k * 100 + unit)
    plans = [[], [0], list(range(len(gpu))), [2, 4], [len(gpu) - 1]]
    for n, changed in enumerate(plans):
        for i in changed:
            bump(gpu[i])
        if n == 3:   # part of a tensor only: a few bytes of one unit
            flat = gpu[2].view(-1).view(torch.uint8)
            flat[int(rng.integers(0, flat.numel() - 4)):][:4] ^= 0x5A
        want = _oracle_slices(k, m, unit, gpu)
        if n % 2:
            pending = codec.snapshot(gpu, changed_tensors=changed)
            for t in gpu:                      # the next step, after the call
                t.view(-1).view(torch.uint8).bitwise_xor_(0x5A)
            meta, sl = pending.result(timeout=120)
            for t in gpu:                      # undone exactly, as if it never ran
                t.view(-1).view(torch.uint8).bitwise_xor_(0x5A)
            torch.cuda.synchronize()
        else:
            meta, sl = codec.encode(gpu, changed_tensors=changed)
        assert meta == want[0], n
        for p, (a, b) in enumerate(zip(sl, want[1])):
            assert np.array_equal(a, b), (n, changed, p)
        codec.release(sl)
    assert len(calls) == len(plans)
    assert codec._resident[0].data_ptr() == block


def test_gpu_incremental_saves_over_misaligned_views(pkg, dev):
    """Tensors that are views of one flat buffer at odd byte offsets (the
    update and the unit copy take their realigning and byte-granular paths):
    incremental saves equal the oracle codec's full encodes, with the bytes
    between the views left alone."""
    from megatron_lm_amd.checkpoint import GpuSliceCodec
    k, m, unit = 6, 3, 2048
    rng = np.random.default_rng(31)
    sizes = [int(x) for x in rng.integers(1, 5 * unit, 9)]
    arena = torch.full((sum(sizes) + 7 * len(sizes),), 0xC3, dtype=torch.uint8, device=dev)
    views, off = [], 0
    for n in sizes:
        off += int(rng.integers(1, 7))
        v = arena[off: off + n]
        v.copy_(torch.from_numpy(rng.integers(0, 256, n, dtype=np.uint8)))
        views.append(v)
        off += n
    gaps = arena.clone()
    codec = GpuSliceCodec(k, m, unit, keep_block=True)
    codec.release(codec.encode(views)[1])
    for changed in ([3], [0, 8], [], list(range(9)), [5]):
        for i in changed:
            views[i].bitwise_xor_(torch.from_numpy(
                rng.integers(1, 256, sizes[i], dtype=np.uint8)).to(dev))
        meta, sl = codec.encode(views, changed_tensors=changed)
        want = _oracle_slices(k, m, unit, views)
        assert meta == want[0]
        for p, (a, b) in enumerate(zip(sl, want[1])):
            assert np.array_equal(a, b), (changed, p)
        codec.release(sl)
    covered = torch.zeros_like(arena, dtype=torch.bool)
    for v in views:
        start = v.data_ptr() - arena.data_ptr()
        covered[start: start + v.numel()] = True
    assert torch.equal(arena[~covered], gaps[~covered])


def test_gpu_incremental_save_codes_only_the_named_tensors(pkg, dev):
    """The incremental path codes only the tensors it is told changed: a
    tensor changed behind its back keeps its old bytes in the slices (the
    caller's contract; this is what makes the save incremental), and a save
    over other tensors, or without changed_tensors, takes the full encode."""
    from megatron_lm_amd.checkpoint import GpuSliceCodec
    k, m, unit = 4, 2, 1024
    gpu = [t.to(dev) for t in make_tensors(3)]
    codec = GpuSliceCodec(k, m, unit, keep_block=True)
    calls = []
    inner = codec._snapshot_delta
    codec._snapshot_delta = lambda *a, **kw: calls.append(1) or inner(*a, **kw)
    before = _oracle_slices(k, m, unit, gpu)
    codec.release(codec.encode(gpu)[1])
    orig1 = gpu[1].clone()
    bump(gpu[0])
    bump(gpu[1])
    _, sl = codec.encode(gpu, changed_tensors=[0])   # gpu[1] changed too, unnamed
    after = _oracle_slices(k, m, unit, gpu)
    stale = _oracle_slices(k, m, unit, [gpu[0], orig1] + gpu[2:])
    assert calls == [1]
    assert all(np.array_equal(a, b) for a, b in zip(sl, stale[1]))
    assert not all(np.array_equal(a, b) for a, b in zip(sl, after[1]))
    assert not all(np.array_equal(a, b) for a, b in zip(sl, before[1]))
    codec.release(sl)
    # a full save (no changed_tensors) brings the block up to date
    _, sl = codec.encode(gpu)
    assert calls == [1] and all(np.array_equal(a, b) for a, b in zip(sl, after[1]))
    codec.release(sl)
    # other tensors (other device bytes): the full encode, whatever is named
    other = [t.clone() for t in gpu]
    _, sl = codec.encode(other, changed_tensors=[])
    assert calls == [1] and all(np.array_equal(a, b) for a, b in zip(sl, after[1]))
    # the kept block does not keep the slices' host array alive
    import gc
    import weakref
    host = weakref.ref(sl[0].base)
    del sl
    gc.collect()
    assert host() is None
    with pytest.raises(ValueError):
        codec.encode(other, changed_tensors=[7])


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


def test_gpu_encode_reuses_host_array_only_after_release(pkg, dev):
    """An encode's host array is written again only after the caller hands
    it back with release(): without that, even with every slice dropped, the
    next encode takes a fresh array; after it, the next encode of the same
    shape writes into the released one, with the right bytes."""
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
    raw = first[0].base.ctypes.data   # a consumer that keeps only the address of the first
    held = first[0].base
    del first
    meta3, third = codec.encode(gpu2)
    assert third[0].base.ctypes.data != raw and np.array_equal(held[0], kept[0])
    want = [s.copy() for s in second]
    base = second[0].base
    codec.release(second)
    del second
    meta4, fourth = codec.encode(gpu2)
    assert fourth[0].base is base     # the released array, written again
    assert meta4 == meta2 and all(np.array_equal(a, b) for a, b in zip(fourth, want))
    _, oracle_slices = OracleSliceCodec(4, 2, 1024).encode([t.cpu() for t in gpu2])
    assert all(np.array_equal(a, b) for a, b in zip(fourth, oracle_slices))


@pytest.mark.parametrize("k,m,unit,chunk_stripes", [(4, 2, 1024, None), (6, 3, 4096, 2),
                                                    (12, 4, 65536, None), (3, 2, 256, 1)])
def test_gpu_snapshot_codes_the_state_at_the_call(pkg, dev, k, m, unit, chunk_stripes):
    """snapshot() codes the tensors as they are when it is called: writes
    enqueued on torch's stream right after it (the next optimizer step) do not
    reach the slices, which equal the oracle's byte for byte, and decode."""
    from megatron_lm_amd.checkpoint import GpuSliceCodec
    kw = {} if chunk_stripes is None else {"chunk_bytes": chunk_stripes * (k + m) * unit}
    cpu = make_tensors(1) + make_tensors(3)
    gpu = [t.to(dev) for t in cpu]
    codec = GpuSliceCodec(k, m, unit, **kw)
    pending = codec.snapshot(gpu)
    for t in gpu:
        bump(t)
    meta, slices = pending.result(timeout=120)
    assert pending.done()
    ometa, oslices = OracleSliceCodec(k, m, unit).encode(cpu)
    assert meta == ometa
    for p, (a, b) in enumerate(zip(slices, oslices)):
        assert np.array_equal(a, b), f"slice {p}"
    keep = list(range(m, k + m))   # the first m data slices lost
    out = codec.decode(meta, {p: slices[p] for p in keep}, dev)
    assert same(out, cpu)


def test_gpu_snapshots_in_flight_together(pkg, dev):
    """Two snapshots staged at once (one codec, different states) both come
    back whole, and a synchronous encode between them is unaffected."""
    from megatron_lm_amd.checkpoint import GpuSliceCodec
    codec = GpuSliceCodec(4, 2, 2048, chunk_bytes=3 * 6 * 2048)
    a_cpu, b_cpu = make_tensors(2), make_tensors(3)
    a, b = [t.to(dev) for t in a_cpu], [t.to(dev) for t in b_cpu]
    pa = codec.snapshot(a)
    pb = codec.snapshot(b)
    _, mid = codec.encode(a)
    _, sa = pa.result(timeout=120)
    _, sb = pb.result(timeout=120)
    oracle = OracleSliceCodec(4, 2, 2048)
    for got, ref in ((sa, oracle.encode(a_cpu)[1]), (sb, oracle.encode(b_cpu)[1]),
                     (mid, oracle.encode(a_cpu)[1])):
        assert all(np.array_equal(x, y) for x, y in zip(got, ref))


def test_gpu_side_stream(pkg, dev):
    """ec_stream_create: one cached stream per (device, CUs); the encode on it
    matches the one on torch's stream, also restricted to 64 CUs."""
    s_all = pkg.side_stream(dev)
    assert pkg.side_stream(dev) is s_all and s_all.device == dev
    s_64 = pkg.side_stream(dev, cus=64)
    assert s_64 is not s_all
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    data = [torch.randint(0, 256, (1 << 20,), dtype=torch.uint8, device=dev, generator=g)
            for _ in range(6)]
    ref = pkg.rs_encode(data, 3)
    for s in (s_all, s_64):
        s.wait_stream(torch.cuda.current_stream(dev))
        out = pkg.rs_encode(data, 3, stream=s)
        s.synchronize()
        assert all(torch.equal(x, y) for x, y in zip(out, ref))


def test_gpu_snapshot_falls_back_to_chunks(pkg, dev):
    """A block over snapshot_bytes is coded by the chunked encode before
    snapshot() returns: the same slices, ready at once."""
    from megatron_lm_amd.checkpoint import GpuSliceCodec
    cpu = make_tensors(2)
    gpu = [t.to(dev) for t in cpu]
    codec = GpuSliceCodec(4, 2, 1024, chunk_bytes=2 * 6 * 1024, snapshot_bytes=0)
    pending = codec.snapshot(gpu)
    assert pending.done()
    for t in gpu:
        bump(t)
    meta, slices = pending.result(timeout=60)
    ometa, oslices = OracleSliceCodec(4, 2, 1024).encode(cpu)
    assert meta == ometa and all(np.array_equal(a, b) for a, b in zip(slices, oslices))


def test_gpu_side_stream_use_outlives_exit_hooks(dev):
    """A tensor that carries a record_stream use of a side stream and lives
    until module teardown (freed after the exit hooks) ends its process
    cleanly: the side streams are not destroyed before the allocator records
    its event on them."""
    code = (
        "import sys; sys.path.insert(0, sys.argv[1])\n"
        "import torch, __graft_entry__\n"
        "ec = __graft_entry__.load_package()\n"
        "dev = torch.device('cuda:0')\n"
        "side = ec.side_stream(dev)\n"
        "held = [torch.randint(0, 256, (1 << 20,), dtype=torch.uint8, device=dev)"
        " for _ in range(4)]\n"
        "side.wait_stream(torch.cuda.current_stream(dev))\n"
        "parity = ec.rs_encode(held, 2, stream=side)\n"
        "for t in held + list(parity):\n"
        "    t.record_stream(side)\n"
        "print('enqueued', flush=True)\n")
    print("case: side-stream use freed after the exit hooks", flush=True)
    r = subprocess.run([sys.executable, "-c", code, ROOT], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0 and "enqueued" in r.stdout, (r.returncode, r.stderr[-2000:])


def test_gpu_encode_reuses_descriptors_of_the_same_buffers(dev):
    """A save of tensors occupying the same device bytes as the last one
    reuses its stripe descriptors; another address, a shorter tensor, another
    order or a changed value in place all give the right slices (the first
    three through fresh descriptors), and the kept descriptors hold no
    reference to the tensors."""
    import weakref
    from megatron_lm_amd.checkpoint import GpuSliceCodec
    k, m, unit = 4, 2, 1024
    cpu = make_tensors(3) + make_tensors(2)
    gpu = [t.to(dev) for t in cpu]
    codec = GpuSliceCodec(k, m, unit)
    oracle = OracleSliceCodec(k, m, unit)

    def check(gt, ct):
        meta, sl = codec.encode(gt)
        assert meta == oracle.encode(ct)[0]
        for p, (a, b) in enumerate(zip(sl, oracle.encode(ct)[1])):
            assert np.array_equal(a, b), f"slice {p}"
        codec.release(sl)

    check(gpu, cpu)
    kept = codec._last_layout
    assert kept.tensors == []
    bump(gpu[1])                             # same bytes, new values: reused
    cpu[1] = gpu[1].cpu()
    check(gpu, cpu)
    assert codec._last_layout is kept
    moved = list(gpu)
    moved[2] = gpu[2].clone()                # another address
    check(moved, cpu)
    assert codec._last_layout is not kept
    kept = codec._last_layout
    short = list(moved)
    short[0] = moved[0].reshape(-1)[:-3]     # the same address, fewer bytes
    check(short, [cpu[0].reshape(-1)[:-3]] + cpu[1:])
    assert codec._last_layout is not kept
    swapped = [moved[1], moved[0]] + moved[2:]
    check(swapped, [cpu[1], cpu[0]] + cpu[2:])
    probe = weakref.ref(swapped[3])
    del gpu, moved, short, swapped
    import gc
    gc.collect()
    assert probe() is None
