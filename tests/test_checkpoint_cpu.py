"""Erasure-coded local checkpoints across ranks on the CPU (gloo), with the
oracle-backed test codec.  Mirrors the recovery contract the reference's
tests pin for the redundancy slot: tests/unit_tests/dist_checkpointing/
test_replication.py:144-160 (lose some ranks' local data, still load the
iteration), test_local.py:246-326 (a failed save raises everywhere and leaves
nothing), test_local.py:225-244 (a new save removes the older one)."""
import glob
import socket

import pytest
import torch.multiprocessing as mp

import ec_ckpt_worker


def _free_port():
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


def launch(tmp_path, scenario, world=6, k=4, m=2, unit=1024, use_gpu=False, jump=1):
    err = str(tmp_path / "err")
    try:
        mp.start_processes(ec_ckpt_worker.run, nprocs=world, start_method="spawn",
                           args=(world, _free_port(), str(tmp_path / "ckpt"), scenario, k, m,
                                 unit, use_gpu, err, jump))
    except Exception as e:  # show the failing rank's traceback
        msgs = [open(f).read() for f in sorted(glob.glob(err + ".*"))]
        raise AssertionError("\n".join(msgs) or str(e))


@pytest.mark.parametrize("scenario", ["recover", "cleanup", "failed_save", "too_many_lost", "async",
                                      "async_write_lost", "tasd", "stray", "background",
                                      "background_fail", "incremental"])
def test_ec_checkpoint_scenarios(tmp_path, scenario):
    launch(tmp_path, scenario)


def test_ec_checkpoint_single_parity(tmp_path):
    launch(tmp_path, "recover", world=3, k=2, m=1, unit=256)


def test_ec_checkpoint_jump_placement(tmp_path):
    """Slices at stride ``jump`` (the reference's --replication-jump,
    megatron/training/arguments.py:2425-2429): file names follow
    (r + p * jump) mod G and one lost rank is still covered."""
    launch(tmp_path, "recover", world=6, k=2, m=1, unit=512, jump=2)


@pytest.mark.parametrize("jump,scenario", [(2, "node_lost"), (1, "node_lost_adjacent")])
def test_ec_checkpoint_node_loss(tmp_path, jump, scenario):
    """Losing a whole two-rank node: survivable with jump = ranks per node,
    not with adjacent placement and a single parity."""
    launch(tmp_path, scenario, world=6, k=2, m=1, unit=512, jump=jump)


def test_ec_strategy_rejects_colliding_jump():
    import __graft_entry__
    __graft_entry__.load_package()
    from megatron_lm_amd.checkpoint import CheckpointingException, ErasureCodedStrategy
    from ec_cpu_codec import OracleSliceCodec

    class Fixed(ErasureCodedStrategy):
        def ranks(self):
            return list(range(8))

    Fixed(2, 2, 256, codec=OracleSliceCodec(2, 2, 256), jump=2).check_group()  # 8/2 = 4 slots
    with pytest.raises(CheckpointingException):
        Fixed(3, 2, 256, codec=OracleSliceCodec(3, 2, 256), jump=2).check_group()
    with pytest.raises(CheckpointingException):
        Fixed(2, 1, 256, codec=OracleSliceCodec(2, 1, 256), jump=4).check_group()
    Fixed(4, 2, 256, codec=OracleSliceCodec(4, 2, 256), jump=3).check_group()  # gcd 1
    assert [Fixed(2, 2, 256, codec=OracleSliceCodec(2, 2, 256), jump=2).holder(5, p)
            for p in range(4)] == [5, 7, 1, 3]


def test_ec_checkpoint_reference_loss_pattern(tmp_path):
    """The reference's replication test deletes the local checkpoints of
    ranks 6, 3 and 4 of 8 and still loads iteration 1
    (tests/unit_tests/dist_checkpointing/test_replication.py:146-160); an
    RS(5,3) code over the 8 ranks survives those three losses."""
    launch(tmp_path, "loss_634", world=8, k=5, m=3, unit=512)


@pytest.mark.parametrize("scenario", ["strided", "cliques"])
def test_ec_checkpoint_sub_groups(tmp_path, scenario):
    """Coding groups other than the world, saving and loading concurrently:
    two strided data-parallel groups that report the NCCL backend (the
    exchange must run on a gloo group of its own; any collective on the given
    group fails the test), and uneven non-contiguous cliques with their gloo
    twins passed in (test_replication.py:75-80 runs such clique lists).
    Ranks 6, 3 and 4 lose their storage in both."""
    launch(tmp_path, scenario, world=8, unit=512)


def _strategy_over(members, k, m, jump):
    import __graft_entry__
    __graft_entry__.load_package()
    from megatron_lm_amd.checkpoint import ErasureCodedStrategy
    from ec_cpu_codec import OracleSliceCodec

    class Fixed(ErasureCodedStrategy):
        def ranks(self):
            return list(members)

    return Fixed(k, m, 256, codec=OracleSliceCodec(k, m, 256), jump=jump)


@pytest.mark.parametrize("tp", [1, 2, 4, 8, 16])
def test_ec_global_jump_places_slices_on_distinct_nodes(tp):
    """A data-parallel group of a 64-rank job with 8 ranks per node and
    tensor parallelism tp (members 0, tp, 2 tp, ...): the reference's
    --replication-jump = 8 (ranks per node) converted to a member spacing puts
    the k + m slices of every rank on k + m different nodes."""
    import __graft_entry__
    __graft_entry__.load_package()
    from megatron_lm_amd.checkpoint import index_jump
    members = list(range(0, 64, tp))
    ij = index_jump(members, 8)
    assert ij == max(1, -(-8 // tp))
    k, m = (4, 2) if len(members) >= 6 else (2, 2)
    st = _strategy_over(members, k, m, ij)
    st.check_group()
    for owner in members:
        nodes = [st.holder(owner, p) // 8 for p in range(k + m)]
        assert len(set(nodes)) == k + m, (tp, owner, nodes)


def test_ec_global_jump_needs_evenly_spaced_members():
    import __graft_entry__
    __graft_entry__.load_package()
    from megatron_lm_amd.checkpoint import CheckpointingException, index_jump
    assert index_jump([0, 1, 5, 9], 1) == 1
    with pytest.raises(CheckpointingException):
        index_jump([0, 1, 5, 9], 8)


def test_ec_nccl_group_without_gloo_is_refused(monkeypatch):
    """A coding group whose backend is NCCL and no gloo group to be had:
    the strategy raises CheckpointingException instead of issuing CPU-tensor
    collectives on it; a ``gloo_group`` that is not gloo is refused too."""
    import torch.distributed as dist
    import __graft_entry__
    __graft_entry__.load_package()
    from megatron_lm_amd.checkpoint import CheckpointingException

    def no_gloo(*a, **kw):
        raise RuntimeError("gloo is not available")

    nccl = object()
    monkeypatch.setattr(dist, "get_backend", lambda group=None: "nccl")
    monkeypatch.setattr(dist, "new_group", no_gloo)
    st = _strategy_over([0, 1, 2, 3], 2, 2, 1)
    st.group = nccl
    with pytest.raises(CheckpointingException, match="gloo"):
        st.comm_group()
    st = _strategy_over([0, 1, 2, 3], 2, 2, 1)
    st.gloo_group = nccl
    with pytest.raises(CheckpointingException, match="not gloo"):
        st.comm_group()


def test_slice_host_arrays_are_reused_only_after_release():
    """GpuSliceCodec's host arrays (host side only, no GPU): the slices own
    their array and the codec keeps no reference to one it handed out, so a
    later encode never writes into memory a caller still uses, held by
    slices or only by address; an array comes back for reuse only through
    ``release``."""
    import gc
    import weakref
    import numpy as np
    import __graft_entry__
    __graft_entry__.load_package()
    from megatron_lm_amd.checkpoint import GpuSliceCodec
    codec = GpuSliceCodec(4, 2, 4096)
    shape = (6, 3 * 4096)
    a = codec._host_out(shape)
    a.fill(0xAB)
    raw, alive = a.ctypes.data, weakref.ref(a)
    slices = [a[p] for p in range(6)]
    del a
    b = codec._host_out(shape)           # not released: a fresh array
    b.fill(0xCD)
    assert b.ctypes.data != raw and all(int(s.min()) == 0xAB for s in slices)
    del slices
    gc.collect()
    assert alive() is None               # the codec held no reference to it
    codec.release([b[p] for p in range(6)])
    c = codec._host_out(shape)
    assert c is b                        # released: reused
    d = codec._host_out(shape)
    assert d is not c                    # handed out again: not reusable until released
    with pytest.raises(ValueError):
        codec.release([c[0], c[1]])       # not all of one encode's slices
    with pytest.raises(ValueError):
        codec.release([np.zeros(10, np.uint8)])
    codec.release([c[p] for p in range(6)])
    e = codec._host_out((6, 4096))       # another shape: fresh (the released one is dropped)
    assert e.shape == (6, 4096) and e is not c
