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
                                      "background_fail"])
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
