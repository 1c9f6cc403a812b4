"""Erasure-coded local checkpoints across ranks on the CPU (gloo), with the
oracle-backed test codec.  Mirrors the recovery contract the reference's
tests pin for the redundancy slot: tests/unit_tests/dist_checkpointing/
test_replication.py:144-160 (lose some ranks' local data, still load the
iteration), test_local.py:246-326 (a failed save raises everywhere and leaves
nothing), test_local.py:225-244 (a new save removes the older one)."""
import glob
import os
import socket

import pytest
import torch.multiprocessing as mp

import ec_ckpt_worker


def _free_port():
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


def launch(tmp_path, scenario, world=6, k=4, m=2, unit=1024, use_gpu=False):
    err = str(tmp_path / "err")
    try:
        mp.start_processes(ec_ckpt_worker.run, nprocs=world, start_method="spawn",
                           args=(world, _free_port(), str(tmp_path / "ckpt"), scenario, k, m,
                                 unit, use_gpu, err))
    except Exception as e:  # show the failing rank's traceback
        msgs = [open(f).read() for f in sorted(glob.glob(err + ".*"))]
        raise AssertionError("\n".join(msgs) or str(e))


@pytest.mark.parametrize("scenario", ["recover", "cleanup", "failed_save", "too_many_lost", "async"])
def test_ec_checkpoint_scenarios(tmp_path, scenario):
    launch(tmp_path, scenario)


def test_ec_checkpoint_single_parity(tmp_path):
    launch(tmp_path, "recover", world=3, k=2, m=1, unit=256)
