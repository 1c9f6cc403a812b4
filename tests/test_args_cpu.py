"""The in_memory opt-in: flags, validation mirroring the reference's rules for
local checkpoints (megatron/training/arguments.py:1049-1056, :2126-2133,
:2422-2431), and the checkpointing context of training.py:806-838."""
import argparse
import socket

import pytest
import torch.distributed as dist

import __graft_entry__

ec = __graft_entry__.load_package()
from megatron_lm_amd import args as ec_args  # noqa: E402


def parse(argv, parser=None):
    p = ec_args.add_erasure_coding_args(parser or argparse.ArgumentParser())
    return p.parse_args(argv)


def test_defaults_and_other_types_untouched():
    a = parse([])
    assert (a.ec_data_units, a.ec_parity_units, a.ec_unit_bytes, a.ec_jump) == (4, 2, 4 << 20, None)
    ec_args.validate_erasure_coding_args(a)  # no checkpoint type: nothing to check
    assert ec_args.build_checkpointing_context(a) == {}
    a = parse(["--non-persistent-ckpt-type", "local", "--ec-data-units", "99"])
    ec_args.validate_erasure_coding_args(a)  # only in_memory is ours
    assert ec_args.build_checkpointing_context(a) == {}


def test_reference_flags_not_duplicated():
    """On the reference's parser the checkpoint flags already exist."""
    p = argparse.ArgumentParser()
    p.add_argument("--non-persistent-ckpt-type", type=str, default=None,
                   choices=["global", "local", "in_memory", None])
    p.add_argument("--non-persistent-local-ckpt-dir", type=str, default=None)
    p.add_argument("--replication", action="store_true", default=False)
    p.add_argument("--replication-jump", default=None, type=int)
    p.add_argument("--replication-factor", default=2, type=int)
    a = parse(["--non-persistent-ckpt-type", "in_memory", "--non-persistent-local-ckpt-dir",
               "/x", "--ec-data-units", "6", "--ec-parity-units", "3", "--ec-jump", "8"], p)
    ec_args.validate_erasure_coding_args(a)
    assert (a.ec_data_units, a.ec_parity_units, a.ec_jump) == (6, 3, 8)


@pytest.mark.parametrize("argv,msg", [
    ([], "without specifying"),
    (["--non-persistent-local-ckpt-dir", "/x", "--replication", "--replication-jump", "2"],
     "--replication"),
    (["--non-persistent-local-ckpt-dir", "/x", "--ec-data-units", "33"], "--ec-data-units"),
    (["--non-persistent-local-ckpt-dir", "/x", "--ec-parity-units", "17"], "--ec-parity-units"),
    (["--non-persistent-local-ckpt-dir", "/x", "--ec-parity-units", "0"], "--ec-parity-units"),
    (["--non-persistent-local-ckpt-dir", "/x", "--ec-unit-bytes", "1000"], "--ec-unit-bytes"),
    (["--non-persistent-local-ckpt-dir", "/x", "--ec-jump", "0"], "--ec-jump"),
])
def test_in_memory_validation(argv, msg):
    a = parse(["--non-persistent-ckpt-type", "in_memory"] + argv)
    with pytest.raises(AssertionError, match=msg):
        ec_args.validate_erasure_coding_args(a)


def test_build_context(tmp_path):
    from ec_cpu_codec import OracleSliceCodec
    from megatron_lm_amd.checkpoint import ECLocalCheckpointManager
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        port = s.getsockname()[1]
    dist.init_process_group("gloo", rank=0, world_size=1, init_method=f"tcp://127.0.0.1:{port}")
    try:
        a = parse(["--non-persistent-ckpt-type", "in_memory", "--non-persistent-local-ckpt-dir",
                   str(tmp_path), "--ec-data-units", "2", "--ec-parity-units", "1",
                   "--ec-unit-bytes", "4096", "--ec-jump", "3"])
        ctx = ec_args.build_checkpointing_context(a, codec=OracleSliceCodec(2, 1, 4096))
        mgr = ctx["local_checkpoint_manager"]
        assert isinstance(mgr, ECLocalCheckpointManager)
        st = mgr.strategy
        # --ec-jump is a spacing in global ranks, converted to a spacing of the
        # coding group's members: over a one-rank world that is one member
        assert (st.k, st.m, st.unit_bytes, st.jump) == (2, 1, 4096, 1)
        assert mgr.local_dir == tmp_path / "0"
        assert mgr.find_latest() == -1
        assert mgr.stage_in_background   # the default
        off = parse(["--non-persistent-ckpt-type", "in_memory", "--non-persistent-local-ckpt-dir",
                     str(tmp_path), "--no-ec-stage-in-background"])
        assert not ec_args.build_checkpointing_context(
            off, codec=OracleSliceCodec(4, 2, 4 << 20))["local_checkpoint_manager"].stage_in_background
    finally:
        dist.destroy_process_group()
