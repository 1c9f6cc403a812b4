"""Command-line opt-in for erasure-coded in-memory checkpoints.

The reference reserves ``--non-persistent-ckpt-type in_memory``
(megatron/training/arguments.py:2126-2133) but rejects it in validation
(:332-333), and builds the local checkpoint context from
``--non-persistent-local-ckpt-dir`` plus the replication flags
``--replication / --replication-jump / --replication-factor``
(:2422-2431, validated at :1049-1056; built at
megatron/training/training.py:806-838).

This module fills the reserved choice:

* ``add_erasure_coding_args(parser)`` adds ``--ec-data-units`` (k),
  ``--ec-parity-units`` (m), ``--ec-unit-bytes``, ``--ec-jump`` and
  ``--[no-]ec-stage-in-background`` to a parser, and the reference's own
  checkpoint flags when the parser lacks them;
* ``validate_erasure_coding_args(args)`` applies the reference's rules to
  ``in_memory`` (a local directory is required, as for ``local``) and checks
  the code's shape;
* ``build_checkpointing_context(args, group, gloo_group)`` returns the
  ``checkpointing_context`` dict that training.py:833-838 builds, with an
  ``ECLocalCheckpointManager`` whose strategy places the slices of rank n on
  the coding-group members at least n + J, n + 2J, ... global ranks apart
  (J = ``--ec-jump``).  ``--ec-jump`` has the meaning of
  ``--replication-jump``; it is a flag of its own because the reference's
  validation clears ``replication_jump`` when ``--replication`` is off
  (arguments.py:1054-1056).

Data-parallel ranks are the coding group, as replication uses them.
"""
from __future__ import annotations

import argparse

IN_MEMORY = "in_memory"

# The engine's batched launcher takes k <= 32, m <= 16 (k <= 16, m <= 4 on
# its instantiated fast path).
MAX_DATA_UNITS = 32
MAX_PARITY_UNITS = 16


def _has(parser: argparse.ArgumentParser, flag: str) -> bool:
    return any(flag in a.option_strings for a in parser._actions)


def add_erasure_coding_args(parser: argparse.ArgumentParser) -> argparse.ArgumentParser:
    """Add the erasure-coding flags (and, for a stand-alone parser, the
    reference's non-persistent checkpoint flags they depend on)."""
    group = parser.add_argument_group(title="erasure-coded in-memory checkpoints")
    if not _has(parser, "--non-persistent-ckpt-type"):
        group.add_argument("--non-persistent-ckpt-type", type=str, default=None,
                           choices=["global", "local", IN_MEMORY, None])
    if not _has(parser, "--non-persistent-local-ckpt-dir"):
        group.add_argument("--non-persistent-local-ckpt-dir", type=str, default=None)
    if not _has(parser, "--replication"):
        group.add_argument("--replication", action="store_true", default=False)
    if not _has(parser, "--replication-jump"):
        group.add_argument("--replication-jump", default=None, type=int)
    if not _has(parser, "--replication-factor"):
        group.add_argument("--replication-factor", default=2, type=int)
    group.add_argument("--ec-data-units", type=int, default=4,
                       help="k: data units per stripe of the erasure code used by "
                            "--non-persistent-ckpt-type in_memory.")
    group.add_argument("--ec-parity-units", type=int, default=2,
                       help="m: parity units per stripe; any m ranks (or, with "
                            "--ec-jump = ranks per node, any m nodes) can lose "
                            "their local checkpoint.")
    group.add_argument("--ec-unit-bytes", type=int, default=4 << 20,
                       help="Bytes per coded unit (a multiple of 16).")
    group.add_argument("--ec-stage-in-background", action=argparse.BooleanOptionalAction,
                       default=True,
                       help="Asynchronous saves (--async-save) code the state into GPU memory, "
                            "hold training only for that, and stage, exchange and write the "
                            "slices from a background thread.")
    group.add_argument("--ec-jump", type=int, default=None,
                       help="Spacing J in global ranks between the ranks holding one rank's "
                            "k + m slices (rank n, then the coding-group members at least "
                            "n + J, n + 2J, ... away), as --replication-jump; set it to the "
                            "ranks per node to survive whole-node losses. Default 1.")
    return parser


def validate_erasure_coding_args(args) -> None:
    """The reference's validation for the local types, extended to
    ``in_memory``: raises AssertionError like arguments.py:1049-1056."""
    if args.non_persistent_ckpt_type != IN_MEMORY:
        return
    assert args.non_persistent_local_ckpt_dir is not None, \
        "Tried to use in_memory checkpointing without specifying --non-persistent-local-ckpt-dir!"
    assert not args.replication, \
        "--replication copies whole checkpoints; in_memory checkpoints use the erasure code " \
        "instead (--ec-data-units / --ec-parity-units)"
    k, m = args.ec_data_units, args.ec_parity_units
    assert 1 <= k <= MAX_DATA_UNITS, f"--ec-data-units must be in [1, {MAX_DATA_UNITS}], got {k}"
    assert 1 <= m <= MAX_PARITY_UNITS, \
        f"--ec-parity-units must be in [1, {MAX_PARITY_UNITS}], got {m}"
    u = args.ec_unit_bytes
    assert u > 0 and u % 16 == 0 and u <= (1 << 31), \
        f"--ec-unit-bytes must be a positive multiple of 16 up to 2 GiB, got {u}"
    jump = args.ec_jump
    assert jump is None or jump >= 1, f"--ec-jump must be positive, got {jump}"


def build_checkpointing_context(args, group=None, codec=None, gloo_group=None) -> dict:
    """``checkpointing_context`` for ``--non-persistent-ckpt-type in_memory``
    (the erasure-coded counterpart of training.py:806-838); an empty dict for
    any other type.  ``group`` is the coding group (the data-parallel group
    with context parallelism in Megatron, megatron/core/parallel_state.py:1240);
    None means the default group.  ``gloo_group`` is its gloo twin
    (``get_data_parallel_group_gloo(with_context_parallel=True)``,
    parallel_state.py:1258), which the slice exchange runs on; without it the
    strategy builds a private gloo group over the coding group's ranks."""
    if args.non_persistent_ckpt_type != IN_MEMORY:
        return {}
    validate_erasure_coding_args(args)
    from .checkpoint import ECLocalCheckpointManager, ErasureCodedStrategy
    strategy = ErasureCodedStrategy.from_ec_params(
        args.ec_data_units, args.ec_parity_units, args.ec_unit_bytes, jump=args.ec_jump or 1,
        group=group, gloo_group=gloo_group, codec=codec)
    return {"local_checkpoint_manager":
            ECLocalCheckpointManager(args.non_persistent_local_ckpt_dir, strategy,
                                     stage_in_background=args.ec_stage_in_background)}
