"""Drop-in entry points for one rank's checkpoint shards.

The reference's local checkpoint save hands ``MCoreTensorAwareStateDict``'s
ragged tensor list (megatron/core/dist_checkpointing/tensor_aware_state_dict.py:179-184)
to ``LocalCheckpointManager.save`` (megatron/training/checkpointing.py:538-541),
whose redundancy step is the ``repl_strategy`` injected at
megatron/training/training.py:825-835; recovery goes through ``manager.load``
(checkpointing.py:891-894).  The reference makes that redundancy by full
replication.  These functions compute m-of-(k+m) erasure-code parity over the
same tensor list instead, and rebuild lost units from it.  The list is used in
order, with no copy, on the GPU.

    pset = encode(tasd_tensors, k=12, m=4, unit_bytes=64 << 10)  # parity on HBM
    ...  # lose up to m unit positions of every stripe
    decode(pset, lost=[0, 13])                 # rebuild them in place
    update(pset, changed_units, old_copies)    # fold a partial change in
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np
import torch

from .layout import StripeLayout


@dataclass
class ParitySet:
    """Parity of a ragged tensor list: ``parity[s, i]`` is parity unit i of
    stripe s (uint8, [n_stripes, m, unit_bytes]) under ``layout``."""
    layout: StripeLayout
    parity: torch.Tensor

    @property
    def k(self) -> int:
        return self.layout.k

    @property
    def m(self) -> int:
        return self.layout.m


def encode(tensors: Sequence[torch.Tensor], k: int, m: int, unit_bytes: int = 64 << 10,
           coeff: Optional[np.ndarray] = None, stream=None) -> ParitySet:
    """Erasure-code a rank's ordered shard tensors in one batched launch."""
    layout = StripeLayout(tensors, k, m, unit_bytes, coeff)
    return ParitySet(layout, layout.encode(stream=stream))


def decode(pset: ParitySet, lost: Sequence[int], stripes=None, stream=None) -> None:
    """Rebuild the units at codeword positions ``lost`` (0..k-1 data, k..k+m-1
    parity) of every stripe (or of ``stripes``) in place."""
    pset.layout.decode(pset.parity, lost, stripes=stripes, stream=stream)


def update(pset: ParitySet, changed_units: Sequence[int], old_units: Sequence[torch.Tensor],
           stream=None) -> None:
    """Incremental parity update after the units ``changed_units`` changed;
    ``old_units`` hold their previous bytes."""
    pset.layout.update(pset.parity, changed_units, old_units, stream=stream)
