"""MI355X (gfx950) erasure-coding engine for Megatron-LM local checkpoints.

Serialized checkpoint shards held in HIP tensors pass through the C ABI of
``include/ec_mi355.h`` (libec_mi355.so, built in-tree) to hand-written gfx950
kernels: XOR parity, GF(2^8) Reed-Solomon encode (polynomial 0x11D, Cauchy
generator), erasure reconstruction and a batched ragged-stripe launcher with
incremental parity update.

Modules:
  codec    equal-size shards: xor_encode, rs_encode, reconstruct, ShardPlan (a
           prepared call for repeated launches), host algebra
  layout   ragged tensor lists -> units -> stripes; batched encode/decode/update,
           and the drop-in entry points encode / decode / update
  checkpoint  ECLocalCheckpointManager + ErasureCodedStrategy (the repl_strategy slot)
  args     --non-persistent-ckpt-type in_memory: flags, validation, checkpointing context
"""
from . import _lib
from ._lib import ECError, ECLibraryMissing, SingularError
from .codec import (ShardPlan, cauchy_matrix, decode_matrix, gf_inv, gf_invert, gf_mul, matvec,
                    reconstruct, rs_encode, side_stream, xor_encode)
from .layout import ParitySet, StripeLayout, decode, encode, update

__all__ = [
    "ECError", "ECLibraryMissing", "SingularError", "ShardPlan", "cauchy_matrix", "decode_matrix",
    "gf_inv", "gf_invert", "gf_mul", "matvec", "reconstruct", "rs_encode", "side_stream",
    "xor_encode",
    "StripeLayout", "ParitySet", "encode", "decode", "update",
]


def library_path() -> str:
    return _lib.LIB_PATH
