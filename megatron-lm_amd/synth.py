"""Seeded synthetic checkpoint shards for the benchmark configurations.

The bytes stand in for serialized optimizer / parameter state: bf16 params
N(0, 0.02); fp32 master weights N(0, 0.02), Adam exp_avg N(0, 1e-3) and
exp_avg_sq |N(0, 1e-6)| (the tensors megatron/core/optimizer/distrib_optimizer.py:860-897
hands to the checkpoint).  Host generators use numpy ``default_rng(seed)``
(bf16 by round-to-nearest-even from fp32), so CPU and GPU runs see the same
bytes.  The multi-GB configurations are generated on the device with a seeded
torch generator instead (numpy would take minutes); the checks for those read
the same device bytes back.
"""
from __future__ import annotations

from typing import List, Tuple

import numpy as np

MiB = 1 << 20
GiB = 1 << 30


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round to nearest even."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    rounded = u + (np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1)))
    return (rounded >> np.uint32(16)).astype(np.uint16)


def normal_bytes(rng: np.random.Generator, nbytes: int, std: float, dtype: str,
                 absolute: bool = False) -> np.ndarray:
    """nbytes of little-endian bf16 or fp32 values drawn N(0, std)."""
    width = 2 if dtype == "bf16" else 4
    if nbytes % width:
        raise ValueError("nbytes must be a multiple of the element size")
    x = rng.standard_normal(nbytes // width, dtype=np.float32)
    x *= np.float32(std)
    if absolute:
        np.abs(x, out=x)
    if dtype == "bf16":
        return bf16_bits(x).view(np.uint8)
    return x.view(np.uint8)


def xor_shards(seed: int, shard_bytes: int = 64 * MiB, k: int = 4) -> List[np.ndarray]:
    """XOR config: k shards of bf16 N(0, 0.02) bytes."""
    rng = np.random.default_rng(seed)
    return [normal_bytes(rng, shard_bytes, 0.02, "bf16") for _ in range(k)]


# Shard j of the RS(6,3) config: (std, absolute) of its fp32 values.
RS63_KINDS = [(0.02, False), (0.02, False),   # master weights
              (1e-3, False), (1e-3, False),   # exp_avg
              (1e-6, True), (1e-6, True)]     # exp_avg_sq


def rs_shards(seed: int, shard_bytes: int = 256 * MiB, k: int = 6) -> List[np.ndarray]:
    """RS config: shards 0-1 fp32 master weights, 2-3 exp_avg, 4-5 exp_avg_sq
    (cycling for k != 6)."""
    rng = np.random.default_rng(seed)
    out = []
    for j in range(k):
        std, absolute = RS63_KINDS[j % len(RS63_KINDS)]
        out.append(normal_bytes(rng, shard_bytes, std, "fp32", absolute))
    return out


def erasures(seed: int, n: int = 9, e: int = 3) -> List[int]:
    """Seeded erasure positions among n shards."""
    return sorted(int(x) for x in np.random.default_rng(seed).choice(n, e, replace=False))


def gpt_rank_params(layers: int = 24, hidden: int = 2048, vocab: int = 50304,
                    seq: int = 2048) -> int:
    """Parameter count of a GPT with learned positions: embeddings, per-layer
    QKV/proj/MLP weights and biases with two layernorms, and a final norm."""
    per_layer = 12 * hidden * hidden + 13 * hidden
    return vocab * hidden + seq * hidden + layers * per_layer + 2 * hidden


def ragged_sizes(seed: int, n: int = 3000, lo: int = 4 << 10, hi: int = 64 * MiB) -> Tuple[np.ndarray, np.ndarray]:
    """Tensor byte sizes log-uniform on [lo, hi] and their dtypes (0 = bf16,
    1 = fp32); sizes are whole elements of their dtype."""
    rng = np.random.default_rng(seed)
    sizes = np.exp(rng.uniform(np.log(lo), np.log(hi), n))
    kinds = rng.integers(0, 2, n)
    width = np.where(kinds == 0, 2, 4)
    sizes = (np.floor(sizes / width) * width).astype(np.int64)
    return sizes, kinds


def perturbed_units(seed: int, n_units: int, fraction: float = 0.01) -> np.ndarray:
    """Seeded sorted choice of round(fraction * n_units) distinct unit indices."""
    rng = np.random.default_rng(seed)
    n = max(1, int(round(fraction * n_units)))
    return np.sort(rng.choice(n_units, n, replace=False))


# ------------------------------------------------------------ device data --

def device_normal_(buf, seed: int, std: float, dtype, absolute: bool = False):
    """Fill a device tensor of dtype bf16/fp32 with seeded N(0, std)."""
    import torch
    g = torch.Generator(device=buf.device)
    g.manual_seed(seed)
    buf.normal_(0.0, std, generator=g)
    if absolute:
        buf.abs_()
    return buf


def gpt_rank_buffer(device, seed: int, nbytes: int = None):
    """One DP rank's checkpoint buffer for GPT 1.3B as one uint8 tensor: the
    segments bf16 params | fp32 master | fp32 exp_avg | fp32 exp_avg_sq, in
    the 2:4:4:4 byte ratio of those states, scaled to ``nbytes`` (default the
    20.8e9 bytes quoted for this configuration; the exact model,
    gpt_rank_params() = 1,315,819,520 params at 14 B each, is 18.42e9)."""
    import torch
    total = int(20.8e9) if nbytes is None else int(nbytes)
    unit = total // 14
    seg = [2 * unit, 4 * unit, 4 * unit, 4 * unit]
    seg = [s - s % 4 for s in seg]
    buf = torch.empty(sum(seg), dtype=torch.uint8, device=device)
    off = 0
    specs = [(torch.bfloat16, 0.02, False), (torch.float32, 0.02, False),
             (torch.float32, 1e-3, False), (torch.float32, 1e-6, True)]
    for n, (dt, std, ab) in zip(seg, specs):
        device_normal_(buf[off: off + n].view(dt), seed + off, std, dt, ab)
        off += n
    return buf
