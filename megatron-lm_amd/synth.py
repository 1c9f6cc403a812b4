"""Seeded synthetic checkpoint shards for the benchmark configurations.

The bytes stand in for serialized optimizer / parameter state: bf16 params
N(0, 0.02); fp32 master weights N(0, 0.02), Adam exp_avg N(0, 1e-3) and
exp_avg_sq |N(0, 1e-6)| (the tensors megatron/core/optimizer/distrib_optimizer.py:860-897
hands to the checkpoint).  Every configuration is generated on the host with
numpy ``default_rng`` (bf16 by round-to-nearest-even from fp32), so CPU and
GPU runs see the same bytes.  The multi-GB configurations (the 20.8 GB rank
buffer, the 3,000 ragged tensors) are drawn in 64 MiB chunks, chunk c of a
segment from ``default_rng([seed, segment, c])``, on a thread pool: the bytes
do not depend on the thread count.
"""
from __future__ import annotations

import os
from concurrent.futures import ThreadPoolExecutor
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


def perturbation_bytes(seed: int, lengths) -> List[np.ndarray]:
    """The new bytes of a seeded perturbation: one uint8 array of lengths[n]
    uniform random bytes per changed unit n, drawn in one piece from
    default_rng([seed, 1]) (a stream apart from perturbed_units')."""
    lengths = np.asarray(lengths, np.int64).reshape(-1)
    flat = np.random.default_rng([seed, 1]).integers(0, 256, int(lengths.sum()), dtype=np.uint8)
    return np.split(flat, np.cumsum(lengths)[:-1])


# ------------------------------------------------- multi-GB host buffers --

GEN_CHUNK = 64 * MiB  # bytes per independently seeded chunk


def _threads(threads) -> int:
    return threads or max(1, min(16, len(os.sched_getaffinity(0))))


def _fill_chunk(out: np.ndarray, c0: int, seed: int, segment: int, std: float, dtype: str,
                absolute: bool) -> None:
    """Bytes [c0, c0 + GEN_CHUNK) of the uint8 array ``out``: dtype values
    N(0, std) (|N| with ``absolute``) from default_rng([seed, segment, chunk])."""
    c1 = min(out.size, c0 + GEN_CHUNK)
    rng = np.random.default_rng([seed, segment, c0 // GEN_CHUNK])
    if dtype == "fp32":
        x = out[c0:c1].view(np.float32)
        rng.standard_normal(out=x, dtype=np.float32)
    else:
        x = rng.standard_normal((c1 - c0) // 2, dtype=np.float32)
    x *= np.float32(std)
    if absolute:
        np.abs(x, out=x)
    if dtype == "bf16":
        out[c0:c1].view(np.uint16)[:] = bf16_bits(x)


def fill_normal(segments, seed: int, threads: int = 0) -> None:
    """Fill each (uint8 array, segment id, std, dtype, absolute) of
    ``segments`` chunk by chunk on a thread pool (numpy releases the
    interpreter lock while it draws)."""
    work = []
    for out, seg, std, dtype, absolute in segments:
        width = 2 if dtype == "bf16" else 4
        if out.size % width:
            raise ValueError("segment size must be a multiple of the element size")
        work += [(out, c0, seg, std, dtype, absolute) for c0 in range(0, out.size, GEN_CHUNK)]
    with ThreadPoolExecutor(_threads(threads)) as ex:
        for f in [ex.submit(_fill_chunk, o, c0, seed, seg, std, dt, ab)
                  for o, c0, seg, std, dt, ab in work]:
            f.result()


# Config 4's segments: (share of the 14 bytes per parameter, std, dtype, absolute)
GPT_SEGMENTS = [(2, 0.02, "bf16", False),   # bf16 params
                (4, 0.02, "fp32", False),   # fp32 master weights
                (4, 1e-3, "fp32", False),   # Adam exp_avg
                (4, 1e-6, "fp32", True)]    # Adam exp_avg_sq


def gpt_rank_buffer_host(seed: int, nbytes: int = None, threads: int = 0) -> np.ndarray:
    """One DP rank's checkpoint buffer for GPT 1.3B as one uint8 host array:
    the segments bf16 params | fp32 master | fp32 exp_avg | fp32 exp_avg_sq,
    in the 2:4:4:4 byte ratio of those states, scaled to ``nbytes`` (default
    the 20.8e9 bytes quoted for this configuration; the exact model,
    gpt_rank_params() = 1,315,819,520 params at 14 B each, is 18.42e9)."""
    total = int(20.8e9) if nbytes is None else int(nbytes)
    unit = total // 14
    seg = [share * unit - (share * unit) % 4 for share, *_ in GPT_SEGMENTS]
    buf = np.empty(sum(seg), np.uint8)
    parts, off = [], 0
    for i, (n, (_, std, dtype, absolute)) in enumerate(zip(seg, GPT_SEGMENTS)):
        parts.append((buf[off: off + n], i, std, dtype, absolute))
        off += n
    fill_normal(parts, seed, threads)
    return buf


def ragged_host(seed: int, threads: int = 0, n: int = 3000):
    """Config 5's tensors on the host: (block, views, kinds) where ``views``
    are the byte arrays of the tensors (sizes from ragged_sizes, back to back
    in one 64-byte-aligned block), bf16 N(0, 0.02) for kind 0, fp32
    N(0, 1e-3) for kind 1; tensor i is segment 5000 + i."""
    sizes, kinds = ragged_sizes(seed, n)
    starts = np.concatenate([[0], np.cumsum((sizes + 63) // 64 * 64)])
    raw = np.empty(int(starts[-1]) + 64, np.uint8)
    lead = (-raw.ctypes.data) % 64
    block = raw[lead: lead + int(starts[-1])]
    views = [block[int(a): int(a) + int(sz)] for a, sz in zip(starts[:-1], sizes)]
    fill_normal([(v, 5000 + i, 0.02 if kd == 0 else 1e-3, "bf16" if kd == 0 else "fp32", False)
                 for i, (v, kd) in enumerate(zip(views, kinds.tolist()))], seed, threads)
    return block, views, kinds


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
