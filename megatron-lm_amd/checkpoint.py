"""Erasure-coded local checkpoints: the ``repl_strategy`` slot, filled with a code.

The reference hands one rank's ``MCoreTensorAwareStateDict`` to an external
``LocalCheckpointManager(root, repl_strategy=...)``:

* construction, with ``CliqueReplicationStrategy`` as the redundancy policy:
  megatron/training/training.py:825-835;
* ``manager.save(tasd, iteration, is_async)``: megatron/training/checkpointing.py:538-541;
* ``manager.find_latest()``: megatron/training/checkpointing.py:864;
* ``manager.load() -> (tasd, name)``: megatron/training/checkpointing.py:891-894.

Its tests pin what the slot must do: per-rank files ``iter_{:07d}_{rank}_local*``
under ``root/<rank>/`` (tests/unit_tests/dist_checkpointing/test_replication.py:141-143);
loading iteration 1 after the local directories of some ranks were deleted
(:146-160); a failed save on one rank raising and loading nothing (test_local.py:246-326);
saving iteration 2 removing iteration 1 (test_local.py:225-244).

``ECLocalCheckpointManager`` keeps those call-site names and semantics.
``ErasureCodedStrategy`` replaces full replicas with an (k, m) erasure code over
each rank's ordered tensor list:

* the rank's tensors are cut into stripes of k units of ``unit_bytes``
  (``StripeLayout``) and m parity units are computed on the GPU;
* codeword position p (data 0..k-1, parity k..k+m-1) of the stripes of the
  rank at index i of the group's rank list is a *slice* of
  n_stripes * unit_bytes bytes held by the rank at index (i + p * jump) mod G,
  so the storage of any m ranks can be lost and every rank still decodes (the
  k + m holders must be distinct: G / gcd(jump, G) >= k + m);
* ``ErasureCodedStrategy.from_ec_params`` takes ``jump`` with the meaning of
  the reference's ``--replication-jump`` (megatron/training/arguments.py:2425-2429:
  copies of rank n go to n + J, n + 2J, ... in global ranks) and converts it
  to a spacing of group members (``index_jump``).  With ranks numbered
  node-major and J = ranks per node, the k + m slices of a rank sit on k + m
  different nodes, so losing up to m whole nodes still loads;
* storage is (k + m) / k of the data per rank, and a save moves
  (k + m - 1) / k of it over the network.  Replication with factor F stores
  F times the data and tolerates F - 1 losses.

Slices and inventories are exchanged as CPU tensors (send/recv, all_gather)
over a gloo group with the coding group's ranks (``comm_group``: the coding
group itself when it is gloo, a given gloo twin, or a private gloo group built
from the coding group's ranks, since the reference's data-parallel group is
NCCL), and files are written as a
JSON header plus raw bytes.  The one serialized object is the hollow state of
a ``MCoreTensorAwareStateDict`` (its non-tensor part, torch.save), stored
with the slices so that ``load`` returns the object it was given, as the
reference's local manager does.  The GPU work (encode, gather of units into
slices, scatter and reconstruction on load) goes through the engine's C ABI;
the ``codec`` argument exists so the exchange can be tested without a GPU.
"""
from __future__ import annotations

import atexit
import io
import json
import os
import re
import threading
import time
import weakref
from dataclasses import dataclass, field
from pathlib import Path
from typing import Callable, Dict, List, NamedTuple, Optional, Sequence, Tuple

import numpy as np
import torch
import torch.distributed as dist

GENERATOR_ID = "gf256-0x11d-cauchy1"
_MAGIC = b"ECMI355\x00"
_NAME_RE = re.compile(r"^iter_(\d{7})_(\d+)_local\.ec(\d+)$")


class CheckpointingException(RuntimeError):
    """A save or load that did not complete on every rank of the group."""


# ----------------------------------------------------------------- state --

@dataclass
class TensorListState:
    """The part of a tensor-aware state dict the redundancy step sees: an
    ordered list of tensors (MCoreTensorAwareStateDict.tensors order,
    megatron/core/dist_checkpointing/tensor_aware_state_dict.py:162-184) and
    a JSON-able ``common`` dict that travels with them."""
    tensors: List[torch.Tensor]
    common: dict = field(default_factory=dict)

    def pop_tensors(self) -> List[torch.Tensor]:
        t, self.tensors = self.tensors, []
        return t

    def insert_tensors(self, tensors: Sequence[torch.Tensor]) -> None:
        if self.tensors:
            raise ValueError("state already holds tensors")
        self.tensors = list(tensors)

    @property
    def is_hollow(self) -> bool:
        return not self.tensors


def _tensor_meta(tensors: Sequence[torch.Tensor]) -> list:
    return [{"dtype": str(t.dtype).replace("torch.", ""), "shape": list(t.shape),
             "nbytes": t.numel() * t.element_size()} for t in tensors]


def _dtype(name: str) -> torch.dtype:
    dt = getattr(torch, name, None)
    if not isinstance(dt, torch.dtype):
        raise CheckpointingException(f"unknown dtype {name!r} in checkpoint header")
    return dt


# ----------------------------------------------------------------- codec --

_staging_threads: "weakref.WeakSet[threading.Thread]" = weakref.WeakSet()


def _join_staging_threads() -> None:
    """At interpreter exit: let background staging finish (its transfers
    land and its threads end) before the hook that waits for the engine's
    streams and devices (codec._finish_side_streams, registered earlier, at
    that module's import, so it runs after this one)."""
    for t in list(_staging_threads):
        t.join()


atexit.register(_join_staging_threads)


class PendingSlices:
    """The slices of a ``GpuSliceCodec.snapshot``, being staged to host memory
    by a background thread.  ``coded`` is the device event after which the
    tensors may change; ``result()`` waits for the staging and returns
    ``(meta, slices)`` (or raises what the staging raised)."""

    def __init__(self, coded: torch.cuda.Event,
                 stage: Optional[Callable[[], Tuple[dict, list]]] = None,
                 ready: Optional[Tuple[dict, list]] = None):
        """``stage`` runs in the background thread and returns ``(meta,
        slices)``; without it ``ready`` is the result, available at once."""
        self.coded = coded
        self._result: Optional[Tuple[dict, list]] = ready
        self._error: Optional[BaseException] = None
        self._done = threading.Event()
        self._thread: Optional[threading.Thread] = None
        if stage is None:
            self._done.set()
            return
        self._thread = threading.Thread(target=self._run, args=(stage,), daemon=True,
                                        name="ec-stage")
        _staging_threads.add(self._thread)
        self._thread.start()

    def _run(self, stage) -> None:
        try:
            self._result = stage()
        except BaseException as e:  # noqa: BLE001 - handed to result()
            self._error = e
        finally:
            self._done.set()

    def done(self) -> bool:
        return self._done.is_set()

    def staged_event(self) -> threading.Event:
        """An event set once the staging has ended (its transfers have landed
        or it failed); holding it does not keep the slices alive."""
        return self._done

    def result(self, timeout: Optional[float] = None) -> Tuple[dict, List[np.ndarray]]:
        if not self._done.wait(timeout):
            raise TimeoutError("checkpoint slices still being staged")
        if self._thread is not None:
            self._thread.join()
        if self._error is not None:
            raise self._error
        return self._result


def _lib_call(name: str, coeff: np.ndarray, *args) -> None:
    """Call the batched entry point ``name`` of the C ABI with a host
    coefficient matrix first and (stream, device) last."""
    from . import _lib
    from .codec import stream_handle
    *rest, stream, dev = args
    _lib.check(getattr(_lib.lib(), name)(_lib.u8ptr(np.ascontiguousarray(coeff, np.uint8)), *rest,
                                         stream_handle(stream, dev)), name)


class GpuSliceCodec:
    """Encode a rank's tensors into k + m slices and back, on the GPU.

    Slice p is the concatenation over stripes of codeword position p (units
    zero-padded to ``unit_bytes``): n_stripes * unit_bytes bytes, returned as
    rows of one pageable host array.

    ``encode`` codes the state into one (k + m) / k block in HBM when that
    fits (see ``snapshot``) and stages it with ``ec_stage_stripes_to_host``;
    otherwise the work goes in chunks of stripes of at most ``chunk_bytes``,
    double-buffered on the device and in pinned host memory: 2 * chunk_bytes
    of extra HBM and of page-locked memory.  ``decode`` likewise takes one
    (k, stripes, unit_bytes) block when it fits, else chunks, and moves the
    slices up with ``ec_stage_to_device``.

    The slices own their host array (they are views of it): the codec keeps
    no reference to an array it handed out, so nothing the caller holds,
    even only by address, is written again behind its back.  A caller done
    with the slices hands the array back with ``release(slices)``, and the
    next encode of the same shape writes into it: a fresh array costs the
    kernel's page faults and zeroing on first touch, which on a 27 GB
    checkpoint halves the staging rate.

    Encode, per chunk: one launch writes the parity units into the device
    buffer's parity rows and, in the same pass over the data, the data units
    (zero-padded) into its data rows; the buffer goes to pinned memory on a
    copy stream, and four threads move it into the result while the next
    chunk is coded and transferred.  Decode, per chunk (one, when the block
    fits): ``ec_stage_to_device`` moves the k slices' part up, one scatter
    launch puts the data rows into fresh tensors and one decode launch
    rebuilds the lost data positions.

    ``snapshot`` is the save path that keeps training running: it codes the
    whole state into one HBM block (288 GB of HBM per MI355X holds a rank's
    (k + m) / k copy) on a stream with its own hardware queue, holds torch's
    stream only for that launch, and stages the block to host memory
    in a background thread while training goes on.  Transfers use ordinary
    streams: issued on the CU-masked side stream they held the host and
    slowed the training kernels beside them."""

    def __init__(self, k: int, m: int, unit_bytes: int, chunk_bytes: int = 1 << 30,
                 snapshot_bytes: Optional[int] = None, keep_block: bool = False):
        from . import layout as _layout
        self._layout = _layout
        self.k, self.m, self.unit_bytes = k, m, unit_bytes
        self.chunk_bytes = chunk_bytes
        self.snapshot_bytes = snapshot_bytes
        self.keep_block = keep_block
        self.stage_threads = 8   # host threads of the staging calls
        self._free: Optional[np.ndarray] = None   # released by the caller, reusable
        self._host_lock = threading.Lock()
        self._last_layout = None   # descriptors of the last encode, without its tensors
        self._last_ptrs = None     # (block key, parity table, data table) of the last snapshot
        # keep_block: (block, event set when its staging has ended) of the last
        # save, when that save coded the whole state into one block (the
        # snapshot path).  Not the PendingSlices itself: that holds the slices,
        # and the codec keeps no reference to a host array it handed out.
        self._resident: Optional[Tuple[torch.Tensor, threading.Event]] = None
        # ec_stage_last_stats of the last staging call (a diagnostic: the
        # transfer waits, host copies and device time of that call)
        self.last_stage_stats: Optional[dict] = None

    def _stripe_layout(self, tensors: List[torch.Tensor]):
        """(layout, reused): the StripeLayout of the tensors to encode, and
        whether they occupy the same device bytes as at the last encode (a
        training run saves the same buffers every time).  Then its
        descriptors are reused: no descriptor build and no upload on the path
        that holds training."""
        prev = self._last_layout
        lay = prev.rebind(tensors) if prev is not None else None
        if lay is not None:
            return lay, True
        lay = self._layout.StripeLayout(tensors, self.k, self.m, self.unit_bytes)
        self._last_layout = lay.descriptors_only()
        return lay, False

    def _host_out(self, shape: Tuple[int, int]) -> np.ndarray:
        """The released host array when it has this shape, else a new one.
        A released array of another shape is dropped."""
        with self._host_lock:
            buf, self._free = self._free, None
        if buf is not None and buf.shape == shape:
            return buf
        del buf
        return np.empty(shape, np.uint8)

    def release(self, slices: Sequence[np.ndarray]) -> None:
        """Hand back the host array of the k + m slices an ``encode`` or a
        ``snapshot`` returned, for the next encode of the same shape to write
        into.  The caller must not use the slices (or their memory) after
        this.  ValueError for anything that is not one encode's slices."""
        slices = list(slices)
        if not slices:
            return
        base = slices[0].base
        if (not isinstance(base, np.ndarray) or base.ndim != 2 or base.dtype != np.uint8
                or len(slices) != base.shape[0]
                or any(sl.base is not base or sl.size != base.shape[1] for sl in slices)):
            raise ValueError("release() takes the slices of one encode or snapshot")
        with self._host_lock:
            self._free = base

    def _chunk_stripes(self, n_stripes: int, rows: int) -> int:
        return max(1, min(n_stripes, self.chunk_bytes // (rows * self.unit_bytes)))

    @staticmethod
    def _rows(block: torch.Tensor, p: int) -> np.ndarray:
        """Device addresses of the units of row p of a (rows, stripes,
        unit_bytes) device block."""
        S, U = block.shape[1], block.shape[2]
        return np.uint64(block[p].data_ptr()) + np.arange(S, dtype=np.uint64) * np.uint64(U)

    def _block_ptrs(self, block: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        """(parity, data) unit-address tables of a snapshot block.  They
        depend only on the block's address and shape, and the caching
        allocator usually hands the same block back at the next save, so the
        last pair is kept and reused when it matches."""
        key = (block.device, block.data_ptr(), tuple(block.shape))
        last = self._last_ptrs
        if last is not None and last[0] == key:
            return last[1], last[2]
        with torch.cuda.device(block.device):
            pp = self._unit_ptrs(block, self.k, self.m)
            gp = self._unit_ptrs(block, 0, self.k)
        self._last_ptrs = (key, pp, gp)
        return pp, gp

    @staticmethod
    def _unit_ptrs(block: torch.Tensor, first: int, count: int) -> torch.Tensor:
        """[stripes, count] device addresses of positions first .. first +
        count - 1 of every stripe of a stripe-major (stripes, positions,
        unit_bytes) device block, computed on the device (no host array, no
        upload)."""
        S, P, U = block.shape
        stripe = torch.arange(S, dtype=torch.int64, device=block.device).unsqueeze(1) * (P * U)
        pos = torch.arange(first, first + count, dtype=torch.int64,
                           device=block.device).unsqueeze(0) * U
        return (stripe + pos).add_(block.data_ptr())

    @staticmethod
    def _dev(a: np.ndarray, dt, device) -> torch.Tensor:
        return torch.from_numpy(np.ascontiguousarray(a).view(dt)).to(device)

    def _snapshot_limit(self, dev) -> int:
        """Largest snapshot block: ``snapshot_bytes``, or by default the
        device's free memory plus what torch's allocator holds unused, less
        an eighth of the device."""
        if self.snapshot_bytes is not None:
            return self.snapshot_bytes
        free, total = torch.cuda.mem_get_info(dev)
        idle = torch.cuda.memory_reserved(dev) - torch.cuda.memory_allocated(dev)
        return free + idle - total // 8

    def _meta(self, lay, tensors) -> dict:
        return {"k": self.k, "m": self.m, "unit_bytes": self.unit_bytes,
                "n_stripes": lay.n_stripes, "n_units": lay.n_units,
                "tensors": _tensor_meta(tensors), "generator": GENERATOR_ID}

    def encode(self, tensors: Sequence[torch.Tensor],
               changed_tensors: Optional[Sequence[int]] = None) -> Tuple[dict, List[np.ndarray]]:
        """Code the tensors into k + m slices in host memory; returns when
        they are there.  Through one HBM block when it fits (``snapshot``,
        waited for), else in bounded chunks: the same slices either way.
        ``changed_tensors`` as for ``snapshot``."""
        return self.snapshot(tensors, changed_tensors=changed_tensors).result()

    def _encode_chunked(self, tensors: Sequence[torch.Tensor]) -> Tuple[dict, List[np.ndarray]]:
        """Code and stage in bounded chunks of stripes; returns when the slices
        are in host memory.  Each chunk is one copying-encode launch on torch's
        current stream (ordered after the work that produced the tensors) into
        a stripe-major (stripes, k + m, unit_bytes) device buffer, which
        ``ec_stage_stripes_to_host`` then moves into the slice rows (on a
        copy engine, after the chunk's coding, which an ordinary stream
        carries).  Two buffers alternate: chunk n + 1 is coded while chunk
        n is staged."""
        from . import _lib
        from .codec import stream_handle
        k, m, U = self.k, self.m, self.unit_bytes
        tensors = list(tensors)
        lay, _ = self._stripe_layout(tensors)
        S, dev = lay.n_stripes, lay.device
        C = self._chunk_stripes(S, k + m)
        chunks = [(c0, min(C, S - c0)) for c0 in range(0, S, C)]
        nb = min(2, len(chunks))
        out = self._host_out((k + m, S * U))
        rows = [out[p].ctypes.data for p in range(k + m)]
        with torch.cuda.device(dev):
            # the staging follows xfer's work (a wait for the chunk's coding)
            comp, xfer = torch.cuda.current_stream(dev), torch.cuda.Stream(dev)
            bufs = [torch.empty((C, k + m, U), dtype=torch.uint8, device=dev) for _ in range(nb)]
            pp = [self._unit_ptrs(b, k, m) for b in bufs]
            gp = [self._unit_ptrs(b, 0, k) for b in bufs]
            for b in bufs:
                b.record_stream(xfer)
            pinned = torch.empty(min(2 * self.chunk_bytes, 2 * C * (k + m) * U),
                                 dtype=torch.uint8, pin_memory=True)

            def code(n):
                c0, c = chunks[n]
                b = n % nb
                _lib.check(_lib.lib().ec_encode_batched_copy(
                    _lib.u8ptr(lay.coeff), k, m, lay.d_ptrs.data_ptr() + c0 * k * 8,
                    lay.d_len.data_ptr() + c0 * k * 4, pp[b].data_ptr(), gp[b].data_ptr(), c,
                    U, stream_handle(comp, dev)), "ec_encode_batched_copy")
                ready = torch.cuda.Event()
                ready.record(comp)
                return ready

            ready = code(0)
            for n, (c0, c) in enumerate(chunks):
                xfer.wait_event(ready)
                # the other buffer's last chunk (n - 1) was staged by the call
                # before, which returned once its bytes were in host memory
                ready = code(n + 1) if n + 1 < len(chunks) else None
                _lib.check(_lib.lib().ec_stage_stripes_to_host(
                    bufs[n % nb].data_ptr(), c, k + m, U,
                    _lib.ptr_array([r + c0 * U for r in rows]), pinned.data_ptr(),
                    pinned.numel(), self.stage_threads, stream_handle(xfer, dev)),
                    "ec_stage_stripes_to_host")
        return self._meta(lay, tensors), [out[p] for p in range(k + m)]

    def snapshot(self, tensors: Sequence[torch.Tensor], hold: bool = True,
                 changed_tensors: Optional[Sequence[int]] = None) -> "PendingSlices":
        """Code the tensors into one stripe-major (stripes, k + m, unit_bytes)
        block in HBM and stage it to host memory in the background.

        One launch (parity plus the copy of every data unit, one read of the
        data) runs on the device's side stream (its own hardware queue) after
        the work already enqueued on torch's current stream; with ``hold`` the
        current stream then waits for it, so later work there (the next
        optimizer step) cannot change the tensors before they are coded.  That
        wait is the whole stall of a save: the block is (k + m) / k of the
        state in HBM, written at HBM speed (stripe-major, so that the k + m
        units a workgroup writes are adjacent: faster than k + m separate
        rows).  A background thread moves the block to host memory, one
        (k + m, stripes * unit_bytes) host array whose row p is slice p, and
        frees it;
        ``PendingSlices.result()`` returns ``(meta, slices)`` as ``encode``
        would.  Without ``hold`` the caller must order its own writes after
        ``PendingSlices.coded``.

        When the block is larger than ``snapshot_bytes`` (by default: than
        what leaves an eighth of the device's memory free, so that the next
        training steps keep their room) or the allocator cannot provide it,
        the state is coded and staged by ``encode`` before this returns (the
        bounded chunked path: a longer stall, the same slices), and the
        result is ready at once.

        Incremental saves (a codec built with ``keep_block``): the block
        stays in HBM after staging, holding the last save's data units and
        parity.  A save that passes ``changed_tensors`` (indices into
        ``tensors`` of every tensor whose bytes may differ from the last
        save's) over the same device bytes as the last save (the same
        addresses and sizes, in order) then codes only those tensors' units:
        ``ec_parity_update`` folds new XOR old (the block's copy) into the
        block's parity, and the new units are copied into the block, so it
        again holds the whole state coded, and is staged as above.  The
        slices are those a full encode gives, as long as no tensor outside
        ``changed_tensors`` changed: the caller vouches for that.  Anything
        else (no block from the last save, other tensors, no
        ``changed_tensors``) takes the full encode.  The update waits for the
        last save's staging to finish reading the block."""
        from .codec import side_stream
        k, m, U = self.k, self.m, self.unit_bytes
        tensors = list(tensors)
        lay, reused = self._stripe_layout(tensors)
        S, dev = lay.n_stripes, lay.device
        cur = torch.cuda.current_stream(dev)
        res, self._resident = self._resident, None
        if (changed_tensors is not None and self.keep_block and reused and res is not None
                and tuple(res[0].shape) == (S, k + m, U) and res[0].device == dev):
            return self._snapshot_delta(lay, tensors, res, changed_tensors, hold)
        del res
        block = None
        if (k + m) * S * U <= self._snapshot_limit(dev):
            try:
                with torch.cuda.device(dev):
                    block = torch.empty((S, k + m, U), dtype=torch.uint8, device=dev)
            except torch.OutOfMemoryError:
                block = None
        if block is None:
            ready = self._encode_chunked(tensors)
            coded = torch.cuda.Event()
            coded.record(cur)
            return PendingSlices(coded, ready=ready)
        side = side_stream(dev)
        pp, gp = self._block_ptrs(block)
        for t in (block, pp, gp, lay.d_ptrs, lay.d_len):
            t.record_stream(side)
        side.wait_stream(cur)   # the tensors' producers and the descriptor uploads
        _lib_call("ec_encode_batched_copy", lay.coeff, k, m, lay.d_ptrs.data_ptr(),
                  lay.d_len.data_ptr(), pp.data_ptr(), gp.data_ptr(), S, U, side, dev)
        return self._stage_block(lay, tensors, block, side, cur, hold)

    def _stage_block(self, lay, tensors, block: torch.Tensor, side, cur,
                     hold: bool) -> "PendingSlices":
        """The end of a snapshot once its kernels are enqueued on ``side``:
        the ``coded`` event (torch's stream waits for it with ``hold``), and a
        background thread staging the block to host memory.  With
        ``keep_block`` the block is kept for the next save."""
        from . import _lib
        from .codec import stream_handle
        k, m, U = self.k, self.m, self.unit_bytes
        S, dev = lay.n_stripes, lay.device
        coded = torch.cuda.Event()
        coded.record(side)
        if hold:
            cur.wait_event(coded)

        def stage():
            nonlocal block
            # tensor shapes and dtypes cannot change in place: read them here,
            # off the caller's critical path
            meta = self._meta(lay, tensors)
            out = self._host_out((k + m, S * U))
            pinned = torch.empty(min(2 * self.chunk_bytes, 2 * (k + m) * S * U),
                                 dtype=torch.uint8, pin_memory=True)
            # One foreign call that holds no interpreter lock: it waits for
            # xfer's work (the coding), then copies on an SDMA engine, which
            # leaves training's hardware queue alone.
            with torch.cuda.device(dev):
                xfer = torch.cuda.Stream(dev)
                xfer.wait_event(coded)
                block.record_stream(xfer)
                _lib.check(_lib.lib().ec_stage_stripes_to_host(
                    block.data_ptr(), S, k + m, U,
                    _lib.ptr_array([out[p].ctypes.data for p in range(k + m)]),
                    pinned.data_ptr(), pinned.numel(), self.stage_threads,
                    stream_handle(xfer, dev)), "ec_stage_stripes_to_host")
            self.last_stage_stats = _lib.last_stage_stats()
            block = None   # back to the allocator (unless kept): the last transfer has landed
            return meta, [out[p] for p in range(k + m)]

        kept = block
        pending = PendingSlices(coded, stage)
        if self.keep_block:
            self._resident = (kept, pending.staged_event())
        del kept
        return pending

    def _snapshot_delta(self, lay, tensors, res, changed_tensors,
                        hold: bool) -> "PendingSlices":
        """The incremental save of ``snapshot``: the changed tensors' units
        folded into the kept block (parity update, then the copy of the new
        units), on the side stream."""
        from .codec import side_stream
        block, staged = res
        staged.wait()   # the last save's staging has read the block
        k, m, U = self.k, self.m, self.unit_bytes
        S, dev = lay.n_stripes, lay.device
        cur = torch.cuda.current_stream(dev)
        side = side_stream(dev)
        ct = np.unique(np.asarray(changed_tensors, np.int64).reshape(-1))
        if ct.size and (ct[0] < 0 or ct[-1] >= len(tensors)):
            raise ValueError(f"changed_tensors must index the {len(tensors)} tensors")
        units = np.flatnonzero(np.isin(lay.unit_tensor, ct))
        desc = ()
        if units.size:
            stripe, pos = units // k, units % k
            st, inv = np.unique(stripe, return_inverse=True)
            base, row = np.uint64(block.data_ptr()), np.uint64((k + m) * U)
            old = base + stripe.astype(np.uint64) * row + pos.astype(np.uint64) * np.uint64(U)
            nptr = np.zeros((st.size, k), np.uint64)
            optr = np.zeros((st.size, k), np.uint64)
            ln = np.zeros((st.size, k), np.uint32)
            nptr[inv, pos] = lay.host_ptrs[stripe, pos]
            optr[inv, pos] = old
            ln[inv, pos] = lay.host_len[stripe, pos]
            pptr = (base + st.astype(np.uint64)[:, None] * row
                    + (np.uint64(k) + np.arange(m, dtype=np.uint64))[None, :] * np.uint64(U))
            full = np.full(units.size, U, np.uint32)
            with torch.cuda.device(dev):
                up = self._layout._upload
                desc = (up(nptr.view(np.int64), dev), up(optr.view(np.int64), dev),
                        up(ln.view(np.int32), dev), up(pptr.view(np.int64), dev),
                        up(lay.host_ptrs[stripe, pos].view(np.int64), dev),
                        up(lay.host_len[stripe, pos].view(np.int32), dev),
                        up(old.view(np.int64), dev), up(full.view(np.int32), dev))
        for t in (block,) + desc:
            t.record_stream(side)
        side.wait_stream(cur)   # the tensors' producers and the descriptor uploads
        if units.size:
            d_n, d_o, d_l, d_p, d_src, d_srclen, d_dst, d_full = desc
            # parity ^= C (new ^ old), old being the block's copy of each unit
            _lib_call("ec_parity_update", lay.coeff, k, m, d_n.data_ptr(), d_o.data_ptr(),
                      d_l.data_ptr(), d_p.data_ptr(), int(st.size), U, side, dev)
            # then the new units over the old ones, zero-padded (a 1 x 1 decode)
            _lib_call("ec_decode_batched", np.ones((1, 1), np.uint8), 1, 1, d_src.data_ptr(),
                      d_srclen.data_ptr(), d_dst.data_ptr(), d_full.data_ptr(),
                      int(units.size), U, side, dev)
        return self._stage_block(lay, tensors, block, side, cur, hold)

    def decode(self, meta: dict, slices: Dict[int, np.ndarray], device) -> List[torch.Tensor]:
        from . import _lib
        from .codec import decode_matrix, stream_handle
        k, m, U, S = meta["k"], meta["m"], meta["unit_bytes"], meta["n_stripes"]
        if len(slices) < k:
            raise CheckpointingException(f"only {len(slices)} of the {k} slices needed")
        avail = sorted(slices)[:k]
        for p in avail:
            if slices[p].size != S * U:
                raise CheckpointingException(f"slice {p} has {slices[p].size} bytes, not {S * U}")
        tensors = [torch.empty(tm["shape"], dtype=_dtype(tm["dtype"]), device=device)
                   for tm in meta["tensors"]]
        lay = self._layout.StripeLayout(tensors, k, m, U, device=device)
        if lay.n_stripes != S or lay.n_units != meta["n_units"]:
            raise CheckpointingException("checkpoint header does not match its tensors")
        have = [(r, p) for r, p in enumerate(avail) if p < k]
        lost_data = [p for p in range(k) if p not in avail]
        rows = None
        if lost_data:
            erased = [p for p in range(k + m) if p not in avail]
            surv, rows = decode_matrix(lay.coeff, erased)
            if surv != avail:
                raise CheckpointingException("decode plan does not match the slices read")
            rows = np.ascontiguousarray(rows[[erased.index(p) for p in lost_data]])
        # One chunk when the (k, S, U) block fits beside training (the bound of
        # snapshot), else chunks of at most chunk_bytes, double-buffered.
        C = S if k * S * U <= self._snapshot_limit(device) else self._chunk_stripes(S, k)
        one = np.ones((1, 1), np.uint8)
        hp = [p for _, p in have]
        src = [np.ascontiguousarray(slices[p]).reshape(-1) for p in avail]
        with torch.cuda.device(device):
            comp, copy = torch.cuda.current_stream(device), torch.cuda.Stream(device)
            while True:
                chunks = [(c0, min(C, S - c0)) for c0 in range(0, S, C)]
                nb = min(2, len(chunks))
                try:
                    bufs = [torch.empty((k, C, U), dtype=torch.uint8, device=device)
                            for _ in range(nb)]
                    break
                except torch.OutOfMemoryError:
                    if C == self._chunk_stripes(S, k):
                        raise
                    C = self._chunk_stripes(S, k)
            for bf in bufs:
                bf.record_stream(copy)
            pinned = torch.empty(min(2 * self.chunk_bytes, 2 * k * C * U), dtype=torch.uint8,
                                 pin_memory=True)
            # Every descriptor array is uploaded once, stripe-major, so that a
            # chunk's descriptors are a contiguous slice (a pointer offset).
            full = torch.full((C * k,), U, dtype=torch.int32, device=device)
            scat_src = [self._dev(np.stack([self._rows(bf, r) for r, _ in have], axis=1)
                                  if have else np.zeros(1, np.uint64), np.int64, device)
                        for bf in bufs]
            scat_dst = self._dev(lay.host_ptrs[:, hp], np.int64, device)
            scat_len = self._dev(lay.host_len[:, hp], np.int32, device)
            dec_src = [self._dev(np.stack([self._rows(bf, r) for r in range(k)], axis=1),
                                 np.int64, device) for bf in bufs]
            dec_dst = self._dev(lay.host_ptrs[:, lost_data], np.int64, device)
            dec_len = self._dev(lay.host_len[:, lost_data], np.int32, device)
            consumed: List[torch.cuda.Event] = []  # chunk n is decoded out of bufs[n % nb]
            for n, (c0, c) in enumerate(chunks):
                b = n % nb
                if n >= nb:
                    copy.wait_event(consumed[n - nb])  # device buffer b is free again
                # the k slices' part of the chunk into the buffer's rows, in one
                # native call (host threads fill pinned halves, the copy stream
                # sends them up); it returns once the bytes are on the device
                _lib.check(_lib.lib().ec_stage_to_device(
                    _lib.ptr_array([a.ctypes.data + c0 * U for a in src]), k, c * U,
                    bufs[b].data_ptr(), C * U, pinned.data_ptr(), pinned.numel(),
                    self.stage_threads, stream_handle(copy, device)), "ec_stage_to_device")
                self.last_stage_stats = _lib.last_stage_stats()
                comp.wait_stream(copy)
                if have:  # the data slices we have go into the tensors
                    h = len(have)
                    _lib.check(_lib.lib().ec_decode_batched(
                        _lib.u8ptr(one), 1, 1, scat_src[b].data_ptr(), full.data_ptr(),
                        scat_dst.data_ptr() + c0 * h * 8, scat_len.data_ptr() + c0 * h * 4,
                        c * h, U, stream_handle(comp, device)), "ec_decode_batched (scatter)")
                if lost_data:  # rebuild the missing data positions from the k rows
                    nl = len(lost_data)
                    _lib.check(_lib.lib().ec_decode_batched(
                        _lib.u8ptr(rows), k, nl, dec_src[b].data_ptr(), full.data_ptr(),
                        dec_dst.data_ptr() + c0 * nl * 8, dec_len.data_ptr() + c0 * nl * 4,
                        c, U, stream_handle(comp, device)), "ec_decode_batched")
                consumed.append(torch.cuda.Event())
                consumed[-1].record(comp)
            comp.synchronize()
        return tensors


# -------------------------------------------------------------- strategy --

def _is_gloo(group) -> bool:
    """Whether CPU tensors in collectives on ``group`` (None: the default
    group) go to gloo: a gloo group, or a multi-device group with a gloo
    part ("cpu:gloo,cuda:nccl")."""
    try:
        return "gloo" in str(dist.get_backend(group)).lower()
    except (RuntimeError, ValueError):
        return False


# One private gloo group per rank set and default group, created by the
# members only (use_local_synchronization): its name is a hash of the ranks,
# so a second group over the same ranks cannot be created in this process.
_private_gloo: Dict[Tuple[int, ...], Tuple[object, object]] = {}
_private_gloo_lock = threading.Lock()


def private_gloo_group(ranks: Sequence[int]):
    """A gloo group over ``ranks`` that only the erasure-coded checkpoint
    code uses, created on first use by the members (collective over them
    only) and kept for the life of the default group.  Raises
    CheckpointingException if gloo cannot build it."""
    key = tuple(sorted(int(r) for r in ranks))
    world = dist.group.WORLD
    with _private_gloo_lock:
        hit = _private_gloo.get(key)
        if hit is not None and hit[0] is world:
            return hit[1]
        try:
            g = dist.new_group(ranks=list(key), backend="gloo", use_local_synchronization=True)
        except (RuntimeError, ValueError) as e:
            raise CheckpointingException(
                f"cannot create a gloo group over ranks {list(key)} for the checkpoint "
                f"exchange: {e}") from e
        _private_gloo[key] = (world, g)
        return g


def index_jump(ranks: Sequence[int], jump: int) -> int:
    """The group-index spacing that puts consecutive holders at least
    ``jump`` global ranks apart, for the reference's ``--replication-jump``
    (megatron/training/arguments.py:2425-2429: copies of rank n go to n + J,
    n + 2J, ...) applied to a coding group whose members are evenly spaced
    (a data-parallel group: stride TP x PP, or 1).  ceil(jump / stride).
    Raises CheckpointingException for a jump above 1 on a group whose ranks
    are not evenly spaced."""
    if jump < 1:
        raise ValueError("jump must be positive")
    r = sorted(int(x) for x in ranks)
    if jump == 1 or len(r) < 2:
        return 1
    strides = {b - a for a, b in zip(r, r[1:])}
    if len(strides) != 1:
        raise CheckpointingException(
            f"a global-rank jump of {jump} needs evenly spaced group ranks, got {r}; "
            "pass a group-index jump to ErasureCodedStrategy instead")
    s = strides.pop()
    return -(-jump // s)


class ErasureCodedStrategy:
    """(k, m) erasure code over each rank's tensors; slice p of the rank at
    index i of the group's rank list is held by the rank at index
    (i + p * jump) mod G (see module docstring).  ``jump`` here counts group
    members; ``from_ec_params`` takes the reference's global-rank spacing.

    ``group`` is the coding group (in Megatron the data-parallel group with
    context parallelism, an NCCL group).  The exchange moves CPU tensors, so
    every collective runs on a gloo group over the same ranks: ``gloo_group``
    when given (Megatron's ``get_data_parallel_group_gloo(
    with_context_parallel=True)``, megatron/core/parallel_state.py:1258), else
    ``group`` itself when its backend takes CPU tensors (gloo), else a
    private gloo group built from ``group``'s ranks on first use
    (``private_gloo_group``)."""

    def __init__(self, k: int, m: int, unit_bytes: int = 4 << 20,
                 group: Optional[dist.ProcessGroup] = None, codec=None, jump: int = 1,
                 gloo_group: Optional[dist.ProcessGroup] = None):
        if k < 1 or m < 1:
            raise ValueError("k and m must be positive")
        if jump < 1:
            raise ValueError("jump must be positive")
        self.k, self.m, self.unit_bytes = k, m, unit_bytes
        self.group, self.jump = group, jump
        self.gloo_group = gloo_group
        self._comm: Optional[Tuple[object]] = None
        self.codec = codec if codec is not None else GpuSliceCodec(k, m, unit_bytes)

    @classmethod
    def from_ec_params(cls, k: int, m: int, unit_bytes: int = 4 << 20, jump: int = 1,
                       group: Optional[dist.ProcessGroup] = None,
                       gloo_group: Optional[dist.ProcessGroup] = None,
                       codec=None) -> "ErasureCodedStrategy":
        """Counterpart of the reference's
        ``CliqueReplicationStrategy.from_replication_params(jump, factor)``
        (megatron/training/training.py:826-828): the code's shape replaces the
        replication factor, and ``jump`` has the meaning of
        ``--replication-jump``, a spacing in global ranks, converted to a
        spacing in the group's members by ``index_jump``.  With jump = ranks
        per node (ranks numbered node-major) consecutive holders of a rank's
        slices sit on different nodes."""
        members = dist.get_process_group_ranks(group) if group is not None \
            else list(range(dist.get_world_size()))
        return cls(k, m, unit_bytes, group=group, codec=codec, jump=index_jump(members, jump),
                   gloo_group=gloo_group)

    # group helpers
    def ranks(self) -> List[int]:
        if self.group is None:
            return list(range(dist.get_world_size()))
        return dist.get_process_group_ranks(self.group)

    def comm_group(self):
        """The gloo group every CPU-tensor collective of the manager runs on
        (None: the default group, when that is gloo).  Resolved once."""
        if self._comm is None:
            if self.gloo_group is not None:
                if not _is_gloo(self.gloo_group):
                    raise CheckpointingException(
                        f"gloo_group has backend {dist.get_backend(self.gloo_group)!r}, not gloo")
                if sorted(dist.get_process_group_ranks(self.gloo_group)) != sorted(self.ranks()):
                    raise CheckpointingException(
                        "gloo_group does not have the ranks of the coding group")
                self._comm = (self.gloo_group,)
            elif _is_gloo(self.group):
                self._comm = (self.group,)
            else:
                self._comm = (private_gloo_group(self.ranks()),)
        return self._comm[0]

    def holder(self, owner: int, pos: int) -> int:
        r = self.ranks()
        return r[(r.index(owner) + pos * self.jump) % len(r)]

    def check_group(self) -> None:
        g = len(self.ranks())
        # (r + p * jump) mod g takes g / gcd(jump, g) distinct values as p runs.
        if g // np.gcd(self.jump, g) < self.k + self.m:
            raise CheckpointingException(
                f"group of {g} ranks with jump {self.jump} cannot hold k + m = "
                f"{self.k + self.m} distinct slices")

    def _exchange(self, outgoing: Dict[Tuple[int, int, int], object],
                  incoming: List[Tuple[int, int, int, object]],
                  group: Optional[dist.ProcessGroup] = None) -> Dict[Tuple[int, int, int], np.ndarray]:
        """Point-to-point exchange.  outgoing[(dst, owner, pos)] = a byte
        array, or a tuple of byte arrays sent as one message each (a slice's
        head and payload, never copied together); incoming = [(src, owner,
        pos, sizes)], sizes the byte count or the tuple of part sizes, each
        received as one array with the parts back to back.  Every rank passes
        the lists the plan gives it; transfers are ordered by (owner, pos) so
        that both sides agree on tags."""
        me = dist.get_rank()
        group = self.comm_group() if group is None else group
        reqs, recv = [], {}
        for (src, owner, pos, sizes) in sorted(incoming, key=lambda x: (x[1], x[2])):
            if src == me:
                continue
            parts = sizes if isinstance(sizes, tuple) else (sizes,)
            buf = torch.empty(sum(parts), dtype=torch.uint8)
            recv[(src, owner, pos)] = buf
            off = 0
            for q, n in enumerate(parts):
                if n:
                    reqs.append(dist.irecv(buf[off: off + n], src=src, group=group,
                                           tag=(owner * 4096 + pos) * 2 + q))
                off += n
        for (dst, owner, pos), data in sorted(outgoing.items(), key=lambda x: (x[0][1], x[0][2])):
            if dst == me:
                continue
            for q, part in enumerate(data if isinstance(data, tuple) else (data,)):
                if part.size:
                    reqs.append(dist.isend(torch.from_numpy(np.ascontiguousarray(part)), dst=dst,
                                           group=group, tag=(owner * 4096 + pos) * 2 + q))
        for r in reqs:
            r.wait()
        return {key: v.numpy() for key, v in recv.items()}


def _pack_head(header: dict, state: bytes = b"") -> np.ndarray:
    """The bytes of a slice file before its payload: magic, u64 header
    length, JSON header (whose ``state_bytes`` gives the length of what
    follows), then the serialized hollow state (empty for a plain tensor
    list).  The slice bytes follow it in the file."""
    h = json.dumps({**header, "state_bytes": len(state)}, sort_keys=True).encode()
    return np.frombuffer(_MAGIC + np.uint64(len(h)).tobytes() + h + state, np.uint8).copy()


def _pack(header: dict, payload: np.ndarray, state: bytes = b"") -> np.ndarray:
    """A whole slice file in one array (head, then the slice bytes)."""
    return np.concatenate([_pack_head(header, state), payload.reshape(-1)])


def _unpack(blob: np.ndarray) -> Tuple[dict, bytes, np.ndarray]:
    if bytes(blob[: len(_MAGIC)]) != _MAGIC:
        raise CheckpointingException("not an erasure-coded checkpoint slice")
    start = len(_MAGIC) + 8
    n = int(np.frombuffer(bytes(blob[len(_MAGIC): start]), np.uint64)[0])
    header = json.loads(bytes(blob[start: start + n]).decode())
    ns = int(header.get("state_bytes", 0))
    state = bytes(blob[start + n: start + n + ns])
    return header, state, blob[start + n + ns:]


def _hollow_state(state) -> bytes:
    """The state without its tensors, serialized, for a state that follows
    the tensor protocol of MCoreTensorAwareStateDict (pop_tensors /
    insert_tensors, megatron/core/dist_checkpointing/tensor_aware_state_dict.py:195-232):
    the tensors are popped, the hollow object is saved with torch.save (as the
    reference's local manager saves the whole object), and the tensors are
    put back, so the caller's state is unchanged.  Empty for a plain list or
    a TensorListState, whose ``common`` dict travels as JSON instead."""
    if isinstance(state, TensorListState) or not (
            hasattr(state, "pop_tensors") and hasattr(state, "insert_tensors")):
        return b""
    tensors = state.pop_tensors()
    try:
        buf = io.BytesIO()
        torch.save(state, buf)
        return buf.getvalue()
    finally:
        state.insert_tensors(tensors)


# --------------------------------------------------------------- manager --

def _delta_kw(changed_tensors) -> dict:
    """The codec keyword of an incremental save (none for a full save, so
    that codecs without incremental support are called as before)."""
    return {} if changed_tensors is None else {"changed_tensors": changed_tensors}


class ECLocalCheckpointManager:
    """Local (non-persistent) checkpoint manager with erasure-coded
    redundancy, called like the reference's LocalCheckpointManager:
    ``save(state, iteration, is_async)``, ``find_latest()``, ``load()``."""

    def __init__(self, root_dir, repl_strategy: ErasureCodedStrategy,
                 stage_in_background: bool = False):
        self.root = Path(root_dir)
        self.strategy = repl_strategy
        self.rank = dist.get_rank()
        self.latest_iteration = -1
        self.stage_in_background = stage_in_background
        self._bg_group = None
        self._bg_last: Optional[threading.Thread] = None

    # paths
    @property
    def local_dir(self) -> Path:
        return self.root / str(self.rank)

    def _ckpt_id(self, iteration: int, owner: Optional[int] = None) -> str:
        return f"iter_{iteration:07d}_{self.rank if owner is None else owner}_local"

    def _slice_path(self, iteration: int, owner: int, pos: int) -> Path:
        return self.local_dir / f"{self._ckpt_id(iteration, owner)}.ec{pos}"

    def _inventory(self) -> Dict[int, List[Tuple[int, int, int]]]:
        """{iteration: [(owner, pos, nbytes)]} of slices in this rank's dir."""
        inv: Dict[int, List[Tuple[int, int, int]]] = {}
        if self.local_dir.is_dir():
            for f in self.local_dir.iterdir():
                mt = _NAME_RE.match(f.name)
                if mt:
                    inv.setdefault(int(mt.group(1)), []).append(
                        (int(mt.group(2)), int(mt.group(3)), f.stat().st_size))
        return inv

    def _gather_inventories(self) -> List[np.ndarray]:
        """Every rank's inventory as int64 rows (iteration, owner, pos,
        nbytes), exchanged as tensors (no pickled objects): the row counts
        first, then the rows padded to the longest list."""
        st = self.strategy
        rows = np.array([(it, o, p, n) for it, entries in sorted(self._inventory().items())
                         for o, p, n in sorted(entries)], np.int64).reshape(-1, 4)
        g = len(st.ranks())
        count = torch.tensor([rows.shape[0]], dtype=torch.int64)
        counts = [torch.empty_like(count) for _ in range(g)]
        dist.all_gather(counts, count, group=st.comm_group())
        width = max(1, max(int(c[0]) for c in counts))
        mine = torch.zeros((width, 4), dtype=torch.int64)
        mine[: rows.shape[0]] = torch.from_numpy(rows)
        every = [torch.empty_like(mine) for _ in range(g)]
        dist.all_gather(every, mine, group=st.comm_group())
        return [e[: int(c[0])].numpy() for e, c in zip(every, counts)]

    # save
    def save(self, state, iteration: int, is_async: bool = False,
             changed_tensors: Optional[Sequence[int]] = None):
        """Encode this rank's tensors, place the k + m slices on their holders
        and write them.  Collective over the strategy's group.  Raises
        CheckpointingException on every rank if any rank fails; then no slice
        of this iteration is left behind.

        ``changed_tensors`` (not in the reference's call,
        checkpointing.py:538-541, which saves the whole state every time):
        the indices, into the state's tensor list, of every tensor whose bytes
        may have changed since this manager's last save, for a caller that
        knows (frozen layers, sparse updates).  A codec that keeps its last
        coded block in HBM (``GpuSliceCodec(keep_block=True)``) then codes
        only those tensors' units, through the incremental parity update;
        the slices and files are those of a full save.  Other codecs ignore
        it.

        With is_async the GPU work and the exchange still run here (no GPU
        work may move to a writer process, megatron/core/dist_checkpointing/
        strategies/async_utils.py:199), and the file writes are returned as an
        ``AsyncSaveRequest``: the fields and methods of the reference's
        ``AsyncRequest`` (async_utils.py:37-95), which checkpointing.py:616-645
        extends with ``add_finalize_fn`` and hands to ``schedule_async_save``.
        Its ``async_fn`` is a module-level function of picklable arguments, so
        either async caller (forked or persistent) can run it; its finalize
        function checks the files and agrees on success across the group.
        ``execute_sync()`` runs it all in place.

        With is_async on a manager built with ``stage_in_background``, only
        the coding runs here (``codec.snapshot``: torch's stream waits for it,
        after which the tensors may change); staging to host memory, the
        exchange (over a gloo group of its own) and the writes run in a
        background thread of this process, and the request's ``async_fn``
        waits for that thread's marker file."""
        st = self.strategy
        st.check_group()
        if is_async and self.stage_in_background:
            return self._save_in_background(state, iteration, changed_tensors)
        self._quiesce()
        error, blobs, slices = None, None, None
        try:
            # .tensors of MCoreTensorAwareStateDict is an iterator: take it once
            tensors = list(state.tensors) if hasattr(state, "tensors") else list(state)
            hollow, common = _hollow_state(state), _common(state)
            meta, slices = st.codec.encode(tensors, **_delta_kw(changed_tensors))
            blobs = self._blobs(meta, slices, hollow, common, iteration)
        except Exception as e:  # noqa: BLE001 - reported collectively below
            error = e
        received = self._place(blobs, st.comm_group())
        if received is None:
            self._release(slices)
            raise CheckpointingException(
                f"erasure-coded save of iteration {iteration} failed on some rank") from error
        jobs, expected = self._jobs(iteration, received)
        del received, blobs

        def finalize():
            try:
                self._finish_save(iteration, _files_complete(expected))
            finally:   # the files are written (or failed): the host array is free
                self._release(slices)

        self.local_dir.mkdir(parents=True, exist_ok=True)
        if is_async:
            return AsyncSaveRequest(_write_slice_files, (jobs,), [finalize])
        try:
            _write_slice_files(jobs)
        except OSError:
            pass  # finalize() sees the missing files and fails the save everywhere
        finalize()
        return None

    def _release(self, slices) -> None:
        """Hand an encode's host array back to the codec once the slices are
        on disk (codecs without ``release`` keep no arrays)."""
        release = getattr(self.strategy.codec, "release", None)
        if slices is not None and release is not None:
            release(slices)

    def _blobs(self, meta: dict, slices, hollow: bytes, common: dict,
               iteration: int) -> Dict[int, Tuple[np.ndarray, np.ndarray]]:
        """Each slice as (file head, payload): the payload stays the codec's
        array, which is sent and written as it is."""
        meta = {**meta, "common": common, "owner": self.rank, "iteration": iteration}
        return {p: (_pack_head({**meta, "pos": p}, hollow), sl.reshape(-1))
                for p, sl in enumerate(slices)}

    def _place(self, blobs: Optional[Dict[int, Tuple[np.ndarray, np.ndarray]]],
               group) -> Optional[Dict[Tuple[int, int], object]]:
        """Every rank's (head, payload) sizes to every rank (-1: that rank
        failed), then, if none failed, the exchange: {(owner, pos): blob} this
        rank holds (a received array, or this rank's own (head, payload)).
        None on every rank if any rank failed.  Collective over ``group``."""
        st, me = self.strategy, self.rank
        n = st.k + st.m
        sizes = torch.full((n, 2), -1, dtype=torch.int64) if blobs is None else \
            torch.tensor([[blobs[p][0].size, blobs[p][1].size] for p in range(n)],
                         dtype=torch.int64)
        ranks = st.ranks()
        all_sizes = [torch.empty_like(sizes) for _ in ranks]
        dist.all_gather(all_sizes, sizes, group=group)
        if any(int(sz[0, 0]) < 0 for sz in all_sizes):
            return None
        outgoing = {(st.holder(me, p), me, p): blobs[p] for p in range(n)}
        incoming = [(owner, owner, p, (int(sz[p, 0]), int(sz[p, 1])))
                    for owner, sz in zip(ranks, all_sizes)
                    for p in range(n) if st.holder(owner, p) == me]
        received = {(owner, p): buf for (_, owner, p), buf in
                    st._exchange(outgoing, incoming, group).items()}
        for p in range(n):
            if st.holder(me, p) == me:
                received[(me, p)] = blobs[p]
        return received

    def _jobs(self, iteration: int, received):
        """(path, [CPU uint8 tensors written one after the other]) per slice
        file this rank holds, and the file sizes to expect."""
        jobs = [(str(self._slice_path(iteration, owner, p)),
                 [torch.from_numpy(part) for part in (blob if isinstance(blob, tuple) else (blob,))])
                for (owner, p), blob in sorted(received.items())]
        return jobs, [(path, sum(int(t.numel()) for t in parts)) for path, parts in jobs]

    def _background_group(self):
        """The gloo group of the background thread's collectives: the
        strategy's private group over its ranks, never the caller's group, so
        that they do not interleave with collectives the caller issues on its
        own group.  When the strategy's foreground collectives use the same
        private group (an NCCL coding group), the foreground calls wait for
        the background thread first (``_quiesce``)."""
        if self._bg_group is None:
            self._bg_group = private_gloo_group(self.strategy.ranks())
        return self._bg_group

    def _quiesce(self) -> None:
        """Wait for the background save in flight, if any: its collectives
        may use the group the foreground ones are about to use, and a load or
        a newer save must see the files it writes."""
        last = self._bg_last
        if last is not None:
            last.join()

    def _save_in_background(self, state, iteration: int,
                            changed_tensors: Optional[Sequence[int]] = None) -> "AsyncSaveRequest":
        st = self.strategy
        error, pending, hollow, common = None, None, b"", {}
        try:
            tensors = list(state.tensors) if hasattr(state, "tensors") else list(state)
            hollow, common = _hollow_state(state), _common(state)
            pending = st.codec.snapshot(tensors, **_delta_kw(changed_tensors))
        except Exception as e:  # noqa: BLE001 - reported collectively by the thread
            error = e
        group = self._background_group()
        self.local_dir.mkdir(parents=True, exist_ok=True)
        marker = self.local_dir / f".iter_{iteration:07d}.staged"
        marker.unlink(missing_ok=True)
        prev, box = self._bg_last, {"ok": False}

        def body():
            try:
                if prev is not None:
                    prev.join()   # one save's collectives at a time, in save order
                blobs, slices = None, None
                try:
                    if error is not None:
                        raise error
                    meta, slices = pending.result()
                    blobs = self._blobs(meta, slices, hollow, common, iteration)
                except Exception as e:  # noqa: BLE001 - reported collectively
                    box["error"] = e
                received = self._place(blobs, group)
                if received is not None:
                    jobs, expected = self._jobs(iteration, received)
                    del received, blobs
                    try:
                        _write_slice_files(jobs)
                    except OSError as e:
                        box["error"] = e
                    del jobs
                    box["ok"] = _files_complete(expected)
                self._release(slices)
            except Exception as e:  # noqa: BLE001 - finalize fails the save everywhere
                box.setdefault("error", e)
            try:
                # Agree on success over the background group, in this thread:
                # every collective of a background save stays in the chain of
                # background threads, in save order.
                box["ok"] = self._agree(box["ok"], group)
            except Exception as e:  # noqa: BLE001
                box["ok"] = False
                box.setdefault("error", e)
            finally:
                tmp = marker.with_name(marker.name + ".tmp")
                tmp.write_text("ok" if box["ok"] else "failed")
                os.replace(tmp, marker)

        thread = threading.Thread(target=body, daemon=True, name=f"ec-save-{iteration}")
        thread.start()
        self._bg_last = thread

        def finalize():
            thread.join()
            marker.unlink(missing_ok=True)
            self._conclude_save(iteration, box["ok"])

        return AsyncSaveRequest(_await_marker, (str(marker),), [finalize])

    @staticmethod
    def _agree(ok: bool, group) -> bool:
        """True on every rank of ``group`` iff ``ok`` on every rank."""
        flag = torch.tensor([0 if ok else 1], dtype=torch.int64)
        dist.all_reduce(flag, group=group)
        return int(flag[0]) == 0

    def _finish_save(self, iteration: int, ok: bool) -> None:
        """Agree on the save over the coding group, then conclude it."""
        self._conclude_save(iteration, self._agree(ok, self.strategy.comm_group()))

    def _conclude_save(self, iteration: int, agreed: bool) -> None:
        """After every rank agreed on the outcome: drop the iteration on
        failure, else the older ones."""
        if not agreed:
            self._remove(lambda it: it == iteration)
            raise CheckpointingException(f"writing iteration {iteration} failed on some rank")
        self._remove(lambda it: it < iteration)
        self.latest_iteration = max(self.latest_iteration, iteration)

    def _remove(self, pred) -> None:
        if not self.local_dir.is_dir():
            return
        for f in self.local_dir.iterdir():
            mt = _NAME_RE.match(f.name)
            if mt and pred(int(mt.group(1))):
                f.unlink()

    # find / load
    def _plan(self) -> Tuple[int, Dict[int, List[Tuple[int, int, int]]]]:
        """Agree on the newest iteration every owner can decode, and for each
        owner the k slices to read: {owner: [(holder, pos, nbytes)]}."""
        st = self.strategy
        gathered = self._gather_inventories()
        by_iter: Dict[int, Dict[int, Dict[int, Tuple[int, int]]]] = {}
        members = set(st.ranks())
        for holder, rows in zip(st.ranks(), gathered):
            for it, owner, pos, n in rows.tolist():
                if owner not in members or pos >= st.k + st.m or st.holder(owner, pos) != holder:
                    continue  # stray file (another group, code or placement)
                by_iter.setdefault(it, {}).setdefault(owner, {})[pos] = (holder, n)
        for it in sorted(by_iter, reverse=True):
            owners = by_iter[it]
            if all(len(owners.get(o, {})) >= st.k for o in st.ranks()):
                plan = {}
                for o in st.ranks():
                    avail = owners[o]
                    chosen = sorted(avail)[: st.k]  # data positions first: no decode needed
                    plan[o] = [(avail[p][0], p, avail[p][1]) for p in chosen]
                return it, plan
        return -1, {}

    def find_latest(self) -> int:
        self._quiesce()
        it, _ = self._plan()
        self.latest_iteration = it
        return it

    def load(self) -> Tuple[object, str]:
        """Read back the newest iteration all ranks can decode, rebuilding this
        rank's lost slices from any k of its k + m.  Collective.

        Returns (state, name).  A state saved through the tensor protocol (a
        MCoreTensorAwareStateDict) comes back as that object, restored from
        the files this manager wrote (torch.load of the hollow object, as the
        reference's local manager loads its own files) with the rebuilt
        tensors inserted, ready for ``to_state_dict``
        (megatron/training/checkpointing.py:891-899).  Anything else comes
        back as a TensorListState."""
        st = self.strategy
        self._quiesce()
        it, plan = self._plan()
        if it < 0:
            raise CheckpointingException("no erasure-coded checkpoint can be decoded")
        me = self.rank
        outgoing, incoming, local = {}, [], {}
        for owner, reads in plan.items():
            for holder, pos, n in reads:
                if holder == me:
                    blob = np.fromfile(self._slice_path(it, owner, pos), dtype=np.uint8)
                    if owner == me:
                        local[pos] = blob
                    else:
                        outgoing[(owner, owner, pos)] = blob
                if owner == me and holder != me:
                    incoming.append((holder, owner, pos, n))
        got = st._exchange(outgoing, incoming)
        blobs = dict(local)
        for (src, owner, pos), buf in got.items():
            blobs[pos] = buf
        slices, meta, hollow = {}, None, b""
        for pos, blob in blobs.items():
            header, state_bytes, payload = _unpack(blob)
            if header.get("owner") != me or header.get("iteration") != it or header.get("pos") != pos:
                raise CheckpointingException("slice header does not match its name")
            if header.get("generator") != GENERATOR_ID:
                raise CheckpointingException(f"unknown generator {header.get('generator')!r}")
            meta = header
            hollow = hollow or state_bytes
            slices[pos] = payload
        device = torch.device("cuda", torch.cuda.current_device()) if torch.cuda.is_available() else torch.device("cpu")
        tensors = st.codec.decode(meta, slices, device)
        self.latest_iteration = it
        if hollow:
            state = torch.load(io.BytesIO(hollow), weights_only=False)
            state.insert_tensors(tensors)
            return state, self._ckpt_id(it)
        return TensorListState(tensors, meta.get("common", {})), self._ckpt_id(it)


def _common(state) -> dict:
    return state.common if isinstance(state, TensorListState) else {}


def _files_complete(expected: Sequence[Tuple[str, int]]) -> bool:
    return all(os.path.isfile(path) and os.path.getsize(path) == n for path, n in expected)


def _await_marker(path: str, timeout: float = 3600.0) -> None:
    """``async_fn`` of a save staged in the background: returns once the
    trainer's background thread has finished this rank's part and written its
    marker file (whether it succeeded is the finalize function's business).
    No GPU work; module-level with picklable arguments, so it can run in a
    forked or a spawned writer."""
    end = time.monotonic() + timeout
    while not os.path.exists(path):
        if time.monotonic() > end:
            raise TimeoutError(f"{path} did not appear within {timeout} s")
        time.sleep(0.01)


def _write_slice_files(jobs: Sequence[Tuple[str, Sequence[torch.Tensor]]]) -> None:
    """``async_fn`` of an asynchronous save: write each file from its uint8
    CPU tensors, one after the other, atomically (tmp + rename).  No GPU
    work; module-level with picklable arguments, so it can run in a forked or
    a spawned writer."""
    for path, parts in jobs:
        tmp = path + ".tmp"
        with open(tmp, "wb") as f:
            for t in parts:
                f.write(memoryview(t.numpy()))
        os.replace(tmp, path)


class AsyncSaveRequest(NamedTuple):
    """The reference's ``AsyncRequest``
    (megatron/core/dist_checkpointing/strategies/async_utils.py:37-95) field
    for field, so that its async queue schedules it unchanged (it checks the
    field count, freezes the request, and ships it without the finalize
    functions to the writer, :510-519).  ``async_fn(*async_fn_args)`` writes
    the files; the finalize functions run afterwards on every rank."""
    async_fn: Optional[Callable]
    async_fn_args: Tuple
    finalize_fns: List[Callable]
    async_fn_kwargs: Dict = {}
    preload_fn: Optional[Callable] = None
    is_frozen: bool = False
    call_idx: int = 0

    def add_finalize_fn(self, fn: Callable) -> None:
        if self.is_frozen:
            raise RuntimeError("Cannot add finalization functions to a frozen AsyncRequest")
        self.finalize_fns.append(fn)

    def execute_sync(self) -> None:
        """Write, then finalize, in the caller.  The reference's version
        takes a world-wide barrier between the two; here the first finalize
        function is itself a collective over the coding group (the agreement
        on the save's success), so ranks of disjoint coding groups finalize
        independently and no rank outside the group is waited for."""
        if self.async_fn is not None:
            try:
                self.async_fn(*self.async_fn_args, **self.async_fn_kwargs)
            except OSError:
                pass  # the finalize function sees the missing files
        for fn in self.finalize_fns:
            fn()

    def freeze(self) -> "AsyncSaveRequest":
        return self._replace(is_frozen=True)
