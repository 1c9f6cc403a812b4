"""Ragged shard lists cut into fixed-size units and grouped into stripes.

A checkpoint rank holds an ordered, ragged list of shard tensors (the
``MCoreTensorAwareStateDict.tensors`` list of
megatron/core/dist_checkpointing/tensor_aware_state_dict.py:179-184, in
``nested_values`` order, :162-177).  ``StripeLayout`` cuts each tensor's
bytes, in order, into units of ``unit_bytes`` (the last unit of a tensor is
short) and groups consecutive units into stripes of k; the last stripe is
completed with absent units.  A short or absent unit counts as zero-padded
to ``unit_bytes``.  Nothing is copied: the descriptors hold device addresses
into the caller's tensors, and they stay valid only while those tensors
live.  One batched launch then encodes, decodes or updates every stripe.
"""
from __future__ import annotations

import copy
from dataclasses import dataclass
from typing import Optional, Sequence, Tuple

import numpy as np
import torch

from . import _lib
from .codec import _dev, cauchy_matrix, decode_matrix, stream_handle


def stripe_descriptors(base: np.ndarray, size: np.ndarray, k: int,
                       unit_bytes: int) -> Tuple[int, np.ndarray, np.ndarray]:
    """Cut tensors (device base addresses ``base``, byte sizes ``size``), in
    order, into units of ``unit_bytes`` and group them into stripes of k.
    Returns (n_units, ptrs, lens): [n_stripes, k] arrays of unit addresses
    (0 = absent slot of the last stripe) and valid lengths.  Zero-byte
    tensors contribute no unit; an empty list gives one empty stripe.

    Unit u of the flat order belongs to tensor t with first[t] <= u <
    first[t] + n[t] (first = exclusive prefix sum of the unit counts n), so
    its address is (base[t] - first[t] * unit_bytes) + u * unit_bytes, and
    every unit is full except each tensor's last: the work per unit is one
    multiply-add, the rest is per tensor (a save codes ~3,000 tensors cut
    into ~300,000 units, on the path that holds training)."""
    base = np.asarray(base, np.uint64).reshape(-1)
    size = np.asarray(size, np.int64).reshape(-1)
    n = (size + unit_bytes - 1) // unit_bytes
    total = int(n.sum())
    n_stripes = max(1, (total + k - 1) // k)
    ptr = np.zeros(n_stripes * k, np.uint64)
    ln = np.zeros(n_stripes * k, np.uint32)
    if total:
        first = np.cumsum(n) - n
        addr = np.arange(total, dtype=np.int64)
        addr *= unit_bytes
        addr += np.repeat(base.view(np.int64) - first * unit_bytes, n)
        ptr[:total] = addr.view(np.uint64)
        ln[:total] = unit_bytes
        has = n > 0
        ln[(first + n - 1)[has]] = (size - (n - 1) * unit_bytes)[has]
    return total, ptr.reshape(n_stripes, k), ln.reshape(n_stripes, k)


def unit_owners(size: np.ndarray, unit_bytes: int) -> Tuple[np.ndarray, np.ndarray]:
    """(unit_tensor, unit_index) of the flat unit order of ``stripe_descriptors``:
    each unit's tensor and its index inside that tensor."""
    size = np.asarray(size, np.int64).reshape(-1)
    n = (size + unit_bytes - 1) // unit_bytes
    unit_tensor = np.repeat(np.arange(size.size), n)
    unit_index = np.arange(unit_tensor.size) - np.repeat(np.cumsum(n) - n, n)
    return unit_tensor, unit_index


def unit_table(base: np.ndarray, size: np.ndarray, k: int, unit_bytes: int):
    """(unit_tensor, unit_index, ptrs, lens): ``unit_owners`` and
    ``stripe_descriptors`` together."""
    _, ptr, ln = stripe_descriptors(base, size, k, unit_bytes)
    return (*unit_owners(size, unit_bytes), ptr, ln)


def _upload(a: np.ndarray, device) -> torch.Tensor:
    """A device copy of a host array, enqueued on the current stream from
    pinned memory (torch keeps the pinned block until the copy has run)."""
    src = torch.from_numpy(np.ascontiguousarray(a))
    pinned = torch.empty(src.shape, dtype=src.dtype, pin_memory=True)
    pinned.copy_(src)
    return pinned.to(device, non_blocking=True)


def _spans(tensors: Sequence[torch.Tensor], device) -> Tuple[np.ndarray, np.ndarray]:
    """(base addresses, byte sizes) of contiguous HIP tensors on ``device``.
    A save codes thousands of tensors on the path that holds training, so the
    checks and the reads run in the torch-tensor binding (about 0.1 us per
    tensor); a tensor that fails a check raises ValueError (TypeError for
    something that is not a tensor)."""
    tensors = list(tensors)
    idx = torch.device(device).index if device is not None else None
    if idx is None:
        if tensors:
            _dev(tensors[0], "tensors[0]", device)
        raise ValueError(f"tensors must be on a HIP device, not {device}")
    base, size = _lib.shards().spans(tensors, idx)
    return np.frombuffer(base, np.uint64), np.frombuffer(size, np.int64)


@dataclass
class BatchPlan:
    """Device descriptors of one batched decode or update launch."""
    kind: str                 # "decode" or "update"
    rows: np.ndarray          # e x k decode rows, or the m x k coefficients
    outputs: int              # rows of output per stripe (e, or m)
    n_stripes: int
    desc: Tuple[torch.Tensor, ...]


def _hold(stream, *tensors) -> None:
    """Keep descriptor tensors alive until work on ``stream`` has read them.

    They were allocated on torch's current stream; the caching allocator
    orders their reuse after work on that stream, and record_stream extends
    it to a caller-provided side stream."""
    if stream is not None:
        for t in tensors:
            t.record_stream(stream)


class StripeLayout:
    def __init__(self, tensors: Sequence[torch.Tensor], k: int, m: int,
                 unit_bytes: int = 64 << 10, coeff: Optional[np.ndarray] = None,
                 device=None):
        if unit_bytes <= 0 or unit_bytes % 16:
            raise ValueError("unit_bytes must be a positive multiple of 16")
        if not (1 <= k <= 32 and 1 <= m <= 16):
            raise ValueError("batched stripes support 1 <= k <= 32 and 1 <= m <= 16")
        self.k, self.m, self.unit_bytes = k, m, unit_bytes
        self.coeff = cauchy_matrix(k, m) if coeff is None else np.ascontiguousarray(coeff, np.uint8)
        if self.coeff.shape != (m, k):
            raise ValueError("coefficient matrix must be m x k")
        self.tensors = list(tensors)
        if self.tensors:
            self.device = getattr(self.tensors[0], "device", None)
        else:  # an empty list codes as one stripe of absent (zero) units
            self.device = torch.device(device) if device is not None else \
                torch.device("cuda", torch.cuda.current_device())
        base, size = _spans(self.tensors, self.device)
        self._bytes_key = (base.tobytes(), size.tobytes())
        self.tensor_bytes = size
        self.n_units, self.host_ptrs, self.host_len = stripe_descriptors(base, size, k,
                                                                         unit_bytes)
        self._owners = None
        self.n_stripes = self.host_ptrs.shape[0]
        self.data_bytes = int(size.sum())
        # Through pinned memory, asynchronously on the device's current stream:
        # the host does not wait for that stream's earlier work.  Launches on
        # another stream wait for ``uploaded`` first.
        with torch.cuda.device(self.device):
            self.d_ptrs = _upload(self.host_ptrs.view(np.int64), self.device)
            self.d_len = _upload(self.host_len.view(np.int32), self.device)
            self.uploaded = torch.cuda.Event()
            self.uploaded.record()

    def rebind(self, tensors: Sequence[torch.Tensor]) -> Optional["StripeLayout"]:
        """This layout for ``tensors`` when they occupy exactly the device bytes
        this layout was built over (the same addresses and byte sizes, in the
        same order, on the same device), else None.  The descriptors depend
        on nothing else, so the result shares them, on the host and on the
        device: no descriptor build and no upload.  A training run
        checkpoints the same parameter and optimizer buffers at every save.
        The tensors are checked as the constructor checks them."""
        tensors = list(tensors)
        if not tensors or getattr(tensors[0], "device", None) != self.device:
            return None
        base, size = _spans(tensors, self.device)
        if (base.tobytes(), size.tobytes()) != self._bytes_key:
            return None
        twin = copy.copy(self)
        twin.tensors = tensors
        return twin

    def descriptors_only(self) -> "StripeLayout":
        """A copy that holds no reference to the tensors (for keeping the
        descriptors between saves without keeping the tensors alive); only
        ``rebind`` and the descriptor fields may be used on it."""
        bare = copy.copy(self)
        bare.tensors = []
        return bare

    @property
    def unit_tensor(self) -> np.ndarray:
        """Tensor of each unit, in the flat unit order (built on first use)."""
        if self._owners is None:
            self._owners = unit_owners(self.tensor_bytes, self.unit_bytes)
        return self._owners[0]

    @property
    def unit_index(self) -> np.ndarray:
        """Index of each unit inside its tensor (built on first use)."""
        if self._owners is None:
            self._owners = unit_owners(self.tensor_bytes, self.unit_bytes)
        return self._owners[1]

    # ------------------------------------------------------------ parity --

    def alloc_parity(self) -> torch.Tensor:
        return torch.empty((self.n_stripes, self.m, self.unit_bytes), dtype=torch.uint8,
                           device=self.device)

    def _parity_ptrs(self, parity: torch.Tensor) -> torch.Tensor:
        self._parity_ptrs_check(parity)
        base = parity.data_ptr()
        idx = np.arange(self.n_stripes * self.m, dtype=np.uint64) * np.uint64(self.unit_bytes)
        return torch.from_numpy((idx + np.uint64(base)).view(np.int64)).to(self.device)

    def encode(self, parity: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
        """All parity units in one launch: parity[s, i] = XOR_j C[i][j] * unit[s, j]."""
        parity = self.alloc_parity() if parity is None else parity
        cached = getattr(self, "_pp", None)
        if cached is None or cached[0] != parity.data_ptr():
            cached = (parity.data_ptr(), self._parity_ptrs(parity))
            self._pp = cached
        else:
            self._parity_ptrs_check(parity)
        pp = cached[1]
        if stream is not None:
            stream.wait_event(self.uploaded)
        _lib.check(_lib.lib().ec_encode_batched(
            _lib.u8ptr(self.coeff), self.k, self.m, self.d_ptrs.data_ptr(), self.d_len.data_ptr(),
            pp.data_ptr(), self.n_stripes, self.unit_bytes, stream_handle(stream, self.device)),
            "ec_encode_batched")
        _hold(stream, pp)
        return parity

    def _parity_ptrs_check(self, parity: torch.Tensor) -> None:
        if parity.shape != (self.n_stripes, self.m, self.unit_bytes) or parity.dtype != torch.uint8:
            raise ValueError("parity must be uint8 [n_stripes, m, unit_bytes]")
        _dev(parity, "parity", self.device)

    def _to_dev(self, a: np.ndarray, dt) -> torch.Tensor:
        return torch.from_numpy(np.ascontiguousarray(a).view(dt).copy()).to(self.device)

    # ------------------------------------------------------------ decode --

    def plan_decode(self, parity: torch.Tensor, lost: Sequence[int],
                    stripes: Optional[np.ndarray] = None) -> Optional[BatchPlan]:
        """Descriptors for rebuilding the units at codeword positions ``lost``
        (data positions 0..k-1 into the tensors, parity positions k..k+m-1
        into ``parity``) of the given stripes (default: all); at most m
        positions.  None if nothing is lost or no stripe is given."""
        lost = sorted(set(int(x) for x in lost))
        if not lost:
            return None
        k, m = self.k, self.m
        surv, rows = decode_matrix(self.coeff, lost)
        if stripes is None:
            st = np.arange(self.n_stripes)
        else:
            st = np.asarray(stripes, np.int64).reshape(-1)
            if st.size and (st.min() < 0 or st.max() >= self.n_stripes or
                            np.unique(st).size != st.size):
                raise ValueError(f"stripes must be distinct indices in [0, {self.n_stripes})")
            if st.size == 0:
                return None
        self._parity_ptrs_check(parity)
        par_base = np.uint64(parity.data_ptr())

        def slot(pos):
            if pos < k:
                return self.host_ptrs[st, pos], self.host_len[st, pos]
            addr = par_base + (st.astype(np.uint64) * np.uint64(m) + np.uint64(pos - k)) \
                * np.uint64(self.unit_bytes)
            return addr, np.full(st.size, self.unit_bytes, np.uint32)

        sp = np.zeros((st.size, k), np.uint64)
        sl = np.zeros((st.size, k), np.uint32)
        for t, pos in enumerate(surv):
            sp[:, t], sl[:, t] = slot(pos)
        op = np.zeros((st.size, len(lost)), np.uint64)
        ol = np.zeros((st.size, len(lost)), np.uint32)
        for r, pos in enumerate(lost):
            op[:, r], ol[:, r] = slot(pos)
        return BatchPlan("decode", rows, len(lost), int(st.size),
                         (self._to_dev(sp, np.int64), self._to_dev(sl, np.int32),
                          self._to_dev(op, np.int64), self._to_dev(ol, np.int32)))

    def decode(self, parity: torch.Tensor, lost: Sequence[int],
               stripes: Optional[np.ndarray] = None, stream=None) -> None:
        """Rebuild the lost units in place (see plan_decode); the lost units'
        current bytes are ignored."""
        plan = self.plan_decode(parity, lost, stripes)
        if plan is not None:
            self.run(plan, stream)

    # ------------------------------------------------------------ update --

    def plan_update(self, parity: torch.Tensor, changed_units: Sequence[int],
                    old_units: Sequence[torch.Tensor]) -> Optional[BatchPlan]:
        """Descriptors for folding changed units into the parity:
        parity[s, i] ^= C[i][j] * (new ^ old) for each changed unit (s, j).
        ``changed_units`` are global unit indices (order of the layout) whose
        new bytes are in the tensors when the plan runs; ``old_units[n]``
        holds the previous bytes of ``changed_units[n]`` (at least its valid
        length).  None if nothing changed."""
        k, m = self.k, self.m
        cu = np.asarray(changed_units, np.int64)
        if cu.size == 0:
            return None
        if cu.size != len(old_units):
            raise ValueError("one old unit per changed unit")
        if np.unique(cu).size != cu.size or cu.min() < 0 or cu.max() >= self.n_units:
            raise ValueError("changed units must be distinct unit indices")
        stripe = cu // k
        pos = cu % k
        st, inv = np.unique(stripe, return_inverse=True)
        nptr = np.zeros((st.size, k), np.uint64)
        optr = np.zeros((st.size, k), np.uint64)
        ln = np.zeros((st.size, k), np.uint32)
        for n, (r, j) in enumerate(zip(inv, pos)):
            p, nb = _dev(old_units[n], f"old_units[{n}]", self.device)
            if nb < self.host_len[stripe[n], j]:
                raise ValueError(f"old_units[{n}] is shorter than the unit")
            nptr[r, j] = self.host_ptrs[stripe[n], j]
            optr[r, j] = p
            ln[r, j] = self.host_len[stripe[n], j]
        self._parity_ptrs_check(parity)
        pb = np.uint64(parity.data_ptr())
        pptr = (pb + (st.astype(np.uint64)[:, None] * np.uint64(m)
                      + np.arange(m, dtype=np.uint64)[None, :]) * np.uint64(self.unit_bytes))
        return BatchPlan("update", self.coeff, m, int(st.size),
                         (self._to_dev(nptr, np.int64), self._to_dev(optr, np.int64),
                          self._to_dev(ln, np.int32), self._to_dev(pptr, np.int64)))

    def update(self, parity: torch.Tensor, changed_units: Sequence[int],
               old_units: Sequence[torch.Tensor], stream=None) -> None:
        """Fold changed units into the parity in place (see plan_update)."""
        plan = self.plan_update(parity, changed_units, old_units)
        if plan is not None:
            self.run(plan, stream)

    # --------------------------------------------------------------- run --

    def run(self, plan: "BatchPlan", stream=None) -> None:
        """Launch a decode or update plan (one kernel launch)."""
        a, b, c, d = plan.desc
        if plan.kind == "decode":
            st = _lib.lib().ec_decode_batched(
                _lib.u8ptr(plan.rows), self.k, plan.outputs, a.data_ptr(), b.data_ptr(),
                c.data_ptr(), d.data_ptr(), plan.n_stripes, self.unit_bytes,
                stream_handle(stream, self.device))
            _lib.check(st, "ec_decode_batched")
        else:
            st = _lib.lib().ec_parity_update(
                _lib.u8ptr(plan.rows), self.k, self.m, a.data_ptr(), b.data_ptr(), c.data_ptr(),
                d.data_ptr(), plan.n_stripes, self.unit_bytes,
                stream_handle(stream, self.device))
            _lib.check(st, "ec_parity_update")
        _hold(stream, a, b, c, d)

    # ----------------------------------------------------------- helpers --

    def unit_view(self, u: int) -> torch.Tensor:
        """uint8 view of unit u's valid bytes inside its tensor."""
        t = self.tensors[int(self.unit_tensor[u])]
        flat = t.view(-1).view(torch.uint8) if t.dim() else t.view(1).view(torch.uint8)
        off = int(self.unit_index[u]) * self.unit_bytes
        return flat[off: off + int(self.host_len.reshape(-1)[u])]


# --------------------------------------------- drop-in tensor-list entry points --
# The reference hands MCoreTensorAwareStateDict's ragged tensor list
# (tensor_aware_state_dict.py:179-184) to LocalCheckpointManager.save
# (checkpointing.py:538-541), whose redundancy is full replication; these
# compute m-of-(k+m) parity over the same list instead, and rebuild lost units
# from it (manager.load, checkpointing.py:891-894):
#
#     pset = encode(tasd_tensors, k=12, m=4, unit_bytes=64 << 10)  # parity on HBM
#     decode(pset, lost=[0, 13])                 # rebuild those positions in place
#     update(pset, changed_units, old_copies)    # fold a partial change in

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
