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

from typing import Dict, List, Optional, Sequence

import numpy as np
import torch

from . import _lib
from .codec import _dev, cauchy_matrix, decode_matrix, stream_handle


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
                 unit_bytes: int = 64 << 10, coeff: Optional[np.ndarray] = None):
        if unit_bytes <= 0 or unit_bytes % 16:
            raise ValueError("unit_bytes must be a positive multiple of 16")
        if not (1 <= k <= 16 and 1 <= m <= 4):
            raise ValueError("batched stripes support 1 <= k <= 16 and 1 <= m <= 4")
        self.k, self.m, self.unit_bytes = k, m, unit_bytes
        self.coeff = cauchy_matrix(k, m) if coeff is None else np.ascontiguousarray(coeff, np.uint8)
        if self.coeff.shape != (m, k):
            raise ValueError("coefficient matrix must be m x k")
        self.tensors = list(tensors)
        if not self.tensors:
            raise ValueError("no tensors")
        self.device = self.tensors[0].device
        base = np.zeros(len(self.tensors), np.uint64)
        size = np.zeros(len(self.tensors), np.int64)
        for i, t in enumerate(self.tensors):
            if t.device != self.device:
                raise ValueError("all tensors must be on one device")
            p, nb = _dev(t, f"tensors[{i}]")
            base[i], size[i] = p, nb
        self.tensor_bytes = size
        n_units = (size + unit_bytes - 1) // unit_bytes
        self.unit_tensor = np.repeat(np.arange(len(size)), n_units)       # owning tensor
        first = np.concatenate([[0], np.cumsum(n_units)[:-1]]).astype(np.int64)
        self.unit_index = np.arange(self.unit_tensor.size) - np.repeat(first, n_units)
        self.unit_first = first                                          # first unit per tensor
        self.n_units = int(self.unit_tensor.size)
        self.n_stripes = max(1, (self.n_units + k - 1) // k)
        slots = self.n_stripes * k
        ptr = np.zeros(slots, np.uint64)
        ln = np.zeros(slots, np.uint32)
        off = self.unit_index.astype(np.uint64) * np.uint64(unit_bytes)
        ptr[: self.n_units] = base[self.unit_tensor] + off
        ln[: self.n_units] = np.minimum(size[self.unit_tensor] - off.astype(np.int64),
                                        unit_bytes).astype(np.uint32)
        self.host_ptrs = ptr.reshape(self.n_stripes, k)
        self.host_len = ln.reshape(self.n_stripes, k)
        self.data_bytes = int(size.sum())
        self.d_ptrs = torch.from_numpy(self.host_ptrs.view(np.int64).copy()).to(self.device)
        self.d_len = torch.from_numpy(self.host_len.view(np.int32).copy()).to(self.device)

    # ------------------------------------------------------------ parity --

    def alloc_parity(self) -> torch.Tensor:
        return torch.empty((self.n_stripes, self.m, self.unit_bytes), dtype=torch.uint8,
                           device=self.device)

    def _parity_ptrs(self, parity: torch.Tensor) -> torch.Tensor:
        if parity.shape != (self.n_stripes, self.m, self.unit_bytes) or parity.dtype != torch.uint8:
            raise ValueError("parity must be uint8 [n_stripes, m, unit_bytes]")
        _dev(parity, "parity")
        base = parity.data_ptr()
        idx = np.arange(self.n_stripes * self.m, dtype=np.uint64) * np.uint64(self.unit_bytes)
        return torch.from_numpy((idx + np.uint64(base)).view(np.int64)).to(self.device)

    def encode(self, parity: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
        """All parity units in one launch: parity[s, i] = XOR_j C[i][j] * unit[s, j]."""
        parity = self.alloc_parity() if parity is None else parity
        pp = self._parity_ptrs(parity)
        _lib.check(_lib.lib().ec_encode_batched(
            _lib.u8ptr(self.coeff), self.k, self.m, self.d_ptrs.data_ptr(), self.d_len.data_ptr(),
            pp.data_ptr(), self.n_stripes, self.unit_bytes, stream_handle(stream)),
            "ec_encode_batched")
        _hold(stream, pp)
        return parity

    # ------------------------------------------------------------ decode --

    def decode(self, parity: torch.Tensor, lost: Sequence[int],
               stripes: Optional[np.ndarray] = None, stream=None) -> None:
        """Rebuild, in place, the units at codeword positions ``lost`` (data
        positions 0..k-1 into the tensors, parity positions k..k+m-1 into
        ``parity``) of the given stripes (default: all).  The lost units'
        current bytes are ignored; at most m positions."""
        lost = sorted(set(int(x) for x in lost))
        if not lost:
            return
        k, m = self.k, self.m
        surv, rows = decode_matrix(self.coeff, lost)
        st = np.arange(self.n_stripes) if stripes is None else np.asarray(stripes, np.int64)
        par_base = np.uint64(parity.data_ptr())
        self._parity_ptrs(parity)

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
        dev = lambda a, dt: torch.from_numpy(a.view(dt).copy()).to(self.device)
        d_sp, d_sl, d_op, d_ol = dev(sp, np.int64), dev(sl, np.int32), dev(op, np.int64), dev(ol, np.int32)
        _lib.check(_lib.lib().ec_decode_batched(
            _lib.u8ptr(rows), k, len(lost), d_sp.data_ptr(), d_sl.data_ptr(), d_op.data_ptr(),
            d_ol.data_ptr(), int(st.size), self.unit_bytes, stream_handle(stream)),
            "ec_decode_batched")
        _hold(stream, d_sp, d_sl, d_op, d_ol)

    # ------------------------------------------------------------ update --

    def update(self, parity: torch.Tensor, changed_units: Sequence[int],
               old_units: Sequence[torch.Tensor], stream=None) -> None:
        """Fold changed units into the parity in place:
        parity[s, i] ^= C[i][j] * (new ^ old) for each changed unit (s, j).
        ``changed_units`` are global unit indices (order of the layout) whose
        new bytes are already in the tensors; ``old_units[n]`` holds the
        previous bytes of ``changed_units[n]`` (at least its valid length)."""
        k, m = self.k, self.m
        cu = np.asarray(changed_units, np.int64)
        if cu.size == 0:
            return
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
            p, nb = _dev(old_units[n], f"old_units[{n}]")
            if nb < self.host_len[stripe[n], j]:
                raise ValueError(f"old_units[{n}] is shorter than the unit")
            nptr[r, j] = self.host_ptrs[stripe[n], j]
            optr[r, j] = p
            ln[r, j] = self.host_len[stripe[n], j]
        pb = np.uint64(parity.data_ptr())
        self._parity_ptrs(parity)
        pptr = (pb + (st.astype(np.uint64)[:, None] * np.uint64(m)
                      + np.arange(m, dtype=np.uint64)[None, :]) * np.uint64(self.unit_bytes))
        dev = lambda a, dt: torch.from_numpy(np.ascontiguousarray(a).view(dt).copy()).to(self.device)
        d_n, d_o, d_l, d_p = dev(nptr, np.int64), dev(optr, np.int64), dev(ln, np.int32), dev(pptr, np.int64)
        _lib.check(_lib.lib().ec_parity_update(
            _lib.u8ptr(self.coeff), k, m, d_n.data_ptr(), d_o.data_ptr(), d_l.data_ptr(),
            d_p.data_ptr(), int(st.size), self.unit_bytes, stream_handle(stream)),
            "ec_parity_update")
        _hold(stream, d_n, d_o, d_l, d_p)

    # ----------------------------------------------------------- helpers --

    def unit_view(self, u: int) -> torch.Tensor:
        """uint8 view of unit u's valid bytes inside its tensor."""
        t = self.tensors[int(self.unit_tensor[u])]
        flat = t.view(-1).view(torch.uint8) if t.dim() else t.view(1).view(torch.uint8)
        off = int(self.unit_index[u]) * self.unit_bytes
        return flat[off: off + int(self.host_len.reshape(-1)[u])]
