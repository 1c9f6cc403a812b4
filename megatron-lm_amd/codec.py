"""Shard-level erasure coding of device tensors (flat shards of equal size).

Every function takes contiguous HIP tensors (any dtype; their bytes are the
shards, viewed without a copy) and enqueues the work on the given stream, or
on torch's current stream, through the C ABI of ``include/ec_mi355.h``.

The reference has no encoder; these are the operations its local-checkpoint
redundancy slot (``repl_strategy`` built at megatron/training/training.py:825-835,
used by ``manager.save`` at megatron/training/checkpointing.py:538-541 and
``manager.load`` at :891-894) would call on one rank's shards.
"""
from __future__ import annotations

import atexit
import ctypes
import threading
import warnings
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch

from . import _lib


def _dev(t: torch.Tensor, what: str, device: Optional[torch.device] = None):
    """(address, byte size) of a contiguous device tensor, optionally checked
    to live on ``device``."""
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{what} must be a torch.Tensor")
    if not t.is_cuda:
        raise ValueError(f"{what} must be a device (HIP) tensor")
    if not t.is_contiguous():
        raise ValueError(f"{what} must be contiguous")
    if device is not None and t.device != device:
        raise ValueError(f"{what} is on {t.device}, the other operands on {device}")
    return t.data_ptr(), t.numel() * t.element_size()


def stream_handle(stream: Optional[torch.cuda.Stream] = None,
                  device: Optional[torch.device] = None) -> ctypes.c_void_p:
    """The opaque ``ec_stream_t`` of ``stream``, or of the current stream of
    ``device`` (torch's current device if None).  The kernels run on the
    stream's device, so a stream on another device than the data is
    rejected."""
    return ctypes.c_void_p(_raw_stream(stream, device))


def _raw_stream(stream, device) -> int:
    """The raw handle behind ``stream_handle``, as an int."""
    if stream is None:
        if device is None:
            return _lib.shards().current_stream(-1)
        dev = torch.device(device)
        return _lib.shards().current_stream(-1 if dev.index is None else dev.index)
    if device is not None and stream.device != torch.device(device):
        raise ValueError(f"stream is on {stream.device}, the tensors on {device}")
    return stream.cuda_stream


_side: Dict[Tuple[int, int], torch.cuda.ExternalStream] = {}
_side_lock = threading.Lock()


def _finish_side_streams() -> None:
    """At interpreter exit, before any library's static destructors: let the
    work on the streams of ``side_stream`` finish, then every device the
    engine made such a stream on, so that no kernel or copy the engine
    enqueued is in flight while the process tears down.  (The staging
    threads of the checkpoint codec are joined before this: their hook is
    registered after this one, at that module's import, and exit hooks run
    last-registered first.)  The streams themselves are never destroyed
    here: tensors that outlive this hook (module globals, freed after it)
    may carry ``record_stream`` uses of them, and the caching allocator
    records an event on each such stream when it frees them; the end of the
    process releases the streams with the rest of the HIP context, as it
    does torch's own streams."""
    with _side_lock:
        devices = sorted({idx for idx, _ in _side})
        for s in _side.values():
            s.synchronize()
    for idx in devices:
        try:
            torch.cuda.synchronize(idx)
        except RuntimeError:   # a device already in error: nothing more to wait for
            pass


atexit.register(_finish_side_streams)


def side_stream(device=None, cus: int = 0) -> torch.cuda.ExternalStream:
    """A stream of ``device`` with a hardware queue of its own
    (``ec_stream_create``), for checkpoint kernels that should run beside the
    training stream rather than behind it: torch's pooled streams share a few
    hardware queues with the current stream, and work on one queue runs in
    order.  Kernels only: copies between host and device belong on an
    ordinary stream (issued on this CU-masked stream they held the host and
    slowed the kernels beside them).
    ``cus`` > 0 restricts it to the first ``cus`` CUs.  One stream per
    (device, cus), created on first use and kept for the life of the process
    (the runtime hands out few such queues).  If the runtime refuses one, a
    warning says so and a stream from torch's pool stands in."""
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None \
        else torch.device(device)
    if dev.type != "cuda":
        raise ValueError(f"side_stream needs a HIP device, got {dev}")
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    key = (idx, max(0, int(cus)))
    with _side_lock:
        s = _side.get(key)
        if s is None:
            h = ctypes.c_void_p()
            status = _lib.lib().ec_stream_create(idx, key[1], ctypes.byref(h))
            if status == _lib.EC_OK:
                s = torch.cuda.ExternalStream(h.value, device=torch.device("cuda", idx))
            else:  # the kernels still run; only the overlap with training is lost
                warnings.warn(f"ec_stream_create on device {idx}: {_lib.strerror(status)}; "
                              "checkpoint work uses a stream from torch's pool, which may run "
                              "behind the training stream's work", RuntimeWarning)
                s = torch.cuda.Stream(device=torch.device("cuda", idx))
            _side[key] = s
        return s


# ------------------------------------------------------------ host algebra --

def gf_mul(a: int, b: int) -> int:
    return int(_lib.lib().ec_gf_mul(a, b))


def gf_inv(a: int) -> int:
    return int(_lib.lib().ec_gf_inv(a))


def cauchy_matrix(k: int, m: int) -> np.ndarray:
    """The m x k parity block C[i][j] = inv((k+i) ^ j) of G = [I_k ; C]."""
    out = np.zeros((m, k), np.uint8)
    _lib.check(_lib.lib().ec_cauchy_matrix(k, m, _lib.u8ptr(out)), "ec_cauchy_matrix")
    return out


_cauchy_bytes: Dict[Tuple[int, int], bytes] = {}


def _cauchy_cached(k: int, m: int) -> bytes:
    """cauchy_matrix(k, m) as bytes, computed once per (k, m)."""
    b = _cauchy_bytes.get((k, m))
    if b is None:
        b = _cauchy_bytes.setdefault((k, m), cauchy_matrix(k, m).tobytes())
    return b


def gf_invert(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, np.uint8)
    n = a.shape[0]
    if a.shape != (n, n):
        raise ValueError("square matrix expected")
    out = np.zeros((n, n), np.uint8)
    _lib.check(_lib.lib().ec_gf_invert(_lib.u8ptr(a), _lib.u8ptr(out), n), "ec_gf_invert")
    return out


def decode_matrix(coeff: np.ndarray, erased: Sequence[int]):
    """(survivors, rows): the k shard indices read and the e x k matrix that
    maps them to the erased shards (data 0..k-1, parity k..k+m-1)."""
    coeff = np.ascontiguousarray(coeff, np.uint8)
    m, k = coeff.shape
    e = len(erased)
    er = (ctypes.c_int * max(1, e))(*erased)
    surv = (ctypes.c_int * k)()
    rows = np.zeros((max(1, e), k), np.uint8)
    _lib.check(_lib.lib().ec_decode_matrix(_lib.u8ptr(coeff), k, m, er, e, surv,
                                           _lib.u8ptr(rows)), "ec_decode_matrix")
    return list(surv), rows[:e].copy()


# ------------------------------------------------------------ device work --

def _shards(shards: Sequence[torch.Tensor], what: str):
    if len(shards) == 0:
        raise ValueError(f"no {what}")
    device = shards[0].device if isinstance(shards[0], torch.Tensor) else None
    ptrs, sizes = zip(*[_dev(t, f"{what}[{i}]", device) for i, t in enumerate(shards)])
    if len(set(sizes)) != 1:
        raise ValueError(f"{what} differ in byte size: {sorted(set(sizes))}")
    return list(ptrs), sizes[0]


def _outputs(out, n: int, nbytes: int, device, what: str) -> List[torch.Tensor]:
    if out is None:
        return [torch.empty(nbytes, dtype=torch.uint8, device=device) for _ in range(n)]
    out = list(out)
    if len(out) != n:
        raise ValueError(f"{what}: expected {n} tensors, got {len(out)}")
    for i, t in enumerate(out):
        _, nb = _dev(t, f"{what}[{i}]", device)
        if nb != nbytes:
            raise ValueError(f"{what}[{i}] has {nb} bytes, shards have {nbytes}")
    return out


# The eager calls below go through the torch-tensor binding (_lib.shards()):
# it checks the tensors, allocates missing outputs, finds torch's current
# stream and makes the C call in one crossing from Python.

def _shard_call(op: int, coeff: bytes, m: int, shards, out, stream, what: str):
    if len(shards) == 0:
        raise ValueError("no shards")
    raw = None if stream is None else _raw_stream(stream, getattr(shards[0], "device", None))
    status, outs = _lib.shards().shard_call(op, coeff, m, shards,
                                            None if out is None else list(out), raw)
    if status != _lib.EC_OK:
        _lib.check(status, what)
    if stream is not None and out is None:
        # Outputs allocated here belong to torch's current stream; the kernel
        # writes them on `stream`, so their memory must not be handed out
        # again before that stream's work is done.
        for t in outs:
            t.record_stream(stream)
    return outs


def xor_encode(shards: Sequence[torch.Tensor], out: Optional[torch.Tensor] = None,
               stream=None) -> torch.Tensor:
    """Single XOR parity of k equal-size shards."""
    return _shard_call(0, b"", 1, shards, None if out is None else [out], stream,
                       "ec_xor_encode")[0]


def matvec(coeff: np.ndarray, shards: Sequence[torch.Tensor], out=None, stream=None,
           what: str = "ec_rs_encode") -> List[torch.Tensor]:
    """out[i] = XOR_j coeff[i][j] * shards[j] (bytewise over GF(2^8))."""
    coeff = np.ascontiguousarray(coeff, np.uint8)
    if coeff.ndim != 2:
        raise ValueError(f"coefficient matrix must be 2-D, got shape {coeff.shape}")
    m, k = coeff.shape
    if len(shards) != k:
        raise ValueError(f"coefficient matrix has {k} columns, got {len(shards)} shards")
    if what not in ("ec_rs_encode", "ec_rs_decode"):
        raise ValueError(f"unknown entry point {what!r}")
    return _shard_call(1 if what == "ec_rs_encode" else 2, coeff.tobytes(), m, shards, out,
                       stream, what)


class ShardPlan:
    """One flat-shard call (``ec_rs_encode``, ``ec_rs_decode`` or
    ``ec_xor_encode``) prepared once and launched many times: the checks, the
    host arrays of device addresses, the coefficient bytes and the stream
    handle are built here, so a launch is one foreign call.  For callers
    that code the same shards repeatedly (small shards especially, where
    matvec's per-call Python work, about 10 us, would otherwise exceed the
    kernel).

    ``what`` is "ec_rs_encode" (``coeff`` m x k, outputs the parity),
    "ec_rs_decode" (``coeff`` the e x k rows of ``decode_matrix``, inputs the
    survivors) or "ec_xor_encode" (``coeff`` ignored, one output).  The plan
    keeps the tensors alive; it launches on ``stream`` (default: torch's
    current stream of the shards' device when the plan is made), or on the
    stream given to the call."""

    def __init__(self, coeff: Optional[np.ndarray], shards: Sequence[torch.Tensor], out=None,
                 stream=None, what: str = "ec_rs_encode"):
        if what not in ("ec_rs_encode", "ec_rs_decode", "ec_xor_encode"):
            raise ValueError(f"unknown entry point {what!r}")
        ptrs, nbytes = _shards(shards, "shards")
        device = shards[0].device
        L = _lib.lib()
        if what == "ec_xor_encode":
            k, m = len(ptrs), 1
            self._coeff = None
        else:
            self._coeff = np.ascontiguousarray(coeff, np.uint8)
            m, k = self._coeff.shape
            if len(ptrs) != k:
                raise ValueError(f"coefficient matrix has {k} columns, got {len(ptrs)} shards")
        self.inputs = list(shards)
        self.outputs = _outputs(out, m, nbytes, device, "out")
        # Outputs allocated here come from torch's current stream; launched
        # on another stream, the caching allocator must not hand their memory
        # out again before that stream's work has run.
        self._owned = out is None
        self.device, self.what, self.nbytes = device, what, nbytes
        self._stream = stream_handle(stream, device)
        self._hold_outputs(stream)
        self._fn = getattr(L, what)
        data = _lib.ptr_array(ptrs)
        if what == "ec_xor_encode":
            self._head = (data, ctypes.c_int(k), ctypes.c_void_p(self.outputs[0].data_ptr()),
                          ctypes.c_uint64(nbytes))
        else:
            self._head = (_lib.u8ptr(self._coeff), ctypes.c_int(k), ctypes.c_int(m), data,
                          _lib.ptr_array([t.data_ptr() for t in self.outputs]),
                          ctypes.c_uint64(nbytes))

    def _hold_outputs(self, stream) -> None:
        """record_stream of the plan's own outputs on ``stream`` when that is
        not the stream they were allocated on."""
        if not self._owned or stream is None:
            return
        if stream.cuda_stream != torch.cuda.current_stream(self.device).cuda_stream:
            for t in self.outputs:
                t.record_stream(stream)

    def __call__(self, stream=None) -> List[torch.Tensor]:
        if stream is None:
            st = self._stream
        else:
            st = stream_handle(stream, self.device)
            self._hold_outputs(stream)
        status = self._fn(*self._head, st)
        if status != _lib.EC_OK:
            _lib.check(status, self.what)
        return self.outputs


def rs_encode(shards: Sequence[torch.Tensor], m: int, coeff: Optional[np.ndarray] = None,
              out=None, stream=None) -> List[torch.Tensor]:
    """m Reed-Solomon parity shards of k equal-size data shards."""
    if coeff is not None:
        return matvec(coeff, shards, out=out, stream=stream)
    k = len(shards)
    if k == 0:
        raise ValueError("no shards")
    return _shard_call(1, _cauchy_cached(k, m), m, shards, out, stream, "ec_rs_encode")


def reconstruct(codeword: Sequence[Optional[torch.Tensor]], k: int, m: int,
                coeff: Optional[np.ndarray] = None, out=None, stream=None) -> dict:
    """Recover the missing (None) entries of a k+m codeword [data..., parity...].

    Returns {shard index: recovered tensor}.  Raises SingularError when more
    than m shards are missing."""
    if len(codeword) != k + m:
        raise ValueError(f"codeword must have k+m = {k + m} entries")
    coeff = cauchy_matrix(k, m) if coeff is None else coeff
    erased = [g for g, t in enumerate(codeword) if t is None]
    if not erased:
        return {}
    surv, rows = decode_matrix(coeff, erased)
    recovered = matvec(rows, [codeword[s] for s in surv], out=out, stream=stream,
                       what="ec_rs_decode")
    return dict(zip(erased, recovered))
