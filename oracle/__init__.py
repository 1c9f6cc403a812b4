"""CPU oracle of the erasure-coding hot path (ctypes over libec_oracle.so).

TEST INFRASTRUCTURE.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
checker or the timed CPU baseline; the product under ``megatron-lm_amd/`` never
does.

The reference (duihuhu/Megatron-LM) has no erasure coder, so the arithmetic is
restated from the mathematics (GF(2^8)/0x11D, Cauchy generator
``C[i][j] = inv((k+i) ^ j)``), see ``ec_oracle.h``.  ``pyref`` is a second,
independent pure-Python restatement used to cross-check this one.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libec_oracle.so")
_lib = None

_u8p = ctypes.POINTER(ctypes.c_uint8)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_u64p = ctypes.POINTER(ctypes.c_uint64)
_intp = ctypes.POINTER(ctypes.c_int)


def build() -> str:
    """Compile libec_oracle.so with the Makefile next to this file."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"{_LIB_PATH} is not built; run `make -C oracle`")
        L = ctypes.CDLL(_LIB_PATH)
        L.ecref_gf_mul.restype = ctypes.c_uint8
        L.ecref_gf_mul.argtypes = [ctypes.c_uint8, ctypes.c_uint8]
        L.ecref_gf_inv.restype = ctypes.c_uint8
        L.ecref_gf_inv.argtypes = [ctypes.c_uint8]
        L.ecref_cauchy.argtypes = [ctypes.c_int, ctypes.c_int, _u8p]
        L.ecref_gf_invert.argtypes = [_u8p, _u8p, ctypes.c_int]
        L.ecref_decode_matrix.argtypes = [_u8p, ctypes.c_int, ctypes.c_int, _intp,
                                          ctypes.c_int, _intp, _u8p]
        L.ecref_xor_encode.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
                                       ctypes.c_uint64]
        L.ecref_rs_encode.argtypes = [_u8p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                      ctypes.c_void_p, ctypes.c_uint64]
        L.ecref_encode_batched.argtypes = [_u8p, ctypes.c_int, ctypes.c_int, _u64p, _u32p,
                                           _u64p, ctypes.c_uint32, ctypes.c_uint32]
        L.ecref_parity_update.argtypes = [_u8p, ctypes.c_int, ctypes.c_int, _u64p, _u64p,
                                          _u32p, _u64p, ctypes.c_uint32, ctypes.c_uint32]
        L.ecfast_isa.restype = ctypes.c_char_p
        L.ecfast_xor_encode.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
                                        ctypes.c_uint64, ctypes.c_int]
        L.ecfast_rs_encode.argtypes = [_u8p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                       ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int]
        L.ecfast_force_isa.argtypes = [ctypes.c_char_p]
        L.ecfast_encode_batched.restype = ctypes.c_int
        L.ecfast_encode_batched.argtypes = [_u8p, ctypes.c_int, ctypes.c_int, _u64p, _u32p,
                                            _u64p, ctypes.c_uint32, ctypes.c_uint32,
                                            ctypes.c_int]
        L.ecfast_parity_update.restype = ctypes.c_int
        L.ecfast_parity_update.argtypes = [_u8p, ctypes.c_int, ctypes.c_int, _u64p, _u64p,
                                           _u32p, _u64p, ctypes.c_uint32, ctypes.c_uint32,
                                           ctypes.c_int]
        _lib = L
    return _lib


def _u8(a: np.ndarray):
    return a.ctypes.data_as(_u8p)


def _ptr_array(arrays) -> ctypes.Array:
    return (ctypes.c_void_p * len(arrays))(*[a.ctypes.data for a in arrays])


def _check_shards(arrays, n=None):
    out = []
    for a in arrays:
        a = np.ascontiguousarray(a).view(np.uint8).reshape(-1)
        if n is not None and a.size < n:
            raise ValueError("shard shorter than nbytes")
        out.append(a)
    return out


# ---------------------------------------------------------------- algebra ---

def gf_mul(a: int, b: int) -> int:
    return int(lib().ecref_gf_mul(a, b))


def gf_inv(a: int) -> int:
    return int(lib().ecref_gf_inv(a))


def cauchy(k: int, m: int) -> np.ndarray:
    out = np.zeros((m, k), np.uint8)
    if lib().ecref_cauchy(k, m, _u8(out)) != 0:
        raise ValueError("bad (k, m)")
    return out


def gf_invert(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, np.uint8)
    n = a.shape[0]
    out = np.zeros((n, n), np.uint8)
    st = lib().ecref_gf_invert(_u8(a), _u8(out), n)
    if st != 0:
        raise np.linalg.LinAlgError("singular over GF(2^8)")
    return out


def decode_matrix(coeff: np.ndarray, k: int, m: int, erased):
    coeff = np.ascontiguousarray(coeff, np.uint8)
    er = (ctypes.c_int * max(1, len(erased)))(*erased)
    surv = (ctypes.c_int * k)()
    rows = np.zeros((max(1, len(erased)), k), np.uint8)
    st = lib().ecref_decode_matrix(_u8(coeff), k, m, er, len(erased), surv, _u8(rows))
    if st == -3:
        raise np.linalg.LinAlgError("not decodable")
    if st != 0:
        raise ValueError("bad erasure list")
    return list(surv), rows[: len(erased)]


# ----------------------------------------------------------------- encode ---

def xor_encode(shards) -> np.ndarray:
    shards = _check_shards(shards)
    n = shards[0].size
    out = np.empty(n, np.uint8)
    lib().ecref_xor_encode(_ptr_array(shards), len(shards), out.ctypes.data, n)
    return out


def rs_encode(coeff: np.ndarray, shards) -> list:
    coeff = np.ascontiguousarray(coeff, np.uint8)
    m, k = coeff.shape
    shards = _check_shards(shards)
    assert len(shards) == k
    n = shards[0].size
    outs = [np.empty(n, np.uint8) for _ in range(m)]
    lib().ecref_rs_encode(_u8(coeff), k, m, _ptr_array(shards), _ptr_array(outs), n)
    return outs


def encode_batched(coeff, units, lens, unit_bytes):
    """units: list (stripes) of k arrays (or None); lens: n_stripes x k."""
    coeff = np.ascontiguousarray(coeff, np.uint8)
    m, k = coeff.shape
    ns = len(units)
    keep = []
    dptr = np.zeros((ns, k), np.uint64)
    for s in range(ns):
        for j in range(k):
            u = units[s][j]
            if u is not None:
                u = np.ascontiguousarray(u).view(np.uint8).reshape(-1)
                keep.append(u)
                dptr[s, j] = u.ctypes.data
    lens = np.ascontiguousarray(lens, np.uint32)
    par = np.zeros((ns, m, unit_bytes), np.uint8)
    pptr = np.array([[par[s, i].ctypes.data for i in range(m)] for s in range(ns)],
                    np.uint64).reshape(ns, m)
    lib().ecref_encode_batched(_u8(coeff), k, m, dptr.ctypes.data_as(_u64p),
                               lens.ctypes.data_as(_u32p), pptr.ctypes.data_as(_u64p),
                               ns, unit_bytes)
    return par


def parity_update(coeff, new_units, old_units, lens, parity: np.ndarray, unit_bytes):
    """In-place update of parity (n_stripes x m x unit_bytes)."""
    coeff = np.ascontiguousarray(coeff, np.uint8)
    m, k = coeff.shape
    ns = len(new_units)
    keep = []
    nptr = np.zeros((ns, k), np.uint64)
    optr = np.zeros((ns, k), np.uint64)
    for s in range(ns):
        for j in range(k):
            if new_units[s][j] is not None:
                a = np.ascontiguousarray(new_units[s][j]).view(np.uint8).reshape(-1)
                b = np.ascontiguousarray(old_units[s][j]).view(np.uint8).reshape(-1)
                keep += [a, b]
                nptr[s, j] = a.ctypes.data
                optr[s, j] = b.ctypes.data
    lens = np.ascontiguousarray(lens, np.uint32)
    assert parity.flags.c_contiguous and parity.dtype == np.uint8
    pptr = np.array([[parity[s, i].ctypes.data for i in range(m)] for s in range(ns)],
                    np.uint64).reshape(ns, m)
    lib().ecref_parity_update(_u8(coeff), k, m, nptr.ctypes.data_as(_u64p),
                              optr.ctypes.data_as(_u64p), lens.ctypes.data_as(_u32p),
                              pptr.ctypes.data_as(_u64p), ns, unit_bytes)
    return parity


# ------------------------------------------------------ SIMD CPU baseline ---

def fast_isa() -> str:
    return lib().ecfast_isa().decode()


def fast_force_isa(name: str) -> bool:
    return bool(lib().ecfast_force_isa(name.encode()))


def fast_xor_encode(shards, out=None, nthreads: int = 1) -> np.ndarray:
    shards = _check_shards(shards)
    n = shards[0].size
    out = np.empty(n, np.uint8) if out is None else out
    lib().ecfast_xor_encode(_ptr_array(shards), len(shards), out.ctypes.data, n, nthreads)
    return out


def fast_rs_encode(coeff, shards, outs=None, nthreads: int = 1) -> list:
    coeff = np.ascontiguousarray(coeff, np.uint8)
    m, k = coeff.shape
    shards = _check_shards(shards)
    n = shards[0].size
    outs = [np.empty(n, np.uint8) for _ in range(m)] if outs is None else outs
    lib().ecfast_rs_encode(_u8(coeff), k, m, _ptr_array(shards), _ptr_array(outs), n,
                           nthreads)
    return outs


def fast_encode_batched(coeff, dptr: np.ndarray, dlen: np.ndarray, pptr: np.ndarray,
                        unit_bytes: int, nthreads: int = 1) -> None:
    """ecfast_encode_batched over descriptor arrays of host addresses:
    dptr / dlen [n_stripes, k] (0 = absent unit), pptr [n_stripes, m]; the
    caller keeps the memory they point at alive."""
    coeff = np.ascontiguousarray(coeff, np.uint8)
    m, k = coeff.shape
    dptr = np.ascontiguousarray(dptr, np.uint64)
    dlen = np.ascontiguousarray(dlen, np.uint32)
    pptr = np.ascontiguousarray(pptr, np.uint64)
    ns = dptr.shape[0]
    if dptr.shape != (ns, k) or dlen.shape != (ns, k) or pptr.shape != (ns, m):
        raise ValueError("descriptor shapes do not match (n_stripes, k) / (n_stripes, m)")
    if lib().ecfast_encode_batched(_u8(coeff), k, m, dptr.ctypes.data_as(_u64p),
                                   dlen.ctypes.data_as(_u32p), pptr.ctypes.data_as(_u64p),
                                   ns, unit_bytes, nthreads) != 0:
        raise MemoryError("ecfast_encode_batched failed")


def fast_parity_update(coeff, nptr: np.ndarray, optr: np.ndarray, dlen: np.ndarray,
                       pptr: np.ndarray, unit_bytes: int, nthreads: int = 1) -> None:
    """ecfast_parity_update over descriptor arrays of host addresses: nptr /
    optr / dlen [n_stripes, k] (nptr 0 = unchanged unit), pptr [n_stripes, m];
    the parity units are updated in place.  The caller keeps the memory they
    point at alive."""
    coeff = np.ascontiguousarray(coeff, np.uint8)
    m, k = coeff.shape
    nptr = np.ascontiguousarray(nptr, np.uint64)
    optr = np.ascontiguousarray(optr, np.uint64)
    dlen = np.ascontiguousarray(dlen, np.uint32)
    pptr = np.ascontiguousarray(pptr, np.uint64)
    ns = nptr.shape[0]
    if (nptr.shape != (ns, k) or optr.shape != (ns, k) or dlen.shape != (ns, k)
            or pptr.shape != (ns, m)):
        raise ValueError("descriptor shapes do not match (n_stripes, k) / (n_stripes, m)")
    if lib().ecfast_parity_update(_u8(coeff), k, m, nptr.ctypes.data_as(_u64p),
                                  optr.ctypes.data_as(_u64p), dlen.ctypes.data_as(_u32p),
                                  pptr.ctypes.data_as(_u64p), ns, unit_bytes, nthreads) != 0:
        raise MemoryError("ecfast_parity_update failed")
