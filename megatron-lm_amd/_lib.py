"""ctypes binding of the C ABI in ``include/ec_mi355.h`` (libec_mi355.so).

The shared library is built in-tree by ``__graft_entry__.build()``.  There is
no fallback: if the library is missing, every call raises
``ECLibraryMissing``.  ``shards()`` loads the torch-tensor binding of the
flat-shard calls, built beside it.
"""
from __future__ import annotations

import ctypes
import os
import threading

LIB_NAME = "libec_mi355.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)
ABI_VERSION = 3

EC_OK = 0
EC_EINVAL = -1
EC_EALIGN = -2
EC_ESINGULAR = -3
EC_EHIP = -4
EC_ERANGE = -5
EC_MAX_K = 32
EC_MAX_M = 16

# Every symbol include/ec_mi355.h declares (tests check the export list).
EXPORTS = (
    "ec_abi_version",
    "ec_strerror",
    "ec_gf_mul",
    "ec_gf_inv",
    "ec_cauchy_matrix",
    "ec_gf_invert",
    "ec_decode_matrix",
    "ec_xor_encode",
    "ec_rs_encode",
    "ec_rs_decode",
    "ec_encode_batched",
    "ec_encode_batched_copy",
    "ec_decode_batched",
    "ec_parity_update",
    "ec_stream_create",
    "ec_stream_destroy",
    "ec_stage_to_host",
    "ec_stage_stripes_to_host",
    "ec_stage_to_device",
    "ec_stage_last_stats",
)


class StageStats(ctypes.Structure):
    """ec_stage_stats: the timings of a staging call."""
    _fields_ = [("chunks", ctypes.c_uint32), ("copy_engine", ctypes.c_uint32),
                ("wall_s", ctypes.c_double), ("wait_s", ctypes.c_double),
                ("host_copy_s", ctypes.c_double), ("max_wait_s", ctypes.c_double),
                ("device_s", ctypes.c_double)]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) if kind is ctypes.c_uint32 else round(getattr(self, name), 4)
                for name, kind in self._fields_}


def last_stage_stats() -> dict:
    """ec_stage_last_stats of the calling thread, as a dict."""
    st = StageStats()
    check(lib().ec_stage_last_stats(ctypes.byref(st)), "ec_stage_last_stats")
    return st.as_dict()


class ECLibraryMissing(RuntimeError):
    pass


class ECError(RuntimeError):
    def __init__(self, status: int, what: str):
        self.status = status
        super().__init__(f"{what}: {strerror(status)} (status {status})")


class SingularError(ECError):
    pass


_lib = None

_u8p = ctypes.POINTER(ctypes.c_uint8)
_vp = ctypes.c_void_p
_i = ctypes.c_int
_u32 = ctypes.c_uint32
_u64 = ctypes.c_uint64


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ECLibraryMissing(
            f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'`")
    L = ctypes.CDLL(LIB_PATH)
    L.ec_abi_version.restype = _i
    L.ec_abi_version.argtypes = []
    if L.ec_abi_version() != ABI_VERSION:
        raise ECLibraryMissing(f"{LIB_PATH} has ABI {L.ec_abi_version()}, expected {ABI_VERSION}")
    missing = [name for name in EXPORTS if not hasattr(L, name)]
    if missing:
        raise ECLibraryMissing(f"{LIB_PATH} lacks {', '.join(missing)}; rebuild it")
    L.ec_strerror.restype = ctypes.c_char_p
    L.ec_strerror.argtypes = [_i]
    L.ec_gf_mul.restype = ctypes.c_uint8
    L.ec_gf_mul.argtypes = [ctypes.c_uint8, ctypes.c_uint8]
    L.ec_gf_inv.restype = ctypes.c_uint8
    L.ec_gf_inv.argtypes = [ctypes.c_uint8]
    L.ec_cauchy_matrix.restype = _i
    L.ec_cauchy_matrix.argtypes = [_i, _i, _u8p]
    L.ec_gf_invert.restype = _i
    L.ec_gf_invert.argtypes = [_u8p, _u8p, _i]
    L.ec_decode_matrix.restype = _i
    L.ec_decode_matrix.argtypes = [_u8p, _i, _i, ctypes.POINTER(_i), _i, ctypes.POINTER(_i), _u8p]
    L.ec_xor_encode.restype = _i
    L.ec_xor_encode.argtypes = [_vp, _i, _vp, _u64, _vp]
    L.ec_rs_encode.restype = _i
    L.ec_rs_encode.argtypes = [_u8p, _i, _i, _vp, _vp, _u64, _vp]
    L.ec_rs_decode.restype = _i
    L.ec_rs_decode.argtypes = [_u8p, _i, _i, _vp, _vp, _u64, _vp]
    L.ec_encode_batched.restype = _i
    L.ec_encode_batched.argtypes = [_u8p, _i, _i, _vp, _vp, _vp, _u32, _u32, _vp]
    L.ec_encode_batched_copy.restype = _i
    L.ec_encode_batched_copy.argtypes = [_u8p, _i, _i, _vp, _vp, _vp, _vp, _u32, _u32, _vp]
    L.ec_decode_batched.restype = _i
    L.ec_decode_batched.argtypes = [_u8p, _i, _i, _vp, _vp, _vp, _vp, _u32, _u32, _vp]
    L.ec_parity_update.restype = _i
    L.ec_parity_update.argtypes = [_u8p, _i, _i, _vp, _vp, _vp, _vp, _u32, _u32, _vp]
    L.ec_stream_create.restype = _i
    L.ec_stream_create.argtypes = [_i, _i, ctypes.POINTER(_vp)]
    L.ec_stream_destroy.restype = _i
    L.ec_stream_destroy.argtypes = [_vp]
    L.ec_stage_to_host.restype = _i
    L.ec_stage_to_host.argtypes = [_vp, _u64, _vp, _u64, _u32, _u64, _vp, _u64, _i, _vp]
    L.ec_stage_stripes_to_host.restype = _i
    L.ec_stage_stripes_to_host.argtypes = [_vp, _u32, _u32, _u64, _vp, _vp, _u64, _i, _vp]
    L.ec_stage_to_device.restype = _i
    L.ec_stage_to_device.argtypes = [_vp, _u32, _u64, _vp, _u64, _vp, _u64, _i, _vp]
    L.ec_stage_last_stats.restype = _i
    L.ec_stage_last_stats.argtypes = [ctypes.POINTER(StageStats)]
    _lib = L
    return L


SHARDS_NAME = "_ec_shards"
SHARDS_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), SHARDS_NAME + ".so")
_shards_mod = None
_shards_lock = threading.Lock()


def shards():
    """The torch-tensor binding of the flat-shard calls (``_ec_shards.so``,
    csrc/shards_torch.cpp), which links libec_mi355.so.  Raises
    ``ECLibraryMissing`` when it is not built; there is no fallback."""
    global _shards_mod
    if _shards_mod is not None:
        return _shards_mod
    with _shards_lock:   # one load, also when threads race to the first call
        if _shards_mod is not None:
            return _shards_mod
        lib()  # the C library first: checks its ABI version and gives the extension its symbols
        if not os.path.exists(SHARDS_PATH):
            raise ECLibraryMissing(
                f"{SHARDS_PATH} is not built; run `python -c 'import __graft_entry__ as g; "
                "g.build()'`")
        import importlib.machinery
        import importlib.util
        import torch  # noqa: F401  (the extension needs torch's libraries loaded)
        loader = importlib.machinery.ExtensionFileLoader(SHARDS_NAME, SHARDS_PATH)
        spec = importlib.util.spec_from_file_location(SHARDS_NAME, SHARDS_PATH, loader=loader)
        mod = importlib.util.module_from_spec(spec)
        loader.exec_module(mod)
        _shards_mod = mod
    return mod


def strerror(status: int) -> str:
    try:
        return lib().ec_strerror(status).decode()
    except ECLibraryMissing:
        return "library not built"


def check(status: int, what: str) -> None:
    if status == EC_OK:
        return
    if status == EC_ESINGULAR:
        raise SingularError(status, what)
    raise ECError(status, what)


def u8ptr(buf) -> "ctypes._Pointer":
    """Pointer to a host uint8 numpy array."""
    return buf.ctypes.data_as(_u8p)


def ptr_array(addrs) -> ctypes.Array:
    """Host array of device addresses (a `const uint8_t* const*`)."""
    return (ctypes.c_void_p * len(addrs))(*[int(a) for a in addrs])
