"""C ABI checks that need no GPU: libec_mi355.so loads, exports every symbol
include/ec_mi355.h declares, its host-side algebra agrees with the oracle, and
argument errors come back as status codes before any device work."""
import ctypes
import itertools
import os
import re
import subprocess

import numpy as np
import pytest

import oracle
from oracle import pyref
from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "ec_mi355.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ec_\w+)\s*\(", text)))


def test_header_matches_binding(pkg):
    assert declared_functions() == sorted(pkg._lib.EXPORTS)


def test_integration_stub_binds_every_symbol(pkg):
    """The ctypes stub a reference maintainer would add (the first Python
    block of the integration notes at the repository root) names every
    declared entry point and runs against the built library."""
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    start = text.index("```python") + len("```python")
    stub = text[start:text.index("```", start)]
    assert sorted(set(re.findall(r"_L\.(ec_\w+)", stub))) == declared_functions()
    stub = stub.replace('ctypes.CDLL("libec_mi355.so")', f'ctypes.CDLL({pkg._lib.LIB_PATH!r})')
    assert pkg._lib.LIB_PATH in stub
    exec(compile(stub, "integration stub", "exec"), {})


def test_library_exports_every_declared_symbol(pkg):
    so = pkg._lib.LIB_PATH
    out = subprocess.run(["nm", "-D", "--defined-only", so], check=True, capture_output=True,
                         text=True).stdout
    exported = set(re.findall(r"\bT (ec_\w+)$", out, flags=re.M))
    missing = set(declared_functions()) - exported
    assert not missing, f"not exported: {sorted(missing)}"
    L = pkg._lib.lib()
    for name in declared_functions():
        assert hasattr(L, name)


def test_abi_version_and_strerror(pkg):
    L = pkg._lib.lib()
    assert L.ec_abi_version() == pkg._lib.ABI_VERSION
    for st in (0, -1, -2, -3, -4, -5):
        assert L.ec_strerror(st)
    assert L.ec_strerror(-99) == b"unknown status"


def test_library_missing_an_export_is_refused(pkg, monkeypatch):
    """A stale library (one that lacks a symbol the binding declares) is
    refused when it loads, with ECLibraryMissing, not later with an
    AttributeError on the first call of the missing entry point."""
    lib_mod = pkg._lib
    monkeypatch.setattr(lib_mod, "_lib", None)
    monkeypatch.setattr(lib_mod, "EXPORTS", lib_mod.EXPORTS + ("ec_not_in_this_library",))
    with pytest.raises(lib_mod.ECLibraryMissing, match="ec_not_in_this_library"):
        lib_mod.lib()


def test_host_gf_mul_inv_match_oracle(pkg):
    t = pyref.mul_table()
    L = pkg._lib.lib()
    got = np.array([[L.ec_gf_mul(a, b) for b in range(256)] for a in range(256)], np.uint8)
    assert np.array_equal(got, t)
    assert [pkg.gf_inv(a) for a in range(256)] == [oracle.gf_inv(a) for a in range(256)]


@pytest.mark.parametrize("k,m", [(4, 1), (6, 3), (8, 2), (12, 4), (16, 4), (32, 16), (200, 56)])
def test_host_cauchy_matches_oracle(pkg, k, m):
    assert np.array_equal(pkg.cauchy_matrix(k, m), oracle.cauchy(k, m))


@pytest.mark.parametrize("k,m", [(6, 3), (12, 4), (8, 2)])
def test_host_decode_matrix_all_patterns(pkg, k, m):
    C = oracle.cauchy(k, m)
    for e in range(1, m + 1):
        for lost in itertools.combinations(range(k + m), e):
            s1, r1 = pkg.decode_matrix(C, list(lost))
            s2, r2 = oracle.decode_matrix(C, k, m, list(lost))
            assert s1 == s2 and np.array_equal(r1, r2)


def test_host_invert_and_errors(pkg):
    rng = np.random.default_rng(1)
    a = rng.integers(0, 256, (7, 7), dtype=np.uint8)
    assert np.array_equal(pkg.gf_invert(a), oracle.gf_invert(a))
    with pytest.raises(pkg.SingularError):
        pkg.gf_invert(np.array([[3, 6], [1, 2]], np.uint8))
    with pytest.raises(pkg.SingularError):
        pkg.decode_matrix(pkg.cauchy_matrix(6, 3), [0, 1, 2, 3])
    with pytest.raises(pkg.ECError):
        pkg.decode_matrix(pkg.cauchy_matrix(6, 3), [0, 0])
    with pytest.raises(pkg.ECError):
        pkg.cauchy_matrix(200, 57)


def test_device_entry_points_reject_bad_arguments(pkg):
    """Validation happens on the host, before any HIP call (safe without a GPU)."""
    L = pkg._lib.lib()
    C = pkg.cauchy_matrix(6, 3)
    c = C.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8))
    nulls = (ctypes.c_void_p * 6)()
    assert L.ec_rs_encode(c, 6, 3, None, None, 16, None) == pkg._lib.EC_EINVAL
    assert L.ec_rs_encode(c, 0, 3, nulls, nulls, 16, None) == pkg._lib.EC_EINVAL
    assert L.ec_rs_encode(c, 33, 3, nulls, nulls, 16, None) == pkg._lib.EC_ERANGE
    assert L.ec_rs_encode(c, 6, 3, nulls, nulls, 16, None) == pkg._lib.EC_EINVAL
    assert L.ec_xor_encode(nulls, 4, None, 16, None) == pkg._lib.EC_EINVAL
    # zero bytes: a no-op that succeeds even with the null addresses of empty tensors
    assert L.ec_rs_encode(c, 6, 3, nulls, nulls, 0, None) == pkg._lib.EC_OK
    assert L.ec_rs_decode(c, 6, 3, nulls, nulls, 0, None) == pkg._lib.EC_OK
    assert L.ec_xor_encode(nulls, 4, None, 0, None) == pkg._lib.EC_OK
    assert L.ec_rs_encode(c, 0, 3, nulls, nulls, 0, None) == pkg._lib.EC_EINVAL
    assert L.ec_rs_decode(c, 6, 17, nulls, nulls, 16, None) == pkg._lib.EC_ERANGE
    one = ctypes.c_void_p(16)
    assert L.ec_encode_batched(c, 6, 3, one, one, one, 1, 100, None) == pkg._lib.EC_EALIGN
    assert L.ec_encode_batched(c, 33, 3, one, one, one, 1, 64, None) == pkg._lib.EC_ERANGE
    assert L.ec_encode_batched(c, 6, 17, one, one, one, 1, 64, None) == pkg._lib.EC_ERANGE
    # the copying encode: copy addresses are required; same limits
    assert L.ec_encode_batched_copy(c, 6, 3, one, one, one, None, 1, 64, None) == \
        pkg._lib.EC_EINVAL
    assert L.ec_encode_batched_copy(c, 33, 3, one, one, one, one, 1, 64, None) == \
        pkg._lib.EC_ERANGE
    assert L.ec_encode_batched_copy(c, 6, 3, one, one, one, one, 1, 100, None) == \
        pkg._lib.EC_EALIGN
    assert L.ec_encode_batched_copy(c, 6, 3, one, one, one, one, 0, 64, None) == pkg._lib.EC_OK
    assert L.ec_decode_batched(c, 6, 3, one, one, one, None, 1, 64, None) == pkg._lib.EC_EINVAL
    assert L.ec_parity_update(c, 6, 3, one, one, None, one, 1, 64, None) == pkg._lib.EC_EINVAL
    assert L.ec_stage_last_stats(None) == pkg._lib.EC_EINVAL


def test_stage_stats_struct_matches_the_header(pkg):
    """The ctypes mirror of ec_stage_stats has the header's fields, in order,
    with the C layout (two uint32 then five doubles: 48 bytes), and a thread
    that staged nothing reads zeros."""
    import ctypes
    import threading
    text = open(HEADER).read()
    end = text.index("} ec_stage_stats;")
    body = text[text.rindex("typedef struct {", 0, end): end]
    names = re.findall(r"\b(?:uint32_t|double)\s+(\w+);", body)
    assert names == [n for n, _ in pkg._lib.StageStats._fields_]
    assert ctypes.sizeof(pkg._lib.StageStats) == 48
    got = {}
    t = threading.Thread(target=lambda: got.update(pkg._lib.last_stage_stats()))
    t.start()
    t.join()
    assert got == {"chunks": 0, "copy_engine": 0, "wall_s": 0.0, "wait_s": 0.0,
                   "host_copy_s": 0.0, "max_wait_s": 0.0, "device_s": 0.0}


def test_shard_binding_loads_and_checks_operands(pkg):
    """The torch-tensor binding of the flat-shard calls loads, maps the same
    libec_mi355.so as the ctypes binding (one copy in the process), and
    refuses host tensors, bad coefficient sizes and unknown operations with
    ValueError before any device work."""
    import torch
    B = pkg._lib.shards()
    pkg._lib.lib()
    maps = [ln.split() for ln in open("/proc/self/maps") if "libec_mi355.so" in ln]
    assert {ln[-1] for ln in maps} == {os.path.realpath(pkg._lib.LIB_PATH)}
    assert sum(1 for ln in maps if int(ln[2], 16) == 0) == 1  # mapped once
    host = [torch.zeros(64, dtype=torch.uint8) for _ in range(6)]
    coeff = oracle.cauchy(6, 3).tobytes()
    for args in ((B.ENCODE, coeff, 3, host), (B.XOR, b"", 1, host),
                 (B.ENCODE, coeff[:-1], 3, host), (B.DECODE, coeff, 0, host),
                 (7, coeff, 3, host), (B.ENCODE, coeff, 3, [])):
        with pytest.raises(ValueError):
            B.shard_call(*args)
    with pytest.raises(ValueError, match="device"):
        pkg.rs_encode(host, 3)
    with pytest.raises(ValueError, match="columns"):
        pkg.matvec(oracle.cauchy(6, 3), host[:5])


def test_missing_shard_binding_fails_loudly(pkg, monkeypatch):
    import torch
    monkeypatch.setattr(pkg._lib, "_shards_mod", None)
    monkeypatch.setattr(pkg._lib, "SHARDS_PATH", "/nonexistent/_ec_shards.so")
    with pytest.raises(pkg.ECLibraryMissing):
        pkg.rs_encode([torch.zeros(64, dtype=torch.uint8)] * 6, 3)


def test_missing_library_fails_loudly(pkg, monkeypatch):
    monkeypatch.setattr(pkg._lib, "_lib", None)
    monkeypatch.setattr(pkg._lib, "LIB_PATH", "/nonexistent/libec_mi355.so")
    with pytest.raises(pkg.ECLibraryMissing):
        pkg.cauchy_matrix(6, 3)


def test_stage_to_host_rejects_bad_arguments(pkg):
    """Host-side validation of ec_stage_to_host (no device work)."""
    L = pkg._lib.lib()
    p = ctypes.c_void_p(4096)
    assert L.ec_stage_to_host(p, 64, p, 64, 0, 64, p, 256, 4, None) == pkg._lib.EC_OK
    assert L.ec_stage_to_host(p, 64, p, 64, 2, 0, p, 256, 4, None) == pkg._lib.EC_OK
    assert L.ec_stage_to_host(None, 64, p, 64, 2, 64, p, 256, 4, None) == pkg._lib.EC_EINVAL
    assert L.ec_stage_to_host(p, 64, p, 64, 2, 64, None, 256, 4, None) == pkg._lib.EC_EINVAL
    assert L.ec_stage_to_host(p, 32, p, 64, 2, 64, p, 256, 4, None) == pkg._lib.EC_EINVAL
    assert L.ec_stage_to_host(p, 64, p, 64, 2, 64, p, 256, 0, None) == pkg._lib.EC_EINVAL
    assert L.ec_stage_to_host(p, 64, p, 64, 2, 64, p, 256, 65, None) == pkg._lib.EC_EINVAL
    assert L.ec_stage_to_host(p, 64, p, 64, 4, 64, p, 6, 4, None) == pkg._lib.EC_EINVAL


def test_stage_stripes_to_host_rejects_bad_arguments(pkg):
    """Host-side validation of ec_stage_stripes_to_host (no device work)."""
    L = pkg._lib.lib()
    p = ctypes.c_void_p(4096)
    rows = (ctypes.c_void_p * 2)(4096, 8192)
    hole = (ctypes.c_void_p * 2)(4096, None)
    ok, bad = pkg._lib.EC_OK, pkg._lib.EC_EINVAL
    assert L.ec_stage_stripes_to_host(p, 0, 2, 64, rows, p, 256, 4, None) == ok
    assert L.ec_stage_stripes_to_host(p, 3, 0, 64, rows, p, 256, 4, None) == ok
    assert L.ec_stage_stripes_to_host(p, 3, 2, 0, rows, p, 256, 4, None) == ok
    assert L.ec_stage_stripes_to_host(None, 3, 2, 64, rows, p, 256, 4, None) == bad
    assert L.ec_stage_stripes_to_host(p, 3, 2, 64, None, p, 256, 4, None) == bad
    assert L.ec_stage_stripes_to_host(p, 3, 2, 64, hole, p, 256, 4, None) == bad
    assert L.ec_stage_stripes_to_host(p, 3, 2, 64, rows, None, 256, 4, None) == bad
    assert L.ec_stage_stripes_to_host(p, 3, 2, 64, rows, p, 256, 0, None) == bad
    assert L.ec_stage_stripes_to_host(p, 3, 2, 64, rows, p, 256, 65, None) == bad
    assert L.ec_stage_stripes_to_host(p, 3, 2, 64, rows, p, 1, 4, None) == bad
    assert L.ec_stage_stripes_to_host(p, 1 << 31, 2, 1 << 33, rows, p, 256, 4, None) == bad


def test_stage_to_device_rejects_bad_arguments(pkg):
    """Host-side validation of ec_stage_to_device (no device work)."""
    L = pkg._lib.lib()
    p = ctypes.c_void_p(4096)
    rows = (ctypes.c_void_p * 2)(4096, 8192)
    hole = (ctypes.c_void_p * 2)(4096, None)
    assert L.ec_stage_to_device(rows, 0, 64, p, 64, p, 256, 4, None) == pkg._lib.EC_OK
    assert L.ec_stage_to_device(rows, 2, 0, p, 64, p, 256, 4, None) == pkg._lib.EC_OK
    assert L.ec_stage_to_device(None, 2, 64, p, 64, p, 256, 4, None) == pkg._lib.EC_EINVAL
    assert L.ec_stage_to_device(hole, 2, 64, p, 64, p, 256, 4, None) == pkg._lib.EC_EINVAL
    assert L.ec_stage_to_device(rows, 2, 64, None, 64, p, 256, 4, None) == pkg._lib.EC_EINVAL
    assert L.ec_stage_to_device(rows, 2, 64, p, 32, p, 256, 4, None) == pkg._lib.EC_EINVAL
    assert L.ec_stage_to_device(rows, 2, 64, p, 64, p, 256, 0, None) == pkg._lib.EC_EINVAL
    assert L.ec_stage_to_device(rows, 2, 64, p, 64, p, 2, 4, None) == pkg._lib.EC_EINVAL
