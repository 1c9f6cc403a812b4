"""Randomised checks of the host-side logic around the kernels (hypothesis,
CPU only): the unit/stripe table, the slice file format, and slice
placement across a group."""
import math

import numpy as np
import pytest
from hypothesis import HealthCheck, given, settings, strategies as st

import __graft_entry__
from test_layout_cpu import loop_layout

ec = __graft_entry__.load_package()
from megatron_lm_amd import checkpoint as ck  # noqa: E402
from megatron_lm_amd.layout import stripe_descriptors, unit_table  # noqa: E402


@settings(max_examples=80, deadline=None, suppress_health_check=[HealthCheck.too_slow])
@given(k=st.integers(1, 16), unit16=st.integers(1, 256), seed=st.integers(0, 2**32 - 1),
       n=st.integers(0, 40))
def test_unit_table_random(k, unit16, seed, n):
    unit = 16 * unit16
    rng = np.random.default_rng(seed)
    size = rng.integers(0, 5 * unit + 1, n)
    size[rng.random(n) < 0.2] = 0
    base = np.cumsum(np.concatenate([[1 << 40], size[:-1] + 256])).astype(np.uint64) if n else \
        np.zeros(0, np.uint64)
    owner, idx, P, L = unit_table(base, size, k, unit)
    o2, P2, L2 = loop_layout(base, size, k, unit)
    assert np.array_equal(owner, o2) and np.array_equal(P, P2) and np.array_equal(L, L2)
    assert int(L.sum()) == int(size.sum())
    assert P.shape[0] == max(1, -(-owner.size // k))
    assert stripe_descriptors(base, size, k, unit)[0] == owner.size
    # absent slots of the last stripe are (0, 0); present units are non-empty
    flat_l, flat_p = L.reshape(-1), P.reshape(-1)
    assert (flat_l[: owner.size] > 0).all() and not flat_l[owner.size:].any()
    assert not flat_p[owner.size:].any()
    # every unit lies inside its tensor
    off = idx.astype(np.uint64) * np.uint64(unit)
    assert (flat_p[: owner.size] == base[owner] + off).all()
    assert (off.astype(np.int64) + flat_l[: owner.size] <= size[owner]).all()


json_values = st.recursive(
    st.none() | st.booleans() | st.integers(-2**40, 2**40) | st.text(max_size=8),
    lambda kids: st.lists(kids, max_size=3) | st.dictionaries(st.text(max_size=5), kids,
                                                              max_size=3),
    max_leaves=8)


@settings(max_examples=80, deadline=None)
@given(header=st.dictionaries(st.text(min_size=1, max_size=6).filter(lambda s: s != "state_bytes"),
                              json_values, max_size=5),
       state=st.binary(max_size=300), payload=st.binary(max_size=2000))
def test_slice_format_round_trip(header, state, payload):
    blob = ck._pack(header, np.frombuffer(payload, np.uint8), state)
    h, s, p = ck._unpack(blob)
    assert s == state and bytes(p) == payload
    assert h == {**header, "state_bytes": len(state)}
    # a save sends and writes the head and the payload as separate parts
    assert bytes(ck._pack_head(header, state)) + payload == bytes(blob)


def test_slice_files_written_from_parts(tmp_path):
    """_write_slice_files writes a file's parts back to back, atomically
    (no temporary file is left)."""
    import torch
    head = ck._pack_head({"pos": 3, "owner": 1}, b"hollow")
    payload = np.arange(1000, dtype=np.uint8)
    path = str(tmp_path / "iter_0000001_1_local.ec3")
    ck._write_slice_files([(path, [torch.from_numpy(head), torch.from_numpy(payload)])])
    blob = np.fromfile(path, np.uint8)
    h, st, p = ck._unpack(blob)
    assert h["pos"] == 3 and st == b"hollow" and np.array_equal(p, payload)
    assert sorted(f.name for f in tmp_path.iterdir()) == ["iter_0000001_1_local.ec3"]


def test_slice_format_rejects_foreign_bytes():
    with pytest.raises(ck.CheckpointingException):
        ck._unpack(np.frombuffer(b"not a slice at all, just bytes", np.uint8))


class _FixedGroup(ck.ErasureCodedStrategy):
    def __init__(self, g, *a, **kw):
        super().__init__(*a, **kw)
        self._g = g

    def ranks(self):
        return list(range(self._g))


@settings(max_examples=150, deadline=None)
@given(g=st.integers(1, 32), k=st.integers(1, 12), m=st.integers(1, 4), jump=st.integers(1, 16))
def test_placement(g, k, m, jump):
    s = _FixedGroup(g, k, m, 4096, codec=object(), jump=jump)
    fits = g // math.gcd(g, jump) >= k + m
    if not fits:
        with pytest.raises(ck.CheckpointingException):
            s.check_group()
        return
    s.check_group()
    for owner in range(g):
        holders = [s.holder(owner, p) for p in range(k + m)]
        assert len(set(holders)) == k + m            # k + m distinct ranks
        assert holders == [(owner + p * jump) % g for p in range(k + m)]
    for p in range(k + m):                            # each rank holds one slice per position
        assert sorted(s.holder(o, p) for o in range(g)) == list(range(g))
    # with jump = ranks per node and node-major numbering, one rank's slices
    # land on k + m different nodes
    if g % jump == 0 and g // jump >= k + m:
        for owner in range(g):
            assert len({s.holder(owner, p) // jump for p in range(k + m)}) == k + m


def test_unit_addresses_on_device_match_the_block():
    """The snapshot's device-computed unit addresses are those of the units
    of its stripe-major (stripes, positions, unit_bytes) block."""
    import torch
    block = torch.empty((5, 7, 48), dtype=torch.uint8)
    for first, count in ((0, 4), (4, 3), (2, 1)):
        want = np.array([[block[s, p].data_ptr() for p in range(first, first + count)]
                         for s in range(5)], dtype=np.int64)
        got = ck.GpuSliceCodec._unit_ptrs(block, first, count).numpy()
        assert np.array_equal(got, want), (first, count)


def test_await_marker(tmp_path):
    """async_fn of a background save: returns once the marker exists, raises
    TimeoutError when it never comes."""
    import threading
    import time
    marker = tmp_path / ".iter_0000001.staged"
    threading.Timer(0.1, lambda: marker.write_text("ok")).start()
    t0 = time.monotonic()
    ck._await_marker(str(marker), timeout=10)
    assert time.monotonic() - t0 < 5
    with pytest.raises(TimeoutError):
        ck._await_marker(str(tmp_path / "never"), timeout=0.05)
