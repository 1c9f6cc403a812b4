"""Host-side stripe layout (no device work): units and stripes of a ragged
tensor list, checked against a direct loop over the tensors."""
import numpy as np
import pytest


def loop_layout(base, size, k, unit):
    ptrs, lens, owner = [], [], []
    for t, (b, n) in enumerate(zip(base, size)):
        for off in range(0, int(n), unit):
            ptrs.append(int(b) + off)
            lens.append(min(unit, int(n) - off))
            owner.append(t)
    ns = max(1, -(-len(ptrs) // k))
    P = np.zeros((ns, k), np.uint64)
    L = np.zeros((ns, k), np.uint32)
    P.reshape(-1)[: len(ptrs)] = ptrs
    L.reshape(-1)[: len(lens)] = lens
    return np.array(owner, np.int64), P, L


@pytest.mark.parametrize("k,unit", [(12, 65536), (8, 4 << 20), (6, 16), (1, 4096)])
def test_unit_table_matches_loop(pkg, k, unit):
    from megatron_lm_amd.layout import unit_table
    rng = np.random.default_rng(k + unit)
    size = rng.integers(0, 5 * unit, 50)
    size[[3, 17]] = 0                      # empty tensors own no units
    size[5] = unit                         # exact multiple: no short tail
    base = np.cumsum(np.concatenate([[1 << 40], size[:-1] + 256])).astype(np.uint64)
    owner, idx, P, L = unit_table(base, size, k, unit)
    o2, P2, L2 = loop_layout(base, size, k, unit)
    assert np.array_equal(owner, o2)
    assert np.array_equal(P, P2) and np.array_equal(L, L2)
    assert L.sum() == size.sum()
    # unit index restarts at 0 in every tensor
    for t in np.unique(owner):
        assert np.array_equal(idx[owner == t], np.arange((owner == t).sum()))


def test_unit_table_config4_shape(pkg):
    from megatron_lm_amd.layout import unit_table
    n = int(20.8e9) // 14 * 14
    owner, idx, P, L = unit_table(np.array([1 << 40], np.uint64), np.array([n]), 8, 4 << 20)
    assert P.shape == (-(-n // (32 << 20)), 8)     # 620 stripes of 8 x 4 MiB
    assert P.shape[0] == 620
    assert L.sum() == n and (L[:-1] == 4 << 20).all()


def test_unit_table_empty(pkg):
    from megatron_lm_amd.layout import unit_table
    owner, idx, P, L = unit_table(np.array([5], np.uint64), np.array([0]), 4, 64)
    assert owner.size == 0 and P.shape == (1, 4) and not P.any() and not L.any()


def test_unit_table_empty_list(pkg):
    from megatron_lm_amd.layout import unit_table
    owner, idx, P, L = unit_table(np.zeros(0, np.uint64), np.zeros(0, np.int64), 6, 64)
    assert owner.size == 0 and P.shape == (1, 6) and not P.any() and not L.any()


def test_host_tensors_are_rejected_loudly(pkg):
    """No CPU fallback: host tensors are an error, not a silent slow path."""
    import torch
    cpu = [torch.zeros(64, dtype=torch.uint8) for _ in range(4)]
    for call in (lambda: pkg.xor_encode(cpu), lambda: pkg.rs_encode(cpu, 2),
                 lambda: pkg.encode(cpu, 4, 2, 64)):
        with pytest.raises(ValueError, match="device"):
            call()


def test_stripe_descriptors_high_addresses_and_large_tensors(pkg):
    """Addresses near the top of the 47-bit device range and tensors of tens
    of GB: the per-unit address arithmetic stays exact (int64 throughout)."""
    from megatron_lm_amd.layout import stripe_descriptors
    unit = 4 << 20
    size = np.array([(24 << 30) + 12345, 0, 7, (3 << 30) + unit], np.int64)
    base = np.array([0x7F00_0000_0000, 0x7F10_0000_0000, 0x7F20_0000_0000, 0x7FF0_0000_0000],
                    np.uint64)
    n_units, P, L = stripe_descriptors(base, size, 8, unit)
    o2, P2, L2 = loop_layout(base, size, 8, unit)
    assert n_units == o2.size
    assert np.array_equal(P, P2) and np.array_equal(L, L2)
    assert int(P.max()) == 0x7FF0_0000_0000 + (3 << 30)
