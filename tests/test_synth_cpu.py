"""The seeded host generators of the benchmark configurations: the bytes of
the multi-GB configurations do not depend on the thread count, bf16 values
are fp32 draws rounded to nearest even, and the distributions have the
stated scale."""
import numpy as np
import pytest

import __graft_entry__

synth = None


@pytest.fixture(autouse=True)
def _synth(monkeypatch):
    global synth
    __graft_entry__.load_package()
    from megatron_lm_amd import synth as s
    # small chunks, so that a few MB cross many chunk boundaries
    monkeypatch.setattr(s, "GEN_CHUNK", 1 << 16)
    synth = s


def test_rank_buffer_independent_of_threads():
    a = synth.gpt_rank_buffer_host(7, nbytes=14 * 300_000, threads=1)
    b = synth.gpt_rank_buffer_host(7, nbytes=14 * 300_000, threads=5)
    assert a.size == b.size and np.array_equal(a, b)
    c = synth.gpt_rank_buffer_host(8, nbytes=14 * 300_000, threads=3)
    assert not np.array_equal(a, c)


def test_rank_buffer_segments():
    """bf16 params | fp32 master | fp32 exp_avg | fp32 exp_avg_sq in the
    2:4:4:4 byte ratio, with the stated standard deviations (and |N| for
    exp_avg_sq)."""
    n = 14 * 200_000
    buf = synth.gpt_rank_buffer_host(3, nbytes=n, threads=2)
    unit = n // 14
    seg = [2 * unit, 4 * unit, 4 * unit, 4 * unit]
    off = np.cumsum([0] + seg)
    bf = buf[off[0]:off[1]].view(np.uint16).astype(np.uint32) << 16
    vals = [bf.view(np.float32)] + [buf[off[i]:off[i + 1]].view(np.float32) for i in (1, 2, 3)]
    for v, (_, std, _, absolute) in zip(vals, synth.GPT_SEGMENTS):
        if absolute:
            assert v.min() >= 0 and abs(v.mean() / std - np.sqrt(2 / np.pi)) < 0.02
        else:
            assert abs(v.std() / std - 1) < 0.02 and abs(v.mean()) < 0.02 * std


def test_bf16_round_to_nearest_even():
    x = np.array([1.0, 1.00390625, 1.01171875, -2.5, 3.0e-8], np.float32)
    # 1 + 2^-8 is halfway between bf16 1.0 and 1 + 2^-7: ties to even (1.0);
    # 1 + 3 * 2^-8 ties up to 1 + 2^-6 (even mantissa)
    got = (synth.bf16_bits(x).astype(np.uint32) << 16).view(np.float32)
    assert got.tolist()[:4] == [1.0, 1.0, 1.015625, -2.5]


def test_ragged_host_independent_of_threads():
    block1, views1, kinds1 = synth.ragged_host(5, threads=1, n=40)
    block2, views2, kinds2 = synth.ragged_host(5, threads=6, n=40)
    assert np.array_equal(block1, block2) and np.array_equal(kinds1, kinds2)
    sizes, _ = synth.ragged_sizes(5, 40)
    assert [v.size for v in views1] == sizes.tolist()
    assert all(v.ctypes.data % 64 == 0 for v in views1)


def test_perturbation_is_seeded():
    """The 1 % perturbation: the unit choice and the new bytes are functions
    of the seed alone (the GPU tests and the bench draw them on the host and
    upload them, so a CPU re-encode sees the same bytes)."""
    u1 = synth.perturbed_units(5, 10_000, 0.01)
    assert u1.size == 100 and np.array_equal(u1, np.unique(u1))
    assert np.array_equal(u1, synth.perturbed_units(5, 10_000, 0.01))
    lens = np.array([65536, 17, 0, 4096])
    a = synth.perturbation_bytes(5, lens)
    b = synth.perturbation_bytes(5, lens)
    assert [x.size for x in a] == lens.tolist()
    assert all(np.array_equal(x, y) for x, y in zip(a, b))
    c = synth.perturbation_bytes(6, lens)
    assert not np.array_equal(a[0], c[0])
    # roughly uniform bytes
    assert abs(a[0].mean() - 127.5) < 2
