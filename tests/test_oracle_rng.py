"""The oracle's counter-based generator for the race's uniforms (Philox-4x32-10, Salmon et al.,
SC 2011), pinned by the published known-answer vectors of the Random123 library (kat_vectors:
philox4x32 with 10 rounds), and the mapping of its words to uniforms in (0, 1)."""
import numpy as np
import pytest

from oracle import sampler as O

KAT = [
    ([0x00000000, 0x00000000, 0x00000000, 0x00000000], [0x00000000, 0x00000000],
     [0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8]),
    ([0xffffffff, 0xffffffff, 0xffffffff, 0xffffffff], [0xffffffff, 0xffffffff],
     [0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd]),
    ([0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344], [0xa4093822, 0x299f31d0],
     [0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1]),
]


@pytest.mark.parametrize("ctr,key,want", KAT)
def test_philox_known_answers(ctr, key, want):
    assert O.philox4x32_10(ctr, key) == want


def test_uniform_mapping():
    """Token t takes word t % 4 of the block at counter (t / 4, offset lo, offset hi, 0), keyed
    by (seed lo, seed hi), as (2 floor(w / 2^9) + 1) 2^-24."""
    seed, off = 0x0123456789ABCDEF, 0x00000007FFFFFFFE
    u = O.philox_uniforms(np.array([seed], np.uint64), 64, np.array([off], np.uint64))[0]
    for t in range(64):
        w = O.philox4x32_10([t // 4, off & 0xFFFFFFFF, off >> 32, 0], [seed & 0xFFFFFFFF, seed >> 32])[t % 4]
        assert u[t] == np.float32((2 * (w >> 9) + 1) * 2.0 ** -24)


def test_uniforms_open_interval_and_distribution():
    seeds = np.arange(1, 65, dtype=np.uint64) * np.uint64(0x9E3779B97F4A7C15)
    u = O.philox_uniforms(seeds, 20000)
    assert u.dtype == np.float32 and u.shape == (64, 20000)
    assert np.all(u > 0) and np.all(u < 1)
    k = np.round(u.astype(np.float64) * 2 ** 24).astype(np.int64)
    assert np.all(k % 2 == 1)                      # odd multiples of 2^-24, exact
    assert abs(u.mean() - 0.5) < 2e-3
    hist = np.bincount(np.minimum((u * 16).astype(np.int64), 15).ravel(), minlength=16)
    expected = u.size / 16
    chi2 = float(((hist - expected) ** 2 / expected).sum())
    assert chi2 < 45.0                             # 15 degrees of freedom: p ~ 1e-4
    # rows with different seeds, and offsets, decorrelate
    assert abs(np.corrcoef(u[0], u[1])[0, 1]) < 0.05
    v = O.philox_uniforms(seeds[:1], 20000, np.array([1], np.uint64))
    assert not np.array_equal(u[:1], v)
