"""Pins of the oracle's counter-based noise (oracle/rng.c): published Philox4x32-10 known-answer vectors, an
independent numpy Philox, accuracy of the ln / sin / cos polynomials against libm in double, and normality of the
buffer."""
import math

import numpy as np
import pytest
from scipy import stats

from oracle import rng

# Random123 kat_vectors (Salmon et al., SC'11): philox4x32 with 10 rounds; (counter, key) -> output
KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize('ctr,key,want', KAT)
def test_philox_known_answers(ctr, key, want):
    assert rng.philox(ctr, key) == want


def test_philox_matches_independent_numpy():
    r = np.random.default_rng(0)
    c = r.integers(0, 2 ** 32, size=(4, 2000), dtype=np.uint64).astype(np.uint32)
    k0, k1 = 0x12345678, 0x9ABCDEF0
    out = rng.philox_numpy(*c, k0, k1)
    for j in range(0, 2000, 97):
        assert rng.philox(tuple(int(x) for x in c[:, j]), (k0, k1)) == tuple(int(o[j]) for o in out)


def test_ln_accuracy():
    us = np.concatenate([np.arange(1, 5000) * 2.0 ** -24, np.linspace(1e-6, 1.0, 20001)]).astype(np.float32)
    worst = 0.0
    for u in us[::7]:
        got = rng.ln(float(u))
        want = math.log(float(u))
        worst = max(worst, abs(got - want) / max(abs(want), 1e-30))
    assert worst < 5e-7, worst
    assert rng.ln(1.0) == 0.0


def test_sincos_accuracy():
    worst = 0.0
    for k in range(0, 1 << 24, 4099):
        u = k * 2.0 ** -24
        s, c = rng.sincos2pi(u)
        worst = max(worst, abs(s - math.sin(2 * math.pi * u)), abs(c - math.cos(2 * math.pi * u)))
    assert worst < 4e-7, worst


def test_buffer_is_standard_normal():
    z = rng.buffer(0, 0, 1 << 22).astype(np.float64)
    n = z.size
    assert abs(z.mean()) < 5 / math.sqrt(n)
    assert abs(z.var() - 1) < 5 * math.sqrt(2 / n)
    assert abs(stats.kurtosis(z)) < 0.02
    assert stats.kstest(z[::4], 'norm').pvalue > 1e-4
    # lanes 0-3 of a quad are independent draws
    q = z.reshape(-1, 4)
    cc = np.corrcoef(q.T)
    assert np.abs(cc - np.eye(4)).max() < 0.01


def test_buffer_slices_are_consistent():
    full = rng.buffer(9, 1000, 5000)
    for start, n in [(1000, 1), (1001, 7), (1003, 4000), (5999, 1)]:
        assert np.array_equal(rng.buffer(9, start, n), full[start - 1000:start - 1000 + n])


def test_offsets_range_and_rows():
    width = 4096 + 512
    off = rng.offsets(0, 3, 2, width, 5000)
    assert off.min() >= 0 and off.max() < rng.NOISE - width
    assert len(np.unique(off)) > 4990  # 2^28 range: collisions are rare
    # other step / parameter -> other offsets
    assert not np.array_equal(off, rng.offsets(0, 4, 2, width, 5000))
    assert not np.array_equal(off, rng.offsets(0, 3, 1, width, 5000))
    rows = rng.rows(0, off[:3], width)
    for j in range(3):
        assert np.array_equal(rows[j], rng.buffer(0, int(off[j]), width))
