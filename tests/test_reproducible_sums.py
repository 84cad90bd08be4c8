"""The split behind the ATM kernels' reproducible atomic sums (csrc/atm.hip atm_acc): each
addend v is cut into a head, v rounded to a multiple of 2^-40, and a tail, the rest rounded
to a multiple of 2^-70; the heads and the tails are summed apart in float64. Checked here
in numpy against exact rational sums (math.fsum): the split is exact, every summation order
gives the same bits, and head + tail stays within 2^-71 per addend of the exact total."""
import math

import numpy as np


def _split(v):
    h = np.rint(v * 2.0 ** 40) * 2.0 ** -40
    t = np.rint((v - h) * 2.0 ** 70) * 2.0 ** -70
    return h, t


def test_the_split_is_exact_and_order_free():
    rng = np.random.default_rng(0)
    # magnitudes over 25 decades, both signs, as the kernels' gradient terms have, within
    # the range the exactness needs (sum |head| < 2^13)
    v = rng.standard_normal(20000) * 10.0 ** rng.uniform(-25, 0, 20000)
    h, t = _split(v)
    assert float(np.abs(h).sum()) < 2.0 ** 13
    # the head and the remainder v - h are exact: h + (v - h) gives v back
    assert np.array_equal(h + (v - h), v)
    assert float(np.abs(v - h).max()) <= 2.0 ** -41
    assert float(np.abs(v - h - t).max()) <= 2.0 ** -71
    totals = set()
    for seed in range(6):
        order = np.random.default_rng(seed).permutation(v.size)
        hs = ts = 0.0
        for i in order:                     # one float64 addition at a time, as the atomics
            hs += h[i]
            ts += t[i]
        assert hs == math.fsum(h) and ts == math.fsum(t)
        totals.add((hs + ts).hex())
    assert len(totals) == 1
    exact = math.fsum(v)
    got = float.fromhex(totals.pop())
    assert abs(got - exact) <= v.size * 2.0 ** -71 + abs(exact) * 2.0 ** -52


def test_a_plain_float64_sum_is_not_order_free():
    """The reason for the split: the same addends summed directly differ between orders."""
    rng = np.random.default_rng(0)
    v = rng.standard_normal(20000) * 10.0 ** rng.uniform(-25, 0, 20000)
    totals = set()
    for seed in range(6):
        s = 0.0
        for i in np.random.default_rng(seed).permutation(v.size):
            s += v[i]
        totals.add(s.hex())
    assert len(totals) > 1
