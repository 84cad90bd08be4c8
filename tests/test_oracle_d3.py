"""The D3 oracle pinned against the reference's golden values and closed forms
(tests/common/test_d3.py:112-157). CPU only."""
import os

import numpy as np
import pytest

import oracle.d3 as D3
from oracle.d4 import BOHR

HERE = os.path.dirname(os.path.abspath(__file__))
WATER = (np.array([[0.0, 0.0, 0.119262], [0.0, 0.763239, -0.477047],
                   [0.0, -0.763239, -0.477047]]), [8, 1, 1])


@pytest.fixture(scope="module")
def tables():
    return dict(np.load(os.path.join(HERE, "golden", "d3_tables_hcnoar.npz"), allow_pickle=False))


def test_water_matches_simple_dftd3(tables):
    """PBE0-D3(BJ) and PBE0-D3(0) water, simple-dftd3 1.6.0 (test_d3.py:112-119)."""
    assert abs(float(D3.d3(*WATER, tables, "bj")["energy"]) - (-2.768885028766e-04)) < 1e-14
    assert abs(float(D3.d3(*WATER, tables, "zero")["energy"]) - (-4.644598055357e-06)) < 1e-16


@pytest.mark.parametrize("damping", ["bj", "zero", "mzero", "op"])
def test_damping_closed_forms_on_an_argon_dimer(tables, damping):
    """Each damping reproduces its formula on Ar2 at 5 A (test_d3.py:123-157)."""
    prm = dict(D3.PBE0_D3BJ if damping in ("bj", "op") else D3.PBE0_D3ZERO)
    if damping == "mzero":
        prm["bet"] = 0.1
    if damping == "op":
        prm["bet"] = 6.0
    out = D3.d3(np.array([[0.0, 0, 0], [5.0, 0, 0]]), [18, 18], tables, damping, prm)
    import torch
    c6 = float(D3.pair_c6(D3.species_of(tables, [18, 18]), out["weights"], torch.tensor([0]),
                          torch.tensor([1]), tables))
    r = 5.0 / BOHR
    q = float(tables["r4r2"][list(tables["z"]).index(18)])
    rr = 3 * q * q
    s6, s8, alp = prm["s6"], prm["s8"], prm["alp"]
    rvdw = float(tables["rvdw"][4, 4])
    if damping == "bj":
        r0 = prm["a1"] * rr ** 0.5 + prm["a2"]
        e = -c6 * (s6 / (r ** 6 + r0 ** 6) + s8 * rr / (r ** 8 + r0 ** 8))
    elif damping == "zero":
        e = -c6 * (s6 / (1 + 6 * (prm["rs6"] * rvdw / r) ** alp) / r ** 6
                   + s8 * rr / (1 + 6 * (prm["rs8"] * rvdw / r) ** (alp + 2)) / r ** 8)
    elif damping == "mzero":
        b = prm["bet"] * rvdw
        e = -c6 * (s6 / (1 + 6 * (r / (prm["rs6"] * rvdw) + b) ** (-alp)) / r ** 6
                   + s8 * rr / (1 + 6 * (r / (prm["rs8"] * rvdw) + b) ** (-alp - 2)) / r ** 8)
    else:
        r0 = prm["a1"] * rr ** 0.5 + prm["a2"]
        b = prm["bet"]
        e = -c6 * (s6 * r ** b / (r ** (6 + b) + r0 ** (6 + b))
                   + s8 * rr * r ** b / (r ** (8 + b) + r0 ** (8 + b)))
    assert abs(float(out["energy"]) - e) < 1e-15 * max(1.0, abs(e) * 1e3)


def test_reference_table_sanity(tables):
    """C6 of free Ar near the 2010 paper's 64.2 (test_d3.py:100-110), H/C reference
    counts, table symmetry, C-C pair radius 2.9103 A."""
    zs = list(tables["z"])
    ar, c = zs.index(18), zs.index(6)
    assert abs(float(tables["c6ref"][0, 0, ar, ar]) / 64.2 - 1) < 0.02
    assert int(tables["nref"][zs.index(1)]) == 2 and int(tables["nref"][c]) == 5
    np.testing.assert_array_equal(tables["c6ref"], tables["c6ref"].transpose(1, 0, 3, 2))
    assert abs(float(tables["rvdw"][c, c]) * BOHR - 2.9103) < 1e-6
