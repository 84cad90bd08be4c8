"""The ATM three-body kernels (xnn_atm_plan / xnn_atm_energy / xnn_atm_energy_backward)
against the oracle's edge-list restatement of the reference (oracle/d4.py atm_edges,
dispersion.py:124-222), energies and first derivatives, float64.

Systems as in the reference's tests (tests/common/test_dispersion_fast.py:21-70): rigid
water boxes on a 3.104 A grid with a 6 A three-body cutoff and a 1 A switch; the 3^3 cell
(9.3 A) is narrower than twice the cutoff, so it has repeated-atom triangles (all with a
third side beyond the cutoff), the 4^3 cell (12.4 A) has none, and the cluster has no
cell; the 2^3 cell (6.2 A) with a 7 A cutoff has atoms that see their own images and
repeated-atom triangles that count. Tolerance: 1e-11 relative to the largest
value (the reference's fast-path tolerance for float64, test_dispersion_fast.py:102-115).
"""
import math

import numpy as np
import pytest
import torch

import oracle.d4 as D

pytestmark = pytest.mark.gpu

WATER = np.array([[0.0, 0.0, 0.119262], [0.0, 0.763239, -0.477047],
                  [0.0, -0.763239, -0.477047]])
SPACING = 3.104
TOL = 1e-11


def _water_box(n_side, periodic, seed=3):
    rng = np.random.default_rng(seed)
    pos = []
    for i in range(n_side):
        for j in range(n_side):
            for k in range(n_side):
                q, _ = np.linalg.qr(rng.normal(size=(3, 3)))
                q *= np.sign(np.linalg.det(q))
                pos.extend((WATER - WATER[0]) @ q.T + np.array([i, j, k]) * SPACING
                           + rng.normal(scale=0.1, size=3))
    cell = np.eye(3) * SPACING * n_side if periodic else None
    return np.array(pos), cell, [8, 1, 1] * n_side ** 3


SYSTEMS = {"small_cell": (3, True, 6.0), "cell": (4, True, 6.0), "cluster": (3, False, 6.0),
           "tiny_cell": (2, True, 7.0)}


def _case(system, k=23, width_aa=1.0, seed=0):
    n_side, periodic, cutoff_aa = SYSTEMS[system]
    pos, cell, z = _water_box(n_side, periodic)
    dst, src, sh = D.pair_images(pos, cell, cutoff_aa)
    perm = torch.randperm(len(dst), generator=torch.Generator().manual_seed(seed))
    ei = torch.stack([torch.as_tensor(src), torch.as_tensor(dst)])[:, perm]
    sh = torch.as_tensor(sh, dtype=torch.float64)[perm]
    n = len(z)
    g = torch.Generator().manual_seed(seed + 1)
    fa = torch.rand(n, k, dtype=torch.float64, generator=g) + 0.2
    # C6 factors as in D4 and D3: <fa[x], fb[y]> symmetric in x, y (fb = fa M, M symmetric);
    # which edge of a pair comes first is then immaterial
    r = torch.rand(k, k, dtype=torch.float64, generator=g)
    mix = torch.eye(k, dtype=torch.float64) + 0.1 * (r @ r.t()) / k
    tables = dict(np.load(D_TABLES, allow_pickle=False))
    table, species = D.bj_radius_factors(torch.tensor(z), tables, 0.40085597, 5.02928789)
    return dict(ei=ei, shift=sh, pos=torch.as_tensor(pos),
                cell=None if cell is None else torch.as_tensor(cell), fa=fa, mix=mix,
                species=species, table=table, n=n,
                cutoff=cutoff_aa / D.BOHR, width=width_aa / D.BOHR)


D_TABLES = __import__("os").path.join(__import__("os").path.dirname(__file__), "golden",
                                      "d4_tables_hcnoar.npz")


def _rel(a, b):
    scale = float(b.abs().max())
    return float((a.detach().cpu() - b.detach()).abs().max()) / max(scale, 1e-300)


def _geometry(c, dev):
    """Edge vectors (bohr) as a differentiable function of positions and cell: per-edge
    gradients are not unique (an edge and its reverse carry the same geometry, and the
    kernels assign each distinct triangle to one corner's edges), the forces and the
    cell gradient are."""
    pos = c["pos"].detach().to(dev).clone().requires_grad_(True)
    cell = None if c["cell"] is None else c["cell"].detach().to(dev).clone().requires_grad_(True)
    ei = c["ei"].to(dev)
    vec = pos[ei[1]] - pos[ei[0]]
    if cell is not None:
        vec = vec + c["shift"].to(dev) @ cell
    return pos, cell, vec / D.BOHR


def _grads(e, go, pos, cell, fa):
    (e * go).sum().backward()
    return (e.detach(), pos.grad, fa.grad) + (() if cell is None else (cell.grad,))


def _oracle(c, same=False, s9=1.0, alp3=16.0 / 3.0, go=None):
    pos, cell, vec = _geometry(c, "cpu")
    fa = c["fa"].clone().requires_grad_(True)
    fb = fa if same else fa @ c["mix"]
    e = D.atm_edges(c["ei"], vec, fa, fb, c["species"], c["table"], s9, alp3, c["cutoff"],
                    c["width"], c["n"])
    return _grads(e, go, pos, cell, fa)


def _hip(c, same=False, s9=1.0, alp3=16.0 / 3.0, go=None):
    from xnn_amd import dispersion as XD
    dev = torch.device("cuda:0")
    pos, cell, vec = _geometry(c, dev)
    fa = c["fa"].to(dev).requires_grad_(True)
    fb = fa if same else fa @ c["mix"].to(dev)
    consts = XD.ATMConstants(c["species"].to(dev), c["table"].to(dev), s9, alp3, c["cutoff"],
                             c["width"])
    e = XD.atm_energy(c["ei"].to(dev), vec, fa, fb, consts, c["n"])
    out = _grads(e, go.to(dev), pos, cell, fa)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("system", list(SYSTEMS))
@pytest.mark.parametrize("k,width_aa", [(23, 1.0), (28, 0.0), (7, 1.0), (32, 1.0)])
def test_atm_matches_the_oracle(system, k, width_aa):
    print(f"[atm] {system} k={k} width={width_aa}", flush=True)
    c = _case(system, k=k, width_aa=width_aa)
    go = torch.rand(c["n"], dtype=torch.float64, generator=torch.Generator().manual_seed(9)) + 0.5
    ref = _oracle(c, go=go)
    out = _hip(c, go=go)
    assert float(ref[0].abs().max()) > 0
    for name, a, b in zip(("energy", "grad_pos", "grad_feat", "grad_cell"), out, ref):
        assert _rel(a, b) < TOL, (name, _rel(a, b))


def test_atm_shared_factors_and_plan_modes():
    """feat_a is feat_b (the D4 use) sums both factor gradients; the small cell has
    repeated-atom triangles and the 12.4 A cell none (test_dispersion_fast.py:118-131)."""
    from xnn_amd import dispersion as XD
    c = _case("small_cell", k=23)
    go = torch.ones(c["n"], dtype=torch.float64)
    ref = _oracle(c, same=True, go=go)
    out = _hip(c, same=True, go=go)
    for name, a, b in zip(("energy", "grad_pos", "grad_f", "grad_cell"), out, ref):
        assert _rel(a, b) < TOL, name
    _, info = XD.atm_plan(c["ei"].cuda(), c["n"])
    assert info[0] >= 1 and info[1] == 1
    big = _case("cell", k=23)
    _, info = XD.atm_plan(big["ei"].cuda(), big["n"])
    assert info[1] == 0


def test_atm_edge_cases():
    """No edges, a lone pair (no triangle), s9 = 0, and an index out of range."""
    from xnn_amd import dispersion as XD
    dev = torch.device("cuda:0")
    consts = XD.ATMConstants(torch.zeros(3, dtype=torch.int32, device=dev),
                             torch.ones(1, 1, dtype=torch.float64, device=dev), 1.0, 16 / 3, 10.0,
                             0.0)
    f = torch.ones(3, 23, dtype=torch.float64, device=dev)
    e = XD.atm_energy(torch.zeros(2, 0, dtype=torch.long, device=dev),
                      torch.zeros(0, 3, dtype=torch.float64, device=dev), f, f, consts, 3)
    assert e.shape == (3,) and float(e.abs().sum()) == 0.0
    ei = torch.tensor([[0, 1], [1, 0]], device=dev)
    v = torch.tensor([[1.0, 0, 0], [-1.0, 0, 0]], dtype=torch.float64, device=dev)
    assert float(XD.atm_energy(ei, v, f, f, consts, 3).abs().sum()) == 0.0
    c = _case("cluster", k=23)
    go = torch.ones(c["n"], dtype=torch.float64)
    out = _hip(c, s9=0.0, go=go)
    assert float(out[0].abs().max()) == 0.0 and float(out[1].abs().max()) == 0.0
    bad = torch.tensor([[0, 5], [1, 0]], device=dev)
    with pytest.raises(RuntimeError, match="outside"):
        XD.atm_energy(bad, v, f, f, consts, 3)


def test_atm_counts_match_a_direct_enumeration():
    """xnn_atm_count (the roofline's triangle counts): pairs of edges to larger-index
    neighbors per center, the distinct triangles among them with the third side within
    the cutoff, and the repeated-atom visits, against a direct enumeration on the CPU."""
    import ctypes
    from xnn_amd import _lib
    from xnn_amd import dispersion as XD
    c = _case("tiny_cell", k=23)
    pos, cell, vec = _geometry(c, "cpu")
    vec = vec.detach()
    n, ei = c["n"], c["ei"]
    key = ei[1] * n + ei[0]
    order = torch.argsort(key, stable=True)
    src, dst, v = ei[0][order].numpy(), ei[1][order], vec[order].numpy()
    lo = torch.searchsorted(dst, torch.arange(n + 1))
    cut2 = c["cutoff"] ** 2
    tested = kept = repeated = 0
    for cc in range(n):
        l, h = int(lo[cc]), int(lo[cc + 1])
        row = src[l:h]
        up = [p for p in range(l, h) if int(src[p]) > cc]
        tested += len(up) * (len(up) - 1) // 2
        for ia, a in enumerate(up):
            for b in up[ia + 1:]:
                w2 = float(((v[a] - v[b]) ** 2).sum())
                kept += int(src[a] != src[b] and 2.220446049250313e-16 < w2 <= cut2)
        for a in range(l, h):
            for b in range(a + 1, h):
                if src[a] == cc or src[b] == cc or src[a] == src[b]:
                    w2 = float(((v[a] - v[b]) ** 2).sum())
                    repeated += int(2.220446049250313e-16 < w2 <= cut2)
    dev = torch.device("cuda:0")
    plan, info = XD.atm_plan(ei.to(dev), n)
    counts = (ctypes.c_int64 * 3)()
    vd = vec.to(dev).contiguous()
    _lib.call("xnn_atm_count", _lib.ptr(plan), int(ei.shape[1]), n, info[0], _lib.ptr(vd),
              c["cutoff"], counts, _lib.stream(dev))
    assert (counts[0], counts[1], counts[2]) == (tested, kept, repeated)
    assert repeated > 0 and kept > 0


@pytest.mark.parametrize("shape", ["equilateral", "right_isosceles"])
def test_atm_kernel_triangle_closed_forms(shape):
    """One triangle of identical atoms through the HIP kernels: each corner gets a third of
    s9 C6^(3/2) (3 cos a cos b cos c + 1) / (r1 r2 r3)^3 / (1 + 6 (R0^3 / (r1 r2 r3))^alp3)
    -- the equilateral angular factor 3/8 + 1, the right angle's 1 -- with C6 = <f, f>."""
    from xnn_amd import dispersion as XD
    dev = torch.device("cuda:0")
    a = 6.5
    if shape == "equilateral":
        pos = np.array([[0.0, 0, 0], [a, 0, 0], [a / 2, a * math.sqrt(3) / 2, 0]])
        sides = (a, a, a)
    else:
        pos = np.array([[0.0, 0, 0], [a, 0, 0], [0, a, 0]])
        sides = (a, a, a * math.sqrt(2))
    f = torch.full((3, 23), 0.7, dtype=torch.float64, device=dev)
    c6 = float((f[0] * f[0]).sum())
    r0 = 4.3
    consts = XD.ATMConstants(torch.zeros(3, dtype=torch.int32, device=dev),
                             torch.full((1, 1), r0, dtype=torch.float64, device=dev), 1.0,
                             16.0 / 3.0, 50.0, 0.0)
    pt = torch.tensor(pos, dtype=torch.float64, device=dev)
    ei = torch.tensor([[j, i] for i in range(3) for j in range(3) if i != j], device=dev).t()
    e = XD.atm_energy(ei, pt[ei[1]] - pt[ei[0]], f, f, consts, 3)
    r1, r2, r3 = sides
    cos = [(r2 * r2 + r3 * r3 - r1 * r1) / (2 * r2 * r3), (r1 * r1 + r3 * r3 - r2 * r2) / (2 * r1 * r3),
           (r1 * r1 + r2 * r2 - r3 * r3) / (2 * r1 * r2)]
    prod = r1 * r2 * r3
    want = c6 ** 1.5 * (3 * cos[0] * cos[1] * cos[2] + 1) / prod ** 3 / (1 + 6 * (r0 ** 3 / prod) ** (16 / 3))
    np.testing.assert_allclose(e.cpu().numpy(), want / 3.0, rtol=1e-13)


@pytest.mark.parametrize("same", [True, False])
def test_atm_structure_energy_from_the_backward_launch(same):
    """atm_structure_energy: per-structure energies and their gradients from one launch of
    the ATM backward at unit seeds (each triangle's energy homogeneous of degree three in the
    features: total = 1/3 sum_i (fa_i . dE/dfa_i + fb_i . dE/dfb_i)), against the energy
    launch plus its backward: a periodic and a molecular structure in one batch, seeds 2 and
    -1.5 on their energies; with shared factors (the D4 form) also the per-atom energies."""
    from xnn_amd import dispersion as XD
    dev = torch.device("cuda:0")
    print(f"[gpu-case] atm structure energy, same={same}", flush=True)
    c1, c2 = _case("small_cell", seed=4), _case("cluster", seed=5)
    n1, n2 = c1["n"], c2["n"]
    ei = torch.cat([c1["ei"], c2["ei"] + n1], 1).to(dev)
    node_ptr = torch.tensor([0, n1, n1 + n2], dtype=torch.int64, device=dev)
    batch32 = torch.cat([torch.zeros(n1), torch.ones(n2)]).to(device=dev, dtype=torch.int32)
    seed = torch.tensor([2.0, -1.5], dtype=torch.float64, device=dev)
    fa0 = torch.cat([c1["fa"], c2["fa"]]).to(dev)
    consts = XD.ATMConstants(torch.cat([c1["species"], c2["species"]]).to(dev),
                             c1["table"].to(dev), 1.0, 16.0 / 3.0, c1["cutoff"], c1["width"])
    res = []
    for fused in (False, True):
        pos1, cell1, v1 = _geometry(c1, dev)
        pos2, _, v2 = _geometry(c2, dev)
        vec = torch.cat([v1, v2])
        fa = fa0.clone().requires_grad_(True)
        fb = fa if same else fa @ c1["mix"].to(dev)
        if fused:
            e_b, e_atom = XD.atm_structure_energy(ei, vec, fa, fb, consts, node_ptr, batch32)
            assert not e_atom.requires_grad
        else:
            e_atom = XD.atm_energy(ei, vec, fa, fb, consts, n1 + n2)
            e_b = torch.stack([e_atom[:n1].sum(), e_atom[n1:].sum()])
        (e_b * seed).sum().backward()
        res.append((e_b.detach(), e_atom.detach(), pos1.grad, cell1.grad, pos2.grad, fa.grad))
    torch.cuda.synchronize()
    ref, got = res
    assert _rel(got[0].cpu(), ref[0].cpu()) < 1e-12
    for a, b in zip(got[2:], ref[2:]):
        assert _rel(a.cpu(), b.cpu()) < 1e-11
    if same:
        assert _rel(got[1].cpu(), ref[1].cpu()) < 1e-11


@pytest.mark.parametrize("system", ["tiny_cell", "large_cell"])
def test_atm_is_reproducible_bit_for_bit(system):
    """Two evaluations of the energies and of every gradient give the same bits: the kernels'
    atomic sums are exact sums of fixed-quantum parts (a head of multiples of 2^-40 and a
    tail of multiples of 2^-70), whose value does not depend on the order of the atomics.
    The tiny cell has repeated-atom triangles; the 6^3 cell with an 8 A cutoff (648 atoms)
    gives every factor-gradient row thousands of atomic contributions."""
    print(f"[gpu-case] atm run twice, {system}", flush=True)
    if system == "large_cell":
        SYSTEMS["large_cell"] = (6, True, 8.0)
    try:
        c = _case(system, k=23)
    finally:
        SYSTEMS.pop("large_cell", None)
    go = torch.rand(c["n"], dtype=torch.float64, generator=torch.Generator().manual_seed(9)) + 0.5
    first = _hip(c, go=go)
    second = _hip(c, go=go)
    assert float(first[0].abs().max()) > 0
    for name, a, b in zip(("energy", "grad_pos", "grad_feat", "grad_cell"), first, second):
        assert torch.equal(a, b), name


def _second(c, dev, same, width_aa, seed=11):
    """Second derivatives of a force-loss-like scalar through the ATM energies: with
    L1 = sum_i go_i E_i and g = dL1/d(pos, feat[, cell]) formed with create_graph,
    L2 = <g, (U, V[, C])>, the gradients of L2 in pos, feat, go[, cell] (the Hessian of L1
    times the direction, and the energies' derivative along it)."""
    from xnn_amd import dispersion as XD
    g = torch.Generator().manual_seed(seed)
    n, k = c["fa"].shape
    go = (torch.rand(n, dtype=torch.float64, generator=g) + 0.5).to(dev).requires_grad_(True)
    U = torch.randn(n, 3, dtype=torch.float64, generator=g).to(dev)
    V = torch.randn(n, k, dtype=torch.float64, generator=g).to(dev)
    C = torch.randn(3, 3, dtype=torch.float64, generator=g).to(dev)
    pos, cell, vec = _geometry(c, dev)
    fa = c["fa"].to(dev).clone().requires_grad_(True)
    fb = fa if same else fa @ c["mix"].to(dev)
    if dev == "cpu":
        e = D.atm_edges(c["ei"], vec, fa, fb, c["species"], c["table"], 1.0, 16.0 / 3.0,
                        c["cutoff"], c["width"], c["n"])
    else:
        consts = XD.ATMConstants(c["species"].to(dev), c["table"].to(dev), 1.0, 16.0 / 3.0,
                                 c["cutoff"], c["width"])
        e = XD.atm_energy(c["ei"].to(dev), vec, fa, fb, consts, c["n"])
    wrt = [pos, fa] + ([] if cell is None else [cell])
    first = torch.autograd.grad((e * go).sum(), wrt, create_graph=True)
    l2 = (first[0] * U).sum() + (first[1] * V).sum()
    if cell is not None:
        l2 = l2 + (first[2] * C).sum()
    out = torch.autograd.grad(l2, wrt + [go])
    if dev != "cpu":
        torch.cuda.synchronize()
    return [x.detach().cpu() for x in out]


@pytest.mark.parametrize("system", list(SYSTEMS))
@pytest.mark.parametrize("same,width_aa", [(False, 1.0), (True, 0.0)])
def test_atm_second_derivatives_match_the_oracle(system, same, width_aa):
    """The ATM gradient is itself differentiable (dispersion_fast/atm.py:446-509): the
    Hessian-vector products in positions, factors and cell and the derivative in the
    energy cotangents, against autograd's second derivatives of the oracle's edge-list
    formula; every plan mode (repeated-atom triangles in the 2^3 and 3^3 cells), both
    switches, shared and separate factor matrices. Tolerance 1e-10 of the largest value
    (forward-mode numbers through the closed-form gradient vs. autograd's reverse-over-
    reverse: different rounding paths)."""
    print(f"[atm second] {system} same={same} width={width_aa}", flush=True)
    c = _case(system, k=23, width_aa=width_aa)
    ref = _second(c, "cpu", same, width_aa)
    out = _second(c, "cuda:0", same, width_aa)
    names = ["pos", "feat"] + (["cell"] if c["cell"] is not None else []) + ["go"]
    for name, a, b in zip(names, out, ref):
        assert float(b.abs().max()) > 0, name
        assert _rel(a, b) < 1e-10, (name, _rel(a, b))
    again = _second(c, "cuda:0", same, width_aa)
    for name, a, b in zip(names, out, again):
        assert torch.equal(a, b), f"{name}: the second derivatives differ run to run"


def test_atm_third_derivative_is_refused():
    """Second derivatives with a graph of their own (a third derivative) are refused, as
    the reference's once_differentiable tangent backward does (atm.py:494)."""
    from xnn_amd import dispersion as XD
    c = _case("cluster", k=23)
    dev = "cuda:0"
    pos, _, vec = _geometry(c, dev)
    fa = c["fa"].to(dev)
    consts = XD.ATMConstants(c["species"].to(dev), c["table"].to(dev), 1.0, 16.0 / 3.0,
                             c["cutoff"], c["width"])
    e = XD.atm_energy(c["ei"].to(dev), vec, fa, fa, consts, c["n"])
    (g,) = torch.autograd.grad(e.sum(), [pos], create_graph=True)
    with pytest.raises(RuntimeError, match="differentiable twice"):
        torch.autograd.grad((g * g).sum(), [pos], create_graph=True)
