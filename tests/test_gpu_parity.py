"""GPU parity: every HIP entry point against the oracle on the same seeded inputs.

Bars: edge sets bit-exact after canonical sort (margin-checked inputs), integer/CSR
outputs exact, float32 energies rtol 1e-6, forces and stress atol 1e-5 (eV/A), float64
paths 1e-10; reductions bitwise reproducible run to run; the native library must be the
code that ran (call counters).
"""
import copy
import sys

import numpy as np
import pytest
import torch

from conftest import margin_checked_seed

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _note(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from xnn_amd import _lib
    _lib.load()  # the native library must load on a GPU box


def _canon_t(ei, sh):
    from oracle.nl import canonical
    return canonical(ei.cpu().numpy(), sh.cpu().numpy())


# --------------------------------------------------------------------------- radius graph
@pytest.mark.parametrize("name", ["argon", "water_small", "triclinic", "slab", "unwrapped"])
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_radius_graph_bit_exact(name, dtype):
    import xnn_amd as xa
    from xnn_amd import synthetic
    from oracle.nl import canonical
    tdt = torch.float32 if dtype == np.float32 else torch.float64
    if name == "argon":
        make, rc = (lambda seed: synthetic.argon_fcc(n_cells=4, seed=seed)), 6.0
    elif name == "water_small":
        make, rc = (lambda seed: synthetic.water_box(n_molecules=343, box=21.7, grid=7,
                                                     seed=seed)), 5.0
    elif name == "triclinic":
        def make(seed):
            rng = np.random.default_rng(seed)
            cell = np.array([[13.1, 0.0, 0.0], [2.7, 12.8, 0.0], [1.3, -2.4, 14.4]])
            pos = rng.uniform(0, 1, (300, 3)) @ cell
            return synthetic.Structure(pos, np.ones(300, np.int64), cell, np.array([1, 1, 1], bool))
        rc = 4.5
    elif name == "slab":
        def make(seed):
            rng = np.random.default_rng(seed)
            cell = np.eye(3) * 12.0
            pos = rng.uniform(0, 12, (250, 3))
            return synthetic.Structure(pos, np.ones(250, np.int64), cell, np.array([1, 0, 1], bool))
        rc = 4.0
    else:
        def make(seed):
            s = synthetic.argon_fcc(n_cells=3, seed=seed)
            rng = np.random.default_rng(seed + 100)
            s.pos = s.pos + rng.integers(-3, 4, s.pos.shape) @ s.cell
            return s
        rc = 6.0
    seed, s, ei, sh = margin_checked_seed(make, rc, dtype=dtype)
    _note(f"radius_graph {name} {dtype.__name__} seed={seed} N={len(s.pos)}")
    pos = torch.tensor(s.pos, dtype=tdt, device=DEV)
    e2, s2 = xa.build_neighbor_list(pos, rc, torch.tensor(s.cell, dtype=tdt, device=DEV),
                                    torch.tensor(s.pbc))
    assert e2.shape[1] == ei.shape[1]
    assert np.array_equal(_canon_t(e2, s2), canonical(ei, sh))
    # grouped by receiver: the CSR order of the kernels
    assert bool((e2[1][1:] >= e2[1][:-1]).all())


def test_radius_graph_full_water_box_bit_exact():
    import xnn_amd as xa
    from xnn_amd import synthetic
    from oracle.nl import canonical
    seed, s, ei, sh = margin_checked_seed(lambda sd: synthetic.water_box(seed=sd), 5.0)
    _note(f"radius_graph water 9000 seed={seed}")
    pos = torch.tensor(s.pos, dtype=torch.float32, device=DEV)
    e2, s2 = xa.build_neighbor_list(pos, 5.0, torch.tensor(s.cell, dtype=torch.float32,
                                                            device=DEV), torch.tensor(s.pbc))
    assert e2.shape[1] == ei.shape[1] > 400_000
    assert np.array_equal(_canon_t(e2, s2), canonical(ei, sh))


@pytest.mark.parametrize("case", ["cluster_16384", "cluster_16385", "cluster_20000_f64",
                                  "dilute_box_many_bins"])
def test_radius_graph_binning_paths(case):
    """The count step bins up to 16,384 atoms over at most 8,191 bins in one workgroup and
    larger systems through the general scatter and sort: both, at and past the boundary,
    against the oracle. Coordinates lie on a 1/8 A grid and the cutoff is 4.03 A, so every
    squared distance is a multiple of 1/64 at least 0.0066 from the cutoff's square: no pair
    lies near the cutoff."""
    import xnn_amd as xa
    from oracle.nl import canonical, neighbor_list
    rng = np.random.default_rng(7)
    rc, dtype = 4.03, (np.float64 if case.endswith("f64") else np.float32)
    if case.startswith("cluster"):
        n = int(case.split("_")[1])
        side = (n / 0.1) ** (1.0 / 3.0)
        pos, cell, pbc = np.round(rng.uniform(0, side, (n, 3)) * 8) / 8, None, None
    else:
        n, side = 1500, 100.0                  # 24^3 = 13,824 bins
        pos = np.round(rng.uniform(0, side, (n, 3)) * 8) / 8
        cell, pbc = np.eye(3) * side, [True] * 3
    _note(f"radius_graph binning path {case} N={n}")
    ei, sh, near = neighbor_list(pos, rc, cell, pbc, dtype=dtype, margin=1e-5)
    assert near == 0 and ei.shape[1] > 0
    tdt = torch.float32 if dtype == np.float32 else torch.float64
    args = (torch.tensor(pos, dtype=tdt, device=DEV), rc)
    kw = {} if cell is None else {"cell": torch.tensor(cell, dtype=tdt, device=DEV),
                                  "pbc": torch.tensor(pbc)}
    e2, s2 = xa.build_neighbor_list(*args, **kw)
    assert np.array_equal(_canon_t(e2, s2), canonical(ei, sh))
    assert bool((e2[1][1:] >= e2[1][:-1]).all())
    e3, s3 = xa.build_neighbor_list(*args, **kw)
    assert torch.equal(e2, e3) and torch.equal(s2, s3)


def test_radius_graph_edge_cases():
    import xnn_amd as xa
    from oracle.nl import canonical, neighbor_list
    _note("radius_graph edge cases")
    # empty and single atom
    e, s = xa.build_neighbor_list(torch.zeros((0, 3), device=DEV), 5.0)
    assert e.shape == (2, 0) and s.shape == (0, 3)
    e, s = xa.build_neighbor_list(torch.zeros((1, 3), device=DEV), 5.0)
    assert e.shape == (2, 0)
    # molecule, self-interaction, small cell (several images per axis)
    rng = np.random.default_rng(0)
    mol = rng.uniform(0, 6, (40, 3))
    e, s = xa.build_neighbor_list(torch.tensor(mol, device=DEV, dtype=torch.float64), 3.0)
    ei, sh, _ = neighbor_list(mol, 3.0, None, None, dtype=np.float64)
    assert np.array_equal(_canon_t(e, s), canonical(ei, sh))
    cell = np.eye(3) * 3.1
    pos = rng.uniform(0, 3.1, (5, 3))
    for si in (False, True):
        e, s = xa.build_neighbor_list(torch.tensor(pos, device=DEV, dtype=torch.float64), 4.0,
                                      torch.tensor(cell, device=DEV), torch.ones(3, dtype=torch.bool),
                                      self_interaction=si)
        ei, sh, _ = neighbor_list(pos, 4.0, cell, [True] * 3, self_interaction=si,
                                  dtype=np.float64)
        assert np.array_equal(_canon_t(e, s), canonical(ei, sh))
    # cells narrower than a third of the cutoff (the replicated-supercell listing): a
    # triclinic cell with every axis short, and one short axis of a slab
    tri = np.array([[4.1, 0.0, 0.0], [0.9, 3.8, 0.0], [-0.5, 0.7, 4.4]])
    pos = rng.uniform(0, 1, (7, 3)) @ tri
    for cut, pb in ((13.5, [True] * 3), (12.0, [True, False, True])):
        for si in (False, True):
            e, s = xa.build_neighbor_list(torch.tensor(pos, device=DEV, dtype=torch.float64), cut,
                                          torch.tensor(tri, device=DEV), torch.tensor(pb),
                                          self_interaction=si)
            ei, sh, _ = neighbor_list(pos, cut, tri, pb, self_interaction=si, dtype=np.float64)
            assert e.shape[1] == ei.shape[1] > 0
            assert np.array_equal(_canon_t(e, s), canonical(ei, sh))
            assert bool((e[1][1:] >= e[1][:-1]).all())
    # non-finite positions raise before any kernel runs
    bad = torch.tensor([[0.0, 0.0, float("nan")], [1.0, 0, 0]], device=DEV)
    with pytest.raises(ValueError, match="finite"):
        xa.build_neighbor_list(bad, 3.0)


def test_periodic_plan_reuse_keeps_the_edge_set():
    """A fully periodic cell tensor reused unchanged reuses its grid plan (no bounds read):
    positions that drift by whole and fractional cells (unwrapped), or a cell changed in
    place, give the edge set of a fresh build; a non-finite position still raises."""
    import oracle.nl as N
    import xnn_amd as xa
    from xnn_amd import data as D, synthetic
    from oracle.nl import canonical
    _note("periodic plan reuse")
    s = synthetic.water_box(n_molecules=216, box=18.6, grid=6, seed=10)   # margin-checked
    cell = torch.tensor(s.cell, dtype=torch.float32, device=DEV)
    pbc = torch.tensor(s.pbc)
    pos0 = torch.tensor(s.pos, dtype=torch.float32, device=DEV)
    xa.build_neighbor_list(pos0, 5.0, cell, pbc)              # plans and caches the grid
    key = (str(pos0.device), pos0.shape[0], torch.float32, 5.0, False)
    assert D._PERIODIC_PLANS[key][0]() is cell
    shift = torch.tensor([2.0, -1.0, 3.0], device=DEV) @ cell + 0.37
    jitter = 0.01 * torch.randn(pos0.shape, generator=torch.Generator().manual_seed(1))
    for pos in (pos0 + jitter.to(DEV), pos0 + shift):
        ei, sh = xa.build_neighbor_list(pos, 5.0, cell, pbc)
        ei_o, sh_o, near = N.neighbor_list(pos.cpu().numpy(), 5.0, s.cell, s.pbc,
                                           dtype=np.float32, margin=1e-5)
        assert near == 0             # no pair within 1e-5 A of the cutoff: the sets are exact
        assert np.array_equal(canonical(ei.cpu().numpy(), sh.cpu().numpy()), canonical(ei_o, sh_o))
    # the cell changed in place: a new plan (the version moved)
    with torch.no_grad():
        cell.mul_(1.05)
    ei, sh = xa.build_neighbor_list(pos0, 5.0, cell, pbc)
    assert D._PERIODIC_PLANS[key][1] == cell._version
    ei_o, sh_o, near = N.neighbor_list(pos0.cpu().numpy(), 5.0, cell.cpu().double().numpy(),
                                       s.pbc, dtype=np.float32, margin=1e-5)
    assert near == 0
    assert np.array_equal(canonical(ei.cpu().numpy(), sh.cpu().numpy()), canonical(ei_o, sh_o))
    # the same atoms compressed into another cell tensor: a new plan
    small = (cell / 1.05 * 0.8).contiguous()
    pos_small = (pos0 * 0.8).contiguous()
    ei, sh = xa.build_neighbor_list(pos_small, 5.0, small, pbc)
    assert D._PERIODIC_PLANS[key][0]() is small
    ei_o, sh_o, near = N.neighbor_list(pos_small.cpu().numpy(), 5.0, small.cpu().double().numpy(),
                                       s.pbc, dtype=np.float32, margin=1e-5)
    if near == 0:
        assert np.array_equal(canonical(ei.cpu().numpy(), sh.cpu().numpy()), canonical(ei_o, sh_o))
    else:
        assert abs(ei.shape[1] - ei_o.shape[1]) <= near
    bad = pos0.clone()
    bad[7, 1] = float("nan")
    with pytest.raises(ValueError, match="not finite"):
        xa.build_neighbor_list(bad, 5.0, cell, pbc)
    # a reused plan sizes its outputs from the last list (+5 %): a list that outgrows that
    # room (the atoms packed into half the cell, four times the edges) is filled again
    # exactly, and the next, smaller list fits the room of the larger one
    fresh = torch.tensor(s.cell, dtype=torch.float32, device=DEV)
    e0 = xa.build_neighbor_list(pos0, 5.0, fresh, pbc)[0].shape[1]
    packed = (pos0 * 0.5).contiguous()
    for pos in (packed, pos0):
        ei, sh = xa.build_neighbor_list(pos, 5.0, fresh, pbc)
        assert ei.is_contiguous() and sh.is_contiguous()
        ei_o, sh_o, near = N.neighbor_list(pos.cpu().numpy(), 5.0, s.cell, s.pbc,
                                           dtype=np.float32, margin=1e-5)
        print(f"capacity room: {ei.shape[1]} edges after {e0}; {near} pairs near the cutoff",
              flush=True)
        if near == 0:
            assert np.array_equal(canonical(ei.cpu().numpy(), sh.cpu().numpy()),
                                  canonical(ei_o, sh_o))
        else:
            assert abs(ei.shape[1] - ei_o.shape[1]) <= near
    assert ei.shape[1] == e0 and D._PERIODIC_PLANS[key][5][0] == e0


def test_neighbor_list_capacity_mode_eager_and_captured():
    """The capacity mode (grid_pairs.py:414-499 semantics): the edges of the ordinary list
    in the first n_edges entries, the rest repeating the first edge, n_edges on the device
    and above the capacity when the list does not fit; a call captured in a HIP graph and
    replayed on moved positions (eager work between replays) equals the ordinary list of
    those positions, periodic and molecular (atoms moving within the planned margin)."""
    import xnn_amd as xa
    from xnn_amd import synthetic
    from oracle.nl import canonical
    _note("neighbor list capacity mode")
    s = synthetic.water_box(n_molecules=216, box=18.6, grid=6, seed=5)
    rng = np.random.default_rng(11)
    for periodic in (True, False):
        pos0 = torch.tensor(s.pos, dtype=torch.float64, device=DEV)
        cell = torch.tensor(s.cell, dtype=torch.float64, device=DEV) if periodic else None
        pbc = torch.tensor(s.pbc) if periodic else None
        ei, sh = xa.build_neighbor_list(pos0, 5.0, cell, pbc)
        E = ei.shape[1]
        plan = xa.NeighborListPlan(pos0, 5.0, cell, pbc, margin=1.0)
        e2, s2, m = plan(pos0, E + 37)
        assert int(m) == E
        assert np.array_equal(canonical(e2[:, :E].cpu().numpy(), s2[:E].cpu().numpy()),
                              canonical(ei.cpu().numpy(), sh.cpu().numpy()))
        assert bool((e2[:, E:] == e2[:, :1]).all()) and bool((s2[E:] == s2[:1]).all())
        _, _, m_small = plan(pos0, E - 100)
        assert int(m_small) == E
        # captured: the static positions buffer is refilled before every replay
        cap = E + 2000
        pos_static = pos0.clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                plan(pos_static, cap)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = plan(pos_static, cap)
        for k in range(3):
            moved = pos0 + torch.tensor(rng.normal(0.0, 0.15, s.pos.shape), device=DEV)
            pos_static.copy_(moved)
            graph.replay()
            torch.cuda.synchronize()
            ref_ei, ref_sh = xa.build_neighbor_list(moved, 5.0, cell, pbc)   # eager work
            torch.cuda.synchronize()
            n = int(out[2])
            assert n == ref_ei.shape[1] <= cap, (periodic, k)
            assert np.array_equal(canonical(out[0][:, :n].cpu().numpy(), out[1][:n].cpu().numpy()),
                                  canonical(ref_ei.cpu().numpy(), ref_sh.cpu().numpy())), (periodic, k)


def test_unique_pairs_on_the_gpu_equal_the_cpu_pairs():
    """unique_pairs from the HIP cell list: the CPU formulation's pairs, sorted by the first
    atom (test_neighborlist_backends.py:156-174), for positions inside the cell or not."""
    import xnn_amd as xa
    from xnn_amd import synthetic
    _note("unique_pairs gpu")
    s = synthetic.water_box(n_molecules=100, box=14.4, grid=5, seed=3)
    for offset in (0.0, -3.7):
        pos = torch.tensor(s.pos, dtype=torch.float64) + offset * torch.diagonal(
            torch.tensor(s.cell))
        cell, pbc = torch.tensor(s.cell, dtype=torch.float64), torch.tensor(s.pbc)
        i0, k0, s0 = xa.unique_pairs(pos, 3.5, cell, pbc)
        i, k, sh = xa.unique_pairs(pos.to(DEV), 3.5, cell.to(DEV), pbc.to(DEV))
        want = {(int(a), int(b), *map(int, v)) for a, b, v in zip(i0, k0, s0)}
        got = {(int(a), int(b), *map(int, v)) for a, b, v in zip(i.cpu(), k.cpu(), sh.cpu())}
        assert got == want and len(got) == i.shape[0]
        assert bool((i[1:] >= i[:-1]).all())


def test_batched_molecules_match_per_structure():
    import xnn_amd as xa
    from xnn_amd import synthetic
    from oracle.nl import canonical, neighbor_list
    mols = synthetic.ragged_molecules(64, seed=3)
    _note("batched molecule radius graph, 64 ragged molecules")
    pos = torch.tensor(np.concatenate([m.pos for m in mols]), dtype=torch.float32, device=DEV)
    n_atoms = torch.tensor([len(m.pos) for m in mols])
    e, s = xa.batched_neighbor_list(pos, n_atoms, 5.0)
    parts, off = [], 0
    for m in mols:
        ei, sh, _ = neighbor_list(m.pos, 5.0, None, None, dtype=np.float32)
        parts.append((ei + off, sh))
        off += len(m.pos)
    ei = np.concatenate([p[0] for p in parts], 1)
    sh = np.concatenate([p[1] for p in parts], 0)
    assert np.array_equal(_canon_t(e, s), canonical(ei, sh))


# --------------------------------------------------------------------------- edge features
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_edge_vectors_and_their_backward(dtype):
    import oracle.reference as R
    import xnn_amd as xa
    from xnn_amd import synthetic
    from xnn_amd.ops import edge_vectors
    _note(f"edge_vectors {dtype}")
    s = synthetic.water_box(n_molecules=343, box=21.7, grid=7, seed=1)
    pos = torch.tensor(s.pos, dtype=dtype, device=DEV, requires_grad=True)
    cell = torch.tensor(s.cell, dtype=dtype, device=DEV, requires_grad=True)
    ei, sh = xa.build_neighbor_list(pos.detach(), 5.0, cell.detach(), torch.tensor(s.pbc))
    g = xa.AtomicGraph(pos=pos, atomic_numbers=torch.tensor(s.numbers, device=DEV), edge_index=ei,
                       cell_shifts=sh, batch=torch.zeros(len(s.pos), dtype=torch.long, device=DEV),
                       n_atoms=torch.tensor([len(s.pos)], device=DEV), cell=cell[None],
                       pbc=torch.tensor(s.pbc)[None])
    vec = g.edge_vectors()
    w = torch.randn(vec.shape, dtype=dtype, device=DEV, generator=torch.Generator(DEV).manual_seed(0))
    gp, gc = torch.autograd.grad((vec * w).sum(), (pos, cell))
    pos_c = pos.detach().cpu().double().requires_grad_(True)
    cell_c = cell.detach().cpu().double().requires_grad_(True)
    ref = R.edge_vectors(pos_c, ei.cpu(), sh.cpu(), cell_c[None])
    rp, rcl = torch.autograd.grad((ref * w.cpu().double()).sum(), (pos_c, cell_c))
    tol = 1e-5 if dtype == torch.float32 else 1e-12
    np.testing.assert_allclose(vec.detach().cpu().double(), ref.detach(), atol=tol)
    np.testing.assert_allclose(gp.cpu().double(), rp, atol=10 * tol)
    np.testing.assert_allclose(gc.cpu().double(), rcl, rtol=tol, atol=100 * tol)
    # bitwise reproducible
    gp2, gc2 = torch.autograd.grad((g.edge_vectors() * w).sum(), (pos, cell))
    assert torch.equal(gp, gp2) and torch.equal(gc, gc2)


@pytest.mark.parametrize("radial,envelope,l_max,sign", [("bessel", "polynomial", 3, 1),
                                                        ("bessel", "cosine", 2, -1),
                                                        ("gaussian", "polynomial", 1, 1),
                                                        ("gaussian", "cosine", 0, 1)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_edge_embed_and_backward(radial, envelope, l_max, sign, dtype):
    import oracle.reference as R
    from xnn_amd.featurizers import SphericalHarmonicEdgeEmbedding
    _note(f"edge_embed {radial} {envelope} l={l_max} sign={sign} {dtype}")
    gen = torch.Generator().manual_seed(4)
    vec = (torch.randn(5000, 3, generator=gen, dtype=torch.float64) * 2.5)
    vec[:3] = torch.tensor([[0.0, 0.0, 5.5], [1e-9, 0, 0], [0.0, 4.999, 0.0]], dtype=torch.float64)
    old = torch.get_default_dtype()
    torch.set_default_dtype(dtype)   # buffers (frequencies, centers) built in the run's dtype
    try:
        emb = SphericalHarmonicEdgeEmbedding(l_max=l_max, n_rbf=8, cutoff=5.0,
                                             radial_type=radial, envelope=envelope).to(DEV)
    finally:
        torch.set_default_dtype(old)
    emb.fast_active = True
    v = vec.to(DEV, dtype).requires_grad_(True)
    length, sh, rad = emb.embed(v, sh_sign=sign)
    wl = torch.randn(length.shape, generator=gen, dtype=torch.float64)
    ws = torch.randn(sh.shape, generator=gen, dtype=torch.float64)
    wr = torch.randn(rad.shape, generator=gen, dtype=torch.float64)
    loss = (length * wl.to(DEV, dtype)).sum() + (sh * ws.to(DEV, dtype)).sum() + \
        (rad * wr.to(DEV, dtype)).sum()
    (gv,) = torch.autograd.grad(loss, v)
    vc = vec.clone().requires_grad_(True)
    lr = torch.linalg.norm(vc, dim=-1)
    shr = R.e3nn_sh(l_max, vc if sign == 1 else -vc)
    rr = R.radial_features(lr, 8, 5.0, radial, envelope)
    lossr = (lr * wl).sum() + (shr * ws).sum() + (rr * wr).sum()
    (gr,) = torch.autograd.grad(lossr, vc)
    tol = 2e-5 if dtype == torch.float32 else 1e-11
    np.testing.assert_allclose(length.detach().cpu().double(), lr.detach(), rtol=tol, atol=tol)
    np.testing.assert_allclose(sh.detach().cpu().double()[3:], shr.detach()[3:], atol=tol * 5)
    np.testing.assert_allclose(rad.detach().cpu().double(), rr.detach(), atol=tol * 5)
    np.testing.assert_allclose(gv.cpu().double()[3:], gr[3:], rtol=tol * 10, atol=tol * 20)


# --------------------------------------------------------------------------- aggregation
@pytest.mark.parametrize("C,l_max,mfma", [(128, 3, True), (128, 3, False), (64, 3, True),
                                          (48, 3, True), (16, 3, True), (32, 2, True),
                                          (96, 1, True), (96, 1, False), (64, 0, True),
                                          (200, 0, True), (256, 3, True)])
def test_sh_message_sum_forward_backward(C, l_max, mfma, monkeypatch):
    """Matrix-core kernels (C = 16 T, T in 1..4, 6, 8) and vector-ALU kernels (the rest,
    or XNN_AMD_MESSAGE_MFMA=0) against the materialized messages of the oracle."""
    import oracle.reference as R
    import xnn_amd as xa
    from xnn_amd import synthetic
    from xnn_amd.ops import sh_message_sum
    monkeypatch.setenv("XNN_AMD_MESSAGE_MFMA", "1" if mfma else "0")
    _note(f"sh_message_sum C={C} l_max={l_max} mfma={mfma}")
    s = synthetic.water_box(n_molecules=216, box=18.6, grid=6, seed=2)
    g = xa.structure_to_graph(s.as_dict(), 5.0, device=DEV)
    g.pos = g.pos.float()
    vec = g.edge_vectors().detach().requires_grad_(True)
    gen = torch.Generator().manual_seed(C)
    phi = torch.randn(vec.shape[0], C, generator=gen).to(DEV).requires_grad_(True)
    A = sh_message_sum(vec, phi, g.plan(), l_max, 1)
    dA = torch.randn(A.shape, generator=gen).to(DEV)
    gvec, gphi = torch.autograd.grad((A * dA).sum(), (vec, phi))
    vc = vec.detach().cpu().double().requires_grad_(True)
    pc = phi.detach().cpu().double().requires_grad_(True)
    Y = R.e3nn_sh(l_max, vc)
    msg = (pc[:, :, None] * Y[:, None, :]).reshape(vc.shape[0], -1)
    Ar = R.scatter_sum(msg, g.edge_index[1].cpu(), g.num_nodes).reshape(A.shape)
    gv_r, gp_r = torch.autograd.grad((Ar * dA.cpu().double()).sum(), (vc, pc), allow_unused=True)
    if gv_r is None:                       # l_max = 0: Y_0 does not depend on the vector
        gv_r = torch.zeros_like(vc)
    scale = float(Ar.detach().abs().max())
    np.testing.assert_allclose(A.detach().cpu().double(), Ar.detach(), atol=2e-6 * scale)
    np.testing.assert_allclose(gphi.cpu().double(), gp_r, atol=2e-5 * float(gp_r.abs().max()))
    np.testing.assert_allclose(gvec.cpu().double(), gv_r, atol=2e-5 * max(1.0, float(gv_r.abs().max())))
    A2 = sh_message_sum(vec, phi, g.plan(), l_max, 1)
    assert torch.equal(A, A2)


@pytest.mark.parametrize("C,l_max,K", [(128, 3, 8), (64, 3, 8), (32, 2, 8), (64, 1, 5),
                                        (128, 2, 3)])
def test_sh_linear_message_sum_forward_backward(C, l_max, K):
    """The fused linear + message kernels against the oracle's materialized messages with
    phi = h W, for A, d_h, the edge-vector gradient and d_W (the last through the
    unfused backward)."""
    import oracle.reference as R
    import xnn_amd as xa
    from xnn_amd import synthetic
    from xnn_amd.ops import sh_linear_message_sum
    _note(f"sh_linear_message_sum C={C} l_max={l_max} K={K}")
    s = synthetic.water_box(n_molecules=216, box=18.6, grid=6, seed=3)
    g = xa.structure_to_graph(s.as_dict(), 5.0, device=DEV)
    g.pos = g.pos.float()
    vec = g.edge_vectors().detach().requires_grad_(True)
    gen = torch.Generator().manual_seed(100 * C + K)
    h = torch.randn(vec.shape[0], K, generator=gen).to(DEV).requires_grad_(True)
    W = (torch.randn(K, C, generator=gen) / K ** 0.5).to(DEV).requires_grad_(True)
    A = sh_linear_message_sum(vec, h, W, g.plan(), l_max, 1)
    dA = torch.randn(A.shape, generator=gen).to(DEV)
    gvec, gh, gW = torch.autograd.grad((A * dA).sum(), (vec, h, W))
    vc = vec.detach().cpu().double().requires_grad_(True)
    hc = h.detach().cpu().double().requires_grad_(True)
    Wc = W.detach().cpu().double().requires_grad_(True)
    Y = R.e3nn_sh(l_max, vc)
    phi = hc @ Wc
    msg = (phi[:, :, None] * Y[:, None, :]).reshape(vc.shape[0], -1)
    Ar = R.scatter_sum(msg, g.edge_index[1].cpu(), g.num_nodes).reshape(A.shape)
    gv_r, gh_r, gW_r = torch.autograd.grad((Ar * dA.cpu().double()).sum(), (vc, hc, Wc))
    scale = float(Ar.detach().abs().max())
    np.testing.assert_allclose(A.detach().cpu().double(), Ar.detach(), atol=2e-6 * scale)
    np.testing.assert_allclose(gh.cpu().double(), gh_r, atol=2e-5 * float(gh_r.abs().max()))
    np.testing.assert_allclose(gvec.cpu().double(), gv_r, atol=2e-5 * max(1.0, float(gv_r.abs().max())))
    np.testing.assert_allclose(gW.cpu().double(), gW_r, atol=2e-5 * float(gW_r.abs().max()))
    # without weight gradients the d_W pass is skipped; the rest is unchanged
    gvec2, gh2 = torch.autograd.grad((sh_linear_message_sum(vec, h, W.detach(), g.plan(), l_max, 1)
                                      * dA).sum(), (vec, h))
    assert torch.equal(gvec2, gvec) and torch.equal(gh2, gh)
    A2 = sh_linear_message_sum(vec, h, W, g.plan(), l_max, 1)
    assert torch.equal(A, A2)


@pytest.mark.parametrize("C,l_max,K,radial,envelope,sign,rc",
                         [(128, 3, 8, "bessel", "polynomial", 1, 5.0),
                          (64, 2, 8, "bessel", "cosine", -1, 5.0),
                          (128, 3, 8, "bessel_detuned", "polynomial", 1, 5.0),
                          (32, 1, 6, "gaussian", "polynomial", 1, 5.0),
                          (128, 3, 4, "gaussian", "cosine", 1, 5.0),
                          (128, 3, 8, "bessel", "polynomial", 1, 6.5)])
def test_sh_radial_message_sum_forward_backward(C, l_max, K, radial, envelope, sign, rc):
    """Radial basis, linear layer and message in one kernel each way, against the oracle's
    radial features (radial.py / cutoff.py restated), materialized messages and float64
    autograd; also against the two-kernel composition (edge_embed + the fused linear
    message), which must agree to float32 rounding."""
    import oracle.reference as R
    import xnn_amd as xa
    from xnn_amd import synthetic
    from xnn_amd.featurizers import SphericalHarmonicEdgeEmbedding
    from xnn_amd.ops import sh_linear_message_sum
    _note(f"sh_radial_message_sum C={C} l_max={l_max} K={K} {radial} {envelope} sign={sign} rc={rc}")
    s = synthetic.water_box(n_molecules=216, box=18.6, grid=6, seed=4)
    g = xa.structure_to_graph(s.as_dict(), rc, device=DEV)
    if rc > 6.0:
        # receiver rows longer than one 64-edge batch
        assert int(torch.bincount(g.edge_index[1]).max()) > 64
    g.pos = g.pos.float()
    vec = g.edge_vectors().detach().requires_grad_(True)
    emb = SphericalHarmonicEdgeEmbedding(l_max=l_max, n_rbf=K, cutoff=rc,
                                         radial_type=radial.split("_")[0],
                                         envelope=envelope).to(DEV)
    freqs = None
    if radial == "bessel_detuned":
        # frequencies off the n pi progression: the kernels evaluate one sincos per
        # function instead of the harmonic recurrence
        freqs = emb.rbf.freqs * (1.0 + 0.01 * torch.arange(K, device=DEV))
        emb.rbf.freqs.copy_(freqs)
    emb.fast_active = True
    gen = torch.Generator().manual_seed(7 * C + K)
    W = (torch.randn(K, C, generator=gen) / K ** 0.5).to(DEV)
    A = emb.radial_message_sum(vec, W, g.plan(), sign)
    dA = torch.randn(A.shape, generator=gen).to(DEV)
    (gvec,) = torch.autograd.grad((A * dA).sum(), (vec,))
    # oracle, float64
    vc = vec.detach().cpu().double().requires_grad_(True)
    Y = R.e3nn_sh(l_max, vc if sign == 1 else -vc)
    length = torch.linalg.norm(vc, dim=-1)
    if freqs is None:
        rad = R.radial_features(length, K, rc, radial, envelope)
    else:
        env = (R.polynomial_envelope(length, rc, 6) if envelope == "polynomial"
               else R.cosine_envelope(length, rc))
        rad = R.bessel(length, K, rc, freqs=freqs.cpu().double()) * env[:, None]
    phi = rad @ W.cpu().double()
    msg = (phi[:, :, None] * Y[:, None, :]).reshape(vc.shape[0], -1)
    Ar = R.scatter_sum(msg, g.edge_index[1].cpu(), g.num_nodes).reshape(A.shape)
    (gv_r,) = torch.autograd.grad((Ar * dA.cpu().double()).sum(), (vc,))
    scale = float(Ar.detach().abs().max())
    np.testing.assert_allclose(A.detach().cpu().double(), Ar.detach(), atol=2e-6 * scale)
    np.testing.assert_allclose(gvec.cpu().double(), gv_r, atol=2e-5 * max(1.0, float(gv_r.abs().max())))
    # the composition: radial features stored, then the fused linear message
    u = emb.radial(vec)
    A_c = sh_linear_message_sum(vec, u, W, g.plan(), l_max, sign)
    (gvec_c,) = torch.autograd.grad((A_c * dA).sum(), (vec,))
    np.testing.assert_allclose(A.detach().cpu(), A_c.detach().cpu(), atol=1e-6 * scale)
    np.testing.assert_allclose(gvec.cpu(), gvec_c.cpu(), atol=1e-6 * max(1.0, float(gv_r.abs().max())))
    # reproducible run to run
    A2 = emb.radial_message_sum(vec, W, g.plan(), sign)
    assert torch.equal(A, A2)
    # parameter gradients are refused, not silently dropped
    with pytest.raises(NotImplementedError):
        torch.autograd.grad(emb.radial_message_sum(vec, W.clone().requires_grad_(True), g.plan(),
                                                   sign).sum(), (vec,))


@pytest.mark.parametrize("C,l_max,K,radial,envelope,sign,rc",
                         [(128, 3, 8, "bessel", "polynomial", 1, 5.0),
                          (64, 2, 8, "bessel", "cosine", -1, 5.0),
                          (32, 1, 6, "gaussian", "polynomial", 1, 6.5),
                          (128, 3, 8, "bessel", "polynomial", 1, 6.5)])
def test_sh_radial_message_energy_forward_backward(C, l_max, K, radial, envelope, sign, rc):
    """The readout fused into the radial message kernels: E_i = <U, A_i> + bias[z_i] and the
    edge-vector gradient of sum_i g_i E_i, against the oracle (float64 autograd through the
    materialized messages and the readout) and against the A-row kernels followed by the
    readout (float32 rounding); a broadcast cotangent (the -1 seed of forces) equals the
    same cotangent spelled out per atom, bit for bit."""
    import oracle.reference as R
    import xnn_amd as xa
    from xnn_amd import synthetic
    from xnn_amd.featurizers import SphericalHarmonicEdgeEmbedding
    from xnn_amd.ops import node_readout_op
    _note(f"sh_radial_message_energy C={C} l_max={l_max} K={K} {radial} {envelope} sign={sign}")
    s = synthetic.water_box(n_molecules=216, box=18.6, grid=6, seed=4)
    g = xa.structure_to_graph(s.as_dict(), rc, device=DEV)
    g.pos = g.pos.float()
    vec = g.edge_vectors().detach().requires_grad_(True)
    emb = SphericalHarmonicEdgeEmbedding(l_max=l_max, n_rbf=K, cutoff=rc, radial_type=radial,
                                         envelope=envelope).to(DEV)
    emb.fast_active = True
    L = (l_max + 1) ** 2
    gen = torch.Generator().manual_seed(11 * C + K)
    W = (torch.randn(K, C, generator=gen) / K ** 0.5).to(DEV)
    U = (torch.randn(C, L, generator=gen) / (C * L) ** 0.5).to(DEV)
    bias = torch.randn(10, generator=gen).to(DEV)
    z = g.atomic_numbers
    E = emb.radial_message_energy(vec, W, U, z, bias, g.plan(), sign)
    gi = torch.randn(E.shape, generator=gen).to(DEV)
    (gvec,) = torch.autograd.grad((E * gi).sum(), (vec,))
    # the A-row kernels and the readout kernel
    A = emb.radial_message_sum(vec, W, g.plan(), sign)
    E_rows = node_readout_op(A.reshape(A.shape[0], -1), U.reshape(-1), z, bias)
    (gvec_rows,) = torch.autograd.grad((E_rows * gi).sum(), (vec,))
    e_scale = float(E_rows.abs().max())
    np.testing.assert_allclose(E.detach().cpu(), E_rows.detach().cpu(), atol=2e-6 * e_scale)
    g_scale = max(1.0, float(gvec_rows.abs().max()))
    np.testing.assert_allclose(gvec.cpu(), gvec_rows.cpu(), atol=1e-6 * g_scale)
    # oracle, float64
    vc = vec.detach().cpu().double().requires_grad_(True)
    Y = R.e3nn_sh(l_max, vc if sign == 1 else -vc)
    rad = R.radial_features(torch.linalg.norm(vc, dim=-1), K, rc, radial, envelope)
    msg = ((rad @ W.cpu().double())[:, :, None] * Y[:, None, :]).reshape(vc.shape[0], -1)
    Ar = R.scatter_sum(msg, g.edge_index[1].cpu(), g.num_nodes)
    Er = Ar @ U.cpu().double().reshape(-1) + bias.cpu().double()[z.cpu()]
    (gv_r,) = torch.autograd.grad((Er * gi.cpu().double()).sum(), (vc,))
    np.testing.assert_allclose(E.detach().cpu().double(), Er.detach(),
                               atol=2e-6 * float(Er.abs().max()))
    np.testing.assert_allclose(gvec.cpu().double(), gv_r,
                               atol=2e-5 * max(1.0, float(gv_r.abs().max())))
    # the broadcast seed equals the spelled-out one; run to run bit for bit
    minus = torch.full((1,), -1.0, device=DEV).expand(E.shape[0])
    (g_b,) = torch.autograd.grad([emb.radial_message_energy(vec, W, U, z, bias, g.plan(), sign)],
                                 [vec], grad_outputs=[minus])
    (g_f,) = torch.autograd.grad([emb.radial_message_energy(vec, W, U, z, bias, g.plan(), sign)],
                                 [vec], grad_outputs=[torch.full_like(E, -1.0)])
    assert torch.equal(g_b, g_f)
    assert torch.equal(E, emb.radial_message_energy(vec, W, U, z, bias, g.plan(), sign))
    # no bias; an atomic number outside the bias table is NaN, not a stray read
    E0 = emb.radial_message_energy(vec, W, U, z, None, g.plan(), sign)
    np.testing.assert_allclose((E - E0).detach().cpu(), bias[z].cpu(), atol=1e-5)
    E_bad = emb.radial_message_energy(vec.detach(), W, U, torch.full_like(z, 99), bias, g.plan(), sign)
    assert torch.isnan(E_bad).all()
    # one pass (energies and gradients from the backward launch alone): the same energies
    # to float32 rounding; gradients for a per-atom cotangent, a broadcast one and the
    # forces' cached -1 seed, against the forward + backward launches
    from xnn_amd.outputs import _minus_one
    E1 = emb.radial_message_energy(vec, W, U, z, bias, g.plan(), sign, one_pass=True)
    np.testing.assert_allclose(E1.detach().cpu(), E.detach().cpu(), atol=2e-6 * e_scale)
    (g1,) = torch.autograd.grad((E1 * gi).sum(), (vec,))
    np.testing.assert_allclose(g1.cpu(), gvec.cpu(), atol=1e-6 * g_scale)
    for seed in (torch.full((1,), 2.5, device=DEV).expand(E.shape[0]),
                 _minus_one(E).expand(E.shape[0])):
        (g1,) = torch.autograd.grad(
            [emb.radial_message_energy(vec, W, U, z, bias, g.plan(), sign, one_pass=True)],
            [vec], grad_outputs=[seed])
        (g0,) = torch.autograd.grad([emb.radial_message_energy(vec, W, U, z, bias, g.plan(), sign)],
                                    [vec], grad_outputs=[seed])
        np.testing.assert_allclose(g1.cpu(), g0.cpu(), atol=1e-6 * g_scale * 2.5)
    E1_bad = emb.radial_message_energy(vec, W, U, torch.full_like(z, 99), bias, g.plan(), sign,
                                       one_pass=True)
    assert torch.isnan(E1_bad).all()


def test_force_reduce_visit_order_keeps_every_sum():
    """The force reduction taken in the plan's spatial order (space-filling curve, XCD-wise
    runs) gives the forces and the per-atom cell and virial partials bit for bit as in
    index order (each atom's sums keep their order); the visit order is a permutation."""
    import xnn_amd as xa
    from xnn_amd import _lib, synthetic
    _note("force reduce visit order")
    for dtype in (torch.float32, torch.float64):
        s = synthetic.water_box(n_molecules=216, box=18.6, grid=6, seed=3)
        g = xa.structure_to_graph(s.as_dict(), 5.0, device=DEV)
        g.pos, g.cell = g.pos.to(dtype), g.cell.to(dtype)
        plan = g.plan()
        assert torch.equal(torch.sort(plan.visit.long()).values,
                           torch.arange(g.num_nodes, device=DEV))
        vec = g.edge_vectors().detach().contiguous()
        ge = torch.randn(vec.shape, generator=torch.Generator().manual_seed(5),
                         dtype=torch.float64).to(DEV, dtype)
        E, N, code = vec.shape[0], g.num_nodes, _lib.dtype_code(dtype)

        def run(visit):
            gp = torch.empty((N, 3), dtype=dtype, device=DEV)
            cp = torch.empty((N, 9), dtype=torch.float64, device=DEV)
            vp = torch.empty((N, 9), dtype=torch.float64, device=DEV)
            _lib.call("xnn_edge_force_reduce", code, code, _lib.ptr(ge), E, _lib.ptr(plan.ptr_dst),
                      _lib.ptr(plan.perm_dst), _lib.ptr(plan.ptr_src), _lib.ptr(plan.perm_src),
                      _lib.ptr(plan.shift), _lib.ptr(visit), N, _lib.ptr(gp), _lib.ptr(cp),
                      _lib.ptr(vec), _lib.ptr(vp), _lib.stream(vec.device))
            return gp, cp, vp

        for a, b in zip(run(None), run(plan.visit)):
            assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_force_reduce_with_virial_finish_matches_the_two_step_path(dtype):
    """xnn_edge_force_reduce_virial (one structure; block sums of the strain derivative
    added by one finishing block) gives the forces of xnn_edge_force_reduce bit for bit and
    the virial of its per-atom partials + xnn_virial_reduce to float64 rounding; repeated
    calls give the same bits; an empty structure gives a zero virial."""
    import xnn_amd as xa
    from xnn_amd import _lib, synthetic
    _note(f"force reduce + virial finish {dtype}")
    s = synthetic.water_box(n_molecules=216, box=18.6, grid=6, seed=3)
    g = xa.structure_to_graph(s.as_dict(), 5.0, device=DEV)
    g.pos, g.cell = g.pos.to(dtype), g.cell.to(dtype)
    plan = g.plan()
    vec = g.edge_vectors().detach().contiguous()
    ge = torch.randn(vec.shape, generator=torch.Generator().manual_seed(7),
                     dtype=torch.float64).to(DEV, dtype)
    E, N, code = vec.shape[0], g.num_nodes, _lib.dtype_code(dtype)
    gp = torch.empty((N, 3), dtype=dtype, device=DEV)
    vp = torch.empty((N, 9), dtype=torch.float64, device=DEV)
    _lib.call("xnn_edge_force_reduce", code, code, _lib.ptr(ge), E, _lib.ptr(plan.ptr_dst),
              _lib.ptr(plan.perm_dst), _lib.ptr(plan.ptr_src), _lib.ptr(plan.perm_src), None,
              _lib.ptr(plan.visit), N, _lib.ptr(gp), None, _lib.ptr(vec), _lib.ptr(vp),
              _lib.stream(vec.device))
    node_ptr = torch.tensor([0, N], dtype=torch.int64, device=DEV)
    want = _lib.virial_reduce(vp, N, node_ptr, 1, None, True, torch.float64)

    def fused(n_edges, n_nodes, vdt):
        need = int(_lib.load().xnn_edge_force_reduce_virial_workspace_bytes(n_edges, n_nodes))
        ws = torch.full((max(need, 1),), 255, dtype=torch.uint8, device=DEV)
        out_pos = torch.full((max(n_nodes, 1), 3), float("nan"), dtype=dtype, device=DEV)
        vir = torch.full((1, 3, 3), float("nan"), dtype=vdt, device=DEV)
        _lib.call("xnn_edge_force_reduce_virial", code, code, _lib.ptr(ge), n_edges,
                  _lib.ptr(plan.ptr_dst), _lib.ptr(plan.perm_dst), _lib.ptr(plan.ptr_src),
                  _lib.ptr(plan.perm_src), _lib.ptr(plan.visit), n_nodes, _lib.ptr(out_pos),
                  _lib.ptr(vec), _lib.dtype_code(vdt), _lib.ptr(vir), _lib.ptr(ws), need,
                  _lib.stream(vec.device))
        return out_pos, vir

    p1, v1 = fused(E, N, torch.float64)
    assert torch.equal(p1, gp)
    scale = float(vp.abs().sum(0).max())
    np.testing.assert_allclose(v1.cpu(), want.cpu(), rtol=0, atol=1e-13 * scale)
    np.testing.assert_allclose(v1.cpu(), v1.cpu().transpose(1, 2), rtol=0, atol=0)
    for _ in range(3):
        p2, v2 = fused(E, N, torch.float64)
        assert torch.equal(p2, p1) and torch.equal(v2, v1)
    p3, v3 = fused(E, N, torch.float32)
    assert torch.equal(p3, gp) and torch.equal(v3, v1.float())
    _, v0 = fused(0, 0, torch.float64)
    assert torch.equal(v0.cpu(), torch.zeros(1, 3, 3, dtype=torch.float64))


def test_scatter_sum_sees_an_index_changed_in_place():
    """The CSR of an index is cached while its contents stay the same: an index tensor
    changed in place between two calls (its version moves) gets a new CSR, so the second
    sum equals index_add over the new index, not the old one."""
    from xnn_amd.functional import scatter_sum
    _note("scatter_sum with an index changed in place")
    gen = torch.Generator().manual_seed(31)
    src = torch.randn(500, 7, generator=gen).to(DEV)
    index = torch.randint(0, 40, (500,), generator=gen).to(DEV)
    first = scatter_sum(src, index, 40)
    ref = torch.zeros(40, 7, device=DEV).index_add_(0, index, src)
    torch.testing.assert_close(first, ref, rtol=1e-6, atol=1e-6)
    index[:250] = (index[:250] + 7) % 40          # same tensor object, new contents
    second = scatter_sum(src, index, 40)
    ref2 = torch.zeros(40, 7, device=DEV).index_add_(0, index, src)
    torch.testing.assert_close(second, ref2, rtol=1e-6, atol=1e-6)
    assert not torch.allclose(first, second)


def test_segment_gather_and_structure_sums():
    import oracle.reference as R
    import xnn_amd as xa
    _note("segment_sum / gather_rows / structure_sum")
    gen = torch.Generator().manual_seed(0)
    for F in (1, 3, 17, 64, 130):
        src = torch.randn(5000, F, generator=gen, dtype=torch.float64)
        index = torch.randint(0, 300, (5000,), generator=gen)
        got = xa.scatter_sum(src.to(DEV), index.to(DEV), 300)
        np.testing.assert_allclose(got.cpu(), R.scatter_sum(src, index, 300), atol=1e-12)
        # float32 summed in edge order equals the CPU index_add bit for bit
        s32 = src.float()
        got32 = xa.scatter_sum(s32.to(DEV), index.to(DEV), 300)
        order = torch.argsort(index, stable=True)
        want32 = torch.zeros(300, F).index_add_(0, index[order], s32[order])
        assert torch.equal(got32.cpu(), want32)
        gr = xa.gather_rows(src.to(DEV), index.to(DEV))
        assert torch.equal(gr.cpu(), src[index])
    vals = torch.randn(36800, generator=gen, dtype=torch.float64) * 10
    n_atoms = torch.randint(10, 61, (1024,), generator=gen)
    n_atoms = n_atoms[: int((n_atoms.cumsum(0) <= 36800).sum())]
    batch = torch.repeat_interleave(torch.arange(len(n_atoms)), n_atoms)
    vals = vals[: len(batch)]
    got = xa.structure_sum(vals.to(DEV), batch.to(DEV), len(n_atoms))
    np.testing.assert_allclose(got.cpu(), R.structure_sum(vals, batch, len(n_atoms)), rtol=1e-13)
    got1 = xa.structure_sum(vals.float().to(DEV), torch.zeros(len(vals), dtype=torch.long,
                                                              device=DEV), 1)
    assert got1.dtype == torch.float64
    assert abs(float(got1[0]) - float(vals.float().double().sum())) < 1e-9
    # an index not grouped by structure (the reference takes any index): float32 rows
    # summed in float64 along the stable order equal the CPU index_add bit for bit
    shuffle = torch.randperm(len(batch), generator=gen)
    vs, bs = vals.float()[shuffle], batch[shuffle]
    got_s = xa.structure_sum(vs.to(DEV), bs.to(DEV), len(n_atoms))
    order = torch.argsort(bs, stable=True)
    want_s = torch.zeros(len(n_atoms), dtype=torch.float64).index_add_(0, bs[order],
                                                                      vs[order].double())
    np.testing.assert_allclose(got_s.cpu(), torch.zeros(len(n_atoms), dtype=torch.float64)
                               .index_add_(0, bs, vs.double()), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(got_s.cpu(), want_s, rtol=1e-14, atol=1e-13)
    # and its gradient reaches every row in the caller's order
    leaf = vs.to(DEV).requires_grad_(True)
    w = torch.randn(len(n_atoms), generator=gen, dtype=torch.float64)
    (g_rows,) = torch.autograd.grad((xa.structure_sum(leaf, bs.to(DEV), len(n_atoms))
                                     * w.to(DEV)).sum(), [leaf])
    assert torch.equal(g_rows.cpu(), w[bs].float())


@pytest.mark.parametrize("F", [1, 3, 9, 16, 64, 65])
def test_single_structure_reduction(F):
    """One segment (one structure): the flat two-level kernel (F <= 64) and the row-chunked
    one (F > 64) against float64 sums on the CPU, for the whole array and for a sub-range,
    reproducible bit for bit."""
    from xnn_amd import _lib
    _note(f"single-structure reduction F={F}")
    gen = torch.Generator().manual_seed(F)
    for n, (s0, s1) in [(9000, (0, 9000)), (9000, (17, 8001)), (100, (0, 100)),
                        (250_000, (0, 250_000))]:
        for dt in (torch.float32, torch.float64):
            src = (torch.randn(n, F, generator=gen, dtype=torch.float64) * 3).to(dt)
            seg = torch.tensor([s0, s1], dtype=torch.int64, device=DEV)
            out = torch.empty(1, F, dtype=torch.float64, device=DEV)
            d = src.to(DEV)
            _lib.segment_reduce_f64(d, n, F, seg, 1, out)
            want = src[s0:s1].double().sum(0)
            np.testing.assert_allclose(out[0].cpu(), want, rtol=1e-12, atol=1e-9)
            out2 = torch.empty_like(out)
            _lib.segment_reduce_f64(d, n, F, seg, 1, out2)
            assert torch.equal(out, out2)


@pytest.mark.parametrize("F", [2048, 2050, 36, 1])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_node_readout_forward_backward(F, dtype):
    """The model's readout E_i = rows_i . w + bias[z_i] and its gradients in rows, w and
    bias against float64 PyTorch on the CPU (float32 rtol 1e-5, float64 1e-12), the
    vector and scalar row paths, a broadcast cotangent read as one value, a z outside the
    bias table giving NaN, and bitwise repeatability."""
    from xnn_amd import _lib
    from xnn_amd.ops import node_readout_op
    _note(f"node readout F={F} {dtype}")
    gen = torch.Generator().manual_seed(F)
    n = 1003
    rows = torch.randn(n, F, generator=gen, dtype=torch.float64)
    w = torch.randn(F, generator=gen, dtype=torch.float64)
    bias = torch.randn(9, generator=gen, dtype=torch.float64)
    z = torch.randint(0, 9, (n,), generator=gen)
    g = torch.randn(n, generator=gen, dtype=torch.float64)
    tol = dict(rtol=1e-5, atol=1e-5 * F ** 0.5) if dtype == torch.float32 else \
        dict(rtol=1e-12, atol=1e-12 * F ** 0.5)
    rd = rows.to(dtype).to(DEV).requires_grad_(True)
    wd = w.to(dtype).to(DEV).requires_grad_(True)
    bd = bias.to(dtype).to(DEV).requires_grad_(True)
    calls = _lib.calls.get("xnn_node_readout", 0)
    out = node_readout_op(rd, wd, z.to(DEV), bd)
    assert _lib.calls["xnn_node_readout"] == calls + 1
    want = rows.to(dtype).double() @ w.to(dtype).double() + bias.to(dtype).double()[z]
    np.testing.assert_allclose(out.detach().cpu().double(), want, **tol)
    assert torch.equal(out, node_readout_op(rd, wd, z.to(DEV), bd))
    d_rows, d_w, d_b = torch.autograd.grad(out, [rd, wd, bd], g.to(dtype).to(DEV))
    gq = g.to(dtype).double()
    np.testing.assert_allclose(d_rows.cpu().double(), gq[:, None] * w.to(dtype).double()[None],
                               rtol=tol["rtol"], atol=tol["rtol"])
    np.testing.assert_allclose(d_w.cpu().double(), rows.to(dtype).double().t() @ gq,
                               rtol=tol["rtol"], atol=tol["atol"] * n ** 0.5)
    np.testing.assert_allclose(d_b.cpu().double(), torch.zeros(9, dtype=torch.float64)
                               .index_add_(0, z, gq), rtol=tol["rtol"], atol=tol["atol"])
    # a broadcast (stride-0) cotangent, as a force evaluation seeds it
    seed = torch.full((1,), -1.0, dtype=dtype, device=DEV).expand(n)
    (d_rows2,) = torch.autograd.grad(node_readout_op(rd, wd, z.to(DEV), bd), [rd], seed)
    assert torch.equal(d_rows2, (-wd.detach())[None].expand(n, F))
    bad = node_readout_op(rd.detach()[:2], wd.detach(), torch.tensor([0, 9], device=DEV),
                          bd.detach())
    assert torch.isfinite(bad[0]) and torch.isnan(bad[1])


def test_stress_and_virial_finish_kernels():
    """sym(M + term) cast, and scale * g / |det cell| with zero stress for zero cells and
    non-periodic structures, against the PyTorch formulation."""
    from xnn_amd.ops import stress_finish, virial_finish
    from xnn_amd.functional import cell_volume
    _note("stress / virial finish")
    gen = torch.Generator().manual_seed(11)
    B = 5
    M = torch.randn(B, 9, generator=gen, dtype=torch.float64)
    term = torch.randn(B, 9, generator=gen, dtype=torch.float64)
    for t in (None, term):
        for dt in (torch.float32, torch.float64):
            got = virial_finish(M.to(DEV), None if t is None else t.to(DEV), dt)
            X = (M if t is None else M + t).view(B, 3, 3)
            np.testing.assert_allclose(got.cpu().double(), 0.5 * (X + X.transpose(1, 2)),
                                       rtol=1e-6 if dt == torch.float32 else 1e-15)
    # per-atom partials -> per-structure virial in one call: one structure of few atoms
    # (one block), of many (chunked), several structures
    from xnn_amd import _lib
    for counts in ([50], [9000], [3000, 17, 4000], [100_000]):
        n = sum(counts)
        part = torch.randn(n, 9, generator=gen, dtype=torch.float64)
        seg = torch.tensor([0] + list(np.cumsum(counts)), dtype=torch.int64)
        tm = torch.randn(len(counts), 9, generator=gen, dtype=torch.float64)
        for t, sym in ((None, False), (tm, True)):
            got = _lib.virial_reduce(part.to(DEV), n, seg.to(DEV), len(counts),
                                     None if t is None else t.to(DEV), sym, torch.float64)
            X = torch.stack([part[a:b].sum(0) for a, b in zip(seg[:-1], seg[1:])])
            if t is not None:
                X = X + t
            X = X.view(-1, 3, 3)
            want = 0.5 * (X + X.transpose(1, 2)) if sym else X
            np.testing.assert_allclose(got.cpu(), want, rtol=1e-12, atol=1e-10)
            again = _lib.virial_reduce(part.to(DEV), n, seg.to(DEV), len(counts),
                                       None if t is None else t.to(DEV), sym, torch.float64)
            assert torch.equal(got, again)
    cell = torch.randn(B, 3, 3, generator=gen, dtype=torch.float64) + 4 * torch.eye(3, dtype=torch.float64)
    cell[1] = 0.0                                  # a molecule of the batch
    pbc = torch.ones(B, 3, dtype=torch.bool)
    pbc[3] = False                                 # a cell that is not periodic
    g = torch.randn(B, 3, 3, generator=gen, dtype=torch.float64)
    vol = cell_volume(cell)
    periodic = (vol > 1e-8) & pbc.any(-1)
    want = torch.where(periodic[:, None, None], -g / torch.where(periodic, vol, torch.ones_like(vol))[:, None, None],
                       torch.zeros_like(g))
    for p in (pbc, pbc.to(DEV), None):
        for dt in (torch.float32, torch.float64):
            got = stress_finish(g.to(DEV, dt), cell.to(DEV, dt), p, -1.0)
            w = want if p is not None else torch.where((vol > 1e-8)[:, None, None],
                                                       -g / torch.where(vol > 1e-8, vol, torch.ones_like(vol))[:, None, None],
                                                       torch.zeros_like(g))
            np.testing.assert_allclose(got.cpu().double(), w, rtol=1e-6 if dt == torch.float32 else 1e-13,
                                       atol=1e-7 if dt == torch.float32 else 1e-15)


def test_energy_stress_finish_matches_the_two_kernels():
    """One structure's energy total and stress in one launch: the energy equals the
    structure sum bit for bit where that sum is one flat block (2,048 to 16,384 atoms) and
    the float64 sum to rounding elsewhere; the stress equals xnn_stress_finish bit for bit
    (a periodic cell, a zero cell, pbc all False)."""
    import xnn_amd as xa
    from xnn_amd.ops import energy_stress_finish, energy_stress_supported, stress_finish
    _note("energy + stress finish")
    gen = torch.Generator().manual_seed(12)
    g = torch.randn(1, 3, 3, generator=gen, dtype=torch.float64)
    cell = torch.randn(1, 3, 3, generator=gen, dtype=torch.float64) + 4 * torch.eye(3, dtype=torch.float64)
    for n in (0, 7, 2048, 9000, 16384, 40000):
        for edt in (torch.float32, torch.float64):
            e = (torch.randn(n, generator=gen, dtype=torch.float64) * 3).to(DEV, edt)
            assert energy_stress_supported(e)
            for gdt in (torch.float32, torch.float64):
                for c, pbc in ((cell, None), (cell, torch.zeros(1, 3, dtype=torch.bool)),
                               (torch.zeros(1, 3, 3, dtype=torch.float64), None)):
                    E, S = energy_stress_finish(e, g.to(DEV, gdt), c.to(DEV, gdt), pbc, -1.0)
                    S2 = stress_finish(g.to(DEV, gdt), c.to(DEV, gdt), pbc, -1.0)
                    assert torch.equal(S, S2)
                    want = xa.structure_sum(e, torch.zeros(n, dtype=torch.long, device=DEV), 1)
                    if 2048 <= n <= 16384:
                        assert torch.equal(E, want)
                    else:
                        np.testing.assert_allclose(E.cpu(), e.double().sum().cpu().reshape(1),
                                                   rtol=1e-14, atol=1e-13)
                    E2, _ = energy_stress_finish(e, g.to(DEV, gdt), c.to(DEV, gdt), pbc, -1.0)
                    assert torch.equal(E, E2)


# --------------------------------------------------------------------------- full model
def _float32_floor(R, g, params, cpu_pos, cell, ref, err):
    """The energy bar where float32 cannot give 1e-6 of E.

    With random-init weights on small molecules a structure's energy is a sum with heavy
    cancellation (sum_{i,k} |U_k A_ik| is ~50 |E|), and the reference's formulation itself,
    evaluated in float32 on the CPU (the oracle's messages, index_add and readout in
    float32 on the same float32 vectors), misses 1e-6 of E. The bar is then that float32
    floor: scaled by each structure's rounding scale S_b = sum_{i in b, k} |U_k A_ik|
    (float64), the HIP path's largest deviation from the float64 energies may be at most
    twice the float32 reference formulation's."""
    ei, batch = g.edge_index.cpu(), g.batch.cpu()
    vec32 = R.edge_vectors(cpu_pos.float(), ei, g.cell_shifts.cpu(),
                           None if cell is None else cell.float(), batch)
    p32 = dict(params, W=params["W"].float(), U=params["U"].float(),
               atom_ref=params["atom_ref"].float())
    node32 = R.sh_edge_node_energy(vec32, ei, g.num_nodes, g.atomic_numbers.cpu(), **p32)
    e32 = R.structure_sum(node32, batch, g.num_graphs)
    err32 = (e32 - ref["energy"]).abs()
    # S_b: the readout's terms in absolute value (|U| against |A|, A by the same chunks)
    v = vec32.double()
    u = R.radial_features(torch.linalg.norm(v, dim=-1), params["n_rbf"], params["cutoff"],
                          params["radial"], params["envelope"])
    y = R.e3nn_sh(params["l_max"], v if params.get("sh_sign", 1) == 1 else -v)
    phi = u @ params["W"]
    C, L = phi.shape[1], y.shape[1]
    A = torch.zeros((g.num_nodes, C * L), dtype=torch.float64)
    for e0 in range(0, v.shape[0], 1 << 15):
        e1 = min(v.shape[0], e0 + (1 << 15))
        A.index_add_(0, ei[1, e0:e1], (phi[e0:e1, :, None] * y[e0:e1, None, :]).reshape(-1, C * L))
    S = R.structure_sum(A.abs() @ params["U"].abs().reshape(-1), batch, g.num_graphs)
    floor, ours = float((err32 / S).max()), float((err / S).max())
    print(f"float32 reference formulation: rel err max {float((err32 / ref['energy'].abs()).max()):.3e}; "
          f"err / S max: float32 formulation {floor:.3e}, HIP {ours:.3e}", flush=True)
    assert float((err32 / ref["energy"].abs()).max()) > 1e-6, \
        "the float32 formulation meets 1e-6 of E here: so must the HIP path"
    assert ours <= 2.0 * floor, (ours, floor)


@pytest.mark.parametrize("config,fused", [("water", "radial"), ("water", "radial_rows"),
                                          ("water", "linear"),
                                          ("water", "unfused"), ("argon", "radial"),
                                          ("ragged", "radial"), ("ragged", "linear"),
                                          ("ragged_1024", "radial"),
                                          ("nequip_molecules", "radial"),
                                          ("nequip_molecules", "unfused"),
                                          ("periodic_batch", "radial"),
                                          ("water", "one_pass"), ("argon", "one_pass"),
                                          ("ragged", "one_pass"), ("ragged_1024", "one_pass"),
                                          ("periodic_batch", "one_pass")])
def test_model_energy_forces_stress(config, fused):
    import oracle.reference as R
    import xnn_amd as xa
    from xnn_amd import _lib, synthetic
    if config == "water":
        s, rc = synthetic.water_box(seed=0), 5.0
        kw = dict(n_rbf=8, l_max=3, channels=128, radial_type="bessel", envelope="polynomial")
        structs = [s]
    elif config == "argon":
        s, rc = synthetic.argon_fcc(), 6.0
        kw = dict(n_rbf=8, l_max=3, channels=64, radial_type="bessel", envelope="cosine")
        structs = [s]
    elif config == "ragged":
        structs, rc = synthetic.ragged_molecules(256, seed=1), 5.0
        kw = dict(n_rbf=8, l_max=3, channels=64, radial_type="bessel", envelope="polynomial")
    elif config == "ragged_1024":
        # the C3 configuration at its stated size (1,024 molecules, ~750k edges)
        structs, rc = synthetic.ragged_molecules(1024, seed=0), 5.0
        kw = dict(n_rbf=8, l_max=3, channels=64, radial_type="bessel", envelope="polynomial")
    elif config == "periodic_batch":
        # three periodic cells of different sizes and kinds: per-structure virials
        structs, rc = [synthetic.water_box(n_molecules=64, box=12.4, grid=4, seed=5),
                       synthetic.argon_fcc(n_cells=3, seed=6),
                       synthetic.organic_box(n_atoms=300, box=14.0, seed=7)], 5.0
        kw = dict(n_rbf=8, l_max=3, channels=64, radial_type="bessel", envelope="polynomial")
    else:
        structs, rc = synthetic.random_molecules(32, seed=2), 5.0
        kw = dict(n_rbf=8, l_max=2, channels=32, radial_type="bessel", envelope="polynomial",
                  sh_sign=-1)
    _note(f"model {config} fused={fused}")
    graphs = [xa.structure_to_graph(st.as_dict(), rc, device=DEV) for st in structs]
    g = graphs[0] if len(graphs) == 1 else xa.collate(graphs)
    g.pos = g.pos.float()
    if g.cell is not None:
        g.cell = g.cell.float()
    # one_pass: the readout path with energies and gradients from one backward launch
    model = xa.ShEdgePotential(cutoff=rc, species=(1, 6, 7, 8, 18),
                               fused_linear=fused != "unfused",
                               fused_radial=fused in ("radial", "radial_rows", "one_pass"),
                               fused_readout=fused in ("radial", "one_pass"), **kw).to(DEV)
    model.one_pass = fused == "one_pass"
    before = dict(_lib.calls)
    out = xa.ForceStressOutput(model, compute_stress=g.cell is not None).eval()(g)
    msg = {"radial": "xnn_sh_radial_message_energy", "radial_rows": "xnn_sh_radial_message_sum",
           "linear": "xnn_sh_linear_message_sum", "unfused": "xnn_sh_message_sum",
           "one_pass": "xnn_sh_radial_message_energy"}[fused]
    ran = ([msg + "_forces"] if fused == "one_pass" else [msg, msg + "_backward"]) + \
        ["xnn_edge_featurize"]
    if fused not in ("radial", "radial_rows", "one_pass"):
        ran.append("xnn_edge_featurize_backward")
    if fused == "one_pass":
        for name in (msg, msg + "_backward"):
            assert _lib.calls.get(name, 0) == before.get(name, 0), f"{name} ran"
    for name in ran:
        assert _lib.calls.get(name, 0) > before.get(name, 0), f"{name} did not run"
    # one structure: the force reduction finishes the strain derivative in the same launch
    reduce_names = ("xnn_edge_force_reduce", "xnn_edge_force_reduce_virial")
    assert (sum(_lib.calls.get(n, 0) for n in reduce_names)
            > sum(before.get(n, 0) for n in reduce_names)), "the force reduction did not run"
    params = dict(W=model.W.detach().cpu().double(), U=model.U.detach().cpu().double(),
                  atom_ref=model.atom_ref.detach().cpu().double(), l_max=kw["l_max"],
                  n_rbf=kw["n_rbf"], cutoff=rc, radial=kw["radial_type"],
                  envelope=kw["envelope"], sh_sign=kw.get("sh_sign", 1))
    cpu_pos = torch.tensor(np.concatenate([st.pos for st in structs]), dtype=torch.float32).double()
    cell = None if g.cell is None else g.cell.detach().cpu().double()
    ref = R.energy_forces_stress(cpu_pos, g.atomic_numbers.cpu(), g.edge_index.cpu(),
                                 g.cell_shifts.cpu(), cell, g.batch.cpu(), g.num_graphs, params,
                                 stress=cell is not None, geometry_dtype=torch.float32)
    # energies: rtol 1e-6 of each structure's energy against the float64 oracle on the
    # same float32 vectors; sum_i |E_i| is printed beside it
    scale = R.structure_sum(ref["node_energy"].abs(), g.batch.cpu(), g.num_graphs)
    err = (out["energy"].detach().cpu() - ref["energy"]).abs()
    rel = err / ref["energy"].abs()
    print(f"energy rel err max {float(rel.max()):.3e}; err / sum|E_i| max "
          f"{float((err / scale).max()):.3e}; E={ref['energy'][:3].tolist()}", flush=True)
    if not bool((rel <= 1e-6).all()):
        msg = (f"model {config} fused={fused}: energy bar from the float32 floor "
               f"(rel err {float(rel.max()):.3e} > 1e-6)")
        _note(msg)
        import warnings
        warnings.warn(msg)       # listed in pytest's warnings summary of the run
        _float32_floor(R, g, params, cpu_pos, cell, ref, err)
    np.testing.assert_allclose(out["forces"].detach().cpu().double(), ref["forces"], atol=1e-5)
    if cell is not None:
        np.testing.assert_allclose(out["stress"].detach().cpu().double(), ref["stress"], atol=1e-5)
    # bitwise reproducible forces
    g2 = graphs[0] if len(graphs) == 1 else xa.collate(graphs)
    g2.pos = g2.pos.float()
    if g2.cell is not None:
        g2.cell = g2.cell.float()
    out2 = xa.ForceStressOutput(model, compute_stress=g2.cell is not None).eval()(g2)
    assert torch.equal(out["forces"], out2["forces"])
    assert torch.equal(out["energy"], out2["energy"])


def test_stress_from_edge_virial_matches_deformation():
    """The strain derivative formed by the edge-vector backward (sym sum_e r_e (x) dE/dr_e)
    equals the one autograd carries back through deformed positions and cells."""
    import xnn_amd as xa
    from xnn_amd import synthetic
    _note("edge virial vs deformation")
    structs = [synthetic.water_box(n_molecules=64, box=12.4, grid=4, seed=8),
               synthetic.argon_fcc(n_cells=3, seed=9)]
    g = xa.collate([xa.structure_to_graph(st.as_dict(), 5.0, device=DEV) for st in structs])
    g.pos, g.cell = g.pos.float(), g.cell.float()
    model = xa.ShEdgePotential(cutoff=5.0, species=(1, 8, 18), channels=64, seed=3).to(DEV)
    wrapped = xa.ForceStressOutput(model, compute_stress=True).eval()
    out_probe = wrapped(copy.copy(g))
    model.edge_virial = False              # instance override: deform pos and cell instead
    out_deform = wrapped(copy.copy(g))
    scale = float(out_deform["stress"].abs().max())
    np.testing.assert_allclose(out_probe["stress"].detach().cpu().double(),
                               out_deform["stress"].detach().cpu().double(), atol=1e-6 * scale)
    np.testing.assert_allclose(out_probe["forces"].detach().cpu().double(),
                               out_deform["forces"].detach().cpu().double(), atol=1e-6)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_strain_apply_matches_the_broadcast_formulation(dtype):
    """The HIP strain deformation and its backward against the PyTorch formulation of
    outputs.py:166-180 (batch of three cells, a nonzero strain), forward and gradients."""
    from xnn_amd.ops import strain_apply_op
    _note(f"strain_apply {dtype}")
    gen = torch.Generator().manual_seed(5)
    counts = [7, 11, 5]
    pos = torch.randn(sum(counts), 3, generator=gen, dtype=torch.float64) * 3
    cell = torch.randn(3, 3, 3, generator=gen, dtype=torch.float64) + 6 * torch.eye(3, dtype=torch.float64)
    eps = torch.randn(3, 3, 3, generator=gen, dtype=torch.float64) * 0.01
    batch = torch.repeat_interleave(torch.arange(3), torch.tensor(counts))
    node_ptr = torch.tensor([0, 7, 18, 23])
    gp = torch.randn(pos.shape, generator=gen, dtype=torch.float64)
    gc = torch.randn(cell.shape, generator=gen, dtype=torch.float64)
    # reference, in float64 on the CPU
    e_r = eps.clone().requires_grad_(True)
    p_r, c_r = pos.clone().requires_grad_(True), cell.clone().requires_grad_(True)
    sym = 0.5 * (e_r + e_r.transpose(-1, -2))
    p2 = p_r + (p_r[:, :, None] * sym.index_select(0, batch)).sum(1)
    c2 = c_r + (c_r[:, :, :, None] * sym[:, None]).sum(2)
    ge_r, gp_r, gc_r = torch.autograd.grad((p2 * gp).sum() + (c2 * gc).sum(), [e_r, p_r, c_r])
    # HIP
    e = eps.to(DEV, dtype).requires_grad_(True)
    p = pos.to(DEV, dtype).requires_grad_(True)
    c = cell.to(DEV, dtype).requires_grad_(True)
    p3, c3 = strain_apply_op(p, c, e, batch.to(DEV, torch.int32), node_ptr.to(DEV))
    ge, gpp, gcc = torch.autograd.grad((p3 * gp.to(DEV, dtype)).sum() + (c3 * gc.to(DEV, dtype)).sum(),
                                       [e, p, c])
    tol = 1e-12 if dtype == torch.float64 else 2e-5
    for got, want in ((p3, p2), (c3, c2), (ge, ge_r), (gpp, gp_r), (gcc, gc_r)):
        np.testing.assert_allclose(got.detach().cpu().double(), want.detach(),
                                   atol=tol * max(1.0, float(want.abs().max())))


def test_training_step_differentiates_forces_twice():
    """A force-loss training step (create_graph=True): the featurizer takes the PyTorch
    formulation, the edge vectors / sums stay on the HIP ops (differentiable to any
    order), and the parameter gradients of the force loss equal the CPU reference's."""
    import xnn_amd as xa
    from xnn_amd import _lib, synthetic
    _note("training step, double backward")
    s = synthetic.water_box(n_molecules=64, box=12.4, grid=4, seed=5)

    def run(device):
        torch.manual_seed(0)
        g = xa.structure_to_graph(s.as_dict(), 4.5, device=device)
        g.pos, g.cell = g.pos.double(), g.cell.double()
        model = xa.ShEdgePotential(n_rbf=8, l_max=2, channels=16, cutoff=4.5, seed=3).double()
        model = model.to(device)
        wrapped = xa.ForceStressOutput(model, compute_stress=True).train()
        out = wrapped(g)
        loss = (out["forces"] ** 2).sum() + out["energy"].sum() + (out["stress"] ** 2).sum()
        grads = torch.autograd.grad(loss, [model.W, model.U, model.atom_ref])
        return out, [x.detach().cpu() for x in grads]

    before = _lib.calls.get("xnn_edge_force_reduce", 0)
    out_g, grads_g = run(DEV)
    assert _lib.calls.get("xnn_edge_force_reduce", 0) > before
    out_c, grads_c = run("cpu")
    np.testing.assert_allclose(out_g["forces"].detach().cpu(), out_c["forces"].detach(), atol=1e-10)
    for a, b in zip(grads_g, grads_c):
        np.testing.assert_allclose(a, b, rtol=1e-9, atol=1e-9)


@pytest.mark.parametrize("edge_virial", [False, True])
def test_graph_replays_match_the_eager_step(edge_virial):
    """The whole step captured as one HIP graph: every replay, with eager work and
    synchronizations between replays, reproduces the eager forces, stress and energy; with
    the strain deformation and with the edge-virial form of the stress."""
    import copy
    import xnn_amd as xa
    from xnn_amd import synthetic
    _note(f"HIP graph replay edge_virial={edge_virial}")
    s = synthetic.water_box(n_molecules=216, box=18.6, grid=6, seed=4)
    g = xa.structure_to_graph(s.as_dict(), 5.0, device=DEV)
    model = xa.ShEdgePotential(n_rbf=8, l_max=3, channels=64, cutoff=5.0, seed=1).to(DEV)
    model.edge_virial = edge_virial
    wrapped = xa.ForceStressOutput(model, compute_stress=True).eval()
    g.plan()

    def step():
        return wrapped(copy.copy(g))

    eager = step()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static = step()
    for k in range(4):
        graph.replay()
        torch.cuda.synchronize()
        for key in ("energy", "forces", "stress"):
            assert torch.equal(static[key], eager[key]), (k, key)
        other = step()                      # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(other["forces"], eager["forces"])


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_nearest_edges_on_the_gpu(dtype):
    """max_neighbors on the GPU (xnn_nearest_edges_count/_fill) against the brute-force
    oracle: ties broken by edge id, ungrouped and grouped receivers, rows below k; and
    structure_to_graph(max_neighbors=12) of a dense water box equal to the CPU graph."""
    import oracle.nl as N
    import xnn_amd as xa
    from xnn_amd import _lib, synthetic
    from xnn_amd.data import nearest_edges
    _note(f"nearest edges {dtype}")
    rng = np.random.default_rng(7)
    for n, e, k in ((40, 2000, 7), (300, 9000, 31), (5, 400, 1)):
        dst = rng.integers(0, n, e)
        d = np.round(rng.uniform(0, 4, e), 1)
        for grouped in (False, True):
            if grouped:
                o = np.argsort(dst, kind="stable")
                dst, d = dst[o], d[o]
            before = _lib.calls.get("xnn_nearest_edges_fill", 0)
            keep, _ = nearest_edges(torch.tensor(d, dtype=dtype, device=DEV),
                                    torch.tensor(dst, device=DEV), n, k)
            assert _lib.calls.get("xnn_nearest_edges_fill", 0) == before + 1
            want = N.nearest_edges(d.astype(np.float32) if dtype == torch.float32 else d, dst, n, k)
            np.testing.assert_array_equal(keep.cpu().numpy(), want)
    # NaN lengths rank after every number (every slot of the kept rows written once)
    dst = np.repeat(np.arange(30), 20)
    d = np.round(rng.uniform(0, 4, dst.size), 1)
    d[rng.random(dst.size) < 0.7] = np.nan
    keep, _ = nearest_edges(torch.tensor(d, dtype=dtype, device=DEV), torch.tensor(dst, device=DEV),
                            30, 9)
    np.testing.assert_array_equal(keep.cpu().numpy(), N.nearest_edges(d, dst, 30, 9))
    s = synthetic.water_box(n_molecules=216, box=18.6, grid=6, seed=2)
    gpu = xa.structure_to_graph(s.as_dict(), 5.0, device=DEV, max_neighbors=12)
    cpu = xa.structure_to_graph(s.as_dict(), 5.0, max_neighbors=12)
    assert torch.equal(gpu.edge_index.cpu(), cpu.edge_index)
    assert torch.equal(gpu.cell_shifts.cpu(), cpu.cell_shifts)


@pytest.mark.parametrize("case", ["water", "molecule"])
def test_pair_style_entry_matches_force_stress_output(case):
    """xnn_sh_pair_energy_forces (through deploy.LAMMPSWrapper, the pair-style tensor ABI of
    lammps.py:83-145) against ForceStressOutput on the same graph: total and per-atom
    energies, forces, and the virial W = -V sigma; an edge index outside [0, N) is an error."""
    import xnn_amd as xa
    from xnn_amd import _lib, synthetic
    from xnn_amd.deploy import LAMMPSWrapper
    _note(f"pair-style entry {case}")
    if case == "water":
        s = synthetic.water_box(n_molecules=216, box=18.6, grid=6, seed=6)
        kw = dict(l_max=3, channels=128, sh_sign=1)
    else:
        s = synthetic.random_molecules(1, seed=4)[0]
        kw = dict(l_max=2, channels=32, sh_sign=-1)
    g = xa.structure_to_graph(s.as_dict(), 5.0, device=DEV)
    g.pos = g.pos.float()
    if g.cell is not None:
        g.cell = g.cell.float()
    model = xa.ShEdgePotential(cutoff=5.0, species=(1, 6, 7, 8), **kw).to(DEV)
    out = xa.ForceStressOutput(model, compute_stress=g.cell is not None).eval()(g)
    cell = g.cell[0] if g.cell is not None else torch.zeros(3, 3, device=DEV)
    before = _lib.calls.get("xnn_sh_pair_energy_forces", 0)
    pair = LAMMPSWrapper(model)(g.pos, g.edge_index, g.cell_shifts, g.atomic_numbers, cell)
    assert _lib.calls.get("xnn_sh_pair_energy_forces", 0) == before + 1
    e_ref = float(out["energy"].detach().reshape(-1)[0])
    assert abs(float(pair["total_energy"][0]) - e_ref) <= 1e-6 * max(1.0, abs(e_ref))
    torch.testing.assert_close(pair["node_energy"], out["node_energy"].double(), atol=1e-5, rtol=0)
    torch.testing.assert_close(pair["forces"].double(), out["forces"].double(), atol=1e-5, rtol=0)
    if g.cell is not None:
        vol = float(torch.det(g.cell[0].double()))
        want = -vol * out["stress"][0].double()
        torch.testing.assert_close(pair["virial"], want, atol=1e-4 * max(1.0, float(want.abs().max())),
                                   rtol=0)
    else:
        # a molecule: sum_e r_e (x) dE/dr_e = sum_i r_i (x) dE/dr_i (translation invariance)
        grad = -out["forces"].double()
        M = (g.pos.double()[:, :, None] * grad[:, None, :]).sum(0)
        torch.testing.assert_close(pair["virial"], -0.5 * (M + M.T), atol=1e-4, rtol=0)
    bad = g.edge_index.clone()
    bad[0, 0] = g.num_nodes + 5
    with pytest.raises(_lib.XnnError, match="outside"):
        LAMMPSWrapper(model)(g.pos, bad, g.cell_shifts, g.atomic_numbers, cell)


@pytest.mark.parametrize("case", ["d4_fused_core", "d4_other_core", "d4_alone"])
def test_pair_style_wrapper_with_dispersion_and_other_cores(case):
    """deploy.LAMMPSWrapper on a model wrapped in D4 (lammps.py:70-79, 128-134): the core on
    the edges within its own cutoff of a longer pair-style list (6.5 A against the model's
    5.0), the D4 head's per-atom energies, forces and virial added; against
    ForceStressOutput(D4Dispersion(core)) on the core's own graph. The cores: the fused
    pair-style kernels, a core they do not take (48 channels: the ForceStressOutput path),
    and no core (D4 alone)."""
    import os
    import xnn_amd as xa
    from xnn_amd import _lib, synthetic
    from xnn_amd.deploy import LAMMPSWrapper
    from xnn_amd.dispersion import D4Dispersion
    _note(f"pair-style wrapper {case}")
    tables = os.path.join(os.path.dirname(__file__), "golden", "d4_tables_hcnoar.npz")
    s = synthetic.organic_box(n_atoms=300, box=14.0, seed=7)
    g = xa.structure_to_graph(s.as_dict(), 5.0, device=DEV)
    g.pos, g.cell = g.pos.float(), g.cell.float()
    if case == "d4_alone":
        model = D4Dispersion(None, tables=tables).to(DEV)
    else:
        kw = dict(channels=48) if case == "d4_other_core" else dict(channels=64)
        core = xa.ShEdgePotential(cutoff=5.0, species=(1, 6, 7, 8), l_max=2, **kw).to(DEV)
        model = D4Dispersion(core, tables=tables).to(DEV)
    out = xa.ForceStressOutput(model, compute_stress=True).eval()(g)
    wide = xa.structure_to_graph(s.as_dict(), 6.5, device=DEV)
    wrapper = LAMMPSWrapper(model, cutoff=6.5)
    assert wrapper.fused_core == (case == "d4_fused_core")
    before = _lib.calls.get("xnn_sh_pair_energy_forces", 0)
    pair = wrapper(wide.pos.float(), wide.edge_index, wide.cell_shifts, wide.atomic_numbers,
                   wide.cell[0].float())
    assert _lib.calls.get("xnn_sh_pair_energy_forces", 0) == before + int(wrapper.fused_core)
    e_ref = float(out["energy"].detach().reshape(-1)[0])
    assert abs(float(pair["total_energy"][0]) - e_ref) <= 1e-6 * max(1.0, abs(e_ref)), \
        (float(pair["total_energy"][0]), e_ref)
    torch.testing.assert_close(pair["node_energy"], out["node_energy"].detach().double(),
                               atol=1e-5, rtol=0)
    torch.testing.assert_close(pair["forces"].double(), out["forces"].double(), atol=1e-5, rtol=0)
    vol = float(torch.det(g.cell[0].double()))
    want = -vol * out["stress"][0].double()
    torch.testing.assert_close(pair["virial"], want, atol=1e-4 * max(1.0, float(want.abs().max())),
                               rtol=0)
    # the list must reach the model's cutoff
    if case != "d4_alone":
        with pytest.raises(ValueError, match="must reach"):
            LAMMPSWrapper(model, cutoff=4.0)


@pytest.mark.parametrize("basis", ["bessel", "gaussian"])
def test_every_envelope_is_zero_from_the_cutoff(basis):
    """The envelopes of the kernels vanish for r >= rc (cutoff.py:41, 125), the unit
    envelope (XNN_ENV_NONE) included: radial features of edges of a list longer than the
    cutoff are zero, their gradient too; inside the cutoff the unit envelope leaves the
    basis as it is."""
    import oracle.reference as R
    from xnn_amd.ops import edge_embed
    _note(f"envelopes at the cutoff {basis}")
    rc, K = 4.0, 6
    r = torch.linspace(0.3, 1.6 * rc, 801, dtype=torch.float64)
    d = torch.randn(801, 3, dtype=torch.float64, generator=torch.Generator().manual_seed(3))
    vec = (d / d.norm(dim=1, keepdim=True) * r[:, None]).to(DEV).requires_grad_(True)
    table = (torch.arange(1, K + 1, dtype=torch.float64) * np.pi if basis == "bessel"
             else torch.linspace(0.0, rc, K, dtype=torch.float64))
    gamma = 0.5 / (rc / (K - 1)) ** 2
    inside = (r < rc).to(DEV)
    for env in ("none", "polynomial", "cosine"):
        _, _, rad = edge_embed(vec, table.to(DEV), n_rbf=K, basis=basis, envelope=env,
                               poly_p=6, l_max=1, cutoff=rc, prefactor=(2.0 / rc) ** 0.5,
                               gamma=gamma, sh_sign=1)
        assert torch.equal(rad[~inside], torch.zeros_like(rad[~inside])), env
        (g,) = torch.autograd.grad(rad.sum(), (vec,))
        assert torch.equal(g[~inside], torch.zeros_like(g[~inside])), env
        if env == "none":
            rr = r[inside.cpu()].to(DEV)
            want = (R.bessel(rr.cpu(), K, rc, prefactor=(2.0 / rc) ** 0.5) if basis == "bessel"
                    else torch.exp(-gamma * (rr.cpu()[:, None] - table[None, :]) ** 2))
            torch.testing.assert_close(rad[inside].cpu(), want, rtol=1e-12, atol=1e-12)


def test_deployment_neighbor_list_matches_the_reference_semantics():
    """deploy.build_neighbor_list_ts (the exported artifact's neighbor list,
    torchscript.py:124-212) on the GPU: a zero cell or no periodic flag is a molecule; a
    cell with partial periodicity; the edge sets equal the oracle's."""
    import oracle.nl as N
    from oracle.nl import canonical
    from xnn_amd import synthetic
    from xnn_amd.deploy import build_neighbor_list_ts
    _note("deployment neighbor list")
    s = synthetic.water_box(n_molecules=64, box=12.4, grid=4, seed=10)
    pos = torch.tensor(s.pos, dtype=torch.float64, device=DEV)
    cell = torch.tensor(s.cell, dtype=torch.float64, device=DEV)
    for pbc in ([True, True, True], [True, False, True]):
        ei, sh = build_neighbor_list_ts(pos, 4.0, cell, torch.tensor(pbc, device=DEV))
        ei_o, sh_o, near = N.neighbor_list(s.pos, 4.0, s.cell, np.array(pbc), dtype=np.float64,
                                           margin=1e-7)
        assert near == 0
        assert np.array_equal(canonical(ei.cpu().numpy(), sh.cpu().numpy()), canonical(ei_o, sh_o))
    for cl, pbc in ((torch.zeros(3, 3, dtype=torch.float64, device=DEV), [True, True, True]),
                    (cell, [False, False, False])):
        ei, sh = build_neighbor_list_ts(pos, 4.0, cl, torch.tensor(pbc, device=DEV))
        ei_o, sh_o, near = N.neighbor_list(s.pos, 4.0, None, None, dtype=np.float64, margin=1e-7)
        assert near == 0 and int(sh.abs().sum()) == 0
        assert np.array_equal(canonical(ei.cpu().numpy(), sh.cpu().numpy()), canonical(ei_o, sh_o))
