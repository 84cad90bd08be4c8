"""Host-side checks that need no GPU: the C ABI library loads and exports every
entry point of include/xnn_amd.h, the binding declares exactly those, the ops refuse
CPU tensors (no fallback), and the PyTorch formulation of the modules equals the
oracle (so ``use_fast=False`` is the reference function)."""
import math
import ctypes
import os
import re

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _header_functions():
    text = open(os.path.join(ROOT, "include", "xnn_amd.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(xnn_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib_path():
    from xnn_amd import _lib
    if not os.path.exists(_lib.LIBRARY):
        from xnn_amd.build import build
        build()
    return _lib.LIBRARY


def test_library_exports_every_header_entry_point(lib_path):
    lib = ctypes.CDLL(lib_path)
    names = _header_functions()
    assert len(names) >= 15
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_declares_the_header_entry_points(lib_path):
    from xnn_amd import _lib
    assert sorted(_lib.exported_symbols()) == _header_functions()
    lib = _lib.load()
    assert lib.xnn_abi_version() == _lib.ABI_VERSION


def test_argument_errors_come_back_as_status_codes(lib_path):
    """Invalid arguments are rejected on the host before any launch."""
    from xnn_amd import _lib
    lib = _lib.load()
    prm = _lib.FeaturizeParams(8, 0, 0, 6, 7, 1, 5.0, 1.0, 1.0)   # l_max = 7
    code = lib.xnn_edge_featurize(0, 0, 1, None, 0, None, 0, None, None, None, None, 10, prm,
                                  1, None, None, None, None, None)
    assert code == _lib.XNN_EINVAL
    assert b"l_max" in lib.xnn_last_error()
    plan = _lib.GridPlan()
    pbc = (ctypes.c_int32 * 3)(1, 1, 1)
    cell = (ctypes.c_double * 9)(1, 0, 0, 0, 1, 0, 0, 0, 1)
    code = lib.xnn_radius_graph_plan(10, cell, pbc, 5.0, None, None, ctypes.byref(plan))
    assert code == _lib.XNN_EINVAL and b"cutoff" in lib.xnn_last_error()
    cell = (ctypes.c_double * 9)(20, 0, 0, 0, 20, 0, 0, 0, 20)
    assert lib.xnn_radius_graph_plan(10, cell, pbc, 5.0, None, None, ctypes.byref(plan)) == 0
    assert list(plan.nbins) == [3, 3, 3] and list(plan.reach) == [1, 1, 1]
    # the factor solve takes one or two right-hand sides and a work array
    assert lib.xnn_eeq_cholesky_solve(None, 10, None, None, 3, None, None) == _lib.XNN_EINVAL
    assert b"right-hand sides" in lib.xnn_last_error()
    assert lib.xnn_eeq_cholesky_solve(None, 10, None, None, 2, None, None) == _lib.XNN_EINVAL
    assert lib.xnn_eeq_cholesky_solve(None, 0, None, None, 1, None, None) == 0
    # the ATM tangents check their workspace size before anything runs
    size = ctypes.c_size_t()
    assert lib.xnn_atm_tangent_work_size(100, 10, 23, ctypes.byref(size)) == 0
    base = ctypes.c_size_t()
    assert lib.xnn_atm_work_size(100, 10, 23, 1, ctypes.byref(base)) == 0
    assert size.value > base.value
    assert lib.xnn_atm_tangent_work_size(100, 10, 33, ctypes.byref(size)) == _lib.XNN_EINVAL
    prm = _lib.AtmParams(1.0, 16.0 / 3.0, 10.0, 0.0)
    buf = (ctypes.c_double * 8)()
    code = lib.xnn_atm_energy_backward_tangent(
        buf, 100, 10, 1, 0, buf, buf, buf, 23, buf, buf, 1, ctypes.byref(prm), buf, buf, buf,
        buf, buf, buf, buf, buf, buf, base.value, None)
    assert code == _lib.XNN_EINVAL and b"workspace too small" in lib.xnn_last_error()


def test_ops_refuse_cpu_tensors():
    from xnn_amd import ops
    vec = torch.randn(5, 3)
    with pytest.raises(RuntimeError, match="GPU only"):
        ops.edge_embed(vec, torch.ones(8), n_rbf=8, basis="bessel", envelope="polynomial",
                       poly_p=6, l_max=3, cutoff=5.0)


def test_use_fast_true_on_a_cpu_raises():
    import xnn_amd as xa
    from xnn_amd import synthetic
    s = synthetic.random_molecules(1, seed=0)[0]
    g = xa.structure_to_graph(s.as_dict(), 5.0)
    model = xa.ShEdgePotential(channels=8, use_fast=True)
    with pytest.raises(RuntimeError, match="no HIP path"):
        model(g)


@pytest.mark.parametrize("radial,envelope,sign", [("bessel", "polynomial", 1),
                                                  ("gaussian", "cosine", -1)])
def test_reference_formulation_equals_the_oracle(radial, envelope, sign):
    import oracle.reference as R
    import xnn_amd as xa
    from xnn_amd import synthetic
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    try:
        s = synthetic.water_box(n_molecules=64, box=12.4, grid=4, seed=3)
        g = xa.structure_to_graph(s.as_dict(), 4.5)
        model = xa.ShEdgePotential(n_rbf=8, l_max=3, channels=8, cutoff=4.5, radial_type=radial,
                                   envelope=envelope, sh_sign=sign)
        out = xa.ForceStressOutput(model, compute_stress=True)(g)
        g2 = xa.structure_to_graph(s.as_dict(), 4.5)
        params = dict(W=model.W.detach(), U=model.U.detach(), atom_ref=model.atom_ref.detach(),
                      l_max=3, n_rbf=8, cutoff=4.5, radial=radial, envelope=envelope,
                      sh_sign=sign)
        ref = R.energy_forces_stress(g2.pos, g2.atomic_numbers, g2.edge_index, g2.cell_shifts,
                                     g2.cell, g2.batch, 1, params)
        torch.testing.assert_close(out["energy"], ref["energy"], rtol=1e-12, atol=1e-10)
        torch.testing.assert_close(out["forces"], ref["forces"], rtol=1e-10, atol=1e-11)
        torch.testing.assert_close(out["stress"], ref["stress"], rtol=1e-10, atol=1e-12)
    finally:
        torch.set_default_dtype(old)


def test_force_stress_output_leaves_the_callers_tensors_alone():
    """Forces are taken against a fresh leaf per call: the caller's positions stay a plain
    tensor (a leaf kept across calls would carry one call's gradient accumulator, and its
    stream, into the next), and two calls on the same graph agree."""
    import copy
    import xnn_amd as xa
    from xnn_amd import synthetic
    s = synthetic.water_box(n_molecules=8, box=6.2, grid=2, seed=5)
    g = xa.structure_to_graph(s.as_dict(), 4.0)
    model = xa.ShEdgePotential(n_rbf=4, l_max=1, channels=4, cutoff=4.0)
    for stress in (False, True):
        wrapped = xa.ForceStressOutput(model, compute_stress=stress)
        a = wrapped(copy.copy(g))
        b = wrapped(copy.copy(g))
        assert not g.pos.requires_grad and g.pos.grad_fn is None
        assert not g.cell.requires_grad
        torch.testing.assert_close(a["forces"], b["forces"], rtol=0, atol=0)


def test_collate_offsets_and_batch():
    import xnn_amd as xa
    from xnn_amd import synthetic
    mols = synthetic.random_molecules(3, seed=1)
    graphs = [xa.structure_to_graph(m.as_dict(), 4.0) for m in mols]
    b = xa.collate(graphs)
    assert b.num_graphs == 3 and b.num_nodes == 63
    assert b.num_edges == sum(g.num_edges for g in graphs)
    assert int(b.edge_index.max()) < 63 and torch.equal(b.batch.bincount(), torch.tensor([21] * 3))


def test_d4_polarizability_tables_and_argument_checks(lib_path):
    """DFTD4's element-major kernel tables are the reference tables transposed (refalpha
    (23, 7, Z) -> (Z, 7, 23)), the module refuses CPU tensors, and the polarizability and
    readout entry points reject bad arguments on the host (no launch)."""
    import os
    import xnn_amd.dispersion as XD
    from xnn_amd import _lib
    tables = XD.load_d4_tables(os.path.join(os.path.dirname(__file__), "golden",
                                            "d4_tables_hcnoar.npz"))
    d4 = XD.DFTD4(tables)
    ra = torch.as_tensor(tables["refalpha"])
    assert d4.k_refalpha.shape == (ra.shape[2], ra.shape[1], ra.shape[0])
    assert torch.equal(d4.k_refalpha, ra.permute(2, 1, 0))
    assert torch.equal(d4.k_refcn, torch.as_tensor(tables["refcn"]).t())
    assert d4.k_ngw.dtype == torch.int32 and d4.k_nref.dtype == torch.int32
    assert torch.allclose(d4.k_gi, torch.as_tensor(tables["hardness"]) * d4.gc)
    with pytest.raises(RuntimeError, match="GPU"):
        d4.polarizabilities(torch.tensor([1, 8]), torch.zeros(2, dtype=torch.float64),
                            torch.zeros(2, dtype=torch.float64))
    lib = _lib.load()
    empty = _lib.D4AlphaTables()                     # n_elements = 0, NULL tables
    assert lib.xnn_d4_polarizabilities(4, None, None, None, empty, None, None) == _lib.XNN_EINVAL
    assert b"tables" in lib.xnn_last_error()
    assert lib.xnn_node_readout(7, None, 4, 8, None, None, None, 0, None, None) == _lib.XNN_EINVAL
    assert lib.xnn_node_readout(0, None, 4, 8, None, None, 1, 5, None, None) == _lib.XNN_EINVAL
    assert b"bias and z" in lib.xnn_last_error()
    assert lib.xnn_node_readout_backward(0, 1, 2, 4, 8, 1, 1, None) == _lib.XNN_EINVAL
    assert b"g_stride" in lib.xnn_last_error()


def test_periodic_eeq_rows_in_chunks_equal_one_pass():
    """The Ewald EEQ matrix formed in row chunks (bounded memory for thousands of atoms)
    equals the one-pass matrix bit for bit, and its position and cell gradients through the
    recomputed (checkpointed) chunks equal the direct ones. CPU, float64."""
    import math as _m
    import xnn_amd.dispersion as XD
    tables = XD.load_d4_tables(os.path.join(os.path.dirname(__file__), "golden",
                                            "d4_tables_hcnoar.npz"))
    d4 = XD.DFTD4(tables)
    rng = np.random.default_rng(3)
    cell = torch.tensor([[9.0, 0.0, 0.0], [1.2, 8.5, 0.0], [-0.7, 0.9, 10.0]], dtype=torch.float64)
    pos = torch.tensor(rng.uniform(0, 1, (11, 3)), dtype=torch.float64) @ cell
    z = torch.tensor([8, 1, 1, 6, 1, 7, 8, 1, 6, 6, 1])
    rad = d4.eeq_rad[z]
    vol = torch.linalg.det(cell).abs()
    recip = 2.0 * _m.pi * torch.linalg.inv(cell).t()
    a = XD._ewald_alpha(float(torch.linalg.norm(recip, dim=1).min()),
                        float(torch.linalg.norm(cell, dim=1).min()), float(vol))
    whole = XD._ewald_rows(0, 11, a, pos, cell, vol, recip, rad)
    split = torch.cat([XD._ewald_rows(0, 4, a, pos, cell, vol, recip, rad),
                       XD._ewald_rows(4, 9, a, pos, cell, vol, recip, rad),
                       XD._ewald_rows(9, 11, a, pos, cell, vol, recip, rad)])
    assert torch.equal(whole, split)
    assert torch.allclose(whole, whole.t(), rtol=1e-12, atol=1e-14)
    p1, c1 = pos.clone().requires_grad_(True), cell.clone().requires_grad_(True)
    A = d4._coulomb_periodic(z, p1, c1)                   # checkpointed chunks
    w = torch.tensor(rng.normal(size=(11, 11)))
    g1 = torch.autograd.grad((A * w).sum(), [p1, c1])
    p2, c2 = pos.clone().requires_grad_(True), cell.clone().requires_grad_(True)
    vol2 = torch.linalg.det(c2).abs()
    recip2 = 2.0 * _m.pi * torch.linalg.inv(c2).t()
    B = XD._ewald_rows(0, 11, a, p2, c2, vol2, recip2, rad)
    B = B + torch.diag(d4.eeq_eta[z] + _m.sqrt(2.0 / _m.pi) / rad - 2.0 * a / _m.sqrt(_m.pi))
    g2 = torch.autograd.grad((B * w).sum(), [p2, c2])
    assert torch.equal(A.detach(), B.detach())
    for x, y in zip(g1, g2):
        assert torch.allclose(x, y, rtol=1e-12, atol=1e-15)


class _Strict:
    """An object with exactly the given attributes; reading any other raises (a stand-in
    for a reference module, whose attribute names it lists)."""

    def __init__(self, kind, **attrs):
        object.__setattr__(self, "_kind", kind)
        object.__setattr__(self, "_attrs", attrs)

    def __getattr__(self, name):
        attrs = object.__getattribute__(self, "_attrs")
        if name in attrs:
            return attrs[name]
        raise AttributeError(f"{object.__getattribute__(self, '_kind')} has no attribute {name!r}")


def test_integration_adapter_reads_reference_attributes(monkeypatch):
    """The INTEGRATION.md adapter (``xnn_amd.featurizers.fast_embed``) reads only what the
    reference's modules define: SphericalHarmonicEdgeEmbedding (spherical.py:86-101:
    cutoff, l_max, irreps_sh, sph, rbf, envelope, n_rbf), BesselRBF (radial.py:225-231:
    cutoff, freqs, norm), GaussianRBF (radial.py:56-59: centers, width, gamma) and
    PolynomialCutoff (cutoff.py:102-103: cutoff, p); the kernel arguments it forms equal
    those of this package's mirrored module. The HIP call is replaced by a recorder."""
    import xnn_amd.ops as ops
    from xnn_amd import featurizers as F
    seen = []
    monkeypatch.setattr(ops, "edge_embed", lambda vec, table, **kw: seen.append((table, kw)))
    for radial_type in ("bessel", "gaussian"):
        mine = F.SphericalHarmonicEdgeEmbedding(l_max=3, n_rbf=8, cutoff=4.5, p=5,
                                                radial_type=radial_type, rbf_prefactor=0.7)
        if radial_type == "bessel":
            rbf = _Strict("BesselRBF", cutoff=4.5, freqs=mine.rbf.freqs, norm=mine.rbf.norm)
        else:
            rbf = _Strict("GaussianRBF", centers=mine.rbf.centers, width=mine.rbf.width,
                          gamma=mine.rbf.gamma)
        ref = _Strict("SphericalHarmonicEdgeEmbedding", cutoff=4.5, l_max=3, irreps_sh=None,
                      sph=None, n_rbf=8, rbf=rbf,
                      envelope=_Strict("PolynomialCutoff", cutoff=4.5, p=5))
        vec = torch.randn(5, 3)
        F.fast_embed(ref, vec)
        mine.fast_active = True
        mine.embed(vec)
        (t_ref, kw_ref), (t_mine, kw_mine) = seen[-2], seen[-1]
        assert t_ref is t_mine and kw_ref == kw_mine
        assert kw_ref["basis"] == radial_type and kw_ref["envelope"] == "polynomial"
        assert kw_ref["poly_p"] == 5 and kw_ref["l_max"] == 3 and kw_ref["cutoff"] == 4.5
        if radial_type == "bessel":
            assert kw_ref["prefactor"] == 0.7
    # a basis the kernels do not have is an error, not a different function
    odd = _Strict("SphericalHarmonicEdgeEmbedding", cutoff=4.5, l_max=3, n_rbf=8,
                  rbf=_Strict("ExpNormalSmearing", means=None, betas=None),
                  envelope=_Strict("PolynomialCutoff", cutoff=4.5, p=6))
    with pytest.raises(TypeError, match="radial basis"):
        F.fast_embed(odd, torch.randn(2, 3))


def test_force_stress_output_contract_branches():
    """The wrapper's other branches (outputs.py:136-151, 187-194): a float64 geometry for a
    float32 model sets compute_dtype and differentiates at the float64 leaves; a model
    without an energy is returned as is; a model that predicts forces keeps them; one that
    forms its own forces and virial is not differentiated at all; direct forces with
    add-on energy terms are refused."""
    import copy
    import xnn_amd as xa
    from xnn_amd import synthetic
    s = synthetic.water_box(n_molecules=8, box=6.2, grid=2, seed=5)
    g = xa.structure_to_graph(s.as_dict(), 4.0)
    g.pos, g.cell = g.pos.double(), g.cell.double()
    model = xa.ShEdgePotential(n_rbf=4, l_max=1, channels=4, cutoff=4.0)   # float32
    g64 = copy.copy(g)
    out = xa.ForceStressOutput(model, compute_stress=True)(g64)
    assert g64.compute_dtype == torch.float32 and g.compute_dtype is None
    assert out["node_energy"].dtype == torch.float32 and out["forces"].dtype == torch.float64
    # the same model in float64 agrees to float32 rounding
    m64 = copy.deepcopy(model).double()
    ref = xa.ForceStressOutput(m64, compute_stress=True)(copy.copy(g))
    torch.testing.assert_close(out["forces"], ref["forces"], rtol=1e-4, atol=1e-5)

    class NoEnergy(torch.nn.Module):
        def forward(self, data):
            return {"properties": data.pos.sum(0)}

    out = xa.ForceStressOutput(NoEnergy(), compute_stress=True)(copy.copy(g))
    assert set(out) == {"properties"}

    class Direct(torch.nn.Module):
        def __init__(self, extra=False):
            super().__init__()
            self.extra = extra

        def forward(self, data):
            e = (data.pos ** 2).sum().reshape(1)
            out = {"energy": e, "forces": torch.ones_like(data.pos)}
            if self.extra:
                out["energy_sr"] = e
            return out

    out = xa.ForceStressOutput(Direct())(copy.copy(g))
    assert torch.equal(out["forces"], torch.ones_like(g.pos))
    with pytest.raises(ValueError, match="predicted by the model itself"):
        xa.ForceStressOutput(Direct(extra=True))(copy.copy(g))

    class FormsForces(torch.nn.Module):
        def forms_forces(self, data):
            return True

        def forward_direct(self, data):
            n = data.num_nodes
            return {"energy": torch.zeros(1, dtype=torch.float64),
                    "forces": torch.full((n, 3), 2.0, dtype=torch.float64),
                    "virial": torch.eye(3, dtype=torch.float64)[None]}

        def forward(self, data):
            raise AssertionError("the direct evaluation was expected")

    out = xa.ForceStressOutput(FormsForces(), compute_stress=True).eval()(copy.copy(g))
    vol = float(torch.linalg.det(g.cell[0]).abs())
    torch.testing.assert_close(out["stress"][0], torch.eye(3, dtype=torch.float64) / vol)
    assert "virial" not in out and float(out["forces"][0, 0]) == 2.0


def test_atomic_graph_subset_and_label_fields():
    """AtomicGraph carries the reference's label and mask fields, and ``subset`` keeps the
    flagged structures with renumbered atoms and edges (atomic_data.py:284-340)."""
    import xnn_amd as xa
    from xnn_amd import synthetic
    mols = synthetic.random_molecules(3, seed=1)
    graphs = [xa.structure_to_graph(m.as_dict(), 4.0) for m in mols]
    b = xa.collate(graphs)
    b.energy = torch.tensor([1.0, 2.0, 3.0], dtype=torch.float64)
    b.forces = torch.arange(b.num_nodes * 3, dtype=torch.float64).reshape(-1, 3)
    b.energy_mask = torch.tensor([True, False, True])
    b.charges = torch.arange(b.num_nodes, dtype=torch.float64)
    sub = b.subset(torch.tensor([True, False, True]))
    assert sub.num_graphs == 2 and sub.num_nodes == 42
    assert torch.equal(sub.energy, torch.tensor([1.0, 3.0], dtype=torch.float64))
    assert torch.equal(sub.energy_mask, torch.tensor([True, True]))
    assert torch.equal(sub.charges, torch.cat([b.charges[:21], b.charges[42:]]))
    assert torch.equal(sub.forces, torch.cat([b.forces[:21], b.forces[42:]]))
    assert sub.num_edges == graphs[0].num_edges + graphs[2].num_edges
    assert torch.equal(sub.edge_index[:, graphs[0].num_edges:],
                       graphs[2].edge_index + 21)
    assert torch.equal(sub.batch.bincount(), torch.tensor([21, 21]))
    for name in ("dipole", "polarizability", "spin_multiplicity", "weight", "head", "state",
                 "site_species", "energy_weight", "atom_force_weight", "fragment_charges"):
        assert getattr(sub, name) is None


def test_fast_selection_warns_once_for_float32_and_skips_unsupported_modules(monkeypatch):
    """fast.select: "auto" activates only the modules with a HIP path and warns once for
    float32 (fast.py:171-201, 41-59); explicit True with an unsupported module raises."""
    import warnings
    from xnn_amd import fast

    class Yes(fast.FastPathModule):
        def fast_supported(self, device, dtype):
            return True

    class No(fast.FastPathModule):
        def fast_supported(self, device, dtype):
            return False

    monkeypatch.setattr(fast._lib, "load", lambda: None)
    monkeypatch.setattr(fast, "_warned_float32", [False])
    mods = [Yes(), No()]
    policy = fast.AutoPolicy(default_min_edges=0)
    monkeypatch.setattr(policy, "decide", lambda device, dtype, n: True)
    with warnings.catch_warnings(record=True) as rec:
        warnings.simplefilter("always")
        assert fast.select(mods, "auto", policy, torch.device("cuda"), torch.float32, 10)
        fast.select(mods, "auto", policy, torch.device("cuda"), torch.float32, 10)
    assert [m.fast_active for m in mods] == [True, False]
    assert sum(issubclass(w.category, fast.FastPathPrecisionWarning) for w in rec) == 1
    with pytest.raises(RuntimeError, match="no HIP path"):
        fast.select(mods, True, policy, torch.device("cuda"), torch.float64, 10)


def test_bessel_exact_constants():
    from xnn_amd.featurizers import BesselRBF
    rbf = BesselRBF(8, 5.0).double()
    rbf.freqs.copy_(rbf.freqs.float().double())          # a float32 round trip
    assert rbf.exact_constants()
    assert torch.equal(rbf.freqs, math.pi * torch.arange(1, 9, dtype=torch.float64))
    assert not rbf.exact_constants()
    rbf.freqs[2] = 7.0                                     # not n pi: kept
    assert not rbf.exact_constants() and rbf.freqs[2] == 7.0
    assert not BesselRBF(8, 5.0).exact_constants()         # float32 buffer
    assert not BesselRBF(8, 5.0, trainable=True).double().exact_constants()


def test_no_alloc_entry_refuses_sizes_beyond_its_scratch_array_before_any_device_call():
    """xnn_segment_reduce_f64_noalloc checks the partial sums' size against its file-scope
    scratch array before it touches the device: the refusal needs no GPU and no buffers
    (NULL pointers here), so an oversized call can never reach a kernel."""
    import ctypes
    from xnn_amd import _lib
    lib = _lib.load()
    cap = int(lib.xnn_segment_reduce_noalloc_max_bytes())
    n, F = 1 << 20, 1024       # 256 chunks of 1024 features: 2 MiB of partials
    assert int(lib.xnn_segment_reduce_workspace_bytes(n, F, 1)) > cap
    rc = lib.xnn_segment_reduce_f64_noalloc(_lib.XNN_F32, None, n, F, None, 1, None, None)
    assert rc == _lib.XNN_EINVAL
    assert b"scratch" in lib.xnn_last_error()
    # within the limit the same call would go on to the device: not made here
    assert int(lib.xnn_segment_reduce_workspace_bytes(1 << 10, 8, 1)) <= cap


def test_factorized_reciprocal_product_equals_the_direct_sum():
    """The conjugate-gradient regime's reciprocal product (xnn_amd.eeq.FactorizedReciprocal:
    per-axis phase tables, columns of fixed (m1, m2), two stacked real GEMMs) against the
    direct cos / sin sum over the half set, for two right-hand sides, with the column table
    kept and formed again in blocks; its diagonal is sum_G w_G. Also the own-image diagonal
    against a direct sum and the Morton order (a permutation)."""
    from scipy.special import erf
    from xnn_amd import eeq as E
    g0 = torch.Generator().manual_seed(0)
    cell = torch.tensor([[9.0, 0, 0], [1.2, 8.5, 0], [-0.7, 0.9, 10.0]], dtype=torch.float64) / 0.5291772109
    pos = torch.rand(40, 3, dtype=torch.float64, generator=g0) @ cell * 1.3 - 2.0
    alpha = E.ewald_alpha(20.0)
    m = E.reciprocal_half_set(cell, alpha)
    g, w = E.reciprocal_weights(m, cell, alpha)
    v = torch.randn(40, 2, dtype=torch.float64, generator=g0)
    want = torch.stack([E.reciprocal_apply(pos, g, w, v[:, k]) for k in range(2)], 1)
    fr = E.FactorizedReciprocal(pos, cell, m, alpha)
    assert fr.table is not None
    torch.testing.assert_close(fr.apply(v), want, rtol=0, atol=1e-13)
    fr.block, fr.table = 7, None                  # the blocked form of a large system
    torch.testing.assert_close(fr.apply(v), want, rtol=0, atol=1e-13)
    assert abs(fr.diagonal - float(w.sum())) < 1e-15
    # own images within 25 bohr of a 9 A cell
    rad = torch.tensor([0.9, 2.1], dtype=torch.float64)
    got = E.own_image_diagonal(cell, rad, alpha, 25.0)
    want = np.zeros(2)
    c = cell.numpy()
    for a in range(-4, 5):
        for b in range(-4, 5):
            for k in range(-4, 5):
                r = float(np.linalg.norm(a * c[0] + b * c[1] + k * c[2]))
                if 0 < r <= 25.0:
                    gam = 1 / (math.sqrt(2) * rad.numpy())
                    want += (erf(gam * r) - erf(alpha * r)) / r
    assert want[0] != 0.0
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-13)
    order = E.morton_order(torch.rand(1000, 3, dtype=torch.float64, generator=g0))
    assert torch.equal(torch.sort(order).values, torch.arange(1000))


def test_low_rank_preconditioner_inverts_its_matrix():
    """The conjugate-gradient regime's preconditioner M = D + U W U^T (U the cos / sin of the
    smallest reciprocal vectors at the ordered positions, D the full diagonal less their
    part) applied through the Woodbury identity: M (M^-1 r) = r for two columns, with M
    formed explicitly; the set-up runs no device code."""
    from xnn_amd import eeq as E
    g0 = torch.Generator().manual_seed(3)
    cell = torch.tensor([[9.0, 0, 0], [1.2, 8.5, 0], [-0.7, 0.9, 10.0]], dtype=torch.float64) / 0.5291772109
    n = 60
    pos = torch.rand(n, 3, dtype=torch.float64, generator=g0) @ cell
    rad = torch.rand(n, dtype=torch.float64, generator=g0) + 1.0
    diag = torch.rand(n, dtype=torch.float64, generator=g0) + 0.5
    alpha = E.ewald_alpha(20.0)
    system = E.IterativeEEQSystem(pos, cell, rad, diag - 2 * alpha / math.sqrt(math.pi), alpha, 20.0)
    assert system.U is not None and system.U.shape == (n, 2 * min(E.LOW_K_VECTORS, len(system.m)))
    g, w = E.reciprocal_weights(system.m, cell, alpha)
    L = system.U.shape[1] // 2
    wl = w[torch.argsort((g * g).sum(1))[:L]]
    M = torch.diag(1.0 / system.inv_d) + system.U @ torch.diag(torch.cat([wl, wl])) @ system.U.t()
    r = torch.randn(n, 2, dtype=torch.float64, generator=g0)
    torch.testing.assert_close(M @ system.precondition(r), r, rtol=0, atol=1e-11)
