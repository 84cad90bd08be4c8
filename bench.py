"""Benchmark of the per-edge hot path on one MI355X (the BASELINE.json metric).

Workload (``--config water``, the default): the 9,000-atom liquid water box (3,000 rigid
H2O at 1.0 g/cm^3, cubic periodic cell of 44.8 A), cutoff 5.0 A, 8 Bessel radial
functions x polynomial envelope, real SH l <= 3 (16 components), 128 float32 channels.
A step is one evaluation of ``ForceStressOutput(ShEdgePotential)`` (``--variant rows``, the
default, the metric's pipeline): edge vectors -> radial basis + radial linear + SH message
sum into the (N, 128, 16) rows A in one kernel, written to HBM (the radial features u are
evaluated per lane, the sum is taken as A_i = W^T sum_e u_e (x) Y_e, so phi = u W is never
formed) -> readout as its own op (reads A) -> float64 energy -> backward: the readout's
backward writes the rows' cotangent (N, 128, 16), the message backward reads it (a general
cotangent, as a model whose rows feed PyTorch layers hands back) and returns the edge
vectors' gradient -> force and virial reduction, all on the GPU with inputs resident in
HBM. ``--variant readout`` / ``one_pass`` time the kernels that apply the readout
themselves (no rows in memory) as labelled secondary lines. The neighbor list is timed
separately (``neighbor_list_ms``).

Prints one JSON line. ``value`` = edges / (forward + force/stress backward time).
``roofline`` is the dominant kernel's algorithmic work per launch (HBM bytes, or fp32
matrix-core flops when those bound it) divided by its mean launch time, measured with
HIP events on its launch stream over back-to-back launches on the workload's inputs.
``cpu_baseline`` times the oracle's PyTorch-CPU restatement of the same step on the
host cores (rank 0, N = 1 only).
"""
from __future__ import annotations

import argparse
import copy
import ctypes
import json
import math
import os
import sys
import time

import numpy as np
import torch

HBM_PEAK_GBS = 8000.0
ctypes_i64 = ctypes.c_int64
ROOT = os.path.dirname(os.path.abspath(__file__))
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "hbm_traffic_message_kernels_water_box.md")


def measured_traffic(kernel: str, workload: str):
    """HBM bytes per launch of ``kernel`` from the committed counter profile (FETCH_SIZE
    and WRITE_SIZE passes scaled by the copy calibration), for the water box only."""
    if workload != "water_box_9000_atoms_rc5" or not os.path.exists(TRAFFIC_PROFILE):
        return None
    for line in open(TRAFFIC_PROFILE):
        f = line.split()
        if len(f) == 3 and f[0] == "traffic_bytes_per_launch" and f[1] == kernel:
            return int(f[2])
    return None


def copy_calibration() -> None:
    """A plain device copy of 256 MiB, three launches: the known-size kernel that scales
    the FETCH_SIZE / WRITE_SIZE counters of a profile run to bytes."""
    n = 64 * 1024 * 1024
    a = torch.ones(n, device="cuda")
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_per_launch": 4 * n, "launches": 3}), flush=True)


MFMA_F32_PEAK_TFLOPS = 157.3


def copy_bandwidth_gbs(mib: int = 1024, reps: int = 20) -> float:
    """Measured device-to-device copy rate (bytes read + written per second) of a plain
    ``mib`` MiB copy between HIP events on the current stream: the attainable HBM rate
    reported next to the fractions of the 8 TB/s vendor peak."""
    n = mib * 1024 * 1024 // 4
    a = torch.ones(n, device="cuda")
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(reps):
        b.copy_(a)
    end.record()
    torch.cuda.synchronize()
    t = start.elapsed_time(end) * 1e-3 / reps
    return 2 * 4 * n / t / 1e9


def kernel_costs(E: int, N: int, C: int, L: int = 16, K: int = 8, grouped: bool = True) -> dict:
    """Compulsory HBM bytes and matrix-core flops per launch of each kernel: int32
    indices, float32 features, edge vectors given (12 B per edge), no perm when the edges
    come grouped by receiver. Flops count the true dimensions (no padding)."""
    perm = 0 if grouped else 4
    return {
        # the readout in the kernels: each edge's share h_e^T (W U) Y_e of its receiver's
        # energy (2 K L + 2 K flops), its gradient g_i ((W U) Y_e, (W U)^T h_e) (4 K L)
        "xnn_sh_radial_message_energy": {                  # radial basis and readout in-kernel
            "bytes": E * (12 + perm) + N * (4 + 4 + 8) + 4 * C * L,  # vec in; ptr, z; E_i out
            "flops": E * (2 * K * L + 2 * K)},
        "xnn_sh_radial_message_energy_backward": {
            "bytes": E * (12 + perm + 12) + N * 4 + 4 * C * L,   # vec in, g_vec out; ptr; U
            "flops": E * 4 * K * L},
        "xnn_sh_radial_message_energy_forces": {           # the backward, + each edge's share
            "bytes": E * (12 + perm + 12 + 4) + N * 4 + 4 * C * L,   # of E_i out (no forward)
            "flops": E * (4 * K * L + 2 * K)},
        # the rows kernels apply the linear layer per atom, A_i = W^T sum_e u_e (x) Y_e:
        # 2 K L flops per edge for the feature-row sums, 2 C K L per atom for W^T B_i;
        # backward 2 C K L per atom for dB_i = W G_i and 4 K L per edge for d u_e and dY_e
        "xnn_sh_radial_message_sum": {                     # radial basis evaluated in-kernel
            "bytes": E * (12 + perm) + N * (4 * C * L + 4),   # vec in; ptr; A out
            "flops": E * 2 * K * L + N * 2 * C * K * L},
        "xnn_sh_radial_message_sum_backward": {
            "bytes": E * (12 + perm + 12) + N * (4 * C * L + 4),  # vec in, g_vec out; G in
            "flops": E * 4 * K * L + N * 2 * C * K * L},
        "xnn_sh_linear_message_sum": {
            "bytes": E * (12 + 4 * K + perm) + N * (4 * C * L + 4),
            "flops": E * 2 * K * L + N * 2 * C * K * L},
        "xnn_sh_linear_message_sum_backward": {
            "bytes": E * (12 + 4 * K + perm + 4 * K + 12) + N * (4 * C * L + 4),
            "flops": E * 4 * K * L + N * 2 * C * K * L},
        "xnn_node_readout": {                              # rows in, z in, E_i out
            "bytes": N * (4 * C * L + 8 + 4) + 4 * C * L, "flops": N * 2 * C * L},
        "xnn_node_readout_backward": {                     # broadcast seed, d_rows out
            "bytes": N * 4 * C * L + 4 * C * L, "flops": N * C * L},
        "xnn_sh_message_sum": {
            "bytes": E * (12 + 4 * C + perm) + N * (4 * C * L + 4),
            "flops": E * 2 * C * L},
        "xnn_sh_message_sum_backward": {
            "bytes": E * (12 + 4 * C + perm + 4 * C + 12) + N * (4 * C * L + 4),
            "flops": E * 4 * C * L},
        "xnn_edge_featurize": {"bytes": E * (12 + 4 * K + 4), "flops": 0},
        "xnn_edge_featurize_backward": {"bytes": E * (12 + 4 * K + 4 + 12 + 12), "flops": 0},
        "xnn_edge_force_reduce": {"bytes": E * (12 + 4) + N * (12 + 72 + 8), "flops": 0},
    }


def step_bytes(E: int, N: int, C: int, L: int, K: int, msg: str) -> int:
    """Compulsory traffic of one whole step: edge vectors from positions, featurizer
    (unless the message kernels evaluate the radial basis), message sum, readout (reads
    A), its backward (writes d_A), message backward, featurizer backward, force reduction.
    With the readout in the message kernels no (N, C, L) rows exist."""
    kc = kernel_costs(E, N, C, L, K)
    if msg == "xnn_sh_radial_message_energy_forces":     # one launch: energies and forces
        return (E * 24 + N * 12 + kc[msg]["bytes"] + E * 4 + N * 4
                + kc["xnn_edge_force_reduce"]["bytes"])
    if msg == "xnn_sh_radial_message_energy":
        return (E * 24 + N * 12 + kc[msg]["bytes"] + kc[msg + "_backward"]["bytes"]
                + kc["xnn_edge_force_reduce"]["bytes"])
    feat = 0 if msg == "xnn_sh_radial_message_sum" else (
        kc["xnn_edge_featurize"]["bytes"] + kc["xnn_edge_featurize_backward"]["bytes"])
    linear = 2 * (E * 4 * (K + C)) if msg == "xnn_sh_message_sum" else 0  # u @ W, d_phi @ W^T
    return (E * 24 + N * 12 + feat + kc[msg]["bytes"] + N * 4 * C * L + N * 4 * C * L
            + kc[msg + "_backward"]["bytes"] + kc["xnn_edge_force_reduce"]["bytes"] + linear)


def pipeline_bytes(E: int, N: int, C: int) -> int:
    """Algorithmic bytes of the unfused featurize -> phi -> message -> readout -> backward
    pipeline that the metric's HBM roofline is quoted on: E (124 + 12 C) + N (76 + 8 C 16)
    (the edge streams, phi and d_phi per edge; the (C, 16) node rows and their cotangent)."""
    return E * (124 + 12 * C) + N * (76 + 8 * C * 16)


def message_launches(msg: str, g, model, kw: dict) -> dict:
    """The C-ABI calls of the step's message kernels, forward and backward, on the
    workload's own inputs (edge vectors, weights, a random node cotangent), as
    ``name -> (args, keep)``: replayed back to back they time one launch without the host
    gaps of the eager step."""
    from xnn_amd import _lib
    from xnn_amd.ops import _params
    feat = model.edge_feat
    plan = g.plan()
    vec = g.edge_vectors().detach().float().contiguous()
    E, N = vec.shape[0], g.num_nodes
    C, L = kw["channels"], (kw["l_max"] + 1) ** 2
    W = model.W.detach().float().contiguous()
    K = W.shape[0]
    gen = torch.Generator(device=vec.device).manual_seed(0)
    d_out = torch.randn((N, C, L), device=vec.device, generator=gen)
    out = torch.empty((N, C, L), device=vec.device)
    g_vec = torch.empty_like(vec)
    s = _lib.stream(vec.device)
    rbf = feat.rbf
    table = feat._table().detach().float().contiguous()
    prm = _params([K, _lib.BASIS[feat.radial_type], _lib.ENVELOPE[feat.envelope_type],
                   int(getattr(feat.envelope, "p", 1)), kw["l_max"], model.sh_sign],
                  [float(feat.cutoff), float(getattr(rbf, "norm", 1.0)),
                   float(getattr(rbf, "gamma", 1.0))])
    head = (_lib.XNN_F32, _lib.ptr(vec), None, N, None, 0, None, None, None, E,
            _lib.ptr(plan.ptr_dst), _lib.ptr(plan.perm_dst))
    keep = (vec, W, d_out, out, g_vec, table, plan)
    if msg in ("xnn_sh_radial_message_energy", "xnn_sh_radial_message_energy_forces"):
        U = model.U.detach().float().reshape(-1).contiguous()
        z = g.atomic_numbers.to(torch.int64).contiguous()
        bias = model.atom_ref.detach().float().contiguous()
        energy = torch.empty(N, device=vec.device)
        g_node = torch.full((1,), -1.0, device=vec.device)          # the forces' seed
        keep = keep + (U, z, bias, energy, g_node)
        if msg.endswith("_forces"):                  # the one launch of a one-pass step
            edge_energy = torch.empty(E, device=vec.device)
            keep = keep + (edge_energy,)
            return {msg: (head + (prm, _lib.ptr(table), C, _lib.ptr(W), _lib.ptr(U),
                                  _lib.ptr(g_node), 0, _lib.ptr(g_vec), _lib.ptr(edge_energy), s),
                          keep)}
        return {msg: (head + (prm, _lib.ptr(table), C, _lib.ptr(W), _lib.ptr(U), _lib.ptr(z),
                              _lib.ptr(bias), bias.shape[0], _lib.ptr(energy), s), keep),
                msg + "_backward": (head + (prm, _lib.ptr(table), C, _lib.ptr(W), _lib.ptr(U),
                                            _lib.ptr(g_node), 0, _lib.ptr(g_vec), s), keep)}
    if msg == "xnn_sh_radial_message_sum":
        return {msg: (head + (prm, _lib.ptr(table), C, _lib.ptr(W), _lib.ptr(out), s), keep),
                msg + "_backward": (head + (prm, _lib.ptr(table), C, _lib.ptr(W),
                                            _lib.ptr(d_out), _lib.ptr(g_vec), s), keep)}
    if msg == "xnn_sh_linear_message_sum":
        h = feat.radial(vec).detach().contiguous()
        d_h = torch.empty_like(h)
        keep = keep + (h, d_h)
        tail = (kw["l_max"], model.sh_sign, K, C, _lib.ptr(h), _lib.ptr(W))
        return {msg: (head + tail + (_lib.ptr(out), s), keep),
                msg + "_backward": (head + tail + (_lib.ptr(d_out), _lib.ptr(d_h),
                                                   _lib.ptr(g_vec), s), keep)}
    return {}


def replay_launch_us(name: str, args: tuple, reps: int = 40) -> float:
    """Mean duration of ``reps`` back-to-back launches of a C-ABI entry point, between HIP
    events recorded on the stream the kernels run on."""
    from xnn_amd import _lib
    fn = getattr(_lib.load(), name)
    for _ in range(3):
        _lib.check(name, fn(*args))
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(reps):
        fn(*args)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / reps * 1e3


def build_workload(config: str, device):
    import xnn_amd as xa
    from xnn_amd import synthetic
    if config == "water":
        s = synthetic.water_box(seed=0)
        rc, kw = 5.0, dict(n_rbf=8, l_max=3, channels=128, radial_type="bessel",
                           envelope="polynomial", p=6)
        structs, workload = [s], "water_box_9000_atoms_rc5"
    elif config == "argon":
        s = synthetic.argon_fcc(seed=0)
        rc, kw = 6.0, dict(n_rbf=8, l_max=3, channels=64, radial_type="bessel", envelope="cosine")
        structs, workload = [s], "argon_fcc_4000_atoms_rc6"
    elif config == "ragged":
        structs = synthetic.ragged_molecules(1024, seed=0)
        rc, kw = 5.0, dict(n_rbf=8, l_max=3, channels=64, radial_type="bessel",
                           envelope="polynomial", p=6)
        workload = "ragged_1024_molecules_rc5"
    else:
        raise SystemExit(f"unknown config {config!r}")
    t0 = time.perf_counter()
    if len(structs) == 1:
        s = structs[0]
        pos = torch.tensor(s.pos, dtype=torch.float32, device=device)
        cell = torch.tensor(s.cell, dtype=torch.float32, device=device)
        pbc = torch.tensor(s.pbc)
        # warm-up builds: the first plans the grid, the second allocates the outputs sized
        # from the plan's last list; the timed builds are the steady state
        for _ in range(5):
            ei, sh = xa.build_neighbor_list(pos, rc, cell, pbc)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        reps = 100
        for _ in range(reps):
            ei, sh = xa.build_neighbor_list(pos, rc, cell, pbc)
        torch.cuda.synchronize()
        nl_ms = (time.perf_counter() - t0) / reps * 1e3
        g = xa.AtomicGraph(pos=pos, atomic_numbers=torch.tensor(s.numbers, device=device),
                           edge_index=ei, cell_shifts=sh,
                           batch=torch.zeros(len(s.pos), dtype=torch.long, device=device),
                           n_atoms=torch.tensor([len(s.pos)], device=device), cell=cell[None],
                           pbc=pbc[None].to(device))
    else:
        pos = torch.tensor(np.concatenate([m.pos for m in structs]), dtype=torch.float32,
                           device=device)
        n_atoms = torch.tensor([len(m.pos) for m in structs], device=device)
        ei, sh = xa.batched_neighbor_list(pos, n_atoms, rc)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        reps = 5
        for _ in range(reps):
            ei, sh = xa.batched_neighbor_list(pos, n_atoms, rc)
        torch.cuda.synchronize()
        nl_ms = (time.perf_counter() - t0) / reps * 1e3
        z = torch.tensor(np.concatenate([m.numbers for m in structs]), device=device)
        batch = torch.repeat_interleave(torch.arange(len(structs), device=device), n_atoms)
        g = xa.AtomicGraph(pos=pos, atomic_numbers=z, edge_index=ei, cell_shifts=sh, batch=batch,
                           n_atoms=n_atoms)
    model = xa.ShEdgePotential(cutoff=rc, species=(1, 6, 7, 8, 18), seed=0, **kw).to(device)
    return g, model, rc, kw, workload, nl_ms, structs


def physical_cores() -> int:
    """Physical cores among the CPUs this process may run on (distinct (package, core)
    pairs of /proc/cpuinfo); the affinity count when that file says nothing."""
    allowed = os.sched_getaffinity(0)
    cores, cpu, pkg = set(), None, "0"
    try:
        for line in open("/proc/cpuinfo"):
            key, _, val = line.partition(":")
            key, val = key.strip(), val.strip()
            if key == "processor":
                cpu = int(val)
            elif key == "physical id":
                pkg = val
            elif key == "core id" and cpu in allowed:
                cores.add((pkg, val))
    except OSError:
        pass
    return len(cores) if cores else len(allowed)


def _cpu_stages(g, params, n_sample: int, stress: bool) -> dict:
    """One float32 step of the oracle's PyTorch-CPU restatement over the first
    ``n_sample`` edges, stage by stage (seconds): edge vectors (atomic_data.py:371-418),
    featurize (radial basis x envelope and SH, spherical.py:115-138), phi = u W, the message
    scatter (index_add, ops.py:403-448), readout and float64 sum (ops.py:531-557), and the
    autograd backward to forces and stress (outputs.py:166-239)."""
    import oracle.reference as R
    t = {}
    clock = time.perf_counter
    pos = g.pos.detach().cpu()
    cell = None if g.cell is None else g.cell.detach().cpu()
    ei, sh = g.edge_index[:, :n_sample].cpu(), g.cell_shifts[:n_sample].cpu()
    batch, z = g.batch.cpu(), g.atomic_numbers.cpu()
    t0 = clock()
    strain = torch.zeros((g.num_graphs, 3, 3), dtype=pos.dtype, requires_grad=True)
    sym = 0.5 * (strain + strain.transpose(-1, -2))
    leaf = pos.clone().requires_grad_(True)
    p2 = leaf + (leaf[:, :, None] * sym.index_select(0, batch)).sum(1)
    c2 = None if cell is None else cell + (cell[:, :, :, None] * sym[:, None]).sum(2)
    vec = R.edge_vectors(p2, ei, sh, c2, batch, None)
    t1 = clock()
    length = torch.linalg.norm(vec, dim=-1)
    u = R.radial_features(length, params["n_rbf"], params["cutoff"], params["radial"],
                          params["envelope"])
    y = R.e3nn_sh(params["l_max"], vec)
    t2 = clock()
    phi = u @ params["W"]
    t3 = clock()
    C, L = phi.shape[1], y.shape[1]
    A = torch.zeros((pos.shape[0], C * L), dtype=vec.dtype)
    for e0 in range(0, n_sample, 1 << 15):
        e1 = min(n_sample, e0 + (1 << 15))
        A = A.index_add(0, ei[1, e0:e1], (phi[e0:e1, :, None] * y[e0:e1, None, :]).reshape(-1, C * L))
    t4 = clock()
    node = A @ params["U"].reshape(-1) + params["atom_ref"][z]
    energy = R.structure_sum(node, batch, g.num_graphs)
    t5 = clock()
    inputs = [leaf, strain] if (stress and cell is not None) else [leaf]
    torch.autograd.grad(energy.sum(), inputs)
    t6 = clock()
    return {"edge_vectors": t1 - t0, "featurize": t2 - t1, "phi": t3 - t2,
            "segment_sum": t4 - t3, "readout_sum": t5 - t4, "backward": t6 - t5,
            "total": t6 - t0}


def cpu_neighbor_list(g, rc: float) -> dict:
    """The neighbor list on the host: the oracle's brute-force restatement of the
    reference's list (neighborlist.py:462-506, C, one thread) over every structure of the
    workload, timed once (a few seconds for the water box)."""
    import oracle.nl as N
    pos = g.pos.detach().cpu().numpy()
    cells = None if g.cell is None else g.cell.detach().cpu().numpy().reshape(-1, 3, 3)
    pbcs = None if g.pbc is None else g.pbc.detach().cpu().numpy().reshape(-1, 3)
    counts = [int(c) for c in g.n_atoms.cpu()]
    t0 = time.perf_counter()
    start, edges = 0, 0
    for b, n in enumerate(counts):
        ei, _, _ = N.neighbor_list(pos[start:start + n], rc,
                                   None if cells is None else cells[b],
                                   None if pbcs is None else pbcs[b], dtype=np.float32)
        edges += ei.shape[1]
        start += n
    dt = time.perf_counter() - t0
    return {"seconds": round(dt, 3), "value": edges / dt, "unit": "edges/s", "cores": 1,
            "kind": "port", "sample": f"the whole workload's list ({edges} edges of "
                                      f"{len(counts)} structure(s)), brute force over the "
                                      f"image range, float32, one thread"}


def cpu_baseline(g, model, rc, kw, max_edges: int, one_thread_edges: int = 60_000) -> dict:
    """The oracle's PyTorch-CPU restatement of one step (float32) on bounded samples of
    the workload (the edges of the first receivers in CSR order): the median of 5 timed
    steps after 2 warm-ups, with torch on the physical cores, and again on one thread over
    a smaller sample; per-stage medians of the multi-thread run."""
    params = dict(W=model.W.detach().cpu(), U=model.U.detach().cpu(),
                  atom_ref=model.atom_ref.detach().cpu(), l_max=kw["l_max"], n_rbf=kw["n_rbf"],
                  cutoff=rc, radial=kw["radial_type"], envelope=kw["envelope"])
    stress = g.cell is not None
    threads_before = torch.get_num_threads()
    n_phys = physical_cores()

    def run(n_edges: int, threads: int):
        torch.set_num_threads(threads)
        for _ in range(2):
            _cpu_stages(g, params, n_edges, stress)
        runs = [_cpu_stages(g, params, n_edges, stress) for _ in range(5)]
        return {k: float(np.median([r[k] for r in runs])) for k in runs[0]}

    try:
        E = g.num_edges
        n_many = min(E, max_edges)
        many = run(n_many, n_phys)
        n_one = min(E, one_thread_edges)
        one = run(n_one, 1)
    finally:
        torch.set_num_threads(threads_before)
    return {"value": n_many / many["total"], "unit": "edges/s", "cores": n_phys,
            "kind": "port", "statistic": "median of 5 after 2 warm-ups",
            "stage_seconds": {k: round(v, 4) for k, v in many.items()},
            "one_thread": {"value": n_one / one["total"], "edges": n_one,
                           "stage_seconds": {k: round(v, 4) for k, v in one.items()}},
            "neighbor_list": cpu_neighbor_list(g, rc),
            "os_cpu_count": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0)),
            "physical_cores": n_phys, "torch_threads": n_phys,
            "sample": f"float32 forward + force/stress backward of the oracle's PyTorch-CPU "
                      f"restatement over the first {n_many} of {E} edges (receivers in CSR "
                      f"order) on {n_phys} threads, and over the first {n_one} edges on one "
                      f"thread"}


def _d4_sample_pairs(pos: np.ndarray, cell: np.ndarray, k: int, cutoff: float):
    """Directed pair images (dst < k, any src) within ``cutoff`` Angstrom, brute force over
    the image range that covers it: dst, src, shift arrays (the CPU baseline's sample)."""
    inv = np.linalg.inv(cell)
    reps = [int(math.ceil(cutoff * float(np.linalg.norm(inv[:, a])))) for a in range(3)]
    dst, src, sh = [], [], []
    for a in range(-reps[0], reps[0] + 1):
        for b in range(-reps[1], reps[1] + 1):
            for c in range(-reps[2], reps[2] + 1):
                t = a * cell[0] + b * cell[1] + c * cell[2]
                d = pos[:k, None, :] - pos[None, :, :] + t
                r2 = (d * d).sum(-1)
                ii, jj = np.nonzero((r2 <= cutoff * cutoff) & (r2 > 0))
                dst.append(ii)
                src.append(jj)
                sh.append(np.repeat(np.array([[a, b, c]]), len(ii), axis=0))
    return np.concatenate(dst), np.concatenate(src), np.concatenate(sh)


def cpu_baseline_d4(s, tables, alpha: np.ndarray, model, k: int = 200,
                    min_seconds: float = 10.0) -> dict:
    """The oracle's two-body D4 (PyTorch on the CPU, float64) with its position gradient,
    over the pair images of the first ``k`` receivers (enumeration included), repeated
    until about ``min_seconds``; alpha(i w) given (from the GPU run of the same step)."""
    import oracle.d4 as D
    pos, cell = np.asarray(s.pos, dtype=np.float64), np.asarray(s.cell, dtype=np.float64)
    z = torch.as_tensor(np.asarray(s.numbers))
    a_t = torch.as_tensor(alpha)
    prm = dict(D.PBE0_D4)
    cut_aa = model.cutoff_pair
    reps, dt, n_terms = 0, 0.0, 0
    t0 = time.perf_counter()
    while reps < 30 and (reps == 0 or dt < min_seconds):
        dst, src, sh = _d4_sample_pairs(pos, cell, k, cut_aa)
        pt = torch.tensor(pos, requires_grad=True)
        v = D.edge_vectors_au(pt, torch.as_tensor(cell), dst, src, sh)
        r = torch.linalg.norm(v, dim=-1)
        e2 = D.two_body(z, dst, src, r, a_t, tables, prm, cut_aa / D.BOHR, 0.0, len(pos))
        (g,) = torch.autograd.grad(e2.sum(), [pt])
        n_terms = len(dst)
        reps += 1
        dt = time.perf_counter() - t0
    return {"value": reps * n_terms / dt, "unit": "terms/s", "cores": torch.get_num_threads(),
            "kind": "port", "seconds": round(dt, 2), "steps": reps,
            "sample": f"{reps} x the two-body energy + position gradient over the {n_terms} "
                      f"pair-image terms of the first {k} of {len(pos)} receivers (pair "
                      f"enumeration included; alpha(i w) given), oracle PyTorch-CPU float64, "
                      f"torch threads={torch.get_num_threads()}"}


# algorithmic float64 flops per launch of the D4 kernels (M pair-image terms within the
# pair cutoff, P = N (N + 1) / 2 atom pairs, M_cn CN terms): the forward pair and CN
# counts are the survey's 60 M + 46 P and 40 M_cn; the pair backward adds per term the
# r-derivative of the damped sum and the force and cell-gradient products (35) and per
# pair the two atoms' d C6 / d alpha (2 x 46): 95 M + 138 P
# Algorithmic float64 flops of each entry point, counted on the unordered sums (each pair
# image enters the energy once, for both of its atoms): M directed pair-image terms within the
# cutoff are M / 2 unordered ones, P = N (N + 1) / 2 atom pairs, Mc directed CN terms.
# Per pair-image term, the energy: the image vector and r^2 (8), r^4 r^6 r^8 (3), the two
# BJ denominators and their common Newton-refined reciprocal (12), t6 t8 and g (5), the sum (1)
# = 29; the backward adds df/dr / r (10) and its vector, force and cell-moment sums (18) = 57.
# Per atom pair: C6 (46) and the damping radius, r0^6 r0^8, the pair's energy to both atoms
# (16) = 62 forward; the backward's C6, forces to both atoms, the cell moment (51) and dE/d
# alpha of both atoms (2 x 46 + 3) = 170. CN: 40 per unordered term.
D4_FLOPS = {"xnn_d4_two_body": lambda M, P, Mc: 29 * M // 2 + 62 * P,
            "xnn_d4_two_body_backward": lambda M, P, Mc: 57 * M // 2 + 170 * P,
            "xnn_d4_coordination": lambda M, P, Mc: 40 * Mc // 2}
FP64_PEAK_TFLOPS = 78.6


def bench_d4(steps: int, warmup: int, cpu: bool = True, graph: bool = True) -> dict:
    """D4 two-body energy + forces + stress of the 5,000-atom organic box (36.8 A cell,
    cutoffs 60 / 25 / 25 bohr for pair / CN / EEQ CN): CN kernel, polarizabilities, pair kernel and
    both backward kernels per step. The charges come from the EEQ solve once, outside the
    timed steps, as the survey's configuration specifies; the energy evaluation with the
    EEQ solve is timed beside it."""
    import xnn_amd.dispersion as XD
    from xnn_amd import _lib, synthetic
    dev = torch.device("cuda:0")
    s = synthetic.organic_box(seed=0)
    tables = XD.load_d4_tables(os.path.join(ROOT, "tests", "golden", "d4_tables_hcnoar.npz"))
    # pairwise only (the config's s9 = 0); pair cutoff 60 bohr, CN and EEQ-CN cutoffs 25 bohr
    model = XD.DFTD4(tables, s9=0.0, cutoff_cn=25.0 * XD.BOHR,
                     cutoff_eeq_cn=25.0 * XD.BOHR).to(dev)
    z = torch.tensor(s.numbers, device=dev)
    pos0 = torch.tensor(s.pos, dtype=torch.float64, device=dev)
    cell0 = torch.tensor(s.cell, dtype=torch.float64, device=dev)[None]
    pbc = torch.ones((1, 3), dtype=torch.bool)
    n_atoms = torch.tensor([len(s.numbers)])
    with torch.no_grad():                     # warm-up (library initialization)
        q = model.evaluate(z, pos0, cell0, pbc, n_atoms)["charges"].detach()
    # the whole D4 evaluation with its EEQ charges (the large regime's converged Ewald
    # operator on the device, regime="auto" above 500 periodic atoms), energy only
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    with torch.no_grad():
        for _ in range(3):
            q = model.evaluate(z, pos0, cell0, pbc, n_atoms)["charges"].detach()
    torch.cuda.synchronize()
    eeq_ms = (time.perf_counter() - t0) / 3 * 1e3

    def step():
        pos = pos0.clone().requires_grad_(True)
        cell = cell0.clone().requires_grad_(True)
        out = model.evaluate(z, pos, cell, pbc, n_atoms, charges=q, fused_pair=True)
        gp, gc = torch.autograd.grad(out["energy"].sum(), [pos, cell])
        return out, gp, gc

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        out, gp, gc = step()
    torch.cuda.synchronize()
    eager_ms = ms = (time.perf_counter() - t0) / steps * 1e3
    e = out["energy"].detach()
    graph_checked = None
    if graph:
        # the whole step (evaluation, forces and cell gradient) as one HIP graph, replayed;
        # an MD driver copies new positions into pos0 / cell0 before each replay
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(3):
                step()
        torch.cuda.current_stream().wait_stream(side)
        hip_graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(hip_graph):
            s_out, s_gp, s_gc = step()
        for _ in range(max(1, warmup)):
            hip_graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            hip_graph.replay()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) / steps * 1e3
        # several replays, eager work between them, each against the eager step bit for bit
        r_out, r_gp, r_gc = step()
        graph_checked = True
        for _ in range(3):
            hip_graph.replay()
            torch.cuda.synchronize()
            graph_checked = graph_checked and bool(
                torch.equal(s_gp, r_gp) and torch.equal(s_gc, r_gc)
                and torch.equal(s_out["energy"], r_out["energy"]))
            step()
            torch.cuda.synchronize()
        if not graph_checked:
            raise SystemExit("graph replay differs from the eager D4 step")
    # per-kernel HIP events (launch stream) over a second set of steps
    kernels = list(D4_FLOPS) + ["xnn_d4_coordination_backward", "xnn_d4_polarizabilities",
                                "xnn_d4_polarizabilities_backward"]
    _lib.timed.clear()
    _lib.time_launches(*kernels)
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    kernel_us = {k: float(np.mean([a.elapsed_time(b) * 1e3 for a, b in v]))
                 for k, v in _lib.timed.items() if v}
    _lib.timed.clear()
    # pair-image terms within the pair cutoff (for the rate) and CN terms, image by image
    imgs = XD.image_counts(cell0, pbc, model.cutoff_pair)[0].tolist()
    n_terms, n_cn = 0, 0
    with torch.no_grad():
        d0 = pos0[:, None, :] - pos0[None, :, :]
        rc2, rcn2 = model.cutoff_pair ** 2, model.cutoff_cn ** 2
        for a in range(-imgs[0], imgs[0] + 1):
            for b in range(-imgs[1], imgs[1] + 1):
                for c in range(-imgs[2], imgs[2] + 1):
                    t = a * cell0[0, 0] + b * cell0[0, 1] + c * cell0[0, 2]
                    r2 = ((d0 + t) ** 2).sum(-1)
                    n_terms += int(((r2 <= rc2) & (r2 > 0)).sum())
                    n_cn += int(((r2 <= rcn2) & (r2 > 0)).sum())
        del d0
    N = len(s.numbers)
    dominant = max(kernel_us, key=lambda k: kernel_us[k])
    flops = D4_FLOPS[dominant](n_terms, N * (N + 1) // 2, n_cn) if dominant in D4_FLOPS else None
    achieved = flops / (kernel_us[dominant] * 1e-6) / 1e12 if flops else None
    roofline = {"bound": "fp64", "kernel": dominant,
                "achieved": None if achieved is None else round(achieved, 2),
                "peak": FP64_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": None if achieved is None else round(achieved / FP64_PEAK_TFLOPS, 4),
                "traffic": None, "algorithmic_flops": flops,
                "mean_launch_us": round(kernel_us[dominant], 2),
                "timing": "eager step, HIP events on the launch stream"}
    result = {"metric": "D4 pair-image terms/s, energy+forces+stress, 5000-atom organic box",
              "value": n_terms / (ms * 1e-3), "unit": "terms/s", "n_gpus": 1, "steps": steps,
              "warmup": warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
              "vs_baseline": None, "dtype": "f64", "data": "synthetic (seeded generator)",
              "config": {"workload": "d4_organic_box_5000_atoms", "atoms": N,
                         "pair_image_terms": n_terms, "cn_terms": n_cn,
                         # within-cutoff pair-image terms over the 27 N^2 candidates of the
                         # 3 x 3 x 3 image block (the kernels test per-source image windows)
                         "candidate_test_efficiency": round(n_terms / (27.0 * N * N), 4),
                         "cutoff_pair_bohr": 60.0, "cutoff_cn_bohr": 25.0,
                         "cutoff_eeq_cn_bohr": 25.0,
                         "charges": "EEQ charges (large regime: HIP real-space Ewald matrix, "
                                    "device Cholesky), computed outside the timed steps",
                         "eeq_regime": model.select_regime(N, True),
                         "timing": ("HIP graph replay of the step" if graph else "eager step"),
                         "eager_ms_per_step": round(eager_ms, 4),
                         "graph_replay_matches_eager": graph_checked,
                         "energy_with_eeq_ms": round(eeq_ms, 2),
                         "charge_abs_max": float(q.abs().max()),
                         "energy_eV": float(e[0]),
                         "kernel_mean_us": {k: round(v, 2) for k, v in kernel_us.items()}},
              "roofline": roofline}
    if cpu:
        alpha = out["dynamic_polarizabilities"].detach().cpu().numpy()
        result["cpu_baseline"] = cpu_baseline_d4(s, tables, alpha, model)
    return result


def cpu_baseline_d3(s, tables, w: np.ndarray, model, k: int = 200,
                    min_seconds: float = 10.0) -> dict:
    """The oracle's two-body D3 (BJ, PyTorch on the CPU, float64) with its position
    gradient over the pair images of the first ``k`` receivers (enumeration and C6 from the
    reference weights included), repeated until about ``min_seconds``; weights given."""
    import oracle.d3 as D3
    pos, cell = np.asarray(s.pos, dtype=np.float64), np.asarray(s.cell, dtype=np.float64)
    sp = D3.species_of(tables, s.numbers)
    w_t = torch.as_tensor(w)
    prm = dict(D3.PBE0_D3BJ)
    cut_aa = model.cutoff_pair
    reps, dt, n_terms = 0, 0.0, 0
    t0 = time.perf_counter()
    while reps < 30 and (reps == 0 or dt < min_seconds):
        dst, src, sh = _d4_sample_pairs(pos, cell, k, cut_aa)
        pt = torch.tensor(pos, requires_grad=True)
        v = D3.edge_vectors_au(pt, torch.as_tensor(cell), dst, src, sh)
        r = torch.linalg.norm(v, dim=-1)
        c6 = D3.pair_c6(sp, w_t, torch.as_tensor(dst), torch.as_tensor(src), tables)
        e2 = D3.two_body(sp, dst, src, r, c6, tables, prm, "bj", cut_aa / D3.BOHR, 0.0,
                         len(pos))
        (g,) = torch.autograd.grad(e2.sum(), [pt])
        n_terms = len(dst)
        reps += 1
        dt = time.perf_counter() - t0
    return {"value": reps * n_terms / dt, "unit": "terms/s", "cores": torch.get_num_threads(),
            "kind": "port", "seconds": round(dt, 2), "steps": reps,
            "sample": f"{reps} x the BJ two-body energy + position gradient over the {n_terms} "
                      f"pair-image terms of the first {k} of {len(pos)} receivers (pair "
                      f"enumeration and C6 included; reference weights given), oracle "
                      f"PyTorch-CPU float64, torch threads={torch.get_num_threads()}"}


# D3 (BJ) algorithmic float64 flops per launch: per pair-image term as D4 (60 energy, +35
# for the backward); per atom pair C6 = W_i . C6ref . W_j (56 FMA = 112) and, backward,
# both atoms' dC6/dW (2 x 112)
D3_FLOPS = {"xnn_d3_two_body": lambda M, P: 60 * M + 112 * P,
            "xnn_d3_two_body_backward": lambda M, P: 95 * M + 336 * P}


def bench_d3(steps: int, warmup: int, cpu: bool = True) -> dict:
    """D3(BJ) two-body energy + forces + stress of the same 5,000-atom organic box
    (upstream cutoffs 60 / 40 bohr): CN kernel, reference weights, pair kernel and both
    backward kernels per step (row 17 of the path; the survey's configs time D4)."""
    import xnn_amd.dispersion as XD
    from xnn_amd import _lib, synthetic
    dev = torch.device("cuda:0")
    s = synthetic.organic_box(seed=0)
    tables = XD.load_d3_tables(os.path.join(ROOT, "tests", "golden", "d3_tables_hcnoar.npz"))
    model = XD.DFTD3(tables).to(dev)
    z = torch.tensor(s.numbers, device=dev)
    pos0 = torch.tensor(s.pos, dtype=torch.float64, device=dev)
    cell0 = torch.tensor(s.cell, dtype=torch.float64, device=dev)[None]
    pbc = torch.ones((1, 3), dtype=torch.bool)
    n_atoms = torch.tensor([len(s.numbers)])

    def step():
        pos = pos0.clone().requires_grad_(True)
        cell = cell0.clone().requires_grad_(True)
        out = model.evaluate(z, pos, cell, pbc, n_atoms, fused_pair=True)
        gp, gc = torch.autograd.grad(out["energy"].sum(), [pos, cell])
        return out, gp, gc

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        out, gp, gc = step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / steps * 1e3
    kernels = list(D3_FLOPS) + ["xnn_d3_coordination", "xnn_d3_coordination_backward"]
    _lib.timed.clear()
    _lib.time_launches(*kernels)
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    kernel_us = {k: float(np.mean([a.elapsed_time(b) * 1e3 for a, b in v]))
                 for k, v in _lib.timed.items() if v}
    _lib.timed.clear()
    imgs = XD.image_counts(cell0, pbc, model.cutoff_pair)[0].tolist()
    n_terms = 0
    with torch.no_grad():
        d0 = pos0[:, None, :] - pos0[None, :, :]
        rc2 = model.cutoff_pair ** 2
        for a in range(-imgs[0], imgs[0] + 1):
            for b in range(-imgs[1], imgs[1] + 1):
                for c in range(-imgs[2], imgs[2] + 1):
                    t = a * cell0[0, 0] + b * cell0[0, 1] + c * cell0[0, 2]
                    r2 = ((d0 + t) ** 2).sum(-1)
                    n_terms += int(((r2 <= rc2) & (r2 > 0)).sum())
        del d0
    N = len(s.numbers)
    dominant = max(kernel_us, key=lambda k: kernel_us[k])
    flops = D3_FLOPS[dominant](n_terms, N * (N + 1) // 2) if dominant in D3_FLOPS else None
    achieved = flops / (kernel_us[dominant] * 1e-6) / 1e12 if flops else None
    result = {"metric": "D3(BJ) pair-image terms/s, energy+forces+stress, 5000-atom organic box",
              "value": n_terms / (ms * 1e-3), "unit": "terms/s", "n_gpus": 1, "steps": steps,
              "warmup": warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
              "vs_baseline": None, "dtype": "f64", "data": "synthetic (seeded generator)",
              "config": {"workload": "d3bj_organic_box_5000_atoms", "atoms": N,
                         "pair_image_terms": n_terms, "cutoff_pair_bohr": 60.0,
                         "cutoff_cn_bohr": 40.0, "energy_eV": float(out["energy"].detach()[0]),
                         "kernel_mean_us": {k: round(v, 2) for k, v in kernel_us.items()}},
              "roofline": {"bound": "fp64", "kernel": dominant,
                           "achieved": None if achieved is None else round(achieved, 2),
                           "peak": FP64_PEAK_TFLOPS, "unit": "TFLOP/s",
                           "frac": None if achieved is None else round(achieved / FP64_PEAK_TFLOPS, 4),
                           "traffic": None, "algorithmic_flops": flops,
                           "mean_launch_us": round(kernel_us[dominant], 2),
                           "timing": "eager step, HIP events on the launch stream"}}
    if cpu:
        result["cpu_baseline"] = cpu_baseline_d3(s, tables, out["weights"].detach().cpu().numpy(),
                                                 model)
    return result


# ATM float64 flops (FMA = 2, division = square root = exp = log = 1) per edge pair tested
# by the distinct-triangle walk (third side: 3 differences + squared norm = 8) and per kept
# triangle: forward 82 more (C6_jk over the 23 frequencies 46, damping radius 2, 1/r^3 and
# powers 6, (R0/r^3)^alp3 4, damping 3, angular factor 11, C9 3, energy 5, sum 1, switch
# off); backward 235 (forward + the three squared-side derivatives 55, vector and C6
# gradients of both edges 16, factor gradients of both atoms 2 x 46 + the slot products)
ATM_FLOPS = {"xnn_atm_energy": lambda P, M: 8 * P + 82 * M,
             "xnn_atm_energy_backward": lambda P, M: 8 * P + 235 * M}


def cpu_baseline_atm(ei: np.ndarray, vec: np.ndarray, feat: np.ndarray, species: np.ndarray,
                     table: np.ndarray, consts, n_atoms: int, centers: int = 2,
                     min_seconds: float = 10.0) -> dict:
    """The oracle's ATM (every corner visited, PyTorch on the CPU, float64) with its
    gradients in the edge vectors and the C6 factors, over the triangles at the first
    ``centers`` atoms (all pairs of their edges), repeated until about ``min_seconds``."""
    import oracle.d4 as D
    sel = np.isin(ei[1], np.arange(centers))
    e_t = torch.as_tensor(ei[:, sel])
    v_t = torch.as_tensor(vec[sel])
    f_t = torch.as_tensor(feat)
    sp, tab = torch.as_tensor(species).long(), torch.as_tensor(table)
    counts = np.bincount(ei[1][sel], minlength=centers)[:centers]
    visits = int(sum(int(m) * (int(m) - 1) // 2 for m in counts))
    reps, dt = 0, 0.0
    t0 = time.perf_counter()
    while reps < 20 and (reps == 0 or dt < min_seconds):
        v = v_t.clone().requires_grad_(True)
        f = f_t.clone().requires_grad_(True)
        e = D.atm_edges(e_t, v, f, f, sp, tab, consts.s9, consts.alp3, consts.cutoff,
                        consts.width, n_atoms)
        torch.autograd.grad(e.sum(), [v, f])
        reps += 1
        dt = time.perf_counter() - t0
    return {"value": reps * visits / dt, "unit": "triangle visits/s",
            "cores": torch.get_num_threads(), "kind": "port", "seconds": round(dt, 2),
            "steps": reps,
            "sample": f"{reps} x the ATM energy + gradients (edge vectors, C6 factors) of the "
                      f"{visits} edge pairs at the first {centers} of {n_atoms} centers "
                      f"(every corner visited, third side tested), oracle PyTorch-CPU "
                      f"float64, torch threads={torch.get_num_threads()}"}


def bench_atm(steps: int, warmup: int, cpu: bool = True) -> dict:
    """D4 ATM three-body energy + gradients on the 5,000-atom organic box (36.8 A cell) at
    the upstream three-body cutoff (40 bohr, sharp): the triplet plan, the energy kernels
    and the backward per step, with the edge list (HIP radius graph at 40 bohr), its
    vectors and the neutral-atom C6 factors resident in HBM (the graph is timed apart)."""
    import xnn_amd.dispersion as XD
    from xnn_amd import _lib, synthetic
    dev = torch.device("cuda:0")
    s = synthetic.organic_box(seed=0)
    tables = XD.load_d4_tables(os.path.join(ROOT, "tests", "golden", "d4_tables_hcnoar.npz"))
    model = XD.DFTD4(tables).to(dev)
    z = torch.tensor(s.numbers, device=dev)
    pos = torch.tensor(s.pos, dtype=torch.float64, device=dev)
    cell = torch.tensor(s.cell, dtype=torch.float64, device=dev)[None]
    pbc = torch.ones((1, 3), dtype=torch.bool)
    N = len(s.numbers)
    with torch.no_grad():
        out = model.evaluate(z, pos, cell, pbc, torch.tensor([N]),
                             charges=torch.zeros(N, dtype=torch.float64, device=dev))
        cn = out["coordination_numbers"]
        uniq, species = torch.unique(z, return_inverse=True)
        alpha0 = model.polarizabilities(z, cn, torch.zeros_like(cn))
        feat = (alpha0 * torch.sqrt((3.0 / math.pi) * XD.cp_weights(alpha0))).contiguous()
        q4 = model.r4r2[uniq]
        table = model.a1 * torch.sqrt(3.0 * q4[:, None] * q4[None, :]) + model.a2
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ei, vec = XD.triple_graph(pos, cell, pbc, [N], model.cutoff_triple)
    torch.cuda.synchronize()
    graph_ms = (time.perf_counter() - t0) * 1e3
    vec = vec.contiguous()
    consts = XD.ATMConstants(species.to(torch.int32), table, model.s9, model.alp / 3.0,
                             model.cutoff_triple / XD.BOHR, model.switch_width_triple / XD.BOHR)

    node_ptr = torch.tensor([0, N], dtype=torch.int64, device=dev)
    batch32 = torch.zeros(N, dtype=torch.int32, device=dev)

    def step():
        # energies and gradients from one launch of the backward kernels at unit seeds
        v = vec.detach().requires_grad_(True)
        f = feat.detach().requires_grad_(True)
        e, _ = XD.atm_structure_energy(ei, v, f, f, consts, node_ptr, batch32)
        gv, gf = torch.autograd.grad(e.sum(), [v, f])
        return e, gv, gf

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        e, gv, gf = step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / steps * 1e3
    kernels = ["xnn_atm_plan", "xnn_atm_energy", "xnn_atm_energy_backward"]
    _lib.timed.clear()
    _lib.time_launches(*kernels)
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    kernel_us = {k: float(np.mean([a.elapsed_time(b) * 1e3 for a, b in v]))
                 for k, v in _lib.timed.items() if v}
    _lib.timed.clear()

    # one second-derivative step (a force-training loss through the ATM term): the
    # energies, their gradient with a graph, and the gradient of <gradient, direction>
    # (the Hessian-vector product of xnn_atm_energy_backward_tangent)
    u_vec, u_feat = torch.randn_like(vec), torch.randn_like(feat)

    def second_step():
        v = vec.detach().requires_grad_(True)
        f = feat.detach().requires_grad_(True)
        e3 = XD.atm_energy(ei, v, f, f, consts, N)
        gv, gf = torch.autograd.grad(e3.sum(), [v, f], create_graph=True)
        return torch.autograd.grad((gv * u_vec).sum() + (gf * u_feat).sum(), [v, f])

    second_step()
    torch.cuda.synchronize()
    _lib.time_launches("xnn_atm_energy_backward_tangent")
    t0 = time.perf_counter()
    second_step()
    torch.cuda.synchronize()
    second_ms = (time.perf_counter() - t0) * 1e3
    tangent_us = float(np.mean([a.elapsed_time(b) * 1e3
                                for a, b in _lib.timed["xnn_atm_energy_backward_tangent"]]))
    _lib.timed.clear()
    plan, info = XD.atm_plan(ei, N)
    counts = (ctypes_i64 * 3)()
    _lib.call("xnn_atm_count", _lib.ptr(plan), int(ei.shape[1]), N, info[0], _lib.ptr(vec),
              consts.cutoff, counts, _lib.stream(dev))
    tested, kept, repeated = int(counts[0]), int(counts[1]), int(counts[2])
    triangles = kept + repeated
    dominant = max((k for k in ATM_FLOPS if k in kernel_us), key=lambda k: kernel_us[k])
    flops = ATM_FLOPS[dominant](tested, triangles)
    achieved = flops / (kernel_us[dominant] * 1e-6) / 1e12
    roofline = {"bound": "fp64", "kernel": dominant, "achieved": round(achieved, 2),
                "peak": FP64_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / FP64_PEAK_TFLOPS, 4), "traffic": None,
                "algorithmic_flops": flops, "mean_launch_us": round(kernel_us[dominant], 2),
                "timing": "eager step, HIP events around the entry point on the launch stream"}
    result = {"metric": "D4 ATM triangles/s, energy+gradients, 5000-atom organic box",
              "value": triangles / (ms * 1e-3), "unit": "triangles/s", "n_gpus": 1,
              "steps": steps, "warmup": warmup, "ms_per_step": ms, "higher_is_better": True,
              "scaling": "weak", "vs_baseline": None, "dtype": "f64",
              "data": "synthetic (seeded generator)",
              "config": {"workload": "d4_atm_organic_box_5000_atoms", "atoms": N,
                         "edges": int(ei.shape[1]), "cutoff_triple_bohr": 40.0,
                         "edge_pairs_tested": tested, "distinct_triangles": kept,
                         "repeated_atom_visits": repeated, "graph_ms": round(graph_ms, 2),
                         "energy_3body_hartree": float(e.sum()),
                         "kernel_mean_us": {k: round(v, 2) for k, v in kernel_us.items()},
                         "second_derivative_step_ms": round(second_ms, 2),
                         "tangent_kernel_us": round(tangent_us, 2)},
              "roofline": roofline}
    if cpu:
        result["cpu_baseline"] = cpu_baseline_atm(
            ei.cpu().numpy(), vec.cpu().numpy(), feat.cpu().numpy(),
            species.cpu().numpy(), table.cpu().numpy(), consts, N)
    return result


def bench_nl(steps: int, warmup: int, cpu: bool = True) -> dict:
    """The default workload's neighbor list alone (``--config nl``): the water box's radius
    graph rebuilt with ``build_neighbor_list`` at an unchanged cell (its grid plan kept,
    outputs sized from the plan's last list, one status read per build), ``warmup``
    untimed builds then ``steps`` timed ones; roofline on 12 N + 40 E bytes (positions read,
    int64 edge index and shifts written) per build."""
    import xnn_amd as xa
    from xnn_amd import synthetic
    dev = torch.device("cuda:0")
    s = synthetic.water_box(seed=0)
    rc = 5.0
    pos = torch.tensor(s.pos, dtype=torch.float32, device=dev)
    cell = torch.tensor(s.cell, dtype=torch.float32, device=dev)
    pbc = torch.tensor(s.pbc)
    for _ in range(max(warmup, 2)):
        ei, sh = xa.build_neighbor_list(pos, rc, cell, pbc)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        ei, sh = xa.build_neighbor_list(pos, rc, cell, pbc)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / steps * 1e3
    N, E = len(s.pos), int(ei.shape[1])
    nbytes = 12 * N + 40 * E
    result = {"metric": "neighbor-list edges/s, 9k-atom water box, 5 A cutoff, 1 MI355X",
              "value": E / (ms * 1e-3), "unit": "edges/s", "n_gpus": 1, "steps": steps,
              "warmup": warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
              "vs_baseline": None, "dtype": "f32", "data": "synthetic (seeded generator)",
              "config": {"workload": "water_box_9000_atoms_rc5_neighbor_list", "atoms": N,
                         "edges": E, "cutoff": rc, "periodic": True},
              "roofline": {"bound": "hbm", "achieved": round(nbytes / (ms * 1e-3) / 1e9, 1),
                           "peak": HBM_PEAK_GBS, "unit": "GB/s",
                           "frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                           "traffic": None, "algorithmic_bytes": nbytes,
                           "timing": "wall clock over the builds (five dependent launches "
                                     "and one status read each)"}}
    if cpu:
        import oracle.nl as ON
        t0 = time.perf_counter()
        eo, _, _ = ON.neighbor_list(s.pos, rc, s.cell, s.pbc, dtype=np.float32)
        dt = time.perf_counter() - t0
        assert eo.shape[1] == E
        result["cpu_baseline"] = {"value": E / dt, "unit": "edges/s", "cores": 1,
                                  "kind": "port", "sample": "the whole list once: the "
                                  "oracle's brute force over the image range, float32"}
    return result


def bench_eeq_cg(steps: int, warmup: int) -> dict:
    """Large-regime EEQ in its conjugate-gradient regime (``--config eeq_cg``): a
    24,000-atom organic box (the C5 density), D4's EEQ widths, hardness and
    electronegativities by element, a seeded CN in [0, 4], the 60-bohr real-space range.
    Builds ``IterativeEEQSystem``, times ``steps`` two-column operator products after
    ``warmup``, then one ``solve_augmented`` (the charge and the constraint right-hand sides
    in lockstep). ``value`` is the solve's wall time."""
    import oracle.d4 as D
    from xnn_amd import eeq as XE, synthetic
    dev = torch.device("cuda:0")
    tables = dict(np.load(os.path.join(ROOT, "tests", "golden", "d4_tables_hcnoar.npz"),
                          allow_pickle=False))
    n = 24000
    s = synthetic.organic_box(n, box=36.8 * (n / 5000) ** (1 / 3), seed=1)
    z = np.asarray([int(v) for v in s.numbers])
    cn = np.random.default_rng(7).uniform(0, 4, n)
    rad = torch.tensor(tables["eeq_rad"][z], device=dev)
    x = torch.tensor(-tables["eeq_chi"][z] + tables["eeq_kcnchi"][z] * cn / np.sqrt(cn + 1e-14),
                     device=dev)
    diag = torch.tensor(tables["eeq_eta"][z], device=dev) + math.sqrt(2 / math.pi) / rad
    p = torch.tensor(s.pos / D.BOHR, device=dev)
    c = torch.tensor(s.cell / D.BOHR, device=dev)
    alpha = XE.ewald_alpha(60.0)
    system = XE.IterativeEEQSystem(p, c, rad, diag - 2 * alpha / math.sqrt(math.pi), alpha, 60.0)
    v = torch.randn(n, 2, dtype=torch.float64, device=dev,
                    generator=torch.Generator(device=dev).manual_seed(0))
    for _ in range(warmup):
        system._matvec(v)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        system._matvec(v)
    torch.cuda.synchronize()
    matvec_ms = (time.perf_counter() - t0) / steps * 1e3
    t0 = time.perf_counter()
    system.solve_augmented(x, torch.zeros((), dtype=torch.float64, device=dev))
    torch.cuda.synchronize()
    solve_s = time.perf_counter() - t0
    return {"metric": "EEQ conjugate-gradient solve, 24000-atom organic box, 1 MI355X",
            "value": solve_s, "unit": "s", "n_gpus": 1, "steps": steps, "warmup": warmup,
            "ms_per_step": matvec_ms, "higher_is_better": False, "scaling": "weak",
            "vs_baseline": None, "dtype": "f64", "data": "synthetic (seeded generator)",
            "config": {"workload": "eeq_cg_organic_box_24000_atoms", "atoms": n,
                       "real_space_cutoff_bohr": 60.0, "iterations": system.iterations,
                       "two_column_product_ms": round(matvec_ms, 3)}}


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="water",
                    choices=["water", "argon", "ragged", "d4", "d3", "atm", "nl", "eeq_cg"])
    ap.add_argument("--graph", action=argparse.BooleanOptionalAction, default=True,
                    help="time replays of the step captured as one HIP graph")
    ap.add_argument("--cpu-edges", type=int, default=480_000,
                    help="edges of the CPU-baseline sample (0 skips it)")
    ap.add_argument("--fused", action=argparse.BooleanOptionalAction, default=True,
                    help="radial linear layer inside the message kernels (ShEdgePotential "
                         "fused_linear)")
    ap.add_argument("--fused-radial", action=argparse.BooleanOptionalAction, default=True,
                    help="radial basis evaluated inside the message kernels (ShEdgePotential "
                         "fused_radial)")
    ap.add_argument("--variant", default="rows", choices=["rows", "readout", "one_pass"],
                    help="rows (the metric's pipeline): the message kernels write the (N, C, 16) "
                         "rows and the readout is its own op, whose backward hands back a "
                         "general cotangent; readout: the message kernels apply the readout "
                         "(no rows in memory); one_pass: energies and forces from one backward "
                         "launch of the readout kernels")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run the 256 MiB copy that calibrates the HBM byte counters")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(collectives and sharding are out of scope); run with --gpus 1", file=sys.stderr)
        raise SystemExit(2)
    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a GPU")
    if args.copy_calibration:
        copy_calibration()
        return
    if args.config == "d4":
        print(json.dumps(bench_d4(args.steps, args.warmup, cpu=args.cpu_edges > 0,
                                  graph=args.graph)), flush=True)
        return
    if args.config == "d3":
        print(json.dumps(bench_d3(args.steps, args.warmup, cpu=args.cpu_edges > 0)), flush=True)
        return
    if args.config == "atm":
        print(json.dumps(bench_atm(args.steps, args.warmup, cpu=args.cpu_edges > 0)), flush=True)
        return
    if args.config == "nl":
        print(json.dumps(bench_nl(args.steps, args.warmup, cpu=args.cpu_edges > 0)), flush=True)
        return
    if args.config == "eeq_cg":
        print(json.dumps(bench_eeq_cg(args.steps, args.warmup)), flush=True)
        return
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    from xnn_amd import _lib
    import xnn_amd as xa
    _lib.load()

    g, model, rc, kw, workload, nl_ms, structs = build_workload(args.config, device)
    model.fused_linear = bool(args.fused)
    model.fused_radial = bool(args.fused_radial)
    model.fused_readout = args.variant in ("readout", "one_pass")
    model.one_pass = args.variant == "one_pass"
    E, N = g.num_edges, g.num_nodes
    C, L = kw["channels"], (kw["l_max"] + 1) ** 2
    wrapped = xa.ForceStressOutput(model, compute_stress=g.cell is not None).eval()
    g.plan()                                    # edge plan: once per neighbor list

    def step():
        data = copy.copy(g)                     # ForceStressOutput rebinds pos / cell
        return wrapped(data)

    _lib.calls.clear()
    for _ in range(args.warmup):
        out = step()
    # the message entry point the step took (radial basis in the kernel, linear layer in
    # the kernel, or the linear layer in PyTorch)
    # (or, one pass: energies and forces from the readout backward alone)
    msg = next(m for m in ("xnn_sh_radial_message_energy_forces",
                           "xnn_sh_radial_message_energy", "xnn_sh_radial_message_sum",
                           "xnn_sh_linear_message_sum", "xnn_sh_message_sum")
               if _lib.calls.get(m))
    fused = msg != "xnn_sh_message_sum"
    kernels = ([msg] if msg.endswith("_forces") else [msg, msg + "_backward"]) + \
        ["xnn_edge_featurize", "xnn_edge_featurize_backward", "xnn_edge_force_reduce",
         "xnn_edge_force_reduce_virial", "xnn_node_readout", "xnn_node_readout_backward"]
    # eager pass: per-kernel HIP events on the launch stream
    _lib.timed.clear()
    _lib.time_launches(*kernels)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        out = step()
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t0) / args.steps * 1e3
    eager_forces = out["forces"].clone()
    timed = {k: list(v) for k, v in _lib.timed.items()}
    _lib.timed.clear()
    assert torch.isfinite(out["forces"]).all()

    ms = eager_ms
    graph_checked = None
    if args.graph:
        # the whole step (forward, forces and stress backward) as one HIP graph
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(3):
                step()
        torch.cuda.current_stream().wait_stream(side)
        hip_graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(hip_graph):
            static_out = step()
        for _ in range(max(1, args.warmup)):
            hip_graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            hip_graph.replay()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) / args.steps * 1e3
        # every replay must reproduce the eager forces bit for bit
        graph_checked = bool(torch.equal(static_out["forces"], eager_forces))
        eager_check = step()["forces"]
        hip_graph.replay()
        torch.cuda.synchronize()
        graph_checked = graph_checked and bool(torch.equal(static_out["forces"], eager_check))
        if not graph_checked:
            raise SystemExit("graph replay differs from the eager step")

    per_kernel, total_us = {}, {}
    for name in kernels:
        ev = timed.get(name, [])
        if ev:
            d = [s.elapsed_time(e) * 1e3 for s, e in ev]          # us
            per_kernel[name] = float(np.mean(d))
            total_us[name] = float(np.sum(d)) / args.steps       # per step, all launches
    _lib.timed.clear()
    kc = kernel_costs(E, N, C, L, kw["n_rbf"], grouped=g.plan().perm_dst is None)
    # the eager step's events also hold the host's launch gaps; the message kernels are
    # timed again back to back, the figure the roofline uses
    replay_us = {}
    for name, (call_args, _keep) in message_launches(msg, g, model, kw).items():
        replay_us[name] = replay_launch_us(name, call_args)
        total_us[name] = replay_us[name]
    # the dominant kernel among those with an algorithmic cost
    dominant = max((k for k in total_us if k in kc), key=lambda k: total_us[k])
    launch_us = replay_us.get(dominant, per_kernel.get(dominant))
    launch_s = launch_us * 1e-6
    cost = kc[dominant]
    # the bound is whichever resource the kernel's compulsory work needs longer on
    t_hbm = cost["bytes"] / (HBM_PEAK_GBS * 1e9)
    t_mfma = cost["flops"] / (MFMA_F32_PEAK_TFLOPS * 1e12)
    if t_mfma > t_hbm:
        achieved = cost["flops"] / launch_s / 1e12
        roofline = {"bound": "mfma", "kernel": dominant, "achieved": round(achieved, 2),
                    "peak": MFMA_F32_PEAK_TFLOPS, "unit": "TFLOP/s",
                    "frac": round(achieved / MFMA_F32_PEAK_TFLOPS, 4)}
    else:
        achieved = cost["bytes"] / launch_s / 1e9
        roofline = {"bound": "hbm", "kernel": dominant, "achieved": round(achieved, 1),
                    "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4)}
    roofline.update({"traffic": measured_traffic(dominant, workload),
                     "algorithmic_bytes": cost["bytes"], "algorithmic_flops": cost["flops"],
                     "hbm_GBs": round(cost["bytes"] / launch_s / 1e9, 1),
                     "mean_launch_us": round(launch_us, 2),
                     "timing": ("back-to-back launches, HIP events on the launch stream"
                                if dominant in replay_us else "eager step, HIP events")})
    sb = step_bytes(E, N, C, L, kw["n_rbf"], msg)
    copy_gbs = copy_bandwidth_gbs()
    step_gbs = sb / (ms * 1e-3) / 1e9
    result = {
        "metric": ("edges/s fwd+force-bwd and % HBM roofline, 9k-atom water box, 1 MI355X"
                   if args.config == "water" else f"edges/s fwd+force-bwd, {workload}, 1 MI355X"),
        "value": E / (ms * 1e-3), "unit": "edges/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic (seeded generator, random-init weights)",
        "config": {"workload": workload, "atoms": N, "edges": E, "channels": C, "sh_components": L,
                   "n_rbf": kw["n_rbf"], "cutoff": rc, "stress": g.cell is not None,
                   "variant": args.variant,
                   "neighbor_list_ms": round(nl_ms, 3),
                   # the neighbor list's algorithmic bytes (positions in, the int64 edge
                   # index and shifts out: 12 N + 40 E) over its wall time per build
                   "neighbor_list_roofline": {
                       "bytes": 12 * N + 40 * E,
                       "GBs": round((12 * N + 40 * E) / (nl_ms * 1e-3) / 1e9, 1),
                       "frac": round((12 * N + 40 * E) / (nl_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
                   "hip_graph": bool(args.graph), "eager_ms_per_step": round(eager_ms, 4),
                   "graph_replay_matches_eager": graph_checked,
                   "fused_linear": fused, "message_kernel": msg,
                   # the metric's "% HBM roofline": the fused step's compulsory bytes
                   # over its time, against the 8 TB/s peak
                   "step_algorithmic_bytes": sb,
                   "step_hbm_fraction": round(step_gbs / HBM_PEAK_GBS, 4),
                   "step_GBs": round(step_gbs, 1),
                   # a plain 1 GiB device copy on the same GPU: the attainable rate
                   "copy_GBs": round(copy_gbs, 1),
                   "step_fraction_of_copy": round(step_gbs / copy_gbs, 4),
                   # an equivalent-bytes figure, not a traffic measurement: the bytes the
                   # unfused pipeline would move, E (124 + 12 C) + N (76 + 8 C 16), over
                   # the fused step's time
                   "unfused_pipeline_equivalent_bytes": pipeline_bytes(E, N, C),
                   "unfused_pipeline_equivalent_hbm_fraction": round(
                       pipeline_bytes(E, N, C) / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                   "kernel_mean_us": {k: round(v, 2) for k, v in replay_us.items()},
                   "eager_kernel_event_us": {k: round(v, 2) for k, v in per_kernel.items()}},
        "roofline": roofline,
    }
    if args.cpu_edges > 0:
        result["cpu_baseline"] = cpu_baseline(g, model, rc, kw, args.cpu_edges)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
