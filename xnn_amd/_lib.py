"""ctypes binding of the C ABI in ``include/xnn_amd.h`` (``libxnn_amd.so``).

The library is loaded once per process. Loading fails loudly: there is no
silent fallback to another implementation when the HIP library is missing.
"""
from __future__ import annotations

import ctypes
import os
import threading
from typing import Optional

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY = os.path.join(HERE, "libxnn_amd.so")
ABI_VERSION = 2

XNN_OK, XNN_EINVAL, XNN_ECAPACITY, XNN_EHIP = 0, 1, 2, 3
XNN_F32, XNN_F64 = 0, 1
BASIS = {"bessel": 0, "gaussian": 1}
ENVELOPE = {"polynomial": 0, "cosine": 1, "none": 2}

c_i32p = ctypes.POINTER(ctypes.c_int32)
c_i64p = ctypes.POINTER(ctypes.c_int64)
c_f64p = ctypes.POINTER(ctypes.c_double)
vp = ctypes.c_void_p
i64 = ctypes.c_int64
i32 = ctypes.c_int32
c_int = ctypes.c_int
dbl = ctypes.c_double
sz = ctypes.c_size_t


class FeaturizeParams(ctypes.Structure):
    """``xnn_featurize_params``."""
    _fields_ = [("n_rbf", i32), ("basis", i32), ("envelope", i32), ("poly_p", i32),
                ("l_max", i32), ("sh_sign", i32), ("cutoff", dbl), ("rbf_prefactor", dbl),
                ("gaussian_gamma", dbl)]


class GridPlan(ctypes.Structure):
    """``xnn_grid_plan``."""
    _fields_ = [("nbins", i32 * 3), ("reach", i32 * 3), ("periodic", i32 * 3), ("has_cell", i32),
                ("lo", dbl * 3), ("width", dbl * 3), ("inv_cell", dbl * 9), ("n_bins", i64),
                ("workspace_bytes", sz)]


class D4CnParams(ctypes.Structure):
    """``xnn_d4_cn_params``."""
    _fields_ = [("cutoff_cn", dbl), ("cutoff_eeq_cn", dbl), ("kcn", dbl), ("k4", dbl),
                ("k5", dbl), ("k6", dbl)]


class D4PairParams(ctypes.Structure):
    """``xnn_d4_pair_params``."""
    _fields_ = [("s6", dbl), ("s8", dbl), ("a1", dbl), ("a2", dbl), ("cutoff", dbl),
                ("width", dbl)]


class D4AlphaTables(ctypes.Structure):
    """``xnn_d4_alpha_tables`` (device pointers)."""
    _fields_ = [("n_elements", i32), ("nref", vp), ("ngw", vp), ("refcn", vp), ("refq", vp),
                ("zeff", vp), ("gi", vp), ("refalpha", vp), ("ga", dbl), ("wf", dbl)]


class D3PairParams(ctypes.Structure):
    """``xnn_d3_pair_params``."""
    _fields_ = [("s6", dbl), ("s8", dbl), ("a1", dbl), ("a2", dbl), ("rs6", dbl), ("rs8", dbl),
                ("alp", dbl), ("bet", dbl), ("cutoff", dbl), ("width", dbl), ("damping", i32)]


class AtmParams(ctypes.Structure):
    """``xnn_atm_params``."""
    _fields_ = [("s9", dbl), ("alp3", dbl), ("cutoff", dbl), ("width", dbl)]


class UvuPath(ctypes.Structure):
    """``xnn_uvu_path``."""
    _fields_ = [("l1", i32), ("l2", i32), ("l3", i32), ("mul", i32), ("off1", i32), ("off2", i32),
                ("off_out", i32), ("off_w", i32), ("block", i32), ("coef", ctypes.c_float)]


def uvu_paths(ints, coefs):
    """A ctypes array of ``xnn_uvu_path`` from 9 ints per path and the coefficients."""
    n = len(coefs)
    arr = (UvuPath * n)()
    for p in range(n):
        arr[p] = UvuPath(*ints[9 * p:9 * p + 9], float(coefs[p]))
    return arr


class ShPairModel(ctypes.Structure):
    """``xnn_sh_pair_model``."""
    _fields_ = [("prm", ctypes.POINTER(FeaturizeParams)), ("rbf_table", vp), ("n_channels", i32),
                ("W", vp), ("U", vp), ("atom_ref", vp), ("n_atom_ref", i64)]


# name -> argtypes (restype int unless listed in _RESTYPES)
_SIGNATURES = {
    "xnn_last_error": [],
    "xnn_abi_version": [],
    "xnn_edge_featurize": [c_int, c_int, vp, vp, i64, vp, i64, vp, vp, vp, vp, i64,
                           ctypes.POINTER(FeaturizeParams), vp, vp, vp, vp, vp, vp],
    "xnn_edge_featurize_backward": [c_int, c_int, vp, vp, i64, vp, i64, vp, vp, vp, vp, i64,
                                    ctypes.POINTER(FeaturizeParams), vp, vp, vp, vp, vp, vp, vp,
                                    vp],
    "xnn_edge_force_reduce": [c_int, c_int, vp, i64, vp, vp, vp, vp, vp, vp, i64, vp, vp, vp, vp,
                              vp],
    "xnn_edge_force_reduce_virial_workspace_bytes": [i64, i64],
    "xnn_energy_stress_max_nodes": [],
    "xnn_energy_stress_finish": [c_int, vp, i64, c_int, vp, c_int, vp, vp, dbl, vp, vp, vp],
    "xnn_edge_force_reduce_virial": [c_int, c_int, vp, i64, vp, vp, vp, vp, vp, i64, vp, vp, c_int,
                                     vp, vp, sz, vp],
    "xnn_sh_message_sum": [c_int, vp, vp, i64, vp, i64, vp, vp, vp, i64, vp, vp, i32, i32, i32,
                           vp, vp, vp],
    "xnn_sh_message_sum_backward": [c_int, vp, vp, i64, vp, i64, vp, vp, vp, i64, vp, vp, i32,
                                    i32, i32, vp, vp, vp, vp, vp],
    "xnn_sh_linear_message_sum": [c_int, vp, vp, i64, vp, i64, vp, vp, vp, i64, vp, vp, i32, i32,
                                  i32, i32, vp, vp, vp, vp],
    "xnn_sh_linear_message_sum_backward": [c_int, vp, vp, i64, vp, i64, vp, vp, vp, i64, vp, vp,
                                           i32, i32, i32, i32, vp, vp, vp, vp, vp, vp],
    "xnn_sh_radial_message_sum": [c_int, vp, vp, i64, vp, i64, vp, vp, vp, i64, vp, vp,
                                  ctypes.POINTER(FeaturizeParams), vp, i32, vp, vp, vp],
    "xnn_sh_radial_message_sum_backward": [c_int, vp, vp, i64, vp, i64, vp, vp, vp, i64, vp, vp,
                                           ctypes.POINTER(FeaturizeParams), vp, i32, vp, vp, vp,
                                           vp],
    "xnn_sh_radial_message_energy": [c_int, vp, vp, i64, vp, i64, vp, vp, vp, i64, vp, vp,
                                     ctypes.POINTER(FeaturizeParams), vp, i32, vp, vp, vp, vp,
                                     i64, vp, vp],
    "xnn_sh_radial_message_energy_backward": [c_int, vp, vp, i64, vp, i64, vp, vp, vp, i64, vp,
                                              vp, ctypes.POINTER(FeaturizeParams), vp, i32, vp,
                                              vp, vp, i64, vp, vp],
    "xnn_sh_radial_message_energy_forces": [c_int, vp, vp, i64, vp, i64, vp, vp, vp, i64, vp,
                                            vp, ctypes.POINTER(FeaturizeParams), vp, i32, vp,
                                            vp, vp, i64, vp, vp, vp],
    "xnn_node_energy_from_edges": [vp, vp, vp, i64, vp, vp, i64, vp, vp],
    "xnn_radial_hidden": [vp, i64, c_int, c_int, vp, vp, vp, vp, vp],
    "xnn_radial_hidden_backward": [vp, vp, i64, c_int, c_int, vp, vp, vp, vp, vp],
    "xnn_uvu_conv": [vp, i64, i32, vp, i32, vp, i64, i32, vp, vp, i64, vp, vp, vp, i32, vp, i32,
                     vp],
    "xnn_uvu_conv_backward": [vp, i64, i32, vp, i32, vp, i64, i32, vp, vp, vp, i64, vp, vp, vp,
                              vp, vp, i32, vp, i32, vp, vp, vp, vp, sz, vp],
    "xnn_uvu_conv_workspace_bytes": [i64, i32, vp, i32],
    "xnn_sh_pair_workspace_bytes": [i64, i64],
    "xnn_sh_pair_energy_forces": [ctypes.POINTER(ShPairModel), c_int, vp, i64, vp, vp, vp, i64, vp,
                                  ctypes.POINTER(dbl), vp, vp, vp, vp, sz, vp],
    "xnn_stress_finish": [c_int, vp, c_int, vp, vp, i64, dbl, vp, vp],
    "xnn_virial_finish": [c_int, vp, vp, i64, i32, vp, vp],
    "xnn_virial_reduce_workspace_bytes": [i64, i64],
    "xnn_virial_reduce": [c_int, vp, i64, vp, i64, vp, i32, vp, vp, sz, vp],
    "xnn_d4_workspace_bytes": [i64, i64, i64],
    "xnn_d4_image_counts": [vp, vp, i64, dbl, vp, vp],
    "xnn_d4_plan_bytes": [i64, i64],
    "xnn_d4_plan": [vp, i64, vp, i64, vp, vp, vp, sz, vp],
    "xnn_d4_coordination": [vp, i64, vp, vp, vp, i64, i64, vp, vp, vp, vp, vp,
                            ctypes.POINTER(D4CnParams), vp, vp, vp, sz, vp],
    "xnn_d4_coordination_backward": [vp, i64, vp, vp, vp, i64, i64, vp, vp, vp, vp, vp,
                                     ctypes.POINTER(D4CnParams), vp, vp, vp, vp, vp, sz, vp],
    "xnn_d4_two_body": [vp, i64, vp, vp, vp, i64, i64, vp, vp, vp, vp, vp,
                        ctypes.POINTER(D4PairParams), vp, vp, sz, vp],
    "xnn_d3_weights": [i64, vp, vp, i32, vp, vp, dbl, vp, vp],
    "xnn_d3_weights_backward": [i64, vp, vp, i32, vp, vp, dbl, vp, vp, vp],
    "xnn_node_readout": [i32, vp, i64, i64, vp, vp, vp, i64, vp, vp],
    "xnn_atm_plan_size": [i64, i64, ctypes.POINTER(sz)],
    "xnn_atm_plan": [vp, i64, i64, vp, sz, ctypes.POINTER(i64), vp],
    "xnn_atm_work_size": [i64, i64, i32, i32, ctypes.POINTER(sz)],
    "xnn_atm_count": [vp, i64, i64, i64, vp, dbl, ctypes.POINTER(i64), vp],
    "xnn_atm_energy": [vp, i64, i64, i64, i64, vp, vp, vp, i32, vp, vp, i32,
                       ctypes.POINTER(AtmParams), vp, vp, sz, vp],
    "xnn_atm_energy_backward": [vp, i64, i64, i64, i64, vp, vp, vp, i32, vp, vp, i32,
                                ctypes.POINTER(AtmParams), vp, vp, vp, vp, vp, sz, vp],
    "xnn_atm_tangent_work_size": [i64, i64, i32, ctypes.POINTER(sz)],
    "xnn_atm_energy_backward_tangent": [vp, i64, i64, i64, i64, vp, vp, vp, i32, vp, vp, i32,
                                        ctypes.POINTER(AtmParams), vp, vp, vp, vp, vp, vp, vp,
                                        vp, vp, sz, vp],
    "xnn_node_readout_backward": [i32, vp, i64, i64, i64, vp, vp, vp],
    "xnn_d4_polarizabilities": [i64, vp, vp, vp, ctypes.POINTER(D4AlphaTables), vp, vp],
    "xnn_d4_polarizabilities_backward": [i64, vp, vp, vp, ctypes.POINTER(D4AlphaTables), vp, vp,
                                         vp, vp],
    "xnn_d4_two_body_backward": [vp, i64, vp, vp, vp, i64, i64, vp, vp, vp, vp, vp,
                                 ctypes.POINTER(D4PairParams), vp, vp, vp, vp, vp, sz, vp],
    "xnn_d3_coordination": [vp, i64, vp, vp, vp, i64, i64, vp, vp, vp, dbl, dbl, vp, vp, sz, vp],
    "xnn_d3_coordination_backward": [vp, i64, vp, vp, vp, i64, i64, vp, vp, vp, dbl, dbl, vp, vp,
                                     vp, vp, sz, vp],
    "xnn_d3_two_body": [vp, i64, vp, vp, vp, i64, i64, vp, vp, vp, vp, vp, i32, vp,
                        ctypes.POINTER(D3PairParams), vp, vp, sz, vp],
    "xnn_d3_two_body_backward": [vp, i64, vp, vp, vp, i64, i64, vp, vp, vp, vp, vp, i32, vp,
                                 ctypes.POINTER(D3PairParams), vp, vp, vp, vp, vp, sz, vp],
    "xnn_strain_apply": [c_int, vp, i64, vp, vp, i64, vp, vp, vp, vp],
    "xnn_strain_apply_backward": [c_int, vp, i64, vp, vp, i64, vp, vp, vp, vp, vp, vp, vp, vp],
    "xnn_segment_sum": [c_int, vp, i64, i64, vp, vp, i64, vp, vp],
    "xnn_gather_rows": [c_int, vp, i64, i64, vp, i64, vp, vp],
    "xnn_segment_reduce_workspace_bytes": [i64, i64, i64],
    "xnn_segment_reduce_f64": [c_int, vp, i64, i64, vp, i64, vp, vp, sz, vp],
    "xnn_segment_reduce_noalloc_max_bytes": [],
    "xnn_eeq_real_matrix": [vp, i64, vp, vp, dbl, dbl, vp, vp],
    "xnn_eeq_real_grad": [vp, i64, vp, vp, dbl, dbl, vp, vp, vp, vp, vp],
    "xnn_eeq_cholesky_block": [vp, i64, i64, i64, vp, vp, vp],
    "xnn_eeq_cholesky_solve": [vp, i64, vp, vp, i32, vp, vp],
    "xnn_eeq_real_apply_work_size": [i64, c_int, ctypes.POINTER(ctypes.c_size_t)],
    "xnn_eeq_real_apply": [vp, i64, vp, vp, dbl, dbl, vp, vp, c_int, vp, vp, ctypes.c_size_t, vp],
    "xnn_segment_reduce_f64_noalloc": [c_int, vp, i64, i64, vp, i64, vp, vp],
    "xnn_radius_graph_plan": [i64, c_f64p, c_i32p, dbl, c_f64p, c_f64p, ctypes.POINTER(GridPlan)],
    "xnn_radius_graph_bounds": [c_int, vp, i64, vp, vp, vp],
    "xnn_radius_graph_count": [c_int, vp, i64, vp, dbl, i32, ctypes.POINTER(GridPlan), vp, vp, vp],
    "xnn_radius_graph_status": [c_int, i64, ctypes.POINTER(GridPlan), vp, vp, vp, vp],
    "xnn_radius_graph_fill": [c_int, vp, i64, vp, dbl, i32, ctypes.POINTER(GridPlan), vp, vp, i64,
                              vp, vp, vp, vp, vp, vp, vp],
    "xnn_radius_graph_fill_capacity": [c_int, vp, i64, vp, dbl, i32, ctypes.POINTER(GridPlan), vp,
                                       vp, i64, vp, vp, vp, vp],
    "xnn_radius_graph_molecules_count": [c_int, vp, i64, vp, vp, i64, dbl, i32, vp, vp],
    "xnn_radius_graph_molecules_fill": [c_int, vp, i64, vp, vp, i64, dbl, i32, vp, i64, vp, vp,
                                        vp, vp, vp, vp],
    "xnn_nearest_edges_count": [vp, i64, i32, vp, vp],
    "xnn_nearest_edges_fill": [c_int, vp, i64, vp, vp, i64, i32, vp, vp, vp],
    "xnn_scan_workspace_bytes": [i64],
    "xnn_scan_counts": [vp, i64, vp, vp],
    "xnn_edge_plan_workspace_bytes": [i64, i64],
    "xnn_edge_plan": [vp, vp, i64, i64, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp],
}
_RESTYPES = {"xnn_last_error": ctypes.c_char_p, "xnn_scan_workspace_bytes": sz,
             "xnn_edge_plan_workspace_bytes": sz, "xnn_segment_reduce_workspace_bytes": sz,
             "xnn_d4_workspace_bytes": sz, "xnn_virial_reduce_workspace_bytes": sz,
             "xnn_d4_plan_bytes": sz, "xnn_edge_force_reduce_virial_workspace_bytes": sz,
             "xnn_energy_stress_max_nodes": i64,
             "xnn_segment_reduce_noalloc_max_bytes": sz, "xnn_uvu_conv_workspace_bytes": sz,
             "xnn_sh_pair_workspace_bytes": sz}

_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None


class XnnError(RuntimeError):
    """A call into the HIP library failed (bad argument, capacity or HIP error)."""

    def __init__(self, name: str, code: int, message: str):
        super().__init__(f"{name} failed ({['ok', 'invalid argument', 'capacity', 'HIP error'][code] if 0 <= code < 4 else code}): {message}")
        self.code = code


def load() -> ctypes.CDLL:
    """Load ``libxnn_amd.so`` (raises ``RuntimeError`` if it is not built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIBRARY):
            raise RuntimeError(
                f"{LIBRARY} is missing: build it with `python -m xnn_amd.build` "
                "(the HIP kernels have no fallback)")
        lib = ctypes.CDLL(LIBRARY)
        for name, args in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = _RESTYPES.get(name, ctypes.c_int)
        if lib.xnn_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIBRARY} has ABI {lib.xnn_abi_version()}, expected {ABI_VERSION}")
        _lib = lib
        return lib


def available() -> bool:
    """Whether the library file exists (does not load it)."""
    return os.path.exists(LIBRARY)


def exported_symbols() -> list[str]:
    """Names of the entry points this binding declares."""
    return list(_SIGNATURES)


def check(name: str, code: int) -> None:
    """Raise :class:`XnnError` for a non-zero status of ``name``."""
    if code != XNN_OK:
        msg = load().xnn_last_error()
        raise XnnError(name, code, msg.decode() if msg else "")


#: entry point name -> list of (start, end) HIP events recorded around each launch,
#: for the names a profiler asked for (see :func:`time_launches`)
timed: dict = {}


def time_launches(*names: str) -> None:
    """Record HIP events around every later launch of ``names`` on the launch stream."""
    for n in names:
        timed.setdefault(n, [])


def call(name: str, *args) -> None:
    """Call entry point ``name`` and raise on a non-zero status."""
    count_call(name)
    fn = getattr(load(), name)
    events = timed.get(name)
    if events is None:
        check(name, fn(*args))
        return
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    code = fn(*args)
    end.record()
    events.append((start, end))
    check(name, code)


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    """Device pointer of a tensor (``None`` -> NULL)."""
    if t is None:
        return None
    return t.data_ptr()


def stream(device: torch.device) -> int:
    """The current HIP stream of ``device`` as an integer handle."""
    return torch.cuda.current_stream(device).cuda_stream


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float32:
        return XNN_F32
    if dtype == torch.float64:
        return XNN_F64
    raise TypeError(f"unsupported dtype {dtype} (float32 or float64)")


calls: dict = {}


def count_call(name: str) -> None:
    """Record that a HIP entry point ran (tests assert the native path was taken)."""
    calls[name] = calls.get(name, 0) + 1


def virial_reduce(partial: torch.Tensor, n_rows: int, seg_ptr: torch.Tensor, n_graphs: int,
                  term: Optional[torch.Tensor], symmetrize: bool,
                  dtype: torch.dtype) -> torch.Tensor:
    """``xnn_virial_reduce``: (B, 3, 3) in ``dtype`` from float64 per-atom partials."""
    out = torch.empty((n_graphs, 3, 3), dtype=dtype, device=partial.device)
    need = int(load().xnn_virial_reduce_workspace_bytes(n_rows, n_graphs))
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=partial.device)
    call("xnn_virial_reduce", dtype_code(dtype), ptr(partial), n_rows, ptr(seg_ptr), n_graphs,
         ptr(term), 1 if symmetrize else 0, ptr(out), ptr(ws), need, stream(partial.device))
    return out


def segment_reduce_f64(src: torch.Tensor, n_rows: int, n_features: int, seg_ptr: torch.Tensor,
                       n_segments: int, out: torch.Tensor) -> None:
    """``xnn_segment_reduce_f64`` with its workspace from the caching allocator."""
    need = int(load().xnn_segment_reduce_workspace_bytes(n_rows, n_features, n_segments))
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=out.device) if need else None
    call("xnn_segment_reduce_f64", dtype_code(src.dtype), ptr(src), n_rows, n_features,
         ptr(seg_ptr), n_segments, ptr(out), ptr(ws), need, stream(out.device))


def radial_hidden(x: torch.Tensor, weights, scales, out: torch.Tensor,
                  grad_out: Optional[torch.Tensor] = None) -> None:
    """``xnn_radial_hidden`` (or its backward when ``grad_out`` is given) with the host
    arrays of widths, weight pointers and scales built here."""
    n = len(weights)
    widths = (ctypes.c_int32 * n)(*[int(w.shape[1]) for w in weights])
    wptrs = (ctypes.c_void_p * n)(*[w.data_ptr() for w in weights])
    sc = (ctypes.c_float * n)(*[float(c) for c in scales])
    rows, n_in = int(x.shape[0]), int(x.shape[1])
    if grad_out is None:
        call("xnn_radial_hidden", ptr(x), rows, n_in, n, ctypes.addressof(widths),
             ctypes.addressof(wptrs), ctypes.addressof(sc), ptr(out), stream(x.device))
    else:
        call("xnn_radial_hidden_backward", ptr(x), ptr(grad_out), rows, n_in, n,
             ctypes.addressof(widths), ctypes.addressof(wptrs), ctypes.addressof(sc), ptr(out),
             stream(x.device))
