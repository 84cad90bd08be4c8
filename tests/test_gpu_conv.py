"""GPU parity of the uvu convolution kernels (xnn_uvu_conv and its backward, through
``ConvTensorProduct.conv``) against the float64 oracle (oracle/tp.py) for the forward and
against the module's PyTorch path in float64 for the gradients (that path is pinned to
the oracle on the CPU). Float32 sums of ~50 terms: 1e-5 of the output scale."""
import sys
import time

import numpy as np
import pytest
import torch

import oracle.tp as T
from xnn_amd import irreps as I

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _note(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def _close(got, want, tol=1e-5):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape
    if want.size == 0:
        return
    scale = max(1.0, float(np.abs(want).max()))
    err = float(np.abs(got - want).max())
    assert err <= tol * scale, (err, scale)


def _setup(mul, lsh, n, e, seed, pairs=False):
    from xnn_amd.conv import ConvTensorProduct
    irreps1 = I.Irreps(f"{mul}x0e+{mul}x1o+{mul}x2e" + (f"+{mul}x3o" if lsh == 3 else ""))
    sh = I.spherical_harmonics_irreps(lsh)
    mid, ins = I.tp_out_irreps_with_instructions(
        irreps1, sh, f"{mul}x0e+{mul}x0o+{mul}x1o+{mul}x1e+{mul}x2e+{mul}x2o+{mul}x3o+{mul}x3e",
        sort_instructions=False)
    tp = ConvTensorProduct(irreps1, sh, mid, ins, shared_weights=False, internal_weights=False)
    rng = np.random.default_rng(seed)
    src, dst = rng.integers(0, n, e), rng.integers(0, n, e)
    dst[dst == 1] = 2                                    # node 1 receives nothing
    src[src == 3] = 4                                    # node 3 sends nothing
    order = np.argsort(dst, kind="stable") if seed % 2 else np.arange(e)
    src, dst = src[order], dst[order]
    h = rng.standard_normal((n, irreps1.dim)).astype(np.float32)
    y = rng.standard_normal((e, sh.dim)).astype(np.float32)
    rows = e // 2 if pairs else e
    w = rng.standard_normal((rows, tp.weight_numel)).astype(np.float32)
    widx = rng.integers(0, rows, e) if pairs else None
    return tp, irreps1, sh, mid, ins, src, dst, h, y, w, widx


CASES = [(8, 2, 40, 300, 0, None, False), (32, 2, 70, 900, 1, 3.0, False),
         (80, 2, 30, 200, 2, None, True), (5, 3, 25, 160, 3, 1.7, True), (16, 1, 1, 0, 4, None, False)]


@pytest.mark.parametrize("mul,lsh,n,e,seed,divisor,pairs", CASES)
def test_conv_matches_the_oracle_and_the_pytorch_gradients(mul, lsh, n, e, seed, divisor, pairs):
    from xnn_amd import _lib
    _note(f"uvu conv mul={mul} lsh={lsh} n={n} e={e} divisor={divisor} pairs={pairs}")
    tp, irreps1, sh, mid, ins, src, dst, h, y, w, widx = _setup(mul, lsh, n, e, seed, pairs)
    assert tp.fast_eligible
    want = T.uvu_conv(h.astype(np.float64), y.astype(np.float64), w.astype(np.float64), src, dst, n,
                      repr(irreps1), repr(sh), repr(mid), [(a, b, c) for a, b, c, _, _ in ins],
                      divisor, widx)
    ei = torch.tensor(np.stack([src, dst]), device=DEV)
    hd = torch.tensor(h, device=DEV, requires_grad=True)
    yd = torch.tensor(y, device=DEV, requires_grad=True)
    wd = torch.tensor(w, device=DEV, requires_grad=True)
    wi = None if widx is None else torch.tensor(widx, device=DEV)
    tp.fast_active = True
    before = _lib.calls.get("xnn_uvu_conv", 0)
    out = tp.conv(hd, yd, wd, ei, n, divisor, weight_index=wi)
    assert _lib.calls.get("xnn_uvu_conv", 0) == before + 1
    _close(out.detach().cpu().numpy(), want)
    g = torch.randn(out.shape, generator=torch.Generator().manual_seed(seed)).to(DEV)
    gh, gy, gw = torch.autograd.grad(out, [hd, yd, wd], g)
    tp.fast_active = False
    ref = tp.double()
    h64, y64, w64 = (torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in (h, y, w))
    out64 = ref.conv(h64, y64, w64, torch.tensor(np.stack([src, dst])), n, divisor,
                     weight_index=None if widx is None else torch.tensor(widx))
    _close(out64.detach().numpy(), want, tol=1e-12)
    rh, ry, rw = torch.autograd.grad(out64, [h64, y64, w64], g.cpu().double(), allow_unused=True)
    for got_g, ref_g in ((gh, rh), (gy, ry), (gw, rw)):
        _close(got_g.cpu().numpy(), np.zeros(got_g.shape) if ref_g is None else ref_g.numpy())
    # run to run, bit for bit
    tp.float().fast_active = True
    again = tp.conv(hd, yd, wd, ei, n, divisor, weight_index=wi)
    assert torch.equal(again, out)


def test_conv_water_box_graph_timing():
    """The same layer on the water box's own neighbor list (9,000 atoms, 477,698 edges, 5 A
    cutoff, receivers in CSR order, atoms in the generator's spatial order), where the
    senders of nearby receivers are shared: forward against the oracle on a sample of nodes,
    and the time per launch."""
    import xnn_amd as xa
    from xnn_amd import synthetic
    from xnn_amd.conv import plan_of
    _note("uvu conv on the water box's neighbor list")
    s = synthetic.water_box(seed=0)
    n = len(s.pos)
    ei, _ = xa.build_neighbor_list(torch.tensor(s.pos, dtype=torch.float32, device=DEV), 5.0,
                                   torch.tensor(s.cell, dtype=torch.float32, device=DEV),
                                   torch.tensor(s.pbc))
    e = ei.shape[1]
    src, dst = (a.cpu().numpy() for a in ei)
    assert bool((dst[1:] >= dst[:-1]).all())
    tp, irreps1, sh, mid, ins, _, _, h, y, w, _ = _setup(32, 2, n, e, 7)
    hd, yd, wd = (torch.tensor(a, device=DEV) for a in (h, y, w))
    tp.fast_active = True
    plan = plan_of(ei, n)
    out = tp.conv(hd, yd, wd, ei, n, plan=plan)
    torch.cuda.synchronize()
    pick = np.arange(0, n, 97)
    sel = np.isin(dst, pick)
    want = T.uvu_conv(h.astype(np.float64), y[sel].astype(np.float64), w[sel].astype(np.float64),
                      src[sel], dst[sel], n, repr(irreps1), repr(sh), repr(mid),
                      [(a, b, c) for a, b, c, _, _ in ins])
    _close(out.cpu().numpy()[pick], want[pick])
    hr, yr, wr = (t.clone().requires_grad_() for t in (hd, yd, wd))
    g = torch.randn_like(out)
    times = {}
    for name in ("forward", "backward"):
        for rep in range(6):
            if rep == 1:
                torch.cuda.synchronize()
                t0 = time.perf_counter()
            if name == "forward":
                tp.conv(hd, yd, wd, ei, n, plan=plan)
            else:
                o = tp.conv(hr, yr, wr, ei, n, plan=plan)
                torch.autograd.grad(o, [hr, yr, wr], g)
        torch.cuda.synchronize()
        times[name] = (time.perf_counter() - t0) / 5 * 1e6
    print(f"uvu conv water box graph {n} nodes / {e} edges: forward {times['forward']:.0f} us, "
          f"forward+backward {times['backward']:.0f} us", flush=True)


def test_conv_water_size_timing():
    """A NequIP-sized layer on the water box's graph shape (9,000 nodes, 450k edges, 32
    channels of 0e + 1o + 2e, harmonics to l = 2): forward and backward against the
    PyTorch path on a sample of nodes, and the time per launch."""
    from xnn_amd.conv import plan_of
    _note("uvu conv 450k edges")
    n, e = 9000, 450_000
    tp, irreps1, sh, mid, ins, src, dst, h, y, w, widx = _setup(32, 2, n, e, 7)
    order = np.argsort(dst, kind="stable")
    src, dst, y, w = src[order], dst[order], y[order], w[order]
    ei = torch.tensor(np.stack([src, dst]), device=DEV)
    hd, yd, wd = (torch.tensor(a, device=DEV) for a in (h, y, w))
    tp.fast_active = True
    plan = plan_of(ei, n)
    out = tp.conv(hd, yd, wd, ei, n, plan=plan)
    torch.cuda.synchronize()
    pick = np.arange(0, n, 97)
    sel = np.isin(dst, pick)
    want = T.uvu_conv(h.astype(np.float64), y[sel].astype(np.float64), w[sel].astype(np.float64),
                      src[sel], dst[sel], n, repr(irreps1), repr(sh), repr(mid),
                      [(a, b, c) for a, b, c, _, _ in ins])
    _close(out.cpu().numpy()[pick], want[pick])
    hr, yr, wr = (t.clone().requires_grad_() for t in (hd, yd, wd))
    g = torch.randn_like(out)
    times = {}
    for name in ("forward", "backward"):
        for rep in range(6):
            if rep == 1:
                torch.cuda.synchronize()
                t0 = time.perf_counter()
            if name == "forward":
                tp.conv(hd, yd, wd, ei, n, plan=plan)
            else:
                o = tp.conv(hr, yr, wr, ei, n, plan=plan)
                torch.autograd.grad(o, [hr, yr, wr], g)
        torch.cuda.synchronize()
        times[name] = (time.perf_counter() - t0) / 5 * 1e6
    print(f"uvu conv 9000 nodes / 450k edges, 32x(0e+1o+2e) x sh2 -> {mid.dim} per node, "
          f"{len(ins)} paths: forward {times['forward']:.0f} us, forward+backward "
          f"{times['backward']:.0f} us", flush=True)
