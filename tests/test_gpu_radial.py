"""GPU parity of the fused radial-network kernels (xnn_radial_hidden and its backward,
through ``xnn_amd.radial``) against the float64 oracle (oracle/radial.py) and the
module's own PyTorch evaluation. Float32 products over at most 128 terms: outputs and
gradients to 2e-5 of their scale."""
import sys
import time

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle.radial as R

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _note(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def _close(got, want, tol=2e-5):
    got = np.asarray(got, dtype=np.float64)
    assert got.shape == want.shape
    if want.size == 0:
        return
    scale = max(1.0, float(np.abs(want).max()))
    err = float(np.abs(got - want).max())
    assert err <= tol * scale, (err, scale)


CASES = [(1000, 8, [64, 64, 64]), (37, 3, [50]), (4096, 12, [100, 128]), (0, 8, [64, 64, 64]),
         (5000, 32, [128, 128, 128]), (17, 8, [16, 7, 5]), (2049, 16, [32, 32]),
         (3001, 8, [128, 96, 128])]


@pytest.mark.parametrize("rows,n_in,widths", CASES)
def test_fused_hidden_matches_the_oracle(rows, n_in, widths):
    from xnn_amd import _lib, ops
    _note(f"radial hidden rows={rows} n_in={n_in} widths={widths}")
    g = torch.Generator().manual_seed(rows + n_in)
    x = torch.randn(rows, n_in, generator=g)
    dims = [n_in] + widths
    ws = [torch.randn(a, b, generator=g) for a, b in zip(dims, dims[1:])]
    sc = [1.0 / np.sqrt(a) * (1.68 if i else 1.0) for i, a in enumerate(dims[:-1])]
    go = torch.randn(rows, widths[-1], generator=g)
    want, vjp = R.hidden_chain(x.numpy(), [w.numpy() for w in ws], sc)
    want_gx = vjp(go.numpy())
    xd, wd, god = x.to(DEV), [w.to(DEV) for w in ws], go.to(DEV)
    before = _lib.calls.get("xnn_radial_hidden", 0)
    out = ops.radial_hidden_op(xd, wd, sc)
    gx = ops.radial_hidden_backward_op(xd, god, wd, sc)
    torch.cuda.synchronize()
    assert _lib.calls.get("xnn_radial_hidden", 0) == before + 1
    assert out.shape == (rows, widths[-1]) and gx.shape == (rows, n_in)
    _close(out.cpu().numpy(), want)
    _close(gx.cpu().numpy(), want_gx)
    # bit for bit run to run
    assert torch.equal(ops.radial_hidden_op(xd, wd, sc), out)


def test_radialnet_fast_path_forward_and_gradients():
    """RadialNet([8, 64, 64, 64, 40]) in evaluation mode: the fused path against the same
    module's PyTorch path (fast_active off) in float64; forces-style gradients (input only)
    run the HIP backward, and weight gradients / double backward take the PyTorch formula."""
    from xnn_amd import _lib
    from xnn_amd.radial import RadialNet
    _note("radialnet fast path")
    torch.manual_seed(0)
    net = RadialNet([8, 64, 64, 64, 40], F.silu).to(DEV).eval()
    ref = RadialNet([8, 64, 64, 64, 40], F.silu).to(DEV).double().eval()
    ref.load_state_dict({k: v.double() for k, v in net.state_dict().items()})
    x = torch.randn(3000, 8, device=DEV)
    net.fast_active = True
    xr = x.clone().requires_grad_()
    bwd_before = _lib.calls.get("xnn_radial_hidden_backward", 0)
    y = net(xr)
    xd = x.double().requires_grad_()
    yd = ref(xd)
    _close(y.detach().cpu().numpy(), yd.detach().cpu().numpy())
    cot = torch.randn_like(y)
    (gx,) = torch.autograd.grad(y, [xr], cot)
    (gxd,) = torch.autograd.grad(yd, [xd], cot.double())
    assert _lib.calls.get("xnn_radial_hidden_backward", 0) == bwd_before + 1
    _close(gx.cpu().numpy(), gxd.cpu().numpy())
    # weights' gradients: the PyTorch formula (no HIP backward call)
    y = net(xr)
    (y * cot).sum().backward()
    (ref(xd) * cot.double()).sum().backward()
    assert _lib.calls.get("xnn_radial_hidden_backward", 0) == bwd_before + 1
    for a, b in zip(net.parameters(), ref.parameters()):
        _close(a.grad.cpu().numpy(), b.grad.cpu().numpy())
    # double backward (a force loss): differentiable again
    xr2 = x.clone().requires_grad_()
    (g1,) = torch.autograd.grad((net(xr2) * cot).sum(), [xr2], create_graph=True)
    (g2,) = torch.autograd.grad(g1.square().sum(), [xr2])
    xd2 = x.double().requires_grad_()
    (h1,) = torch.autograd.grad((ref(xd2) * cot.double()).sum(), [xd2], create_graph=True)
    (h2,) = torch.autograd.grad(h1.square().sum(), [xd2])
    _close(g2.cpu().numpy(), h2.cpu().numpy(), tol=1e-4)


def test_fused_hidden_water_size_timing():
    """The water box's edge count (450k) through [8, 64, 64, 64]: forward and input
    gradient against the oracle on a sample of rows, and the time per launch."""
    from xnn_amd import ops
    _note("radial hidden 450k edges")
    g = torch.Generator().manual_seed(5)
    rows, dims = 450_000, [8, 64, 64, 64]
    ws = [torch.randn(a, b, generator=g) for a, b in zip(dims, dims[1:])]
    sc = [1 / np.sqrt(8), 1.68 / 8, 1.68 / 8]
    x = torch.rand(rows, 8, generator=g) * 2 - 1
    go = torch.randn(rows, 64, generator=g)
    xd, wd, god = x.to(DEV), [w.to(DEV) for w in ws], go.to(DEV)
    out = ops.radial_hidden_op(xd, wd, sc)
    gx = ops.radial_hidden_backward_op(xd, god, wd, sc)
    torch.cuda.synchronize()
    pick = torch.randperm(rows, generator=g)[:4000]
    want, vjp = R.hidden_chain(x[pick].numpy(), [w.numpy() for w in ws], sc)
    _close(out.cpu()[pick].numpy(), want)
    _close(gx.cpu()[pick].numpy(), vjp(go[pick].numpy()))
    ms = {}
    for name, fn in (("forward", lambda: ops.radial_hidden_op(xd, wd, sc)),
                     ("backward", lambda: ops.radial_hidden_backward_op(xd, god, wd, sc))):
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(20):
            fn()
        torch.cuda.synchronize()
        ms[name] = (time.perf_counter() - t0) / 20 * 1e3
    flops = 2 * rows * (8 * 64 + 64 * 64 * 2)
    print(f"radial hidden 450k x [8,64,64,64]: forward {ms['forward']*1e3:.1f} us "
          f"({flops / ms['forward'] / 1e9:.1f} TFLOP/s), backward {ms['backward']*1e3:.1f} us "
          f"({2 * flops / ms['backward'] / 1e9:.1f} TFLOP/s)", flush=True)
