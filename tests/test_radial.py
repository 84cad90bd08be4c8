"""The radial network (xnn_amd.radial) on the CPU: the e3nn layer rule and its folded
evaluation against the oracle (oracle/radial.py), the oracle pinned by what the
mathematics fixes (the normalization constant as a Gaussian integral, the unit second
moment the normalization exists for, finite differences of the hidden chain)."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle.radial as R
from xnn_amd import radial as X


def test_second_moment_constant_is_the_gaussian_integral():
    """e3nn's seeded Monte Carlo estimate of E[f(z)^2]^(-1/2) agrees with the quadrature
    value to its sampling error (~1e-3 at 10^6 draws), for silu and tanh; a wrong power or
    a missing square root is off by far more."""
    for f_t, f_n in ((F.silu, R.silu), (torch.tanh, np.tanh)):
        mc = X.second_moment_constant(f_t)
        exact = R.exact_second_moment_constant(f_n)
        assert abs(mc / exact - 1) < 3e-3, (mc, exact)
        assert X.second_moment_constant(f_t) == mc           # seeded: the same every time
    # the quadrature itself: E[z^2] = 1, E[z^4] = 3
    assert abs(R.exact_second_moment_constant(lambda z: z) - 1.0) < 1e-12
    assert abs(R.exact_second_moment_constant(lambda z: z * z) - 3 ** -0.5) < 1e-12


def test_oracle_network_keeps_unit_second_moment():
    """The point of the e3nn normalization: with standard normal weights and inputs of
    variance var_in, every layer's output has second moment ~1 and the last ~var_out."""
    rng = np.random.default_rng(0)
    cst = R.exact_second_moment_constant(R.silu)
    hs = [16, 256, 256, 8]
    ws = [rng.standard_normal((a, b)) for a, b in zip(hs, hs[1:])]
    for var_in, var_out in ((1.0, 1.0), (4.0, 1.0), (1.0, 9.0)):
        x = rng.standard_normal((20000, 16)) * math.sqrt(var_in)
        y = R.fully_connected(x, ws, cst, variance_in=var_in, variance_out=var_out)
        m2 = float(np.mean(y ** 2))
        assert 0.75 * var_out < m2 < 1.3 * var_out, (var_in, var_out, m2)


@pytest.mark.parametrize("hs,out_act,var", [([8, 64, 64, 64, 40], False, (1.0, 1.0)),
                                             ([5, 32, 17], True, (2.0, 0.5)),
                                             ([3, 9], False, (1.0, 3.0)),
                                             ([12, 48, 48, 48, 48, 6], False, (1.0, 1.0))])
def test_radialnet_matches_the_layer_by_layer_network(hs, out_act, var):
    torch.manual_seed(0)
    net = X.RadialNet(hs, F.silu, variance_in=var[0], variance_out=var[1],
                      out_act=out_act).double()
    assert [k for k in net.state_dict()] == [f"layer{i}.weight" for i in range(len(hs) - 1)]
    x = torch.randn(300, hs[0], dtype=torch.float64)
    ws = [m.weight.detach().numpy() for m in net]
    cst = net.layer0.act.cst if net.layer0.act is not None else 1.0
    want = R.fully_connected(x.numpy(), ws, cst, variance_in=var[0], variance_out=var[1],
                             out_act=out_act)
    np.testing.assert_allclose(net(x).detach().numpy(), want, rtol=1e-12, atol=1e-12)
    # the layers as written (nn.Sequential) give the same values
    seq = x
    for m in net:
        seq = m(seq)
    np.testing.assert_allclose(seq.detach().numpy(), want, rtol=1e-12, atol=1e-12)
    # the column map: output columns out_index times out_scale
    idx = torch.randperm(hs[-1])[: max(1, hs[-1] - 2)]
    scale = torch.rand(len(idx), dtype=torch.float64) + 0.5
    np.testing.assert_allclose(net(x, idx, scale).detach().numpy(),
                               want[:, idx.numpy()] * scale.numpy(), rtol=1e-12, atol=1e-12)
    # recomputation in the backward gives the same gradients
    xr = x.clone().requires_grad_()
    (g_keep,) = torch.autograd.grad(net(xr).square().sum(), [xr])
    X.set_recompute_radial(net, "on")
    (g_rec,) = torch.autograd.grad(net(xr).square().sum(), [xr])
    assert torch.equal(g_keep, g_rec)


def test_hidden_chain_vjp_matches_finite_differences():
    rng = np.random.default_rng(1)
    ws = [rng.standard_normal((6, 10)), rng.standard_normal((10, 7)), rng.standard_normal((7, 5))]
    sc = [0.4, 0.3, 0.35]
    x = rng.standard_normal((4, 6))
    g = rng.standard_normal((4, 5))
    _, vjp = R.hidden_chain(x, ws, sc)
    gx = vjp(g)
    h = 1e-6
    for (i, k) in [(0, 0), (1, 3), (3, 5), (2, 2)]:
        xp, xm = x.copy(), x.copy()
        xp[i, k] += h
        xm[i, k] -= h
        fd = (np.sum(g * R.hidden_chain(xp, ws, sc)[0]) - np.sum(g * R.hidden_chain(xm, ws, sc)[0])) / (2 * h)
        assert abs(fd - gx[i, k]) < 1e-8, (i, k, fd, gx[i, k])


def test_torch_vjp_of_the_fused_layers_matches_autograd():
    """The PyTorch backward the fused op takes for the weights' gradients (and double
    backward): input and weight gradients equal autograd's of the same chain."""
    torch.manual_seed(2)
    ws = [torch.randn(8, 16, dtype=torch.float64, requires_grad=True),
          torch.randn(16, 12, dtype=torch.float64, requires_grad=True)]
    sc = [0.35, 0.25]
    x = torch.randn(20, 8, dtype=torch.float64, requires_grad=True)
    g = torch.randn(20, 12, dtype=torch.float64)
    s = x
    for w, c in zip(ws, sc):
        s = F.silu((s @ w) * c)
    want = torch.autograd.grad(s, [x, *ws], g)
    got = X._vjp_torch(x.detach(), [w.detach() for w in ws], sc, g)
    for a, b in zip(got, want):
        torch.testing.assert_close(a, b, rtol=1e-12, atol=1e-12)
    _, vjp = R.hidden_chain(x.detach().numpy(), [w.detach().numpy() for w in ws], sc)
    np.testing.assert_allclose(got[0].numpy(), vjp(g.numpy()), rtol=1e-12, atol=1e-12)


def test_fast_path_needs_a_gpu_and_silu_layers():
    net = X.RadialNet([8, 64, 64, 64, 10], F.silu)
    assert not net.fast_supported(torch.device("cpu"), torch.float32)
    assert net.fast_supported(torch.device("cuda"), torch.float32)
    assert not net.fast_supported(torch.device("cuda"), torch.float64)
    assert not X.RadialNet([8, 64, 10], torch.tanh).fast_supported(torch.device("cuda"), torch.float32)
    assert not X.RadialNet([8, 200, 10], F.silu).fast_supported(torch.device("cuda"), torch.float32)
    assert not X.RadialNet([8, 64, 64, 64, 64, 10], F.silu).fast_supported(torch.device("cuda"),
                                                                           torch.float32)
    assert not X.RadialNet([40, 64, 10], F.silu).fast_supported(torch.device("cuda"), torch.float32)


def test_oracle_torch_network_equals_the_numpy_oracle():
    """oracle.radial.fully_connected_torch against oracle.radial.fully_connected."""
    import oracle.radial as OR
    rng = np.random.default_rng(2)
    ws = [rng.standard_normal((8, 16)), rng.standard_normal((16, 16)), rng.standard_normal((16, 5))]
    x = rng.standard_normal((40, 8))
    cst = OR.exact_second_moment_constant(OR.silu)
    want = OR.fully_connected(x, ws, cst, variance_in=0.7, variance_out=1.3)
    got = OR.fully_connected_torch(torch.tensor(x), [torch.tensor(w) for w in ws], cst,
                                   variance_in=0.7, variance_out=1.3)
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-13, atol=1e-13)
