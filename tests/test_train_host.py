"""CPU checks of the twice-differentiable operator forms (ops.differentiable_twice).

The torch forms of the radial basis, spherical harmonics, shared linear and
gate that the training path uses, against the oracle's independent
restatements (the W3j recursion for the harmonics) and against the
inference operators where those run on the CPU; second derivatives by
autograd agree with central differences of first derivatives.
"""

import math

import torch

from oracle import model as om
from oracle import so3 as oso3
from tace_amd import model as pm, ops


def test_spherical_harmonics_match_the_recursion():
    g = torch.Generator().manual_seed(0)
    v = torch.randn(200, 3, generator=g, dtype=torch.float64)
    u = v / v.norm(dim=1, keepdim=True)
    for lmax in range(4):
        a = ops.spherical_harmonics(u, lmax)
        b = oso3.spherical_harmonics(lmax, u)
        assert a.shape == b.shape
        assert (a - b).abs().max().item() < 1e-13, lmax


def test_edge_basis_matches_the_oracle_radial_basis():
    g = torch.Generator().manual_seed(1)
    v = torch.randn(300, 3, generator=g, dtype=torch.float64) * 2.0
    rc, nb, p = 5.0, 8, 5
    rb = om.RadialBasis(rc, nb, p).double()
    R, Y = ops._edge_basis_autograd(v, rb.radial_fn.bessel_weights, float(rb.radial_fn.prefactor), rc, p, 3)
    r = v.norm(dim=1, keepdim=True) + 1e-9
    assert (R - rb(r)).abs().max().item() < 1e-13
    assert (Y - oso3.spherical_harmonics(3, v / r)).abs().max().item() < 1e-13


def test_edge_basis_second_derivative():
    """autograd of the gradient against central differences of the gradient."""
    g = torch.Generator().manual_seed(2)
    v = (torch.randn(20, 3, generator=g, dtype=torch.float64) * 1.5).requires_grad_(True)
    wR = torch.randn(20, 8, generator=g, dtype=torch.float64)
    wY = torch.randn(20, 16, generator=g, dtype=torch.float64)
    bw = math.pi / 5.0 * torch.linspace(1.0, 8.0, 8, dtype=torch.float64)

    def grad_of(vv, create):
        R, Y = ops._edge_basis_autograd(vv, bw, math.sqrt(0.4), 5.0, 5, 3)
        return torch.autograd.grad((R * wR).sum() + (Y * wY).sum(), vv, create_graph=create)[0]

    gv = grad_of(v, True)
    d = torch.randn(20, 3, generator=g, dtype=torch.float64)
    (hv,) = torch.autograd.grad((gv * d).sum(), v)
    h = 1e-5
    with torch.no_grad():
        vp, vm = (v + h * d).requires_grad_(True), (v - h * d).requires_grad_(True)
    fd = ((grad_of(vp, False) - grad_of(vm, False)) / (2 * h) * 1.0)
    # H d (symmetric Hessian) against the directional derivative of the gradient
    assert (hv - fd).abs().max().item() < 1e-6 * max(1.0, fd.abs().max().item())


def test_functional_linear_equals_linear_fn():
    torch.set_default_dtype(torch.float64)
    try:
        for irr_in, irr_out in [("8x0e+5x0e+6x1o+4x1o+3x2e", "7x0e+6x1o+5x2e+2x3o"), ("16x0e+16x1o", "32x0e+16x1o")]:
            lin = pm.e3nnLinear(irr_in, irr_out)
            with torch.no_grad():
                if lin.bias is not None:
                    lin.bias.normal_()
            x = torch.randn(11, lin.lay.dim_in, requires_grad=True)
            a = lin(x, 0.7)
            b = pm._linear_autograd(x, lin.weight, lin.bias, lin.lay, None, 0.7)
            assert (a - b).abs().max().item() < 1e-13
            gout = torch.randn_like(a)
            ga = torch.autograd.grad(a, [x, lin.weight], gout)
            gb = torch.autograd.grad(b, [x, lin.weight], gout)
            for u, w in zip(ga, gb):
                assert (u - w).abs().max().item() < 1e-13
    finally:
        torch.set_default_dtype(torch.float32)


def test_functional_gate_equals_gate_fn():
    from tace_amd.so3 import Irreps
    C = 4
    lin = pm.GMLayout(Irreps(f"{4 * C}x0e+{C}x1o+{C}x2e"))   # 3 C gates + the gated 0e, then 1o, 2e
    lout = pm.GMLayout(Irreps(f"{C}x0e+{C}x1o+{C}x2e"))
    x = torch.randn(5, lin.dim, dtype=torch.float64, requires_grad=True)
    a = pm._GateFn.apply(x, lin, lout, C)
    with ops.differentiable_twice():
        b = pm._gate(x, lin, lout, C)
    assert (a - b).abs().max().item() < 1e-14
    gout = torch.randn_like(a)
    (ga,) = torch.autograd.grad(a, x, gout)
    (gb,) = torch.autograd.grad(b, x, gout)
    assert (ga - gb).abs().max().item() < 1e-14


def test_mode_is_restored():
    assert not ops.MODE.double
    with ops.differentiable_twice():
        assert ops.MODE.double
        with ops.differentiable_twice(False):
            assert not ops.MODE.double
        assert ops.MODE.double
    assert not ops.MODE.double
