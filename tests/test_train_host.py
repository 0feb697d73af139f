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


def test_edge_wigner_matches_the_oracle_frames():
    """The torch edge frames / Wigner blocks of the training path against the
    oracle's restatement, including edges along +-y (the chart blend's ends)."""
    from oracle import tece as ot
    g = torch.Generator().manual_seed(3)
    v = torch.randn(200, 3, generator=g, dtype=torch.float64) * 2.0
    v[0] = torch.tensor([0.0, 1.5, 0.0], dtype=torch.float64)
    v[1] = torch.tensor([0.0, -2.0, 0.0], dtype=torch.float64)
    v[2] = torch.tensor([1e-3, -2.0, 0.0], dtype=torch.float64)
    for lmax in (1, 2, 3):
        a = ops._edge_wigner_autograd(v, lmax)
        b, _ = ot.edge_wigner(v, lmax, lmax)
        assert (a - b).abs().max().item() < 1e-12, lmax


def test_tece_convolution_autograd_matches_the_oracle():
    """The training path's torch TECE convolution on group-major, permuted
    feature rows against the oracle's convolution on a random graph: output
    and the gradients of a scalar function of it (inputs and parameters)."""
    from oracle import tece as ot
    from tace_amd import tece as pt
    lmax, C, H, A, nr = 2, 8, 2, 4, 8
    K = (lmax + 1) ** 2
    g = torch.Generator().manual_seed(4)
    torch.manual_seed(5)
    ref = ot.TeceConvolution(lmax, lmax, C, H, A, nr).double()
    with torch.no_grad():
        for name, p in ref.named_parameters():
            if "radial_proj" in name:
                p.copy_(0.7 * torch.randn(p.shape, generator=g, dtype=p.dtype))
            elif "temperature_logit" in name:
                p.copy_(torch.randn(p.shape, generator=g, dtype=p.dtype))
    torch.set_default_dtype(torch.float64)
    try:
        conv = pt.TeceConvolution(lmax, lmax, C, H, A, nr)
    finally:
        torch.set_default_dtype(torch.float32)
    conv.load_state_dict(ref.state_dict(), strict=False)
    N, E = 12, 60
    src = torch.randint(0, N, (E,), generator=g)
    dst = torch.randint(0, N, (E,), generator=g)
    vec = torch.randn(E, 3, generator=g, dtype=torch.float64)
    x_l = torch.randn(N, K, C, generator=g, dtype=torch.float64, requires_grad=True)
    w = torch.randn(E, conv.weight_numel, generator=g, dtype=torch.float64, requires_grad=True)
    R = torch.randn(E, nr, generator=g, dtype=torch.float64)
    W, Wi = ot.edge_wigner(vec, lmax, lmax)
    want = ref(x_l, w, torch.stack([src, dst]), W, Wi, R)
    # group-major rows in a permuted order (row perm^-1[n] holds node n)
    perm = torch.randperm(N, generator=g)
    node_map = torch.empty_like(perm)
    node_map[perm] = torch.arange(N)
    x_rows = x_l[perm]
    x_gm = torch.cat([x_rows[:, l * l:(l + 1) ** 2].reshape(-1) for l in range(lmax + 1)]).view(N, K * C)
    got = conv._forward_autograd(x_gm, w, node_map.to(torch.int32), src, dst, ops._edge_wigner_autograd(vec, lmax), R)
    got_l = torch.cat([got.reshape(-1)[N * C * l * l:N * C * (l + 1) ** 2].view(N, 2 * l + 1, C)
                       for l in range(lmax + 1)], dim=1)[node_map]
    assert (got_l - want).abs().max().item() < 1e-12 * max(1.0, want.abs().max().item())
    probe = torch.randn(N, K, C, generator=g, dtype=torch.float64)
    own = dict(conv.named_parameters())
    names = [n for n, _ in ref.named_parameters()]
    ga = torch.autograd.grad((got_l * probe).sum(), [x_l, w] + [own[n] for n in names])
    gb = torch.autograd.grad((want * probe).sum(), [x_l, w] + [dict(ref.named_parameters())[n] for n in names])
    for a, b in zip(ga, gb):
        assert (a - b).abs().max().item() < 1e-11 * max(1.0, b.abs().max().item())


def test_bilinear_split_backward_equals_autograd_of_the_slices():
    """The bilinear-gate product basis splits linear_up's output into path
    weights (SiLU), node and base features (prod.py:178-214); its one-pass
    backward gives the bits of autograd through the slices, also with an
    output left unused."""
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    try:
        torch.manual_seed(0)
        m = pm.CgtpACE(0, 2, "16x0e+16x1o+16x2e", 16, 2, 2, 2, 3, bilinear=True)
    finally:
        torch.set_default_dtype(prev)
    u = torch.randn(7, m._up_lay.dim, dtype=torch.float64, requires_grad=True)
    gs = None
    for keep in (3, 2):
        a = m._split_up_torch(u)
        b = pm._SplitUpFn.apply(u, m)
        for x, y in zip(a, b):
            assert torch.equal(x, y)
        if gs is None:
            gs = [torch.randn_like(o) for o in a]
        ga = torch.autograd.grad(a[:keep], u, gs[:keep])[0]
        gb = torch.autograd.grad(b[:keep], u, gs[:keep])[0]
        assert torch.equal(ga, gb), keep
