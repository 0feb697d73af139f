"""Export of the slot operators on the GPU, the way the reference exports its
model (``tace/models/compile/aot.py:229-250``): ``make_fx`` symbolic trace of
a function that takes forces by ``torch.autograd.grad``, then
``torch.export.export(strict=False)`` with dynamic node and edge counts.  The
exported program, run on a graph of other sizes, gives the eager results."""

import pytest
import torch
from torch.fx.experimental.proxy_tensor import make_fx

from tace_amd import slot

pytestmark = pytest.mark.gpu


def _graph(N, E, tp, g, cuda, dtype):
    x = torch.randn(N, tp.irreps_in1.dim, generator=g, dtype=dtype).to(cuda)
    y = torch.randn(E, tp.irreps_in2.dim, generator=g, dtype=dtype).to(cuda)
    w = torch.randn(E, tp.weight_numel, generator=g, dtype=dtype).to(cuda)
    ei = torch.randint(0, N, (2, E), generator=g).to(cuda)
    return x, y, w, ei


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_exported_uvu_slot_with_forces(cuda, dtype):
    tp = slot.e3nnHipScatterTensorProduct("32x0e+32x1o+32x2e+32x3o", "1x0e+1x1o+1x2e+1x3o",
                                          "32x0e+32x1o+32x2e+32x3o")

    def fn(x, y, w, edge_index):
        x = x.detach().requires_grad_(True)
        y = y.detach().requires_grad_(True)
        out = tp(x, y, w, edge_index)
        e = (out * out).sum()
        gx, gy = torch.autograd.grad(e, [x, y])
        return e, gx, gy

    g = torch.Generator().manual_seed(1)
    sample = _graph(23, 170, tp, g, cuda, dtype)
    traced = make_fx(fn, tracing_mode="symbolic", _allow_non_fake_inputs=True)(*sample)
    n, e = torch.export.Dim("num_nodes", min=2), torch.export.Dim("num_edges", min=2)
    ep = torch.export.export(traced, sample, dynamic_shapes=({0: n}, {0: e}, {0: e}, {1: e}), strict=False)
    other = _graph(41, 333, tp, g, cuda, dtype)
    got = ep.module()(*other)
    want = fn(*other)
    tol = 1e-12 if dtype == torch.float64 else 1e-5
    for a, b in zip(got, want):
        assert a.shape == b.shape
        assert ((a - b).abs().max() / b.abs().max()).item() < tol


def test_exported_uuu_slot_with_gradient(cuda):
    irr = "16x0e+16x1o+16x2e+16x3o"
    tp = slot.e3nnHipUuuTensorProduct(irr, irr, irr, identical_inputs=True)

    def fn(x1):
        x1 = x1.detach().requires_grad_(True)
        out = tp(x1, x1)
        (gr,) = torch.autograd.grad((out * out).sum(), [x1])
        return out.detach(), gr

    g = torch.Generator().manual_seed(2)
    sample = (torch.randn(17, 16 * 16, generator=g, dtype=torch.float64).to(cuda),)
    traced = make_fx(fn, tracing_mode="symbolic", _allow_non_fake_inputs=True)(*sample)
    ep = torch.export.export(traced, sample, dynamic_shapes=({0: torch.export.Dim("num_nodes", min=2)},),
                             strict=False)
    other = torch.randn(35, 16 * 16, generator=g, dtype=torch.float64).to(cuda)
    for a, b in zip(ep.module()(other), fn(other)):
        assert ((a - b).abs().max() / b.abs().max()).item() < 1e-12


def test_exported_tece_slot_with_gradients(cuda):
    """The TECE convolution slot (frozen parameters, random weights) traced
    with its gradients to x, the radial weights and the radial basis,
    exported with dynamic node / edge counts and run on another graph."""
    from oracle import tece as ot
    lmax, C, H, A, nr = 2, 32, 2, 16, 8
    K = (lmax + 1) ** 2
    torch.manual_seed(3)
    conv = slot.HipTeceConvolution(lmax, lmax, C, H, True, A, None, nr, "w1", True, True, True).double()
    with torch.no_grad():
        for prm in conv.parameters():
            prm.copy_(0.5 * torch.randn_like(prm))
    conv = conv.to(cuda)
    for prm in conv.parameters():
        prm.requires_grad_(False)

    def fn(x, w, edge_index, wigner, R):
        x = x.detach().requires_grad_(True)
        w = w.detach().requires_grad_(True)
        R = R.detach().requires_grad_(True)
        out = conv(x, w, edge_index, None, wigner, wigner.transpose(1, 2), R)
        gx, gw, gR = torch.autograd.grad((out * out).sum(), [x, w, R])
        return out.detach(), gx, gw, gR

    g = torch.Generator().manual_seed(4)

    def graph(N, E):
        x = torch.randn(N, K * C, generator=g, dtype=torch.float64).to(cuda)
        w = torch.randn(E, conv.weight_numel, generator=g, dtype=torch.float64).to(cuda)
        ei = torch.randint(0, N, (2, E), generator=g).to(cuda)
        v = torch.randn(E, 3, generator=g, dtype=torch.float64)
        W, _ = ot.edge_wigner(v / v.norm(dim=1, keepdim=True) * 2.0, lmax, lmax)
        R = torch.randn(E, nr, generator=g, dtype=torch.float64).to(cuda)
        return x, w, ei, W.to(cuda).contiguous(), R

    sample = graph(30, 260)
    traced = make_fx(fn, tracing_mode="symbolic", _allow_non_fake_inputs=True)(*sample)
    n, e = torch.export.Dim("num_nodes", min=2), torch.export.Dim("num_edges", min=2)
    ep = torch.export.export(traced, sample, dynamic_shapes=({0: n}, {0: e}, {1: e}, {0: e}, {0: e}), strict=False)
    other = graph(47, 511)
    for a, b in zip(ep.module()(*other), fn(*other)):
        assert a.shape == b.shape
        assert ((a - b).abs().max() / b.abs().max()).item() < 1e-10
