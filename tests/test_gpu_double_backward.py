"""Double backward of the slot operators (training with a force loss,
create_graph=True, as tace/lightning/lit_model.py:150 trains through
forces): second derivatives of the uvu scatter product and the uuu product
against torch autograd through the oracle's products, in float64.  The
energy-like scalar is sum(out^2), so the upstream gradient of the backward
depends on the inputs and every term of the double backward is exercised."""

import pytest
import torch

from oracle import model as om
from oracle import so3 as oso3
from tace_amd import slot

pytestmark = pytest.mark.gpu


def _close(a, b, tol=1e-10, what=""):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    err = ((a - b).abs().max() / max(b.abs().max().item(), 1e-30)).item()
    assert err < tol, f"{what}: {err:.3e}"


def _second(fn, inputs, rs):
    """d/d(inputs) of sum_i <r_i, d(sum out^2)/d(input_i)> for the first len(rs) inputs."""
    out = fn(*inputs)
    first = torch.autograd.grad((out * out).sum(), inputs[:len(rs)], create_graph=True)
    L = sum((f * r).sum() for f, r in zip(first, rs))
    return torch.autograd.grad(L, inputs)


@pytest.mark.parametrize("lmax", [1, 3])
def test_uvu_scatter_double_backward(cuda, lmax):
    C = 16
    ls = list(range(lmax + 1))
    irr = "+".join(f"{C}x{l}{'e' if l % 2 == 0 else 'o'}" for l in ls)
    sh = "+".join(f"1x{l}{'e' if l % 2 == 0 else 'o'}" for l in ls)
    tp = slot.e3nnHipScatterTensorProduct(irr, sh, irr)
    ref = om.ScatterTP([(C, (l, (-1) ** l)) for l in ls], oso3.sh_irreps(lmax), [(1, (l, (-1) ** l)) for l in ls])
    g = torch.Generator().manual_seed(lmax)
    N, E = 19, 120
    x = torch.randn(N, tp.irreps_in1.dim, generator=g, dtype=torch.float64)
    y = torch.randn(E, (lmax + 1) ** 2, generator=g, dtype=torch.float64)
    w = torch.randn(E, tp.weight_numel, generator=g, dtype=torch.float64)
    ei = torch.randint(0, N, (2, E), generator=g)
    rx, ry = torch.randn_like(x), torch.randn_like(y)
    want = _second(lambda a, b, c: ref(a, b, c, ei), [t.clone().requires_grad_(True) for t in (x, y, w)], [rx, ry])
    got = _second(lambda a, b, c: tp(a, b, c, ei.to(cuda)),
                  [t.to(cuda).requires_grad_(True) for t in (x, y, w)], [rx.to(cuda), ry.to(cuda)])
    for a, b, n in zip(got, want, "xyw"):
        _close(a, b, what=n)


@pytest.mark.parametrize("weighted", [False, True])
def test_uuu_double_backward(cuda, weighted):
    C = 16
    full = [0, 1, 2]
    ir = lambda ls: "+".join(f"{C}x{l}{'e' if l % 2 == 0 else 'o'}" for l in ls)
    base = full + [0] if weighted else full
    tp = slot.e3nnHipUuuTensorProduct(ir(full), ir(base), ir(full), identical_inputs=not weighted)
    ref = om.UUUTP([(C, (l, (-1) ** l)) for l in full], [(C, (l, (-1) ** l)) for l in base],
                   [(1, (l, (-1) ** l)) for l in full], not weighted)
    g = torch.Generator().manual_seed(7 + weighted)
    Nn = 13
    x1 = torch.randn(Nn, sum(C * (2 * l + 1) for l in full), generator=g, dtype=torch.float64)
    x2 = torch.randn(Nn, sum(C * (2 * l + 1) for l in base), generator=g, dtype=torch.float64)
    if weighted:
        ws = torch.randn(Nn, len(ref.paths) * C, generator=g, dtype=torch.float64)
        r1, r2 = torch.randn_like(x1), torch.randn_like(x2)
        want = _second(lambda a, b, c: ref(a, b, c), [t.clone().requires_grad_(True) for t in (x1, x2, ws)], [r1, r2])
        got = _second(lambda a, b, c: tp(a, b, c), [t.to(cuda).requires_grad_(True) for t in (x1, x2, ws)],
                      [r1.to(cuda), r2.to(cuda)])
    else:
        r1 = torch.randn_like(x1)
        want = _second(lambda a: ref(a, a), [x1.clone().requires_grad_(True)], [r1])
        got = _second(lambda a: tp(a, a), [x1.to(cuda).requires_grad_(True)], [r1.to(cuda)])
    for a, b in zip(got, want):
        _close(a, b)
