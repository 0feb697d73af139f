"""The slot operators as torch custom operators (tace_amd.library), traced on
the host: ``make_fx`` over a function that takes forces with
``torch.autograd.grad`` (as tace/models/compile/compile.py:53-80 traces the
reference model) keeps the forward and backward operators as single nodes,
with shapes from their fake implementations and symbolic sizes."""

import torch
from torch.fx.experimental.proxy_tensor import make_fx

from tace_amd import slot


def _toy(tp):
    def fn(x, y, w, edge_index):
        x = x.detach().requires_grad_(True)
        y = y.detach().requires_grad_(True)
        out = tp(x, y, w, edge_index)
        e = (out * out).sum()
        gx, gy = torch.autograd.grad(e, [x, y])
        return e, gx, gy
    return fn


def test_uvu_slot_traces_to_custom_ops():
    tp = slot.e3nnHipScatterTensorProduct("16x0e+16x1o+16x2e+16x3o", "1x0e+1x1o+1x2e+1x3o",
                                          "16x0e+16x1o+16x2e+16x3o")
    N, E = 11, 40
    args = (torch.empty(N, 16 * 16, device="meta"), torch.empty(E, 16, device="meta"),
            torch.empty(E, tp.weight_numel, device="meta"), torch.empty(2, E, dtype=torch.int64, device="meta"))
    g = make_fx(_toy(tp), tracing_mode="symbolic")(*args)
    targets = [str(n.target) for n in g.graph.nodes if n.op == "call_function"]
    assert "tace_amd.uvu_scatter.default" in targets
    assert "tace_amd.uvu_scatter_backward.default" in targets
    outs = [n for n in g.graph.nodes if n.op == "output"][0].args[0]
    # grad_x / grad_y keep the symbolic node / edge counts of x / y
    gx, gy = outs[1].meta["val"], outs[2].meta["val"]
    assert isinstance(gx.shape[0], torch.SymInt) and isinstance(gy.shape[0], torch.SymInt)
    assert tuple(gx.shape[1:]) == (16 * 16,) and tuple(gy.shape[1:]) == (16,)


def test_uuu_slot_traces_to_custom_ops():
    irr = "8x0e+8x1o+8x2e"
    tp = slot.e3nnHipUuuTensorProduct(irr, irr, irr, identical_inputs=True)
    N = 9

    def fn(x1):
        x1 = x1.detach().requires_grad_(True)
        out = tp(x1, x1)
        (g,) = torch.autograd.grad((out * out).sum(), [x1])
        return g

    g = make_fx(fn, tracing_mode="symbolic")(torch.empty(N, 8 * 9, device="meta"))
    targets = [str(n.target) for n in g.graph.nodes if n.op == "call_function"]
    assert "tace_amd.uuu.default" in targets and "tace_amd.uuu_backward.default" in targets


def test_tece_slot_traces_to_custom_ops():
    """The TECE convolution slot: all its kernels trace as custom operators,
    with their backward operators under a traced autograd.grad."""
    lmax, C, H, A, nr = 2, 16, 2, 8, 8
    conv = slot.HipTeceConvolution(lmax, lmax, C, H, True, A, None, nr, "w1", True, True, True).to("meta")
    for prm in conv.parameters():
        prm.requires_grad_(False)
    N, E, K = 13, 57, (lmax + 1) ** 2

    def fn(x, w, edge_index, wigner, R):
        x = x.detach().requires_grad_(True)
        w = w.detach().requires_grad_(True)
        R = R.detach().requires_grad_(True)
        out = conv(x, w, edge_index, None, wigner, wigner.transpose(1, 2), R)
        return torch.autograd.grad((out * out).sum(), [x, w, R])

    args = (torch.empty(N, K * C, device="meta"), torch.empty(E, conv.weight_numel, device="meta"),
            torch.empty(2, E, dtype=torch.int64, device="meta"), torch.empty(E, K, K, device="meta"),
            torch.empty(E, nr, device="meta"))
    g = make_fx(fn, tracing_mode="symbolic", _allow_non_fake_inputs=True)(*args)
    targets = {str(n.target) for n in g.graph.nodes if n.op == "call_function"}
    for op in ("receiver_csr", "tece_rotate_in", "tece_score", "tece_softmax", "tece_edge_ace", "tece_rotate_out"):
        assert f"tace_amd.{op}.default" in targets, op
    for op in ("tece_rotate_in", "tece_score", "tece_softmax", "tece_edge_ace", "tece_rotate_out"):
        assert f"tace_amd.{op}_backward.default" in targets, op
