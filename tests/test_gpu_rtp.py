"""Parity of the radial-fused edge tensor product (``ops.edge_rtp_scatter``:
the radial MLP's last layer made on MFMA inside the product kernels) with
the CPU oracle and with the unfused GPU path (GPU).

The oracle computes w = alpha * h @ W and the scatter product
(``oracle.model.ScatterTP``) in float64 from the same float32 inputs;
tolerance 2e-5 relative to the largest magnitude (float32 sums in another
order).  The cases cover receivers without edges, with fewer than one
16-edge block and with many blocks, unsorted edges (a slot -> edge map),
both operand layouts, a permuted feature-row order and 64 / 128 / 192
channels.
"""

import pytest
import torch

from oracle import model as om
from oracle import so3 as oso3
from tace_amd import ops

pytestmark = pytest.mark.gpu

TOL = 2e-5


def close(got, want, what=""):
    got = got.detach().double().cpu()
    want = want.detach().double().cpu()
    scale = max(want.abs().max().item(), 1e-30)
    err = (got - want).abs().max().item() / scale
    assert err < TOL, f"{what}: max rel err {err:.3e} (scale {scale:.3e})"


def _graph(g, Nn, E, sorted_edges):
    """Random edges with one receiver of many edges (several 16-edge blocks)
    and the last receivers without edges."""
    src = torch.randint(0, Nn, (E,), generator=g)
    dst = torch.randint(0, Nn - 3, (E,), generator=g)
    dst[: E // 6] = 5
    if sorted_edges:
        order = torch.argsort(dst, stable=True)
        src, dst = src[order], dst[order]
    return torch.stack([src, dst])


def _case(g, in1, lmax, C, E, Nn):
    tp = om.ScatterTP([(C, (l, (-1) ** l)) for l in in1], oso3.sh_irreps(lmax),
                      [(1, (l, (-1) ** l)) for l in range(lmax + 1)])
    f32 = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64).float()
    x = f32(Nn, oso3.irreps_dim([(C, (l, (-1) ** l)) for l in in1]))
    y = f32(E, (lmax + 1) ** 2)
    h = f32(E, 64)
    W = f32(64, tp.weight_numel)
    return tp, x, y, h, W


RTP_CASES = [([0], 3, 128), ([0, 1, 2, 3], 3, 128), ([0, 1, 2], 2, 64), ([0, 1], 1, 64), ([0, 1, 2], 3, 192),
             ([0, 1, 2, 3], 3, 64)]


@pytest.mark.parametrize("in1,lmax,C", RTP_CASES)
@pytest.mark.parametrize("sorted_edges", [True, False])
def test_edge_rtp_matches_oracle(cuda, in1, lmax, C, sorted_edges):
    g = torch.Generator().manual_seed(7 * C + lmax + len(in1) + int(sorted_edges))
    Nn, E = 37, 700
    ei = _graph(g, Nn, E, sorted_edges)
    tp, x, y, h, W = _case(g, in1, lmax, C, E, Nn)
    alpha = 0.125
    xo, yo, ho = (t.double().requires_grad_(True) for t in (x, y, h))
    out_o = tp(xo, yo, alpha * ho @ W.double(), ei)
    go = torch.randn(out_o.shape, generator=g, dtype=torch.float64).float()
    gx_o, gy_o, gh_o = torch.autograd.grad((out_o * go.double()).sum(), [xo, yo, ho])

    var = ops.find_variant(ops.variant_key("uvu", in1, list(range(lmax + 1)), list(range(lmax + 1))))
    plan = ops.EdgePlan.from_edge_index(ei.to(cuda), Nn)
    assert (plan.eid is None) == sorted_edges
    xg, yg, hg = (t.to(cuda).requires_grad_(True) for t in (x, y, h))
    out = ops.edge_rtp_scatter(xg, yg, hg, W.to(cuda), alpha, plan, var, C)
    close(out, out_o, "out")
    gx, gy, gh = torch.autograd.grad((out * go.to(cuda)).sum(), [xg, yg, hg])
    close(gx, gx_o, "grad_x")
    close(gy, gy_o, "grad_y")
    close(gh, gh_o, "grad_h")


@pytest.mark.parametrize("layout", [0, 3])
def test_edge_rtp_equals_unfused_path(cuda, layout):
    """Same outputs and gradients as the last layer on its own kernel followed
    by ``edge_tp_scatter``, with a permuted feature-row order and grouped
    layouts; the per-edge weight gradient equals the unfused grad_w."""
    g = torch.Generator().manual_seed(3 + layout)
    in1, lmax, C, Nn, E = [0, 1, 2, 3], 3, 128, 53, 1500
    ei = _graph(g, Nn, E, False).to(cuda)
    _, x, y, h, W = _case(g, in1, lmax, C, E, Nn)
    x, y, h, W = (t.to(cuda) for t in (x, y, h, W))
    alpha = 0.5
    var = ops.find_variant(ops.variant_key("uvu", in1, list(range(lmax + 1)), list(range(lmax + 1))))
    plan = ops.EdgePlan.from_edge_index(ei, Nn)
    perm = torch.randperm(Nn, generator=g).to(cuda)
    node_map = torch.empty_like(perm)
    node_map[perm] = torch.arange(Nn, device=cuda)
    node_map = node_map.to(torch.int32)
    go = torch.randn(Nn, C * var.dout, generator=g).to(cuda)

    xa, ya, ha = (t.clone().requires_grad_(True) for t in (x, y, h))
    out_a = ops.edge_tp_scatter(xa, ya, ops.radial_mlp_out(ha, W, alpha), plan, var, C, layout, node_map)
    gxa, gya, gha = torch.autograd.grad((out_a * go).sum(), [xa, ya, ha])
    xb, yb, hb = (t.clone().requires_grad_(True) for t in (x, y, h))
    out_b = ops.edge_rtp_scatter(xb, yb, hb, W, alpha, plan, var, C, layout, node_map)
    gxb, gyb, ghb = torch.autograd.grad((out_b * go).sum(), [xb, yb, hb])
    close(out_b, out_a, "out")
    close(gxb, gxa, "grad_x")
    close(gyb, gya, "grad_y")
    close(ghb, gha, "grad_h")
    # the per-edge weight gradient itself
    w = ops.radial_mlp_out(h, W, alpha).requires_grad_(True)
    (gw_a,) = torch.autograd.grad((ops.edge_tp_scatter(x, y, w, plan, var, C, layout, node_map) * go).sum(), [w])
    _, _, gw_b = ops.launch_edge_rtp_bwd(x, y, h, W, alpha, go, plan, var, C, layout, node_map, False)
    close(gw_b, gw_a, "grad_w")


def test_edge_rtp_repeats_bit_for_bit(cuda):
    g = torch.Generator().manual_seed(1)
    in1, lmax, C, Nn, E = [0, 1, 2, 3], 3, 128, 60, 2000
    ei = _graph(g, Nn, E, False).to(cuda)
    _, x, y, h, W = _case(g, in1, lmax, C, E, Nn)
    x, y, h, W = (t.to(cuda) for t in (x, y, h, W))
    var = ops.find_variant(ops.variant_key("uvu", in1, list(range(lmax + 1)), list(range(lmax + 1))))
    plan = ops.EdgePlan.from_edge_index(ei, Nn)
    go = torch.randn(Nn, C * var.dout, generator=g).to(cuda)
    runs = []
    for _ in range(2):
        out = ops.launch_edge_rtp_fwd(x, y, h, W, 0.25, plan, var, C)
        runs.append((out,) + ops.launch_edge_rtp_bwd(x, y, h, W, 0.25, go, plan, var, C))
    for a, b in zip(*runs):
        assert torch.equal(a, b)


def test_edge_rtp_rejects_unsupported(cuda):
    var = ops.find_variant(ops.variant_key("uvu", [0, 1], [0, 1], [0, 1]))
    plan = ops.EdgePlan.from_edge_index(torch.tensor([[0, 1], [1, 0]], device=cuda), 2)
    x = torch.zeros(2, 96 * var.d1, device=cuda)
    with pytest.raises(ValueError):
        ops.edge_rtp_scatter(x, torch.zeros(2, var.d2, device=cuda), torch.zeros(2, 64, device=cuda),
                             torch.zeros(64, 96 * var.npath, device=cuda), 1.0, plan, var, 96)
