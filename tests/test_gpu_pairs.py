"""Edge pairs and the pair-shared radial weights (GPU).

The two directions of an edge (i -> j with shift S, j -> i with -S) have the
same length, so the radial MLP's output is the same for both; the model makes
it once per pair.  Checked here: the pairing against the neighbour list's own
edge set (every edge of a full periodic list has exactly one reverse), the
rows of unpaired edges, and the product with pair rows against the product
with the same weights expanded to every edge (forward and input gradients
bit for bit, the h gradient to float rounding of the pair sum).
"""

import numpy as np
import pytest
import torch

from tace_amd import ops, structures

pytestmark = pytest.mark.gpu


def _nl(s, rc, cuda):
    pos = torch.as_tensor(s["positions"], dtype=torch.float64, device=cuda)
    rowptr, src, sh = ops.neighbour_list(pos, s["cell"], s["pbc"], rc)
    E = int(src.shape[0])
    return ops.EdgePlan(len(s["positions"]), E, rowptr, src, None), sh


@pytest.mark.parametrize("which", ["si", "water", "dense", "tiny_cell"])
def test_pairs_match_the_edge_set(cuda, which):
    if which == "si":
        s, rc = structures.si_diamond(seed=3), 5.0
    elif which == "water":
        s, rc = structures.water_box(n_side=4, box=49.7 / 16 * 4, seed=5), 6.0
    elif which == "dense":   # ~250 edges per receiver: several 64-edge runs, several 128-candidate rounds
        s, rc = structures.water_box(n_side=4, box=49.7 / 16 * 4, seed=6), 8.5
    else:   # self-images: edges i -> i with S != 0
        s, rc = structures.bcc_fe(reps=(1, 1, 1), seed=2), 5.0
    plan, sh = _nl(s, rc, cuda)
    pairs = plan.edge_pairs(sh)
    E = plan.n_edges
    assert pairs.n_rows * 2 == E
    rp = plan.rowptr.cpu().numpy()
    dst = np.repeat(np.arange(plan.n_nodes), np.diff(rp))
    src = plan.src.cpu().numpy()
    S = sh.cpu().numpy()
    ra, rb = pairs.row_edges.cpu().numpy(), pairs.row_partner.cpu().numpy()
    assert (rb >= 0).all() and (ra < rb).all()
    assert (src[ra] == dst[rb]).all() and (dst[ra] == src[rb]).all() and (S[ra] == -S[rb]).all()
    rows = pairs.w_rows.cpu().numpy()
    assert sorted(np.concatenate([ra, rb]).tolist()) == list(range(E))
    assert (rows[ra] == np.arange(pairs.n_rows)).all() and (rows[rb] == np.arange(pairs.n_rows)).all()


def test_unpaired_edges_get_their_own_rows(cuda):
    s = structures.si_diamond(seed=4)
    plan, sh = _nl(s, 5.0, cuda)
    # drop every 7th edge: its reverse loses its partner
    keep = torch.ones(plan.n_edges, dtype=torch.bool, device=cuda)
    keep[::7] = False
    rp = plan.rowptr.cpu().numpy()
    dst = torch.as_tensor(np.repeat(np.arange(plan.n_nodes), np.diff(rp)), device=cuda)
    ei = torch.stack([plan.src.long(), dst])[:, keep]
    sub = ops.EdgePlan.from_edge_index(ei, plan.n_nodes)
    pairs = sub.edge_pairs(sh[keep])
    E = sub.n_edges
    rb = pairs.row_partner.cpu().numpy()
    n_unpaired = int((rb < 0).sum())
    assert n_unpaired > 0 and pairs.n_rows == (E + n_unpaired) // 2
    rows = pairs.w_rows.cpu().numpy()
    assert sorted(set(rows.tolist())) == list(range(pairs.n_rows))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_pair_rows_equal_expanded_weights(cuda, dtype):
    s = structures.water_box(n_side=3, box=49.7 / 16 * 3, seed=6)
    plan, sh = _nl(s, 6.0, cuda)
    pairs = plan.edge_pairs(sh)
    C, lmax = 64, 3
    var = ops.find_variant(ops.variant_key("uvu", [0, 1, 2, 3], [0, 1, 2, 3], [0, 1, 2, 3]))
    g = torch.Generator().manual_seed(1)
    Nn, E = plan.n_nodes, plan.n_edges
    x = torch.randn(Nn, C * var.d1, generator=g, dtype=dtype).to(cuda).requires_grad_(True)
    y = torch.randn(E, var.d2, generator=g, dtype=dtype).to(cuda).requires_grad_(True)
    h = torch.randn(pairs.n_rows, 64, generator=g, dtype=dtype).to(cuda).requires_grad_(True)
    W = torch.randn(64, C * var.npath, generator=g, dtype=dtype).to(cuda)
    alpha = 0.125
    out = ops.edge_tp_scatter_pairs(x, y, h, W, alpha, plan, pairs, var, C)
    # reference: the same weights for every edge, as the per-edge path sees them
    hx = h.index_select(0, pairs.w_rows)
    w_all = ops.radial_mlp_out(hx, W, alpha)
    ref = ops.edge_tp_scatter(x, y, w_all, plan, var, C)
    go = torch.randn(out.shape, generator=g, dtype=dtype).to(cuda)
    gx, gy, gh = torch.autograd.grad(out, [x, y, h], go)
    rx, ry, rh = torch.autograd.grad(ref, [x, y, h], go)
    if dtype == torch.float32:
        # the same last-layer kernel makes the same rows: identical products
        assert torch.equal(out, ref)
        assert torch.equal(gx, rx) and torch.equal(gy, ry)
    else:
        # float64 makes w with a library GEMM whose blocking depends on the row count
        for a, b in ((out, ref), (gx, rx), (gy, ry)):
            assert ((a - b).abs().max() / b.abs().max()).item() < 1e-13
    tol = 1e-5 if dtype == torch.float32 else 1e-12
    err = ((gh - rh).abs().max() / rh.abs().max()).item()
    assert err < tol, err


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_self_and_duplicate_edges_get_their_own_rows(cuda, dtype):
    """A zero-shift self edge i -> i finds itself as its reverse, and a
    duplicated edge shares its reverse with the original: only mutual pairs
    share a row, every other edge gets its own, and the pair-row product
    still equals the product with the weights expanded to every edge."""
    s = structures.si_diamond(seed=4)
    plan, sh = _nl(s, 5.0, cuda)
    rp = plan.rowptr.cpu().numpy()
    dst = np.repeat(np.arange(plan.n_nodes), np.diff(rp))
    src = plan.src.cpu().numpy()
    S = sh.cpu().numpy()
    # extra edges: 3 -> 3 with S = 0, and copies of edges 10 and 25
    src2 = np.concatenate([src, [3, src[10], src[25]]])
    dst2 = np.concatenate([dst, [3, dst[10], dst[25]]])
    S2 = np.concatenate([S, [[0, 0, 0], S[10], S[25]]]).astype(S.dtype)
    order = np.argsort(dst2, kind="stable")
    ei = torch.as_tensor(np.stack([src2[order], dst2[order]]), device=cuda)
    sh2 = torch.as_tensor(S2[order], device=cuda)
    sub = ops.EdgePlan.from_edge_index(ei, plan.n_nodes)
    pairs = sub.edge_pairs(sh2)
    E = sub.n_edges
    ra, rb = pairs.row_edges.cpu().numpy(), pairs.row_partner.cpu().numpy()
    rows = pairs.w_rows.cpu().numpy()
    # the self edge and the two copies are unpaired (each original keeps its reverse)
    assert int((rb < 0).sum()) == 3 and pairs.n_rows == (E + 3) // 2
    assert sorted(set(rows.tolist())) == list(range(pairs.n_rows))
    owners = np.concatenate([ra, rb[rb >= 0]])
    assert sorted(owners.tolist()) == list(range(E))
    assert (rows[ra] == np.arange(pairs.n_rows)).all() and (rows[rb[rb >= 0]] == np.nonzero(rb >= 0)[0]).all()
    # the product through the pair rows equals the per-edge product
    C = 64
    var = ops.find_variant(ops.variant_key("uvu", [0, 1, 2], [0, 1, 2], [0, 1, 2]))
    g = torch.Generator().manual_seed(2)
    x = torch.randn(plan.n_nodes, C * var.d1, generator=g, dtype=dtype).to(cuda).requires_grad_(True)
    y = torch.randn(E, var.d2, generator=g, dtype=dtype).to(cuda).requires_grad_(True)
    h = torch.randn(pairs.n_rows, 64, generator=g, dtype=dtype).to(cuda).requires_grad_(True)
    W = torch.randn(64, C * var.npath, generator=g, dtype=dtype).to(cuda)
    out = ops.edge_tp_scatter_pairs(x, y, h, W, 0.125, sub, pairs, var, C)
    w_all = ops.radial_mlp_out(h.index_select(0, pairs.w_rows), W, 0.125)
    ref = ops.edge_tp_scatter(x, y, w_all, sub, var, C)
    go = torch.randn(out.shape, generator=g, dtype=dtype).to(cuda)
    grads = torch.autograd.grad(out, [x, y, h], go)
    refs = torch.autograd.grad(ref, [x, y, h], go)
    tol = 1e-5 if dtype == torch.float32 else 1e-12
    for a, b in zip((out,) + grads, (ref,) + refs):
        assert ((a - b).abs().max() / b.abs().max()).item() < tol
