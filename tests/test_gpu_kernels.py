"""Operator-level parity of the HIP kernels against the CPU oracle (GPU).

Tolerances: float64 to 1e-11 (relative to the largest magnitude), float32
to 2e-5 relative -- the kernels and the oracle sum in different orders.
"""

import itertools
import math

import numpy as np
import pytest
import torch

from oracle import model as om
from oracle import neighbours as onl
from oracle import so3 as oso3
from tace_amd import ops, structures

pytestmark = pytest.mark.gpu

TOL = {torch.float64: 1e-11, torch.float32: 2e-5}


def close(got, want, dtype, what=""):
    got = got.detach().double().cpu()
    want = want.detach().double().cpu()
    scale = max(want.abs().max().item(), 1e-30)
    err = (got - want).abs().max().item() / scale
    assert err < TOL[dtype], f"{what}: max rel err {err:.3e} (scale {scale:.3e})"


def _irreps(ls, C):
    return [(C, (l, (-1) ** l)) for l in ls]


# ------------------------------------------------------------ edge basis ----
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("lmax", [0, 1, 2, 3])
def test_edge_basis_matches_oracle(cuda, dtype, lmax):
    g = torch.Generator().manual_seed(lmax)
    E, rc, nb, p = 3000, 5.0, 8, 5
    d = torch.randn(E, 3, generator=g, dtype=torch.float64)
    d = d / d.norm(dim=1, keepdim=True) * (0.3 + 6.5 * torch.rand(E, 1, generator=g, dtype=torch.float64))
    vec = d.to(dtype).double().requires_grad_(True)  # same values the GPU sees
    torch.set_default_dtype(dtype)
    try:
        rb = om.RadialBasis(rc, nb, p).double()  # buffers built in the model dtype, as the reference does
    finally:
        torch.set_default_dtype(torch.float32)
    length = (vec ** 2).sum(1, keepdim=True).sqrt() + 1e-9
    R_o = rb(length)
    Y_o = oso3.spherical_harmonics(lmax, vec / length)
    gR = torch.randn(E, nb, generator=g, dtype=torch.float64)
    gY = torch.randn(E, (lmax + 1) ** 2, generator=g, dtype=torch.float64)
    (gv_o,) = torch.autograd.grad((R_o * gR).sum() + (Y_o * gY).sum(), vec)

    v = vec.detach().to(dtype).to(cuda).requires_grad_(True)
    bw = rb.radial_fn.bessel_weights.to(dtype).to(cuda)  # the oracle's own buffer
    R, Y = ops.edge_basis(v, bw, math.sqrt(2.0 / rc), rc, p, lmax)
    close(R, R_o, dtype, "radial")
    close(Y, Y_o, dtype, "sh")
    (gv,) = torch.autograd.grad((R * gR.to(dtype).to(cuda)).sum() + (Y * gY.to(dtype).to(cuda)).sum(), v)
    tol = {torch.float64: 1e-10, torch.float32: 1e-4}[dtype]
    err = ((gv.double().cpu() - gv_o).abs().max() / gv_o.abs().max()).item()
    assert err < tol, err


# ------------------------------------------------- edge tensor product ----
# channel counts cover one partial wavefront (16), several wavefronts per
# workgroup with a partial last one (96, 200) and the maximum (512)
TP_CASES = [([0], 2, 64), ([0], 3, 128), ([0, 1, 2], 2, 64), ([0, 1, 2, 3], 3, 128), ([0, 1, 2], 3, 64),
            ([0, 1], 1, 96), ([0, 1, 2, 3], 3, 200), ([0, 1], 1, 16), ([0, 1, 2, 3], 3, 512)]


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("in1,lmax,C", TP_CASES)
@pytest.mark.parametrize("sorted_edges", [True, False])
def test_edge_tp_scatter_matches_oracle(cuda, dtype, in1, lmax, C, sorted_edges):
    g = torch.Generator().manual_seed(C + lmax + len(in1))
    Nn, E = 37, 260
    src = torch.randint(0, Nn, (E,), generator=g)
    dst = torch.randint(0, Nn - 3, (E,), generator=g)  # the last receivers get no edges
    if sorted_edges:
        order = torch.argsort(dst, stable=True)
        src, dst = src[order], dst[order]
    ei = torch.stack([src, dst])
    tp = om.ScatterTP(_irreps(in1, C), oso3.sh_irreps(lmax), [(1, (l, (-1) ** l)) for l in range(lmax + 1)])
    x = torch.randn(Nn, oso3.irreps_dim(_irreps(in1, C)), generator=g, dtype=torch.float64).to(dtype).double()
    y = torch.randn(E, (lmax + 1) ** 2, generator=g, dtype=torch.float64).to(dtype).double()
    w = torch.randn(E, tp.weight_numel, generator=g, dtype=torch.float64).to(dtype).double()
    x.requires_grad_(True), y.requires_grad_(True), w.requires_grad_(True)
    out_o = tp(x, y, w, ei)
    go = torch.randn(out_o.shape, generator=g, dtype=torch.float64).to(dtype).double()
    gx_o, gy_o, gw_o = torch.autograd.grad((out_o * go).sum(), [x, y, w])

    key = ops.variant_key("uvu", in1, list(range(lmax + 1)), list(range(lmax + 1)))
    var = ops.find_variant(key)
    plan = ops.EdgePlan.from_edge_index(ei.to(cuda), Nn)
    assert (plan.eid is None) == sorted_edges
    xg, yg, wg = (t.detach().to(dtype).to(cuda).requires_grad_(True) for t in (x, y, w))
    out = ops.edge_tp_scatter(xg, yg, wg, plan, var, C)
    close(out, out_o, dtype, "out")
    gx, gy, gw = torch.autograd.grad((out * go.to(dtype).to(cuda)).sum(), [xg, yg, wg])
    close(gx, gx_o, dtype, "grad_x")
    close(gy, gy_o, dtype, "grad_y")
    close(gw, gw_o, dtype, "grad_w")


def test_edge_tp_forward_is_deterministic(cuda):
    g = torch.Generator().manual_seed(0)
    Nn, E, C = 50, 900, 128
    ei = torch.stack([torch.randint(0, Nn, (E,), generator=g), torch.randint(0, Nn, (E,), generator=g)]).to(cuda)
    var = ops.find_variant(ops.variant_key("uvu", [0, 1, 2, 3], [0, 1, 2, 3], [0, 1, 2, 3]))
    x = torch.randn(Nn, C * 16, generator=g).to(cuda)
    y = torch.randn(E, 16, generator=g).to(cuda)
    w = torch.randn(E, C * var.npath, generator=g).to(cuda)
    plan = ops.EdgePlan.from_edge_index(ei, Nn)
    a = ops.edge_tp_scatter(x, y, w, plan, var, C)
    b = ops.edge_tp_scatter(x, y, w, plan, var, C)
    assert torch.equal(a, b)


# ------------------------------------------------------------------ uuu ----
def _uuu_cases():
    out = []
    for L in (1, 2, 3):
        full = list(range(L + 1))
        nu2 = om.UUUTP(_irreps(full, 1), _irreps(full, 1), [(1, (l, (-1) ** l)) for l in full], True)
        nu2_ls = [ir[0] for _, ir in nu2.out]
        out.append((full, full, full))
        out.append((full, full, [0]))
        out.append((nu2_ls, full, full))
        out.append((nu2_ls, full, [0]))
    # a product whose backward runs in parts with summed grad_x2 partials
    out.append((nu2_ls, full, [0, 1, 2]))
    return out


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("in1,in2,outl", _uuu_cases())
def test_uuu_matches_oracle(cuda, dtype, in1, in2, outl):
    C = 64 if len(in1) > 8 else 96
    g = torch.Generator().manual_seed(len(in1) * 7 + len(outl))
    Nn = 29
    ident = in1 == in2
    tp = om.UUUTP(_irreps(in1, C), _irreps(in2, C), [(1, (l, (-1) ** l)) for l in outl], ident)
    x1 = torch.randn(Nn, oso3.irreps_dim(_irreps(in1, C)), generator=g, dtype=torch.float64).to(dtype).double()
    x2 = torch.randn(Nn, oso3.irreps_dim(_irreps(in2, C)), generator=g, dtype=torch.float64).to(dtype).double()
    x1.requires_grad_(True), x2.requires_grad_(True)
    o = tp(x1, x2)
    go = torch.randn(o.shape, generator=g, dtype=torch.float64).to(dtype).double()
    g1o, g2o = torch.autograd.grad((o * go).sum(), [x1, x2])
    var = ops.find_variant(ops.variant_key("uuu", in1, in2, outl))
    a, b = (t.detach().to(dtype).to(cuda).requires_grad_(True) for t in (x1, x2))
    out = ops.uuu_tp(a, b, var, C)
    close(out, o, dtype, "out")
    g1, g2 = torch.autograd.grad((out * go.to(dtype).to(cuda)).sum(), [a, b])
    close(g1, g1o, dtype, "g1")
    close(g2, g2o, dtype, "g2")


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("case", ["one_part", "parts", "identical"])
def test_uuu_backward_accumulate_adds_to_given_gradients(cuda, dtype, case):
    """tace_uuu_bwd's accumulate bits add grad_x1 / grad_x2 to what g1 / g2
    hold (the same bits as the overwriting call plus a separate add); with
    both bits and one array for g1 and g2 (a product of a tensor with
    itself) the array receives both gradients."""
    C, Nn, L = 64, 37, 3
    full = list(range(L + 1))
    nu2 = om.UUUTP(_irreps(full, 1), _irreps(full, 1), [(1, (l, (-1) ** l)) for l in full], True)
    nu2_ls = [ir[0] for _, ir in nu2.out]
    in1, outl = {"one_part": (full, full), "parts": (nu2_ls, [0, 1, 2]), "identical": (full, full)}[case]
    var = ops.find_variant(ops.variant_key("uuu", in1, full, outl))
    lay = ops.LAYOUT_ALL_GROUPED
    g = torch.Generator().manual_seed(11)
    mk = lambda n: torch.randn(Nn, n, generator=g, dtype=torch.float64).to(dtype).to(cuda)
    d1 = sum(C * (2 * l + 1) for l in in1)
    d2 = sum(C * (2 * l + 1) for l in full)
    x1, x2 = mk(d1), mk(d2)
    if case == "identical":
        x1 = x2
    go = mk(C * var.dout)
    g1, g2, _ = ops.launch_uuu_bwd(x1, x2, None, go, var, C, lay)
    if case == "identical":
        a = mk(d2)
        want = (a + g1) + g2
        got = a.clone()
        r1, r2, _ = ops.launch_uuu_bwd(x1, x2, None, go, var, C, lay, acc1=got, acc2=got)
        assert r1.data_ptr() == r2.data_ptr() == got.data_ptr()
        assert torch.equal(got, want)
        return
    a1, a2 = mk(d1), mk(d2)
    for acc in ((True, False), (False, True), (True, True)):
        t1 = a1.clone() if acc[0] else None
        t2 = a2.clone() if acc[1] else None
        r1, r2, _ = ops.launch_uuu_bwd(x1, x2, None, go, var, C, lay, acc1=t1, acc2=t2)
        assert torch.equal(r1, a1 + g1 if acc[0] else g1), acc
        assert torch.equal(r2, a2 + g2 if acc[1] else g2), acc
        if acc[0]:
            assert r1.data_ptr() == t1.data_ptr()
        if acc[1]:
            assert r2.data_ptr() == t2.data_ptr()


# ------------------------------------------------------------ neighbours ----
def _nl_cases():
    rng = np.random.default_rng(11)
    cases = [("si", structures.si_diamond(seed=1), 5.0),
             ("si_perfect", structures.si_diamond(sigma=0.0), 5.0),
             ("fcc", structures.fcc_alloy(reps=(4, 4, 3), seed=2), 5.0),
             ("bcc", structures.bcc_fe(reps=(5, 5, 5), seed=3), 5.0),
             ("water", structures.water_box(n_side=4, box=12.425, seed=4), 6.0)]
    for k in range(4):
        cases.append((f"tri{k}", structures.random_crystal(rng, int(rng.integers(4, 40)), [1, 8, 26]), 6.0))
    s = structures.si_diamond(seed=5)
    s = dict(s, positions=s["positions"] + np.array([7.0, -13.0, 30.0]))  # atoms far outside the cell
    cases.append(("shifted", s, 5.0))
    return cases


@pytest.mark.parametrize("name,s,rc", _nl_cases(), ids=[c[0] for c in _nl_cases()])
def test_neighbour_list_bit_exact_edge_set(cuda, name, s, rc):
    ei_o, S_o = onl.neighbour_list(s["positions"], s["cell"], s["pbc"], rc)
    pos = torch.as_tensor(np.asarray(s["positions"], dtype=np.float64), device=cuda)
    rowptr, src, sh = ops.neighbour_list(pos, s["cell"], s["pbc"], rc)
    n = len(s["positions"])
    counts = (rowptr[1:] - rowptr[:-1]).cpu().numpy()
    dst = np.repeat(np.arange(n), counts)
    src = src.cpu().numpy().astype(np.int64)
    sh = sh.cpu().numpy().astype(np.int64)
    got = sorted(zip(src.tolist(), dst.tolist(), map(tuple, sh.tolist())))
    want = sorted(zip(ei_o[0].tolist(), ei_o[1].tolist(), map(tuple, S_o.tolist())))
    assert len(got) == len(want)
    assert got == want
    # deterministic output order
    r2, s2, h2 = ops.neighbour_list(pos, s["cell"], s["pbc"], rc)
    assert torch.equal(r2, rowptr) and np.array_equal(s2.cpu().numpy(), src) and np.array_equal(h2.cpu().numpy(), sh)


@pytest.mark.parametrize("mode", [1, 2])
def test_neighbour_list_batch_equals_per_structure(cuda, mode):
    """The batched search (a thread or a wavefront per receiver) gives every
    structure's edges exactly as the single-structure search does, in the
    same order, with batch-global node ids; the batch mixes all the
    single-structure cases (skewed and shifted cells, a perfect lattice, tiny
    triclinic crystals), a non-periodic molecule and a one-atom cell."""
    structs = [s for _, s, _rc in _nl_cases()]
    mol = structures.water_box(n_side=2, box=6.2, seed=9)
    structs.append(dict(mol, pbc=[False, False, False], cell=np.eye(3) * 30.0))
    structs.append(dict(positions=np.array([[0.3, 0.2, 0.1]]), numbers=np.array([26]),
                        cell=np.eye(3) * 2.5, pbc=[True, True, True]))
    rc = 5.5
    sizes = [len(s["positions"]) for s in structs]
    pos = torch.as_tensor(np.concatenate([np.asarray(s["positions"], dtype=np.float64) for s in structs]),
                          device=cuda)
    rowptr, src, sh = ops.neighbour_list_batch(pos, sizes, [s["cell"] for s in structs],
                                               [s["pbc"] for s in structs], rc, mode=mode)
    a = 0
    for s, n in zip(structs, sizes):
        r1, s1, h1 = ops.neighbour_list(pos[a:a + n].contiguous(), s["cell"], s["pbc"], rc)
        e0, e1 = int(rowptr[a]), int(rowptr[a + n])
        assert torch.equal((rowptr[a:a + n + 1] - e0).cpu(), r1.cpu())
        assert torch.equal((src[e0:e1] - a).cpu(), s1.cpu())
        assert torch.equal(sh[e0:e1].cpu(), h1.cpu())
        a += n
    assert int(rowptr[-1]) == src.shape[0]


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("layout", [2, 3, 7])
@pytest.mark.parametrize("L", [2, 3])
def test_uuu_grouped_layouts_match_oracle(cuda, dtype, layout, L):
    """The group-major operand layouts (x1, out, x2) give the e3nn-layout results."""
    C = 64
    full = list(range(L + 1))
    nu2 = om.UUUTP(_irreps(full, 1), _irreps(full, 1), [(1, (l, (-1) ** l)) for l in full], True)
    nu2_ls = [ir[0] for _, ir in nu2.out]
    in1 = nu2_ls if layout & ops.LAYOUT_IN1_GROUPED else full
    tp = om.UUUTP(_irreps(in1, C), _irreps(full, C), [(1, (l, (-1) ** l)) for l in full], in1 == full)
    out_ls = [ir[0] for _, ir in tp.out]
    g = torch.Generator().manual_seed(L * 10 + layout)
    Nn = 23
    x1 = torch.randn(Nn, oso3.irreps_dim(_irreps(in1, C)), generator=g, dtype=torch.float64).to(dtype).double()
    x2 = torch.randn(Nn, oso3.irreps_dim(_irreps(full, C)), generator=g, dtype=torch.float64).to(dtype).double()
    x1.requires_grad_(True), x2.requires_grad_(True)
    o = tp(x1, x2)
    go = torch.randn(o.shape, generator=g, dtype=torch.float64).to(dtype).double()
    g1o, g2o = torch.autograd.grad((o * go).sum(), [x1, x2])
    var = ops.find_variant(ops.variant_key("uuu", in1, full, full))
    a = x1.detach().to(dtype).to(cuda)
    if layout & ops.LAYOUT_IN1_GROUPED:
        a = ops.to_grouped(a, in1, C)
    a.requires_grad_(True)
    b = x2.detach().to(dtype).to(cuda)
    if layout & ops.LAYOUT_IN2_GROUPED:
        b = ops.to_grouped(b, full, C)
    b.requires_grad_(True)
    out = ops.uuu_tp(a, b, var, C, layout)
    close(ops.from_grouped(out, out_ls, C), o, dtype, "out")
    gg = ops.to_grouped(go.to(dtype).to(cuda), out_ls, C)
    g1, g2 = torch.autograd.grad((out * gg).sum(), [a, b])
    if layout & ops.LAYOUT_IN1_GROUPED:
        g1 = ops.from_grouped(g1, in1, C)
    if layout & ops.LAYOUT_IN2_GROUPED:
        g2 = ops.from_grouped(g2, full, C)
    close(g1, g1o, dtype, "g1")
    close(g2, g2o, dtype, "g2")


def test_grouped_layout_helpers_roundtrip():
    x = torch.randn(5, 8 * (1 + 3 + 3 + 5), dtype=torch.float64)
    ls = [0, 1, 1, 2]
    torch.testing.assert_close(ops.from_grouped(ops.to_grouped(x, ls, 8), ls, 8), x, rtol=0, atol=0)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("in1,lmax,C", [([0], 3, 128), ([0, 1, 2, 3], 3, 128), ([0, 1, 2], 2, 64),
                                        ([0, 1, 2, 3], 3, 80)])
@pytest.mark.parametrize("layout", [1, 2, 3])
def test_edge_tp_grouped_layouts_match_oracle(cuda, dtype, in1, lmax, C, layout):
    """Group-major x / grad_x (IN1_GROUPED) and out / grad_out (OUT_GROUPED)
    give the e3nn-layout results."""
    g = torch.Generator().manual_seed(7 + C + layout)
    Nn, E = 31, 200
    ei = torch.stack([torch.randint(0, Nn, (E,), generator=g), torch.randint(0, Nn, (E,), generator=g)])
    tp = om.ScatterTP(_irreps(in1, C), oso3.sh_irreps(lmax), [(1, (l, (-1) ** l)) for l in range(lmax + 1)])
    out_ls = [ir[0] for _, ir in tp.out]
    x = torch.randn(Nn, oso3.irreps_dim(_irreps(in1, C)), generator=g, dtype=torch.float64).to(dtype).double()
    y = torch.randn(E, (lmax + 1) ** 2, generator=g, dtype=torch.float64).to(dtype).double()
    w = torch.randn(E, tp.weight_numel, generator=g, dtype=torch.float64).to(dtype).double()
    x.requires_grad_(True), y.requires_grad_(True), w.requires_grad_(True)
    out_o = tp(x, y, w, ei)
    go = torch.randn(out_o.shape, generator=g, dtype=torch.float64).to(dtype).double()
    gx_o, gy_o, gw_o = torch.autograd.grad((out_o * go).sum(), [x, y, w])
    var = ops.find_variant(ops.variant_key("uvu", in1, list(range(lmax + 1)), list(range(lmax + 1))))
    plan = ops.EdgePlan.from_edge_index(ei.to(cuda), Nn)
    gin = bool(layout & ops.LAYOUT_IN1_GROUPED)
    gout = bool(layout & ops.LAYOUT_OUT_GROUPED)
    x_dev = x.detach().to(dtype).to(cuda)
    xg = (ops.to_grouped(x_dev, in1, C) if gin else x_dev).requires_grad_(True)
    yg, wg = (t.detach().to(dtype).to(cuda).requires_grad_(True) for t in (y, w))
    out = ops.edge_tp_scatter(xg, yg, wg, plan, var, C, layout)
    close(ops.from_grouped(out, out_ls, C) if gout else out, out_o, dtype, "out")
    gg = go.to(dtype).to(cuda)
    gg = ops.to_grouped(gg, out_ls, C) if gout else gg
    gx, gy, gw = torch.autograd.grad((out * gg).sum(), [xg, yg, wg])
    close(ops.from_grouped(gx, in1, C) if gin else gx, gx_o, dtype, "grad_x")
    close(gy, gy_o, dtype, "grad_y")
    close(gw, gw_o, dtype, "grad_w")


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("two_graphs", [False, True])
@pytest.mark.parametrize("sorted_edges", [True, False])
def test_edge_vectors_and_position_gradient(cuda, dtype, two_graphs, sorted_edges):
    g = torch.Generator().manual_seed(3)
    Nn, E = 40, 500
    src = torch.randint(0, Nn, (E,), generator=g)
    dst = torch.randint(0, Nn, (E,), generator=g)
    if sorted_edges:
        o = torch.argsort(dst, stable=True)
        src, dst = src[o], dst[o]
    pos = torch.randn(Nn, 3, generator=g, dtype=torch.float64).to(dtype).double().requires_grad_(True)
    B = 2 if two_graphs else 1
    lat = (torch.eye(3, dtype=torch.float64) * 7 + torch.randn(B, 3, 3, generator=g, dtype=torch.float64)).to(dtype).double()
    lat.requires_grad_(True)
    batch = (torch.arange(Nn) >= Nn // 2).long() if two_graphs else torch.zeros(Nn, dtype=torch.long)
    sh = torch.randint(-1, 2, (E, 3), generator=g).double()
    eg = batch[src]
    ref = pos[dst] - pos[src] + torch.einsum("ni,nij->nj", sh, lat[eg])
    gv = torch.randn(E, 3, generator=g, dtype=torch.float64).to(dtype).double()
    gp_o, gl_o = torch.autograd.grad((ref * gv).sum(), [pos, lat])
    plan = ops.EdgePlan.from_edge_index(torch.stack([src, dst]).to(cuda), Nn)
    p = pos.detach().to(dtype).to(cuda).requires_grad_(True)
    L = lat.detach().to(dtype).to(cuda).requires_grad_(True)
    vec = ops.edge_vectors(p, L, sh.to(dtype).to(cuda), plan, dst.to(cuda), eg.to(cuda) if two_graphs else None)
    close(vec, ref, dtype, "vec")
    gp, gl = torch.autograd.grad((vec * gv.to(dtype).to(cuda)).sum(), [p, L])
    close(gp, gp_o, dtype, "grad_pos")
    close(gl, gl_o, dtype, "grad_lattice")


def test_slot_adapter_matches_oracle_with_unsorted_edges(cuda):
    """The plug-in-slot contract of fused.py:259-271 through tace_amd.slot."""
    from tace_amd import slot

    C, lmax = 64, 2
    node = "+".join(f"{C}x{l}{'e' if l % 2 == 0 else 'o'}" for l in range(lmax + 1))
    sh = "+".join(f"1x{l}{'e' if l % 2 == 0 else 'o'}" for l in range(lmax + 1))
    tp_h = slot.e3nnHipScatterTensorProduct(node, sh, node)
    tp_o = om.ScatterTP(oso3.parse_irreps(node), oso3.sh_irreps(lmax), oso3.parse_irreps(node))
    g = torch.Generator().manual_seed(9)
    Nn, E = 25, 300
    ei = torch.stack([torch.randint(0, Nn, (E,), generator=g), torch.randint(0, Nn, (E,), generator=g)])
    x = torch.randn(Nn, oso3.irreps_dim(oso3.parse_irreps(node)), generator=g, dtype=torch.float64)
    y = torch.randn(E, (lmax + 1) ** 2, generator=g, dtype=torch.float64)
    w = torch.randn(E, tp_o.weight_numel, generator=g, dtype=torch.float64)
    close(tp_h(x.to(cuda), y.to(cuda), w.to(cuda), ei.to(cuda)), tp_o(x, y, w, ei), torch.float64, "slot out")


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("layout", [0, 3])
def test_edge_tp_node_map_matches_identity_order(cuda, dtype, layout):
    """Features stored in a permuted row order (node_map[n] = row of node n)
    give the same per-node results and gradients as the identity order."""
    g = torch.Generator().manual_seed(11 + layout)
    Nn, E, C, in1, lmax = 41, 500, 96, [0, 1, 2, 3], 3
    ei = torch.stack([torch.randint(0, Nn, (E,), generator=g), torch.randint(0, Nn, (E,), generator=g)]).to(cuda)
    var = ops.find_variant(ops.variant_key("uvu", in1, list(range(lmax + 1)), list(range(lmax + 1))))
    plan = ops.EdgePlan.from_edge_index(ei, Nn)
    x = torch.randn(Nn, C * var.d1, generator=g, dtype=torch.float64).to(dtype).to(cuda)
    y = torch.randn(E, var.d2, generator=g, dtype=torch.float64).to(dtype).to(cuda)
    w = torch.randn(E, C * var.npath, generator=g, dtype=torch.float64).to(dtype).to(cuda)
    go = torch.randn(Nn, C * var.dout, generator=g, dtype=torch.float64).to(dtype).to(cuda)
    perm = torch.randperm(Nn, generator=g).to(cuda)          # row r holds node perm[r]
    node_map = torch.empty_like(perm)
    node_map[perm] = torch.arange(Nn, device=cuda)
    node_map = node_map.to(torch.int32)

    xa, ya, wa = (t.clone().requires_grad_(True) for t in (x, y, w))
    out_a = ops.edge_tp_scatter(xa, ya, wa, plan, var, C, 0)
    gxa, gya, gwa = torch.autograd.grad((out_a * go).sum(), [xa, ya, wa])

    out_ls = var_out_ls(var, in1, lmax)
    xs = x.index_select(0, perm)
    gos = go.index_select(0, perm)
    if layout:
        xs, gos = ops.to_grouped(xs, in1, C), ops.to_grouped(gos, out_ls, C)
    xb, yb, wb = (t.clone().requires_grad_(True) for t in (xs, y, w))
    out_b = ops.edge_tp_scatter(xb, yb, wb, plan, var, C, layout, node_map)
    gxb, gyb, gwb = torch.autograd.grad((out_b * gos).sum(), [xb, yb, wb])
    if layout:
        out_b, gxb = ops.from_grouped(out_b, out_ls, C), ops.from_grouped(gxb, in1, C)
    inv = node_map.long()
    close(out_b.index_select(0, inv), out_a, dtype, "out")
    close(gxb.index_select(0, inv), gxa, dtype, "grad_x")
    close(gyb, gya, dtype, "grad_y")
    close(gwb, gwa, dtype, "grad_w")


def var_out_ls(var, in1, lmax):
    tp = om.ScatterTP(_irreps(in1, 1), oso3.sh_irreps(lmax), [(1, (l, (-1) ** l)) for l in range(lmax + 1)])
    return [ir[0] for _, ir in tp.out]


# ------------------------------------------------------------ radial MLP ----
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("dims", [[8, 64, 64, 64, 2944], [8, 64, 64, 64, 1536], [10, 64, 96], [8, 64, 64, 64, 64, 7],
                                  [7, 64, 64, 30]])
def test_radial_mlp_matches_oracle(cuda, dtype, dims):
    """Fused width-64 hidden layers + last-layer GEMM against the oracle MLP (same weights)."""
    from tace_amd import model as pm
    torch.manual_seed(len(dims) + dims[-1])
    ref = om.MLP(dims).double()
    g = torch.Generator().manual_seed(dims[-1])
    E = 3001
    R = torch.randn(E, dims[0], generator=g, dtype=torch.float64).to(dtype).double().requires_grad_(True)
    out_o = ref(R)
    go = torch.randn(out_o.shape, generator=g, dtype=torch.float64)
    (gR_o,) = torch.autograd.grad((out_o * go).sum(), R)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(dtype)
    try:
        mlp = pm.MLP(dims)
    finally:
        torch.set_default_dtype(prev)
    mlp.load_state_dict({k: v.to(dtype) for k, v in ref.state_dict().items()})
    mlp = mlp.to(cuda)
    assert mlp.fused
    r = R.detach().to(dtype).to(cuda).requires_grad_(True)
    out = mlp(r)
    close(out, out_o, dtype, "mlp out")
    (gR,) = torch.autograd.grad((out * go.to(dtype).to(cuda)).sum(), r)
    close(gR, gR_o, dtype, "grad radial")


# --------------------------------------------------- per-species linears ----
def _element_linear_reference(x, W, b, irreps_in, irreps_out, species, alpha):
    """Per node: y_o = alpha (sum_{i -> o} pw x_i @ W[species](i, o) + bias[species]),
    in e3nn's o3.Linear instruction order (every pair of equal irreps,
    path weight (sum of mul_in into o)^-1/2), on [Z, 2l+1, mul] views."""
    from tace_amd.so3 import Irreps
    ii, io = Irreps(irreps_in), Irreps(irreps_out)
    Z = x.shape[0]

    # group-major: block of mul m, dim d starts at element Z * s
    def blocks(t, irr):
        out, s = [], 0
        for m, ir in irr:
            out.append(t.reshape(-1)[Z * s:Z * (s + m * ir.dim)].view(Z, ir.dim, m))
            s += m * ir.dim
        return out
    xb = blocks(x, ii)
    pairs = [(i, o) for i, (_, a) in enumerate(ii) for o, (_, q) in enumerate(io) if a == q]
    fan = {}
    for i, o in pairs:
        fan[o] = fan.get(o, 0) + ii[i][0]
    yb = [torch.zeros(Z, ir.dim, m, dtype=x.dtype) for m, ir in io]
    off = 0
    for i, o in pairs:
        mi, mo = ii[i][0], io[o][0]
        Ws = W[:, off:off + mi * mo].view(-1, mi, mo)[species]          # [Z, mi, mo]
        yb[o] = yb[o] + fan[o] ** -0.5 * torch.einsum("zdi,zio->zdo", xb[i], Ws)
        off += mi * mo
    boff = 0
    for o, (m, ir) in enumerate(io):
        if ir.l == 0 and ir.p == 1:
            yb[o] = yb[o] + b[:, boff:boff + m][species][:, None, :]
            boff += m
    return alpha * torch.cat([t.reshape(-1) for t in yb]).view(Z, -1)


SEG_CASES = [("8x0e+5x0e+6x1o+4x1o+3x2e", "70x0e+6x1o+65x2e+2x3o", [0, 1, 17, 64, 65, 3, 130, 0]),
             ("64x0e+36x0e+132x1o+20x2e", "260x0e+68x1o+40x2e", [140, 0, 3, 290, 1]),
             # long k into 256-wide blocks, and back (1100-wide gradient blocks)
             ("1100x0e+300x1o", "256x0e+256x1o", [0, 300, 7, 129]),
             # short k into wide blocks (the short-k task kernel: k 128, 100,
             # 20 and 8 into 300, 1100, 260 and 40 columns; a 513-wide block
             # no instruction writes), and back (k 100 and 64 into 1100 and
             # 300 columns)
             ("128x0e+100x1o+20x2e+8x3o", "300x0e+1100x1o+260x2e+40x3o+513x3e", [0, 300, 7, 129, 1]),
             ("1100x0e+300x1o", "100x0e+64x1o", [130, 0, 5, 256]),
             # the 64-row task kernel: k 200 and 256 into 300 and 700 columns
             ("200x0e+256x1o", "300x0e+700x1o", [70, 0, 3, 140])]


@pytest.mark.parametrize("dtype,tile,presplit", [(torch.float64, 64, False), (torch.float32, 128, True),
                                                (torch.float32, 128, False), (torch.float32, 64, False)])
@pytest.mark.parametrize("irr_in,irr_out,counts", SEG_CASES)
def test_seg_linear_matches_reference(cuda, dtype, tile, presplit, irr_in, irr_out, counts, monkeypatch):
    """One-launch per-species linear (tace_seg_linear) against an independent
    per-node restatement: several inputs into one output block (two 0e, two
    1o), a 65-wide block (two column tiles, one partial), an output block no
    instruction writes (3o: zeros), species with 0, 1, 17, 64, 65 and 130
    nodes; then wide, 4-aligned blocks with k tails (36, 20) over several
    128-row and 128-column tiles; forward with bias, then the input
    gradient."""
    from tace_amd import model as pm
    monkeypatch.setattr(pm, "SEG_LINEAR_TILE_F32", tile)
    monkeypatch.setattr(pm, "SEG_LINEAR_PRESPLIT", presplit)
    S, Z = len(counts), sum(counts)
    species = torch.repeat_interleave(torch.arange(S), torch.tensor(counts))
    attrs = torch.nn.functional.one_hot(species, S).to(dtype)
    g = torch.Generator().manual_seed(5)
    lin = pm.e3nnElementLinear(irr_in, irr_out, S).to(dtype)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(lin.weight.shape, generator=g, dtype=dtype))
        lin.bias.copy_(torch.randn(lin.bias.shape, generator=g, dtype=dtype))
    x = torch.randn(Z, lin.lay.dim_in, generator=g, dtype=dtype)
    go = torch.randn(Z, lin.lay.dim_out, generator=g, dtype=dtype)
    alpha = 0.7
    xr = x.clone().requires_grad_(True)
    want = _element_linear_reference(xr, lin.weight.detach(), lin.bias.detach(), irr_in, irr_out, species, alpha)
    (gx_want,) = torch.autograd.grad(want, xr, go)
    lin = lin.to(cuda)
    sp = pm.SpeciesPlan(attrs.to(cuda))
    assert len(sp.ranges) >= pm.SEG_LINEAR_MIN_RANGES[dtype]  # the segmented kernel runs
    for rep in range(2):   # second call: cached plan
        xg = x.to(cuda).requires_grad_(True)
        got = lin(xg, sp, alpha)
        (gx,) = torch.autograd.grad(got, xg, go.to(cuda))
        close(got, want, dtype, f"seg linear fwd (call {rep})")
        close(gx, gx_want, dtype, f"seg linear grad x (call {rep})")
    # the weight gradient (library GEMM path) next to the segmented forward
    xg = x.to(cuda)
    wr = lin.weight.detach().cpu().clone().requires_grad_(True)
    ref = _element_linear_reference(x, wr, lin.bias.detach().cpu(), irr_in, irr_out, species, alpha)
    (gw_want,) = torch.autograd.grad(ref, wr, go)
    (gw,) = torch.autograd.grad(lin(xg, sp, alpha), lin.weight, go.to(cuda))
    close(gw, gw_want, dtype, "seg linear grad w")


@pytest.mark.parametrize("dtype,tile,presplit,tfrag", [(torch.float64, 64, False, False),
                                                      (torch.float32, 128, True, True),
                                                      (torch.float32, 128, True, False),
                                                      (torch.float32, 128, False, False),
                                                      (torch.float32, 64, False, False)])
@pytest.mark.parametrize("irr_in,irr_out,counts", SEG_CASES)
def test_seg_linear_addend(cuda, dtype, tile, presplit, tfrag, irr_in, irr_out, counts, monkeypatch):
    """Every segmented-linear kernel (FMA tiles, the MFMA tile kernels with
    weights split in the launch, pre-split or in fragment order, and the
    short-k tasks) adds the addend to each output, forward and input
    gradient: into a separate output and in place (y += ...), equal to the
    separate sum up to rounding (the MFMA kernels start their sums from the
    addend instead of adding it at the end)."""
    from tace_amd import model as pm
    monkeypatch.setattr(pm, "SEG_LINEAR_TILE_F32", tile)
    monkeypatch.setattr(pm, "SEG_LINEAR_PRESPLIT", presplit)
    monkeypatch.setattr(ops, "SEG_TILE_FRAG", tfrag)
    S, Z = len(counts), sum(counts)
    species = torch.repeat_interleave(torch.arange(S), torch.tensor(counts))
    attrs = torch.nn.functional.one_hot(species, S).to(dtype).to(cuda)
    g = torch.Generator().manual_seed(21)
    lin = pm.e3nnElementLinear(irr_in, irr_out, S).to(dtype)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(lin.weight.shape, generator=g, dtype=dtype))
        lin.bias.copy_(torch.randn(lin.bias.shape, generator=g, dtype=dtype))
    lin = lin.to(cuda)
    sp = pm.SpeciesPlan(attrs)
    for kind, din, dout in (("fwd", lin.lay.dim_in, lin.lay.dim_out), ("bwd", lin.lay.dim_out, lin.lay.dim_in)):
        x = torch.randn(Z, din, generator=g, dtype=dtype).to(cuda)
        add = torch.randn(Z, dout, generator=g, dtype=dtype).to(cuda)
        rr, seg = pm._linear_route(x, lin.weight, lin.lay, sp.ranges)
        bias = lin.bias if kind == "fwd" else None
        y0 = pm._linear_apply(x, lin.weight, bias, lin.lay, rr, seg, 0.8, kind=kind)
        want = add + y0
        y1 = pm._linear_apply(x, lin.weight, bias, lin.lay, rr, seg, 0.8, kind=kind, addend=add)
        y2 = add.clone()
        pm._linear_apply(x, lin.weight, bias, lin.lay, rr, seg, 0.8, kind=kind, out=y2, addend=y2)
        for got, nm in ((y1, "separate"), (y2, "in place")):
            close(got, want, dtype, f"{kind} {nm}")
        if seg:   # the kernels take the addend as y itself or apart from y
            buf = torch.zeros(Z * dout + 1, dtype=dtype, device=cuda)
            with pytest.raises(ValueError, match="overlaps"):
                pm._linear_apply(x, lin.weight, bias, lin.lay, rr, seg, 0.8, kind=kind, out=buf[1:].view(Z, dout),
                                 addend=buf[:-1].view(Z, dout))


@pytest.mark.parametrize("irr_in,irr_out,counts", SEG_CASES)
def test_seg_linear_presplit_equals_in_kernel_split(cuda, irr_in, irr_out, counts, monkeypatch):
    """The pre-split weight planes (tace_bf16x3_split_blocks +
    tace_seg_linear_presplit) and the fragment-order weights
    (tace_seg_linear_presplit_frag, with B read from global memory) give the
    same bits as the kernel that splits the weights in every launch: the same
    bf16 terms, the same products in the same order.  After an in-place
    weight update the planes are rebuilt."""
    from tace_amd import model as pm
    monkeypatch.setattr(pm, "SEG_LINEAR_TILE_F32", 128)
    monkeypatch.setattr(ops, "SEG_SPLIT_SLOTS", None)   # split k sums in another order
    S, Z = len(counts), sum(counts)
    species = torch.repeat_interleave(torch.arange(S), torch.tensor(counts))
    attrs = torch.nn.functional.one_hot(species, S).float().to(cuda)
    g = torch.Generator().manual_seed(9)
    lin = pm.e3nnElementLinear(irr_in, irr_out, S)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(lin.weight.shape, generator=g) * 3.0)
        lin.bias.copy_(torch.randn(lin.bias.shape, generator=g))
    lin = lin.to(cuda)
    sp = pm.SpeciesPlan(attrs)
    x = torch.randn(Z, lin.lay.dim_in, generator=g).to(cuda).requires_grad_(True)
    go = torch.randn(Z, lin.lay.dim_out, generator=g).to(cuda)
    for step in range(2):
        outs = {}
        for presplit, tfrag in ((False, False), (True, False), (True, True)):
            monkeypatch.setattr(pm, "SEG_LINEAR_PRESPLIT", presplit)
            monkeypatch.setattr(ops, "SEG_TILE_FRAG", tfrag)
            y = lin(x, sp, 0.9)
            (gx,) = torch.autograd.grad(y, x, go)
            outs[(presplit, tfrag)] = (y.detach(), gx)
        for key in ((True, False), (True, True)):
            assert torch.equal(outs[key][0], outs[(False, False)][0]), f"forward differs {key} (step {step})"
            assert torch.equal(outs[key][1], outs[(False, False)][1]), f"input gradient differs {key} (step {step})"
        with torch.no_grad():
            lin.weight.mul_(-0.5)   # a new weight version: the cached planes must be rebuilt


@pytest.mark.parametrize("irr_in,irr_out,counts", SEG_CASES)
def test_seg_linear_split_k(cuda, irr_in, irr_out, counts, monkeypatch):
    """The fragment-order tile kernel with each tile's k split over several
    workgroups (tace_seg_linear_presplit_frag_split: partial tiles, then
    their sum in split order with addend and bias) against the unsplit
    kernel, forward and input gradient, with and without an addend (in
    place): equal up to float32 summation order, the same bits on a repeat;
    tiles with two contributions stay unsplit."""
    from tace_amd import model as pm
    monkeypatch.setattr(pm, "SEG_LINEAR_TILE_F32", 128)
    monkeypatch.setattr(pm, "SEG_LINEAR_PRESPLIT", True)
    monkeypatch.setattr(ops, "SEG_TILE_FRAG", True)
    S, Z = len(counts), sum(counts)
    species = torch.repeat_interleave(torch.arange(S), torch.tensor(counts))
    attrs = torch.nn.functional.one_hot(species, S).float().to(cuda)
    g = torch.Generator().manual_seed(31)
    lin = pm.e3nnElementLinear(irr_in, irr_out, S)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(lin.weight.shape, generator=g))
        lin.bias.copy_(torch.randn(lin.bias.shape, generator=g))
    lin = lin.to(cuda)
    sp = pm.SpeciesPlan(attrs)
    n_split = 0
    for kind, din, dout in (("fwd", lin.lay.dim_in, lin.lay.dim_out), ("bwd", lin.lay.dim_out, lin.lay.dim_in)):
        x = torch.randn(Z, din, generator=g).to(cuda)
        add = torch.randn(Z, dout, generator=g).to(cuda)
        rr, seg = pm._linear_route(x, lin.weight, lin.lay, sp.ranges)
        bias = lin.bias if kind == "fwd" else None
        res = {}
        for target, steps in ((None, 8), (4096, 1)):
            monkeypatch.setattr(ops, "SEG_SPLIT_SLOTS", target)
            monkeypatch.setattr(ops, "SEG_SPLIT_MIN_STEPS", steps)
            if seg:
                n_split += lin.lay.seg_plan(kind, rr, Z, x, lin.weight, bias).splits > 1
            y = pm._linear_apply(x, lin.weight, bias, lin.lay, rr, seg, 0.8, kind=kind)
            y_again = pm._linear_apply(x, lin.weight, bias, lin.lay, rr, seg, 0.8, kind=kind)
            assert torch.equal(y, y_again), (kind, target)
            y_acc = add.clone()
            pm._linear_apply(x, lin.weight, bias, lin.lay, rr, seg, 0.8, kind=kind, out=y_acc, addend=y_acc)
            res[target] = (y, y_acc)
        close(res[4096][0], res[None][0], torch.float32, f"{kind} split k")
        close(res[4096][1], res[None][1], torch.float32, f"{kind} split k, addend in place")
    # every case but the first (two inputs into one output block in both
    # directions) has a direction with one contribution per tile
    if irr_in != SEG_CASES[0][0]:
        assert n_split > 0


def test_seg_linear_split_k_rejects_tiles_with_two_contributions(cuda, monkeypatch):
    """A tile with two contributions handed to the split-k entry point gets
    NaN in every output (the plan never splits such tiles); the other tiles
    of the launch are right."""
    from tace_amd import _native as N
    from tace_amd import model as pm
    monkeypatch.setattr(pm, "SEG_LINEAR_TILE_F32", 128)
    monkeypatch.setattr(pm, "SEG_LINEAR_PRESPLIT", True)
    monkeypatch.setattr(ops, "SEG_TILE_FRAG", True)
    monkeypatch.setattr(ops, "SEG_SPLIT_SLOTS", None)
    irr_in, irr_out, counts = "40x0e+72x0e+16x1o", "64x0e+32x1o", [150, 20]
    S, Z = len(counts), sum(counts)
    species = torch.repeat_interleave(torch.arange(S), torch.tensor(counts))
    attrs = torch.nn.functional.one_hot(species, S).float().to(cuda)
    g = torch.Generator().manual_seed(4)
    lin = pm.e3nnElementLinear(irr_in, irr_out, S)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(lin.weight.shape, generator=g))
    lin = lin.to(cuda)
    sp = pm.SpeciesPlan(attrs)
    x = torch.randn(Z, lin.lay.dim_in, generator=g).to(cuda)
    rr, seg = pm._linear_route(x, lin.weight, lin.lay, sp.ranges)
    assert seg
    plan = lin.lay.seg_plan("fwd", rr, Z, x, lin.weight, None)
    assert plan.tile_frag and plan.splits == 1 and plan.n_ks == 0
    want = pm._linear_apply(x, lin.weight, None, lin.lay, rr, seg, 1.0, kind="fwd")
    frag = lin.lay.split_weights("fwd", lin.weight, frag=True)[0]
    t = plan.tiles.cpu().numpy()
    multi = (t[:, 6] - t[:, 5]) > 1
    assert multi.any() and (~multi).any()
    y = torch.zeros_like(want)
    pe = plan.n_tiles * 2 * 16384
    partials = torch.empty(pe, device=cuda)
    N.check(N.lib().tace_seg_linear_presplit_frag_split(x.data_ptr(), y.data_ptr(), None, frag.data_ptr(), None,
                                                        plan.tiles.data_ptr(), plan.n_tiles,
                                                        plan.contribs.data_ptr(), int(plan.tile_aligned), 2,
                                                        partials.data_ptr(), pe, 1.0, N.stream_ptr(cuda)),
            "split k")
    torch.cuda.synchronize()
    yf = y.view(-1)
    for (ob, rows, n, c0, _b, cb, ce, _u) in t.tolist():
        idx = ob + torch.arange(rows, device=cuda)[:, None] * n + c0 + torch.arange(min(128, n - c0), device=cuda)
        if ce - cb > 1:
            assert torch.isnan(yf[idx]).all()
        else:
            close(yf[idx], want.view(-1)[idx], torch.float32, "one-contribution tile")
    with pytest.raises(RuntimeError, match="partials hold fewer"):
        N.check(N.lib().tace_seg_linear_presplit_frag_split(x.data_ptr(), y.data_ptr(), None, frag.data_ptr(), None,
                                                            plan.tiles.data_ptr(), plan.n_tiles,
                                                            plan.contribs.data_ptr(), 1, 2, partials.data_ptr(),
                                                            pe - 1, 1.0, N.stream_ptr(cuda)), "split k")


def test_seg_linear_f32_error_matches_float32_gemm(cuda):
    """The float32 segmented GEMM (three-term bfloat16 split on the bf16
    MFMA) against the float64 truth of the same float32 inputs, next to the
    error of a float32 CPU GEMM of those inputs: long k (2048, 1100) so that
    the rounding of the sums dominates, inputs spanning 2^-20 .. 2^20 so that
    a split that dropped the third term (a 16-bit significand) would be off by
    ~2^-17 instead of ~2^-24.  The forward and the input gradient."""
    from tace_amd import model as pm
    counts = [300, 5, 130]
    irr_in, irr_out = "2048x0e+1100x1o", "256x0e+192x1o"
    S, Z = len(counts), sum(counts)
    species = torch.repeat_interleave(torch.arange(S), torch.tensor(counts))
    attrs = torch.nn.functional.one_hot(species, S).float()
    g = torch.Generator().manual_seed(11)
    lin = pm.e3nnElementLinear(irr_in, irr_out, S, bias=False)

    def spread(shape):
        return (torch.randn(shape, generator=g, dtype=torch.float64)
                * torch.exp2(torch.randint(-20, 21, shape, generator=g).double())).float()
    with torch.no_grad():
        lin.weight.copy_(spread(lin.weight.shape))
    x, go = spread((Z, lin.lay.dim_in)), spread((Z, lin.lay.dim_out))
    w64 = lin.weight.detach().double()
    xr = x.double().requires_grad_(True)
    want = _element_linear_reference(xr, w64, torch.zeros(S, 256, dtype=torch.float64), irr_in, irr_out, species, 1.0)
    (gx_want,) = torch.autograd.grad(want, xr, go.double())
    xc = x.clone().requires_grad_(True)
    cpu = _element_linear_reference(xc, lin.weight.detach(), torch.zeros(S, 256), irr_in, irr_out, species, 1.0)
    (gx_cpu,) = torch.autograd.grad(cpu, xc, go)
    sp = pm.SpeciesPlan(attrs.to(cuda))
    xg = x.to(cuda).requires_grad_(True)
    got = lin.to(cuda)(xg, sp, 1.0)
    (gx,) = torch.autograd.grad(got, xg, go.to(cuda))

    def err(a, b):   # max |a - b| over the row's scale, per output row block
        a, b = a.detach().double().cpu(), b.detach().double()
        return ((a - b).abs().amax(1) / b.abs().amax(1).clamp_min(1e-300)).max().item()
    for what, gpu, ref, truth in (("fwd", got, cpu, want), ("grad x", gx, gx_cpu, gx_want)):
        e_gpu, e_cpu = err(gpu, truth), err(ref, truth)
        print(f"seg linear {what}: rel err {e_gpu:.3e} (float32 CPU GEMM {e_cpu:.3e})")
        assert e_gpu < 4 * e_cpu + 1e-7, f"{what}: {e_gpu:.3e} vs float32 GEMM {e_cpu:.3e}"


def test_mlp_out_f32_error_matches_float32_gemm(cuda):
    """The radial MLP's last layer (three-term bfloat16 split on the bf16
    MFMA) against the float64 truth of the same float32 inputs, next to a
    float32 CPU GEMM's error: inputs spanning 2^-20 .. 2^20, so that a split
    that dropped its third term (a 16-bit significand) would be off by ~2^-17
    instead of ~2^-24; a ragged edge count (not a multiple of 32 or of the
    1024-edge chunk) and a width that is not a multiple of 32 or 256; then
    the input gradient the same way."""
    g = torch.Generator().manual_seed(3)
    E, N = 2 * 1024 + 77, 600

    def spread(shape):
        return (torch.randn(shape, generator=g, dtype=torch.float64)
                * torch.exp2(torch.randint(-20, 21, shape, generator=g).double())).float()
    h, W = spread((E, 64)), spread((64, N))
    alpha = 0.37
    truth = alpha * (h.double() @ W.double())
    cpu = alpha * (h @ W)
    got = ops.launch_mlp_out_f32(h.to(cuda), W.to(cuda), alpha).double().cpu()

    def err(a):   # per-row max error over the row's scale
        return ((a.double() - truth).abs().amax(1) / truth.abs().amax(1).clamp_min(1e-300)).max().item()
    e_gpu, e_cpu = err(got), err(cpu)
    print(f"mlp out: rel err {e_gpu:.3e} (float32 CPU GEMM {e_cpu:.3e})")
    assert e_gpu < 4 * e_cpu + 1e-8, f"{e_gpu:.3e} vs float32 GEMM {e_cpu:.3e}"
    # the input gradient g_h = alpha g @ W^T (tace_radial_mlp_out_bwd_f32),
    # widths with a partial last 32-slab (600) and not a multiple of 4 (601)
    for n in (600, 601):
        Wn, gn = spread((64, n)), spread((E, n))
        truth = alpha * (gn.double() @ Wn.double().t())
        cpu = alpha * (gn @ Wn.t())
        got = ops.launch_mlp_out_bwd_f32(gn.to(cuda), Wn.to(cuda), alpha).double().cpu()
        e_gpu, e_cpu = err(got), err(cpu)
        print(f"mlp out grad h (n_out {n}): rel err {e_gpu:.3e} (float32 CPU GEMM {e_cpu:.3e})")
        assert e_gpu < 4 * e_cpu + 1e-8, f"grad h, n_out {n}: {e_gpu:.3e} vs float32 GEMM {e_cpu:.3e}"


# ------------------------------------------------------ segmented row sums ----
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("width", [1152, 37])
def test_rows_accumulate_matches_index_add(cuda, dtype, width):
    """tace_rows_accumulate (fixed-order segmented sums added into out) against
    index_add_: receiver-CSR segments with target rows, a sender CSR over all
    rows (empty segments included), and rows whose width is not a multiple
    of the vector length."""
    g = torch.Generator().manual_seed(width)
    E, Nr = 900, 120
    rows = torch.randn(E, width, generator=g, dtype=torch.float64)
    base = torch.randn(Nr, width, generator=g, dtype=torch.float64)
    src = torch.randint(0, Nr - 7, (E,), generator=g)          # rows >= Nr-7 get nothing
    want = base.clone().index_add_(0, src, rows)
    rp, slot = ops.sender_csr(src.to(cuda), Nr)
    got = ops.rows_accumulate(base.to(dtype).to(cuda), rows.to(dtype).to(cuda), rp, slot)
    close(got, want, dtype, "sender segments")
    # receiver-grouped segments written to permuted target rows
    counts = torch.randint(0, 15, (Nr,), generator=g)
    counts[3] = 0
    Eg = int(counts.sum())
    rows2 = torch.randn(Eg, width, generator=g, dtype=torch.float64)
    rowptr = torch.zeros(Nr + 1, dtype=torch.int64)
    rowptr[1:] = torch.cumsum(counts, 0)
    target = torch.randperm(Nr, generator=g)
    want2 = base.clone().index_add_(0, torch.repeat_interleave(target, counts), rows2)
    got2 = ops.rows_accumulate(base.to(dtype).to(cuda), rows2.to(dtype).to(cuda), rowptr.to(torch.int32).to(cuda),
                               None, target.to(torch.int32).to(cuda))
    close(got2, want2, dtype, "receiver segments")


# ------------------------------------------- TECE SO(2) GEMM under bf16 mixing ----
@pytest.mark.parametrize("ktiled", [False, True])
@pytest.mark.parametrize("m,k,n,bias,pad", [(5000, 96, 384, True, 0), (3000, 384, 384, True, 0),
                                            (2500, 768, 1152, True, 0), (2100, 1152, 768, False, 0),
                                            (4099, 256, 256, False, 0), (777, 100, 70, True, 0),
                                            (1500, 128, 96, False, 24), (33, 512, 192, False, 8),
                                            (300, 1000, 300, True, 4), (129, 40, 257, False, 0)])
def test_so2_gemm_bf16_matches_float32_product(cuda, m, k, n, bias, pad, ktiled):
    """``tace_so2_gemm_bf16`` and its k-tiled variant against the float32
    product of the same bf16 values (exact products, so only the order of the
    float32 sums differs): the SO(2) linear shapes of the TECE layer, k and n
    tails (k not a multiple of 32 or 64, n past a 256-column tile), rows past
    the last full tile, a row stride above k."""
    from tace_amd import ops
    g = torch.Generator().manual_seed(k + n)
    a_full = torch.randn(m, k + pad, generator=g).to(torch.bfloat16).to(cuda)
    a = a_full[:, :k]
    B = torch.randn(k, n, generator=g).to(torch.bfloat16).to(cuda)
    b = torch.randn(n, generator=g).to(cuda) if bias else None
    got = ops.so2_gemm_bf16(a, ops.bf16_fragment_order(B), n, k, b, ktiled=ktiled)
    want = a.float() @ B.float() + (b if bias else 0.0)
    scale = (a.float().abs() @ B.float().abs()).amax(1, keepdim=True) + 1e-30
    err = ((got - want).abs() / scale).max().item()
    assert got.shape == (m, n) and err < 2e-6, err


@pytest.mark.parametrize("fn", ["tace_so2_gemm_bf16", "tace_so2_gemm_bf16_kt"])
@pytest.mark.parametrize("n,ldo", [(6, 8), (70, 76), (33, 40)])
def test_so2_gemm_bf16_padded_output_rows_untouched(cuda, n, ldo, fn):
    """Through the C ABI with an output row stride above n: columns n..ldo-1
    of every row (a strided view's neighbours) keep their sentinel."""
    from tace_amd import _native as N
    m, k = 300, 96
    g = torch.Generator().manual_seed(n)
    a = torch.randn(m, k, generator=g).to(torch.bfloat16).to(cuda)
    B = torch.randn(k, n, generator=g).to(torch.bfloat16).to(cuda)
    bias = torch.randn(n, generator=g).to(cuda)
    bf = ops.bf16_fragment_order(B)
    out = torch.full((m, ldo), 12345.0, dtype=torch.float32, device=cuda)
    N.check(getattr(N.lib(), fn)(a.data_ptr(), k, bf.data_ptr(), bias.data_ptr(), out.data_ptr(), ldo, m, n, k,
                                 N.stream_ptr(a.device)), fn)
    torch.cuda.synchronize()
    assert bool((out[:, n:] == 12345.0).all()), "the kernel wrote past column n"
    want = a.float() @ B.float() + bias
    scale = (a.float().abs() @ B.float().abs()).amax(1, keepdim=True) + 1e-30
    assert ((out[:, :n] - want).abs() / scale).max().item() < 2e-6


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("k,n,bias", [(8, 8, True), (8, 8, False), (1, 64, True), (64, 3, False)])
def test_narrow_linear_matches_torch(cuda, dtype, k, n, bias):
    """``tace_narrow_linear`` (the TECE radial projection and its input
    gradient) against a float64 product, rows not a multiple of the block."""
    g = torch.Generator().manual_seed(k * 100 + n)
    x = torch.randn(1037, k, generator=g, dtype=torch.float64)
    m = torch.randn(k, n, generator=g, dtype=torch.float64)
    b = torch.randn(n, generator=g, dtype=torch.float64) if bias else None
    got = ops.narrow_linear(x.to(dtype).to(cuda), m.to(dtype).to(cuda), None if b is None else b.to(dtype).to(cuda))
    want = x @ m + (b if bias else 0.0)
    close(got, want, dtype, "narrow linear")
