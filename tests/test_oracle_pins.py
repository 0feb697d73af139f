"""Pins of the CPU oracle (CPU only).

Each part of the oracle is checked against something that does not depend on
its own formulas: an independent implementation, a closed form, a symmetry or
a reference-held constant.  The reference's own tests hold no golden vectors
for this path; the activation constants (tace/models/mlp.py:34,43,52, pinned
to e3nn by tests/test_o2.py:360-377 of the reference) are the reference-held
fixtures used here.
"""

import itertools
import math

import numpy as np
import pytest
import torch

from oracle import model as om
from oracle import neighbours as onl
from oracle import so3 as oso3
from tace_amd import so3 as pso3
from tace_amd import structures


def _rot(seed):
    q = np.random.default_rng(seed).normal(size=4)
    q /= np.linalg.norm(q)
    w, x, y, z = q
    return np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - z * w), 2 * (x * z + y * w)],
                     [2 * (x * y + z * w), 1 - 2 * (x * x + z * z), 2 * (y * z - x * w)],
                     [2 * (x * z - y * w), 2 * (y * z + x * w), 1 - 2 * (x * x + y * y)]])


def _sh_np(lmax, v):
    return oso3.spherical_harmonics(lmax, torch.as_tensor(v, dtype=torch.float64)).numpy()


def _wigner_D(l, R):
    """D^l(R) fitted from SH values: Y^l(R v) = D^l Y^l(v)."""
    v = np.random.default_rng(7).normal(size=(64, 3))
    v /= np.linalg.norm(v, axis=1, keepdims=True)
    a = _sh_np(l, v)[:, l * l:(l + 1) ** 2]
    b = _sh_np(l, v @ R.T)[:, l * l:(l + 1) ** 2]
    D, *_ = np.linalg.lstsq(a, b, rcond=None)
    return D.T


# ------------------------------------------------------------------ W3j ----
TRIPLES = [(a, b, c) for a, b, c in itertools.product(range(5), repeat=3) if abs(a - b) <= c <= a + b]


@pytest.mark.parametrize("l1,l2,l3", TRIPLES)
def test_w3j_two_independent_implementations_agree(l1, l2, l3):
    # oracle: sympy Clebsch-Gordan; product: own Racah-formula code
    np.testing.assert_allclose(oso3.wigner_3j(l1, l2, l3), pso3.wigner_3j(l1, l2, l3), atol=1e-14)


def test_w3j_closed_forms():
    np.testing.assert_allclose(oso3.wigner_3j(1, 1, 0)[:, :, 0], np.eye(3) / math.sqrt(3), atol=1e-15)
    eps = np.zeros((3, 3, 3))
    for i, j, k in itertools.permutations(range(3)):
        eps[i, j, k] = np.linalg.det(np.eye(3)[[i, j, k]])
    np.testing.assert_allclose(oso3.wigner_3j(1, 1, 1), eps / math.sqrt(6), atol=1e-15)
    for l in range(5):
        np.testing.assert_allclose(oso3.wigner_3j(l, 0, l)[:, 0, :], np.eye(2 * l + 1) / math.sqrt(2 * l + 1),
                                   atol=1e-15)
        np.testing.assert_allclose(oso3.wigner_3j(0, l, l)[0], np.eye(2 * l + 1) / math.sqrt(2 * l + 1), atol=1e-15)


@pytest.mark.parametrize("l1,l2,l3", [t for t in TRIPLES if max(t) <= 3])
def test_w3j_invariant_under_rotation(l1, l2, l3):
    R = _rot(3)
    C = oso3.wigner_3j(l1, l2, l3)
    D1, D2, D3 = _wigner_D(l1, R), _wigner_D(l2, R), _wigner_D(l3, R)
    np.testing.assert_allclose(np.einsum("ijk,ai,bj,ck->abc", C, D1, D2, D3), C, atol=1e-10)


def test_w3j_orthogonality():
    for l1, l2 in itertools.product(range(4), repeat=2):
        for l3 in range(abs(l1 - l2), l1 + l2 + 1):
            C = oso3.wigner_3j(l1, l2, l3)
            G = np.einsum("ijk,ijm->km", C, C)
            np.testing.assert_allclose(G, np.eye(2 * l3 + 1) / (2 * l3 + 1), atol=1e-13)


# ------------------------------------------------------------------- SH ----
def test_sh_component_normalisation_and_l1():
    v = np.random.default_rng(0).normal(size=(32, 3))
    u = v / np.linalg.norm(v, axis=1, keepdims=True)
    Y = _sh_np(4, u)
    np.testing.assert_allclose(Y[:, 1:4], math.sqrt(3) * u, atol=1e-15)
    for l in range(5):
        np.testing.assert_allclose((Y[:, l * l:(l + 1) ** 2] ** 2).sum(1), 2 * l + 1, atol=1e-12)


def test_sh_homogeneous_polynomials():
    v = np.random.default_rng(1).normal(size=(8, 3))
    for s in (0.3, 2.7):
        Y1, Ys = _sh_np(3, v), _sh_np(3, s * v)
        for l in range(4):
            np.testing.assert_allclose(Ys[:, l * l:(l + 1) ** 2], s ** l * Y1[:, l * l:(l + 1) ** 2], rtol=1e-12)


def test_sh_oracle_recursion_equals_generated_closed_forms():
    """The kernels' SH (closed-form polynomials emitted by the code generator)
    equal the oracle's SH built from the W3j recursion, off the sphere too."""
    import sympy as sp

    from tace_amd.csrc.codegen import _sh_polys

    (x, y, z), polys = _sh_polys(3)
    flat = [e for blk in polys for e in blk]
    f = sp.lambdify((x, y, z), flat, "numpy")
    v = np.random.default_rng(2).normal(size=(16, 3)) * 1.7
    mine = np.stack([np.broadcast_to(np.asarray(c, dtype=float), (16,)) for c in f(v[:, 0], v[:, 1], v[:, 2])], 1)
    np.testing.assert_allclose(mine, _sh_np(3, v), rtol=1e-12, atol=1e-12)
    for e in flat:  # harmonic
        assert sp.simplify(sp.diff(e, x, 2) + sp.diff(e, y, 2) + sp.diff(e, z, 2)) == 0


def test_sh_wigner_D_is_a_representation():
    R1, R2 = _rot(11), _rot(12)
    for l in range(4):
        D1, D2, D12 = _wigner_D(l, R1), _wigner_D(l, R2), _wigner_D(l, R1 @ R2)
        np.testing.assert_allclose(D1 @ D1.T, np.eye(2 * l + 1), atol=1e-10)
        np.testing.assert_allclose(D12, D1 @ D2, atol=1e-10)
    np.testing.assert_allclose(_wigner_D(1, R1), R1, atol=1e-12)  # l=1 block is the rotation itself


# ------------------------------------------------------ activations/radial ----
def test_normalize2mom_constants_match_reference_literals():
    # tace/models/mlp.py:34 (silu), :43 (sigmoid), :52 (tanh)
    assert om.normalize2mom_cst("silu") == 1.6791767923989418
    assert om.normalize2mom_cst("sigmoid") == 1.8467055342154763
    # tanh is off this path; its last bit depends on the host's reduction order
    assert abs(om.normalize2mom_cst("tanh") - 1.5937334472592695) < 1e-15


def test_radial_basis_closed_form_and_envelope():
    torch.set_default_dtype(torch.float64)
    try:
        rb = om.RadialBasis(cutoff=1.0, num_basis=3, p=5).double()
        r = torch.tensor([[0.2], [0.7], [1.0], [1.3]])
        got = rb(r).numpy()
    finally:
        torch.set_default_dtype(torch.float32)
    rr = r.numpy()
    x = rr
    env = 1 - 21 * x ** 5 + 35 * x ** 6 - 15 * x ** 7
    want = math.sqrt(2.0) * np.sin(np.pi * np.arange(1, 4) * rr) / rr * env * (rr < 1.0)
    np.testing.assert_allclose(got, want, atol=1e-14)
    # C2 envelope: f(1) = f'(1) = f''(1) = 0, f(0) = 1
    f = np.polynomial.Polynomial([1, 0, 0, 0, 0, -21, 35, -15])
    assert abs(f(1.0)) < 1e-13 and abs(f.deriv()(1.0)) < 1e-12 and abs(f.deriv(2)(1.0)) < 1e-11 and f(0.0) == 1


# ------------------------------------------------------------- neighbours ----
@pytest.mark.parametrize("which", ["si", "fcc", "tri", "water_small"])
def test_neighbour_list_two_brute_forces_agree(which):
    rng = np.random.default_rng(4)
    if which == "si":
        s, rc = structures.si_diamond(seed=1), 5.0
    elif which == "fcc":
        s, rc = structures.fcc_alloy(reps=(3, 3, 2), seed=2), 5.0
    elif which == "tri":
        s, rc = structures.random_crystal(rng, 12, [1, 8, 26]), 6.0
    else:
        s, rc = structures.water_box(n_side=3, box=9.3, seed=3), 6.0
    a = onl.neighbour_list(s["positions"], s["cell"], s["pbc"], rc)
    b = onl.neighbour_list_numpy(s["positions"], s["cell"], s["pbc"], rc, nimg=4)
    np.testing.assert_array_equal(a[0], b[0])
    np.testing.assert_array_equal(a[1], b[1])
    # (i, j, S) <-> (j, i, -S)
    fwd = set(zip(a[0][0], a[0][1], *a[1].T))
    assert fwd == set(zip(a[0][1], a[0][0], *(-a[1]).T))


@pytest.mark.parametrize("kind,rc,count", [("si", 5.0, 28), ("fcc", 5.0, 42), ("bcc", 5.0, 58)])
def test_neighbour_shell_counts_of_perfect_lattices(kind, rc, count):
    if kind == "si":
        s = structures.si_diamond(sigma=0.0)
    elif kind == "fcc":
        s = structures.fcc_alloy(reps=(3, 3, 3), sigma=0.0)
    else:
        s = structures.bcc_fe(reps=(4, 4, 4), sigma=0.0)
    ei, _ = onl.neighbour_list(s["positions"], s["cell"], s["pbc"], rc)
    assert np.all(np.bincount(ei[1], minlength=len(s["positions"])) == count)


# ------------------------------------------------------ tensor products ----
def test_uvu_tp_equivariance_and_component_normalisation():
    torch.manual_seed(0)
    C, lmax = 4, 3
    in1 = [(C, (l, (-1) ** l)) for l in range(lmax + 1)]
    sh = oso3.sh_irreps(lmax)
    tp = om.ScatterTP(in1, sh, [(1, (l, (-1) ** l)) for l in range(lmax + 1)])
    n = 3
    x = torch.randn(n, oso3.irreps_dim(in1), dtype=torch.float64)
    v = torch.randn(n, 3, dtype=torch.float64)
    Y = oso3.spherical_harmonics(lmax, v / v.norm(dim=1, keepdim=True))
    w = torch.randn(n, tp.weight_numel, dtype=torch.float64)
    ei = torch.stack([torch.arange(n), torch.arange(n)])
    out = tp(x, Y, w, ei)
    R = _rot(5)
    Ds = {l: torch.as_tensor(_wigner_D(l, R)) for l in range(lmax + 1)}

    def rot(feat, irreps):
        cols, o = [], 0
        for m, (l, _) in irreps:
            d = 2 * l + 1
            cols.append((feat[:, o:o + m * d].reshape(-1, m, d) @ Ds[l].T).reshape(-1, m * d))
            o += m * d
        return torch.cat(cols, 1)

    Yr = oso3.spherical_harmonics(lmax, (v @ torch.as_tensor(R).T) / v.norm(dim=1, keepdim=True))
    out_r = tp(rot(x, in1), Yr, w, ei)
    torch.testing.assert_close(out_r, rot(out, tp.out), atol=1e-10, rtol=1e-10)
    # component normalisation: unit second moment per output component for
    # unit-variance inputs and weights (e3nn irrep_normalization="component")
    n = 20000
    g = torch.Generator().manual_seed(1)
    x = torch.randn(n, oso3.irreps_dim(in1), dtype=torch.float64, generator=g)
    yv = torch.randn(n, 16, dtype=torch.float64, generator=g)
    w = torch.randn(n, tp.weight_numel, dtype=torch.float64, generator=g)
    ei = torch.stack([torch.arange(n), torch.arange(n)])
    m2 = tp(x, yv, w, ei).pow(2).mean().item()
    assert abs(m2 - 1.0) < 0.05


# ------------------------------------------------------------ full model ----
def _si_setup(dtype=torch.float64, seed=0):
    from tace_amd import configs, data

    s = structures.si_diamond(seed=1)
    ei, S = onl.neighbour_list(s["positions"], s["cell"], s["pbc"], 5.0)
    cfg = configs.model_cfg("si64", [14], ei.shape[1] / 64, num_channel=8)
    torch.manual_seed(seed)
    m = om.TACE(cfg).to(dtype)
    for p in m.parameters():  # make the readout non-trivial
        p.data.mul_(1.0)
    d = data.collate([s], [(ei, S)], cfg["atomic_numbers"], dtype=dtype)
    return m, d, s


def test_model_forces_and_stress_match_finite_differences():
    m, d, _ = _si_setup()
    out = om.compute(m, d, forces=True, stress=True)
    F, S = out["forces"], out["stress"]
    assert abs(F.sum(0)).max() < 1e-12
    h = 1e-5
    for (a, k) in [(0, 0), (17, 1), (40, 2)]:
        dp, dm = d["positions"].clone(), d["positions"].clone()
        dp[a, k] += h
        dm[a, k] -= h
        ep = om.compute(m, {**d, "positions": dp}, forces=False)["energy"]
        em = om.compute(m, {**d, "positions": dm}, forces=False)["energy"]
        assert abs(-(ep - em).item() / (2 * h) - F[a, k].item()) < 1e-8
    # stress: strain both positions and cell, S = (1/V) dE/d(eps)
    vol = abs(np.linalg.det(d["lattice"][0].numpy()))
    for (i, j) in [(0, 0), (0, 1), (2, 2)]:
        eps = torch.zeros(3, 3, dtype=torch.float64)
        eps[i, j] += h / 2
        eps[j, i] += h / 2

        def e_of(sign):
            T = torch.eye(3, dtype=torch.float64) + sign * eps
            dd = {**d, "positions": d["positions"] @ T, "lattice": d["lattice"] @ T}
            return om.compute(m, dd, forces=False)["energy"].item()

        fd = (e_of(1) - e_of(-1)) / (2 * h) / vol
        assert abs(fd - S[0, i, j].item()) < 1e-8


def test_model_invariances():
    m, d, _ = _si_setup()
    out = om.compute(m, d, forces=True)
    R = torch.as_tensor(_rot(9))
    dr = {**d, "positions": d["positions"] @ R.T, "lattice": d["lattice"] @ R.T}
    out_r = om.compute(m, dr, forces=True)
    torch.testing.assert_close(out_r["energy"], out["energy"], rtol=1e-12, atol=1e-10)
    torch.testing.assert_close(out_r["forces"], out["forces"] @ R.T, rtol=1e-8, atol=1e-10)
    # translation
    dt = {**d, "positions": d["positions"] + torch.tensor([0.3, -1.1, 2.0], dtype=torch.float64)}
    torch.testing.assert_close(om.compute(m, dt, forces=False)["energy"], out["energy"], rtol=1e-12, atol=1e-10)


def test_model_fp32_tracks_fp64():
    m64, d64, _ = _si_setup(torch.float64)
    m32, d32, _ = _si_setup(torch.float32)
    m32.load_state_dict({k: v.to(torch.float32) if v.is_floating_point() else v for k, v in m64.state_dict().items()})
    o64 = om.compute(m64, d64, forces=True)
    o32 = om.compute(m32, d32, forces=True)
    assert abs((o32["energy"].double() - o64["energy"]) / o64["energy"]).max() < 1e-5
    assert (o32["forces"].double() - o64["forces"]).abs().max() < 1e-4
