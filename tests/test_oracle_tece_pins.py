"""Pins of the CPU restatement of the TECE convolution (oracle/tece.py).

None of these retypes the restated formulas: the frames are checked by what
they must do (map the edge onto +y, be rotations), the Wigner blocks by the
group law and by the spherical harmonics they must rotate (an independent
implementation), the SO(2) operations by their equivariance under rotations
about the edge axis, and the whole model by rotation / translation /
permutation invariance and finite differences.
"""

import math

import numpy as np
import pytest
import torch

from oracle import model as om
from oracle import neighbours as onl
from oracle import so3 as oso3
from oracle import tece
from tace_amd import configs, data, structures


def _rand_rot(g, n=1):
    q = torch.randn(n, 4, generator=g, dtype=torch.float64)
    q = q / q.norm(dim=1, keepdim=True)
    w, x, y, z = q.unbind(1)
    return torch.stack([
        torch.stack([1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)], -1),
        torch.stack([2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)], -1),
        torch.stack([2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)], -1)], -2)


def _directions(g, n=400):
    v = torch.randn(n, 3, generator=g, dtype=torch.float64) * (0.5 + 3 * torch.rand(n, 1, generator=g, dtype=torch.float64))
    poles = torch.tensor([[0, 1.0, 0], [0, -1.0, 0], [1e-9, 1.0, 0], [0, -1.0, 1e-8], [0.3, -2.0, 0.1],
                          [0.0, 0.0, 1.0], [1.0, 0.0, 0.0]], dtype=torch.float64)
    return torch.cat([v, poles])


def test_edge_frame_maps_edge_to_plus_y_and_is_a_rotation():
    g = torch.Generator().manual_seed(0)
    v = _directions(g)
    R = tece.edge_rotation(v)
    u = v / v.norm(dim=1, keepdim=True)
    I = torch.eye(3, dtype=torch.float64)
    torch.testing.assert_close(R @ R.transpose(1, 2), I.expand_as(R), rtol=0, atol=1e-12)
    torch.testing.assert_close(torch.linalg.det(R), torch.ones(len(v), dtype=torch.float64), rtol=0, atol=1e-12)
    torch.testing.assert_close((R @ u.unsqueeze(-1)).squeeze(-1),
                               torch.tensor([0.0, 1.0, 0.0], dtype=torch.float64).expand_as(u), rtol=0, atol=1e-7)


def test_smooth_step_is_the_cinf_blend():
    x = torch.tensor([-1.0, 0.0, 0.25, 0.5, 0.75, 1.0, 2.0], dtype=torch.float64)
    f = tece._smooth_step(x)
    a = lambda t: math.exp(-1 / t)
    ref = [0, 0, a(.25) / (a(.25) + a(.75)), 0.5, a(.75) / (a(.75) + a(.25)), 1, 1]
    torch.testing.assert_close(f, torch.tensor(ref, dtype=torch.float64), rtol=0, atol=1e-15)


@pytest.mark.parametrize("lmax", [2, 3])
def test_wigner_blocks_group_law_and_orthogonality(lmax):
    g = torch.Generator().manual_seed(lmax)
    R1, R2 = _rand_rot(g, 16), _rand_rot(g, 16)
    D1, D2, D12 = (tece.wigner_blocks(R, lmax) for R in (R1, R2, R1 @ R2))
    for l in range(lmax + 1):
        torch.testing.assert_close(D12[l], D1[l] @ D2[l], rtol=0, atol=1e-12)
        I = torch.eye(2 * l + 1, dtype=torch.float64).expand_as(D1[l])
        torch.testing.assert_close(D1[l] @ D1[l].transpose(1, 2), I, rtol=0, atol=1e-12)


@pytest.mark.parametrize("lmax", [2, 3])
def test_wigner_blocks_rotate_the_spherical_harmonics(lmax):
    """Y^l(R v) = D^l(R) Y^l(v), with Y from the oracle's SH (W3j recursion)."""
    g = torch.Generator().manual_seed(10 + lmax)
    R = _rand_rot(g, 32)
    v = torch.randn(32, 3, generator=g, dtype=torch.float64)
    v = v / v.norm(dim=1, keepdim=True)
    Y = oso3.spherical_harmonics(lmax, v)
    YR = oso3.spherical_harmonics(lmax, (R @ v.unsqueeze(-1)).squeeze(-1))
    for l, D in enumerate(tece.wigner_blocks(R, lmax)):
        sl = slice(l * l, (l + 1) ** 2)
        torch.testing.assert_close(YR[:, sl], (D @ Y[:, sl].unsqueeze(-1)).squeeze(-1), rtol=0, atol=1e-12)


def test_edge_frame_puts_the_edge_harmonics_on_m0():
    """In the edge frame the edge direction is +y, the SH polar axis: only
    the m = 0 rows of wigner . Y(edge) survive, and they equal Y(+y)."""
    g = torch.Generator().manual_seed(3)
    v = _directions(g)
    L = 3
    W, Winv = tece.edge_wigner(v, L, L)
    Y = oso3.spherical_harmonics(L, v / v.norm(dim=1, keepdim=True))
    Ym = (W @ Y.unsqueeze(-1)).squeeze(-1)
    Yy = oso3.spherical_harmonics(L, torch.tensor([[0.0, 1.0, 0.0]], dtype=torch.float64))[0]
    torch.testing.assert_close(Ym[:, :L + 1], Yy[[l * l + l for l in range(L + 1)]].expand(len(v), -1),
                               rtol=0, atol=2e-7)
    assert Ym[:, L + 1:].abs().max() < 2e-7
    torch.testing.assert_close(Winv @ W, torch.eye((L + 1) ** 2, dtype=torch.float64).expand(len(v), -1, -1),
                               rtol=0, atol=1e-12)


def _roll(x, mmax, lmax, theta, full):
    """Rotate m-layout features about the edge axis: (+m, -m) pairs turn by m*theta."""
    out = x.clone()
    n0 = lmax + 1
    off = n0
    for m in range(1, mmax + 1):
        n = lmax + 1 if full else lmax + 1 - m
        re, im = x[:, off:off + n], x[:, off + n:off + 2 * n]
        c, s = math.cos(m * theta), math.sin(m * theta)
        out[:, off:off + n] = c * re - s * im
        out[:, off + n:off + 2 * n] = s * re + c * im
        off += 2 * n
    return out


def test_so2_linear_and_complex_product_commute_with_edge_axis_rotations():
    torch.manual_seed(0)
    mmax = lmax = 2
    lin = tece.SO2Linear(mmax, lmax, 6, 5).double()
    x = torch.randn(7, 9, 6, dtype=torch.float64)
    th = 0.731
    torch.testing.assert_close(lin(_roll(x, mmax, lmax, th, False)), _roll(lin(x), mmax, lmax, th, False),
                               rtol=0, atol=1e-12)
    full = tece.SO2Linear(mmax, lmax, 6, 4, nout=[3, 3, 3]).double()
    torch.testing.assert_close(full(_roll(x, mmax, lmax, th, False)), _roll(full(x), mmax, lmax, th, True),
                               rtol=0, atol=1e-12)
    cp = tece.ComplexProduct(mmax, lmax, 4)
    a, b = torch.randn(7, 15, 4, dtype=torch.float64), torch.randn(7, 15, 4, dtype=torch.float64)
    w = torch.randn(7, cp.weight_numel, dtype=torch.float64)
    torch.testing.assert_close(cp(_roll(a, mmax, lmax, th, True), _roll(b, mmax, lmax, th, True), w),
                               _roll(cp(a, b, w), mmax, lmax, th, True), rtol=0, atol=1e-12)


def test_graph_softmax_normalises_per_receiver_and_ignores_offsets():
    g = torch.Generator().manual_seed(4)
    dst = torch.randint(0, 9, (200,), generator=g)
    s = 5 * torch.randn(200, 4, generator=g, dtype=torch.float64)
    a = tece.graph_softmax(s, dst, 12)
    tot = torch.zeros(12, 4, dtype=torch.float64).index_add(0, dst, a)
    has = torch.bincount(dst, minlength=12) > 0
    torch.testing.assert_close(tot[has], torch.ones_like(tot[has]), rtol=0, atol=1e-12)
    shift = torch.randn(12, 4, generator=g, dtype=torch.float64)
    torch.testing.assert_close(tece.graph_softmax(s + shift[dst], dst, 12), a, rtol=0, atol=1e-12)
    for n in range(9):
        sel = dst == n
        if sel.any():
            torch.testing.assert_close(a[sel], torch.softmax(s[sel], dim=0), rtol=0, atol=1e-12)


def _tece_model(seed=0, C=16, radial_phase=True):
    cfg = configs.model_cfg("tece", [26, 28], 30.0, num_channel=C, edge_ace_hidden=8)
    torch.manual_seed(seed)
    m = om.TACE(cfg).double()
    if radial_phase:  # non-zero radial_proj exercises bias and rotary phase
        for inter in m.representation.interactions:
            if hasattr(inter.rejector, "radial_proj"):
                torch.nn.init.normal_(inter.rejector.radial_proj.weight, std=0.7)
                torch.nn.init.normal_(inter.rejector.radial_proj.bias, std=0.7)
                inter.rejector.temperature_logit.data.normal_()
    return m, cfg


def _cluster(seed, n=14):
    rng = np.random.default_rng(seed)
    pos = rng.uniform(0, 6.0, (n, 3))
    return dict(positions=pos, cell=np.eye(3) * 40.0, numbers=rng.choice([26, 28], n), pbc=(False,) * 3)


def _energy_forces(m, cfg, s, rc=5.0):
    ei, S = onl.neighbour_list(s["positions"], s["cell"], s["pbc"], rc)
    d = data.collate([s], [(ei, S)], cfg["atomic_numbers"], dtype=torch.float64)
    out = om.compute(m, d, forces=True)
    return out["energy"].item(), out["forces"]


def test_tece_model_is_rotation_translation_permutation_invariant():
    m, cfg = _tece_model()
    s = _cluster(1)
    E, F = _energy_forces(m, cfg, s)
    g = torch.Generator().manual_seed(5)
    R = _rand_rot(g)[0].numpy()
    sr = dict(s, positions=s["positions"] @ R.T + np.array([1.0, -2.0, 0.5]))
    Er, Fr = _energy_forces(m, cfg, sr)
    assert abs(Er - E) < 1e-10 * abs(E)
    torch.testing.assert_close(Fr, F @ torch.from_numpy(R).T, rtol=0, atol=1e-10)
    p = np.random.default_rng(2).permutation(len(s["numbers"]))
    sp = dict(s, positions=s["positions"][p], numbers=s["numbers"][p])
    Ep, Fp = _energy_forces(m, cfg, sp)
    assert abs(Ep - E) < 1e-10 * abs(E)
    torch.testing.assert_close(Fp, F[p], rtol=0, atol=1e-10)


def test_tece_forces_are_minus_energy_gradient():
    m, cfg = _tece_model(seed=3)
    s = _cluster(2)
    E, F = _energy_forces(m, cfg, s)
    h = 1e-5
    for a, c in [(0, 0), (3, 1), (7, 2)]:
        sp, sm = (dict(s, positions=s["positions"].copy()) for _ in range(2))
        sp["positions"][a, c] += h
        sm["positions"][a, c] -= h
        fd = -(_energy_forces(m, cfg, sp)[0] - _energy_forces(m, cfg, sm)[0]) / (2 * h)
        assert abs(fd - F[a, c].item()) < 1e-7 * max(1.0, abs(fd)), (a, c, fd, F[a, c].item())


def test_tece_frame_roll_leaves_the_convolution_unchanged():
    """Rolling every edge frame about its edge axis (another valid frame)
    changes nothing: the convolution is SO(2)-equivariant in the frame."""
    m, cfg = _tece_model(seed=4)
    conv = m.representation.interactions[1].rejector
    g = torch.Generator().manual_seed(6)
    N, E = 9, 40
    ei = torch.stack([torch.randint(0, N, (E,), generator=g), torch.randint(0, N, (E,), generator=g)])
    v = torch.randn(E, 3, generator=g, dtype=torch.float64)
    x = torch.randn(N, 9, conv.C, generator=g, dtype=torch.float64)
    w = torch.randn(E, conv.weight_numel, generator=g, dtype=torch.float64)
    Rb = torch.randn(E, 8, generator=g, dtype=torch.float64)
    W, Wi = tece.edge_wigner(v, 2, 2)
    th = torch.rand(E, generator=g, dtype=torch.float64) * 6.28
    c, s = torch.cos(th), torch.sin(th)
    z, o = torch.zeros_like(th), torch.ones_like(th)
    Ry = torch.stack([torch.stack([c, z, s], -1), torch.stack([z, o, z], -1), torch.stack([-s, z, c], -1)], -2)
    R2 = Ry @ tece.edge_rotation(v)
    D = tece.wigner_blocks(R2, 2)
    Dfull = v.new_zeros(E, 9, 9)
    for l, b in enumerate(D):
        Dfull[:, l * l:(l + 1) ** 2, l * l:(l + 1) ** 2] = b
    W2 = Dfull[:, tece.m_order(2, 2), :]
    a = conv(x, w, ei, W, Wi, Rb)
    b = conv(x, w, ei, W2, W2.transpose(1, 2), Rb)
    torch.testing.assert_close(a, b, rtol=0, atol=1e-11)
