"""Pins of the oracle's gate and readout activations (CPU only).

The reference applies e3nn ``Activation`` modules in two places on this path:
* ``O3Gate`` (``tace/models/_e3nn/nonlinear.py:27-42, 93-143``): the gate
  scalars go through ``Activation(irreps_gates, [sigmoid] * n)`` and multiply
  the gated irreps through ``ElementwiseTensorProduct(irreps_gated,
  irreps_gates)``;
* ``ScalarReadOut`` (``tace/models/_e3nn/readout.py:54-64, 80-84``): the hidden
  16x0e features go through ``Activation(hidden, [silu])`` between the two
  linears (``scalar_act`` is "silu" for a 0e output, ``_e3nn/base.py:378``).

e3nn's ``Activation`` multiplies each function by its ``normalize2mom``
constant, so that a unit normal input gives a unit second moment output; the
constants themselves are reference-held literals (``tace/models/mlp.py:34,43``)
pinned elsewhere.  These tests fix what the constants alone leave open:
* that the factor is applied (a gate without it has second moment 0.293, a
  SiLU without it 0.355);
* that the elementwise product with a 0e gate is the plain product at every l
  (e3nn "component" normalisation: sqrt(2l+1) * W3j(l, 0, l) = identity, one
  path per output, so a missing or doubled sqrt(2l+1) changes the l > 0 blocks
  by a factor 2l+1);
* that gated irrep copy k takes gate scalar k: ``irreps_gates`` is built as
  ``[(mul, 0e) for mul, _ in irreps_gated]`` (``nonlinear.py:29-30``) and
  ``ElementwiseTensorProduct`` pairs the i-th irrep copy of its first operand
  with the i-th of its second.  With blocks of distinct multiplicity a layout
  that strides the gates by a fixed channel count, or pairs them by component,
  fails;
* that the layout of the gate input is [all gate scalars | gated irreps], the
  order ``_Sortcut(irreps_gates, irreps_gated)`` gives after its stable sort by
  irrep (all 0e first, the gates before the gated 0e block).
"""

import math

import pytest
import torch

from oracle import model as om


def _gated(muls, ls):
    return [(m, (l, (-1) ** l)) for m, l in zip(muls, ls)]


@pytest.mark.parametrize("muls", [(8, 8, 8, 8), (3, 5, 2, 4)])
def test_gate_output_has_unit_second_moment(muls):
    g = torch.Generator().manual_seed(11)
    gated = _gated(muls, (0, 1, 2, 3))
    gate = om.Gate(gated)
    ngate = sum(muls)
    dim = ngate + sum(m * (2 * l + 1) for m, (l, _) in gated)
    x = torch.randn(200_000, dim, generator=g, dtype=torch.float64)
    with torch.no_grad():
        y = gate(x)
    assert y.shape == (x.shape[0], dim - ngate)
    m2 = y.square().mean(0)
    # 5 sigma of the estimate is ~0.03; without normalize2mom every column sits at 0.293
    assert (m2 - 1.0).abs().max().item() < 0.04, m2
    # the product must not depend on l: every block has the same moment
    off = 0
    for m, (l, _) in gated:
        blk = m2[off:off + m * (2 * l + 1)]
        assert abs(blk.mean().item() - 1.0) < 0.015, (l, blk.mean().item())
        off += m * (2 * l + 1)


def test_gate_pairs_irrep_copies_with_gate_scalars_in_order():
    muls, ls = (3, 5, 2, 4), (0, 1, 2, 3)
    gated = _gated(muls, ls)
    gate = om.Gate(gated)
    ngate = sum(muls)
    g = torch.Generator().manual_seed(3)
    feats = torch.randn(4, sum(m * (2 * l + 1) for m, l in zip(muls, ls)), generator=g, dtype=torch.float64)
    # a distinct gate value per irrep copy
    gates = torch.linspace(-3.0, 3.0, ngate, dtype=torch.float64).repeat(4, 1) + torch.arange(4.0)[:, None]
    with torch.no_grad():
        y = gate(torch.cat([gates, feats], 1))
    # expected from the e3nn pairing rule: expand both operands into their irrep
    # copies and zip them (independent of block offsets)
    copies = []
    off = 0
    for m, l in zip(muls, ls):
        d = 2 * l + 1
        for u in range(m):
            copies.append((off + u * d, d))
        off += m * d
    assert len(copies) == ngate
    c = 1.8467055342154763  # tace/models/mlp.py:43
    want = torch.empty_like(feats)
    for i, (s, d) in enumerate(copies):
        want[:, s:s + d] = feats[:, s:s + d] * (c * torch.sigmoid(gates[:, i:i + 1]))
    torch.testing.assert_close(y, want, rtol=1e-14, atol=1e-14)


def test_gate_reads_gates_before_the_gated_scalars():
    # one 0e gated block: the input is [gates (m) | gated 0e (m)]; swapping the
    # halves must change the result unless both halves are equal
    gate = om.Gate(_gated((4,), (0,)))
    a = torch.tensor([[-2.0, -1.0, 1.0, 2.0]], dtype=torch.float64)
    b = torch.tensor([[0.5, 1.5, 2.5, 3.5]], dtype=torch.float64)
    with torch.no_grad():
        y = gate(torch.cat([a, b], 1))
    torch.testing.assert_close(y, b * 1.8467055342154763 * torch.sigmoid(a), rtol=1e-14, atol=0)


def test_scalar_readout_hidden_activation_is_moment_normalised():
    torch.manual_seed(5)
    C = 32
    ro = om.ScalarReadOut([(C, (0, 1))], hidden=(16,)).double()
    g = torch.Generator().manual_seed(6)
    x = torch.randn(2_000, C, generator=g, dtype=torch.float64)
    acc, n = 0.0, 400
    with torch.no_grad():
        for _ in range(n):
            # the reference's init: N(0, 1) weights (tace/models/linear.py:319-327)
            for lin in ro.linear2:
                lin.weight.normal_()
            acc += ro(x).square().mean().item()
    m2 = acc / n
    # E_W,x[y^2] = E[h^2] for y = sum_a W_a h_a / sqrt(16) with N(0,1) W;
    # normalize2mom puts E[h^2] at 1, plain SiLU at 0.355
    assert abs(m2 - 1.0) < 0.08, m2


def test_scalar_readout_is_linear_silu_linear():
    # at a point where the hidden pre-activations are known exactly
    C = 4
    ro = om.ScalarReadOut([(C, (0, 1))], hidden=(2,)).double()
    with torch.no_grad():
        ro.linear2[0].weight.copy_(torch.tensor([1.0, 0.0, 0.0, 1.0, 0.0, 0.0, 0.0, 0.0], dtype=torch.float64))
        ro.linear2[1].weight.copy_(torch.tensor([1.0, -1.0], dtype=torch.float64))
        x = torch.tensor([[2.0, 3.0, 5.0, 7.0]], dtype=torch.float64)
        y = ro(x)
    # o3.Linear path weight 1/sqrt(fan_in): hidden = (2, 3) / 2; output / sqrt(2)
    c = 1.6791767923989418  # tace/models/mlp.py:34
    h = c * torch.nn.functional.silu(torch.tensor([1.0, 1.5], dtype=torch.float64))
    want = (h[0] - h[1]) / math.sqrt(2.0)
    assert abs(y.item() - want.item()) < 1e-14
