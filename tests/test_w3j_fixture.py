"""W3j sign and index convention pinned to the reference's own Clebsch-Gordan
routine (CPU only).

``tests/golden/w3j_l4.npz`` holds, unnormalised and in the routine's index
order [m, m1, m2], the output of ``so3_clebsch_gordan(l, l1, l2)``
(tace/models/eqt/equitorch/structs/__init__.py:376-393, "adapted from
e3nn"), written by ``tests/golden/make_w3j.py``.  e3nn's
``wigner_3j(l1, l2, l)`` is the same tensor with the output index last,
divided by its Frobenius norm (e3nn o3/_wigner.py ``_so3_clebsch_gordan``):
both build it from Condon-Shortley SU(2) coefficients and the same real <->
complex change of basis with the (-i)^l phase.  So for every triple

    W3j(l1, l2, l)[m1, m2, m] = cg[m, m1, m2] / ||cg||

with the sign of every entry exact.  The oracle (sympy coefficients) and the
product's own Racah-formula code are both checked, for every triangle-valid
triple with l <= 4 -- including the odd-sum triples natural parity never uses.
"""

import os

import numpy as np
import pytest

from oracle import so3 as oso3
from tace_amd import so3 as pso3

FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "w3j_l4.npz")


def _fixture():
    with np.load(FIX) as z:
        return {tuple(int(t) for t in k.split("_")[1:]): z[k] for k in z.files}


REF = _fixture()
TRIPLES = sorted(REF)


def test_fixture_covers_every_triple_to_l4():
    want = {(l, l1, l2) for l in range(5) for l1 in range(5) for l2 in range(5) if abs(l1 - l2) <= l <= l1 + l2}
    assert set(REF) == want
    for (l, l1, l2), a in REF.items():
        assert a.shape == (2 * l + 1, 2 * l1 + 1, 2 * l2 + 1)


@pytest.mark.parametrize("impl", ["oracle", "product"])
@pytest.mark.parametrize("l,l1,l2", TRIPLES)
def test_w3j_equals_reference_cg(impl, l, l1, l2):
    ref = REF[(l, l1, l2)]
    want = np.transpose(ref, (1, 2, 0)) / np.linalg.norm(ref)
    got = (oso3 if impl == "oracle" else pso3).wigner_3j(l1, l2, l)
    assert got.shape == want.shape
    # the sign of the dominant entry first, for a readable failure
    k = np.unravel_index(np.argmax(np.abs(want)), want.shape)
    assert np.sign(got[k]) == np.sign(want[k]), f"sign of W3j({l1},{l2},{l}) flipped"
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-13)


def test_reference_cg_of_l1_l1_l1_is_the_levi_civita_tensor():
    """A closed form independent of both restatements: in e3nn's real basis
    (m = -1, 0, 1 <-> y, z, x) the l=1 x l=1 -> l=1 coupling is the
    antisymmetric unit tensor, up to one overall sign that the reference fixes."""
    w = np.transpose(REF[(1, 1, 1)], (1, 2, 0)) / np.linalg.norm(REF[(1, 1, 1)])
    eps = np.zeros((3, 3, 3))
    for (i, j, k), s in {(0, 1, 2): 1, (1, 2, 0): 1, (2, 0, 1): 1, (0, 2, 1): -1, (2, 1, 0): -1, (1, 0, 2): -1}.items():
        eps[i, j, k] = s
    sign = np.sign(w[0, 1, 2])
    np.testing.assert_allclose(w, sign * eps / np.sqrt(6), atol=1e-15)
