"""SO(3) bookkeeping for the MI355X TACE path: irreps algebra and real Wigner-3j.

This module is host-side table generation only (float64 numpy). It reproduces
the conventions that the reference inherits from e3nn so that the HIP kernels
compute the same numbers as ``e3nn.o3.TensorProduct`` / ``o3.Linear`` do in

* ``tace/models/_e3nn/fused.py:17-95, 172-271``  (uuu / uvu tensor products)
* ``tace/models/_e3nn/paths.py:30-71``            (path enumeration order)
* ``tace/models/_e3nn/base.py:16-30``             (``_to_possible_tp_irreps``)

Conventions (e3nn's published algorithm, restated):

* An irrep is ``(l, p)`` with ``p = +1`` (even) or ``-1`` (odd); ordering is the
  tuple ordering, so ``Irreps.sort`` sorts by ``l`` then ``p``.
* ``Irreps * n`` repeats the list ``n`` times (tuple repetition), ``regroup`` is
  ``sort`` followed by ``simplify`` (merge *adjacent* equal irreps).
* ``wigner_3j(l1, l2, l3)`` is the SU(2) Clebsch-Gordan tensor (Condon-Shortley
  phase, Racah formula) mapped to the real basis by
  ``Q_l = (-i)^l q_l`` (``q_l`` the real->complex change of basis), made real and
  divided by its Frobenius norm, with no further sign fixing.
"""

from __future__ import annotations

import functools
import math
from fractions import Fraction
from typing import Iterable, List, Sequence, Tuple

import numpy as np


# --------------------------------------------------------------------------
# irreps
# --------------------------------------------------------------------------
class Irrep(tuple):
    """``(l, p)``; ``p`` is +1/-1. ``Irrep("2e")`` and ``Irrep(2, 1)`` both work."""

    def __new__(cls, l, p=None):
        if p is None:
            if isinstance(l, Irrep):
                return l
            if isinstance(l, str):
                s = l.strip()
                p = {"e": 1, "o": -1}[s[-1]]
                l = int(s[:-1])
            else:
                l, p = l
        assert l >= 0 and p in (1, -1)
        return super().__new__(cls, (int(l), int(p)))

    @property
    def l(self) -> int:
        return self[0]

    @property
    def p(self) -> int:
        return self[1]

    @property
    def dim(self) -> int:
        return 2 * self[0] + 1

    def __mul__(self, other: "Irrep") -> List["Irrep"]:
        p = self.p * other.p
        return [Irrep(l, p) for l in range(abs(self.l - other.l), self.l + other.l + 1)]

    def __repr__(self) -> str:
        return f"{self.l}{'e' if self.p == 1 else 'o'}"


class Irreps(tuple):
    """Tuple of ``(mul, Irrep)`` with the handful of e3nn operations the path needs."""

    def __new__(cls, items=()):
        if isinstance(items, Irreps):
            return items
        if isinstance(items, str):
            out = []
            for tok in items.split("+"):
                tok = tok.strip()
                if not tok:
                    continue
                if "x" in tok:
                    m, ir = tok.split("x")
                    out.append((int(m), Irrep(ir)))
                else:
                    out.append((1, Irrep(tok)))
            return super().__new__(cls, tuple(out))
        out = []
        for it in items:
            if isinstance(it, Irrep):
                out.append((1, it))
            elif isinstance(it, str):
                out.append((1, Irrep(it)))
            else:
                mul, ir = it
                out.append((int(mul), Irrep(ir)))
        return super().__new__(cls, tuple(out))

    @property
    def dim(self) -> int:
        return sum(m * ir.dim for m, ir in self)

    @property
    def num_irreps(self) -> int:
        return sum(m for m, _ in self)

    @property
    def ls(self) -> List[int]:
        return [ir.l for m, ir in self for _ in range(m)]

    @property
    def lmax(self) -> int:
        return max(ir.l for _, ir in self)

    def slices(self) -> List[slice]:
        out, acc = [], 0
        for m, ir in self:
            out.append(slice(acc, acc + m * ir.dim))
            acc += m * ir.dim
        return out

    def simplify(self) -> "Irreps":
        out: List[Tuple[int, Irrep]] = []
        for m, ir in self:
            if out and out[-1][1] == ir:
                out[-1] = (out[-1][0] + m, ir)
            elif m > 0:
                out.append((m, ir))
        return Irreps(out)

    def sort(self) -> "Irreps":
        return Irreps([(m, ir) for ir, _, m in sorted((ir, i, m) for i, (m, ir) in enumerate(self))])

    def regroup(self) -> "Irreps":
        return self.sort().simplify()

    def __mul__(self, n: int) -> "Irreps":
        return Irreps(tuple(self) * n)

    def __add__(self, other) -> "Irreps":
        return Irreps(tuple(self) + tuple(Irreps(other)))

    def __repr__(self) -> str:
        return "+".join(f"{m}x{ir}" for m, ir in self)


def spherical_harmonics_irreps(lmax: int) -> Irreps:
    """``o3.Irreps.spherical_harmonics(lmax, p=-1)`` = 1x0e+1x1o+1x2e+..."""
    return Irreps([(1, Irrep(l, (-1) ** l)) for l in range(lmax + 1)])


def possible_tp_irreps(in1: Irreps, in2: Irreps, parity: bool, lmax: int) -> Irreps:
    """Restates ``_to_possible_tp_irreps`` (``tace/models/_e3nn/base.py:16-30``)."""
    s = set()
    for _, ir1 in in1:
        for _, ir2 in in2:
            for ir3 in ir1 * ir2:
                if ir3.l <= lmax and (parity or ir3.p == (-1) ** ir3.l):
                    s.add(ir3)
    return Irreps(sorted(s)).regroup()


def generate_paths(irreps_out: Irreps, in1: Irreps, in2: Irreps, mode: str,
                   identical_inputs: bool = False):
    """Restates ``generate_paths`` (``tace/models/_e3nn/paths.py:30-71``) with no
    ``l1l2`` restriction: loop ir_out, then in1 index i, then in2 index j; every
    admissible path gets its own output block of multiplicity ``mul(in1[i])``.

    Returns ``(paths, irreps_out_actual)`` with ``paths = [(i, j, k), ...]``.
    """
    paths, outs = [], []
    for _, ir_out in irreps_out:
        for i, (mul, ir1) in enumerate(in1):
            for j, (_, ir2) in enumerate(in2):
                if ir_out in ir1 * ir2:
                    if identical_inputs and i == j and (ir1.l + ir2.l - ir_out.l) % 2 == 1:
                        continue
                    paths.append((i, j, len(outs)))
                    outs.append((mul, ir_out))
    return paths, Irreps(outs)


# --------------------------------------------------------------------------
# Wigner 3j
# --------------------------------------------------------------------------
def _fact(n: int) -> int:
    return math.factorial(int(n))


def _su2_cg(j1: int, m1: int, j2: int, m2: int, j3: int, m3: int) -> float:
    """<j1 m1 j2 m2 | j3 m3>, integer spins, Racah's closed form (exact rationals)."""
    if m3 != m1 + m2 or abs(m1) > j1 or abs(m2) > j2 or abs(m3) > j3:
        return 0.0
    if not (abs(j1 - j2) <= j3 <= j1 + j2):
        return 0.0
    pref = Fraction((2 * j3 + 1) * _fact(j3 + j1 - j2) * _fact(j3 - j1 + j2) * _fact(j1 + j2 - j3),
                    _fact(j1 + j2 + j3 + 1))
    pref *= Fraction(_fact(j3 + m3) * _fact(j3 - m3) * _fact(j1 - m1) * _fact(j1 + m1)
                     * _fact(j2 - m2) * _fact(j2 + m2))
    s = Fraction(0)
    for k in range(0, j1 + j2 - j3 + 1):
        a = j1 + j2 - j3 - k
        b = j1 - m1 - k
        c = j2 + m2 - k
        d = j3 - j2 + m1 + k
        e = j3 - j1 - m2 + k
        if min(a, b, c, d, e) < 0:
            continue
        s += Fraction((-1) ** k, _fact(k) * _fact(a) * _fact(b) * _fact(c) * _fact(d) * _fact(e))
    val = math.sqrt(pref) * float(s) if pref >= 0 else 0.0
    return val


def real_to_complex(l: int) -> np.ndarray:
    """e3nn ``change_basis_real_to_complex(l)`` including the ``(-i)^l`` factor."""
    q = np.zeros((2 * l + 1, 2 * l + 1), dtype=np.complex128)
    s2 = 1.0 / math.sqrt(2.0)
    for m in range(-l, 0):
        q[l + m, l + abs(m)] = s2
        q[l + m, l - abs(m)] = -1j * s2
    q[l, l] = 1.0
    for m in range(1, l + 1):
        q[l + m, l + abs(m)] = (-1) ** m * s2
        q[l + m, l - abs(m)] = 1j * (-1) ** m * s2
    return ((-1j) ** l) * q


@functools.lru_cache(maxsize=None)
def wigner_3j(l1: int, l2: int, l3: int) -> np.ndarray:
    """Real, unit-Frobenius-norm coupling tensor of shape [2l1+1, 2l2+1, 2l3+1]."""
    C = np.zeros((2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1))
    for m1 in range(-l1, l1 + 1):
        for m2 in range(-l2, l2 + 1):
            m3 = m1 + m2
            if abs(m3) <= l3:
                C[l1 + m1, l2 + m2, l3 + m3] = _su2_cg(l1, m1, l2, m2, l3, m3)
    Q1, Q2, Q3 = real_to_complex(l1), real_to_complex(l2), real_to_complex(l3)
    R = np.einsum("ij,kl,mn,ikn->jlm", Q1, Q2, np.conj(Q3.T), C.astype(np.complex128))
    assert np.abs(R.imag).max() < 1e-10, (l1, l2, l3)
    R = R.real
    n = np.linalg.norm(R)
    R = R / n
    R[np.abs(R) < 1e-15] = 0.0
    return R


# --------------------------------------------------------------------------
# path tables consumed by the kernel generator
# --------------------------------------------------------------------------
def tp_path_table(in1: Irreps, in2: Irreps, paths) -> List[dict]:
    """For each path: l1, l2, l3, offsets of the in1/in2 components and the
    (sqrt(2 l3 + 1)-scaled) nonzero CG entries ``[(i, j, k, c), ...]``."""
    out = []
    for (i, j, k) in paths:
        l1, l2 = in1[i][1].l, in2[j][1].l
        out.append(dict(i_in1=i, i_in2=j, i_out=k, l1=l1, l2=l2))
    return out


def path_l3(irreps_out: Irreps, paths) -> List[int]:
    return [irreps_out[k][1].l for (_, _, k) in paths]
