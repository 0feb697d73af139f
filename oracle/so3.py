"""Oracle SO(3) helpers (test infrastructure; see ``oracle/__init__.py``).

Restates the e3nn pieces the reference imports:

* ``wigner_3j``  -- e3nn ``o3.wigner_3j`` (used by ``o3.TensorProduct`` in
  ``tace/models/_e3nn/fused.py:44-51, 203-210``).  Algorithm: SU(2)
  Clebsch-Gordan tensor (here from ``sympy.physics.wigner.clebsch_gordan``, an
  implementation independent of the product's Racah code), change of basis to
  e3nn's real basis ``Q_l = (-i)^l q_l``, real part, unit Frobenius norm.
* ``spherical_harmonics`` -- e3nn ``_spherical_harmonics`` with
  ``normalization="component"`` (``tace/models/angular.py:288-315``).  Built
  here by the coupling recursion ``Y^{l+1} = c_l W3j(1,l,l+1)^T (Y^1 (x) Y^l)``
  with ``c_l > 0`` fixed on the unit sphere; this yields homogeneous
  polynomials of degree l, i.e. the same function as e3nn's closed forms also
  off the unit sphere.
"""

from __future__ import annotations

import functools
import math

import numpy as np
import torch


# ---------------------------------------------------------------- irreps ----
def ir_str(l: int, p: int) -> str:
    return f"{l}{'e' if p == 1 else 'o'}"


def parse_irreps(s):
    """'128x0e+1x1o' -> [(128, (0, 1)), (1, (1, -1))]  (e3nn ``o3.Irreps``)."""
    if isinstance(s, list):
        return s
    out = []
    for tok in s.split("+"):
        tok = tok.strip()
        mul, ir = (tok.split("x") if "x" in tok else ("1", tok))
        out.append((int(mul), (int(ir[:-1]), 1 if ir[-1] == "e" else -1)))
    return out


def irreps_dim(irreps) -> int:
    return sum(m * (2 * ir[0] + 1) for m, ir in irreps)


def simplify(irreps):
    """e3nn ``Irreps.simplify``: merge adjacent equal irreps."""
    out = []
    for m, ir in irreps:
        if out and out[-1][1] == ir:
            out[-1] = (out[-1][0] + m, ir)
        elif m > 0:
            out.append((m, ir))
    return out


def regroup(irreps):
    """e3nn ``Irreps.regroup`` = sort (by irrep, then position) + simplify."""
    srt = sorted(((ir, i, m) for i, (m, ir) in enumerate(irreps)))
    return simplify([(m, ir) for ir, _, m in srt])


def ir_mul(ir1, ir2):
    """e3nn ``Irrep.__mul__``: all l3 in |l1-l2|..l1+l2 with p1*p2."""
    p = ir1[1] * ir2[1]
    return [(l, p) for l in range(abs(ir1[0] - ir2[0]), ir1[0] + ir2[0] + 1)]


def possible_tp_irreps(in1, in2, parity: bool, lmax: int):
    """``_to_possible_tp_irreps`` (``tace/models/_e3nn/base.py:16-30``)."""
    s = set()
    for _, a in in1:
        for _, b in in2:
            for c in ir_mul(a, b):
                if c[0] <= lmax and (parity or c[1] == (-1) ** c[0]):
                    s.add(c)
    return regroup([(1, c) for c in s])


def times(irreps, n: int):
    """``o3.Irreps * n`` (tuple repetition)."""
    return list(irreps) * n


def sh_irreps(lmax: int):
    """``o3.Irreps.spherical_harmonics(lmax, p=-1)``."""
    return [(1, (l, (-1) ** l)) for l in range(lmax + 1)]


def generate_paths(irreps_out, in1, in2, mode: str, identical_inputs: bool = False):
    """``generate_paths`` (``tace/models/_e3nn/paths.py:30-71``), no l-restrictions."""
    paths, outs = [], []
    for _, ir_out in irreps_out:
        for i, (mul, ir1) in enumerate(in1):
            for j, (_, ir2) in enumerate(in2):
                if ir_out in ir_mul(ir1, ir2):
                    if identical_inputs and i == j and (ir1[0] + ir2[0] - ir_out[0]) % 2 == 1:
                        continue
                    paths.append((i, j, len(outs)))
                    outs.append((mul, ir_out))
    return paths, outs


# ------------------------------------------------------------- wigner 3j ----
def _q_real_to_complex(l: int) -> np.ndarray:
    """e3nn ``change_basis_real_to_complex`` (with the (-i)^l phase)."""
    q = np.zeros((2 * l + 1, 2 * l + 1), dtype=complex)
    r = 2 ** -0.5
    for m in range(-l, l + 1):
        if m < 0:
            q[l + m, l - m] = r
            q[l + m, l + m] = -1j * r
        elif m == 0:
            q[l, l] = 1.0
        else:
            q[l + m, l + m] = (-1) ** m * r
            q[l + m, l - m] = 1j * (-1) ** m * r
    return (-1j) ** l * q


@functools.lru_cache(maxsize=None)
def wigner_3j(l1: int, l2: int, l3: int) -> np.ndarray:
    from sympy.physics.wigner import clebsch_gordan

    cg = np.zeros((2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1), dtype=complex)
    for a in range(2 * l1 + 1):
        for b in range(2 * l2 + 1):
            m1, m2 = a - l1, b - l2
            m3 = m1 + m2
            if -l3 <= m3 <= l3:
                cg[a, b, m3 + l3] = float(clebsch_gordan(l1, l2, l3, m1, m2, m3))
    q1, q2, q3 = _q_real_to_complex(l1), _q_real_to_complex(l2), _q_real_to_complex(l3)
    # C_real[j, l, m] = sum_{i,k,n} q1[i, j] q2[k, l] conj(q3)[n, m] cg[i, k, n]
    c = np.einsum("ij,kl,nm,ikn->jlm", q1, q2, np.conj(q3), cg)
    assert np.max(np.abs(c.imag)) < 1e-10
    c = c.real
    return c / np.linalg.norm(c)


def w3j_torch(l1, l2, l3, dtype, device="cpu") -> torch.Tensor:
    return torch.tensor(wigner_3j(l1, l2, l3), dtype=dtype, device=device)


# ------------------------------------------------------ spherical harmonics ----
@functools.lru_cache(maxsize=None)
def _sh_recursion_constants(lmax: int):
    """Positive constants c_l s.t. Y^{l+1} = c_l W3j(1,l,l+1)^T(Y^1 x Y^l) has
    component normalization sum_m (Y^{l+1}_m)^2 = 2l+3 on the unit sphere."""
    rng = np.random.default_rng(0)
    v = rng.normal(size=(16, 3))
    v /= np.linalg.norm(v, axis=1, keepdims=True)
    ys = [np.ones((16, 1)), np.sqrt(3.0) * v]
    consts = []
    for l in range(1, lmax):
        t = np.einsum("ijk,ni,nj->nk", wigner_3j(1, l, l + 1), ys[1], ys[l])
        c = np.sqrt((2 * l + 3) / np.mean(np.sum(t * t, axis=1)))
        consts.append(float(c))
        ys.append(c * t)
    return consts


def spherical_harmonics(lmax: int, vec: torch.Tensor) -> torch.Tensor:
    """Component-normalized real SH of ``vec`` (not normalized first), e3nn order:
    [Y0, Y1(-1..1), Y2(-2..2), ...]; Y^1 = sqrt(3) (x, y, z)."""
    one = torch.ones_like(vec[..., :1])
    if lmax == 0:
        return one
    ys = [one, math.sqrt(3.0) * vec]
    consts = _sh_recursion_constants(lmax)
    for l in range(1, lmax):
        w = w3j_torch(1, l, l + 1, vec.dtype, vec.device)
        ys.append(consts[l - 1] * torch.einsum("ijk,...i,...j->...k", w, ys[1], ys[l]))
    return torch.cat(ys, dim=-1)
