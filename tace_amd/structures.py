"""Seeded synthetic structures for the benchmark configurations.

Each builder returns a dict ``{positions [N,3] f64, cell [3,3] f64 (rows are
lattice vectors), numbers [N] int64, pbc (bool,)*3}`` built with
``numpy.random.default_rng(seed)``.  Shapes follow the configurations quoted
on the reference path (1: Si diamond 2x2x2, 2: FCC 8x8x4 4-species alloy,
3: 4,096-molecule water box, 4: 128 random triclinic crystals,
5: bcc Fe 37^3).
"""

from __future__ import annotations

import math
from typing import Dict, List, Sequence

import numpy as np

# The 89 elements of the MPTrj statistics (Z = 1-83 and 89-94).
MPTRJ_ELEMENTS: List[int] = list(range(1, 84)) + list(range(89, 95))


def _supercell(basis_frac: np.ndarray, a: float, reps: Sequence[int]):
    reps = np.asarray(reps)
    grid = np.stack(np.meshgrid(*[np.arange(r) for r in reps], indexing="ij"), -1).reshape(-1, 3)
    frac = (grid[:, None, :] + basis_frac[None, :, :]).reshape(-1, 3)
    return frac * a, np.diag(reps * a).astype(np.float64)


def si_diamond(reps=(2, 2, 2), a: float = 5.43, sigma: float = 0.05, seed: int = 0) -> Dict:
    fcc = np.array([[0, 0, 0], [0, .5, .5], [.5, 0, .5], [.5, .5, 0]], dtype=np.float64)
    basis = np.concatenate([fcc, fcc + 0.25])
    pos, cell = _supercell(basis, a, reps)
    rng = np.random.default_rng(seed)
    pos = pos + rng.normal(0.0, sigma, pos.shape)
    return dict(positions=pos, cell=cell, numbers=np.full(len(pos), 14, dtype=np.int64), pbc=(True,) * 3)


def fcc_alloy(reps=(8, 8, 4), a: float = 3.6, sigma: float = 0.1, species=(26, 27, 28, 29),
              seed: int = 0) -> Dict:
    fcc = np.array([[0, 0, 0], [0, .5, .5], [.5, 0, .5], [.5, .5, 0]], dtype=np.float64)
    pos, cell = _supercell(fcc, a, reps)
    rng = np.random.default_rng(seed)
    numbers = rng.choice(np.asarray(species, dtype=np.int64), size=len(pos))
    pos = pos + rng.normal(0.0, sigma, pos.shape)
    return dict(positions=pos, cell=cell, numbers=numbers, pbc=(True,) * 3)


def bcc_fe(reps=(37, 37, 37), a: float = 2.87, sigma: float = 0.05, seed: int = 0) -> Dict:
    bcc = np.array([[0, 0, 0], [.5, .5, .5]], dtype=np.float64)
    pos, cell = _supercell(bcc, a, reps)
    rng = np.random.default_rng(seed)
    pos = pos + rng.normal(0.0, sigma, pos.shape)
    return dict(positions=pos, cell=cell, numbers=np.full(len(pos), 26, dtype=np.int64), pbc=(True,) * 3)


def _random_rotations(rng, n):
    q = rng.normal(size=(n, 4))
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    w, x, y, z = q.T
    return np.stack([
        np.stack([1 - 2 * (y * y + z * z), 2 * (x * y - z * w), 2 * (x * z + y * w)], -1),
        np.stack([2 * (x * y + z * w), 1 - 2 * (x * x + z * z), 2 * (y * z - x * w)], -1),
        np.stack([2 * (x * z - y * w), 2 * (y * z + x * w), 1 - 2 * (x * x + y * y)], -1),
    ], 1)


def water_box(n_side: int = 16, box: float = 49.7, jitter: float = 0.3, seed: int = 0) -> Dict:
    """n_side^3 H2O on a jittered cubic grid, O-H 0.96 A, H-O-H 104.5 deg,
    uniformly random orientations (normalised Gaussian quaternions)."""
    rng = np.random.default_rng(seed)
    sp = box / n_side
    g = np.stack(np.meshgrid(*[np.arange(n_side)] * 3, indexing="ij"), -1).reshape(-1, 3)
    O = (g + 0.5) * sp + rng.normal(0.0, jitter, (len(g), 3))
    half = math.radians(104.5) / 2
    h = 0.96 * np.array([[math.sin(half), math.cos(half), 0.0], [-math.sin(half), math.cos(half), 0.0]])
    R = _random_rotations(rng, len(g))
    H = O[:, None, :] + np.einsum("nij,hj->nhi", R, h)
    pos = np.concatenate([O[:, None, :], H], axis=1).reshape(-1, 3)
    numbers = np.tile(np.array([8, 1, 1], dtype=np.int64), len(g))
    return dict(positions=pos, cell=np.eye(3) * box, numbers=numbers, pbc=(True,) * 3)


def random_crystal(rng, n: int, species: Sequence[int], vol_range=(10.0, 25.0), dmin: float = 1.5,
                   max_tries: int = 2000) -> Dict:
    """Random triclinic cell (angles 60-120 deg, lengths within 0.8-1.25 of the
    mean) of volume n * U[vol_range], uniform positions with minimum-image
    distance >= dmin (rejection), species uniform over ``species``."""
    vol = n * rng.uniform(*vol_range)
    while True:
        lengths = rng.uniform(0.8, 1.25, 3)
        al, be, ga = np.radians(rng.uniform(60, 120, 3))
        a = np.array([1.0, 0.0, 0.0])
        b = np.array([math.cos(ga), math.sin(ga), 0.0])
        cx = math.cos(be)
        cy = (math.cos(al) - math.cos(be) * math.cos(ga)) / math.sin(ga)
        cz2 = 1.0 - cx * cx - cy * cy
        if cz2 < 0.05:
            continue
        c = np.array([cx, cy, math.sqrt(cz2)])
        cell = np.stack([a, b, c]) * lengths[:, None]
        break
    cell *= (vol / abs(np.linalg.det(cell))) ** (1.0 / 3.0)
    inv = np.linalg.inv(cell)
    frac = []
    tries = 0
    while len(frac) < n:
        f = rng.uniform(0, 1, 3)
        ok = True
        if frac:
            d = np.asarray(frac) - f
            d -= np.round(d)
            best = np.full(len(frac), np.inf)
            for s in np.stack(np.meshgrid(*[np.arange(-1, 2)] * 3, indexing="ij"), -1).reshape(-1, 3):
                best = np.minimum(best, np.linalg.norm((d + s) @ cell, axis=1))
            ok = best.min() >= dmin
        if ok:
            frac.append(f)
        tries += 1
        if tries > max_tries * n:
            raise RuntimeError("random_crystal: rejection sampling did not converge")
    pos = np.asarray(frac) @ cell
    numbers = rng.choice(np.asarray(species, dtype=np.int64), size=n)
    return dict(positions=pos, cell=cell, numbers=numbers, pbc=(True,) * 3)


def ragged_batch(num: int = 128, nmin: int = 8, nmax: int = 200, seed: int = 0,
                 species=tuple(MPTRJ_ELEMENTS)) -> List[Dict]:
    rng = np.random.default_rng(seed)
    return [random_crystal(rng, int(rng.integers(nmin, nmax + 1)), species) for _ in range(num)]
