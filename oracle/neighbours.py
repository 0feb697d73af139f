"""Brute-force neighbour list oracle (test infrastructure).

``neighbour_list`` restates ``get_neighborhood`` (``tace/dataset/
neighbour_list.py:195-298``): every ordered (i, j, S) with
|r_j - r_i + S.cell|^2 < r_c^2, minus true self loops (286-292), S = 0 on
non-periodic axes (295); ``edge_index = [i; j]`` (296).  The C kernel in
``nl_bruteforce.c`` tests every pair against every admissible image; the
pure-numpy ``neighbour_list_numpy`` is a second, independent brute force used
to pin it on small cells.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


def _lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "_build", "libnl_oracle.so")
        if not os.path.exists(path):
            subprocess.check_call(["make", "-s", "-C", _HERE])
        lib = ctypes.CDLL(path)
        lib.nl_bruteforce.restype = ctypes.c_int64
        lib.nl_bruteforce.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p,
                                      ctypes.c_double, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        _LIB = lib
    return _LIB


def neighbour_list(positions, cell, pbc, cutoff):
    """Returns (edge_index [2,E] int64, shifts [E,3] int64), (i, j, S)-sorted."""
    pos = np.ascontiguousarray(positions, dtype=np.float64)
    cell = np.ascontiguousarray(cell, dtype=np.float64)
    pbc = np.ascontiguousarray(np.broadcast_to(np.asarray(pbc, dtype=np.int32), (3,)))
    lib = _lib()
    n = pos.shape[0]
    cnt = lib.nl_bruteforce(pos.ctypes.data, n, cell.ctypes.data, pbc.ctypes.data, float(cutoff),
                            None, None, None)
    i = np.empty(cnt, dtype=np.int64)
    j = np.empty(cnt, dtype=np.int64)
    s = np.empty((cnt, 3), dtype=np.int64)
    lib.nl_bruteforce(pos.ctypes.data, n, cell.ctypes.data, pbc.ctypes.data, float(cutoff),
                      i.ctypes.data, j.ctypes.data, s.ctypes.data)
    return np.stack([i, j]), s


def neighbour_list_numpy(positions, cell, pbc, cutoff, nimg: int = 3):
    """Independent O(N^2 * images) numpy brute force over a fixed image box
    [-nimg, nimg]^3 (periodic axes only); for small test cells."""
    pos = np.asarray(positions, dtype=np.float64)
    cell = np.asarray(cell, dtype=np.float64)
    pbc = np.broadcast_to(np.asarray(pbc, dtype=bool), (3,))
    rng = [range(-nimg, nimg + 1) if p else range(0, 1) for p in pbc]
    out_i, out_j, out_s = [], [], []
    d = pos[None, :, :] - pos[:, None, :]  # [i, j, 3] = r_j - r_i
    for a in rng[0]:
        for b in rng[1]:
            for c in rng[2]:
                S = np.array([a, b, c])
                v = d + S @ cell
                r2 = np.einsum("ijk,ijk->ij", v, v)
                m = r2 < cutoff * cutoff
                if a == 0 and b == 0 and c == 0:
                    np.fill_diagonal(m, False)
                ii, jj = np.nonzero(m)
                out_i.append(ii)
                out_j.append(jj)
                out_s.append(np.repeat(S[None], len(ii), axis=0))
    i = np.concatenate(out_i)
    j = np.concatenate(out_j)
    s = np.concatenate(out_s).astype(np.int64)
    order = np.lexsort((s[:, 2], s[:, 1], s[:, 0], j, i))
    return np.stack([i[order], j[order]]), s[order]
