"""Write ``w3j_l4.npz``: the reference's own real-basis Clebsch-Gordan tensors.

The reference vendors an e3nn-derived SO(3) Clebsch-Gordan routine,
``so3_clebsch_gordan(l, l1, l2)`` in
``tace/models/eqt/equitorch/structs/__init__.py:376-393`` (real <-> complex
change of basis ``_change_basis_real_to_complex`` 396-408, SU(2) coefficients
``_su2_clebsch_gordan`` 411-443).  It is the only code in the reference tree
that fixes the per-triple sign of e3nn's ``wigner_3j``, which the oracle and
the kernels both restate; no e3nn is installed here.

This script runs in the build container only (it imports the routine from
``/root/reference``, which does not exist on the GPU box) and writes its raw
output, in the routine's own index order [m (l), m1 (l1), m2 (l2)] and
without any normalisation, for every triangle-valid triple with l, l1, l2 <= 4.
The fixture is data; ``tests/test_w3j_fixture.py`` compares it with both
restatements.

    python tests/golden/make_w3j.py
"""

import os
import sys

import numpy as np

REF_EQT = "/root/reference/tace/models/eqt"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "w3j_l4.npz")
LMAX = 4


def main() -> None:
    sys.path.insert(0, REF_EQT)
    from equitorch.structs import so3_clebsch_gordan  # noqa: E402  (reference code, build container only)

    arrays = {}
    for l in range(LMAX + 1):
        for l1 in range(LMAX + 1):
            for l2 in range(LMAX + 1):
                if not abs(l1 - l2) <= l <= l1 + l2:
                    continue
                c = so3_clebsch_gordan(l, l1, l2)
                a = np.array(c.tolist(), dtype=np.complex128)
                assert np.abs(a.imag).max() < 1e-12, (l, l1, l2)
                arrays[f"cg_{l}_{l1}_{l2}"] = a.real.astype(np.float64)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {len(arrays)} triples to {OUT}")


if __name__ == "__main__":
    main()
