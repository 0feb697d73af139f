"""CPU oracle for the TACE/TECE energy-and-force path.

TEST INFRASTRUCTURE ONLY.  This package is a from-scratch, pure-PyTorch (CPU)
restatement of the reference algorithm (xvzemin/tace ``e3nnTACE`` behind
``TensorModel``) used as the *checker* for the MI355X HIP implementation in
``tace_amd``.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it; the product package never
does, and nothing here is ever timed as the GPU result.

Every function cites the reference file:line it restates.  The reference
itself depends on e3nn / torch_geometric / matscipy, none of which is
installed, so e3nn's published algorithms are restated here:

* ``so3.py``        Wigner-3j (via sympy's independent Clebsch-Gordan), real SH
                    (built by the W3j(1,l,l+1) recursion), irreps bookkeeping.
* ``model.py``      e3nnTACE forward (species-grouped linears, edge-chunked
                    tensor product + scatter) with autograd forces / stress.
* ``neighbours.py`` brute-force periodic neighbour list (matscipy ``ijSd``
                    semantics) in float64 numpy.

The parity pins (what fixes each part independently of this code: closed
forms, independent implementations, invariances, finite differences) are the
tests of ``tests/test_oracle_pins.py`` and ``tests/test_oracle_tece_pins.py``.
"""
