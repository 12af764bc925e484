"""CD polish (the reference's ``mpq.polish`` namespace).

* ``uniform_scalar_diag_greedy_cd``  reference ``mpq/polish/triton_scalar_cd.py:164-307``
* ``polish_uniform_rankspace`` / ``polish_e8p12_rankspace``: the solver-level dispatchers live in
  ``mpq_amd.solver`` (reference ``mpq/solver.py:260-423``).
"""
from .triton_scalar_cd import uniform_scalar_diag_greedy_cd

__all__ = ["uniform_scalar_diag_greedy_cd"]
