"""ORACLE (test infrastructure only): the QUIP# randomized Hadamard transform in fp64 closed form.

``patches/quip_sharp.patch:211-218`` (RHT_H, RHT_W) and ``:340-375`` (incoherence_process) with
quip-sharp's ``matmul_hadU`` for power-of-two widths and the patch's block fallback
(``_hadU_or_block``, ``:171-185``) otherwise, written as explicit matrices:

* ``Hr   = Had_n D_U H D_U Had_n``
* ``Wr   = Had_m D_V W D_U Had_n``
* ``hatW = D_V Had_m hatWr Had_n D_U``  (the inverse)

``Had_k`` is the orthonormal Sylvester matrix (``scipy.linalg.hadamard(k) / sqrt(k)``), block-diagonal
with blocks of the largest power-of-two factor when ``k`` is not a power of two.  Pinned by
tests/test_oracle_rht.py (orthogonality, the Sylvester recursion, inverse o forward = identity).
"""
from __future__ import annotations

import numpy as np
import scipy.linalg
import torch


def had_matrix(k: int) -> torch.Tensor:
    b = k & -k
    blk = torch.from_numpy(scipy.linalg.hadamard(b).astype(np.float64)) / np.sqrt(b)
    return torch.block_diag(*([blk] * (k // b)))


def rht_h(H, SU):
    n = H.shape[0]
    Hd = had_matrix(n)
    D = torch.diag(SU.double())
    return Hd @ D @ H.double() @ D @ Hd


def rht_w(W, SU, SV):
    m, n = W.shape
    return had_matrix(m) @ torch.diag(SV.double()) @ W.double() @ torch.diag(SU.double()) @ had_matrix(n)


def incoherence_process(hatWr, SU, SV):
    m, n = hatWr.shape
    return torch.diag(SV.double()) @ had_matrix(m) @ hatWr.double() @ had_matrix(n) @ torch.diag(SU.double())
