"""E8P12 codebook: 2^16 points of the E8 lattice shifted by +-1/4 ("E8P").

The reference never builds this table itself: it calls quip-sharp's
``E8P12_codebook`` (un-vendored, quip-sharp@1d8f873e) and consumes it only
through the factor cache of ``mpq/priors/e8p12.py:83-151``.  That cache
needs exactly this structure:

* 256 absolute-value patterns ``abs_k`` (8 half-odd-integer entries each);
* index layout ``idx = (k << 8) | s`` with an 8-bit sign field ``s``;
* branch ``b = popcount(s) & 1`` selects the shift ``+1/4`` (b=0) or
  ``-1/4`` (b=1) (``mpq/priors/e8p12.py:112-116``);
* ``grid[idx] - shift = sign * abs_k`` where the sign pattern has the parity
  fixed by ``abs_k`` (even coordinate sum of the D8+1/2 point), checked at
  ``mpq/priors/e8p12.py:121-130``.

The abs patterns are the 227 points of (D8 + 1/2) with squared norm <= 10
(1 + 8 + 28 + 56 + 70 + 8 + 56) plus 29 points of squared norm 12.  QUIP#'s
own choice of the 29 norm-12 patterns, its pattern order and its sign-bit
layout live only in quip-sharp's ``lib/codebook/latticee8_padded12.py``; this
module uses a documented stand-in (the first 29 lexicographic patterns with
five 3/2 and three 1/2 entries; all 256 patterns in lexicographic order;
sign field ``s`` maps to the sign pattern ``s ^ ((b ^ parity_k) << 7)``).
Swapping in QUIP#'s table is a change of data (``ABS2_TABLE``), not of any
kernel: the HIP search kernel is generated from this table at build time.
"""
from __future__ import annotations

import itertools
from functools import lru_cache
from typing import Optional, Tuple

import numpy as np

CODESZ = 8
N_ABS = 256
N_CODES = 1 << 16


def _abs2_patterns() -> np.ndarray:
    """Return the 256 abs patterns in units of 1/2 (entries 1, 3, 5), lexicographic."""
    small = []
    norm12_five_threes = []
    for tup in itertools.product((1, 3, 5), repeat=CODESZ):
        sq4 = sum(v * v for v in tup)  # 4 * squared norm
        if sq4 <= 40:
            small.append(tup)
        elif sq4 == 48 and tup.count(3) == 5 and tup.count(1) == 3:
            norm12_five_threes.append(tup)
    small.sort()
    norm12_five_threes.sort()
    if len(small) != 227 or len(norm12_five_threes) != 56:
        raise RuntimeError("E8P12 abs-pattern enumeration is inconsistent")
    table = sorted(small + norm12_five_threes[:29])
    return np.asarray(table, dtype=np.int8)


ABS2_TABLE: np.ndarray = _abs2_patterns()  # (256, 8) int8, values 1/3/5 (= 2*|x|)


def base_parity() -> np.ndarray:
    """Parity of the number of negative signs allowed for each abs pattern.

    A point ``sign * abs`` of D8 + 1/2 must have an even coordinate sum; flipping
    one sign changes the sum by an odd integer, so the allowed sign patterns have
    ``#negatives == sum(abs) (mod 2)``.
    """
    sums_half = ABS2_TABLE.astype(np.int64).sum(axis=1)  # 2 * sum(abs)
    return ((sums_half // 2) & 1).astype(np.int32)


@lru_cache(maxsize=1)
def _grid_np() -> np.ndarray:
    idx = np.arange(N_CODES, dtype=np.int64)
    k = idx >> 8
    s = idx & 255
    bits = (s[:, None] >> np.arange(CODESZ)) & 1
    branch = bits.sum(axis=1) & 1
    signs = s ^ (((branch ^ base_parity()[k]) & 1) << 7)
    sbits = (signs[:, None] >> np.arange(CODESZ)) & 1
    absv = ABS2_TABLE[k].astype(np.float32) * np.float32(0.5)
    shift = np.where(branch == 0, np.float32(0.25), np.float32(-0.25)).astype(np.float32)
    grid = shift[:, None] + np.where(sbits == 1, -absv, absv)
    return grid.astype(np.float32)


def grid_numpy() -> np.ndarray:
    """(65536, 8) float32 codebook; every entry is exact in fp32."""
    return _grid_np().copy()


def packed_abs() -> np.ndarray:
    """256 int64 words holding the abs codes (2*|x| in 4-bit fields, coordinate i at bits 4i)."""
    shifts = (4 * np.arange(CODESZ, dtype=np.int64))[None, :]
    return (ABS2_TABLE.astype(np.int64) << shifts).sum(axis=1)


def index_of(branch: int, k: int, sign_id: int) -> int:
    """Codeword index for (shift branch, abs pattern, sign pattern with the right parity)."""
    return (int(k) << 8) | (int(sign_id) ^ (((int(branch) ^ int(base_parity()[k])) & 1) << 7))


_GRID_ON: dict = {}


def require_standin_table(cb, where: str) -> None:
    """Raise ValueError unless ``cb`` is None or its ``grid`` equals, element by element, the table
    compiled into libmpq_amd (``grid_numpy()``).  The kernels search that table and emit its index
    layout, so a codebook with another table (quip-sharp's real ``E8P12_codebook``) would mix two
    layouts: refused until its table is swapped in here and the library is rebuilt."""
    if cb is None:
        return
    import torch

    grid = getattr(cb, "grid", None)
    if grid is None:
        raise ValueError(f"{where}: the codebook object has no `grid`")
    g = torch.as_tensor(grid)
    key = str(g.device)
    ref = _GRID_ON.get(key)
    if ref is None:
        ref = _GRID_ON[key] = torch.from_numpy(grid_numpy()).to(g.device)
    if tuple(g.shape) != tuple(ref.shape) or not torch.equal(g.to(torch.float32), ref):
        raise ValueError(
            f"{where}: cb.grid differs from the E8P12 table compiled into libmpq_amd (the documented "
            "stand-in table of mpq_amd/codebook.py; QUIP#'s own table is not available to this build). "
            "Swap QUIP#'s table into ABS2_TABLE and rebuild before passing this codebook.")


class E8P12_codebook:  # noqa: N801 - class name is part of the reference protocol
    """Codebook object with the protocol the reference consumes.

    Protocol (``mpq/priors/e8p12.py:83-151``, ``mpq/adapters/quip_sharp.py:212-262``,
    ``mpq/polish/block_cd.py:663-739``): ``grid`` (65536x8 fp32), ``grid_packed_abs``
    (256), ``codesz``, ``idx_dtype``, ``packsz``, ``quantize``, ``maybe_pack_idxs``,
    ``by_idxs``.  ``quantize`` is the exact nearest-codeword search on the HIP kernel
    (the MAP search with unit precision and no prior).
    """

    codesz = CODESZ
    packsz = 1
    pack_out = False
    idx_dtype = None  # filled lazily with torch.int64 (keeps torch import out of module import)

    def __init__(self, device: Optional[object] = None) -> None:
        import torch

        type(self).idx_dtype = torch.int64
        dev = torch.device("cpu") if device is None else torch.device(device)
        self.grid = torch.from_numpy(grid_numpy()).to(dev)
        self.grid_packed_abs = torch.from_numpy(packed_abs()).to(dev)
        self.grid_norm = self.grid.square().sum(dim=-1)

    def to(self, device: object) -> "E8P12_codebook":
        out = E8P12_codebook.__new__(E8P12_codebook)
        out.grid = self.grid.to(device)
        out.grid_packed_abs = self.grid_packed_abs.to(device)
        out.grid_norm = self.grid_norm.to(device)
        return out

    def quantize(self, X, return_idx: bool = True, **kwargs) -> Tuple[object, object] | object:
        """Nearest codeword of each row of ``X`` (``(..., 8)``) with first-index ties."""
        import torch

        from .priors.e8p12 import e8p12_nearest

        del kwargs  # resid_scale_override etc. have no effect on an exact search
        shape = X.shape
        flat = X.reshape(-1, CODESZ).to(dtype=torch.float32).contiguous()
        idx, vals = e8p12_nearest(flat, return_vals=True)
        vals = vals.view(shape).to(dtype=X.dtype)
        if return_idx:
            return vals, idx.view(shape[:-1])
        return vals

    def maybe_pack_idxs(self, idxs):
        """Identity packing stand-in: QUIP#'s kernel-specific permutation is unpinned."""
        return idxs

    def by_idxs(self, idxs, **kwargs):
        del kwargs
        return self.grid.to(idxs.device)[idxs.long()]
