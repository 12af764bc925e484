"""Oracle (test infrastructure only) for the GPTQModel int32 packing of MPQ results.

GPTQModel's packer is upstream code the reference calls (``scripts/backend_gptq.py:843``,
``patches/gptqmodel.patch:359-395``); it is absent here.  Its layout for 2, 3, 4 and 8 bits is a
little-endian bit stream: along the packed dimension, value j occupies bits [bits*j, bits*(j+1))
of the stream, cut into 32-bit words (for 3 bits that gives the familiar 32-values-in-3-words
pattern).  This module restates the layout in that form with numpy bit arrays -- a formulation
independent of the kernel's per-word shifts -- and provides the inverse.  Parity with
GPTQModel's own packer: unpinned (absent); the layout is pinned by the closed-form examples in
``tests/test_oracle_gptq_pack.py``.
"""
from __future__ import annotations

from typing import Dict

import numpy as np


def _pack_stream(vals: np.ndarray, bits: int) -> np.ndarray:
    """Pack the last axis of ``vals`` (non-negative ints < 2^bits) as a little-endian bit
    stream into int32 words; the last axis length times ``bits`` must be a multiple of 32."""
    v = np.asarray(vals, dtype=np.uint32) & np.uint32((1 << bits) - 1)
    lead = v.shape[:-1]
    n = v.shape[-1]
    assert (n * bits) % 32 == 0
    # bit k of value j -> stream position bits*j + k
    shifts = np.arange(bits, dtype=np.uint32)
    bitarr = ((v[..., None] >> shifts) & 1).astype(np.uint8).reshape(*lead, n * bits)
    words = bitarr.reshape(*lead, n * bits // 32, 32)
    weights = (np.uint64(1) << np.arange(32, dtype=np.uint64))
    w = (words.astype(np.uint64) * weights).sum(axis=-1).astype(np.uint64)
    return w.astype(np.uint32).view(np.int32)


def _unpack_stream(words: np.ndarray, bits: int, n: int) -> np.ndarray:
    w = np.asarray(words).view(np.uint32)
    lead = w.shape[:-1]
    bitarr = ((w[..., None] >> np.arange(32, dtype=np.uint32)) & 1).reshape(*lead, -1)[..., : n * bits]
    bitarr = bitarr.reshape(*lead, n, bits)
    return (bitarr.astype(np.uint32) << np.arange(bits, dtype=np.uint32)).sum(axis=-1).astype(np.uint32)


def pack_gptq(q: np.ndarray, scale: np.ndarray, zero: np.ndarray, bits: int, group_size: int,
              fmt: str = "v2") -> Dict[str, np.ndarray]:
    """q (out x in) codes, scale/zero (out x G) -> qweight [in*bits/32, out], qzeros
    [G, out*bits/32] (v1: zero - 1), scales fp16 [G, out], g_idx [in]."""
    q = np.asarray(q)
    rows, n = q.shape
    qweight = _pack_stream(q, bits).T.copy()  # pack along in, then [words, out]
    z = np.rint(np.asarray(zero, dtype=np.float32)).astype(np.int64)
    if fmt == "v1":
        z = z - 1
    qzeros = _pack_stream((z.T & ((1 << bits) - 1)).astype(np.uint32), bits)  # [G, out] packed along out
    scales = np.asarray(scale, dtype=np.float32).T.astype(np.float16)
    g_idx = (np.arange(n) // group_size).astype(np.int32)
    return {"qweight": qweight, "qzeros": qzeros, "scales": scales, "g_idx": g_idx}


def unpack_qweight(qweight: np.ndarray, bits: int, n: int) -> np.ndarray:
    """Inverse of the qweight packing: [in*bits/32, out] -> codes (out x in)."""
    return _unpack_stream(np.asarray(qweight).T.copy(), bits, n)


def unpack_qzeros(qzeros: np.ndarray, bits: int, rows: int, fmt: str = "v2") -> np.ndarray:
    z = _unpack_stream(qzeros, bits, rows).astype(np.int64)  # [G, out]
    if fmt == "v1":
        z = (z + 1) & ((1 << bits) - 1) if bits < 8 else z + 1
    return z.T
