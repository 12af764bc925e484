"""GPTQModel packing of MPQ results (the step after the per-linear solve on the GPTQModel path).

* ``pack_gptq``              -> ``mpq_gptq_pack``: ``qweight`` / ``qzeros`` / ``scales`` / ``g_idx`` in
                                GPTQModel's int32 layout (format ``GPTQ_V2`` by default, as
                                ``scripts/backend_gptq.py:843`` selects; ``v1`` stores ``zero - 1``)
* ``packed_basis_weight``    -> ``mpq_dequant``: ``scale * (q - zero)`` in the packed (solver) basis
                                (``patches/gptqmodel.patch:381-391``)

Tensors live on the ROCm device; there is no CPU path.
"""
from __future__ import annotations

from typing import Dict

import torch

from . import _lib, ops


@torch.inference_mode()
def pack_gptq(q_int: torch.Tensor, scale_groups: torch.Tensor, zero_groups: torch.Tensor, *, bits: int,
              group_size: int, fmt: str = "v2") -> Dict[str, torch.Tensor]:
    """Pack codes (out x in, values in [0, 2^bits)) and group parameters (out x G)."""
    fmt = str(fmt).strip().lower()
    if fmt not in ("v1", "v2"):
        raise ValueError(f"unsupported GPTQ format {fmt!r}; expected 'v1' or 'v2'")
    dev = ops._dev(q_int, scale_groups, zero_groups)
    rows, n = q_int.shape
    bits = int(bits)
    if bits not in (2, 3, 4, 8):
        raise ValueError(f"GPTQ packing supports bits 2, 3, 4, 8; got {bits}")
    q = q_int.to(torch.uint8).contiguous()
    G = (n + int(group_size) - 1) // int(group_size)
    sc = ops._f32c(scale_groups)
    zr = ops._f32c(zero_groups)
    if tuple(sc.shape) != (rows, G) or tuple(zr.shape) != (rows, G):
        raise ValueError(f"scale/zero must be ({rows}, {G})")
    qweight = torch.empty(n * bits // 32, rows, dtype=torch.int32, device=dev)
    qzeros = torch.empty(G, rows * bits // 32, dtype=torch.int32, device=dev)
    scales = torch.empty(G, rows, dtype=torch.float16, device=dev)
    g_idx = torch.empty(n, dtype=torch.int32, device=dev)
    _lib.call("mpq_gptq_pack", _lib.ptr(q), _lib.ptr(sc), _lib.ptr(zr), rows, n, int(group_size), bits,
              int(fmt == "v1"), _lib.ptr(qweight), _lib.ptr(qzeros), _lib.ptr(scales), _lib.ptr(g_idx),
              _lib.stream_handle(dev))
    return {"qweight": qweight, "qzeros": qzeros, "scales": scales, "g_idx": g_idx}


@torch.inference_mode()
def packed_basis_weight(q_int: torch.Tensor, scale_groups: torch.Tensor, zero_groups: torch.Tensor, *,
                        group_size: int) -> torch.Tensor:
    """``scale * (q - zero)`` (fp32) with group parameters expanded by ``i // group_size``."""
    return ops.dequant(q_int.to(torch.uint8), scale_groups, zero_groups, int(group_size))
