"""Uniform scalar-grid prior on the HIP kernels (reference ``mpq/priors/uniform.py``).

* ``discrete_uniform_mmse`` (reference :99-213) -> ``mpq_uniform_denoise``
* ``nearest_atom_idx``      (reference :287-299)
* ``dequant_from_q``        (reference :302-309) -> ``mpq_dequant`` for uint8 codes

Per-entry parameters ``scale_full``/``zero_full`` may be given expanded (B x n, as
the reference does) — they are then passed with group size 1.
"""
from __future__ import annotations

from typing import Dict

import torch

from .. import _lib, ops

_BACKENDS = {"eager", "compile", "triton", "auto"}


@torch.inference_mode()
def discrete_uniform_mmse(
    *,
    r1: torch.Tensor,
    gamma1: torch.Tensor,
    scale_full: torch.Tensor,
    zero_full: torch.Tensor,
    maxq: int,
    prior_center: torch.Tensor,
    prior_tau: float,
    need_stats: bool,
    atoms: torch.Tensor | None = None,
    vamp_backend: str = "auto",
) -> Dict[str, torch.Tensor | float | str]:
    """Exact discrete MMSE over a uniform scalar grid per entry (HIP kernel).

    ``vamp_backend`` accepts the reference's strings; all map to the HIP kernel.
    Posterior diagnostics (``need_stats``) are not computed by this backend and
    raise, as the reference's Triton backend does (reference :119-120).
    ``atoms`` is ignored: the kernel forms ``s * (q - z)`` on the fly.
    """
    del atoms
    backend = str(vamp_backend or "auto").strip().lower()
    if backend not in _BACKENDS:
        raise ValueError(f"unsupported vamp_backend={vamp_backend!r}; expected eager|compile|triton|auto.")
    if need_stats:
        raise ValueError("HIP uniform VAMP backend does not support posterior diagnostics.")
    dev = ops._dev(r1, gamma1, scale_full, zero_full, prior_center)
    r1 = r1.to(torch.float32).contiguous()
    rows, n = r1.shape
    gamma = gamma1.to(device=dev, dtype=torch.float32).contiguous().reshape(-1)
    if gamma.numel() != rows:
        raise ValueError(f"expected gamma1 with shape (B,1), got {tuple(gamma1.shape)}")
    for name, t in (("scale_full", scale_full), ("zero_full", zero_full), ("prior_center", prior_center)):
        if tuple(t.shape) != (rows, n):
            raise ValueError("r1, scale_full, zero_full, and prior_center must have matching shapes.")
    mean = torch.empty_like(r1)
    var = torch.empty_like(r1)
    map_idx = torch.empty(rows, n, dtype=torch.int64, device=dev)
    map_value = torch.empty_like(r1)
    alpha1 = torch.empty(rows, 1, dtype=torch.float32, device=dev)
    center = prior_center.to(torch.float32).contiguous()
    for r0 in range(0, rows, 65535):
        r1_ = min(rows, r0 + 65535)
        _lib.call("mpq_uniform_denoise", r1_ - r0, n, int(maxq), _lib.ptr(r1[r0:r1_]), _lib.ptr(gamma[r0:r1_]),
                  _lib.ptr(center[r0:r1_]), n, _lib.ptr(ops._f32c(scale_full)[r0:r1_]),
                  _lib.ptr(ops._f32c(zero_full)[r0:r1_]), 1, float(prior_tau), _lib.ptr(mean[r0:r1_]),
                  _lib.ptr(var[r0:r1_]), _lib.ptr(map_idx[r0:r1_]), _lib.ptr(map_value[r0:r1_]),
                  _lib.ptr(alpha1[r0:r1_]), ops._stream(dev))
    return {
        "mean": mean,
        "var": var,
        "map_value": map_value,
        "map_idx": map_idx,
        "alpha1": alpha1,
        "entropy": 0.0,
        "margin": 0.0,
        "vamp_backend": "hip",
    }


@torch.inference_mode()
def nearest_atom_idx(*, x: torch.Tensor, scale_full: torch.Tensor, zero_full: torch.Tensor, maxq: int) -> torch.Tensor:
    """q = clamp(round(x / max(s, 1e-12) + z), 0, maxq) as int32 (reference :287-299)."""
    ops._dev(x, scale_full, zero_full)
    q = torch.round(x.to(torch.float32) / scale_full.to(torch.float32).clamp_min(1e-12) + zero_full.to(torch.float32))
    return torch.clamp(q, 0, int(maxq)).to(torch.int32)


@torch.inference_mode()
def dequant_from_q(*, q_int: torch.Tensor, scale_full: torch.Tensor, zero_full: torch.Tensor) -> torch.Tensor:
    """x = s * (q - z) (reference :302-309)."""
    if q_int.dtype == torch.uint8 and q_int.dim() == 2:
        return ops.dequant(q_int, scale_full, zero_full, 1)
    return scale_full.to(torch.float32) * (q_int.to(torch.float32) - zero_full.to(torch.float32))
