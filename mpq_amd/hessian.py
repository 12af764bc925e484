"""Per-linear Hessian accumulation on the HIP SYRK kernel (the step before the per-linear solve).

* ``accumulate``        -> ``mpq_hessian_accumulate``: ``H = beta H + alpha X^T X`` (+ column sums)
* ``GPTQHessian``       GPTQModel's ``add_batch`` convention, ``H = 2/m sum_t x_t x_t^T`` with m the
                        number of samples seen (mpq/adapters/gptqmodel.py:39 relies on it and halves H)
* ``QuipHessian``       QUIP#'s hook convention: ``sum x x^T``, ``sum x`` and the count, finalised as
                        ``H / ct - mu mu^T`` with ``mu = sum x / ct`` (mpq/quip_generic.py:823-921)

GPTQModel and quip-sharp are upstream (absent); both conventions are restated from the reference's
call sites and the published GPTQ / QUIP# algorithms.  Tensors live on the ROCm device.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib, ops


@torch.inference_mode()
def accumulate(H: torch.Tensor, X: torch.Tensor, *, alpha: float = 1.0, beta: float = 1.0,
               colsum: Optional[torch.Tensor] = None) -> torch.Tensor:
    """In place ``H = beta H + alpha X^T X`` for X (T x n, fp32 or bf16; leading dims flattened)."""
    dev = ops._dev(H, X, colsum)
    n = int(H.shape[0])
    if tuple(H.shape) != (n, n) or H.dtype != torch.float32 or not H.is_contiguous():
        raise ValueError("H must be a contiguous fp32 (n, n) tensor")
    X2 = X.reshape(-1, X.shape[-1])
    if int(X2.shape[1]) != n:
        raise ValueError(f"X has {X2.shape[1]} features, H is {n} x {n}")
    if X2.dtype not in (torch.float32, torch.bfloat16):
        X2 = X2.to(torch.float32)
    X2 = X2.contiguous()
    if colsum is not None and (colsum.dtype != torch.float32 or int(colsum.numel()) != n or not colsum.is_contiguous()):
        raise ValueError("colsum must be a contiguous fp32 tensor of n entries")
    _lib.call("mpq_hessian_accumulate", _lib.ptr(X2), int(X2.dtype == torch.bfloat16), int(X2.shape[0]), n, n,
              float(alpha), float(beta), _lib.ptr(H), n, _lib.ptr(colsum), _lib.stream_handle(dev))
    return H


class GPTQHessian:
    """GPTQ's running Hessian: ``H <- H * m / (m + b); m <- m + b; H += (2 / m) X^T X`` per batch of
    ``b`` samples (``inp.shape[0]`` of a 3-D input, 1 for a 2-D one)."""

    def __init__(self, n: int, device) -> None:
        self.H = torch.zeros(int(n), int(n), dtype=torch.float32, device=device)
        self.nsamples = 0

    @torch.inference_mode()
    def add_batch(self, inp: torch.Tensor) -> None:
        if inp.dim() == 2:
            inp = inp.unsqueeze(0)
        tmp = int(inp.shape[0])
        beta = self.nsamples / (self.nsamples + tmp)
        self.nsamples += tmp
        accumulate(self.H, inp.reshape(-1, inp.shape[-1]), alpha=2.0 / self.nsamples, beta=beta)


class QuipHessian:
    """QUIP#'s hook accumulation: ``sum x x^T``, ``sum x``, count; ``finalize()`` returns
    ``(H / ct - mu mu^T, mu, ct)``."""

    def __init__(self, n: int, device) -> None:
        self.H = torch.zeros(int(n), int(n), dtype=torch.float32, device=device)
        self.mu = torch.zeros(int(n), dtype=torch.float32, device=device)
        self.ct = 0

    @torch.inference_mode()
    def add_batch(self, inp: torch.Tensor) -> None:
        x = inp.reshape(-1, inp.shape[-1])
        accumulate(self.H, x, alpha=1.0, beta=1.0, colsum=self.mu)
        self.ct += int(x.shape[0])

    @torch.inference_mode()
    def finalize(self) -> Tuple[torch.Tensor, torch.Tensor, int]:
        mu = self.mu / self.ct
        H = self.H / self.ct
        H.addmm_(-mu.unsqueeze(-1), mu.unsqueeze(0))
        return H, mu, self.ct
