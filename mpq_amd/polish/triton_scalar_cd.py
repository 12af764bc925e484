"""Exact scalar diagonal greedy CD on the HIP sweep kernel.

Drop-in for the reference's ``mpq/polish/triton_scalar_cd.py:164-307``
(``uniform_scalar_diag_greedy_cd``): same keyword signature, start state, per-sweep greedy order,
accept test, return value and ``cd_trace`` items.  Both ``update_backend`` values run the HIP sweeps
(one launch sequence per sweep; 128 decisions per window with the deferred rank-1 updates applied in
the per-column order of the reference's torch loop), each with its backend's RTN target:
``"torch"`` forms ``x + rhs * (1 / diag)`` as the torch loop does (:266,
``mpq_uniform_cd_sweeps_recip``), ``"triton"`` forms ``x + rhs / diag`` as the sweep kernel does
(:73, ``mpq_uniform_cd_sweeps``).  ``assignment_changes_from_cd0`` re-rounds the current values as
the reference does (:292-296).

Differences from the reference, both documented there as free choices:
* the greedy order is a stable descending sort of the gain (ties by column index; the reference's
  ``argsort`` is unstable);
* the gain is summed over rows in row order.
"""
from __future__ import annotations

from typing import Any, Dict, Optional

import torch

from .. import ops


def _objective_mean(target: torch.Tensor, x: torch.Tensor, gram: torch.Tensor) -> float:
    """Mean row-wise (target - x) gram (target - x)^T (reference ``mpq/linear.py:98-121``)."""
    if target.shape != x.shape:
        raise ValueError(f"target/x shape mismatch: {tuple(target.shape)} != {tuple(x.shape)}")
    if gram.ndim != 2 or gram.shape != (x.shape[1], x.shape[1]):
        raise ValueError(f"invalid gram shape {tuple(gram.shape)} for x={tuple(x.shape)}")
    if x.numel() == 0:
        return 0.0
    d = (target.to(torch.float32) - x).contiguous()
    return float((ops.gemm(d, gram.to(torch.float32)) * d).sum(dim=1).mean().item())


@torch.inference_mode()
def uniform_scalar_diag_greedy_cd(
    *,
    x: torch.Tensor,
    Y_u: torch.Tensor,
    Vs: torch.Tensor,
    gram_full: torch.Tensor,
    scale: torch.Tensor,
    zero: torch.Tensor,
    maxq: int,
    sweeps: int,
    accept_tol: float = 0.0,
    update_backend: str = "torch",
    raw_target: Optional[torch.Tensor] = None,
    raw_gram: Optional[torch.Tensor] = None,
) -> tuple[torch.Tensor, Dict[str, Any]]:
    """Greedy scalar CD in rank space from ``x`` (rows x n) with per-element ``scale``/``zero``
    (rows x n, the reference's expanded group parameters); returns (x, stats) with
    ``accepted_updates`` and the per-sweep ``cd_trace``."""
    backend = str(update_backend or "torch").strip().lower()
    if backend not in {"torch", "triton"}:
        raise ValueError(f"unsupported update_backend={update_backend!r}; expected 'torch'|'triton'.")
    if (raw_target is None) != (raw_gram is None):
        raise ValueError("raw_target and raw_gram must be provided together.")
    if x.ndim != 2 or scale.shape != x.shape or zero.shape != x.shape:
        raise ValueError("x, scale and zero must be (rows, n) tensors of one shape")
    rows, n = x.shape
    x_work = x.to(dtype=torch.float32).clone().contiguous()
    scale_f = scale.to(device=x_work.device, dtype=torch.float32).contiguous()
    zero_f = zero.to(device=x_work.device, dtype=torch.float32).contiguous()
    gram = gram_full.to(device=x_work.device, dtype=torch.float32).contiguous()
    Vs_f = Vs.to(dtype=torch.float32).contiguous()
    residual = Y_u.to(torch.float32) - ops.gemm(x_work, Vs_f)
    rhs = ops.gemm(residual, Vs_f, trans_b=True)
    res_norm = residual.square().sum(dim=1).contiguous()
    del residual
    diag = Vs_f.square().sum(dim=1).clamp_min_(1e-12).contiguous()
    q_initial = torch.round(x_work / scale_f.clamp_min(1e-12) + zero_f).clamp_(0, int(maxq)).to(torch.int32)
    q = q_initial.to(torch.uint8)
    accepted = torch.zeros(rows, dtype=torch.int32, device=x_work.device)

    def trace_item(budget: int, swept: int, total: int) -> Dict[str, float | int]:
        q_current = torch.round(x_work / scale_f.clamp_min(1e-12) + zero_f).clamp_(0, int(maxq)).to(torch.int32)
        item: Dict[str, float | int] = {
            "budget": int(budget),
            "stabilized_objective_mean": float(res_norm.mean().item()),
            "accepted_updates_sweep": int(swept),
            "accepted_updates_cumulative": int(total),
            "assignment_changes_from_cd0": int((q_current != q_initial).sum().item()),
            "assignments_total": int(q_initial.numel()),
        }
        if raw_target is not None and raw_gram is not None:
            item["raw_objective_mean"] = _objective_mean(raw_target, x_work, raw_gram)
        return item

    trace = [trace_item(0, 0, 0)]
    total = 0
    for sweep in range(max(int(sweeps), 0)):
        if rows == 0 or n == 0:
            trace.append(trace_item(sweep + 1, 0, total))
            continue
        ops.uniform_cd_sweeps(rhs, x_work, q, res_norm, accepted, scale_f, zero_f, 1, int(maxq), diag, gram,
                              block_rows=rows, sweeps=1, accept_tol=float(accept_tol),
                              target_rule="recip" if backend == "torch" else "div")
        now = int(accepted.sum().item())
        trace.append(trace_item(sweep + 1, now - total, now))
        total = now
    return x_work.to(dtype=x.dtype), {"accepted_updates": float(total), "cd_trace": trace}
