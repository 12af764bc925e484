"""AWQ scale search for a single linear layer on the HIP kernels (the step before the solve).

* ``compute_w_mean``            -> ``mpq_awq_w_mean``   (reference ``mpq/awq_scale.py:49-83``)
* ``search_best_scale_linear``  -> ``mpq_awq_search``   (reference ``mpq/awq_scale.py:491-580``)

The reference scores each ratio by running the inspected module on calibration activations; for
one linear layer that output error is ``sum_rows D H D^T / rows`` with ``D = W - Wq`` and
``H = X^T X / T``, which the kernel evaluates with one MFMA GEMM per ratio.  Modules that are not a
single linear map (attention, gated MLP) are outside this search.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Sequence, Tuple

import torch

from . import _lib, ops


@torch.inference_mode()
def compute_w_mean(weights: Sequence[torch.Tensor], group_size: int) -> torch.Tensor:
    """Mean over all rows of ``|W| / (group abs-max + 1e-6)`` per input channel (fp32)."""
    if not weights:
        raise ValueError("no weights")
    dev = ops._dev(*weights)
    n = int(weights[0].shape[1])
    w_sum = torch.zeros(n, dtype=torch.float32, device=dev)
    rows_total = 0
    for W in weights:
        W = ops._f32c(W)
        rows, nn = W.shape
        if nn != n:
            raise ValueError(f"Expected consistent in_features across layers ({n}), got {nn}.")
        ws = ops.workspace(4 * rows * max(n // int(group_size), 1) + 256, dev)
        _lib.call("mpq_awq_w_mean", _lib.ptr(W), rows, n, int(group_size), _lib.ptr(w_sum), _lib.ptr(ws),
                  int(ws.numel()), _lib.stream_handle(dev))
        rows_total += rows
    return w_sum / float(rows_total)


@torch.inference_mode()
def search_best_scale_linear(W: torch.Tensor, H: torch.Tensor, x_mean: torch.Tensor, *, bits: int,
                             group_size: int, sym: bool = False, prev_scale_hint: Optional[float] = None,
                             w_mean: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, float, float, torch.Tensor]:
    """Returns (best_scales (n,), best_error, best_ratio, losses (20,))."""
    dev = ops._dev(W, H, x_mean, w_mean)
    W = ops._f32c(W)
    rows, n = W.shape
    if w_mean is None:
        w_mean = compute_w_mean([W], group_size)
    w_mean = ops._f32c(w_mean).reshape(-1)
    if prev_scale_hint is not None:
        w_mean = w_mean * float(prev_scale_hint)
    lib = _lib.load()
    ws = ops.workspace(int(lib.mpq_awq_workspace_size(rows, n)), dev)
    scales = torch.empty(n, dtype=torch.float32, device=dev)
    losses = torch.empty(20, dtype=torch.float32, device=dev)
    be = ctypes.c_float(0.0)
    br = ctypes.c_float(0.0)
    _lib.call("mpq_awq_search", _lib.ptr(W), rows, n, _lib.ptr(ops._f32c(H)), _lib.ptr(ops._f32c(x_mean)),
              _lib.ptr(w_mean), int(group_size), int(bits), int(bool(sym)), _lib.ptr(scales), _lib.ptr(losses),
              ctypes.addressof(be), ctypes.addressof(br), _lib.ptr(ws), int(ws.numel()), _lib.stream_handle(dev))
    return scales, float(be.value), float(br.value), losses
