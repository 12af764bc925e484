"""Oracle (test infrastructure only): CPU restatement of the reference's AWQ scale search pieces
for a single linear layer, torch fp32 in the reference's operation order.

* ``compute_w_mean``       mpq/awq_scale.py:49-83
* ``candidate_scales``     mpq/awq_scale.py:338-348
* ``pseudo_quantize``      mpq/awq_scale.py:108-157
* ``search_linear``        mpq/awq_scale.py:491-580 with the single-linear output error
                           sum_rows D H D^T / rows (H = X^T X / T)
Pinned by tests/test_oracle_awq.py (closed forms: normalisation, grid membership, the output-MSE
identity).
"""
from __future__ import annotations

import torch


def compute_w_mean(weights, group_size: int) -> torch.Tensor:
    n = weights[0].shape[1]
    w_sum = torch.zeros(n, dtype=torch.float32)
    rows = 0
    for W in weights:
        wa = W.abs().view(-1, group_size)
        gs = wa.amax(dim=1, keepdim=True) + 1e-6
        w_sum += (wa / gs).view(W.shape).sum(dim=0, dtype=torch.float32)
        rows += W.shape[0]
    return w_sum / rows


def candidate_scales(x_mean: torch.Tensor, w_mean: torch.Tensor, ratio: float) -> torch.Tensor:
    s = (x_mean.pow(ratio) / (w_mean.pow(1 - ratio) + 1e-4)).clamp(min=1e-4)
    s = s / (s.max() * s.min()).sqrt()
    s[torch.isinf(s)] = 1
    s[torch.isnan(s)] = 1
    return s


def pseudo_quantize(W: torch.Tensor, bits: int, group_size: int, sym: bool) -> torch.Tensor:
    v = W.reshape(-1, group_size)
    out = v.clone()
    if not sym:
        mx = v.amax(dim=1, keepdim=True)
        mn = v.amin(dim=1, keepdim=True)
        max_int = 2 ** bits - 1
        scales = (mx - mn).clamp(min=1e-5) / max_int
        zeros = (-torch.round(mn / scales)).clamp_(0, max_int)
        out.div_(scales)
        torch.round(out, out=out)
        out.add_(zeros)
        out.clamp_(0, max_int)
        out.sub_(zeros)
        out.mul_(scales)
    else:
        mx = v.abs().amax(dim=1, keepdim=True).clamp(min=1e-5)
        max_int = 2 ** (bits - 1) - 1
        scales = mx / max_int
        out.div_(scales)
        torch.round(out, out=out)
        out.clamp_(-(2 ** (bits - 1)), max_int)
        out.mul_(scales)
    return out.view(W.shape)


def delta(W, s, bits, group_size, sym):
    Wq = pseudo_quantize(W * s.view(1, -1), bits, group_size, sym) / s.view(1, -1)
    return W - Wq


def search_linear(W, H, x_mean, w_mean, bits, group_size, sym=False):
    losses = []
    for k in range(20):
        s = candidate_scales(x_mean, w_mean, k / 20.0)
        D = delta(W, s, bits, group_size, sym)
        losses.append(float(((D @ H) * D).sum() / W.shape[0]))
    best = min(range(20), key=lambda k: (losses[k], k))
    return candidate_scales(x_mean, w_mean, best / 20.0), losses[best], best / 20.0, losses
