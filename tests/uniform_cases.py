"""Seeded synthetic inputs shaped like BASELINE config 0 (scaled down for the CPU oracle)."""
from __future__ import annotations

import torch

from oracle.uniform import stable_seed


def make_layer(rows: int, cols: int, *, tokens: int = 2048, seed_key: str = "cfg0", heavy: bool = False):
    """W ~ 0.02 N(0,1); X with lognormal channel scales and 1% x20 outlier channels;
    H = X^T X / T + 0.01 mean(diag) I.  Returns (W, H) fp32 CPU."""
    gw = torch.Generator().manual_seed(stable_seed(f"{seed_key}:W"))
    gx = torch.Generator().manual_seed(stable_seed(f"{seed_key}:X"))
    W = 0.02 * torch.randn(rows, cols, generator=gw)
    Z = torch.randn(tokens, cols, generator=gx)
    if heavy:
        chi = torch.distributions.Chi2(torch.tensor(4.0)).sample((tokens, cols))
        Z = Z / torch.sqrt(chi / 4.0)
    c = torch.exp(torch.randn(cols, generator=gx))
    out = torch.randperm(cols, generator=gx)[: max(1, round(0.01 * cols))]
    c[out] *= 20.0
    X = Z * c
    H = X.T.matmul(X) / tokens
    H = H + 0.01 * torch.diagonal(H).mean() * torch.eye(cols)
    return W.float(), H.float()


class QCfg:
    def __init__(self, bits: int, group_size: int, rotation: str = "none"):
        self.bits = bits
        self.group_size = group_size
        self.desc_act = False

        class _M:
            pass

        self.mpq = _M()
        self.mpq.rotation_mode = rotation
        self.mpq.solver = "vamp"


RECIPE = dict(iters=16, damping=0.5, prior_tau=0.2, polish_sweeps=3, gamma_start=1.0, gamma_retry_factor=4.0,
              gamma_retry_steps=3, em_obs_precision=True, em_obs_precision_damping=0.3,
              em_obs_precision_min=1e-4, em_obs_precision_max=1e8, obs_precision=0.0)
