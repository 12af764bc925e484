"""CPU: pins the oracle's VAMP loops on their non-recipe options against vectors the reference itself
wrote (tests/golden/make_golden.py ``options``: the reference's solve_uniform_rankspace_vamp and
solve_e8p12_rankspace_vamp on their CPU dispatch, no polish).

Uniform loop (mpq/solver.py:426-830, 64 x 256, 4-bit): r1 started from the float weight or zero
(:472-479), EM off, a fixed observation precision alone and with a caller's warm start (the warm
start wins, :486-489), no damping, and the round-mean final decision (:833-850).  E8P12 loop
(mpq/solver.py:853-1276, 32 x 128): best-iterate tracking (:940-958, 1083-1121), no prior, a fixed
observation precision, the rms / mean |W| / unit prior scales (mpq/priors/e8p12.py:48-63).  Checked: codes, best / stop iteration and the final observation precision."""
import os

import numpy as np
import pytest
import torch

from mpq_amd import codebook
from oracle import e8p12 as oe8
from oracle import uniform as ou

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "vamp_options.npz")

UNIFORM = {"init_float": (dict(init_from="float"), None), "init_zero": (dict(init_from="zero"), None),
           "em_off": (dict(em_obs_precision=False), None), "obs_fixed": (dict(obs_precision=50.0), None),
           "obs_warm_start": (dict(obs_precision=50.0), 200.0), "undamped": (dict(damping=1.0), None),
           "round_mean": (dict(final_decision="round_mean", gamma_start=0.01, prior_tau=2.0), None)}
E8P12 = {"best_iterate": dict(best_iterate=True), "no_prior": dict(prior_tau=0.0), "obs_fixed": dict(obs_precision=0.1),
         "prior_rms": dict(prior_tau_scale_mode="rms"), "prior_mean_abs": dict(prior_tau_scale_mode="mean_abs"),
         "prior_unit": dict(prior_tau_scale_mode="none")}


def _gold():
    d = np.load(GOLD)
    return {k: (torch.from_numpy(d[k]) if d[k].ndim else d[k].item()) for k in d.files}


@pytest.mark.parametrize("name", list(UNIFORM))
def test_uniform_options_reproduce_reference(name):
    g = _gold()
    extra, obs_init = UNIFORM[name]
    cfg = dict(iters=16, damping=0.5, prior_tau=0.2, polish_sweeps=0, gamma_start=1.0, gamma_retry_factor=4.0,
               gamma_retry_steps=3)
    cfg.update(extra)
    V, S = g["V"], g["S"]
    q, _, _, _, st = ou.solve_uniform_rankspace_vamp(g["W"], g["x_rtn"], g["scale_full"], g["zero_full"], g["maxq"],
                                                     V, V.T.contiguous(), S, V * S.unsqueeze(0), cfg,
                                                     obs_precision_init=obs_init)
    assert torch.equal(q.to(torch.int64), g[f"u_{name}_q"].to(torch.int64))
    assert st["best_iter"] == g[f"u_{name}_best_iter"] and st["stop_iter"] == g[f"u_{name}_stop_iter"]
    assert abs(st["obs_final"] - g[f"u_{name}_obs_final"]) <= 1e-9 * g[f"u_{name}_obs_final"]


@pytest.mark.parametrize("name", list(E8P12))
def test_e8p12_options_reproduce_reference(name):
    g = _gold()
    grid = torch.from_numpy(codebook.grid_numpy())
    cache = oe8.factor_cache(grid)
    cfg = dict(iters=16, damping=0.5, prior_tau=0.25, polish_sweeps=0)
    cfg.update(E8P12[name])
    _, idx, _, st = oe8.solve_e8p12_rankspace_vamp(g["e_Wr"], g["e_hat0"], g["e_V"], g["e_S"], grid, cache, cfg)
    assert torch.equal(idx, g[f"e_{name}_idx"].to(idx.dtype))
    assert st["best_iter"] == g[f"e_{name}_best_iter"] and st["stop_iter"] == g[f"e_{name}_stop_iter"]
    assert abs(st["obs_final"] - g[f"e_{name}_obs_final"]) <= 1e-6 * g[f"e_{name}_obs_final"]
