"""CPU: pin the E8P12 posterior, VAMP loop and gram-metric CD of the oracle against the reference."""
import os

import numpy as np
import torch

from mpq_amd import codebook
from oracle import e8p12 as oe8

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    d = np.load(os.path.join(GOLD, name + ".npz"))
    return {k: torch.from_numpy(d[k]) if d[k].ndim else d[k].item() for k in d.files}


def test_posterior_matches_reference_golden_and_bruteforce():
    g = _load("e8p12_posterior")
    grid = codebook.grid_numpy()
    cache = oe8.factor_cache(torch.from_numpy(grid))
    post = oe8.posterior(g["r1"], g["gamma1"], cache, prior_center_blocks=g["center"], prior_tau=0.25)
    assert torch.equal(post["map_idxs"], g["map_idxs"])
    assert torch.allclose(post["x1_blocks"], g["x1"], rtol=1e-5, atol=1e-6)
    assert torch.allclose(post["var1"], g["var1"], rtol=1e-4, atol=1e-7)
    assert torch.allclose(post["alpha1"], g["alpha1"], rtol=1e-5)
    assert torch.allclose(post["logZ"], g["logZ"], rtol=1e-5, atol=1e-4)
    # brute force over all 65536 codewords (prior folded into r, gamma)
    r, c = g["r1"].reshape(-1, 8), g["center"].reshape(-1, 8)
    gam = g["gamma1"].repeat_interleave(g["r1"].shape[1], 0).reshape(-1)
    s = c.abs().amax(-1).clamp_min(1e-12)
    pp = 1.0 / (0.25 * s) ** 2
    gw = gam + pp
    rw = (gam[:, None] * r + pp[:, None] * c) / gw[:, None]
    sel = slice(0, 64)
    m, v, _ = oe8.posterior_bruteforce(rw[sel].numpy(), gw[sel].numpy(), grid)
    hi = gw[sel] >= 1e3
    got = post["x1_blocks"].reshape(-1, 8)[sel]
    assert np.allclose(got[~hi].numpy(), m[~hi.numpy()], rtol=1e-4, atol=1e-5)
    assert np.allclose(post["var1"].reshape(-1)[sel][~hi].numpy(), v[~hi.numpy()], rtol=1e-3, atol=1e-6)


def test_e8p12_vamp_loop_matches_reference_golden():
    g = _load("e8p12_vamp")
    torch.set_num_threads(1)
    grid = torch.from_numpy(codebook.grid_numpy())
    cache = oe8.factor_cache(grid)
    cfg = dict(iters=16, damping=0.5, prior_tau=0.25, polish_sweeps=0)
    hat, idx, err, st = oe8.solve_e8p12_rankspace_vamp(g["Wr"], g["hat0"], g["V"], g["S"], grid, cache, cfg)
    agree = float((idx == g["idx_vamp"]).float().mean())
    assert agree >= 0.999, agree
    assert abs(st["obs_final"] - g["obs_final"]) <= 1e-3 * g["obs_final"]
    hat, idx, err, st = oe8.solve_e8p12_rankspace_vamp(g["Wr"], g["hat0"], g["V"], g["S"], grid, cache,
                                                       dict(cfg, polish_sweeps=3))
    agree = float((idx == g["idx_final"]).float().mean())
    assert agree >= 0.999, agree
    assert torch.allclose(err, g["err_final"], rtol=1e-3)


def test_refine_codebook_matches_reference_golden():
    """The QUIP# adapter driver's glue (nearest-codeword start, rank-space warm start of the
    observation precision, its carry over two 128-row blocks, per-block VAMP + 3 gram-CD sweeps)
    against the reference's mpq_refine_codebook run on the CPU (tests/golden/make_golden.py).  On this
    input the reference's EM drives the precision to its 1e-4 clamp in the first block; the carry
    hands that value to the second block."""
    g = _load("e8p12_refine")
    torch.set_num_threads(1)
    grid = torch.from_numpy(codebook.grid_numpy())
    cache = oe8.factor_cache(grid)
    info = {}
    hat, idx, obs = oe8.refine_codebook(g["Wr"], g["H"], grid, cache,
                                        dict(iters=16, damping=0.5, prior_tau=0.25, polish_sweeps=3),
                                        block_rows=128, info=info)
    assert torch.equal(idx, g["idx"])
    assert torch.equal(hat, g["hat"])
    assert abs(info["obs_initial"] - g["obs_initial"]) <= 1e-6 * g["obs_initial"]
    assert obs == g["obs_final"]


def test_posterior_stats_bruteforce_pinned():
    """The brute-force diagnostics: logZ equals the reference's golden logZ_blocks; the entropy lies in
    [0, log 65536] and tends to log 65536 as gamma -> 0 (uniform posterior); a lone codeword far
    ahead gives entropy ~0 and the closed-form margin g/2 (d2 - d1)."""
    g = _load("e8p12_posterior")
    grid = codebook.grid_numpy()
    r, c = g["r1"].reshape(-1, 8), g["center"].reshape(-1, 8)
    gam = g["gamma1"].repeat_interleave(g["r1"].shape[1], 0).reshape(-1)
    s = c.abs().amax(-1).clamp_min(1e-12)
    pp = 1.0 / (0.25 * s) ** 2
    gw = gam + pp
    rw = (gam[:, None] * r + pp[:, None] * c) / gw[:, None]
    sel = slice(0, 48)
    logz, ent, margin = oe8.posterior_stats_bruteforce(rw[sel].numpy(), gw[sel].numpy(), grid)
    assert np.allclose(logz, g["logZ"].reshape(-1)[sel].numpy(), rtol=1e-5, atol=1e-4)
    assert np.all(ent >= -1e-9) and np.all(ent <= np.log(65536) + 1e-9) and np.all(margin >= 0)
    lz0, ent0, m0 = oe8.posterior_stats_bruteforce(np.zeros((1, 8)), np.array([1e-9]), grid)
    assert abs(ent0[0] - np.log(65536)) < 1e-6 and m0[0] < 1e-8
    x = grid[1234].astype(np.float64)
    d = ((grid.astype(np.float64) - x) ** 2).sum(1)
    d2 = np.partition(d, 1)[1]
    _, ent1, m1 = oe8.posterior_stats_bruteforce(x[None], np.array([50.0]), grid)
    assert ent1[0] < 1e-6 and abs(m1[0] - 25.0 * d2) < 1e-9 * 25.0 * d2


def test_factorized_diagnostics_match_bruteforce():
    """The oracle's restatement of the reference's factorized diagnostics (need_stats) equals the
    exact codeword-level logZ, entropy and margin at moderate precisions."""
    grid = torch.from_numpy(codebook.grid_numpy())
    cache = oe8.factor_cache(grid)
    for gs in (0.3, 3.0):
        g = torch.Generator().manual_seed(77)
        r1 = torch.randn(8, 12, 8, generator=g) * 0.8
        gam = torch.exp(torch.randn(8, 1, generator=g)) * gs
        post = oe8.posterior(r1, gam, cache, need_stats=True)
        lz, ent, mg = oe8.posterior_stats_bruteforce(r1.reshape(-1, 8).numpy(),
                                                     gam.repeat_interleave(12, 0).reshape(-1).numpy(), grid.numpy())
        assert np.allclose(post["logZ"].reshape(-1).numpy(), lz, rtol=1e-6, atol=1e-5)
        assert np.allclose(post["entropy"].reshape(-1).numpy(), ent, rtol=1e-5, atol=1e-4)
        assert np.allclose(post["margin"].reshape(-1).numpy(), mg, rtol=1e-5, atol=1e-4)
