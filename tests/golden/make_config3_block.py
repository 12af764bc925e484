"""Oracle fixture for one 128-row block of BASELINE config 3's down linear (Llama-3.2-1B-shaped,
2-bit E8P12, 2048 x 8192): the oracle's E8P12 VAMP (16 iterations, tau 0.2) and its 3 gram-metric CD
sweeps, precomputed in the build container because the CPU oracle needs minutes at this size
(tests/test_gpu_config3.py compares the GPU against it in seconds).

The inputs are rebuilt by ``case()`` from seeds with element-wise CPU arithmetic only (no reductions
or BLAS calls whose rounding depends on the CPU), so the test and this script form identical inputs:

* eigenbasis V = diag(d) Had_8192 / sqrt(8192) (d random signs; orthonormal up to fp32 rounding) and
  a decaying, heavy-tailed spectrum S^2 -- an explicit decomposition both sides share, as the GPU
  tests of config 4 share one decomposition between the GPU and the oracle;
* Wr = RHT(0.02 N(0,1) rounded to bf16) / 0.02 (right randomized Hadamard over all 8192 columns).

Recorded: the warm-start precision, the oracle's VAMP codes (before the polish) and final EM
precision, and the oracle's polish of its own VAMP result (codes, row errors, accepted moves).
Codes are stored as uint16 (E8P12 indices are < 2^16).

Also recorded (``floors``): the oracle's own polish agreement when only the last bits of Vs change
(two seeded roundings), the greedy cascade's noise floor at this size.

Usage:  python tests/golden/make_config3_block.py [floors]     (about 10 minutes on 8 cores)
Output: tests/golden/c3_down_block.npz
"""
from __future__ import annotations

import os
import sys
import time

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

ROWS, N = 128, 8192
TAU = 0.2


def case():
    """(Wr, V, S) of the block, from seeds, with element-wise CPU arithmetic only."""
    from oracle import uniform as ou

    g = torch.Generator().manual_seed(ou.stable_seed("cfg3:down:block"))
    d = (torch.randint(0, 2, (N,), generator=g) * 2 - 1).to(torch.float32)
    V = ou.hadamard_rows(torch.diag(d), N)
    # spectrum: exp(2 Z) sorted descending (the Student-t Hessians' eigenvalues spread over about
    # eight decades), plus the 1% damping of the configs' Hessians relative to exp(2)
    lam = torch.exp(2.0 * torch.randn(N, generator=g)).sort(descending=True).values + 0.01 * float(np.exp(2.0))
    S = torch.sqrt(lam)
    su = (torch.randint(0, 2, (N,), generator=g) * 2 - 1).to(torch.float32)
    W = (0.02 * torch.randn(ROWS, N, generator=g)).to(torch.bfloat16).to(torch.float32)
    Wr = ou.hadamard_rows(W * su.view(1, -1), N) / 0.02
    return Wr, V, S


def nearest_init(Wr, grid, cache):
    """Nearest codeword of every 8-block (the RTN init, mpq/adapters/quip_sharp.py:212-241) by the
    oracle's factorized MAP search at gamma = 1 without prior."""
    from oracle import e8p12 as oe8

    nb = N // 8
    idx, _ = oe8.map_search(Wr.reshape(-1, 8).numpy(), np.ones(ROWS, np.float32), nb, cache)
    idx = torch.from_numpy(np.asarray(idx, dtype=np.int64)).view(ROWS, nb)
    return grid[idx.reshape(-1)].view(ROWS, N), idx


def main() -> None:
    from mpq_amd import codebook
    from oracle import e8p12 as oe8
    from oracle import uniform as ou

    torch.set_num_threads(min(8, os.cpu_count() or 1))
    t0 = time.time()
    Wr, V, S = case()
    grid = torch.from_numpy(codebook.grid_numpy())
    cache = oe8.factor_cache(grid)
    hat0, idx0 = nearest_init(Wr, grid, cache)
    Vs = V * S.unsqueeze(0)
    Yu = Wr.matmul(Vs)
    obs0 = 1.0 / max(float((Yu - hat0.matmul(Vs)).square().mean()), 1e-12)
    print(f"inputs {time.time() - t0:.1f} s, obs0 {obs0:.6g}", flush=True)
    cfg = dict(iters=16, damping=0.5, prior_tau=TAU, polish_sweeps=0)
    hat_v, idx_v, err_v, st = oe8.solve_e8p12_rankspace_vamp(Wr, hat0, V, S, grid, cache, cfg,
                                                              obs_precision_init=obs0)
    print(f"vamp {time.time() - t0:.1f} s, obs final {st['obs_final']:.6g}", flush=True)
    hat_p, idx_p, acc = oe8.gram_block_cd(hat_v, idx_v, Yu, Vs, grid, 3)
    err_p = ou.rankspace_error(Yu, hat_p, Vs)
    print(f"polish {time.time() - t0:.1f} s, accepted {acc}", flush=True)
    np.savez_compressed(
        os.path.join(HERE, "c3_down_block.npz"),
        idx0=idx0.numpy().astype(np.uint16),
        obs_initial=np.float64(obs0),
        idx_vamp=idx_v.numpy().astype(np.uint16),
        err_vamp=err_v.numpy().astype(np.float32),
        obs_final=np.float64(st["obs_final"]),
        idx_polished=idx_p.numpy().astype(np.uint16),
        err_polished=err_p.numpy().astype(np.float32),
        accepted=np.int64(acc),
    )
    print(f"written in {time.time() - t0:.1f} s", flush=True)


def _vs_jitter(Vs, seed):
    """Every entry of Vs moved to a random one of its two neighbouring floats or kept (seeded)."""
    gen = torch.Generator().manual_seed(int(seed))
    step = torch.randint(-1, 2, Vs.shape, generator=gen)
    up = torch.nextafter(Vs, torch.full_like(Vs, float("inf")))
    dn = torch.nextafter(Vs, torch.full_like(Vs, float("-inf")))
    return torch.where(step > 0, up, torch.where(step < 0, dn, Vs))


def floors() -> None:
    """The oracle's agreement with itself through the polish when only the last bits of its input
    factorisation change (two seeded roundings of Vs): the greedy cascade's noise floor, added to the
    fixture as ``polish_floor`` (the lowest) and ``polish_jitter_agree``."""
    from mpq_amd import codebook
    from oracle import e8p12 as oe8

    torch.set_num_threads(min(8, os.cpu_count() or 1))
    path = os.path.join(HERE, "c3_down_block.npz")
    d = dict(np.load(path))
    Wr, V, S = case()
    grid = torch.from_numpy(codebook.grid_numpy())
    Vs = V * S.unsqueeze(0)
    idx_v = torch.from_numpy(d["idx_vamp"].astype(np.int64))
    x_v = grid[idx_v.reshape(-1)].view(ROWS, N)
    agree = []
    for seed in (1, 2):
        Vj = _vs_jitter(Vs, seed)
        _, idx_j, _ = oe8.gram_block_cd(x_v, idx_v, Wr.matmul(Vj), Vj, grid, 3)
        agree.append(float((idx_j.numpy() == d["idx_polished"].astype(np.int64)).mean()))
        print(f"jitter {seed}: polish agreement {agree[-1]:.5f}", flush=True)
    d["polish_jitter_agree"] = np.asarray(agree, np.float64)
    d["polish_floor"] = np.float64(min(agree))
    np.savez_compressed(path, **d)


if __name__ == "__main__":
    if len(sys.argv) > 1 and sys.argv[1] == "floors":
        floors()
    else:
        main()
        floors()
