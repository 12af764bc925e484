"""CPU: pin the uniform-path oracle (oracle/uniform.py) by closed forms, brute force and golden vectors."""
import os

import numpy as np
import pytest
import scipy.linalg
import torch

from oracle import uniform as ou
from tests.uniform_cases import RECIPE

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    d = np.load(os.path.join(GOLD, name + ".npz"))
    return {k: torch.from_numpy(d[k]) if d[k].ndim else d[k].item() for k in d.files}


# ---- closed forms ---------------------------------------------------------

def test_hadamard_matches_sylvester_matrix():
    for had in (2, 8, 128):
        X = torch.randn(5, 3 * had, dtype=torch.float32)
        Hm = torch.from_numpy(scipy.linalg.hadamard(had)).double() / np.sqrt(had)
        ref = (X.double().view(5, 3, had) @ Hm.T).view(5, -1)
        got = ou.hadamard_rows(X, had)
        assert torch.allclose(got.double(), ref, atol=1e-5)
        assert torch.allclose(ou.hadamard_rows(got, had), X, atol=1e-5)  # involution (orthonormal, symmetric)


def test_denoiser_matches_bruteforce_fp64():
    g = torch.Generator().manual_seed(0)
    B, n, maxq = 8, 40, 15
    s = torch.rand(B, n, generator=g) * 0.01 + 1e-3
    z = torch.randint(0, 16, (B, n), generator=g).float()
    W = s * (torch.rand(B, n, generator=g) * 15 - z)
    r1 = W + 0.003 * torch.randn(B, n, generator=g)
    gam = torch.exp(torch.randn(B, 1, generator=g)) * 1e4
    out = ou.discrete_uniform_mmse(r1, gam, s, z, maxq, W, 0.2)
    q = torch.arange(maxq + 1, dtype=torch.float64)
    a = s.double().unsqueeze(-1) * (q - z.double().unsqueeze(-1))
    sc = -0.5 * gam.double().unsqueeze(-1) * (a - r1.double().unsqueeze(-1)) ** 2
    sc = sc - 0.5 * (a - W.double().unsqueeze(-1)) ** 2 / (0.2 * s.double().unsqueeze(-1)) ** 2
    p = torch.softmax(sc, dim=-1)
    mean = (p * a).sum(-1)
    var = (p * a * a).sum(-1) - mean ** 2
    assert torch.allclose(out["mean"].double(), mean, rtol=1e-5, atol=1e-9)
    # var = E[a^2] - mean^2 in fp32 (the reference's formula) carries cancellation error ~ ulp(E[a^2])
    second = (p * a * a).sum(-1)
    assert bool(((out["var"].double() - var.clamp_min(0)).abs() <= 1e-3 * var.abs() + 8 * 2.0 ** -23 * second).all())
    assert torch.equal(out["map_idx"], sc.argmax(-1))
    assert bool((out["mean"] >= a.min(-1).values.float() - 1e-6).all() and (out["mean"] <= a.max(-1).values.float() + 1e-6).all())


def test_lmmse_matches_dense_solve():
    g = torch.Generator().manual_seed(1)
    n, B = 24, 5
    A = torch.randn(n, n, generator=g)
    Hf = A @ A.T / n + 0.1 * torch.eye(n)
    lam, V = torch.linalg.eigh(Hf)
    lam, V = lam.flip(0), V.flip(1)
    S = lam.sqrt()
    Vs = V * S
    w = torch.randn(B, n, generator=g)
    r2 = torch.randn(B, n, generator=g)
    g2 = torch.rand(B, 1, generator=g) + 0.5
    obs = 3.7
    x2, a2, res = ou.linear_mmse_exact(r2, g2, w @ Vs, V, V.T, S, obs)
    Hd = (Vs @ Vs.T).double()
    for b in range(B):
        M = obs * Hd + float(g2[b]) * torch.eye(n, dtype=torch.float64)
        ref = torch.linalg.solve(M, obs * Hd @ w[b].double() + float(g2[b]) * r2[b].double())
        assert torch.allclose(x2[b].double(), ref, rtol=1e-4, atol=1e-5)
        alpha_ref = float(g2[b]) / n * torch.trace(torch.linalg.inv(M))
        assert abs(float(a2[b]) - float(alpha_ref)) < 1e-5
    # EM closed form: beta = R / mean_rows(|res|^2 + sum s^2/(obs s^2 + g2)), damped geometrically
    beta = ou.em_update_obs_precision(res, g2, S, obs, n, damping=1.0, lo=0, hi=1e30)
    s2 = S.double() ** 2
    den = np.mean([float((res[b].double() ** 2).sum() + (s2 / (obs * s2 + float(g2[b]))).sum()) for b in range(B)])
    assert abs(beta - n / den) < 1e-4 * beta


def test_nearest_atom_roundtrip_and_cd_fixed_point():
    g = torch.Generator().manual_seed(2)
    B, n, maxq = 6, 10, 3
    s = torch.rand(B, n, generator=g) * 0.02 + 0.001
    z = torch.randint(0, 4, (B, n), generator=g).float()
    q = torch.randint(0, maxq + 1, (B, n), generator=g)
    x = ou.dequant_from_q(q, s, z)
    assert torch.equal(ou.nearest_atom_idx(x, s, z, maxq).long(), q)
    # greedy CD on a tiny problem: objective non-increasing and a coordinate-wise fixed point
    A = torch.randn(n, n, generator=g)
    H = A @ A.T + 0.5 * torch.eye(n)
    lam, V = torch.linalg.eigh(H)
    Vs = V.flip(1) * lam.flip(0).sqrt()
    W = x + 0.01 * torch.randn(B, n, generator=g)
    Yu = W @ Vs
    xp, _ = ou.scalar_greedy_cd(x, Yu, Vs, Vs @ Vs.T, s, z, maxq, sweeps=30)
    e0 = ou.rankspace_error(Yu, x, Vs)
    e1 = ou.rankspace_error(Yu, xp, Vs)
    assert bool((e1 <= e0 + 1e-6).all())
    for b in range(B):
        for j in range(n):
            for qq in range(maxq + 1):
                xt = xp[b].clone()
                xt[j] = s[b, j] * (qq - z[b, j])
                assert float(((Yu[b] - xt @ Vs) ** 2).sum()) >= float(e1[b]) - 1e-5


# ---- golden vectors from the reference (tests/golden/make_golden.py) -----------------

@pytest.mark.parametrize("name", ["uvamp_r0_b4", "uvamp_r1_b3", "uvamp_r1_b4"])
def test_vamp_loop_matches_reference_golden(name):
    g = _load(name)
    torch.set_num_threads(1)
    cfg = dict(RECIPE, polish_sweeps=0)
    V, S = g["V"], g["S"]
    Vs = V * S.unsqueeze(0)
    q, x, e, rtn, tr = ou.solve_uniform_rankspace_vamp(g["W"], g["x_rtn"], g["scale_full"], g["zero_full"], g["maxq"],
                                                       V, V.T.contiguous(), S, Vs, cfg, gram_full=g["H"])
    assert tr["best_iter"] == g["best_iter"] and tr["stop_iter"] == g["stop_iter"]
    assert torch.equal(q, g["q_vamp"])
    assert torch.allclose(e, g["err_vamp"], rtol=1e-6, atol=0)
    assert abs(tr["obs_final"] - g["obs_final_vamp"]) <= 1e-9 * abs(g["obs_final_vamp"])
    # CD sweep (torch twin of the GPU kernel, update_backend="torch") from the VAMP output
    Yu = g["W"] @ Vs
    xv = ou.dequant_from_q(q, g["scale_full"], g["zero_full"])
    xt, _ = ou.scalar_greedy_cd(xv, Yu, Vs, g["H"], g["scale_full"], g["zero_full"], g["maxq"], 3, target_div=False)
    assert torch.equal(xt, g["x_cd_twin"])
    # the CPU dispatch polish (block_coordinate_descent_rankspace) for the final codes
    q2, _, e2, rtn2, _ = ou.solve_uniform_rankspace_vamp(g["W"], g["x_rtn"], g["scale_full"], g["zero_full"],
                                                        g["maxq"], V, V.T.contiguous(), S, Vs, RECIPE,
                                                        gram_full=g["H"], polish="block_cd")
    agree = float((q2 == g["q_final"]).float().mean())
    assert agree >= 0.999, agree
    assert torch.allclose(rtn2, g["rtn_err"], rtol=1e-6)


def test_reference_cd_dispatches_disagree():
    """Noise floor of code agreement: the reference's GPU-style sweep (rank-1 updates with H) and its
    CPU block CD (rank-space updates with Vs) differ only in rounding, yet not every code matches."""
    g = _load("uvamp_r1_b3")
    V, S = g["V"], g["S"]
    Vs = V * S.unsqueeze(0)
    Yu = g["W"] @ Vs
    xv = ou.dequant_from_q(g["q_vamp"], g["scale_full"], g["zero_full"])
    xa, _ = ou.scalar_greedy_cd(xv, Yu, Vs, g["H"], g["scale_full"], g["zero_full"], g["maxq"], 3)
    xb, _ = ou.block_cd_scalar(xv, Yu, Vs, g["scale_full"], g["zero_full"], g["maxq"], 3)
    agree = float((xa == xb).float().mean())
    print("reference CD dispatch agreement", agree)
    assert agree > 0.98
    ea = float(ou.rankspace_error(Yu, xa, Vs).mean())
    eb = float(ou.rankspace_error(Yu, xb, Vs).mean())
    assert abs(ea - eb) <= 0.005 * eb


def test_gptq_find_params_hand_computed():
    """The asymmetric min-max quantizer (GPTQModel Quantizer.find_params, un-vendored) against values
    computed by hand from its published formula: xmin = min(min(x), 0), xmax = max(max(x), 0), an
    all-zero group widened to [-1, 1], scale = (xmax - xmin) / maxq, zero = round(-xmin / scale)."""
    W = torch.tensor([
        [0.5, 1.0, 2.0, 3.0],     # all positive: xmin = 0 -> scale 3/3 = 1, zero 0
        [-1.5, 0.25, 3.0, 1.0],   # 4.5 / 15 rounds to fp32(0.3); 1.5 / fp32(0.3) = 4.99999982 -> zero 5
        [-2.0, -1.0, -0.5, -4.0],  # all negative: xmax = 0 -> scale fp32(4/7); 4 / fp32(4/7) = 7 -> zero 7
        [0.0, 0.0, 0.0, 0.0],     # all zero: [-1, 1] -> scale fp32(2/15) = 0.13333334;
                                  # 1 / 0.13333334 = 7.4999995 in fp32 -> round -> 7 (not 8)
    ])
    maxqs = [3, 15, 7, 15]
    want_scale = [1.0, float(torch.tensor(0.3)), float(torch.tensor(4.0) / 7), 0.13333334028720856]
    want_zero = [0.0, 5.0, 7.0, 7.0]
    for r, maxq in enumerate(maxqs):
        s, z = ou.gptq_find_params(W[r:r + 1], maxq)
        assert float(s) == want_scale[r], (r, float(s))
        assert float(z) == want_zero[r], (r, float(z))
    # the codes of the all-positive row: round(w / 1) + 0 clamped to [0, 3]
    s, z = ou.gptq_find_params(W[:1], 3)
    q = torch.clamp(torch.round(W[:1] / s) + z, 0, 3)
    assert q.tolist() == [[0.0, 1.0, 2.0, 3.0]]


def test_greedy_cd_sweeps_gain_order_only_changes_rounding():
    """With integer-valued data every sum is exact, so the row-order gain (``seq_gain``, the GPU's
    order) and torch's reduction order give bit-identical sweeps."""
    g = torch.Generator().manual_seed(11)
    rows, n = 24, 40
    Vs = torch.randint(-3, 4, (n, n), generator=g).float()
    H = Vs @ Vs.T
    scale = torch.ones(rows, n)
    zero = torch.full((rows, n), 4.0)
    x = torch.randint(-4, 4, (rows, n), generator=g).float()
    target = torch.randint(-40, 40, (rows, n), generator=g).float()
    Yu = target @ Vs
    res_u = Yu - x @ Vs
    rhs = res_u @ Vs.T
    res = res_u.square().sum(1)
    diag = Vs.square().sum(1).clamp_min(1e-12)
    a = ou.greedy_cd_sweeps(x, rhs, res, H, diag, scale, zero, 7, 3, seq_gain=False)
    b = ou.greedy_cd_sweeps(x, rhs, res, H, diag, scale, zero, 7, 3, seq_gain=True)
    assert int(a[3].sum()) > 0
    for u, v in zip(a, b):
        assert torch.equal(u, v)
    # every accepted move lowered the exact objective: the tracked residual equals the recomputed one
    assert torch.equal(a[2], (Yu - a[0] @ Vs).square().sum(1))
