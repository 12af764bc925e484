"""ORACLE (test infrastructure only) — uniform-grid per-layer path restated on the CPU.

torch CPU ops in the reference's operation order:

* ``discrete_uniform_mmse``      mpq/priors/uniform.py:99-213 (eager branch :177-213)
* ``nearest_atom_idx`` / ``dequant_from_q``   mpq/priors/uniform.py:287-309
* ``linear_mmse_exact``          mpq/linear.py:10-56
* ``em_update_obs_precision``    mpq/linear.py:59-82
* ``rankspace_error``            mpq/linear.py:85-94
* ``log_damp`` / masks           mpq/utils.py:25-68
* ``scalar_greedy_cd``           mpq/polish/triton_scalar_cd.py:164-307, update_backend="torch"
                                 (the column-at-a-time twin of the GPU sweep kernel)
* ``block_cd_scalar``            mpq/polish/block_cd.py:332-625 + UniformScalarProvider :628-653
                                 (the reference's CPU dispatch, block_size=1, metric diag)
* ``solve_uniform_rankspace_vamp``  mpq/solver.py:426-830
* ``gptq_find_params``           GPTQ asymmetric min-max quantizer (GPTQModel Quantizer.find_params,
                                 un-vendored: parity unpinned, standard published GPTQ formula)
* ``run_mpq_quantization``       mpq/adapters/gptqmodel.py:650-1163 (vamp solver, desc_act optional)
"""
from __future__ import annotations

import math
from typing import Any, Dict, Optional, Tuple

import torch

ALPHA_EPS = 1e-7

# Product rounding of the solve.  "fp32": torch's fp32 products (the reference's own arithmetic).
# "fp64": every product of the solve formed in fp64 and rounded to fp32 -- another valid rounding of
# the same products, used to measure how far last-bit differences move the discrete decisions.
_PRODUCTS = {"mode": "fp32"}


def _mm(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    if _PRODUCTS["mode"] == "fp64":
        out = a.double().matmul(b.double()).float()
        gen = _PRODUCTS.get("jitter")
        if gen is not None:  # move each entry to a random neighbouring float (or keep it)
            step = torch.randint(-1, 2, out.shape, generator=gen).to(torch.float32)
            up = torch.nextafter(out, torch.full_like(out, float("inf")))
            dn = torch.nextafter(out, torch.full_like(out, float("-inf")))
            out = torch.where(step > 0, up, torch.where(step < 0, dn, out))
        return out
    return a.matmul(b)


class products_in_fp64:
    """Context manager: the solve's products rounded from fp64 (see ``_PRODUCTS``); with ``jitter_seed``
    every entry of every product then moves to a random one of its two neighbouring floats or stays:
    a random valid fp32 rounding of the same products (errors well inside an fp32 GEMM's)."""

    def __init__(self, jitter_seed=None):
        self._seed = jitter_seed

    def __enter__(self):
        self._prev = dict(_PRODUCTS)
        _PRODUCTS["mode"] = "fp64"
        _PRODUCTS["jitter"] = None if self._seed is None else torch.Generator().manual_seed(int(self._seed))
        return self

    def __exit__(self, *exc):
        _PRODUCTS.clear()
        _PRODUCTS.update(self._prev)
        return False


# ---- utils (mpq/utils.py:18-68) --------------------------------------------

def stable_seed(key: str, base_seed: int = 0) -> int:
    import hashlib

    extra = int.from_bytes(hashlib.sha256(str(key).encode("utf-8")).digest()[:4], "little")
    return int((int(base_seed) + extra) % (2 ** 31 - 1))


def log_damp(prev: torch.Tensor, new: torch.Tensor, d: float) -> torch.Tensor:
    if d >= 1.0:
        return new
    if d <= 0.0:
        return prev
    return torch.exp((1.0 - d) * torch.log(prev.clamp_min(1e-12)) + d * torch.log(new.clamp_min(1e-12)))


def log_damp_scalar(prev: float, new: float, d: float) -> float:
    if d >= 1.0:
        return float(new)
    if d <= 0.0:
        return float(prev)
    return float(math.exp((1.0 - d) * math.log(max(prev, 1e-12)) + d * math.log(max(new, 1e-12))))


def alpha_valid(a: torch.Tensor) -> torch.Tensor:
    return torch.isfinite(a) & (a > ALPHA_EPS) & (a < 1.0 - ALPHA_EPS)


def prec_valid(g: torch.Tensor) -> torch.Tensor:
    return torch.isfinite(g) & (g > 1e-12)


# ---- prior (mpq/priors/uniform.py) ----------------------------------------

def discrete_uniform_mmse(r1, gamma1, scale_full, zero_full, maxq, prior_center, prior_tau):
    atoms = scale_full.unsqueeze(-1) * (
        torch.arange(maxq + 1, dtype=torch.float32).view(1, 1, -1) - zero_full.unsqueeze(-1))
    scores = -0.5 * gamma1.unsqueeze(-1) * (atoms - r1.unsqueeze(-1)).square()
    if prior_tau > 0.0:
        st2 = (prior_tau * scale_full.clamp_min(1e-12)).square().unsqueeze(-1)
        scores = scores - 0.5 * (atoms - prior_center.unsqueeze(-1)).square() / st2
    log_probs = scores - torch.logsumexp(scores, dim=-1, keepdim=True)
    probs = torch.exp(log_probs)
    mean = (probs * atoms).sum(dim=-1)
    second = (probs * atoms.square()).sum(dim=-1)
    var = (second - mean.square()).clamp_min_(0.0)
    map_idx = torch.argmax(scores, dim=-1)
    map_value = torch.gather(atoms, -1, map_idx.unsqueeze(-1)).squeeze(-1)
    alpha1 = gamma1 * var.mean(dim=1, keepdim=True)
    return {"mean": mean, "var": var, "map_value": map_value, "map_idx": map_idx, "alpha1": alpha1}


def nearest_atom_idx(x, scale_full, zero_full, maxq):
    q = torch.round(x / scale_full.clamp_min(1e-12) + zero_full)
    return torch.clamp(q, 0, int(maxq)).to(torch.int32)


def dequant_from_q(q, scale_full, zero_full):
    return scale_full * (q.to(torch.float32) - zero_full)


# ---- linear module (mpq/linear.py) ----------------------------------------

def linear_mmse_exact(r2, gamma2, Y_u, V, Vh, S, obs):
    n = r2.shape[1]
    R = S.numel()
    s = S.unsqueeze(0)
    denom = float(obs) * s.square() + gamma2
    r2v = _mm(r2, V)
    rb = Y_u - r2v * s
    coeff = float(obs) * s / denom
    x2 = r2 + _mm(rb * coeff, Vh)
    alpha2 = 1.0 - (float(R) / float(n)) + (gamma2 / float(n)) * (1.0 / denom).sum(dim=1, keepdim=True)
    return x2, alpha2, rb * (gamma2 / denom)


def em_update_obs_precision(residual_u, gamma2, S, obs, num_obs, damping=0.3, lo=1e-4, hi=1e8):
    s2 = S.square().unsqueeze(0)
    trace = (s2 / (float(obs) * s2 + gamma2)).sum(dim=1, keepdim=True)
    resid = residual_u.square().sum(dim=1, keepdim=True)
    den = (resid + trace).mean().clamp_min_(1e-12)
    beta_new = float(num_obs / den.item())
    beta = log_damp_scalar(max(float(obs), 1e-12), beta_new, damping)
    return float(min(max(beta, lo), hi))


def rankspace_error(Y_u, x, Vs):
    return (Y_u - _mm(x, Vs)).square().sum(dim=1)


# ---- polish ----------------------------------------------------------------

def scalar_greedy_cd(x, Y_u, Vs, gram, scale, zero, maxq, sweeps, accept_tol=0.0, target_div=True,
                     seq_gain=False, f64_products=False):
    """mpq/polish/triton_scalar_cd.py:164-307 (per-column order, torch ops).

    ``target_div=True`` forms the RTN target as ``x + rhs / diag`` like the GPU sweep kernel the
    reference dispatches on CUDA (:73); ``False`` uses the torch twin's ``x + rhs * (1/diag)`` (:265).
    ``seq_gain``: see ``greedy_cd_sweeps``.  ``f64_products`` forms the starting residual, rhs and
    diagonal in fp64 and rounds them to fp32 (another valid rounding of the same start, used to
    measure how far last-bit differences of the products move the greedy decisions).
    """
    x = x.to(torch.float32).clone()
    if f64_products:
        V64 = Vs.double()
        ru = Y_u.double() - x.double().matmul(V64)
        rhs = ru.matmul(V64.T).float()
        res = ru.square().sum(dim=1).float()
        diag = V64.square().sum(dim=1).float().clamp_min_(1e-12)
        gen = _PRODUCTS.get("jitter")
        if gen is not None:
            step = torch.randint(-1, 2, rhs.shape, generator=gen).to(torch.float32)
            up = torch.nextafter(rhs, torch.full_like(rhs, float("inf")))
            dn = torch.nextafter(rhs, torch.full_like(rhs, float("-inf")))
            rhs = torch.where(step > 0, up, torch.where(step < 0, dn, rhs))
    else:
        res_u = Y_u - x.matmul(Vs)
        rhs = res_u.matmul(Vs.T.contiguous())
        res = res_u.square().sum(dim=1)
        diag = Vs.square().sum(dim=1).clamp_min_(1e-12)
    x, rhs, res, acc_rows = greedy_cd_sweeps(x, rhs, res, gram, diag, scale, zero, maxq, sweeps,
                                             accept_tol=accept_tol, target_div=target_div, seq_gain=seq_gain)
    return x, int(acc_rows.sum())


def greedy_cd_sweeps(x, rhs, res, gram, diag, scale, zero, maxq, sweeps, accept_tol=0.0, target_div=True,
                     seq_gain=False):
    """The sweeps of mpq/polish/triton_scalar_cd.py:240-288 on given state (x, rhs = residual Vs^T,
    res = |residual|^2 per row, diag = |Vs_j|^2 floored); returns new (x, rhs, res, accepted per row).

    Per sweep: gain = mean over rows of rhs^2 * (1/diag) (:241), stable descending order (:242; the
    reference's argsort is unstable, ties are broken by index here), then per column in order the RTN
    target, the accept test ``cand + 1e-12 < res * (1 + tol)`` and the rank-1 update
    ``rhs -= delta * gram[col, :]`` (:265-288), each operation rounded to fp32 as torch evaluates it.
    ``seq_gain=True`` sums the gain over rows in row order (one fp32 addition per row, as the GPU
    sweep does) instead of torch's reduction order; everything else is the same.
    """
    x = x.to(torch.float32).clone()
    rhs = rhs.to(torch.float32).clone()
    res = res.to(torch.float32).clone()
    dinv = diag.reciprocal()
    rows = x.shape[0]
    acc_rows = torch.zeros(rows, dtype=torch.int64)
    zero_d = torch.zeros(rows)
    for _ in range(sweeps):
        terms = rhs.square() * dinv.unsqueeze(0)
        if seq_gain:
            g = torch.zeros(rhs.shape[1])
            for r in range(rows):
                g = g + terms[r]
            gain = g / float(max(rows, 1))
        else:
            gain = terms.sum(dim=0) / float(max(rows, 1))
        order = torch.argsort(gain, descending=True, stable=True)
        for col in order.tolist():
            r = rhs[:, col]
            xc = x[:, col]
            sc = scale[:, col].clamp_min(1e-12)
            zc = zero[:, col]
            target = xc + r / diag[col] if target_div else xc + r * dinv[col]
            q = torch.clamp(torch.round(target / sc + zc), 0, maxq).to(torch.int32)
            xq = sc * (q.to(torch.float32) - zc)
            d = xq - xc
            cand = (res + d.square() * diag[col] - 2.0 * r * d).clamp_min_(0.0)
            acc = cand + 1e-12 < res * (1.0 + accept_tol)
            if not bool(acc.any()):
                continue
            x[:, col] = torch.where(acc, xq, xc)
            res = torch.where(acc, cand, res)
            acc_rows += acc.to(torch.int64)
            rhs.sub_(torch.where(acc, d, zero_d).unsqueeze(1) * gram[col].unsqueeze(0))
    return x, rhs, res, acc_rows


def block_cd_scalar(x, Y_u, Vs, scale, zero, maxq, sweeps, accept_tol=0.0, max_cols=0, order_mode="greedy_gain"):
    """mpq/polish/block_cd.py:332-625, block_size=1, metric diag (CPU dispatch); ``order_mode``
    greedy_gain (per sweep, :505-507), static (trace of each column's gram, descending, :418-420) or
    cyclic (:508-509), stable sorts.

    ``max_cols`` > 0 stops each sweep after that many columns (a bounded sample for timing).
    """
    B, n = x.shape
    x = x.to(torch.float32).clone()
    Vs_t = Vs.T.contiguous()
    res_u = Y_u - x.matmul(Vs)
    res = res_u.square().sum(dim=1)
    gram_diag = Vs.square().sum(dim=1)
    dinv_all = gram_diag.clamp_min(1e-12).reciprocal()
    accepted = 0
    static = torch.argsort(gram_diag, descending=True, stable=True).tolist()
    for _ in range(sweeps):
        if order_mode == "greedy_gain":
            rhs_all = res_u.matmul(Vs_t)
            gain = (rhs_all.square() * dinv_all.unsqueeze(0)).mean(dim=0)
            order = torch.argsort(gain, descending=True, stable=True).tolist()
        elif order_mode == "static":
            order = list(static)
        else:
            order = list(range(n))
        if max_cols > 0:
            order = order[:max_cols]
        for j in order:
            xb = x[:, j:j + 1]
            rhs = res_u.matmul(Vs_t[:, j:j + 1])
            target = xb + rhs * dinv_all[j]
            sc = scale[:, j:j + 1].clamp_min(1e-12)
            q = torch.clamp(torch.round(target / sc + zero[:, j:j + 1]), 0, maxq).to(torch.int32)
            cand_v = sc * (q.to(torch.float32) - zero[:, j:j + 1])
            delta = cand_v - xb
            cross = (rhs * delta).sum(dim=1)
            dn = (delta.matmul(gram_diag[j].view(1, 1)) * delta).sum(dim=1).clamp_min_(0.0)
            cand = (res + dn - 2.0 * cross).clamp_min_(0.0)
            acc = cand + 1e-12 < res * (1.0 + accept_tol)
            x[:, j:j + 1] = torch.where(acc.unsqueeze(1), cand_v, xb)
            delta = delta * acc.unsqueeze(1)
            res_u.sub_(delta.matmul(Vs[j:j + 1]))
            res = torch.where(acc, cand, res)
            accepted += int(acc.sum())
    return x, accepted


# ---- solver (mpq/solver.py:426-830) ------------------------------------------

def solve_uniform_rankspace_vamp(W, x_rtn, scale_full, zero_full, maxq, V, Vh, S, Vs, cfg: Dict[str, Any],
                                 gram_full=None, obs_precision_init=None, polish: str = "twin"):
    """Returns (q int32, x, err, rtn_err, stats).  polish: "twin" (the CUDA sweep's semantics) |
    "twin_rowsum" (the same with the greedy gain summed over rows in row order) | "twin_f64prod" (the
    same with the polish's starting products rounded from fp64) | "block_cd" (CPU)."""
    iters = int(cfg.get("iters", 16))
    damping = float(cfg.get("damping", 0.5))
    tau = float(cfg.get("prior_tau", 0.2))
    gamma_start = float(cfg.get("gamma_start", 1.0))
    retry_factor = max(float(cfg.get("gamma_retry_factor", 4.0)), 1.000001)
    retry_steps = max(int(cfg.get("gamma_retry_steps", 3)), 0)
    em_on = bool(cfg.get("em_obs_precision", True)) and float(cfg.get("obs_precision", 0.0)) <= 0.0
    sweeps = int(cfg.get("polish_sweeps", 3))
    R = S.numel()
    # r1 start (mpq/solver.py:472-479): the RTN decision, the float weight or zero
    init_from = str(cfg.get("init_from", "rtn") or "rtn").strip().lower()
    r1 = {"rtn": x_rtn, "float": W, "zero": torch.zeros_like(W)}[init_from].clone()
    gamma1 = gamma_start * (0.25 / (W - x_rtn).square().mean(dim=1, keepdim=True).clamp_min_(1e-12))
    Y_u = _mm(W, Vs)
    requested = float(cfg.get("obs_precision", 0.0))
    if obs_precision_init is not None and obs_precision_init > 0:
        obs = float(obs_precision_init)
    elif math.isfinite(requested) and requested > 0.0:  # _resolve_obs_precision (mpq/solver.py:147-161)
        obs = requested
    else:
        obs = 1.0 / float((Y_u - _mm(x_rtn, Vs)).square().mean().clamp_min_(1e-12).item())

    # final decision (mpq/solver.py:833-850): the MAP atom, or "round_mean" the posterior mean rounded
    round_mean = str(cfg.get("final_decision", "map") or "map").strip().lower() == "round_mean"

    def hard(r, g):
        post = discrete_uniform_mmse(r, g, scale_full, zero_full, maxq, W, tau)
        q = nearest_atom_idx(post["mean"] if round_mean else post["map_value"], scale_full, zero_full, maxq)
        xs = dequant_from_q(q, scale_full, zero_full)
        return q, xs, rankspace_error(Y_u, xs, Vs)

    best_q, best_x, best_err = hard(r1, gamma1)
    best_mean = float(best_err.mean().item())
    best_obs = obs
    r2_prev = g2_prev = None
    trace = {"best_iter": -1, "stop_iter": -1, "obs": [], "err": [best_mean], "gamma2_invalid": 0}
    for it in range(iters):
        g1w = gamma1
        for attempt in range(retry_steps + 1):
            post = discrete_uniform_mmse(r1, g1w, scale_full, zero_full, maxq, W, tau)
            a1 = post["alpha1"]
            if bool(alpha_valid(a1).all()):
                x1 = post["mean"]
                break
            if attempt >= retry_steps:
                if not bool(torch.isfinite(a1).all()):
                    raise RuntimeError("alpha1 invalid")
                a1 = torch.nan_to_num(a1, nan=0.5, posinf=1.0 - ALPHA_EPS, neginf=ALPHA_EPS).clamp(
                    min=ALPHA_EPS, max=1.0 - ALPHA_EPS)
                x1 = post["mean"]
                break
            g1w = torch.where(a1 <= ALPHA_EPS, g1w / retry_factor, g1w)
            g1w = torch.where(a1 >= 1.0 - ALPHA_EPS, g1w * retry_factor, g1w).clamp_min_(1e-12)
        eta1 = g1w / a1
        g2n = torch.nan_to_num(eta1 - g1w, nan=1e-12, posinf=1e12, neginf=1e-12).clamp_min_(1e-12)
        if not bool(prec_valid(g2n).all()):
            trace["gamma2_invalid"] += 1
            continue
        r2n = (eta1 * x1 - g1w * r1) / g2n
        if r2_prev is None or damping >= 1.0:
            g2, r2 = g2n, r2n
        else:
            g2 = log_damp(g2_prev, g2n, damping)
            r2 = (1.0 - damping) * r2_prev + damping * r2n
        if not bool(prec_valid(g2).all()):
            trace["gamma2_invalid"] += 1
            continue
        x2, a2, res_u = linear_mmse_exact(r2, g2, Y_u, V, Vh, S, obs)
        a2 = torch.nan_to_num(a2, nan=0.5, posinf=1.0 - ALPHA_EPS, neginf=ALPHA_EPS).clamp(
            min=ALPHA_EPS, max=1.0 - ALPHA_EPS)
        if em_on:
            obs = em_update_obs_precision(res_u, g2, S, obs, R,
                                          float(cfg.get("em_obs_precision_damping", 0.3)),
                                          float(cfg.get("em_obs_precision_min", 1e-4)),
                                          float(cfg.get("em_obs_precision_max", 1e8)))
        eta2 = g2 / a2
        g1n = torch.nan_to_num(eta2 - g2, nan=1e-12, posinf=1e12, neginf=1e-12).clamp_min_(1e-12)
        r1n = (eta2 * x2 - g2 * r2) / g1n
        if damping >= 1.0:
            gamma1, r1 = g1n, r1n
        else:
            gamma1 = log_damp(gamma1, g1n, damping)
            r1 = (1.0 - damping) * r1 + damping * r1n
        r2_prev, g2_prev = r2, g2
        trace["obs"].append(obs)
        cq, cx, ce = hard(r1, gamma1)
        cm = float(ce.mean().item())
        trace["err"].append(cm)
        tol = max(1e-10, abs(best_mean) * 1e-8)
        if cm + tol < best_mean:
            best_q, best_x, best_err, best_mean, best_obs = cq, cx, ce, cm, obs
            trace["best_iter"] = it
        else:
            obs = best_obs
            trace["stop_iter"] = it
            break
    q_final, x_final, err_final = best_q, best_x, best_err
    trace["vamp_err"] = best_err.clone()
    trace["q_vamp"] = best_q.clone()
    if sweeps > 0:
        err_before = rankspace_error(Y_u, x_final, Vs)
        if polish in ("twin", "twin_rowsum", "twin_f64prod"):
            gram = gram_full if gram_full is not None else Vs.matmul(Vs.T)
            xp, acc = scalar_greedy_cd(x_final, Y_u, Vs, gram, scale_full, zero_full, maxq, sweeps,
                                       seq_gain=polish == "twin_rowsum",
                                       f64_products=polish == "twin_f64prod" or _PRODUCTS["mode"] == "fp64")
        else:
            xp, acc = block_cd_scalar(x_final, Y_u, Vs, scale_full, zero_full, maxq, sweeps)
        qp = nearest_atom_idx(xp, scale_full, zero_full, maxq)
        xo = dequant_from_q(qp, scale_full, zero_full)
        err_after = rankspace_error(Y_u, xo, Vs)
        imp = err_after + 1e-12 < err_before
        q_final = torch.where(imp.unsqueeze(-1), qp, q_final)
        x_final = torch.where(imp.unsqueeze(-1), xo, x_final)
        err_final = torch.where(imp, err_after, err_final)
        trace["polish_accepted"] = acc
    trace["obs_final"] = obs
    rtn_err = rankspace_error(Y_u, x_rtn, Vs)
    return q_final, x_final, err_final, rtn_err, trace


# ---- adapter (mpq/adapters/gptqmodel.py:650-1163) -----------------------------

def gptq_find_params(Wg: torch.Tensor, maxq: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Asymmetric min-max GPTQ quantizer parameters per row (parity unpinned: GPTQModel absent)."""
    tmp = torch.zeros(Wg.shape[0])
    xmin = torch.minimum(Wg.min(dim=1).values, tmp)
    xmax = torch.maximum(Wg.max(dim=1).values, tmp)
    both = (xmin == 0) & (xmax == 0)
    xmin[both] = -1
    xmax[both] = +1
    scale = (xmax - xmin) / maxq
    zero = torch.round(-xmin / scale)
    return scale.unsqueeze(1), zero.unsqueeze(1)


def hessian_eigen(H: torch.Tensor, jitter_base=1e-6, floor_scale=1e-6):
    """mpq/adapters/gptqmodel.py:276-310."""
    H = 0.5 * (H + H.T)
    if not torch.isfinite(H).all():
        H = torch.nan_to_num(H, nan=0.0, posinf=0.0, neginf=0.0)
    lam, V = torch.linalg.eigh(H)
    max_lam = float(lam.max().item())
    diag_mean = float(torch.diagonal(H).mean().abs().item())
    floor = max(jitter_base, floor_scale * max(diag_mean, max_lam, 1e-12))
    return lam.clamp_min_(floor).flip(0).contiguous(), V.flip(1).contiguous(), floor


def hadamard_rows(X: torch.Tensor, had: int) -> torch.Tensor:
    """Sylvester block Walsh-Hadamard along the last dim, strides 1,2,4,... (mpq/rotation.py:135-156)."""
    shape = X.shape
    x = X.reshape(-1, had).clone()
    h = 1
    while h < had:
        x = x.view(-1, had // (2 * h), 2, h)
        a = x[:, :, 0, :].clone()
        b = x[:, :, 1, :].clone()
        x[:, :, 0, :] = a + b
        x[:, :, 1, :] = a - b
        x = x.reshape(-1, had)
        h *= 2
    return (x / torch.tensor(had).sqrt()).reshape(shape)


def rotation_plan(n: int, module_name: str, seed: int = 0):
    had = n & -n
    if had < 2:
        return None
    g = torch.Generator(device="cpu")
    g.manual_seed(stable_seed(f"{module_name}:full", base_seed=seed))
    signs = torch.randint(0, 2, (n,), generator=g, dtype=torch.int64).to(torch.float32).mul_(2.0).sub_(1.0)
    return signs, had


def run_mpq_quantization(W, H, bits, group_size, module_name, cfg, rotation="none", block_rows=128,
                         polish: str = "twin", hessian_scale=0.5, desc_act: bool = False):
    """CPU restatement of the per-linear scalar driver; returns dict with Q, q_int, scale, zero, stats.
    ``desc_act``: columns in descending order of the solver-basis Hessian's diagonal (stable sort;
    mpq/adapters/gptqmodel.py:733-740), the decomposition of that permuted Hessian (:716-722 apply
    only without it), the results permuted back (:1090-1095)."""
    W = W.to(torch.float32)
    rows, cols = W.shape
    maxq = 2 ** bits - 1
    H_work = float(hessian_scale) * H.to(torch.float32)
    if not desc_act:
        lam, V, floor = hessian_eigen(H_work)
    plan = rotation_plan(cols, module_name) if rotation == "internal_hadamard" else None
    if plan is not None:
        signs, had = plan
        W_work = hadamard_rows(W * signs.view(1, -1), had)
        Hm = hadamard_rows(H_work.T.contiguous() * signs.view(1, -1), had).T.contiguous()
        Hm = hadamard_rows(Hm * signs.view(1, -1), had)
        if not desc_act:
            V = hadamard_rows(V.T.contiguous() * signs.view(1, -1), had).T.contiguous()
    else:
        W_work, Hm = W, H_work
    invperm = None
    if desc_act:
        perm = torch.argsort(torch.diagonal(Hm), descending=True, stable=True)
        invperm = torch.argsort(perm)
        W_work = W_work.index_select(1, perm).contiguous()
        Hm = Hm.index_select(0, perm).index_select(1, perm).contiguous()
        lam, V, floor = hessian_eigen(Hm)
    S = torch.sqrt(lam)
    Vs = V * S.unsqueeze(0)
    Vh = V.T.contiguous()
    G = (cols + group_size - 1) // group_size
    sc, zc = [], []
    for g in range(G):
        s, z = gptq_find_params(W_work[:, g * group_size:(g + 1) * group_size], maxq)
        sc.append(s)
        zc.append(z)
    scale_g = torch.cat(sc, 1)
    zero_g = torch.cat(zc, 1)
    widths = torch.tensor([min(group_size, cols - g * group_size) for g in range(G)])
    sum_sq = 0.0
    count = 0
    for r0 in range(0, rows, block_rows):
        rb = slice(r0, min(r0 + block_rows, rows))
        sf = torch.repeat_interleave(scale_g[rb], widths, dim=1)
        zf = torch.repeat_interleave(zero_g[rb], widths, dim=1)
        qr = torch.clamp(torch.round(W_work[rb] / sf) + zf, 0, maxq)
        du = _mm(W_work[rb] - sf * (qr - zf), Vs)
        sum_sq += float(du.square().sum().item())
        count += du.numel()
    obs = 1.0 / max(sum_sq / max(count, 1), 1e-12)
    Q_work = torch.empty_like(W_work)
    q_int = torch.empty(rows, cols, dtype=torch.uint8)
    obs_block = obs
    traces = []
    for r0 in range(0, rows, block_rows):
        rb = slice(r0, min(r0 + block_rows, rows))
        sf = torch.repeat_interleave(scale_g[rb], widths, dim=1)
        zf = torch.repeat_interleave(zero_g[rb], widths, dim=1)
        qr = torch.clamp(torch.round(W_work[rb] / sf) + zf, 0, maxq)
        xr = sf * (qr - zf)
        q, x, err, rtn_err, tr = solve_uniform_rankspace_vamp(W_work[rb], xr, sf, zf, maxq, V, Vh, S, Vs, cfg,
                                                              gram_full=Hm, obs_precision_init=obs_block,
                                                              polish=polish)
        Q_work[rb] = x
        q_int[rb] = q.to(torch.uint8)
        obs_block = tr["obs_final"]
        traces.append(tr)
    delta = W_work - Q_work
    proxy = (delta.matmul(Hm) * delta).sum(dim=1)
    g_idx = torch.arange(cols, dtype=torch.int32) // int(group_size)
    if invperm is not None:
        Q_work = Q_work.index_select(1, invperm)
        q_int = q_int.index_select(1, invperm)
        g_idx = g_idx.index_select(0, invperm)
    if plan is not None:
        signs, had = plan
        Q = hadamard_rows(Q_work, had) * signs.view(1, -1)
    else:
        Q = Q_work
    return {"Q": Q, "Q_work": Q_work, "q_int": q_int, "scale": scale_g, "zero": zero_g, "g_idx": g_idx, "obs_initial": obs,
            "obs_final": obs_block, "proxy_rows": proxy, "traces": traces, "W_work": W_work, "H_metric": Hm,
            "V": V, "S": S, "eigen_floor": floor}
