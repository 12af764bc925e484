"""ORACLE (test infrastructure only) — E8P12 prior restated on the CPU.

* ``factor_cache``        follows mpq/priors/e8p12.py:83-151 (get_e8p12_factor_cache),
                          including its structural invariants (:121-130).
* ``map_search``          wraps the C restatement oracle/e8p12_map.c of
                          mpq/priors/e8p12.py:367-449 + :541-631.
* ``bruteforce_nearest``  exhaustive fp64 search over all 65536 codewords (the
                          mathematical definition the factorized search must equal).
* ``posterior``           follows mpq/priors/e8p12.py:154-308 + :815-968
                          (vamp_vector_discrete_mmse_e8p12) with torch CPU ops in the
                          reference's order.
* ``posterior_bruteforce``  fp64 softmax over all 65536 codewords (pins ``posterior``).
* ``posterior_stats_bruteforce``  fp64 logZ / entropy / margin over all codewords (the
                          diagnostics of mpq/priors/e8p12.py:276-305, 885-953; its logZ is pinned by
                          the reference's golden logZ_blocks).
"""
from __future__ import annotations

import ctypes
import math
import os
from typing import Dict, Optional

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(HERE, "liboracle.so")
_lib = None


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            import subprocess

            subprocess.run(["make", "-C", HERE, "-s"], check=True)
        lib = ctypes.CDLL(_LIB_PATH)
        p = ctypes.c_void_p
        lib.oracle_e8p12_map.argtypes = [p, ctypes.c_int64, p, ctypes.c_int64, p, p, ctypes.c_float,
                                         p, p, p, p, p, p]
        lib.oracle_e8p12_map.restype = None
        lib.oracle_e8p12_sqerr.argtypes = [p, p, ctypes.c_int64, p, p]
        lib.oracle_e8p12_bruteforce.argtypes = [p, ctypes.c_int64, p, p, p]
        _lib = lib
    return _lib


def _sign_parity(ids: torch.Tensor) -> torch.Tensor:
    bits = (ids.unsqueeze(-1) >> torch.arange(8)) & 1
    return bits.sum(dim=-1) & 1


def factor_cache(grid: torch.Tensor) -> Dict[str, torch.Tensor]:
    """Factor tables of a 65536x8 grid; mpq/priors/e8p12.py:83-151."""
    grid = grid.to(dtype=torch.float32, device="cpu")
    if tuple(grid.shape) != (65536, 8):
        raise ValueError("expected a 65536x8 grid")
    seed = torch.arange(256, dtype=torch.long) << 8
    template = grid.index_select(0, seed) - 0.25
    base_parity = ((template < 0).long().sum(dim=-1) & 1)
    base_abs = template.abs()
    base_sqnorm = base_abs.square().sum(dim=-1)
    full = torch.arange(65536, dtype=torch.long)
    abs_idx = full >> 8
    branch = _sign_parity(full & 255)
    offsets = torch.tensor([0.25, -0.25], dtype=torch.float32)
    residual = grid - offsets.index_select(0, branch).unsqueeze(-1)
    sign_id = ((residual < 0).long() * (1 << torch.arange(8))).sum(dim=-1)
    lut = torch.full((2, 256, 256), -1, dtype=torch.long)
    lut[branch, abs_idx, sign_id] = full
    if not torch.allclose(residual.abs(), base_abs.index_select(0, abs_idx), atol=1e-6, rtol=1e-6):
        raise RuntimeError("grid does not factor into 256 abs patterns")
    valid = _sign_parity(torch.arange(256)).view(1, 1, -1) == base_parity.view(1, 256, 1)
    if not torch.all(lut[valid.expand(2, -1, -1)] >= 0):
        raise RuntimeError("missing valid sign entries")
    if not torch.all(lut[~valid.expand(2, -1, -1)] < 0):
        raise RuntimeError("unexpected invalid sign entries")
    return {
        "base_abs": base_abs.contiguous(),
        "base_sqnorm": base_sqnorm.contiguous(),
        "base_parity": base_parity.to(torch.int32).contiguous(),
        "idx_lut": lut.contiguous(),
        "branch_offsets": offsets,
    }


def map_search(r: np.ndarray, gamma: np.ndarray, gamma_div: int, cache: Dict[str, torch.Tensor],
               center: Optional[np.ndarray] = None, scale: Optional[np.ndarray] = None,
               tau: float = 0.0):
    """(idx int64, best score fp32) of the factorized MAP; oracle/e8p12_map.c."""
    lib = _load()
    r = np.ascontiguousarray(r, dtype=np.float32).reshape(-1, 8)
    n = r.shape[0]
    gamma = np.ascontiguousarray(gamma, dtype=np.float32).reshape(-1)
    idx = np.empty(n, dtype=np.int64)
    score = np.empty(n, dtype=np.float32)
    babs = cache["base_abs"].numpy()
    bsq = cache["base_sqnorm"].numpy()
    bpar = cache["base_parity"].numpy()
    lut = cache["idx_lut"].numpy()
    c_arr = s_arr = None
    if center is not None and tau > 0.0:
        c_arr = np.ascontiguousarray(center, dtype=np.float32).reshape(-1, 8)
        if scale is None:
            scale = np.abs(c_arr).max(axis=1)
        s_arr = np.ascontiguousarray(scale, dtype=np.float32).reshape(-1)
    P = lambda a: None if a is None else a.ctypes.data  # noqa: E731
    lib.oracle_e8p12_map(P(r), n, P(gamma), int(gamma_div), P(c_arr), P(s_arr), float(tau),
                         P(babs), P(bsq), P(bpar), P(lut), P(idx), P(score))
    return idx, score


def sqerr(x: np.ndarray, idx: np.ndarray, grid: np.ndarray) -> np.ndarray:
    lib = _load()
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, 8)
    idx = np.ascontiguousarray(idx, dtype=np.int64)
    grid = np.ascontiguousarray(grid, dtype=np.float32)
    out = np.empty(x.shape[0], dtype=np.float32)
    lib.oracle_e8p12_sqerr(x.ctypes.data, idx.ctypes.data, x.shape[0], grid.ctypes.data, out.ctypes.data)
    return out


def bruteforce_nearest(x: np.ndarray, grid: np.ndarray):
    lib = _load()
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, 8)
    grid = np.ascontiguousarray(grid, dtype=np.float32)
    idx = np.empty(x.shape[0], dtype=np.int64)
    dist = np.empty(x.shape[0], dtype=np.float64)
    lib.oracle_e8p12_bruteforce(x.ctypes.data, x.shape[0], grid.ctypes.data, idx.ctypes.data, dist.ctypes.data)
    return idx, dist


# ---------------------------------------------------------------------------
# Posterior (denoiser) restatement, torch CPU, reference op order.
# ---------------------------------------------------------------------------

def _log1mexp(x: torch.Tensor) -> torch.Tensor:
    cutoff = -math.log(2.0)
    return torch.where(x < cutoff, torch.log1p(-torch.exp(x)), torch.log(-torch.expm1(x)))


def _branch_stats(y: torch.Tensor, g: torch.Tensor, offset: float, branch: int, cache,
                  need_stats: bool = False) -> Dict[str, torch.Tensor]:
    """mpq/priors/e8p12.py:169-308 (_branch_factorized_stats_impl)."""
    base_abs = cache["base_abs"].view(1, 256, 8)
    sq = cache["base_sqnorm"].view(1, 256)
    parity_even = (cache["base_parity"] == 0).view(1, 256)
    bits = (1 << torch.arange(8)).view(1, 1, 8)
    n = y.shape[0]
    a = g.view(n, 1, 1) * y.view(n, 1, 8) * base_abs
    y_norm = y.square().sum(dim=-1, keepdim=True)
    const = -0.5 * g[:, :1] * (y_norm + sq)
    logC = torch.logaddexp(a, -a).sum(dim=-1)
    t = torch.tanh(a)
    t_safe = t.clamp(min=-1.0 + 1e-7, max=1.0 - 1e-7)
    log_abs_prod = torch.log(t_safe.abs().clamp_min(1e-7)).sum(dim=-1)
    neg = ((t_safe < 0).sum(dim=-1) & 1).bool()
    prod_abs = torch.exp(log_abs_prod)
    prod = torch.where(neg, -prod_abs, prod_abs)
    one = torch.ones_like(prod)
    zeros = torch.zeros_like(log_abs_prod)
    lp1 = torch.where(neg, _log1mexp(log_abs_prod), torch.logaddexp(zeros, log_abs_prod))
    lm1 = torch.where(neg, torch.logaddexp(zeros, log_abs_prod), _log1mexp(log_abs_prod))
    logZ_even = logC + lp1 - math.log(2.0)
    logZ_odd = logC + lm1 - math.log(2.0)
    logZ_sign = torch.where(parity_even, logZ_even, logZ_odd)
    prefix = []
    acc = one
    for c in range(8):
        prefix.append(acc)
        acc = acc * t_safe[:, :, c]
    sign_mean = torch.empty((n, 256, 8), dtype=torch.float32)
    suffix = one
    de = one + prod
    do = one - prod
    de_s = torch.where(de.abs() > 1e-12, de, torch.ones_like(de))
    do_s = torch.where(do.abs() > 1e-12, do, torch.ones_like(do))
    for c in reversed(range(8)):
        tc = t_safe[:, :, c]
        excl = prefix[c] * suffix
        sign_mean[:, :, c] = torch.where(parity_even, (tc + excl) / de_s, (tc - excl) / do_s)
        suffix = suffix * tc
    sign_mean = torch.nan_to_num(sign_mean, nan=0.0, posinf=0.0, neginf=0.0)
    mu_core = sign_mean * base_abs
    mu = mu_core + float(offset)
    second = sq + 8 * float(offset) * float(offset) + 2.0 * float(offset) * mu_core.sum(dim=-1)
    del bits
    out = {"log_component": const + logZ_sign, "mu_component": mu, "second_component": second}
    if need_stats:  # mpq/priors/e8p12.py:276-305
        abs_a = a.abs()
        sum_abs = abs_a.sum(dim=-1)
        best_parity = (a < 0).long().sum(dim=-1) & 1
        min_pos = abs_a.argmin(dim=-1)
        min_abs = abs_a.gather(-1, min_pos.unsqueeze(-1)).squeeze(-1)
        mismatch = best_parity != cache["base_parity"].view(1, 256)
        out["best_logscore"] = const + (sum_abs - 2.0 * mismatch.to(torch.float32) * min_abs)
        second_abs = abs_a.clone()
        second_abs.scatter_(-1, min_pos.unsqueeze(-1), float("inf"))
        second_min = second_abs.min(dim=-1).values
        second_lin = torch.where(mismatch, sum_abs - 2.0 * second_min, sum_abs - 2.0 * (min_abs + second_min))
        out["second_logscore"] = const + second_lin
        out["sign_entropy"] = torch.where(torch.isfinite(logZ_sign),
                                          (logZ_sign - (a * sign_mean).sum(dim=-1)).clamp_min_(0.0),
                                          torch.zeros_like(logZ_sign))
    return out


def posterior(r1_blocks: torch.Tensor, gamma1: torch.Tensor, cache, *, prior_center_blocks=None,
              prior_scale_blocks=None, prior_tau: float = 0.0, map_idx: Optional[np.ndarray] = None,
              need_stats: bool = False):
    """mpq/priors/e8p12.py:815-968: x1 blocks, var1, alpha1, logZ per block and, with ``need_stats``,
    the per-block entropy and margin (:938-953).

    MAP (idx/vals) comes from ``map_search`` (same arithmetic as the reference's
    per-branch MAP, :411-412 and :933-936).  High-precision snap at gamma >= 1e3
    (:923-926) is applied.
    """
    r1_blocks = r1_blocks.to(dtype=torch.float32, device="cpu")
    B, nb, _ = r1_blocks.shape
    g_base = gamma1.to(torch.float32).view(B, 1, 1).expand(B, nb, 1)
    r_work, g_work = r1_blocks, g_base
    if prior_tau > 0.0 and prior_center_blocks is not None:
        c = prior_center_blocks.to(torch.float32)
        s = prior_scale_blocks
        if s is None:
            s = c.abs().amax(dim=-1, keepdim=True).clamp_min(1e-12)
        s = s.to(torch.float32).clamp_min(1e-12)
        tau2 = (max(float(prior_tau), 1e-12) * s).square()
        pp = 1.0 / tau2
        g_work = g_base + pp
        r_work = (g_base * r1_blocks + pp * c) / g_work
    r_flat = r_work.reshape(B * nb, 8)
    g_flat = g_work.reshape(B * nb, 1)
    outs = []
    for bi, off in enumerate((0.25, -0.25)):
        outs.append(_branch_stats(r_flat - off, g_flat, off, bi, cache, need_stats=need_stats))
    log_comp = torch.stack([o["log_component"] for o in outs], dim=1)
    logZ = torch.logsumexp(log_comp.reshape(B * nb, -1), dim=-1)
    log_w = log_comp - logZ.view(-1, 1, 1)
    w = torch.exp(log_w)
    stats = {}
    if need_stats:
        sent = torch.stack([o["sign_entropy"] for o in outs], dim=1)
        wl = torch.where(torch.isfinite(log_w), w * log_w, torch.zeros_like(log_w))
        stats["entropy"] = (-(wl.sum(dim=(1, 2))) + (w * sent).sum(dim=(1, 2))).view(B, nb)
        best = torch.stack([o["best_logscore"] for o in outs], dim=1).reshape(B * nb, -1)
        sec = torch.stack([o["second_logscore"] for o in outs], dim=1).reshape(B * nb, -1)
        top2 = torch.topk(torch.cat([best, sec], dim=1), k=2, dim=1).values
        stats["margin"] = (top2[:, 0] - top2[:, 1]).view(B, nb)
    mu = torch.zeros((B * nb, 8), dtype=torch.float32)
    second = torch.zeros((B * nb,), dtype=torch.float32)
    for bi in range(2):
        mu += (w[:, bi, :].unsqueeze(-1) * outs[bi]["mu_component"]).sum(dim=1)
        second += (w[:, bi, :] * outs[bi]["second_component"]).sum(dim=1)
    var = ((second - mu.square().sum(dim=-1)) / 8.0).clamp_min_(0.0)
    if map_idx is None:
        center = None if prior_center_blocks is None else prior_center_blocks.reshape(-1, 8).numpy()
        scale = None if prior_scale_blocks is None else prior_scale_blocks.reshape(-1).numpy()
        map_idx, _ = map_search(r1_blocks.reshape(-1, 8).numpy(), gamma1.reshape(-1).numpy(), nb, cache,
                                center=center, scale=scale, tau=prior_tau)
    hi = g_flat.squeeze(-1) >= 1e3
    if bool(hi.any()):
        from mpq_amd.codebook import grid_numpy

        mv = torch.from_numpy(grid_numpy()[np.asarray(map_idx)])
        mu[hi] = mv[hi]
        var[hi] = 0.0
    var1 = var.view(B, nb)
    alpha1 = gamma1.to(torch.float32) * var1.mean(dim=1, keepdim=True)
    return dict({"x1_blocks": mu.view(B, nb, 8), "var1": var1, "alpha1": alpha1,
                 "map_idxs": torch.as_tensor(np.asarray(map_idx)).view(B, nb), "logZ": logZ.view(B, nb)}, **stats)


def posterior_bruteforce(r: np.ndarray, g: np.ndarray, grid: np.ndarray):
    """fp64 posterior over all codewords: p(c) ∝ exp(-g/2 ||c - r||^2).  Returns mean, var (trace/8), logZ."""
    r = np.asarray(r, dtype=np.float64).reshape(-1, 8)
    g = np.asarray(g, dtype=np.float64).reshape(-1)
    G = np.asarray(grid, dtype=np.float64)
    gn = (G * G).sum(axis=1)
    means = np.empty_like(r)
    var = np.empty(r.shape[0])
    logz = np.empty(r.shape[0])
    for i in range(r.shape[0]):
        d = gn - 2.0 * G @ r[i] + r[i] @ r[i]
        s = -0.5 * g[i] * d
        m = s.max()
        w = np.exp(s - m)
        Z = w.sum()
        p = w / Z
        means[i] = p @ G
        var[i] = ((p * gn).sum() - means[i] @ means[i]) / 8.0
        logz[i] = m + math.log(Z)
    return means, var, logz


def posterior_stats_bruteforce(r: np.ndarray, g: np.ndarray, grid: np.ndarray):
    """fp64 diagnostics of p(c) ∝ exp(-g/2 ||c - r||^2) over all codewords: logZ, the entropy
    -sum p log p, and the margin between the two largest log-scores -g/2 ||c - r||^2.  These are
    the quantities the reference's factorized diagnostics sum to (mpq/priors/e8p12.py:276-305,
    885-953): the mixture entropy plus the weighted sign entropies is the entropy over codewords, and
    the top two of every component's best and second-best sign pattern are the top two codewords."""
    r = np.asarray(r, dtype=np.float64).reshape(-1, 8)
    g = np.asarray(g, dtype=np.float64).reshape(-1)
    G = np.asarray(grid, dtype=np.float64)
    gn = (G * G).sum(axis=1)
    logz = np.empty(r.shape[0])
    ent = np.empty(r.shape[0])
    margin = np.empty(r.shape[0])
    for i in range(r.shape[0]):
        s = -0.5 * g[i] * (gn - 2.0 * G @ r[i] + r[i] @ r[i])
        m = s.max()
        w = np.exp(s - m)
        Z = w.sum()
        p = w / Z
        logz[i] = m + math.log(Z)
        ent[i] = logz[i] - (p * s).sum()
        top = np.partition(s, -2)[-2:]
        margin[i] = top.max() - top.min()
    return logz, ent, margin


# ---------------------------------------------------------------------------
# E8P12 VAMP loop and gram-metric block CD (torch CPU, reference op order)
# ---------------------------------------------------------------------------

def stabilize_cholesky(gram: torch.Tensor, jitter: float = 1e-6, max_tries: int = 6) -> torch.Tensor:
    """mpq/linear.py:121-141."""
    floor = float(torch.diag(gram).abs().max().item()) * jitter + jitter
    eye = torch.eye(gram.shape[0], dtype=gram.dtype)
    out = gram
    for k in range(max_tries):
        try:
            return torch.linalg.cholesky(out)
        except RuntimeError:
            out = out + (2.0 ** k) * floor * eye
    return torch.linalg.cholesky(out)


def gram_block_cd(x, idxs, Y_u, Vs, grid, sweeps, accept_tol=0.0, max_blocks=0, metric="gram",
                  order_mode="greedy_gain", scores_fp64=False):
    """mpq/polish/block_cd.py:332-625 with E8P12Provider, greedy_gain order and, for metric "gram", the
    compiled step _cd_gram_step_impl (:212-246): whitened brute-force argmin over all codewords.
    metric "diag": target x + rhs * (1 / diag G) and the nearest codeword (cb.quantize, :740-745);
    order_mode static (trace G descending) or cyclic (:505-511); stable sorts.  ``scores_fp64``: the
    gram step's scores evaluated in fp64 from the same fp32 target and factor (another rounding of
    the reference's fp32 scores, used to measure how far that rounding moves the greedy decisions)."""
    B, n = x.shape
    nb = n // 8
    x = x.to(torch.float32).clone()
    idxs = idxs.clone()
    Vs_t = Vs.T.contiguous()
    res_u = Y_u - x.matmul(Vs)
    res = res_u.square().sum(dim=1)
    meta = []
    for b in range(nb):
        Vb = Vs[8 * b:8 * b + 8]
        G = Vb.matmul(Vb.T).contiguous()
        L = stabilize_cholesky(G)
        Gi = torch.cholesky_inverse(L).contiguous()
        meta.append((Vb.T.contiguous(), Vb.contiguous(), G, L, Gi))
    gi_stack = torch.stack([m[4] for m in meta], 0)
    dinv_stack = torch.stack([torch.diag(m[2]).clamp_min(1e-12).reciprocal() for m in meta], 0)
    static = torch.argsort(torch.stack([torch.diag(m[2]).sum() for m in meta]), descending=True, stable=True).tolist()
    accepted = 0
    for _ in range(sweeps):
        if order_mode == "greedy_gain":
            rhs_all = res_u.matmul(Vs_t).reshape(B, nb, 8).permute(1, 0, 2).contiguous()
            if metric == "gram":
                gain = (rhs_all * torch.bmm(rhs_all, gi_stack)).sum(dim=2).mean(dim=1)
            else:
                gain = (rhs_all.square() * dinv_stack.unsqueeze(1)).sum(dim=2).mean(dim=1)
            order = torch.argsort(gain, descending=True, stable=True).tolist()
        elif order_mode == "static":
            order = list(static)
        else:
            order = list(range(nb))
        if max_blocks > 0:
            order = order[:max_blocks]  # mpq/polish/block_cd.py:510-511
        for b in order:
            Vbt, Vb, G, L, Gi = meta[b]
            xb = x[:, 8 * b:8 * b + 8]
            rhs = res_u.matmul(Vbt)
            if metric == "gram":
                target = xb + rhs.matmul(Gi)
                if scores_fp64:
                    tm = target.double().matmul(L.double())
                    mg = grid.double().matmul(L.double())
                else:
                    tm = target.matmul(L)
                    mg = grid.matmul(L)
                scores = (tm.square().sum(dim=1, keepdim=True) + mg.square().sum(dim=-1).unsqueeze(0)
                          - 2.0 * tm.matmul(mg.T))
            else:
                target = xb + rhs * dinv_stack[b].unsqueeze(0)
                scores = (target.unsqueeze(1) - grid.unsqueeze(0)).square().sum(dim=-1)
            best = torch.argmin(scores, dim=1)
            cand = grid.index_select(0, best)
            delta = cand - xb
            cross = (rhs * delta).sum(dim=1)
            dn = (delta.matmul(G) * delta).sum(dim=1).clamp_min_(0.0)
            ce = (res + dn - 2.0 * cross).clamp_min_(0.0)
            acc = ce + 1e-12 < res * (1.0 + accept_tol)
            m = acc.unsqueeze(1)
            x[:, 8 * b:8 * b + 8] = torch.where(m, cand, xb)
            res_u.sub_((delta * m).matmul(Vb))
            res = torch.where(acc, ce, res)
            idxs[:, b] = torch.where(acc, best.to(idxs.dtype), idxs[:, b])
            accepted += int(acc.sum())
    return x, idxs, accepted


def solve_e8p12_rankspace_vamp(Wr, hat_init, V, S, grid, cache, cfg, obs_precision_init=None):
    """mpq/solver.py:853-1276, with best-iterate tracking when cfg["best_iterate"] (off in the recipe);
    returns (hat, idx, err, stats)."""
    from oracle import uniform as ou

    iters = int(cfg.get("iters", 16))
    damping = float(cfg.get("damping", 0.5))
    tau = float(cfg.get("prior_tau", 0.25))
    retry_factor = max(float(cfg.get("gamma_retry_factor", 4.0)), 1.000001)
    retry_steps = max(int(cfg.get("gamma_retry_steps", 3)), 0)
    sweeps = int(cfg.get("polish_sweeps", 3))
    B, n = Wr.shape
    nb = n // 8
    R = S.numel()
    Vs = V * S.unsqueeze(0)
    Vh = V.T.contiguous()
    Wb = Wr.reshape(B, nb, 8)
    # per-block prior scale (mpq/priors/e8p12.py:48-63): |W|max, rms, mean |W| or 1
    smode = str(cfg.get("prior_tau_scale_mode", "absmax") or "absmax").strip().lower()
    if tau <= 0:
        pscale = None
    elif smode in ("none", "unit", "legacy"):
        pscale = torch.ones(Wb.shape[:-1] + (1,), dtype=torch.float32)
    elif smode in ("rms", "std"):
        pscale = Wb.square().mean(dim=-1, keepdim=True).sqrt().clamp_min(1e-12)
    elif smode in ("mean_abs", "l1"):
        pscale = Wb.abs().mean(dim=-1, keepdim=True).clamp_min(1e-12)
    else:
        pscale = Wb.abs().amax(dim=-1, keepdim=True).clamp_min(1e-12)
    Y_u = Wr.matmul(Vs)
    # the requested precision first, then the caller's warm start (mpq/solver.py:893-899)
    requested = float(cfg.get("obs_precision", 0.0))
    if requested > 0.0:
        obs = requested
    elif obs_precision_init is not None and obs_precision_init > 0:
        obs = float(obs_precision_init)
    else:
        obs = 1.0 / float((Y_u - hat_init.matmul(Vs)).square().mean().clamp_min_(1e-12).item())
    r1 = hat_init.clone()
    gamma1 = float(cfg.get("gamma_start", 1.0)) * (0.25 / (Wr - hat_init).square().mean(dim=1, keepdim=True).clamp_min_(1e-12))
    r2_prev = g2_prev = None
    stats = {"gamma2_invalid": 0, "obs": [], "best_iter": -1, "stop_iter": -1}
    center = Wb.reshape(-1, 8).numpy() if tau > 0 else None
    scl = pscale.reshape(-1).numpy() if pscale is not None else None

    def map_error_mean(r, g):
        """mean rank-space error of the MAP decision of (r, g)"""
        idx_s, _ = map_search(r.reshape(-1, 8).numpy(), g.reshape(-1).numpy(), nb, cache, center=center, scale=scl,
                              tau=tau)
        hat_s = grid.index_select(0, torch.from_numpy(idx_s)).view(B, n)
        return float(ou.rankspace_error(Y_u, hat_s, Vs).mean().item())

    # best iterate (mpq/solver.py:940-958, 1083-1121): keep the state whose MAP decision has the
    # lowest error, stop at the first iterate that does not improve and restore the best state
    best_iterate = bool(cfg.get("best_iterate", False))
    if best_iterate:
        best_err_mean = map_error_mean(r1, gamma1)
        best_state = (r1.clone(), gamma1.clone(), None, None, obs)
    for it in range(iters):
        g1w = gamma1
        for attempt in range(retry_steps + 1):
            post = posterior(r1.reshape(B, nb, 8), g1w, cache, prior_center_blocks=Wb if tau > 0 else None,
                             prior_scale_blocks=pscale, prior_tau=tau)
            a1 = post["alpha1"]
            if bool(ou.alpha_valid(a1).all()):
                break
            if attempt >= retry_steps:
                if not bool(torch.isfinite(a1).all()):
                    raise RuntimeError("alpha1 invalid")
                a1 = torch.nan_to_num(a1, nan=0.5, posinf=1.0 - ou.ALPHA_EPS, neginf=ou.ALPHA_EPS).clamp(
                    min=ou.ALPHA_EPS, max=1.0 - ou.ALPHA_EPS)
                break
            g1w = torch.where(a1 <= ou.ALPHA_EPS, g1w / retry_factor, g1w)
            g1w = torch.where(a1 >= 1.0 - ou.ALPHA_EPS, g1w * retry_factor, g1w).clamp_min_(1e-12)
        x1 = post["x1_blocks"].reshape(B, n)
        eta1 = g1w / a1
        g2n = torch.nan_to_num(eta1 - g1w, nan=1e-12, posinf=1e12, neginf=1e-12).clamp_min_(1e-12)
        if not bool(ou.prec_valid(g2n).all()):
            stats["gamma2_invalid"] += 1
            continue
        r2n = (eta1 * x1 - g1w * r1) / g2n
        if r2_prev is None or damping >= 1.0:
            g2, r2 = g2n, r2n
        else:
            g2 = ou.log_damp(g2_prev, g2n, damping)
            r2 = (1.0 - damping) * r2_prev + damping * r2n
        if not bool(ou.prec_valid(g2).all()):
            stats["gamma2_invalid"] += 1
            continue
        x2, a2, res_u = ou.linear_mmse_exact(r2, g2, Y_u, V, Vh, S, obs)
        a2 = torch.nan_to_num(a2, nan=0.5, posinf=1.0 - ou.ALPHA_EPS, neginf=ou.ALPHA_EPS).clamp(
            min=ou.ALPHA_EPS, max=1.0 - ou.ALPHA_EPS)
        if bool(cfg.get("em_obs_precision", True)) and float(cfg.get("obs_precision", 0.0)) <= 0.0:
            obs = ou.em_update_obs_precision(res_u, g2, S, obs, R)
        eta2 = g2 / a2
        g1n = torch.nan_to_num(eta2 - g2, nan=1e-12, posinf=1e12, neginf=1e-12).clamp_min_(1e-12)
        r1n = (eta2 * x2 - g2 * r2) / g1n
        if damping >= 1.0:
            gamma1, r1 = g1n, r1n
        else:
            gamma1 = ou.log_damp(gamma1, g1n, damping)
            r1 = (1.0 - damping) * r1 + damping * r1n
        r2_prev, g2_prev = r2, g2
        stats["obs"].append(obs)
        if best_iterate:
            cur = map_error_mean(r1, gamma1)
            if cur + max(1e-10, abs(best_err_mean) * 1e-8) < best_err_mean:
                best_err_mean = cur
                best_state = (r1.clone(), gamma1.clone(), r2_prev.clone(), g2_prev.clone(), obs)
                stats["best_iter"] = it
            else:
                r1, gamma1, r2_prev, g2_prev, obs = best_state
                stats["stop_iter"] = it
                break
    idx, _ = map_search(r1.reshape(-1, 8).numpy(), gamma1.reshape(-1).numpy(), nb, cache, center=center,
                        scale=scl, tau=tau)
    idx_t = torch.from_numpy(idx).view(B, nb)
    hat = grid.index_select(0, idx_t.reshape(-1)).view(B, n)
    stats["idx_vamp"] = idx_t.clone()
    stats["err_vamp"] = ou.rankspace_error(Y_u, hat, Vs)
    if sweeps > 0:
        hat, idx_t, acc = gram_block_cd(hat, idx_t, Y_u, Vs, grid, sweeps,
                                        scores_fp64=bool(cfg.get("scores_fp64", False)))
        stats["polish_accepted"] = acc
    err = ou.rankspace_error(Y_u, hat, Vs)
    stats["obs_final"] = obs
    stats["r1"] = r1
    stats["gamma1"] = gamma1
    return hat, idx_t, err, stats


def _jitter_last_bit(V: torch.Tensor, seed: int) -> torch.Tensor:
    """Every entry moved to a random one of its two neighbouring floats or kept (seeded)."""
    g = torch.Generator().manual_seed(int(seed))
    step = torch.randint(-1, 2, V.shape, generator=g)
    up = torch.nextafter(V, torch.full_like(V, float("inf")))
    dn = torch.nextafter(V, torch.full_like(V, float("-inf")))
    return torch.where(step > 0, up, torch.where(step < 0, dn, V))


def refine_codebook(Wr, Hr, grid, cache, cfg, block_rows=128, info=None, v_jitter_seed=None, decomposition=None):
    """mpq/adapters/quip_sharp.py:396-878 for solver "vamp", init "rtn": nearest-codeword init,
    fp64 eigh (:33-67), rank-space warm start (:461-475), per row block VAMP + polish with the
    observation precision carried (:555-586).  Returns (hat, idx, obs_final); ``info`` (a dict,
    optional) receives the warm-start precision as "obs_initial".  ``v_jitter_seed`` moves every entry
    of the fp32 eigenvectors to a random neighbouring float (another valid fp32 rounding of the fp64
    decomposition, for noise floors); ``decomposition`` = (ascending eigenvalues, eigenvectors), fp64
    results of another eigensolver rounded to fp32, replaces LAPACK's.  Pinned by the reference's
    golden vector tests/golden/e8p12_refine.npz."""
    m, n = Wr.shape
    idx0, _ = bruteforce_nearest(Wr.reshape(-1, 8).numpy(), grid.numpy())
    idx0 = torch.from_numpy(np.asarray(idx0)).view(m, n // 8)
    hat0 = grid[idx0.reshape(-1)].view(m, n)
    H64 = 0.5 * (Hr.double() + Hr.double().T)
    if decomposition is None:
        lam, V = torch.linalg.eigh(H64)
        lam, V = lam.float(), V.float()
    else:
        lam, V = decomposition[0].float(), decomposition[1].float()
    if v_jitter_seed is not None:
        V = _jitter_last_bit(V, v_jitter_seed)
    floor = max(1e-6, 1e-6 * max(float(torch.diagonal(H64).mean().abs()), float(lam.max()), 1e-12))
    lam = lam.clamp_min(floor).flip(0).contiguous()
    V = V.flip(1).contiguous()
    S = torch.sqrt(lam)
    Vs = V * S.unsqueeze(0)
    obs = 1.0 / max(float((Wr - hat0).matmul(Vs).square().sum()) / (m * n), 1e-12)
    if info is not None:
        info["obs_initial"] = obs
    hat = hat0.clone()
    idx = idx0.clone()
    for r0 in range(0, m, block_rows):
        sl = slice(r0, min(m, r0 + block_rows))
        h, i, _, st = solve_e8p12_rankspace_vamp(Wr[sl], hat0[sl], V, S, grid, cache, cfg, obs_precision_init=obs)
        hat[sl] = h
        idx[sl] = i
        obs = float(st["obs_final"])
    return hat, idx, obs
