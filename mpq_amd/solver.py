"""Per-layer VAMP solvers on the HIP kernels (drop-in for the reference's ``mpq/solver.py``).

* ``UniformVampConfig``              reference :35-55
* ``solve_uniform_rankspace_vamp``   reference :426-830 -> ``mpq_uniform_vamp_solve`` +
                                     ``mpq_uniform_cd_polish``
* ``polish_uniform_rankspace``       reference :260-366 -> ``mpq_uniform_cd_polish``
* ``E8P12VampConfig``                reference :59-82
* ``solve_e8p12_rankspace_vamp``     reference :853-1276 -> ``mpq_e8p12_vamp_solve`` +
                                     ``mpq_e8p12_cd_polish``
* ``polish_e8p12_rankspace``         reference :369-423 -> ``mpq_e8p12_cd_polish``

All tensors live on the ROCm device.  The rank R must equal n (the adapters
always floor the eigenvalues, so this holds on the reference's own path).
"""
from __future__ import annotations

import weakref

from dataclasses import dataclass
from typing import Any, Dict, Optional, Tuple

import torch

from . import ops
from .codebook import require_standin_table
from .priors.e8p12 import prior_scale_from_center
from .priors.uniform import dequant_from_q, nearest_atom_idx


@dataclass(frozen=True)
class UniformVampConfig:
    iters: int = 10
    damping: float = 0.5
    final_decision: str = "map"  # "map" | "round_mean"
    init_from: str = "rtn"  # "rtn" | "float" | "zero"
    gamma_start: float = 1.0
    gamma_retry_factor: float = 4.0
    gamma_retry_steps: int = 3
    prior_tau: float = 0.2
    obs_precision: float = 0.0
    em_obs_precision: bool = True
    em_obs_precision_damping: float = 0.3
    em_obs_precision_min: float = 1e-4
    em_obs_precision_max: float = 1e8
    polish_sweeps: int = 3
    polish_mode: str = "block_cd"  # "none" | "block_cd" | "topk_block_cd"
    topk_k: int = 16
    vamp_backend: str = "auto"  # accepted for compatibility; every value runs the HIP kernels
    compile_block_cd: bool = True
    block_cd_backend: str = "eager"  # accepted for compatibility


@dataclass(frozen=True)
class E8P12VampConfig:
    """Scalar-precision VAMP config for QUIP E8P12 (reference :59-82)."""

    iters: int = 16
    damping: float = 0.5
    gamma_start: float = 1.0
    gamma_retry_factor: float = 4.0
    gamma_retry_steps: int = 3
    prior_tau: float = 0.25
    prior_tau_scale_mode: str = "absmax"
    compile_prior: bool = True  # accepted for compatibility
    obs_precision: float = 0.0
    em_obs_precision: bool = True
    em_obs_precision_damping: float = 0.3
    em_obs_precision_min: float = 1e-4
    em_obs_precision_max: float = 1e8
    blocks_per_chunk: int = 16  # accepted for compatibility (the kernels stream all blocks)
    polish_sweeps: int = 3
    polish_mode: str = "block_cd"  # "none" | "block_cd" | "topk_block_cd"
    polish_metric: str = "gram"  # "gram" | "diag"
    polish_metric_rows_per_chunk: int = 0
    polish_max_blocks: int = 0
    topk_k: int = 16
    best_iterate: bool = False


def _resolve_e8p12_polish_metric(metric: str) -> str:
    """reference :179-185."""
    m = str(metric or "gram").strip().lower()
    if m in ("isotropic", "diag"):
        return "diag"
    if m == "gram":
        return "gram"
    raise ValueError(f"unsupported polish_metric={metric!r}; expected 'gram'|'diag'.")


def _resolve_polish_mode(*, sweeps: int, mode: str) -> str:
    """reference :164-175."""
    if int(sweeps) <= 0:
        return "none"
    m = str(mode or "block_cd").strip().lower()
    if m in {"none", "off"}:
        return "none"
    if m in {"block_cd", "cd", "full_cd"}:
        return "block_cd"
    if m in {"topk_block_cd", "topk_cd", "topk", "vamp_topk"}:
        return "topk_block_cd"
    raise ValueError(f"unsupported polish_mode={mode!r}; expected none|block_cd|topk_block_cd.")


def _resolve_backend(name: Optional[str], *, field: str) -> str:
    b = str(name or "").strip().lower()
    if b and b not in {"eager", "compile", "triton", "auto"}:
        raise ValueError(f"unsupported {field}={name!r}; expected eager|compile|triton|auto.")
    return "hip"


def _is_expanded(t: torch.Tensor, rows: int, n: int) -> bool:
    return t.dim() == 2 and tuple(t.shape) == (rows, n)


@torch.inference_mode()
def polish_uniform_rankspace(
    *,
    x_init: torch.Tensor,
    Y_u: torch.Tensor,
    Vs: torch.Tensor,
    scale_full: torch.Tensor,
    zero_full: torch.Tensor,
    maxq: int,
    sweeps: int,
    polish_mode: str,
    topk_values: Optional[torch.Tensor] = None,
    topk_q: Optional[torch.Tensor] = None,
    compile_block_cd: bool = True,
    block_cd_backend: Optional[str] = None,
    gram_full: Optional[torch.Tensor] = None,
    order_mode: str = "greedy_gain",
    raw_target: Optional[torch.Tensor] = None,
    raw_gram: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, Dict[str, float]]:
    """Greedy scalar CD polish (reference :260-366); returns (q int32, x, err, stats).

    The recipe case (block_cd, greedy order) runs the fused sweeps (``mpq_uniform_cd_polish``);
    ``topk_block_cd`` (with ``topk_values``) and the static / cyclic orders run the generic block CD
    (``mpq_amd.polish.block_cd``) with the reference's providers, as its CPU dispatch does (:334-366).
    """
    del compile_block_cd
    mode = _resolve_polish_mode(sweeps=int(sweeps), mode=str(polish_mode))
    _resolve_backend(block_cd_backend, field="block_cd_backend")
    rows, n = x_init.shape
    x_work = x_init.to(torch.float32).contiguous()
    q0 = nearest_atom_idx(x=x_work, scale_full=scale_full, zero_full=zero_full, maxq=maxq)
    if mode == "none" or Vs.numel() == 0:
        x_out = dequant_from_q(q_int=q0, scale_full=scale_full, zero_full=zero_full)
        err = (Y_u - ops.gemm(x_out, Vs)).square().sum(dim=1)
        return q0, x_out, err, {"accepted_updates": 0.0}
    order = str(order_mode or "greedy_gain").strip().lower()
    if mode == "topk_block_cd" or order != "greedy_gain":
        from .polish.block_cd import (BlockCDConfig, UniformScalarProvider, UniformTopKProvider,
                                      block_coordinate_descent_rankspace)

        if mode == "topk_block_cd":
            if topk_values is None:
                raise ValueError("topk_block_cd requires topk_values for uniform polish.")
            provider = UniformTopKProvider(topk_values=topk_values, topk_q=topk_q)
        else:
            provider = UniformScalarProvider(scale=scale_full, zero=zero_full, maxq=maxq)
        x_pol, q_pol, st = block_coordinate_descent_rankspace(
            x=x_work, Y_u=Y_u, Vs=Vs, block_size=1, provider=provider,
            cfg=BlockCDConfig(sweeps=int(sweeps), metric="diag", accept_tol=0.0, order_mode=order),
            idxs_init=q0, raw_target=raw_target, raw_gram=raw_gram)
        if q_pol is not None and bool((q_pol >= 0).all().item()):
            q_out = q_pol.to(torch.int32)
        else:
            q_out = nearest_atom_idx(x=x_pol, scale_full=scale_full, zero_full=zero_full, maxq=maxq)
        x_out = dequant_from_q(q_int=q_out, scale_full=scale_full, zero_full=zero_full)
        err = (Y_u - ops.gemm(x_out, Vs)).square().sum(dim=1)
        st = dict(st)
        st["block_cd_backend"] = "hip"
        return q_out, x_out, err, st
    del topk_values, topk_q, raw_target, raw_gram
    gram = gram_full if gram_full is not None else ops.gemm(Vs, Vs, trans_b=True)
    q, eb, ea, _imp, acc = ops.uniform_cd_polish(
        None, q0.to(torch.uint8), scale_full, zero_full, 1, maxq, Vs, gram, block_rows=rows,
        sweeps=int(sweeps), select=False, Yu=Y_u, x_in=x_work)
    q_i32 = q.to(torch.int32)
    x_out = dequant_from_q(q_int=q, scale_full=scale_full, zero_full=zero_full)
    return q_i32, x_out, ea, {"accepted_updates": float(acc.sum().item()), "block_cd_backend": "hip"}


@torch.inference_mode()
def solve_uniform_rankspace_vamp(
    *,
    W: torch.Tensor,
    x_rtn: torch.Tensor,
    scale_full: torch.Tensor,
    zero_full: torch.Tensor,
    maxq: int,
    V: torch.Tensor,
    Vh: torch.Tensor,
    S: torch.Tensor,
    Vs: torch.Tensor,
    cfg: UniformVampConfig,
    gram_full: Optional[torch.Tensor] = None,
    obs_precision_init: Optional[float] = None,
    log_stats: bool = True,
    debug_out: Optional[Dict[str, Any]] = None,
    group_size: Optional[int] = None,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, Dict[str, Any]]:
    """Scalar uniform exact-full VAMP in rank space with the greedy CD polish.

    ``scale_full``/``zero_full`` are per-entry (B x n) as in the reference, or
    group form (B x G) when ``group_size`` is given.  ``log_stats`` diagnostics
    (entropy/margin) are reported as 0.0.  Returns (q int32, x, err, rtn_err, stats).
    """
    del Vh, log_stats
    rows, n = W.shape
    gs = 1 if group_size is None else int(group_size)
    if group_size is None and not _is_expanded(scale_full, rows, n):
        raise ValueError("scale_full/zero_full must be (B, n) unless group_size is given")
    _resolve_backend(getattr(cfg, "vamp_backend", "auto"), field="vamp_backend")
    polish_sweeps = max(int(cfg.polish_sweeps), 0)
    polish_mode = _resolve_polish_mode(sweeps=polish_sweeps, mode=str(getattr(cfg, "polish_mode", "block_cd")))
    if polish_mode == "topk_block_cd":
        raise ValueError("mpq_amd implements polish_mode='block_cd' (the recipe default); topk_block_cd is not provided.")
    q, _, err, rtn_err, st = ops.uniform_vamp_solve(W, x_rtn, scale_full, zero_full, gs, maxq, V, S, Vs, cfg,
                                                    obs_init=float(obs_precision_init or 0.0))
    q_stage1 = q
    polish_stats: Dict[str, Any] = {}
    polish_gain = 0.0
    if polish_mode != "none":
        gram = gram_full if gram_full is not None else ops.gemm(Vs, Vs, trans_b=True)
        q, eb, ea, imp, acc = ops.uniform_cd_polish(W, q, scale_full, zero_full, gs, maxq, Vs, gram,
                                                    block_rows=rows, sweeps=polish_sweeps, select=True)
        err = torch.where(imp.bool(), ea, err)
        polish_gain = float((eb - ea).mean().item()) if bool(imp.any().item()) else 0.0
        polish_stats = {"accepted_updates": float(acc.sum().item()), "block_cd_backend": "hip"}
    x_final = ops.dequant(q, scale_full, zero_full, gs)
    if debug_out is not None:
        debug_out["solver"] = "uniform_exact_vamp"
        if bool(debug_out.get("summary_only", False)):
            debug_out["changed_count"] = int((q_stage1 != q).sum().item())
            debug_out["changed_total"] = int(q.numel())
        else:
            debug_out["q_pre_polish"] = q_stage1.to(torch.int32).cpu()
            debug_out["q_post_polish"] = q.to(torch.int32).cpu()
    stats: Dict[str, Any] = {
        "solver": "uniform_exact_vamp",
        "iters": int(st["iters"]),
        "rank": int(S.numel()),
        "init_from": str(cfg.init_from),
        "damping": float(cfg.damping),
        "prior_tau": float(cfg.prior_tau),
        "vamp_backend": str(getattr(cfg, "vamp_backend", "auto")),
        "vamp_backend_used": "hip",
        "gamma_start": float(cfg.gamma_start),
        "obs_precision_initial": float(st["obs_precision_initial"]),
        "obs_precision_final": float(st["obs_precision_final"]),
        "obs_precision_mean": float(st["obs_precision_mean"]),
        "alpha1_retry_count": int(st["alpha1_retry_count"]),
        "alpha2_clip_count": int(st["alpha2_clip_count"]),
        "gamma2_invalid_count": int(st["gamma2_invalid_count"]),
        "alpha1_mean": float(st["alpha1_mean"]),
        "alpha2_mean": float(st["alpha2_mean"]),
        "mean_entropy": 0.0,
        "mean_margin": 0.0,
        "final_decision": str(cfg.final_decision),
        "best_iterate_enabled": True,
        "best_iter": int(st["best_iter"]),
        "stop_iter": int(st["stop_iter"]),
        "best_rankspace_error_mean": float(st["best_rankspace_error_mean"]),
        "polish_sweeps": int(polish_sweeps),
        "polish_mode": polish_mode,
        "polish_gain": float(polish_gain),
        "polish_updates": float(polish_stats.get("accepted_updates", 0.0)),
        "polish_trace": polish_stats,
        "block_cd_backend": "hip",
        "rankspace_error_mean": float(err.mean().item()),
        "rtn_rankspace_error_mean": float(rtn_err.mean().item()),
    }
    return q.to(torch.int32), x_final, err, rtn_err, stats


# ---- E8P12 -----------------------------------------------------------------------

_CD_CTX: Dict[str, Any] = {}


def _tensor_version(t: torch.Tensor) -> Optional[int]:
    """torch's in-place modification counter of ``t`` (None for inference tensors, which keep none)."""
    try:
        return int(t._version)
    except RuntimeError:
        return None


def _e8p12_cd_context(Vs: torch.Tensor) -> torch.Tensor:
    """Per-layer polish context for the last Vs seen (the reference-signature solvers call the
    polish once per row block with the same Vs).  A hit requires the very same tensor object and an
    unchanged in-place modification counter; anything else rebuilds the context.  Inference tensors
    keep no such counter, so for them an in-place change between calls is not seen: callers that
    modify Vs in place pass ``cd_context`` explicitly.  Only a weak reference to Vs is kept, and the
    context is dropped when Vs is freed."""
    ref = _CD_CTX.get("ref")
    if ref is not None and ref() is Vs and _CD_CTX.get("version") == _tensor_version(Vs):
        return _CD_CTX["ctx"]
    _CD_CTX.clear()
    ctx = ops.e8p12_cd_prepare(Vs)
    _CD_CTX["ref"] = weakref.ref(Vs, _drop_cd_context)
    _CD_CTX["version"] = _tensor_version(Vs)
    _CD_CTX["ctx"] = ctx
    return ctx


def _drop_cd_context(dead_ref) -> None:
    if _CD_CTX.get("ref") is dead_ref:
        _CD_CTX.clear()


def clear_e8p12_cd_context() -> None:
    """Drop the cached polish context (called when a layer's solve finishes)."""
    _CD_CTX.clear()


@torch.inference_mode()
def polish_e8p12_rankspace(
    *,
    x_init: torch.Tensor,
    idxs_init: torch.Tensor,
    Y_u: torch.Tensor,
    Vs: torch.Tensor,
    cb: object,
    sweeps: int,
    polish_mode: str,
    polish_metric: str,
    metric_rows_per_chunk: int = 0,
    polish_max_blocks: int = 0,
    topk_idxs: Optional[torch.Tensor] = None,
    order_mode: str = "greedy_gain",
    snapshot_budgets: Optional[set] = None,
    snapshots_out: Optional[Dict[int, torch.Tensor]] = None,
    block_rows: Optional[int] = None,
    cd_context: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, Dict[str, Any]]:
    """Gram-metric block CD over E8P12 codewords (reference :369-423).

    The rows of ``x_init`` form one greedy-order group unless ``block_rows`` splits them
    (every group of ``block_rows`` rows then has its own order, as separate calls would).
    ``cd_context`` (``ops.e8p12_cd_prepare(Vs)``, optional) is the per-layer context; without
    it the context of the last Vs is reused when Vs is element-wise identical.
    Returns (x, idxs, err, stats).
    """
    require_standin_table(cb, "polish_e8p12_rankspace")
    mode = _resolve_polish_mode(sweeps=int(sweeps), mode=str(polish_mode))
    metric = _resolve_e8p12_polish_metric(str(polish_metric))
    x_work = x_init.to(dtype=torch.float32)
    if mode == "none" or Vs.numel() == 0:
        err = (Y_u - ops.gemm(x_work, Vs)).square().sum(dim=1)
        return x_work, idxs_init, err, {"accepted_updates": 0.0}
    order = str(order_mode or "greedy_gain").strip().lower()
    if mode == "topk_block_cd" or metric != "gram" or order != "greedy_gain" or snapshot_budgets:
        # the reference's generic dispatch (:402-423) with its providers, one greedy group for all rows
        from .polish.block_cd import BlockCDConfig, E8P12Provider, E8P12TopKProvider, block_coordinate_descent_rankspace

        if mode == "topk_block_cd":
            if topk_idxs is None:
                raise ValueError("topk_block_cd requires topk_idxs for E8P12 polish.")
            provider = E8P12TopKProvider(cb=cb, topk_idxs=topk_idxs)
        else:
            provider = E8P12Provider(cb=cb, metric_rows_per_chunk=int(metric_rows_per_chunk))
        x_out, idx_out, st = block_coordinate_descent_rankspace(
            x=x_work.contiguous(), Y_u=Y_u, Vs=Vs, block_size=int(getattr(cb, "codesz", 8)), provider=provider,
            cfg=BlockCDConfig(sweeps=int(sweeps), metric="gram" if metric == "gram" else "diag", accept_tol=0.0,
                              metric_rows_per_chunk=int(metric_rows_per_chunk),
                              max_blocks_per_sweep=int(polish_max_blocks), order_mode=order),
            idxs_init=idxs_init, snapshot_budgets=snapshot_budgets, snapshots_out=snapshots_out)
        if idx_out is None:
            raise RuntimeError("E8P12 polish must return block indices.")
        err = (Y_u - ops.gemm(x_out.contiguous(), Vs)).square().sum(dim=1)
        return x_out, idx_out, err, st
    del cb, metric_rows_per_chunk, topk_idxs, snapshots_out
    rows = int(x_work.shape[0])
    ctx = cd_context if cd_context is not None else _e8p12_cd_context(Vs.to(dtype=torch.float32).contiguous())
    x, idx, eb, ea, acc = ops.e8p12_cd_polish(x_work, idxs_init, Vs, ctx, sweeps=int(sweeps),
                                              block_rows=int(block_rows or rows), Yu=Y_u,
                                              max_blocks=int(polish_max_blocks))
    stats = {"accepted_updates": float(acc.sum().item()), "block_cd_backend": "hip",
             "stabilized_objective_nonincreasing": bool((ea <= eb * (1 + 1e-6) + 1e-8).all().item())}
    return x, idx, ea, stats


@torch.inference_mode()
def solve_e8p12_rankspace_vamp(
    *,
    Wr: torch.Tensor,
    hatWr_init: torch.Tensor,
    cb: object,
    V: torch.Tensor,
    Vh: torch.Tensor,
    S: torch.Tensor,
    Vs: torch.Tensor,
    cfg: E8P12VampConfig,
    module_name: str = "",
    obs_precision_init: Optional[float] = None,
    log_stats: bool = True,
    debug_out: Optional[Dict[str, Any]] = None,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, Dict[str, Any]]:
    """Scalar-precision VAMP for QUIP E8P12 in rank space, with the gram-metric polish
    (reference :853-1276).  Returns (hatWr, Qidxs int64, err, stats); ``log_stats``
    diagnostics (entropy/margin) are reported as 0.0."""
    del Vh, log_stats
    require_standin_table(cb, "solve_e8p12_rankspace_vamp")
    Wr = Wr.to(dtype=torch.float32)
    rows, n = Wr.shape
    codesz = int(getattr(cb, "codesz", 8)) if cb is not None else 8
    if codesz != 8 or n % codesz:
        raise ValueError(f"E8P12 solver expects n divisible by 8; got n={n}, codesz={codesz}.")
    nblocks = n // 8
    polish_sweeps = max(int(cfg.polish_sweeps), 0)
    polish_mode = _resolve_polish_mode(sweeps=polish_sweeps, mode=str(getattr(cfg, "polish_mode", "block_cd")))
    polish_metric = _resolve_e8p12_polish_metric(str(cfg.polish_metric or "gram"))
    prior_tau = float(cfg.prior_tau)
    mode = str(cfg.prior_tau_scale_mode or "absmax").strip().lower()
    prior_scale = None
    if prior_tau > 0.0 and mode not in ("absmax", "exact_full", "exact_full_absmax"):
        prior_scale = prior_scale_from_center(Wr.reshape(rows, nblocks, 8), mode).reshape(-1)
    capture_r1 = debug_out is not None and bool(debug_out.get("capture_r1", False))
    idx, hat, err, r1, g1, st = ops.e8p12_vamp_solve(Wr, hatWr_init, V, S, Vs, cfg, prior_scale=prior_scale,
                                                     obs_init=float(obs_precision_init or 0.0), want_state=True)
    idx_stage1 = idx
    polish_stats: Dict[str, Any] = {}
    polish_gain = 0.0
    polish_updates = 0.0
    if polish_mode != "none":
        Y_u = ops.gemm(Wr, Vs)
        err_before = err
        hat, idx, err, polish_stats = polish_e8p12_rankspace(
            x_init=hat, idxs_init=idx, Y_u=Y_u, Vs=Vs, cb=cb, sweeps=polish_sweeps, polish_mode=polish_mode,
            polish_metric=polish_metric, polish_max_blocks=int(cfg.polish_max_blocks))
        polish_gain = float((err_before - err).mean().item())
        polish_updates = float(polish_stats.get("accepted_updates", 0.0))
    if debug_out is not None:
        summary_only = bool(debug_out.get("summary_only", False))
        debug_out["solver"] = "e8p12_exact_vamp"
        g64 = g1.to(torch.float64)
        debug_out["gamma1_sum"] = float(g64.sum().item())
        debug_out["gamma1_count"] = int(g64.numel())
        debug_out["gamma1_min"] = float(g64.min().item())
        debug_out["gamma1_max"] = float(g64.max().item())
        if capture_r1:
            debug_out["r1"] = r1.detach().to(device="cpu")
        if summary_only:
            debug_out["changed_count"] = int((idx_stage1 != idx).sum().item())
            debug_out["changed_total"] = int(idx.numel())
        else:
            debug_out["idxs_pre_polish"] = idx_stage1.detach().to(device="cpu")
            debug_out["gamma1"] = g1.detach().to(device="cpu")
            debug_out["idxs_post_polish"] = idx.detach().to(device="cpu")
            debug_out["changed_mask"] = debug_out["idxs_pre_polish"] != debug_out["idxs_post_polish"]
        if bool(debug_out.get("capture_weights", False)):
            debug_out["W"] = Wr.detach().to(device="cpu")
    stats: Dict[str, Any] = {
        "solver": "e8p12_exact_vamp",
        "module": str(module_name),
        "iters": int(st["iters"]),
        "rank": int(S.numel()),
        "nblocks": int(nblocks),
        "damping": float(cfg.damping),
        "prior_tau": prior_tau,
        "prior_tau_scale_mode": mode,
        "compile_prior": bool(getattr(cfg, "compile_prior", True)),
        "gamma_start": float(cfg.gamma_start),
        "gamma_retry_factor": float(max(float(cfg.gamma_retry_factor), 1.000001)),
        "gamma_retry_steps": int(max(int(cfg.gamma_retry_steps), 0)),
        "obs_precision_initial": float(st["obs_precision_initial"]),
        "obs_precision_final": float(st["obs_precision_final"]),
        "obs_precision_mean": float(st["obs_precision_mean"]),
        "alpha1_retry_count": int(st["alpha1_retry_count"]),
        "alpha2_clip_count": int(st["alpha2_clip_count"]),
        "gamma2_invalid_count": int(st["gamma2_invalid_count"]),
        "alpha1_mean": float(st["alpha1_mean"]),
        "alpha2_mean": float(st["alpha2_mean"]),
        "mean_entropy": 0.0,
        "mean_margin": 0.0,
        "blocks_per_chunk": int(cfg.blocks_per_chunk),
        "polish_sweeps": int(polish_sweeps),
        "polish_mode": polish_mode,
        "polish_metric": polish_metric,
        "topk_k": int(cfg.topk_k),
        "polish_gain": float(polish_gain),
        "polish_updates": float(polish_updates),
        "polish_trace": polish_stats,
        "best_iterate_enabled": bool(cfg.best_iterate),
        "best_iter": int(st["best_iter"]),
        "stop_iter": int(st["stop_iter"]),
        "best_rankspace_error_mean": float(st["rankspace_error_mean"]) if bool(cfg.best_iterate) else 0.0,
        "rankspace_error_mean": float(err.mean().item()),
    }
    return hat, idx, err, stats
