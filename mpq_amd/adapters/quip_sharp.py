"""QUIP# adapter: refine E8P12 codebook decisions with VAMP + gram-metric polish on the HIP kernels.

Drop-in for the reference's ``mpq/adapters/quip_sharp.py`` entry point
``mpq_refine_codebook`` (:396-878) as called by the patched ``quip.quantize``
(``patches/quip_sharp.patch:405-421``):

* init ``rtn`` (nearest codeword, ``cb.quantize``), ``random``, ``float``, ``zero`` or
  ``ldlq`` (:426-447, helpers :191-261);
* fp64 eigendecomposition of Hr, floored and descending (:33-67);
* observation-precision warm start from the init mismatch in rank space (:461-475);
* the sequential row-block VAMP chain with the precision carried between blocks
  (:555-586), then the gram-metric block-CD polish of every row block with its own
  greedy order (one launch sequence for all blocks; each block's polish depends only
  on its own VAMP result);
* the exact surrogate audits ``(Wr - hat) Hr (Wr - hat)^T`` per row block against the
  LDLQ result (:70-117, :805-818).

Supported solver combinations: ``vamp`` (polish ``block_cd`` or ``none``, metric ``gram`` or
``diag``) and ``ldlq`` (polish ``block_cd`` or ``none``).  The reference's baseline solvers (cdquant,
quantease, ojbkq) and the top-k polish (whose candidates come from the solver's top-k posterior) are
outside this build and raise ``ValueError``.
"""
from __future__ import annotations

import math
import re
import time
from dataclasses import dataclass
from typing import Any, Dict, Optional, Tuple

import torch

from .. import ops
from ..codebook import require_standin_table
from ..solver import E8P12VampConfig, _resolve_e8p12_polish_metric, _resolve_polish_mode
from ..priors.e8p12 import prior_scale_from_center
from ..utils import stable_seed


@dataclass(frozen=True)
class QuipAdapterConfig:
    block_rows: int = 128
    jitter_base: float = 1e-6
    eigen_floor_scale: float = 1e-6
    # rank-space products as fp32-accurate bf16-plane products on the matrix cores (ops.gemm_x6)
    # when n % 128 == 0 and n >= ops.X6_MIN_N; False keeps every product on the fp32 MFMA kernel
    x6_products: bool = True


def _resolve_block_rows(rows: int, requested: int) -> int:
    return min(int(rows), max(int(requested), 1))


@torch.inference_mode()
def _vamp_hessian_eigen(H: torch.Tensor, *, jitter_base: float = 1e-6, floor_scale: float = 1e-6):
    """fp64 eigendecomposition, floored, descending (reference :33-67).
    Returns (lam, S, V, Vs, rank, floor)."""
    n = int(H.shape[0])
    H64 = H.to(dtype=torch.float64)
    H64 = 0.5 * (H64 + H64.T)
    if not bool(torch.isfinite(H64).all()):
        H64 = torch.nan_to_num(H64, nan=0.0, posinf=0.0, neginf=0.0)
    lam64, V64 = ops.syevd(H64)
    lam32 = lam64.to(torch.float32)
    V32 = V64.to(torch.float32).contiguous()
    del V64
    max_lam = float(lam32.max().item()) if lam32.numel() else 0.0
    diag_mean = float(torch.diagonal(H64).mean().abs().item()) if H64.numel() else 0.0
    floor = max(float(jitter_base), float(floor_scale) * max(diag_mean, max_lam, 1e-12))
    lam, S, V, Vs = ops.eigh_postprocess(lam32, V32, floor)
    return lam, S, V, Vs, n, float(floor)


def _surrogate_rows(Wr: torch.Tensor, hat: torch.Tensor, Hr: torch.Tensor) -> torch.Tensor:
    delta = (Wr - hat).to(torch.float32).contiguous()
    return (ops.gemm(delta, Hr) * delta).sum(dim=1)


def _chunk_means(rows_vals: torch.Tensor, block_rows: int) -> Tuple[float, list]:
    vals = rows_vals.double().cpu()
    m = int(vals.numel())
    means = [float(vals[r0:r0 + block_rows].mean()) for r0 in range(0, m, block_rows)]
    return float(vals.sum() / max(m, 1)), means


def _quantize_blocks(cb: Any, X: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    vals, idx = cb.quantize(X, return_idx=True)
    return vals, idx


@torch.inference_mode()
def _rtn_e8p12_init(*, Wr: torch.Tensor, cb: Any, resid_scale_override: Optional[float] = None):
    """Nearest codeword of every 8-block (reference :212-241)."""
    del resid_scale_override
    m, n = Wr.shape
    if n % 8:
        raise ValueError(f"mpq RTN init expects E8P12 codesz=8; got codesz=8, n={n}.")
    vals, idx = _quantize_blocks(cb, Wr.reshape(-1, 8).contiguous())
    return vals.reshape(m, n).to(Wr.dtype), idx.view(m, n // 8).to(torch.int64)


@torch.inference_mode()
def _zero_e8p12_init(*, Wr: torch.Tensor, cb: Any, resid_scale_override: Optional[float] = None):
    """Zero values with the indices of the nearest codeword to 0 (reference :244-261)."""
    del resid_scale_override
    m, n = Wr.shape
    if n % 8:
        raise ValueError(f"mpq zero init expects E8P12 codesz=8; got codesz=8, n={n}.")
    _, idx = _quantize_blocks(cb, Wr.new_zeros((m * (n // 8), 8)))
    return Wr.new_zeros((m, n)), idx.view(m, n // 8).to(torch.int64)


@torch.inference_mode()
def _random_e8p12_init(*, cb: Any, rows: int, nblocks: int, seed_key: str, base_seed: int,
                       device: torch.device, dtype: torch.dtype):
    """Uniform random codewords from a CPU generator seeded by stable_seed (reference :191-209)."""
    grid = cb.grid.to(device=device, dtype=torch.float32)
    gen = torch.Generator(device="cpu")
    gen.manual_seed(stable_seed(seed_key, base_seed=int(base_seed)))
    idxs = torch.randint(0, int(grid.shape[0]), (int(rows), int(nblocks)), generator=gen, dtype=torch.int64)
    idxs = idxs.to(device=device)
    vals = grid.index_select(0, idxs.reshape(-1)).view(int(rows), int(nblocks) * 8)
    return vals.to(dtype=dtype), idxs


def _resolve_combo(args: Any) -> Tuple[str, str]:
    """(solver, polish_mode) from the reference's argument conventions (:1003-1031)."""
    quant_solver = getattr(args, "quant_solver", None)
    if quant_solver is None:
        quant_solver = getattr(args, "mpq_solver", None)
    if quant_solver is not None:
        solver = str(quant_solver).strip().lower()
        polish = str(getattr(args, "quant_polish_mode", getattr(args, "mpq_polish_mode", "none")) or "none")
    else:
        legacy = str(getattr(args, "mpq_method", "vamp") or "vamp").strip().lower()
        solver = "vamp"
        polish = "topk_block_cd" if legacy == "vamp-topk-polish" else "block_cd"
        if int(getattr(args, "mpq_polish_sweeps", 3) or 0) <= 0:
            polish = "none"
    polish = str(polish).strip().lower()
    if solver not in ("vamp", "ldlq"):
        raise ValueError(f"mpq_amd QUIP adapter provides solvers 'vamp' and 'ldlq'; got {solver!r} "
                         "(baseline solvers are not part of this build).")
    if polish in ("topk_block_cd", "topk_cd", "topk", "vamp_topk"):
        raise ValueError("mpq_amd implements polish_mode='block_cd' (the recipe default); topk_block_cd is not provided.")
    return solver, polish


def _build_vamp_cfg(args: Any, *, polish_mode: str) -> E8P12VampConfig:
    """reference :1034-1058."""
    return E8P12VampConfig(
        iters=int(getattr(args, "mpq_iters", 16)),
        damping=float(getattr(args, "mpq_damping", 0.5)),
        gamma_start=float(getattr(args, "mpq_gamma_start", 1.0)),
        gamma_retry_factor=float(getattr(args, "mpq_gamma_retry_factor", 4.0)),
        gamma_retry_steps=int(getattr(args, "mpq_gamma_retry_steps", 3)),
        prior_tau=float(getattr(args, "mpq_prior_tau", 0.25)),
        prior_tau_scale_mode=str(getattr(args, "mpq_prior_tau_scale_mode", "absmax")),
        compile_prior=bool(getattr(args, "mpq_compile_prior", True)),
        obs_precision=float(getattr(args, "mpq_obs_precision", 0.0)),
        em_obs_precision=bool(getattr(args, "mpq_em_obs_precision", True)),
        em_obs_precision_damping=float(getattr(args, "mpq_em_obs_precision_damping", 0.3)),
        em_obs_precision_min=float(getattr(args, "mpq_em_obs_precision_min", 1e-4)),
        em_obs_precision_max=float(getattr(args, "mpq_em_obs_precision_max", 1e8)),
        blocks_per_chunk=int(getattr(args, "mpq_blocks_per_chunk", 16)),
        polish_sweeps=int(getattr(args, "mpq_polish_sweeps", 3)),
        polish_mode=str(polish_mode),
        polish_metric=str(getattr(args, "mpq_polish_metric", "gram")),
        polish_metric_rows_per_chunk=int(getattr(args, "mpq_metric_rows_per_chunk", 0)),
        polish_max_blocks=int(getattr(args, "mpq_polish_max_blocks", 0)),
        topk_k=int(getattr(args, "mpq_topk_k", getattr(args, "quant_topk_k", 16)) or 16),
        best_iterate=bool(getattr(args, "mpq_best_iterate", False)),
    )


def _layer_index(module_name: str) -> Optional[int]:
    m = re.search(r"(?:^|\.)layers\.(\d+)(?:\.|$)", str(module_name))
    return int(m.group(1)) if m else None


@torch.inference_mode()
def mpq_refine_codebook(
    Wr: torch.Tensor,
    Hr: torch.Tensor,
    hatWr0: torch.Tensor,
    Qidxs0: torch.Tensor,
    cb: Any,
    args: Any,
    *,
    module_name: str = "",
    adapter_cfg: QuipAdapterConfig = QuipAdapterConfig(),
) -> Tuple[torch.Tensor, torch.Tensor, Dict[str, Any]]:
    """QUIP# adapter: refine codebook decisions via MPQ (VAMP + greedy polish).  Returns
    (hatWr, Qidxs int64 (m, n/8), stats)."""
    start = time.time()
    if not Wr.is_cuda:
        raise ValueError(f"Wr must be on a ROCm device (got {Wr.device}); mpq_amd has no CPU path.")
    Wr = Wr.to(dtype=torch.float32).contiguous()
    Hr = Hr.to(device=Wr.device, dtype=torch.float32).contiguous()
    device = Wr.device
    m, n = Wr.shape
    codesz = int(getattr(cb, "codesz", 8))
    if codesz != 8 or n % codesz:
        raise ValueError(f"mpq QUIP adapter expects E8P12 codesz=8; got codesz={codesz}, n={n}.")
    nblocks = n // 8
    if hasattr(cb, "grid") and cb.grid.device != device:
        cb = cb.to(device) if hasattr(cb, "to") else cb
    require_standin_table(cb, "mpq_refine_codebook")
    timings: Dict[str, float] = {}

    init_mode = str(getattr(args, "mpq_init", "rtn") or "rtn").strip().lower()
    seed = int(getattr(args, "seed", getattr(args, "mpq_seed", 0)) or 0)
    if init_mode == "random":
        hat_init, idx_init = _random_e8p12_init(cb=cb, rows=m, nblocks=nblocks, seed_key=f"{module_name}:mpq_init",
                                                base_seed=seed, device=device, dtype=Wr.dtype)
    elif init_mode == "rtn":
        hat_init, idx_init = _rtn_e8p12_init(Wr=Wr, cb=cb)
    elif init_mode in {"float", "paper", "unquantized"}:
        hat_init = Wr.clone()
        _, idx_init = _rtn_e8p12_init(Wr=Wr, cb=cb)
    elif init_mode == "zero":
        hat_init, idx_init = _zero_e8p12_init(Wr=Wr, cb=cb)
    elif init_mode == "ldlq":
        hat_init = hatWr0.to(device=device, dtype=torch.float32).contiguous()
        idx_init = Qidxs0.to(device=device, dtype=torch.int64)
    else:
        raise ValueError(f"unknown mpq_init={init_mode!r} (expected 'float', 'random', 'rtn', 'zero', or 'ldlq').")

    t0 = time.time()
    _, S, V, Vs, rank, eigen_floor = _vamp_hessian_eigen(Hr, jitter_base=float(adapter_cfg.jitter_base),
                                                         floor_scale=float(adapter_cfg.eigen_floor_scale))
    torch.cuda.synchronize(device)
    timings["eigh_s"] = time.time() - t0

    block_rows = _resolve_block_rows(m, int(getattr(args, "mpq_block_rows", adapter_cfg.block_rows)
                                            or adapter_cfg.block_rows))
    # the rank-space operator packed once for the bf16-plane products (None: fp32 path)
    packed = (ops.rankspace_pack(V, Vs) if bool(getattr(adapter_cfg, "x6_products", True)) and n >= ops.X6_MIN_N
              else None)
    requested_obs = float(getattr(args, "mpq_obs_precision", 0.0) or 0.0)
    if requested_obs > 0.0:
        obs_precision = requested_obs
    elif packed is not None:
        du = ops.gemm_x6((Wr - hat_init).contiguous(), packed[2 * n * n:], n)
        sq = du.square().sum(dim=1).double()
        mse = max(float(sq.sum().item()) / max(m * n, 1), 1e-12)
        obs_precision = 1.0 / mse
    else:
        du = ops.gemm((Wr - hat_init).contiguous(), Vs)
        sq = du.square().sum(dim=1).double()
        mse = max(float(sq.sum().item()) / max(m * n, 1), 1e-12)
        obs_precision = 1.0 / mse

    solver, polish_req = _resolve_combo(args)
    vamp_cfg = _build_vamp_cfg(args, polish_mode=polish_req)
    hat0 = hatWr0.to(device=device, dtype=torch.float32).contiguous()
    exact_ldlq, exact_ldlq_chunks = _chunk_means(_surrogate_rows(Wr, hat0, Hr), block_rows)
    if solver == "ldlq":
        if init_mode == "random":
            final_hat, final_idx = hat_init.clone(), idx_init.clone()
        else:
            final_hat, final_idx = hat0.clone(), Qidxs0.to(device=device, dtype=torch.int64).clone()
    else:
        final_hat, final_idx = hat_init.clone(), idx_init.clone()
    exact_before, exact_before_chunks = _chunk_means(_surrogate_rows(Wr, final_hat, Hr), block_rows)

    obs_block = float(obs_precision)
    gamma_sum, gamma_count, gamma_min, gamma_max = 0.0, 0, math.inf, -math.inf
    gamma_blocks = []
    block_stats = []
    t0 = time.time()
    if solver == "vamp":
        mode = str(vamp_cfg.prior_tau_scale_mode or "absmax").strip().lower()
        ws = ops.workspace(int(ops._lib.load().mpq_e8p12_vamp_workspace_size(block_rows, n)), device)
        for r0 in range(0, m, block_rows):
            r1 = min(m, r0 + block_rows)
            pscale = None
            if float(vamp_cfg.prior_tau) > 0.0 and mode not in ("absmax", "exact_full", "exact_full_absmax"):
                pscale = prior_scale_from_center(Wr[r0:r1].reshape(r1 - r0, nblocks, 8), mode).reshape(-1)
            idx_b, hat_b, _, _, g1_b, st = ops.e8p12_vamp_solve(Wr[r0:r1], final_hat[r0:r1], V, S, Vs, vamp_cfg,
                                                                prior_scale=pscale, obs_init=obs_block,
                                                                want_state=True, ws=ws, packed=packed)
            final_hat[r0:r1] = hat_b
            final_idx[r0:r1] = idx_b
            if bool(vamp_cfg.em_obs_precision) and float(vamp_cfg.obs_precision) <= 0.0:
                obs_block = float(st["obs_precision_final"])
            # the block's gamma1 sum (fp64), min and max stay on the device until the loop ends
            g64 = g1_b.double()
            gamma_blocks.append(torch.stack([g64.sum(), g64.min(), g64.max()]))
            gamma_count += int(g64.numel())
            block_stats.append(st)
        for g_sum, g_min, g_max in (torch.stack(gamma_blocks).tolist() if gamma_blocks else []):
            gamma_sum += g_sum
            gamma_min = min(gamma_min, g_min)
            gamma_max = max(gamma_max, g_max)
        del ws
    del packed
    torch.cuda.synchronize(device)
    timings["vamp_s"] = time.time() - t0

    t0 = time.time()
    sweeps = max(int(getattr(args, "mpq_polish_sweeps", 3) if solver == "ldlq" else vamp_cfg.polish_sweeps), 0)
    polish_mode = _resolve_polish_mode(sweeps=sweeps, mode=polish_req)
    _resolve_e8p12_polish_metric(str(getattr(args, "mpq_polish_metric", vamp_cfg.polish_metric)))
    polish_updates = 0.0
    changed = 0
    max_blocks = int(getattr(args, "mpq_polish_max_blocks", vamp_cfg.polish_max_blocks) or 0)
    if polish_mode == "block_cd" and _resolve_e8p12_polish_metric(
            str(getattr(args, "mpq_polish_metric", "gram"))) == "gram":
        ctx = ops.e8p12_cd_prepare(Vs)
        x_p, idx_p, _, _, acc = ops.e8p12_cd_polish(final_hat, final_idx, Vs, ctx, sweeps=sweeps,
                                                    block_rows=block_rows, W=Wr, max_blocks=max_blocks)
        changed = int((idx_p != final_idx).sum().item())
        final_hat, final_idx = x_p, idx_p
        polish_updates = float(acc.sum().item())
    elif polish_mode == "block_cd":
        # the diag metric: the generic block CD with the codebook's nearest codeword, per row block
        from ..solver import polish_e8p12_rankspace

        before = final_idx.clone()
        for r0 in range(0, m, block_rows):
            r1 = min(m, r0 + block_rows)
            Yu_b = ops.gemm(Wr[r0:r1].contiguous(), Vs)
            x_b, i_b, _, st_b = polish_e8p12_rankspace(
                x_init=final_hat[r0:r1].contiguous(), idxs_init=final_idx[r0:r1].contiguous(), Y_u=Yu_b, Vs=Vs,
                cb=cb, sweeps=sweeps, polish_mode="block_cd", polish_metric="diag", polish_max_blocks=max_blocks)
            final_hat[r0:r1] = x_b
            final_idx[r0:r1] = i_b
            polish_updates += float(st_b.get("accepted_updates", 0.0))
        changed = int((final_idx != before).sum().item())
    torch.cuda.synchronize(device)
    timings["polish_s"] = time.time() - t0

    exact_after, exact_after_chunks = _chunk_means(_surrogate_rows(Wr, final_hat, Hr), block_rows)
    violation_count, max_delta, max_ratio = 0, 0.0, 0.0
    for ldlq_val, mpq_val in zip(exact_ldlq_chunks, exact_after_chunks):
        if mpq_val > ldlq_val + 1e-8:
            violation_count += 1
            max_delta = max(max_delta, float(mpq_val - ldlq_val))
            if ldlq_val > 0:
                max_ratio = max(max_ratio, float(mpq_val / ldlq_val))
    total = m * nblocks
    gamma_mean = gamma_sum / max(gamma_count, 1)
    stats: Dict[str, Any] = {
        "method": "mpq",
        "backend": "quip",
        "solver": solver,
        "polish_mode": polish_mode,
        "module": str(module_name),
        "init_mode": init_mode,
        "seed": seed,
        "m": int(m),
        "n": int(n),
        "rank": int(rank),
        "eigen_floor": float(eigen_floor),
        "obs_precision_initial": float(obs_precision),
        "obs_precision_final": float(obs_block),
        "block_rows": int(block_rows),
        "exact_surrogate_ldlq_mean": exact_ldlq,
        "exact_surrogate_ldlq_chunk_means": exact_ldlq_chunks,
        "exact_surrogate_before_mean": exact_before,
        "exact_surrogate_before_chunk_means": exact_before_chunks,
        "exact_surrogate_after_mean": exact_after,
        "exact_surrogate_after_chunk_means": exact_after_chunks,
        "exact_surrogate_gain_mean": float(exact_before - exact_after),
        "surrogate_chunk_violation_count": int(violation_count),
        "surrogate_chunk_violation_max_delta": float(max_delta),
        "surrogate_chunk_violation_max_ratio": float(max_ratio),
        "solver_time_s": float(time.time() - start),
        "solver_stats": block_stats[-1] if block_stats else {},
        "polish_updates": polish_updates,
        "timings": timings,
        "mechanism": {
            "regime": "2bit_e8p12",
            "cleanup_unit": "e8p12_block",
            "module": str(module_name),
            "layer_index": _layer_index(module_name),
            "bits": 2,
            "rows": int(m),
            "cols": int(n),
            "nblocks": int(nblocks),
            "stage1_gamma1_mean": float(gamma_mean),
            "stage1_gamma1_min": float(gamma_min) if math.isfinite(gamma_min) else float(gamma_mean),
            "stage1_gamma1_max": float(gamma_max) if math.isfinite(gamma_max) else float(gamma_mean),
            "stage1_gamma1_count": int(gamma_count),
            "cleanup_changed_count": int(changed),
            "cleanup_total_count": int(total),
            "cleanup_changed_fraction": float(changed / max(total, 1)),
            "cleanup_agreement_fraction": float(1.0 - changed / max(total, 1)),
        },
    }
    return final_hat.to(dtype=hatWr0.dtype), final_idx, stats
