"""GPTQModel adapter: per-linear uniform-grid MPQ solve on MI355X.

Drop-in for the reference's ``mpq/adapters/gptqmodel.py``:

* ``GPTQAdapterConfig``          reference :37-43
* ``run_mpq_quantization``       reference :650-1163 (``solver="vamp"`` path)

Pipeline (all on the ROCm device):
  H <- hessian_scale * H; eigh of the unrotated H (``mpq_syevd``: the library's own
  tridiagonalisation, divide and conquer on the tridiagonal matrix and compact-WY
  back-transformation on its MFMA GEMM) -> ``mpq_eigh_postprocess`` (floor, descending order,
  S, Vs); internal block-Hadamard rotation of W, H (both sides) and V
  (``mpq_block_hadamard``); GPTQ group parameters (``quantizer.find_params`` if a
  quantizer is given, else ``mpq_gptq_find_params``); RTN (``mpq_uniform_rtn``);
  observation-precision warm start; the sequential row-block VAMP chain
  (``mpq_uniform_vamp_solve``, EM precision carried block to block); one batched
  greedy CD polish over all rows (``mpq_uniform_cd_polish``, greedy order per row
  block, identical to polishing block by block); proxy-loss audit
  ``(W-Q) H (W-Q)^T``; inverse rotation of Q.

Row blocks use exactly ``adapter_cfg.block_rows`` rows (the reference enlarges
them from free memory on CUDA, mpq/adapters/gptqmodel.py:313-327, which changes
results; pass ``auto_block_rows=True`` for that behaviour).
"""
from __future__ import annotations

import time
from dataclasses import dataclass
from typing import Any, Dict, List, Optional, Tuple

import torch

from .. import ops
from ..rotation import (
    apply_left_block_hadamard,
    apply_right_block_hadamard,
    apply_right_block_hadamard_inverse,
    resolve_block_hadamard_plan,
    sample_rademacher_signs,
)
from ..solver import UniformVampConfig, _resolve_polish_mode


@dataclass(frozen=True)
class GPTQAdapterConfig:
    hessian_scale: float = 0.5  # GPTQModel stores H = 2/m X^T X
    block_rows: int = 128
    jitter_base: float = 1e-6
    eigen_floor_scale: float = 1e-6
    rotation_seed: int = 0
    auto_block_rows: bool = False
    eigen_cache: bool = True  # reuse the decomposition of an identical Hessian (q/k/v, gate/up)
    # rank-space products as fp32-accurate bf16-plane products on the matrix cores (ops.gemm_x6)
    # when cols % 128 == 0 and cols >= ops.X6_MIN_N; False keeps every product on the fp32 MFMA kernel
    x6_products: bool = True


class MinMaxQuantizer:
    """GPTQ asymmetric min-max quantizer with the ``find_params`` protocol, on the HIP kernel."""

    def __init__(self, bits: int):
        self.maxq = torch.tensor(2 ** int(bits) - 1)
        self.scale = None
        self.zero = None

    def find_params(self, x: torch.Tensor, weight: bool = True) -> None:
        s, z = ops.gptq_find_params(x, int(x.shape[1]), int(self.maxq))
        self.scale, self.zero = s, z


def resolve_internal_rotation(*, requested: str, cols: int, module_name: str, seed: int,
                              device: torch.device) -> Dict[str, Any]:
    """reference :46-118."""
    req = str(requested or "none").strip().lower()
    if req in {"", "none"}:
        return {"requested": "none", "effective": "none", "mode": "none", "signs": None, "block_dim": 1,
                "fallback_reason": "", "internal": False}
    if req in {"model_random", "model_hadamard"}:
        return {"requested": req, "effective": req, "mode": "none", "signs": None, "block_dim": 1,
                "fallback_reason": "", "internal": False}
    if req != "internal_hadamard":
        raise ValueError("mpq only supports rotation in {none, model_hadamard, model_random, internal_hadamard}; "
                         f"got rotation={requested!r}.")
    mode, block_dim = resolve_block_hadamard_plan(int(cols))
    if mode == "none":
        return {"requested": "internal_hadamard", "effective": "none", "mode": "none", "signs": None,
                "block_dim": 1, "fallback_reason": f"unsupported_block_hadamard_width:{int(cols)}",
                "internal": False}
    signs = sample_rademacher_signs(width=int(cols), key=f"{module_name}:full", seed=int(seed), device=device)
    return {"requested": "internal_hadamard", "effective": "internal_block_hadamard", "mode": "block",
            "signs": signs, "block_dim": int(block_dim), "fallback_reason": "", "internal": True}


# The most recent eigendecomposition per device.  The linears of one block that read the same
# input (q/k/v, gate/up) carry identical Hessians; their decomposition is reused when the
# symmetrized matrix is element-for-element equal, which returns exactly the bits a fresh
# computation would (the solver is deterministic).  The entries are read-only to callers.
_EIGEN_CACHE: Dict[Any, Tuple[torch.Tensor, Tuple[float, float], tuple]] = {}


def clear_eigen_cache() -> None:
    """Drop the cached eigendecompositions (and the Hessian copies they are keyed on)."""
    _EIGEN_CACHE.clear()


@torch.inference_mode()
def vamp_hessian_eigen(H: torch.Tensor, *, jitter_base: float = 1e-6, floor_scale: float = 1e-6,
                       use_cache: bool = True):
    """Floored descending eigendecomposition (reference :276-310).  Returns (lam, S, V, Vs, floor)."""
    Hs = 0.5 * (H + H.T)
    if not bool(torch.isfinite(Hs).all()):
        Hs = torch.nan_to_num(Hs, nan=0.0, posinf=0.0, neginf=0.0)
    key = (Hs.device, tuple(Hs.shape))
    params = (float(jitter_base), float(floor_scale))
    if use_cache:
        hit = _EIGEN_CACHE.get(key)
        if hit is not None and hit[1] == params and hit[0].dtype == Hs.dtype and torch.equal(hit[0], Hs):
            return hit[2]
    lam_asc, V_asc = ops.syevd(Hs)
    max_lam = float(lam_asc[-1].item()) if lam_asc.numel() else 0.0
    diag_mean = float(torch.diagonal(Hs).mean().abs().item()) if Hs.numel() else 0.0
    floor = max(float(jitter_base), float(floor_scale) * max(diag_mean, max_lam, 1e-12))
    lam, S, V, Vs = ops.eigh_postprocess(lam_asc, V_asc, floor)
    del V_asc
    out = (lam, S, V, Vs, float(floor))
    if use_cache:
        _EIGEN_CACHE.clear()  # one entry: the newest decomposition
        _EIGEN_CACHE[key] = (Hs, params, out)
    return out


def _resolve_block_rows(rows: int, cols: int, maxq: int, requested: int, device: torch.device, auto: bool) -> int:
    block_rows = min(int(rows), max(int(requested), 1))
    if not auto:
        return block_rows
    free_bytes, _ = torch.cuda.mem_get_info(device)
    bytes_per_row = 4 * (8 * int(cols) + 4 * int(cols) * (int(maxq) + 1))
    budget = min(4 * 1024 ** 3, int(free_bytes) // 2)
    automatic = max(8, min(int(rows), int(budget // max(bytes_per_row, 1))))
    return min(int(rows), max(block_rows, int(automatic)))


@torch.inference_mode()
def run_mpq_quantization(
    *,
    W: torch.Tensor,
    H: torch.Tensor,
    quantizer: Any,
    qcfg: Any,
    module_name: str,
    vamp_cfg: UniformVampConfig,
    adapter_cfg: GPTQAdapterConfig = GPTQAdapterConfig(),
    precomputed_eigen: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
) -> Tuple[torch.Tensor, Optional[torch.Tensor], Optional[torch.Tensor], Optional[torch.Tensor],
           Optional[torch.Tensor], float, Dict[str, Any]]:
    """Per-linear MPQ (uniform grid) on one GPU.

    Returns (Q fp32 rows x cols in the original basis, q_int uint8 (solver basis),
    scale_groups, zero_groups, g_idx int32, quant_time_s, stats) as the reference.
    ``precomputed_eigen`` = (floored descending eigenvalues, eigenvectors) of the
    unrotated ``hessian_scale * H`` -- with ``qcfg.desc_act``, of the rotated and
    column-permuted Hessian the solver works on -- replaces the device ``eigh`` (used to
    compare against another eigensolver's output on identical inputs).
    """
    start = time.time()
    device = W.device
    if device.type != "cuda":
        raise ValueError("run_mpq_quantization: W must be on a ROCm device (mpq_amd has no CPU path).")
    W = W.to(torch.float32)
    H = H.to(device=device, dtype=torch.float32)
    rows, cols = W.shape
    bits = int(getattr(qcfg, "bits"))
    maxq = int(2 ** bits - 1)
    group_size = int(getattr(qcfg, "group_size", cols))
    if group_size == -1:
        group_size = cols
    mpq_cfg = getattr(qcfg, "mpq", None)
    solver_name = str(getattr(mpq_cfg, "dispatch_solver", getattr(mpq_cfg, "solver", "vamp")) or "vamp").strip().lower()
    if solver_name != "vamp":
        raise ValueError(f"mpq_amd implements solver='vamp'; got {solver_name!r}.")
    use_activation_order = bool(getattr(qcfg, "desc_act", False))
    rotation = resolve_internal_rotation(
        requested=str(getattr(mpq_cfg, "rotation_mode", getattr(qcfg, "rotation", None) or "none")),
        cols=int(cols), module_name=str(module_name), seed=int(adapter_cfg.rotation_seed), device=device)
    timings: Dict[str, float] = {}

    H_work = float(adapter_cfg.hessian_scale) * H
    t0 = time.time()
    if use_activation_order:
        # the reference decomposes the rotated, permuted Hessian in the solver basis (:716-722 take the
        # unrotated decomposition only without activation order); formed below
        lam = S = V = Vs = None
        eigen_floor = 0.0
    elif precomputed_eigen is not None:
        lam = precomputed_eigen[0].to(device=device, dtype=torch.float32).contiguous()
        V = precomputed_eigen[1].to(device=device, dtype=torch.float32).contiguous()
        S = torch.sqrt(lam)
        Vs = ops.scale_columns(V, S)
        eigen_floor = float(lam.min().item())
    else:
        lam, S, V, Vs, eigen_floor = vamp_hessian_eigen(H_work, jitter_base=adapter_cfg.jitter_base,
                                                        floor_scale=adapter_cfg.eigen_floor_scale,
                                                        use_cache=bool(adapter_cfg.eigen_cache))
    torch.cuda.synchronize(device)
    timings["eigh_s"] = time.time() - t0
    signs = rotation["signs"]
    had = int(rotation["block_dim"])
    if rotation["mode"] == "block":
        W_work = apply_right_block_hadamard(W, signs=signs, had_dim=had)
        H_metric = apply_right_block_hadamard(apply_left_block_hadamard(H_work, signs=signs, had_dim=had),
                                              signs=signs, had_dim=had)
        if V is not None:
            V = apply_left_block_hadamard(V, signs=signs, had_dim=had)
            Vs = ops.scale_columns(V, S)  # Vs = V * S after the rotation (reference :887-890)
    else:
        W_work = W.contiguous()
        H_metric = H_work.contiguous()
    perm = invperm = None
    if use_activation_order:
        # columns by descending diagonal of the solver-basis Hessian (reference :733-740; a stable sort,
        # ties by column index, where the reference's argsort is unstable)
        diag = torch.diagonal(H_metric).to("cpu", torch.float64).tolist()
        order = sorted(range(cols), key=lambda j: -diag[j])
        perm = torch.tensor(order, dtype=torch.int32, device=device)
        inv = [0] * cols
        for pos, j in enumerate(order):
            inv[j] = pos
        invperm = torch.tensor(inv, dtype=torch.int32, device=device)
        W_work = ops.permute_columns(W_work.to(torch.float32), perm)
        H_metric = ops.permute_symmetric(H_metric, perm)
    dead = torch.diagonal(H_metric) == 0
    has_dead = bool(dead.any().item())
    if use_activation_order and not has_dead:
        t0 = time.time()
        if precomputed_eigen is not None:
            lam = precomputed_eigen[0].to(device=device, dtype=torch.float32).contiguous()
            V = precomputed_eigen[1].to(device=device, dtype=torch.float32).contiguous()
            S = torch.sqrt(lam)
            Vs = ops.scale_columns(V, S)
            eigen_floor = float(lam.min().item())
        else:
            lam, S, V, Vs, eigen_floor = vamp_hessian_eigen(H_metric, jitter_base=adapter_cfg.jitter_base,
                                                            floor_scale=adapter_cfg.eigen_floor_scale,
                                                            use_cache=bool(adapter_cfg.eigen_cache))
        torch.cuda.synchronize(device)
        timings["eigh_s"] += time.time() - t0
    if has_dead:
        H_metric = H_metric.clone()
        W_work = W_work.clone()
        H_metric[dead, dead] = 1
        W_work[:, dead] = 0
        lam, S, V, Vs, eigen_floor = vamp_hessian_eigen(H_metric, jitter_base=adapter_cfg.jitter_base,
                                                        floor_scale=adapter_cfg.eigen_floor_scale,
                                                        use_cache=bool(adapter_cfg.eigen_cache))

    # group parameters in the solver basis
    if quantizer is not None and hasattr(quantizer, "find_params") and not isinstance(quantizer, MinMaxQuantizer):
        sc, zc = [], []
        for g0 in range(0, cols, group_size):
            quantizer.find_params(W_work[:, g0:g0 + group_size].contiguous(), weight=True)
            sc.append(quantizer.scale.to(device=device, dtype=torch.float32).reshape(rows, -1)[:, :1].clone())
            zc.append(quantizer.zero.to(device=device, dtype=torch.float32).reshape(rows, -1)[:, :1].clone())
        scale_groups = torch.cat(sc, 1).contiguous()
        zero_groups = torch.cat(zc, 1).contiguous()
    else:
        scale_groups, zero_groups = ops.gptq_find_params(W_work, group_size, maxq)
    block_rows = _resolve_block_rows(rows, cols, maxq, int(adapter_cfg.block_rows), device,
                                     bool(adapter_cfg.auto_block_rows))
    _, x_rtn = ops.uniform_rtn(W_work, scale_groups, zero_groups, group_size, maxq, want_q=False)

    # Rank-space targets W Vs and the RTN decision's x_rtn Vs, formed once for all rows (the
    # reference forms them per row block inside the solver, mpq/solver.py:467-480); the row blocks
    # and the polish take slices, and each block returns its best decision's x Vs for the polish.
    # The rank-space operator packed once per linear for the bf16-plane products (None: fp32 path).
    packed = ops.rankspace_pack(V, Vs) if bool(adapter_cfg.x6_products) and cols >= ops.X6_MIN_N else None
    if packed is not None:
        Vs_packed = packed[2 * cols * cols:]
        Yu_all = ops.gemm_x6(W_work, Vs_packed, cols)
        XR_all = ops.gemm_x6(x_rtn, Vs_packed, cols)
    else:
        Yu_all = ops.gemm(W_work, Vs)
        XR_all = ops.gemm(x_rtn, Vs)
    # observation-precision warm start (reference :920-941): per block sums accumulated in double
    if float(getattr(vamp_cfg, "obs_precision", 0.0)) > 0.0:
        obs_precision = float(vamp_cfg.obs_precision)
    else:
        sq = (Yu_all - XR_all).square().sum(dim=1)
        # one device sum per block (as the reference's per-block loop forms them), read back at once
        sums = torch.stack([sq[r0:r0 + block_rows].sum() for r0 in range(0, rows, block_rows)]).tolist()
        mse = max(sum(sums) / max(rows * cols, 1), 1e-12)
        obs_precision = 1.0 / mse

    torch.cuda.synchronize(device)
    t_solve = time.time()
    q_int = torch.empty(rows, cols, dtype=torch.uint8, device=device)
    err_vamp = torch.empty(rows, dtype=torch.float32, device=device)
    rtn_err = torch.empty(rows, dtype=torch.float32, device=device)
    XP_all = torch.empty(rows, cols, dtype=torch.float32, device=device)
    ws = ops.workspace(int(ops._lib.load().mpq_uniform_vamp_workspace_size(block_rows, cols)), device)
    obs_block = float(obs_precision)
    block_stats: List[Dict[str, Any]] = []
    for r0 in range(0, rows, block_rows):
        r1 = min(rows, r0 + block_rows)
        _, _, _, _, st = ops.uniform_vamp_solve(
            W_work[r0:r1], x_rtn[r0:r1], scale_groups[r0:r1], zero_groups[r0:r1], group_size, maxq, V, S, Vs,
            vamp_cfg, obs_init=obs_block, ws=ws, Yu=Yu_all[r0:r1], xr=XR_all[r0:r1], xprod_out=XP_all[r0:r1],
            packed=packed, q_out=q_int[r0:r1], err_out=err_vamp[r0:r1], rtn_err_out=rtn_err[r0:r1])
        if bool(getattr(vamp_cfg, "em_obs_precision", True)):
            obs_block = float(st["obs_precision_final"])
        block_stats.append(st)
    del ws, XR_all
    torch.cuda.synchronize(device)
    timings["vamp_s"] = time.time() - t_solve

    t_pol = time.time()
    sweeps = max(int(getattr(vamp_cfg, "polish_sweeps", 3)), 0)
    mode = _resolve_polish_mode(sweeps=sweeps, mode=str(getattr(vamp_cfg, "polish_mode", "block_cd")))
    if mode == "topk_block_cd":
        raise ValueError("mpq_amd implements polish_mode='block_cd'.")
    polish_updates = 0.0
    changed = 0
    if mode == "block_cd":
        q_pol, eb, ea, imp, acc = ops.uniform_cd_polish(None, q_int, scale_groups, zero_groups, group_size, maxq,
                                                        Vs, H_metric, block_rows=block_rows, sweeps=sweeps,
                                                        select=True, Yu=Yu_all, xprod=XP_all,
                                                        S=None if packed is None else S, packed=packed)
        final_err = torch.where(imp.bool(), ea, err_vamp)
        changed = int((q_pol != q_int).sum().item())
        q_int = q_pol
        polish_updates = float(acc.sum().item())
    else:
        final_err = err_vamp
    torch.cuda.synchronize(device)
    timings["polish_s"] = time.time() - t_pol
    del packed

    Q_work = ops.dequant(q_int, scale_groups, zero_groups, group_size)
    delta = W_work - Q_work
    raw_rows = (ops.gemm(delta, H_metric) * delta).sum(dim=1)
    g_idx = torch.arange(cols, device=device, dtype=torch.int32) // int(group_size)
    if invperm is not None:
        # back to the column order of the solver basis (reference :1090-1095)
        Q_work = ops.permute_columns(Q_work, invperm)
        q_int = ops.permute_columns(q_int, invperm)
        g_idx = g_idx.index_select(0, invperm.long())
    if rotation["mode"] == "block":
        Q = apply_right_block_hadamard_inverse(Q_work, signs=signs, had_dim=had)
    else:
        Q = Q_work
    if mpq_cfg is not None:
        for k, v in (("rotation_requested", rotation["requested"]), ("rotation_effective", rotation["effective"]),
                     ("rotation_internal", rotation["internal"]), ("rotation_block_dim", rotation["block_dim"]),
                     ("rotation_fallback_reason", rotation["fallback_reason"])):
            try:
                setattr(mpq_cfg, k, v)
            except Exception:  # frozen configs
                pass
    layer_err_sum = float(final_err.sum().item())
    raw_sum = float(raw_rows.sum().item())
    torch.cuda.synchronize(device)
    quant_time = time.time() - start
    stats: Dict[str, Any] = {
        "method": "mpq",
        "solver": "vamp",
        "polish_mode": mode,
        "module": str(module_name),
        "bits": bits,
        "group_size": group_size,
        "rotation_requested": str(rotation["requested"]),
        "rotation_effective": str(rotation["effective"]),
        "rotation_internal": bool(rotation["internal"]),
        "rotation_block_dim": had,
        "rotation_fallback_reason": str(rotation["fallback_reason"]),
        "desc_act": bool(use_activation_order),
        "rows": int(rows),
        "cols": int(cols),
        "rank": int(S.numel()),
        "eigen_floor": float(eigen_floor),
        "block_rows": int(block_rows),
        "block_cd_backend": "hip",
        "obs_precision_initial": float(obs_precision),
        "obs_precision_final": float(obs_block),
        "layer_error_sum": layer_err_sum,
        "stabilized_objective_mean_final": layer_err_sum / max(rows, 1),
        "raw_objective_mean_final": raw_sum / max(rows, 1),
        "proxy_loss": raw_sum,
        "rankspace_raw_abs_diff_mean": float((final_err - raw_rows).abs().sum().item()) / max(rows, 1),
        "rtn_error_sum": float(rtn_err.sum().item()),
        "vamp_iters": [int(b["best_iter"]) + 1 for b in block_stats],
        "vamp_iters_entered": [
            (int(b["stop_iter"]) + 1 if int(b["stop_iter"]) >= 0 else int(b["iters"])) for b in block_stats],
        "block_stats": block_stats,
        "polish_updates": polish_updates,
        "changed_by_polish": changed,
        "timings": timings,
        "quant_time_s": float(quant_time),
    }
    return Q, q_int, scale_groups, zero_groups, g_idx, float(quant_time), stats


@torch.inference_mode()
def prepare_gptq_internal_hadamard(
    *,
    W: torch.Tensor,
    H: torch.Tensor,
    qcfg: Any,
    module_name: str,
    adapter_cfg: GPTQAdapterConfig = GPTQAdapterConfig(),
) -> Tuple[torch.Tensor, torch.Tensor, Dict[str, Any]]:
    """Rotate a linear into the internal block-Hadamard basis before GPTQModel's own solver (reference
    mpq/adapters/gptqmodel.py:593-632, called from the GPTQ hook when ``solver="gptq"`` runs with
    ``rotation_mode="internal_hadamard"``): ``W_work = W diag(signs) Had``, ``H_work`` rotated on both
    sides, and the rotation plan for ``finalize_gptq_internal_hadamard``.  Without an internal
    rotation W and H are returned as fp32.  The reference's optional file-backed paired (W, H) cache
    (``qcfg.mpq.paired_matrix_cache_dir``) is not provided: setting it raises ValueError."""
    mpq_cfg = getattr(qcfg, "mpq", None)
    if getattr(mpq_cfg, "paired_matrix_cache_dir", None):
        raise ValueError("mpq_amd does not provide the file-backed paired matrix cache (paired_matrix_cache_dir).")
    if float(adapter_cfg.hessian_scale) <= 0.0:
        raise ValueError(f"hessian_scale must be positive, got {float(adapter_cfg.hessian_scale)}")
    requested = getattr(mpq_cfg, "rotation_mode", getattr(qcfg, "rotation", None) or "none")
    plan = resolve_internal_rotation(requested=str(requested), cols=int(W.shape[1]), module_name=str(module_name),
                                     seed=int(adapter_cfg.rotation_seed), device=W.device)
    W32 = W.to(dtype=torch.float32).contiguous()
    H32 = H.to(dtype=torch.float32).contiguous()
    if not bool(plan["internal"]):
        return W32, H32, plan
    had, signs = int(plan["block_dim"]), plan["signs"]
    W_work = apply_right_block_hadamard(W32, signs=signs, had_dim=had)
    H_work = apply_right_block_hadamard(apply_left_block_hadamard(H32, signs=signs, had_dim=had), signs=signs,
                                        had_dim=had)
    # the reference stores the scaled Hessian and divides the scale back out (exact for the default 0.5)
    hs = float(adapter_cfg.hessian_scale)
    H_work = (hs * H_work) / hs
    return W_work.contiguous(), H_work.contiguous(), plan


@torch.inference_mode()
def finalize_gptq_internal_hadamard(*, Q_work: torch.Tensor, rotation_plan: Dict[str, Any]) -> torch.Tensor:
    """Rotate a result back to the original basis (reference mpq/adapters/gptqmodel.py:635-647)."""
    if not bool(rotation_plan.get("internal", False)):
        return Q_work.to(dtype=torch.float32).contiguous()
    return apply_right_block_hadamard_inverse(Q_work.to(dtype=torch.float32).contiguous(),
                                              signs=rotation_plan["signs"],
                                              had_dim=int(rotation_plan["block_dim"])).contiguous()


def install_internal_hadamard_input_hooks(model: torch.nn.Module, *, rotation_seed: int = 0) -> int:
    """Forward pre-hooks that rotate each packed module's input into the solver basis
    (reference ``mpq/adapters/gptqmodel.py:1166-1247``).

    Packed internal-Hadamard weights stay in the solver basis; applying the module's signed block
    Hadamard (signs from ``stable_seed(f"{name}:full", rotation_seed)``, block = largest power-of-2
    factor of the input width) to its input reproduces the dense inverse-rotated weight.  Returns
    the number of modules hooked.  Inputs must be ROCm tensors (the rotation runs on the HIP kernel).
    """
    installed = 0
    for module_name, module in model.named_modules():
        if not module_name or getattr(module, "_mpq_internal_hadamard_hook", None) is not None:
            continue
        if not all(hasattr(module, attr) for attr in ("qweight", "qzeros", "scales")):
            continue
        width = int(getattr(module, "in_features", 0) or getattr(module, "infeatures", 0) or 0)
        if width <= 0:
            qweight = getattr(module, "qweight", None)
            bits = int(getattr(module, "bits", 0) or 0)
            pack_dtype = getattr(qweight, "dtype", torch.int32)
            pack_bits = (torch.iinfo(pack_dtype).bits
                         if isinstance(pack_dtype, torch.dtype) and not pack_dtype.is_floating_point else 32)
            if isinstance(qweight, torch.Tensor) and bits > 0:
                width = int(qweight.shape[0]) * int(pack_bits // bits)
        if width <= 0:
            raise RuntimeError(f"Cannot determine MPQ input width for quantized module {module_name!r}")
        mode, block_dim = resolve_block_hadamard_plan(width)
        if mode == "none":
            continue
        signs_by_device: Dict[torch.device, torch.Tensor] = {}

        def _rotate_input(_module, args, *, _name=module_name, _width=width, _block_dim=block_dim,
                          _cache=signs_by_device):
            if not args or not isinstance(args[0], torch.Tensor):
                return args
            value = args[0]
            if int(value.shape[-1]) != int(_width):
                raise RuntimeError(
                    f"MPQ input width mismatch for {_name!r}: expected {_width}, got {int(value.shape[-1])}")
            signs = _cache.get(value.device)
            if signs is None:
                signs = sample_rademacher_signs(width=int(_width), key=f"{_name}:full", seed=int(rotation_seed),
                                                device=value.device, dtype=torch.float32)
                _cache[value.device] = signs
            flat = value.reshape(-1, int(_width)).to(torch.float32).contiguous()
            rotated = apply_right_block_hadamard(flat, signs=signs, had_dim=int(_block_dim))
            return (rotated.reshape(value.shape).to(dtype=value.dtype), *args[1:])

        handle = module.register_forward_pre_hook(_rotate_input)
        setattr(module, "_mpq_internal_hadamard_hook", handle)
        installed += 1
    return installed


@torch.inference_mode()
def postprocess_gptq_quantization(
    *,
    W: torch.Tensor,
    H: torch.Tensor,
    Q_init: torch.Tensor,
    scale_groups: torch.Tensor,
    zero_groups: torch.Tensor,
    g_idx: torch.Tensor,
    qcfg: Any,
    module_name: str,
    adapter_cfg: GPTQAdapterConfig = GPTQAdapterConfig(),
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, float, Dict[str, Any]]:
    """Greedy-CD polish of a finished GPTQ result (reference ``mpq/adapters/gptqmodel.py:1250-1470``).

    The codes ``round(Q_init / s + z)`` are polished in the rank space of ``hessian_scale * H`` with
    one greedy order over all rows, each row keeps the polished codes only if its error drops, and
    the module falls back to ``Q_init`` when the mean error would rise (fail-closed).  Column c
    takes group ``g_idx[c]``'s scale and zero (the reference's ``_expand_group_params_from_gidx``):
    with GPTQModel's act-order layout the parameters are expanded to one per column.
    Returns ``(Q, q_int, scale_groups, zero_groups, g_idx, time_s, stats)``.
    """
    start = time.time()
    if not W.is_cuda:
        raise ValueError(f"W must be on a ROCm device (got {W.device}); mpq_amd has no CPU path.")
    device = W.device
    W = W.to(torch.float32).contiguous()
    H = H.to(device=device, dtype=torch.float32)
    Q_init = Q_init.to(device=device, dtype=torch.float32).contiguous()
    scale_groups = scale_groups.to(device=device, dtype=torch.float32).contiguous()
    zero_groups = zero_groups.to(device=device, dtype=torch.float32).contiguous()
    g_idx = g_idx.to(device=device, dtype=torch.int32)
    bits = int(getattr(qcfg, "bits"))
    maxq = int(2 ** bits - 1)
    rows, cols = W.shape
    group_size = int(getattr(qcfg, "group_size", cols) or cols)
    if group_size <= 0:
        group_size = cols
    if int(g_idx.numel()) != cols:
        raise ValueError(f"g_idx must hold one group per column ({cols}), got {int(g_idx.numel())}")
    n_groups = int(scale_groups.shape[1])
    if tuple(scale_groups.shape) != (rows, n_groups) or tuple(zero_groups.shape) != (rows, n_groups):
        raise ValueError("scale_groups and zero_groups must be rows x groups")
    if int(g_idx.min().item()) < 0 or int(g_idx.max().item()) >= n_groups:
        raise ValueError(f"g_idx entries must lie in [0, {n_groups})")
    expected = torch.arange(cols, device=device, dtype=torch.int32) // group_size
    if n_groups == (cols + group_size - 1) // group_size and bool(torch.equal(g_idx, expected)):
        sg_w, zg_w, gs_w = scale_groups, zero_groups, group_size
    else:  # act-order (or any other) layout: one scale and zero per column
        sg_w = scale_groups.index_select(1, g_idx.long()).contiguous()
        zg_w = zero_groups.index_select(1, g_idx.long()).contiguous()
        gs_w = 1
    mpq_cfg = getattr(qcfg, "mpq", None)
    H_work = float(adapter_cfg.hessian_scale) * H
    _, S, V, Vs, eigen_floor = vamp_hessian_eigen(H_work, jitter_base=adapter_cfg.jitter_base,
                                                  floor_scale=adapter_cfg.eigen_floor_scale)
    q_init, _ = ops.uniform_rtn(Q_init, sg_w.clamp_min(1e-12), zg_w, gs_w, maxq, want_x=False)
    polish_mode = str(getattr(mpq_cfg, "polish_mode", "none") or "none").strip().lower()
    polish_sweeps = int(getattr(mpq_cfg, "polish_sweeps", 0) or 0)
    mode = _resolve_polish_mode(sweeps=polish_sweeps, mode=polish_mode)
    if mode == "topk_block_cd":
        raise ValueError("mpq_amd implements polish_mode='block_cd'; topk_block_cd is not provided.")
    Yu = ops.gemm(W, Vs)

    def _err(x):
        return (Yu - ops.gemm(x, Vs)).square().sum(dim=1)

    err_before = _err(Q_init)
    delta0 = W - Q_init
    raw_before = (ops.gemm(delta0, H_work) * delta0).sum(dim=1)
    polish_updates = 0.0
    if mode == "block_cd":
        q_pol, eb, ea, imp, acc = ops.uniform_cd_polish(None, q_init, sg_w, zg_w, gs_w, maxq,
                                                        Vs, H_work, block_rows=rows, sweeps=polish_sweeps,
                                                        select=True, Yu=Yu, x_in=Q_init)
        err_after = ea
        polish_updates = float(acc.sum().item())
        q_final = q_pol
        Q_final = torch.where(imp.bool().unsqueeze(1), ops.dequant(q_pol, sg_w, zg_w, gs_w), Q_init)
    else:
        err_after = err_before
        q_final = q_init
        Q_final = Q_init
    err_final = _err(Q_final)
    before_mean = float(err_before.mean().item())
    final_mean = float(err_final.mean().item())
    fail_closed = (not bool(torch.isfinite(err_final).all().item())) or (final_mean > before_mean + 1e-9)
    if fail_closed:
        Q_final, q_final, err_final, final_mean = Q_init, q_init, err_before, before_mean
    delta = W - Q_final
    raw_final = (ops.gemm(delta, H_work) * delta).sum(dim=1)
    stats: Dict[str, Any] = {
        "method": "mpq",
        "solver": "gptq",
        "polish_mode": mode,
        "module": str(module_name),
        "bits": bits,
        "group_size": group_size,
        "rows": int(rows),
        "cols": int(cols),
        "rank": int(S.numel()),
        "eigen_floor": float(eigen_floor),
        "block_rows": int(rows),
        "polish_sweeps": int(polish_sweeps),
        "rankspace_error_mean_before": before_mean,
        "rankspace_error_mean_after": float(err_after.mean().item()),
        "rankspace_error_mean_final": final_mean,
        "raw_objective_mean_before": float(raw_before.mean().item()),
        "raw_objective_mean_final": float(raw_final.mean().item()),
        "polish_gain": float((err_before - err_after).mean().item()),
        "polish_updates": polish_updates,
        "polish_assignment_changes": int((q_final != q_init).sum().item()),
        "polish_assignments_total": int(q_init.numel()),
        "block_cd_backend": "hip",
        "module_fail_closed": bool(fail_closed),
        "quant_time_s": float(time.time() - start),
    }
    if mpq_cfg is not None:
        bucket = getattr(mpq_cfg, "_layer_stats", None)
        if not isinstance(bucket, list):
            bucket = []
            try:
                setattr(mpq_cfg, "_layer_stats", bucket)
            except Exception:  # frozen configs
                pass
        bucket.append(stats)
    return Q_final, q_final.to(torch.int32), scale_groups, zero_groups, g_idx, float(time.time() - start), stats
