"""Generic rank-space block coordinate descent (drop-in for the reference's ``mpq/polish/block_cd.py``).

* ``CandidateProvider``                   reference :12-25 (protocol)
* ``BlockCDConfig``                       reference :309-318
* ``block_coordinate_descent_rankspace``  reference :332-625
* ``UniformScalarProvider``               reference :628-653 -> ``mpq_bcd_uniform_propose``
* ``UniformTopKProvider``                 reference :656-682 -> ``mpq_bcd_topk_scalar_propose``
* ``E8P12Provider``                       reference :685-761 -> ``mpq_e8p12_metric_argmin`` (gram metric),
                                          the codebook's nearest-codeword search (diag metric)
* ``E8P12TopKProvider``                   reference :764-861 -> ``mpq_bcd_e8_topk_propose``

Objective: minimise ``|Y_u - x Vs|^2`` over blocks of ``block_size`` columns with candidates from the
provider.  The block loop runs on the host (a provider is caller code); its steps run on the HIP
kernels of ``csrc/block_cd.hip`` and the MFMA GEMM: per block ``rhs = residual_u Vs_blk^T``, the
target, the provider's candidates, the accept test, ``residual_u -= delta Vs_blk``.  Two recipe
cases take the fused polish kernels instead (the same objective, decisions and trace; the rounding of
the running ``rhs`` differs as in the reference's own compiled and eager variants):

* ``UniformScalarProvider``, block size 1, metric diag, greedy order, all blocks:
  ``mpq_uniform_cd_sweeps_recip`` (128-column windows; target ``x + rhs * (1 / diag)`` as :585);
* ``E8P12Provider``, block size 8, metric gram, greedy order, square ``Vs`` and the build's codebook
  table: ``mpq_e8p12_cd_polish`` one sweep per call (the compiled gram step of :212-246).

Differences from the reference (free choices there): greedy and static orders are stable sorts (ties
by block index; ``torch.argsort`` is unstable); without ``idxs_init`` the index of a block that never
accepts a move is the start's own (the codebook's nearest codeword for E8P12, the rounded level for
the uniform grid) or -1 for other providers (the reference leaves it uninitialised).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Dict, Optional, Protocol, Tuple

import torch

from .. import _lib, ops
from ..codebook import require_standin_table

F32 = torch.float32
I64 = torch.int64


class CandidateProvider(Protocol):
    @torch.inference_mode()
    def propose(
        self,
        *,
        block_idx: int,
        start: int,
        end: int,
        x_block: torch.Tensor,  # (B, bs)
        target: torch.Tensor,  # (B, bs)
        metric: str,  # "diag" | "gram"
        gram_chol: Optional[torch.Tensor],  # (bs, bs) if metric == "gram"
    ) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
        """Return (cand_vals, cand_idxs) for this block."""


@dataclass(frozen=True)
class BlockCDConfig:
    sweeps: int = 3
    metric: str = "diag"  # "diag" | "gram"
    accept_tol: float = 0.0
    metric_rows_per_chunk: int = 0  # accepted for compatibility (the argmin kernel streams the codebook)
    max_blocks_per_sweep: int = 0  # if > 0, only the first K blocks of each sweep's order
    order_mode: str = "greedy_gain"  # "static" | "cyclic" | "greedy_gain"
    compile_steps: bool = True  # accepted for compatibility (every step runs on the HIP kernels)


def _stream(t: torch.Tensor) -> int:
    return _lib.stream_handle(t.device)


def _f32c(t: torch.Tensor) -> torch.Tensor:
    return t.to(dtype=F32).contiguous()


def _resolve_blocks(n: int, block_size: int) -> Tuple[Tuple[int, int], ...]:
    """reference :321-329."""
    if block_size <= 0:
        raise ValueError(f"block_size must be > 0, got {block_size}.")
    if n % block_size != 0:
        raise ValueError(f"n must be divisible by block_size; got n={n}, block_size={block_size}.")
    return tuple((s, s + block_size) for s in range(0, n, block_size))


class _BlockMeta:
    """Per-block gram, Cholesky factor, inverse (or diag inverse) and importance of one Vs."""

    def __init__(self, Vs: torch.Tensor, bs: int, metric: str) -> None:
        n, R = Vs.shape
        nb = n // bs
        dev = Vs.device
        self.gram_chol = metric == "gram"
        self.gram = torch.empty(nb, bs, bs, dtype=F32, device=dev)
        self.chol = torch.empty(nb, bs, bs, dtype=F32, device=dev) if self.gram_chol else None
        self.ginv = torch.empty(nb, bs, bs, dtype=F32, device=dev)
        self.importance = torch.empty(nb, dtype=F32, device=dev)
        status = torch.empty(nb, dtype=torch.int32, device=dev)
        _lib.call("mpq_bcd_prepare", n, R, bs, int(self.gram_chol), _lib.ptr(Vs), _lib.ptr(self.gram),
                  _lib.ptr(self.chol), _lib.ptr(self.ginv), _lib.ptr(self.importance), _lib.ptr(status),
                  _stream(Vs))
        if self.gram_chol and bool((status != 0).any().item()):
            bad = int((status != 0).nonzero()[0].item())
            raise RuntimeError(f"linalg.cholesky: the factorization of block {bad}'s gram could not be completed "
                               "after the diagonal jitter retries (the input is not positive-definite).")


def _stable_desc(values: torch.Tensor) -> list:
    vals = values.detach().to("cpu", torch.float64).tolist()
    return sorted(range(len(vals)), key=lambda i: -vals[i])


@torch.inference_mode()
def block_coordinate_descent_rankspace(
    *,
    x: torch.Tensor,  # (B, n)
    Y_u: torch.Tensor,  # (B, R)
    Vs: torch.Tensor,  # (n, R)
    block_size: int,
    provider: CandidateProvider,
    cfg: BlockCDConfig,
    idxs_init: Optional[torch.Tensor] = None,  # (B, n_blocks)
    snapshot_budgets: Optional[set] = None,
    snapshots_out: Optional[Dict[int, torch.Tensor]] = None,
    raw_target: Optional[torch.Tensor] = None,
    raw_gram: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, Optional[torch.Tensor], Dict[str, Any]]:
    """Generic rank-space block-coordinate polish (reference :332-625).

    Returns (x_new (B, n), idxs (provider-defined or None), stats with ``accepted_updates``,
    ``sweep_trace`` and ``stabilized_objective_nonincreasing``)."""
    sweeps = max(int(cfg.sweeps), 0)
    if sweeps <= 0 or x.numel() == 0 or Vs.numel() == 0:
        return x, idxs_init, {"accepted_updates": 0.0, "sweep_trace": [], "stabilized_objective_nonincreasing": True}
    metric = str(cfg.metric or "diag").strip().lower()
    if metric not in ("diag", "gram", "isotropic"):
        raise ValueError(f"unsupported metric={metric!r}; expected 'diag'|'gram'.")
    if metric == "isotropic":
        metric = "diag"
    order_mode = str(getattr(cfg, "order_mode", "greedy_gain") or "greedy_gain").strip().lower()
    if order_mode not in ("static", "cyclic", "greedy_gain"):
        raise ValueError(f"unsupported order_mode={order_mode!r}; expected 'static'|'cyclic'|'greedy_gain'.")
    if not x.is_cuda:
        raise ValueError(f"x must be on a ROCm device (got {x.device}); mpq_amd has no CPU path.")
    if (raw_target is None) != (raw_gram is None):
        raise ValueError("raw_target and raw_gram must be provided together.")
    B, n = x.shape
    bs = int(block_size)
    blocks = _resolve_blocks(n, bs)
    if bs > 16:
        raise ValueError(f"mpq_amd's block CD supports block_size <= 16, got {bs}.")
    nb = len(blocks)
    R = int(Vs.shape[1])
    if tuple(Vs.shape) != (n, R) or tuple(Y_u.shape) != (B, R):
        raise ValueError(f"shape mismatch: x {tuple(x.shape)}, Y_u {tuple(Y_u.shape)}, Vs {tuple(Vs.shape)}")
    if idxs_init is not None and tuple(idxs_init.shape) != (B, nb):
        raise ValueError(f"idxs_init must be (B, n_blocks) = {(B, nb)}, got {tuple(idxs_init.shape)}")
    accept_tol = max(float(cfg.accept_tol), 0.0)
    max_blocks = int(getattr(cfg, "max_blocks_per_sweep", 0) or 0)
    requested = {int(b) for b in (snapshot_budgets or set()) if 0 <= int(b) <= sweeps}
    Vs_f = _f32c(Vs)
    x_work = x.to(dtype=F32).clone().contiguous()

    def objective_mean(xv: torch.Tensor) -> float:
        d = (raw_target.to(device=xv.device, dtype=F32) - xv).contiguous()
        return float((ops.gemm(d, _f32c(raw_gram)) * d).sum(dim=1).mean().item())

    trace: list = []

    def trace_item(budget, swept, total, changes, res_norm, assignments_total):
        item: Dict[str, Any] = {
            "budget": int(budget),
            "stabilized_objective_mean": float(res_norm.mean().item()),
            "accepted_updates_sweep": int(swept),
            "accepted_updates_cumulative": int(total),
            "assignment_changes_from_cd0": int(changes),
            "assignments_total": int(assignments_total),
        }
        if raw_target is not None:
            item["raw_objective_mean"] = objective_mean(x_work)
        return item

    def snapshot(budget: int, idxs: Optional[torch.Tensor]) -> None:
        if snapshots_out is not None and idxs is not None and budget in requested:
            snapshots_out[budget] = idxs.detach().to(device="cpu").clone()

    def finish(total: int) -> Tuple[torch.Tensor, Optional[torch.Tensor], Dict[str, Any]]:
        objs = [float(t["stabilized_objective_mean"]) for t in trace]
        nonincreasing = all(a2 <= a1 + max(1e-8, abs(a1) * 1e-7) for a1, a2 in zip(objs, objs[1:]))
        return x_work.to(dtype=x.dtype), None, {"accepted_updates": float(total), "sweep_trace": trace,
                                                "stabilized_objective_nonincreasing": bool(nonincreasing)}

    # ---- fused case: scalar grid, greedy order (mpq_uniform_cd_sweeps_recip) ----------------------
    if (isinstance(provider, UniformScalarProvider) and bs == 1 and metric == "diag" and order_mode == "greedy_gain"
            and max_blocks == 0 and R == n and 1 <= int(provider.maxq) <= 255 and n <= 16384):
        scale_f = _f32c(provider.scale)
        zero_f = _f32c(provider.zero)
        if tuple(scale_f.shape) != (B, n) or tuple(zero_f.shape) != (B, n):
            raise ValueError("UniformScalarProvider scale/zero must be (B, n)")
        maxq = int(provider.maxq)
        residual = Y_u.to(F32) - ops.gemm(x_work, Vs_f)
        rhs = ops.gemm(residual, Vs_f, trans_b=True)
        res_norm = residual.square().sum(dim=1).contiguous()
        del residual
        diag = Vs_f.square().sum(dim=1).clamp_min_(1e-12).contiguous()
        gram = ops.gemm(Vs_f, Vs_f, trans_b=True)
        q0 = torch.round(x_work / scale_f.clamp_min(1e-12) + zero_f).clamp_(0, maxq).to(torch.int32)
        q = (idxs_init if idxs_init is not None else q0).to(torch.int32).clamp(0, 255).to(torch.uint8).contiguous()
        cd0 = q.clone()
        accepted = torch.zeros(B, dtype=torch.int32, device=x.device)
        out_dtype = idxs_init.dtype if idxs_init is not None else torch.int32
        snapshot(0, q.to(out_dtype))
        trace.append(trace_item(0, 0, 0, 0, res_norm, q.numel()))
        total = 0
        for sweep in range(1, sweeps + 1):
            ops.uniform_cd_sweeps(rhs, x_work, q, res_norm, accepted, scale_f, zero_f, 1, maxq, diag, gram,
                                  block_rows=B, sweeps=1, accept_tol=accept_tol, target_rule="recip")
            now = int(accepted.sum().item())
            trace.append(trace_item(sweep, now - total, now, int((q != cd0).sum().item()), res_norm, q.numel()))
            total = now
            snapshot(sweep, q.to(out_dtype))
        x_out, _, stats = finish(total)
        return x_out, q.to(out_dtype), stats

    # ---- fused case: E8P12 codebook, gram metric, greedy order (mpq_e8p12_cd_polish) --------------
    if (type(provider) is E8P12Provider and bs == 8 and metric == "gram" and order_mode == "greedy_gain"
            and R == n and _standin_ok(provider.cb)):
        from ..solver import _e8p12_cd_context

        ctx = _e8p12_cd_context(Vs_f)
        idx = (idxs_init.to(I64).contiguous() if idxs_init is not None
               else provider.cb.quantize(x_work.view(B, nb, 8))[1].reshape(B, nb).to(I64).contiguous())
        cd0 = idx.clone()
        Yu_f = _f32c(Y_u)
        res_norm = (Yu_f - ops.gemm(x_work, Vs_f)).square().sum(dim=1)
        out_dtype = idxs_init.dtype if idxs_init is not None else getattr(provider.cb, "idx_dtype", None) or I64
        snapshot(0, idx.to(out_dtype))
        trace.append(trace_item(0, 0, 0, 0, res_norm, idx.numel()))
        total = 0
        for sweep in range(1, sweeps + 1):
            xn, idxn, _, ea, acc = ops.e8p12_cd_polish(x_work, idx, Vs_f, ctx, sweeps=1, block_rows=B, Yu=Yu_f,
                                                       max_blocks=max_blocks, accept_tol=accept_tol)
            x_work.copy_(xn)
            idx = idxn
            now = total + int(acc.sum().item())
            trace.append(trace_item(sweep, now - total, now, int((idx != cd0).sum().item()), ea, idx.numel()))
            total = now
            snapshot(sweep, idx.to(out_dtype))
        x_out, _, stats = finish(total)
        return x_out, idx.to(out_dtype), stats

    # ---- generic loop ------------------------------------------------------------------------------
    meta = _BlockMeta(Vs_f, bs, metric)
    residual_u = _f32c(Y_u).clone()
    ops.gemm(x_work, Vs_f, out=residual_u, alpha=-1.0, beta=1.0)
    res_norm = residual_u.square().sum(dim=1).contiguous()
    static_order = _stable_desc(meta.importance)
    cyclic_order = list(range(nb))
    idxs_out: Optional[torch.Tensor] = idxs_init.to(I64).contiguous().clone() if idxs_init is not None else None
    out_dtype = idxs_init.dtype if idxs_init is not None else None
    idxs_cd0 = idxs_out.clone() if idxs_out is not None else None
    accepted = torch.zeros(B, dtype=torch.int32, device=x.device)
    delta = torch.empty(B, bs, dtype=F32, device=x.device)
    target = torch.empty(B, bs, dtype=F32, device=x.device)
    stream = _stream(x_work)
    snapshot(0, idxs_out if out_dtype is None else idxs_out.to(out_dtype))
    trace.append(trace_item(0, 0, 0, 0, res_norm, idxs_out.numel() if idxs_out is not None else 0))
    total = 0
    for sweep in range(1, sweeps + 1):
        if order_mode == "greedy_gain":
            rhs_all = ops.gemm(residual_u, Vs_f, trans_b=True)
            gain = torch.empty(nb, dtype=F32, device=x.device)
            _lib.call("mpq_bcd_gain", B, n, bs, int(meta.gram_chol), _lib.ptr(rhs_all), _lib.ptr(meta.ginv),
                      _lib.ptr(gain), stream)
            del rhs_all
            order = _stable_desc(gain)
        elif order_mode == "cyclic":
            order = list(cyclic_order)
        else:
            order = list(static_order)
        if max_blocks > 0:
            order = order[:max_blocks]
        for bi in order:
            start, end = blocks[bi]
            Vs_blk = Vs_f[start:end]
            rhs = ops.gemm(residual_u, Vs_blk, trans_b=True)
            _lib.call("mpq_bcd_target", B, n, bs, bi, int(meta.gram_chol), _lib.ptr(x_work), _lib.ptr(rhs),
                      _lib.ptr(meta.ginv), _lib.ptr(target), stream)
            cand_vals, cand_idxs = provider.propose(block_idx=bi, start=start, end=end, x_block=x_work[:, start:end],
                                                    target=target, metric=metric,
                                                    gram_chol=meta.chol[bi] if meta.gram_chol else None)
            cand_vals = _f32c(cand_vals).reshape(B, bs)
            ci = None
            if cand_idxs is not None:
                if out_dtype is None:
                    out_dtype = cand_idxs.dtype
                ci = cand_idxs.to(device=x.device, dtype=I64).reshape(B).contiguous()
                if idxs_out is None:
                    idxs_out = torch.full((B, nb), -1, dtype=I64, device=x.device)
            _lib.call("mpq_bcd_accept", B, n, bs, bi, _lib.ptr(cand_vals), _lib.ptr(rhs), _lib.ptr(meta.gram),
                      float(accept_tol), _lib.ptr(ci), _lib.ptr(x_work), _lib.ptr(res_norm), _lib.ptr(idxs_out),
                      _lib.ptr(accepted), _lib.ptr(delta), stream)
            ops.gemm(delta, Vs_blk, out=residual_u, alpha=-1.0, beta=1.0)
        now = int(accepted.sum().item())
        changes = (int((idxs_out != idxs_cd0).sum().item())
                   if idxs_out is not None and idxs_cd0 is not None else 0)
        trace.append(trace_item(sweep, now - total, now, changes, res_norm,
                                idxs_out.numel() if idxs_out is not None else 0))
        total = now
        snapshot(sweep, idxs_out if idxs_out is None or out_dtype is None else idxs_out.to(out_dtype))
    x_out, _, stats = finish(total)
    if idxs_out is not None and out_dtype is not None:
        idxs_out = idxs_out.to(out_dtype)
    return x_out, idxs_out, stats


def _standin_ok(cb: Any) -> bool:
    try:
        require_standin_table(cb, "block_coordinate_descent_rankspace")
        return True
    except ValueError:
        return False


# ---- providers ----------------------------------------------------------------------------------

@dataclass(frozen=True)
class UniformScalarProvider:
    scale: torch.Tensor  # (B, n)
    zero: torch.Tensor  # (B, n)
    maxq: int

    @torch.inference_mode()
    def propose(self, *, block_idx: int, start: int, end: int, x_block: torch.Tensor, target: torch.Tensor,
                metric: str, gram_chol: Optional[torch.Tensor]) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
        del block_idx, metric, gram_chol
        if end != start + 1:
            raise ValueError("UniformScalarProvider expects block_size=1.")
        B = int(target.shape[0])
        scale, zero = _f32c(self.scale), _f32c(self.zero)
        n = int(scale.shape[1])
        t = _f32c(target).reshape(B)
        vals = torch.empty(B, 1, dtype=F32, device=t.device)
        q = torch.empty(B, dtype=I64, device=t.device)
        _lib.call("mpq_bcd_uniform_propose", B, n, int(start), int(self.maxq), _lib.ptr(t), _lib.ptr(scale),
                  _lib.ptr(zero), _lib.ptr(vals), _lib.ptr(q), _stream(t))
        return vals.to(dtype=x_block.dtype), q.to(torch.int32)


@dataclass(frozen=True)
class UniformTopKProvider:
    topk_values: torch.Tensor  # (B, n, k)
    topk_q: Optional[torch.Tensor] = None  # (B, n, k)

    @torch.inference_mode()
    def propose(self, *, block_idx: int, start: int, end: int, x_block: torch.Tensor, target: torch.Tensor,
                metric: str, gram_chol: Optional[torch.Tensor]) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
        del block_idx, metric, gram_chol
        if end != start + 1:
            raise ValueError("UniformTopKProvider expects block_size=1.")
        dev = x_block.device
        vals_k = self.topk_values.to(device=dev, dtype=F32).contiguous()
        B, n, k = (int(s) for s in vals_k.shape)
        qk = None if self.topk_q is None else self.topk_q.to(device=dev, dtype=I64).contiguous()
        t = _f32c(target).reshape(B)
        vals = torch.empty(B, 1, dtype=F32, device=dev)
        q = torch.empty(B, dtype=I64, device=dev) if qk is not None else None
        _lib.call("mpq_bcd_topk_scalar_propose", B, n, int(start), k, _lib.ptr(t), _lib.ptr(vals_k), _lib.ptr(qk),
                  _lib.ptr(vals), _lib.ptr(q), _stream(t))
        return vals.to(dtype=x_block.dtype), (None if q is None else q.to(torch.int32))


@dataclass
class E8P12Provider:
    cb: object
    metric_rows_per_chunk: int = 0

    @torch.inference_mode()
    def propose(self, *, block_idx: int, start: int, end: int, x_block: torch.Tensor, target: torch.Tensor,
                metric: str, gram_chol: Optional[torch.Tensor]) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
        del block_idx
        if (end - start) != int(getattr(self.cb, "codesz", 8)):
            raise ValueError("E8P12Provider expects block_size=codesz.")
        if metric == "gram":
            if gram_chol is None:
                raise ValueError("metric='gram' requires gram_chol.")
            require_standin_table(self.cb, "E8P12Provider")
            t = _f32c(target)
            rows = int(t.shape[0])
            vals = torch.empty(rows, 8, dtype=F32, device=t.device)
            idx = torch.empty(rows, dtype=I64, device=t.device)
            ws = ops.workspace(int(_lib.load().mpq_e8p12_metric_argmin_workspace_size(rows)), t.device)
            _lib.call("mpq_e8p12_metric_argmin", rows, _lib.ptr(t), _lib.ptr(_f32c(gram_chol)), _lib.ptr(vals),
                      _lib.ptr(idx), _lib.ptr(ws), int(ws.numel()), _stream(t))
            return vals.to(dtype=x_block.dtype), idx.to(dtype=getattr(self.cb, "idx_dtype", None) or I64)
        if not hasattr(self.cb, "quantize"):
            raise ValueError("cb.quantize is required for isotropic polish.")
        cand_vals, cand_idxs = self.cb.quantize(target, resid_scale_override=-1)
        return cand_vals.to(dtype=x_block.dtype), cand_idxs


@dataclass
class E8P12TopKProvider:
    cb: object
    topk_idxs: torch.Tensor  # (rows, nblocks, k)

    @torch.inference_mode()
    def propose(self, *, block_idx: int, start: int, end: int, x_block: torch.Tensor, target: torch.Tensor,
                metric: str, gram_chol: Optional[torch.Tensor]) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
        codesz = int(getattr(self.cb, "codesz", 8))
        if int(end - start) != codesz:
            raise ValueError(f"E8P12TopKProvider expects block_size={codesz}, got {int(end - start)}.")
        if metric == "gram" and gram_chol is None:
            raise ValueError("metric='gram' requires gram_chol.")
        require_standin_table(self.cb, "E8P12TopKProvider")
        dev = x_block.device
        tk = self.topk_idxs.to(device=dev, dtype=I64).contiguous()
        rows, nb, k = (int(s) for s in tk.shape)
        t = _f32c(target)
        vals = torch.empty(rows, 8, dtype=F32, device=dev)
        idx = torch.empty(rows, dtype=I64, device=dev)
        chol = _f32c(gram_chol) if metric == "gram" else None
        _lib.call("mpq_bcd_e8_topk_propose", rows, nb, int(block_idx), k, _lib.ptr(tk), _lib.ptr(t), _lib.ptr(chol),
                  _lib.ptr(vals), _lib.ptr(idx), _stream(t))
        return vals.to(dtype=x_block.dtype), idx.to(dtype=getattr(self.cb, "idx_dtype", None) or I64)
