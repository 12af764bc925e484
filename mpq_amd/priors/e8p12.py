"""E8P12 lattice prior: MAP search and posterior on the HIP kernels.

Drop-in for ``mpq/priors/e8p12.py``:

* ``vamp_vector_map_e8p12``  -> ``mpq_e8p12_map``  (reference ``:541-631``)
* ``vamp_vector_discrete_mmse_e8p12`` -> ``mpq_e8p12_denoise`` (reference ``:815-968``)
* ``e8p12_nearest``          -> ``mpq_e8p12_map`` with unit precision, no prior
  (the codebook's exact nearest-codeword quantizer)
* ``prior_scale_from_center``  (reference ``:45-61``)

Tensors must live on a ROCm device; there is no CPU path in the product.
"""
from __future__ import annotations

from typing import Dict, Optional, Tuple

import torch

from .. import _lib


def _require_device(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be on a ROCm device (got {t.device}); mpq_amd has no CPU path.")


@torch.inference_mode()
def prior_scale_from_center(prior_center_blocks: Optional[torch.Tensor], mode: str) -> Optional[torch.Tensor]:
    """Per-block prior scale (reference ``mpq/priors/e8p12.py:45-61``)."""
    if prior_center_blocks is None:
        return None
    mode = str(mode or "absmax").strip().lower()
    if mode in ("none", "unit", "legacy"):
        shape = prior_center_blocks.shape[:-1] + (1,)
        return torch.ones(shape, dtype=torch.float32, device=prior_center_blocks.device)
    if mode in ("absmax", "exact_full", "exact_full_absmax"):
        scale = prior_center_blocks.abs().amax(dim=-1, keepdim=True)
    elif mode in ("rms", "std"):
        scale = prior_center_blocks.square().mean(dim=-1, keepdim=True).sqrt()
    elif mode in ("mean_abs", "l1"):
        scale = prior_center_blocks.abs().mean(dim=-1, keepdim=True)
    else:
        raise ValueError(f"unsupported prior_tau_scale_mode={mode!r}; supported: none|absmax|rms|mean_abs")
    return scale.to(dtype=torch.float32).clamp_min_(1e-12)


@torch.inference_mode()
def e8p12_map_flat(
    r: torch.Tensor,  # (N, 8) fp32
    gamma: torch.Tensor,  # (N // gamma_div,) fp32
    *,
    gamma_div: int = 1,
    center: Optional[torch.Tensor] = None,  # (N, 8)
    scale: Optional[torch.Tensor] = None,  # (N,) or None for in-kernel absmax
    tau: float = 0.0,
    want_idx64: bool = True,
    want_idx16: bool = False,
    want_vals: bool = False,
    want_err: bool = False,
    want_score: bool = False,
) -> Dict[str, torch.Tensor]:
    """Low-level launcher of ``mpq_e8p12_map`` on flat (N, 8) blocks."""
    _require_device(r, "r")
    if r.dim() != 2 or int(r.shape[1]) != 8:
        raise ValueError(f"expected r with shape (N, 8), got {tuple(r.shape)}")
    r = r.to(dtype=torch.float32).contiguous()
    n = int(r.shape[0])
    gamma = gamma.to(device=r.device, dtype=torch.float32).contiguous().reshape(-1)
    if n and int(gamma.numel()) * int(gamma_div) < n:
        raise ValueError(f"gamma has {gamma.numel()} entries for {n} vectors with gamma_div={gamma_div}")
    use_prior = center is not None and float(tau) > 0.0
    if use_prior:
        center = center.to(device=r.device, dtype=torch.float32).contiguous()
        if tuple(center.shape) != tuple(r.shape):
            raise ValueError("prior center must match r in shape")
        if scale is not None:
            scale = scale.to(device=r.device, dtype=torch.float32).contiguous().reshape(-1)
            if int(scale.numel()) != n:
                raise ValueError("prior scale must have one entry per vector")
    else:
        center = None
        scale = None
    out: Dict[str, torch.Tensor] = {}
    dev = r.device
    if want_idx64:
        out["idx"] = torch.empty(n, dtype=torch.int64, device=dev)
    if want_idx16:
        out["idx16"] = torch.empty(n, dtype=torch.uint16, device=dev)
    if want_vals:
        out["vals"] = torch.empty(n, 8, dtype=torch.float32, device=dev)
    if want_err:
        out["err"] = torch.empty(n, dtype=torch.float32, device=dev)
    if want_score:
        out["score"] = torch.empty(n, dtype=torch.float32, device=dev)
    if n == 0:
        return out
    _lib.call(
        "mpq_e8p12_map",
        _lib.ptr(r), n, _lib.ptr(gamma), int(gamma_div),
        _lib.ptr(center), _lib.ptr(scale), float(tau) if use_prior else 0.0,
        _lib.ptr(out.get("idx")), _lib.ptr(out.get("idx16")), _lib.ptr(out.get("vals")),
        _lib.ptr(out.get("err")), _lib.ptr(out.get("score")),
        _lib.stream_handle(dev),
    )
    return out


@torch.inference_mode()
def posterior_stats(r_flat: torch.Tensor, rows: int, n_blocks: int, gamma1: torch.Tensor, *,
                    center: Optional[torch.Tensor], scale: Optional[torch.Tensor], tau: float,
                    want_logz: bool = True, want_entropy: bool = True, want_margin: bool = True
                    ) -> Dict[str, Optional[torch.Tensor]]:
    """Per-block posterior diagnostics (``mpq_e8p12_posterior_stats``): logZ, entropy, margin,
    each (rows, n_blocks) fp32 or None when not requested."""
    dev = r_flat.device
    out: Dict[str, Optional[torch.Tensor]] = {}
    for key, want in (("logz", want_logz), ("entropy", want_entropy), ("margin", want_margin)):
        out[key] = torch.empty(rows, n_blocks, dtype=torch.float32, device=dev) if want else None
    if rows * n_blocks:
        _lib.call("mpq_e8p12_posterior_stats", _lib.ptr(r_flat.to(torch.float32).contiguous()), int(rows),
                  int(n_blocks), _lib.ptr(gamma1.to(device=dev, dtype=torch.float32).contiguous()),
                  _lib.ptr(None if center is None else center.to(device=dev, dtype=torch.float32).contiguous()),
                  _lib.ptr(None if scale is None else scale.to(device=dev, dtype=torch.float32).contiguous()),
                  float(tau), _lib.ptr(out["logz"]), _lib.ptr(out["entropy"]), _lib.ptr(out["margin"]),
                  _lib.stream_handle(dev))
    return out


@torch.inference_mode()
def e8p12_nearest(x: torch.Tensor, *, return_vals: bool = False) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Exact nearest E8P12 codeword of each row of ``x`` (N, 8); first index on ties."""
    _require_device(x, "x")
    one = torch.ones(1, dtype=torch.float32, device=x.device)
    out = e8p12_map_flat(x, one, gamma_div=max(int(x.shape[0]), 1), want_vals=return_vals)
    return out["idx"], out.get("vals")


@torch.inference_mode()
def vamp_vector_map_e8p12(
    *,
    r1_blocks: torch.Tensor,  # (B, n_blocks, 8)
    gamma1: torch.Tensor,  # (B, 1)
    cb: object,
    blocks_per_chunk: int = 64,
    need_stats: bool = False,
    prior_center_blocks: Optional[torch.Tensor] = None,
    prior_scale_blocks: Optional[torch.Tensor] = None,
    prior_tau: float = 0.0,
    prior_tau_scale_mode: str = "absmax",
) -> Dict[str, torch.Tensor | float]:
    """Factorized E8P12 MAP per 8-block (reference ``mpq/priors/e8p12.py:541-631``).

    ``blocks_per_chunk`` is accepted for signature compatibility; the kernel has no chunking.
    ``need_stats`` adds ``margin``, the mean over all blocks of the gap between the two largest
    candidate log-scores (the reference averages per chunk of blocks).
    """
    del blocks_per_chunk, cb
    batch, n_blocks, codesz = r1_blocks.shape
    if int(codesz) != 8:
        raise ValueError(f"E8P12 MAP expects codesz=8, got {codesz}.")
    if gamma1.ndim != 2 or int(gamma1.shape[-1]) != 1 or int(gamma1.shape[0]) != int(batch):
        raise ValueError(f"expected scalar gamma1 with shape (B,1), got {tuple(gamma1.shape)}")
    center = None
    scale = None
    tau = 0.0
    if float(prior_tau) > 0.0 and prior_center_blocks is not None:
        center = prior_center_blocks.reshape(-1, 8)
        tau = float(prior_tau)
        mode = str(prior_tau_scale_mode or "absmax").strip().lower()
        if prior_scale_blocks is not None:
            scale = prior_scale_blocks.reshape(-1)
        elif mode not in ("absmax", "exact_full", "exact_full_absmax"):
            scale = prior_scale_from_center(prior_center_blocks, mode).reshape(-1)
    out = e8p12_map_flat(
        r1_blocks.reshape(-1, 8), gamma1.reshape(-1), gamma_div=max(int(n_blocks), 1),
        center=center, scale=scale, tau=tau, want_vals=True,
    )
    if need_stats:
        st = posterior_stats(r1_blocks.reshape(-1, 8), int(batch), int(n_blocks), gamma1, center=center,
                             scale=scale, tau=tau, want_logz=False, want_entropy=False)
        return {
            "map_idxs": out["idx"].view(batch, n_blocks),
            "map_vals": out["vals"].view(batch, n_blocks, 8).to(dtype=r1_blocks.dtype),
            "margin": float(st["margin"].double().mean().item()) if st["margin"].numel() else 0.0,
        }
    return {
        "map_idxs": out["idx"].view(batch, n_blocks),
        "map_vals": out["vals"].view(batch, n_blocks, 8).to(dtype=r1_blocks.dtype),
    }


@torch.inference_mode()
def vamp_vector_discrete_mmse_e8p12(
    *,
    r1_blocks: torch.Tensor,  # (B, n_blocks, 8)
    gamma1: torch.Tensor,  # (B, 1)
    cb: object,
    blocks_per_chunk: int = 16,
    need_stats: bool = False,
    prior_center_blocks: Optional[torch.Tensor] = None,
    prior_scale_blocks: Optional[torch.Tensor] = None,
    prior_tau: float = 0.0,
    prior_tau_scale_mode: str = "absmax",
    compile_prior: bool = True,
    return_logZ_blocks: bool = False,
    return_margin_blocks: bool = False,
    return_entropy_blocks: bool = False,
) -> Dict[str, torch.Tensor | float]:
    """Posterior mean/variance over the 2^16 codewords (reference ``mpq/priors/e8p12.py:815-968``).

    Returns ``x1_blocks`` (B, n_blocks, 8), ``var1`` (B, n_blocks), ``alpha1`` (B, 1),
    ``map_idxs`` (B, n_blocks), ``map_vals`` (B, n_blocks, 8), ``entropy`` and ``margin`` (means over
    all blocks when ``need_stats`` or a per-block diagnostic is requested, else 0.0; the reference
    averages per chunk of blocks) and, on request, ``logZ_blocks``, ``margin_blocks`` and
    ``entropy_blocks`` (B, n_blocks).  ``blocks_per_chunk`` and ``compile_prior`` are accepted for
    signature compatibility (the kernel streams all blocks in one launch).
    """
    del blocks_per_chunk, cb, compile_prior
    need_stats = bool(need_stats) or bool(return_margin_blocks) or bool(return_entropy_blocks)
    _require_device(r1_blocks, "r1_blocks")
    batch, n_blocks, codesz = r1_blocks.shape
    if int(codesz) != 8:
        raise ValueError(f"E8P12 posterior expects codesz=8, got {codesz}.")
    if gamma1.ndim != 2 or int(gamma1.shape[-1]) != 1 or int(gamma1.shape[0]) != int(batch):
        raise ValueError(f"expected scalar gamma1 with shape (B,1), got {tuple(gamma1.shape)}")
    dev = r1_blocks.device
    r = r1_blocks.to(dtype=torch.float32).contiguous()
    g = gamma1.to(device=dev, dtype=torch.float32).contiguous()
    center = None
    scale = None
    tau = 0.0
    if float(prior_tau) > 0.0 and prior_center_blocks is not None:
        center = prior_center_blocks.to(device=dev, dtype=torch.float32).reshape(-1, 8).contiguous()
        tau = float(prior_tau)
        mode = str(prior_tau_scale_mode or "absmax").strip().lower()
        if prior_scale_blocks is not None:
            scale = prior_scale_blocks.to(device=dev, dtype=torch.float32).reshape(-1).contiguous()
        elif mode not in ("absmax", "exact_full", "exact_full_absmax"):
            scale = prior_scale_from_center(prior_center_blocks, mode).reshape(-1).contiguous()
    nblk = int(batch) * int(n_blocks)
    x1 = torch.empty(batch, n_blocks, 8, dtype=torch.float32, device=dev)
    var = torch.empty(batch, n_blocks, dtype=torch.float32, device=dev)
    idx = torch.empty(batch, n_blocks, dtype=torch.int64, device=dev)
    vals = torch.empty(batch, n_blocks, 8, dtype=torch.float32, device=dev)
    alpha1 = torch.empty(batch, 1, dtype=torch.float32, device=dev)
    if nblk:
        _lib.call(
            "mpq_e8p12_denoise",
            _lib.ptr(r), int(batch), int(n_blocks), _lib.ptr(g), _lib.ptr(center), _lib.ptr(scale), float(tau),
            _lib.ptr(x1), _lib.ptr(var), _lib.ptr(idx), _lib.ptr(vals), _lib.ptr(alpha1),
            _lib.stream_handle(dev),
        )
    out: Dict[str, torch.Tensor | float] = {"x1_blocks": x1, "var1": var, "alpha1": alpha1, "map_idxs": idx,
                                            "map_vals": vals, "entropy": 0.0, "margin": 0.0}
    if need_stats or return_logZ_blocks:
        st = posterior_stats(r, int(batch), int(n_blocks), g, center=center, scale=scale, tau=tau,
                             want_logz=bool(return_logZ_blocks), want_entropy=need_stats, want_margin=need_stats)
        if need_stats:
            out["entropy"] = float(st["entropy"].double().mean().item()) if nblk else 0.0
            out["margin"] = float(st["margin"].double().mean().item()) if nblk else 0.0
        if return_logZ_blocks:
            out["logZ_blocks"] = st["logz"]
        if return_margin_blocks:
            out["margin_blocks"] = st["margin"]
        if return_entropy_blocks:
            out["entropy_blocks"] = st["entropy"]
    return out
