"""QUIP# checkpoint writer of the E8P12 path: the both-sided randomized Hadamard transform (RHT) around
``mpq_refine_codebook`` and the per-layer ``{idx}_{name}.pt`` dicts of a QUIP# ``ckpt/`` directory.

Reference (the QUIP# hook and MPQ's own QUIP# orchestration):

* ``rht_h`` / ``rht_w``           ``patches/quip_sharp.patch:211-218`` (RHT_H, RHT_W without structured
                                  states: the ``incoh_mode="had"`` path)
* ``incoherence_preprocess``      ``patches/quip_sharp.patch:221-330`` (``had``: signs SU, SV, then RHT)
* ``incoherence_process``         ``patches/quip_sharp.patch:340-375`` (inverse transform, ``had``)
* ``quantize_weights_to_attr``    ``mpq/quip_generic.py:356-422`` with the quantize step of
                                  ``patches/quip_sharp.patch:374-470`` (solver ``mpq``)
* ``save_quantized_attr``         ``mpq/quip_generic.py:425-426``; file names ``{idx}_{name}.pt``
                                  (``mpq/quip_generic.py:628``)
* ``decompress_saved_quip`` / ``load_split_weights``   ``mpq/quip_generic.py:737-767``

The Hadamard products run on the HIP block-Hadamard kernel (``mpq_block_hadamard``).  A power-of-two
width uses one Sylvester transform over the full width, which is what quip-sharp's ``matmul_hadU``
computes for such widths (and its transpose, ``matmul_hadUt``, is the same symmetric transform).  Other
widths (a fused qkv of 3072 rows, 14336 columns) are where the two differ: quip-sharp transforms them
with its had-K factors (``matmul_hadU`` with a 12- or 28-point factor), which live only in the
un-vendored quip-sharp, and the reference's loader (``_decompress_saved_quip`` ->
``incoherence_process`` -> ``_hadU_or_block``, ``patches/quip_sharp.patch:171-185``) tries that
transform first.  Such widths therefore raise ``ValueError`` unless the caller passes
``allow_block_hadamard=True``; the writer then uses blocks of the largest power-of-two factor (the
patch's own fallback) and records it as ``rotation_family="block_had"`` with the block sizes
(``left_had_dim`` / ``right_had_dim``), which ``decompress_saved_quip`` here reads back; quip-sharp's
loader does not, so such a checkpoint is only for this build's decoder.

Steps that live only in the un-vendored quip-sharp@1d8f873e are restated from its published algorithm
and are parity unpinned: the Hessian regularisation (``H / mean(diag H) + sigma_reg I``), the weight
scale ``Wscale = rms(Wr) / opt_scale`` (``scale_override`` when positive) that is fused into ``SV``,
LDLQ (replaced here by the codebook's nearest-codeword start, ``mpq_init="rtn"``), QUIP#'s own
Hadamard factors for widths that are not powers of two, and ``maybe_pack_idxs`` (this build's codebook
keeps indices unpacked: ``E8P12_codebook.maybe_pack_idxs`` is the identity).
"""
from __future__ import annotations

import hashlib
import os
from typing import Any, Dict, List, Optional, Sequence, Tuple

import torch

from . import ops
from .adapters.quip_sharp import mpq_refine_codebook
from .codebook import require_standin_table


def hadamard_plan(width: int, allow_block: bool = False) -> Tuple[int, str]:
    """(transform width, fallback reason): the full width when it is a power of two; other widths raise
    ``ValueError`` unless ``allow_block`` (then blocks of the largest power-of-two factor)."""
    w = int(width)
    if w <= 0:
        raise ValueError(f"width must be positive, got {w}")
    had = w & -w
    if had == w:
        return w, ""
    if not allow_block:
        raise ValueError(
            f"width={w} is not a power of two: quip-sharp transforms it with its had-K factors (matmul_hadU), "
            f"which this build does not provide; pass allow_block_hadamard=True for a block Hadamard of {had} "
            "(rotation_family 'block_had', read by this build's decoder only)")
    return had, f"width={w} is not a power of two: block Hadamard of {had}"


def _had_rows(X: torch.Tensor, signs: Optional[torch.Tensor], had: int, inverse: bool = False) -> torch.Tensor:
    return ops.block_hadamard(X.contiguous(), int(had), signs=signs, inverse=inverse)


def rht_h(H: torch.Tensor, SU: torch.Tensor, allow_block: bool = False) -> torch.Tensor:
    """``hadUt(hadUt(H * SU).T * SU)`` (patches/quip_sharp.patch:211-212)."""
    had, _ = hadamard_plan(H.shape[-1], allow_block)
    A = _had_rows(H, SU, had)  # Had applied to the rows of H diag(SU)
    return _had_rows(ops.transpose(A), SU, had)


def rht_w(W: torch.Tensor, SU: torch.Tensor, SV: torch.Tensor, allow_block: bool = False) -> torch.Tensor:
    """``hadUt((SV[:, None] * hadUt(W * SU)).T).T`` (patches/quip_sharp.patch:215-218)."""
    had_n, _ = hadamard_plan(W.shape[1], allow_block)
    had_m, _ = hadamard_plan(W.shape[0], allow_block)
    A = _had_rows(W, SU, had_n)
    return ops.transpose(_had_rows(ops.transpose(A), SV, had_m))


def incoherence_process(hatWr: torch.Tensor, SU: torch.Tensor, SV: torch.Tensor, allow_block: bool = False, *,
                        had_dims: Optional[Tuple[int, int]] = None) -> torch.Tensor:
    """``(hadU((hadU(hatWr) * SU).T) * SV).T`` (patches/quip_sharp.patch:347-350): the inverse RHT;
    ``SV`` may carry the fused weight scale.  ``had_dims`` = (left, right) block sizes as recorded in a
    checkpoint (default: :func:`hadamard_plan` of each width)."""
    m, n = hatWr.shape
    if had_dims is None:
        had_dims = (hadamard_plan(m, allow_block)[0], hadamard_plan(n, allow_block)[0])
    had_m, had_n = (int(h) for h in had_dims)
    A = _had_rows(hatWr.to(torch.float32), SU.to(device=hatWr.device, dtype=torch.float32), had_n, inverse=True)
    return ops.transpose(_had_rows(ops.transpose(A), SV.to(device=hatWr.device, dtype=torch.float32), had_m,
                                   inverse=True))


def rht_signs(n: int, m: int, device) -> Tuple[torch.Tensor, torch.Tensor]:
    """``SU``, ``SV`` as the reference draws them (patches/quip_sharp.patch:252-253), from the caller's
    generator state."""
    SU = (torch.randn(int(n), device=device).sign() + 1e-5).sign().to(torch.float32)
    SV = (torch.randn(int(m), device=device).sign() + 1e-5).sign().to(torch.float32)
    return SU, SV


def incoherence_preprocess(H: torch.Tensor, W: torch.Tensor, SU: torch.Tensor, SV: torch.Tensor,
                           allow_block: bool = False) -> Tuple[torch.Tensor, torch.Tensor, str, str]:
    """RHT of H and W for ``incoh_mode="had"``: returns (Hr, Wr, left fallback reason, right fallback
    reason) (patches/quip_sharp.patch:221-330; the equilibration and structured modes are not
    provided).  Widths that are not powers of two need ``allow_block`` (see :func:`hadamard_plan`)."""
    m, n = W.shape
    if tuple(H.shape) != (n, n):
        raise ValueError(f"H must be {n} x {n}, got {tuple(H.shape)}")
    left_reason = hadamard_plan(m, allow_block)[1]
    right_reason = hadamard_plan(n, allow_block)[1]
    Hr = rht_h(H.to(torch.float32).contiguous(), SU, allow_block)
    Wr = rht_w(W.to(torch.float32).contiguous(), SU, SV, allow_block)
    return Hr, Wr, left_reason, right_reason


def regularize_h(H: torch.Tensor, sigma_reg: float) -> torch.Tensor:
    """quip-sharp's ``utils.regularize_H`` (un-vendored; parity unpinned): ``H / mean(diag H) + sigma I``."""
    H = H.to(torch.float32) / torch.diagonal(H).mean()
    idx = torch.arange(H.shape[0], device=H.device)
    H[idx, idx] += float(sigma_reg)
    return H


def tensor_sha256(t: torch.Tensor) -> str:
    return hashlib.sha256(t.detach().to("cpu").contiguous().numpy().tobytes(order="C")).hexdigest()


def _local_seed(save_name: str, base_seed: int) -> int:
    digest = hashlib.sha256(str(save_name).encode("utf-8")).digest()
    return int((int(base_seed) + int.from_bytes(digest[:8], byteorder="little", signed=False)) % (2 ** 31 - 1))


@torch.inference_mode()
def quantize_weights_to_attr(*, weights: Sequence[torch.Tensor], H: torch.Tensor, cb: Any, args: Any,
                             save_name: str, device=None,
                             allow_block_hadamard: bool = False) -> Tuple[Dict[str, Any], float, float, torch.Tensor]:
    """One (fused) linear to its QUIP# ckpt dict (mpq/quip_generic.py:356-422 with the ``mpq`` solver of
    patches/quip_sharp.patch:583-601).  ``weights`` are the fused pieces (q, k, v or up, gate, or one
    weight); ``H`` is the regularised input Hessian.  Returns (attr, relative Frobenius error, relative
    proxy error, hatW in the fused original basis).  A width that is not a power of two raises
    ``ValueError`` unless ``allow_block_hadamard`` (see :func:`hadamard_plan`)."""
    if bool(getattr(args, "use_fp64", False)):
        raise ValueError("mpq_amd's RHT runs in fp32 (use_fp64 is not provided).")
    if str(getattr(args, "incoh_mode", "had") or "had").strip().lower() != "had":
        raise ValueError("mpq_amd implements incoh_mode='had'.")
    if bool(getattr(args, "rescale_WH", False)) or str(getattr(args, "quant_preprocess", "none")) == "equil":
        raise ValueError("mpq_amd does not provide the W/H equilibration preprocess.")
    if int(getattr(args, "lora_rank", 0) or 0) > 0:
        raise ValueError("mpq_amd does not provide the low-rank (lora_rank > 0) QUIP# path.")
    require_standin_table(cb, "quantize_weights_to_attr")
    dev = torch.device(device) if device is not None else torch.device("cuda")
    shapes = [tuple(w.shape) for w in weights]
    scales = [w.to(dev, torch.float32).square().mean().sqrt() for w in weights]
    W = torch.vstack([w.to(dev, torch.float32) / s for w, s in zip(weights, scales)]).contiguous()
    H = H.to(dev, torch.float32).contiguous()
    m, n = W.shape
    if n % 8:
        raise ValueError(f"E8P12 needs n divisible by 8, got n={n}")
    had_m, _ = hadamard_plan(m, allow_block_hadamard)
    had_n, _ = hadamard_plan(n, allow_block_hadamard)

    # signs from a per-projection seed (mpq/quip_generic.py:381-394), generator state restored after
    cpu_state = torch.random.get_rng_state()
    dev_state = torch.cuda.get_rng_state(dev)
    try:
        seed = _local_seed(save_name, int(getattr(args, "seed", 0) or 0))
        torch.manual_seed(seed)
        torch.cuda.manual_seed_all(seed)
        SU, SV = rht_signs(n, m, dev)
    finally:
        torch.random.set_rng_state(cpu_state)
        torch.cuda.set_rng_state(dev_state, dev)
    Hr, Wr, left_reason, right_reason = incoherence_preprocess(H, W, SU, SV, allow_block_hadamard)

    # weight scale fused into SV (quip-sharp quantize, un-vendored)
    opt_scale = float(getattr(args, "scale_override", 0.0) or 0.0)
    if opt_scale <= 0.0:
        opt_scale = float(getattr(cb, "opt_scale", 1.0))
    Wscale = Wr.square().mean().sqrt() / opt_scale
    Wr_s = (Wr / Wscale).contiguous()

    # LDLQ start (un-vendored): the codebook's nearest codewords
    hat0, idx0 = cb.quantize(Wr_s.reshape(m, n // 8, 8), return_idx=True)
    hat0 = hat0.reshape(m, n).contiguous()
    idx0 = idx0.reshape(m, n // 8)
    hatWr, Qidxs, mpq_stats = mpq_refine_codebook(Wr_s, Hr, hat0, idx0, cb, args, module_name=str(save_name))
    hatW = incoherence_process(hatWr, SU, SV * Wscale, had_dims=(had_m, had_n))
    fam_m = "had" if had_m == m else "block_had"
    fam_n = "had" if had_n == n else "block_had"

    attr: Dict[str, Any] = {
        "Qidxs": cb.maybe_pack_idxs(Qidxs).to("cpu"),
        "SU": SU.to(torch.float16).to("cpu"),
        "SV": (SV * Wscale).to(torch.float16).to("cpu"),  # Wscale fused into SV
        "scaleWH": None,
        "rotation_family": "had" if fam_m == fam_n == "had" else "block_had",
        "left_rotation_family": fam_m,
        "right_rotation_family": fam_n,
        "left_had_dim": int(had_m),
        "right_had_dim": int(had_n),
        "left_rotation_fallback_reason": left_reason,
        "right_rotation_fallback_reason": right_reason,
        "mpq_stats": _plain(mpq_stats),
    }
    scale_vals: List[float] = [float(s) for s in scales]
    if len(scales) == 1:
        attr["SV"] *= scales[0].to("cpu")
        scale_vals = [1.0]
    attr.update({
        "fused": len(shapes) > 1,
        "shapes": [torch.Size(s) for s in shapes],
        "scales": scale_vals,
        "input_fingerprint": {
            "protocol": "paired_w_h_sha256_v1",
            "w_sha256": tensor_sha256(W),
            "h_sha256": tensor_sha256(H),
            "w_shape": [int(d) for d in W.shape],
            "h_shape": [int(d) for d in H.shape],
            "basis": "pre_incoherence",
        },
    })
    diff = hatW - W
    err_frob = float(diff.square().sum() / W.square().sum().clamp_min(1e-12))
    err_proxy = float((ops.gemm(diff, H) * diff).sum() / (ops.gemm(W, H) * W).sum().abs().clamp_min(1e-12))
    return attr, err_frob, err_proxy, hatW


def _plain(obj):
    """Stats as plain Python values (loadable with ``torch.load(weights_only=True)``)."""
    if isinstance(obj, dict):
        return {str(k): _plain(v) for k, v in obj.items()}
    if isinstance(obj, (list, tuple)):
        return [_plain(v) for v in obj]
    if isinstance(obj, torch.Tensor):
        return obj.item() if obj.numel() == 1 else obj.detach().to("cpu").tolist()
    if obj is None or isinstance(obj, (bool, int, float, str)):
        return obj
    return str(obj)


def save_quantized_attr(attr: Dict[str, Any], save_path: str) -> None:
    """mpq/quip_generic.py:425-426."""
    torch.save(attr, save_path)


def layer_ckpt_path(save_dir: str, idx: int, name: str) -> str:
    """``{save_dir}/{idx}_{name}.pt`` with name in {qkv, o, up, down} (mpq/quip_generic.py:628)."""
    if name not in ("qkv", "o", "up", "down"):
        raise ValueError(f"QUIP# ckpt linear name must be qkv, o, up or down, got {name!r}")
    return os.path.join(str(save_dir), f"{int(idx)}_{name}.pt")


@torch.inference_mode()
def quantize_layer_to_ckpt(*, save_dir: str, idx: int, linears: Dict[str, Tuple[Sequence[torch.Tensor], torch.Tensor]],
                           cb: Any, args: Any, device=None,
                           allow_block_hadamard: bool = False) -> Dict[str, Dict[str, float]]:
    """Write ``{idx}_{name}.pt`` for each fused linear of a decoder layer: ``linears`` maps
    qkv / o / up / down to (weights, regularised Hessian).  Returns the errors per linear."""
    os.makedirs(str(save_dir), exist_ok=True)
    out: Dict[str, Dict[str, float]] = {}
    for name, (weights, H) in linears.items():
        path = layer_ckpt_path(save_dir, idx, name)
        attr, ef, ep, _ = quantize_weights_to_attr(weights=weights, H=H, cb=cb, args=args,
                                                   save_name=os.path.basename(path), device=device,
                                                   allow_block_hadamard=allow_block_hadamard)
        save_quantized_attr(attr, path)
        out[name] = {"err_frob": ef, "err_proxy": ep}
    return out


def _saved_had_dim(saved_layer: Dict[str, Any], side: str, width: int) -> int:
    """Transform size of one side of a saved linear from its rotation family."""
    fam = str(saved_layer.get(f"{side}_rotation_family", saved_layer.get("rotation_family", "had")))
    if fam == "had":
        if width & (width - 1):
            raise ValueError(f"{side} width {width} with rotation_family 'had' needs quip-sharp's had-K transform, "
                             "which this build does not provide")
        return width
    if fam == "block_had":
        had = int(saved_layer.get(f"{side}_had_dim", width & -width))
        if had <= 0 or had & (had - 1) or width % had:
            raise ValueError(f"{side}_had_dim={had} does not tile width {width}")
        return had
    raise ValueError(f"unknown {side} rotation family {fam!r}")


@torch.inference_mode()
def decompress_saved_quip(saved_layer: Dict[str, Any], cb: Any, *, device) -> torch.Tensor:
    """hatW of a saved linear (mpq/quip_generic.py:737-749): codewords of ``Qidxs`` in the RHT basis,
    then the inverse RHT with ``SU`` and the scale-carrying ``SV``, each side with the transform its
    rotation family records."""
    dev = torch.device(device)
    SU = saved_layer["SU"].to(dev)
    SV = saved_layer["SV"].to(dev)
    Qidxs = saved_layer["Qidxs"].to(dev)
    n, m = len(SU), len(SV)
    had_dims = (_saved_had_dim(saved_layer, "left", m), _saved_had_dim(saved_layer, "right", n))
    hatWr = cb.by_idxs(Qidxs).reshape(m, n).to(torch.float32).contiguous()
    return incoherence_process(hatWr, SU, SV, had_dims=had_dims)


def load_split_weights(path: str, cb: Any, *, device) -> List[torch.Tensor]:
    """The per-projection weights of a saved linear (mpq/quip_generic.py:752-760)."""
    saved = torch.load(path, map_location="cpu", weights_only=True)
    hatW = decompress_saved_quip(saved, cb, device=device)
    sizes = [int(s[0]) for s in saved["shapes"]]
    scales = list(saved.get("scales", [1.0] * len(sizes)))
    return [w * float(scales[i]) for i, w in enumerate(torch.split(hatW, sizes, dim=0))]
