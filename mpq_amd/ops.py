"""Typed wrappers of the C-ABI entry points (one function per ``mpq_*`` symbol).

Every wrapper checks shapes/dtypes on the host, allocates outputs with torch's
caching allocator (device memory plumbing only), and enqueues the HIP kernels
on torch's current stream.  No wrapper has a CPU path.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch

from . import _lib

F32 = torch.float32


def _dev(*ts: Optional[torch.Tensor]) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError(f"mpq_amd operates on ROCm device tensors only (got a tensor on {t.device}).")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError("all tensors must be on the same device")
    if dev is None:
        raise ValueError("no device tensor given")
    return dev


def _f32c(t: torch.Tensor) -> torch.Tensor:
    return t.to(dtype=F32).contiguous()


def _stream(dev: torch.device) -> int:
    return _lib.stream_handle(dev)


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


# ---- GEMM -----------------------------------------------------------------

def gemm(A: torch.Tensor, B: torch.Tensor, *, trans_b: bool = False, b_rows: Optional[torch.Tensor] = None,
         out: Optional[torch.Tensor] = None, alpha: float = 1.0, beta: float = 0.0) -> torch.Tensor:
    """C = alpha * A @ op(B) + beta * C on the fp32 MFMA kernel (deterministic split-K)."""
    dev = _dev(A, B)
    A = _f32c(A)
    B = _f32c(B)
    M, K = A.shape
    if b_rows is not None:
        b_rows = b_rows.to(device=dev, dtype=torch.int32).contiguous()
        if trans_b or int(b_rows.numel()) != K:
            raise ValueError("b_rows needs trans_b=False and K entries")
        N = int(B.shape[1])
    elif trans_b:
        N = int(B.shape[0])
        if int(B.shape[1]) != K:
            raise ValueError(f"shape mismatch: A {tuple(A.shape)} vs B^T of {tuple(B.shape)}")
    else:
        N = int(B.shape[1])
        if int(B.shape[0]) != K:
            raise ValueError(f"shape mismatch: A {tuple(A.shape)} vs B {tuple(B.shape)}")
    if out is None:
        if beta != 0.0:
            raise ValueError("beta != 0 needs out")
        out = torch.empty(M, N, dtype=F32, device=dev)
    elif out.dtype != F32 or not out.is_contiguous() or tuple(out.shape) != (M, N):
        raise ValueError("out must be a contiguous fp32 (M, N) tensor")
    ws_floats = 32 * M * N if K >= 512 else 0
    ws = torch.empty(max(ws_floats, 1), dtype=F32, device=dev)
    _lib.call("mpq_gemm_f32", M, N, K, _lib.ptr(A), K, _lib.ptr(B), int(B.shape[1]), int(bool(trans_b)),
              _lib.ptr(b_rows), _lib.ptr(out), N, float(alpha), float(beta), _lib.ptr(ws), ws_floats,
              _stream(dev))
    return out


def _check_index_range(idx: torch.Tensor, bound: int) -> None:
    """The kernels read through ``idx`` unchecked: every entry must lie in [0, bound)."""
    if idx.numel() and (int(idx.min().item()) < 0 or int(idx.max().item()) >= bound):
        raise ValueError(f"index entries must lie in [0, {bound})")


def permute_columns(X: torch.Tensor, perm: torch.Tensor) -> torch.Tensor:
    """out[:, c] = X[:, perm[c]] (fp32 or uint8 rows x cols)."""
    dev = _dev(X, perm)
    if X.dtype not in (F32, torch.uint8) or X.dim() != 2:
        raise ValueError("permute_columns takes a 2-D float32 or uint8 tensor")
    X = X.contiguous()
    rows, cols = X.shape
    perm = perm.to(device=dev, dtype=torch.int32).contiguous()
    if int(perm.numel()) != cols:
        raise ValueError("perm must hold one entry per column")
    _check_index_range(perm, cols)
    out = torch.empty_like(X)
    _lib.call("mpq_permute_columns", _lib.ptr(X), rows, cols, _lib.ptr(perm), _lib.ptr(out),
              1 if X.dtype == torch.uint8 else 4, _stream(dev))
    return out


def permute_symmetric(H: torch.Tensor, perm: torch.Tensor) -> torch.Tensor:
    """out[i][j] = H[perm[i]][perm[j]] (fp32 n x n)."""
    dev = _dev(H, perm)
    H = _f32c(H)
    n = int(H.shape[0])
    perm = perm.to(device=dev, dtype=torch.int32).contiguous()
    if tuple(H.shape) != (n, n) or int(perm.numel()) != n:
        raise ValueError("permute_symmetric takes an n x n matrix and n entries")
    _check_index_range(perm, n)
    out = torch.empty_like(H)
    _lib.call("mpq_permute_symmetric", _lib.ptr(H), n, _lib.ptr(perm), _lib.ptr(out), _stream(dev))
    return out


def gemm_f64(A: torch.Tensor, B: torch.Tensor, *, trans_b: bool = False, out: Optional[torch.Tensor] = None,
             alpha: float = 1.0, beta: float = 0.0) -> torch.Tensor:
    """C = alpha * A @ op(B) + beta * C in fp64 on the fp64 matrix cores (the eigensolver's kernel)."""
    dev = _dev(A, B)
    A = A.to(dtype=torch.float64).contiguous()
    B = B.to(dtype=torch.float64).contiguous()
    M, K = A.shape
    N = int(B.shape[0]) if trans_b else int(B.shape[1])
    if int(B.shape[1] if trans_b else B.shape[0]) != K:
        raise ValueError(f"shape mismatch: A {tuple(A.shape)} vs op(B) of {tuple(B.shape)}")
    if out is None:
        if beta != 0.0:
            raise ValueError("beta != 0 needs out")
        out = torch.empty(M, N, dtype=torch.float64, device=dev)
    elif out.dtype != torch.float64 or not out.is_contiguous() or tuple(out.shape) != (M, N):
        raise ValueError("out must be a contiguous fp64 (M, N) tensor")
    lib = _lib.load()
    wsb = int(lib.mpq_gemm_f64_workspace_size(M, N, K))
    ws = workspace(wsb, dev) if wsb > 0 else None
    _lib.call("mpq_gemm_f64", M, N, K, _lib.ptr(A), K, _lib.ptr(B), int(B.shape[1]), int(bool(trans_b)),
              _lib.ptr(out), N, float(alpha), float(beta), _lib.ptr(ws), wsb, _stream(dev))
    return out


def gemm_x6_pack_b(B: torch.Tensor, *, trans_b: bool = False) -> torch.Tensor:
    """op(B) (K x N; N % 128 == 0, K % 32 == 0) packed for :func:`gemm_x6` (K * N floats)."""
    dev = _dev(B)
    B = _f32c(B)
    K, N = (int(B.shape[1]), int(B.shape[0])) if trans_b else (int(B.shape[0]), int(B.shape[1]))
    out = torch.empty(K * N, dtype=F32, device=dev)
    _lib.call("mpq_gemm_x6_pack_b", K, N, _lib.ptr(B), int(B.shape[1]), int(bool(trans_b)), _lib.ptr(out),
              _stream(dev))
    return out


def gemm_x6(A: torch.Tensor, B_packed: torch.Tensor, N: int, *, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """C = A @ op(B) with op(B) packed by :func:`gemm_x6_pack_b`: fp32 product on the bf16 matrix
    cores (three bf16 planes per operand, six plane products)."""
    dev = _dev(A, B_packed)
    A = _f32c(A)
    M, K = A.shape
    if int(B_packed.numel()) != K * int(N) or B_packed.dtype != F32:
        raise ValueError("B_packed must hold K * N float32 values from gemm_x6_pack_b")
    if out is None:
        out = torch.empty(M, int(N), dtype=F32, device=dev)
    elif out.dtype != F32 or not out.is_contiguous() or tuple(out.shape) != (M, int(N)):
        raise ValueError("out must be a contiguous fp32 (M, N) tensor")
    lib = _lib.load()
    need = int(lib.mpq_gemm_x6_workspace_size(M, int(N), K))
    ws = workspace(need, dev)
    _lib.call("mpq_gemm_x6", M, int(N), K, _lib.ptr(A), K, _lib.ptr(B_packed), _lib.ptr(out), int(N), _lib.ptr(ws),
              int(ws.numel()), _stream(dev))
    return out


def gemm_x6_pack_a(A: torch.Tensor) -> torch.Tensor:
    """A (M x K, K % 32 == 0) split into bf16 planes and packed for :func:`gemm_x6_splitk` (uint8 buffer)."""
    dev = _dev(A)
    A = _f32c(A)
    M, K = A.shape
    lib = _lib.load()
    out = torch.empty(int(lib.mpq_gemm_x6_packed_a_size(M, K)), dtype=torch.uint8, device=dev)
    _lib.call("mpq_gemm_x6_pack_a", M, K, _lib.ptr(A), K, _lib.ptr(out), _stream(dev))
    return out


def gemm_x6_splitk(A_packed: torch.Tensor, B_packed: torch.Tensor, M: int, N: int, K: int, *,
                   splits: Optional[int] = None, out: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, int]:
    """Split-K partials (splits, M, N) of the x6 product from packed operands (the VAMP solvers' launch)."""
    dev = _dev(A_packed, B_packed, out)
    lib = _lib.load()
    s = int(splits) if splits is not None else int(lib.mpq_gemm_x6_split_count(M, N, K))
    if out is None:
        out = torch.empty(s, M, N, dtype=F32, device=dev)
    elif tuple(out.shape) != (s, M, N) or out.dtype != F32 or not out.is_contiguous():
        raise ValueError("out must be a contiguous fp32 (splits, M, N) tensor")
    _lib.call("mpq_gemm_x6_splitk", M, N, K, _lib.ptr(A_packed), _lib.ptr(B_packed), _lib.ptr(out), s, _stream(dev))
    return out, s


# Smallest n for which the adapters run the rank-space products as x6 products: a 128 x n x n
# product at n = 2048 is launch-latency bound, and the extra pack of A made the E8P12 solver slower
# there (up/gate VAMP 428 -> 451 ms on a Llama-3.2-1B layer), while n = 4096 (Llama-3-8B q/k/v/o,
# gate/up: 405 -> 380 ms) and larger gain.
X6_MIN_N = 4096


def rankspace_pack(V: torch.Tensor, Vs: torch.Tensor) -> Optional[torch.Tensor]:
    """The packed rank-space operator (V for r V, V for x V^T, Vs for x Vs) of the VAMP solvers' x6
    products, or None when n has no x6 path (n % 128 != 0)."""
    dev = _dev(V, Vs)
    n = int(V.shape[0])
    if tuple(V.shape) != (n, n) or tuple(Vs.shape) != (n, n):
        raise ValueError("rankspace_pack needs square V and Vs of the same order")
    lib = _lib.load()
    floats = int(lib.mpq_rankspace_pack_floats(n))
    if floats == 0:
        return None
    out = torch.empty(floats, dtype=F32, device=dev)
    _lib.call("mpq_rankspace_pack", n, _lib.ptr(_f32c(V)), _lib.ptr(_f32c(Vs)), _lib.ptr(out), _stream(dev))
    return out


# ---- quantizer helpers ----------------------------------------------------

def gemm_splitk(A: torch.Tensor, B: torch.Tensor, *, trans_b: bool = False, splits: Optional[int] = None,
                out: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, int]:
    """Split-K partial products (splits, M, N) of A op(B); ``splits`` defaults to the library's choice."""
    dev = _dev(A, B, out)
    A = _f32c(A)
    B = _f32c(B)
    M, K = A.shape
    N = int(B.shape[0] if trans_b else B.shape[1])
    lib = _lib.load()
    s = int(splits) if splits is not None else int(lib.mpq_gemm_f32_split_count(M, N, K))
    if out is None:
        out = torch.empty(s, M, N, dtype=F32, device=dev)
    elif tuple(out.shape) != (s, M, N) or out.dtype != F32 or not out.is_contiguous():
        raise ValueError("out must be a contiguous fp32 (splits, M, N) tensor")
    _lib.call("mpq_gemm_f32_splitk", M, N, K, _lib.ptr(A), K, _lib.ptr(B), int(B.shape[1]), int(bool(trans_b)),
              _lib.ptr(out), s, _stream(dev))
    return out, s


def gptq_find_params(W: torch.Tensor, group_size: int, maxq: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Asymmetric min-max GPTQ parameters per (row, group): (scale, zero) of shape (rows, G)."""
    dev = _dev(W)
    W = _f32c(W)
    rows, n = W.shape
    G = (n + group_size - 1) // group_size
    scale = torch.empty(rows, G, dtype=F32, device=dev)
    zero = torch.empty(rows, G, dtype=F32, device=dev)
    for r0 in range(0, rows, 65535):
        r1 = min(rows, r0 + 65535)
        _lib.call("mpq_gptq_find_params", _lib.ptr(W[r0:r1]), r1 - r0, n, n, int(group_size), int(maxq),
                  _lib.ptr(scale[r0:r1]), _lib.ptr(zero[r0:r1]), _stream(dev))
    return scale, zero


def uniform_rtn(W: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor, group_size: int, maxq: int,
                want_q: bool = True, want_x: bool = True):
    dev = _dev(W, scale, zero)
    W = _f32c(W)
    rows, n = W.shape
    scale = _f32c(scale)
    zero = _f32c(zero)
    q = torch.empty(rows, n, dtype=torch.uint8, device=dev) if want_q else None
    x = torch.empty(rows, n, dtype=F32, device=dev) if want_x else None
    _lib.call("mpq_uniform_rtn", _lib.ptr(W), rows, n, n, _lib.ptr(scale), _lib.ptr(zero), int(group_size),
              int(maxq), _lib.ptr(q), _lib.ptr(x), _stream(dev))
    return q, x


def dequant(q: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor, group_size: int) -> torch.Tensor:
    dev = _dev(q, scale, zero)
    q = q.to(torch.uint8).contiguous()
    rows, n = q.shape
    x = torch.empty(rows, n, dtype=F32, device=dev)
    _lib.call("mpq_dequant", _lib.ptr(q), rows, n, _lib.ptr(_f32c(scale)), _lib.ptr(_f32c(zero)),
              int(group_size), _lib.ptr(x), _stream(dev))
    return x


# ---- rotation -------------------------------------------------------------

def block_hadamard(X: torch.Tensor, had_dim: int, signs: Optional[torch.Tensor] = None,
                   inverse: bool = False) -> torch.Tensor:
    """Signed block Walsh-Hadamard along the last dim (forward: X*signs then H; inverse: H then *signs)."""
    dev = _dev(X, signs)
    shape = X.shape
    X2 = _f32c(X).reshape(-1, shape[-1])
    rows, width = X2.shape
    out = torch.empty_like(X2)
    sg = None if signs is None else _f32c(signs)
    for r0 in range(0, rows, 65535):
        r1 = min(rows, r0 + 65535)
        _lib.call("mpq_block_hadamard", _lib.ptr(X2[r0:r1]), width, _lib.ptr(out[r0:r1]), width, r1 - r0, width,
                  int(had_dim), _lib.ptr(sg), int(bool(inverse)), _stream(dev))
    return out.reshape(shape)


def transpose(X: torch.Tensor) -> torch.Tensor:
    dev = _dev(X)
    X = _f32c(X)
    rows, cols = X.shape
    out = torch.empty(cols, rows, dtype=F32, device=dev)
    _lib.call("mpq_transpose", _lib.ptr(X), rows, cols, cols, _lib.ptr(out), rows, _stream(dev))
    return out


def scale_columns(X: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """out = X * scale[None, :]."""
    dev = _dev(X, scale)
    X = _f32c(X)
    rows, cols = X.shape
    out = torch.empty_like(X)
    _lib.call("mpq_scale_columns", _lib.ptr(X), rows, cols, _lib.ptr(_f32c(scale)), _lib.ptr(out), _stream(dev))
    return out


def syevd(H: torch.Tensor, method: int = 0) -> Tuple[torch.Tensor, torch.Tensor]:
    """Eigendecomposition of a symmetric matrix: (lam ascending, V with eigenvectors as columns).
    float64 input runs in fp64 (mpq_syevd_f64), anything else in fp32 (mpq_syevd_method; method 0
    = automatic, 1 = one-stage tridiagonalisation, 2 = two-stage band reduction)."""
    dev = _dev(H)
    f64 = H.dtype == torch.float64
    H = H.contiguous() if f64 else _f32c(H)
    n = int(H.shape[0])
    if tuple(H.shape) != (n, n):
        raise ValueError("H must be square")
    lib = _lib.load()
    name = "mpq_syevd_f64" if f64 else "mpq_syevd"
    ws = workspace(int(getattr(lib, name + "_workspace_size")(n)), dev)
    lam = torch.empty(n, dtype=H.dtype, device=dev)
    V = torch.empty(n, n, dtype=H.dtype, device=dev)
    if f64:
        if method not in (0, 1):
            raise ValueError("the fp64 eigensolver has the one-stage reduction only")
        _lib.call(name, n, _lib.ptr(H), _lib.ptr(lam), _lib.ptr(V), _lib.ptr(ws), int(ws.numel()), _stream(dev))
    else:
        _lib.call("mpq_syevd_method", n, _lib.ptr(H), _lib.ptr(lam), _lib.ptr(V), _lib.ptr(ws), int(ws.numel()),
                  int(method), _stream(dev))
    return lam, V


def eigh_postprocess(lam_asc: torch.Tensor, V_asc: torch.Tensor, floor: float):
    """(lam, S, V, Vs): descending order, floored eigenvalues, S = sqrt(lam), Vs = V * S."""
    dev = _dev(lam_asc, V_asc)
    lam_asc = _f32c(lam_asc)
    V_asc = _f32c(V_asc)
    n = int(lam_asc.numel())
    lam = torch.empty(n, dtype=F32, device=dev)
    S = torch.empty(n, dtype=F32, device=dev)
    V = torch.empty(n, n, dtype=F32, device=dev)
    Vs = torch.empty(n, n, dtype=F32, device=dev)
    _lib.call("mpq_eigh_postprocess", _lib.ptr(lam_asc), _lib.ptr(V_asc), n, float(floor), _lib.ptr(lam),
              _lib.ptr(S), _lib.ptr(V), _lib.ptr(Vs), _stream(dev))
    return lam, S, V, Vs


# ---- uniform VAMP and CD ------------------------------------------------------

def vamp_config_c(cfg) -> "_lib.UniformVampConfigC":
    fd = str(getattr(cfg, "final_decision", "map") or "map").strip().lower()
    if fd not in ("map", "round_mean"):
        raise ValueError(f"unsupported final_decision={fd!r}")
    init = str(getattr(cfg, "init_from", "rtn") or "rtn").strip().lower()
    if init not in ("rtn", "float", "zero"):
        raise ValueError(f"unknown init_from={init!r} (expected 'rtn', 'float', or 'zero').")
    c = _lib.UniformVampConfigC()
    c.iters = max(int(cfg.iters), 0)
    c.damping = float(cfg.damping)
    c.final_decision = 0 if fd == "map" else 1
    c.init_from = {"rtn": 0, "float": 1, "zero": 2}[init]
    c.gamma_start = float(cfg.gamma_start)
    c.gamma_retry_factor = float(cfg.gamma_retry_factor)
    c.gamma_retry_steps = int(cfg.gamma_retry_steps)
    c.prior_tau = float(cfg.prior_tau)
    c.obs_precision = float(cfg.obs_precision)
    c.em_obs_precision = int(bool(cfg.em_obs_precision))
    c.em_obs_precision_damping = float(cfg.em_obs_precision_damping)
    c.em_obs_precision_min = float(cfg.em_obs_precision_min)
    c.em_obs_precision_max = float(cfg.em_obs_precision_max)
    return c


def uniform_vamp_solve(W, x_init, scale, zero, group_size, maxq, V, S, Vs, cfg, obs_init: float = 0.0,
                       want_x: bool = False, ws: Optional[torch.Tensor] = None, Yu=None, xr=None,
                       xprod_out: Optional[torch.Tensor] = None, packed: Optional[torch.Tensor] = None,
                       q_out: Optional[torch.Tensor] = None, err_out: Optional[torch.Tensor] = None,
                       rtn_err_out: Optional[torch.Tensor] = None):
    """One row block of the uniform VAMP loop.  Returns (q uint8, x|None, err, rtn_err, stats dict).
    ``Yu`` = W Vs and ``xr`` = x_init Vs may come from the caller (formed once for all row blocks);
    ``xprod_out`` (rows x n, contiguous fp32) then receives x_best Vs of the returned codes.
    ``packed`` (from :func:`rankspace_pack`) runs the solver's products on the bf16 matrix cores.
    ``q_out`` (uint8 rows x n), ``err_out`` and ``rtn_err_out`` (float32 rows), contiguous, receive the
    results in place of new tensors."""
    dev = _dev(W, x_init, scale, zero, V, S, Vs, Yu, xr, xprod_out, packed)
    W = _f32c(W)
    x_init = _f32c(x_init)
    rows, n = W.shape
    if tuple(V.shape) != (n, n) or int(S.numel()) != n or tuple(Vs.shape) != (n, n):
        raise ValueError("mpq_amd uniform VAMP needs full rank: V, Vs (n x n) and S (n)")
    lib = _lib.load()
    if packed is not None and (packed.dtype != F32 or not packed.is_contiguous()
                               or int(packed.numel()) != int(lib.mpq_rankspace_pack_floats(n)) or n % 128):
        raise ValueError("packed must be the float32 rank-space operator from rankspace_pack for this n")
    need = int(lib.mpq_uniform_vamp_workspace_size(rows, n))
    if ws is None or ws.numel() < need:
        ws = workspace(need, dev)
    for name, t, dt, shape in (("q_out", q_out, torch.uint8, (rows, n)), ("err_out", err_out, F32, (rows,)),
                               ("rtn_err_out", rtn_err_out, F32, (rows,))):
        if t is not None and (tuple(t.shape) != shape or t.dtype != dt or not t.is_contiguous()):
            raise ValueError(f"{name} must be a contiguous {dt} tensor of shape {shape}")
    q = q_out if q_out is not None else torch.empty(rows, n, dtype=torch.uint8, device=dev)
    x = torch.empty(rows, n, dtype=F32, device=dev) if want_x else None
    err = err_out if err_out is not None else torch.empty(rows, dtype=F32, device=dev)
    rtn_err = rtn_err_out if rtn_err_out is not None else torch.empty(rows, dtype=F32, device=dev)
    st = _lib.UniformVampStatsC()
    c = vamp_config_c(cfg)
    for name, t in (("Yu", Yu), ("xr", xr), ("xprod_out", xprod_out)):
        if t is not None and (tuple(t.shape) != (rows, n) or t.dtype != F32 or not t.is_contiguous()):
            raise ValueError(f"{name} must be a contiguous float32 tensor of shape {(rows, n)}")
    _lib.call("mpq_uniform_vamp_solve_ex", rows, n, int(maxq), _lib.ptr(W), n, _lib.ptr(x_init),
              _lib.ptr(_f32c(scale)), _lib.ptr(_f32c(zero)), int(group_size), _lib.ptr(_f32c(V)),
              _lib.ptr(_f32c(S)), _lib.ptr(_f32c(Vs)), ctypes.byref(c), float(obs_init or 0.0), _lib.ptr(Yu),
              _lib.ptr(xr), _lib.ptr(packed), _lib.ptr(q), _lib.ptr(x), _lib.ptr(err), _lib.ptr(rtn_err),
              _lib.ptr(xprod_out),
              ctypes.byref(st), _lib.ptr(ws), int(ws.numel()), _stream(dev))
    stats = {name: getattr(st, name) for name, _ in st._fields_}
    return q, x, err, rtn_err, stats


def uniform_cd_polish(W, q_in, scale, zero, group_size, maxq, Vs, H, *, block_rows: int, sweeps: int,
                      accept_tol: float = 0.0, select: bool = True, Yu=None, x_in=None, xprod=None,
                      S=None, packed=None, ws: Optional[torch.Tensor] = None):
    """Greedy scalar CD over all rows (greedy order per row block).  ``W`` may be None when ``Yu``
    is given; ``xprod`` (optional) is the start's x Vs.  ``S`` with ``packed`` (``rankspace_pack``,
    n % 128 == 0) runs the two full products as x6 products.  Returns (q, err_before, err_after,
    improved, accepted_per_row)."""
    if (S is None) != (packed is None):
        raise ValueError("uniform_cd_polish: S and packed go together")
    if packed is not None and packed.numel() != 3 * Vs.shape[0] * Vs.shape[0]:
        raise ValueError("uniform_cd_polish: packed must hold 3 n^2 floats (rankspace_pack)")
    dev = _dev(q_in, scale, zero, Vs, H, W, Yu, x_in, xprod)
    W = None if W is None else _f32c(W)
    Yu = None if Yu is None else _f32c(Yu)
    x_in = None if x_in is None else _f32c(x_in)
    rows, n = q_in.shape
    lib = _lib.load()
    need = int(lib.mpq_uniform_cd_workspace_size(rows, n, int(block_rows)))
    if ws is None or ws.numel() < need:
        ws = workspace(need, dev)
    q_out = torch.empty(rows, n, dtype=torch.uint8, device=dev)
    eb = torch.empty(rows, dtype=F32, device=dev)
    ea = torch.empty(rows, dtype=F32, device=dev)
    imp = torch.zeros(rows, dtype=torch.int32, device=dev)
    acc = torch.zeros(rows, dtype=torch.int32, device=dev)
    xprod = None if xprod is None else _f32c(xprod)
    _lib.call("mpq_uniform_cd_polish_ex", rows, n, int(maxq), int(block_rows), int(sweeps), float(accept_tol),
              _lib.ptr(W), n, _lib.ptr(Yu), _lib.ptr(q_in.to(torch.uint8).contiguous()), _lib.ptr(x_in),
              _lib.ptr(xprod), _lib.ptr(_f32c(scale)),
              _lib.ptr(_f32c(zero)), int(group_size), _lib.ptr(_f32c(Vs)),
              _lib.ptr(None if S is None else _f32c(S)), _lib.ptr(packed), _lib.ptr(_f32c(H)), int(bool(select)),
              _lib.ptr(q_out), _lib.ptr(eb), _lib.ptr(ea), _lib.ptr(imp), _lib.ptr(acc), _lib.ptr(ws),
              int(ws.numel()), _stream(dev))
    return q_out, eb, ea, imp, acc


def uniform_cd_sweeps(rhs, x, q, res_norm, accepted, scale, zero, group_size, maxq, diag, H, *,
                      block_rows: int, sweeps: int, accept_tol: float = 0.0, target_rule: str = "div"):
    """The greedy sweeps in place on (rhs, x, q, res_norm, accepted): the state the reference's
    persistent sweep kernel takes (mpq/polish/triton_scalar_cd.py:113-161).  ``target_rule`` "div"
    forms the RTN target x + rhs / diag (the sweep kernel, :73), "recip" x + rhs * (1 / diag) (the
    torch update loop, :266)."""
    if target_rule not in ("div", "recip"):
        raise ValueError(f"target_rule must be 'div' or 'recip', got {target_rule!r}")
    dev = _dev(rhs, x, q, res_norm, accepted, scale, zero, diag, H)
    rows, n = rhs.shape
    for name, t, dt, shape in (("rhs", rhs, F32, (rows, n)), ("x", x, F32, (rows, n)),
                               ("q", q, torch.uint8, (rows, n)), ("res_norm", res_norm, F32, (rows,)),
                               ("accepted", accepted, torch.int32, (rows,))):
        if tuple(t.shape) != shape or t.dtype != dt or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous {dt} tensor of shape {shape}")
    lib = _lib.load()
    need = int(lib.mpq_uniform_cd_sweeps_workspace_size(rows, n, int(block_rows)))
    ws = workspace(need, dev)
    entry = "mpq_uniform_cd_sweeps" if target_rule == "div" else "mpq_uniform_cd_sweeps_recip"
    _lib.call(entry, rows, n, int(maxq), int(block_rows), int(sweeps), float(accept_tol),
              _lib.ptr(rhs), _lib.ptr(x), _lib.ptr(q), _lib.ptr(res_norm), _lib.ptr(accepted),
              _lib.ptr(_f32c(scale)), _lib.ptr(_f32c(zero)), int(group_size), _lib.ptr(_f32c(diag)),
              _lib.ptr(_f32c(H)), _lib.ptr(ws), int(ws.numel()), _stream(dev))


# ---- E8P12 VAMP ----------------------------------------------------------------

def e8p12_vamp_config_c(cfg) -> "_lib.E8P12VampConfigC":
    c = _lib.E8P12VampConfigC()
    c.iters = max(int(cfg.iters), 0)
    c.damping = float(cfg.damping)
    c.gamma_start = float(cfg.gamma_start)
    c.gamma_retry_factor = float(cfg.gamma_retry_factor)
    c.gamma_retry_steps = int(cfg.gamma_retry_steps)
    c.prior_tau = float(cfg.prior_tau)
    c.obs_precision = float(cfg.obs_precision)
    c.em_obs_precision = int(bool(cfg.em_obs_precision))
    c.em_obs_precision_damping = float(cfg.em_obs_precision_damping)
    c.em_obs_precision_min = float(cfg.em_obs_precision_min)
    c.em_obs_precision_max = float(cfg.em_obs_precision_max)
    c.best_iterate = int(bool(getattr(cfg, "best_iterate", False)))
    return c


def e8p12_vamp_solve(Wr, hat_init, V, S, Vs, cfg, *, prior_scale: Optional[torch.Tensor] = None,
                     obs_init: float = 0.0, want_state: bool = False, ws: Optional[torch.Tensor] = None,
                     packed: Optional[torch.Tensor] = None):
    """One row block of the E8P12 VAMP loop (no polish).  ``packed`` (from :func:`rankspace_pack`)
    runs the solver's products on the bf16 matrix cores.

    Returns (idx int64 (rows, n/8), hat (rows, n), err (rows), r1|None, gamma1|None, stats dict)."""
    dev = _dev(Wr, hat_init, V, S, Vs, prior_scale, packed)
    Wr = _f32c(Wr)
    hat_init = _f32c(hat_init)
    rows, n = Wr.shape
    if n % 8:
        raise ValueError(f"E8P12 solver expects n divisible by 8; got n={n}, codesz=8.")
    if tuple(V.shape) != (n, n) or int(S.numel()) != n or tuple(Vs.shape) != (n, n):
        raise ValueError("mpq_amd E8P12 VAMP needs full rank: V, Vs (n x n) and S (n)")
    if prior_scale is not None:
        prior_scale = _f32c(prior_scale).reshape(-1)
        if int(prior_scale.numel()) != rows * (n // 8):
            raise ValueError("prior_scale must hold one entry per 8-block")
    lib = _lib.load()
    if packed is not None and (packed.dtype != F32 or not packed.is_contiguous()
                               or int(packed.numel()) != int(lib.mpq_rankspace_pack_floats(n)) or n % 128):
        raise ValueError("packed must be the float32 rank-space operator from rankspace_pack for this n")
    need = int(lib.mpq_e8p12_vamp_workspace_size(rows, n))
    if ws is None or ws.numel() < need:
        ws = workspace(need, dev)
    idx = torch.empty(rows, n // 8, dtype=torch.int64, device=dev)
    hat = torch.empty(rows, n, dtype=F32, device=dev)
    err = torch.empty(rows, dtype=F32, device=dev)
    r1 = torch.empty(rows, n, dtype=F32, device=dev) if want_state else None
    g1 = torch.empty(rows, 1, dtype=F32, device=dev) if want_state else None
    st = _lib.E8P12VampStatsC()
    c = e8p12_vamp_config_c(cfg)
    _lib.call("mpq_e8p12_vamp_solve_ex", rows, n, _lib.ptr(Wr), _lib.ptr(hat_init), _lib.ptr(_f32c(V)),
              _lib.ptr(_f32c(S)), _lib.ptr(_f32c(Vs)), _lib.ptr(prior_scale), ctypes.byref(c),
              float(obs_init or 0.0), _lib.ptr(packed), _lib.ptr(idx), _lib.ptr(hat), _lib.ptr(err), _lib.ptr(r1),
              _lib.ptr(g1),
              ctypes.byref(st), _lib.ptr(ws), int(ws.numel()), _stream(dev))
    stats = {name: getattr(st, name) for name, _ in st._fields_}
    return idx, hat, err, r1, g1, stats


# ---- E8P12 gram-metric polish ----------------------------------------------------

def e8p12_cd_prepare(Vs: torch.Tensor) -> torch.Tensor:
    """Per-layer context (H, per-block G/L/Gi, grid, |L^T c|^2 tables) as an opaque uint8 tensor."""
    dev = _dev(Vs)
    Vs = _f32c(Vs)
    n = int(Vs.shape[0])
    if tuple(Vs.shape) != (n, n) or n % 8:
        raise ValueError("E8P12 polish needs a square Vs with n divisible by 8")
    lib = _lib.load()
    ctx = workspace(int(lib.mpq_e8p12_cd_context_size(n)), dev)
    _lib.call("mpq_e8p12_cd_prepare", n, _lib.ptr(Vs), _lib.ptr(ctx), int(ctx.numel()), _stream(dev))
    return ctx


def e8p12_cd_polish(x_in, idx_in, Vs, ctx, *, sweeps: int, block_rows: int, W=None, Yu=None,
                    max_blocks: int = 0, accept_tol: float = 0.0, ws: Optional[torch.Tensor] = None):
    """Gram-metric E8P12 block CD over all rows (greedy order per row block).

    Returns (x, idx, err_before, err_after, accepted_per_row)."""
    dev = _dev(x_in, idx_in, Vs, ctx, W, Yu)
    if (W is None) == (Yu is None):
        raise ValueError("give exactly one of W or Yu")
    x_in = _f32c(x_in)
    rows, n = x_in.shape
    idx_in = idx_in.to(dtype=torch.int64).contiguous()
    if tuple(idx_in.shape) != (rows, n // 8):
        raise ValueError("idx_in must be (rows, n/8)")
    W = None if W is None else _f32c(W)
    Yu = None if Yu is None else _f32c(Yu)
    lib = _lib.load()
    need = int(lib.mpq_e8p12_cd_workspace_size(rows, n, int(block_rows)))
    if ws is None or ws.numel() < need:
        ws = workspace(need, dev)
    x = torch.empty_like(x_in)
    idx = torch.empty_like(idx_in)
    eb = torch.empty(rows, dtype=F32, device=dev)
    ea = torch.empty(rows, dtype=F32, device=dev)
    acc = torch.empty(rows, dtype=torch.int32, device=dev)
    _lib.call("mpq_e8p12_cd_polish", rows, n, int(block_rows), int(sweeps), int(max_blocks), float(accept_tol),
              _lib.ptr(W), _lib.ptr(Yu), _lib.ptr(x_in), _lib.ptr(idx_in), _lib.ptr(_f32c(Vs)), _lib.ptr(ctx),
              _lib.ptr(x), _lib.ptr(idx), _lib.ptr(eb), _lib.ptr(ea), _lib.ptr(acc), _lib.ptr(ws),
              int(ws.numel()), _stream(dev))
    return x, idx, eb, ea, acc
