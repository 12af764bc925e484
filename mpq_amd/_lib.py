"""ctypes binding of ``libmpq_amd.so`` (the C-ABI in ``include/mpq_amd.h``).

The library is loaded from the package directory only.  There is no CPU or
PyTorch fallback: if the library is missing or a call fails, the caller gets an
exception.  Pointers are raw device addresses (``tensor.data_ptr()``); every
call is asynchronous on the given HIP stream (default: torch's current stream).
"""
from __future__ import annotations

import atexit
import ctypes
import os
import threading
from typing import Optional

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmpq_amd.so")

_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None

c_i64 = ctypes.c_int64
c_int = ctypes.c_int
c_float = ctypes.c_float
c_double = ctypes.c_double
c_ptr = ctypes.c_void_p

# name -> (restype, argtypes); every entry point returns an int status.
SIGNATURES = {
    "mpq_last_error": (ctypes.c_char_p, []),
    "mpq_last_error_code": (c_int, []),
    "mpq_clear_error": (None, []),
    "mpq_e8p12_map": (c_int, [c_ptr, c_i64, c_ptr, c_i64, c_ptr, c_ptr, c_float,
                              c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr]),
    "mpq_e8p12_denoise": (c_int, [c_ptr, c_i64, c_i64, c_ptr, c_ptr, c_ptr, c_float, c_ptr, c_ptr, c_ptr,
                                  c_ptr, c_ptr, c_ptr]),
    "mpq_e8p12_vamp_workspace_size": (c_i64, [c_i64, c_i64]),
    "mpq_e8p12_vamp_solve": (c_int, [c_i64, c_i64, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_double,
                                     c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_ptr]),
    "mpq_e8p12_vamp_solve_ex": (c_int, [c_i64, c_i64, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_double,
                                        c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_ptr]),
    "mpq_e8p12_cd_context_size": (c_i64, [c_i64]),
    "mpq_e8p12_cd_prepare": (c_int, [c_i64, c_ptr, c_ptr, c_i64, c_ptr]),
    "mpq_e8p12_cd_workspace_size": (c_i64, [c_i64, c_i64, c_i64]),
    "mpq_e8p12_cd_polish": (c_int, [c_i64, c_i64, c_i64, c_int, c_i64, c_float, c_ptr, c_ptr, c_ptr, c_ptr,
                                    c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_ptr]),
    "mpq_gemm_f32": (c_int, [c_i64, c_i64, c_i64, c_ptr, c_i64, c_ptr, c_i64, c_int, c_ptr,
                             c_ptr, c_i64, c_float, c_float, c_ptr, c_i64, c_ptr]),
    "mpq_gemm_f32_split_count": (c_int, [c_i64, c_i64, c_i64]),
    "mpq_gemm_f64_workspace_size": (c_i64, [c_i64, c_i64, c_i64]),
    "mpq_gemm_f64": (c_int, [c_i64, c_i64, c_i64, c_ptr, c_i64, c_ptr, c_i64, c_int, c_ptr, c_i64, c_double,
                             c_double, c_ptr, c_i64, c_ptr]),
    "mpq_release_thread_resources": (c_int, []),
    "mpq_permute_columns": (c_int, [c_ptr, c_i64, c_i64, c_ptr, c_ptr, c_int, c_ptr]),
    "mpq_permute_symmetric": (c_int, [c_ptr, c_i64, c_ptr, c_ptr, c_ptr]),
    "mpq_bcd_prepare": (c_int, [c_i64, c_i64, c_int, c_int, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr]),
    "mpq_bcd_gain": (c_int, [c_i64, c_i64, c_int, c_int, c_ptr, c_ptr, c_ptr, c_ptr]),
    "mpq_bcd_target": (c_int, [c_i64, c_i64, c_int, c_i64, c_int, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr]),
    "mpq_bcd_accept": (c_int, [c_i64, c_i64, c_int, c_i64, c_ptr, c_ptr, c_ptr, c_float, c_ptr, c_ptr, c_ptr,
                               c_ptr, c_ptr, c_ptr, c_ptr]),
    "mpq_bcd_uniform_propose": (c_int, [c_i64, c_i64, c_i64, c_int, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr]),
    "mpq_bcd_topk_scalar_propose": (c_int, [c_i64, c_i64, c_i64, c_i64, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr]),
    "mpq_e8p12_metric_argmin_workspace_size": (c_i64, [c_i64]),
    "mpq_e8p12_metric_argmin": (c_int, [c_i64, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_ptr]),
    "mpq_bcd_e8_topk_propose": (c_int, [c_i64, c_i64, c_i64, c_i64, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr]),
    "mpq_gemm_f32_splitk": (c_int, [c_i64, c_i64, c_i64, c_ptr, c_i64, c_ptr, c_i64, c_int, c_ptr, c_int, c_ptr]),
    "mpq_gptq_find_params": (c_int, [c_ptr, c_i64, c_i64, c_i64, c_i64, c_int, c_ptr, c_ptr, c_ptr]),
    "mpq_uniform_rtn": (c_int, [c_ptr, c_i64, c_i64, c_i64, c_ptr, c_ptr, c_i64, c_int, c_ptr, c_ptr,
                                c_ptr]),
    "mpq_awq_workspace_size": (c_i64, [c_i64, c_i64]),
    "mpq_awq_w_mean": (c_int, [c_ptr, c_i64, c_i64, c_i64, c_ptr, c_ptr, c_i64, c_ptr]),
    "mpq_awq_search": (c_int, [c_ptr, c_i64, c_i64, c_ptr, c_ptr, c_ptr, c_i64, c_int, c_int, c_ptr, c_ptr, c_ptr,
                               c_ptr, c_ptr, c_i64, c_ptr]),
    "mpq_hessian_accumulate": (c_int, [c_ptr, c_int, c_i64, c_i64, c_i64, c_float, c_float, c_ptr, c_i64, c_ptr,
                                       c_ptr]),
    "mpq_gptq_pack": (c_int, [c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_int, c_int, c_ptr, c_ptr, c_ptr, c_ptr,
                              c_ptr]),
    "mpq_dequant": (c_int, [c_ptr, c_i64, c_i64, c_ptr, c_ptr, c_i64, c_ptr, c_ptr]),
    "mpq_block_hadamard": (c_int, [c_ptr, c_i64, c_ptr, c_i64, c_i64, c_i64, c_i64, c_ptr, c_int, c_ptr]),
    "mpq_transpose": (c_int, [c_ptr, c_i64, c_i64, c_i64, c_ptr, c_i64, c_ptr]),
    "mpq_syevd_workspace_size": (c_i64, [c_i64]),
    "mpq_syevd": (c_int, [c_i64, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_ptr]),
    "mpq_syevd_method": (c_int, [c_i64, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_int, c_ptr]),
    "mpq_syevd_f64_workspace_size": (c_i64, [c_i64]),
    "mpq_syevd_f64": (c_int, [c_i64, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_ptr]),
    "mpq_scale_columns": (c_int, [c_ptr, c_i64, c_i64, c_ptr, c_ptr, c_ptr]),
    "mpq_eigh_postprocess": (c_int, [c_ptr, c_ptr, c_i64, c_float, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr]),
    "mpq_uniform_denoise": (c_int, [c_i64, c_i64, c_int, c_ptr, c_ptr, c_ptr, c_i64, c_ptr, c_ptr, c_i64,
                                    c_float, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr]),
    "mpq_uniform_vamp_workspace_size": (c_i64, [c_i64, c_i64]),
    "mpq_uniform_vamp_solve": (c_int, [c_i64, c_i64, c_int, c_ptr, c_i64, c_ptr, c_ptr, c_ptr, c_i64,
                                       c_ptr, c_ptr, c_ptr, c_ptr, c_double, c_ptr, c_ptr, c_ptr, c_ptr,
                                       c_ptr, c_ptr, c_i64, c_ptr]),
    "mpq_uniform_cd_workspace_size": (c_i64, [c_i64, c_i64, c_i64]),
    "mpq_uniform_cd_polish": (c_int, [c_i64, c_i64, c_int, c_i64, c_int, c_float, c_ptr, c_i64, c_ptr,
                                      c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_ptr, c_ptr, c_int, c_ptr,
                                      c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_ptr]),
    "mpq_uniform_vamp_solve_ex": (c_int, [c_i64, c_i64, c_int, c_ptr, c_i64, c_ptr, c_ptr, c_ptr, c_i64,
                                          c_ptr, c_ptr, c_ptr, c_ptr, c_double, c_ptr, c_ptr, c_ptr, c_ptr,
                                          c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_ptr]),
    "mpq_gemm_x6_pack_b": (c_int, [c_i64, c_i64, c_ptr, c_i64, c_int, c_ptr, c_ptr]),
    "mpq_gemm_x6_workspace_size": (c_i64, [c_i64, c_i64, c_i64]),
    "mpq_gemm_x6": (c_int, [c_i64, c_i64, c_i64, c_ptr, c_i64, c_ptr, c_ptr, c_i64, c_ptr, c_i64, c_ptr]),
    "mpq_gemm_x6_split_count": (c_int, [c_i64, c_i64, c_i64]),
    "mpq_gemm_x6_packed_a_size": (c_i64, [c_i64, c_i64]),
    "mpq_gemm_x6_pack_a": (c_int, [c_i64, c_i64, c_ptr, c_i64, c_ptr, c_ptr]),
    "mpq_gemm_x6_splitk": (c_int, [c_i64, c_i64, c_i64, c_ptr, c_ptr, c_ptr, c_int, c_ptr]),
    "mpq_rankspace_pack_floats": (c_i64, [c_i64]),
    "mpq_rankspace_pack": (c_int, [c_i64, c_ptr, c_ptr, c_ptr, c_ptr]),
    "mpq_uniform_cd_polish_ex": (c_int, [c_i64, c_i64, c_int, c_i64, c_int, c_float, c_ptr, c_i64, c_ptr,
                                         c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_ptr, c_ptr, c_ptr, c_ptr,
                                         c_int, c_ptr,
                                         c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_ptr]),
    "mpq_uniform_cd_sweeps_workspace_size": (c_i64, [c_i64, c_i64, c_i64]),
    "mpq_uniform_cd_sweeps": (c_int, [c_i64, c_i64, c_int, c_i64, c_int, c_float, c_ptr, c_ptr, c_ptr, c_ptr,
                                      c_ptr, c_ptr, c_ptr, c_i64, c_ptr, c_ptr, c_ptr, c_i64, c_ptr]),
    "mpq_uniform_cd_sweeps_recip": (c_int, [c_i64, c_i64, c_int, c_i64, c_int, c_float, c_ptr, c_ptr, c_ptr, c_ptr,
                                            c_ptr, c_ptr, c_ptr, c_i64, c_ptr, c_ptr, c_ptr, c_i64, c_ptr]),
    "mpq_uniform_cd_sweeps_noalloc_max_bytes": (c_i64, []),
    "mpq_uniform_cd_sweeps_noalloc": (c_int, [c_i64, c_i64, c_int, c_i64, c_int, c_float, c_ptr, c_ptr, c_ptr,
                                              c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_ptr, c_ptr, c_ptr]),
    "mpq_e8p12_posterior_stats": (c_int, [c_ptr, c_i64, c_i64, c_ptr, c_ptr, c_ptr, c_float, c_ptr, c_ptr, c_ptr,
                                          c_ptr]),
}


class UniformVampConfigC(ctypes.Structure):
    """Mirror of MpqUniformVampConfig (include/mpq_amd.h)."""

    _fields_ = [
        ("iters", ctypes.c_int),
        ("damping", ctypes.c_float),
        ("final_decision", ctypes.c_int),
        ("init_from", ctypes.c_int),
        ("gamma_start", ctypes.c_float),
        ("gamma_retry_factor", ctypes.c_float),
        ("gamma_retry_steps", ctypes.c_int),
        ("prior_tau", ctypes.c_float),
        ("obs_precision", ctypes.c_double),
        ("em_obs_precision", ctypes.c_int),
        ("em_obs_precision_damping", ctypes.c_double),
        ("em_obs_precision_min", ctypes.c_double),
        ("em_obs_precision_max", ctypes.c_double),
    ]


class UniformVampStatsC(ctypes.Structure):
    """Mirror of MpqUniformVampStats (include/mpq_amd.h)."""

    _fields_ = [
        ("iters", ctypes.c_int),
        ("best_iter", ctypes.c_int),
        ("stop_iter", ctypes.c_int),
        ("alpha1_retry_count", ctypes.c_int),
        ("alpha2_clip_count", ctypes.c_int),
        ("gamma2_invalid_count", ctypes.c_int),
        ("obs_precision_initial", ctypes.c_double),
        ("obs_precision_final", ctypes.c_double),
        ("obs_precision_mean", ctypes.c_double),
        ("alpha1_mean", ctypes.c_double),
        ("alpha2_mean", ctypes.c_double),
        ("best_rankspace_error_mean", ctypes.c_double),
        ("rtn_rankspace_error_mean", ctypes.c_double),
    ]


class E8P12VampConfigC(ctypes.Structure):
    """Mirror of MpqE8P12VampConfig (include/mpq_amd.h)."""

    _fields_ = [
        ("iters", ctypes.c_int),
        ("damping", ctypes.c_float),
        ("gamma_start", ctypes.c_float),
        ("gamma_retry_factor", ctypes.c_float),
        ("gamma_retry_steps", ctypes.c_int),
        ("prior_tau", ctypes.c_float),
        ("obs_precision", ctypes.c_double),
        ("em_obs_precision", ctypes.c_int),
        ("em_obs_precision_damping", ctypes.c_double),
        ("em_obs_precision_min", ctypes.c_double),
        ("em_obs_precision_max", ctypes.c_double),
        ("best_iterate", ctypes.c_int),
    ]


class E8P12VampStatsC(ctypes.Structure):
    """Mirror of MpqE8P12VampStats (include/mpq_amd.h)."""

    _fields_ = [
        ("iters", ctypes.c_int),
        ("best_iter", ctypes.c_int),
        ("stop_iter", ctypes.c_int),
        ("alpha1_retry_count", ctypes.c_int),
        ("alpha2_clip_count", ctypes.c_int),
        ("gamma2_invalid_count", ctypes.c_int),
        ("obs_precision_initial", ctypes.c_double),
        ("obs_precision_final", ctypes.c_double),
        ("obs_precision_mean", ctypes.c_double),
        ("alpha1_mean", ctypes.c_double),
        ("alpha2_mean", ctypes.c_double),
        ("rankspace_error_mean", ctypes.c_double),
    ]


class MPQLibraryError(RuntimeError):
    """Raised when the HIP library is missing or a C-ABI call reports an error."""


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise MPQLibraryError(
                f"mpq_amd HIP library not found at {LIB_PATH}; build it with "
                "`python -m mpq_amd.build` (or __graft_entry__.build())."
            )
        lib = ctypes.CDLL(LIB_PATH)
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
        atexit.register(_release_at_exit)
        return lib


def _release_at_exit() -> None:
    """Free this thread's pinned host buffers (status mailboxes, staging) while the HIP runtime is
    still up: the library's thread-lifetime allocations are not left to process teardown."""
    lib = _lib
    if lib is None:
        return
    try:
        lib.mpq_release_thread_resources()
    except Exception:  # the interpreter is shutting down; nothing to report to
        pass


def exported_symbols() -> list:
    return sorted(SIGNATURES)


def check(status: int, name: str) -> None:
    if status != 0:
        lib = load()
        msg = lib.mpq_last_error()
        text = msg.decode("utf-8", "replace") if msg else ""
        if status == -1:
            raise ValueError(f"{name}: {text}")
        if status == -4:  # numerical failure, reported as the reference does (RuntimeError)
            raise RuntimeError(text)
        raise MPQLibraryError(f"{name} failed (status {status}): {text}")


# Tensors whose pointers were taken for the next call(): an argument such as ptr(x.contiguous())
# would otherwise free its temporary as soon as the address is read, and a later argument's
# temporary could take the same block before the library reads it.  Kept until the call returns;
# after that the work is enqueued on torch's current stream, whose allocator reuses a freed block
# only for work ordered after it.
_keep = threading.local()


def call(name: str, *args) -> None:
    fn = getattr(load(), name)
    try:
        check(fn(*args), name)
    finally:
        _keep.tensors = []


def ptr(t) -> Optional[int]:
    """Device pointer of a tensor, or None (NULL) for None; `t` stays alive until the next call()."""
    if t is None:
        return None
    held = getattr(_keep, "tensors", None)
    if held is None:
        held = _keep.tensors = []
    held.append(t)
    return int(t.data_ptr())


def stream_handle(device=None) -> int:
    import torch

    return int(torch.cuda.current_stream(device).cuda_stream)
