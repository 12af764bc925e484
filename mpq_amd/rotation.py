"""Internal block-Hadamard rotation (reference ``mpq/rotation.py``), HIP kernels.

* ``resolve_block_hadamard_plan`` (reference :42-47): largest power-of-two factor of the width.
* ``sample_rademacher_signs`` (reference :325-340): +-1 signs from a CPU ``torch.Generator``
  seeded with ``stable_seed(key, seed)`` (host-side, identical to the reference).
* ``apply_right_block_hadamard[_inverse]`` (reference :431-438) -> ``mpq_block_hadamard``.
* ``apply_left_block_hadamard`` rotates columns (transpose + rows + transpose), as the
  reference's ``apply_right(X.T).T`` does for H and V (mpq/adapters/gptqmodel.py:727-731, :877-884).
"""
from __future__ import annotations

from typing import Tuple

import torch

from . import ops
from .utils import stable_seed


def largest_pow2_factor(n: int) -> int:
    n = int(n)
    if n <= 0:
        raise ValueError(f"expected positive n, got {n}.")
    return int(n & -n)


def resolve_block_hadamard_plan(width: int) -> Tuple[str, int]:
    had = largest_pow2_factor(int(width))
    if had >= 2:
        return "block", int(had)
    return "none", 1


@torch.inference_mode()
def sample_rademacher_signs(*, width: int, key: str, seed: int = 0, device, dtype=torch.float32) -> torch.Tensor:
    gen = torch.Generator(device="cpu")
    gen.manual_seed(stable_seed(str(key), base_seed=int(seed)))
    signs = torch.randint(0, 2, (int(width),), generator=gen, dtype=torch.int64)
    signs = signs.to(dtype=torch.float32).mul_(2.0).sub_(1.0)
    return signs.to(device=device, dtype=dtype)


@torch.inference_mode()
def apply_block_hadamard(matrix: torch.Tensor, *, had_dim: int) -> torch.Tensor:
    if int(had_dim) <= 1:
        return matrix.to(dtype=torch.float32).contiguous()
    return ops.block_hadamard(matrix, int(had_dim))


@torch.inference_mode()
def apply_right_block_hadamard(matrix: torch.Tensor, *, signs: torch.Tensor, had_dim: int) -> torch.Tensor:
    return ops.block_hadamard(matrix, int(had_dim), signs=signs, inverse=False)


@torch.inference_mode()
def apply_right_block_hadamard_inverse(matrix: torch.Tensor, *, signs: torch.Tensor, had_dim: int) -> torch.Tensor:
    return ops.block_hadamard(matrix, int(had_dim), signs=signs, inverse=True)


@torch.inference_mode()
def apply_left_block_hadamard(matrix: torch.Tensor, *, signs: torch.Tensor, had_dim: int) -> torch.Tensor:
    """Rotate every column: equals ``apply_right_block_hadamard(matrix.T).T`` bit for bit."""
    t = ops.transpose(matrix)
    t = ops.block_hadamard(t, int(had_dim), signs=signs, inverse=False)
    return ops.transpose(t)
