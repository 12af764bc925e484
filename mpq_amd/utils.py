"""Host-side helpers with the reference's semantics (mpq/utils.py:11-68)."""
from __future__ import annotations

import hashlib
import math


def stable_int_hash(key: str, *, bytes_: int = 8) -> int:
    """Little-endian integer of the first ``bytes_`` bytes of sha256(key) (mpq/utils.py:11-15)."""
    if bytes_ <= 0:
        raise ValueError(f"bytes_ must be > 0, got {bytes_}.")
    digest = hashlib.sha256(str(key).encode("utf-8")).digest()
    return int.from_bytes(digest[: min(bytes_, len(digest))], byteorder="little", signed=False)


def stable_seed(key: str, *, base_seed: int = 0) -> int:
    """31-bit seed derived from a string key (mpq/utils.py:18-22)."""
    return int((int(base_seed) + stable_int_hash(key, bytes_=4)) % (2 ** 31 - 1))


def log_damp_positive_scalar(prev: float, new: float, damping: float) -> float:
    """Geometric damping of a positive scalar (mpq/utils.py:37-46)."""
    damping = float(damping)
    if damping >= 1.0:
        return float(new)
    if damping <= 0.0:
        return float(prev)
    prev = max(float(prev), 1e-12)
    new = max(float(new), 1e-12)
    return float(math.exp((1.0 - damping) * math.log(prev) + damping * math.log(new)))
