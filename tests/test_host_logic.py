"""CPU: host-side logic of the product that needs no GPU -- the QUIP# checkpoint writer's rotation
plan (fail closed on widths whose quip-sharp transform is not provided) and the library's release of
its per-thread pinned buffers (a no-op before any GPU call)."""
import os

import pytest

from mpq_amd import _lib, quip_ckpt


def test_hadamard_plan_power_of_two_and_fail_closed():
    assert quip_ckpt.hadamard_plan(2048) == (2048, "")
    assert quip_ckpt.hadamard_plan(1) == (1, "")
    # fused qkv of config 3 (3072 = 12 x 256) and 14336 = 28 x 512: quip-sharp's had-K widths
    for w, blk in ((3072, 1024), (14336, 2048), (384, 128)):
        with pytest.raises(ValueError, match="had-K"):
            quip_ckpt.hadamard_plan(w)
        had, reason = quip_ckpt.hadamard_plan(w, allow_block=True)
        assert had == blk and str(blk) in reason
    with pytest.raises(ValueError):
        quip_ckpt.hadamard_plan(0)


def test_saved_rotation_family_is_checked():
    # the decoder takes each side's transform from the checkpoint's family, and refuses what it cannot do
    assert quip_ckpt._saved_had_dim({"left_rotation_family": "had"}, "left", 4096) == 4096
    assert quip_ckpt._saved_had_dim({"left_rotation_family": "block_had", "left_had_dim": 1024}, "left", 3072) == 1024
    with pytest.raises(ValueError, match="had-K"):
        quip_ckpt._saved_had_dim({"left_rotation_family": "had"}, "left", 3072)
    with pytest.raises(ValueError, match="does not tile"):
        quip_ckpt._saved_had_dim({"left_rotation_family": "block_had", "left_had_dim": 2048}, "left", 3072)
    with pytest.raises(ValueError, match="unknown"):
        quip_ckpt._saved_had_dim({"right_rotation_family": "kron"}, "right", 64)


def test_release_thread_resources_without_gpu_work():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libmpq_amd.so not built")
    lib = _lib.load()
    # nothing was allocated on this thread: nothing to free, no HIP call made
    assert lib.mpq_release_thread_resources() == 0
    assert lib.mpq_release_thread_resources() == 0
