"""CPU: pins the oracle's per-linear scalar driver (oracle/uniform.py run_mpq_quantization, following
mpq/adapters/gptqmodel.py:650-1163) and its rotation signs against vectors the reference itself wrote
(tests/golden/make_golden.py ``udriver``: the reference's run_mpq_quantization on its CPU dispatch,
with GPTQModel's quantizer replaced by the same min-max formula, 384 x 256, three 128-row blocks).

Checked exactly: the rotation signs (mpq/rotation.py:325-340 seeded by mpq/utils.py:18-22), the
group scale/zero, the warm-start precision summed over row blocks (:920-941), the precision carried
block to block (:1065-1066), each block's best/stop iteration, the codes q_int and the eigenvalue
floor of the unrotated Hessian (:702-722)."""
import os

import numpy as np
import pytest
import torch

from oracle import uniform as ou
from tests.uniform_cases import RECIPE, make_layer

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
NAME = "model.layers.0.mlp.up_proj"


def test_rotation_plan_reproduces_reference_signs():
    d = np.load(os.path.join(HERE, "rademacher_signs.npz"))
    assert len(d.files) == 6
    for k in d.files:
        _, key, width = k.split("|")
        signs, had = ou.rotation_plan(int(width), key)
        assert had == int(width)
        assert np.array_equal(signs.numpy(), d[k]), k


@pytest.mark.parametrize("rotation,desc_act", [("none", False), ("internal_hadamard", False),
                                               ("internal_hadamard", True)])
def test_driver_reproduces_reference(rotation, desc_act):
    tag = rotation + ("_desc_act" if desc_act else "")
    d = np.load(os.path.join(HERE, f"udriver_{tag}.npz"))
    bits = int(d["bits"])
    W, _ = make_layer(384, 256, tokens=1024, seed_key=f"golden:udriver:{tag}")
    H = torch.from_numpy(d["H"])
    prev = torch.get_num_threads()
    torch.set_num_threads(1)  # the reference's vectors were written on one thread
    try:
        r = ou.run_mpq_quantization(W, H, bits, 128, NAME, dict(RECIPE), rotation=rotation, polish="block_cd",
                                    desc_act=desc_act)
        _, _, floor = ou.hessian_eigen(0.5 * H)
    finally:
        torch.set_num_threads(prev)
    if desc_act:  # decomposed after the rotation and the column order (mpq/adapters/gptqmodel.py:716-722, :886-892)
        floor = r["eigen_floor"]
    assert np.array_equal(r["scale"].numpy(), d["scale"])
    assert np.array_equal(r["zero"].numpy(), d["zero"])
    assert np.array_equal(r["g_idx"].numpy(), d["g_idx"])
    assert r["obs_initial"] == float(d["obs_initial"])
    assert [t["best_iter"] for t in r["traces"]] == d["block_best_iter"].tolist()
    assert [t["stop_iter"] for t in r["traces"]] == d["block_stop_iter"].tolist()
    assert r["obs_final"] == float(d["obs_final"])
    assert floor == float(d["eigen_floor"])
    agree = float((r["q_int"].numpy() == d["q_int"]).mean())
    assert agree == 1.0, agree
    # Q is the inverse rotation of the dequantised codes, as the reference returns it
    assert float(np.abs(r["Q"].numpy() - d["Q"]).max()) <= 1e-6 * float(np.abs(d["Q"]).max())


def test_driver_golden_catches_a_per_block_warm_start():
    """A plausible slip -- the warm start from the first row block only instead of the sum over all
    blocks -- moves the initial precision off the reference's value."""
    d = np.load(os.path.join(HERE, "udriver_internal_hadamard.npz"))
    bits = int(d["bits"])
    W, _ = make_layer(384, 256, tokens=1024, seed_key="golden:udriver:internal_hadamard")
    H = torch.from_numpy(d["H"])
    prev = torch.get_num_threads()
    torch.set_num_threads(1)
    try:
        r = ou.run_mpq_quantization(W[:128], H, bits, 128, NAME, dict(RECIPE, iters=0, polish_sweeps=0),
                                    rotation="internal_hadamard", polish="block_cd")
    finally:
        torch.set_num_threads(prev)
    assert r["obs_initial"] != float(d["obs_initial"])
