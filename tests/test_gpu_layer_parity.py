"""Whole-layer parity at BASELINE config 0's real size (1024 x 1024, 4096 tokens, 4-bit, group 128,
VAMP + 3 CD sweeps, 128-row blocks) against the oracle, over five seeds and both rotations.

The oracle follows the reference's CUDA dispatch order (``polish="twin"``).  Code agreement has a floor
that the reference itself sets: VAMP's best-iterate stop and the greedy CD's shared column order turn
last-bit differences of any product into different discrete decisions for whole row blocks.  The floor
of a seed comes from the agreements the reference shows with itself on that input:

* its two CD dispatches (the CUDA sweep and the CPU block CD, mpq/solver.py:299-366);
* the CUDA-order solve with the greedy gain summed in row order instead of torch's reduction order;
* that solve with every product rounded from fp64 (``oracle.uniform.products_in_fp64``): another
  valid fp32 rounding of the same algorithm, the kind of difference the GPU's products have;
* the unchanged oracle with another BLAS thread count: its products' sums partitioned differently.
  On these layers that alone moves whole row blocks (one block's best-iterate stop moves from
  iteration 3 to 11 on seed 4 with internal Hadamard): the oracle agrees with itself on only ~94.6 %
  of the codes between 8, 4 and 1 threads there.

The floor of a seed is the lowest of these agreements.  Two further variants, with every product
entry then moved at random to a neighbouring float, are printed for information only.

Codes must agree with the oracle on >= 99.9 % of entries or, averaged over the five seeds, on at least
as many entries as the reference's floor.  The proxy loss tr((W-Q)H(W-Q)^T) must be within 0.5 % of
the oracle's for every seed.
"""
import pytest
import torch

from mpq_amd import ops
from mpq_amd.adapters.gptqmodel import GPTQAdapterConfig, run_mpq_quantization, vamp_hessian_eigen
from mpq_amd.solver import UniformVampConfig
from oracle import uniform as ou
from tests.uniform_cases import RECIPE, QCfg, make_layer

pytestmark = pytest.mark.gpu

NAME = "model.layers.0.mlp.up_proj"
SEEDS = range(5)
_RESULTS = {}


def _case(seed):
    W, H = make_layer(1024, 1024, tokens=4096, seed_key=f"cfg0:{seed}")
    return W, 2.0 * H  # GPTQModel convention; the adapter halves it (mpq/adapters/gptqmodel.py:702)


def _gpu_layer(gpu, W, Hg, rotation, eigen=None):
    return run_mpq_quantization(W=W.to(gpu), H=Hg.to(gpu), quantizer=None, qcfg=QCfg(4, 128, rotation),
                                module_name=NAME, vamp_cfg=UniformVampConfig(**RECIPE),
                                adapter_cfg=GPTQAdapterConfig(block_rows=128, eigen_cache=False),
                                precomputed_eigen=eigen)


def _oracle(W, Hg, rotation, **kw):
    return ou.run_mpq_quantization(W, Hg, 4, 128, NAME, RECIPE, rotation=rotation, **kw)


def _agree(a, b):
    return float((a == b).float().mean())


@pytest.mark.parametrize("rotation", ["none", "internal_hadamard"])
@pytest.mark.parametrize("seed", SEEDS)
def test_config0_layer_matches_oracle(gpu, rotation, seed):
    W, Hg = _case(seed)
    ref = _oracle(W, Hg, rotation)
    lam, V, _ = ou.hessian_eigen(0.5 * Hg)
    Q, q, s, z, g_idx, _, st = _gpu_layer(gpu, W, Hg, rotation, eigen=(lam, V))
    agree = _agree(q.cpu(), ref["q_int"])
    proxy_ref = float(ref["proxy_rows"].sum())
    rel = (st["proxy_loss"] - proxy_ref) / proxy_ref
    floor, jit = 1.0, []
    if agree < 0.999:
        variants = [_oracle(W, Hg, rotation, polish="block_cd"), _oracle(W, Hg, rotation, polish="twin_rowsum")]
        with ou.products_in_fp64():
            variants.append(_oracle(W, Hg, rotation, polish="twin_rowsum"))
        # the same oracle code with another BLAS thread count (another partition of every product's sums)
        prev = torch.get_num_threads()
        torch.set_num_threads(4 if prev != 4 else 2)
        try:
            variants.append(_oracle(W, Hg, rotation))
        finally:
            torch.set_num_threads(prev)
        floor = min(_agree(v["q_int"], ref["q_int"]) for v in variants)
        # reported only: the fp64 products moved at random to a neighbouring float
        for js in (1, 2):
            with ou.products_in_fp64(jitter_seed=js):
                jit.append(_agree(_oracle(W, Hg, rotation, polish="twin_rowsum")["q_int"], ref["q_int"]))
    _RESULTS[(rotation, seed)] = (agree, floor)
    print(f"seed {seed} {rotation}: codes {agree:.5f} (reference floor {floor:.5f}; last-bit jitter variants "
          f"{' '.join(f'{j:.5f}' for j in jit) or '-'}), proxy {rel:+.5f}")
    assert torch.equal(s.cpu(), ref["scale"]) and torch.equal(z.cpu(), ref["zero"])
    assert torch.equal(g_idx.cpu(), torch.arange(1024, dtype=torch.int32) // 128)
    assert abs(rel) <= 0.005
    # Q is the inverse rotation of the dequantised codes
    sf = torch.repeat_interleave(s.cpu(), 128, dim=1)
    zf = torch.repeat_interleave(z.cpu(), 128, dim=1)
    Qw = sf * (q.cpu().float() - zf)
    if rotation == "internal_hadamard":
        signs, had = ou.rotation_plan(1024, NAME)
        Qw = ou.hadamard_rows(Qw, had) * signs.view(1, -1)
    assert float((Q.cpu() - Qw).abs().max()) <= 1e-6 * float(Qw.abs().max())


@pytest.mark.parametrize("rotation", ["none", "internal_hadamard"])
def test_config0_code_agreement_within_reference_floor(gpu, rotation):
    got = [_RESULTS.get((rotation, s)) for s in SEEDS]
    if any(r is None for r in got):
        pytest.skip("needs every seed of test_config0_layer_matches_oracle in the same session")
    mean_agree = sum(a for a, _ in got) / len(got)
    mean_floor = sum(f for _, f in got) / len(got)
    print(f"{rotation}: mean code agreement {mean_agree:.5f}, mean reference floor {mean_floor:.5f}")
    assert mean_agree >= min(0.999, mean_floor)


@pytest.mark.parametrize("rotation", ["none", "internal_hadamard"])
@pytest.mark.parametrize("seed", SEEDS)
def test_config0_layer_device_eigh(gpu, rotation, seed):
    """The shipped path: the device eigensolver (mpq_syevd) instead of the oracle's LAPACK ssyevd.

    1. The device decomposition of this Hessian is as accurate as LAPACK's fp32 one (reconstruction,
       orthogonality and eigenvalue errors against fp64 within 2x of LAPACK's).
    2. Given that decomposition, the GPU layer matches the oracle fed the same decomposition: proxy
       loss within 0.5 %.
    3. Against the LAPACK-based oracle the proxy loss is within 0.5 %, or else the oracle itself moves
       by that much when only the decomposition is swapped (two equally accurate fp32 eigenbases can
       stop VAMP's best-iterate rule at different iterations): the GPU then stays within 0.5 % of
       that moved oracle.
    """
    W, Hg = _case(seed)
    Hw = 0.5 * Hg
    lam_d, S_d, V_d, Vs_d, fl = vamp_hessian_eigen(Hw.to(gpu), use_cache=False)
    # (1) accuracy against fp64, compared with LAPACK's fp32 ssyevd on the same matrix
    lam64, V64 = torch.linalg.eigh(Hw.double())
    lam32, V32 = torch.linalg.eigh(Hw)
    la_asc, Va_asc = ops.syevd(Hw.to(gpu))

    def errs(l, V):
        l, V = l.double().cpu(), V.double().cpu()
        rec = float((V @ torch.diag(l) @ V.T - Hw.double()).norm() / Hw.double().norm())
        orth = float((V.T @ V - torch.eye(V.shape[0], dtype=torch.float64)).abs().max())
        ev = float((l - lam64).abs().max() / lam64.abs().max())
        return rec, orth, ev

    e_dev, e_lap = errs(la_asc, Va_asc), errs(lam32, V32)
    for d, lp in zip(e_dev, e_lap):
        assert d <= 2.0 * lp + 1e-12, (e_dev, e_lap)
    # (2) the layer against the oracle fed the same decomposition
    Q, q, s, z, g_idx, _, st = _gpu_layer(gpu, W, Hg, rotation)
    orig = ou.hessian_eigen
    ou.hessian_eigen = lambda H, jitter_base=1e-6, floor_scale=1e-6: (lam_d.cpu(), V_d.cpu(), fl)
    try:
        ref_dev = _oracle(W, Hg, rotation)
    finally:
        ou.hessian_eigen = orig
    p_dev = float(ref_dev["proxy_rows"].sum())
    rel_same = (st["proxy_loss"] - p_dev) / p_dev
    assert abs(rel_same) <= 0.005
    # (3) against the LAPACK-based oracle
    ref = _oracle(W, Hg, rotation)
    p_ref = float(ref["proxy_rows"].sum())
    rel = (st["proxy_loss"] - p_ref) / p_ref
    shift = (p_dev - p_ref) / p_ref
    print(f"seed {seed} {rotation} device eigh: proxy {rel:+.5f} vs LAPACK oracle, {rel_same:+.5f} vs oracle on "
          f"the device eigenbasis (oracle's own shift {shift:+.5f}); codes {_agree(q.cpu(), ref['q_int']):.5f}")
    assert torch.equal(s.cpu(), ref["scale"]) and torch.equal(z.cpu(), ref["zero"])
    # within 0.5 % of the LAPACK-based oracle, or -- when the oracle itself moves by more than that on
    # the device eigenbasis -- within 0.5 % of the moved oracle and no further from the LAPACK-based
    # one than that move plus 0.5 %
    assert abs(rel) <= 0.005 or (abs(rel_same) <= 0.005 <= abs(shift) and abs(rel) <= abs(shift) + 0.005)
