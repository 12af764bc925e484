"""GPU parity: E8P12 MAP kernel vs the C oracle (bit-exact indices, scores, errors)."""
import numpy as np
import pytest
import torch

from mpq_amd import codebook
from mpq_amd.priors import e8p12 as ke8
from oracle import e8p12 as oe8

pytestmark = pytest.mark.gpu

GRID = codebook.grid_numpy()


@pytest.fixture(scope="module")
def cache():
    return oe8.factor_cache(torch.from_numpy(GRID))


def _run(x, gamma, gamma_div, dev, center=None, tau=0.0, scale=None):
    xt = torch.from_numpy(x).to(dev)
    gt = torch.from_numpy(gamma).to(dev)
    ct = None if center is None else torch.from_numpy(center).to(dev)
    st = None if scale is None else torch.from_numpy(scale).to(dev)
    out = ke8.e8p12_map_flat(xt, gt, gamma_div=gamma_div, center=ct, scale=st, tau=tau,
                             want_idx16=True, want_vals=True, want_err=True, want_score=True)
    torch.cuda.synchronize()
    return {k: v.cpu().numpy() for k, v in out.items()}


@pytest.mark.parametrize("scale", [1.0, 0.3, 7.0])
def test_unit_precision_bit_exact(gpu, cache, scale):
    rng = np.random.default_rng(10)
    n = 1 << 18
    x = (rng.standard_normal((n, 8)) * scale).astype(np.float32)
    out = _run(x, np.ones(1, np.float32), n, gpu)
    idx, score = oe8.map_search(x, np.ones(1, np.float32), n, cache)
    assert np.array_equal(out["idx"], idx)
    assert np.array_equal(out["idx16"].astype(np.int64), idx & 0xFFFF)
    assert np.array_equal(out["score"].view(np.uint32), score.view(np.uint32))
    assert np.array_equal(out["vals"], GRID[idx])
    assert np.array_equal(out["err"].view(np.uint32), oe8.sqerr(x, idx, GRID).view(np.uint32))


def test_one_lane_path_bit_exact(gpu, cache):
    """From 2^19 vectors the kernel searches one vector per lane; below, four waves split each
    vector's search (every other test here).  Both must give the oracle's results bit for bit."""
    rng = np.random.default_rng(14)
    n = (1 << 19) + 77
    x = (rng.standard_normal((n, 8)) * 1.3).astype(np.float32)
    out = _run(x, np.ones(1, np.float32), n, gpu)
    idx, score = oe8.map_search(x, np.ones(1, np.float32), n, cache)
    assert np.array_equal(out["idx"], idx)
    assert np.array_equal(out["score"].view(np.uint32), score.view(np.uint32))
    assert np.array_equal(out["err"].view(np.uint32), oe8.sqerr(x, idx, GRID).view(np.uint32))


def test_row_precision_and_prior_bit_exact(gpu, cache):
    rng = np.random.default_rng(11)
    rows, nb = 64, 512
    x = rng.standard_normal((rows * nb, 8)).astype(np.float32)
    gamma = np.exp(rng.standard_normal(rows) * 2).astype(np.float32)
    out = _run(x, gamma, nb, gpu)
    idx, score = oe8.map_search(x, gamma, nb, cache)
    assert np.array_equal(out["idx"], idx)
    assert np.array_equal(out["score"].view(np.uint32), score.view(np.uint32))
    center = (x + 0.3 * rng.standard_normal(x.shape)).astype(np.float32)
    for scl in (None, np.abs(rng.standard_normal(rows * nb)).astype(np.float32) + 0.1):
        out = _run(x, gamma, nb, gpu, center=center, tau=0.25, scale=scl)
        idx, score = oe8.map_search(x, gamma, nb, cache, center=center, scale=scl, tau=0.25)
        assert np.array_equal(out["idx"], idx)
        assert np.array_equal(out["score"].view(np.uint32), score.view(np.uint32))


def test_ties_codewords_zeros_and_tiny_precision(gpu, cache):
    rng = np.random.default_rng(12)
    pick = rng.integers(0, 65536, size=(4096, 2))
    exact = GRID[pick[:, 0]]
    mid = 0.5 * (GRID[pick[:, 0]] + GRID[pick[:, 1]])  # equidistant points: ties
    zeros = np.zeros((64, 8), np.float32)
    quarter = np.full((64, 8), 0.25, np.float32)  # equidistant from many codewords
    x = np.concatenate([exact, mid, zeros, quarter]).astype(np.float32)
    out = _run(x, np.ones(1, np.float32), x.shape[0], gpu)
    idx, score = oe8.map_search(x, np.ones(1, np.float32), x.shape[0], cache)
    assert np.array_equal(out["idx"], idx)
    assert np.array_equal(out["idx"][:4096], pick[:, 0])
    # denormal precisions exercise the exact per-base fallback of the kernel
    gamma = np.array([1e-44, 1e-40, 1e-38, 3e-39], np.float32)
    x2 = rng.standard_normal((4 * 256, 8)).astype(np.float32)
    out = _run(x2, gamma, 256, gpu)
    idx, score = oe8.map_search(x2, gamma, 256, cache)
    assert np.array_equal(out["idx"], idx)
    assert np.array_equal(out["score"].view(np.uint32), score.view(np.uint32))


def test_unaligned_and_empty(gpu, cache):
    rng = np.random.default_rng(13)
    n = 1000
    buf = torch.from_numpy(rng.standard_normal(n * 8 + 1).astype(np.float32)).to(gpu)
    xt = buf[1:].view(n, 8)  # 4-byte aligned only: scalar-load path
    out = ke8.e8p12_map_flat(xt, torch.ones(1, device=gpu), gamma_div=n)
    idx, _ = oe8.map_search(xt.cpu().numpy(), np.ones(1, np.float32), n, cache)
    assert np.array_equal(out["idx"].cpu().numpy(), idx)
    empty = ke8.e8p12_map_flat(torch.empty(0, 8, device=gpu), torch.ones(1, device=gpu))
    assert empty["idx"].numel() == 0


def test_codebook_quantize_and_reference_signature(gpu, cache):
    rng = np.random.default_rng(14)
    W = torch.from_numpy(rng.standard_normal((32, 64)).astype(np.float32)).to(gpu)
    cb = codebook.E8P12_codebook(device=gpu)
    vals, idx = cb.quantize(W.reshape(-1, 8), return_idx=True)
    ref_idx, _ = oe8.map_search(W.reshape(-1, 8).cpu().numpy(), np.ones(1, np.float32), 256, cache)
    assert np.array_equal(idx.cpu().numpy(), ref_idx)
    gamma = torch.full((32, 1), 2.0, device=gpu)
    out = ke8.vamp_vector_map_e8p12(r1_blocks=W.view(32, 8, 8), gamma1=gamma, cb=cb,
                                    prior_center_blocks=W.view(32, 8, 8) * 0.9, prior_tau=0.25)
    ref_idx, _ = oe8.map_search(W.reshape(-1, 8).cpu().numpy(), np.full(32, 2.0, np.float32), 8, cache,
                                center=(W * 0.9).reshape(-1, 8).cpu().numpy(), tau=0.25)
    assert np.array_equal(out["map_idxs"].reshape(-1).cpu().numpy(), ref_idx)
    # need_stats adds the mean margin between the two best candidate log-scores (:541-631 with
    # need_stats): against the oracle's per-block margins
    st = ke8.vamp_vector_map_e8p12(r1_blocks=W.view(32, 8, 8), gamma1=gamma, cb=cb, need_stats=True)
    assert torch.equal(st["map_idxs"], ke8.vamp_vector_map_e8p12(r1_blocks=W.view(32, 8, 8), gamma1=gamma,
                                                                  cb=cb)["map_idxs"])
    ref = oe8.posterior(W.view(32, 8, 8).cpu(), gamma.cpu(), cache, need_stats=True)
    ref_margin = float(ref["margin"].double().mean())
    assert abs(st["margin"] - ref_margin) <= 1e-4 * (1.0 + abs(ref_margin))
    with pytest.raises(ValueError):
        ke8.vamp_vector_map_e8p12(r1_blocks=W.view(32, 8, 8), gamma1=gamma[:4], cb=cb)
