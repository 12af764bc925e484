"""CPU: pin the E8P12 oracle (table structure, factor cache, factorized MAP)."""
import numpy as np
import torch

from mpq_amd import codebook
from oracle import e8p12 as oe8


def test_table_counts_and_lattice_membership():
    t = codebook.ABS2_TABLE.astype(np.int64)
    sq4 = (t * t).sum(axis=1)
    assert t.shape == (256, 8)
    assert int((sq4 <= 40).sum()) == 227  # 1+8+28+56+70+8+56 points of D8+1/2, |x|^2 <= 10
    assert int((sq4 == 48).sum()) == 29
    assert len({tuple(r) for r in t.tolist()}) == 256
    assert list(map(tuple, t.tolist())) == sorted(map(tuple, t.tolist()))  # lexicographic
    g = codebook.grid_numpy().astype(np.float64)
    assert len(np.unique(g, axis=0)) == 65536
    # every codeword minus its shift is a point of D8 + 1/2 with even coordinate sum
    idx = np.arange(65536)
    branch = np.array([bin(s).count("1") & 1 for s in (idx & 255)])
    shift = np.where(branch == 0, 0.25, -0.25)
    core = g - shift[:, None]
    assert np.all(np.abs(core * 2 - np.round(core * 2)) == 0)
    assert np.all(np.round(core * 2) % 2 != 0)
    assert np.all(np.round(core.sum(axis=1)) % 2 == 0)


def test_factor_cache_invariants_and_index_formula():
    cache = oe8.factor_cache(torch.from_numpy(codebook.grid_numpy()))
    lut = cache["idx_lut"].numpy()
    par = codebook.base_parity()
    assert np.array_equal(cache["base_parity"].numpy(), par)
    assert np.allclose(cache["base_abs"].numpy(), codebook.ABS2_TABLE * 0.5)
    rng = np.random.default_rng(0)
    for _ in range(2000):
        br, k = int(rng.integers(2)), int(rng.integers(256))
        sign = int(rng.integers(256))
        if bin(sign).count("1") % 2 != par[k]:
            sign ^= 1
        assert lut[br, k, sign] == codebook.index_of(br, k, sign)


def test_factorized_map_equals_bruteforce_nearest():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3000, 8)).astype(np.float32) * 1.2
    cache = oe8.factor_cache(torch.from_numpy(codebook.grid_numpy()))
    idx, score = oe8.map_search(x, np.ones(1, np.float32), 3000, cache)
    bidx, bdist = oe8.bruteforce_nearest(x, codebook.grid_numpy())
    g = codebook.grid_numpy().astype(np.float64)
    d_fact = ((x.astype(np.float64) - g[idx]) ** 2).sum(axis=1)
    # same codeword, or an exact/near tie in distance
    same = idx == bidx
    assert same.mean() > 0.999
    assert np.allclose(d_fact[~same], bdist[~same], rtol=1e-5, atol=1e-5)
    # with unit precision the best score is -1/2 * squared distance
    assert np.allclose(score, -0.5 * d_fact, rtol=1e-5, atol=1e-5)


def test_map_precision_invariance_and_prior_folding():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((512, 8)).astype(np.float32)
    cache = oe8.factor_cache(torch.from_numpy(codebook.grid_numpy()))
    i1, _ = oe8.map_search(x, np.ones(1, np.float32), 512, cache)
    i4, _ = oe8.map_search(x, np.full(1, 4.0, np.float32), 512, cache)  # power of 2: exact scaling
    assert np.array_equal(i1, i4)
    # prior folding with a centre equal to the input leaves the argmin unchanged
    center = x.copy()
    ip, _ = oe8.map_search(x, np.full(8, 3.0, np.float32), 64, cache, center=center, tau=0.25)
    assert np.array_equal(ip, i1)


def test_planted_mistake_is_caught():
    """A wrong parity convention in the oracle must break agreement with brute force."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal((500, 8)).astype(np.float32)
    cache = oe8.factor_cache(torch.from_numpy(codebook.grid_numpy()))
    bad = dict(cache)
    bad["base_parity"] = (1 - cache["base_parity"]).to(torch.int32)
    bad_lut = cache["idx_lut"].clone()
    bad_lut[bad_lut < 0] = 0
    bad["idx_lut"] = bad_lut
    idx, _ = oe8.map_search(x, np.ones(1, np.float32), 500, bad)
    bidx, _ = oe8.bruteforce_nearest(x, codebook.grid_numpy())
    assert (idx == bidx).mean() < 0.9
