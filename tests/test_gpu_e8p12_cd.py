"""GPU parity of the E8P12 gram-metric block-CD polish against the CPU oracle (oracle/e8p12.py
gram_block_cd, which follows mpq/polish/block_cd.py:212-246 and :332-625)."""
import numpy as np
import pytest
import torch

from mpq_amd import codebook, ops
from oracle import e8p12 as oe8
from oracle import uniform as ou
from tests.uniform_cases import make_layer

pytestmark = pytest.mark.gpu


def _eigen_one_thread(H):
    """The oracle's decomposition on one CPU thread: LAPACK's result depends on the thread count
    (sign and rounding of the eigenvectors), so a fixed count keeps the test input the same on
    every machine."""
    prev = torch.get_num_threads()
    torch.set_num_threads(1)
    try:
        return ou.hessian_eigen(H)
    finally:
        torch.set_num_threads(prev)


def _case(rows, n, seed_key, jitter=0.0, with_h=False):
    W, H = make_layer(rows, n, tokens=1024, seed_key=seed_key, heavy=True)
    Wr = W / W.square().mean().sqrt()
    lam, V, _ = _eigen_one_thread(H)
    Vs = V * torch.sqrt(lam).unsqueeze(0)
    grid = torch.from_numpy(codebook.grid_numpy())
    # start from the nearest codeword of a perturbed target so that the polish has work to do
    gen = torch.Generator().manual_seed(rows + n)
    start = Wr + jitter * torch.randn(Wr.shape, generator=gen)
    idx0, _ = oe8.bruteforce_nearest(start.reshape(-1, 8).numpy(), grid.numpy())
    idx0 = torch.from_numpy(np.asarray(idx0)).view(rows, n // 8)
    x0 = grid[idx0.reshape(-1)].view(rows, n)
    if with_h:
        return Wr, Vs, x0, idx0, grid, H
    return Wr, Vs, x0, idx0, grid


def _vs_fp64_rounding(H, Vs):
    """Vs of an fp64 decomposition of the same H (floored as the oracle floors it), columns signed
    like Vs, rounded to fp32: another valid fp32 rounding of the same factorisation."""
    Hd = 0.5 * (H.double() + H.double().T)
    lam, V = torch.linalg.eigh(Hd)
    floor = max(1e-6, 1e-6 * max(float(torch.diagonal(Hd).mean().abs()), float(lam.max()), 1e-12))
    lam, V = lam.clamp_min(floor).flip(0), V.flip(1)
    V64 = V * torch.sqrt(lam).unsqueeze(0)
    sign = torch.sign((V64 * Vs.double()).sum(dim=0))
    sign[sign == 0] = 1.0
    return (V64 * sign.unsqueeze(0)).float()


def _vs_jitter(Vs, seed):
    """Every entry of Vs moved to a random one of its two neighbouring floats or kept (seeded)."""
    gen = torch.Generator().manual_seed(int(seed))
    step = torch.randint(-1, 2, Vs.shape, generator=gen)
    up = torch.nextafter(Vs, torch.full_like(Vs, float("inf")))
    dn = torch.nextafter(Vs, torch.full_like(Vs, float("-inf")))
    return torch.where(step > 0, up, torch.where(step < 0, dn, Vs))


def _oracle_blocks(Wr, Vs, x0, idx0, grid, block_rows, sweeps, max_blocks=0, scores_fp64=False):
    Yu = Wr.matmul(Vs)
    xs, ids = [], []
    for r0 in range(0, Wr.shape[0], block_rows):
        sl = slice(r0, r0 + block_rows)
        x, idx, _ = oe8.gram_block_cd(x0[sl], idx0[sl], Yu[sl], Vs, grid, sweeps, max_blocks=max_blocks,
                                      scores_fp64=scores_fp64)
        xs.append(x)
        ids.append(idx)
    x = torch.cat(xs)
    return x, torch.cat(ids), ou.rankspace_error(Yu, x, Vs)


@pytest.mark.parametrize("rows,n,block_rows,max_blocks", [(64, 256, 64, 0), (200, 128, 64, 0),
                                                           (256, 256, 128, 0), (96, 512, 96, 7)])
def test_polish_matches_oracle(gpu, rows, n, block_rows, max_blocks):
    """Codes agree with the oracle on >= 99.9 % of the blocks, or on at least as many as the oracle
    agrees with itself when only roundings change (the lowest agreement over an fp64 factorisation
    rounded to fp32, two random last-bit roundings of Vs, and the step's argmin scores evaluated in
    fp64 instead of the reference's fp32 matmuls -- the GPU's scores are products of exact bf16
    planes, closer to the latter): greedy block CD turns last-bit differences of the gains and
    scores into different decisions that cascade along a row."""
    Wr, Vs, x0, idx0, grid, H = _case(rows, n, f"e8cd:{rows}:{n}", jitter=0.15, with_h=True)
    ref_x, ref_idx, ref_err = _oracle_blocks(Wr, Vs, x0, idx0, grid, block_rows, 3, max_blocks)
    ctx = ops.e8p12_cd_prepare(Vs.to(gpu))
    x, idx, eb, ea, acc = ops.e8p12_cd_polish(x0.to(gpu), idx0.to(gpu), Vs.to(gpu), ctx, sweeps=3,
                                              block_rows=block_rows, W=Wr.to(gpu), max_blocks=max_blocks)
    x, idx, eb, ea = x.cpu(), idx.cpu(), eb.cpu(), ea.cpu()
    # state consistency: values are the codewords of the indices
    assert torch.equal(x, grid[idx.reshape(-1)].view_as(x))
    Yu = Wr.matmul(Vs)
    e0 = ou.rankspace_error(Yu, x0, Vs)
    assert torch.allclose(eb, e0, rtol=1e-4)
    assert torch.allclose(ea, ou.rankspace_error(Yu, x, Vs), rtol=1e-4)
    # the polish only accepts decreasing moves
    assert bool((ea <= eb * (1 + 1e-5)).all())
    agree = float((idx == ref_idx).float().mean())
    floor = 1.0
    for alt in (_vs_fp64_rounding(H, Vs), _vs_jitter(Vs, 1), _vs_jitter(Vs, 2)):
        _, alt_idx, _ = _oracle_blocks(Wr, alt, x0, idx0, grid, block_rows, 3, max_blocks)
        floor = min(floor, float((alt_idx == ref_idx).float().mean()))
    _, f64_idx, _ = _oracle_blocks(Wr, Vs, x0, idx0, grid, block_rows, 3, max_blocks, scores_fp64=True)
    floor = min(floor, float((f64_idx == ref_idx).float().mean()))
    print(f"codes agree {agree:.5f} (reference floor {floor:.5f}; with the oracle's fp64-score variant "
          f"{float((idx == f64_idx).float().mean()):.5f})")
    assert agree >= min(0.999, floor), (agree, floor)
    rel = abs(float(ea.mean()) - float(ref_err.mean())) / float(ref_err.mean())
    assert rel <= 5e-3, rel
    assert int(acc.sum()) > 0


def test_polish_zero_sweeps_is_identity_and_yu_path(gpu):
    Wr, Vs, x0, idx0, grid = _case(48, 128, "e8cd:id", jitter=0.1)
    ctx = ops.e8p12_cd_prepare(Vs.to(gpu))
    x, idx, eb, ea, acc = ops.e8p12_cd_polish(x0.to(gpu), idx0.to(gpu), Vs.to(gpu), ctx, sweeps=0, block_rows=48,
                                              W=Wr.to(gpu))
    assert torch.equal(x.cpu(), x0) and torch.equal(idx.cpu(), idx0)
    assert torch.equal(eb.cpu(), ea.cpu())
    # Yu given instead of W: identical results
    Yu = ops.gemm(Wr.to(gpu), Vs.to(gpu))
    a = ops.e8p12_cd_polish(x0.to(gpu), idx0.to(gpu), Vs.to(gpu), ctx, sweeps=2, block_rows=48, W=Wr.to(gpu))
    b = ops.e8p12_cd_polish(x0.to(gpu), idx0.to(gpu), Vs.to(gpu), ctx, sweeps=2, block_rows=48, Yu=Yu)
    assert torch.equal(a[1].cpu(), b[1].cpu())


def test_first_step_is_exact_whitened_argmin(gpu):
    """One step (max_blocks=1, one sweep): each row's candidate is the fp64 argmin of
    |L^T (target - c)|^2 over all codewords, up to fp32 near-ties."""
    Wr, Vs, x0, idx0, grid = _case(64, 64, "e8cd:argmin", jitter=0.3)
    rows, n = Wr.shape
    Yu = Wr.matmul(Vs)
    ctx = ops.e8p12_cd_prepare(Vs.to(gpu))
    x, idx, eb, ea, acc = ops.e8p12_cd_polish(x0.to(gpu), idx0.to(gpu), Vs.to(gpu), ctx, sweeps=1, block_rows=rows,
                                              W=Wr.to(gpu), max_blocks=1)
    x = x.cpu()
    changed = (x != x0).any(dim=1)
    blk = int(((x != x0).reshape(rows, n // 8, 8).any(-1).any(0)).nonzero().flatten()[0]) if bool(changed.any()) else None
    assert blk is not None
    # recompute the step in fp64
    R = (Yu - x0.matmul(Vs)).double()
    Vb = Vs[8 * blk:8 * blk + 8].double()
    G = Vb @ Vb.T
    L = torch.linalg.cholesky(G)
    Gi = torch.cholesky_inverse(L)
    rhs = R @ Vb.T
    target = x0[:, 8 * blk:8 * blk + 8].double() + rhs @ Gi
    g64 = grid.double()
    d = ((target @ L).unsqueeze(1) - (g64 @ L).unsqueeze(0)).square().sum(-1)  # rows x 65536
    best = d.argmin(dim=1)
    dmin = d.min(dim=1).values
    got = idx.cpu()[:, blk]
    for r in range(rows):
        if not bool(changed[r]):
            continue
        gi = int(got[r])
        # the chosen codeword is the fp64 argmin, or within fp32 rounding of it
        assert gi == int(best[r]) or float(d[r, gi] - dmin[r]) <= 1e-5 * float(dmin[r] + (target[r] @ L).square().sum())


def test_polish_deterministic_with_more_work_groups_than_fit(gpu):
    """Every greedy step is one launch of row tiles x codeword chunks whose work-groups each finish the
    previous step's decision from all chunks' partial results.  At 16384 rows the launch holds 8192
    work-groups, far more than the GPU runs at once, so early work-groups finish before late ones
    start: the partials of consecutive steps live in separate buffers (by step parity), and the
    result must not depend on the schedule -- two runs agree bit for bit."""
    rows, n = 16384, 256
    W, H = make_layer(512, n, tokens=1024, seed_key="e8cd:det", heavy=True)
    lam, V, _ = _eigen_one_thread(H)
    Vs = (V * torch.sqrt(lam).unsqueeze(0)).to(gpu)
    g = torch.Generator(device=gpu)
    g.manual_seed(17)
    Wr = torch.randn(rows, n, device=gpu, generator=g)
    cb = codebook.E8P12_codebook(gpu)
    x0, idx0 = cb.quantize((Wr + 0.3 * torch.randn(rows, n, device=gpu, generator=g)).reshape(-1, 8))
    x0, idx0 = x0.view(rows, n), idx0.view(rows, n // 8)
    ctx = ops.e8p12_cd_prepare(Vs)
    runs = [ops.e8p12_cd_polish(x0, idx0, Vs, ctx, sweeps=2, block_rows=128, W=Wr) for _ in range(2)]
    (x1, i1, eb1, ea1, a1), (x2, i2, eb2, ea2, a2) = runs
    print(f"16384 rows: accepted {int(a1.sum())}, mean error {float(eb1.mean()):.5g} -> {float(ea1.mean()):.5g}")
    assert int(a1.sum()) > 0
    assert torch.equal(i1, i2) and torch.equal(x1, x2) and torch.equal(ea1, ea2) and torch.equal(a1, a2)
    assert bool((ea1 <= eb1 * (1 + 1e-5)).all())
    assert torch.equal(x1, cb.grid[i1.reshape(-1)].view(rows, n))
