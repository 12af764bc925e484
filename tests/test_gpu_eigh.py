"""GPU: symmetric eigendecomposition (mpq_syevd: one-stage tridiagonalisation or the two-stage band
reduction with bulge chasing, divide and conquer on the tridiagonal matrix, back-transformation on
this library's MFMA GEMM) against fp64 LAPACK on the CPU, with the fp32 accuracy of
torch.linalg.eigh on the same GPU as the yardstick for residual and orthogonality.  Both reductions
are tested explicitly (mpq_syevd_method 1 and 2) at the sizes the automatic choice does not pick."""
import pytest
import torch

from mpq_amd import ops
from tests.uniform_cases import make_layer

pytestmark = pytest.mark.gpu


def _quality(H, lam, V):
    n = H.shape[0]
    Hd, lam, V = H.double().cpu(), lam.double().cpu(), V.double().cpu()
    resid = float((Hd @ V - V * lam.unsqueeze(0)).norm() / Hd.norm())
    orth = float((V.T @ V - torch.eye(n, dtype=torch.float64)).abs().max())
    return resid, orth


@pytest.mark.parametrize("method", [1, 2])
@pytest.mark.parametrize("n", [256, 1000, 2048, 4100])
def test_syevd_matches_fp64(gpu, n, method):
    _, H = make_layer(8, n, tokens=2 * n, seed_key=f"eigh:{n}")
    Hg = H.to(gpu)
    lam, V = ops.syevd(Hg, method=method)
    ref = torch.linalg.eigvalsh(H.double())
    scale = float(ref.abs().max())
    assert float((lam.cpu().double() - ref).abs().max()) <= 2e-5 * scale
    assert bool((lam[1:] >= lam[:-1]).all())
    resid, orth = _quality(H, lam, V)
    lt, Vt = torch.linalg.eigh(Hg)
    resid_t, orth_t = _quality(H, lt, Vt)
    assert resid <= max(2.0 * resid_t, 1e-5), (resid, resid_t)
    assert orth <= max(2.0 * orth_t, 2e-5), (orth, orth_t)


def test_syevd_two_stage_8192(gpu):
    """Two-stage path (the automatic choice from n = 1024) at a size where stage 1 runs in panel pairs
    with 256-row X tiles (255 panels: 127 pairs and a last panel alone) and Q1 in block pairs (64
    blocks of 128 reflectors): eigenvalues against fp64 eigvalsh, residual and orthogonality against
    torch's fp32 eigh, all on the GPU (H = X^T X / 2n with log-normal channel scales)."""
    n = 8192
    g = torch.Generator(device=gpu).manual_seed(8192)
    c = torch.exp(torch.randn(n, generator=g, device=gpu))
    X = torch.randn(2 * n, n, generator=g, device=gpu) * c
    H = X.T @ X / (2 * n)
    del X
    H = 0.5 * (H + H.T)
    lam, V = ops.syevd(H)
    ref = torch.linalg.eigvalsh(H.double())
    scale = float(ref.abs().max())
    assert float((lam.double() - ref).abs().max()) <= 2e-5 * scale
    assert bool((lam[1:] >= lam[:-1]).all())

    def quality(lv, Vv):
        Hd, Vd = H.double(), Vv.double()
        resid = float((Hd @ Vd - Vd * lv.double().unsqueeze(0)).norm() / Hd.norm())
        orth = float((Vd.T @ Vd - torch.eye(n, dtype=torch.float64, device=gpu)).abs().max())
        return resid, orth

    resid, orth = quality(lam, V)
    lt, Vt = torch.linalg.eigh(H)
    resid_t, orth_t = quality(lt, Vt)
    assert resid <= max(2.0 * resid_t, 1e-5), (resid, resid_t)
    assert orth <= max(2.0 * orth_t, 2e-5), (orth, orth_t)


def test_syevd_large_remainder_paths(gpu):
    # n = 17000: the first trailing matrices exceed the tridiagonalisation kernels' fixed load
    # batches (over 512 norm partials, 8192 symv partials and 256 column strips), so their
    # remainder loops run.  Yardstick: torch's fp32 eigh on the same GPU; residual and
    # orthogonality in fp64 on the GPU.
    n = 17000
    g = torch.Generator(device=gpu).manual_seed(17000)
    X = torch.randn(2 * n, n, generator=g, device=gpu) * torch.exp(torch.randn(n, generator=g, device=gpu))
    Hg = X.T @ X / (2 * n)
    del X
    Hg = 0.5 * (Hg + Hg.T)
    lam, V = ops.syevd(Hg)
    lt = torch.linalg.eigvalsh(Hg)
    scale = float(lt.abs().max())
    assert float((lam - lt).abs().max()) <= 2e-5 * scale
    assert bool((lam[1:] >= lam[:-1]).all())
    Hd, Vd = Hg.double(), V.double()
    resid = float((Hd @ Vd - Vd * lam.double().unsqueeze(0)).norm() / Hd.norm())
    orth = float((Vd.T @ Vd - torch.eye(n, dtype=torch.float64, device=gpu)).abs().max())
    assert resid < 1e-4 and orth < 1e-4, (resid, orth)


def test_syevd_small_and_diagonal(gpu):
    # n = 1, 2 (no or one reflector), a diagonal matrix (all reflectors trivial), repeated eigenvalues
    for H in (torch.tensor([[3.0]]), torch.tensor([[2.0, 1.0], [1.0, 2.0]]),
              torch.diag(torch.arange(300, dtype=torch.float32)), torch.eye(129) * 5.0):
        lam, V = ops.syevd(H.to(gpu), method=1)
        ref = torch.linalg.eigvalsh(H.double())
        assert float((lam.cpu().double() - ref).abs().max()) <= 1e-5 * max(1.0, float(ref.abs().max()))
        resid, orth = _quality(H, lam, V)
        assert resid < 1e-5 and orth < 1e-5, (H.shape, resid, orth)


def test_syevd_two_stage_edge_cases(gpu):
    """Two-stage path: no panel (n <= 32: already a band), one panel of one row (n = 33), ragged
    sizes; zero panels (a diagonal matrix, 5 I: the Cholesky QR fails and the tall-skinny
    Householder QR runs; every bulge reflector trivial); a matrix whose panels have zero columns."""
    g = torch.Generator().manual_seed(7)
    cases = []
    for n in (3, 32, 33, 64, 65, 100, 300):
        X = torch.randn(2 * n, n, generator=g) * torch.exp(torch.randn(n, generator=g))
        cases.append(X.T @ X / (2 * n))
    cases += [torch.diag(torch.arange(300, dtype=torch.float32)), torch.eye(129) * 5.0]
    X = torch.randn(600, 300, generator=g)
    X[:, 40:70] = 0.0  # dead channels: zero rows and columns in H, zero columns in the panels
    cases.append(X.T @ X / 600 + torch.diag((torch.arange(300) % 7).float()))
    for H in cases:
        H = 0.5 * (H + H.T)
        lam, V = ops.syevd(H.to(gpu), method=2)
        ref = torch.linalg.eigvalsh(H.double())
        scale = max(1.0, float(ref.abs().max()))
        assert float((lam.cpu().double() - ref).abs().max()) <= 2e-5 * scale, H.shape
        assert bool((lam[1:] >= lam[:-1]).all())
        resid, orth = _quality(H, lam, V)
        assert resid < 2e-5 and orth < 2e-5, (H.shape, resid, orth)


def test_syevd_method_rejects_bad_arguments(gpu):
    with pytest.raises(ValueError, match="method"):
        ops.syevd(torch.eye(4, device=gpu), method=3)
    with pytest.raises(ValueError, match="two-stage"):
        ops.syevd(torch.eye(2, device=gpu), method=2)


@pytest.mark.parametrize("n", [200, 1000, 2048])
def test_syevd_f64_matches_lapack(gpu, n):
    # fp64 path (the QUIP# adapter's float64 Hessian): eigenvalues, residual and orthogonality at
    # fp64 accuracy against LAPACK on the CPU
    _, H = make_layer(8, n, tokens=2 * n, seed_key=f"eigh64:{n}")
    H = H.double()
    H = 0.5 * (H + H.T)  # exactly symmetric in fp64, as the adapter passes it (both solvers read one triangle)
    lam, V = ops.syevd(H.to(gpu))
    assert lam.dtype == torch.float64 and V.dtype == torch.float64
    lam, V = lam.cpu(), V.cpu()
    ref = torch.linalg.eigvalsh(H)
    scale = float(ref.abs().max())
    assert float((lam - ref).abs().max()) <= 1e-11 * scale
    assert bool((lam[1:] >= lam[:-1]).all())
    resid = float((H @ V - V * lam.unsqueeze(0)).norm() / H.norm())
    orth = float((V.T @ V - torch.eye(n, dtype=torch.float64)).abs().max())
    assert resid < 1e-12 and orth < 1e-12, (resid, orth)


def test_syevd_f64_small(gpu):
    for H in (torch.tensor([[3.0]], dtype=torch.float64), torch.diag(torch.arange(70, dtype=torch.float64)),
              torch.eye(65, dtype=torch.float64) * 2.0):
        lam, V = ops.syevd(H.to(gpu))
        ref = torch.linalg.eigvalsh(H)
        assert float((lam.cpu() - ref).abs().max()) <= 1e-12 * max(1.0, float(ref.abs().max()))
        Vc = V.cpu()
        assert float((Vc.T @ Vc - torch.eye(H.shape[0], dtype=torch.float64)).abs().max()) < 1e-12


def test_eigen_cache_exact_match_only(gpu):
    # the adapter reuses the decomposition of an element-for-element identical Hessian (q/k/v,
    # gate/up) and recomputes for any other input or floor parameters
    from mpq_amd.adapters.gptqmodel import clear_eigen_cache, vamp_hessian_eigen

    _, H = make_layer(8, 256, tokens=512, seed_key="eigen-cache")
    H = H.to(gpu)
    clear_eigen_cache()
    a = vamp_hessian_eigen(H)
    b = vamp_hessian_eigen(H.clone())
    assert all(x is y for x, y in zip(a[:4], b[:4])) and a[4] == b[4]
    H2 = H.clone()
    H2[3, 5] += 1e-3
    H2[5, 3] += 1e-3
    c = vamp_hessian_eigen(H2)
    assert c[2] is not a[2]
    assert float((c[0] - a[0]).abs().max()) > 0.0
    d = vamp_hessian_eigen(H2, floor_scale=1e-3)
    assert d[2] is not c[2]
    e = vamp_hessian_eigen(H2, floor_scale=1e-3, use_cache=False)
    assert e[2] is not d[2]
    assert torch.equal(e[2], d[2]) and torch.equal(e[0], d[0])  # deterministic: same bits either way
    clear_eigen_cache()
