"""GPU: the fp64 matrix-core GEMM of the fp64 eigensolver (mpq_gemm_f64) against fp64 products on the
CPU: both operand layouts, alpha/beta, ragged shapes (partial tiles in every dimension, K not a
multiple of the 16-deep slab), split-K (small M x N with long K) and K = 0."""
import pytest
import torch

from mpq_amd import ops

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (17, 33, 5), (128, 64, 16), (130, 70, 200), (64, 64, 8192),
                                   (1000, 64, 1000), (300, 513, 64), (8, 8, 3000)])
@pytest.mark.parametrize("trans_b", [False, True])
@pytest.mark.parametrize("alpha,beta", [(0.75, -0.5), (-1.0, 1.0), (1.0, -0.5)])
def test_gemm_f64_matches_cpu(gpu, M, N, K, trans_b, alpha, beta):
    """alpha = +-1 with beta != 0 (the eigensolver's updates) starts the accumulators from C."""
    g = torch.Generator().manual_seed(M * 7919 + N * 31 + K)
    A = torch.randn(M, K, generator=g, dtype=torch.float64)
    B = torch.randn(N, K, generator=g, dtype=torch.float64) if trans_b else torch.randn(K, N, generator=g,
                                                                                          dtype=torch.float64)
    C0 = torch.randn(M, N, generator=g, dtype=torch.float64)
    ref = alpha * (A @ (B.T if trans_b else B)) + beta * C0
    out = C0.to(gpu)
    ops.gemm_f64(A.to(gpu), B.to(gpu), trans_b=trans_b, out=out, alpha=alpha, beta=beta)
    scale = float((A.abs() @ (B.abs().T if trans_b else B.abs())).max()) + 1.0
    err = float((out.cpu() - ref).abs().max())
    assert err <= 64 * K * 2.0 ** -53 * scale + 1e-300, (err, scale)
    # beta == 0 never reads C (NaN there must not leak into the result)
    out2 = torch.full((M, N), float("nan"), dtype=torch.float64, device=gpu)
    ops.gemm_f64(A.to(gpu), B.to(gpu), trans_b=trans_b, out=out2)
    assert bool(torch.isfinite(out2).all())
    assert float((out2.cpu() - A @ (B.T if trans_b else B)).abs().max()) <= 64 * K * 2.0 ** -53 * scale


def test_gemm_f64_zero_k(gpu):
    C = torch.ones(5, 7, dtype=torch.float64, device=gpu)
    ops.gemm_f64(torch.empty(5, 0, dtype=torch.float64, device=gpu), torch.empty(0, 7, dtype=torch.float64, device=gpu),
                 out=C, alpha=1.0, beta=2.0)
    assert bool((C == 2.0).all())


def test_gemm_f64_deterministic(gpu):
    g = torch.Generator().manual_seed(5)
    A = torch.randn(64, 4096, generator=g, dtype=torch.float64).to(gpu)
    B = torch.randn(4096, 64, generator=g, dtype=torch.float64).to(gpu)
    a = ops.gemm_f64(A, B)
    b = ops.gemm_f64(A, B)
    assert torch.equal(a, b)
