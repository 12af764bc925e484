"""GPU: Hessian accumulation (mpq_hessian_accumulate, fp32 MFMA SYRK) against fp64 products, and
the GPTQ / QUIP# accumulation conventions (mpq_amd/hessian.py) against fp64 restatements."""
import math

import pytest
import torch

from mpq_amd import hessian

pytestmark = pytest.mark.gpu


def _rel(a, b):
    return float((a.double() - b.double()).norm() / b.double().norm())


@pytest.mark.parametrize("T,n", [(1000, 256), (37, 384), (4096, 1024), (0, 128)])
def test_syrk_matches_fp64(gpu, T, n):
    g = torch.Generator().manual_seed(T + n)
    X = torch.randn(T, n, generator=g) * torch.exp(torch.randn(n, generator=g))
    H0 = torch.randn(n, n, generator=g)
    H0 = H0 + H0.T
    H = H0.clone().to(gpu)
    hessian.accumulate(H, X.to(gpu), alpha=0.75, beta=0.5)
    H = H.cpu()
    ref = 0.5 * H0.double() + 0.75 * X.double().T @ X.double()
    assert _rel(H, ref) < 2e-6
    assert torch.equal(H, H.T)


def test_syrk_bf16_input_and_colsum(gpu):
    g = torch.Generator().manual_seed(3)
    X = torch.randn(3, 100, 512, generator=g).to(torch.bfloat16)
    H = torch.zeros(512, 512, device=gpu)
    cs = torch.zeros(512, device=gpu)
    hessian.accumulate(H, X.to(gpu), colsum=cs)
    Xd = X.reshape(-1, 512).double()
    assert _rel(H.cpu(), Xd.T @ Xd) < 2e-6
    assert torch.allclose(cs.cpu().double(), Xd.sum(0), rtol=1e-5, atol=1e-4)


def test_gptq_convention(gpu):
    g = torch.Generator().manual_seed(5)
    n = 256
    acc = hessian.GPTQHessian(n, gpu)
    Href = torch.zeros(n, n, dtype=torch.float64)
    ns = 0
    for b in (3, 1, 4):
        inp = torch.randn(b, 64, n, generator=g)
        acc.add_batch(inp.to(gpu))
        # classic GPTQ add_batch in fp64
        Href *= ns / (ns + b)
        ns += b
        x = math.sqrt(2 / ns) * inp.reshape(-1, n).double().T
        Href += x @ x.T
    assert acc.nsamples == ns
    assert _rel(acc.H.cpu(), Href) < 2e-6


def test_quip_convention(gpu):
    g = torch.Generator().manual_seed(6)
    n = 128
    acc = hessian.QuipHessian(n, gpu)
    xs = [torch.randn(200, n, generator=g) + 0.3 for _ in range(3)]
    for x in xs:
        acc.add_batch(x.to(gpu))
    H, mu, ct = acc.finalize()
    X = torch.cat(xs).double()
    mu_ref = X.mean(0)
    H_ref = X.T @ X / X.shape[0] - torch.outer(mu_ref, mu_ref)
    assert ct == X.shape[0]
    assert torch.allclose(mu.cpu().double(), mu_ref, atol=1e-5)
    assert _rel(H.cpu(), H_ref) < 1e-5


def test_rejects_bad_width(gpu):
    with pytest.raises(ValueError):
        hessian.accumulate(torch.zeros(100, 100, device=gpu), torch.zeros(10, 100, device=gpu))
