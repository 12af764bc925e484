"""GPU: AWQ scale search (mpq_awq_w_mean, mpq_awq_search) against the CPU oracle (oracle/awq.py)."""
import pytest
import torch

from mpq_amd import awq
from oracle import awq as oa
from tests.uniform_cases import make_layer

pytestmark = pytest.mark.gpu


def test_w_mean(gpu):
    g = torch.Generator().manual_seed(4)
    Ws = [torch.randn(64, 512, generator=g) * 0.02, torch.randn(32, 512, generator=g)]
    got = awq.compute_w_mean([w.to(gpu) for w in Ws], 128).cpu()
    ref = oa.compute_w_mean(Ws, 128)
    assert torch.allclose(got, ref, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("bits,sym", [(4, False), (3, False), (4, True)])
def test_search_matches_oracle(gpu, bits, sym):
    W, H = make_layer(96, 256, tokens=1024, seed_key=f"awq:{bits}:{sym}")
    g = torch.Generator().manual_seed(9)
    X = torch.randn(1024, 256, generator=g) * torch.exp(torch.randn(256, generator=g))
    x_mean = X.abs().mean(0)
    w_mean = oa.compute_w_mean([W], 128)
    s_ref, e_ref, r_ref, l_ref = oa.search_linear(W, H, x_mean, w_mean, bits, 128, sym)
    s, e, r, losses = awq.search_best_scale_linear(W.to(gpu), H.to(gpu), x_mean.to(gpu), bits=bits, group_size=128,
                                                   sym=sym, w_mean=w_mean.to(gpu))
    losses = losses.cpu()
    assert torch.allclose(losses, torch.tensor(l_ref), rtol=2e-4)
    assert abs(r - r_ref) < 1e-6
    assert abs(e - e_ref) <= 2e-4 * e_ref
    assert torch.allclose(s.cpu(), s_ref, rtol=1e-5)
