"""CPU: pin the AWQ oracle (oracle/awq.py) with closed forms."""
import torch

from oracle import awq as oa


def test_candidate_scales_normalised():
    g = torch.Generator().manual_seed(0)
    x = torch.rand(256, generator=g) * 3
    w = torch.rand(256, generator=g)
    for r in (0.0, 0.35, 0.95):
        s = oa.candidate_scales(x, w, r)
        assert abs(float(s.max() * s.min()) - 1.0) < 1e-5
    s0 = oa.candidate_scales(x, w, 0.0)
    ref = (1.0 / (w + 1e-4)).clamp(min=1e-4)
    assert torch.allclose(s0, ref / (ref.max() * ref.min()).sqrt(), rtol=1e-6)


def test_pseudo_quantize_on_grid():
    g = torch.Generator().manual_seed(1)
    W = torch.randn(8, 256, generator=g)
    for sym in (False, True):
        Q = oa.pseudo_quantize(W, 4, 128, sym)
        v = W.view(-1, 128)
        q = Q.view(-1, 128)
        if sym:
            scale = v.abs().amax(1, keepdim=True) / 7
        else:
            scale = (v.amax(1, keepdim=True) - v.amin(1, keepdim=True)) / 15
        k = q / scale
        assert torch.allclose(k, torch.round(k), atol=1e-3)  # values on the group grid
        assert float(((q - v).abs() / scale).max()) <= 0.5 + 1e-4  # nearest grid point
        assert torch.equal(oa.pseudo_quantize(Q, 4, 128, sym), Q)  # re-quantizing a grid point is exact


def test_linear_loss_is_output_mse():
    g = torch.Generator().manual_seed(2)
    T, rows, n = 512, 16, 128
    X = torch.randn(T, n, generator=g).double()
    D = torch.randn(rows, n, generator=g).double()
    H = X.T @ X / T
    lhs = float(((X @ D.T) ** 2).mean())
    rhs = float(((D @ H) * D).sum() / rows)
    assert abs(lhs - rhs) <= 1e-10 * abs(lhs)


def test_w_mean_closed_form():
    W = torch.tensor([[1.0, -2.0, 4.0, 0.5]])
    got = oa.compute_w_mean([W], 2)
    ref = torch.tensor([1.0 / (2 + 1e-6), 2.0 / (2 + 1e-6), 4.0 / (4 + 1e-6), 0.5 / (4 + 1e-6)])
    assert torch.allclose(got, ref)
