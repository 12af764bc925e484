"""CPU: pins oracle/rht.py (the QUIP# randomized Hadamard transform in closed form)."""
import torch

from oracle import rht


def test_had_matrix_is_orthonormal_sylvester():
    for k in (2, 8, 64, 384):
        Hk = rht.had_matrix(k)
        assert torch.allclose(Hk @ Hk.T, torch.eye(k, dtype=torch.float64), atol=1e-12)
        assert torch.allclose(Hk, Hk.T)
    H8, H4 = rht.had_matrix(8), rht.had_matrix(4)
    # Sylvester recursion H_2k = [[H_k, H_k], [H_k, -H_k]] / sqrt(2)
    assert torch.allclose(H8, torch.cat([torch.cat([H4, H4], 1), torch.cat([H4, -H4], 1)], 0) / 2 ** 0.5)
    # a width that is not a power of two: blocks of its largest power-of-two factor (384 = 3 x 128)
    H384 = rht.had_matrix(384)
    assert torch.equal(H384[:128, 128:], torch.zeros(128, 256, dtype=torch.float64))


def test_inverse_undoes_forward_and_preserves_proxy():
    g = torch.Generator().manual_seed(0)
    m, n = 48, 64
    W = torch.randn(m, n, generator=g, dtype=torch.float64)
    X = torch.randn(200, n, generator=g, dtype=torch.float64)
    H = X.T @ X
    SU = torch.randint(0, 2, (n,), generator=g).double() * 2 - 1
    SV = torch.randint(0, 2, (m,), generator=g).double() * 2 - 1
    Wr, Hr = rht.rht_w(W, SU, SV), rht.rht_h(H, SU)
    assert torch.allclose(rht.incoherence_process(Wr, SU, SV), W, atol=1e-12)
    # the transform is orthogonal on both sides: tr(W H W^T) is invariant
    assert abs(float(((Wr @ Hr) * Wr).sum()) - float(((W @ H) * W).sum())) <= 1e-9 * float(((W @ H) * W).sum())
