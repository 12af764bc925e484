"""GPU: the bf16-plane ("x6") fp32 products (mpq_gemm_x6, mpq_rankspace_pack) against fp64 and
against the fp32 MFMA kernel (mpq_gemm_f32), and the VAMP solver on the packed operator."""
import pytest
import torch

from mpq_amd import ops

pytestmark = pytest.mark.gpu


def _op(B, trans):
    return B.T if trans else B


def test_gemm_x6_known_answer_pins_the_plane_products(gpu):
    """a = 1 + 2^-9 + 2^-18 and b = 1 + 2^-10 + 2^-19 split into bf16 planes (1, 2^-9, 2^-18) and
    (1, 2^-10, 2^-19).  The six kept products sum to 1 + 2^-9 + 2^-10 + 2^-17 exactly (the dropped
    a1 b2, a2 b1, a2 b2 are below 2^-27, under half an fp32 ulp of the product), so with K = 32
    equal terms every entry is exactly 32 * that; dropping or mis-pairing any one plane product
    moves an entry by at least 32 * 2^-19 = 2^-14."""
    M, N, K = 160, 256, 32
    a = 1.0 + 2.0 ** -9 + 2.0 ** -18
    b = 1.0 + 2.0 ** -10 + 2.0 ** -19
    sign_r = torch.where(torch.arange(M) % 3 == 0, -1.0, 1.0)
    sign_c = torch.where(torch.arange(N) % 5 == 1, -1.0, 1.0)
    A = (sign_r.view(-1, 1) * a).expand(M, K).contiguous().float()
    B = (sign_c.view(1, -1) * b).expand(K, N).contiguous().float()
    assert float(A[1, 0]) == a and float(B[0, 0]) == b  # representable in fp32
    exact = 32.0 * (1.0 + 2.0 ** -9 + 2.0 ** -10 + 2.0 ** -17)
    for trans in (False, True):
        Bp = ops.gemm_x6_pack_b((B.T.contiguous() if trans else B).to(gpu), trans_b=trans)
        C = ops.gemm_x6(A.to(gpu), Bp, N).cpu().double()
        ref = exact * sign_r.view(-1, 1).double() * sign_c.view(1, -1).double()
        assert torch.equal(C, ref), float((C - ref).abs().max())


@pytest.mark.parametrize("M,N,K,trans", [(128, 512, 512, False), (128, 512, 512, True), (100, 256, 1024, False),
                                         (384, 1024, 2048, True), (1, 128, 32, False), (257, 384, 4096, False),
                                         (130, 256, 96, True)])
def test_gemm_x6_matches_fp64(gpu, M, N, K, trans):
    """Entry-wise error relative to sum_k |a_k b_k| against fp64: within twice the fp32 MFMA kernel's
    on the same operands, and below 2e-6.  K slices of a multiple of four 16-k slabs run the LDS-ring
    kernel, the others (K = 32, 96 here) the register-staged one (a dropped 2^-16-order plane product shows at K = 32 as
    ~3e-6 and above; the known-answer test pins the plane set exactly)."""
    g = torch.Generator().manual_seed(M * 13 + N + K)
    # columns of A and rows of op(B) with a spread of magnitudes (1e-3 .. 1e3)
    A = torch.randn(M, K, generator=g) * torch.exp(3.0 * torch.randn(1, K, generator=g))
    B = torch.randn(N, K, generator=g) if trans else torch.randn(K, N, generator=g)
    Bp = ops.gemm_x6_pack_b(B.to(gpu), trans_b=trans)
    C6 = ops.gemm_x6(A.to(gpu), Bp, N).cpu().double()
    Cf = ops.gemm(A.to(gpu), B.to(gpu), trans_b=trans).cpu().double()
    Bo = _op(B.double(), trans)
    ref = A.double() @ Bo
    mag = A.double().abs() @ Bo.abs()
    e6 = float(((C6 - ref).abs() / mag).max())
    ef = float(((Cf - ref).abs() / mag).max())
    print(f"x6 {e6:.3e} fp32 {ef:.3e}")
    assert e6 <= max(2.0 * ef, 2e-7) and e6 < 2e-6
    # deterministic (fixed split order)
    assert torch.equal(ops.gemm_x6(A.to(gpu), Bp, N).cpu().double(), C6)


def test_gemm_x6_pack_nn_equals_nt(gpu):
    g = torch.Generator().manual_seed(3)
    A = torch.randn(200, 768, generator=g)
    B = torch.randn(768, 640, generator=g)
    p1 = ops.gemm_x6_pack_b(B.to(gpu), trans_b=False)
    p2 = ops.gemm_x6_pack_b(B.T.contiguous().to(gpu), trans_b=True)
    assert torch.equal(p1.cpu(), p2.cpu())
    assert torch.equal(ops.gemm_x6(A.to(gpu), p1, 640).cpu(), ops.gemm_x6(A.to(gpu), p2, 640).cpu())


def test_gemm_x6_rejects_unsupported_shapes(gpu):
    A = torch.randn(8, 96, device=gpu)
    with pytest.raises(ValueError):
        ops.gemm_x6_pack_b(torch.randn(96, 100, device=gpu))   # N % 128 != 0
    with pytest.raises(ValueError):
        ops.gemm_x6_pack_b(torch.randn(48, 128, device=gpu))   # K % 32 != 0
    assert ops.rankspace_pack(torch.randn(200, 200, device=gpu), torch.randn(200, 200, device=gpu)) is None
    Bp = ops.gemm_x6_pack_b(torch.randn(96, 128, device=gpu))
    C = ops.gemm_x6(A, Bp, 128)
    assert C.shape == (8, 128)


def test_rankspace_pack_layout(gpu):
    """The packed operator is [V for r V | V for x V^T | Vs for x Vs]: each third gives the same
    product as mpq_gemm_x6 on the matching packing."""
    n = 256
    g = torch.Generator().manual_seed(9)
    V = torch.linalg.qr(torch.randn(n, n, generator=g, dtype=torch.float64))[0].float()
    S = torch.rand(n, generator=g) + 0.1
    Vs = V * S.view(1, -1)
    X = torch.randn(64, n, generator=g)
    pk = ops.rankspace_pack(V.to(gpu), Vs.to(gpu))
    assert pk is not None and pk.numel() == 3 * n * n
    Xg = X.to(gpu)
    for part, ref in ((0, X.double() @ V.double()), (1, X.double() @ V.double().T), (2, X.double() @ Vs.double())):
        C = ops.gemm_x6(Xg, pk[part * n * n:(part + 1) * n * n], n).cpu().double()
        assert float((C - ref).abs().max()) <= 2e-6 * float(ref.abs().max())


def test_gemm_x6_splitk_partials_sum_to_the_product(gpu):
    """mpq_gemm_x6_pack_a + mpq_gemm_x6_splitk (the VAMP solvers' launches): the partials added in
    split order are bit-identical to mpq_gemm_x6, and each partial is its K slice's product."""
    M, N, K = 128, 384, 2048
    g = torch.Generator().manual_seed(21)
    A = torch.randn(M, K, generator=g)
    B = torch.randn(K, N, generator=g)
    Bp = ops.gemm_x6_pack_b(B.to(gpu))
    Ap = ops.gemm_x6_pack_a(A.to(gpu))
    P, splits = ops.gemm_x6_splitk(Ap, Bp, M, N, K)
    assert splits > 1
    acc = P[0].clone()
    for s in range(1, splits):
        acc += P[s]
    assert torch.equal(acc.cpu(), ops.gemm_x6(A.to(gpu), Bp, N).cpu())
    ks = K // splits
    for s in (0, splits - 1):
        ref = A[:, s * ks:(s + 1) * ks].double() @ B[s * ks:(s + 1) * ks].double()
        assert float((P[s].cpu().double() - ref).abs().max()) <= 2e-6 * float(ref.abs().max())
