"""The GPU greedy sweeps (mpq_uniform_cd_sweeps, mpq_uniform_cd_sweeps_recip) against the oracle's
column-at-a-time sweeps from the same state: bit-identical codes, values, residual norms, rhs and accept
counts.

The GPU runs 128 decisions per window with the window's rank-1 updates in registers and applies the
deferred update of every other column as a sequential multiply-then-subtract chain in window order,
which is the per-column update order and rounding of the reference (mpq/polish/triton_scalar_cd.py:
258-288).  Its greedy gain is summed over a block's rows in row order (the oracle's ``seq_gain``).
"""
import pytest
import torch

from mpq_amd import ops
from oracle import uniform as ou
from tests.uniform_cases import make_layer

pytestmark = pytest.mark.gpu


def _state(rows, n, bits, gs, key, tokens):
    W, H = make_layer(rows, n, tokens=tokens, seed_key=key)
    lam, V, _ = ou.hessian_eigen(H)
    Vs = V * torch.sqrt(lam).unsqueeze(0)
    maxq = 2 ** bits - 1
    G = (n + gs - 1) // gs
    sc, zc = [], []
    for g in range(G):
        s, z = ou.gptq_find_params(W[:, g * gs:(g + 1) * gs], maxq)
        sc.append(s)
        zc.append(z)
    sg, zg = torch.cat(sc, 1), torch.cat(zc, 1)
    widths = torch.tensor([min(gs, n - g * gs) for g in range(G)])
    sf = torch.repeat_interleave(sg, widths, dim=1)
    zf = torch.repeat_interleave(zg, widths, dim=1)
    q0 = torch.clamp(torch.round(W / sf) + zf, 0, maxq)
    x0 = sf * (q0 - zf)
    res_u = W.matmul(Vs) - x0.matmul(Vs)
    rhs0 = res_u.matmul(Vs.T.contiguous())
    res0 = res_u.square().sum(dim=1)
    diag = Vs.square().sum(dim=1).clamp_min_(1e-12)
    return H, sg, zg, sf, zf, maxq, q0.to(torch.uint8), x0, rhs0, res0, diag


@pytest.mark.parametrize("rows,n,bits,gs,block_rows,tokens,key", [
    (1024, 1024, 4, 128, 128, 4096, "cfg0:0"),   # BASELINE config 0 size, 8 row blocks
    (1024, 1024, 3, 128, 128, 4096, "cfg0:1"),
    (300, 260, 4, 128, 100, 1024, "ragged"),     # ragged blocks, n % 4 == 0 but not % 1024, partial group
    (70, 131, 2, 64, 48, 512, "odd"),            # n % 4 != 0, block of 22 rows at the end
])
def test_cd_sweeps_bit_identical_to_oracle(gpu, rows, n, bits, gs, block_rows, tokens, key):
    H, sg, zg, sf, zf, maxq, q0, x0, rhs0, res0, diag = _state(rows, n, bits, gs, key, tokens)
    rhs, x, q = rhs0.to(gpu), x0.to(gpu), q0.to(gpu)
    res = res0.to(gpu)
    acc = torch.zeros(rows, dtype=torch.int32, device=gpu)
    ops.uniform_cd_sweeps(rhs, x, q, res, acc, sg.to(gpu), zg.to(gpu), gs, maxq, diag.to(gpu), H.to(gpu),
                          block_rows=block_rows, sweeps=3)
    xs, rhss, ress, accs = [], [], [], []
    for r0 in range(0, rows, block_rows):
        rb = slice(r0, min(r0 + block_rows, rows))
        xr, rr, er, ar = ou.greedy_cd_sweeps(x0[rb], rhs0[rb], res0[rb], H, diag, sf[rb], zf[rb], maxq, 3,
                                             seq_gain=True)
        xs.append(xr)
        rhss.append(rr)
        ress.append(er)
        accs.append(ar)
    x_ref, rhs_ref, res_ref, acc_ref = torch.cat(xs), torch.cat(rhss), torch.cat(ress), torch.cat(accs)
    q_ref = ou.nearest_atom_idx(x_ref, sf, zf, maxq)
    print(key, "accepted", int(acc_ref.sum()), "codes equal", float((q.cpu().long() == q_ref.long()).float().mean()))
    assert int(acc_ref.sum()) > 0
    assert torch.equal(acc.cpu().long(), acc_ref)
    assert torch.equal(q.cpu().long(), q_ref.long())
    assert torch.equal(x.cpu(), x_ref)
    assert torch.equal(res.cpu(), res_ref)
    assert torch.equal(rhs.cpu(), rhs_ref)


@pytest.mark.parametrize("rows,n,bits,gs,block_rows,tokens,key", [
    (1024, 1024, 4, 128, 128, 4096, "cfg0:2"),
    (300, 260, 4, 128, 100, 1024, "ragged-r"),
])
def test_cd_sweeps_recip_rule_bit_identical_to_oracle(gpu, rows, n, bits, gs, block_rows, tokens, key):
    """mpq_uniform_cd_sweeps_recip: the RTN target x + rhs * (1 / diag) of the reference's torch update
    loop (mpq/polish/triton_scalar_cd.py:266) against the oracle with ``target_div=False``."""
    H, sg, zg, sf, zf, maxq, q0, x0, rhs0, res0, diag = _state(rows, n, bits, gs, key, tokens)
    rhs, x, q = rhs0.to(gpu), x0.to(gpu), q0.to(gpu)
    res = res0.to(gpu)
    acc = torch.zeros(rows, dtype=torch.int32, device=gpu)
    ops.uniform_cd_sweeps(rhs, x, q, res, acc, sg.to(gpu), zg.to(gpu), gs, maxq, diag.to(gpu), H.to(gpu),
                          block_rows=block_rows, sweeps=3, target_rule="recip")
    xs, rhss, ress, accs = [], [], [], []
    for r0 in range(0, rows, block_rows):
        rb = slice(r0, min(r0 + block_rows, rows))
        xr, rr, er, ar = ou.greedy_cd_sweeps(x0[rb], rhs0[rb], res0[rb], H, diag, sf[rb], zf[rb], maxq, 3,
                                             target_div=False, seq_gain=True)
        xs.append(xr)
        rhss.append(rr)
        ress.append(er)
        accs.append(ar)
    x_ref, rhs_ref, res_ref, acc_ref = torch.cat(xs), torch.cat(rhss), torch.cat(ress), torch.cat(accs)
    assert int(acc_ref.sum()) > 0
    assert torch.equal(acc.cpu().long(), acc_ref)
    assert torch.equal(x.cpu(), x_ref)
    assert torch.equal(res.cpu(), res_ref)
    assert torch.equal(rhs.cpu(), rhs_ref)
    with pytest.raises(ValueError, match="target_rule"):
        ops.uniform_cd_sweeps(rhs, x, q, res, acc, sg.to(gpu), zg.to(gpu), gs, maxq, diag.to(gpu), H.to(gpu),
                              block_rows=block_rows, sweeps=1, target_rule="exact")


def test_cd_sweeps_rejects_bad_arguments(gpu):
    rhs = torch.zeros(4, 8, device=gpu)
    x = torch.zeros(4, 8, device=gpu)
    q = torch.zeros(4, 8, dtype=torch.uint8, device=gpu)
    res = torch.zeros(4, device=gpu)
    acc = torch.zeros(4, dtype=torch.int32, device=gpu)
    s = torch.ones(4, 1, device=gpu)
    d = torch.ones(8, device=gpu)
    H = torch.eye(8, device=gpu)
    with pytest.raises(ValueError, match="maxq"):
        ops.uniform_cd_sweeps(rhs, x, q, res, acc, s, s, 8, 0, d, H, block_rows=4, sweeps=1)
    with pytest.raises(ValueError):
        ops.uniform_cd_sweeps(rhs, x, q.float(), res, acc, s, s, 8, 3, d, H, block_rows=4, sweeps=1)


@pytest.mark.parametrize("backend", ["torch", "triton"])
def test_reference_signature_scalar_cd_matches_oracle(gpu, backend):
    """mpq_amd.polish.uniform_scalar_diag_greedy_cd (reference mpq/polish/triton_scalar_cd.py:164-307):
    expanded scale/zero, one greedy order over all rows, per-sweep trace.  The oracle's sweeps run from
    the start state the wrapper forms on the device (the same deterministic products), so x and the
    accept counts must be identical; each backend with its RTN target rule (torch: x + rhs * (1/diag),
    :266; triton: x + rhs / diag, :73)."""
    from mpq_amd.polish import uniform_scalar_diag_greedy_cd

    rows, n, bits, gs = 96, 256, 4, 128
    H, sg, zg, sf, zf, maxq, q0, x0, rhs0, res0, diag = _state(rows, n, bits, gs, "ref-sig", 1024)
    lam, V, _ = ou.hessian_eigen(H)
    Vs = V * torch.sqrt(lam).unsqueeze(0)
    W, _ = make_layer(rows, n, tokens=1024, seed_key="ref-sig")
    Yu = W.matmul(Vs)
    xg, Vsg = x0.to(gpu), Vs.to(gpu)
    res_u = Yu.to(gpu) - ops.gemm(xg, Vsg)
    rhs_dev = ops.gemm(res_u, Vsg, trans_b=True).cpu()
    res_dev = res_u.square().sum(dim=1).cpu()
    diag_dev = Vsg.square().sum(dim=1).clamp_min_(1e-12).cpu()
    x_out, st = uniform_scalar_diag_greedy_cd(x=xg, Y_u=Yu.to(gpu), Vs=Vsg, gram_full=H.to(gpu), scale=sf.to(gpu),
                                              zero=zf.to(gpu), maxq=maxq, sweeps=3, raw_target=W.to(gpu),
                                              raw_gram=H.to(gpu), update_backend=backend)
    x_ref, _, res_ref, acc_ref = ou.greedy_cd_sweeps(x0, rhs_dev, res_dev, H, diag_dev, sf, zf, maxq, 3,
                                                     target_div=backend == "triton", seq_gain=True)
    assert torch.equal(x_out.cpu(), x_ref)
    assert st["accepted_updates"] == float(acc_ref.sum()) > 0
    tr = st["cd_trace"]
    assert [t["budget"] for t in tr] == [0, 1, 2, 3]
    assert sum(t["accepted_updates_sweep"] for t in tr) == int(acc_ref.sum())
    assert abs(tr[-1]["stabilized_objective_mean"] - float(res_ref.mean())) <= 1e-6 * float(res_ref.mean())
    q_ref = ou.nearest_atom_idx(x_ref, sf, zf, maxq)
    assert tr[-1]["assignment_changes_from_cd0"] == int((q_ref.long() != q0.long()).sum())
    objs = [t["raw_objective_mean"] for t in tr]
    assert all(b <= a * (1 + 1e-5) for a, b in zip(objs, objs[1:]))
    with pytest.raises(ValueError, match="update_backend"):
        uniform_scalar_diag_greedy_cd(x=xg, Y_u=Yu.to(gpu), Vs=Vsg, gram_full=H.to(gpu), scale=sf.to(gpu),
                                      zero=zf.to(gpu), maxq=maxq, sweeps=1, update_backend="cuda")
