"""GPU parity of the uniform-grid path against the CPU oracle (oracle/uniform.py)."""
import numpy as np
import pytest
import torch

from mpq_amd import ops
from mpq_amd.priors.uniform import discrete_uniform_mmse
from mpq_amd.solver import UniformVampConfig
from oracle import uniform as ou
from tests.uniform_cases import RECIPE, make_layer

pytestmark = pytest.mark.gpu


def _rel(a, b):
    return float((a.double() - b.double()).norm() / b.double().norm().clamp_min(1e-30))


@pytest.mark.parametrize("M,N,K,trans", [(128, 512, 512, False), (128, 512, 512, True), (100, 72, 37, False),
                                         (100, 72, 37, True), (256, 1024, 2048, False), (384, 640, 1536, True)])
def test_gemm_matches_fp64(gpu, M, N, K, trans):
    g = torch.Generator().manual_seed(M * 7 + N + K)
    A = torch.randn(M, K, generator=g)
    B = torch.randn(N, K, generator=g) if trans else torch.randn(K, N, generator=g)
    C = ops.gemm(A.to(gpu), B.to(gpu), trans_b=trans).cpu()
    ref = A.double() @ (B.double().T if trans else B.double())
    assert _rel(C, ref) < 2e-6
    # deterministic: bit-identical on a second call
    C2 = ops.gemm(A.to(gpu), B.to(gpu), trans_b=trans).cpu()
    assert torch.equal(C, C2)


def test_gemm_gather_and_axpby(gpu):
    g = torch.Generator().manual_seed(5)
    A = torch.randn(256, 128, generator=g)
    B = torch.randn(700, 300, generator=g)
    rows = torch.randperm(700, generator=g)[:128].to(torch.int32)
    C0 = torch.randn(256, 300, generator=g)
    out = C0.clone().to(gpu)
    ops.gemm(A.to(gpu), B.to(gpu), b_rows=rows.to(gpu), out=out, alpha=-1.0, beta=1.0)
    ref = C0.double() - A.double() @ B.double()[rows.long()]
    assert _rel(out.cpu(), ref) < 2e-6


def test_hadamard_transpose_scale_bit_exact(gpu):
    g = torch.Generator().manual_seed(6)
    for had, width in ((128, 512), (2048, 14336), (4, 12)):
        X = torch.randn(37, width, generator=g)
        signs = torch.randint(0, 2, (width,), generator=g).float() * 2 - 1
        got = ops.block_hadamard(X.to(gpu), had, signs=signs.to(gpu)).cpu()
        ref = ou.hadamard_rows(X * signs.view(1, -1), had)
        assert torch.equal(got, ref)
        inv = ops.block_hadamard(got.to(gpu), had, signs=signs.to(gpu), inverse=True).cpu()
        assert torch.allclose(inv, X, atol=1e-5)
    X = torch.randn(77, 130, generator=g)
    assert torch.equal(ops.transpose(X.to(gpu)).cpu(), X.T)
    s = torch.randn(130, generator=g)
    assert torch.equal(ops.scale_columns(X.to(gpu), s.to(gpu)).cpu(), X * s.view(1, -1))


@pytest.mark.parametrize("bits,gs", [(4, 128), (3, 128), (2, 64)])
def test_find_params_and_rtn_exact(gpu, bits, gs):
    W, _ = make_layer(96, 512, tokens=16, seed_key=f"fp{bits}")
    W[3, :gs] = 0.0  # all-zero group -> (-1, +1) range
    maxq = 2 ** bits - 1
    s, z = ops.gptq_find_params(W.to(gpu), gs, maxq)
    rs, rz = [], []
    for g0 in range(0, 512, gs):
        a, b = ou.gptq_find_params(W[:, g0:g0 + gs], maxq)
        rs.append(a)
        rz.append(b)
    rs, rz = torch.cat(rs, 1), torch.cat(rz, 1)
    assert torch.equal(s.cpu(), rs) and torch.equal(z.cpu(), rz)
    q, x = ops.uniform_rtn(W.to(gpu), s, z, gs, maxq)
    sf = torch.repeat_interleave(rs, gs, dim=1)
    zf = torch.repeat_interleave(rz, gs, dim=1)
    qr = torch.clamp(torch.round(W / sf) + zf, 0, maxq)
    assert torch.equal(q.cpu().long(), qr.long())
    assert torch.equal(x.cpu(), sf * (qr - zf))


def test_denoiser_matches_oracle(gpu):
    W, _ = make_layer(64, 384, tokens=16, seed_key="dn")
    s, z = ou.gptq_find_params(W, 15)
    sf, zf = s.expand(-1, 384).contiguous(), z.expand(-1, 384).contiguous()
    g = torch.Generator().manual_seed(9)
    r1 = W + 0.01 * torch.randn(W.shape, generator=g)
    gam = torch.exp(torch.randn(64, 1, generator=g)) * 3e3
    ref = ou.discrete_uniform_mmse(r1, gam, sf, zf, 15, W, 0.2)
    got = discrete_uniform_mmse(r1=r1.to(gpu), gamma1=gam.to(gpu), scale_full=sf.to(gpu), zero_full=zf.to(gpu),
                                maxq=15, prior_center=W.to(gpu), prior_tau=0.2, need_stats=False)
    assert torch.equal(got["map_idx"].cpu(), ref["map_idx"])
    assert torch.equal(got["map_value"].cpu(), ref["map_value"])
    assert _rel(got["mean"].cpu(), ref["mean"]) < 1e-5
    assert float(((got["mean"].cpu() - ref["mean"]).abs() / ref["mean"].abs().clamp_min(1e-3)).max()) < 1e-4
    assert _rel(got["var"].cpu(), ref["var"]) < 1e-3
    assert _rel(got["alpha1"].cpu(), ref["alpha1"]) < 1e-4


def _setup_block(rows, cols, bits, gs, key, rotate=False):
    W, H = make_layer(rows, cols, tokens=2048, seed_key=key)
    Hw = 0.5 * (2.0 * H)
    lam, V, _ = ou.hessian_eigen(Hw)
    if rotate:
        signs, had = ou.rotation_plan(cols, key)
        W = ou.hadamard_rows(W * signs.view(1, -1), had)
        Hw = ou.hadamard_rows(Hw.T.contiguous() * signs.view(1, -1), had).T.contiguous()
        Hw = ou.hadamard_rows(Hw * signs.view(1, -1), had)
        V = ou.hadamard_rows(V.T.contiguous() * signs.view(1, -1), had).T.contiguous()
    S = torch.sqrt(lam)
    Vs = V * S.unsqueeze(0)
    maxq = 2 ** bits - 1
    sc, zc = [], []
    for g0 in range(0, cols, gs):
        a, b = ou.gptq_find_params(W[:, g0:g0 + gs], maxq)
        sc.append(a)
        zc.append(b)
    sg, zg = torch.cat(sc, 1), torch.cat(zc, 1)
    sf = torch.repeat_interleave(sg, gs, dim=1)
    zf = torch.repeat_interleave(zg, gs, dim=1)
    xr = sf * (torch.clamp(torch.round(W / sf) + zf, 0, maxq) - zf)
    return W, Hw, V, S, Vs, sg, zg, sf, zf, xr, maxq


@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("rotate,bits", [(False, 4), (True, 4), (True, 3)])
def test_vamp_block_matches_oracle(gpu, rotate, bits, packed):
    """fp32 MFMA products, and (packed) the bf16-plane products on the packed rank-space operator."""
    W, Hw, V, S, Vs, sg, zg, sf, zf, xr, maxq = _setup_block(128, 512, bits, 128, f"vb{bits}", rotate=rotate)
    cfg = dict(RECIPE, polish_sweeps=0)
    q_ref, x_ref, e_ref, rtn_ref, tr = ou.solve_uniform_rankspace_vamp(W, xr, sf, zf, maxq, V, V.T, S, Vs, cfg)
    vcfg = UniformVampConfig(**{k: v for k, v in RECIPE.items()})
    pk = ops.rankspace_pack(V.to(gpu), Vs.to(gpu)) if packed else None
    assert (pk is not None) == packed
    q, x, e, rtn, st = ops.uniform_vamp_solve(W.to(gpu), xr.to(gpu), sg.to(gpu), zg.to(gpu), 128, maxq, V.to(gpu),
                                              S.to(gpu), Vs.to(gpu), vcfg, want_x=True, packed=pk)
    agree = float((q.cpu().long() == q_ref.long()).float().mean())
    print("vamp block agreement", agree, "best_iter", st["best_iter"], tr["best_iter"], "stop", st["stop_iter"],
          tr["stop_iter"], "obs", st["obs_precision_final"], tr["obs_final"])
    assert agree >= 0.999
    assert st["best_iter"] == tr["best_iter"] and st["stop_iter"] == tr["stop_iter"]
    assert abs(st["obs_precision_final"] - tr["obs_final"]) <= 1e-4 * tr["obs_final"]
    assert _rel(rtn.cpu(), rtn_ref) < 1e-4
    assert abs(float(e.mean()) - float(e_ref.mean())) <= 5e-3 * float(e_ref.mean())


@pytest.mark.parametrize("extra", [dict(init_from="float"), dict(init_from="zero"), dict(em_obs_precision=False),
                                   dict(obs_precision=50.0), dict(obs_precision=50.0, obs_init=200.0),
                                   dict(damping=1.0)],
                         ids=["init_float", "init_zero", "em_off", "obs_fixed", "obs_warm_start_first", "undamped"])
def test_vamp_block_config_options_match_oracle(gpu, extra):
    """The solver's other options (mpq/solver.py:426-830): the r1 start (float weight, zero), EM off,
    a fixed observation precision (a caller's warm start still comes first, :486-489), no damping.
    Each takes its own trajectory on this input (1-5 % of the codes and the best / stop iterations
    move against the recipe in the oracle)."""
    W, Hw, V, S, Vs, sg, zg, sf, zf, xr, maxq = _setup_block(128, 512, 4, 128, "vb4", rotate=True)
    extra = dict(extra)
    obs_init = extra.pop("obs_init", None)
    cfg = dict(RECIPE, polish_sweeps=0, **extra)
    q_ref, x_ref, e_ref, rtn_ref, tr = ou.solve_uniform_rankspace_vamp(W, xr, sf, zf, maxq, V, V.T, S, Vs, cfg,
                                                                      obs_precision_init=obs_init)
    vcfg = UniformVampConfig(**{k: v for k, v in cfg.items()})
    pk = ops.rankspace_pack(V.to(gpu), Vs.to(gpu))
    q, x, e, rtn, st = ops.uniform_vamp_solve(W.to(gpu), xr.to(gpu), sg.to(gpu), zg.to(gpu), 128, maxq, V.to(gpu),
                                              S.to(gpu), Vs.to(gpu), vcfg, want_x=True, packed=pk,
                                              obs_init=float(obs_init or 0.0))
    if obs_init:
        assert st["obs_precision_initial"] == obs_init
    agree = float((q.cpu().long() == q_ref.long()).float().mean())
    print(extra, "agreement", agree, "best/stop", st["best_iter"], st["stop_iter"], "obs", st["obs_precision_final"])
    assert agree >= 0.999
    assert st["best_iter"] == tr["best_iter"] and st["stop_iter"] == tr["stop_iter"]
    assert abs(st["obs_precision_final"] - tr["obs_final"]) <= 1e-4 * tr["obs_final"]
    assert abs(float(e.mean()) - float(e_ref.mean())) <= 5e-3 * float(e_ref.mean())


@pytest.mark.parametrize("packed", [False, True])
def test_vamp_block_round_mean_matches_oracle(gpu, packed):
    """final_decision="round_mean" (mpq/solver.py:833-850): every hard state rounds the posterior mean
    to the grid instead of taking the MAP atom (the fused LMMSE / hard-decision kernel's second mode).
    A weak prior (tau 2) and a small gamma1 start keep the posteriors broad, so the two decisions
    differ (on about 6 % of the codes in the oracle, with other best / stop iterations)."""
    W, Hw, V, S, Vs, sg, zg, sf, zf, xr, maxq = _setup_block(128, 512, 4, 128, "vb4", rotate=True)
    cfg = dict(RECIPE, polish_sweeps=0, final_decision="round_mean", gamma_start=0.01, prior_tau=2.0)
    q_ref, x_ref, e_ref, rtn_ref, tr = ou.solve_uniform_rankspace_vamp(W, xr, sf, zf, maxq, V, V.T, S, Vs, cfg)
    cfg_map = dict(cfg, final_decision="map")
    q_map, _, _, _, _ = ou.solve_uniform_rankspace_vamp(W, xr, sf, zf, maxq, V, V.T, S, Vs, cfg_map)
    vcfg = UniformVampConfig(**{k: v for k, v in cfg.items()})
    pk = ops.rankspace_pack(V.to(gpu), Vs.to(gpu)) if packed else None
    q, x, e, rtn, st = ops.uniform_vamp_solve(W.to(gpu), xr.to(gpu), sg.to(gpu), zg.to(gpu), 128, maxq, V.to(gpu),
                                              S.to(gpu), Vs.to(gpu), vcfg, want_x=True, packed=pk)
    agree = float((q.cpu().long() == q_ref.long()).float().mean())
    differs = float((q_ref.long() != q_map.long()).float().mean())
    print("round_mean agreement", agree, "oracle codes differing from the MAP decision", differs,
          "best/stop", st["best_iter"], st["stop_iter"])
    assert differs > 0  # the two decisions are not the same on this input
    assert agree >= 0.999
    assert st["best_iter"] == tr["best_iter"] and st["stop_iter"] == tr["stop_iter"]
    assert abs(float(e.mean()) - float(e_ref.mean())) <= 5e-3 * float(e_ref.mean())


@pytest.mark.parametrize("packed", [False, True])
def test_vamp_block_gamma_retries_match_oracle(gpu, packed):
    """gamma_start 100: the first denoiser pass finds alpha1 outside (1e-7, 1 - 1e-7) on most rows and
    the loop retries with rescaled gamma1 twice before alpha1 is valid (the oracle's posterior runs
    five times).  The r2 message and first LMMSE product, queued before the first pass's status is
    read, are discarded and run again from the retried pass."""
    W, Hw, V, S, Vs, sg, zg, sf, zf, xr, maxq = _setup_block(128, 512, 4, 128, "vb4", rotate=True)
    cfg = dict(RECIPE, polish_sweeps=0, gamma_start=100.0)
    q_ref, x_ref, e_ref, rtn_ref, tr = ou.solve_uniform_rankspace_vamp(W, xr, sf, zf, maxq, V, V.T, S, Vs, cfg)
    vcfg = UniformVampConfig(**{k: v for k, v in cfg.items()})
    pk = ops.rankspace_pack(V.to(gpu), Vs.to(gpu)) if packed else None
    q, x, e, rtn, st = ops.uniform_vamp_solve(W.to(gpu), xr.to(gpu), sg.to(gpu), zg.to(gpu), 128, maxq, V.to(gpu),
                                              S.to(gpu), Vs.to(gpu), vcfg, want_x=True, packed=pk)
    agree = float((q.cpu().long() == q_ref.long()).float().mean())
    print("retries", st["alpha1_retry_count"], "agreement", agree, "best/stop", st["best_iter"], st["stop_iter"])
    assert st["alpha1_retry_count"] > 0
    assert agree >= 0.999
    assert st["best_iter"] == tr["best_iter"] and st["stop_iter"] == tr["stop_iter"]
    assert abs(st["obs_precision_final"] - tr["obs_final"]) <= 1e-4 * tr["obs_final"]
    assert abs(float(e.mean()) - float(e_ref.mean())) <= 5e-3 * float(e_ref.mean())


def test_vamp_block_with_caller_products(gpu):
    # mpq_uniform_vamp_solve_ex: W Vs and x_init Vs from the caller (one product over all rows), and
    # the returned x_best Vs; matches the oracle like the per-block path, and x_best Vs is the
    # product of the returned codes
    W, Hw, V, S, Vs, sg, zg, sf, zf, xr, maxq = _setup_block(128, 512, 4, 128, "vbx", rotate=True)
    cfg = dict(RECIPE, polish_sweeps=0)
    q_ref, x_ref, e_ref, rtn_ref, tr = ou.solve_uniform_rankspace_vamp(W, xr, sf, zf, maxq, V, V.T, S, Vs, cfg)
    vcfg = UniformVampConfig(**{k: v for k, v in RECIPE.items()})
    Wg, xg, Vsg = W.to(gpu), xr.to(gpu), Vs.to(gpu)
    Yu, XR = ops.gemm(Wg, Vsg), ops.gemm(xg, Vsg)
    xp = torch.empty_like(Yu)
    q, x, e, rtn, st = ops.uniform_vamp_solve(Wg, xg, sg.to(gpu), zg.to(gpu), 128, maxq, V.to(gpu), S.to(gpu), Vsg,
                                              vcfg, want_x=True, Yu=Yu, xr=XR, xprod_out=xp)
    assert float((q.cpu().long() == q_ref.long()).float().mean()) >= 0.999
    assert st["best_iter"] == tr["best_iter"] and st["stop_iter"] == tr["stop_iter"]
    assert _rel(rtn.cpu(), rtn_ref) < 1e-4
    assert abs(float(e.mean()) - float(e_ref.mean())) <= 5e-3 * float(e_ref.mean())
    xp_ref = x.double().cpu() @ Vs.double()
    assert float((xp.double().cpu() - xp_ref).abs().max()) <= 1e-5 * float(xp_ref.abs().max())
    # the polish started from that product equals the polish that forms it
    a = ops.uniform_cd_polish(None, q, sg.to(gpu), zg.to(gpu), 128, maxq, Vsg, Hw.to(gpu), block_rows=128,
                              sweeps=3, select=True, Yu=Yu, xprod=xp)
    b = ops.uniform_cd_polish(None, q, sg.to(gpu), zg.to(gpu), 128, maxq, Vsg, Hw.to(gpu), block_rows=128,
                              sweeps=3, select=True, Yu=Yu)
    assert float((a[0] == b[0]).float().mean()) >= 0.999
    assert _rel(a[1].cpu(), b[1].cpu()) < 1e-4 and _rel(a[2].cpu(), b[2].cpu()) < 1e-4


def test_cd_polish_matches_oracle(gpu):
    W, Hw, V, S, Vs, sg, zg, sf, zf, xr, maxq = _setup_block(256, 512, 4, 128, "cd")
    q0 = torch.clamp(torch.round(W / sf) + zf, 0, maxq).to(torch.uint8)
    Y_u = W @ Vs
    x_pol, acc_ref = ou.scalar_greedy_cd(xr[:128], Y_u[:128], Vs, Hw, sf[:128], zf[:128], maxq, 3)
    q_ref = ou.nearest_atom_idx(x_pol, sf[:128], zf[:128], maxq)
    q, eb, ea, imp, acc = ops.uniform_cd_polish(W.to(gpu), q0.to(gpu), sg.to(gpu), zg.to(gpu), 128, maxq, Vs.to(gpu),
                                                Hw.to(gpu), block_rows=128, sweeps=3, select=False)
    agree = float((q[:128].cpu().long() == q_ref.long()).float().mean())
    print("cd agreement", agree, "accepted", int(acc[:128].sum()), acc_ref)
    assert agree >= 0.999
    err_ref = ou.rankspace_error(Y_u[:128], ou.dequant_from_q(q_ref, sf[:128], zf[:128]), Vs)
    assert abs(float(ea[:128].mean()) - float(err_ref.mean())) <= 1e-3 * float(err_ref.mean())
    # the error never increases, and row blocks are independent (second block polished alone)
    assert bool((ea <= eb * (1 + 1e-5) + 1e-9).all())
    q2, _, ea2, _, _ = ops.uniform_cd_polish(W[128:].to(gpu), q0[128:].to(gpu), sg[128:].to(gpu), zg[128:].to(gpu),
                                            128, maxq, Vs.to(gpu), Hw.to(gpu), block_rows=128, sweeps=3,
                                            select=False)
    assert float((q2.cpu() == q[128:].cpu()).float().mean()) >= 0.999


def test_cd_polish_x6_products_match_oracle(gpu):
    # the polish's two full products (rhs = residual Vs^T as (residual diag(S)) V^T, final x Vs) on
    # the packed rank-space operator: same codes as the oracle and as the fp32-kernel polish
    W, Hw, V, S, Vs, sg, zg, sf, zf, xr, maxq = _setup_block(256, 512, 4, 128, "cd6")
    q0 = torch.clamp(torch.round(W / sf) + zf, 0, maxq).to(torch.uint8)
    Y_u = W @ Vs
    x_pol, _ = ou.scalar_greedy_cd(xr[:128], Y_u[:128], Vs, Hw, sf[:128], zf[:128], maxq, 3)
    q_ref = ou.nearest_atom_idx(x_pol, sf[:128], zf[:128], maxq)
    Vg, Sg, Vsg = V.to(gpu), S.to(gpu), Vs.to(gpu)
    pk = ops.rankspace_pack(Vg, Vsg)
    args = (W.to(gpu), q0.to(gpu), sg.to(gpu), zg.to(gpu), 128, maxq, Vsg, Hw.to(gpu))
    q, eb, ea, imp, acc = ops.uniform_cd_polish(*args, block_rows=128, sweeps=3, select=False, S=Sg, packed=pk)
    assert float((q[:128].cpu().long() == q_ref.long()).float().mean()) >= 0.999
    err_ref = ou.rankspace_error(Y_u[:128], ou.dequant_from_q(q_ref, sf[:128], zf[:128]), Vs)
    assert abs(float(ea[:128].mean()) - float(err_ref.mean())) <= 1e-3 * float(err_ref.mean())
    q32, eb32, ea32, _, _ = ops.uniform_cd_polish(*args, block_rows=128, sweeps=3, select=False)
    assert float((q == q32).float().mean()) >= 0.999
    assert _rel(eb.cpu(), eb32.cpu()) < 1e-4 and _rel(ea.cpu(), ea32.cpu()) < 1e-4
    with pytest.raises(ValueError):
        ops.uniform_cd_polish(*args, block_rows=128, sweeps=3, select=False, S=Sg)


@pytest.mark.parametrize("layout", ["contiguous", "act_order"])
def test_postprocess_gptq_polish_matches_oracle(gpu, layout):
    """postprocess_gptq_quantization (mpq/adapters/gptqmodel.py:1250-1470): one greedy order over all
    rows, keep-if-better per row, module fail-closed; against the oracle's scalar CD.  ``act_order``:
    GPTQModel's desc_act layout, groups formed over the columns in descending order of diag(H) and
    column c taking group g_idx[c] (the reference's _expand_group_params_from_gidx)."""
    from mpq_amd.adapters.gptqmodel import postprocess_gptq_quantization

    rows, n, gs, bits = 96, 256, 128, 3
    maxq = 2 ** bits - 1
    W, H = make_layer(rows, n, tokens=1024, seed_key="post:gptq")
    if layout == "act_order":
        perm = torch.argsort(torch.diagonal(H), descending=True, stable=True)
        g_idx = (torch.argsort(perm) // gs).to(torch.int32)
        Wp = W[:, perm]
    else:
        g_idx = torch.arange(n, dtype=torch.int32) // gs
        Wp = W
    sg, zg = ou.gptq_find_params(Wp.reshape(-1, gs), maxq)
    sg, zg = sg.reshape(rows, n // gs), zg.reshape(rows, n // gs)
    sf, zf = sg[:, g_idx.long()], zg[:, g_idx.long()]
    Q0 = sf * (torch.clamp(torch.round(W / sf) + zf, 0, maxq) - zf)

    class Q:
        pass

    qcfg = Q()
    qcfg.bits, qcfg.group_size = bits, gs
    qcfg.mpq = Q()
    qcfg.mpq.polish_mode, qcfg.mpq.polish_sweeps = "block_cd", 3
    Qf, qf, _, _, _, _, st = postprocess_gptq_quantization(W=W.to(gpu), H=(2.0 * H).to(gpu), Q_init=Q0.to(gpu),
                                                           scale_groups=sg.to(gpu), zero_groups=zg.to(gpu),
                                                           g_idx=g_idx.to(gpu), qcfg=qcfg, module_name="m")
    # oracle: same eigenbasis, scalar greedy CD over all rows, keep-if-better
    lam, V, _ = ou.hessian_eigen(H)
    Vs = V * torch.sqrt(lam).unsqueeze(0)
    Yu = W.matmul(Vs)
    x_pol, _ = ou.scalar_greedy_cd(Q0, Yu, Vs, H, sf, zf, maxq, 3)
    e0 = ou.rankspace_error(Yu, Q0, Vs)
    e1 = ou.rankspace_error(Yu, x_pol, Vs)
    ref = torch.where((e1 + 1e-12 < e0).unsqueeze(1), x_pol, Q0)
    e_ref = ou.rankspace_error(Yu, ref, Vs)
    got = Qf.cpu()
    e_got = ou.rankspace_error(Yu, got, Vs)
    assert float(e_got.mean()) <= float(e0.mean()) + 1e-6
    assert abs(float(e_got.mean()) - float(e_ref.mean())) <= 5e-3 * float(e_ref.mean())
    agree = float((got == ref).float().mean())
    floor = 1.0
    if agree < 0.999:
        # the reference's other dispatch of the same polish (its CPU block CD, mpq/solver.py:336-366)
        x_blk, _ = ou.block_cd_scalar(Q0, Yu, Vs, sf, zf, maxq, 3)
        e_blk = ou.rankspace_error(Yu, x_blk, Vs)
        ref_blk = torch.where((e_blk + 1e-12 < e0).unsqueeze(1), x_blk, Q0)
        floor = float((ref_blk == ref).float().mean())
    print(f"postprocess polish ({layout}): codes {agree:.5f} (reference floor {floor:.5f})")
    assert agree >= min(0.999, floor), (agree, floor)
    assert not st["module_fail_closed"] and st["polish_updates"] > 0
    assert torch.equal(got, sf * (qf.cpu().float() - zf))


def test_vamp_early_stop_then_call_on_another_stream(gpu):
    """Status mailbox (two slots, one per pending publish): a block that stops at the best iterate
    leaves the look-ahead pass's status publish queued; the driver waits for it before returning, so
    a second call from the same thread on another stream, started right away, reads only its own
    statuses.  Both results must equal the same solves run alone on the default stream."""
    cases = []
    for key in ("mb0", "mb3"):  # oracle: best-iterate stops at 7 and 9 of 16 iterations
        W, Hw, V, S, Vs, sg, zg, sf, zf, xr, maxq = _setup_block(128, 512, 4, 128, key, rotate=True)
        cases.append([t.to(gpu) for t in (W, xr, sg, zg)] + [maxq] + [t.to(gpu) for t in (V, S, Vs)])
    vcfg = UniformVampConfig(**{k: v for k, v in RECIPE.items()})

    def solve(c):
        W, xr, sg, zg, maxq, V, S, Vs = c
        return ops.uniform_vamp_solve(W, xr, sg, zg, 128, maxq, V, S, Vs, vcfg)

    alone = [solve(c) for c in cases]
    torch.cuda.synchronize()
    assert all(r[4]["stop_iter"] < 15 for r in alone), [r[4]["stop_iter"] for r in alone]
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    with torch.cuda.stream(sa):
        ra = solve(cases[0])
    with torch.cuda.stream(sb):
        rb = solve(cases[1])
    torch.cuda.synchronize()
    for got, ref in ((ra, alone[0]), (rb, alone[1])):
        assert torch.equal(got[0], ref[0])
        assert torch.equal(got[2], ref[2])
        assert got[4]["stop_iter"] == ref[4]["stop_iter"] and got[4]["best_iter"] == ref[4]["best_iter"]
