"""Write golden input/output vectors from the reference implementation (run in the build container only).

Only functions whose results no closed form, brute force or invariant pins bit for bit are
recorded here: the VAMP loops (discrete control flow: gamma retries, damping, best-iterate stop,
EM chain), the greedy coordinate-descent sweeps (near-tie accept cascades) and the E8P12
posterior (torch's reduction orders).  The reference runs on its CPU dispatch (eager denoisers,
``block_coordinate_descent_rankspace`` / ``uniform_scalar_diag_greedy_cd(update_backend="torch")``).
The E8P12 functions need a codebook object of class ``E8P12_codebook``; the build's own table
(mpq_amd/codebook.py) is passed in.

Usage:  python tests/golden/make_golden.py /root/reference [all|refine|udriver|options]
Output: tests/golden/*.npz (inputs and outputs only; no reference code is stored).
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))


def _np(d):
    out = {}
    for k, v in d.items():
        if isinstance(v, torch.Tensor):
            out[k] = v.detach().cpu().numpy()
        elif isinstance(v, (int, float, bool)):
            out[k] = np.asarray(v)
    return out


def main(ref_root: str) -> None:
    sys.path.insert(0, ROOT)
    sys.path.insert(0, ref_root)
    torch.set_num_threads(1)  # fixed BLAS partition for reproducible vectors
    from mpq.linear import vamp_rankspace_error  # noqa: F401  (reference)
    from mpq.polish.triton_scalar_cd import uniform_scalar_diag_greedy_cd  # reference
    from mpq.priors.e8p12 import vamp_vector_discrete_mmse_e8p12, vamp_vector_map_e8p12  # reference
    from mpq.solver import (  # reference
        E8P12VampConfig as RefE8Cfg,
        UniformVampConfig as RefUCfg,
        solve_e8p12_rankspace_vamp,
        solve_uniform_rankspace_vamp,
    )

    from mpq_amd.codebook import E8P12_codebook, grid_numpy
    from oracle import uniform as ou
    from tests.uniform_cases import make_layer

    # ---- uniform VAMP row blocks (CPU dispatch, polish via block_coordinate_descent_rankspace)
    for name, rotate, bits, rows, cols in (("uvamp_r0_b4", False, 4, 64, 256), ("uvamp_r1_b3", True, 3, 64, 256),
                                           ("uvamp_r1_b4", True, 4, 64, 256)):
        W, H = make_layer(rows, cols, tokens=1024, seed_key=f"golden:{name}")
        lam, V, _ = ou.hessian_eigen(H)
        if rotate:
            signs, had = ou.rotation_plan(cols, name)
            W = ou.hadamard_rows(W * signs.view(1, -1), had)
            H = ou.hadamard_rows(ou.hadamard_rows(H.T.contiguous() * signs.view(1, -1), had).T.contiguous()
                                 * signs.view(1, -1), had)
            V = ou.hadamard_rows(V.T.contiguous() * signs.view(1, -1), had).T.contiguous()
        S = torch.sqrt(lam)
        Vs = V * S.unsqueeze(0)
        maxq = 2 ** bits - 1
        sc, zc = zip(*[ou.gptq_find_params(W[:, g:g + 128], maxq) for g in range(0, cols, 128)])
        sf = torch.repeat_interleave(torch.cat(sc, 1), 128, dim=1)
        zf = torch.repeat_interleave(torch.cat(zc, 1), 128, dim=1)
        xr = sf * (torch.clamp(torch.round(W / sf) + zf, 0, maxq) - zf)
        cfg = RefUCfg(iters=16, damping=0.5, prior_tau=0.2, polish_sweeps=3, polish_mode="block_cd",
                      vamp_backend="eager", block_cd_backend="eager")
        cfg0 = RefUCfg(iters=16, damping=0.5, prior_tau=0.2, polish_sweeps=0, vamp_backend="eager")
        q0, x0, e0, r0, st0 = solve_uniform_rankspace_vamp(W=W, x_rtn=xr, scale_full=sf, zero_full=zf, maxq=maxq,
                                                           V=V, Vh=V.T.contiguous(), S=S, Vs=Vs, cfg=cfg0,
                                                           gram_full=H, log_stats=False)
        q, x, e, r, st = solve_uniform_rankspace_vamp(W=W, x_rtn=xr, scale_full=sf, zero_full=zf, maxq=maxq, V=V,
                                                      Vh=V.T.contiguous(), S=S, Vs=Vs, cfg=cfg, gram_full=H,
                                                      log_stats=False)
        Yu = W.matmul(Vs)
        xt, _ = uniform_scalar_diag_greedy_cd(x=x0, Y_u=Yu, Vs=Vs, gram_full=H, scale=sf, zero=zf, maxq=maxq,
                                              sweeps=3, update_backend="torch")
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **_np({
            "W": W, "H": H, "V": V, "S": S, "scale_full": sf, "zero_full": zf, "x_rtn": xr, "maxq": maxq,
            "q_vamp": q0, "err_vamp": e0, "best_iter": st0["best_iter"], "stop_iter": st0["stop_iter"],
            "obs_final_vamp": st0["obs_precision_final"], "q_final": q, "err_final": e, "rtn_err": r,
            "obs_initial": st["obs_precision_initial"], "x_cd_twin": xt}))
        print(name, "best_iter", st0["best_iter"], "stop", st0["stop_iter"], "polish updates", st["polish_updates"])

    # ---- E8P12: MAP, posterior, VAMP loop with the build's table as the codebook
    cb = E8P12_codebook()
    g = torch.Generator().manual_seed(1234)
    rows, nb = 16, 32
    r1 = torch.randn(rows, nb, 8, generator=g) * 0.7
    center = r1 + 0.2 * torch.randn(rows, nb, 8, generator=g)
    gam = torch.exp(torch.randn(rows, 1, generator=g)) * 2.0
    mp = vamp_vector_map_e8p12(r1_blocks=r1, gamma1=gam, cb=cb, prior_center_blocks=center, prior_tau=0.25)
    post = vamp_vector_discrete_mmse_e8p12(r1_blocks=r1, gamma1=gam, cb=cb, prior_center_blocks=center,
                                           prior_tau=0.25, compile_prior=False, return_logZ_blocks=True)
    np.savez_compressed(os.path.join(HERE, "e8p12_posterior.npz"), **_np({
        "r1": r1, "gamma1": gam, "center": center, "map_idxs": mp["map_idxs"], "x1": post["x1_blocks"],
        "var1": post["var1"], "alpha1": post["alpha1"], "logZ": post["logZ_blocks"],
        "post_map_idxs": post["map_idxs"]}))
    print("e8p12 posterior written")

    W, H = make_layer(32, 128, tokens=1024, seed_key="golden:e8vamp", heavy=True)
    Wr = W / W.square().mean().sqrt()
    lamq, Vq, _ = ou.hessian_eigen(H)
    S = torch.sqrt(lamq)
    Vs = Vq * S.unsqueeze(0)
    cb_t = torch.from_numpy(grid_numpy())
    hat0 = cb_t[torch.from_numpy(np.asarray(vamp_vector_map_e8p12(
        r1_blocks=Wr.view(32, 16, 8), gamma1=torch.ones(32, 1), cb=cb)["map_idxs"]).reshape(-1))].view(32, 128)
    ecfg = RefE8Cfg(iters=16, polish_sweeps=3, compile_prior=False)
    hat, idx, err, est = solve_e8p12_rankspace_vamp(Wr=Wr, hatWr_init=hat0, cb=cb, V=Vq, Vh=Vq.T.contiguous(), S=S,
                                                    Vs=Vs, cfg=ecfg, log_stats=False)
    ecfg0 = RefE8Cfg(iters=16, polish_sweeps=0, compile_prior=False)
    hatv, idxv, errv, estv = solve_e8p12_rankspace_vamp(Wr=Wr, hatWr_init=hat0, cb=cb, V=Vq, Vh=Vq.T.contiguous(),
                                                        S=S, Vs=Vs, cfg=ecfg0, log_stats=False)
    np.savez_compressed(os.path.join(HERE, "e8p12_vamp.npz"), **_np({
        "Wr": Wr, "H": H, "V": Vq, "S": S, "hat0": hat0, "idx_vamp": idxv, "err_vamp": errv, "idx_final": idx,
        "err_final": err, "obs_initial": est["obs_precision_initial"], "obs_final": est["obs_precision_final"]}))
    print("e8p12 vamp written; polish updates", est["polish_updates"])


def refine_golden(ref_root: str) -> None:
    """The QUIP# adapter driver (mpq_refine_codebook, solver vamp, init rtn) on the CPU: its glue --
    the nearest-codeword start, the rank-space warm start of the observation precision and its carry
    across row blocks -- is pinned by no closed form."""
    sys.path.insert(0, ROOT)
    sys.path.insert(0, ref_root)
    torch.set_num_threads(1)
    import types

    from mpq.adapters.quip_sharp import mpq_refine_codebook  # reference

    from mpq_amd.codebook import grid_numpy, packed_abs
    from oracle import e8p12 as oe8
    from tests.uniform_cases import make_layer

    class E8P12_codebook:  # noqa: N801 - the reference's factor cache requires this class name
        """CPU stand-in with the build's table: exact nearest codeword by brute force (first index)."""
        codesz = 8
        packsz = 1
        idx_dtype = torch.int64

        def __init__(self):
            self.grid = torch.from_numpy(grid_numpy())
            self.grid_packed_abs = torch.from_numpy(packed_abs())

        def quantize(self, X, return_idx=True, **kwargs):
            shape = X.shape
            idx, _ = oe8.bruteforce_nearest(X.reshape(-1, 8).numpy(), self.grid.numpy())
            idx = torch.from_numpy(np.asarray(idx))
            vals = self.grid[idx].view(shape)
            return (vals, idx.view(shape[:-1])) if return_idx else vals

        def maybe_pack_idxs(self, idxs):
            return idxs

        def by_idxs(self, idxs, **kwargs):
            return self.grid[idxs.long()]

    cb = E8P12_codebook()
    W, H = make_layer(256, 128, tokens=1024, seed_key="golden:refine", heavy=True)
    H = H / torch.diagonal(H).mean() + 1e-2 * torch.eye(128)  # QUIP#'s regularised Hessian scale
    Wr = W / W.square().mean().sqrt()
    hat0, idx0 = cb.quantize(Wr.reshape(256, 16, 8))
    hat0 = hat0.reshape(256, 128)
    args = types.SimpleNamespace(mpq_init="rtn", mpq_iters=16, mpq_prior_tau=0.25, mpq_polish_sweeps=3,
                                 mpq_compile_prior=False, mpq_block_rows=128)
    hat, idx, st = mpq_refine_codebook(Wr, H, hat0, idx0, cb, args, module_name="golden.refine")
    np.savez_compressed(os.path.join(HERE, "e8p12_refine.npz"), **_np({
        "Wr": Wr, "H": H, "hat": hat, "idx": idx, "obs_initial": float(st["obs_precision_initial"]),
        "obs_final": float(st["obs_precision_final"])}))
    print("refine written; obs", st["obs_precision_initial"], "->", st["obs_precision_final"])


def udriver_golden(ref_root: str) -> None:
    """The GPTQ adapter's per-linear driver (run_mpq_quantization, solver vamp) on the CPU: its glue --
    the rotation signs, the eigenvalue floor of the unrotated Hessian, the rotated eigenbasis, the
    group parameters, the rank-space warm start summed over row blocks and the observation precision
    carried across row blocks -- is pinned by no closed form.  GPTQModel's quantizer is not vendored;
    the stand-in is the min-max formula the oracle uses (oracle/uniform.py gptq_find_params)."""
    sys.path.insert(0, ROOT)
    sys.path.insert(0, ref_root)
    torch.set_num_threads(1)
    import types

    from mpq.adapters.gptqmodel import GPTQAdapterConfig, run_mpq_quantization  # reference
    from mpq.rotation import sample_rademacher_signs  # reference
    from mpq.solver import UniformVampConfig as RefUCfg  # reference

    from oracle import uniform as ou
    from tests.uniform_cases import make_layer

    class MinMaxQuantizer:
        """GPTQModel's Quantizer interface (find_params sets .scale / .zero per row)."""

        def __init__(self, maxq):
            self.maxq = maxq

        def find_params(self, x, weight=True):
            self.scale, self.zero = ou.gptq_find_params(x.to(torch.float32), self.maxq)

    out = {}
    for key in ("model.layers.0.mlp.up_proj", "model.layers.3.self_attn.q_proj", "golden.udriver"):
        for width in (512, 1024):
            out[f"signs:{key}:{width}"] = sample_rademacher_signs(width=width, key=f"{key}:full", seed=0,
                                                                  device=torch.device("cpu"))
    np.savez_compressed(os.path.join(HERE, "rademacher_signs.npz"),
                        **{k.replace(":", "|"): v.numpy() for k, v in out.items()})
    print("rademacher signs written")

    rows, cols = 384, 256
    for rotation, bits, desc_act in (("none", 4, False), ("internal_hadamard", 3, False),
                                     ("internal_hadamard", 4, True)):
        name = "model.layers.0.mlp.up_proj"
        tag = rotation + ("_desc_act" if desc_act else "")
        W, H = make_layer(rows, cols, tokens=1024, seed_key=f"golden:udriver:{tag}")
        Hg = 2.0 * H  # GPTQModel convention: the adapter halves it (mpq/adapters/gptqmodel.py:702)
        qcfg = types.SimpleNamespace(bits=bits, group_size=128, desc_act=desc_act,
                                     mpq=types.SimpleNamespace(rotation_mode=rotation, solver="vamp"))
        vcfg = RefUCfg(iters=16, damping=0.5, prior_tau=0.2, polish_sweeps=3, polish_mode="block_cd",
                       vamp_backend="eager", block_cd_backend="eager")
        Q, q, sc, zr, g_idx, _, st = run_mpq_quantization(W=W, H=Hg, quantizer=MinMaxQuantizer(2 ** bits - 1),
                                                          qcfg=qcfg, module_name=name, vamp_cfg=vcfg,
                                                          adapter_cfg=GPTQAdapterConfig(block_rows=128))
        bst = st["block_stats"]
        # W is rebuilt from its seed by the test (a draw from torch's CPU generator); H is stored
        # (X^T X on the CPU rounds by the BLAS partition)
        np.savez_compressed(os.path.join(HERE, f"udriver_{tag}.npz"), **_np({
            "bits": bits, "H": Hg, "Q": Q, "q_int": q, "scale": sc, "zero": zr, "g_idx": g_idx,
            "obs_initial": float(st["obs_precision_initial"]), "obs_final": float(st["obs_precision_final"]),
            "eigen_floor": float(st["eigen_floor"]), "layer_error_sum": float(st["layer_error_sum"]),
            "block_obs_final": torch.tensor([float(b["obs_precision_final"]) for b in bst], dtype=torch.float64),
            "block_best_iter": torch.tensor([int(b["best_iter"]) for b in bst]),
            "block_stop_iter": torch.tensor([int(b["stop_iter"]) for b in bst]),
            "polish_updates": torch.tensor([float(b.get("polish_updates", 0.0)) for b in bst], dtype=torch.float64)}))
        print("udriver", tag, "obs", st["obs_precision_initial"], "->", st["obs_precision_final"],
              "stops", [b["stop_iter"] for b in bst])


def options_golden(ref_root: str) -> None:
    """The VAMP solvers' non-recipe options: the uniform loop with another r1 start, EM off, a fixed
    observation precision (alone and with a caller's warm start), no damping and the round-mean final
    decision; the E8P12 loop with best-iterate tracking, without a prior, with a fixed precision and
    with the other prior scales (rms, mean |W|, unit)."""
    sys.path.insert(0, ROOT)
    sys.path.insert(0, ref_root)
    torch.set_num_threads(1)
    from mpq.priors.e8p12 import vamp_vector_map_e8p12  # reference
    from mpq.solver import (  # reference
        E8P12VampConfig as RefE8Cfg,
        UniformVampConfig as RefUCfg,
        solve_e8p12_rankspace_vamp,
        solve_uniform_rankspace_vamp,
    )

    from mpq_amd.codebook import E8P12_codebook, grid_numpy
    from oracle import uniform as ou
    from tests.uniform_cases import make_layer

    rows, cols, bits = 64, 256, 4
    W, H = make_layer(rows, cols, tokens=1024, seed_key="golden:options")
    lam, V, _ = ou.hessian_eigen(H)
    S = torch.sqrt(lam)
    Vs = V * S.unsqueeze(0)
    maxq = 2 ** bits - 1
    sc, zc = zip(*[ou.gptq_find_params(W[:, g:g + 128], maxq) for g in range(0, cols, 128)])
    sf = torch.repeat_interleave(torch.cat(sc, 1), 128, dim=1)
    zf = torch.repeat_interleave(torch.cat(zc, 1), 128, dim=1)
    xr = sf * (torch.clamp(torch.round(W / sf) + zf, 0, maxq) - zf)
    out = {"W": W, "H": H, "V": V, "S": S, "scale_full": sf, "zero_full": zf, "x_rtn": xr, "maxq": maxq}
    variants = {"init_float": (dict(init_from="float"), None), "init_zero": (dict(init_from="zero"), None),
                "em_off": (dict(em_obs_precision=False), None), "obs_fixed": (dict(obs_precision=50.0), None),
                "obs_warm_start": (dict(obs_precision=50.0), 200.0), "undamped": (dict(damping=1.0), None),
                "round_mean": (dict(final_decision="round_mean", gamma_start=0.01, prior_tau=2.0), None)}
    for name, (extra, obs_init) in variants.items():
        kw = dict(iters=16, damping=0.5, prior_tau=0.2, polish_sweeps=0, vamp_backend="eager")
        kw.update(extra)
        q, x, e, r, st = solve_uniform_rankspace_vamp(W=W, x_rtn=xr, scale_full=sf, zero_full=zf, maxq=maxq, V=V,
                                                      Vh=V.T.contiguous(), S=S, Vs=Vs, cfg=RefUCfg(**kw),
                                                      obs_precision_init=obs_init, log_stats=False)
        out.update({f"u_{name}_q": q, f"u_{name}_best_iter": int(st["best_iter"]),
                    f"u_{name}_stop_iter": int(st["stop_iter"]),
                    f"u_{name}_obs_final": float(st["obs_precision_final"])})
        print("uniform", name, "best/stop", st["best_iter"], st["stop_iter"], "obs", st["obs_precision_final"])

    cb = E8P12_codebook()
    We, He = make_layer(32, 128, tokens=1024, seed_key="golden:e8options", heavy=True)
    Wr = We / We.square().mean().sqrt()
    lamq, Vq, _ = ou.hessian_eigen(He)
    Sq = torch.sqrt(lamq)
    Vsq = Vq * Sq.unsqueeze(0)
    cb_t = torch.from_numpy(grid_numpy())
    hat0 = cb_t[torch.from_numpy(np.asarray(vamp_vector_map_e8p12(
        r1_blocks=Wr.view(32, 16, 8), gamma1=torch.ones(32, 1), cb=cb)["map_idxs"]).reshape(-1))].view(32, 128)
    out.update({"e_Wr": Wr, "e_H": He, "e_V": Vq, "e_S": Sq, "e_hat0": hat0})
    e_variants = {"best_iterate": dict(best_iterate=True), "no_prior": dict(prior_tau=0.0),
                  "obs_fixed": dict(obs_precision=0.1), "prior_rms": dict(prior_tau_scale_mode="rms"),
                  "prior_mean_abs": dict(prior_tau_scale_mode="mean_abs"),
                  "prior_unit": dict(prior_tau_scale_mode="none")}
    for name, extra in e_variants.items():
        ecfg = RefE8Cfg(iters=16, polish_sweeps=0, compile_prior=False, **extra)
        hat, idx, err, est = solve_e8p12_rankspace_vamp(Wr=Wr, hatWr_init=hat0, cb=cb, V=Vq, Vh=Vq.T.contiguous(),
                                                        S=Sq, Vs=Vsq, cfg=ecfg, log_stats=False)
        out.update({f"e_{name}_idx": idx, f"e_{name}_best_iter": int(est["best_iter"]),
                    f"e_{name}_stop_iter": int(est["stop_iter"]),
                    f"e_{name}_obs_final": float(est["obs_precision_final"])})
        print("e8p12", name, "best/stop", est["best_iter"], est["stop_iter"], "obs", est["obs_precision_final"])
    np.savez_compressed(os.path.join(HERE, "vamp_options.npz"), **_np(out))


if __name__ == "__main__":
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    part = sys.argv[2] if len(sys.argv) > 2 else "all"
    if part == "refine":
        refine_golden(ref)
    elif part == "udriver":
        udriver_golden(ref)
    elif part == "options":
        options_golden(ref)
    else:
        main(ref)
        refine_golden(ref)
        udriver_golden(ref)
        options_golden(ref)
