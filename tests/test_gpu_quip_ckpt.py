"""GPU: the QUIP# checkpoint writer (mpq_amd/quip_ckpt.py): the RHT on the HIP kernels against the fp64
closed form (oracle/rht.py), and a written decoder layer's ckpt dicts (layout and round trip)."""
import types

import pytest
import torch

from mpq_amd import codebook, quip_ckpt
from oracle import rht
from tests.uniform_cases import make_layer

pytestmark = pytest.mark.gpu


def _rel(a, b):
    return float((a.double() - b.double()).norm() / b.double().norm())


@pytest.mark.parametrize("m,n", [(512, 256), (384, 256), (256, 2048)])
def test_rht_matches_closed_form(gpu, m, n):
    g = torch.Generator().manual_seed(m + n)
    W = torch.randn(m, n, generator=g)
    X = torch.randn(2 * n, n, generator=g)
    H = X.T @ X / (2 * n)
    SU = torch.randint(0, 2, (n,), generator=g).float() * 2 - 1
    SV = torch.randint(0, 2, (m,), generator=g).float() * 2 - 1
    pow2 = (m & (m - 1)) == 0
    if not pow2:  # quip-sharp's had-K transform is not provided: refused unless the block fallback is asked for
        with pytest.raises(ValueError, match="not a power of two"):
            quip_ckpt.incoherence_preprocess(H.to(gpu), W.to(gpu), SU.to(gpu), SV.to(gpu))
    Hr, Wr, lr, rr = quip_ckpt.incoherence_preprocess(H.to(gpu), W.to(gpu), SU.to(gpu), SV.to(gpu),
                                                      allow_block=not pow2)
    assert _rel(Hr.cpu(), rht.rht_h(H, SU)) < 1e-6
    assert _rel(Wr.cpu(), rht.rht_w(W, SU, SV)) < 1e-6
    assert rr == "" and (lr == "") == pow2
    back = quip_ckpt.incoherence_process(Wr, SU.to(gpu), SV.to(gpu), allow_block=not pow2)
    assert _rel(back.cpu(), W) < 1e-6
    assert _rel(back.cpu(), rht.incoherence_process(Wr.cpu(), SU, SV)) < 1e-6


def _args():
    return types.SimpleNamespace(mpq_init="rtn", mpq_iters=8, mpq_prior_tau=0.25, mpq_polish_sweeps=3, seed=0,
                                 incoh_mode="had", use_fp64=False, lora_rank=0, scale_override=0.0)


def test_layer_ckpt_layout_and_round_trip(gpu, tmp_path):
    hidden, inter = 256, 512
    cb = codebook.E8P12_codebook(gpu)
    g = torch.Generator().manual_seed(7)

    def w(o, i):
        return (0.02 * torch.randn(o, i, generator=g)).to(torch.bfloat16).float()

    def hess(n, key):
        _, H = make_layer(8, n, tokens=4 * n, seed_key=key, heavy=True)
        return quip_ckpt.regularize_h(H, 1e-2)

    H_attn, H_o, H_down = hess(hidden, "ck:attn"), hess(hidden, "ck:o"), hess(inter, "ck:down")
    linears = {
        "qkv": ([w(hidden, hidden), w(64, hidden), w(64, hidden)], H_attn),
        "o": ([w(hidden, hidden)], H_o),
        "up": ([w(inter, hidden), w(inter, hidden)], H_attn),
        "down": ([w(hidden, inter)], H_down),
    }
    # the fused qkv has 384 rows (not a power of two): refused without the block-Hadamard opt-in
    with pytest.raises(ValueError, match="not a power of two"):
        quip_ckpt.quantize_layer_to_ckpt(save_dir=str(tmp_path / "refused"), idx=3, linears={"qkv": linears["qkv"]},
                                         cb=cb, args=_args(), device=gpu)
    errs = quip_ckpt.quantize_layer_to_ckpt(save_dir=str(tmp_path), idx=3, linears=linears, cb=cb, args=_args(),
                                            device=gpu, allow_block_hadamard=True)
    for name, (weights, H) in linears.items():
        path = tmp_path / f"3_{name}.pt"
        saved = torch.load(path, map_location="cpu", weights_only=True)
        m = sum(x.shape[0] for x in weights)
        n = weights[0].shape[1]
        assert saved["Qidxs"].dtype == torch.int64 and tuple(saved["Qidxs"].shape) == (m, n // 8)
        assert saved["SU"].dtype == torch.float16 and tuple(saved["SU"].shape) == (n,)
        assert saved["SV"].dtype == torch.float16 and tuple(saved["SV"].shape) == (m,)
        assert bool((saved["SU"].abs() == 1).all())
        assert saved["fused"] == (len(weights) > 1)
        assert [tuple(s) for s in saved["shapes"]] == [tuple(x.shape) for x in weights]
        assert len(saved["scales"]) == len(weights)
        if len(weights) == 1:
            assert saved["scales"] == [1.0]
        assert saved["input_fingerprint"]["w_shape"] == [m, n]
        assert saved["scaleWH"] is None
        pow2 = (m & (m - 1)) == 0
        assert saved["rotation_family"] == ("had" if pow2 else "block_had")
        assert saved["left_rotation_family"] == ("had" if pow2 else "block_had")
        assert saved["left_had_dim"] == (m & -m) and saved["right_had_dim"] == n
        assert saved["right_rotation_family"] == "had"
        assert saved["mpq_stats"]["solver"] == "vamp"
        # round trip: the decoded weights equal the writer's hatW up to the fp16 rounding of SV, and
        # approximate the original weights as a 2-bit code does
        dec = quip_ckpt.load_split_weights(str(path), cb, device=gpu)
        for orig, got in zip(weights, dec):
            assert tuple(got.shape) == tuple(orig.shape)
            rel = _rel(got.cpu(), orig)
            assert rel < 0.45, (name, rel)
        assert 0.0 < errs[name]["err_proxy"] < 0.25
        # the codes decode exactly to codewords of the table
        grid = torch.from_numpy(codebook.grid_numpy())
        hatWr = grid[saved["Qidxs"].reshape(-1)].reshape(m, n)
        back = rht.incoherence_process(hatWr, saved["SU"].float(), saved["SV"].float())
        dec_full = quip_ckpt.decompress_saved_quip(saved, cb, device=gpu).cpu()
        assert _rel(dec_full, back) < 1e-6
        if not pow2:  # a block-Hadamard side recorded as plain 'had' is refused, not decoded another way
            bad = dict(saved, left_rotation_family="had")
            with pytest.raises(ValueError, match="had-K"):
                quip_ckpt.decompress_saved_quip(bad, cb, device=gpu)


def test_refuses_foreign_codebook_and_unsupported_modes(gpu):
    class Foreign:
        codesz = 8
        grid = torch.zeros(65536, 8)

    W = [torch.randn(16, 64)]
    H = torch.eye(64)
    with pytest.raises(ValueError, match="stand-in"):
        quip_ckpt.quantize_weights_to_attr(weights=W, H=H, cb=Foreign(), args=_args(), save_name="x", device=gpu)
    a = _args()
    a.incoh_mode = "kron"
    with pytest.raises(ValueError, match="had"):
        quip_ckpt.quantize_weights_to_attr(weights=W, H=H, cb=codebook.E8P12_codebook(gpu), args=a, save_name="x",
                                           device=gpu)
