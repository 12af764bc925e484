"""GPU: the entry points GPTQModel's hook imports besides the per-linear driver (mpq/adapters/gptqmodel.py
:593-647, :1166-1247): ``prepare_gptq_internal_hadamard`` rotates a linear into the internal
block-Hadamard basis before GPTQModel's own solver, ``finalize_gptq_internal_hadamard`` rotates the
result back, and ``install_internal_hadamard_input_hooks`` rotates a packed module's input instead.

Checked against the oracle's rotation (oracle/uniform.py ``rotation_plan``, whose signs are pinned on
the reference's own vectors, and ``hadamard_rows``): W diag(signs) Had and the two-sided rotation of H
bit for bit, the inverse within fp32 rounding, the pass-through without an internal rotation, and
the fail-closed options.
"""
import types

import pytest
import torch

from mpq_amd.adapters.gptqmodel import (GPTQAdapterConfig, finalize_gptq_internal_hadamard,
                                        install_internal_hadamard_input_hooks, prepare_gptq_internal_hadamard)
from oracle import uniform as ou
from tests.uniform_cases import make_layer

pytestmark = pytest.mark.gpu


def _qcfg(rotation, **extra):
    return types.SimpleNamespace(bits=4, group_size=128, desc_act=False,
                                 mpq=types.SimpleNamespace(rotation_mode=rotation, solver="gptq", **extra))


@pytest.mark.parametrize("name,rows,cols", [("model.layers.0.mlp.up_proj", 256, 1024),
                                            ("model.layers.3.self_attn.q_proj", 96, 512),
                                            ("model.layers.1.mlp.down_proj", 64, 1536)])
def test_prepare_and_finalize_match_oracle_rotation(gpu, name, rows, cols):
    W, H = make_layer(rows, cols, tokens=512, seed_key=f"hooks:{name}")
    Wp, Hp, plan = prepare_gptq_internal_hadamard(W=W.to(gpu), H=H.to(gpu), qcfg=_qcfg("internal_hadamard"),
                                                  module_name=name)
    signs, had = ou.rotation_plan(cols, name)
    assert plan["internal"] and int(plan["block_dim"]) == had == (cols & -cols)
    assert torch.equal(plan["signs"].cpu(), signs)
    W_ref = ou.hadamard_rows(W * signs.view(1, -1), had)
    H_ref = ou.hadamard_rows(H.T.contiguous() * signs.view(1, -1), had).T.contiguous()
    H_ref = ou.hadamard_rows(H_ref * signs.view(1, -1), had)
    assert Wp.dtype == torch.float32 and Hp.dtype == torch.float32
    assert torch.equal(Wp.cpu(), W_ref)
    assert torch.equal(Hp.cpu(), H_ref)
    # back to the original basis: Had diag(signs) (oracle run_mpq_quantization's inverse)
    Q = finalize_gptq_internal_hadamard(Q_work=Wp, rotation_plan=plan)
    Q_ref = ou.hadamard_rows(W_ref, had) * signs.view(1, -1)
    scale = float(W.abs().max())
    assert float((Q.cpu() - Q_ref).abs().max()) <= 1e-6 * scale
    assert float((Q.cpu() - W).abs().max()) <= 1e-5 * scale


def test_prepare_without_rotation_passes_through(gpu):
    W, H = make_layer(64, 256, tokens=256, seed_key="hooks:none")
    Wb = W.to(gpu, torch.bfloat16)
    Wp, Hp, plan = prepare_gptq_internal_hadamard(W=Wb, H=H.to(gpu), qcfg=_qcfg("none"), module_name="m")
    assert not plan["internal"]
    assert Wp.dtype == torch.float32 and torch.equal(Wp, Wb.float())
    assert torch.equal(Hp.cpu(), H)
    Q = finalize_gptq_internal_hadamard(Q_work=Wb, rotation_plan=plan)
    assert Q.dtype == torch.float32 and torch.equal(Q, Wb.float())


def test_prepare_fail_closed_options(gpu):
    W, H = make_layer(64, 256, tokens=256, seed_key="hooks:opts")
    with pytest.raises(ValueError):
        prepare_gptq_internal_hadamard(W=W.to(gpu), H=H.to(gpu), module_name="m",
                                       qcfg=_qcfg("internal_hadamard", paired_matrix_cache_dir="/tmp/x"))
    with pytest.raises(ValueError):
        prepare_gptq_internal_hadamard(W=W.to(gpu), H=H.to(gpu), qcfg=_qcfg("internal_hadamard"), module_name="m",
                                       adapter_cfg=GPTQAdapterConfig(hessian_scale=0.0))


class _Packed(torch.nn.Module):
    """A packed linear as GPTQModel leaves it (qweight / qzeros / scales present) with the dense
    solver-basis weight kept for the check."""

    def __init__(self, W_work):
        super().__init__()
        self.in_features = int(W_work.shape[1])
        self.qweight = torch.zeros(1, dtype=torch.int32)
        self.qzeros = torch.zeros(1, dtype=torch.int32)
        self.scales = torch.zeros(1)
        self.W_work = W_work

    def forward(self, x):
        return x @ self.W_work.T


def test_input_hook_reproduces_dense_weight(gpu):
    """A packed module keeps its weight in the solver basis; with the input hook its output equals the
    dense original-basis weight applied to the unrotated input."""
    name, rows, cols = "proj", 48, 768
    W, H = make_layer(rows, cols, tokens=256, seed_key="hooks:input")
    Wp, _, plan = prepare_gptq_internal_hadamard(W=W.to(gpu), H=H.to(gpu), qcfg=_qcfg("internal_hadamard"),
                                                 module_name=name)
    model = torch.nn.Module()
    model.add_module(name, _Packed(Wp))
    assert install_internal_hadamard_input_hooks(model) == 1
    assert install_internal_hadamard_input_hooks(model) == 0  # already hooked
    x = torch.randn(5, 7, cols, generator=torch.Generator().manual_seed(3)).to(gpu)
    y = getattr(model, name)(x)
    y_ref = x.cpu() @ W.T
    assert tuple(y.shape) == (5, 7, rows)
    assert float((y.cpu() - y_ref).abs().max()) <= 1e-4 * float(y_ref.abs().max())
    with pytest.raises(RuntimeError):
        getattr(model, name)(torch.randn(2, cols + 1, device=gpu))
