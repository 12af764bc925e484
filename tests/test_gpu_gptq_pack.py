"""GPU: GPTQModel int32 packing (mpq_gptq_pack) bit-exact against the bit-stream oracle
(oracle/gptq_pack.py), the packed-basis weight rebuild, and the internal-Hadamard input hooks
(mpq/adapters/gptqmodel.py:1166-1247)."""
import numpy as np
import pytest
import torch

from mpq_amd import ops
from mpq_amd.adapters.gptqmodel import install_internal_hadamard_input_hooks
from mpq_amd.packing import pack_gptq, packed_basis_weight
from mpq_amd.rotation import apply_right_block_hadamard, resolve_block_hadamard_plan, sample_rademacher_signs
from oracle import gptq_pack as og

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
@pytest.mark.parametrize("fmt", ["v1", "v2"])
@pytest.mark.parametrize("rows,n,gs", [(64, 256, 128), (96, 1024, 128), (32, 96, 32)])
def test_pack_bit_exact(gpu, bits, fmt, rows, n, gs):
    rng = np.random.default_rng(bits * 131 + rows)
    q = rng.integers(0, 1 << bits, size=(rows, n)).astype(np.uint8)
    G = (n + gs - 1) // gs
    zero = rng.integers(1 if fmt == "v1" else 0, 1 << bits, size=(rows, G)).astype(np.float32)
    scale = (rng.random((rows, G)) * 0.01 + 1e-4).astype(np.float32)
    got = pack_gptq(torch.from_numpy(q).to(gpu), torch.from_numpy(scale).to(gpu), torch.from_numpy(zero).to(gpu),
                    bits=bits, group_size=gs, fmt=fmt)
    ref = og.pack_gptq(q, scale, zero, bits, gs, fmt)
    for k in ("qweight", "qzeros", "g_idx"):
        assert np.array_equal(got[k].cpu().numpy(), ref[k]), k
    assert np.array_equal(got["scales"].cpu().numpy().view(np.uint16), ref["scales"].view(np.uint16))


def test_pack_rejects_bad_shapes(gpu):
    q = torch.zeros(30, 64, dtype=torch.uint8, device=gpu)
    s = torch.ones(30, 1, device=gpu)
    with pytest.raises(ValueError):
        pack_gptq(q, s, s, bits=4, group_size=64)
    with pytest.raises(ValueError):
        pack_gptq(torch.zeros(32, 64, dtype=torch.uint8, device=gpu), s[:1].expand(32, 1).contiguous(),
                  s[:1].expand(32, 1).contiguous(), bits=5, group_size=64)


def test_packed_basis_weight(gpu):
    rng = np.random.default_rng(7)
    q = rng.integers(0, 8, size=(64, 256)).astype(np.uint8)
    scale = rng.random((64, 2)).astype(np.float32)
    zero = rng.integers(0, 8, size=(64, 2)).astype(np.float32)
    got = packed_basis_weight(torch.from_numpy(q).to(gpu), torch.from_numpy(scale).to(gpu),
                              torch.from_numpy(zero).to(gpu), group_size=128).cpu()
    sf = torch.from_numpy(scale).repeat_interleave(128, 1)
    zf = torch.from_numpy(zero).repeat_interleave(128, 1)
    assert torch.equal(got, sf * (torch.from_numpy(q).float() - zf))


class _Packed(torch.nn.Module):
    def __init__(self, in_features, out_features):
        super().__init__()
        self.in_features = in_features
        self.register_buffer("qweight", torch.zeros(in_features * 4 // 32, out_features, dtype=torch.int32))
        self.register_buffer("qzeros", torch.zeros(1, out_features * 4 // 32, dtype=torch.int32))
        self.register_buffer("scales", torch.zeros(1, out_features, dtype=torch.float16))
        self.seen = None

    def forward(self, x):
        self.seen = x
        return x


def test_internal_hadamard_input_hooks(gpu):
    model = torch.nn.Module()
    model.layers = torch.nn.ModuleList([_Packed(1024, 64), _Packed(3 * 512, 64)])
    model.plain = torch.nn.Linear(8, 8)
    model.to(gpu)
    assert install_internal_hadamard_input_hooks(model, rotation_seed=0) == 2
    assert install_internal_hadamard_input_hooks(model, rotation_seed=0) == 0  # idempotent
    for name, mod, width in (("layers.0", model.layers[0], 1024), ("layers.1", model.layers[1], 1536)):
        x = torch.randn(2, 5, width, device=gpu, dtype=torch.bfloat16)
        mod(x)
        _, had = resolve_block_hadamard_plan(width)
        signs = sample_rademacher_signs(width=width, key=f"{name}:full", seed=0, device=gpu)
        ref = apply_right_block_hadamard(x.reshape(-1, width).float(), signs=signs, had_dim=had)
        assert mod.seen.dtype == torch.bfloat16 and mod.seen.shape == x.shape
        assert torch.equal(mod.seen.reshape(-1, width), ref.to(torch.bfloat16))
    with pytest.raises(RuntimeError):
        model.layers[0](torch.randn(3, 100, device=gpu))
