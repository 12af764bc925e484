"""mpq_uniform_cd_sweeps_noalloc (static per-GPU scratch, no allocation) against mpq_uniform_cd_sweeps
(caller workspace), called through the C-ABI: bit-identical state on two calls in a row, the second
with a smaller problem; a problem beyond the static scratch is rejected."""
import pytest
import torch

from mpq_amd import _lib, ops
from tests.test_gpu_cd_exact import _state

pytestmark = pytest.mark.gpu


def _run(noalloc, gpu, case):
    rows, n, bits, gs, block_rows, tokens, key = case
    H, sg, zg, sf, zf, maxq, q0, x0, rhs0, res0, diag = _state(rows, n, bits, gs, key, tokens)
    rhs, x, q, res = rhs0.to(gpu), x0.to(gpu), q0.to(gpu), res0.to(gpu)
    acc = torch.zeros(rows, dtype=torch.int32, device=gpu)
    sg, zg, diag, H = sg.to(gpu), zg.to(gpu), diag.to(gpu), H.to(gpu)
    stream = _lib.stream_handle(gpu)
    head = (rows, n, maxq, block_rows, 3, 0.0, _lib.ptr(rhs), _lib.ptr(x), _lib.ptr(q), _lib.ptr(res), _lib.ptr(acc),
            _lib.ptr(sg), _lib.ptr(zg), gs, _lib.ptr(diag), _lib.ptr(H))
    if noalloc:
        _lib.call("mpq_uniform_cd_sweeps_noalloc", *head, stream)
    else:
        need = int(_lib.load().mpq_uniform_cd_sweeps_workspace_size(rows, n, block_rows))
        ws = ops.workspace(need, gpu)
        _lib.call("mpq_uniform_cd_sweeps", *head, _lib.ptr(ws), int(ws.numel()), stream)
    torch.cuda.synchronize(gpu)
    return rhs.cpu(), x.cpu(), q.cpu(), res.cpu(), acc.cpu()


def test_noalloc_sweeps_match_workspace_entry(gpu):
    assert int(_lib.load().mpq_uniform_cd_sweeps_noalloc_max_bytes()) == 8 << 20
    big = (1024, 1024, 4, 128, 128, 4096, "cfg0:0")
    small = (300, 260, 4, 128, 100, 1024, "ragged")
    for case in (big, small):  # the second call reuses the array the first one filled
        want = _run(False, gpu, case)
        got = _run(True, gpu, case)
        assert int(want[4].sum()) > 0
        for a, b in zip(want, got):
            assert torch.equal(a, b)


def test_noalloc_rejects_problems_beyond_scratch(gpu):
    rows, n = 4096, 4096
    block_rows = 16  # 256 row blocks: greedy orders and gains alone need 8 MiB
    need = int(_lib.load().mpq_uniform_cd_sweeps_workspace_size(rows, n, block_rows))
    assert need > 8 << 20
    t = torch.zeros(1, device=gpu)
    with pytest.raises(ValueError, match="scratch"):
        _lib.call("mpq_uniform_cd_sweeps_noalloc", rows, n, 15, block_rows, 1, 0.0, _lib.ptr(t), _lib.ptr(t),
                  _lib.ptr(t), _lib.ptr(t), _lib.ptr(t), _lib.ptr(t), _lib.ptr(t), 128, _lib.ptr(t), _lib.ptr(t),
                  _lib.stream_handle(gpu))
