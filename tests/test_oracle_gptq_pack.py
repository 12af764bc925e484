"""CPU: pin the GPTQ packing oracle (oracle/gptq_pack.py) with closed-form examples of the layout."""
import numpy as np
import pytest

from oracle import gptq_pack as og


def test_four_bit_nibbles():
    # values 1..8 along the input dimension of one column -> 0x87654321
    q = np.arange(1, 9, dtype=np.uint8).reshape(1, 8)
    q = np.repeat(q, 32, axis=0)  # 32 output columns
    w = og._pack_stream(q, 4)
    assert w.shape == (32, 1)
    assert int(w[0, 0].view(np.uint32)) == 0x87654321


def test_two_and_eight_bit_closed_form():
    q = np.array([[3, 0, 1, 2] * 4], dtype=np.uint8)
    assert int(og._pack_stream(q, 2)[0, 0].view(np.uint32)) == sum(v << (2 * j) for j, v in enumerate([3, 0, 1, 2] * 4))
    q8 = np.array([[0x11, 0x22, 0x33, 0xF4]], dtype=np.uint8)
    assert int(og._pack_stream(q8, 8)[0, 0].view(np.uint32)) == 0xF4332211


def test_three_bit_words_match_the_gptq_pattern():
    # the 32-values-in-3-words pattern written out word by word
    rng = np.random.default_rng(0)
    v = rng.integers(0, 8, size=32).astype(np.uint32)
    w0 = sum(int(v[j]) << (3 * j) for j in range(10)) | ((int(v[10]) << 30) & 0xFFFFFFFF)
    w1 = ((int(v[10]) >> 2) & 1) | sum(int(v[j]) << (3 * (j - 11) + 1) for j in range(11, 21)) | ((int(v[21]) << 31) & 0xFFFFFFFF)
    w2 = ((int(v[21]) >> 1) & 3) | sum(int(v[j]) << (3 * (j - 22) + 2) for j in range(22, 32))
    got = og._pack_stream(v.reshape(1, 32), 3).view(np.uint32).reshape(-1)
    assert [int(x) for x in got] == [w0 & 0xFFFFFFFF, w1 & 0xFFFFFFFF, w2 & 0xFFFFFFFF]


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
@pytest.mark.parametrize("fmt", ["v1", "v2"])
def test_round_trip(bits, fmt):
    rng = np.random.default_rng(bits)
    rows, n, gs = 64, 256, 128
    q = rng.integers(0, 1 << bits, size=(rows, n)).astype(np.uint8)
    zero = rng.integers(1 if fmt == "v1" else 0, 1 << bits, size=(rows, n // gs)).astype(np.float32)
    scale = rng.random((rows, n // gs)).astype(np.float32)
    p = og.pack_gptq(q, scale, zero, bits, gs, fmt)
    assert p["qweight"].shape == (n * bits // 32, rows) and p["qweight"].dtype == np.int32
    assert p["qzeros"].shape == (n // gs, rows * bits // 32)
    assert np.array_equal(og.unpack_qweight(p["qweight"], bits, n), q)
    assert np.array_equal(og.unpack_qzeros(p["qzeros"], bits, rows, fmt), zero.astype(np.int64))
    assert np.array_equal(p["g_idx"], np.arange(n) // gs)
