"""Pins the oracle's activation quantizer (quantize_row_q8_0_act vllm_safetensors.c:7893-7920).

Closed-form cases fix the arithmetic (IEEE division, +0.5, truncation toward zero, clamp, the
1e-10 floor); the reference's own function built in oracle/_ref fixes everything else bit for bit.
"""
import numpy as np
import pytest


def q(orc, x):
    x = np.asarray(x, np.float32).reshape(1, -1)
    return orc.quantize(x, x.shape[1])


def test_zero_block(orc):
    xq, xd = q(orc, np.zeros(32))
    assert (xq == 0).all()
    assert xd[0, 0] == np.float32(1e-10) / np.float32(127)


def test_amax_127_closed_form(orc):
    # amax = 127 -> d = 1 exactly, so q = trunc(x + 0.5): half-up for x >= 0, toward zero below
    x = np.zeros(32, np.float32)
    x[:12] = [127, -127, 2.5, -2.5, -0.5, 0.5, 0.49999997, -0.49999997, 1.5, -1.5, 126.5, -126.6]
    xq, xd = q(orc, x)
    assert xd[0, 0] == 1.0
    # 0.49999997f + 0.5f = 1 - 2^-25 is a tie in binary32 and rounds to even (1.0) -> q = 1
    assert list(xq[0, :12]) == [127, -126, 3, -2, 0, 1, 1, 0, 2, -1, 127, -126]


def test_negative_amax_maps_to_minus_126(orc):
    rng = np.random.default_rng(3)
    for _ in range(50):
        x = rng.standard_normal(32).astype(np.float32)
        i = int(np.argmax(np.abs(x)))
        x[i] = -abs(x[i])
        xq, _ = q(orc, x)
        assert xq[0, i] == -126
        x[i] = abs(x[i])
        xq, _ = q(orc, x)
        assert xq[0, i] == 127


def test_division_not_reciprocal(orc):
    """x/d vs x*(1/d) differ for some inputs; the oracle must follow the division."""
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((4096, 32)) * 3).astype(np.float32)
    xq, xd = orc.quantize(x, 32)
    d = xd[:, 0]
    v_div = (x / d[:, None]).astype(np.float32)
    v_rcp = (x * (np.float32(1) / d)[:, None]).astype(np.float32)
    q_div = np.clip(np.trunc(v_div + np.float32(0.5)), -127, 127).astype(np.int8)
    q_rcp = np.clip(np.trunc(v_rcp + np.float32(0.5)), -127, 127).astype(np.int8)
    assert (q_div != q_rcp).any(), "test data must separate division from reciprocal"
    assert np.array_equal(xq, q_div)


@pytest.mark.parametrize("scale", [1.0, 1e-3, 1e-30, 1e30, 1e-41])
def test_against_reference(orc, ref, scale):
    rng = np.random.default_rng(int(abs(np.log10(scale))) + 5)
    x = (rng.standard_normal((64, 256)) * scale).astype(np.float32)
    x[3, :32] = 0.0
    x[5, 40] = -x[5, 32:64].__abs__().max() - 1
    xq, xd = orc.quantize(x, 256)
    for t in range(x.shape[0]):
        rq = np.empty(256, np.int8)
        rd = np.empty(8, np.float32)
        ref.kref_quantize_row(x[t].ctypes.data, rq.ctypes.data, rd.ctypes.data, 256)
        assert np.array_equal(xq[t], rq)
        assert np.array_equal(xd[t].view(np.uint32), rd.view(np.uint32))
