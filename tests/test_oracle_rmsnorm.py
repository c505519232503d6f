"""Pins the oracle's RMSNorm (kqo_rms_norm) in both of the reference's summation orders.

  * bit for bit against the reference's own dyn_rms_norm (chunked order) and
    dyn_rms_norm_batch (serial order) built in oracle/_ref from /root/reference;
  * exact cases that fix the formula without the reference: constant rows (ss = d*c^2 exactly,
    so rms and the output follow in closed form), a zero row (rms = 1/sqrt(eps)), and a row
    whose sum of squares rounds differently in the two orders (so swapping them fails).
"""
import numpy as np
import pytest

F32 = np.float32


def rows(n, d, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, d)).astype(F32)
    x[0] *= 1e3
    if n > 1:
        x[1] *= 1e-3
    w = (1.0 + 0.1 * rng.standard_normal(d)).astype(F32)
    return x, w


@pytest.mark.parametrize("d", [8, 13, 64, 2048, 4096, 4099])
def test_chunked_matches_reference(orc, ref, d):
    x, w = rows(4, d, d)
    got = orc.rms_norm(x, w, d, 1e-6, chunked=True)
    for t in range(4):
        want = np.empty(d, F32)
        ref.kref_rms_norm(want.ctypes.data, np.ascontiguousarray(x[t]).ctypes.data, w.ctypes.data,
                          d, 1e-6)
        assert np.array_equal(got[t].view(np.uint32), want.view(np.uint32)), (d, t)


@pytest.mark.parametrize("d", [8, 13, 64, 2048, 4096, 4099])
def test_serial_matches_reference_batch(orc, ref, d):
    x, w = rows(5, d, d + 1)
    got = orc.rms_norm(x, w, d, 1e-5, chunked=False)
    want = np.empty_like(x)
    ref.kref_rms_norm_batch(want.ctypes.data, x.ctypes.data, w.ctypes.data, 5, d, 1e-5)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("chunked", [True, False])
def test_closed_forms(orc, chunked):
    d = 256
    w = np.linspace(-2, 2, d).astype(F32)
    x = np.full((1, d), 0.5, F32)                     # ss = 64 exactly in any order
    got = orc.rms_norm(x, w, d, 0.0, chunked)[0]
    rms = F32(1.0) / np.sqrt(F32(64.0) / F32(d))       # = 2 exactly
    assert rms == 2.0
    assert np.array_equal(got, (x[0] * rms) * w)
    z = orc.rms_norm(np.zeros((1, d), F32), w, d, 1e-6, chunked)[0]
    assert np.all(z == 0)
    ones = orc.rms_norm(np.ones((1, d), F32), np.ones(d, F32), d, 1e-6, chunked)[0]
    assert np.all(ones == F32(1.0) / np.sqrt(F32(1.0) + F32(1e-6)))


def test_orders_differ_where_rounding_differs(orc):
    """A row of 16 elements whose squares are 2^24 then fifteen 1s: summed in order the 1s are
    lost one by one (2^24 + 1 rounds back to 2^24); in 8-element chunks the 1s are first added
    to each other, so the chunked total keeps 14 of them."""
    x = np.ones((1, 16), F32)
    x[0, 0] = 4096.0                                    # square 2^24
    w = np.ones(16, F32)
    a = orc.rms_norm(x, w, 16, 0.0, chunked=True)[0]
    b = orc.rms_norm(x, w, 16, 0.0, chunked=False)[0]
    ss_chunked = F32(2 ** 24) + F32(14)                 # (2^24+1+..)+(8 ones): see hsum8 tree
    assert a[1] == F32(1.0) / np.sqrt(ss_chunked / F32(16))
    assert b[1] == F32(1.0) / np.sqrt(F32(2 ** 24) / F32(16))
    assert not np.array_equal(a, b)
