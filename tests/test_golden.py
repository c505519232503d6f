"""The committed golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle reproduces the fixtures made by the reference's own code (quantizer, weight
codec, MoE int8 track) bit for bit, and its own dense fixtures (a regression pin for the chains
tests/test_oracle_matmul.py pins). GPU: the HIP path reproduces them through the C ABI
(quantizer and integer block sums bit-exact; dense outputs and MoE within 1e-5 of max|ref|).
These tests read only the fixtures, so they run where /root/reference does not exist."""
import os

import numpy as np
import pytest

from conftest import rel_err

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return dict(np.load(os.path.join(GOLD, name), allow_pickle=False))


# ---- CPU: oracle against the fixtures -------------------------------------------------------

def test_quantizer_matches_reference_fixture(orc):
    g = load("quant.npz")
    q, d = orc.quantize(g["x"], g["x"].shape[1])
    assert np.array_equal(q, g["q"])
    assert np.array_equal(d.view(np.uint32), g["d"].view(np.uint32))


def test_codec_matches_reference_fixture(orc):
    g = load("codec.npz")
    rows, cols = int(g["rows"]), int(g["cols"])
    legacy = np.empty_like(g["legacy"])
    orc.lib().kqo_f32_to_q4_0(legacy.ctypes.data, np.ascontiguousarray(g["w"]).ctypes.data,
                              g["w"].size)
    assert np.array_equal(legacy, g["legacy"])
    tiles = np.empty_like(g["tiles"])
    assert orc.lib().kqo_repack_q4_0_4x4(legacy.ctypes.data, tiles.ctypes.data, rows, cols) == 0
    assert np.array_equal(tiles, g["tiles"])


def test_moe_matches_reference_fixture(orc):
    g = load("moe.npz")
    d, ne, tk, ef = (int(v) for v in g["shape"])
    sel, pr = orc.moe_route(orc.router_logits(g["router"], g["X"], ne, d), tk)
    Y = orc.moe_ffn(g["X"], sel, pr, g["G"], g["U"], g["D"], ne, d, ef)
    assert np.array_equal(Y.view(np.uint32), g["Y"].view(np.uint32))


def test_dense_fixture_regression(orc):
    g = load("dense.npz")
    rows, cols = int(g["rows"]), int(g["cols"])
    lo, hi = orc.block_sums(g["w"], g["xq"], rows, cols)
    assert np.array_equal(lo, g["s_lo"]) and np.array_equal(hi, g["s_hi"])
    for c in range(4):
        assert np.array_equal(orc.matmul(g["w"], g["x"], rows, cols, chain=c), g[f"out_c{c}"])
        assert np.array_equal(orc.matmul(g["w"], g["x"], rows, cols, residual=g["residual"],
                                         chain=c), g[f"res_c{c}"])


# ---- GPU: the HIP path against the same fixtures --------------------------------------------

def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.gpu
def test_gpu_quantizer_fixture(kq4, torch_dev):
    torch = torch_dev
    g = load("quant.npz")
    n, cols = g["x"].shape
    xq = torch.empty((n, cols), dtype=torch.int8, device="cuda")
    xd = torch.empty((n, cols // 32), dtype=torch.float32, device="cuda")
    kq4.quantize_dev(_dev(torch, g["x"]), xq, xd)
    torch.cuda.synchronize()
    assert np.array_equal(xq.cpu().numpy(), g["q"])
    assert np.array_equal(xd.cpu().numpy().view(np.uint32), g["d"].view(np.uint32))


@pytest.mark.gpu
def test_gpu_dense_fixture(kq4, torch_dev):
    torch = torch_dev
    g = load("dense.npz")
    rows, cols = int(g["rows"]), int(g["cols"])
    n = g["x"].shape[0]
    w = kq4.prepare_dev(_dev(torch, g["w"]), rows, cols)
    x, res = _dev(torch, g["x"]), _dev(torch, g["residual"])
    lo = torch.empty((n, rows, cols // 32), dtype=torch.int32, device="cuda")
    hi = torch.empty_like(lo)
    kq4.block_sums_dev(lo, hi, _dev(torch, g["xq"]), w, rows, cols, n)
    out = torch.empty((n, rows), dtype=torch.float32, device="cuda")
    for c in range(4):
        kq4.matmul_dev(out, x, w, rows, cols, chain=c)
        torch.cuda.synchronize()
        r, a = rel_err(out.cpu().numpy(), g[f"out_c{c}"])
        assert r <= 1e-5, (c, r, a)
        kq4.matmul_dev(out, x, w, rows, cols, residual=res, chain=c)
        torch.cuda.synchronize()
        r, a = rel_err(out.cpu().numpy(), g[f"res_c{c}"])
        assert r <= 1e-5, (c, r, a)
    assert np.array_equal(lo.cpu().numpy(), g["s_lo"]) and np.array_equal(hi.cpu().numpy(),
                                                                           g["s_hi"])


@pytest.mark.gpu
def test_gpu_moe_fixture(kq4, orc):
    g = load("moe.npz")
    d, ne, tk, ef = (int(v) for v in g["shape"])
    sel, pr = orc.moe_route(orc.router_logits(g["router"], g["X"], ne, d), tk)
    Y = kq4.moe_ffn(g["X"], sel, pr, g["G"], g["U"], g["D"], ne, d, ef)
    r, a = rel_err(Y, g["Y"])
    assert r <= 1e-5, (r, a)
