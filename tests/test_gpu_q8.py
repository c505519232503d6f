"""GPU parity of the Q8_0 path (q8 stream layout, GEMV and GEMM) against the oracle, through
the C ABI. The oracle's Q8_0 chains are pinned in tests/test_oracle_q8.py.

Bars (as for q4): the prefill GEMM replays each output's chain in block order, so it is
bit-exact; the decode GEMV splits K over waves, so it is within max|got-ref| / max|ref| <= 1e-5
of the oracle (max-abs reported)."""
import ctypes

import numpy as np
import pytest

import synth
from conftest import rel_err
from test_stream_layout import q8_tiles_synth

pytestmark = pytest.mark.gpu

TOL = 1e-5


def to_dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


GEMV = [(8, 32, 8), (24, 160, 8), (104, 2080, 8), (20, 96, 4), (256, 4096, 8), (4096, 4096, 8),
        (1024, 12288, 8)]


@pytest.mark.parametrize("n", [1, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("rows,cols,g", GEMV)
def test_q8_gemv(kq4, torch_dev, orc, rows, cols, g, n):
    torch = torch_dev
    w = q8_tiles_synth(rows, cols, g, rows + cols + n)
    x = synth.make_activations(n, cols, n + cols)
    res = synth.make_activations(n, rows, n + rows)
    want = orc.q8_matmul(w, x, rows, cols, residual=res, g=g)
    W = kq4.q8_prepare_dev(w, rows, cols, g=g)
    out = torch.empty((n, rows), dtype=torch.float32, device="cuda")
    kq4.q8_matmul_dev(out, to_dev(torch, x), W, rows, cols, residual=to_dev(torch, res))
    torch.cuda.synchronize()
    rel, mx = rel_err(out.cpu().numpy(), want)
    assert rel <= TOL, (rel, mx)


@pytest.mark.parametrize("chain", [0, 2, 4])
@pytest.mark.parametrize("n", [9, 33, 64])
@pytest.mark.parametrize("rows,cols,g", [(24, 160, 8), (256, 2048, 8), (100, 512, 4)])
def test_q8_gemm_bit_exact(kq4, torch_dev, orc, rows, cols, g, n, chain):
    torch = torch_dev
    w = q8_tiles_synth(rows, cols, g, rows * n + cols)
    x = synth.make_activations(n, cols, 3 * n + cols)
    res = synth.make_activations(n, rows, n + 7)
    want = orc.q8_matmul(w, x, rows, cols, residual=res, chain=chain, g=g)
    W = kq4.q8_prepare_dev(w, rows, cols, g=g)
    out = torch.empty((n, rows), dtype=torch.float32, device="cuda")
    with kq4.options(gemm_split=1):   # K unsplit: the single chain, bit for bit
        kq4.q8_matmul_dev(out, to_dev(torch, x), W, rows, cols, residual=to_dev(torch, res),
                          chain=chain)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))


# 128x128 tiles (2048 tokens x 4096 rows: 512 tiles) and 64x128 (2048 rows); short K keeps the
# oracle quick; tiles 2 and 4 force the 64x128 and 128x64 forms (planner option gemm_tile)
@pytest.mark.parametrize("tile", [0, 2, 4])
@pytest.mark.parametrize("n,rows,chain", [(2048, 4096, 0), (2048, 4096, 4), (2048, 2048, 2)])
def test_q8_gemm_large_tiles_bit_exact(kq4, torch_dev, orc, n, rows, chain, tile):
    torch = torch_dev
    cols = 256
    w = q8_tiles_synth(rows, cols, 8, rows + chain)
    x = synth.make_activations(n, cols, 5 + chain)
    want = orc.q8_matmul(w, x, rows, cols, chain=chain, g=8)
    W = kq4.q8_prepare_dev(w, rows, cols, g=8)
    out = torch.empty((n, rows), dtype=torch.float32, device="cuda")
    with kq4.options(gemm_tile=tile):
        kq4.q8_matmul_dev(out, to_dev(torch, x), W, rows, cols, chain=chain)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("n", [1, 6])
def test_q8_gemv_explicit_chains(kq4, torch_dev, orc, n):
    """GEMV32 (fused, f32 scale) and Q8GEMM (unfused, f16 scale) forced at decode sizes."""
    torch = torch_dev
    rows, cols = 64, 1024
    w = q8_tiles_synth(rows, cols, 8, 91)
    x = synth.make_activations(n, cols, 92)
    W = kq4.q8_prepare_dev(w, rows, cols)
    for chain in (kq4.CHAIN_GEMV32, kq4.CHAIN_Q8GEMM):
        want = orc.q8_matmul(w, x, rows, cols, chain=chain)
        out = torch.empty((n, rows), dtype=torch.float32, device="cuda")
        kq4.q8_matmul_dev(out, to_dev(torch, x), W, rows, cols, chain=chain)
        torch.cuda.synchronize()
        assert rel_err(out.cpu().numpy(), want)[0] <= TOL


def test_q8_multi_and_host_wrappers(kq4, orc):
    rows, cols, n = 256, 1024, 5
    wg = q8_tiles_synth(rows, cols, 8, 5)
    wu = q8_tiles_synth(rows, cols, 8, 6)
    x = synth.make_activations(n, cols, 7)
    g_o = orc.q8_matmul(wg, x, rows, cols)
    u_o = orc.q8_matmul(wu, x, rows, cols)
    g_out = np.empty((n, rows), np.float32)
    u_out = np.empty((n, rows), np.float32)
    P = ctypes.c_void_p
    rc = kq4.lib().kq4_dyn_matvec_q8_fused_gate_up_batched(
        P(g_out.ctypes.data), P(u_out.ctypes.data), P(wg.ctypes.data), P(wu.ctypes.data),
        P(x.ctypes.data), rows, cols, n)
    assert rc == 1, kq4.last_error()
    assert rel_err(g_out, g_o)[0] <= TOL and rel_err(u_out, u_o)[0] <= TOL
    # down with residual, single token and batched (cached under the host pointer)
    wd = q8_tiles_synth(128, 1024, 8, 8)
    res = synth.make_activations(n, 128, 9)
    want = orc.q8_matmul(wd, x, 128, 1024, residual=res)
    out = np.empty((n, 128), np.float32)
    rc = kq4.lib().kq4_dyn_matvec_q8_fused_down_residual_batched(
        P(out.ctypes.data), P(res.ctypes.data), P(wd.ctypes.data), P(x.ctypes.data), 128, 1024, n)
    assert rc == 1 and rel_err(out, want)[0] <= TOL
    got1 = kq4.q8_matmul(wd, x[:1], 128, 1024, residual=res[:1], wkey=0x77)
    assert rel_err(got1, orc.q8_matmul(wd, x[:1], 128, 1024, residual=res[:1]))[0] <= TOL


# Seeded random shapes: 4x4 or 8x8 tiles, rows a multiple of the tile, K a multiple of 32 up to
# 3072 (partial 8-block stages), 1-8 tokens (GEMV, within 1e-5) or 9-300 (GEMM, bit-exact below
# K = 2048, where the planner never splits K), chains AUTO / VDOT / GEMM, with a residual.
@pytest.mark.parametrize("i", range(16))
def test_q8_random_shapes(kq4, torch_dev, orc, i):
    torch = torch_dev
    rng = np.random.default_rng(9000 + i)
    g = 4 if i % 2 else 8
    rows = g * int(rng.integers(1, 1024 // g + 1))
    cols = 32 * int(rng.integers(1, 97))
    n = int(rng.integers(1, 9)) if i % 4 < 2 else int(rng.integers(9, 301))
    chain = (0, 2, 4)[int(rng.integers(0, 3))]
    w = q8_tiles_synth(rows, cols, g, 9100 + i)
    x = synth.make_activations(n, cols, 9200 + i)
    res = synth.make_activations(n, rows, 9300 + i)
    want = orc.q8_matmul(w, x, rows, cols, residual=res, chain=chain, g=g)
    W = kq4.q8_prepare_dev(w, rows, cols, g=g)
    out = torch.empty((n, rows), dtype=torch.float32, device="cuda")
    kq4.q8_matmul_dev(out, to_dev(torch, x), W, rows, cols, residual=to_dev(torch, res),
                      chain=chain)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    rel, mx = rel_err(got, want)
    print(f"q8 random {i}: g={g} rows={rows} cols={cols} n={n} chain={chain}: rel={rel:.3e}")
    if n > 8 and cols < 2048:   # on the GEMM, K unsplit
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert rel <= TOL, (rel, mx)
