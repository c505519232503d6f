"""GPU side of the VQF loader: a layer's q4 matrix goes from the mmap'd file
(tests/golden/synth_dual.vqf, written by the reference's own converter) to HBM in the stream layout
(kq4_vqf_prepare_dev: byte-equal to the layout's definition) and into the host-pointer API's
weight cache under the reference's key layer << 32 | proj (kq4_vqf_upload); the matmul over either
agrees with the oracle on the file's tiles (GEMV bar, max|got-ref| / max|ref| <= 1e-5)."""
import os
import sys

import numpy as np
import pytest

import synth
from conftest import rel_err

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
SYNTH = os.path.join(HERE, "golden", "synth_dual.vqf")
sys.path.insert(0, HERE)
from test_stream_layout import stream_layout  # noqa: E402


@pytest.mark.parametrize("proj,layer", [(0, 0), (1, 1), (3, 1), (4, 0), (6, 1), (7, 0)])
def test_prepare_and_matmul_from_vqf(kq4, torch_dev, orc, proj, layer):
    torch = torch_dev
    with kq4.Vqf(SYNTH) as v:
        tiles, rows, cols = v.q4_matrix(proj, layer)
        tiles = tiles.copy()
        W, r2, c2 = v.prepare_dev(proj, layer)
    assert (r2, c2) == (rows, cols)
    torch.cuda.synchronize()
    assert np.array_equal(W.cpu().numpy(), stream_layout(tiles, rows, cols))
    for n in (1, 4):
        x = synth.make_activations(n, cols, proj * 10 + layer + n)
        want = orc.matmul(tiles, x, rows, cols)
        out = torch.empty((n, rows), dtype=torch.float32, device="cuda")
        kq4.matmul_dev(out, torch.from_numpy(x).cuda(), W, rows, cols)
        torch.cuda.synchronize()
        assert rel_err(out.cpu().numpy(), want)[0] <= 1e-5


def test_upload_under_reference_key(kq4, orc):
    with kq4.Vqf(SYNTH) as v:
        key = v.upload(kq4.PROJ_DOWN, 1)
        tiles, rows, cols = v.q4_matrix(kq4.PROJ_DOWN, 1)
        tiles = tiles.copy()
    assert key == (1 << 32) | kq4.PROJ_DOWN
    x = synth.make_activations(2, cols, 5)
    got = kq4.matmul(tiles, x, rows, cols, wkey=key)       # served from the cache entry
    assert rel_err(got, orc.matmul(tiles, x, rows, cols))[0] <= 1e-5


@pytest.mark.parametrize("proj,layer", [(0, 1), (4, 0), (6, 1)])
def test_q8_prepare_and_gemm_from_vqf(kq4, torch_dev, orc, proj, layer):
    """The dual file's Q8_0 prefill weights to HBM and through the q8 GEMM (bit-exact chain)."""
    from test_stream_layout import q8_stream_layout
    torch = torch_dev
    with kq4.Vqf(SYNTH) as v:
        tiles, rows, cols, g = v.q8_matrix(proj, layer)
        tiles = tiles.copy()
        W, _, _ = v.prepare_q8_dev(proj, layer)
    torch.cuda.synchronize()
    assert np.array_equal(W.cpu().numpy(), q8_stream_layout(tiles, g, rows, cols))
    x = synth.make_activations(24, cols, proj + 3 * layer)   # a GEMM batch (over 16 tokens)
    want = orc.q8_matmul(tiles, x, rows, cols, g=g)
    out = torch.empty((24, rows), dtype=torch.float32, device="cuda")
    kq4.q8_matmul_dev(out, torch.from_numpy(x).cuda(), W, rows, cols)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))
