"""GPU parity of the RMSNorm (kq4_rms_norm_dev) and of the fused RMSNorm + quantize + matmul
(kq4_rmsnorm_matmul_multi_dev) against the oracle, through the C ABI.

Bars: the RMSNorm output bit-exact in both summation orders; the fused op's normed output
bit-exact, its matmul outputs bit-identical to the unfused device matmul fed with the oracle's
normed input (so its int8 codes are the oracle's) and within the GEMV bar
(max|got-ref| / max|ref| <= 1e-5) of the oracle."""
import numpy as np
import pytest

import synth
from conftest import rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-5
F32 = np.float32


def to_dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def rows(n, d, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, d)).astype(F32)
    x[0] *= 1e3
    if n > 2:
        x[1] *= 1e-3
        x[2, : d // 2] = 0
    w = (1.0 + 0.1 * rng.standard_normal(d)).astype(F32)
    return x, w


# (300, 1032) and (513, 4096): the serial order's many-token path (one chain per lane, then the
# normalisation), with a ragged last wave of tokens
@pytest.mark.parametrize("order", [0, 1])
@pytest.mark.parametrize("n,d", [(1, 8), (3, 64), (1, 2048), (5, 4096), (64, 2048), (2, 8200),
                                 (1, 16384), (300, 1032), (513, 4096)])
def test_rms_norm_bit_exact(kq4, torch_dev, orc, n, d, order):
    torch = torch_dev
    x, w = rows(n, d, d + n)
    want = orc.rms_norm(x, w, d, 1e-6, chunked=(order == 0))
    out = torch.empty((n, d), dtype=torch.float32, device="cuda")
    kq4.rms_norm_dev(out, to_dev(torch, x), to_dev(torch, w), 1e-6, order=order)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))


CASES = [([20, 8, 8], 160), ([2048, 512, 512], 2048), ([6144, 6144], 2048),
         ([4096, 1024, 1024], 4096)]


@pytest.mark.parametrize("n", [1, 2, 4, 8, 16, 33, 300])
@pytest.mark.parametrize("mats,cols", CASES)
def test_rmsnorm_matmul_multi(kq4, torch_dev, orc, mats, cols, n):
    torch = torch_dev
    order = 0 if n <= 8 else 1                # decode norm / prefill batch norm
    x, nw = rows(n, cols, cols + n)
    ws = [synth.make_q4_weights(r, cols, 100 + i) for i, r in enumerate(mats)]
    normed = orc.rms_norm(x, nw, cols, 1e-6, chunked=(order == 0))
    want = [orc.matmul(w, normed, r, cols) for w, r in zip(ws, mats)]

    W = [kq4.prepare_dev(to_dev(torch, w), r, cols) for w, r in zip(ws, mats)]
    outs = [torch.empty((n, r), dtype=torch.float32, device="cuda") for r in mats]
    nd = torch.empty((n, cols), dtype=torch.float32, device="cuda")
    kq4.rmsnorm_matmul_multi_dev(outs, to_dev(torch, x), to_dev(torch, nw), 1e-6, W, mats, cols,
                                 order=order, normed=nd)
    refs = [torch.empty_like(o) for o in outs]
    kq4.matmul_multi_dev(refs, to_dev(torch, normed), W, mats, cols)
    torch.cuda.synchronize()
    assert np.array_equal(nd.cpu().numpy().view(np.uint32), normed.view(np.uint32))
    for o, r, wnt in zip(outs, refs, want):
        got = o.cpu().numpy()
        assert np.array_equal(got.view(np.uint32), r.cpu().numpy().view(np.uint32))
        rel, mx = rel_err(got, wnt)
        assert rel <= TOL, (rel, mx)


@pytest.mark.parametrize("n", [1, 2])   # one token keeps the fp32 norm in the workspace
def test_rmsnorm_matmul_without_normed_buffer(kq4, torch_dev, orc, n):
    torch = torch_dev
    mats, cols = [6144, 6144], 2048
    x, nw = rows(n, cols, 11 + n)
    ws = [synth.make_q4_weights(r, cols, 200 + i) for i, r in enumerate(mats)]
    normed = orc.rms_norm(x, nw, cols, 1e-6, chunked=True)
    W = [kq4.prepare_dev(to_dev(torch, w), r, cols) for w, r in zip(ws, mats)]
    outs = [torch.empty((n, r), dtype=torch.float32, device="cuda") for r in mats]
    kq4.rmsnorm_matmul_multi_dev(outs, to_dev(torch, x), to_dev(torch, nw), 1e-6, W, mats, cols)
    refs = [torch.empty_like(o) for o in outs]
    kq4.matmul_multi_dev(refs, to_dev(torch, normed), W, mats, cols)
    torch.cuda.synchronize()
    for o, r in zip(outs, refs):
        assert np.array_equal(o.cpu().numpy().view(np.uint32), r.cpu().numpy().view(np.uint32))


def test_rms_norm_rejects_bad_shapes(kq4, torch_dev):
    torch = torch_dev
    x = torch.zeros((1, 12), dtype=torch.float32, device="cuda")
    rc = kq4.lib().kq4_rms_norm_dev(x.data_ptr(), x.data_ptr(), x.data_ptr(), 1, 12, 1e-6, 0, None)
    assert rc != 0                                   # d % 8 != 0
    y = torch.zeros((1, 64), dtype=torch.float32, device="cuda")
    rc = kq4.lib().kq4_rms_norm_dev(y.data_ptr(), y.data_ptr(), y.data_ptr(), 1, 64, 1e-6, 7, None)
    assert rc != 0                                   # unknown order
