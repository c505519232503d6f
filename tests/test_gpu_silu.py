"""GPU parity of the dense FFN's SiLU-multiply (kq4_silu_mul_dev) and of the fused
SiLU-multiply + down projection (kq4_matmul_silu_dev / kq4_matmul_silu / the kq4_ops wrappers)
against the oracle, through the C ABI.

Bars: silu_mul bit-exact for every element the reference's NEON loop covers (i < n & ~3); the
scalar tail (last n % 4) within 4e-7 relative (libm expf vs a correctly rounded exp). The fused
op forms the same product inside the GEMV / quantizer, so its output is bit-identical to the
unfused device op fed with the oracle's product (the int8 codes are the same), and within the
matmul bar (max|got-ref| / max|ref| <= 1e-5) of the oracle."""
import ctypes

import numpy as np
import pytest

import synth
from conftest import rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-5
F32 = np.float32


def to_dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def silu_inputs(n, seed):
    rng = np.random.default_rng(seed)
    g = np.concatenate([np.linspace(-100, 100, n // 4), rng.standard_normal(n - n // 4 - 16) * 5,
                        [0.0, -0.0, 20.0, -20.0, 87.0, -87.0, 88.0, -88.0, 1e-30, -1e-30, 1e30,
                         -1e30, 1e-42, -1e-42, 3.5, -3.5]]).astype(F32)
    u = (rng.standard_normal(n) * 2).astype(F32)
    u[:8] = [1.0, -1.0, 0.0, 1e-30, 1e30, -2.0, 0.5, 1e-42]
    return g, u


def test_silu_mul_bit_exact(kq4, torch_dev, orc):
    torch = torch_dev
    n = 1 << 20
    g, u = silu_inputs(n, 1)
    want = orc.silu_mul(g, u)
    G = to_dev(torch, g)
    kq4.silu_mul_dev(G, to_dev(torch, u))
    torch.cuda.synchronize()
    got = G.cpu().numpy()
    bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
    assert bad.size == 0, (bad[:5], g[bad[:5]], u[bad[:5]], got[bad[:5]], want[bad[:5]])


def test_silu_mul_every_reciprocal_bucket(kq4, torch_dev, orc):
    """Denominators 1 + e^-g over every 8-bit FRECPE bucket of every exponent the SiLU reaches:
    g = -ln(den - 1) for den spread over [1, 2^126)."""
    torch = torch_dev
    e = np.arange(0, 126)
    f = np.arange(256)
    den = np.ldexp(1.0 + (f[None, :] + 0.5) / 256.0, e[:, None]).ravel()
    g = (-np.log(np.maximum(den - 1.0, 1e-300))).astype(F32)
    g = np.concatenate([g, np.nextafter(g, F32(np.inf)), np.nextafter(g, F32(-np.inf))])
    g = g[np.isfinite(g)]
    g = g[: (g.size // 4) * 4]
    u = np.ones_like(g)
    want = orc.silu_mul(g, u)
    G = to_dev(torch, g)
    kq4.silu_mul_dev(G, to_dev(torch, u))
    torch.cuda.synchronize()
    assert np.array_equal(G.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("n", [1, 2, 3, 7, 1027])
def test_silu_mul_scalar_tail(kq4, torch_dev, orc, n):
    torch = torch_dev
    rng = np.random.default_rng(n)
    g = (rng.standard_normal(n) * 10).astype(F32)
    u = rng.standard_normal(n).astype(F32)
    want = orc.silu_mul(g, u)
    G = to_dev(torch, g)
    kq4.silu_mul_dev(G, to_dev(torch, u))
    torch.cuda.synchronize()
    got = G.cpu().numpy()
    nv = n & ~3
    assert np.array_equal(got[:nv].view(np.uint32), want[:nv].view(np.uint32))
    d = np.abs(got[nv:].astype(np.float64) - want[nv:])
    assert np.all(d <= 4e-7 * np.abs(want[nv:]) + 1e-38)


SHAPES = [(20, 160), (100, 2080), (2048, 6144), (4096, 12288)]


# every token count on the smaller shapes; n = 1, 4, 16 on the full-size 8B down projection
SILU_CASES = [(r, c, n) for r, c in SHAPES for n in (1, 2, 3, 4, 5, 8, 16, 33)
              if r * c <= 2048 * 6144 or n in (1, 4, 16)]


@pytest.mark.parametrize("rows,cols,n", SILU_CASES)
def test_matmul_silu_dev(kq4, torch_dev, orc, rows, cols, n):
    torch = torch_dev
    w = synth.make_q4_weights(rows, cols, rows + n)
    rng = np.random.default_rng(cols + n)
    g = (rng.standard_normal((n, cols)) * 3).astype(F32)
    u = rng.standard_normal((n, cols)).astype(F32)
    res = rng.standard_normal((n, rows)).astype(F32)
    av = orc.silu_mul(g, u).reshape(n, cols)
    want = orc.matmul(w, av, rows, cols, residual=res)

    W = kq4.prepare_dev(to_dev(torch, w), rows, cols)
    R = to_dev(torch, res)
    out = torch.empty((n, rows), dtype=torch.float32, device="cuda")
    kq4.matmul_silu_dev(out, to_dev(torch, g), to_dev(torch, u), W, rows, cols, residual=R)
    ref_dev = torch.empty_like(out)
    kq4.matmul_dev(ref_dev, to_dev(torch, av), W, rows, cols, residual=R)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref_dev.cpu().numpy().view(np.uint32))
    rel, mx = rel_err(got, want)
    assert rel <= TOL, (rel, mx)


def test_matmul_silu_host_and_ops(kq4, orc):
    rows, cols = 256, 2048
    w = synth.make_q4_weights(rows, cols, 77)
    rng = np.random.default_rng(77)
    for n in (1, 3, 6):
        g = (rng.standard_normal((n, cols)) * 3).astype(F32)
        u = rng.standard_normal((n, cols)).astype(F32)
        res = rng.standard_normal((n, rows)).astype(F32)
        want = orc.matmul_silu(w, g, u, rows, cols, residual=res)
        got = kq4.matmul_silu(w, g, u, rows, cols, residual=res, wkey=0x5000 + n)
        assert rel_err(got, want)[0] <= TOL

        out = np.empty((n, rows), F32)
        P = ctypes.c_void_p
        if n == 1:
            rc = kq4.lib().kq4_silu_mul_down_residual(
                P(out.ctypes.data), P(res.ctypes.data), P(w.ctypes.data), P(g.ctypes.data),
                P(u.ctypes.data), rows, cols)
        else:
            rc = kq4.lib().kq4_silu_mul_down_residual_batched(
                P(out.ctypes.data), P(res.ctypes.data), P(w.ctypes.data), P(g.ctypes.data),
                P(u.ctypes.data), rows, cols, n)
        assert rc == 1, kq4.last_error()
        assert rel_err(out, want)[0] <= TOL


def test_matmul_silu_rejects_bad_arguments(kq4, torch_dev):
    torch = torch_dev
    g = torch.zeros((1, 64), dtype=torch.float32, device="cuda")
    W = kq4.prepare_dev(np.zeros(72 * 2, np.uint8), 4, 64)
    out = torch.empty((1, 4), dtype=torch.float32, device="cuda")
    rc = kq4.lib().kq4_matmul_silu_dev(out.data_ptr(), g.data_ptr(), None, None, W.data_ptr(), 4,
                                       64, 1, 0, None)
    assert rc != 0
    rc = kq4.lib().kq4_matmul_silu_dev(out.data_ptr(), g.data_ptr(), g.data_ptr() + 4, None,
                                       W.data_ptr(), 4, 64, 1, 0, None)
    assert rc != 0                                        # up not 16-byte aligned
