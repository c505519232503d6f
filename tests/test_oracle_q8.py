"""Pins the oracle's Q8_0 path (kqo_f32_to_q8_0, kqo_repack_q8_0_tiled, kqo_q8_matmul*):
  * encoder and both tile repacks byte for byte against the reference's own converter code
    (f32_to_q8_0, repack_q8_0_8x8_inplace, repack_q8_0_4x4_inplace, built in oracle/_ref);
  * the matmul's integer block sums against a numpy decode of the tiles (an independent reading
    of the 8x8 / 4x4 layouts) and numpy's integer dot;
  * the two fp32 chains by an exact rational emulation of each NEON instruction sequence
    (VDOT: one fused multiply-add per block; GEMM: unfused, f16-rounded activation scale), by
    exact cases (power-of-two scales: both chains equal the float64 sum), and by the AUTO
    dispatch (1 token -> VDOT, >= 2 -> GEMM for every token).
The reference computes these chains only in AArch64 NEON code, so no reference run pins them."""
from fractions import Fraction

import numpy as np
import pytest

from conftest import rn32

F32 = np.float32


def weights(rows, cols, seed, scale=0.05):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((rows, cols)) * scale).astype(F32)
    w[0, :32] = 0                                   # an all-zero block: scale floor 1e-10
    w[1, 3] = 2.5                                    # a block with one large element
    w[2, 32:64] = np.linspace(-1, 1, 32)            # exact halves after scaling
    return w


def test_encoder_matches_reference(orc, ref):
    for seed in range(4):
        w = weights(8, 256, seed, scale=10.0 ** (seed - 2))
        a = np.empty(8 * 256 // 32 * 34, np.uint8)
        ref.kref_f32_to_q8_0(a.ctypes.data, w.ctypes.data, w.size)
        b = np.empty_like(a)
        orc.lib().kqo_f32_to_q8_0(b.ctypes.data, w.ctypes.data, w.size)
        assert np.array_equal(a, b), seed


@pytest.mark.parametrize("g", [8, 4])
def test_repack_matches_reference(orc, ref, g):
    rows, cols = 24, 160
    w = weights(rows, cols, 7)
    legacy = np.empty(rows * cols // 32 * 34, np.uint8)
    ref.kref_f32_to_q8_0(legacy.ctypes.data, w.ctypes.data, w.size)
    (ref.kref_repack_q8_0_8x8 if g == 8 else ref.kref_repack_q8_0_4x4)(legacy.ctypes.data,
                                                                       rows, cols)
    assert np.array_equal(legacy, orc.q8_tiles(w, rows, cols, g))


def decode(tiles, rows, cols, g):
    """numpy decode of tiled Q8_0: codes [rows][cols] int8, scales [rows][nb] f32."""
    nb = cols // 32
    t = tiles.reshape(rows // g, nb, 34 * g)
    sc = t[:, :, :2 * g].copy().view(np.float16).astype(F32)             # [G][nb][g]
    q = t[:, :, 2 * g:].view(np.int8).reshape(rows // g, nb, 8, g, 4)      # k, m, i
    codes = q.transpose(0, 3, 1, 2, 4).reshape(rows, cols)
    return codes, sc.transpose(0, 2, 1).reshape(rows, nb)


def chain_emul(S, wd, xs, gemm):
    """One output's chain in exact rationals, one binary32 rounding per NEON instruction."""
    acc = F32(0)
    for s, w, x in zip(S, wd, xs):
        if gemm:
            xh = F32(np.float16(x))
            sc = rn32(Fraction(float(w)) * Fraction(float(xh)))
            acc = rn32(Fraction(float(acc)) + Fraction(float(rn32(Fraction(float(sc)) * int(s)))))
        else:
            sc = rn32(Fraction(float(w)) * Fraction(float(x)))
            acc = rn32(Fraction(int(s)) * Fraction(float(sc)) + Fraction(float(acc)))
    return acc


@pytest.mark.parametrize("g", [8, 4])
def test_chains_against_emulation(orc, g):
    rows, cols, n = 8, 192, 3
    tiles = orc.q8_tiles(weights(rows, cols, 11), rows, cols, g)
    x = np.random.default_rng(12).standard_normal((n, cols)).astype(F32)
    xq, xd = orc.quantize(x, cols)
    codes, wsc = decode(tiles, rows, cols, g)
    S = np.einsum("rbe,tbe->trb", codes.reshape(rows, -1, 32).astype(np.int64),
                  xq.reshape(n, -1, 32).astype(np.int64))
    vdot = orc.q8_matmul_q(tiles, xq, xd, rows, cols, chain=orc.CHAIN_GEMV32, g=g)
    gemm = orc.q8_matmul_q(tiles, xq, xd, rows, cols, chain=orc.CHAIN_Q8GEMM, g=g)
    for t in range(n):
        for r in range(rows):
            assert vdot[t, r] == chain_emul(S[t, r], wsc[r], xd[t], False), (t, r)
            assert gemm[t, r] == chain_emul(S[t, r], wsc[r], xd[t], True), (t, r)
    assert not np.array_equal(vdot, gemm)                        # the chains do differ here
    auto1 = orc.q8_matmul_q(tiles, xq[:1], xd[:1], rows, cols, g=g)
    auto3 = orc.q8_matmul_q(tiles, xq, xd, rows, cols, g=g)
    assert np.array_equal(auto1, vdot[:1]) and np.array_equal(auto3, gemm)


def test_exact_case_equals_float64(orc):
    """Power-of-two weight and activation scales with small integer codes: every product and
    partial sum is exact, so both chains equal the float64 sum (a dropped block, a wrong code
    or a transposed layout fails)."""
    rows, cols = 16, 256
    rng = np.random.default_rng(5)
    codes = rng.integers(-20, 21, (rows, cols))
    wsc = 2.0 ** rng.integers(-8, -2, (rows, cols // 32))
    # build the tiles directly from codes and scales (legacy blocks, then the oracle repack)
    legacy = np.zeros((rows, cols // 32, 34), np.uint8)
    legacy[:, :, :2] = wsc.astype(np.float16).view(np.uint8).reshape(rows, -1, 2)
    legacy[:, :, 2:] = codes.reshape(rows, -1, 32).astype(np.int8).view(np.uint8)
    tiles = np.empty(legacy.size, np.uint8)
    orc.lib().kqo_repack_q8_0_tiled(legacy.ctypes.data, tiles.ctypes.data, 8, rows, cols)
    xq = rng.integers(-30, 31, (2, cols)).astype(np.int8)
    xd = (2.0 ** rng.integers(-6, -1, (2, cols // 32))).astype(F32)
    want = np.einsum("rbe,tbe,rb,tb->tr", codes.reshape(rows, -1, 32).astype(np.float64),
                     xq.reshape(2, -1, 32).astype(np.float64), wsc, xd.astype(np.float64))
    for chain in (orc.CHAIN_GEMV32, orc.CHAIN_Q8GEMM):
        got = orc.q8_matmul_q(tiles, xq, xd, rows, cols, chain=chain)
        assert np.array_equal(got.astype(np.float64), want), chain


def test_gemm_rounds_activation_scale_to_f16(orc):
    """xd = 1 + 2^-12 is not an f16 value (f16 keeps 10 fraction bits): the GEMM chain multiplies
    by 1.0, the VDOT chain by the f32 value."""
    rows, cols = 8, 32
    legacy = np.zeros((rows, 1, 34), np.uint8)
    legacy[:, :, :2] = np.array([1.0], np.float16).view(np.uint8)
    legacy[:, :, 2] = 1                                          # code 1 at element 0
    tiles = np.empty(legacy.size, np.uint8)
    orc.lib().kqo_repack_q8_0_tiled(legacy.ctypes.data, tiles.ctypes.data, 8, rows, cols)
    xq = np.zeros((1, cols), np.int8)
    xq[0, 0] = 100
    xd = np.array([[1.0 + 2.0 ** -12]], F32)
    assert orc.q8_matmul_q(tiles, xq, xd, rows, cols, chain=orc.CHAIN_Q8GEMM)[0, 0] == 100.0
    assert orc.q8_matmul_q(tiles, xq, xd, rows, cols, chain=orc.CHAIN_GEMV32)[0, 0] == \
        F32(100.0 * (1.0 + 2.0 ** -12))
