"""Pins the oracle's integer block sums and fp32 chains (vllm_safetensors.c:4133-4251,
4593-4631; llama_gemm_q4_0_4x4_asm.c:151-161).

The reference's NEON chains cannot run here, so the chains are pinned by what the mathematics
fixes: brute-force integer sums, exact-arithmetic cases (power-of-two scales: every fp32 step is
exact, so any correct chain equals the exact sum), constructed cases where the lo/hi split and
the f16-rounded activation scale change the fp32 result, and the float64 error budget.
"""
from fractions import Fraction

import numpy as np
import pytest

import synth
from conftest import rn32


def rand_case(rows, cols, n, seed, **kw):
    w = synth.make_q4_weights(rows, cols, seed, **kw)
    x = synth.make_activations(n, cols, seed + 100)
    return w, x


def test_block_sums_brute_force(orc):
    rows, cols, n = 12, 128, 3
    w, x = rand_case(rows, cols, n, 1)
    xq, xd = orc.quantize(x, cols)
    lo, hi = orc.block_sums(w, xq, rows, cols)
    wi = synth.tile_weights_int(w, rows, cols).astype(np.int64).reshape(rows, cols // 32, 32)
    q = xq.astype(np.int64).reshape(n, cols // 32, 32)
    want_lo = np.einsum("rbe,tbe->trb", wi[:, :, :16], q[:, :, :16])
    want_hi = np.einsum("rbe,tbe->trb", wi[:, :, 16:], q[:, :, 16:])
    assert np.array_equal(lo, want_lo) and np.array_equal(hi, want_hi)


def test_block_sum_bound(orc):
    """|S| <= 32*8*127 = 32512: extreme codes (-8 everywhere, q = -127 where x = -amax... and
    +127 elsewhere) reach the bound's order and stay exact in int32 / fp32."""
    rows, cols = 4, 32
    w = np.zeros((1, 1, 72), np.uint8)
    w[0, 0, :8] = np.frombuffer(np.float16([1, 1, 1, 1]).tobytes(), np.uint8)
    w[0, 0, 8:] = 0x00 ^ 0x88            # stored n^8 = 8 -> n = 0 -> weight -8
    x = np.full((1, 32), 1.0, np.float32)
    xq, _ = orc.quantize(x, cols)
    lo, hi = orc.block_sums(w, xq, rows, cols)
    assert (lo == -8 * 127 * 16).all() and (hi == -8 * 127 * 16).all()


def exact_case(n, cols, rows, seed):
    """Power-of-two scales and activations that quantize to exact multiples: every fp32
    product and partial sum below is exact."""
    rng = np.random.default_rng(seed)
    w = synth.make_q4_weights(rows, cols, seed)
    g, nb = rows // 4, cols // 32
    sc = (2.0 ** rng.integers(-6, 2, size=(g, nb, 4))).astype(np.float16)
    w[:, :, :8] = sc.view(np.uint8).reshape(g, nb, 8)
    q = rng.integers(-127, 128, size=(n, cols)).astype(np.float32)
    q[:, ::32] = 127.0                                   # amax = 127 * 2^k -> d = 2^k
    k = rng.integers(-4, 3, size=(n, nb)).astype(np.float32)
    x = (q.reshape(n, nb, 32) * (2.0 ** k)[:, :, None]).reshape(n, cols).astype(np.float32)
    return w, x


@pytest.mark.parametrize("chain", [1, 2, 3])
def test_chains_exact_arithmetic(orc, chain):
    rows, cols, n = 8, 256, 2
    w, x = exact_case(n, cols, rows, 3)
    xq, xd = orc.quantize(x, cols)
    got = orc.matmul(w, x, rows, cols, chain=chain)
    want = orc.matmul_f64(w, xq, xd, rows, cols)
    assert np.array_equal(got.astype(np.float64), want)
    res = np.random.default_rng(1).standard_normal((n, rows)).astype(np.float32)
    got_r = orc.matmul(w, x, rows, cols, residual=res, chain=chain)
    assert np.array_equal(got_r, (res + got).astype(np.float32))


def test_ctile_lo_hi_split_is_observable(orc):
    """Row 0 holds weight +1 at element 0 of blocks 0 and 1 and -1 at element 16 of block 1;
    q = 127 at those elements; s = 1 for block 0 and s = 2048 * 8192 = 2^24 for block 1.
    V2 (one accumulator): 127 + 0 * 2^24 = 127.
    V1: lo = fl(127 + 127 * 2^24) = 127 * 2^24 + 128 (spacing 128 there), hi = -127 * 2^24,
    out = 128. A chain that ignored the lo/hi split would give 127."""
    rows, cols = 4, 64
    w = np.zeros((1, 2, 72), np.uint8)                    # stored nibble 0 = n 8 = weight 0
    w[0, 0, :8] = np.frombuffer(np.float16([1, 1, 1, 1]).tobytes(), np.uint8)
    w[0, 1, :8] = np.frombuffer(np.float16([2048] * 4).tobytes(), np.uint8)
    w[0, 0, 8] = 0x01                                     # element 0: stored 1 -> n 9 -> +1
    w[0, 1, 8] = 0xF1                                     # + element 16: stored 15 -> n 7 -> -1
    x = np.zeros((1, cols), np.float32)
    x[0, 0] = 127.0                                       # block 0: d = 1
    x[0, 32] = 127.0 * 8192                               # block 1: d = 8192
    x[0, 48] = 127.0 * 8192
    xq, xd = orc.quantize(x, cols)
    assert xd[0, 0] == 1.0 and xd[0, 1] == 8192.0
    lo, hi = orc.block_sums(w, xq, rows, cols)
    assert list(lo[0, 0]) == [127, 127] and list(hi[0, 0]) == [0, -127]
    assert orc.matmul(w, x, rows, cols, chain=2)[0, 0] == 127.0
    assert orc.matmul(w, x, rows, cols, chain=1)[0, 0] == 128.0


def test_asm_chain_rounds_activation_scale_to_f16(orc):
    """With xd not representable in f16 the ASM chain equals the float64 sum computed with
    f16(xd), and differs from the one with the f32 xd."""
    rows, cols, n = 16, 512, 4
    w, x = rand_case(rows, cols, n, 8)
    xq, xd = orc.quantize(x, cols)
    got = orc.matmul(w, x, rows, cols, chain=3).astype(np.float64)
    xdh = xd.astype(np.float16).astype(np.float32)
    want_h = orc.matmul_f64(w, xq, xdh, rows, cols)
    want_f = orc.matmul_f64(w, xq, xd, rows, cols)
    m = np.abs(want_h).max()
    assert np.abs(got - want_h).max() / m < 2e-6
    assert np.abs(got - want_f).max() / m > 2e-5


def test_auto_dispatch(orc):
    """n_batch <= 3: CTILE for all; n_batch > 3: ASM on n & ~3 tokens, CTILE on the tail."""
    rows, cols = 8, 256
    for n in (1, 3, 4, 6, 11):
        w, x = rand_case(rows, cols, n, 20 + n)
        auto = orc.matmul(w, x, rows, cols, chain=0)
        for t in range(n):
            c = 3 if (n > 3 and t < (n & ~3)) else 1
            single = orc.matmul(w, x, rows, cols, chain=c)[t]
            assert np.array_equal(auto[t], single), (n, t)


def test_error_budget_vs_float64(orc):
    rows, cols, n = 32, 4096, 2
    w, x = rand_case(rows, cols, n, 30, sigma=0.015, floor=0.0)
    xq, xd = orc.quantize(x, cols)
    want = orc.matmul_f64(w, xq, xd, rows, cols)
    for chain in (1, 2):
        got = orc.matmul(w, x, rows, cols, chain=chain)
        assert np.abs(got - want).max() / np.abs(want).max() < 1e-6


def test_sample_matches_full(orc):
    rows, cols, n = 16, 256, 6
    w, x = rand_case(rows, cols, n, 40)
    xq, xd = orc.quantize(x, cols)
    full = orc.matmul_q(w, xq, xd, rows, cols)
    tok = np.array([0, 3, 4, 5, 5], np.int32)
    row = np.array([0, 15, 7, 1, 14], np.int32)
    s = orc.matmul_q_sample(w, xq, xd, rows, cols, n, tok, row)
    assert np.array_equal(s, full[tok, row])


def q4_chain_emul(s_lo, s_hi, wd, xd, chain, fused=True):
    """One output (token, row) of the reference's q4 chain in exact rationals, one binary32
    rounding per NEON instruction:
      V1 C-tile (q4x4_dot1_group16, vllm_safetensors.c:4190-4216, collapse :4250):
         dsv = fmul(wd, xd); lo = fmla(lo, scvtf(16*S_lo, #4), dsv); hi likewise; lo + hi
      V2 M4f (q4x4_dot1_group16_gemv, :4233-4251): one fmla chain over S_lo + S_hi
      V3 asm (llama_gemm_q4_0_4x4_asm.c:151-161): fcvtl of the f16 activation scale,
         fmul by the weight scale, scvtf #4, fmla
    scvtf(16*S, #4) = S exactly. fused=False is a planted mistake: fmla as fmul then fadd."""
    R = lambda v: Fraction(float(v))  # noqa: E731

    def fmla(acc, s, d):
        if fused:
            return rn32(R(s) * R(d) + R(acc))
        return rn32(R(rn32(R(s) * R(d))) + R(acc))

    if chain == 1:
        lo = hi = np.float32(0)
        for sl, sh, w, x in zip(s_lo, s_hi, wd, xd):
            dsv = rn32(R(w) * R(x))
            lo = fmla(lo, int(sl), dsv)
            hi = fmla(hi, int(sh), dsv)
        return rn32(R(lo) + R(hi))
    acc = np.float32(0)
    for sl, sh, w, x in zip(s_lo, s_hi, wd, xd):
        xs = np.float32(np.float16(x)) if chain == 3 else x
        acc = fmla(acc, int(sl) + int(sh), rn32(R(w) * R(xs)))
    return acc


@pytest.mark.parametrize("chain", [1, 2, 3])
def test_chains_against_instruction_emulation(orc, chain):
    """Every output of each q4 chain equals the exact-rational emulation of its instruction
    sequence, and a planted unfused multiply-add (fmul + fadd: two roundings) disagrees with the
    oracle on some output, so the oracle's fmaf is what the reference's fmla computes. Scales
    near 1 with many blocks make the products inexact."""
    rows, cols, n = 8, 1024, 2
    w, x = rand_case(rows, cols, n, 50 + chain, sigma=0.5, floor=0.25)
    xq, xd = orc.quantize(x, cols)
    lo, hi = orc.block_sums(w, xq, rows, cols)
    wd = synth.tile_scales(w, rows, cols)
    res = np.random.default_rng(chain).standard_normal((n, rows)).astype(np.float32)
    got = orc.matmul_q(w, xq, xd, rows, cols, chain=chain)
    got_r = orc.matmul_q(w, xq, xd, rows, cols, residual=res, chain=chain)
    unfused_differs = 0
    for t in range(n):
        for r in range(rows):
            e = q4_chain_emul(lo[t, r], hi[t, r], wd[r], xd[t], chain)
            assert got[t, r] == e, (t, r, got[t, r], e)
            assert got_r[t, r] == rn32(Fraction(float(res[t, r])) + Fraction(float(e)))
            u = q4_chain_emul(lo[t, r], hi[t, r], wd[r], xd[t], chain, fused=False)
            unfused_differs += int(u != got[t, r])
    assert unfused_differs > 0


def test_chain_emulation_separates_the_chains(orc):
    """The three emulated chains give three different results on one case, so a chain swapped
    for another (e.g. V2's single accumulator where V1 keeps lo and hi apart) fails the test
    above."""
    rows, cols, n = 8, 1024, 1
    w, x = rand_case(rows, cols, n, 60, sigma=0.5, floor=0.25)
    xq, xd = orc.quantize(x, cols)
    outs = [orc.matmul_q(w, xq, xd, rows, cols, chain=c) for c in (1, 2, 3)]
    assert not np.array_equal(outs[0], outs[1])
    assert not np.array_equal(outs[1], outs[2])
    assert not np.array_equal(outs[0], outs[2])
