"""Pins the oracle's dense SiLU-multiply (kqo_exp_neon, kqo_frecpe, kqo_silu_mul_neon,
kqo_fast_silu, kqo_silu_mul_rows) - the AArch64 form of vllm_silu_mul_worker
(vllm_safetensors.c:10932-10958), which no machine here can run.

What pins each piece, beyond the restatement itself:
  * exp_neon4: exp(0) = 1 exactly; relative error against float64 exp below 2e-7 + 2e-9*|n| on
    [-87, 87] (a dropped, swapped or mis-scaled Taylor term is far outside it); the clamp;
    and an independent emulation of the instruction sequence in exact rational arithmetic with
    one binary32 rounding per NEON instruction (catches an unfused multiply-add, a wrong
    operand order or a wrong rounding of n).
  * FRECPE: the documented FRECPE(1.0) = 0.998046875, every estimate within 2^-8 of 1/x, monotone
    in x, exact exponent symmetry; after the two Newton steps the reciprocal is within 1 ulp of
    1/den.
  * silu_mul: against float64 g*sigmoid(g)*u, relative 1e-6.
  * fast_silu (the worker's scalar tail): bit for bit against the reference's own x86-64 build
    of the worker (oracle/_ref), whose non-NEON body is fast_silu(g) * u with the same libm.
"""
from fractions import Fraction

import numpy as np
import pytest

F32 = np.float32


def rn32(q):
    """The binary32 value nearest to the rational q, ties to even."""
    f = F32(float(q))
    cands = [f, np.nextafter(f, F32(np.inf)), np.nextafter(f, F32(-np.inf))]
    return min(cands, key=lambda c: (abs(Fraction(float(c)) - q),
                                     int(np.array(c, F32).view(np.uint32)) & 1))


def fma(a, b, c):
    return rn32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def mul(a, b):
    return rn32(Fraction(float(a)) * Fraction(float(b)))


def exp_neon_emul(x):
    """exp_neon4 (vllm_safetensors.c:4041-4068) instruction by instruction: vmaxq, vminq,
    vmulq, vrndnq (ties to even), vfmsq (fused), six vfmaq (fused), vcvtq_s32, shift, add."""
    x = F32(max(F32(x), F32(-87.0)))
    x = F32(min(x, F32(87.0)))
    n = F32(np.rint(mul(x, F32(1.4426950408889634))))
    r = fma(-n, F32(0.6931471805599453), x)
    p = F32(0.001388888888888889)
    for c in (0.008333333333333333, 0.041666666666666664, 0.16666666666666666, 0.5, 1.0, 1.0):
        p = fma(p, r, F32(c))
    bits = (int(np.array(p, F32).view(np.uint32)) + (int(n) << 23)) & 0xFFFFFFFF
    return np.array(bits, np.uint32).view(F32)[()]


def test_exp_neon_special_values(orc):
    L = orc.lib()
    assert L.kqo_exp_neon(0.0) == 1.0
    assert L.kqo_exp_neon(-0.0) == 1.0
    assert L.kqo_exp_neon(100.0) == L.kqo_exp_neon(87.0)
    assert L.kqo_exp_neon(-1e30) == L.kqo_exp_neon(-87.0)
    assert np.isfinite(L.kqo_exp_neon(87.0)) and L.kqo_exp_neon(-87.0) > 0


def test_exp_neon_error_bound(orc):
    L = orc.lib()
    xs = np.concatenate([np.linspace(-87, 87, 20001), np.linspace(-1, 1, 2001)]).astype(F32)
    got = np.array([L.kqo_exp_neon(float(x)) for x in xs], np.float64)
    want = np.exp(xs.astype(np.float64))
    # degree-6 Taylor remainder (|r| <= ln2/2: 1.2e-7) + a few roundings, plus n times the error
    # of ln2 in binary32 (1.9e-9) carried by r = x - n*ln2; dropping the 1/720 term alone would
    # cost 2.4e-6
    bound = 2e-7 + 2e-9 * np.abs(np.rint(xs.astype(np.float64) * 1.4426950408889634))
    assert np.all(np.abs(got - want) / want < bound)


def test_exp_neon_instruction_emulation(orc):
    L = orc.lib()
    rng = np.random.default_rng(5)
    xs = np.concatenate([rng.uniform(-90, 90, 1500), rng.standard_normal(500) * 3,
                         [0.34657359, -0.34657359, 0.5 * np.log(2), 10.0, -10.0, 86.99, -86.99,
                          1e-8, -1e-8]]).astype(F32)
    for x in xs:
        got = F32(L.kqo_exp_neon(float(x)))
        want = exp_neon_emul(x)
        assert got.view(np.uint32) == want.view(np.uint32), float(x)


def test_frecpe_documented_value_and_bound(orc):
    L = orc.lib()
    assert L.kqo_frecpe(1.0) == 0.998046875
    assert L.kqo_frecpe(2.0) == 0.998046875 / 2
    xs = (1.0 + np.arange(0, 2 ** 23, 61) / 2 ** 23).astype(F32)
    r = np.array([L.kqo_frecpe(float(x)) for x in xs], np.float64)
    assert np.abs(r * xs.astype(np.float64) - 1).max() < 2.0 ** -8
    assert np.all(np.diff(r) <= 0)                       # monotone non-increasing in x
    for k in (-120, -20, -1, 1, 30, 124):
        for x in (1.0, 1.3, 1.99):
            assert L.kqo_frecpe(float(np.ldexp(F32(x), k))) == \
                np.ldexp(F32(L.kqo_frecpe(x)), -k)
    assert np.isnan(L.kqo_frecpe(0.0)) and np.isnan(L.kqo_frecpe(-1.0))


def test_newton_reciprocal_within_one_ulp(orc):
    L = orc.lib()
    for den in np.geomspace(1.0, 6e37, 4000).astype(F32):
        rec = F32(L.kqo_frecpe(float(den)))
        for _ in range(2):
            rec = F32(rec * fma(-den, rec, F32(2.0)))
        want = F32(1.0 / np.float64(den))
        assert abs(int(rec.view(np.int32)) - int(want.view(np.int32))) <= 1, float(den)


def test_silu_mul_against_float64(orc):
    L = orc.lib()
    rng = np.random.default_rng(9)
    g = np.concatenate([np.linspace(-60, 60, 6001), rng.standard_normal(2000) * 4]).astype(F32)
    u = rng.uniform(0.5, 2.0, g.size).astype(F32)
    got = np.array([L.kqo_silu_mul_neon(float(a), float(b)) for a, b in zip(g, u)], np.float64)
    g64 = g.astype(np.float64)
    want = g64 / (1.0 + np.exp(-g64)) * u
    assert np.all(np.abs(got - want) <= 1e-6 * np.abs(want) + 1e-37)


def test_silu_rows_tail_rule(orc):
    """Elements below n & ~3 take the NEON form, the last n % 4 fast_silu (tasks of 16)."""
    L = orc.lib()
    rng = np.random.default_rng(3)
    for n in (1, 3, 4, 17, 35, 64):
        g = (rng.standard_normal(n) * 30).astype(F32)
        u = rng.standard_normal(n).astype(F32)
        got = orc.silu_mul(g, u)
        nv = n & ~3
        for i in range(n):
            want = (L.kqo_silu_mul_neon(float(g[i]), float(u[i])) if i < nv else
                    F32(F32(L.kqo_fast_silu(float(g[i]))) * u[i]))
            assert F32(got[i]).view(np.uint32) == F32(want).view(np.uint32), (n, i)


def test_fast_silu_matches_reference_x86(orc, ref):
    rng = np.random.default_rng(11)
    g = np.concatenate([rng.standard_normal(3000) * 8, rng.uniform(-25, 25, 1000),
                        [0.0, -0.0, -20.0, 20.0, -20.000002, 20.000002, 1e-30, -1e-30, 88.0,
                         -88.0, 1e30, -1e30]]).astype(F32)
    u = rng.standard_normal(g.size).astype(F32)
    got = g.copy()
    ref.kref_silu_mul(got.ctypes.data, u.ctypes.data, g.size)
    L = orc.lib()
    want = np.array([F32(L.kqo_fast_silu(float(a))) * b for a, b in zip(g, u)], F32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("n", [1, 4])
def test_matmul_silu_composition(orc, n):
    import synth
    rows, cols = 20, 160
    w = synth.make_q4_weights(rows, cols, 4)
    rng = np.random.default_rng(n)
    g = rng.standard_normal((n, cols)).astype(F32) * 3
    u = rng.standard_normal((n, cols)).astype(F32)
    res = rng.standard_normal((n, rows)).astype(F32)
    got = orc.matmul_silu(w, g, u, rows, cols, residual=res)
    want = orc.matmul(w, orc.silu_mul(g, u).reshape(n, cols), rows, cols, residual=res)
    assert np.array_equal(got, want)


def recip_estimate_midpoint(a):
    """FRECPE's 9-bit estimate for the 8-bit mantissa bucket a (256..511) stated independently
    of the pseudocode's integer steps: the reciprocal of the bucket's midpoint (a + 1/2)/256,
    scaled to 9 bits and rounded half up, in exact rational arithmetic. (The pseudocode's
    b = 2^19 DIV (2a+1), r = (b+1) DIV 2 is floor(v/2 + 1/2) of v = 2^19/(2a+1), the same
    number.)"""
    from fractions import Fraction
    from math import floor
    return floor(Fraction(1 << 17) / (Fraction(a) + Fraction(1, 2)) + Fraction(1, 2))


def test_frecpe_every_bucket_matches_independent_statement(orc):
    L = orc.lib()
    rng = np.random.default_rng(8)
    table = {a: recip_estimate_midpoint(a) for a in range(256, 512)}
    assert all(256 <= r <= 511 for r in table.values())
    assert table[256] == 511 and table[511] == 256          # 1.0 -> 0.998046875
    for a, r in table.items():
        for e in (1, 64, 127, 128, 200, 252):
            low = int(rng.integers(0, 1 << 15))
            x = np.uint32((e << 23) | ((a - 256) << 15) | low).view(F32)
            want = np.uint32(((253 - e) << 23) | ((r - 256) << 15)).view(F32)
            got = F32(L.kqo_frecpe(float(x)))
            assert got.view(np.uint32) == want.view(np.uint32), (a, e)


def test_frecpe_check_catches_planted_rounding_mistakes():
    """The per-bucket check above separates the pseudocode's rounding from plausible
    transcription slips: r = b DIV 2 (no +1) keeps FRECPE(1.0) = 0.998046875, so the documented
    value alone would miss it, and a = 2*scaled (no +1) also changes buckets; both differ from
    the statement above in many buckets."""
    good = {a: recip_estimate_midpoint(a) for a in range(256, 512)}
    no_round = {a: ((1 << 19) // (2 * a + 1)) // 2 for a in range(256, 512)}
    no_half = {a: ((1 << 19) // (2 * a) + 1) // 2 for a in range(256, 512)}
    assert no_round[256] == good[256] == 511
    for bad in (no_round, no_half):
        assert sum(bad[a] != good[a] for a in good) >= 32
