"""Pins the oracle's f16 <-> f32 conversions (vllm_safetensors.c:3614-3670).

f16 -> f32 is checked exhaustively against numpy's IEEE conversion; f32 -> f16 (RNE, subnormals,
overflow) against numpy on every f16 value, every midpoint between neighbours (exact ties, where
round-half-even decides), the f32 neighbours of those midpoints, and random bit patterns. Both
are also checked against the reference's own functions built in oracle/_ref.
"""
import numpy as np
import pytest


def all_f16_codes():
    return np.arange(65536, dtype=np.uint32).astype(np.uint16)


def test_f16_to_f32_exhaustive(orc):
    h = all_f16_codes()
    want = h.view(np.float16).astype(np.float32).view(np.uint32)
    f = orc.lib().kqo_f16_to_f32_bits
    got = np.array([f(int(v)) for v in h], np.uint32)
    nan = np.isnan(h.view(np.float16))
    assert np.array_equal(got[~nan], want[~nan])
    # NaN keeps its payload and is still NaN
    assert np.isnan(got[nan].view(np.float32)).all()


def _f32_probe_set():
    h = all_f16_codes()
    f = h.view(np.float16).astype(np.float32)
    f = f[np.isfinite(f)]
    fs = np.sort(np.unique(f[f >= 0]))
    mids = ((fs[:-1].astype(np.float64) + fs[1:].astype(np.float64)) / 2).astype(np.float32)
    up = np.nextafter(mids, np.float32(np.inf))
    dn = np.nextafter(mids, np.float32(-np.inf))
    rng = np.random.default_rng(7)
    rnd = rng.integers(0, 2**32, size=200000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    rnd = rnd[np.isfinite(rnd)]
    edge = np.array([65504.0, 65519.99, 65520.0, 1e9, 2.0**-24, 2.0**-25, 2.0**-26,
                     3 * 2.0**-26, 2.0**-14, 2.0**-14 - 2.0**-25, 0.0, np.inf], np.float32)
    pos = np.concatenate([f, mids, up, dn, rnd, edge]).astype(np.float32)
    return np.concatenate([pos, -pos])


def test_f32_to_f16_rne(orc):
    x = _f32_probe_set()
    want = x.astype(np.float16).view(np.uint16)
    f = orc.lib().kqo_f32_to_f16_bits
    got = np.array([f(float(v)) for v in x], np.uint16)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{bad.size} mismatches, first x={x[bad[0]]!r}"


def test_f16_against_reference(orc, ref):
    h = all_f16_codes()
    got = np.array([orc.lib().kqo_f16_to_f32_bits(int(v)) for v in h], np.uint32)
    want = np.array([ref.kref_f16_to_f32_bits(int(v)) for v in h], np.uint32)
    assert np.array_equal(got, want)
    # the MoE decoder vq_f16 (:10976-10998) decodes the same values
    vq = np.array([ref.kref_vq_f16(int(v)) for v in h[:31744]], np.float32).view(np.uint32)
    assert np.array_equal(vq, want[:31744])
    x = _f32_probe_set()[::7]
    g = np.array([orc.lib().kqo_f32_to_f16_bits(float(v)) for v in x], np.uint16)
    r = np.array([ref.kref_f32_to_f16_bits(float(v)) for v in x], np.uint16)
    assert np.array_equal(g, r)


@pytest.mark.parametrize("mistake", ["truncate", "ftz"])
def test_planted_mistakes_are_caught(mistake):
    """A plausible wrong encoder (mantissa truncation, or flush subnormals to zero, the
    reference's own earlier bug noted at :3634-3638) fails the numpy comparison above."""
    x = _f32_probe_set()
    want = x.astype(np.float16).view(np.uint16)
    if mistake == "truncate":
        u = x.view(np.uint32)
        bad = ((u >> 16) & 0x8000) | np.clip(((u >> 23) & 0xFF).astype(np.int64) - 112, 0, 31) << 10
        got = (bad | ((u >> 13) & 0x3FF)).astype(np.uint16)
    else:
        got = x.astype(np.float16)
        got[np.abs(got) < np.float16(2.0**-14)] = 0
        got = got.view(np.uint16)
    assert (got != want).any()
