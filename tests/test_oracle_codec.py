"""Pins the weight codec: legacy Q4_0 encoder (vqf_convert/src/quant_kernels.c:118-151), the
legacy -> 4x4 tile repack (qk_repack.c:19-46) and the oracle's tile decoder, against the
reference's own converter code built in oracle/_ref, a round trip, and an independent numpy
decoder; the tile layout is also pinned against the reference engine's own x86 decode path."""
import numpy as np

import synth


def legacy_weights(rows, cols, seed):
    """Reference-style weights incl. all-zero rows and a +-1000 row (vqf_convert/test/qk_test.c)."""
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)
    w[min(32, rows - 1)] = 0
    w[min(39, rows - 1), ::2] = 1000.0
    w[min(39, rows - 1), 1::2] = -1000.0
    return w


def encode(orc, w):
    rows, cols = w.shape
    out = np.empty(rows * cols // 32 * 18, np.uint8)
    orc.lib().kqo_f32_to_q4_0(out.ctypes.data, np.ascontiguousarray(w).ctypes.data, w.size)
    return out


def repack(orc, legacy, rows, cols):
    t = np.empty(rows // 4 * cols // 32 * 72, np.uint8)
    assert orc.lib().kqo_repack_q4_0_4x4(legacy.ctypes.data, t.ctypes.data, rows, cols) == 0
    return t


def test_encoder_and_repack_match_reference(orc, ref):
    rows, cols = 48, 256
    w = legacy_weights(rows, cols, 1)
    mine = encode(orc, w)
    theirs = np.empty_like(mine)
    ref.kref_f32_to_q4_0(theirs.ctypes.data, w.ctypes.data, w.size)
    assert np.array_equal(mine, theirs)
    t_mine = repack(orc, mine, rows, cols)
    buf = theirs.copy()
    assert ref.kref_repack_q4_0_4x4(buf.ctypes.data, rows, cols) == 0
    assert np.array_equal(t_mine, buf[: t_mine.size])


def test_repack_round_trip(orc):
    rows, cols = 16, 128
    legacy = np.random.default_rng(2).integers(0, 256, rows * cols // 32 * 18, dtype=np.uint8)
    t = repack(orc, legacy, rows, cols)
    back = np.empty_like(legacy)
    assert orc.lib().kqo_unpack_4x4_to_q4_0(t.ctypes.data, back.ctypes.data, rows, cols) == 0
    assert np.array_equal(back, legacy)


def test_tile_layout_closed_form(orc):
    """Row r, element e of a repacked tile: byte 8 + 16*(e&15>>2) + 4r + (e&3), nibble lo/hi,
    value = nibble(n) - 8 with the stored nibble n^8."""
    rows, cols = 4, 32
    legacy = np.zeros(4 * 18, np.uint8)
    for r in range(4):
        legacy[r * 18:r * 18 + 2] = np.frombuffer(np.float16(r + 1).tobytes(), np.uint8)
        for j in range(16):
            lo, hi = (j + r) % 16, (15 - j + r) % 16
            legacy[r * 18 + 2 + j] = lo | (hi << 4)
    t = repack(orc, legacy, rows, cols)
    for r in range(4):
        assert np.frombuffer(t[2 * r:2 * r + 2].tobytes(), np.float16)[0] == r + 1
        for e in range(32):
            j = e & 15
            n = (j + r) % 16 if e < 16 else (15 - j + r) % 16
            assert orc.lib().kqo_tile_weight(t.ctypes.data, r, e) == n - 8
            byte = t[8 + (j >> 2) * 16 + r * 4 + (j & 3)]
            assert ((byte & 15) if e < 16 else (byte >> 4)) == n ^ 8


def test_oracle_decoder_matches_numpy_decoder(orc):
    rows, cols = 8, 96
    t = synth.make_q4_weights(rows, cols, 9).reshape(-1)
    wi = synth.tile_weights_int(t, rows, cols)
    nb = cols // 32
    for n in range(rows):
        for e in range(cols):
            tile = t[((n // 4) * nb + e // 32) * 72:]
            assert orc.lib().kqo_tile_weight(tile.ctypes.data, n % 4, e % 32) == wi[n, e]


def test_layout_against_reference_engine_decode(orc, ref):
    """The reference's x86 single-token path (q4_dense4_x86, fp32 activations) decodes the same
    4x4 tiles; a float64 dot over our decoded weights must reproduce it to fp32 rounding."""
    rows, cols = 64, 512
    t = synth.make_q4_weights(rows, cols, 4)
    x = synth.make_activations(1, cols, 5)
    out = np.empty(rows, np.float32)
    ref.kref_matvec(out.ctypes.data, t.ctypes.data, x.ctypes.data, rows, cols)
    w = synth.tile_weights_int(t, rows, cols).astype(np.float64)
    sc = np.repeat(synth.tile_scales(t, rows, cols).astype(np.float64), 32, axis=1)
    want = (w * sc) @ x[0].astype(np.float64)
    err = np.abs(out - want).max() / np.abs(want).max()
    assert err < 1e-5, err
    # a transposed row order inside the tile would not pass
    w_bad = w.reshape(rows // 4, 4, cols)[:, ::-1].reshape(rows, cols)
    assert np.abs((w_bad * sc) @ x[0] - out).max() / np.abs(want).max() > 1e-2
