"""The stream layout of the device weights (kq4_weights_prepare_dev): a pure regrouping of the
VQF 4x4 tiles, every tile byte kept, padding zero.

CPU: the numpy construction below (reshape/transpose of the padded tile array) agrees with the
per-byte address formula the kernels use (kq4_stream_off), and with the size the library
reports. GPU: the library's repack kernel writes exactly the numpy construction."""
import numpy as np
import pytest

import synth

CHUNK, CB = 9216, 16


def stream_layout(w, rows, cols):
    """[set][stage] chunks of 9216 B. Nibble part: unit i, lane l = 32*h + row at
    1024*i + 16*l = 8 bytes for block 2i then 8 for block 2i+1, byte 4d+k = code of element
    16h+8d+k | code of element 16h+8d+4+k << 4. Scale part at 8192 + 16*l: the f16 scales of
    blocks 8h .. 8h+7 of the row."""
    G, nb = rows // 4, cols // 32
    sets, nst = -(-rows // 32), -(-nb // CB)
    t = np.asarray(w, np.uint8).reshape(G, nb, 72)
    # per row: the 16 code bytes and the f16 scale of every block
    qs = t[:, :, 8:].reshape(G, nb, 4, 4, 4).transpose(0, 3, 1, 2, 4).reshape(rows, nb, 16)
    sc = t[:, :, :8].copy().view(np.uint16).transpose(0, 2, 1).reshape(rows, nb)
    code = np.concatenate([qs & 0xF, qs >> 4], axis=2)          # (rows, nb, 32), element order
    C = np.zeros((sets * 32, nst * CB, 32), np.uint8)
    C[:rows, :nb] = code
    S = np.zeros((sets * 32, nst * CB), np.uint16)
    S[:rows, :nb] = sc
    C = C.reshape(sets * 32, nst * CB, 2, 2, 2, 4)                # h, d, nibble, k
    H = (C[..., 0, :] | (C[..., 1, :] << 4)).reshape(sets * 32, nst * CB, 2, 8)
    nib = H.reshape(sets, 32, nst, 8, 2, 2, 8).transpose(0, 2, 3, 5, 1, 4, 6)
    nib = nib.reshape(sets, nst, 8192)
    scl = S.reshape(sets, 32, nst, 2, 8).transpose(0, 2, 3, 1, 4).reshape(sets, nst, 512)
    scl = np.ascontiguousarray(scl).view(np.uint8)
    return np.ascontiguousarray(np.concatenate([nib, scl], axis=2)).reshape(-1)


def stream_nib(row, b, h, nst):
    return (((row >> 5) * nst + (b >> 4)) * CHUNK + 1024 * ((b & 15) >> 1)
            + 16 * ((row & 31) + 32 * h) + 8 * (b & 1))


def stream_scale(row, b, nst):
    return (((row >> 5) * nst + (b >> 4)) * CHUNK + 8192
            + 16 * ((row & 31) + 32 * ((b & 15) >> 3)) + 2 * (b & 7))


SHAPES = [(4, 32), (20, 160), (100, 1056), (64, 512), (36, 608)]


@pytest.mark.parametrize("rows,cols", SHAPES)
def test_layout_matches_address_formula(rows, cols):
    """Every weight element and scale read back through the kernels' address formulas equals
    the VQF definition: element e of row m of a tile is byte 8 + 16*(j>>2) + 4m + (j&3),
    j = e & 15, low nibble for e < 16, high for e >= 16; its scale is f16 at byte 2m."""
    w = synth.make_q4_weights(rows, cols, 3)
    s = stream_layout(w, rows, cols)
    G, nb = rows // 4, cols // 32
    nst = -(-nb // CB)
    assert s.size == -(-rows // 32) * nst * CHUNK
    tiles = w.reshape(G, nb, 72)
    seen = np.zeros(s.size, bool)
    for row in range(rows):
        g, m = divmod(row, 4)
        for b in range(nb):
            for e in range(32):
                j = e & 15
                byte = tiles[g, b, 8 + 16 * (j >> 2) + 4 * m + (j & 3)]
                want = byte & 0xF if e < 16 else byte >> 4
                h, jj = divmod(e, 16)
                d, r = divmod(jj, 8)
                nibble, k = divmod(r, 4)
                off = stream_nib(row, b, h, nst) + 4 * d + k
                assert (s[off] >> (4 * nibble)) & 0xF == want, (row, b, e)
                seen[off] = True
            off = stream_scale(row, b, nst)
            assert s[off] == tiles[g, b, 2 * m] and s[off + 1] == tiles[g, b, 2 * m + 1]
            seen[off:off + 2] = True
    assert not s[~seen].any()                      # everything else is padding, zero


def test_library_size(kq4_cpu):
    for rows, cols in SHAPES:
        nb = cols // 32
        assert kq4_cpu.lib().kq4_weights_stream_bytes(rows, cols) == \
            -(-rows // 32) * -(-nb // CB) * CHUNK
    assert kq4_cpu.lib().kq4_weights_stream_bytes(6, 32) == 0
    assert kq4_cpu.lib().kq4_weights_stream_bytes(8, 48) == 0


@pytest.mark.gpu
@pytest.mark.parametrize("rows,cols", SHAPES + [(132, 4096), (100, 2080), (6144, 2048)])
def test_gpu_prepare_matches_layout(kq4, torch_dev, rows, cols):
    torch = torch_dev
    w = synth.make_q4_weights(rows, cols, rows + cols)
    dst = kq4.prepare_dev(torch.from_numpy(w).cuda(), rows, cols)
    torch.cuda.synchronize()
    assert np.array_equal(dst.cpu().numpy(), stream_layout(w, rows, cols))


# ---- q8 stream layout: [set][stage] chunks of 8704 B, 8 blocks per stage ------------------------
CHUNK8, CB8 = 8704, 8


def q8_stream_layout(tiles, g, rows, cols):
    """Codes: lane l = 32*h + row at 1024*i + 16*l = the 16 int8 codes of elements 16h .. 16h+15
    of block i of the stage; scales at 8192 + 16*row: the row's 8 f16 scales."""
    nb = cols // 32
    sets, nst = -(-rows // 32), -(-nb // CB8)
    t = np.asarray(tiles, np.uint8).reshape(rows // g, nb, 34 * g)
    sc = t[:, :, :2 * g].copy().view(np.uint16).transpose(0, 2, 1).reshape(rows, nb)
    q = t[:, :, 2 * g:].reshape(rows // g, nb, 8, g, 4).transpose(0, 3, 1, 2, 4).reshape(rows, nb, 32)
    C = np.zeros((sets * 32, nst * CB8, 32), np.uint8)
    C[:rows, :nb] = q
    S = np.zeros((sets * 32, nst * CB8), np.uint16)
    S[:rows, :nb] = sc
    code = C.reshape(sets, 32, nst, 8, 2, 16).transpose(0, 2, 3, 4, 1, 5).reshape(sets, nst, 8192)
    scl = S.reshape(sets, 32, nst, 8).transpose(0, 2, 1, 3).reshape(sets, nst, 256)
    scl = np.ascontiguousarray(scl).view(np.uint8)
    return np.ascontiguousarray(np.concatenate([code, scl], axis=2)).reshape(-1)


def q8_tiles_synth(rows, cols, g, seed):
    """Random Q8_0 tiles: codes uniform in [-127, 127], f16 scales |N(0, 0.02)|."""
    rng = np.random.default_rng(seed)
    nb = cols // 32
    t = np.zeros((rows // g, nb, 34 * g), np.uint8)
    t[:, :, :2 * g] = np.abs(rng.standard_normal((rows // g, nb, g)) * 0.02).astype(
        np.float16).view(np.uint8).reshape(rows // g, nb, 2 * g)
    t[:, :, 2 * g:] = rng.integers(-127, 128, (rows // g, nb, 32 * g)).astype(np.int8).view(np.uint8)
    return t.reshape(-1)


Q8_SHAPES = [(8, 32, 8), (24, 160, 8), (40, 288, 8), (20, 96, 4), (36, 608, 4)]


@pytest.mark.parametrize("rows,cols,g", Q8_SHAPES)
def test_q8_layout_matches_address_formula(rows, cols, g):
    """Every code and scale read back at the kernels' q8 addresses (kq8_stream_code /
    kq8_stream_scale) equals the tile definition: row m of a tile, element 4k+i at byte
    2g + 4g*k + 4m + i, scale f16 at byte 2m."""
    w = q8_tiles_synth(rows, cols, g, rows + cols)
    s = q8_stream_layout(w, g, rows, cols)
    nb = cols // 32
    nst = -(-nb // CB8)
    assert s.size == -(-rows // 32) * nst * CHUNK8
    tiles = w.reshape(rows // g, nb, 34 * g)
    seen = np.zeros(s.size, bool)
    for row in range(rows):
        gi, m = divmod(row, g)
        for b in range(nb):
            base = ((row >> 5) * nst + (b >> 3)) * CHUNK8
            for e in range(32):
                k, i = divmod(e, 4)
                want = tiles[gi, b, 2 * g + 4 * g * k + 4 * m + i]
                h, j = divmod(e, 16)
                off = base + 1024 * (b & 7) + 16 * ((row & 31) + 32 * h) + j
                assert s[off] == want, (row, b, e)
                seen[off] = True
            off = base + 8192 + 16 * (row & 31) + 2 * (b & 7)
            assert s[off] == tiles[gi, b, 2 * m] and s[off + 1] == tiles[gi, b, 2 * m + 1]
            seen[off:off + 2] = True
    assert not s[~seen].any()


def test_q8_library_size(kq4_cpu):
    for rows, cols, g in Q8_SHAPES:
        nb = cols // 32
        assert kq4_cpu.lib().kq4_q8_weights_stream_bytes(rows, cols) == \
            -(-rows // 32) * -(-nb // CB8) * CHUNK8


@pytest.mark.gpu
@pytest.mark.parametrize("rows,cols,g", Q8_SHAPES + [(4096, 4096, 8), (128, 12288, 4)])
def test_gpu_q8_prepare_matches_layout(kq4, torch_dev, rows, cols, g):
    torch = torch_dev
    w = q8_tiles_synth(rows, cols, g, rows * 3 + cols)
    dst = kq4.q8_prepare_dev(torch.from_numpy(w).cuda(), rows, cols, g=g)
    dst2 = kq4.q8_prepare_dev(w, rows, cols, g=g)                  # from host memory
    torch.cuda.synchronize()
    want = q8_stream_layout(w, g, rows, cols)
    assert np.array_equal(dst.cpu().numpy(), want)
    assert np.array_equal(dst2.cpu().numpy(), want)
