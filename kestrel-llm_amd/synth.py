"""Seeded synthetic inputs in the reference's formats (numpy, host side).

Weights are written directly in the VQF 4x4 tile layout (72 B per 4 rows x 32 columns: 4 f16 row
scales, then nibble byte 8+16k+4r+i = legacy qs byte 4k+i of row r XOR 0x88, as
vqf_convert/src/qk_repack.c:19-46 lays them out). Nibble codes are uniform in 0..15 (weights
n-8 in [-8, 7]); scales are f16(|N(0, sigma)| + floor) (config 3 uses no
floor so f16 subnormal and zero scales occur). Activations are fp32 N(0, 1). The generator is
numpy's PCG64 (np.random.default_rng(seed)), so a seed names the same bytes on every machine.
"""
import numpy as np

# Shapes of the BASELINE.json configurations.
QWEN3VL_2B = dict(hidden=2048, q_heads=16, kv_heads=8, head_dim=128, ffn=6144, layers=28,
                  vocab=151936)
QWEN3_8B = dict(hidden=4096, q_heads=32, kv_heads=8, head_dim=128, ffn=12288, layers=36,
                vocab=151936)
QWEN3_30B_A3B_MOE = dict(hidden=2048, experts=128, top_k=8, ef=768)

SCALE_2B = dict(sigma=0.02, floor=1e-4)
SCALE_8B = dict(sigma=0.015, floor=0.0)


def q4_tile_bytes(rows, cols):
    return (rows // 4) * (cols // 32) * 72


def make_q4_weights(rows, cols, seed, sigma=0.02, floor=1e-4):
    """uint8 [rows/4, cols/32, 72] 4x4 tiles with uniform codes and f16 |N(0,sigma)|+floor scales."""
    assert rows % 4 == 0 and cols % 32 == 0
    rng = np.random.default_rng(seed)
    g, nb = rows // 4, cols // 32
    tiles = np.empty((g, nb, 72), np.uint8)
    sc = (np.abs(rng.standard_normal((g, nb, 4), dtype=np.float32)) * np.float32(sigma)
          + np.float32(floor)).astype(np.float16)
    tiles[:, :, :8] = sc.view(np.uint8).reshape(g, nb, 8)
    # uniform codes n in 0..15 for both nibbles; the stored nibble is n ^ 8
    codes = rng.integers(0, 256, size=(g, nb, 64), dtype=np.uint8)
    tiles[:, :, 8:] = codes ^ np.uint8(0x88)
    return tiles


def make_q8_weights(rows, cols, seed, sigma=0.015, g=8):
    """uint8 Q8_0 tiles of g rows (block_q8_0x8 for g = 8): codes uniform in [-127, 127], f16
    |N(0, sigma)| row scales (the q8 counterpart of the config-3 q4 weights)."""
    assert rows % g == 0 and cols % 32 == 0
    rng = np.random.default_rng(seed)
    G, nb = rows // g, cols // 32
    tiles = np.empty((G, nb, 34 * g), np.uint8)
    sc = (np.abs(rng.standard_normal((G, nb, g), dtype=np.float32)) * np.float32(sigma)).astype(
        np.float16)
    tiles[:, :, :2 * g] = sc.view(np.uint8).reshape(G, nb, 2 * g)
    tiles[:, :, 2 * g:] = rng.integers(-127, 128, size=(G, nb, 32 * g), dtype=np.int8).view(np.uint8)
    return tiles


def make_activations(n, cols, seed):
    return np.random.default_rng(seed).standard_normal((n, cols), dtype=np.float32)


def tile_weights_int(tiles, rows, cols):
    """Signed weights n-8 as int8 [rows, cols] (decoder for checks; vq4x4_w semantics)."""
    g, nb = rows // 4, cols // 32
    t = tiles.reshape(g, nb, 72)
    qs = t[:, :, 8:].reshape(g, nb, 4, 4, 4)           # [g][b][k][r][i]
    lo = (qs & 15).astype(np.int16) ^ 8
    hi = (qs >> 4).astype(np.int16) ^ 8
    lo = lo.transpose(0, 3, 1, 2, 4).reshape(g, 4, nb, 16)   # [g][r][b][4k+i]
    hi = hi.transpose(0, 3, 1, 2, 4).reshape(g, 4, nb, 16)
    w = np.concatenate([lo, hi], axis=3) - 8                  # element e<16 lo, e>=16 hi
    return w.reshape(rows, cols).astype(np.int8)


def tile_scales(tiles, rows, cols):
    """f32 row scales [rows, cols/32]."""
    g, nb = rows // 4, cols // 32
    sc = tiles.reshape(g, nb, 72)[:, :, :8].copy().view(np.float16).reshape(g, nb, 4)
    return sc.astype(np.float32).transpose(0, 2, 1).reshape(rows, nb)


def layer_shapes(cfg):
    """(name, rows, cols) of one decoder layer's linear set: QKV, O, gate, up, down."""
    h, hd = cfg["hidden"], cfg["head_dim"]
    q, kv = cfg["q_heads"] * hd, cfg["kv_heads"] * hd
    return [("q", q, h), ("k", kv, h), ("v", kv, h), ("o", h, q), ("gate", cfg["ffn"], h),
            ("up", cfg["ffn"], h), ("down", h, cfg["ffn"])]


def make_moe(cfg, seed, sigma=0.02, floor=1e-4):
    """G/U [ne*ef, d] and D [d, ne*ef] 4x4 tiles for one MoE layer (config 5 gives no scale
    distribution; the config-1/2 one is used)."""
    d, ne, ef = cfg["hidden"], cfg["experts"], cfg["ef"]
    G = make_q4_weights(ne * ef, d, seed, sigma, floor)
    U = make_q4_weights(ne * ef, d, seed + 1, sigma, floor)
    D = make_q4_weights(d, ne * ef, seed + 2, sigma, floor)
    return G, U, D


def make_logits(T, ne, seed):
    return np.random.default_rng(seed).standard_normal((T, ne), dtype=np.float32)
