"""The VQF loader (include/kq4_vqf.h) on the CPU - header and directory validation, per-layer q4
matrices - against two files the reference made itself:
  * tests/golden/synth_dual.vqf: the reference's own converter (vqf_convert, tests/golden/
    make_vqf.py) on a seeded synthetic model; every layer's q4 matrix read through the loader
    must equal the oracle's quantization + 4x4 repack of the same bf16 weights (those two
    oracle functions are pinned byte for byte to the reference's converter code in
    tests/test_oracle_codec.py);
  * tests/golden/vqf_header_legacy_qwen3vl8b.bin: the 4 KB header of a real Qwen3-VL-8B VQF that
    the reference keeps (docs/bench/20260915-rk3588-llama-ab/kv2_16k/vqf_hdr_orig.bin), written
    with the legacy 41-field VQFArch, so its data_offset/file_len sit 16 B earlier.
No GPU: nothing here uploads."""
import os
import struct

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden")
SYNTH = os.path.join(GOLD, "synth_dual.vqf")
LEGACY = os.path.join(GOLD, "vqf_header_legacy_qwen3vl8b.bin")

import sys  # noqa: E402
sys.path.insert(0, GOLD)
import make_vqf  # noqa: E402


def q4_tiles(orc, bits, rows, cols):
    """The oracle's VQF 4x4 tiles of a bf16 weight matrix: f32_to_q4_0 per row-major element
    run, then repack_q4_0_4x4."""
    f = np.ascontiguousarray(make_vqf.bf16_to_f32(bits).reshape(rows, cols))
    legacy = np.empty(rows * cols // 32 * 18, np.uint8)
    orc.lib().kqo_f32_to_q4_0(legacy.ctypes.data, f.ctypes.data, rows * cols)
    tiles = np.empty_like(legacy)
    assert orc.lib().kqo_repack_q4_0_4x4(legacy.ctypes.data, tiles.ctypes.data, rows, cols) == 0
    return tiles


def test_legacy_header_fixture(kq4_cpu):
    buf = open(LEGACY, "rb").read()
    file_len = struct.unpack_from("<Q", buf, 192)[0]
    info = kq4_cpu.vqf_parse_header(buf, file_len + 8)          # plaintext: 8-B FNV trailer
    assert info.legacy_header == 1 and info.version == 2 and info.flags == 0x63
    assert (info.dim, info.n_layers, info.n_heads, info.n_kv_heads, info.head_dim,
            info.ffn_dim, info.vocab_size) == (4096, 36, 32, 8, 128, 12288, 151936)
    assert info.data_offset == 4096 and info.file_len == 6601514048
    assert info.n_experts == 0 and info.n_tensors == 41
    # the 8B gate matrix: 36 layers x 12288 x 4096 at 18 B per 32 weights
    e = buf[448 + 64 * 10:448 + 64 * 11]
    assert e[:7] == b"q4_gate" and struct.unpack_from("<Q", e, 56)[0] == 36 * 12288 * 4096 // 32 * 18
    # any other size makes both candidate layouts inconsistent
    with pytest.raises(kq4_cpu.KQ4Error, match="undetermined"):
        kq4_cpu.vqf_parse_header(buf, file_len + 9)


def test_synth_file_info_and_directory(kq4_cpu):
    with kq4_cpu.Vqf(SYNTH, verify_checksum=True) as v:
        i, c = v.info, make_vqf.CONFIG
        assert i.legacy_header == 0 and i.version == 2
        assert i.flags & 0x2                                      # VQF_FLAG_Q4_4X4
        assert (i.dim, i.n_layers, i.n_heads, i.n_kv_heads, i.head_dim, i.ffn_dim,
                i.vocab_size) == (c["hidden_size"], c["num_hidden_layers"],
                                  c["num_attention_heads"], c["num_key_value_heads"],
                                  c["head_dim"], c["intermediate_size"], c["vocab_size"])
        assert abs(i.norm_eps - 1e-6) < 1e-12
        names = [e[0] for e in v.entries()]
        for n in ("q4_q", "q4_k", "q4_v", "q4_o", "q4_gate", "q4_up", "q4_down", "q4_lm"):
            assert n in names


PROJ = {0: "self_attn.q_proj", 1: "self_attn.k_proj", 2: "self_attn.v_proj",
        3: "self_attn.o_proj", 4: "mlp.gate_proj", 5: "mlp.up_proj", 6: "mlp.down_proj"}


def test_every_layer_matrix_matches_the_oracle(kq4_cpu, orc):
    T = make_vqf.model_tensors()
    with kq4_cpu.Vqf(SYNTH) as v:
        for layer in range(make_vqf.CONFIG["num_hidden_layers"]):
            for proj, name in PROJ.items():
                tiles, rows, cols = v.q4_matrix(proj, layer)
                src = T[f"model.layers.{layer}.{name}.weight"]
                assert src.shape == (rows, cols), (proj, src.shape, rows, cols)
                assert np.array_equal(tiles, q4_tiles(orc, src, rows, cols)), (layer, name)
        tiles, rows, cols = v.q4_matrix(kq4_cpu.PROJ_LM, 0)
        assert np.array_equal(tiles, q4_tiles(orc, T["lm_head.weight"], rows, cols))


def test_every_layer_q8_matrix_matches_the_oracle(kq4_cpu, orc):
    """The dual file's Q8_0 8x8 prefill weights: the oracle's f32_to_q8_0 + 8x8 repack (both
    pinned byte for byte to the reference's converter code in tests/test_oracle_q8.py)."""
    T = make_vqf.model_tensors()
    with kq4_cpu.Vqf(SYNTH) as v:
        assert v.info.flags & 0x1                                  # VQF_FLAG_Q8_8X8
        for layer in range(make_vqf.CONFIG["num_hidden_layers"]):
            for proj, name in PROJ.items():
                tiles, rows, cols, g = v.q8_matrix(proj, layer)
                assert g == 8
                f = make_vqf.bf16_to_f32(T[f"model.layers.{layer}.{name}.weight"])
                assert np.array_equal(tiles, orc.q8_tiles(f, rows, cols, 8)), (layer, name)
        tiles, rows, cols, g = v.q8_matrix(kq4_cpu.PROJ_LM, 0)
        assert np.array_equal(tiles, orc.q8_tiles(make_vqf.bf16_to_f32(T["lm_head.weight"]),
                                                  rows, cols, 8))


def test_rejects_bad_files(kq4_cpu, tmp_path):
    data = bytearray(open(SYNTH, "rb").read())

    def write(b, name):
        p = tmp_path / name
        p.write_bytes(bytes(b))
        return str(p)

    bad = bytearray(data)
    bad[-100] ^= 0x55                                              # a data byte
    kq4_cpu.Vqf(write(bad, "flip.vqf")).close()                    # opens without the check
    with pytest.raises(kq4_cpu.KQ4Error, match="checksum"):
        kq4_cpu.Vqf(write(bad, "flip.vqf"), verify_checksum=True)
    with pytest.raises(kq4_cpu.KQ4Error, match="undetermined"):
        kq4_cpu.Vqf(write(data[:-1], "short.vqf"))
    bad = bytearray(data)
    bad[0] ^= 1
    with pytest.raises(kq4_cpu.KQ4Error, match="magic"):
        kq4_cpu.Vqf(write(bad, "magic.vqf"))
    bad = bytearray(data)
    struct.pack_into("<I", bad, 4, 7)
    with pytest.raises(kq4_cpu.KQ4Error, match="version"):
        kq4_cpu.Vqf(write(bad, "ver.vqf"))
    bad = bytearray(data)
    struct.pack_into("<I", bad, 8, struct.unpack_from("<I", bad, 8)[0] | 0x80)   # VQF_FLAG_ENC
    bad += b"\0" * 24                                              # 32-B HMAC trailer
    struct.pack_into("<Q", bad, 208, len(bad) - 32)
    with pytest.raises(kq4_cpu.KQ4Error, match="encrypted"):
        kq4_cpu.Vqf(write(bad, "enc.vqf"))
    bad = bytearray(data)
    struct.pack_into("<I", bad, 8, struct.unpack_from("<I", bad, 8)[0] & ~0x2)   # no Q4_4X4
    with kq4_cpu.Vqf(write(bad, "noq4.vqf")) as v:
        with pytest.raises(kq4_cpu.KQ4Error, match="4x4"):
            v.q4_matrix(0, 0)
    with kq4_cpu.Vqf(SYNTH) as v:
        with pytest.raises(kq4_cpu.KQ4Error, match="layer"):
            v.q4_matrix(4, make_vqf.CONFIG["num_hidden_layers"])
        with pytest.raises(kq4_cpu.KQ4Error, match="projection"):
            v.q4_matrix(9, 0)


def test_layer_bound_does_not_wrap(kq4_cpu, tmp_path):
    """A crafted arch (dim = ffn_dim = 2^30, 256 layers) makes a gate layer 9 * 2^56 bytes, so
    layer 255 ends at 9 * 2^64: a product-based bound wraps to 0 and would hand out a wild
    pointer. The loader bounds layers by division and refuses it."""
    data = bytearray(open(SYNTH, "rb").read())
    struct.pack_into("<I", data, 16, 1 << 30)                     # VQFArch.dim
    struct.pack_into("<I", data, 20, 256)                         # n_layers
    struct.pack_into("<I", data, 36, 1 << 30)                     # ffn_dim
    p = tmp_path / "wrap.vqf"
    p.write_bytes(bytes(data))
    with kq4_cpu.Vqf(str(p)) as v:
        for layer in (0, 255):
            with pytest.raises(kq4_cpu.KQ4Error, match="too few"):
                v.q4_matrix(kq4_cpu.PROJ_GATE, layer)
