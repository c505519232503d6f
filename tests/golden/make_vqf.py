"""Writes tests/golden/synth_dual.vqf: a genuine VQF file made by the reference's own converter
(vqf_convert, built from /root/reference by `make -C oracle conv` into oracle/_ref/vqf_conv, in
its default "dual" mode: Q4_0 4x4 decode weights and Q8_0 8x8 prefill weights) from a tiny
synthetic Qwen3-shaped model defined here (bf16 safetensors + config.json, seeded). The VQF
loader tests read it back and check every layer's q4 and q8 matrix against the oracle's own
quantization of the same weights (model_tensors() regenerates them).

    python tests/golden/make_vqf.py
"""
import json
import os
import struct
import subprocess
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
OUT = os.path.join(HERE, "synth_dual.vqf")

CONFIG = dict(model_type="qwen3", hidden_size=128, num_hidden_layers=2, num_attention_heads=2,
              num_key_value_heads=1, head_dim=64, intermediate_size=256, vocab_size=64,
              max_position_embeddings=512, bos_token_id=1, eos_token_id=2, rope_theta=1000000.0,
              rms_norm_eps=1e-06, tie_word_embeddings=False)


def bf16_bits(a):
    """float32 -> bfloat16 bits, round to nearest even."""
    u = np.asarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f32(b):
    return (np.asarray(b, np.uint32) << 16).view(np.float32)


def model_tensors():
    """name -> bf16 bits (uint16 array), in file order; seeded."""
    c = CONFIG
    d, ff, V, hd = c["hidden_size"], c["intermediate_size"], c["vocab_size"], c["head_dim"]
    qo, ko = c["num_attention_heads"] * hd, c["num_key_value_heads"] * hd
    rng = np.random.default_rng(2024)
    T = {"model.embed_tokens.weight": rng.standard_normal((V, d)) * 0.05,
         "model.norm.weight": 1 + 0.1 * rng.standard_normal(d),
         "lm_head.weight": rng.standard_normal((V, d)) * 0.05}
    for layer in range(c["num_hidden_layers"]):
        p = f"model.layers.{layer}."
        T[p + "input_layernorm.weight"] = 1 + 0.1 * rng.standard_normal(d)
        T[p + "post_attention_layernorm.weight"] = 1 + 0.1 * rng.standard_normal(d)
        T[p + "self_attn.q_proj.weight"] = rng.standard_normal((qo, d)) * 0.05
        T[p + "self_attn.k_proj.weight"] = rng.standard_normal((ko, d)) * 0.05
        T[p + "self_attn.v_proj.weight"] = rng.standard_normal((ko, d)) * 0.05
        T[p + "self_attn.o_proj.weight"] = rng.standard_normal((d, qo)) * 0.05
        T[p + "mlp.gate_proj.weight"] = rng.standard_normal((ff, d)) * 0.05
        T[p + "mlp.up_proj.weight"] = rng.standard_normal((ff, d)) * 0.05
        T[p + "mlp.down_proj.weight"] = rng.standard_normal((d, ff)) * 0.05
    return {k: bf16_bits(v) for k, v in T.items()}


def write_model(d):
    with open(os.path.join(d, "config.json"), "w") as f:
        json.dump(CONFIG, f)
    hdr, blobs, off = {}, [], 0
    for k, v in model_tensors().items():
        b = v.tobytes()
        hdr[k] = {"dtype": "BF16", "shape": list(v.shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    h = json.dumps(hdr).encode()
    h += b" " * ((8 - len(h) % 8) % 8)
    with open(os.path.join(d, "model.safetensors"), "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def main():
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "conv"], check=True)
    conv = os.path.join(ROOT, "oracle", "_ref", "vqf_conv")
    with tempfile.TemporaryDirectory() as d:
        write_model(d)
        subprocess.run([conv, "--model", d, "--convert-vqf", OUT, "--wmode", "dual"], check=True)
    print("wrote", OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    sys.exit(main())
