"""Writes the committed golden fixtures under tests/golden/ (run in the build container, where
/root/reference exists).

The reference holds no golden vectors for this path, so the fixtures are made here:
  quant.npz   activation quantizer: outputs of the reference's own quantize_row_q8_0_act
              (vllm_safetensors.c:7893-7920, built from /root/reference into oracle/_ref)
  codec.npz   legacy Q4_0 encoder + 4x4 repack: outputs of the reference's own f32_to_q4_0
              (vqf_convert/src/quant_kernels.c:118-151) and repack_q4_0_4x4_inplace
              (vqf_convert/src/qk_repack.c:19-46), built the same way
  moe.npz     MoE FFN, int8 activation track (VLLM_ACTQ=1 VLLM_ACTQ16=0): outputs of the
              reference's own st_moe_ffn_sparse_q4 (vllm_safetensors.c:12921-13398) per token,
              router included
  dense.npz   dense op per fp32 chain (CTILE / GEMV32 / ASM / AUTO dispatch) and the integer
              block sums: outputs of the oracle (oracle/kq4_oracle.c), since the reference
              computes these chains only in AArch64 NEON code that cannot run here; the oracle's
              chains are pinned by tests/test_oracle_matmul.py
Each file also stores its inputs, so a test needs nothing but numpy.load(allow_pickle=False).

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (os.path.join(ROOT, "oracle"), os.path.join(ROOT, "kestrel-llm_amd")):
    sys.path.insert(0, p)
os.environ.setdefault("VLLM_ACTQ", "1")
os.environ.setdefault("VLLM_ACTQ16", "0")

import oracle  # noqa: E402
import synth  # noqa: E402

P = lambda a: a.ctypes.data  # noqa: E731


def quant_fixture(ref):
    rng = np.random.default_rng(101)
    x = rng.standard_normal((16, 256)).astype(np.float32)
    x[0, :32] = 0.0                                    # all-zero block -> d = 1e-10/127
    x[1, :32] *= np.float32(1e-30)
    x[2, 32:64] = 127.0
    x[2, 40] = -127.0                                  # -amax -> -126
    x[3, :32] = np.float32(1e-41)                      # subnormal inputs
    x[4] *= np.float32(1e4)
    x[5, 64:96] = np.float32(0.49999997)
    x[6, 96:128] = np.linspace(-127, 127, 32, dtype=np.float32) + np.float32(0.5)
    x[7] *= np.float32(3e-3)
    q = np.empty((16, 256), np.int8)
    d = np.empty((16, 8), np.float32)
    for t in range(16):
        ref.kref_quantize_row(P(x[t]), P(q[t]), P(d[t]), 256)
    return dict(x=x, q=q, d=d)


def codec_fixture(ref):
    rows, cols = 8, 96
    rng = np.random.default_rng(102)
    w = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)
    w[3] = 0.0
    w[5, ::2] = 1000.0
    w[5, 1::2] = -1000.0
    legacy = np.empty(rows * cols // 32 * 18, np.uint8)
    ref.kref_f32_to_q4_0(P(legacy), P(w), w.size)
    tiles = legacy.copy()
    assert ref.kref_repack_q4_0_4x4(P(tiles), rows, cols) == 0
    return dict(w=w, legacy=legacy, tiles=tiles[: rows // 4 * cols // 32 * 72], rows=rows,
                cols=cols)


def moe_fixture(ref):
    d, ne, tk, ef, T = 64, 8, 2, 32, 3
    cfg = dict(hidden=d, experts=ne, top_k=tk, ef=ef)
    G, U, D = synth.make_moe(cfg, 103)
    router = (np.random.default_rng(104).standard_normal((ne, d)) * 0.2).astype(np.float32)
    X = synth.make_activations(T, d, 105)
    Y = np.empty((T, d), np.float32)
    for t in range(T):
        xt = np.ascontiguousarray(X[t:t + 1])
        assert ref.kref_moe_ffn(P(Y[t]), P(xt), 1, P(router), P(G), P(U), P(D), ne, tk, d,
                                ef) == 1
    return dict(G=G.reshape(-1), U=U.reshape(-1), D=D.reshape(-1), router=router, X=X, Y=Y,
                shape=np.array([d, ne, tk, ef], np.int32))


def dense_fixture():
    rows, cols, n = 12, 96, 5
    w = synth.make_q4_weights(rows, cols, 106, sigma=0.015, floor=0.0).reshape(-1)
    x = synth.make_activations(n, cols, 107)
    res = synth.make_activations(n, rows, 108)
    xq, xd = oracle.quantize(x, cols)
    lo, hi = oracle.block_sums(w, xq, rows, cols)
    out = {f"out_c{c}": oracle.matmul(w, x, rows, cols, chain=c) for c in range(4)}
    out.update({f"res_c{c}": oracle.matmul(w, x, rows, cols, residual=res, chain=c)
                for c in range(4)})
    return dict(w=w, x=x, residual=res, xq=xq, xd=xd, s_lo=lo, s_hi=hi, rows=rows, cols=cols,
                **out)


def main():
    oracle.build(with_ref=True)
    if not oracle.ref_available():
        sys.exit("needs the reference harness (oracle/_ref, built from /root/reference)")
    ref = oracle.ref(1)
    np.savez_compressed(os.path.join(HERE, "quant.npz"), **quant_fixture(ref))
    np.savez_compressed(os.path.join(HERE, "codec.npz"), **codec_fixture(ref))
    np.savez_compressed(os.path.join(HERE, "moe.npz"), **moe_fixture(ref))
    np.savez_compressed(os.path.join(HERE, "dense.npz"), **dense_fixture())
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
