"""The decode GEMV's in-kernel activation quantization, pinned code for code.

The decode GEMV quantizes its fp32 activations itself, every wave for its own stage (the FQ form
of kq4_gemv_kernel, in passes of up to 4 tokens), and with the SiLU product (FQ = 2, passes of
2 tokens). That is the path the decode hot path runs, including the headline benchmark; the
tests force it on (planner option gemv_fq = 1) at every token count 1..8. These tests run it against the same
kernel, same plan and same dot kind, fed with the oracle's codes through the pre-quantized entry
point (kq4_matmul_q_dev): the two launches differ only in where the codes come from, so the
outputs are bit-identical exactly when the in-kernel codes and scales are the oracle's
(quantize_row_q8_0_act vllm_safetensors.c:7893-7920), whose own pin is the reference-written
fixture tests/golden/quant.npz. Its rows carry the edge cases: an all-zero block (d = 1e-10/127),
a 1e-30-scaled block, +-amax (-> +127 / -126), subnormal inputs, x1e4 scales, 0.49999997,
exact .5 ties and tiny scales.

Every output row mixes all of a token's codes with random 4-bit weights and non-zero scales, so a
single differing code changes most outputs."""
import os

import numpy as np
import pytest

import synth

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def to_dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def quant_rows():
    return np.load(os.path.join(GOLD, "quant.npz"), allow_pickle=False)["x"]   # [16][256]


def bits(t):
    return t.cpu().numpy().view(np.uint32)


# rows 256 (8 row sets): quarter-set workgroups; 4096 (128): half sets; 16384 (512): full sets;
# all within the in-kernel quantization's work limit at cols = 256
@pytest.mark.parametrize("rows", [256, 4096, 16384])
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8])
def test_fq_codes_match_reference_quantizer(kq4, torch_dev, orc, rows, m):
    torch = torch_dev
    xs = quant_rows()
    cols = xs.shape[1]
    w = kq4.prepare_dev(to_dev(torch, synth.make_q4_weights(rows, cols, 900 + rows)), rows, cols)
    for start in range(0, xs.shape[0], m):
        x = xs[[(start + i) % xs.shape[0] for i in range(m)]]
        xq, xd = orc.quantize(x, cols)
        a = torch.empty((m, rows), dtype=torch.float32, device="cuda")
        b = torch.empty_like(a)
        with kq4.options(gemv_fq=1):
            kq4.matmul_dev(a, to_dev(torch, x), w, rows, cols)
        kq4.matmul_q_dev(b, to_dev(torch, xq), to_dev(torch, xd), w, rows, cols, m)
        torch.cuda.synchronize()
        assert np.array_equal(bits(a), bits(b)), (rows, m, start)


@pytest.mark.parametrize("m", [1, 2, 3, 4, 7, 8])
def test_fq_silu_codes_match_oracle(kq4, torch_dev, orc, m):
    """FQ = 2: the down projection forms silu_mul(gate, up) and quantizes it in the kernel; fed
    with the oracle's codes of the oracle's product instead, the outputs are bit-identical."""
    torch = torch_dev
    xs = quant_rows()
    rows, cols = 4096, xs.shape[1]
    w = kq4.prepare_dev(to_dev(torch, synth.make_q4_weights(rows, cols, 950)), rows, cols)
    rng = np.random.default_rng(951)
    for start in range(0, xs.shape[0], m):
        g = xs[[(start + i) % xs.shape[0] for i in range(m)]] * np.float32(0.05)
        u = rng.uniform(-3, 3, g.shape).astype(np.float32)
        u[:, :32] = 1.0
        xq, xd = orc.quantize(orc.silu_mul(g, u), cols)
        a = torch.empty((m, rows), dtype=torch.float32, device="cuda")
        b = torch.empty_like(a)
        with kq4.options(gemv_fq=1):
            kq4.matmul_silu_dev(a, to_dev(torch, g), to_dev(torch, u), w, rows, cols)
        kq4.matmul_q_dev(b, to_dev(torch, xq), to_dev(torch, xd), w, rows, cols, m)
        torch.cuda.synchronize()
        assert np.array_equal(bits(a), bits(b)), (m, start)


@pytest.mark.parametrize("m", [1, 2, 4, 8])
def test_fq_full_size_gate_up(kq4, torch_dev, orc, m):
    """The Qwen3-8B fused gate/up at M = 1, 2, 4, 8 with the planner's own launch shape, with the
    fixture's edge rows in its first blocks: the fp32-input launch is bit-identical to the one
    fed with the oracle's codes."""
    torch = torch_dev
    h, f = synth.QWEN3_8B["hidden"], synth.QWEN3_8B["ffn"]
    x = synth.make_activations(m, h, 960 + m)
    xs = quant_rows()
    for i in range(m):
        x[i, :256] = xs[(5 * i) % 16]
        x[i, 256:512] = xs[(5 * i + 2) % 16]
    xq, xd = orc.quantize(x, h)
    ws = [kq4.prepare_dev(to_dev(torch, synth.make_q4_weights(f, h, 961 + k, **synth.SCALE_8B)),
                          f, h) for k in range(2)]
    a = [torch.empty((m, f), dtype=torch.float32, device="cuda") for _ in range(2)]
    b = [torch.empty_like(t) for t in a]
    kq4.matmul_multi_dev(a, to_dev(torch, x), ws, [f, f], h)
    kq4.matmul_multi_q_dev(b, to_dev(torch, xq), to_dev(torch, xd), ws, [f, f], h, m)
    torch.cuda.synchronize()
    for p, q in zip(a, b):
        assert np.array_equal(bits(p), bits(q))
