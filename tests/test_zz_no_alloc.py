"""kq4_matmul_noalloc_dev, the matmul entry point that allocates nothing: its quantized
activations live in a fixed per-device scratch array instead of the growable workspace. It runs
the same kernels as kq4_matmul_dev, so its outputs must be bit-identical to that entry point's,
through the C ABI, on two calls in a row (the second smaller, so it reads a scratch that still
holds the first call's data), on a one-token call (in-kernel quantization, no scratch) and on a
shape too large for the scratch (refused before anything runs)."""
import numpy as np
import pytest

import synth

pytestmark = pytest.mark.gpu


def to_dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def bits(t):
    return t.cpu().numpy().view(np.uint32)


def run_both(kq4, torch, rows, cols, n, seed, residual):
    w = kq4.prepare_dev(to_dev(torch, synth.make_q4_weights(rows, cols, seed)), rows, cols)
    x = to_dev(torch, synth.make_activations(n, cols, seed + 1))
    res = to_dev(torch, synth.make_activations(n, rows, seed + 2)) if residual else None
    a = torch.empty((n, rows), dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    kq4.matmul_noalloc_dev(a, x, w, rows, cols, residual=res)
    torch.cuda.synchronize()
    kq4.matmul_dev(b, x, w, rows, cols, residual=res)
    torch.cuda.synchronize()
    return a, b


def test_noalloc_matches_matmul_dev(kq4, torch_dev):
    torch = torch_dev
    # 1: prefill GEMM, 512 tokens x 4096 columns (4.5 MB of scratch)
    a, b = run_both(kq4, torch, 1024, 4096, 512, 11, residual=True)
    assert np.array_equal(bits(a), bits(b))
    # 2: smaller, right after: a 6-token GEMV from the separate quantizer launch
    a, b = run_both(kq4, torch, 768, 2048, 6, 21, residual=False)
    assert np.array_equal(bits(a), bits(b))
    # one token (quantized inside the GEMV; the scratch is not used)
    a, b = run_both(kq4, torch, 512, 2048, 1, 31, residual=True)
    assert np.array_equal(bits(a), bits(b))


def test_noalloc_largest_fits_and_beyond_is_refused(kq4, torch_dev):
    torch = torch_dev
    # 2048 tokens x 12288 columns (the Qwen3-8B down prefill): 53.5 MB of fp8 GEMM operands,
    # within the 64 MiB scratch
    a, b = run_both(kq4, torch, 128, 12288, 2048, 41, residual=False)
    assert np.array_equal(bits(a), bits(b))
    rows, cols, n = 128, 16384, 2048                     # 71.3 MB: refused
    w = torch.zeros(kq4.stream_bytes(rows, cols), dtype=torch.uint8, device="cuda")
    x = torch.empty((n, cols), dtype=torch.float32, device="cuda")
    out = torch.empty((n, rows), dtype=torch.float32, device="cuda")
    with pytest.raises(kq4.KQ4Error, match="scratch"):
        kq4.matmul_noalloc_dev(out, x, w, rows, cols)
