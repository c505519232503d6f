"""kq4_matmul_noalloc_dev, the matmul entry point that allocates nothing: its quantized
activations live in a fixed per-device scratch array instead of the growable workspace. It runs
the same kernels as kq4_matmul_dev, so its outputs must be bit-identical to that entry point's,
through the C ABI, on two calls in a row (the second smaller, so it reads a scratch that still
holds the first call's data), on a one-token call (in-kernel quantization, no scratch) and on a
shape too large for the scratch (refused before anything runs). It is captured in a HIP graph
at the largest shape the scratch holds and every replay matches the eager kq4_matmul_dev bit for
bit; the largest shapes also run the fp8-operand GEMM (option gemm_kind = 1), whose operands
(n_batch * cols * 17/8 bytes) fill the scratch."""
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
    # 2048 tokens x 12288 columns (the Qwen3-8B down prefill): 28.3 MB of int8 operands, and
    # with gemm_kind = 1 53.5 MB of fp8 operands, within the 64 MiB scratch
    a, b = run_both(kq4, torch, 128, 12288, 2048, 41, residual=False)
    assert np.array_equal(bits(a), bits(b))
    with kq4.options(gemm_kind=1):
        a, b = run_both(kq4, torch, 128, 12288, 2048, 43, residual=True)
    assert np.array_equal(bits(a), bits(b))
    rows, cols, n = 128, 16384, 2048                     # 71.3 MB: refused
    w = torch.zeros(kq4.stream_bytes(rows, cols), dtype=torch.uint8, device="cuda")
    x = torch.empty((n, cols), dtype=torch.float32, device="cuda")
    out = torch.empty((n, rows), dtype=torch.float32, device="cuda")
    with pytest.raises(kq4.KQ4Error, match="scratch"):
        kq4.matmul_noalloc_dev(out, x, w, rows, cols)


def test_noalloc_under_graph_capture(kq4, torch_dev):
    """2048 tokens x 15392 columns, first on int8 operands with the K-split partial sums in the
    scratch, then on fp8 operands: 64 MiB less 128 KiB of scratch. torch
    captures in the global mode, in which HIP refuses a hipMalloc from any thread and the
    capture fails, so a capture that succeeds and replays shows that the call allocated
    nothing. The graph is replayed three times, with eager calls of other shapes in between that
    overwrite the scratch, and matches the eager kq4_matmul_dev bit for bit each time."""
    torch = torch_dev
    rows, cols, n = 128, 15392, 2048
    need = n * (cols // 32) * 68
    assert (64 << 20) - (256 << 10) < need <= kq4.NOALLOC_SCRATCH_BYTES
    w = kq4.prepare_dev(to_dev(torch, synth.make_q4_weights(rows, cols, 51)), rows, cols)
    x = to_dev(torch, synth.make_activations(n, cols, 52))
    res = to_dev(torch, synth.make_activations(n, rows, 53))
    got = torch.full((n, rows), float("nan"), dtype=torch.float32, device="cuda")
    # the int8 form: 35.5 MB of operands and the K-split partial sums (16 tiles, 4 slices)
    g8 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g8):
        kq4.matmul_noalloc_dev(got, x, w, rows, cols, residual=res,
                               stream=torch.cuda.current_stream())
    want8 = torch.empty_like(got)
    kq4.matmul_dev(want8, x, w, rows, cols, residual=res)
    torch.cuda.synchronize()
    for rep in range(2):
        got.fill_(float("nan"))
        a, b = run_both(kq4, torch, 256, 4096, 96 + 32 * rep, 70 + rep, residual=True)
        assert np.array_equal(bits(a), bits(b))
        g8.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bits(got), bits(want8)), rep
    del g8
    with kq4.options(gemm_kind=1):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            kq4.matmul_noalloc_dev(got, x, w, rows, cols, residual=res,
                                   stream=torch.cuda.current_stream())
        want = torch.empty_like(got)
        kq4.matmul_dev(want, x, w, rows, cols, residual=res)
        torch.cuda.synchronize()
        for rep in range(3):
            got.fill_(float("nan"))
            # other calls between the replays overwrite the scratch
            a, b = run_both(kq4, torch, 256, 4096, 64 + 32 * rep, 60 + rep, residual=False)
            assert np.array_equal(bits(a), bits(b))
            g.replay()
            torch.cuda.synchronize()
            assert np.array_equal(bits(got), bits(want)), rep
