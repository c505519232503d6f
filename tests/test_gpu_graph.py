"""The device API under HIP graph capture: a decode-style GEMV (quantization fused), a GEMV from a
separate quantize launch, a prefill GEMM and a MoE FFN are captured once and replayed several
times, with eager launches and host synchronisations between the replays; every replay must
reproduce the eager result bit for bit (same kernels, same inputs, deterministic reductions)."""
import numpy as np
import pytest

import synth
from conftest import rel_err

pytestmark = pytest.mark.gpu


def to_dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def test_graph_replays_match_eager(kq4, torch_dev):
    torch = torch_dev
    cols, rows, rows2 = 1024, 512, 256
    w = kq4.prepare_dev(to_dev(torch, synth.make_q4_weights(rows, cols, 1)), rows, cols)
    w2 = kq4.prepare_dev(to_dev(torch, synth.make_q4_weights(rows2, cols, 2)), rows2, cols)
    x1 = to_dev(torch, synth.make_activations(1, cols, 3))
    x6 = to_dev(torch, synth.make_activations(6, cols, 4))
    x64 = to_dev(torch, synth.make_activations(64, cols, 5))
    res = to_dev(torch, synth.make_activations(6, rows, 6))
    cfg = dict(hidden=256, experts=16, top_k=4, ef=64)
    G, U, D = (kq4.prepare_dev(to_dev(torch, a), r, c)
               for a, r, c in zip(synth.make_moe(cfg, 7), (1024, 1024, 256), (256, 256, 1024)))
    X = to_dev(torch, synth.make_activations(3, 256, 8))
    lg = to_dev(torch, synth.make_logits(3, 16, 9))
    sel = torch.empty((3, 4), dtype=torch.int32, device="cuda")
    pr = torch.empty((3, 4), dtype=torch.float32, device="cuda")

    outs = dict(a=torch.empty((1, rows), device="cuda"), b=torch.empty((1, rows2), device="cuda"),
                c=torch.empty((6, rows), device="cuda"), d=torch.empty((64, rows), device="cuda"),
                y=torch.empty((3, 256), device="cuda"))

    def work():
        st = torch.cuda.current_stream()
        kq4.matmul_multi_dev([outs["a"], outs["b"]], x1, [w, w2], [rows, rows2], cols, stream=st)
        kq4.matmul_dev(outs["c"], x6, w, rows, cols, residual=res, stream=st)
        kq4.matmul_dev(outs["d"], x64, w, rows, cols, stream=st)
        kq4.moe_route_dev(sel, pr, lg, 4, stream=st)
        kq4.moe_ffn_dev(outs["y"], X, sel, pr, G, U, D, 16, 256, 64, stream=st)

    work()                                     # eager; also sizes the library's workspace
    torch.cuda.synchronize()
    want = {k: v.clone() for k, v in outs.items()}

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        work()
    for rep in range(4):
        for v in outs.values():
            v.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for k in outs:
            got, exp = outs[k].cpu().numpy(), want[k].cpu().numpy()
            assert np.array_equal(got.view(np.uint32), exp.view(np.uint32)), (rep, k)
        work()                                 # eager work between replays
        torch.cuda.synchronize()


def test_graph_survives_workspace_growth(kq4, torch_dev):
    """A graph captured around calls that use the library's workspace (the separate quantizer
    launch of a 6-token GEMV, a 64-token GEMM) stays valid after the workspace grows: growth
    keeps the old buffer for the graph, and the eager calls after it use the new one. Every
    replay reproduces the eager result bit for bit."""
    torch = torch_dev
    rows, cols = 512, 1024
    w = kq4.prepare_dev(to_dev(torch, synth.make_q4_weights(rows, cols, 21)), rows, cols)
    x6 = to_dev(torch, synth.make_activations(6, cols, 22))
    x64 = to_dev(torch, synth.make_activations(64, cols, 23))
    o6, o64 = torch.empty((6, rows), device="cuda"), torch.empty((64, rows), device="cuda")

    def work():
        st = torch.cuda.current_stream()
        kq4.matmul_dev(o6, x6, w, rows, cols, stream=st)
        kq4.matmul_dev(o64, x64, w, rows, cols, stream=st)

    work()
    torch.cuda.synchronize()
    want = [o6.clone(), o64.clone()]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        work()
    # grow the workspace well past anything used so far, then overwrite the new one eagerly
    kq4.workspace_reserve(512 << 20)
    big_n, big_cols = 1024, 8192
    wb = kq4.prepare_dev(to_dev(torch, synth.make_q4_weights(64, big_cols, 24)), 64, big_cols)
    xb = to_dev(torch, synth.make_activations(big_n, big_cols, 25))
    ob = torch.empty((big_n, 64), device="cuda")
    for rep in range(3):
        o6.fill_(float("nan"))
        o64.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for got, exp in zip((o6, o64), want):
            assert np.array_equal(got.cpu().numpy().view(np.uint32),
                                  exp.cpu().numpy().view(np.uint32)), rep
        kq4.matmul_dev(ob, xb, wb, 64, big_cols)   # eager, in the grown workspace
        torch.cuda.synchronize()


def test_growth_during_capture_is_refused(kq4, torch_dev):
    """A call that would have to grow the workspace while its stream is captured fails with
    KQ4_EINVAL before launching anything, and the capture stays usable. Its inputs are never
    read (the call returns first), so they are left uninitialised."""
    torch = torch_dev
    rows, cols, n = 4, 32 * 5120, 4096            # 755 MB of quantized activations
    assert kq4.matmul_workspace_bytes(n, cols) > (640 << 20)
    w = torch.zeros(kq4.stream_bytes(rows, cols), dtype=torch.uint8, device="cuda")
    x = torch.empty((n, cols), dtype=torch.float32, device="cuda")
    out = torch.empty((n, rows), device="cuda")
    marker = torch.empty(16, device="cuda")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        marker.fill_(7.0)
        with pytest.raises(kq4.KQ4Error, match="captured"):
            kq4.matmul_dev(out, x, w, rows, cols, stream=torch.cuda.current_stream())
    marker.zero_()
    graph.replay()
    torch.cuda.synchronize()
    assert float(marker.sum()) == 7.0 * 16


def test_workspace_trim_frees_outgrown_workspaces(kq4, torch_dev, orc):
    """Growth keeps every outgrown workspace for graphs captured before it; once no such graph is
    alive kq4_workspace_trim frees them (the device's free memory rises by at least the 1.25 GiB
    buffer that the second growth retired), and calls after it run in the current workspace."""
    torch = torch_dev
    kq4.workspace_reserve(1 << 30)            # the workspace is now >= 1.25 GiB
    kq4.workspace_reserve(2 << 30)            # ... and that one is retired
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    kq4.workspace_trim()
    free1, _ = torch.cuda.mem_get_info()
    print(f"trim freed {(free1 - free0) / 2**30:.2f} GiB")
    assert free1 - free0 >= (5 << 30) // 4
    kq4.workspace_trim()                      # nothing left to free
    rows, cols, n = 256, 2048, 64
    w = synth.make_q4_weights(rows, cols, 31)
    x = synth.make_activations(n, cols, 32)
    out = torch.empty((n, rows), device="cuda")
    with kq4.options(gemm_split=1):   # the single chain, bit for bit
        kq4.matmul_dev(out, to_dev(torch, x), kq4.prepare_dev(to_dev(torch, w), rows, cols),
                       rows, cols)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint32),
                          orc.matmul(w, x, rows, cols).view(np.uint32))


def test_graph_split_k_gemm(kq4, torch_dev, orc):
    """A K-split prefill GEMM (planner: 64 tiles of 64 x 128, K = 8192 in 8 slices; the slices'
    partial sums in the workspace, a reduction launch adding them and the residual) captured in
    a graph: every replay, with eager work of other shapes between them, reproduces the eager
    result bit for bit, which is within 1e-5 of the oracle's single chain."""
    torch = torch_dev
    n, rows, cols = 512, 1024, 8192
    w = synth.make_q4_weights(rows, cols, 41)
    x = synth.make_activations(n, cols, 42)
    res = synth.make_activations(n, rows, 43)
    W = kq4.prepare_dev(to_dev(torch, w), rows, cols)
    X, R = to_dev(torch, x), to_dev(torch, res)
    out = torch.empty((n, rows), device="cuda")
    st = torch.cuda.current_stream()
    kq4.matmul_dev(out, X, W, rows, cols, residual=R, stream=st)
    torch.cuda.synchronize()
    want = out.cpu().numpy().copy()
    xq, xd = orc.quantize(x, cols)
    rng = np.random.default_rng(44)
    tok = rng.integers(0, n, 2048).astype(np.int32)
    row = rng.integers(0, rows, 2048).astype(np.int32)
    ref = orc.matmul_q_sample(w, xq, xd, rows, cols, n, tok, row, residual=res)
    d = np.abs(want[tok, row].astype(np.float64) - ref).max() / np.abs(ref).max()
    assert d <= 1e-5, d
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        kq4.matmul_dev(out, X, W, rows, cols, residual=R, stream=torch.cuda.current_stream())
    other = torch.empty((64, rows), device="cuda")
    for rep in range(3):
        out.fill_(float("nan"))
        kq4.matmul_dev(other, X[:64], W, rows, cols)   # eager, the same workspace
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32)), rep


def test_graph_gemv_chunks_and_small_batch_split(kq4, torch_dev, orc):
    """A 12-token q4 matmul (one launch of the 16-token GEMV kernel) and a 40-token one the
    planner splits over 64 x 64 tiles (K = 4096 in 4 slices,
    partial sums in the workspace, a reduction launch) captured in one graph: every replay, with
    eager calls of other shapes on the same workspace between them, reproduces the eager result
    bit for bit, and both are within 1e-5 of the oracle."""
    torch = torch_dev
    rows, cols = 1024, 4096
    w = synth.make_q4_weights(rows, cols, 51)
    W = kq4.prepare_dev(to_dev(torch, w), rows, cols)
    xs = {n: synth.make_activations(n, cols, 52 + n) for n in (12, 40)}
    X = {n: to_dev(torch, x) for n, x in xs.items()}
    out = {n: torch.empty((n, rows), device="cuda") for n in xs}
    assert kq4.gemm_plan(12, rows, cols) == (0, 0)
    assert kq4.gemm_plan(40, rows, cols, chain=kq4.CHAIN_ASM)[1] > 1

    def work():
        st = torch.cuda.current_stream()
        for n in xs:
            kq4.matmul_dev(out[n], X[n], W, rows, cols, stream=st)

    work()
    torch.cuda.synchronize()
    want = {n: out[n].cpu().numpy().copy() for n in xs}
    for n, x in xs.items():
        e, _ = rel_err(want[n], orc.matmul(w, x, rows, cols))
        assert e <= 1e-5, (n, e)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        work()
    other = torch.empty((300, rows), device="cuda")
    xo = to_dev(torch, synth.make_activations(300, cols, 59))
    for rep in range(3):
        for n in xs:
            out[n].fill_(float("nan"))
        kq4.matmul_dev(other, xo, W, rows, cols)   # eager, the same workspace
        graph.replay()
        torch.cuda.synchronize()
        for n in xs:
            assert np.array_equal(out[n].cpu().numpy().view(np.uint32),
                                  want[n].view(np.uint32)), (rep, n)
