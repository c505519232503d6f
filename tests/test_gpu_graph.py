"""The device API under HIP graph capture: a decode-style GEMV (quantization fused), a GEMV from a
separate quantize launch, a prefill GEMM and a MoE FFN are captured once and replayed several
times, with eager launches and host synchronisations between the replays; every replay must
reproduce the eager result bit for bit (same kernels, same inputs, deterministic reductions)."""
import numpy as np
import pytest

import synth

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
