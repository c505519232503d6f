"""GPU parity of BASELINE.json configs[1]: one Qwen3-VL-2B decoder layer's decode-step linear
set, launched exactly as bench.py's timed step issues it, at M = 1 and M = 4 with the config's
seeded weights (int4 uniform, f16 scales |N(0, 0.02)| + 1e-4) and N(0, 1) activations:

  fused QKV      2048 -> 2048 + 1024 + 1024   dyn_matvec_q4_q8_fused_qkv_batched
                                              (vllm_safetensors.c:8684)
  O + residual   2048 -> 2048                 dyn_matvec_q4_q8_fused_o_residual_batched (:8713)
  fused gate/up  2048 -> 6144 + 6144          dyn_matvec_q4_q8_fused_gate_up_batched
  down + resid.  6144 -> 2048                 dyn_matvec_q4_q8_down_residual_batched

Every output is compared with the oracle (M = 1: the C-tile chain; M = 4: the asm-GEMM chain on
all four tokens, q4x4_gemm_batched :4593-4631) at max|got-ref| / max|ref| <= 1e-5, the
reference's own verify metric (:1177-1181), max-abs printed. The step runs eagerly and as a
replayed HIP graph (how the bench times it), with eager work between the replays."""
import numpy as np
import pytest

import synth
from conftest import rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-5
CFG = synth.QWEN3VL_2B


def layer(kq4, torch):
    """The bench's per-layer matrices (bench.make_model: seed 1 + position in layer_shapes)."""
    shapes = {name: (r, c) for name, r, c in synth.layer_shapes(CFG)}
    host = {name: synth.make_q4_weights(r, c, 1 + i, **synth.SCALE_2B)
            for i, (name, (r, c)) in enumerate(shapes.items())}
    dev = {k: kq4.prepare_dev(torch.from_numpy(v.reshape(-1)).cuda(), *shapes[k])
           for k, v in host.items()}
    return shapes, host, dev


@pytest.fixture(scope="module")
def model(kq4, torch_dev):
    return layer(kq4, torch_dev)


@pytest.mark.parametrize("m", [1, 4])
def test_decode_step_linear_set(kq4, torch_dev, orc, model, m):
    torch = torch_dev
    shapes, W, D = model
    h, f = CFG["hidden"], CFG["ffn"]
    q, kv = shapes["q"][0], shapes["k"][0]
    xs = {k: synth.make_activations(m, n, s) for k, n, s in
          (("x", h, 7), ("attn", q, 8), ("act", f, 9), ("resid", h, 10))}
    X = {k: torch.from_numpy(v).cuda() for k, v in xs.items()}
    dev = lambda n: torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")  # noqa
    outs = dict(q=dev(q), k=dev(kv), v=dev(kv), o=dev(h), gate=dev(f), up=dev(f), down=dev(h))

    def step(st):
        kq4.matmul_multi_dev([outs["q"], outs["k"], outs["v"]], X["x"],
                             [D["q"], D["k"], D["v"]], [q, kv, kv], h, stream=st)
        kq4.matmul_dev(outs["o"], X["attn"], D["o"], h, q, residual=X["resid"], stream=st)
        kq4.matmul_multi_dev([outs["gate"], outs["up"]], X["x"], [D["gate"], D["up"]], [f, f],
                             h, stream=st)
        kq4.matmul_dev(outs["down"], X["act"], D["down"], h, f, residual=X["resid"], stream=st)

    inputs = dict(q="x", k="x", v="x", o="attn", gate="x", up="x", down="act")
    want = {}
    for name, (rows, cols) in shapes.items():
        res = xs["resid"] if name in ("o", "down") else None
        want[name] = orc.matmul(W[name], xs[inputs[name]], rows, cols, residual=res)

    def check(tag):
        torch.cuda.synchronize()
        for name in shapes:
            got = outs[name].cpu().numpy()
            r, a = rel_err(got, want[name])
            print(f"config2 M={m} {tag} {name} {shapes[name]}: rel={r:.3e} maxabs={a:.3e}")
            assert np.isfinite(got).all() and r <= TOL, (tag, name, r, a)

    step(torch.cuda.current_stream())
    check("eager")

    graph = torch.cuda.CUDAGraph()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        step(st)                                   # sizes the workspace before capture
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        step(torch.cuda.current_stream())
    for rep in range(3):
        for o in outs.values():
            o.fill_(float("nan"))
        # eager work of another shape between replays overwrites the shared workspace
        junk = torch.empty((8, h), dtype=torch.float32, device="cuda")
        kq4.matmul_dev(junk, torch.ones((8, f), dtype=torch.float32, device="cuda"), D["down"],
                       h, f)
        graph.replay()
        check(f"graph replay {rep}")
