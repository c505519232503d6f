"""GPU parity of the MoE FFN (int8 track) against the oracle (which is pinned bit-exact to the
reference's own MoE in tests/test_oracle_moe.py), stage by stage:
  router logits (fp32 serial chains)      bit-exact
  routing (device top-k/softmax)          sel exact, pr within 2 ulp (expf bits)
  gate / up (V4 chains)                   bit-exact
  SiLU product av                          within 4 ulp (exp evaluated on the device)
  down partials fed with the oracle's av   bit-exact (then Y bit-exact with the oracle's routing)
  end to end Y                             max|dY|/max|Y| <= 1e-5, max-abs reported
"""
import numpy as np
import pytest

import synth
from conftest import rel_err

pytestmark = pytest.mark.gpu


def to_dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.cpu().numpy()


def ulps(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(a - b).max() if a.size else 0


SHAPES = {"small": dict(hidden=256, experts=16, top_k=4, ef=64),
          "qwen3_30b_a3b": synth.QWEN3_30B_A3B_MOE,
          # the largest hidden size the kernels take (8 stages of 16 blocks)
          "wide": dict(hidden=4096, experts=12, top_k=3, ef=96),
          # top-16 and 32-block bands: the one-token down + combine kernel at its limits
          # (16 waves, four band lines per lane)
          "k16": dict(hidden=512, experts=32, top_k=16, ef=1024),
          # bands of one and two 8-block half stages (the one-wave-per-row-set down kernel's
          # other instantiations; Qwen3-30B-A3B has three, k16 four)
          "nh1": dict(hidden=512, experts=32, top_k=8, ef=256),
          "nh2": dict(hidden=1024, experts=16, top_k=4, ef=512),
          # Qwen3-30B-A3B's 24-block bands with many pairs per expert: the down kernel's
          # 8-pair passes (the launch averages more than 4 pairs per expert slot at T = 64)
          "nh3_dense": dict(hidden=512, experts=8, top_k=4, ef=768)}


def test_route(kq4, torch_dev, orc):
    torch = torch_dev
    lg = synth.make_logits(64, 128, 3)
    lg[:, 7] = lg[:, 3]
    sel_o, pr_o = orc.moe_route(lg, 8)
    sel = torch.empty((64, 8), dtype=torch.int32, device="cuda")
    pr = torch.empty((64, 8), dtype=torch.float32, device="cuda")
    kq4.moe_route_dev(sel, pr, to_dev(torch, lg), 8)
    torch.cuda.synchronize()
    assert np.array_equal(host(sel), sel_o)
    assert ulps(host(pr), pr_o) <= 2


@pytest.mark.parametrize("ne,tk", [(100, 8), (2048, 32), (64, 1)])
def test_route_edge_cases(kq4, torch_dev, orc, ne, tk):
    """Ragged expert counts, the largest ne and top-k, NaN / -inf / signed-zero logits, ties,
    and tokens with fewer than k candidates (their tail ids are -1, probabilities 0)."""
    torch = torch_dev
    T = 6
    lg = synth.make_logits(T, ne, 17 + ne)
    lg[1, ::3] = np.nan
    lg[1, 1::7] = -np.inf
    lg[2, :] = 0.5                                   # all tied: ids 0 .. tk-1 in order
    lg[3, :] = 0.0
    lg[3, ::2] = -0.0                                # +0 and -0 compare equal: ties by id
    lg[4, :] = np.nan
    lg[4, [ne - 1, ne // 2, 0][:min(3, ne)]] = [1.0, -np.inf, 2.0][:min(3, ne)]
    lg[5, :] = -np.inf                               # only -inf candidates
    lg[5, ne // 3] = 3.0
    sel_o, pr_o = orc.moe_route(lg, tk)
    sel = torch.empty((T, tk), dtype=torch.int32, device="cuda")
    pr = torch.empty((T, tk), dtype=torch.float32, device="cuda")
    kq4.moe_route_dev(sel, pr, to_dev(torch, lg), tk)
    torch.cuda.synchronize()
    assert np.array_equal(host(sel), sel_o)
    assert np.array_equal(np.isnan(host(pr)), np.isnan(pr_o))
    fin = ~np.isnan(pr_o)
    assert ulps(host(pr)[fin], pr_o[fin]) <= 2


@pytest.mark.parametrize("T", [1, 7, 64])
@pytest.mark.parametrize("shape", ["small", "qwen3_30b_a3b", "wide", "k16", "nh1", "nh2",
                                   "nh3_dense"])
def test_moe_stages(kq4, torch_dev, orc, shape, T):
    check_stages(kq4, torch_dev, orc, SHAPES[shape], T, 40 + T, shape)


def check_stages(kq4, torch, orc, cfg, T, seed, name):
    """Stage by stage against the oracle: gate and up bit-exact, av within 4 ulp, Y within 1e-5;
    the down stage fed the oracle's av bit-exact; the FFN without stage outputs the same bits."""
    d, ne, tk, ef = cfg["hidden"], cfg["experts"], cfg["top_k"], cfg["ef"]
    G, U, D = synth.make_moe(cfg, seed)
    X = synth.make_activations(T, d, seed + 10)
    sel, pr = orc.moe_route(synth.make_logits(T, ne, seed + 20), tk)
    Y_o, st = orc.moe_ffn(X, sel, pr, G, U, D, ne, d, ef, stages=True)

    dG, dU = (kq4.prepare_dev(to_dev(torch, a), ne * ef, d) for a in (G, U))
    dD = kq4.prepare_dev(to_dev(torch, D), d, ne * ef)
    dX, dsel, dpr = to_dev(torch, X), to_dev(torch, sel), to_dev(torch, pr)
    Y = torch.empty((T, d), dtype=torch.float32, device="cuda")
    gate = torch.zeros((T * tk, ef), dtype=torch.float32, device="cuda")
    up = torch.zeros_like(gate)
    av = torch.zeros_like(gate)
    kq4.moe_ffn_stages_dev(Y, dX, dsel, dpr, dG, dU, dD, ne, d, ef, gate=gate, up=up, av=av)
    torch.cuda.synchronize()
    assert np.array_equal(host(gate).view(np.uint32), st["gate"].view(np.uint32))
    assert np.array_equal(host(up).view(np.uint32), st["up"].view(np.uint32))
    # exp() on the device vs the host's libm expf: a last-ulp difference in exp can move
    # fl(g / fl(1 + e)) * u by a few ulp
    assert ulps(host(av), st["av"]) <= 4
    r, a = rel_err(host(Y), Y_o)
    print(f"moe {name} T={T}: Y rel={r:.3e} maxabs={a:.3e} "
          f"bit-exact={np.array_equal(host(Y), Y_o)}")
    assert r <= 1e-5

    # down stage fed with the oracle's av: bit-exact partials and output
    Y2 = torch.empty_like(Y)
    kq4.moe_ffn_stages_dev(Y2, dX, dsel, dpr, dG, dU, dD, ne, d, ef,
                           av_in=to_dev(torch, st["av"]))
    torch.cuda.synchronize()
    assert np.array_equal(host(Y2).view(np.uint32), Y_o.view(np.uint32))
    # the FFN without stage outputs gives the same bits
    Y3 = torch.empty_like(Y)
    kq4.moe_ffn_dev(Y3, dX, dsel, dpr, dG, dU, dD, ne, d, ef)
    torch.cuda.synchronize()
    assert np.array_equal(host(Y3).view(np.uint32), host(Y).view(np.uint32))


# Seeded random shapes: hidden a multiple of 32 up to 1024 (partial stream stages), expert width
# a multiple of 32 up to 1024 (bands of any block count: both down kernels, odd bands, the
# one-token down + combine and its fallback), 2-40 experts, top-k up to min(16, experts), 1-40
# tokens.
@pytest.mark.parametrize("i", range(12))
def test_moe_random_shapes(kq4, torch_dev, orc, i):
    rng = np.random.default_rng(8000 + i)
    ne = int(rng.integers(2, 41))
    cfg = dict(hidden=32 * int(rng.integers(1, 33)), experts=ne,
               top_k=int(rng.integers(1, min(16, ne) + 1)), ef=32 * int(rng.integers(1, 33)))
    T = 1 if i % 4 == 0 else int(rng.integers(2, 41))
    check_stages(kq4, torch_dev, orc, cfg, T, 8100 + 30 * i, f"random {i} {cfg}")


@pytest.mark.parametrize("shape", ["small", "qwen3_30b_a3b"])
def test_moe_one_token_all_ids_invalid(kq4, torch_dev, orc, shape):
    """No valid rank at one token: the output is zero (the combine adds nothing), with and
    without stage outputs."""
    torch = torch_dev
    cfg = SHAPES[shape]
    d, ne, tk, ef = cfg["hidden"], cfg["experts"], cfg["top_k"], cfg["ef"]
    G, U, D = synth.make_moe(cfg, 93)
    dG, dU = (kq4.prepare_dev(to_dev(torch, a), ne * ef, d) for a in (G, U))
    dD = kq4.prepare_dev(to_dev(torch, D), d, ne * ef)
    dX = to_dev(torch, synth.make_activations(1, d, 94))
    dsel = to_dev(torch, np.array([[-1] * (tk - 1) + [ne]], np.int32))
    dpr = to_dev(torch, np.full((1, tk), 0.25, np.float32))
    Y = torch.full((1, d), float("nan"), dtype=torch.float32, device="cuda")
    kq4.moe_ffn_dev(Y, dX, dsel, dpr, dG, dU, dD, ne, d, ef)
    gate = torch.zeros((tk, ef), dtype=torch.float32, device="cuda")
    up = torch.zeros_like(gate)
    Y2 = torch.full((1, d), float("nan"), dtype=torch.float32, device="cuda")
    kq4.moe_ffn_stages_dev(Y2, dX, dsel, dpr, dG, dU, dD, ne, d, ef, gate=gate, up=up)
    torch.cuda.synchronize()
    assert np.array_equal(host(Y), np.zeros((1, d), np.float32))
    assert np.array_equal(host(Y2), np.zeros((1, d), np.float32))


@pytest.mark.parametrize("T", [1, 3])   # T = 1 takes the kernels' one-token mode (no grouping)
def test_moe_invalid_expert_ids_skipped(kq4, torch_dev, orc, T):
    torch = torch_dev
    cfg = SHAPES["small"]
    d, ne, tk, ef = cfg["hidden"], cfg["experts"], cfg["top_k"], cfg["ef"]
    G, U, D = synth.make_moe(cfg, 90)
    X = synth.make_activations(T, d, 91)
    sel, pr = orc.moe_route(synth.make_logits(T, ne, 92), tk)
    sel[T - 1, 1] = -1
    sel[T // 2, 0] = ne + 5
    Y_o = orc.moe_ffn(X, sel, pr, G, U, D, ne, d, ef)
    Y = kq4.moe_ffn(X, sel, pr, G, U, D, ne, d, ef)
    r, _ = rel_err(Y, Y_o)
    assert r <= 1e-5


def make_router(ne, d, seed):
    return (np.random.default_rng(seed).standard_normal((ne, d)) * 0.02).astype(np.float32)


@pytest.mark.parametrize("T,ne,d", [(1, 128, 2048), (7, 60, 96), (64, 128, 2048), (3, 300, 64)])
def test_router_logits_bit_exact(kq4, torch_dev, orc, T, ne, d):
    """fp32 router logits: the reference's serial chain per (token, expert), bit for bit."""
    torch = torch_dev
    R = make_router(ne, d, T + ne)
    X = synth.make_activations(T, d, d + T)
    want = orc.router_logits(R, X, ne, d)
    lg = torch.empty((T, ne), dtype=torch.float32, device="cuda")
    kq4.moe_router_logits_dev(lg, to_dev(torch, R), to_dev(torch, X))
    torch.cuda.synchronize()
    assert np.array_equal(host(lg).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("T", [1, 64])
@pytest.mark.parametrize("shape", ["small", "qwen3_30b_a3b"])
def test_moe_layer_dev(kq4, torch_dev, orc, shape, T):
    """Router logits + routing + expert FFN in one call against the oracle's layer (its router
    and FFN are each pinned to the reference's own MoE)."""
    torch = torch_dev
    cfg = SHAPES[shape]
    d, ne, tk, ef = cfg["hidden"], cfg["experts"], cfg["top_k"], cfg["ef"]
    G, U, D = synth.make_moe(cfg, 70 + T)
    R = make_router(ne, d, 71 + T)
    X = synth.make_activations(T, d, 72 + T)
    sel_o, pr_o = orc.moe_route(orc.router_logits(R, X, ne, d), tk)
    Y_o = orc.moe_ffn(X, sel_o, pr_o, G, U, D, ne, d, ef)

    dG, dU = (kq4.prepare_dev(to_dev(torch, a), ne * ef, d) for a in (G, U))
    dD = kq4.prepare_dev(to_dev(torch, D), d, ne * ef)
    Y = torch.empty((T, d), dtype=torch.float32, device="cuda")
    sel = torch.empty((T, tk), dtype=torch.int32, device="cuda")
    pr = torch.empty((T, tk), dtype=torch.float32, device="cuda")
    kq4.moe_layer_dev(Y, to_dev(torch, X), to_dev(torch, R), dG, dU, dD, ne, tk, d, ef,
                      sel=sel, pr=pr)
    torch.cuda.synchronize()
    assert np.array_equal(host(sel), sel_o)
    assert ulps(host(pr), pr_o) <= 2
    r, a = rel_err(host(Y), Y_o)
    print(f"moe layer {shape} T={T}: Y rel={r:.3e} maxabs={a:.3e}")
    assert r <= 1e-5
